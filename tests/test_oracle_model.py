"""Pins the oracle's forward pass (src/model.rs) on the CPU.

An independent numpy forward of the Qwen3 block, written from the model
definition (not from the oracle's loops), checks the op order: RMSNorm, the
q/k/v projections, QK-norm *before* NeoX RoPE, GQA head sharing
(kv = h / (H/KVH)), causal softmax attention, the residual adds, SwiGLU and
the tied/untied logits. The numpy model runs in f64 with the same Q8
activation quantisation points as the reference's integer path; remaining
differences are f32-vs-f64 rounding (plus rare Q8 rounding flips they
cause), so the bars are loose in absolute terms but far below what any op
order mistake produces (those give O(1) relative errors).
"""
import os

import numpy as np
import pytest

import oracle
import rlh
from golden import ggml_formats as gf
from helpers import bits, rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def q8_dequant(x):
    """Q8 blocks of x (closed form, ties to even) dequantised: q * d."""
    q, d, _, _ = gf.quantize_q8_closed_form(np.asarray(x, np.float32), "even")
    return q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)


class NumpyQwen3:
    def __init__(self, spec, tensors):
        self.s = spec
        self.w = {}
        for kind, layer, ty, cols, rows, buf in tensors:
            m = gf.dequant(ty, buf, cols * rows).astype(np.float64)
            self.w[(kind, layer)] = m.reshape(rows, cols) if rows > 1 else m
        s = spec
        self.inv_freq = np.array([np.float32(np.power(np.float32(s.rope_theta), np.float32(
            np.float32(-2.0 * i) / np.float32(s.head_dim)))) for i in range(s.head_dim // 2)], np.float64)

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.s.rms_eps) * w

    def rope(self, v, pos):
        hd = self.s.head_dim
        a = (np.float32(pos) * self.inv_freq.astype(np.float32)).astype(np.float64)
        x0, x1 = v[:hd // 2].copy(), v[hd // 2:].copy()
        return np.concatenate([x0 * np.cos(a) - x1 * np.sin(a), x0 * np.sin(a) + x1 * np.cos(a)])

    def forward(self, tokens, q8=True, dump=None):
        s, W = self.s, self.w
        hd, H, KVH = s.head_dim, s.n_head, s.n_head_kv
        grp = H // KVH
        qz = q8_dequant if q8 else (lambda v: np.asarray(v, np.float64))
        xs = [W[(rlh.T_TOKEN_EMBD, 0)][t].copy() for t in tokens]
        K = [[] for _ in range(s.n_layer)]
        V = [[] for _ in range(s.n_layer)]
        for l in range(s.n_layer):
            for i, x in enumerate(xs):
                h = qz(self.rms(x, W[(rlh.T_ATTN_NORM, l)]))
                q = W[(rlh.T_ATTN_Q, l)] @ h
                k = W[(rlh.T_ATTN_K, l)] @ h
                v = W[(rlh.T_ATTN_V, l)] @ h
                q = np.concatenate([self.rope(self.rms(q[j * hd:(j + 1) * hd], W[(rlh.T_ATTN_Q_NORM, l)]), i)
                                    for j in range(H)])
                k = np.concatenate([self.rope(self.rms(k[j * hd:(j + 1) * hd], W[(rlh.T_ATTN_K_NORM, l)]), i)
                                    for j in range(KVH)])
                K[l].append(k)
                V[l].append(v)
                att = np.empty(H * hd)
                for j in range(H):
                    kv = j // grp
                    ks = np.stack([kk[kv * hd:(kv + 1) * hd] for kk in K[l]])
                    vs = np.stack([vv[kv * hd:(kv + 1) * hd] for vv in V[l]])
                    sc = ks @ q[j * hd:(j + 1) * hd] / np.sqrt(hd)
                    p = np.exp(sc - sc.max())
                    p /= p.sum()
                    att[j * hd:(j + 1) * hd] = p @ vs
                x = x + W[(rlh.T_ATTN_OUTPUT, l)] @ qz(att)
                h2 = qz(self.rms(x, W[(rlh.T_FFN_NORM, l)]))
                g = W[(rlh.T_FFN_GATE, l)] @ h2
                u = W[(rlh.T_FFN_UP, l)] @ h2
                x = x + W[(rlh.T_FFN_DOWN, l)] @ qz(g / (1 + np.exp(-g)) * u)
                xs[i] = x
            if dump is not None:
                dump.append(np.stack(xs))
        out_w = W[(rlh.T_OUTPUT, 0)] if (rlh.T_OUTPUT, 0) in W else W[(rlh.T_TOKEN_EMBD, 0)]
        return out_w @ q8_dequant(self.rms(xs[-1], W[(rlh.T_OUTPUT_NORM, 0)]))


@pytest.fixture(scope="module", params=["tiny-q4km", "tiny-q4km-untied", "tiny-q8_0"])
def model(request):
    spec = rlh.SPECS[request.param]
    tensors = rlh.synth_model(spec, 77)
    return spec, tensors, oracle.OracleModel(spec, tensors), NumpyQwen3(spec, tensors)


def test_forward_matches_numpy_model(model):
    spec, tensors, om, npm = model
    prompt = rlh.synth_tokens(78, 6, spec.vocab)
    oc = om.new_cache(32)
    oc.enable_dump(len(prompt))
    got = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    dump = []
    want = npm.forward(prompt, q8=True, dump=dump)
    for l in range(spec.n_layer):
        assert rel_l2(oc.hidden(l, len(prompt)), dump[l]) < 2e-3, l
    assert rel_l2(got, want) < 5e-3
    assert int(np.argmax(got)) == int(np.argmax(want)) or np.sort(want)[-1] - np.sort(want)[-2] < 1e-2


def test_default_prefill_matches_f32_numpy_model(model):
    """The default (f32 dequant, no activation quantisation) prefill path:
    hidden states track the unquantised f64 model tightly."""
    spec, tensors, om, npm = model
    prompt = rlh.synth_tokens(79, 5, spec.vocab)
    oc = om.new_cache(32)
    oc.enable_dump(len(prompt))
    oc.forward_into(prompt, 0, oracle.MODE_DEFAULT)
    dump = []
    npm.forward(prompt, q8=False, dump=dump)
    for l in range(spec.n_layer):
        assert rel_l2(oc.hidden(l, len(prompt)), dump[l]) < 2e-5, l


def test_batch_int_prefill_equals_sequential_decode(model):
    """forward_batch in BATCH_INT mode performs, per token, exactly the
    arithmetic of forward_one: bit-identical logits, hidden states and KV."""
    spec, tensors, om, _ = model
    prompt = rlh.synth_tokens(80, 7, spec.vocab)
    a = om.new_cache(32)
    a.enable_dump(len(prompt))
    la = a.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    b = om.new_cache(32)
    b.enable_dump(1)
    for i, t in enumerate(prompt):
        lb = b.forward_into(np.array([t], np.uint32), i, oracle.MODE_DEFAULT)
        for l in range(spec.n_layer):
            assert np.array_equal(bits(b.hidden(l, 1)[0]), bits(a.hidden(l, len(prompt))[i]))
    assert np.array_equal(bits(la), bits(lb))
    for l in range(spec.n_layer):
        for which in (0, 1):
            assert np.array_equal(bits(a.read_kv(l, which, len(prompt))), bits(b.read_kv(l, which, len(prompt))))


def test_kv_layout_and_truncation(model):
    """KV rows are [pos][kv_head][head_dim] (model.rs:116-129); a batch that
    overruns the cache is truncated to max_ctx - start_pos (model.rs:392)."""
    spec, tensors, om, npm = model
    oc = om.new_cache(4)
    prompt = rlh.synth_tokens(81, 9, spec.vocab)
    oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert oc.len == 4


def test_golden_tiny_trace():
    """Regression fixture: the oracle still reproduces tiny_trace.npz."""
    f = np.load(os.path.join(GOLDEN, "tiny_trace.npz"))
    spec = rlh.SPECS["tiny-q4km"]
    tensors = rlh.synth_model(spec, int(f["seed"]))
    om = oracle.OracleModel(spec, tensors)
    oc = om.new_cache(64)
    prompt = f["prompt"]
    oc.enable_dump(len(prompt))
    logits = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(logits), bits(f["logits"]))
    for l in range(spec.n_layer):
        assert np.array_equal(bits(oc.hidden(l, len(prompt))), bits(f["hidden"][l]))
    lib = oracle.load()
    toks = [lib.orc_argmax(logits.ctypes.data, len(logits))]
    for i in range(16):
        lg = oc.forward_into(np.array([toks[-1]], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        toks.append(lib.orc_argmax(lg.ctypes.data, len(lg)))
    assert toks == list(map(int, f["tokens"]))


def test_split_k_summation_order_breaks_the_parity_bars():
    """Why the device path keeps the reference's summation order: on the
    0.6B Q8_0 workload (48-token prompt, 128 greedy tokens), taking only the
    decode attention's softmax sum and PV sums over four position splits
    (the order of a split-K decode kernel; everything else bit-identical)
    moves the first decode step's logits by more than the 2e-3 relative L2
    bar and changes the greedy sequence within the workload's 128 tokens.
    A Q8 activation block rounds a value to the other side of a .5 boundary
    for a perturbation of one ulp, and that changes the next product by a
    whole quantization step."""
    name, P, N, _ = rlh.WORKLOADS[2]
    spec = rlh.SPECS[name]
    tensors = rlh.synth_model(spec, rlh.WORKLOAD_SEED)
    prompt = rlh.synth_tokens(rlh.WORKLOAD_SEED + 1, P, spec.vocab)
    lib = oracle.load()
    om = oracle.OracleModel(spec, tensors)
    runs = {}
    for mode in (oracle.MODE_DEFAULT, oracle.MODE_SPLIT_ATTN):
        oc = om.new_cache(P + N + 1)
        lg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
        toks, first = [lib.orc_argmax(lg.ctypes.data, len(lg))], None
        for i in range(N):
            lg = oc.forward_into(np.array([toks[-1]], np.uint32), P + i, mode)
            first = lg if first is None else first
            toks.append(lib.orc_argmax(lg.ctypes.data, len(lg)))
        runs[mode] = (toks, first)
        oc.close()
    om.close()
    (a, la), (b, lb) = runs[oracle.MODE_DEFAULT], runs[oracle.MODE_SPLIT_ATTN]
    assert rel_l2(lb, la) > 2e-3
    assert a != b
