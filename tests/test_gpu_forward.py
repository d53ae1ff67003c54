"""End-to-end parity of the device token loop against the CPU oracle.

Reference modes: decode = the AVX2 integer path (ops.rs:93-128); prefill =
RUST_LLAMA_BATCH_INT=1 (ops.rs:192-236). Required bars:
per-layer hidden states within 1e-3 relative L2, logits within 2e-3,
identical greedy tokens. The device path is built to match bit for bit, and
these tests assert that stronger property (the L2 numbers are printed).
"""
import ctypes

import numpy as np
import pytest

import oracle
import rlh
from helpers import bits, rel_l2

pytestmark = pytest.mark.gpu

_models = {}


def _get(name, seed=1234):
    key = (name, seed)
    if key not in _models:
        spec = rlh.SPECS[name]
        tensors = rlh.synth_model(spec, seed)
        _models[key] = (spec, tensors, rlh.Model(spec, tensors), oracle.OracleModel(spec, tensors))
    return _models[key]


def _greedy_ref(oc, prompt, n_gen):
    """main.rs:500-516 loop on the oracle: argmax after every step."""
    lib = oracle.load()
    logits = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    toks = [lib.orc_argmax(logits.ctypes.data, len(logits))]
    per_step = []
    for i in range(n_gen):
        lg = oc.forward_into(np.array([toks[-1]], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        per_step.append(lg)
        toks.append(lib.orc_argmax(lg.ctypes.data, len(lg)))
    return logits, toks, per_step


@pytest.mark.parametrize("name", ["tiny-q4km", "tiny-q8_0", "tiny-q4_0", "tiny-q4km-untied", "small-q4km",
                                  "tiny-smallvocab"])
def test_prefill_and_decode_bit_exact(name):
    print(f"forward parity {name}", flush=True)
    spec, tensors, m, om = _get(name)
    n_prompt, n_gen = 12, 10
    prompt = rlh.synth_tokens(99, n_prompt, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    c.set_debug(True)
    oc.enable_dump(n_prompt)
    logits = c.forward_into(prompt, 0)
    ref_logits = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    print(f"  prefill logits rel L2 {rel_l2(logits, ref_logits):.3e}")
    for l in range(spec.n_layer):
        h = c.layer_hidden(l, n_prompt)
        r = oc.hidden(l, n_prompt)
        assert rel_l2(h, r) <= 1e-3
        assert np.array_equal(bits(h), bits(r)), f"layer {l} hidden differs"
    for l in range(spec.n_layer):
        for which in (0, 1):
            assert np.array_equal(bits(c.read_kv(l, which, n_prompt)), bits(oc.read_kv(l, which, n_prompt)))
    assert rel_l2(logits, ref_logits) <= 2e-3
    assert np.array_equal(bits(logits), bits(ref_logits))
    assert c.len == n_prompt and oc.len == n_prompt

    # decode: one step at a time through forward_into (n == 1 -> forward_one)
    lib = oracle.load()
    tok = lib.orc_argmax(ref_logits.ctypes.data, len(ref_logits))
    assert c.greedy_next() == tok
    for i in range(n_gen):
        lg = c.forward_into(np.array([tok], np.uint32), n_prompt + i)
        rg = oc.forward_into(np.array([tok], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ (rel {rel_l2(lg, rg):.2e})"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
        assert c.greedy_next() == tok
    c.close()
    oc.close()


@pytest.mark.parametrize("name", ["tiny-q4km", "small-q4km"])
def test_decode_ring_plans_bit_exact(name, monkeypatch):
    """Decode with ring plans forced (RLH_MV_RING=1 when the cache, and with
    it the captured step, is made): ffn_down's row chains are added round by
    round while the producers stream the next tiles."""
    print(f"ring decode parity {name}", flush=True)
    monkeypatch.setenv("RLH_MV_RING", "1")
    spec, tensors, m, om = _get(name)
    n_prompt = 8
    prompt = rlh.synth_tokens(98, n_prompt, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    c.forward_into(prompt, 0)
    ref = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    lib = oracle.load()
    tok = lib.orc_argmax(ref.ctypes.data, len(ref))
    for i in range(6):
        lg = c.forward_into(np.array([tok], np.uint32), n_prompt + i)
        rg = oc.forward_into(np.array([tok], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ (rel {rel_l2(lg, rg):.2e})"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    c.close()
    oc.close()


@pytest.mark.parametrize("max_ctx,n_prompt", [(64, 40), (6000, 40), (1600, 700), (4400, 4100)])
def test_decode_attention_paths(max_ctx, n_prompt):
    """Decode attention with 8 query heads per KV head (the 32B grouping):
    the softmax kernel and the PV kernel that streams p and V through an
    8-slot LDS ring. 40 positions fit one 64-position chunk; 700 and 4100
    positions wrap the ring many times, hand chunks two ahead from the
    producers to the ordered adds and end on a clamped ragged tail (4100 is
    the 32B workload's context). The 700- and 4100-token prompts also run
    the prefill in several 512-token chunks with 8 heads per KV head.
    Logits bit-exact in every step."""
    print(f"decode attention g8 max_ctx {max_ctx} prompt {n_prompt}", flush=True)
    spec, tensors, m, om = _get("tiny-g8-q4km")
    prompt = rlh.synth_tokens(77, n_prompt, spec.vocab)
    c = m.new_cache(max_ctx)
    oc = om.new_cache(max_ctx)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg))
    lib = oracle.load()
    tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for i in range(6):
        lg = c.forward_into(np.array([tok], np.uint32), len(prompt) + i)
        rg = oc.forward_into(np.array([tok], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ (rel {rel_l2(lg, rg):.2e})"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    c.close()
    oc.close()


@pytest.mark.parametrize("max_ctx,n_prompt", [(300, 62), (1200, 250), (1200, 600), (1200, 1100), (4096, 130),
                                              (8000, 70)])
def test_decode_attention_g4_paths(max_ctx, n_prompt):
    """Decode attention with 4 query heads per KV head. Caches up to about
    1200 positions take the kernel that keeps its V slices in LDS (the
    products run two 64-position chunks ahead of the ordered adds, the
    exponentials 256-position chunks ahead of the softmax sums: the steps
    cross chunk boundaries, end on ragged chunks and, at 600 and 1100
    positions, use three and five exponential chunks), 4096 and 8000
    positions the softmax kernel and the PV kernel that streams p and V
    through LDS rings. Logits bit-exact in every step."""
    print(f"decode attention g4 max_ctx {max_ctx} prompt {n_prompt}", flush=True)
    spec, tensors, m, om = _get("tiny-g4-q4km")
    prompt = rlh.synth_tokens(55, n_prompt, spec.vocab)
    c = m.new_cache(max_ctx)
    oc = om.new_cache(max_ctx)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg))
    lib = oracle.load()
    tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for i in range(6):
        lg = c.forward_into(np.array([tok], np.uint32), n_prompt + i)
        rg = oc.forward_into(np.array([tok], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ (rel {rel_l2(lg, rg):.2e})"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    c.close()
    oc.close()


@pytest.mark.parametrize("name,max_ctx,n_prompt", [("tiny-g1-q4km", 64, 30), ("tiny-g1-q4km", 2000, 200),
                                                   ("tiny-g2-q4km", 64, 30), ("tiny-g2-q4km", 2000, 130),
                                                   ("tiny-g3-q4km", 64, 30), ("tiny-g3-q4km", 1200, 1100),
                                                   ("tiny-g3-q4km", 3000, 1300),
                                                   ("tiny-g5-q4km", 64, 30), ("tiny-g5-q4km", 3000, 1300),
                                                   ("tiny-g6-q4km", 64, 30), ("tiny-g6-q4km", 3000, 700),
                                                   ("tiny-g7-q4km", 64, 30), ("tiny-g7-q4km", 3000, 1300),
                                                   ("tiny-wide-q4km", 64, 20), ("tiny-wide-q4km", 3000, 100)])
def test_decode_attention_groupings(name, max_ctx, n_prompt):
    """Decode attention with 1, 2 and 3 query heads per KV head (the
    resident-V kernel for short caches, the softmax + streamed-ring PV
    kernels past ~1200-1500 positions), with 5, 6 and 7 (groups that do not
    divide the prefill kernels' 64 (token, head) pairs or the decode
    kernels' 64-lane chains: ragged pair tiles, 8-wide ring slices) and with
    13312-wide attention rows, where attn_output reads the Q8 blocks the
    attention kernels write (the fused streamed kernel for 64 positions, the
    softmax kernel + the streamed PV kernel for 3000). Prompts of 700-1300
    tokens run the prefill in two or three 512-token chunks, and decode rows
    of 1024 positions or more take the softmax sum by monosum run pairs.
    Logits bit-exact."""
    print(f"decode attention {name} max_ctx {max_ctx} prompt {n_prompt}", flush=True)
    spec, tensors, m, om = _get(name)
    prompt = rlh.synth_tokens(66, n_prompt, spec.vocab)
    c = m.new_cache(max_ctx)
    oc = om.new_cache(max_ctx)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg))
    lib = oracle.load()
    tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for i in range(5):
        lg = c.forward_into(np.array([tok], np.uint32), n_prompt + i)
        rg = oc.forward_into(np.array([tok], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ (rel {rel_l2(lg, rg):.2e})"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    c.close()
    oc.close()


@pytest.mark.parametrize("name", ["tiny-q4km", "small-q4km"])
def test_generate_greedy_matches_cpu_tokens(name):
    spec, tensors, m, om = _get(name)
    prompt = rlh.synth_tokens(5, 9, spec.vocab)
    n_gen = 24
    c = m.new_cache(64)
    oc = om.new_cache(64)
    logits = c.forward_into(prompt, 0)
    first = c.greedy_next()
    toks = c.generate_greedy(first, n_gen)
    _, ref_toks, _ = _greedy_ref(oc, prompt, n_gen)
    assert list(map(int, toks)) == ref_toks
    assert c.len == len(prompt) + n_gen
    c.close()
    oc.close()


@pytest.mark.parametrize("name", ["tiny-q4km", "small-q4km"])
def test_generate_sampled_matches_cpu(name):
    """Model::generate with temperature / top-k / top-p / repetition penalty
    (the SamplingParams defaults, sampler.rs:15-26): same tokens as the oracle,
    and generation stops at EOS."""
    print(f"sampled generate {name}", flush=True)
    spec, tensors, m, om = _get(name)
    prompt = rlh.synth_tokens(31, 10, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    params = rlh.sampling_params(seed=0xC0FFEE)
    oparams = oracle.SamplingParams(0.7, 40, 0.95, 1.1, 64, 0xC0FFEE)
    eos = spec.vocab + 7  # never sampled: full length
    toks = c.generate(prompt, 24, params, eos)
    ref = oc.generate(prompt, 24, oparams, eos)
    assert list(map(int, toks)) == list(map(int, ref))
    assert len(toks) == 24 and c.len == len(prompt) + 24
    eos = int(toks[5])
    first = int(np.flatnonzero(toks == eos)[0])
    toks2 = c.generate(prompt, 24, params, eos)
    assert list(map(int, toks2)) == list(map(int, toks[:first]))
    c.close()
    oc.close()


def test_forward_errors():
    spec, tensors, m, om = _get("tiny-q4km")
    c = m.new_cache(16)
    with pytest.raises(rlh.RlhError) as e:
        c.forward_into(np.array([spec.vocab], np.uint32), 0)
    assert e.value.code == rlh.RLH_EINVAL
    with pytest.raises(rlh.RlhError) as e:
        c.forward_into(np.array([1], np.uint32), 16)
    assert e.value.code == rlh.RLH_ECTX
    # batch truncation to max_ctx - start_pos (model.rs:392)
    c.forward_into(np.arange(20, dtype=np.uint32), 0)
    assert c.len == 16
    with pytest.raises(rlh.RlhError) as e:
        c.generate_greedy(1, 4)
    assert e.value.code == rlh.RLH_ECTX
    c.reset()
    assert c.len == 0
    c.close()


def test_cache_max_ctx_clamped_to_n_ctx():
    spec, tensors, m, om = _get("tiny-q4km")
    c = m.new_cache(10 ** 6)
    assert c.max_ctx == spec.n_ctx
    c.close()


def test_long_prefill_chunks_and_continuation():
    """A prompt longer than one prefill chunk (512 tokens), then a second
    batch continuing at start_pos > 0: logits and every K/V row bit-exact
    against the oracle's single forward_batch calls."""
    spec, tensors, m, om = _get("small-q4km")
    prompt = rlh.synth_tokens(123, 600, spec.vocab)
    more = rlh.synth_tokens(321, 30, spec.vocab)
    c = m.new_cache(700)
    oc = om.new_cache(700)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    print(f"  600-token prefill logits rel L2 {rel_l2(lg, rg):.3e}", flush=True)
    assert np.array_equal(bits(lg), bits(rg))
    lg2 = c.forward_into(more, 600)
    rg2 = oc.forward_into(more, 600, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg2), bits(rg2))
    for l in (0, spec.n_layer - 1):
        for which in (0, 1):
            assert np.array_equal(bits(c.read_kv(l, which, 630)), bits(oc.read_kv(l, which, 630)))
    assert c.len == 630
    c.close()
    oc.close()


def test_prefill_softmax_row_kernels():
    """Prefill rows of up to 4988 positions take the softmax kernel with one
    wave per row (16, 8 or 4 rows per block by row length), longer rows the
    kernel with one block per row: a 5200-token prompt in 512-token chunks
    uses the first for the chunks that end at or below position 4988
    (among them the chunk ending at 4608, whose 4 rows exceed 64 KB of LDS)
    and the second for the last two chunks (ending at 5120 and 5200). Logits and the last layer's K/V rows
    bit-exact against the oracle."""
    spec, tensors, m, om = _get("tiny-g4-q4km")
    prompt = rlh.synth_tokens(77, 5200, spec.vocab)
    c = m.new_cache(5300)
    oc = om.new_cache(5300)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg)), f"logits differ (rel {rel_l2(lg, rg):.2e})"
    for which in (0, 1):
        l = spec.n_layer - 1
        assert np.array_equal(bits(c.read_kv(l, which, 5200)), bits(oc.read_kv(l, which, 5200)))
    c.close()
    oc.close()


@pytest.mark.parametrize("grid_only", ["0", "1"])
def test_prefill_scores_kernels(monkeypatch, grid_only):
    """Prefill scores through the persistent kernel (few blocks per CU: every
    shape here) and, with RLH_QK_PRE_GRID=1, through the kernel with a block
    per work item: a 4300-token prompt (9 chunks of up to 512 tokens, 4
    query heads per KV head) and a 600-token prompt continued by 30 tokens
    at start_pos 600 on small-q4km, logits and the last layer's K/V rows
    bit-exact against the oracle."""
    monkeypatch.setenv("RLH_QK_PRE_GRID", grid_only)
    spec, tensors, m, om = _get("tiny-g4-q4km")
    prompt = rlh.synth_tokens(91, 4300, spec.vocab)
    c = m.new_cache(4400)
    oc = om.new_cache(4400)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg)), f"logits differ (rel {rel_l2(lg, rg):.2e})"
    c.close()
    oc.close()
    spec, tensors, m, om = _get("small-q4km")
    prompt = rlh.synth_tokens(92, 600, spec.vocab)
    more = rlh.synth_tokens(93, 30, spec.vocab)
    c = m.new_cache(700)
    oc = om.new_cache(700)
    assert np.array_equal(bits(c.forward_into(prompt, 0)), bits(oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)))
    assert np.array_equal(bits(c.forward_into(more, 600)), bits(oc.forward_into(more, 600, oracle.MODE_BATCH_INT)))
    l = spec.n_layer - 1
    for which in (0, 1):
        assert np.array_equal(bits(c.read_kv(l, which, 630)), bits(oc.read_kv(l, which, 630)))
    c.close()
    oc.close()


def test_nan_logits_argmax_semantics():
    """NaN logits: every 8th row of the untied output matrix has a NaN Q6_K
    scale, so every logits block starts with a NaN row and logits[0] is NaN.
    The device greedy argmax follows main.rs:453-463 (NaN never wins) in the
    standalone argmax and in the fused greedy loop, and rlh_sample_next's
    greedy fast path follows sampler.rs:62-70 (index 0 kept when logits[0]
    is NaN), both as the oracle."""
    spec = rlh.SPECS["tiny-q4km-untied"]
    tensors = rlh.synth_model(spec, 4321)
    for kind, layer, ty, cols, rows, buf in tensors:
        if kind == rlh.T_OUTPUT:
            assert ty == rlh.Q6_K
            rb = rlh.row_bytes(ty, cols)
            for r in range(0, rows, 8):
                buf[r * rb + 208] = 0x00  # f16 NaN 0x7e00 in d of the first super-block
                buf[r * rb + 209] = 0x7E
    m = rlh.Model(spec, tensors)
    om = oracle.OracleModel(spec, tensors)
    lib = oracle.load()
    prompt = rlh.synth_tokens(8, 9, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    try:
        lg = c.forward_into(prompt, 0)
        rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
        nan = np.isnan(rg)
        assert nan[0] and nan.sum() == spec.vocab // 8
        assert np.array_equal(np.isnan(lg), nan)
        assert np.array_equal(bits(lg[~nan]), bits(rg[~nan]))
        tok = c.greedy_next()
        assert tok == lib.orc_argmax(rg.ctypes.data, len(rg)) and tok % 8 != 0
        greedy = rlh.sampling_params(temperature=0.0, repetition_penalty=1.0)
        ogreedy = oracle.SamplingParams(0.0, 40, 0.95, 1.0, 64, 1)
        s = lib.orc_sampler_create(1)
        assert c.sample_next(greedy, prompt, ctypes.c_uint64(1)) == 0
        assert lib.orc_sampler_sample(s, rg.ctypes.data, len(rg), ogreedy, prompt.ctypes.data, len(prompt)) == 0
        lib.orc_sampler_destroy(s)
        toks = c.generate_greedy(tok, 6)
        ref = [tok]
        for i in range(6):
            r = oc.forward_into(np.array([ref[-1]], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
            ref.append(lib.orc_argmax(r.ctypes.data, len(r)))
        assert list(map(int, toks)) == ref
    finally:
        c.close()
        oc.close()
        m.close()
        om.close()


def test_qwen2_biases_bit_exact():
    """q/k/v biases (Qwen2, model.rs:444-464 prefill and 626-640 decode): added
    after the products, before QK-norm and RoPE; prefill and decode logits
    bit-exact against the oracle."""
    spec = rlh.SPECS["tiny-q4km"]
    tensors = rlh.synth_model(spec, 606)
    lib = rlh.load()
    qd, kvd = spec.n_head * spec.head_dim, spec.n_head_kv * spec.head_dim
    for layer in range(spec.n_layer):
        for kind, n in ((rlh.T_ATTN_Q_BIAS, qd), (rlh.T_ATTN_K_BIAS, kvd), (rlh.T_ATTN_V_BIAS, kvd)):
            v = np.empty(n, np.float32)
            lib.rlh_synth_normal(606, rlh.tensor_id(kind, layer), 0, n, 0.0, 0.5, v.ctypes.data)
            tensors.append((kind, layer, rlh.F32, n, 1, v.view(np.uint8)))
    m = rlh.Model(spec, tensors)
    om = oracle.OracleModel(spec, tensors)
    olib = oracle.load()
    prompt = rlh.synth_tokens(607, 13, spec.vocab)
    c = m.new_cache(32)
    oc = om.new_cache(32)
    try:
        lg = c.forward_into(prompt, 0)
        rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
        assert np.array_equal(bits(lg), bits(rg))
        # without the biases the logits differ (the biases are applied)
        m0 = rlh.Model(spec, [t for t in tensors if t[0] < rlh.T_ATTN_Q_BIAS])
        c0 = m0.new_cache(32)
        assert not np.array_equal(bits(c0.forward_into(prompt, 0)), bits(lg))
        c0.close()
        m0.close()
        tok = olib.orc_argmax(rg.ctypes.data, len(rg))
        for i in range(5):
            lg = c.forward_into(np.array([tok], np.uint32), len(prompt) + i)
            rg = oc.forward_into(np.array([tok], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
            assert np.array_equal(bits(lg), bits(rg)), f"decode step {i} logits differ"
            tok = olib.orc_argmax(rg.ctypes.data, len(rg))
    finally:
        c.close()
        oc.close()
        m.close()
        om.close()


@pytest.mark.parametrize("n_prompt", [1100, 4100])
def test_softmax_walk_replays_bit_exact(n_prompt, monkeypatch):
    """The decode softmax's exact parallel sum (rows of 1024 positions or
    more; 8 query heads per KV head take k_attn_softmax) with its replay
    paths forced by RLH_SOFTMAX_WALK_SHIFT, which moves the runs' predicted
    binades: 1 every run's one up, 2 one down (every run is replayed from
    its exact start, a walk pass per run, stops at every lane of a 64-run
    group including the last), 3 every third run's one up (scans that pass
    two runs, then stop). The sum, and so every logit, must not change:
    bit-exact against the oracle's sequential loop in every mode, six decode
    steps each, and equal to the unforced run."""
    print(f"softmax walk replays, prompt {n_prompt}", flush=True)
    spec, tensors, m, om = _get("tiny-g8-q4km")
    prompt = rlh.synth_tokens(78, n_prompt, spec.vocab)
    max_ctx = n_prompt + 16
    lib = oracle.load()
    oc = om.new_cache(max_ctx)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    toks, refs = [lib.orc_argmax(rg.ctypes.data, len(rg))], []
    for i in range(6):
        rg = oc.forward_into(np.array([toks[-1]], np.uint32), n_prompt + i, oracle.MODE_DEFAULT)
        refs.append(rg)
        toks.append(lib.orc_argmax(rg.ctypes.data, len(rg)))
    oc.close()
    for mode in ("0", "1", "2", "3"):
        print(f"  walk shift mode {mode}", flush=True)
        monkeypatch.setenv("RLH_SOFTMAX_WALK_SHIFT", mode)
        c = m.new_cache(max_ctx)
        try:
            c.forward_into(prompt, 0)
            for i in range(6):
                lg = c.forward_into(np.array([toks[i]], np.uint32), n_prompt + i)
                assert np.array_equal(bits(lg), bits(refs[i])), \
                    f"mode {mode} step {i}: logits differ (rel {rel_l2(lg, refs[i]):.2e})"
        finally:
            c.close()
