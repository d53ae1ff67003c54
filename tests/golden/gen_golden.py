"""Writes the committed golden fixtures of tests/golden (run from the repo root:
`python tests/golden/gen_golden.py`).

- blocks_<type>.npz: random block bytes with finite scales and their values,
  decoded by the independent numpy decoder (ggml_formats.py).
- q8_rows.npz: activation rows (normal, exact .5 ties, zero blocks) and their
  Q8 blocks from the quantiser's closed form (ties to even, as AVX2 rounds).
- int_dots.npz: int64 brute-force partial dots of weight blocks against Q8
  bytes.
- tiny_trace.npz: a 2-layer E=256 synthetic model's per-layer hidden states,
  prefill logits and 16 greedy tokens from the CPU oracle (a regression
  fixture of the oracle itself, pinned separately by test_oracle_model.py).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "llama.rs_amd"), os.path.join(ROOT, "oracle")]

from golden import ggml_formats as gf  # noqa: E402
from helpers import BLOCK, random_blocks  # noqa: E402


def blocks():
    rng = np.random.default_rng(2026)
    for name, ty in (("q4_k", 12), ("q6_k", 14), ("q8_0", 8), ("q4_0", 2)):
        bs, ts = BLOCK[ty]
        n = 2 * 256
        data = random_blocks(ty, n // bs, rng)
        np.savez_compressed(os.path.join(HERE, f"blocks_{name}.npz"), ty=ty, n=n, data=data,
                            values=gf.dequant(ty, data, n))


def q8_rows():
    rng = np.random.default_rng(17)
    normal = (rng.standard_normal(256) * 2).astype(np.float32)
    ties = (rng.integers(-254, 255, 256) / 2.0).astype(np.float32)
    ties[::32] = 127.0
    zeros = np.zeros(256, np.float32)
    zeros[40] = -1.5
    x = np.stack([normal, ties, zeros])
    out = {"x": x}
    for i in range(3):
        q, d, s, s16 = gf.quantize_q8_closed_form(x[i], "even")
        out[f"qs{i}"], out[f"d{i}"], out[f"s{i}"], out[f"s16_{i}"] = q, d, s, s16
    np.savez_compressed(os.path.join(HERE, "q8_rows.npz"), **out)


def int_dots():
    rng = np.random.default_rng(99)
    out = {}
    for name, ty in (("q4_k", 12), ("q6_k", 14), ("q8_0", 8), ("q4_0", 2)):
        bs, ts = BLOCK[ty]
        cols = 512
        w = random_blocks(ty, cols // bs, rng)
        a = rng.integers(-128, 128, cols).astype(np.int8)
        group = 16 if ty == 14 else 32
        out[f"{name}_w"] = w
        out[f"{name}_a"] = a
        out[f"{name}_dots"] = (gf.int_values(ty, w) * a.astype(np.int64)).reshape(-1, group).sum(1)
    np.savez_compressed(os.path.join(HERE, "int_dots.npz"), **out)


def tiny_trace():
    import oracle
    import rlh

    spec = rlh.SPECS["tiny-q4km"]
    tensors = rlh.synth_model(spec, 4242)
    om = oracle.OracleModel(spec, tensors)
    oc = om.new_cache(64)
    prompt = rlh.synth_tokens(4243, 12, spec.vocab)
    oc.enable_dump(len(prompt))
    logits = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    hidden = np.stack([oc.hidden(l, len(prompt)) for l in range(spec.n_layer)])
    lib = oracle.load()
    toks = [lib.orc_argmax(logits.ctypes.data, len(logits))]
    for i in range(16):
        lg = oc.forward_into(np.array([toks[-1]], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        toks.append(lib.orc_argmax(lg.ctypes.data, len(lg)))
    np.savez_compressed(os.path.join(HERE, "tiny_trace.npz"), prompt=prompt, logits=logits, hidden=hidden,
                        tokens=np.array(toks, np.uint32), seed=4242)


if __name__ == "__main__":
    blocks()
    q8_rows()
    int_dots()
    tiny_trace()
    print("golden fixtures written to", HERE)
