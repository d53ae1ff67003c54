"""The weight types without an integer path in the reference: Q4_1, Q5_0,
Q5_1 (32-value blocks with a min and/or a fifth bit) and float rows (F16,
BF16, F32).

Decode (ops::matmul, ops.rs:67-141): Q4_1/Q5_0/Q5_1 and BF16 take
quant::dequant_dot; the AVX2 fused kernels cover F16 and F32 bytes
(simd.rs:248-258, 382-419), the other types the generic fallback
(quant.rs:528-539: one 32-value block dequantized, dot_f32_avx2 of the block,
added to the row total in block order) or the scalar chain (BF16,
quant.rs:426-433). F32 tensors take ops::dot per row (ops.rs:77-83).
Prefill (ops::matmul_batch, ops.rs:150-313): F32 tensors ops::dot per token
(ops.rs:167-175); every other type dequantizes rows and runs
dot_multi_rows::<3, 4>. Bar: bit-exact against the oracle, which restates
those paths."""
import numpy as np
import pytest

import oracle
import rlh
from helpers import BF16, F16, F32, Q4_1, Q5_0, Q5_1, bits, random_blocks

pytestmark = pytest.mark.gpu

TYPES = [Q4_1, Q5_0, Q5_1, F16, BF16, F32]
NAMES = {Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", F16: "f16", BF16: "bf16", F32: "f32"}


def _bs(ty):
    return 32 if ty in (Q4_1, Q5_0, Q5_1) else 1


@pytest.mark.parametrize("ty", TYPES, ids=[NAMES[t] for t in TYPES])
def test_dequant_bit_exact(ty):
    rng = np.random.default_rng(ty + 40)
    n = 4096
    data = random_blocks(ty, n // _bs(ty), rng)
    assert np.array_equal(bits(rlh.dequant(ty, data, n)), bits(oracle.dequant_row(ty, data, n)))


SHAPES = [(1, 256), (5, 512), (33, 2048), (100, 1024), (70, 4096), (7, 12288)]


@pytest.mark.parametrize("ty", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_bit_exact(ty, rows, cols):
    print(f"{NAMES[ty]} matvec {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + ty)
    w = random_blocks(ty, rows * cols // _bs(ty), rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(ty, w, rows, cols, x)
    ref = oracle.matmul(ty, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref)), f"max diff {np.max(np.abs(got - ref))}"


@pytest.mark.parametrize("ty", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("rows,cols,n", [(16, 256, 2), (33, 1024, 5), (20, 2048, 16), (40, 4096, 35),
                                         (64, 512, 130)])
def test_matmul_batch_bit_exact(ty, rows, cols, n):
    """Token groups of 4 (8-lane chains) and the n % 4 tail (dot_f32_avx2);
    F32 tensors: ops::dot per token."""
    print(f"{NAMES[ty]} matmul_batch {rows}x{cols} n={n}", flush=True)
    rng = np.random.default_rng(rows + cols * 3 + n + ty)
    w = random_blocks(ty, rows * cols // _bs(ty), rng)
    xs = rng.standard_normal(n * cols).astype(np.float32)
    got = rlh.matmul_batch(ty, w, rows, cols, xs, n)
    ref = oracle.matmul_batch(ty, w, rows, cols, xs, n, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("name", ["tiny-q4_1", "tiny-q5_0", "tiny-q5_1", "tiny-f16", "tiny-bf16", "tiny-f32",
                                  "tiny-mix", "tiny-longff-q5"])
def test_forward_bit_exact(name):
    """Every matrix (and the embedding / logits matrix) in one type, the mix
    of eight types, or Q4_1/Q5_0/Q5_1 with a 13056-wide FFN (ffn_down takes
    the ring plan in decode): prefill of 11 tokens (3 in the n % 4 tail),
    then decode with greedy tokens; the KV cache afterwards."""
    print(f"forward {name}", flush=True)
    spec = rlh.SPECS[name]
    tensors = rlh.synth_model(spec, 777)
    m = rlh.Model(spec, tensors)
    om = oracle.OracleModel(spec, tensors)
    prompt = rlh.synth_tokens(91, 11, spec.vocab)
    c = m.new_cache(64)
    oc = om.new_cache(64)
    lg = c.forward_into(prompt, 0)
    rg = oc.forward_into(prompt, 0, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(lg), bits(rg))
    lib = oracle.load()
    tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    for i in range(5):
        lg = c.forward_into(np.array([tok], np.uint32), len(prompt) + i)
        rg = oc.forward_into(np.array([tok], np.uint32), len(prompt) + i, oracle.MODE_DEFAULT)
        assert np.array_equal(bits(lg), bits(rg)), f"decode step {i}"
        tok = lib.orc_argmax(rg.ctypes.data, len(rg))
    n = len(prompt) + 5
    for l in range(spec.n_layer):
        for which in (0, 1):
            assert np.array_equal(bits(c.read_kv(l, which, n)), bits(oc.read_kv(l, which, n)))
    c.close()
    oc.close()
    m.close()
