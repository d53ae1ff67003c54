"""Batched prefill products on int8 MFMA against the oracle's
ops::matmul_batch with RUST_LLAMA_BATCH_INT=1 (src/ops.rs:192-236).

Bar: bit-exact. Every (token, row) output is the reference's ordered f32
chain of per-block terms; only the integer block dots move to MFMA, and
they are exact. Shapes cover partial token tiles (n % 64), partial row
tiles, every tile width of the weight layout (items per row divisible by
4, 2 or 1) and the Qwen3 row lengths.
"""
import numpy as np
import pytest

import oracle
import rlh
from helpers import Q4_0, Q4_K, Q6_K, Q8_0, BLOCK, bits, random_blocks

pytestmark = pytest.mark.gpu

TYPES = [Q4_K, Q6_K, Q8_0, Q4_0]
SHAPES = [(64, 256, 2), (100, 1024, 5), (33, 2048, 64), (130, 4096, 70), (48, 12288, 17), (20, 2560, 9),
          (7, 9728, 3), (96, 768, 129), (64, 5120, 65)]


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("rows,cols,n", SHAPES)
def test_matmul_batch_bit_exact(ty, rows, cols, n):
    print(f"matmul_batch ty={ty} {rows}x{cols} n={n}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + n + ty)
    bs, _ = BLOCK[ty]
    w = random_blocks(ty, rows * cols // bs, rng)
    xs = rng.standard_normal(n * cols).astype(np.float32)
    got = rlh.matmul_batch(ty, w, rows, cols, xs, n)
    ref = oracle.matmul_batch(ty, w, rows, cols, xs, n, oracle.MODE_BATCH_INT)
    assert np.array_equal(bits(got), bits(ref))


def test_matmul_batch_equals_matvec_per_token():
    """The batched products equal n decode matvecs bit for bit (the property
    that makes batched prefill and token-by-token decode agree)."""
    rng = np.random.default_rng(5)
    rows, cols, n = 256, 4096, 40
    w = random_blocks(Q6_K, rows * cols // 256, rng)
    xs = rng.standard_normal(n * cols).astype(np.float32)
    got = rlh.matmul_batch(Q6_K, w, rows, cols, xs, n).reshape(n, rows)
    for k in (0, 17, 39):
        assert np.array_equal(bits(got[k]), bits(rlh.matvec(Q6_K, w, rows, cols, xs[k * cols:(k + 1) * cols])))
