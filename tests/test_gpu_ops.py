"""Op-level parity: HIP kernels (through the C ABI) against the CPU oracle.

Bars: bit-exact for dequantisation, Q8 activation blocks and integer block
dots (the required bar), and bit-exact for the matvec rows too (the kernel
sums the per-group terms in the reference order).
"""
import numpy as np
import pytest

import oracle
import rlh
from helpers import Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, BLOCK, bits, random_activation, random_blocks

pytestmark = pytest.mark.gpu

TYPES = [Q4_K, Q6_K, Q8_0, Q4_0]


@pytest.mark.parametrize("kind", ["normal", "ties", "sparse"])
@pytest.mark.parametrize("n", [32, 256, 4096, 12288])
def test_quantize_q8_bit_exact(n, kind):
    print(f"quantize_q8 n={n} kind={kind}", flush=True)
    rng = np.random.default_rng(n + len(kind))
    x = random_activation(n, rng, kind)
    got = rlh.quantize_q8(x)
    ref = oracle.quantize_q8(x, mode=1)  # AVX2 rounding (ties to even)
    for g, r, name in zip(got, ref, ["qs", "scales", "sums", "sums16"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(r).view(np.uint8)), name


def test_quantize_q8_zero_block():
    x = np.zeros(64, np.float32)
    x[40] = -3.0
    qs, d, s, s16 = rlh.quantize_q8(x)
    assert d[0] == 0.0 and not qs[:32].any() and s[0] == 0
    rq, rd, rs, rs16 = oracle.quantize_q8(x, mode=1)
    assert np.array_equal(qs, rq) and np.array_equal(bits(d), bits(rd))


@pytest.mark.parametrize("ty", TYPES + [0, 1])
def test_dequant_bit_exact(ty):
    print(f"dequant ty={ty}", flush=True)
    rng = np.random.default_rng(ty)
    bs, ts = BLOCK[ty]
    n = 4096
    if ty == 0:
        data = rng.standard_normal(n).astype(np.float32).view(np.uint8)
    elif ty == 1:
        data = rng.standard_normal(n).astype(np.float16).view(np.uint8)
    else:
        data = random_blocks(ty, n // bs, rng)
    got = rlh.dequant(ty, data, n)
    ref = oracle.dequant_row(ty, data, n)
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("rows,cols", [(3, 256), (17, 1024), (64, 4096)])
def test_block_dots_exact(ty, rows, cols):
    print(f"block_dots ty={ty} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * cols + ty)
    bs, ts = BLOCK[ty]
    w = random_blocks(ty, rows * cols // bs, rng)
    qs, _, _, _ = oracle.quantize_q8(rng.standard_normal(cols).astype(np.float32), mode=1)
    got = rlh.block_dots(ty, w, rows, cols, qs)
    ref = oracle.block_dots(ty, w, rows, cols, qs)
    assert np.array_equal(got, ref)


# Shapes of the Qwen3 matrices (0.6B .. 32B) at reduced row counts plus odd
# row counts that leave partial row blocks.
SHAPES = [(1, 256), (5, 512), (16, 1024), (33, 2048), (100, 2560), (64, 3072), (48, 4096), (7, 9728),
          (20, 12288), (9, 25600)]


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_bit_exact(ty, rows, cols):
    print(f"matvec ty={ty} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows + cols + ty)
    bs, ts = BLOCK[ty]
    w = random_blocks(ty, rows * cols // bs, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(ty, w, rows, cols, x)
    ref = oracle.matmul(ty, w, rows, cols, x, oracle.MODE_DEFAULT)  # AVX2 integer path
    assert np.array_equal(bits(got), bits(ref)), f"max diff {np.max(np.abs(got - ref))}"


def test_matvec_large_rows():
    """A full 8B-size ffn_down-like matrix (4096 x 12288, Q6_K)."""
    rng = np.random.default_rng(5)
    rows, cols = 4096, 12288
    w = random_blocks(Q6_K, rows * cols // 256, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(Q6_K, w, rows, cols, x)
    ref = oracle.matmul(Q6_K, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref))


def test_matvec_32b_ffn_down_shape():
    """The 32B ffn_down (5120 x 25600, Q6_K): whole-row terms would leave one
    block per CU and 320 blocks, so the launch takes the ring plan (two rounds
    of four producers' tiles in LDS, chained by wave 0 as they complete)."""
    rng = np.random.default_rng(6)
    rows, cols = 5120, 25600
    w = random_blocks(Q6_K, rows * cols // 256, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(Q6_K, w, rows, cols, x)
    ref = oracle.matmul(Q6_K, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref))


# Ring plans forced on small shapes (RLH_MV_RING=1; at most seven producer
# waves): one round (2048-4096 values), three rounds with a short last one
# and a slot reused (9728: 19 tiles of 2 items over 7 producers), two rounds
# (12288: 12 tiles), four rounds with a four-tile last round (25600: 25
# tiles), for every tiled type (Q5_K and the 32-value types through their
# f32 products).
RING_TYPES = [Q4_K, Q6_K, Q8_0, Q4_0, Q5_K, Q4_1, Q5_0, Q5_1]


@pytest.mark.parametrize("ty", RING_TYPES)
@pytest.mark.parametrize("rows,cols", [(33, 2048), (100, 2560), (48, 4096), (7, 9728), (20, 12288), (9, 25600)])
def test_matvec_ring_plan_bit_exact(ty, rows, cols, monkeypatch):
    print(f"ring matvec ty={ty} {rows}x{cols}", flush=True)
    monkeypatch.setenv("RLH_MV_RING", "1")
    rng = np.random.default_rng(rows * 3 + cols + ty)
    bs, ts = BLOCK[ty]
    w = random_blocks(ty, rows * cols // bs, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(ty, w, rows, cols, x)
    ref = oracle.matmul(ty, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref)), f"max diff {np.max(np.abs(got - ref))}"


@pytest.mark.parametrize("ty", [Q4_1, Q5_0, Q5_1, Q5_K])
@pytest.mark.parametrize("rows,cols", [(300, 13056), (130, 25600), (70, 27648)])
def test_matvec_long_rows_f32_types(ty, rows, cols):
    """Rows of the f32-product types (quant.rs:528-539: every block
    dequantized, then dot_f32_avx2 against the f32 activation) longer than
    12288 values: the f32 row staged in LDS and the row's whole terms no
    longer fit together, so the launch stages no Q8 row (these types never
    read it) and takes a ring plan on its own (no RLH_MV_RING). 13056 values
    are 51 super-blocks (one item per tile, 51 tiles per row), 25600 the 32B
    FFN width, 27648 the Qwen2.5-32B FFN width. Bit-exact."""
    print(f"long-row matvec ty={ty} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows + cols + 7 * ty)
    bs, ts = BLOCK[ty]
    w = random_blocks(ty, rows * cols // bs, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = rlh.matvec(ty, w, rows, cols, x)
    ref = oracle.matmul(ty, w, rows, cols, x, oracle.MODE_DEFAULT)
    assert np.array_equal(bits(got), bits(ref)), f"max diff {np.max(np.abs(got - ref))}"


def test_matvec_rejects_bad_shape():
    w = np.zeros(144, np.uint8)
    with pytest.raises(rlh.RlhError) as e:
        rlh.matvec(Q4_K, w, 1, 100, np.zeros(100, np.float32))
    assert e.value.code == rlh.RLH_EINVAL
