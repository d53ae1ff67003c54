"""Pins the oracle's ops (src/ops.rs, src/simd.rs float kernels) on the CPU:
the reference's own self-consistency tests restated with its inputs and bars,
plus f64 closed forms."""
import ctypes

import numpy as np
import pytest

import oracle
from golden import ggml_formats as gf
from helpers import Lcg, bits, random_blocks

F32 = np.float32


def P(a):
    return a.ctypes.data


def lcg_vec(rng, n):
    return np.array([rng.f32() for _ in range(n)], F32)


def test_rmsnorm_matches_scalar_reference_test():
    """simd.rs:1170-1202 (abs 1e-5, out-of-place and in place)."""
    lib = oracle.load()
    rng = Lcg(31)
    for n in [1, 7, 8, 9, 64, 128, 1024]:
        x = lcg_vec(rng, n)
        w = np.array([abs(rng.f32()) + F32(0.25) for _ in range(n)], F32)
        ss = F32(0)
        for v in x:
            ss = F32(ss + v * v)
        s = F32(1.0) / np.sqrt(F32(ss / F32(n) + F32(1e-6)))
        expect = (x * s * w).astype(F32)
        got = np.empty(n, F32)
        lib.orc_rmsnorm(P(got), P(x), P(w), n, 1e-6, 0)
        assert np.abs(expect - got).max() < 1e-5
        inplace = x.copy()
        lib.orc_rmsnorm_head(P(inplace), P(w), n, 1e-6, 0)
        assert np.abs(expect - inplace).max() < 1e-5
        # f64 closed form
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
        assert np.abs(got - ref).max() <= 4e-7 * max(1.0, np.abs(ref).max())


def test_dot_f32_matches_scalar_reference_test():
    """simd.rs:1141-1156."""
    lib = oracle.load()
    rng = Lcg(7)
    for n in [1, 7, 8, 9, 16, 33, 128]:
        a = lcg_vec(rng, n)
        b = lcg_vec(rng, n)
        s = F32(0)
        for x, y in zip(a, b):
            s = F32(s + x * y)
        v = lib.orc_dot_f32_avx2(P(a), P(b), n)
        assert abs(s - v) < 1e-4
        assert abs(v - float(np.dot(a.astype(np.float64), b))) < 1e-5


def test_saxpy_is_bit_identical_reference_test():
    """simd.rs:1370-1396: AVX2 saxpy equals the scalar mul-then-add loop."""
    lib = oracle.load()
    rng = Lcg(0x5A079911)
    for n in [1, 7, 8, 9, 64, 128, 1024]:
        dst = lcg_vec(rng, n)
        x = lcg_vec(rng, n)
        expect = (dst + (F32(0.37) * x).astype(F32)).astype(F32)
        lib.orc_saxpy_avx2(P(dst), 0.37, P(x), n)
        assert np.array_equal(bits(dst), bits(expect))


def test_dot_multi_wide_matches_sequential_reference_test():
    """simd.rs:1398-1419."""
    lib = oracle.load()
    rng = Lcg(0xD07C417E)
    cols, n = 1024, 13
    buf = lcg_vec(rng, cols)
    xs = lcg_vec(rng, n * cols)
    got = np.zeros(n, F32)
    lib.orc_dot_multi(P(buf), cols, P(xs), 0, cols, n, P(got), 1)
    for k in range(n):
        s = np.dot(buf.astype(np.float64), xs[k * cols:(k + 1) * cols])
        assert abs(got[k] - s) / max(abs(s), 1.0) < 1e-4


def test_dot_multi_rows_matches_serial_bits_reference_test():
    """simd.rs:1421-1484: the RB=3/TB=4 row-blocked kernel is bit-identical
    to one-row-at-a-time dot_multi."""
    lib = oracle.load()
    rng = np.random.default_rng(0x5EED1234)
    for cols in [1024, 3072]:
        for n in [1, 2, 3, 5, 13, 32]:
            for rows in [1, 3, 4, 5, 9, 11]:
                xs = rng.uniform(-1, 1, n * cols).astype(F32)
                w = rng.uniform(-1, 1, rows * cols).astype(F32)
                want = np.zeros(n * rows, F32)
                got = np.zeros(n * rows, F32)
                for r in range(rows):
                    row = np.ascontiguousarray(w[r * cols:(r + 1) * cols])
                    lib.orc_dot_multi(P(row), cols, P(xs), 0, cols, n, want.ctypes.data + 4 * r, rows)
                bufs = np.zeros(3 * cols, F32)
                r = 0
                while r < rows:
                    cnt = min(3, rows - r)
                    bufs[:] = 0
                    bufs[:cnt * cols] = w[r * cols:(r + cnt) * cols]
                    lib.orc_dot_multi_rows_3_4(P(bufs), cols, P(xs), n, cnt, got.ctypes.data + 4 * r, rows)
                    r += cnt
                assert np.array_equal(bits(want), bits(got)), (cols, n, rows)


def test_matmul_batch_matches_sequential_reference_test():
    """ops.rs:478-517 (F32 fast path)."""
    rows, cols, n = 17, 40, 5
    w = np.array([((i * 2654435761 % 1000) / 1000.0) - 0.5 for i in range(rows * cols)], F32)
    xs = np.array([((i * 40503 % 1000) / 1000.0) - 0.5 for i in range(n * cols)], F32)
    batched = oracle.matmul_batch(0, w.view(np.uint8), rows, cols, xs, n)
    for k in range(n):
        y = oracle.matmul(0, w.view(np.uint8), rows, cols, xs[k * cols:(k + 1) * cols])
        assert np.abs(batched[k * rows:(k + 1) * rows] - y).max() < 1e-5


def test_matmul_batch_q4k_matches_scalar_reference_test():
    """ops.rs:522-573 (default f32 prefill path vs scalar dequant + dot)."""
    rows, cols, n = 6, 256, 3
    st = 0x123456789ABCDEF0
    raw = []
    for _ in range(rows * 144):
        st = (st * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        raw.append((st >> 33) & 0xFF)
    b = np.array(raw, np.uint8)
    for r in range(rows):
        b[r * 144:r * 144 + 2] = [0x00, 0x38]
        b[r * 144 + 2:r * 144 + 4] = [0x00, 0x34]
    xs = np.array([((i * 40503 % 1000) / 1000.0) - 0.5 for i in range(n * cols)], F32)
    # default mode only, as the reference test runs (BATCH_INT unset); the
    # integer batch path is pinned by test_batch_int_equals_sequential_int_matmul
    for mode in (oracle.MODE_DEFAULT,):
        batched = oracle.matmul_batch(12, b, rows, cols, xs, n, mode)
        for k in range(n):
            for r in range(rows):
                row = oracle.dequant_row(12, b[r * 144:(r + 1) * 144], cols)
                s = float(np.dot(row.astype(np.float64), xs[k * cols:(k + 1) * cols]))
                assert abs(batched[k * rows + r] - s) / max(abs(s), 1.0) < 0.02


@pytest.mark.parametrize("ty", [12, 14, 8, 2])
def test_batch_int_equals_sequential_int_matmul(ty):
    """BATCH_INT matmul_batch (ops.rs:192-236) runs the same integer dot per
    (row, token) as matmul (ops.rs:93-128): bit-identical."""
    rng = np.random.default_rng(ty)
    rows, cols, n = 9, 512, 4
    bs = 256 if ty in (12, 14) else 32
    w = random_blocks(ty, rows * cols // bs, rng)
    xs = rng.standard_normal(n * cols).astype(F32)
    b = oracle.matmul_batch(ty, w, rows, cols, xs, n, oracle.MODE_BATCH_INT)
    for k in range(n):
        y = oracle.matmul(ty, w, rows, cols, xs[k * cols:(k + 1) * cols])
        assert np.array_equal(bits(b[k * rows:(k + 1) * rows]), bits(y))


def _block_size(ty):
    return 256 if ty in (12, 13, 14) else (1 if ty in (0, 1, 30) else 32)


@pytest.mark.parametrize("ty,mode", [(12, 1), (14, 1), (8, 1), (13, 1), (13, 0), (3, 0), (6, 0), (7, 0), (1, 0),
                                     (30, 0), (0, 0)])
def test_no_int_matmul_against_f64(ty, mode):
    """ops.rs:131-140 fused f32 path (RUST_LLAMA_NO_INT, and the default
    mode for Q5_K, which has no integer kernel: ops.rs:93-128 skips it):
    close to the f64 dot of the weights decoded by the independent numpy
    decoder with x. Q5_K's fused kernel is the generic fallback
    (quant.rs:528-539)."""
    rng = np.random.default_rng(3 + ty + 17 * mode)
    rows, cols = 8, 1024
    w = random_blocks(ty, rows * cols // _block_size(ty), rng)
    x = rng.standard_normal(cols).astype(F32)
    y = oracle.matmul(ty, w, rows, cols, x, mode)
    wd = gf.dequant(ty, w, rows * cols).astype(np.float64).reshape(rows, cols)
    ref = wd @ x
    scale = np.abs(wd * x).sum(1)
    assert (np.abs(y - ref) <= 1e-5 * scale).all()


def test_q5k_fused_dot_is_blockwise_dequant_then_dot():
    """The Q5_K generic fallback (quant.rs:528-539) dequantizes one 256-value
    block at a time and adds ops::dot(block, x) to the row total in block
    order. Rebuilt from the independent numpy decoder's values and ops::dot
    (pinned by its own tests) it matches bit for bit, so a dropped 5th bit,
    a wrong min term or another accumulation order would fail here."""
    lib = oracle.load()
    rng = np.random.default_rng(55)
    cols = 1024
    for trial in range(4):
        w = random_blocks(13, cols // 256, rng)
        x = rng.standard_normal(cols).astype(F32)
        wd = gf.dequant(13, w, cols).astype(F32)
        y = oracle.matmul(13, w, 1, cols, x, oracle.MODE_DEFAULT)
        acc = F32(0.0)
        for b in range(cols // 256):
            wb = np.ascontiguousarray(wd[b * 256:(b + 1) * 256])
            xb = np.ascontiguousarray(x[b * 256:(b + 1) * 256])
            acc = F32(acc + F32(lib.orc_dot(P(wb), P(xb), 256)))
        assert bits(y)[0] == bits(np.array([acc], F32))[0], trial


@pytest.mark.parametrize("ty", [3, 6, 7])
def test_small_block_fused_dot_is_blockwise_dequant_then_dot(ty):
    """Q4_1/Q5_0/Q5_1 have no AVX2 kernel in the reference: dequant_dot takes
    the generic fallback (quant.rs:528-539), one 32-value block dequantized
    and ops::dot(block, x) added to the row total in block order. Rebuilt
    from the independent numpy decoder and ops::dot it matches bit for bit
    (a dropped fifth bit or min, a wrong nibble order or another
    accumulation order fails here)."""
    lib = oracle.load()
    rng = np.random.default_rng(57 + ty)
    cols = 512
    for trial in range(8):
        w = random_blocks(ty, cols // 32, rng)
        x = _wide(rng, cols)
        wd = gf.dequant(ty, w, cols).astype(F32)
        y = oracle.matmul(ty, w, 1, cols, x, oracle.MODE_DEFAULT)
        acc = F32(0.0)
        for b in range(cols // 32):
            wb = np.ascontiguousarray(wd[b * 32:(b + 1) * 32])
            xb = np.ascontiguousarray(x[b * 32:(b + 1) * 32])
            acc = F32(acc + F32(lib.orc_dot(P(wb), P(xb), 32)))
        assert bits(y)[0] == bits(np.array([acc], F32))[0], trial


def test_bf16_dot_is_the_scalar_chain():
    """BF16 weights take dequant_dot_scalar (quant.rs:426-433): acc += w * x
    in index order, the product rounded before the add; restated here with
    numpy float32 steps on the numpy decoder's values."""
    rng = np.random.default_rng(31)
    cols = 512
    for trial in range(8):
        w = random_blocks(30, cols, rng)
        x = _wide(rng, cols)
        wd = gf.dequant(30, w, cols).astype(F32)
        y = oracle.matmul(30, w, 1, cols, x, oracle.MODE_DEFAULT)
        acc = F32(0.0)
        for i in range(cols):
            acc = F32(acc + F32(wd[i] * x[i]))
        assert bits(y)[0] == bits(np.array([acc], F32))[0], trial


def _fma32(a, b, c):
    """f32 fused multiply-add: the product of two f32 values is exact in f64
    and the f64 sum is rounded once more to f32 (a double rounding that can
    only differ from the single one on an exact f32 tie, which these
    continuous random inputs do not produce)."""
    return F32(np.float64(a) * np.float64(b) + np.float64(c))


def _wide(rng, n):
    """N(0, 1) values scaled by 2^-8 .. 2^8: partial sums of very different
    magnitudes, so that a different summation order or rounding step changes
    the result in most trials."""
    return (rng.standard_normal(n) * np.exp2(rng.integers(-8, 9, n))).astype(F32)


def _tree8(A):
    return F32(F32(F32(A[0] + A[4]) + F32(A[2] + A[6])) + F32(F32(A[1] + A[5]) + F32(A[3] + A[7])))


def test_f16_dot_is_eight_fma_chains():
    """F16 weights take the AVX2 f16 kernel (simd.rs:401-419): eight FMA
    chains, lane l over elements 8i + l, then the hsum tree (simd.rs:261-272).
    Restated with f64-emulated FMA on the numpy decoder's values."""
    rng = np.random.default_rng(32)
    cols = 256
    for trial in range(8):
        w = random_blocks(1, cols, rng)
        x = _wide(rng, cols)
        wd = gf.dequant(1, w, cols).astype(F32)
        y = oracle.matmul(1, w, 1, cols, x, oracle.MODE_DEFAULT)
        A = [F32(0.0)] * 8
        for i in range(0, cols, 8):
            for l in range(8):
                A[l] = _fma32(wd[i + l], x[i + l], A[l])
        assert bits(y)[0] == bits(np.array([_tree8(A)], F32))[0], trial


def test_f32_weights_dot_is_dot_f32_avx2():
    """F32 tensors take ops::dot per row (ops.rs:77-83), dot_f32_avx2
    (simd.rs:328-377): 32 FMA chains, chain (m, l) over elements 32c + 8m + l,
    then (a0 + a1) + (a2 + a3) per lane and the hsum tree."""
    rng = np.random.default_rng(33)
    cols = 256
    for trial in range(8):
        w = rng.standard_normal(cols).astype(F32)
        x = _wide(rng, cols)
        y = oracle.matmul(0, w.view(np.uint8), 1, cols, x, oracle.MODE_DEFAULT)
        acc = [[F32(0.0)] * 8 for _ in range(4)]
        for c in range(0, cols, 32):
            for m in range(4):
                for l in range(8):
                    acc[m][l] = _fma32(w[c + 8 * m + l], x[c + 8 * m + l], acc[m][l])
        A = [F32(F32(acc[0][l] + acc[1][l]) + F32(acc[2][l] + acc[3][l])) for l in range(8)]
        assert bits(y)[0] == bits(np.array([_tree8(A)], F32))[0], trial


@pytest.mark.parametrize("ty", [13, 12, 14, 3, 6, 7, 1, 30, 0])
def test_default_matmul_batch_against_f64(ty):
    """matmul_batch's default route (ops.rs:237-312: dequantize three rows,
    dot_multi_rows over groups of four tokens; Q5_K always takes it, also
    with RUST_LLAMA_BATCH_INT; F32 tensors take ops::dot per token,
    ops.rs:167-175): close to the f64 products of the numpy decoder's
    weights, with a ragged token tail (n % 4 = 3)."""
    rng = np.random.default_rng(70 + ty)
    rows, cols, n = 7, 512, 7
    w = random_blocks(ty, rows * cols // _block_size(ty), rng)
    xs = rng.standard_normal(n * cols).astype(F32)
    wd = gf.dequant(ty, w, rows * cols).astype(np.float64).reshape(rows, cols)
    modes = (oracle.MODE_DEFAULT, oracle.MODE_BATCH_INT) if ty == 13 else (oracle.MODE_DEFAULT,)
    for mode in modes:
        ys = oracle.matmul_batch(ty, w, rows, cols, xs, n, mode).reshape(n, rows)
        for k in range(n):
            xk = xs[k * cols:(k + 1) * cols].astype(np.float64)
            ref = wd @ xk
            scale = np.abs(wd * xk).sum(1)
            assert (np.abs(ys[k] - ref) <= 1e-5 * scale).all(), (mode, k)


def test_softmax_silu_against_f64():
    lib = oracle.load()
    rng = np.random.default_rng(1)
    for n in [1, 2, 17, 1000]:
        x = (rng.standard_normal(n) * 4).astype(F32)
        y = x.copy()
        lib.orc_softmax_inplace(P(y), n)
        e = np.exp(x.astype(np.float64) - x.max())
        ref = e / e.sum()
        assert np.abs(y - ref).max() < 2e-6 * max(1.0, ref.max()) + 1e-7
    for v in [-50.0, -3.5, -1e-3, 0.0, 0.25, 2.0, 30.0]:
        s = lib.orc_silu(v)
        assert abs(s - v / (1 + np.exp(-v))) <= 2e-6 * max(1.0, abs(v))


def test_softmax_empty_and_equal():
    lib = oracle.load()
    x = np.zeros(0, F32)
    lib.orc_softmax_inplace(P(np.zeros(1, F32)), 0)
    y = np.full(8, 3.0, F32)
    lib.orc_softmax_inplace(P(y), 8)
    assert np.allclose(y, 0.125)


def test_rope_against_closed_form():
    """ops.rs:426-446: rotation of (x_i, x_{i+64}) by pos*theta^(-2i/hd);
    norms of each pair are preserved."""
    lib = oracle.load()
    rng = np.random.default_rng(4)
    hd, nh, theta = 128, 3, 1e6
    inv = np.array([F32(theta) ** F32(-2.0 * i / hd) for i in range(hd // 2)], F32)
    inv = np.array([np.float32(np.power(np.float32(theta), np.float32(np.float32(-2.0 * i) / np.float32(hd))))
                    for i in range(hd // 2)], F32)
    for pos in [0, 1, 7, 511, 4095]:
        x = rng.standard_normal(nh * hd).astype(F32)
        y = x.copy()
        lib.orc_rope_neox_freqs(P(y), nh, hd, pos, P(inv))
        for h in range(nh):
            # the angle is the f32 product pos * inv_freq (ops.rs:439)
            a = (np.float32(pos) * inv).astype(F32).astype(np.float64)
            x0 = x[h * hd:h * hd + 64].astype(np.float64)
            x1 = x[h * hd + 64:(h + 1) * hd].astype(np.float64)
            r0 = x0 * np.cos(a) - x1 * np.sin(a)
            r1 = x0 * np.sin(a) + x1 * np.cos(a)
            tol = 2e-6 * max(1.0, np.abs(x).max())
            assert np.abs(y[h * hd:h * hd + 64] - r0).max() < tol
            assert np.abs(y[h * hd + 64:(h + 1) * hd] - r1).max() < tol
        if pos == 0:
            assert np.array_equal(bits(y), bits(x))
