"""Pins the oracle's block formats, f16 conversion, Q8 activation quantiser
and integer block dots (CPU only).

Checks are independent of the oracle's code: a numpy decoder written from
the layouts (tests/golden/ggml_formats.py), brute-force integer dots in
int64, the closed form of the Q8 quantiser, and the committed golden
fixtures (tests/golden/*.npz, made by tests/golden/gen_golden.py from that
decoder). The reference ships no golden vectors of its own for this path.
"""
import os

import numpy as np
import pytest

import oracle
from golden import ggml_formats as gf
from helpers import BLOCK, Lcg, bits, random_blocks

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ALL_TYPES = [0, 1, 30, 2, 3, 6, 7, 8, 12, 13, 14]


def test_block_sizes_match_ggml():
    lib = oracle.load()
    for ty, (bs, ts) in BLOCK.items():
        assert lib.orc_type_block_size(ty) == bs
        assert lib.orc_type_size(ty) == ts
    assert lib.orc_type_block_size(99) == 0


def test_f16_every_value():
    """quant.rs:115-157: scalar and F16C conversions equal IEEE half->single
    for all 65536 bit patterns (NaNs: both NaN)."""
    lib = oracle.load()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got_s = np.array([lib.orc_f16_to_f32_scalar(int(v)) for v in h], np.float32)
    got_c = np.array([lib.orc_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got_s)[~nan], bits(want)[~nan])
    assert np.array_equal(bits(got_c)[~nan], bits(want)[~nan])
    assert np.isnan(got_s[nan]).all() and np.isnan(got_c[nan]).all()


def test_scale_min_k4_roundtrip():
    """get_scale_min_k4 (quant.rs:176-185) against the layout unpacker on
    every byte pattern position; and pack -> unpack of random 6-bit pairs."""
    lib = oracle.load()
    rng = np.random.default_rng(0)
    import ctypes

    for _ in range(200):
        q = rng.integers(0, 256, 12, dtype=np.uint8)
        sc_ref, m_ref = gf.unpack_scale_min_k4(q[None, :])
        for j in range(8):
            sc = ctypes.c_uint8()
            m = ctypes.c_uint8()
            lib.orc_get_scale_min_k4(j, q.ctypes.data, ctypes.byref(sc), ctypes.byref(m))
            assert (sc.value, m.value) == (sc_ref[0, j], m_ref[0, j])


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_dequant_matches_independent_decoder(ty):
    rng = np.random.default_rng(100 + ty)
    bs, ts = BLOCK[ty]
    n = 1024
    if ty == 0:
        data = rng.standard_normal(n).astype(np.float32).view(np.uint8)
    elif ty == 1:
        data = (rng.standard_normal(n) * 100).astype(np.float16).view(np.uint8)
    elif ty == 30:
        data = rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    else:
        data = random_blocks(ty, n // bs, rng)
        if ty in (3, 7):  # Q4_1/Q5_1 min field at bytes 2..3: finite halves
            raw = data.reshape(-1, ts)
            h = rng.uniform(-1, 1, raw.shape[0]).astype(np.float16).view(np.uint16)
            raw[:, 2] = (h & 0xFF).astype(np.uint8)
            raw[:, 3] = (h >> 8).astype(np.uint8)
        if ty in (3, 6, 7):
            raw = data.reshape(-1, ts)
            h = rng.uniform(0.01, 1, raw.shape[0]).astype(np.float16).view(np.uint16)
            raw[:, 0] = (h & 0xFF).astype(np.uint8)
            raw[:, 1] = (h >> 8).astype(np.uint8)
        if ty == 13:
            raw = data.reshape(-1, ts)
            for col in (0, 2):
                h = rng.uniform(0.001, 0.02, raw.shape[0]).astype(np.float16).view(np.uint16)
                raw[:, col] = (h & 0xFF).astype(np.uint8)
                raw[:, col + 1] = (h >> 8).astype(np.uint8)
    want = gf.dequant(ty, data, n)
    got = oracle.dequant_row(ty, data, n)
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0", "q4_0"])
def test_golden_dequant_fixture(name):
    f = np.load(os.path.join(GOLDEN, f"blocks_{name}.npz"))
    got = oracle.dequant_row(int(f["ty"]), f["data"], int(f["n"]))
    assert np.array_equal(bits(got), bits(f["values"]))


@pytest.mark.parametrize("kind", ["normal", "ties", "zeros", "single"])
def test_quantize_q8_closed_form(kind):
    """simd.rs:116-203 (AVX2, ties to even) and 206-244 (scalar, ties away)."""
    rng = np.random.default_rng(7)
    n = 1024
    if kind == "normal":
        x = (rng.standard_normal(n) * 3).astype(np.float32)
    elif kind == "ties":
        x = (rng.integers(-254, 255, n) / 2.0).astype(np.float32)
        x[::32] = 127.0
    elif kind == "zeros":
        x = np.zeros(n, np.float32)
    else:
        x = np.zeros(n, np.float32)
        x[5::32] = rng.standard_normal(n // 32).astype(np.float32)
    for mode, rounding in ((1, "even"), (2, "away")):
        got = oracle.quantize_q8(x, mode)
        want = gf.quantize_q8_closed_form(x, rounding)
        for g, w in zip(got, want):
            assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), (kind, mode)
    if kind == "ties":  # the two roundings really differ on ties
        assert not np.array_equal(oracle.quantize_q8(x, 1)[0], oracle.quantize_q8(x, 2)[0])


def test_q8_row_roundtrip_reference_invariants():
    """simd.rs:1204-1230 (q8_row_roundtrip): exact sums and |q*d - x| <= d/2."""
    rng = Lcg(55)
    x = np.array([rng.f32() * np.float32(3.0) for _ in range(256)], np.float32)
    qs, d, s, s16 = oracle.quantize_q8(x, 0)
    assert len(d) == 8 and len(qs) == 256
    q = qs.astype(np.int32).reshape(8, 32)
    assert np.array_equal(q.sum(1), s)
    assert np.array_equal(q[:, :16].sum(1), s16[0::2])
    assert np.array_equal(q[:, 16:].sum(1), s16[1::2])
    err = np.abs(q.astype(np.float32) * d[:, None] - x.reshape(8, 32)).max(1)
    assert (err <= d * 0.5 + 1e-6).all()


@pytest.mark.parametrize("ty", [12, 14, 8, 2])
def test_block_dots_brute_force(ty):
    """Integer partial dots equal int64 brute force; Q6_K also satisfies
    sum((u-32)*a) = sum(u*a) - 32*sum(a) against sums16 (simd.rs:598-663)."""
    rng = np.random.default_rng(ty)
    bs, ts = BLOCK[ty]
    cols = 1024
    w = random_blocks(ty, cols // bs, rng)
    qs, d, s, s16 = oracle.quantize_q8(rng.standard_normal(cols).astype(np.float32), 1)
    got = oracle.block_dots(ty, w, 1, cols, qs)[0]
    iv = gf.int_values(ty, w)
    a = qs.astype(np.int64)
    group = 16 if ty == 14 else 32
    want = (iv * a).reshape(-1, group).sum(1)
    assert np.array_equal(got, want)
    if ty == 14:
        signed = ((iv - 32) * a).reshape(-1, 16).sum(1)
        assert np.array_equal(signed, want - 32 * s16.astype(np.int64))


@pytest.mark.parametrize("ty", [12, 14, 8, 2])
def test_int_dot_float_combine_against_f64(ty):
    """dot_qk_q8_row (simd.rs:898-910) equals, to f32 rounding of the
    combine, sum(dequant(w)[i] * q[i] * d_block) evaluated in f64 — the exact
    value the integer path approximates with per-group roundings. A dropped
    min term, a wrong sign or a transposed scale breaks this by far more
    than the tolerance."""
    rng = np.random.default_rng(31 + ty)
    bs, ts = BLOCK[ty]
    cols = 4096
    for trial in range(5):
        w = random_blocks(ty, cols // bs, rng)
        x = rng.standard_normal(cols).astype(np.float32)
        q8 = oracle.quantize_q8(x, 1)
        got = float(oracle.dot_qk_q8_row(ty, w, q8))
        wd = gf.dequant(ty, w, cols).astype(np.float64)
        xa = q8[0].astype(np.float64) * np.repeat(q8[1].astype(np.float64), 32)
        want = float(np.dot(wd, xa))
        scale = float(np.abs(wd * xa).sum())
        assert abs(got - want) <= 2e-6 * scale, (trial, got, want)


def lcg_blocks(ty, nblocks, seed, set_scales):
    rng = Lcg(seed)
    bs, ts = BLOCK[ty]
    src = np.array([rng.u8() for _ in range(ts * nblocks)], np.uint8)
    for i in range(nblocks):
        set_scales(src[i * ts:(i + 1) * ts])
    return src, rng


def _f16le(b, off, bits16):
    b[off] = bits16 & 0xFF
    b[off + 1] = bits16 >> 8


@pytest.mark.parametrize("ty,bs,ts,seed,setter", [
    (12, 256, 144, 0x9E374B21, lambda b: (_f16le(b, 0, 0x3800), _f16le(b, 2, 0x3400))),
    (14, 256, 210, 0x51AB6E09, lambda b: _f16le(b, 208, 0x3800)),
    (2, 32, 18, 0x40E01234, lambda b: _f16le(b, 0, 0x3800)),
    (8, 32, 34, 0x80808080, lambda b: _f16le(b, 0, 0x3800)),
])
def test_reference_int_dot_tests(ty, bs, ts, seed, setter):
    """simd.rs:1232-1338 restated: integer dot vs scalar fused f32 dequant-dot
    on the reference's LCG inputs, rel 2e-2."""
    nblocks = 3 if bs == 256 else 5
    src, rng = lcg_blocks(ty, nblocks, seed, setter)
    x = np.array([rng.f32() for _ in range(bs * nblocks)], np.float32)
    lib = oracle.load()
    s = lib.orc_dequant_dot_scalar(ty, src.ctypes.data, x.ctypes.data, len(x))
    v = float(oracle.dot_qk_q8_row(ty, src, oracle.quantize_q8(x, 0)))
    assert abs(s - v) / max(abs(s), 1.0) < 0.02


@pytest.mark.parametrize("ty,bs,ts,setter", [
    (12, 256, 144, lambda b: (_f16le(b, 0, 0x3800), _f16le(b, 2, 0x3400))),
    (14, 256, 210, lambda b: _f16le(b, 208, 0x3800)),
    (8, 32, 34, lambda b: _f16le(b, 0, 0x3800)),
    (2, 32, 18, lambda b: _f16le(b, 0, 0x3800)),
])
def test_reference_fused_dot_tests(ty, bs, ts, setter):
    """simd.rs:1073-1124 restated: AVX2 fused dequant-dot vs scalar, 7 blocks,
    rel 1e-4."""
    src, rng = lcg_blocks(ty, 7, 0x12345678, setter)
    x = np.array([rng.f32() for _ in range(bs * 7)], np.float32)
    lib = oracle.load()
    s = lib.orc_dequant_dot_scalar(ty, src.ctypes.data, x.ctypes.data, len(x))
    v = lib.orc_dequant_dot(ty, src.ctypes.data, x.ctypes.data, len(x))
    assert abs(s - v) / max(abs(s), 1.0) < 1e-4


def test_split_dequant_q4k_matches_scalar():
    """simd.rs:1340-1368: AVX2 split dequant equals scalar; other layouts and
    bad lengths fall back (return false)."""
    src, _ = lcg_blocks(12, 2, 0xD3C017, lambda b: (_f16le(b, 0, 0x3800), _f16le(b, 2, 0x3400)))
    lib = oracle.load()
    got = np.empty(512, np.float32)
    assert lib.orc_split_dequant(12, src.ctypes.data, 512, got.ctypes.data) == 1
    assert np.array_equal(bits(got), bits(oracle.dequant_row(12, src, 512)))
    tmp = np.empty(32, np.float32)
    assert lib.orc_split_dequant(8, src.ctypes.data, 32, tmp.ctypes.data) == 0
    assert lib.orc_split_dequant(12, src.ctypes.data, 100, tmp.ctypes.data) == 0


def _f32(x):
    return np.float32(x)


def _wide_q8(rng, cols):
    """Activations spread over 2^-6 .. 2^6 per 32-value block (scales of very
    different sizes), so reordering the row's float terms changes the
    rounded total in most trials."""
    x = rng.standard_normal(cols) * np.repeat(np.exp2(rng.integers(-6, 7, cols // 32)), 32)
    return oracle.quantize_q8(x.astype(np.float32), 1)


@pytest.mark.parametrize("ty", [12, 14, 8, 2])
def test_int_dot_float_combine_bit_exact(ty):
    """The integer dots' float combines in the reference's expression and
    order, restated step by step in float32 from the independent decoder's
    integers and scales, bit for bit against the oracle's row:
    Q4_K (simd.rs:556-581) total += da*(d1*i1 - mm1*sa) + db*(d2*i2 - mm2*sb)
    per 64-value group, d1 = d*sc, mm1 = dmin*m;
    Q6_K (simd.rs:612-663) total += d*sc*(ss - 32*sa)*da, left to right, in
    the order half, sub, c (16-value groups 8*half + 2*c + sub);
    Q4_0 (simd.rs:856-863) total += d*(i0 + i1 - 8*sum) as f32 * scale;
    Q8_0 (simd.rs:882-891) total += d*i as f32 * scale."""
    rng = np.random.default_rng(90 + ty)
    bs, ts = BLOCK[ty]
    cols = 2048
    for trial in range(6):
        w = random_blocks(ty, cols // bs, rng)
        qs, dsc, sums, sums16 = _wide_q8(rng, cols)
        got = oracle.dot_qk_q8_row(ty, w, (qs, dsc, sums, sums16))
        iv = gf.int_values(ty, w)
        a = qs.astype(np.int64)
        b = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, ts)
        total = _f32(0.0)
        if ty == 12:
            dot32 = (iv * a).reshape(-1, 32).sum(1)
            d = gf.f16(b[:, 0], b[:, 1])
            dmin = gf.f16(b[:, 2], b[:, 3])
            sc, m = gf.unpack_scale_min_k4(b[:, 4:16])
            for bi in range(b.shape[0]):
                for g in range(4):
                    ab = bi * 8 + 2 * g
                    d1, mm1 = _f32(d[bi] * _f32(sc[bi, 2 * g])), _f32(dmin[bi] * _f32(m[bi, 2 * g]))
                    d2, mm2 = _f32(d[bi] * _f32(sc[bi, 2 * g + 1])), _f32(dmin[bi] * _f32(m[bi, 2 * g + 1]))
                    ta = _f32(dsc[ab] * _f32(_f32(d1 * _f32(dot32[ab])) - _f32(mm1 * _f32(sums[ab]))))
                    tb = _f32(dsc[ab + 1] * _f32(_f32(d2 * _f32(dot32[ab + 1])) - _f32(mm2 * _f32(sums[ab + 1]))))
                    total = _f32(total + _f32(ta + tb))
        elif ty == 14:
            dot16 = (iv * a).reshape(-1, 16).sum(1)
            d = gf.f16(b[:, 208], b[:, 209])
            scl = b[:, 192:208].view(np.int8)
            for bi in range(b.shape[0]):
                for half in range(2):
                    for sub in range(2):
                        for c in range(4):
                            g16 = bi * 16 + half * 8 + 2 * c + sub
                            s = _f32(scl[bi, half * 8 + sub + 2 * c])
                            diff = _f32(_f32(dot16[g16]) - _f32(_f32(32.0) * _f32(sums16[g16])))
                            term = _f32(_f32(_f32(d[bi] * s) * diff) * dsc[bi * 8 + half * 4 + c])
                            total = _f32(total + term)
        else:
            dot32 = (iv * a).reshape(-1, 32).sum(1)
            d = gf.f16(b[:, 0], b[:, 1])
            for bi in range(b.shape[0]):
                i = dot32[bi] - 8 * int(sums[bi]) if ty == 2 else dot32[bi]
                total = _f32(total + _f32(_f32(d[bi] * _f32(i)) * dsc[bi]))
        assert np.float32(got).view(np.uint32) == total.view(np.uint32), (trial, got, total)


def test_rmsnorm_core_bit_exact():
    """rmsnorm_core (simd.rs:282-326) restated in float32 with FMA emulated in
    f64 (exact product, one rounding): accumulator a_m lane l takes elements
    32i + 8m + l while 32 remain, then a_0 takes whole 8-blocks, the lanes
    combine as (a0 + a1) + (a2 + a3) and the hsum tree ((A0+A4)+(A2+A6)) +
    ((A1+A5)+(A3+A7)), the scalar tail adds v*v rounded; s = 1/sqrt(ss/n +
    eps); out = (x*s)*w. Bit-exact on wide-range rows of every tail length."""
    lib = oracle.load()
    rng = np.random.default_rng(77)

    def fma(x, y, z):
        return _f32(np.float64(x) * np.float64(y) + np.float64(z))

    for n in (32, 40, 47, 64, 96, 1000, 1024, 4101):
        for trial in range(3):
            x = (rng.standard_normal(n) * np.exp2(rng.integers(-6, 7, n))).astype(np.float32)
            w = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
            acc = [[_f32(0.0)] * 8 for _ in range(4)]
            i = 0
            while i + 32 <= n:
                for mm in range(4):
                    for l in range(8):
                        v = x[i + 8 * mm + l]
                        acc[mm][l] = fma(v, v, acc[mm][l])
                i += 32
            while i + 8 <= n:
                for l in range(8):
                    acc[0][l] = fma(x[i + l], x[i + l], acc[0][l])
                i += 8
            A = [_f32(_f32(acc[0][l] + acc[1][l]) + _f32(acc[2][l] + acc[3][l])) for l in range(8)]
            ss = _f32(_f32(_f32(A[0] + A[4]) + _f32(A[2] + A[6])) + _f32(_f32(A[1] + A[5]) + _f32(A[3] + A[7])))
            while i < n:
                ss = _f32(ss + _f32(x[i] * x[i]))
                i += 1
            s = _f32(_f32(1.0) / np.sqrt(_f32(_f32(ss / _f32(n)) + _f32(1e-6))))
            want = ((x * s).astype(np.float32) * w).astype(np.float32)
            got = np.empty(n, np.float32)
            lib.orc_rmsnorm_avx2(got.ctypes.data, x.ctypes.data, w.ctypes.data, n, 1e-6)
            assert np.array_equal(bits(got), bits(want)), (n, trial)
