"""The exact parallel evaluation of sequential f32 sums and differences
(llama.rs_amd/csrc/monosum.h), as the device sampler's chains run it
(wave_chain, k_run_pairs + k_run_walk in sampler_dev.hip), against the plain
sequential loop. CPU only.

The reference adds non-negative f32 terms one after another in three places
the device sampler restates: the softmax sum over the vocabulary in index
order (ops.rs:411-414), the top-p running sum over the sorted probabilities
(sampler.rs:137-145) and the draw's running difference (sampler.rs:154-160).
The device evaluates each as passes of a scan over increment pairs; the shim
runs those passes on the CPU with the device's lane, term and run counts and
with small ones that force many restarts, on data chosen to hit every branch:
ties to even at the binade spacing (terms with few mantissa bits), binade
crossings by one large term, sums through the subnormal region, zeros, powers
of two as starting values of a difference, and terms far above the sum."""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))

pytestmark = pytest.mark.skipif(not shutil.which("g++"), reason="needs g++")

F32P = ctypes.POINTER(ctypes.c_float)


@pytest.fixture(scope="module")
def shim(tmp_path_factory):
    out = tmp_path_factory.mktemp("mono") / "libmono_shim.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-shared", "-o", str(out),
                    os.path.join(HERE, "monosum_shim.cpp")], check=True)
    lib = ctypes.CDLL(str(out))
    lib.shim_seq.restype = ctypes.c_uint32
    lib.shim_seq.argtypes = [ctypes.c_int, F32P, ctypes.c_uint32, ctypes.c_float, ctypes.c_int, ctypes.c_float, F32P]
    lib.shim_chain.restype = ctypes.c_uint32
    lib.shim_chain.argtypes = [ctypes.c_int, F32P, ctypes.c_uint32, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_float, F32P, ctypes.POINTER(ctypes.c_uint64)]
    lib.shim_softwalk.restype = ctypes.c_uint32
    lib.shim_softwalk.argtypes = [F32P, ctypes.c_uint32, ctypes.c_int, F32P, ctypes.POINTER(ctypes.c_uint64)]
    lib.shim_runwalk.restype = ctypes.c_uint32
    lib.shim_runwalk.argtypes = [ctypes.c_int, F32P, ctypes.c_uint32, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_float, ctypes.c_int, F32P, ctypes.POINTER(ctypes.c_uint64),
                                 ctypes.POINTER(ctypes.c_uint64)]
    return lib


def _run(shim, dec, y, s0, stop, thr, T, E, runwalk=None):
    """Sequential loop vs the device algorithm: wave_chain with T lanes of E
    terms, or (runwalk = (R, cu_shift)) the run walk with T runs of R terms."""
    y = np.ascontiguousarray(y, np.float32)
    p = y.ctypes.data_as(F32P)
    v1, v2 = ctypes.c_float(), ctypes.c_float()
    passes, misses = ctypes.c_uint64(), ctypes.c_uint64()
    j1 = shim.shim_seq(dec, p, len(y), s0, stop, thr, ctypes.byref(v1))
    if runwalk is None:
        j2 = shim.shim_chain(dec, p, len(y), s0, T, E, stop, thr, ctypes.byref(v2), ctypes.byref(passes))
    else:
        R, shift = runwalk
        j2 = shim.shim_runwalk(dec, p, len(y), s0, T, R, stop, thr, shift, ctypes.byref(v2), ctypes.byref(passes),
                               ctypes.byref(misses))
    b1 = np.float32(v1.value).view(np.uint32)
    b2 = np.float32(v2.value).view(np.uint32)
    return j1, j2, b1, b2, passes.value


# (lanes, terms per lane): the device's one-wave chains use 64 lanes with 1
# or 4 terms; the others force many restarts
SHAPES = [(64, 1), (64, 4), (8, 4), (3, 1), (1024, 16)]
# (runs per pass, terms per run, candidate shift): the device's walk is
# (128, 64, 0); shifted candidates force replays of runs whose window misses
RUNWALKS = [(128, 64, 0), (64, 64, 0), (4, 8, 0), (128, 64, 5), (2, 16, -3)]


def _softmax_terms(rng, n, scale):
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    return np.exp(x - x.max()).astype(np.float32)


def _few_bits(rng, n, lo, hi):
    """Terms m * 2^e with m < 16: sums of them hit exact half-spacing ties."""
    m = rng.integers(0, 16, n)
    e = rng.integers(lo, hi, n)
    return np.ldexp(m.astype(np.float64), e).astype(np.float32)


def _cases():
    rng = np.random.default_rng(2026)
    out = []
    for scale in (0.5, 2.0, 8.0, 30.0):
        out.append(("softmax%g" % scale, _softmax_terms(rng, 20000, scale)))
    out.append(("fewbits", _few_bits(rng, 20000, -30, -10)))
    out.append(("fewbits_wide", _few_bits(rng, 20000, -60, 0)))
    out.append(("subnormal", _few_bits(rng, 5000, -149, -120)))
    z = _few_bits(rng, 6000, -40, -20)
    z[rng.random(6000) < 0.5] = 0.0
    out.append(("zeros", z))
    big = _few_bits(rng, 5000, -40, -20)
    big[rng.integers(0, 5000, 20)] = np.float32(3e30)
    out.append(("jumps", big))
    out.append(("ones", np.ones(40000, np.float32)))
    out.append(("halfulp", np.full(5000, np.float32(2.0 ** -24))))
    return out


@pytest.mark.parametrize("T,E", SHAPES)
def test_sum_equals_sequential(shim, T, E):
    for name, y in _cases():
        j1, j2, b1, b2, passes = _run(shim, 0, y, 0.0, 0, 0.0, T, E)
        assert (j1, b1) == (j2, b2), name
        assert passes <= len(y) + 1, name


@pytest.mark.parametrize("T,R,shift", RUNWALKS)
def test_run_walk_equals_sequential(shim, T, R, shift):
    """The long-chain form: sums, running sums to a threshold and draws."""
    rng = np.random.default_rng(T * 100 + R + shift)
    for name, y in _cases():
        j1, j2, b1, b2, _ = _run(shim, 0, y, 0.0, 0, 0.0, T, 0, (R, shift))
        assert (j1, b1) == (j2, b2), name
        p = np.sort(y / np.float32(max(float(y.sum()), 1e-30)))[::-1].astype(np.float32)
        for thr in (0.3, 0.95, 0.999, 2.0):
            j1, j2, b1, b2, _ = _run(shim, 0, p, 0.0, 1, thr, T, 0, (R, shift))
            assert (j1, b1) == (j2, b2), (name, thr)
        total = np.float32(0)
        for v in p:
            total = np.float32(total + v)
        for s0 in [float(np.float32(rng.random()) * total) for _ in range(3)] + [float(total), 0.0, 0.5]:
            j1, j2, b1, b2, _ = _run(shim, 1, p, s0, 2, 0.0, T, 0, (R, shift))
            assert (j1, b1) == (j2, b2), (name, s0)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_softmax_walk_equals_sequential(shim, mode):
    """The attention softmax's sum (block_softmax_sum in attention.hip):
    256 runs with pairs at predicted binades, scanned 64 at a time, the
    first miss replayed with f32 adds (modes 1-3 shift every prediction to
    force replays): equal bits to the plain loop; with true predictions
    few runs are replayed."""
    rng = np.random.default_rng(11)
    extra = [("softmax_4k%g" % sc, _softmax_terms(rng, 4160, sc)) for sc in (0.5, 4.0, 30.0)]
    for name, y in _cases() + extra + [("short", np.float32([0.25, 1.0, 3e-8])), ("one", np.float32([0.7]))]:
        seq = np.float32(0)
        for v in y:
            seq = np.float32(seq + v)
        out, rep = ctypes.c_float(), ctypes.c_uint64()
        nr = shim.shim_softwalk(y.ctypes.data_as(F32P), len(y), mode, ctypes.byref(out), ctypes.byref(rep))
        assert np.float32(out.value).view(np.uint32) == seq.view(np.uint32), (name, mode)
        if mode == 1:
            assert rep.value == nr, name  # every prediction misses
        if mode == 0 and name.startswith("softmax"):
            assert rep.value < nr // 8, (name, rep.value)


@pytest.mark.parametrize("T,E", SHAPES)
def test_running_sum_threshold(shim, T, E):
    """Top-p: the first index whose running sum reaches the threshold, on
    descending probabilities, and the sum there."""
    rng = np.random.default_rng(7)
    for name, y in _cases():
        p = np.sort(y / np.float32(max(float(y.sum()), 1e-30)))[::-1].astype(np.float32)
        for thr in (0.0, 0.3, 0.9, 0.95, 0.999, 1.0, 2.0):
            j1, j2, b1, b2, _ = _run(shim, 0, p, 0.0, 1, thr, T, E)
            assert (j1, b1) == (j2, b2), (name, thr)
        j1, j2, b1, b2, _ = _run(shim, 0, y, 0.0, 1, float(rng.random()), T, E)
        assert (j1, b1) == (j2, b2), name
        # thresholds equal to partial sums: the event lands exactly on them
        part = np.float32(0)
        marks = set(rng.integers(0, len(p), 6).tolist())
        for j, v in enumerate(p):
            part = np.float32(part + v)
            if j in marks and part > 0:
                j1, j2, b1, b2, _ = _run(shim, 0, p, 0.0, 1, float(part), T, E)
                assert (j1, b1) == (j2, b2), (name, j)
                assert j1 <= j


@pytest.mark.parametrize("T,E", SHAPES)
def test_draw_difference(shim, T, E):
    """The draw: r = u * sum, then r -= p_j until r <= 0, for many u, and from
    starting values that are powers of two (the binade's floor)."""
    rng = np.random.default_rng(11)
    for name, y in _cases():
        p = np.sort(y)[::-1].astype(np.float32)
        total = np.float32(0)
        for v in p[:4000]:
            total = np.float32(total + v)
        starts = [float(np.float32(rng.random()) * total) for _ in range(6)]
        starts += [float(total), 0.0, 1.0, 2.0 ** -3, 2.0 ** -126, 2.0 ** -140, 2.0 ** 20]
        for s0 in starts:
            j1, j2, b1, b2, passes = _run(shim, 1, p[:4000], s0, 2, 0.0, T, E)
            assert (j1, b1) == (j2, b2), (name, s0)
            assert passes <= 4001


def test_difference_to_exhaustion(shim):
    """Differences that never reach 0 (values far below the start) and ones
    that cross many binades one term at a time."""
    rng = np.random.default_rng(5)
    y = _few_bits(rng, 30000, -60, -30)
    for s0 in (1.0, 0.75, 2.0 ** -20):
        for T, E in SHAPES:
            j1, j2, b1, b2, _ = _run(shim, 1, y, s0, 2, 0.0, T, E)
            assert (j1, b1) == (j2, b2)
    halves = np.array([2.0 ** -k for k in range(1, 150)], np.float32)
    for T, E in SHAPES:
        j1, j2, b1, b2, _ = _run(shim, 1, halves, 1.0, 2, 0.0, T, E)
        assert (j1, b1) == (j2, b2)
        j1, j2, b1, b2, _ = _run(shim, 0, halves[::-1], 0.0, 0, 0.0, T, E)
        assert (j1, b1) == (j2, b2)


def test_landing_on_binade_edges(shim):
    """Runs whose model result lands exactly on the binade's floor (a
    difference) or top (a sum) with a fractional remainder: below a power of
    two the spacing halves, so a result the model rounds to the floor may be
    a float below it, and the run must be finished with real steps."""
    for k in (0, -10, -100, -124, -125, 20):
        ulp = 2.0 ** (k - 23)
        for j in (1, 2, 3, 5):
            for f in (0.0, 0.25, 0.5, 0.75):
                tail = [ulp / 8, 0.0, ulp / 4]
                y = np.array([(j + f) * ulp] + tail, np.float32)
                for T, E in SHAPES:
                    s0 = float(np.float32(2.0 ** k + j * ulp))
                    j1, j2, b1, b2, _ = _run(shim, 1, y, s0, 2, 0.0, T, E)
                    assert (j1, b1) == (j2, b2), (k, j, f, T, E)
                    s1 = float(np.float32(2.0 ** (k + 1) - j * ulp))
                    j1, j2, b1, b2, _ = _run(shim, 0, y, s1, 0, 0.0, T, E)
                    assert (j1, b1) == (j2, b2), (k, j, f, T, E)
                    thr = float(np.float32(2.0 ** (k + 1)))
                    j1, j2, b1, b2, _ = _run(shim, 0, y, s1, 1, thr, T, E)
                    assert (j1, b1) == (j2, b2), (k, j, f, T, E, "threshold")


def test_random_exhaustive_small(shim):
    """Brute force over short random sequences of few-bit terms, both
    directions, every shape: a mistake in the tie rule, the parity
    composition or the crossing test shows as a mismatch here."""
    rng = np.random.default_rng(99)
    for trial in range(3000):
        n = int(rng.integers(1, 40))
        lo = int(rng.integers(-149, -20))
        y = _few_bits(rng, n, lo, lo + int(rng.integers(1, 30)))
        T, E = SHAPES[trial % len(SHAPES)]
        walk = None
        if trial % 3 == 0:  # the run walk: 2 runs of 4 terms per pass
            T, walk = 2, (4, trial % 7 - 3)
        j1, j2, b1, b2, _ = _run(shim, 0, y, 0.0, 0, 0.0, T, E, walk)
        assert (j1, b1) == (j2, b2), (trial, y.tolist())
        thr = float(np.float32(y.sum() * rng.random()))
        j1, j2, b1, b2, _ = _run(shim, 0, y, 0.0, 1, thr, T, E, walk)
        assert (j1, b1) == (j2, b2), (trial, thr, y.tolist())
        s0 = float(np.float32(y.sum() * rng.random() * 1.5))
        j1, j2, b1, b2, _ = _run(shim, 1, y, s0, 2, 0.0, T, E, walk)
        assert (j1, b1) == (j2, b2), (trial, s0, y.tolist())
