"""librlh's expf restatements against the C library's expf (CPU only).

The reference calls the platform expf through f32::exp (softmax_inplace,
ops.rs:410; silu, ops.rs:394). librlh restates glibc's expf (x86-64 FMA
variant) twice: the AVX2 path of the host sampler's softmax and
expf_glibc_t in expf_glibc.h, the source the kernels compile. Both are
compared bit for bit with the C library over all 2^32 float bit patterns
(normal, subnormal and zero inputs, results that overflow, underflow or are
subnormal, +-inf and NaN), after a few values every correct expf has.
"""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.dirname(os.path.abspath(__file__))


def _has_avx2_fma():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return " avx2" in flags and " fma" in flags


pytestmark = pytest.mark.skipif(not (_has_avx2_fma() and shutil.which("g++")),
                                reason="needs an AVX2+FMA host and g++")


@pytest.fixture(scope="module")
def shim(tmp_path_factory):
    out = tmp_path_factory.mktemp("expf") / "libexpf_shim.so"
    # the flags librlh's host objects are built with (llama.rs_amd/Makefile)
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-shared", "-o", str(out),
                    os.path.join(HERE, "expf_shim.cpp"), "-lpthread", "-lm"], check=True)
    lib = ctypes.CDLL(str(out))
    lib.shim_expf.restype = ctypes.c_float
    lib.shim_expf.argtypes = [ctypes.c_float, ctypes.c_int]
    lib.shim_expf_mismatches.restype = ctypes.c_uint64
    lib.shim_expf_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_uint64)]
    return lib


def _bits(v):
    return int(np.array([v], np.float32).view(np.uint32)[0])


@pytest.mark.parametrize("which", [0, 1, 2])
def test_known_values(shim, which):
    """Facts of expf itself, so that the comparison below cannot pass on two
    wrong functions that agree: exp(0) = 1, exp(-inf) = 0, exp(inf) = inf,
    overflow above 88.73 and underflow to 0 below -103.98, NaN stays NaN,
    exp(1) and exp(-87.5) within one ulp of the f64 value (the latter
    subnormal-adjacent), and exp(-100) a subnormal."""
    f = lambda x: shim.shim_expf(x, which)  # noqa: E731
    assert _bits(f(0.0)) == _bits(np.float32(1.0))
    assert _bits(f(-0.0)) == _bits(np.float32(1.0))
    assert f(float("-inf")) == 0.0
    assert f(float("inf")) == float("inf")
    assert f(89.0) == float("inf")
    assert f(-104.0) == 0.0
    assert np.isnan(f(float("nan")))
    for x in (1.0, -87.5, 10.0, -0.5):
        ref = np.float32(np.exp(np.float64(x)))
        assert abs(_bits(np.float32(f(x))) - _bits(ref)) <= 1, x
    v = np.float32(f(-100.0))
    assert 0.0 < v < np.finfo(np.float32).tiny


@pytest.mark.parametrize("which", [0, 1])
def test_every_float_matches_the_c_library(shim, which):
    """All 2^32 bit patterns: identical bits (any NaN for NaN)."""
    nthreads = max(1, min(16, len(os.sched_getaffinity(0))))
    first = ctypes.c_uint64()
    bad = shim.shim_expf_mismatches(0, 1 << 32, which, nthreads, ctypes.byref(first))
    assert bad == 0, f"{bad} mismatches, first at bit pattern {first.value:#010x}"
