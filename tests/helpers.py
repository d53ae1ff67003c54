"""Shared input generators for the parity tests."""
import numpy as np

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
BLOCK = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 0: (1, 4), 1: (1, 2), 30: (1, 2)}


class Lcg:
    """The reference tests' byte generator (simd.rs:1055-1067)."""

    def __init__(self, seed):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def u8(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        return (self.s >> 33) & 0xFF

    def f32(self):
        return np.float32(np.float32(self.u8()) / np.float32(255.0) * np.float32(2.0) - np.float32(1.0))


def f16_bits(v):
    return np.array([v], np.float16).view(np.uint16)[0]


def random_blocks(ty, nblocks, rng, scale_lo=0.01, scale_hi=1.0):
    """Random block bytes with finite, positive f16 scale fields."""
    bs, ts = BLOCK[ty]
    raw = rng.integers(0, 256, size=nblocks * ts, dtype=np.uint8).reshape(nblocks, ts)

    def put(col, vals):
        h = np.asarray(vals, np.float16).view(np.uint16)
        raw[:, col] = (h & 0xFF).astype(np.uint8)
        raw[:, col + 1] = (h >> 8).astype(np.uint8)

    n = nblocks
    if ty in (0, 1, 30):  # float rows: N(0, 1) values, rounded to the type
        v = rng.standard_normal(nblocks).astype(np.float32)
        if ty == 0:
            return v.view(np.uint8).copy()
        if ty == 1:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    if ty in (3, 7):  # Q4_1 / Q5_1: d and m
        put(0, rng.uniform(scale_lo, scale_hi, n) / 16)
        put(2, rng.uniform(-scale_hi, scale_hi, n))
    elif ty == 6:  # Q5_0
        put(0, rng.uniform(scale_lo, scale_hi, n) / 16)
    elif ty in (Q4_K, Q5_K):
        put(0, rng.uniform(scale_lo, scale_hi, n) / 64)
        put(2, rng.uniform(scale_lo, scale_hi, n) / 64)
    elif ty == Q6_K:
        put(208, rng.uniform(scale_lo, scale_hi, n) / 64)
    elif ty in (Q8_0, Q4_0):
        put(0, rng.uniform(scale_lo, scale_hi, n) / 16)
    return raw.reshape(-1)


def random_activation(n, rng, kind="normal"):
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float32)
    if kind == "ties":
        # values landing exactly on .5 after scaling by 127/amax: the block
        # amax is 127 so inv = 1 and x*inv hits the tie exactly.
        x = (rng.integers(-254, 255, n) / 2.0).astype(np.float32)
        x[::32] = 127.0
        return x
    if kind == "sparse":
        x = np.zeros(n, np.float32)
        x[rng.integers(0, n, max(1, n // 64))] = rng.standard_normal(max(1, n // 64)).astype(np.float32)
        return x
    raise ValueError(kind)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


class HipBuffers:
    """Device buffers through libamdhip64 (ctypes), for entry points that take
    device addresses. Copies are synchronous."""

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.h = ctypes.CDLL("libamdhip64.so")
        self.bufs = []

    def malloc(self, nbytes):
        p = self.ct.c_void_p()
        assert self.h.hipMalloc(self.ct.byref(p), self.ct.c_size_t(max(nbytes, 4))) == 0
        self.bufs.append(p)
        return p

    def h2d(self, dst, arr):
        a = np.ascontiguousarray(arr)
        assert self.h.hipMemcpy(dst, a.ctypes.data_as(self.ct.c_void_p), self.ct.c_size_t(a.nbytes), 1) == 0

    def d2h(self, src, n, dtype=np.float32):
        out = np.zeros(n, dtype)
        if n:
            assert self.h.hipMemcpy(out.ctypes.data_as(self.ct.c_void_p), src, self.ct.c_size_t(out.nbytes), 2) == 0
        return out

    def sync(self):
        assert self.h.hipDeviceSynchronize() == 0

    def free(self):
        self.sync()
        for p in self.bufs:
            self.h.hipFree(p)
        self.bufs = []
