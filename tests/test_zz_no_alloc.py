"""rlh_argmax_noalloc (the greedy argmax over device logits that allocates
nothing) through the C ABI: first under HIP stream capture (its first call in
the process, replayed as a graph with the logits changed between replays)
with the device's free memory unchanged by repeated calls; then against
rlh_greedy_next, the entry point it is a variant of: two calls in a row on
the same GPU, the second with a smaller input, each on the logits of a real
forward call; then ties, NaN and -inf rows against the oracle's main.rs
argmax; then the argument checks."""
import ctypes

import numpy as np
import pytest

import oracle
import rlh

pytestmark = pytest.mark.gpu


class _Hip:
    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.bufs = []

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.h.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)) == 0
        self.bufs.append(p)
        return p

    def h2d(self, dst, arr):
        a = np.ascontiguousarray(arr)
        assert self.h.hipMemcpy(dst, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) == 0

    def d2h_u32(self, src):
        out = np.zeros(1, np.uint32)
        assert self.h.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), src, ctypes.c_size_t(4), 2) == 0
        return int(out[0])

    def sync(self):
        assert self.h.hipDeviceSynchronize() == 0

    def free_mem(self):
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        assert self.h.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return free.value

    def free(self):
        for p in self.bufs:
            self.h.hipFree(p)
        self.bufs = []


def _noalloc(lib, hip, dev_logits, n, dev_tok):
    rc = lib.rlh_argmax_noalloc(dev_logits, n, dev_tok, None)
    assert rc == 0, lib.rlh_last_error()
    hip.sync()
    return hip.d2h_u32(dev_tok)


def test_noalloc_argmax_first_call_under_graph_capture():
    """The first call of the process is made while a non-null stream is
    being captured (global mode, the strictest: any call that is not legal
    under capture fails it). The graph is instantiated and replayed five
    times with new logits copied in between (eager work and
    synchronizations between the replays); every replay's token equals the
    oracle's argmax of the current logits. Then 200 eager calls leave the
    device's free memory unchanged."""
    print("no-alloc argmax: first call under stream capture, five replays", flush=True)
    lib = rlh.load()
    orc = oracle.load()
    hip = _Hip()
    h = hip.h
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    n = 3000
    try:
        dev_logits = hip.malloc(4 * n)
        dev_tok = hip.malloc(4)
        rng = np.random.default_rng(12)
        hip.h2d(dev_logits, rng.standard_normal(n).astype(np.float32))
        assert h.hipStreamCreate(ctypes.byref(stream)) == 0
        assert h.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        rc = lib.rlh_argmax_noalloc(dev_logits, n, dev_tok, stream)
        err = lib.rlh_last_error()
        assert h.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0, err
        assert rc == 0, err
        assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        for rep in range(5):
            x = rng.standard_normal(n).astype(np.float32)
            x[rng.integers(0, n, 3)] = 7.5  # tied maxima
            hip.h2d(dev_logits, x)
            hip.sync()
            assert h.hipGraphLaunch(exe, stream) == 0
            assert h.hipStreamSynchronize(stream) == 0
            assert hip.d2h_u32(dev_tok) == orc.orc_argmax(x.ctypes.data, n), rep
        hip.sync()
        free0 = hip.free_mem()
        for _ in range(200):
            assert lib.rlh_argmax_noalloc(dev_logits, n, dev_tok, stream) == 0
        assert h.hipStreamSynchronize(stream) == 0
        assert hip.free_mem() == free0
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        if stream.value:
            h.hipStreamDestroy(stream)
        hip.free()


def test_noalloc_argmax_matches_greedy_next_twice_then_smaller():
    print("no-alloc argmax: two model logits in a row (2048, then 1000)", flush=True)
    lib = rlh.load()
    hip = _Hip()
    models = []
    try:
        dev_logits = hip.malloc(4 * 4096)
        dev_tok = hip.malloc(4)
        for name, seed in (("tiny-q4km-untied", 17), ("tiny-q4km", 23)):  # vocab 2048, then 1000
            spec = rlh.SPECS[name]
            m = rlh.Model(spec, rlh.synth_model(spec, seed))
            c = m.new_cache(32)
            models.append((m, c))
            lg = c.forward_into(rlh.synth_tokens(seed, 7, spec.vocab), 0)
            want = c.greedy_next()
            hip.h2d(dev_logits, lg)
            got = _noalloc(lib, hip, dev_logits, spec.vocab, dev_tok)
            assert got == want, (name, got, want)

        # the edges of main.rs argmax, against the oracle
        orc = oracle.load()
        nan, inf = np.float32("nan"), np.float32("inf")
        cases = [np.array([1.0, 3.0, 3.0, 2.0], np.float32),
                 np.array([nan, 1.0, 5.0, 5.0, 2.0], np.float32),
                 np.array([-inf, -inf, -inf], np.float32),
                 np.array([nan, -inf, nan], np.float32),
                 np.array([nan, nan], np.float32)]
        rng = np.random.default_rng(3)
        big = rng.standard_normal(4096).astype(np.float32)
        big[[100, 2000, 4095]] = 9.0  # tied maxima across partial blocks
        big[::97] = nan
        cases.append(big)
        for x in cases:
            hip.h2d(dev_logits, x)
            got = _noalloc(lib, hip, dev_logits, len(x), dev_tok)
            assert got == orc.orc_argmax(x.ctypes.data, len(x)), x[:8]

        # arguments: sizes outside [1, 2^32 - 1], null and host pointers
        assert lib.rlh_argmax_noalloc(dev_logits, 0, dev_tok, None) == rlh.RLH_EINVAL
        assert lib.rlh_argmax_noalloc(dev_logits, 1 << 32, dev_tok, None) == rlh.RLH_EINVAL
        assert b"outside" in lib.rlh_last_error()
        assert lib.rlh_argmax_noalloc(None, 4, dev_tok, None) == rlh.RLH_EINVAL
        host = np.zeros(4, np.float32)
        assert lib.rlh_argmax_noalloc(host.ctypes.data, 4, dev_tok, None) == rlh.RLH_EINVAL
    finally:
        for m, c in models:
            c.close()
            m.close()
        hip.free()


def test_noalloc_argmax_at_the_largest_n():
    """n = 2^32 - 1, the largest count the entry point accepts (16 GiB of
    logits): the partial kernel's grid-stride index runs in 64 bits, so its
    last stride ends past n instead of wrapping below it. All values -1.0
    except a maximum at index n - 1 (found only if the loop reaches the end),
    then an equal maximum at index 5 as well (the lower index wins)."""
    print("no-alloc argmax: n = 2^32 - 1 (16 GiB of logits)", flush=True)
    lib = rlh.load()
    hip = _Hip()
    n = (1 << 32) - 1
    try:
        dev_logits = hip.malloc(4 * n)
        dev_tok = hip.malloc(4)
        minus_one = int(np.array([-1.0], np.float32).view(np.uint32)[0])
        assert hip.h.hipMemsetD32(dev_logits, ctypes.c_int(minus_one - (1 << 32)), ctypes.c_size_t(n)) == 0
        top = np.array([3.5], np.float32)
        last = ctypes.c_void_p(dev_logits.value + 4 * (n - 1))
        hip.h2d(last, top)
        assert _noalloc(lib, hip, dev_logits, n, dev_tok) == n - 1
        hip.h2d(ctypes.c_void_p(dev_logits.value + 4 * 5), top)
        assert _noalloc(lib, hip, dev_logits, n, dev_tok) == 5
    finally:
        hip.free()
