"""The device sampler (rlh_dsampler_*, Sampler::sample sampler.rs:56-163 and
ops::softmax_inplace ops.rs:398-419 on device values) against the oracle's
sampler and softmax, and against the library's host sampler: identical
probabilities bit for bit, identical token sequences from one RNG state.

Cases cover each way the device picks a token — the argmax (temperature 0,
with and without the penalty), the on-chip candidate list (top-k up to 4096,
top-p over a prefix), the full radix sort (top-k 0 without top-p, top-k above
4096, candidate lists that do not fit) — and the inputs that decide between
them: distinct logits, logits on a few levels (ties at the top-k edge, where
both order equal probabilities by id), one flat row, wide ranges whose
exponentials underflow, a full-size vocabulary of 151936."""
import ctypes

import numpy as np
import pytest

import oracle
import rlh
from helpers import HipBuffers

pytestmark = pytest.mark.gpu

VOCAB = 151936


@pytest.fixture(scope="module")
def hip():
    h = HipBuffers()
    yield h
    h.free()


@pytest.fixture(scope="module")
def dev(hip):
    return hip.malloc(VOCAB * 4 + 64)


def _logits(kind, n, rng):
    if kind == "llm":
        x = (rng.standard_normal(n) * 2.5).astype(np.float32)
        x[rng.integers(0, n, 12)] += np.float32(9.0)
        return x
    if kind == "distinct":
        return rng.permutation(np.linspace(-12.0, 9.0, n).astype(np.float32))
    if kind == "levels":
        return np.linspace(-4.0, 3.0, 12).astype(np.float32)[rng.integers(0, 12, n)]
    if kind == "flat":
        return np.zeros(n, np.float32)
    if kind == "wide":
        return (rng.standard_normal(n) * 40.0).astype(np.float32)
    raise ValueError(kind)


def _params(temp, top_k, top_p, pen, last_n, seed):
    return rlh.SamplingParams(temp, top_k, top_p, pen, last_n, seed), \
        oracle.SamplingParams(temp, top_k, top_p, pen, last_n, seed)


def _run_sequence(hip, dev, kind, n, temp, top_k, top_p, pen, last_n, steps, seed, cap=None):
    """`steps` draws with one RNG state on fresh logits each step, feeding
    every token into the penalty history; device, host and oracle samplers
    must agree on every token, device and host on every RNG state."""
    rng = np.random.default_rng(seed)
    p, op = _params(temp, top_k, top_p, pen, last_n, seed)
    lib = oracle.load()
    orc = lib.orc_sampler_create(seed)
    host = rlh.Sampler(seed)
    paths = set()
    with rlh.DeviceSampler(seed, VOCAB) as ds:
        if cap is not None:
            ds.set_candidate_cap(cap)
        recent = list(map(int, rng.integers(0, n, 80)))
        for step in range(steps):
            x = _logits(kind, n, rng)
            hip.h2d(dev, x)
            r = np.asarray(recent, np.uint32)
            got = ds.sample(dev, n, p, r)
            paths.add(ds.last_path)
            want = lib.orc_sampler_sample(orc, x.ctypes.data, n, ctypes.byref(op), r.ctypes.data, len(r))
            h = host.sample(x, p, r)
            assert got == want == h, (kind, step, got, want, h)
            assert ds.state.value == host.state.value, (kind, step)
            recent.append(got)
    lib.orc_sampler_destroy(orc)
    return paths


@pytest.mark.parametrize("case", ["normal", "wide", "ties", "nan_first", "nan_later", "inf", "tiny", "one", "two",
                                  "all_neg_inf", "signed_zeros", "flat"])
def test_softmax_bit_exact(hip, dev, case):
    """rlh_dsampler_softmax against the oracle's softmax_inplace and the host
    rlh_softmax: identical bits, NaN rule of the max included (a NaN first
    value propagates, later NaNs are skipped; any NaN exponential leaves the
    sum NaN and the values unscaled)."""
    print(f"device softmax {case}", flush=True)
    rng = np.random.default_rng(7)
    n = {"tiny": 5, "one": 1, "two": 2}.get(case, VOCAB)
    x = (rng.standard_normal(n) * {"wide": 40.0}.get(case, 3.0)).astype(np.float32)
    if case == "ties":
        x = np.round(x * 4) / 4
    elif case == "nan_first":
        x[0] = np.nan
    elif case == "nan_later":
        x[17] = np.nan
        x[n - 2] = np.nan
    elif case == "inf":
        x[3] = -np.inf
        x[9] = np.inf
    elif case == "wide":
        x[11] = 200.0
        x[12] = -300.0
    elif case == "all_neg_inf":
        x[:] = -np.inf
    elif case == "signed_zeros":
        x[:] = 0.0
        x[::3] = -0.0
    elif case == "flat":
        x[:] = 1.5
    want = x.copy()
    oracle.load().orc_softmax_inplace(want.ctypes.data, n)
    host = x.copy()
    assert rlh.load().rlh_softmax(host.ctypes.data, n) == 0
    hip.h2d(dev, x)
    with rlh.DeviceSampler(1, VOCAB) as ds:
        ds.softmax(dev, n)
        hip.sync()
    got = hip.d2h(dev, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(host.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("temp", [0.0, 0.7, 1.3])
@pytest.mark.parametrize("top_k", [0, 1, 40, 5000])
@pytest.mark.parametrize("top_p", [1.0, 0.95, 0.3])
@pytest.mark.parametrize("pen,last_n", [(1.0, 64), (1.1, 64), (0.8, 0)])
def test_sequence_matches_oracle(hip, dev, temp, top_k, top_p, pen, last_n):
    print(f"device sampler t={temp} k={top_k} p={top_p} pen={pen}/{last_n}", flush=True)
    _run_sequence(hip, dev, "distinct", 20000, temp, top_k, top_p, pen, last_n, 6,
                  int(temp * 10) * 1000 + top_k + int(top_p * 100) + int(pen * 10))


@pytest.mark.parametrize("kind", ["llm", "levels", "flat", "wide"])
@pytest.mark.parametrize("top_k,top_p", [(40, 0.95), (40, 1.0), (7, 0.5), (0, 0.9), (0, 1.0), (3000, 0.99)])
def test_full_vocabulary(hip, dev, kind, top_k, top_p):
    """151936 logits with the default temperature and penalty: language-model
    like rows, rows on 12 levels (every kept probability tied), one flat row
    (a single tie class: the candidate list cannot hold it), wide rows."""
    print(f"device sampler vocab {kind} k={top_k} p={top_p}", flush=True)
    paths = _run_sequence(hip, dev, kind, VOCAB, 0.7, top_k, top_p, 1.1, 64, 4, 17 + top_k)
    if top_k == 0 and top_p >= 1.0:
        assert paths == {rlh.DSAMPLER_PATH_SORT}
    if kind == "llm" and top_k == 40:
        assert paths == {rlh.DSAMPLER_PATH_CANDIDATES}
    if kind == "flat" and top_k > 0:
        assert paths == {rlh.DSAMPLER_PATH_SORT | rlh.DSAMPLER_PATH_FALLBACK}


@pytest.mark.parametrize("cap", [4096, 64, 1, 0])
def test_candidate_cap_changes_path_not_tokens(hip, dev, cap):
    """The same draws whatever the on-chip list holds: small caps push top-k
    and top-p searches to the radix sort, cap 0 always sorts."""
    print(f"device sampler cap {cap}", flush=True)
    for top_k, top_p in [(40, 0.95), (0, 0.8), (50, 1.0)]:
        paths = _run_sequence(hip, dev, "levels", 30000, 0.8, top_k, top_p, 1.1, 64, 5, 5 + top_k, cap=cap)
        if cap == 0:
            assert paths == {rlh.DSAMPLER_PATH_SORT}
        if cap == 1:
            assert rlh.DSAMPLER_PATH_CANDIDATES not in paths


def test_small_vocabularies(hip, dev):
    """n smaller than one block of the elementwise kernels, n = 1, top-k at
    n - 1 and above n."""
    for n in (2, 3, 17, 1000, 1025):
        for top_k in (0, 1, n - 1, n + 5):
            _run_sequence(hip, dev, "llm", n, 0.9, top_k, 0.9, 1.2, 4, 4, n * 7 + top_k)
    with rlh.DeviceSampler(3, VOCAB) as ds:
        host = rlh.Sampler(3)
        x = np.array([2.0], np.float32)
        hip.h2d(dev, x)
        p = rlh.SamplingParams(0.7, 40, 0.95, 1.1, 64, 3)
        assert ds.sample(dev, 1, p, []) == host.sample(x, p, []) == 0
        assert ds.state.value == host.state.value
        assert ds.sample(dev, 0, p, []) == 0


def test_greedy_paths(hip, dev):
    """Temperature 0: the first maximum (sampler.rs:62-70, 104-112), with
    logits[0] kept when it is NaN, ties to the lowest id, -inf rows to 0, and
    the penalty applied first when set. The RNG is not touched."""
    nan, inf = float("nan"), float("inf")
    rows = [[nan, 1.0, 5.0, 2.0], [1.0, nan, 5.0, 2.0], [-inf, -inf, -inf], [-inf, -inf, 3.0],
            [1.0, 3.0, 3.0, 2.0], [3.0, -2.0, 3.0, 2.9]]
    with rlh.DeviceSampler(9, VOCAB) as ds:
        for row in rows:
            x = np.array(row, np.float32)
            hip.h2d(dev, x)
            for pen, recent in [(1.0, []), (1.5, [0, 2]), (0.5, [1, 1, 3])]:
                p = rlh.SamplingParams(0.0, 40, 0.95, pen, 64, 9)
                host = rlh.Sampler(9)
                before = ds.state.value
                assert ds.sample(dev, len(x), p, recent) == host.sample(x, p, recent), (row, pen)
                assert ds.last_path == rlh.DSAMPLER_PATH_GREEDY
                assert ds.state.value == before


def test_nonfinite_logits_are_refused(hip, dev):
    """Sampling (temperature > 0) from logits that give a NaN probability — a
    NaN, a +inf, all -inf, or an overflow by the temperature — is an error,
    as the reference's partial_cmp().unwrap() sort panics on it; the RNG state
    is left as it was."""
    rng = np.random.default_rng(3)
    with rlh.DeviceSampler(5, VOCAB) as ds:
        for how in ("nan", "inf", "neg_inf_all", "overflow"):
            x = (rng.standard_normal(5000)).astype(np.float32)
            temp = 0.7
            if how == "nan":
                x[100] = np.nan
            elif how == "inf":
                x[7] = np.inf
            elif how == "neg_inf_all":
                x[:] = -np.inf
            else:
                x[9] = 3e38
                temp = 1e-3
            hip.h2d(dev, x)
            before = ds.state.value
            with pytest.raises(rlh.RlhError) as e:
                ds.sample(dev, len(x), rlh.SamplingParams(temp, 40, 0.95, 1.0, 64, 5), [])
            assert e.value.code == rlh.RLH_EINVAL
            assert ds.state.value == before
        x = rng.standard_normal(5000).astype(np.float32)
        hip.h2d(dev, x)
        host = rlh.Sampler(5)
        p = rlh.SamplingParams(0.7, 40, 0.95, 1.0, 64, 5)
        assert ds.sample(dev, len(x), p, []) == host.sample(x, p, [])


def test_arguments_rejected(dev):
    lib = rlh.load()
    h = ctypes.c_void_p()
    assert lib.rlh_dsampler_create(0, ctypes.byref(h)) == rlh.RLH_EINVAL
    with rlh.DeviceSampler(1, 100) as ds:
        p = rlh.SamplingParams(0.7, 40, 0.95, 1.0, 64, 1)
        with pytest.raises(rlh.RlhError) as e:
            ds.sample(dev, 101, p, [])
        assert e.value.code == rlh.RLH_EINVAL
        with pytest.raises(rlh.RlhError):
            ds.set_candidate_cap(4097)
        t = ctypes.c_uint32()
        st = ctypes.c_uint64(1)
        assert lib.rlh_dsampler_sample(ds.h, None, 5, ctypes.byref(p), None, 0, ctypes.byref(st),
                                       ctypes.byref(t), None) == rlh.RLH_EINVAL
