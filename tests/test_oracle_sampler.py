"""Pins the oracle's sampler (src/sampler.rs) and argmax (src/main.rs:453-463)."""
import ctypes

import numpy as np

import oracle


def params(temp=0.0, top_k=0, top_p=1.0, pen=1.0, last_n=64, seed=1):
    return oracle.SamplingParams(temp, top_k, top_p, pen, last_n, seed)


def sample(logits, p, recent, seed=1):
    lib = oracle.load()
    s = lib.orc_sampler_create(seed)
    lg = np.asarray(logits, np.float32)
    r = np.asarray(recent, np.uint32)
    out = lib.orc_sampler_sample(s, lg.ctypes.data, len(lg), ctypes.byref(p), r.ctypes.data, len(r))
    lib.orc_sampler_destroy(s)
    return out


def test_repetition_penalty_applies_once_per_distinct_token():
    """sampler.rs:181-189."""
    assert sample([10.0, 1.0], params(pen=2.0, last_n=64), [0, 0, 0, 0]) == 0


def test_repetition_penalty_respects_window():
    """sampler.rs:191-199."""
    assert sample([10.0, 1.0], params(pen=20.0, last_n=2), [7, 7, 0]) == 1
    assert sample([10.0, 1.0], params(pen=20.0, last_n=2), [0, 7, 7]) == 0


def test_repetition_penalty_disabled_is_identity():
    """sampler.rs:201-206."""
    assert sample([10.0, 1.0], params(pen=1.0, last_n=64), [0, 0, 0]) == 0


def test_xorshift64star_closed_form():
    """sampler.rs:33-54: state = seed | 1; xorshift64* then (x >> 40) / 2^24."""
    lib = oracle.load()
    for seed in [0, 1, 0x123456789ABCDEF0, 2 ** 64 - 1]:
        s = lib.orc_sampler_create(seed)
        st = (seed | 1) & 0xFFFFFFFFFFFFFFFF
        for _ in range(50):
            x = st
            x ^= x >> 12
            x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
            x ^= x >> 27
            st = x
            want = (x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
            assert lib.orc_sampler_next_u64(s) == want
        lib.orc_sampler_destroy(s)
    s = lib.orc_sampler_create(5)
    for _ in range(1000):
        f = lib.orc_sampler_next_f32(s)
        assert 0.0 <= f < 1.0
    lib.orc_sampler_destroy(s)


def test_greedy_tie_lowest_index_and_argmax():
    """Strict '>' from index 0: the lowest index of equal maxima wins
    (sampler.rs:62-70, main.rs:453-463); NaN never wins in argmax."""
    lib = oracle.load()
    lg = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert sample(lg, params(), []) == 1
    assert lib.orc_argmax(lg.ctypes.data, len(lg)) == 1
    lg2 = np.array([np.nan, 1.0, 5.0, 5.0], np.float32)
    assert lib.orc_argmax(lg2.ctypes.data, len(lg2)) == 2


def test_sampled_distribution_follows_softmax():
    """temperature / top-k / top-p draw: empirical frequencies follow the
    renormalised softmax over the kept set (sampler.rs:115-162)."""
    lib = oracle.load()
    logits = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -5.0], np.float32)
    p = params(temp=0.7, top_k=4, top_p=0.95, pen=1.0)
    s = lib.orc_sampler_create(1234)
    counts = np.zeros(len(logits))
    n = 20000
    for _ in range(n):
        counts[lib.orc_sampler_sample(s, logits.ctypes.data, len(logits), ctypes.byref(p), None, 0)] += 1
    lib.orc_sampler_destroy(s)
    z = np.exp((logits.astype(np.float64) / 0.7) - (logits.max() / 0.7))
    z /= z.sum()
    order = np.argsort(-z)[:4]
    keep = []
    cum = 0.0
    for i in order:
        keep.append(i)
        cum += z[i]
        if cum >= 0.95:
            break
    want = np.zeros(len(logits))
    want[keep] = z[keep] / z[keep].sum()
    assert counts[want == 0].sum() == 0
    assert np.abs(counts / n - want).max() < 0.02
