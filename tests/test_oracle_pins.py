"""Pins for the oracle beyond the reference's own tests: published constants,
brute force on small inputs, IEEE single-operation exactness and the libm
identity of the expf restatement.
"""
import math
import random
import struct

import numpy as np
import pytest

from oracle import oracle as o

F32 = np.float32


def tkey(v):
    u = struct.unpack("<I", struct.pack("<f", float(v)))[0]
    return (~u & 0xFFFFFFFF) if (u & 0x80000000) else (u | 0x80000000)


def splitmix64_first(seed):
    # Published SplitMix64 (Steele, Lea, Flood 2014): state += golden gamma,
    # then the Stafford Mix13 finalizer. new(seed) == first output for seed.
    M = (1 << 64) - 1
    z = (seed + 0x9E3779B97F4A7C15) & M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_rng_splitmix_published_value():
    # SplitMix64's published first output for seed 1.
    assert o.Xorshift64(1).state.value == 0x910A2DEC89025CC1
    for s in (1, 2, 42, 12345, 0xC0FFEE, 2**63 + 5):
        assert o.Xorshift64(s).state.value == splitmix64_first(s)
    # seed 0 falls back to 0xDEADBEEFCAFEBABE before mixing
    assert o.Xorshift64(0).state.value == splitmix64_first(0xDEADBEEFCAFEBABE)


def test_rng_xorshift_closed_form():
    M = (1 << 64) - 1
    r = o.Xorshift64(777)
    x = r.state.value
    for _ in range(200):
        x ^= (x << 13) & M
        x ^= x >> 7
        x ^= (x << 17) & M
        want_f = float(F32(x >> 40) * F32(2.0 ** -24))
        assert r.next_f32() == want_f
        assert r.state.value == x


def test_rng_known_answers_seed0():
    r = o.Xorshift64(0)
    assert r.state.value == 0x0D7D93560D1929D2
    got = [r.next_f32() for _ in range(3)]
    assert np.allclose(got, [0.27650404, 0.46752965, 0.29386067], atol=1e-7)


def test_argmax_brute_force_total_cmp():
    rng = np.random.default_rng(1)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1.0, 1.0],
                        dtype=np.float32)
    for trial in range(300):
        n = int(rng.integers(1, 40))
        v = rng.choice(np.concatenate([specials, rng.integers(-3, 4, 8).astype(np.float32)]), n)
        v = v.astype(np.float32)
        keys = [tkey(x) for x in v]
        best = max(keys)
        assert o.argmax(v) == keys.index(best)


def test_top_k_brute_force_keep_all_ties():
    rng = np.random.default_rng(2)
    for trial in range(300):
        n = int(rng.integers(2, 50))
        v = (rng.integers(-5, 6, n) / 2.0).astype(np.float32)
        k = int(rng.integers(1, n))
        got = o.apply_top_k(v, k)
        keys = [tkey(x) for x in v]
        if k == 1:
            keep = keys.index(max(keys))
            want = [x if i == keep else -np.inf for i, x in enumerate(v)]
        else:
            cutoff = sorted(keys, reverse=True)[k - 1]
            want = [x if tkey(x) >= cutoff else -np.inf for x in v]
        assert np.array_equal(got, np.array(want, dtype=np.float32))


def test_penalty_single_rounding():
    # Each reference operation is one IEEE binary32 op: the result must equal
    # the exactly-rounded value of each step computed in f64 then rounded.
    rng = np.random.default_rng(3)
    for _ in range(2000):
        v = F32(rng.normal(0, 5))
        rep = F32(rng.uniform(0.5, 2.0))
        pres = F32(rng.uniform(0, 2))
        freq = F32(rng.uniform(0, 2))
        c = int(rng.integers(1, 20))
        p = o.Params(temperature=1.0, repetition_penalty=float(rep), presence_penalty=float(pres),
                     frequency_penalty=float(freq))
        got = o.apply_penalties([v], p, [0] * c)[0]
        x = F32(float(v) / float(rep)) if v > 0 else F32(float(v) * float(rep))
        x = F32(float(x) - float(pres))
        fc = F32(float(freq) * float(c))
        x = F32(float(x) - float(fc))
        assert struct.pack("<f", got) == struct.pack("<f", x)


def test_penalty_ignores_out_of_range_ids():
    l = o.apply_penalties([1.0, 2.0], o.Params(temperature=1.0, presence_penalty=1.0), [5, 7, 1])
    assert list(l) == [1.0, 1.0]


def test_top_p_brute_force_small():
    # Brute force: enumerate all ranks, sequential f32 cum in stable-sorted
    # order, with the softmax computed by the oracle's own primitive.
    rng = np.random.default_rng(4)
    for _ in range(200):
        n = int(rng.integers(2, 30))
        v = (rng.integers(-4, 5, n) / 4.0).astype(np.float32)
        p = float(rng.choice([0.3, 0.5, 0.8, 0.95]))
        probs = o.softmax_inplace(v.copy())
        order = sorted(range(n), key=lambda i: (-tkey(probs[i]), i))
        cum = F32(0)
        kept = 0
        for rank, i in enumerate(order):
            cum = F32(cum + probs[i])
            kept = rank + 1
            if cum >= p:
                break
        want = v.copy()
        for i in order[kept:]:
            want[i] = -np.inf
        assert np.array_equal(o.apply_top_p(v, p), want)


def test_softmax_sum_matches_exact_within_bound():
    rng = np.random.default_rng(5)
    v = rng.normal(0, 2, 5000).astype(np.float32)
    p = o.softmax_inplace(v.copy())
    mx = float(v.max())
    exact = [math.exp(float(F32(float(x) - mx))) for x in v]
    s = math.fsum(exact)
    # each expf within 1 ulp, sequential sum within n*eps relative
    assert abs(float(np.sum(p, dtype=np.float64)) - 1.0) < 5000 * 2 ** -23
    assert all(abs(float(pi) - e / s) <= 1e-5 * max(e / s, 1e-30) + 1e-12
               for pi, e in zip(p[:200], exact[:200]))


def test_categorical_strict_less_than():
    probs = np.array([0.25, 0.25, 0.25, 0.25], dtype=np.float32)
    assert o.sample_categorical(probs, 0.0) == 0
    assert o.sample_categorical(probs, 0.25) == 1  # r == cum is not taken
    assert o.sample_categorical(probs, 0.9999999) == 3
    # fall-through returns the last index even when its probability is zero
    assert o.sample_categorical(np.array([0.5, 0.25, 0.0], np.float32), 0.9) == 2


def test_min_p_log_bound():
    v = np.array([5.0, 2.7, 2.69, 0.0], dtype=np.float32)
    got = o.apply_min_p(v, 0.1)
    bound = F32(F32(5.0) + F32(math.log(0.1)))
    assert list(np.isfinite(got)) == [x >= bound for x in v]


def test_expf_restatement_matches_libm_sampled():
    # The restated glibc expf must equal the system expf bit-for-bit; the
    # full 2^32 sweep was run once at development time; here a 2^22 window
    # around the softmax domain (x <= 0) plus random patterns.
    neg_one = struct.unpack("<I", struct.pack("<f", -1.0))[0]
    bad, first = o.expf_check_range(neg_one - (1 << 21), 1 << 22)
    assert bad == 0, hex(first)
    rnd = random.Random(6)
    for _ in range(64):
        start = rnd.randrange(0, 2**32 - 4096)
        bad, first = o.expf_check_range(start, 4096)
        assert bad == 0, hex(first)


@pytest.mark.slow
def test_expf_restatement_matches_libm_negative_half():
    # every x in [-inf, -0.0] (2^31 patterns)
    bad, first = o.expf_check_range(0x80000000, 1 << 31)
    assert bad == 0, hex(first)


def test_expf_table_is_exp2_i_over_32():
    tab = o.expf_table()
    for i, t in enumerate(tab):
        d = struct.unpack("<d", struct.pack("<Q", (t + (i << 47)) & (2**64 - 1)))[0]
        assert abs(d - 2 ** (i / 32)) <= 2 ** -52
