"""Pins the CPU oracle against the reference's own unit tests.

Each test restates one `#[test]` of crates/lumen-runtime/src/sampling.rs
(lines cited) or crates/lumen-runtime/src/engine.rs, with the same inputs and
the same expectations, run against the C oracle.
"""
import math

import numpy as np
import pytest

from oracle import oracle as o

NEG_INF = float("-inf")


class Sampler:
    """sampling.rs:397-434: params + history + RNG; sample() records."""

    def __init__(self, params: o.Params, rng=None):
        self.params = params
        self.history = []
        self.rng = rng or o.Xorshift64(42 if params.seed is None else params.seed)
        self.decoder = None

    def record(self, t):
        self.history.append(t)

    def sample(self, logits):
        t = o.sample_logits(np.array(logits, dtype=np.float32), self.params, self.history,
                            self.rng, self.decoder)
        self.record(t)
        return t


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- greedy (sampling.rs:1026-1139) -------------------------------------

def test_greedy_returns_argmax_with_all_default_params():  # :1026-1034
    s = Sampler(o.Params(temperature=0.0))
    assert s.sample([1.0, 5.0, 3.0, 2.0]) == 1


def test_argmax_breaks_ties_to_lowest_index():  # :1037-1058
    assert o.argmax([1.0, 5.0, 3.0, 2.0]) == 1
    assert o.argmax([0.0, 0.0, 0.0, 9.0, 9.0, 9.0]) == 3
    assert o.argmax([7.0, 7.0, 7.0, 7.0]) == 0
    assert o.argmax([4.0, 4.0, 1.0]) == 0
    assert o.argmax(np.zeros(0, dtype=np.float32)) == 0
    assert o.argmax([42.0]) == 0
    assert o.argmax([-3.0, -1.0, -1.0, -5.0]) == 1
    assert o.guarded_argmax([2.0, 9.0, 9.0, 1.0], []) == 1


def test_greedy_ignores_distribution_shaping_but_applies_penalties():  # :1061-1083
    s = Sampler(o.Params(temperature=0.0, top_p=0.5, top_k=1, min_p=0.9,
                         repetition_penalty=2.0, presence_penalty=10.0,
                         frequency_penalty=10.0))
    s.record(1)
    assert s.sample([1.0, 5.0, 3.0, 2.0]) == 2


def test_greedy_unaffected_when_penalties_disabled():  # :1086-1099
    s = Sampler(o.Params(temperature=0.0, top_p=0.5, top_k=1, min_p=0.9))
    s.record(1)
    assert s.sample([1.0, 5.0, 3.0, 2.0]) == 1


def test_greedy_with_repeat_last_n_windows_penalty():  # :1102-1119
    s = Sampler(o.Params(temperature=0.0, frequency_penalty=10.0, repeat_last_n=2))
    for t in (0, 0, 1, 1):
        s.record(t)
    assert s.sample([3.0, 3.5]) == 0


def test_windowed_penalty_ignores_tokens_outside_window():  # :1122-1139
    s = Sampler(o.Params(temperature=0.0, frequency_penalty=10.0, repeat_last_n=1))
    for t in (0, 0, 0, 1):
        s.record(t)
    assert s.sample([3.0, 3.5]) == 0


# ---- determinism (sampling.rs:1143-1160) ---------------------------------

def test_determinism_same_seed_same_output():
    base = np.sin(np.arange(1000, dtype=np.float32) * np.float32(0.01)).astype(np.float32)

    def params():
        return o.Params(temperature=0.7, seed=0xC0FFEE, top_p=0.9, top_k=40)

    s1, s2 = Sampler(params()), Sampler(params())
    for _ in range(100):
        assert s1.sample(base) == s2.sample(base)


# ---- top-k (sampling.rs:1164-1360) ----------------------------------------

def test_top_k_one_acts_as_greedy():  # :1164-1176
    s = Sampler(o.Params(temperature=1.0, top_k=1, seed=1))
    for _ in range(50):
        assert s.sample([1.0, 5.0, 3.0, 2.0, 4.0]) == 1


def test_top_k_one_exact_tie_breaks_to_lowest_index():  # :1179-1212
    logits = [1.0, 2.0, 2.0, 0.5]
    for seed in (1, 2, 7, 42, 0xC0FFEE, 0xDEADBEEF):
        s = Sampler(o.Params(temperature=1.0, top_k=1, seed=seed))
        for _ in range(50):
            assert s.sample(logits) == 1
    l = o.apply_top_k(logits, 1)
    assert l[1] == 2.0 and l[0] == NEG_INF and l[2] == NEG_INF and l[3] == NEG_INF


def _top_k_prefix_reference(logits, k):
    # the pre-fix implementation embedded in sampling.rs:1221-1230
    a = np.array(logits, dtype=np.float32)
    keys = sorted(a.tolist(), key=lambda v: o_total_key(v), reverse=True)
    cutoff = o_total_key(keys[k - 1])
    return np.array([NEG_INF if o_total_key(v) < cutoff else v for v in a.tolist()],
                    dtype=np.float32)


def o_total_key(v):
    u = int(np.array([v], dtype=np.float32).view(np.uint32)[0])
    return (~u & 0xFFFFFFFF) if (u & 0x80000000) else (u | 0x80000000)


def test_apply_top_k_differential_only_k1_ties_change():  # :1215-1306
    non_tie = [[1.0, 5.0, 3.0, 2.0, 4.0], [-3.0, -1.0, -2.0, -5.0, -0.5],
               [0.0, 10.0, 20.0, 5.0, 15.0, 7.5], [9.0, 8.0, 7.0, 6.0, 5.0, 4.0, 3.0]]
    for base in non_tie:
        for k in range(1, len(base)):
            assert (bits(o.apply_top_k(base, k)) == bits(_top_k_prefix_reference(base, k))).all()
    tied = [[1.0, 2.0, 2.0, 0.5], [7.0, 7.0, 7.0, 7.0], [0.0, 9.0, 9.0, 9.0, 1.0],
            [4.0, 4.0, 1.0, 4.0, 2.0]]
    for base in tied:
        for k in range(2, len(base)):
            assert (bits(o.apply_top_k(base, k)) == bits(_top_k_prefix_reference(base, k))).all()
    for base in tied:
        got = o.apply_top_k(base, 1)
        want = _top_k_prefix_reference(base, 1)
        keep = o.argmax(base)
        assert [i for i, v in enumerate(got) if math.isfinite(v)] == [keep]
        if sum(1 for v in base if v == base[keep]) > 1:
            assert not (bits(got) == bits(want)).all()


def test_greedy_path_tie_unaffected_by_fix():  # :1309-1323
    s = Sampler(o.Params(temperature=0.0, top_k=1, seed=1))
    for _ in range(20):
        assert s.sample([1.0, 2.0, 2.0, 0.5]) == 1


def test_top_k_zero_disables():  # :1326-1346
    off = Sampler(o.Params(temperature=1.0, top_k=0, seed=99))
    none = Sampler(o.Params(temperature=1.0, top_k=None, seed=99))
    for _ in range(20):
        assert off.sample([1.0, 2.0, 3.0, 4.0]) == none.sample([1.0, 2.0, 3.0, 4.0])


def test_top_k_larger_than_vocab_is_noop():  # :1349-1360
    s = Sampler(o.Params(temperature=1.0, top_k=10, seed=6))
    assert s.sample([1.0, 2.0, 3.0]) < 3


# ---- top-p (sampling.rs:1364-1400) ----------------------------------------

def test_top_p_keeps_only_nucleus():  # :1364-1376
    s = Sampler(o.Params(temperature=1.0, top_p=0.5, seed=2))
    for _ in range(50):
        assert s.sample([0.0, 0.0, 0.0, 10.0]) == 3


def test_top_p_one_is_noop():  # :1379-1400
    one = Sampler(o.Params(temperature=1.0, top_p=1.0, seed=8))
    none = Sampler(o.Params(temperature=1.0, top_p=None, seed=8))
    for _ in range(30):
        assert one.sample([1.0, 2.0, 3.0, 4.0]) == none.sample([1.0, 2.0, 3.0, 4.0])


# ---- min-p (sampling.rs:1404-1439) ------------------------------------------

def test_min_p_drops_low_probability_tokens():  # :1404-1416
    s = Sampler(o.Params(temperature=1.0, min_p=0.5, seed=3))
    for _ in range(50):
        assert s.sample([0.0, 0.0, 0.0, 10.0]) == 3


def test_min_p_zero_is_noop():  # :1419-1439
    z = Sampler(o.Params(temperature=1.0, min_p=0.0, seed=9))
    n = Sampler(o.Params(temperature=1.0, min_p=None, seed=9))
    for _ in range(30):
        assert z.sample([1.0, 2.0, 3.0, 4.0]) == n.sample([1.0, 2.0, 3.0, 4.0])


# ---- penalties (sampling.rs:1443-1528) --------------------------------------

def test_repetition_penalty_suppresses_history_tokens():  # :1443-1470
    params = o.Params(temperature=1.0, repetition_penalty=10.0, seed=4)
    rng = o.Xorshift64(4)
    ones = 0
    for _ in range(1000):
        if o.sample_logits([1.0, 1.0], params, [0], rng) == 1:
            ones += 1
    assert ones > 650


def test_repetition_penalty_sign_aware_for_negative_logits():  # :1473-1489
    l = o.apply_penalties([-1.0, 1.0], o.Params(temperature=1.0, repetition_penalty=2.0), [0, 1])
    assert abs(l[0] - -2.0) < 1e-6 and abs(l[1] - 0.5) < 1e-6


def test_presence_penalty_uniform_subtraction():  # :1494-1507
    l = o.apply_penalties([2.0, 2.0], o.Params(temperature=1.0, presence_penalty=0.5), [0, 0])
    assert abs(l[0] - 1.5) < 1e-6 and abs(l[1] - 2.0) < 1e-6


def test_frequency_penalty_scales_with_count():  # :1512-1528
    l = o.apply_penalties([2.0, 2.0, 2.0], o.Params(temperature=1.0, frequency_penalty=0.5),
                          [0, 1, 1, 1])
    assert abs(l[0] - 1.5) < 1e-6 and abs(l[1] - 0.5) < 1e-6 and abs(l[2] - 2.0) < 1e-6


# ---- composition (sampling.rs:1532-1564) ------------------------------------

def test_composition_top_p_top_k_and_repetition_penalty():
    params = o.Params(temperature=1.0, top_p=0.6, top_k=2, repetition_penalty=10.0, seed=5)
    rng = o.Xorshift64(5)
    counts = [0, 0, 0, 0]
    for _ in range(500):
        counts[o.sample_logits([3.0, 2.0, 1.0, 0.5], params, [3], rng)] += 1
    assert counts == [500, 0, 0, 0]


# ---- state (sampling.rs:1568-1589) ------------------------------------------

def test_sampler_records_token_after_sample():
    s = Sampler(o.Params(temperature=0.0))
    assert s.sample([1.0, 0.0, 0.0]) == 0
    assert s.history == [0]


# ---- edge cases (sampling.rs:1593-1629) -------------------------------------

def test_empty_logits_returns_zero():
    s = Sampler(o.Params())
    assert s.sample(np.zeros(0, dtype=np.float32)) == 0


def test_default_params_match_pre_z1_behavior():  # :1600-1629
    base = [1.0, 2.0, 3.0, 4.0]
    s = Sampler(o.Params(temperature=1.0, seed=42))
    rng_ref = o.Xorshift64(42)
    for _ in range(30):
        probs = o.softmax_inplace(base)
        r = rng_ref.next_f32()
        cum = np.float32(0.0)
        want = len(probs) - 1
        for i, p in enumerate(probs):
            cum = np.float32(cum + p)
            if r <= cum:
                want = i
                break
        assert s.sample(base) == want


# ---- RNG first draw (sampling.rs:1633-1678) ---------------------------------

def test_rng_seed_42_first_draw_is_no_longer_zero():
    r0 = o.Xorshift64(42).next_f32()
    assert 0.0 < r0 < 1.0


def test_rng_first_draw_does_not_select_index_zero_under_skewed_dist():
    s = Sampler(o.Params(temperature=1.0, seed=42))
    assert s.sample([-5.0, 5.0, 0.0, 0.0]) != 0


# ---- ordering (sampling.rs:1682-1752) ---------------------------------------

def test_temperature_applies_after_top_p_min_p_filters():
    s = Sampler(o.Params(temperature=0.5, top_p=0.85, seed=0xC0FFEE))
    seen = set(s.sample([4.0, 3.0, 2.0, 1.0]) for _ in range(500))
    assert 1 in seen
    assert 2 not in seen and 3 not in seen


def test_min_p_on_logits_equivalent_to_log_shift():
    s = Sampler(o.Params(temperature=1.0, min_p=0.1, seed=11))
    for _ in range(100):
        assert s.sample([5.0, 2.0, 1.0, 0.0]) == 0


# ---- anti-restate guard (sampling.rs:1756-2098) -----------------------------

DEC = {10: b" multiplication", 11: b"lication", 12: b" into", 13: b"ing", 14: b" running",
       15: b"lications", 16: b" distrib", 17: b"utive", 20: b"17", 21: b" times", 22: b" 23"}


def decoder_table(n=128):
    return [DEC.get(i, b"") for i in range(n)]


def guarded(logits, history, dec=True):
    s = Sampler(o.Params(temperature=0.0, anti_restate=True), rng=o.Xorshift64(1))
    s.history = list(history)
    s.decoder = decoder_table(len(logits)) if dec else None
    return s.sample(logits)


def vec(n, **kv):
    v = [0.0] * n
    for k, x in kv.items():
        v[int(k[1:])] = x
    return v


def test_anti_restate_is_noop_without_flag():
    s = Sampler(o.Params(temperature=0.0), rng=o.Xorshift64(1))
    s.history = [10]
    s.decoder = decoder_table(32)
    assert s.sample(vec(32, t11=5.0, t12=4.9)) == 11


def test_anti_restate_vetoes_subword_doubling():
    assert guarded(vec(32, t11=5.0, t12=4.9), [10]) == 12


def test_anti_restate_vetoes_subword_doubling_with_trailing_char():
    assert guarded(vec(32, t11=5.0, t15=4.9, t12=4.8), [10]) == 12


def test_anti_restate_allows_legit_multitoken_word():
    assert guarded(vec(32, t17=5.0), [16]) == 17


def test_anti_restate_allows_legit_word_continuation():
    assert guarded(vec(32, t13=5.0), [20]) == 13


def test_anti_restate_vetoes_ngram_restate_without_decoder():
    assert guarded(vec(32, t22=5.0, t12=4.0), [20, 21, 22, 20, 21], dec=False) == 12


def test_anti_restate_allows_legit_short_repeat():
    assert guarded(vec(32, t20=5.0), [20, 21], dec=False) == 20


def test_anti_restate_allows_legit_two_token_repeat():
    assert guarded(vec(32, t21=5.0), [20, 21, 20], dec=False) == 21


def test_anti_restate_vetoes_backtoback_multitoken_loop():
    assert guarded(vec(64, t33=5.0, t12=4.0), [30, 31, 32, 33, 30, 31, 32], dec=False) == 12


def test_anti_restate_breaks_dense_runaway_loop():
    assert guarded(vec(128, t16=5.0, t12=4.0), [16, 99] * 5, dec=False) == 12


def test_anti_restate_allows_sparse_legit_reuse():
    h = [16, 40, 41, 16, 42, 43, 16, 44, 45, 16, 46, 47]
    assert guarded(vec(128, t50=5.0), h, dec=False) == 50


def test_anti_restate_falls_back_when_all_degenerate():
    l = [NEG_INF] * 32
    l[11] = 5.0
    assert guarded(l, [10]) == 11


def test_anti_restate_noop_on_empty_history():
    assert guarded(vec(32, t11=5.0), []) == 11


# ---- engine.rs tests (engine.rs:913-1036) -----------------------------------

def test_xorshift64_zero_seed_uses_fallback():
    assert o.Xorshift64(0).next_u64() != 0


def test_xorshift64_determinism():
    a, b = o.Xorshift64(42), o.Xorshift64(42)
    for _ in range(100):
        assert a.next_u64() == b.next_u64()


def test_xorshift64_next_f32_in_range():
    r = o.Xorshift64(12345)
    for _ in range(1000):
        v = r.next_f32()
        assert 0.0 <= v < 1.0


def test_softmax_edge_cases():
    assert o.softmax_inplace(np.zeros(0, dtype=np.float32)).size == 0
    assert abs(o.softmax_inplace([5.0])[0] - 1.0) < 1e-6
    assert np.allclose(o.softmax_inplace([3.0] * 4), 0.25, atol=1e-6)
    assert np.allclose(o.softmax_inplace([float("nan")] * 3), 1 / 3, atol=1e-6)
    assert np.allclose(o.softmax_inplace([NEG_INF] * 3), 1 / 3, atol=1e-6)


def test_sample_token_shims():
    assert o.sample_logits(np.zeros(0, np.float32), o.Params(temperature=1.0), [],
                           o.Xorshift64(42)) == 0
    assert o.sample_logits([1.0, 5.0, 3.0, 2.0], o.Params(temperature=0.0), [],
                           o.Xorshift64(42)) == 1
    t1 = o.sample_logits([1.0, 2.0, 3.0, 4.0], o.Params(temperature=0.8), [], o.Xorshift64(42))
    t2 = o.sample_logits([1.0, 2.0, 3.0, 4.0], o.Params(temperature=0.8), [], o.Xorshift64(42))
    assert t1 == t2
