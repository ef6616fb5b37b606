"""The anti-restate guard's host half (lumen_anti_restate_select) on the CPU.

The device half returns 9 candidates per row (the raw argmax, then the 8
largest finite values in (value desc, id asc) order); `candidates` below
computes the same from numpy, so these tests pin the selection rules:
against the reference's own guard tests (sampling.rs:1778-2083), and
against the oracle's guarded_argmax (itself pinned by those tests) on
random logits, histories and decoders.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from lumen_amd.sampling import TokenBytes, anti_restate_select
from oracle import oracle as o

NONE = 0xFFFFFFFF

DEC = {10: b" multiplication", 11: b"lication", 12: b" into", 13: b"ing", 14: b" running",
       15: b"lications", 16: b" distrib", 17: b"utive", 20: b"17", 21: b" times", 22: b" 23"}


def decoder_table(n=128):
    return [DEC.get(i, b"") for i in range(n)]


def total_keys(v):
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def candidates(v):
    v = np.asarray(v, dtype=np.float32)
    k = total_keys(v)
    raw = int(np.argmax(k))  # first maximal key = lowest index on ties
    fin = np.nonzero(np.isfinite(v))[0]
    order = fin[np.lexsort((fin, -k[fin].astype(np.int64)))][:8]
    out = [raw] + [int(i) for i in order]
    return out + [NONE] * (9 - len(out))


def vec(n, **kv):
    v = [0.0] * n
    for key, x in kv.items():
        v[int(key[1:])] = x
    return v


def sel(logits, history, dec=True):
    return anti_restate_select(candidates(logits), history,
                               decoder_table(len(logits)) if dec else None)


def test_reference_guard_cases():
    # sampling.rs:1798-2083, each case's asserted token
    assert sel(vec(32, t11=5.0, t12=4.9), [10]) == 12
    assert sel(vec(32, t11=5.0, t15=4.9, t12=4.8), [10]) == 12
    assert sel(vec(32, t17=5.0), [16]) == 17
    assert sel(vec(32, t13=5.0), [20]) == 13
    assert sel(vec(32, t22=5.0, t12=4.0), [20, 21, 22, 20, 21], dec=False) == 12
    assert sel(vec(32, t20=5.0), [20, 21], dec=False) == 20
    assert sel(vec(32, t21=5.0), [20, 21, 20], dec=False) == 21
    assert sel(vec(64, t33=5.0, t12=4.0), [30, 31, 32, 33, 30, 31, 32], dec=False) == 12
    assert sel(vec(128, t16=5.0, t12=4.0), [16, 99] * 5, dec=False) == 12
    sparse = [16, 40, 41, 16, 42, 43, 16, 44, 45, 16, 46, 47]
    assert sel(vec(128, t50=5.0), sparse, dec=False) == 50
    ninf = [float("-inf")] * 32
    ninf[11] = 5.0
    assert sel(ninf, [10]) == 11
    assert sel(vec(32, t11=5.0), []) == 11
    # the lowest index wins a tie (sampling.rs:1055-1057)
    assert sel([2.0, 9.0, 9.0, 1.0], []) == 1


def test_candidates_helper_is_the_probe_order():
    # NaN and +inf are the raw argmax but never probed again; -0.0 < +0.0
    v = np.array([1.0, np.nan, 3.0, np.inf, 3.0, -0.0, 0.0, -np.inf], np.float32)
    c = candidates(v)
    assert c[0] == 1  # positive NaN is the total_cmp maximum
    assert c[1:7] == [2, 4, 0, 6, 5, NONE][:6]


def random_decoder(rng, V):
    alpha = [b"a", b"b", b"ab", b"ba", b" ", b"c"]
    out = []
    for _ in range(V):
        n = int(rng.integers(0, 5))
        out.append(b"".join(alpha[int(rng.integers(0, len(alpha)))] for _ in range(n)))
    return out


def test_select_matches_oracle_guard_random():
    rng = np.random.default_rng(5)
    for case in range(400):
        V = int(rng.integers(2, 40))
        v = rng.integers(-3, 4, size=V).astype(np.float32)  # many exact ties
        special = rng.random(V)
        v[special < 0.05] = np.nan
        v[(special >= 0.05) & (special < 0.1)] = np.inf
        v[(special >= 0.1) & (special < 0.2)] = -np.inf
        hl = int(rng.integers(0, 40))
        # histories with loops and dense repeats so every rule fires sometimes
        base = rng.integers(0, min(V, 6), size=max(1, hl // 3))
        h = np.resize(base, hl).astype(np.uint32)
        dec = random_decoder(rng, V) if rng.random() < 0.7 else None
        want = o.guarded_argmax(v, h, dec)
        got = anti_restate_select(candidates(v), h, dec)
        assert got == want, (case, v.tolist(), h.tolist(), dec)


def test_rule_gates_from_the_environment():
    # LUMEN_ANTI_RESTATE_NGRAM=off disables the span rule only (sampling.rs:625-662)
    code = ("from tests.test_anti_restate_cpu import sel, vec;"
            "print(sel(vec(32, t22=5.0, t12=4.0), [20, 21, 22, 20, 21], dec=False),"
            " sel(vec(128, t16=5.0, t12=4.0), [16, 99] * 5, dec=False))")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for val, want in (("off", "22 12"), ("1", "12 12")):
        env = dict(os.environ, LUMEN_ANTI_RESTATE_NGRAM=val)
        r = subprocess.run([sys.executable, "-c", code], cwd=root, env=env,
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert r.stdout.split() == want.split()
