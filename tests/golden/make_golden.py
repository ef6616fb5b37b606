"""Writes the small golden vectors of the sampler under tests/golden/.

Each fixture file holds explicit inputs (f32 logits, per-row parameters,
penalty histories, uniforms) and the CPU oracle's outputs for them: the token
and the intermediate values of the chain (top-k survivors, top-p sum and kept
count, final max, final sum, the CDF value at the crossing). The inputs are
stored, not regenerated from seeds, so the fixtures stay valid across numpy
versions. Test infrastructure: run by hand after a deliberate change of the
oracle (`python tests/golden/make_golden.py`), never by the product.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as o  # noqa: E402

# parameter columns; NaN (or -1 for repeat_last_n, 0 for top_k) means None
PARAM_COLS = ("temperature", "top_k", "top_p", "min_p", "repetition_penalty",
              "presence_penalty", "frequency_penalty", "repeat_last_n")
TRACE_KEYS = ("greedy", "topk_applied", "topk_survivors", "topk_cutoff_key", "topp_applied",
              "topp_sum", "topp_kept", "final_max", "final_uniform", "final_sum", "cdf_at")


def _row_params(**kw):
    v = np.full(len(PARAM_COLS), np.nan)
    v[PARAM_COLS.index("top_k")] = 0
    v[PARAM_COLS.index("repeat_last_n")] = -1
    for k, x in kw.items():
        v[PARAM_COLS.index(k)] = x
    return v


def params_from_row(v) -> dict:
    """Fixture row -> keyword arguments of SamplingParams / oracle Params."""
    d = {}
    for k, x in zip(PARAM_COLS, v):
        if k == "top_k":
            d[k] = int(x) if x > 0 else None
        elif k == "repeat_last_n":
            d[k] = int(x) if x >= 0 else None
        else:
            d[k] = None if np.isnan(x) else float(x)
    if d["temperature"] is None:
        d["temperature"] = 1.0
    return d


def cases(V: int, rng):
    """(logits row, params row, history) triples covering every stage."""
    out = []
    hist = lambda n: rng.integers(0, V, n).astype(np.uint32)  # noqa: E731
    normal = lambda s=2.0: rng.normal(0, s, V).astype(np.float32)  # noqa: E731
    out.append((normal(), _row_params(temperature=0.0), hist(0)))
    out.append((normal(), _row_params(temperature=0.0, repetition_penalty=1.3), hist(40)))
    out.append((normal(), _row_params(temperature=0.8), hist(0)))
    out.append((normal(), _row_params(temperature=1.0, top_k=20), hist(0)))
    out.append((normal(), _row_params(temperature=1.0, top_k=1), hist(0)))
    out.append((normal(), _row_params(temperature=1.0, top_p=0.9), hist(0)))
    out.append((normal(), _row_params(temperature=1.0, top_p=1e-6), hist(0)))
    out.append((normal(), _row_params(temperature=1.0, top_p=0.9999), hist(0)))
    out.append((normal(), _row_params(temperature=0.7, min_p=0.05), hist(0)))
    out.append((normal(), _row_params(temperature=0.7, top_k=40, top_p=0.95, min_p=0.01,
                                      repetition_penalty=1.1, presence_penalty=0.5,
                                      frequency_penalty=0.3), hist(200)))
    out.append((normal(), _row_params(temperature=0.9, presence_penalty=1.5,
                                      frequency_penalty=0.5, repeat_last_n=16), hist(100)))
    out.append((normal(4.0), _row_params(temperature=2.0, top_p=0.5), hist(0)))
    ties = (rng.integers(-3, 4, V) * 0.5).astype(np.float32)          # heavy exact ties
    out.append((ties, _row_params(temperature=1.0, top_p=0.6), hist(0)))
    out.append((ties.copy(), _row_params(temperature=0.0), hist(0)))
    ninf = normal()
    ninf[rng.random(V) < 0.7] = -np.inf                               # mostly masked row
    out.append((ninf, _row_params(temperature=1.0, top_k=50, top_p=0.8), hist(0)))
    out.append((np.full(V, -np.inf, np.float32), _row_params(temperature=1.0, top_p=0.9),
                hist(0)))                                             # nothing finite
    nan = normal()
    nan[rng.integers(0, V, 3)] = np.nan
    out.append((nan, _row_params(temperature=1.0), hist(0)))
    return out


def make(V: int, seed: int, path: str) -> None:
    rng = np.random.default_rng(seed)
    cs = cases(V, rng)
    B = len(cs)
    logits = np.stack([c[0] for c in cs]).astype(np.float32)
    params = np.stack([c[1] for c in cs]).astype(np.float64)
    hists = [c[2] for c in cs]
    hist_off = np.zeros(B + 1, np.uint32)
    hist_off[1:] = np.cumsum([h.size for h in hists])
    hist_ids = np.concatenate(hists).astype(np.uint32) if hist_off[-1] else np.zeros(0, np.uint32)
    uniforms = rng.random(B).astype(np.float32)
    uniforms[::5] = 0.0
    uniforms[1::7] = np.float32(0.99999994)
    tokens = np.zeros(B, np.uint32)
    trace = {k: np.zeros(B, np.float32 if k in ("topp_sum", "final_max", "final_sum", "cdf_at")
                         else np.uint32) for k in TRACE_KEYS}
    for b in range(B):
        p = o.Params(**params_from_row(params[b]))
        t, tr = o.sample_logits_r(logits[b], p, hists[b], float(uniforms[b]))
        tokens[b] = t
        for k in TRACE_KEYS:
            trace[k][b] = tr[k]
    np.savez_compressed(path, logits=logits, params=params, hist_off=hist_off, hist_ids=hist_ids,
                        uniforms=uniforms, tokens=tokens,
                        **{"trace_" + k: v for k, v in trace.items()})
    print(f"wrote {path}: B={B} V={V}")


FIXTURES = (("sampler_v257.npz", 257, 11), ("sampler_v4096.npz", 4096, 12))

if __name__ == "__main__":
    for name, V, seed in FIXTURES:
        make(V, seed, os.path.join(HERE, name))
