"""The committed golden vectors (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU oracle).

* CPU: the oracle still reproduces every stored token and intermediate value
  bit for bit, so a change to the oracle cannot silently move the target the
  GPU tests compare against. The oracle's stages are pinned independently by
  brute force and closed forms in test_oracle_pins.py.
* GPU: the engine reproduces the stored tokens and intermediate values, in
  both launch modes, without running the oracle.
"""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from tests.golden.make_golden import FIXTURES, TRACE_KEYS, params_from_row

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FLOATS = ("topp_sum", "final_max", "final_sum", "cdf_at")


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    off = d["hist_off"]
    d["hists"] = [d["hist_ids"][off[b]:off[b + 1]] for b in range(off.size - 1)]
    return d


def fbits(x) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def same(a, b) -> bool:
    if np.isnan(a) or np.isnan(b):
        return bool(np.isnan(a) and np.isnan(b))
    return fbits(a) == fbits(b)


def checked_fields(d, b):
    """The intermediate values the chain actually computed for row b."""
    t = {k: d["trace_" + k][b] for k in TRACE_KEYS}
    if t["greedy"]:
        return []
    out = []
    if t["topk_applied"]:
        out += ["topk_survivors", "topk_cutoff_key"]
    if t["topp_applied"]:
        out += ["topp_sum", "topp_kept"]
    out += ["final_max", "cdf_at"]
    if not t["final_uniform"]:
        out.append("final_sum")
    return out


@pytest.mark.parametrize("name", [f[0] for f in FIXTURES])
def test_golden_fixture_shapes(name):
    d = load(name)
    B, V = d["logits"].shape
    assert d["params"].shape[0] == B and d["uniforms"].shape == (B,) and d["tokens"].shape == (B,)
    assert V <= 4096 and B >= 16
    assert all(int(t) < V for t in d["tokens"])


@pytest.mark.parametrize("name", [f[0] for f in FIXTURES])
def test_oracle_reproduces_golden(name):
    from oracle import oracle as o

    d = load(name)
    for b in range(d["logits"].shape[0]):
        p = o.Params(**params_from_row(d["params"][b]))
        t, tr = o.sample_logits_r(d["logits"][b], p, d["hists"][b], float(d["uniforms"][b]))
        assert t == int(d["tokens"][b]), (name, b)
        for k in checked_fields(d, b):
            want = d["trace_" + k][b]
            if k in FLOATS:
                assert same(tr[k], want), (name, b, k, tr[k], want)
            else:
                assert int(tr[k]) == int(want), (name, b, k, tr[k], want)


@pytest.fixture(scope="module", params=["split", "single"])
def eng(request):
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from lumen_amd.sampling import Engine

    if request.param == "single":
        os.environ["LUMEN_SAMPLER_SINGLE"] = "1"
    else:
        os.environ.pop("LUMEN_SAMPLER_SINGLE", None)
    e = Engine(0)
    yield e
    e.close()
    os.environ.pop("LUMEN_SAMPLER_SINGLE", None)


@pytest.mark.gpu
@pytest.mark.parametrize("name", [f[0] for f in FIXTURES])
def test_engine_matches_golden(eng, name):
    import torch

    from lumen_amd.sampling import SamplingParams
    from tests.parity import decode_trace

    d = load(name)
    print(f"case golden {name}", flush=True)
    B, V = d["logits"].shape
    params = [SamplingParams(**params_from_row(d["params"][b])) for b in range(B)]
    dev = torch.from_numpy(d["logits"]).cuda()
    trace = torch.zeros((B, 16), dtype=torch.int32, device="cuda")
    _, host = eng.sample_batch(dev, params, histories=d["hists"], uniforms=d["uniforms"],
                               trace=trace)
    torch.cuda.synchronize()
    tr = decode_trace(trace.cpu().numpy().view(np.uint32))
    bad = []
    for b in range(B):
        if int(host[b]) != int(d["tokens"][b]):
            bad.append((b, "token", host[b], int(d["tokens"][b])))
        for k in checked_fields(d, b):
            if k in ("topk_applied", "topp_applied"):
                continue
            want = d["trace_" + k][b]
            got = tr[b][k]
            ok = same(got, want) if k in FLOATS else int(got) == int(want)
            if not ok:
                bad.append((b, k, got, want))
    assert not bad, (name, bad)
