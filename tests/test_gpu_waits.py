"""Bounded cross-workgroup waits, forced from the host.

A row split over several workgroups waits for its other workgroups at a few
points (the row barrier, the exact-sum walker). lumen_sampler_set_wait_limit
bounds every such wait by the device wall clock; 0 makes every wait give up
at once. Then every split row that waits must fall back to the exact
single-workgroup path: every kernel still exits normally, the tokens and
intermediate sums stay identical to the oracle's, the give-ups are counted,
and the rows' coordination blocks are left clean for the next calls (checked
by alternating forced and normal calls on the same context).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from lumen_amd.sampling import SamplingParams as SP  # noqa: E402
from tests import parity  # noqa: E402


@pytest.fixture(scope="module")
def eng():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from lumen_amd.sampling import Engine

    e = Engine(0)
    yield e
    e.close()


def _batch(seed, B, V):
    rng = np.random.default_rng(seed)
    lg = (rng.normal(0, 3, (B, V)) + rng.gumbel(0, 1, (B, V))).astype(np.float32)
    kinds = [SP(temperature=1.0, top_p=0.9),                       # register-resident top-p
             SP(temperature=0.8),                                  # plain temperature
             SP(temperature=0.7, repetition_penalty=1.05),         # plain + penalties
             SP(temperature=1.0, top_p=0.95, presence_penalty=0.5),  # top-p + penalties
             SP(temperature=0.0),                                  # greedy (no waits)
             SP(temperature=0.6, top_k=100, top_p=0.95),           # top-k (no waits)
             SP(temperature=1.0, top_p=0.99, min_p=0.05),
             SP(temperature=1.3, top_p=0.5)]
    params = [kinds[b % len(kinds)] for b in range(B)]
    hists = [rng.integers(0, V, int(rng.integers(0, 400))).astype(np.uint32) for _ in range(B)]
    u = rng.random(B).astype(np.float32)
    return lg, params, hists, u


def _check(eng, lg, params, hists, u, name):
    rep = parity.compare(eng, lg, params, hists, u)
    assert not rep["token_mismatch"], f"{name}: {rep['token_mismatch'][:5]}"
    assert not rep["trace_mismatch"], f"{name}: {rep['trace_mismatch'][:3]}"
    assert set(rep["status"]) <= {0}, f"{name}: status {set(rep['status'])}"


@pytest.mark.parametrize("B,V", [(8, 248_320), (64, 151_936), (2, 600_000)])
def test_forced_give_up_is_exact_and_counted(eng, B, V):
    lg, params, hists, u = _batch(1000 + B, B, V)
    before = eng.wait_timeouts()
    try:
        eng.set_wait_limit(0)
        for rep in range(2):
            print(f"forced give-up B={B} V={V} call {rep}", flush=True)
            _check(eng, lg, params, hists, u, f"limit 0, call {rep}")
        forced = eng.wait_timeouts() - before
        assert forced > 0, "no wait gave up with a zero limit"
    finally:
        eng.set_wait_limit(2000)
    # the same context, the bound back to its default: the coordination
    # blocks the forced calls left behind must be clean
    mid = eng.wait_timeouts()
    for rep in range(2):
        print(f"default limit B={B} V={V} call {rep}", flush=True)
        _check(eng, lg, params, hists, u, f"default limit, call {rep}")
    assert eng.wait_timeouts() == mid, "a wait gave up with the GPU to this process alone"


def test_wait_limit_arguments(eng):
    from lumen_amd import _native

    L = _native.load()
    assert L.lumen_sampler_set_wait_limit(None, 5) == -1
    assert L.lumen_sampler_wait_timeouts(eng._h, None) == -1
