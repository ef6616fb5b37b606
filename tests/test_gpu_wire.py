"""Wire-level requests sampled on the GPU against the oracle.

An OpenAI request body is resolved into SamplingParams by lumen_amd/wire.py
(ranges, server defaults, zero-normalized penalties, the env overrides and the
per-request seed: lumen-server/src/wire/openai.rs:184-243, 357-381 and
wire/mod.rs:69-92), then every resolved request is decoded for several steps
by the reference's own loop, Sampler::sample (sampling.rs:397-434: draw from
the request's Xorshift64, then record the token), once on the gfx950 engine
through the C ABI and once by the oracle. Tokens must be identical at every
step.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from lumen_amd import wire  # noqa: E402
from lumen_amd.sampling import SamplingParams  # noqa: E402
from oracle import oracle as o  # noqa: E402
from tests import parity  # noqa: E402

# request bodies as a client sends them (JSON numbers); every resolved field
# is exercised: the defaults, explicit zeros that the server turns into None,
# explicit seeds and missing ones, top-k / top-p / min-p and greedy
REQUESTS = [
    {},
    {"seed": 11},
    {"temperature": 0, "seed": 3},
    {"temperature": 0, "presence_penalty": 0.0, "frequency_penalty": 0.0},
    {"temperature": 1.0, "top_p": 0.9, "seed": 5},
    {"temperature": 0.8, "top_k": 40, "top_p": 0.95, "seed": 6},
    {"temperature": 0.6, "top_p": 0.95, "min_p": 0.05, "presence_penalty": 0.5,
     "frequency_penalty": 0.25, "seed": 7},
    {"temperature": 1.3, "top_k": 4096, "frequency_penalty": 0.0, "seed": 8},
    {"temperature": 2.0, "top_p": 1.0, "seed": 9},
    {"temperature": 0.7, "top_p": 0.0, "presence_penalty": 1.5, "seed": 10},
]


@pytest.fixture(scope="module")
def eng():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from lumen_amd.sampling import Engine

    e = Engine(0)
    yield e
    e.close()


def _decode(eng, params, logits_steps, hist0):
    """Sampler::sample on the engine and on the oracle, step by step, each
    side with its own history and its own Xorshift64 from the request seed."""
    import torch

    B = len(params)
    rng_gpu = [o.Xorshift64(p.seed) for p in params]
    rng_ref = [o.Xorshift64(p.seed) for p in params]
    hist_gpu = [list(h) for h in hist0]
    hist_ref = [list(h) for h in hist0]
    mism = []
    for step, lg in enumerate(logits_steps):
        # greedy rows consume no draw (sampling.rs:468-476)
        u_gpu = np.array([rng_gpu[b].next_f32() if params[b].temperature > 0 else 0.0
                          for b in range(B)], np.float32)
        _, got = eng.sample_batch(torch.from_numpy(lg).cuda(), params,
                                  histories=[np.asarray(h, np.uint32) for h in hist_gpu],
                                  uniforms=u_gpu)
        for b in range(B):
            r = rng_ref[b].next_f32() if params[b].temperature > 0 else 0.0
            want = o.sample_logits_r(lg[b], parity.to_oracle_params(params[b]),
                                     np.asarray(hist_ref[b], np.uint32), r)[0]
            if int(got[b]) != want:
                mism.append((step, b, int(got[b]), want))
            hist_gpu[b].append(int(got[b]))
            hist_ref[b].append(want)
    return mism


@pytest.mark.parametrize("moe,env", [
    (False, {}),
    (True, {"LUMEN_REPEAT_LAST_N": "64"}),
    (False, {"LUMEN_REPETITION_PENALTY": "1.2", "LUMEN_FREQUENCY_PENALTY": "0.1",
             "LUMEN_REPEAT_LAST_N": "0"}),
])
def test_wire_requests_decode_like_the_oracle(eng, monkeypatch, moe, env):
    for k in ("LUMEN_REPEAT_LAST_N", "LUMEN_REPETITION_PENALTY", "LUMEN_FREQUENCY_PENALTY",
              "LUMEN_ANTI_RESTATE"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    params = [wire.sampling_from_request(r, wire.ModelHint(moe=moe)) for r in REQUESTS]
    assert all(isinstance(p, SamplingParams) and p.seed is not None for p in params)
    # what the wire layer resolved is what the tests below sample with
    assert params[0].temperature == pytest.approx(0.7)
    assert params[0].repetition_penalty == (float(np.float32(1.2)) if "LUMEN_REPETITION_PENALTY" in env
                                           else (1.03 if moe else 1.05))
    assert params[3].presence_penalty is None
    rng = np.random.default_rng(404 + len(env))
    B, V, steps = len(params), 151_936, 6
    hist0 = [rng.integers(0, V, int(rng.integers(0, 600))).astype(np.uint32) for _ in range(B)]
    logits_steps = []
    for _ in range(steps):
        lg = (rng.normal(0, 2.5, (B, V)) + rng.gumbel(0, 1, (B, V))).astype(np.float32)
        # the recent history is boosted so that the penalties change the winner
        for b in range(B):
            lg[b, hist0[b][-20:]] += 6.0
        logits_steps.append(lg)
    mism = _decode(eng, params, logits_steps, hist0)
    assert not mism, f"wire-resolved decode differs from the oracle: {mism[:8]}"


def test_wire_rejects_before_sampling():
    """A request outside the server's ranges never reaches the sampler
    (openai.rs:357-381): the error names the field."""
    for bad, field in (({"temperature": -0.1}, "temperature"), ({"top_p": 1.01}, "top_p")):
        with pytest.raises(wire.WireError) as e:
            wire.sampling_from_request(bad)
        assert e.value.field == field
