"""GPU: the device-resident decode loop against the oracle's Sampler::sample
loop (sampling.rs:429-433: sample_logits, then record), from the fresh-run
seeding of lumen_sampler_decode_seed (GpuSamplerRunCfg, compute/mod.rs:202-227).

Every step's token is compared with the oracle's, the oracle keeping the
history and the Xorshift64 state on the host exactly as the reference does.
The rings are small so they wrap, with penalty windows below, equal to and
above the ring's capacity (whole-history windows carried past it).
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from lumen_amd.sampling import SamplingParams as SP  # noqa: E402


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


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_params(p: SP):
    from oracle import oracle as o

    return o.Params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                    repetition_penalty=p.repetition_penalty, presence_penalty=p.presence_penalty,
                    frequency_penalty=p.frequency_penalty, repeat_last_n=p.repeat_last_n)


def run_loop(eng, V, params, seeds, prompts, cap, steps, seed_params=True, hot=4.0, seed=0):
    """Device loop vs the oracle's loop; returns the device state."""
    import torch
    from lumen_amd.sampling import DeviceDecodeState
    from oracle import oracle as o

    B = len(params)
    rng = np.random.default_rng(seed)
    ds = DeviceDecodeState(eng, seeds, cap=cap, histories=prompts,
                           params=params if seed_params else None, vocab=V)
    orng = [o.Xorshift64(s) for s in seeds]
    ops = [oracle_params(p) for p in params]
    hist = [list(map(int, p)) for p in prompts]
    for step in range(steps):
        # logits that favour recently sampled ids, so the penalties decide
        lg = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        for b in range(B):
            for tok in hist[b][-3:]:
                lg[b, tok] += hot
        want = [o.sample_logits(lg[b].copy(), ops[b], np.array(hist[b], np.uint32), orng[b])
                for b in range(B)]
        x = torch.from_numpy(lg).to("cuda:0")
        log(f"case decode V={V} cap={cap} step {step}")
        _, got = ds.step(eng, x, params)
        assert got == want, f"step {step}: {got} vs {want}"
        for b in range(B):
            hist[b].append(want[b])  # SamplerState::record
    lens = ds.lens.cpu().numpy()
    ring = ds.ring.cpu().numpy().view(np.uint32)
    st = ds.rng.cpu().numpy().view(np.uint64)
    for b in range(B):
        assert lens[b] == len(hist[b])
        for k in range(max(0, len(hist[b]) - cap), len(hist[b])):
            assert ring[b, k % cap] == hist[b][k], (b, k)
        assert int(st[b]) == orng[b].state.value, b
    return ds


def _rows_for_cap(cap):
    return [
        SP(temperature=0.7, top_p=0.9, repetition_penalty=1.05),                # whole history
        SP(temperature=0.0, repetition_penalty=1.5, repeat_last_n=cap - 3),      # below the ring
        SP(temperature=0.9, top_k=40, frequency_penalty=0.7, repeat_last_n=cap),  # equal to it
        SP(temperature=1.0, presence_penalty=0.6, repeat_last_n=cap + 4),        # above it
        SP(temperature=1.1, min_p=0.05, repetition_penalty=1.2, repeat_last_n=1),
        SP(temperature=0.0, frequency_penalty=1.0),                              # whole history
    ]


@pytest.mark.parametrize("V", [248320])
def test_decode_20_steps_vs_oracle(eng, V):
    # 20+ tokens at the headline vocabulary, ring of 8 wrapping twice, prompts
    # longer and shorter than the ring
    cap = 8
    params = _rows_for_cap(cap)
    rng = np.random.default_rng(77)
    prompts = [rng.integers(0, V, size=n).astype(np.uint32) for n in (12, 3, 9, 2, 20, 5)]
    # rows whose window exceeds the ring only work while nothing has to be
    # counted again: row 3 (window 12) runs its 20 steps from a 2-token prompt
    # and fails once a token leaves its window (checked in the overflow test)
    run_loop(eng, V, params[:3] + params[4:], [11, 12, 13, 15, 16],
             [prompts[i] for i in (0, 1, 2, 4, 5)], cap, 22, seed=1)


def test_decode_small_vocab_long_run(eng):
    # 60 steps at V=600 (ids repeat, so the counts move both ways); ring of 8
    cap = 8
    params = _rows_for_cap(cap)
    params[3] = SP(temperature=1.0, presence_penalty=0.6, repeat_last_n=0)
    rng = np.random.default_rng(78)
    prompts = [rng.integers(0, 600, size=n).astype(np.uint32) for n in (30, 0, 8, 7, 1, 17)]
    run_loop(eng, 600, params, [21, 22, 23, 24, 25, 26], prompts, cap, 60, hot=2.0, seed=2)


def test_decode_unseeded_counts_follow_past_ring(eng):
    # without params at seeding the sampler counts the prompt itself; a
    # whole-history window then keeps following past the ring's capacity
    V, cap = 3000, 8
    params = [SP(temperature=0.0, repetition_penalty=1.5),
              SP(temperature=0.8, top_p=0.9, frequency_penalty=0.8)]
    rng = np.random.default_rng(79)
    prompts = [rng.integers(0, V, size=n).astype(np.uint32) for n in (3, 8)]
    run_loop(eng, V, params, [5, 6], prompts, cap, 25, seed_params=False, seed=3)


def test_decode_window_above_ring_overflows_when_counted_again(eng):
    # a window longer than the ring: counted while nothing leaves it, then
    # the first token that leaves cannot be found in the ring (status 3)
    import torch
    from lumen_amd.sampling import DeviceDecodeState

    V, cap = 500, 8
    params = [SP(temperature=0.0, repetition_penalty=1.5, repeat_last_n=10)]
    ds = DeviceDecodeState(eng, [1], cap=cap, histories=[[1, 2]], params=params, vocab=V)
    rng = np.random.default_rng(4)
    tr = torch.zeros((1, 16), dtype=torch.int32, device="cuda:0")
    statuses = []
    for step in range(12):
        x = torch.from_numpy(rng.standard_normal((1, V)).astype(np.float32)).cuda()
        toks, _ = ds.step(eng, x, params, trace=tr, sync=False)
        torch.cuda.synchronize()
        statuses.append(int(tr.cpu().numpy()[0, 0]))
        if statuses[-1]:
            break
    # lengths 2..10 are counted (nothing leaves a 10-token window); at
    # length 11 the leaving token (position 0) is no longer in a ring of 8
    assert statuses == [0] * 9 + [3], statuses


def test_decode_empty_vocab_records_token_0(eng):
    # an empty vocabulary samples token 0 and records it (sampling.rs:458-460,
    # 429-433); the next call's counts follow it
    import torch
    from lumen_amd.sampling import DeviceDecodeState
    from oracle import oracle as o

    params = [SP(temperature=0.0, frequency_penalty=1.0), SP(temperature=0.9)]
    ds = DeviceDecodeState(eng, [3, 4], cap=4, histories=[[7, 7], [1]], params=params, vocab=50)
    empty = torch.empty((2, 0), dtype=torch.float32, device="cuda:0")
    toks, _ = ds.step(eng, empty, params, sync=False)
    torch.cuda.synchronize()
    assert toks.cpu().tolist() == [0, 0]
    assert ds.lens.cpu().tolist() == [3, 2]
    lg = np.random.default_rng(9).standard_normal((2, 50)).astype(np.float32)
    lg[0, 0] = lg[0].max() + 0.5  # token 0's count (1) must pull it below others
    orng = [o.Xorshift64(3), o.Xorshift64(4)]
    want = [o.sample_logits(lg[0].copy(), oracle_params(params[0]), np.array([7, 7, 0], np.uint32), orng[0]),
            o.sample_logits(lg[1].copy(), oracle_params(params[1]), np.array([1, 0], np.uint32), orng[1])]
    _, got = ds.step(eng, torch.from_numpy(lg).cuda(), params)
    assert got == want


def test_first_call_under_capture_is_refused():
    # A fresh context's first call must set up device buffers; under stream
    # capture it refuses with a clear error instead of recording a memset or
    # an allocation into the graph. After one eager call the same step
    # captures.
    import torch
    from lumen_amd.sampling import DeviceDecodeState, Engine

    e = Engine(0)
    try:
        V = 2000
        params = [SP(temperature=0.8, top_p=0.9, repetition_penalty=1.2, repeat_last_n=4)] * 2
        x = torch.from_numpy(np.random.default_rng(1).standard_normal((2, V)).astype(np.float32)).cuda()
        ds = DeviceDecodeState(e, [1, 2], cap=16, histories=[[1, 2], [3]])
        tok = torch.empty(2, dtype=torch.int32, device="cuda:0")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        err = None
        try:
            with torch.cuda.graph(g):
                ds.step(e, x, params, tokens_out=tok, sync=False)
        except Exception as ex:  # noqa: BLE001
            err = str(ex)
        assert err is not None and "capture" in err, err
        torch.cuda.synchronize()
        # eager once, then the capture works
        ds.step(e, x, params, tokens_out=tok, sync=False)
        torch.cuda.synchronize()
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2):
            ds.step(e, x, params, tokens_out=tok, sync=False)
        g2.replay()
        torch.cuda.synchronize()
        assert ds.lens.cpu().tolist() == [4, 3]
    finally:
        e.close()


def test_sampler_state_decoder_reaches_the_guard():
    # Sampler.sample with a decoder on its SamplerState (sampling.rs:343-378):
    # the anti-restate sub-word rule sees it, as in the oracle's loop
    import torch
    from lumen_amd.sampling import Sampler, TokenBytes, Xorshift64
    from oracle import oracle as o

    V = 400
    rng = np.random.default_rng(12)
    alpha = [b"ab", b"ba", b"abab", b" ab", b"b", b"cab"]
    table = [alpha[int(i)] * int(rng.integers(1, 3)) for i in rng.integers(0, len(alpha), V)]
    p = SP(temperature=0.0, anti_restate=True)
    smp = Sampler(p, Xorshift64(1))
    smp.state.decoder = TokenBytes(table)
    hist = []
    op = o.Params(temperature=0.0, anti_restate=True)
    vetoed = 0
    for step in range(12):
        lg = (rng.standard_normal(V) * 2).astype(np.float32)
        for j, tok in enumerate(sorted(set(hist[-6:]))):
            lg[tok] = 9.0 - 0.25 * j  # the recent tokens lead
        want = o.sample_logits(lg.copy(), op, np.array(hist, np.uint32), o.Xorshift64(1), table)
        no_dec = o.sample_logits(lg.copy(), op, np.array(hist, np.uint32), o.Xorshift64(1), None)
        vetoed += want != no_dec
        log(f"case sampler decoder step {step}")
        got = smp.sample(torch.from_numpy(lg).cuda())
        assert got == want, (step, got, want)
        hist.append(want)
    assert smp.state.history == hist
    assert vetoed > 0  # the decoder changed at least one choice
