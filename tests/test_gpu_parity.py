"""GPU parity: the gfx950 engine against the CPU oracle, through the C ABI.

Bar: token ids, top-k cutoff and survivor counts, penalized logits and every
intermediate f32 sum (top-p softmax sum, final softmax sum, the CDF value at
the draw) must be bit-identical to the oracle's.
"""
import math
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from lumen_amd.sampling import SamplingParams as SP  # noqa: E402
from tests import parity  # noqa: E402


@pytest.fixture(scope="module", params=["split", "single"])
def eng(request):
    """The engine in its default mode (several workgroups per row) and with
    one workgroup per row (LUMEN_SAMPLER_SINGLE)."""
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


def assert_clean(rep, name):
    msg = f"{name}: tokens {rep['token_mismatch'][:5]} trace {rep['trace_mismatch'][:3]} " \
          f"pen {rep['pen_mismatch'][:3]} status {set(rep['status'])}"
    assert not rep["token_mismatch"], msg
    assert not rep["trace_mismatch"], msg
    assert not rep["pen_mismatch"], msg
    assert set(rep["status"]) <= {0}, msg


def run_case(eng, logits, params, hists=None, uniforms=None, name="case", **kw):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    B = logits.shape[0]
    if hists is None:
        hists = [np.zeros(0, np.uint32)] * B
    if uniforms is None:
        rng = np.random.default_rng(abs(hash(name)) % 2**32)
        uniforms = rng.random(B).astype(np.float32)
    log(f"case {name} B={B} V={logits.shape[1]}")
    rep = parity.compare(eng, logits, params, hists, uniforms, **kw)
    assert_clean(rep, name)
    return rep


# ---- the reference's own small cases, on the GPU ---------------------------

def test_reference_small_cases(eng):
    cases = [
        ([1.0, 5.0, 3.0, 2.0], SP(temperature=0.0), []),
        ([0.0, 0.0, 0.0, 9.0, 9.0, 9.0], SP(temperature=0.0), []),
        ([7.0, 7.0, 7.0, 7.0], SP(temperature=0.0), []),
        ([1.0, 5.0, 3.0, 2.0], SP(temperature=0.0, top_p=0.5, top_k=1, min_p=0.9,
                                  repetition_penalty=2.0, presence_penalty=10.0,
                                  frequency_penalty=10.0), [1]),
        ([3.0, 3.5], SP(temperature=0.0, frequency_penalty=10.0, repeat_last_n=2), [0, 0, 1, 1]),
        ([3.0, 3.5], SP(temperature=0.0, frequency_penalty=10.0, repeat_last_n=1), [0, 0, 0, 1]),
        ([1.0, 5.0, 3.0, 2.0, 4.0], SP(temperature=1.0, top_k=1), []),
        ([1.0, 2.0, 2.0, 0.5], SP(temperature=1.0, top_k=1), []),
        ([0.0, 0.0, 0.0, 10.0], SP(temperature=1.0, top_p=0.5), []),
        ([0.0, 0.0, 0.0, 10.0], SP(temperature=1.0, min_p=0.5), []),
        ([3.0, 2.0, 1.0, 0.5], SP(temperature=1.0, top_p=0.6, top_k=2, repetition_penalty=10.0), [3]),
        ([4.0, 3.0, 2.0, 1.0], SP(temperature=0.5, top_p=0.85), []),
        ([5.0, 2.0, 1.0, 0.0], SP(temperature=1.0, min_p=0.1), []),
        ([-5.0, 5.0, 0.0, 0.0], SP(temperature=1.0), []),
        ([1.0, 1.0], SP(temperature=1.0, repetition_penalty=10.0), [0]),
    ]
    for i, (lg, p, h) in enumerate(cases):
        for r in (0.0, 0.1, 0.5, 0.73, 0.999):
            run_case(eng, np.array(lg, np.float32), [p], [np.array(h, np.uint32)],
                     np.array([r], np.float32), name=f"ref{i}_r{r}", check_pen=True)


def test_determinism_sin_logits(eng):
    base = np.sin(np.arange(1000, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    B = 32
    lg = np.tile(base, (B, 1))
    rng = np.random.default_rng(7)
    params = [SP(temperature=0.7, top_p=0.9, top_k=40)] * B
    run_case(eng, lg, params, uniforms=rng.random(B).astype(np.float32), name="sin1000")


# ---- randomized small-V sweep over the parameter surface --------------------

def random_params(rng, V):
    T = float(rng.choice([0.0, 0.0, 0.3, 0.7, 1.0, 1.5, 1e-3]))
    p = SP(temperature=T)
    if rng.random() < 0.5:
        p.top_k = int(rng.choice([1, 2, 3, 5, 40, V - 1, V, V + 5]))
    if rng.random() < 0.5:
        p.top_p = float(rng.choice([0.1, 0.5, 0.9, 0.95, 0.999, 1.0]))
    if rng.random() < 0.3:
        p.min_p = float(rng.choice([0.01, 0.1, 0.5]))
    if rng.random() < 0.4:
        p.repetition_penalty = float(rng.choice([1.05, 1.1, 2.0, 0.9]))
    if rng.random() < 0.3:
        p.presence_penalty = float(rng.choice([0.5, 1.5, -0.3]))
    if rng.random() < 0.3:
        p.frequency_penalty = float(rng.choice([0.25, 0.8]))
    if rng.random() < 0.2:
        p.repeat_last_n = int(rng.choice([1, 4, 64]))
    return p


def random_logits(rng, V, style):
    if style == 0:
        return rng.normal(0, 3, V).astype(np.float32)
    if style == 1:  # heavy ties
        return (np.round(rng.normal(0, 2, V) * 4) / 4).astype(np.float32)
    if style == 2:  # very peaked
        x = rng.normal(0, 1, V).astype(np.float32)
        x[rng.integers(0, V)] += 40
        return x
    if style == 3:  # with -inf holes
        x = rng.normal(0, 2, V).astype(np.float32)
        x[rng.random(V) < 0.3] = -np.inf
        return x
    if style == 4:  # flat
        return rng.normal(0, 0.1, V).astype(np.float32)
    return rng.uniform(-100, 100, V).astype(np.float32)


@pytest.mark.parametrize("V", [1, 2, 3, 17, 64, 1000, 4099])
def test_random_small_vocab(eng, V):
    rng = np.random.default_rng(V)
    B = 48
    lg = np.stack([random_logits(rng, V, b % 6) for b in range(B)])
    params = [random_params(rng, V) for _ in range(B)]
    hists = [rng.integers(0, V + 3, int(rng.integers(0, 40))).astype(np.uint32) for _ in range(B)]
    run_case(eng, lg, params, hists, rng.random(B).astype(np.float32), name=f"rand{V}",
             check_pen=True)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("V,dtype", [(151_936, "f32"), (248_320, "f32"), (151_936, "bf16")])
def test_random_full_vocab(eng, V, dtype, seed):
    # random parameter mixes over full-size rows: every split path and its
    # fallbacks, the weighted block plan of a mixed batch, penalties from
    # random histories, and bf16 rows
    from lumen_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(V + (7 if dtype == "bf16" else 0) + 1000 * seed)
    B = 24
    lg = np.stack([random_logits(rng, V, b % 6) for b in range(B)])
    params = []
    for _ in range(B):
        p = random_params(rng, V)
        if p.top_k is not None and p.top_k > V:
            p.top_k = int(rng.choice([50, 1024, 3000]))
        params.append(p)
    hists = [rng.integers(0, V, int(rng.integers(0, 3000))).astype(np.uint32) for _ in range(B)]
    u = rng.random(B).astype(np.float32)
    log(f"case random full V={V} {dtype} seed {seed}")
    if dtype == "bf16":
        bits = to_bf16_bits(lg)
        f32 = (bits.astype(np.uint32) << 16).view(np.float32)
        rep = parity.compare(eng, f32, params, hists, u, dtype="bf16", bf16_bits=bits)
    else:
        rep = parity.compare(eng, lg, params, hists, u)
    assert_clean(rep, f"random full V={V} {dtype}")


@pytest.mark.parametrize("B,seed", [(1, 0), (1, 1), (1, 2), (5, 0), (5, 1), (64, 0), (64, 1)])
def test_random_full_vocab_batch_sizes(eng, B, seed):
    # batch sizes that change the grid: 16 slices per row (B = 1, 5), the
    # weighted block plan (B = 64)
    rng = np.random.default_rng(10_000 + 100 * B + seed)
    V = 248_320
    lg = np.stack([random_logits(rng, V, int(rng.integers(0, 6))) for b in range(B)])
    params = []
    for _ in range(B):
        p = random_params(rng, V)
        if p.top_k is not None and p.top_k > V:
            p.top_k = int(rng.choice([20, 500, 2048, 4000]))
        params.append(p)
    hists = [rng.integers(0, V, int(rng.integers(0, 5000))).astype(np.uint32) for _ in range(B)]
    run_case(eng, lg, params, hists, rng.random(B).astype(np.float32),
             name=f"random B={B} seed {seed}")


@pytest.mark.parametrize("seed", list(range(12)))
def test_fuzz_shapes(eng, seed):
    # random vocabularies (unaligned sizes too), batch sizes, dtypes, row
    # strides, logit styles and parameter mixes
    from lumen_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(50_000 + seed)
    V = int(rng.choice([100_003, 151_936, 200_001, 248_320, 262_139]))
    B = int(rng.integers(1, 41))
    bf16 = bool(rng.random() < 0.35)
    lg = np.stack([random_logits(rng, V, int(rng.integers(0, 6))) for _ in range(B)])
    params = []
    for _ in range(B):
        p = random_params(rng, V)
        if p.top_k is not None and p.top_k > V:
            p.top_k = int(rng.choice([1, 7, 64, 1000, 2048, 2049, 5000]))
        if rng.random() < 0.15:
            p.top_p = float(rng.choice([0.99999, 0.9999, 1e-6]))
        if rng.random() < 0.1:
            p.temperature = float(rng.choice([1e-4, 2.0, 1.9999]))
        params.append(p)
    hists = [rng.integers(0, V, int(rng.integers(0, 6000))).astype(np.uint32) for _ in range(B)]
    u = rng.random(B).astype(np.float32)
    stride = V + int(rng.choice([0, 0, 1, 7, 64]))
    log(f"case fuzz seed {seed} B={B} V={V} bf16={bf16} stride={stride}")
    if bf16:
        bits = to_bf16_bits(lg)
        f32 = (bits.astype(np.uint32) << 16).view(np.float32)
        rep = parity.compare(eng, f32, params, hists, u, dtype="bf16", bf16_bits=bits,
                             row_stride=stride)
    else:
        rep = parity.compare(eng, lg, params, hists, u, row_stride=stride)
    assert_clean(rep, f"fuzz seed {seed}")


def test_huge_tie_groups(eng):
    # probability groups larger than a window: one value repeated 20,000
    # times with the top-p crossing inside the group (its lowest ids are
    # kept), +0 and -0 together (two keys, one p), and groups above and below
    # the crossing
    rng = np.random.default_rng(91)
    V = 248_320
    rows, params = [], []
    r = rng.normal(0, 1, V).astype(np.float32)
    r[rng.choice(V, 20_000, replace=False)] = 1.0
    rows.append(r)
    params.append(SP(temperature=1.0, top_p=0.5))
    r = (np.round(rng.normal(0, 2, V) * 4) / 4).astype(np.float32)  # +0 and -0: ~12K tokens
    rows.append(r)
    params.append(SP(temperature=0.9, top_p=0.995))
    r = np.zeros(V, np.float32)
    r[: V // 2] = -0.0
    r[rng.choice(V, 30, replace=False)] = 3.0
    rows.append(r)
    params.append(SP(temperature=1.0, top_p=0.3))
    r = rng.integers(-3, 4, V).astype(np.float32)  # 7 values, ~35K tokens each
    rows.append(r)
    params.append(SP(temperature=1.2, top_p=0.97, min_p=0.01))
    B = len(rows)
    lg = np.stack(rows)
    for draws in (rng.random(B), np.full(B, 0.9999)):
        run_case(eng, lg, params, [np.zeros(0, np.uint32)] * B, draws.astype(np.float32),
                 name="huge_ties")


def test_window_edge_probability_ties(eng):
    # Logits on a 1/4 grid with ~7,500 exact zeros: a top-p window edge
    # planned between +0 and the smallest subnormal key leaves the zeros,
    # whose p equals the edge's, below the edge. The window must move its
    # edge up rather than overflow (this once reported a row failure).
    rng = np.random.default_rng(77)
    V, B = 151_936, 4
    lg = (np.round(rng.normal(0, 2, (B, V)) * 4) / 4).astype(np.float32)
    params = [SP(temperature=1.5, top_p=0.999, presence_penalty=1.5),
              SP(temperature=1.0, top_p=0.9999),
              SP(temperature=0.7, top_p=0.99999, min_p=0.001),
              SP(temperature=1.0, top_p=0.999, top_k=3000)]
    hists = [rng.integers(0, V, 89).astype(np.uint32), np.zeros(0, np.uint32),
             np.zeros(0, np.uint32), rng.integers(0, V, 10).astype(np.uint32)]
    run_case(eng, lg, params, hists, rng.random(B).astype(np.float32), name="edge_ties")


def test_special_values(eng):
    V = 300
    rows, params = [], []
    nan = np.float32(np.nan)
    mk = []
    x = np.zeros(V, np.float32); x[5] = np.inf; mk.append(x)
    x = np.full(V, -np.inf, np.float32); mk.append(x)
    x = np.zeros(V, np.float32); x[7] = nan; mk.append(x)
    x = np.linspace(-1, 1, V).astype(np.float32); x[9] = nan; x[10] = np.inf; mk.append(x)
    x = np.zeros(V, np.float32); x[3] = -0.0; mk.append(x)
    x = np.full(V, 3.0, np.float32); mk.append(x)
    x = np.linspace(-200, 0, V).astype(np.float32); mk.append(x)
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    x = np.zeros(V, np.float32); x[11] = neg_nan; mk.append(x)
    for x in mk:
        for p in (SP(temperature=0.0), SP(temperature=1.0), SP(temperature=1.0, top_k=5),
                  SP(temperature=0.8, top_p=0.9), SP(temperature=1.0, top_k=1),
                  SP(temperature=2.0, min_p=0.2), SP(temperature=1.0, top_k=10, top_p=0.5)):
            rows.append(x)
            params.append(p)
    lg = np.stack(rows)
    rng = np.random.default_rng(11)
    run_case(eng, lg, params, uniforms=rng.random(len(params)).astype(np.float32),
             name="special")


def test_denormal_probabilities(eng):
    # probabilities in the subnormal range exercise the low end of the exact sums
    V = 2000
    x = np.linspace(-103.5, 0, V).astype(np.float32)
    lg = np.stack([x, x[::-1].copy(), np.concatenate([x[:1000], np.full(1000, -90, np.float32)])])
    params = [SP(temperature=1.0), SP(temperature=1.0, top_p=0.999), SP(temperature=0.5)]
    run_case(eng, lg, params, uniforms=np.array([0.9999, 0.5, 0.999999], np.float32),
             name="denormal")


def test_draw_edges(eng):
    # r = 0, r just below 1 (fall-through), r equal to a CDF value
    V = 8
    lg = np.tile(np.zeros(V, np.float32), (4, 1))
    params = [SP(temperature=1.0)] * 4
    us = np.array([0.0, 0.99999994, 0.125, 0.875], np.float32)
    run_case(eng, lg, params, uniforms=us, name="draw_edges")


# ---- streaming path: no top-k, windows over the probability order ---------

@pytest.mark.parametrize("V,sd,p", [(50_000, 1.0, 0.99), (50_000, 0.05, 0.9), (20_000, 3.0, 0.5)])
def test_large_path_topp_windows(eng, V, sd, p):
    rng = np.random.default_rng(V + int(sd * 100))
    B = 6
    lg = rng.normal(0, sd, (B, V)).astype(np.float32)
    params = [SP(temperature=1.0, top_p=p), SP(temperature=0.7, top_p=p),
              SP(temperature=1.0, top_p=p, min_p=0.05), SP(temperature=1.3),
              SP(temperature=1.0, top_p=p, repetition_penalty=1.3),
              SP(temperature=1.0, top_k=V // 2, top_p=p)]
    hists = [rng.integers(0, V, 100).astype(np.uint32) for _ in range(B)]
    run_case(eng, lg, params, hists, rng.random(B).astype(np.float32), name=f"win{V}_{sd}_{p}",
             check_pen=True)


def test_unaligned_and_strided_rows(eng):
    rng = np.random.default_rng(99)
    V = 10_001
    B = 5
    lg = rng.normal(0, 2, (B, V)).astype(np.float32)
    params = [SP(temperature=0.0), SP(temperature=1.0, top_k=30), SP(temperature=1.0, top_p=0.8),
              SP(temperature=0.9), SP(temperature=1.0, top_k=3, top_p=0.5)]
    run_case(eng, lg, params, uniforms=rng.random(B).astype(np.float32), name="stride",
             row_stride=V + 3)


def test_bf16_rows(eng):
    from lumen_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(5)
    V, B = 30_000, 8
    bits = to_bf16_bits(rng.normal(0, 1, (B, V)).astype(np.float32))
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    params = [SP(temperature=1.0, top_p=0.99)] * 4 + [SP(temperature=0.0), SP(temperature=1.0, top_k=20),
                                                     SP(temperature=0.8), SP(temperature=1.0, top_p=0.5)]
    log("case bf16")
    rep = parity.compare(eng, f32, params, [np.zeros(0, np.uint32)] * B,
                         rng.random(B).astype(np.float32), dtype="bf16", bf16_bits=bits)
    assert_clean(rep, "bf16")


def test_bf16_topp_by_value(eng):
    # bf16 rows take the top-p walk over distinct values (one workgroup per
    # row): flat rows with large nuclei, heavy exact ties, distinct values
    # whose probabilities round equal (tiny p), a top-k mask in front
    # (top_k > 2048), min-p and temperature after, and crossings at
    # low and high top_p
    from lumen_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(17)
    V = 40_000
    rows, params = [], []
    for top_p in (0.3, 0.9, 0.99, 0.9999):
        rows.append(rng.normal(0, 1, V))
        params.append(SP(temperature=1.0, top_p=top_p))
    rows.append(rng.integers(-4, 5, V) * 0.5)                     # 17 distinct values
    params.append(SP(temperature=0.7, top_p=0.95))
    rows.append(rng.normal(0, 1, V) - 60.0 * (rng.random(V) < 0.5))  # a tail of tiny p
    params.append(SP(temperature=1.0, top_p=0.999999))
    rows.append(rng.normal(0, 2, V))
    params.append(SP(temperature=1.3, top_p=0.97, top_k=5000, min_p=0.001))
    rows.append(np.full(V, 1.5))                                  # one value everywhere
    params.append(SP(temperature=1.0, top_p=0.5))
    # distinct tiny values whose probabilities all round to 1/S1: the boundary
    # group holds the row maximum (placed last), so only part of it is kept
    rows.append(np.r_[rng.normal(0, 1, V - 1) * 1e-30, 4e-30])
    params.append(SP(temperature=1.0, top_p=0.5))
    rows.append(rng.integers(-4, 5, V) * 0.5)                     # tied maxima kept whole at T = 1
    params.append(SP(temperature=1.0, top_p=0.9))
    # a maximum of +0 and -0 (the key maximum is taken again with f32::max
    # semantics), exact zeros below the exp table's window
    z = np.minimum(rng.normal(0, 1, V), 0.0)
    z[rng.random(V) < 0.2] = 0.0
    z[rng.random(V) < 0.2] = -0.0
    rows.append(z)
    params.append(SP(temperature=1.0, top_p=0.9))
    bits = to_bf16_bits(np.array(rows, dtype=np.float32))
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    B = len(rows)
    for rep_i, u in enumerate((rng.random(B), np.full(B, 0.999), np.zeros(B))):
        log(f"case bf16 by value {rep_i}")
        rep = parity.compare(eng, f32, params, [np.zeros(0, np.uint32)] * B,
                             u.astype(np.float32), dtype="bf16", bf16_bits=bits)
        assert_clean(rep, f"bf16 by value {rep_i}")


def test_run_to_run_bit_identity(eng):
    import torch

    from lumen_amd.workloads import config3

    w = config3(seed=31, V=40_000, B=16)
    dev = torch.from_numpy(w.logits).cuda()
    u = np.random.default_rng(1).random(16).astype(np.float32)
    outs = []
    for _ in range(3):
        tr = torch.zeros((16, 16), dtype=torch.int32, device="cuda")
        t, h = eng.sample_batch(dev, w.params, histories=w.histories, uniforms=u, trace=tr)
        outs.append((h, tr.cpu().numpy().tobytes()))
    assert outs[0] == outs[1] == outs[2]


# ---- the benchmark configurations at full size ------------------------------

def _run_workload(eng, w, n_rows=None, seeds_offset=0):
    rows = range(w.batch) if n_rows is None else range(n_rows)
    rows = list(rows)
    from lumen_amd.sampling import Xorshift64

    u = np.array([Xorshift64(w.seeds[b] + seeds_offset).next_f32() for b in rows], np.float32)
    lg = w.logits_f32()[rows]
    params = [w.params[b] for b in rows]
    hists = [w.histories[b] for b in rows]
    log(f"case {w.name} rows={len(rows)} V={w.vocab}")
    if w.dtype == "bf16":
        rep = parity.compare(eng, lg, params, hists, u, dtype="bf16", bf16_bits=w.logits[rows])
    else:
        rep = parity.compare(eng, lg, params, hists, u, check_pen=True)
    assert_clean(rep, w.name)
    return rep


def test_config1_full(eng):
    from lumen_amd.workloads import config1, config1_greedy

    _run_workload(eng, config1())
    _run_workload(eng, config1_greedy())


def test_config3_full(eng):
    from lumen_amd.workloads import config3

    _run_workload(eng, config3())


def test_config5_full(eng):
    from lumen_amd.workloads import config5

    _run_workload(eng, config5())


def test_defaults_full(eng):
    # the parameter sets callers send most: the reference default (T 1.0
    # alone), the server default without top_p (T 0.7, repetition 1.05), that
    # with top_p 0.9, and min_p + top_p + top_k 4,096, at full vocabulary
    from lumen_amd.workloads import defaults

    _run_workload(eng, defaults())


def test_plain_temperature_rows(eng):
    # plain temperature rows (no top-k / top-p / min-p) over several batch
    # shapes and temperatures, f32 and bf16, with and without penalties
    rng = np.random.default_rng(77)
    for B, V, dt in ((4, 248_320, "f32"), (16, 151_936, "bf16"), (64, 131_072, "f32"),
                     (8, 32_768, "f32")):
        lg = (rng.normal(0, 2.0, (B, V)) + rng.gumbel(0, 1, (B, V))).astype(np.float32)
        params = [SP(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.3])),
                     repetition_penalty=(1.1 if b % 2 else None),
                     frequency_penalty=(0.4 if b % 3 == 0 else None)) for b in range(B)]
        hists = [rng.integers(0, V, int(rng.integers(0, 3000))).astype(np.uint32) for _ in range(B)]
        u = rng.random(B).astype(np.float32)
        if dt == "bf16":
            bits = (lg.view(np.uint32) >> 16).astype(np.uint16)
            lg = (bits.astype(np.uint32) << 16).view(np.float32)
            rep = parity.compare(eng, lg, params, hists, u, dtype="bf16", bf16_bits=bits)
        else:
            rep = parity.compare(eng, lg, params, hists, u, check_pen=True)
        assert_clean(rep, f"plain B={B} V={V} {dt}")


def test_config4_full(eng):
    # B=256 bf16 rows over a flat distribution with top_p 0.99: the nucleus
    # spans most of the vocabulary (the sort / prefix-sum worst case)
    from lumen_amd.workloads import config4

    _run_workload(eng, config4())


def test_config2_sequential_draws(eng):
    # B=1 latency workload: successive draws from one Xorshift64 stream, each
    # sampled token recorded into the history (Sampler::sample,
    # sampling.rs:429-433), so the penalties change from draw to draw
    from lumen_amd.sampling import Xorshift64
    from lumen_amd.workloads import config2

    w = config2()
    rng = Xorshift64(w.seeds[0])
    hist = np.asarray(w.histories[0], dtype=np.uint32)
    lg = w.logits_f32()
    for d in range(200):
        u = np.array([rng.next_f32()], np.float32)
        log(f"case config2 draw {d} history {hist.size}")
        rep = parity.compare(eng, lg, w.params, [hist], u, check_pen=d % 10 == 0)
        assert_clean(rep, f"config2 draw {d}")
        hist = np.append(hist, np.uint32(rep["gpu"][0]))


def test_device_rng_states(eng):
    # rng_states_dev: the kernel draws Xorshift64::next_f32 (sampling.rs:45-106)
    # from each row's device-resident state and stores the advanced state;
    # greedy rows (temperature 0) keep theirs. Three calls in a row must give
    # the tokens that host-side draws from the same streams give, and the
    # states must equal the host generators' afterwards.
    import torch
    from lumen_amd.sampling import Xorshift64

    B, V = 24, 5000
    rng = np.random.default_rng(11)
    lg = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    params = [SP(temperature=0.0) if b % 4 == 0 else
              SP(temperature=0.8, top_p=0.9, top_k=50 if b % 3 else None) for b in range(B)]
    seeds = [1000 + 7 * b for b in range(B)]
    host = [Xorshift64(s) for s in seeds]
    dev = torch.tensor([np.int64(np.uint64(h.state()).view(np.int64)) for h in host],
                       dtype=torch.int64, device="cuda:0")
    x = torch.from_numpy(lg).to("cuda:0")
    for call in range(3):
        log(f"case device_rng call {call} B={B} V={V}")
        want = [0] * B
        u = np.zeros(B, np.float32)
        for b in range(B):
            if params[b].temperature > 0:
                u[b] = host[b].next_f32()
        _, want = eng.sample_batch(x, params, uniforms=u)
        _, got = eng.sample_batch(x, params, rng_states_dev=dev)
        assert got == want, f"call {call}: {got} vs {want}"
        st = dev.cpu().numpy().view(np.uint64)
        assert [int(v) for v in st] == [h.state() for h in host], f"call {call} states"


def _decode_rows(B, rng):
    params = []
    for b in range(B):
        k = b % 6
        if k == 0:
            params.append(SP(temperature=0.0, repetition_penalty=1.3, repeat_last_n=4))
        elif k == 1:
            params.append(SP(temperature=0.9, top_k=40, frequency_penalty=0.7))
        elif k == 2:
            params.append(SP(temperature=0.7, top_p=0.9, presence_penalty=0.5, repeat_last_n=3))
        elif k == 3:
            params.append(SP(temperature=1.1, repetition_penalty=1.2, min_p=0.05))
        elif k == 4:
            params.append(SP(temperature=0.8, top_p=0.95))
        else:
            params.append(SP(temperature=0.0, frequency_penalty=2.0))
    return params


@pytest.mark.parametrize("V", [600, 248320])
def test_device_decode_state(eng, V):
    # A decode loop with the history ring and the RNG states in device memory
    # against the same loop driven from the host (SamplerState::history and
    # Xorshift64 on the host, Sampler::sample at sampling.rs:429-433): every
    # step's tokens must agree, and the ring must hold the tokens recorded.
    import torch
    from lumen_amd.sampling import DeviceDecodeState, Xorshift64

    B = 12 if V < 10000 else 6
    rng = np.random.default_rng(V)
    params = _decode_rows(B, rng)
    seeds = [900 + b for b in range(B)]
    prompt = [rng.integers(0, V, size=int(rng.integers(0, 5))).astype(np.uint32) for _ in range(B)]
    cap = 64
    ds = DeviceDecodeState(eng, seeds, cap=cap, histories=prompt)
    host_rng = [Xorshift64(s) for s in seeds]
    hist = [list(p) for p in prompt]
    steps = 20 if V < 10000 else 6
    for step in range(steps):
        # logits that favour recently sampled ids, so the penalties matter
        lg = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        for b in range(B):
            for tok in hist[b][-3:]:
                lg[b, tok] += 4.0
        x = torch.from_numpy(lg).to("cuda:0")
        log(f"case device_decode V={V} step {step}")
        _, want = eng.sample_batch(x, params, histories=[np.array(h, np.uint32) for h in hist],
                                   rngs=host_rng)
        _, got = ds.step(eng, x, params)
        assert got == want, f"step {step}: {got} vs {want}"
        for b in range(B):
            hist[b].append(want[b])
    lens = ds.lens.cpu().numpy()
    ring = ds.ring.cpu().numpy().view(np.uint32)
    for b in range(B):
        assert lens[b] == len(hist[b])
        for k in range(max(0, len(hist[b]) - cap), len(hist[b])):
            assert ring[b, k % cap] == hist[b][k]
    st = ds.rng.cpu().numpy().view(np.uint64)
    assert [int(v) for v in st] == [r.state() for r in host_rng]


def test_device_ring_wrap_against_oracle(eng):
    # A ring of 8 tokens over 24 decode steps, so it wraps three times:
    # windows below the ring (3), equal to it (8) and the whole history
    # (repeat_last_n 0, which grows past the ring and is carried by the
    # token-by-token count updates). Every step's tokens and the penalized
    # logits are checked against the oracle's Sampler::sample loop
    # (sampling.rs:429-433: sample_logits, then record), with the reference
    # RNG advanced only by sampled rows.
    import torch
    from lumen_amd.sampling import DeviceDecodeState
    from oracle import oracle as o

    V, cap, steps = 500, 8, 24
    params = [SP(temperature=0.8, repetition_penalty=1.3, repeat_last_n=3),
              SP(temperature=0.0, frequency_penalty=1.0, repeat_last_n=8),
              SP(temperature=0.9, top_k=40, presence_penalty=0.8, repeat_last_n=0),
              SP(temperature=1.1, repetition_penalty=1.2, min_p=0.05, repeat_last_n=5)]
    B = len(params)
    seeds = [71, 72, 73, 74]
    rng = np.random.default_rng(17)
    prompt = [rng.integers(0, V, size=3).astype(np.uint32) for _ in range(B)]
    ds = DeviceDecodeState(eng, seeds, cap=cap, histories=prompt)
    orngs = [o.Xorshift64(sd) for sd in seeds]
    hist = [list(int(x) for x in p_) for p_ in prompt]
    for step in range(steps):
        lg = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        for b in range(B):
            lg[b, hist[b][-4:]] += 3.0
        x = torch.from_numpy(lg).to("cuda:0")
        pen = torch.empty((B, V), dtype=torch.float32, device="cuda:0")
        log(f"case ring wrap step {step}")
        _, got = ds.step(eng, x, params, penalized_out=pen)
        pen_h = pen.cpu().numpy()
        for b in range(B):
            op = parity.to_oracle_params(params[b])
            want_pen = o.apply_penalties(lg[b].copy(), op, hist[b]) if (
                params[b].penalties_active() and hist[b]) else lg[b]
            assert np.array_equal(pen_h[b].view(np.uint32),
                                  np.asarray(want_pen, np.float32).view(np.uint32)), (step, b)
            want = o.sample_logits(lg[b], op, hist[b], orngs[b])
            assert got[b] == want, (step, b, got[b], want)
            hist[b].append(int(want))
    lens = ds.lens.cpu().numpy()
    ring = ds.ring.cpu().numpy().view(np.uint32)
    for b in range(B):
        assert lens[b] == len(hist[b])
        for k in range(len(hist[b]) - cap, len(hist[b])):
            assert ring[b, k % cap] == hist[b][k]


def test_device_history_rewrite(eng):
    # counts updated token by token across calls, then the ring rewritten by
    # the caller (a new prompt, a new epoch): the counts are made again, and
    # the following calls update them again
    import torch
    from lumen_amd.sampling import DeviceDecodeState, Xorshift64, next_epoch

    V, B = 3000, 4
    rng = np.random.default_rng(5)
    params = [SP(temperature=0.0, repetition_penalty=1.5, repeat_last_n=3),
              SP(temperature=0.8, frequency_penalty=1.0),
              SP(temperature=0.0, presence_penalty=2.0, repeat_last_n=1),
              SP(temperature=1.0, top_k=30, repetition_penalty=1.3, repeat_last_n=5)]
    seeds = [1, 2, 3, 4]
    ds = DeviceDecodeState(eng, seeds, cap=32, histories=[[1, 2, 3]] * B)
    hist = [[1, 2, 3] for _ in range(B)]
    host_rng = [Xorshift64(s) for s in seeds]
    for phase in range(2):
        for step in range(6):
            lg = (rng.standard_normal((B, V)) * 2).astype(np.float32)
            for b in range(B):
                lg[b, hist[b][-4:]] += 3.0
            x = torch.from_numpy(lg).to("cuda:0")
            log(f"case history rewrite phase {phase} step {step}")
            _, want = eng.sample_batch(x, params, histories=[np.array(h, np.uint32) for h in hist],
                                       rngs=host_rng)
            _, got = ds.step(eng, x, params)
            assert got == want, (phase, step, got, want)
            for b in range(B):
                hist[b].append(want[b])
        # a new prompt written by the caller
        prompt = rng.integers(0, V, size=5).astype(np.uint32)
        ring = np.zeros((B, 32), np.uint32)
        ring[:, :5] = prompt
        ds.ring.copy_(torch.from_numpy(ring.view(np.int32)))
        ds.lens.fill_(5)
        ds.epoch = next_epoch()
        hist = [list(prompt) for _ in range(B)]


def test_device_history_overflow(eng):
    # a whole-history penalty window longer than the ring cannot be counted:
    # that row reports an error (status 3) and the other rows are unaffected
    import torch
    from lumen_amd import _native
    from lumen_amd.sampling import DeviceDecodeState

    V = 300
    params = [SP(temperature=0.0, repetition_penalty=1.5),
              SP(temperature=0.0, repetition_penalty=1.5, repeat_last_n=8),
              SP(temperature=0.0)]
    hist = [list(range(20))] * 3
    ds = DeviceDecodeState(eng, [1, 2, 3], cap=16, histories=hist)
    lg = torch.from_numpy(np.random.default_rng(3).standard_normal((3, V)).astype(np.float32)).cuda()
    tr = torch.zeros((3, 16), dtype=torch.int32, device="cuda:0")
    toks, _ = ds.step(eng, lg, params, trace=tr, sync=False)
    torch.cuda.synchronize()
    t = toks.cpu().numpy().view(np.uint32)
    st = tr.cpu().numpy()[:, 0]
    assert t[0] == 0xFFFFFFFF and st[0] == 3
    assert t[1] != 0xFFFFFFFF and st[1] == 0 and t[2] != 0xFFFFFFFF
    _, want = eng.sample_batch(lg[1:], params[1:], histories=[np.array(h, np.uint32) for h in hist[1:]])
    assert list(t[1:]) == want
    lens = ds.lens.cpu().numpy()
    assert list(lens) == [20, 21, 21]
    with pytest.raises(RuntimeError):
        ds.step(eng, lg, params)


@pytest.mark.parametrize("V", [3000, 248320])
def test_anti_restate_guard(eng, V):
    # Greedy rows with anti_restate (sampling.rs:472-474): the device picks the
    # guard's candidates from the (penalized) row, the host applies the rules.
    # Tokens against the oracle's sample_logits with the same history and
    # decoder; candidates against numpy's top finite keys.
    import torch
    from lumen_amd.sampling import TokenBytes
    from oracle import oracle as o
    from tests.test_anti_restate_cpu import candidates

    rng = np.random.default_rng(V + 1)
    B = 16
    alpha = [b"ab", b"ba", b"abab", b" ab", b"b", b"cab"]
    table = [alpha[int(i)] * int(rng.integers(1, 3)) for i in rng.integers(0, len(alpha), V)]
    dec = TokenBytes(table)
    lg = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    params, hists = [], []
    for b in range(B):
        loop = rng.integers(0, V, size=int(rng.integers(1, 5))).astype(np.uint32)
        h = np.resize(loop, int(rng.integers(0, 30))).astype(np.uint32)
        # make the restating / looping tokens the leaders
        for j, tok in enumerate(np.unique(h)[:6]):
            lg[b, tok] = 9.0 - 0.25 * j
        if b % 4 == 3:
            lg[b, int(rng.integers(0, V))] = np.nan
        if b % 5 == 4:
            lg[b, rng.integers(0, V, size=3)] = np.inf
        pen = {} if b % 2 else dict(repetition_penalty=1.3, repeat_last_n=8)
        params.append(SP(temperature=0.0, anti_restate=True, **pen))
        hists.append(h)
    x = torch.from_numpy(lg).to("cuda:0")
    log(f"case anti_restate V={V} sync")
    _, got = eng.sample_batch(x, params, histories=hists, decoder=dec)
    want = []
    for b in range(B):
        op = o.Params(temperature=0.0, anti_restate=True,
                      repetition_penalty=params[b].repetition_penalty,
                      repeat_last_n=params[b].repeat_last_n)
        want.append(o.sample_logits(lg[b].copy(), op, hists[b], o.Xorshift64(1), table))
    assert got == want
    # asynchronous: raw argmax in tokens, candidates in guard_out
    log(f"case anti_restate V={V} async")
    gout = torch.full((B, 9), -7, dtype=torch.int32, device="cuda:0")
    toks, _ = eng.sample_batch(x, params, histories=hists, guard_out=gout, sync=False)
    torch.cuda.synchronize()
    g = gout.cpu().numpy().view(np.uint32)
    t = toks.cpu().numpy().view(np.uint32)
    for b in range(B):
        if params[b].repetition_penalty is None:
            assert list(g[b]) == candidates(lg[b]), b
        assert t[b] == g[b][0]
    # the sync tokens are the guard's choice over those candidates
    from lumen_amd.sampling import anti_restate_select
    assert [anti_restate_select(g[b], hists[b], dec) for b in range(B)] == want
    with pytest.raises(Exception):
        eng.sample_batch(x, params, histories=hists, sync=False)


def test_decode_step_in_a_graph(eng):
    # A decode step with every input on the device (RNG states, history ring,
    # logits) captured into a HIP graph and replayed: each replay must give
    # the tokens and state of the same step run eagerly, with eager work
    # (new logits, readbacks, synchronizations) between the replays
    import torch
    from lumen_amd.sampling import DeviceDecodeState

    B, V, steps = 4, 50_000, 8
    rng = np.random.default_rng(23)
    params = [SP(temperature=0.8, top_p=0.9, repetition_penalty=1.2, repeat_last_n=16),
              SP(temperature=0.0, frequency_penalty=0.5),
              SP(temperature=1.0, top_k=40, presence_penalty=0.4),
              SP(temperature=0.7)]
    seeds = [5, 6, 7, 8]
    prompts = [rng.integers(0, V, size=n).astype(np.uint32) for n in (3, 0, 10, 1)]
    seq = [torch.from_numpy((rng.standard_normal((B, V)) * 3).astype(np.float32)).cuda()
           for _ in range(steps)]
    x = torch.empty((B, V), dtype=torch.float32, device="cuda:0")
    # eager
    de = DeviceDecodeState(eng, seeds, cap=256, histories=prompts)
    te = torch.empty(B, dtype=torch.int32, device="cuda:0")
    want = []
    for st in range(steps):
        x.copy_(seq[st])
        de.step(eng, x, params, tokens_out=te, sync=False)
        want.append(te.cpu().tolist())
    # warm-up on a throwaway state (the context allocates its buffers here),
    # then capture one step of a fresh state
    dw = DeviceDecodeState(eng, seeds, cap=256, histories=prompts)
    dg = DeviceDecodeState(eng, seeds, cap=256, histories=prompts)
    tg = torch.empty(B, dtype=torch.int32, device="cuda:0")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dw.step(eng, x, params, tokens_out=tg, sync=False)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    log(f"case graph capture B={B} V={V}")
    with torch.cuda.graph(g):
        dg.step(eng, x, params, tokens_out=tg, sync=False)
    for st in range(steps):
        x.copy_(seq[st])
        g.replay()
        torch.cuda.synchronize()
        assert tg.cpu().tolist() == want[st], f"replay {st}"
    assert torch.equal(dg.rng, de.rng) and torch.equal(dg.ring, de.ring)
    assert torch.equal(dg.lens, de.lens)


def test_prepared_batch_matches_sample_batch(eng):
    # Engine.prepare builds the C description once; each run() must give what
    # sample_batch gives for the same draws, sync and async
    import torch
    from lumen_amd.sampling import Xorshift64

    rng = np.random.default_rng(31)
    B, V = 3, 20_000
    x = torch.from_numpy((rng.standard_normal((B, V)) * 2).astype(np.float32)).cuda()
    params = [SP(temperature=0.7, top_k=20, top_p=0.8), SP(temperature=0.0),
              SP(temperature=1.2, min_p=0.05)]
    pb = eng.prepare(x, params)
    r = Xorshift64(5)
    for call in range(6):
        u = [r.next_f32() for _ in range(B)]
        _, want = eng.sample_batch(x, params, uniforms=u)
        if call % 2:
            assert pb.run(u, sync=False) is None
            torch.cuda.synchronize()
            got = pb.tokens.cpu().tolist()
        else:
            got = pb.run(u)
        assert got == want, f"call {call}"


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_anti_restate_fuzz(eng, seed):
    # random greedy anti-restate rows (with and without penalties, windows,
    # NaN / inf / tied logits, looping histories, random byte decoders)
    # against the oracle's sample_logits, through the synchronous call
    import torch
    from lumen_amd.sampling import TokenBytes
    from oracle import oracle as o

    rng = np.random.default_rng(700 + seed)
    V = int(rng.choice([97, 5000, 151_936]))
    B = int(rng.integers(4, 24))
    alpha = [b"a", b"b", b"ab", b" ", b"ba ", b"\t", b"abab", b"c"]
    table = [b"".join(alpha[int(i)] for i in rng.integers(0, len(alpha), int(rng.integers(0, 4))))
             for _ in range(V)]
    dec = TokenBytes(table)
    lg = np.stack([random_logits(rng, V, int(rng.integers(0, 6))) for _ in range(B)])
    params, hists = [], []
    for b in range(B):
        loop = rng.integers(0, V, size=int(rng.integers(1, 6))).astype(np.uint32)
        h = np.resize(loop, int(rng.integers(0, 40))).astype(np.uint32)
        for j, tok in enumerate(np.unique(h)[:8]):
            if rng.random() < 0.7:
                lg[b, tok] = np.float32(lg[b].max() + 1.0 - 0.01 * j)
        p = SP(temperature=0.0, anti_restate=True)
        if rng.random() < 0.4:
            p.repetition_penalty = float(rng.choice([1.1, 2.0]))
            p.repeat_last_n = int(rng.choice([0, 3, 16]))
        if rng.random() < 0.2:
            p.frequency_penalty = 0.5
        params.append(p)
        hists.append(h)
    x = torch.from_numpy(lg).to("cuda:0")
    log(f"case anti_restate fuzz seed {seed} B={B} V={V}")
    _, got = eng.sample_batch(x, params, histories=hists, decoder=dec)
    want = []
    for b in range(B):
        p = params[b]
        op = o.Params(temperature=0.0, anti_restate=True, repetition_penalty=p.repetition_penalty,
                      repeat_last_n=p.repeat_last_n, frequency_penalty=p.frequency_penalty)
        want.append(o.sample_logits(lg[b].copy(), op, hists[b], o.Xorshift64(1), table))
    assert got == want

