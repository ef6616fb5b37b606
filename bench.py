#!/usr/bin/env python3
"""Benchmark: Lumen's token sampler on one MI355X.

Metric: samples/sec @B=64 V=248,320; p50 us/sample @B=1;
% of HBM roofline.

A step is one lumen_sampler_sample_batch call over the config-3 batch
(B=64, V=248,320 fp32 logits, mixed rows: 16 greedy, 16 top_k=50, 16
top_p=0.9, 16 full stack T=0.6 top_k=100 top_p=0.95 rep=1.05 with histories
of up to 8,192 Zipf ids). Inputs are resident in HBM before timing: logits,
the per-row penalty counts (the SamplerState.freq map in device form) and the
per-row draws (Xorshift64::new(seed_b).next_f32()); per-row parameters are
staged once and then reused by the library's staging cache, so a timed step
issues exactly one kernel launch and no copies.

The JSON line also carries:
  roofline      the kernel's achieved logit bandwidth (B*V*4 bytes per
                launch / average launch time from HIP events on the launch
                stream) against MI355X's 8 TB/s
  cpu_baseline  the C restatement of the reference sampler (oracle/) timed on
                this host, single thread, over the same 64 rows
  b1_latency    config 2 (B=1, V=248,320): p50/p99 wall time per draw of
                sequential draws through a prepared batch (one C-ABI call:
                launch + kernel + 4-byte readback), and the p50 through the
                convenience API
  b1_decode_device_state  the same as a decode loop with the RNG state and
                the history on the device (no host draw, no history upload)
  b1_graph_decode  those decode steps captured 32 to a HIP graph: time per
                token without host work between steps
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "samples/sec @B=64 V=248,320; p50 µs/sample @B=1; % of HBM roofline"


def penalty_csr(w, device):
    """Per-row (distinct id, count) over each row's repeat_last_n window."""
    import torch

    offs, ids, cnts = [0], [], []
    for p, h in zip(w.params, w.histories):
        h = np.asarray(h, dtype=np.uint32)
        if p.repeat_last_n:
            h = h[-p.repeat_last_n:]
        if p.penalties_active() and h.size:
            u, c = np.unique(h, return_counts=True)
            ids.append(u.astype(np.uint32))
            cnts.append(c.astype(np.uint32))
            offs.append(offs[-1] + u.size)
        else:
            offs.append(offs[-1])
    cat = lambda xs: np.concatenate(xs) if xs else np.zeros(1, np.uint32)
    t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.uint32).view(np.int32)).to(device)
    return t(np.array(offs, dtype=np.uint32)), t(cat(ids)), t(cat(cnts))


def first_draws(w):
    from lumen_amd.sampling import Xorshift64

    return np.array([Xorshift64(s).next_f32() for s in w.seeds], dtype=np.float32)


def traffic_from_profiles(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_baseline(w, uniforms, budget_s=20.0):
    from oracle import oracle as o

    lg = w.logits_f32()
    ops = [o.Params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                    repetition_penalty=p.repetition_penalty, presence_penalty=p.presence_penalty,
                    frequency_penalty=p.frequency_penalty, repeat_last_n=p.repeat_last_n)
           for p in w.params]
    rows = 0
    t0 = time.perf_counter()
    reps = 0
    done = False
    while not done:
        for b in range(w.batch):
            o.sample_logits_r(lg[b], ops[b], w.histories[b], float(uniforms[b]))
            rows += 1
            if time.perf_counter() - t0 > budget_s:
                done = True
                break
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s / 2 or reps >= 5:
            break
    return rows / el, rows, reps, el


def cpu_baseline_threads(w, uniforms, threads, budget_s=10.0):
    """The same rows on `threads` host threads (rows statically partitioned)."""
    from oracle import oracle as o

    lg = w.logits_f32()
    ops = [o.Params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                    repetition_penalty=p.repetition_penalty, presence_penalty=p.presence_penalty,
                    frequency_penalty=p.frequency_penalty, repeat_last_n=p.repeat_last_n)
           for p in w.params]
    rows = 0
    reps = 0
    t0 = time.perf_counter()
    while True:
        o.sample_batch(lg, ops, w.histories, uniforms, threads=threads)
        rows += w.batch
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s / 2 or reps >= 5:
            break
    return rows / el, rows, reps, el


def host_cores():
    """CPU threads this process may use (the GPU box grants a share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit():
        n = min(n, int(cap))
    return max(1, n)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def b1_latency(eng, draws=10_000, api_draws=2_000):
    """Config 2, sequential draws. The batch description is prepared once
    (Engine.prepare, the decode-loop form of the C ABI), so a draw is one
    C-ABI call: staging of the draw, the launch, the kernel and the 4-byte
    readback. Also returns the p50 through the convenience API
    (Engine.sample_batch), which rebuilds the description per call."""
    import torch

    from lumen_amd.sampling import Xorshift64
    from lumen_amd.workloads import config2

    w = config2()
    dev = torch.from_numpy(w.logits).cuda()
    csr = penalty_csr(w, dev.device)
    rng = Xorshift64(w.seeds[0])
    tok = torch.empty(1, dtype=torch.int32, device=dev.device)
    pb = eng.prepare(dev, w.params, penalty_counts=csr, tokens_out=tok)
    times = []
    for i in range(draws + 50):
        u = [rng.next_f32()]
        t0 = time.perf_counter()
        pb.run(u)
        t1 = time.perf_counter()
        if i >= 50:
            times.append((t1 - t0) * 1e6)
    api = []
    for i in range(api_draws + 50):
        u = [rng.next_f32()]
        t0 = time.perf_counter()
        eng.sample_batch(dev, w.params, penalty_counts=csr, uniforms=u, tokens_out=tok, sync=True)
        t1 = time.perf_counter()
        if i >= 50:
            api.append((t1 - t0) * 1e6)
    times = np.array(times)
    return (float(np.percentile(times, 50)), float(np.percentile(times, 99)), len(times),
            float(np.percentile(np.array(api), 50)))


def b1_decode_device_state(eng, draws=10_000):
    """Config 2 as its configuration states it: `draws` sequential draws from
    the fixed seed with the history growing by each drawn token
    (Sampler::sample, sampling.rs:429-433: draw, then record). The history
    ring (whole-history penalty window, its counts updated on the device each
    draw) and the Xorshift64 state live in HBM; per draw one call (the
    window-count kernel and the sampler) and a 4-byte readback. Returns the
    latencies and the drawn tokens."""
    import torch

    from lumen_amd.sampling import DeviceDecodeState
    from lumen_amd.workloads import config2

    w = config2()
    dev = torch.from_numpy(w.logits).cuda()
    ds = DeviceDecodeState(eng, w.seeds, cap=8192, histories=w.histories)
    tok = torch.empty(1, dtype=torch.int32, device=dev.device)
    times, drawn = [], []
    for i in range(draws):
        t0 = time.perf_counter()
        _, host = ds.step(eng, dev, w.params, tokens_out=tok, sync=True)
        t1 = time.perf_counter()
        drawn.append(int(host[0]))
        if i >= 50:
            times.append((t1 - t0) * 1e6)
    times = np.array(times)
    return float(np.percentile(times, 50)), float(np.percentile(times, 99)), len(times), drawn


def b1_decode_parity(drawn, threads):
    """The oracle's Sampler::sample loop beside the device decode loop (outside
    any timed region): step i is the oracle's sample_logits on the history
    prompt + drawn[:i] with the i-th draw of Xorshift64(seed). While the two
    loops agree, that is exactly the oracle's own loop, so the steps are
    checked in parallel; the first mismatch is reported with the count."""
    from concurrent.futures import ThreadPoolExecutor

    from lumen_amd.workloads import config2
    from oracle import oracle as o

    w = config2()
    op = oracle_params(w)[0]
    rng = o.Xorshift64(w.seeds[0])
    rs = [rng.next_f32() for _ in drawn]
    hist = np.concatenate([np.asarray(w.histories[0], np.uint32),
                           np.asarray(drawn, np.uint32)])
    h0 = len(w.histories[0])
    row = w.logits[0]

    def one(i):
        return o.sample_logits_r(row, op, hist[:h0 + i], rs[i])[0]

    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        want = list(ex.map(one, range(len(drawn))))
    bad = [i for i, (g, r) in enumerate(zip(drawn, want)) if g != r]
    return {"steps": len(drawn), "match": len(drawn) - len(bad), "mismatch": len(bad),
            "first_mismatch_step": bad[0] if bad else None,
            "distinct_tokens": len(set(drawn)), "history_at_end": h0 + len(drawn),
            "oracle_threads": threads, "oracle_s": round(time.perf_counter() - t0, 1)}


def b1_graph_decode(eng, per_graph=32, replays=20):
    """Config 2 decode steps with the state on the device, captured in one
    HIP graph of `per_graph` consecutive steps: GPU time per token with no
    host work between steps."""
    import torch

    from lumen_amd.sampling import DeviceDecodeState
    from lumen_amd.workloads import config2

    w = config2()
    dev = torch.from_numpy(w.logits).cuda()
    tok = torch.empty(1, dtype=torch.int32, device=dev.device)
    warm = DeviceDecodeState(eng, w.seeds, cap=8192, histories=w.histories)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm.step(eng, dev, w.params, tokens_out=tok, sync=False)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ds = DeviceDecodeState(eng, w.seeds, cap=8192, histories=w.histories)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            ds.step(eng, dev, w.params, tokens_out=tok, sync=False)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return dt / (replays * per_graph) * 1e6, replays * per_graph


def oracle_params(w):
    from oracle import oracle as o

    return [o.Params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                     repetition_penalty=p.repetition_penalty, presence_penalty=p.presence_penalty,
                     frequency_penalty=p.frequency_penalty, repeat_last_n=p.repeat_last_n)
            for p in w.params]


def row_kind(p):
    if p.temperature <= 0:
        return "greedy"
    return "+".join(k for k, on in (("top_k", p.top_k), ("top_p", p.top_p), ("min_p", p.min_p),
                                      ("penalties", p.penalties_active())) if on) or "plain"


def logit_variants(name, w, total_bytes):
    """The workload's logits plus further draws of the same generator (other
    seeds), enough buffers that cycling through them exceeds `total_bytes`
    (the MI355X's 256 MB Infinity Cache), so every launch reads HBM."""
    from lumen_amd import workloads

    per = w.logits.nbytes
    k = max(1, min(8, -(-total_bytes // per)))
    gen = workloads.CONFIGS[name]
    out = [w.logits]
    for j in range(1, k):
        out.append(gen(seed=1000 + 17 * j).logits)
    return out


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def logit_buffers_note(lgs):
    """What the rotated buffers mean for where a launch reads its logits."""
    total = int(sum(lg.nbytes for lg in lgs))
    if total > MALL_BYTES:
        why = ("cycled so that every launch reads its logits from HBM, not from the "
               "256 MB Infinity Cache")
    else:
        why = (f"{len(lgs)} buffers of {lgs[0].nbytes / 1e6:.2f} MB fit the 256 MB Infinity "
               "Cache: this figure is for cache-resident logits")
    return {"count": len(lgs), "bytes": total, "cache_resident": total <= MALL_BYTES, "why": why}


def to_device(w, lg):
    import torch

    if w.dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(lg).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(lg)).cuda()


def parity_check(w, lgs, toks, traces, u_host, threads):
    """Tokens of the timed buffers against the oracle (outside the timed
    region). A mismatch counts as inside the 1e-6 zone when the draw lies
    within 1e-6 of the CDF value at or before the token (GPU trace)."""
    from oracle import oracle as o

    ops = oracle_params(w)
    out = {"rows": 0, "match": 0, "mismatch_in_1e-6": 0, "mismatch_outside": 0,
           "greedy_rows": 0, "greedy_exact": 0, "topk_rows": 0, "topk_set_exact": 0}
    for lg, tk, tr in zip(lgs, toks, traces):
        lf = lg if w.dtype == "f32" else (lg.astype(np.uint32) << 16).view(np.float32)
        ref = o.sample_batch(lf, ops, w.histories, u_host, threads=threads)
        for b in range(w.batch):
            out["rows"] += 1
            ok = int(ref[b]) == int(tk[b])
            if w.params[b].temperature <= 0:
                out["greedy_rows"] += 1
                out["greedy_exact"] += int(ok)
            if ok:
                out["match"] += 1
                continue
            cb, ca = tr[b, 10].view(np.float32), tr[b, 11].view(np.float32)
            near = min(abs(float(u_host[b]) - float(ca)), abs(float(u_host[b]) - float(cb))) <= 1e-6
            out["mismatch_in_1e-6" if near else "mismatch_outside"] += 1
    # top-k candidate sets (cutoff key and survivor count) on the first buffer
    lf = lgs[0] if w.dtype == "f32" else (lgs[0].astype(np.uint32) << 16).view(np.float32)
    for b, p in enumerate(w.params):
        if p.temperature > 0 and p.top_k and p.top_k < w.vocab:
            _, rt = o.sample_logits_r(lf[b], ops[b], w.histories[b], float(u_host[b]))
            out["topk_rows"] += 1
            tr = traces[0][b]
            out["topk_set_exact"] += int(rt["topk_survivors"] == int(tr[3]) and
                                         rt["topk_cutoff_key"] == int(tr[2]))
    return out


def measure(eng, name, steps, warmup, graph, rotate_bytes, cpu=True, cpu_budget=12.0):
    """One workload: `steps` timed launches (HIP graph replays of `graph`
    launches, cycling through the rotated logits buffers), kernel time from
    HIP events on the launch stream, parity of the timed tokens, and the CPU
    oracle on the same rows."""
    import torch

    from lumen_amd import workloads

    w = workloads.CONFIGS[name]()
    B, V = w.logits.shape
    lgs = logit_variants(name, w, rotate_bytes)
    devs = [to_device(w, lg) for lg in lgs]
    nbuf = len(devs)
    csr = penalty_csr(w, devs[0].device)
    u_host = first_draws(w)
    u_dev = torch.from_numpy(u_host).cuda()
    toks = [torch.empty(B, dtype=torch.int32, device="cuda") for _ in range(nbuf)]
    pbs = [eng.prepare(d, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=t)
           for d, t in zip(devs, toks)]
    for i in range(warmup):
        pbs[i % nbuf].run(sync=False)
    torch.cuda.synchronize()
    # stream launches, one HIP-event pair per step
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        pbs[i % nbuf].run(sync=False)
        ends[i].record()
    torch.cuda.synchronize()
    el_stream = time.perf_counter() - t0
    kern_stream = float(np.mean([a.elapsed_time(b) for a, b in zip(starts, ends)]))
    el, kern_ms, mode = el_stream, kern_stream, "stream launches"
    if graph > 1 and steps >= graph:
        # the launch-bound loop captured, as a serving loop captures its
        # sampler: each launch is one kernel node (parameters and draws are
        # resident), every replay runs the full kernel over its buffer
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            gpbs = [eng.prepare(d, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=t)
                    for d, t in zip(devs, toks)]
            for i in range(graph):
                gpbs[i % nbuf].run(sync=False)
        g.replay()
        torch.cuda.synchronize()
        reps, rem = divmod(steps, graph)
        gs = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        ge = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(reps):
            gs[i].record()
            g.replay()
            ge[i].record()
        for i in range(rem):
            pbs[i % nbuf].run(sync=False)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        kern_ms = float(np.mean([a.elapsed_time(b) for a, b in zip(gs, ge)])) / graph
        mode = f"HIP graph replays of {graph} launches"
    logit_bytes = B * V * (2 if w.dtype == "bf16" else 4)
    # one workgroup per row (lumen_sample_rows_single) once the rows fill the CUs
    kernel = "lumen_sample_rows_single" if B >= 256 else "lumen_sample_rows"
    achieved = logit_bytes / (kern_ms * 1e-3) / 1e9
    # the tokens the timed launches wrote (each buffer's last timed launch),
    # copied before anything else runs
    tok_host = [t.cpu().numpy().view(np.uint32).copy() for t in toks]
    # traces of one more call per buffer, into token buffers of their own:
    # passes and CDF values for the parity report
    traces, trace_toks = [], []
    for d in devs:
        tr = torch.zeros((B, 16), dtype=torch.int32, device="cuda")
        tt = torch.empty(B, dtype=torch.int32, device="cuda")
        eng.sample_batch(d, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=tt,
                         trace=tr, sync=False)
        traces.append(tr)
        trace_toks.append(tt)
    torch.cuda.synchronize()
    traces = [tr.cpu().numpy().view(np.uint32) for tr in traces]
    traced_same = all(np.array_equal(a, t.cpu().numpy().view(np.uint32))
                      for a, t in zip(tok_host, trace_toks))
    kinds = {}
    for b, p in enumerate(w.params):
        kinds.setdefault(row_kind(p), []).append(int(traces[0][b, 13]))
    res = {
        "workload": workload_desc(w),
        "batch": B, "vocab": V, "dtype": "f32" if w.dtype == "f32" else "bf16",
        "samples_per_s": round(B * steps / el, 1),
        "us_per_sample": round(el / steps / B * 1e6, 4),
        "ms_per_step": round(el / steps * 1e3, 4),
        "launch": mode,
        "stream_launches": {"samples_per_s": round(B * steps / el_stream, 1),
                            "kernel_ms": round(kern_stream, 5)},
        "logit_buffers": logit_buffers_note(lgs),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(f"{kernel}_{name}_pmc.txt"),
                     "kernel": kernel, "kernel_ms": round(kern_ms, 5),
                     "bytes_per_launch": logit_bytes},
        "logit_passes_per_row": {k: round(float(np.mean(v)), 2) for k, v in kinds.items()},
    }
    nt = host_cores()
    res["parity"] = parity_check(w, lgs, tok_host, traces, u_host, nt)
    res["parity"]["tokens_checked"] = "the timed launches' own tokens"
    res["parity"]["traced_call_same_tokens"] = bool(traced_same)
    if cpu:
        rate, rows, reps, cel = cpu_baseline(w, u_host, budget_s=cpu_budget)
        res["cpu_baseline"] = {"value": round(rate, 2), "unit": "samples/s", "cores": 1,
                               "kind": "port",
                               "sample": f"{w.name}: {rows} rows ({reps} passes over the first "
                                         f"buffer, {cel:.1f} s), same inputs, single thread, "
                                         "oracle/sampling_ref.c -O2",
                               "cpu": cpu_model()}
        if nt > 1:
            rate_mt, rows_mt, reps_mt, cel_mt = cpu_baseline_threads(w, u_host, nt,
                                                                     budget_s=cpu_budget / 2)
            res["cpu_baseline_all_cores"] = {
                "value": round(rate_mt, 2), "unit": "samples/s", "cores": nt, "kind": "port",
                "sample": f"{w.name}: {rows_mt} rows ({reps_mt} passes, {cel_mt:.1f} s), rows "
                          f"split over {nt} threads"}
    return res


def workload_desc(w):
    kinds = {}
    for p in w.params:
        kinds[row_kind(p)] = kinds.get(row_kind(p), 0) + 1
    mix = ", ".join(f"{n} {k}" for k, n in kinds.items())
    return f"{w.name}: B={w.batch} V={w.vocab} {w.dtype} logits; rows: {mix}"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="config3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-b1", action="store_true", help="skip the B=1 latency legs")
    ap.add_argument("--no-configs", action="store_true",
                    help="measure only the headline workload (no per-config entries)")
    ap.add_argument("--b1-draws", type=int, default=10_000)
    ap.add_argument("--graph", type=int, default=10,
                    help="time the steps as replays of a HIP graph of this many launches")
    ap.add_argument("--rotate-mb", type=int, default=300,
                    help="cycle through logits buffers totalling at least this many MB")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (PMC calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent: N GPUs would each take B/N of the rows)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        a = torch.empty(64 * 2**20, dtype=torch.float32, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(10):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": a.numel() * 4, "copy_bytes_written": b.numel() * 4}))
        return

    from lumen_amd.sampling import Engine

    eng = Engine(0)
    rot = args.rotate_mb * 2**20
    head = measure(eng, args.workload, args.steps, args.warmup, args.graph, rot,
                   cpu=not args.no_cpu, cpu_budget=20.0)
    line = {
        "metric": METRIC,
        "value": head["samples_per_s"],
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded generators in lumen_amd/workloads.py)",
        "config": {"workload": head["workload"], "batch": head["batch"], "vocab": head["vocab"]},
        "us_per_sample": head["us_per_sample"],
        "launch": head["launch"],
        "stream_launches": head["stream_launches"],
        "logit_buffers": head["logit_buffers"],
        "roofline": head["roofline"],
        "logit_passes_per_row": head["logit_passes_per_row"],
        "parity": head["parity"],
    }
    for k in ("cpu_baseline", "cpu_baseline_all_cores"):
        if k in head:
            line[k] = head[k]
    if not args.no_b1:
        p50, p99, n, api50 = b1_latency(eng, args.b1_draws)
        line["b1_latency"] = {"p50_us": round(p50, 2), "p99_us": round(p99, 2), "draws": n,
                              "workload": "config2: B=1 V=248320 f32, top_k 20 top_p 0.8 "
                                          "presence 1.5 frequency 0.5",
                              "call": "prepared batch (Engine.prepare(...).run): one C-ABI "
                                      "sync call per draw",
                              "p50_us_sample_batch_api": round(api50, 2)}
        us, n = b1_graph_decode(eng)
        line["b1_graph_decode"] = {
            "us_per_token": round(us, 2), "tokens": n,
            "workload": "config2 decode steps (device RNG and history ring) captured 32 to a "
                        "HIP graph; wall time per token over graph replays"}
        p50, p99, n, drawn = b1_decode_device_state(eng, args.b1_draws)
        line["b1_decode_device_state"] = {
            "p50_us": round(p50, 2), "p99_us": round(p99, 2), "draws": len(drawn),
            "timed_draws": n,
            "workload": "config2 as configured: sequential draws from the fixed seed, the "
                        "history (4,096 prompt ids) growing by each drawn token; RNG state "
                        "and the history ring on the device, whole-history penalty window",
            "parity": b1_decode_parity(drawn, host_cores())}
    if not args.no_configs:
        line["configs"] = {}
        for name, steps in (("config1", 200), ("config4", 40), ("config5", 100),
                            ("defaults", 40)):
            if name == args.workload:
                continue
            print(f"bench: measuring {name}", file=sys.stderr, flush=True)
            line["configs"][name] = measure(eng, name, steps, 5, 10, rot, cpu=not args.no_cpu,
                                            cpu_budget=8.0)
    eng.close()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
