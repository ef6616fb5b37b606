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
    while True:
        for b in range(w.batch):
            o.sample_logits_r(lg[b], ops[b], w.histories[b], float(uniforms[b]))
            rows += 1
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


def b1_decode_device_state(eng, draws=2_000):
    """Config 2 as a decode loop with the state on the device: the history
    ring (whole-history penalty window, counted on the device each draw) and
    the Xorshift64 state live in HBM; per draw one call (the window-count
    kernel and the sampler) and a 4-byte readback."""
    import torch

    from lumen_amd.sampling import DeviceDecodeState
    from lumen_amd.workloads import config2

    w = config2()
    dev = torch.from_numpy(w.logits).cuda()
    ds = DeviceDecodeState(eng, w.seeds, cap=8192, histories=w.histories)
    tok = torch.empty(1, dtype=torch.int32, device=dev.device)
    times = []
    for i in range(draws + 50):
        t0 = time.perf_counter()
        ds.step(eng, dev, w.params, tokens_out=tok, sync=True)
        t1 = time.perf_counter()
        if i >= 50:
            times.append((t1 - t0) * 1e6)
    times = np.array(times)
    return float(np.percentile(times, 50)), float(np.percentile(times, 99)), len(times)


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="config3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-b1", action="store_true", help="skip the B=1 latency leg")
    ap.add_argument("--b1-draws", type=int, default=10_000)
    ap.add_argument("--graph", type=int, default=10,
                    help="also time the steps as replays of a HIP graph of this many launches")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (PMC calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent; see DESIGN.md for how the path would shard)",
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

    from lumen_amd import workloads
    from lumen_amd.sampling import Engine

    w = workloads.CONFIGS[args.workload]()
    B, V = w.logits.shape
    eng = Engine(0)
    if w.dtype == "bf16":
        dev = torch.from_numpy(w.logits.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        dev = torch.from_numpy(w.logits).cuda()
    csr = penalty_csr(w, dev.device)
    u_host = first_draws(w)
    u_dev = torch.from_numpy(u_host).cuda()
    tok = torch.empty(B, dtype=torch.int32, device=dev.device)

    def step():
        eng.sample_batch(dev, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=tok,
                         sync=False)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # stream launches, one HIP-event pair per step
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record()
        step()
        ends[i].record()
    torch.cuda.synchronize()
    el_stream = time.perf_counter() - t0
    kern_ms_stream = float(np.mean([s.elapsed_time(e) for s, e in zip(starts, ends)]))
    el, kern_ms, mode = el_stream, kern_ms_stream, "stream launches"
    if args.graph > 1:
        # The same K steps as replays of a HIP graph of `graph` sampler
        # launches (parameters and draws are resident, so each launch records
        # one kernel node and nothing else): the launch-bound loop captured,
        # as a serving loop that captures its sampler runs it. Any remainder
        # of K runs as stream launches inside the timed region.
        pb = eng.prepare(dev, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=tok)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            gpb = eng.prepare(dev, w.params, penalty_counts=csr, uniforms_dev=u_dev,
                              tokens_out=tok)
            for _ in range(args.graph):
                gpb.run(sync=False)
        g.replay()
        torch.cuda.synchronize()
        reps, rem = divmod(args.steps, args.graph)
        gs = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        ge = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(reps):
            gs[i].record()
            g.replay()
            ge[i].record()
        for _ in range(rem):
            pb.run(sync=False)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        if reps:
            kern_ms = float(np.mean([a.elapsed_time(b) for a, b in zip(gs, ge)])) / args.graph
        mode = f"HIP graph replays of {args.graph} launches"

    logit_bytes = B * V * (2 if w.dtype == "bf16" else 4)
    achieved = logit_bytes / (kern_ms * 1e-3) / 1e9
    value = B * args.steps / el
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(el / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "bf16",
        "data": "synthetic (seeded generators in lumen_amd/workloads.py)",
        "config": {"workload": f"{w.name}: B={B} V={V} {w.dtype} logits, mixed sampling rows",
                   "batch": B, "vocab": V},
        "us_per_sample": round(el / args.steps / B * 1e6, 4),
        "launch": mode,
        "stream_launches": {"value": round(B * args.steps / el_stream, 1),
                            "ms_per_step": round(el_stream / args.steps * 1e3, 4),
                            "kernel_ms": round(kern_ms_stream, 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(f"lumen_sample_rows_{w.name}_pmc.txt"),
                     "kernel": "lumen_sample_rows", "kernel_ms": round(kern_ms, 5),
                     "bytes_per_launch": logit_bytes},
    }
    # logit passes per row, from the row traces of one more call
    trace = torch.zeros((B, 16), dtype=torch.int32, device=dev.device)
    eng.sample_batch(dev, w.params, penalty_counts=csr, uniforms_dev=u_dev, tokens_out=tok,
                     trace=trace, sync=False)
    torch.cuda.synchronize()
    passes = trace.cpu().numpy().view(np.uint32)[:, 13]
    kinds = {}
    for b, p in enumerate(w.params):
        kind = ("greedy" if p.temperature <= 0 else
                "+".join(k for k, on in (("top_k", p.top_k), ("top_p", p.top_p),
                                          ("penalties", p.penalties_active())) if on) or "plain")
        kinds.setdefault(kind, []).append(int(passes[b]))
    line["logit_passes_per_row"] = {k: round(float(np.mean(v)), 2) for k, v in kinds.items()}
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
        p50, p99, n = b1_decode_device_state(eng)
        line["b1_decode_device_state"] = {
            "p50_us": round(p50, 2), "p99_us": round(p99, 2), "draws": n,
            "workload": "config2 decode loop: RNG state and a 8192-token history ring on "
                        "the device, whole-history penalty window counted per draw"}
    if not args.no_cpu:
        rate, rows, reps, cel = cpu_baseline(w, u_host)
        line["cpu_baseline"] = {"value": round(rate, 2), "unit": "samples/s", "cores": 1,
                                "kind": "port",
                                "sample": f"{w.name}: all {B} rows x {reps} passes "
                                          f"({rows} samples, {cel:.1f} s), same inputs, "
                                          "single thread, oracle/sampling_ref.c -O2",
                                "cpu": cpu_model()}
        nt = host_cores()
        if nt > 1:
            rate_mt, rows_mt, reps_mt, cel_mt = cpu_baseline_threads(w, u_host, nt)
            line["cpu_baseline_all_cores"] = {
                "value": round(rate_mt, 2), "unit": "samples/s", "cores": nt, "kind": "port",
                "sample": f"{w.name}: all {B} rows x {reps_mt} passes ({rows_mt} samples, "
                          f"{cel_mt:.1f} s), rows split over {nt} threads"}
    eng.close()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
