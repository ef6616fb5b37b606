"""Parity harness: runs the gfx950 engine and the CPU oracle on the same
rows (logits, params, history, uniform) and compares token ids, penalized
logits and the intermediate sums, bit for bit.

Test infrastructure (imports the oracle).
"""
from __future__ import annotations

import math
import struct
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oracle import oracle as o

TRACE_FIELDS = ("status", "path", "topk_cutoff_key", "topk_survivors", "topp_sum", "topp_kept",
                "topp_cum", "windows", "final_max", "final_sum", "cdf_before", "cdf_at", "token",
                "passes")
FLOAT_FIELDS = {"topp_sum", "topp_cum", "final_max", "final_sum", "cdf_before", "cdf_at"}


def to_oracle_params(p) -> o.Params:
    return o.Params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                    repetition_penalty=p.repetition_penalty, presence_penalty=p.presence_penalty,
                    frequency_penalty=p.frequency_penalty, repeat_last_n=p.repeat_last_n,
                    anti_restate=p.anti_restate)


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def same_float(a, b):
    a, b = float(a), float(b)
    if math.isnan(a) or math.isnan(b):
        return math.isnan(a) and math.isnan(b)
    return fbits(a) == fbits(b)


def decode_trace(t_np):
    """[B, 16] uint32 -> list of dicts."""
    out = []
    for row in t_np:
        d = {}
        for i, name in enumerate(TRACE_FIELDS):
            v = int(row[i])
            d[name] = struct.unpack("<f", struct.pack("<I", v))[0] if name in FLOAT_FIELDS else v
        out.append(d)
    return out


def oracle_rows(logits_f32, params, histories, uniforms, workers=8):
    def one(b):
        return o.sample_logits_r(logits_f32[b], to_oracle_params(params[b]), histories[b],
                                 float(uniforms[b]))
    with ThreadPoolExecutor(workers) as ex:
        return list(ex.map(one, range(len(params))))


def gpu_rows(engine, logits_dev, params, histories, uniforms, want_pen=False):
    import torch

    B, V = logits_dev.shape
    trace = torch.zeros((B, 16), dtype=torch.int32, device=logits_dev.device)
    pen = torch.empty((B, V), dtype=torch.float32, device=logits_dev.device) if want_pen else None
    toks, host = engine.sample_batch(logits_dev, params, histories=histories, uniforms=uniforms,
                                     trace=trace, penalized_out=pen)
    torch.cuda.synchronize()
    tr = decode_trace(trace.cpu().numpy().view(np.uint32))
    return host, tr, (pen.cpu().numpy() if want_pen else None)


def compare(engine, logits_f32, params, histories, uniforms, dtype="f32", bf16_bits=None,
            check_pen=False, check_trace=True, row_stride=None):
    """Runs both sides; returns a report dict; asserts nothing."""
    import torch

    B, V = logits_f32.shape
    if dtype == "bf16":
        src = torch.from_numpy(bf16_bits.view(np.int16)).view(torch.bfloat16)
    else:
        src = torch.from_numpy(np.ascontiguousarray(logits_f32))
    if row_stride is not None and row_stride != V:
        big = torch.zeros((B, row_stride), dtype=src.dtype)
        big[:, :V] = src
        dev = big.cuda()[:, :V]
    else:
        dev = src.cuda()
    host, tr, pen = gpu_rows(engine, dev, params, histories, uniforms, want_pen=check_pen)
    ref = oracle_rows(logits_f32, params, histories, uniforms)
    rep = {"rows": B, "token_mismatch": [], "trace_mismatch": [], "pen_mismatch": [],
           "status": [t["status"] for t in tr], "gpu": host, "ref": [r[0] for r in ref],
           "traces": tr, "ref_traces": [r[1] for r in ref]}
    for b in range(B):
        rt, rtr = ref[b]
        gt, gtr = host[b], tr[b]
        if gt != rt:
            rep["token_mismatch"].append((b, gt, rt))
        if check_trace:
            diffs = []
            if rtr["greedy"] == 0:
                if rtr["topk_applied"]:
                    if gtr["topk_survivors"] != rtr["topk_survivors"]:
                        diffs.append(("topk_survivors", gtr["topk_survivors"],
                                      rtr["topk_survivors"]))
                    if gtr["topk_cutoff_key"] != rtr["topk_cutoff_key"]:
                        diffs.append(("topk_cutoff_key", gtr["topk_cutoff_key"],
                                      rtr["topk_cutoff_key"]))
                if rtr["topp_applied"]:
                    if not same_float(gtr["topp_sum"], rtr["topp_sum"]):
                        diffs.append(("topp_sum", gtr["topp_sum"], rtr["topp_sum"]))
                    if gtr["topp_kept"] != rtr["topp_kept"]:
                        diffs.append(("topp_kept", gtr["topp_kept"], rtr["topp_kept"]))
                if not same_float(gtr["final_max"], rtr["final_max"]):
                    diffs.append(("final_max", gtr["final_max"], rtr["final_max"]))
                if not rtr["final_uniform"] and not same_float(gtr["final_sum"], rtr["final_sum"]):
                    diffs.append(("final_sum", gtr["final_sum"], rtr["final_sum"]))
                if not same_float(gtr["cdf_at"], rtr["cdf_at"]):
                    diffs.append(("cdf_at", gtr["cdf_at"], rtr["cdf_at"]))
            if diffs:
                rep["trace_mismatch"].append((b, diffs))
        if check_pen:
            want = o.apply_penalties(logits_f32[b].copy(), to_oracle_params(params[b]),
                                     histories[b]) if (
                params[b].penalties_active() and len(histories[b]) > 0) else logits_f32[b]
            got = pen[b]
            if not np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32)):
                bad = np.nonzero(got.view(np.uint32) != np.asarray(want, np.float32).view(np.uint32))[0]
                rep["pen_mismatch"].append((b, bad[:5].tolist()))
    return rep


def classify_mismatch(logits_row, params, history, r, eps=1e-6):
    """For a token mismatch: is the draw within eps of a CDF boundary or the
    top-p crossing within eps of p (the tolerated class)?"""
    t, tr = o.sample_logits_r(logits_row, to_oracle_params(params), history, r)
    near_draw = abs(r - tr["cdf_before"]) < eps or abs(r - tr["cdf_at"]) < eps
    near_topp = tr["topp_applied"] and abs(tr["topp_cum_at_cross"] - params.top_p) < eps
    return bool(near_draw or near_topp)
