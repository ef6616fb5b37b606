"""Seeded synthetic inputs for the benchmark configurations.

Each generator returns host (numpy) data; nothing here touches the GPU:
    logits     [B, V] float32 (or bfloat16 bit patterns as uint16 for bf16)
    params     list of SamplingParams, one per row
    histories  list of SamplerState.history (token id lists)
    seeds      per-row Xorshift64 seeds (row b draws from new(seed_b))

Configurations (the workload the metric is quoted on is `config3`):
  1  B=1,   V=151,936 f32 N(0, 2.5^2), 20 ids boosted by +10, history 512
     ids ~ U[0, V); rep 1.1, T 0.8, top_k 40, top_p 0.95 (and a greedy pass)
  2  B=1,   V=248,320 f32 3*t(nu=3), history 4,096 ids ~ Zipf(1.1);
     T 0.7, top_k 20, top_p 0.8, presence 1.5, frequency 0.5; sequential draws
  3  B=64,  V=248,320 f32 N(0, 3^2) + Gumbel(0, 1); rows 0-15 greedy,
     16-31 top_k 50, 32-47 top_p 0.9, 48-63 T 0.6 top_k 100 top_p 0.95
     rep 1.05; history lengths ~ U[0, 8192], ids ~ Zipf(1.1)
  4  B=256, V=151,936 bf16 N(0, 1); T 1.0, top_p 0.99; no history
  5  B=128, V=248,320 f32 in {j/16}, clamp [-8, 8]; history 2,048 ids
     ~ Zipf(1.3); T 0.9, top_k 1,024, top_p 0.98, frequency 0.8
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import numpy as np

from .sampling import SamplingParams


@dataclass
class Workload:
    name: str
    logits: np.ndarray          # float32 [B, V] or uint16 bf16 bits [B, V]
    dtype: str                  # "f32" | "bf16"
    params: List[SamplingParams]
    histories: List[np.ndarray]
    seeds: List[int]

    @property
    def batch(self):
        return self.logits.shape[0]

    @property
    def vocab(self):
        return self.logits.shape[1]

    def logits_f32(self) -> np.ndarray:
        if self.dtype == "f32":
            return self.logits
        return (self.logits.astype(np.uint32) << 16).view(np.float32)


def zipf_ids(rng, n, V, s, perm):
    ranks = np.arange(1, V + 1, dtype=np.float64)
    w = ranks ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    r = np.minimum(r, V - 1)
    return perm[r].astype(np.uint32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def config1(seed=1, V=151_936) -> Workload:
    rng = np.random.default_rng(seed)
    lg = rng.normal(0.0, 2.5, size=(1, V)).astype(np.float32)
    boost = rng.choice(V, 20, replace=False)
    lg[0, boost] += np.float32(10.0)
    hist = rng.integers(0, V, 512).astype(np.uint32)
    p = SamplingParams(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1, seed=seed)
    return Workload("config1", lg, "f32", [p], [hist], [seed])


def config1_greedy(seed=1, V=151_936) -> Workload:
    w = config1(seed, V)
    w.params = [SamplingParams(temperature=0.0, repetition_penalty=1.1)]
    w.name = "config1_greedy"
    return w


def config2(seed=2, V=248_320) -> Workload:
    rng = np.random.default_rng(seed)
    lg = (3.0 * rng.standard_t(3, size=(1, V))).astype(np.float32)
    perm = rng.permutation(V)
    hist = zipf_ids(rng, 4096, V, 1.1, perm)
    p = SamplingParams(temperature=0.7, top_k=20, top_p=0.8, presence_penalty=1.5,
                       frequency_penalty=0.5, seed=seed)
    return Workload("config2", lg, "f32", [p], [hist], [seed])


def config3(seed=3, V=248_320, B=64) -> Workload:
    rng = np.random.default_rng(seed)
    lg = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
    lg += rng.gumbel(0.0, 1.0, size=(B, V)).astype(np.float32)
    perm = rng.permutation(V)
    params, hists = [], []
    q = max(B // 4, 1)
    for b in range(B):
        kind = min(b // q, 3)
        if kind == 0:
            p = SamplingParams(temperature=0.0)
        elif kind == 1:
            p = SamplingParams(temperature=1.0, top_k=50)
        elif kind == 2:
            p = SamplingParams(temperature=1.0, top_p=0.9)
        else:
            p = SamplingParams(temperature=0.6, top_k=100, top_p=0.95, repetition_penalty=1.05)
        params.append(p)
        hists.append(zipf_ids(rng, int(rng.integers(0, 8193)), V, 1.1, perm))
    return Workload("config3", lg, "f32", params, hists, [seed * 1000 + b for b in range(B)])


def config4(seed=4, V=151_936, B=256) -> Workload:
    rng = np.random.default_rng(seed)
    lg = to_bf16_bits(rng.normal(0.0, 1.0, size=(B, V)).astype(np.float32))
    params = [SamplingParams(temperature=1.0, top_p=0.99) for _ in range(B)]
    return Workload("config4", lg, "bf16", params, [np.zeros(0, np.uint32)] * B,
                    [seed * 1000 + b for b in range(B)])


def config5(seed=5, V=248_320, B=128) -> Workload:
    rng = np.random.default_rng(seed)
    lg = np.clip(np.round(rng.normal(0.0, 3.0, size=(B, V)) * 16.0) / 16.0, -8.0, 8.0)
    lg = lg.astype(np.float32)
    perm = rng.permutation(V)
    hists = [zipf_ids(rng, 2048, V, 1.3, perm) for _ in range(B)]
    params = [SamplingParams(temperature=0.9, top_k=1024, top_p=0.98, frequency_penalty=0.8)
              for _ in range(B)]
    return Workload("config5", lg, "f32", params, hists, [seed * 1000 + b for b in range(B)])


def defaults(seed=6, V=248_320, B=64) -> Workload:
    """The parameter sets real callers send most, on config 3's logits
    distribution: 16 rows of the reference default SamplingParams (T 1.0,
    nothing else; sampling.rs:313-325), 16 of the server default for a
    request without top_p (T 0.7, repetition penalty 1.05;
    runtime_defaults.rs:431, :486), 16 of that with top_p 0.9, and 16 with
    min_p 0.05 + top_p 0.95 + top_k 4,096 (T 0.8)."""
    rng = np.random.default_rng(seed)
    lg = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
    lg += rng.gumbel(0.0, 1.0, size=(B, V)).astype(np.float32)
    perm = rng.permutation(V)
    params, hists = [], []
    q = max(B // 4, 1)
    for b in range(B):
        kind = min(b // q, 3)
        if kind == 0:
            p = SamplingParams(temperature=1.0)
        elif kind == 1:
            p = SamplingParams(temperature=0.7, repetition_penalty=1.05)
        elif kind == 2:
            p = SamplingParams(temperature=0.7, repetition_penalty=1.05, top_p=0.9)
        else:
            p = SamplingParams(temperature=0.8, top_k=4096, top_p=0.95, min_p=0.05)
        params.append(p)
        hists.append(zipf_ids(rng, int(rng.integers(0, 4097)), V, 1.1, perm))
    return Workload("defaults", lg, "f32", params, hists, [seed * 1000 + b for b in range(B)])


CONFIGS = {"config1": config1, "config1_greedy": config1_greedy, "config2": config2,
           "config3": config3, "config4": config4, "config5": config5,
           "defaults": defaults}
