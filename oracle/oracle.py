"""ctypes binding of the CPU oracle (oracle/sampling_ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg. The product package
(lumen_amd) never imports this module.

The oracle restates Lumen's CPU sampler (crates/lumen-runtime/src/sampling.rs)
and is the definition of "correct" for the GPU engine.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liblumen_oracle.so")


def build() -> str:
    """Compile the oracle with its Makefile (gcc -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class RefParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint64),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("repeat_last_n", ctypes.c_uint64),
        ("anti_restate", ctypes.c_int32),
    ]


class RefTrace(ctypes.Structure):
    _fields_ = [
        ("greedy", ctypes.c_int32),
        ("topk_applied", ctypes.c_int32),
        ("topk_survivors", ctypes.c_uint32),
        ("topk_cutoff_key", ctypes.c_uint32),
        ("topp_applied", ctypes.c_int32),
        ("topp_sum", ctypes.c_float),
        ("topp_kept", ctypes.c_uint32),
        ("topp_cum_at_cross", ctypes.c_float),
        ("topp_cum_before", ctypes.c_float),
        ("minp_applied", ctypes.c_int32),
        ("final_max", ctypes.c_float),
        ("final_sum", ctypes.c_float),
        ("final_uniform", ctypes.c_int32),
        ("draw_r", ctypes.c_float),
        ("cdf_before", ctypes.c_float),
        ("cdf_at", ctypes.c_float),
        ("token", ctypes.c_uint32),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class RefDecoder(ctypes.Structure):
    _fields_ = [
        ("bytes", ctypes.POINTER(ctypes.c_uint8)),
        ("offsets", ctypes.POINTER(ctypes.c_uint64)),
        ("vocab", ctypes.c_size_t),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        u64p = ctypes.POINTER(ctypes.c_uint64)
        sz = ctypes.c_size_t
        L.ref_xorshift64_new.restype = ctypes.c_uint64
        L.ref_xorshift64_new.argtypes = [ctypes.c_uint64]
        L.ref_xorshift64_next_u64.restype = ctypes.c_uint64
        L.ref_xorshift64_next_u64.argtypes = [u64p]
        L.ref_xorshift64_next_f32.restype = ctypes.c_float
        L.ref_xorshift64_next_f32.argtypes = [u64p]
        L.ref_softmax_inplace.argtypes = [f32p, sz]
        L.ref_argmax.restype = sz
        L.ref_argmax.argtypes = [f32p, sz]
        L.ref_penalties_active.restype = ctypes.c_int
        L.ref_penalties_active.argtypes = [ctypes.POINTER(RefParams)]
        L.ref_apply_penalties.argtypes = [f32p, sz, ctypes.POINTER(RefParams), u32p, sz]
        L.ref_apply_top_k.argtypes = [f32p, sz, sz]
        L.ref_apply_top_p_on_logits.argtypes = [f32p, sz, ctypes.c_float]
        L.ref_apply_min_p_on_logits.argtypes = [f32p, sz, ctypes.c_float]
        L.ref_sample_categorical.restype = ctypes.c_uint32
        L.ref_sample_categorical.argtypes = [f32p, sz, ctypes.c_float]
        L.ref_sample_logits.restype = ctypes.c_uint32
        L.ref_sample_logits.argtypes = [f32p, sz, ctypes.POINTER(RefParams), u32p, sz,
                                        ctypes.POINTER(RefDecoder), u64p]
        L.ref_sample_logits_r.restype = ctypes.c_uint32
        L.ref_sample_logits_r.argtypes = [f32p, sz, ctypes.POINTER(RefParams), u32p, sz,
                                          ctypes.c_float, ctypes.POINTER(RefTrace)]
        L.ref_guarded_argmax.restype = ctypes.c_uint32
        L.ref_guarded_argmax.argtypes = [f32p, sz, u32p, sz, ctypes.POINTER(RefDecoder)]
        L.ref_sample_batch.argtypes = [f32p, sz, sz, ctypes.POINTER(RefParams), u64p, u32p,
                                       f32p, u32p, ctypes.c_int]
        L.ref_glibc_expf.restype = ctypes.c_float
        L.ref_glibc_expf.argtypes = [ctypes.c_float]
        L.ref_expf_check_range.restype = ctypes.c_uint64
        L.ref_expf_check_range.argtypes = [ctypes.c_uint32, ctypes.c_uint64, u32p]
        L.ref_expf_table.argtypes = [u64p]
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


@dataclass
class Params:
    """Python view of SamplingParams (sampling.rs:239-325); None == neutral."""

    temperature: float = 1.0
    top_k: Optional[int] = None
    top_p: Optional[float] = None
    min_p: Optional[float] = None
    repetition_penalty: Optional[float] = None
    presence_penalty: Optional[float] = None
    frequency_penalty: Optional[float] = None
    repeat_last_n: Optional[int] = None
    anti_restate: bool = False
    seed: Optional[int] = None

    def to_c(self) -> RefParams:
        return RefParams(
            float(self.temperature),
            int(self.top_k or 0),
            float(1.0 if self.top_p is None else self.top_p),
            float(0.0 if self.min_p is None else self.min_p),
            float(1.0 if self.repetition_penalty is None else self.repetition_penalty),
            float(0.0 if self.presence_penalty is None else self.presence_penalty),
            float(0.0 if self.frequency_penalty is None else self.frequency_penalty),
            int(self.repeat_last_n or 0),
            int(bool(self.anti_restate)),
        )


class Xorshift64:
    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(lib().ref_xorshift64_new(seed))

    def next_u64(self) -> int:
        return lib().ref_xorshift64_next_u64(ctypes.byref(self.state))

    def next_f32(self) -> float:
        return lib().ref_xorshift64_next_f32(ctypes.byref(self.state))


def softmax_inplace(v):
    a, p = _f32(v)
    lib().ref_softmax_inplace(p, a.size)
    return a


def argmax(v) -> int:
    a, p = _f32(v)
    return lib().ref_argmax(p, a.size)


def apply_penalties(logits, params: Params, history: Sequence[int]):
    a, p = _f32(logits)
    h, hp = _u32(np.asarray(history, dtype=np.uint32).reshape(-1))
    c = params.to_c()
    lib().ref_apply_penalties(p, a.size, ctypes.byref(c), hp, h.size)
    return a


def apply_top_k(logits, k: int):
    a, p = _f32(logits)
    lib().ref_apply_top_k(p, a.size, k)
    return a


def apply_top_p(logits, top_p: float):
    a, p = _f32(logits)
    lib().ref_apply_top_p_on_logits(p, a.size, top_p)
    return a


def apply_min_p(logits, min_p: float):
    a, p = _f32(logits)
    lib().ref_apply_min_p_on_logits(p, a.size, min_p)
    return a


def sample_categorical(probs, r: float) -> int:
    a, p = _f32(probs)
    return lib().ref_sample_categorical(p, a.size, r)


def _decoder(table):
    if table is None:
        return None, None
    blobs = [bytes(b) for b in table]
    offs = np.zeros(len(blobs) + 1, dtype=np.uint64)
    offs[1:] = np.cumsum([len(b) for b in blobs])
    data = np.frombuffer(b"".join(blobs) or b"\0", dtype=np.uint8).copy()
    d = RefDecoder(data.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                   offs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), len(blobs))
    return d, (data, offs)


def sample_logits(logits, params: Params, history: Sequence[int], rng: Xorshift64,
                  decoder_table=None) -> int:
    """sampling.rs:452-527 with the reference RNG."""
    a, p = _f32(logits)
    h, hp = _u32(np.asarray(history, dtype=np.uint32).reshape(-1))
    c = params.to_c()
    d, keep = _decoder(decoder_table)
    return lib().ref_sample_logits(p, a.size, ctypes.byref(c), hp, h.size,
                                   ctypes.byref(d) if d is not None else None,
                                   ctypes.byref(rng.state))


def sample_logits_r(logits, params: Params, history: Sequence[int], r: float):
    """Same chain with a given uniform; returns (token, trace dict)."""
    a, p = _f32(np.array(logits, dtype=np.float32, copy=True))
    h, hp = _u32(np.asarray(history, dtype=np.uint32).reshape(-1))
    c = params.to_c()
    tr = RefTrace()
    t = lib().ref_sample_logits_r(p, a.size, ctypes.byref(c), hp, h.size, float(r),
                                  ctypes.byref(tr))
    return t, tr.as_dict()


def guarded_argmax(logits, history, decoder_table=None) -> int:
    a, p = _f32(logits)
    h, hp = _u32(np.asarray(history, dtype=np.uint32).reshape(-1))
    d, keep = _decoder(decoder_table)
    return lib().ref_guarded_argmax(p, a.size, hp, h.size,
                                    ctypes.byref(d) if d is not None else None)


def sample_batch(logits2d, params_list, histories, uniforms, threads: int = 1):
    """Rows sampled independently with given uniforms (CPU baseline driver)."""
    L = np.ascontiguousarray(logits2d, dtype=np.float32)
    B, V = L.shape
    arr = (RefParams * B)(*[p.to_c() for p in params_list])
    offs = np.zeros(B + 1, dtype=np.uint64)
    offs[1:] = np.cumsum([len(h) for h in histories])
    flat = np.concatenate([np.asarray(h, dtype=np.uint32).reshape(-1) for h in histories]
                          + [np.zeros(1, dtype=np.uint32)])
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    out = np.zeros(B, dtype=np.uint32)
    lib().ref_sample_batch(L.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), B, V, arr,
                           offs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                           flat.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                           u.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), threads)
    return out


def glibc_expf(x: float) -> float:
    return lib().ref_glibc_expf(x)


def expf_check_range(start: int, count: int):
    bad_first = ctypes.c_uint32(0)
    n = lib().ref_expf_check_range(start, count, ctypes.byref(bad_first))
    return n, bad_first.value


def expf_table():
    t = (ctypes.c_uint64 * 32)()
    lib().ref_expf_table(t)
    return [int(x) for x in t]
