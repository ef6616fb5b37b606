"""ctypes binding of liblumen_sampler.so (include/lumen_sampler.h).

The library is built in-tree by `python -m lumen_amd.build`. There is no
fallback: if it is missing, importing the sampler raises.
"""
from __future__ import annotations

import ctypes
import os

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "liblumen_sampler.so")

LUMEN_OK = 0
LUMEN_ERR_INVALID = -1
LUMEN_ERR_HIP = -2
LUMEN_ERR_CODE_OBJECT = -3
LUMEN_ERR_NO_DEVICE = -4
LUMEN_ERR_UNSUPPORTED = -5
LUMEN_ERR_ROW = -6
TOKEN_ERROR = 0xFFFFFFFF

DTYPE_F32 = 0
DTYPE_BF16 = 1

# Every symbol include/lumen_sampler.h declares.
EXPORTS = (
    "lumen_sampler_create",
    "lumen_sampler_destroy",
    "lumen_sampler_sample_batch",
    "lumen_sampler_sample_batch_noalloc",
    "lumen_sampler_sample_batch_sync",
    "lumen_sampler_decode_seed",
    "lumen_xorshift64_new",
    "lumen_xorshift64_next_u64",
    "lumen_xorshift64_next_f32",
    "lumen_sampler_version",
    "lumen_sampler_set_wait_limit",
    "lumen_sampler_wait_timeouts",
    "lumen_sampler_last_error",
    "lumen_sampling_params_validate",
    "lumen_anti_restate_select",
)


class SamplingParamsC(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("top_k", ctypes.c_uint64),
        ("repeat_last_n", ctypes.c_uint64),
        ("anti_restate", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class RowTraceC(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_uint32),
        ("path", ctypes.c_uint32),
        ("topk_cutoff_key", ctypes.c_uint32),
        ("topk_survivors", ctypes.c_uint32),
        ("topp_sum", ctypes.c_float),
        ("topp_kept", ctypes.c_uint32),
        ("topp_cum", ctypes.c_float),
        ("windows", ctypes.c_uint32),
        ("final_max", ctypes.c_float),
        ("final_sum", ctypes.c_float),
        ("cdf_before", ctypes.c_float),
        ("cdf_at", ctypes.c_float),
        ("token", ctypes.c_uint32),
        ("passes", ctypes.c_uint32),
        ("pad", ctypes.c_uint32 * 2),
    ]


TRACE_WORDS = ctypes.sizeof(RowTraceC) // 4


class TokenBytesC(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("count", ctypes.c_uint64),
    ]


class BatchC(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32),
        ("row_stride", ctypes.c_uint64),
        ("params", ctypes.POINTER(SamplingParamsC)),
        ("history_offsets", ctypes.POINTER(ctypes.c_uint64)),
        ("history", ctypes.POINTER(ctypes.c_uint32)),
        ("pen_offsets", ctypes.c_void_p),
        ("pen_ids", ctypes.c_void_p),
        ("pen_counts", ctypes.c_void_p),
        ("uniforms", ctypes.POINTER(ctypes.c_float)),
        ("rng_states", ctypes.POINTER(ctypes.c_uint64)),
        ("uniforms_dev", ctypes.c_void_p),
        ("tokens", ctypes.c_void_p),
        ("trace", ctypes.c_void_p),
        ("penalized_out", ctypes.c_void_p),
        ("rng_states_dev", ctypes.c_void_p),
        ("hist_ring_dev", ctypes.c_void_p),
        ("hist_len_dev", ctypes.c_void_p),
        ("hist_cap", ctypes.c_uint32),
        ("hist_epoch", ctypes.c_uint32),
        ("guard_out", ctypes.c_void_p),
        ("decoder", ctypes.POINTER(TokenBytesC)),
    ]


class DecodeSeedC(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32),
        ("params", ctypes.POINTER(SamplingParamsC)),
        ("rng_seed_states", ctypes.POINTER(ctypes.c_uint64)),
        ("prompt_offsets", ctypes.POINTER(ctypes.c_uint64)),
        ("prompt_ids", ctypes.POINTER(ctypes.c_uint32)),
        ("rng_states_dev", ctypes.c_void_p),
        ("hist_ring_dev", ctypes.c_void_p),
        ("hist_len_dev", ctypes.c_void_p),
        ("hist_cap", ctypes.c_uint32),
        ("hist_epoch", ctypes.c_uint32),
    ]


_lib = None


def load():
    """Loads the in-tree library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"lumen_amd native library not found at {LIB_PATH}; build it with "
            "`python -m lumen_amd.build` (there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    L.lumen_sampler_create.restype = ctypes.c_int
    L.lumen_sampler_create.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int]
    L.lumen_sampler_destroy.restype = None
    L.lumen_sampler_destroy.argtypes = [ctypes.c_void_p]
    L.lumen_sampler_sample_batch.restype = ctypes.c_int
    L.lumen_sampler_sample_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(BatchC),
                                             ctypes.c_void_p]
    L.lumen_sampler_sample_batch_noalloc.restype = ctypes.c_int
    L.lumen_sampler_sample_batch_noalloc.argtypes = L.lumen_sampler_sample_batch.argtypes
    L.lumen_sampler_sample_batch_sync.restype = ctypes.c_int
    L.lumen_sampler_sample_batch_sync.argtypes = [ctypes.c_void_p, ctypes.POINTER(BatchC),
                                                  ctypes.POINTER(ctypes.c_uint32),
                                                  ctypes.c_void_p]
    L.lumen_xorshift64_new.restype = ctypes.c_uint64
    L.lumen_sampler_decode_seed.restype = ctypes.c_int
    L.lumen_sampler_decode_seed.argtypes = [ctypes.c_void_p, ctypes.POINTER(DecodeSeedC),
                                            ctypes.c_void_p]
    L.lumen_xorshift64_new.argtypes = [ctypes.c_uint64]
    L.lumen_xorshift64_next_u64.restype = ctypes.c_uint64
    L.lumen_xorshift64_next_u64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.lumen_xorshift64_next_f32.restype = ctypes.c_float
    L.lumen_xorshift64_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.lumen_sampler_set_wait_limit.restype = ctypes.c_int
    L.lumen_sampler_set_wait_limit.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    L.lumen_sampler_wait_timeouts.restype = ctypes.c_int
    L.lumen_sampler_wait_timeouts.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)]
    L.lumen_sampler_version.restype = ctypes.c_char_p
    L.lumen_sampler_version.argtypes = []
    L.lumen_sampler_last_error.restype = ctypes.c_char_p
    L.lumen_sampler_last_error.argtypes = []
    L.lumen_anti_restate_select.restype = ctypes.c_uint32
    L.lumen_anti_restate_select.argtypes = [ctypes.POINTER(ctypes.c_uint32),
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint64,
                                            ctypes.POINTER(TokenBytesC)]
    L.lumen_sampling_params_validate.restype = ctypes.c_int
    L.lumen_sampling_params_validate.argtypes = [ctypes.POINTER(SamplingParamsC)]
    _lib = L
    return L


def check(rc: int, what: str):
    if rc != LUMEN_OK:
        names = {LUMEN_ERR_INVALID: "invalid argument", LUMEN_ERR_HIP: "HIP runtime error",
                 LUMEN_ERR_CODE_OBJECT: "gfx950 code object missing or corrupt",
                 LUMEN_ERR_NO_DEVICE: "no GPU device",
                 LUMEN_ERR_UNSUPPORTED: "unsupported parameter combination",
                 LUMEN_ERR_ROW: "a row could not be resolved"}
        why = load().lumen_sampler_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {names.get(rc, rc)} ({rc}): {why}")
