"""Request-level sampling parameters: the server wire layer's validation,
defaults and seed policy, resolved into SamplingParams for the sampler.

Follows crates/lumen-server/src/wire/openai.rs:184-243 (chat) and :290-338
(completions), the `diag_*` resolvers of crates/lumen-server/src/wire/mod.rs
and crates/lumen-runtime/src/runtime_defaults.rs:391-519, 970-999. Ranges are
checked by the library (lumen_sampling_params_validate) so every binding
rejects the same requests.
"""
from __future__ import annotations

import ctypes
import itertools
import os
import re
import threading
import time
from dataclasses import dataclass
from typing import Any, Mapping, Optional

import numpy as np

from . import _native
from .sampling import SamplingParams

# Rust's f32 / usize `FromStr` grammars (no surrounding whitespace, no '_')
_F32_RE = re.compile(r"^[+-]?(?:(?:\d+\.?\d*|\.\d+)(?:[eE][+-]?\d+)?|inf|infinity|nan)$",
                     re.IGNORECASE)
_USIZE_RE = re.compile(r"^\+?\d+$")


def _parse_f32(v: Optional[str]) -> Optional[float]:
    if v is None or not _F32_RE.match(v):
        return None
    return float(np.float32(float(v)))


def _parse_usize(v: Optional[str]) -> Optional[int]:
    if v is None or not _USIZE_RE.match(v):
        return None
    n = int(v)
    return n if n < 2**64 else None


@dataclass
class ModelHint:
    """What the server knows about the loaded model (runtime_defaults.rs:
    MODEL_IS_MOE and the dense-quant hint)."""

    moe: bool = False
    bf16: bool = False


def default_temperature() -> float:
    """runtime_defaults.rs:486-488."""
    return 0.7


def repetition_penalty_default(model: ModelHint) -> float:
    """runtime_defaults.rs:431-452: 1.03 for MoE (every quant), 1.05 dense."""
    return 1.03 if model.moe else 1.05


def diag_repetition_penalty(model: ModelHint) -> float:
    """wire/mod.rs:111-117: LUMEN_REPETITION_PENALTY when finite and > 0."""
    v = _parse_f32(os.environ.get("LUMEN_REPETITION_PENALTY"))
    if v is not None and np.isfinite(v) and v > 0.0:
        return v
    return repetition_penalty_default(model)


def frequency_penalty_resolved() -> float:
    """runtime_defaults.rs:499-505: LUMEN_FREQUENCY_PENALTY when finite and >= 0."""
    v = _parse_f32(os.environ.get("LUMEN_FREQUENCY_PENALTY"))
    if v is not None and np.isfinite(v) and v >= 0.0:
        return v
    return 0.0


def repeat_last_n_resolved() -> Optional[int]:
    """runtime_defaults.rs:517-521: LUMEN_REPEAT_LAST_N, else the whole history."""
    return _parse_usize(os.environ.get("LUMEN_REPEAT_LAST_N"))


def anti_restate_default(model: ModelHint) -> bool:
    """runtime_defaults.rs:970-999: LUMEN_ANTI_RESTATE 0/false/no/off -> off,
    any other value -> on; unset -> on only for a BF16 MoE model."""
    v = os.environ.get("LUMEN_ANTI_RESTATE")
    if v is not None:
        return v not in ("0", "false", "no", "off")
    return model.moe and model.bf16


def normalize_zero_penalty(v: Optional[float]) -> Optional[float]:
    """wire/mod.rs:218-220: 0, -0 and non-finite values mean `None`."""
    if v is None:
        return None
    v = float(np.float32(v))
    return v if np.isfinite(v) and v != 0.0 else None


_seed_lock = threading.Lock()
_seed_counter = itertools.count()
_seed_start: Optional[int] = None


def next_random_seed() -> int:
    """wire/mod.rs:81-91: the process start time in ns plus a shared counter
    (wrapping at 2^64), so concurrent requests never share a seed."""
    global _seed_start
    with _seed_lock:
        if _seed_start is None:
            _seed_start = time.time_ns() & (2**64 - 1)
        return (_seed_start + next(_seed_counter)) & (2**64 - 1)


class WireError(ValueError):
    """An HTTP 400 of the wire layer: message and the offending field."""

    def __init__(self, message: str, field: str):
        super().__init__(message)
        self.field = field
        self.code = "invalid_value"


def validate_sampler_ranges(temperature: Optional[float], top_p: Optional[float]) -> None:
    """openai.rs:357-381 through lumen_sampling_params_validate."""
    L = _native.load()
    p = SamplingParams(temperature=1.0 if temperature is None else temperature, top_p=top_p).to_c()
    if L.lumen_sampling_params_validate(ctypes.byref(p)) != 0:
        msg = L.lumen_sampler_last_error().decode(errors="replace")
        raise WireError(msg, "temperature" if msg.startswith("temperature") else "top_p")


def sampling_from_request(req: Mapping[str, Any], model: ModelHint = ModelHint()) -> SamplingParams:
    """The SamplingParams of an OpenAI chat / completions request body
    (openai.rs:184-243, 290-338): ranges checked first, then the defaults."""
    t = req.get("temperature")
    top_p = req.get("top_p")
    validate_sampler_ranges(t, top_p)
    presence = normalize_zero_penalty(req.get("presence_penalty"))
    freq = normalize_zero_penalty(req.get("frequency_penalty"))
    if freq is None:
        freq = frequency_penalty_resolved()
    seed = req.get("seed")
    return SamplingParams(
        temperature=default_temperature() if t is None else float(np.float32(t)),
        seed=next_random_seed() if seed is None else int(seed),
        top_p=None if top_p is None else float(np.float32(top_p)),
        top_k=req.get("top_k"),
        min_p=None if req.get("min_p") is None else float(np.float32(req["min_p"])),
        repetition_penalty=diag_repetition_penalty(model),
        presence_penalty=presence,
        frequency_penalty=freq,
        repeat_last_n=repeat_last_n_resolved(),
        anti_restate=anti_restate_default(model),
    )
