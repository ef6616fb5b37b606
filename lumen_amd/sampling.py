"""Host-side mirror of Lumen's sampler API over the gfx950 engine.

Same names, argument meaning and behaviour as
crates/lumen-runtime/src/sampling.rs:
  SamplingParams (:239-338), Xorshift64 (:45-106), SamplerState (:352-393),
  Sampler (:397-434), sample_logits (:452-527),
plus the engine shims sample_token / sample_token_with_state
(crates/lumen-runtime/src/engine.rs:61-88).

Logits are device tensors (torch, fp32 or bf16, on the GPU). They are never
modified (the reference overwrites its slice; callers must not rely on that
either way). Every call goes through liblumen_sampler.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import itertools
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import _native

F32_EPSILON = float(np.finfo(np.float32).eps)


@dataclass
class SamplingParams:
    """sampling.rs:239-325. `None` behaves exactly like the reference's None."""

    temperature: float = 1.0
    seed: Optional[int] = None
    top_p: Optional[float] = None
    top_k: Optional[int] = None
    min_p: Optional[float] = None
    repetition_penalty: Optional[float] = None
    presence_penalty: Optional[float] = None
    frequency_penalty: Optional[float] = None
    repeat_last_n: Optional[int] = None
    anti_restate: bool = False

    def penalties_active(self) -> bool:
        """sampling.rs:332-337 (f32 arithmetic)."""
        rep = np.float32(1.0 if self.repetition_penalty is None else self.repetition_penalty)
        presence = np.float32(self.presence_penalty or 0.0)
        freq = np.float32(self.frequency_penalty or 0.0)
        return bool(abs(np.float32(rep - np.float32(1.0))) >= np.float32(F32_EPSILON)
                    or presence != 0.0 or freq != 0.0)

    def validate(self) -> None:
        """Wire-level range check (crates/lumen-server/src/wire/openai.rs:357-381)
        through the library: temperature finite in [0, 2], top_p finite in
        [0, 1] (None passes). Raises ValueError with the reference's message."""
        c = self.to_c()
        L = _native.load()
        if L.lumen_sampling_params_validate(ctypes.byref(c)) != 0:
            raise ValueError(L.lumen_sampler_last_error().decode(errors="replace"))

    def to_c(self) -> _native.SamplingParamsC:
        return _native.SamplingParamsC(
            float(self.temperature),
            float(1.0 if self.top_p is None else self.top_p),
            float(0.0 if self.min_p is None else self.min_p),
            float(1.0 if self.repetition_penalty is None else self.repetition_penalty),
            float(0.0 if self.presence_penalty is None else self.presence_penalty),
            float(0.0 if self.frequency_penalty is None else self.frequency_penalty),
            int(self.top_k or 0),
            int(self.repeat_last_n or 0),
            int(bool(self.anti_restate)),
            0,
        )


class Xorshift64:
    """sampling.rs:45-106, through the library's C implementation."""

    def __init__(self, seed: int):
        self._state = ctypes.c_uint64(_native.load().lumen_xorshift64_new(seed & (2**64 - 1)))

    @classmethod
    def new(cls, seed: int) -> "Xorshift64":
        return cls(seed)

    def next_u64(self) -> int:
        return _native.load().lumen_xorshift64_next_u64(ctypes.byref(self._state))

    def next_f32(self) -> float:
        return _native.load().lumen_xorshift64_next_f32(ctypes.byref(self._state))

    def state(self) -> int:
        return self._state.value

    def set_state(self, s: int):
        self._state.value = s


@dataclass
class SamplerState:
    """sampling.rs:352-393: history and per-token counts."""

    history: List[int] = field(default_factory=list)
    freq: Dict[int, int] = field(default_factory=dict)
    # the embedder's byte decoder (SamplerState::decoder): a TokenBytes, a
    # list of bytes per id, or None (the anti-restate sub-word rule is off)
    decoder: Optional[object] = None

    def record(self, token: int):
        self.history.append(int(token))
        self.freq[int(token)] = self.freq.get(int(token), 0) + 1

    def clear(self):
        self.history.clear()
        self.freq.clear()


def _as_device_logits(logits):
    import torch

    if not isinstance(logits, torch.Tensor) or not logits.is_cuda:
        raise TypeError("logits must be a GPU torch.Tensor (fp32 or bf16)")
    if logits.dtype == torch.float32:
        dt = _native.DTYPE_F32
    elif logits.dtype == torch.bfloat16:
        dt = _native.DTYPE_BF16
    else:
        raise TypeError(f"unsupported logits dtype {logits.dtype}")
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit stride along V")
    return logits, dt


class Engine:
    """One lumen_sampler context on one GPU (the C-ABI object)."""

    def __init__(self, device: int = 0):
        L = _native.load()
        h = ctypes.c_void_p()
        _native.check(L.lumen_sampler_create(ctypes.byref(h), int(device)), "lumen_sampler_create")
        self._h = h
        self.device = device

    def close(self):
        if self._h:
            _native.load().lumen_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_wait_limit(self, microseconds: int):
        """Bound of every cross-workgroup wait (lumen_sampler_set_wait_limit);
        0 makes every such wait give up at once."""
        _native.check(_native.load().lumen_sampler_set_wait_limit(self._h, int(microseconds)),
                      "lumen_sampler_set_wait_limit")

    def wait_timeouts(self) -> int:
        """Cross-workgroup waits that gave up since the context was created."""
        n = ctypes.c_uint64()
        _native.check(_native.load().lumen_sampler_wait_timeouts(self._h, ctypes.byref(n)),
                      "lumen_sampler_wait_timeouts")
        return int(n.value)

    def prepare(self, logits, params: Sequence[SamplingParams], **kw) -> "PreparedBatch":
        """A reusable batch description (see PreparedBatch)."""
        return PreparedBatch(self, logits, params, **kw)

    def sample_batch(self, logits, params: Sequence[SamplingParams],
                     histories: Optional[Sequence[Sequence[int]]] = None,
                     uniforms: Optional[Sequence[float]] = None,
                     rngs: Optional[Sequence[Xorshift64]] = None,
                     penalty_counts=None, tokens_out=None, trace=None, penalized_out=None,
                     sync: bool = True, stream=None, uniforms_dev=None, rng_states_dev=None,
                     hist_ring_dev=None, hist_len_dev=None, hist_epoch=0, guard_out=None, decoder=None,
                    noalloc: bool = False):
        """Samples every row of `logits` [B, V].

        histories: SamplerState.history per row (the window is applied here),
        or penalty_counts = (offsets, ids, counts) device int32 tensors already
        windowed (the caller-resident SamplerState.freq).
        uniforms: one draw per row; or rngs: Xorshift64 per row (advanced);
        or uniforms_dev: a float32 device tensor of draws (no staging copy);
        or rng_states_dev: an int64 device tensor of Xorshift64 states, drawn
        from and advanced by the kernel (greedy rows keep their state).
        hist_ring_dev / hist_len_dev: device-resident history (an int32
        [B, cap] ring and an int32 [B] count of recorded tokens); the window
        is counted on the device and each row's token recorded there;
        hist_epoch: changed by the caller whenever it writes the ring itself
        (between calls that only the library appended to, the counts are
        updated by the one new token instead of counted again).
        guard_out: an int32 device [B, 9] tensor for the anti-restate
        candidates (required for anti_restate rows when sync=False);
        decoder: TokenBytes (or a list of bytes per id) for the guard's
        sub-word rule.
        noalloc: use lumen_sampler_sample_batch_noalloc (asynchronous, at
        most 8 rows; nothing allocated).
        Returns the token tensor (device); with sync=True also a host list.
        """
        import torch

        L = _native.load()
        lg, dt = _as_device_logits(logits)
        B, V = lg.shape
        if len(params) != B:
            raise ValueError("one SamplingParams per row")
        pc = (_native.SamplingParamsC * B)(*[p.to_c() for p in params])
        bt = _native.BatchC()
        bt.logits = lg.data_ptr()
        bt.dtype = dt
        bt.batch = B
        bt.vocab = V
        bt.row_stride = lg.stride(0) if B > 1 else V  # a size-1 dim may carry any stride
        bt.params = pc
        keep = []
        if penalty_counts is not None:
            offs, ids, cnts = penalty_counts
            bt.pen_offsets = offs.data_ptr()
            bt.pen_ids = ids.data_ptr()
            bt.pen_counts = cnts.data_ptr()
        elif histories is not None:
            offs = np.zeros(B + 1, dtype=np.uint64)
            offs[1:] = np.cumsum([len(h) for h in histories])
            flat = np.concatenate([np.asarray(h, dtype=np.uint32).reshape(-1) for h in histories]
                                  + [np.zeros(1, np.uint32)])
            keep += [offs, flat]
            bt.history_offsets = offs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
            bt.history = flat.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
        if hist_ring_dev is not None:
            if histories is not None or penalty_counts is not None:
                raise ValueError("hist_ring_dev excludes histories and penalty_counts")
            if hist_len_dev is None or hist_ring_dev.dim() != 2 or hist_ring_dev.shape[0] < B \
                    or hist_ring_dev.element_size() != 4 or not hist_ring_dev.is_contiguous() \
                    or hist_len_dev.element_size() != 4 or hist_len_dev.numel() < B \
                    or hist_ring_dev.device != lg.device or hist_len_dev.device != lg.device:
                raise ValueError("hist_ring_dev: a contiguous 4-byte [B, cap] tensor and "
                                 "hist_len_dev a 4-byte [B] tensor on the logits' device")
            bt.hist_ring_dev = hist_ring_dev.data_ptr()
            bt.hist_len_dev = hist_len_dev.data_ptr()
            bt.hist_cap = hist_ring_dev.shape[1]
            bt.hist_epoch = int(hist_epoch) & 0xFFFFFFFF
        if guard_out is not None:
            bt.guard_out = guard_out.data_ptr()
        if decoder is not None:
            if not isinstance(decoder, TokenBytes):
                decoder = TokenBytes(decoder)
            keep.append(decoder)
            bt.decoder = ctypes.pointer(decoder.c)
        if uniforms_dev is not None:
            bt.uniforms_dev = uniforms_dev.data_ptr()
        elif rng_states_dev is not None:
            if rng_states_dev.numel() < B or rng_states_dev.element_size() != 8 \
                    or not rng_states_dev.is_contiguous() or rng_states_dev.device != lg.device:
                raise ValueError("rng_states_dev: a contiguous 8-byte tensor of B states "
                                 "on the logits' device")
            bt.rng_states_dev = rng_states_dev.data_ptr()
        elif rngs is not None:
            st = np.array([r.state() for r in rngs], dtype=np.uint64)
            keep.append(st)
            bt.rng_states = st.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
        else:
            u = np.zeros(B, dtype=np.float32) if uniforms is None else \
                np.ascontiguousarray(uniforms, dtype=np.float32)
            keep.append(u)
            bt.uniforms = u.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        dev = lg.device
        if tokens_out is None:
            tokens_out = torch.empty(B, dtype=torch.int32, device=dev)
        bt.tokens = tokens_out.data_ptr()
        if trace is not None:
            bt.trace = trace.data_ptr()
        if penalized_out is not None:
            bt.penalized_out = penalized_out.data_ptr()
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        if noalloc:
            if sync:
                raise ValueError("noalloc is asynchronous: pass sync=False")
            rc = L.lumen_sampler_sample_batch_noalloc(self._h, ctypes.byref(bt), s)
        elif sync:
            host = (ctypes.c_uint32 * B)()
            rc = L.lumen_sampler_sample_batch_sync(self._h, ctypes.byref(bt), host, s)
        else:
            rc = L.lumen_sampler_sample_batch(self._h, ctypes.byref(bt), s)
        if rngs is not None and uniforms_dev is None and rng_states_dev is None:
            for r, v in zip(rngs, st.tolist()):
                r.set_state(int(v))
        _native.check(rc, "lumen_sampler_sample_batch")
        return (tokens_out, list(host)) if sync else (tokens_out, None)


class TokenBytes:
    """The embedder's per-id byte decoder (SamplerState::decoder,
    sampling.rs:343-378) as a table: table[i] is the bytes of id i."""

    def __init__(self, table: Sequence[bytes]):
        blobs = [bytes(b) for b in table]
        self.offsets = np.zeros(len(blobs) + 1, dtype=np.uint64)
        self.offsets[1:] = np.cumsum([len(b) for b in blobs])
        self.data = np.frombuffer(b"".join(blobs) + b"\0", dtype=np.uint8).copy()
        self.c = _native.TokenBytesC(self.data.ctypes.data, self.offsets.ctypes.data, len(blobs))


def anti_restate_select(candidates: Sequence[int], history: Sequence[int],
                        decoder=None) -> int:
    """guarded_argmax (sampling.rs:563-603) from the 9 device candidates of
    a row (guard_out[b]) and its history, through the library."""
    L = _native.load()
    c = (ctypes.c_uint32 * 9)(*[int(x) & 0xFFFFFFFF for x in candidates])
    h = np.ascontiguousarray(np.asarray(history, dtype=np.uint32).reshape(-1))
    d = None
    if decoder is not None:
        if not isinstance(decoder, TokenBytes):
            decoder = TokenBytes(decoder)
        d = ctypes.pointer(decoder.c)
    return int(L.lumen_anti_restate_select(
        c, h.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), h.size, d))


_epochs = itertools.count(1)


def next_epoch() -> int:
    """A fresh DeviceDecodeState epoch (see lumen_batch.hist_epoch)."""
    return next(_epochs)


class DeviceDecodeState:
    """Per-row decode state kept in device memory: the Xorshift64 state
    (Sampler::rng, sampling.rs:395-403) and the history ring
    (SamplerState::history, sampling.rs:353-389) of `cap` tokens. It is
    seeded through lumen_sampler_decode_seed from the seeds and the prompts
    (GpuSamplerRunCfg.rng_seed_state / prompt_history, compute/mod.rs:202-227);
    with `params` and `vocab` the prompts' penalty windows are counted there
    too. A decode step samples with `step(engine, logits, params)`: no host
    draw, no history upload, and the sampled tokens are recorded on the
    device. Writing `ring` or `lens` directly (a new prompt) must be followed
    by `self.epoch = next_epoch()`, so the window counts are made again."""

    def __init__(self, eng: "Engine", seeds: Sequence[int], cap: int = 4096,
                 histories: Optional[Sequence[Sequence[int]]] = None,
                 params: Optional[Sequence[SamplingParams]] = None, vocab: int = 0,
                 stream=None):
        import torch

        B = len(seeds)
        dev = torch.device("cuda", eng.device)
        self.rng = torch.empty(B, dtype=torch.int64, device=dev)
        self.ring = torch.empty((B, cap), dtype=torch.int32, device=dev)
        self.lens = torch.empty(B, dtype=torch.int32, device=dev)
        self.epoch = next(_epochs)
        st = np.array([Xorshift64(s).state() for s in seeds], dtype=np.uint64)
        hs = [np.asarray(h, dtype=np.uint32).reshape(-1) for h in (histories or [])]
        hs += [np.zeros(0, dtype=np.uint32)] * (B - len(hs))
        offs = np.zeros(B + 1, dtype=np.uint64)
        offs[1:] = np.cumsum([h.size for h in hs])
        ids = np.concatenate(hs + [np.zeros(1, dtype=np.uint32)])
        d = _native.DecodeSeedC()
        d.batch = B
        d.vocab = int(vocab)
        keep = [st, offs, ids]
        if params is not None:
            pc = (_native.SamplingParamsC * B)(*[p.to_c() for p in params])
            keep.append(pc)
            d.params = pc
        d.rng_seed_states = st.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
        d.prompt_offsets = offs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
        d.prompt_ids = ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
        d.rng_states_dev = self.rng.data_ptr()
        d.hist_ring_dev = self.ring.data_ptr()
        d.hist_len_dev = self.lens.data_ptr()
        d.hist_cap = cap
        d.hist_epoch = self.epoch
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        rc = _native.load().lumen_sampler_decode_seed(eng._h, ctypes.byref(d), s)
        _native.check(rc, "lumen_sampler_decode_seed")
        del keep  # staged into pinned memory before the call returned

    def step(self, eng: "Engine", logits, params: Sequence[SamplingParams], **kw):
        return eng.sample_batch(logits, params, rng_states_dev=self.rng,
                                hist_ring_dev=self.ring, hist_len_dev=self.lens,
                                hist_epoch=self.epoch, **kw)


class PreparedBatch:
    """A batch whose C description is built once and reused across calls:
    the decode-loop form of Engine.sample_batch. Between calls only the
    per-row draws change (`run(uniforms)`); the logits, parameters, penalty
    counts and outputs are the tensors given here, read again on every call
    (update them in place). The per-call host cost is one C-ABI call."""

    def __init__(self, eng: "Engine", logits, params: Sequence[SamplingParams],
                 penalty_counts=None, tokens_out=None, trace=None, stream=None,
                 uniforms_dev=None, rng_states_dev=None):
        import torch

        lg, dt = _as_device_logits(logits)
        B, V = lg.shape
        if len(params) != B:
            raise ValueError("one SamplingParams per row")
        self._eng = eng
        self._keep = [lg]
        self.params_c = (_native.SamplingParamsC * B)(*[p.to_c() for p in params])
        bt = _native.BatchC()
        bt.logits = lg.data_ptr()
        bt.dtype = dt
        bt.batch = B
        bt.vocab = V
        bt.row_stride = lg.stride(0) if B > 1 else V
        bt.params = self.params_c
        if penalty_counts is not None:
            offs, ids, cnts = penalty_counts
            self._keep += [offs, ids, cnts]
            bt.pen_offsets = offs.data_ptr()
            bt.pen_ids = ids.data_ptr()
            bt.pen_counts = cnts.data_ptr()
        self.uniforms = np.zeros(B, dtype=np.float32)
        if uniforms_dev is not None:
            self._keep.append(uniforms_dev)
            bt.uniforms_dev = uniforms_dev.data_ptr()
        elif rng_states_dev is not None:
            self._keep.append(rng_states_dev)
            bt.rng_states_dev = rng_states_dev.data_ptr()
        else:
            bt.uniforms = self.uniforms.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        if tokens_out is None:
            tokens_out = torch.empty(B, dtype=torch.int32, device=lg.device)
        self.tokens = tokens_out
        bt.tokens = tokens_out.data_ptr()
        if trace is not None:
            self._keep.append(trace)
            bt.trace = trace.data_ptr()
        self._bt = bt
        self._bref = ctypes.byref(bt)
        self._host = (ctypes.c_uint32 * B)()
        self._stream = stream if stream is not None else \
            torch.cuda.current_stream(lg.device).cuda_stream
        L = _native.load()
        self._sync = L.lumen_sampler_sample_batch_sync
        self._async = L.lumen_sampler_sample_batch

    def run(self, uniforms: Optional[Sequence[float]] = None, sync: bool = True):
        """One call. uniforms: this call's draws (host form only); returns the
        host token list (sync) or None (the tokens are in `self.tokens`)."""
        if uniforms is not None:
            self.uniforms[:] = uniforms
        if sync:
            rc = self._sync(self._eng._h, self._bref, self._host, self._stream)
            if rc:
                _native.check(rc, "lumen_sampler_sample_batch_sync")
            return list(self._host)
        rc = self._async(self._eng._h, self._bref, self._stream)
        if rc:
            _native.check(rc, "lumen_sampler_sample_batch")
        return None


_engines: Dict[int, Engine] = {}


def engine(device: int = 0) -> Engine:
    if device not in _engines:
        _engines[device] = Engine(device)
    return _engines[device]


def sample_logits(logits, params: SamplingParams, state: SamplerState, rng: Xorshift64) -> int:
    """sampling.rs:452-527 for one row; does not record (as the reference)."""
    dev = logits.device.index or 0
    if logits.numel() == 0:
        return 0
    _, toks = engine(dev).sample_batch(logits, [params], histories=[state.history], rngs=[rng],
                                       decoder=state.decoder)
    return int(toks[0])


class Sampler:
    """sampling.rs:397-434."""

    def __init__(self, params: SamplingParams, rng: Optional[Xorshift64] = None):
        self.params = params
        self.state = SamplerState()
        self.rng = rng if rng is not None else Xorshift64(42 if params.seed is None
                                                          else params.seed)

    @classmethod
    def with_rng(cls, params: SamplingParams, rng: Xorshift64) -> "Sampler":
        return cls(params, rng)

    def sample(self, logits) -> int:
        token = sample_logits(logits, self.params, self.state, self.rng)
        self.state.record(token)
        return token


def sample_token(logits, params: SamplingParams, rng: Xorshift64) -> int:
    """engine.rs:61-70: transient empty state."""
    return sample_logits(logits, params, SamplerState(), rng)


def sample_token_with_state(logits, params: SamplingParams, state: SamplerState,
                            rng: Xorshift64) -> int:
    """engine.rs:80-88: samples then records."""
    t = sample_logits(logits, params, state, rng)
    state.record(t)
    return t
