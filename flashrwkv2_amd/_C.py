"""Native-layer operator surface of the WKV7 path, on the gfx950 C ABI.

This module plays the role of the reference's private pybind module
``flashrwkv2._C`` for the WKV7 path: the same function names, positional
order, keyword defaults, ticket class and ``RuntimeError`` texts where the
reference's tests match on them.  Argument checks run here in Python; every
computation runs in the HIP kernels of ``lib/libflashrwkv2_amd.so`` through
:mod:`flashrwkv2_amd._native`.  There is no other execution path.

Reference bindings mirrored:
  csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cpp:45-434
  csrc/validation.cpp:12-129
  csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:20-55
  csrc/sm120/tmix/wkv7/infer_chunk_bf16_forward_varlen.cpp:44-204
  csrc/sm120/tmix/wkv7/rl_infctx_chunk_fp32io16_forward.cpp:73-241
  csrc/sm120/tmix/wkv7/rl_infctx_chunk_fp32io16_backward.cpp:22-135
  csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cpp:26-56
  csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_backward.cpp:34-82
"""

from __future__ import annotations

import ctypes
import functools
import math
from typing import Sequence

import torch

from . import _native as N
from ._align import aligned_io
from ._statetune_plan import statetune_padded_plan as _statetune_padded_plan

INT32_MAX = 2**31 - 1
_TOKEN_DTYPES = {torch.float16: N.FR2_DTYPE_FLOAT16, torch.bfloat16: N.FR2_DTYPE_BFLOAT16}

def _check(cond: bool, *msg: object) -> None:
    if not cond:
        raise RuntimeError("".join(str(m) for m in msg))


def check_cuda_contiguous(t: torch.Tensor, name: str) -> None:
    """validation.cpp:12-15."""
    _check(isinstance(t, torch.Tensor) and t.is_cuda, name, " must be CUDA")
    _check(t.is_contiguous(), name, " must be contiguous")


def check_same_device(ref: torch.Tensor, t: torch.Tensor, name: str) -> None:
    """validation.cpp:17-25."""
    _check(t.device == ref.device, name, " must be on the same device as state")


def _tensor_version(t: torch.Tensor) -> int | None:
    if t.is_inference():
        return None
    return t._version


_raw_stream = torch._C._cuda_getCurrentRawStream
_get_device = torch._C._cuda_getDevice
_set_device = torch._C._cuda_setDevice


def _stream(device: torch.device) -> int:
    """The current HIP stream handle of `device` (raw getter: no Stream object)."""
    idx = device.index
    return _raw_stream(_get_device() if idx is None else idx)


class _on_device:
    """``torch.cuda.device`` without its bookkeeping: switches the current
    device only when it differs, and switches back on exit."""

    __slots__ = ("_idx", "_prev")

    def __init__(self, device):
        self._idx = device.index if isinstance(device, torch.device) else device

    def __enter__(self):
        self._prev = _get_device()
        if self._idx is not None and self._idx != self._prev:
            _set_device(self._idx)

    def __exit__(self, *exc):
        if self._idx is not None and self._idx != self._prev:
            _set_device(self._prev)
        return False


_aux_streams: dict[int, torch.cuda.Stream] = {}


def _aux_stream(device: torch.device) -> int:
    """The second stream of the pipelined sequence split (piece 0 runs on it
    next to the summary pass), one per device, default priority.  The library
    orders it against the caller's stream with events, so it joins a graph
    capture of the caller's stream."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _aux_streams.get(idx)
    if s is None:
        s = _aux_streams[idx] = torch.cuda.Stream(device=idx)
    return s.cuda_stream


def _dtype_code(t: torch.Tensor) -> int:
    return _TOKEN_DTYPES[t.dtype]


def handoff_fault_count(device: torch.device | None = None, *, reset: bool = False) -> int:
    """Blocks of the chunked MFMA kernels on ``device`` that failed closed
    since the last reset: a bounded wave hand-off wait gave up, so the block
    wrote NaN outputs and left its state slots untouched.  Synchronises the
    current stream (call it after the work it should cover)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    count = ctypes.c_int32(0)
    with _on_device(device):
        N.check(N.load().fr2_handoff_fault_count(ctypes.byref(count), int(reset),
                                                 _stream(device)), "fr2_handoff_fault_count")
    return int(count.value)


def _set_handoff_spin_limit(polls: int) -> None:
    """Test hook: polls a hand-off wait makes before it gives up, for later
    launches in this process (negative restores the default)."""
    N.check(N.load().fr2_debug_set_handoff_spin_limit(int(polls)),
            "fr2_debug_set_handoff_spin_limit")


def _set_handoff_stall(on: bool) -> None:
    """Test hook: while on, the chunked kernel's key waves never publish their
    operators, so every block stalls at its first operator wait and fails
    closed after the spin limit."""
    N.check(N.load().fr2_debug_set_handoff_stall(int(bool(on))), "fr2_debug_set_handoff_stall")


def _set_chunk_ring(on: bool) -> None:
    """Test hook: selects the workgroup chunked kernel's variant for later
    fp32-state launches: True = one key wave per whole chunk over a ring of
    four chunk operator blocks (the default), False = two key waves per chunk
    with the token-token blocks summed through LDS."""
    N.check(N.load().fr2_debug_set_chunk_ring(int(bool(on))), "fr2_debug_set_chunk_ring")


# ---------------------------------------------------------------------------
# Metadata tickets
# ---------------------------------------------------------------------------
class _RecurrentMetadataTicket:
    """Validated packed metadata bound to a stream.

    Mirrors RecurrentMetadataTicket
    (infer_recurrent_fp32io16_forward_varlen.cpp:89-225): it keeps the
    validated snapshot (static form) or the live buffers (graph form), the
    device status, and the identity/version/shape/stream facts that every
    consumer re-checks.
    """

    def __init__(self, qsl, slots, qsl_snap, slots_snap, status, workspace,
                 live_tokens, live_seqs, total_tokens, pool_size, max_seqlen,
                 graph_mode, stream):
        self._qsl = qsl
        self._slots = slots
        self._qsl_snap = qsl_snap
        self._slots_snap = slots_snap
        self._status_t = status
        self._workspace = workspace
        self._live_tokens = live_tokens
        self._live_seqs = live_seqs
        self._qsl_version = _tensor_version(qsl)
        self._slots_version = _tensor_version(slots)
        self._qsl_ptr = qsl.data_ptr()
        self._slots_ptr = slots.data_ptr()
        self._qsl_geom = (tuple(qsl.shape), tuple(qsl.stride()))
        self._slots_geom = (tuple(slots.shape), tuple(slots.stride()))
        self._total_tokens = int(total_tokens)
        self._pool_size = int(pool_size)
        self._max_seqlen_v = int(max_seqlen)
        self._graph = bool(graph_mode)
        self._device = qsl.device
        self._stream_handle = stream
        # the same facts for the native fast path (hostpath.cpp)
        self._facts = N.hostpath().TicketFacts(qsl, slots, qsl_snap, slots_snap, status,
                                                self._total_tokens, self._pool_size,
                                                self._max_seqlen_v, self._graph, stream)

    def _check_compatible(self, query_start_loc, state_indices, total_tokens,
                          state_pool_size, max_seqlen) -> None:
        if (query_start_loc is self._qsl and state_indices is self._slots
                and query_start_loc.data_ptr() == self._qsl_ptr
                and state_indices.data_ptr() == self._slots_ptr
                and (self._graph or self._qsl_version is None
                     or _tensor_version(query_start_loc) == self._qsl_version)
                and (self._graph or self._slots_version is None
                     or _tensor_version(state_indices) == self._slots_version)
                and int(total_tokens) == self._total_tokens
                and int(state_pool_size) == self._pool_size
                and (max_seqlen <= 0 or int(max_seqlen) == self._max_seqlen_v)
                and _stream(self._device) == self._stream_handle
                and (tuple(query_start_loc.shape), tuple(query_start_loc.stride())) == self._qsl_geom
                and (tuple(state_indices.shape), tuple(state_indices.stride())) == self._slots_geom):
            return   # same tensors, same storage, same device (the identity implies it)
        _check(query_start_loc is self._qsl,
               "validated_metadata query_start_loc identity mismatch")
        _check(state_indices is self._slots,
               "validated_metadata state_indices identity mismatch")
        _check(query_start_loc.data_ptr() == self._qsl_ptr
               and state_indices.data_ptr() == self._slots_ptr,
               "validated_metadata metadata data_ptr mismatch")
        _check((tuple(query_start_loc.shape), tuple(query_start_loc.stride())) == self._qsl_geom
               and (tuple(state_indices.shape), tuple(state_indices.stride())) == self._slots_geom,
               "validated_metadata metadata shape or stride mismatch")
        if not self._graph and self._qsl_version is not None:
            _check(_tensor_version(query_start_loc) == self._qsl_version,
                   "validated_metadata query_start_loc version mismatch")
        if not self._graph and self._slots_version is not None:
            _check(_tensor_version(state_indices) == self._slots_version,
                   "validated_metadata state_indices version mismatch")
        _check(query_start_loc.device == self._device and state_indices.device == self._device,
               "validated_metadata device mismatch")
        _check(int(total_tokens) == self._total_tokens,
               "validated_metadata total_tokens mismatch")
        _check(int(state_pool_size) == self._pool_size,
               "validated_metadata state_pool_size mismatch")
        if max_seqlen > 0:
            _check(int(max_seqlen) == self._max_seqlen_v,
                   "validated_metadata max_seqlen mismatch")
        _check(_stream(self._device) == self._stream_handle,
               "validated_metadata stream mismatch; prepare and consume the ticket "
               "on the same CUDA stream")

    def _query_start_loc_snapshot(self) -> torch.Tensor:
        return self._qsl_snap

    def _state_indices_snapshot(self) -> torch.Tensor:
        return self._slots_snap

    def _status(self) -> torch.Tensor:
        return self._status_t

    def _max_seqlen(self) -> int:
        return self._max_seqlen_v

    def _is_graph(self) -> bool:
        return self._graph

    def _num_active_tokens(self):
        return self._live_tokens

    def _num_active_sequences(self):
        return self._live_seqs


def _launch_validation(qsl, slots, live_tokens, live_seqs, total_tokens, num_seqs,
                       pool_size, max_seqlen, snapshot):
    """Device validation (recurrent_metadata.cu:134-194): status, workspace,
    and private snapshots for the static form."""
    dev = qsl.device
    with _on_device(dev):
        status = torch.empty(3, device=dev, dtype=torch.int32)
        seen = torch.empty(pool_size, device=dev, dtype=torch.int32)
        qsl_snap = torch.empty_like(qsl) if snapshot else qsl
        slots_snap = torch.empty_like(slots) if snapshot else slots
        rc = N.fast().prepare_metadata(
            qsl.data_ptr(), slots.data_ptr(), int(num_seqs), int(total_tokens),
            int(pool_size), int(max_seqlen),
            N.ptr(live_tokens), N.ptr(live_seqs), status.data_ptr(), seen.data_ptr(),
            qsl_snap.data_ptr() if snapshot else None,
            slots_snap.data_ptr() if snapshot else None, _stream(dev))
    N.check(rc, "prepare_tmix_wkv7_recurrent_metadata")
    return qsl_snap, slots_snap, status, seen


def _host_metadata_max_seqlen(qsl, slots, total_tokens, pool_size) -> int:
    """Host check of the metadata values (…fp32io16_forward_varlen.cpp:45-80);
    returns the longest sequence."""
    offsets = qsl.to("cpu").tolist()
    slot_list = slots.to("cpu").tolist()
    n = len(slot_list)
    _check(offsets[0] == 0, "query_start_loc must start at 0")
    _check(offsets[n] == total_tokens,
           "the final query_start_loc offset must equal total_tokens")
    seen: set[int] = set()
    longest = 0
    for i in range(n):
        lo, hi = offsets[i], offsets[i + 1]
        _check(lo >= 0 and hi > lo and hi <= total_tokens,
               "query_start_loc must be strictly increasing with non-empty sequences")
        s = slot_list[i]
        _check(0 <= s < pool_size, "state_indices entries must be within the state pool")
        _check(s not in seen, "state_indices must be unique within one call")
        seen.add(s)
        longest = max(longest, hi - lo)
    return longest


def prepare_tmix_wkv7_recurrent_metadata(query_start_loc, state_indices, total_tokens,
                                         state_pool_size, max_seqlen=-1):
    """Static ticket (…fp32io16_forward_varlen.cpp:227-275)."""
    check_cuda_contiguous(query_start_loc, "query_start_loc")
    check_cuda_contiguous(state_indices, "state_indices")
    _check(state_indices.device == query_start_loc.device,
           "state_indices must be on the same device as state")
    _check(query_start_loc.dtype == torch.int32 and state_indices.dtype == torch.int32,
           "recurrent metadata must be int32")
    _check(query_start_loc.dim() == 1 and state_indices.dim() == 1
           and state_indices.numel() > 0
           and query_start_loc.numel() == state_indices.numel() + 1,
           "query_start_loc must have shape [B+1] and state_indices shape [B]")
    _check(state_indices.numel() <= 65535,
           "state_indices must contain at most 65535 sequences")
    _check(0 < total_tokens <= INT32_MAX, "total_tokens must be positive and fit in int32")
    _check(0 < state_pool_size <= INT32_MAX,
           "state_pool_size must be positive and fit in int32")
    inferred = _host_metadata_max_seqlen(query_start_loc, state_indices, int(total_tokens),
                                         int(state_pool_size))
    if max_seqlen <= 0:
        max_seqlen = inferred
    else:
        _check(max_seqlen == inferred,
               "max_seqlen must equal the largest packed sequence length")
    stream = _stream(query_start_loc.device)
    snap_q, snap_s, status, seen = _launch_validation(
        query_start_loc, state_indices, None, None, total_tokens,
        state_indices.numel(), state_pool_size, total_tokens, True)
    return _RecurrentMetadataTicket(query_start_loc, state_indices, snap_q, snap_s, status,
                                    seen, None, None, total_tokens, state_pool_size,
                                    max_seqlen, False, stream)


def _prepare_graph_fast(query_start_loc, state_indices, num_active_tokens,
                        num_active_sequences, token_capacity, sequence_capacity,
                        state_pool_size, max_seqlen_capacity):
    """The graph ticket through the native fast path (hostpath.cpp), or None
    when the call is not plainly valid there (the caller then runs
    prepare_tmix_wkv7_recurrent_graph_metadata, which raises or prepares)."""
    try:
        stream = _raw_stream(query_start_loc.get_device())
        res = N.hostpath().prepare_graph(query_start_loc, state_indices, num_active_tokens,
                                         num_active_sequences, token_capacity,
                                         sequence_capacity, state_pool_size,
                                         max_seqlen_capacity, stream)
    except (TypeError, RuntimeError, AttributeError):
        return None
    if res is None:
        return None
    if isinstance(res, int):
        N.check(res, "prepare_tmix_wkv7_recurrent_metadata")
    status, seen = res
    return _RecurrentMetadataTicket(query_start_loc, state_indices, query_start_loc,
                                    state_indices, status, seen, num_active_tokens,
                                    num_active_sequences, token_capacity, state_pool_size,
                                    max_seqlen_capacity, True, stream)


def _check_graph_scalar(t, ref, name):
    _check(isinstance(t, torch.Tensor) and t.is_cuda, name, " must be a CUDA tensor")
    _check(t.is_contiguous(), name, " must be contiguous")
    _check(t.device == ref.device, name, " must share the metadata CUDA device")
    _check(t.dtype == torch.int32, name, " must have dtype int32")
    _check(t.numel() == 1, name, " must contain one element")


def prepare_tmix_wkv7_recurrent_graph_metadata(query_start_loc, state_indices,
                                               num_active_tokens, num_active_sequences,
                                               token_capacity, sequence_capacity,
                                               state_pool_size, max_seqlen_capacity):
    """Live capacity ticket for warmup / graph capture (…cpp:277-326)."""
    if not _graph_metadata_ok(query_start_loc, state_indices, num_active_tokens,
                              num_active_sequences, token_capacity, sequence_capacity,
                              state_pool_size, max_seqlen_capacity):
        _graph_metadata_error(query_start_loc, state_indices, num_active_tokens,
                              num_active_sequences, token_capacity, sequence_capacity,
                              state_pool_size, max_seqlen_capacity)
    stream = _stream(query_start_loc.device)
    snap_q, snap_s, status, seen = _launch_validation(
        query_start_loc, state_indices, num_active_tokens, num_active_sequences,
        token_capacity, sequence_capacity, state_pool_size, max_seqlen_capacity, False)
    return _RecurrentMetadataTicket(query_start_loc, state_indices, snap_q, snap_s, status,
                                    seen, num_active_tokens, num_active_sequences,
                                    token_capacity, state_pool_size, max_seqlen_capacity,
                                    True, stream)


def _graph_metadata_ok(qsl, slots, live_tokens, live_seqs, token_capacity, sequence_capacity,
                       state_pool_size, max_seqlen_capacity) -> bool:
    """The valid case of prepare_tmix_wkv7_recurrent_graph_metadata in one expression."""
    try:
        dev = qsl.get_device()
        return (all(t.is_cuda and t.is_contiguous() and t.get_device() == dev
                    and t.dtype == torch.int32 for t in (qsl, slots, live_tokens, live_seqs))
                and 0 < sequence_capacity <= 65535 and slots.dim() == 1
                and slots.numel() == sequence_capacity and qsl.dim() == 1
                and qsl.numel() == sequence_capacity + 1
                and 0 < token_capacity <= INT32_MAX and 0 < state_pool_size <= INT32_MAX
                and 0 < max_seqlen_capacity <= token_capacity
                and live_tokens.numel() == 1 and live_seqs.numel() == 1)
    except (AttributeError, TypeError):
        return False


def _graph_metadata_error(query_start_loc, state_indices, num_active_tokens,
                          num_active_sequences, token_capacity, sequence_capacity,
                          state_pool_size, max_seqlen_capacity):
    """The checks of the graph-ticket entry in order: raises the first failure."""
    check_cuda_contiguous(query_start_loc, "query_start_loc")
    check_cuda_contiguous(state_indices, "state_indices")
    _check(state_indices.device == query_start_loc.device,
           "state_indices must be on the same device as state")
    _check(query_start_loc.dtype == torch.int32 and state_indices.dtype == torch.int32,
           "recurrent metadata must be int32")
    _check(0 < sequence_capacity <= 65535 and state_indices.dim() == 1
           and state_indices.numel() == sequence_capacity
           and query_start_loc.dim() == 1
           and query_start_loc.numel() == sequence_capacity + 1,
           "graph metadata shapes must match sequence_capacity")
    _check(0 < token_capacity <= INT32_MAX,
           "token_capacity must be positive and fit in int32")
    _check(0 < state_pool_size <= INT32_MAX,
           "state_pool_size must be positive and fit in int32")
    _check(0 < max_seqlen_capacity <= token_capacity,
           "max_seqlen_capacity must be positive and not exceed token_capacity")
    _check_graph_scalar(num_active_tokens, query_start_loc, "num_active_tokens")
    _check_graph_scalar(num_active_sequences, query_start_loc, "num_active_sequences")


# ---------------------------------------------------------------------------
# fp32-state packed recurrence
# ---------------------------------------------------------------------------
_LAYOUT_NAMES = ("query_start_loc", "state_indices", "state", "r", "decay_logits", "k", "v",
                 "a", "b", "output")


def check_recurrent_layout(qsl, slots, state, r, decay_logits, k, v, a, b, output, scale):
    """validation.cpp:27-129.  The common, valid case is decided by one
    expression; only a failing call walks the checks in order for its message."""
    tensors = (qsl, slots, state, r, decay_logits, k, v, a, b, output)
    try:
        n, h, d = slots.numel(), state.size(1), state.size(2)
        dev, rs, rd = state.get_device(), r.shape, r.dtype
        ok = (all(t.is_cuda and t.is_contiguous() and t.get_device() == dev for t in tensors)
              and qsl.dtype == torch.int32 and slots.dtype == torch.int32
              and state.dtype == torch.float32 and rd in _TOKEN_DTYPES
              and math.isfinite(scale) and 0 < n <= 65535 and slots.dim() == 1
              and qsl.dim() == 1 and qsl.size(0) == n + 1 and state.dim() == 4
              and state.size(0) > 0 and 0 < h <= INT32_MAX and state.size(3) == d
              and d in (64, 128, 256) and state.size(0) <= INT32_MAX and len(rs) == 3
              and 0 < rs[0] <= INT32_MAX and rs[1] == h and rs[2] == d
              and all(t.shape == rs and t.dtype == rd
                      for t in (decay_logits, k, v, a, b, output)))
    except (AttributeError, TypeError, IndexError, RuntimeError):
        ok = False
    if ok:
        return n, h, d
    return _recurrent_layout_error(tensors, scale)


def _recurrent_layout_error(tensors, scale):
    qsl, slots, state, r, decay_logits, k, v, a, b, output = tensors
    if not all(isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous() for t in tensors):
        for t, name in zip(tensors, _LAYOUT_NAMES):   # the first offender's message
            check_cuda_contiguous(t, name)
    _check(qsl.dtype == torch.int32, "query_start_loc must be int32")
    _check(slots.dtype == torch.int32, "state_indices must be int32")
    _check(math.isfinite(scale), "scale must be finite")
    n = slots.numel()
    _check(0 < n <= 65535, "state_indices must contain 1..65535 sequences")
    _check(slots.dim() == 1, "state_indices must have shape [N]")
    _check(qsl.dim() == 1 and qsl.size(0) == n + 1, "query_start_loc must have shape [N+1]")
    _check(state.dim() == 4 and state.size(0) > 0 and state.size(1) > 0
           and state.size(2) == state.size(3), "state must have square shape [slots,H,D,D]")
    _check(state.dtype == torch.float32, "state must be float32")
    d = state.size(2)
    _check(d in (64, 128, 256), "recurrent head size must be 64, 128, or 256, got ", d)
    _check(state.size(0) <= INT32_MAX, "state slot count must fit in int32")
    h = state.size(1)
    _check(h <= INT32_MAX, "head count must fit in int32")
    _check(r.dim() == 3 and r.size(0) > 0 and r.size(1) == h and r.size(2) == d,
           "r must have shape [total_tokens,H,D] matching state")
    _check(r.size(0) <= INT32_MAX, "token count must fit in int32")
    _check(all(t.shape == r.shape for t in (decay_logits, k, v, a, b, output)),
           "r,decay_logits,k,v,a,b,output shape mismatch")
    _check(r.dtype in _TOKEN_DTYPES, "token tensors must be float16 or bfloat16")
    _check(all(t.dtype == r.dtype for t in (decay_logits, k, v, a, b, output)),
           "r,decay_logits,k,v,a,b,output dtype mismatch")
    dev = state.get_device()
    if not all(t.get_device() == dev for t in tensors):
        for t, name in zip(tensors, _LAYOUT_NAMES):
            if t is not state:
                check_same_device(state, t, name)
    return n, h, d


def _check_decay_bias(decay_bias, state, r, h, d, dtype_msg):
    check_cuda_contiguous(decay_bias, "decay_bias")
    check_same_device(state, decay_bias, "decay_bias")
    _check(decay_bias.dtype == r.dtype, dtype_msg)
    _check((decay_bias.dim() == 1 and decay_bias.numel() == h * d)
           or (decay_bias.dim() == 2 and decay_bias.size(0) == h and decay_bias.size(1) == d),
           "decay_bias must have shape [H*D] or [H,D]")


def _resolve_launch_metadata(qsl, slots, total_tokens, pool_size, max_seqlen, ticket):
    """Ticket path or an implicit device-only validation (…cpp:360-380)."""
    if ticket is not None:
        ticket._check_compatible(qsl, slots, total_tokens, pool_size, max_seqlen)
        return (ticket._query_start_loc_snapshot(), ticket._state_indices_snapshot(),
                ticket._status(), ticket._max_seqlen(), ticket)
    snap_q, snap_s, status, seen = _launch_validation(
        qsl, slots, None, None, total_tokens, slots.numel(), pool_size, total_tokens, True)
    keep = (snap_q, snap_s, status, seen)
    return snap_q, snap_s, status, max_seqlen, keep


def _recurrent_launch(kernel, qsl, slots, state, r, decay_logits, k, v, a, b, output,
                      scale, decay_bias, validated_metadata, max_seqlen, split_pieces=None):
    n, h, d = check_recurrent_layout(qsl, slots, state, r, decay_logits, k, v, a, b,
                                     output, scale)
    if decay_bias is not None:
        _check_decay_bias(decay_bias, state, r, h, d,
                          "decay_bias must match the token tensor dtype")
    lq, ls, status, max_seqlen, keep = _resolve_launch_metadata(
        qsl, slots, r.size(0), state.size(0), int(max_seqlen), validated_metadata)
    lib = N.load()
    common = (lq.data_ptr(), ls.data_ptr(), status.data_ptr(), n, h, d, r.size(0),
              int(max_seqlen), _dtype_code(r), state.data_ptr(), r.data_ptr(),
              decay_logits.data_ptr(), N.ptr(decay_bias), k.data_ptr(), v.data_ptr(),
              a.data_ptr(), b.data_ptr(), output.data_ptr(), float(scale))
    pieces, piece_len, lead_len, ws_bytes = 1, 0, 0, 0
    if kernel is None or kernel == N.KERNEL_SPLIT:
        # the forced split without a known max_seqlen bounds it by the token count
        ms = int(max_seqlen) if (kernel is None or int(max_seqlen) > 0) else r.size(0)
        pieces, piece_len, lead_len, ws_bytes = split_plan(n, h, d, ms, split_pieces)
        if kernel == N.KERNEL_SPLIT and pieces < 2:
            raise RuntimeError("sequence split needs head size 64 and at least two pieces")
    with _on_device(state.device):
        stream = _stream(state.device)
        if pieces > 1:
            # workspace from the caching allocator on this stream: it is only
            # handed out again to work queued later on the same stream
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=state.device)
            aux = _aux_stream(state.device) if lead_len > 0 else None
            rc = lib.fr2_wkv7_recurrent_fp32_forward_split(*common, pieces, piece_len, lead_len,
                                                           ws.data_ptr(), ws_bytes, stream, aux)
            del ws
        elif kernel is None:
            rc = N.fast().recurrent_fp32_forward(*common, stream)
        else:
            rc = N.fast().recurrent_fp32_forward_kernel(int(kernel), *common, stream)
    N.check(rc, "tmix_wkv7_recurrent_fp32_from_decay_logits")


def tmix_wkv7_recurrent_fp32_from_kk_gate(query_start_loc, state_indices, state, r,
                                          decay_logits, k, v, a12, k_k, a0, k_a, new_k, output,
                                          scale, decay_bias=None, validated_metadata=None,
                                          max_seqlen=-1):
    """The recurrence with wkv_prepare's kk / a-gate stage in its load stage:
    k is the projected key, a12 the a-gate logits, k_k / a0 / k_a the
    per-channel parameters ([H*D] or [H,D], token dtype); the gated key is
    written to new_k.  For fp16 tokens where the library's policy picks no
    chunked kernel (head size other than 64, or the longest sequence at most 4
    tokens, 6 with many units: the decode kernel), and for fp16 batches that
    the library's plan splits by sequence (few long sequences: the split
    outruns one block per unit), the gate runs as its own kernel and the
    recurrence through the public path.  bf16 batches at head size 64 always
    run fused (short batches on the wavefront chunked kernel)."""
    n, h, d = check_recurrent_layout(query_start_loc, state_indices, state, r, decay_logits, k,
                                     v, a12, new_k, output, scale)
    for t, name in ((k_k, "k_k"), (a0, "a0"), (k_a, "k_a")):
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
        _check(t.dtype == r.dtype, name, " must have the token dtype")
        _check(t.numel() == h * d, name, " must have shape [H*D] or [H,D]")
    if decay_bias is not None:
        _check_decay_bias(decay_bias, state, r, h, d,
                          "decay_bias must match the token tensor dtype")
    lq, ls, status, ms, keep = _resolve_launch_metadata(
        query_start_loc, state_indices, r.size(0), state.size(0), int(max_seqlen),
        validated_metadata)
    fp16 = r.dtype == torch.float16
    rc = N.FR2_ERR_UNSUPPORTED
    if not (fp16 and d == 64 and int(ms) > 0 and split_plan(n, h, d, int(ms))[0] > 1):
        with _on_device(state.device):
            rc = N.load().fr2_wkv7_recurrent_fp32_forward_kk_gate(
                lq.data_ptr(), ls.data_ptr(), status.data_ptr(), n, h, d, r.size(0), int(ms),
                _dtype_code(r), state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(),
                N.ptr(decay_bias), k.data_ptr(), v.data_ptr(), a12.data_ptr(), k_k.data_ptr(),
                a0.data_ptr(), k_a.data_ptr(), new_k.data_ptr(), output.data_ptr(),
                float(scale), _stream(state.device))
    if rc == N.FR2_ERR_UNSUPPORTED:
        _check(fp16, "the kk / a-gate stage outside the chunked family needs float16 tokens")
        a = torch.empty_like(k)
        b = torch.empty_like(k)
        with _on_device(state.device):
            N.check(N.load().fr2_tmix_kk_a_gate_forward(
                r.size(0), h, d, k.data_ptr(), k_k.data_ptr(), a0.data_ptr(), a12.data_ptr(),
                k_a.data_ptr(), new_k.data_ptr(), a.data_ptr(), b.data_ptr(),
                _stream(state.device)), "fr2_tmix_kk_a_gate_forward")
        _recurrent_launch(None, query_start_loc, state_indices, state, r, decay_logits, new_k,
                          v, a, b, output, scale, decay_bias, validated_metadata, max_seqlen)
        del keep
        return
    N.check(rc, "tmix_wkv7_recurrent_fp32_from_kk_gate")
    del keep


def tmix_wkv7_recurrent_fp32_from_kk_gate_readout(query_start_loc, state_indices, state, r,
                                                  decay_logits, k, v, a12, g, k_k, a0, k_a, r_k,
                                                  ln_weight, ln_bias, new_k, readout, output,
                                                  scale, decay_bias=None,
                                                  validated_metadata=None, max_seqlen=-1):
    """tmix_wkv7_recurrent_fp32_from_kk_gate with the readout's elementwise
    stage in the output write-back: readout = (GroupNorm(y) ln_weight + ln_bias
    + (sum r k' r_k) v) g per (token, head); `output` (y) may be None.  Where
    the fused kernel does not apply (as for the kk-gate entry) the stages run
    as separate kernels (fp16 tokens)."""
    # the layout check's output slot takes y when given, else the readout
    # (same shape and dtype)
    n, h, d = check_recurrent_layout(query_start_loc, state_indices, state, r, decay_logits, k,
                                     v, a12, new_k, output if output is not None else readout,
                                     scale)
    for t, name in ((g, "g"), (readout, "readout")):
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
        _check(t.dtype == r.dtype and t.shape == r.shape, name,
               " must have the shape and dtype of the token tensors")
    for t, name in ((k_k, "k_k"), (a0, "a0"), (k_a, "k_a"), (r_k, "r_k"),
                    (ln_weight, "ln_weight"), (ln_bias, "ln_bias")):
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
        _check(t.dtype == r.dtype, name, " must have the token dtype")
        _check(t.numel() == h * d, name, " must have shape [H*D] or [H,D]")
    if decay_bias is not None:
        _check_decay_bias(decay_bias, state, r, h, d,
                          "decay_bias must match the token tensor dtype")
    lq, ls, status, ms, keep = _resolve_launch_metadata(
        query_start_loc, state_indices, r.size(0), state.size(0), int(max_seqlen),
        validated_metadata)
    fp16 = r.dtype == torch.float16
    rc = N.FR2_ERR_UNSUPPORTED
    if not (fp16 and d == 64 and int(ms) > 0 and split_plan(n, h, d, int(ms))[0] > 1):
        with _on_device(state.device):
            rc = N.load().fr2_wkv7_recurrent_fp32_forward_kk_gate_readout(
                lq.data_ptr(), ls.data_ptr(), status.data_ptr(), n, h, d, r.size(0), int(ms),
                _dtype_code(r), state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(),
                N.ptr(decay_bias), k.data_ptr(), v.data_ptr(), a12.data_ptr(), k_k.data_ptr(),
                a0.data_ptr(), k_a.data_ptr(), g.data_ptr(), r_k.data_ptr(),
                ln_weight.data_ptr(), ln_bias.data_ptr(), new_k.data_ptr(), readout.data_ptr(),
                N.ptr(output), float(scale), _stream(state.device))
    if rc == N.FR2_ERR_UNSUPPORTED:
        _check(fp16, "the fused readout outside the chunked family needs float16 tokens")
        y = output if output is not None else torch.empty_like(v)
        tmix_wkv7_recurrent_fp32_from_kk_gate(
            query_start_loc, state_indices, state, r, decay_logits, k, v, a12, k_k, a0, k_a,
            new_k, y, scale, decay_bias, validated_metadata, max_seqlen)
        with _on_device(state.device):
            N.check(N.load().fr2_tmix_readout_prelinear_forward(
                r.size(0), h, d, y.data_ptr(), r.data_ptr(), new_k.data_ptr(), v.data_ptr(),
                r_k.data_ptr(), ln_weight.data_ptr(), ln_bias.data_ptr(), g.data_ptr(),
                readout.data_ptr(), _stream(state.device)), "fr2_tmix_readout_prelinear_forward")
        del keep
        return
    N.check(rc, "tmix_wkv7_recurrent_fp32_from_kk_gate_readout")
    del keep


@functools.lru_cache(maxsize=256)
def _library_split_plan(num_sequences: int, num_heads: int, head_size: int,
                        max_seqlen: int) -> tuple[int, int, int, int]:
    lib = N.load()
    pc, pl, ll, wb = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    N.check(lib.fr2_wkv7_recurrent_fp32_split_plan(num_sequences, num_heads, head_size,
                                                   max_seqlen, ctypes.byref(pc),
                                                   ctypes.byref(pl), ctypes.byref(ll),
                                                   ctypes.byref(wb)),
            "fr2_wkv7_recurrent_fp32_split_plan")
    return pc.value, pl.value, ll.value, wb.value


_FAMILY_KERNELS = {
    N.KERNEL_SERIAL: "serial64w_kernel<{io},StF32>",
    N.KERNEL_DECODE: "decode64_kernel<{io},StF32>",
    N.KERNEL_CHUNKED: "chunk64r_kernel<{io}>",
    N.KERNEL_CHUNKED_WAVE: "chunk64w_kernel<{io},false>",
    5: "chunk64w_kernel<{io},true>",
}


def dispatch_kernel_name(num_sequences: int, num_heads: int, head_size: int,
                         total_tokens: int, max_seqlen: int, dtype=torch.bfloat16) -> str:
    """Name of the kernel the public fp32-state call runs for this shape: the
    sequence split when the library's plan cuts the sequences, otherwise the
    family fr2_wkv7_recurrent_fp32_dispatch reports (the library's own
    policy, not a restatement of it)."""
    if split_plan(num_sequences, num_heads, head_size, max_seqlen)[0] > 1:
        return "split:lead+summary+combine+pieces"
    lib = N.load()
    fam = ctypes.c_int32()
    N.check(lib.fr2_wkv7_recurrent_fp32_dispatch(int(num_sequences), int(num_heads),
                                                 int(head_size), int(total_tokens),
                                                 int(max_seqlen), ctypes.byref(fam)),
            "fr2_wkv7_recurrent_fp32_dispatch")
    io = "IoBF16" if dtype == torch.bfloat16 else "IoF16"
    name = _FAMILY_KERNELS[fam.value].format(io=io)
    if fam.value == N.KERNEL_SERIAL and head_size != 64:
        name = f"serial_kernel<{head_size},{io},StF32>"
    return name


def split_plan(num_sequences: int, num_heads: int, head_size: int, max_seqlen: int,
               pieces=None) -> tuple[int, int, int, int]:
    """(pieces, piece_len, lead_len, workspace_bytes) of the chunked prefill's
    sequence split: the library's plan (the pipelined split), or, for tests,
    `pieces` equal pieces of the classic split (lead_len 0) or, with
    `pieces=(P, lead_len)`, P pieces of the pipelined split whose piece 0 has
    lead_len tokens."""
    if pieces is None:
        return _library_split_plan(int(num_sequences), int(num_heads), int(head_size),
                                   int(max_seqlen))
    lead = 0
    if isinstance(pieces, tuple):
        pieces, lead = pieces
    if head_size != 64 or pieces < 2:
        return 1, max_seqlen, 0, 0
    if lead > 0:
        plen = -(-max(max_seqlen - lead, 1) // (pieces - 1))
    else:
        plen = -(-max(max_seqlen, 1) // pieces)
    plen = -(-plen // 32) * 32
    ws = num_sequences * (3 * pieces - 2) * num_heads * 64 * 64 * 4
    return pieces, plen, lead, ws
    # Implicit validation buffers (`keep`) are released after the launch; the
    # caching allocator only hands them out again to work queued later on this
    # same stream, which runs after the kernels that read them.
    del keep


def _recurrent_fp32_fast(query_start_loc, state_indices, state, r, decay_logits, k, v, a, b,
                         scale, ticket, max_seqlen):
    """The ticketed recurrence without decay bias through the native fast path
    (hostpath.cpp): the output, or None when the call is not plainly valid
    there or needs the sequence split (the caller then runs the full path,
    which raises or launches)."""
    facts = getattr(ticket, "_facts", None)
    if facts is None:
        return None
    try:
        res = N.hostpath().recurrent_fp32(facts, query_start_loc, state_indices, state, r,
                                          decay_logits, k, v, a, b, scale, max_seqlen,
                                          _raw_stream(ticket._device.index))
    except (TypeError, RuntimeError):
        return None
    if isinstance(res, int):
        N.check(res, "tmix_wkv7_recurrent_fp32_from_decay_logits")
    return res


def tmix_wkv7_recurrent_fp32_from_decay_logits(query_start_loc, state_indices, state, r,
                                               decay_logits, k, v, a, b, output, scale,
                                               decay_bias=None, validated_metadata=None,
                                               max_seqlen=-1):
    """In-place fp32-state packed recurrence (…fp32io16_forward_varlen.cpp:330-387)."""
    _recurrent_launch(None, query_start_loc, state_indices, state, r, decay_logits, k, v,
                      a, b, output, scale, decay_bias, validated_metadata, max_seqlen)


def tmix_wkv7_recurrent_fp32_kernel_forced(kernel, query_start_loc, state_indices, state, r,
                                           decay_logits, k, v, a, b, output, scale,
                                           decay_bias=None, validated_metadata=None,
                                           max_seqlen=-1, split_pieces=None):
    """Same contract with the kernel family forced (0 serial, 1 decode,
    2 chunked MFMA, 3 chunked with the sequence split, `split_pieces` pieces
    or the library's plan).  No reference counterpart: used to pin each
    kernel."""
    _recurrent_launch(int(kernel), query_start_loc, state_indices, state, r, decay_logits,
                      k, v, a, b, output, scale, decay_bias, validated_metadata, max_seqlen,
                      split_pieces)


# ---------------------------------------------------------------------------
# FP16-state ("Albatross") packed recurrence
# ---------------------------------------------------------------------------
def _check_fp16_recurrent_layout(qsl, slots, elapsed, state, r, decay_logits, k, v, a, b,
                                 output, scale):
    """check_fp16_recurrent_layout, infer_recurrent_fp16_forward_varlen.cpp:49-120."""
    for t, name in ((qsl, "query_start_loc"), (slots, "state_indices"),
                    (elapsed, "elapsed_state_pool"), (state, "state"), (r, "r"),
                    (decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
                    (output, "output")):
        check_cuda_contiguous(t, name)
    for t, name in ((qsl, "query_start_loc"), (slots, "state_indices"),
                    (elapsed, "elapsed_state_pool"), (r, "r"), (decay_logits, "decay_logits"),
                    (k, "k"), (v, "v"), (a, "a"), (b, "b"), (output, "output")):
        check_same_device(state, t, name)
    _check(qsl.dtype == torch.int32 and slots.dtype == torch.int32
           and elapsed.dtype == torch.int32, "recurrent metadata must be int32")
    n = slots.numel()
    _check(slots.dim() == 1 and n > 0 and qsl.dim() == 1 and qsl.numel() == n + 1,
           "query_start_loc must have shape [B+1] and state_indices shape [B]")
    _check(n <= 65535, "state_indices must contain 1..65535 sequences")
    _check(elapsed.dim() == 1 and elapsed.size(0) == state.size(0),
           "elapsed_state_pool must have shape [state_pool_slots]")
    _check(state.dim() == 4 and state.dtype == torch.float16 and state.size(0) > 0
           and state.size(1) > 0 and state.size(2) == state.size(3),
           "state must be contiguous float16 [slots,H,D,D]")
    h, d = state.size(1), state.size(2)
    _check(d in (64, 128, 256), "recurrent head size must be 64, 128, or 256, got ", d)
    _check(r.dim() == 3 and r.size(0) > 0 and r.size(1) == h and r.size(2) == d,
           "r must have packed shape [total_tokens,H,D] matching state")
    _check(r.size(0) <= INT32_MAX, "token count must fit in int32")
    _check(all(t.shape == r.shape for t in (decay_logits, k, v, a, b, output)),
           "r,decay_logits,k,v,a,b,output shape mismatch")
    _check(all(t.dtype == torch.float16 for t in (r, decay_logits, k, v, a, b, output)),
           "FP16-state recurrent token tensors must be float16")
    _check(math.isfinite(scale), "scale must be finite")
    return n, h, d


def tmix_wkv7_recurrent_fp16_from_decay_logits(query_start_loc, state_indices, elapsed_state,
                                               state, r, decay_logits, k, v, a, b, output,
                                               scale, decay_bias=None, validated_metadata=None,
                                               max_seqlen=-1):
    """In-place FP16-state packed recurrence, then the elapsed-count advance
    (infer_recurrent_fp16_forward_varlen.cpp:121-187)."""
    n, h, d = _check_fp16_recurrent_layout(query_start_loc, state_indices, elapsed_state,
                                           state, r, decay_logits, k, v, a, b, output, scale)
    if decay_bias is not None:
        check_cuda_contiguous(decay_bias, "decay_bias")
        check_same_device(state, decay_bias, "decay_bias")
        _check(decay_bias.dtype == torch.float16
               and ((decay_bias.dim() == 1 and decay_bias.numel() == h * d)
                    or (decay_bias.dim() == 2 and decay_bias.size(0) == h
                        and decay_bias.size(1) == d)),
               "decay_bias must be float16 with shape [H*D] or [H,D]")
    lq, ls, status, max_seqlen, keep = _resolve_launch_metadata(
        query_start_loc, state_indices, r.size(0), state.size(0), int(max_seqlen),
        validated_metadata)
    with _on_device(state.device):
        rc = N.load().fr2_wkv7_recurrent_fp16_forward(
            lq.data_ptr(), ls.data_ptr(), status.data_ptr(), elapsed_state.data_ptr(), n, h, d,
            r.size(0), int(max_seqlen), state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(),
            N.ptr(decay_bias), k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
            output.data_ptr(), float(scale), _stream(state.device))
    N.check(rc, "tmix_wkv7_recurrent_fp16_from_decay_logits")
    del keep


# ---------------------------------------------------------------------------
# pretrain [B,T,H,D] forward
# ---------------------------------------------------------------------------
def pretrain_tmix_wkv7_recurrent_forward(r, w, k, v, a, b, output, boundary, state_dot_a,
                                         head_size):
    """pretrain_recurrent_bf16_forward.cpp:20-27 (bf16 [B,T,H,N])."""
    _check(head_size in (64, 128, 256), "head_size must be one of 64, 128, or 256")
    _check(r.size(3) == head_size, "input head dimension must equal head_size")
    B, T, H, _ = r.shape
    for t, name in ((r, "r"), (w, "w"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
                    (output, "output"), (boundary, "boundary"), (state_dot_a, "state_dot_a")):
        check_cuda_contiguous(t, name)
    _check(all(t.dtype == torch.bfloat16 for t in (r, w, k, v, a, b, output)),
           "pretrain token tensors must be bfloat16")
    _check(all(t.shape == r.shape for t in (w, k, v, a, b, output)),
           "pretrain token tensors must share shape [B,T,H,N]")
    _check(T % 16 == 0, "T must be divisible by the canonical chunk length 16")
    _check(tuple(boundary.shape) == (B, H, T // 16, head_size, head_size)
           and boundary.dtype == torch.float32, "boundary must be float32 [B,H,T/16,N,N]")
    _check(state_dot_a.shape == r.shape and state_dot_a.dtype == torch.float32,
           "state_dot_a must be float32 [B,T,H,N]")
    with _on_device(r.device):
        rc = N.load().fr2_wkv7_pretrain_forward(
            B, T, H, head_size, r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(),
            a.data_ptr(), b.data_ptr(), output.data_ptr(), boundary.data_ptr(),
            state_dot_a.data_ptr(), _stream(r.device))
    N.check(rc, "pretrain_tmix_wkv7_recurrent_forward")


def pretrain_tmix_wkv7_recurrent_backward(r, w, k, v, a, b, grad_output, boundary,
                                          state_dot_a, grad_r, grad_w, grad_k, grad_v,
                                          grad_a, grad_b, head_size):
    """pretrain_recurrent_bf16_forward.cpp:29-46 (backward over bf16 [B,T,H,N]).

    Fills the six bf16 gradient tensors in place.  The fp32 workspace that
    carries d(sa) (and, at N=64, the value pass's gradient snapshots) between
    the passes is allocated here (the reference allocates a d(sa) buffer for
    its N=256 path).
    """
    _check(head_size in (64, 128, 256), "head_size must be one of 64, 128, or 256")
    _check(r.size(3) == head_size, "input head dimension must equal head_size")
    B, T, H, _ = r.shape
    tensors = ((r, "r"), (w, "w"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
               (grad_output, "grad_output"), (boundary, "boundary"),
               (state_dot_a, "state_dot_a"), (grad_r, "grad_r"), (grad_w, "grad_w"),
               (grad_k, "grad_k"), (grad_v, "grad_v"), (grad_a, "grad_a"), (grad_b, "grad_b"))
    for t, name in tensors:
        check_cuda_contiguous(t, name)
        check_same_device(r, t, name)
    bf16 = (r, w, k, v, a, b, grad_output, grad_r, grad_w, grad_k, grad_v, grad_a, grad_b)
    _check(all(t.dtype == torch.bfloat16 for t in bf16),
           "pretrain token tensors and gradients must be bfloat16")
    _check(all(t.shape == r.shape for t in bf16),
           "pretrain token tensors must share shape [B,T,H,N]")
    _check(T % 16 == 0, "T must be divisible by the canonical chunk length 16")
    _check(tuple(boundary.shape) == (B, H, T // 16, head_size, head_size)
           and boundary.dtype == torch.float32, "boundary must be float32 [B,H,T/16,N,N]")
    _check(state_dot_a.shape == r.shape and state_dot_a.dtype == torch.float32,
           "state_dot_a must be float32 [B,T,H,N]")
    nws = N.load().fr2_wkv7_pretrain_backward_workspace_floats(B, T, H, head_size)
    _check(nws > 0, "pretrain backward: unsupported shape")
    workspace = torch.empty(nws, device=r.device, dtype=torch.float32)
    with _on_device(r.device):
        rc = N.load().fr2_wkv7_pretrain_backward(
            B, T, H, head_size, r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(),
            a.data_ptr(), b.data_ptr(), grad_output.data_ptr(), boundary.data_ptr(),
            state_dot_a.data_ptr(), workspace.data_ptr(), grad_r.data_ptr(),
            grad_w.data_ptr(), grad_k.data_ptr(), grad_v.data_ptr(), grad_a.data_ptr(),
            grad_b.data_ptr(), _stream(r.device))
    N.check(rc, "pretrain_tmix_wkv7_recurrent_backward")


# ---------------------------------------------------------------------------
# StateTune (trainable initial state over a chunk list)
# ---------------------------------------------------------------------------
def _statetune_check(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state,
                     tokens):
    for t, name in ((sequence_chunk_offsets, "sequence_chunk_offsets"),
                    (chunk_token_starts, "chunk_token_starts"),
                    (chunk_token_ends, "chunk_token_ends"), (state, "state")):
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
    for t in (sequence_chunk_offsets, chunk_token_starts, chunk_token_ends):
        _check(t.dtype == torch.int32, "chunk metadata must be int32")
    _check(state.dtype == torch.float32 and state.dim() == 4
           and state.size(2) == state.size(3), "state must be float32 [B,H,D,D]")
    D = state.size(3)
    _check(D in (64, 128, 256), "head_size must be one of 64, 128, or 256")
    r = tokens[0][0]
    _check(r.dtype in _TOKEN_DTYPES, "token tensors must be float16 or bfloat16")
    for t, name in tokens:
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
        _check(t.dtype == r.dtype, name, " must have the dtype of r")
        _check(t.shape == r.shape, name, " must match r shape")
    _check(r.dim() == 3 and r.size(1) == state.size(1) and r.size(2) == D,
           "token tensors must have shape [total_tokens,H,D]")
    _check(sequence_chunk_offsets.numel() == state.size(0) + 1,
           "sequence_chunk_offsets must have shape [B+1]")
    _check(chunk_token_starts.numel() > 0
           and chunk_token_ends.numel() == chunk_token_starts.numel(),
           "chunk token metadata must have matching shape [C]")
    return state.size(0), chunk_token_starts.numel(), r.size(0), state.size(1), D


def _statetune_uniform_chunk_len(offsets, starts, ends, B, C, T, D, dtype):
    """The chunk length when the chunk list is B sequences of equal length
    packed back to back, each cut into equal chunks of a multiple of 16
    tokens (D = 64, bf16): the layout the chunked MFMA kernels take.
    Reads the (small) chunk metadata on the host."""
    if D != 64 or dtype != torch.bfloat16 or C % B or T % B:
        return None
    nck, per_seq = C // B, T // B
    if per_seq % nck or (per_seq // nck) % 16:
        return None
    length = per_seq // nck
    dev = starts.device
    want = torch.arange(C + 1, dtype=torch.int32, device=dev) * length
    ok = (torch.equal(offsets, torch.arange(B + 1, dtype=torch.int32, device=dev) * nck)
          and torch.equal(starts, want[:-1]) and torch.equal(ends, want[1:]))
    return length if ok else None


# tests set this to run every non-uniform chunk list token-serial
_statetune_force_serial = False


def statetune_tmix_wkv7_recurrent_fp32io16_forward(sequence_chunk_offsets, chunk_token_starts,
                                                   chunk_token_ends, state, r, decay_logits,
                                                   k, v, a, b, output, boundary, state_dot_a,
                                                   scale=1.0):
    """statetune_recurrent_fp32io16_forward.cpp:26-56: runs every sequence's
    chunks from ``state`` (updated in place to the final state) and fills
    ``output``, ``boundary`` (start-of-chunk states) and ``state_dot_a``.

    When the chunk list is the uniform layout (D = 64, bf16, equal sequences
    packed back to back, equal chunks of a multiple of 16 tokens) it runs on
    the chunked MFMA kernels and returns the fp32 post-16-token state
    snapshots ``[B,H,T/16,64,64]`` that the fast backward takes.  Any other
    chunk list at D = 64 in bf16 runs on the same kernels over a padded grid
    (_statetune_padded_plan) and returns (snapshots, row_source,
    seq_first_chunk) for the backward.  Otherwise (fp16, D = 128 / 256, or a
    list the grid does not suit) it runs token-serial and returns None (the
    reference returns None)."""
    B, C, T, H, D = _statetune_check(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state,
        ((r, "r"), (decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
         (output, "output")))
    check_cuda_contiguous(boundary, "boundary")
    check_cuda_contiguous(state_dot_a, "state_dot_a")
    _check(boundary.dtype == torch.float32 and tuple(boundary.shape) == (C, H, D, D),
           "boundary must be float32 [C,H,D,D]")
    _check(state_dot_a.dtype == torch.float32 and state_dot_a.shape == r.shape,
           "state_dot_a must be float32 [total_tokens,H,D]")
    length = _statetune_uniform_chunk_len(sequence_chunk_offsets, chunk_token_starts,
                                          chunk_token_ends, B, C, T, D, r.dtype)
    plan = None if (length is not None or _statetune_force_serial) else _statetune_padded_plan(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, B, C, T, D, r.dtype)
    if plan is not None:
        Tp, row_source, chunk_seq, pstart, first = plan
        dev = state.device
        tables = [torch.from_numpy(x).to(dev) for x in (row_source, chunk_seq, pstart, first)]
        snapshots = torch.empty((B, H, Tp // 16, D, D), device=dev, dtype=torch.float32)
        lib = N.load()
        nbytes = lib.fr2_wkv7_statetune_padded_workspace_bytes(B, Tp, H, 0)
        _check(nbytes > 0, "statetune forward: unsupported shape")
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        with _on_device(dev):
            rc = lib.fr2_wkv7_statetune_padded_forward(
                B, Tp, H, C, tables[0].data_ptr(), tables[1].data_ptr(), tables[2].data_ptr(),
                state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(), k.data_ptr(),
                v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(), boundary.data_ptr(),
                state_dot_a.data_ptr(), snapshots.data_ptr(), ws.data_ptr(), float(scale),
                _stream(dev))
        N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_forward")
        del ws
        # what the backward needs: the snapshots and the grid tables
        return snapshots, tables[0], tables[3]
    with _on_device(state.device):
        if length is not None:
            per_seq = T // B
            snapshots = torch.empty((B, H, per_seq // 16, D, D), device=state.device,
                                    dtype=torch.float32)
            rc = N.load().fr2_wkv7_statetune_uniform_forward(
                B, per_seq, H, length, state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(),
                k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(),
                boundary.data_ptr(), state_dot_a.data_ptr(), snapshots.data_ptr(), float(scale),
                _stream(state.device))
            N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_forward")
            return snapshots
        rc = N.load().fr2_wkv7_statetune_forward(
            sequence_chunk_offsets.data_ptr(), chunk_token_starts.data_ptr(),
            chunk_token_ends.data_ptr(), B, C, T, H, D, _dtype_code(r), state.data_ptr(),
            r.data_ptr(), decay_logits.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(),
            b.data_ptr(), output.data_ptr(), boundary.data_ptr(), state_dot_a.data_ptr(),
            float(scale), _stream(state.device))
    N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_forward")
    return None


def statetune_tmix_wkv7_recurrent_fp32io16_backward(sequence_chunk_offsets, chunk_token_starts,
                                                    chunk_token_ends, final_state, r,
                                                    decay_logits, k, v, a, b, state_dot_a,
                                                    grad_output, grad_final_state, boundary,
                                                    grad_r, grad_decay_logits, grad_k, grad_v,
                                                    grad_a, grad_b, grad_initial_state,
                                                    scale=1.0, snapshots=None):
    """statetune_recurrent_fp32io16_backward.cpp:34-82: fills the six token
    gradients and ``grad_initial_state`` in place.  ``grad_output`` and
    ``grad_final_state`` may be None (zero).  ``final_state`` is checked but
    not read: chunk-end states are rebuilt from ``boundary``.  The fp32
    workspace (d(sa) per token and the replayed in-chunk states) is
    allocated here.  ``snapshots`` (not in the reference) is what the
    forward returned on the uniform layout: with it and a ``grad_output``
    the backward runs on the chunked MFMA kernels."""
    grads = ((grad_r, "grad_r"), (grad_decay_logits, "grad_decay_logits"), (grad_k, "grad_k"),
             (grad_v, "grad_v"), (grad_a, "grad_a"), (grad_b, "grad_b"))
    toks = [(r, "r"), (decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
            *grads]
    if grad_output is not None:
        toks.append((grad_output, "grad_output"))
    B, C, T, H, D = _statetune_check(sequence_chunk_offsets, chunk_token_starts,
                                     chunk_token_ends, final_state, tuple(toks))
    for t, name in ((boundary, "boundary"), (state_dot_a, "state_dot_a"),
                    (grad_initial_state, "grad_initial_state")):
        check_cuda_contiguous(t, name)
        check_same_device(final_state, t, name)
    _check(boundary.dtype == torch.float32 and tuple(boundary.shape) == (C, H, D, D),
           "boundary must be float32 [C,H,D,D]")
    _check(state_dot_a.dtype == torch.float32 and state_dot_a.shape == r.shape,
           "state_dot_a must be float32 [total_tokens,H,D]")
    _check(grad_initial_state.dtype == torch.float32
           and grad_initial_state.shape == final_state.shape,
           "grad_initial_state must be float32 [B,H,D,D]")
    if grad_final_state is not None:
        check_cuda_contiguous(grad_final_state, "grad_final_state")
        _check(grad_final_state.dtype == torch.float32
               and grad_final_state.shape == final_state.shape,
               "grad_final_state must be float32 [B,H,D,D]")
    ptr = lambda t: None if t is None else t.data_ptr()
    if isinstance(snapshots, tuple):
        # the padded layout of a ragged chunk list (what the forward returned)
        snaps, row_source, first = snapshots
        Tp = row_source.numel() // B
        _check(D == 64 and r.dtype == torch.bfloat16 and Tp * B == row_source.numel()
               and Tp % 16 == 0 and tuple(snaps.shape) == (B, H, Tp // 16, D, D)
               and first.numel() == B, "snapshots do not match the padded chunk layout")
        if grad_output is None:
            grad_output = torch.zeros_like(r)
        lib = N.load()
        nbytes = lib.fr2_wkv7_statetune_padded_workspace_bytes(B, Tp, H, 1)
        _check(nbytes > 0, "statetune backward: unsupported shape")
        ws = torch.empty(nbytes, device=r.device, dtype=torch.uint8)
        with _on_device(final_state.device):
            rc = lib.fr2_wkv7_statetune_padded_backward(
                B, Tp, H, row_source.data_ptr(), first.data_ptr(), r.data_ptr(),
                decay_logits.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
                state_dot_a.data_ptr(), grad_output.data_ptr(), ptr(grad_final_state),
                boundary.data_ptr(), snaps.data_ptr(), ws.data_ptr(),
                *(g.data_ptr() for g, _ in grads), grad_initial_state.data_ptr(), float(scale),
                _stream(final_state.device))
        N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_backward")
        return
    if snapshots is not None and grad_output is not None:
        per_seq = T // B
        _check(T % B == 0 and C % B == 0 and T % C == 0,
               "snapshots are only for the uniform chunk layout")
        length = T // C
        check_cuda_contiguous(snapshots, "snapshots")
        _check(snapshots.dtype == torch.float32
               and tuple(snapshots.shape) == (B, H, per_seq // 16, D, D)
               and D == 64 and r.dtype == torch.bfloat16 and length % 16 == 0
               and per_seq % length == 0, "snapshots do not match the uniform chunk layout")
        nws = N.load().fr2_wkv7_statetune_uniform_backward_workspace_floats(B, per_seq, H)
        _check(nws > 0, "statetune backward: unsupported shape")
        workspace = torch.empty(nws, device=r.device, dtype=torch.float32)
        with _on_device(final_state.device):
            rc = N.load().fr2_wkv7_statetune_uniform_backward(
                B, per_seq, H, length, r.data_ptr(), decay_logits.data_ptr(), k.data_ptr(),
                v.data_ptr(), a.data_ptr(), b.data_ptr(), state_dot_a.data_ptr(),
                grad_output.data_ptr(), ptr(grad_final_state), boundary.data_ptr(),
                snapshots.data_ptr(), workspace.data_ptr(), *(g.data_ptr() for g, _ in grads),
                grad_initial_state.data_ptr(), float(scale), _stream(final_state.device))
        N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_backward")
        return
    nws = N.load().fr2_wkv7_statetune_backward_workspace_floats(T, H, D)
    _check(nws > 0, "statetune backward: unsupported shape")
    workspace = torch.empty(nws, device=r.device, dtype=torch.float32)
    with _on_device(final_state.device):
        rc = N.load().fr2_wkv7_statetune_backward(
            sequence_chunk_offsets.data_ptr(), chunk_token_starts.data_ptr(),
            chunk_token_ends.data_ptr(), B, C, T, H, D, _dtype_code(r), r.data_ptr(),
            decay_logits.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
            state_dot_a.data_ptr(), ptr(grad_output), ptr(grad_final_state), boundary.data_ptr(),
            workspace.data_ptr(), *(g.data_ptr() for g, _ in grads),
            grad_initial_state.data_ptr(), float(scale), _stream(final_state.device))
    N.check(rc, "statetune_tmix_wkv7_recurrent_fp32io16_backward")


# ---------------------------------------------------------------------------
# bf16-state packed chunk inference
# ---------------------------------------------------------------------------
def _check_bf16(t, ref, name):
    check_cuda_contiguous(t, name)
    check_same_device(ref, t, name)
    _check(t.dtype == torch.bfloat16, name, " must be bf16")


# pieces of the bf16-state chunk entry's sequence split: None = the library's
# plan; tests set a count to force the split on small cases
_chunk_split_pieces = None


def infer_tmix_wkv7_chunk_bf16_forward_varlen(r, decay_logits, k, v, a, b, state_pool,
                                              cu_seqlens, state_indices, chunk_size=16,
                                              max_seqlen=-1, scale=1.0, decay_bias=None,
                                              validated_metadata=None):
    """bf16 state pool updated in place (infer_chunk_bf16_forward_varlen.cpp:77-192)."""
    _check_bf16(r, r, "r")
    for t, name in ((decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"),
                    (b, "b"), (state_pool, "state_pool")):
        _check_bf16(t, r, name)
    _check(math.isfinite(scale), "scale must be finite")
    _check(chunk_size > 0, "chunk_size must be positive")
    _check(max_seqlen > 0, "max_seqlen must be positive")
    _check(r.dim() == 3 and r.size(0) > 0 and r.size(1) > 0 and r.size(2) == 64,
           "chunk token tensors must have shape [total_tokens,H,64]")
    for t, name in ((decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"), (b, "b")):
        _check(t.shape == r.shape, name, " must have the same shape as r")
    _check(state_pool.dim() == 4 and state_pool.size(0) > 0
           and state_pool.size(1) == r.size(1) and state_pool.size(2) == 64
           and state_pool.size(3) == 64, "state_pool must have shape [slots,H,64,64]")
    check_cuda_contiguous(cu_seqlens, "cu_seqlens")
    check_cuda_contiguous(state_indices, "state_indices")
    check_same_device(r, cu_seqlens, "cu_seqlens")
    check_same_device(r, state_indices, "state_indices")
    _check(cu_seqlens.dtype == torch.int32 and state_indices.dtype == torch.int32,
           "chunk metadata must be int32")
    _check(cu_seqlens.dim() == 1 and state_indices.dim() == 1 and state_indices.numel() > 0
           and cu_seqlens.numel() == state_indices.numel() + 1,
           "cu_seqlens must have shape [B+1] and state_indices [B]")
    h = r.size(1)
    if decay_bias is not None:
        _check_bf16(decay_bias, r, "decay_bias")
        _check((decay_bias.dim() == 1 and decay_bias.numel() == h * 64)
               or (decay_bias.dim() == 2 and decay_bias.size(0) == h
                   and decay_bias.size(1) == 64),
               "decay_bias must have shape [H*64] or [H,64]")
    output = torch.empty_like(v)
    lq, ls, status, max_seqlen, keep = _resolve_launch_metadata(
        cu_seqlens, state_indices, r.size(0), state_pool.size(0), int(max_seqlen),
        validated_metadata)
    args = (lq.data_ptr(), ls.data_ptr(), status.data_ptr(), state_indices.numel(), h,
            r.size(0), int(chunk_size), int(max_seqlen), state_pool.data_ptr(),
            r.data_ptr(), decay_logits.data_ptr(), N.ptr(decay_bias), k.data_ptr(),
            v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(), float(scale))
    pieces, piece_len, lead_len, ws_bytes = split_plan(state_indices.numel(), h, 64,
                                                       int(max_seqlen), _chunk_split_pieces)
    with _on_device(r.device):
        if pieces > 1:
            # few long sequences: the sequence split (workspace on this stream)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=r.device)
            aux = _aux_stream(r.device) if lead_len > 0 else None
            rc = N.load().fr2_wkv7_chunk_bf16_forward_split(*args, pieces, piece_len, lead_len,
                                                            ws.data_ptr(), ws_bytes,
                                                            _stream(r.device), aux)
            del ws
        else:
            rc = N.load().fr2_wkv7_chunk_bf16_forward(*args, _stream(r.device))
    N.check(rc, "infer_tmix_wkv7_chunk_bf16_forward_varlen")
    del keep
    return output, state_pool


# ---------------------------------------------------------------------------
# RL/Infctx fp32-state chunk forward and replay
# ---------------------------------------------------------------------------
def _check_chunk_metadata(sco, starts, ends, num_sequences, total_tokens, state):
    """rl_infctx_chunk_fp32io16_forward.cpp:73-132 (host copy of the metadata)."""
    for t, name in ((sco, "sequence_chunk_offsets"), (starts, "chunk_token_starts"),
                    (ends, "chunk_token_ends")):
        check_cuda_contiguous(t, name)
        check_same_device(state, t, name)
        _check(t.dtype == torch.int32, name, " must be int32")
    _check(sco.dim() == 1 and sco.numel() == num_sequences + 1,
           "sequence_chunk_offsets must have shape [B+1]")
    _check(starts.dim() == 1 and starts.numel() > 0 and starts.shape == ends.shape,
           "chunk token metadata must have matching shape [C]")
    _check(starts.numel() * state.size(1) <= INT32_MAX, "chunk/head grid must fit in int32")
    seq = sco.to("cpu").tolist()
    st = starts.to("cpu").tolist()
    en = ends.to("cpu").tolist()
    chunks = len(st)
    _check(seq[0] == 0 and seq[num_sequences] == chunks,
           "sequence_chunk_offsets must cover all chunks")
    prev_end = 0
    longest = 0
    longest_chunk = 0
    for i in range(num_sequences):
        c0, c1 = seq[i], seq[i + 1]
        _check(c0 >= 0 and c1 > c0 and c1 <= chunks,
               "each sequence must own at least one ordered chunk")
        _check(st[c0] == prev_end, "chunks must cover packed tokens without gaps")
        for c in range(c0, c1):
            _check(st[c] >= 0 and en[c] > st[c] and en[c] <= total_tokens
                   and (c == c0 or st[c] == en[c - 1]),
                   "chunk token ranges must be contiguous and non-empty")
            longest_chunk = max(longest_chunk, en[c] - st[c])
        prev_end = en[c1 - 1]
        longest = max(longest, en[c1 - 1] - st[c0])
    _check(prev_end == total_tokens, "chunks must cover exactly all packed tokens")
    return longest, longest_chunk


def rl_infctx_tmix_wkv7_chunk_fp32io16_forward(sequence_chunk_offsets, chunk_token_starts,
                                               chunk_token_ends, state, r, decay_logits, k,
                                               v, a, b, strategy=1, scale=1.0,
                                               decay_bias=None):
    """Returns (output, final_state); `state` itself is not modified
    (rl_infctx_chunk_fp32io16_forward.cpp:158-230)."""
    _check(strategy in (0, 1), "strategy must be 0 (materialized) or 1 (recompute)")
    _check(isinstance(state, torch.Tensor) and state.is_cuda and state.is_contiguous()
           and state.dtype == torch.float32, "RL/Infctx state must be contiguous CUDA float32")
    _check(state.dim() == 4 and state.size(0) > 0 and state.size(1) > 0
           and state.size(2) == state.size(3) and state.size(2) in (64, 128, 256),
           "RL/Infctx state must have shape [B,H,D,D], D in {64,128,256}")
    working = state.clone()
    output = torch.empty_like(v)
    internal_slots = torch.arange(state.size(0), device=state.device, dtype=torch.int32)
    n, h, d = check_recurrent_layout(sequence_chunk_offsets, internal_slots, working, r,
                                     decay_logits, k, v, a, b, output, scale)
    longest, longest_chunk = _check_chunk_metadata(sequence_chunk_offsets, chunk_token_starts,
                                    chunk_token_ends, state.size(0), r.size(0), working)
    if decay_bias is not None:
        _check_decay_bias(decay_bias, working, r, h, d, "decay_bias must match token dtype")
    # The native contract carries no chunk size; the chunk family that the
    # metadata describes is the smallest of 16/32/64 holding every chunk.
    _check(longest_chunk <= 64, "chunk token ranges must not exceed 64 tokens")
    chunk_size = 16 if longest_chunk <= 16 else (32 if longest_chunk <= 32 else 64)
    with _on_device(r.device):
        rc = N.load().fr2_wkv7_rl_infctx_forward(
            sequence_chunk_offsets.data_ptr(), chunk_token_starts.data_ptr(),
            chunk_token_ends.data_ptr(), n, chunk_token_starts.numel(), h, d, r.size(0),
            int(longest), chunk_size, int(strategy), _dtype_code(r), working.data_ptr(),
            r.data_ptr(), decay_logits.data_ptr(), N.ptr(decay_bias), k.data_ptr(),
            v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(), float(scale),
            _stream(r.device))
    N.check(rc, "rl_infctx_tmix_wkv7_chunk_fp32io16_forward")
    return output, working


def rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay(chunk_token_starts, chunk_token_ends,
                                                       boundary, r, decay_logits, k, v, a, b,
                                                       output, state_dot_a, scale=1.0,
                                                       decay_bias=None):
    """Replay of each chunk from its start-of-chunk state
    (rl_infctx_chunk_fp32io16_backward.cpp:22-125)."""
    for t, name in ((boundary, "boundary"), (r, "r"), (decay_logits, "decay_logits"),
                    (k, "k"), (v, "v"), (a, "a"), (b, "b"), (output, "output"),
                    (state_dot_a, "state_dot_a"), (chunk_token_starts, "chunk_token_starts"),
                    (chunk_token_ends, "chunk_token_ends")):
        check_cuda_contiguous(t, name)
    _check(math.isfinite(scale), "scale must be finite")
    _check(chunk_token_starts.dtype == torch.int32 and chunk_token_ends.dtype == torch.int32,
           "chunk token metadata must be int32")
    _check(chunk_token_starts.dim() == 1 and chunk_token_starts.numel() > 0
           and chunk_token_starts.shape == chunk_token_ends.shape,
           "chunk token metadata must have shape [C]")
    _check(boundary.dim() == 4 and boundary.size(0) == chunk_token_starts.numel()
           and boundary.size(1) == r.size(1) and boundary.size(2) == r.size(2)
           and boundary.size(3) == r.size(2) and boundary.dtype == torch.float32,
           "boundary must have shape [C,H,D,D] and be float32")
    _check(r.dim() == 3 and r.size(0) > 0 and r.size(2) in (64, 128, 256),
           "replay token tensors must have shape [N,H,D], D in {64,128,256}")
    for t, name in ((decay_logits, "decay_logits"), (k, "k"), (v, "v"), (a, "a"), (b, "b"),
                    (output, "output")):
        _check(t.shape == r.shape, name, " must match r shape")
        _check(t.dtype == r.dtype, name, " must match r dtype")
        check_same_device(r, t, name)
    _check(r.dtype in _TOKEN_DTYPES, "replay token tensors must be float16 or bfloat16")
    _check(state_dot_a.shape == r.shape and state_dot_a.dtype == torch.float32,
           "state_dot_a must match r shape and be float32")
    for t in (chunk_token_starts, chunk_token_ends, boundary, state_dot_a):
        check_same_device(r, t, "replay metadata/workspace")
    h, d = r.size(1), r.size(2)
    if decay_bias is not None:
        check_cuda_contiguous(decay_bias, "decay_bias")
        check_same_device(r, decay_bias, "decay_bias")
        _check(decay_bias.dtype == r.dtype, "decay_bias must match r dtype")
        _check((decay_bias.dim() == 1 and decay_bias.numel() == h * d)
               or (decay_bias.dim() == 2 and decay_bias.size(0) == h
                   and decay_bias.size(1) == d),
               "decay_bias must have shape [H*D] or [H,D]")
    # The replay kernels read chunk ranges on the device; the host only checks
    # them against the token count so that no launch can run out of bounds.
    st = chunk_token_starts.to("cpu").tolist()
    en = chunk_token_ends.to("cpu").tolist()
    _check(all(0 <= s < e <= r.size(0) for s, e in zip(st, en)),
           "chunk token ranges must be non-empty and within the packed tokens")
    with _on_device(r.device):
        rc = N.load().fr2_wkv7_rl_infctx_replay(
            chunk_token_starts.data_ptr(), chunk_token_ends.data_ptr(),
            chunk_token_starts.numel(), h, d, r.size(0), _dtype_code(r), boundary.data_ptr(),
            r.data_ptr(), decay_logits.data_ptr(), N.ptr(decay_bias), k.data_ptr(),
            v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(),
            state_dot_a.data_ptr(), float(scale), _stream(r.device))
    N.check(rc, "rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay")


# ---------------------------------------------------------------------------
# producer / consumer stages of the layer: wkv_prepare and readout (fp16)
# ---------------------------------------------------------------------------
# The dense and low-rank projections are plain library GEMMs (torch matmul on
# hipBLASLt, fp16 in, fp32 accumulate, fp16 out); every elementwise stage is
# one of this library's HIP kernels.

def _check_half(t, ref, name):
    _check(isinstance(t, torch.Tensor) and t.is_cuda, name, " must be CUDA")
    _check(t.is_contiguous(), name, " must be contiguous")
    _check(t.dtype == torch.float16, name, " must be float16")
    check_same_device(ref, t, name)


def _check_scale(scale, what):
    _check(math.isfinite(scale) and abs(scale) <= 3.4028234663852886e38,
           what, " must be finite and representable as float32")


def _project(x, weight, lora_a, lora_b, lora_scale):
    """wkv_prepare_project_internal, infer_fp16_forward_varlen.cpp:192-232."""
    _check(lora_a is None or lora_b is not None, "lora_a and lora_b must be provided together")
    _check(lora_b is None or lora_a is not None, "lora_a and lora_b must be provided together")
    _check_scale(lora_scale, "lora_scale")
    out = torch.matmul(x, weight.t())
    if lora_a is None:
        return out
    _check_half(lora_a, x, "lora_a")
    _check_half(lora_b, x, "lora_b")
    _check(lora_a.dim() == 2 and lora_a.size(0) > 0 and lora_a.size(1) == x.size(1),
           "lora_a must have shape [R,K]")
    _check(lora_a.size(0) <= 512, "LoRA projection requires R<=512")
    _check(lora_b.dim() == 2 and lora_b.size(0) == weight.size(0)
           and lora_b.size(1) == lora_a.size(0), "lora_b must have shape [N,R]")
    if float(torch.tensor(lora_scale, dtype=torch.float32)) == 0.0:
        return out
    return torch.addmm(out, torch.matmul(x, lora_a.t()), lora_b.t(), alpha=float(lora_scale))


def _rank_weights(x, runtime, original, rank_in):
    """check_rank_dispatch, infer_fp16_forward_varlen.cpp:104-150."""
    _check(runtime is not None or original is not None,
           "one of weight or weight_t must be provided")
    if runtime is not None:
        _check_half(runtime, x, "weight")
        _check(runtime.dim() == 2 and runtime.size(0) == x.size(1),
               "rank-in runtime weight must have shape [input,rank]" if rank_in
               else "rank-out runtime weight must have shape [rank,output]")
    if original is not None:
        _check_half(original, x, "weight_t")
        _check(original.dim() == 2 and original.size(1) == x.size(1),
               "rank-in original weight must have shape [rank,input]" if rank_in
               else "rank-out original weight must have shape [output,rank]")
    if runtime is not None and original is not None:
        r_rank = runtime.size(1) if rank_in else runtime.size(0)
        o_rank = original.size(0) if rank_in else original.size(1)
        _check(r_rank == o_rank, "weight and weight_t must describe the same rank projection")
    rank = ((runtime.size(1) if rank_in else runtime.size(0)) if runtime is not None
            else (original.size(0) if rank_in else original.size(1)))
    _check(rank <= 512, "low-rank projection requires R<=512")


def _rank_mm(x, runtime, original, rank_in):
    _rank_weights(x, runtime, original, rank_in)
    return torch.matmul(x, runtime) if runtime is not None else torch.matmul(x, original.t())


def _lowrank_activate(w1x, g1x):
    tw, sg = torch.empty_like(w1x), torch.empty_like(g1x)
    rc = N.load().fr2_tmix_lowrank_activate(w1x.numel(), w1x.data_ptr(), tw.data_ptr(),
                                            g1x.numel(), g1x.data_ptr(), sg.data_ptr(),
                                            _stream(w1x.device))
    N.check(rc, "fr2_tmix_lowrank_activate")
    return tw, sg


def tmix_wkv_prepare_forward_varlen(
        x_r, x_w, x_k, x_v, x_a, x_g, receptance_weight, key_weight, value_weight,
        w1_t, a1_t, g1_t, v1_t, w2_t, a2_t, g2_t, v2_t, v0, k_k, a0, k_a,
        v_first=None, w1=None, a1=None, g1=None, v1=None, w2=None, a2=None, g2=None, v2=None,
        receptance_lora_a=None, receptance_lora_b=None, receptance_lora_scale=1.0,
        key_lora_a=None, key_lora_b=None, key_lora_scale=1.0,
        value_lora_a=None, value_lora_b=None, value_lora_scale=1.0,
        head_size=64, batch_size=1, max_seqlen=1):
    """tmix_wkv_prepare_forward_varlen, infer_fp16_forward_varlen.cpp:421-530.

    Returns [receptance, decay logits, prepared key, value, a (= -kk),
    b (= kk * a gate), output gate, v_first], each [total_tokens, C] fp16.
    ``w1_t`` .. ``v2_t`` are the original ([rank,C] in, [C,rank] out)
    layouts, ``w1`` .. ``v2`` the runtime ([C,rank] in, [rank,C] out) ones.
    """
    for t, name in ((x_r, "x_r"), (x_w, "x_w"), (x_k, "x_k"), (x_v, "x_v"), (x_a, "x_a"),
                    (x_g, "x_g")):
        _check_half(t, x_r, name)
        _check(t.dim() == 2 and t.size(0) == x_r.size(0),
               name, " must have packed shape [total_tokens,features]")
        _check(t.shape == x_r.shape, name, " must match x_r's packed shape")
    _check(head_size in (64, 128, 256), "head_size must be one of 64, 128, or 256")
    T, C = x_r.shape
    _check(C % head_size == 0, "channels must be divisible by head_size")
    _check(batch_size > 0 and max_seqlen > 0, "batch_size and max_seqlen must be positive")
    for t, name in ((receptance_weight, "receptance_weight"), (key_weight, "key_weight"),
                    (value_weight, "value_weight")):
        _check_half(t, x_r, name)
        _check(t.dim() == 2 and t.size(0) == C and t.size(1) == C, name, " must have shape [C,C]")
    receptance = _project(x_r, receptance_weight, receptance_lora_a, receptance_lora_b,
                          receptance_lora_scale)
    key = _project(x_k, key_weight, key_lora_a, key_lora_b, key_lora_scale)
    value = _project(x_v, value_weight, value_lora_a, value_lora_b, value_lora_scale)
    w1x = _rank_mm(x_w, w1, w1_t, True)
    a1x = _rank_mm(x_a, a1, a1_t, True)
    g1x = _rank_mm(x_g, g1, g1_t, True)
    tw, sg = _lowrank_activate(w1x, g1x)
    decay = _rank_mm(tw, w2, w2_t, False)
    a12 = _rank_mm(a1x, a2, a2_t, False)
    gate = _rank_mm(sg, g2, g2_t, False)
    for t, name in ((decay, "w2"), (a12, "a2"), (gate, "g2")):
        _check(t.size(1) == C, name, " runtime layout must have shape [R,C]")
    if v_first is not None:
        _check_half(v_first, x_r, "v_first")
        _check(v_first.shape == value.shape, "v and v_first must have shape [total_tokens,C]")
        _check_half(v0, x_r, "v0")
        _check(v0.dim() == 1 and v0.size(0) == C, "v0 must have shape [C]")
        v12 = _rank_mm(_rank_mm(x_v, v1, v1_t, True), v2, v2_t, False)
        mixed = torch.empty_like(value)
        rc = N.load().fr2_tmix_vres_forward(T, C, value.data_ptr(), v_first.data_ptr(),
                                            v0.data_ptr(), v12.data_ptr(), mixed.data_ptr(),
                                            _stream(x_r.device))
        N.check(rc, "fr2_tmix_vres_forward")
        value = mixed
        returned_v_first = v_first
    else:
        # the first layer validates the value branch's layouts without running it
        _rank_weights(x_v, v1, v1_t, True)
        v_rank = v1.size(1) if v1 is not None else v1_t.size(0)
        _check(v2 is not None or v2_t is not None, "v2 requires an original or runtime layout")
        if v2_t is not None:
            _check_half(v2_t, x_r, "v2")
            _check(v2_t.dim() == 2 and v2_t.size(0) == C and v2_t.size(1) == v_rank,
                   "v2 original layout must have shape [C,R]")
        if v2 is not None:
            _check_half(v2, x_r, "v2")
            _check(v2.dim() == 2 and v2.size(0) == v_rank and v2.size(1) == C,
                   "v2 runtime layout must have shape [R,C]")
        returned_v_first = value
    for t, name in ((k_k, "k_k"), (a0, "a0"), (k_a, "k_a")):
        _check_half(t, x_r, name)
        _check(t.dim() == 1 and t.size(0) == C, name, " must have shape [C]")
    prepared_key, neg_kk, kka = (torch.empty_like(key) for _ in range(3))
    rc = N.load().fr2_tmix_kk_a_gate_forward(
        T, C // head_size, head_size, key.data_ptr(), k_k.data_ptr(), a0.data_ptr(),
        a12.data_ptr(), k_a.data_ptr(), prepared_key.data_ptr(), neg_kk.data_ptr(),
        kka.data_ptr(), _stream(x_r.device))
    N.check(rc, "fr2_tmix_kk_a_gate_forward")
    return [receptance, decay, prepared_key, value, neg_kk, kka, gate, returned_v_first]


def tmix_readout_forward_varlen(wkv_output, receptance, key, value, r_k, ln_weight, ln_bias,
                                gate, output_weight, output_lora_a=None, output_lora_b=None,
                                output_lora_scale=1.0, head_size=64, batch_size=1, max_seqlen=1):
    """tmix_readout_forward_varlen, csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cpp:88-140:
    the fused group-norm / r.k residual / gate stage (HIP) stored in fp16,
    then the output projection (+ LoRA) as a library GEMM."""
    x = wkv_output
    _check_half(x, x, "x")
    _check(head_size in (64, 128, 256), "head_size must be one of 64, 128, or 256")
    _check(x.dim() == 2 and x.size(0) > 0 and x.size(1) > 0 and x.size(1) % head_size == 0,
           "x must have packed shape [total_tokens,H*head_size]")
    _check(batch_size > 0, "batch_size must be positive")
    _check(max_seqlen > 0, "max_seqlen must be positive")
    T, C = x.shape
    for t, name in ((receptance, "r"), (key, "k"), (value, "v"), (gate, "g")):
        _check_half(t, x, name)
        _check(t.shape == x.shape, name, " must match x's packed shape")
    for t, name in ((r_k, "r_k"), (ln_weight, "weight"), (ln_bias, "bias")):
        _check_half(t, x, name)
        _check(t.dim() == 1 and t.size(0) == C, name, " must have shape [C]")
    pre = torch.empty_like(x)
    rc = N.load().fr2_tmix_readout_prelinear_forward(
        T, C // head_size, head_size, x.data_ptr(), receptance.data_ptr(), key.data_ptr(),
        value.data_ptr(), r_k.data_ptr(), ln_weight.data_ptr(), ln_bias.data_ptr(),
        gate.data_ptr(), pre.data_ptr(), _stream(x.device))
    N.check(rc, "fr2_tmix_readout_prelinear_forward")
    _check_half(output_weight, x, "output_weight")
    _check(output_weight.dim() == 2 and output_weight.size(0) == C and output_weight.size(1) == C,
           "output_weight must have shape [C,C]")
    _check((output_lora_a is None) == (output_lora_b is None),
           "output_lora_a and output_lora_b must be provided together")
    _check_scale(output_lora_scale, "output_lora_scale")
    out = torch.matmul(pre, output_weight.t())
    if output_lora_a is None:
        return out
    _check_half(output_lora_a, x, "output_lora_a")
    _check_half(output_lora_b, x, "output_lora_b")
    _check(output_lora_a.dim() == 2 and output_lora_a.size(1) == C,
           "output_lora_a must have shape [R,C]")
    _check(0 < output_lora_a.size(0) <= 512, "output LoRA projection requires 0<R<=512")
    _check(output_lora_b.dim() == 2 and output_lora_b.size(0) == C
           and output_lora_b.size(1) == output_lora_a.size(0), "output_lora_b must have shape [C,R]")
    if float(torch.tensor(output_lora_scale, dtype=torch.float32)) == 0.0:
        return out
    return torch.addmm(out, torch.matmul(pre, output_lora_a.t()), output_lora_b.t(),
                       alpha=float(output_lora_scale))


def exported_names() -> Sequence[str]:
    return (
        "prepare_tmix_wkv7_recurrent_metadata",
        "prepare_tmix_wkv7_recurrent_graph_metadata",
        "tmix_wkv7_recurrent_fp32_from_decay_logits",
        "tmix_wkv7_recurrent_fp16_from_decay_logits",
        "tmix_wkv7_recurrent_fp32_from_kk_gate",
        "tmix_wkv7_recurrent_fp32_from_kk_gate_readout",
        "pretrain_tmix_wkv7_recurrent_forward",
        "pretrain_tmix_wkv7_recurrent_backward",
        "statetune_tmix_wkv7_recurrent_fp32io16_forward",
        "statetune_tmix_wkv7_recurrent_fp32io16_backward",
        "infer_tmix_wkv7_chunk_bf16_forward_varlen",
        "rl_infctx_tmix_wkv7_chunk_fp32io16_forward",
        "rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay",
        "tmix_wkv_prepare_forward_varlen",
        "tmix_readout_forward_varlen",
    )


# ---------------------------------------------------------------------------
# Misaligned views: every entry below runs them on aligned copies
# ---------------------------------------------------------------------------
for _name in (*exported_names(), "tmix_wkv7_recurrent_fp32_kernel_forced"):
    if _name.startswith("prepare_"):
        continue
    globals()[_name] = aligned_io(globals()[_name])
del _name
