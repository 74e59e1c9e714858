"""Public WKV7 entry points: packed varlen recurrence with an fp32 state pool
and its metadata tickets.

Names, keyword arguments, defaults and the Python-side error types/messages
follow ``flashrwkv2.tmix.wkv7`` (flashrwkv2/tmix/wkv7/__init__.py:8-256) so
that callers can switch packages without code changes.  The native layer is
:mod:`flashrwkv2_amd._C`, backed by the gfx950 HIP library.
"""

from __future__ import annotations

import torch

from .. import _checks as ck


def _extension():
    """The native operator module (…/wkv7/__init__.py:8-17)."""
    import flashrwkv2_amd

    extension = getattr(flashrwkv2_amd, "_C", None)
    if extension is None:
        raise RuntimeError(
            "FlashRWKV2 CUDA extension is not built; build flashrwkv2._C before "
            "using the accelerated recurrent operator"
        )
    return extension


_TOKENS = ("r", "decay_logits", "k", "v", "a", "b")
# rule tables (static: built once, applied per call)
_PACKED_RULES = (
    ck.is_tensor(),
    ck.holds(lambda t: t.ndim == 3, "{name} must have packed shape [total_tokens,H,D]"),
    ck.holds(lambda t: t.is_contiguous(), "{name} must be contiguous"),
)
_FP32_POOL_RULES = (
    ck.is_tensor(),
    ck.holds(lambda t: t.is_contiguous(), "{name} must be contiguous"),
    ck.dtype_in((torch.float32,), "{name} must have dtype float32"),
)
_FP16_POOL_RULES = (
    ck.is_tensor(),
    ck.holds(lambda t: t.is_contiguous(), "{name} must be contiguous"),
    ck.dtype_in((torch.float16,), "FP16-state {name} must have dtype float16"),
)
_CU_SEQLENS_RULES = (ck.is_tensor(),
                     ck.holds(lambda t: t.ndim == 1, "{name} must be one-dimensional"))


# Each validator first tests the common case in one expression and only walks
# the rule table (for the first failing rule's message) when that fails: the
# decode path calls these on every step.
def _validate_packed_inputs(*tensors: torch.Tensor) -> tuple[torch.Tensor, ...]:
    if not all(isinstance(t, torch.Tensor) and t.ndim == 3 and t.is_contiguous()
               for t in tensors):
        ck.verify(ck.each(_TOKENS, tensors, _PACKED_RULES))
    return tensors


def _validate_state(state: torch.Tensor) -> None:
    if not (isinstance(state, torch.Tensor) and state.is_contiguous()
            and state.dtype == torch.float32):
        ck.verify((("state_pool", state, _FP32_POOL_RULES),))


def _check_metadata_inputs(cu_seqlens: torch.Tensor, state_indices: torch.Tensor) -> None:
    if not (isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.ndim == 1
            and isinstance(state_indices, torch.Tensor)):
        ck.verify((("cu_seqlens", cu_seqlens, _CU_SEQLENS_RULES),
                   ("state_indices", state_indices, (ck.is_tensor(),))))


def _resolve_max_seqlen(cu_seqlens: torch.Tensor, max_seqlen: int | None) -> int:
    if max_seqlen is not None:
        value = int(max_seqlen)
        if value <= 0:
            raise ValueError("max_seqlen must be positive")
        return value
    if cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must contain at least one sequence")
    return int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item())


def _positive_int(name: str, value: object) -> None:
    if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")


def prepare_tmix_wkv7_recurrent_metadata(
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    *,
    state_pool_size: int,
    total_tokens: int | None = None,
    max_seqlen: int | None = None,
    token_capacity: int | None = None,
    sequence_capacity: int | None = None,
    max_seqlen_capacity: int | None = None,
    num_active_tokens: torch.Tensor | None = None,
    num_active_sequences: torch.Tensor | None = None,
) -> object:
    """Validate packed metadata once and return a ticket.

    Static form (``total_tokens``): the metadata values are checked on the
    host and on the device, and a private snapshot is validated and used by
    every consumer.  Capacity form (all five capacity/active arguments): the
    metadata and the two device scalars stay live, which is what a HIP graph
    needs; warm up with zero active counts, then prepare again inside capture
    and reuse that ticket for the graph's operators.
    """
    if (num_active_tokens is not None and total_tokens is None and max_seqlen is None
            and type(token_capacity) is int and type(sequence_capacity) is int
            and type(state_pool_size) is int and type(max_seqlen_capacity) is int):
        # the per-step serving case: decided natively when plainly valid
        ticket = _extension()._prepare_graph_fast(
            cu_seqlens, state_indices, num_active_tokens, num_active_sequences,
            token_capacity, sequence_capacity, state_pool_size, max_seqlen_capacity)
        if ticket is not None:
            return ticket
    _check_metadata_inputs(cu_seqlens, state_indices)
    live = (token_capacity, sequence_capacity, max_seqlen_capacity,
            num_active_tokens, num_active_sequences)
    if any(item is not None for item in live):
        if total_tokens is not None or max_seqlen is not None:
            raise ValueError(
                "graph metadata uses capacity arguments, not total_tokens/max_seqlen"
            )
        if any(item is None for item in live):
            raise ValueError(
                "all graph metadata capacity and active-count arguments are required"
            )
        for name, value in (("token_capacity", token_capacity),
                            ("sequence_capacity", sequence_capacity),
                            ("state_pool_size", state_pool_size),
                            ("max_seqlen_capacity", max_seqlen_capacity)):
            _positive_int(name, value)
        dev = cu_seqlens.get_device()
        for name, value in (("num_active_tokens", num_active_tokens),
                            ("num_active_sequences", num_active_sequences)):
            ok = (isinstance(value, torch.Tensor) and value.dtype == torch.int32
                  and value.is_cuda and value.is_contiguous() and value.numel() == 1
                  and value.get_device() == dev)
            if not ok:
                raise ValueError(f"{name} must be a one-element contiguous CUDA int32 tensor")
        return _extension().prepare_tmix_wkv7_recurrent_graph_metadata(
            cu_seqlens, state_indices, num_active_tokens, num_active_sequences,
            token_capacity, sequence_capacity, state_pool_size, max_seqlen_capacity,
        )
    if total_tokens is None:
        raise ValueError("total_tokens is required for static recurrent metadata")
    return _extension().prepare_tmix_wkv7_recurrent_metadata(
        cu_seqlens, state_indices, total_tokens, state_pool_size,
        -1 if max_seqlen is None else int(max_seqlen),
    )


def infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed raw-decay-logit RWKV-7 recurrence, ``state_pool`` updated in place.

    Token tensors are fp16/bf16 ``[total_tokens,H,D]``; ``state_pool`` is fp32
    ``[slots,H,D,D]``; returns the output ``[total_tokens,H,D]`` in the token
    dtype.  (…/wkv7/__init__.py:179-256.)
    """
    if (validated_metadata is not None and decay_bias is None
            and type(scale) in (float, int) and (max_seqlen is None or type(max_seqlen) is int)):
        # the per-step serving case: decided natively when plainly valid
        output = _extension()._recurrent_fp32_fast(
            cu_seqlens, state_indices, state_pool, r, decay_logits, k, v, a, b, float(scale),
            validated_metadata, -1 if max_seqlen is None else max_seqlen)
        if output is not None:
            return output
    packed = _validate_packed_inputs(r, decay_logits, k, v, a, b)
    _validate_state(state_pool)
    _check_metadata_inputs(cu_seqlens, state_indices)
    ticket = validated_metadata
    if ticket is None:
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            cu_seqlens, state_indices, total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0], max_seqlen=max_seqlen,
        )
    output = torch.empty_like(packed[3])
    _extension().tmix_wkv7_recurrent_fp32_from_decay_logits(
        cu_seqlens, state_indices, state_pool, *packed, output, float(scale),
        decay_bias, ticket, -1 if max_seqlen is None else int(max_seqlen),
    )
    return output


def _validate_fp16_state(state: torch.Tensor) -> None:
    """…/wkv7/__init__.py:41-47."""
    ck.verify((("state_pool", state, _FP16_POOL_RULES),))


def _validate_fp16_elapsed_state(elapsed_state_pool: torch.Tensor,
                                 state_pool: torch.Tensor) -> None:
    """…/wkv7/__init__.py:50-62."""
    ck.verify((("elapsed_state_pool", elapsed_state_pool, (
        ck.is_tensor(),
        ck.dtype_in((torch.int32,), "{name} must have dtype torch.int32"),
        ck.cuda_contiguous("{name} must be contiguous CUDA int32"),
        ck.on_device_of(state_pool, "{name} must share state_pool's device"),
        ck.holds(lambda t: t.ndim == 1 and t.shape[0] == state_pool.shape[0],
                 "{name} must have shape [state_pool_slots]"),
    )),))


def infer_tmix_wkv7_recurrent_fp16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    elapsed_state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed recurrence with an FP16 state pool (the Albatross delta/phase
    contract); ``state_pool`` is updated in place and ``elapsed_state_pool``
    advanced by each active sequence's length.  (…/wkv7/__init__.py:259-318.)
    """
    packed = _validate_packed_inputs(r, decay_logits, k, v, a, b)
    _validate_fp16_state(state_pool)
    _validate_fp16_elapsed_state(elapsed_state_pool, state_pool)
    _check_metadata_inputs(cu_seqlens, state_indices)
    if max_seqlen is None:
        # max_seqlen inference belongs to metadata preparation: no device sync
        # on every launch
        launch_max_seqlen = -1
    else:
        if (not isinstance(max_seqlen, int) or isinstance(max_seqlen, bool)
                or max_seqlen <= 0):
            raise ValueError("max_seqlen must be a positive integer")
        launch_max_seqlen = int(max_seqlen)
    ticket = (
        validated_metadata
        if validated_metadata is not None
        else prepare_tmix_wkv7_recurrent_metadata(
            cu_seqlens, state_indices, total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0], max_seqlen=launch_max_seqlen,
        )
    )
    output = torch.empty_like(packed[3])
    _extension().tmix_wkv7_recurrent_fp16_from_decay_logits(
        cu_seqlens, state_indices, elapsed_state_pool, state_pool, *packed, output,
        float(scale), decay_bias, ticket, launch_max_seqlen,
    )
    return output


__all__ = [
    "infer_tmix_wkv7_recurrent_fp32io16_forward_varlen",
    "infer_tmix_wkv7_recurrent_fp16_forward_varlen",
    "prepare_tmix_wkv7_recurrent_metadata",
]

from .pretrain import pretrain_tmix_wkv7_recurrent_bf16  # noqa: E402
from .chunk import infer_tmix_wkv7_chunk_bf16_forward_varlen  # noqa: E402
from .rl_infctx import (  # noqa: E402
    rl_infctx_tmix_wkv7_chunk_fp32io16,
    rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute,
)
from .statetune import statetune_tmix_wkv7_recurrent_fp32io16  # noqa: E402
from .fused import (  # noqa: E402
    infer_tmix_wkv7_kk_gate_recurrent_forward_varlen,
    infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen,
)

__all__ += [
    "infer_tmix_wkv7_kk_gate_recurrent_forward_varlen",
    "infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen",
    "statetune_tmix_wkv7_recurrent_fp32io16",
    "pretrain_tmix_wkv7_recurrent_bf16",
    "infer_tmix_wkv7_chunk_bf16_forward_varlen",
    "rl_infctx_tmix_wkv7_chunk_fp32io16",
    "rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute",
]
