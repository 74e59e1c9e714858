"""StateTune: the packed WKV7 recurrence from a trainable initial state.

Mirrors ``flashrwkv2.tmix.wkv7.statetune`` (flashrwkv2/tmix/wkv7/statetune.py:12-236):
the same public function, keyword-only ``scale``, validation messages and
return tuple ``(output, final_state, boundary, state_dot_a)`` (``boundary`` is
the fp32 state at the start of every chunk, ``[C,H,D,D]``; ``state_dot_a`` the
fp32 pre-update ``S^T a`` of every token).  The backward returns gradients for
the six token tensors and the initial state.  The kernels are the gfx950
StateTune kernels of ``lib/libflashrwkv2_amd.so``.

Beyond the reference's checks, all six token tensors must share one dtype
(the reference's kernel reads every one of them as the dtype of ``r``).
"""

from __future__ import annotations

import math

import torch

from . import _extension


def _check_cuda_contiguous(tensor: torch.Tensor, name: str) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not tensor.is_cuda or not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous CUDA")


def _check_metadata(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state) -> None:
    for name, tensor in (
        ("sequence_chunk_offsets", sequence_chunk_offsets),
        ("chunk_token_starts", chunk_token_starts),
        ("chunk_token_ends", chunk_token_ends),
    ):
        _check_cuda_contiguous(tensor, name)
        if tensor.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
        if tensor.device != state.device:
            raise ValueError(f"{name} must share the state device")
    if sequence_chunk_offsets.ndim != 1:
        raise ValueError("sequence_chunk_offsets must be one-dimensional")
    if chunk_token_starts.ndim != 1 or chunk_token_ends.shape != chunk_token_starts.shape:
        raise ValueError("chunk token metadata must have matching shape [C]")
    if chunk_token_starts.numel() == 0:
        raise ValueError("at least one training chunk is required")


def _check_token_inputs(state, r, decay_logits, k, v, a, b) -> None:
    _check_cuda_contiguous(state, "state")
    if state.dtype != torch.float32:
        raise TypeError("state must be float32")
    if state.ndim != 4 or state.shape[0] <= 0 or state.shape[1] <= 0:
        raise ValueError("state must have shape [B,H,D,D]")
    if state.shape[2] != state.shape[3] or state.shape[2] not in (64, 128, 256):
        raise ValueError("state head size must be 64, 128, or 256")
    tensors = {"r": r, "decay_logits": decay_logits, "k": k, "v": v, "a": a, "b": b}
    for name, tensor in tensors.items():
        _check_cuda_contiguous(tensor, name)
        if tensor.device != state.device:
            raise ValueError(f"{name} must share the state device")
        if tensor.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"{name} must be float16 or bfloat16")
        if tensor.shape != r.shape:
            raise ValueError(f"{name} must match r shape")
        if tensor.dtype != r.dtype:
            raise TypeError(f"{name} must have the dtype of r")
    if r.ndim != 3 or r.shape[0] <= 0 or r.shape[1:] != state.shape[1:3]:
        raise ValueError("token tensors must have shape [total_tokens,H,D]")


class _StateTune(torch.autograd.Function):
    """statetune.py:79-199 of the reference."""

    @staticmethod
    def forward(ctx, initial_state, sequence_chunk_offsets, chunk_token_starts,
                chunk_token_ends, r, decay_logits, k, v, a, b, scale):  # type: ignore[override]
        state = initial_state.detach().contiguous().clone()
        output = torch.empty_like(v)
        boundary = torch.empty(
            (chunk_token_starts.numel(), state.shape[1], state.shape[2], state.shape[3]),
            device=state.device, dtype=torch.float32)
        state_dot_a = torch.empty_like(r, dtype=torch.float32)
        # on the uniform layout (D = 64, bf16, equal sequences and chunks) the
        # native forward runs the chunked MFMA kernels and also returns the
        # post-16-token state snapshots its backward reads
        snapshots = _extension().statetune_tmix_wkv7_recurrent_fp32io16_forward(
            sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state, r,
            decay_logits, k, v, a, b, output, boundary, state_dot_a, float(scale))
        ctx.has_snapshots = snapshots is not None
        ctx.save_for_backward(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends,
                              state, r, decay_logits, k, v, a, b, state_dot_a, boundary,
                              *(() if snapshots is None else (snapshots,)))
        ctx.scale = float(scale)
        ctx.mark_non_differentiable(boundary, state_dot_a)
        return output, state, boundary, state_dot_a

    @staticmethod
    def backward(ctx, grad_output, grad_final_state, _grad_boundary, _grad_state_dot_a):  # type: ignore[override]
        saved = ctx.saved_tensors
        (offsets, starts, ends, final_state, r, decay_logits, k, v, a, b, state_dot_a,
         boundary) = saved[:12]
        snapshots = saved[12] if ctx.has_snapshots else None
        if grad_output is not None:
            grad_output = grad_output.contiguous().to(v.dtype)
        if grad_final_state is not None:
            grad_final_state = grad_final_state.contiguous().float()
        gradients = [torch.empty_like(t) for t in (r, decay_logits, k, v, a, b)]
        grad_initial = torch.empty_like(final_state)
        _extension().statetune_tmix_wkv7_recurrent_fp32io16_backward(
            offsets, starts, ends, final_state, r, decay_logits, k, v, a, b, state_dot_a,
            grad_output, grad_final_state, boundary, *gradients, grad_initial, ctx.scale,
            snapshots=snapshots)
        return (grad_initial, None, None, None, *gradients, None)


def statetune_tmix_wkv7_recurrent_fp32io16(initial_state, sequence_chunk_offsets,
                                           chunk_token_starts, chunk_token_ends, r,
                                           decay_logits, k, v, a, b, *, scale: float = 1.0):
    """Run StateTune with a nonzero state and direct initial-state gradient
    (statetune.py:202-236 of the reference)."""
    _check_token_inputs(initial_state, r, decay_logits, k, v, a, b)
    _check_metadata(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, initial_state)
    if sequence_chunk_offsets.numel() != initial_state.shape[0] + 1:
        raise ValueError("sequence_chunk_offsets must have shape [B+1]")
    if not isinstance(scale, (int, float)) or not math.isfinite(float(scale)):
        raise ValueError("scale must be finite")
    return _StateTune.apply(initial_state, sequence_chunk_offsets, chunk_token_starts,
                            chunk_token_ends, r, decay_logits, k, v, a, b, float(scale))


__all__ = ["statetune_tmix_wkv7_recurrent_fp32io16"]
