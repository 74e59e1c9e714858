"""``[B,T,C]`` bf16 training-layout WKV7 forward with zero initial state.

Mirrors ``flashrwkv2.tmix.wkv7.pretrain`` (flashrwkv2/tmix/wkv7/pretrain.py:14-130):
same validation messages, the same ``boundary`` (post-chunk state every 16
tokens, fp32 ``[B,H,T/16,N,N]``) and ``state_dot_a`` (fp32 ``[B,T,H,N]``)
checkpoints, and the backward (pretrain.py:88-114 of the reference) that
consumes them through ``pretrain_tmix_wkv7_recurrent_backward``.
"""

from __future__ import annotations

import torch

from . import _extension

CHUNK_LEN = 16


def _validate_inputs(tensors: tuple[torch.Tensor, ...], head_size: int) -> tuple[int, int, int]:
    if head_size not in {64, 128, 256}:
        raise ValueError("head_size must be one of 64, 128, or 256")
    if len(tensors) != 6:
        raise ValueError("clampw requires r, w, k, v, a, and b")
    r = tensors[0]
    if not isinstance(r, torch.Tensor):
        raise TypeError("r must be a torch.Tensor")
    if r.ndim != 3 or min(r.shape) <= 0:
        raise ValueError("r must have shape [B,T,C] with nonzero dimensions")
    if r.dtype != torch.bfloat16:
        raise TypeError("r must be bfloat16")
    if not r.is_cuda or not r.is_contiguous():
        raise ValueError("r must be contiguous CUDA")
    for name, tensor in zip(("w", "k", "v", "a", "b"), tensors[1:]):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16")
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous CUDA")
        if tensor.shape != r.shape:
            raise ValueError(f"{name} must match r shape")
        if tensor.device != r.device:
            raise ValueError(f"{name} must share the r device")
    batch, tokens, channels = r.shape
    if channels % head_size != 0:
        raise ValueError("C must be divisible by head_size")
    if tokens % CHUNK_LEN != 0:
        raise ValueError("T must be divisible by the canonical chunk length 16")
    return batch, tokens, channels


class _PretrainRecurrent(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, w, k, v, a, b, head_size):  # type: ignore[override]
        batch, tokens, channels = _validate_inputs((r, w, k, v, a, b), head_size)
        heads = channels // head_size
        values = tuple(t.view(batch, tokens, heads, head_size) for t in (r, w, k, v, a, b))
        output = torch.empty_like(values[3])
        boundary = torch.empty((batch, heads, tokens // CHUNK_LEN, head_size, head_size),
                               device=r.device, dtype=torch.float32)
        state_dot_a = torch.empty((batch, tokens, heads, head_size), device=r.device,
                                  dtype=torch.float32)
        _extension().pretrain_tmix_wkv7_recurrent_forward(
            *values, output, boundary, state_dot_a, head_size)
        ctx.save_for_backward(*values, boundary, state_dot_a)
        ctx.input_shape = (batch, tokens, channels)
        ctx.head_size = head_size
        return output.view(batch, tokens, channels)

    @staticmethod
    def backward(ctx, grad_output):  # type: ignore[override]
        r, w, k, v, a, b, boundary, state_dot_a = ctx.saved_tensors
        batch, tokens, channels = ctx.input_shape
        head_size = ctx.head_size
        heads = channels // head_size
        grad_output_4d = grad_output.contiguous().view(batch, tokens, heads, head_size)
        if grad_output_4d.dtype != torch.bfloat16:
            grad_output_4d = grad_output_4d.to(torch.bfloat16)
        gradients = tuple(torch.empty_like(t) for t in (r, w, k, v, a, b))
        _extension().pretrain_tmix_wkv7_recurrent_backward(
            r, w, k, v, a, b, grad_output_4d, boundary, state_dot_a, *gradients, head_size)
        return tuple(g.view(batch, tokens, channels) for g in gradients) + (None,)


def pretrain_tmix_wkv7_recurrent_bf16(
    r: torch.Tensor,
    w: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    head_size: int = 64,
) -> torch.Tensor:
    """WKV7 over ``[B,T,C]`` bf16 inputs (``w`` holds decay logits), zero state."""
    _validate_inputs((r, w, k, v, a, b), head_size)
    return _PretrainRecurrent.apply(r, w, k, v, a, b, head_size)


__all__ = ["pretrain_tmix_wkv7_recurrent_bf16"]
