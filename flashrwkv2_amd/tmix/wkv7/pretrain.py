"""``[B,T,C]`` bf16 training-layout WKV7 with zero initial state, with autograd.

Public contract of ``flashrwkv2.tmix.wkv7.pretrain`` (flashrwkv2/tmix/wkv7/pretrain.py:14-130):
the same function, keyword ``head_size`` and error messages.  The forward
keeps two checkpoints for the backward: the post-chunk state every 16 tokens
(``boundary``, fp32 ``[B,H,T/16,N,N]``) and every token's pre-update ``S^T a``
(``state_dot_a``, fp32 ``[B,T,H,N]``); the backward consumes them through
``pretrain_tmix_wkv7_recurrent_backward``.
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from . import _extension

CHUNK_LEN = 16
_NAMES = ("r", "w", "k", "v", "a", "b")


def _rows(tensors):
    r = tensors[0]
    first = [
        ck.is_tensor(),
        ck.holds(lambda t: t.ndim == 3 and min(t.shape) > 0,
                 "r must have shape [B,T,C] with nonzero dimensions"),
        ck.dtype_in((torch.bfloat16,), "{name} must be bfloat16"),
        ck.cuda_contiguous(),
    ]
    rest = [
        ck.is_tensor(),
        ck.dtype_in((torch.bfloat16,), "{name} must be bfloat16"),
        ck.cuda_contiguous(),
        ck.matches(r, "{name} must match r shape", device=False),
        ck.on_device_of(r, "{name} must share the r device"),
    ]
    return [("r", r, first), *ck.each(_NAMES[1:], tensors[1:], rest)]


def _layout(tensors, head_size):
    """(batch, tokens, channels) after every argument check."""
    if head_size not in (64, 128, 256):
        raise ValueError("head_size must be one of 64, 128, or 256")
    if len(tensors) != len(_NAMES):
        raise ValueError("clampw requires r, w, k, v, a, and b")
    ck.verify(_rows(tensors))
    batch, tokens, channels = tensors[0].shape
    ck.verify([
        ("C", channels, [ck.holds(lambda c: c % head_size == 0,
                                  "C must be divisible by head_size")]),
        ("T", tokens, [ck.holds(lambda t: t % CHUNK_LEN == 0,
                                "T must be divisible by the canonical chunk length 16")]),
    ])
    return batch, tokens, channels


def _heads(t: torch.Tensor, head_size: int) -> torch.Tensor:
    """[B,T,C] -> [B,T,H,N] view."""
    b, n, c = t.shape
    return t.view(b, n, c // head_size, head_size)


class _PretrainWKV7(torch.autograd.Function):
    """Forward on the chunked kernels with checkpoints; backward from them."""

    @staticmethod
    def forward(ctx, head_size, *inputs):  # type: ignore[override]
        x = [_heads(t, head_size) for t in inputs]
        batch, tokens, heads, _ = x[0].shape
        f32 = dict(device=inputs[0].device, dtype=torch.float32)
        out = torch.empty_like(x[3])
        boundary = torch.empty((batch, heads, tokens // CHUNK_LEN, head_size, head_size), **f32)
        sa = torch.empty((batch, tokens, heads, head_size), **f32)
        _extension().pretrain_tmix_wkv7_recurrent_forward(*x, out, boundary, sa, head_size)
        ctx.head_size = head_size
        ctx.save_for_backward(*x, boundary, sa)
        return out.view_as(inputs[0])

    @staticmethod
    def backward(ctx, grad_out):  # type: ignore[override]
        *x, boundary, sa = ctx.saved_tensors
        dy = _heads(grad_out.to(torch.bfloat16).contiguous(), ctx.head_size)
        grads = [torch.empty_like(t) for t in x]
        _extension().pretrain_tmix_wkv7_recurrent_backward(*x, dy, boundary, sa, *grads,
                                                           ctx.head_size)
        flat = dy.shape[:2] + (dy.shape[2] * dy.shape[3],)
        return (None, *(g.view(flat) for g in grads))


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
    _layout((r, w, k, v, a, b), head_size)
    return _PretrainWKV7.apply(head_size, r, w, k, v, a, b)


__all__ = ["pretrain_tmix_wkv7_recurrent_bf16"]
