"""Packed bf16 WKV7 inference with a bf16 state pool.

Public contract of ``flashrwkv2.tmix.wkv7.chunk`` (flashrwkv2/tmix/wkv7/chunk.py:17-128):
the same function name, keyword arguments, defaults and error messages.  The
state is carried in fp32 inside the call and rounded to bf16 once per
sequence when it is written back to the pool.
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from . import (
    _check_metadata_inputs,
    _extension,
    _resolve_max_seqlen,
    prepare_tmix_wkv7_recurrent_metadata,
)

_TOKENS = ("r", "decay_logits", "k", "v", "a", "b")
_HEAD = 64


def _argument_rows(tokens, state_pool, chunk_size, scale):
    r = tokens[0]
    token_rules = [
        ck.is_tensor(),
        ck.cuda_contiguous_of(torch.bfloat16, "{name} must be contiguous CUDA bfloat16"),
        ck.on_device_of(r, "{name} must share r's device"),
        ck.matches(r, "{name} must have the same shape as r", device=False),
    ]
    pool_ok = ck.holds(
        lambda s: isinstance(s, torch.Tensor) and s.dtype == torch.bfloat16 and s.is_cuda
        and s.is_contiguous() and s.ndim == 4 and s.device == r.device
        and tuple(s.shape[1:]) == (r.shape[1], _HEAD, _HEAD),
        "state_pool must be contiguous CUDA bfloat16 [slots,H,64,64]")
    return [
        ("chunk_size", chunk_size, [ck.holds(ck.is_int, "chunk_size must be an integer", TypeError),
                                    ck.holds(lambda n: n > 0, "chunk_size must be positive")]),
        ("scale", scale, [ck.holds(ck.finite, "scale must be finite")]),
        *ck.each(_TOKENS, tokens, token_rules),
        ("r", r, [ck.holds(lambda t: t.ndim == 3 and t.shape[0] > 0 and t.shape[1] > 0
                           and t.shape[2] == _HEAD,
                           "packed chunk inputs must have shape [total_tokens,H,64]")]),
        ("state_pool", state_pool, [pool_ok]),
    ]


def _metadata_rows(r, cu_seqlens, state_indices):
    meta_ok = ck.holds(
        lambda t: t.dtype == torch.int32 and t.is_cuda and t.is_contiguous()
        and t.device == r.device, "chunk metadata must be contiguous CUDA int32")
    return ck.each(("cu_seqlens", "state_indices"), (cu_seqlens, state_indices), [meta_ok])


def _bias_rows(r, decay_bias):
    heads = r.shape[1]
    return [("decay_bias", decay_bias, ck.optional([
        ck.holds(lambda t: t.dtype == torch.bfloat16 and t.is_cuda and t.is_contiguous()
                 and t.device == r.device and tuple(t.shape) in {(heads, _HEAD), (heads * _HEAD,)},
                 "decay_bias must be contiguous CUDA bfloat16 [H,64] or [H*64]")]))]


def infer_tmix_wkv7_chunk_bf16_forward_varlen(
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
    chunk_size: int = 16,
    max_seqlen: int | None = None,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Run packed requests against a bf16 ``[slots,H,64,64]`` pool, in place."""
    tokens = (r, decay_logits, k, v, a, b)
    ck.verify(_argument_rows(tokens, state_pool, chunk_size, scale))
    _check_metadata_inputs(cu_seqlens, state_indices)
    ck.verify(_metadata_rows(r, cu_seqlens, state_indices))
    # a ticket carries the sequence bound it was validated with
    if validated_metadata is not None and max_seqlen is None:
        bound = int(validated_metadata._max_seqlen())
    else:
        bound = _resolve_max_seqlen(cu_seqlens, max_seqlen)
    ticket = validated_metadata
    if ticket is None:
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            cu_seqlens, state_indices, total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0], max_seqlen=bound)
    ck.verify(_bias_rows(r, decay_bias))
    output, _ = _extension().infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *tokens, state_pool, cu_seqlens, state_indices, int(chunk_size), int(bound),
        float(scale), decay_bias=decay_bias, validated_metadata=ticket)
    return output


__all__ = ["infer_tmix_wkv7_chunk_bf16_forward_varlen"]
