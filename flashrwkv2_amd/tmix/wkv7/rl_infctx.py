"""Packed RL/Infctx chunked WKV7 forward with an fp32 state pool (not in place).

Public contract of ``flashrwkv2.tmix.wkv7.rl_infctx`` (flashrwkv2/tmix/wkv7/rl_infctx.py:12-162):
the same functions, keyword arguments, defaults and error messages.  The
call returns ``(output, new_pool)``: the selected pool rows are gathered into
a working state, the native forward runs over fixed-size chunks of every
sequence (16, 32 or 64 tokens; the last chunk of a sequence may be short),
and the final states are scattered into a copy of the pool.  The input pool
is never written.
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from . import _extension

_TOKENS = ("r", "decay_logits", "k", "v", "a", "b")
_STRATEGY = {"materialized": 0, "recompute": 1}


def _token_rows(tokens):
    r = tokens[0]
    base = [ck.is_tensor(), ck.cuda_contiguous(),
            ck.dtype_in((torch.float16, torch.bfloat16), "{name} must be float16 or bfloat16")]
    rows = ck.each(_TOKENS, tokens, base)
    rows.append(("r", r, [ck.holds(
        lambda t: t.ndim == 3 and t.shape[0] > 0 and t.shape[1] > 0 and t.shape[2] in (64, 128, 256),
        "RL/Infctx token tensors must have shape [N,H,D]")]))
    rows.append(("tokens", tokens, [ck.holds(
        lambda ts: all(t.shape == r.shape and t.device == r.device for t in ts),
        "RL/Infctx token tensors must match r and share a device")]))
    return rows


def _bias_rows(r, decay_bias):
    return [("decay_bias", decay_bias, ck.optional([
        ck.is_tensor(), ck.cuda_contiguous(),
        ck.holds(lambda t: t.dtype == r.dtype and t.device == r.device,
                 "decay_bias must match token dtype and device", TypeError),
        ck.shape_is(((r.shape[1] * r.shape[2],), (r.shape[1], r.shape[2])),
                    "decay_bias must have shape [H*D] or [H,D]"),
    ]))]


def _int32_rows(name, t):
    return [(name, t, [ck.is_tensor(), ck.cuda_contiguous(),
                       ck.dtype_in((torch.int32,), "{name} must have dtype torch.int32")])]


def _host_offsets(cu_seqlens: torch.Tensor, total_tokens: int, device) -> torch.Tensor:
    """Host copy of cu_seqlens (int64) after the layout and range checks."""
    ck.verify([("cu_seqlens", cu_seqlens, [
        ck.holds(lambda t: t.device == device, "cu_seqlens must share the token device"),
        ck.holds(lambda t: t.ndim == 1 and t.numel() >= 2, "cu_seqlens must have shape [B+1]"),
    ])])
    offsets = cu_seqlens.cpu().to(torch.int64)
    lengths = offsets[1:] - offsets[:-1]
    ck.verify([("cu_seqlens", offsets, [
        ck.holds(lambda o: int(o[0]) == 0, "cu_seqlens must start at zero"),
        ck.holds(lambda o: int(o[-1]) == total_tokens, "cu_seqlens must end at total_tokens"),
        ck.holds(lambda o: bool((lengths > 0).all()),
                 "each RL/Infctx sequence must be non-empty"),
    ])])
    return offsets


def _chunk_table(offsets: torch.Tensor, chunk_size: int, device):
    """Per-sequence chunk offsets [B+1] and each chunk's [start, end) token range,
    built with tensor arithmetic on the host copy of cu_seqlens."""
    lengths = offsets[1:] - offsets[:-1]
    per_seq = (lengths + chunk_size - 1) // chunk_size
    seq_chunks = torch.zeros(per_seq.numel() + 1, dtype=torch.int64)
    torch.cumsum(per_seq, 0, out=seq_chunks[1:])
    owner = torch.repeat_interleave(torch.arange(per_seq.numel()), per_seq)
    rank = torch.arange(int(seq_chunks[-1])) - seq_chunks[owner]
    starts = offsets[owner] + rank * chunk_size
    ends = torch.minimum(starts + chunk_size, offsets[owner + 1])
    return tuple(t.to(device=device, dtype=torch.int32) for t in (seq_chunks, starts, ends))


def rl_infctx_tmix_wkv7_chunk_fp32io16(
    r, decay_logits, k, v, a, b, *, state_pool=None, cu_seqlens, state_indices=None,
    chunk_size: int = 16, strategy: str = "recompute", scale: float = 1.0,
    decay_bias=None,
):
    """Returns ``(output, new_pool)``; the input pool is left unchanged."""
    ck.verify([
        ("chunk_size", chunk_size, [ck.holds(lambda c: c in (16, 32, 64),
                                             "chunk_size must be one of 16, 32, or 64")]),
        ("strategy", strategy, [ck.holds(lambda s: s in _STRATEGY,
                                         "strategy must be 'materialized' or 'recompute'")]),
        ("scale", scale, [ck.holds(ck.finite, "scale must be finite")]),
    ])
    tokens = (r, decay_logits, k, v, a, b)
    ck.verify(_token_rows(tokens))
    ck.verify(_bias_rows(r, decay_bias))
    ck.verify(_int32_rows("cu_seqlens", cu_seqlens))
    offsets = _host_offsets(cu_seqlens, r.shape[0], r.device)
    batch = offsets.numel() - 1
    heads, d = r.shape[1], r.shape[2]
    if state_indices is None:
        state_indices = torch.arange(batch, device=r.device, dtype=torch.int32)
    ck.verify(_int32_rows("state_indices", state_indices))
    ck.verify([("state_indices", state_indices, [
        ck.holds(lambda t: t.ndim == 1 and t.numel() == batch, "state_indices must have shape [B]"),
        ck.on_device_of(r, "state_indices must share the token device"),
    ])])
    slots = state_indices.cpu()
    if slots.unique().numel() != slots.numel():
        raise ValueError("state_indices must not contain duplicates")
    if state_pool is None:
        state_pool = torch.zeros(batch, heads, d, d, device=r.device, dtype=torch.float32)
    ck.verify([("state_pool", state_pool, [
        ck.is_tensor(), ck.cuda_contiguous(),
        ck.dtype_in((torch.float32,), "{name} must have dtype torch.float32"),
        ck.holds(lambda s: s.ndim == 4 and tuple(s.shape[1:]) == (heads, d, d),
                 "state_pool must have shape [slots,H,D,D]"),
    ])])
    if batch and (int(slots.min()) < 0 or int(slots.max()) >= state_pool.shape[0]):
        raise ValueError("state_indices must be within state_pool")
    rows = state_indices.to(torch.int64)
    output, final = _extension().rl_infctx_tmix_wkv7_chunk_fp32io16_forward(
        *_chunk_table(offsets, chunk_size, r.device), state_pool.index_select(0, rows), *tokens,
        _STRATEGY[strategy], float(scale), decay_bias)
    new_pool = state_pool.clone()
    new_pool[rows] = final
    return output, new_pool


def rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute(*args, **kwargs):
    """The ``strategy="recompute"`` form of :func:`rl_infctx_tmix_wkv7_chunk_fp32io16`."""
    return rl_infctx_tmix_wkv7_chunk_fp32io16(*args, **{**kwargs, "strategy": "recompute"})


__all__ = ["rl_infctx_tmix_wkv7_chunk_fp32io16",
           "rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute"]
