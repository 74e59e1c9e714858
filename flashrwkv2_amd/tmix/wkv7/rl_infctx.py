"""Packed RL/Infctx chunked WKV7 forward with an fp32 state pool (not in place).

Mirrors ``flashrwkv2.tmix.wkv7.rl_infctx`` (flashrwkv2/tmix/wkv7/rl_infctx.py:12-162):
the chunk metadata (per-sequence chunk offsets and chunk token ranges for
chunk sizes 16/32/64) is built once on the host, the selected pool rows are
gathered, the native forward runs, and the final states are scattered into a
clone of the pool, which is returned with the output.
"""

from __future__ import annotations

import math

import torch

from . import _extension


def _check_tensor(tensor, name, dtype=None):
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not tensor.is_cuda or not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous CUDA")
    if dtype is not None and tensor.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}")


def _validate_cu_seqlens(cu_seqlens: torch.Tensor, *, total_tokens: int,
                         device: torch.device) -> list[int]:
    if cu_seqlens.dtype != torch.int32:
        raise TypeError("cu_seqlens must have dtype torch.int32")
    if not cu_seqlens.is_cuda or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be contiguous CUDA int32")
    if cu_seqlens.device != device:
        raise ValueError("cu_seqlens must share the token device")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must have shape [B+1]")
    offsets = cu_seqlens.cpu().tolist()
    if offsets[0] != 0:
        raise ValueError("cu_seqlens must start at zero")
    if offsets[-1] != total_tokens:
        raise ValueError("cu_seqlens must end at total_tokens")
    if any(hi - lo <= 0 for lo, hi in zip(offsets[:-1], offsets[1:])):
        raise ValueError("each RL/Infctx sequence must be non-empty")
    return offsets


def _make_chunk_metadata(offsets: list[int], chunk_size: int, device: torch.device):
    """Per-sequence chunk offsets plus chunk [start, end) token ranges."""
    seq_chunks = [0]
    starts: list[int] = []
    ends: list[int] = []
    for lo, hi in zip(offsets[:-1], offsets[1:]):
        for start in range(lo, hi, chunk_size):
            starts.append(start)
            ends.append(min(start + chunk_size, hi))
        seq_chunks.append(len(starts))
    as_i32 = dict(device=device, dtype=torch.int32)
    return (torch.tensor(seq_chunks, **as_i32), torch.tensor(starts, **as_i32),
            torch.tensor(ends, **as_i32))


def rl_infctx_tmix_wkv7_chunk_fp32io16(
    r, decay_logits, k, v, a, b, *, state_pool=None, cu_seqlens, state_indices=None,
    chunk_size: int = 16, strategy: str = "recompute", scale: float = 1.0,
    decay_bias=None,
):
    """Returns ``(output, new_pool)``; the input pool is left unchanged."""
    if chunk_size not in {16, 32, 64}:
        raise ValueError("chunk_size must be one of 16, 32, or 64")
    if strategy not in {"materialized", "recompute"}:
        raise ValueError("strategy must be 'materialized' or 'recompute'")
    if not math.isfinite(float(scale)):
        raise ValueError("scale must be finite")
    tensors = {"r": r, "decay_logits": decay_logits, "k": k, "v": v, "a": a, "b": b}
    for name, tensor in tensors.items():
        _check_tensor(tensor, name)
        if tensor.dtype not in {torch.float16, torch.bfloat16}:
            raise TypeError(f"{name} must be float16 or bfloat16")
    if r.ndim != 3 or r.shape[0] <= 0 or r.shape[1] <= 0 or r.shape[2] not in {64, 128, 256}:
        raise ValueError("RL/Infctx token tensors must have shape [N,H,D]")
    if any(t.shape != r.shape or t.device != r.device for t in tensors.values()):
        raise ValueError("RL/Infctx token tensors must match r and share a device")
    if decay_bias is not None:
        _check_tensor(decay_bias, "decay_bias")
        if decay_bias.dtype != r.dtype or decay_bias.device != r.device:
            raise TypeError("decay_bias must match token dtype and device")
        if decay_bias.shape not in {(r.shape[1] * r.shape[2],), (r.shape[1], r.shape[2])}:
            raise ValueError("decay_bias must have shape [H*D] or [H,D]")
    _check_tensor(cu_seqlens, "cu_seqlens", torch.int32)
    offsets = _validate_cu_seqlens(cu_seqlens, total_tokens=r.shape[0], device=r.device)
    batch = len(offsets) - 1
    if state_indices is None:
        state_indices = torch.arange(batch, device=r.device, dtype=torch.int32)
    _check_tensor(state_indices, "state_indices", torch.int32)
    if state_indices.ndim != 1 or state_indices.numel() != batch:
        raise ValueError("state_indices must have shape [B]")
    if state_indices.device != r.device:
        raise ValueError("state_indices must share the token device")
    slots = state_indices.cpu().tolist()
    if len(set(slots)) != len(slots):
        raise ValueError("state_indices must not contain duplicates")
    if state_pool is None:
        state_pool = torch.zeros(batch, r.shape[1], r.shape[2], r.shape[2], device=r.device,
                                 dtype=torch.float32)
    _check_tensor(state_pool, "state_pool", torch.float32)
    if state_pool.ndim != 4 or state_pool.shape[1:] != (r.shape[1], r.shape[2], r.shape[2]):
        raise ValueError("state_pool must have shape [slots,H,D,D]")
    if max(slots, default=-1) >= state_pool.shape[0] or min(slots, default=0) < 0:
        raise ValueError("state_indices must be within state_pool")
    chunk_metadata = _make_chunk_metadata(offsets, chunk_size, r.device)
    rows = state_indices.to(torch.int64)
    working = state_pool.index_select(0, rows)
    output, final_working = _extension().rl_infctx_tmix_wkv7_chunk_fp32io16_forward(
        *chunk_metadata, working, r, decay_logits, k, v, a, b,
        0 if strategy == "materialized" else 1, float(scale), decay_bias,
    )
    return output, state_pool.clone().index_copy(0, rows, final_working)


def rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute(*args, **kwargs):
    """Explicit ``strategy="recompute"`` entry."""
    kwargs["strategy"] = "recompute"
    return rl_infctx_tmix_wkv7_chunk_fp32io16(*args, **kwargs)


__all__ = ["rl_infctx_tmix_wkv7_chunk_fp32io16",
           "rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute"]
