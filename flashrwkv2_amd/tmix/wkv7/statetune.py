"""StateTune: the packed WKV7 recurrence from a trainable initial state.

Public contract of ``flashrwkv2.tmix.wkv7.statetune`` (flashrwkv2/tmix/wkv7/statetune.py:12-236):
the same function, keyword-only ``scale``, error messages and return tuple
``(output, final_state, boundary, state_dot_a)``.  ``boundary`` is the fp32
state at the start of every chunk (``[C,H,D,D]``) and ``state_dot_a`` the fp32
pre-update ``S^T a`` of every token; both are checkpoints for the backward,
which returns gradients for the six token tensors and the initial state.

Beyond the reference's checks, all six token tensors must share one dtype
(the reference's kernel reads every one of them as the dtype of ``r``).
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from . import _extension

_TOKENS = ("r", "decay_logits", "k", "v", "a", "b")
_META = ("sequence_chunk_offsets", "chunk_token_starts", "chunk_token_ends")


def _state_and_token_rows(state, tokens):
    r = tokens[0]
    state_rules = [
        ck.is_tensor(), ck.cuda_contiguous(),
        ck.dtype_in((torch.float32,), "state must be float32"),
        ck.holds(lambda s: s.ndim == 4 and s.shape[0] > 0 and s.shape[1] > 0,
                 "state must have shape [B,H,D,D]"),
        ck.holds(lambda s: s.shape[2] == s.shape[3] and s.shape[2] in (64, 128, 256),
                 "state head size must be 64, 128, or 256"),
    ]
    token_rules = [
        ck.is_tensor(), ck.cuda_contiguous(),
        ck.on_device_of(state, "{name} must share the state device"),
        ck.dtype_in((torch.float16, torch.bfloat16), "{name} must be float16 or bfloat16"),
        ck.matches(r, "{name} must match r shape", device=False),
        ck.holds(lambda t: t.dtype == r.dtype, "{name} must have the dtype of r", TypeError),
    ]
    return [
        ("state", state, state_rules),
        *ck.each(_TOKENS, tokens, token_rules),
        ("r", r, [ck.holds(lambda t: t.ndim == 3 and t.shape[0] > 0
                           and t.shape[1:] == state.shape[1:3],
                           "token tensors must have shape [total_tokens,H,D]")]),
    ]


def _metadata_rows(state, meta):
    offsets, starts, ends = meta
    rules = [ck.is_tensor(), ck.cuda_contiguous(),
             ck.dtype_in((torch.int32,), "{name} must be int32"),
             ck.on_device_of(state, "{name} must share the state device")]
    return [
        *ck.each(_META, meta, rules),
        ("sequence_chunk_offsets", offsets,
         [ck.holds(lambda t: t.ndim == 1, "sequence_chunk_offsets must be one-dimensional")]),
        ("chunk_token_starts", starts,
         [ck.holds(lambda t: t.ndim == 1 and ends.shape == t.shape,
                   "chunk token metadata must have matching shape [C]"),
          ck.holds(lambda t: t.numel() > 0, "at least one training chunk is required")]),
        ("sequence_chunk_offsets", offsets,
         [ck.holds(lambda t: t.numel() == state.shape[0] + 1,
                   "sequence_chunk_offsets must have shape [B+1]")]),
    ]


class _StateTuneWKV7(torch.autograd.Function):
    """Forward with checkpoints; backward to the tokens and the initial state."""

    @staticmethod
    def forward(ctx, scale, initial_state, offsets, starts, ends, *tokens):  # type: ignore[override]
        state = initial_state.detach().contiguous().clone()   # becomes the final state
        r, v = tokens[0], tokens[3]
        out = torch.empty_like(v)
        boundary = state.new_empty((starts.numel(),) + tuple(state.shape[1:]))
        sa = torch.empty_like(r, dtype=torch.float32)
        # At D = 64 in bf16 the native forward runs the chunked MFMA kernels
        # and also returns what its backward reads: the post-16-token state
        # snapshots (uniform layout) or those plus the padded grid's tables
        # (other chunk lists); otherwise None.
        snapshots = _extension().statetune_tmix_wkv7_recurrent_fp32io16_forward(
            offsets, starts, ends, state, *tokens, out, boundary, sa, scale)
        extra = () if snapshots is None else tuple(snapshots) if isinstance(snapshots, tuple) \
            else (snapshots,)
        ctx.scale = scale
        ctx.save_for_backward(offsets, starts, ends, state, *tokens, sa, boundary, *extra)
        ctx.mark_non_differentiable(boundary, sa)
        return out, state, boundary, sa

    @staticmethod
    def backward(ctx, d_out, d_final, _d_boundary, _d_sa):  # type: ignore[override]
        offsets, starts, ends, final, *rest = ctx.saved_tensors
        tokens, (sa, boundary), extra = rest[:6], rest[6:8], rest[8:]
        if d_out is not None:
            d_out = d_out.contiguous().to(tokens[3].dtype)
        if d_final is not None:
            d_final = d_final.contiguous().float()
        d_tokens = [torch.empty_like(t) for t in tokens]
        d_initial = torch.empty_like(final)
        _extension().statetune_tmix_wkv7_recurrent_fp32io16_backward(
            offsets, starts, ends, final, *tokens, sa, d_out, d_final, boundary, *d_tokens,
            d_initial, ctx.scale,
            snapshots=None if not extra else extra[0] if len(extra) == 1 else tuple(extra))
        return (None, d_initial, None, None, None, *d_tokens)


def statetune_tmix_wkv7_recurrent_fp32io16(initial_state, sequence_chunk_offsets,
                                           chunk_token_starts, chunk_token_ends, r,
                                           decay_logits, k, v, a, b, *, scale: float = 1.0):
    """Run StateTune with a nonzero state and direct initial-state gradient
    (statetune.py:202-236 of the reference)."""
    tokens = (r, decay_logits, k, v, a, b)
    meta = (sequence_chunk_offsets, chunk_token_starts, chunk_token_ends)
    ck.verify(_state_and_token_rows(initial_state, tokens))
    ck.verify(_metadata_rows(initial_state, meta))
    ck.verify([("scale", scale, [ck.holds(lambda s: ck.real_number(s) and ck.finite(s),
                                          "scale must be finite")])])
    return _StateTuneWKV7.apply(float(scale), initial_state, *meta, *tokens)


__all__ = ["statetune_tmix_wkv7_recurrent_fp32io16"]
