"""The recurrence with wkv_prepare's kk / a-gate stage folded into it, and
optionally the readout's elementwise stage folded into its write-back.

In the reference the gate runs as its own kernel
(csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/infer_fp16_forward_varlen.cu):
it reads the projected key and the a-gate logits and writes the gated key,
a = -kk and b = kk * sigmoid(a0 + a12), which the recurrence then reads back.
Here the chunked recurrence forms k, a and b in its load stage and writes
only the gated key (the readout's input), so a and b never reach HBM.  The
result equals running ``tmix_wkv_prepare``'s gate stage and then
``infer_tmix_wkv7_recurrent_fp32io16_forward_varlen`` on its outputs, up to
the fp16/bf16 rounding of a and b that the fused form skips.
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from . import (
    _check_metadata_inputs,
    _extension,
    _validate_packed_inputs,
    _validate_state,
    prepare_tmix_wkv7_recurrent_metadata,
)


def infer_tmix_wkv7_kk_gate_recurrent_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    a12: torch.Tensor,
    *,
    k_k: torch.Tensor,
    a0: torch.Tensor,
    k_a: torch.Tensor,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns ``(output, gated_key)``; ``state_pool`` is updated in place.

    ``key`` is the projected key before the gate, ``a12`` the low-rank a-gate
    logits (both ``[total_tokens,H,D]``), ``k_k``, ``a0``, ``k_a`` the
    per-channel parameters (``[H*D]`` or ``[H,D]``), all in the token dtype.
    """
    _validate_packed_inputs(r, decay_logits, key, value, a12, a12)
    _validate_state(state_pool)
    _check_metadata_inputs(cu_seqlens, state_indices)
    ck.verify(ck.each(("k_k", "a0", "k_a"), (k_k, a0, k_a), [ck.is_tensor()]))
    ticket = validated_metadata
    if ticket is None:
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            cu_seqlens, state_indices, total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0], max_seqlen=max_seqlen)
    output = torch.empty_like(value)
    gated = torch.empty_like(key)
    _extension().tmix_wkv7_recurrent_fp32_from_kk_gate(
        cu_seqlens, state_indices, state_pool, r, decay_logits, key, value, a12, k_k, a0, k_a,
        gated, output, float(scale), decay_bias, ticket,
        -1 if max_seqlen is None else int(max_seqlen))
    return output, gated


def infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    a12: torch.Tensor,
    gate: torch.Tensor,
    *,
    k_k: torch.Tensor,
    a0: torch.Tensor,
    k_a: torch.Tensor,
    r_k: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
    return_wkv_output: bool = False,
):
    """The kk / a gate, the recurrence and the readout's elementwise stage in
    one kernel.  Returns ``(readout, gated_key)`` (plus the recurrence output
    ``y`` when ``return_wkv_output``); ``state_pool`` is updated in place.

    ``readout`` is what the reference's readout stage
    (csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cu) hands to the output
    projection: per (token, head), ``(GroupNorm(y) * ln_weight + ln_bias +
    (sum r k' r_k) * v) * gate`` with the group norm over the head's channels
    of ``y`` as rounded to the token dtype (eps 64e-5).  ``gate`` is
    ``[total_tokens,H,D]``; ``r_k``, ``ln_weight``, ``ln_bias`` are ``[H*D]``
    or ``[H,D]``; all in the token dtype.
    """
    _validate_packed_inputs(r, decay_logits, key, value, a12, gate)
    _validate_state(state_pool)
    _check_metadata_inputs(cu_seqlens, state_indices)
    ck.verify(ck.each(("k_k", "a0", "k_a", "r_k", "ln_weight", "ln_bias"),
                      (k_k, a0, k_a, r_k, ln_weight, ln_bias), [ck.is_tensor()]))
    ticket = validated_metadata
    if ticket is None:
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            cu_seqlens, state_indices, total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0], max_seqlen=max_seqlen)
    readout = torch.empty_like(value)
    gated = torch.empty_like(key)
    y = torch.empty_like(value) if return_wkv_output else None
    _extension().tmix_wkv7_recurrent_fp32_from_kk_gate_readout(
        cu_seqlens, state_indices, state_pool, r, decay_logits, key, value, a12, gate, k_k, a0,
        k_a, r_k, ln_weight, ln_bias, gated, readout, y, float(scale), decay_bias, ticket,
        -1 if max_seqlen is None else int(max_seqlen))
    if return_wkv_output:
        return readout, gated, y
    return readout, gated


__all__ = ["infer_tmix_wkv7_kk_gate_recurrent_forward_varlen",
           "infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen"]
