"""The WKV7 path's consumer: head group-norm, r.k residual, output gate and
output projection of one TMix layer.

Mirrors ``flashrwkv2.tmix.readout.infer_tmix_readout_forward_varlen``
(flashrwkv2/tmix/readout/__init__.py:10-77): same signature, defaults,
Python-side checks and messages.  The fused normalisation / residual / gate
stage is a HIP kernel whose fp16 result feeds the output projection (a
library GEMM), the same numerical boundary as the reference.
"""

from __future__ import annotations

import torch

from .. import _checks as ck
from ..wkv7 import _extension

_FP16_CONTIGUOUS = "{name} must be contiguous CUDA float16"
_PACKED = ("wkv_output", "receptance", "key", "value", "gate")
_PER_CHANNEL = ("r_k", "ln_weight", "ln_bias")


def _rows(packed, per_channel, output_weight, lora, head_size):
    ref = packed[0]
    rows = [("head_size", head_size, [ck.holds(lambda n: n in (64, 128, 256),
                                               "head_size must be one of 64, 128, or 256")])]
    rows += ck.each(_PACKED, packed, [
        ck.is_tensor(),
        ck.cuda_contiguous_of(torch.float16, _FP16_CONTIGUOUS),
        ck.matches(ref, "{name} must match wkv_output's packed shape and device"),
    ])
    rows.append(("wkv_output", ref, [ck.holds(
        lambda t: t.ndim == 2 and t.shape[0] > 0 and t.shape[1] % head_size == 0,
        "wkv_output must have packed shape [total_tokens,H*head_size]")]))
    channels = lambda: ref.shape[1]   # noqa: E731  (read after the layout rows)
    rows += ck.each(_PER_CHANNEL, per_channel, [
        ck.cuda_contiguous_of(torch.float16, _FP16_CONTIGUOUS),
        ck.holds(lambda t: t.device == ref.device and tuple(t.shape) == (channels(),),
                 "{name} must have shape [C] on wkv_output's device"),
    ])
    rows.append(("output_weight", output_weight, [
        ck.cuda_contiguous_of(torch.float16, _FP16_CONTIGUOUS),
        ck.holds(lambda w: w.device == ref.device and tuple(w.shape) == (channels(),) * 2,
                 "{name} must have shape [C,C]"),
    ]))
    rows.append(("output", lora, [ck.holds(lambda p: (p[0] is None) == (p[1] is None),
                                           "{name}_lora_a and {name}_lora_b must be provided "
                                           "together")]))
    return rows


def infer_tmix_readout_forward_varlen(
    wkv_output: torch.Tensor,
    receptance: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    r_k: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    gate: torch.Tensor,
    output_weight: torch.Tensor,
    *,
    output_lora_a: torch.Tensor | None = None,
    output_lora_b: torch.Tensor | None = None,
    output_lora_scale: float = 1.0,
    head_size: int = 64,
    batch_size: int = 1,
    max_seqlen: int | None = None,
) -> torch.Tensor:
    """Run head normalization, RKV residual, gate and output projection."""
    ck.verify(_rows((wkv_output, receptance, key, value, gate), (r_k, ln_weight, ln_bias),
                    output_weight, (output_lora_a, output_lora_b), head_size))
    if max_seqlen is None:
        max_seqlen = wkv_output.shape[0]
    return _extension().tmix_readout_forward_varlen(
        wkv_output, receptance, key, value, r_k, ln_weight, ln_bias, gate, output_weight,
        output_lora_a, output_lora_b, float(output_lora_scale), int(head_size),
        int(batch_size), int(max_seqlen),
    )


__all__ = ["infer_tmix_readout_forward_varlen"]
