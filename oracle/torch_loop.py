"""Pure-torch per-token WKV7 recurrence in fp32 — TEST INFRASTRUCTURE ONLY.

The form of the reference's own test oracle (tests/tmix/wkv7/test.py:66-83:
one Python iteration per token, the state as a [H, D, D] tensor, the decay
from the logits by csrc/sm120/tmix/wkv7/recurrent_decay.cuh:10-22), here
vectorised over heads.  ``bench.py`` times it on the host as the planned
pure-torch CPU baseline (config 0 and one config-2 decode step); it is
checked against the fp64 C oracle in tests/test_oracle.py.
"""

from __future__ import annotations

import math

import torch

_C = math.exp(-0.5)


def wkv7_torch_loop(r, decay_logits, k, v, a, b, state, *, scale: float = 1.0):
    """One sequence: token tensors [T, H, D], state [H, D, D] (k rows, v
    columns), all fp32.  Returns (y [T, H, D], final state); `state` is not
    modified."""
    w = torch.exp(-_C * torch.sigmoid(decay_logits))
    s = state.clone()
    y = torch.empty_like(v)
    for t in range(r.shape[0]):
        sa = torch.einsum("hkv,hk->hv", s, a[t])
        s = (s * w[t].unsqueeze(-1) + b[t].unsqueeze(-1) * sa.unsqueeze(1)
             + k[t].unsqueeze(-1) * v[t].unsqueeze(1))
        y[t] = scale * torch.einsum("hkv,hk->hv", s, r[t])
    return y, s


def wkv7_torch_packed(r, decay_logits, k, v, a, b, cu_seqlens, states, *, scale: float = 1.0):
    """Packed sequences [ΣT, H, D] with per-sequence states [N, H, D, D]
    (sequence n uses states[n]); returns (y, final states)."""
    y = torch.empty_like(v)
    out = torch.empty_like(states)
    for n in range(len(cu_seqlens) - 1):
        lo, hi = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
        y[lo:hi], out[n] = wkv7_torch_loop(r[lo:hi], decay_logits[lo:hi], k[lo:hi], v[lo:hi],
                                           a[lo:hi], b[lo:hi], states[n], scale=scale)
    return y, out
