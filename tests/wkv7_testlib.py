"""Shared helpers of the WKV7 test-suite: seeded cases, tolerances and the
comparison against the CPU oracle (oracle/, test infrastructure)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

# fp32-state recurrent gates of the reference (tests/fixtures/tolerances-v1.json:9-12):
# relative RMSE (tests/tmix/wkv7/test.py:164-167) <= 2e-3 for output and state.
OUTPUT_REL_RMSE = 2.0e-3
STATE_REL_RMSE = 2.0e-3
# Per-element output bound, normalised by max(1, |y_ref|), and per-(sequence,
# head) Frobenius state bound, both against the fp64 oracle.
OUTPUT_MAX_NORM = 2.0e-2
STATE_FRO_REL = 1.0e-3


def gpu_available() -> bool:
    return torch.cuda.is_available()


def require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("MI355X GPU required")
    import flashrwkv2_amd

    assert flashrwkv2_amd._C is not None, "GPU present but the HIP backend did not load"
    return flashrwkv2_amd._C


def relative_rmse(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    base = max(np.sqrt(np.mean(e * e)), 1.0e-6)
    return float(np.sqrt(np.mean((a - e) ** 2)) / base)


def max_norm_err(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(1.0, np.abs(e)))) if e.size else 0.0


def state_fro_rel(actual, expected) -> float:
    """max over leading (slot, head) of ||dS||_F / max(||S||_F, 1e-6)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    a = a.reshape(-1, a.shape[-2] * a.shape[-1])
    e = e.reshape(-1, e.shape[-2] * e.shape[-1])
    num = np.linalg.norm(a - e, axis=1)
    den = np.maximum(np.linalg.norm(e, axis=1), 1.0e-6)
    return float(np.max(num / den)) if num.size else 0.0


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def make_case(*, dtype=torch.bfloat16, head_size=64, lengths=(1, 15, 16, 17, 65),
              with_decay_bias=False, num_heads=2, state_pool_slots=None, seed=None,
              scales=(0.12, 3.5, 0.06, 0.06, 0.06, 0.06), state_scale=0.03,
              device="cuda"):
    """Packed case shaped like the reference's _make_case
    (tests/tmix/wkv7/test.py:170-230): slots [5,0,7,2,4] for <= 5 sequences,
    pool of max(9, n) slots, the same per-tensor scales; drawn on the CPU
    from our own seed and moved to `device`."""
    g = torch.Generator().manual_seed(seed if seed is not None
                                      else 20260804 + head_size + int(with_decay_bias))
    total = sum(lengths)
    n = len(lengths)
    slots_n = state_pool_slots if state_pool_slots is not None else max(9, n)
    shape = (total, num_heads, head_size)
    names = ("r", "decay_logits", "k", "v", "a", "b")
    case = {name: (torch.randn(shape, generator=g) * s).to(dtype).to(device)
            for name, s in zip(names, scales)}
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    case["cu_seqlens"] = torch.tensor(offsets, dtype=torch.int32, device=device)
    if n <= 5:
        slots = torch.tensor([5, 0, 7, 2, 4][:n], dtype=torch.int32)
    else:
        slots = torch.arange(n, dtype=torch.int32)
    case["state_indices"] = slots.to(device)
    case["state_pool"] = (torch.randn((slots_n, num_heads, head_size, head_size), generator=g)
                          * state_scale).float().to(device)
    case["decay_bias"] = None
    if with_decay_bias:
        case["decay_bias"] = (torch.randn((num_heads, head_size), generator=g) * 0.2).to(
            dtype).to(device)
    return case


def tokens(case):
    return tuple(case[n] for n in ("r", "decay_logits", "k", "v", "a", "b"))


def oracle_expect(case, *, scale=1.0, state_pool=None):
    """fp64 oracle on exactly the kernel's (rounded) inputs."""
    pool = case["state_pool"] if state_pool is None else state_pool
    y, new_pool, _, _ = oracle.wkv7_f64(
        *(to_np(t) for t in tokens(case)),
        cu_seqlens=case["cu_seqlens"].cpu().numpy(),
        state_indices=case["state_indices"].cpu().numpy(),
        state_pool=to_np(pool),
        decay_bias=None if case["decay_bias"] is None else to_np(case["decay_bias"]),
        scale=scale)
    return y, new_pool


def assert_output_close(actual, expected, *, rmse=OUTPUT_REL_RMSE, max_norm=OUTPUT_MAX_NORM):
    a = to_np(actual) if isinstance(actual, torch.Tensor) else actual
    assert np.isfinite(a).all(), "non-finite output"
    rr = relative_rmse(a, expected)
    mn = max_norm_err(a, expected)
    assert rr <= rmse, f"output relative RMSE {rr:.3e} > {rmse:.1e}"
    assert mn <= max_norm, f"output max |dy|/max(1,|y|) {mn:.3e} > {max_norm:.1e}"


def assert_state_close(actual, expected, *, rmse=STATE_REL_RMSE, fro=STATE_FRO_REL):
    a = to_np(actual) if isinstance(actual, torch.Tensor) else actual
    assert np.isfinite(a).all(), "non-finite state"
    rr = relative_rmse(a, expected)
    fr = state_fro_rel(a, expected)
    assert rr <= rmse, f"state relative RMSE {rr:.3e} > {rmse:.1e}"
    assert fr <= fro, f"state Frobenius relative error {fr:.3e} > {fro:.1e}"
