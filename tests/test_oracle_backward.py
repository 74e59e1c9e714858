"""Pins the fp64 backward oracle (``oracle.pretrain_backward_f64``).

Two checks that do not restate its adjoint formulas:

* central differences of the fp64 forward oracle ``wkv7_f64`` (itself pinned in
  test_oracle.py) on ``L = sum(y * dy)``, for sampled elements of every input;
  a dropped term, a transposed operand or a sign error in any gradient moves
  it far outside the 1e-5 relative bound;
* torch autograd of an independent fp64 per-token loop written with einsum
  (the form of the reference's own test oracle,
  tests/tmix/wkv7/pretrain/test.py:44-65), compared on every element.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle

NAMES = ("r", "w", "k", "v", "a", "b")


def _case(seed, B, T, H, D, scale=0.4):
    rng = np.random.default_rng(seed)
    shape = (B, T, H, D)
    vals = [(rng.standard_normal(shape) * scale).astype(np.float32) for _ in range(6)]
    vals[1] = (rng.standard_normal(shape) * 1.5).astype(np.float32)  # decay logits
    dy = rng.standard_normal(shape).astype(np.float32)
    return vals, dy


def _loss(vals, dy):
    B, T, H, D = vals[0].shape
    flat = [x.reshape(B * T, H, D) for x in vals]
    cu = np.arange(B + 1, dtype=np.int32) * T
    y, *_ = oracle.wkv7_f64(*flat, cu_seqlens=cu)
    return float(np.sum(y * dy.reshape(B * T, H, D).astype(np.float64)))


def test_backward_oracle_matches_central_differences():
    vals, dy = _case(11, 2, 21, 2, 8)
    grads = oracle.pretrain_backward_f64(*vals, dy)
    rng = np.random.default_rng(5)
    for which, g in enumerate(grads):
        for _ in range(12):
            idx = tuple(int(rng.integers(0, n)) for n in vals[0].shape)
            x0 = float(vals[which][idx])
            eps = 2e-3 * max(1.0, abs(x0))
            plus = [v.copy() for v in vals]
            minus = [v.copy() for v in vals]
            plus[which][idx] = np.float32(x0 + eps)
            minus[which][idx] = np.float32(x0 - eps)
            delta = float(plus[which][idx]) - float(minus[which][idx])
            fd = (_loss(plus, dy) - _loss(minus, dy)) / delta
            assert math.isclose(g[idx], fd, rel_tol=1e-5, abs_tol=1e-7), (NAMES[which], idx, g[idx], fd)


def _torch_loop(r, w, k, v, a, b):
    B, T, H, D = r.shape
    state = torch.zeros((B, H, D, D), dtype=torch.float64)
    out = []
    for t in range(T):
        ret = torch.exp(-math.exp(-0.5) / (1.0 + torch.exp(-w[:, t])))
        sa = torch.einsum("bhkv,bhk->bhv", state, a[:, t])
        state = (state * ret.unsqueeze(-1) + b[:, t].unsqueeze(-1) * sa.unsqueeze(-2)
                 + k[:, t].unsqueeze(-1) * v[:, t].unsqueeze(-2))
        out.append(torch.einsum("bhkv,bhk->bhv", state, r[:, t]))
    return torch.stack(out, dim=1)


@pytest.mark.parametrize("B,T,H,D", [(1, 16, 1, 16), (2, 33, 2, 12)])
def test_backward_oracle_matches_torch_autograd(B, T, H, D):
    vals, dy = _case(100 + T, B, T, H, D)
    grads = oracle.pretrain_backward_f64(*vals, dy)
    leaves = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in vals]
    y = _torch_loop(*leaves)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    for name, leaf, g in zip(NAMES, leaves, grads):
        np.testing.assert_allclose(g, leaf.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)


def test_backward_oracle_zero_cotangent_and_causality():
    """dy = 0 gives zero gradients; dy only on the last token leaves dv, dk
    of earlier tokens generally nonzero but gives dr = 0 before it (y_t
    depends on r only at t)."""
    vals, dy = _case(3, 1, 9, 1, 6)
    for g in oracle.pretrain_backward_f64(*vals, np.zeros_like(dy)):
        assert not np.any(g)
    dy_last = np.zeros_like(dy)
    dy_last[:, -1] = dy[:, -1]
    dr, dw, dk, dv, da, db = oracle.pretrain_backward_f64(*vals, dy_last)
    assert not np.any(dr[:, :-1])
    assert np.all(np.abs(dv[:, :-1]).sum(axis=-1) > 0)
