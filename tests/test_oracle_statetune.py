"""Pins the fp64 StateTune oracle (``oracle.statetune_f64``).

None of these restates its loop:

* with a zero initial state, one chunk per sequence and scale 1 it reduces
  to the packed recurrence ``wkv7_f64`` and its gradients to
  ``pretrain_backward_f64`` (both pinned in test_oracle*.py);
* with a nonzero initial state its outputs and final state equal
  ``wkv7_f64`` run from that state as a slot pool, times ``scale``;
* splitting a chunk in two changes nothing but adds the intermediate state
  as the second chunk's boundary; token rows outside every chunk stay zero;
* central differences of its own forward on
  ``L = sum(y * dy) + sum(S_final * dfinal)`` for every gradient, the
  initial state's included;
* torch autograd of an fp64 loop in the form of the reference's test oracle
  (tests/tmix/wkv7/statetune/test.py:43-91) with the reference's loss
  ``sum(y^2) + sum(S_final^2)``.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle

GRADS = ("dr", "dw", "dk", "dv", "da", "db")


def _tokens(seed, T, H, D, s=0.3):
    rng = np.random.default_rng(seed)
    vals = [(rng.standard_normal((T, H, D)) * s).astype(np.float32) for _ in range(6)]
    vals[1] = (rng.standard_normal((T, H, D)) * 1.5).astype(np.float32)
    return rng, vals


def test_reduces_to_packed_recurrence_and_pretrain_backward():
    B, L, H, D = 2, 11, 2, 8
    rng, vals = _tokens(1, B * L, H, D)
    dy = rng.standard_normal((B * L, H, D)).astype(np.float32)
    offsets = np.arange(B + 1)
    starts, ends = np.arange(B) * L, np.arange(1, B + 1) * L
    out = oracle.statetune_f64(np.zeros((B, H, D, D), np.float32), offsets, starts, ends, *vals,
                               dy=dy)
    y, _, sa, _ = oracle.wkv7_f64(*vals, cu_seqlens=np.arange(B + 1) * L, want_sa=True)
    np.testing.assert_allclose(out["y"], y, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(out["sa"], sa, rtol=1e-13, atol=1e-15)
    assert not np.any(out["boundary"])          # start-of-chunk = zero state
    four = [x.reshape(B, L, H, D) for x in vals]
    ref = oracle.pretrain_backward_f64(*four, dy.reshape(B, L, H, D))
    for name, g in zip(GRADS, ref):
        np.testing.assert_allclose(out[name], g.reshape(B * L, H, D), rtol=1e-11, atol=1e-13,
                                   err_msg=name)


def test_initial_state_and_scale_match_slot_pool():
    B, L, H, D = 3, 7, 1, 8
    rng, vals = _tokens(2, B * L, H, D)
    s0 = (rng.standard_normal((B, H, D, D)) * 0.5).astype(np.float32)
    out = oracle.statetune_f64(s0, np.arange(B + 1), np.arange(B) * L, np.arange(1, B + 1) * L,
                               *vals, scale=0.75)
    y, pool, _, _ = oracle.wkv7_f64(*vals, cu_seqlens=np.arange(B + 1) * L, state_pool=s0,
                                    scale=0.75)
    np.testing.assert_allclose(out["y"], y, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(out["state"], pool, rtol=1e-13, atol=1e-15)
    np.testing.assert_array_equal(out["boundary"], s0.astype(np.float64))


def test_chunk_split_invariance_gaps_and_empty_chunks():
    T, H, D = 20, 2, 6
    rng, vals = _tokens(3, T, H, D)
    s0 = (rng.standard_normal((2, H, D, D)) * 0.3).astype(np.float32)
    dy = rng.standard_normal((T, H, D)).astype(np.float32)
    df = rng.standard_normal((2, H, D, D)).astype(np.float32)
    # sequence 0 = tokens [0, 9), sequence 1 = tokens [12, 20); 9..11 unused
    one = oracle.statetune_f64(s0, [0, 1, 2], [0, 12], [9, 20], *vals, scale=1.3, dy=dy, dfinal=df)
    split = oracle.statetune_f64(s0, [0, 3, 5], [0, 4, 4, 12, 15], [4, 4, 9, 15, 20], *vals,
                                 scale=1.3, dy=dy, dfinal=df)
    for key in ("y", "sa", "state", "dstate0", *GRADS):
        np.testing.assert_allclose(split[key], one[key], rtol=1e-12, atol=1e-14, err_msg=key)
    for key in ("y", "sa", *GRADS):
        assert not np.any(one[key][9:12]), key
    # the split chunks' boundaries are the intermediate states
    mid = oracle.statetune_f64(s0[:1], [0, 1], [0], [4], *vals)["state"][0]
    np.testing.assert_allclose(split["boundary"][1], mid, rtol=1e-13)
    np.testing.assert_allclose(split["boundary"][2], mid, rtol=1e-13)
    np.testing.assert_array_equal(split["boundary"][0], s0[0])


def _loss(s0, vals, dy, df, meta, scale):
    out = oracle.statetune_f64(s0, *meta, *vals, scale=scale)
    return float(np.sum(out["y"] * dy) + np.sum(out["state"] * df))


def test_gradients_match_central_differences():
    T, H, D = 13, 2, 6
    rng, vals = _tokens(4, T, H, D)
    s0 = (rng.standard_normal((2, H, D, D)) * 0.4).astype(np.float32)
    dy = rng.standard_normal((T, H, D)).astype(np.float32)
    df = rng.standard_normal((2, H, D, D)).astype(np.float32)
    meta = ([0, 2, 3], [0, 5, 8], [5, 8, 13])
    out = oracle.statetune_f64(s0, *meta, *vals, scale=0.6, dy=dy, dfinal=df)
    pick = np.random.default_rng(9)
    for which, name in enumerate(GRADS):
        for _ in range(8):
            idx = tuple(int(pick.integers(0, n)) for n in (T, H, D))
            x0 = float(vals[which][idx])
            eps = 2e-3 * max(1.0, abs(x0))
            plus = [v.copy() for v in vals]
            minus = [v.copy() for v in vals]
            plus[which][idx] = np.float32(x0 + eps)
            minus[which][idx] = np.float32(x0 - eps)
            delta = float(plus[which][idx]) - float(minus[which][idx])
            fd = (_loss(s0, plus, dy, df, meta, 0.6) - _loss(s0, minus, dy, df, meta, 0.6)) / delta
            assert math.isclose(out[name][idx], fd, rel_tol=1e-5, abs_tol=1e-7), (name, idx)
    for _ in range(10):
        idx = tuple(int(pick.integers(0, n)) for n in s0.shape)
        x0 = float(s0[idx])
        eps = 2e-3 * max(1.0, abs(x0))
        plus, minus = s0.copy(), s0.copy()
        plus[idx] = np.float32(x0 + eps)
        minus[idx] = np.float32(x0 - eps)
        delta = float(plus[idx]) - float(minus[idx])
        fd = (_loss(plus, vals, dy, df, meta, 0.6) - _loss(minus, vals, dy, df, meta, 0.6)) / delta
        assert math.isclose(out["dstate0"][idx], fd, rel_tol=1e-5, abs_tol=1e-7), ("dstate0", idx)


def _torch_reference(state, meta, r, w, k, v, a, b, scale):
    offsets, starts, ends = meta
    T, H, D = r.shape
    rows = [None] * T
    finals = []
    for s in range(state.shape[0]):
        cur = state[s]
        for c in range(offsets[s], offsets[s + 1]):
            for t in range(starts[c], ends[c]):
                ret = torch.exp(-math.exp(-0.5) / (1.0 + torch.exp(-w[t])))
                dot = torch.einsum("hkv,hk->hv", cur, a[t])
                cur = (ret.unsqueeze(-1) * cur + b[t].unsqueeze(-1) * dot.unsqueeze(-2)
                       + k[t].unsqueeze(-1) * v[t].unsqueeze(-2))
                rows[t] = scale * torch.einsum("hkv,hk->hv", cur, r[t])
        finals.append(cur)
    return torch.stack(rows), torch.stack(finals)


@pytest.mark.parametrize("D", [8, 16])
def test_gradients_match_torch_autograd_of_reference_loss(D):
    """The reference's case shape (B=2, H=1, 5 tokens, chunks [0,1) [1,3) |
    [3,5)) with its loss sum(y^2) + sum(S_final^2); the cotangents the
    oracle takes are then dy = 2y and dfinal = 2 S_final."""
    T, H = 5, 1
    rng, vals = _tokens(20 + D, T, H, D, s=0.5)
    s0 = (rng.standard_normal((2, H, D, D)) * 0.5).astype(np.float32)
    meta = ([0, 2, 3], [0, 1, 3], [1, 3, 5])
    leaves = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (s0, *vals)]
    y, fin = _torch_reference(leaves[0], meta, *leaves[1:], 0.75)
    (y.square().sum() + fin.square().sum()).backward()
    fwd = oracle.statetune_f64(s0, *meta, *vals, scale=0.75)
    np.testing.assert_allclose(fwd["y"], y.detach().numpy(), rtol=1e-12, atol=1e-15)
    out = oracle.statetune_f64(s0, *meta, *vals, scale=0.75, dy=(2 * fwd["y"]).astype(np.float32),
                               dfinal=(2 * fwd["state"]).astype(np.float32))
    # the cotangents went through float32: compare at that precision
    for name, leaf in zip(("dstate0", *GRADS), leaves):
        np.testing.assert_allclose(out[name], leaf.grad.numpy(), rtol=2e-6, atol=1e-8,
                                   err_msg=name)
