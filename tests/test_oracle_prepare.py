"""Pins oracle/prepare.py (producer / consumer stages) by invariants and
special cases, none of which restates its formulas:

* kk is unit-norm per head and points along -(k * k_k); scaling k leaves it
  unchanged; a zero head gives zeros (the 1e-12 floor, no NaN);
* k_a = 0 leaves the key unchanged, k_a = 1 multiplies it by the a gate, and
  the gate saturates to 0 / 1 for a0 -> -inf / +inf;
* the value residual is the identity when v_first == value and selects
  v_first / value at the gate's limits, the midpoint at zero logits;
* the readout's group norm has zero mean and variance var / (var + 64e-5)
  per head; ln_bias shifts it; the r.k residual reduces to v * g for
  r = k = 1, r_k = 1/D and a constant WKV output;
* the dense projection with LoRA is linear in the LoRA scale, and the
  low-rank branches use the two weight layouts interchangeably.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import prepare as P

RNG = np.random.default_rng(42)


def _r(*shape, s=1.0):
    return RNG.standard_normal(shape) * s


@pytest.mark.parametrize("D", [64, 128, 256])
def test_kk_unit_norm_direction_and_scale_invariance(D):
    T, H = 3, 2
    C = H * D
    k, k_k, a0, a12, k_a = _r(T, C), _r(C), _r(C), _r(T, C), RNG.random(C)
    new_k, neg_kk, kka = P.kk_a_gate_f64(k, k_k, a0, a12, k_a, D)
    kk = -neg_kk.reshape(T, H, D)
    np.testing.assert_allclose(np.linalg.norm(kk, axis=-1), 1.0, rtol=1e-12)
    u = (k * k_k).reshape(T, H, D)
    cos = np.sum(kk * u, axis=-1) / np.linalg.norm(u, axis=-1)
    np.testing.assert_allclose(cos, 1.0, rtol=1e-12)
    _, neg2, _ = P.kk_a_gate_f64(3.7 * k, k_k, a0, a12, k_a, D)
    np.testing.assert_allclose(neg2, neg_kk, rtol=1e-12, atol=1e-15)
    # kka / neg_kk = -gate, the same gate for every element of the head
    gate = -kka / neg_kk
    assert np.all((gate > 0) & (gate < 1))


def test_kk_zero_head_is_finite_and_zero():
    D = 64
    k = np.zeros((1, D))
    new_k, neg_kk, kka = P.kk_a_gate_f64(k, np.ones(D), np.zeros(D), np.zeros((1, D)),
                                         np.zeros(D), D)
    assert np.all(np.isfinite(neg_kk)) and not np.any(neg_kk) and not np.any(kka)


def test_key_gate_identity_and_limits():
    D, T = 64, 4
    k, k_k, a12 = _r(T, D), _r(D), _r(T, D)
    new_k, _, _ = P.kk_a_gate_f64(k, k_k, _r(D), a12, np.zeros(D), D)
    np.testing.assert_allclose(new_k, k, rtol=0, atol=0)
    big = np.full(D, 60.0)
    new_k, neg_kk, kka = P.kk_a_gate_f64(k, k_k, big, a12, np.ones(D), D)
    np.testing.assert_allclose(new_k, k, rtol=1e-12)          # gate -> 1
    np.testing.assert_allclose(kka, -neg_kk, rtol=1e-12)
    new_k, _, kka = P.kk_a_gate_f64(k, k_k, -big, a12, np.ones(D), D)
    np.testing.assert_allclose(new_k, 0.0, atol=1e-20)        # gate -> 0
    np.testing.assert_allclose(kka, 0.0, atol=1e-20)


def test_value_residual_identity_limits_and_midpoint():
    T, C = 3, 128
    value, first, v12 = _r(T, C), _r(T, C), _r(T, C)
    np.testing.assert_allclose(P.vres_f64(value, value, _r(C), v12), value, rtol=1e-15)
    np.testing.assert_allclose(P.vres_f64(value, first, np.full(C, 80.0), np.zeros((T, C))),
                               first, rtol=1e-12)
    np.testing.assert_allclose(P.vres_f64(value, first, np.full(C, -80.0), np.zeros((T, C))),
                               value, rtol=1e-12)
    np.testing.assert_allclose(P.vres_f64(value, first, np.zeros(C), np.zeros((T, C))),
                               0.5 * (value + first), rtol=1e-12)


@pytest.mark.parametrize("D", [64, 256])
def test_readout_group_norm_moments_and_bias(D):
    T, H = 5, 3
    C = H * D
    x = _r(T, C, s=0.3) + 2.0
    zeros, ones = np.zeros((T, C)), np.ones((T, C))
    out = P.readout_prelinear_f64(x, zeros, zeros, zeros, np.zeros(C), np.ones(C), np.zeros(C),
                                  ones, D).reshape(T, H, D)
    xh = x.reshape(T, H, D)
    var = xh.var(axis=-1)
    np.testing.assert_allclose(out.mean(axis=-1), 0.0, atol=1e-12)
    np.testing.assert_allclose(out.var(axis=-1), var / (var + 64e-5), rtol=1e-10)
    bias = _r(C)
    shifted = P.readout_prelinear_f64(x, zeros, zeros, zeros, np.zeros(C), np.ones(C), bias,
                                      ones, D)
    np.testing.assert_allclose(shifted - out.reshape(T, C), np.broadcast_to(bias, (T, C)),
                               atol=1e-12)


def test_readout_residual_closed_form():
    D, H, T = 64, 2, 3
    C = H * D
    x = np.ones((T, C))                       # constant per head: normalises to 0
    v, g = _r(T, C), _r(T, C)
    out = P.readout_prelinear_f64(x, np.ones((T, C)), np.ones((T, C)), v, np.full(C, 1.0 / D),
                                  np.ones(C), np.zeros(C), g, D)
    np.testing.assert_allclose(out, v * g, rtol=1e-12)


def test_projection_lora_linearity_and_rank_layouts():
    T, C, R, Rl = 3, 64, 8, 4
    x, W, A, B = _r(T, C), _r(C, C), _r(Rl, C), _r(C, Rl)
    base = P._project(x, W)
    one = P._project(x, W, A, B, 1.0)
    half = P._project(x, W, A, B, 0.5)
    np.testing.assert_allclose(half - base, 0.5 * (one - base), rtol=1e-10, atol=1e-12)
    w_orig = _r(R, C)
    np.testing.assert_allclose(P._rank_in(x, w_orig.T.copy(), None), P._rank_in(x, None, w_orig),
                               rtol=1e-13)
    h, w2_orig = _r(T, R), _r(C, R)
    np.testing.assert_allclose(P._rank_out(h, w2_orig.T.copy(), None),
                               P._rank_out(h, None, w2_orig), rtol=1e-13)


def test_wkv_prepare_first_layer_returns_value_as_v_first():
    T, C, R, D = 2, 128, 8, 64
    xs = [_r(T, C, s=0.1) for _ in range(6)]
    dense = [_r(C, C, s=0.05) for _ in range(3)]
    r_in = [_r(R, C, s=0.1) for _ in range(4)]
    r_out = [_r(C, R, s=0.1) for _ in range(4)]
    vec = [_r(C, s=0.1) for _ in range(4)]
    out = P.wkv_prepare_f64(*xs, *dense, *r_in, *r_out, *vec, head_size=D)
    assert len(out) == 8
    np.testing.assert_array_equal(out[7], out[3])
    later = P.wkv_prepare_f64(*xs, *dense, *r_in, *r_out, *vec, v_first=out[7], head_size=D)
    # v_first equal to the layer's own value: the residual is the identity
    np.testing.assert_allclose(later[3], out[3], rtol=1e-13)
