"""fp64 numpy restatement of the WKV7 path's producer / consumer stages —
TEST INFRASTRUCTURE ONLY (imported by tests/ and bench.py's checks, never by
the product).

* ``kk_a_gate_f64``   — csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/
  infer_fp16_forward_varlen.cu (tmix_kk_a_gate_kernel): per (token, head)
  u = k*k_k, kk = u/max(|u|, 1e-12), a = sigmoid(a0 + a12),
  new_k = k*(a*k_a + 1 - k_a), neg_kk = -kk, kka = kk*a.
* ``vres_f64``        — …/lowrank/infer_vres_fp16_forward_varlen.cu:
  value + (v_first - value)*sigmoid(v0 + v12).
* ``readout_prelinear_f64`` — csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cu
  (tmix_lnx_rkvres_xg kernels): per (token, head) group norm with eps 64e-5,
  plus sum(r*k*r_k)*v, times g.
* ``wkv_prepare_f64`` / ``readout_f64`` — the whole stages as
  csrc/sm120/tmix/wkv_prepare/infer_fp16_forward_varlen.cpp:421-530 and
  csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cpp:88-140 compose them
  (dense projections x W^T with optional scaled LoRA, low-rank branches
  tanh(x w1) w2, x a1 a2, sigmoid(x g1) g2, x v1 v2), in fp64 without the
  fp16 rounding of intermediates.

Pinned in tests/test_oracle_prepare.py by invariants and special cases
(unit-norm kk, gate limits, identity cases, group-norm moments, closed-form
residuals, LoRA linearity).
"""

from __future__ import annotations

import numpy as np


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def kk_a_gate_f64(k, k_k, a0, a12, k_a, head_size):
    k, a12 = _f64(k), _f64(a12)
    T, C = k.shape
    H = C // head_size
    u = (k * _f64(k_k)).reshape(T, H, head_size)
    norm = np.sqrt(np.sum(u * u, axis=-1, keepdims=True))
    kk = (u / np.maximum(norm, 1.0e-12)).reshape(T, C)
    a = _sigmoid(_f64(a0) + a12)
    ka = _f64(k_a)
    new_k = k * (a * ka + 1.0 - ka)
    return new_k, -kk, kk * a


def vres_f64(value, v_first, v0, v12):
    value = _f64(value)
    return value + (_f64(v_first) - value) * _sigmoid(_f64(v0) + _f64(v12))


def readout_prelinear_f64(x, r, k, v, r_k, ln_weight, ln_bias, g, head_size):
    x = _f64(x)
    T, C = x.shape
    H = C // head_size
    xh = x.reshape(T, H, head_size)
    mean = xh.mean(axis=-1, keepdims=True)
    var = ((xh - mean) ** 2).mean(axis=-1, keepdims=True)
    norm = ((xh - mean) / np.sqrt(var + 64.0e-5)).reshape(T, C)
    rkv = (_f64(r) * _f64(k) * _f64(r_k)).reshape(T, H, head_size).sum(axis=-1, keepdims=True)
    res = (rkv * _f64(v).reshape(T, H, head_size)).reshape(T, C)
    return (norm * _f64(ln_weight) + _f64(ln_bias) + res) * _f64(g)


def _project(x, weight, lora_a=None, lora_b=None, scale=1.0):
    out = _f64(x) @ _f64(weight).T
    if lora_a is not None:
        out = out + scale * ((_f64(x) @ _f64(lora_a).T) @ _f64(lora_b).T)
    return out


def _rank_in(x, runtime, original):
    return _f64(x) @ (_f64(runtime) if runtime is not None else _f64(original).T)


def _rank_out(h, runtime, original):
    return h @ (_f64(runtime) if runtime is not None else _f64(original).T)


def wkv_prepare_f64(x_r, x_w, x_k, x_v, x_a, x_g, receptance_weight, key_weight, value_weight,
                    w1_t, a1_t, g1_t, v1_t, w2_t, a2_t, g2_t, v2_t, v0, k_k, a0, k_a, *,
                    v_first=None, w1=None, a1=None, g1=None, v1=None, w2=None, a2=None, g2=None,
                    v2=None, lora=None, head_size=64):
    """Eight outputs in the reference's order.  ``lora`` maps 'receptance' /
    'key' / 'value' to (a, b, scale)."""
    lora = lora or {}
    receptance = _project(x_r, receptance_weight, *lora.get("receptance", (None, None, 1.0)))
    key = _project(x_k, key_weight, *lora.get("key", (None, None, 1.0)))
    value = _project(x_v, value_weight, *lora.get("value", (None, None, 1.0)))
    decay = _rank_out(np.tanh(_rank_in(x_w, w1, w1_t)), w2, w2_t)
    a12 = _rank_out(_rank_in(x_a, a1, a1_t), a2, a2_t)
    gate = _rank_out(_sigmoid(_rank_in(x_g, g1, g1_t)), g2, g2_t)
    if v_first is not None:
        v12 = _rank_out(_rank_in(x_v, v1, v1_t), v2, v2_t)
        value = vres_f64(value, v_first, v0, v12)
        returned = _f64(v_first)
    else:
        returned = value
    new_k, neg_kk, kka = kk_a_gate_f64(key, k_k, a0, a12, k_a, head_size)
    return receptance, decay, new_k, value, neg_kk, kka, gate, returned


def readout_f64(x, r, k, v, r_k, ln_weight, ln_bias, g, output_weight, *, lora=None,
                head_size=64, round_prelinear=True):
    """``round_prelinear`` keeps the fp16 store of the fused stage before the
    output projection (the reference's public numerical boundary)."""
    pre = readout_prelinear_f64(x, r, k, v, r_k, ln_weight, ln_bias, g, head_size)
    if round_prelinear:
        pre = pre.astype(np.float16).astype(np.float64)
    out = pre @ _f64(output_weight).T
    if lora is not None:
        a, b, scale = lora
        out = out + scale * ((pre @ _f64(a).T) @ _f64(b).T)
    return out
