"""Writes the golden WKV7 vectors under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The expected values come from a plain numpy fp64 per-token loop written here,
independently of the C oracle (oracle/wkv7_oracle.c), following the reference
recurrence of tests/tmix/wkv7/test.py:29-85 (bias added before the sigmoid,
retention exp(-exp(-1/2) sigmoid(x)) as recurrent_decay.cuh:10-22, sa from the
pre-update state, y from the post-update state, scale on y only, slots
gathered and scattered, untouched slots unchanged).  The C oracle and every
GPU kernel family are then checked against these files.

Inputs are stored as the exact 16-bit token values (uint16 bit patterns), the
states as float32; expected values as float32 (rounded from fp64).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

NAMES = ("r", "decay_logits", "k", "v", "a", "b")


def bits_to_f64(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def f32_to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round-to-nearest-even to bf16 or fp16, returned as uint16 bits."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def recurrence_f64(tok, cu, slots, pool, bias, scale):
    """Per-token fp64 loop over packed sequences; returns (y, new_pool)."""
    r, x, k, v, a, b = tok
    total, H, D = r.shape
    y = np.zeros((total, H, D))
    pool = pool.copy()
    for n in range(len(cu) - 1):
        for h in range(H):
            S = pool[slots[n], h].copy()          # S[key, value]
            for t in range(cu[n], cu[n + 1]):
                xl = x[t, h] + (bias[h] if bias is not None else 0.0)
                w = np.exp(-np.exp(-0.5) / (1.0 + np.exp(-xl)))
                sa = S.T @ a[t, h]
                S = w[:, None] * S + np.outer(b[t, h], sa) + np.outer(k[t, h], v[t, h])
                y[t, h] = scale * (S.T @ r[t, h])
            pool[slots[n], h] = S
    return y, pool


def make_case(name, lengths, heads, dtype, *, seed, slots=None, pool_slots=None, bias=False,
              scale=1.0, u_range=(-6.0, -0.5), state_std=0.1):
    """Inputs drawn with the BASELINE distributions: decay_logits =
    logit(exp(u + 1/2)) so that the retention is exp(-exp(u)); r, k, v ~ N(0,1);
    kk = unit-norm N(0,1); a = -kk; b = kk * sigmoid(N(0,1))."""
    g = np.random.default_rng(seed)
    total, D = int(sum(lengths)), 64
    shape = (total, heads, D)
    u = g.uniform(*u_range, size=shape)
    e = np.exp(u + 0.5)
    logits = np.log(e) - np.log1p(-e)
    kk = g.standard_normal(shape)
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    vals = {"r": g.standard_normal(shape), "decay_logits": logits, "k": g.standard_normal(shape),
            "v": g.standard_normal(shape), "a": -kk,
            "b": kk / (1.0 + np.exp(-g.standard_normal(shape)))}
    bits = {n: f32_to_bits(vals[n], dtype) for n in NAMES}
    n = len(lengths)
    slots = np.arange(n, dtype=np.int32) if slots is None else np.asarray(slots, np.int32)
    pool_slots = pool_slots or int(slots.max()) + 1
    pool = (g.standard_normal((pool_slots, heads, D, D)) * state_std).astype(np.float32)
    bias_bits = f32_to_bits(g.standard_normal((heads, D)) * 0.2, dtype) if bias else None
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    tok = tuple(bits_to_f64(bits[nm], dtype) for nm in NAMES)
    bias_f = None if bias_bits is None else bits_to_f64(bias_bits, dtype)
    y, new_pool = recurrence_f64(tok, cu, slots, pool.astype(np.float64), bias_f, scale)
    out = {f"in_{nm}": bits[nm] for nm in NAMES}
    out.update(cu_seqlens=cu, state_indices=slots, state_pool=pool,
               scale=np.float64(scale), dtype=np.array(dtype),
               y=y.astype(np.float32), new_state_pool=new_pool.astype(np.float32))
    if bias_bits is not None:
        out["in_decay_bias"] = bias_bits
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print(f"wrote {name}.npz: {total} tokens, H={heads}, {dtype}")


CASES = {
    # BASELINE config 0 shape (B=1, T=64, H=4), bf16 token values, zero initial state
    "wkv7_cfg0_B1_T64_H4_bf16": dict(lengths=(64,), heads=4, dtype="bf16", seed=2000,
                                    state_std=0.0),
    # ragged packed batch with permuted slots (one slot untouched), decay bias, scale
    "wkv7_ragged_bias_bf16": dict(lengths=(1, 15, 16, 17, 65, 160), heads=1, dtype="bf16",
                                 seed=2001, slots=(5, 0, 7, 2, 4, 1), pool_slots=9, bias=True,
                                 scale=0.75),
    "wkv7_ragged_fp16": dict(lengths=(3, 33, 130), heads=1, dtype="fp16", seed=2002,
                            slots=(2, 0, 1), scale=1.0),
    # long-memory decay (BASELINE config 4 distribution) over 256 tokens
    "wkv7_long_memory_bf16": dict(lengths=(256,), heads=1, dtype="bf16", seed=2003,
                                 u_range=(-9.0, -4.0), state_std=0.0),
}

if __name__ == "__main__":
    for case_name, kw in CASES.items():
        make_case(case_name, **kw)
