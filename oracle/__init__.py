"""CPU oracle for the WKV7 path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the
timed CPU baseline).  The product path (``flashrwkv2_amd``) never imports it.

The arithmetic lives in ``wkv7_oracle.c`` (built by ``make -C oracle`` into
``oracle/_build/libwkv7_oracle.so``); this module binds it with ctypes and
adds numpy conveniences.  What each function restates:

* ``retention``    — csrc/sm120/tmix/wkv7/recurrent_decay.cuh:10-22
* ``wkv7_f64``     — tests/tmix/wkv7/test.py:29-85 (packed varlen, slots,
  decay_bias, scale) and, with ``boundary_len``/``want_sa``, the post-chunk
  boundary and state_dot_a of
  csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cu:32-97
* ``pretrain_backward_f64`` — reverse-mode gradients of the ``[B,T,H,D]``
  zero-state path, the backward of
  csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cu:163-286; pinned in
  tests/test_oracle_backward.py by central differences of ``wkv7_f64`` and
  by torch autograd of an fp64 per-token loop.
* ``statetune_f64`` — the trainable-initial-state recurrence over a chunk
  list, csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cu:32-131
  (start-of-chunk boundary, state_dot_a, scale) and the gradients its
  backward (statetune_recurrent_fp32io16_backward.cu:50-240) returns,
  including the initial state's; pinned in tests/test_oracle_statetune.py
  by the pretrain oracle (zero state, one chunk), chunk-split invariance,
  state linearity, central differences and torch autograd.
* ``prepare`` (numpy, ``oracle/prepare.py``) — the producer / consumer
  stages either side of the recurrence (wkv_prepare's kk / a gate, low-rank
  branches and value residual; readout's group norm, residual, gate and
  projection); pinned in tests/test_oracle_prepare.py.
* ``wkv7_cpu_f32`` — the same recurrence in float, OpenMP over
  (sequence, head): the CPU baseline that bench.py times.
* ``albatross_dither`` / ``wkv7_fp16_state`` (numpy) — the FP16-state
  contract: csrc/sm120/tmix/wkv7/recurrent_decay.cuh:36-46 and
  tests/tmix/wkv7/test.py:88-149 (delta = fp16(w - 1 + dither(phase)), the
  update S + S*delta + b*sa + k*v rounded to fp16 each token, y from the
  rounded state, elapsed phase base per slot); pinned in
  tests/test_oracle_fp16.py.

How the oracle is pinned (tests/test_oracle.py): the retention against its
closed form and limits; the recurrence against an explicit-matrix fp64 form
(S_t = (diag w_t + b_t a_t^T) S_{t-1} + k_t v_t^T), the prefix-sum linear
attention closed form (a = b = 0, w = 1), pure decay (k = a = b = 0),
the idempotent projection (w = 1, b = -a = kk, |kk| = 1), split/packing/slot
invariance, scale linearity, boundary snapshots vs split runs, and the
committed golden fixture of BASELINE config 0.  The reference ships no golden
vectors for this path (its only fixture is tests/fixtures/tolerances-v1.json).
"""

from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_double, c_int, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libwkv7_oracle.so"

_lib: ctypes.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        lib.wkv7_oracle_retention.restype = c_double
        lib.wkv7_oracle_retention.argtypes = [c_double]
        lib.wkv7_oracle_f64.restype = None
        lib.wkv7_oracle_f64.argtypes = [c_int, c_int, c_int] + [c_void_p] * 10 + [
            c_double, c_void_p, c_void_p, c_void_p, c_int, c_int]
        lib.wkv7_cpu_f32.restype = None
        lib.wkv7_cpu_f32.argtypes = [c_int, c_int, c_int] + [c_void_p] * 10 + [
            c_double, c_void_p, c_int]
        lib.wkv7_oracle_pretrain_bwd_f64.restype = None
        lib.wkv7_oracle_pretrain_bwd_f64.argtypes = [c_int] * 4 + [c_void_p] * 13
        lib.wkv7_oracle_statetune_f64.restype = None
        lib.wkv7_oracle_statetune_f64.argtypes = [c_int] * 4 + [c_void_p] * 10 + [
            c_double] + [c_void_p] * 13
        lib.wkv7_cpu_max_threads.restype = c_int
        lib.wkv7_cpu_max_threads.argtypes = []
        _lib = lib
    return _lib


def _p(x: np.ndarray | None):
    return None if x is None else x.ctypes.data


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def retention(x: float) -> float:
    return _load().wkv7_oracle_retention(float(x))


def wkv7_f64(r, logits, k, v, a, b, *, cu_seqlens, state_indices=None, state_pool=None,
             decay_bias=None, scale=1.0, want_sa=False, boundary_len=0):
    """fp64 evaluation of the packed recurrence.

    Token arrays are ``[total, H, D]`` (any float dtype; widened from the
    values they hold).  Returns ``(y, pool, sa, boundary)`` as float64; ``pool``
    is a copy of ``state_pool`` with the touched slots updated (``None`` when
    no pool was given: zero initial states).  ``boundary`` is
    ``[n, H, L/boundary_len, D, D]`` for uniform lengths L.
    """
    arrs = [_f32(t) for t in (r, logits, k, v, a, b)]
    total, H, D = arrs[0].shape
    cu = _i32(cu_seqlens)
    n = cu.size - 1
    slots = None if state_indices is None else _i32(state_indices)
    pool = None if state_pool is None else np.array(state_pool, dtype=np.float64, order="C")
    bias = None if decay_bias is None else _f32(decay_bias).reshape(H, D)
    y = np.zeros((total, H, D), dtype=np.float64)
    sa = np.zeros((total, H, D), dtype=np.float64) if want_sa else None
    boundary = None
    per_seq = 0
    if boundary_len:
        lens = np.diff(cu)
        per_seq = int(lens.max()) // boundary_len
        boundary = np.zeros((n, H, per_seq, D, D), dtype=np.float64)
    _load().wkv7_oracle_f64(n, H, D, _p(cu), _p(slots), _p(pool), *(_p(t) for t in arrs[:2]),
                            _p(bias), *(_p(t) for t in arrs[2:]), float(scale), _p(y), _p(sa),
                            _p(boundary), int(boundary_len or 1), per_seq)
    return y, pool, sa, boundary


def wkv7_cpu_f32(r, logits, k, v, a, b, *, cu_seqlens, state_indices=None, state_pool=None,
                 decay_bias=None, scale=1.0, threads=0):
    """fp32 CPU recurrence (the timed baseline).  Returns ``(y, pool)``."""
    arrs = [_f32(t) for t in (r, logits, k, v, a, b)]
    total, H, D = arrs[0].shape
    cu = _i32(cu_seqlens)
    slots = None if state_indices is None else _i32(state_indices)
    pool = None if state_pool is None else np.array(state_pool, dtype=np.float32, order="C")
    bias = None if decay_bias is None else _f32(decay_bias).reshape(H, D)
    y = np.zeros((total, H, D), dtype=np.float32)
    _load().wkv7_cpu_f32(cu.size - 1, H, D, _p(cu), _p(slots), _p(pool),
                         *(_p(t) for t in arrs[:2]), _p(bias), *(_p(t) for t in arrs[2:]),
                         float(scale), _p(y), int(threads))
    return y, pool


def pretrain_backward_f64(r, logits, k, v, a, b, dy):
    """fp64 gradients of ``sum(y * dy)`` for the ``[B,T,H,D]`` zero-state path.

    Returns ``(dr, dlogit, dk, dv, da, db)`` as float64 ``[B,T,H,D]``.
    """
    arrs = [_f32(t) for t in (r, logits, k, v, a, b, dy)]
    B, T, H, D = arrs[0].shape
    outs = [np.zeros((B, T, H, D), dtype=np.float64) for _ in range(6)]
    _load().wkv7_oracle_pretrain_bwd_f64(B, T, H, D, *(_p(t) for t in arrs),
                                         *(_p(o) for o in outs))
    return tuple(outs)


def statetune_f64(state0, offsets, starts, ends, r, logits, k, v, a, b, *, scale=1.0,
                  dy=None, dfinal=None):
    """fp64 StateTune forward and backward over a chunk list.

    ``state0`` is ``[B,H,D,D]``, the token tensors ``[T,H,D]``; ``offsets``
    ``[B+1]`` index the chunk list ``starts`` / ``ends`` ``[C]``.  Returns a
    dict with ``y``, ``sa``, ``boundary`` (start-of-chunk states), ``state``
    (final) and the gradients ``dr, dw, dk, dv, da, db, dstate0`` of
    ``sum(y * dy) + sum(state * dfinal)`` (token rows outside every chunk
    are zero in every per-token output).
    """
    arrs = [_f32(t) for t in (r, logits, k, v, a, b)]
    T, H, D = arrs[0].shape
    s0 = _f32(state0)
    B = s0.shape[0]
    off, st, en = _i32(offsets), _i32(starts), _i32(ends)
    C = st.size
    tok = lambda: np.zeros((T, H, D), dtype=np.float64)
    out = {"y": tok(), "sa": tok(), "boundary": np.zeros((C, H, D, D)),
           "state": np.zeros((B, H, D, D))}
    grads = {n: tok() for n in ("dr", "dw", "dk", "dv", "da", "db")}
    grads["dstate0"] = np.zeros((B, H, D, D))
    dyf = None if dy is None else _f32(dy)
    dff = None if dfinal is None else _f32(dfinal)
    _load().wkv7_oracle_statetune_f64(
        B, T, H, D, _p(off), _p(st), _p(en), _p(s0), *(_p(t) for t in arrs), float(scale),
        _p(dyf), _p(dff), _p(out["y"]), _p(out["sa"]), _p(out["boundary"]), _p(out["state"]),
        *(_p(grads[n]) for n in ("dr", "dw", "dk", "dv", "da", "db", "dstate0")))
    out.update(grads)
    return out


def cpu_threads() -> int:
    return int(_load().wkv7_cpu_max_threads())


# ---------------------------------------------------------------------------
# FP16-state ("Albatross") contract, numpy
# ---------------------------------------------------------------------------
def albatross_dither(phase):
    """dither(phase) = int32(0x9E3779B9 * phase mod 2^32) * 2^-41 as float32
    (recurrent_decay.cuh:36-40)."""
    ph = np.asarray(phase, dtype=np.int64)
    bits = (ph * 0x9E3779B9) & 0xFFFFFFFF
    signed = np.where(bits >= 0x80000000, bits - 0x100000000, bits)
    return (signed.astype(np.float32) * np.float32(2.0 ** -41)).astype(np.float32)


def wkv7_fp16_state(r, logits, k, v, a, b, *, cu_seqlens, state_indices, state_pool,
                    elapsed_state_pool, decay_bias=None, scale=1.0):
    """FP16-state packed recurrence (tests/tmix/wkv7/test.py:88-149).

    Token arrays ``[total, H, D]`` (fp16 values); ``state_pool`` fp16
    ``[slots, H, D, D]``; ``elapsed_state_pool`` int ``[slots]``.  Arithmetic
    in float32 with the contract's fp16 rounding points.  Returns
    ``(y fp16, new_pool fp16, new_elapsed)``; the elapsed counts advance by
    each sequence's length, as the native entry does after its kernel.
    """
    tok = [np.asarray(t, dtype=np.float32) for t in (r, logits, k, v, a, b)]
    r_, x_, k_, v_, a_, b_ = tok
    total, H, D = r_.shape
    cu = _i32(cu_seqlens)
    slots = _i32(state_indices)
    pool = np.array(state_pool, dtype=np.float16)
    elapsed = np.array(elapsed_state_pool, dtype=np.int64)
    bias = None if decay_bias is None else np.asarray(decay_bias, dtype=np.float32).reshape(H, D)
    y = np.zeros((total, H, D), dtype=np.float16)
    hk = np.arange(H * D, dtype=np.int64).reshape(H, D)
    for n in range(cu.size - 1):
        slot = int(slots[n])
        S = pool[slot].astype(np.float32)                      # [H, K, V]
        base = int(elapsed[slot])
        for t in range(int(cu[n]), int(cu[n + 1])):
            x = x_[t] if bias is None else x_[t] + bias
            w = np.exp(np.float32(-0.6065306597126334) / (1.0 + np.exp(-x))).astype(np.float32)
            dither = albatross_dither(hk + base + (t - int(cu[n])))
            delta = (w - np.float32(1.0) + dither).astype(np.float16).astype(np.float32)
            sa = np.einsum("hk,hkv->hv", a_[t], S).astype(np.float32)
            S = (S + S * delta[:, :, None] + b_[t][:, :, None] * sa[:, None, :]
                 + k_[t][:, :, None] * v_[t][:, None, :]).astype(np.float16).astype(np.float32)
            y[t] = (np.float32(scale) * np.einsum("hk,hkv->hv", r_[t], S)).astype(np.float16)
        pool[slot] = S.astype(np.float16)
        elapsed[slot] += int(cu[n + 1]) - int(cu[n])
    return y, pool, elapsed.astype(np.int32)
