"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so that a plausible mistake in the restated recurrence
fails it: a dropped term, a transposed operand (a vs b, k vs v, state
orientation), the pre-/post-update state confusion for sa and y, a wrong sign
in the retention, a misplaced bias or scale, or a wrong slot / boundary index.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle

D = 64
NEG_BIG = -1.0e4  # sigmoid underflows to exactly 0 in fp64: retention == 1


def _rand_case(rng, lengths, H, *, scale=0.3, logit_scale=2.0, pool_slots=None):
    total = sum(lengths)
    shape = (total, H, D)
    r, k, v, a, b = (rng.standard_normal(shape).astype(np.float32) * scale for _ in range(5))
    logits = (rng.standard_normal(shape) * logit_scale).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    n = len(lengths)
    pool_slots = pool_slots or n + 3
    pool = rng.standard_normal((pool_slots, H, D, D)) * 0.05
    slots = rng.permutation(pool_slots)[:n].astype(np.int32)
    return dict(r=r, logits=logits, k=k, v=v, a=a, b=b, cu=cu, slots=slots, pool=pool)


def _run(c, **kw):
    return oracle.wkv7_f64(c["r"], c["logits"], c["k"], c["v"], c["a"], c["b"],
                           cu_seqlens=c["cu"], state_indices=c["slots"],
                           state_pool=c["pool"], **kw)


def _matrix_form(c, *, bias=None, scale=1.0):
    """Explicit-matrix fp64 evaluation: S_t = (diag(w_t) + b_t a_t^T) S_{t-1}
    + k_t v_t^T; y_t = scale * S_t^T r_t — a different formulation from the
    oracle's element loops."""
    pool = np.array(c["pool"], dtype=np.float64)
    total, H, _ = c["r"].shape
    y = np.zeros((total, H, D))
    for s in range(len(c["cu"]) - 1):
        slot = c["slots"][s]
        for h in range(H):
            S = pool[slot, h].copy()
            for t in range(c["cu"][s], c["cu"][s + 1]):
                x = c["logits"][t, h].astype(np.float64)
                if bias is not None:
                    x = x + bias[h].astype(np.float64)
                w = np.exp(-math.exp(-0.5) / (1.0 + np.exp(-x)))
                f64 = {n: c[n][t, h].astype(np.float64) for n in ("a", "b", "k", "v")}
                G = np.diag(w) + np.outer(f64["b"], f64["a"])
                S = G @ S + np.outer(f64["k"], f64["v"])
                y[t, h] = scale * (S.T @ c["r"][t, h].astype(np.float64))
            pool[slot, h] = S
    return y, pool


def test_retention_matches_base2_constant_form_and_limits():
    # recurrent_retention (recurrent_decay.cuh:18-22) uses exp2 with two
    # rounded constants; the pretrain form (pretrain_recurrent_bf16_forward.cu:26,56)
    # uses exp with W_SCALE = -exp(-1/2).
    for x in np.linspace(-30, 30, 241):
        ref2 = 2.0 ** (-0.8750387749145276 / (1.0 + 2.0 ** (-1.4426950408889634 * x)))
        refe = math.exp(-0.6065306597 / (1.0 + math.exp(-x)))
        got = oracle.retention(x)
        assert got == pytest.approx(ref2, rel=1e-14)
        assert got == pytest.approx(refe, rel=1e-9)
    assert oracle.retention(NEG_BIG) == 1.0
    assert oracle.retention(1.0e4) == pytest.approx(math.exp(-math.exp(-0.5)), rel=1e-15)
    assert oracle.retention(0.0) == pytest.approx(math.exp(-math.exp(-0.5) / 2), rel=1e-15)
    # monotone decreasing in the logit
    xs = np.linspace(-20, 20, 101)
    vals = [oracle.retention(x) for x in xs]
    assert all(a > b for a, b in zip(vals, vals[1:]))


@pytest.mark.parametrize("with_bias,scale", [(False, 1.0), (True, 0.75)])
def test_recurrence_matches_explicit_matrix_form(with_bias, scale):
    rng = np.random.default_rng(7 + int(with_bias))
    c = _rand_case(rng, (1, 5, 16, 3), H=2)
    bias = (rng.standard_normal((2, D)) * 0.5).astype(np.float32) if with_bias else None
    y, pool, _, _ = _run(c, decay_bias=bias, scale=scale)
    y_ref, pool_ref = _matrix_form(c, bias=bias, scale=scale)
    np.testing.assert_allclose(y, y_ref, rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(pool, pool_ref, rtol=1e-11, atol=1e-13)


def test_linear_attention_closed_form():
    """a = b = 0 and retention 1: y_t = r_t (S_0 + sum_{s<=t} k_s v_s^T)."""
    rng = np.random.default_rng(11)
    c = _rand_case(rng, (9, 4), H=1)
    c["a"][:] = 0
    c["b"][:] = 0
    c["logits"][:] = NEG_BIG
    y, pool, _, _ = _run(c, scale=1.0)
    for s in range(2):
        t0, t1 = c["cu"][s], c["cu"][s + 1]
        S0 = c["pool"][c["slots"][s], 0]
        kv = np.einsum("tk,tv->tkv", c["k"][t0:t1, 0].astype(np.float64),
                       c["v"][t0:t1, 0].astype(np.float64))
        S = S0[None] + np.cumsum(kv, axis=0)
        y_ref = np.einsum("tk,tkv->tv", c["r"][t0:t1, 0].astype(np.float64), S)
        np.testing.assert_allclose(y[t0:t1, 0], y_ref, rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(pool[c["slots"][s], 0], S[-1], rtol=1e-12, atol=1e-13)


def test_pure_decay_closed_form():
    """k = a = b = 0: S_t = diag(prod_{s<=t} w_s) S_0."""
    rng = np.random.default_rng(13)
    c = _rand_case(rng, (12,), H=1)
    c["k"][:] = 0
    c["a"][:] = 0
    c["b"][:] = 0
    y, pool, _, _ = _run(c)
    x = c["logits"][:, 0].astype(np.float64)
    w = np.exp(-math.exp(-0.5) / (1.0 + np.exp(-x)))
    gam = np.cumprod(w, axis=0)
    S0 = c["pool"][c["slots"][0], 0]
    y_ref = np.einsum("tk,tk,kv->tv", c["r"][:, 0].astype(np.float64), gam, S0)
    np.testing.assert_allclose(y[:, 0], y_ref, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(pool[c["slots"][0], 0], gam[-1][:, None] * S0, rtol=1e-12)


def test_idempotent_projection():
    """w = 1, b = kk, a = -kk with |kk| = 1, k = v = 0: S <- (I - kk kk^T) S,
    a projection: the second application changes nothing and kk^T S = 0."""
    rng = np.random.default_rng(17)
    c = _rand_case(rng, (2,), H=1)
    kk = rng.standard_normal(D)
    kk /= np.linalg.norm(kk)
    # keep kk exactly representable in fp32 so that |kk| = 1 holds to fp32
    kk32 = kk.astype(np.float32)
    c["a"][:, 0] = -kk32
    c["b"][:, 0] = kk32
    c["k"][:] = 0
    c["v"][:] = 0
    c["logits"][:] = NEG_BIG
    _, pool, _, _ = _run(c)
    S0 = c["pool"][c["slots"][0], 0]
    kkd = kk32.astype(np.float64)
    P = np.eye(D) - np.outer(kkd, kkd)
    np.testing.assert_allclose(pool[c["slots"][0], 0], P @ P @ S0, rtol=1e-10, atol=1e-12)
    # P is idempotent up to |kk|^2 - 1 ~ fp32 rounding of kk
    np.testing.assert_allclose(P @ P @ S0, P @ S0, atol=1e-6)
    assert np.abs(kkd @ pool[c["slots"][0], 0]).max() < 1e-6


def test_split_invariance_packing_and_untouched_slots():
    rng = np.random.default_rng(19)
    c = _rand_case(rng, (37,), H=2)
    y_full, pool_full, _, _ = _run(c)
    first = dict(c, cu=np.array([0, 20], np.int32))
    first = {k: (v[:20] if k in ("r", "logits", "k", "v", "a", "b") else v)
             for k, v in first.items()}
    y1, pool1, _, _ = _run(first)
    second = {k: (v[20:] if k in ("r", "logits", "k", "v", "a", "b") else v)
              for k, v in c.items()}
    second["cu"] = np.array([0, 17], np.int32)
    second["pool"] = pool1
    y2, pool2, _, _ = _run(second)
    assert np.array_equal(np.concatenate([y1, y2]), y_full)
    assert np.array_equal(pool2, pool_full)
    untouched = [i for i in range(c["pool"].shape[0]) if i not in set(c["slots"].tolist())]
    assert np.array_equal(pool_full[untouched], c["pool"][untouched])


def test_sequence_order_and_slot_permutation_invariance():
    rng = np.random.default_rng(23)
    c = _rand_case(rng, (3, 8, 5), H=1)
    y, pool, _, _ = _run(c)
    order = [2, 0, 1]
    lens = np.diff(c["cu"])
    pieces = [np.arange(c["cu"][i], c["cu"][i + 1]) for i in range(3)]
    perm_tokens = np.concatenate([pieces[i] for i in order])
    c2 = {k: (v[perm_tokens] if k in ("r", "logits", "k", "v", "a", "b") else v)
          for k, v in c.items()}
    c2["cu"] = np.concatenate([[0], np.cumsum(lens[order])]).astype(np.int32)
    c2["slots"] = c["slots"][order]
    y2, pool2, _, _ = _run(c2)
    assert np.array_equal(y2, y[perm_tokens])
    assert np.array_equal(pool2, pool)


def test_scale_is_linear_and_only_on_output():
    rng = np.random.default_rng(29)
    c = _rand_case(rng, (6, 2), H=1)
    y1, p1, _, _ = _run(c, scale=1.0)
    y2, p2, _, _ = _run(c, scale=0.5)
    assert np.array_equal(y2, 0.5 * y1)
    assert np.array_equal(p1, p2)


def test_boundary_and_state_dot_a_match_split_runs():
    rng = np.random.default_rng(31)
    T = 48
    c = _rand_case(rng, (T, T), H=1)
    c["pool"][:] = 0.0
    _, _, sa, boundary = _run(c, want_sa=True, boundary_len=16)
    assert boundary.shape == (2, 1, 3, D, D)
    for s in range(2):
        t0 = c["cu"][s]
        for chunk in range(3):
            n = 16 * (chunk + 1)
            part = {k: (v[t0:t0 + n] if k in ("r", "logits", "k", "v", "a", "b") else v)
                    for k, v in c.items()}
            part["cu"] = np.array([0, n], np.int32)
            part["slots"] = np.array([0], np.int32)
            part["pool"] = np.zeros((1, 1, D, D))
            _, pool_n, _, _ = _run(part)
            np.testing.assert_array_equal(boundary[s, 0, chunk], pool_n[0, 0])
        # sa_t = a_t^T S_{t-1}
        prev = np.zeros((D, D))
        for t in range(t0, t0 + T):
            if t > t0:
                part = {k: (v[t0:t] if k in ("r", "logits", "k", "v", "a", "b") else v)
                        for k, v in c.items()}
                part["cu"] = np.array([0, t - t0], np.int32)
                part["slots"] = np.array([0], np.int32)
                part["pool"] = np.zeros((1, 1, D, D))
                _, pool_t, _, _ = _run(part)
                prev = pool_t[0, 0]
            if (t - t0) % 7 == 0:  # a sample of tokens keeps the check fast
                np.testing.assert_allclose(sa[t, 0], c["a"][t, 0].astype(np.float64) @ prev,
                                           rtol=1e-12, atol=1e-14)


def test_cpu_fp32_baseline_tracks_fp64():
    rng = np.random.default_rng(37)
    c = _rand_case(rng, (40, 9), H=3)
    y64, p64, _, _ = _run(c)
    y32, p32 = oracle.wkv7_cpu_f32(c["r"], c["logits"], c["k"], c["v"], c["a"], c["b"],
                                   cu_seqlens=c["cu"], state_indices=c["slots"],
                                   state_pool=c["pool"], threads=2)
    assert np.abs(y32 - y64).max() <= 1e-5 * max(1.0, np.abs(y64).max())
    assert np.abs(p32 - p64).max() <= 1e-5 * max(1.0, np.abs(p64).max())


def test_torch_loop_baseline_matches_the_fp64_oracle():
    """The pure-torch per-token loop bench.py times as the planned CPU
    baseline computes the same recurrence as the fp64 C oracle (fp32
    rounding only), on config-0 shapes with a nonzero state and scale."""
    import torch

    from oracle.torch_loop import wkv7_torch_packed
    from flashrwkv2_amd import workloads

    wl = workloads.config(0, "cpu", dtype=torch.float32)
    g = torch.Generator().manual_seed(4)
    states = torch.randn((1, 4, 64, 64), generator=g) * 0.1
    toks = [t.float() for t in wl.tokens]
    y, s = wkv7_torch_packed(*toks, wl.cu_seqlens.tolist(), states, scale=0.5)
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(*(t.numpy() for t in toks),
                                            cu_seqlens=wl.cu_seqlens.numpy(),
                                            state_pool=states.numpy(), scale=0.5)
    np.testing.assert_allclose(y.numpy(), y_ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(s.numpy(), pool_ref, rtol=1e-4, atol=1e-4)
