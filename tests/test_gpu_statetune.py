"""GPU parity of StateTune (trainable initial state over a chunk list)
against the fp64 oracle (oracle.statetune_f64, pinned in
test_oracle_statetune.py).

The first test is the reference's own case and bounds
(tests/tmix/wkv7/statetune/test.py:93-165): B=2, H=1, five tokens in chunks
[0,1) [1,3) | [3,5), state and tokens 0.01 * randn, scale 0.75, the loss
sum(y^2) + sum(S_final^2); forward atol = rtol = 8e-3 (bf16) / 3e-4 (fp16),
gradients atol 8e-3 / 3e-4 and rtol 1e-2 / 3e-3, for D in {64, 128, 256}.
The oracle is fed the cotangents the backward actually received
(dy = 2y rounded to the token dtype, dS_final = 2 S_final).

The others widen the cases: ragged, empty and long chunks, gaps, several
heads, O(1) inputs in the model's operand structure (there the gradients
meet a relative RMSE bound and the allclose bound with its absolute part
scaled by the gradient's RMS), zero cotangents, determinism, and that the
caller's initial state is not modified.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from wkv7_testlib import relative_rmse, require_gpu, to_np

pytestmark = pytest.mark.gpu

from flashrwkv2_amd.tmix.wkv7 import statetune_tmix_wkv7_recurrent_fp32io16  # noqa: E402

TOKEN_GRADS = ("dr", "dw", "dk", "dv", "da", "db")


def _meta(offsets, starts, ends):
    return [torch.tensor(x, dtype=torch.int32, device="cuda") for x in (offsets, starts, ends)]


def _run(state, meta, vals, scale):
    state = state.clone().requires_grad_()
    vals = [v.clone().requires_grad_() for v in vals]
    out = statetune_tmix_wkv7_recurrent_fp32io16(state, *meta, *vals, scale=scale)
    return state, vals, out


def _grads(state, vals):
    return {"dstate0": state.grad, **{n: v.grad for n, v in zip(TOKEN_GRADS, vals)}}


def _oracle(state, meta, vals, scale, dy=None, dfinal=None):
    return oracle.statetune_f64(to_np(state), *(m.cpu().numpy() for m in meta),
                                *(to_np(v) for v in vals), scale=scale,
                                dy=None if dy is None else to_np(dy),
                                dfinal=None if dfinal is None else to_np(dfinal))


def _allclose(actual, expected, atol, rtol, what):
    a = to_np(actual).astype(np.float64)
    assert np.isfinite(a).all(), what
    worst = float(np.max(np.abs(a - expected) - (atol + rtol * np.abs(expected))))
    assert worst <= 0.0, (what, worst)


@pytest.mark.parametrize("head_size", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_statetune_reference_case(dtype, head_size):
    require_gpu()
    g = torch.Generator().manual_seed(20260805 + head_size)
    B, H, T = 2, 1, 5
    state0 = (torch.randn((B, H, head_size, head_size), generator=g) * 0.01).cuda()
    vals = [(torch.randn((T, H, head_size), generator=g) * 0.01).to(dtype).cuda()
            for _ in range(6)]
    meta = _meta([0, 2, 3], [0, 1, 3], [1, 3, 5])
    snapshot = state0.clone()
    state, leaves, (y, fin, boundary, sa) = _run(state0, meta, vals, 0.75)
    torch.cuda.synchronize()
    ref = _oracle(state0, meta, vals, 0.75)
    tol = 8e-3 if dtype == torch.bfloat16 else 3e-4
    assert y.dtype == dtype and fin.dtype == torch.float32
    assert tuple(boundary.shape) == (3, H, head_size, head_size)
    for got, key in ((y, "y"), (fin, "state"), (boundary, "boundary"), (sa, "sa")):
        _allclose(got, ref[key], tol, tol, key)

    (y.float().square().sum() + fin.square().sum()).backward()
    torch.cuda.synchronize()
    dy = (2.0 * y.detach().float()).to(dtype)
    ref = _oracle(state0, meta, vals, 0.75, dy=dy, dfinal=2.0 * fin.detach())
    rtol = 1e-2 if dtype == torch.bfloat16 else 3e-3
    got = _grads(state, leaves)
    for key in ("dstate0", *TOKEN_GRADS):
        _allclose(got[key], ref[key], tol, rtol, key)
    assert got["dstate0"].dtype == torch.float32 and got["dr"].dtype == dtype
    assert torch.equal(state0, snapshot)


def _structured(T, H, D, dtype, g, logit_scale=1.0):
    """The model's operand structure at O(1) scale: r, k, v ~ N(0,1),
    kk = L2-normalised N(0,1), a = -kk, b = kk * sigmoid(N(0,1))."""
    vals = [torch.randn((T, H, D), generator=g) for _ in range(6)]
    kk = torch.randn((T, H, D), generator=g)
    kk = kk / kk.norm(dim=-1, keepdim=True)
    vals[1] = torch.randn((T, H, D), generator=g) * logit_scale
    vals[4] = -kk
    vals[5] = kk * torch.sigmoid(torch.randn((T, H, D), generator=g))
    return [v.to(dtype).cuda() for v in vals]


def _check_strong(got, ref, keys, rel=1e-2, atol=0.03, rtol=0.05):
    for key in keys:
        a, e = to_np(got[key]).astype(np.float64), ref[key]
        assert np.isfinite(a).all(), key
        assert relative_rmse(a, e) <= rel, (key, relative_rmse(a, e))
        bound = atol * max(1.0, float(np.sqrt(np.mean(e * e)))) + rtol * np.abs(e)
        assert float(np.max(np.abs(a - e) - bound)) <= 0.0, key


@pytest.mark.parametrize("head_size", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_statetune_ragged_chunks_gaps_and_empty_chunks(dtype, head_size):
    """Sequence 0: chunks of 1, 17, 0 and 40 tokens; tokens 58..60 belong to
    no chunk; sequence 1: chunks of 33 and 7 tokens; sequence 2: no chunks."""
    require_gpu()
    g = torch.Generator().manual_seed(7 * head_size + (dtype == torch.float16))
    H, T = 2, 101
    D = head_size
    vals = _structured(T, H, D, dtype, g)
    state0 = (torch.randn((3, H, D, D), generator=g) * 0.5).cuda()
    meta = _meta([0, 4, 6, 6], [0, 1, 18, 18, 61, 94], [1, 18, 18, 58, 94, 101])
    state, leaves, (y, fin, boundary, sa) = _run(state0, meta, vals, 0.5)
    dy = torch.randn((T, H, D), generator=g).to(dtype).cuda()
    dfin = torch.randn((3, H, D, D), generator=g).cuda()
    torch.autograd.backward([y, fin], [dy, dfin])
    torch.cuda.synchronize()
    ref = _oracle(state0, meta, vals, 0.5, dy=dy, dfinal=dfin)
    used = np.r_[0:58, 61:101]
    fwd = {"y": y[used], "sa": sa[used]}
    _check_strong(fwd, {k: ref[k][used] for k in ("y", "sa")}, ("y", "sa"), rel=5e-3)
    for got, key in ((fin, "state"), (boundary, "boundary")):
        assert relative_rmse(to_np(got), ref[key]) <= 2e-3, key
    # the sequence without chunks keeps its state and passes dS_final through
    assert torch.equal(fin[2], state0[2])
    got = _grads(state, leaves)
    assert torch.equal(got["dstate0"][2], dfin[2])
    _check_strong({k: got[k][used] for k in TOKEN_GRADS}, {k: ref[k][used] for k in TOKEN_GRADS},
                  TOKEN_GRADS)
    _check_strong(got, ref, ("dstate0",))


@pytest.mark.parametrize("head_size", [64, 256])
def test_statetune_long_chunk(head_size):
    """One 600-token chunk per sequence: the key pass restarts from the
    replay snapshots every 16 (8 at D = 256) tokens."""
    require_gpu()
    g = torch.Generator().manual_seed(600 + head_size)
    H, L, D = 2, 600, head_size
    vals = _structured(2 * L, H, D, torch.bfloat16, g, logit_scale=1.5)
    state0 = (torch.randn((2, H, D, D), generator=g) * 0.3).cuda()
    meta = _meta([0, 1, 2], [0, L], [L, 2 * L])
    state, leaves, (y, fin, _, _) = _run(state0, meta, vals, 1.0)
    dy = torch.randn((2 * L, H, D), generator=g).to(torch.bfloat16).cuda()
    dfin = (torch.randn((2, H, D, D), generator=g) * 0.1).cuda()
    torch.autograd.backward([y, fin], [dy, dfin])
    torch.cuda.synchronize()
    ref = _oracle(state0, meta, vals, 1.0, dy=dy, dfinal=dfin)
    _check_strong({"y": y}, ref, ("y",), rel=5e-3)
    _check_strong(_grads(state, leaves), ref, ("dstate0", *TOKEN_GRADS))


def test_statetune_zero_cotangents_through_native_entry():
    """grad_output / grad_final_state = None through the native backward
    (the reference's nullptr paths) against the oracle with zero cotangents
    on the other input."""
    C = require_gpu()
    g = torch.Generator().manual_seed(11)
    H, T, D = 1, 40, 64
    vals = _structured(T, H, D, torch.bfloat16, g)
    state0 = (torch.randn((1, H, D, D), generator=g) * 0.5).cuda()
    meta = _meta([0, 2], [0, 13], [13, 40])
    st = state0.clone()
    y = torch.empty_like(vals[3])
    boundary = torch.empty((2, H, D, D), device="cuda")
    sa = torch.empty((T, H, D), device="cuda")
    C.statetune_tmix_wkv7_recurrent_fp32io16_forward(*meta, st, *vals, y, boundary, sa, 1.0)
    dy = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
    dfin = torch.randn((1, H, D, D), generator=g).cuda()
    for gy, gf in ((dy, None), (None, dfin)):
        grads = [torch.empty_like(v) for v in vals]
        g0 = torch.empty_like(st)
        C.statetune_tmix_wkv7_recurrent_fp32io16_backward(*meta, st, *vals, sa, gy, gf, boundary,
                                                          *grads, g0, 1.0)
        torch.cuda.synchronize()
        ref = _oracle(state0, meta, vals, 1.0, dy=gy, dfinal=gf)
        got = {"dstate0": g0, **dict(zip(TOKEN_GRADS, grads))}
        _check_strong(got, ref, ("dstate0", *TOKEN_GRADS))


def test_statetune_is_deterministic_and_validates():
    require_gpu()
    g = torch.Generator().manual_seed(5)
    H, T, D = 2, 50, 128
    vals = _structured(T, H, D, torch.float16, g)
    state0 = (torch.randn((2, H, D, D), generator=g) * 0.2).cuda()
    meta = _meta([0, 1, 2], [0, 20], [20, 50])
    runs = []
    for _ in range(2):
        state, leaves, (y, fin, _, _) = _run(state0, meta, vals, 0.9)
        (y.float().square().sum() + fin.square().sum()).backward()
        runs.append([y, fin, state.grad, *(v.grad for v in leaves)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    with pytest.raises(TypeError, match="dtype of r"):
        statetune_tmix_wkv7_recurrent_fp32io16(state0, *meta, vals[0], vals[1].bfloat16(),
                                               *vals[2:])
    with pytest.raises(ValueError, match=r"shape \[B\+1\]"):
        statetune_tmix_wkv7_recurrent_fp32io16(state0, meta[0][:2], *meta[1:], *vals)
    with pytest.raises(ValueError, match="scale must be finite"):
        statetune_tmix_wkv7_recurrent_fp32io16(state0, *meta, *vals, scale=float("nan"))


# ------------------------------------------------ uniform layout: MFMA kernels
def _uniform_meta(B, per_seq, length):
    nck = per_seq // length
    starts = [c * length for c in range(B * nck)]
    return _meta([s * nck for s in range(B + 1)], starts, [s + length for s in starts])


@pytest.mark.parametrize("B,per_seq,length,scale", [
    (3, 128, 32, 1.0),
    (2, 256, 16, 0.75),
    (1, 64, 64, 1.0),
    (2, 1024, 256, 1.0),     # several 8-chunk spans of the key pass
])
def test_statetune_uniform_layout_runs_chunked_kernels(B, per_seq, length, scale):
    """D = 64, bf16, equal sequences cut into equal chunks of a multiple of 16
    tokens: the forward runs the chunked MFMA kernel (it returns the
    post-16-token snapshots) and the backward the chunked value and key
    passes; both against the fp64 oracle and against the token-serial
    kernels on the same inputs."""
    C = require_gpu()
    g = torch.Generator().manual_seed(B * 1000 + per_seq + length)
    H, D, T = 2, 64, B * per_seq
    vals = _structured(T, H, D, torch.bfloat16, g, logit_scale=1.5)
    state0 = (torch.randn((B, H, D, D), generator=g) * 0.5).cuda()
    meta = _uniform_meta(B, per_seq, length)
    nck = B * (per_seq // length)
    dy = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
    dfin = torch.randn((B, H, D, D), generator=g).cuda()

    outs = {}
    for name in ("chunked", "serial"):
        st = state0.clone()
        y = torch.empty_like(vals[3])
        bnd = torch.empty((nck, H, D, D), device="cuda")
        sa = torch.empty((T, H, D), device="cuda")
        if name == "chunked":
            snaps = C.statetune_tmix_wkv7_recurrent_fp32io16_forward(*meta, st, *vals, y, bnd, sa,
                                                                     scale)
            assert snaps is not None and tuple(snaps.shape) == (B, H, per_seq // 16, D, D)
        else:
            snaps = None
            from flashrwkv2_amd import _native as Nn
            rc = Nn.load().fr2_wkv7_statetune_forward(
                *(m.data_ptr() for m in meta), B, nck, T, H, D, Nn.FR2_DTYPE_BFLOAT16,
                st.data_ptr(), *(v.data_ptr() for v in vals), y.data_ptr(), bnd.data_ptr(),
                sa.data_ptr(), scale, torch.cuda.current_stream().cuda_stream)
            Nn.check(rc, "fr2_wkv7_statetune_forward")
        grads = [torch.empty_like(v) for v in vals]
        g0 = torch.empty_like(st)
        C.statetune_tmix_wkv7_recurrent_fp32io16_backward(*meta, st, *vals, sa, dy, dfin, bnd,
                                                          *grads, g0, scale, snapshots=snaps)
        torch.cuda.synchronize()
        outs[name] = {"y": y, "state": st, "boundary": bnd, "sa": sa, "dstate0": g0,
                      **dict(zip(TOKEN_GRADS, grads))}

    ref = _oracle(state0, meta, vals, scale, dy=dy, dfinal=dfin)
    got = outs["chunked"]
    _check_strong(got, ref, ("y", "sa"), rel=5e-3)
    for key in ("state", "boundary"):
        assert relative_rmse(to_np(got[key]), ref[key]) <= 2e-3, key
    _check_strong(got, ref, ("dstate0", *TOKEN_GRADS))
    # the two kernel families agree with each other as closely as with fp64
    for key in ("y", "state", "dstate0", *TOKEN_GRADS):
        assert relative_rmse(to_np(got[key]), to_np(outs["serial"][key])) <= 1e-2, key


def test_statetune_uniform_autograd_and_fallbacks():
    """The public function takes the chunked path on the uniform layout and
    the padded chunked path on a ragged layout of the same tokens; both match
    the oracle and each other."""
    require_gpu()
    g = torch.Generator().manual_seed(77)
    B, per_seq, length, H, D = 2, 96, 32, 2, 64
    T = B * per_seq
    vals = _structured(T, H, D, torch.bfloat16, g)
    state0 = (torch.randn((B, H, D, D), generator=g) * 0.5).cuda()
    dy = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
    dfin = torch.randn((B, H, D, D), generator=g).cuda()
    runs = {}
    for name, meta in (("uniform", _uniform_meta(B, per_seq, length)),
                       ("ragged", _meta([0, 2, 5], [0, 32, 96, 100, 150], [32, 96, 100, 150, 192]))):
        state, leaves, (y, fin, _, _) = _run(state0, meta, vals, 1.0)
        torch.autograd.backward([y, fin], [dy, dfin])
        torch.cuda.synchronize()
        runs[name] = {"y": y, "state": fin, **_grads(state, leaves)}
        ref = _oracle(state0, meta, vals, 1.0, dy=dy, dfinal=dfin)
        _check_strong(runs[name], ref, ("y", "dstate0", *TOKEN_GRADS))
    for key in ("y", "state", "dstate0", *TOKEN_GRADS):
        assert relative_rmse(to_np(runs["uniform"][key]), to_np(runs["ragged"][key])) <= 1e-2, key


def _ragged_meta(B, per_seq, rng, gap=0):
    """B sequences of per_seq tokens packed back to back, each cut into
    chunks of random lengths (some empty, some not a multiple of 16), with
    `gap` tokens at the end of every sequence in no chunk."""
    offsets, starts, ends = [0], [], []
    for b in range(B):
        t, end = b * per_seq, (b + 1) * per_seq - gap
        while t < end:
            n = min(int(rng.integers(0, 300)), end - t)
            starts.append(t)
            ends.append(t + n)
            t += n
        offsets.append(len(starts))
    return _meta(offsets, starts, ends)


@pytest.mark.parametrize("B,per_seq,H,gap", [(3, 700, 2, 0), (2, 1500, 3, 37)])
def test_statetune_ragged_chunk_list_runs_the_padded_chunked_path(B, per_seq, H, gap):
    """A ragged chunk list at D = 64 in bf16 runs on the chunked MFMA kernels
    over the padded grid (the forward returns the grid's tables); forward,
    final state, boundaries and every gradient match the fp64 oracle and the
    token-serial kernels on the same inputs."""
    C = require_gpu()
    import flashrwkv2_amd._C as CC

    rng = np.random.default_rng(B * per_seq + gap)
    g = torch.Generator().manual_seed(B * per_seq + H)
    D, T = 64, B * per_seq
    vals = _structured(T, H, D, torch.bfloat16, g, logit_scale=1.5)
    state0 = (torch.randn((B, H, D, D), generator=g) * 0.5).cuda()
    meta = _ragged_meta(B, per_seq, rng, gap)
    print(f"case statetune ragged B={B} T={per_seq} H={H} gap={gap} chunks={meta[1].numel()}",
          flush=True)
    dy = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
    dfin = torch.randn((B, H, D, D), generator=g).cuda()
    # the forward takes the padded path (tables returned for the backward)
    st = state0.clone()
    probe = C.statetune_tmix_wkv7_recurrent_fp32io16_forward(
        *meta, st, *vals, torch.empty_like(vals[3]),
        torch.empty((meta[1].numel(), H, D, D), device="cuda"),
        torch.empty((T, H, D), device="cuda"), 1.0)
    assert isinstance(probe, tuple) and len(probe) == 3
    runs = {}
    for name, serial in (("padded", False), ("serial", True)):
        CC._statetune_force_serial = serial
        try:
            state, leaves, (y, fin, bnd, sa) = _run(state0, meta, vals, 1.0)
            torch.autograd.backward([y, fin], [dy, dfin])
            torch.cuda.synchronize()
        finally:
            CC._statetune_force_serial = False
        runs[name] = {"y": y, "sa": sa, "state": fin, "boundary": bnd, **_grads(state, leaves)}
    ref = _oracle(state0, meta, vals, 1.0, dy=dy, dfinal=dfin)
    starts, ends = meta[1].cpu().numpy(), meta[2].cpu().numpy()
    used = np.concatenate([np.arange(s0, e0) for s0, e0 in zip(starts, ends)])
    got = runs["padded"]
    _check_strong({k: got[k][used] for k in ("y", "sa")}, {k: ref[k][used] for k in ("y", "sa")},
                  ("y", "sa"), rel=5e-3)
    for key in ("state", "boundary"):
        assert relative_rmse(to_np(got[key]), ref[key]) <= 2e-3, key
    _check_strong({k: got[k][used] for k in TOKEN_GRADS}, {k: ref[k][used] for k in TOKEN_GRADS},
                  TOKEN_GRADS)
    _check_strong(got, ref, ("dstate0",))
    for key in ("y", "sa", *TOKEN_GRADS):
        assert relative_rmse(to_np(got[key][used]), to_np(runs["serial"][key][used])) <= 1e-2, key
    for key in ("state", "boundary", "dstate0"):
        assert relative_rmse(to_np(got[key]), to_np(runs["serial"][key])) <= 1e-2, key
