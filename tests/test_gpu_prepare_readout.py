"""GPU parity of the WKV7 path's producer (wkv_prepare) and consumer
(readout) stages against the fp64 numpy oracle (oracle/prepare.py).

Cases mirror tests/tmix/wkv_prepare/test.py and tests/tmix/readout/test.py
of the reference (rows 2, C = 4096, ranks 32, head sizes 64/128/256, first
and later layer, LoRA), with the reference's tolerances (wkv_prepare atol
0.10 / rtol 0.06, readout atol 0.08 / rtol 0.05).  Each fused kernel is also
checked alone through the C ABI on exactly its fp16 inputs, where the only
error left is the fp16 store (rtol 2e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import prepare as P
from wkv7_testlib import require_gpu, to_np

pytestmark = pytest.mark.gpu

from flashrwkv2_amd import _native as N  # noqa: E402
from flashrwkv2_amd.tmix.readout import infer_tmix_readout_forward_varlen  # noqa: E402
from flashrwkv2_amd.tmix.wkv_prepare import infer_tmix_wkv_prepare_forward_varlen  # noqa: E402


def _h(g, shape, s):
    return (torch.randn(shape, generator=g) * s).half().cuda()


def _close(actual, expected, atol, rtol, what=""):
    a = to_np(actual).astype(np.float64)
    assert np.isfinite(a).all(), what
    excess = np.abs(a - expected) - (atol + rtol * np.abs(expected))
    assert float(excess.max()) <= 0.0, (what, float(excess.max()))


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("later_layer", [False, True])
@pytest.mark.parametrize("head_size", [64, 128, 256])
def test_wkv_prepare_first_and_later_layer(later_layer, head_size):
    require_gpu()
    g = torch.Generator().manual_seed(20260818 + head_size + int(later_layer))
    rows, C, R = 2, 4096, 32
    shifted = [_h(g, (rows, C), 0.03) for _ in range(6)]
    dense = [_h(g, (C, C), 0.01) for _ in range(3)]
    rank_in = [_h(g, (R, C), 0.02) for _ in range(4)]
    rank_out = [_h(g, (C, R), 0.02) for _ in range(4)]
    runtime_in = [w.t().contiguous() for w in rank_in]
    runtime_out = [w.t().contiguous() for w in rank_out]
    vectors = [_h(g, (C,), 0.1) for _ in range(4)]
    v_first = _h(g, (rows, C), 0.03) if later_layer else None
    outs = infer_tmix_wkv_prepare_forward_varlen(
        *shifted, *dense, *rank_in, *rank_out, *vectors, v_first=v_first,
        w1_runtime=runtime_in[0], a1_runtime=runtime_in[1], g1_runtime=runtime_in[2],
        v1_runtime=runtime_in[3], w2_runtime=runtime_out[0], a2_runtime=runtime_out[1],
        g2_runtime=runtime_out[2], v2_runtime=runtime_out[3], head_size=head_size,
        batch_size=1, max_seqlen=rows)
    torch.cuda.synchronize()
    assert len(outs) == 8 and all(o.dtype == torch.float16 for o in outs)
    expected = P.wkv_prepare_f64(
        *(to_np(t) for t in shifted), *(to_np(t) for t in dense),
        *(to_np(t) for t in rank_in), *(to_np(t) for t in rank_out),
        *(to_np(t) for t in vectors), v_first=None if v_first is None else to_np(v_first),
        head_size=head_size)
    names = ("receptance", "decay", "key", "value", "a", "b", "gate", "v_first")
    for name, out, ref in zip(names, outs, expected):
        _close(out, ref, 0.10, 0.06, name)
    # tighter: a = -kk is unit-norm per head
    kk = to_np(outs[4]).reshape(rows, C // head_size, head_size)
    np.testing.assert_allclose(np.linalg.norm(kk, axis=-1), 1.0, rtol=3e-3)
    if not later_layer:
        assert torch.equal(outs[7], outs[3])
    else:
        assert torch.equal(outs[7], v_first)


def test_wkv_prepare_original_layouts_and_lora():
    require_gpu()
    g = torch.Generator().manual_seed(20260819)
    rows, C, R, Rl = 3, 1024, 32, 8
    shifted = [_h(g, (rows, C), 0.02) for _ in range(6)]
    dense = [_h(g, (C, C), 0.01) for _ in range(3)]
    rank_in = [_h(g, (R, C), 0.02) for _ in range(4)]
    rank_out = [_h(g, (C, R), 0.02) for _ in range(4)]
    vectors = [_h(g, (C,), 0.1) for _ in range(4)]
    la, lb = _h(g, (Rl, C), 0.02), _h(g, (C, Rl), 0.02)
    outs = infer_tmix_wkv_prepare_forward_varlen(
        *shifted, *dense, *rank_in, *rank_out, *vectors, receptance_lora_a=la,
        receptance_lora_b=lb, receptance_lora_scale=0.5)
    torch.cuda.synchronize()
    expected = P.wkv_prepare_f64(
        *(to_np(t) for t in shifted), *(to_np(t) for t in dense),
        *(to_np(t) for t in rank_in), *(to_np(t) for t in rank_out),
        *(to_np(t) for t in vectors), lora={"receptance": (to_np(la), to_np(lb), 0.5)})
    for out, ref in zip(outs, expected):
        _close(out, ref, 0.08, 0.05)
    with pytest.raises(ValueError, match="provided together"):
        infer_tmix_wkv_prepare_forward_varlen(
            *shifted, *dense, *rank_in, *rank_out, *vectors, receptance_lora_a=la)


@pytest.mark.parametrize("head_size", [64, 128, 256])
def test_readout_matches_oracle(head_size):
    require_gpu()
    g = torch.Generator().manual_seed(20260816 + head_size)
    rows, C = 2, 4096
    packed = [torch.randn((rows, C), generator=g).half().cuda() for _ in range(5)]
    vectors = [torch.randn((C,), generator=g).half().cuda() for _ in range(3)]
    weight = torch.randn((C, C), generator=g).half().cuda()
    out = infer_tmix_readout_forward_varlen(packed[0], packed[1], packed[2], packed[3],
                                            vectors[0], vectors[1], vectors[2], packed[4],
                                            weight, head_size=head_size, batch_size=1,
                                            max_seqlen=rows)
    torch.cuda.synchronize()
    ref = P.readout_f64(*(to_np(t) for t in packed[:4]), *(to_np(t) for t in vectors),
                        to_np(packed[4]), to_np(weight), head_size=head_size)
    assert out.dtype == torch.float16 and out.shape == (rows, C)
    _close(out, ref, 0.08, 0.05)


def test_readout_lora_and_rejects():
    require_gpu()
    g = torch.Generator().manual_seed(5)
    rows, C, Rl = 4, 512, 16
    packed = [torch.randn((rows, C), generator=g).half().cuda() for _ in range(5)]
    vectors = [torch.randn((C,), generator=g).half().cuda() for _ in range(3)]
    weight = (torch.randn((C, C), generator=g) * 0.05).half().cuda()
    la, lb = _h(g, (Rl, C), 0.05), _h(g, (C, Rl), 0.05)
    out = infer_tmix_readout_forward_varlen(*packed[:4], *vectors, packed[4], weight,
                                            output_lora_a=la, output_lora_b=lb,
                                            output_lora_scale=0.25)
    torch.cuda.synchronize()
    ref = P.readout_f64(*(to_np(t) for t in packed[:4]), *(to_np(t) for t in vectors),
                        to_np(packed[4]), to_np(weight), lora=(to_np(la), to_np(lb), 0.25))
    _close(out, ref, 0.08, 0.05)
    with pytest.raises(ValueError, match="provided together"):
        infer_tmix_readout_forward_varlen(*packed[:4], *vectors, packed[4], weight,
                                          output_lora_a=la)
    with pytest.raises(ValueError, match="must match wkv_output"):
        infer_tmix_readout_forward_varlen(packed[0], packed[1][:2], *packed[2:4], *vectors,
                                          packed[4], weight)


# ------------------------------------------------------ kernels through the C ABI
@pytest.mark.parametrize("head_size", [64, 128, 256])
def test_kk_a_gate_kernel_exact_inputs(head_size):
    require_gpu()
    g = torch.Generator().manual_seed(head_size)
    T, H = 37, 512 // head_size * 2
    C = H * head_size
    k, a12 = _h(g, (T, C), 1.0), _h(g, (T, C), 1.0)
    k_k, a0 = _h(g, (C,), 1.0), _h(g, (C,), 1.0)
    k_a = torch.rand((C,), generator=g).half().cuda()
    k[3, :head_size] = 0          # a zero head: the 1e-12 floor, no NaN
    outs = [torch.empty_like(k) for _ in range(3)]
    rc = N.load().fr2_tmix_kk_a_gate_forward(T, H, head_size, k.data_ptr(), k_k.data_ptr(),
                                             a0.data_ptr(), a12.data_ptr(), k_a.data_ptr(),
                                             *(o.data_ptr() for o in outs), _stream())
    N.check(rc, "fr2_tmix_kk_a_gate_forward")
    torch.cuda.synchronize()
    ref = P.kk_a_gate_f64(to_np(k), to_np(k_k), to_np(a0), to_np(a12), to_np(k_a), head_size)
    for out, r in zip(outs, ref):
        _close(out, r, 1e-3, 2e-3)
    assert not torch.any(outs[1][3, :head_size])


def test_lowrank_activate_and_vres_kernels_exact_inputs():
    require_gpu()
    g = torch.Generator().manual_seed(9)
    w1x, g1x = _h(g, (5, 37), 2.0), _h(g, (5, 32), 2.0)    # 185 values: a scalar tail
    tw, sg = torch.empty_like(w1x), torch.empty_like(g1x)
    rc = N.load().fr2_tmix_lowrank_activate(w1x.numel(), w1x.data_ptr(), tw.data_ptr(),
                                            g1x.numel(), g1x.data_ptr(), sg.data_ptr(),
                                            _stream())
    N.check(rc, "fr2_tmix_lowrank_activate")
    T, C = 9, 256
    value, first, v12 = (_h(g, (T, C), 1.0) for _ in range(3))
    v0 = _h(g, (C,), 1.0)
    out = torch.empty_like(value)
    rc = N.load().fr2_tmix_vres_forward(T, C, value.data_ptr(), first.data_ptr(), v0.data_ptr(),
                                        v12.data_ptr(), out.data_ptr(), _stream())
    N.check(rc, "fr2_tmix_vres_forward")
    torch.cuda.synchronize()
    _close(tw, np.tanh(to_np(w1x).astype(np.float64)), 1e-3, 2e-3, "tanh")
    _close(sg, 1 / (1 + np.exp(-to_np(g1x).astype(np.float64))), 1e-3, 2e-3, "sigmoid")
    _close(out, P.vres_f64(to_np(value), to_np(first), to_np(v0), to_np(v12)), 2e-3, 2e-3, "vres")


@pytest.mark.parametrize("head_size", [64, 128, 256])
def test_readout_prelinear_kernel_exact_inputs(head_size):
    require_gpu()
    g = torch.Generator().manual_seed(100 + head_size)
    T, C = 21, 1024
    x, r, k, v, gt = (_h(g, (T, C), 1.0) for _ in range(5))
    r_k, w, b = (_h(g, (C,), 1.0) for _ in range(3))
    out = torch.empty_like(x)
    rc = N.load().fr2_tmix_readout_prelinear_forward(
        T, C // head_size, head_size, *(t.data_ptr() for t in (x, r, k, v, r_k, w, b, gt)),
        out.data_ptr(), _stream())
    N.check(rc, "fr2_tmix_readout_prelinear_forward")
    torch.cuda.synchronize()
    ref = P.readout_prelinear_f64(*(to_np(t) for t in (x, r, k, v, r_k, w, b, gt)), head_size)
    _close(out, ref, 2e-3, 3e-3)
