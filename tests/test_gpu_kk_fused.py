"""The chunked recurrence with wkv_prepare's kk / a-gate stage in its load
stage, against the fp64 oracle composed from its two stages:
``oracle.prepare.kk_a_gate_f64`` (the gate: gated key, a = -kk, b = kk*g)
followed by ``oracle.wkv7_f64`` on exactly those values.

The fused kernel forms a and b in fp32 and never rounds them to the token
dtype, so it is compared with the unrounded fp64 composition, under the same
output/state gates as every recurrent test (tests/wkv7_testlib.py).  The
gated key it writes is compared elementwise with the oracle's: one rounding
of an fp32 value to the token dtype, so |dk| <= 2^-p |k| + 1e-6 with p = 10
for fp16 and 7 for bf16 (one ulp; half an ulp plus the fp32 arithmetic).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from wkv7_testlib import assert_output_close, assert_state_close, require_gpu, to_np

import oracle
from oracle.prepare import kk_a_gate_f64

pytestmark = pytest.mark.gpu

_ULP_BITS = {torch.float16: 10, torch.bfloat16: 7}


def _case(lengths, heads, dtype, seed, *, bias=False):
    g = torch.Generator().manual_seed(seed)
    total, d = sum(lengths), 64
    shape = (total, heads, d)

    def rnd(*s, scale=1.0, shift=0.0):
        return (torch.randn(s, generator=g) * scale + shift).to(dtype)

    c = {
        "r": rnd(*shape, scale=0.3),
        "w": (torch.rand(shape, generator=g) * 5.5 - 6.0).to(dtype),
        "k": rnd(*shape, scale=0.7),
        "v": rnd(*shape, scale=0.5),
        "a12": rnd(*shape, scale=1.0),
        "k_k": rnd(heads * d, scale=0.2, shift=0.85),
        "a0": rnd(heads * d, scale=0.5),
        "k_a": torch.rand(heads * d, generator=g).to(dtype),
        "bias": rnd(heads, d, scale=0.2) if bias else None,
    }
    n = len(lengths)
    c["cu"] = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    c["slots"] = torch.randperm(n + 3, generator=g)[:n].to(torch.int32)
    c["pool"] = torch.randn((n + 3, heads, d, d), generator=g) * 0.05
    return c


def _expected(c, scale):
    total, heads, d = c["k"].shape
    flat = lambda t: to_np(t).reshape(total, heads * d)   # noqa: E731
    new_k, a, b = kk_a_gate_f64(flat(c["k"]), to_np(c["k_k"]), to_np(c["a0"]), flat(c["a12"]),
                                to_np(c["k_a"]), d)
    shaped = [x.reshape(total, heads, d) for x in (new_k, a, b)]
    y, pool, _, _ = oracle.wkv7_f64(
        to_np(c["r"]), to_np(c["w"]), shaped[0], to_np(c["v"]), shaped[1], shaped[2],
        cu_seqlens=c["cu"].numpy(), state_indices=c["slots"].numpy(),
        state_pool=c["pool"].numpy(),
        decay_bias=None if c["bias"] is None else to_np(c["bias"]), scale=scale)
    return y, pool, shaped[0]


def _run(c, scale, max_seqlen=None):
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_kk_gate_recurrent_forward_varlen
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    pool = dev["pool"].clone()
    y, new_k = infer_tmix_wkv7_kk_gate_recurrent_forward_varlen(
        dev["r"], dev["w"], dev["k"], dev["v"], dev["a12"], k_k=dev["k_k"], a0=dev["a0"],
        k_a=dev["k_a"], state_pool=pool, cu_seqlens=dev["cu"], state_indices=dev["slots"],
        scale=scale, decay_bias=dev["bias"], max_seqlen=max_seqlen)
    torch.cuda.synchronize()
    return y, pool, new_k


def _check_key(actual, expected, dtype):
    a = to_np(actual).astype(np.float64)
    bound = 2.0 ** -_ULP_BITS[dtype] * np.abs(expected) + 1.0e-6
    worst = float(np.max(np.abs(a - expected) - bound))
    assert worst <= 0.0, f"gated key off by {worst:.3e} beyond one ulp"


# 300 sequences x 4 heads = 1 200 units: the chunked kernel with one
# wavefront per unit (the others run on the workgroup-per-unit kernel)
_MANY = tuple((7 * i) % 97 + 5 for i in range(300))
# 100 sequences x 8 heads = 800 units, one of 400 tokens and the rest 50:
# the wavefront kernel in longest-first order of the sequences
_SKEWED = (50,) * 37 + (400,) + (50,) * 62


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("lengths,heads,bias", [
    ((40, 1, 63, 130, 17), 3, False),
    ((300, 64, 96, 41), 4, True),
    (_MANY, 4, True),
    (_SKEWED, 8, True),
], ids=["ragged", "bias", "many-units", "skewed-order-bias"])
def test_fused_kk_gate_matches_the_two_stage_oracle(dtype, lengths, heads, bias):
    require_gpu()
    print(f"case kk-gate fused {dtype} {len(lengths)} sequences H {heads} bias {bias}", flush=True)
    c = _case(lengths, heads, dtype, seed=sum(lengths) + heads, bias=bias)
    y, pool, new_k = _run(c, 0.8)
    ey, epool, ek = _expected(c, 0.8)
    assert_output_close(y, ey)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])
    untouched = sorted(set(range(c["pool"].shape[0])) - set(touched.tolist()))
    assert torch.equal(pool.cpu()[untouched], c["pool"][untouched])
    _check_key(new_k, ek, dtype)


def test_short_batches_run_the_two_kernel_form():
    """Below the chunked threshold (longest sequence <= 4 at this unit count)
    the gate runs as its own kernel (fp16)."""
    require_gpu()
    print("case kk-gate short fp16", flush=True)
    c = _case((1, 4, 3), 2, torch.float16, seed=9)
    y, pool, new_k = _run(c, 1.0)
    ey, epool, ek = _expected(c, 1.0)
    # a and b are rounded to fp16 between the two kernels here
    assert_output_close(y, ey)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])
    _check_key(new_k, ek, torch.float16)


def test_short_bf16_batches_run_the_wavefront_kernel():
    """Below the chunked threshold bf16 batches (whose gate has no separate
    kernel) run the fused stage on the wavefront chunked kernel, which takes
    sequences of any length; with and without the readout stage."""
    require_gpu()
    for lengths, heads, seed in (((2, 4), 2, 11), ((1, 3, 4, 1), 3, 12)):
        print(f"case kk-gate short bf16 lengths {lengths} H {heads}", flush=True)
        c = _case(lengths, heads, torch.bfloat16, seed=seed, bias=seed == 12)
        y, pool, new_k = _run(c, 1.0)
        ey, epool, ek = _expected(c, 1.0)
        assert_output_close(y, ey)
        touched = c["slots"].long()
        assert_state_close(to_np(pool)[touched], epool[touched])
        _check_key(new_k, ek, torch.bfloat16)
        c = _readout_params(c, seed)
        readout, new_k, y, pool = _run_readout(c, 0.7)
        ero, ey, epool, ek = _expected_readout(c, 0.7)
        assert_output_close(readout, ero)
        assert_output_close(y, ey)
        assert_state_close(to_np(pool)[touched], epool[touched])


def test_config1_shape_fp16():
    """BASELINE config 1 (8 x 4096 tokens, 32 heads) through the fused entry."""
    require_gpu()
    print("case kk-gate config-1 shape fp16", flush=True)
    c = _case([4096] * 8, 32, torch.float16, seed=1001)
    y, pool, new_k = _run(c, 1.0)
    ey, epool, ek = _expected(c, 1.0)
    assert_output_close(y, ey)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])
    _check_key(new_k, ek, torch.float16)


def test_few_long_fp16_sequences_take_the_split():
    """Few long fp16 sequences: the library's plan splits them by sequence, so
    the gate runs as its own kernel and the recurrence takes the split."""
    require_gpu()
    from flashrwkv2_amd import _C

    print("case kk-gate long fp16 split", flush=True)
    c = _case([3000], 8, torch.float16, seed=21)
    assert _C.split_plan(1, 8, 64, 3000)[0] > 1
    y, pool, new_k = _run(c, 1.0)
    ey, epool, ek = _expected(c, 1.0)
    assert_output_close(y, ey)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])
    _check_key(new_k, ek, torch.float16)


# ---------------------------------------------------------------------------
# the readout's elementwise stage in the write-back
# ---------------------------------------------------------------------------
def _readout_params(c, seed):
    g = torch.Generator().manual_seed(seed)
    total, heads, d = c["k"].shape
    dtype = c["k"].dtype
    c["g"] = torch.sigmoid(torch.randn((total, heads, d), generator=g)).to(dtype)
    c["r_k"] = (torch.randn(heads * d, generator=g) * 0.3).to(dtype)
    c["ln_w"] = (1.0 + 0.1 * torch.randn(heads * d, generator=g)).to(dtype)
    c["ln_b"] = (0.1 * torch.randn(heads * d, generator=g)).to(dtype)
    return c


def _expected_readout(c, scale):
    """fp64 composition: gate -> recurrence -> readout prelinear, the readout
    reading y and the gated key as rounded to the token dtype (what the
    reference's three kernels pass through HBM)."""
    from oracle.prepare import readout_prelinear_f64

    y, pool, ek = _expected(c, scale)
    total, heads, d = c["k"].shape
    dtype = c["k"].dtype
    rnd = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dtype).double().numpy()  # noqa: E731
    flat = lambda a: np.asarray(a).reshape(total, heads * d)   # noqa: E731
    out = readout_prelinear_f64(flat(rnd(y)), flat(to_np(c["r"])), flat(rnd(ek)),
                                flat(to_np(c["v"])), to_np(c["r_k"]), to_np(c["ln_w"]),
                                to_np(c["ln_b"]), flat(to_np(c["g"])), d)
    return out.reshape(total, heads, d), y, pool, ek


def _run_readout(c, scale, want_y=True):
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    pool = dev["pool"].clone()
    res = infer_tmix_wkv7_kk_gate_recurrent_readout_forward_varlen(
        dev["r"], dev["w"], dev["k"], dev["v"], dev["a12"], dev["g"], k_k=dev["k_k"],
        a0=dev["a0"], k_a=dev["k_a"], r_k=dev["r_k"], ln_weight=dev["ln_w"],
        ln_bias=dev["ln_b"], state_pool=pool, cu_seqlens=dev["cu"], state_indices=dev["slots"],
        scale=scale, decay_bias=dev["bias"], return_wkv_output=want_y)
    torch.cuda.synchronize()
    return (*res, pool)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("lengths,heads,bias", [
    ((40, 1, 63, 130, 17), 3, True),
    ((300, 64, 96, 41), 4, False),
    (_MANY, 4, True),
    (_SKEWED, 8, False),
], ids=["ragged-bias", "long", "many-units", "skewed-order"])
def test_fused_readout_matches_the_three_stage_oracle(dtype, lengths, heads, bias):
    require_gpu()
    print(f"case kk-gate+readout {dtype} {len(lengths)} sequences H {heads} bias {bias}",
          flush=True)
    c = _readout_params(_case(lengths, heads, dtype, seed=7 * sum(lengths) + heads, bias=bias), 3)
    readout, new_k, y, pool = _run_readout(c, 0.9)
    ero, ey, epool, ek = _expected_readout(c, 0.9)
    assert_output_close(readout, ero)
    assert_output_close(y, ey)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])
    _check_key(new_k, ek, dtype)


def test_fused_readout_without_y_and_below_the_threshold():
    """No y requested (the kernel then writes only the readout); and a short
    fp16 batch, where the three stages run as separate kernels."""
    require_gpu()
    for lengths, seed in (((64, 50), 31), ((1, 4, 3), 32)):
        print(f"case kk-gate+readout fp16 lengths {lengths}", flush=True)
        c = _readout_params(_case(lengths, 2, torch.float16, seed=seed), seed)
        readout, new_k, pool = _run_readout(c, 1.0, want_y=False)
        ero, ey, epool, ek = _expected_readout(c, 1.0)
        assert_output_close(readout, ero)
        touched = c["slots"].long()
        assert_state_close(to_np(pool)[touched], epool[touched])


def test_fused_readout_config1_shape_fp16():
    require_gpu()
    print("case kk-gate+readout config-1 shape fp16", flush=True)
    c = _readout_params(_case([4096] * 8, 32, torch.float16, seed=1001), 1001)
    readout, new_k, pool = _run_readout(c, 1.0, want_y=False)
    ero, ey, epool, ek = _expected_readout(c, 1.0)
    assert_output_close(readout, ero)
    touched = c["slots"].long()
    assert_state_close(to_np(pool)[touched], epool[touched])


def test_fused_readout_fails_closed_on_invalid_metadata():
    """Device-detected metadata errors: the fused kernel writes NaN to the
    readout (and y) and leaves the state pool untouched."""
    C = require_gpu()
    print("case kk-gate+readout fail-closed", flush=True)
    c = _readout_params(_case((48,), 2, torch.float16, seed=41), 41)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    bad_cu = torch.tensor([1, 48], device="cuda", dtype=torch.int32)   # must start at 0
    pool = dev["pool"].clone()
    before = pool.clone()
    readout = torch.zeros_like(dev["v"])
    y = torch.zeros_like(dev["v"])
    new_k = torch.zeros_like(dev["k"])
    C.tmix_wkv7_recurrent_fp32_from_kk_gate_readout(
        bad_cu, dev["slots"], pool, dev["r"], dev["w"], dev["k"], dev["v"], dev["a12"], dev["g"],
        dev["k_k"], dev["a0"], dev["k_a"], dev["r_k"], dev["ln_w"], dev["ln_b"], new_k, readout,
        y, 1.0, None, None, 48)
    torch.cuda.synchronize()
    assert torch.isnan(readout).all()
    assert torch.isnan(y).all()
    assert torch.equal(pool, before)
