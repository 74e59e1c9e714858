"""Views with an odd storage offset (misaligned for the kernels' 16-byte
accesses) are accepted, as the reference accepts any contiguous view: the
native layer runs the call on aligned copies and copies back (CPU: the
wrapper's bookkeeping; GPU: results equal the aligned call's)."""

from __future__ import annotations

import pytest
import torch

from flashrwkv2_amd._align import aligned_io

pytestmark = []


def _offset_view(x: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of x whose data pointer is 2 bytes past a 16-byte
    boundary."""
    flat = torch.empty(x.numel() + 8, dtype=x.dtype, device=x.device)
    v = flat[1:1 + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.is_contiguous() and v.data_ptr() % 16 != 0
    return v


def test_wrapper_swaps_misaligned_tensors_and_copies_back():
    seen = {}

    def fn(x, y, out, *, pool):
        for name, t in (("x", x), ("y", y), ("out", out), ("pool", pool)):
            seen[name] = t.data_ptr() % 16
        out.copy_(x + y)
        pool.add_(1.0)
        return out, pool

    wrapped = aligned_io(fn)
    x = _offset_view(torch.arange(24, dtype=torch.float16).view(4, 6))
    y = torch.ones(4, 6, dtype=torch.float16)
    out = _offset_view(torch.zeros(4, 6, dtype=torch.float16))
    pool = _offset_view(torch.zeros(3, dtype=torch.float32))
    o, p = wrapped(x, y, out, pool=pool)
    assert all(v == 0 for v in seen.values()), seen
    assert o is out and p is pool
    assert torch.equal(out, torch.arange(24, dtype=torch.float16).view(4, 6) + 1)
    assert torch.equal(pool, torch.ones(3))


def test_wrapper_passes_aligned_arguments_through():
    args = []
    wrapped = aligned_io(lambda *a: args.extend(a))
    t = torch.zeros(8, dtype=torch.bfloat16)
    i = torch.zeros(3, dtype=torch.int32)
    wrapped(t, i, 1.0)
    assert args[0] is t and args[1] is i


@pytest.mark.gpu
def test_misaligned_token_views_match_the_aligned_call():
    from wkv7_testlib import make_case, require_gpu, tokens

    require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_recurrent_fp32io16_forward_varlen

    print("case misaligned views, lengths (37, 100), H=2, decay bias", flush=True)
    case = make_case(lengths=(37, 100), num_heads=2, seed=91)
    toks = tokens(case)
    bias = torch.randn((2, 64), device="cuda").to(toks[0].dtype)
    pool_a = case["state_pool"].clone()
    y_a = infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
        *toks, state_pool=pool_a, cu_seqlens=case["cu_seqlens"],
        state_indices=case["state_indices"], decay_bias=bias)
    pool_b = case["state_pool"].clone()
    y_b = infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
        *(_offset_view(t) for t in toks), state_pool=pool_b, cu_seqlens=case["cu_seqlens"],
        state_indices=case["state_indices"], decay_bias=_offset_view(bias))
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b)
    assert torch.equal(pool_a, pool_b)
