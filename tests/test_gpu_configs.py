"""BASELINE configurations at their full shapes through the public entry,
against the fp64 CPU oracle on exactly the kernel's inputs.

Config 3 (varlen packed prefill, 7B-class head layout): 64 sequences with
lengths ~ U{1..2048}, H = 64, per-sequence fp32 initial states ~ N(0, 0.1).
The mix of short and long sequences in one chunked launch is the case the
reduced tests do not reach.  Gates as everywhere else (tests/wkv7_testlib.py):
relative RMSE 2e-3 and |dy| <= 2e-2 max(1, |y|) on outputs, relative
Frobenius 1e-3 per (slot, head) on states.
"""

from __future__ import annotations

import pytest
import torch

from wkv7_testlib import assert_output_close, assert_state_close, require_gpu, to_np

import oracle

pytestmark = pytest.mark.gpu


def test_config3_full_shape_matches_the_oracle():
    require_gpu()
    from flashrwkv2_amd import workloads
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_recurrent_fp32io16_forward_varlen

    w = workloads.config(3, "cuda")
    lengths = (w.cu_seqlens[1:] - w.cu_seqlens[:-1]).cpu()
    print(f"case config 3: {w.state_indices.numel()} sequences, sum T {w.total_tokens}, "
          f"H {w.num_heads}, lengths {int(lengths.min())}..{int(lengths.max())}", flush=True)
    assert w.state_indices.numel() == 64 and w.num_heads == 64
    assert int(lengths.max()) > 1024 and int(lengths.min()) < 128
    # slots permuted so that sequence n does not update slot n
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    slots = perm.cuda()
    pool = torch.cat([w.state_pool, torch.zeros_like(w.state_pool[:4])])   # 4 untouched slots
    pool[64:] = 7.0
    pool_in = pool.clone()
    out = infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
        *w.tokens, state_pool=pool, cu_seqlens=w.cu_seqlens, state_indices=slots)
    torch.cuda.synchronize()
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(
        *(to_np(t) for t in w.tokens), cu_seqlens=w.cu_seqlens.cpu().numpy(),
        state_indices=perm.numpy(), state_pool=to_np(pool_in))
    assert_output_close(to_np(out), y_ref)
    assert_state_close(to_np(pool[:64]), pool_ref[:64])
    assert torch.equal(pool[64:], pool_in[64:])


def test_config1_full_shape_bf16_entry_matches_the_oracle():
    """BASELINE config 1 (the headline prefill: B 8, T 4096, H 32, bf16
    tokens, zero fp32 start state) through the public bf16 entry
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen, with permuted slots and
    untouched slots, against the fp64 oracle (tests/tmix/wkv7/test.py:29-85
    of the reference is the contract)."""
    require_gpu()
    from flashrwkv2_amd import _C as CC
    from flashrwkv2_amd import workloads
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_recurrent_fp32io16_forward_varlen

    w = workloads.config(1, "cuda")
    n = w.state_indices.numel()
    print(f"case config 1: {n} sequences x {w.total_tokens // n} tokens, H {w.num_heads}, "
          f"kernel {CC.dispatch_kernel_name(n, w.num_heads, 64, w.total_tokens, 4096)}",
          flush=True)
    assert n == 8 and w.num_heads == 32 and w.total_tokens == 8 * 4096
    assert w.tokens[0].dtype == torch.bfloat16
    perm = torch.tensor([5, 2, 7, 0, 3, 6, 1, 4], dtype=torch.int32)
    pool = torch.cat([w.state_pool, torch.zeros_like(w.state_pool[:3])])   # 3 untouched slots
    pool[8:] = -3.0
    pool_in = pool.clone()
    out = infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
        *w.tokens, state_pool=pool, cu_seqlens=w.cu_seqlens, state_indices=perm.cuda())
    torch.cuda.synchronize()
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(
        *(to_np(t) for t in w.tokens), cu_seqlens=w.cu_seqlens.cpu().numpy(),
        state_indices=perm.numpy(), state_pool=to_np(pool_in))
    assert_output_close(to_np(out), y_ref)
    assert_state_close(to_np(pool[:8]), pool_ref[:8])
    assert torch.equal(pool[8:], pool_in[8:])
