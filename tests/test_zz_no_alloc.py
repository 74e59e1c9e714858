"""The no-allocation split entry (fr2_wkv7_recurrent_fp32_forward_split_noalloc)
against the allocating one (fr2_wkv7_recurrent_fp32_forward_split).

Both run the same split plan on the same inputs, called through the C ABI;
the no-allocation form keeps its workspace in the library's device scratch
array.  Two calls in a row, the second with a smaller input, check that the
scratch left by the first call does not leak into the second.  The split
runs the same kernels on one stream either way, so the outputs and states
must be bit-identical; the first case is also checked against the fp64
oracle.  A plan larger than the scratch must be rejected.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from wkv7_testlib import (
    assert_output_close,
    assert_state_close,
    make_case,
    oracle_expect,
    require_gpu,
    to_np,
    tokens,
)

pytestmark = pytest.mark.gpu


def _ticket(case, pool):
    from flashrwkv2_amd.tmix.wkv7 import prepare_tmix_wkv7_recurrent_metadata

    return prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=pool.shape[0])


def _args(case, pool, out, ticket, max_seqlen):
    from flashrwkv2_amd import _native as N

    r = case["r"]
    bias = case["decay_bias"]
    return (ticket._query_start_loc_snapshot().data_ptr(),
            ticket._state_indices_snapshot().data_ptr(), ticket._status().data_ptr(),
            case["state_indices"].numel(), r.shape[1], r.shape[2], r.shape[0], max_seqlen,
            N.FR2_DTYPE_BFLOAT16 if r.dtype == torch.bfloat16 else N.FR2_DTYPE_FLOAT16,
            pool.data_ptr(), *(t.data_ptr() for t in tokens(case)[:2]),
            None if bias is None else bias.data_ptr(),
            *(t.data_ptr() for t in tokens(case)[2:]), out.data_ptr(), 0.75)


def _both(case, pieces):
    from flashrwkv2_amd import _C as C
    from flashrwkv2_amd import _native as N

    lib = N.load()
    n, h = case["state_indices"].numel(), case["r"].shape[1]
    lengths = (case["cu_seqlens"][1:] - case["cu_seqlens"][:-1])
    max_seqlen = int(lengths.max())
    pc, plen, lead, ws_bytes = C.split_plan(n, h, 64, max_seqlen, pieces)
    assert pc >= 2
    stream = torch.cuda.current_stream().cuda_stream
    results = []
    for noalloc in (False, True):
        pool = case["state_pool"].clone()
        out = torch.empty_like(case["v"])
        ticket = _ticket(case, pool)
        args = _args(case, pool, out, ticket, max_seqlen)
        if noalloc:
            rc = lib.fr2_wkv7_recurrent_fp32_forward_split_noalloc(*args, pc, plen, lead, stream)
        else:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
            rc = lib.fr2_wkv7_recurrent_fp32_forward_split(*args, pc, plen, lead, ws.data_ptr(),
                                                           ws_bytes, stream, None)
        N.check(rc, "split")
        torch.cuda.synchronize()
        results.append((out, pool))
    return results


def test_noalloc_split_matches_the_allocating_entry_on_two_calls():
    require_gpu()
    print("case noalloc split: 2 x 1500 tokens H=8 (lead split), then 1 x 700 H=3", flush=True)
    big = make_case(lengths=(1500, 1500), num_heads=8, seed=5, with_decay_bias=True)
    (y_a, p_a), (y_n, p_n) = _both(big, (4, 512))
    assert torch.equal(y_a, y_n) and torch.equal(p_a, p_n)
    y_ref, pool_ref = oracle_expect(big, scale=0.75)
    active = big["state_indices"].long()
    assert_output_close(to_np(y_n), y_ref)
    assert_state_close(to_np(p_n[active]), pool_ref[active.cpu().numpy()])
    print("case noalloc split: second, smaller call", flush=True)
    small = make_case(lengths=(700,), num_heads=3, seed=6)
    (y_a, p_a), (y_n, p_n) = _both(small, 3)
    assert torch.equal(y_a, y_n) and torch.equal(p_a, p_n)


def test_noalloc_split_rejects_a_plan_beyond_the_scratch():
    require_gpu()
    from flashrwkv2_amd import _native as N

    lib = N.load()
    case = make_case(lengths=(640,), num_heads=2, seed=9)
    pool = case["state_pool"].clone()
    out = torch.empty_like(case["v"])
    ticket = _ticket(case, pool)
    args = list(_args(case, pool, out, ticket, 640))
    # 300 sequences x 64 heads x (3*4 - 2) x 16 KiB is far beyond 16 MiB; the
    # size check runs before anything is launched
    args[3], args[4] = 300, 64
    before = pool.clone()
    rc = lib.fr2_wkv7_recurrent_fp32_forward_split_noalloc(
        *args, 4, 160, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == N.FR2_ERR_INVALID_ARGUMENT
    assert b"scratch" in lib.fr2_last_error()
    torch.cuda.synchronize()
    assert torch.equal(pool, before)
