"""The chunked kernels' bounded wave hand-off fails closed.

Every wait between the key and state waves of the chunked MFMA kernel is
bounded.  A wait that gives up must not pass wrong numbers off as results: the
block writes NaN outputs, leaves its state slots untouched and counts itself
in the library's fault counter.  The test forces the give-up from the host
with a spin limit of zero polls (the state waves' first wait then always
finds its counter short, since the key waves cannot have built any operator
yet), so every kernel still runs to its normal end.
"""

from __future__ import annotations

import numpy as np
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


@pytest.fixture(autouse=True)
def _default_chunk_variant():
    """Tests that select the workgroup chunked kernel's variant leave the
    default (the ring variant) behind, pass or fail."""
    yield
    if torch.cuda.is_available():
        require_gpu()._set_chunk_ring(True)

CHUNKED = 2


def _forced_chunked(C, case, pool):
    from flashrwkv2_amd.tmix.wkv7 import prepare_tmix_wkv7_recurrent_metadata

    out = torch.empty_like(case["v"])
    ticket = prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=pool.shape[0])
    C.tmix_wkv7_recurrent_fp32_kernel_forced(
        CHUNKED, case["cu_seqlens"], case["state_indices"], pool, *tokens(case), out, 1.0,
        case["decay_bias"], ticket)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("ring", [True, False])
def test_handoff_give_up_fails_closed_and_is_counted(ring):
    C = require_gpu()
    print(f"case handoff spin limit 0, lengths (200, 300), H=2, ring={ring}", flush=True)
    C._set_chunk_ring(ring)
    case = make_case(lengths=(200, 300), num_heads=2, seed=71)
    C.handoff_fault_count(reset=True)
    pool = case["state_pool"].clone()
    before = pool.clone()
    C._set_handoff_spin_limit(0)
    try:
        out = _forced_chunked(C, case, pool)
    finally:
        C._set_handoff_spin_limit(-1)
    faults = C.handoff_fault_count(reset=True)
    # one block per (sequence, head), each gives up at its first wait
    assert faults == 4, faults
    assert torch.isnan(out.float()).all()
    assert torch.equal(pool, before), "a failed-closed block must leave its state untouched"

    # default limit again: no fault, results match the oracle
    pool = case["state_pool"].clone()
    out = _forced_chunked(C, case, pool)
    assert C.handoff_fault_count(reset=True) == 0
    y_ref, pool_ref = oracle_expect(case)
    assert_output_close(to_np(out), y_ref)
    assert_state_close(to_np(pool), pool_ref)
    C._set_chunk_ring(True)


@pytest.mark.parametrize("ring", [True, False])
def test_real_stall_fails_closed_after_one_wait(ring):
    """A producer that never publishes (forced from the host: the key waves
    skip their operator signal) makes the first operator wait give up; every
    later wait of that block must then return at once instead of polling to
    its limit, so a long sequence still ends in about one wait's limit."""
    import time

    C = require_gpu()
    print(f"case handoff stall, spin limit 20000, length 16384, H=1, ring={ring}", flush=True)
    C._set_chunk_ring(ring)
    case = make_case(lengths=(16384,), num_heads=1, seed=72)
    C.handoff_fault_count(reset=True)
    pool = case["state_pool"].clone()
    before = pool.clone()
    _forced_chunked(C, make_case(lengths=(64,), num_heads=1, seed=73),
                    make_case(lengths=(64,), num_heads=1, seed=73)["state_pool"].clone())
    C._set_handoff_spin_limit(20000)
    C._set_handoff_stall(True)
    try:
        t0 = time.perf_counter()
        out = _forced_chunked(C, case, pool)
        dt = time.perf_counter() - t0
    finally:
        C._set_handoff_stall(False)
        C._set_handoff_spin_limit(-1)
        C._set_chunk_ring(True)
    print(f"stalled call took {dt * 1e3:.1f} ms", flush=True)
    assert C.handoff_fault_count(reset=True) == 1
    assert torch.isnan(out.float()).all()
    assert torch.equal(pool, before)
    # 512 groups; polling every hand-off to the limit takes seconds
    assert dt < 0.5, dt


@pytest.mark.parametrize("ring", [True, False])
def test_value_pass_give_up_fails_closed(ring):
    """The training backward's value pass (the chunked kernel's reverse mode)
    under a spin limit of zero: every block gives up at its first wait,
    counts itself and writes NaN for dv (and for the dsa the key pass reads),
    so no finite gradient of v comes out of a failed hand-off."""
    C = require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import pretrain_tmix_wkv7_recurrent_bf16

    print(f"case value pass spin limit 0, B=2 T=64 H=2, ring={ring}", flush=True)
    C._set_chunk_ring(ring)
    g = torch.Generator().manual_seed(74)
    shape = (2, 64, 2 * 64)
    vals = [(torch.randn(shape, generator=g) * 0.1).to(torch.bfloat16).cuda().requires_grad_()
            for _ in range(6)]
    dy = torch.randn(shape, generator=g).to(torch.bfloat16).cuda()
    y = pretrain_tmix_wkv7_recurrent_bf16(*vals, head_size=64)   # forward at the normal limit
    torch.cuda.synchronize()
    C.handoff_fault_count(reset=True)
    C._set_handoff_spin_limit(0)
    try:
        y.backward(dy)
        torch.cuda.synchronize()
    finally:
        C._set_handoff_spin_limit(-1)
        C._set_chunk_ring(True)
    assert C.handoff_fault_count(reset=True) == 4   # one per (batch, head) block
    assert torch.isnan(vals[3].grad.float()).all()
