"""GPU parity of the sequence-split chunked prefill (few long sequences).

A split run cuts every sequence into pieces: a summary pass computes each
piece's zero-start final state F and transition Phi, a combine kernel chains
S(j+1) = Phi_j S(j) + F_j, and the chunked kernel runs the pieces from those
start states.  The results must match the fp64 oracle on exactly the
kernel's inputs with the same gates as the unsplit kernels (relative RMSE
2e-3 from tests/fixtures/tolerances-v1.json:9-12 of the reference, plus
|dy| <= 2e-2 max(1, |y|) and ||dS|| / ||S|| <= 1e-3 per (slot, head)), and
agree with the unsplit chunked kernel to fp32-level accuracy.
"""

from __future__ import annotations

import pytest
import torch

from wkv7_testlib import (
    assert_output_close,
    assert_state_close,
    make_case,
    oracle_expect,
    require_gpu,
    tokens,
)

pytestmark = pytest.mark.gpu

from flashrwkv2_amd.tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
    prepare_tmix_wkv7_recurrent_metadata,
)

CHUNKED, SPLIT = 2, 3


def _forced(C, kernel, case, pool, scale=1.0, pieces=None):
    out = torch.empty_like(case["v"])
    ticket = prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=pool.shape[0])
    C.tmix_wkv7_recurrent_fp32_kernel_forced(
        kernel, case["cu_seqlens"], case["state_indices"], pool, *tokens(case), out, scale,
        case["decay_bias"], ticket, split_pieces=pieces)
    torch.cuda.synchronize()
    return out


def _close_to_unsplit(y_split, y_chunk, p_split, p_chunk, active):
    dy = y_split.float() - y_chunk.float()
    rel = (dy.square().mean().sqrt() / y_chunk.float().square().mean().sqrt()).item()
    assert rel <= 2e-3, rel   # two bf16/fp16 roundings of nearly the same value
    ds = (p_split[active] - p_chunk[active]).flatten(0, 1).norm(dim=(1, 2))
    base = p_chunk[active].flatten(0, 1).norm(dim=(1, 2))
    assert (ds / base).max().item() <= 1e-4


@pytest.mark.parametrize("lengths,pieces", [
    ((1024,), 2),
    ((1024,), 4),
    ((700, 64, 1, 129, 1024), 4),       # sequences of 1..4 pieces, ragged last pieces
    ((2000, 33), 3),
    ((96, 96, 96), 3),                  # pieces of 32 tokens
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_matches_oracle_and_unsplit(lengths, pieces, dtype):
    C = require_gpu()
    print(f"case split lengths={lengths} pieces={pieces} dtype={dtype}", flush=True)
    case = make_case(dtype=dtype, head_size=64, lengths=lengths, with_decay_bias=True,
                     num_heads=3)
    y_ref, pool_ref = oracle_expect(case, scale=0.75)
    active = case["state_indices"].long()
    p_split = case["state_pool"].clone()
    before = p_split.clone()
    y_split = _forced(C, SPLIT, case, p_split, scale=0.75, pieces=pieces)
    assert_output_close(y_split, y_ref)
    assert_state_close(p_split[active], pool_ref[active.cpu().numpy()])
    untouched = [i for i in range(before.shape[0]) if i not in set(active.tolist())]
    assert torch.equal(p_split[untouched], before[untouched])
    p_chunk = case["state_pool"].clone()
    y_chunk = _forced(C, CHUNKED, case, p_chunk, scale=0.75)
    _close_to_unsplit(y_split, y_chunk, p_split, p_chunk, active)
    # deterministic
    p2 = case["state_pool"].clone()
    y2 = _forced(C, SPLIT, case, p2, scale=0.75, pieces=pieces)
    assert torch.equal(y2, y_split) and torch.equal(p2, p_split)


def test_public_call_splits_a_long_single_sequence():
    """B = 1 prefill (4 heads): the public entry takes the split by itself
    (the plan gives 8 pieces of 1024 tokens) and matches the oracle."""
    C = require_gpu()
    from flashrwkv2_amd import _C as CC

    assert CC.split_plan(1, 4, 64, 8192)[:2] == (8, 1024)
    assert CC.split_plan(8, 32, 64, 4096)[0] == 1      # config 1: 256 units, no split
    case = make_case(dtype=torch.bfloat16, head_size=64, lengths=(8192,), num_heads=4,
                     seed=7)
    y_ref, pool_ref = oracle_expect(case)
    out = wkv7(*tokens(case), state_pool=case["state_pool"], cu_seqlens=case["cu_seqlens"],
               state_indices=case["state_indices"])
    torch.cuda.synchronize()
    active = case["state_indices"].long()
    assert_output_close(out, y_ref)
    assert_state_close(case["state_pool"][active], pool_ref[active.cpu().numpy()])


def test_split_fails_closed_on_invalid_metadata():
    """Device-detected metadata errors: NaN output, state pool untouched, on
    every kernel of the split (summary, combine, pieces)."""
    C = require_gpu()
    case = make_case(dtype=torch.bfloat16, lengths=(2048,))
    pool = case["state_pool"]
    bad_cu = torch.tensor([1, 2048], device="cuda", dtype=torch.int32)
    slots = torch.tensor([0], device="cuda", dtype=torch.int32)
    out = torch.zeros_like(case["v"])
    before = pool.clone()
    C.tmix_wkv7_recurrent_fp32_kernel_forced(SPLIT, bad_cu, slots, pool, *tokens(case), out,
                                             1.0, None, None, split_pieces=4)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    assert torch.equal(pool, before)
