"""GPU parity of the sequence-split chunked prefill (few long sequences).

A split run cuts every sequence into pieces: a summary pass computes each
piece's zero-start final state F and transition Phi, a combine kernel chains
S(j+1) = Phi_j S(j) + F_j, and the chunked kernel runs the pieces from those
start states.  The classic split (equal pieces) chains from the slot state;
the pipelined split runs piece 0 (its own length) from the slot state on a
second stream next to the summary pass and chains from its end state.  The results must match the fp64 oracle on exactly the
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
    # pipelined split: (pieces, piece 0's length)
    ((1024,), (2, 512)),                # no summary pass, no combine
    ((1024,), (4, 352)),
    ((700, 64, 1, 129, 1024), (4, 320)),   # sequences ending inside piece 0 and later
    ((2000, 33), (3, 1024)),
    ((96, 96, 96), (3, 32)),
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
    (the plan cuts it into pieces of at least 384 tokens) and matches the oracle."""
    C = require_gpu()
    from flashrwkv2_amd import _C as CC

    pieces, plen, lead, _ = CC.split_plan(1, 4, 64, 8192)
    assert pieces >= 3 and plen >= 384 and lead >= plen and lead % 32 == 0 == plen % 32
    assert lead + (pieces - 2) * plen < 8192 <= lead + (pieces - 1) * plen
    assert CC.split_plan(1, 64, 64, 65536)[:3] == (5, 12992, 13568)   # config 4
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
    for pieces in (4, (4, 640)):
        out.zero_()
        C.tmix_wkv7_recurrent_fp32_kernel_forced(SPLIT, bad_cu, slots, pool, *tokens(case),
                                                 out, 1.0, None, None, split_pieces=pieces)
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all()
        assert torch.equal(pool, before)


@pytest.mark.cuda_graph
def test_split_under_graph_capture_with_live_metadata():
    """Graph ticket (live cu_seqlens / counts, capacity-sized plan): the split
    path is captured once (its workspace comes from the graph's pool) and
    every replay equals the eager call on the same ticket kind and the
    oracle; a replay after the live metadata changed follows the new
    sequences."""
    C = require_gpu()
    from flashrwkv2_amd import _C as CC

    dev = torch.device("cuda")
    case = make_case(dtype=torch.bfloat16, head_size=64, lengths=(3000, 1000), num_heads=2,
                     seed=11)
    packed = tokens(case)
    slots_n = case["state_pool"].shape[0]
    initial = case["state_pool"].clone()
    cu = torch.tensor([0, 3000, 4000], device=dev, dtype=torch.int32)
    idx = case["state_indices"].clone()
    n_tok = torch.full((1,), 4000, device=dev, dtype=torch.int32)
    n_seq = torch.full((1,), 2, device=dev, dtype=torch.int32)
    live = dict(state_pool_size=slots_n, token_capacity=4000, sequence_capacity=2,
                max_seqlen_capacity=4000, num_active_tokens=n_tok, num_active_sequences=n_seq)
    assert CC.split_plan(2, 2, 64, 4000)[0] >= 3           # the capacity plan splits
    y_ref, pool_ref = oracle_expect(case)
    active = case["state_indices"].long()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        eager_state = initial.clone()
        t_eager = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
        eager = wkv7(*packed, state_pool=eager_state, cu_seqlens=cu, state_indices=idx,
                     validated_metadata=t_eager)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert_output_close(eager, y_ref)
    assert_state_close(eager_state[active], pool_ref[active.cpu().numpy()])
    state = initial.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ticket = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
        graph_out = wkv7(*packed, state_pool=state, cu_seqlens=cu, state_indices=idx,
                         validated_metadata=ticket)
    for _ in range(3):
        state.copy_(initial)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out, eager)
        assert torch.equal(state, eager_state)
    # one live sequence of 2500 tokens: the replay follows the new metadata
    state.copy_(initial)
    cu.copy_(torch.tensor([0, 2500, -1], device=dev, dtype=torch.int32))
    n_tok.fill_(2500)
    n_seq.fill_(1)
    graph.replay()
    torch.cuda.synchronize()
    one = dict(case)
    one.update({n: t[:2500] for n, t in zip(("r", "decay_logits", "k", "v", "a", "b"), packed)})
    one["cu_seqlens"] = torch.tensor([0, 2500], device=dev, dtype=torch.int32)
    one["state_indices"] = idx[:1].clone()
    y1, p1 = oracle_expect(one, state_pool=initial)
    assert_output_close(graph_out[:2500], y1)
    s0 = int(idx[0])
    assert_state_close(state[s0:s0 + 1], p1[s0:s0 + 1])
    others = [i for i in range(slots_n) if i != s0]
    assert torch.equal(state[others], initial[others])
