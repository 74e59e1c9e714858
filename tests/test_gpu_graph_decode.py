"""Graph-captured serving decode loop (T = 1 steps) on the graph-ticket path.

The reference's graph contract (tests/tmix/wkv7/test.py:239-373) captures one
ticket + recurrence pair.  A serving loop captures many consecutive decode
steps in one graph: every step re-validates the live metadata on the device
(no host synchronisation inside the graph) and carries the state pool to the
next step.  Each replay must equal the same steps run eagerly, bit for bit,
with eager work between replays; changing the live active count between
replays must leave the padded slots untouched.
"""

from __future__ import annotations

import pytest
import torch

from wkv7_testlib import assert_output_close, assert_state_close, oracle_expect, require_gpu

pytestmark = [pytest.mark.gpu, pytest.mark.cuda_graph]

from flashrwkv2_amd.tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
    prepare_tmix_wkv7_recurrent_metadata,
)

STEPS, SEQ_CAP, SLOTS, H, D = 6, 48, 64, 4, 64


def _tokens(g, dev):
    """STEPS x (r, logits, k, v, a, b) of [SEQ_CAP, H, D] fp16; kk-structured a/b."""
    out = []
    for _ in range(STEPS):
        r, k, v = (torch.randn((SEQ_CAP, H, D), generator=g) for _ in range(3))
        logits = torch.randn((SEQ_CAP, H, D), generator=g) * 1.5
        kk = torch.randn((SEQ_CAP, H, D), generator=g)
        kk = kk / kk.norm(dim=-1, keepdim=True)
        gate = torch.sigmoid(torch.randn((SEQ_CAP, H, D), generator=g))
        out.append(tuple(t.half().to(dev) for t in (r, logits, k, v, -kk, kk * gate)))
    return out


def _step_all(steps, state, cu, idx, live):
    outs = []
    for toks in steps:
        ticket = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
        outs.append(wkv7(*toks, state_pool=state, cu_seqlens=cu, state_indices=idx,
                         validated_metadata=ticket))
    return outs


def test_graph_decode_loop_matches_eager_and_oracle():
    require_gpu()
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(777)
    steps = _tokens(g, dev)
    initial = (torch.randn((SLOTS, H, D, D), generator=g) * 0.1).to(dev)
    perm = torch.randperm(SLOTS, generator=g)[:SEQ_CAP].to(torch.int32)
    cu = torch.arange(SEQ_CAP + 1, dtype=torch.int32).to(dev)
    idx = perm.to(dev)
    n_tok = torch.full((1,), SEQ_CAP, device=dev, dtype=torch.int32)
    n_seq = torch.full((1,), SEQ_CAP, device=dev, dtype=torch.int32)
    live = dict(state_pool_size=SLOTS, token_capacity=SEQ_CAP, sequence_capacity=SEQ_CAP,
                max_seqlen_capacity=1, num_active_tokens=n_tok, num_active_sequences=n_seq)

    # eager reference of the whole loop
    eager_state = initial.clone()
    eager_outs = _step_all(steps, eager_state, cu, idx, live)
    torch.cuda.synchronize()

    # and against the fp64 oracle, step by step
    pool = initial.clone()
    for s, toks in enumerate(steps):
        case = dict(zip(("r", "decay_logits", "k", "v", "a", "b"), toks))
        case.update(cu_seqlens=cu, state_indices=idx, state_pool=pool, decay_bias=None)
        y_ref, pool_ref = oracle_expect(case)
        assert_output_close(eager_outs[s], y_ref)
        pool = torch.from_numpy(pool_ref).float().to(dev)
    assert_state_close(eager_state, pool_ref)

    state = initial.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):       # warm the capture shapes
        _step_all(steps, state, cu, idx, live)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = _step_all(steps, state, cu, idx, live)
    for _ in range(3):
        state.copy_(initial)
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for s in range(STEPS):
            assert torch.equal(outs[s], eager_outs[s]), s
        assert torch.equal(state, eager_state)

    # fewer live sequences: the tail slots keep their initial state
    half = SEQ_CAP // 2
    n_tok.fill_(half)
    n_seq.fill_(half)
    state.copy_(initial)
    graph.replay()
    torch.cuda.synchronize()
    live_slots = perm[:half].long().to(dev)
    idle_slots = perm[half:].long().to(dev)
    assert torch.equal(state[idle_slots], initial[idle_slots])
    assert torch.equal(state[live_slots], eager_state[live_slots])
