"""The native per-step fast path (csrc/hostpath.cpp) against the full path.

For a ticketed call without decay bias the public wrapper first asks the
native fast path; when the call is plainly valid there, it launches and the
Python checks are skipped.  These tests check that (a) the fast path is
actually taken for the serving-loop calls, (b) its results equal the full
Python path's bit for bit (same kernels, same arguments), and (c) every
call it declines still gets the full path's behaviour: decay bias, ticket
mismatches and bad arguments raise the same errors as before.
"""

from __future__ import annotations

import pytest
import torch

from wkv7_testlib import make_case, require_gpu, tokens

pytestmark = pytest.mark.gpu


def _counting(monkeypatch, C, name):
    seen = {"taken": 0, "declined": 0}
    inner = getattr(C, name)

    def wrapped(*args, **kwargs):
        out = inner(*args, **kwargs)
        seen["taken" if out is not None else "declined"] += 1
        return out

    monkeypatch.setattr(C, name, wrapped)
    return seen


@pytest.mark.parametrize("lengths", [(1,) * 8, (1, 3, 2, 4), (60, 1, 45)],
                         ids=["decode", "short", "chunked"])
def test_fast_path_is_taken_and_equals_the_full_path(monkeypatch, lengths):
    C = require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import (
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
        prepare_tmix_wkv7_recurrent_metadata as prep,
    )

    print(f"case hostpath lengths {lengths}", flush=True)
    case = make_case(lengths=lengths, num_heads=4, seed=5)
    n = len(lengths)
    dev = case["r"].device
    total = case["r"].shape[0]
    rec = _counting(monkeypatch, C, "_recurrent_fp32_fast")
    grf = _counting(monkeypatch, C, "_prepare_graph_fast")
    n_tok = torch.full((1,), total, device=dev, dtype=torch.int32)
    n_seq = torch.full((1,), n, device=dev, dtype=torch.int32)
    live = dict(state_pool_size=case["state_pool"].shape[0], token_capacity=total,
                sequence_capacity=n, max_seqlen_capacity=max(lengths),
                num_active_tokens=n_tok, num_active_sequences=n_seq)

    for ticket_kind in ("graph", "static"):
        if ticket_kind == "graph":
            ticket = prep(case["cu_seqlens"], case["state_indices"], **live)
        else:
            ticket = prep(case["cu_seqlens"], case["state_indices"], total_tokens=total,
                          state_pool_size=case["state_pool"].shape[0])
        pool_fast = case["state_pool"].clone()
        y_fast = wkv7(*tokens(case), state_pool=pool_fast, cu_seqlens=case["cu_seqlens"],
                      state_indices=case["state_indices"], validated_metadata=ticket)
        pool_full = case["state_pool"].clone()
        y_full = torch.empty_like(case["v"])
        C.tmix_wkv7_recurrent_fp32_from_decay_logits(
            case["cu_seqlens"], case["state_indices"], pool_full, *tokens(case), y_full, 1.0,
            None, ticket)
        torch.cuda.synchronize()
        assert torch.equal(y_fast, y_full), ticket_kind
        assert torch.equal(pool_fast, pool_full), ticket_kind
    assert rec["taken"] == 2 and rec["declined"] == 0, rec
    assert grf["taken"] == 1 and grf["declined"] == 0, grf


def test_declined_calls_keep_the_full_paths_behaviour(monkeypatch):
    C = require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import (
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
        prepare_tmix_wkv7_recurrent_metadata as prep,
    )

    print("case hostpath declines", flush=True)
    case = make_case(lengths=(1, 1, 1), num_heads=2, seed=6, with_decay_bias=True)
    total = case["r"].shape[0]
    pool_size = case["state_pool"].shape[0]
    rec = _counting(monkeypatch, C, "_recurrent_fp32_fast")
    ticket = prep(case["cu_seqlens"], case["state_indices"], total_tokens=total,
                  state_pool_size=pool_size)

    # decay bias: not taken by the fast path, same result as the full path
    pool_a = case["state_pool"].clone()
    y_a = wkv7(*tokens(case), state_pool=pool_a, cu_seqlens=case["cu_seqlens"],
               state_indices=case["state_indices"], validated_metadata=ticket,
               decay_bias=case["decay_bias"])
    pool_b = case["state_pool"].clone()
    y_b = torch.empty_like(case["v"])
    C.tmix_wkv7_recurrent_fp32_from_decay_logits(
        case["cu_seqlens"], case["state_indices"], pool_b, *tokens(case), y_b, 1.0,
        case["decay_bias"], ticket)
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b) and torch.equal(pool_a, pool_b)
    assert rec["taken"] == 0

    # ticket bound to other metadata tensors: the full path's identity error
    other = case["cu_seqlens"].clone()
    with pytest.raises(RuntimeError, match="query_start_loc identity mismatch"):
        wkv7(*tokens(case), state_pool=case["state_pool"].clone(), cu_seqlens=other,
             state_indices=case["state_indices"], validated_metadata=ticket)
    # metadata modified in place after validation: the version check
    qsl = case["cu_seqlens"].clone()
    t2 = prep(qsl, case["state_indices"], total_tokens=total, state_pool_size=pool_size)
    qsl.add_(0)
    with pytest.raises(RuntimeError, match="version mismatch"):
        wkv7(*tokens(case), state_pool=case["state_pool"].clone(), cu_seqlens=qsl,
             state_indices=case["state_indices"], validated_metadata=t2)
    # a non-finite scale
    with pytest.raises(RuntimeError, match="scale must be finite"):
        wkv7(*tokens(case), state_pool=case["state_pool"].clone(),
             cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"],
             validated_metadata=ticket, scale=float("nan"))
    # a wrong token dtype
    bad = list(tokens(case))
    bad[2] = bad[2].float()
    with pytest.raises((RuntimeError, TypeError, ValueError)):
        wkv7(*bad, state_pool=case["state_pool"].clone(), cu_seqlens=case["cu_seqlens"],
             state_indices=case["state_indices"], validated_metadata=ticket)
    assert rec["taken"] == 0, rec
