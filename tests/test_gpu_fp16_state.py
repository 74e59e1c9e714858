"""GPU tests of the FP16-state ("Albatross") packed recurrence,
infer_tmix_wkv7_recurrent_fp16_forward_varlen, against the numpy oracle
(oracle.wkv7_fp16_state) on the kernel's exact inputs.  Cases follow
tests/tmix/wkv7/test.py:883-1100 of the reference (family correctness over
head sizes and lengths, dispatch boundaries at H = 64, the metadata-ticket
contract, the fp16-only checks); the gate is the reference's relative RMSE
<= 4e-3 on outputs and active states (test.py:958-961), plus exact elapsed
counts, untouched slots, fail-closed NaN output and split-call equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from wkv7_testlib import relative_rmse, require_gpu, to_np

pytestmark = pytest.mark.gpu

from flashrwkv2_amd.tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_recurrent_fp16_forward_varlen as wkv7_fp16,
    prepare_tmix_wkv7_recurrent_metadata,
)

import oracle  # noqa: E402

NAMES = ("r", "decay_logits", "k", "v", "a", "b")
GATE = 3.0e-3   # the reference fixture's FP16 gate (tests/fixtures/tolerances-v1.json:24-38)


def make_case(*, head_size=64, lengths=(1, 2, 4), num_heads=2, with_decay_bias=True,
              state_pool_slots=None, seed=77):
    g = torch.Generator().manual_seed(seed + head_size + len(lengths))
    total = sum(lengths)
    n = len(lengths)
    slots_n = state_pool_slots if state_pool_slots is not None else max(9, n)
    shape = (total, num_heads, head_size)
    scales = (0.12, 3.5, 0.06, 0.06, 0.06, 0.06)
    case = {nm: (torch.randn(shape, generator=g) * s).half().cuda() for nm, s in zip(NAMES, scales)}
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    case["cu_seqlens"] = torch.tensor(offsets, dtype=torch.int32, device="cuda")
    slots = (torch.tensor([5, 0, 7, 2, 4][:n], dtype=torch.int32) if n <= 5
             else torch.arange(n, dtype=torch.int32))
    case["state_indices"] = slots.cuda()
    case["state_pool"] = (torch.randn((slots_n, num_heads, head_size, head_size), generator=g)
                          * 0.03).half().cuda()
    case["elapsed_state_pool"] = (torch.arange(slots_n, dtype=torch.int32) * 11).cuda()
    case["decay_bias"] = ((torch.randn((num_heads, head_size), generator=g) * 0.2).half().cuda()
                          if with_decay_bias else None)
    return case


def tokens(case):
    return tuple(case[n] for n in NAMES)


def expect(case, scale=1.0):
    return oracle.wkv7_fp16_state(
        *(to_np(t) for t in tokens(case)), cu_seqlens=case["cu_seqlens"].cpu().numpy(),
        state_indices=case["state_indices"].cpu().numpy(),
        state_pool=case["state_pool"].cpu().numpy(),
        elapsed_state_pool=case["elapsed_state_pool"].cpu().numpy(),
        decay_bias=None if case["decay_bias"] is None else to_np(case["decay_bias"]),
        scale=scale)


def run(case, *, scale=1.0, **kw):
    state = case["state_pool"].clone()
    elapsed = case["elapsed_state_pool"].clone()
    out = wkv7_fp16(*tokens(case), state_pool=state, elapsed_state_pool=elapsed,
                    cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"],
                    scale=scale, decay_bias=case["decay_bias"], **kw)
    torch.cuda.synchronize()
    return out, state, elapsed


def check_against_oracle(case, out, state, elapsed, scale=1.0):
    y_ref, pool_ref, el_ref = expect(case, scale)
    assert out.dtype == torch.float16 and state.dtype == torch.float16
    assert torch.isfinite(out).all() and torch.isfinite(state).all()
    assert relative_rmse(to_np(out), y_ref.astype(np.float64)) <= GATE
    act = case["state_indices"].long().cpu().numpy()
    got = to_np(state)
    assert relative_rmse(got[act], pool_ref[act].astype(np.float64)) <= GATE
    untouched = np.setdiff1d(np.arange(got.shape[0]), act)
    assert np.array_equal(got[untouched], to_np(case["state_pool"])[untouched])
    assert np.array_equal(elapsed.cpu().numpy(), el_ref)


@pytest.mark.parametrize("head_size", (64, 128, 256))
@pytest.mark.parametrize("lengths", ((1,), (1, 2, 4), (8, 8), (3, 40)))
def test_fp16_state_family_correctness(head_size, lengths):
    require_gpu()
    print(f"case fp16-state D={head_size} lengths={lengths}", flush=True)
    case = make_case(head_size=head_size, lengths=lengths)
    out, state, elapsed = run(case, scale=0.75)
    check_against_oracle(case, out, state, elapsed, scale=0.75)


@pytest.mark.parametrize("lengths", ((1,), (1,) * 17, (1,) * 128, (2,) * 32, (8,), (4,) * 16))
def test_fp16_state_grid_boundaries_at_64_heads(lengths):
    require_gpu()
    print(f"case fp16-state H=64 lengths={lengths[:3]}x{len(lengths)}", flush=True)
    case = make_case(lengths=lengths, num_heads=64, state_pool_slots=max(9, len(lengths)))
    out, state, elapsed = run(case)
    check_against_oracle(case, out, state, elapsed)


def test_fp16_state_ticket_contract_and_elapsed_advance():
    require_gpu()
    case = make_case(lengths=(2, 3))
    ticket = prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=case["state_pool"].shape[0])
    out_a, st_a, el_a = run(case)
    out_b, st_b, el_b = run(case, validated_metadata=ticket)
    assert torch.equal(out_a, out_b) and torch.equal(st_a, st_b) and torch.equal(el_a, el_b)
    case["cu_seqlens"][1] += 1
    with pytest.raises(RuntimeError, match="version"):
        run(case, validated_metadata=ticket)
    case["cu_seqlens"][1] -= 1


def test_fp16_state_split_calls_equal_one_call():
    """Two calls with the elapsed count advanced in between reproduce one call
    bitwise (the phase continues through elapsed_state_pool)."""
    require_gpu()
    case = make_case(lengths=(11,))
    out, state, elapsed = run(case)
    cut = 5
    first = {k: (v[:cut] if k in NAMES else v) for k, v in case.items()}
    first["cu_seqlens"] = torch.tensor([0, cut], dtype=torch.int32, device="cuda")
    out1, st1, el1 = run(first)
    second = {k: (v[cut:] if k in NAMES else v) for k, v in case.items()}
    second["cu_seqlens"] = torch.tensor([0, 11 - cut], dtype=torch.int32, device="cuda")
    second["state_pool"], second["elapsed_state_pool"] = st1, el1
    out2, st2, el2 = run(second)
    assert torch.equal(torch.cat([out1, out2]), out)
    assert torch.equal(st2, state) and torch.equal(el2, elapsed)


def test_fp16_state_invalid_metadata_fails_closed():
    """Duplicate slots reach the device validation through the _C entry with
    implicit metadata (the public wrapper's ticket rejects them on the host):
    the output is NaN and neither the pool nor the elapsed counts change."""
    C = require_gpu()
    case = make_case(lengths=(2, 3))
    slots = torch.tensor([1, 1], dtype=torch.int32, device="cuda")
    state = case["state_pool"].clone()
    elapsed = case["elapsed_state_pool"].clone()
    out = torch.empty_like(case["v"])
    C.tmix_wkv7_recurrent_fp16_from_decay_logits(
        case["cu_seqlens"], slots, elapsed, state, *tokens(case), out, 1.0,
        case["decay_bias"], None, -1)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    assert torch.equal(state, case["state_pool"])
    assert torch.equal(elapsed, case["elapsed_state_pool"])


def test_fp16_state_rejects_non_fp16_state_and_tokens():
    require_gpu()
    case = make_case(lengths=(2,))
    with pytest.raises(TypeError, match="FP16-state state_pool"):
        wkv7_fp16(*tokens(case), state_pool=case["state_pool"].float(),
                  elapsed_state_pool=case["elapsed_state_pool"],
                  cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"])
    toks = tokens(case)
    with pytest.raises((TypeError, RuntimeError), match="float16"):
        wkv7_fp16(toks[0].bfloat16(), *toks[1:], state_pool=case["state_pool"],
                  elapsed_state_pool=case["elapsed_state_pool"],
                  cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"])
    with pytest.raises(TypeError, match="int32"):
        wkv7_fp16(*toks, state_pool=case["state_pool"],
                  elapsed_state_pool=case["elapsed_state_pool"].long(),
                  cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"])


def test_fp16_state_decode_and_serial_paths_agree():
    """max_seqlen <= 4 at D = 64 selects the state-streaming decode kernel;
    an unknown max_seqlen selects the token-serial kernel.  They reduce the
    a^T S and r^T S dot products in different orders (so an fp16 rounding can
    differ by one unit), and each meets the oracle gate."""
    require_gpu()
    from flashrwkv2_amd import _native as N

    case = make_case(lengths=(1, 2, 4, 3), num_heads=8)
    lib = N.load()
    results = []
    for max_seqlen in (4, -1):
        state = case["state_pool"].clone()
        elapsed = case["elapsed_state_pool"].clone()
        out = torch.empty_like(case["v"])
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            case["cu_seqlens"], case["state_indices"], total_tokens=out.shape[0],
            state_pool_size=state.shape[0])
        rc = lib.fr2_wkv7_recurrent_fp16_forward(
            ticket._query_start_loc_snapshot().data_ptr(),
            ticket._state_indices_snapshot().data_ptr(), ticket._status().data_ptr(),
            elapsed.data_ptr(), case["state_indices"].numel(), 8, 64, out.shape[0], max_seqlen,
            state.data_ptr(), *(t.data_ptr() for t in tokens(case)[:2]),
            case["decay_bias"].data_ptr(), *(t.data_ptr() for t in tokens(case)[2:]),
            out.data_ptr(), 1.0, torch.cuda.current_stream().cuda_stream)
        N.check(rc, "fr2_wkv7_recurrent_fp16_forward")
        torch.cuda.synchronize()
        results.append((out, state, elapsed))
    (o1, s1, e1), (o2, s2, e2) = results
    assert torch.equal(e1, e2)
    assert relative_rmse(to_np(o1), to_np(o2)) <= 1e-3
    assert relative_rmse(to_np(s1), to_np(s2)) <= 1e-3
    check_against_oracle(case, o1, s1, e1)
    check_against_oracle(case, o2, s2, e2)


@pytest.mark.parametrize("lengths", ((1,) * 9, (3, 40, 7)))
def test_fp16_state_update_then_advance_equals_the_combined_entry(lengths):
    """fr2_wkv7_recurrent_fp16_update followed by
    fr2_wkv7_recurrent_fp16_advance_elapsed (the reference's two native calls)
    leave exactly what fr2_wkv7_recurrent_fp16_forward leaves; the update
    alone leaves elapsed_state untouched."""
    require_gpu()
    from flashrwkv2_amd import _native as N
    from flashrwkv2_amd.tmix.wkv7 import prepare_tmix_wkv7_recurrent_metadata

    print(f"case fp16 update/advance split lengths={lengths}", flush=True)
    case = make_case(lengths=lengths, seed=301)
    lib = N.load()
    stream = torch.cuda.current_stream().cuda_stream
    max_seqlen = max(lengths)
    results = []
    for split in (False, True):
        state = case["state_pool"].clone()
        elapsed = case["elapsed_state_pool"].clone()
        out = torch.empty_like(case["v"])
        t = prepare_tmix_wkv7_recurrent_metadata(
            case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
            state_pool_size=state.shape[0])
        meta = (t._query_start_loc_snapshot().data_ptr(), t._state_indices_snapshot().data_ptr(),
                t._status().data_ptr(), elapsed.data_ptr())
        rest = (len(lengths), case["r"].shape[1], 64, case["r"].shape[0], max_seqlen,
                state.data_ptr(), case["r"].data_ptr(), case["decay_logits"].data_ptr(),
                case["decay_bias"].data_ptr(), *(case[n].data_ptr() for n in NAMES[2:]),
                out.data_ptr(), 0.5, stream)
        if split:
            N.check(lib.fr2_wkv7_recurrent_fp16_update(*meta, *rest), "update")
            torch.cuda.synchronize()
            assert torch.equal(elapsed, case["elapsed_state_pool"])
            N.check(lib.fr2_wkv7_recurrent_fp16_advance_elapsed(*meta, len(lengths), stream),
                    "advance")
        else:
            N.check(lib.fr2_wkv7_recurrent_fp16_forward(*meta, *rest), "forward")
        torch.cuda.synchronize()
        results.append((out, state, elapsed))
    for a, b in zip(*results):
        assert torch.equal(a, b)
    check_against_oracle(case, *results[1], scale=0.5)


def _forced_update(case, kernel, max_seqlen):
    """fr2_wkv7_recurrent_fp16_update_kernel with the kernel forced; returns
    (y, state) and leaves the case untouched."""
    from flashrwkv2_amd import _native as N

    lib = N.load()
    state = case["state_pool"].clone()
    out = torch.empty_like(case["v"])
    t = prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=state.shape[0])
    bias = case["decay_bias"]
    rc = lib.fr2_wkv7_recurrent_fp16_update_kernel(
        kernel, t._query_start_loc_snapshot().data_ptr(), t._state_indices_snapshot().data_ptr(),
        t._status().data_ptr(), case["elapsed_state_pool"].data_ptr(),
        case["state_indices"].numel(), case["r"].shape[1], case["r"].shape[2], out.shape[0],
        max_seqlen, state.data_ptr(), *(x.data_ptr() for x in tokens(case)[:2]),
        None if bias is None else bias.data_ptr(), *(x.data_ptr() for x in tokens(case)[2:]),
        out.data_ptr(), 0.75, torch.cuda.current_stream().cuda_stream)
    N.check(rc, "fr2_wkv7_recurrent_fp16_update_kernel")
    torch.cuda.synchronize()
    return out, state


@pytest.mark.parametrize("lengths,heads,bias", [
    ((1, 2, 4), 2, True),
    ((17, 33, 5, 64), 3, False),
    ((300, 129), 4, True),
    ((4096,) * 8, 32, False),          # BASELINE config 1's shape in fp16 (256 units)
], ids=["short", "ragged", "long-bias", "config1-shape"])
def test_barrier_free_fp16_kernel_matches_the_workgroup_kernel(lengths, heads, bias):
    """The barrier-free D = 64 kernel (6) updates the state with the same
    fp32 FMAs and the same fp16 rounding as the workgroup kernel (0); its two
    dot products per token run on the matrix cores (exact fp16 products, fp32
    sums in the hardware's order), so an fp16 rounding can land one unit
    apart now and then.  The two agree far inside the oracle gate, and the
    small cases meet the oracle."""
    require_gpu()
    print(f"case fp16 barrier-free vs workgroup lengths={lengths[:4]} H={heads} bias={bias}",
          flush=True)
    case = make_case(lengths=lengths, num_heads=heads, with_decay_bias=bias, seed=401)
    y0, s0 = _forced_update(case, 0, max(lengths))
    y6, s6 = _forced_update(case, 6, max(lengths))
    assert torch.isfinite(y6).all() and torch.isfinite(s6).all()
    act = case["state_indices"].long()
    assert relative_rmse(to_np(y6), to_np(y0).astype(np.float64)) <= 2e-4
    assert relative_rmse(to_np(s6[act]), to_np(s0[act]).astype(np.float64)) <= 2e-4
    untouched = np.setdiff1d(np.arange(s6.shape[0]), act.cpu().numpy())
    assert np.array_equal(to_np(s6)[untouched], to_np(case["state_pool"])[untouched])
    if sum(lengths) * heads <= 4096:
        el = case["elapsed_state_pool"].clone()
        lens = (case["cu_seqlens"][1:] - case["cu_seqlens"][:-1]).to(torch.int32)
        el.index_add_(0, act, lens)
        check_against_oracle(case, y6, s6, el, scale=0.75)


def test_barrier_free_fp16_kernel_many_units_meets_the_oracle():
    """Above 256 units the workgroup kernel splits keys 4 ways (another sum
    order); the barrier-free kernel keeps its order and meets the oracle."""
    require_gpu()
    lengths = tuple(5 + (7 * i) % 23 for i in range(100))
    print("case fp16 barrier-free 100 sequences x 4 heads", flush=True)
    case = make_case(lengths=lengths, num_heads=4, with_decay_bias=True, seed=402)
    y6, s6 = _forced_update(case, 6, max(lengths))
    el = case["elapsed_state_pool"].clone()
    lens = (case["cu_seqlens"][1:] - case["cu_seqlens"][:-1]).to(torch.int32)
    el.index_add_(0, case["state_indices"].long(), lens)
    check_against_oracle(case, y6, s6, el, scale=0.75)
