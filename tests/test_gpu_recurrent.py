"""GPU parity and contract tests of the packed fp32-state WKV7 recurrence.

Every numerical check compares the HIP kernels (through the C ABI) against the
fp64 CPU oracle on exactly the kernel's inputs; tolerances are the
reference's relative-RMSE gate (tests/fixtures/tolerances-v1.json:9-12) plus a
per-element bound |dy| <= 2e-2 * max(1, |y|) on outputs and a per-(slot, head)
Frobenius bound ||dS||/||S|| <= 1e-3 on states.  Cases and behavioural
checks mirror tests/tmix/wkv7/test.py of the reference.
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

from flashrwkv2_amd.tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
    prepare_tmix_wkv7_recurrent_metadata,
)

SERIAL, DECODE, CHUNKED, CHUNKED_WAVE = 0, 1, 2, 4


def _run(case, *, state_pool=None, **kw):
    pool = case["state_pool"] if state_pool is None else state_pool
    return wkv7(*tokens(case), state_pool=pool, cu_seqlens=case["cu_seqlens"],
                state_indices=case["state_indices"], decay_bias=case["decay_bias"], **kw)


def _run_kernel(C, kernel, case, pool, scale=1.0):
    out = torch.empty_like(case["v"])
    ticket = prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], total_tokens=case["r"].shape[0],
        state_pool_size=pool.shape[0])
    C.tmix_wkv7_recurrent_fp32_kernel_forced(
        kernel, case["cu_seqlens"], case["state_indices"], pool, *tokens(case), out, scale,
        case["decay_bias"], ticket)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_size", [64, 128, 256])
@pytest.mark.parametrize("with_bias", [False, True])
def test_packed_fp32_state_precision_and_state_safety(dtype, head_size, with_bias):
    require_gpu()
    print(f"case dtype={dtype} D={head_size} bias={with_bias}", flush=True)
    case = make_case(dtype=dtype, head_size=head_size, with_decay_bias=with_bias)
    y_ref, pool_ref = oracle_expect(case)
    before = case["state_pool"].clone()
    out = _run(case)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == case["v"].shape
    active = case["state_indices"].long()
    assert_output_close(out, y_ref)
    assert_state_close(case["state_pool"][active], pool_ref[active.cpu().numpy()])
    untouched = [i for i in range(before.shape[0]) if i not in set(active.tolist())]
    assert torch.equal(case["state_pool"][untouched], before[untouched])
    assert not torch.equal(case["state_pool"][active], before[active])
    # determinism: a second run from the same state is bitwise identical
    second = before.clone()
    out2 = _run(case, state_pool=second)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert torch.equal(case["state_pool"], second)


@pytest.mark.parametrize("kernel", [SERIAL, DECODE, CHUNKED, CHUNKED_WAVE])
@pytest.mark.parametrize("lengths", [(1,), (1, 2, 4), (1, 15, 16, 17, 65), (3,) * 12,
                                     (200, 31, 48)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_each_kernel_family_matches_oracle(kernel, lengths, dtype):
    C = require_gpu()
    print(f"case kernel={kernel} lengths={lengths} dtype={dtype}", flush=True)
    case = make_case(dtype=dtype, head_size=64, lengths=lengths, with_decay_bias=True,
                     num_heads=3)
    y_ref, pool_ref = oracle_expect(case, scale=0.75)
    pool = case["state_pool"].clone()
    out = _run_kernel(C, kernel, case, pool, scale=0.75)
    active = case["state_indices"].long()
    assert_output_close(out, y_ref)
    assert_state_close(pool[active], pool_ref[active.cpu().numpy()])


@pytest.mark.parametrize("ring", [False, True])
@pytest.mark.parametrize("kw", [
    dict(lengths=(1, 15, 16, 17, 65), num_heads=2),
    dict(lengths=(40, 1, 63, 130, 17), num_heads=3, with_decay_bias=True),
    dict(lengths=(5,), num_heads=1),
    dict(lengths=(300, 64, 96, 41), num_heads=4, with_decay_bias=True),
    dict(lengths=(1000, 777), num_heads=2, dtype=torch.float16),
    dict(lengths=(2048,), num_heads=2, scales=(0.5, 2.0, 0.5, 0.5, 0.2, 0.2)),
])
def test_both_workgroup_chunk_variants_match_oracle(ring, kw):
    """The workgroup chunked kernel has two key-side organisations (a ring of
    whole chunks per key wave, the default; key halves per wave pair): each
    matches the oracle over partial chunks, ragged batches, a decay bias,
    fp16 tokens and large-magnitude inputs, and leaves unused slots alone."""
    C = require_gpu()
    print(f"case ring={ring} {kw}", flush=True)
    case = make_case(seed=11, **kw)
    y_ref, pool_ref = oracle_expect(case, scale=0.8)
    pool = case["state_pool"].clone()
    C._set_chunk_ring(ring)
    try:
        out = _run_kernel(C, CHUNKED, case, pool, scale=0.8)
    finally:
        C._set_chunk_ring(True)
    active = case["state_indices"].long()
    assert_output_close(out, y_ref)
    assert_state_close(pool[active], pool_ref[active.cpu().numpy()])
    untouched = np.setdiff1d(np.arange(pool.shape[0]), active.cpu().numpy())
    assert torch.equal(pool[untouched], case["state_pool"][untouched])


def test_serial_and_decode_agree_closely():
    C = require_gpu()
    case = make_case(dtype=torch.bfloat16, lengths=(1, 2, 3, 4), num_heads=4)
    p0 = case["state_pool"].clone()
    p1 = case["state_pool"].clone()
    y0 = _run_kernel(C, SERIAL, case, p0)
    y1 = _run_kernel(C, DECODE, case, p1)
    assert (y0.float() - y1.float()).abs().max().item() <= 2e-2 * max(1.0, y0.float().abs().max().item())
    assert torch.allclose(p0, p1, rtol=1e-5, atol=1e-6)


def test_public_rejects_structural_arguments_without_launching():
    require_gpu()
    case = make_case(dtype=torch.float16, head_size=64)
    args = tokens(case)
    pool = case["state_pool"]
    kw = dict(state_pool=pool, cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"])
    bad_shape = torch.zeros((args[0].shape[0], args[0].shape[1], 63), device="cuda",
                            dtype=args[0].dtype)
    for bad_r, err, msg in [(args[0].transpose(0, 1), ValueError, "contiguous"),
                            (bad_shape, RuntimeError, "shape"),
                            (args[0].float(), RuntimeError, "float16 or bfloat16")]:
        with pytest.raises(err, match=msg):
            wkv7(bad_r, *args[1:], **kw)
    with pytest.raises(TypeError, match="r must be a torch.Tensor"):
        wkv7(object(), *args[1:], **kw)
    with pytest.raises(ValueError, match=r"packed shape \[total_tokens,H,D\]"):
        wkv7(args[0].reshape(-1, 64), *args[1:], **kw)
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        wkv7(args[0], args[1].to(torch.bfloat16), *args[2:], **kw)
    with pytest.raises(TypeError, match="float32"):
        wkv7(*args, state_pool=pool.half(), cu_seqlens=case["cu_seqlens"],
             state_indices=case["state_indices"])
    with pytest.raises(RuntimeError, match="square"):
        wkv7(*args, state_pool=pool[:, :, :, :-1].contiguous(),
             cu_seqlens=case["cu_seqlens"], state_indices=case["state_indices"])
    with pytest.raises(RuntimeError, match="square"):
        wkv7(*args, state_pool=pool.reshape(-1), cu_seqlens=case["cu_seqlens"],
             state_indices=case["state_indices"])
    small = make_case(dtype=torch.float16, head_size=32, lengths=(4,))
    with pytest.raises(RuntimeError, match="64, 128, or 256"):
        wkv7(*tokens(small), state_pool=small["state_pool"], cu_seqlens=small["cu_seqlens"],
             state_indices=small["state_indices"])


@pytest.mark.parametrize("kind", ["wrong_rank", "wrong_length", "wrong_dtype", "wrong_start",
                                  "wrong_end", "non_increasing", "empty_sequence",
                                  "wrong_slot_length", "duplicate_slot", "negative_slot",
                                  "out_of_range_slot"])
def test_invalid_metadata_is_rejected_and_state_preserved(kind):
    require_gpu()
    case = make_case(dtype=torch.bfloat16)
    cu, slots, pool = case["cu_seqlens"], case["state_indices"], case["state_pool"]
    bad_cu, bad_slots = cu, slots
    if kind == "wrong_rank":
        bad_cu = cu.reshape(1, -1)
    elif kind == "wrong_length":
        bad_cu = cu[:-1]
    elif kind == "wrong_dtype":
        bad_cu = cu.to(torch.int64)
    elif kind == "wrong_start":
        bad_cu = cu + 1
    elif kind == "wrong_end":
        bad_cu = cu.clone()
        bad_cu[-1] -= 1
    elif kind == "non_increasing":
        bad_cu = cu.clone()
        bad_cu[2] = bad_cu[1] - 1
    elif kind == "empty_sequence":
        bad_cu = cu.clone()
        bad_cu[2] = bad_cu[1]
    elif kind == "wrong_slot_length":
        bad_slots = slots[:-1]
    elif kind == "duplicate_slot":
        bad_slots = slots.clone()
        bad_slots[1] = bad_slots[0]
    elif kind == "negative_slot":
        bad_slots = slots.clone()
        bad_slots[0] = -1
    else:
        bad_slots = slots.clone()
        bad_slots[0] = pool.shape[0]
    before = pool.clone()
    with pytest.raises((TypeError, ValueError, RuntimeError)):
        wkv7(*tokens(case), state_pool=pool, cu_seqlens=bad_cu, state_indices=bad_slots)
    torch.cuda.synchronize()
    assert torch.equal(pool, before)


def test_public_rejects_devices_bias_scale_and_index_contracts():
    require_gpu()
    case = make_case(dtype=torch.float16)
    args = tokens(case)
    pool, cu, slots = case["state_pool"], case["cu_seqlens"], case["state_indices"]
    kw = dict(state_pool=pool, cu_seqlens=cu, state_indices=slots)
    with pytest.raises((ValueError, RuntimeError), match="CUDA"):
        wkv7(*(t.cpu() for t in args), state_pool=pool.cpu(), cu_seqlens=cu.cpu(),
             state_indices=slots.cpu())
    with pytest.raises((ValueError, RuntimeError), match="decay_bias"):
        wkv7(*args, decay_bias=torch.zeros(2, 63, device="cuda", dtype=args[0].dtype), **kw)
    with pytest.raises((TypeError, RuntimeError), match="decay_bias"):
        wkv7(*args, decay_bias=torch.zeros(2, 64, device="cuda", dtype=torch.float32), **kw)
    with pytest.raises((ValueError, RuntimeError), match="contiguous"):
        wkv7(*args, decay_bias=torch.zeros(64, 2, device="cuda", dtype=args[0].dtype).t(), **kw)
    with pytest.raises(TypeError, match="cu_seqlens must be a torch.Tensor"):
        wkv7(*args, state_pool=pool, cu_seqlens=[0, args[0].shape[0]], state_indices=slots)
    with pytest.raises(TypeError, match="state_indices must be a torch.Tensor"):
        wkv7(*args, state_pool=pool, cu_seqlens=cu, state_indices=[0] * slots.numel())
    for bad in (float("nan"), float("inf")):
        with pytest.raises(RuntimeError, match="finite"):
            wkv7(*args, scale=bad, **kw)
    with pytest.raises(TypeError, match="state_pool"):
        wkv7(*args, cu_seqlens=cu, state_indices=slots)


def test_ticket_rejects_identity_version_and_stream_mismatches():
    require_gpu()
    case = make_case(dtype=torch.bfloat16, lengths=(4, 5))
    args = tokens(case)
    cu, slots, pool = case["cu_seqlens"], case["state_indices"], case["state_pool"]
    ticket = prepare_tmix_wkv7_recurrent_metadata(cu, slots, total_tokens=args[0].shape[0],
                                                  state_pool_size=pool.shape[0])
    with pytest.raises(RuntimeError, match="identity"):
        wkv7(*args, state_pool=pool.clone(), cu_seqlens=cu.clone(), state_indices=slots,
             validated_metadata=ticket)
    short = tuple(t[:-1].contiguous() for t in args)
    with pytest.raises(RuntimeError, match="total_tokens"):
        wkv7(*short, state_pool=pool.clone(), cu_seqlens=cu, state_indices=slots,
             validated_metadata=ticket)
    with pytest.raises(RuntimeError, match="state_pool_size"):
        wkv7(*args, state_pool=torch.cat((pool, torch.zeros_like(pool[:1]))), cu_seqlens=cu,
             state_indices=slots, validated_metadata=ticket)
    cu[1] += 1
    with pytest.raises(RuntimeError, match="version"):
        wkv7(*args, state_pool=pool.clone(), cu_seqlens=cu, state_indices=slots,
             validated_metadata=ticket)
    cu[1] -= 1
    ticket2 = prepare_tmix_wkv7_recurrent_metadata(cu, slots, total_tokens=args[0].shape[0],
                                                   state_pool_size=pool.shape[0])
    other = torch.cuda.Stream()
    with torch.cuda.stream(other), pytest.raises(RuntimeError, match="stream"):
        wkv7(*args, state_pool=pool.clone(), cu_seqlens=cu, state_indices=slots,
             validated_metadata=ticket2)
    other.synchronize()
    # the ticket's snapshot is what the kernels read
    pool_a = pool.clone()
    out_a = wkv7(*args, state_pool=pool_a, cu_seqlens=cu, state_indices=slots,
                 validated_metadata=ticket2)
    pool_b = pool.clone()
    out_b = wkv7(*args, state_pool=pool_b, cu_seqlens=cu, state_indices=slots)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.equal(pool_a, pool_b)


def test_low_level_invalid_metadata_fails_closed_without_state_write():
    C = require_gpu()
    case = make_case(dtype=torch.float16, lengths=(4,))
    pool = case["state_pool"]
    bad_cu = torch.tensor([1, 4], device="cuda", dtype=torch.int32)
    slots = torch.tensor([0], device="cuda", dtype=torch.int32)
    out = torch.zeros_like(case["v"])
    before = pool.clone()
    C.tmix_wkv7_recurrent_fp32_from_decay_logits(bad_cu, slots, pool, *tokens(case), out, 1.0,
                                                 None, None)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    assert torch.equal(pool, before)


@pytest.mark.cuda_graph
def test_zero_active_warmup_then_graph_replay_with_live_metadata():
    """Mirrors test_fp32_wkv_zero_active_precapture_warmup_then_graph_replay
    (tests/tmix/wkv7/test.py:239-373)."""
    require_gpu()
    g = torch.Generator().manual_seed(20260809)
    dev = torch.device("cuda")
    tok_cap, seq_cap, slots_n, H, D = 4, 4, 2, 1, 64
    packed = tuple((torch.randn((tok_cap, H, D), generator=g) * s).half().to(dev)
                   for s in (0.1, 2.0, 0.05, 0.05, 0.05, 0.05))
    initial = (torch.randn((slots_n, H, D, D), generator=g) * 0.02).to(dev)
    state = initial.clone()
    cu = torch.tensor([0, -1, -1, -1, -1], device=dev, dtype=torch.int32)
    idx = torch.full((seq_cap,), 99, device=dev, dtype=torch.int32)
    n_tok = torch.zeros(1, device=dev, dtype=torch.int32)
    n_seq = torch.zeros(1, device=dev, dtype=torch.int32)
    addrs = (cu.data_ptr(), idx.data_ptr())
    live = dict(state_pool_size=slots_n, token_capacity=tok_cap, sequence_capacity=seq_cap,
                max_seqlen_capacity=3, num_active_tokens=n_tok, num_active_sequences=n_seq)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        warm = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
        wkv7(*packed, state_pool=state, cu_seqlens=cu, state_indices=idx,
             validated_metadata=warm)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert warm._is_graph()
    assert torch.equal(state, initial)
    cu.copy_(torch.tensor([0, 1, 4, -1, -1], device=dev, dtype=torch.int32))
    idx.copy_(torch.tensor([1, 0, 99, 99], device=dev, dtype=torch.int32))
    n_tok.fill_(4)
    n_seq.fill_(2)
    expected_state = initial.clone()
    t_exp = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
    expected = wkv7(*packed, state_pool=expected_state, cu_seqlens=cu, state_indices=idx,
                    validated_metadata=t_exp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ticket = prepare_tmix_wkv7_recurrent_metadata(cu, idx, **live)
        graph_out = wkv7(*packed, state_pool=state, cu_seqlens=cu, state_indices=idx,
                         validated_metadata=ticket)
    for _ in range(3):
        state.copy_(initial)
        graph.replay()
        torch.cuda.synchronize()
        assert addrs == (cu.data_ptr(), idx.data_ptr())
        assert torch.equal(graph_out, expected)
        assert torch.equal(state, expected_state)
    state.copy_(initial)
    cu.copy_(torch.tensor([0, 2, -1, -1, -1], device=dev, dtype=torch.int32))
    idx.copy_(torch.tensor([0, 99, 99, 99], device=dev, dtype=torch.int32))
    n_tok.fill_(2)
    n_seq.fill_(1)
    graph.replay()
    torch.cuda.synchronize()
    assert not torch.equal(state[0], initial[0])
    assert torch.equal(state[1], initial[1])
    # duplicate slots: device validation fails closed, state untouched
    state.copy_(initial)
    cu.copy_(torch.tensor([0, 1, 2, -1, -1], device=dev, dtype=torch.int32))
    idx.copy_(torch.tensor([1, 1, 99, 99], device=dev, dtype=torch.int32))
    n_tok.fill_(2)
    n_seq.fill_(2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(state, initial)


# --------------------------------------------------------------------------
# BASELINE configurations (synthetic inputs of flashrwkv2_amd.workloads)
# --------------------------------------------------------------------------
def _oracle_on_workload(w, scale=1.0):
    import oracle

    y, pool, _, _ = oracle.wkv7_f64(*(to_np(t) for t in w.tokens),
                                    cu_seqlens=w.cu_seqlens.cpu().numpy(),
                                    state_indices=w.state_indices.cpu().numpy(),
                                    state_pool=to_np(w.state_pool), scale=scale)
    return y, pool


@pytest.mark.parametrize("cfg,overrides", [
    (0, {}),
    (1, dict(batch=2, tokens=256, heads=4)),
    (2, {}),
    (3, dict(sequences=8, heads=4, max_len=300)),
    (4, dict(tokens=2048, heads=2)),
])
def test_baseline_configs_match_fp64_oracle(cfg, overrides):
    require_gpu()
    from flashrwkv2_amd import workloads

    print(f"case config={cfg} {overrides}", flush=True)
    w = workloads.config(cfg, "cuda", **overrides)
    y_ref, pool_ref = _oracle_on_workload(w)
    pool = w.state_pool.clone()
    out = wkv7(*w.tokens, state_pool=pool, cu_seqlens=w.cu_seqlens,
               state_indices=w.state_indices)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    assert_state_close(pool, pool_ref)


@pytest.mark.parametrize("cfg,overrides", [
    (1, dict(batch=2, tokens=1024, heads=2)),
    (4, dict(tokens=8192, heads=1)),
    (4, dict(heads=8)),
])
def test_chunked_kernel_long_sequences_match_fp64_oracle(cfg, overrides):
    """Chunked MFMA form over many chunks (fp32 carry drift vs fp64); the
    last case is BASELINE config 4 at its full length (65 536 tokens, 4 096
    chunks, long-memory decays) on eight of its heads."""
    C = require_gpu()
    from flashrwkv2_amd import workloads

    print(f"case chunked config={cfg} {overrides}", flush=True)
    w = workloads.config(cfg, "cuda", **overrides)
    y_ref, pool_ref = _oracle_on_workload(w)
    case = dict(zip(("r", "decay_logits", "k", "v", "a", "b"), w.tokens),
                cu_seqlens=w.cu_seqlens, state_indices=w.state_indices, decay_bias=None)
    pool = w.state_pool.clone()
    out = _run_kernel(C, CHUNKED, case, pool)
    assert_output_close(out, y_ref)
    assert_state_close(pool, pool_ref)
    # the public entry on the same inputs: with few (sequence, head) units it
    # cuts the sequence into pieces (summary, combine, pieces)
    pool2 = w.state_pool.clone()
    out2 = wkv7(*w.tokens, state_pool=pool2, cu_seqlens=w.cu_seqlens,
                state_indices=w.state_indices)
    torch.cuda.synchronize()
    assert_output_close(out2, y_ref)
    assert_state_close(pool2, pool_ref)


def test_chunked_and_serial_agree_at_full_prefill_size():
    """BASELINE config 1 at full size (B8 T4096 H32): the chunked MFMA kernel
    and the token-serial kernel (pinned to the oracle above) agree to
    fp32-level accuracy on outputs and final states."""
    C = require_gpu()
    from flashrwkv2_amd import workloads

    w = workloads.config(1, "cuda")
    case = dict(zip(("r", "decay_logits", "k", "v", "a", "b"), w.tokens),
                cu_seqlens=w.cu_seqlens, state_indices=w.state_indices, decay_bias=None)
    p_serial = w.state_pool.clone()
    p_chunk = w.state_pool.clone()
    y_serial = _run_kernel(C, SERIAL, case, p_serial)
    y_chunk = _run_kernel(C, CHUNKED, case, p_chunk)
    dy = (y_chunk.float() - y_serial.float())
    rel = (dy.square().mean().sqrt() / y_serial.float().square().mean().sqrt()).item()
    assert rel <= 2e-3, rel  # two independent bf16 roundings of the same output
    ds = (p_chunk - p_serial).flatten(0, 1).norm(dim=(1, 2))
    base = p_serial.flatten(0, 1).norm(dim=(1, 2))
    assert (ds / base).max().item() <= 1e-4
