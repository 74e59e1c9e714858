"""GPU parity tests of the pretrain [B,T,C] forward, the bf16-state chunk
entry and the RL/Infctx chunk forward / replay, against the fp64 oracle.
Cases mirror tests/tmix/wkv7/{pretrain,chunk,rl_infctx}/test.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from wkv7_testlib import (
    assert_output_close,
    assert_state_close,
    relative_rmse,
    require_gpu,
    to_np,
)

pytestmark = pytest.mark.gpu

import flashrwkv2_amd  # noqa: E402
from flashrwkv2_amd.tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_chunk_bf16_forward_varlen,
    prepare_tmix_wkv7_recurrent_metadata,
    pretrain_tmix_wkv7_recurrent_bf16,
    rl_infctx_tmix_wkv7_chunk_fp32io16,
)


def _randn(shape, g, scale, dtype, device="cuda"):
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


# ----------------------------------------------------------------- pretrain
def _pretrain_inputs(shape, head_size, g, structured):
    """structured=False: every input 0.05 * randn (the reference's
    tests/tmix/wkv7/pretrain/test.py:25-41); True: O(1) inputs with the
    model's operand structure (kk unit-norm per head, a = -kk,
    b = kk * sigmoid(N(0,1)), logits ~ N(0, 1.5^2))."""
    if not structured:
        return tuple(_randn(shape, g, 0.05, torch.bfloat16) for _ in range(6))
    B, T, C = shape
    kk = torch.randn((B, T, C // head_size, head_size), generator=g)
    kk = kk / kk.norm(dim=-1, keepdim=True)
    gate = torch.sigmoid(torch.randn(kk.shape, generator=g))
    r, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    w = torch.randn(shape, generator=g) * 1.5
    vals = (r, w, k, v, (-kk).reshape(shape), (kk * gate).reshape(shape))
    return tuple(t.to(torch.bfloat16).cuda() for t in vals)


@pytest.mark.parametrize("batch,tokens,heads,head_size,structured",
                         [(1, 16, 1, 64, False), (2, 32, 2, 64, False), (2, 32, 2, 64, True),
                          (1, 64, 3, 64, True), (1, 272, 2, 64, True), (1, 16, 1, 128, False),
                          (1, 48, 2, 128, True), (1, 16, 1, 256, False), (1, 32, 1, 256, True)])
def test_pretrain_forward_matches_oracle(batch, tokens, heads, head_size, structured):
    C = require_gpu()
    g = torch.Generator().manual_seed(20260806 + batch + tokens + heads)
    shape = (batch, tokens, heads * head_size)
    vals = _pretrain_inputs(shape, head_size, g, structured)
    y = pretrain_tmix_wkv7_recurrent_bf16(*vals, head_size=head_size)
    torch.cuda.synchronize()
    assert y.shape == shape and y.dtype == torch.bfloat16
    flat = [to_np(t).reshape(batch * tokens, heads, head_size) for t in vals]
    cu = np.arange(0, batch * tokens + 1, tokens, dtype=np.int32)
    y_ref, _, sa_ref, bd_ref = oracle.wkv7_f64(*flat, cu_seqlens=cu, want_sa=True,
                                               boundary_len=16)
    assert_output_close(y.reshape(batch * tokens, heads, head_size), y_ref)
    assert torch.equal(y, pretrain_tmix_wkv7_recurrent_bf16(*vals, head_size=head_size))
    # native forward: boundary (post-chunk) and state_dot_a checkpoints
    v4 = tuple(t.view(batch, tokens, heads, head_size) for t in vals)
    out = torch.empty_like(v4[3])
    boundary = torch.empty((batch, heads, tokens // 16, head_size, head_size), device="cuda")
    sa = torch.empty((batch, tokens, heads, head_size), device="cuda")
    C.pretrain_tmix_wkv7_recurrent_forward(*v4, out, boundary, sa, head_size)
    torch.cuda.synchronize()
    assert relative_rmse(to_np(sa).reshape(sa_ref.shape), sa_ref) <= 1e-4
    assert_state_close(boundary, bd_ref)


def test_pretrain_rejects_invalid_inputs():
    require_gpu()
    g = torch.Generator().manual_seed(1)
    valid = [_randn((1, 16, 64), g, 0.05, torch.bfloat16) for _ in range(6)]
    with pytest.raises(TypeError, match="bfloat16"):
        pretrain_tmix_wkv7_recurrent_bf16(valid[0].float(), *valid[1:])
    with pytest.raises(ValueError, match="T must be divisible"):
        pretrain_tmix_wkv7_recurrent_bf16(*[t[:, :15].contiguous() for t in valid])
    with pytest.raises(ValueError, match="C must be divisible"):
        pretrain_tmix_wkv7_recurrent_bf16(*[t[:, :, :63].contiguous() for t in valid])
    with pytest.raises(ValueError, match="must match r shape"):
        pretrain_tmix_wkv7_recurrent_bf16(valid[0], valid[1][:, :, :32].contiguous(), *valid[2:])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        pretrain_tmix_wkv7_recurrent_bf16(valid[0].transpose(1, 2), *valid[1:])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        pretrain_tmix_wkv7_recurrent_bf16(*(t.cpu() for t in valid))


# ----------------------------------------------------------- bf16-state chunk
def _chunk_reference(inputs, pool_bf16, cu, slots, scale, bias=None):
    y, pool, _, _ = oracle.wkv7_f64(*(to_np(t) for t in inputs), cu_seqlens=cu.cpu().numpy(),
                                    state_indices=slots.cpu().numpy(),
                                    state_pool=to_np(pool_bf16), scale=scale,
                                    decay_bias=None if bias is None else to_np(bias))
    return y, pool


@pytest.mark.parametrize("chunk_size", [8, 16, 64])
def test_chunk_bf16_ragged_tail_and_slot_update(chunk_size):
    require_gpu()
    g = torch.Generator().manual_seed(11)
    lengths = [1, 9, 17]
    total, h, d = sum(lengths), 1, 64
    inputs = [_randn((total, h, d), g, s, torch.bfloat16)
              for s in (0.12, 3.5, 0.06, 0.06, 0.06, 0.06)]
    cu = torch.tensor([0, 1, 10, 27], device="cuda", dtype=torch.int32)
    slots = torch.tensor([2, 0, 3], device="cuda", dtype=torch.int32)
    pool = _randn((5, h, d, d), g, 0.05, torch.bfloat16)
    before = pool.clone()
    y_ref, pool_ref = _chunk_reference(inputs, pool, cu, slots, 0.5)
    out = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *inputs, state_pool=pool, cu_seqlens=cu, state_indices=slots, chunk_size=chunk_size,
        max_seqlen=17, scale=0.5)
    torch.cuda.synchronize()
    assert out.shape == inputs[3].shape and out.dtype == torch.bfloat16
    assert_output_close(out, y_ref)
    active = [2, 0, 3]
    # the pool is bf16: one rounding of the final fp32 state (2^-9 relative)
    assert_state_close(pool[active], pool_ref[active], rmse=4e-3, fro=4e-3)
    assert torch.equal(pool[[1, 4]], before[[1, 4]])


def test_chunk_bf16_long_requests_on_the_chunked_kernel():
    """max_seqlen >= 128 runs the chunked MFMA kernel with a bf16 state load
    and store (the state stays fp32 inside the call, as the reference's K2
    keeps it, infer_chunk_bf16_forward_varlen.cu:195-270); checked against the
    oracle and against the token-serial path on the same inputs."""
    require_gpu()
    g = torch.Generator().manual_seed(12)
    lengths = [130, 1, 300, 77]
    total, h, d = sum(lengths), 2, 64
    cu_list = [0]
    for n in lengths:
        cu_list.append(cu_list[-1] + n)
    kk = torch.randn((total, h, d), generator=g)
    kk = kk / kk.norm(dim=-1, keepdim=True)
    gate = torch.sigmoid(torch.randn((total, h, d), generator=g))
    inputs = [(torch.randn((total, h, d), generator=g) * s).to(torch.bfloat16).cuda()
              for s in (1.0, 1.5, 1.0, 1.0)]
    inputs = inputs[:4] + [(-kk).to(torch.bfloat16).cuda(), (kk * gate).to(torch.bfloat16).cuda()]
    cu = torch.tensor(cu_list, device="cuda", dtype=torch.int32)
    slots = torch.tensor([4, 0, 2, 5], device="cuda", dtype=torch.int32)
    pool = _randn((6, h, d, d), g, 0.1, torch.bfloat16)
    before = pool.clone()
    y_ref, pool_ref = _chunk_reference(inputs, pool, cu, slots, 1.0)
    out = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *inputs, state_pool=pool, cu_seqlens=cu, state_indices=slots, max_seqlen=300)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    active = [4, 0, 2, 5]
    assert_state_close(pool[active], pool_ref[active], rmse=4e-3, fro=4e-3)
    assert torch.equal(pool[[1, 3]], before[[1, 3]])
    # the same call on the wavefront-per-unit kernel: max_seqlen is only a
    # dispatch hint to this entry (the kernels run every sequence to its end),
    # and below 5 tokens it picks that kernel
    pool2 = before.clone()
    from flashrwkv2_amd import _native as N
    import flashrwkv2_amd
    C = flashrwkv2_amd._C
    out2 = torch.empty_like(out)
    lq, ls, status, _, keep = C._resolve_launch_metadata(cu, slots, total, 6, 300, None)
    rc = N.load().fr2_wkv7_chunk_bf16_forward(
        lq.data_ptr(), ls.data_ptr(), status.data_ptr(), 4, h, total, 16, 4,
        pool2.data_ptr(), *(t.data_ptr() for t in inputs[:2]), None,
        *(t.data_ptr() for t in inputs[2:]), out2.data_ptr(), 1.0,
        torch.cuda.current_stream().cuda_stream)
    N.check(rc, "fr2_wkv7_chunk_bf16_forward")
    torch.cuda.synchronize()
    del keep
    assert_output_close(out2, y_ref)
    assert_state_close(pool2[active], pool_ref[active], rmse=4e-3, fro=4e-3)


@pytest.mark.parametrize("pieces", [2, 3, (3, 320), (2, 96)])
def test_chunk_bf16_sequence_split(monkeypatch, pieces):
    """The bf16-state chunk entry with the sequence split forced (summary
    pass, combine from the widened bf16 slot state, pieces; each sequence's
    last piece rounds the slot once): the oracle's values and the unsplit
    call's, untouched slots unchanged."""
    require_gpu()
    import flashrwkv2_amd

    g = torch.Generator().manual_seed(31)
    lengths = [700, 5, 260, 64]
    total, h, d = sum(lengths), 3, 64
    cu_list = [0]
    for n in lengths:
        cu_list.append(cu_list[-1] + n)
    kk = torch.randn((total, h, d), generator=g)
    kk = kk / kk.norm(dim=-1, keepdim=True)
    gate = torch.sigmoid(torch.randn((total, h, d), generator=g))
    inputs = [(torch.randn((total, h, d), generator=g) * s).to(torch.bfloat16).cuda()
              for s in (1.0, 1.5, 1.0, 1.0)]
    inputs = inputs[:4] + [(-kk).to(torch.bfloat16).cuda(), (kk * gate).to(torch.bfloat16).cuda()]
    cu = torch.tensor(cu_list, device="cuda", dtype=torch.int32)
    slots = torch.tensor([4, 0, 2, 5], device="cuda", dtype=torch.int32)
    pool = _randn((6, h, d, d), g, 0.1, torch.bfloat16)
    before = pool.clone()
    y_ref, pool_ref = _chunk_reference(inputs, pool, cu, slots, 0.5)
    monkeypatch.setattr(flashrwkv2_amd._C, "_chunk_split_pieces", pieces)
    out = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *inputs, state_pool=pool, cu_seqlens=cu, state_indices=slots, max_seqlen=700,
        scale=0.5)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    active = [4, 0, 2, 5]
    assert_state_close(pool[active], pool_ref[active], rmse=4e-3, fro=4e-3)
    assert torch.equal(pool[[1, 3]], before[[1, 3]])
    monkeypatch.setattr(flashrwkv2_amd._C, "_chunk_split_pieces", None)
    pool2 = before.clone()
    out2 = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *inputs, state_pool=pool2, cu_seqlens=cu, state_indices=slots, max_seqlen=700,
        scale=0.5)
    torch.cuda.synchronize()
    dy = out.float() - out2.float()
    assert (dy.square().mean().sqrt() / out2.float().square().mean().sqrt()).item() <= 2e-3
    # both round the same fp32 state once; a split can move a value across a
    # bf16 rounding boundary, so the pools agree to one bf16 ulp
    assert ((pool.float() - pool2.float()).abs() <= pool2.float().abs() * 2 ** -7 + 1e-30).all()


def test_chunk_bf16_rejects_non_bf16_and_duplicate_slots_without_state_write():
    require_gpu()
    tensors = [torch.zeros((2, 1, 64), device="cuda", dtype=torch.bfloat16) for _ in range(6)]
    state = torch.randn((2, 1, 64, 64), device="cuda").to(torch.bfloat16)
    before = state.clone()
    with pytest.raises(ValueError, match="bfloat16"):
        infer_tmix_wkv7_chunk_bf16_forward_varlen(
            tensors[0].float(), *tensors[1:], state_pool=state,
            cu_seqlens=torch.tensor([0, 2], device="cuda", dtype=torch.int32),
            state_indices=torch.tensor([0], device="cuda", dtype=torch.int32))
    with pytest.raises(RuntimeError, match="unique"):
        infer_tmix_wkv7_chunk_bf16_forward_varlen(
            *tensors, state_pool=state,
            cu_seqlens=torch.tensor([0, 1, 2], device="cuda", dtype=torch.int32),
            state_indices=torch.tensor([0, 0], device="cuda", dtype=torch.int32), max_seqlen=1)
    torch.cuda.synchronize()
    assert torch.equal(state, before)


@pytest.mark.cuda_graph
def test_chunk_bf16_graph_consumes_live_metadata_ticket():
    require_gpu()
    g = torch.Generator().manual_seed(23)
    tok_cap, seq_cap, nslots = 3, 2, 4
    inputs = tuple(_randn((tok_cap, 1, 64), g, 0.02, torch.bfloat16) for _ in range(6))
    initial = _randn((nslots, 1, 64, 64), g, 0.002, torch.bfloat16)
    state = initial.clone()
    cu = torch.tensor([0, 1, 3], device="cuda", dtype=torch.int32)
    slots = torch.tensor([3, 1], device="cuda", dtype=torch.int32)
    n_tok = torch.tensor([3], device="cuda", dtype=torch.int32)
    n_seq = torch.tensor([2], device="cuda", dtype=torch.int32)
    expected_state = initial.clone()
    expected = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *inputs, state_pool=expected_state, cu_seqlens=cu, state_indices=slots, chunk_size=2,
        max_seqlen=2)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            cu, slots, state_pool_size=nslots, token_capacity=tok_cap,
            sequence_capacity=seq_cap, max_seqlen_capacity=2, num_active_tokens=n_tok,
            num_active_sequences=n_seq)
        out = infer_tmix_wkv7_chunk_bf16_forward_varlen(
            *inputs, state_pool=state, cu_seqlens=cu, state_indices=slots, chunk_size=2,
            validated_metadata=ticket)
    for _ in range(2):
        state.copy_(initial)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
        assert torch.equal(state, expected_state)
    state.copy_(initial)
    cu.copy_(torch.tensor([0, 2, -1], device="cuda", dtype=torch.int32))
    slots.copy_(torch.tensor([2, 99], device="cuda", dtype=torch.int32))
    n_tok.fill_(2)
    n_seq.fill_(1)
    graph.replay()
    torch.cuda.synchronize()
    assert not torch.equal(state[2], initial[2])
    assert torch.equal(state[[0, 1, 3]], initial[[0, 1, 3]])
    state.copy_(initial)
    cu.copy_(torch.tensor([0, 1, 2], device="cuda", dtype=torch.int32))
    slots.copy_(torch.tensor([1, 1], device="cuda", dtype=torch.int32))
    n_tok.fill_(2)
    n_seq.fill_(2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(state, initial)


# ------------------------------------------------------------------ RL/Infctx
@pytest.mark.parametrize("d", [64, 128, 256])
def test_rl_infctx_ragged_materialized_and_recompute(d):
    require_gpu()
    g = torch.Generator().manual_seed(37)
    total, h = 7, 1
    inputs = [_randn((total, h, d), g, 0.3, torch.float16) for _ in range(6)]
    pool = _randn((4, h, d, d), g, 0.05, torch.float32)
    original = pool.clone()
    cu = torch.tensor([0, 2, 7], device="cuda", dtype=torch.int32)
    slots = torch.tensor([3, 1], device="cuda", dtype=torch.int32)
    bias = _randn((h, d), g, 0.3, torch.float16)
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(*(to_np(t) for t in inputs),
                                            cu_seqlens=cu.cpu().numpy(),
                                            state_indices=slots.cpu().numpy(),
                                            state_pool=to_np(pool), decay_bias=to_np(bias))
    outs = []
    for strategy in ("materialized", "recompute"):
        out, new_pool = rl_infctx_tmix_wkv7_chunk_fp32io16(
            *inputs, state_pool=pool, cu_seqlens=cu, state_indices=slots, chunk_size=16,
            strategy=strategy, decay_bias=bias)
        torch.cuda.synchronize()
        assert out.dtype == torch.float16 and out.shape == inputs[3].shape
        assert_output_close(out, y_ref)
        assert_state_close(new_pool[[3, 1]], pool_ref[[3, 1]])
        assert torch.equal(new_pool[[0, 2]], pool[[0, 2]])
        outs.append((out, new_pool))
    assert torch.equal(pool, original)
    assert torch.equal(outs[0][0], outs[1][0])


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rl_infctx_chunk_sizes_and_tail(d):
    require_gpu()
    g = torch.Generator().manual_seed(43)
    total = 65
    inputs = [_randn((total, 1, d), g, 0.3, torch.bfloat16) for _ in range(6)]
    pool = _randn((3, 1, d, d), g, 0.05, torch.float32)
    cu = torch.tensor([0, total], device="cuda", dtype=torch.int32)
    slots = torch.tensor([2], device="cuda", dtype=torch.int32)
    bias = _randn((1, d), g, 0.3, torch.bfloat16)
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(*(to_np(t) for t in inputs),
                                            cu_seqlens=cu.cpu().numpy(),
                                            state_indices=slots.cpu().numpy(),
                                            state_pool=to_np(pool), decay_bias=to_np(bias),
                                            scale=0.75)
    for chunk_size in (16, 32, 64):
        for strategy in ("materialized", "recompute"):
            out, new_pool = rl_infctx_tmix_wkv7_chunk_fp32io16(
                *inputs, state_pool=pool, cu_seqlens=cu, state_indices=slots,
                chunk_size=chunk_size, strategy=strategy, scale=0.75, decay_bias=bias)
            torch.cuda.synchronize()
            assert out.dtype == torch.bfloat16
            assert_output_close(out, y_ref)
            assert_state_close(new_pool[[2]], pool_ref[[2]])


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rl_infctx_backward_replay_matches_recurrence(d):
    C = require_gpu()
    g = torch.Generator().manual_seed(41 + d)
    total, heads = 40, 2
    # keep |y| well inside the fp16 range at every head size
    inputs = [_randn((total, heads, d), g, 0.3 * (64 / d) ** 0.5, torch.float16)
              for _ in range(6)]
    init = _randn((1, heads, d, d), g, 0.05, torch.float32)
    bias = _randn((heads, d), g, 0.3, torch.float16)
    cu = np.array([0, total], np.int32)
    y_ref, _, sa_ref, _ = oracle.wkv7_f64(*(to_np(t) for t in inputs), cu_seqlens=cu,
                                          state_indices=np.array([0], np.int32),
                                          state_pool=to_np(init), decay_bias=to_np(bias),
                                          scale=0.75, want_sa=True)
    assert np.abs(y_ref).max() < 1e4
    # chunks [0,16), [16,32), [32,40) with their start-of-chunk states
    starts, ends = [0, 16, 32], [16, 32, 40]
    bounds = [to_np(init)[0]]
    for s in starts[1:]:
        _, p, _, _ = oracle.wkv7_f64(*(to_np(t)[:s] for t in inputs),
                                     cu_seqlens=np.array([0, s], np.int32),
                                     state_indices=np.array([0], np.int32),
                                     state_pool=to_np(init), decay_bias=to_np(bias))
        bounds.append(p[0])
    boundary = torch.tensor(np.stack(bounds), dtype=torch.float32, device="cuda")
    out = torch.empty_like(inputs[3])
    sa = torch.empty(inputs[0].shape, device="cuda", dtype=torch.float32)
    C.rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay(
        torch.tensor(starts, device="cuda", dtype=torch.int32),
        torch.tensor(ends, device="cuda", dtype=torch.int32), boundary, *inputs, out, sa,
        0.75, bias)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    assert relative_rmse(to_np(sa), sa_ref) <= 1e-4


def test_rl_infctx_rejects_duplicates_and_bad_boundaries():
    require_gpu()
    values = [torch.zeros((2, 1, 64), device="cuda", dtype=torch.float16) for _ in range(6)]
    with pytest.raises(ValueError, match="duplicates"):
        rl_infctx_tmix_wkv7_chunk_fp32io16(
            *values, state_pool=torch.zeros(2, 1, 64, 64, device="cuda"),
            cu_seqlens=torch.tensor([0, 1, 2], device="cuda", dtype=torch.int32),
            state_indices=torch.tensor([0, 0], device="cuda", dtype=torch.int32))
    state = torch.zeros(1, 1, 64, 64, device="cuda")
    slots = torch.zeros(1, device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError, match="start at zero"):
        rl_infctx_tmix_wkv7_chunk_fp32io16(
            *values, state_pool=state,
            cu_seqlens=torch.tensor([1, 2], device="cuda", dtype=torch.int32),
            state_indices=slots)
    with pytest.raises(ValueError, match="end at total_tokens"):
        rl_infctx_tmix_wkv7_chunk_fp32io16(
            *values, state_pool=state,
            cu_seqlens=torch.tensor([0, 1], device="cuda", dtype=torch.int32),
            state_indices=slots)


def test_backend_is_the_in_tree_hip_library():
    require_gpu()
    from flashrwkv2_amd import _native

    assert flashrwkv2_amd._C is not None
    lib = _native.load()
    assert lib.fr2_abi_version() == 200
    with open("/proc/self/maps") as fh:
        maps = fh.read()
    assert str(_native.LIB_PATH) in maps or _native.LIB_PATH.name in maps


def test_rl_infctx_replay_many_chunks_matches_recurrence():
    """2 048 ragged chunks x 8 heads (16 384 (chunk, head) units; at D = 64
    the replay runs on the chunked kernel with one wavefront per unit, which
    also writes sa), each from its own start-of-chunk state, against the fp64
    recurrence with per-token sa."""
    C = require_gpu()
    print("case rl_infctx replay 2048 chunks x 8 heads", flush=True)
    g = torch.Generator().manual_seed(77)
    heads, n = 8, 2048
    lengths = torch.randint(1, 33, (n,), generator=g).numpy()
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    total = int(cu[-1])
    inputs = [_randn((total, heads, 64), g, s, torch.bfloat16)
              for s in (0.3, 2.0, 0.3, 0.3, 0.1, 0.1)]
    boundary = _randn((n, heads, 64, 64), g, 0.05, torch.float32)
    y_ref, _, sa_ref, _ = oracle.wkv7_f64(*(to_np(t) for t in inputs), cu_seqlens=cu,
                                          state_indices=np.arange(n, dtype=np.int32),
                                          state_pool=to_np(boundary), scale=0.5, want_sa=True)
    out = torch.empty_like(inputs[3])
    sa = torch.empty(inputs[0].shape, device="cuda", dtype=torch.float32)
    C.rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay(
        torch.tensor(cu[:-1], device="cuda", dtype=torch.int32),
        torch.tensor(cu[1:], device="cuda", dtype=torch.int32), boundary.cuda(), *inputs, out,
        sa, 0.5, None)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    assert relative_rmse(to_np(sa), sa_ref) <= 1e-4
