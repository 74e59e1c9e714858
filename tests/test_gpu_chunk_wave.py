"""GPU parity of the chunked kernel with one wavefront per (sequence, head)
unit (csrc/chunkw.hip, kernel family 4), the public policy's kernel for
launches with many units.

Every case runs the kernel through the C ABI (forced family, and the public
entry where its policy picks this kernel) and checks it against the fp64 CPU
oracle on exactly the kernel's inputs, with the suite's gates (relative RMSE
2e-3 and |dy| <= 2e-2 max(1, |y|) on outputs, relative Frobenius 1e-3 per
(slot, head) on states).  The cases cover ragged batches with partial last
chunks, the longest-first unit order of small packed batches (ties, permuted
slots, inactive sequences of a graph ticket), fp16 and bf16 tokens, decay
bias and scale; at a full serving-size shape the two chunked kernels are
checked against each other.
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
    tokens,
)

pytestmark = pytest.mark.gpu

CHUNKED, CHUNKED_WAVE = 2, 4


def _ticket(case, pool, **kw):
    from flashrwkv2_amd.tmix.wkv7 import prepare_tmix_wkv7_recurrent_metadata

    if not kw:
        kw = dict(total_tokens=case["r"].shape[0])
    return prepare_tmix_wkv7_recurrent_metadata(
        case["cu_seqlens"], case["state_indices"], state_pool_size=pool.shape[0], **kw)


def _forced(C, kernel, case, pool, scale=1.0, ticket=None):
    out = torch.empty_like(case["v"])
    ticket = ticket if ticket is not None else _ticket(case, pool)
    C.tmix_wkv7_recurrent_fp32_kernel_forced(
        kernel, case["cu_seqlens"], case["state_indices"], pool, *tokens(case), out, scale,
        case["decay_bias"], ticket)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_many_units_ragged_batch_matches_oracle(dtype):
    """1 200 units (300 sequences x 4 heads), lengths 1..150 with partial last
    chunks: the forced kernel and the public entry (whose policy picks this
    kernel here) against the oracle."""
    C = require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7

    rng = np.random.default_rng(11)
    lengths = tuple(int(x) for x in rng.integers(1, 151, size=300))
    print(f"case wave ragged dtype={dtype} units=1200 max={max(lengths)}", flush=True)
    case = make_case(dtype=dtype, lengths=lengths, num_heads=4, with_decay_bias=True, seed=21)
    y_ref, pool_ref = oracle_expect(case, scale=0.8)
    active = case["state_indices"].long()
    pool = case["state_pool"].clone()
    out = _forced(C, CHUNKED_WAVE, case, pool, scale=0.8)
    assert_output_close(out, y_ref)
    assert_state_close(pool[active], pool_ref[active.cpu().numpy()])
    pool2 = case["state_pool"].clone()
    out2 = wkv7(*tokens(case), state_pool=pool2, cu_seqlens=case["cu_seqlens"],
                state_indices=case["state_indices"], decay_bias=case["decay_bias"], scale=0.8)
    torch.cuda.synchronize()
    # same kernel on the same inputs: bitwise equal
    assert torch.equal(out, out2) and torch.equal(pool, pool2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_longest_first_order_with_ties_permuted_slots_and_inactive_sequences(dtype):
    """40 sequences (the longest-first order applies) with repeated lengths,
    permuted slots and a graph ticket that leaves the last 7 inactive: the
    active ones match the oracle, the inactive ones' slots and output rows
    stay untouched."""
    C = require_gpu()
    rng = np.random.default_rng(5)
    # the order applies to batches whose longest sequence has >= 256 tokens
    base = [97, 16, 16, 1, 33, 97, 64, 2, 300, 15, 17, 31]
    lengths = tuple(base[i % len(base)] if i % 3 else int(rng.integers(1, 260))
                    for i in range(40))
    print(f"case wave order {dtype} lengths={lengths}", flush=True)
    case = make_case(dtype=dtype, lengths=lengths, num_heads=8, seed=9,
                     state_pool_slots=48)
    perm = torch.from_numpy(rng.permutation(48)[:40].astype(np.int32))
    case["state_indices"] = perm.cuda()
    n_act = 33
    act_tokens = int(case["cu_seqlens"][n_act])
    pool = case["state_pool"].clone()
    before = pool.clone()
    ticket = _ticket(case, pool,
                     token_capacity=case["r"].shape[0], sequence_capacity=40,
                     max_seqlen_capacity=max(lengths),
                     num_active_tokens=torch.full((1,), act_tokens, device="cuda",
                                                  dtype=torch.int32),
                     num_active_sequences=torch.full((1,), n_act, device="cuda",
                                                     dtype=torch.int32))
    out = torch.full_like(case["v"], 3.0)
    C.tmix_wkv7_recurrent_fp32_kernel_forced(
        CHUNKED_WAVE, case["cu_seqlens"], case["state_indices"], pool, *tokens(case), out, 1.0,
        None, ticket)
    torch.cuda.synchronize()
    sub = dict(case)
    sub["cu_seqlens"] = case["cu_seqlens"][:n_act + 1]
    sub["state_indices"] = case["state_indices"][:n_act]
    for name in ("r", "decay_logits", "k", "v", "a", "b"):
        sub[name] = case[name][:act_tokens]
    y_ref, pool_ref = oracle_expect(sub, state_pool=before)
    act = sub["state_indices"].long()
    assert_output_close(out[:act_tokens], y_ref)
    assert_state_close(pool[act], pool_ref[act.cpu().numpy()])
    idle = sorted(set(range(48)) - set(act.tolist()))
    assert torch.equal(pool[idle], before[idle])
    assert bool((out[act_tokens:] == 3.0).all())


def test_wave_and_workgroup_kernels_agree_at_serving_size():
    """16 384 units (512 sequences x 64 tokens x 32 heads, per-sequence states
    ~ N(0, 0.1)): the two chunked kernels evaluate the same chunk algebra in
    a different key order, so they agree to fp32 level (outputs within one
    bf16 rounding, states to 1e-5 relative)."""
    C = require_gpu()
    from flashrwkv2_amd import workloads

    toks = workloads.make_tokens(512 * 64, 32, u_range=(-6.0, -0.5), seed=31, device="cuda")
    w = workloads._pack("serving", toks, [64] * 512, 32, 0.1, 31, "cuda", {})
    print("case wave vs workgroup 512 x 64 x 32", flush=True)
    case = dict(zip(("r", "decay_logits", "k", "v", "a", "b"), w.tokens))
    case.update(cu_seqlens=w.cu_seqlens, state_indices=w.state_indices, decay_bias=None)
    pools, outs = [], []
    for kernel in (CHUNKED, CHUNKED_WAVE):
        pool = w.state_pool.clone()
        outs.append(_forced(C, kernel, case, pool).float())
        pools.append(pool)
    dy = ((outs[0] - outs[1]).abs() / outs[0].abs().clamp(min=1.0)).max().item()
    assert dy <= 2 ** -7, dy
    ds = ((pools[0] - pools[1]).norm() / pools[0].norm()).item()
    assert ds <= 1e-5, ds


def test_bf16_state_pool_on_many_units():
    """The bf16-state chunk entry runs this kernel for many units (1 200 here)
    with a bf16 state load and store (fp32 inside the call, one rounding at
    the end): against the oracle from the same bf16 pool."""
    require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_chunk_bf16_forward_varlen

    import oracle
    from wkv7_testlib import to_np

    rng = np.random.default_rng(17)
    lengths = tuple(int(x) for x in rng.integers(1, 120, size=300))
    print(f"case wave bf16 state units=1200 max={max(lengths)}", flush=True)
    case = make_case(dtype=torch.bfloat16, lengths=lengths, num_heads=4, seed=23)
    pool = case["state_pool"].to(torch.bfloat16)
    before = pool.clone()
    y_ref, pool_ref, _, _ = oracle.wkv7_f64(
        *(to_np(t) for t in tokens(case)), cu_seqlens=case["cu_seqlens"].cpu().numpy(),
        state_indices=case["state_indices"].cpu().numpy(), state_pool=to_np(pool), scale=0.5)
    out = infer_tmix_wkv7_chunk_bf16_forward_varlen(
        *tokens(case), state_pool=pool, cu_seqlens=case["cu_seqlens"],
        state_indices=case["state_indices"], max_seqlen=max(lengths), scale=0.5)
    torch.cuda.synchronize()
    assert_output_close(out, y_ref)
    act = case["state_indices"].long()
    # one bf16 rounding of the final fp32 state (2^-9 relative)
    assert_state_close(pool[act], pool_ref[act.cpu().numpy()], rmse=4e-3, fro=4e-3)
    idle = sorted(set(range(pool.shape[0])) - set(act.tolist()))
    assert torch.equal(pool[idle], before[idle])
