"""CPU-side checks of the public surface: names, signatures, and the
behaviour without a GPU (tests/test_runtime.py and the signature tests of
tests/tmix/wkv7/test.py:376-400 in the reference)."""

from __future__ import annotations

import inspect

import pytest
import torch

import flashrwkv2_amd
from flashrwkv2_amd import workloads
from flashrwkv2_amd.tmix.wkv7 import (
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen,
    pretrain_tmix_wkv7_recurrent_bf16,
    rl_infctx_tmix_wkv7_chunk_fp32io16,
    statetune_tmix_wkv7_recurrent_fp32io16,
)

EXPECTED = {
    "infer_tmix_wkv7_chunk_bf16_forward_varlen",
    "infer_tmix_wkv7_recurrent_fp16_forward_varlen",
    "infer_tmix_wkv7_recurrent_fp32io16_forward_varlen",
    "prepare_tmix_wkv7_recurrent_metadata",
    "pretrain_tmix_wkv7_recurrent_bf16",
    "rl_infctx_tmix_wkv7_chunk_fp32io16",
    "rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute",
    "statetune_tmix_wkv7_recurrent_fp32io16",
}


def test_root_exports():
    assert EXPECTED <= set(flashrwkv2_amd.__all__)
    for name in EXPECTED:
        assert callable(getattr(flashrwkv2_amd, name))


def test_public_signature_is_raw_only():
    sig = inspect.signature(infer_tmix_wkv7_recurrent_fp32io16_forward_varlen)
    params = sig.parameters
    assert "decay_logits" in params and "state_pool" in params
    for absent in ("initial_state", "output_final_state", "log_decay", "elapsed_t"):
        assert absent not in params
    assert params["scale"].default == 1.0
    assert params["decay_bias"].default is None
    assert params["max_seqlen"].default is None
    assert params["validated_metadata"].default is None
    with pytest.raises(TypeError, match="log_decay"):
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
            None, None, None, None, None, None, state_pool=None, cu_seqlens=None,
            log_decay=None)


def test_pretrain_contract_signature():
    sig = inspect.signature(pretrain_tmix_wkv7_recurrent_bf16)
    assert tuple(sig.parameters) == ("r", "w", "k", "v", "a", "b", "head_size")
    assert sig.parameters["head_size"].default == 64


@pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only behaviour")
def test_without_gpu_backend_is_none_and_entry_points_raise():
    assert flashrwkv2_amd._C is None
    t = torch.zeros((2, 1, 64), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="not built"):
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
            t, t, t, t, t, t, state_pool=torch.zeros(1, 1, 64, 64),
            cu_seqlens=torch.tensor([0, 2], dtype=torch.int32),
            state_indices=torch.tensor([0], dtype=torch.int32))


def test_python_side_validation_precedes_the_native_layer():
    t = torch.zeros((2, 1, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        pretrain_tmix_wkv7_recurrent_bf16(*(torch.zeros((1, 16, 64), dtype=torch.bfloat16),) * 6)
    with pytest.raises(ValueError, match="chunk_size must be one of"):
        rl_infctx_tmix_wkv7_chunk_fp32io16(t, t, t, t, t, t, cu_seqlens=None, chunk_size=8)
    with pytest.raises(ValueError, match="strategy"):
        rl_infctx_tmix_wkv7_chunk_fp32io16(t, t, t, t, t, t, cu_seqlens=None, strategy="x")
    with pytest.raises(TypeError, match="state_pool must be a torch.Tensor"):
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen(
            t, t, t, t, t, t, state_pool=None, cu_seqlens=None, state_indices=None)


def test_workload_distributions_follow_the_config_contract():
    w = workloads.config(0, "cpu", dtype=torch.float32)
    assert w.r.shape == (64, 4, 64)
    import math

    # retention implied by the logits lies in exp(-exp(u)) for u in [-6, -0.5]
    x = w.decay_logits.double()
    ret = torch.exp(-math.exp(-0.5) * torch.sigmoid(x))
    assert ret.min() >= math.exp(-math.exp(-0.5)) - 1e-6
    assert ret.max() <= math.exp(-math.exp(-6.0)) + 1e-6
    # a = -kk with |kk| = 1 per (token, head); b = kk * sigmoid(.) so |b| <= |kk|
    kk = -w.a.double()
    assert torch.allclose(kk.norm(dim=-1), torch.ones(64, 4, dtype=torch.float64), atol=1e-6)
    ratio = w.b.double() / kk
    assert ((ratio > 0) & (ratio < 1)).all()
    w2 = workloads.config(2, "cpu", batch=8, heads=2)
    assert w2.state_pool.shape == (8, 2, 64, 64)
    assert 0.07 < w2.state_pool.std().item() < 0.13
    w3 = workloads.config(3, "cpu", sequences=5, heads=2, max_len=50)
    lens = (w3.cu_seqlens[1:] - w3.cu_seqlens[:-1])
    assert (lens >= 1).all() and (lens <= 50).all()


def test_fp16_public_signature_is_raw_only_and_has_no_elapsed_alias():
    """Mirrors tests/tmix/wkv7/test.py:883-895 of the reference."""
    import inspect

    from flashrwkv2_amd.tmix.wkv7 import infer_tmix_wkv7_recurrent_fp16_forward_varlen as f

    params = inspect.signature(f).parameters
    for name in ("decay_logits", "state_pool", "elapsed_state_pool", "max_seqlen"):
        assert name in params
    for name in ("log_decay", "elapsed_t"):
        assert name not in params
    assert params["scale"].default == 1.0 and params["decay_bias"].default is None


def test_statetune_signature_and_python_checks():
    """statetune.py:202-236 of the reference: keyword-only scale, the
    reference's check order and messages (CPU tensors are rejected before
    anything reaches the native layer)."""
    sig = inspect.signature(statetune_tmix_wkv7_recurrent_fp32io16)
    assert tuple(sig.parameters)[:10] == (
        "initial_state", "sequence_chunk_offsets", "chunk_token_starts", "chunk_token_ends",
        "r", "decay_logits", "k", "v", "a", "b")
    assert sig.parameters["scale"].kind is inspect.Parameter.KEYWORD_ONLY
    assert sig.parameters["scale"].default == 1.0
    t = torch.zeros((5, 1, 64), dtype=torch.bfloat16)
    meta = [torch.tensor(x, dtype=torch.int32) for x in ([0, 1], [0], [5])]
    with pytest.raises(ValueError, match="state must be contiguous CUDA"):
        statetune_tmix_wkv7_recurrent_fp32io16(torch.zeros((1, 1, 64, 64)), *meta, *(t,) * 6)
    with pytest.raises(TypeError, match="state must be a torch.Tensor"):
        statetune_tmix_wkv7_recurrent_fp32io16(None, *meta, *(t,) * 6)


def test_statetune_uniform_layout_detection():
    """The chunk lists the chunked MFMA StateTune kernels take: equal
    sequences packed back to back, equal chunks of a multiple of 16 tokens,
    D = 64, bf16 (checked on CPU metadata; the same code reads it on the
    device)."""
    import importlib

    C = importlib.import_module("flashrwkv2_amd._C")
    detect = C._statetune_uniform_chunk_len
    i32 = lambda x: torch.tensor(x, dtype=torch.int32)
    bf = torch.bfloat16
    # 2 sequences x 64 tokens as chunks of 32
    assert detect(i32([0, 2, 4]), i32([0, 32, 64, 96]), i32([32, 64, 96, 128]), 2, 4, 128, 64,
                  bf) == 32
    assert detect(i32([0, 1, 2]), i32([0, 64]), i32([64, 128]), 2, 2, 128, 64, bf) == 64
    # not a multiple of 16, unequal chunks, a gap, fp16, D = 128
    assert detect(i32([0, 2, 4]), i32([0, 8, 16, 24]), i32([8, 16, 24, 32]), 2, 4, 32, 64,
                  bf) is None
    assert detect(i32([0, 2, 4]), i32([0, 16, 64, 96]), i32([16, 64, 96, 128]), 2, 4, 128, 64,
                  bf) is None
    assert detect(i32([0, 1, 2]), i32([0, 80]), i32([64, 144]), 2, 2, 128, 64, bf) is None
    assert detect(i32([0, 1, 2]), i32([0, 64]), i32([64, 128]), 2, 2, 128, 64,
                  torch.float16) is None
    assert detect(i32([0, 1, 2]), i32([0, 64]), i32([64, 128]), 2, 2, 128, 128, bf) is None
