"""The ring variant of the workgroup chunked kernel is the default for every
inference contract (the bf16-state pool, rl_infctx chunk lists, the fused
kk / a-gate stage, the real and summary passes of the sequence split).  With
the ring switched off (`_C._set_chunk_ring(False)`) the same entries run on
the key-half kernel instead; these cases re-run representative parity tests
of each entry in that configuration, so both kernels stay checked against
the fp64 oracle.  The training backward's value pass (the reverse mode) is
on the ring as well, and is re-run here on the key-half kernel too."""

from __future__ import annotations

import pytest
import torch

import test_gpu_kk_fused as kk_tests
import test_gpu_other_entries as entry_tests
import test_gpu_pretrain_backward as bwd_tests
import test_gpu_split as split_tests
import test_gpu_statetune as st_tests
from wkv7_testlib import require_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture
def ring_off():
    C = require_gpu()
    C._set_chunk_ring(False)
    try:
        yield
    finally:
        C._set_chunk_ring(True)


def test_chunk_bf16_state_on_the_key_half_kernel(ring_off):
    entry_tests.test_chunk_bf16_ragged_tail_and_slot_update(16)
    entry_tests.test_chunk_bf16_long_requests_on_the_chunked_kernel()


def test_rl_infctx_on_the_key_half_kernel(ring_off):
    entry_tests.test_rl_infctx_ragged_materialized_and_recompute(64)
    entry_tests.test_rl_infctx_chunk_sizes_and_tail(64)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_fused_kk_gate_on_the_key_half_kernel(ring_off, dtype):
    kk_tests.test_fused_kk_gate_matches_the_two_stage_oracle(dtype, (300, 64, 96, 41), 4, True)


@pytest.mark.parametrize("lengths,pieces", [((700, 64, 1, 129, 1024), 4),
                                            ((700, 64, 1, 129, 1024), (4, 320))])
def test_split_summary_on_the_key_half_kernel(ring_off, lengths, pieces):
    split_tests.test_split_matches_oracle_and_unsplit(lengths, pieces, torch.bfloat16)


def test_pretrain_backward_value_pass_on_the_key_half_kernel(ring_off):
    bwd_tests.test_backward_multi_chunk_strong_inputs(1, 256, 2, 64)
    bwd_tests.test_backward_long_sequence()
    bwd_tests.test_backward_extreme_decay(-6.0)


def test_statetune_value_pass_on_the_key_half_kernel(ring_off):
    st_tests.test_statetune_uniform_layout_runs_chunked_kernels(2, 256, 16, 0.75)
