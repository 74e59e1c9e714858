"""Golden-vector tests (tests/golden/*.npz, written by tests/golden/make_golden.py
from an independent numpy fp64 per-token loop).

CPU: the C oracle reproduces every golden file, and the tolerance gates used
by this suite are at least as strict as the reference's own fixture
(tests/fixtures/tolerances-v1.json, copied as tests/golden/tolerances-v1.json).
GPU: every kernel family and the public entry point reproduce the golden
outputs and states.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from wkv7_testlib import (OUTPUT_REL_RMSE, STATE_REL_RMSE, assert_output_close,
                          assert_state_close, require_gpu)

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in GOLDEN.glob("wkv7_*.npz"))
NAMES = ("r", "decay_logits", "k", "v", "a", "b")


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits_to_f32(bits, dtype):
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def test_golden_files_present():
    assert len(CASES) >= 4, CASES


def test_suite_gates_are_at_least_as_strict_as_the_reference_fixture():
    fx = json.loads((GOLDEN / "tolerances-v1.json").read_text())
    gate = fx["fp32io16_recurrent"]
    assert OUTPUT_REL_RMSE <= gate["output_relative_rmse"]
    assert STATE_REL_RMSE <= gate["state_relative_rmse"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    g = load(name)
    dt = str(g["dtype"])
    toks = [bits_to_f32(g[f"in_{n}"], dt) for n in NAMES]
    bias = bits_to_f32(g["in_decay_bias"], dt) if "in_decay_bias" in g else None
    y, pool, _, _ = oracle.wkv7_f64(*toks, cu_seqlens=g["cu_seqlens"],
                                    state_indices=g["state_indices"],
                                    state_pool=g["state_pool"], decay_bias=bias,
                                    scale=float(g["scale"]))
    np.testing.assert_allclose(y, g["y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(pool, g["new_state_pool"], rtol=1e-5, atol=1e-7)


def _gpu_case(g):
    dt = str(g["dtype"])
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    dev = "cuda"

    def tok(bits):
        return torch.from_numpy(bits.astype(np.int16)).view(tdt).to(dev)

    case = {n: tok(g[f"in_{n}"]) for n in NAMES}
    case["decay_bias"] = tok(g["in_decay_bias"]) if "in_decay_bias" in g else None
    case["cu_seqlens"] = torch.from_numpy(g["cu_seqlens"]).to(dev)
    case["state_indices"] = torch.from_numpy(g["state_indices"]).to(dev)
    case["state_pool"] = torch.from_numpy(g["state_pool"]).to(dev)
    return case


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", [None, 0, 1, 2])
@pytest.mark.parametrize("name", CASES)
def test_gpu_reproduces_golden(name, kernel):
    C = require_gpu()
    from flashrwkv2_amd.tmix.wkv7 import (
        infer_tmix_wkv7_recurrent_fp32io16_forward_varlen as wkv7,
        prepare_tmix_wkv7_recurrent_metadata,
    )

    print(f"case golden={name} kernel={kernel}", flush=True)
    g = load(name)
    case = _gpu_case(g)
    pool = case["state_pool"].clone()
    toks = tuple(case[n] for n in NAMES)
    scale = float(g["scale"])
    if kernel is None:
        out = wkv7(*toks, state_pool=pool, cu_seqlens=case["cu_seqlens"],
                   state_indices=case["state_indices"], scale=scale,
                   decay_bias=case["decay_bias"])
    else:
        out = torch.empty_like(case["v"])
        ticket = prepare_tmix_wkv7_recurrent_metadata(
            case["cu_seqlens"], case["state_indices"], total_tokens=out.shape[0],
            state_pool_size=pool.shape[0])
        C.tmix_wkv7_recurrent_fp32_kernel_forced(
            kernel, case["cu_seqlens"], case["state_indices"], pool, *toks, out, scale,
            case["decay_bias"], ticket)
    torch.cuda.synchronize()
    assert_output_close(out, g["y"])
    touched = g["state_indices"].astype(np.int64)
    got = pool.cpu().numpy()
    assert_state_close(got[touched], g["new_state_pool"][touched])
    untouched = np.setdiff1d(np.arange(got.shape[0]), touched)
    assert np.array_equal(got[untouched], g["state_pool"][untouched])
