"""The C-ABI library loads and exports exactly what include/flashrwkv2_amd.h
declares; argument validation answers without touching a GPU (CPU-only)."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from flashrwkv2_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashrwkv2_amd.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(fr2_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        pytest.fail(f"{N.LIB_PATH} missing: run python -m flashrwkv2_amd.build")
    return N.load()


def test_header_declares_the_expected_entry_points():
    names = _declared()
    assert "fr2_wkv7_recurrent_fp32_forward" in names
    assert "fr2_wkv7_prepare_metadata" in names
    assert len(names) >= 10


def test_every_declared_symbol_is_exported_and_bound(lib):
    for name in _declared():
        assert hasattr(lib, name), f"{name} not exported by {N.LIB_PATH.name}"
        assert name in N.SIGNATURES, f"{name} has no ctypes signature"
    assert sorted(N.SIGNATURES) == _declared()


def test_version_and_status_strings(lib):
    assert lib.fr2_abi_version() == 200
    assert lib.fr2_status_string(N.FR2_OK) == b"ok"
    assert lib.fr2_status_string(N.FR2_ERR_INVALID_ARGUMENT) == b"invalid argument"
    assert lib.fr2_status_string(N.FR2_ERR_UNSUPPORTED) == b"unsupported configuration"
    assert lib.fr2_last_error() == b""


def test_null_pointers_and_bad_sizes_are_rejected_before_any_launch(lib):
    nul = None
    assert lib.fr2_wkv7_recurrent_fp32_forward(
        nul, nul, nul, 1, 1, 64, 1, 1, N.FR2_DTYPE_BFLOAT16, nul, nul, nul, nul, nul,
        nul, nul, nul, nul, 1.0, nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_prepare_metadata(
        nul, nul, 1, 1, 1, 1, nul, nul, nul, nul, nul, nul, nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_pretrain_forward(
        1, 15, 1, 64, nul, nul, nul, nul, nul, nul, nul, nul, nul, nul) == N.FR2_ERR_INVALID_ARGUMENT
    fake = 0x1000  # never dereferenced: the size checks fail first
    assert lib.fr2_wkv7_pretrain_forward(
        1, 15, 1, 64, *([fake] * 10), nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_pretrain_forward(
        1, 16, 1, 32, *([fake] * 10), nul) == N.FR2_ERR_UNSUPPORTED
    assert lib.fr2_wkv7_pretrain_backward(
        1, 16, 1, 64, *([fake] * 9), nul, *([fake] * 6), nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_pretrain_backward(
        1, 24, 1, 64, *([fake] * 16), nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_pretrain_backward(
        1, 16, 1, 96, *([fake] * 16), nul) == N.FR2_ERR_UNSUPPORTED
    # workspace: dsa [B,T,H,D] plus, at D = 64, one P snapshot per span of chunks
    assert lib.fr2_wkv7_pretrain_backward_workspace_floats(2, 32, 3, 128) == 2 * 32 * 3 * 128
    n64 = lib.fr2_wkv7_pretrain_backward_workspace_floats(2, 4096, 3, 64)
    assert n64 > 2 * 4096 * 3 * 64 and (n64 - 2 * 4096 * 3 * 64) % (2 * 3 * 64 * 64) == 0
    assert lib.fr2_wkv7_pretrain_backward_workspace_floats(1, 24, 1, 64) == -1
    assert lib.fr2_wkv7_recurrent_fp32_forward(
        fake, fake, fake, 1, 1, 32, 1, 1, N.FR2_DTYPE_BFLOAT16, *([fake] * 9), 1.0,
        nul) == N.FR2_ERR_UNSUPPORTED
    assert lib.fr2_wkv7_recurrent_fp32_forward(
        fake, fake, fake, 0, 1, 64, 1, 1, N.FR2_DTYPE_BFLOAT16, *([fake] * 9), 1.0,
        nul) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_rl_infctx_forward(
        fake, fake, fake, 1, 1, 1, 64, 1, 1, 8, 1, N.FR2_DTYPE_BFLOAT16, *([fake] * 9),
        1.0, nul) == N.FR2_ERR_UNSUPPORTED
    assert lib.fr2_wkv7_recurrent_fp32_forward_kernel(
        7, fake, fake, fake, 1, 1, 64, 1, 1, N.FR2_DTYPE_BFLOAT16, *([fake] * 9), 1.0,
        nul) == N.FR2_ERR_INVALID_ARGUMENT


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        N.load(tmp_path / "libmissing.so")
