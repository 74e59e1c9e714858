"""The C-ABI library loads and exports exactly what include/flashrwkv2_amd.h
declares; argument validation answers without touching a GPU (CPU-only)."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

import torch

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
    # kernel ids: 0 serial, 1 decode, 2 / 4 the two chunked forms; 3 is the
    # Python layer's split selector, not a library kernel
    for bad in (3, 5, 7, -2):
        assert lib.fr2_wkv7_recurrent_fp32_forward_kernel(
            bad, fake, fake, fake, 1, 1, 64, 1, 1, N.FR2_DTYPE_BFLOAT16, *([fake] * 9), 1.0,
            nul) == N.FR2_ERR_INVALID_ARGUMENT


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        N.load(tmp_path / "libmissing.so")


def _plan(lib, n, h, d, maxlen):
    import ctypes
    pc, pl, ll, wb = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    rc = lib.fr2_wkv7_recurrent_fp32_split_plan(n, h, d, maxlen, ctypes.byref(pc),
                                                ctypes.byref(pl), ctypes.byref(ll),
                                                ctypes.byref(wb))
    assert rc == N.FR2_OK
    return pc.value, pl.value, ll.value, wb.value


def test_split_plan_config4_and_no_split_cases(lib):
    """The pipelined split plan (host code, no GPU): BASELINE config 4 gets
    5 pieces with a longer piece 0; config 1 (256 units), D != 64, short
    sequences and more than 128 units are not split."""
    assert _plan(lib, 1, 64, 64, 65536) == (5, 12992, 13568, (3 * 5 - 2) * 64 * 64 * 64 * 4)
    for args in ((8, 32, 64, 4096), (1, 64, 128, 65536), (1, 32, 64, 1024), (1, 129, 64, 65536),
                 (4, 32, 64, 127)):
        assert _plan(lib, *args)[0] == 1, args


@pytest.mark.parametrize("n,h,maxlen", [(1, 4, 8192), (2, 2, 4000), (2, 32, 4096), (1, 64, 2048),
                                        (3, 32, 65536), (1, 8, 65536), (128, 1, 3000)])
def test_split_plan_invariants(lib, n, h, maxlen):
    """Every split plan covers max_seqlen exactly with its pieces, keeps
    pieces of at least 384 tokens in multiples of 32, gives piece 0 at least
    the others' length, fills at most one workgroup per CU in each phase, and
    asks for the classic workspace bound."""
    P, plen, lead, ws = _plan(lib, n, h, 64, maxlen)
    assert P >= 3
    assert plen >= 384 and plen % 32 == 0 and lead % 32 == 0 and lead >= plen
    assert lead + (P - 2) * plen < maxlen <= lead + (P - 1) * plen
    assert (P - 1) * n * h <= 256
    assert ws == n * (3 * P - 2) * h * 64 * 64 * 4


def test_split_plan_rejects_bad_arguments(lib):
    import ctypes
    one = ctypes.c_int32()
    wb = ctypes.c_int64()
    assert lib.fr2_wkv7_recurrent_fp32_split_plan(0, 4, 64, 8192, ctypes.byref(one),
                                                  ctypes.byref(one), ctypes.byref(one),
                                                  ctypes.byref(wb)) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_recurrent_fp32_split_plan(1, 4, 64, 8192, None, ctypes.byref(one),
                                                  ctypes.byref(one),
                                                  ctypes.byref(wb)) == N.FR2_ERR_INVALID_ARGUMENT


def test_misaligned_token_pointers_are_rejected_before_any_launch(lib):
    """Token rows are accessed as 16-byte vectors: a token pointer that is not
    16-byte aligned (e.g. a contiguous view with an odd storage offset) is
    an invalid argument, answered before any HIP call."""
    fake, odd = 0x1000, 0x1002
    for pos in range(7):   # r, decay_logits, k, v, a, b, output
        toks = [fake] * 7
        toks[pos] = odd
        r, l, k, v, a, b, out = toks
        assert lib.fr2_wkv7_recurrent_fp32_forward(
            fake, fake, fake, 1, 1, 64, 1, 1, N.FR2_DTYPE_BFLOAT16, fake, r, l, None, k, v, a,
            b, out, 1.0, None) == N.FR2_ERR_INVALID_ARGUMENT, pos
    assert lib.fr2_wkv7_pretrain_forward(
        1, 16, 1, 64, odd, *([fake] * 9), None) == N.FR2_ERR_INVALID_ARGUMENT


def test_handoff_hooks_validate_their_arguments(lib):
    assert lib.fr2_handoff_fault_count(None, 0, None) == N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_debug_set_handoff_spin_limit(-1) == N.FR2_OK


def test_fast_call_and_host_path_modules_load(lib):
    """Both per-step modules are built next to the library and load on a
    machine without a GPU (no compute calls)."""
    from flashrwkv2_amd import _native as N

    fast = N.fast()
    for name in ("prepare_metadata", "recurrent_fp32_forward", "recurrent_fp32_forward_kernel"):
        assert callable(getattr(fast, name))
    host = N.hostpath()
    for name in ("TicketFacts", "recurrent_fp32", "prepare_graph"):
        assert hasattr(host, name)
    # a CPU tensor is never plainly valid for the fast path: it declines
    t = torch.zeros(1, dtype=torch.int32)
    assert host.prepare_graph(t, t, t, t, 1, 1, 1, 1, 0) is None


@pytest.mark.parametrize("n,h,d,total,maxlen,want", [
    (8, 32, 64, 8 * 4096, 4096, 2),        # config 1: one workgroup per unit
    (256, 32, 64, 256, 1, 1),              # config 2: decode
    (2048, 32, 64, 2048 * 100, 100, 4),    # many mid-length units: one wave per unit
    (64, 64, 64, 68041, 2048, 5),          # config 3: longest-first order
    (64, 64, 64, 60000, 2048, 2),          # longest above twice the mean: workgroup kernel
    (64, 64, 64, 64 * 2048, 2048, 4),      # equal lengths: no order
    (8, 32, 128, 8 * 4096, 4096, 0),       # head size 128: token-serial
    (8, 32, 64, 8 * 4096, 0, 0),           # unknown max_seqlen: token-serial
])
def test_dispatch_query_reports_the_policy(lib, n, h, d, total, maxlen, want):
    import ctypes
    fam = ctypes.c_int32(-1)
    assert lib.fr2_wkv7_recurrent_fp32_dispatch(n, h, d, total, maxlen, ctypes.byref(fam)) == 0
    assert fam.value == want


def test_dispatch_query_rejects_bad_arguments(lib):
    import ctypes
    fam = ctypes.c_int32(-1)
    assert lib.fr2_wkv7_recurrent_fp32_dispatch(0, 4, 64, 10, 10, ctypes.byref(fam)) == \
        N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_recurrent_fp32_dispatch(4, 4, 64, 10, 10, None) == \
        N.FR2_ERR_INVALID_ARGUMENT
    assert lib.fr2_wkv7_recurrent_fp32_dispatch(4, 4, 96, 10, 10, ctypes.byref(fam)) == \
        N.FR2_ERR_UNSUPPORTED


def _brute_span(batch, tokens, heads):
    """The key pass's span length by brute force: every candidate's
    workgroups (each (batch, head)'s full spans first, then its last span)
    placed one by one on the least loaded of 768 slots, each costing its
    chunks plus one; the shortest makespan wins, ties to the longer span."""
    import heapq

    units, nchunk = batch * heads, tokens // 16
    if units * ((nchunk + 15) // 16) < 2048:
        return 8
    best = None
    for cps in range(17, 7, -1):
        nspan = -(-nchunk // cps)
        last = nchunk - (nspan - 1) * cps
        slots = [0.0] * 768
        for d in [cps + 1.0] * (units * (nspan - 1)) + [last + 1.0] * units:
            heapq.heappush(slots, heapq.heappop(slots) + d)
        t = max(slots)
        if best is None or t < best[1]:
            best = (cps, t)
    return best[0]


@pytest.mark.parametrize("batch,tokens,heads", [
    (8, 4096, 32), (1, 4096, 128), (4, 8192, 64), (8, 2048, 32), (64, 1024, 64),
    (2, 4096, 32), (3, 6144, 48), (16, 4096, 40), (64, 4096, 64), (5, 3072, 24),
    (1, 16384, 40), (7, 4000, 33),
])
def test_key_pass_span_matches_a_brute_force_schedule(lib, batch, tokens, heads):
    ws = lib.fr2_wkv7_pretrain_backward_workspace_floats(batch, tokens, heads, 64)
    nspan = (ws - batch * tokens * heads * 64) // (batch * heads * 64 * 64)
    cps = _brute_span(batch, tokens, heads)
    assert nspan == -(-(tokens // 16) // cps)
