"""CPU tests of the shared declarative argument checks and of the host-side
chunk table the RL/Infctx wrapper builds (rl_infctx.py:41-63 of the
reference builds the same table with Python loops)."""

from __future__ import annotations

import pytest
import torch

from flashrwkv2_amd.tmix import _checks as ck
from flashrwkv2_amd.tmix.wkv7.rl_infctx import _chunk_table


def test_verify_stops_at_the_first_failing_rule_in_row_order():
    t = torch.zeros(2, 3)
    rows = [
        ("a", t, [ck.is_tensor(), ck.dtype_in((torch.float32,), "{name} dtype")]),
        ("b", None, [ck.is_tensor()]),
        ("c", 5, [ck.holds(lambda x: x > 10, "{name} small")]),
    ]
    with pytest.raises(TypeError, match="^b must be a torch.Tensor$"):
        ck.verify(rows)
    ck.verify(rows[:1])
    with pytest.raises(ValueError, match="^c small$"):
        ck.verify(rows[2:])


def test_rules_and_optional_values():
    t = torch.zeros(2, 3, dtype=torch.float16)
    with pytest.raises(ValueError, match="x must be contiguous CUDA"):
        ck.verify([("x", t, [ck.cuda_contiguous()])])
    with pytest.raises(ValueError, match="y wrong"):
        ck.verify([("y", torch.zeros(3, 2), [ck.matches(t, "{name} wrong")])])
    ck.verify([("z", None, ck.optional([ck.is_tensor()]))])
    with pytest.raises(TypeError):
        ck.verify([("z", 3, ck.optional([ck.is_tensor()]))])
    assert ck.positive_int(3) and not ck.positive_int(True) and not ck.positive_int(0)
    assert ck.finite(1.5) and not ck.finite(float("nan")) and not ck.finite("x")


@pytest.mark.parametrize("chunk", [16, 32, 64])
def test_chunk_table_matches_a_direct_enumeration(chunk):
    g = torch.Generator().manual_seed(chunk)
    lengths = torch.randint(1, 200, (37,), generator=g)
    offsets = torch.zeros(38, dtype=torch.int64)
    offsets[1:] = torch.cumsum(lengths, 0)
    seq_chunks, starts, ends = _chunk_table(offsets, chunk, "cpu")
    want_sc, want_s, want_e = [0], [], []
    for lo, hi in zip(offsets[:-1].tolist(), offsets[1:].tolist()):
        for s in range(lo, hi, chunk):
            want_s.append(s)
            want_e.append(min(s + chunk, hi))
        want_sc.append(len(want_s))
    assert seq_chunks.dtype == torch.int32
    assert seq_chunks.tolist() == want_sc
    assert starts.tolist() == want_s and ends.tolist() == want_e
