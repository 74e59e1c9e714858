"""The padded grid of a StateTune chunk list (host logic, CPU): every chunk
starts on a 16-token boundary of its sequence's grid rows, each grid row
maps to its token or to -1 (identity), and the lists the grid does not suit
are refused."""

from __future__ import annotations

import numpy as np
import torch

from flashrwkv2_amd._statetune_plan import statetune_padded_plan


def _plan(offsets, starts, ends, T, B=None, dtype=torch.bfloat16, D=64):
    t = lambda x: torch.tensor(x, dtype=torch.int32)   # noqa: E731
    B = len(offsets) - 1 if B is None else B
    return statetune_padded_plan(t(offsets), t(starts), t(ends), B, len(starts), T, D, dtype)


def test_ragged_gaps_and_empty_chunks():
    # sequence 0: chunks of 1, 17, 0 and 40 tokens (tokens 58..60 in no
    # chunk); sequence 1: 33 and 7 tokens; sequence 2: no chunks
    Tp, rows, cseq, pstart, first = _plan([0, 4, 6, 6], [0, 1, 18, 18, 61, 94],
                                          [1, 18, 18, 58, 94, 101], 101)
    assert Tp == 96   # sequence 0: 16 + 32 + 0 + 48 = 96
    assert cseq.tolist() == [0, 0, 0, 0, 1, 1]
    assert pstart.tolist() == [0, 16, 48, 48, 0, 48]
    assert first.tolist() == [0, 4, -1]
    g = rows.reshape(3, Tp)
    assert g[0, 0] == 0 and (g[0, 1:16] == -1).all()
    assert g[0, 16:33].tolist() == list(range(1, 18)) and (g[0, 33:48] == -1).all()
    assert g[0, 48:88].tolist() == list(range(18, 58)) and (g[0, 88:] == -1).all()
    assert g[1, :33].tolist() == list(range(61, 94)) and g[1, 48:55].tolist() == list(range(94, 101))
    assert (g[2] == -1).all()
    # every covered token appears exactly once, gap tokens never
    used = rows[rows >= 0]
    assert sorted(used.tolist()) == list(range(0, 58)) + list(range(61, 101))


def test_uniform_list_maps_one_to_one():
    B, per, L = 2, 64, 32
    offs = [0, 2, 4]
    starts = [0, 32, 64, 96]
    Tp, rows, cseq, pstart, first = _plan(offs, starts, [s + L for s in starts], B * per)
    assert Tp == per and np.array_equal(rows, np.arange(B * per))
    assert pstart.tolist() == [0, 32, 0, 32] and first.tolist() == [0, 2]


def test_refused_lists():
    # fp16 tokens, head size 128, a token row in two chunks, rows out of range,
    # and a grid four times larger than its tokens (1-token chunks)
    assert _plan([0, 1], [0], [8], 8, dtype=torch.float16) is None
    assert _plan([0, 1], [0], [8], 8, D=128) is None
    assert _plan([0, 2], [0, 4], [8, 12], 12) is None
    assert _plan([0, 1], [0], [9], 8) is None
    assert _plan([0, 4], [0, 1, 2, 3], [1, 2, 3, 4], 4) is None
