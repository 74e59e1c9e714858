"""Host-side layout of StateTune's ragged chunk lists for the chunked
kernels (fr2_wkv7_statetune_padded_forward / _backward)."""

from __future__ import annotations

import torch


def statetune_padded_plan(offsets, starts, ends, B, C, T, D, dtype):
    """The padded layout of any chunk list (D = 64, bf16): sequence b's chunks
    back to back from grid row b * Tp, each starting on a 16-token boundary,
    identity tokens in between.  Returns (Tp, row_source [B*Tp], chunk_seq
    [C], chunk_pstart [C], seq_first_chunk [B]) as host int32 arrays, or None
    when the list does not suit it (out-of-range or shared token rows, or a
    grid more than four times the tokens it carries: many tiny chunks run
    faster token-serial).  Reads the chunk metadata on the host."""
    import numpy as np

    if D != 64 or dtype != torch.bfloat16:
        return None
    meta = torch.cat([offsets, starts, ends]).cpu().numpy().astype(np.int64)
    off, st, en = meta[:B + 1], meta[B + 1:B + 1 + C], meta[B + 1 + C:]
    lens = en - st
    if (off[0] != 0 or off[-1] != C or np.any(np.diff(off) < 0) or np.any(lens < 0)
            or np.any(st < 0) or np.any(en > T)):
        return None
    padded = (lens + 15) // 16 * 16
    chunk_seq = np.repeat(np.arange(B), np.diff(off))
    # padded start of each chunk within its sequence: exclusive cumsum per sequence
    csum = np.concatenate([[0], np.cumsum(padded)])
    pstart = csum[:-1] - csum[off[chunk_seq]]
    seq_len = csum[off[1:]] - csum[off[:-1]]
    Tp = int(max(16, -(-int(seq_len.max(initial=0)) // 16) * 16))
    used = int(lens.sum())
    if B * Tp > 4 * max(used, 1):
        return None
    row_source = np.full(B * Tp, -1, dtype=np.int64)
    if used:
        cid = np.repeat(np.arange(C), lens)
        within = np.arange(used) - np.repeat(np.cumsum(lens) - lens, lens)
        src = st[cid] + within
        if np.unique(src).size != used:
            return None
        row_source[chunk_seq[cid] * Tp + pstart[cid] + within] = src
    first = np.where(np.diff(off) > 0, off[:-1], -1)
    i32 = lambda a: a.astype(np.int32)   # noqa: E731
    return Tp, i32(row_source), i32(chunk_seq), i32(pstart), i32(first)
