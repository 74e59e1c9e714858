"""Misaligned tensor views at the native boundary.

The kernels read and write token rows and per-channel parameters as 16-byte
vectors, and the C ABI rejects pointers that are not 16-byte aligned.  The
reference accepts any contiguous view, including one with an odd storage
offset; :func:`aligned_io` lets each ``_C`` entry do the same.
"""

from __future__ import annotations

import functools

import torch

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def aligned_io(fn):
    """The kernels read and write token rows and per-channel parameters as
    16-byte vectors, and the C ABI rejects pointers that are not 16-byte
    aligned.  The reference accepts any contiguous view, including one with
    an odd storage offset; so does this layer: a misaligned floating-point
    CUDA tensor argument is replaced by an aligned contiguous copy for the
    call, and copied back afterwards (it may be an output or an in-place
    state pool).  (CPU tensors go through the same steps; the checks behind
    reject them anyway.)  Returned tensors that are such copies are mapped back to
    the caller's tensors.  Aligned arguments (every tensor torch allocates)
    pass through untouched."""

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        swaps = None
        for i, a in enumerate(args):
            if type(a) is torch.Tensor and a.data_ptr() & 15 and a.dtype in _FLOAT_DTYPES:
                swaps = swaps or {}
                swaps[("a", i)] = a
        for key, a in kwargs.items():
            if type(a) is torch.Tensor and a.data_ptr() & 15 and a.dtype in _FLOAT_DTYPES:
                swaps = swaps or {}
                swaps[("k", key)] = a
        if swaps is None:
            return fn(*args, **kwargs)
        args = list(args)
        copies = {}   # id of the caller's tensor -> aligned copy (one per tensor)
        for (kind, key), a in swaps.items():
            c = copies.get(id(a))
            if c is None:
                c = copies[id(a)] = a.contiguous().clone() if a.is_contiguous() else a
            if kind == "a":
                args[key] = c
            else:
                kwargs[key] = c
        res = fn(*args, **kwargs)
        back = {}
        for a in {id(t): t for t in swaps.values()}.values():
            c = copies[id(a)]
            if c is not a:
                a.copy_(c)
                back[id(c)] = a

        def remap(x):
            if type(x) is torch.Tensor and id(x) in back:
                return back[id(x)]
            if isinstance(x, tuple):
                return tuple(remap(y) for y in x)
            return x

        return remap(res)

    return wrapper
