"""ctypes binding of the gfx950 C-ABI library (``include/flashrwkv2_amd.h``).

The library is built in-tree by :mod:`flashrwkv2_amd.build`.  Loading never
falls back to anything: a missing library raises, so no code path can silently
run elsewhere than the HIP kernels.  ``torch`` is imported first so that the
library binds to the HIP runtime torch already loaded (both carry the
``libamdhip64.so.7`` soname).
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_void_p, c_char_p, POINTER
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see docstring)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libflashrwkv2_amd.so"

FR2_OK = 0
FR2_ERR_INVALID_ARGUMENT = 1
FR2_ERR_UNSUPPORTED = 2
FR2_ERR_LAUNCH = 3

FR2_DTYPE_FLOAT16 = 0
FR2_DTYPE_BFLOAT16 = 1

KERNEL_SERIAL = 0
KERNEL_DECODE = 1
KERNEL_CHUNKED = 2
KERNEL_SPLIT = 3   # chunked, long sequences cut into pieces (Python-side selector)
KERNEL_CHUNKED_WAVE = 4   # chunked, one wavefront per (sequence, head)

_i32p = POINTER(c_int32)

# name -> (restype, argtypes); mirrors include/flashrwkv2_amd.h exactly.
SIGNATURES: dict[str, tuple] = {
    "fr2_abi_version": (c_int32, []),
    "fr2_status_string": (c_char_p, [c_int32]),
    "fr2_last_error": (c_char_p, []),
    "fr2_handoff_fault_count": (c_int32, [_i32p, c_int32, c_void_p]),
    "fr2_debug_set_handoff_spin_limit": (c_int32, [c_int32]),
    "fr2_debug_set_handoff_stall": (c_int32, [c_int32]),
    "fr2_debug_set_chunk_ring": (c_int32, [c_int32]),
    "fr2_wkv7_prepare_metadata": (
        c_int32,
        [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_forward": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_forward_kernel": (
        c_int32,
        [c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
         c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_dispatch": (
        c_int32, [c_int32, c_int32, c_int32, c_int64, c_int32, _i32p],
    ),
    "fr2_wkv7_recurrent_fp32_split_plan": (
        c_int32, [c_int32, c_int32, c_int32, c_int32, _i32p, _i32p, _i32p, POINTER(c_int64)],
    ),
    "fr2_wkv7_recurrent_fp32_forward_split": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32,
         c_int32, c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_forward_split_noalloc": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32,
         c_int32, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_forward_kk_gate": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_int32] + [c_void_p] * 12 + [c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp32_forward_kk_gate_readout": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_int32] + [c_void_p] * 17 + [c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp16_forward": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp16_update": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp16_update_kernel": (
        c_int32,
        [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64,
         c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_recurrent_fp16_advance_elapsed": (
        c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p],
    ),
    "fr2_wkv7_pretrain_forward": (
        c_int32,
        [c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "fr2_wkv7_pretrain_backward_workspace_floats": (
        c_int64, [c_int32, c_int32, c_int32, c_int32],
    ),
    "fr2_wkv7_pretrain_backward": (
        c_int32,
        [c_int32, c_int32, c_int32, c_int32] + [c_void_p] * 17,
    ),
    "fr2_wkv7_statetune_forward": (
        c_int32,
        [c_void_p] * 3 + [c_int32, c_int32, c_int64, c_int32, c_int32, c_int32]
        + [c_void_p] * 10 + [c_float, c_void_p],
    ),
    "fr2_wkv7_statetune_backward_workspace_floats": (
        c_int64, [c_int64, c_int32, c_int32],
    ),
    "fr2_wkv7_statetune_backward": (
        c_int32,
        [c_void_p] * 3 + [c_int32, c_int32, c_int64, c_int32, c_int32, c_int32]
        + [c_void_p] * 18 + [c_float, c_void_p],
    ),
    "fr2_wkv7_statetune_uniform_forward": (
        c_int32, [c_int32] * 4 + [c_void_p] * 11 + [c_float, c_void_p],
    ),
    "fr2_wkv7_statetune_uniform_backward_workspace_floats": (
        c_int64, [c_int32] * 3,
    ),
    "fr2_wkv7_statetune_padded_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "fr2_wkv7_statetune_padded_forward": (
        c_int32,
        [c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p] + [c_void_p] * 12
        + [c_float, c_void_p],
    ),
    "fr2_wkv7_statetune_padded_backward": (
        c_int32,
        [c_int32, c_int32, c_int32, c_void_p, c_void_p] + [c_void_p] * 19 + [c_float, c_void_p],
    ),
    "fr2_wkv7_statetune_uniform_backward": (
        c_int32, [c_int32] * 4 + [c_void_p] * 19 + [c_float, c_void_p],
    ),
    "fr2_tmix_kk_a_gate_forward": (
        c_int32, [c_int64, c_int32, c_int32] + [c_void_p] * 9,
    ),
    "fr2_tmix_lowrank_activate": (
        c_int32, [c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p],
    ),
    "fr2_tmix_vres_forward": (
        c_int32, [c_int64, c_int32] + [c_void_p] * 6,
    ),
    "fr2_tmix_readout_prelinear_forward": (
        c_int32, [c_int64, c_int32, c_int32] + [c_void_p] * 10,
    ),
    "fr2_wkv7_chunk_bf16_forward": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int64, c_int32,
         c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
    "fr2_wkv7_chunk_bf16_forward_split": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int64, c_int32,
         c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32, c_int32,
         c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "fr2_wkv7_rl_infctx_forward": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
         c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_float, c_void_p],
    ),
    "fr2_wkv7_rl_infctx_replay": (
        c_int32,
        [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int32,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_float, c_void_p],
    ),
}

_LIB: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with every signature bound."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.exists():
        raise RuntimeError(
            f"flashrwkv2_amd native library not built: {lib_path} is missing; "
            "run `python -m flashrwkv2_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _LIB = lib
    return lib


_FAST = None


def fast():
    """The CPython fast-call module over the same library (built next to it by
    :mod:`flashrwkv2_amd.build`): the per-step entries without ctypes'
    argument conversion.  Loaded once, after the library itself."""
    global _FAST
    if _FAST is None:
        import importlib.machinery
        import importlib.util

        from .build import fastcall_name

        load()
        path = LIB_PATH.parent / fastcall_name()
        if not path.exists():
            raise RuntimeError(f"flashrwkv2_amd fast-call module not built: {path} is missing; "
                               "run `python -m flashrwkv2_amd.build`")
        loader = importlib.machinery.ExtensionFileLoader("_fastcall", str(path))
        spec = importlib.util.spec_from_file_location("_fastcall", path, loader=loader)
        module = importlib.util.module_from_spec(spec)
        loader.exec_module(module)
        _FAST = module
    return _FAST


_HOST = None


def hostpath():
    """The torch C++ extension with the native fast path of the per-step
    ticket and recurrence calls (built next to the library by
    :mod:`flashrwkv2_amd.build`; it links the library).  Loaded once."""
    global _HOST
    if _HOST is None:
        import importlib.machinery
        import importlib.util

        from .build import hostpath_name

        load()
        path = LIB_PATH.parent / hostpath_name()
        if not path.exists():
            raise RuntimeError(f"flashrwkv2_amd host-path module not built: {path} is missing; "
                               "run `python -m flashrwkv2_amd.build`")
        loader = importlib.machinery.ExtensionFileLoader("_hostpath", str(path))
        spec = importlib.util.spec_from_file_location("_hostpath", path, loader=loader)
        module = importlib.util.module_from_spec(spec)
        loader.exec_module(module)
        _HOST = module
    return _HOST


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero fr2_status_t."""
    if status == FR2_OK:
        return
    lib = load()
    text = lib.fr2_status_string(status).decode()
    detail = lib.fr2_last_error().decode()
    raise RuntimeError(f"{what} failed: {text}{(': ' + detail) if detail else ''}")


def ptr(t: "torch.Tensor | None") -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: "torch.device") -> int:
    return torch.cuda.current_stream(device).cuda_stream
