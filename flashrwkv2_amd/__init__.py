"""flashrwkv2_amd — MI355X (gfx950) WKV7 operator with the flashrwkv2.tmix.wkv7 API.

``import flashrwkv2_amd`` loads the in-tree HIP library
(``lib/libflashrwkv2_amd.so``, built by ``python -m flashrwkv2_amd.build``)
when a GPU is present, mirroring the reference's import-time backend load
(flashrwkv2/__init__.py:38-55) with one gfx950 build instead of a
compute-capability selector.  On a host without a GPU ``_C`` is ``None`` and
every entry point raises, exactly like the reference on CPU.
"""

from __future__ import annotations

import sys as _sys

import torch as _torch


def _load_native_backend():
    if not _torch.cuda.is_available():
        return None
    from . import _native, _C as module

    _native.load()  # raises if the library is missing: no silent fallback
    _sys.modules[f"{__name__}._C"] = module
    return module


_C = _load_native_backend()

from .tmix.wkv7 import (  # noqa: E402
    infer_tmix_wkv7_chunk_bf16_forward_varlen,
    infer_tmix_wkv7_recurrent_fp16_forward_varlen,
    infer_tmix_wkv7_recurrent_fp32io16_forward_varlen,
    prepare_tmix_wkv7_recurrent_metadata,
    pretrain_tmix_wkv7_recurrent_bf16,
    rl_infctx_tmix_wkv7_chunk_fp32io16,
    rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute,
    statetune_tmix_wkv7_recurrent_fp32io16,
)

from .tmix.readout import infer_tmix_readout_forward_varlen  # noqa: E402
from .tmix.wkv_prepare import infer_tmix_wkv_prepare_forward_varlen  # noqa: E402

__all__ = [
    "infer_tmix_readout_forward_varlen",
    "infer_tmix_wkv_prepare_forward_varlen",
    "infer_tmix_wkv7_chunk_bf16_forward_varlen",
    "infer_tmix_wkv7_recurrent_fp16_forward_varlen",
    "infer_tmix_wkv7_recurrent_fp32io16_forward_varlen",
    "prepare_tmix_wkv7_recurrent_metadata",
    "pretrain_tmix_wkv7_recurrent_bf16",
    "rl_infctx_tmix_wkv7_chunk_fp32io16",
    "rl_infctx_tmix_wkv7_chunk_fp32io16_factor_recompute",
    "statetune_tmix_wkv7_recurrent_fp32io16",
]

__version__ = "0.1.0"
