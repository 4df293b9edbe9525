"""ctypes binding of the in-tree HIP library ``mzoo_amd/_mzk.so`` (C ABI in ``include/mzk.h``).

``torch`` is imported first so that the library binds to the HIP runtime torch already
loaded (both carry the SONAME ``libamdhip64.so.7``); kernels are then launched on torch's
streams.  There is no fallback: if the library is missing, or no GPU is visible, the
call raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import re

import torch

# MZOO_AMD_LIB names another build of the library (the sanitizer build of the host code)
LIB_PATH = pathlib.Path(os.environ.get("MZOO_AMD_LIB") or pathlib.Path(__file__).resolve().parent / "_mzk.so")
HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "mzk.h"

MZK_F32, MZK_BF16, MZK_F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: MZK_F32, torch.bfloat16: MZK_BF16, torch.float16: MZK_F16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> argtypes (restype is c_int unless listed in _RESTYPE)
_SIGS = {
    "mzk_version": [],
    "mzk_last_error": [],
    "mzk_fake_quant_fp8_block": [_P, _P, _I32, _I64, _I64, _I32, _P],
    "mzk_fake_quant_fp4_block": [_P, _P, _I32, _I64, _I64, _I32, _I32, _P],
    "mzk_quant_fp8_block": [_P, _I32, _I64, _I64, _I32, _P, _P, _P],
    "mzk_quant_mxfp4": [_P, _I32, _I64, _I64, _P, _P, _P],
    "mzk_dequant_fp8_block": [_P, _P, _I64, _I64, _I32, _P, _I32, _P],
    "mzk_dequant_mxfp4": [_P, _P, _I64, _I64, _P, _I32, _P],
    "mzk_pack_latent_fp8_b128": [_P, _I32, _I64, _I32, _I32, _P, _P, _P],
    "mzk_decode_prologue": [_P, _I32, _I64, _I32, _I32, _P, _P, _I64, _I32, _P, _I32, _I64, _I32, _I32, _P, _P, _P,
                            _P],
    "mzk_unpack_latent_fp8_b128": [_P, _I64, _I32, _I32, _P, _I32, _P],
    "mzk_pack_cache_v41": [_P, _I32, _I64, _I32, _I32, _P, _P, _P],
    "mzk_unpack_cache_v41": [_P, _I64, _I32, _I32, _P, _I32, _P],
    "mzk_topk_rows": [_P, _I64, _I64, _I64, _I32, _P, _I64, _P],
    "mzk_topk_workspace_bytes": [_I64, _I64, ctypes.POINTER(_I64)],
    "mzk_topk_rows_ws": [_P, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _P],
    "mzk_candidate_blocks_workspace_bytes": [_I64, _I64, _I32, _I32, ctypes.POINTER(_I64)],
    "mzk_candidate_blocks": [_P, _I64, _I64, _I64, _P, _I32, _I32, _P, _I64, _P, _P, _I64, _P],
    "mzk_indexer_candidate_scores_fp8": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64,
                                         _I32, _I32, _P, _I64, _P],
    "mzk_indexer_candidate_scores_mxfp4": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P,
                                           _I64, _I32, _I32, _P, _I64, _P],
    "mzk_candidate_positions": [_P, _I64, _I32, _I64, _P, _I64, _I32, _I32, _P, _I64, _P],
    "mzk_candidate_topk": [_P, _I64, _I64, _I64, _I32, _P, _I64, _I32, _I32, _P, _I64, _P],
    "mzk_indexer_scores_fp8": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P],
    "mzk_indexer_decode_fp8": [_P, _P, _P, _P, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P, _P, _P, _I32, _I32,
                               _P, _I64, _I32, _P],
    "mzk_indexer_decode_mxfp4": [_P, _P, _P, _P, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P, _P, _P, _I32,
                                 _I32, _P, _I64, _I32, _P],
    "mzk_indexer_scores_mxfp4": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P],
    "mzk_indexer_scores_bf16": [_P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P],
    "mzk_compress": [_P, _P, _I64, _I64, _I32, _I32, _I64, _P, _I32, _F32, _P, _I32, _P],
    "mzk_rope": [_P, _I32, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P],
    "mzk_sparse_mqa": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _I32, _P, _I64, _I32, _I32, _P,
                       _I64, _I64, _P, _I64, _I32, _P, _I32, _P, _I64, _P, _P, _P],
    "mzk_sparse_mqa_combine": [_P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P, _P],
    "mzk_sparse_mqa_workspace_bytes": [_I64, _I32, _I32, _I32, ctypes.POINTER(_I64)],
    "mzk_sparse_mqa_set_merge": [_I32],
    "mzk_sparse_mqa_rope": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _I32, _P, _I64, _I32, _I32,
                            _P, _I64, _I64, _P, _I64, _I32, _P, _I32, _P, _I64, _P, _P, _P, _P, _I32, _P],
    "mzk_sparse_mqa_advance": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _I32, _P, _I64, _I32,
                               _I32, _P, _I64, _I64, _P, _I64, _I32, _P, _I32, _P, _I64, _P, _P, _P, _P, _I32, _P],
    "mzk_sparse_mqa_select": [_P, _I64, _I32, _I32, _I32, _I32, _P, _I32, _P, _I64, _I32, _I32, _P, _I64, _I32, _I32,
                              _P, _I64, _I64, _P, _I64, _I32, _P, _I64, _P, _I32, _P, _I64, _P, _P, _P, _P, _I32, _P],
    "mzk_sparse_mqa_part": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _I32, _P, _I64, _I32, _I32,
                            _P, _I64, _I64, _P, _I64, _I32, _I32, _I32, _I32, _P, _I64, _P, _P, _I32, _P],
    "mzk_sparse_mqa_combine_rope": [_P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P, _I32, _P, _P, _P],
    "mzk_rms_norm": [_P, _I32, _I64, _I32, _I64, _P, _I32, _F32, _P, _I32, _P],
    "mzk_topk_bias": [_P, _I64, _I32, _I64, _I64, _P, _I64, _P],
    "mzk_mask_to_indices": [_P, _I32, _I64, _I64, _I64, _I32, _P, _P, _P, _P],
    "mzk_decode_emit": [_P, _I64, _P, _P, _P, _P, _I32, _P, _F32, _P, _I64, _I64, _P, _P, _F32, _I32, _P, _P, _I64, _P,
                        _I64, _P, _P, _P, _P, _F32, _P, _I64, _I32, _P, _I32, _P, _P, _P],
    "mzk_decode_emit_scores": [_P, _I64, _P, _P, _P, _P, _I32, _P, _F32, _P, _I64, _I64, _P, _P, _F32, _I32, _P, _P, _I64,
                               _P, _I64, _P, _P, _P, _P, _F32, _P, _I64, _I32, _P, _P, _I32, _I64, _P, _I64,
                               _P, _P, _P, _P, _I32, _P, _F32, _P, _I64, _I64, _P, _P],
    "mzk_decode_emit_pair": [_P, _I64, _P, _P, _P, _P, _I32, _P, _F32, _P, _I64, _I64, _P, _P, _F32, _I32, _P, _P, _I64, _P, _I64, _P, _P, _P, _P, _F32, _P, _I64, _I32, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _P, _F32, _P, _I64, _I64, _P],
    "mzk_sparse_mqa_noalloc": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _I32, _P, _I64, _I32, _I32,
                               _P, _I64, _I64, _P, _I64, _I32, _P, _I32, _P, _P, _P, _P, _I32, _P],
    "mzk_indexer_decode_fused": [_I32, _P, _P, _P, _P, _I64, _I32, _I32, _I64, _I64, _P, _I32, _P, _I64, _P, _P, _P,
                                 _P, _I32, _P, _P, _F32, _P, _P, _I32, _I32, _P, _I64, _I32, _P],
}
_RESTYPE = {"mzk_last_error": ctypes.c_char_p}

_lib = None


class MzkError(RuntimeError):
    """A C-ABI call returned a negative status."""


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(mzk_[a-z0-9_]+)\s*\(", text)))


def load(path: pathlib.Path | None = None) -> ctypes.CDLL:
    """Load the library (once) and attach the signatures.  Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path or LIB_PATH)
    if not p.exists():
        raise ImportError(f"mzoo_amd HIP library not built: {p} is missing "
                          f"(run `python -m mzoo_amd.build`); there is no CPU fallback")
    lib = ctypes.CDLL(str(p))
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    if path is None:
        _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise ``MzkError`` on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mzk_last_error().decode()
        raise MzkError(f"{name} failed ({rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype} (float32, bfloat16, float16)") from None


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("mzoo_amd runs on the GPU only: got a tensor on " + str(t.device))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream
