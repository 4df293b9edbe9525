"""Drop-in block quantizers on the GPU (piece 1).

Same names, signatures, dtype/shape contract and pass-through behaviour as the
reference's ``src/mzoo/archs/owlet1/quant.py``:

* ``_fake_quant_fp8_block(x, block_size=32)``  -- quant.py:72-86
* ``_fake_quant_fp4_block(x, block_size, e4m3_scales=False)`` -- quant.py:49-66

both out of place, returning ``x.dtype`` / ``x.shape``, and returning ``x`` itself
(unquantized) when ``x.shape[-1] % block_size``.  Packed forms for the caches:

* ``quant_fp8_block`` / ``dequant_fp8_block``  -- e4m3 codes + fp32 pow2 scales
* ``quant_mxfp4`` / ``dequant_mxfp4``          -- e2m1 nibbles + e8m0 bytes (block 32)
* ``pack_latent_fp8_b128`` / ``unpack_latent_fp8_b128`` -- the 656 B latent entry
"""

from __future__ import annotations

import torch

from . import _lib

ENTRY_NOPE = 512
ENTRY_ROPE = 64


def entry_bytes(nope: int = ENTRY_NOPE, rope: int = ENTRY_ROPE) -> int:
    return nope + 4 * (nope // 128) + 2 * rope


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.shape[-1] else 0


def _fake_quant_fp8_block(x: torch.Tensor, block_size: int = 32) -> torch.Tensor:
    """owlet1/quant.py:72-86 on the GPU: ue8m0 (pow2, rounded up) scale per block of
    ``block_size`` channels, e4m3 round trip, out of place, ``x.dtype`` out."""
    n = x.shape[-1]
    if n % block_size:
        return x
    _lib.require_gpu(x)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    _lib.call("mzk_fake_quant_fp8_block", xc.data_ptr(), y.data_ptr(), _lib.dtype_code(x.dtype), _rows(xc), n,
              block_size, _lib.stream_of(x))
    return y.view(x.shape)


def _fake_quant_fp4_block(x: torch.Tensor, block_size: int, e4m3_scales: bool = False) -> torch.Tensor:
    """owlet1/quant.py:49-66 on the GPU: e2m1 round trip with ue8m0 (default) or e4m3
    block scales, out of place, ``x.dtype`` out."""
    n = x.shape[-1]
    if n % block_size:
        return x
    _lib.require_gpu(x)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    _lib.call("mzk_fake_quant_fp4_block", xc.data_ptr(), y.data_ptr(), _lib.dtype_code(x.dtype), _rows(xc), n,
              block_size, int(bool(e4m3_scales)), _lib.stream_of(x))
    return y.view(x.shape)


def quant_fp8_block(x: torch.Tensor, block_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """x [..., n] -> (codes uint8 [..., n], scales fp32 [..., n/block_size])."""
    _lib.require_gpu(x)
    n = x.shape[-1]
    if n % block_size:
        raise ValueError(f"quant_fp8_block: n={n} is not a multiple of block_size={block_size}")
    xc = x.contiguous()
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(*x.shape[:-1], n // block_size, dtype=torch.float32, device=x.device)
    _lib.call("mzk_quant_fp8_block", xc.data_ptr(), _lib.dtype_code(x.dtype), _rows(xc), n, block_size,
              codes.data_ptr(), scales.data_ptr(), _lib.stream_of(x))
    return codes, scales


def dequant_fp8_block(codes: torch.Tensor, scales: torch.Tensor, block_size: int = 128,
                      dtype: torch.dtype = torch.float32) -> torch.Tensor:
    _lib.require_gpu(codes, scales)
    c = codes.contiguous()
    s = scales.contiguous().float()
    y = torch.empty(c.shape, dtype=dtype, device=c.device)
    _lib.call("mzk_dequant_fp8_block", c.data_ptr(), s.data_ptr(), _rows(c), c.shape[-1], block_size, y.data_ptr(),
              _lib.dtype_code(dtype), _lib.stream_of(c))
    return y


def quant_mxfp4(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [..., n] -> (packed uint8 [..., n/2], e8m0 uint8 [..., n/32]) of
    ``_fake_quant_fp4_block(x, 32)``."""
    _lib.require_gpu(x)
    n = x.shape[-1]
    if n % 32:
        raise ValueError(f"quant_mxfp4: n={n} is not a multiple of 32")
    xc = x.contiguous()
    packed = torch.empty(*x.shape[:-1], n // 2, dtype=torch.uint8, device=x.device)
    e8m0 = torch.empty(*x.shape[:-1], n // 32, dtype=torch.uint8, device=x.device)
    _lib.call("mzk_quant_mxfp4", xc.data_ptr(), _lib.dtype_code(x.dtype), _rows(xc), n, packed.data_ptr(),
              e8m0.data_ptr(), _lib.stream_of(x))
    return packed, e8m0


def dequant_mxfp4(packed: torch.Tensor, e8m0: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    _lib.require_gpu(packed, e8m0)
    p = packed.contiguous()
    e = e8m0.contiguous()
    n = p.shape[-1] * 2
    y = torch.empty(*p.shape[:-1], n, dtype=dtype, device=p.device)
    _lib.call("mzk_dequant_mxfp4", p.data_ptr(), e.data_ptr(), _rows(y), n, y.data_ptr(), _lib.dtype_code(dtype),
              _lib.stream_of(p))
    return y


def pack_latent_fp8_b128(x: torch.Tensor, rope: int = ENTRY_ROPE, out: torch.Tensor | None = None,
                         dst_index: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., nope+rope] -> FP8-b128 entries uint8 [..., entry_bytes].  With ``out`` (a
    cache viewed as [entries, entry_bytes]) and ``dst_index`` (int64 [rows]) the rows are
    written into those cache entries instead."""
    _lib.require_gpu(x)
    d = x.shape[-1]
    nope = d - rope
    xc = x.contiguous()
    rows = _rows(xc)
    eb = entry_bytes(nope, rope)
    if out is None:
        out = torch.empty(*x.shape[:-1], eb, dtype=torch.uint8, device=x.device)
    if out.dtype != torch.uint8 or out.shape[-1] != eb or not out.is_contiguous():
        raise ValueError(f"pack_latent_fp8_b128: out must be contiguous uint8 [..., {eb}]")
    if dst_index is not None:
        dst_index = dst_index.to(device=x.device, dtype=torch.int64).contiguous()
        if dst_index.numel() != rows:
            raise ValueError("pack_latent_fp8_b128: dst_index needs one entry per row")
    elif out.numel() // eb < rows:
        raise ValueError("pack_latent_fp8_b128: out holds fewer entries than x has rows")
    _lib.call("mzk_pack_latent_fp8_b128", xc.data_ptr(), _lib.dtype_code(x.dtype), rows, nope, rope,
              _lib.ptr(dst_index), out.data_ptr(), _lib.stream_of(x))
    return out


def unpack_latent_fp8_b128(entries: torch.Tensor, nope: int = ENTRY_NOPE, rope: int = ENTRY_ROPE,
                           dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    _lib.require_gpu(entries)
    e = entries.contiguous()
    rows = _rows(e)
    y = torch.empty(*e.shape[:-1], nope + rope, dtype=dtype, device=e.device)
    _lib.call("mzk_unpack_latent_fp8_b128", e.data_ptr(), rows, nope, rope, y.data_ptr(), _lib.dtype_code(dtype),
              _lib.stream_of(e))
    return y


# ---- DeepSeek-V4.1 cache entries (FlashMLA kv_cache_format) -------------------------------
V41_FORMATS = {"fp8": 0, "fp4": 1}


def v41_entry_bytes(d: int, fmt: str) -> int:
    """Bytes of one V4.1 cache entry of D channels: fp8 D + D/32 (528 at D=512), fp4
    D/2 + D/16 (288 at D=512)."""
    return d + d // 32 if fmt == "fp8" else d // 2 + d // 16


def pack_cache_v41(x: torch.Tensor, fmt: str, out: torch.Tensor | None = None,
                   dst_index: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., D] -> V4.1 entries uint8 [..., v41_entry_bytes(D, fmt)]: ``fmt`` "fp8" is
    ``_fake_quant_fp8_block(x, 32)`` (owlet1/quant.py:72-86) stored as e4m3 codes then e8m0
    scales, "fp4" is ``_fake_quant_fp4_block(x, 16, e4m3_scales=True)`` (quant.py:49-66)
    stored as e2m1 nibbles then e4m3 scales.  With ``out`` (a cache viewed as [entries,
    bytes]) and ``dst_index`` (int64 [rows]) the rows go to those entries."""
    if fmt not in V41_FORMATS:
        raise ValueError(f"pack_cache_v41: fmt must be 'fp8' or 'fp4', got {fmt!r}")
    _lib.require_gpu(x)
    d = x.shape[-1]
    if d % 32:
        raise ValueError(f"pack_cache_v41: D must be a multiple of 32, got {d}")
    xc = x.contiguous()
    rows = _rows(xc)
    eb = v41_entry_bytes(d, fmt)
    if out is None:
        out = torch.empty(*x.shape[:-1], eb, dtype=torch.uint8, device=x.device)
    if out.dtype != torch.uint8 or out.shape[-1] != eb or not out.is_contiguous():
        raise ValueError(f"pack_cache_v41: out must be contiguous uint8 [..., {eb}]")
    if dst_index is not None:
        dst_index = dst_index.to(device=x.device, dtype=torch.int64).contiguous()
        if dst_index.numel() != rows:
            raise ValueError("pack_cache_v41: dst_index needs one entry per row")
    elif out.numel() // eb < rows:
        raise ValueError("pack_cache_v41: out holds fewer entries than x has rows")
    _lib.call("mzk_pack_cache_v41", xc.data_ptr(), _lib.dtype_code(x.dtype), rows, d, V41_FORMATS[fmt],
              out.data_ptr(), _lib.ptr(dst_index), _lib.stream_of(x))
    return out


def unpack_cache_v41(entries: torch.Tensor, d: int, fmt: str, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """V4.1 entries uint8 [..., bytes] -> the fake-quantized values [..., D]."""
    if fmt not in V41_FORMATS:
        raise ValueError(f"unpack_cache_v41: fmt must be 'fp8' or 'fp4', got {fmt!r}")
    _lib.require_gpu(entries)
    e = entries.contiguous()
    if e.shape[-1] != v41_entry_bytes(d, fmt):
        raise ValueError(f"unpack_cache_v41: entries of {v41_entry_bytes(d, fmt)} bytes expected")
    rows = _rows(e)
    y = torch.empty(*e.shape[:-1], d, dtype=dtype, device=e.device)
    _lib.call("mzk_unpack_cache_v41", e.data_ptr(), rows, d, V41_FORMATS[fmt], y.data_ptr(), _lib.dtype_code(dtype),
              _lib.stream_of(e))
    return y
