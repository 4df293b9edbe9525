"""CPU restatement of the reference's block quantizers (test infrastructure only).

Follows ``src/mzoo/archs/owlet1/quant.py`` (identical to
``src/mzoo/archs/dsv4/modeling_deepseek_v41.py:343-402``):

* ``pow2_ceil_scale``      -- ``_pow2_ceil_scale``        quant.py:23-31
* ``e2m1_codes``           -- ``_e2m1_codes``             quant.py:34-46
* ``fake_quant_fp4_block`` -- ``_fake_quant_fp4_block``   quant.py:49-66
* ``fake_quant_fp8_block`` -- ``_fake_quant_fp8_block``   quant.py:72-86

plus the cast the reference borrows from torch, ``Tensor.to(torch.float8_e4m3fn)``
(OCP e4m3fn: bias 7, no infinities, max 448, subnormals down to 2^-9,
round-to-nearest-even), restated as integer arithmetic in ``e4m3_encode``.

Packed formats (the reference only ever fake-quantizes; these layouts are the build's
cache formats, chosen to match the FlashMLA / SGLang layouts quoted in
``src/mzoo/layers/attn/fp_attn_notes.md:1085-1131``):

* FP8-b128 latent entry, 656 B: 512 e4m3 codes of the nope slice, 4 fp32 ue8m0 scales
  (one per 128 channels), 64 bf16 rope channels.
* FP8 indexer row: ``Di`` e4m3 codes + one fp32 scale per 128 channels (132 B at 128).
* MXFP4 indexer row: e2m1 codes packed two per byte (element ``2i`` in the low nibble)
  + one e8m0 byte per 32 channels (``2^(byte-127)``); 68 B at 128.

All arithmetic is numpy float32 / integer, so every result is reproducible bit for bit.
Inputs are float32 arrays; ``dtype`` names the tensor dtype the reference would have
been called with (its outputs are cast back with ``.to(x.dtype)``).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
FP4_MAX = F32(6.0)
FP8_MAX = F32(448.0)
# quant.py:8-11 -- the e2m1 value table indexed by the 4-bit code (bit 3 = sign).
# Code 8 decodes to +0.0 (not -0.0), which the product must reproduce.
FP4_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=F32)


def f32_bits(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=F32).view(np.uint32)


def bits_f32(b) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint32).view(F32)


# ---------------------------------------------------------------------------------------
# dtype rounding (what ``.to(x.dtype)`` does at the end of every reference quantizer)
# ---------------------------------------------------------------------------------------

def round_bf16(x) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even), returned as float32 values; NaN stays NaN."""
    b = f32_bits(x).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    out = bits_f32(rounded.astype(np.uint32))
    return np.where(np.isnan(x), np.asarray(x, F32), out)


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of ``round_bf16(x)``."""
    return (f32_bits(round_bf16(x)) >> 16).astype(np.uint16)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return np.asarray(x, F32)
    if dtype == "bfloat16":
        return round_bf16(x)
    if dtype == "float16":
        return np.asarray(x, F32).astype(np.float16).astype(F32)
    raise ValueError(f"unsupported dtype {dtype!r}")


# ---------------------------------------------------------------------------------------
# scalar codecs
# ---------------------------------------------------------------------------------------

def pow2_ceil_scale(t) -> np.ndarray:
    """quant.py:23-31: ``2^(E - 127 + (M != 0))`` from the fp32 exponent field E and
    mantissa field M of ``t`` -- the ue8m0 (power-of-two, rounded up) scale."""
    b = f32_bits(t).astype(np.int64)
    k = ((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFF) != 0)
    return np.ldexp(np.ones_like(k, dtype=F32), k.astype(np.int32)).astype(F32)


_E2M1_BOUNDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=F32)
_E2M1_TIES_UP = np.array([False, True, False, True, False, True, False])
# quant.py:40-44: at an even-code midpoint an exact tie must round down, so the
# threshold moves one ulp up; at an odd-code midpoint the tie rounds up.
_E2M1_THRESH = np.where(_E2M1_TIES_UP, _E2M1_BOUNDS,
                        np.nextafter(_E2M1_BOUNDS, np.full_like(_E2M1_BOUNDS, np.inf)))


def e2m1_codes(q) -> np.ndarray:
    """quant.py:34-46: code = number of thresholds ``<= |q|``; sign bit 3 from
    ``signbit`` (so -0.0 gives code 8).  ``q`` is pre-clamped to [-6, 6]."""
    q = np.asarray(q, F32)
    mag = np.abs(q)
    codes = (mag[..., None] >= _E2M1_THRESH).sum(-1).astype(np.uint8)
    return codes | (np.signbit(q).astype(np.uint8) << 3)


def e4m3_encode(x) -> np.ndarray:
    """``float -> float8_e4m3fn`` code (uint8): round to nearest, ties to even; values at
    or above 480 in magnitude (the first that would round past 448) become NaN (0x7F
    with the sign); subnormals are multiples of 2^-9; the sign of zero is kept."""
    x = np.asarray(x, F32)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    out = np.zeros(a.shape, np.uint8)
    # normal range [2^-6, 480): round the fp32 mantissa to 3 bits (ties to even)
    b = f32_bits(a).astype(np.int64)
    keep = (b >> 20) & 1
    r = (b + 0x7FFFF + keep) >> 20                  # exponent:mantissa, 3-bit mantissa
    exp = (r >> 3) - 127 + 7                        # e4m3 biased exponent
    normal_code = ((exp << 3) | (r & 7)).astype(np.int64)
    is_normal = a >= F32(2.0 ** -6)
    # subnormal range: multiples of 2^-9, nearest even (np.rint is half-to-even);
    # a * 2^9 is exact, and rint(...) == 8 is the smallest normal (code 0x08)
    sub_code = np.rint(a.astype(np.float64) * 512.0).astype(np.int64)
    code = np.where(is_normal, normal_code, sub_code)
    nan = (a >= F32(480.0)) | np.isnan(a)
    code = np.where(nan, 0x7F, code)
    out[...] = code.astype(np.uint8)
    return out | sign


def e4m3_decode(codes) -> np.ndarray:
    c = np.asarray(codes, np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return (s * mag).astype(F32)


def e8m0_from_pow2(scale) -> np.ndarray:
    """Power-of-two fp32 scale -> e8m0 byte (``2^(byte - 127)``)."""
    b = f32_bits(scale).astype(np.int64)
    e = (b >> 23) & 0xFF
    if np.any((b & 0x7FFFFF) != 0) or np.any(e == 0):
        raise ValueError("e8m0 needs a normal power-of-two scale")
    return e.astype(np.uint8)


def e8m0_decode(byte) -> np.ndarray:
    return np.ldexp(np.ones(np.shape(byte), F32), np.asarray(byte, np.int32) - 127).astype(F32)


# ---------------------------------------------------------------------------------------
# block quantizers (value-level round trips, as the reference defines them)
# ---------------------------------------------------------------------------------------

def _blocks(x, block_size):
    x = np.asarray(x, F32)
    n = x.shape[-1]
    return x.reshape(*x.shape[:-1], n // block_size, block_size)


def fp8_block_scales(x, block_size: int) -> np.ndarray:
    """quant.py:81-83: ``pow2ceil(max(amax, 1e-4) * fp32(1/448))`` per block."""
    amax = np.maximum(np.abs(_blocks(x, block_size)).max(-1), F32(1e-4))
    return pow2_ceil_scale(amax * F32(1.0 / 448.0))


def fp8_block_codes(x, block_size: int):
    """(codes uint8 [..., n], scales fp32 [..., n/bs]) of ``_fake_quant_fp8_block``."""
    blocks = _blocks(x, block_size)
    scale = fp8_block_scales(x, block_size)
    q = np.clip(blocks / scale[..., None], -FP8_MAX, FP8_MAX)     # quant.py:84
    codes = e4m3_encode(q)
    return codes.reshape(*codes.shape[:-2], -1), scale


def fake_quant_fp8_block(x, block_size: int = 32, dtype: str = "float32"):
    """quant.py:72-86.  Pass-through (returns ``x`` itself) when ``n % block_size``."""
    x = np.asarray(x, F32)
    n = x.shape[-1]
    if n % block_size:
        return x
    codes, scale = fp8_block_codes(x, block_size)
    deq = e4m3_decode(codes).reshape(*x.shape[:-1], n // block_size, block_size) * scale[..., None]
    return round_to(deq.reshape(x.shape), dtype)


def fp4_block_scales(x, block_size: int, e4m3_scales: bool = False) -> np.ndarray:
    """quant.py:58-62: ue8m0 ``pow2ceil(max(amax, 6*2^-126) * fp32(1/6))`` or e4m3
    ``e4m3(max(amax, 6*2^-9) / 6)``."""
    amax = np.abs(_blocks(x, block_size)).max(-1)
    if e4m3_scales:
        return e4m3_decode(e4m3_encode(np.maximum(amax, F32(6.0 * 2.0 ** -9)) / FP4_MAX))
    return pow2_ceil_scale(np.maximum(amax, F32(6.0 * 2.0 ** -126)) * F32(1.0 / 6.0))


def fp4_block_codes(x, block_size: int, e4m3_scales: bool = False):
    """(codes uint8 [..., n] one code per byte, scales fp32 [..., n/bs])."""
    blocks = _blocks(x, block_size)
    scale = fp4_block_scales(x, block_size, e4m3_scales)
    q = np.clip(blocks / scale[..., None], -FP4_MAX, FP4_MAX)    # quant.py:63
    codes = e2m1_codes(q)
    return codes.reshape(*codes.shape[:-2], -1), scale


def fake_quant_fp4_block(x, block_size: int, e4m3_scales: bool = False, dtype: str = "float32"):
    """quant.py:49-66.  Pass-through when ``n % block_size``."""
    x = np.asarray(x, F32)
    n = x.shape[-1]
    if n % block_size:
        return x
    codes, scale = fp4_block_codes(x, block_size, e4m3_scales)
    vals = FP4_TABLE[codes.astype(np.int64)].reshape(*x.shape[:-1], n // block_size, block_size)
    return round_to((vals * scale[..., None]).reshape(x.shape), dtype)


# ---------------------------------------------------------------------------------------
# packed formats
# ---------------------------------------------------------------------------------------

LATENT_NOPE = 512
LATENT_ROPE = 64
ENTRY_BYTES = LATENT_NOPE + 4 * (LATENT_NOPE // 128) + 2 * LATENT_ROPE   # 656


def pack_latent_fp8_b128(x, nope: int = LATENT_NOPE) -> np.ndarray:
    """[..., nope+rope] float32 -> [..., nope + 4*nope/128 + 2*rope] uint8: e4m3 codes
    of ``_fake_quant_fp8_block(x[..., :nope], 128)``, their fp32 scales, then the rope
    slice as bf16 (round to nearest even)."""
    x = np.asarray(x, F32)
    codes, scales = fp8_block_codes(x[..., :nope], 128)
    rope = bf16_bits(x[..., nope:]).view(np.uint8).reshape(*x.shape[:-1], -1)
    return np.concatenate([codes, scales.astype("<f4").view(np.uint8).reshape(*x.shape[:-1], -1), rope], -1)


def unpack_latent_fp8_b128(entries, nope: int = LATENT_NOPE, rope: int = LATENT_ROPE) -> np.ndarray:
    """Inverse of ``pack_latent_fp8_b128``: the dequantized float32 latent."""
    e = np.ascontiguousarray(entries, np.uint8)
    nb = nope // 128
    codes = e[..., :nope]
    scales = e[..., nope:nope + 4 * nb].copy().view("<f4").astype(F32)
    rbits = e[..., nope + 4 * nb:nope + 4 * nb + 2 * rope].copy().view("<u2").astype(np.uint32) << 16
    deq = e4m3_decode(codes).reshape(*e.shape[:-1], nb, 128) * scales[..., None]
    return np.concatenate([deq.reshape(*e.shape[:-1], nope), bits_f32(rbits)], -1)


def quant_mxfp4(x):
    """MXFP4 of ``_fake_quant_fp4_block(x, 32)``: (packed codes uint8 [..., n/2] with
    element 2i in the low nibble, e8m0 scale bytes uint8 [..., n/32])."""
    codes, scale = fp4_block_codes(x, 32)
    packed = (codes[..., 0::2] & 0xF) | ((codes[..., 1::2] & 0xF) << 4)
    return packed.astype(np.uint8), e8m0_from_pow2(scale)


def dequant_mxfp4(packed, e8m0) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    codes = np.stack([p & 0xF, p >> 4], -1).reshape(*p.shape[:-1], -1)
    vals = FP4_TABLE[codes.astype(np.int64)]
    scale = e8m0_decode(e8m0)
    return (vals.reshape(*vals.shape[:-1], -1, 32) * scale[..., None]).reshape(vals.shape)


def dequant_fp8_block(codes, scales, block_size: int) -> np.ndarray:
    c = np.asarray(codes, np.uint8)
    v = e4m3_decode(c).reshape(*c.shape[:-1], -1, block_size) * np.asarray(scales, F32)[..., None]
    return v.reshape(c.shape)


def pack_cache_v41(x, fmt: str) -> np.ndarray:
    """DeepSeek-V4.1 cache entries (FlashMLA ``kv_cache_format`` rows "V4.1" / "V4.1 fp4",
    ``layers/attn/fp_attn_notes.md:1123-1131``) of x [..., D]: "fp8" = the e4m3 codes of
    ``_fake_quant_fp8_block(x, 32)`` then their e8m0 scale bytes; "fp4" = the e2m1 codes of
    ``_fake_quant_fp4_block(x, 16, e4m3_scales=True)`` two per byte (element 2i low) then
    their e4m3 scale bytes."""
    x = np.asarray(x, F32)
    lead = x.shape[:-1]
    if fmt == "fp8":
        codes, scales = fp8_block_codes(x, 32)
        return np.concatenate([codes.astype(np.uint8), e8m0_from_pow2(scales).reshape(*lead, -1)], -1)
    codes, scales = fp4_block_codes(x, 16, e4m3_scales=True)
    packed = ((codes[..., 0::2] & 0xF) | ((codes[..., 1::2] & 0xF) << 4)).astype(np.uint8)
    return np.concatenate([packed, e4m3_encode(scales).astype(np.uint8).reshape(*lead, -1)], -1)
