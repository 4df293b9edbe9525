"""CPU restatement of the KV compressor and its RMSNorm / RoPE (test infrastructure only).

Follows
* ``DeepseekV41Compressor.forward``  ``src/mzoo/archs/owlet1/cache.py:142-172``
  (``latent = sum_r kv * softmax_r(gate)`` in fp32, ``.to(dtype)``, then ``self.norm``;
  ratio 1: ``norm(kv)``),
* ``DeepseekV41RMSNorm.forward``     ``owlet1/norm_rope.py:25-30``
  (``h * rsqrt(mean(h^2) + eps)``, ``.to(dtype)``, ``weight * h``),
* ``apply_rotary_pos_emb``           ``owlet1/norm_rope.py:126-145``
  (interleaved (even, odd) pairs on the trailing rope slice, fp32 math, ``inverse``
  negates ``sin``),
* ``DeepseekV41CSACache.store_compression_weights`` ``owlet1/cache.py:96-113``
  (group alignment and the partial-group carry, as ``split_groups``),
* the decode prologue of the new token's latent ``owlet1/attention.py:150-151``
  (``rope(kv_norm(kv))``, as ``decode_kv_latent``: a composition of the two above).

The reference evaluates ``softmax`` / ``mean`` with torch, whose exp and reduction order
are implementation-defined (they differ between torch's CPU and GPU builds in the last
bits).  To make "bit-exact" a checkable statement this restatement fixes both, and the
HIP kernel evaluates the same sequence of IEEE float32 operations:

* ``exp_f32``: Cody-Waite reduction ``x = n*ln2 + r`` (``n = rint(x*log2e)``, ln2 split
  into a 16-bit head and a tail), degree-7 Taylor polynomial in Horner form, scaling by
  ``2^n`` through the exponent field (two steps below 2^-126).  No fused multiply-add.
* softmax over ``r``: max, ``exp(g_r - max)``, sequential sum from 0, divide.
* pooled sum over ``r``: sequential from 0, ``kv_r * p_r`` per term.
* RMSNorm sum of squares: 64 partial sums (partial ``l`` takes channels ``l, l+64, ...``
  in order, starting from 0), then combined by the xor butterfly
  ``p[l] += p[l ^ m]`` for ``m = 32, 16, 8, 4, 2, 1``; ``var = sum / D``;
  ``rsqrt(v) = 1 / sqrt(v)`` (two correctly rounded operations).

``tests/test_oracle_compressor.py`` pins this restatement against torch's own softmax and
RMSNorm to a few ulp, and the kernel against this restatement bit for bit.
"""

from __future__ import annotations

import numpy as np

from .quant import round_to

F32 = np.float32
_LOG2E = F32(1.44269504088896341)
_LN2_HI = F32(0.693145751953125)        # 0x3F317200: 16 significant bits, n*_LN2_HI exact
_LN2_LO = F32(1.42860682030941723e-06)  # ln2 - _LN2_HI
_INV_FACT = [F32(1.0 / f) for f in (1, 1, 2, 6, 24, 120, 720, 5040)]


def _pow2(n: np.ndarray) -> np.ndarray:
    """2^n for integer n in [-126, 127] as float32 via the exponent field."""
    return ((n.astype(np.int64) + 127) << 23).astype(np.uint32).view(F32)


def exp_f32(x) -> np.ndarray:
    """Deterministic float32 exp (see module docstring).  Max error ~2 ulp."""
    x = np.asarray(x, F32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = np.rint(x * _LOG2E)
        n = np.clip(n, F32(-160), F32(160))
        r = (x - n * _LN2_HI) - n * _LN2_LO
        p = _INV_FACT[7]
        for c in _INV_FACT[6::-1]:
            p = p * r + c
        ni = n.astype(np.int64)
        hi = _pow2(np.clip(ni, -126, 127))
        out = p * hi
        # below 2^-126: scale by 2^(n+64) (normal, exact) then by 2^-64 (one rounding)
        small = ni < -126
        if np.any(small):
            lo = p * _pow2(np.clip(ni + 64, -126, 127)) * F32(2.0 ** -64)
            out = np.where(small, lo, out)
        out = np.where(x < F32(-104.0), F32(0.0), out)
        out = np.where(x > F32(88.8), F32(np.inf), out)
        out = np.where(np.isnan(x), x, out)
    return out.astype(F32)


def softmax_pool(kv, gate) -> np.ndarray:
    """cache.py:168-172 without the norm: kv/gate [..., r, D] fp32 -> [..., D] fp32."""
    kv = np.asarray(kv, F32)
    gate = np.asarray(gate, F32)
    r = gate.shape[-2]
    m = gate[..., 0, :]
    for i in range(1, r):
        m = np.maximum(m, gate[..., i, :])
    e = [exp_f32(gate[..., i, :] - m) for i in range(r)]
    s = np.zeros_like(m)
    for i in range(r):
        s = s + e[i]
    acc = np.zeros_like(m)
    for i in range(r):
        acc = acc + kv[..., i, :] * (e[i] / s)
    return acc.astype(F32)


def sum_sq_butterfly(h) -> np.ndarray:
    """Sum of squares over the last axis in the pinned 64-partial / xor-butterfly order."""
    h = np.asarray(h, F32)
    d = h.shape[-1]
    sq = h * h
    parts = np.zeros((64,) + h.shape[:-1], F32)
    for lane in range(64):
        acc = np.zeros(h.shape[:-1], F32)
        for c in range(lane, d, 64):
            acc = acc + sq[..., c]
        parts[lane] = acc
    m = 32
    while m >= 1:
        parts = parts + parts[np.arange(64) ^ m]
        m //= 2
    return parts[0]


def rms_norm(x, weight, eps: float, dtype: str) -> np.ndarray:
    """norm_rope.py:25-30.  ``x`` float32 values already representable in ``dtype``."""
    h = np.asarray(x, F32)
    var = sum_sq_butterfly(h) / F32(h.shape[-1])
    inv = F32(1.0) / np.sqrt(var + F32(eps))
    normed = round_to(h * inv[..., None], dtype)
    return round_to(np.asarray(weight, F32) * normed, dtype)


def compress(kv, gate, ratio: int, weight, eps: float, dtype: str) -> np.ndarray:
    """cache.py:157-172 on group-aligned input.  kv/gate [B, n*ratio, D] fp32 (the fp32
    projections), returns the normed pre-RoPE latent [B, n, D] as float32 values of ``dtype``.
    Ratio 1 (``gate`` None): ``norm(kv)`` with ``kv`` already in ``dtype``."""
    kv = np.asarray(kv, F32)
    if ratio == 1:
        return rms_norm(round_to(kv, dtype), weight, eps, dtype)
    b, t, d = kv.shape
    n = t // ratio
    pooled = softmax_pool(kv[:, :n * ratio].reshape(b, n, ratio, d),
                          np.asarray(gate, F32)[:, :n * ratio].reshape(b, n, ratio, d))
    return rms_norm(round_to(pooled, dtype), weight, eps, dtype)


def split_groups(buffered: int, new_tokens: int, ratio: int):
    """cache.py:96-113: with ``buffered`` tokens carried from earlier calls and
    ``new_tokens`` arriving, return (tokens consumed into complete groups, tokens left
    buffered)."""
    total = buffered + new_tokens
    usable = (total // ratio) * ratio
    return usable, total - usable


def rope(x, cos, sin, inverse: bool = False, dtype: str = "float32") -> np.ndarray:
    """norm_rope.py:126-145: x [..., D] with the rope slice the trailing ``2*len(cos)``
    channels; cos/sin [..., rd/2] broadcast over x's leading axes (heads included)."""
    x = np.asarray(x, F32)
    cos = np.asarray(cos, F32)
    sin = np.asarray(sin, F32)
    if inverse:
        sin = -sin
    rd = cos.shape[-1] * 2
    nope, r = x[..., :-rd], x[..., -rd:]
    even, odd = r[..., 0::2], r[..., 1::2]
    out = np.empty_like(r)
    out[..., 0::2] = even * cos - odd * sin
    out[..., 1::2] = even * sin + odd * cos
    return np.concatenate([nope, round_to(out, dtype)], -1)


def decode_kv_latent(kv, weight, eps: float, cos, sin, dtype: str = "bfloat16") -> np.ndarray:
    """The new token's window latent, ``owlet1/attention.py:150-151``:
    ``apply_rotary_pos_emb(kv_norm(wkv(x)), cos, sin)`` on the projection ``kv`` [..., D]
    (values of ``dtype``) with cos/sin [..., rd/2]; the result is what the window cache
    stores before its FP8 packing."""
    return rope(rms_norm(kv, weight, eps, dtype), cos, sin, dtype=dtype)


def rope_tables(positions, rope_dim: int, theta: float):
    """``compute_default_rope_parameters`` (dsv4 modeling_deepseek_v41.py:127-137) and
    ``DeepseekV41RotaryEmbedding.forward`` (norm_rope.py:108-124) for plain (non-YaRN)
    RoPE: ``inv_freq = theta^(-2i/rd)``, cos/sin of ``pos * inv_freq`` in fp32."""
    import torch
    inv = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float) / rope_dim))
    pos = torch.as_tensor(np.asarray(positions)).float()
    freqs = pos[..., None] * inv
    return freqs.cos().numpy(), freqs.sin().numpy()


def linear_pinned(x, w, dtype: str = "bfloat16") -> np.ndarray:
    """``nn.Linear`` (no bias) of x [..., D] by w [out, D] in the order the decode-step
    emission kernel evaluates it (D a multiple of 64): the row is cut into 16-byte chunks of
    8 channels; partial j (j = 0..7) sums, in float32 from 0, chunk j, j+8, j+16, ... with its
    8 channels in order (a bf16 x bf16 product is exact in float32); the partials meet in an
    xor butterfly -- ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)) -- and the total is rounded to
    ``dtype``.  Differs from a library GEMM's order only in float32 rounding (tests bound it
    against float64)."""
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    d = x.shape[-1]
    nchunk = d // 8
    parts = []
    for j in range(8):
        a = np.zeros(x.shape[:-1] + (w.shape[0],), F32)
        for c in range(j, nchunk, 8):
            for e in range(8):
                i = 8 * c + e
                a = a + x[..., i:i + 1] * w[:, i]
        parts.append(a)
    s1 = [parts[j] + parts[j ^ 4] for j in range(8)]
    s2 = [s1[j] + s1[j ^ 2] for j in range(8)]
    total = s2[0] + s2[1]
    return round_to(total, dtype)


def emit_group(kv, gate, ratio: int, norm_w, eps: float, cos, sin, wk=None, k_norm_w=None, k_eps: float = 1e-6,
               dtype: str = "bfloat16"):
    """One compressed group as the decode step emits it: ``kv`` / ``gate`` [B, ratio, D] fp32
    (the group's compressor projections, owlet1/cache.py:155-158), ``cos`` / ``sin`` [B, rd/2]
    the compress RoPE at the group's position ``g * ratio`` (attention.py:174-180).

    Returns (rotated latent [B, D] -- what the main cache stores before its packing,
    attention.py:180 --, index key [B, Di] or None -- ``rope(k_norm(wk(latent)))`` before its
    quantization, indexer.py:96-103).  The latent is ``compress`` (pool + RMSNorm,
    cache.py:168-172); the key projection uses ``linear_pinned``."""
    latent = compress(kv, gate, ratio, norm_w, eps, dtype)[:, 0]
    rot = rope(latent, cos, sin, dtype=dtype)
    if wk is None:
        return rot, None
    k = rms_norm(linear_pinned(latent, wk, dtype), k_norm_w, k_eps, dtype)
    return rot, rope(k, cos, sin, dtype=dtype)
