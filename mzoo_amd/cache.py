"""KV compressor, RoPE and the group-carry state on the GPU (piece 2).

* ``apply_rotary_pos_emb(x, cos, sin, inverse=False)`` -- drop-in of
  ``owlet1/norm_rope.py:126-145`` (interleaved (even, odd) pairs on the trailing rope
  slice; ``cos``/``sin`` carry ``rope_dim/2`` entries, ``[B,S,rd/2]``, broadcast over the
  head axis of a ``[B,S,H,D]`` input).
* ``compress(kv, gate, ratio, norm_weight, eps, dtype)`` -- the pooling + RMSNorm of
  ``DeepseekV41Compressor.forward`` (``owlet1/cache.py:142-172``) on the fp32
  projections, one launch.
* ``GroupCarry`` -- ``DeepseekV41CSACache.store_compression_weights`` /
  ``update_compressor_states`` (``owlet1/cache.py:96-124``): partial groups carried
  across calls, ``entry_count * ratio`` = position of the next group's first token.
* ``compressor_forward`` -- ``DeepseekV41Compressor.forward`` given the fp32 ``kv`` /
  ``gate`` projections: returns ``(latent | None, first_group_position)``.
"""

from __future__ import annotations

import torch

from . import _lib


def apply_rotary_pos_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """owlet1/norm_rope.py:126-145 on the GPU (fp32 math, output in ``x.dtype``)."""
    _lib.require_gpu(x)
    rd = cos.shape[-1] * 2
    d = x.shape[-1]
    heads = x.shape[2] if x.dim() == 4 else 1
    xc = x.contiguous()
    c = cos.float().contiguous()
    s = sin.float().contiguous()
    rows = xc.numel() // d
    if c.numel() * heads != rows * (rd // 2):
        raise ValueError(f"cos/sin {tuple(cos.shape)} do not match x {tuple(x.shape)}")
    y = torch.empty_like(xc)
    _lib.call("mzk_rope", xc.data_ptr(), _lib.dtype_code(x.dtype), c.data_ptr(), s.data_ptr(), rows, d, rd, heads,
              int(bool(inverse)), y.data_ptr(), _lib.stream_of(x))
    return y


def compress(kv: torch.Tensor, gate: torch.Tensor | None, ratio: int, norm_weight: torch.Tensor, eps: float,
             dtype: torch.dtype, n_groups: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """kv/gate fp32 [B, T, D] -> normed pre-RoPE latent [B, n_groups, D] in ``dtype``
    (``n_groups`` defaults to ``T // ratio``)."""
    _lib.require_gpu(kv, norm_weight)
    if kv.dtype != torch.float32 or (gate is not None and gate.dtype != torch.float32):
        raise TypeError("compress: kv and gate must be the fp32 projections")
    if ratio > 1 and gate is None:
        raise ValueError("compress: ratio > 1 needs the gate")
    b, t, d = kv.shape
    n = t // ratio if n_groups is None else n_groups
    kvc = kv.contiguous()
    gc = gate.contiguous() if gate is not None else None
    w = norm_weight.contiguous()
    if out is None:
        out = torch.empty(b, n, d, dtype=dtype, device=kv.device)
    _lib.call("mzk_compress", kvc.data_ptr(), _lib.ptr(gc), b, n, ratio, d, t, w.data_ptr(), _lib.dtype_code(w.dtype),
              float(eps), out.data_ptr(), _lib.dtype_code(dtype), _lib.stream_of(kv))
    return out


class GroupCarry:
    """Partial-group carry of one compressed branch (owlet1/cache.py:96-124)."""

    def __init__(self):
        self.buffer_kv: torch.Tensor | None = None
        self.buffer_gate: torch.Tensor | None = None
        self.entry_count = 0

    def store(self, kv: torch.Tensor, gate: torch.Tensor | None, ratio: int):
        """cache.py:96-113: prepend the buffered tokens, peel off the longest group-aligned
        prefix, keep the remainder; returns (chunk_kv, chunk_gate, first_group_position)."""
        first = self.entry_count * ratio
        if self.buffer_kv is not None and self.buffer_kv.shape[1]:
            kv = torch.cat([self.buffer_kv, kv], dim=1)
            if gate is not None:
                gate = torch.cat([self.buffer_gate, gate], dim=1)
        usable = (kv.shape[1] // ratio) * ratio
        self.buffer_kv = kv[:, usable:]
        self.buffer_gate = None if gate is None else gate[:, usable:]
        return kv[:, :usable], None if gate is None else gate[:, :usable], first

    def emitted(self, n: int) -> None:
        """cache.py:122-123: groups emitted so far."""
        self.entry_count += n


def compressor_forward(kv: torch.Tensor, gate: torch.Tensor | None, ratio: int, norm_weight: torch.Tensor,
                       eps: float, dtype: torch.dtype, carry: GroupCarry | None = None):
    """DeepseekV41Compressor.forward (owlet1/cache.py:157-172) from the fp32 projections:
    returns ``(latent [B, n, D] | None, first_group_position)``."""
    if ratio == 1:
        first = 0 if carry is None else carry.entry_count
        latent = compress(kv, None, 1, norm_weight, eps, dtype)
        return latent, first
    if carry is None:
        usable = (kv.shape[1] // ratio) * ratio
        chunk_kv, chunk_gate, first = kv[:, :usable], gate[:, :usable], 0
    else:
        chunk_kv, chunk_gate, first = carry.store(kv, gate, ratio)
    if chunk_kv.shape[1] == 0:
        return None, first
    return compress(chunk_kv, chunk_gate, ratio, norm_weight, eps, dtype), first
