"""Lightning indexer on the GPU (pieces 3 and 4): scores on MFMA, radix top-k.

Kernel-level drop-ins with the reference's signatures and output contracts:

* ``fwd(q, k, w, *, compress_ratio)``        -- ``layers/attn/indexer/fwd.py:112-132``
  bf16 ``q [B,S,Hi,Di]``, ``k [B,T,Di]``, fp32 ``w [B,S,Hi]`` (already x ``Hi**-0.5``)
  -> fp32 ``[B,S,T]``, ``-inf`` where ``t >= (s+1)//compress_ratio``.
* ``attn(q, k, w, *, compress_ratio, topk)`` -- ``layers/attn/indexer/attn.py:67-81``
  -> int32 ``[B,S,topk]``, ``-1`` = empty slot.

Quantized paths used by the decode step (same math on packed operands):

* ``scores_fp8``   -- FP8-e4m3 q/k with one pow2 fp32 scale per row (V3.2 layout)
* ``scores_mxfp4`` -- MXFP4 q/k (e2m1 + e8m0 per 32), the model's own indexer quantizer
* ``topk``         -- per-row top-k, lowest index wins ties, ascending output, ``-1`` pad
* ``candidate_block_list`` / ``candidate_scores_*`` / ``candidate_topk`` -- the two-level
  selection: level one's compact block list, level two's scores over the gathered
  candidates only (cost flat in the cache length) and their top-k as key positions

``positions`` (int64 ``[B,S]``) gives absolute query positions for the group-causal
rule; omitted, query ``s`` sits at position ``s`` (a prefill from position 0).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def _positions(positions, b, s, device):
    if positions is None:
        return None
    p = torch.as_tensor(positions, device=device).to(torch.int64).expand(b, s).contiguous()
    return p


def topk_workspace_bytes(rows: int, g: int) -> int:
    """Workspace bytes ``topk`` needs for ``rows`` rows of ``g`` scores (0: none): long rows
    are split over several workgroups, which exchange partial counts through it."""
    n = ctypes.c_int64(0)
    _lib.call("mzk_topk_workspace_bytes", rows, g, ctypes.byref(n))
    return n.value


def topk(scores: torch.Tensor, k: int, out: torch.Tensor | None = None,
         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """scores fp32 [..., G] -> int32 [..., k]: the ``min(k, G)`` best columns (lower index
    first among equal scores), never a ``-inf`` one, ascending, then ``-1``.  Rows longer
    than 8192 use a workspace of ``topk_workspace_bytes`` bytes: the caller's (kept at a
    fixed address for graph capture) or, if none is given, one allocated here."""
    _lib.require_gpu(scores)
    if scores.dtype != torch.float32:
        raise TypeError(f"topk: scores must be float32, got {scores.dtype}")
    g = scores.shape[-1]
    sc = scores if scores.stride(-1) == 1 else scores.contiguous()
    flat = sc.reshape(-1, g) if sc.dim() != 2 else sc
    rows = flat.shape[0]
    if out is None:
        out = torch.empty(*scores.shape[:-1], k, dtype=torch.int32, device=scores.device)
    of = out.view(-1, k)
    need = topk_workspace_bytes(rows, g) if rows and k else 0
    if need == 0:
        _lib.call("mzk_topk_rows", flat.data_ptr(), rows, g, flat.stride(0) if rows else g, k, of.data_ptr(), k,
                  _lib.stream_of(scores))
        return out
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        if workspace is not None:
            raise ValueError(f"topk: the workspace holds {workspace.numel() * workspace.element_size()} bytes, "
                             f"{need} are needed")
        workspace = torch.empty(need, dtype=torch.uint8, device=scores.device)
    _lib.call("mzk_topk_rows_ws", flat.data_ptr(), rows, g, flat.stride(0), k, of.data_ptr(), k,
              workspace.data_ptr(), workspace.numel() * workspace.element_size(), _lib.stream_of(scores))
    return out


_topk_rows = topk


def select_candidate_blocks(logits: torch.Tensor, compress_lens: torch.Tensor, topk_blocks: int,
                            block_size: int) -> torch.Tensor:
    """Level one of the two-level top-k (reference ``select_candidate_blocks``): keep the
    ``topk_blocks`` highest-scoring blocks of ``block_size`` positions per query, the block
    holding the query's newest position pinned in; bool mask shaped like ``logits``.
    ``compress_lens`` carries a trailing axis ([..., 1]) as in the reference.  Among equal
    block scores the lower block index wins (the reference leaves ties unspecified)."""
    _lib.require_gpu(logits, compress_lens)
    if logits.dtype != torch.float32:
        raise TypeError(f"select_candidate_blocks: logits must be float32, got {logits.dtype}")
    width = logits.shape[-1]
    lead = logits.shape[:-1]
    rows = 1
    for d in lead:
        rows *= d
    cl = torch.as_tensor(compress_lens, device=logits.device).to(torch.int64).expand(*lead, 1).reshape(rows)
    cl = cl.contiguous()
    flat = logits.reshape(rows, width)
    if width and flat.stride(-1) != 1:
        flat = flat.contiguous()
    mask = torch.empty(*lead, width, dtype=torch.bool, device=logits.device)
    if rows == 0 or width == 0:
        return mask
    n = ctypes.c_int64(0)
    _lib.call("mzk_candidate_blocks_workspace_bytes", rows, width, block_size, topk_blocks, ctypes.byref(n))
    ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=logits.device)
    _lib.call("mzk_candidate_blocks", flat.data_ptr(), rows, width, flat.stride(0), cl.data_ptr(), topk_blocks,
              block_size, mask.data_ptr(), width, None, ws.data_ptr(), ws.numel(), _lib.stream_of(logits))
    return mask


def candidate_block_list(logits: torch.Tensor, compress_lens: torch.Tensor, topk_blocks: int, block_size: int,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Level one in the compact form level two gathers from: the blocks
    ``select_candidate_blocks`` keeps, as int32 [..., topk_blocks] block indices ascending,
    then ``-1`` (tickets/0009-indexer-hierarchical.md:36-37 asks for an index list, not a
    mask).  ``out`` (int32 [..., topk_blocks], contiguous) is filled when given."""
    _lib.require_gpu(logits, compress_lens)
    if logits.dtype != torch.float32:
        raise TypeError(f"candidate_block_list: logits must be float32, got {logits.dtype}")
    width = logits.shape[-1]
    lead = logits.shape[:-1]
    rows = 1
    for d in lead:
        rows *= d
    if out is None:
        out = torch.empty(*lead, topk_blocks, dtype=torch.int32, device=logits.device)
    elif out.shape != (*lead, topk_blocks) or out.dtype != torch.int32 or not out.is_contiguous():
        raise ValueError(f"candidate_block_list: out must be contiguous int32 {(*lead, topk_blocks)}")
    if rows == 0 or topk_blocks == 0:
        return out
    if width == 0:
        return out.fill_(-1)
    cl = torch.as_tensor(compress_lens, device=logits.device).to(torch.int64).expand(*lead, 1).reshape(rows)
    cl = cl.contiguous()
    flat = logits.reshape(rows, width)
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    n = ctypes.c_int64(0)
    _lib.call("mzk_candidate_blocks_workspace_bytes", rows, width, block_size, topk_blocks, ctypes.byref(n))
    ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=logits.device)
    _lib.call("mzk_candidate_blocks", flat.data_ptr(), rows, width, flat.stride(0), cl.data_ptr(), topk_blocks,
              block_size, None, 0, out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(logits))
    return out


def _check_cand(cand_blocks, b, s, block_size):
    if cand_blocks.dtype != torch.int32 or cand_blocks.dim() != 3 or cand_blocks.shape[:2] != (b, s) \
            or cand_blocks.stride(-1) != 1 or cand_blocks.stride(0) != s * cand_blocks.stride(1):
        raise ValueError("candidate list must be int32 [B, S, n_blocks] with unit column stride")
    if block_size < 1:
        raise ValueError(f"block_size must be >= 1, got {block_size}")
    return cand_blocks.shape[2]


def candidate_scores_fp8(q_codes: torch.Tensor, q_scales: torch.Tensor, w: torch.Tensor, k_codes: torch.Tensor,
                         k_scales: torch.Tensor, cand_blocks: torch.Tensor, *, block_size: int, compress_ratio: int,
                         positions=None, groups: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Level two on FP8 operands (as ``scores_fp8``): only the candidates' scores, on the
    candidate axis -- fp32 [B, S, n_blocks * block_size], slot j the key
    ``cand_blocks[b, s, j // block_size] * block_size + j % block_size`` (``-inf`` for a
    ``-1`` block, a key >= ``groups`` or one not yet visible).  The bits of a slot equal
    ``scores_fp8``'s score of its key (decode-shape rows).  Cost follows the candidate
    count, not the cache length (tickets/0009-indexer-hierarchical.md:29-32)."""
    b, s, hi, di = q_codes.shape
    gcap = k_codes.shape[1]
    g = gcap if groups is None else groups
    if k_codes.shape != (b, gcap, di) or k_scales.shape != (b, gcap) or q_scales.shape != (b, s, hi) \
            or w.shape != (b, s, hi) or q_codes.dtype != torch.uint8 or k_codes.dtype != torch.uint8:
        raise ValueError("candidate_scores_fp8: shape/dtype mismatch")
    _lib.require_gpu(q_codes, k_codes, cand_blocks)
    nb = _check_cand(cand_blocks, b, s, block_size)
    out = _check_scores_out(b, s, nb * block_size, q_codes.device, out)
    pos = _positions(positions, b, s, q_codes.device)
    qc, qs, wc, kc, ks = (q_codes.contiguous(), q_scales.float().contiguous(), w.float().contiguous(),
                          k_codes.contiguous(), k_scales.float().contiguous())
    _lib.call("mzk_indexer_candidate_scores_fp8", qc.data_ptr(), qs.data_ptr(), wc.data_ptr(), kc.data_ptr(),
              ks.data_ptr(), b, s, hi, di, g, gcap, _lib.ptr(pos), compress_ratio, cand_blocks.data_ptr(),
              cand_blocks.stride(1), nb, block_size, out.data_ptr(), out.stride(1), _lib.stream_of(q_codes))
    return out


def candidate_scores_mxfp4(q_packed: torch.Tensor, q_e8m0: torch.Tensor, w: torch.Tensor, k_packed: torch.Tensor,
                           k_e8m0: torch.Tensor, cand_blocks: torch.Tensor, *, block_size: int, compress_ratio: int,
                           positions=None, groups: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``candidate_scores_fp8`` on MXFP4 operands (as ``scores_mxfp4``)."""
    b, s, hi, half = q_packed.shape
    di = half * 2
    gcap = k_packed.shape[1]
    g = gcap if groups is None else groups
    if k_packed.shape != (b, gcap, half) or k_e8m0.shape != (b, gcap, di // 32) \
            or q_e8m0.shape != (b, s, hi, di // 32) or w.shape != (b, s, hi):
        raise ValueError("candidate_scores_mxfp4: shape mismatch")
    _lib.require_gpu(q_packed, k_packed, cand_blocks)
    nb = _check_cand(cand_blocks, b, s, block_size)
    out = _check_scores_out(b, s, nb * block_size, q_packed.device, out)
    pos = _positions(positions, b, s, q_packed.device)
    qp, qe, wc, kp, ke = (q_packed.contiguous(), q_e8m0.contiguous(), w.float().contiguous(), k_packed.contiguous(),
                          k_e8m0.contiguous())
    _lib.call("mzk_indexer_candidate_scores_mxfp4", qp.data_ptr(), qe.data_ptr(), wc.data_ptr(), kp.data_ptr(),
              ke.data_ptr(), b, s, hi, di, g, gcap, _lib.ptr(pos), compress_ratio, cand_blocks.data_ptr(),
              cand_blocks.stride(1), nb, block_size, out.data_ptr(), out.stride(1), _lib.stream_of(q_packed))
    return out


def candidate_positions(slot_idx: torch.Tensor, cand_blocks: torch.Tensor, block_size: int,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """Top-k picks on the candidate axis (int32 [..., k], ``-1`` = empty) -> key positions
    (same shape; ``out`` may be ``slot_idx`` itself).  Ascending slots give ascending keys."""
    _lib.require_gpu(slot_idx, cand_blocks)
    k = slot_idx.shape[-1]
    nb = cand_blocks.shape[-1]
    if slot_idx.dtype != torch.int32 or not slot_idx.is_contiguous() or cand_blocks.dtype != torch.int32 \
            or cand_blocks.shape[:-1] != slot_idx.shape[:-1] or not cand_blocks.is_contiguous():
        raise ValueError("candidate_positions: slot_idx / cand_blocks must be contiguous int32 [..., k] / [..., nb]")
    if out is None:
        out = torch.empty_like(slot_idx)
    elif out.shape != slot_idx.shape or out.dtype != torch.int32 or not out.is_contiguous():
        raise ValueError("candidate_positions: out must be contiguous int32 like slot_idx")
    rows = slot_idx.numel() // k if k else 0
    _lib.call("mzk_candidate_positions", slot_idx.data_ptr(), rows, k, k, cand_blocks.data_ptr(), nb, nb, block_size,
              out.data_ptr(), k, _lib.stream_of(slot_idx))
    return out


def candidate_topk(scores: torch.Tensor, cand_blocks: torch.Tensor, block_size: int, k: int,
                   out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Top-k of candidate-axis scores as key positions: the same list ``topk`` gives on the
    dense row masked to the candidates (owlet1/indexer.py:150-151 then :158-161), since
    slot order follows key order -- ascending, lower key first among equal scores, ``-1``
    pad.  Up to 32768 slots one launch (``mzk_candidate_topk``); longer candidate axes take
    ``topk`` (with ``workspace``) and ``candidate_positions``."""
    _lib.require_gpu(scores, cand_blocks)
    slots = scores.shape[-1]
    nb = cand_blocks.shape[-1]
    if slots > 32768:
        idx = topk(scores, k, out=out, workspace=workspace)
        return candidate_positions(idx, cand_blocks, block_size, out=idx)
    if scores.dtype != torch.float32 or cand_blocks.dtype != torch.int32 or not cand_blocks.is_contiguous() \
            or cand_blocks.shape[:-1] != scores.shape[:-1] or slots != nb * block_size:
        raise ValueError("candidate_topk: scores fp32 [..., n_blocks * block_size], cand_blocks int32 [..., n_blocks]")
    sc = scores if scores.stride(-1) == 1 else scores.contiguous()
    flat = sc.reshape(-1, slots) if sc.dim() != 2 else sc
    rows = flat.shape[0]
    if out is None:
        out = torch.empty(*scores.shape[:-1], k, dtype=torch.int32, device=scores.device)
    elif out.shape != (*scores.shape[:-1], k) or out.dtype != torch.int32 or not out.is_contiguous():
        raise ValueError("candidate_topk: out must be contiguous int32 [..., k]")
    if rows == 0 or k == 0:
        return out
    _lib.call("mzk_candidate_topk", flat.data_ptr(), rows, slots, flat.stride(0) if slots else max(slots, 1), k,
              cand_blocks.data_ptr(), nb, nb, block_size, out.data_ptr(), k, _lib.stream_of(scores))
    return out


def _check_scores_out(b, s, g, device, out):
    if out is None:
        return torch.empty(b, s, g, dtype=torch.float32, device=device)
    if out.shape != (b, s, g) or out.dtype != torch.float32 or out.stride(-1) != 1 or out.stride(0) != s * out.stride(1):
        raise ValueError("scores out must be fp32 [B, S, G] with unit column stride")
    return out


def fwd(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, *, compress_ratio: int, positions=None) -> torch.Tensor:
    """Lightning-indexer score matrix (reference ``indexer.fwd``)."""
    assert q.dtype == k.dtype == torch.bfloat16, f"q/k must be bf16, got {q.dtype}/{k.dtype}"
    batch, seq_len, heads, dim = q.shape
    assert k.shape[0] == batch and k.shape[2] == dim, f"k must be [B, T, {dim}], got {tuple(k.shape)}"
    assert w.shape == (batch, seq_len, heads), f"w must be [B, S, Hi]={(batch, seq_len, heads)}, got {tuple(w.shape)}"
    assert compress_ratio >= 1, f"compress_ratio must be >= 1, got {compress_ratio}"
    _lib.require_gpu(q, k, w)
    seq_kv = k.shape[1]
    out = torch.empty(batch, seq_len, seq_kv, dtype=torch.float32, device=q.device)
    if seq_kv == 0 or batch * seq_len == 0:
        return out
    qc, kc, wc = q.contiguous(), k.contiguous(), w.float().contiguous()
    pos = _positions(positions, batch, seq_len, q.device)
    _lib.call("mzk_indexer_scores_bf16", qc.data_ptr(), wc.data_ptr(), kc.data_ptr(), batch, seq_len, heads, dim, seq_kv,
              seq_kv, _lib.ptr(pos), compress_ratio, out.data_ptr(), seq_kv, _lib.stream_of(q))
    return out


def attn(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, *, compress_ratio: int, topk: int,
         positions=None) -> torch.Tensor:
    """Indices int32 [B, S, topk] (``-1`` = empty slot) -- reference ``indexer.attn``."""
    batch, seq_len = q.shape[0], q.shape[1]
    assert topk >= 0, f"topk must be >= 0, got {topk}"
    idx = torch.full((batch, seq_len, topk), -1, dtype=torch.int32, device=q.device)
    if topk == 0 or k.shape[1] == 0:
        return idx
    scores = fwd(q, k, w, compress_ratio=compress_ratio, positions=positions)
    return _topk_rows(scores, topk, out=idx)


def scores_fp8(q_codes: torch.Tensor, q_scales: torch.Tensor, w: torch.Tensor, k_codes: torch.Tensor,
               k_scales: torch.Tensor, *, compress_ratio: int, positions=None, groups: int | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """FP8 indexer scores.  q_codes uint8 [B,S,Hi,Di], q_scales fp32 [B,S,Hi], w fp32
    [B,S,Hi], k_codes uint8 [B,Gcap,Di], k_scales fp32 [B,Gcap]; ``groups`` (default Gcap)
    keys of each batch row are scored -> fp32 [B,S,groups]."""
    b, s, hi, di = q_codes.shape
    gcap = k_codes.shape[1]
    g = gcap if groups is None else groups
    if k_codes.shape != (b, gcap, di) or k_scales.shape != (b, gcap) or q_scales.shape != (b, s, hi) \
            or w.shape != (b, s, hi) or q_codes.dtype != torch.uint8 or k_codes.dtype != torch.uint8:
        raise ValueError("scores_fp8: shape/dtype mismatch")
    _lib.require_gpu(q_codes, k_codes)
    out = _check_scores_out(b, s, g, q_codes.device, out)
    pos = _positions(positions, b, s, q_codes.device)
    # converted copies stay referenced until the launch is queued: a temporary freed after
    # data_ptr() would return its memory to the caching allocator for the next copy
    qc, qs, wc, kc, ks = (q_codes.contiguous(), q_scales.float().contiguous(), w.float().contiguous(),
                          k_codes.contiguous(), k_scales.float().contiguous())
    _lib.call("mzk_indexer_scores_fp8", qc.data_ptr(), qs.data_ptr(), wc.data_ptr(), kc.data_ptr(), ks.data_ptr(),
              b, s, hi, di, g, gcap, _lib.ptr(pos), compress_ratio, out.data_ptr(), out.stride(1),
              _lib.stream_of(q_codes))
    return out


def decode_fp8(q_idx: torch.Tensor, w: torch.Tensor, k_codes: torch.Tensor, k_scales: torch.Tensor, *,
               compress_ratio: int, positions: torch.Tensor, out: torch.Tensor | None = None,
               q_codes: torch.Tensor | None = None, q_scales: torch.Tensor | None = None,
               kv: torch.Tensor | None = None, win_cache: torch.Tensor | None = None, nope: int = 512,
               rope: int = 64) -> torch.Tensor:
    """Decode-step FP8 indexer with the step's prologue fused in (one launch): q_idx bf16
    [B,Hi,128] is quantized in the kernel (FP8 b128) and scored against k_codes uint8
    [B,Gcap,128] / k_scales fp32 [B,Gcap] -> fp32 [B,1,Gcap].  Optionally also writes the
    quantized query (q_codes uint8 [B,Hi,128] + q_scales fp32 [B,Hi]) and appends the new
    latent kv bf16 [B, nope+rope] to the window ring win_cache uint8 [B,W,entry] at slot
    positions[b] % W -- what ``quant_fp8_block`` + the window write of the step would do."""
    b, hi, di = q_idx.shape
    gcap = k_codes.shape[1]
    if q_idx.dtype != torch.bfloat16 or k_codes.shape != (b, gcap, di) or k_scales.shape != (b, gcap) \
            or w.shape[-1] != hi or w.numel() != b * hi:
        raise ValueError("decode_fp8: shape/dtype mismatch")
    if (q_codes is None) != (q_scales is None):
        raise ValueError("decode_fp8: q_codes and q_scales go together")
    if kv is not None and (kv.dtype != torch.bfloat16 or kv.shape != (b, nope + rope) or win_cache is None):
        raise ValueError("decode_fp8: kv must be bf16 [B, nope+rope] with a window cache")
    _lib.require_gpu(q_idx, k_codes, positions)
    out = _check_scores_out(b, 1, gcap, q_idx.device, out)
    pos = torch.as_tensor(positions, device=q_idx.device).to(torch.int64).reshape(b).contiguous()  # [B] or [B,1]
    for t in (q_codes, q_scales, win_cache):
        if t is not None and not t.is_contiguous():
            raise ValueError("decode_fp8: q_codes, q_scales and win_cache must be contiguous")
    qc = q_idx.contiguous()
    kvc = None if kv is None else kv.contiguous()
    wcap = 0 if win_cache is None else win_cache.shape[1]
    wc, kc, ks = w.float().contiguous(), k_codes.contiguous(), k_scales.float().contiguous()
    _lib.call("mzk_indexer_decode_fp8", qc.data_ptr(), wc.data_ptr(), kc.data_ptr(),
              ks.data_ptr(), b, hi, di, gcap, gcap, pos.data_ptr(), compress_ratio,
              out.data_ptr(), out.stride(1), _lib.ptr(q_codes), _lib.ptr(q_scales), _lib.ptr(kvc), nope, rope,
              _lib.ptr(win_cache), wcap, wcap, _lib.stream_of(qc))
    return out


def decode_mxfp4(q_idx: torch.Tensor, w: torch.Tensor, k_packed: torch.Tensor, k_e8m0: torch.Tensor, *,
                 compress_ratio: int, positions: torch.Tensor, out: torch.Tensor | None = None,
                 q_packed: torch.Tensor | None = None, q_e8m0: torch.Tensor | None = None,
                 kv: torch.Tensor | None = None, win_cache: torch.Tensor | None = None, nope: int = 512,
                 rope: int = 64) -> torch.Tensor:
    """Decode-step MXFP4 indexer with the step's prologue fused in (one launch): q_idx bf16
    [B,Hi,128] is quantized in the kernel (MXFP4, block 32, ue8m0 scales) and scored against
    k_packed uint8 [B,Gcap,64] / k_e8m0 uint8 [B,Gcap,4] -> fp32 [B,1,Gcap].  Optionally
    also writes the quantized query (q_packed uint8 [B,Hi,64] + q_e8m0 uint8 [B,Hi,4]) and
    appends the new latent kv bf16 [B, nope+rope] to the window ring, as ``decode_fp8``."""
    b, hi, di = q_idx.shape
    gcap = k_packed.shape[1]
    if q_idx.dtype != torch.bfloat16 or k_packed.shape != (b, gcap, di // 2) or k_e8m0.shape != (b, gcap, di // 32) \
            or w.shape[-1] != hi or w.numel() != b * hi:
        raise ValueError("decode_mxfp4: shape/dtype mismatch")
    if (q_packed is None) != (q_e8m0 is None):
        raise ValueError("decode_mxfp4: q_packed and q_e8m0 go together")
    if kv is not None and (kv.dtype != torch.bfloat16 or kv.shape != (b, nope + rope) or win_cache is None):
        raise ValueError("decode_mxfp4: kv must be bf16 [B, nope+rope] with a window cache")
    _lib.require_gpu(q_idx, k_packed, positions)
    out = _check_scores_out(b, 1, gcap, q_idx.device, out)
    pos = torch.as_tensor(positions, device=q_idx.device).to(torch.int64).reshape(b).contiguous()  # [B] or [B,1]
    for t in (q_packed, q_e8m0, win_cache):
        if t is not None and not t.is_contiguous():
            raise ValueError("decode_mxfp4: q_packed, q_e8m0 and win_cache must be contiguous")
    qc = q_idx.contiguous()
    kvc = None if kv is None else kv.contiguous()
    wcap = 0 if win_cache is None else win_cache.shape[1]
    wc, kp, ke = w.float().contiguous(), k_packed.contiguous(), k_e8m0.contiguous()
    _lib.call("mzk_indexer_decode_mxfp4", qc.data_ptr(), wc.data_ptr(),
              kp.data_ptr(), ke.data_ptr(), b, hi, di, gcap, gcap, pos.data_ptr(),
              compress_ratio, out.data_ptr(), out.stride(1), _lib.ptr(q_packed), _lib.ptr(q_e8m0), _lib.ptr(kvc),
              nope, rope, _lib.ptr(win_cache), wcap, wcap, _lib.stream_of(qc))
    return out


def decode_fused(q_idx: torch.Tensor, w: torch.Tensor, k: torch.Tensor, k_scales: torch.Tensor, *, fmt: str,
                 compress_ratio: int, positions: torch.Tensor, q_rope: tuple, kv: torch.Tensor,
                 kv_weight: torch.Tensor, kv_eps: float, kv_rope: tuple, win_cache: torch.Tensor,
                 out: torch.Tensor | None = None, q_codes: torch.Tensor | None = None,
                 q_scales: torch.Tensor | None = None, nope: int = 512, rope: int = 64) -> torch.Tensor:
    """The decode step's whole prologue and indexer in one launch (``fmt`` "fp8" or "mxfp4").

    The unrotated indexer query q_idx bf16 [B,Hi,128] is rotated with ``q_rope`` = (cos,
    sin) bf16 [B, rd/2] (the compress RoPE; ``owlet1/indexer.py:126-128``), quantized and
    scored as in ``decode_fp8`` / ``decode_mxfp4``; the new token's kv projection kv bf16
    [B, nope+rope] is normalized (RMSNorm with ``kv_weight`` bf16 [nope+rope] and
    ``kv_eps``), its rope slice rotated with ``kv_rope`` = (cos, sin) bf16 [B, rope/2] and the
    FP8-b128 entry appended to the window ring -- ``owlet1/attention.py:150-155`` for one
    token.  k / k_scales: FP8 codes [B,Gcap,128] + fp32 [B,Gcap], or MXFP4 [B,Gcap,64] +
    e8m0 [B,Gcap,4]."""
    if fmt not in ("fp8", "mxfp4"):
        raise ValueError(f"decode_fused: fmt must be 'fp8' or 'mxfp4', got {fmt!r}")
    b, hi, di = q_idx.shape
    gcap = k.shape[1]
    fp8 = fmt == "fp8"
    kshape, sshape = ((b, gcap, di), (b, gcap)) if fp8 else ((b, gcap, di // 2), (b, gcap, di // 32))
    if q_idx.dtype != torch.bfloat16 or k.shape != kshape or k_scales.shape != sshape or w.numel() != b * hi:
        raise ValueError("decode_fused: shape/dtype mismatch")
    qc_, qs_ = (t.contiguous() for t in q_rope)
    kc_, ks_ = (t.contiguous() for t in kv_rope)
    for name, t, shape in (("q_rope", qc_, None), ("q_rope", qs_, qc_.shape), ("kv_rope", kc_, (b, rope // 2)),
                           ("kv_rope", ks_, (b, rope // 2))):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.shape[0] != b or (shape is not None and t.shape != shape):
            raise ValueError(f"decode_fused: {name} cos/sin must be bf16 [B, rd/2] of one shape")
    if kv.dtype != torch.bfloat16 or kv.shape != (b, nope + rope) or kv_weight.dtype != torch.bfloat16 \
            or kv_weight.numel() != nope + rope:
        raise ValueError("decode_fused: kv and kv_weight must be bf16 [B, nope+rope] / [nope+rope]")
    if (q_codes is None) != (q_scales is None):
        raise ValueError("decode_fused: q_codes and q_scales go together")
    for t in (q_codes, q_scales, win_cache):
        if t is not None and not t.is_contiguous():
            raise ValueError("decode_fused: q_codes, q_scales and win_cache must be contiguous")
    _lib.require_gpu(q_idx, k, positions, kv, win_cache)
    out = _check_scores_out(b, 1, gcap, q_idx.device, out)
    pos = torch.as_tensor(positions, device=q_idx.device).to(torch.int64).reshape(b).contiguous()
    qc = q_idx.contiguous()
    kscales = k_scales.float().contiguous() if fp8 else k_scales.contiguous()
    wcap = win_cache.shape[1]
    wc, kk, kvc, kvw = w.float().contiguous(), k.contiguous(), kv.contiguous(), kv_weight.contiguous()
    _lib.call("mzk_indexer_decode_fused", 0 if fp8 else 1, qc.data_ptr(), wc.data_ptr(),
              kk.data_ptr(), kscales.data_ptr(), b, hi, di, gcap, gcap, pos.data_ptr(), compress_ratio,
              out.data_ptr(), out.stride(1), _lib.ptr(q_codes), _lib.ptr(q_scales), qc_.data_ptr(), qs_.data_ptr(),
              2 * qc_.shape[1], kvc.data_ptr(), kvw.data_ptr(), float(kv_eps),
              kc_.data_ptr(), ks_.data_ptr(), nope, rope, win_cache.data_ptr(), wcap, wcap, _lib.stream_of(qc))
    return out


def scores_mxfp4(q_packed: torch.Tensor, q_e8m0: torch.Tensor, w: torch.Tensor, k_packed: torch.Tensor,
                 k_e8m0: torch.Tensor, *, compress_ratio: int, positions=None, groups: int | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """MXFP4 indexer scores.  q_packed uint8 [B,S,Hi,Di/2], q_e8m0 uint8 [B,S,Hi,Di/32],
    k_packed uint8 [B,Gcap,Di/2], k_e8m0 uint8 [B,Gcap,Di/32] -> fp32 [B,S,groups]."""
    b, s, hi, half = q_packed.shape
    di = half * 2
    gcap = k_packed.shape[1]
    g = gcap if groups is None else groups
    if k_packed.shape != (b, gcap, half) or k_e8m0.shape != (b, gcap, di // 32) \
            or q_e8m0.shape != (b, s, hi, di // 32) or w.shape != (b, s, hi):
        raise ValueError("scores_mxfp4: shape mismatch")
    _lib.require_gpu(q_packed, k_packed)
    out = _check_scores_out(b, s, g, q_packed.device, out)
    pos = _positions(positions, b, s, q_packed.device)
    qp, qe, wc, kp, ke = (q_packed.contiguous(), q_e8m0.contiguous(), w.float().contiguous(), k_packed.contiguous(),
                          k_e8m0.contiguous())
    _lib.call("mzk_indexer_scores_mxfp4", qp.data_ptr(), qe.data_ptr(), wc.data_ptr(), kp.data_ptr(), ke.data_ptr(),
              b, s, hi, di, g, gcap, _lib.ptr(pos), compress_ratio, out.data_ptr(), out.stride(1),
              _lib.stream_of(q_packed))
    return out
