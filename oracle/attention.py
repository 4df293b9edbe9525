"""CPU restatement of the reference's attention/indexer math (test infrastructure only).

torch fp32 on the CPU, following ``src/mzoo/layers/attn/golden_ref.py``:

* ``golden``          -- ``golden`` 103-168 with ``_attend`` 83-100 (levels ``latent``,
                         ``window``, ``compressed``, ``sparse``; sink in the
                         denominator only; lse in natural log, sink included)
* ``indexer_scores``  -- ``indexer_scores`` 213-227 (= ``owlet1/indexer.py:124-143``),
                         generalised to explicit absolute query positions so the same
                         function covers decode rows
* ``topk_indices``    -- ``topk_indices`` 230-243 (= ``owlet1/indexer.py:158-165``) with
                         this build's tie rule made explicit: among equal scores the lower
                         index wins, and the kept indices are listed in ascending order
                         followed by the ``-1`` padding
* ``select_candidate_blocks`` -- ``owlet1/indexer.py:14-40`` (level one of the two-level
                         top-k), its top-k over block scores with the same tie rule
* ``attend_entries``  -- one query row against an explicit list of K==V latent entries
                         plus a sink: what ``eager_attention_forward``
                         (``owlet1/attention.py:42-71``) computes for one decode row once
                         the window mask and ``topk_bias`` have removed the invisible
                         columns.
"""

from __future__ import annotations

import numpy as np
import torch


def _bias(visible: torch.Tensor) -> torch.Tensor:
    return torch.zeros_like(visible, dtype=torch.float32).masked_fill(~visible, float("-inf"))


def _attend(q, k, v, mask, sinks):
    """golden_ref.py:83-100 in fp32: q [B,H,S,D], k/v [B,1,T,D] -> (o [B,S,H,D], lse [B,H,S])."""
    logits = torch.matmul(q.float(), k.float().transpose(-1, -2)) * q.shape[-1] ** -0.5
    if mask is not None:
        logits = logits + mask
    if sinks is not None:
        col = sinks.float().view(1, -1, 1, 1).expand(logits.shape[0], -1, logits.shape[2], 1)
        logits = torch.cat([logits, col], dim=-1)
    lse = torch.logsumexp(logits, dim=-1)
    probs = torch.softmax(logits, dim=-1)
    if sinks is not None:
        probs = probs[..., :-1]
    o = torch.matmul(probs, v.float())
    return o.transpose(1, 2), lse


def golden(q, kv, *, level, sinks=None, window=None, main_kv=None, compress_ratio=None, indices=None):
    """golden_ref.py:103-168 (causal only).  q [B,S,H,D], kv [B,S,1,D], main_kv [B,G,1,D],
    indices [B,S,topk] (-1 = empty slot; trusted, no group-causal re-check)."""
    b, s, h, d = q.shape
    qt = q.transpose(1, 2)
    lat = kv.transpose(1, 2)
    t_idx = torch.arange(s).view(-1, 1)
    k_idx = torch.arange(s).view(1, -1)
    causal = k_idx <= t_idx
    if level == "latent":
        return _attend(qt, lat, lat, _bias(causal).view(1, 1, s, s), sinks)
    win_mask = _bias(causal & (k_idx > t_idx - window)).view(1, 1, s, s)   # golden_ref.py:73-76
    if level == "window":
        return _attend(qt, lat, lat, win_mask, sinks)
    g = main_kv.shape[1]
    main = main_kv.transpose(1, 2)
    g_idx = torch.arange(g).view(1, -1)
    k = torch.cat([lat, main], dim=2)
    if level == "compressed":
        main_mask = _bias(g_idx < (t_idx + 1) // compress_ratio).view(1, 1, s, g)   # golden_ref.py:151-154
        return _attend(qt, k, k, torch.cat([win_mask, main_mask], -1), sinks)
    assert level == "sparse"
    idx = indices.long()
    safe = torch.where(idx < 0, torch.full_like(idx, g), idx)        # golden_ref.py:162-165
    sparse = torch.full((b, s, g + 1), float("-inf")).scatter_(-1, safe, 0.0)[..., :g].view(b, 1, s, g)
    return _attend(qt, k, k, torch.cat([win_mask.expand(b, 1, s, s), sparse], -1), sinks)


def indexer_scores(q, k, w, compress_ratio, positions=None):
    """golden_ref.py:213-227: ``sum_h w[b,s,h] * relu(q[b,s,h]·k[b,g]) * Di^-0.5`` in fp32,
    ``-inf`` where ``g >= (pos+1) // compress_ratio``.  ``positions`` [B,S] absolute query
    positions (default ``0..S-1``, the prefill case)."""
    q, k, w = (torch.as_tensor(t).float() for t in (q, k, w))
    b, s, hi, di = q.shape
    g = k.shape[1]
    raw = torch.einsum("bshd,bgd->bshg", q, k).relu_() * di ** -0.5
    scores = (raw * w.unsqueeze(-1)).sum(dim=2)
    if positions is None:
        positions = torch.arange(s).view(1, s).expand(b, s)
    positions = torch.as_tensor(positions).long().view(b, s, 1)
    visible = torch.arange(g).view(1, 1, g) < (positions + 1) // compress_ratio
    return scores.masked_fill(~visible, float("-inf"))


def indexer_abs_scores(q, k, w, compress_ratio, positions=None):
    """``Di^-0.5 * sum_h |w[b,s,h]| * sum_d |q[b,s,h,d] * k[b,g,d]|`` -- the magnitude the
    rounding error of any fp32 accumulation order of ``indexer_scores`` scales with (the
    scale the relative tolerance is stated against).  Masked entries are ``-inf``."""
    q, k, w = (torch.as_tensor(t).float() for t in (q, k, w))
    mag = torch.einsum("bshd,bgd->bshg", q.abs(), k.abs()) * q.shape[-1] ** -0.5
    out = (mag * w.abs().unsqueeze(-1)).sum(dim=2)
    ref = indexer_scores(q[..., :1] * 0, k[..., :1] * 0, w, compress_ratio, positions)
    return out.masked_fill(torch.isinf(ref), float("-inf"))


def topk_indices(scores, topk: int) -> np.ndarray:
    """golden_ref.py:230-243 / indexer.py:158-165 with the lowest-index tie rule.

    ``scores`` [..., G] fp32 -> int64 [..., topk]: the ``min(topk, G)`` best entries
    (larger score first, lower index first among equals), dropping ``-inf`` picks, listed
    in ascending index order, then ``-1`` up to ``topk``."""
    sc = np.asarray(torch.as_tensor(scores).float().numpy() if not isinstance(scores, np.ndarray) else scores,
                    np.float32)
    lead = sc.shape[:-1]
    g = sc.shape[-1]
    if g == 0 or sc.size == 0:
        return np.full((*lead, topk), -1, np.int64)
    flat = sc.reshape(-1, g)
    out = np.full((flat.shape[0], topk), -1, np.int64)
    kk = min(topk, g)
    idx = np.arange(g)
    for r in range(flat.shape[0]):
        row = flat[r]
        order = np.lexsort((idx, -row.astype(np.float64)))[:kk]
        order = order[row[order] > -np.inf]
        order.sort()
        out[r, :len(order)] = order
    return out.reshape(*lead, topk)


def select_candidate_blocks(logits, compress_lens, topk_blocks: int, block_size: int) -> np.ndarray:
    """owlet1/indexer.py:14-40: block maxima of ``logits`` [..., W] over blocks of
    ``block_size`` (the tail padded with -inf), the block ``(compress_lens - 1) //
    block_size`` (floor division, so a length of 0 pins nothing) set to +inf, the top
    ``min(topk_blocks, blocks)`` blocks whose score is above -inf (``topk_indices``: lower
    block first among equals), expanded to a bool mask [..., W].  ``compress_lens`` carries
    a trailing axis ([..., 1]) as in the reference."""
    x = np.asarray(logits, np.float32)
    w = x.shape[-1]
    lead = x.shape[:-1]
    nb = -(-w // block_size)
    pad = np.full((*lead, nb * block_size - w), -np.inf, np.float32)
    blocks = np.concatenate([x, pad], -1).reshape(*lead, nb, block_size).max(-1)
    cl = np.broadcast_to(np.asarray(compress_lens, np.int64), (*lead, 1))
    last = (cl - 1) // block_size
    blocks = np.where(np.arange(nb) == last, np.float32(np.inf), blocks)
    sel = topk_indices(blocks, min(topk_blocks, nb))
    keep = np.zeros((*lead, nb), bool)
    flat_keep, flat_sel = keep.reshape(-1, nb), sel.reshape(-1, sel.shape[-1])
    for r in range(flat_sel.shape[0]):
        chosen = flat_sel[r][flat_sel[r] >= 0]
        flat_keep[r, chosen] = True
    return np.repeat(keep, block_size, axis=-1)[..., :w]


def attend_entries(q, entries, sinks=None):
    """One decode row: q [H,D] fp32 against K==V ``entries`` [T,D] fp32 (already filtered to
    the visible ones) with an optional per-head sink column.  Returns (o [H,D], lse [H])."""
    q = torch.as_tensor(q).float()
    e = torch.as_tensor(entries).float()
    logits = (q @ e.T) * q.shape[-1] ** -0.5
    if sinks is not None:
        logits = torch.cat([logits, torch.as_tensor(sinks).float().view(-1, 1)], -1)
    lse = torch.logsumexp(logits, -1)
    p = torch.softmax(logits, -1)
    if sinks is not None:
        p = p[:, :-1]
    return p @ e, lse
