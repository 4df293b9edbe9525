"""Sparse shared-latent MQA attention on the GPU (piece 5).

Kernel-level drop-ins with the reference's signatures
(``src/mzoo/layers/attn/csa2_attn/{fwd,attn}.py``):

* ``fwd(q, kv, main_kv, indices, *, window, compress_ratio, causal=True, sinks=None)``
  -> ``(o bf16 [B,S,H,D], lse fp32 [B,H,S])``   (csa2_attn/fwd.py:238-286)
* ``attn(...)`` -> ``o``                          (csa2_attn/attn.py:40-55, forward only)

``q`` bf16 [B,S,H,D], ``kv`` bf16 [B,S,1,D] (raw latent, K == V), ``main_kv`` bf16
[B,G,1,D], ``indices`` int32/int64 [B,S,topk] (``-1`` = empty).  Window ``W`` counts the
query itself (tokens ``t-W+1..t``); ``compress_ratio`` is documentation only: the
group-causal rule is baked into ``indices`` by the indexer, as in the reference.

Decode form over the packed caches (used by ``mzoo_amd.decode``):

* ``sparse_mqa_decode(q, positions, win_cache, window, ...)`` -- FP8-b128 (656 B) ring
  window cache, optional dense compressed cache and gathered top-k cache, split-KV.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

FMT_BF16, FMT_FP8 = 0, 1


def workspace_bytes(rows: int, heads: int, dim: int, nsplit: int) -> int:
    """Split-KV workspace: each split's output O/l in bf16, then its (m, l) in fp32, then the
    records of the split merge inside the attention launch (``mzk_sparse_mqa_workspace_bytes``)."""
    if nsplit <= 1:
        return 0
    n = ctypes.c_int64(0)
    _lib.call("mzk_sparse_mqa_workspace_bytes", rows, heads, dim, nsplit, ctypes.byref(n))
    return n.value


def new_workspace(rows: int, heads: int, dim: int, nsplit: int, device) -> torch.Tensor:
    """A split-KV workspace for ``sparse_mqa_decode`` (zero-filled, as the in-launch merge's
    records must be before their first use)."""
    return torch.zeros(max((workspace_bytes(rows, heads, dim, nsplit) + 3) // 4, 1), dtype=torch.float32,
                       device=device)


def set_merge(mode: int) -> None:
    """Where split partials are merged: 0 the merge kernel (default), 1 inside the attention
    launch where it applies, 2 inside with the cross-XCD cache path forced (tests)."""
    _lib.call("mzk_sparse_mqa_set_merge", mode)


def merge_status(workspace: torch.Tensor, rows: int, heads: int, dim: int, nsplit: int) -> tuple[int, int]:
    """The in-launch merge's status words of a workspace: (1 if a split ever gave up waiting
    for its siblings, else 0; the number of (row, 64-head group) merges done inside attention
    launches since the workspace was zeroed)."""
    off = workspace_bytes(rows, heads, dim, nsplit) - 16
    w = workspace.view(torch.uint8)[off:off + 8].view(torch.int32).cpu()
    return int(w[0]), int(w[1])


def sparse_mqa_decode_select(q: torch.Tensor, positions: torch.Tensor, win_cache: torch.Tensor, window: int, *,
                             main_cache: torch.Tensor, scores: torch.Tensor, topk: int,
                             idx_out: torch.Tensor | None = None, dense_cache: torch.Tensor | None = None,
                             dense_ratio: int = 1, sinks: torch.Tensor | None = None, nsplit: int = 1,
                             nope: int = 512, workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                             lse: torch.Tensor | None = None, rope: tuple | None = None, advance: bool = False):
    """``sparse_mqa_decode`` over the top-``topk`` of the indexer ``scores`` (fp32 [B, G], the
    keys of ``main_cache``'s first G entries) -- the reference's ``index_scores.topk``
    (``owlet1/indexer.py:158-165``, lowest index first among equal scores) feeding its
    sparse attention -- with the selection inside the attention launch where it fits
    (``mzk_sparse_mqa_select``).  Returns (o, lse, idx int32 [B, topk]: the list the attention
    read, ascending picks then -1)."""
    b, h, d = q.shape
    _lib.require_gpu(q, positions, win_cache, main_cache, scores)
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.shape[0] != b or scores.stride(1) != 1:
        raise ValueError(f"sparse_mqa_decode_select: scores must be fp32 [{b}, G] with unit column stride")
    for name, t, dt, shape in (("q", q, torch.bfloat16, (b, h, d)), ("positions", positions, torch.int64, (b,)),
                               ("win_cache", win_cache, torch.uint8, None), ("main_cache", main_cache, torch.uint8, None),
                               ("dense_cache", dense_cache, torch.uint8, None), ("sinks", sinks, torch.float32, (h,)),
                               ("out", out, torch.bfloat16, (b, h, d)), ("lse", lse, torch.float32, (b, h)),
                               ("idx_out", idx_out, torch.int32, (b, topk))):
        if t is None:
            continue
        if t.dtype != dt or not t.is_contiguous() or (shape is not None and tuple(t.shape) != shape):
            raise ValueError(f"sparse_mqa_decode_select: {name} must be a contiguous {dt} tensor"
                             + (f" of shape {list(shape)}" if shape is not None else ""))
    rc = rs = None
    if rope is not None:
        rc, rs = (t.contiguous() for t in rope)
        if rc.dtype != torch.bfloat16 or rs.dtype != torch.bfloat16 or rc.shape != (b, (d - nope) // 2) \
                or rs.shape != rc.shape:
            raise ValueError(f"sparse_mqa_decode_select: rope cos/sin must be bf16 [B, {(d - nope) // 2}]")
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty(b, h, dtype=torch.float32, device=q.device) if lse is None else lse
    idx_out = torch.empty(b, topk, dtype=torch.int32, device=q.device) if idx_out is None else idx_out
    need = workspace_bytes(b, h, d, nsplit)
    if nsplit > 1 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = new_workspace(b, h, d, nsplit, q.device)
    g = scores.shape[1]
    _lib.call("mzk_sparse_mqa_select", q.data_ptr(), b, h, d, FMT_FP8, nope, positions.data_ptr(), int(advance),
              win_cache.data_ptr(), win_cache.shape[1], win_cache.shape[1], window,
              _lib.ptr(dense_cache), 0 if dense_cache is None else dense_cache.shape[1],
              0 if dense_cache is None else dense_cache.shape[1], dense_ratio, main_cache.data_ptr(),
              main_cache.shape[1], g, scores.data_ptr(), scores.stride(0), topk, idx_out.data_ptr(), topk,
              _lib.ptr(sinks), nsplit, _lib.ptr(workspace), need, out.data_ptr(), lse.data_ptr(), _lib.ptr(rc),
              _lib.ptr(rs), 0 if rope is None else d - nope, _lib.stream_of(q))
    return out, lse, idx_out


def fwd(q: torch.Tensor, kv: torch.Tensor, main_kv: torch.Tensor, indices: torch.Tensor, *, window: int,
        compress_ratio: int, causal: bool = True, sinks: torch.Tensor | None = None):
    """Sliding-window + top-k gathered compressed shared-latent MQA forward."""
    assert causal, "csa2_attn is causal-only: a non-causal sliding window is not a model shape"
    assert isinstance(window, int) and window >= 1, f"window must be a positive int, got {window!r}"
    assert isinstance(compress_ratio, int) and compress_ratio >= 1, (
        f"compress_ratio must be a positive int, got {compress_ratio!r}")
    assert q.dtype == torch.bfloat16, f"expected bf16, got {q.dtype}"
    batch, seq_len, heads, dim = q.shape
    assert kv.shape == (batch, seq_len, 1, dim), f"kv must be [B, S, 1, D]={(batch, seq_len, 1, dim)}, got {tuple(kv.shape)}"
    groups = main_kv.shape[1]
    assert main_kv.shape == (batch, groups, 1, dim), f"main_kv must be [B, G, 1, D], got {tuple(main_kv.shape)}"
    assert indices.dtype in (torch.int32, torch.int64), f"indices must be int32/int64, got {indices.dtype}"
    assert indices.dim() == 3 and indices.shape[:2] == (batch, seq_len), (
        f"indices must be [B, S, topk]=[{batch}, {seq_len}, *], got {tuple(indices.shape)}")
    if sinks is not None:
        assert sinks.shape == (heads,), f"sinks must be [H]={heads}, got {tuple(sinks.shape)}"
    _lib.require_gpu(q, kv, main_kv, indices)
    topk = indices.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(batch, heads, seq_len, dtype=torch.float32, device=q.device)
    if batch * seq_len == 0:
        return o, lse
    qc = q.contiguous()
    kvc = kv.contiguous().view(batch, seq_len, dim)
    has_main = groups > 0 and topk > 0
    main = main_kv.contiguous().view(batch, groups, dim) if has_main else None
    idx = indices.to(torch.int32).contiguous() if has_main else None
    pos = torch.arange(seq_len, device=q.device, dtype=torch.int64).repeat(batch)
    sk = sinks.detach().float().contiguous() if sinks is not None else None
    _lib.call("mzk_sparse_mqa", qc.data_ptr(), batch, seq_len, heads, dim, FMT_BF16, dim, pos.data_ptr(),
              kvc.data_ptr(), seq_len, 0, min(window, seq_len), None, 0, 0, 1,
              _lib.ptr(main), groups, groups, _lib.ptr(idx), topk, topk if has_main else 0, _lib.ptr(sk), 1, None, 0,
              o.data_ptr(), lse.data_ptr(), _lib.stream_of(q))
    return o, lse


def attn(q, kv, main_kv, indices, *, window: int, compress_ratio: int, causal: bool = True, sinks=None):
    """Forward of ``csa2_attn.attn`` (no autograd: this build is inference-only)."""
    return fwd(q, kv, main_kv, indices, window=window, compress_ratio=compress_ratio, causal=causal, sinks=sinks)[0]


def sparse_mqa_decode(q: torch.Tensor, positions: torch.Tensor, win_cache: torch.Tensor, window: int, *,
                      main_cache: torch.Tensor | None = None, groups: int = 0, indices: torch.Tensor | None = None,
                      dense_cache: torch.Tensor | None = None, dense_ratio: int = 1,
                      sinks: torch.Tensor | None = None, nsplit: int = 1, nope: int = 512,
                      workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                      lse: torch.Tensor | None = None, rope: tuple | None = None, advance: bool = False):
    """One decode token per batch row over FP8-b128 caches.

    q bf16 [B,H,D]; positions int64 [B] (absolute position of the new token, whose own
    entry is already in the window ring); win_cache uint8 [B,Wcap,EB] ring (token t at slot
    t % Wcap); main_cache uint8 [B,Gcap,EB] with int32 ``indices`` [B,topk] over its first
    ``groups`` entries; dense_cache uint8 [B,Dcap,EB] scanned over its first
    ``(pos+1)//dense_ratio`` entries.  Returns (o bf16 [B,H,D], lse fp32 [B,H]).

    ``rope=(cos, sin)`` (bf16 [B, (D-nope)/2], the row's ``position_embeddings``): q arrives
    unrotated and the kernels apply ``apply_rotary_pos_emb`` to it on load and the inverse
    rotation to the output (``owlet1/attention.py:147`` and ``:226`` fused in).

    ``advance=True`` also adds 1 to ``positions`` once the call's launches have read them, in
    the split merge's launch (no launch of its own for a decode step's ``positions += 1``;
    ``mzk_sparse_mqa_advance``)."""
    b, h, d = q.shape
    _lib.require_gpu(q, positions, win_cache)
    # the kernels read these buffers through raw pointers with the layouts below: a wrong
    # dtype or a strided view would be read as other data, so it is rejected, not converted
    checks = (("q", q, torch.bfloat16, (b, h, d)), ("positions", positions, torch.int64, None),
              ("win_cache", win_cache, torch.uint8, None), ("main_cache", main_cache, torch.uint8, None),
              ("dense_cache", dense_cache, torch.uint8, None), ("indices", indices, torch.int32, None),
              ("sinks", sinks, torch.float32, (h,)), ("out", out, torch.bfloat16, (b, h, d)),
              ("lse", lse, torch.float32, (b, h)))
    for name, t, dt, shape in checks:
        if t is None:
            continue
        if t.dtype != dt or not t.is_contiguous() or (shape is not None and tuple(t.shape) != shape):
            raise ValueError(f"sparse_mqa_decode: {name} must be a contiguous {dt} tensor"
                             + (f" of shape {list(shape)}" if shape is not None else "")
                             + f", got {t.dtype} {list(t.shape)}{'' if t.is_contiguous() else ' (strided)'}")
    if positions.numel() != b or (indices is not None and (indices.dim() != 2 or indices.shape[0] != b)):
        raise ValueError("sparse_mqa_decode: positions [B] and indices [B, topk] expected")
    rc = rs = None
    if rope is not None:
        rc, rs = (t.contiguous() for t in rope)
        if rc.dtype != torch.bfloat16 or rs.dtype != torch.bfloat16 or rc.shape != (b, (d - nope) // 2) \
                or rs.shape != rc.shape:
            raise ValueError(f"sparse_mqa_decode: rope cos/sin must be bf16 [B, {(d - nope) // 2}]")
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty(b, h, dtype=torch.float32, device=q.device)
    need = workspace_bytes(b, h, d, nsplit)
    if nsplit > 1 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = new_workspace(b, h, d, nsplit, q.device)
    topk = 0 if indices is None else indices.shape[-1]
    args = (q.data_ptr(), b, 1, h, d, FMT_FP8, nope, positions.data_ptr(),
            win_cache.data_ptr(), win_cache.shape[1], win_cache.shape[1], window,
            _lib.ptr(dense_cache), 0 if dense_cache is None else dense_cache.shape[1],
            0 if dense_cache is None else dense_cache.shape[1], dense_ratio,
            _lib.ptr(main_cache), 0 if main_cache is None else main_cache.shape[1], groups,
            _lib.ptr(indices), topk, topk, _lib.ptr(sinks), nsplit, _lib.ptr(workspace), need,
            out.data_ptr(), lse.data_ptr())
    if advance:
        _lib.call("mzk_sparse_mqa_advance", *args, _lib.ptr(rc), _lib.ptr(rs), 0 if rope is None else d - nope,
                  _lib.stream_of(q))
    elif rope is None:
        _lib.call("mzk_sparse_mqa", *args, _lib.stream_of(q))
    else:
        _lib.call("mzk_sparse_mqa_rope", *args, rc.data_ptr(), rs.data_ptr(), d - nope, _lib.stream_of(q))
    return out, lse
