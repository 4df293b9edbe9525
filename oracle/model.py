"""CPU restatement of one CSA2 attention layer as a module (test infrastructure only).

Composes the pinned pieces of this package the way the reference's module does, on the
CPU in float32 (torch + numpy):

* ``layer_forward``  -- ``DeepseekV41Attention.forward``  ``owlet1/attention.py:129-236``
  (q / kv projections and norms, RoPE, the window FP8 fake quant ``:154``, the window
  cache ``:155-156``, compressor -> indexer -> compressed RoPE + FP4 fake quant ``:158-200``,
  the mask extension by the indexer's selection ``:202-214``, the eager attention with sink
  ``:42-71``, the inverse RoPE and the grouped output projection ``:231-235``, ``:20-39``);
* ``compressor``     -- ``DeepseekV41Compressor.forward``  ``owlet1/cache.py:142-172`` with
  the group carry of ``DeepseekV41CSACache.store_compression_weights`` ``:96-113``;
* ``indexer``        -- ``DeepseekV41Indexer.forward``  ``owlet1/indexer.py:78-165`` (key
  publication ``:96-117``, scores ``:124-133``, visibility ``:141-143``, top-k ``:158-165``;
  the two-level candidates are off, as in the benchmark configurations);
* ``LayerState``     -- the cache layer's state ``owlet1/cache.py:39-46`` / ``:84-124``.

``cfg`` is a dict with the config fields the layer reads (``hidden_size``,
``num_attention_heads``, ``head_dim``, ``qk_rope_head_dim``, ``q_lora_rank``, ``o_groups``,
``o_lora_rank``, ``index_n_heads``, ``index_head_dim``, ``index_topk``, ``compress_ratio``,
``sliding_window``, ``rms_norm_eps``, ``compress_rope_theta``); ``params`` maps the
reference's parameter names to float32 tensors.  RMSNorm, the compressor's pooling and the
quantizers are the pinned functions of ``oracle.compressor`` / ``oracle.quant``; the
projections are torch float32 matmuls; the top-k uses ``attention.topk_indices``'s lowest-
index tie rule.  ``select`` overrides the top-k with a given selection (the reference's
``torch.topk`` breaks ties in an unspecified, shape-dependent order).

Parity of this composition is pinned against ``tests/golden/module_fixture.npz``, written by
running the reference's module itself on the CPU (``tests/golden/make_module_fixture.py``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import attention as OA
from . import compressor as C
from . import quant as Q

F32 = np.float32


def _np(t) -> np.ndarray:
    return np.ascontiguousarray(torch.as_tensor(t).float().numpy(), F32)


def _t(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, F32))


def rope_tables(positions, rope_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """``DeepseekV41RotaryEmbedding.forward`` (norm_rope.py:108-124) for the default RoPE:
    ``inv_freq = 1 / theta^(arange(0, rd, 2) / rd)`` (dsv4 modeling_deepseek_v41.py:127-137,
    ``dim = int(head_dim * partial_rotary_factor)`` = qk_rope_head_dim), then
    ``(inv_freq @ positions).T`` cos / sin in float32 -> [..., rd/2]."""
    inv = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float) / rope_dim))
    pos = torch.as_tensor(np.array(positions, np.float32))
    freqs = (inv.view(-1, 1) @ pos.reshape(1, -1)).T.reshape(*pos.shape, -1)
    return freqs.cos().numpy(), freqs.sin().numpy()


def rms_norm(x, weight, eps) -> np.ndarray:
    return C.rms_norm(_np(x), _np(weight), eps, "float32")


def linear(x, w) -> np.ndarray:
    return (_t(x) @ torch.as_tensor(w).float().T).numpy()


@dataclass
class LayerState:
    """``DeepseekV41CSACache`` (owlet1/cache.py:39-124): the window keeps the last W-1
    entries, the buffers carry a partial group across calls, ``compressed`` / ``index_k``
    are the running caches and ``entry_count`` the groups emitted so far."""
    window: np.ndarray | None = None         # [B, <= W-1, D]
    buffer_kv: np.ndarray | None = None      # [B, < r, D] fp32
    buffer_gate: np.ndarray | None = None
    compressed: np.ndarray | None = None     # [B, G, D]
    index_k: np.ndarray | None = None        # [B, G, Di]
    entry_count: int = 0
    positions_seen: int = 0
    extra: dict = field(default_factory=dict)


def compressor(params, cfg, x, state: LayerState | None):
    """cache.py:142-172 (ratio > 1).  Returns (pre-RoPE latent [B, n, D] or None,
    first_group_position)."""
    r = cfg["compress_ratio"]
    kv = linear(x, params["compressor.wkv.weight"])
    gate = linear(x, params["compressor.wgate.weight"])
    if state is None:
        usable = (kv.shape[1] // r) * r
        ck, cg, fgp = kv[:, :usable], gate[:, :usable], 0
    else:
        fgp = state.entry_count * r                                    # cache.py:104
        if state.buffer_kv is not None and state.buffer_kv.shape[1]:
            kv = np.concatenate([state.buffer_kv, kv], 1)
            gate = np.concatenate([state.buffer_gate, gate], 1)
        usable = (kv.shape[1] // r) * r
        state.buffer_kv, state.buffer_gate = kv[:, usable:], gate[:, usable:]
        ck, cg = kv[:, :usable], gate[:, :usable]
    if ck.shape[1] == 0:
        return None, fgp
    latent = C.compress(ck, cg, r, _np(params["compressor.norm.weight"]), cfg["rms_norm_eps"], "float32")
    return latent, fgp


def indexer(params, cfg, x, q_residual, latent, fgp, positions, state, shared, select=None):
    """indexer.py:78-165 for an index source that owns its keys.  Publishes
    ``shared["index_k"]``, ``shared["selection"]`` (bool [B, S, G]) and ``shared["scores"]``."""
    b, s, _ = x.shape
    r, hi, di = cfg["compress_ratio"], cfg["index_n_heads"], cfg["index_head_dim"]
    rd = cfg["qk_rope_head_dim"]
    theta = cfg["compress_rope_theta"]
    if latent is not None:                                            # indexer.py:96-117
        k = rms_norm(linear(latent, params["indexer.wk.weight"]), params["indexer.k_norm.weight"],
                     cfg["rms_norm_eps"])
        gpos = fgp + r * np.arange(latent.shape[1])
        cos, sin = rope_tables(np.broadcast_to(gpos, (b, len(gpos))), rd, theta)
        k = C.rope(k, cos, sin)
        k = Q.fake_quant_fp4_block(k, 32)
        if state is not None:
            state.index_k = k if state.index_k is None else np.concatenate([state.index_k, k], 1)
        else:
            shared["index_k"] = k if shared.get("index_k") is None else np.concatenate([shared["index_k"], k], 1)
    if state is not None:
        shared["index_k"] = state.index_k
    index_k = shared.get("index_k")
    g = 0 if index_k is None else index_k.shape[1]
    if g == 0:
        return
    cos_q, sin_q = rope_tables(positions, rd, theta)                  # indexer.py:124-126
    q = linear(q_residual, params["indexer.wq_b.weight"]).reshape(b, s, hi, di)
    q = C.rope(q, cos_q[:, :, None], sin_q[:, :, None])
    q = Q.fake_quant_fp4_block(q, 32)
    w = linear(x, params["indexer.weights_proj.weight"]) * F32(hi ** -0.5)
    scores = OA.indexer_scores(_t(q), _t(index_k), _t(w), r, torch.as_tensor(positions))
    shared["scores"] = scores
    if select is None:                                                # indexer.py:158-165
        idx = OA.topk_indices(scores, min(cfg["index_topk"], g))
        sel = np.zeros((b, s, g + 1), bool)
        np.put_along_axis(sel, np.where(idx < 0, g, idx), True, -1)
        select = sel[..., :g]
    shared["selection"] = np.asarray(select, bool)[..., :g]


def layer_forward(params, cfg, x, positions, state: LayerState | None = None, select=None):
    """attention.py:129-236 for a KV + index source layer.  x [B, S, hidden] fp32, positions
    [B, S] absolute; ``state`` (LayerState) for a cached call.  Returns (out [B, S, hidden],
    shared) with ``shared["selection"]`` the compressed entries each query attended."""
    x = _np(x)
    positions = np.asarray(positions, np.int64)
    b, s, _ = x.shape
    h, d, rd, w_ = cfg["num_attention_heads"], cfg["head_dim"], cfg["qk_rope_head_dim"], cfg["sliding_window"]
    eps = cfg["rms_norm_eps"]
    r = cfg["compress_ratio"]
    cos, sin = rope_tables(positions, rd, cfg["compress_rope_theta"])   # position_embeddings["compress"]
    shared: dict = {}

    q_res = rms_norm(linear(x, params["wq_a.weight"]), params["q_norm.weight"], eps)
    q = linear(q_res, params["wq_b.weight"]).reshape(b, s, h, d)
    q = C.rope(q, cos[:, :, None], sin[:, :, None])                    # [B, S, H, D]
    kv = rms_norm(linear(x, params["wkv.weight"]), params["kv_norm.weight"], eps)
    kv = C.rope(kv, cos, sin)
    kv = Q.fake_quant_fp8_block(kv, 32)                                # attention.py:154
    if state is not None:                                              # cache.py:84-94
        win = kv if state.window is None else np.concatenate([state.window, kv], 1)
        state.window = win[:, -(w_ - 1):] if w_ > 1 else win[:, :0]
    else:
        win = kv
    win_pos0 = positions[0, 0] - (win.shape[1] - s)                    # absolute position of win[:, 0]

    latent, fgp = compressor(params, cfg, x, state)
    indexer(params, cfg, x, q_res, latent, fgp, positions, state, shared, select)
    if latent is not None:                                             # attention.py:173-192
        gpos = fgp + r * np.arange(latent.shape[1])
        cc, ss = rope_tables(np.broadcast_to(gpos, (b, len(gpos))), rd, cfg["compress_rope_theta"])
        rot = Q.fake_quant_fp4_block(C.rope(latent, cc, ss), 16, e4m3_scales=True)
        if state is not None:
            state.compressed = rot if state.compressed is None else np.concatenate([state.compressed, rot], 1)
            state.entry_count += rot.shape[1]
        else:
            shared["compress_kv"] = rot
    if state is not None:
        shared["compress_kv"] = state.compressed
    comp = shared.get("compress_kv")

    # mask: window band (attention.py / masking: k in (t - W, t]) then the selection
    t = positions[:, :, None]
    kpos = win_pos0 + np.arange(win.shape[1])[None, None, :]
    visible = (kpos <= t) & (kpos > t - w_)
    keys = win
    if comp is not None and comp.shape[1]:
        sel = shared.get("selection")
        if sel is None:
            sel = np.zeros((b, s, comp.shape[1]), bool)                # attention.py:208-214
        visible = np.concatenate([visible, sel], -1)
        keys = np.concatenate([win, comp], 1)
    bias = np.where(visible, F32(0), F32(-np.inf))[:, None]           # [B, 1, S, T]
    o, _ = OA._attend(_t(q).transpose(1, 2), _t(keys)[:, None], _t(keys)[:, None], _t(bias),
                      torch.as_tensor(params["attn_sink"]).float())
    o = C.rope(o.numpy(), cos[:, :, None], sin[:, :, None], inverse=True)   # attention.py:233
    og = cfg["o_groups"]
    grouped = _t(o).reshape(b, s, og, -1)                              # attention.py:20-39, :234-235
    wa = torch.as_tensor(params["wo_a.weight"]).float()
    wa = wa.view(og, -1, grouped.shape[-1]).transpose(1, 2)
    y = torch.bmm(grouped.reshape(-1, og, grouped.shape[-1]).transpose(0, 1), wa).transpose(0, 1)
    y = y.reshape(b, s, -1)
    out = y @ torch.as_tensor(params["wo_b.weight"]).float().T
    if state is not None:
        state.positions_seen += s
    return out.numpy(), shared
