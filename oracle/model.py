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
``sliding_window``, ``rms_norm_eps``, ``compress_rope_theta``, optionally ``compress_yarn``:
the compress rope's YaRN settings, see ``rope_tables``); ``params`` maps the
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


def rope_tables(positions, rope_dim: int, theta: float, yarn: dict | None = None) -> tuple[np.ndarray, np.ndarray]:
    """``DeepseekV41RotaryEmbedding.forward`` (norm_rope.py:108-124): ``inv_freq = 1 /
    theta^(arange(0, rd, 2) / rd)`` for the default RoPE (dsv4 modeling_deepseek_v41.py:127-137,
    ``dim = int(head_dim * partial_rotary_factor)`` = qk_rope_head_dim), or, with ``yarn`` (the
    compress rope's YaRN settings, owlet1/config.py:419-434), the frequencies and attention
    factor of the library routine the reference calls for it (transformers'
    ``ROPE_INIT_FUNCTIONS["yarn"]``, norm_rope.py:70-73); then ``(inv_freq @ positions).T``
    cos / sin in float32, times the attention factor -> [..., rd/2]."""
    scale = 1.0
    if yarn is None:
        inv = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float) / rope_dim))
    else:
        inv, scale = _yarn_library(theta, rope_dim, yarn)
    pos = torch.as_tensor(np.array(positions, np.float32))
    freqs = (inv.view(-1, 1) @ pos.reshape(1, -1)).T.reshape(*pos.shape, -1)
    return (freqs.cos() * scale).numpy(), (freqs.sin() * scale).numpy()


def _yarn_library(theta: float, rope_dim: int, yarn: dict):
    """transformers' YaRN frequencies for a rope of ``rope_dim`` channels (a config whose
    head_dim is rope_dim, partial factor 1); ``yarn`` holds the rope_parameters sub-dict keys
    (factor, original_max_position_embeddings, beta_fast, beta_slow, attention_factor, mscale,
    mscale_all_dim) and optionally ``truncate`` (top level of rope_parameters, where the library
    reads it) and ``max_position_embeddings``."""
    from transformers import PretrainedConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    sub = {k: v for k, v in yarn.items() if k not in ("truncate", "max_position_embeddings")}
    sub.update(rope_type="yarn", rope_theta=theta, partial_rotary_factor=1.0)
    rp = {"compress": sub}
    if "truncate" in yarn:
        rp["truncate"] = yarn["truncate"]
    c = PretrainedConfig(head_dim=rope_dim, hidden_size=rope_dim, num_attention_heads=1,
                         max_position_embeddings=yarn.get("max_position_embeddings", 1 << 20), rope_parameters=rp)
    inv, scale = ROPE_INIT_FUNCTIONS["yarn"](c, None, layer_type="compress")
    return inv.float(), float(scale)


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
    """cache.py:142-172.  Ratio > 1 pools with the softmax gate (fp32); ratio 1 is the plain
    per-token projection + norm (no gate, cache.py:148-151).  Returns (pre-RoPE latent
    [B, n, D] or None, first_group_position)."""
    r = cfg["compress_ratio"]
    if r == 1:                                                         # cache.py:148-151
        latent = rms_norm(linear(x, params["compressor.wkv.weight"]), params["compressor.norm.weight"],
                          cfg["rms_norm_eps"])
        fgp = 0 if state is None else state.entry_count
        return latent, fgp
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


def indexer(params, cfg, x, q_residual, latent, fgp, positions, state, shared, select=None, *, owns_k=True,
            candidate_source=False, uses_candidates=False, candidates=None):
    """indexer.py:78-165.  An index source that owns its keys publishes the keys of the
    groups completed in this call (``:96-117``); a Reindex layer (``owns_k=False``) scores
    the keys its group's source published in this forward.  Scores (``:124-133``),
    visibility (``:141-143``), the two-level candidates (``:145-152``: the candidate source
    publishes ``shared["candidates"]``, a later index source scores inside it; ``candidates``
    imposes the candidate source's mask), top-k (``:158-165``).  Publishes ``shared["index_k"]``, ``shared["selection"]`` (bool
    [B, S, G]) and ``shared["scores"]``."""
    b, s, _ = x.shape
    r, hi, di = cfg["compress_ratio"], cfg["index_n_heads"], cfg["index_head_dim"]
    rd = cfg["qk_rope_head_dim"]
    theta = cfg["compress_rope_theta"]
    if owns_k:
        if latent is not None:                                        # indexer.py:96-117
            k = rms_norm(linear(latent, params["indexer.wk.weight"]), params["indexer.k_norm.weight"],
                         cfg["rms_norm_eps"])
            gpos = fgp + r * np.arange(latent.shape[1])
            cos, sin = rope_tables(np.broadcast_to(gpos, (b, len(gpos))), rd, theta, cfg.get("compress_yarn"))
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
    cos_q, sin_q = rope_tables(positions, rd, theta, cfg.get("compress_yarn"))  # indexer.py:124-126
    q = linear(q_residual, params["indexer.wq_b.weight"]).reshape(b, s, hi, di)
    q = C.rope(q, cos_q[:, :, None], sin_q[:, :, None])
    q = Q.fake_quant_fp4_block(q, 32)
    w = linear(x, params["indexer.weights_proj.weight"]) * F32(hi ** -0.5)
    scores = OA.indexer_scores(_t(q), _t(index_k), _t(w), r, torch.as_tensor(positions))
    if candidate_source:                                              # indexer.py:147-150
        lens = (np.asarray(positions, np.int64)[..., None] + 1) // r
        shared["candidates"] = OA.select_candidate_blocks(scores, lens, cfg["candidate_topk_blocks"],
                                                          cfg["candidate_block_size"])
        if candidates is not None:
            shared["candidates"] = np.asarray(candidates, bool)[..., :g]
    elif uses_candidates and shared.get("candidates") is not None:    # indexer.py:151-152
        scores = scores.masked_fill(~torch.as_tensor(np.asarray(shared["candidates"], bool)), float("-inf"))
    shared["scores"] = scores
    # the magnitude the scores' rounding scales with (the indexer tolerance's basis)
    shared["abs_scores"] = OA.indexer_abs_scores(_t(q), _t(index_k), _t(w), r, torch.as_tensor(positions))
    if select is None:                                                # indexer.py:158-165
        idx = OA.topk_indices(scores, min(cfg["index_topk"], g))
        sel = np.zeros((b, s, g + 1), bool)
        np.put_along_axis(sel, np.where(idx < 0, g, idx), True, -1)
        select = sel[..., :g]
    shared["selection"] = np.asarray(select, bool)[..., :g]


# keys a KV-source layer drops from `shared` when there is no cache: each group starts
# fresh (archs/dsv4/modeling_deepseek_v41.py:722-732; tickets/done/0012)
_GROUP_KEYS = ("compress_kv", "index_k", "selection", "scores", "abs_scores", "candidates")


def role(cfg, i: int) -> dict:
    """Layer i's role in a schedule (owlet1/attention.py:95-127, indexer.py:60-64)."""
    kv, ix = cfg["kv_source_layer_ids"], cfg["index_source_layer_ids"]
    cand = cfg.get("candidate_source_layer_id", -1)
    cand = -1 if cand is None else cand
    return dict(ratio=cfg["compress_ratios"][i], kv_source=i in kv, index_source=i in ix,
                owns_k=i in kv and i in ix, candidate_source=i == cand, uses_candidates=0 <= cand < i)


def attention_layer(params, cfg, i: int, x, positions, state: LayerState | None, shared: dict, live=None,
                    select=None, candidates=None):
    """attention.py:129-236 for layer i of the schedule ``cfg`` (one layer of a forward
    whose layers share ``shared``).  x [B, S, hidden] fp32; positions [B, S] absolute (the
    running token count); ``state`` the layer's cache (window for every layer, group state
    on a KV source) for a cached call; ``live`` bool [B, T] the liveness of every token seen
    so far (the model's 2-D attention mask; None = all live); ``select`` an imposed
    selection for an index source, ``candidates`` an imposed candidate mask for the candidate
    source (the reference's ``torch.topk`` breaks ties between equal block scores in its own
    order).  Returns out [B, S, hidden]."""
    x = _np(x)
    positions = np.asarray(positions, np.int64)
    b, s, _ = x.shape
    ro = role(cfg, i)
    r = ro["ratio"]
    h, d, rd, w_ = cfg["num_attention_heads"], cfg["head_dim"], cfg["qk_rope_head_dim"], cfg["sliding_window"]
    eps = cfg["rms_norm_eps"]
    lcfg = dict(cfg, compress_ratio=r)
    theta = cfg["compress_rope_theta"] if r else cfg.get("rope_theta", 10000.0)   # attention.py:100, :143
    cos, sin = rope_tables(positions, rd, theta, cfg.get("compress_yarn") if r else None)

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
    seen = state.positions_seen if state is not None else 0            # running index of this call's first token
    win0 = seen + s - win.shape[1]                                     # running index of win[:, 0]

    keys = win
    sel = None
    comp = None
    if r:
        if ro["kv_source"] and state is None:
            for key in _GROUP_KEYS:
                shared.pop(key, None)
        latent, fgp = (None, 0)
        if ro["kv_source"]:
            latent, fgp = compressor(params, lcfg, x, state)
        if ro["index_source"]:
            indexer(params, lcfg, x, q_res, latent, fgp, positions, state, shared, select, owns_k=ro["owns_k"],
                    candidate_source=ro["candidate_source"], uses_candidates=ro["uses_candidates"],
                    candidates=candidates)
        sel = shared.get("selection")
        if latent is not None:                                         # attention.py:173-192
            gpos = fgp + r * np.arange(latent.shape[1])
            cc, ss = rope_tables(np.broadcast_to(gpos, (b, len(gpos))), rd, cfg["compress_rope_theta"],
                                 cfg.get("compress_yarn"))
            rot = Q.fake_quant_fp4_block(C.rope(latent, cc, ss), 16, e4m3_scales=True)
            if state is not None:
                state.compressed = rot if state.compressed is None else np.concatenate([state.compressed, rot], 1)
                state.entry_count += rot.shape[1]
            else:
                shared["compress_kv"] = rot if shared.get("compress_kv") is None else np.concatenate(
                    [shared["compress_kv"], rot], 1)
        if ro["kv_source"] and state is not None:
            shared["compress_kv"] = state.compressed
        comp = shared.get("compress_kv")

    # mask: the model's sliding causal mask over the running token index (k in (t - W, t],
    # the key live), then the selection (attention.py:202-214)
    t = seen + np.arange(s)[None, :, None]
    kpos = win0 + np.arange(win.shape[1])[None, None, :]
    visible = (kpos <= t) & (kpos > t - w_)
    if live is not None:
        lv = np.asarray(live, bool)
        visible = visible & lv[:, kpos[0, 0]][:, None, :]
    visible = np.broadcast_to(visible, (b, s, win.shape[1]))
    if comp is not None and comp.shape[1]:
        if sel is None or sel.shape[-1] != comp.shape[1]:
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
    return out.numpy()


def stack_forward(params, cfg, xs, positions, states=None, live=None, select=None, candidates=None):
    """One forward of a layer schedule: layer i of ``cfg`` (``compress_ratios``,
    ``kv_source_layer_ids``, ``index_source_layer_ids``, ``candidate_source_layer_id``, ...)
    runs on its own input ``xs[i]`` with ``params[i]``; the layers share one ``shared`` dict,
    as the reference decoder passes one per forward (owlet1/decoder.py:318-330).  ``states``
    a list of LayerState (a cached call) or None; ``select`` {layer: imposed selection};
    ``candidates`` an imposed candidate mask for the candidate source.
    Returns (outs [layers] of [B, S, hidden], {layer: what the layer's indexer published})."""
    shared: dict = {}
    outs, published = [], {}
    for i in range(len(cfg["compress_ratios"])):
        st = None if states is None else states[i]
        outs.append(attention_layer(params[i], cfg, i, xs[i], positions, st, shared, live,
                                    None if select is None else select.get(i), candidates))
        if role(cfg, i)["index_source"]:
            published[i] = {k: shared.get(k) for k in ("selection", "scores", "abs_scores", "index_k", "candidates")}
    return outs, published


def layer_forward(params, cfg, x, positions, state: LayerState | None = None, select=None):
    """attention.py:129-236 for a layer that is its group's KV and index source (ratio
    ``cfg["compress_ratio"]``).  x [B, S, hidden] fp32, positions [B, S] absolute; ``state``
    (LayerState) for a cached call.  Returns (out [B, S, hidden], shared) with
    ``shared["selection"]`` the compressed entries each query attended."""
    one = dict(cfg, compress_ratios=[cfg["compress_ratio"]], kv_source_layer_ids=[0], index_source_layer_ids=[0],
               candidate_source_layer_id=-1)
    shared: dict = {}
    out = attention_layer(params, one, 0, x, positions, state, shared, None, select)
    return out, shared
