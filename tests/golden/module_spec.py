"""Shared specification of the attention-module fixtures: configurations, seeded weights
and inputs.  Used by ``make_module_fixture.py`` (which runs the reference's module on the
CPU to write ``module_fixture.npz``) and by the tests that compare the oracle and the HIP
drop-in against that fixture, so all three see the same weights and activations.

Weights follow BASELINE config 1: every linear weight and the attention sink ~N(0, 0.02)
(``config.initializer_range``), RMSNorm weights at their init value 1; activations ~N(0, 1);
one ``torch.Generator`` seeded per configuration draws the weights in the sorted order of
the parameter names, then the hidden states.
"""

from __future__ import annotations

import torch

# Fields of DeepseekV41TextConfig the attention layer reads (owlet1/config.py:226-296).
# One layer that is both the KV source and the index source of its group, compress ratio r.
CONFIGS = {
    # small: every path (fake quant on, partial groups, top-k smaller than the visible
    # groups) at a size whose full outputs fit a small fixture
    "small": dict(hidden_size=96, num_attention_heads=4, head_dim=64, qk_rope_head_dim=16, q_lora_rank=48,
                  o_groups=2, o_lora_rank=32, index_n_heads=2, index_head_dim=32, index_topk=6,
                  compress_ratio=4, sliding_window=8, seq=45, batch=2, seed=1),
    # B1 S1024, 8 heads over a 128 + 32 latent, indexer 4 x 64, ratio 4,
    # top-128, window 64, fp32, seed 0 (hidden / low-rank sizes are not named by the config)
    "config1": dict(hidden_size=512, num_attention_heads=8, head_dim=160, qk_rope_head_dim=32, q_lora_rank=256,
                    o_groups=2, o_lora_rank=128, index_n_heads=4, index_head_dim=64, index_topk=128,
                    compress_ratio=4, sliding_window=64, seq=1024, batch=1, seed=0),
}
ROPE_THETA = 10000.0
COMPRESS_ROPE_THETA = 160000.0
RMS_NORM_EPS = 1e-20  # owlet1/config.py:296 default


def param_shapes(c: dict) -> dict[str, tuple]:
    """name -> shape of every parameter of DeepseekV41Attention for a KV + index source
    layer (owlet1/attention.py:106-127, cache.py:134-140, indexer.py:63-76)."""
    h, d, hid, ql = c["num_attention_heads"], c["head_dim"], c["hidden_size"], c["q_lora_rank"]
    hi, di, og, orank = c["index_n_heads"], c["index_head_dim"], c["o_groups"], c["o_lora_rank"]
    return {
        "wq_a.weight": (ql, hid), "q_norm.weight": (ql,), "wq_b.weight": (h * d, ql),
        "wkv.weight": (d, hid), "kv_norm.weight": (d,),
        "wo_a.weight": (og * orank, h * d // og), "wo_b.weight": (hid, og * orank), "attn_sink": (h,),
        "compressor.wkv.weight": (d, hid), "compressor.wgate.weight": (d, hid), "compressor.norm.weight": (d,),
        "indexer.wq_b.weight": (hi * di, ql), "indexer.weights_proj.weight": (hi, hid),
        "indexer.wk.weight": (di, d), "indexer.k_norm.weight": (di,),
    }


def make_params_and_inputs(c: dict):
    """(params {name: fp32 tensor}, hidden_states [B, S, hidden] fp32, position_ids [B, S])."""
    g = torch.Generator().manual_seed(c["seed"])
    params = {}
    for name, shape in sorted(param_shapes(c).items()):
        if name.endswith("norm.weight"):
            params[name] = torch.ones(shape)
        else:
            params[name] = torch.randn(shape, generator=g) * 0.02
    x = torch.randn(c["batch"], c["seq"], c["hidden_size"], generator=g)
    pos = torch.arange(c["seq"]).unsqueeze(0).expand(c["batch"], -1).contiguous()
    return params, x, pos


def chunks(c: dict) -> list[int]:
    """How the cached run feeds the sequence: two prefill chunks that end mid-group, then
    one-token decode steps (exercises the partial-group carry, cache.py:96-113)."""
    s = c["seq"]
    first = s // 2 + 1
    second = s - first - 6
    return [first, second] + [1] * 6


# ---- multi-layer schedules ------------------------------------------------------------------
# Layers of one forward share a single ``shared`` dict (the reference decoder passes one per
# forward to every layer, owlet1/decoder.py:318-330); each layer gets its own hidden-state
# input, since the decoder's residual streams and FFNs around the attention are outside this
# path.  Layer roles follow owlet1/config.py:323-404: ratio 0 = sliding window only ("main"
# RoPE); a KV source owns the group's compressor (ratio 1: no gate, cache.py:148-151); an
# index source runs the indexer (it owns the keys when it is also the KV source, else it is
# a "Reindex" layer scoring the source's keys, indexer.py:49-60); other layers with a ratio
# "Reuse" the group's compressed cache and selection (attention.py:83-89, :171, :198); the
# candidate source publishes the two-level candidate mask every later index source scores
# inside (indexer.py:145-152).
STACKS = {
    # archs/dsv4/model_test.py:76-97's schedule: a sliding-only layer, a ratio-2 group (its
    # source, then a Reuse layer), a ratio-1 group (its own source)
    "two_groups": dict(CONFIGS["small"], compress_ratios=[0, 2, 2, 1], kv_source_layer_ids=[1, 3],
                       index_source_layer_ids=[1, 3], candidate_source_layer_id=-1, seed=11),
    # one ratio-4 group: the source is also the candidate source; a Reuse layer; a Reindex
    # layer that scores inside the candidates; a Reuse layer of the Reindex selection
    "reindex": dict(CONFIGS["small"], compress_ratios=[0, 4, 4, 4, 4], kv_source_layer_ids=[1],
                    index_source_layer_ids=[1, 3], candidate_source_layer_id=1, candidate_topk_blocks=3,
                    candidate_block_size=2, index_topk=4, seq=61, seed=12),
    # the two-group schedule on a left-padded batch: row 1's first `pad` tokens are padding
    # (the model's 2-D attention mask is 0 there), so the sliding causal mask also masks them
    "padded": dict(CONFIGS["small"], compress_ratios=[0, 2, 2, 1], kv_source_layer_ids=[1, 3],
                   index_source_layer_ids=[1, 3], candidate_source_layer_id=-1, pad=[0, 5], seed=13),
}


def role(c: dict, i: int) -> dict:
    """The role flags of layer i of a schedule (owlet1/attention.py:95-127, indexer.py:60-64)."""
    kv, ix = c["kv_source_layer_ids"], c["index_source_layer_ids"]
    cand = c.get("candidate_source_layer_id", -1)
    return dict(ratio=c["compress_ratios"][i], kv_source=i in kv, index_source=i in ix,
                owns_k=i in kv and i in ix, candidate_source=i == cand, uses_candidates=0 <= cand < i)


def layer_param_shapes(c: dict, i: int) -> dict[str, tuple]:
    """name -> shape of every parameter of DeepseekV41Attention(config, i): the common
    projections, the compressor on a KV source (no gate at ratio 1), the indexer on an index
    source (its key projection only when it owns the keys)."""
    r = role(c, i)
    shapes = {k: v for k, v in param_shapes(c).items() if not k.startswith(("compressor.", "indexer."))}
    h, d, hid, ql = c["num_attention_heads"], c["head_dim"], c["hidden_size"], c["q_lora_rank"]
    hi, di = c["index_n_heads"], c["index_head_dim"]
    if r["kv_source"]:
        shapes.update({"compressor.wkv.weight": (d, hid), "compressor.norm.weight": (d,)})
        if r["ratio"] > 1:
            shapes["compressor.wgate.weight"] = (d, hid)
    if r["index_source"]:
        shapes.update({"indexer.wq_b.weight": (hi * di, ql), "indexer.weights_proj.weight": (hi, hid)})
        if r["owns_k"]:
            shapes.update({"indexer.wk.weight": (di, d), "indexer.k_norm.weight": (di,)})
    return shapes


def make_stack_params_and_inputs(c: dict):
    """([params of layer i], [hidden_states of layer i] fp32 [B, S, hidden], position_ids
    [B, S], liveness [B, S] bool or None).  One generator draws every layer's weights (layer
    order, names sorted) and then every layer's input."""
    g = torch.Generator().manual_seed(c["seed"])
    n = len(c["compress_ratios"])
    params = []
    for i in range(n):
        p = {}
        for name, shape in sorted(layer_param_shapes(c, i).items()):
            p[name] = torch.ones(shape) if name.endswith("norm.weight") else torch.randn(shape, generator=g) * 0.02
        params.append(p)
    xs = [torch.randn(c["batch"], c["seq"], c["hidden_size"], generator=g) for _ in range(n)]
    pos = torch.arange(c["seq"]).unsqueeze(0).expand(c["batch"], -1).contiguous()
    live = None
    if c.get("pad"):
        live = torch.ones(c["batch"], c["seq"], dtype=torch.bool)
        for b, p in enumerate(c["pad"]):
            live[b, :p] = False
    return params, xs, pos, live
