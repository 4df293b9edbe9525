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
