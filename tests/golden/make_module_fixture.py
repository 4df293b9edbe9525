"""Write ``module_fixture.npz``: the reference's own ``DeepseekV41Attention`` (with its
compressor, indexer and cache layer) run on the CPU in this container, for the inputs of
``module_spec.py``.

Why an import: the module's composition -- the ``shared`` protocol, the mask extension by
``topk_bias``, the compressed-RoPE positions, the inverse RoPE and grouped output
projection, and the compressor's partial-group carry across calls -- has no closed form
or invariant that pins a restatement of it (``owlet1/attention.py:129-236``,
``owlet1/cache.py:84-172``, ``owlet1/indexer.py:78-165``).  The reference is imported only
here, only to write this data file; nothing that runs on the GPU box reads the reference.

Run from the repository root:  python tests/golden/make_module_fixture.py
The reference lives at /root/reference (MZOO_REFERENCE overrides).  Recorded per
configuration of ``module_spec.CONFIGS``:

* no cache, one forward over the whole sequence: the layer output, the top-k selection
  (the finite entries of ``shared["topk_bias"]``), the published indexer keys and
  compressed latents (``shared["index_k"]``, ``shared["compress_kv"]``);
* with a cache layer, the sequence fed in ``module_spec.chunks`` calls: every call's
  output, the per-call selections, and the final cache state (indexer keys, compressed
  latents, the window, the group count and the carried partial group).

Large outputs (config 1) are kept for sampled rows only; the selections of every row are
stored as packed bits.
"""

from __future__ import annotations

import json
import os
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import module_spec as spec  # noqa: E402

REF_SRC = pathlib.Path(os.environ.get("MZOO_REFERENCE", "/root/reference")) / "src"
SAMPLE_ROWS = [0, 1, 2, 3, 4, 62, 63, 64, 65, 127, 128, 255, 256, 511, 512, 513, 700, 1000, 1022, 1023]


def _reference():
    sys.path.insert(0, str(REF_SRC))
    from transformers.cache_utils import Cache
    from transformers.masking_utils import create_sliding_window_causal_mask

    from mzoo.archs.owlet1.attention import DeepseekV41Attention
    from mzoo.archs.owlet1.cache import DeepseekV41CSACache
    from mzoo.archs.owlet1.config import DeepseekV41TextConfig
    from mzoo.archs.owlet1.norm_rope import DeepseekV41RotaryEmbedding
    return dict(Cache=Cache, mask=create_sliding_window_causal_mask, Attention=DeepseekV41Attention,
                CSACache=DeepseekV41CSACache, Config=DeepseekV41TextConfig, Rotary=DeepseekV41RotaryEmbedding)


def _config(R, c):
    cfg = R["Config"](
        vocab_size=64, hidden_size=c["hidden_size"], num_hidden_layers=1,
        num_attention_heads=c["num_attention_heads"], head_dim=c["head_dim"],
        qk_rope_head_dim=c["qk_rope_head_dim"], q_lora_rank=c["q_lora_rank"], o_lora_rank=c["o_lora_rank"],
        o_groups=c["o_groups"], compress_ratios=[c["compress_ratio"]], kv_source_layer_ids=[0],
        index_source_layer_ids=[0], candidate_source_layer_id=-1, sliding_window=c["sliding_window"],
        index_n_heads=c["index_n_heads"], index_head_dim=c["index_head_dim"], index_topk=c["index_topk"],
        rope_theta=spec.ROPE_THETA, compress_rope_theta=spec.COMPRESS_ROPE_THETA, rms_norm_eps=spec.RMS_NORM_EPS,
        moe_intermediate_size=16, n_routed_experts=1, num_experts_per_tok=1, n_shared_experts=1,
        num_nextn_predict_layers=0, use_cache=False, dspark_noise_token_id=0, tie_word_embeddings=True,
        bos_token_id=0, eos_token_id=1, max_position_embeddings=1 << 16,
    )
    cfg._attn_implementation = "eager"
    return cfg


def _selection(shared, seq, groups):
    """bool [B, S, groups]: the entries the indexer kept (zero bias), padded to `groups`."""
    bias = shared.get("topk_bias")
    if bias is None:
        return None
    sel = (bias[:, 0] == 0)
    out = torch.zeros(sel.shape[0], seq, groups, dtype=torch.bool)
    out[:, :, :sel.shape[-1]] = sel
    return out


def _forward(R, cfg, mod, rot, x, pos, cache):
    pe = {"main": rot(x, pos, layer_type="main"), "compress": rot(x, pos, layer_type="compress")}
    mask = R["mask"](config=cfg, inputs_embeds=x, attention_mask=None, past_key_values=cache, position_ids=pos)
    shared = {}
    with torch.no_grad():
        out, _ = mod(x, position_embeddings=pe, attention_mask=mask, past_key_values=cache, shared=shared,
                     position_ids=pos)
    return out, shared


def run(name: str, R) -> dict:
    c = spec.CONFIGS[name]
    cfg = _config(R, c)
    mod = R["Attention"](cfg, 0).eval()
    params, x, pos = spec.make_params_and_inputs(c)
    names = dict(mod.named_parameters())
    assert set(names) == set(params), (sorted(set(names) ^ set(params)))
    with torch.no_grad():
        for k, v in params.items():
            assert tuple(names[k].shape) == tuple(v.shape), (k, names[k].shape, v.shape)
            names[k].copy_(v)
    rot = R["Rotary"](cfg)
    groups = c["seq"] // c["compress_ratio"]
    rec = {}

    out, shared = _forward(R, cfg, mod, rot, x, pos, None)
    rec["nocache_out"] = out
    rec["nocache_sel"] = _selection(shared, c["seq"], groups)
    rec["nocache_index_k"] = shared["index_k"][:, 0]
    rec["nocache_compress_kv"] = shared["compress_kv"][:, 0]

    cache = R["Cache"](layers=[R["CSACache"](cfg)])
    outs, sels, start = [], [], 0
    for n in spec.chunks(c):
        o, sh = _forward(R, cfg, mod, rot, x[:, start:start + n], pos[:, start:start + n], cache)
        outs.append(o)
        s = _selection(sh, n, groups)
        sels.append(s if s is not None else torch.zeros(c["batch"], n, groups, dtype=torch.bool))
        start += n
    layer = cache.layers[0]
    rec["cached_out"] = torch.cat(outs, 1)
    rec["cached_sel"] = torch.cat(sels, 1)
    rec["cached_index_k"] = layer.compressed_kv["indexer"][:, 0]
    rec["cached_compress_kv"] = layer.compressed_kv["compressor"][:, 0]
    rec["cached_window"] = layer.keys[:, 0]
    rec["cached_entry_count"] = torch.tensor(layer.entry_count["compressor"])
    rec["cached_buffer_kv"] = layer.buffer_kv["compressor"]
    rec["cached_buffer_gate"] = layer.buffer_gate["compressor"]

    arrays = {}
    for k, v in rec.items():
        v = v.detach()
        if k.endswith("_sel"):
            arrays[k] = np.packbits(v.numpy().astype(np.uint8), axis=-1)
        elif name == "config1" and k.endswith("_out"):
            arrays[k] = v[:, SAMPLE_ROWS].float().numpy()
        elif name == "config1" and (k.endswith("compress_kv") or k.startswith("cached_buffer")):
            continue  # large; the small configuration records them in full
        else:
            arrays[k] = v.float().numpy()
    if name == "config1":
        arrays["sample_rows"] = np.array(SAMPLE_ROWS, np.int64)
    return {f"{name}/{k}": a for k, a in arrays.items()}


def main() -> None:
    R = _reference()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    out = {}
    for name in spec.CONFIGS:
        out.update(run(name, R))
        print(f"{name}: done", flush=True)
    out["about"] = np.frombuffer(json.dumps({
        "writer": "tests/golden/make_module_fixture.py",
        "reference": "pmonad/mzoo src/mzoo/archs/owlet1 (attention.py, cache.py, indexer.py, norm_rope.py, quant.py)",
        "torch": torch.__version__,
    }).encode(), dtype=np.uint8)
    path = HERE / "module_fixture.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
