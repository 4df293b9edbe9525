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

For each multi-layer schedule of ``module_spec.STACKS`` (sliding-only layers, KV + index
sources at ratios 1, 2 and 4, Reuse and Reindex layers, a candidate source and user, a
left-padded batch) the reference's modules run layer by layer on per-layer inputs with one
``shared`` dict per forward, as the reference decoder passes it (owlet1/decoder.py:318-330):

* no cache: every layer's output, each index source's selection, the candidate mask, the
  model's sliding causal mask (create_sliding_window_causal_mask, with the padding);
* through per-layer caches (DeepseekV41CSACache on KV sources, the sliding window on the
  others) in ``module_spec.chunks`` calls: every layer's outputs, selections, candidate
  masks and each call's mask, then every layer's window and each source's group state.

Large outputs (config 1) are kept for sampled rows only; the selections, candidate masks and
masks of every row are stored as packed bits.
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
    from transformers.cache_utils import Cache, DynamicSlidingWindowLayer
    from transformers.masking_utils import create_sliding_window_causal_mask

    from mzoo.archs.owlet1.attention import DeepseekV41Attention
    from mzoo.archs.owlet1.cache import DeepseekV41CSACache
    from mzoo.archs.owlet1.config import DeepseekV41TextConfig
    from mzoo.archs.owlet1.norm_rope import DeepseekV41RotaryEmbedding
    return dict(Cache=Cache, mask=create_sliding_window_causal_mask, Attention=DeepseekV41Attention,
                CSACache=DeepseekV41CSACache, Config=DeepseekV41TextConfig, Rotary=DeepseekV41RotaryEmbedding,
                Sliding=DynamicSlidingWindowLayer)


def _config(R, c, stack=False):
    n = len(c["compress_ratios"]) if stack else 1
    cfg = R["Config"](
        vocab_size=64, hidden_size=c["hidden_size"], num_hidden_layers=n,
        num_attention_heads=c["num_attention_heads"], head_dim=c["head_dim"],
        qk_rope_head_dim=c["qk_rope_head_dim"], q_lora_rank=c["q_lora_rank"], o_lora_rank=c["o_lora_rank"],
        o_groups=c["o_groups"],
        compress_ratios=list(c["compress_ratios"]) if stack else [c["compress_ratio"]],
        kv_source_layer_ids=list(c["kv_source_layer_ids"]) if stack else [0],
        index_source_layer_ids=list(c["index_source_layer_ids"]) if stack else [0],
        candidate_source_layer_id=c.get("candidate_source_layer_id", -1) if stack else -1,
        candidate_topk_blocks=c.get("candidate_topk_blocks", 2048), candidate_block_size=c.get("candidate_block_size", 8),
        sliding_window=c["sliding_window"],
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


# ---- multi-layer schedules ------------------------------------------------------------------

# The reset a KV-source layer applies to `shared` when there is no cache: the reference's
# dsv4 module does it (archs/dsv4/modeling_deepseek_v41.py:722-732, tickets/done/0012), the
# owlet1 split lists it as an open upstream gap (archs/owlet1/GAPS.md, item 2) and without it
# a second group's layers append to the first group's compressed entries and keys.  Applied
# here, outside the owlet1 module, so the no-cache run is the one the cached run must equal.
_RESET = ("compress_kv", "index_k", "topk_bias", "candidates")


def _stack_forward(R, cfg, mods, rot, xs, pos, cache, live):
    pe = {"main": rot(xs[0], pos, layer_type="main"), "compress": rot(xs[0], pos, layer_type="compress")}
    mask = R["mask"](config=cfg, inputs_embeds=xs[0], attention_mask=live, past_key_values=cache, position_ids=pos)
    shared, outs, sels = {}, [], {"mask": mask}
    for i, mod in enumerate(mods):
        if cache is None and mod.is_kv_source:
            for key in _RESET:
                shared.pop(key, None)
        with torch.no_grad():
            out, _ = mod(xs[i], position_embeddings=pe, attention_mask=mask, past_key_values=cache, shared=shared,
                         position_ids=pos)
        outs.append(out)
        if mod.is_index_source:
            sels[i] = shared.get("topk_bias")
            if mod.indexer.is_candidate_source:
                sels["candidates"] = shared.get("candidates")
    return outs, sels


def run_stack(name: str, R) -> dict:
    c = spec.STACKS[name]
    cfg = _config(R, c, stack=True)
    params, xs, pos, live = spec.make_stack_params_and_inputs(c)
    n_layers = len(c["compress_ratios"])
    mods = []
    for i in range(n_layers):
        mod = R["Attention"](cfg, i).eval()
        names = dict(mod.named_parameters())
        assert set(names) == set(params[i]), (i, sorted(set(names) ^ set(params[i])))
        with torch.no_grad():
            for k, v in params[i].items():
                assert tuple(names[k].shape) == tuple(v.shape), (i, k, names[k].shape, v.shape)
                names[k].copy_(v)
        mods.append(mod)
    rot = R["Rotary"](cfg)
    b, s = c["batch"], c["seq"]

    def groups(i):
        r = c["compress_ratios"][i]
        return s // r if r else 0

    rec = {}
    outs, sels = _stack_forward(R, cfg, mods, rot, xs, pos, None, live)
    rec["nocache_out"] = torch.stack(outs)
    rec["nocache_mask"] = sels.pop("mask")[:, 0] == 0
    cand = sels.pop("candidates", None)
    for i, bias in sels.items():
        rec[f"nocache_sel{i}"] = _sel_of(bias, s, groups(i))
    if cand is not None:
        rec["nocache_candidates"] = cand

    cache = R["Cache"](layers=[R["CSACache"](cfg) if t == "shared_compressed_attention"
                               else R["Sliding"](sliding_window=cfg.sliding_window) for t in cfg.layer_types])
    call_outs, call_sels, call_cand, start, call = [], {i: [] for i in sels}, [], 0, 0
    for n in spec.chunks(c):
        lv = None if live is None else live[:, :start + n]
        o, sl = _stack_forward(R, cfg, mods, rot, [x[:, start:start + n] for x in xs], pos[:, start:start + n],
                               cache, lv)
        call_outs.append(torch.stack(o))
        rec[f"cached_mask{call}"] = sl.pop("mask")[:, 0] == 0
        call += 1
        for i in call_sels:
            call_sels[i].append(_sel_of(sl.get(i), n, groups(i)))
        if cand is not None:
            m = torch.zeros(b, n, groups(c["candidate_source_layer_id"]), dtype=torch.bool)
            if sl.get("candidates") is not None:
                m[..., :sl["candidates"].shape[-1]] = sl["candidates"]
            call_cand.append(m)
        start += n
    rec["cached_out"] = torch.cat(call_outs, 2)
    if call_cand:
        rec["cached_candidates"] = torch.cat(call_cand, 1)
    for i, v in call_sels.items():
        rec[f"cached_sel{i}"] = torch.cat(v, 1)
    for i, layer in enumerate(cache.layers):
        rec[f"cached_window{i}"] = layer.keys[:, 0]
        if i in c["kv_source_layer_ids"]:
            rec[f"cached_compress_kv{i}"] = layer.compressed_kv["compressor"][:, 0]
            if layer.compressed_kv["indexer"] is not None:
                rec[f"cached_index_k{i}"] = layer.compressed_kv["indexer"][:, 0]
            rec[f"cached_entry_count{i}"] = torch.tensor(layer.entry_count["compressor"])
            if layer.buffer_kv["compressor"] is not None:
                rec[f"cached_buffer_kv{i}"] = layer.buffer_kv["compressor"]

    arrays = {}
    for k, v in rec.items():
        v = v.detach()
        if "_sel" in k or k.endswith("_candidates") or "_mask" in k:
            arrays[k] = np.packbits(v.numpy().astype(np.uint8), axis=-1)
        else:
            arrays[k] = v.float().numpy()
    return {f"{name}/{k}": a for k, a in arrays.items()}


def _sel_of(bias, seq, groups):
    """bool [B, S, groups] of a published bias (the kept entries), zero-padded to `groups`."""
    if bias is None:
        return torch.zeros(1, seq, groups, dtype=torch.bool)
    sel = bias[:, 0] == 0
    out = torch.zeros(sel.shape[0], seq, groups, dtype=torch.bool)
    out[:, :, :sel.shape[-1]] = sel
    return out


def main() -> None:
    R = _reference()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    out = {}
    for name in spec.CONFIGS:
        out.update(run(name, R))
        print(f"{name}: done", flush=True)
    for name in spec.STACKS:
        out.update(run_stack(name, R))
        print(f"stack {name}: done", flush=True)
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
