"""GPU: the module drop-ins (mzoo_amd/owlet1.py) as a multi-layer schedule.

Each schedule of ``tests/golden/module_spec.STACKS`` runs layer by layer on per-layer inputs
with one ``shared`` dict per forward (owlet1/decoder.py:318-330): sliding-only layers, KV +
index sources at ratios 1, 2 and 4 (the ratio-1 compressor has no gate), Reuse layers that
read their group's compressed cache and selection, a Reindex layer scoring the source's keys
inside the candidate source's blocks, a Reuse layer of the Reindex selection, and a
left-padded batch.  The model's mask is the one the reference built (recorded in the
fixture).  Checked for every layer, without a cache and through per-layer caches (two
prefill chunks ending mid-group, then decode steps):

* against the oracle (oracle/model.py) with the GPU's selections and candidate mask
  imposed, on every row: the attention bar;
* the selections against the oracle's top-k up to near-ties of the k-th score, the
  candidate blocks against the oracle's up to near-ties of the weakest block kept;
* against the reference's own modules (fixture) on the rows whose selection is the
  reference's;
* cache == no cache on the rows whose selections agree;
* the mask-free path (the sliding window in token order) against the mask path.
"""

import pathlib
import sys

import numpy as np
import pytest
import torch

from mzoo_amd import owlet1 as MO
from oracle import model as OM
from tests.helpers import ATTN_COS_MIN, ATTN_MAXABS, SCORE_RTOL, cosine

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))
import module_spec as spec  # noqa: E402

pytestmark = pytest.mark.gpu
FIX = np.load(HERE / "golden" / "module_fixture.npz")


def _config(c):
    return MO.AttentionConfig(
        hidden_size=c["hidden_size"], num_attention_heads=c["num_attention_heads"], head_dim=c["head_dim"],
        qk_rope_head_dim=c["qk_rope_head_dim"], q_lora_rank=c["q_lora_rank"], o_groups=c["o_groups"],
        o_lora_rank=c["o_lora_rank"], rope_theta=spec.ROPE_THETA, compress_rope_theta=spec.COMPRESS_ROPE_THETA,
        sliding_window=c["sliding_window"], compress_ratios=list(c["compress_ratios"]),
        kv_source_layer_ids=list(c["kv_source_layer_ids"]), index_source_layer_ids=list(c["index_source_layer_ids"]),
        candidate_source_layer_id=c.get("candidate_source_layer_id", -1),
        candidate_topk_blocks=c.get("candidate_topk_blocks", 2048), candidate_block_size=c.get("candidate_block_size", 8),
        index_n_heads=c["index_n_heads"], index_head_dim=c["index_head_dim"], index_topk=c["index_topk"],
        rms_norm_eps=spec.RMS_NORM_EPS)


def _ocfg(c):
    return dict(c, rms_norm_eps=spec.RMS_NORM_EPS, compress_rope_theta=spec.COMPRESS_ROPE_THETA,
                rope_theta=spec.ROPE_THETA)


def _modules(c, dev):
    params, xs, pos, live = spec.make_stack_params_and_inputs(c)
    cfg = _config(c)
    mods = []
    for i, p in enumerate(params):
        m = MO.DeepseekV41Attention(cfg, i)
        r = m.load_state_dict(p, strict=True)
        assert not r.missing_keys and not r.unexpected_keys
        mods.append(m.to(dev).eval())
    return mods, params, xs, pos, live


def _groups(c, i):
    r = c["compress_ratios"][i]
    return c["seq"] // r if r else 0


def _unpack(key, cols):
    return np.unpackbits(FIX[key], axis=-1)[..., :cols].astype(bool)


def _mask(key, s, t, dev, kind="lowest"):
    """The reference's mask (bool [B, S, T] kept) as the model hands it to the layers:
    [B, 1, S, T] additive with transformers' eager fill (the dtype's lowest value), -inf,
    or bool."""
    keep = torch.from_numpy(_unpack(key, t)).reshape(-1, s, t)[:, None]
    if kind == "bool":
        return keep.to(dev)
    fill = torch.finfo(torch.float32).min if kind == "lowest" else float("-inf")
    return torch.zeros(keep.shape).masked_fill(~keep, fill).to(dev)


def _selection(shared, b, s, g):
    sel = np.zeros((b, s, g + 1), bool)
    idx = shared.get("topk_idx")
    if idx is None:
        return sel[..., :g]
    i = idx.cpu().numpy().astype(np.int64).reshape(b, s, -1)
    np.put_along_axis(sel, np.where(i < 0, g, i), True, -1)
    return sel[..., :g]


def _run(mods, c, xs, pos, dev, cache=None, mask=None):
    """One forward of the schedule; returns (outs [layers] cpu, {index source: selection},
    candidate mask or None)."""
    rot = MO.DeepseekV41RotaryEmbedding(mods[0].config).to(dev)
    pd = pos.to(dev)
    x0 = xs[0].to(dev)
    pe = {"main": rot(x0, pd, "main"), "compress": rot(x0, pd, "compress")}
    shared = MO.SharedState()
    b, s = pos.shape
    outs, sels, cand = [], {}, None
    with torch.no_grad():
        for i, m in enumerate(mods):
            o, w = m(xs[i].to(dev), position_embeddings=pe, attention_mask=mask, past_key_values=cache,
                     shared=shared, position_ids=pd)
            assert w is None
            outs.append(o.float().cpu())
            if m.is_index_source:
                g = shared["index_k"].shape[2]
                sels[i] = _selection(shared, b, s, g)
                if m.indexer.is_candidate_source:
                    cand = shared["candidates"].cpu().numpy().astype(bool)
    torch.cuda.synchronize()
    return outs, sels, cand


def _assert_attn(got, ref, what):
    got = torch.as_tensor(np.asarray(got)).float().flatten()
    ref = torch.as_tensor(np.asarray(ref)).float().flatten()
    c = cosine(got, ref)
    m = float((got - ref).abs().max())
    assert c >= ATTN_COS_MIN and m <= ATTN_MAXABS, f"{what}: cosine {c:.7f}, max-abs {m:.3e}"


def _near_ties(sel_gpu, scores, absref, what):
    """Every entry where the GPU's selection differs from the oracle's lowest-index top-k of
    the oracle's scores is a near-tie of the k-th score (the indexer bar, relative to the
    scores' magnitude before cancellation)."""
    sc = scores.numpy()
    ab = absref.numpy()
    for b, s in np.argwhere(np.ones(sel_gpu.shape[:2], bool)):
        row = sc[b, s]
        fin = np.isfinite(row)
        k = int(sel_gpu[b, s].sum())
        if not fin.any():
            assert k == 0, f"{what}: row ({b},{s}) selects {k} entries with none visible"
            continue
        order = np.lexsort((np.arange(len(row)), -row.astype(np.float64)))
        want = np.zeros_like(sel_gpu[b, s])
        want[order[:k]] = True
        want &= fin
        if np.array_equal(want, sel_gpu[b, s]):
            continue
        kth = row[order[k - 1]]
        for e in np.nonzero(want != sel_gpu[b, s])[0]:
            tol = 2 * SCORE_RTOL * (ab[b, s, e] + ab[b, s, order[k - 1]]) + 1e-12
            assert np.isfinite(row[e]) and abs(row[e] - kth) <= tol, \
                f"{what}: row ({b},{s}) entry {e} (score {row[e]:.8g}) is not a near-tie of the k-th {kth:.8g}"


def _candidate_near_ties(cand_gpu, scores, absref, topk_blocks, block, lens, what):
    """The GPU's candidate blocks against the oracle's scores: a block kept by one rule and
    not the other scores within the indexer bar of the weakest block kept."""
    b, s, g = cand_gpu.shape
    nb = -(-g // block)
    pad = np.full((b, s, nb * block), -np.inf, np.float32)
    pad[..., :g] = scores
    bmax = pad.reshape(b, s, nb, block).max(-1)
    np.put_along_axis(bmax, (lens[..., None] - 1) // block, np.inf, -1)
    from oracle.attention import select_candidate_blocks
    want = select_candidate_blocks(torch.from_numpy(scores), torch.from_numpy(lens[..., None]), topk_blocks, block)
    abmax = np.where(np.isfinite(absref), absref, 0).max(-1)
    for bi, si in np.argwhere((np.asarray(want) != cand_gpu).any(-1)):
        got = np.zeros(nb * block, bool)
        got[:g] = cand_gpu[bi, si]
        gb = got.reshape(nb, block).any(-1)
        kept = bmax[bi, si][gb]
        weakest = kept[np.isfinite(kept)].min()
        scale = abmax[bi, si]
        ref = np.zeros(nb * block, bool)
        ref[:g] = np.asarray(want)[bi, si]
        for blk in np.nonzero(ref.reshape(nb, block).any(-1) != gb)[0]:
            assert abs(bmax[bi, si, blk] - weakest) <= 4 * SCORE_RTOL * scale + 1e-12, \
                f"{what}: row ({bi},{si}) block {blk} is not a near-tie of the weakest kept block"


def _group_source(c, i):
    """The index source whose selection layer i attends (the last one at or before i in i's
    group), or None for a sliding-only layer."""
    if not c["compress_ratios"][i]:
        return None
    start = max(k for k in c["kv_source_layer_ids"] if k <= i)
    srcs = [k for k in c["index_source_layer_ids"] if start <= k <= i]
    return max(srcs) if srcs else None


def _check_vs_reference(c, name, run, outs, sels, what):
    """Rows whose selection (of the layer's group source) is the reference's: the layer's
    output against the reference's module."""
    ref = FIX[f"{name}/{run}_out"]
    b, s = c["batch"], c["seq"]
    for i, o in enumerate(outs):
        src = _group_source(c, i)
        if src is None:
            rows = [(bi, si) for bi in range(b) for si in range(s)]
        else:
            rsel = _unpack(f"{name}/{run}_sel{src}", _groups(c, src))
            rows = [(bi, si) for bi in range(b) for si in range(s) if np.array_equal(sels[src][bi, si], rsel[bi, si])]
        assert len(rows) >= 0.75 * b * s, f"{what} layer {i}: only {len(rows)} rows share the reference's selection"
        got = np.stack([o[bi, si].numpy() for bi, si in rows])
        want = np.stack([ref[i, bi, si] for bi, si in rows])
        _assert_attn(got, want, f"{what} layer {i} vs the reference module")


@pytest.mark.parametrize("name", list(spec.STACKS))
def test_stack_nocache(dev, name):
    c = spec.STACKS[name]
    print(f"stack {name}: no cache", flush=True)
    mods, params, xs, pos, live = _modules(c, dev)
    s = c["seq"]
    mask = _mask(f"{name}/nocache_mask", s, s, dev)
    outs, sels, cand = _run(mods, c, xs, pos, dev, mask=mask)
    # the oracle with the GPU's selections and candidates, every row of every layer
    ref, own = OM.stack_forward(params, _ocfg(c), xs, pos, live=live, select=sels, candidates=cand)
    for i, o in enumerate(outs):
        _assert_attn(o, ref[i], f"{name} layer {i} vs oracle")
    # selections and candidates against the oracle's own choices on the same scores
    for i in c["index_source_layer_ids"]:
        _near_ties(sels[i], own[i]["scores"], own[i]["abs_scores"], f"{name} layer {i} selection")
    if cand is not None:
        src = c["candidate_source_layer_id"]
        lens = (pos.numpy() + 1) // c["compress_ratios"][src]
        _candidate_near_ties(cand, own[src]["scores"].numpy(), own[src]["abs_scores"].numpy(),
                             c["candidate_topk_blocks"], c["candidate_block_size"], lens, f"{name} candidates")
        assert cand.sum() < np.isfinite(own[src]["scores"].numpy()).sum(), "the candidates restrict nothing"
    _check_vs_reference(c, name, "nocache", outs, sels, name)


@pytest.mark.parametrize("name", list(spec.STACKS))
def test_stack_chunked_cache(dev, name):
    from transformers.cache_utils import Cache, DynamicSlidingWindowLayer
    c = spec.STACKS[name]
    print(f"stack {name}: chunked through the caches", flush=True)
    mods, params, xs, pos, live = _modules(c, dev)
    cfg = mods[0].config
    layers = len(mods)
    cache = Cache(layers=[MO.DeepseekV41CSACache(cfg) if i in c["kv_source_layer_ids"]
                          else DynamicSlidingWindowLayer(sliding_window=cfg.sliding_window) for i in range(layers)])
    states = [OM.LayerState() for _ in range(layers)]
    w = c["sliding_window"]
    outs, refs, sels_all, start, call = [], [], {i: [] for i in c["index_source_layer_ids"]}, 0, 0
    for n in spec.chunks(c):
        t = min(start, w - 1) + n
        mask = _mask(f"{name}/cached_mask{call}", n, t, dev)
        xs_c = [x[:, start:start + n] for x in xs]
        o, sels, cand = _run(mods, c, xs_c, pos[:, start:start + n], dev, cache=cache, mask=mask)
        r, _ = OM.stack_forward(params, _ocfg(c), xs_c, pos[:, start:start + n], states,
                                None if live is None else live[:, :start + n], sels, cand)
        outs.append(torch.stack(o))
        refs.append(np.stack(r))
        for i, sl in sels.items():
            full = np.zeros((c["batch"], n, _groups(c, i)), bool)
            full[..., :sl.shape[-1]] = sl
            sels_all[i].append(full)
        start += n
        call += 1
    got = torch.cat(outs, 2).numpy()
    want = np.concatenate(refs, 2)
    for i in range(layers):
        _assert_attn(got[i], want[i], f"{name} layer {i} chunked vs oracle")
    for i in c["kv_source_layer_ids"]:
        layer, st = cache.layers[i], states[i]
        assert layer.entry_count["compressor"] == st.entry_count == int(FIX[f"{name}/cached_entry_count{i}"])
        lat = layer.compressed_kv["compressor"][:, 0].float().cpu().numpy()
        assert np.mean(lat == st.compressed) > 0.999, f"layer {i} compressed cache"
        assert np.array_equal(layer.compressed_bf16().float().cpu().numpy(),
                              layer.compressed_kv["compressor"][:, 0].bfloat16().float().cpu().numpy())
    for i in range(layers):
        assert np.mean(cache.layers[i].keys[:, 0].float().cpu().numpy() == states[i].window) > 0.999, \
            f"layer {i} window cache"
    sels = {i: np.concatenate(v, 1) for i, v in sels_all.items()}
    outs_cpu = [torch.from_numpy(got[i]) for i in range(layers)]
    _check_vs_reference(c, name, "cached", outs_cpu, sels, f"{name} chunked")
    # cache == no cache, on the rows whose selections agree (torch.topk's tie order aside,
    # the reference's own cached and uncached runs agree the same way)
    nc, nsels, _ = _run(mods, c, xs, pos, dev, mask=_mask(f"{name}/nocache_mask", c["seq"], c["seq"], dev))
    for i in range(layers):
        src = _group_source(c, i)
        keep = np.ones((c["batch"], c["seq"]), bool) if src is None else (nsels[src] == sels[src]).all(-1)
        assert keep.mean() >= 0.75, f"{name} layer {i}: cached and uncached selections differ on many rows"
        _assert_attn(got[i][keep], nc[i].numpy()[keep], f"{name} layer {i} cache == no cache")


def test_mask_forms_and_the_mask_free_window(dev):
    """The same causal sliding mask as transformers' lowest-value fill, as -inf and as bool,
    and no mask at all (the window in token order) give the same layer outputs."""
    c = spec.STACKS["two_groups"]
    mods, params, xs, pos, live = _modules(c, dev)
    s = c["seq"]
    base, bsel, _ = _run(mods, c, xs, pos, dev, mask=_mask("two_groups/nocache_mask", s, s, dev))
    for kind in ("-inf", "bool"):
        o, sl, _ = _run(mods, c, xs, pos, dev, mask=_mask("two_groups/nocache_mask", s, s, dev, kind))
        for i in range(len(mods)):
            assert torch.equal(o[i], base[i]), f"{kind} mask, layer {i}"
    o, sl, _ = _run(mods, c, xs, pos, dev, mask=None)
    for i in range(len(mods)):
        _assert_attn(o[i], base[i], f"mask-free window, layer {i}")


def test_padding_is_honoured(dev):
    """The padded batch against the same batch with the padding ignored: the padded row
    changes, the unpadded row does not."""
    c = spec.STACKS["padded"]
    mods, params, xs, pos, live = _modules(c, dev)
    s = c["seq"]
    padded, _, _ = _run(mods, c, xs, pos, dev, mask=_mask("padded/nocache_mask", s, s, dev))
    plain, _, _ = _run(mods, c, xs, pos, dev, mask=None)
    diff = (padded[0] - plain[0]).abs().amax(-1)          # the sliding-only layer: no selection involved
    assert float(diff[0].max()) < 1e-6
    assert float(diff[1].max()) > 1e-2 * float(plain[0].abs().max())


def test_mask_errors(dev):
    c = spec.STACKS["two_groups"]
    mods, params, xs, pos, live = _modules(c, dev)
    s = c["seq"]
    soft = _mask("two_groups/nocache_mask", s, s, dev)
    soft[:, :, 3, 0] = -0.5
    with pytest.raises(NotImplementedError, match="values other"):
        _run(mods, c, xs, pos, dev, mask=soft)
    with pytest.raises(ValueError, match="does not cover"):
        _run(mods, c, xs, pos, dev, mask=_mask("two_groups/nocache_mask", s, s, dev)[..., :-1])


def test_reuse_of_another_groups_selection_raises(dev):
    """A group whose source is not an index source would attend the previous group's
    selection against its own entries (the reference's mask and KV axes then disagree):
    raised, with a cache; without one the group's fresh start leaves nothing selected."""
    from transformers.cache_utils import Cache, DynamicSlidingWindowLayer
    c = dict(spec.STACKS["two_groups"], index_source_layer_ids=[1])
    mods, params, xs, pos, live = _modules(c, dev)
    cfg = mods[0].config
    cache = Cache(layers=[MO.DeepseekV41CSACache(cfg) if i in c["kv_source_layer_ids"]
                          else DynamicSlidingWindowLayer(sliding_window=cfg.sliding_window) for i in range(4)])
    s = c["seq"]
    with pytest.raises(ValueError, match="selection published"):
        _run(mods, c, xs, pos, dev, cache=cache, mask=_mask("two_groups/nocache_mask", s, s, dev))
    outs, _, _ = _run(mods, c, xs, pos, dev, mask=_mask("two_groups/nocache_mask", s, s, dev))
    ref, _ = OM.stack_forward(params, _ocfg(c), xs, pos)
    _assert_attn(outs[3], ref[3], "a group without an index source attends no compressed entry")
