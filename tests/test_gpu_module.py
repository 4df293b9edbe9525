"""GPU: the module drop-ins (mzoo_amd/owlet1.py) end to end, BASELINE config 1 included.

``DeepseekV41Attention`` with the reference's parameter names runs a whole layer on the GPU
(projections on hipBLASLt, every per-token op in the HIP library) and is compared with

* the oracle's module composition (oracle/model.py) with the GPU's selection imposed, on
  every row -- the attention bar (cosine >= 0.9999, max-abs <= 2e-2 against outputs of
  magnitude ~0.3);
* the reference's own module (tests/golden/module_fixture.npz) on every recorded row whose
  selection is the reference's;
* the selection itself: equal to the oracle's top-k except near-ties of the k-th score
  (the indexer bar: 1e-5 relative), ReLU's exact-zero ties included;

without a cache and through a cache fed in chunks that end mid-group, then one-token
decode steps.  The RMSNorm kernel is bit-exact against the oracle's pinned order; the
selection-format kernels (top-k bias, mask -> index lists) are exact; the attention
interface registered for transformers runs the reference's mask semantics.
"""

import pathlib
import sys

import numpy as np
import pytest
import torch

from mzoo_amd import owlet1 as MO
from oracle import attention as OA
from oracle import compressor as OC
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
        sliding_window=c["sliding_window"], compress_ratios=[c["compress_ratio"]], kv_source_layer_ids=[0],
        index_source_layer_ids=[0], candidate_source_layer_id=-1, index_n_heads=c["index_n_heads"],
        index_head_dim=c["index_head_dim"], index_topk=c["index_topk"], rms_norm_eps=spec.RMS_NORM_EPS)


def _ocfg(c):
    return dict(c, rms_norm_eps=spec.RMS_NORM_EPS, compress_rope_theta=spec.COMPRESS_ROPE_THETA)


def _module(c, dev):
    params, x, pos = spec.make_params_and_inputs(c)
    mod = MO.DeepseekV41Attention(_config(c), 0)
    missing = mod.load_state_dict(params, strict=True)
    assert not missing.missing_keys and not missing.unexpected_keys
    return mod.to(dev).eval(), params, x, pos


def _forward(mod, x, pos, cache, dev):
    rot = MO.DeepseekV41RotaryEmbedding(mod.config).to(dev)
    xd, pd = x.to(dev), pos.to(dev)
    pe = {"main": rot(xd, pd, "main"), "compress": rot(xd, pd, "compress")}
    shared = MO.SharedState()
    with torch.no_grad():
        out, _ = mod(xd, position_embeddings=pe, attention_mask=None, past_key_values=cache, shared=shared,
                     position_ids=pd)
    return out, shared


def _selection(shared, b, s, g):
    sel = np.zeros((b, s, g + 1), bool)
    idx = shared.get("topk_idx")
    if idx is None:
        return sel[..., :g]
    i = idx.cpu().numpy().astype(np.int64)
    np.put_along_axis(sel, np.where(i < 0, g, i), True, -1)
    return sel[..., :g]


def _check_selection(sel_gpu, scores, absref, what):
    """sel_gpu against the oracle's lowest-index top-k of the oracle's scores: differing
    entries must be near-ties of the k-th score."""
    sc = scores.numpy()
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
            tol = 2 * SCORE_RTOL * (absref[b, s, e] + abs(kth)) + 1e-12
            assert np.isfinite(row[e]) and abs(row[e] - kth) <= tol, \
                f"{what}: row ({b},{s}) entry {e} (score {row[e]:.8g}) is not a near-tie of the k-th {kth:.8g}"


def _abs_scores(params, c, x, pos, g, index_k):
    """The magnitude the score tolerance is relative to (oracle.attention.indexer_abs_scores)."""
    q_res = OM.rms_norm(OM.linear(x, params["wq_a.weight"]), params["q_norm.weight"], spec.RMS_NORM_EPS)
    b, s = pos.shape
    q = OM.linear(q_res, params["indexer.wq_b.weight"]).reshape(b, s, c["index_n_heads"], c["index_head_dim"])
    cos, sin = OM.rope_tables(pos.numpy(), c["qk_rope_head_dim"], spec.COMPRESS_ROPE_THETA)
    q = OC.rope(q, cos[:, :, None], sin[:, :, None])
    w = OM.linear(x, params["indexer.weights_proj.weight"]) * np.float32(c["index_n_heads"] ** -0.5)
    return OA.indexer_abs_scores(torch.from_numpy(q), torch.from_numpy(index_k), torch.from_numpy(w),
                                 c["compress_ratio"], pos).numpy()


def _assert_attn(got, ref, what):
    got = torch.as_tensor(got).float().flatten()
    ref = torch.as_tensor(ref).float().flatten()
    c = cosine(got, ref)
    m = float((got - ref).abs().max())
    assert c >= ATTN_COS_MIN and m <= ATTN_MAXABS, f"{what}: cosine {c:.7f}, max-abs {m:.3e}"


@pytest.mark.parametrize("name", list(spec.CONFIGS))
def test_layer_nocache(dev, name):
    c = spec.CONFIGS[name]
    print(f"module {name}: no cache", flush=True)
    mod, params, x, pos = _module(c, dev)
    out, shared = _forward(mod, x, pos, None, dev)
    torch.cuda.synchronize()
    b, s, g = c["batch"], c["seq"], c["seq"] // c["compress_ratio"]
    sel = _selection(shared, b, s, g)
    # the oracle with the GPU's selection: every row
    ref, oshared = OM.layer_forward(params, _ocfg(c), x, pos, select=sel)
    _assert_attn(out.cpu(), ref, f"{name} layer vs oracle")
    # the published keys: the GPU's projections differ from the CPU's in the last bits, so
    # the fake-quantized keys match the oracle's up to rare rounding-boundary flips
    gk = shared["index_k"][:, 0].float().cpu().numpy()
    assert np.mean(gk == oshared["index_k"]) > 0.999, "published indexer keys"
    # the selection: the oracle's top-k up to near-ties
    _, own = OM.layer_forward(params, _ocfg(c), x, pos)
    absref = _abs_scores(params, c, x, pos, g, oshared["index_k"])
    _check_selection(sel, own["scores"], absref, f"{name} selection")
    # the reference's module, on the rows whose selection is the reference's
    ref_sel = np.unpackbits(FIX[f"{name}/nocache_sel"], axis=-1)[..., :g].astype(bool)
    rows = FIX["config1/sample_rows"] if name == "config1" else np.arange(s)
    fix = FIX[f"{name}/nocache_out"]
    same = [(bi, j) for bi in range(b) for j, r in enumerate(rows) if np.array_equal(sel[bi, r], ref_sel[bi, r])]
    assert len(same) >= 0.8 * b * len(rows), f"only {len(same)} rows share the reference's selection"
    got = out.cpu().numpy()[:, rows]
    _assert_attn(np.stack([got[bi, j] for bi, j in same]), np.stack([fix[bi, j] for bi, j in same]),
                 f"{name} layer vs the reference module")


@pytest.mark.parametrize("name", list(spec.CONFIGS))
def test_layer_chunked_cache(dev, name):
    """Two prefill chunks that end mid-group, then one-token decode steps, through
    DeepseekV41CSACache: outputs, the window, the key and latent caches and the carry."""
    from transformers.cache_utils import Cache
    c = spec.CONFIGS[name]
    print(f"module {name}: chunked through the cache", flush=True)
    mod, params, x, pos = _module(c, dev)
    cache = Cache(layers=[MO.DeepseekV41CSACache(mod.config)])
    state = OM.LayerState()
    outs, refs, start = [], [], 0
    b, r = c["batch"], c["compress_ratio"]
    for n in spec.chunks(c):
        xs, ps = x[:, start:start + n], pos[:, start:start + n]
        o, shared = _forward(mod, xs, ps, cache, dev)
        groups_now = (start + n) // r
        sel = _selection(shared, b, n, groups_now)
        ref, _ = OM.layer_forward(params, _ocfg(c), xs, ps, state, select=sel)
        outs.append(o.cpu())
        refs.append(ref)
        start += n
    torch.cuda.synchronize()
    _assert_attn(torch.cat(outs, 1), np.concatenate(refs, 1), f"{name} chunked layer vs oracle")
    layer = cache.layers[0]
    assert layer.entry_count["compressor"] == state.entry_count == int(FIX[f"{name}/cached_entry_count"])
    assert np.mean(layer.keys[:, 0].float().cpu().numpy() == state.window) > 0.999, "window cache"
    assert layer.compressed_kv["indexer"].shape[2] == state.index_k.shape[1]
    assert layer.buffer_kv["compressor"].shape == state.buffer_kv.shape
    np.testing.assert_allclose(layer.buffer_kv["compressor"].cpu().numpy(), state.buffer_kv, rtol=1e-5, atol=1e-6)
    lat = layer.compressed_kv["compressor"][:, 0].float().cpu().numpy()
    assert np.mean(lat == state.compressed) > 0.999, "compressed cache"


def test_rms_norm_bit_exact(dev):
    g = torch.Generator().manual_seed(5)
    for d, dt in ((64, torch.float32), (160, torch.float32), (576, torch.bfloat16), (1536, torch.bfloat16),
                  (100, torch.float32), (7, torch.float16)):
        x = (torch.randn(37, d, generator=g) * torch.exp(torch.randn(37, 1, generator=g) * 3)).to(dt)
        norm = MO.DeepseekV41RMSNorm(d, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(1 + 0.1 * torch.randn(d, generator=g))
        norm = norm.to(dev, dtype=dt)
        got = norm(x.to(dev)).float().cpu().numpy()
        name = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}[dt]
        want = OC.rms_norm(x.float().numpy(), norm.weight.detach().float().cpu().numpy(), 1e-6, name)
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"rms_norm D={d} {dt}"


def test_selection_formats(dev):
    g = torch.Generator().manual_seed(6)
    rows, groups, k = 50, 300, 40
    idx = torch.stack([torch.randperm(groups, generator=g)[:k] for _ in range(rows)]).int()
    idx[3, 5:] = -1
    idx = idx.sort(-1).values
    bias = MO._topk_bias(idx.view(5, 10, k).to(dev), groups).cpu()
    want = torch.full((rows, groups + 1), float("-inf")).scatter_(-1, torch.where(idx < 0, groups, idx).long(), 0.0)
    assert torch.equal(bias.view(rows, groups), want[:, :groups])
    # mask -> index lists: 0 kept; -inf and the dtype's lowest value masked
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        m = torch.where(torch.rand(rows, 700, generator=g) < 0.1, torch.tensor(0.0), torch.tensor(float("-inf")))
        m[::2] = torch.where(m[::2] == 0, m[::2], torch.tensor(torch.finfo(dt).min))
        m = m.to(dt)
        got = MO._mask_to_indices(m.to(dev), 700).cpu()
        for r in range(rows):
            vis = torch.nonzero(m[r] == 0).flatten().int()
            assert torch.equal(got[r, :len(vis)], vis) and bool((got[r, len(vis):] == -1).all()), f"row {r} {dt}"
    with pytest.raises(ValueError, match="more than"):
        MO._mask_to_indices(torch.zeros(2, 64, device=dev), 10)
    with pytest.raises(NotImplementedError, match="values other"):
        MO._mask_to_indices(torch.full((2, 64), -1.5, device=dev), 64)


def test_shared_state_builds_the_bias_lazily(dev):
    idx = torch.tensor([[[0, 3, -1], [1, 2, 3]]], dtype=torch.int32, device=dev)
    lazy = MO.SharedState()
    MO._publish_selection(lazy, idx, 5)
    assert not dict.__contains__(lazy, "topk_bias") and "topk_bias" in lazy
    eager = {}
    MO._publish_selection(eager, idx, 5)
    assert torch.equal(lazy["topk_bias"], eager["topk_bias"])
    assert eager["topk_bias"].shape == (1, 1, 2, 5)
    assert eager["topk_bias"][0, 0, 0].tolist() == [0, float("-inf"), float("-inf"), 0, float("-inf")]


def test_attention_interface_matches_eager(dev):
    """sparse_attention_forward under the reference's calling convention: query [B,H,S,D],
    key == value [B,1,T,D] (window entries then compressed ones), the sliding causal mask
    (transformers' lowest-value fill) extended by a top-k bias, the module's sink."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    name = MO.register_attention_interface()
    assert ALL_ATTENTION_FUNCTIONS[name] is MO.sparse_attention_forward
    gen = torch.Generator().manual_seed(9)
    b, h, s, d, g, w, k = 2, 8, 96, 160, 24, 16, 8
    cfg = MO.AttentionConfig(num_attention_heads=h, head_dim=d, sliding_window=w, index_topk=k,
                             compress_ratios=[4], hidden_size=64, q_lora_rank=32, o_groups=2, o_lora_rank=16,
                             qk_rope_head_dim=32, index_n_heads=2, index_head_dim=32)
    mod = MO.DeepseekV41Attention(cfg, 0)
    with torch.no_grad():
        mod.attn_sink.copy_(torch.randn(h, generator=gen))
    q = torch.randn(b, h, s, d, generator=gen)
    kv = torch.randn(b, 1, s + g, d, generator=gen).bfloat16().float()
    t = torch.arange(s).view(-1, 1)
    kk = torch.arange(s).view(1, -1)
    lowest = torch.finfo(torch.float32).min
    band = torch.where((kk <= t) & (kk > t - w), torch.tensor(0.0), torch.tensor(lowest))
    sc = torch.randn(b, s, g, generator=gen).masked_fill(torch.arange(g) >= (t + 1) // 4, float("-inf"))
    sel = torch.from_numpy(OA.topk_indices(sc, k))
    tb = torch.full((b, s, g + 1), float("-inf")).scatter_(-1, torch.where(sel < 0, g, sel), 0.0)[..., :g]
    mask = torch.cat([band.expand(b, s, s), tb], -1).unsqueeze(1)
    mod = mod.to(dev)
    got, weights = MO.sparse_attention_forward(mod, q.to(dev), kv.to(dev), kv.to(dev), mask.to(dev), d ** -0.5)
    assert weights is None and got.shape == (b, s, h, d)
    ref, _ = OA._attend(q, kv, kv, mask, mod.attn_sink.detach().cpu())
    _assert_attn(got.cpu(), ref, "attention interface")


def test_layer_with_yarn(dev):
    """The compress RoPE extended with YaRN (owlet1/config.py:419-434: the reference's
    rope_parameters layout, YaRN on the compressed branch only): the drop-in layer against the
    oracle composition, whose YaRN tables come from the library routine the reference calls.
    The original context is short enough that YaRN changes most pairs' frequencies at these
    positions, so the default-RoPE composition misses the bar."""
    c = spec.CONFIGS["small"]
    yarn = dict(factor=8.0, original_max_position_embeddings=64, attention_factor=1.0)
    params, x, pos = spec.make_params_and_inputs(c)
    cfg = _config(c)
    partial = c["qk_rope_head_dim"] / c["head_dim"]
    cfg.rope_parameters = {
        "main": {"rope_type": "default", "rope_theta": spec.ROPE_THETA, "partial_rotary_factor": partial},
        "compress": dict(yarn, rope_type="yarn", rope_theta=spec.COMPRESS_ROPE_THETA, partial_rotary_factor=partial)}
    mod = MO.DeepseekV41Attention(cfg, 0)
    res = mod.load_state_dict(params, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    mod = mod.to(dev).eval()
    out, shared = _forward(mod, x, pos, None, dev)
    torch.cuda.synchronize()
    b, s, g = c["batch"], c["seq"], c["seq"] // c["compress_ratio"]
    sel = _selection(shared, b, s, g)
    ref, oshared = OM.layer_forward(params, dict(_ocfg(c), compress_yarn=yarn), x, pos, select=sel)
    _assert_attn(out.cpu(), ref, "small layer with YaRN vs oracle")
    gk = shared["index_k"][:, 0].float().cpu().numpy()
    assert np.mean(gk == oshared["index_k"]) > 0.999, "published indexer keys (YaRN)"
    plain, _ = OM.layer_forward(params, _ocfg(c), x, pos, select=sel)
    assert cosine(torch.from_numpy(plain).flatten(), out.cpu().float().flatten()) < ATTN_COS_MIN, \
        "YaRN made no difference at these positions"
