"""GPU: BASELINE's decode and prefill configurations at their full sizes.

Decode (one step of the device-resident layer, ``SparseDecodeLayer.step``):
  config 2 -- B=32 at position 32767: FP8 index over 8192 groups, top-2048, window 128;
  config 4 -- B=8 at position 131071: MXFP4 index over 32768 groups, top-2048;
  config 5 -- B=4 at position 524287: dense coarse branch of 4096 entries (ratio 128),
              MXFP4 fine index over 131072 groups, top-2048, window 128.
Prefill (config 3) -- B=1, S=8192, 128 heads: FP8 indexer scores over 2048 groups ->
top-2048 -> ``csa2_attn.fwd`` with window 128 on every one of the 8192 query rows.

Every row of a launch runs the same code, so the CPU oracle checks a sample of rows (the
first, the last and some in between), which it finishes in seconds: index sets equal up to
near-ties of the k-th score, attention to the cosine / max-abs bar.  In the prefill
top-2048 of 2048 groups selects every visible group, so the index list of query t must be
exactly 0 .. (t+1)//4 - 1 followed by -1 -- a bit-exact check of the indexer mask and the
top-k compaction at full size.
"""

import pytest
import torch

from mzoo_amd import csa2_attn, indexer, quant
from mzoo_amd.decode import DecodeConfig, SparseDecodeLayer
from oracle import attention as OA
from oracle import quant as Q
from tests.helpers import assert_attn_close, assert_scores_close, assert_topk_sets_match

pytestmark = pytest.mark.gpu

DECODE = {
    # name: (batch, position, groups, index format, coarse ratio, coarse groups, nsplit)
    "config2": (32, 32767, 8192, "fp8", 0, 0, 4),
    "config4": (8, 131071, 32768, "mxfp4", 0, 0, 14),
    "config5": (4, 524287, 131072, "mxfp4", 128, 4096, 32),
}


def _decode_layer(dev, name, seed):
    b, pos, groups, fmt, cr, cg, nsplit = DECODE[name]
    cfg = DecodeConfig(batch=b, max_groups=groups, topk=2048, index_format=fmt, nsplit=nsplit, coarse_ratio=cr,
                       coarse_groups=cg)
    gen = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    layer = SparseDecodeLayer(cfg, dev, sinks=rnd(cfg.heads))
    d = cfg.dim
    layer.fill_window(rnd(b, cfg.window, d).bfloat16(), pos - 1)
    layer.append_groups(0, rnd(b, groups, d).bfloat16(), rnd(b, groups, cfg.index_dim).bfloat16())
    if cr:
        layer.fill_coarse(rnd(b, cg, d).bfloat16())
    layer.set_positions(pos)
    inputs = (rnd(b, cfg.heads, d).bfloat16(), rnd(b, d).bfloat16(), rnd(b, cfg.index_heads, cfg.index_dim).bfloat16(),
              rnd(b, cfg.index_heads) * cfg.index_heads ** -0.5)
    return layer, inputs


def _decode_oracle_rows(layer, inputs, rows):
    """The oracle's decode step for the given rows (after the layer's step, whose window
    append the oracle reads back from the ring)."""
    cfg = layer.cfg
    q, _, q_idx, w = (t.float().cpu()[rows] for t in inputs)
    pos = int(layer.positions[0])
    if cfg.index_format == "fp8":
        kd = Q.dequant_fp8_block(layer.k_codes[rows].cpu().numpy(), layer.k_scales[rows].cpu().numpy()[..., None], 128)
        qd = Q.fake_quant_fp8_block(q_idx.numpy(), 128)
    else:
        kd = Q.dequant_mxfp4(layer.k_packed[rows].cpu().numpy(), layer.k_e8m0[rows].cpu().numpy())
        qd = Q.fake_quant_fp4_block(q_idx.numpy(), 32)
    kd, qd = torch.from_numpy(kd), torch.from_numpy(qd)
    positions = torch.full((len(rows), 1), pos, dtype=torch.int64)
    sc = OA.indexer_scores(qd.unsqueeze(1), kd, w.unsqueeze(1), cfg.ratio, positions)[:, 0]
    mag = OA.indexer_abs_scores(qd.unsqueeze(1), kd, w.unsqueeze(1), cfg.ratio, positions)[:, 0]
    got_idx = layer.idx[rows].cpu()
    win = torch.from_numpy(Q.unpack_latent_fp8_b128(layer.win[rows].cpu().numpy()))
    outs = []
    for i, r in enumerate(rows):
        nw = min(cfg.window, pos + 1)
        toks = [(pos - nw + 1 + j) % cfg.window for j in range(nw)]
        ents = [win[i, toks]]
        if layer.coarse is not None:
            nc = min(cfg.coarse_groups, (pos + 1) // cfg.coarse_ratio)
            ents.append(torch.from_numpy(Q.unpack_latent_fp8_b128(layer.coarse[r, :nc].cpu().numpy())))
        # attention over the kernel's own selection (checked against the oracle's separately)
        sel = got_idx[i][got_idx[i] >= 0].long()
        ents.append(torch.from_numpy(Q.unpack_latent_fp8_b128(layer.main[r, sel.to(layer.main.device)].cpu().numpy())))
        outs.append(OA.attend_entries(q[i], torch.cat(ents), layer.sinks.cpu())[0])
    return torch.stack(outs), sc, mag, got_idx


@pytest.mark.parametrize("name", list(DECODE))
def test_decode_step_full_size(dev, name):
    layer, inputs = _decode_layer(dev, name, seed={"config2": 1, "config4": 2, "config5": 4}[name])
    out = layer.step(*inputs)
    torch.cuda.synchronize()
    b = layer.cfg.batch
    rows = sorted({0, b // 2, b - 1})
    print(f"{name}: checking rows {rows} of {b}", flush=True)
    ref, sc, mag, got_idx = _decode_oracle_rows(layer, inputs, rows)
    assert_topk_sets_match(got_idx, sc, mag, layer.cfg.topk)
    assert_attn_close(out[rows], ref)


def test_prefill_config3_full_size(dev):
    b, s, h, d, g, k, win, ratio, hi, di = 1, 8192, 128, 576, 2048, 2048, 128, 4, 64, 128
    gen = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    q = rnd(b, s, h, d).bfloat16()
    kv = rnd(b, s, 1, d).bfloat16()
    main = rnd(b, g, 1, d).bfloat16()
    q_idx = rnd(b, s, hi, di).bfloat16()
    k_idx = rnd(b, g, di).bfloat16()
    w = rnd(b, s, hi) * hi ** -0.5
    sinks = rnd(h)
    # FP8 indexer (b128 blocks), prefill positions 0..S-1 -> top-k -> attention
    qc, qs = quant.quant_fp8_block(q_idx, 128)
    kc, ks = quant.quant_fp8_block(k_idx, 128)
    scores = indexer.scores_fp8(qc, qs[..., 0], w, kc, ks[..., 0], compress_ratio=ratio)
    idx = indexer.topk(scores, k)
    o, lse = csa2_attn.fwd(q, kv, main, idx, window=win, compress_ratio=ratio, sinks=sinks)
    torch.cuda.synchronize()
    assert o.shape == (b, s, h, d) and lse.shape == (b, h, s)

    # top-2048 of 2048 groups: every visible group, ascending, then -1 (all rows, exact)
    t = torch.arange(s, device=dev)
    vis = (t + 1) // ratio
    col = torch.arange(k, device=dev)
    expect = torch.where(col.view(1, -1) < vis.view(-1, 1), col.view(1, -1).expand(s, k), torch.full_like(col, -1))
    assert torch.equal(idx[0].long(), expect), "prefill top-k must select exactly the visible groups"

    rows = [0, 3, 4, 127, 128, 1000, 4095, 4096, 6143, 8191]
    print(f"config3: checking query rows {rows} of {s}", flush=True)
    # scores of the sampled rows against the oracle (FP8 fake-quant inputs, fp32 sums)
    qd = torch.from_numpy(Q.fake_quant_fp8_block(q_idx[:, rows].float().cpu().numpy(), 128))
    kd = torch.from_numpy(Q.fake_quant_fp8_block(k_idx.float().cpu().numpy(), 128))
    pos = torch.tensor(rows, dtype=torch.int64).view(1, -1)
    ref_sc = OA.indexer_scores(qd, kd, w[:, rows].cpu(), ratio, pos)
    mag = OA.indexer_abs_scores(qd, kd, w[:, rows].cpu(), ratio, pos)
    assert_scores_close(scores[:, rows], ref_sc, mag)

    kv_c, main_c, q_c = kv[0, :, 0].float().cpu(), main[0, :, 0].float().cpu(), q[0, rows].float().cpu()
    idx_c = idx[0, rows].long().cpu()
    lse_c = lse[0, :, rows].cpu()
    for i, tq in enumerate(rows):
        lo = max(0, tq - win + 1)
        sel = idx_c[i][idx_c[i] >= 0]
        ents = torch.cat([kv_c[lo:tq + 1], main_c[sel]])
        ref_o, ref_lse = OA.attend_entries(q_c[i], ents, sinks.cpu())
        assert_attn_close(o[0, tq], ref_o, name=f"o[t={tq}]")
        torch.testing.assert_close(lse_c[:, i], ref_lse.float(), atol=2e-3, rtol=2e-3, msg=f"lse[t={tq}]")


@pytest.mark.parametrize("name", ["config2", "config5"])
def test_decode_step_fused_full_size(dev, name):
    """The fused prologue / epilogue at full size: a layer stepped on the raw projections
    with the RoPE tables equals, bit for bit, an identically filled layer stepped on the
    oracle's normed and rotated inputs (window ring, top-k, output after the inverse RoPE)."""
    import numpy as np
    from oracle import compressor as C
    b, pos, groups, fmt, cr, cg, nsplit = DECODE[name]
    gen = torch.Generator(device=dev).manual_seed(31)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    cfg = DecodeConfig(batch=b, max_groups=groups, topk=2048, index_format=fmt, nsplit=nsplit, coarse_ratio=cr,
                       coarse_groups=cg)
    d = cfg.dim
    sinks, kv_w = rnd(cfg.heads), (1.0 + 0.1 * rnd(d)).bfloat16()
    hist = (rnd(b, cfg.window, d).bfloat16(), rnd(b, groups, d).bfloat16(), rnd(b, groups, cfg.index_dim).bfloat16(),
            rnd(b, max(cg, 1), d).bfloat16())
    layers = []
    for _ in range(2):
        layer = SparseDecodeLayer(cfg, dev, sinks=sinks, kv_norm_weight=kv_w)
        layer.fill_window(hist[0], pos - 1)
        layer.append_groups(0, hist[1], hist[2])
        if cr:
            layer.fill_coarse(hist[3][:, :cg])
        layer.set_positions(pos)
        layers.append(layer)
    q, kv, q_idx = rnd(b, cfg.heads, d).bfloat16(), (3 * rnd(b, d)).bfloat16(), rnd(b, 64, 128).bfloat16()
    w = rnd(b, 64) * 0.125
    tabs = []
    for theta in (10000.0, 160000.0):
        c, s = C.rope_tables(np.full(b, pos), 64, theta)
        tabs += [torch.from_numpy(c).bfloat16().to(dev), torch.from_numpy(s).bfloat16().to(dev)]
    print(f"{name}: fused step at full size, B={b} G={groups}", flush=True)
    out_f = layers[0].step(q, kv, q_idx, w, rope=tuple(tabs)).clone()
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    cos, sin, icos, isin = (f(t) for t in tabs)
    q_rot = torch.from_numpy(C.rope(f(q), cos[:, None], sin[:, None], dtype="bfloat16")).bfloat16().to(dev)
    qi_rot = torch.from_numpy(C.rope(f(q_idx), icos[:, None], isin[:, None], dtype="bfloat16")).bfloat16().to(dev)
    kv_rot = torch.from_numpy(C.decode_kv_latent(f(kv), f(kv_w), 1e-6, cos, sin)).bfloat16().to(dev)
    out_u = layers[1].step(q_rot, kv_rot, qi_rot, w).clone()
    torch.cuda.synchronize()
    assert torch.equal(layers[0].win, layers[1].win), "window rings differ"
    assert torch.equal(layers[0].idx, layers[1].idx), "top-k differs"
    back = torch.from_numpy(C.rope(f(out_u), cos[:, None], sin[:, None], inverse=True, dtype="bfloat16")).bfloat16()
    assert torch.equal(out_f.cpu(), back)
