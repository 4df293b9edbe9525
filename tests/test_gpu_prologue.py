"""GPU: the fused decode prologue and epilogue.

``indexer.decode_fused`` normalizes and rotates the new token's kv projection and appends
its FP8-b128 entry to the window ring, and rotates the indexer query before quantizing it,
inside the indexer launch; ``sparse_mqa_decode(rope=...)`` rotates q as the attention kernel
loads it and applies the inverse rotation to the output (in the split merge, or in the
kernel's own write with one split).  Checked:

* the window entry, bit for bit, against the oracle's ``decode_kv_latent``
  (RMSNorm -> RoPE, ``owlet1/attention.py:150-151``) packed by ``pack_latent_fp8_b128``; the
  other ring slots are untouched;
* the quantized query, bit for bit, against the oracle's quantizer on the oracle's rotated
  query, and the scores bit for bit against the unfused launch on that rotated query;
* the attention output, bit for bit, against the unfused kernels on the oracle's rotated q
  followed by the oracle's inverse rotation (``attention.py:226``), lse unchanged, and
  against the oracle's attention to the attention bar;
* the whole decode step with ``rope`` against the unfused step on the oracle's rotated
  inputs (window ring, top-k, output), and its graph replays against the eager step.
"""

import numpy as np
import pytest
import torch

from mzoo_amd import csa2_attn, indexer, quant
from mzoo_amd.decode import DecodeConfig, SparseDecodeLayer
from oracle import attention as OA
from oracle import compressor as C
from oracle import quant as Q
from tests.helpers import assert_attn_close

pytestmark = pytest.mark.gpu

THETA, THETA_C = 10000.0, 160000.0  # main and compress RoPE bases (any values serve)


def _tables(positions, theta, dev, edge=False):
    """position_embeddings as the reference returns them: bf16 cos / sin [B, 32].  With
    ``edge`` the first rows hold engineered tables that make the rotation's bf16 rounding
    meet its edge cases: with cos = 1 + 2^-7 and sin = 2^-8 (both exact in bf16) the fp32
    results are exact and about one in 128 lies exactly halfway between bf16 neighbours
    (resolved to even); tables of 2^-130 give subnormal products and results; a zero table
    gives signed zeros; cos 0, sin 1 swaps the pair."""
    cos, sin = C.rope_tables(np.asarray(positions), 64, theta)
    if edge:
        cos[0], sin[0] = 1.0 + 2.0 ** -7, 2.0 ** -8
        cos[1], sin[1] = 2.0 ** -130, -(2.0 ** -129)
        cos[2], sin[2] = 0.0, 0.0
        cos[3], sin[3] = 0.0, 1.0
    return (torch.from_numpy(cos).bfloat16().to(dev), torch.from_numpy(sin).bfloat16().to(dev))


def _np(t):
    return t.float().cpu().numpy()


def _rotated(x, cs, inverse=False):
    """The oracle's apply_rotary_pos_emb of x [B, ..., D] with per-row tables, as bf16."""
    cos, sin = _np(cs[0]), _np(cs[1])
    extra = (None,) * (x.dim() - 2)
    y = C.rope(_np(x), cos[(slice(None),) + extra], sin[(slice(None),) + extra], inverse=inverse,
               dtype="bfloat16")
    return torch.from_numpy(y).bfloat16().to(x.device)


def _positions_case(b):
    # ring wrap, the first token, group boundaries and a long position
    return [0, 1, 127, 128, 4099, 131071, 2046][:b]


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_fused_indexer_prologue(dev, fmt):
    b, hi, di, g, wcap, ratio = 6, 64, 128, 1000, 128, 4
    gen = torch.Generator().manual_seed(11)
    rnd = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    pos = _positions_case(b)
    print(f"fused indexer prologue {fmt}: B={b} G={g} positions {pos}", flush=True)
    positions = torch.tensor(pos, dtype=torch.int64, device=dev)
    # rows of very different magnitudes, so the norm's scale matters
    kv = (rnd(b, 576) * torch.tensor([1e-3, 1.0, 30.0, 0.2, 5.0, 1e2])[:, None]).bfloat16().to(dev)
    kv_w = (1.0 + 0.1 * rnd(576)).bfloat16().to(dev)
    eps = 1e-6
    q_idx = rnd(b, hi, di).bfloat16().to(dev)
    w = (rnd(b, hi) * hi ** -0.5).to(dev)
    keys = rnd(b, g, di).bfloat16().to(dev)
    cs, ics = _tables(pos, THETA, dev, edge=True), _tables(pos, THETA_C, dev, edge=True)
    win0 = torch.randint(0, 256, (b, wcap, 656), generator=gen, dtype=torch.uint8).to(dev)
    win = win0.clone()
    if fmt == "fp8":
        kc, ks = quant.quant_fp8_block(keys, 128)
        ks = ks[..., 0].contiguous()
        qc = torch.empty(b, hi, di, dtype=torch.uint8, device=dev)
        qs = torch.empty(b, hi, dtype=torch.float32, device=dev)
    else:
        kc, ks = quant.quant_mxfp4(keys)
        qc = torch.empty(b, hi, di // 2, dtype=torch.uint8, device=dev)
        qs = torch.empty(b, hi, di // 32, dtype=torch.uint8, device=dev)
    scores = indexer.decode_fused(q_idx, w, kc, ks, fmt=fmt, compress_ratio=ratio, positions=positions,
                                  q_rope=ics, kv=kv, kv_weight=kv_w, kv_eps=eps, kv_rope=cs, win_cache=win,
                                  q_codes=qc, q_scales=qs)
    torch.cuda.synchronize()

    # window entry of each row: the oracle's normalized, rotated latent, packed
    lat = C.decode_kv_latent(_np(kv), _np(kv_w), eps, _np(cs[0]), _np(cs[1]))
    ref_ent = Q.pack_latent_fp8_b128(lat)
    got_win = win.cpu().numpy()
    exp_win = win0.cpu().numpy().copy()
    for r, p_ in enumerate(pos):
        exp_win[r, p_ % wcap] = ref_ent[r]
    assert np.array_equal(got_win, exp_win), "window ring differs from the oracle's appended entries"

    # the quantized query: oracle quantizer on the oracle's rotated query
    q_rot = _rotated(q_idx, ics)
    if fmt == "fp8":
        codes, scales = Q.fp8_block_codes(_np(q_rot), 128)
        assert np.array_equal(qc.cpu().numpy(), codes)
        assert np.array_equal(qs.cpu().numpy(), scales[..., 0])
        ref_scores = indexer.decode_fp8(q_rot, w, kc, ks, compress_ratio=ratio, positions=positions)
    else:
        packed, e8 = Q.quant_mxfp4(_np(q_rot))
        assert np.array_equal(qc.cpu().numpy(), packed)
        assert np.array_equal(qs.cpu().numpy(), e8)
        ref_scores = indexer.decode_mxfp4(q_rot, w, kc, ks, compress_ratio=ratio, positions=positions)
    assert torch.equal(scores, ref_scores), "fused scores differ from the unfused launch on the rotated query"


def _attention_inputs(dev, seed, b=4, pos=1500):
    cfg = DecodeConfig(batch=b, max_groups=512, topk=128, index_format="fp8", nsplit=4)
    gen = torch.Generator().manual_seed(seed)
    layer = SparseDecodeLayer(cfg, dev, sinks=torch.randn(cfg.heads, generator=gen))
    d = cfg.dim
    layer.fill_window(torch.randn(b, cfg.window, d, generator=gen).bfloat16().to(dev), pos)
    layer.append_groups(0, torch.randn(b, cfg.max_groups, d, generator=gen).bfloat16().to(dev),
                        torch.randn(b, cfg.max_groups, cfg.index_dim, generator=gen).bfloat16().to(dev))
    layer.set_positions(pos)
    idx = torch.stack([torch.randperm(cfg.max_groups, generator=gen)[:cfg.topk] for _ in range(b)]).int().to(dev)
    idx[0, 100:] = -1  # a ragged row
    q = torch.randn(b, cfg.heads, d, generator=gen).bfloat16().to(dev)
    return layer, idx, q


@pytest.mark.parametrize("nsplit,pos", [(1, 1500), (4, 1500), (4, 9)])
def test_sparse_mqa_rope(dev, nsplit, pos):
    layer, idx, q = _attention_inputs(dev, seed=12, pos=pos)
    cfg = layer.cfg
    pos = int(layer.positions[0])
    print(f"sparse_mqa rope: nsplit {nsplit} position {pos}", flush=True)
    cs = _tables([pos] * cfg.batch, THETA, dev, edge=True)
    kw = dict(main_cache=layer.main, groups=cfg.max_groups, indices=idx, sinks=layer.sinks, nsplit=nsplit)
    o_f, lse_f = csa2_attn.sparse_mqa_decode(q, layer.positions, layer.win, cfg.window, rope=cs, **kw)
    q_rot = _rotated(q, cs)
    o_u, lse_u = csa2_attn.sparse_mqa_decode(q_rot, layer.positions, layer.win, cfg.window, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_f, _rotated(o_u, cs, inverse=True)), "fused output != inverse RoPE of the unfused output"
    assert torch.equal(lse_f, lse_u)
    # against the oracle's attention on the rotated query, rotated back
    win = torch.from_numpy(Q.unpack_latent_fp8_b128(layer.win.cpu().numpy()))
    main = torch.from_numpy(Q.unpack_latent_fp8_b128(layer.main.cpu().numpy()))
    outs = []
    nw = min(cfg.window, pos + 1)
    for r in range(cfg.batch):
        toks = [(pos - nw + 1 + i) % cfg.window for i in range(nw)]
        sel = idx[r].cpu()
        ents = torch.cat([win[r, toks], main[r, sel[sel >= 0].long()]])
        outs.append(OA.attend_entries(q_rot[r].float().cpu(), ents, layer.sinks.cpu())[0])
    ref = torch.stack(outs)
    ref = torch.from_numpy(C.rope(ref.numpy(), _np(cs[0])[:, None], _np(cs[1])[:, None], inverse=True))
    assert_attn_close(o_f, ref)


def _step_layers(dev, fmt, coarse, seed, pos=2047):
    cfg = DecodeConfig(batch=4, max_groups=512, topk=128, index_format=fmt, nsplit=3,
                       coarse_ratio=64 if coarse else 0, coarse_groups=32 if coarse else 0)
    gen = torch.Generator().manual_seed(seed)
    sinks = torch.randn(cfg.heads, generator=gen)
    kv_w = (1.0 + 0.1 * torch.randn(cfg.dim, generator=gen)).bfloat16()
    b, d = cfg.batch, cfg.dim
    hist = (torch.randn(b, cfg.window, d, generator=gen).bfloat16().to(dev),
            torch.randn(b, cfg.max_groups, d, generator=gen).bfloat16().to(dev),
            torch.randn(b, cfg.max_groups, cfg.index_dim, generator=gen).bfloat16().to(dev),
            torch.randn(b, max(cfg.coarse_groups, 1), d, generator=gen).bfloat16().to(dev))
    layers = []
    for _ in range(2):
        layer = SparseDecodeLayer(cfg, dev, sinks=sinks, kv_norm_weight=kv_w, kv_norm_eps=1e-6)
        layer.fill_window(hist[0], pos - 1)
        layer.append_groups(0, hist[1], hist[2])
        if coarse:
            layer.fill_coarse(hist[3][:, :cfg.coarse_groups])
        layer.set_positions(pos)
        layers.append(layer)
    q = torch.randn(b, cfg.heads, d, generator=gen).bfloat16().to(dev)
    kv = (torch.randn(b, d, generator=gen) * 3).bfloat16().to(dev)
    q_idx = torch.randn(b, cfg.index_heads, cfg.index_dim, generator=gen).bfloat16().to(dev)
    w = (torch.randn(b, cfg.index_heads, generator=gen) * cfg.index_heads ** -0.5).to(dev)
    rope = _tables([pos] * b, THETA, dev) + _tables([pos] * b, THETA_C, dev)
    return layers, (q, kv, q_idx, w), rope, kv_w


@pytest.mark.parametrize("fmt,coarse,pos", [("fp8", False, 2047), ("mxfp4", False, 2047), ("mxfp4", True, 2047),
                                            ("fp8", False, 6)])
def test_decode_step_fused_matches_unfused(dev, fmt, coarse, pos):
    (lf, lu), (q, kv, q_idx, w), rope, kv_w = _step_layers(dev, fmt, coarse, seed=13, pos=pos)
    print(f"decode step fused {fmt} coarse={coarse}", flush=True)
    out_f = lf.step(q, kv, q_idx, w, rope=rope).clone()
    cs, ics = rope[:2], rope[2:]
    lat = C.decode_kv_latent(_np(kv), _np(kv_w), 1e-6, _np(cs[0]), _np(cs[1]))
    kv_rot = torch.from_numpy(lat).bfloat16().to(dev)
    out_u = lu.step(_rotated(q, cs), kv_rot, _rotated(q_idx, ics), w).clone()
    torch.cuda.synchronize()
    assert torch.equal(lf.win, lu.win), "window rings differ"
    assert torch.equal(lf.idx, lu.idx), "top-k differs"
    assert torch.equal(out_f, _rotated(out_u, cs, inverse=True))


def test_decode_step_fused_graph_replay(dev):
    (layer, _), inputs, rope, _ = _step_layers(dev, "fp8", False, seed=14)
    eager = layer.step(*inputs, rope=rope).clone()
    win_eager = layer.win.clone()
    layer.capture(*inputs, rope=rope)
    for i in range(3):
        torch.randn(1000, device=dev).sum()  # unrelated eager work between replays
        out = layer.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager step"
        assert torch.equal(layer.win, win_eager)


def test_grouped_output_projection(dev):
    """wo_b(wo_a(grouped)) of owlet1/attention.py:20-39, :233-235 against the reference's
    steps in float32 on the CPU (GroupedLinear's view / transpose / bmm, then the linear);
    bf16 operands, fp32 accumulation."""
    from mzoo_amd.decode import GroupedOutputProjection
    gen = torch.Generator().manual_seed(15)
    b, h, d, groups, rank, hidden = 6, 128, 576, 8, 64, 256
    o = torch.randn(b, h, d, generator=gen).bfloat16()
    wa = (torch.randn(groups * rank, h * d // groups, generator=gen) * (h * d // groups) ** -0.5).bfloat16()
    wb = (torch.randn(hidden, groups * rank, generator=gen) * (groups * rank) ** -0.5).bfloat16()
    proj = GroupedOutputProjection(wa.to(dev), wb.to(dev), groups)
    got = proj(o.to(dev)).float().cpu()
    # the reference's formulation, float32
    x = o.float().reshape(b, 1, groups, -1)
    w = wa.float().view(groups, -1, x.shape[-1]).transpose(1, 2)
    y = torch.bmm(x.reshape(-1, groups, x.shape[-1]).transpose(0, 1), w).transpose(0, 1).reshape(b, 1, groups, -1)
    ref = torch.nn.functional.linear(y.flatten(2), wb.float())[:, 0]
    assert got.shape == ref.shape
    assert_attn_close(got, ref, name="projected output")


@pytest.mark.parametrize("path", ["decode_fp8", "decode_fused"])
def test_negative_position_appends_nothing(dev, path):
    """A row at position -1 has no ring slot: its window ring stays as it was (the other
    rows append as usual) and all its scores are -inf."""
    b, hi, g, wcap = 4, 64, 512, 128
    gen = torch.Generator().manual_seed(16)
    pos = torch.tensor([5, -1, 300, -1], dtype=torch.int64, device=dev)
    kv = torch.randn(b, 576, generator=gen).bfloat16().to(dev)
    q_idx = torch.randn(b, hi, 128, generator=gen).bfloat16().to(dev)
    w = (torch.randn(b, hi, generator=gen) * hi ** -0.5).to(dev)
    kc, ks = quant.quant_fp8_block(torch.randn(b, g, 128, generator=gen).bfloat16().to(dev), 128)
    ks = ks[..., 0].contiguous()
    win0 = torch.randint(0, 256, (b, wcap, 656), generator=gen, dtype=torch.uint8).to(dev)
    win = win0.clone()
    print(f"negative position: {path}", flush=True)
    if path == "decode_fp8":
        scores = indexer.decode_fp8(q_idx, w, kc, ks, compress_ratio=4, positions=pos, kv=kv, win_cache=win)
    else:
        cs = _tables([5, 0, 300, 0], THETA, dev)
        scores = indexer.decode_fused(q_idx, w, kc, ks, fmt="fp8", compress_ratio=4, positions=pos, q_rope=cs, kv=kv,
                                      kv_weight=torch.ones(576, dtype=torch.bfloat16, device=dev), kv_eps=1e-6,
                                      kv_rope=cs, win_cache=win)
    torch.cuda.synchronize()
    for r in (1, 3):
        assert torch.equal(win[r], win0[r]), f"row {r} (position -1) changed its ring"
        assert bool(torch.isinf(scores[r]).all()) and bool((scores[r] < 0).all())
    for r, p_ in ((0, 5), (2, 300)):
        changed = (win[r] != win0[r]).any(-1)
        assert bool(changed[p_ % wcap]) and int(changed.sum()) == 1, f"row {r}: exactly slot {p_ % wcap} is written"
