"""GPU: the decode step with in-step group emission, captured once and replayed with
advancing positions across group boundaries, against the oracle's step-by-step decode.

The layer starts mid-sequence (groups emitted from the history's compressor projections by
the oracle, the partial group in the carry ring, the window holding the last tokens).  Each
replay gets new inputs (q, kv, the indexer query and weights, the compressor projections of
the token) through the graph's static buffers and advances every row's position; on the
device the step emits each completed group into the main cache and the key cache, gathers
the token's RoPE tables from the position table, appends the window entry, rotates and
quantizes the indexer query, scores, selects and attends.  Checked after every replay:

* the RoPE table against the oracle's tables, bit for bit;
* the window ring, the main-cache entries, the index keys and the quantized indexer query
  (FP8 b128 or MXFP4), bit for bit against the oracle (``compressor.emit_group`` + the packers; ``decode_kv_latent``);
* the selection against the oracle's top-k of the oracle's scores up to near-ties;
* the output (inverse RoPE applied) against the oracle's attention over the window, the
  coarse entries (hierarchical case) and the selected entries, to the attention bar.
"""

import numpy as np
import pytest
import torch

from mzoo_amd.decode import CompressorWeights, DecodeConfig, SparseDecodeLayer
from oracle import attention as OA
from oracle import compressor as C
from oracle import quant as Q
from tests.helpers import assert_attn_close, assert_scores_close, assert_topk_sets_match

pytestmark = pytest.mark.gpu

D, HI, DI, W = 576, 64, 128, 128
THETA_C = 160000.0


def _bf(x):
    return Q.round_bf16(np.asarray(x, np.float32))


def _keys(keys, fmt):
    if fmt == "fp8":
        codes, scales = Q.fp8_block_codes(keys, 128)
        return codes, scales[..., 0]
    return Q.quant_mxfp4(keys)


def _dequant_keys(a, s, fmt):
    return Q.dequant_fp8_block(a, s[..., None], 128) if fmt == "fp8" else Q.dequant_mxfp4(a, s)


def _emit_history(kv, gate, ratio, ngroups, nw, cos_t, sin_t, wk=None, kw=None):
    rots, keys = [], []
    for g in range(ngroups):
        c, s = cos_t[g * ratio][None], sin_t[g * ratio][None]
        c = np.repeat(c, kv.shape[0], 0)
        s = np.repeat(s, kv.shape[0], 0)
        rot, key = C.emit_group(kv[:, g * ratio:(g + 1) * ratio], gate[:, g * ratio:(g + 1) * ratio], ratio, nw,
                                1e-6, c, s, wk, kw, 1e-6)
        rots.append(rot)
        keys.append(key)
    return np.stack(rots, 1), (np.stack(keys, 1) if wk is not None else None)


@pytest.mark.parametrize("fmt,coarse,merged", [("fp8", False, True), ("fp8", False, False), ("mxfp4", False, True),
                                               ("mxfp4", 8, True), ("mxfp4", 8, False), ("fp8", 40, True)])
def test_replays_across_group_boundaries(dev, fmt, coarse, merged):
    """``coarse``: the coarse branch's ratio (40: its carried slots stream through the
    kernel in more than one batch, the last one partial).  ``merged``: the emission (both
    branches) runs inside the indexer launch (``DecodeConfig.merged_emit``); otherwise in a
    launch of its own, whose prologue also writes the quantized query."""
    b, ratio, gcap, topk, p0, steps = 3, 4, 64, 16, 150, 11
    cratio, cgroups = (coarse, 32) if coarse else (0, 0)
    gen = torch.Generator().manual_seed(31 + bool(coarse))
    rnd = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    print(f"emission replay: fmt={fmt} coarse={coarse} merged={merged} positions {p0}..{p0 + steps - 1}", flush=True)
    nw, kvw = _bf(1 + 0.1 * rnd(D).numpy()), _bf(1 + 0.1 * rnd(D).numpy())
    wk, kw = _bf(0.04 * rnd(DI, D).numpy()), _bf(1 + 0.1 * rnd(DI).numpy())
    cnw = _bf(1 + 0.1 * rnd(D).numpy())
    sinks = rnd(128)
    cfg = DecodeConfig(batch=b, max_groups=gcap, topk=topk, index_format=fmt, nsplit=2, coarse_ratio=cratio,
                       coarse_groups=cgroups, merged_emit=merged)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    cw = CompressorWeights(t(nw), t(wk), t(kw), 1e-6, 1e-6, t(cnw) if coarse else None, THETA_C)
    layer = SparseDecodeLayer(cfg, dev, sinks=sinks, kv_norm_weight=t(kvw), kv_norm_eps=1e-6, compressor=cw)

    # the position table: the reference's cos / sin (fp32) rounded to bf16
    tab = layer.rope_table.cpu()
    cos_t, sin_t = C.rope_tables(np.arange(tab.shape[0]), 64, THETA_C)
    cos_t, sin_t = _bf(cos_t), _bf(sin_t)
    assert np.array_equal(tab[:, :32].float().numpy(), cos_t) and np.array_equal(tab[:, 32:].float().numpy(), sin_t)

    # history: compressor projections of tokens 0..p0-1 -> groups emitted by the oracle
    hkv, hgate = rnd(b, p0, D).numpy(), rnd(b, p0, D).numpy()
    n0 = p0 // ratio
    rots, keys = _emit_history(hkv, hgate, ratio, n0, nw, cos_t, sin_t, wk, kw)
    main = np.zeros((b, gcap, 656), np.uint8)
    main[:, :n0] = Q.pack_latent_fp8_b128(rots)
    ka, ks = _keys(keys, fmt)
    key_a = np.zeros((b, gcap) + ka.shape[2:], np.uint8)
    key_s = (np.ones((b, gcap), np.float32) if fmt == "fp8" else np.full((b, gcap, DI // 32), 127, np.uint8))
    key_a[:, :n0], key_s[:, :n0] = ka, ks
    if fmt == "fp8":
        layer.k_codes.copy_(t(key_a)), layer.k_scales.copy_(t(key_s))
    else:
        layer.k_packed.copy_(t(key_a)), layer.k_e8m0.copy_(t(key_s))
    layer.main.copy_(t(main))
    layer.set_carry(t(hkv[:, n0 * ratio:]), t(hgate[:, n0 * ratio:]))
    coarse_ent = None
    if coarse:
        cn0 = p0 // cratio
        crots, _ = _emit_history(hkv, hgate, cratio, cn0, cnw, cos_t, sin_t)
        coarse_ent = np.zeros((b, cgroups, 656), np.uint8)
        coarse_ent[:, :cn0] = Q.pack_latent_fp8_b128(crots)
        layer.coarse.copy_(t(coarse_ent))
        layer.set_carry(t(hkv[:, cn0 * cratio:]), t(hgate[:, cn0 * cratio:]), coarse=True)
    # window: the last W tokens' entries
    win = np.zeros((b, W, 656), np.uint8)
    for tok in range(p0 - W, p0):
        win[:, tok % W] = Q.pack_latent_fp8_b128(_bf(rnd(b, D).numpy()))
    layer.win.copy_(t(win))
    layer.set_positions(p0)
    carry = np.zeros((b, ratio, D), np.float32), np.zeros((b, ratio, D), np.float32)
    carry[0][:, :p0 % ratio], carry[1][:, :p0 % ratio] = hkv[:, n0 * ratio:], hgate[:, n0 * ratio:]
    if coarse:
        ccarry = np.zeros((b, cratio, D), np.float32), np.zeros((b, cratio, D), np.float32)
        ccarry[0][:, :p0 % cratio], ccarry[1][:, :p0 % cratio] = hkv[:, cn0 * cratio:], hgate[:, cn0 * cratio:]

    def new_inputs():
        ins = [rnd(b, 128, D).bfloat16(), rnd(b, D).bfloat16(), rnd(b, HI, DI).bfloat16(), rnd(b, HI) * HI ** -0.5,
               rnd(b, D), rnd(b, D)]
        if coarse:
            ins += [rnd(b, D), rnd(b, D)]
        return ins

    first = [x.to(dev) for x in new_inputs()]
    layer.capture(*first[:4], advance=True, rope="table", compress=tuple(first[4:]))
    for i in range(steps):
        pos = p0 + i
        ins = new_inputs()
        for dst, src in zip(layer.static_inputs, ins):
            dst.copy_(src)
        out = layer.replay().clone()
        torch.cuda.synchronize()
        q, kv, q_idx, w, kvc, gate = [x.float().numpy() for x in ins[:6]]
        cs, sn = np.repeat(cos_t[pos][None], b, 0), np.repeat(sin_t[pos][None], b, 0)
        # window entry
        win[:, pos % W] = Q.pack_latent_fp8_b128(C.decode_kv_latent(kv, kvw, 1e-6, cs, sn))
        assert np.array_equal(layer.win.cpu().numpy(), win), f"step {i}: window ring"
        # carry + emission
        carry[0][:, pos % ratio], carry[1][:, pos % ratio] = kvc, gate
        if (pos + 1) % ratio == 0:
            g = (pos + 1) // ratio - 1
            cg, sg = np.repeat(cos_t[g * ratio][None], b, 0), np.repeat(sin_t[g * ratio][None], b, 0)
            rot, key = C.emit_group(carry[0], carry[1], ratio, nw, 1e-6, cg, sg, wk, kw, 1e-6)
            main[:, g] = Q.pack_latent_fp8_b128(rot)
            ka, ks = _keys(key[:, None], fmt)
            key_a[:, g], key_s[:, g] = ka[:, 0], ks[:, 0]
        assert np.array_equal(layer.main.cpu().numpy(), main), f"step {i} (position {pos}): main cache"
        ga, gs = (layer.k_codes, layer.k_scales) if fmt == "fp8" else (layer.k_packed, layer.k_e8m0)
        assert np.array_equal(ga.cpu().numpy(), key_a), f"step {i} (position {pos}): key codes"
        assert np.array_equal(gs.cpu().numpy().view(np.uint8), key_s.view(np.uint8)), f"step {i}: key scales"
        if coarse:
            ccarry[0][:, pos % cratio], ccarry[1][:, pos % cratio] = ins[6].numpy(), ins[7].numpy()
            if (pos + 1) % cratio == 0:
                g = (pos + 1) // cratio - 1
                cg, sg = np.repeat(cos_t[g * cratio][None], b, 0), np.repeat(sin_t[g * cratio][None], b, 0)
                rot, _ = C.emit_group(ccarry[0], ccarry[1], cratio, cnw, 1e-6, cg, sg)
                coarse_ent[:, g] = Q.pack_latent_fp8_b128(rot)
            assert np.array_equal(layer.coarse.cpu().numpy(), coarse_ent), f"step {i}: coarse cache"
        # indexer + top-k
        q_rot = C.rope(q_idx, cs[:, None], sn[:, None], dtype="bfloat16")
        if not merged:
            # the quantized indexer query the emission launch's prologue wrote
            qa, qsc = _keys(q_rot, fmt)
            gq = layer.q_codes.cpu().numpy().reshape(qa.shape)
            gqs = (layer.q_scales if fmt == "fp8" else layer.q_e8m0).cpu().numpy().reshape(qsc.shape)
            assert np.array_equal(gq, qa), f"step {i}: indexer query codes"
            assert np.array_equal(gqs.view(np.uint8), qsc.view(np.uint8)), f"step {i}: indexer query scales"
        qd = Q.fake_quant_fp8_block(q_rot, 128) if fmt == "fp8" else Q.fake_quant_fp4_block(q_rot, 32)
        kd = _dequant_keys(key_a, key_s, fmt)
        posv = torch.full((b, 1), pos)
        sc = OA.indexer_scores(torch.from_numpy(qd)[:, None], torch.from_numpy(kd), torch.from_numpy(w)[:, None],
                               ratio, posv)
        mag = OA.indexer_abs_scores(torch.from_numpy(qd)[:, None], torch.from_numpy(kd),
                                    torch.from_numpy(w)[:, None], ratio, posv)
        assert_scores_close(layer.scores[:, 0].cpu(), sc[:, 0], mag[:, 0])
        assert_topk_sets_match(layer.idx, sc[:, 0], mag[:, 0], topk)
        # attention over the window, the coarse entries and the GPU's own selection
        wd = Q.unpack_latent_fp8_b128(win)
        md = Q.unpack_latent_fp8_b128(main)
        qr = C.rope(q, cs[:, None], sn[:, None], dtype="bfloat16")
        idx = layer.idx.cpu().numpy()
        refs = []
        for r in range(b):
            ents = [wd[r, [(pos - W + 1 + j) % W for j in range(W)]]]
            if coarse:
                ents.append(Q.unpack_latent_fp8_b128(coarse_ent[r, :(pos + 1) // cratio]))
            ents.append(md[r, idx[r][idx[r] >= 0]])
            o, _ = OA.attend_entries(torch.from_numpy(qr[r]), torch.from_numpy(np.concatenate(ents)), sinks)
            refs.append(C.rope(o.numpy(), cs[r][None], sn[r][None], inverse=True))
        assert_attn_close(out, torch.from_numpy(np.stack(refs)), name=f"step {i} output")
    assert int(layer.positions[0]) == p0 + steps


def test_capture_advance_requires_emission(dev):
    cfg = DecodeConfig(batch=2, max_groups=64, topk=16)
    layer = SparseDecodeLayer(cfg, dev)
    ins = (torch.zeros(2, 128, D, dtype=torch.bfloat16, device=dev), None,
           torch.zeros(2, HI, DI, dtype=torch.bfloat16, device=dev), torch.zeros(2, HI, device=dev))
    with pytest.raises(ValueError, match="in-step group emission"):
        layer.capture(*ins, advance=True)


@pytest.mark.parametrize("ratio", [2, 8, 40, 128, 160])
def test_emission_kernels_agree(dev, ratio):
    """``mzk_decode_emit`` pools a keyless branch of ratio <= 128 on nine workgroups per row
    (the coarse branch's kernel) and a branch with an index key, or a longer ratio, on one
    workgroup per row: for the same group both write the same main-cache entry, bit for bit,
    equal to the oracle's packed entry; carry-only steps leave the entries alone."""
    from mzoo_amd import _lib
    b, cap = 3, 6
    rng = np.random.default_rng(ratio)
    groups = np.array([0, 2, 5])
    pos = (groups + 1) * ratio - 1  # every row completes its group
    rows = int(cap * ratio)
    tab = _bf(rng.uniform(-1, 1, (rows, 64)).astype(np.float32))
    nw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    wk = _bf(rng.normal(0, 0.05, (DI, D)).astype(np.float32))
    kw = _bf(rng.uniform(0.5, 1.5, DI).astype(np.float32))
    carry_kv = rng.normal(0, 1, (b, ratio, D)).astype(np.float32)
    carry_gate = rng.normal(0, 2, (b, ratio, D)).astype(np.float32)
    kv, gate = carry_kv[:, -1].copy(), carry_gate[:, -1].copy()
    carry_kv[:, -1] = carry_gate[:, -1] = 1e30  # the token's slot: written by the launch
    bf16 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).bfloat16().to(dev)  # noqa: E731
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731  (keeps the dtype)
    tab_d, nw_d, wk_d, kw_d = bf16(tab), bf16(nw), bf16(wk), bf16(kw)

    def emit(key, position):
        cache = torch.zeros(b, cap, 656, dtype=torch.uint8, device=dev)
        ckv, cgt = dv(carry_kv), dv(carry_gate)
        kc = torch.zeros(b, cap, DI, dtype=torch.uint8, device=dev)
        ks = torch.zeros(b, cap, dtype=torch.float32, device=dev)
        k = (wk_d.data_ptr(), kw_d.data_ptr(), 1e-6, 0, kc.data_ptr(), ks.data_ptr(), cap) if key else \
            (None, None, 0.0, 0, None, None, 0)
        p_d, kv_d, gate_d = dv(position), dv(kv), dv(gate)
        _lib.call("mzk_decode_emit", p_d.data_ptr(), b, kv_d.data_ptr(), gate_d.data_ptr(),
                  ckv.data_ptr(), cgt.data_ptr(), ratio, nw_d.data_ptr(), 1e-6, cache.data_ptr(), cap, cap, *k,
                  tab_d.data_ptr(), rows, None, None, None, None, 0.0, None, 0, 0, None, 0, None, None,
                  _lib.stream_of(cache))
        torch.cuda.synchronize()
        return cache.cpu().numpy(), ckv.cpu().numpy()

    pos_d = pos.astype(np.int64)
    plain, ckv_plain = emit(False, pos_d)
    keyed, _ = emit(True, pos_d)
    assert np.array_equal(plain, keyed)
    for r in range(b):
        g = groups[r]
        kvg = carry_kv[r:r + 1].copy()
        gtg = carry_gate[r:r + 1].copy()
        kvg[:, -1], gtg[:, -1] = kv[r], gate[r]
        cs, sn = tab[g * ratio:g * ratio + 1, :32], tab[g * ratio:g * ratio + 1, 32:]
        rot, _ = C.emit_group(kvg, gtg, ratio, nw, 1e-6, cs, sn)
        assert np.array_equal(plain[r, g], Q.pack_latent_fp8_b128(rot)[0]), f"row {r}: main entry"
        assert np.array_equal(ckv_plain[r, -1], kv[r]), f"row {r}: the token's carry slot"
    # a step that completes no group writes only the carry slot
    idle, ckv_idle = emit(False, pos_d - 1)
    assert not idle.any()
    for r in range(b):
        assert np.array_equal(ckv_idle[r, -2], kv[r])


def test_emission_pair_equals_two_launches(dev):
    """``mzk_decode_emit_pair`` (the fine branch with its index key and step tables, and a
    keyless coarse branch, in one launch) writes what the two ``mzk_decode_emit`` calls write,
    bit for bit -- caches, keys, carried slots, step tables -- over steps that complete groups
    of both branches and steps that only carry."""
    from mzoo_amd import _lib
    b, fr, cr, fcap, ccap = 3, 4, 8, 8, 4
    rng = np.random.default_rng(77)
    rows = 64
    tab = _bf(rng.uniform(-1, 1, (rows, 64)).astype(np.float32))
    nw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    cnw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    wk = _bf(rng.normal(0, 0.05, (DI, D)).astype(np.float32))
    kw = _bf(rng.uniform(0.5, 1.5, DI).astype(np.float32))
    bf16 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).bfloat16().to(dev)  # noqa: E731
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731  (keeps the dtype)
    tab_d, nw_d, cnw_d, wk_d, kw_d = bf16(tab), bf16(nw), bf16(cnw), bf16(wk), bf16(kw)

    def state():
        return dict(fkv=torch.zeros(b, fr, D, device=dev), fgt=torch.zeros(b, fr, D, device=dev),
                    ckv=torch.zeros(b, cr, D, device=dev), cgt=torch.zeros(b, cr, D, device=dev),
                    main=torch.zeros(b, fcap, 656, dtype=torch.uint8, device=dev),
                    coarse=torch.zeros(b, ccap, 656, dtype=torch.uint8, device=dev),
                    kc=torch.zeros(b, fcap, DI, dtype=torch.uint8, device=dev),
                    ks=torch.zeros(b, fcap, dtype=torch.float32, device=dev),
                    scos=torch.zeros(b, 32, dtype=torch.bfloat16, device=dev),
                    ssin=torch.zeros(b, 32, dtype=torch.bfloat16, device=dev))

    pair, two = state(), state()
    start = np.array([0, 5, 13], dtype=np.int64)
    for step in range(3 * cr):
        print(f"emission pair: step {step}", flush=True)
        pos_d = dv(start + step)
        kv, gt = dv(rng.normal(0, 1, (b, D)).astype(np.float32)), dv(rng.normal(0, 2, (b, D)).astype(np.float32))
        ckv, cgt = dv(rng.normal(0, 1, (b, D)).astype(np.float32)), dv(rng.normal(0, 2, (b, D)).astype(np.float32))
        st = _lib.stream_of(pos_d)
        for s, paired in ((pair, True), (two, False)):
            fine = (pos_d.data_ptr(), b, kv.data_ptr(), gt.data_ptr(), s["fkv"].data_ptr(), s["fgt"].data_ptr(), fr,
                    nw_d.data_ptr(), 1e-6, s["main"].data_ptr(), fcap, fcap, wk_d.data_ptr(), kw_d.data_ptr(), 1e-6, 0,
                    s["kc"].data_ptr(), s["ks"].data_ptr(), fcap, tab_d.data_ptr(), rows, s["scos"].data_ptr(),
                    s["ssin"].data_ptr(), None, None, 0.0, None, 0, 0, None, 0, None, None)
            coarse = (ckv.data_ptr(), cgt.data_ptr(), s["ckv"].data_ptr(), s["cgt"].data_ptr(), cr, cnw_d.data_ptr(),
                      1e-6, s["coarse"].data_ptr(), ccap, ccap)
            if paired:
                _lib.call("mzk_decode_emit_pair", *fine, *coarse, st)
            else:
                _lib.call("mzk_decode_emit", *fine, st)
                _lib.call("mzk_decode_emit", pos_d.data_ptr(), b, *coarse[:6], coarse[6], *coarse[7:], None, None,
                          0.0, 0, None, None, 0, tab_d.data_ptr(), rows, None, None, None, None, 0.0, None, 0, 0,
                          None, 0, None, None, st)
        torch.cuda.synchronize()
        for name in pair:
            assert torch.equal(pair[name], two[name]), f"step {step}: {name} differs"
    # groups of both branches were written
    assert pair["main"].any() and pair["coarse"].any() and pair["kc"].any()


@pytest.mark.parametrize("fmt,hi,cratio,cap,b", [("fp8", 64, 0, 1100, 5), ("mxfp4", 64, 0, 1100, 5),
                                                 ("fp8", 32, 0, 1100, 5), ("mxfp4", 20, 0, 1100, 5),
                                                 ("mxfp4", 64, 8, 1100, 5), ("fp8", 64, 40, 1100, 5),
                                                 ("fp8", 64, 0, 30000, 5), ("mxfp4", 64, 8, 30000, 5),
                                                 ("fp8", 64, 0, 60000, 5), ("mxfp4", 64, 8, 60000, 5),
                                                 ("fp8", 64, 0, 720, 300), ("mxfp4", 32, 8, 720, 300)])
def test_emit_scores_equals_two_launches(dev, fmt, hi, cratio, cap, b):
    """``mzk_decode_emit_scores`` (the emission, the window entry, the indexer query's RoPE +
    quantization and the scores in one launch, the new key scored by its emission workgroup;
    with ``cratio`` a keyless coarse branch too) writes what the emission launch followed by
    the fused scorer (``mzk_decode_emit`` / ``mzk_decode_emit_pair`` + ``mzk_indexer_decode_fused``
    on the step's tables) writes, bit for bit -- carries, main and coarse caches, keys, window
    ring, step tables and every score -- over steps that complete groups and steps that only
    carry, with an inactive row (position -1) and a key axis of several scoring workgroups
    with a partial last one.  The key axis takes each form of the scoring workgroups: four
    tiles per wave (``cap`` 1100), eight (30000) and sixteen (60000: the 16-tile ring); 300
    rows make the grid larger than one round of resident workgroups."""
    from mzoo_amd import _lib
    ratio, wcap, ccap = 4, 16, 120
    rows_tab = 4 * cap + 8
    steps = max(2 * ratio, cratio) + 1
    rng = np.random.default_rng(5 + hi + cratio)
    tab = _bf(rng.uniform(-1, 1, (rows_tab, 64)).astype(np.float32))
    nw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    cnw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    kvw = _bf(rng.uniform(0.5, 1.5, D).astype(np.float32))
    wk = _bf(rng.normal(0, 0.05, (DI, D)).astype(np.float32))
    kw = _bf(rng.uniform(0.5, 1.5, DI).astype(np.float32))
    bf16 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().to(dev)  # noqa: E731
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731  (keeps the dtype)
    tab_d, nw_d, cnw_d, kvw_d, wk_d, kw_d = bf16(tab), bf16(nw), bf16(cnw), bf16(kvw), bf16(wk), bf16(kw)
    ka, ks = _keys(_bf(rng.normal(0, 1, (b, cap, DI)).astype(np.float32)), fmt)
    fp8 = fmt == "fp8"

    def state():
        s = dict(ckv=torch.zeros(b, ratio, D, device=dev), cgt=torch.zeros(b, ratio, D, device=dev),
                 main=torch.zeros(b, cap, 656, dtype=torch.uint8, device=dev),
                 ka=dv(ka), ks=dv(ks), win=torch.zeros(b, wcap, 656, dtype=torch.uint8, device=dev),
                 scos=torch.zeros(b, 32, dtype=torch.bfloat16, device=dev),
                 ssin=torch.zeros(b, 32, dtype=torch.bfloat16, device=dev),
                 scores=torch.full((b, cap), 7.0, device=dev))
        if cratio:
            s.update(cckv=torch.zeros(b, cratio, D, device=dev), ccgt=torch.zeros(b, cratio, D, device=dev),
                     coarse=torch.zeros(b, ccap, 656, dtype=torch.uint8, device=dev))
        return s

    one, two = state(), state()
    key_half = torch.zeros(b, 40, dtype=torch.int64, device=dev)  # the merged launch's handoff
    # five phases of the group (an inactive row first), repeated with shifts for more rows
    start = np.array([-1, 0, 5, 13, 4 * 700 + 2], dtype=np.int64)
    if b > 5:
        start = np.array([start[i % 5] + (i // 5) % 4 if i % 5 else -1 for i in range(b)], dtype=np.int64)
    for step in range(steps):
        print(f"emit+scores ({fmt}, Hi={hi}, coarse ratio {cratio}, G={cap}): step {step}", flush=True)
        pos_d = dv(start + step)
        kv, gt = dv(rng.normal(0, 1, (b, D)).astype(np.float32)), dv(rng.normal(0, 2, (b, D)).astype(np.float32))
        ckv_in, cgt_in = dv(rng.normal(0, 1, (b, D)).astype(np.float32)), dv(rng.normal(0, 2, (b, D)).astype(np.float32))
        kvp = bf16(rng.normal(0, 3, (b, D)).astype(np.float32))
        q_idx = bf16(rng.normal(0, 1, (b, hi, DI)).astype(np.float32))
        w = dv((rng.normal(0, 1, (b, hi)) * hi ** -0.5).astype(np.float32))
        st = _lib.stream_of(pos_d)
        for s, merged in ((one, True), (two, False)):
            emit = (pos_d.data_ptr(), b, kv.data_ptr(), gt.data_ptr(), s["ckv"].data_ptr(), s["cgt"].data_ptr(),
                    ratio, nw_d.data_ptr(), 1e-6, s["main"].data_ptr(), cap, cap, wk_d.data_ptr(), kw_d.data_ptr(),
                    1e-6, 0 if fp8 else 1, s["ka"].data_ptr(), s["ks"].data_ptr(), cap, tab_d.data_ptr(), rows_tab,
                    s["scos"].data_ptr(), s["ssin"].data_ptr())
            coarse = (ckv_in.data_ptr(), cgt_in.data_ptr(), s["cckv"].data_ptr(), s["ccgt"].data_ptr(), cratio,
                      cnw_d.data_ptr(), 1e-6, s["coarse"].data_ptr(), ccap, ccap) if cratio else \
                (None,) * 4 + (0, None, 0.0, None, 0, 0)
            if merged:
                _lib.call("mzk_decode_emit_scores", *emit, kvp.data_ptr(), kvw_d.data_ptr(), 1e-6,
                          s["win"].data_ptr(), wcap, wcap, q_idx.data_ptr(), w.data_ptr(), hi, cap,
                          s["scores"].data_ptr(), cap, *coarse, key_half.data_ptr(), st)
            else:
                no_pro = (None, None, 0.0, None, 0, 0, None, 0, None, None)
                if cratio:
                    _lib.call("mzk_decode_emit_pair", *emit, *no_pro, *coarse, st)
                else:
                    _lib.call("mzk_decode_emit", *emit, *no_pro, st)
                _lib.call("mzk_indexer_decode_fused", 0 if fp8 else 1, q_idx.data_ptr(), w.data_ptr(),
                          s["ka"].data_ptr(), s["ks"].data_ptr(), b, hi, DI, cap, cap, pos_d.data_ptr(), ratio,
                          s["scores"].data_ptr(), cap, None, None, s["scos"].data_ptr(), s["ssin"].data_ptr(), 64,
                          kvp.data_ptr(), kvw_d.data_ptr(), 1e-6, s["scos"].data_ptr(), s["ssin"].data_ptr(), 512,
                          64, s["win"].data_ptr(), wcap, wcap, st)
        torch.cuda.synchronize()
        for name in one:
            a, c = one[name], two[name]
            same = torch.equal(a.view(torch.int32), c.view(torch.int32)) if a.dtype == torch.float32 \
                else torch.equal(a, c)
            assert same, f"step {step}: {name} differs"
    # groups were emitted and the window written; each row's last step scored exactly its
    # visible keys, min(cap, (pos + 1) // ratio), the last of them emitted by that step or before
    assert one["main"].any() and one["win"].any()
    if cratio:
        assert one["coarse"].any()
    last = start + steps - 1
    finite = torch.isfinite(one["scores"]).sum(1).cpu().numpy()
    assert np.array_equal(finite, np.minimum(cap, (last + 1) // ratio)), finite
    # the handoff: one count per group step that emits a key, no wait given up
    kh = key_half.cpu().numpy()
    groups = [sum((q + 1) % ratio == 0 and q >= 0 and (q + 1) // ratio - 1 < cap and (q + 1) // ratio * ratio - ratio
                  < rows_tab for q in range(s0, s0 + steps)) for s0 in start]
    assert np.array_equal(kh[:, 0], np.array(groups)) and not kh[:, 33].any(), (kh[:, 0], groups)
