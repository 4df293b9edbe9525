"""GPU parity of the indexer score kernels (piece 3) and the top-k kernel (piece 4).

Scores: against ``oracle.attention.indexer_scores`` (fp32 einsum on the dequantized
operands) within ``SCORE_RTOL`` (1e-5) relative to ``sum_h |w_h| relu(q.k) Di^-0.5``;
the group-causal ``-inf`` mask must be identical.  Top-k: bit-exact index lists against
``oracle.attention.topk_indices`` (same scores in, deliberate ties included); end to end
(scores + top-k) the sets must equal the oracle's except at near-ties of the k-th score.
Shapes follow the reference tests (``layers/attn/indexer/fwd_test.py:52-83``,
``attn_test.py:126-139``) plus the BASELINE decode shapes.
"""

import json
import pathlib

import numpy as np
import pytest
import torch

from mzoo_amd import indexer as MI
from mzoo_amd import quant as MQ
from oracle import attention as OA
from oracle import quant as Q
from tests.helpers import assert_scores_close, assert_topk_sets_match

pytestmark = pytest.mark.gpu
KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "kat.json").read_text())


def _inputs(b, s, hi, di, g, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, hi, di, generator=gen).bfloat16()
    k = torch.randn(b, g, di, generator=gen).bfloat16()
    w = torch.randn(b, s, hi, generator=gen) * hi ** -0.5
    return q, k, w


# ---- top-k ------------------------------------------------------------------------------

def test_topk_kat_dummy_slot(dev):
    k = KAT["topk_dummy_slot"]
    sc = torch.tensor([[[1.0, 2.0, float("-inf"), float("-inf")]]], device=dev)
    idx = MI.topk(sc, k["topk"])
    assert sorted(idx[0, 0, :2].tolist()) == k["first_set"] and idx[0, 0, 2:].tolist() == k["tail"]
    idx = MI.topk(sc[..., :k["padded_scores_cols"]], k["padded_topk"])
    assert sorted(idx[0, 0, :2].tolist()) == k["first_set"] and idx[0, 0, 2:].tolist() == k["padded_tail"]


@pytest.mark.parametrize("rows,g,k", [(32, 8192, 2048), (8, 32768, 2048), (4, 131072, 2048), (7, 1000, 128),
                                      (3, 100, 135), (5, 4097, 4096), (2, 0, 16), (64, 256, 1), (3, 8000, 5000)])
def test_topk_exact_with_ties(dev, rows, g, k):
    gen = torch.Generator().manual_seed(rows * 7 + g)
    sc = torch.randn(rows, g, generator=gen)
    sc = torch.round(sc * 64) / 64                     # heavy ties
    if g:
        sc[:, ::7] = float("-inf")                     # invisible entries
        sc[0, :] = float("-inf")                       # a row with nothing visible
        sc[-1, g // 2:] = float("-inf")                # a row with fewer visible than k
        if rows > 2:
            sc[1, :] = 0.25                             # a row of all-equal scores
    got = MI.topk(sc.to(dev), k).cpu().numpy()
    want = OA.topk_indices(sc.numpy(), k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,g,k,kind", [(4, 131072, 2048, "distinct"), (3, 40003, 2048, "distinct"),
                                           (2, 524288, 2048, "distinct"), (5, 16384, 16384, "ties"),
                                           (2, 40000, 40000, "ties"), (6, 9000, 100, "ties"),
                                           (6, 33000, 100, "ties"), (4, 65536, 4096, "three_values"),
                                           (3, 20000, 2048, "negative"), (3, 36000, 2048, "negative"),
                                           (2, 30000, 2048, "three_values")])
def test_topk_long_rows_split_over_workgroups(dev, rows, g, k, kind):
    """Rows of 32769 .. 524288 scores go through mzk_topk_rows_ws (chunk histograms ->
    per-row selection -> index-ordered write), shorter ones through the single-workgroup
    kernel: exact against the oracle, and the workspace entry equal to mzk_topk_rows.  'distinct' keeps the k-th key's bin small (its keys are
    selected in LDS); 'three_values' puts tens of thousands of equal keys in that bin (the
    selection streams the row instead); partial last chunks, k = G, -inf entries and rows
    with fewer visible entries than k are covered too."""
    from mzoo_amd import _lib
    gen = torch.Generator().manual_seed(rows * 13 + g)
    if kind == "distinct":
        sc = torch.randn(rows, g, generator=gen)
    elif kind == "ties":
        sc = torch.round(torch.randn(rows, g, generator=gen) * 16) / 16
        sc[:, ::5] = float("-inf")
        sc[-1, g // 3:] = float("-inf")
    elif kind == "three_values":
        sc = torch.randint(0, 3, (rows, g), generator=gen).float()
    else:
        sc = -torch.rand(rows, g, generator=gen) - 1.0
        sc[0, :] = float("-inf")
    assert (MI.topk_workspace_bytes(rows, g) > 0) == (g > 32768)
    got = MI.topk(sc.to(dev), k).cpu().numpy()
    want = OA.topk_indices(sc.numpy(), k)
    assert np.array_equal(got, want)
    single = torch.empty(rows, k, dtype=torch.int32, device=dev)
    scd = sc.to(dev)
    _lib.call("mzk_topk_rows", scd.data_ptr(), rows, g, g, k, single.data_ptr(), k, _lib.stream_of(scd))
    assert np.array_equal(single.cpu().numpy(), want)


def test_topk_long_rows_reuse_one_workspace(dev):
    """One workspace serves calls of different row counts, lengths, data and k in a row,
    never cleared: every launch writes the state the next one reads (chunk histograms,
    counts, the per-row selection, the candidates it reads back), so no call depends on
    what an earlier call left.  The workspace starts filled with garbage to show it needs
    no initialization."""
    shapes = [(4, 131072, 2048, "distinct"), (8, 65537, 512, "ties"), (2, 262144, 4096, "three_values"),
              (4, 131072, 2048, "distinct"), (1, 524288, 16384, "negative"), (8, 40000, 2048, "ties")]
    size = max(MI.topk_workspace_bytes(r, g) for r, g, _, _ in shapes)
    assert size > 0
    ws = torch.randint(-2**31, 2**31 - 1, ((size + 15) // 16 * 4,), dtype=torch.int32, device=dev)
    for i, (rows, g, k, kind) in enumerate(shapes):
        gen = torch.Generator().manual_seed(1000 + i)
        if kind == "distinct":
            sc = torch.randn(rows, g, generator=gen)
        elif kind == "ties":
            sc = torch.round(torch.randn(rows, g, generator=gen) * 8) / 8
            sc[:, 3::7] = float("-inf")
        elif kind == "three_values":
            sc = torch.randint(0, 3, (rows, g), generator=gen).float()
        else:
            sc = -torch.rand(rows, g, generator=gen) - 1.0
        got = MI.topk(sc.to(dev), k, workspace=ws).cpu().numpy()
        assert np.array_equal(got, OA.topk_indices(sc.numpy(), k)), (i, rows, g, k, kind)


@pytest.mark.parametrize("case", ["distinct", "near_lowest_float", "mixed_sign_few_exponents"])
def test_topk_exact_distinct_and_extreme(dev, case):
    """Distinct scores (the radix search usually stops once the k-th key's bin is taken
    whole), finite scores next to -FLT_MAX (the k-th key's leading byte is 0), and scores
    sharing a handful of exponents."""
    gen = torch.Generator().manual_seed(11)
    rows, g, k = 16, 8192, 2048
    if case == "distinct":
        sc = torch.randn(rows, g, generator=gen)
    elif case == "near_lowest_float":
        sc = -3.4e38 * (0.55 + 0.45 * torch.rand(rows, g, generator=gen))
        sc[:, ::5] = float("-inf")
    else:
        sc = torch.sign(torch.randn(rows, g, generator=gen)) * torch.exp2(torch.randint(-2, 3, (rows, g), generator=gen).float())
        sc = sc * (1 + torch.rand(rows, g, generator=gen) * 2 ** -20)
    got = MI.topk(sc.to(dev), k).cpu().numpy()
    want = OA.topk_indices(sc.numpy(), k)
    assert np.array_equal(got, want)

# ---- scores -----------------------------------------------------------------------------

@pytest.mark.parametrize("hi", [4, 32, 64])
@pytest.mark.parametrize("di", [64, 96, 128, 256])
def test_bf16_scores_match_oracle(dev, hi, di):
    q, k, w = _inputs(2, 256, hi, di, 128)
    got = MI.fwd(q.to(dev), k.to(dev), w.to(dev), compress_ratio=2)
    ref = OA.indexer_scores(q.float(), k.float(), w, 2)
    assert_scores_close(got, ref, OA.indexer_abs_scores(q.float(), k.float(), w, 2))


@pytest.mark.parametrize("ratio,g", [(1, 256), (4, 64), (2, 400), (2, 7)])
def test_bf16_ratios_and_lengths(dev, ratio, g):
    q, k, w = _inputs(1, 256, 32, 128, g, seed=ratio)
    got = MI.fwd(q.to(dev), k.to(dev), w.to(dev), compress_ratio=ratio)
    ref = OA.indexer_scores(q.float(), k.float(), w, ratio)
    assert_scores_close(got, ref, OA.indexer_abs_scores(q.float(), k.float(), w, ratio))


def test_bf16_empty_kv(dev):
    q, k, w = _inputs(1, 16, 32, 128, 0)
    assert MI.fwd(q.to(dev), k.to(dev), w.to(dev), compress_ratio=2).shape == (1, 16, 0)
    idx = MI.attn(q.to(dev), k.to(dev), w.to(dev), compress_ratio=2, topk=64)
    assert idx.shape == (1, 16, 64) and bool((idx == -1).all())


@pytest.mark.parametrize("topk", [64, 135])
@pytest.mark.parametrize("ratio", [1, 2, 4])
def test_attn_indices_match_oracle(dev, ratio, topk):
    q, k, w = _inputs(2, 256, 32, 128, 128, seed=10 + ratio)
    got = MI.attn(q.to(dev), k.to(dev), w.to(dev), compress_ratio=ratio, topk=topk)
    assert got.dtype == torch.int32 and got.shape == (2, 256, topk)
    ref = OA.indexer_scores(q.float(), k.float(), w, ratio)
    assert_topk_sets_match(got, ref, OA.indexer_abs_scores(q.float(), k.float(), w, ratio), topk)


def _fp8_operands(q, k):
    di = q.shape[-1]
    qc, qs = Q.fp8_block_codes(q.float().numpy(), di)
    kc, ks = Q.fp8_block_codes(k.float().numpy(), di)
    qd = torch.from_numpy(Q.dequant_fp8_block(qc, qs, di))
    kd = torch.from_numpy(Q.dequant_fp8_block(kc, ks, di))
    return (torch.from_numpy(qc), torch.from_numpy(qs[..., 0]), torch.from_numpy(kc), torch.from_numpy(ks[..., 0]),
            qd, kd)


@pytest.mark.parametrize("b,s,g,ratio,pos", [(32, 1, 8192, 4, 32767), (2, 64, 512, 2, None), (3, 1, 1000, 4, 2000)])
def test_fp8_scores_match_oracle(dev, b, s, g, ratio, pos):
    q, k, w = _inputs(b, s, 64, 128, g, seed=g)
    qc, qs, kc, ks, qd, kd = _fp8_operands(q, k)
    positions = None if pos is None else torch.full((b, s), pos, dtype=torch.int64)
    got = MI.scores_fp8(qc.to(dev), qs.to(dev), w.to(dev), kc.to(dev), ks.to(dev), compress_ratio=ratio,
                        positions=None if positions is None else positions.to(dev))
    ref = OA.indexer_scores(qd, kd, w, ratio, positions)
    assert_scores_close(got, ref, OA.indexer_abs_scores(qd, kd, w, ratio, positions))


@pytest.mark.parametrize("b,s,hi,g,ratio,base", [(2, 300, 64, 1000, 4, None), (1, 200, 40, 700, 1, 5000),
                                                  (1, 128, 64, 64, 4, None), (3, 64, 64, 2048, 4, 0)])
def test_fp8_prefill_kernel_matches_row_kernel(dev, b, s, hi, g, ratio, base):
    """From 64 rows per batch the FP8 scores run the prefill tiling (key tiles held, query
    rows streamed); it sums in the row kernel's order, so the scores must equal, bit for
    bit, the row kernel's over chunks of 32 rows with the same positions (ragged row and
    key counts, fewer than 64 heads, chunked-prefill positions, fully masked key blocks)."""
    q, k, w = _inputs(b, s, hi, 128, g, seed=s + g)
    qc, qs, kc, ks, qd, kd = _fp8_operands(q, k)
    pos = torch.arange(s, dtype=torch.int64).expand(b, s) + (0 if base is None else base)
    qc, qs, w_d, kc, ks = (t.to(dev) for t in (qc, qs, w, kc, ks))
    print(f"prefill fp8 scores: B={b} S={s} Hi={hi} G={g} ratio={ratio} base={base}", flush=True)
    full = MI.scores_fp8(qc, qs, w_d, kc, ks, compress_ratio=ratio, positions=None if base is None else pos.to(dev))
    parts = [MI.scores_fp8(qc[:, c:c + 32], qs[:, c:c + 32], w_d[:, c:c + 32], kc, ks, compress_ratio=ratio,
                           positions=pos[:, c:c + 32].to(dev)) for c in range(0, s, 32)]
    rows = [0, 31, 32, s // 2, s - 1]
    ref = OA.indexer_scores(qd[:, rows], kd, w[:, rows], ratio, pos[:, rows])
    mag = OA.indexer_abs_scores(qd[:, rows], kd, w[:, rows], ratio, pos[:, rows])
    chunked = torch.cat(parts, 1)
    assert_scores_close(chunked[:, rows], ref, mag)
    assert_scores_close(full[:, rows], ref, mag)
    assert torch.equal(full, chunked)


def test_fp8_quantizer_feeds_scores(dev):
    """GPU quantizer -> GPU scores equals oracle quantizer -> oracle scores."""
    q, k, w = _inputs(4, 1, 64, 128, 2048, seed=3)
    qc, qs = MQ.quant_fp8_block(q.to(dev), 128)
    kc, ks = MQ.quant_fp8_block(k.to(dev), 128)
    pos = torch.full((4, 1), 8191, dtype=torch.int64, device=dev)
    got = MI.scores_fp8(qc, qs[..., 0], w.to(dev), kc, ks[..., 0], compress_ratio=4, positions=pos)
    _, _, _, _, qd, kd = _fp8_operands(q, k)
    ref = OA.indexer_scores(qd, kd, w, 4, pos.cpu())
    assert_scores_close(got, ref, OA.indexer_abs_scores(qd, kd, w, 4, pos.cpu()))


@pytest.mark.parametrize("b,s,g,ratio,pos", [(8, 1, 4096, 4, 16383), (2, 32, 256, 2, None), (1, 1, 300, 1, 150)])
def test_mxfp4_scores_match_oracle(dev, b, s, g, ratio, pos):
    q, k, w = _inputs(b, s, 64, 128, g, seed=g + 1)
    qp, qe = Q.quant_mxfp4(q.float().numpy())
    kp, ke = Q.quant_mxfp4(k.float().numpy())
    qd, kd = torch.from_numpy(Q.dequant_mxfp4(qp, qe)), torch.from_numpy(Q.dequant_mxfp4(kp, ke))
    positions = None if pos is None else torch.full((b, s), pos, dtype=torch.int64)
    got = MI.scores_mxfp4(torch.from_numpy(qp).to(dev), torch.from_numpy(qe).to(dev), w.to(dev),
                          torch.from_numpy(kp).to(dev), torch.from_numpy(ke).to(dev), compress_ratio=ratio,
                          positions=None if positions is None else positions.to(dev))
    ref = OA.indexer_scores(qd, kd, w, ratio, positions)
    assert_scores_close(got, ref, OA.indexer_abs_scores(qd, kd, w, ratio, positions))


def test_fp8_decode_topk_end_to_end(dev):
    """BASELINE config-2 indexer: B=32 rows at position 32767, 8192 FP8 keys, top-2048."""
    q, k, w = _inputs(32, 1, 64, 128, 8192, seed=2)
    qc, qs, kc, ks, qd, kd = _fp8_operands(q, k)
    pos = torch.full((32, 1), 32767, dtype=torch.int64)
    sc = MI.scores_fp8(qc.to(dev), qs.to(dev), w.to(dev), kc.to(dev), ks.to(dev), compress_ratio=4,
                       positions=pos.to(dev))
    idx = MI.topk(sc, 2048)
    ref = OA.indexer_scores(qd, kd, w, 4, pos)
    assert_topk_sets_match(idx, ref, OA.indexer_abs_scores(qd, kd, w, 4, pos), 2048)


@pytest.mark.parametrize("b,hi,g,append", [(5, 64, 1000, True), (3, 20, 512, True), (4, 64, 2048, False)])
def test_fused_decode_indexer_fp8(dev, b, hi, g, append):
    """mzk_indexer_decode_fp8 = query quantization + window append + FP8 scores in one
    launch: the quantized query and the appended window entry are bit-exact against the
    oracle's quantizer / packer, and the scores are bit-identical to the two-launch path
    (mzk_indexer_scores_fp8 on the oracle-quantized query), within tolerance of the
    oracle's fp32 scores, with the group-causal mask."""
    q, k, w = _inputs(b, 1, hi, 128, g, seed=hi + g)
    q = q[:, 0]                                                     # [B, Hi, 128]
    q[0, 0, :5] = torch.tensor([0.0, -0.0, 1e-30, 3e-3, -6.0])     # zeros, underflow, the block max
    q[1 % b, hi - 1] = 0                                             # an all-zero head (scale floor)
    qc_ref, qs_ref = Q.fp8_block_codes(q.float().numpy(), 128)
    _, _, kc, ks, qd, kd = _fp8_operands(q[:, None], k)
    pos = torch.tensor([4 * g - 1, 37, 4 * g + 9, 0, 1000][:b], dtype=torch.int64)
    wcap = 16
    kv = torch.randn(b, 576, generator=torch.Generator().manual_seed(b)).bfloat16()
    win = torch.zeros(b, wcap, 656, dtype=torch.uint8, device=dev)
    q_codes = torch.zeros(b, hi, 128, dtype=torch.uint8, device=dev)
    q_scales = torch.zeros(b, hi, dtype=torch.float32, device=dev)
    got = MI.decode_fp8(q.to(dev), w[:, 0].to(dev), kc.to(dev), ks.to(dev), compress_ratio=4,
                        positions=pos.to(dev), q_codes=q_codes, q_scales=q_scales,
                        kv=kv.to(dev) if append else None, win_cache=win if append else None)
    assert np.array_equal(q_codes.cpu().numpy().reshape(qc_ref.shape), qc_ref)
    assert np.array_equal(q_scales.cpu().numpy().reshape(qs_ref.shape).view(np.int32), qs_ref.view(np.int32))
    wc = win.cpu().numpy()
    if append:
        want = Q.pack_latent_fp8_b128(kv.float().numpy())
        for r in range(b):
            assert np.array_equal(wc[r, int(pos[r]) % wcap], want[r])
            others = [i for i in range(wcap) if i != int(pos[r]) % wcap]
            assert not wc[r, others].any()
    else:
        assert not wc.any()
    two = MI.scores_fp8(torch.from_numpy(qc_ref).reshape(b, 1, hi, 128).to(dev),
                        torch.from_numpy(qs_ref).reshape(b, 1, hi).to(dev), w.to(dev), kc.to(dev), ks.to(dev),
                        compress_ratio=4, positions=pos.view(b, 1).to(dev))
    assert torch.equal(got, two)
    ref = OA.indexer_scores(qd, kd, w, 4, pos.view(b, 1))
    assert_scores_close(got, ref, OA.indexer_abs_scores(qd, kd, w, 4, pos.view(b, 1)))


@pytest.mark.parametrize("b,hi,g,append", [(5, 64, 1000, True), (3, 20, 512, True), (4, 64, 2048, False)])
def test_fused_decode_indexer_mxfp4(dev, b, hi, g, append):
    """mzk_indexer_decode_mxfp4 = query MXFP4 quantization + window append + MXFP4 scores in
    one launch: the packed query and its e8m0 scales, and the appended window entry, are
    bit-exact against the oracle's quantizer / packer; the scores are bit-identical to the
    two-launch path (mzk_indexer_scores_mxfp4 on the oracle-quantized query) and within
    tolerance of the oracle's fp32 scores, with the group-causal mask."""
    q, k, w = _inputs(b, 1, hi, 128, g, seed=2 * hi + g)
    q = q[:, 0]                                                     # [B, Hi, 128]
    q[0, 0, :6] = torch.tensor([0.0, -0.0, 1e-30, 3e-3, -6.0, 0.25])  # zeros, underflow, ties of the grid
    q[1 % b, hi - 1] = 0                                             # an all-zero head (scale floor)
    qp_ref, qe_ref = Q.quant_mxfp4(q.float().numpy())
    kp, ke = Q.quant_mxfp4(k.float().numpy())
    qd, kd = torch.from_numpy(Q.dequant_mxfp4(qp_ref, qe_ref)), torch.from_numpy(Q.dequant_mxfp4(kp, ke))
    pos = torch.tensor([4 * g - 1, 37, 4 * g + 9, 0, 1000][:b], dtype=torch.int64)
    wcap = 16
    kv = torch.randn(b, 576, generator=torch.Generator().manual_seed(b + 1)).bfloat16()
    win = torch.zeros(b, wcap, 656, dtype=torch.uint8, device=dev)
    q_packed = torch.zeros(b, hi, 64, dtype=torch.uint8, device=dev)
    q_e8m0 = torch.zeros(b, hi, 4, dtype=torch.uint8, device=dev)
    kpd, ked = torch.from_numpy(kp).to(dev), torch.from_numpy(ke).to(dev)
    got = MI.decode_mxfp4(q.to(dev), w[:, 0].to(dev), kpd, ked, compress_ratio=4, positions=pos.to(dev),
                          q_packed=q_packed, q_e8m0=q_e8m0, kv=kv.to(dev) if append else None,
                          win_cache=win if append else None)
    assert np.array_equal(q_packed.cpu().numpy(), qp_ref)
    assert np.array_equal(q_e8m0.cpu().numpy(), qe_ref)
    wc = win.cpu().numpy()
    if append:
        want = Q.pack_latent_fp8_b128(kv.float().numpy())
        for r in range(b):
            assert np.array_equal(wc[r, int(pos[r]) % wcap], want[r])
            others = [i for i in range(wcap) if i != int(pos[r]) % wcap]
            assert not wc[r, others].any()
    else:
        assert not wc.any()
    two = MI.scores_mxfp4(torch.from_numpy(qp_ref).reshape(b, 1, hi, 64).to(dev),
                          torch.from_numpy(qe_ref).reshape(b, 1, hi, 4).to(dev), w.to(dev), kpd, ked,
                          compress_ratio=4, positions=pos.view(b, 1).to(dev))
    assert torch.equal(got, two)
    ref = OA.indexer_scores(qd.unsqueeze(1), kd, w, 4, pos.view(b, 1))
    assert_scores_close(got, ref, OA.indexer_abs_scores(qd.unsqueeze(1), kd, w, 4, pos.view(b, 1)))


@pytest.mark.parametrize("b,s,t,bs,k,kind", [(2, 3, 13, 8, 1, "distinct"), (2, 5, 1000, 8, 20, "ties"),
                                             (1, 4, 16384, 8, 2048, "distinct"), (1, 2, 65536, 8, 2048, "ties"),
                                             (3, 2, 37, 4, 50, "distinct"), (1, 3, 40, 8, 2, "all_masked")])
def test_select_candidate_blocks(dev, b, s, t, bs, k, kind):
    """Level one of the two-level top-k (owlet1/indexer.py:14-40) against the oracle: bool
    mask equal, with the newest partial block pinned, unreachable blocks dropped, T not a
    multiple of the block size and the ticket-0009 sizes; ties resolve to the lower block
    (the same rule in both)."""
    gen = torch.Generator().manual_seed(b * 7 + t)
    logits = torch.randn(b, s, t, generator=gen)
    if kind == "ties":
        logits = torch.round(logits * 4) / 4
    pos = torch.randint(0, 4 * t, (b, s), generator=gen)
    lens = ((pos + 1) // 4).clamp(max=t).unsqueeze(-1)
    if kind == "all_masked":
        lens[0, 0, 0] = 0
    logits = logits.masked_fill(torch.arange(t).view(1, 1, -1) >= lens, float("-inf"))
    got = MI.select_candidate_blocks(logits.to(dev), lens.to(dev), k, bs)
    assert got.dtype == torch.bool and got.shape == logits.shape
    want = OA.select_candidate_blocks(logits.numpy(), lens.numpy(), k, bs)
    assert np.array_equal(got.cpu().numpy(), want)
