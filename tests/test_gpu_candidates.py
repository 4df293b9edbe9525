"""GPU parity of the two-level selection's level two (the candidate scorer).

Level two replaces a candidate-using layer's dense scores plus
``index_scores.masked_fill(~candidates, -inf)`` (owlet1/indexer.py:150-151) and its top-k
(:158-161) by scores over the gathered candidates only
(tickets/0009-indexer-hierarchical.md:29-32).  Checks:

* a candidate slot's score has the same bits as the dense row kernel's score of its key
  (which the indexer tests pin to the oracle at 1e-5); empty, out-of-range and not yet
  visible slots are ``-inf``;
* level one's compact block list expands to the oracle's bool mask;
* the candidate top-k, mapped back to key positions, equals the oracle's top-k of the dense
  scores masked with ``~candidates`` (same lowest-index tie rule), ties included.
"""

import numpy as np
import pytest
import torch

from mzoo_amd import indexer as MI
from oracle import attention as OA
from oracle import quant as Q

pytestmark = pytest.mark.gpu
NEG = float("-inf")


def _inputs(b, s, hi, g, seed, ties=False):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, hi, 128, generator=gen).bfloat16()
    k = torch.randn(b, g, 128, generator=gen).bfloat16()
    if ties:  # odd keys repeat their even neighbour: equal scores at adjacent positions
        k[:, 1::2] = k[:, 0::2][:, :k[:, 1::2].shape[1]]
    w = torch.randn(b, s, hi, generator=gen) * hi ** -0.5
    return q, k, w


def _fp8(q, k):
    qc, qs = Q.fp8_block_codes(q.float().numpy(), 128)
    kc, ks = Q.fp8_block_codes(k.float().numpy(), 128)
    return [torch.from_numpy(x) for x in (qc, qs[..., 0], kc, ks[..., 0])]


def _mxfp4(q, k):
    qp, qe = Q.quant_mxfp4(q.float().numpy())
    kp, ke = Q.quant_mxfp4(k.float().numpy())
    return [torch.from_numpy(x) for x in (qp, qe, kp, ke)]


def _random_lists(b, s, g, bs, nb, seed, extra_blocks=0):
    """Per row: a random ascending set of distinct blocks (some beyond the cache when
    ``extra_blocks``), then -1 up to nb."""
    gen = torch.Generator().manual_seed(seed)
    total = -(-g // bs) + extra_blocks
    out = torch.full((b, s, nb), -1, dtype=torch.int32)
    for r in range(b * s):
        n = int(torch.randint(0, min(nb, total) + 1, (1,), generator=gen)) if r else min(nb, total)
        pick = torch.randperm(total, generator=gen)[:n].sort().values
        out.view(-1, nb)[r, :n] = pick.int()
    return out


def _gather(dense, cand, bs, g):
    """Host restatement of the candidate axis: slot j <- dense[key(j)] or -inf."""
    b, s, nb = cand.shape
    j = torch.arange(nb * bs)
    blk = cand[..., j // bs].long()
    key = blk * bs + j % bs
    valid = (blk >= 0) & (key < g)
    out = torch.full((b, s, nb * bs), NEG)
    picked = dense.gather(-1, key.clamp(0, max(g - 1, 0)))
    out[valid] = picked[valid]
    return out


def _scores(fmt, ops, w, dev, ratio, pos, cand=None, bs=8):
    ops = [t.to(dev) for t in ops]
    kw = dict(compress_ratio=ratio, positions=pos.to(dev))
    if fmt == "fp8":
        if cand is None:
            return MI.scores_fp8(ops[0], ops[1], w.to(dev), ops[2], ops[3], **kw)
        return MI.candidate_scores_fp8(ops[0], ops[1], w.to(dev), ops[2], ops[3], cand.to(dev), block_size=bs, **kw)
    if cand is None:
        return MI.scores_mxfp4(ops[0], ops[1], w.to(dev), ops[2], ops[3], **kw)
    return MI.candidate_scores_mxfp4(ops[0], ops[1], w.to(dev), ops[2], ops[3], cand.to(dev), block_size=bs, **kw)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
@pytest.mark.parametrize("b,s,hi,g,bs,nb,ratio,pos", [
    (4, 1, 64, 65531, 8, 2048, 4, 262000),   # partial last block; keys past the position invisible
    (2, 3, 64, 5000, 8, 700, 4, 17000),      # several rows per batch (positions pos + s)
    (3, 1, 20, 1000, 4, 300, 1, 999),        # fewer heads; slots beyond the cache
    (1, 1, 64, 16384, 8, 2048, 4, 65535),    # every block a candidate: the dense row itself
    (5, 1, 64, 777, 8, 1, 4, 2000),          # one candidate block per row
])
def test_candidate_scores_bit_identical_to_dense(dev, fmt, b, s, hi, g, bs, nb, ratio, pos):
    q, k, w = _inputs(b, s, hi, g, seed=g + nb)
    ops = _fp8(q, k) if fmt == "fp8" else _mxfp4(q, k)
    positions = pos + torch.arange(s, dtype=torch.int64).expand(b, s)
    cand = _random_lists(b, s, g, bs, nb, seed=g, extra_blocks=3)
    if nb * bs == (-(-g // bs)) * bs and nb == 2048:  # the full-coverage case
        cand = torch.arange(nb, dtype=torch.int32).expand(b, s, nb).contiguous()
    print(f"candidate scores {fmt}: B={b} S={s} Hi={hi} G={g} bs={bs} nb={nb} ratio={ratio} pos={pos}", flush=True)
    dense = _scores(fmt, ops, w, dev, ratio, positions).cpu()
    got = _scores(fmt, ops, w, dev, ratio, positions, cand=cand, bs=bs).cpu()
    want = _gather(dense, cand, bs, g)
    assert got.shape == (b, s, nb * bs)
    assert torch.equal(got, want)
    if nb * bs == g:
        assert torch.equal(got, dense)


@pytest.mark.parametrize("fmt,kind", [("fp8", "distinct"), ("fp8", "ties"), ("mxfp4", "distinct")])
def test_two_level_topk_matches_oracle(dev, fmt, kind):
    """Level one on a source layer's scores, level two on another layer's keys: the top-512
    key positions equal the oracle's top-k of the dense scores masked to the candidates."""
    b, g, ratio, bs, nblk, topk = 4, 65536, 4, 8, 2048, 512
    pos = torch.tensor([[262143], [262143], [100000], [40003]], dtype=torch.int64)
    lens = ((pos + 1) // ratio).clamp(max=g)
    # the source layer: plain fp32 logits with its visibility mask
    gen = torch.Generator().manual_seed(11)
    src = torch.randn(b, 1, g, generator=gen).masked_fill(torch.arange(g).view(1, 1, -1) >= lens.unsqueeze(-1), NEG)
    print(f"two-level: fmt={fmt} kind={kind} B={b} G={g}", flush=True)
    cand = MI.candidate_block_list(src.to(dev), lens.unsqueeze(-1).to(dev), nblk, bs)
    mask = OA.select_candidate_blocks(src.numpy(), lens.unsqueeze(-1).numpy(), nblk, bs)
    cl = cand.cpu()
    # the list: ascending blocks then -1, expanding to the oracle's mask
    expanded = np.zeros_like(mask)
    for r in range(b):
        blocks = cl[r, 0][cl[r, 0] >= 0].numpy()
        assert np.all(np.diff(blocks) > 0) and np.all(cl[r, 0, len(blocks):].numpy() == -1)
        for blk in blocks:
            expanded[r, 0, blk * bs:(blk + 1) * bs] = True
    assert np.array_equal(expanded[..., :g], mask)
    # the candidate-using layer
    q, k, w = _inputs(b, 1, 64, g, seed=5, ties=kind == "ties")
    ops = _fp8(q, k) if fmt == "fp8" else _mxfp4(q, k)
    dense = _scores(fmt, ops, w, dev, ratio, pos).cpu()
    cs = _scores(fmt, ops, w, dev, ratio, pos, cand=cl, bs=bs)
    got = MI.candidate_topk(cs, cand, bs, topk).cpu().numpy()
    want = OA.topk_indices(dense.masked_fill(~torch.from_numpy(mask), NEG), topk)
    assert np.array_equal(got, want)


def test_candidate_edge_cases(dev):
    """Empty lists: all -1 gives all -inf and an all -1 top-k; zero blocks gives an empty
    candidate axis; the position map works in place."""
    b, g = 2, 300
    q, k, w = _inputs(b, 1, 64, g, seed=1)
    ops = _fp8(q, k)
    pos = torch.full((b, 1), 4 * g, dtype=torch.int64)
    empty = torch.full((b, 1, 16), -1, dtype=torch.int32)
    sc = _scores("fp8", ops, w, dev, 4, pos, cand=empty)
    assert sc.shape == (b, 1, 128) and bool(torch.all(sc == NEG))
    idx = MI.candidate_topk(sc, empty.to(dev), 8, 32)
    assert bool(torch.all(idx == -1))
    none = torch.empty((b, 1, 0), dtype=torch.int32)
    sc0 = _scores("fp8", ops, w, dev, 4, pos, cand=none)
    assert sc0.shape == (b, 1, 0)
    slots = torch.tensor([[[0, 12, 17, 25, 200, -1]]], dtype=torch.int32).expand(b, 1, 6).contiguous().to(dev)
    blocks = torch.tensor([[[3, 9, 30, -1]]], dtype=torch.int32).expand(b, 1, 4).contiguous().to(dev)
    out = MI.candidate_positions(slots, blocks, 8, out=slots)
    assert out.data_ptr() == slots.data_ptr()
    assert out.cpu().tolist() == [[[24, 76, 241, -1, -1, -1]]] * b


@pytest.mark.parametrize("rows,nb,bs,k", [(3, 40, 8, 64), (4, 2048, 8, 2048), (2, 5000, 8, 2048), (5, 300, 4, 1000)])
def test_candidate_topk_one_launch_equals_two(dev, rows, nb, bs, k):
    """mzk_candidate_topk (one launch up to 32768 slots) equals mzk_topk_rows followed by
    mzk_candidate_positions, with ties, empty blocks and -inf slots; past 32768 slots the
    wrapper takes the two-step path (checked against the oracle's top-k mapped by hand)."""
    gen = torch.Generator().manual_seed(rows * 31 + nb)
    sc = torch.round(torch.randn(rows, nb * bs, generator=gen) * 8) / 8  # ties
    cand = torch.stack([torch.randperm(4 * nb, generator=gen)[:nb].sort().values for _ in range(rows)]).int()
    cand[:, -3:] = -1
    sc.view(rows, nb, bs)[:, -3:] = NEG  # empty blocks score -inf (as the scorer writes)
    sc[:, ::7] = NEG
    print(f"candidate top-k: rows={rows} nb={nb} bs={bs} k={k}", flush=True)
    got = MI.candidate_topk(sc.to(dev), cand.to(dev), bs, k).cpu().numpy()
    slots = OA.topk_indices(sc.numpy(), k)
    want = np.where(slots >= 0, cand.numpy()[np.arange(rows)[:, None], np.maximum(slots, 0) // bs] * bs + slots % bs, -1)
    assert np.array_equal(got, want)
    if nb * bs <= 32768:
        two = MI.candidate_positions(MI.topk(sc.to(dev), k), cand.to(dev), bs).cpu().numpy()
        assert np.array_equal(got, two)
