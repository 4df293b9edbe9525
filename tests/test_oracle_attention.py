"""Pins the CPU oracle's attention / indexer / top-k restatement (oracle/attention.py).

Each check is chosen so a plausible slip in the restatement (a dropped sink, the wrong
window edge, a transposed operand, a missing ``Di^-0.5`` or ReLU, a wrong tie rule) fails:

* closed forms the reference's own tests use: window 1 returns the token's own value
  (``golden_ref_test.py:69-79``); ratio 1 with the main stream a copy of the raw stream
  doubles every visible key, so the output is the latent one and lse grows by ln 2
  (``:82-106``); sparse with every visible index selected equals the compressed level
  (``:109-129``); the ``topk_indices`` dummy-slot vector (``:147-157``, tests/golden/kat.json);
* the library routine the reference compares against (``torch`` SDPA, ``:35-44``);
* a sink of ``-inf`` is no sink, and a very large sink takes all the mass;
* the log-sum-exp merge identity over a split of the entry list (what split-KV relies on);
* brute force in float64 on tiny inputs for the indexer scores and the top-k order.
"""

import json
import math
import pathlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as OA

KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "kat.json").read_text())


def _rand(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def test_latent_matches_sdpa():
    q, kv = _rand(2, 9, 3, 16, seed=1), _rand(2, 9, 1, 16, seed=2)
    o, lse = OA.golden(q, kv, level="latent")
    k = kv.transpose(1, 2).expand(2, 3, 9, 16)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2).double(), k.double(), k.double(), is_causal=True)
    torch.testing.assert_close(o.double(), ref.transpose(1, 2), rtol=1e-5, atol=1e-5)
    logits = (q.transpose(1, 2).double() @ k.double().transpose(-1, -2)) / 4.0
    logits = logits.masked_fill(torch.ones(9, 9, dtype=torch.bool).triu(1), float("-inf"))
    torch.testing.assert_close(lse.double(), torch.logsumexp(logits, -1), rtol=1e-5, atol=1e-5)


def test_window_one_returns_own_value():
    q, kv = _rand(1, 7, 2, 8, seed=3), _rand(1, 7, 1, 8, seed=4)
    o, lse = OA.golden(q, kv, level="window", window=1)
    torch.testing.assert_close(o, kv.expand(1, 7, 2, 8), rtol=0, atol=1e-6)
    own = (q * kv).sum(-1).transpose(1, 2) * 8 ** -0.5
    torch.testing.assert_close(lse, own, rtol=1e-6, atol=1e-6)


def test_window_edge_includes_self():
    # token t sees t-W+1 .. t: with W=2 the output is a 2-way softmax over (t-1, t)
    q, kv = _rand(1, 5, 1, 4, seed=5), _rand(1, 5, 1, 4, seed=6)
    o, _ = OA.golden(q, kv, level="window", window=2)
    t = 3
    s = [(q[0, t, 0] @ kv[0, j, 0]).item() / 2.0 for j in (t - 1, t)]
    p = np.exp(np.array(s) - max(s))
    p /= p.sum()
    want = p[0] * kv[0, t - 1, 0] + p[1] * kv[0, t, 0]
    torch.testing.assert_close(o[0, t, 0], want, rtol=1e-5, atol=1e-6)


def test_ratio_one_duplicate_stream():
    q, kv = _rand(1, 6, 2, 8, seed=7), _rand(1, 6, 1, 8, seed=8)
    o_lat, lse_lat = OA.golden(q, kv, level="latent")
    o, lse = OA.golden(q, kv, level="compressed", window=6, main_kv=kv, compress_ratio=1)
    torch.testing.assert_close(o, o_lat, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lse, lse_lat + math.log(2.0), rtol=1e-5, atol=1e-5)


def test_sparse_all_visible_equals_compressed():
    b, s, h, d, g, r = 2, 12, 2, 8, 3, 4
    q, kv, main = _rand(b, s, h, d, seed=9), _rand(b, s, 1, d, seed=10), _rand(b, g, 1, d, seed=11)
    sinks = _rand(h, seed=12)
    idx = torch.full((b, s, g), -1, dtype=torch.int64)
    for t in range(s):
        n = (t + 1) // r
        idx[:, t, :n] = torch.arange(n)
    o_c, l_c = OA.golden(q, kv, level="compressed", window=3, main_kv=main, compress_ratio=r, sinks=sinks)
    o_s, l_s = OA.golden(q, kv, level="sparse", window=3, main_kv=main, compress_ratio=r, sinks=sinks, indices=idx)
    torch.testing.assert_close(o_s, o_c, rtol=0, atol=0)
    torch.testing.assert_close(l_s, l_c, rtol=0, atol=0)


def test_sink_neg_inf_is_no_sink_and_large_sink_takes_mass():
    q, kv = _rand(1, 5, 3, 8, seed=13), _rand(1, 5, 1, 8, seed=14)
    o0, l0 = OA.golden(q, kv, level="latent")
    o1, l1 = OA.golden(q, kv, level="latent", sinks=torch.full((3,), float("-inf")))
    torch.testing.assert_close(o1, o0, rtol=0, atol=0)
    torch.testing.assert_close(l1, l0, rtol=0, atol=0)
    o2, l2 = OA.golden(q, kv, level="latent", sinks=torch.full((3,), 80.0))
    assert o2.abs().max() < 1e-20
    torch.testing.assert_close(l2, torch.full_like(l2, 80.0), rtol=1e-6, atol=1e-6)
    # sink in the denominator only: o(sink) = o(no sink) * (1 - p_sink)
    sk = torch.tensor([0.3, -1.0, 2.0])
    o3, l3 = OA.golden(q, kv, level="latent", sinks=sk)
    p_sink = torch.exp(sk.view(1, 3, 1) - l3).transpose(1, 2).unsqueeze(-1)
    torch.testing.assert_close(o3, o0 * (1 - p_sink), rtol=1e-5, atol=1e-6)


def test_attend_entries_matches_golden_sparse_row():
    b, s, h, d, g, r, w = 1, 16, 4, 8, 4, 4, 3
    q, kv, main = _rand(b, s, h, d, seed=15), _rand(b, s, 1, d, seed=16), _rand(b, g, 1, d, seed=17)
    sinks = _rand(h, seed=18)
    idx = torch.tensor([[[2, 0, -1]] * s])
    o, lse = OA.golden(q, kv, level="sparse", window=w, main_kv=main, sinks=sinks, indices=idx)
    t = 11
    ents = torch.cat([kv[0, t - w + 1:t + 1, 0], main[0, [0, 2], 0]])
    o_r, l_r = OA.attend_entries(q[0, t], ents, sinks)
    torch.testing.assert_close(o_r, o[0, t], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(l_r, lse[0, :, t], rtol=1e-5, atol=1e-6)


def test_lse_merge_identity():
    q, ents, sinks = _rand(4, 16, seed=19), _rand(40, 16, seed=20), _rand(4, seed=21)
    o, lse = OA.attend_entries(q, ents, sinks)
    oa, la = OA.attend_entries(q, ents[:17])
    ob, lb = OA.attend_entries(q, ents[17:])
    big = torch.logsumexp(torch.stack([la, lb, sinks]), 0)
    merged = (oa * torch.exp(la - big).unsqueeze(-1) + ob * torch.exp(lb - big).unsqueeze(-1))
    torch.testing.assert_close(merged, o, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(big, lse, rtol=1e-6, atol=1e-6)


def test_indexer_scores_brute_force():
    b, s, hi, di, g, r = 2, 5, 3, 8, 6, 2
    q, k, w = _rand(b, s, hi, di, seed=22), _rand(b, g, di, seed=23), _rand(b, s, hi, seed=24)
    pos = torch.tensor([[0, 3, 5, 9, 11], [1, 2, 4, 7, 12]])
    got = OA.indexer_scores(q, k, w, r, positions=pos).numpy()
    qn, kn, wn = q.double().numpy(), k.double().numpy(), w.double().numpy()
    for bi in range(b):
        for si in range(s):
            for gi in range(g):
                if gi >= (int(pos[bi, si]) + 1) // r:
                    assert got[bi, si, gi] == -np.inf
                    continue
                want = sum(wn[bi, si, h] * max(0.0, float(qn[bi, si, h] @ kn[bi, gi])) for h in range(hi)) / math.sqrt(di)
                assert abs(got[bi, si, gi] - want) <= 1e-5 * (1 + abs(want))


def test_indexer_prefill_default_positions():
    q, k, w = _rand(1, 8, 2, 4, seed=25), _rand(1, 2, 4, seed=26), _rand(1, 8, 2, seed=27).abs()
    sc = OA.indexer_scores(q, k, w, 4)
    vis = torch.isfinite(sc)
    for t in range(8):
        assert vis[0, t].tolist() == [j < (t + 1) // 4 for j in range(2)]
    assert (sc[vis] >= 0).all()  # relu with non-negative weights


def test_topk_kat_dummy_slot():
    kat = KAT["topk_dummy_slot"]
    sc = np.array([[[float(x) for x in row] for row in kat["scores"][0]]], np.float32)
    out = OA.topk_indices(sc, kat["topk"])
    assert sorted(out[0, 0, :len(kat["first_set"])].tolist()) == kat["first_set"]
    assert out[0, 0, len(kat["first_set"]):].tolist() == kat["tail"]
    out2 = OA.topk_indices(sc[..., :kat["padded_scores_cols"]], kat["padded_topk"])
    assert out2[0, 0, 2:].tolist() == kat["padded_tail"]


@pytest.mark.parametrize("seed", range(6))
def test_topk_brute_force_with_ties(seed):
    rng = np.random.default_rng(seed)
    g = int(rng.integers(1, 40))
    sc = rng.integers(-3, 4, size=(3, g)).astype(np.float32)  # many ties
    sc[rng.random((3, g)) < 0.2] = -np.inf
    k = int(rng.integers(1, 50))
    out = OA.topk_indices(sc, k)
    for r in range(3):
        ranked = sorted(range(g), key=lambda i: (-float(sc[r, i]), i))[:min(k, g)]
        keep = sorted(i for i in ranked if sc[r, i] > -np.inf)
        assert out[r].tolist() == keep + [-1] * (k - len(keep))


def test_topk_empty():
    assert OA.topk_indices(np.zeros((2, 0), np.float32), 3).tolist() == [[-1] * 3] * 2


# ---- select_candidate_blocks (owlet1/indexer.py:14-40) ------------------------------------

def _torch_candidate_blocks(logits, compress_lens, topk_blocks, block_size):
    """The reference's steps in torch ops (pad/amax/masked_fill/topk/scatter), valid where
    no two block scores tie at the selection boundary."""
    import torch.nn.functional as F
    width = logits.size(-1)
    sc = F.pad(logits, (0, -width % block_size), value=float("-inf"))
    sc = sc.unflatten(-1, (-1, block_size)).amax(dim=-1)
    nb = sc.size(-1)
    last = (compress_lens - 1) // block_size
    sc = sc.masked_fill(torch.arange(nb).view(-1) == last, torch.inf)
    top = sc.topk(min(topk_blocks, nb), dim=-1)
    keep = torch.zeros_like(sc, dtype=torch.bool).scatter_(-1, top.indices, top.values > float("-inf"))
    return keep.repeat_interleave(block_size, dim=-1)[..., :width]


@pytest.mark.parametrize("b,s,t,bs,k", [(2, 3, 13, 8, 1), (1, 4, 64, 8, 3), (2, 2, 1000, 8, 20), (1, 3, 37, 4, 50)])
def test_candidate_blocks_match_torch_formulation(b, s, t, bs, k):
    gen = torch.Generator().manual_seed(b * 100 + t)
    logits = torch.randn(b, s, t, generator=gen)          # distinct block maxima: no ties
    pos = torch.randint(0, 4 * t, (b, s), generator=gen)
    lens = ((pos + 1) // 4).clamp(max=t).unsqueeze(-1)
    logits = logits.masked_fill(torch.arange(t).view(1, 1, -1) >= lens, float("-inf"))
    want = _torch_candidate_blocks(logits, lens, k, bs).numpy()
    got = OA.select_candidate_blocks(logits.numpy(), lens.numpy(), k, bs)
    assert np.array_equal(got, want)


def test_candidate_blocks_ticket_cases():
    """tickets/0009-indexer-hierarchical.md acceptance cases: T not a multiple of 8, fewer
    reachable blocks than topk_blocks (only reachable ones kept), the newest (partial)
    block pinned even when it scores lowest, and when it also scores highest."""
    ninf = float("-inf")
    # T = 13, block 8: two blocks; newest position 12 is in block 1, which scores lowest
    x = np.array([[5.0] * 8 + [1.0] * 5], np.float32)
    got = OA.select_candidate_blocks(x, np.array([[13]]), 1, 8)
    assert got.tolist() == [[False] * 8 + [True] * 5]      # the pinned partial block wins
    # fewer reachable blocks than topk_blocks: unreachable (-inf) blocks are never kept
    x = np.array([[3.0, 1.0, ninf, ninf, ninf, ninf]], np.float32)
    got = OA.select_candidate_blocks(x, np.array([[2]]), 3, 2)
    assert got.tolist() == [[True, True, False, False, False, False]]
    # newest block also the highest: kept once, the next best fills the other slot
    x = np.array([[1.0, 2.0, 9.0, 3.0, 4.0, 8.0]], np.float32)
    got = OA.select_candidate_blocks(x, np.array([[6]]), 2, 2)
    assert got.tolist() == [[False, False, True, True, True, True]]
    # nothing visible yet (length 0): nothing is pinned and every block is -inf
    x = np.full((1, 5), ninf, np.float32)
    assert not OA.select_candidate_blocks(x, np.array([[0]]), 4, 2).any()


def test_candidate_blocks_invariants():
    gen = np.random.default_rng(7)
    for _ in range(20):
        t, bs = int(gen.integers(1, 200)), int(gen.integers(1, 9))
        k = int(gen.integers(1, 12))
        x = np.round(gen.standard_normal((3, t)) * 4).astype(np.float32)    # ties
        lens = gen.integers(0, t + 1, (3, 1))
        x = np.where(np.arange(t) < lens, x, -np.inf).astype(np.float32)
        m = OA.select_candidate_blocks(x, lens, k, bs)
        nb = -(-t // bs)
        for r in range(3):
            kept = {p // bs for p in range(t) if m[r, p]}
            # a block is kept whole or not at all
            assert all(m[r, p] == ((p // bs) in kept) for p in range(t))
            reachable = {j for j in range(nb) if np.isfinite(x[r, j * bs:(j + 1) * bs]).any()}
            if lens[r, 0] > 0:
                last = (lens[r, 0] - 1) // bs
                assert last in kept
                reachable.add(last)
            assert kept <= reachable and len(kept) == min(k, nb, len(reachable))
