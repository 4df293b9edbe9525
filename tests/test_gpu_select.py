"""GPU: the decode step's top-k inside the attention launch (``mzk_sparse_mqa_select``).

Every attention workgroup of a row selects the row's sparse list from the indexer scores
itself.  Its list (written out by the row's first workgroup), output and lse must equal the
top-k launch followed by the attention over that list (``indexer.topk`` +
``sparse_mqa_decode``) bit for bit: scores with ties and ``-inf`` entries, rows with fewer
finite scores than topk and rows with none, the fused RoPE, a dense branch, one to sixteen
splits, the merge inside the attention launch, the position advance, graph replays, and the
form that falls back to the two launches (a key count that is not a multiple of 4, or more
than 8192 keys: config 4's 32768 among them).  The list also equals the oracle's top-k, and
the output meets the attention bar against the oracle.
"""

import numpy as np
import pytest
import torch

from mzoo_amd import csa2_attn as MA
from mzoo_amd import indexer as MI
from mzoo_amd import quant as MQ
from oracle import attention as OA
from tests.helpers import assert_attn_close
from tests.test_gpu_attention import _decode_oracle

pytestmark = pytest.mark.gpu
H, D = 128, 576


@pytest.fixture(autouse=True)
def _restore_merge_mode():
    yield
    MA.set_merge(0)


def _case(dev, b, g, pos, seed, kind="normal", dense=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, H, D, generator=gen).bfloat16()
    win_c = MQ.pack_latent_fp8_b128(torch.randn(b, 128, D, generator=gen).bfloat16().to(dev))
    main_c = MQ.pack_latent_fp8_b128(torch.randn(b, g, D, generator=gen).bfloat16().to(dev))
    dense_c = MQ.pack_latent_fp8_b128(torch.randn(b, dense, D, generator=gen).bfloat16().to(dev)) if dense else None
    sc = torch.randn(b, g, generator=gen)
    if kind == "ties":
        sc = torch.round(sc * 4) / 4
    vis = min(g, (pos + 1) // 4)
    sc[:, vis:] = float("-inf")                     # groups the row cannot see yet
    sc[0, 5:] = float("-inf")                       # a row with fewer finite scores than topk
    if b > 2:
        sc[2, :] = float("-inf")                    # and one with none
    sinks = torch.randn(H, generator=gen)
    return q, win_c, main_c, dense_c, sc, sinks


def _two_launches(qd, pos_d, win_c, main_c, dense_c, scd, topk, skd, nsplit, rope):
    b, g = scd.shape
    idx = MI.topk(scd, topk)
    o, lse = MA.sparse_mqa_decode(qd, pos_d, win_c, 128, main_cache=main_c, groups=g, indices=idx,
                                  dense_cache=dense_c, dense_ratio=16, sinks=skd, nsplit=nsplit, rope=rope)
    return o, lse, idx


def _rope(b, dev, seed):
    gen = torch.Generator().manual_seed(seed)
    ang = torch.rand(b, 32, generator=gen) * 6.28
    return torch.cos(ang).bfloat16().to(dev), torch.sin(ang).bfloat16().to(dev)


@pytest.mark.parametrize("b,g,topk,nsplit,kind,use_rope,dense", [
    (32, 8192, 2048, 4, "normal", True, 0), (8, 8192, 2048, 4, "ties", True, 0), (8, 8192, 2048, 1, "normal", True, 0),
    (8, 8192, 2048, 16, "ties", False, 0), (4, 4096, 512, 4, "normal", True, 256), (6, 1000, 128, 2, "ties", False, 0),
    (5, 8190, 2048, 4, "normal", True, 0), (8, 32768, 2048, 16, "normal", True, 0), (8, 32768, 2048, 16, "ties", True, 0),
    (4, 16384, 2048, 8, "normal", False, 0), (3, 20000, 512, 4, "ties", True, 128), (2, 40000, 2048, 8, "normal", True, 0)])
def test_select_equals_topk_then_attention(dev, b, g, topk, nsplit, kind, use_rope, dense):
    pos = 4 * g + 3 if kind != "ties" else 3 * g  # ties: a quarter of the groups still invisible
    q, win_c, main_c, dense_c, sc, sinks = _case(dev, b, g, pos, seed=b + g + nsplit, kind=kind, dense=dense)
    qd, scd, skd = q.to(dev), sc.to(dev), sinks.to(dev)
    pos_d = torch.full((b,), pos, dtype=torch.int64, device=dev)
    rope = _rope(b, dev, 7) if use_rope else None
    ref_o, ref_l, ref_i = _two_launches(qd, pos_d, win_c, main_c, dense_c, scd, topk, skd, nsplit, rope)
    o, lse, idx = MA.sparse_mqa_decode_select(qd, pos_d, win_c, 128, main_cache=main_c, scores=scd, topk=topk,
                                              dense_cache=dense_c, dense_ratio=16, sinks=skd, nsplit=nsplit,
                                              rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(idx, ref_i), "selected list"
    assert torch.equal(o, ref_o) and torch.equal(lse, ref_l), "attention output"
    want = OA.topk_indices(sc.numpy()[:, None], topk)[:, 0]
    assert np.array_equal(idx.cpu().numpy(), want)
    if not use_rope and not dense:
        ref, _ = _decode_oracle(q, win_c, main_c, None, torch.from_numpy(want), sinks, pos, 128, 1, g)
        assert_attn_close(o.cpu(), ref)


@pytest.mark.parametrize("merge,nsplit", [(1, 4), (1, 8), (0, 4)])
def test_select_with_inlaunch_merge_and_advance(dev, merge, nsplit):
    """With the split merge inside the launch and the positions advanced by the call."""
    b, g, topk, pos = 8, 8192, 2048, 40000
    q, win_c, main_c, _, sc, sinks = _case(dev, b, g, pos, seed=31 + nsplit)
    qd, scd, skd = q.to(dev), sc.to(dev), sinks.to(dev)
    rope = _rope(b, dev, 9)
    pos_d = torch.full((b,), pos, dtype=torch.int64, device=dev)
    ref_o, ref_l, ref_i = _two_launches(qd, pos_d, win_c, main_c, None, scd, topk, skd, nsplit, rope)
    MA.set_merge(merge)
    ws = MA.new_workspace(b, H, D, nsplit, dev)
    p = pos_d.clone()
    o, lse, idx = MA.sparse_mqa_decode_select(qd, p, win_c, 128, main_cache=main_c, scores=scd, topk=topk,
                                              sinks=skd, nsplit=nsplit, workspace=ws, rope=rope, advance=True)
    torch.cuda.synchronize()
    assert torch.equal(idx, ref_i) and torch.equal(o, ref_o) and torch.equal(lse, ref_l)
    assert torch.equal(p, pos_d + 1)
    if merge:
        assert MA.merge_status(ws, b, H, D, nsplit) == (0, b * 2)


def test_select_graph_replays(dev):
    """A graph of the selecting call replayed with new scores written between the replays:
    every replay equals the two launches on those scores."""
    b, g, topk, nsplit, pos = 16, 8192, 2048, 4, 33000
    q, win_c, main_c, _, sc, sinks = _case(dev, b, g, pos, seed=55)
    qd, skd = q.to(dev), sinks.to(dev)
    rope = _rope(b, dev, 11)
    pos_d = torch.full((b,), pos, dtype=torch.int64, device=dev)
    scd = sc.to(dev)
    ws = MA.new_workspace(b, H, D, nsplit, dev)
    out = torch.empty(b, H, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(b, H, dtype=torch.float32, device=dev)
    idx = torch.empty(b, topk, dtype=torch.int32, device=dev)

    def run():
        MA.sparse_mqa_decode_select(qd, pos_d, win_c, 128, main_cache=main_c, scores=scd, topk=topk, idx_out=idx,
                                    sinks=skd, nsplit=nsplit, workspace=ws, out=out, lse=lse, rope=rope)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        gen = torch.Generator().manual_seed(100 + rep)
        new = torch.randn(b, g, generator=gen)
        new[:, (pos + 1) // 4:] = float("-inf")
        scd.copy_(new.to(dev))
        graph.replay()
        torch.cuda.synchronize()
        ref_o, ref_l, ref_i = _two_launches(qd, pos_d, win_c, main_c, None, scd, topk, skd, nsplit, rope)
        torch.cuda.synchronize()
        assert torch.equal(idx, ref_i) and torch.equal(out, ref_o) and torch.equal(lse, ref_l), f"replay {rep}"
