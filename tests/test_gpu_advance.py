"""GPU: the decode step's position advance inside the attention call (``mzk_sparse_mqa_advance``).

``sparse_mqa_decode(..., advance=True)`` must give the output and lse of the same call
without it, bit for bit, and leave every row's position one higher: in the split merge's
launch (nsplit > 1), in a launch of its own after the attention (nsplit 1, or the merge
inside the attention launch), with and without the fused RoPE.  A replayed graph holding the
advancing call decodes consecutive positions: after replay r the output equals an eager call
at the start position + r, and the positions have moved by the number of replays.  (The
decode layer advances through this call: its replayed steps are checked position by position
against the oracle in test_gpu_decode_emit.py.)
"""

import pytest
import torch

from mzoo_amd import _lib
from mzoo_amd import csa2_attn as MA
from tests.helpers import assert_attn_close
from tests.test_gpu_attention import _decode_case, _decode_oracle

pytestmark = pytest.mark.gpu
H, D = 128, 576


@pytest.fixture(autouse=True)
def _restore_merge_mode():
    yield
    MA.set_merge(0)


def _rope(b, seed):
    gen = torch.Generator().manual_seed(seed)
    ang = torch.rand(b, 32, generator=gen) * 6.28
    return torch.cos(ang).bfloat16(), torch.sin(ang).bfloat16()


@pytest.mark.parametrize("nsplit,merge,use_rope", [(4, 0, True), (4, 0, False), (1, 0, True), (8, 1, True),
                                                   (16, 0, False)])
def test_advance_equals_plain_call(dev, nsplit, merge, use_rope):
    b, pos, gcap, topk = 8, 8191, 2048, 512
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, gcap, topk, pos, seed=11 + nsplit)
    qd, idxd, sk = q.to(dev), idx.to(dev), sinks.to(dev)
    rope = tuple(t.to(dev) for t in _rope(b, 3)) if use_rope else None
    base = torch.arange(b, dtype=torch.int64, device=dev) + pos - b  # rows at different positions
    MA.set_merge(merge)

    def call(positions, advance):
        ws = MA.new_workspace(b, H, D, nsplit, dev)
        return MA.sparse_mqa_decode(qd, positions, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk,
                                    nsplit=nsplit, workspace=ws, rope=rope, advance=advance)

    ref_o, ref_l = call(base.clone(), False)
    p = base.clone()
    o, lse = call(p, True)
    torch.cuda.synchronize()
    assert torch.equal(o, ref_o) and torch.equal(lse, ref_l)
    assert torch.equal(p, base + 1)
    if merge:  # the merge ran inside the attention launch, so the advance had a launch of its own
        ws = MA.new_workspace(b, H, D, nsplit, dev)
        MA.sparse_mqa_decode(qd, p, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk, nsplit=nsplit,
                             workspace=ws, rope=rope, advance=True)
        torch.cuda.synchronize()
        assert MA.merge_status(ws, b, H, D, nsplit) == (0, b * 2)
        assert torch.equal(p, base + 2)


def test_advance_in_graph_replays(dev):
    """Each replay decodes the next position: output equal to an eager call there."""
    b, nsplit, pos0, gcap, topk = 8, 4, 4000, 1024, 256
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, gcap, topk, pos0 + 3, seed=21)
    qd, idxd, sk = q.to(dev), idx.to(dev), sinks.to(dev)
    rope = tuple(t.to(dev) for t in _rope(b, 4))
    ws = MA.new_workspace(b, H, D, nsplit, dev)
    out = torch.empty(b, H, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(b, H, dtype=torch.float32, device=dev)
    p = torch.full((b,), pos0, dtype=torch.int64, device=dev)

    def run():
        MA.sparse_mqa_decode(qd, p, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk, nsplit=nsplit,
                             workspace=ws, out=out, lse=lse, rope=rope, advance=True)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()
    p.fill_(pos0)
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        at = torch.full((b,), pos0 + r, dtype=torch.int64, device=dev)
        want = MA.sparse_mqa_decode(qd, at, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk,
                                    nsplit=nsplit, rope=rope)
        torch.cuda.synchronize()
        assert torch.equal(out, want[0]) and torch.equal(lse, want[1]), f"replay {r}"
        assert int(p.min()) == int(p.max()) == pos0 + r + 1
    # and the eager result at the last position meets the oracle's bar (no RoPE form)
    o, _ = MA.sparse_mqa_decode(qd, torch.full((b,), pos0 + 3, dtype=torch.int64, device=dev), win_c, 128,
                                main_cache=main_c, groups=g, indices=idxd, sinks=sk, nsplit=nsplit)
    ref, _ = _decode_oracle(q, win_c, main_c, None, idx, sinks, pos0 + 3, 128, 1, g)
    assert_attn_close(o.cpu(), ref)


def test_advance_refuses_prefill_rows(dev):
    b = 2
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, 256, 64, 1000, seed=5)
    qd = q.to(dev)
    p = torch.full((b,), 1000, dtype=torch.int64, device=dev)
    o = torch.empty_like(qd)
    lse = torch.empty(b, H, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="one query per row"):
        _lib.call("mzk_sparse_mqa_advance", qd.data_ptr(), 1, b, H, D, 1, 512, p.data_ptr(), win_c.data_ptr(), 128,
                  128, 128, None, 0, 0, 1, None, 0, 0, None, 0, 0, None, 1, None, 0, o.data_ptr(), lse.data_ptr(),
                  None, None, 0, torch.cuda.current_stream().cuda_stream)
    assert int(p.min()) == 1000
