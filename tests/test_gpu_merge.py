"""GPU: the split merge inside the attention launch (``mzk_sparse_mqa_set_merge(1)``).

With nsplit > 1 the attention launch of the FP8 latent decode can merge its own splits: the
workgroups of one (row, 64-head group) run on one XCD, wait for each other and each merge
64 / nsplit of the heads with the merge kernel's arithmetic.  Its output and lse must equal
the separate merge kernel's bit for bit (``mzk_sparse_mqa_set_merge(0)``), with the
cross-XCD release / acquire path forced as well (mode 2), call after call on one workspace
(each call leaves its records zeroed for the next), inside a replayed HIP graph, with the
fused RoPE, for both workgroup mappings (rows a multiple of 8: a row's workgroups on one
XCD; 4 rows: each (row, head group) on its own XCD), and against the CPU oracle.  The
status words confirm the merge ran inside the launch and no split gave up waiting.
"""

import pytest
import torch

from mzoo_amd import csa2_attn as MA
from tests.helpers import assert_attn_close
from tests.test_gpu_attention import LSE_TOL, _decode_case, _decode_oracle

pytestmark = pytest.mark.gpu
H, D = 128, 576


@pytest.fixture(autouse=True)
def _restore_merge_mode():
    yield
    MA.set_merge(0)


def _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, ws, rope=None):
    return MA.sparse_mqa_decode(qd, positions, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk,
                                nsplit=nsplit, workspace=ws, rope=rope)


@pytest.mark.parametrize("b,nsplit", [(8, 2), (8, 4), (8, 8), (8, 16), (4, 4), (4, 32)])
def test_inlaunch_merge_equals_merge_kernel(dev, b, nsplit):
    pos, gcap, topk = 8191, 2048, 512
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, gcap, topk, pos, seed=40 + nsplit + b)
    qd, idxd, sk = q.to(dev), idx.to(dev), sinks.to(dev)
    positions = torch.full((b,), pos, dtype=torch.int64, device=dev)
    MA.set_merge(0)
    ref_o, ref_l = _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, MA.new_workspace(b, H, D, nsplit, dev))
    groups = b * (H // 64)
    for mode in (1, 2):
        MA.set_merge(mode)
        ws = MA.new_workspace(b, H, D, nsplit, dev)
        for call in range(3):
            o, lse = _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, ws)
            torch.cuda.synchronize()
            assert torch.equal(o, ref_o) and torch.equal(lse, ref_l), f"mode {mode}, call {call}"
            err, merged = MA.merge_status(ws, b, H, D, nsplit)
            assert err == 0 and merged == groups * (call + 1), (mode, call, err, merged)
        # the records are zero again after every complete call
        recs = ws.view(torch.uint8)[MA.workspace_bytes(b, H, D, nsplit) - 16 - 16 * groups:][:16 * groups]
        assert not recs.any()
    ref, ref_lse = _decode_oracle(q, win_c, main_c, None, idx, sinks, pos, 128, 1, g)
    assert_attn_close(ref_o.cpu(), ref)
    torch.testing.assert_close(ref_l.cpu(), ref_lse, **LSE_TOL)


def test_inlaunch_merge_with_rope(dev):
    """The fused RoPE form: the inverse rotation of the merged output happens in the
    in-launch merge as in the merge kernel."""
    b, nsplit, pos, gcap, topk = 8, 4, 4095, 1024, 256
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, gcap, topk, pos, seed=77)
    qd, idxd, sk = q.to(dev), idx.to(dev), sinks.to(dev)
    positions = torch.full((b,), pos, dtype=torch.int64, device=dev)
    gen = torch.Generator().manual_seed(5)
    ang = torch.rand(b, 32, generator=gen) * 6.28
    rope = (torch.cos(ang).bfloat16().to(dev), torch.sin(ang).bfloat16().to(dev))
    MA.set_merge(0)
    ref = _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, MA.new_workspace(b, H, D, nsplit, dev), rope)
    MA.set_merge(1)
    ws = MA.new_workspace(b, H, D, nsplit, dev)
    got = _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, ws, rope)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    assert MA.merge_status(ws, b, H, D, nsplit) == (0, b * 2)


def test_inlaunch_merge_graph_replays(dev):
    """A graph holding two merged attention calls on two workspaces, replayed with eager
    work in between: every replay equals the eager result, and each replay counts its
    merges."""
    b, nsplit, pos, gcap, topk = 8, 4, 8191, 2048, 512
    cases = [_decode_case(dev, b, H, gcap, topk, pos, seed=90 + i) for i in range(2)]
    positions = torch.full((b,), pos, dtype=torch.int64, device=dev)
    MA.set_merge(1)
    dev_cases = []
    for q, win_c, main_c, _, idx, sinks, g in cases:
        dev_cases.append((q.to(dev), win_c, main_c, g, idx.to(dev), sinks.to(dev),
                          MA.new_workspace(b, H, D, nsplit, dev), torch.empty(b, H, D, dtype=torch.bfloat16, device=dev),
                          torch.empty(b, H, dtype=torch.float32, device=dev)))

    def run():
        for qd, win_c, main_c, g, idxd, sk, ws, out, lse in dev_cases:
            MA.sparse_mqa_decode(qd, positions, win_c, 128, main_cache=main_c, groups=g, indices=idxd, sinks=sk,
                                 nsplit=nsplit, workspace=ws, out=out, lse=lse)

    run()
    torch.cuda.synchronize()
    eager = [(c[7].clone(), c[8].clone()) for c in dev_cases]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for c in dev_cases:
            c[7].zero_()
            c[8].zero_()
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1024, device=dev).sum().item()  # eager work between replays
        for c, (eo, el) in zip(dev_cases, eager):
            assert torch.equal(c[7], eo) and torch.equal(c[8], el), f"replay {rep}"
    for c in dev_cases:
        err, merged = MA.merge_status(c[6], b, H, D, nsplit)
        assert err == 0 and merged == b * 2 * (1 + 1 + 4), merged  # eager, warm-up, 4 replays


def test_merge_falls_back_without_records(dev):
    """A workspace holding only the split partials (the size before the merge records)
    takes the merge kernel: same result, nothing counted."""
    b, nsplit, pos, gcap, topk = 8, 4, 8191, 2048, 512
    q, win_c, main_c, _, idx, sinks, g = _decode_case(dev, b, H, gcap, topk, pos, seed=3)
    qd, idxd, sk = q.to(dev), idx.to(dev), sinks.to(dev)
    positions = torch.full((b,), pos, dtype=torch.int64, device=dev)
    MA.set_merge(1)
    ws = MA.new_workspace(b, H, D, nsplit, dev)
    ref = _call(qd, positions, win_c, main_c, g, idxd, sk, nsplit, ws)
    small = torch.zeros(b * nsplit * H * (2 * D + 8) // 4, dtype=torch.float32, device=dev)
    from mzoo_amd import _lib
    o = torch.empty_like(qd)
    lse = torch.empty(b, H, dtype=torch.float32, device=dev)
    _lib.call("mzk_sparse_mqa", qd.data_ptr(), b, 1, H, D, 1, 512, positions.data_ptr(), win_c.data_ptr(), 128, 128,
              128, None, 0, 0, 1, main_c.data_ptr(), gcap, g, idxd.data_ptr(), topk, topk, sk.data_ptr(), nsplit,
              small.data_ptr(), small.numel() * 4, o.data_ptr(), lse.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(o, ref[0]) and torch.equal(lse, ref[1])
