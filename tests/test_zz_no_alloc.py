"""GPU: the allocation-free attention entry point (``mzk_sparse_mqa_noalloc``) against the
workspace form it varies (``mzk_sparse_mqa_rope``), through the C ABI.

The two run the same kernels on the same inputs, so their outputs and lse must be equal bit
for bit (and both meet the attention bar against the oracle).  Two calls in a row, the
second with fewer rows and splits than the first, check that the device scratch array keeps
no state a later call depends on; a request above the scratch size is an argument error
raised before any launch.
"""

import pytest
import torch

from mzoo_amd import _lib
from mzoo_amd import csa2_attn as MA
from mzoo_amd import quant as MQ
from oracle import attention as OA
from oracle import quant as Q
from tests.helpers import assert_attn_close

pytestmark = pytest.mark.gpu

D, NOPE = 576, 512


def _case(dev, b, h, gcap, topk, pos, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, D, generator=gen).bfloat16().to(dev)
    win = MQ.pack_latent_fp8_b128(torch.randn(b, 128, D, generator=gen).bfloat16().to(dev))
    main = MQ.pack_latent_fp8_b128(torch.randn(b, gcap, D, generator=gen).bfloat16().to(dev))
    g = min((pos + 1) // 4, gcap)
    idx = torch.stack([torch.randperm(g, generator=gen)[:topk] for _ in range(b)]).int().to(dev)
    sinks = torch.randn(h, generator=gen).to(dev)
    ang = torch.rand(b, 32, generator=gen) * 6.28
    cos, sin = ang.cos().bfloat16().to(dev), ang.sin().bfloat16().to(dev)
    positions = torch.full((b,), pos, dtype=torch.int64, device=dev)
    return q, win, main, g, idx, sinks, cos, sin, positions


def _args(q, win, main, g, idx, sinks, positions, nsplit):
    b, h, _ = q.shape
    topk = idx.shape[1]
    return (q.data_ptr(), b, 1, h, D, 1, NOPE, positions.data_ptr(), win.data_ptr(), win.shape[1], win.shape[1], 128,
            None, 0, 0, 1, main.data_ptr(), main.shape[1], g, idx.data_ptr(), topk, topk, sinks.data_ptr(), nsplit)


def _run_both(dev, b, h, gcap, topk, pos, nsplit, seed, rope):
    q, win, main, g, idx, sinks, cos, sin, positions = _case(dev, b, h, gcap, topk, pos, seed)
    st = torch.cuda.current_stream().cuda_stream
    rope_args = (cos.data_ptr(), sin.data_ptr(), 64) if rope else (None, None, 0)
    out_w = torch.empty(b, h, D, dtype=torch.bfloat16, device=dev)
    lse_w = torch.empty(b, h, dtype=torch.float32, device=dev)
    ws = MA.new_workspace(b, h, D, nsplit, dev)
    args = _args(q, win, main, g, idx, sinks, positions, nsplit)
    if rope:
        _lib.call("mzk_sparse_mqa_rope", *args, ws.data_ptr(), ws.numel() * ws.element_size(), out_w.data_ptr(),
                  lse_w.data_ptr(), *rope_args, st)
    else:
        _lib.call("mzk_sparse_mqa", *args, ws.data_ptr(), ws.numel() * ws.element_size(), out_w.data_ptr(),
                  lse_w.data_ptr(), st)
    out_n = torch.full((b, h, D), float("nan"), dtype=torch.bfloat16, device=dev)
    lse_n = torch.full((b, h), float("nan"), dtype=torch.float32, device=dev)
    _lib.call("mzk_sparse_mqa_noalloc", *args, out_n.data_ptr(), lse_n.data_ptr(), *rope_args, st)
    torch.cuda.synchronize()
    assert torch.equal(out_n, out_w), f"output differs from the workspace form (B={b}, nsplit={nsplit})"
    assert torch.equal(lse_n, lse_w), f"lse differs from the workspace form (B={b}, nsplit={nsplit})"
    if not rope:
        winf = torch.from_numpy(Q.unpack_latent_fp8_b128(win.cpu().numpy()))
        mainf = torch.from_numpy(Q.unpack_latent_fp8_b128(main.cpu().numpy()))
        for r in range(min(b, 3)):
            toks = [(pos - 127 + i) % 128 for i in range(128)]
            ents = torch.cat([winf[r, toks], mainf[r, idx[r].long().cpu()]])
            ref, _ = OA.attend_entries(q[r].float().cpu(), ents, sinks.cpu())
            assert_attn_close(out_n[r], ref, name=f"noalloc row {r}")
    return out_n


@pytest.mark.parametrize("rope", [False, True])
def test_noalloc_matches_workspace_form_twice(dev, rope):
    print(f"noalloc: rope={rope} call 1 (B=32, nsplit=4)", flush=True)
    _run_both(dev, 32, 128, 1024, 512, 4095, 4, 21, rope)
    print(f"noalloc: rope={rope} call 2 (B=3, nsplit=2)", flush=True)
    _run_both(dev, 3, 128, 512, 256, 2047, 2, 22, rope)


def test_noalloc_single_split_and_limit(dev):
    """One split writes the output directly (no scratch use); a request above the scratch
    size fails in the argument check, before any launch."""
    _run_both(dev, 2, 64, 256, 64, 1023, 1, 23, False)
    q, win, main, g, idx, sinks, cos, sin, positions = _case(dev, 2, 128, 256, 64, 1023, 24)
    st = torch.cuda.current_stream().cuda_stream
    out = torch.empty(2, 128, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(2, 128, dtype=torch.float32, device=dev)
    big_rows = (32 << 20) // (8 * 128 * (2 * D + 8)) + 1     # rows x 8 splits above 32 MiB
    args = list(_args(q, win, main, g, idx, sinks, positions, 8))
    args[1] = big_rows                                        # B: never launched (argument error)
    with pytest.raises(_lib.MzkError, match="scratch"):
        _lib.call("mzk_sparse_mqa_noalloc", *args, out.data_ptr(), lse.data_ptr(), None, None, 0, st)
