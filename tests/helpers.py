"""Shared test helpers: tolerances stated once, comparisons that report what differs."""

from __future__ import annotations

import numpy as np
import torch

# Indexer scores: fp32 accumulation, relative to the magnitude the sum is built from
# (sum_h |w_h| relu(q.k) Di^-0.5); the -inf mask must match exactly.
SCORE_RTOL = 1e-5
# Attention outputs (bf16): cosine and max-abs bars.
ATTN_COS_MIN = 0.9999
ATTN_MAXABS = 2e-2


def assert_scores_close(got: torch.Tensor, ref: torch.Tensor, absref: torch.Tensor, rtol: float = SCORE_RTOL):
    got = got.detach().float().cpu()
    ref = ref.float().cpu()
    absref = absref.float().cpu()
    gi, ri = torch.isinf(got), torch.isinf(ref)
    assert torch.equal(gi, ri), f"-inf mask differs at {int((gi != ri).sum())} entries"
    assert torch.equal(got[gi], ref[ri]), "masked entries must be -inf"
    fin = ~ri
    err = (got[fin] - ref[fin]).abs()
    bound = rtol * absref[fin] + 1e-12
    bad = err > bound
    assert not bad.any(), (f"{int(bad.sum())} scores out of tolerance; worst err {err.max():.3e}, "
                           f"rel {(err / absref[fin].clamp_min(1e-30)).max():.3e}")


def assert_topk_sets_match(got_idx, ref_scores, absref, k: int, rtol: float = SCORE_RTOL):
    """Per row: the index set must equal the oracle's top-k of the oracle scores, except
    for entries whose score is within tolerance of the k-th score (a near-tie the kernel
    may break the other way)."""
    got = np.asarray(got_idx.cpu() if torch.is_tensor(got_idx) else got_idx).reshape(-1, k)
    sc = ref_scores.float().cpu().numpy().reshape(got.shape[0], -1)
    ab = absref.float().cpu().numpy().reshape(got.shape[0], -1)
    from oracle.attention import topk_indices
    ref = topk_indices(sc, k)
    for r in range(got.shape[0]):
        a = set(got[r][got[r] >= 0].tolist())
        b = set(ref[r][ref[r] >= 0].tolist())
        if a == b:
            continue
        assert len(a) == len(b), f"row {r}: {len(a)} picks vs {len(b)}"
        fin = sc[r][np.isfinite(sc[r])]
        kth = np.sort(fin)[::-1][min(k, len(fin)) - 1]
        for e in a ^ b:
            tol = 2 * rtol * (ab[r, e] + abs(kth)) + 1e-12
            assert abs(sc[r, e] - kth) <= tol, (f"row {r}: entry {e} (score {sc[r, e]:.8g}) differs and is not a "
                                                f"near-tie of the k-th score {kth:.8g}")


def cosine(a, b) -> float:
    a = a.float().flatten()
    b = b.float().flatten()
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-30))


def assert_attn_close(got, ref, name="o"):
    got = got.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    c = cosine(got, ref)
    m = (got - ref).abs().max().item()
    assert c >= ATTN_COS_MIN and m <= ATTN_MAXABS, f"{name}: cosine {c:.6f} (min {ATTN_COS_MIN}), max-abs {m:.3e}"
