"""CPU: pin the compressor / RMSNorm / RoPE oracle (oracle/compressor.py).

The oracle fixes the float32 evaluation order that torch leaves implementation-defined;
these checks show it still computes the reference's functions:
* ``exp_f32`` within 2 ulp of float64 ``exp`` over the softmax range (and exact at 0);
* ``softmax_pool`` within a few ulp of the reference expression evaluated by torch's own
  ``softmax`` (``owlet1/cache.py:171``), plus closed forms: a one-hot gate returns that
  token's kv exactly, a constant gate returns the mean;
* ``rms_norm`` within a few ulp of torch's ``x * rsqrt(mean(x^2) + eps)``; a constant
  vector normalises to +-weight;
* ``rope``: position 0 is the identity, inverse after forward restores x, and the
  rotation preserves each pair's norm;
* ``split_groups``: the carry invariant of ``store_compression_weights``;
* ``decode_kv_latent`` against the reference's norm-then-rotate steps run by torch in
  bf16, and at position 0 equal to the plain norm.
"""

import numpy as np
import pytest
import torch

from oracle import compressor as C
from oracle import quant as Q


def _ulps(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b) / np.spacing(np.abs(b).astype(np.float32)).astype(np.float64)


def test_exp_accuracy():
    x = np.concatenate([-np.random.default_rng(0).exponential(6, 2_000_000),
                        np.linspace(-103, 0, 100001), [0.0, -0.0]]).astype(np.float32)
    got = C.exp_f32(x)
    ref = np.exp(x.astype(np.float64))
    normal = ref >= 2.0 ** -126
    assert _ulps(got[normal], ref[normal]).max() <= 2.0
    assert np.all(np.abs(got[~normal] - ref[~normal]) <= 2.0 ** -149)
    assert C.exp_f32(np.float32(0.0)) == 1.0
    assert C.exp_f32(np.float32(-np.inf)) == 0.0


def test_softmax_pool_matches_torch_softmax():
    rng = np.random.default_rng(1)
    kv = rng.standard_normal((4, 64, 4, 576)).astype(np.float32)
    gate = (rng.standard_normal((4, 64, 4, 576)) * 3).astype(np.float32)
    got = C.softmax_pool(kv, gate)
    t_kv, t_g = torch.from_numpy(kv), torch.from_numpy(gate)
    ref = (t_kv * t_g.softmax(dim=2, dtype=torch.float32)).sum(dim=2).numpy()   # cache.py:171
    err = np.abs(got.astype(np.float64) - ref)
    scale = np.abs(kv).max(axis=2)
    assert (err / scale).max() < 4 * 2.0 ** -23


def test_softmax_pool_closed_forms():
    rng = np.random.default_rng(2)
    kv = rng.standard_normal((3, 5, 4, 32)).astype(np.float32)
    onehot = np.full((3, 5, 4, 32), -200.0, np.float32)
    onehot[:, :, 2, :] = 0.0
    assert np.array_equal(C.softmax_pool(kv, onehot), kv[:, :, 2, :])
    const = np.zeros((3, 5, 4, 32), np.float32)
    mean = ((kv[:, :, 0] + kv[:, :, 1]) + kv[:, :, 2] + kv[:, :, 3]) * np.float32(0.25)
    assert np.allclose(C.softmax_pool(kv, const), mean, rtol=0, atol=4e-7 * np.abs(kv).max())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rms_norm_matches_torch(dtype):
    rng = np.random.default_rng(3)
    x = Q.round_to(rng.standard_normal((256, 576)).astype(np.float32) * 3, dtype)
    w = Q.round_to(rng.uniform(0.5, 1.5, 576).astype(np.float32), dtype)
    got = C.rms_norm(x, w, 1e-20, dtype)
    tdt = torch.float32 if dtype == "float32" else torch.bfloat16
    h = torch.from_numpy(x).float()
    ref = (torch.from_numpy(w).to(tdt) * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-20)).to(tdt)).float()
    ulp = 2.0 ** -23 if dtype == "float32" else 2.0 ** -8
    assert np.max(np.abs(got - ref.numpy()) / np.maximum(np.abs(ref.numpy()), 1e-30)) <= 4 * ulp


def test_rms_norm_constant_vector():
    x = np.full((2, 160), -3.0, np.float32)
    w = np.linspace(0.5, 2, 160).astype(np.float32)
    got = C.rms_norm(x, w, 1e-20, "float32")
    assert np.allclose(got, -w, rtol=2e-7, atol=0)


def test_compress_ratio1_is_plain_norm():
    rng = np.random.default_rng(4)
    kv = rng.standard_normal((2, 8, 160)).astype(np.float32)
    w = np.ones(160, np.float32)
    assert np.array_equal(C.compress(kv, None, 1, w, 1e-6, "float32"), C.rms_norm(kv, w, 1e-6, "float32"))


def test_rope_identities():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 7, 4, 160)).astype(np.float32)
    cos0, sin0 = C.rope_tables(np.zeros((2, 7)), 32, 160000.0)
    assert np.array_equal(C.rope(x, cos0[:, :, None], sin0[:, :, None]), x)
    cos, sin = C.rope_tables(rng.integers(0, 100000, (2, 7)), 32, 160000.0)
    y = C.rope(x, cos[:, :, None], sin[:, :, None])
    back = C.rope(y, cos[:, :, None], sin[:, :, None], inverse=True)
    assert np.allclose(back, x, atol=1e-5)
    assert np.array_equal(y[..., :128], x[..., :128])
    n_in = x[..., 128::2] ** 2 + x[..., 129::2] ** 2
    n_out = y[..., 128::2] ** 2 + y[..., 129::2] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)


def _torch_decode_latent(kv, w, eps, cos, sin):
    """attention.py:150-151 stated with torch's own ops in bf16: kv_norm (norm_rope.py:25-30)
    then apply_rotary_pos_emb (norm_rope.py:126-145) on the trailing 2*len(cos) channels."""
    h = kv.float()
    normed = w * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    rd = cos.shape[-1] * 2
    nope, rope = normed[..., :-rd], normed[..., -rd:]
    even, odd = rope[..., 0::2].float(), rope[..., 1::2].float()
    rot = torch.stack([even * cos - odd * sin, even * sin + odd * cos], dim=-1).flatten(-2)
    return torch.cat([nope, rot.to(torch.bfloat16)], -1)


def test_decode_kv_latent_matches_torch():
    """The composition order (norm, weight in bf16, then the rotation of the trailing 64
    channels) against the reference's steps run by torch: equal up to torch's own rsqrt /
    mean rounding (a bf16 ulp on a few channels)."""
    rng = np.random.default_rng(8)
    kv = Q.round_bf16(rng.standard_normal((64, 576)).astype(np.float32) * rng.uniform(0.01, 50, (64, 1)))
    w = Q.round_bf16(rng.uniform(0.5, 1.5, 576).astype(np.float32))
    cos, sin = C.rope_tables(rng.integers(0, 1 << 19, 64), 64, 10000.0)
    cos, sin = Q.round_bf16(cos), Q.round_bf16(sin)
    got = C.decode_kv_latent(kv, w, 1e-6, cos, sin)
    ref = _torch_decode_latent(torch.from_numpy(kv).bfloat16(), torch.from_numpy(w).bfloat16(), 1e-6,
                               torch.from_numpy(cos).bfloat16(), torch.from_numpy(sin).bfloat16()).float().numpy()
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert np.max(rel) <= 2 * 2.0 ** -8
    assert np.mean(got == ref) > 0.98
    # the rope slice is rotated and the nope slice is not: swapping the two steps, or
    # rotating the leading channels, breaks the match above; and at position 0 the latent
    # is the plain norm
    c0, s0 = C.rope_tables(np.zeros(64), 64, 10000.0)
    assert np.array_equal(C.decode_kv_latent(kv, w, 1e-6, Q.round_bf16(c0), Q.round_bf16(s0)),
                          C.rms_norm(kv, w, 1e-6, "bfloat16"))
    assert not np.array_equal(got[:, 512:], C.rms_norm(kv, w, 1e-6, "bfloat16")[:, 512:])
    assert np.array_equal(got[:, :512], C.rms_norm(kv, w, 1e-6, "bfloat16")[:, :512])


def test_split_groups_carry():
    buffered, emitted, ratio = 0, 0, 4
    for new in [5, 1, 1, 1, 9, 0, 3]:
        usable, buffered = C.split_groups(buffered, new, ratio)
        assert usable % ratio == 0 and 0 <= buffered < ratio
        emitted += usable // ratio
    assert emitted == (5 + 1 + 1 + 1 + 9 + 0 + 3) // ratio


def test_rope_is_complex_multiplication():
    """norm_rope.py:128-131 names the convention: the (even, odd) pairs of the rope slice are
    complex numbers ``view_as_complex(x.unflatten(-1, (-1, 2)))`` multiplied by
    ``cos + i sin``; the inverse multiplies by the conjugate.  Checked against torch's
    complex arithmetic (not a restatement of the oracle's real-arithmetic formula), so a
    flipped sign of ``sin`` or swapped pair order fails here."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 5, 4, 96)).astype(np.float32)
    cos, sin = C.rope_tables(rng.integers(0, 1 << 20, (3, 5)), 32, 10000.0)
    got = C.rope(x, cos[:, :, None], sin[:, :, None])
    z = torch.view_as_complex(torch.from_numpy(x[..., 64:]).double().unflatten(-1, (-1, 2)).contiguous())
    rot = torch.complex(torch.from_numpy(cos).double(), torch.from_numpy(sin).double())[:, :, None]
    want = torch.view_as_real(z * rot).flatten(-2).numpy()
    assert np.allclose(got[..., 64:], want, rtol=0, atol=2e-6)
    assert np.array_equal(got[..., :64], x[..., :64])
    inv = C.rope(x, cos[:, :, None], sin[:, :, None], inverse=True)
    want_inv = torch.view_as_real(z * rot.conj()).flatten(-2).numpy()
    assert np.allclose(inv[..., 64:], want_inv, rtol=0, atol=2e-6)


def test_rope_quarter_turn_closed_form():
    """cos = 0, sin = 1 is multiplication by i: (e, o) -> (-o, e); the inverse gives (o, -e)."""
    x = np.arange(1, 9, dtype=np.float32).reshape(1, 8)
    c, s = np.zeros((1, 2), np.float32), np.ones((1, 2), np.float32)
    assert C.rope(x, c, s).tolist() == [[1, 2, 3, 4, -6, 5, -8, 7]]
    assert C.rope(x, c, s, inverse=True).tolist() == [[1, 2, 3, 4, 6, -5, 8, -7]]


def test_rope_tables_closed_form():
    """inv_freq_i = theta^(-2i/rd) (dsv4 modeling_deepseek_v41.py:127-137): pair 0 rotates by
    the position itself, pair i by pos * theta^(-2i/rd); checked in float64 math."""
    pos = np.array([0, 1, 2, 3, 1000, 65535], np.float64)
    for rd, theta in ((64, 10000.0), (32, 160000.0)):
        cos, sin = C.rope_tables(pos, rd, theta)
        assert np.allclose(cos[:, 0], np.cos(pos), atol=1e-6) and np.allclose(sin[:, 0], np.sin(pos), atol=1e-6)
        i = np.arange(rd // 2)
        ang = pos[:, None] * theta ** (-2.0 * i / rd)
        # fp32 angle rounding grows with the position: |pos * inv_freq| ulp
        tol = 4 * np.abs(ang) * 2.0 ** -24 + 1e-6
        assert np.all(np.abs(cos - np.cos(ang)) <= tol) and np.all(np.abs(sin - np.sin(ang)) <= tol)


def test_linear_pinned_against_float64():
    """The pinned-order key projection: within one float32 rounding chain of the exact
    (float64) product, and after rounding to bf16 equal to the exact product's rounding
    except where the exact value sits within that error of a bf16 rounding boundary."""
    rng = np.random.default_rng(12)
    x = Q.round_bf16(rng.standard_normal((64, 576)).astype(np.float32))
    w = Q.round_bf16((rng.standard_normal((128, 576)) * 0.05).astype(np.float32))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    got32 = C.linear_pinned(x, w, "float32")
    bound = 576 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got32 - exact) <= bound)
    got = C.linear_pinned(x, w, "bfloat16")
    want = Q.round_bf16(exact.astype(np.float32))
    mism = got != want
    assert mism.mean() < 0.01
    # a mismatch only where the exact value is close to a bf16 midpoint
    ulp = np.abs(want) * 2.0 ** -8
    assert np.all(np.abs(got[mism] - exact[mism]) <= ulp[mism] + bound[mism])


def test_emit_group_matches_the_reference_steps():
    """emit_group against the reference's own steps run by torch in bf16: compressor pooling
    (fp32 softmax-weighted sum, cache.py:168-172) -> kv norm -> RoPE, and k_norm(wk(latent))
    -> RoPE (indexer.py:96-103) with torch's bf16 linear: equal up to torch's own rounding
    (exp / rsqrt / GEMM order), a bf16 ulp on a few channels."""
    rng = np.random.default_rng(13)
    b, r, d, di = 8, 4, 576, 128
    kv = rng.standard_normal((b, r, d)).astype(np.float32)
    gate = rng.standard_normal((b, r, d)).astype(np.float32)
    nw = Q.round_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    wk = Q.round_bf16((rng.standard_normal((di, d)) * 0.04).astype(np.float32))
    kw = Q.round_bf16(rng.uniform(0.5, 1.5, di).astype(np.float32))
    cos, sin = C.rope_tables(np.arange(b) * 4 * 97, 64, 160000.0)
    cos, sin = Q.round_bf16(cos), Q.round_bf16(sin)
    rot, key = C.emit_group(kv, gate, r, nw, 1e-6, cos, sin, wk, kw, 1e-6)

    def norm(h, w, eps):
        hf = h.float()
        return w * (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)

    def rot_t(x, c, s):
        rd = c.shape[-1] * 2
        even, odd = x[..., -rd::2].float(), x[..., -rd + 1::2].float()
        out = torch.stack([even * c - odd * s, even * s + odd * c], -1).flatten(-2).to(torch.bfloat16)
        return torch.cat([x[..., :-rd], out], -1)

    kt, gt = torch.from_numpy(kv), torch.from_numpy(gate)
    lat = norm((kt * gt.softmax(dim=1, dtype=torch.float32)).sum(1).to(torch.bfloat16),
               torch.from_numpy(nw).bfloat16(), 1e-6)
    ct, st = torch.from_numpy(cos).bfloat16(), torch.from_numpy(sin).bfloat16()
    ref_rot = rot_t(lat, ct, st).float().numpy()
    k = torch.nn.functional.linear(lat, torch.from_numpy(wk).bfloat16())
    ref_key = rot_t(norm(k, torch.from_numpy(kw).bfloat16(), 1e-6), ct, st).float().numpy()
    for got, ref in ((rot, ref_rot), (key, ref_key)):
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert np.max(rel) <= 4 * 2.0 ** -8
        assert np.mean(got == ref) > 0.95
