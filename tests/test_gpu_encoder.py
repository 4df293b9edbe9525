"""GPU: the hardware e4m3 encoder against the oracle's integer encoder, exhaustively over
bf16 inputs, and the quantizers on non-finite inputs.

Three FP8 quantizers encode with gfx950's ``v_cvt_pk_fp8_f32`` instead of the integer
encoder of the other kernels: the packed block quantizer (``quant_fp8_block``), the fused
decode indexer's query quantization (``decode_fp8``) and the fused prologue's query
quantization (``decode_fused``).  The FP8 codes of the reference are torch's
``float8_e4m3fn`` cast of ``clamp(x / s, +-448)`` (``owlet1/quant.py:81-85``); the oracle's
``e4m3_encode`` is pinned against that cast on the CPU.  Here every encoder is fed

* every finite bf16 value t with |t| <= 448 (the clamped domain, bf16 subnormals and both
  zeros included) as the encoder's own input: each block of 128 holds one anchor 448,
  which makes the block scale exactly 1, so the encoder sees t itself;
* every finite bf16 bit pattern, shuffled into blocks with their natural scales;

and the codes and scales must equal the oracle's bit for bit.

The non-finite cases follow the reference's arithmetic: torch's ``amax`` and ``clamp``
keep a NaN, so a block holding a NaN or an infinity gets an infinite power-of-two scale
(``_pow2_ceil_scale`` of a NaN / inf) and dequantizes to NaN throughout (0 * inf), and an
e4m3 scale that overflows e4m3 is NaN (``quant.py:60``).
"""

import numpy as np
import pytest
import torch

from mzoo_amd import indexer
from mzoo_amd import quant as MQ
from oracle import compressor as C
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _bf16_values(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _domain_blocks() -> np.ndarray:
    """[n, 128] fp32 (bf16-exact) blocks: column 0 = 448, then every finite bf16 t with
    |t| <= 448, each exactly once (the tail padded with zeros)."""
    v = _bf16_values(np.arange(1 << 16))
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    per = 127
    n = -(-v.size // per)
    body = np.zeros(n * per, np.float32)
    body[:v.size] = v
    blocks = np.concatenate([np.full((n, 1), 448.0, np.float32), body.reshape(n, per)], 1)
    return blocks


def _all_pattern_blocks() -> np.ndarray:
    v = _bf16_values(np.arange(1 << 16))
    v = v[np.isfinite(v)]
    v = v[np.random.default_rng(0).permutation(v.size)]
    n = -(-v.size // 128)
    out = np.zeros(n * 128, np.float32)
    out[:v.size] = v
    return out.reshape(n, 128)


def test_domain_blocks_cover_the_encoder_domain():
    """The blocks' scales are all 1, so the encoder inputs are exactly the bf16 domain."""
    blocks = _domain_blocks()
    assert np.all(Q.fp8_block_scales(blocks, 128) == 1.0)
    inputs = np.unique(blocks.view(np.uint32))
    v = _bf16_values(np.arange(1 << 16))
    want = np.unique(v[np.isfinite(v) & (np.abs(v) <= 448)].view(np.uint32))
    assert np.array_equal(np.intersect1d(inputs, want), want)


def _check_codes(codes, scales, blocks, tag):
    c_ref, s_ref = Q.fp8_block_codes(blocks, 128)
    got = codes.reshape(blocks.shape).cpu().numpy()
    bad = np.argwhere(got != c_ref)
    assert bad.size == 0, (f"{tag}: {len(bad)} codes differ, first input {blocks[tuple(bad[0])]!r}: "
                           f"{got[tuple(bad[0])]:#x} vs {c_ref[tuple(bad[0])]:#x}")
    assert np.array_equal(scales.reshape(-1).cpu().numpy().view(np.int32), s_ref.reshape(-1).view(np.int32)), \
        f"{tag}: scales differ"


@pytest.mark.parametrize("which", ["domain", "all_patterns"])
def test_quant_fp8_block_hardware_encoder_exhaustive(dev, which):
    blocks = _domain_blocks() if which == "domain" else _all_pattern_blocks()
    x = torch.from_numpy(blocks).bfloat16().to(dev)
    print(f"quant_fp8_block exhaustive: {which} {tuple(x.shape)}", flush=True)
    codes, scales = MQ.quant_fp8_block(x, 128)
    torch.cuda.synchronize()
    _check_codes(codes, scales, blocks, f"quant_fp8_block/{which}")


def _decode_inputs(blocks, dev, hi=64, g=64):
    n = blocks.shape[0]
    b = -(-n // hi)
    q = np.zeros((b * hi, 128), np.float32)
    q[:n] = blocks
    q_idx = torch.from_numpy(q).bfloat16().view(b, hi, 128).to(dev)
    gen = torch.Generator().manual_seed(3)
    w = (torch.randn(b, hi, generator=gen) * hi ** -0.5).to(dev)
    kc, ks = MQ.quant_fp8_block(torch.randn(b, g, 128, generator=gen).bfloat16().to(dev), 128)
    return b, hi, q, q_idx, w, kc, ks[..., 0].contiguous()


@pytest.mark.parametrize("path", ["decode_fp8", "decode_fused"])
@pytest.mark.parametrize("which", ["domain", "all_patterns"])
def test_decode_query_hardware_encoder_exhaustive(dev, path, which):
    """The fused decode indexers quantize the bf16 query in the kernel; with identity RoPE
    tables (cos 1, sin 0) the fused prologue's encoder sees the query itself except for the
    sign of zeros in odd channels, which the oracle's rotation gives."""
    blocks = _domain_blocks() if which == "domain" else _all_pattern_blocks()
    b, hi, q, q_idx, w, kc, ks = _decode_inputs(blocks, dev)
    pos = torch.full((b,), 1023, dtype=torch.int64, device=dev)
    q_codes = torch.empty(b, hi, 128, dtype=torch.uint8, device=dev)
    q_scales = torch.empty(b, hi, dtype=torch.float32, device=dev)
    print(f"{path} query encoder: {which} B={b}", flush=True)
    if path == "decode_fp8":
        indexer.decode_fp8(q_idx, w, kc, ks, compress_ratio=4, positions=pos, q_codes=q_codes, q_scales=q_scales)
    else:
        ones = torch.ones(b, 32, dtype=torch.bfloat16, device=dev)
        zeros = torch.zeros(b, 32, dtype=torch.bfloat16, device=dev)
        win = torch.zeros(b, 128, 656, dtype=torch.uint8, device=dev)
        kv = torch.randn(b, 576, generator=torch.Generator().manual_seed(4)).bfloat16().to(dev)
        indexer.decode_fused(q_idx, w, kc, ks, fmt="fp8", compress_ratio=4, positions=pos, q_rope=(ones, zeros),
                             kv=kv, kv_weight=torch.ones(576, dtype=torch.bfloat16, device=dev), kv_eps=1e-6,
                             kv_rope=(ones, zeros), win_cache=win, q_codes=q_codes, q_scales=q_scales)
    torch.cuda.synchronize()
    if path == "decode_fused":
        # the rotation is not the identity on signed zeros: an odd channel -0.0 becomes
        # e*0 + (-0)*1 = +0 (norm_rope.py:144), so the encoder's input is the oracle's rotation
        one, zero = np.ones((q.shape[0], 1, 32), np.float32), np.zeros((q.shape[0], 1, 32), np.float32)
        q = C.rope(q[:, None, :], one, zero, dtype="bfloat16")[:, 0, :]
    _check_codes(q_codes.view(-1, 128), q_scales, q, f"{path}/{which}")


def _fp4_domain_blocks() -> np.ndarray:
    """[n, 128] fp32 (bf16-exact) rows of four MXFP4 blocks of 32: each block = 6 then 31
    values, so its scale is exactly 1 and the encoder sees every finite bf16 t with |t| <= 6
    (the saturating domain, bf16 subnormals and both zeros included) itself."""
    v = _bf16_values(np.arange(1 << 16))
    v = v[np.isfinite(v) & (np.abs(v) <= 6)]
    per = 31
    nb = -(-v.size // per)
    nb = -(-nb // 4) * 4
    body = np.zeros(nb * per, np.float32)
    body[:v.size] = v
    blocks = np.concatenate([np.full((nb, 1), 6.0, np.float32), body.reshape(nb, per)], 1)
    return blocks.reshape(-1, 128)


@pytest.mark.parametrize("path", ["decode_mxfp4", "decode_fused"])
@pytest.mark.parametrize("which", ["domain", "all_patterns", "nonfinite"])
def test_decode_query_mxfp4_encoder_exhaustive(dev, path, which):
    """The MXFP4 decode indexers quantize the bf16 query in the kernel (the scaled e2m1
    conversion for blocks with a finite maximum, the software encoder for a block with a NaN
    or an infinity); codes and e8m0 scales must equal the oracle's (``quant_mxfp4``) bit for
    bit -- every finite bf16 value in the saturating domain as the encoder's own input, every
    finite bf16 pattern with natural block scales, and blocks holding NaN / +-inf."""
    if which == "domain":
        blocks = _fp4_domain_blocks()
    elif which == "all_patterns":
        blocks = _all_pattern_blocks()
    else:
        blocks = _nonfinite_inputs(64 * 4, 128, 11).numpy()
        blocks = Q.round_bf16(blocks)
    hi = 64
    n = blocks.shape[0]
    b = -(-n // hi)
    q = np.zeros((b * hi, 128), np.float32)
    q[:n] = blocks
    q_idx = torch.from_numpy(q).bfloat16().view(b, hi, 128).to(dev)
    gen = torch.Generator().manual_seed(5)
    w = (torch.randn(b, hi, generator=gen) * hi ** -0.5).to(dev)
    kp, ke = MQ.quant_mxfp4(torch.randn(b, 64, 128, generator=gen).bfloat16().to(dev))
    pos = torch.full((b,), 255, dtype=torch.int64, device=dev)
    qp = torch.empty(b, hi, 64, dtype=torch.uint8, device=dev)
    qe = torch.empty(b, hi, 4, dtype=torch.uint8, device=dev)
    print(f"{path} MXFP4 query encoder: {which} B={b}", flush=True)
    if path == "decode_mxfp4":
        indexer.decode_mxfp4(q_idx, w, kp, ke, compress_ratio=4, positions=pos, q_packed=qp, q_e8m0=qe)
    else:
        ones = torch.ones(b, 32, dtype=torch.bfloat16, device=dev)
        zeros = torch.zeros(b, 32, dtype=torch.bfloat16, device=dev)
        win = torch.zeros(b, 128, 656, dtype=torch.uint8, device=dev)
        kv = torch.randn(b, 576, generator=torch.Generator().manual_seed(4)).bfloat16().to(dev)
        indexer.decode_fused(q_idx, w, kp, ke, fmt="mxfp4", compress_ratio=4, positions=pos, q_rope=(ones, zeros),
                             kv=kv, kv_weight=torch.ones(576, dtype=torch.bfloat16, device=dev), kv_eps=1e-6,
                             kv_rope=(ones, zeros), win_cache=win, q_codes=qp, q_scales=qe)
        # an odd channel's -0.0 is rotated to +0 (norm_rope.py:144): the encoder's input is the
        # oracle's rotation with the identity tables
        one, zero = np.ones((q.shape[0], 1, 32), np.float32), np.zeros((q.shape[0], 1, 32), np.float32)
        q = C.rope(q[:, None, :], one, zero, dtype="bfloat16")[:, 0, :]
    torch.cuda.synchronize()
    p_ref, e_ref = Q.quant_mxfp4(q.reshape(b, hi, 128))
    got_p, got_e = qp.cpu().numpy(), qe.cpu().numpy()
    assert np.array_equal(got_e, e_ref), f"{path}/{which}: e8m0 scales differ"
    # a block with a NaN or an infinity has an infinite scale and dequantizes to NaN whatever
    # its codes (0 * inf); the sign of a NaN code there (x86's default NaN of the oracle's
    # inf / inf is negative) is no part of the format: such blocks compare dequantized
    fin = np.isfinite(q.reshape(b, hi, 4, 32)).all(-1)                     # [b, hi, 4]
    fin_bytes = np.repeat(fin, 16, -1)                                     # [b, hi, 64]
    bad = np.argwhere((got_p != p_ref) & fin_bytes)
    assert bad.size == 0, (f"{path}/{which}: {len(bad)} code bytes differ, first at {tuple(bad[0])}: "
                           f"{got_p[tuple(bad[0])]:#x} vs {p_ref[tuple(bad[0])]:#x}")
    if not fin.all():
        _same_values(torch.from_numpy(Q.dequant_mxfp4(got_p, got_e)), Q.dequant_mxfp4(p_ref, e_ref))


# ---- non-finite inputs -------------------------------------------------------------------

def _nonfinite_inputs(rows, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n, generator=g) * 3
    specials = [float("nan"), float("inf"), float("-inf"), -float("nan")]
    for r in range(0, rows, 3):
        x[r, (r * 7) % n] = specials[(r // 3) % 4]
    x[1, :] = 5000.0       # large amax: the e4m3-scaled FP4 scale overflows e4m3 (NaN)
    return x


def _same_values(got: torch.Tensor, want: np.ndarray) -> None:
    g = got.float().cpu().numpy()
    w = np.asarray(want, np.float32)
    assert np.array_equal(np.isnan(g), np.isnan(w)), f"NaN pattern differs at {int((np.isnan(g) != np.isnan(w)).sum())}"
    ok = ~np.isnan(w)
    assert np.array_equal(g[ok].view(np.int32), w[ok].view(np.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["fp8_32", "fp8_128", "fp4_32", "fp4_16_e4m3"])
def test_fake_quant_nonfinite(dev, dtype, kind):
    x = _nonfinite_inputs(97, 256, 7).to(dtype)
    xn = x.float().numpy()
    name = {torch.float32: "float32", torch.bfloat16: "bfloat16"}[dtype]
    if kind.startswith("fp8"):
        bs = int(kind.split("_")[1])
        got = MQ._fake_quant_fp8_block(x.to(dev), bs)
        want = Q.fake_quant_fp8_block(xn, bs, dtype=name)
    else:
        bs = int(kind.split("_")[1])
        e4 = kind.endswith("e4m3")
        got = MQ._fake_quant_fp4_block(x.to(dev), bs, e4m3_scales=e4)
        want = Q.fake_quant_fp4_block(xn, bs, e4, dtype=name)
    torch.cuda.synchronize()
    assert np.isnan(want).any()
    _same_values(got, want)


def test_packed_quant_nonfinite(dev):
    """The packed forms dequantize to the fake quantizer's values (NaN blocks included)."""
    x = _nonfinite_inputs(60, 128, 8).bfloat16()
    xn = x.float().numpy()
    codes, scales = MQ.quant_fp8_block(x.to(dev), 128)
    _same_values(MQ.dequant_fp8_block(codes, scales, 128), Q.fake_quant_fp8_block(xn, 128))
    lat = torch.cat([x, x.flip(0), x.flip(1), x, torch.zeros(60, 64, dtype=x.dtype)], 1)   # nope 512 + rope 64
    e = MQ.pack_latent_fp8_b128(lat.to(dev))
    back = MQ.unpack_latent_fp8_b128(e, dtype=torch.float32)[:, :512]
    _same_values(back, Q.fake_quant_fp8_block(lat[:, :512].float().numpy(), 128))
