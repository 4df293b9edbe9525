"""CPU: pin the quantizer oracle (oracle/quant.py) before trusting it as the checker.

Pins, each chosen so a plausible slip fails one of them:
* the reference's own known answers (owlet1/quant.md:46-48 tie table, -0 -> code 8,
  the e2m1 value table quant.py:8-11) from tests/golden/kat.json;
* ``pow2_ceil_scale`` against the closed form ``2^ceil(log2 t)`` from ``math.frexp``;
* ``e2m1_codes`` against brute force "nearest grid value, ties to the even code";
* ``e4m3_encode`` against torch's own ``float8_e4m3fn`` cast (the library the reference
  calls, quant.py:60,85) on every fp32 of 2^13 mantissa patterns x all exponents in
  [2^-20, 480) plus all subnormal-fp8 neighbourhoods;
* invariants of the composed quantizers: the ceil rule never clips, outputs lie on the
  scaled grid, pass-through when ``n % block_size``, floors, the +0.0 of code 8.
"""

import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import quant as Q

KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "kat.json").read_text())


def test_e2m1_tie_table_kat():
    k = KAT["e2m1_ties"]
    assert Q.e2m1_codes(np.array(k["q"], np.float32)).tolist() == k["codes"]
    assert int(Q.e2m1_codes(np.array([-0.0], np.float32))[0]) == k["negative_zero_code"]
    assert Q.FP4_TABLE.tolist() == KAT["fp4_table"]["values"]


def _nearest_even_e2m1(a: float) -> int:
    grid = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    d = [abs(a - g) for g in grid]
    best = min(d)
    cands = [i for i, v in enumerate(d) if v == best]
    return min(cands, key=lambda i: (i % 2, i))  # ties go to the even code


def test_e2m1_brute_force_nearest_even():
    rng = np.random.default_rng(0)
    vals = [0.0, 6.0] + list(np.linspace(0, 6, 20001))
    for b in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0):   # every tie and its fp32 neighbours
        x = np.float32(b)
        for _ in range(8):
            vals += [float(x)]
            x = np.nextafter(x, np.float32(7))
        x = np.float32(b)
        for _ in range(8):
            x = np.nextafter(x, np.float32(-1))
            vals += [float(x)]
    vals += list(rng.uniform(0, 6, 20000))
    a = np.array(vals, np.float32)
    got = Q.e2m1_codes(a)
    want = np.array([_nearest_even_e2m1(float(v)) for v in a])
    assert np.array_equal(got, want)
    assert np.array_equal(Q.e2m1_codes(-a[a > 0]), want[a > 0] | 8)


def test_pow2_ceil_closed_form():
    rng = np.random.default_rng(1)
    t = np.concatenate([rng.uniform(1e-30, 1e30, 5000).astype(np.float32),
                        np.exp2(np.arange(-126, 127)).astype(np.float32),
                        np.float32(2.0) ** np.arange(-20, 20).astype(np.float32) * np.float32(1.0000001)])
    got = Q.pow2_ceil_scale(t)
    for v, g in zip(t.tolist(), got.tolist()):
        m, e = math.frexp(v)           # v = m * 2^e, m in [0.5, 1)
        want = 2.0 ** (e - 1) if m == 0.5 else 2.0 ** e
        assert g == want, (v, g, want)


def _all_mantissas(exp_lo, exp_hi, step=1 << 10):
    out = []
    for e in range(exp_lo, exp_hi):
        m = np.arange(0, 1 << 23, step, dtype=np.uint32)
        m = np.concatenate([m, m + 1, m + (step >> 1), m + (step >> 1) - 1, m + (step >> 1) + 1])
        m = m[m < (1 << 23)]
        out.append(((np.uint32(e) << 23) | m).view(np.float32))
    return np.concatenate(out)


def test_e4m3_encode_matches_torch_cast():
    x = _all_mantissas(127 - 20, 127 + 9)
    x = x[np.abs(x) < 480]
    x = np.concatenate([x, -x, np.array([0.0, -0.0, 1e-45, -1e-45], np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(Q.e4m3_encode(x), ref)
    dec = torch.from_numpy(np.arange(256, dtype=np.uint8)).view(torch.float8_e4m3fn).float().numpy()
    mine = Q.e4m3_decode(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(dec), np.isnan(mine))
    ok = ~np.isnan(dec)
    assert np.array_equal(dec[ok].view(np.uint32), mine[ok].view(np.uint32))


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32),
                        _all_mantissas(120, 125, step=1 << 12)])
    ref = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(Q.round_bf16(x).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("bs", [16, 32, 128])
def test_fp8_fake_quant_invariants(bs):
    rng = np.random.default_rng(bs)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    codes, scale = Q.fp8_block_codes(x, bs)
    blocks = np.abs(x.reshape(64, -1, bs))
    amax = np.maximum(blocks.max(-1), np.float32(1e-4))
    assert np.all(amax / scale <= 448.0)                     # ceil rule: clamp never clips
    assert np.all(amax / scale > 224.0 - 1e-3)               # ... and the scale is the smallest such pow2
    assert np.all(np.log2(scale) == np.round(np.log2(scale)))
    y = Q.fake_quant_fp8_block(x, bs)
    assert np.all(np.abs(y - x) <= np.repeat(scale, bs, -1) * 16)   # half an e4m3 ulp at the top binade
    assert np.array_equal(Q.fake_quant_fp8_block(y, bs), y)         # idempotent
    assert Q.fake_quant_fp8_block(x[:, :250], bs) is not None
    z = x[:, :250]
    assert Q.fake_quant_fp8_block(z, bs) is z or 250 % bs == 0      # pass-through object


def test_fp8_floor_and_zero_sign():
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = -0.0
    x[0, 1] = 1e-6
    codes, s = Q.fp8_block_codes(x, 32)
    assert s[0, 0] == Q.pow2_ceil_scale(np.float32(1e-4) * np.float32(1 / 448))
    assert codes[0, 0] == 0x80                                   # -0.0 keeps its sign in fp8
    y = Q.fake_quant_fp8_block(x, 32)
    assert np.signbit(y[0, 0])


@pytest.mark.parametrize("e4m3", [False, True])
@pytest.mark.parametrize("bs", [16, 32])
def test_fp4_fake_quant_invariants(bs, e4m3):
    rng = np.random.default_rng(7 + bs)
    x = (rng.standard_normal((32, 128)) * np.exp(rng.uniform(-4, 4, (32, 1)))).astype(np.float32)
    codes, scale = Q.fp4_block_codes(x, bs, e4m3)
    y = Q.fake_quant_fp4_block(x, bs, e4m3)
    grid = Q.FP4_TABLE[codes.astype(int)] * np.repeat(scale, bs, -1)
    assert np.array_equal(grid, y)
    if not e4m3:
        amax = np.abs(x.reshape(32, -1, bs)).max(-1)
        assert np.all(amax / scale <= 6.0)
    # a negative value that rounds to zero decodes to +0.0 (code 8 -> +0.0)
    tiny = np.zeros((1, bs), np.float32)
    tiny[0, 0], tiny[0, 1] = 1.0, -1e-3
    assert not np.signbit(Q.fake_quant_fp4_block(tiny, bs, e4m3)[0, 1])


def test_fp4_scale_floors():
    z = np.zeros((1, 32), np.float32)
    assert Q.fp4_block_scales(z, 32)[0, 0] == Q.pow2_ceil_scale(np.float32(6 * 2.0 ** -126) * np.float32(1 / 6))
    assert Q.fp4_block_scales(z, 32, True)[0, 0] == np.float32(2.0 ** -9)


def test_packed_formats_roundtrip():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((10, 576)).astype(np.float32)
    e = Q.pack_latent_fp8_b128(x)
    assert e.shape == (10, 656) and e.dtype == np.uint8
    back = Q.unpack_latent_fp8_b128(e)
    assert np.array_equal(back[:, :512], Q.fake_quant_fp8_block(x[:, :512], 128))
    assert np.array_equal(back[:, 512:], Q.round_bf16(x[:, 512:]))
    p, s = Q.quant_mxfp4(x[:, :128])
    assert p.shape == (10, 64) and s.shape == (10, 4)
    assert np.array_equal(Q.dequant_mxfp4(p, s), Q.fake_quant_fp4_block(x[:, :128], 32))
    c, sc = Q.fp8_block_codes(x[:, :128], 128)
    assert np.array_equal(Q.dequant_fp8_block(c, sc, 128), Q.fake_quant_fp8_block(x[:, :128], 128))


def _decode_v41(entries, d, fmt):
    """The V4.1 entry layout read back independently of the packer (codes, then scales)."""
    e = np.asarray(entries, np.uint8)
    if fmt == "fp8":
        codes, sc = e[..., :d], e[..., d:d + d // 32]
        vals = Q.e4m3_decode(codes).reshape(*e.shape[:-1], d // 32, 32)
        scale = Q.e8m0_decode(sc)
        return (vals * scale[..., None]).reshape(*e.shape[:-1], d)
    nib = e[..., :d // 2]
    codes = np.stack([nib & 0xF, nib >> 4], -1).reshape(*e.shape[:-1], d)
    vals = Q.FP4_TABLE[codes.astype(np.int64)].reshape(*e.shape[:-1], d // 16, 16)
    scale = Q.e4m3_decode(e[..., d // 2:d // 2 + d // 16])
    return (vals * scale[..., None]).reshape(*e.shape[:-1], d)


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_v41_cache_entries_decode_to_fake_quant(fmt):
    """FlashMLA's V4.1 rows (fp_attn_notes.md:1123-1131): 528 / 288 bytes per 512-channel
    token, and the entry decodes exactly to the reference quantizer the cache stands for."""
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((5, 512)) * rng.uniform(1e-3, 300, (5, 1))).astype(np.float32)
    x[0, :32] = 0.0                       # an all-zero scale block
    # a block with a large outlier (within the e4m3 scale's range, amax / 6 <= 448, for fp4)
    x[1, 40] = 448.0 * 2.0 ** 20 if fmt == "fp8" else 2000.0
    e = Q.pack_cache_v41(x, fmt)
    assert e.shape == (5, 528 if fmt == "fp8" else 288) and e.dtype == np.uint8
    ref = Q.fake_quant_fp8_block(x, 32) if fmt == "fp8" else Q.fake_quant_fp4_block(x, 16, e4m3_scales=True)
    assert np.array_equal(_decode_v41(e, 512, fmt), ref)


def test_v41_fp4_nibble_order():
    """Element 2i sits in the low nibble: a block whose first value is its amax (code 7 =
    6.0 x scale) and whose second is 0 packs its first byte as 0x07."""
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 3.0
    e = Q.pack_cache_v41(x, "fp4")
    assert e[0, 0] == 0x07
    assert Q.e4m3_decode(e[0, 16:17])[0] == np.float32(0.5)   # scale amax / 6 = 0.5, exact in e4m3


def test_nonfinite_blocks_follow_torch_semantics():
    """A NaN or an infinity in a block: the reference's torch ops keep it through ``amax``
    and ``clamp_min`` (checked here on the library), ``_pow2_ceil_scale`` of a NaN / inf is
    2^129 / 2^128 = inf, so ``x / scale`` is 0 (or NaN) and the block dequantizes to NaN
    everywhere (0 * inf); an e4m3 scale above e4m3's range casts to NaN.  Blocks without
    such values are untouched by their neighbours."""
    t = torch.tensor([[1.0, float("nan"), 2.0]])
    assert torch.isnan(t.abs().amax(-1)).all() and torch.isnan(t.abs().amax(-1).clamp_min(1e-4)).all()
    assert torch.isnan(torch.tensor([float("nan")]).clamp(-448.0, 448.0)).all()
    e4 = torch.tensor([float("nan"), float("inf"), 500.0, 470.0]).to(torch.float8_e4m3fn).float()
    assert torch.isnan(e4).all()
    assert math.isinf(float(torch.exp2(torch.tensor(129.0))))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    x[0, 5], x[1, 40], x[2, 17], x[3, :] = np.nan, np.inf, -np.inf, 5000.0
    with np.errstate(all="ignore"):
        for fq, bs, bad in ((lambda v: Q.fake_quant_fp8_block(v, 32), 32, {(0, 0), (1, 1), (2, 0)}),
                            (lambda v: Q.fake_quant_fp4_block(v, 32), 32, {(0, 0), (1, 1), (2, 0)}),
                            (lambda v: Q.fake_quant_fp4_block(v, 16, True), 16,
                             {(0, 0), (1, 2), (2, 1), (3, 0), (3, 1), (3, 2), (3, 3)})):
            y = fq(x)
            clean = fq(np.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0))
            for r in range(6):
                for blk in range(64 // bs):
                    sl = y[r, blk * bs:(blk + 1) * bs]
                    if (r, blk) in bad:
                        assert np.isnan(sl).all(), (r, blk)
                    elif not np.isnan(x[r, blk * bs:(blk + 1) * bs]).any() and np.isfinite(x[r, blk * bs:(blk + 1) * bs]).all():
                        assert np.array_equal(sl, clean[r, blk * bs:(blk + 1) * bs]), (r, blk)


def test_latent_entry_byte_layout_known_answer():
    """The 656 B FP8-b128 entry byte by byte, independently of the pack / unpack pair:
    512 e4m3 codes, four little-endian fp32 block scales at bytes 512..527, 64 bf16 rope
    channels at bytes 528..655 (FlashMLA's V3.2 layout, layers/attn/fp_attn_notes.md)."""
    x = np.zeros((1, 576), np.float32)
    x[0, 0], x[0, 1], x[0, 2], x[0, 3] = 448.0, -1.0, 0.5, 2.0 ** -9      # block 0: scale 1
    x[0, 128] = 224.0                                                       # block 1: scale 1/2
    x[0, 384] = 1000.0                                                      # block 3: scale 4; 250 -> 256
    x[0, 512], x[0, 513], x[0, 575] = 1.0, -2.5, 3.140625                  # rope (bf16-exact)
    e = Q.pack_latent_fp8_b128(x)[0]
    assert e[0] == 0x7E and e[1] == 0xB8 and e[2] == 0x30 and e[3] == 0x01   # 448, -1, 0.5, 2^-9
    assert e[128] == 0x7E and e[384] == 0x78 and not e[4:128].any() and not e[256:384].any()
    scales = [bytes(e[512 + 4 * i:516 + 4 * i]) for i in range(4)]
    assert scales[0] == bytes([0, 0, 0x80, 0x3F])                  # 1.0
    assert scales[1] == bytes([0, 0, 0, 0x3F])                     # 0.5
    assert scales[2] == bytes([0, 0, 0x80, 0x34])                  # 2^-22: the 1e-4 amax floor
    assert scales[3] == bytes([0, 0, 0x80, 0x40])                  # 4.0
    assert bytes(e[528:532]) == bytes([0x80, 0x3F, 0x20, 0xC0])    # 1.0, -2.5
    assert bytes(e[654:656]) == bytes([0x49, 0x40]) and not e[532:654].any()
    # and a hand-written entry reads back as the values its bytes spell
    h = np.zeros(656, np.uint8)
    h[5] = 0x7E                                                     # channel 5: 448 x block-0 scale 1
    h[200] = 0xB8                                                   # channel 200: -1 x block-1 scale
    h[512:516] = [0, 0, 0x80, 0x3F]
    h[516:520] = [0, 0, 0, 0x40]                                    # block 1 scale 2.0
    h[528 + 2 * 7:528 + 2 * 8] = [0x20, 0xC0]                       # rope channel 7 = -2.5
    v = Q.unpack_latent_fp8_b128(h[None])[0]
    assert v[5] == 448.0 and v[200] == -2.0 and v[512 + 7] == -2.5
    assert np.count_nonzero(v) == 3
