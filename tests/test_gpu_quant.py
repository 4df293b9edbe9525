"""GPU parity of the quantizer kernels (piece 1) against the CPU oracle: bit-exact.

Bit patterns are compared (so -0.0 vs +0.0 counts), for every dtype the reference's
helpers accept and the block sizes the model uses (16 e4m3-scaled compressed KV, 32
indexer/window, 128 the FP8-b128 caches), on inputs spanning many binades plus the
special values (zeros of both signs, e2m1 ties, subnormal-fp8 magnitudes).
"""

import numpy as np
import pytest
import torch

from mzoo_amd import quant as MQ
from oracle import quant as Q

pytestmark = pytest.mark.gpu
DTYPES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _inputs(rows, n, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n, generator=g) * torch.exp(torch.empty(rows, 1).uniform_(-6, 6, generator=g))
    x[0, :8] = torch.tensor([0.0, -0.0, 0.25, -0.75, 1.25, 5.0, 1e-7, -3e-6])
    if dtype == torch.float16:
        x = x.clamp(-6e4, 6e4)
    return x.to(dtype)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy()
    return t.view(torch.int16).numpy()


def _oracle_bits(y32: np.ndarray, dtype) -> np.ndarray:
    return _bits(torch.from_numpy(np.ascontiguousarray(y32)).to(dtype))


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("bs", [16, 32, 128])
def test_fake_quant_fp8_bit_exact(dev, dtype, bs):
    x = _inputs(257, 512, bs, dtype)
    got = MQ._fake_quant_fp8_block(x.to(dev), bs)
    assert got.dtype == dtype and got.shape == x.shape
    want = Q.fake_quant_fp8_block(x.float().numpy(), bs, dtype=DTYPES[dtype])
    assert np.array_equal(_bits(got), _oracle_bits(want, dtype))


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("bs,e4m3", [(16, True), (32, False), (16, False), (32, True)])
def test_fake_quant_fp4_bit_exact(dev, dtype, bs, e4m3):
    x = _inputs(129, 576, 100 + bs, dtype)
    got = MQ._fake_quant_fp4_block(x.to(dev), bs, e4m3_scales=e4m3)
    want = Q.fake_quant_fp4_block(x.float().numpy(), bs, e4m3, dtype=DTYPES[dtype])
    assert np.array_equal(_bits(got), _oracle_bits(want, dtype))


def test_pass_through_and_shapes(dev):
    x = torch.randn(2, 3, 100, device=dev, dtype=torch.bfloat16)
    assert MQ._fake_quant_fp8_block(x, 32) is x
    assert MQ._fake_quant_fp4_block(x, 32) is x
    y = torch.randn(2, 3, 4, 96, device=dev)   # 4-D, block 96 exercises the serial kernel
    got = MQ._fake_quant_fp8_block(y, 96)
    want = Q.fake_quant_fp8_block(y.cpu().numpy(), 96)
    assert np.array_equal(_bits(got), want.view(np.int32))


def test_packed_fp8_and_mxfp4_bit_exact(dev):
    x = _inputs(300, 128, 5, torch.bfloat16)
    codes, scales = MQ.quant_fp8_block(x.to(dev), 128)
    c_ref, s_ref = Q.fp8_block_codes(x.float().numpy(), 128)
    assert np.array_equal(codes.cpu().numpy(), c_ref)
    assert np.array_equal(scales.cpu().numpy().view(np.int32), s_ref.view(np.int32))
    back = MQ.dequant_fp8_block(codes, scales, 128)
    assert np.array_equal(_bits(back), Q.fake_quant_fp8_block(x.float().numpy(), 128).view(np.int32))
    packed, e8 = MQ.quant_mxfp4(x.to(dev))
    p_ref, e_ref = Q.quant_mxfp4(x.float().numpy())
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(e8.cpu().numpy(), e_ref)
    back = MQ.dequant_mxfp4(packed, e8)
    assert np.array_equal(_bits(back), Q.fake_quant_fp4_block(x.float().numpy(), 32).view(np.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_latent_entry_pack_bit_exact(dev, dtype):
    x = _inputs(513, 576, 9, dtype)
    e = MQ.pack_latent_fp8_b128(x.to(dev))
    assert e.shape == (513, 656)
    assert np.array_equal(e.cpu().numpy(), Q.pack_latent_fp8_b128(x.float().numpy()))
    back = MQ.unpack_latent_fp8_b128(e, dtype=torch.float32)
    assert np.array_equal(_bits(back), Q.unpack_latent_fp8_b128(e.cpu().numpy()).view(np.int32))
    # scatter into cache slots
    cache = torch.zeros(1000, 656, dtype=torch.uint8, device=dev)
    dst = torch.randperm(1000)[:513].to(dev)
    MQ.pack_latent_fp8_b128(x.to(dev), out=cache, dst_index=dst)
    assert torch.equal(cache[dst], e)


def test_small_model_dims(dev):
    """Config-1 latent: 128 nope + 32 rope (D=160)."""
    x = _inputs(64, 160, 11, torch.float32)
    e = MQ.pack_latent_fp8_b128(x.to(dev), rope=32)
    assert e.shape == (64, 128 + 4 + 64)
    assert np.array_equal(e.cpu().numpy(), Q.pack_latent_fp8_b128(x.numpy(), nope=128))


def test_unpack_bf16_all_codes_and_scales(dev):
    """The bf16 unpack runs the hardware e4m3 -> bf16 conversion the attention kernel
    dequantizes with: every code (0..255) under scales 2^-40 .. 2^20 must decode to the
    oracle's value exactly (NaN codes to NaN)."""
    rows = 16
    rng = np.random.default_rng(0)
    e = np.zeros((rows, 656), np.uint8)
    for r in range(rows):
        e[r, :512] = (np.arange(512) + 37 * r) % 256
        sc = np.array([2.0 ** (-40 + 4 * r), 2.0 ** -7, 1.0, 2.0 ** (r % 21)], np.float32)
        e[r, 512:528] = sc.view(np.uint8)
        e[r, 528:] = Q.bf16_bits(rng.standard_normal(64).astype(np.float32)).view(np.uint8)
    got = MQ.unpack_latent_fp8_b128(torch.from_numpy(e).to(dev), dtype=torch.bfloat16).cpu()
    want = torch.from_numpy(Q.unpack_latent_fp8_b128(e)).bfloat16()
    gnan, wnan = torch.isnan(got.float()), torch.isnan(want.float())
    assert torch.equal(gnan, wnan)
    assert torch.equal(got[~gnan].view(torch.int16), want[~wnan].view(torch.int16))


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_decode_prologue_bit_exact(dev, fmt):
    """mzk_decode_prologue = the window-ring write of each row's new token (slot
    positions[b] % W of row b) + the indexer-query quantization, bit-exact against the
    oracle's packer and block quantizers."""
    from mzoo_amd import _lib
    b, w, hi, di = 5, 16, 8, 128
    kv = _inputs(b, 576, 21, torch.bfloat16)
    q = _inputs(b * hi, di, 22, torch.bfloat16)
    pos = torch.tensor([0, 15, 16, 1000, 31], dtype=torch.int64)
    win = torch.zeros(b, w, 656, dtype=torch.uint8, device=dev)
    if fmt == "fp8":
        codes = torch.empty(b * hi, di, dtype=torch.uint8, device=dev)
        scales = torch.empty(b * hi, 1, dtype=torch.float32, device=dev)
        e8 = None
    else:
        codes = torch.empty(b * hi, di // 2, dtype=torch.uint8, device=dev)
        scales = None
        e8 = torch.empty(b * hi, di // 32, dtype=torch.uint8, device=dev)
    kvd, qd, posd = kv.to(dev), q.to(dev), pos.to(dev)
    _lib.call("mzk_decode_prologue", kvd.data_ptr(), 1, b, 512, 64, posd.data_ptr(), win.data_ptr(), w, w,
              qd.data_ptr(), 1, b * hi, di, 0 if fmt == "fp8" else 1, codes.data_ptr(), _lib.ptr(scales),
              _lib.ptr(e8), torch.cuda.current_stream().cuda_stream)
    want = Q.pack_latent_fp8_b128(kv.float().numpy())
    wc = win.cpu().numpy()
    for r in range(b):
        assert np.array_equal(wc[r, int(pos[r]) % w], want[r])
    if fmt == "fp8":
        c_ref, s_ref = Q.fp8_block_codes(q.float().numpy(), 128)
        assert np.array_equal(codes.cpu().numpy(), c_ref)
        assert np.array_equal(scales.cpu().numpy().reshape(s_ref.shape).view(np.int32), s_ref.view(np.int32))
    else:
        p_ref, e_ref = Q.quant_mxfp4(q.float().numpy())
        assert np.array_equal(codes.cpu().numpy(), p_ref)
        assert np.array_equal(e8.cpu().numpy(), e_ref)


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
@pytest.mark.parametrize("d", [512, 576])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_pack_cache_v41_bit_exact(dev, fmt, d, dtype):
    """V4.1 cache entries (FlashMLA kv_cache_format): the packed bytes equal the oracle's,
    the unpacked values equal the reference quantizer's, and dst_index scatters rows."""
    from mzoo_amd import quant as MQ
    gen = torch.Generator().manual_seed(d + (7 if fmt == "fp4" else 0))
    # rows spread over about 2^-9 .. 2^9 in scale; values stay below 6 * 448, the largest
    # amax an e4m3 fp4 scale represents (a larger one makes the reference's scale NaN)
    x = (torch.randn(37, d, generator=gen).clamp(-4, 4) * torch.exp(torch.randn(37, 1, generator=gen).clamp(-4, 4) * 1.5))
    x = x.to(dtype)
    x[0, :32] = 0
    x[1, 5] = 2000.0 if dtype != torch.float16 else 1000.0
    xf = x.float().numpy()
    got = MQ.pack_cache_v41(x.to(dev), fmt)
    assert np.array_equal(got.cpu().numpy(), Q.pack_cache_v41(xf, fmt))
    back = MQ.unpack_cache_v41(got, d, fmt).cpu().numpy()
    ref = Q.fake_quant_fp8_block(xf, 32) if fmt == "fp8" else Q.fake_quant_fp4_block(xf, 16, e4m3_scales=True)
    assert np.array_equal(back, ref)
    # scattered into a cache of 64 entries
    cache = torch.zeros(64, MQ.v41_entry_bytes(d, fmt), dtype=torch.uint8, device=dev)
    dst = torch.randperm(64, generator=gen)[:37]
    MQ.pack_cache_v41(x.to(dev), fmt, out=cache, dst_index=dst)
    assert torch.equal(cache[dst.to(dev)], got)
