"""GPU parity of the compressor (piece 2) and RoPE: bit-exact against the CPU oracle.

Both evaluate the same pinned float32 operation sequence (oracle/compressor.py), so every
output bit must match, for fp32 and bf16 models, ratios 1/2/4/128 and the two latent
widths (576 = 512+64, 160 = 128+32).  Also: the group carry across calls
(``store_compression_weights``, owlet1/cache.py:96-113) gives the same latents as one call.
"""

import numpy as np
import pytest
import torch

from mzoo_amd import cache as MC
from oracle import compressor as C

pytestmark = pytest.mark.gpu
NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16"}


def _bits(t):
    t = t.cpu()
    return t.view(torch.int32).numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy()


def _obits(x, dtype):
    return _bits(torch.from_numpy(np.ascontiguousarray(x)).to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ratio,d", [(4, 576), (2, 160), (128, 576), (1, 576), (4, 160)])
def test_compress_bit_exact(dev, dtype, ratio, d):
    gen = torch.Generator().manual_seed(ratio * 1000 + d)
    b, n = 3, 40 if ratio < 128 else 3
    kv = torch.randn(b, n * ratio + 1, d, generator=gen)            # one trailing token left over
    gate = torch.randn(b, n * ratio + 1, d, generator=gen) * 4
    w = (1 + 0.1 * torch.randn(d, generator=gen)).to(dtype)
    got = MC.compress(kv.to(dev), gate.to(dev) if ratio > 1 else None, ratio, w.to(dev), 1e-20, dtype, n_groups=n)
    want = C.compress(kv[:, :n * ratio].numpy(), gate[:, :n * ratio].numpy(), ratio, w.float().numpy(), 1e-20,
                      NAMES[dtype])
    assert np.array_equal(_bits(got), _obits(want, dtype))


def test_compressor_carry_matches_one_shot(dev):
    gen = torch.Generator().manual_seed(9)
    kv = torch.randn(2, 37, 576, generator=gen).to(dev)
    gate = torch.randn(2, 37, 576, generator=gen).to(dev)
    w = torch.ones(576, dtype=torch.bfloat16, device=dev)
    one, first = MC.compressor_forward(kv, gate, 4, w, 1e-20, torch.bfloat16, MC.GroupCarry())
    assert first == 0 and one.shape == (2, 9, 576)
    carry, parts, starts = MC.GroupCarry(), [], []
    for a, z in [(0, 3), (3, 4), (4, 11), (11, 12), (12, 37)]:
        lat, f = MC.compressor_forward(kv[:, a:z], gate[:, a:z], 4, w, 1e-20, torch.bfloat16, carry)
        if lat is not None:
            parts.append(lat)
            starts.append(f)
            carry.emitted(lat.shape[1])
    # tokens 0-3 complete in call 2, 4-7 in call 3, 8-11 in call 4, 12-35 in call 5
    assert starts == [0, 4, 8, 12]
    assert torch.equal(torch.cat(parts, 1), one)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_bit_exact(dev, dtype):
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(2, 9, 4, 576, generator=gen).to(dtype)
    cos, sin = C.rope_tables(np.random.default_rng(0).integers(0, 32768, (2, 9)), 64, 160000.0)
    for inverse in (False, True):
        got = MC.apply_rotary_pos_emb(x.to(dev), torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev),
                                      inverse=inverse)
        want = C.rope(x.float().numpy(), cos[:, :, None], sin[:, :, None], inverse, NAMES[dtype])
        assert np.array_equal(_bits(got), _obits(want, dtype))
