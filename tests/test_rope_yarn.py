"""YaRN on the compress RoPE (owlet1/config.py:419-434, norm_rope.py:48-124), CPU only.

``mzoo_amd.rope.yarn_inv_freq`` restates the YaRN frequency blend; the reference takes it
from transformers' ``ROPE_INIT_FUNCTIONS["yarn"]`` (installed here: the library routine the
reference calls), which pins it bit for bit over the parameter variants the routine reads.
The closed forms YaRN reduces to are checked too: factor 1 is the default RoPE, the pairs
below the ramp keep their frequency, the pairs above it are divided by the factor.  The
module drop-in's rotary embedding and the decode layer's position table built with YaRN
settings equal the tables of the oracle, which calls the library.
"""

import math
import types

import numpy as np
import pytest
import torch

from mzoo_amd import owlet1 as MO
from mzoo_amd.decode import rope_table
from mzoo_amd.rope import rope_inv_freq, yarn_inv_freq
from oracle import model as OM

THETA, RD = 160000.0, 64
VARIANTS = [
    dict(factor=16.0, original_max_position_embeddings=65536, attention_factor=1.0),
    dict(factor=40.0, original_max_position_embeddings=4096, beta_fast=16, beta_slow=2, attention_factor=1.0),
    dict(factor=8.0, original_max_position_embeddings=8192, attention_factor=None),
    dict(factor=32.0, original_max_position_embeddings=16384, attention_factor=None, mscale=1.0, mscale_all_dim=0.5),
    dict(factor=4.0, original_max_position_embeddings=32768, attention_factor=1.0, truncate=False),
]


def _library(yarn, rd=RD, theta=THETA):
    return OM._yarn_library(theta, rd, yarn)


@pytest.mark.parametrize("yarn", VARIANTS)
def test_yarn_inv_freq_equals_library(yarn):
    inv, scale = yarn_inv_freq(THETA, RD, **yarn)
    ref_inv, ref_scale = _library(yarn)
    assert inv.dtype == torch.float32 and torch.equal(inv, ref_inv)
    assert scale == ref_scale


def test_yarn_closed_forms():
    base, _ = rope_inv_freq(THETA, RD)
    # factor 1: interpolation and extrapolation coincide -- the default RoPE
    inv1, s1 = yarn_inv_freq(THETA, RD, factor=1.0, original_max_position_embeddings=65536)
    assert torch.equal(inv1, base) and s1 == 1.0
    # the ramp's ends: the pair index where the turn count over the original context is
    # beta_fast (below it: the frequency is kept) and beta_slow (above it: divided by factor)
    L, f = 65536, 16.0
    inv, _ = yarn_inv_freq(THETA, RD, factor=f, original_max_position_embeddings=L, attention_factor=1.0)
    turn = lambda n: RD * math.log(L / (n * 2 * math.pi)) / (2 * math.log(THETA))  # noqa: E731
    lo, hi = math.floor(turn(32)), math.ceil(turn(1))
    assert 0 < lo < hi < RD // 2
    assert torch.equal(inv[:lo + 1], base[:lo + 1])
    torch.testing.assert_close(inv[hi:], base[hi:] / f, rtol=1e-6, atol=0)
    between = inv[lo + 1:hi]
    assert ((between < base[lo + 1:hi]) & (between > base[lo + 1:hi] / f)).all()
    # the paper's attention factor when none is given
    _, s = yarn_inv_freq(THETA, RD, factor=f, original_max_position_embeddings=L)
    assert s == pytest.approx(0.1 * math.log(f) + 1.0)


def _yarn_config(yarn):
    """A config carrying the reference's post-init rope_parameters layout (main: default,
    compress: YaRN) -- what owlet1/config.py:419-434 builds from a flat rope_scaling."""
    partial = RD / 512
    compress = {k: v for k, v in yarn.items() if k != "truncate"}
    compress.update(rope_type="yarn", rope_theta=THETA, partial_rotary_factor=partial)
    rp = {"main": {"rope_type": "default", "rope_theta": 10000.0, "partial_rotary_factor": partial}, "compress": compress}
    if "truncate" in yarn:
        rp["truncate"] = yarn["truncate"]
    return types.SimpleNamespace(head_dim=512, qk_rope_head_dim=RD, rope_theta=10000.0, compress_rope_theta=THETA,
                                 rope_parameters=rp, max_position_embeddings=1 << 20)


@pytest.mark.parametrize("yarn", VARIANTS)
def test_rotary_embedding_with_yarn_equals_oracle(yarn):
    rot = MO.DeepseekV41RotaryEmbedding(_yarn_config(yarn))
    pos = torch.tensor([[0, 1, 7, 4095, 65535, 200000]])
    x = torch.zeros(1, dtype=torch.float32)
    cos, sin = rot(x, pos, "compress")
    rc, rs = OM.rope_tables(pos.numpy(), RD, THETA, yarn)
    assert np.array_equal(cos.numpy(), rc) and np.array_equal(sin.numpy(), rs)
    # the main rope stays the default one
    mc, ms = rot(x, pos, "main")
    dc, ds = OM.rope_tables(pos.numpy(), RD, 10000.0)
    assert np.array_equal(mc.numpy(), dc) and np.array_equal(ms.numpy(), ds)


def test_decode_position_table_with_yarn():
    yarn = VARIANTS[0]
    tab = rope_table(4096, RD, THETA, yarn)
    rc, rs = OM.rope_tables(np.arange(4096)[None], RD, THETA, yarn)
    want = torch.cat([torch.from_numpy(rc[0]), torch.from_numpy(rs[0])], -1).to(torch.bfloat16)
    assert torch.equal(tab, want)


def test_unknown_rope_type_is_rejected():
    cfg = _yarn_config(VARIANTS[0])
    cfg.rope_parameters["compress"]["rope_type"] = "longrope"
    with pytest.raises(NotImplementedError, match="longrope"):
        MO.DeepseekV41RotaryEmbedding(cfg)
