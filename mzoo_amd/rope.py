"""RoPE frequencies of the rotary embeddings (host side, computed once per module or
decode layer): the default RoPE and YaRN (``owlet1/norm_rope.py:48-124``,
``owlet1/config.py:419-434``)."""

from __future__ import annotations

import math

import torch


def yarn_inv_freq(theta: float, dim: int, factor: float, original_max_position_embeddings: int,
                  beta_fast: float = 32, beta_slow: float = 1, attention_factor: float | None = None,
                  mscale: float | None = None, mscale_all_dim: float | None = None,
                  truncate: bool = True) -> tuple[torch.Tensor, float]:
    """YaRN's frequencies (Peng et al. 2023, "YaRN: Efficient Context Window Extension of
    Large Language Models", NTK-by-parts), as the reference's rotary embedding obtains them
    (``ROPE_INIT_FUNCTIONS["yarn"]``, norm_rope.py:70-73).  Pair i rotates at
    theta^(-2i/dim); a pair that turns more than ``beta_fast`` times over the original
    context keeps its frequency, one that turns fewer than ``beta_slow`` times is
    interpolated to 1/factor of it, and a linear ramp over the pair index blends the two in
    between -- the ramp's ends are the pair indices where the turn counts equal beta_fast
    and beta_slow, i = dim ln(L / (2 pi n)) / (2 ln theta) for n turns over L positions
    (rounded outward when ``truncate``).  The attention factor that scales cos / sin is the
    paper's 0.1 ln(factor) + 1 unless given (owlet1 gives 1.0).  float32 throughout, in the
    library's operation order, so the tables are the reference's bit for bit.  Returns
    (inv_freq float32 [dim / 2], attention_factor)."""
    def mscale_of(scale, m=1.0):
        return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0

    if attention_factor is None:
        attention_factor = (float(mscale_of(factor, mscale) / mscale_of(factor, mscale_all_dim))
                            if mscale and mscale_all_dim else mscale_of(factor))

    def turn_dim(turns):
        return (dim * math.log(original_max_position_embeddings / (turns * 2 * math.pi))) / (2 * math.log(theta))

    lo, hi = turn_dim(beta_fast), turn_dim(beta_slow)
    if truncate:
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, dim - 1)
    if lo == hi:
        hi += 0.001  # a one-point ramp
    ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - lo) / (hi - lo), 0, 1)
    pos_freqs = theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim)
    keep = 1 - ramp  # the share of the original frequency
    inv = (1.0 / (factor * pos_freqs)) * (1 - keep) + (1.0 / pos_freqs) * keep
    return inv, float(attention_factor)


def rope_inv_freq(theta: float, dim: int, yarn: dict | None = None) -> tuple[torch.Tensor, float]:
    """(inv_freq float32 [dim / 2], cos / sin scale) of the default RoPE
    (``1 / theta^(arange(0, dim, 2) / dim)``, scale 1) or of YaRN (``yarn_inv_freq``)."""
    if yarn is None:
        return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim)), 1.0
    return yarn_inv_freq(theta, dim, **yarn)
