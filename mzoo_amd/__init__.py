"""mzoo_amd: MI355X-native (gfx950 HIP) implementation of mzoo's DeepSeek-V4.1-style
sparse-attention inference path, behind the reference's own Python call signatures.

Modules
-------
quant      block FP8 / FP4 quantizers and the packed cache formats (piece 1)
cache      KV compressor, RoPE and the group carry (piece 2)
indexer    lightning-indexer scores and top-k (pieces 3, 4)
csa2_attn  sparse shared-latent MQA (piece 5)
decode     the graph-captured decode step (piece 6)
owlet1     the module drop-ins (DeepseekV41Attention / Compressor / Indexer / CSACache)
_lib       ctypes binding of the C ABI in ``include/mzk.h`` (``_mzk.so``)
build      compiles ``csrc/*.hip`` into ``_mzk.so`` for gfx950
"""

__all__ = ["quant", "cache", "indexer", "csa2_attn", "decode", "owlet1"]
