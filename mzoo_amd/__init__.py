"""mzoo_amd: MI355X-native (gfx950 HIP) implementation of mzoo's DeepSeek-V4.1-style
sparse-attention inference path, behind the reference's own Python call signatures.

Modules
-------
quant      block FP8 / FP4 quantizers and the packed cache formats (piece 1)
_lib       ctypes binding of the C ABI in ``include/mzk.h`` (``_mzk.so``)
build      compiles ``csrc/*.hip`` into ``_mzk.so`` for gfx950
"""

__all__ = ["quant"]
