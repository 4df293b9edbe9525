"""CPU: the C-ABI library loads and exports every symbol include/mzk.h declares.

No compute call is made (there is no GPU here); only symbol resolution, the version and
the argument checks that fail before any launch.
"""

import ctypes

import pytest

from mzoo_amd import _lib


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    missing = [s for s in _lib.header_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared in include/mzk.h but not exported: {missing}"


def test_every_header_symbol_has_a_python_signature():
    assert set(_lib.header_symbols()) <= set(_lib._SIGS), set(_lib.header_symbols()) - set(_lib._SIGS)


def test_version_and_error_text():
    lib = _lib.load()
    assert lib.mzk_version() >= 100
    # an invalid call fails in the argument check (before any HIP call) and sets the text
    rc = lib.mzk_fake_quant_fp8_block(None, None, 0, 1, 32, 32, None)
    assert rc == -1
    assert b"null pointer" in lib.mzk_last_error()
    rc = lib.mzk_quant_mxfp4(ctypes.c_void_p(8), 0, 1, 33, ctypes.c_void_p(8), ctypes.c_void_p(8), None)
    assert rc == -1 and b"multiple of 32" in lib.mzk_last_error()


def test_missing_library_raises(tmp_path):
    with pytest.raises(ImportError, match="not built"):
        _lib.load(tmp_path / "nope.so")
