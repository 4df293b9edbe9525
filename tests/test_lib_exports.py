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


def test_candidate_entry_points_reject_bad_shapes():
    """The level-two entry points fail in their argument checks, before any HIP call."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    args = [p] * 5 + [70000, 1, 64, 128, 4096, 4096, None, 4, p, 2048, 2048, 8, p, 16384, None]
    assert lib.mzk_indexer_candidate_scores_fp8(*args) == -1
    assert b"65535" in lib.mzk_last_error()
    args = [p] * 5 + [4, 1, 64, 128, 4096, 4096, None, 4, p, 2048, 2048, 8, p, 8192, None]
    assert lib.mzk_indexer_candidate_scores_mxfp4(*args) == -1
    assert b"score stride" in lib.mzk_last_error()
    args = [p] * 5 + [4, 1, 64, 128, 4096, 4096, None, 4, p, 100, 2048, 8, p, 16384, None]
    assert lib.mzk_indexer_candidate_scores_fp8(*args) == -1
    assert b"candidate list shape" in lib.mzk_last_error()
    # in place with different strides
    assert lib.mzk_candidate_positions(p, 2, 16, 32, p, 8, 8, 8, p, 16, None) == -1
    assert b"in place" in lib.mzk_last_error()


def test_noalloc_argument_checks():
    """mzk_sparse_mqa_noalloc refuses a call whose merged output has nowhere to go (the
    partials would stay in its private array) and a row count past 2^31 before it sizes the
    scratch -- both before any HIP call."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    common = [p, 4, 1, 128, 576, 1, 512, p, p, 128, 128, 128, None, 0, 0, 1, p, 8192, 8192, p, 2048, 2048, p, 4]
    assert lib.mzk_sparse_mqa_noalloc(*common, None, None, None, None, 0, None) == -1
    assert b"out and lse are required" in lib.mzk_last_error()
    big = [p, 1 << 20, 1 << 12] + common[3:]
    assert lib.mzk_sparse_mqa_noalloc(*big, p, p, None, None, 0, None) == -1
    assert b"too many rows" in lib.mzk_last_error()
