"""CPU: the library's host code under AddressSanitizer.

``python -m mzoo_amd.build --asan`` builds the library with the host code -- argument checks,
dispatch, the error text -- instrumented (``-Xarch_host -fsanitize=address``; the device code
is the product's).  This test builds it when it is missing or older than the sources, then,
in a child process that preloads the sanitizer runtime and points ``MZOO_AMD_LIB`` at it,
runs the C-ABI tests and calls every entry point the header declares with sizes every
argument check refuses (negative counts, null buffers): each must fail with an error text,
and the sanitizer must report nothing.  No GPU is touched.
"""

import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CLANG = pathlib.Path("/opt/rocm/lib/llvm/bin/clang")

CHILD = r"""
import ctypes, sys
from mzoo_amd import _lib
lib = _lib.load()
assert "asan" in str(_lib.LIB_PATH), _lib.LIB_PATH
maps = open("/proc/self/maps").read()
assert "libclang_rt.asan" in maps, "the sanitizer runtime is not loaded"
assert hasattr(lib, "__asan_report_load8") or "__asan" in open(_lib.LIB_PATH, "rb").read().decode("latin-1")
skip = {"mzk_version", "mzk_last_error", "mzk_sparse_mqa_set_merge"}
calls = failed = 0
for name, sig in _lib._SIGS.items():
    if name in skip:
        continue
    args = []
    for a in sig:
        if a in (_lib._I32, _lib._I64):
            args.append(-3)
        elif a is _lib._F32:
            args.append(0.0)
        else:
            args.append(None)
    rc = getattr(lib, name)(*args)
    calls += 1
    msg = lib.mzk_last_error()
    if rc != 0:
        failed += 1
        assert isinstance(msg, bytes) and len(msg) > 0, name
print(f"asan child: {calls} entry points called, {failed} refused", flush=True)
assert failed == calls, f"{calls - failed} entry points accepted negative sizes"
"""


def _runtime():
    if not CLANG.exists():
        return None
    p = subprocess.run([str(CLANG), "--print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = pathlib.Path(p.stdout.strip())
    return path if path.is_absolute() and path.exists() else None


def _asan_lib():
    sys.path.insert(0, str(ROOT))
    from mzoo_amd import build as B
    srcs = list(B.CSRC.glob("*.hip")) + list(B.CSRC.glob("*.cpp")) + list(B.CSRC.glob("*.h")) + [ROOT / "include" / "mzk.h"]
    newest = max(f.stat().st_mtime for f in srcs)
    if not B.ASAN_OUT.exists() or B.ASAN_OUT.stat().st_mtime < newest:
        B.build(verbose=False, asan=True)
    return B.ASAN_OUT


def test_host_code_under_address_sanitizer():
    rt = _runtime()
    if rt is None:
        pytest.skip("no AddressSanitizer runtime in this toolchain")
    lib = _asan_lib()
    env = dict(os.environ, LD_PRELOAD=str(rt), MZOO_AMD_LIB=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0")
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                          str(ROOT / "tests" / "test_lib_exports.py")], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0 and "AddressSanitizer" not in out, out[-4000:]
    res = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0 and "AddressSanitizer" not in out, out[-4000:]
    assert "entry points called" in out
