"""Build the in-tree HIP library ``mzoo_amd/_mzk.so`` for gfx950.

Every ``csrc/*.hip`` / ``csrc/*.cpp`` file is compiled with ``hipcc`` into one shared
library.  Flags:

* ``--offload-arch=gfx950``: MI355X only, no other targets.
* ``-ffp-contract=off``: no implicit fused multiply-adds, so the kernels evaluate
  exactly the float32 operation sequence they spell out (fused steps use ``fmaf``).
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: fp32 ``/`` and ``sqrt`` are the
  correctly rounded IEEE operations (the compressor's bit-exact RMSNorm relies on it).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` disables the packed fp32
  instructions (v_pk_*_f32), keeping every float32 op scalar.
* ``-fgpu-flush-denormals-to-zero`` is NOT given: fp32 denormals are kept.

Run ``python -m mzoo_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "_mzk.so"
OBJ = ROOT.parent / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-I", str(ROOT.parent / "include"),
]


# The AddressSanitizer variant (``build(asan=True)``): the host code -- argument checks,
# dispatch, the error text -- instrumented, the device code as in the product.  It loads into
# a process that preloads the sanitizer runtime (tests/test_asan_host.py).
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
ASAN_OUT = OBJ / "asan" / "_mzk_asan.so"


def _compile(src: pathlib.Path, obj_dir: pathlib.Path = OBJ, extra: tuple = ()) -> pathlib.Path:
    obj = obj_dir / (src.name + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *[f for f in COMMON if f not in ("--offload-arch=gfx950",)], *extra, "-x", "c++", "-c",
               str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True, asan: bool = False) -> pathlib.Path:
    out = ASAN_OUT if asan else OUT
    obj_dir = out.parent if asan else OBJ
    obj_dir.mkdir(parents=True, exist_ok=True)
    extra = tuple(ASAN_FLAGS) if asan else ()
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda f: _compile(f, obj_dir, extra), sources))
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *extra, *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources")
    return out


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    OUT.unlink(missing_ok=True)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build(asan="--asan" in sys.argv)
