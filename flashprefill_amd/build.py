"""Build the gfx950 shared library ``libflashprefill.so`` in-tree with hipcc.

Every HIP source under ``csrc/`` is compiled to its own object (in parallel,
under ``_build/``) and the objects are linked into one shared object that
exports the C ABI declared in ``include/flashprefill.h``. Packed-fp32 VALU
instructions are disabled for the device code (``-packed-fp32-ops``).

Per-file code-generation options, if a source needs any, go in ``FILE_FLAGS``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libflashprefill.so"
LIB_PATH = PKG_DIR / LIB_NAME
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
BUILD_DIR = PKG_DIR / "_build"
FILE_FLAGS: dict = {}


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def compile_cmd(src: str, out: Path):
    return [
        HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-c",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}",
        *FILE_FLAGS.get(Path(src).name, []), src, "-o", str(out),
    ]


def link_cmd(objs, out: Path):
    return [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(out)]


def _run(cmd, verbose: bool):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = [ln for ln in res.stderr.splitlines()
            if ln and "packed-fp32-ops" not in ln and "warning" not in ln]
    return res, errs


def build(verbose: bool = False) -> Path:
    """Compile the library (always recompiles) and return its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [BUILD_DIR / (Path(s).stem + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(os.cpu_count() or 1, 8)))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda so: _run(compile_cmd(*so), verbose), zip(srcs, objs)))
    for (res, errs), src in zip(results, srcs):
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed on {src} with exit code {res.returncode}")
        if verbose and errs:
            print("\n".join(errs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    res, errs = _run(link_cmd(objs, tmp), verbose)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc link failed with exit code {res.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
