"""Build the gfx950 shared library ``libflashprefill.so`` in-tree with hipcc.

All HIP sources under ``csrc/`` are compiled into one shared object that
exports the C ABI declared in ``include/flashprefill.h``. Packed-fp32 VALU
instructions are disabled for the device code (``-packed-fp32-ops``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libflashprefill.so"
LIB_PATH = PKG_DIR / LIB_NAME
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def compile_cmd(out: Path):
    return [
        HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}",
        *sources(), "-o", str(out),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library (always recompiles) and return its path."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_cmd(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    errs = [ln for ln in res.stderr.splitlines()
            if ln and "packed-fp32-ops" not in ln and "warning" not in ln]
    if verbose and errs:
        print("\n".join(errs))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
