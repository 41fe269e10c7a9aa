"""Code-generation guard for the attention kernel's block loop (CPU: hipcc
cross-compiles fp_attn.hip to gfx950 assembly; no GPU needed).

The S and P.V loops issue their LDS operand reads four MFMAs ahead of use
(sched_group_barrier order); each MFMA then waits for its own operands only:
`s_waitcnt lgkmcnt(3)` in the S loop (one K read per MFMA, three later ones
still in flight) and `s_waitcnt lgkmcnt(6)` in the P.V loop (two V^T reads
per MFMA) instead of lgkmcnt(0). That schedule is fragile: unrelated code in
the same kernel has made the compiler drop it in the persistent kernel with
no change in register counts (a loop over the split-row chunks in the merge:
P.V loop, 8 % more attention time at 128K; a scalar load left in flight
across the block: S loop, 7 %). This test fails when either loop loses the
read-ahead in the 16-bit kernels at d = 128."""

import os
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(shutil.which(HIPCC) is None and not Path(HIPCC).exists(),
                    reason="hipcc not available")
def test_attention_block_loop_keeps_lds_read_ahead():
    src = ROOT / "flashprefill_amd" / "csrc" / "fp_attn.hip"
    with tempfile.TemporaryDirectory() as td:
        out = Path(td) / "fp_attn.s"
        cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "--offload-device-only", "-S",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               f"-I{ROOT / 'include'}", f"-I{src.parent}", str(src), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stderr[-2000:]
        asm = out.read_text()
    checked = 0
    for name in re.findall(r"^(_ZN2fp6k_attnI\S+):", asm, re.M):
        # 16-bit inputs, d = 128, block 128 and 64, both grid forms
        if "Li128ELi128E" not in name and "Li128ELi64E" not in name:
            continue
        i = asm.index(name + ":")
        body = asm[i:asm.index(".Lfunc_end", i)]
        # per block size: the plain block's 32 (16) MFMAs per loop
        pv, sl = body.count("lgkmcnt(6)"), body.count("lgkmcnt(3)")
        want_pv, want_s = (20, 24) if "Li128ELi128E" in name else (8, 10)
        assert pv >= want_pv, f"{name}: {pv} P.V read-ahead waits (want >= {want_pv})"
        assert sl >= want_s, f"{name}: {sl} S read-ahead waits (want >= {want_s})"
        checked += 1
    assert checked == 8
