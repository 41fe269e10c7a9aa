"""Write the golden fixtures of this directory from the CPU oracle.

The reference repository ships no golden vectors (it has no tests), so the
fixtures are the oracle's outputs on small seeded inputs; they freeze the
oracle (regression) and give the GPU tests fixed data to compare against
without re-running the oracle. bf16 tensors are stored as their uint16 bit
patterns. Run: python tests/golden/make_golden.py
"""

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import flashprefill_oracle as O  # noqa: E402

CASES = {
    # varlen, bf16, ragged lengths incl. one shorter than a block and one just past it
    "varlen_bf16_ragged": dict(lens=[300, 129, 1, 200], Hq=2, Hkv=1, d=64, dtype="bf16", seed=5,
                               alpha=0.18, native=False, scale=1.5),
    # batched (native normalisation), MHA, bf16, S not a multiple of 128
    "native_bf16_b2": dict(lens=[257, 257], Hq=2, Hkv=2, d=64, dtype="bf16", seed=6, alpha=0.7,
                           native=True, scale=1.5),
    # fp32 plumbing shape of config 1, shortened (CPU oracle only)
    "config1_fp32_short": dict(lens=[384], Hq=2, Hkv=1, d=64, dtype="fp32", seed=0, alpha=0.18,
                               native=True, scale=1.0),
}


def _inputs(c):
    g = torch.Generator().manual_seed(c["seed"])
    T = sum(c["lens"])
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    q = (torch.randn(T, c["Hq"], c["d"], generator=g) * c["scale"]).to(dt)
    k = (torch.randn(T, c["Hkv"], c["d"], generator=g) * c["scale"]).to(dt)
    v = torch.randn(T, c["Hkv"], c["d"], generator=g).to(dt)
    k[:4] *= 4  # sink rows
    cu = np.cumsum([0] + c["lens"]).astype(np.int32)
    return q, k, v, cu


def _store(t):
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def run_case(name, c):
    q, k, v, cu = _inputs(c)
    if c["native"]:
        B = len(c["lens"])
        S = c["lens"][0]
        r = O.flash_prefill(q.view(B, S, *q.shape[1:]), k.view(B, S, *k.shape[1:]),
                            v.view(B, S, *v.shape[1:]), 128, 2, 4, c["alpha"], 2, 0)
        out = r.out.reshape(q.shape)
    else:
        r = O.flash_prefill_varlen_func(q, k, v, cu, max(c["lens"]), c["alpha"])
        out = r.out
    arrays = dict(q=_store(q), k=_store(k), v=_store(v), cu=cu, out=_store(out))
    for b, tr in enumerate(r.traces):
        arrays[f"sel{b}"] = tr.sel.numpy()
        arrays[f"p{b}"] = tr.p.numpy()
        arrays[f"m{b}"] = tr.m.numpy()
        arrays[f"mk{b}"] = _store(tr.mk)
    return arrays


def main():
    for name, c in CASES.items():
        arrays = run_case(name, c)
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, {k: v.shape for k, v in arrays.items() if k in ("q", "out")},
              os.path.getsize(HERE / f"{name}.npz"))


if __name__ == "__main__":
    main()
