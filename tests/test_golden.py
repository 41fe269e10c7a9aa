"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py
from the oracle). CPU: the oracle still reproduces them. GPU: the HIP path
matches them to the parity bars."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import flashprefill_oracle as O
from tests._parity import OUT_MAX_ABS, OUT_MEAN_ABS

HERE = Path(__file__).resolve().parent / "golden"
CASES = ["varlen_bf16_ragged", "native_bf16_b2", "config1_fp32_short"]
NATIVE = {"varlen_bf16_ragged": False, "native_bf16_b2": True, "config1_fp32_short": True}
ALPHA = {"varlen_bf16_ragged": 0.18, "native_bf16_b2": 0.7, "config1_fp32_short": 0.18}


def _load(name):
    z = np.load(HERE / f"{name}.npz")
    is_bf16 = z["q"].dtype == np.int16

    def t(key):
        a = torch.from_numpy(z[key].copy())
        return a.view(torch.bfloat16) if is_bf16 else a

    cu = z["cu"].tolist()
    nseq = len(cu) - 1
    traces = [dict(sel=torch.from_numpy(z[f"sel{b}"]), p=torch.from_numpy(z[f"p{b}"]),
                   m=torch.from_numpy(z[f"m{b}"]), mk=t(f"mk{b}")) for b in range(nseq)]
    return t("q"), t("k"), t("v"), cu, t("out"), traces


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    q, k, v, cu, out, traces = _load(name)
    lens = [cu[b + 1] - cu[b] for b in range(len(cu) - 1)]
    if NATIVE[name]:
        B, S = len(lens), lens[0]
        r = O.flash_prefill(q.view(B, S, *q.shape[1:]), k.view(B, S, *k.shape[1:]),
                            v.view(B, S, *v.shape[1:]), 128, 2, 4, ALPHA[name], 2, 0)
        got = r.out.reshape(q.shape)
    else:
        r = O.flash_prefill_varlen_func(q, k, v, cu, max(lens), ALPHA[name])
        got = r.out
    for tr, gold in zip(r.traces, traces):
        assert torch.equal(tr.sel, gold["sel"])
        assert torch.equal(tr.mk, gold["mk"])
        torch.testing.assert_close(tr.p, gold["p"], rtol=1e-6, atol=0)
        torch.testing.assert_close(tr.m, gold["m"], rtol=1e-6, atol=0)
    torch.testing.assert_close(got.float(), out.float(), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["varlen_bf16_ragged", "native_bf16_b2"])
def test_gpu_matches_golden(name):
    from flashprefill_amd.runtime import FlashPrefillCall
    q, k, v, cu, out, traces = _load(name)
    dev = torch.device("cuda:0")
    lens = [cu[b + 1] - cu[b] for b in range(len(cu) - 1)]
    o = torch.empty_like(q, device=dev)
    call = FlashPrefillCall(q.to(dev), k.to(dev), v.to(dev), o,
                            torch.tensor(cu, dtype=torch.int32, device=dev), max(lens),
                            alpha=ALPHA[name], native_normalize=NATIVE[name])
    call.run()
    torch.cuda.synchronize()
    sels = call.selection_masks()
    flips = sum(int((s != tr["sel"]).sum()) for s, tr in zip(sels, traces))
    cells = sum(int(torch.tril(torch.ones_like(tr["sel"][0])).sum()) * tr["sel"].shape[0]
                for tr in traces)
    print(f"\n  {name}: selection flips vs golden {flips}/{cells}")
    assert flips <= max(2, cells // 500)
    # output against the oracle's attention over the GPU's own selection
    ref = torch.cat([O.sparse_attention(q[cu[b]:cu[b + 1]], k[cu[b]:cu[b + 1]],
                                        v[cu[b]:cu[b + 1]], sels[b])
                     for b in range(len(lens))])
    d = (o.cpu().float() - ref.float()).abs()
    assert d.max().item() <= OUT_MAX_ABS and d.mean().item() <= OUT_MEAN_ABS
    if flips == 0:
        d2 = (o.cpu().float() - out.float()).abs()
        assert d2.max().item() <= OUT_MAX_ABS and d2.mean().item() <= OUT_MEAN_ABS
