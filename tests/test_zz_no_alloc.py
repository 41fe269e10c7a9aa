"""The allocation-free entry point fp_flashprefill_noalloc, called through the
C ABI: its output must equal fp_flashprefill's (same kernels, bit for bit) on
two calls in a row, the second with a smaller problem (the static scratch
keeps the first call's contents, which the second must not depend on), and a
problem larger than the static scratch is rejected before any launch."""

import ctypes

import pytest
import torch

from flashprefill_amd import _lib
from flashprefill_amd.runtime import FlashPrefillCall

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(lens, Hq, Hkv, d, seed):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = (torch.randn(T, Hq, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(T, Hkv, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    v = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    cu = [0]
    for s in lens:
        cu.append(cu[-1] + s)
    return q, k, v, torch.tensor(cu, dtype=torch.int32, device=DEV)


def _noalloc(call, o):
    """fp_flashprefill_noalloc on the descriptor of ``call`` with output ``o``."""
    P = _lib.FpProblem()
    ctypes.pointer(P)[0] = call.P
    P.o = o.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.load().fp_flashprefill_noalloc(ctypes.byref(P), stream))


def test_noalloc_matches_workspace_entry_point_on_two_calls():
    cases = [([4096, 1000, 77], 8, 2, 128, 0.18, 1), ([300, 129], 4, 1, 64, 0.12, 2)]
    for lens, Hq, Hkv, d, alpha, seed in cases:
        print(f"\n  noalloc case lens={lens} Hq={Hq} Hkv={Hkv} d={d}", flush=True)
        q, k, v, cu = _inputs(lens, Hq, Hkv, d, seed)
        o_ws = torch.full_like(q, float("nan"))
        call = FlashPrefillCall(q, k, v, o_ws, cu, max(lens), alpha=alpha)
        assert call.layout.total_bytes <= _lib.NOALLOC_SCRATCH_BYTES
        call.run()
        o_na = torch.full_like(q, float("nan"))
        _noalloc(call, o_na)
        torch.cuda.synchronize()
        assert call.status() == 0
        assert not torch.isnan(o_na).any(), "unwritten output rows"
        assert torch.equal(o_na, o_ws), "allocation-free output differs from fp_flashprefill's"


def test_noalloc_rejects_problems_beyond_the_scratch():
    # 128K tokens with 64 query heads needs ~140 MB of index lists
    T = 131072
    q = torch.empty(T, 64, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    call = FlashPrefillCall(q, k, k, q, cu, T, alpha=0.18)
    assert call.layout.total_bytes > _lib.NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="static scratch"):
        _noalloc(call, q)
