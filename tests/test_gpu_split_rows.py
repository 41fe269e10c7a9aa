"""Parity of the split-row path: the last_n rows of a sequence select every
causal block, and rows longer than the host's chunk size run as chunk
workgroups whose fp32 partials are merged (by the row's last chunk inside the
attention kernel when Hq is a multiple of 8, else by k_merge). Ragged batches
with several split sequences (bf16 / block 128 and fp16 / d 64 / block 64,
last_n above 2) go through every stage against the oracle, the full attention
output included, after checking that the plan emitted the expected chunk
units. Few heads over a long sequence (a tensor-parallel shard) make the
chunks short and many (8 per dense row, the most, merged by k_merge and
inside the kernel); those cases check sampled rows against the oracle and
every row against the closed form."""

import pytest
import torch

from tests._parity import OUT_MAX_ABS, OUT_MEAN_ABS, run_stages
from flashprefill_amd.runtime import FlashPrefillCall

pytestmark = pytest.mark.gpu


def _inputs(lens, Hq, Hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = (torch.randn(T, Hq, d, generator=g) * 1.5).to(dtype)
    k = (torch.randn(T, Hkv, d, generator=g) * 1.5).to(dtype)
    v = torch.randn(T, Hkv, d, generator=g).to(dtype)
    cu = [0]
    for s in lens:
        cu.append(cu[-1] + s)
    return q, k, v, cu


def _expected_units(lens, block, last_n, C):
    n = 0
    for L in lens:
        nb = -(-L // block)
        for i in range(max(nb - last_n, 0), nb):
            if i + 1 > C:
                n += -(-(i + 1) // C)
    return n


def _planned_units(q, k, v, cu, block, last_n):
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cud = torch.tensor(cu, dtype=torch.int32, device=dev)
    lens = [b - a for a, b in zip(cu, cu[1:])]
    call = FlashPrefillCall(qd, kd, vd, torch.empty_like(qd), cud, max(lens), alpha=0.18,
                            last_n_block=last_n, block_size=block)
    call.plan()
    torch.cuda.synchronize()
    L = call.layout
    return L.split_blocks, L.unit_cap, int(call._view(L.units_off, torch.int32, 1)[0])


@pytest.mark.parametrize("lens,Hq,Hkv,d,dtype,block,last_n,seed", [
    ([2048, 1500, 3000, 200, 1100], 8, 2, 128, torch.bfloat16, 128, 3, 11),
    ([4096, 2000, 70], 4, 1, 64, torch.float16, 64, 2, 12),
])
def test_split_rows_match_oracle(lens, Hq, Hkv, d, dtype, block, last_n, seed):
    q, k, v, cu = _inputs(lens, Hq, Hkv, d, dtype, seed)
    C, cap, n = _planned_units(q, k, v, cu, block, last_n)
    want = _expected_units(lens, block, last_n, C)
    print(f"\n  lens={lens} block={block} last_n={last_n}: chunk size {C} blocks, "
          f"{n} units planned (capacity {cap})", flush=True)
    assert C > 0 and n == want > 0 and n <= cap
    rep = run_stages(q, k, v, cu, max(lens), alpha=0.18, last_n=last_n, block=block)
    print(f"  e2e_flips={rep.e2e_flips}/{rep.cells} out_max={rep.out_max_abs:.2e} "
          f"out_mean={rep.out_mean_abs:.2e}", flush=True)
    assert rep.sel_from_gpu_scores_mismatch == 0
    assert rep.sel_from_oracle_scores_mismatch == 0
    assert rep.e2e_flips <= max(2, 2e-3 * rep.cells)
    assert rep.out_max_abs <= OUT_MAX_ABS
    assert rep.out_mean_abs <= OUT_MEAN_ABS


@pytest.mark.parametrize("S,Hq,Hkv,want_chunks,seed", [
    (32768, 4, 1, 8, 13),    # Hq % 8 != 0: k_merge combines 8 partials per row
    (16384, 8, 2, 8, 14),    # Hq % 8 == 0: the row's last chunk merges 8 partials
])
def test_many_chunks_per_row(S, Hq, Hkv, want_chunks, seed):
    q, k, v, cu = _inputs([S], Hq, Hkv, 128, torch.bfloat16, seed)
    C, cap, n = _planned_units(q, k, v, cu, 128, 2)
    nb = S // 128
    print(f"\n  S={S} Hq={Hq}: chunk size {C} blocks, {n} units planned", flush=True)
    assert -(-nb // C) == want_chunks and n == _expected_units([S], 128, 2, C) <= cap
    rows = {0: [(0, nb - 1), (Hq - 1, nb - 2), (Hq // 2, nb // 2), (1, 3)]}
    rep = run_stages(q, k, v, cu, S, alpha=0.18, last_n=2, attn_rows=rows)
    print(f"  e2e_flips={rep.e2e_flips}/{rep.cells} out_max={rep.out_max_abs:.2e} "
          f"out_mean={rep.out_mean_abs:.2e} rows checked={rep.full_rows}", flush=True)
    assert rep.full_rows > 0
    assert rep.sel_from_gpu_scores_mismatch == 0
    assert rep.sel_from_oracle_scores_mismatch == 0
    assert rep.e2e_flips <= max(2, 2e-3 * rep.cells)
    assert rep.out_max_abs <= OUT_MAX_ABS
    assert rep.out_mean_abs <= OUT_MEAN_ABS
