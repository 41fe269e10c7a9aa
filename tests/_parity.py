"""Shared helpers of the GPU parity tests: run the HIP path stage by stage
through the C ABI and compare every intermediate with the CPU oracle."""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from flashprefill_amd.runtime import FlashPrefillCall, attn_key_tile
from oracle import flashprefill_oracle as O

OUT_MAX_ABS = 2e-2   # north-star output tolerance (bf16)
OUT_MEAN_ABS = 2e-3


def ulp_diff_16(a: torch.Tensor, b: torch.Tensor) -> int:
    """Max distance in units of the last place between two bf16/fp16 tensors."""
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotone integer line
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return int((ia - ib).abs().max().item()) if ia.numel() else 0


@dataclass
class StageReport:
    pool_ulp: int = 0
    m_max_rel: float = 0.0
    p_max_rel: float = 0.0
    sel_from_gpu_scores_mismatch: int = 0
    sel_from_oracle_scores_mismatch: int = 0
    e2e_flips: int = 0
    cells: int = 0
    out_max_abs: float = 0.0
    out_mean_abs: float = 0.0
    density: float = 0.0
    notes: List[str] = field(default_factory=list)


def seq_slices(cu: Sequence[int]):
    return [(int(cu[b]), int(cu[b + 1])) for b in range(len(cu) - 1)]


def run_stages(q, k, v, cu_list, max_seq_len, *, alpha, sink=2, window=4, last_n=2,
               native=False, check_oracle_scores=True, attention=True,
               min_budget=0) -> StageReport:
    """Run plan/pool/search(dump)/select/attn on the GPU and compare each stage
    with the oracle. q/k/v are CPU tensors (T, H, d); cu_list python ints."""
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    od = torch.full_like(qd, float("nan"))
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    call = FlashPrefillCall(qd, kd, vd, od, cu, max_seq_len, alpha=alpha, attention_sink=sink,
                            window_size=window, last_n_block=last_n, native_normalize=native,
                            min_budget=min_budget)
    rep = StageReport()
    call.plan()
    call.pool()
    dump_p, dump_m = call.search(dump=True)
    torch.cuda.synchronize()
    assert call.status() == 0
    tile, tri, start, lens = call.seq_tables()
    assert lens == [b - a for a, b in seq_slices(cu_list)]
    mk_gpu = call.pooled_k().cpu()
    gpu_sel = call.selection_masks()
    assert call.ordered_lists_ok()
    gp = call.untri_scores(dump_p)
    gm = call.untri_scores(dump_m)
    oracle_ps, oracle_ms = [], []
    for b, (s0, s1) in enumerate(seq_slices(cu_list)):
        if s1 == s0:
            assert gpu_sel[b].numel() == 0
            oracle_ps.append(torch.zeros(q.shape[1], 0, 0))
            oracle_ms.append(torch.zeros(q.shape[1], 0, 0))
            continue
        mk_o = O.pool_k(k[s0:s1])
        rep.pool_ulp = max(rep.pool_ulp, ulp_diff_16(mk_gpu[tile[b]:tile[b + 1]], mk_o))
        # scores from the GPU's own pooled K (isolates the score kernel)
        p_o, m_o = O.block_score(q[s0:s1], mk_gpu[tile[b]:tile[b + 1]])
        nb = p_o.shape[-1]
        tril = torch.tril(torch.ones(nb, nb, dtype=torch.bool)).expand_as(p_o)
        dm = (gm[b][tril] - m_o[tril]).abs() / m_o[tril].abs().clamp_min(1.0)
        dp = (gp[b][tril] - p_o[tril]).abs() / p_o[tril].abs()
        rep.m_max_rel = max(rep.m_max_rel, dm.max().item())
        rep.p_max_rel = max(rep.p_max_rel, dp.max().item())
        # exact selection from the GPU's fp32 scores
        sel_g = O.select_from_scores(gp[b].nan_to_num(0.0).where(tril, torch.zeros(())),
                                     gm[b].where(tril, torch.tensor(float("-inf"))),
                                     native, alpha, sink, window, last_n, min_budget)
        rep.sel_from_gpu_scores_mismatch += int((sel_g != gpu_sel[b]).sum())
        # end-to-end selection vs the oracle's own scores (tie flips)
        p_e, m_e = O.block_score(q[s0:s1], mk_o)
        sel_e = O.select_from_scores(p_e, m_e, native, alpha, sink, window, last_n, min_budget)
        rep.e2e_flips += int((sel_e != gpu_sel[b]).sum())
        rep.cells += int(tril.sum())
        rep.density += int(gpu_sel[b].sum())
        oracle_ps.append(p_e)
        oracle_ms.append(m_e)
    rep.density = rep.density / max(rep.cells, 1)

    if check_oracle_scores:
        # exact selection on the GPU from the oracle's fp32 scores
        call.select(call.tri_scores(oracle_ps), call.tri_scores(oracle_ms))
        torch.cuda.synchronize()
        sel2 = call.selection_masks()
        for b, (s0, s1) in enumerate(seq_slices(cu_list)):
            if s1 == s0:
                continue
            want = O.select_from_scores(oracle_ps[b], oracle_ms[b], native, alpha, sink, window,
                                        last_n, min_budget)
            rep.sel_from_oracle_scores_mismatch += int((sel2[b] != want).sum())
        # restore the GPU's own selection for the attention stage
        call.search()

    if attention:
        call.attn()
        torch.cuda.synchronize()
        out = od.cpu()
        diffs = []
        for b, (s0, s1) in enumerate(seq_slices(cu_list)):
            if s1 == s0:
                continue
            ref = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], gpu_sel[b],
                                     k_tile=attn_key_tile())
            diffs.append((out[s0:s1].float() - ref.float()).abs().reshape(-1))
        d = torch.cat(diffs)
        assert not torch.isnan(d).any(), "NaN in GPU output"
        rep.out_max_abs = d.max().item()
        rep.out_mean_abs = d.mean().item()
    return rep
