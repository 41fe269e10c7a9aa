"""Shared helpers of the GPU parity tests: run the HIP path stage by stage
through the C ABI and compare every intermediate with the CPU oracle."""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from flashprefill_amd.runtime import FlashPrefillCall
from oracle import flashprefill_oracle as O

OUT_MAX_ABS = 2e-2   # north-star output tolerance (bf16)
OUT_MEAN_ABS = 2e-3


OUT_MAX_ABS_F32 = 1e-4  # fp32 inputs: fp32 MFMA against the oracle's exact-then-rounded dots
OUT_MEAN_ABS_F32 = 1e-5


def ulp_diff_16(a: torch.Tensor, b: torch.Tensor) -> int:
    """Max distance in units of the last place between two bf16 / fp16 (or
    two fp32) tensors."""
    if a.dtype == torch.float32:
        ia = a.contiguous().view(torch.int32).to(torch.int64)
        ib = b.contiguous().view(torch.int32).to(torch.int64)
        ia = torch.where(ia < 0, -(2 ** 31) - ia, ia)
        ib = torch.where(ib < 0, -(2 ** 31) - ib, ib)
        return int((ia - ib).abs().max().item()) if ia.numel() else 0
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotone integer line
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return int((ia - ib).abs().max().item()) if ia.numel() else 0


@dataclass
class StageReport:
    pool_ulp: int = 0               # over the well-conditioned elements (see pool_errors)
    pool_bound_violations: int = 0  # elements outside the fp32 summation bound
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


def pool_errors(mk_gpu: torch.Tensor, mk_o: torch.Tensor, k_seq: torch.Tensor, block: int):
    """Pooled K of the GPU against the oracle's (fp64 sum, one rounding).

    The GPU sums a block's rows in fp32 (16-bit inputs) and rounds the mean
    once, so |gpu - oracle| <= ulp(max(|gpu|, |oracle|)) + 128 * 2^-24 *
    mean|k| (the fp32 summation bound, mean|k| over the block's rows of that
    column). Where the mean does not cancel (|oracle| >= 2^-8 mean|k|) that is
    within 1.5 ulp, and the ulp distance itself is reported; near
    cancellation the ulp distance is meaningless (values on either side of
    zero are thousands of ulps apart) and only the bound is checked.
    Returns (max ulp distance over the well-conditioned elements, number of
    elements outside the bound, the worst element as text)."""
    nb, hh, d = mk_o.shape
    S = k_seq.shape[0]
    kp = torch.zeros(nb * block, hh, d, dtype=torch.float64)
    kp[:S] = k_seq.double().abs()
    rows = torch.clamp(S - torch.arange(nb) * block, max=block).double()
    mean_abs = kp.view(nb, block, hh, d).sum(1) / rows.view(nb, 1, 1)
    g, o = mk_gpu.double(), mk_o.double()
    mbits = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[mk_o.dtype]
    _, ex = torch.frexp(torch.maximum(g.abs(), o.abs()))
    ulp = torch.ldexp(torch.ones_like(g), ex - 1 - mbits)
    excess = (g - o).abs() - (ulp + 128 * 2.0 ** -24 * mean_abs)
    bad = int((excess > 0).sum())
    well = o.abs() >= mean_abs * 2.0 ** -8
    ulp_well = ulp_diff_16(mk_gpu[well], mk_o[well]) if bool(well.any()) else 0
    i = int(excess.argmax())
    worst = (f"gpu {g.flatten()[i].item():.6g} oracle {o.flatten()[i].item():.6g} "
             f"mean|k| {mean_abs.flatten()[i].item():.4g}")
    return ulp_well, bad, worst


def seq_slices(cu: Sequence[int]):
    return [(int(cu[b]), int(cu[b + 1])) for b in range(len(cu) - 1)]


def run_stages(q, k, v, cu_list, max_seq_len, *, alpha, sink=2, window=4, last_n=2,
               native=False, check_oracle_scores=True, attention=True,
               min_budget=0, attn_rows=None, block=128) -> StageReport:
    """Run plan/pool/search(dump)/select/attn on the GPU and compare each stage
    with the oracle. q/k/v are CPU tensors (T, H, d); cu_list python ints.
    ``attn_rows`` {sequence: [(head, q-block), ...]} restricts the attention
    comparison to those rows (the oracle's attention over the GPU's lists of
    just those rows), for sequences whose full oracle attention is slow."""
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    od = torch.full_like(qd, float("nan"))
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    call = FlashPrefillCall(qd, kd, vd, od, cu, max_seq_len, alpha=alpha, attention_sink=sink,
                            window_size=window, last_n_block=last_n, native_normalize=native,
                            min_budget=min_budget, block_size=block)
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
        mk_o = O.pool_k(k[s0:s1], block)
        ulp_well, bad, worst = pool_errors(mk_gpu[tile[b]:tile[b + 1]], mk_o, k[s0:s1], block)
        rep.pool_ulp = max(rep.pool_ulp, ulp_well)
        rep.pool_bound_violations += bad
        if bad:
            rep.notes.append(f"pooled K outside the fp32 bound, seq {b}: {worst}")
        # scores from the GPU's own pooled K (isolates the score kernel)
        p_o, m_o = O.block_score(q[s0:s1], mk_gpu[tile[b]:tile[b + 1]], block)
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
        p_e, m_e = O.block_score(q[s0:s1], mk_o, block)
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
            k_tile = min(block, 128)
            if attn_rows is None:
                ref = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], gpu_sel[b], block, k_tile)
                diffs.append((out[s0:s1].float() - ref.float()).abs().reshape(-1))
                continue
            sub = torch.zeros_like(gpu_sel[b])
            for h, i in attn_rows.get(b, []):
                sub[h, i] = gpu_sel[b][h, i]
            ref = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], sub, block, k_tile)
            for h, i in attn_rows.get(b, []):
                r0, r1 = i * block, min((i + 1) * block, s1 - s0)
                diffs.append((out[s0 + r0:s0 + r1, h].float() - ref[r0:r1, h].float())
                             .abs().reshape(-1))
        d = torch.cat(diffs)
        assert not torch.isnan(d).any(), "NaN in GPU output"
        rep.out_max_abs = d.max().item()
        rep.out_mean_abs = d.mean().item()
    return rep


def oracle_head_scores(q_seq, mk, h):
    """The oracle's fp32 block scores (p, m) of query head h alone, from pooled
    keys ``mk`` (NB, Hkv, d): (1, NB, NB) each."""
    G = q_seq.shape[1] // mk.shape[1]
    return O.block_score(q_seq[:, h:h + 1], mk[:, h // G:h // G + 1])


def check_every_row_selection(call, q_cpu, k_cpu, *, native, alpha, sink=2, window=4, last_n=2,
                              min_budget=0, oracle_heads=None):
    """Selection parity on every (head, sequence, q-block) row of a call whose
    plan and pooling stages have run: the search kernel's fp32 scores are
    dumped, and the oracle's selection from those scores must equal the GPU's
    index lists on every row. Then, for the (sequence, head) pairs in
    ``oracle_heads``, the GPU selection kernel is fed the oracle's own fp32
    scores (computed from the oracle's pooled K) and must reproduce the
    oracle's selection exactly (all other heads keep the GPU's scores).
    Returns (rows checked, selected cells)."""
    dump_p, dump_m = call.search(dump=True)
    torch.cuda.synchronize()
    assert call.status() == 0
    assert call.ordered_lists_ok()
    tile, tri, start, lens = call.seq_tables()
    gpu_sel = call.selection_masks()
    gp = call.untri_scores(dump_p)
    gm = call.untri_scores(dump_m)
    rows = selected = 0
    for b, L in enumerate(lens):
        nb = gp[b].shape[-1]
        if nb == 0:
            assert L == 0
            continue
        tril = torch.tril(torch.ones(nb, nb, dtype=torch.bool))
        want = O.select_from_scores(gp[b].nan_to_num(0.0).where(tril, torch.zeros(())),
                                    gm[b].where(tril, torch.tensor(float("-inf"))),
                                    native, alpha, sink, window, last_n, min_budget)
        bad = int((want != gpu_sel[b]).sum())
        assert bad == 0, f"sequence {b}: {bad} cells differ from the oracle's selection of the GPU scores"
        rows += gpu_sel[b].shape[0] * nb
        selected += int(gpu_sel[b].sum())
    if oracle_heads:
        p_in = [x.clone() for x in gp]
        m_in = [x.clone() for x in gm]
        wants = {}
        for b, h in oracle_heads:
            t0, L = start[b], lens[b]
            mk_o = O.pool_k(k_cpu[t0:t0 + L])
            p_o, m_o = oracle_head_scores(q_cpu[t0:t0 + L], mk_o, h)
            p_in[b][h] = p_o[0]
            m_in[b][h] = m_o[0]
            wants[(b, h)] = O.select_from_scores(p_o, m_o, native, alpha, sink, window, last_n,
                                                 min_budget)[0]
        call.select(call.tri_scores([x.nan_to_num(0.0) for x in p_in]),
                    call.tri_scores([x.nan_to_num(float("-inf")) for x in m_in]))
        torch.cuda.synchronize()
        sel2 = call.selection_masks()
        for (b, h), want in wants.items():
            bad = int((sel2[b][h] != want).sum())
            assert bad == 0, f"sequence {b} head {h}: GPU selection of the oracle's scores differs in {bad} cells"
        call.search()  # restore the GPU's own lists
    return rows, selected
