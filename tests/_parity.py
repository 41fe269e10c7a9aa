"""Shared helpers of the GPU parity tests: run the HIP path stage by stage
through the C ABI and compare every intermediate with the CPU oracle."""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch

from flashprefill_amd.runtime import FlashPrefillCall
from oracle import flashprefill_oracle as O

OUT_MAX_ABS = 2e-2   # north-star output tolerance (bf16)
OUT_MEAN_ABS = 2e-3


OUT_MAX_ABS_F32 = 1e-4  # fp32 inputs: fp32 MFMA against the oracle's exact-then-rounded dots
OUT_MEAN_ABS_F32 = 1e-5


def _ulp_line(x: torch.Tensor) -> torch.Tensor:
    """bf16 / fp16 / fp32 bit patterns mapped to a monotone integer line (+0
    and -0 coincide), so that differences count units in the last place."""
    if x.dtype == torch.float32:
        i = x.contiguous().view(torch.int32).to(torch.int64)
        return torch.where(i < 0, -(2 ** 31) - i, i)
    i = x.contiguous().view(torch.int16).to(torch.int64)
    return torch.where(i < 0, -32768 - i, i)


def ulp_diff_16(a: torch.Tensor, b: torch.Tensor) -> int:
    """Max distance in units of the last place between two bf16 / fp16 (or
    two fp32) tensors."""
    if a.numel() == 0:
        return 0
    return int((_ulp_line(a) - _ulp_line(b)).abs().max().item())


@dataclass
class StageReport:
    pool_ulp: int = 0               # max ulp distance over every pooled-K element
    pool_mismatch: int = 0          # pooled-K elements not bit-equal to the oracle's
    pool_exact: bool = True         # 16-bit inputs: fp64 block sums are exact, bit equality expected
    m_max_rel: float = 0.0
    p_max_rel: float = 0.0
    sel_from_gpu_scores_mismatch: int = 0
    sel_from_oracle_scores_mismatch: int = 0
    e2e_flips: int = 0
    cells: int = 0
    out_max_abs: float = 0.0        # over the elements whose output spacing is within the bar
    out_mean_abs: float = 0.0       # over every element
    out_coarse: int = 0             # elements whose output spacing exceeds the bar (|ref| >= 4 in bf16)
    out_coarse_ulp: int = 0         # max ulp distance over those (at most 1)
    density: float = 0.0
    full_rows: int = 0              # (head, q-block) rows checked against the GPU closed form
    notes: List[str] = field(default_factory=list)


def pool_errors(mk_gpu: torch.Tensor, mk_o: torch.Tensor):
    """Pooled K of the GPU against the oracle's (exact fp64 block mean, cast
    to the dtype through fp32). The kernel sums in fp64 and rounds along the
    same path, so bit equality is expected; the bar is <= 1 ulp on every
    element. Returns (max ulp distance, number of elements that are not
    bit-equal, the worst element as text)."""
    if mk_o.numel() == 0:
        return 0, 0, ""
    dist = (_ulp_line(mk_gpu) - _ulp_line(mk_o)).abs().reshape(-1)
    i = int(dist.argmax())
    worst = (f"element {i}: gpu {mk_gpu.reshape(-1)[i].item():.8g} "
             f"oracle {mk_o.reshape(-1)[i].item():.8g} ({int(dist[i])} ulp)")
    return int(dist[i]), int((dist != 0).sum()), worst


def output_spacing(ref: torch.Tensor) -> torch.Tensor:
    """Spacing of ref's dtype at |ref| (one unit in the last place; zero and
    subnormals get the spacing at the smallest normal)."""
    fi = torch.finfo(ref.dtype)
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[ref.dtype]
    a = ref.float().abs().clamp_min(fi.tiny)
    return torch.exp2(torch.floor(torch.log2(a)) - mant)


def output_errors(out: torch.Tensor, ref: torch.Tensor, bar: float):
    """Element errors of an output against the oracle's, both rounded to the
    same dtype. Where that dtype's spacing at |ref| exceeds the max-abs bar
    (bf16 at |ref| >= 4, spacing 2^-5 = 0.031 > 2e-2), two results that each
    round a nearly equal fp32 value can differ by one spacing from the final
    rounding alone, so such "coarse" elements are held to <= 1 ulp instead;
    the bar applies to every other element. Returns (abs errors of the
    bar-checked elements, abs errors of every element, number of coarse
    elements, max ulp distance among them)."""
    d = (out.float() - ref.float()).abs().reshape(-1)
    coarse = (output_spacing(ref) > bar).reshape(-1)
    n = int(coarse.sum())
    ulp = 0
    if n:
        dist = (_ulp_line(out.reshape(-1)[coarse]) - _ulp_line(ref.reshape(-1)[coarse])).abs()
        ulp = int(dist.max())
    return d[~coarse], d, n, ulp


def assert_pool(rep: StageReport) -> None:
    """The pooled-K bar: <= 1 ulp on every element, and bit equality for
    16-bit inputs, whose fp64 block sums are exact on both sides."""
    assert rep.pool_ulp <= 1, rep.notes
    if rep.pool_exact:
        assert rep.pool_mismatch == 0, rep.notes


@torch.no_grad()
def every_row_vs_closed_form(call, out: torch.Tensor, *, block: int = 128,
                             max_blocks: int = 2048) -> Tuple[float, float, int]:
    """Every output row of a finished call against the closed form
    softmax(Q K^T / sqrt(d)) V over the row's selected key blocks, computed
    with torch fp32 on the GPU from the kernel's own index lists (the lists
    are pinned to the oracle's selection separately). Per (head, q-block):
    the listed K / V blocks are gathered, keys past the sequence end and, on
    the diagonal block, keys after the query are masked; an empty list gives
    a zero row (the reference's l = 1 start). This is the dense closed form
    of ``oracle.sparse_attention`` (oracle/flashprefill_oracle.py), without
    its per-tile rounding of P. Rows are processed in batches of similar list
    length holding at most ``max_blocks`` gathered blocks. Returns (max abs
    error, mean abs error, rows checked) over every valid query row."""
    q, k, v, _ = call.tensors
    Hq, Hkv, d = call.Hq, call.Hkv, call.d
    G = Hq // Hkv
    tile, tri, start, lens = call.seq_tables()
    cnt_all = call.counts()
    idx_all = call.index_lists()
    tri_cap = idx_all.shape[1]
    dev = q.device
    scale = 1.0 / math.sqrt(d)
    r_q = torch.arange(block, device=dev).view(1, block, 1, 1)
    r_k = torch.arange(block, device=dev).view(1, 1, 1, block)
    err_max, err_sum, n_el, n_rows = 0.0, 0.0, 0, 0
    for b, L in enumerate(lens):
        if L == 0:
            continue
        nb, t0 = tile[b + 1] - tile[b], start[b]
        for kvh in range(Hkv):
            Kb = torch.zeros(nb * block, d, device=dev)
            Vb = torch.zeros(nb * block, d, device=dev)
            Kb[:L] = k[t0:t0 + L, kvh].float()
            Vb[:L] = v[t0:t0 + L, kvh].float()
            Kb, Vb = Kb.view(nb, block, d), Vb.view(nb, block, d)
            for h in range(kvh * G, (kvh + 1) * G):
                Qb = torch.zeros(nb * block, d, device=dev)
                Qb[:L] = q[t0:t0 + L, h].float()
                Qb = Qb.view(nb, block, d)
                Ob = torch.zeros(nb * block, d, device=dev)
                Ob[:L] = out[t0:t0 + L, h].float()
                Ob = Ob.view(nb, block, d)
                counts = cnt_all[h, tile[b]:tile[b] + nb].long().cpu()
                order = torch.argsort(counts, stable=True).tolist()
                pos = 0
                while pos < nb:
                    # rows sorted by count: take rows while n * max count fits
                    end = pos + 1
                    while end < nb and \
                            (end + 1 - pos) * max(int(counts[order[end]]), 1) <= max_blocks:
                        end += 1
                    rows = torch.tensor(order[pos:end], device=dev)
                    pos = end
                    n = rows.numel()
                    c = cnt_all[h, tile[b] + rows].long()
                    mc = max(int(c.max()), 1)
                    slot = torch.arange(mc, device=dev).view(1, mc)
                    valid = slot < c.view(n, 1)
                    base = tri[b] + rows * (rows + 1) // 2
                    at = torch.clamp(base.view(n, 1) + slot, max=tri_cap - 1)
                    j = torch.where(valid, idx_all[h][at].long(), torch.zeros((), dtype=torch.long,
                                                                          device=dev))
                    assert bool(((j >= 0) & (j <= rows.view(n, 1))).all()), "list entry out of range"
                    Kg = Kb[j].reshape(n, mc * block, d)
                    Vg = Vb[j].reshape(n, mc * block, d)
                    s = torch.bmm(Qb[rows], Kg.transpose(1, 2).contiguous()) * scale
                    s = s.view(n, block, mc, block)
                    key = j.view(n, 1, mc, 1) * block + r_k
                    keep = valid.view(n, 1, mc, 1) & (key < L) & \
                        ((j.view(n, 1, mc, 1) != rows.view(n, 1, 1, 1)) | (r_k <= r_q))
                    s = s.masked_fill(~keep, float("-inf")).view(n, block, mc * block)
                    p = torch.softmax(s, dim=-1).nan_to_num(0.0)
                    ref = torch.bmm(p, Vg)
                    qrow = rows.view(n, 1) * block + torch.arange(block, device=dev).view(1, block)
                    live = (qrow < L).view(n, block, 1)
                    diff = ((Ob[rows] - ref).abs() * live)
                    assert not bool(torch.isnan(Ob[rows]).any()), f"NaN output, sequence {b} head {h}"
                    err_max = max(err_max, float(diff.max()))
                    err_sum += float(diff.sum(dtype=torch.float64))
                    n_el += int(live.sum()) * d
                    n_rows += n
    return err_max, err_sum / max(n_el, 1), n_rows


def expand_sel(sel: torch.Tensor, ratio: int, nb_plan: int) -> torch.Tensor:
    """A (Hq, NB, NB) selection over selection blocks (256 tokens at ratio 2)
    as the (Hq, nb_plan, nb_plan) lists over the plan's 128-token blocks must
    hold it: plan block c of plan row r is listed iff selection block c // 2
    is selected for selection row r // 2 and c <= r (the upper half of the
    diagonal 256-block is after every query of the lower plan row)."""
    if ratio == 1:
        return sel
    r = torch.arange(nb_plan)
    blk = r // ratio
    return sel[:, blk][:, :, blk] & (r.view(-1, 1) >= r.view(1, -1))


def collapse_sel(sel_plan: torch.Tensor, ratio: int) -> torch.Tensor:
    """The selection-block view of plan-granularity lists: (row 2i, block 2j)
    stands for selection cell (i, j)."""
    return sel_plan if ratio == 1 else sel_plan[:, ::ratio, ::ratio]


def seq_slices(cu: Sequence[int]):
    return [(int(cu[b]), int(cu[b + 1])) for b in range(len(cu) - 1)]


def run_stages(q, k, v, cu_list, max_seq_len, *, alpha, sink=2, window=4, last_n=2,
               native=False, check_oracle_scores=True, attention=True,
               min_budget=0, attn_rows=None, block=128) -> StageReport:
    """Run plan/pool/search(dump)/select/attn on the GPU and compare each stage
    with the oracle. q/k/v are CPU tensors (T, H, d); cu_list python ints.
    ``attn_rows`` {sequence: [(head, q-block), ...]} restricts the oracle's
    attention comparison to those rows (the oracle's attention over the GPU's
    lists of just those rows), for sequences whose full oracle attention is
    slow; every row is then compared with the closed form on the GPU
    (every_row_vs_closed_form), and the output figures are the worse of the
    two comparisons."""
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    od = torch.full_like(qd, float("nan"))
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    call = FlashPrefillCall(qd, kd, vd, od, cu, max_seq_len, alpha=alpha, attention_sink=sink,
                            window_size=window, last_n_block=last_n, native_normalize=native,
                            min_budget=min_budget, block_size=block)
    rep = StageReport(pool_exact=k.dtype != torch.float32)
    ratio = call.ratio  # 2 at block 256: selection blocks of two plan blocks
    call.plan()
    call.pool()
    dump_p, dump_m = call.search(dump=True)
    torch.cuda.synchronize()
    assert call.status() == 0
    tile, tri, start, lens = call.seq_tables()
    assert lens == [b - a for a, b in seq_slices(cu_list)]
    stile = call.sel_tables()
    mk_gpu = call.pooled_k().cpu()
    plan_sel = call.selection_masks()
    # the plan-granularity lists are exactly the expansion of the selection
    gpu_sel = [collapse_sel(x, ratio) for x in plan_sel]
    for b in range(len(plan_sel)):
        assert torch.equal(expand_sel(gpu_sel[b], ratio, plan_sel[b].shape[-1]), plan_sel[b]), \
            f"sequence {b}: plan lists are not the expansion of the selection"
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
        ulp, diff, worst = pool_errors(mk_gpu[stile[b]:stile[b + 1]], mk_o)
        rep.pool_ulp = max(rep.pool_ulp, ulp)
        rep.pool_mismatch += diff
        if diff:
            rep.notes.append(f"pooled K differs from the oracle's, seq {b}: {worst}")
        # scores from the GPU's own pooled K (isolates the score kernel)
        p_o, m_o = O.block_score(q[s0:s1], mk_gpu[stile[b]:stile[b + 1]], block)
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
            rep.sel_from_oracle_scores_mismatch += int(
                (sel2[b] != expand_sel(want, ratio, sel2[b].shape[-1])).sum())
        # restore the GPU's own selection for the attention stage
        call.search()

    if attention:
        call.attn()
        torch.cuda.synchronize()
        out = od.cpu()
        f32 = q.dtype == torch.float32
        bar = OUT_MAX_ABS_F32 if f32 else OUT_MAX_ABS
        diffs, diffs_all = [], []

        def add(o, r):
            dm, da, n, ulp = output_errors(o, r, bar)
            diffs.append(dm)
            diffs_all.append(da)
            rep.out_coarse += n
            rep.out_coarse_ulp = max(rep.out_coarse_ulp, ulp)
        for b, (s0, s1) in enumerate(seq_slices(cu_list)):
            if s1 == s0:
                continue
            # the attention walks 128-key tiles; at head_dim 256 it takes each
            # block in 32-key passes, and the oracle uses the reference's
            # K_TILE_SIZE 64 there (the two differ at rounding level)
            k_tile = 64 if q.shape[-1] > 128 else min(block, 128)
            if attn_rows is None:
                ref = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], gpu_sel[b], block, k_tile)
                add(out[s0:s1], ref)
                continue
            sub = torch.zeros_like(gpu_sel[b])
            for h, i in attn_rows.get(b, []):
                sub[h, i] = gpu_sel[b][h, i]
            ref = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], sub, block, k_tile)
            for h, i in attn_rows.get(b, []):
                r0, r1 = i * block, min((i + 1) * block, s1 - s0)
                add(out[s0 + r0:s0 + r1, h], ref[r0:r1, h])
        d, d_all = torch.cat(diffs), torch.cat(diffs_all)
        assert not torch.isnan(d_all).any(), "NaN in GPU output"
        assert rep.out_coarse_ulp <= 1, \
            f"{rep.out_coarse_ulp} ulp on an output element whose spacing exceeds {bar}"
        rep.out_max_abs = d.max().item() if d.numel() else 0.0
        rep.out_mean_abs = d_all.mean().item()
        if attn_rows is not None:
            # the oracle saw sampled rows only: every row against the closed
            # form on the GPU, from the same lists, under the same bars
            fmax, fmean, rows = every_row_vs_closed_form(call, od, block=block // ratio)
            rep.notes.append(f"closed form, every row: {rows} rows, max {fmax:.2e} "
                             f"mean {fmean:.2e}")
            rep.out_max_abs = max(rep.out_max_abs, fmax)
            rep.out_mean_abs = max(rep.out_mean_abs, fmean)
            rep.full_rows = rows
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
