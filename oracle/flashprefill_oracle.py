"""CPU restatement of the FlashPrefill sparse-prefill attention algorithm.

TEST INFRASTRUCTURE ONLY. This module is the parity oracle: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or as the timed CPU baseline). The product
path (``flashprefill_amd``) never calls it and has no CPU fallback.

It restates, in plain PyTorch-on-CPU arithmetic (fp32 with fp64 where noted),
the two reference operator files:

* ``ops/flashprefill_native_forward.py`` (batched ``(B, S, H, d)`` entry point)
* ``ops/flashprefill_varlen_func.py``    (packed ``cu_seqlens`` entry point)

Each function cites the reference lines it follows. Where the reference's
arithmetic is not reproducible bit-for-bit (Triton's bf16 tree sums, NVIDIA's
``ex2.approx``, the reduction order of inductor kernels, autotuned tile
sizes), the oracle fixes one canonical arithmetic and says so:

* pooled K: fp64 sum of the block's valid rows / n_valid in fp64, converted to
  the input dtype by torch's cast (fp64 -> fp32 -> bf16 / fp16, each round to
  nearest even); the sum of at most 256 16-bit values is exact in fp64 unless
  their exponents span more than ~38 binades (the reference sums in the input
  dtype, ``…native_forward.py:53``);
* dot products: exact (fp64) then rounded once to fp32 (the reference's
  ``tl.dot`` accumulates in fp32 in an unspecified order);
* ``exp2`` in the normalisation/selection stage: computed in fp64 from the
  fp32 argument and rounded to fp32 (i.e. correctly rounded fp32 exp2);
* row sums in the native normalisation: fp64 sum of the fp32 terms, rounded
  once to fp32 (order independent);
* attention: the online softmax runs over key tiles of ``k_tile`` keys (128 by
  default; 64 matches the reference's other autotuned K_TILE_SIZE and the GPU
  persistent kernel), P is rounded to V's dtype before P@V, exactly as
  ``…native_forward.py:298-331`` does.

Pinning status (what checks each function, see ``tests/test_oracle.py``):
  pool_k            closed form (fp64 block mean), exact rational mean rounded
                    to fp64, fp32 then the dtype + mutation check
  block_score       brute-force pure-Python loops on tiny inputs + closed-form
                    diagonal rule (row 127 only) + mutation checks
  normalize_scores  brute-force loops on the formula + invariants
  select_blocks     brute-force loops + invariants (causal, diagonal in window,
                    sink, last-n rows full, ascending lists)
  sparse_attention  dense fp64 masked softmax (closed form) and, with every
                    block selected, torch's scaled_dot_product_attention
                    (causal) + mutation checks
  layouts           round-trip/invariant checks against the selection mask
  min_budget top-k  parity unpinned where ties among equal scores decide the
                    top-k set (the reference uses torch.topk, whose tie order is
                    unspecified); pinned by brute force otherwise.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

LOG2E = 1.4426950408889634  # ops/flashprefill_native_forward.py:144,280


def _f32(x: float) -> torch.Tensor:
    """Round a Python float to an fp32 scalar tensor (Triton/torch scalar args)."""
    return torch.tensor(x, dtype=torch.float32)


def sm_scale_f32(head_dim: int) -> torch.Tensor:
    """fp32 ``scale * log2(e)`` with ``scale = 1/sqrt(d)``.

    ``…native_forward.py:439`` passes ``1 / (head_dim ** 0.5)`` as an fp32 kernel
    argument and ``:144`` multiplies it by the fp32 literal 1.4426950408889634.
    """
    return _f32(1.0 / (head_dim ** 0.5)) * _f32(LOG2E)


def exp2_f32(x: torch.Tensor) -> torch.Tensor:
    """Correctly rounded fp32 exp2 of an fp32 tensor (fp64 evaluation)."""
    assert x.dtype == torch.float32
    return torch.exp2(x.double()).float()


def num_blocks(seq_len: int, block: int) -> int:
    return (seq_len + block - 1) // block


def get_cu_tile_seqlens(cu_seqlens: Sequence[int], block: int) -> Tuple[List[int], List[int]]:
    """Block-count prefix sums ``cu_tile`` and ``cu_tile2`` (``…varlen_func.py:8-18``)."""
    cu_tile, cu_tile2 = [0], [0]
    for b in range(len(cu_seqlens) - 1):
        nb = num_blocks(int(cu_seqlens[b + 1]) - int(cu_seqlens[b]), block)
        cu_tile.append(cu_tile[-1] + nb)
        cu_tile2.append(cu_tile2[-1] + nb * nb)
    return cu_tile, cu_tile2


# ---------------------------------------------------------------------------
# a1: pooled K (…native_forward.py:21-67, …varlen_func.py:35-85)
# ---------------------------------------------------------------------------

def pool_k(k_seq: torch.Tensor, block: int = 128) -> torch.Tensor:
    """Mean of each ``block``-row slab of K over its valid rows.

    k_seq: (S, Hkv, d) one sequence. Returns (NB, Hkv, d) in k_seq.dtype.
    Rows past S do not count (``num_ele`` = number of valid rows, :55-58).
    The fp64 mean reaches a 16-bit dtype through fp32 (torch's cast rounds
    fp64 -> fp32 -> bf16 / fp16), a rounding path the GPU kernel repeats.
    """
    S, Hkv, d = k_seq.shape
    nb = num_blocks(S, block)
    kp = torch.zeros(nb * block, Hkv, d, dtype=torch.float64)
    kp[:S] = k_seq.double()
    sums = kp.view(nb, block, Hkv, d).sum(dim=1)
    counts = torch.full((nb,), float(block), dtype=torch.float64)
    if S % block:
        counts[-1] = float(S % block)
    return (sums / counts.view(nb, 1, 1)).to(k_seq.dtype)


# ---------------------------------------------------------------------------
# a2: block score (…native_forward.py:87-188, …varlen_func.py:106-217)
# ---------------------------------------------------------------------------

def block_score(q_seq: torch.Tensor, mk: torch.Tensor, block: int = 128
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-(head, q-block i, k-block j) row-max ``m`` and exp2-sum ``p``.

    For q-block i and pooled key j the 128 query rows r give
    ``s_r = fl32(fl32(Q[128i+r] . mk_j) * sm_scale)`` (:156,160). Causal block
    mask ``128i + r >= 128j + 127`` (:157): all rows for j < i, only row 127 for
    j == i, none for j > i. Query rows past S are zero and still count for j < i
    (:135-139). ``m_ij = max_r s_r``; ``p_ij = sum_r exp2(s_r - m_ij)`` (:162-174).

    Returns p, m of shape (Hq, NB, NB) fp32 with p = 0, m = -inf for j > i.
    """
    S, Hq, d = q_seq.shape
    nb, Hkv, _ = mk.shape
    G = Hq // Hkv
    c = sm_scale_f32(d)
    qp = torch.zeros(nb * block, Hq, d, dtype=torch.float64)
    qp[:S] = q_seq.double()
    r = torch.arange(block).view(1, block, 1)
    i_idx = torch.arange(nb).view(nb, 1, 1)
    j_idx = torch.arange(nb).view(1, 1, nb)
    mask = (block * i_idx + r) >= (block * j_idx + block - 1)  # (nb, block, nb)
    p_out = torch.zeros(Hq, nb, nb, dtype=torch.float32)
    m_out = torch.full((Hq, nb, nb), float("-inf"), dtype=torch.float32)
    for h in range(Hq):
        raw = (qp[:, h, :] @ mk[:, h // G, :].double().T).float()  # exact dot, one rounding
        s = (raw * c).view(nb, block, nb)
        s = torch.where(mask, s, torch.tensor(float("-inf")))
        m = s.max(dim=1).values  # (nb, nb)
        diff = s - m.unsqueeze(1)  # fp32 subtraction as in :166
        e = torch.where(mask, torch.exp2(diff.double()), torch.zeros((), dtype=torch.float64))
        p = e.sum(dim=1).float()
        causal = torch.tril(torch.ones(nb, nb, dtype=torch.bool))
        p_out[h] = torch.where(causal, p, torch.zeros(()))
        m_out[h] = torch.where(causal, m, torch.tensor(float("-inf")))
    return p_out, m_out


# ---------------------------------------------------------------------------
# a3: normalisation (…native_forward.py:388-403; …varlen_func.py:240-304,656)
# ---------------------------------------------------------------------------

def normalize_scores(p: torch.Tensor, m: torch.Tensor, native: bool) -> torch.Tensor:
    """``S_ij = p_ij * exp2(m_ij - M_i)`` on the causal triangle, 0 elsewhere.

    ``M_i = max_j m_ij`` over causal j (:393; the varlen kernel's NaN-ignoring
    max gives the same value, :279-286). Native mode additionally divides by
    ``sum_j S_ij + 1e-9`` (:401); varlen mode does not (:656).
    p, m: (..., NB, NB) fp32. Returns fp32 of the same shape.
    """
    nb = p.shape[-1]
    causal = torch.tril(torch.ones(nb, nb, dtype=torch.bool))
    mm = torch.where(causal, m, torch.tensor(float("-inf")))
    M = mm.max(dim=-1, keepdim=True).values
    e = exp2_f32(torch.where(causal, m - M, torch.zeros(())))
    S = torch.where(causal, p * e, torch.zeros(()))
    if native:
        tot = S.double().sum(dim=-1, keepdim=True).float()
        denom = tot + _f32(1e-9)
        S = torch.where(causal, S / denom, torch.zeros(()))
    return S


# ---------------------------------------------------------------------------
# a4: dynamic thresholding / pattern selection
#     (…native_forward.py:347-385; …varlen_func.py:327-409)
# ---------------------------------------------------------------------------

def select_blocks(S: torch.Tensor, alpha: float, attention_sink: int, window: int,
                  last_n: int, min_budget: int = 0) -> torch.Tensor:
    """Boolean selection ``sel[..., i, j]``.

    ``sel = causal & (S >= fl32(max_j S * fl32(alpha)) | j < sink |
    0 <= i-j < window | i >= NB - last_n)`` (:359-375, :392-396).
    ``min_budget > 0`` (native only, :353-357): the ``min_budget`` largest causal
    scores are forced on and the threshold is relative to the top-1 (ties among
    equal scores are broken towards the lower j; torch.topk leaves that order
    unspecified, so such ties are parity unpinned).
    """
    nb = S.shape[-1]
    i_idx = torch.arange(nb).view(nb, 1)
    j_idx = torch.arange(nb).view(1, nb)
    causal = j_idx <= i_idx
    Sc = torch.where(causal, S, torch.zeros(()))
    maxS = Sc.max(dim=-1, keepdim=True).values
    thr = maxS * _f32(alpha)
    mask_score = S >= thr
    if min_budget > 0:
        # rank causal cells by (value desc, j asc); take the first min_budget
        key = torch.where(causal, Sc, torch.tensor(float("-inf")))
        order = torch.sort(key, dim=-1, descending=True, stable=True).indices
        topk = torch.zeros_like(mask_score)
        topk.scatter_(-1, order[..., :min_budget], True)
        mask_score = mask_score | topk
    dist = i_idx - j_idx
    mask_sink = j_idx < attention_sink
    mask_window = (dist >= 0) & (dist < window)
    mask_last = i_idx >= (nb - last_n)
    return (mask_score | mask_sink | mask_window | mask_last) & causal


def select_from_scores(p: torch.Tensor, m: torch.Tensor, native: bool, alpha: float,
                       attention_sink: int, window: int, last_n: int,
                       min_budget: int = 0) -> torch.Tensor:
    return select_blocks(normalize_scores(p, m, native), alpha, attention_sink,
                         window, last_n, min_budget)


# ---------------------------------------------------------------------------
# a5: block-sparse flash attention (…native_forward.py:227-344;
#     …varlen_func.py:449-575)
# ---------------------------------------------------------------------------

def sparse_attention(q_seq: torch.Tensor, k_seq: torch.Tensor, v_seq: torch.Tensor,
                     sel: torch.Tensor, block: int = 128, k_tile: int = 128) -> torch.Tensor:
    """Online-softmax attention over the selected key blocks, in list order.

    Per (head h, q-block i) the selected blocks j are visited in ascending order
    (:289-331) and each block in key tiles of ``k_tile`` keys (the reference's
    autotuned K_TILE_SIZE, 64 or 128, :298). Per tile: ``qk = Q K^T`` (fp32),
    the diagonal block masks ``q_pos < k_pos`` to -inf (:312-315),
    ``qk *= sm_scale``; then ``m_new = max(m, rowmax)``, ``p = exp2(qk - m_new)``,
    ``alpha = exp2(m - m_new)`` with NaN -> 1 (:323-325), ``l = l*alpha + sum p``,
    ``acc = acc*alpha + p.to(v.dtype) @ v`` (:326-330). ``m`` starts at -inf and
    ``l`` at 1.0 (:282-283). Output ``acc / l`` cast to q.dtype (:333-344).
    Key rows past S load as zeros (:300-309).

    q_seq (S, Hq, d); k_seq, v_seq (S, Hkv, d); sel (Hq, NB, NB) bool.
    """
    S, Hq, d = q_seq.shape
    Hkv = k_seq.shape[1]
    G = Hq // Hkv
    nb = num_blocks(S, block)
    assert block % k_tile == 0
    c = sm_scale_f32(d)
    pad = nb * block
    qf = torch.zeros(pad, Hq, d, dtype=torch.float64)
    kf = torch.zeros(pad, Hkv, d, dtype=torch.float64)
    vf = torch.zeros(pad, Hkv, d, dtype=torch.float32)
    qf[:S] = q_seq.double()
    kf[:S] = k_seq.double()
    vf[:S] = v_seq.float()
    out = torch.zeros(pad, Hq, d, dtype=torch.float32)
    ninf = torch.tensor(float("-inf"))
    qpos = torch.arange(block).view(block, 1)
    for h in range(Hq):
        kvh = h // G
        for i in range(nb):
            js = torch.nonzero(sel[h, i]).flatten().tolist()
            qi = qf[i * block:(i + 1) * block, h, :]
            m_i = torch.full((block,), float("-inf"))
            l_i = torch.ones(block)
            acc = torch.zeros(block, d)
            for j in js:
                for k0 in range(j * block, (j + 1) * block, k_tile):
                    kj = kf[k0:k0 + k_tile, kvh, :]
                    vj = vf[k0:k0 + k_tile, kvh, :]
                    qk = (qi @ kj.T).float()
                    if j == i:
                        kpos = torch.arange(k0 - j * block, k0 - j * block + k_tile).view(1, k_tile)
                        qk = torch.where(qpos >= kpos, qk, ninf)
                    qk = qk * c
                    m_new = torch.maximum(m_i, qk.max(dim=1).values)
                    p = exp2_f32(qk - m_new.view(block, 1))
                    lij = p.double().sum(dim=1).float()
                    alpha = exp2_f32(m_i - m_new)
                    alpha = torch.where(torch.isnan(alpha), torch.ones(()), alpha)
                    acc = acc * alpha.view(block, 1)
                    l_i = l_i * alpha + lij
                    pv = p.to(v_seq.dtype).float()
                    acc = acc + (pv.double() @ vj.double()).float()
                    m_i = m_new
            out[i * block:(i + 1) * block, h, :] = acc * (1.0 / l_i).view(block, 1)
    return out[:S].to(q_seq.dtype)


def dense_masked_attention_fp64(q_seq: torch.Tensor, k_seq: torch.Tensor,
                                v_seq: torch.Tensor, sel: torch.Tensor,
                                block: int = 128) -> torch.Tensor:
    """Closed form: ``softmax(Q K^T / sqrt(d) + mask) V`` in fp64, where the mask
    allows key t for query s iff block(t) is selected for (head, block(s)) and
    t <= s inside the diagonal block (t < s is implied elsewhere by causality of
    the selection). Used to pin ``sparse_attention``."""
    S, Hq, d = q_seq.shape
    Hkv = k_seq.shape[1]
    G = Hq // Hkv
    qb = torch.arange(S) // block
    allow_blk = sel[:, qb][:, :, qb]  # (Hq, S, S) block-level selection
    causal = torch.arange(S).view(S, 1) >= torch.arange(S).view(1, S)
    out = torch.zeros(S, Hq, d, dtype=torch.float64)
    for h in range(Hq):
        qh = q_seq[:, h, :].double()
        kh = k_seq[:, h // G, :].double()
        vh = v_seq[:, h // G, :].double()
        s = (qh @ kh.T) / math.sqrt(d)
        allow = allow_blk[h] & causal
        s = torch.where(allow, s, torch.tensor(float("-inf"), dtype=torch.float64))
        w = torch.softmax(s, dim=-1)
        w = torch.nan_to_num(w, nan=0.0)
        out[:, h, :] = w @ vh
    return out


def flashprefill_rows(q_seq: torch.Tensor, k_seq: torch.Tensor, v_seq: torch.Tensor,
                      rows: Sequence[Tuple[int, int]], *, alpha: float, attention_sink: int,
                      window: int, last_n: int, native: bool, block: int = 128,
                      mk: Optional[torch.Tensor] = None
                      ) -> Dict[Tuple[int, int], Tuple[torch.Tensor, torch.Tensor]]:
    """The whole pipeline restricted to some (head, q-block) rows of one
    sequence: pooled K (all blocks), the block scores of each listed row,
    its normalisation and selection, and its attention output. Same arithmetic
    as block_score / normalize_scores / select_blocks / sparse_attention
    applied to one row; used to time a bounded sample of a long sequence.
    Returns {(h, i): (sel_row (NB,) bool, out (rows_in_block, d))}."""
    S, Hq, d = q_seq.shape
    Hkv = k_seq.shape[1]
    G = Hq // Hkv
    nb = num_blocks(S, block)
    c = sm_scale_f32(d)
    if mk is None:
        mk = pool_k(k_seq, block)
    ninf = torch.tensor(float("-inf"))
    r = torch.arange(block).view(block, 1)
    pos = torch.arange(block)
    diag_mask = pos.view(block, 1) >= pos.view(1, block)
    res = {}
    for h, i in rows:
        kvh = h // G
        q0, q1 = i * block, min(S, (i + 1) * block)
        qi = torch.zeros(block, d, dtype=torch.float64)
        qi[:q1 - q0] = q_seq[q0:q1, h].double()
        raw = (qi @ mk[:i + 1, kvh].double().T).float()  # (block, i+1)
        s = raw * c
        mask = (block * i + r) >= (block * torch.arange(i + 1).view(1, -1) + block - 1)
        s = torch.where(mask, s, ninf)
        m_row = s.max(dim=0).values
        e = torch.where(mask, torch.exp2((s - m_row.view(1, -1)).double()),
                        torch.zeros((), dtype=torch.float64))
        p_row = e.sum(dim=0).float()
        # normalisation and selection of row i (all j <= i are causal)
        M = m_row.max()
        S_row = p_row * exp2_f32(m_row - M)
        if native:
            tot = S_row.double().sum().float()
            S_row = S_row / (tot + _f32(1e-9))
        thr = S_row.max() * _f32(alpha)
        jj = torch.arange(i + 1)
        keep = (S_row >= thr) | (jj < attention_sink) | ((i - jj) < window) | (i >= nb - last_n)
        sel_row = torch.zeros(nb, dtype=torch.bool)
        sel_row[:i + 1] = keep
        # attention of this row over its selected blocks
        js = torch.nonzero(sel_row).flatten().tolist()
        m_i = torch.full((block,), float("-inf"))
        l_i = torch.ones(block)
        acc = torch.zeros(block, d)
        for j in js:
            k0, k1 = j * block, min(S, (j + 1) * block)
            kj = torch.zeros(block, d, dtype=torch.float64)
            vj = torch.zeros(block, d, dtype=torch.float32)
            kj[:k1 - k0] = k_seq[k0:k1, kvh].double()
            vj[:k1 - k0] = v_seq[k0:k1, kvh].float()
            qk = (qi @ kj.T).float()
            if j == i:
                qk = torch.where(diag_mask, qk, ninf)
            qk = qk * c
            m_new = torch.maximum(m_i, qk.max(dim=1).values)
            p = exp2_f32(qk - m_new.view(block, 1))
            lij = p.double().sum(dim=1).float()
            a_ = exp2_f32(m_i - m_new)
            a_ = torch.where(torch.isnan(a_), torch.ones(()), a_)
            acc = acc * a_.view(block, 1)
            l_i = l_i * a_ + lij
            acc = acc + (p.to(v_seq.dtype).float().double() @ vj.double()).float()
            m_i = m_new
        out = (acc * (1.0 / l_i).view(block, 1))[:q1 - q0].to(q_seq.dtype)
        res[(h, i)] = (sel_row, out)
    return res


# ---------------------------------------------------------------------------
# layouts of the selection (…native_forward.py:377-385; …varlen_func.py:683-698)
# ---------------------------------------------------------------------------

def native_index_layout(sel: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """sel (B, Hq, NB, NB) -> (compact_indices (B, NB, NB, Hq) int64 ascending,
    padded with NB; counts (B, NB, Hq) int32) exactly as ``deal_output_score``."""
    B, Hq, nb, _ = sel.shape
    k_ids = torch.arange(nb).view(1, 1, 1, nb).expand(B, Hq, nb, nb)
    filled = torch.where(sel, k_ids, torch.full((), nb))
    compact = torch.sort(filled, dim=-1).values.to(torch.int64)
    counts = sel.sum(dim=-1).to(torch.int32)
    return compact.permute(0, 2, 3, 1).contiguous(), counts.permute(0, 2, 1).contiguous()


def varlen_index_layout(sels: Sequence[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-sequence selections sels[b] (Hq, NB_b, NB_b) -> (flat out_index int32
    ordered head -> sequence -> q-block -> ascending j, out_number_cu int32 of
    length Hq * sum(NB_b) + 1) as ``…varlen_func.py:683-698`` builds them."""
    Hq = sels[0].shape[0]
    idx: List[torch.Tensor] = []
    counts: List[torch.Tensor] = []
    for h in range(Hq):
        for s in sels:
            nb = s.shape[-1]
            for i in range(nb):
                js = torch.nonzero(s[h, i]).flatten().to(torch.int32)
                idx.append(js)
                counts.append(torch.tensor([js.numel()], dtype=torch.int32))
    flat = torch.cat(idx) if idx else torch.zeros(0, dtype=torch.int32)
    cnt = torch.cat(counts)
    cu = torch.zeros(cnt.numel() + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(cnt, dim=0)
    return flat, cu


# ---------------------------------------------------------------------------
# a6: the two operator entry points (…native_forward.py:405-499;
#     …varlen_func.py:577-743)
# ---------------------------------------------------------------------------

@dataclass
class SeqTrace:
    """Intermediates of one sequence (for parity checks)."""
    mk: torch.Tensor
    p: torch.Tensor
    m: torch.Tensor
    S: torch.Tensor
    sel: torch.Tensor


@dataclass
class OracleResult:
    out: torch.Tensor
    traces: List[SeqTrace] = field(default_factory=list)


def flashprefill_sequence(q_seq, k_seq, v_seq, *, alpha: float, attention_sink: int,
                          window: int, last_n: int, native: bool, min_budget: int = 0,
                          block: int = 128, with_output: bool = True
                          ) -> Tuple[Optional[torch.Tensor], SeqTrace]:
    """All stages for one sequence: pool -> score -> normalise -> select -> attend."""
    assert q_seq.shape[1] % k_seq.shape[1] == 0, "num_q_heads must be a multiple of num_k_heads"
    mk = pool_k(k_seq, block)
    p, m = block_score(q_seq, mk, block)
    S = normalize_scores(p, m, native)
    sel = select_blocks(S, alpha, attention_sink, window, last_n, min_budget)
    out = sparse_attention(q_seq, k_seq, v_seq, sel, block) if with_output else None
    return out, SeqTrace(mk=mk, p=p, m=m, S=S, sel=sel)


def flash_prefill_varlen_func(q, k, v, cu_seqlens, max_seq_len: int, alpha: float,
                              block_size: int = 128, attention_sink: int = 2,
                              window_size: int = 4, last_n_block: int = 2,
                              with_output: bool = True) -> OracleResult:
    """Varlen entry point (``…varlen_func.py:722-743``): q (T, Hq, d), k/v (T, Hkv, d)."""
    cu = [int(x) for x in torch.as_tensor(cu_seqlens).tolist()]
    out = torch.zeros_like(q) if with_output else None
    res = OracleResult(out=out)
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        if s1 == s0:
            res.traces.append(SeqTrace(*(torch.zeros(0),) * 5))
            continue
        o, tr = flashprefill_sequence(q[s0:s1], k[s0:s1], v[s0:s1], alpha=alpha,
                                      attention_sink=attention_sink, window=window_size,
                                      last_n=last_n_block, native=False, block=block_size,
                                      with_output=with_output)
        if with_output:
            out[s0:s1] = o
        res.traces.append(tr)
    return res


def flash_prefill(q, k, v, block_size: int, attention_sink: int, window_size: int,
                  alpha: float, last_n_block_full: int, min_budget: int = 0,
                  with_output: bool = True) -> OracleResult:
    """Batched entry point (``…native_forward.py:480-499``): q (B, S, Hq, d),
    k/v (B, S, Hkv, d) (the code reads ``(b, s, h, d)``, :416)."""
    B = q.shape[0]
    out = torch.zeros_like(q) if with_output else None
    res = OracleResult(out=out)
    for b in range(B):
        o, tr = flashprefill_sequence(q[b], k[b], v[b], alpha=alpha,
                                      attention_sink=attention_sink, window=window_size,
                                      last_n=last_n_block_full, native=True,
                                      min_budget=min_budget, block=block_size,
                                      with_output=with_output)
        if with_output:
            out[b] = o
        res.traces.append(tr)
    return res
