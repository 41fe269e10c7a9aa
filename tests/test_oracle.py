"""Pins of the CPU oracle (oracle/flashprefill_oracle.py) by brute force,
closed forms, library routines and invariants. The reference ships no golden
vectors (it has no tests at all), so every oracle function is pinned here
instead; the "planted mistake" tests show each check fails on a plausible
error in the oracle's arithmetic.
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import flashprefill_oracle as O

F32 = np.float32


def _c(d):
    return F32(F32(1.0 / d ** 0.5) * F32(O.LOG2E))


def _rand(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# --------------------------------------------------------------------------
# a1 pooled K: closed form (block mean over valid rows)
# --------------------------------------------------------------------------

def _pool_closed_form(k, block):
    S = k.shape[0]
    nb = (S + block - 1) // block
    out = []
    for j in range(nb):
        rows = k[j * block:min(S, (j + 1) * block)].double()
        out.append(rows.mean(dim=0))
    return torch.stack(out)


@pytest.mark.parametrize("S,block", [(300, 128), (256, 128), (1, 128), (100, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pool_k_closed_form(S, block, dtype):
    k = _rand((S, 3, 16), 1, dtype)
    got = O.pool_k(k, block)
    ref = _pool_closed_form(k, block)
    assert got.dtype == dtype
    # one rounding of the fp64 mean to the storage dtype
    torch.testing.assert_close(got.double(), ref.to(dtype).double(), rtol=0, atol=0)


def _bf16_rne_bits(f32: np.ndarray) -> np.ndarray:
    # round-to-nearest-even of fp32 bit patterns to bf16 (finite inputs)
    u = f32.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pool_k_exact_rational_mean(dtype):
    # Exact rational block mean (fractions), rounded to fp64, then fp32, then
    # the 16-bit dtype, each by round to nearest even outside torch. Columns
    # whose mean cancels to ~0 and one whose mean sits at an fp32 rounding
    # midpoint are included.
    g = torch.Generator().manual_seed(8)
    S, block = 200, 128
    k = (torch.randn(S, 2, 8, generator=g) * 3).to(dtype)
    k[:128, 0, 0] = 3.0
    k[1:128:2, 0, 0] = -3.0
    k[0, 0, 0] = 3.015625
    # block mean = M + 2^-27 with M a midpoint between two neighbouring 16-bit
    # values: fp32 drops the 2^-27, so the cast through fp32 ties to even (M
    # rounds down to 1.0) where a direct fp64 -> 16-bit rounding rounds up
    k[:128, 1, 1] = 1.0
    k[0, 1, 1] = 2.5 if dtype == torch.bfloat16 else 2.0625
    k[1, 1, 1] = 2.0 ** -20
    got = O.pool_k(k, block)
    mid = 1.0 + (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)
    assert got[0, 1, 1].item() == 1.0
    direct = np.float64(mid + 2.0 ** -27)
    assert direct > mid  # a direct rounding would give the upper neighbour
    kv = k.float().numpy().astype(np.float64)
    for j in range(2):
        rows = kv[j * block:min(S, (j + 1) * block)]
        for h in range(2):
            for x in range(8):
                mean = sum(Fraction(float(v)) for v in rows[:, h, x]) / len(rows)
                f32 = np.array([float(mean)], dtype=np.float64).astype(np.float32)
                if dtype == torch.bfloat16:
                    want = int(_bf16_rne_bits(f32)[0])
                else:
                    want = int(f32.astype(np.float16).view(np.uint16)[0])
                have = int(got[j, h, x].view(torch.int16).item()) & 0xFFFF
                assert have == want, (j, h, x, float(mean))


def test_pool_k_planted_divisor_mistake():
    k = _rand((300, 2, 8), 2)
    S, block = 300, 128
    wrong = torch.stack([k[j * block:(j + 1) * block].double().sum(0) / block for j in range(3)])
    assert not torch.allclose(wrong, _pool_closed_form(k, block))  # last block has 44 rows


# --------------------------------------------------------------------------
# a2 block score: pure-Python brute force
# --------------------------------------------------------------------------

def _brute_block_score(q, mk, block):
    S, Hq, d = q.shape
    nb, Hkv, _ = mk.shape
    G = Hq // Hkv
    c = _c(d)
    qd = q.double().numpy()
    kd = mk.double().numpy()
    p = np.zeros((Hq, nb, nb), F32)
    m = np.full((Hq, nb, nb), -np.inf, F32)
    for h in range(Hq):
        for i in range(nb):
            for j in range(i + 1):
                vals = []
                for r in range(block):
                    pos = block * i + r
                    if pos < block * j + block - 1:
                        continue
                    row = qd[pos, h] if pos < S else np.zeros(d)
                    dot = F32(math.fsum(float(row[x]) * float(kd[j, h // G, x]) for x in range(d)))
                    vals.append(F32(dot * c))
                mm = max(vals)
                m[h, i, j] = mm
                p[h, i, j] = F32(math.fsum(2.0 ** float(F32(v - mm)) for v in vals))
    return p, m


@pytest.mark.parametrize("S,block,Hq,Hkv,d", [(300, 128, 2, 1, 8), (100, 16, 4, 2, 8),
                                              (64, 16, 2, 2, 16)])
def test_block_score_brute_force(S, block, Hq, Hkv, d):
    q = _rand((S, Hq, d), 3, torch.bfloat16, 2.0)
    k = _rand((S, Hkv, d), 4, torch.bfloat16, 2.0)
    mk = O.pool_k(k, block)
    p, m = O.block_score(q, mk, block)
    bp, bm = _brute_block_score(q, mk, block)
    np.testing.assert_array_equal(m.numpy(), bm)
    np.testing.assert_allclose(p.numpy(), bp, rtol=1e-6, atol=0)


def test_block_score_diagonal_uses_row_127_only():
    S, block = 384, 128
    q = _rand((S, 2, 16), 5, torch.bfloat16, 3.0)
    k = _rand((S, 1, 16), 6, torch.bfloat16, 3.0)
    mk = O.pool_k(k, block)
    p, m = O.block_score(q, mk, block)
    c = _c(16)
    for i in range(3):
        assert p[0, i, i].item() == 1.0  # a single row: exp2(0)
        dot = F32(float(q[block * i + 127, 0].double() @ mk[i, 0].double()))
        assert m[0, i, i].item() == float(F32(dot * c))
    # planted mistake: using all 128 rows on the diagonal gives p_ii > 1
    s_all = (q[0:128, 0].double() @ mk[0, 0].double()).float() * c
    p_all = torch.exp2((s_all - s_all.max()).double()).sum()
    assert p_all.item() > 1.5


def test_block_score_padding_rows_count_below_diagonal():
    # S = 130: q-block 1 has 2 real rows and 126 zero rows; for j = 0 all 128 rows count.
    S, block = 130, 128
    q = _rand((S, 1, 8), 7, torch.float32, 4.0)
    k = _rand((S, 1, 8), 8, torch.float32, 4.0)
    mk = O.pool_k(k, block)
    p, m = O.block_score(q, mk, block)
    bp, bm = _brute_block_score(q, mk, block)
    np.testing.assert_allclose(p.numpy(), bp, rtol=1e-6)
    # planted mistake: skipping the 126 zero rows changes p_10 (they add exp2(0 - m))
    c = _c(8)
    s_real = (q[128:130, 0].double() @ mk[0, 0].double()).float() * c
    mm = max(s_real.max().item(), 0.0)
    p_wrong = torch.exp2(s_real.double() - mm).sum().item()
    assert m[0, 1, 0].item() == F32(mm)
    assert abs(p[0, 1, 0].item() - p_wrong) > 1e-3 * p_wrong
    # j == i == 1 uses row 255, a padding row: s = 0
    assert m[0, 1, 1].item() == 0.0 and p[0, 1, 1].item() == 1.0


# --------------------------------------------------------------------------
# a3 + a4 normalisation and selection: brute force loops
# --------------------------------------------------------------------------

def _brute_select(p, m, native, alpha, sink, window, last_n):
    Hq, nb, _ = p.shape
    sel = np.zeros((Hq, nb, nb), bool)
    for h in range(Hq):
        for i in range(nb):
            M = max(F32(m[h, i, j]) for j in range(i + 1))
            S = [F32(F32(p[h, i, j]) * F32(2.0 ** float(F32(F32(m[h, i, j]) - M))))
                 for j in range(i + 1)]
            if native:
                denom = F32(F32(math.fsum(float(s) for s in S)) + F32(1e-9))
                S = [F32(s / denom) for s in S]
            thr = F32(max(S) * F32(alpha))
            for j in range(i + 1):
                sel[h, i, j] = bool(S[j] >= thr or j < sink or (i - j) < window or i >= nb - last_n)
    return sel


def _random_scores(Hq, nb, seed):
    g = torch.Generator().manual_seed(seed)
    m = (torch.randn(Hq, nb, nb, generator=g) * 3).float()
    p = (torch.rand(Hq, nb, nb, generator=g) * 127 + 1).float()
    tril = torch.tril(torch.ones(nb, nb, dtype=torch.bool))
    m = torch.where(tril, m, torch.tensor(float("-inf")))
    p = torch.where(tril, p, torch.zeros(()))
    return p, m


@pytest.mark.parametrize("native", [False, True])
@pytest.mark.parametrize("alpha,sink,window,last_n", [(0.18, 2, 4, 2), (0.7, 0, 1, 0),
                                                      (0.08, 3, 0, 1), (1.0, 0, 0, 0)])
def test_select_brute_force(native, alpha, sink, window, last_n):
    p, m = _random_scores(3, 12, 11)
    got = O.select_from_scores(p, m, native, alpha, sink, window, last_n)
    ref = _brute_select(p.numpy(), m.numpy(), native, alpha, sink, window, last_n)
    np.testing.assert_array_equal(got.numpy(), ref)


def test_select_invariants():
    p, m = _random_scores(4, 20, 12)
    sel = O.select_from_scores(p, m, False, 0.18, 2, 4, 2)
    nb = 20
    for i in range(nb):
        assert sel[:, i, i].all()                        # diagonal is in the window
        assert sel[:, i, :min(2, i + 1)].all()           # sinks
        assert not sel[:, i, i + 1:].any()               # causal
        assert sel[:, i, max(0, i - 3):i + 1].all()      # window 4
    assert sel[:, nb - 2:, :].sum() == 4 * sum(i + 1 for i in (nb - 2, nb - 1))  # last-n full


def test_select_planted_window_mistake():
    p, m = _random_scores(2, 10, 13)
    ref = _brute_select(p.numpy(), m.numpy(), False, 0.9, 0, 4, 0)
    wrong = _brute_select(p.numpy(), m.numpy(), False, 0.9, 0, 5, 0)
    assert (ref != wrong).any()


def test_min_budget_brute_force():
    p, m = _random_scores(2, 16, 14)
    S = O.normalize_scores(p, m, True)
    sel = O.select_blocks(S, 0.9, 0, 1, 0, min_budget=5)
    for h in range(2):
        for i in range(16):
            row = S[h, i, :i + 1]
            thr = F32(row.max().item() * F32(0.9))
            top = set(torch.argsort(row, descending=True, stable=True)[:5].tolist())
            want = {j for j in range(i + 1) if row[j].item() >= thr or j in top or j == i}
            assert set(torch.nonzero(sel[h, i]).flatten().tolist()) == want


# --------------------------------------------------------------------------
# a5 sparse attention: dense fp64 closed form and SDPA
# --------------------------------------------------------------------------

def _random_sel(Hq, nb, seed, density=0.4):
    g = torch.Generator().manual_seed(seed)
    sel = torch.rand(Hq, nb, nb, generator=g) < density
    sel |= torch.eye(nb, dtype=torch.bool).unsqueeze(0)
    return sel & torch.tril(torch.ones(nb, nb, dtype=torch.bool))


@pytest.mark.parametrize("S,dtype,tol", [(300, torch.float32, 2e-5), (384, torch.bfloat16, 1e-2)])
def test_sparse_attention_closed_form(S, dtype, tol):
    Hq, Hkv, d = 4, 2, 16
    q = _rand((S, Hq, d), 21, dtype, 1.5)
    k = _rand((S, Hkv, d), 22, dtype, 1.5)
    v = _rand((S, Hkv, d), 23, dtype)
    nb = (S + 127) // 128
    sel = _random_sel(Hq, nb, 24)
    got = O.sparse_attention(q, k, v, sel).double()
    ref = O.dense_masked_attention_fp64(q, k, v, sel)
    assert (got - ref).abs().max().item() < tol
    # planted mistake: without the in-block causal mask on the diagonal block
    qb = torch.arange(S) // 128
    allow = sel[:, qb][:, :, qb]
    wrong = torch.zeros_like(ref)
    for h in range(Hq):
        s = (q[:, h].double() @ k[:, h // 2].double().T) / d ** 0.5
        s = torch.where(allow[h], s, torch.tensor(float("-inf"), dtype=torch.float64))
        wrong[:, h] = torch.softmax(s, -1) @ v[:, h // 2].double()
    assert (wrong - ref).abs().max().item() > 10 * tol


def test_sparse_attention_all_blocks_equals_sdpa():
    S, Hq, Hkv, d = 320, 4, 1, 32
    q = _rand((S, Hq, d), 31)
    k = _rand((S, Hkv, d), 32)
    v = _rand((S, Hkv, d), 33)
    nb = 3
    sel = torch.tril(torch.ones(Hq, nb, nb, dtype=torch.bool))
    got = O.sparse_attention(q, k, v, sel).double()
    qq = q.double().permute(1, 0, 2)
    kk = k.double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
    vv = v.double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
    assert (got - ref.permute(1, 0, 2)).abs().max().item() < 1e-5


def test_sparse_attention_empty_list_gives_zero():
    # l starts at 1.0 and acc at 0, so a row with no blocks outputs exactly 0 (:282-284,333)
    q = _rand((128, 1, 8), 41)
    k = _rand((128, 1, 8), 42)
    v = _rand((128, 1, 8), 43)
    sel = torch.zeros(1, 1, 1, dtype=torch.bool)
    assert O.sparse_attention(q, k, v, sel).abs().max().item() == 0.0


# --------------------------------------------------------------------------
# a6 entry points and layouts
# --------------------------------------------------------------------------

def test_varlen_equals_per_sequence_native_without_division():
    # the varlen op is the per-sequence op with varlen normalisation
    g = torch.Generator().manual_seed(51)
    lens = [200, 33, 300]
    T = sum(lens)
    q = torch.randn(T, 4, 16, generator=g)
    k = torch.randn(T, 2, 16, generator=g)
    v = torch.randn(T, 2, 16, generator=g)
    cu = [0, 200, 233, 533]
    res = O.flash_prefill_varlen_func(q, k, v, cu, 300, 0.3)
    for b, (s0, s1) in enumerate(zip(cu[:-1], cu[1:])):
        o, tr = O.flashprefill_sequence(q[s0:s1], k[s0:s1], v[s0:s1], alpha=0.3, attention_sink=2,
                                        window=4, last_n=2, native=False)
        assert torch.equal(res.out[s0:s1], o)
        assert torch.equal(res.traces[b].sel, tr.sel)


def test_index_layouts():
    sel = _random_sel(3, 6, 61).unsqueeze(0)
    compact, counts = O.native_index_layout(sel)
    assert compact.shape == (1, 6, 6, 3) and counts.shape == (1, 6, 3)
    for i in range(6):
        for h in range(3):
            c = int(counts[0, i, h])
            js = torch.nonzero(sel[0, h, i]).flatten()
            assert torch.equal(compact[0, i, :c, h], js)
            assert (compact[0, i, c:, h] == 6).all()
    flat, cu = O.varlen_index_layout([sel[0]])
    assert cu[-1].item() == flat.numel() == int(sel.sum())
    # head-major then q-block then ascending j
    pos = 0
    for h in range(3):
        for i in range(6):
            js = torch.nonzero(sel[0, h, i]).flatten().to(torch.int32)
            assert torch.equal(flat[pos:pos + js.numel()], js)
            pos += js.numel()


@pytest.mark.parametrize("native", [False, True])
def test_rows_pipeline_equals_full_pipeline(native):
    # the bounded-sample helper used for CPU timing computes exactly the full rows
    g = torch.Generator().manual_seed(71)
    S, Hq, Hkv, d = 700, 4, 2, 32
    q = (torch.randn(S, Hq, d, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(S, Hkv, d, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(S, Hkv, d, generator=g).to(torch.bfloat16)
    out, tr = O.flashprefill_sequence(q, k, v, alpha=0.3, attention_sink=1, window=2, last_n=1,
                                      native=native)
    rows = [(h, i) for h in range(Hq) for i in range(6)]
    res = O.flashprefill_rows(q, k, v, rows, alpha=0.3, attention_sink=1, window=2, last_n=1,
                              native=native)
    for (h, i), (sel_row, o_row) in res.items():
        assert torch.equal(sel_row, tr.sel[h, i])
        assert torch.equal(o_row, out[i * 128:(i + 1) * 128, h])


def test_sparse_attention_key_tile_64_matches_closed_form():
    # the 64-key online-softmax tiling (the reference's other K_TILE_SIZE) is the same function
    S, Hq, Hkv, d = 300, 2, 1, 16
    q = _rand((S, Hq, d), 81, torch.float32, 1.5)
    k = _rand((S, Hkv, d), 82, torch.float32, 1.5)
    v = _rand((S, Hkv, d), 83)
    sel = _random_sel(Hq, 3, 84)
    got = O.sparse_attention(q, k, v, sel, k_tile=64).double()
    ref = O.dense_masked_attention_fp64(q, k, v, sel)
    assert (got - ref).abs().max().item() < 2e-5
