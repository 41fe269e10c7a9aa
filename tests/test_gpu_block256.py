"""GPU parity at block_size 256 (ops/flashprefill_native_forward.py:219-225
admits any block of at least the 64 / 128-token tiles; the reference's own
callers all pass 128).

Here block_size 256 pools K, scores and selects 256-token blocks and writes
each 256-row's selection as the index lists of its two 128-token plan rows;
the attention runs on those lists in 128-key tiles, as the reference's
kernels walk a 256-block in K tiles of at most 128 keys. The stage checks
are those of test_gpu_parity.py, against the oracle at block 256 (pooled K,
scores and selection over 256-token blocks, attention in 128-key tiles),
plus: the plan-granularity lists equal the expansion of the 256-token
selection exactly (tests/_parity.py run_stages).
"""

import pytest
import torch

from flashprefill_amd import flash_prefill, flash_prefill_varlen_func, synth
from oracle import flashprefill_oracle as O
from tests._parity import OUT_MAX_ABS, OUT_MEAN_ABS, assert_pool, run_stages

pytestmark = pytest.mark.gpu


def _check(rep, max_flip_frac=2e-3):
    print(f"\n  pool_ulp={rep.pool_ulp} pool_mismatch={rep.pool_mismatch} "
          f"m_rel={rep.m_max_rel:.2e} p_rel={rep.p_max_rel:.2e} "
          f"sel_mismatch(gpu scores)={rep.sel_from_gpu_scores_mismatch} "
          f"sel_mismatch(oracle scores)={rep.sel_from_oracle_scores_mismatch} "
          f"e2e_flips={rep.e2e_flips}/{rep.cells} density={rep.density:.3f} "
          f"out_max={rep.out_max_abs:.2e} out_mean={rep.out_mean_abs:.2e} {rep.notes}",
          flush=True)
    assert_pool(rep)
    assert rep.m_max_rel < 1e-4
    assert rep.p_max_rel < 1e-3
    assert rep.sel_from_gpu_scores_mismatch == 0
    assert rep.sel_from_oracle_scores_mismatch == 0
    assert rep.e2e_flips <= max(2, max_flip_frac * rep.cells)
    assert rep.out_max_abs <= OUT_MAX_ABS
    assert rep.out_mean_abs <= OUT_MEAN_ABS


def _rand_inputs(lens, Hq, Hkv, d, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = (torch.randn(T, Hq, d, generator=g) * scale).to(dtype)
    k = (torch.randn(T, Hkv, d, generator=g) * scale).to(dtype)
    v = torch.randn(T, Hkv, d, generator=g).to(dtype)
    cu = [0]
    for s in lens:
        cu.append(cu[-1] + s)
    return q, k, v, cu


@pytest.mark.parametrize("native", [False, True])
def test_ragged_varlen_bf16(native):
    # lengths with a 256-block whose second half is missing (300, 129, 1), a
    # partial second half (700, 1000), whole blocks (256, 2048), and odd and
    # even numbers of 128-token plan blocks
    lens = [1000, 700, 300, 129, 256, 2048, 1]
    q, k, v, cu = _rand_inputs(lens, 8, 2, 128, torch.bfloat16, 31, scale=1.5)
    print(f"\n  block256 ragged bf16 native={native} lens={lens}", flush=True)
    _check(run_stages(q, k, v, cu, max(lens), alpha=0.18, native=native, block=256))


def test_fp16_d64_heads_not_multiple_of_8():
    # 28 q / 4 kv heads: the split dense rows merge in k_merge
    lens = [4096, 1555]
    q, k, v, cu = _rand_inputs(lens, 28, 4, 64, torch.float16, 32, scale=1.2)
    print(f"\n  block256 fp16 d64 lens={lens}", flush=True)
    _check(run_stages(q, k, v, cu, max(lens), alpha=0.08, block=256))


@pytest.mark.parametrize("min_budget", [3, 8])
def test_native_min_budget(min_budget):
    # structured inputs at alpha 0.9 with sink 1 and window 1: sparse rows in
    # which the budget forces blocks on
    spec = synth.SynthSpec(seq_lens=(6000, 1700), num_q_heads=4, num_kv_heads=1, head_dim=128,
                           seed=33)
    q, k, v, cu = synth.make_inputs(spec)
    print(f"\n  block256 native min_budget={min_budget}", flush=True)
    rep = run_stages(q, k, v, cu.tolist(), 6000, alpha=0.9, sink=1, window=1, native=True,
                     min_budget=min_budget, block=256)
    assert rep.density < 0.9
    _check(rep)


@pytest.mark.parametrize("native", [False, True])
def test_sparse_ragged_selection(native):
    # high alpha, sink 1, window 1: sparse rows whose lists expand into
    # non-adjacent 128-token block pairs; partial last blocks of both kinds
    lens = (8192, 5000, 2900, 333)
    spec = synth.SynthSpec(seq_lens=lens, num_q_heads=16, num_kv_heads=4, head_dim=128, seed=36)
    q, k, v, cu = synth.make_inputs(spec)
    rows = {0: [(0, 31), (5, 17), (15, 0)], 1: [(3, 19), (12, 10)], 2: [(9, 11)], 3: [(2, 1)]}
    print(f"\n  block256 sparse ragged native={native} lens={lens}", flush=True)
    rep = run_stages(q, k, v, cu.tolist(), max(lens), alpha=0.9, sink=1, window=1, native=native,
                     block=256, attn_rows=rows)
    assert rep.density < 0.7
    _check(rep)


def test_fp32_native_d64():
    lens = [4096, 900]
    q, k, v, cu = _rand_inputs(lens, 8, 2, 64, torch.float32, 34)
    print("\n  block256 fp32 d64 native", flush=True)
    _check(run_stages(q, k, v, cu, max(lens), alpha=0.18, native=True, block=256))


def test_structured_16k_every_row():
    # 64 selection rows (two 32-key score tiles per wave), persistent-size
    # attention grid, split dense rows; sampled rows against the oracle and
    # every row against the closed form from the GPU's lists
    spec = synth.llama_spec(16384, seed=16)
    q, k, v, cu = synth.make_inputs(spec)
    rows = {0: [(0, 63), (7, 40), (19, 5), (31, 0)]}
    print("\n  block256 llama 16K structured", flush=True)
    rep = run_stages(q, k, v, cu.tolist(), 16384, alpha=0.18, block=256, attn_rows=rows)
    assert rep.full_rows > 0
    _check(rep)


def test_public_entry_points_match_the_oracle():
    # the whole-operator calls (plan and pooling in one launch) at block 256
    dev = torch.device("cuda:0")
    lens = [1500, 640, 77]
    q, k, v, cu = _rand_inputs(lens, 8, 2, 128, torch.bfloat16, 35, scale=1.5)
    print("\n  block256 public varlen", flush=True)
    o = torch.empty_like(q, device=dev)
    flash_prefill_varlen_func(q.to(dev), k.to(dev), v.to(dev), o,
                              torch.tensor(cu, dtype=torch.int32, device=dev), max(lens), 0.18,
                              block_size=256)
    torch.cuda.synchronize()
    ref = O.flash_prefill_varlen_func(q, k, v, cu, max(lens), 0.18, block_size=256).out
    d = (o.cpu().float() - ref.float()).abs()
    print(f"  varlen out_max={float(d.max()):.2e} out_mean={float(d.mean()):.2e}", flush=True)
    assert float(d.max()) <= OUT_MAX_ABS and float(d.mean()) <= OUT_MEAN_ABS
    # batched (B, S, H, d), native normalisation
    print("  block256 public native", flush=True)
    qb = q[:1280].view(2, 640, 8, 128)
    kb = k[:1280].view(2, 640, 2, 128)
    vb = v[:1280].view(2, 640, 2, 128)
    ob = torch.empty_like(qb, device=dev)
    flash_prefill(qb.to(dev), kb.to(dev), vb.to(dev), ob, 256, 2, 4, 0.18, 2, 0)
    torch.cuda.synchronize()
    refb = O.flash_prefill(qb, kb, vb, 256, 2, 4, 0.18, 2, 0).out
    d = (ob.cpu().float() - refb.float()).abs()
    print(f"  native out_max={float(d.max()):.2e} out_mean={float(d.mean()):.2e}", flush=True)
    assert float(d.max()) <= OUT_MAX_ABS and float(d.mean()) <= OUT_MEAN_ABS
