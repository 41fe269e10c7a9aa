"""fp32 inputs on the GPU (fp32 MFMA kernels) against the oracle.

The reference runs fp32 q / k / v through the same Triton kernels, where
tl.dot of fp32 operands uses TF32; here pooling sums in fp64, scores and
attention use fp32 products with fp32 accumulation, and P stays fp32 before
P.V (its cast to V's dtype is the identity). Bars: pooled K within 1 fp32
ulp, scores within fp32 relative error, selection exact in both directions
from identical fp32 scores, output within max-abs 1e-4 / mean-abs 1e-5 of the
oracle (far inside the bf16 bar, and inside what TF32 would reach)."""

import pytest
import torch

from flashprefill_amd import flash_prefill, flash_prefill_varlen_func, synth
from oracle import flashprefill_oracle as O
from tests._parity import OUT_MAX_ABS_F32, OUT_MEAN_ABS_F32, assert_pool, run_stages

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check(rep, max_flip_frac=2e-3):
    print(f"\n  pool_ulp={rep.pool_ulp} pool_mismatch={rep.pool_mismatch} "
          f"m_rel={rep.m_max_rel:.2e} p_rel={rep.p_max_rel:.2e} "
          f"sel_mismatch(gpu scores)={rep.sel_from_gpu_scores_mismatch} "
          f"sel_mismatch(oracle scores)={rep.sel_from_oracle_scores_mismatch} "
          f"e2e_flips={rep.e2e_flips}/{rep.cells} density={rep.density:.3f} "
          f"out_max={rep.out_max_abs:.2e} out_mean={rep.out_mean_abs:.2e}", flush=True)
    assert_pool(rep)
    assert rep.m_max_rel < 1e-5
    assert rep.p_max_rel < 1e-4
    assert rep.sel_from_gpu_scores_mismatch == 0
    assert rep.sel_from_oracle_scores_mismatch == 0
    assert rep.e2e_flips <= max(2, max_flip_frac * rep.cells)
    assert rep.out_max_abs <= OUT_MAX_ABS_F32
    assert rep.out_mean_abs <= OUT_MEAN_ABS_F32


@pytest.mark.parametrize("alpha", [0.08, 0.12, 0.18, 0.7])
def test_config1_full_size_fp32(alpha):
    # config 1 at its own size and dtype: 4096 tokens, 8 q / 2 kv heads,
    # d = 64, fp32, unscaled N(0, 1) with sinks and 16 stripe columns, seed 0;
    # native normalisation as in the reference's native forward; the alphas
    # of the reference's Qwen2 / Qwen3-MoE / Llama callers and its class
    # default (ruler/models/qwen2.py:89, qwen3.py:126, llama.py:235,
    # ops/flashprefill_native_forward.py:410)
    spec = synth.config1_spec(seed=0)
    q, k, v, cu = synth.make_inputs(spec)
    assert q.dtype == torch.float32
    _check(run_stages(q, k, v, cu.tolist(), 4096, alpha=alpha, native=True))


@pytest.mark.parametrize("block", [128, 64])
def test_ragged_varlen_fp32_d128(block):
    g = torch.Generator().manual_seed(40 + block)
    lens = [300, 0, 128, 1, 640, 129]
    T = sum(lens)
    q = torch.randn(T, 8, 128, generator=g) * 1.5
    k = torch.randn(T, 2, 128, generator=g) * 1.5
    v = torch.randn(T, 2, 128, generator=g)
    cu = [0]
    for s in lens:
        cu.append(cu[-1] + s)
    _check(run_stages(q, k, v, cu, max(lens), alpha=0.18, block=block))


def test_native_min_budget_fp32_d64():
    g = torch.Generator().manual_seed(44)
    lens = [1000, 555]
    q = torch.randn(sum(lens), 4, 64, generator=g) * 2.0
    k = torch.randn(sum(lens), 4, 64, generator=g) * 2.0
    v = torch.randn(sum(lens), 4, 64, generator=g)
    _check(run_stages(q, k, v, [0, 1000, 1555], 1000, alpha=0.9, native=True, min_budget=6))


def test_public_entry_points_fp32():
    g = torch.Generator().manual_seed(45)
    B, S, Hq, Hkv, d = 2, 700, 8, 2, 64
    q = torch.randn(B, S, Hq, d, generator=g) * 1.5
    k = torch.randn(B, S, Hkv, d, generator=g) * 1.5
    v = torch.randn(B, S, Hkv, d, generator=g)
    out = torch.empty(B, S, Hq, d, device=DEV)
    flash_prefill(q.to(DEV), k.to(DEV), v.to(DEV), out, 128, 2, 4, 0.7, 2, 0)
    ref = O.flash_prefill(q, k, v, 128, 2, 4, 0.7, 2, 0).out
    o2 = torch.empty(B * S, Hq, d, device=DEV)
    cu = torch.tensor([0, S, 2 * S], dtype=torch.int32, device=DEV)
    flash_prefill_varlen_func(q.reshape(B * S, Hq, d).to(DEV), k.reshape(B * S, Hkv, d).to(DEV),
                              v.reshape(B * S, Hkv, d).to(DEV), o2, cu, S, 0.18)
    ref2 = O.flash_prefill_varlen_func(q.reshape(B * S, Hq, d), k.reshape(B * S, Hkv, d),
                                       v.reshape(B * S, Hkv, d), cu.cpu(), S, 0.18).out
    torch.cuda.synchronize()
    for got, want in ((out, ref), (o2, ref2)):
        dd = (got.cpu() - want).abs()
        print(f"\n  max {dd.max().item():.2e} mean {dd.mean().item():.2e}", flush=True)
        assert dd.max().item() <= OUT_MAX_ABS_F32 and dd.mean().item() <= OUT_MEAN_ABS_F32


def test_all_blocks_selected_fp32_is_dense_causal():
    g = torch.Generator().manual_seed(46)
    T, Hq, Hkv, d = 1000, 4, 1, 128
    q = torch.randn(T, Hq, d, generator=g) * 1.5
    k = torch.randn(T, Hkv, d, generator=g) * 1.5
    v = torch.randn(T, Hkv, d, generator=g)
    o = torch.empty(T, Hq, d, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    flash_prefill_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), o, cu, T, 0.0)
    torch.cuda.synchronize()
    qq = q.double().permute(1, 0, 2)
    kk = k.double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    vv = v.double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
    dd = (o.cpu().double() - ref.permute(1, 0, 2)).abs()
    print(f"\n  dense fp32 vs fp64 SDPA: max {dd.max().item():.2e} mean {dd.mean().item():.2e}")
    assert dd.max().item() <= OUT_MAX_ABS_F32 and dd.mean().item() <= OUT_MEAN_ABS_F32


def test_structured_8k_fp32_sparse_selection():
    # Llama head shapes and the structured distribution in fp32: a sparse
    # selection (sinks, stripes, band, hot blocks), sampled attention rows
    spec = synth.llama_spec(8192, seed=8, dtype=torch.float32)
    q, k, v, cu = synth.make_inputs(spec)
    rows = {0: [(0, 63), (9, 40), (17, 20), (31, 5), (4, 0)]}
    rep = run_stages(q, k, v, cu.tolist(), 8192, alpha=0.18, attn_rows=rows)
    assert rep.density < 0.6
    _check(rep)
