"""GPU test of the prefill attention block: the FlashPrefill call inside it
against the oracle on the block's own rotated q/k/v, and the whole block
against an fp32 composition of the same pieces."""

import pytest
import torch

from flashprefill_amd.attention_layer import PrefillAttention
from oracle import flashprefill_oracle as O
from tests._parity import OUT_MAX_ABS, OUT_MEAN_ABS

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qk_norm", [False, True])
def test_block_matches_oracle_composition(qk_norm):
    dev = "cuda:0"
    hidden, Hq, Hkv, d = 512, 8, 2, 128
    lens = [700, 300]
    T = sum(lens)
    cu = torch.tensor([0, 700, 1000], dtype=torch.int32, device=dev)
    layer = PrefillAttention(hidden, Hq, Hkv, d, qk_norm=qk_norm, alpha=0.12, device=dev, seed=4)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, hidden, generator=g).to(torch.bfloat16).to(dev)
    out = layer(x, cu, max(lens))
    q, k, v = layer.project_qkv(x, cu)
    torch.cuda.synchronize()
    # the op inside the block, against the oracle on the same q / k / v
    ref_attn = O.flash_prefill_varlen_func(q.cpu(), k.cpu(), v.contiguous().cpu(), cu.cpu(),
                                           max(lens), 0.12).out
    o = torch.empty_like(q)
    from flashprefill_amd import flash_prefill_varlen_func
    flash_prefill_varlen_func(q, k, v, o, cu, max(lens), 0.12)
    torch.cuda.synchronize()
    da = (o.float().cpu() - ref_attn.float()).abs()
    assert da.max().item() <= OUT_MAX_ABS and da.mean().item() <= OUT_MEAN_ABS
    # the block = O projection of that attention (fp32 GEMM of bf16 operands)
    want = ref_attn.float().reshape(T, Hq * d) @ layer.w_o.float().cpu().t()
    dl = (out.float().cpu() - want).abs()
    scale = want.abs().mean().item()
    print(f"\n  block out max {dl.max().item():.3e} mean {dl.mean().item():.3e} (|out| mean {scale:.3e})")
    assert dl.mean().item() <= 2e-2 * scale
    assert not torch.isnan(out).any()
