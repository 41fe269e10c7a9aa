"""The decoder-layer block's fused q/k RMSNorm + RoPE kernel (fp_rope_qk)
against the torch composition of the same steps (RMSNorm in fp32 rounded to
the input dtype, times the weight rounded again as transformers'
Qwen3MoeRMSNorm does, then rotate-half RoPE with fp64-derived fp32 tables), on
ragged batches, bf16 and fp16, d 128 and 64, with and without the norms, on
the strided q / k views of a fused QKV projection. Without the norms the
result is the same bits. With them the fp32 sum of squares is reduced in
another order than torch's, so a normalised element can round one ulp apart,
and a rotation that nearly cancels turns that into a tiny output many ulps
away: there the bar is the absolute error at the row's scale (2 ulps of the
row's largest element)."""

import pytest
import torch

from flashprefill_amd.attention_layer import PrefillAttention, positions_from_cu_seqlens
from tests._parity import ulp_diff_16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,d,qk_norm", [(torch.bfloat16, 128, False),
                                              (torch.bfloat16, 128, True),
                                              (torch.float16, 64, True)])
def test_fused_rope_matches_torch_composition(dtype, d, qk_norm):
    dev = "cuda:0"
    lens = [3000, 1, 517, 4096]
    T = sum(lens)
    cu = torch.tensor([0, 3000, 3001, 3518, T], dtype=torch.int32, device=dev)
    layer = PrefillAttention(256, 8, 2, d, rope_theta=1e6, qk_norm=qk_norm, dtype=dtype,
                             device=dev, seed=7)
    if qk_norm:  # non-trivial norm weights
        g = torch.Generator(device=dev).manual_seed(3)
        layer.q_norm.copy_((torch.rand(d, generator=g, device=dev) + 0.5).to(dtype))
        layer.k_norm.copy_((torch.rand(d, generator=g, device=dev) + 0.5).to(dtype))
    g = torch.Generator(device=dev).manual_seed(11)
    x = (torch.randn(T, 256, generator=g, device=dev) * 2).to(dtype)
    q, k, v = layer.project_qkv(x, cu)  # fused kernel, in place on the projection
    qkv = (x @ layer.w_qkv.t()).view(T, 8 + 2 * 2, d)
    pos = positions_from_cu_seqlens(cu, T)
    q_ref, k_ref, _ = layer.project_qkv_reference(qkv[:, :8], qkv[:, 8:10], qkv[:, 10:], pos)
    torch.cuda.synchronize()
    uq, uk = ulp_diff_16(q.cpu(), q_ref.cpu()), ulp_diff_16(k.cpu(), k_ref.cpu())
    nq = int((q != q_ref).sum())
    print(f"\n  {dtype} d={d} qk_norm={qk_norm}: max ulp q {uq} k {uk}, differing q elements {nq}",
          flush=True)
    if not qk_norm:
        assert uq == 0 and uk == 0
    for got, ref in ((q, q_ref), (k, k_ref)):
        g32, r32 = got.float(), ref.float()
        row = r32.abs().amax(dim=-1, keepdim=True)
        bar = 2.0 ** (-6 if dtype == torch.bfloat16 else -9) * row  # 2 ulps at the row's scale
        assert bool(((g32 - r32).abs() <= bar).all())
    assert nq <= 1e-3 * q.numel()
    assert torch.equal(v, qkv[:, 10:])  # v untouched
