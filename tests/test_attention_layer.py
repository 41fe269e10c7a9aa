"""CPU tests of the prefill attention block's host-side pieces: per-sequence
positions, rotary embedding (closed form and the relative-position property),
per-head RMSNorm, and the fused QKV projection's views."""

import math

import pytest

import torch

from flashprefill_amd.attention_layer import (PrefillAttention, apply_rope,
                                              positions_from_cu_seqlens, rms_norm_heads,
                                              rope_tables)


def test_positions_restart_per_sequence():
    cu = torch.tensor([0, 3, 3, 7], dtype=torch.int32)
    assert positions_from_cu_seqlens(cu, 7).tolist() == [0, 1, 2, 0, 1, 2, 3]


def test_rope_matches_closed_form():
    g = torch.Generator().manual_seed(0)
    T, H, d, theta = 37, 3, 16, 1e6
    x = torch.randn(T, H, d, generator=g)
    pos = torch.arange(T) * 7 + 3
    cos, sin = rope_tables(pos, d, theta)
    got = apply_rope(x, cos, sin).double()
    want = torch.empty(T, H, d, dtype=torch.float64)
    for t in range(T):
        for k in range(d // 2):
            a = float(pos[t]) * theta ** (-2.0 * k / d)
            c, s = math.cos(a), math.sin(a)
            lo, hi = x[t, :, k].double(), x[t, :, k + d // 2].double()
            want[t, :, k] = lo * c - hi * s
            want[t, :, k + d // 2] = hi * c + lo * s
    assert (got - want).abs().max().item() < 1e-5


def test_rope_scores_depend_on_relative_position_only():
    g = torch.Generator().manual_seed(1)
    d = 32
    q = torch.randn(1, 1, d, generator=g)
    k = torch.randn(1, 1, d, generator=g)
    dots = []
    for t in (5, 105, 1005):
        cq, sq = rope_tables(torch.tensor([t + 9]), d, 1e4)
        ck, sk = rope_tables(torch.tensor([t]), d, 1e4)
        dots.append(float((apply_rope(q, cq, sq) * apply_rope(k, ck, sk)).sum()))
    assert max(dots) - min(dots) < 1e-4 * max(1.0, abs(dots[0]))


def test_rms_norm_heads_closed_form():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 2, 8, generator=g)
    w = torch.randn(8, generator=g)
    got = rms_norm_heads(x, w, 1e-6)
    want = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    assert torch.allclose(got, want, atol=1e-6)


def test_qkv_projection_views_share_storage():
    layer = PrefillAttention(64, 4, 2, 16, dtype=torch.float32, seed=3)
    x = torch.randn(10, 64)
    cu = torch.tensor([0, 6, 10], dtype=torch.int32)
    q, k, v = layer.project_qkv(x, cu)
    assert q.shape == (10, 4, 16) and k.shape == (10, 2, 16) and v.shape == (10, 2, 16)
    assert not v.is_contiguous() and v.stride(-1) == 1  # a view into the fused projection
    full = x @ layer.w_qkv.t()
    assert torch.allclose(v.reshape(10, -1), full[:, 6 * 16:])


def test_rms_norm_heads_bit_equal_to_transformers_qwen3_moe_rmsnorm():
    # the reference's Qwen3 attention applies q_norm / k_norm
    # (ruler/models/qwen3.py:171-172), transformers' Qwen3MoeRMSNorm: the
    # normalised row is cast to the input dtype before the weight multiply
    mod = pytest.importorskip("transformers.models.qwen3_moe.modeling_qwen3_moe")
    g = torch.Generator().manual_seed(4)
    for dtype in (torch.bfloat16, torch.float16):
        x = (torch.randn(64, 4, 128, generator=g) * 3).to(dtype)
        norm = mod.Qwen3MoeRMSNorm(128, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(torch.rand(128, generator=g) * 2)
        norm = norm.to(dtype)
        want = norm(x)
        got = rms_norm_heads(x, norm.weight.detach(), 1e-6)
        assert got.dtype == dtype
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        # one rounding (the weight multiply in fp32) differs on many elements
        xf = x.float()
        once = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) *
                norm.weight.float()).to(dtype)
        assert not torch.equal(once, want)
