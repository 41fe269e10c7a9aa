"""Prefill attention block around the FlashPrefill op: QKV projection ->
(optional per-head q/k RMSNorm) -> rotary embedding -> FlashPrefill sparse
attention (varlen signature) -> O projection.

This is the attention-module pattern of the reference's model callers
(ruler/models/llama.py:260-337 without the norms, ruler/models/qwen3.py:159-214
with q_norm / k_norm), written as one module over packed varlen tokens
``(T, hidden)`` so that the op is called exactly as the vLLM patch calls it
(patches/patch_loader_vllm_0_12_0.py:187-199). Q, K and V are views into one
fused QKV projection (the op takes strided inputs; no copies), RoPE uses the
rotate-half convention with per-sequence positions taken from ``cu_seqlens``.
The projections are plain library GEMMs (torch -> hipBLASLt).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .flashprefill_varlen_func import flash_prefill_varlen_func


def positions_from_cu_seqlens(cu_seqlens: torch.Tensor, total: int) -> torch.Tensor:
    """Position of every packed token inside its own sequence (int64, on the
    device of ``cu_seqlens``)."""
    cu = cu_seqlens.to(torch.int64)
    lens = cu[1:] - cu[:-1]
    starts = torch.repeat_interleave(cu[:-1], lens, output_size=total)
    return torch.arange(total, device=cu.device, dtype=torch.int64) - starts


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin of shape (T, head_dim) in fp32 for the rotate-half layout:
    angle(t, k) = pos_t * theta^(-2k/d) for k < d/2, repeated for the second half."""
    inv = theta ** (-torch.arange(0, head_dim, 2, device=positions.device,
                                  dtype=torch.float64) / head_dim)
    ang = positions.to(torch.float64).view(-1, 1) * inv.view(1, -1)
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().float(), ang.sin().float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x (T, H, d) -> x*cos + rotate_half(x)*sin, computed in fp32 and rounded
    once to x's dtype; returns a new contiguous tensor."""
    d = x.shape[-1]
    xf = x.float()
    rot = torch.cat([-xf[..., d // 2:], xf[..., :d // 2]], dim=-1)
    return (xf * cos.unsqueeze(1) + rot * sin.unsqueeze(1)).to(x.dtype)


def rms_norm_heads(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-head RMSNorm over the head dim (Qwen3 q_norm / k_norm), fp32 math."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


class PrefillAttention(torch.nn.Module):
    def __init__(self, hidden: int, num_q_heads: int, num_kv_heads: int, head_dim: int, *,
                 rope_theta: float = 1e6, qk_norm: bool = False, rms_eps: float = 1e-6,
                 alpha: float = 0.12, block_size: int = 128, attention_sink: int = 2,
                 window_size: int = 4, last_n_block: int = 2,
                 dtype: torch.dtype = torch.bfloat16, device=None, seed: Optional[int] = None):
        super().__init__()
        self.hidden, self.Hq, self.Hkv, self.d = hidden, num_q_heads, num_kv_heads, head_dim
        self.rope_theta, self.qk_norm, self.rms_eps = rope_theta, qk_norm, rms_eps
        self.alpha, self.block_size = alpha, block_size
        self.attention_sink, self.window_size, self.last_n_block = (attention_sink, window_size,
                                                                    last_n_block)
        g = torch.Generator().manual_seed(0 if seed is None else seed)
        nqkv = (num_q_heads + 2 * num_kv_heads) * head_dim
        # random init with unit-variance projections of unit-variance inputs
        self.w_qkv = torch.nn.Parameter(
            (torch.randn(nqkv, hidden, generator=g) / hidden ** 0.5).to(dtype).to(device),
            requires_grad=False)
        self.w_o = torch.nn.Parameter(
            (torch.randn(hidden, num_q_heads * head_dim, generator=g) /
             (num_q_heads * head_dim) ** 0.5).to(dtype).to(device), requires_grad=False)
        self.q_norm = torch.nn.Parameter(torch.ones(head_dim, dtype=dtype, device=device),
                                         requires_grad=False)
        self.k_norm = torch.nn.Parameter(torch.ones(head_dim, dtype=dtype, device=device),
                                         requires_grad=False)

    def project_qkv(self, x: torch.Tensor, cu_seqlens: torch.Tensor
                    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(T, hidden) -> rotated q (T, Hq, d), rotated k (T, Hkv, d) and v, a
        strided view into the fused projection."""
        T = x.shape[0]
        qkv = (x @ self.w_qkv.t()).view(T, self.Hq + 2 * self.Hkv, self.d)
        q = qkv[:, :self.Hq]
        k = qkv[:, self.Hq:self.Hq + self.Hkv]
        v = qkv[:, self.Hq + self.Hkv:]
        if self.qk_norm:
            q = rms_norm_heads(q, self.q_norm, self.rms_eps)
            k = rms_norm_heads(k, self.k_norm, self.rms_eps)
        cos, sin = rope_tables(positions_from_cu_seqlens(cu_seqlens, T), self.d, self.rope_theta)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v

    def forward(self, x: torch.Tensor, cu_seqlens: torch.Tensor, max_seq_len: int
                ) -> torch.Tensor:
        q, k, v = self.project_qkv(x, cu_seqlens)
        o = torch.empty_like(q)
        flash_prefill_varlen_func(q, k, v, o, cu_seqlens, max_seq_len, self.alpha,
                                  self.block_size, self.attention_sink, self.window_size,
                                  self.last_n_block)
        return o.view(x.shape[0], self.Hq * self.d) @ self.w_o.t()
