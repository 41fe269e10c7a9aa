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
The projections are plain library GEMMs (torch -> hipBLASLt). On the GPU
the q/k RMSNorm and RoPE run as one HIP kernel in place on the projection
(``fp_rope_qk``; the torch functions below are its reference and produce the
same bits).
"""

from __future__ import annotations

from typing import Optional, Tuple

import ctypes

import torch

from . import _lib
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


_TABLES = {}


def rope_position_tables(num_positions: int, head_dim: int, theta: float, device
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin per position (num_positions, head_dim / 2), fp32 from fp64
    angles (the values rope_tables repeats for both halves), cached per
    (size, head_dim, theta, device); grown to the next power of two."""
    n = 1 << max(int(num_positions) - 1, 1).bit_length()
    key = (head_dim, float(theta), str(torch.device(device)))
    hit = _TABLES.get(key)
    if hit is None or hit[0].shape[0] < n:
        pos = torch.arange(n, device=device, dtype=torch.float64)
        inv = theta ** (-torch.arange(0, head_dim, 2, device=device, dtype=torch.float64) / head_dim)
        ang = pos.view(-1, 1) * inv.view(1, -1)
        hit = (ang.cos().float().contiguous(), ang.sin().float().contiguous())
        _TABLES[key] = hit
    return hit


def fused_rope_qk(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, theta: float,
                  q_norm: Optional[torch.Tensor] = None, k_norm: Optional[torch.Tensor] = None,
                  eps: float = 1e-6, max_position: Optional[int] = None) -> None:
    """RMSNorm (when the weights are given) and RoPE of q (T, Hq, d) and k
    (T, Hkv, d) in place with the HIP kernel (bf16 / fp16 on the GPU; no
    fallback). ``positions`` (T,) int64 on the same device."""
    T, Hq, d = q.shape
    n = int(max_position) if max_position is not None else int(positions.max().item()) + 1
    cos, sin = rope_position_tables(max(n, 1), d, theta, q.device)
    a = _lib.FpRopeArgs()
    a.q, a.q_stride_tok, a.q_stride_head = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_tok, a.k_stride_head = k.data_ptr(), k.stride(0), k.stride(1)
    a.positions, a.num_tokens = positions.data_ptr(), T
    a.cos_table, a.sin_table, a.num_positions = cos.data_ptr(), sin.data_ptr(), cos.shape[0]
    a.q_norm = q_norm.data_ptr() if q_norm is not None else None
    a.k_norm = k_norm.data_ptr() if k_norm is not None else None
    a.eps = eps
    a.num_q_heads, a.num_kv_heads, a.head_dim = Hq, k.shape[1], d
    a.dtype = {torch.bfloat16: _lib.FP_DTYPE_BF16, torch.float16: _lib.FP_DTYPE_F16}[q.dtype]
    _lib.check(_lib.load().fp_rope_qk(ctypes.byref(a),
                                      torch.cuda.current_stream(q.device).cuda_stream))


def rms_norm_heads(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-head RMSNorm over the head dim (Qwen3 q_norm / k_norm,
    ruler/models/qwen3.py:171-172): fp32 math, the normalised row cast to the
    input dtype, then multiplied by the weight in that dtype (the composition
    of transformers' Qwen3MoeRMSNorm, so two roundings)."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return weight * y.to(x.dtype)


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
        pos = positions_from_cu_seqlens(cu_seqlens, T)
        if qkv.is_cuda and qkv.dtype in (torch.bfloat16, torch.float16):
            # one kernel, in place on the projection (q and k stay views of it)
            fused_rope_qk(q, k, pos, self.rope_theta,
                          self.q_norm if self.qk_norm else None,
                          self.k_norm if self.qk_norm else None, self.rms_eps,
                          max_position=T)
            return q, k, v
        return self.project_qkv_reference(q, k, v, pos)

    def project_qkv_reference(self, q, k, v, pos):
        """The torch composition of the same steps (the fused kernel's
        reference): RMSNorm rounded to the input dtype, then RoPE."""
        if self.qk_norm:
            q = rms_norm_heads(q, self.q_norm, self.rms_eps)
            k = rms_norm_heads(k, self.k_norm, self.rms_eps)
        cos, sin = rope_tables(pos, self.d, self.rope_theta)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v

    def forward(self, x: torch.Tensor, cu_seqlens: torch.Tensor, max_seq_len: int
                ) -> torch.Tensor:
        q, k, v = self.project_qkv(x, cu_seqlens)
        o = torch.empty_like(q)
        flash_prefill_varlen_func(q, k, v, o, cu_seqlens, max_seq_len, self.alpha,
                                  self.block_size, self.attention_sink, self.window_size,
                                  self.last_n_block)
        return o.view(x.shape[0], self.Hq * self.d) @ self.w_o.t()
