"""Batched FlashPrefill operator: drop-in for ``flash_prefill``
(``ops/flashprefill_native_forward.py:480-499``), the entry point of the HF
model callers (``ruler/models/llama.py:303``, ``ruler/models/qwen2.py:149``,
``ruler/models/qwen3.py:189``, ``patches/patch_qwen2_5_vl.py:58``,
``patches/patch_qwen3_moe_vl.py:49``).

Inputs are ``(B, S, H, d)`` (the code reads ``(b, s, h, d)``, :416, whatever
its docstring says). The batch is run as B sequences of S tokens through the
same kernels as the varlen entry point, with the native normalisation
``S /= (sum_j S + 1e-9)`` (:401).
"""

from __future__ import annotations

import torch

from .runtime import FlashPrefillCall


def _readable_in_place(t: torch.Tensor) -> bool:
    """True when (B, S, H, d) packs along tokens with the head dim contiguous
    and 16-byte aligned rows, so the kernels can use it without a copy."""
    S = t.shape[1]
    vec = 16 // t.element_size()
    return (t.stride(-1) == 1 and t.stride(0) == S * t.stride(1)
            and t.stride(1) % vec == 0 and t.stride(2) % vec == 0 and t.data_ptr() % 16 == 0)


def _packed_view(t: torch.Tensor) -> torch.Tensor:
    """(B, S, H, d) -> (B*S, H, d) view of ``t`` (or of a contiguous copy when
    ``t`` cannot be read in place; the reference forces contiguity, :408)."""
    B, S, H, d = t.shape
    src = t if _readable_in_place(t) else t.contiguous()
    return src.as_strided((B * S, H, d), (src.stride(1), src.stride(2), 1))


@torch.no_grad()
def flash_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    block_size: int,
    attention_sink: int,
    window_size: int,
    alpha: float,
    last_n_block_full: int,
    min_budget: int,
) -> None:
    """q (B, S, Hq, d), k/v (B, S, Hkv, d); ``out`` (B, S, Hq, d) written in place."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or out.dim() != 4:
        raise ValueError("flash_prefill expects (batch, seq, heads, head_dim) tensors")
    B, S, Hq, d = q.shape
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} != q shape {tuple(q.shape)}")
    q2, k2, v2 = _packed_view(q), _packed_view(k), _packed_view(v)
    direct = _readable_in_place(out)
    # a copy of the caller's out when the kernels cannot write it in place
    o2 = _packed_view(out) if direct else _packed_view(out.contiguous().clone())
    call = FlashPrefillCall(q2, k2, v2, o2, None, max(S, 1), alpha=float(alpha),
                            attention_sink=attention_sink, window_size=window_size,
                            last_n_block=last_n_block_full, native_normalize=True,
                            min_budget=min_budget, block_size=block_size, batch=B,
                            uniform_seq_len=S, cached_workspace=True)
    call.run()
    if not direct:
        out.copy_(o2.view(B, S, Hq, d))


class FlashPrefill(torch.autograd.Function):
    """Class-level entry of the reference, which ``flash_prefill`` wraps
    (``ops/flashprefill_native_forward.py:405-476``, called at :496-499):
    ``FlashPrefill.apply(q, k, v, out, block_size, k_stride, attention_sink,
    window, alpha, last_n_blocks_full, n_uniform, min_buget, topk)``.

    Forward only; writes ``out`` in place and returns None, as there.
    ``k_stride`` must equal ``block_size`` (:415; ValueError here, an assert
    there); ``n_uniform`` and ``topk`` are accepted and unused, as there;
    ``min_buget`` keeps the reference's spelling and is ``flash_prefill``'s
    ``min_budget``."""

    @staticmethod
    def forward(ctx, q, k, v, out, block_size=128, k_stride=128, attention_sink=2, window=4,
                alpha=0.7, last_n_blocks_full=2, n_uniform=0, min_buget=0, topk=0):
        if block_size != k_stride:
            raise ValueError(f"block_size ({block_size}) must equal k_stride ({k_stride})")
        flash_prefill(q, k, v, out, block_size, attention_sink, window, alpha,
                      last_n_blocks_full, min_buget)
