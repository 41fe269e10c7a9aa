"""Varlen FlashPrefill operator: drop-in for ``flash_prefill_varlen_func``
(``ops/flashprefill_varlen_func.py:722-743``), the entry point the vLLM patch
loaders call (``patches/patch_loader_vllm_0_12_0.py:187-199``,
``patches/patch_loader_vllm_0_10_0.py:246-258``).

Same arguments, defaults and in-place ``o`` semantics. The work runs on the
current torch stream through the C ABI (``include/flashprefill.h``): plan ->
pool K -> search (score + select) -> block-sparse attention, with no host
synchronisation (the reference syncs three times, :680,:696,:716).
"""

from __future__ import annotations

import torch

from .runtime import FlashPrefillCall


def _in_place_ok(t: torch.Tensor) -> bool:
    """Head dim contiguous and 16-byte aligned rows: the kernels read / write
    ``t`` where it is."""
    vec = 16 // t.element_size()
    return (t.stride(-1) == 1 and all(s % vec == 0 for s in t.stride()[:-1])
            and t.data_ptr() % 16 == 0)


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` itself when the kernels can read it in place, else a
    contiguous copy — the reference forces contiguity for the same purpose
    (``fla.utils.contiguous``, :580)."""
    return t if _in_place_ok(t) else t.contiguous()


@torch.no_grad()
def flash_prefill_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seq_len: int,
    alpha: float,
    block_size: int = 128,
    attention_sink: int = 2,
    window_size: int = 4,
    last_n_block: int = 2,
) -> None:
    """q (T, Hq, d), k/v (T, Hkv, d), o (T, Hq, d) written in place;
    cu_seqlens int32 (B+1,) token offsets; max_seq_len >= every length.

    Raises ValueError for malformed arguments and NotImplementedError for
    arguments the reference accepts but this build does not (head_dim other
    than 64 / 128 / 256, head_dim 256 with fp32 inputs or at block_size 256,
    block_size other than 64 / 128 / 256).
    """
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    target = o
    if not _in_place_ok(o):
        # the kernels write a copy of the caller's o; rows of sequences the
        # plan skips (status flags) keep the caller's values after copy-back
        o = torch.empty(o.shape, dtype=o.dtype, device=o.device).copy_(target)
    call = FlashPrefillCall(q, k, v, o, cu_seqlens, int(max_seq_len), alpha=float(alpha),
                            attention_sink=attention_sink, window_size=window_size,
                            last_n_block=last_n_block, native_normalize=False,
                            block_size=block_size, cached_workspace=True)
    call.run()
    if o is not target:
        target.copy_(o)


class FlashPrefill_varlen(torch.autograd.Function):
    """Class-level entry of the reference, which ``flash_prefill_varlen_func``
    wraps (``ops/flashprefill_varlen_func.py:577-720``, called at :739-743):
    ``FlashPrefill_varlen.apply(q, k, v, o, cu_seqlens, max_seq_len,
    block_size, k_stride, attention_sink, window, alpha, last_n_blocks)``.

    Forward only; writes ``o`` in place and returns None, as there.
    ``k_stride`` must equal ``block_size`` (:590; ValueError here, an assert
    there)."""

    @staticmethod
    def forward(ctx, q, k, v, o, cu_seqlens, max_seq_len, block_size=128, k_stride=128,
                attention_sink=2, window=4, alpha=0.7, last_n_blocks=2):
        if block_size != k_stride:
            raise ValueError(f"block_size ({block_size}) must equal k_stride ({k_stride})")
        flash_prefill_varlen_func(q, k, v, o, cu_seqlens, max_seq_len, alpha, block_size,
                                  attention_sink, window, last_n_blocks)
