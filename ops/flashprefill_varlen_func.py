"""Reference module path ops/flashprefill_varlen_func.py
(flash_prefill_varlen_func, :722-743, and the FlashPrefill_varlen class it
wraps, :577-720) backed by flashprefill_amd."""

from flashprefill_amd.flashprefill_varlen_func import FlashPrefill_varlen, flash_prefill_varlen_func

__all__ = ["FlashPrefill_varlen", "flash_prefill_varlen_func"]
