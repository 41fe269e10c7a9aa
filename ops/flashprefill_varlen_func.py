"""Reference module path ops/flashprefill_varlen_func.py
(flash_prefill_varlen_func, :722-743) backed by flashprefill_amd."""

from flashprefill_amd.flashprefill_varlen_func import flash_prefill_varlen_func

__all__ = ["flash_prefill_varlen_func"]
