"""Drop-in shim with the reference's module layout (ops/__init__.py:1-2): the
reference's callers keep ``from ops import flash_prefill_varlen_func,
flash_prefill`` and ``from ops.flashprefill_native_forward import
flash_prefill`` unchanged and get the gfx950 implementation."""

from .flashprefill_native_forward import flash_prefill
from .flashprefill_varlen_func import flash_prefill_varlen_func

__all__ = ["flash_prefill", "flash_prefill_varlen_func"]
