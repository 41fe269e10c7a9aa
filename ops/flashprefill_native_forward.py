"""Reference module path ops/flashprefill_native_forward.py (flash_prefill,
:480-499) backed by flashprefill_amd."""

from flashprefill_amd.flashprefill_native_forward import flash_prefill

__all__ = ["flash_prefill"]
