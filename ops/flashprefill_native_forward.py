"""Reference module path ops/flashprefill_native_forward.py (flash_prefill,
:480-499, and the FlashPrefill class it wraps, :405-476) backed by
flashprefill_amd."""

from flashprefill_amd.flashprefill_native_forward import FlashPrefill, flash_prefill

__all__ = ["FlashPrefill", "flash_prefill"]
