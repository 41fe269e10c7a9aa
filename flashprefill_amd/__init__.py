"""MI355X (gfx950) FlashPrefill sparse-prefill attention.

Drop-in operator surface of qhfan/FlashPrefill ``ops/__init__.py``:
``flash_prefill_varlen_func`` (packed varlen, the vLLM entry point) and
``flash_prefill`` (batched, the HF entry point), backed by hand-written HIP
kernels behind the C ABI in ``include/flashprefill.h``.
"""

from .flashprefill_native_forward import flash_prefill
from .flashprefill_varlen_func import flash_prefill_varlen_func
from .runtime import FlashPrefillCall

__all__ = ["flash_prefill", "flash_prefill_varlen_func", "FlashPrefillCall"]
