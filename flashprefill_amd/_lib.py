"""ctypes binding of the C ABI in ``include/flashprefill.h``.

The shared library is built in-tree by ``flashprefill_amd.build``; loading
fails loudly if it is missing (there is no CPU fallback). ``torch`` is
imported first so that the library binds to the HIP runtime torch already
loaded (same SONAME), i.e. torch's streams and device pointers are valid in
the library.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "libflashprefill.so"

FP_OK = 0
FP_E_INVALID_ARG = -1
FP_E_UNSUPPORTED = -2
FP_E_LAUNCH = -3
FP_DTYPE_BF16 = 0
FP_DTYPE_F16 = 1
FP_DTYPE_F32 = 2
FP_STATUS_SEQ_TOO_LONG = 1
FP_STATUS_BAD_CU_SEQLENS = 2
ABI_VERSION = 6

EXPORTS = (
    "fp_workspace_layout", "fp_workspace_bytes", "fp_flashprefill", "fp_plan", "fp_pool_k",
    "fp_search", "fp_select", "fp_sparse_attn_fwd", "fp_read_status", "fp_last_error",
    "fp_abi_version", "fp_flashprefill_noalloc", "fp_kv_cache_write", "fp_rope_qk",
)
NOALLOC_SCRATCH_BYTES = 96 * 1024 * 1024


class FpProblem(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_stride_tok", ctypes.c_int64), ("q_stride_head", ctypes.c_int64),
        ("k_stride_tok", ctypes.c_int64), ("k_stride_head", ctypes.c_int64),
        ("v_stride_tok", ctypes.c_int64), ("v_stride_head", ctypes.c_int64),
        ("o_stride_tok", ctypes.c_int64), ("o_stride_head", ctypes.c_int64),
        ("cu_seqlens", ctypes.c_void_p),
        ("batch", ctypes.c_int32), ("uniform_seq_len", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("total_tokens", ctypes.c_int64),
        ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("attention_sink", ctypes.c_int32), ("window_size", ctypes.c_int32),
        ("last_n_block", ctypes.c_int32), ("native_normalize", ctypes.c_int32),
        ("min_budget", ctypes.c_int32),
    ]


class FpWsLayout(ctypes.Structure):
    _fields_ = [
        ("total_bytes", ctypes.c_size_t), ("status_off", ctypes.c_size_t),
        ("seq_tile_off", ctypes.c_size_t), ("seq_tri_off", ctypes.c_size_t),
        ("seq_start_off", ctypes.c_size_t), ("seq_len_off", ctypes.c_size_t),
        ("items_off", ctypes.c_size_t),
        ("mk_off", ctypes.c_size_t),
        ("cnt_off", ctypes.c_size_t), ("rowrec_off", ctypes.c_size_t),
        ("idx_off", ctypes.c_size_t), ("units_off", ctypes.c_size_t),
        ("part_off", ctypes.c_size_t),
        ("nb_sum_cap", ctypes.c_int64), ("tri_cap", ctypes.c_int64),
        ("unit_cap", ctypes.c_int64),
        ("nb_max", ctypes.c_int32), ("split_blocks", ctypes.c_int32),
    ]


class FpRopeArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride_tok", ctypes.c_int64), ("q_stride_head", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_stride_tok", ctypes.c_int64), ("k_stride_head", ctypes.c_int64),
        ("positions", ctypes.c_void_p), ("num_tokens", ctypes.c_int64),
        ("cos_table", ctypes.c_void_p), ("sin_table", ctypes.c_void_p),
        ("num_positions", ctypes.c_int64),
        ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p), ("eps", ctypes.c_float),
        ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32),
    ]


class FpKvCacheArgs(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_void_p), ("value", ctypes.c_void_p),
        ("k_stride_tok", ctypes.c_int64), ("k_stride_head", ctypes.c_int64),
        ("v_stride_tok", ctypes.c_int64), ("v_stride_head", ctypes.c_int64),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("kc_stride_block", ctypes.c_int64), ("kc_stride_slot", ctypes.c_int64),
        ("kc_stride_head", ctypes.c_int64),
        ("vc_stride_block", ctypes.c_int64), ("vc_stride_slot", ctypes.c_int64),
        ("vc_stride_head", ctypes.c_int64),
        ("slot_mapping", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int64), ("num_blocks", ctypes.c_int64),
        ("block_size", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32),
    ]


_LIB = None


def load(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the library with argument types declared."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not path.exists():
        raise RuntimeError(
            f"{path.name} is not built ({path}); run `python -m flashprefill_amd.build` "
            "(the FlashPrefill GPU path has no fallback)")
    lib = ctypes.CDLL(str(path))
    P = ctypes.POINTER(FpProblem)
    vp = ctypes.c_void_p
    fp = ctypes.POINTER(ctypes.c_float)
    lib.fp_workspace_layout.argtypes = [P, ctypes.POINTER(FpWsLayout)]
    lib.fp_workspace_bytes.argtypes = [P]
    lib.fp_workspace_bytes.restype = ctypes.c_size_t
    for name in ("fp_flashprefill", "fp_plan", "fp_pool_k", "fp_sparse_attn_fwd"):
        getattr(lib, name).argtypes = [P, vp, vp]
    lib.fp_flashprefill_noalloc.argtypes = [P, vp]
    lib.fp_kv_cache_write.argtypes = [ctypes.POINTER(FpKvCacheArgs), vp]
    lib.fp_rope_qk.argtypes = [ctypes.POINTER(FpRopeArgs), vp]
    lib.fp_search.argtypes = [P, vp, vp, vp, vp]
    lib.fp_select.argtypes = [P, vp, vp, vp, vp]
    lib.fp_read_status.argtypes = [P, vp, vp, ctypes.POINTER(ctypes.c_uint32)]
    lib.fp_last_error.restype = ctypes.c_char_p
    lib.fp_abi_version.restype = ctypes.c_int
    for name in EXPORTS:
        if name not in ("fp_workspace_bytes", "fp_last_error", "fp_abi_version"):
            getattr(lib, name).restype = ctypes.c_int
    if lib.fp_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path.name} ABI {lib.fp_abi_version()} != expected {ABI_VERSION}")
    _LIB = lib
    return lib


class FlashPrefillError(RuntimeError):
    pass


def check(rc: int) -> None:
    """Raise on a non-zero status: ValueError for invalid arguments,
    NotImplementedError for unsupported ones, RuntimeError otherwise."""
    if rc == FP_OK:
        return
    msg = load().fp_last_error().decode(errors="replace")
    if rc == FP_E_INVALID_ARG:
        raise ValueError(msg)
    if rc == FP_E_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise FlashPrefillError(msg)
