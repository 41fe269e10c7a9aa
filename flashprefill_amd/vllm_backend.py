"""vLLM attention-backend hook: FlashPrefill for prefill steps.

Two forwards, one per reference patch:

* ``make_forward`` / ``apply_patch``: vLLM's v1 engine
  (``patches/patch_loader_vllm_0_12_0.py:57-253``), described below;
* ``make_forward_v0`` / ``apply_patch_v0``: the v0 engine's backend
  (``patches/patch_loader_vllm_0_10_0.py:55-376``), whose metadata splits a
  batch into prefill tokens first and decode tokens after them.

The v1 forward mirrors what the 0.12 patch does to
``FlashAttentionImpl.forward``:

* write the step's key / value rows into the paged KV cache
  (``reshape_and_cache_flash``, :140-149) -- here the HIP kernel behind
  ``fp_kv_cache_write``;
* ``is_prefill = max_query_len > 1`` (:169): prefill batches go to
  ``flash_prefill_varlen_func`` over the step's own packed q / k / v with the
  per-model selection config (:186-200);
* decode batches (one query per sequence) go to a paged decode attention over
  the cache (:201-225, vLLM's ``flash_attn_varlen_func``);
* a profiling run (``attn_metadata is None``) zero-fills the output (:95-97),
  encoder attention and cascade attention are delegated unchanged (:104-114,
  :226-252), fused output quantisation is rejected (:90-93).

vLLM is not a dependency: the forward only touches the attributes of the
impl object and the metadata that the reference's forward reads, and the two
vLLM operations it cannot provide itself (decode over the paged cache, and
the encoder / cascade paths) are injected. ``apply_patch`` installs the
forward on vLLM's ``FlashAttentionImpl`` when vLLM is importable, or on any
class passed to it (the tests use stand-ins).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any, Callable, Dict, Optional

import torch

from . import _lib
from .flashprefill_varlen_func import flash_prefill_varlen_func

# Per-model selection configs of the reference patch
# (patches/patch_loader_vllm_0_12_0.py:13-40): block 128, sink 2, window 4,
# last 2 q-blocks dense; alpha per model family.
ATTENTION_CONFIGS: Dict[str, Dict[str, Any]] = {
    "flashprefill_llama": {"block_size": 128, "attention_sink": 2, "window_size": 4,
                           "alpha": 0.18, "last_n_full_block": 2},
    "flashprefill_qwen2": {"block_size": 128, "attention_sink": 2, "window_size": 4,
                           "alpha": 0.08, "last_n_full_block": 2},
    "flashprefill_qwen3moe": {"block_size": 128, "attention_sink": 2, "window_size": 4,
                              "alpha": 0.12, "last_n_full_block": 2},
}
DEFAULT_CONFIG = "flashprefill_qwen2"  # the reference patch's choice (:43)

_DTYPES = {torch.bfloat16: _lib.FP_DTYPE_BF16, torch.float16: _lib.FP_DTYPE_F16}


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Write key / value (tokens, Hkv, d) into the paged caches
    (num_blocks, block_size, Hkv, d) at ``slot_mapping`` (int64, one slot per
    token; the mapping's length is the number of tokens written, negative
    slots are padding and skipped), on the current stream."""
    if key.dtype not in _DTYPES or value.dtype != key.dtype or key_cache.dtype != key.dtype or \
            value_cache.dtype != key.dtype:
        raise NotImplementedError(
            f"kv-cache write supports bf16 / fp16 caches of the key dtype, got key {key.dtype}, "
            f"cache {key_cache.dtype} (fp8 caches are not built)")
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must have a contiguous head dimension")
    if key_cache.dim() != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be (num_blocks, block_size, num_kv_heads, head_dim)")
    nb, bs, hkv, d = key_cache.shape
    n = slot_mapping.numel()
    if key.shape[1:] != (hkv, d) or value.shape[1:] != (hkv, d) or key.shape[0] < n or \
            value.shape[0] < n:
        raise ValueError(f"key {tuple(key.shape)} / value {tuple(value.shape)} do not match the "
                         f"cache {tuple(key_cache.shape)} and {n} slots")
    slots = slot_mapping.to(dtype=torch.int64).contiguous()
    a = _lib.FpKvCacheArgs()
    a.key, a.value = key.data_ptr(), value.data_ptr()
    a.k_stride_tok, a.k_stride_head = key.stride(0), key.stride(1)
    a.v_stride_tok, a.v_stride_head = value.stride(0), value.stride(1)
    a.key_cache, a.value_cache = key_cache.data_ptr(), value_cache.data_ptr()
    a.kc_stride_block, a.kc_stride_slot, a.kc_stride_head = key_cache.stride()[:3]
    a.vc_stride_block, a.vc_stride_slot, a.vc_stride_head = value_cache.stride()[:3]
    a.slot_mapping = slots.data_ptr()
    a.num_tokens, a.num_blocks = n, nb
    a.block_size, a.num_kv_heads, a.head_dim = bs, hkv, d
    a.dtype = _DTYPES[key.dtype]
    lib = _lib.load()
    _lib.check(lib.fp_kv_cache_write(ctypes.byref(a),
                                     torch.cuda.current_stream(key.device).cuda_stream))


def paged_decode_attention(query: torch.Tensor, key_cache: torch.Tensor,
                           value_cache: torch.Tensor, out: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, seqused_k: torch.Tensor,
                           block_table: torch.Tensor, softmax_scale: float) -> None:
    """Decode attention over the paged cache (the role of vLLM's
    ``flash_attn_varlen_func`` with a block table in the reference's decode
    branch): every query row of sequence b attends causally to the first
    ``seqused_k[b]`` cached tokens, the last query sitting at position
    ``seqused_k[b] - 1``. torch GPU ops in fp32 (one small gather per
    sequence); it is the default when no vLLM decode op is injected, not part
    of the prefill path."""
    cu = cu_seqlens_q.tolist()
    used = seqused_k.tolist()
    _, bs, hkv, d = key_cache.shape
    hq = query.shape[1]
    g = hq // hkv
    for b in range(len(cu) - 1):
        q0, q1 = cu[b], cu[b + 1]
        nq, nk = q1 - q0, int(used[b])
        if nq == 0:
            continue
        nblk = (nk + bs - 1) // bs
        blocks = block_table[b, :nblk].long()
        k = key_cache[blocks].reshape(nblk * bs, hkv, d)[:nk].float()
        v = value_cache[blocks].reshape(nblk * bs, hkv, d)[:nk].float()
        q = query[q0:q1].float()  # (nq, hq, d)
        k = k.repeat_interleave(g, dim=1).permute(1, 2, 0).contiguous()  # (hq, d, nk)
        v = v.repeat_interleave(g, dim=1).permute(1, 0, 2).contiguous()  # (hq, nk, d)
        s = torch.matmul(q.permute(1, 0, 2).contiguous(), k) * softmax_scale  # (hq, nq, nk)
        qpos = torch.arange(nk - nq, nk, device=query.device).view(1, nq, 1)
        kpos = torch.arange(nk, device=query.device).view(1, 1, nk)
        s = s.masked_fill(kpos > qpos, float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1), v)  # (hq, nq, d)
        out[q0:q1] = o.permute(1, 0, 2).to(out.dtype)


@dataclass
class HookOps:
    """The operations the hooked forward calls; the defaults are this
    package's (KV-cache write kernel, FlashPrefill, torch paged decode).
    ``encoder`` and ``cascade`` take the impl and the reference's arguments
    and default to raising: they stay vLLM's."""
    cache_write: Callable[..., None] = reshape_and_cache
    prefill: Callable[..., None] = flash_prefill_varlen_func
    decode: Callable[..., None] = paged_decode_attention
    encoder: Optional[Callable[..., torch.Tensor]] = None
    cascade: Optional[Callable[..., torch.Tensor]] = None


def _is_encoder(attn_type) -> bool:
    """vLLM's AttentionType.ENCODER / ENCODER_ONLY ("encoder", "encoder_only";
    an enum member's name works too)."""
    name = str(getattr(attn_type, "value", attn_type)).lower().rsplit(".", 1)[-1]
    return name in ("encoder", "encoder_only")


def make_forward(cfg: Dict[str, Any], ops: Optional[HookOps] = None):
    """The FlashAttentionImpl.forward replacement, closed over the selection
    config ``cfg`` (one of ATTENTION_CONFIGS' values)."""
    ops = ops or HookOps()

    def flash_prefill_forward(self, layer, query, key, value, kv_cache, attn_metadata,
                              output=None, output_scale=None, output_block_scale=None):
        if output is None:
            raise ValueError("Output tensor must be provided.")
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quantization is not supported")
        if attn_metadata is None:  # profiling run
            return output.fill_(0)
        n = attn_metadata.num_actual_tokens
        if _is_encoder(getattr(self, "attn_type", "decoder")):
            if ops.encoder is None:
                raise NotImplementedError("encoder attention is left to vLLM's backend")
            return ops.encoder(self, query[:n], key[:n], value[:n], output[:n], attn_metadata,
                               layer)
        key_cache, value_cache = kv_cache.unbind(0)
        if getattr(self, "kv_sharing_target_layer_name", None) is None and key is not None \
                and value is not None:
            if str(getattr(self, "kv_cache_dtype", "auto")).startswith("fp8"):
                raise NotImplementedError("fp8 KV caches are not supported by this hook")
            ops.cache_write(key, value, key_cache, value_cache, attn_metadata.slot_mapping)
        if getattr(attn_metadata, "use_cascade", False):
            if ops.cascade is None:
                raise NotImplementedError("cascade attention is left to vLLM's backend")
            return ops.cascade(self, query[:n], key_cache, value_cache, output[:n],
                               attn_metadata, layer)
        if getattr(self, "dcp_world_size", 1) > 1:
            raise NotImplementedError("decode context parallelism is left to vLLM's backend")
        cu_seqlens_q = attn_metadata.query_start_loc
        if attn_metadata.max_query_len > 1:  # prefill
            ops.prefill(query[:n], key[:n], value[:n], output[:n], cu_seqlens_q,
                        attn_metadata.max_query_len, cfg["alpha"], cfg["block_size"],
                        cfg["attention_sink"], cfg["window_size"], cfg["last_n_full_block"])
        else:
            ops.decode(query[:n], key_cache, value_cache, output[:n], cu_seqlens_q,
                       attn_metadata.seq_lens, attn_metadata.block_table,
                       getattr(self, "scale", 1.0 / math.sqrt(query.shape[-1])))
        return output

    return flash_prefill_forward


def apply_patch(impl_cls=None, config: str = DEFAULT_CONFIG, ops: Optional[HookOps] = None):
    """Replace ``impl_cls.forward`` (default: vLLM's v1 FlashAttentionImpl)
    with the FlashPrefill forward for ``config``; returns the original forward.
    The reference's per-rank Triton cache directory (:49-54) has no
    counterpart: nothing is compiled at run time here."""
    if impl_cls is None:
        import vllm.v1.attention.backends.flash_attn as fa_backend  # noqa: WPS433
        impl_cls = fa_backend.FlashAttentionImpl
    cfg = ATTENTION_CONFIGS[config]
    if ops is None:
        ops = HookOps()
        try:  # inside vLLM, decode uses vLLM's own paged attention op
            from vllm.attention.utils.fa_utils import flash_attn_varlen_func as vllm_fa

            def vllm_decode(q, kc, vc, out, cu, seqused_k, block_table, scale):
                vllm_fa(q=q, k=kc, v=vc, out=out, cu_seqlens_q=cu, max_seqlen_q=1,
                        seqused_k=seqused_k, max_seqlen_k=int(seqused_k.max()),
                        softmax_scale=scale, causal=True, block_table=block_table)
            ops.decode = vllm_decode
        except ImportError:
            pass
    original = impl_cls.forward
    impl_cls.forward = make_forward(cfg, ops)
    return original


# ---------------------------------------------------------------------------
# vLLM v0 engine (patches/patch_loader_vllm_0_10_0.py)
# ---------------------------------------------------------------------------

def _is_decoder(attn_type) -> bool:
    name = str(getattr(attn_type, "value", attn_type)).lower().rsplit(".", 1)[-1]
    return name == "decoder"


def make_forward_v0(cfg: Dict[str, Any], ops: Optional[HookOps] = None):
    """The v0 engine's FlashAttentionImpl.forward replacement
    (patches/patch_loader_vllm_0_10_0.py:78-376), closed over ``cfg``:

    * the step's key / value rows go into the paged cache at ``slot_mapping``
      when the cache is allocated (:139-172); fp8 caches are rejected;
    * the batch's first ``num_prefill_tokens`` query rows are prefill, the
      ``num_decode_tokens`` after them decode (:186-195);
    * prefill without block tables (or with an empty cache) is FlashPrefill
      over the step's own rows, cu_seqlens = ``seq_start_loc`` and
      max_seq_len = ``max_prefill_seq_len`` (:197-246); prefill with block
      tables (prefix caching) is paged attention over the cache, queries
      ending at ``seq_lens_tensor`` (:270-295), ``ops.decode``'s operation;
    * decode is paged attention over the cache: varlen with
      ``query_start_loc`` when ``max_decode_query_len > 1`` (:313-339), one
      query per sequence otherwise (:340-368).

    Attention types other than decoder go to ``ops.encoder``, cache write
    included (the reference writes encoder-decoder layers through
    ``cross_slot_mapping`` and then runs them through the same causal
    FlashPrefill call, which only suits decoder layers); fused output
    quantisation is rejected (:108-111)."""
    ops = ops or HookOps()

    def flash_prefill_forward_v0(self, layer, query, key, value, kv_cache, attn_metadata,
                                 output=None, output_scale=None):
        if output is None:
            raise ValueError("Output tensor must be provided.")
        if output_scale is not None:
            raise NotImplementedError("fused output quantization is not supported")
        attn_type = getattr(self, "attn_type", "decoder")
        if not _is_decoder(attn_type):
            if ops.encoder is None:
                raise NotImplementedError("encoder and encoder-decoder attention are left to "
                                          "vLLM's backend")
            return ops.encoder(self, query, key, value, output, attn_metadata, layer)
        fp8 = str(getattr(self, "kv_cache_dtype", "auto")).startswith("fp8")
        if fp8:
            raise NotImplementedError("fp8 KV caches are not supported by this hook")
        scale = getattr(self, "scale", 1.0 / math.sqrt(query.shape[-1]))
        key_cache = value_cache = None
        if kv_cache.numel() > 0:
            key_cache, value_cache = kv_cache[0], kv_cache[1]
            if key is not None and value is not None:
                ops.cache_write(key, value, key_cache, value_cache,
                                attn_metadata.slot_mapping.flatten())
        n_pre = attn_metadata.num_prefill_tokens
        n_dec = attn_metadata.num_decode_tokens
        prefill_meta = attn_metadata.prefill_metadata
        if prefill_meta is not None:
            tables = getattr(prefill_meta, "block_tables", None)
            if kv_cache.numel() == 0 or tables is None or tables.numel() == 0:
                ops.prefill(query[:n_pre], key[:n_pre], value[:n_pre], output[:n_pre],
                            prefill_meta.seq_start_loc, prefill_meta.max_prefill_seq_len,
                            cfg["alpha"], cfg["block_size"], cfg["attention_sink"],
                            cfg["window_size"], cfg["last_n_full_block"])
            else:  # prefix caching: the new queries end each cached sequence
                ops.decode(query[:n_pre], key_cache, value_cache, output[:n_pre],
                           prefill_meta.query_start_loc, prefill_meta.seq_lens_tensor, tables,
                           scale)
        decode_meta = attn_metadata.decode_metadata
        if decode_meta is not None:
            dq = query[n_pre:n_pre + n_dec]
            dout = output[n_pre:n_pre + n_dec]
            if (decode_meta.max_decode_query_len or 1) > 1:
                cu = decode_meta.query_start_loc
            else:  # one query per sequence
                cu = torch.arange(decode_meta.seq_lens_tensor.numel() + 1, dtype=torch.int32,
                                  device=query.device)
            ops.decode(dq, key_cache, value_cache, dout, cu, decode_meta.seq_lens_tensor,
                       decode_meta.block_tables, scale)
        return output

    return flash_prefill_forward_v0


def apply_patch_v0(impl_cls=None, config: str = DEFAULT_CONFIG, ops: Optional[HookOps] = None):
    """Replace ``impl_cls.forward`` (default: the v0 engine's
    FlashAttentionImpl, imported from either module path the reference tries,
    patch_loader_vllm_0_10_0.py:57-61) with the v0 FlashPrefill forward for
    ``config``; returns the original forward."""
    if impl_cls is None:
        try:
            import vllm.attention.backends.flash_attn as fa_backend  # noqa: WPS433
        except ImportError:
            import vllm.model_executor.layers.attention.backends.flash_attn as fa_backend  # noqa
        impl_cls = fa_backend.FlashAttentionImpl
    if ops is None:
        ops = HookOps()
        try:  # inside vLLM, paged attention is vLLM's own op (patch :19-20, :270-368)
            from vllm.vllm_flash_attn import flash_attn_varlen_func as vllm_fa

            def vllm_paged(q, kc, vc, out, cu, seqused_k, block_table, scale):
                max_q = int((cu[1:] - cu[:-1]).max())
                vllm_fa(q=q, k=kc, v=vc, out=out, cu_seqlens_q=cu, max_seqlen_q=max_q,
                        seqused_k=seqused_k, max_seqlen_k=int(seqused_k.max()),
                        softmax_scale=scale, causal=True, block_table=block_table)
            ops.decode = vllm_paged
        except ImportError:
            pass
    original = impl_cls.forward
    impl_cls.forward = make_forward_v0(ATTENTION_CONFIGS[config], ops)
    return original
