// Paged KV-cache write for the vLLM-style backend hook: the key and value row
// of every token go to the cache slot slot_mapping[t], i.e. block
// slot / block_size, offset slot % block_size (the write the reference's
// vLLM patch makes with reshape_and_cache_flash before each attention call,
// patches/patch_loader_vllm_0_12_0.py:140-149). Slots < 0 are padding tokens
// and are skipped, as are slots past the cache.
//
// HBM-bound byte copy: one workgroup per token moves its K and V rows
// (num_kv_heads x head_dim elements each) in 16-byte chunks; algorithmic
// bytes per token = 2 (K, V) x num_kv_heads x head_dim x elem_bytes, read
// once and written once.
#include "fp_internal.h"

namespace fp {

__global__ __launch_bounds__(256) void k_kv_cache_write(KvCacheArgs a) {
  const int64_t t = blockIdx.x;
  if (t >= a.num_tokens) return;
  const int64_t slot = a.slot_mapping[t];
  if (slot < 0 || slot >= a.num_slots) return;
  const int64_t blk = slot / a.block_size, off = slot % a.block_size;
  const int cpr = a.row_bytes / 16;  // 16-byte chunks per head row
  const int per = a.num_kv_heads * cpr;
  for (int c = threadIdx.x; c < 2 * per; c += blockDim.x) {
    const bool is_v = c >= per;
    const int cc = is_v ? c - per : c;
    const int h = cc / cpr, x = cc % cpr;
    const char* src = static_cast<const char*>(is_v ? a.value : a.key) +
                      (t * (is_v ? a.v_stride_tok : a.k_stride_tok) +
                       h * (is_v ? a.v_stride_head : a.k_stride_head)) * a.elem_bytes;
    char* dst = static_cast<char*>(is_v ? a.value_cache : a.key_cache) +
                (blk * (is_v ? a.vc_stride_block : a.kc_stride_block) +
                 off * (is_v ? a.vc_stride_slot : a.kc_stride_slot) +
                 h * (is_v ? a.vc_stride_head : a.kc_stride_head)) * a.elem_bytes;
    st16(dst + 16 * x, ld16(src + 16 * x));
  }
}

hipError_t launch_kv_cache_write(const KvCacheArgs& a, hipStream_t s) {
  if (a.num_tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_kv_cache_write, dim3(static_cast<unsigned>(a.num_tokens)), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

}  // namespace fp
