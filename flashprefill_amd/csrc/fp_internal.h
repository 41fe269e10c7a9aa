// Kernel argument blocks and launchers shared between the kernel files and the
// C ABI (fp_capi.hip). Pointers are device pointers into the caller's tensors
// or workspace; strides are in elements.
#pragma once

#include <type_traits>

#include "fp_common.h"

namespace fp {

struct PlanArgs {
  SeqTables tab;
  const int32_t* cu;  // nullable: uniform batch
  int32_t B;
  int32_t uniform_len;
  int32_t max_seq_len;
  int32_t nb_max;
  int64_t total_tokens;
  int64_t nb_sum_cap;  // workspace capacity of sum_b NB_b (items, counts, pooled K)
  int32_t block;       // tokens per block
  int32_t last_n;      // last_n_block of the selection
  int32_t split_blocks;  // blocks per chunk of a split row (0: none)
  int32_t* units;      // chunk units: count at [0], queue words, records from byte 64
  int64_t unit_cap;
  int32_t* arrivals;   // per (head, unit) arrival counters of the split rows, zeroed here
  int64_t n_arrivals;
};

struct PoolArgs {
  SeqTables tab;
  const uint16_t* k;
  int64_t kst, khs;
  uint16_t* mk;  // chunk-major pooled keys (see fp_ws_layout in flashprefill.h)
  int64_t nb_sum_cap;
  int32_t B;
  int32_t Hkv;
  int32_t block;  // tokens per block of the plan and the attention
  int32_t ratio;  // selection blocks are ratio x block tokens (2 at block_size 256, else 1)
};

struct SearchArgs {
  SeqTables tab;
  const uint16_t* q;
  int64_t qst, qhs;
  const uint16_t* mk;
  int32_t* idx;
  int32_t* cnt;
  int32_t* rowrec;    // per (head, item), or per (head, tile) at block_size 256:
                      // {count, first entry, second entry, diagonal kept}
  int64_t tri_cap;
  int64_t nb_sum_cap;
  const float* in_p;  // select-only mode: caller's block scores
  const float* in_m;
  float* dump_p;      // nullable
  float* dump_m;
  int32_t B, Hq, Hkv, nb_max;
  float sm_scale_log2;  // fp32(fp32(1/sqrt(d)) * fp32(log2 e))
  float alpha;
  int32_t sink, window, last_n, native, min_budget;
  int32_t pair_rows;  // 16-bit score kernel: two rows per workgroup (set by launch_search)
  // (Selection blocks of 256 tokens over the 128-token plan, block_size 256:
  // the workgroup of item (b, 2i) scores and selects 256-row i and writes the
  // 128-granularity lists of rows 2i and 2i + 1, those of item (b, 2i + 1)
  // return at once; pooled key block j sits at slot 2j. The search kernels'
  // block template of 256 selects this.)
};

struct AttnArgs {
  SeqTables tab;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t qst, qhs, kst, khs, vst, vhs, ost, ohs;
  const int32_t* idx;
  const int32_t* cnt;
  const int32_t* rowrec;  // per (head, item), or per (head, tile) when ratio > 1:
                          // {count, first entry, second entry, diagonal kept}
  int64_t tri_cap;
  int64_t nb_sum_cap;
  int32_t B, Hq, Hkv;
  float sm_scale_log2;
  // split rows: the first unit_slots workgroups run the chunk units (map_item
  // over num_q_heads x unit_cap, rounded up to a multiple of 8 so that the
  // row workgroups after them keep their XCD), writing fp32 partials that
  // k_merge combines
  int32_t last_n;
  int32_t split_blocks;
  const int32_t* units;
  float* part;
  int64_t unit_cap;
  int64_t unit_slots;
  // persistent grid: the workgroups of XCD x (id % 8) claim the slots
  // x, x + 8, x + 16, ... < total_slots from queue[x] (queue = units + kQueueOff)
  int32_t* queue;
  int64_t total_slots;
  // merge_inline: the last chunk of a split row to finish combines the row's
  // partials (counted in arrivals[h * unit_cap + first unit of the row]);
  // otherwise k_merge does
  int32_t* arrivals;
  int32_t merge_inline;
  int32_t ratio;  // > 1: row records are indexed by tile (block_size 256)
};

struct KvCacheArgs {
  const void* key;
  const void* value;
  int64_t k_stride_tok, k_stride_head, v_stride_tok, v_stride_head;
  void* key_cache;
  void* value_cache;
  int64_t kc_stride_block, kc_stride_slot, kc_stride_head;
  int64_t vc_stride_block, vc_stride_slot, vc_stride_head;
  const int64_t* slot_mapping;
  int64_t num_tokens;
  int64_t num_slots;  // num_blocks * block_size
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t row_bytes;  // head_dim * elem_bytes
  int32_t elem_bytes;
};

struct RopeArgs {
  void* q;
  int64_t q_stride_tok, q_stride_head;
  void* k;
  int64_t k_stride_tok, k_stride_head;
  int32_t num_q_heads, num_kv_heads, head_dim;
  const int64_t* positions;  // per token
  int64_t num_tokens;
  const float* cos_tab;      // (num_positions, head_dim / 2)
  const float* sin_tab;
  int64_t num_positions;
  const void* q_norm;        // nullable: head_dim weights in the input dtype
  const void* k_norm;
  float eps;
};

// f(std::integral_constant<int, D>{}) for the head dim D of the 16-bit
// kernels' instantiations (64, 128, 256; the C ABI rejects any other)
template <typename F>
auto with_head_dim(int head_dim, F&& f) {
  if (head_dim == 256) return f(std::integral_constant<int, 256>{});
  if (head_dim == 128) return f(std::integral_constant<int, 128>{});
  return f(std::integral_constant<int, 64>{});
}

hipError_t launch_plan(const PlanArgs& a, hipStream_t s);
hipError_t launch_rope(const RopeArgs& a, int dtype, hipStream_t s);
hipError_t launch_kv_cache_write(const KvCacheArgs& a, hipStream_t s);
hipError_t launch_pool(const PoolArgs& a, int dtype, int head_dim, int64_t grid, hipStream_t s);
// k_plan then k_pool as one launch (16-bit inputs, batch <= kSmallPlanBatch)
hipError_t launch_plan_pool(const PlanArgs& pa, const PoolArgs& a, int dtype, int head_dim,
                            hipStream_t s);
hipError_t launch_search(const SearchArgs& a, int dtype, int head_dim, int block, int64_t grid,
                         bool from_scores, hipStream_t s);
hipError_t launch_attn(const AttnArgs& a, int dtype, int head_dim, int block, int64_t grid,
                       bool persist, hipStream_t s);
// combines the chunk partials of the split rows into their output rows
hipError_t launch_merge(const AttnArgs& a, int dtype, int head_dim, int block, hipStream_t s);
hipError_t launch_attn_f32(const AttnArgs& a, int head_dim, int block, int64_t grid,
                           hipStream_t s);

}  // namespace fp
