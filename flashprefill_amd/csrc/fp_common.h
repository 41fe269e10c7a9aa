// Device-side building blocks shared by the FlashPrefill gfx950 kernels:
// element types, 16-byte vector moves, MFMA wrappers, wave/block reductions
// and the workgroup -> work-item mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashprefill.h"

namespace fp {

constexpr int kWave = 64;
constexpr int kMaxBatch = 4096;   // sequences per call (plan kernel keeps them in LDS)
constexpr int kMaxBlocks = 8192;  // blocks per sequence (1,048,576 tokens at block 128)
constexpr int kSmallPlanBatch = 16;  // batches planned inside the pooling launch (k_plan_pool)
constexpr int kMaxChunks = 8;        // chunks of one split row (host policy, k_merge)
constexpr int kMaxInlineChunks = 8;  // chunks merged inside the attention kernel

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// element types: 16-bit storage, fp32 math
// ---------------------------------------------------------------------------
struct BF16 {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    __bf16 b = static_cast<__bf16>(f);  // v_cvt_pk_bf16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, b);
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

struct F16 {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename T::vec8 as_vec8(uint4 x) {
  return __builtin_bit_cast(typename T::vec8, x);
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// 16-byte global load / store (address must be 16-byte aligned)
__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// ---------------------------------------------------------------------------
// wave reductions (wave64)
// ---------------------------------------------------------------------------
// Lane exchanges without an address register: v_permlane32_swap between the
// two 32-lane halves, ds_swizzle (bit mode: and 0x1f, or 0, xor M) within a
// half. The reductions are xor butterflies (distance 32, then 16 .. 1).
// v_permlane32_swap(x, x): the first result holds x of lanes 0-31 in both
// halves, the second x of lanes 32-63, so the partner of a lower lane is in
// the second and that of an upper lane in the first.
__device__ __forceinline__ uint32_t xchg32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (threadIdx.x & 32) ? static_cast<uint32_t>(r[0]) : static_cast<uint32_t>(r[1]);
}
template <int M>
__device__ __forceinline__ uint32_t xchg_xor(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_ds_swizzle(static_cast<int>(x), 0x1f | (M << 10)));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, __uint_as_float(xchg32(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xchg_xor<16>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xchg_xor<8>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xchg_xor<4>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xchg_xor<2>(__float_as_uint(x))));
  return fmaxf(x, __uint_as_float(xchg_xor<1>(__float_as_uint(x))));
}
template <int M>
__device__ __forceinline__ double xchg_xor_d(double x) {
  const uint64_t u = __double_as_longlong(x);
  const uint32_t lo = xchg_xor<M>(static_cast<uint32_t>(u));
  const uint32_t hi = xchg_xor<M>(static_cast<uint32_t>(u >> 32));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}
__device__ __forceinline__ double wave_sum_d(double x) {
  const uint64_t u = __double_as_longlong(x);
  const uint32_t lo = xchg32(static_cast<uint32_t>(u)), hi = xchg32(static_cast<uint32_t>(u >> 32));
  x += __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
  x += xchg_xor_d<16>(x);
  x += xchg_xor_d<8>(x);
  x += xchg_xor_d<4>(x);
  x += xchg_xor_d<2>(x);
  return x + xchg_xor_d<1>(x);
}

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// ---------------------------------------------------------------------------
// Work items: (sequence b, q-block i) pairs ordered heaviest first by the plan
// kernel, crossed with query heads. When Hq is a multiple of 8, the eight
// XCDs (workgroups are dispatched round-robin, XCD = id % 8) each get Hq/8
// consecutive heads, i.e. whole GQA groups when Hq/Hkv divides Hq/8, so K/V
// blocks are re-read from the XCD's own L2; each XCD walks its items
// heaviest first.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void map_item(int w, int num_q_heads, int& item, int& head) {
  if ((num_q_heads & 7) == 0) {
    const int x = w & 7, s = w >> 3, hpx = num_q_heads >> 3;
    head = x * hpx + s % hpx;
    item = s / hpx;
  } else {
    head = w % num_q_heads;
    item = w / num_q_heads;
  }
}

// Sequence owning global block g (binary search over seq_tile).
__device__ __forceinline__ int find_seq(const int64_t* seq_tile, int B, int64_t g) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (seq_tile[mid] <= g) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Attention rows. Per-row cost depends on the row's selection, whose density
// differs between heads, so a fixed head -> XCD assignment leaves some XCDs
// with more work than others (10 % at 128K in config 3). When the number of
// KV heads divides 8, the XCDs are split into Hkv sets of R = 8 / Hkv; a set
// serves one GQA group at a time (its G query heads share K / V, which its L2
// holds) and its XCDs take consecutive q-blocks in turn; every `per` q-block
// rounds the sets move on to the next group, so that over the sequence each
// set serves every group 4 times and the XCDs end with equal shares. Rows are
// still walked heaviest first within each XCD. attn_grid() is the matching
// grid size (workgroups past the last row return at once).
__device__ __forceinline__ void map_row(int w, int num_q_heads, int num_kv_heads, int64_t nitems,
                                        int& item, int& head) {
  if ((8 % num_kv_heads) == 0) {
    const int x = w & 7, s = w >> 3;
    const int R = 8 / num_kv_heads, G = num_q_heads / num_kv_heads;
    const int p = s / G, r = s % G;
    const int per = max(4, static_cast<int>(nitems / R / (4 * num_kv_heads)));
    item = R * p + x % R;
    head = ((x / R + p / per) % num_kv_heads) * G + r;
  } else {
    map_item(w, num_q_heads, item, head);
  }
}

inline int64_t attn_grid(int num_q_heads, int num_kv_heads, int64_t nitems_cap) {
  if ((8 % num_kv_heads) == 0) {
    const int64_t R = 8 / num_kv_heads;
    return 8 * static_cast<int64_t>(num_q_heads / num_kv_heads) * ((nitems_cap + R - 1) / R);
  }
  return static_cast<int64_t>(num_q_heads) * nitems_cap;
}

// One work item as the plan kernel records it (32 bytes, read with one scalar
// load by the persistent attention kernel).
struct ItemRec {
  int32_t b, i;  // sequence, q-block
  int32_t L;     // tokens of sequence b
  int32_t tile;  // seq_tile[b] + i: the item's row in the per-block count table
  int64_t t0;    // seq_start[b]
  int64_t tri;   // seq_tri[b] + i (i + 1) / 2: start of the item's index list
};

// One chunk of a split row (48 bytes): the row's item record, the chunk index
// and the row's chunk count. A split row is a last_n row (every causal block
// selected, so its list is 0 .. i) of more than split_blocks blocks; chunk c
// covers list entries c * split_blocks .. min((c + 1) * split_blocks, i + 1) - 1.
struct UnitRec {
  ItemRec r;
  int32_t c, nc;
  int32_t pad[2];
};

// Work queues of the persistent attention grid, in the header of the units
// region (int32 words kQueueOff ..): one claim counter per XCD. The plan
// kernel zeroes them on every call and the attention kernel empties each
// queue again after its last claim, so that an attention launch on its own
// (after one full call) also starts from empty queues.
constexpr int kQueueOff = 4;
constexpr int kQueueWords = 8;

// The rule shared by the plan (which emits the chunks) and the attention
// kernel (which leaves such rows to the chunks): row i of a sequence of nb
// blocks is split when it is one of the last_n rows and has more than
// split_blocks blocks.
__device__ __forceinline__ bool row_is_split(int i, int nb, int last_n, int split_blocks) {
  return split_blocks > 0 && i >= nb - last_n && i + 1 > split_blocks;
}

// Workspace views shared by all kernels (device pointers into the workspace).
struct SeqTables {
  uint32_t* status;
  int64_t* seq_tile;   // [B+1] prefix of NB_b
  int64_t* seq_tri;    // [B+1] prefix of NB_b (NB_b + 1) / 2
  int64_t* seq_start;  // [B]   first token of sequence b
  int32_t* seq_len;    // [B]   tokens of sequence b (0 when skipped)
  ItemRec* items;      // [nb_sum_cap] work items, heaviest first
};

}  // namespace fp
