// Sequence planning and K-block pooling for the FlashPrefill gfx950 path.
//
//   k_plan  — one workgroup turns cu_seqlens into per-sequence tables (block
//             counts, block / triangle prefix sums) and the heaviest-first
//             work-item list; replaces get_cu_tile_seqlens
//             (ops/flashprefill_varlen_func.py:8-18) with no host sync.
//   k_pool  — mean of every K block (block_size tokens) over its valid rows
//             (ops/flashprefill_native_forward.py:21-67,
//              ops/flashprefill_varlen_func.py:35-85). HBM-bound: each K byte
//             is read once with 16-byte loads, sums are kept in fp64 (exact
//             for 16-bit inputs whose exponents span fewer than ~38 binades)
//             and the mean is divided in fp64.
#include "fp_internal.h"

namespace fp {

// Block-wide exclusive scan of one int64 per thread (blockDim.x <= 1024).
__device__ int64_t block_exscan_i64(int64_t v, int64_t* red, int64_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) red[w] = x;
  __syncthreads();
  if (w == 0) {
    int64_t r = lane < nw ? red[lane] : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(r, o);
      if (lane >= o) r += y;
    }
    if (lane < nw) red[lane] = r;
  }
  __syncthreads();
  const int64_t wave_off = w > 0 ? red[w - 1] : 0;
  *total = red[nw - 1];
  __syncthreads();
  return wave_off + x - v;
}

// Block-wide inclusive running maximum of one int64 per thread.
__device__ int64_t block_inscan_max_i64(int64_t v, int64_t* red, int64_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o);
    if (lane >= o) x = max(x, y);
  }
  if (lane == 63) red[w] = x;
  __syncthreads();
  if (w == 0) {
    int64_t r = lane < nw ? red[lane] : INT64_MIN;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(r, o);
      if (lane >= o) r = max(r, y);
    }
    if (lane < nw) red[lane] = r;
  }
  __syncthreads();
  const int64_t res = w > 0 ? max(red[w - 1], x) : x;
  *total = red[nw - 1];
  __syncthreads();
  return res;
}

__global__ __launch_bounds__(1024) void k_plan(PlanArgs a) {
  __shared__ int32_t s_pre[kMaxBatch + 1];  // NB prefix over sequences
  __shared__ int32_t s_lvl[kMaxBlocks];     // per q-block level: counts, then cursors
  __shared__ int64_t s_red[16];
  __shared__ uint32_t s_status;
  const int t = threadIdx.x, nt = blockDim.x;
  const SeqTables& tab = a.tab;
  if (t == 0) s_status = 0u;
  __syncthreads();

  // 1. per-sequence lengths and validity. A sequence is kept only if it lies
  //    inside [0, total_tokens], is not longer than max_seq_len, and starts at
  //    or after every earlier cu_seqlens entry (inclusive running maximum), so
  //    the kept sequences are disjoint and ordered: their lengths add up to at
  //    most total_tokens and sum_b NB_b stays within nb_sum_cap.
  int64_t run_max = INT64_MIN;
  int64_t nb_tot = 0;
  for (int base = 0; base < a.B; base += nt) {
    const int b = base + t;
    int64_t start = 0, end = 0;
    if (b < a.B) {
      if (a.cu) {
        start = a.cu[b];
        end = a.cu[b + 1];
      } else {
        start = static_cast<int64_t>(b) * a.uniform_len;
        end = start + a.uniform_len;
      }
    }
    int64_t chunk_max;
    const int64_t incl = max(run_max, block_inscan_max_i64(b < a.B ? start : INT64_MIN, s_red,
                                                           &chunk_max));
    run_max = max(run_max, chunk_max);
    int64_t nb = 0;
    if (b < a.B) {
      int64_t len = end - start;
      if (start < 0 || len < 0 || end > a.total_tokens || incl > start) {
        atomicOr(&s_status, FP_STATUS_BAD_CU_SEQLENS);
        len = 0;
        start = 0;
      } else if (len > a.max_seq_len) {
        atomicOr(&s_status, FP_STATUS_SEQ_TOO_LONG);
        len = 0;
      }
      tab.seq_start[b] = start;
      tab.seq_len[b] = static_cast<int32_t>(len);
      nb = (len + a.block - 1) / a.block;
      s_pre[b] = static_cast<int32_t>(nb);
    }
    int64_t chunk_nb;
    block_exscan_i64(nb, s_red, &chunk_nb);
    nb_tot += chunk_nb;
  }
  // The rule above bounds sum NB by the workspace capacity; should a table
  // ever exceed it, every sequence is skipped rather than written past it.
  if (nb_tot > a.nb_sum_cap) {
    for (int b = t; b < a.B; b += nt) {
      tab.seq_len[b] = 0;
      s_pre[b] = 0;
    }
    if (t == 0) s_status |= FP_STATUS_BAD_CU_SEQLENS;
  }
  for (int i = t; i < a.nb_max; i += nt) s_lvl[i] = 0;
  __syncthreads();

  // 2. prefix sums of NB_b and NB_b (NB_b + 1) / 2; level histogram; the
  //    chunk units of the split rows (row_is_split), numbered by a prefix sum
  //    over sequences so that the chunks of one row are consecutive
  int64_t carry_tile = 0, carry_tri = 0, carry_unit = 0;
  UnitRec* urec = reinterpret_cast<UnitRec*>(reinterpret_cast<char*>(a.units) + 64);
  const int C = a.split_blocks;
  for (int base = 0; base < a.B; base += nt) {
    const int b = base + t;
    const int64_t nb = b < a.B ? s_pre[b] : 0;
    int64_t nu = 0;
    for (int i = max(static_cast<int>(nb) - a.last_n, 0); i < nb; ++i)
      if (row_is_split(i, static_cast<int>(nb), a.last_n, C)) nu += (i + C) / C;
    int64_t tot1, tot2, tot3;
    const int64_t e1 = block_exscan_i64(nb, s_red, &tot1);
    const int64_t e2 = block_exscan_i64(nb * (nb + 1) / 2, s_red, &tot2);
    const int64_t e3 = block_exscan_i64(nu, s_red, &tot3);
    if (b < a.B) {
      tab.seq_tile[b] = carry_tile + e1;
      tab.seq_tri[b] = carry_tri + e2;
      if (nb > 0) atomicAdd(&s_lvl[nb - 1], 1);
      int64_t u = carry_unit + e3;
      for (int i = max(static_cast<int>(nb) - a.last_n, 0); i < nb; ++i) {
        if (!row_is_split(i, static_cast<int>(nb), a.last_n, C)) continue;
        const int nc = (i + C) / C;
        for (int c = 0; c < nc; ++c, ++u) {
          if (u >= a.unit_cap) continue;  // the host bound makes this unreachable
          UnitRec ur;
          ur.r.b = b;
          ur.r.i = i;
          ur.r.L = tab.seq_len[b];
          ur.r.tile = static_cast<int32_t>(carry_tile + e1 + i);
          ur.r.t0 = tab.seq_start[b];
          ur.r.tri = carry_tri + e2 + static_cast<int64_t>(i) * (i + 1) / 2;
          ur.c = c;
          ur.nc = nc;
          ur.pad[0] = ur.pad[1] = 0;
          urec[u] = ur;
        }
      }
    }
    __syncthreads();  // all reads of s_pre[b] in this chunk are done
    if (b < a.B) s_pre[b] = static_cast<int32_t>(carry_tile + e1);
    carry_tile += tot1;
    carry_tri += tot2;
    carry_unit += tot3;
  }
  if (t == 0) {
    tab.seq_tile[a.B] = carry_tile;
    tab.seq_tri[a.B] = carry_tri;
    s_pre[a.B] = static_cast<int32_t>(carry_tile);
    a.units[0] = static_cast<int32_t>(min(carry_unit, a.unit_cap));
  }
  if (t < kQueueWords) a.units[kQueueOff + t] = 0;  // empty attention work queues
  for (int64_t x = t; x < a.n_arrivals; x += nt) a.arrivals[x] = 0;
  __syncthreads();

  // 3. level sizes c_i = #{b : NB_b > i} (suffix sum of the histogram), then
  //    level offsets in heaviest-first order (exclusive suffix sum of c_i).
  for (int pass = 0; pass < 2; ++pass) {
    int64_t carry = 0;
    for (int base = 0; base < a.nb_max; base += nt) {
      const int i = a.nb_max - 1 - (base + t);  // descending level
      const int64_t v = i >= 0 ? s_lvl[i] : 0;
      int64_t tot;
      const int64_t ex = block_exscan_i64(v, s_red, &tot);
      if (i >= 0) s_lvl[i] = static_cast<int32_t>(carry + (pass == 0 ? ex + v : ex));
      carry += tot;
      __syncthreads();
    }
  }

  // 4. scatter the item records: position = level offset + arrival order
  //    (seq_len / seq_start / seq_tri were written above by this workgroup)
  const int nsum = s_pre[a.B];
  for (int g = t; g < nsum; g += nt) {
    int lo = 0, hi = a.B - 1;  // last b with s_pre[b] <= g
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pre[mid] <= g) lo = mid; else hi = mid - 1;
    }
    const int i = g - s_pre[lo];
    const int pos = atomicAdd(&s_lvl[i], 1);
    ItemRec r;
    r.b = lo;
    r.i = i;
    r.L = tab.seq_len[lo];
    r.tile = g;
    r.t0 = tab.seq_start[lo];
    r.tri = tab.seq_tri[lo] + static_cast<int64_t>(i) * (i + 1) / 2;
    tab.items[pos] = r;
  }
  __syncthreads();
  if (t == 0) *tab.status = s_status;
}

// Mean of key block g of kv head hh (rows t0 .. t0 + rows - 1 of K), by one
// workgroup of 256 threads = R row groups x D / 8 chunks of 16 bytes; each
// thread sums its rows of one chunk in fp64. The R partial sums are added
// within each wave by lane exchanges (its 64 / C row groups), then the four
// waves' sums through LDS, and the mean sum / rows is divided in fp64 and
// converted to fp32 and then to the input dtype (the rounding path of torch's
// float64 -> bfloat16 / float16 cast). A 16-bit value has an 8- or 11-bit
// significand, so a sum of at most 256 of them is exact in fp64 unless their
// exponents span more than ~38 binades: the mean is then the correctly
// rounded block mean whatever the order of the additions. The means are
// stored chunk-major (16-byte chunk c of key block g and kv head hh at entry
// g of chunk row hh * C + c), so that the search kernel's loads of 32
// consecutive keys' chunk are contiguous.
template <typename T, int D>
__device__ __forceinline__ void pool_block(const PoolArgs& a, int64_t g, int hh, int64_t t0,
                                           int rows) {
  constexpr int C = D / 8;    // 16-byte chunks per head row
  constexpr int R = 256 / C;  // row groups
  __shared__ double red[3][C][8];  // sums of waves 1 .. 3
  const int t = threadIdx.x, c = t % C, rg = t / C;
  const uint16_t* src = a.k + t0 * a.kst + hh * a.khs + c * 8;
  double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  for (int r = rg; r < rows; r += R) {
    const uint4 v = ld16(src + static_cast<int64_t>(r) * a.kst);
    const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += static_cast<double>(T::to_f32(e[q]));
  }
  // lanes c, c + C, ... of a wave hold the same chunk: xor exchanges over the
  // lane bits above log2(C) add the wave's row groups
  const int w = t >> 6;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if constexpr (C <= 16) acc[q] += xchg_xor_d<16>(acc[q]);
    if constexpr (C <= 8) acc[q] += xchg_xor_d<8>(acc[q]);
    const uint64_t u = __double_as_longlong(acc[q]);
    const uint32_t lo = xchg32(static_cast<uint32_t>(u)), hi = xchg32(static_cast<uint32_t>(u >> 32));
    acc[q] += __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
  }
  if (w > 0 && (t & 63) < C) {
#pragma unroll
    for (int q = 0; q < 8; ++q) red[w - 1][c][q] = acc[q];
  }
  __syncthreads();
  if (t < C) {
    const double n = static_cast<double>(rows);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += red[0][c][q] + red[1][c][q] + red[2][c][q];
    uint16_t o[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = T::from_f32(static_cast<float>(acc[q] / n));
    // chunk-major: chunk c of (g, hh) is entry g of chunk row hh * C + c
    uint16_t* out = a.mk + ((hh * C + c) * a.nb_sum_cap + g) * 8;
    st16(out, *reinterpret_cast<const uint4*>(o));
  }
}

// One workgroup per (key block g, kv head hh), the sequence found in the
// plan's tables. Several workgroups per block keep short sequences from
// running on a handful of CUs.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_pool(PoolArgs a) {
  const int64_t g = blockIdx.x / a.Hkv;
  const int hh = static_cast<int>(blockIdx.x % a.Hkv);
  const int64_t nsum = a.tab.seq_tile[a.B];
  if (g >= nsum) return;
  const int b = find_seq(a.tab.seq_tile, a.B, g);
  const int i = static_cast<int>(g - a.tab.seq_tile[b]);
  // a selection block of ratio plan blocks is pooled by the workgroup of its
  // first plan block, into that block's slot
  if (i % a.ratio) return;
  const int L = a.tab.seq_len[b];
  pool_block<T, D>(a, g, hh, a.tab.seq_start[b] + static_cast<int64_t>(i) * a.block,
                   min(a.block * a.ratio, L - i * a.block));
}

// ---------------------------------------------------------------------------
// Plan and pooling in one launch, for a few sequences
// ---------------------------------------------------------------------------
// With at most kSmallPlanBatch sequences every workgroup of the pooling grid
// derives the sequence table itself: wave 0 applies k_plan's rules (validity,
// the capacity bound, block and triangle prefix sums, chunk units of the
// split rows) to cu_seqlens in registers and leaves the table in LDS. The
// first workgroup writes the plan's tables, work items and unit records; the
// others pool key block g = (blockIdx.x - 1) / Hkv of kv head
// (blockIdx.x - 1) % Hkv as k_pool does. The plan then costs no launch and
// no latency of its own ahead of the pooling. Work items are written heaviest first as k_plan orders
// them, and by sequence within a level.
struct SmallPlan {
  int64_t start[kSmallPlanBatch];
  int64_t tile[kSmallPlanBatch + 1];  // prefix of NB_b
  int64_t tri[kSmallPlanBatch + 1];   // prefix of NB_b (NB_b + 1) / 2
  int64_t unit[kSmallPlanBatch + 1];  // prefix of the chunk units
  int32_t len[kSmallPlanBatch];
  int32_t nb[kSmallPlanBatch];
  uint32_t status;
};

__device__ __forceinline__ int64_t wave_exscan_i64(int64_t v, int64_t* total) {
  const int lane = threadIdx.x & 63;
  int64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  *total = __shfl(x, 63);
  return x - v;
}

// wave 0: the sequence table of k_plan passes 1 and 2 for B <= 64 sequences
__device__ void small_plan_table(const PlanArgs& a, SmallPlan& sp) {
  const int b = threadIdx.x;  // lane
  int64_t start = 0, end = 0;
  if (b < a.B) {
    if (a.cu) {
      start = a.cu[b];
      end = a.cu[b + 1];
    } else {
      start = static_cast<int64_t>(b) * a.uniform_len;
      end = start + a.uniform_len;
    }
  }
  // inclusive running maximum of the starts (k_plan's ordering rule)
  int64_t incl = b < a.B ? start : INT64_MIN;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(incl, o);
    if (b >= o) incl = max(incl, y);
  }
  uint32_t st = 0;
  int64_t len = 0;
  if (b < a.B) {
    len = end - start;
    if (start < 0 || len < 0 || end > a.total_tokens || incl > start) {
      st = FP_STATUS_BAD_CU_SEQLENS;
      len = 0;
      start = 0;
    } else if (len > a.max_seq_len) {
      st = FP_STATUS_SEQ_TOO_LONG;
      len = 0;
    }
  }
  int64_t nb = (len + a.block - 1) / a.block, nb_tot;
  wave_exscan_i64(nb, &nb_tot);
  if (nb_tot > a.nb_sum_cap) {  // as k_plan: skip every sequence
    len = 0;
    nb = 0;
    st |= FP_STATUS_BAD_CU_SEQLENS;
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) st |= __shfl_xor(st, o);
  const int C = a.split_blocks;
  int64_t nu = 0;
  for (int i = max(static_cast<int>(nb) - a.last_n, 0); i < nb; ++i)
    if (row_is_split(i, static_cast<int>(nb), a.last_n, C)) nu += (i + C) / C;
  int64_t t1, t2, t3;
  const int64_t e1 = wave_exscan_i64(nb, &t1);
  const int64_t e2 = wave_exscan_i64(nb * (nb + 1) / 2, &t2);
  const int64_t e3 = wave_exscan_i64(nu, &t3);
  if (b < a.B) {
    sp.start[b] = start;
    sp.len[b] = static_cast<int32_t>(len);
    sp.nb[b] = static_cast<int32_t>(nb);
    sp.tile[b] = e1;
    sp.tri[b] = e2;
    sp.unit[b] = e3;
  }
  if (b == 0) {
    sp.tile[a.B] = t1;
    sp.tri[a.B] = t2;
    sp.unit[a.B] = t3;
    sp.status = st;
  }
}

// workgroup 0 of k_plan_pool: everything k_plan writes
__device__ void small_plan_write(const PlanArgs& a, const SmallPlan& sp) {
  const int t = threadIdx.x, B = a.B;
  const SeqTables& tab = a.tab;
  if (t < B) {
    tab.seq_start[t] = sp.start[t];
    tab.seq_len[t] = sp.len[t];
    tab.seq_tile[t] = sp.tile[t];
    tab.seq_tri[t] = sp.tri[t];
  }
  if (t == 0) {
    tab.seq_tile[B] = sp.tile[B];
    tab.seq_tri[B] = sp.tri[B];
    *tab.status = sp.status;
    a.units[0] = static_cast<int32_t>(min(sp.unit[B], a.unit_cap));
  }
  if (t < kQueueWords) a.units[kQueueOff + t] = 0;  // empty attention work queues
  for (int64_t x = t; x < a.n_arrivals; x += blockDim.x) a.arrivals[x] = 0;
  // work items: item (b, i) goes after every item of a higher level and
  // after the items of level i of the sequences before b
  const int64_t nsum = sp.tile[B];
  for (int64_t g = t; g < nsum; g += blockDim.x) {
    int b = 0;
    while (b + 1 < B && sp.tile[b + 1] <= g) ++b;
    const int i = static_cast<int>(g - sp.tile[b]);
    int64_t pos = 0;
    for (int x = 0; x < B; ++x) {
      pos += max(sp.nb[x] - 1 - i, 0);
      if (x < b && sp.nb[x] > i) ++pos;
    }
    ItemRec r;
    r.b = b;
    r.i = i;
    r.L = sp.len[b];
    r.tile = static_cast<int32_t>(g);
    r.t0 = sp.start[b];
    r.tri = sp.tri[b] + static_cast<int64_t>(i) * (i + 1) / 2;
    tab.items[pos] = r;
  }
  // chunk units of the split rows, numbered as k_plan numbers them
  if (t < B) {
    UnitRec* urec = reinterpret_cast<UnitRec*>(reinterpret_cast<char*>(a.units) + 64);
    const int C = a.split_blocks, nb = sp.nb[t];
    int64_t u = sp.unit[t];
    for (int i = max(nb - a.last_n, 0); i < nb; ++i) {
      if (!row_is_split(i, nb, a.last_n, C)) continue;
      const int nc = (i + C) / C;
      for (int c = 0; c < nc; ++c, ++u) {
        if (u >= a.unit_cap) continue;  // the host bound makes this unreachable
        UnitRec ur;
        ur.r.b = t;
        ur.r.i = i;
        ur.r.L = sp.len[t];
        ur.r.tile = static_cast<int32_t>(sp.tile[t] + i);
        ur.r.t0 = sp.start[t];
        ur.r.tri = sp.tri[t] + static_cast<int64_t>(i) * (i + 1) / 2;
        ur.c = c;
        ur.nc = nc;
        ur.pad[0] = ur.pad[1] = 0;
        urec[u] = ur;
      }
    }
  }
}

// Workgroup 0 writes the tables and items: dispatched first, it runs beside
// the pooling (as the grid's last workgroup it started only once a pooling
// slot freed up; 4K call -1.4 %, 128K unchanged).
template <typename T, int D>
__global__ __launch_bounds__(256) void k_plan_pool(PlanArgs pa, PoolArgs a) {
  __shared__ SmallPlan sp;
  if (threadIdx.x < 64) small_plan_table(pa, sp);
  __syncthreads();
  if (blockIdx.x == 0) {
    small_plan_write(pa, sp);
    return;
  }
  const int64_t wg = static_cast<int64_t>(blockIdx.x) - 1;
  const int64_t g = wg / a.Hkv;
  const int hh = static_cast<int>(wg % a.Hkv);
  if (g >= sp.tile[a.B]) return;
  int b = 0;
  while (b + 1 < a.B && sp.tile[b + 1] <= g) ++b;
  const int i = static_cast<int>(g - sp.tile[b]);
  if (i % a.ratio) return;
  pool_block<T, D>(a, g, hh, sp.start[b] + static_cast<int64_t>(i) * a.block,
                   min(a.block * a.ratio, sp.len[b] - i * a.block));
}

// fp32 keys: the block mean summed in fp64 (in row order) and rounded once to
// fp32, one thread per dim of one (key block, kv head) per workgroup.
__global__ __launch_bounds__(256) void k_pool_f32(PoolArgs a, int head_dim) {
  const int64_t g = blockIdx.x / a.Hkv;
  const int hh = static_cast<int>(blockIdx.x % a.Hkv);
  const int64_t nsum = a.tab.seq_tile[a.B];
  if (g >= nsum) return;
  const int b = find_seq(a.tab.seq_tile, a.B, g);
  const int i = static_cast<int>(g - a.tab.seq_tile[b]);
  if (i % a.ratio) return;
  const int L = a.tab.seq_len[b];
  const int64_t t0 = a.tab.seq_start[b] + static_cast<int64_t>(i) * a.block;
  const int rows = min(a.block * a.ratio, L - i * a.block);
  const float* k = reinterpret_cast<const float*>(a.k);
  // chunk-major: dims 4c .. 4c+3 of (g, hh) are entry g of chunk row hh * d / 4 + c
  float* out = reinterpret_cast<float*>(a.mk);
  for (int x = threadIdx.x; x < head_dim; x += blockDim.x) {
    const float* src = k + t0 * a.kst + hh * a.khs + x;
    double sum = 0.0;
    for (int r = 0; r < rows; ++r) sum += static_cast<double>(src[static_cast<int64_t>(r) * a.kst]);
    const int64_t row = static_cast<int64_t>(hh) * (head_dim / 4) + x / 4;
    out[(row * a.nb_sum_cap + g) * 4 + x % 4] = static_cast<float>(sum / static_cast<double>(rows));
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_plan(const PlanArgs& a, hipStream_t s) {
  // small problems (few sequences, few blocks each) plan with 4 waves, whose
  // barriers are cheaper (4K: 10.8 -> 8.2 us); larger ones need the 16 waves
  // for the item scatter
  const int threads = a.B <= 256 && a.nb_max <= 256 ? 256 : 1024;
  hipLaunchKernelGGL(k_plan, dim3(1), dim3(threads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_plan_pool(const PlanArgs& pa, const PoolArgs& a, int dtype, int head_dim,
                            hipStream_t s) {
  // one workgroup per (key block, kv head) of the capacity, plus the table writer
  const dim3 g(static_cast<unsigned>(a.nb_sum_cap * a.Hkv + 1)), blk(256);
  with_head_dim(head_dim, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    if (dtype == FP_DTYPE_BF16) hipLaunchKernelGGL((k_plan_pool<BF16, D>), g, blk, 0, s, pa, a);
    else hipLaunchKernelGGL((k_plan_pool<F16, D>), g, blk, 0, s, pa, a);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_pool(const PoolArgs& a, int dtype, int head_dim, int64_t grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  // one workgroup per (key block, kv head)
  const dim3 g(static_cast<unsigned>(grid * a.Hkv)), blk(256);
  if (dtype == FP_DTYPE_F32) {
    hipLaunchKernelGGL(k_pool_f32, g, blk, 0, s, a, head_dim);
  } else {
    with_head_dim(head_dim, [&](auto dc) {
      constexpr int D = decltype(dc)::value;
      if (dtype == FP_DTYPE_BF16) hipLaunchKernelGGL((k_pool<BF16, D>), g, blk, 0, s, a);
      else hipLaunchKernelGGL((k_pool<F16, D>), g, blk, 0, s, a);
      return 0;
    });
  }
  return hipGetLastError();
}

}  // namespace fp
