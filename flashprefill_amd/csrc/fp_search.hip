// Fused block scoring + pattern selection for the FlashPrefill gfx950 path.
//
// One workgroup (4 waves) owns one (query head h, sequence b, q-block i) row:
//
//  1. score (ops/flashprefill_native_forward.py:87-188,
//     ops/flashprefill_varlen_func.py:106-217): the 128 full-resolution query
//     rows of block i against every pooled key j <= i on bf16/fp16 MFMA
//     (v_mfma_f32_32x32x16), S = Q . mk^T. The query block is staged once in
//     LDS (direct-to-LDS loads, chunk-swizzled) and every wave reads it as
//     MFMA A operands while it walks its own 32-column tiles of pooled keys
//     (B operands from L2), so the per-column reductions over the block's rows
//     (m_ij = max_r s_r, p_ij = sum_r exp2(s_r - m_ij)) are in-register plus
//     one cross-half exchange; no partial result is shared between waves. The causal
//     block rule keeps all rows for j < i and only row 127 for j == i (:157).
//     (p, m) of the row stay in LDS (optionally dumped to global for parity
//     tests).
//  2. select (ops/flashprefill_native_forward.py:347-403,
//     ops/flashprefill_varlen_func.py:240-409,656): M = max_j m_ij,
//     S_ij = p_ij * exp2(m_ij - M) [native: / (sum_j S_ij + 1e-9)],
//     keep j if S_ij >= alpha * max_j S_ij, or j < sink, or 0 <= i-j < window,
//     or i >= NB - last_n. No sort, no prefix pass over global memory: the
//     kept j are compacted in ascending order with wave ballots.
//
// Selection arithmetic is made order independent so that the same fp32 (p, m)
// always yields the same index set: exp2 is evaluated in fp64 and rounded
// once to fp32 (correctly rounded fp32 exp2), and the native row sum is
// accumulated in fp64 and rounded once.
#include "fp_attn_common.h"

namespace fp {

__device__ __forceinline__ float exp2_rn(float x) {
  return static_cast<float>(exp2(static_cast<double>(x)));
}

// fp32 -> uint32 whose unsigned order is the float order (non-NaN values)
__device__ __forceinline__ uint32_t sort_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The selection's workgroup barriers wait for LDS operations only
// (lds_barrier): the waves exchange data through LDS alone, and a
// direct-to-LDS load of the next row's query block may be in flight meanwhile.
__device__ __forceinline__ float block_max_lds(float x, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  x = wave_max(x);
  if (lane == 0) red[w] = x;
  lds_barrier();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  lds_barrier();
  return r;
}

// max over lanes l and l ^ 32, in every lane (pair32_max without the operand
// canonicalisation the compiler adds to fmaxf of exchanged bits; for the
// non-NaN scores of the search this is the same value)
__device__ __forceinline__ float pair32_max_raw(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  float y;
  asm("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(static_cast<unsigned>(r[0])), "v"(static_cast<unsigned>(r[1])));
  return y;
}

// LDS scratch of select_row: block-reduction slots and the radix histogram
constexpr int kSelectScratch = 104 + 256 * 4;

// The min_budget largest scores of a row, ranked by (score desc, j asc) as
// the oracle ranks them (native path, ops/flashprefill_native_forward.py:
// 353-357, where torch.topk leaves the order of equal scores unspecified):
// returns the key of the budget-th entry and, in `need_eq`, how many of the
// entries with exactly that key are taken (lowest j first). Radix select over
// the sortable 32-bit keys, 8 bits per pass, MSB first.
__device__ __forceinline__ uint32_t budget_threshold(const float* pl, int n, int kk, uint32_t* hist, int* pick,
                                     int& need_eq) {
  const int t = threadIdx.x, lane = t & 63;
  uint32_t prefix = 0, pmask = 0;
  int need = kk;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[t] = 0;  // 256 bins, one per thread
    lds_barrier();
    for (int j = t; j < n; j += 256) {
      const uint32_t key = sort_key(pl[j]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1u);
    }
    lds_barrier();
    if (t < 64) {  // wave 0: the bin holding the need-th largest key
      const int b0 = 255 - 4 * lane;  // this lane's bins b0 .. b0-3, descending
      const int c0 = hist[b0], c1 = hist[b0 - 1], c2 = hist[b0 - 2], c3 = hist[b0 - 3];
      const int sl = c0 + c1 + c2 + c3;
      int incl = sl;
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const uint64_t hit = __ballot(incl >= need);
      if (lane == __ffsll(static_cast<long long>(hit)) - 1) {
        int rem = need - (incl - sl), bin = b0;
        if (rem > c0) {
          rem -= c0, --bin;
          if (rem > c1) {
            rem -= c1, --bin;
            if (rem > c2) rem -= c2, --bin;
          }
        }
        pick[0] = bin;
        pick[1] = rem;
      }
    }
    lds_barrier();
    prefix |= static_cast<uint32_t>(pick[0]) << shift;
    pmask |= 255u << shift;
    need = pick[1];
    lds_barrier();  // pick and hist are rewritten by the next pass
  }
  need_eq = need;
  return prefix;
}

// Select over p (pl) and m (ml) of one row held in LDS; writes the ascending
// index list and its length. Uses 256 threads; `scratch` is kSelectScratch
// bytes of LDS (the query block's area once scoring is done, so that the
// kernel's LDS stays at 40 KB and four workgroups fit on a CU), or, without
// min_budget, the first 104 of them (the radix histogram is not used), which
// the paired-row kernel takes from the unused tail of ml. ml is overwritten
// (with the min_budget flags).
//
// Two block reductions: M = max_j m_j, then max_j S_j together with the
// native row sum. Since the native division by (sum + 1e-9) is correctly
// rounded and monotone, the max of the normalised scores is the normalised
// max. The compaction loops use alternating count slots, one barrier per
// 256 entries.
//
// At ratio 2 (block_size 256) the row is 256-row i of its sequence and the
// outputs are the 128-granularity lists of plan rows 2i (list / count /
// row_rec) and 2i + 1 (list_b / count_b / row_rec_b, null when the sequence
// ends inside row 2i): a kept 256-block j < i is plan blocks 2j, 2j + 1 in
// both, the kept diagonal j = i is block 2i in row 2i (its keys 256i + 128 ..
// are all after the row's queries) and blocks 2i, 2i + 1 in row 2i + 1.
template <int RATIO>
__device__ __forceinline__ void select_row(float* pl, float* ml, int n, int i, int nb,
                                           const SearchArgs& a,
                           int32_t* list, int32_t* count, int32_t* row_rec, void* scratch,
                           int32_t* list_b = nullptr, int32_t* count_b = nullptr,
                           int32_t* row_rec_b = nullptr) {
#pragma clang fp contract(off)
  float* redf = static_cast<float*>(scratch);
  double* redd = reinterpret_cast<double*>(static_cast<char*>(scratch) + 16);
  int* wtot = reinterpret_cast<int*>(static_cast<char*>(scratch) + 48);  // [2][4]
  int* pick = reinterpret_cast<int*>(static_cast<char*>(scratch) + 80);
  int* head3 = reinterpret_cast<int*>(static_cast<char*>(scratch) + 88);  // row record: j0, j1, diag
  uint32_t* hist = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + 104);
  // the wave index through readfirstlane: the compiler then knows it is
  // wave-uniform, so loops and branches on it are scalar
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
  if (t < 3) head3[t] = 0;

  float lm = -INFINITY;
  for (int j = t; j < n; j += 256) lm = fmaxf(lm, ml[j]);
  const float M = block_max_lds(lm, redf);

  double ls = 0.0;
  float lmax = 0.0f;
  for (int j = t; j < n; j += 256) {
    const float sj = pl[j] * exp2_rn(ml[j] - M);
    pl[j] = sj;
    ls += static_cast<double>(sj);
    lmax = fmaxf(lmax, sj);
  }
  lmax = wave_max(lmax);
  if (a.native) ls = wave_sum_d(ls);
  if (lane == 0) {
    redf[w] = lmax;
    redd[w] = ls;
  }
  lds_barrier();  // redf / redd are not written again in this row
  float maxS = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  if (a.native) {
    const float tot = static_cast<float>(redd[0] + redd[1] + redd[2] + redd[3]);
    const float denom = tot + 1e-9f;
    maxS = maxS / denom;
    for (int j = t; j < n; j += 256) pl[j] = pl[j] / denom;
  }
  const float thr = maxS * a.alpha;
  const bool last_rows = i >= nb - a.last_n;

  // min_budget: flag the budget largest scores in ml (1.0 = forced on)
  const int kk = min(a.min_budget, n);
  if (kk > 0) {
    int need_eq;
    const uint32_t kstar = budget_threshold(pl, n, kk, hist, pick, need_eq);
    int eq_running = 0;
    for (int base = 0, c2 = 0; base < n; base += 256, c2 ^= 4) {
      const int j = base + t;
      const uint32_t key = j < n ? sort_key(pl[j]) : 0u;
      const bool eq = j < n && key == kstar;
      const uint64_t bal = __ballot(eq);
      if (lane == 0) wtot[c2 + w] = __popcll(bal);
      lds_barrier();
      int off = eq_running;
      for (int k = 0; k < w; ++k) off += wtot[c2 + k];
      if (j < n) ml[j] = (key > kstar || (eq && off + lanes_below(bal) < need_eq)) ? 1.0f : 0.0f;
      eq_running += wtot[c2] + wtot[c2 + 1] + wtot[c2 + 2] + wtot[c2 + 3];
    }
    lds_barrier();  // the count slots are reused below
  }

  int running = 0;
  for (int base = 0, c2 = 0; base < n; base += 256, c2 ^= 4) {
    const int j = base + t;
    bool keep = false;
    if (j < n) {
      keep = (pl[j] >= thr) || (j < a.sink) || (i - j < a.window) || last_rows ||
             (kk > 0 && ml[j] != 0.0f);
    }
    const uint64_t bal = __ballot(keep);
    // slot set c2 was last read before the previous chunk's barrier
    if (lane == 0) wtot[c2 + w] = __popcll(bal);
    lds_barrier();
    int off = running;
    for (int k = 0; k < w; ++k) off += wtot[c2 + k];
    if (keep) {
      const int pos = off + lanes_below(bal);
      if constexpr (RATIO == 1) {
        list[pos] = j;
      } else {
        list[2 * pos] = 2 * j;
        if (j < i) list[2 * pos + 1] = 2 * j + 1;
        if (list_b) {
          list_b[2 * pos] = 2 * j;
          list_b[2 * pos + 1] = 2 * j + 1;
        }
      }
      if (pos < 2) head3[pos] = j;
    }
    if (j == i) head3[2] = keep ? 1 : 0;
    running += wtot[c2] + wtot[c2 + 1] + wtot[c2 + 2] + wtot[c2 + 3];
  }
  lds_barrier();  // head3 complete
  if (t == 0) {
    // the attention kernel's row record: one 16-byte load gives the count,
    // the first two entries and whether the diagonal block is kept
    if constexpr (RATIO == 1) {
      *count = running;
      *reinterpret_cast<int4*>(row_rec) = make_int4(running, head3[0], head3[1], head3[2]);
    } else {
      const int f0 = head3[0], dg = head3[2];
      const int ca = 2 * running - dg;
      *count = ca;
      *reinterpret_cast<int4*>(row_rec) = make_int4(ca, 2 * f0, f0 < i ? 2 * f0 + 1 : 0, dg);
      if (list_b) {
        *count_b = 2 * running;
        *reinterpret_cast<int4*>(row_rec_b) = make_int4(2 * running, 2 * f0, 2 * f0 + 1, dg);
      }
    }
  }
}

// LDS chunk swizzle of a 128 x D bf16 tile (16-byte chunks; conflict-free
// MFMA A-operand reads of 16 rows x one chunk column on the 64-bank LDS)
template <int D>
__device__ __forceinline__ int qswz(int r) {
  if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (r >> 1) & 7;
}

// dynamic LDS ahead of p / m: the query block, or select_row's scratch
template <int D, int BLK, bool FROM_SCORES>
constexpr size_t search_q_bytes() { return FROM_SCORES ? kSelectScratch : BLK * D * 2; }

// BLK is the selection block: 64 or 128 (the plan's block, ratio 1), or 256
// over a 128-token plan (ratio 2).
template <typename T, int D, int BLK, bool FROM_SCORES>
__global__ __launch_bounds__(256, (BLK > 128 || D > 128) ? 2 : 4) void k_search(SearchArgs a) {
  // 4 workgroups per CU at BLK = 128: 4 x (32 KB query block + 2 x 4 KB p / m
  // at 1024 blocks) = 160 KB of LDS, and at most 128 VGPRs per wave (BLK =
  // 256: a 64 KB query block and 8 row groups of accumulators; d = 256: a 64
  // KB query block and 16 k-steps of key operands; two per CU)
  constexpr int RG = BLK / 32;  // 32-row groups of the query block
  constexpr int RATIO = BLK > 128 ? 2 : 1;  // selection blocks per plan block
  extern __shared__ uint4 dyn4[];
  uint4* sq = dyn4;  // the query block (score mode only)
  float* pl = reinterpret_cast<float*>(reinterpret_cast<char*>(dyn4) +
                                       search_q_bytes<D, BLK, FROM_SCORES>());
  float* ml = pl + a.nb_max;
  int slot, h;
  map_item(blockIdx.x, a.Hq, slot, h);
  const int64_t nitems = sld(a.tab.seq_tile + a.B);
  // the wave index through readfirstlane: the compiler then knows it is
  // wave-uniform, so loops and branches on it are scalar
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
  // The workgroup's rows: item `slot`, and with pair_rows also the item at the
  // other end of the heaviest-first order, so that every pair holds about the
  // same work (scored second, its query block loads during the first row's
  // selection).
  const int64_t item_a = slot;
  int64_t item_b = -1;
  if (!FROM_SCORES && a.pair_rows) {
    if (item_a >= (nitems + 1) / 2) return;
    item_b = nitems - 1 - item_a;
    if (item_b == item_a) item_b = -1;
  } else if (item_a >= nitems) {
    return;
  }
  // ratio 2: plan row 2i + 1 is selected together with row 2i
  if constexpr (RATIO > 1)
    if (sld(a.tab.items + item_a).i % RATIO) return;
  auto select = [&](const ItemRec& rec, int64_t item, int64_t row_tri, void* scratch) {
    int32_t* list = a.idx + row_tri;
    int32_t* count = a.cnt + static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile;
    const int64_t tile_b = rec.tile - rec.i;
    const int nb = static_cast<int>(sld(a.tab.seq_tile + rec.b + 1) - tile_b);
    if constexpr (RATIO == 1) {
      int32_t* row_rec = a.rowrec + 4 * (static_cast<int64_t>(h) * a.nb_sum_cap + item);
      select_row<1>(pl, ml, rec.i + 1, rec.i, nb, a, list, count, row_rec, scratch);
    } else {
      // 256-row i = rec.i / 2 writes plan rows rec.i and rec.i + 1 (when the
      // sequence has it), records by tile
      const int i = rec.i / RATIO;
      int32_t* row_rec = a.rowrec + 4 * (static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile);
      const bool has_b = rec.i + 1 < nb;
      select_row<RATIO>(pl, ml, i + 1, i, (nb + RATIO - 1) / RATIO, a, list, count, row_rec,
                        scratch, has_b ? list + rec.i + 1 : nullptr, has_b ? count + 1 : nullptr,
                        has_b ? row_rec + 4 : nullptr);
    }
  };

  if constexpr (FROM_SCORES) {
    const ItemRec rec = sld(a.tab.items + item_a);
    const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + rec.tri;
    for (int j = t; j <= rec.i / RATIO; j += 256) {
      pl[j] = a.in_p[row_tri + j];
      ml[j] = a.in_m[row_tri + j];
    }
    __syncthreads();
    select(rec, item_a, row_tri, dyn4);
  } else {
    constexpr int KS = D / 16;  // MFMA k-steps over the head dim
    constexpr int CH = D / 8;
    const int kvh = h / (a.Hq / a.Hkv);
    const int half = lane >> 5, l32 = lane & 31;
    const float c = a.sm_scale_log2;
    // < 2^31: nb_sum_cap < 2^26 (checked on the host)
    const uint32_t half_off = static_cast<uint32_t>(a.nb_sum_cap) * 16u * static_cast<uint32_t>(half);
    // One row: its item record and the wave-uniform base of its pooled keys.
    // Pooled keys are chunk-major: 16-byte chunk x of key block g of kv head
    // kvh at byte ((kvh * CH + x) * nb_sum_cap + g) * 16, so the chunk of 32
    // consecutive keys that one k-step's operands need is 512 contiguous
    // bytes. kb0: chunk row 0 at the sequence's first key; k-step s reads
    // chunk row 2 s (the lower half-wave) and 2 s + 1 (the upper), kb_step
    // bytes apart per s; the lane part of an address is a 32-bit byte offset.
    // Ratio 2: the row is 256-row i = rec.i / 2 and pooled key block j sits
    // at slot 2j of the sequence's 128-token blocks.
    struct Row {
      ItemRec rec;
      int64_t row_tri;
      int i, n, ntiles;  // selection row, its keys, 32-key tiles
      const char* kb0;
    };
    const int64_t kb_step = 2 * a.nb_sum_cap * 16;
    auto setup = [&](int64_t item) {
      Row r;
      r.rec = sld(a.tab.items + item);
      r.row_tri = static_cast<int64_t>(h) * a.tri_cap + r.rec.tri;
      r.i = r.rec.i / RATIO;
      r.n = r.i + 1;
      r.ntiles = (r.n + 31) >> 5;
      const int64_t tile_b = r.rec.tile - r.rec.i;
      r.kb0 = reinterpret_cast<const char*>(a.mk) +
              (static_cast<int64_t>(kvh) * CH * a.nb_sum_cap + tile_b) * 16;
      return r;
    };
    // pooled keys of one 32-key tile as MFMA B operands (lane: key 32 tile +
    // l32, dims 16 s + 8 half .. +7; columns past the row's last key read key
    // n - 1: their scores are computed and never stored)
    typename T::vec8 kb[KS];
    // lane part of a key-operand address: chunk row of the half-wave, key l32
    constexpr uint32_t kstride = 16u * RATIO;  // bytes per key
    const uint32_t koff = half_off + kstride * static_cast<uint32_t>(l32);
    auto load_kb = [&](const Row& r, int tile) {
      // a tile inside the row adds its scalar offset; the row's last tile
      // clamps its keys to n - 1
      uint32_t off = koff + 32u * kstride * static_cast<uint32_t>(tile);
      if (32 * tile + 32 > r.n) {
        asm volatile("" : "+v"(off));  // keep the clamp on the last tile's branch
        off = half_off + kstride * static_cast<uint32_t>(min(32 * tile + l32, r.n - 1));
      }
#pragma unroll
      for (int s = 0; s < KS; ++s)
        kb[s] = as_vec8<T>(*reinterpret_cast<const uint4*>(r.kb0 + s * kb_step + off));
    };
    // The query block is staged in LDS with direct-to-LDS loads, and every
    // wave reads it as MFMA A operands (rows 32*rg + l32, dims 16*s + 8*half
    // .. +7); the wave's first key tile follows (first_kb). land() waits for
    // both and zeroes the rows past the sequence end (they still count for
    // j < i).
    auto issue_q = [&](const Row& r) {
      TileLanes<D, BLK, 4> tq;
      tq.init(a.qst, __builtin_amdgcn_readfirstlane(w), lane);
      issue_tile<D, BLK, 4>(sq, a.q + r.rec.t0 * a.qst + static_cast<int64_t>(h) * a.qhs, a.qst,
                            tq, r.i, r.rec.L, __builtin_amdgcn_readfirstlane(w), lane);
    };
    auto first_kb = [&](const Row& r) {
      if (w < r.ntiles) load_kb(r, w);
    };
    auto land = [&](const Row& r) {
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      if ((r.i + 1) * BLK > r.rec.L) {
        for (int cidx = t; cidx < BLK * CH; cidx += 256)
          if (r.i * BLK + cidx / CH >= r.rec.L) sq[cidx] = zero4();
        __syncthreads();
      }
    };
    auto score = [&](const Row& r) {
      const int n = r.n, ntiles = r.ntiles, i = r.i;
      for (int tile = w; tile < ntiles; tile += 4) {
        const int j = 32 * tile + l32;
        const bool jv = j < n;
        f32x16 acc[RG];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) acc[rg] = f32x16{};
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            const int rr = 32 * rg + l32;
            const uint4 qop = sq[rr * CH + ((2 * s + half) ^ qswz<D>(rr))];
            acc[rg] = T::mfma32(as_vec8<T>(qop), kb[s], acc[rg]);
          }

        // the wave's next key tile, loaded as one burst into kb (dead once the
        // MFMAs above have read it) so that its latency passes behind this
        // tile's max / exp2 / sum; loads issued between the MFMAs instead
        // stalled the MFMA stream and measured slower
        __builtin_amdgcn_sched_barrier(0);
        if (tile + 4 < ntiles) load_kb(r, tile + 4);
        __builtin_amdgcn_sched_barrier(0);
        // acc[rg][v] = Q[32 rg + 8 (v/4) + 4 half + v%4] . mk[j]
        float mx = -INFINITY, sum = 0.0f, m;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, acc[rg][v]);
        if (tile + 1 < ntiles) {  // every column j < i: all BLK rows count
          m = pair32_max_raw(mx) * c;
#pragma unroll
          for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int v = 0; v < 16; ++v) sum += __builtin_amdgcn_exp2f(fmaf(acc[rg][v], c, -m));
          sum = pair32_sum(sum);
          // every column of a tile before the last is a key of the row
          if (half == 0) {
            pl[j] = sum;
            ml[j] = m;
            if (a.dump_p) {
              float* dp = a.dump_p + (r.row_tri + 32 * tile);
              float* dm = a.dump_m + (r.row_tri + 32 * tile);
              dp[l32] = sum;
              dm[l32] = m;
            }
          }
          continue;
        } else {
          // last tile: j < i all rows, j == i the last row BLK - 1 only
          // (acc[RG - 1][15] of the upper half-wave), j > i none. The case is
          // uniform over a lane's values, so the full-tile reduction runs for
          // every lane and one select per lane picks the result (the same
          // arithmetic on the rows that count, no per-element masking)
          const bool full = j < i, rowlast = j == i && half == 1;
          mx = full ? mx : (rowlast ? acc[RG - 1][15] : -INFINITY);
          m = pair32_max(mx) * c;
#pragma unroll
          for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int v = 0; v < 16; ++v) sum += __builtin_amdgcn_exp2f(fmaf(acc[rg][v], c, -m));
          sum = full ? sum
                     : (rowlast ? __builtin_amdgcn_exp2f(fmaf(acc[RG - 1][15], c, -m)) : 0.0f);
        }
        sum = pair32_sum(sum);
        if (half == 0 && jv) {
          pl[j] = sum;
          ml[j] = m;
          if (a.dump_p) {
            a.dump_p[r.row_tri + j] = sum;
            a.dump_m[r.row_tri + j] = m;
          }
        }
      }
      __syncthreads();  // (p, m) complete; every wave is done with the query block
    };

    const Row ra = setup(item_a);
    issue_q(ra);
    first_kb(ra);
    land(ra);
    score(ra);
    // The second row's query-block loads go out before the first row's
    // selection when that selection can keep its reduction scratch
    // (select_row's first 104 bytes) in the unused tail of ml instead of the
    // query block's area; the selection's barriers wait for LDS operations
    // only, so they do not wait for these loads. (Its first key tile follows
    // the selection: held across it in registers, it made the kernel spill.)
    const bool early = item_b >= 0 && ra.n + 32 <= a.nb_max && a.min_budget == 0;
    Row rb;
    if (early) {
      rb = setup(item_b);
      issue_q(rb);
    }
    select(ra.rec, item_a, ra.row_tri, early ? static_cast<void*>(ml + a.nb_max - 32) : dyn4);
    if (item_b < 0) return;
    if (!early) {
      lds_barrier();  // the scratch in the query block's area is read to the end
      rb = setup(item_b);
      issue_q(rb);
    }
    first_kb(rb);
    land(rb);
    score(rb);
    select(rb.rec, item_b, rb.row_tri, dyn4);
  }
}

// fp32 inputs: the same row pipeline with fp32 MFMA (v_mfma_f32_32x32x2_f32,
// full fp32 products; the reference's fp32 path runs tl.dot in TF32). The
// query block sits in LDS with rows padded by 16 bytes (conflict-free A-operand
// reads of 32 rows at one column); MFMA k-step s pairs dim s (lanes 0-31)
// with dim D/2 + s (lanes 32-63), so a lane's key operands are one contiguous
// half row. Selection is select_row, as for 16-bit inputs.
template <int D, int BLK>
__global__ __launch_bounds__(256, 2) void k_search_f32(SearchArgs a) {
  constexpr int RG = BLK / 32, QS = D + 4, KS = D / 2;
  constexpr int RATIO = BLK > 128 ? 2 : 1;  // selection blocks per plan block
  extern __shared__ uint4 dyn4[];
  float* sq = reinterpret_cast<float*>(dyn4);  // BLK rows of QS floats
  float* pl = sq + BLK * QS;
  float* ml = pl + a.nb_max;
  int item, h;
  map_item(blockIdx.x, a.Hq, item, h);
  const int64_t nitems = sld(a.tab.seq_tile + a.B);
  if (item >= nitems) return;
  const ItemRec rec = sld(a.tab.items + item);
  // ratio 2: 256-row i = rec.i / 2 (plan row 2i + 1 is selected with row 2i),
  // pooled key block j at slot 2j
  if (rec.i % RATIO) return;
  const int b = rec.b, i = rec.i / RATIO, L = rec.L;
  const int64_t tile_b = rec.tile - rec.i;
  const int64_t t0 = rec.t0;
  const int n = i + 1;
  const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + rec.tri;
  // the wave index through readfirstlane: the compiler then knows it is
  // wave-uniform, so loops and branches on it are scalar
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int kvh = h / (a.Hq / a.Hkv);
  const float c = a.sm_scale_log2;
  const float* q = reinterpret_cast<const float*>(a.q);
  // chunk-major pooled keys (4 floats per chunk): dims 4x .. 4x+3 of key block g
  // at ((kvh * D / 4 + x) * nb_sum_cap + g) * 4
  const float* mk = reinterpret_cast<const float*>(a.mk) +
                    (static_cast<int64_t>(kvh) * (D / 4) * a.nb_sum_cap + tile_b) * 4;

  // query block -> LDS (rows past the sequence end are zero: they still
  // count for j < i)
  for (int cidx = t; cidx < BLK * (D / 4); cidx += 256) {
    const int r = cidx / (D / 4), x4 = cidx % (D / 4);
    const int gr = i * BLK + r;
    float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
    if (gr < L) val = *reinterpret_cast<const float4*>(q + (t0 + gr) * a.qst + h * a.qhs + 4 * x4);
    *reinterpret_cast<float4*>(sq + r * QS + 4 * x4) = val;
  }
  __syncthreads();
  const int ntiles = (n + 31) >> 5;
  for (int tile = w; tile < ntiles; tile += 4) {
    const int j = 32 * tile + l32;
    const bool jv = j < n;
    float kb[KS];
    // this lane's dims half * KS .. : chunks half * KS / 4 + s4
    const float* kr =
        mk + (static_cast<int64_t>(half) * (KS / 4) * a.nb_sum_cap + (jv ? RATIO * j : 0)) * 4;
#pragma unroll
    for (int s4 = 0; s4 < KS / 4; ++s4) {
      const float4 x = jv ? *reinterpret_cast<const float4*>(kr + s4 * a.nb_sum_cap * 4)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
      kb[4 * s4] = x.x; kb[4 * s4 + 1] = x.y; kb[4 * s4 + 2] = x.z; kb[4 * s4 + 3] = x.w;
    }
    f32x16 acc[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) acc[rg] = f32x16{};
#pragma unroll
    for (int s4 = 0; s4 < KS / 4; ++s4)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const float4 q4 = *reinterpret_cast<const float4*>(sq + (32 * rg + l32) * QS + half * KS + 4 * s4);
        acc[rg] = __builtin_amdgcn_mfma_f32_32x32x2f32(q4.x, kb[4 * s4], acc[rg], 0, 0, 0);
        acc[rg] = __builtin_amdgcn_mfma_f32_32x32x2f32(q4.y, kb[4 * s4 + 1], acc[rg], 0, 0, 0);
        acc[rg] = __builtin_amdgcn_mfma_f32_32x32x2f32(q4.z, kb[4 * s4 + 2], acc[rg], 0, 0, 0);
        acc[rg] = __builtin_amdgcn_mfma_f32_32x32x2f32(q4.w, kb[4 * s4 + 3], acc[rg], 0, 0, 0);
      }
    // acc[rg][v] = Q[32 rg + 8 (v/4) + 4 half + v%4] . mk[j]; the causal
    // block rule as in k_search: all rows for j < i, the last row for j == i
    float mx = -INFINITY, sum = 0.0f;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, acc[rg][v]);
    const bool full = j < i, rowlast = j == i && half == 1;
    mx = full ? mx : (rowlast ? acc[RG - 1][15] : -INFINITY);
    const float m = pair32_max(mx) * c;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int v = 0; v < 16; ++v) sum += __builtin_amdgcn_exp2f(fmaf(acc[rg][v], c, -m));
    sum = full ? sum : (rowlast ? __builtin_amdgcn_exp2f(fmaf(acc[RG - 1][15], c, -m)) : 0.0f);
    sum = pair32_sum(sum);
    if (half == 0 && jv) {
      pl[j] = sum;
      ml[j] = m;
      if (a.dump_p) {
        a.dump_p[row_tri + j] = sum;
        a.dump_m[row_tri + j] = m;
      }
    }
  }
  __syncthreads();
  int32_t* list = a.idx + row_tri;
  int32_t* count = a.cnt + static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile;
  const int nb = static_cast<int>(sld(a.tab.seq_tile + b + 1) - tile_b);
  if constexpr (RATIO == 1) {
    int32_t* row_rec = a.rowrec + 4 * (static_cast<int64_t>(h) * a.nb_sum_cap + item);
    select_row<1>(pl, ml, n, i, nb, a, list, count, row_rec, dyn4);
  } else {
    int32_t* row_rec = a.rowrec + 4 * (static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile);
    const bool has_b = rec.i + 1 < nb;
    select_row<RATIO>(pl, ml, n, i, (nb + RATIO - 1) / RATIO, a, list, count, row_rec, dyn4,
                      has_b ? list + rec.i + 1 : nullptr, has_b ? count + 1 : nullptr,
                      has_b ? row_rec + 4 : nullptr);
  }
}

template <int D, int BLK>
hipError_t launch_search_f32_t(const SearchArgs& a, int64_t grid, hipStream_t s) {
  const size_t shm = BLK * (D + 4) * sizeof(float) + 2 * sizeof(float) * static_cast<size_t>(a.nb_max);
  if (shm > 48 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_search_f32<D, BLK>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(shm));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_search_f32<D, BLK>), dim3(static_cast<unsigned>(grid)), dim3(256), shm, s,
                     a);
  return hipGetLastError();
}

template <typename T, int D, int BLK, bool FROM_SCORES>
hipError_t launch_search_t(const SearchArgs& a, int64_t grid, hipStream_t s) {
  const size_t shm = search_q_bytes<D, BLK, FROM_SCORES>() +
                     2 * sizeof(float) * static_cast<size_t>(a.nb_max);
  if (shm > 48 * 1024) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_search<T, D, BLK, FROM_SCORES>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(shm));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_search<T, D, BLK, FROM_SCORES>), dim3(static_cast<unsigned>(grid)),
                     dim3(256), shm, s, a);
  return hipGetLastError();
}

// block: the selection block (64, 128 or 256)
template <typename T, int D>
hipError_t launch_search_d(const SearchArgs& a, int block, int64_t grid, bool from_scores,
                           hipStream_t s) {
  if (block == 256)
    return from_scores ? launch_search_t<T, D, 256, true>(a, grid, s)
                       : launch_search_t<T, D, 256, false>(a, grid, s);
  if (block == 128)
    return from_scores ? launch_search_t<T, D, 128, true>(a, grid, s)
                       : launch_search_t<T, D, 128, false>(a, grid, s);
  return from_scores ? launch_search_t<T, D, 64, true>(a, grid, s)
                     : launch_search_t<T, D, 64, false>(a, grid, s);
}

template <int D>
hipError_t launch_search_f32_d(const SearchArgs& a, int block, int64_t grid, hipStream_t s) {
  if (block == 256) return launch_search_f32_t<D, 256>(a, grid, s);
  return block == 128 ? launch_search_f32_t<D, 128>(a, grid, s)
                      : launch_search_f32_t<D, 64>(a, grid, s);
}

// Problems of at least this many (head, row) items score two rows per
// workgroup (k_search, 16-bit inputs); smaller ones keep one per workgroup,
// whose grid alone is not much larger than the resident workgroups.
constexpr int64_t kPairRowsMin = 4096;

hipError_t launch_search(const SearchArgs& args, int dtype, int head_dim, int block, int64_t grid,
                         bool from_scores, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  SearchArgs a = args;
  a.pair_rows = 0;
  if (dtype != FP_DTYPE_F32 && !from_scores && block != 256 && grid >= kPairRowsMin) {
    a.pair_rows = 1;
    grid = static_cast<int64_t>(a.Hq) * ((grid / a.Hq + 1) / 2);  // grid = Hq x item capacity
  }
  if (dtype == FP_DTYPE_F32) {
    if (from_scores)  // selection only: no input element is read
      return launch_search_d<BF16, 128>(a, block, grid, true, s);
    return head_dim == 128 ? launch_search_f32_d<128>(a, block, grid, s)
                           : launch_search_f32_d<64>(a, block, grid, s);
  }
  return with_head_dim(head_dim, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return dtype == FP_DTYPE_BF16 ? launch_search_d<BF16, D>(a, block, grid, from_scores, s)
                                  : launch_search_d<F16, D>(a, block, grid, from_scores, s);
  });
}

}  // namespace fp
