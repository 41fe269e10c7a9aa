// Varlen GQA block-sparse flash-attention forward for gfx950
// (ops/flashprefill_native_forward.py:227-344,
//  ops/flashprefill_varlen_func.py:449-575).
//
// A workgroup (4 waves) processes one (query head h, sequence b, q-block i)
// item at a time and walks that row's selected key blocks in ascending order;
// large problems run as a persistent grid whose workgroups claim the next item
// of their XCD from a queue (k_attn below). Wave w owns the
// 32 query rows 32w..32w+31 of the block. Everything is kept in the
// "one query per lane" orientation so the softmax never needs a cross-lane
// transpose:
//
//   S^T (keys x queries) = K . Q^T   A = K rows from LDS, B = Q^T in registers
//   row max / row sum: in-lane over the lane's 64 keys + one half-wave swap
//   O^T (dims x queries) += V^T . P^T
//                                    A = V^T via ds_read_b64_tr_b16 from the
//                                        key-major V tile in LDS,
//                                    B = P^T straight from the S^T registers
//                                        (the MFMA k order is permuted
//                                        identically on both operands)
//
// all on v_mfma_f32_32x32x16 (bf16 or fp16 in, fp32 accumulate).
//
// K and V blocks (128 keys x d) are gathered by index with direct-to-LDS
// loads (global_load_lds_dwordx4, no VGPR staging) into one K and one V
// buffer per workgroup (2 x 32 KB at d = 128, two workgroups per CU). The two
// buffers are pipelined against each other: the next block's K streams in
// while this block's softmax and P.V run, the next block's V while the next
// S = K.Q^T runs. Rows are stored with a 16-byte-chunk XOR swizzle chosen for
// the 64-bank LDS so that the K operand reads (16 rows, one chunk column per
// cycle) and the transposing V reads (4 rows x 4 chunks) are conflict free.
//
// Numerics follow the reference loop: m starts at -inf and l at 1.0, one
// 128-key tile per selected block, alpha = exp2(m_old - m_new) with NaN -> 1,
// P is rounded to the input dtype before P.V, the diagonal block masks
// key > query, and O = acc * (1/l). Two deliberate differences, both at
// rounding level: m is the max of conditional rescaling (it moves only when a
// lane's partial row sum of P against it would exceed kRescaleSum, so P <= 2^8),
// and l adds the rounded P (v_dot2c, two scores per instruction) instead of the
// fp32 p.
#include "fp_attn_common.h"

namespace fp {

template <typename T, int D>
struct AttnState {
  f32x16 o[D / 32];
  float m_run;
  float l_part;
};

// P = exp2(s * c - m) of the lane's KT x 16 scores, rounded to the input type
// in pairs (the B operands of P.V); returns the sum of the rounded values.
// Tiles from `live` on (wave-uniform) are entirely masked: P = 0 there.
template <typename T, int KT>
__device__ __forceinline__ float exp_pack(const f32x16 (&s)[KT], float m, float c, int live,
                                          uint32_t (&pk)[KT][8]) {
  float psum[2] = {0.0f, 0.0f};
#pragma unroll
  for (int t4 = 0; t4 < KT; ++t4) {
    if (t4 >= live) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pk[t4][e] = 0u;
      continue;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(s[t4][2 * e], c, -m));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(s[t4][2 * e + 1], c, -m));
      pk[t4][e] = pack2<T>(p0, p1);
      psum[e & 1] = add_pair<T>(pk[t4][e], psum[e & 1]);
    }
  }
  return psum[0] + psum[1];
}

// How many MFMAs ahead of its use each LDS operand read is issued in the S
// and P.V loops (sched_group_barrier order). Left to itself the scheduler issued the reads one or two MFMAs ahead
// (a wait before nearly every MFMA); four ahead measured 8 % faster at 128K
// (two: 6 %, six or eight: no better), with the same registers and no spills.
constexpr int kReadAhead = 4;

// One selected block (`first`: the row's first, wave-uniform): S = K.Q^T,
// online softmax, O += V^T.P^T, and the pipelined refills of the K / V
// buffers with block `jn` (when jn >= 0). The list entry at `pf` (the block
// after jn, or any valid entry) is read into `jpf` right after the K refill is
// issued, unclamped: the scalar load then
// completes behind the softmax, which reads no LDS, instead of stalling the
// next block (scalar loads share the LDS wait counter, so the compiler waits
// for them at the first LDS read after them).
template <typename T, int D, int BLK, bool DIAG>
__device__ __forceinline__ void attn_block(AttnState<T, D>& st, const typename T::vec8* qb,
                                           const uint4* sk, uint4* sk_w, const uint16_t* sv16,
                                           uint4* sv_w, const uint16_t* kbase,
                                           const uint16_t* vbase, int64_t kst, int64_t vst,
                                           const TileLanes<D, BLK, BLK / 32>& tk,
                                           const TileLanes<D, BLK, BLK / 32>& tv,
                                           int jn, const int32_t* pf, int& jpf, int L, float c,
                                           bool first, int w, int lane) {
  constexpr int CH = D / 8;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int KT = BLK / 32;  // 32-key tiles of S^T per block
  constexpr int NW = BLK / 32;  // waves of the workgroup
  constexpr int NI = TileLanes<D, BLK, NW>::NI;
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * w + l32;

  // On the diagonal block, wave w's query rows 32w .. 32w+31 see keys of the
  // 32-key tiles 0 .. w only: the S and P.V MFMAs of later tiles are skipped
  // (their P is 0), tiles before w need no mask and tile w the per-element one.
  const int live = DIAG ? w + 1 : KT;
  // entered with K of this block landed in every wave's part and the barrier
  // passed (V may still be in flight)
  f32x16 s[KT];
  if constexpr (!DIAG) {
    // k-step outer, tile inner: four independent accumulation chains
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4) s[t4] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int t4 = 0; t4 < KT; ++t4) {
        const int r = 32 * t4 + l32;
        const uint4 kop = sk[r * CH + ((2 * ks + half) ^ swz<D>(r))];
        s[t4] = T::mfma32(as_vec8<T>(kop), qb[ks], s[t4]);
      }
    // the K operand reads run kReadAhead MFMAs ahead of their use
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReadAhead, 0);
#pragma unroll
    for (int k = 0; k < KS * KT - kReadAhead; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 0);
  } else {
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4) {
      s[t4] = f32x16{};
      if (t4 >= live) continue;
      const int r = 32 * t4 + l32;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 kop = sk[r * CH + ((2 * ks + half) ^ swz<D>(r))];
        s[t4] = T::mfma32(as_vec8<T>(kop), qb[ks], s[t4]);
      }
    }
  }
  lds_barrier();  // every wave is done with the K buffer
  if (jn >= 0) issue_tile<D, BLK, NW>(sk_w, kbase, kst, tk, jn, L, w, lane);
  jpf = sld(pf);

  if constexpr (DIAG) {  // key > query is masked on the diagonal block
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4) {
      if (t4 < w) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = 32 * t4 + 8 * (v >> 2) + 4 * half + (v & 3);
        if (t4 > w || key > qrow) s[t4][v] = -INFINITY;
      }
    }
  }
  // P rounded to the input type, packed as the B operands of P.V, is first
  // formed against the running max; l adds the rounded P that P.V consumes.
  // The block is taken again with a moved max (and O, l rescaled) only when
  // some lane's partial row sum exceeds kRescaleSum (every P <= that sum, so
  // P <= 2^8 on the kept path) or is not finite, and always on the row's first
  // block, where m is -inf. The block maximum is then computed only on that
  // path instead of for every block.
  uint32_t pk[KT][8];
  float ps = 0.0f;
  bool move = first;
  if (!first) {
    ps = exp_pack<T, KT>(s, st.m_run, c, live, pk);
    move = __ballot(!(ps <= kRescaleSum)) != 0;
  }
  if (move) {
    float mx = -INFINITY;
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[t4][v]);
    const float m_new = fmaxf(st.m_run, pair32_max(mx) * c);
    float alpha = __builtin_amdgcn_exp2f(st.m_run - m_new);
    if (alpha != alpha) alpha = 1.0f;
    st.l_part *= alpha;
    st.m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) st.o[dt][v] *= alpha;
    ps = exp_pack<T, KT>(s, st.m_run, c, live, pk);
  }
  st.l_part += ps;

  if (jn >= 0) vm_barrier<NI>(); else vm_barrier<0>();  // V of this block has landed
  // O^T += V^T . P^T over BLK / 16 steps of 16 keys. B element e of lane (q, half)
  // is key 16 u + (e < 4 ? 4 half + e : 8 + 4 half + e - 4); the A operand
  // (V^T) is read in the same key order with two transposing reads.
  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);
  // raised wave priority while this wave issues its P.V MFMAs: when both
  // waves of a SIMD are ready, the MFMA stream goes first (measured 1-2 %
  // faster; the same around S, or around the softmax instead, was not)
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int u = 0; u < BLK / 16; ++u) {
    const int t4 = u >> 1, hh = u & 1;
    if (DIAG && t4 >= live) continue;
    const uint4 pu = make_uint4(pk[t4][4 * hh], pk[t4][4 * hh + 1], pk[t4][4 * hh + 2],
                                pk[t4][4 * hh + 3]);
    const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pu);
    const int r1 = 16 * u + tr_row;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int x = 32 * dt + tr_col;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, x)));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, x)));
      const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
      const uint4 va = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      st.o[dt] = T::mfma32(as_vec8<T>(va), pb, st.o[dt]);
    }
  }
  if constexpr (!DIAG) {  // the V^T reads (two per MFMA) run kReadAhead MFMAs ahead
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kReadAhead, 0);
#pragma unroll
    for (int k = 0; k < (BLK / 16) * DT - kReadAhead; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 0);
  }
  __builtin_amdgcn_s_setprio(0);
  if (jn >= 0) {
    // one barrier for two conditions: every wave is done with the V buffer,
    // and every wave's part of the next block's K (the only load in flight)
    // has landed, so the next block starts right after the V refill
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue_tile<D, BLK, NW>(sv_w, vbase, vst, tv, jn, L, w, lane);
  }
}

// d = 256: one selected block in passes of KP 32-key tiles: S, the online
// softmax and O += V^T.P^T per pass, so that a pass's S and P (16 + 8
// registers at KP = 1) sit beside the 128 output accumulators and the 64
// query-operand registers of a wave. (At KP = 2 the compiler spilled ~50
// registers to scratch memory and the attention was 14-16 % slower.) This is
// the online softmax over 32-key tiles, a rounding-level difference from the
// reference's 64- or 128-key K_TILE_SIZE. The K refill follows the last
// pass's S, the V refill the last pass's P.V; the V wait precedes the first
// pass's P.V.
template <typename T, int D, int BLK, bool DIAG>
__device__ __forceinline__ void attn_block_passes(AttnState<T, D>& st, const typename T::vec8* qb,
                                                 const uint4* sk, uint4* sk_w,
                                                 const uint16_t* sv16, uint4* sv_w,
                                                 const uint16_t* kbase, const uint16_t* vbase,
                                                 int64_t kst, int64_t vst,
                                                 const TileLanes<D, BLK, BLK / 32>& tk,
                                                 const TileLanes<D, BLK, BLK / 32>& tv, int jn,
                                                 const int32_t* pf, int& jpf, int L, float c,
                                                 bool first, int w, int lane) {
  constexpr int CH = D / 8;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int KT = BLK / 32;  // 32-key tiles of S^T per block
  constexpr int KP = 1;         // key tiles per pass
  constexpr int NP = KT / KP;   // passes
  constexpr int NW = BLK / 32;
  static_assert(KT % KP == 0, "whole passes");
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * w + l32;
  const int live = DIAG ? w + 1 : KT;
  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    // the pass's live tiles (diagonal block: wave w sees tiles 0 .. w)
    const int live_p = DIAG ? min(max(live - p * KP, 0), KP) : KP;
    f32x16 s[KP];
#pragma unroll
    for (int t = 0; t < KP; ++t) s[t] = f32x16{};
    if constexpr (!DIAG) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < KP; ++t) {
          const int r = 32 * (p * KP + t) + l32;
          const uint4 kop = sk[r * CH + ((2 * ks + half) ^ swz<D>(r))];
          s[t] = T::mfma32(as_vec8<T>(kop), qb[ks], s[t]);
        }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReadAhead, 0);
#pragma unroll
      for (int k = 0; k < KS * KP - kReadAhead; ++k) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 0);
    } else {
#pragma unroll
      for (int t = 0; t < KP; ++t) {
        if (t >= live_p) continue;
        const int r = 32 * (p * KP + t) + l32;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint4 kop = sk[r * CH + ((2 * ks + half) ^ swz<D>(r))];
          s[t] = T::mfma32(as_vec8<T>(kop), qb[ks], s[t]);
        }
      }
    }
    if (p == NP - 1) {
      lds_barrier();  // every wave is done with the K buffer
      if (jn >= 0) issue_tile<D, BLK, NW>(sk_w, kbase, kst, tk, jn, L, w, lane);
      jpf = sld(pf);
    }
    if (DIAG && live_p == 0) continue;  // wave-uniform: no key of this pass is visible

    if constexpr (DIAG) {  // key > query is masked on the diagonal block
#pragma unroll
      for (int t = 0; t < KP; ++t) {
        const int t4 = p * KP + t;
        if (t4 < w) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = 32 * t4 + 8 * (v >> 2) + 4 * half + (v & 3);
          if (t4 > w || key > qrow) s[t][v] = -INFINITY;
        }
      }
    }
    // conditional rescaling as in attn_block, per pass
    uint32_t pk[KP][8];
    float ps = 0.0f;
    bool move = first && p == 0;
    if (!move) {
      ps = exp_pack<T, KP>(s, st.m_run, c, live_p, pk);
      move = __ballot(!(ps <= kRescaleSum)) != 0;
    }
    if (move) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < KP; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[t][v]);
      const float m_new = fmaxf(st.m_run, pair32_max(mx) * c);
      float alpha = __builtin_amdgcn_exp2f(st.m_run - m_new);
      if (alpha != alpha) alpha = 1.0f;
      st.l_part *= alpha;
      st.m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) st.o[dt][v] *= alpha;
      ps = exp_pack<T, KP>(s, st.m_run, c, live_p, pk);
    }
    st.l_part += ps;

    if (p == 0) vm_barrier<0>();  // V of this block has landed (no K refill issued yet)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < 2 * KP; ++u) {
      const int t = u >> 1, hh = u & 1;
      if (DIAG && t >= live_p) continue;
      const uint4 pu = make_uint4(pk[t][4 * hh], pk[t][4 * hh + 1], pk[t][4 * hh + 2],
                                  pk[t][4 * hh + 3]);
      const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pu);
      const int r1 = 16 * (2 * KP * p + u) + tr_row;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int x = 32 * dt + tr_col;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, x)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, x)));
        const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
        const uint4 va = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
        st.o[dt] = T::mfma32(as_vec8<T>(va), pb, st.o[dt]);
      }
    }
    if constexpr (!DIAG) {
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kReadAhead, 0);
#pragma unroll
      for (int k = 0; k < 2 * KP * DT - kReadAhead; ++k) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  if (jn >= 0) {
    // every wave is done with the V buffer, and every wave's part of the next
    // block's K (the only load in flight) has landed
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue_tile<D, BLK, NW>(sv_w, vbase, vst, tv, jn, L, w, lane);
  }
}

// Flash-decoding merge of a split row's chunk partials into its output rows,
// inside the attention kernel (rows of at most kMaxInlineChunks chunks):
// m = max_c m_c, w_c = exp2(m_c - m), O = sum_c w_c acc_c / sum_c w_c l_c,
// with the chunks taken in order (the arithmetic of k_merge, so either path
// gives the same bits). Threads: nt / BLK per query row (2 at BLK = 128 and
// 64), each D / 2 dims in rounds of 16; each round issues all of its loads
// before using them (8 chunks x 16 dims: 128 registers, as many as the
// attention itself leaves free). A loop over the chunks here, in any form
// tried, made the compiler drop the LDS read-ahead schedule of the block loop
// in the persistent kernel, so the chunks are unrolled.
template <typename T, int D, int BLK, typename Args>
__device__ __forceinline__ void merge_row(const Args& a, int h, int u0, int nc,
                                          const ItemRec& rec, int t) {
  constexpr int MAXC = kMaxInlineChunks;  // the host merges inline only up to this
  constexpr int NT = 2 * BLK;      // threads of the workgroup
  constexpr int TPR = NT / BLK;    // threads per query row
  constexpr int XT = D / TPR;      // dims per thread
  constexpr int GP = 16;           // dims per round
  const int r = t / TPR;
  const int qg = rec.i * BLK + r;
  if (qg >= rec.L) return;
  nc = min(nc, MAXC);
  const int64_t S = BLK * D + 2 * BLK;  // floats per partial
  const float* p0 = a.part + (static_cast<int64_t>(h) * a.unit_cap + u0) * S;
  float mc[MAXC], lc[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    mc[c] = c < nc ? p0[c * S + BLK * D + r] : -INFINITY;
    lc[c] = c < nc ? p0[c * S + BLK * D + BLK + r] : 0.0f;
  }
  float m = mc[0];
#pragma unroll
  for (int c = 1; c < MAXC; ++c) m = fmaxf(m, mc[c]);
  float wc[MAXC], lsum = 0.0f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    wc[c] = c < nc ? __builtin_amdgcn_exp2f(mc[c] - m) : 0.0f;
    lsum += wc[c] * lc[c];
  }
  const float rcp = 1.0f / lsum;
  const int xb = XT * (t % TPR);
  uint16_t* op = a.o + (rec.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs + xb;
#pragma unroll 1
  for (int x0 = 0; x0 < XT; x0 += GP) {
    float4 oc[MAXC][GP / 4];
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
#pragma unroll
      for (int q = 0; q < GP / 4; ++q)
        oc[c][q] = c < nc ? *reinterpret_cast<const float4*>(
                                p0 + c * S + static_cast<int64_t>(r) * D + xb + x0 + 4 * q)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int q = 0; q < GP / 4; ++q) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        acc.x += wc[c] * oc[c][q].x;
        acc.y += wc[c] * oc[c][q].y;
        acc.z += wc[c] * oc[c][q].z;
        acc.w += wc[c] * oc[c][q].w;
      }
      uint2 pk;
      pk.x = pack2<T>(acc.x * rcp, acc.y * rcp);
      pk.y = pack2<T>(acc.z * rcp, acc.w * rcp);
      *reinterpret_cast<uint2*>(op + x0 + 4 * q) = pk;
    }
  }
}

// The steps of k_merge (rows of up to kMaxChunks chunks), the same arithmetic
// in the same chunk order as merge_row. A partial is S floats: acc[BLK][D],
// then m[BLK], then l[BLK].

// m and 1 / sum_c w_c l_c of query row r over the nc (<= kMaxChunks) partials
// at p0
template <int D, int BLK>
__device__ __forceinline__ void merge_weights(const float* p0, int r, int nc, float& m,
                                              float& rcp) {
  constexpr int64_t S = BLK * D + 2 * BLK;
  constexpr int G = 4;  // chunks per group of loads
  m = -INFINITY;
#pragma unroll
  for (int c0 = 0; c0 < kMaxChunks; c0 += G) {
    if (c0 >= nc) break;
    float mc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) mc[g] = c0 + g < nc ? p0[(c0 + g) * S + BLK * D + r] : -INFINITY;
#pragma unroll
    for (int g = 0; g < G; ++g) m = fmaxf(m, mc[g]);
  }
  float lsum = 0.0f;
#pragma unroll
  for (int c0 = 0; c0 < kMaxChunks; c0 += G) {
    if (c0 >= nc) break;
    float mc[G], lc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mc[g] = c0 + g < nc ? p0[(c0 + g) * S + BLK * D + r] : -INFINITY;
      lc[g] = c0 + g < nc ? p0[(c0 + g) * S + BLK * D + BLK + r] : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (c0 + g < nc) lsum += __builtin_amdgcn_exp2f(mc[g] - m) * lc[g];
  }
  rcp = 1.0f / lsum;
}

// NX dims of query row r starting at dim x: sum_c w_c acc_c / sum_c w_c l_c,
// stored to op in the output type. The chunks are taken four at a time, every
// load of a group issued before any is used.
template <typename T, int D, int BLK, int NX>
__device__ __forceinline__ void merge_slice(const float* p0, int r, int x, int nc, float m,
                                            float rcp, uint16_t* op) {
  constexpr int64_t S = BLK * D + 2 * BLK;
  constexpr int G = 4;
  float4 acc[NX / 4];
#pragma unroll
  for (int q = 0; q < NX / 4; ++q) acc[q] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int c0 = 0; c0 < nc; c0 += G) {
    float wc[G];
    float4 oc[G][NX / 4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const bool on = c0 + g < nc;
      const float* pc = p0 + (c0 + g) * S;
      wc[g] = on ? pc[BLK * D + r] : -INFINITY;
#pragma unroll
      for (int q = 0; q < NX / 4; ++q)
        oc[g][q] = on ? *reinterpret_cast<const float4*>(pc + static_cast<int64_t>(r) * D + x + 4 * q)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float w = c0 + g < nc ? __builtin_amdgcn_exp2f(wc[g] - m) : 0.0f;
#pragma unroll
      for (int q = 0; q < NX / 4; ++q) {
        acc[q].x += w * oc[g][q].x;
        acc[q].y += w * oc[g][q].y;
        acc[q].z += w * oc[g][q].z;
        acc[q].w += w * oc[g][q].w;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NX / 4; ++q) {
    uint2 pk;
    pk.x = pack2<T>(acc[q].x * rcp, acc[q].y * rcp);
    pk.y = pack2<T>(acc[q].z * rcp, acc[q].w * rcp);
    *reinterpret_cast<uint2*>(op + 4 * q) = pk;
  }
}

// Arrival of one chunk of a split row (its partials stored by every thread):
// the chunk that completes the row's count merges it. All chunks of a row
// run on one XCD (AttnArgs::merge_inline), so they share its L2. Release:
// every thread waits until its stores are done (in L2), then the workgroup
// barrier, then one atomic increment (performed in L2). Acquire, by the last
// chunk: after the atomic returns, this CU's L1 is invalidated, so the other
// chunks' partials are read from L2. (These are the instructions the
// compiler emits for a workgroup-scope release / acquire when a workgroup's
// waves may sit on different CUs of one L2.)
template <typename T, int D, int BLK, typename Args>
__device__ __forceinline__ void merge_if_last(const Args& a, int h, int u0, int nc,
                                              const ItemRec& rec, int t) {
  __shared__ int s_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (t == 0) {
    int32_t* cnt = a.arrivals + static_cast<int64_t>(h) * a.unit_cap + u0;
    s_last = atomicAdd(cnt, 1) == nc - 1;
    // every chunk of the row has arrived: re-arm the counter, so that an
    // attention launch repeated on the same plan starts from zero as well
    if (s_last) atomicExch(cnt, 0);
  }
  __syncthreads();
  if (!s_last) return;
  asm volatile("buffer_inv sc0" ::: "memory");
  merge_row<T, D, BLK>(a, h, u0, nc, rec, t);
}

// One work slot of the attention grid: a chunk unit (slot < unit_slots) or
// a row. Every wave returns together (the early returns depend on the slot
// only). The K and V buffers are the workgroup's static LDS. `tail()` runs
// once the slot's last block is done, before the output is normalised and
// stored (the persistent grid claims its next slot there, so the claim's
// latency passes behind the stores); returns whether it ran.
template <typename T, int D, int BLK, typename Args, typename Tail>
__device__ __forceinline__ bool attn_slot(const Args& a, int slot, int t, Tail tail) {
  constexpr int CH = D / 8;   // 16-byte chunks per row
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-row tiles of O^T
  constexpr int NW = BLK / 32;
  __shared__ uint4 sk[BLK * CH];
  __shared__ uint4 sv[BLK * CH];

  // Work item: the first unit_slots slots take the chunks of the split
  // rows (a slice of a dense row's list, fp32 partials out), the others one
  // (head, sequence, q-block) row each through map_row. For a row, the item
  // record, the row record written by the selection stage (count, first two
  // list entries, diagonal kept) and the item count are three independent
  // scalar loads, so the row's first tile loads follow after one scalar-load
  // latency.
  ItemRec rec;
  int h, ncnt, j0, jraw, unit = -1;
  bool has_diag;
  int64_t first = 0;  // list offset of the chunk
  if (slot < a.unit_slots) {
    int u;
    map_item(static_cast<int>(slot), a.Hq, u, h);
    const int nunits = sld(a.units);
    if (u >= nunits) return false;
    const UnitRec ur =
        sld(reinterpret_cast<const UnitRec*>(reinterpret_cast<const char*>(a.units) + 64) + u);
    rec = ur.r;
    // a split row selects every causal block, so its list is 0 .. i and the
    // chunk's entries are first .. first + ncnt - 1; the diagonal block is the
    // last chunk's last entry
    first = static_cast<int64_t>(ur.c) * a.split_blocks;
    ncnt = max(min(a.split_blocks, rec.i + 1 - static_cast<int>(first)), 0);
    j0 = static_cast<int>(first);
    jraw = j0 + 1;
    has_diag = ncnt > 0 && ur.c == ur.nc - 1;
    unit = u;
  } else {
    int item;
    map_row(static_cast<int>(slot - a.unit_slots), a.Hq, a.Hkv, a.nb_sum_cap, item, h);
    const int64_t nitems = sld(a.tab.seq_tile + a.B);
    // map_row can return items up to 8 / Hkv - 1 past the table's capacity;
    // those (and any item >= nitems) return below, so the loads are clamped
    const int64_t it = min(static_cast<int64_t>(item), a.nb_sum_cap - 1);
    rec = sld(a.tab.items + it);
    int4 rrec = sld(reinterpret_cast<const int4*>(a.rowrec) +
                    static_cast<int64_t>(h) * a.nb_sum_cap + it);
    // block_size 256: the selection wrote the records of a row pair by tile
    // (a second, dependent load; at ratio 1 the first load is independent)
    if (a.ratio > 1)
      rrec = sld(reinterpret_cast<const int4*>(a.rowrec) + static_cast<int64_t>(h) * a.nb_sum_cap +
                 min(max(rec.tile, 0), static_cast<int32_t>(a.nb_sum_cap - 1)));
    if (item >= nitems) return false;
    // the chunks of a split row produce its output
    if (row_is_split(rec.i, (rec.L + BLK - 1) / BLK, a.last_n, a.split_blocks)) return false;
    // counts and entries come from the search stage; clamp them to the row's
    // capacity so a stale workspace can never index outside the sequence
    ncnt = min(max(rrec.x, 0), rec.i + 1);
    j0 = rrec.y;
    jraw = ncnt > 1 ? rrec.z : 0;
    // the diagonal block, when selected, is the last entry of the ascending list
    has_diag = ncnt > 0 && rrec.w != 0;
  }
  const int i = rec.i, L = rec.L;
  const int64_t t0 = rec.t0;
  const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + rec.tri;
  const int32_t* list = a.idx + row_tri + first;
  const int kvh = h / (a.Hq / a.Hkv);

  const int lane = t & 63;  // t: threadIdx.x
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // wave index, kept in an SGPR
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * w + l32;           // query row inside the block
  const int qg = i * BLK + qrow;            // query position inside the sequence
  const bool qvalid = qg < L;
  const float c = a.sm_scale_log2;

  const uint16_t* kbase = a.k + t0 * a.kst + static_cast<int64_t>(kvh) * a.khs;
  const uint16_t* vbase = a.v + t0 * a.vst + static_cast<int64_t>(kvh) * a.vhs;

  TileLanes<D, BLK, NW> tk, tv;
  tk.init(a.kst, w, lane);
  tv.init(a.vst, w, lane);
  if (ncnt > 0) {
    const int jc = min(max(j0, 0), i);
    issue_tile<D, BLK, NW>(sk, kbase, a.kst, tk, jc, L, w, lane);
    issue_tile<D, BLK, NW>(sv, vbase, a.vst, tv, jc, L, w, lane);
  }
  // Q^T as MFMA B operand (lane: query l32, dims 16 s + 8 half .. +7), loaded
  // after the first block's tile loads and waited for here, so one memory
  // latency covers both: vector memory operations complete in issue order, so
  // this wait (and any compiler wait for a register load) also waits for every
  // tile load issued before it. The block loop therefore issues no register
  // loads; list entries come through the scalar cache.
  typename T::vec8 qb[KS];
  {
    const uint16_t* qp = a.q + (t0 + qg) * a.qst + static_cast<int64_t>(h) * a.qhs + 8 * half;
    u32x4 u[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) u[s] = __builtin_bit_cast(u32x4, qvalid ? ld16(qp + 16 * s) : zero4());
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      asm volatile("" : "+v"(u[s]));
      qb[s] = as_vec8<T>(__builtin_bit_cast(uint4, u[s]));
    }
  }
  if (ncnt > 0) vm_barrier<0>();  // the first block's K and V have landed

  AttnState<T, D> st;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) st.o[dt] = f32x16{};
  st.m_run = -INFINITY;
  // the two halves' partial sums add up to l: a row starts from the
  // reference's l = 1.0 (cleared by its first block's rescale, alpha =
  // exp2(-inf) = 0), a chunk of a split row from l = 0
  st.l_part = half == 0 && unit < 0 ? 1.0f : 0.0f;

  const uint16_t* sv16 = reinterpret_cast<const uint16_t*>(sv);
  const int nplain = ncnt - (has_diag ? 1 : 0);
  // block n refills the buffers with entry n + 1 and prefetches entry n + 2
  // (entry ncnt - 1 past the end of the list; not used then)
  for (int n = 0; n < nplain; ++n) {
    const int jn = n + 1 < ncnt ? min(max(jraw, 0), i) : -1;
    if constexpr (D > 128) {
      attn_block_passes<T, D, BLK, false>(st, qb, sk, sk, sv16, sv, kbase, vbase, a.kst, a.vst, tk,
                                         tv, jn, list + min(n + 2, ncnt - 1), jraw, L, c, n == 0,
                                         w, lane);
    } else {
      attn_block<T, D, BLK, false>(st, qb, sk, sk, sv16, sv, kbase, vbase, a.kst, a.vst, tk, tv,
                                   jn, list + min(n + 2, ncnt - 1), jraw, L, c, n == 0, w, lane);
    }
  }
  if (has_diag) {
    int unused;
    if constexpr (D > 128) {
      attn_block_passes<T, D, BLK, true>(st, qb, sk, sk, sv16, sv, kbase, vbase, a.kst, a.vst, tk,
                                        tv, -1, list, unused, L, c, nplain == 0, w, lane);
    } else {
      attn_block<T, D, BLK, true>(st, qb, sk, sk, sv16, sv, kbase, vbase, a.kst, a.vst, tk, tv, -1,
                                  list, unused, L, c, nplain == 0, w, lane);
    }
  }

  tail();
  const float l = pair32_sum(st.l_part);
  if (unit >= 0) {
    // chunk of a split row: unnormalised O^T, the running max and l, for k_merge
    float* pp = a.part + (static_cast<int64_t>(h) * a.unit_cap + unit) *
                             static_cast<int64_t>(BLK * D + 2 * BLK);
    float* orow = pp + static_cast<int64_t>(qrow) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<float4*>(orow + 32 * dt + 8 * g4 + 4 * half) =
            make_float4(st.o[dt][4 * g4], st.o[dt][4 * g4 + 1], st.o[dt][4 * g4 + 2],
                        st.o[dt][4 * g4 + 3]);
    if (half == 0) {
      pp[BLK * D + qrow] = st.m_run;
      pp[BLK * D + BLK + qrow] = l;
    }
    if (a.merge_inline) {
      // the unit record is read again rather than kept live across the block loop
      const UnitRec ur = sld(
          reinterpret_cast<const UnitRec*>(reinterpret_cast<const char*>(a.units) + 64) + unit);
      merge_if_last<T, D, BLK>(a, h, unit - ur.c, ur.nc, ur.r, t);
    }
    return true;
  }
  // The normalised 32 x D output tile of the wave goes through its own slice
  // of the K buffer (idle: the last block's S is done, and no K refill
  // follows it) in the swizzled tile layout, then out as whole rows: 16 bytes
  // per lane, 64 / CH rows per store instruction. (Stored straight from the
  // accumulator layout, each instruction wrote 16 bytes into each of 32 rows.)
  const float rcp = 1.0f / l;
  uint16_t* so = reinterpret_cast<uint16_t*>(sk) + w * (32 * D);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      uint2 pk;
      pk.x = pack2<T>(st.o[dt][4 * g4 + 0] * rcp, st.o[dt][4 * g4 + 1] * rcp);
      pk.y = pack2<T>(st.o[dt][4 * g4 + 2] * rcp, st.o[dt][4 * g4 + 3] * rcp);
      *reinterpret_cast<uint2*>(so + tile_elem<D>(l32, 32 * dt + 8 * g4 + 4 * half)) = pk;
    }
  // lanes read what other lanes of the wave wrote: the wave's LDS operations
  // run in order; this keeps the compiler from moving the reads above the writes
  __builtin_amdgcn_wave_barrier();
  constexpr int RPI = 64 / CH;  // rows per store instruction
  const int oc = lane % CH;  // the lane's 16-byte chunk of a row
#pragma unroll
  for (int k = 0; k < 32 / RPI; ++k) {
    const int r = RPI * k + lane / CH;  // the wave's query row
    const uint4 val = *reinterpret_cast<const uint4*>(so + tile_elem<D>(r, 8 * oc));
    if (i * BLK + 32 * w + r < L)
      *reinterpret_cast<uint4*>(a.o + (t0 + i * BLK + 32 * w + r) * a.ost +
                                static_cast<int64_t>(h) * a.ohs + 8 * oc) = val;
  }
  return true;
}

// BLK = 128: 4 waves, 64 KB of LDS (d = 128), two workgroups per CU;
// BLK = 64: 2 waves, 32 KB, four workgroups per CU. Either way two waves per
// SIMD (the second launch bound is waves per execution unit), i.e. at most
// 256 registers per wave. At d = 256 (32-key passes per block) the output
// accumulators take 128 registers and the query operands 64: a wave runs
// alone on its SIMD (up to 512 registers, VGPRs and AGPRs), one workgroup
// per CU at BLK = 128 (128 KB of LDS), two at BLK = 64.
//
// PERSIST = false: one workgroup per slot (grid = total_slots), in slot order.
// PERSIST = true: a resident grid (a multiple of 8 workgroups, as many as fit)
// whose workgroups on XCD x = id % 8 take the slots x, x + 8, x + 16, ...:
// each its own id first, then claims from queue[x] one at a time, i.e. the
// slots of an XCD in the same order the hardware dispatcher would give them,
// without its gaps between a finished row and the next workgroup. A slot past
// total_slots ends the workgroup's loop; the last claim of a queue empties it
// for the next launch.
template <typename T, int D, int BLK, bool PERSIST>
__global__ __launch_bounds__(2 * BLK, D > 128 ? 1 : 2) void k_attn(AttnArgs a) {
  // The arguments are read from the kernel-argument segment through a
  // pointer (made opaque on every pass of the persistent loop, so that the
  // compiler reloads them per slot with scalar loads instead of keeping ~70 of
  // them live in SGPRs across the loop, which spills).
  const __attribute__((address_space(4))) AttnArgs* ap =
      (const __attribute__((address_space(4))) AttnArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  if constexpr (!PERSIST) {
    attn_slot<T, D, BLK>(*ap, static_cast<int>(blockIdx.x), static_cast<int>(threadIdx.x), [] {});
  } else {
    __shared__ int claim;
    const int x = static_cast<int>(blockIdx.x & 7);
    // the first slot of workgroup b is slot b itself (no claim); the queue of
    // XCD x then hands out its later slots 8 (G + k) + x, k = 0, 1, ..., where
    // G = gridDim.x / 8 workgroups run on each XCD
    const int64_t g8 = gridDim.x >> 3;
    // Claim of the next slot by thread 0 into `claim`. Re-arm: every
    // workgroup of XCD x whose first slot was valid claims until one claim
    // fails, so the claims of this launch end at k = valid + claimers - 1;
    // the workgroup that gets it has made the queue's last access and
    // empties it for the next launch.
    auto claim_next = [&] {
      if (threadIdx.x == 0) {
        const int k = atomicAdd(&ap->queue[x], 1);
        claim = k;
        const int64_t per_x = (ap->total_slots - x + 7) >> 3;  // slots of XCD x
        const int64_t valid = per_x > g8 ? per_x - g8 : 0;      // claimable ones
        const int64_t claimers = per_x < g8 ? per_x : g8;
        if (k == valid + claimers - 1) atomicExch(&ap->queue[x], 0);
      }
    };
    int64_t slot = blockIdx.x;
    for (;;) {
      asm volatile("" : "+s"(ap));
      if (slot >= ap->total_slots) break;
      // the thread index is made opaque per slot, so that lane-derived values
      // (tile-load offsets, operand addresses) are formed per slot rather than
      // hoisted out of this loop, where they would stay live across it
      int t = static_cast<int>(threadIdx.x);
      asm volatile("" : "+v"(t));
      if (!attn_slot<T, D, BLK>(*ap, static_cast<int>(slot), t, claim_next)) claim_next();
      __syncthreads();  // K / V buffers are free and `claim` is set
      slot = 8 * (g8 + claim) + x;
      __syncthreads();  // every wave has read `claim`
    }
  }
}

// Output rows of the split rows. Workgroup (slot, s) of the grid
// (unit_slots x BLK / 32) takes query rows 32 s .. 32 s + 31 of the unit that
// k_attn's chunk slot `slot` ran; only a row's first chunk's slots work. Eight
// threads per query row, D / 8 dims each (merge_weights, then merge_slice:
// about one memory latency per four chunks).
template <typename T, int D, int BLK>
__global__ __launch_bounds__(256) void k_merge(AttnArgs a) {
  constexpr int XT = D / 8;        // dims per thread
  const int slot = static_cast<int>(blockIdx.x / (BLK / 32));
  const int s = static_cast<int>(blockIdx.x % (BLK / 32));
  int u, h;
  map_item(slot, a.Hq, u, h);
  const int nunits = sld(a.units);
  if (u >= nunits) return;
  const UnitRec ur =
      sld(reinterpret_cast<const UnitRec*>(reinterpret_cast<const char*>(a.units) + 64) + u);
  if (ur.c != 0) return;
  const int nc = min(min(ur.nc, nunits - u), kMaxChunks);
  const int r = 32 * s + static_cast<int>(threadIdx.x >> 3);
  const int x0 = XT * static_cast<int>(threadIdx.x & 7);
  const int qg = ur.r.i * BLK + r;
  if (qg >= ur.r.L) return;
  const float* p0 =
      a.part + (static_cast<int64_t>(h) * a.unit_cap + u) * static_cast<int64_t>(BLK * D + 2 * BLK);
  float m, rcp;
  merge_weights<D, BLK>(p0, r, nc, m, rcp);
  uint16_t* op = a.o + (ur.r.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs + x0;
  merge_slice<T, D, BLK, XT>(p0, r, x0, nc, m, rcp, op);
}

template <typename T, int D>
hipError_t launch_attn_t(const AttnArgs& a, int block, int64_t grid, bool persist, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (block == 128) {
    if (persist) hipLaunchKernelGGL((k_attn<T, D, 128, true>), g, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_attn<T, D, 128, false>), g, dim3(256), 0, s, a);
  } else {
    if (persist) hipLaunchKernelGGL((k_attn<T, D, 64, true>), g, dim3(128), 0, s, a);
    else hipLaunchKernelGGL((k_attn<T, D, 64, false>), g, dim3(128), 0, s, a);
  }
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_merge_t(const AttnArgs& a, int block, hipStream_t s) {
  if (block == 128)
    hipLaunchKernelGGL((k_merge<T, D, 128>), dim3(static_cast<unsigned>(a.unit_slots * 4)),
                       dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((k_merge<T, D, 64>), dim3(static_cast<unsigned>(a.unit_slots * 2)),
                       dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_merge(const AttnArgs& a, int dtype, int head_dim, int block, hipStream_t s) {
  if (a.unit_slots <= 0 || dtype == FP_DTYPE_F32) return hipSuccess;
  return with_head_dim(head_dim, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return dtype == FP_DTYPE_BF16 ? launch_merge_t<BF16, D>(a, block, s)
                                  : launch_merge_t<F16, D>(a, block, s);
  });
}

hipError_t launch_attn(const AttnArgs& a, int dtype, int head_dim, int block, int64_t grid,
                       bool persist, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  return with_head_dim(head_dim, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return dtype == FP_DTYPE_BF16 ? launch_attn_t<BF16, D>(a, block, grid, persist, s)
                                  : launch_attn_t<F16, D>(a, block, grid, persist, s);
  });
}

}  // namespace fp
