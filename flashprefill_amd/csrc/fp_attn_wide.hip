// Block-sparse attention with 64 queries per wave for gfx950 (reference:
// ops/flashprefill_native_forward.py:227-344, ops/flashprefill_varlen_func.py:
// 449-575; operand layouts as k_attn in fp_attn.hip).
//
// One workgroup of two waves owns one (query head, sequence, q-block) row;
// wave w owns queries 64w .. 64w+63 as two 32-query MFMA column tiles and runs
// alone on its SIMD (two workgroups per CU). Every K operand (S = K . Q^T) and
// every V^T operand (O^T += V^T . P^T) read from LDS feeds two MFMAs, one per
// query tile, so a wave reads 32 KB of LDS per 64 MFMAs, half of what the
// 32-queries-per-wave kernels read per MFMA.
//
// The selected key blocks are consumed as 64-key half tiles t (the
// reference's K_TILE_SIZE = 64 configuration). With one wave per SIMD nothing
// hides one instruction stream's latency behind another's, so the wave
// software-pipelines its own work and interleaves VALU with MFMA by hand:
//
//   step t (S(t) is in registers, its row max and alpha already known)
//     barrier A   K(t+1) has landed; V(t+1) load issued
//     O *= alpha(t)                                  (only if some max moved)
//     block 2     S(t+1) = K(t+1) . Q^T MFMAs  ||  exp2 / row sum / pack of
//                 the first 20 of S(t)'s 32 value pairs per lane
//     barrier B   V(t) has landed; K(t+3) load issued
//     block 3     O^T += V(t)^T . P(t)^T MFMAs  ||  the remaining 12 pairs
//                 (before the k-steps that need them), then S(t+1) out of
//                 the accumulators, its causal mask, row max and alpha(t+1)
//
// K and V are double-buffered in LDS (64 KB per workgroup at d = 128) and
// loaded with direct-to-LDS loads two steps ahead; every step issues the same
// number of loads (past the row end a step loads the sequence's first rows
// into a buffer that is never read), so the explicit vmcnt waits are
// constants. The row's block list is held in a VGPR (entry n of the current
// 64-entry chunk in lane n % 64) and read with readlane.
//
// The diagonal block, always the last of an ascending list when selected, is
// masked (key > query) when its scores are formed; the main loop runs the
// unmasked steps.
//
// Numerics: the reference loop with a 64-key tile — m = -inf and l = 1.0 at
// row start, alpha = exp2(m_old - m_new) with NaN -> 1, l accumulates the fp32
// p, P is rounded to the input dtype before P.V, O = acc * (1/l) — except that
// m is the reference max of conditional rescaling (kRescaleSlack), so P
// is rounded at a different scale than in the reference (rounding-level
// differences in O).
#include <type_traits>

#include "fp_attn_common.h"

namespace fp {

// Lane offsets of the direct-to-LDS loads of a 64-row half tile shared by the
// NW waves of a workgroup: wave w fills 1 KB slices w*NI .. w*NI+NI-1 (4 rows
// each at d = 128). off[p] is the lane's byte offset inside a slice whose
// index is p modulo the swizzle period; the slice's own row offset goes into
// the scalar base.
template <int D, int NW>
struct WideLanes {
  static constexpr int CH = D / 8;              // 16-byte chunks per row
  static constexpr int RPW = 64 / CH;           // rows per 1 KB slice
  static constexpr int NI = CH / NW;            // slices per wave per half tile
  static constexpr int PER = D == 128 ? 4 : 2;  // period of swz over the slice index
  uint32_t off[PER];
  __device__ __forceinline__ void init(int64_t stride, int w, int lane) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int r = (w * NI + p) * RPW + lane / CH;
      const int c = (lane % CH) ^ swz<D>(r);
      off[p] = static_cast<uint32_t>(((lane / CH) * stride + 8 * c) * 2);
    }
  }
};

// This wave's loads of the half tile whose first row is at `base` into the LDS
// buffer at byte address `lds`; rows at or past `nvalid` read row nvalid - 1
// (their keys are masked).
template <int D, int NW>
__device__ __forceinline__ void wide_tile(uint32_t lds, const uint16_t* base, int stride,
                                          const WideLanes<D, NW>& tl, int nvalid, int w,
                                          int lane) {
  using TL = WideLanes<D, NW>;
  constexpr int CH = TL::CH, RPW = TL::RPW, NI = TL::NI;
  if (nvalid >= 64) {
    // one scalar base per tile; the slices' row offsets are scalar adds
    uint64_t sb = scalar_addr(base);
    // the base was written by VALU (readfirstlane): five wait states before
    // a VMEM instruction reads it; every later use goes through this asm
    asm volatile("s_nop 4" : "+s"(sb));
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int slot = w * NI + q;
      dma16_sbase_m0(lds + slot * 1024, sb + static_cast<uint64_t>(slot * RPW * stride) * 2,
                     tl.off[q % TL::PER]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int slot = w * NI + q;
      const int r = slot * RPW + lane / CH;
      const int c = (lane % CH) ^ swz<D>(r);
      const int gk = min(r, nvalid - 1);
      dma16_vaddr_at(lds + slot * 1024, base + static_cast<int64_t>(gk) * stride + 8 * c);
    }
  }
}

// QT 32-query MFMA column tiles per wave; NW = 4 / QT waves per workgroup
// share the row's 128 queries and its K / V tiles. QT = 2: one wave per SIMD
// (the O, S and Q^T registers of two query tiles need the AGPRs); QT = 1: two
// waves per SIMD, everything in VGPRs.
template <typename T, int D, int QT>
__global__ __launch_bounds__(256 / QT) __attribute__((amdgpu_waves_per_eu(3 - QT, 3 - QT)))
void k_attn_wide(AttnArgs a) {
  constexpr int NW = 4 / QT;   // waves per workgroup
  constexpr int CH = D / 8;   // 16-byte chunks per key row
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-row tiles of O^T
  constexpr int HT = 64 * CH;  // uint4 per half tile
  constexpr int NI = WideLanes<D, NW>::NI;
  constexpr uint32_t TB = HT * 16;  // bytes per half tile
  __shared__ uint4 sk[2][HT];
  __shared__ uint4 sv[2][HT];

  int item, h;
  map_item(blockIdx.x, a.Hq, item, h);
  const int64_t nitems = sld(a.tab.seq_tile + a.B);
  if (item >= nitems) return;
  const ItemRec rec = sld(a.tab.items + item);
  const int i = rec.i, L = rec.L;
  const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + rec.tri;
  // counts and lists come from the search stage; clamp them to the row's
  // capacity so a stale workspace can never index outside the sequence
  const int ncnt = min(max(sld(a.cnt + static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile), 0),
                       i + 1);
  const int32_t* list = a.idx + row_tri;
  const int kvh = h / (a.Hq / a.Hkv);
  const int kst = static_cast<int>(a.kst), vst = static_cast<int>(a.vst);
  const uint16_t* kbase = a.k + rec.t0 * a.kst + static_cast<int64_t>(kvh) * a.khs;
  const uint16_t* vbase = a.v + rec.t0 * a.vst + static_cast<int64_t>(kvh) * a.vhs;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const float c = a.sm_scale_log2;
  const int rem = L - i * kBlock;  // rows of this q-block inside the sequence

  if (ncnt == 0) {  // no block selected: m = -inf, l = 1, O = 0
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qg = i * kBlock + 32 * (QT * w + qt) + l32;
      if (qg < L) {
        uint16_t* op = a.o + (rec.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs;
#pragma unroll
        for (int dd = 0; dd < D; dd += 8) *reinterpret_cast<uint4*>(op + dd) = zero4();
      }
    }
    return;
  }

  // block list, chunk 0, and Q^T as MFMA B operands of both query tiles
  // (lane: query l32, dims 16 s + 8 half .. +7); both are waited for here,
  // before any tile load is in flight
  int chunk = 0;
  int listv = lane < ncnt ? list[lane] : 0;
  typename T::vec8 qb[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qg = i * kBlock + 32 * (QT * w + qt) + l32;
    const bool qvalid = qg < L;
    const uint16_t* qp = a.q + (rec.t0 + qg) * a.qst + static_cast<int64_t>(h) * a.qhs + 8 * half;
    u32x4 u[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) u[s] = __builtin_bit_cast(u32x4, qvalid ? ld16(qp + 16 * s) : zero4());
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      asm volatile("" : "+v"(u[s]));
      if constexpr (QT == 2) asm volatile("" : "+a"(u[s]));  // B operands are read from AGPRs
      qb[qt][s] = as_vec8<T>(__builtin_bit_cast(uint4, u[s]));
    }
  }
  asm volatile("" : "+v"(listv));
  // entry n of the list (n ascending over the row, chunks loaded on demand)
  auto lookup = [&](int n) -> int {
    if ((n >> 6) != chunk) {
      chunk = n >> 6;
      int ln = lane;
      asm volatile("" : "+v"(ln));  // address formed here, not held across the row
      const int e = (n & ~63) + ln;
      listv = e < ncnt ? list[e] : 0;
      // waited for here: a wait at the readlane below would sit in every step
      // and drain the tile loads in flight
      asm volatile("" : "+v"(listv));
    }
    return min(max(__builtin_amdgcn_readlane(listv, n & 63), 0), i);
  };
  const bool diag_last = min(max(sld(list + ncnt - 1), 0), i) == i;
  const int nsteps = 2 * ncnt;  // half tiles of the row

  WideLanes<D, NW> tk, tv;
  tk.init(a.kst, w, lane);
  tv.init(a.vst, w, lane);
  const uint32_t sk0 = lds_addr(&sk[0][0]), sv0 = lds_addr(&sv[0][0]);
  // this wave's loads of half tile s & 1 of block jb (jb < 0: a tile past the
  // row end) into buffer s & 1
  auto tile_rows = [&](int s, int jb, int& row0, int& rows) {
    row0 = 0;
    rows = min(L, 64);
    if (jb >= 0) {
      row0 = jb * kBlock + 64 * (s & 1);
      rows = jb == i ? rem - 64 * (s & 1) : 64;
      if (rows <= 0) {  // second half past the sequence end: its last row
        row0 = L - 1;
        rows = 1;
      }
    }
  };
  auto load_k = [&](int s, int jb) {
    int row0, rows;
    tile_rows(s, jb, row0, rows);
    wide_tile<D, NW>(sk0 + (s & 1) * TB, kbase + static_cast<int64_t>(row0) * a.kst, kst, tk,
                     rows, w, lane);
  };
  auto load_v = [&](int s, int jb) {
    int row0, rows;
    tile_rows(s, jb, row0, rows);
    wide_tile<D, NW>(sv0 + (s & 1) * TB, vbase + static_cast<int64_t>(row0) * a.vst, vst, tv,
                     rows, w, lane);
  };

  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

  f32x16 o[DT][QT];
  float m_cur[QT], alpha_cur[QT], l_part[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt][qt] = f32x16{};
    l_part[qt] = half == 0 ? 1.0f : 0.0f;  // the two halves' partial sums add up to l
    m_cur[qt] = -INFINITY;
    alpha_cur[qt] = 1.0f;
  }

  // block of the latest K and V tile loads
  int jk = lookup(0), jv = jk;
  // prologue: K(0); a V load into the buffer V(1) will use, whose wait keeps
  // the per-step wait counts uniform; K(1)
  load_k(0, jk);
  load_v(1, -1);
  load_k(1, jk);

  float ps[QT][2];  // row sums of the P being formed
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) ps[qt][0] = ps[qt][1] = 0.0f;
  // P as the B operands of the four P.V k-steps. Entries of k-steps 0/1 are
  // rewritten (for S(t)) after the P.V MFMAs of step t-1 that read them have
  // issued, entries of k-steps 2/3 in the next step's block 1, so one buffer
  // serves both steps.
  uint32_t pk[QT][4][4];
  // S accumulators: key tile kt = 1 of S(t) stays here until block 1 of step
  // t+1 has read it, right before that block's kt = 1 MFMAs overwrite it
  f32x16 sacc[2][QT];
  // exp2 / row sum / pack of value pair p2 (values 2 p2, 2 p2 + 1) of key tile
  // kt, query tile qt: B operand k-step 2 kt + p2 / 4, element pair p2 % 4
  auto unit = [&](int kt, int qt, int p2, const f32x16& src) {
    const float p0 = __builtin_amdgcn_exp2f(fmaf(src[2 * p2], c, -m_cur[qt]));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(src[2 * p2 + 1], c, -m_cur[qt]));
    uint32_t& dst = pk[qt][2 * kt + (p2 >> 2)][p2 & 3];
    dst = pack2<T>(p0, p1);
    float& acc = ps[qt][p2 & 1];
    acc = add_pair<T>(dst, acc);  // l adds the rounded P that P.V consumes
    // computed here, in the MFMA block it is interleaved with, not sunk to
    // the P.V MFMAs that read it
    asm volatile("" : "+v"(dst), "+v"(acc));
  };
  // key > query on the diagonal block (half tile hf, key tile kt)
  auto mask = [&](f32x16& x, int hf, int kt, int qt) {
    // key 64 hf + 32 kt + 8 (v / 4) + 4 half + v % 4 > query 32 (QT w + qt) + l32,
    // with the lane part moved to the right so the key constants stay immediates;
    // the lane terms are recomputed here rather than held across the row
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int lim = 32 * (QT * w + qt) + (ln & 31) - 64 * hf - 4 * (ln >> 5) - 32 * kt;
#pragma unroll
    for (int v = 0; v < 16; ++v)
      if (8 * (v >> 2) + (v & 3) > lim) x[v] = -INFINITY;
  };

  // step t: S(t) (HS), P.V of step t-1 (HP), S(t) on the diagonal block (CD),
  // S(t-1) on the diagonal block (PCD). The flags are compile-time constants
  // (std::bool_constant) in the main loop and wave-uniform runtime values in
  // the prologue and the tail, which share one copy of the code.
  auto step = [&](auto hs_c, auto hp_c, auto cd_c, auto pcd_c, int t) {
    const bool HS = hs_c, HP = hp_c, CD = cd_c, PCD = pcd_c;
    if ((t & 1) == 0) {  // V(t) starts the block of K(t); K(t+2) the next one
      jv = jk;
      if (t + 2 < nsteps) jk = lookup((t + 2) >> 1);
    }
    // barrier X: K(t) has landed (after it: V(t-1), K(t+1)); V(t-2) is read.
    // V(t) is issued after the first MFMAs of block 1, K(t+2) after the first
    // MFMAs of block 2.
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * NI) : "memory");
    if (HP) {  // O *= alpha(t-1), between P.V(t-2) and P.V(t-1)
      bool moved = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) moved = moved || alpha_cur[qt] != 1.0f;
      if (__ballot(moved)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            // AGPR-held accumulators are read out only on this (rare) path
            if constexpr (QT == 2) asm volatile("" : "+a"(o[dt][qt]));
            o[dt][qt] *= alpha_cur[qt];
          }
      }
    }

    // block 1: S(t) MFMAs, key tile 0 then key tile 1, interleaved with the
    // units of key tile 1 of S(t-1): its accumulators are read during the
    // key tile 0 MFMAs, before the key tile 1 MFMAs overwrite them
    {
      const uint4* skb = t & 1 ? sk[1] : sk[0];
      auto read_k = [&](int ks, int kt) -> uint4 {
        const int r = 32 * kt + l32;
        return skb[r * CH + ((2 * ks + half) ^ swz<D>(r))];
      };
      f32x16 old1[QT];
      if (HP) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          old1[qt] = sacc[1][qt];
          asm volatile("" : "+v"(old1[qt]));  // read out of the accumulators here
        }
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        uint4 ka[2];
        if (HS) {
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) sacc[kt][qt] = f32x16{};
          ka[0] = read_k(0, kt);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          if (HS) {
            if (ks + 1 < KS) ka[(ks + 1) & 1] = read_k(ks + 1, kt);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
              sacc[kt][qt] = T::mfma32(as_vec8<T>(ka[ks & 1]), qb[qt][ks], sacc[kt][qt]);
          }
          if (kt == 0 && ks == 0) load_v(t, HS ? jv : -1);  // V(t), between MFMAs
          __builtin_amdgcn_sched_barrier(0);
          if (HP) {
            if (kt == 0 && ks == 0) {
              if (PCD) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) mask(old1[qt], (t - 1) & 1, 1, qt);
              }
            }
            // 8 QT units over the 2 * KS k-steps of this block
#pragma unroll
            for (int x = (8 * QT * (kt * KS + ks)) / (2 * KS);
                 x < (8 * QT * (kt * KS + ks + 1)) / (2 * KS); ++x)
              unit(1, x >> 3, x & 7, old1[x >> 3]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    if (HP) {  // l(t-1) = l(t-2) * alpha(t-1) + rowsum(P(t-1))
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        l_part[qt] = l_part[qt] * alpha_cur[qt] + (ps[qt][0] + ps[qt][1]);
        ps[qt][0] = ps[qt][1] = 0.0f;
      }
    }

    // barrier Y: V(t-1) has landed (after it: K(t+1), V(t)); K(t) is read
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * NI) : "memory");

    // block 2: P.V(t-1) MFMAs interleaved with the row max and alpha of S(t)
    // and the units of its key tile 0
    {
      const uint16_t* sv16 = reinterpret_cast<const uint16_t*>((t - 1) & 1 ? sv[1] : sv[0]);
      int trr = tr_row, trc = tr_col;
      asm volatile("" : "+v"(trr), "+v"(trc));
      auto read_v = [&](int u, int dt) -> uint4 {
        const int r1 = 16 * u + trr, xx = 32 * dt + trc;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, xx)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, xx)));
        const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
        return make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      };
      // V^T operands: rolling, the read of k-step u+1 replaces that of u
      uint4 va[DT];
      if (HP) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) va[dt] = read_v(0, dt);
      }
      f32x16 s0[QT];  // key tile 0 of S(t), in VGPRs
      float mx[QT];
      // VALU work of S(t), one piece after each pair of P.V MFMAs: k-step 0 of
      // the P.V loop reads and maxes key tile 0, k-step 1 key tile 1 (then
      // m(t), alpha(t)), k-steps 2 and 3 run the units of key tile 0
      auto task = [&](int u, int j) {
        if (u < 2) {
          const int qt = j >> 1, hv = j & 1;  // query tile, half of the 16 values
          float m;
          if (u == 0) {
            if (hv == 0) {
              s0[qt] = sacc[0][qt];
              if (CD) mask(s0[qt], t & 1, 0, qt);
            }
            m = hv == 0 ? -INFINITY : mx[qt];
#pragma unroll
            for (int v = 0; v < 8; ++v) m = fmaxf(m, s0[qt][8 * hv + v]);
            mx[qt] = m;
          } else {
            f32x16 x = sacc[1][qt];
            if (CD) mask(x, t & 1, 1, qt);
            m = mx[qt];
#pragma unroll
            for (int v = 0; v < 8; ++v) m = fmaxf(m, x[8 * hv + v]);
            mx[qt] = m;
            if (hv == 1) {
              // the reference max moves only when the tile's max exceeds it
              // by more than kRescaleSlack (log2 units)
              const float m_tile = pair32_max(m) * c;
              const float m_new = m_tile > m_cur[qt] + kRescaleSlack ? m_tile : m_cur[qt];
              const float al = __builtin_amdgcn_exp2f(m_cur[qt] - m_new);
              alpha_cur[qt] = al != al ? 1.0f : al;
              m_cur[qt] = m_new;
            }
          }
        } else {
          unit(0, j >> 2, 4 * (u - 2) + (j & 3), s0[j >> 2]);
        }
      };
      constexpr int TPD = (4 * QT + DT - 1) / DT;  // most tasks after one dt
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int nt = u < 2 ? 2 * QT : 4 * QT;  // tasks of this k-step
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          if (HP) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
              const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pk[qt][u]);
              o[dt][qt] = T::mfma32(as_vec8<T>(va[dt]), pb, o[dt][qt]);
            }
            if (u + 1 < 4) va[dt] = read_v(u + 1, dt);
          }
          if (u == 0 && dt == 0 && HS) load_k(t + 2, t + 2 < nsteps ? jk : -1);
          __builtin_amdgcn_sched_barrier(0);
          if (HS) {
            // tasks nt * dt / DT .. nt * (dt + 1) / DT - 1, as a loop of
            // constant trip count so that it unrolls completely
#pragma unroll
            for (int k = 0; k < TPD; ++k) {
              const int j = (nt * dt) / DT + k;
              if (j < (nt * (dt + 1)) / DT) task(u, j);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };

  using T1 = std::true_type;
  using F0 = std::false_type;
  // the first diagonal step (nsteps when the diagonal block is not selected)
  const int d0 = diag_last ? nsteps - 2 : nsteps;
  step(T1{}, F0{}, d0 == 0, false, 0);
  int t = 1;
  for (; t < d0; ++t) step(T1{}, T1{}, F0{}, F0{}, t);  // main loop: unmasked steps
  for (; t < nsteps; ++t) step(T1{}, T1{}, T1{}, t - 1 >= d0, t);  // the diagonal block
  step(F0{}, T1{}, F0{}, diag_last, nsteps);
  // no tile load may still write this workgroup's LDS when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  int ln = lane;
  asm volatile("" : "+v"(ln));  // output addresses formed here, not held across the row
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qg = i * kBlock + 32 * (QT * w + qt) + (ln & 31);
    const float rcp = 1.0f / pair32_sum(l_part[qt]);
    if (qg < L) {
      uint16_t* op = a.o + (rec.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int dd = 32 * dt + 8 * g4 + 4 * half;
          uint2 w2;
          w2.x = pack2<T>(o[dt][qt][4 * g4 + 0] * rcp, o[dt][qt][4 * g4 + 1] * rcp);
          w2.y = pack2<T>(o[dt][qt][4 * g4 + 2] * rcp, o[dt][qt][4 * g4 + 3] * rcp);
          *reinterpret_cast<uint2*>(op + dd) = w2;
        }
    }
  }
}

template <int QT>
hipError_t launch_qt(const AttnArgs& a, int dtype, int head_dim, int64_t grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  const dim3 g(static_cast<unsigned>(grid)), blk(256 / QT);
  if (dtype == FP_DTYPE_BF16) {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_wide<BF16, 128, QT>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_wide<BF16, 64, QT>), g, blk, 0, s, a);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_wide<F16, 128, QT>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_wide<F16, 64, QT>), g, blk, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_attn_wide(const AttnArgs& a, int dtype, int head_dim, int64_t grid,
                            hipStream_t s) {
  return launch_qt<2>(a, dtype, head_dim, grid, s);
}

hipError_t launch_attn_pipe(const AttnArgs& a, int dtype, int head_dim, int64_t grid,
                            hipStream_t s) {
  return launch_qt<1>(a, dtype, head_dim, grid, s);
}

}  // namespace fp
