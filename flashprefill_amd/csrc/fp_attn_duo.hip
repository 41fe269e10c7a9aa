// Two-group ping-pong block-sparse attention for gfx950 (reference:
// ops/flashprefill_native_forward.py:227-344, ops/flashprefill_varlen_func.py:
// 449-575; operand layouts as k_attn in fp_attn.hip).
//
// One workgroup of 8 waves owns one (query head, sequence, q-block) row; one
// workgroup per CU (128 KB LDS). The waves form two groups of four; wave wq of
// group g owns query rows 32 wq .. 32 wq + 31 of the block, so waves w and
// w + 4 (one per group, same queries) share a SIMD. Group g takes key half g
// (keys 64 g .. 64 g + 63) of every selected block: both groups walk the same
// list, take the same number of steps, and at the end their partial softmax
// states (m, l, O) are merged through LDS (split-K over the two key halves).
//
// Every step t of a group is two phases:
//
//   M phase  O += V(t-1)^T . P(t-1)^T and S(t) = K(t) . Q^T: 32 MFMAs, LDS
//            operand reads, nothing else
//   V phase  the K(t+2) and V(t+1) tile loads, then the online softmax of S(t)
//            into P(t): masking on the diagonal block, the row max, the
//            conditional rescale of O and l, exp2, rounding, row sums
//
// and the groups run one phase apart, separated by workgroup barriers: while
// group 0 issues the MFMAs of a step, group 1 runs the softmax of its
// previous step on the same SIMDs, and the other way round in the next phase,
// so one wave's VALU work overlaps its partner's MFMAs. K and V half tiles
// (16 KB each at d = 128) are double-buffered per group and loaded two phases
// before use; every V phase issues the same number of loads (positions past
// the end load the first block into a buffer that is not read again), so the
// waits are constant counts.
//
// Numerics: the reference loop (m = -inf and l = 1.0 at the start, alpha =
// exp2(m_old - m_new) with NaN -> 1, P rounded to the input dtype before P.V,
// key > query masked on the diagonal block, O = acc * (1/l)), per key half,
// with the default kernel's conditional rescaling (kRescaleSlack) and row sums
// of the rounded P; the two halves are then combined exactly as the online
// softmax combines consecutive tiles: m = max(m0, m1), O = O0 f0 + O1 f1,
// l = l0 f0 + l1 f1 with f = exp2(m_g - m).
#include "fp_attn_common.h"

namespace fp {

template <typename T, int D>
__global__ __launch_bounds__(512, 1) void k_attn_duo(AttnArgs a) {
  constexpr int CH = D / 8;    // 16-byte chunks per key row
  constexpr int KS = D / 16;   // MFMA k-steps over the head dim
  constexpr int DT = D / 32;   // 32-row tiles of O^T
  constexpr int HT = 64 * CH;  // uint4 per half tile
  constexpr int NI = HalfLanes<D>::NI;  // tile loads per wave per half tile
  constexpr int RPW = HalfLanes<D>::RPW;
  constexpr uint32_t TB = HT * 16;      // bytes per half tile
  // [group][K, V][parity] half tiles
  __shared__ uint4 smem[2][2][2][HT];

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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave >> 2, wq = wave & 3;
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * wq + l32;
  const int qg = i * kBlock + qrow;
  const float c = a.sm_scale_log2;
  const int rem = L - i * kBlock;  // rows of this q-block inside the sequence

  if (ncnt == 0) {  // no block selected: m = -inf, l = 1, O = 0
    if (g == 0 && qg < L) {
      uint16_t* op = a.o + (rec.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs;
#pragma unroll
      for (int dd = 0; dd < D; dd += 8) *reinterpret_cast<uint4*>(op + dd) = zero4();
    }
    return;
  }

  // list entry n, clamped to the row (n < ncnt); -1 past the end
  auto entry = [&](int n) -> int { return n < ncnt ? min(max(sld(list + n), 0), i) : -1; };

  const uint32_t lds0 = lds_addr(&smem[0][0][0][0]);
  auto buf = [&](int kind, int par) -> uint32_t {  // LDS byte address of a half tile
    return lds0 + ((g * 2 + kind) * 2 + par) * TB;
  };
  // this wave's loads of key half g of block jb (jb < 0: the first rows of the
  // sequence, into a buffer that is not read again)
  auto load_half = [&](int kind, int par, int jb) {
    const uint16_t* basep = kind == 0 ? kbase : vbase;
    const int stride = kind == 0 ? kst : vst;
    int ln = lane;
    asm volatile("" : "+v"(ln));  // lane terms formed here, not held across the loop
    int row0 = 0, rows = min(L, 64);
    if (jb >= 0) {
      row0 = jb * kBlock + 64 * g;
      rows = jb == i ? rem - 64 * g : 64;
      if (rows <= 0) {  // second half past the sequence end: its last row
        row0 = L - 1;
        rows = 1;
      }
    }
    const uint16_t* src = basep + static_cast<int64_t>(row0) * stride;
    const uint32_t lds = buf(kind, par);
    if (rows >= 64) {
      uint64_t sb = scalar_addr(src);
      // the base was written by VALU (readfirstlane): five wait states before
      // a VMEM instruction reads it; every later use goes through this asm
      asm volatile("s_nop 4" : "+s"(sb));
#pragma unroll
      for (int q = 0; q < NI; ++q) {
        // lane ln writes physical chunk ln % CH of row slot * RPW + ln / CH, so
        // it fetches logical chunk (ln % CH) ^ swz(row) of that row
        const int r = (wq * NI + q) * RPW + ln / CH;
        const uint32_t off = static_cast<uint32_t>((r * stride + 8 * ((ln % CH) ^ swz<D>(r))) * 2);
        dma16_sbase_m0(lds + (wq * NI + q) * 1024, sb, off);
      }
    } else {
#pragma unroll
      for (int q = 0; q < NI; ++q) {
        const int slot = wq * NI + q;
        const int r = slot * RPW + ln / CH;
        const int cc = (ln % CH) ^ swz<D>(r);
        const int gk = min(r, rows - 1);
        dma16_vaddr_at(lds + slot * 1024, src + static_cast<int64_t>(gk) * stride + 8 * cc);
      }
    }
  };

  // blocks of steps t, t+1, t+2 of the V phase about to run (scalar), and the
  // raw list entry of step t+3 (read one phase ahead)
  int j0 = entry(0), j1 = entry(1), j2 = entry(2);
  int j3raw = sld(list + min(3, ncnt - 1));
  load_half(0, 0, j0);  // K(0)
  load_half(1, 0, j0);  // V(0)
  load_half(0, 1, j1);  // K(1)

  // Q^T as MFMA B operands (lane: query l32, dims 16 s + 8 half .. +7), loaded
  // after the first tile loads; the wait for it also covers them
  typename T::vec8 qb[KS];
  {
    const bool qvalid = qg < L;
    const uint16_t* qp = a.q + (rec.t0 + qg) * a.qst + static_cast<int64_t>(h) * a.qhs + 8 * half;
    u32x4 u[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) u[s] = __builtin_bit_cast(u32x4, qvalid ? ld16(qp + 16 * s) : zero4());
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      asm volatile("" : "+v"(u[s]));
      qb[s] = as_vec8<T>(__builtin_bit_cast(uint4, u[s]));
    }
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // K(0), V(0), K(1) landed


  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_part = half == 0 ? 1.0f : 0.0f;  // the two halves' partial sums add up to l
  f32x16 s[2];                             // S(t), key tiles 0 / 1 of the half
  uint32_t pk[4][4];                       // P(t-1) as the B operands of 4 P.V k-steps
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[u][e] = 0u;

  // M phase of step t: P.V of step t-1 (t >= 1), S of step t (t < ncnt).
  // Operands are read one k-step ahead of the MFMAs that use them (the fences
  // keep the compiler from hoisting every read of the phase, which would not
  // fit the register budget).
  auto m_phase = [&](int t) {
    if (t >= 1) {
      const uint16_t* vb = reinterpret_cast<const uint16_t*>(&smem[g][1][(t - 1) & 1][0]);
      int ln = lane;
      asm volatile("" : "+v"(ln));  // addresses formed here, not held across the loop
      const int g16 = ln >> 4, i16 = ln & 15;
      const int trr = 4 * (g16 >> 1) + (i16 >> 2), trc = 16 * (g16 & 1) + 4 * (i16 & 3);
      auto read_vt = [&](int u, int dt) -> uint4 {
        const int r1 = 16 * u + trr, x = 32 * dt + trc;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vb + tile_elem<D>(r1, x)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vb + tile_elem<D>(r1 + 8, x)));
        const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
        return make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      };
      uint4 va[2][DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) va[0][dt] = read_vt(0, dt);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u + 1 < 4) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) va[(u + 1) & 1][dt] = read_vt(u + 1, dt);
        }
        const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pk[u]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = T::mfma32(as_vec8<T>(va[u & 1][dt]), pb, o[dt]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (t < ncnt) {
      const uint4* kb = &smem[g][0][t & 1][0];
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int lr = ln & 31, hl = ln >> 5;
      auto read_k = [&](int ks, int kt) -> uint4 {
        const int r = 32 * kt + lr;
        return kb[r * CH + ((2 * ks + hl) ^ swz<D>(r))];
      };
      uint4 ka[2][2];
      ka[0][0] = read_k(0, 0);
      ka[0][1] = read_k(0, 1);
      s[0] = s[1] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
          ka[(ks + 1) & 1][0] = read_k(ks + 1, 0);
          ka[(ks + 1) & 1][1] = read_k(ks + 1, 1);
        }
        s[0] = T::mfma32(as_vec8<T>(ka[ks & 1][0]), qb[ks], s[0]);
        s[1] = T::mfma32(as_vec8<T>(ka[ks & 1][1]), qb[ks], s[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS reads are done
  };

  // V phase of step t (t < ncnt)
  auto v_phase = [&](int t) {
    // refills: K(t+2) into the buffer K(t) used, V(t+1) into the one V(t-1) used
    load_half(0, t & 1, j2);
    load_half(1, (t + 1) & 1, j1);
    const int jd = j0;
    // next step's blocks; the list entry of step t+4 is read one phase ahead
    j0 = j1;
    j1 = j2;
    j2 = t + 3 < ncnt ? min(max(j3raw, 0), i) : -1;
    j3raw = sld(list + min(t + 4, ncnt - 1));

    if (jd == i) {  // diagonal block: key > query is masked
      // key 64 g + 32 kt + 8 (v / 4) + 4 half + v % 4 > query 32 wq + l32,
      // with the lane part moved to the right so the key constants stay
      // immediates (lane terms recomputed, not held across the row)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int lim = 32 * wq + (ln & 31) - 64 * g - 4 * (ln >> 5);
      // a select per element (a divergent branch per element would hold 32
      // lane masks in scalar registers)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          s[kt][v] = 32 * kt + 8 * (v >> 2) + (v & 3) > lim ? -INFINITY : s[kt][v];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt][v]);
    const float m_tile = pair32_max(mx) * c;
    // the running max moves (and O, l are rescaled) only when some row of the
    // wave exceeds it by more than kRescaleSlack
    if (__ballot(m_tile > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, m_tile);
      float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      if (alpha != alpha) alpha = 1.0f;
      l_part *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[dt][v] *= alpha;
    }
    // a row whose keys so far were all masked keeps m = -inf: its p are 0
    const float msub = m_run == -INFINITY ? 0.0f : m_run;
    float psum[2] = {0.0f, 0.0f};
    // B operand of P.V k-step u = 2 kt + v / 8, element pair (v % 8) / 2
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kt][v], c, -msub));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kt][v + 1], c, -msub));
        uint32_t& dst = pk[2 * kt + (v >> 3)][(v & 7) >> 1];
        dst = pack2<T>(p0, p1);
        psum[(v >> 1) & 1] = add_pair<T>(dst, psum[(v >> 1) & 1]);
      }
    l_part += psum[0] + psum[1];
    // K(t+1) and V(t), read by the next M phase, have landed; the 2 NI loads
    // just issued may still be in flight
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * NI) : "memory");
  };

  // ncnt + 1 steps of two barrier slots each, executed by every wave; group 1
  // runs one slot behind group 0, so in every slot one group runs an M phase
  // and the other a V phase (group 1 is idle in the first slot, group 0 in
  // the last). One straight loop per group, so the conditional rescale of O
  // is the only branch O passes through inside a step.
  if (g == 0) {
    for (int t = 0; t <= ncnt; ++t) {
      m_phase(t);
      asm volatile("s_barrier" ::: "memory");
      if (t < ncnt) v_phase(t);
      asm volatile("s_barrier" ::: "memory");
    }
  } else {
    for (int t = 0; t <= ncnt; ++t) {
      if (t >= 1) v_phase(t - 1);
      asm volatile("s_barrier" ::: "memory");
      m_phase(t);
      asm volatile("s_barrier" ::: "memory");
    }
  }
  // no tile load may still write the LDS that the merge below reuses
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

  // merge: group 1 hands its (O, m, l) to the wave of group 0 that owns the
  // same queries; [wq][value][lane] keeps every access a 64-lane row
  float* mb = reinterpret_cast<float*>(&smem[0][0][0][0]);
  constexpr int NV = DT * 16 + 2;
  float* mine = mb + wq * NV * 64 + lane;
  if (g == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mine[(dt * 16 + v) * 64] = o[dt][v];
    mine[(NV - 2) * 64] = m_run;
    mine[(NV - 1) * 64] = l_part;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (g == 1) return;
  const float m1 = mine[(NV - 2) * 64], l1 = mine[(NV - 1) * 64];
  const float m = fmaxf(m_run, m1);
  const float f0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
  const float f1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
  const float l = pair32_sum(l_part * f0 + l1 * f1);
  const float rcp = 1.0f / l;
  if (qg < L) {
    uint16_t* op = a.o + (rec.t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * g4 + e;
          x[e] = (o[dt][v] * f0 + mine[(dt * 16 + v) * 64] * f1) * rcp;
        }
        const int d = 32 * dt + 8 * g4 + 4 * half;
        uint2 pkd;
        pkd.x = pack2<T>(x[0], x[1]);
        pkd.y = pack2<T>(x[2], x[3]);
        *reinterpret_cast<uint2*>(op + d) = pkd;
      }
  }
}

hipError_t launch_attn_duo(const AttnArgs& a, int dtype, int head_dim, int64_t grid,
                           hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  const dim3 gr(static_cast<unsigned>(grid)), blk(512);
  if (dtype == FP_DTYPE_BF16) {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_duo<BF16, 128>), gr, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_duo<BF16, 64>), gr, blk, 0, s, a);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_duo<F16, 128>), gr, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_duo<F16, 64>), gr, blk, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace fp
