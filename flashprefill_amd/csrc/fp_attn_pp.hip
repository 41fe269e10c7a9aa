// Persistent ping-pong block-sparse attention for gfx950 (reference:
// ops/flashprefill_native_forward.py:227-344, ops/flashprefill_varlen_func.py:
// 449-575; same operand layouts as k_attn in fp_attn.hip).
//
// One workgroup per CU, 8 waves = two groups of 4; waves w and w+4 share a
// SIMD. Each group walks a stream of (query head, sequence, q-block) rows
// popped from a per-XCD work queue (heaviest rows first); each wave of the
// group owns 32 query rows of the current row. The selected key blocks of a
// row are consumed as 64-key half tiles (the reference's K_TILE_SIZE = 64
// configuration), and every half tile t goes through two phases:
//
//   M phase  O += V(t-1)^T . P(t-1)^T  and  S(t) = K(t) . Q^T    (32 MFMAs)
//   V phase  online softmax of S(t) -> P(t); direct-to-LDS loads of K(t+2),
//            V(t+1) (double-buffered, two phases of lead); Q of the next row
//
// The two groups run the phases offset by one workgroup barrier, so on every
// SIMD one wave issues MFMAs while its partner runs the softmax. The pipeline continues across row boundaries (a row's Q load,
// first tiles and output store overlap its neighbours' work); row descriptors
// live in a small LDS ring so that the stream state fits in scalar registers.
//
// Numerics: the reference loop with a 64-key tile — m = -inf and l = 1.0 at
// row start, alpha = exp2(m_old - m_new) with NaN -> 1, l accumulates the fp32
// p, P is rounded to the input dtype before P.V, key > query masked on the
// diagonal block, O = acc * (1/l); the accumulator is rescaled only when some
// row's max moved.
#include <type_traits>

#include "fp_attn_common.h"

namespace fp {

struct RowDesc {  // one (head, sequence, q-block) row, 32 bytes in LDS
  int i, L, h, ncnt;
  int64_t t0, row_tri;
};

struct Pos {  // one half tile of a group's stream
  int slot;   // ring slot of the row, -1 once the stream is exhausted
  int n;      // index in the row's list
  int hf;     // which 64-key half of block j
  int j;      // key block, -1 for an empty row (one null position)
  int ncnt;   // list length of the row
  int i;      // q-block of the row
};

template <int P>
using Parity = std::integral_constant<int, P>;

template <typename T, int D>
__global__ __launch_bounds__(512, 1) void k_attn_pp(AttnArgs a) {
  constexpr int CH = D / 8;    // 16-byte chunks per key row
  constexpr int KS = D / 16;   // MFMA k-steps over the head dim
  constexpr int DT = D / 32;   // 32-row tiles of O^T
  constexpr int HT = 64 * CH;  // uint4 per half tile
  constexpr int NDMA = 2 * HalfLanes<D>::NI;  // tile loads per wave per V phase (fixed)
  // Half-tile buffers of even / odd stream positions, [group]. One array per
  // parity, selected at compile time: the compiler then knows that the tile
  // loads of a V phase never write the buffers the next M phase reads, and
  // only waits for the loads of the phase before.
  __shared__ uint4 sk0[2][HT], sk1[2][HT];
  __shared__ uint4 sv0[2][HT], sv1[2][HT];
  __shared__ RowDesc ring[2][4];  // [group][slot]
  __shared__ int s_next[2][2];    // [group][parity]: next row id of the group
  __shared__ int s_done[2][2];    // [iteration parity][group]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave >> 2, wq = wave & 3;
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * wq + l32;
  const float c = a.sm_scale_log2;
  const bool leader = wq == 0 && lane == 0;
  const int G = a.Hq / a.Hkv;

  // queue domain: XCD x (= workgroup id % 8) serves heads x*Hq/8 .. when Hq % 8 == 0
  const int nitems = static_cast<int>(sld(a.tab.seq_tile + a.B));
  int qid = 0, hpx = a.Hq, head0 = 0;
  if ((a.Hq & 7) == 0) {
    qid = blockIdx.x & 7;
    hpx = a.Hq >> 3;
    head0 = qid * hpx;
  }
  const int total = nitems * hpx;
  int32_t* queue = a.sched + qid;

  if (leader) {
    const int v = atomicAdd(queue, 1);
    s_next[g][0] = v < total ? v : -1;
    s_done[0][g] = 0;
    s_done[1][g] = 0;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  auto uni64 = [](int64_t x) -> int64_t {
    const uint64_t u = static_cast<uint64_t>(x);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  };
  // Rows are started in order k = 0, 1, ...: start k reads the id published
  // in s_next[g][k & 1] and the leader publishes the id it popped for start
  // k + 1 in s_next[g][(k + 1) & 1] (a barrier separates consecutive starts).
  int rows_loaded = 0;
  auto next_row_id = [&]() -> int {
    return __builtin_amdgcn_readfirstlane(s_next[g][rows_loaded & 1]);
  };
  auto publish = [&](int v) { s_next[g][rows_loaded & 1] = v < total ? v : -1; };  // after a start
  // start row s (>= 0) at position p: descriptor from the item record
  auto fetch_row = [&](Pos& p, int s) {
    const int slot = rows_loaded & 3;
    ++rows_loaded;
    const int k = s / hpx;
    const int h = head0 + (s - k * hpx);
    const ItemRec r = sld(a.tab.items + k);
    RowDesc d;
    d.i = r.i;
    d.L = r.L;
    d.h = h;
    d.t0 = r.t0;
    d.row_tri = static_cast<int64_t>(h) * a.tri_cap + r.tri;
    d.ncnt = min(max(sld(a.cnt + static_cast<int64_t>(h) * a.nb_sum_cap + r.tile), 0), r.i + 1);
    const int j0 = sld(a.idx + d.row_tri);  // in bounds: the row's list has i + 1 slots
    if (lane == 0) ring[g][slot] = d;      // every wave of the group writes the same values
    p.slot = slot;
    p.n = 0;
    p.hf = 0;
    p.ncnt = d.ncnt;
    p.i = d.i;
    p.j = d.ncnt > 0 ? min(max(j0, 0), d.i) : -1;
  };
  // does the position after p start a new row?
  auto needs_row = [](const Pos& p) {
    return p.slot >= 0 && !(p.j >= 0 && p.hf == 0) && p.n + 1 >= p.ncnt;
  };
  // next position inside p's row (p.slot >= 0 and !needs_row(p))
  auto step_in_row = [&](Pos& p) {
    if (p.j >= 0 && p.hf == 0) {
      p.hf = 1;
    } else {
      ++p.n;
      p.hf = 0;
      const int64_t row_tri = uni64(ring[g][p.slot].row_tri);
      p.j = min(max(sld(a.idx + row_tri + p.n), 0), p.i);
    }
  };
  // the descriptor of position p's row, as wave-uniform (scalar) values
  auto row_of = [&](const Pos& p) -> RowDesc {
    const RowDesc r = ring[g][p.slot];
    RowDesc d;
    d.i = __builtin_amdgcn_readfirstlane(r.i);
    d.L = __builtin_amdgcn_readfirstlane(r.L);
    d.h = __builtin_amdgcn_readfirstlane(r.h);
    d.ncnt = __builtin_amdgcn_readfirstlane(r.ncnt);
    d.t0 = uni64(r.t0);
    d.row_tri = uni64(r.row_tri);
    return d;
  };
  // position after p, synchronously (prologue only)
  auto advance_now = [&](Pos& p) {
    if (needs_row(p)) {
      const int s = next_row_id();
      int v = 0;
      if (s >= 0 && leader) v = atomicAdd(queue, 1);
      if (s >= 0) {
        fetch_row(p, s);
        if (leader) publish(v);
      } else {
        p.slot = -1;
      }
    } else if (p.slot >= 0) {
      step_in_row(p);
    }
  };

  // stream positions t-1 (P.V), t (S, softmax), t+1 (V load, Q), t+2 (K load)
  Pos pm1, p0, p1, p2;
  pm1.slot = p0.slot = p1.slot = -1;
  pm1.j = p0.j = p1.j = -1;
  pm1.n = p0.n = p1.n = pm1.hf = p0.hf = p1.hf = 0;
  pm1.ncnt = p0.ncnt = p1.ncnt = pm1.i = p0.i = p1.i = 0;
  {
    const int s = next_row_id();
    int v = 0;
    if (s >= 0 && leader) v = atomicAdd(queue, 1);
    if (s >= 0) {
      fetch_row(p1, s);
      if (leader) publish(v);
    }
  }
  // the next row id is published by the leader: make it visible before p2
  // may need it (a null first row moves p2 to the next row)
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  p2 = p1;
  advance_now(p2);

  HalfLanes<D> tk, tv;
  tk.init(a.kst, wq, lane);
  tv.init(a.vst, wq, lane);
  if (p1.slot >= 0 && p1.j >= 0) {  // K of the first position -> odd buffer (t + 1 = 1)
    const RowDesc d = row_of(p1);
    issue_half<D>(sk1[g], a.k + d.t0 * a.kst + static_cast<int64_t>(d.h / G) * a.khs, a.kst,
                  tk, p1.j, p1.hf, d.L, wq, lane);
  }

  typename T::vec8 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = as_vec8<T>(zero4());
  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
  f32x16 sc[2];
  uint32_t pk[4][4];  // P of position t-1, packed as P.V B operands
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[u][e] = 0u;
  float m_run = -INFINITY, l_part = 0.0f;

  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

  // M phase of position t (parity P): reads K(t) from sk<P>, V(t-1) from sv<P^1>
  auto m_phase = [&](auto par) {
    constexpr int P = decltype(par)::value;
    const uint4* skb = P == 0 ? sk0[g] : sk1[g];
    const uint16_t* sv16 = reinterpret_cast<const uint16_t*>(P == 0 ? sv1[g] : sv0[g]);
    // per-lane LDS coordinates, re-derived in every phase: keeping the
    // addresses they produce live across the loop costs registers
    int trr = tr_row, trc = tr_col, lr = l32, hl = half;
    asm volatile("" : "+v"(trr), "+v"(trc), "+v"(lr), "+v"(hl));
    if (pm1.slot >= 0 && pm1.j >= 0) {  // O += V(t-1)^T . P(t-1)^T, 16 keys per step
      auto read_v = [&](int u, int dt) -> uint4 {
        const int r1 = 16 * u + trr, xx = 32 * dt + trc;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, xx)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, xx)));
        const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
        return make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      };
      uint4 va[DT];  // rolling: the operand of step u+1 replaces that of step u
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) va[dt] = read_v(0, dt);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pk[u]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          o[dt] = T::mfma32(as_vec8<T>(va[dt]), pb, o[dt]);
          if (u + 1 < 4) va[dt] = read_v(u + 1, dt);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    sc[0] = f32x16{};
    sc[1] = f32x16{};
    if (p0.slot >= 0 && p0.j >= 0) {  // S(t) = K(t) . Q^T, 32 keys per accumulator
      auto read_k = [&](int ks, int t2) -> uint4 {
        const int r = 32 * t2 + lr;
        return skb[r * CH + ((2 * ks + hl) ^ swz<D>(r))];
      };
      uint4 ka[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) ka[t2] = read_k(0, t2);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          sc[t2] = T::mfma32(as_vec8<T>(ka[t2]), qb[ks], sc[t2]);
          if (ks + 1 < KS) ka[t2] = read_k(ks + 1, t2);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // position t-1 closed its row: O = acc * (1/l) -> global
    if (pm1.slot >= 0 && (pm1.j < 0 || (pm1.hf == 1 && pm1.n + 1 >= pm1.ncnt))) {
      const RowDesc d = row_of(pm1);
      const int qg = d.i * kBlock + qrow;
      const float l = l_part + xor32_f(l_part);
      const float rcp = 1.0f / l;
      if (qg < d.L) {
        uint16_t* op = a.o + (d.t0 + qg) * a.ost + static_cast<int64_t>(d.h) * a.ohs;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int dd = 32 * dt + 8 * g4 + 4 * half;
            uint2 w2;
            w2.x = pack2<T>(o[dt][4 * g4 + 0] * rcp, o[dt][4 * g4 + 1] * rcp);
            w2.y = pack2<T>(o[dt][4 * g4 + 2] * rcp, o[dt][4 * g4 + 3] * rcp);
            *reinterpret_cast<uint2*>(op + dd) = w2;
          }
      }
    }
  };

  // V phase of position t (parity P)
  auto v_phase = [&](auto par, int it) {
    constexpr int P = decltype(par)::value;
    uint4* kdst = P == 0 ? sk0[g] : sk1[g];  // K(t+2) has the parity of t
    uint4* vdst = P == 0 ? sv1[g] : sv0[g];  // V(t+1) the other one
    // Loads into registers happen here, before this phase's tile loads, and
    // are waited for at once (the compiler cannot count the direct-to-LDS
    // loads against them, so any later wait would drain every tile load in
    // flight); they happen once per row.
    // a row change after p2: read the row id, pop and publish the one after
    const bool nr = needs_row(p2);
    int s_new = -1;
    if (nr) {
      s_new = next_row_id();
      if (s_new >= 0 && leader) {
        const int v = atomicAdd(queue, 1);
        s_next[g][(rows_loaded + 1) & 1] = v < total ? v : -1;
      }
    }
    // Q of a row that starts at t+1 (S(t) has been computed)
    if (p1.slot >= 0 && p1.n == 0 && p1.hf == 0) {
      const RowDesc d = row_of(p1);
      const int qg = d.i * kBlock + qrow;
      const bool qvalid = qg < d.L;
      const uint16_t* qp =
          a.q + (d.t0 + qg) * a.qst + static_cast<int64_t>(d.h) * a.qhs + 8 * half;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4 u = __builtin_bit_cast(u32x4, qvalid ? ld16(qp + 16 * s) : zero4());
        asm volatile("" : "+v"(u));  // the wait for the load happens here
        qb[s] = as_vec8<T>(__builtin_bit_cast(uint4, u));
      }
    }
    // tile loads two phases ahead, always NDMA per wave (a position with no
    // tile loads row 0 of head 0, which is never read)
    {
      const uint16_t* kbase = a.k;
      int kj = 0, khf = 0, kL = 1;
      if (p2.slot >= 0 && p2.j >= 0) {
        const RowDesc d = row_of(p2);
        kbase = a.k + d.t0 * a.kst + static_cast<int64_t>(d.h / G) * a.khs;
        kj = p2.j;
        khf = p2.hf;
        kL = d.L;
      }
      issue_half<D>(kdst, kbase, a.kst, tk, kj, khf, kL, wq, lane);
      const uint16_t* vbase = a.v;
      int vj = 0, vhf = 0, vL = 1;
      if (p1.slot >= 0 && p1.j >= 0) {
        const RowDesc d = row_of(p1);
        vbase = a.v + d.t0 * a.vst + static_cast<int64_t>(d.h / G) * a.vhs;
        vj = p1.j;
        vhf = p1.hf;
        vL = d.L;
      }
      issue_half<D>(vdst, vbase, a.vst, tv, vj, vhf, vL, wq, lane);
    }
    // successor of p2 (its scalar loads overlap the softmax)
    Pos nx = p2;
    if (nr) {
      if (s_new >= 0) fetch_row(nx, s_new);
      else nx.slot = -1;
    } else if (p2.slot >= 0) {
      step_in_row(nx);
    }
    // online softmax of S(t)
    if (p0.slot >= 0) {
      if (p0.n == 0 && p0.hf == 0) {  // row start: m = -inf, l = 1.0, acc = 0
        m_run = -INFINITY;
        l_part = half == 0 ? 1.0f : 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
      }
      if (p0.j >= 0) {
        if (p0.j == p0.i) {  // diagonal block: key > query is masked
          // (qlim == qrow - 64 hf; deriving it from the row keeps the compares
          // inside the loop instead of hoisted into scalar masks)
          const int qlim = qrow - 64 * p0.hf + (p0.j - p0.i);
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int key = 32 * t2 + 8 * (v >> 2) + 4 * half + (v & 3);
              if (key > qlim) sc[t2][v] = -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[t2][v]);
        mx = fmaxf(mx, xor32_f(mx));
        const float m_new = fmaxf(m_run, mx * c);
        float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        if (alpha != alpha) alpha = 1.0f;
        float psum = 0.0f;
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[t2][v], c, -m_new));
            sc[t2][v] = p;
            psum += p;
          }
        // B-operand key order of step u = 2 t2 + v / 8, element v % 8
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int v = 0; v < 16; v += 2)
            pk[2 * t2 + (v >> 3)][(v & 7) >> 1] = pack2<T>(sc[t2][v], sc[t2][v + 1]);
        l_part = l_part * alpha + psum;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[dt][v] *= alpha;
        }
      }
    }
    pm1 = p0;
    p0 = p1;
    p1 = p2;
    p2 = nx;
    if (leader) s_done[it & 1][g] = (pm1.slot < 0 && p0.slot < 0 && p1.slot < 0) ? 1 : 0;
  };

  // After an M phase nothing but this wave's LDS reads must be complete;
  // after a V phase the tile loads of the V phase before it (read by the
  // next M phase) must have landed: the NDMA loads just issued may still fly.
  auto m_end = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  auto v_end = []() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NDMA) : "memory");
  };

  // Both groups run the same straight-line M -> V loop; group 1 starts one
  // barrier late, so each of its phases runs against the other kind of phase
  // of group 0. Barrier #(2 it + 2) is where both groups look at the done
  // flags (group 0 after its V(it), group 1 after its M(it)) and leave
  // together, having executed the same number of barriers.
  auto done_at = [&](int it) {
    return s_done[it & 1][0] != 0 && s_done[(it + 1) & 1][1] != 0;
  };
  if (g == 1) asm volatile("s_barrier" ::: "memory");
  for (int it = 0;; it += 2) {
    m_phase(Parity<0>{});
    m_end();
    if (g == 1 && done_at(it)) break;
    v_phase(Parity<0>{}, it);
    v_end();
    if (g == 0 && done_at(it)) break;
    m_phase(Parity<1>{});
    m_end();
    if (g == 1 && done_at(it + 1)) break;
    v_phase(Parity<1>{}, it + 1);
    v_end();
    if (g == 0 && done_at(it + 1)) break;
  }

  // the last workgroup to finish re-arms the queues for the next launch
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  if (threadIdx.x == 0) {
    __threadfence();
    const int fin = atomicAdd(a.sched + 8, 1);
    if (fin == static_cast<int>(gridDim.x) - 1) {
      for (int q = 0; q < 9; ++q) atomicExch(a.sched + q, 0);
    }
  }
}

hipError_t launch_attn_pp(const AttnArgs& a, int dtype, int head_dim, int num_wg, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(num_wg)), blk(512);
  if (dtype == FP_DTYPE_BF16) {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_pp<BF16, 128>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_pp<BF16, 64>), g, blk, 0, s, a);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn_pp<F16, 128>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn_pp<F16, 64>), g, blk, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace fp
