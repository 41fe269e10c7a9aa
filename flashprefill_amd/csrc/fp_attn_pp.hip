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
//   M phase  O += V(t-1)^T . P(t-1)^T and S(t) = K(t) . Q^T (32 MFMAs, LDS
//            operands read ahead), then in the MFMA shadow: output store of a finished row, the next stream
//            position (queue pop and row descriptor at row changes), its
//            tile-load addresses and the Q load of a row starting at t+1
//   V phase  online softmax of S(t) -> P(t), with the direct-to-LDS loads of
//            K(t+2), V(t+1) (double-buffered, two phases of lead) spread
//            through it: the CU's memory pipe issues them at its own pace
//            while the softmax runs
//
// The two groups run the phases offset by one workgroup barrier, so on every
// SIMD one wave issues MFMAs while its partner runs the softmax (measured on
// gfx950: an MFMA 32x32x16 takes 32 cycles, a wave64 VALU op about 6, and the
// two co-issue). The pipeline continues across row boundaries. The state of
// the newest position's row (K/V addresses, index list) is kept in scalar
// registers; older rows' descriptors live in a small LDS ring and are read
// only for a row's Q load and output store.
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

// One half tile of a group's stream, packed into two dwords (scalar registers
// are the scarce resource of the persistent kernel):
//   w0 = slot + 1 (bits 0-3; 0 once the stream is exhausted) | hf << 4 |
//        (j + 1) << 5 (14 bits; j = -1 for an empty row's one null position) |
//        i << 19 (q-block of the row, 13 bits)
//   w1 = n (index in the row's list) | ncnt << 16 (list length of the row)
struct Pos {
  uint32_t w0, w1;
  __device__ __forceinline__ int slot() const { return static_cast<int>(w0 & 15u) - 1; }
  __device__ __forceinline__ int hf() const { return (w0 >> 4) & 1; }
  __device__ __forceinline__ int j() const { return static_cast<int>((w0 >> 5) & 0x3fffu) - 1; }
  __device__ __forceinline__ int i() const { return static_cast<int>(w0 >> 19); }
  __device__ __forceinline__ int n() const { return static_cast<int>(w1 & 0xffffu); }
  __device__ __forceinline__ int ncnt() const { return static_cast<int>(w1 >> 16); }
  __device__ __forceinline__ bool live() const { return (w0 & 15u) != 0; }
  __device__ __forceinline__ bool has_tile() const { return live() && j() >= 0; }
  __device__ __forceinline__ bool row_start() const { return n() == 0 && hf() == 0; }
  __device__ __forceinline__ void set(int slot, int hf, int j, int i, int n, int ncnt) {
    w0 = static_cast<uint32_t>(slot + 1) | (static_cast<uint32_t>(hf) << 4) |
         (static_cast<uint32_t>(j + 1) << 5) | (static_cast<uint32_t>(i) << 19);
    w1 = static_cast<uint32_t>(n) | (static_cast<uint32_t>(ncnt) << 16);
  }
  __device__ __forceinline__ void kill() { w0 = 0u; w1 = 0u; }
};

// Where the tile loads of one position read: the first of its 64 key rows and
// how many of them lie inside the sequence (rows past it read the last one).
struct TileSrc {
  const uint16_t* k;
  const uint16_t* v;
  int rows;
};

template <int P>
using Parity = std::integral_constant<int, P>;

constexpr int kRing = 8;  // row descriptors per group: positions t-1 .. t+3 span at most 5 rows

// One direct-to-LDS load (1 KB slice w*NI + q) of a full 64-row half tile:
// 32-bit lane offset from a scalar base.
template <int D>
__device__ __forceinline__ void dma_slice(uint4* lds, const uint16_t* base,
                                          const HalfLanes<D>& tl, int q, int w) {
  dma16_saddr(lds + (w * HalfLanes<D>::NI + q) * 64, base, tl.off[q]);
}

// All loads of a half tile with fewer than 64 rows inside the sequence: rows
// at or past `nvalid` read row nvalid - 1 (masked keys, p = 0).
template <int D>
__device__ __forceinline__ void dma_partial(uint4* lds, const uint16_t* base, int stride,
                                            int nvalid, int w, int lane) {
  constexpr int CH = HalfLanes<D>::CH, RPW = HalfLanes<D>::RPW, NI = HalfLanes<D>::NI;
#pragma unroll
  for (int q = 0; q < NI; ++q) {
    const int slot = w * NI + q;
    const int r = slot * RPW + lane / CH;
    const int c = (lane % CH) ^ swz<D>(r);
    const int gk = min(r, nvalid - 1);
    dma16_vaddr(lds + slot * 64, base + static_cast<int64_t>(gk) * stride + 8 * c);
  }
}

template <typename T, int D>
__global__ __launch_bounds__(512, 1) void k_attn_pp(AttnArgs a) {
  constexpr int KS = D / 16;   // MFMA k-steps over the head dim
  constexpr int DT = D / 32;   // 32-row tiles of O^T
  constexpr int CH = D / 8;    // 16-byte chunks per key row
  constexpr int HT = 64 * CH;  // uint4 per half tile
  constexpr int NI = HalfLanes<D>::NI;
  constexpr int NDMA = 2 * NI;  // tile loads per wave per V phase (fixed)
  // Half-tile buffers of even / odd stream positions, [group]. One array per
  // parity, selected at compile time: the compiler then knows that the tile
  // loads of a V phase never write the buffers the next M phase reads.
  __shared__ uint4 sk0[2][HT], sk1[2][HT];
  __shared__ uint4 sv0[2][HT], sv1[2][HT];
  __shared__ RowDesc ring[2][kRing];  // [group][slot]
  __shared__ int s_next[2][2];        // [group][parity]: next row id of the group
  __shared__ int s_done[2][2];        // [iteration parity][group]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave >> 2, wq = wave & 3;
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * wq + l32;
  const float c = a.sm_scale_log2;
  const bool leader = wq == 0 && lane == 0;
  const int G = a.Hq / a.Hkv;
  // strides fit in 24 bits and index-list offsets in 31 (checked on the host)
  const int qst = static_cast<int>(a.qst), qhs = static_cast<int>(a.qhs);
  const int kst = static_cast<int>(a.kst), khs = static_cast<int>(a.khs);
  const int vst = static_cast<int>(a.vst), vhs = static_cast<int>(a.vhs);
  const int ost = static_cast<int>(a.ost), ohs = static_cast<int>(a.ohs);
  const int tri_cap = static_cast<int>(a.tri_cap);

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
  // the row of the newest stream position, in scalar registers
  const uint16_t* hk = a.k;  // its kv head's K at the sequence start
  const uint16_t* hv = a.v;
  int hrem = 1;              // rows of its q-block inside the sequence (1 .. 128)
  int hrt = 0;               // offset of its index list in idx
  int jpref = 0;             // idx[hrt + n + 1] of the newest position, loaded a phase ahead
  // start the next row at position p (or end the stream); pops and publishes
  // the id after it: the wait for the atomic happens here (the compiler
  // cannot count direct-to-LDS loads against it, so a later wait would drain
  // every tile load in flight); once per row
  auto start_row = [&](Pos& p) {
    const int s = __builtin_amdgcn_readfirstlane(s_next[g][rows_loaded & 1]);
    if (s < 0) {
      p.kill();
      return;
    }
    if (leader) {
      const int v = atomicAdd(queue, 1);
      s_next[g][(rows_loaded + 1) & 1] = v < total ? v : -1;
    }
    const int slot = rows_loaded & (kRing - 1);
    ++rows_loaded;
    const int k = s / hpx;
    const int h = head0 + (s - k * hpx);
    const ItemRec r = sld(a.tab.items + k);
    hrt = h * tri_cap + static_cast<int>(r.tri);
    const int ncnt = min(max(sld(a.cnt + h * static_cast<int>(a.nb_sum_cap) + r.tile), 0),
                         r.i + 1);
    const int j0 = sld(a.idx + hrt);  // in bounds: the row's list has i + 1 slots
    const int64_t kvh = h / G;
    hk = a.k + r.t0 * kst + kvh * khs;
    hv = a.v + r.t0 * vst + kvh * vhs;
    hrem = r.L - r.i * kBlock;
    if (lane == 0) {  // every wave of the group writes the same values
      RowDesc d;
      d.i = r.i;
      d.L = r.L;
      d.h = h;
      d.ncnt = ncnt;
      d.t0 = r.t0;
      d.row_tri = hrt;
      ring[g][slot] = d;
    }
    p.set(slot, 0, ncnt > 0 ? min(max(j0, 0), r.i) : -1, r.i, 0, ncnt);
  };
  // the position after p, p being the newest one (uses the prefetched index)
  auto advance = [&](Pos& p) {
    if (!p.live()) return;
    if (p.j() >= 0 && p.hf() == 0) {
      p.w0 |= 1u << 4;  // second half of block j
    } else if (p.n() + 1 < p.ncnt()) {
      p.set(p.slot(), 0, min(max(jpref, 0), p.i()), p.i(), p.n() + 1, p.ncnt());
    } else {
      start_row(p);
    }
  };
  // tile-load sources of p, p being the newest position
  auto plan = [&](const Pos& p) -> TileSrc {
    TileSrc t;
    t.k = a.k;  // no tile: row 0 of head 0, into a buffer that is never read
    t.v = a.v;
    t.rows = 1;
    if (p.has_tile()) {
      int row0 = p.j() * kBlock + 64 * p.hf();
      int rows = p.j() == p.i() ? hrem - 64 * p.hf() : 64;
      if (rows <= 0) {  // second half past the sequence end: read its last row
        row0 = p.i() * kBlock + hrem - 1;
        rows = 1;
      }
      t.k = hk + static_cast<int64_t>(row0) * kst;
      t.v = hv + static_cast<int64_t>(row0) * vst;
      t.rows = min(rows, 64);
    }
    return t;
  };
  // the descriptor of position p's row (LDS ring), as wave-uniform values
  auto row_of = [&](const Pos& p) -> RowDesc {
    const RowDesc r = ring[g][p.slot()];
    RowDesc d;
    d.i = __builtin_amdgcn_readfirstlane(r.i);
    d.L = __builtin_amdgcn_readfirstlane(r.L);
    d.h = __builtin_amdgcn_readfirstlane(r.h);
    d.ncnt = __builtin_amdgcn_readfirstlane(r.ncnt);
    d.t0 = uni64(r.t0);
    d.row_tri = uni64(r.row_tri);
    return d;
  };
  // load the index after the newest position's (used by the next advance)
  auto prefetch_index = [&](const Pos& p) {
    if (p.live() && p.n() + 1 < p.ncnt()) jpref = sld(a.idx + hrt + p.n() + 1);
  };

  // stream positions t-1 (P.V), t (S, softmax), t+1 (V load, Q), t+2 (K load)
  // and t+3 (looked up during M(t)); tile sources of t+1 (V) .. t+3
  Pos pm1, p0, p1, p2, p3;
  pm1.kill();
  p0.kill();
  p1.kill();
  start_row(p1);
  const TileSrc src1 = plan(p1);
  // the next row id is published by the leader: make it visible before p2
  // may need it (a null first row moves p2 to the next row)
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  prefetch_index(p1);
  p2 = p1;
  advance(p2);
  TileSrc src2 = plan(p2), src3 = src2;
  const uint16_t* v_src1 = src1.v;  // V of t+1
  int rows1 = src1.rows;
  p3 = p2;

  HalfLanes<D> tk, tv;
  tk.init(a.kst, wq, lane);
  tv.init(a.vst, wq, lane);
  // K of the first position -> odd buffer (t + 1 = 1)
  if (src1.rows >= 64) {
#pragma unroll
    for (int q = 0; q < NI; ++q) dma_slice<D>(sk1[g], src1.k, tk, q, wq);
  } else {
    dma_partial<D>(sk1[g], src1.k, kst, src1.rows, wq, lane);
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
    auto read_k = [&](int ks, int t2) -> uint4 {  // A operand of S, keys 32 t2 ..
      // two 8-byte reads: gfx950 streams ds_read_b64 faster than ds_read_b128
      const int r = 32 * t2 + lr;
      const uint2* p = reinterpret_cast<const uint2*>(skb + r * CH + ((2 * ks + hl) ^ swz<D>(r)));
      uint2 x = p[0], y = p[1];
      return make_uint4(x.x, x.y, y.x, y.y);
    };
    auto read_v = [&](int idx) -> uint4 {  // A operand of P.V step idx = u * DT + dt
      const int r1 = 16 * (idx / DT) + trr, xx = 32 * (idx % DT) + trc;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, xx)));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, xx)));
      const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
      return make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
    };
    if (pm1.has_tile()) {  // O += V(t-1)^T . P(t-1)^T, 16 keys per step
      // each operand register is refilled right after its MFMA has issued,
      // DT MFMAs before it is needed (back-to-back MFMAs into one
      // accumulator run at full rate on gfx950)
      uint4 va[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) va[dt] = read_v(dt);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pk[u]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          o[dt] = T::mfma32(as_vec8<T>(va[dt]), pb, o[dt]);
          if (u + 1 < 4) va[dt] = read_v((u + 1) * DT + dt);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    sc[0] = f32x16{};
    sc[1] = f32x16{};
    if (p0.has_tile()) {  // S(t) = K(t) . Q^T, 32 keys per accumulator
      uint4 ka[2][2];  // k-step k+1 is read while k-step k's MFMAs run
      ka[0][0] = read_k(0, 0);
      ka[0][1] = read_k(0, 1);
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const int b = k & 1;
        if (k + 1 < KS) {
          ka[b ^ 1][0] = read_k(k + 1, 0);
          ka[b ^ 1][1] = read_k(k + 1, 1);
        }
        sc[0] = T::mfma32(as_vec8<T>(ka[b][0]), qb[k], sc[0]);
        sc[1] = T::mfma32(as_vec8<T>(ka[b][1]), qb[k], sc[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // position t-1 closed its row: O = acc * (1/l) -> global
    if (pm1.live() && (pm1.j() < 0 || (pm1.hf() == 1 && pm1.n() + 1 >= pm1.ncnt()))) {
      const RowDesc d = row_of(pm1);
      const int qg = d.i * kBlock + qrow;
      const float rcp = 1.0f / pair32_sum(l_part);
      if (qg < d.L) {
        uint16_t* op = a.o + (d.t0 + qg) * ost + static_cast<int64_t>(d.h) * ohs;
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
    // the next position and its tile-load sources
    p3 = p2;
    advance(p3);
    src3 = plan(p3);
    // Q of a row that starts at t+1 (every S MFMA of t has been issued); the
    // wait for the loads happens here, once per row
    if (p1.live() && p1.row_start()) {
      const RowDesc d = row_of(p1);
      const int qg = d.i * kBlock + qrow;
      const bool qvalid = qg < d.L;
      const uint16_t* qp = a.q + (d.t0 + qg) * qst + static_cast<int64_t>(d.h) * qhs + 8 * half;
      u32x4 u[KS];  // all loads in flight before the one wait
#pragma unroll
      for (int s = 0; s < KS; ++s) u[s] = __builtin_bit_cast(u32x4, qvalid ? ld16(qp + 16 * s) : zero4());
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        asm volatile("" : "+v"(u[s]));
        qb[s] = as_vec8<T>(__builtin_bit_cast(uint4, u[s]));
      }
    }
  };

  // V phase of position t (parity P)
  auto v_phase = [&](auto par, int it) {
    constexpr int P = decltype(par)::value;
    uint4* kdst = P == 0 ? sk0[g] : sk1[g];  // K(t+2) has the parity of t
    uint4* vdst = P == 0 ? sv1[g] : sv0[g];  // V(t+1) the other one
    const bool kfull = src2.rows >= 64, vfull = rows1 >= 64;
    if (!kfull) dma_partial<D>(kdst, src2.k, kst, src2.rows, wq, lane);
    if (!vfull) dma_partial<D>(vdst, v_src1, vst, rows1, wq, lane);
    // full tiles: one K and one V slice load per softmax step
    auto dma_step = [&](int q) {
      if (q < NI) {
        if (kfull) dma_slice<D>(kdst, src2.k, tk, q, wq);
        if (vfull) dma_slice<D>(vdst, v_src1, tv, q, wq);
      }
    };
    dma_step(0);
    prefetch_index(p3);
    // online softmax of S(t)
    if (p0.live() && p0.row_start()) {  // row start: m = -inf, l = 1.0, acc = 0
      m_run = -INFINITY;
      l_part = half == 0 ? 1.0f : 0.0f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
    }
    if (p0.has_tile() && p0.j() == p0.i()) {  // diagonal block: key > query is masked
      // (qlim == qrow - 64 hf; deriving it from the row keeps the compares
      // inside the loop instead of hoisted into scalar masks)
      // key 32 t2 + 8 (v / 4) + 4 half + v % 4 > qlim, with the lane part
      // moved to the right so the key constants stay immediates
      const int lim = qrow - 64 * p0.hf() + (p0.j() - p0.i()) - 4 * half;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (32 * t2 + 8 * (v >> 2) + (v & 3) > lim) sc[t2][v] = -INFINITY;
    }
    // Positions without a tile run the softmax on zero scores: their output
    // is 0 (P.V is skipped) and nothing else reads the state they leave.
    float mx = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[t2][v]);
    mx = pair32_max(mx);
    dma_step(1);
    const float m_new = fmaxf(m_run, mx * c);
    float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    if (alpha != alpha) alpha = 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sc[t2][v], c, -m_new));
        sc[t2][v] = p;
        psum += p;
      }
      dma_step(2 + t2);
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
    // shift the stream window
    pm1 = p0;
    p0 = p1;
    p1 = p2;
    p2 = p3;
    v_src1 = src2.v;
    rows1 = src2.rows;
    src2 = src3;
    if (leader) s_done[it & 1][g] = (!pm1.live() && !p0.live() && !p1.live()) ? 1 : 0;
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
