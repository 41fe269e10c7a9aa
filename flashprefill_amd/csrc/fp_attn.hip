// Varlen GQA block-sparse flash-attention forward for gfx950
// (ops/flashprefill_native_forward.py:227-344,
//  ops/flashprefill_varlen_func.py:449-575).
//
// One workgroup (4 waves) owns one (query head h, sequence b, q-block i) item
// and walks that row's selected key blocks in ascending order. Wave w owns the
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
// all on v_mfma_f32_32x32x16 (bf16 or fp16 in, fp32 accumulate). K and V
// blocks (128 keys x d) are gathered by index into LDS with a row-dependent
// 16-byte-chunk XOR swizzle that keeps both the K operand reads and the
// transposing V reads free of bank conflicts.
//
// Numerics follow the reference loop: m starts at -inf and l at 1.0, one
// 128-key tile per selected block, alpha = exp2(m_old - m_new) with NaN -> 1,
// l accumulates the fp32 p, P is rounded to the input dtype before P.V, the
// diagonal block masks key > query, and O = acc * (1/l).
#include "fp_internal.h"

namespace fp {

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// element offset of (row r, column x) in a 128 x D tile
template <int D>
__device__ __forceinline__ int tile_elem(int r, int x) {
  return r * D + ((((x >> 3) ^ swz(r))) << 3) + (x & 7);
}

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void k_attn(AttnArgs a) {
  constexpr int CH = D / 8;   // 16-byte chunks per row
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-row tiles of O^T
  __shared__ uint4 sk[kBlock * CH];
  __shared__ uint4 sv[kBlock * CH];

  int item, h;
  map_item(blockIdx.x, a.Hq, item, h);
  const int64_t nitems = a.tab.seq_tile[a.B];
  if (item >= nitems) return;
  const int b = a.tab.items[2 * item];
  const int i = a.tab.items[2 * item + 1];
  const int64_t tile_b = a.tab.seq_tile[b];
  const int L = a.tab.seq_len[b];
  const int64_t t0 = a.tab.seq_start[b];
  const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + a.tab.seq_tri[b] +
                          static_cast<int64_t>(i) * (i + 1) / 2;
  // counts and lists come from the search stage; clamp them to the row's
  // capacity so a stale workspace can never index outside the sequence
  const int ncnt = min(max(a.cnt[static_cast<int64_t>(h) * a.nb_sum_cap + tile_b + i], 0), i + 1);
  const int32_t* list = a.idx + row_tri;
  const int kvh = h / (a.Hq / a.Hkv);

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * w + l32;           // query row inside the block
  const int qg = i * kBlock + qrow;         // query position inside the sequence
  const bool qvalid = qg < L;
  const float c = a.sm_scale_log2;

  // Q^T as MFMA B operand: lane (query l32, dims 16 s + 8 half .. +7)
  typename T::vec8 qb[KS];
  {
    const uint16_t* qp = a.q + (t0 + qg) * a.qst + static_cast<int64_t>(h) * a.qhs + 8 * half;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = as_vec8<T>(qvalid ? ld16(qp + 16 * s) : zero4());
  }

  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_part = half == 0 ? 1.0f : 0.0f;  // the two halves' partial sums add up to l

  const uint16_t* kbase = a.k + t0 * a.kst + static_cast<int64_t>(kvh) * a.khs;
  const uint16_t* vbase = a.v + t0 * a.vst + static_cast<int64_t>(kvh) * a.vhs;
  const uint16_t* sv16 = reinterpret_cast<const uint16_t*>(sv);

  // transposing-read coordinates of this lane (16-lane groups)
  const int g16 = lane >> 4, i16 = lane & 15;
  const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);       // + 16 u (+ 8)
  const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);    // + 32 dt

  for (int n = 0; n < ncnt; ++n) {
    const int j = min(max(__builtin_amdgcn_readfirstlane(list[n]), 0), i);
    __syncthreads();  // previous block's LDS reads are done
    for (int cidx = t; cidx < kBlock * CH; cidx += 256) {
      const int r = cidx / CH, ch = cidx % CH;
      const int gk = j * kBlock + r;
      uint4 kv = zero4(), vv = zero4();
      if (gk < L) {
        kv = ld16(kbase + static_cast<int64_t>(gk) * a.kst + 8 * ch);
        vv = ld16(vbase + static_cast<int64_t>(gk) * a.vst + 8 * ch);
      }
      const int pos = r * CH + (ch ^ swz(r));
      sk[pos] = kv;
      sv[pos] = vv;
    }
    __syncthreads();

    // S^T = K . Q^T: s[st][v] is key 32 st + 8 (v/4) + 4 half + v%4, query l32
    f32x16 s[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      s[st] = f32x16{};
      const int r = 32 * st + l32;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 kop = sk[r * CH + ((2 * ks + half) ^ swz(r))];
        s[st] = T::mfma32(as_vec8<T>(kop), qb[ks], s[st]);
      }
    }
    if (j == i) {  // diagonal block: key > query is masked
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = 32 * st + 8 * (v >> 2) + 4 * half + (v & 3);
          if (key > qrow) s[st][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[st][v]);
    mx = fmaxf(mx, xor32_f(mx));
    const float m_new = fmaxf(m_run, mx * c);
    float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    if (alpha != alpha) alpha = 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[st][v], c, -m_new));
        s[st][v] = p;
        psum += p;
      }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[dt][v] *= alpha;
    m_run = m_new;

    // O^T += V^T . P^T over 8 steps of 16 keys. B element e of lane (q, half)
    // is key 16 u + (e < 4 ? 4 half + e : 8 + 4 half + e - 4); the A operand
    // (V^T) is read in the same key order with two transposing reads.
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int st = u >> 1, hh = u & 1;
      uint16_t pk[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pk[e] = T::from_f32(s[st][8 * hh + e]);
      const typename T::vec8 pb = __builtin_bit_cast(typename T::vec8, pk);
      const int r1 = 16 * u + tr_row;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int x = 32 * dt + tr_col;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1, x)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(sv16 + tile_elem<D>(r1 + 8, x)));
        short va8[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = T::mfma32(__builtin_bit_cast(typename T::vec8, va8), pb, o[dt]);
      }
    }
  }

  const float l = l_part + xor32_f(l_part);
  const float rcp = 1.0f / l;
  if (qvalid) {
    uint16_t* op = a.o + (t0 + qg) * a.ost + static_cast<int64_t>(h) * a.ohs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * half;
        u16x4 pk;
#pragma unroll
        for (int r = 0; r < 4; ++r) pk[r] = T::from_f32(o[dt][4 * g4 + r] * rcp);
        *reinterpret_cast<u16x4*>(op + d) = pk;
      }
  }
}

hipError_t launch_attn(const AttnArgs& a, int dtype, int head_dim, int64_t grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  const dim3 g(static_cast<unsigned>(grid)), blk(256);
  if (dtype == FP_DTYPE_BF16) {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn<BF16, 128>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn<BF16, 64>), g, blk, 0, s, a);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL((k_attn<F16, 128>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((k_attn<F16, 64>), g, blk, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace fp
