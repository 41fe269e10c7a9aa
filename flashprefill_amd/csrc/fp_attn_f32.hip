// Block-sparse attention forward for fp32 inputs
// (ops/flashprefill_native_forward.py:227-344,
//  ops/flashprefill_varlen_func.py:449-575, run with fp32 q / k / v).
//
// One workgroup (BLK / 32 waves) owns one (query head, sequence, q-block) row
// as in k_attn, in the same "one query per lane" orientation, on fp32 MFMA
// (v_mfma_f32_32x32x2_f32: fp32 products, where the reference's tl.dot of fp32
// inputs uses TF32):
//
//   S^T = K . Q^T    A = K rows from LDS, B = Q^T in registers; k-step s
//                    pairs dim s (lanes 0-31) with dim D/2 + s (lanes 32-63)
//   O^T += V^T . P^T A = V^T read from the key-major V tile in LDS, B = P^T
//                    straight from the S^T accumulators: for accumulator
//                    element v of key tile t, lanes 0-31 hold key
//                    32 t + 8 (v/4) + v%4 and lanes 32-63 that key + 4, which
//                    is the MFMA's k pair, so P never moves between lanes
//
// Numerics follow the reference loop exactly: m starts at -inf and l at 1.0,
// one BLK-key tile per selected block, alpha = exp2(m_old - m_new) with NaN ->
// 1, l = l * alpha + sum p, acc = acc * alpha + p . V with p kept in fp32 (its
// cast to V's dtype is the identity for fp32), the diagonal block masks
// key > query, O = acc / l. K / V tiles are staged through registers into LDS
// (the K rows padded by 16 bytes so that 32 rows read at one column are
// conflict free); rows past the sequence end (only in the diagonal block,
// where they are masked) repeat the last row.
#include "fp_attn_common.h"

namespace fp {

template <int D, int BLK>
__global__ __launch_bounds__(2 * BLK, 1) void k_attn_f32(AttnArgs a) {
  constexpr int NW = BLK / 32;  // waves
  constexpr int KT = BLK / 32;  // 32-key tiles of S^T per block
  constexpr int KS = D / 2;     // MFMA k-steps over the head dim
  constexpr int DT = D / 32;    // 32-dim tiles of O^T
  constexpr int KSTR = D + 4;   // padded K row (floats)
  __shared__ float sk[BLK * KSTR];
  __shared__ float sv[BLK * D];

  const int64_t nitems = sld(a.tab.seq_tile + a.B);
  int item, h;
  map_row(blockIdx.x, a.Hq, a.Hkv, a.nb_sum_cap, item, h);
  if (item >= nitems) return;
  const ItemRec rec = sld(a.tab.items + item);
  const int i = rec.i, L = rec.L;
  const int64_t t0 = rec.t0;
  const int64_t row_tri = static_cast<int64_t>(h) * a.tri_cap + rec.tri;
  const int ncnt =
      min(max(sld(a.cnt + static_cast<int64_t>(h) * a.nb_sum_cap + rec.tile), 0), i + 1);
  const int32_t* list = a.idx + row_tri;
  const int kvh = h / (a.Hq / a.Hkv);

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int qrow = 32 * w + l32;
  const int qg = i * BLK + qrow;
  const bool qvalid = qg < L;
  const float c = a.sm_scale_log2;
  const float* q = reinterpret_cast<const float*>(a.q);
  const float* kbase = reinterpret_cast<const float*>(a.k) + t0 * a.kst + kvh * a.khs;
  const float* vbase = reinterpret_cast<const float*>(a.v) + t0 * a.vst + kvh * a.vhs;

  // Q^T as B operands: qb[s] = Q[query][half * KS + s]
  float qb[KS];
  {
    const float* qp = q + (t0 + (qvalid ? qg : 0)) * a.qst + h * a.qhs + half * KS;
#pragma unroll
    for (int s4 = 0; s4 < KS / 4; ++s4) {
      const float4 x = qvalid ? *reinterpret_cast<const float4*>(qp + 4 * s4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
      qb[4 * s4] = x.x; qb[4 * s4 + 1] = x.y; qb[4 * s4 + 2] = x.z; qb[4 * s4 + 3] = x.w;
    }
  }

  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_part = half == 0 ? 1.0f : 0.0f;  // the two halves' partial sums add up to l

  for (int n = 0; n < ncnt; ++n) {
    const int j = min(max(sld(list + n), 0), i);
    // stage K and V of block j (all waves), then barrier
    for (int cidx = t; cidx < BLK * (D / 4); cidx += 64 * NW) {
      const int r = cidx / (D / 4), x4 = cidx % (D / 4);
      const int64_t gk = min(j * BLK + r, L - 1);
      const float4 kx = *reinterpret_cast<const float4*>(kbase + gk * a.kst + 4 * x4);
      const float4 vx = *reinterpret_cast<const float4*>(vbase + gk * a.vst + 4 * x4);
      *reinterpret_cast<float4*>(sk + r * KSTR + 4 * x4) = kx;
      *reinterpret_cast<float4*>(sv + r * D + 4 * x4) = vx;
    }
    __syncthreads();

    f32x16 s[KT];
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4) {
      s[t4] = f32x16{};
      const float* kr = sk + (32 * t4 + l32) * KSTR + half * KS;
#pragma unroll
      for (int s4 = 0; s4 < KS / 4; ++s4) {
        const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * s4);
        s[t4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.x, qb[4 * s4], s[t4], 0, 0, 0);
        s[t4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.y, qb[4 * s4 + 1], s[t4], 0, 0, 0);
        s[t4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.z, qb[4 * s4 + 2], s[t4], 0, 0, 0);
        s[t4] = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.w, qb[4 * s4 + 3], s[t4], 0, 0, 0);
      }
    }
    if (j == i) {  // key > query is masked on the diagonal block
#pragma unroll
      for (int t4 = 0; t4 < KT; ++t4)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = 32 * t4 + 8 * (v >> 2) + 4 * half + (v & 3);
          if (key > qrow) s[t4][v] = -INFINITY;
        }
    }
    // online softmax over this block (base 2, scores scaled by c)
    float mx = -INFINITY;
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[t4][v]);
    const float m_new = fmaxf(m_run, pair32_max(mx) * c);
    float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    if (alpha != alpha) alpha = 1.0f;
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s[t4][v] = __builtin_amdgcn_exp2f(fmaf(s[t4][v], c, -m_new));
        psum += s[t4][v];
      }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[dt][v] *= alpha;
    // O^T += V^T . P^T
#pragma unroll
    for (int t4 = 0; t4 < KT; ++t4)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = 32 * t4 + 8 * (v >> 2) + 4 * half + (v & 3);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(sv[key * D + 32 * dt + l32], s[t4][v],
                                                      o[dt], 0, 0, 0);
      }
    __syncthreads();  // every wave is done with the K / V tiles
  }

  const float l = pair32_sum(l_part);
  const float rcp = 1.0f / l;
  if (qvalid) {
    float* op = reinterpret_cast<float*>(a.o) + (t0 + qg) * a.ost + h * a.ohs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<float4*>(op + 32 * dt + 8 * g4 + 4 * half) =
            make_float4(o[dt][4 * g4] * rcp, o[dt][4 * g4 + 1] * rcp, o[dt][4 * g4 + 2] * rcp,
                        o[dt][4 * g4 + 3] * rcp);
  }
}

template <int D>
hipError_t launch_attn_f32_t(const AttnArgs& a, int block, int64_t grid, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(grid));
  if (block == 128) hipLaunchKernelGGL((k_attn_f32<D, 128>), g, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((k_attn_f32<D, 64>), g, dim3(128), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_f32(const AttnArgs& a, int head_dim, int block, int64_t grid,
                           hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  return head_dim == 128 ? launch_attn_f32_t<128>(a, block, grid, s)
                         : launch_attn_f32_t<64>(a, block, grid, s);
}

}  // namespace fp
