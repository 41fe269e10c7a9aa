// Rotary position embedding (rotate-half) with optional per-head RMSNorm, in
// place on the query and key heads of the decoder-layer block's fused QKV
// projection: the attention-module step the reference's model callers run in
// torch before the op (ruler/models/llama.py:293-301 apply_rotary_pos_emb,
// ruler/models/qwen3.py:171-176 q_norm / k_norm then RoPE).
//
// Per (token t, head h) row of head_dim elements:
//   [optional] y = round(w * round(x * rsqrt(mean(x^2) + eps)))  (fp32 math;
//                  the two roundings of Qwen3MoeRMSNorm: the normalised row
//                  is cast to the input dtype, then multiplied by the weight)
//   out[k]       = round(y[k] * cos[p][k]    - y[k + d/2] * sin[p][k])
//   out[k + d/2] = round(y[k + d/2] * cos[p][k] + y[k] * sin[p][k])
// with p = positions[t] and cos / sin tables of d/2 angles per position
// (pos * theta^(-2k/d), evaluated by the caller in fp64 and rounded to fp32).
// Each product and sum is rounded separately (no fused multiply-add), as the
// torch elementwise composition of the same steps rounds them, so the result
// is the same bits.
//
// HBM-bound: 16 lanes per row, each lane 2 x d/32 elements (its dims of the
// two halves) and d/32 cos / sin values; algorithmic bytes per row =
// 2 x d x elem_bytes (read and written once) + the tables (L2-resident).
#include "fp_internal.h"

namespace fp {

template <typename T, int D>
__global__ __launch_bounds__(256) void k_rope(RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int E = D / 32;  // elements per lane and half (4 at d = 128, 2 at d = 64)
  typedef uint16_t elems[E];
  const int H = a.num_q_heads + a.num_kv_heads;
  const int64_t rows = a.num_tokens * H;
  const int l = threadIdx.x & 15;
  const int64_t step = (static_cast<int64_t>(gridDim.x) * blockDim.x) >> 4;
  for (int64_t r = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 4; r < rows;
       r += step) {
    const int64_t t = r / H;
    const int h = static_cast<int>(r % H);
    const bool is_q = h < a.num_q_heads;
    uint16_t* row = static_cast<uint16_t*>(is_q ? a.q : a.k) +
                    t * (is_q ? a.q_stride_tok : a.k_stride_tok) +
                    static_cast<int64_t>(is_q ? h : h - a.num_q_heads) *
                        (is_q ? a.q_stride_head : a.k_stride_head);
    float x1[E], x2[E];
    elems u1, u2;
    __builtin_memcpy(&u1, row + E * l, sizeof(elems));
    __builtin_memcpy(&u2, row + D / 2 + E * l, sizeof(elems));
#pragma unroll
    for (int e = 0; e < E; ++e) {
      x1[e] = T::to_f32(u1[e]);
      x2[e] = T::to_f32(u2[e]);
    }
    const uint16_t* w = static_cast<const uint16_t*>(is_q ? a.q_norm : a.k_norm);
    if (w != nullptr) {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, 16);
      const float inv = rsqrtf(ss / static_cast<float>(D) + a.eps);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float n1 = T::to_f32(T::from_f32(x1[e] * inv));
        const float n2 = T::to_f32(T::from_f32(x2[e] * inv));
        x1[e] = T::to_f32(T::from_f32(T::to_f32(w[E * l + e]) * n1));
        x2[e] = T::to_f32(T::from_f32(T::to_f32(w[D / 2 + E * l + e]) * n2));
      }
    }
    const int64_t p = min(max(a.positions[t], int64_t(0)), a.num_positions - 1);
    const float* cs = a.cos_tab + p * (D / 2) + E * l;
    const float* sn = a.sin_tab + p * (D / 2) + E * l;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float c = cs[e], s = sn[e];
      const float lo = x1[e] * c + (-x2[e]) * s;
      const float hi = x2[e] * c + x1[e] * s;
      u1[e] = T::from_f32(lo);
      u2[e] = T::from_f32(hi);
    }
    __builtin_memcpy(row + E * l, &u1, sizeof(elems));
    __builtin_memcpy(row + D / 2 + E * l, &u2, sizeof(elems));
  }
}

hipError_t launch_rope(const RopeArgs& a, int dtype, hipStream_t s) {
  const int64_t rows = a.num_tokens * (a.num_q_heads + a.num_kv_heads);
  if (rows <= 0) return hipSuccess;
  const int64_t want = (rows + 15) / 16;  // 16 rows per workgroup of 256 threads
  const dim3 g(static_cast<unsigned>(want < 65536 ? want : 65536)), b(256);
  with_head_dim(a.head_dim, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    if (dtype == FP_DTYPE_BF16) hipLaunchKernelGGL((k_rope<BF16, D>), g, b, 0, s, a);
    else hipLaunchKernelGGL((k_rope<F16, D>), g, b, 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

}  // namespace fp
