// Building blocks of the gfx950 attention kernels: LDS tile layout (64-bank
// chunk swizzle), direct-to-LDS tile loads, packed conversions and the
// explicit wait + barrier helpers used to pipeline tile loads against MFMA.
#pragma once

#include "fp_internal.h"

namespace fp {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x002;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmemRead = 0x020;
constexpr int kSchedDsRead = 0x100;

// compile-time arguments of generic lambdas (unrolled pipeline stages)
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};
template <int N>
struct IntC {
  static constexpr int value = N;
};

// Load through the scalar cache: the address must be wave-uniform and the
// data must not be written while the kernel runs (tables and index lists
// written by earlier kernels of the stream).
template <typename X>
__device__ __forceinline__ X sld(const X* p) {
  static_assert(sizeof(X) % 4 == 0, "scalar loads move whole dwords");
  const __attribute__((address_space(4))) uint32_t* w =
      reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(
          reinterpret_cast<uintptr_t>(p));
  uint32_t buf[sizeof(X) / 4];
#pragma unroll
  for (unsigned k = 0; k < sizeof(X) / 4; ++k) buf[k] = w[k];
  X x;
  __builtin_memcpy(&x, buf, sizeof(X));
  return x;
}

// chunk swizzle of row r in a 128 x D tile (D/8 chunks of 16 bytes per row):
// rows of 16 or 32 chunks (d = 128, 256) permute the low 4 chunk bits by the
// row's low 4 bits (conflict free for the K operand reads and the transposing
// V reads alike, since a row is a whole number of 256-byte bank cycles), rows
// of 8 chunks (d = 64) the low 3 bits
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (r >> 1) & 7;
}

template <int D>
__device__ __forceinline__ int tile_elem(int r, int x) {
  return r * D + ((((x >> 3) ^ swz<D>(r))) << 3) + (x & 7);
}

// two fp32 -> packed pair of the input type (round to nearest even)
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// p.x + p.y + acc for a packed pair of the input type (v_dot2c_f32_* against
// (1, 1), fp32 accumulate): the row sums of the P that P.V consumes, one VALU
// instruction per two scores
template <typename T>
__device__ __forceinline__ float add_pair(uint32_t p, float acc);
template <>
__device__ __forceinline__ float add_pair<BF16>(uint32_t p, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), bf16x2{1.0, 1.0}, acc,
                                         false);
}
template <>
__device__ __forceinline__ float add_pair<F16>(uint32_t p, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), f16x2{1.0, 1.0}, acc, false);
}

// Conditional rescaling: the running maximum m that P = exp2(s * scale - m)
// is taken against moves only when, against the current m, the sum of a
// lane's P over one tile would exceed kRescaleSum (so P <= 2^8 on every path),
// or on a row's first tile. The output accumulators are rescaled only then
// (about once per row instead of in most steps). O and l are scaled by the
// same factors, so O / l is unchanged up to rounding.
constexpr float kRescaleSum = 256.0f;

// wait for this wave's vector-memory ops down to N outstanding, then barrier
template <int N>
__device__ __forceinline__ void vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(N) : "memory");
}
// all of this wave's LDS reads are done, then barrier (buffer may be refilled)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Direct-to-LDS loads (global_load_lds_dwordx4: 64 lanes x 16 bytes into LDS
// at M0 + 16 * lane) are issued from inline asm. The compiler models a
// global_load_lds it generates as an LDS event of its own kind and, while one
// is outstanding, turns every wait for an ordinary LDS read into lgkmcnt(0)
// and every wait for a register load into vmcnt(0), which serialises the MFMA
// operand reads. The attention kernels need no compiler tracking of these
// loads: they wait for them explicitly (vmcnt at their barriers), and no
// compiler-generated instruction in them uses M0. s_nop 4 gives the five wait
// states a VMEM instruction needs after a VALU write of its SGPRs (the
// readfirstlane of the base) and after the M0 write.
__device__ __forceinline__ uint32_t lds_addr(void* p) {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)p))));
}
// A wave-uniform 64-bit address as a scalar operand. readfirstlane returns
// int: each half goes through uint32_t before widening (no sign extension).
__device__ __forceinline__ uint64_t scalar_addr(const void* p) {
  const uint64_t b = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
// one load: per-lane 64-bit address
__device__ __forceinline__ void dma16_vaddr(void* lds_slice, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_addr(lds_slice)), "v"(src) : "memory", "m0");
}
// one load whose scalar base and LDS address were formed by SALU (no VALU
// write of an SGPR to wait for): only the M0 write needs a wait state
__device__ __forceinline__ void dma16_sbase_m0(uint32_t lds, uint64_t sbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds), "v"(voff), "s"(sbase) : "memory", "m0");
}
// Direct-to-LDS loads of one R x D tile (rows R*j .. R*j+R-1 of a K, V or
// Q head) by NW waves. Wave w fills the 1 KB LDS slices w*NI .. w*NI+NI-1;
// in each slice lane l writes physical chunk l % CH of row slice*RPW + l / CH,
// so it fetches logical chunk (l % CH) ^ swz(row) of that row. Because
// swz(row) only depends on (l / CH) and on the slice index modulo a small
// period, the per-lane part of the source address is a 32-bit byte offset
// from a small precomputed table and the rest is a wave-uniform (scalar)
// base.
template <int D, int R, int NW>
struct TileLanes {
  static constexpr int CH = D / 8;            // chunks per row
  static constexpr int RPW = 64 / CH;         // rows per wave instruction
  static constexpr int NI = R * CH / 64 / NW; // instructions per wave per tile
  static constexpr int PER = D == 256 ? 8 : D == 128 ? 4 : 2;  // period of swz over the slice index
  static_assert(NI >= 1 && NI % PER == 0, "every wave's first slice must start a swizzle period");
  uint32_t off[PER];                          // per-lane byte offsets
  __device__ __forceinline__ void init(int64_t stride, int w, int lane) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = (w * NI + q) * RPW + lane / CH;
      const int c = (lane % CH) ^ swz<D>(r);
      off[q] = static_cast<uint32_t>(((lane / CH) * stride + 8 * c) * 2);
    }
  }
};

template <int D, int R, int NW>
__device__ __forceinline__ void issue_tile(uint4* lds, const uint16_t* base, int64_t stride,
                                           const TileLanes<D, R, NW>& tl, int j, int L, int w,
                                           int lane) {
  typedef TileLanes<D, R, NW> TL;
  constexpr int CH = TL::CH, RPW = TL::RPW, NI = TL::NI;
  if ((j + 1) * R <= L) {
    // one scalar base and LDS address per tile; the slices' offsets are
    // scalar adds, so each load costs an add, the M0 write and one wait state
    uint64_t sb = scalar_addr(reinterpret_cast<const char*>(base) +
                              static_cast<int64_t>(j * R + w * NI * RPW) * stride * 2);
    const uint32_t l0 = lds_addr(lds + w * NI * 64);
    // the base was written by VALU (readfirstlane): five wait states before
    // a VMEM instruction reads it; every later use goes through this asm
    asm volatile("s_nop 4" : "+s"(sb));
    const uint64_t step = static_cast<uint64_t>(RPW) * static_cast<uint64_t>(stride) * 2;
#pragma unroll
    for (int q = 0; q < NI; ++q)
      dma16_sbase_m0(l0 + q * 1024, sb + q * step, tl.off[q % TL::PER]);
  } else {  // partial last block: rows past the end read row L-1 (masked keys, p = 0)
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int slot = w * NI + q;
      const int r = slot * RPW + lane / CH;
      const int c = (lane % CH) ^ swz<D>(r);
      const int gk = min(j * R + r, L - 1);
      dma16_vaddr(lds + slot * 64, base + static_cast<int64_t>(gk) * stride + 8 * c);
    }
  }
}

// Reductions over the two 32-lane halves of a wave (lane l with l ^ 32):
// v_permlane32_swap exchanges the halves of its two operands, so max / sum
// of the pair it returns is the value of the two lanes, in every lane.
__device__ __forceinline__ float pair32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<unsigned>(r[0])),
               __builtin_bit_cast(float, static_cast<unsigned>(r[1])));
}
__device__ __forceinline__ float pair32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return __builtin_bit_cast(float, static_cast<unsigned>(r[0])) +
         __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}

}  // namespace fp
