// Shared device helpers for the gfx950 (CDNA4) kernels of respect_amd.
//
// All kernels are compiled with -ffp-contract=off: every fused multiply-add is
// written out explicitly with __builtin_fmaf, so the same source expression
// produces the same instruction sequence wherever it is inlined.  Bitwise
// reproducibility across call shapes depends on that.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rspx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_huge_valf();

// bf16 <-> fp32.  bf16 -> fp32 is exact (a shift); fp32 -> bf16 rounds to
// nearest even, NaN stays NaN.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// fp32 -> bf16 with round-to-nearest-even on the gfx950 converter
// (v_cvt_pk_bf16_f32); NaN stays NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Round a float to the nearest-even bf16 value, kept in fp32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// SwiGLU's silu in fp32: g / (1 + exp(-g)) with the accurate library
// exponential and an IEEE divide; g -> -inf gives g / inf = -0, as PyTorch does.
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// 2^x on the hardware transcendental unit (v_exp_f32).  -inf -> 0.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Wave-wide lane shuffles (64 lanes).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}
__device__ __forceinline__ float shfl_idx(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}
__device__ __forceinline__ int shfl_idx_i(int v, int src) {
  return __builtin_amdgcn_ds_bpermute(src << 2, v);
}

// The tiled layout of a bf16 activation matrix [M, K] (K % 32 == 0), the
// one the linear layers read their x operand from fastest: per 64-row block
// and 32-wide k-block, the four 16 x 32 MFMA operand tiles of that block,
// 1 KB each, lane n16 + 16 g of a tile holding row n16 of the tile, k
// 8 g .. 8 g + 7 of the k-block.  Element (m, k) sits at tiled_offset(m, k, K);
// the buffer holds ceil(M / 64) * 64 * K elements.
__device__ __forceinline__ int64_t tiled_offset(int m, int k, int K) {
  return ((((int64_t)(m >> 6) * (K >> 5) + (k >> 5)) * 4 + ((m >> 4) & 3)) * 64 + (m & 15) + 16 * ((k >> 3) & 3)) *
             8 +
         (k & 7);
}


// Row stride value that names the tiled layouts (RSPX_TILED of the C ABI).
constexpr int64_t kTiled = -1;

// The output of a K-split linear layer: the fp32 chunk partials of one
// element added in chunk order, ((p0 + p1) + p2) + ... (stride = elements
// between chunks, 1 <= S <= SC).  Every consumer of split partials uses this,
// so the value (and its bf16 rounding) is the same wherever the sum is taken.
// SC (1, 2, 4 or kMaxSplits, a compile-time bound) lets every load be issued
// before the first add, without branches: chunk s >= S re-reads chunk S - 1
// and its add is not taken.  The chunks then arrive in one memory latency
// instead of S in a row.
constexpr int kMaxSplits = 8;
template <int SC>
__device__ __forceinline__ f32x4 sum_parts4(const float* p, int S, int64_t stride) {
  f32x4 q[SC];
#pragma unroll
  for (int s = 0; s < SC; ++s) q[s] = *reinterpret_cast<const f32x4*>(p + (int64_t)(s < S ? s : S - 1) * stride);
  f32x4 v = q[0];
#pragma unroll
  for (int s = 1; s < SC; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = s < S ? v[e] + q[s][e] : v[e];
  return v;
}

// Eight consecutive elements (two f32x4 at p and p + 4) the same way.
template <int SC>
__device__ __forceinline__ void sum_parts8(const float* p, int S, int64_t stride, f32x4& a, f32x4& b) {
  f32x4 qa[SC], qb[SC];
#pragma unroll
  for (int s = 0; s < SC; ++s) {
    const float* ps = p + (int64_t)(s < S ? s : S - 1) * stride;
    qa[s] = *reinterpret_cast<const f32x4*>(ps);
    qb[s] = *reinterpret_cast<const f32x4*>(ps + 4);
  }
  a = qa[0];
  b = qb[0];
#pragma unroll
  for (int s = 1; s < SC; ++s) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = s < S ? a[e] + qa[s][e] : a[e];
      b[e] = s < S ? b[e] + qb[s][e] : b[e];
    }
  }
}

// The compile-time bound SC for a run-time chunk count S (1 <= S <= 8).
#define RSPX_WITH_SPLITS(S, SC, ...)                                  \
  do {                                                                \
    if ((S) <= 1) { constexpr int SC = 1; __VA_ARGS__; }              \
    else if ((S) <= 2) { constexpr int SC = 2; __VA_ARGS__; }         \
    else if ((S) <= 4) { constexpr int SC = 4; __VA_ARGS__; }         \
    else { constexpr int SC = kMaxSplits; __VA_ARGS__; }              \
  } while (0)

}  // namespace rspx
