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

// Row stride value that names the tiled layout (RSPX_TILED of the C ABI).
constexpr int64_t kTiled = -1;

// The output of a K-split linear layer: the fp32 chunk partials of one
// element added in chunk order, ((p0 + p1) + p2) + ... (stride = elements
// between chunks).  Every consumer of split partials uses this, so the value
// (and its bf16 rounding) is the same wherever the sum is taken.
__device__ __forceinline__ f32x4 sum_parts4(const float* p, int S, int64_t stride) {
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  for (int s = 1; s < S; ++s) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(p + s * stride);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] + q[e];
  }
  return v;
}

}  // namespace rspx
