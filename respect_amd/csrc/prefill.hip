// Prefill / Flow element-wise kernels for gfx950, at PyTorch's rounding points.
//
// Replace the Triton kernels of respect/system/fused.py that the Prefill and
// Flow patches use (fused.py:126-194, 78-103):
//   square      q = float(x)^2                                  (_sq_k, :126-132)
//   add_sq      x = bf16(float(r) + float(h)); q = float(x)^2     (_add_sq_k, :135-145)
//   norm_apply  y = bf16(float(w) * bf16(float(x) * rsqrt(var + eps)))
//                                                              (_norm_apply_k, :148-159)
//   rope_vision y = bf16(x * cos + rotate_half(x) * sin), fp32 math, one
//               rounding at the end                            (_rope_v_k, :78-95)
// The RMSNorm mean itself stays with the caller (fused.py:168 takes it with
// PyTorch), so the reduction order is PyTorch's.  No FMA contraction: every
// multiply and add is a separately rounded fp32 operation; rsqrt(v) is a
// correctly rounded square root followed by a correctly rounded divide, the
// same as the decode RMSNorm here.  Each element depends on its own inputs
// (and its row's var), so rows never influence each other.
//
// 8 bf16 per thread: 16-byte loads, 16-byte bf16 stores, 2 x 16-byte fp32
// stores.  Rows may be strided; the innermost dimension is contiguous.  Grid:
// x = blocks of 8-element units along a row, y = rows from row0 (at most
// 65535 per launch), so no thread divides to find its row.

#include "common.h"
#include "respect_amd.h"

namespace rspx {

namespace {
__device__ __forceinline__ float rsqrt_rn(float v) { return 1.0f / __builtin_sqrtf(v); }
}  // namespace
static inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__global__ __launch_bounds__(256) void square_kernel(const uint16_t* x, int64_t sx, float* q, int64_t sq, int vcols,
                                                     int row0) {
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= vcols) return;
  const int row = row0 + blockIdx.y;
  const int c = v * 8;
  const u32x4 xw = *reinterpret_cast<const u32x4*>(x + row * sx + c);
  f32x4 a, b;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float x0 = bf16_lo(xw[i]), x1 = bf16_hi(xw[i]);
    a[2 * i] = x0 * x0;
    a[2 * i + 1] = x1 * x1;
    const float x2 = bf16_lo(xw[i + 2]), x3 = bf16_hi(xw[i + 2]);
    b[2 * i] = x2 * x2;
    b[2 * i + 1] = x3 * x3;
  }
  *reinterpret_cast<f32x4*>(q + row * sq + c) = a;
  *reinterpret_cast<f32x4*>(q + row * sq + c + 4) = b;
}

__global__ __launch_bounds__(256) void add_sq_kernel(const uint16_t* r, int64_t sr, const uint16_t* h, int64_t sh,
                                                     uint16_t* x, int64_t sx, float* q, int64_t sq, int vcols,
                                                     int row0) {
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= vcols) return;
  const int row = row0 + blockIdx.y;
  const int c = v * 8;
  const u32x4 rw = *reinterpret_cast<const u32x4*>(r + row * sr + c);
  const u32x4 hw = *reinterpret_cast<const u32x4*>(h + row * sh + c);
  u32x4 xo;
  float xv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xv[2 * i] = round_bf16(bf16_lo(rw[i]) + bf16_lo(hw[i]));
    xv[2 * i + 1] = round_bf16(bf16_hi(rw[i]) + bf16_hi(hw[i]));
    xo[i] = pack_bf16x2(xv[2 * i], xv[2 * i + 1]);
  }
  *reinterpret_cast<u32x4*>(x + row * sx + c) = xo;
  f32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = xv[i] * xv[i];
    b[i] = xv[4 + i] * xv[4 + i];
  }
  *reinterpret_cast<f32x4*>(q + row * sq + c) = a;
  *reinterpret_cast<f32x4*>(q + row * sq + c + 4) = b;
}

__global__ __launch_bounds__(256) void norm_apply_kernel(const uint16_t* x, int64_t sx, const float* var,
                                                         const uint16_t* w, uint16_t* y, int64_t sy, int vcols,
                                                         float eps, int row0) {
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= vcols) return;
  const int row = row0 + blockIdx.y;
  const int c = v * 8;
  const float rr = rsqrt_rn(var[row] + eps);
  const u32x4 xw = *reinterpret_cast<const u32x4*>(x + row * sx + c);
  const u32x4 ww = *reinterpret_cast<const u32x4*>(w + c);
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float h0 = round_bf16(bf16_lo(xw[i]) * rr), h1 = round_bf16(bf16_hi(xw[i]) * rr);
    out[i] = pack_bf16x2(bf16_lo(ww[i]) * h0, bf16_hi(ww[i]) * h1);
  }
  *reinterpret_cast<u32x4*>(y + row * sy + c) = out;
}

// One thread per 8 consecutive outputs of one (token l, head h) row of D.
// The rotated partner of element d is x[d + D/2] (negated) for d < D/2 and
// x[d - D/2] after; D / 2 is a multiple of 8, so a thread's partner is one
// contiguous 8-element run.
__global__ __launch_bounds__(256) void rope_vision_kernel(const uint16_t* x, int64_t sxl, int64_t sxh,
                                                          const float* cs, const float* sn, int64_t scl, uint16_t* y,
                                                          int NH, int D, int l0) {
  const int vD = D / 8;
  const int u = blockIdx.x * 256 + threadIdx.x;   // unit of token l's NH x vD units
  if (u >= NH * vD) return;
  const int l = blockIdx.y + l0;
  const int h = u / vD, v = u - h * vD;
  const int64_t lh = (int64_t)l * NH + h;
  const int d = 8 * v, half = D / 2;
  const uint16_t* row = x + l * sxl + h * sxh;
  const bool lo = d < half;
  const u32x4 xw = *reinterpret_cast<const u32x4*>(row + d);
  const u32x4 pw = *reinterpret_cast<const u32x4*>(row + (lo ? d + half : d - half));
  const float* cr = cs + l * scl + d;
  const float* sr = sn + l * scl + d;
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cr), c1 = *reinterpret_cast<const f32x4*>(cr + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sr), s1 = *reinterpret_cast<const f32x4*>(sr + 4);
  const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float p0 = bf16_lo(pw[i]), p1 = bf16_hi(pw[i]);
    if (lo) { p0 = -p0; p1 = -p1; }
    const float a0 = bf16_lo(xw[i]) * cv[2 * i], a1 = bf16_hi(xw[i]) * cv[2 * i + 1];
    const float b0 = p0 * sv[2 * i], b1 = p1 * sv[2 * i + 1];
    out[i] = pack_bf16x2(a0 + b0, a1 + b1);
  }
  *reinterpret_cast<u32x4*>(y + lh * D + d) = out;
}

// One launch per 65535 rows: grid (ceil(units / 256), rows), the kernel's
// row0 argument last.
template <class K, class... Args>
static int launch_rows(K kernel, int rows, int units, void* stream, Args... args) {
  const unsigned bx = (unsigned)((units + 255) / 256);
  for (int row0 = 0; row0 < rows; row0 += 65535)
    hipLaunchKernelGGL(kernel, dim3(bx, (unsigned)min(rows - row0, 65535)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), args..., row0);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

}  // namespace rspx

using namespace rspx;

extern "C" int rspx_square(const void* x, int64_t sx, float* q, int64_t sq, int rows, int n, void* stream) {
  if (rows < 0 || n < 0) return RSPX_EINVAL;
  if (n % 8 != 0) return RSPX_EUNSUPPORTED;
  if ((int64_t)rows * n == 0) return RSPX_OK;
  if (!x || !q || sx < n || sq < n) return RSPX_EINVAL;
  if (!al16(x) || !al16(q) || sx % 8 || sq % 4) return RSPX_EALIGN;
  return launch_rows(square_kernel, rows, n / 8, stream, static_cast<const uint16_t*>(x), sx, q, sq, n / 8);
}

extern "C" int rspx_add_sq(const void* r, int64_t sr, const void* h, int64_t sh, void* x, int64_t sx, float* q,
                           int64_t sq, int rows, int n, void* stream) {
  if (rows < 0 || n < 0) return RSPX_EINVAL;
  if (n % 8 != 0) return RSPX_EUNSUPPORTED;
  if ((int64_t)rows * n == 0) return RSPX_OK;
  if (!r || !h || !x || !q || sr < n || sh < n || sx < n || sq < n) return RSPX_EINVAL;
  if (!al16(r) || !al16(h) || !al16(x) || !al16(q) || sr % 8 || sh % 8 || sx % 8 || sq % 4) return RSPX_EALIGN;
  return launch_rows(add_sq_kernel, rows, n / 8, stream, static_cast<const uint16_t*>(r), sr,
                     static_cast<const uint16_t*>(h), sh, static_cast<uint16_t*>(x), sx, q, sq, n / 8);
}

extern "C" int rspx_norm_apply(const void* x, int64_t sx, const float* var, const void* w, void* y, int64_t sy,
                               int rows, int n, float eps, void* stream) {
  if (rows < 0 || n < 0) return RSPX_EINVAL;
  if (n % 8 != 0) return RSPX_EUNSUPPORTED;
  if ((int64_t)rows * n == 0) return RSPX_OK;
  if (!x || !var || !w || !y || sx < n || sy < n) return RSPX_EINVAL;
  if (!al16(x) || !al16(w) || !al16(y) || sx % 8 || sy % 8) return RSPX_EALIGN;
  return launch_rows(norm_apply_kernel, rows, n / 8, stream, static_cast<const uint16_t*>(x), sx, var,
                     static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), sy, n / 8, eps);
}

extern "C" int rspx_rope_vision(const void* x, int64_t sxl, int64_t sxh, const float* cos, const float* sin,
                                int64_t scl, void* y, int L, int NH, int D, void* stream) {
  if (L < 0 || NH < 0 || D <= 0) return RSPX_EINVAL;
  if (D % 16 != 0) return RSPX_EUNSUPPORTED;
  if ((int64_t)L * NH == 0) return RSPX_OK;
  if (!x || !cos || !sin || !y || scl < D) return RSPX_EINVAL;
  if (!al16(x) || !al16(cos) || !al16(sin) || !al16(y) || sxl % 8 || sxh % 8 || scl % 4) return RSPX_EALIGN;
  if ((int64_t)NH * (D / 8) > 0x7fffffff - 255) return RSPX_EUNSUPPORTED;
  return launch_rows(rope_vision_kernel, L, NH * (D / 8), stream, static_cast<const uint16_t*>(x), sxl, sxh, cos,
                     sin, scl, static_cast<uint16_t*>(y), NH, D);
}
