// SwiGLU for gfx950: y = bf16(bf16(silu(g)) * u), silu(g) = g / (1 + exp(-g)).
//
// Replaces silu_mul of respect/system/fused.py:106-123 (and the stock
// act_fn(gate) * up of the HF MLP): silu is computed in fp32 and rounded to
// bf16, then multiplied by u in fp32 and rounded again -- the rounding points
// of PyTorch's bf16 F.silu(g) * u.  No reduction: each element depends on its
// own g and u only, so rows never influence each other.
//
// 8 bf16 per thread (16-byte loads of g and u, one 16-byte store); g and u may
// be strided views (e.g. the two halves of a packed [rows, 2F] gate/up).

#include "common.h"
#include "respect_amd.h"

namespace rspx {

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, int64_t sg, const uint16_t* u,
                                                       int64_t su, uint16_t* y, int64_t sy, int rows, int vcols) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)rows * vcols) return;
  const int row = (int)(gid / vcols);
  const int c = (int)(gid - (int64_t)row * vcols) * 8;
  const u32x4 gw = *reinterpret_cast<const u32x4*>(g + row * sg + c);
  const u32x4 uw = *reinterpret_cast<const u32x4*>(u + row * su + c);
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float g0 = bf16_lo(gw[i]), g1 = bf16_hi(gw[i]);
    const float a0 = round_bf16(silu_f32(g0)), a1 = round_bf16(silu_f32(g1));
    out[i] = pack_bf16x2(a0 * bf16_lo(uw[i]), a1 * bf16_hi(uw[i]));
  }
  *reinterpret_cast<u32x4*>(y + row * sy + c) = out;
}

}  // namespace rspx

using namespace rspx;

extern "C" int rspx_silu_mul(const void* g, int64_t sg, const void* u, int64_t su, void* y, int64_t sy, int rows,
                             int cols, void* stream) {
  if (rows < 0 || cols < 0) return RSPX_EINVAL;
  if (cols % 8 != 0) return RSPX_EUNSUPPORTED;
  if ((int64_t)rows * cols == 0) return RSPX_OK;
  if (!g || !u || !y) return RSPX_EINVAL;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!al(g) || !al(u) || !al(y) || sg % 8 || su % 8 || sy % 8) return RSPX_EALIGN;
  const int vcols = cols / 8;
  const int64_t threads = (int64_t)rows * vcols;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(g), sg,
                     static_cast<const uint16_t*>(u), su, static_cast<uint16_t*>(y), sy, rows, vcols);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
