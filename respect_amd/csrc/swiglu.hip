// SwiGLU for gfx950: y = bf16(bf16(silu(g)) * u), silu(g) = g / (1 + exp(-g)).
//
// Replaces silu_mul of respect/system/fused.py:106-123 (and the stock
// act_fn(gate) * up of the HF MLP): silu is computed in fp32 and rounded to
// bf16, then multiplied by u in fp32 and rounded again -- the rounding points
// of PyTorch's bf16 F.silu(g) * u.  No reduction: each element depends on its
// own g and u only, so rows never influence each other.
//
// Two bf16 per thread (4-byte loads of g and u, one 4-byte store), or one
// where cols is odd or an operand is not 4-byte aligned (the same values).
// On MI355X the packed gate/up [64, 2 x 12288] call takes 3.02 us at two
// elements per thread, 3.09 at four and 3.42 at eight (rotating inputs beyond
// the MALL): a launch this small is bound by memory latency, and more waves
// in flight hide more of it.  Non-temporal stores (not kept in L2) shorten the
// write-back at the kernel's end: 3.02 -> 2.80 us (non-temporal loads 2.86,
// both 2.84).  g and u may be strided views (e.g. the two
// halves of a packed [rows, 2F] gate/up).

#include "common.h"
#include "respect_amd.h"

namespace rspx {

__device__ __forceinline__ float swiglu1(float g, float u) { return round_bf16(silu_f32(g)) * u; }

template <bool PAIR>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, int64_t sg, const uint16_t* u,
                                                       int64_t su, uint16_t* y, int64_t sy, int rows, int units) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)rows * units) return;
  const int row = (int)(gid / units);
  const int c = (int)(gid - (int64_t)row * units) * (PAIR ? 2 : 1);
  if constexpr (PAIR) {
    const uint32_t gw = *reinterpret_cast<const uint32_t*>(g + row * sg + c);
    const uint32_t uw = *reinterpret_cast<const uint32_t*>(u + row * su + c);
    __builtin_nontemporal_store(pack_bf16x2(swiglu1(bf16_lo(gw), bf16_lo(uw)), swiglu1(bf16_hi(gw), bf16_hi(uw))),
                                reinterpret_cast<uint32_t*>(y + row * sy + c));
  } else {
    __builtin_nontemporal_store(
        f32_to_bf16_rne(swiglu1(bf16_to_f32(g[row * sg + c]), bf16_to_f32(u[row * su + c]))), y + row * sy + c);
  }
}

}  // namespace rspx

using namespace rspx;

extern "C" int rspx_silu_mul(const void* g, int64_t sg, const void* u, int64_t su, void* y, int64_t sy, int rows,
                             int cols, void* stream) {
  if (rows < 0 || cols < 0) return RSPX_EINVAL;
  if ((int64_t)rows * cols == 0) return RSPX_OK;
  if (!g || !u || !y) return RSPX_EINVAL;
  auto al = [](const void* p, unsigned a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (!al(g, 2) || !al(u, 2) || !al(y, 2)) return RSPX_EALIGN;
  const bool pair = cols % 2 == 0 && al(g, 4) && al(u, 4) && al(y, 4) && sg % 2 == 0 && su % 2 == 0 && sy % 2 == 0;
  const int units = pair ? cols / 2 : cols;
  const int64_t blocks = ((int64_t)rows * units + 255) / 256;
  if (blocks > 0x7fffffff) return RSPX_EUNSUPPORTED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* G = static_cast<const uint16_t*>(g);
  const uint16_t* U = static_cast<const uint16_t*>(u);
  uint16_t* Y = static_cast<uint16_t*>(y);
  if (pair) hipLaunchKernelGGL(silu_mul_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, G, sg, U, su, Y, sy, rows, units);
  else hipLaunchKernelGGL(silu_mul_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, G, sg, U, su, Y, sy, rows, units);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
