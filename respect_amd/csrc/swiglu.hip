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
// Grid: x = 512-thread blocks along a row, y = rows (one launch per 65535
// rows), so a thread finds its row and column without a division.  On MI355X the
// packed gate/up [64, 2 x 12288] call (rotating inputs beyond the MALL)
// takes 2.48 us; the same kernel indexed by one flat thread number, whose
// row comes from a 64-bit division, took 2.79 us (the division's ~60
// instructions stand before the loads of a call that is one memory round
// trip).  256-thread blocks: 2.54 us; 128: 2.64 us; four elements per
// thread: 3.02 us.  Non-temporal stores (not kept in L2) shorten the
// write-back at the kernel's end (3.02 -> 2.80 us in the flat form).  g and
// u may be strided views (e.g. the two halves of a packed [rows, 2F] gate/up).
#include "common.h"
#include "respect_amd.h"

namespace rspx {

__device__ __forceinline__ float swiglu1(float g, float u) { return round_bf16(silu_f32(g)) * u; }

constexpr int kSwigluThreads = 512;
constexpr int kMaxGridY = 65535;

template <bool PAIR>
__global__ __launch_bounds__(kSwigluThreads) void silu_mul_kernel(const uint16_t* g, int64_t sg, const uint16_t* u,
                                                                  int64_t su, uint16_t* y, int64_t sy, int row0,
                                                                  int units) {
  // Every argument in one scalar-load batch, ahead of the index arithmetic.
  asm volatile("" ::"s"(g), "s"(sg), "s"(u), "s"(su), "s"(y), "s"(sy), "s"(row0), "s"(units));
  const int unit = blockIdx.x * kSwigluThreads + threadIdx.x;
  if (unit >= units) return;
  const int c = unit * (PAIR ? 2 : 1);
  const int row = row0 + blockIdx.y;
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
  const unsigned bx = (unsigned)((units + kSwigluThreads - 1) / kSwigluThreads);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* G = static_cast<const uint16_t*>(g);
  const uint16_t* U = static_cast<const uint16_t*>(u);
  uint16_t* Y = static_cast<uint16_t*>(y);
  for (int row0 = 0; row0 < rows; row0 += kMaxGridY) {   // one launch per 65535 rows
    const dim3 grid(bx, (unsigned)min(rows - row0, kMaxGridY));
    if (pair) hipLaunchKernelGGL(silu_mul_kernel<true>, grid, dim3(kSwigluThreads), 0, s, G, sg, U, su, Y, sy, row0, units);
    else hipLaunchKernelGGL(silu_mul_kernel<false>, grid, dim3(kSwigluThreads), 0, s, G, sg, U, su, Y, sy, row0, units);
  }
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
