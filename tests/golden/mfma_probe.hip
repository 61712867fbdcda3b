// One 16x16x32 bf16 MFMA per workgroup (one wave): D = A B + C, for the fixture
// tests/golden/mfma_16x16x32_bf16.npz.  A [16][32], B [32][16] bf16 bits row-major, C/D
// [16][16] fp32; every index stays inside problem t's 512 / 256 slots.
#include <hip/hip_runtime.h>
#include <stdint.h>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

__global__ void mfma_probe(const uint16_t* A, const uint16_t* B, const float* C, float* D) {
  const int t = blockIdx.x, l = threadIdx.x;
  const uint16_t* a = A + t * 512;
  const uint16_t* b = B + t * 512;
  u16x8 av, bv;
  for (int i = 0; i < 8; ++i) {
    av[i] = a[(l % 16) * 32 + 8 * (l / 16) + i];
    bv[i] = b[(8 * (l / 16) + i) * 16 + l % 16];
  }
  f32x4 c;
  for (int i = 0; i < 4; ++i) c[i] = C[t * 256 + (4 * (l / 16) + i) * 16 + l % 16];
  f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), c, 0, 0, 0);
  for (int i = 0; i < 4; ++i) D[t * 256 + (4 * (l / 16) + i) * 16 + l % 16] = d[i];
}

extern "C" int mfma_probe_launch(const void* A, const void* B, const void* C, void* D, int n, void* stream) {
  hipLaunchKernelGGL(mfma_probe, dim3(n), dim3(64), 0, (hipStream_t)stream, (const uint16_t*)A, (const uint16_t*)B,
                     (const float*)C, (float*)D);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
