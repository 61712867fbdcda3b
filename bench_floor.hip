// Bench-only measurement kernels for the trie-attention roofline (no
// counterpart in the reference; built into bench_floor.so next to bench.py,
// not into the product library): what a launch of the attention's 8B-shape
// grid costs before any arithmetic.  256 workgroups of 512 threads holding 147 KB of LDS each (one
// per CU, as fused_kernel<128, 2>), over K and V of 8 kv heads x 3072 keys x
// head_dim 128 bf16.  Workgroup b takes kv head b % 8, row block (b / 8) % 4
// and key group b / 32 (keys [384 q, 384 q + 384)), as the attention does.
//   0  empty: launch, dispatch and completion only;
//   1  stream: every wave issues its share of the group's K and V (196 KB per
//      workgroup; each byte read by the 4 row blocks) at once into registers;
//   2  stream, unique: row block rb reads only a quarter of the group range
//      (49 KB per workgroup; every byte read once);
//   3  ring: the attention's own load schedule -- direct-to-LDS loads of
//      64 KB rounds into a 2-round ring, a wait and a barrier per round, 3
//      rounds -- without the arithmetic.
// Every load is a raw-buffer load whose descriptor covers exactly one head of
// K (or V), so nothing outside the tensors is read; results feed a
// never-taken store so that no load is dropped.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace floor_probe {

typedef __attribute__((address_space(3))) void lds_void;
constexpr int kKeys = 3072, kHeadBytes = kKeys * 256, kLds = 147 * 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t head(const uint16_t* base, int g) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + (size_t)g * kKeys * 128), (short)0,
                                           kHeadBytes, 0x00020000);
}

__global__ __launch_bounds__(512) void empty_kernel(int* out) {
  extern __shared__ char lds[];
  if (threadIdx.x == 0 && out == nullptr) lds[0] = 1;
}

template <bool UNIQUE>
__global__ __launch_bounds__(512) void stream_kernel(const uint16_t* K, const uint16_t* V, int* out) {
  constexpr int NB = UNIQUE ? 96 * 256 : 384 * 256;   // bytes per tensor per workgroup
  constexpr int PER = NB / 8 / 1024;                   // 1 KB loads per wave per tensor
  const int b = blockIdx.x, g = b % 8, rb = (b / 8) % 4, q = b / 32;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t rk = head(K, g), rv = head(V, g);
  const int base = q * 384 * 256 + (UNIQUE ? rb * NB : 0) + w * (NB / 8) + lane * 16;
  u32x4 a[PER], c[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, base + i * 1024, 0, 0));
    c[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, base + i * 1024, 0, 0));
  }
  u32x4 x = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < PER; ++i) x ^= a[i] ^ c[i];
  if ((x[0] ^ x[1] ^ x[2] ^ x[3]) == 0x9e3779b9u && out) out[b * 512 + threadIdx.x] = 1;
}

__global__ __launch_bounds__(512) void ring_kernel(const uint16_t* K, const uint16_t* V, int* out) {
  extern __shared__ char lds[];
  const int b = blockIdx.x, g = b % 8, q = b / 32;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t rk = head(K, g), rv = head(V, g);
  const int base = q * 384 * 256 + lane * 16;
  auto issue = [&](int r, int slot) {   // round r: 128 keys of K and of V, 4 + 4 KB per wave
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = w * 4 + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(lds + slot * 65536 + c * 1024), 16,
                                               base + r * 32768 + c * 1024, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(lds + slot * 65536 + 32768 + c * 1024), 16,
                                               base + r * 32768 + c * 1024, 0, 0, 0);
    }
  };
  issue(0, 0);
  issue(1, 1);
  uint32_t x = 0;
  for (int r = 0; r < 3; ++r) {
    if (r < 2) __builtin_amdgcn_s_waitcnt(8 | 0x70 | 0xF00);   // vmcnt(8): round r has landed
    else __builtin_amdgcn_s_waitcnt(0x0F70);                   // vmcnt(0)
    __syncthreads();
    x ^= *(volatile uint32_t*)(lds + (r % 2) * 65536 + threadIdx.x * 4);
    __syncthreads();
    if (r == 0) issue(2, 0);
  }
  if (x == 0x9e3779b9u && out) out[b * 512 + threadIdx.x] = 1;
}

}  // namespace floor_probe

using namespace floor_probe;

// which: 0 empty grid, 1 stream, 2 stream with unique shares, 3 ring (above).
// K and V are [HK][P][D] bf16, contiguous; only HK 8, P 3072, D 128 (the shape
// the kernels' descriptors are built for) is accepted, so no load can leave
// the tensors.  Returns 0, or -1 for a bad argument or shape, -5 for a HIP
// error.  out: >= 256 x 512 ints (never written in practice).
extern "C" int rspx_bench_floor_launch(int which, const void* K, const void* V, int HK, int P, int D, void* out,
                                       void* stream) {
  if (which < 0 || which > 3) return -1;
  if (which > 0 && (!K || !V || HK != 8 || P != kKeys || D != 128)) return -1;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -5;
  static bool attr[64];
  if (!attr[dev]) {
    const void* fns[] = {(const void*)empty_kernel, (const void*)stream_kernel<false>, (const void*)stream_kernel<true>,
                         (const void*)ring_kernel};
    for (const void* f : fns)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess) return -5;
    attr[dev] = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* k = static_cast<const uint16_t*>(K);
  const uint16_t* v = static_cast<const uint16_t*>(V);
  int* o = static_cast<int*>(out);
  const dim3 grid(256), blk(512);
  switch (which) {
    case 0: hipLaunchKernelGGL(empty_kernel, grid, blk, kLds, s, o); break;
    case 1: hipLaunchKernelGGL(stream_kernel<false>, grid, blk, kLds, s, k, v, o); break;
    case 2: hipLaunchKernelGGL(stream_kernel<true>, grid, blk, kLds, s, k, v, o); break;
    default: hipLaunchKernelGGL(ring_kernel, grid, blk, kLds, s, k, v, o); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -5;
}
