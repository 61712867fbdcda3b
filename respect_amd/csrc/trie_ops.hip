// Device-side trie plumbing and greedy selection for gfx950.
//
//   rspx_trie_mask     node mask and depths from a parent array (replaces the
//                      host-built mask of respect/decoding/verify.py:22-41 and
//                      the padding rules of respect/kernels/dispatch.py:94-115)
//   rspx_kv_compact    moves the accepted path's KV to consecutive slots
//                      (respect/decoding/kv_buffer.py:93-104 compact), all
//                      layers and heads in one launch
//   rspx_argmax_rows   greedy token per row over fp32 logits with an excluded
//                      vocabulary range (respect/decoding/acceptance.py:11-23)
//
// All three are exact (integer / copy / compare) operations.

#include "common.h"
#include "respect_amd.h"

namespace rspx {

// Row i < N: msk[i][j] = 1 for j < base (prompt-side committed tokens) and for
// j = base + a, a an ancestor of i or i itself; 0 elsewhere.  Rows N..M-1
// (query padding) open slot 0 only, so they never see an empty key set.
// depth[i] = number of proper ancestors.  One workgroup per row.
__global__ __launch_bounds__(256) void trie_mask_kernel(const int* parent, int N, int base, int NN, uint8_t* msk,
                                                        int64_t smm, int* depth) {
  const int i = blockIdx.x;
  uint8_t* row = msk + (int64_t)i * smm;
  for (int j = threadIdx.x; j < NN; j += 256) row[j] = (i < N) ? (j < base ? 1 : 0) : (j == 0 ? 1 : 0);
  __syncthreads();
  if (i >= N || threadIdx.x != 0) return;
  int d = -1;
  for (int a = i, steps = 0; a >= 0 && a < N && steps <= N; a = parent[a], ++steps) {
    if (base + a < NN) row[base + a] = 1;
    ++d;
  }
  depth[i] = d;
}

// The row inputs of one forward from a device-side step descriptor
// desc = [n, base, tok[0..T), parent[0..T)]: row i < n gets token tok[i]
// (clamped into [0, vocab)), cache slot P + base + i, rotary position
// P + base + depth(i) and the mask row of trie_mask_kernel; rows n..T-1 get
// token 0, slot pad0 + i, position 0 and slot 0 only.  A descriptor that does
// not fit (n outside [0, T], base < 0, base + n > NN) counts as n = 0.  One
// workgroup per row.
__global__ __launch_bounds__(256) void step_inputs_kernel(const int* desc, int T, int P, int NN, int pad0, int vocab,
                                                          int* ids, int* slots, int* pos, uint8_t* msk, int64_t smm) {
  const int i = blockIdx.x;
  int n = desc[0];
  const int base = desc[1];
  if (n < 0 || n > T || base < 0 || base > NN - n) n = 0;
  const int* tok = desc + 2;
  const int* parent = desc + 2 + T;
  uint8_t* row = msk + (int64_t)i * smm;
  for (int j = threadIdx.x; j < NN; j += 256) row[j] = (i < n) ? (j < base ? 1 : 0) : (j == 0 ? 1 : 0);
  __syncthreads();
  if (threadIdx.x != 0) return;
  if (i >= n) {
    ids[i] = 0;
    slots[i] = pad0 + i;
    pos[i] = 0;
    return;
  }
  int d = -1;
  for (int a = i, steps = 0; a >= 0 && a < n && steps <= n; a = parent[a], ++steps) {
    row[base + a] = 1;
    ++d;
  }
  const int t = tok[i];
  ids[i] = (t >= 0 && t < vocab) ? t : 0;
  slots[i] = P + base + i;
  pos[i] = P + base + d;
}

// Workgroup (tensor, head): rows src[0..n) of cache tensor `tensor` (one K or
// V of one layer), head `head`, copied to rows dst0 .. dst0 + n - 1.  All
// source rows are read into registers before any row is written, so the
// move is correct however sources and destinations overlap.  A source slot
// outside [0, cap) is skipped (neither read nor written).
constexpr int kCompactMax = 128;
__global__ __launch_bounds__(256) void kv_compact_kernel(const uint64_t* bases, int64_t sh, int64_t sn, int D,
                                                         int cap, int dst0, const int* src, int n) {
  uint16_t* base = reinterpret_cast<uint16_t*>(bases[blockIdx.x]) + blockIdx.y * sh;
  const int vpr = D / 8;                       // 16-byte vectors per row
  const int total = n * vpr;
  u32x4 buf[kCompactMax * 16 / 256];           // D <= 128: at most 8 vectors per thread
#pragma unroll
  for (int k = 0; k < kCompactMax * 16 / 256; ++k) {
    const int idx = threadIdx.x + 256 * k;
    if (idx < total) {
      const int j = idx / vpr, c = idx - j * vpr;
      const int sj = src[j];
      if (sj >= 0 && sj < cap) buf[k] = *reinterpret_cast<const u32x4*>(base + (int64_t)sj * sn + 8 * c);
    }
  }
  __syncthreads();  // every source row of this (tensor, head) has been read
#pragma unroll
  for (int k = 0; k < kCompactMax * 16 / 256; ++k) {
    const int idx = threadIdx.x + 256 * k;
    if (idx < total) {
      const int j = idx / vpr, c = idx - j * vpr;
      const int sj = src[j];
      if (sj >= 0 && sj < cap) *reinterpret_cast<u32x4*>(base + (int64_t)(dst0 + j) * sn + 8 * c) = buf[k];
    }
  }
}

// Greedy token of a row: index of the maximum of the logits with columns
// [off, off + size) replaced by -inf; NaN counts as the largest value; ties go
// to the lowest index.  That is a total order on (value, index), so the result
// does not depend on the reduction order (two passes: 4096-logit chunks, then
// the chunk winners).
__device__ __forceinline__ bool better(float v, int j, float bv, int bj) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || j < bj);
  return v > bv || (v == bv && j < bj);
}

constexpr int kArgChunk = 4096;  // logits per workgroup of the first pass

// Pass 1, workgroup (row, chunk): the best (value, index) of logits
// [chunk * 4096, +4096) of the row; 16 per thread from four 16-byte loads
// issued together.
__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float* logits, int64_t sl, int V, int off, int size,
                                                           float* pv, int* pj) {
  __shared__ float sv[4];
  __shared__ int sj[4];
  const int row = blockIdx.x, c = blockIdx.y, C = gridDim.y;
  const float* lr = logits + (int64_t)row * sl;
  float bv = kNegInf;
  int bj = 0x7fffffff;
  f32x4 v4[4];
  int j0[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    j0[i] = c * kArgChunk + 4 * (threadIdx.x + 256 * i);
    if (j0[i] + 3 < V) v4[i] = *reinterpret_cast<const f32x4*>(lr + j0[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = j0[i] + e;
      if (j < V) {
        float v = (j0[i] + 3 < V) ? v4[i][e] : lr[j];
        if (j >= off && j < off + size) v = kNegInf;
        if (better(v, j, bv, bj)) { bv = v; bj = j; }
      }
    }
  }
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m);
    const int oj = __shfl_xor(bj, m);
    if (better(ov, oj, bv, bj)) { bv = ov; bj = oj; }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[w] = bv; sj[w] = bj; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k)
      if (better(sv[k], sj[k], bv, bj)) { bv = sv[k]; bj = sj[k]; }
    pv[row * C + c] = bv;
    pj[row * C + c] = bj;
  }
}

// Pass 2, one wave per row: the best of the row's chunk results.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* pv, const int* pj, int C, int64_t* out) {
  const int row = blockIdx.x;
  float bv = kNegInf;
  int bj = 0x7fffffff;
  for (int c = threadIdx.x; c < C; c += 64)
    if (better(pv[row * C + c], pj[row * C + c], bv, bj)) { bv = pv[row * C + c]; bj = pj[row * C + c]; }
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m);
    const int oj = __shfl_xor(bj, m);
    if (better(ov, oj, bv, bj)) { bv = ov; bj = oj; }
  }
  if (threadIdx.x == 0) out[row] = bj == 0x7fffffff ? 0 : bj;
}

}  // namespace rspx

using namespace rspx;

extern "C" int rspx_trie_mask(const int32_t* parent, int N, int base, int M, int NN, uint8_t* msk, int64_t smm,
                              int32_t* depth, void* stream) {
  if (N < 0 || base < 0 || M < N || NN < 1 || base + N > NN || smm < NN) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!msk || (N > 0 && (!parent || !depth))) return RSPX_EINVAL;
  hipLaunchKernelGGL(trie_mask_kernel, dim3(M), dim3(256), 0, static_cast<hipStream_t>(stream), parent, N, base, NN,
                     msk, smm, depth);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_step_inputs(const int32_t* desc, int T, int P, int NN, int pad0, int vocab, int32_t* ids,
                                int32_t* slots, int32_t* pos, uint8_t* msk, int64_t smm, void* stream) {
  if (T < 0 || P < 0 || NN < 1 || pad0 < 0 || vocab < 1 || smm < NN) return RSPX_EINVAL;
  if ((int64_t)P + NN > INT32_MAX || (int64_t)pad0 + T > INT32_MAX) return RSPX_EINVAL;
  if (T == 0) return RSPX_OK;
  if (!desc || !ids || !slots || !pos || !msk) return RSPX_EINVAL;
  hipLaunchKernelGGL(step_inputs_kernel, dim3(T), dim3(256), 0, static_cast<hipStream_t>(stream), desc, T, P, NN,
                     pad0, vocab, ids, slots, pos, msk, smm);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_kv_compact(const uint64_t* bases, int n_tensors, int HK, int D, int64_t sh, int64_t sn, int cap,
                               int dst0, const int32_t* src, int n, void* stream) {
  if (n_tensors < 0 || HK <= 0 || n < 0 || dst0 < 0 || dst0 + n > cap) return RSPX_EINVAL;
  if (D % 8 != 0 || D > 128) return RSPX_EUNSUPPORTED;
  if (n > kCompactMax) return RSPX_EUNSUPPORTED;
  if (n == 0 || n_tensors == 0) return RSPX_OK;
  if (!bases || !src) return RSPX_EINVAL;
  if (sh % 8 || sn % 8) return RSPX_EALIGN;
  hipLaunchKernelGGL(kv_compact_kernel, dim3(n_tensors, HK), dim3(256), 0, static_cast<hipStream_t>(stream), bases, sh,
                     sn, D, cap, dst0, src, n);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int64_t rspx_argmax_workspace_bytes(int M, int V) {
  if (M < 0 || V <= 0) return -1;
  return (int64_t)M * ((V + kArgChunk - 1) / kArgChunk) * 8;
}

extern "C" int rspx_argmax_rows(const float* logits, int64_t sl, int M, int V, int off, int size, int64_t* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || V <= 0 || sl < V || off < 0 || size < 0) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!logits || !out) return RSPX_EINVAL;
  if ((reinterpret_cast<uintptr_t>(logits) & 15u) || sl % 4) return RSPX_EALIGN;
  const int C = (V + kArgChunk - 1) / kArgChunk;
  if (!workspace || workspace_bytes < (int64_t)M * C * 8) return RSPX_EWORKSPACE;
  float* pv = static_cast<float*>(workspace);
  int* pj = reinterpret_cast<int*>(pv + (int64_t)M * C);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(argmax_chunk_kernel, dim3(M, C), dim3(256), 0, s, logits, sl, V, off, size, pv, pj);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(M), dim3(64), 0, s, pv, pj, C, out);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
