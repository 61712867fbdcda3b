// The tile-wise ("blocked") trie attention -- the negative control of the
// slot-layout experiment, replacing the development kernel _fused_attn /
// fused_attn of respect/kernels/reference_blocked.py:14-106.
//
// Semantics per (head, query row), as the reference: prompt keys in tiles of
// BN keys (never masked), then node slots in tiles of BN slots (masked by
// msk); per tile one online-softmax update at the tile's row maximum --
// acc = acc * alpha + bf16(p) . V, l = l * alpha + sum(p) -- and
// out = bf16(acc / l).  Because a whole tile of node slots is reduced at once,
// the pairing of partial sums follows where the slots sit, so placing the
// same ancestors in other slots can change the result: this kernel exists to
// show that the trie kernel (trie_attn.hip) does not have that dependence.
// A row whose every key so far is masked keeps acc = l = 0 (alpha = 1, p = 0)
// instead of the NaN the reference would form.
//
// MI355X form: one wave per workgroup, 16 query rows of one head.  A tile's K
// and V go through LDS (row-major [key][D] bf16); S^T = K Q^T by
// v_mfma_f32_16x16x32_bf16 chains over head_dim; the softmax state of row n16
// sits in lanes n16 + 16 g4; O^T += V^T bf16(P)^T with P used in place as the
// B operand (k-slot 8 g4 + i <-> key 4 g4 + i for i < 4, 16 + 4 g4 + i - 4
// otherwise, within each 32-key half of the tile) and V^T gathered from LDS.
// Base-2 exponent with the scale folded into log2(e).
#include "common.h"
#include "respect_amd.h"

namespace rspx {
namespace blocked {

struct Args {
  const uint16_t* q;  int64_t sqh, sqm;
  const uint16_t* kp; int64_t skph, skpn;
  const uint16_t* vp; int64_t svph, svpn;
  const uint16_t* kn; int64_t sknh, sknn;
  const uint16_t* vn; int64_t svnh, svnn;
  const uint8_t* msk; int64_t smm, smn;
  uint16_t* out;      int64_t soh, som;
  int H, HK, M, P, NN;
  float c;   // sm_scale * log2(e)
};

__device__ __forceinline__ float rows4_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  const float s = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_int(s), __float_as_int(s), false, false);
  return fmaxf(__int_as_float(t[0]), __int_as_float(t[1]));
}
__device__ __forceinline__ float rows4_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  const float s = __int_as_float(r[0]) + __int_as_float(r[1]);
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_int(s), __float_as_int(s), false, false);
  return __int_as_float(t[0]) + __int_as_float(t[1]);
}

typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

template <int D, int BN>
__global__ __launch_bounds__(64) void blocked_kernel(Args A) {
  constexpr int DQ = D / 32, DT = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t kt[BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t vt[BN * D];
  const int lane = __lane_id();
  const int n16 = lane & 15, g4 = lane >> 4;
  const int h = blockIdx.y, g = h / (A.H / A.HK);
  const int m0 = 16 * blockIdx.x;
  const int mrow = m0 + n16 < A.M ? m0 + n16 : m0;   // rows past M shadow row m0, never stored

  bf16x8 qop[DQ];
  const uint16_t* qr = A.q + h * A.sqh + mrow * A.sqm + 8 * g4;
#pragma unroll
  for (int i = 0; i < DQ; ++i) qop[i] = *reinterpret_cast<const bf16x8*>(qr + 32 * i);

  float m = kNegInf, l = 0.f;
  f32x4 acc[DT];
#pragma unroll
  for (int j = 0; j < DT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ntp = (A.P + BN - 1) / BN, ntn = (A.NN + BN - 1) / BN;
  for (int tile = 0; tile < ntp + ntn; ++tile) {
    const bool node = tile >= ntp;
    const int t0 = (node ? tile - ntp : tile) * BN;     // first key / slot of the tile
    const int lim = node ? A.NN : A.P;
    const uint16_t* kb = node ? A.kn + g * A.sknh : A.kp + g * A.skph;
    const uint16_t* vb = node ? A.vn + g * A.svnh : A.vp + g * A.svph;
    const int64_t sk = node ? A.sknn : A.skpn, sv = node ? A.svnn : A.svpn;
    // The tile's K and V rows into LDS, 16 bytes per lane per load; rows past the
    // segment are zeros.
    __syncthreads();
    for (int u = lane; u < BN * (D / 8); u += 64) {
      const int key = u / (D / 8), part = u % (D / 8);
      u32x4 kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
      if (t0 + key < lim) {
        kv = *reinterpret_cast<const u32x4*>(kb + (t0 + key) * sk + 8 * part);
        vv = *reinterpret_cast<const u32x4*>(vb + (t0 + key) * sv + 8 * part);
      }
      *(lds_u32x4*)((lds_u16*)kt + key * D + 8 * part) = kv;
      *(lds_u32x4*)((lds_u16*)vt + key * D + 8 * part) = vv;
    }
    __syncthreads();

    // Scores: lane (n16, g4) holds row n16, keys 16 b + 4 g4 + e of the tile.
    float s[BN / 16][4];
    float tm = kNegInf;
#pragma unroll
    for (int b = 0; b < BN / 16; ++b) {
      f32x4 sv4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < DQ; ++i) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, *(const lds_u32x4*)((lds_u16*)kt + (16 * b + n16) * D + 32 * i + 8 * g4));
        sv4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qop[i], sv4, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = t0 + 16 * b + 4 * g4 + e;
        bool ok = key < lim;
        if (node && ok) ok = A.msk[mrow * A.smm + key * A.smn] != 0;
        s[b][e] = ok ? sv4[e] * A.c : kNegInf;
        tm = fmaxf(tm, s[b][e]);
      }
    }
    tm = rows4_max(tm);
    const float mn = fmaxf(m, tm);
    const float alpha = mn == kNegInf ? 1.f : fexp2(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int b = 0; b < BN / 16; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[b][e] = s[b][e] == kNegInf ? 0.f : fexp2(s[b][e] - mn);
        ps = ps + s[b][e];
      }
    l = l * alpha + rows4_sum(ps);
    m = mn;
#pragma unroll
    for (int j = 0; j < DT; ++j) acc[j] = acc[j] * alpha;
    // O^T += V^T bf16(P)^T over each 32-key half of the tile.
#pragma unroll
    for (int hh = 0; hh < BN / 32; ++hh) {
      u32x4 pw;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        pw[i] = pack_bf16x2(s[2 * hh][2 * i], s[2 * hh][2 * i + 1]);
        pw[2 + i] = pack_bf16x2(s[2 * hh + 1][2 * i], s[2 * hh + 1][2 * i + 1]);
      }
      const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        uint16_t vv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int key = 32 * hh + (i < 4 ? 4 * g4 + i : 16 + 4 * g4 + (i - 4));
          vv[i] = ((lds_u16*)vt)[key * D + 16 * j + n16];
        }
        u32x4 vw;
#pragma unroll
        for (int i = 0; i < 4; ++i) vw[i] = uint32_t(vv[2 * i]) | (uint32_t(vv[2 * i + 1]) << 16);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vw), pop, acc[j], 0, 0, 0);
      }
    }
  }
  if (m0 + n16 < A.M) {
    uint16_t* o = A.out + h * A.soh + (m0 + n16) * A.som + 4 * g4;
#pragma unroll
    for (int j = 0; j < DT; ++j) {
      uint32_t w2[2];
      w2[0] = pack_bf16x2(acc[j][0] / l, acc[j][1] / l);
      w2[1] = pack_bf16x2(acc[j][2] / l, acc[j][3] / l);
      *reinterpret_cast<u32x2*>(o + 16 * j) = u32x2{w2[0], w2[1]};
    }
  }
}

}  // namespace blocked
}  // namespace rspx

using namespace rspx;

extern "C" int rspx_blocked_attn(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                                 const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh,
                                 int64_t sknn, const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk,
                                 int64_t smm, int64_t smn, void* out, int64_t soh, int64_t som, int H, int HK, int M,
                                 int P, int NN, int D, int BN, float sm_scale, void* stream) {
  if (H <= 0 || HK <= 0 || H % HK || M < 0 || P < 0 || NN < 0) return RSPX_EINVAL;
  if (D != 32 && D != 64 && D != 128 && D != 256) return RSPX_EUNSUPPORTED;
  if (BN != 32 && BN != 64 && BN != 128) return RSPX_EUNSUPPORTED;
  if (!(sm_scale > 0.f) || sm_scale == __builtin_huge_valf()) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!q || !out || (P > 0 && (!kp || !vp)) || (NN > 0 && (!kn || !vn || !msk))) return RSPX_EINVAL;
  const void* ptrs[] = {q, kp, vp, kn, vn};
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15u)) return RSPX_EALIGN;
  if (reinterpret_cast<uintptr_t>(out) & 7u) return RSPX_EALIGN;
  const int64_t strides[] = {sqh, sqm, skph, skpn, svph, svpn, sknh, sknn, svnh, svnn, soh, som};
  for (int64_t s : strides) {
    if (s < 0) return RSPX_EINVAL;
    if (s % 8) return RSPX_EALIGN;
  }
  if (smm < 0 || smn < 0) return RSPX_EINVAL;
  blocked::Args a;
  a.q = static_cast<const uint16_t*>(q);   a.sqh = sqh;   a.sqm = sqm;
  a.kp = static_cast<const uint16_t*>(kp); a.skph = skph; a.skpn = skpn;
  a.vp = static_cast<const uint16_t*>(vp); a.svph = svph; a.svpn = svpn;
  a.kn = static_cast<const uint16_t*>(kn); a.sknh = sknh; a.sknn = sknn;
  a.vn = static_cast<const uint16_t*>(vn); a.svnh = svnh; a.svnn = svnn;
  a.msk = msk; a.smm = smm; a.smn = smn;
  a.out = static_cast<uint16_t*>(out); a.soh = soh; a.som = som;
  a.H = H; a.HK = HK; a.M = M; a.P = P; a.NN = NN;
  a.c = (float)((double)sm_scale * 1.4426950408889634);
  const dim3 grid((M + 15) / 16, H);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define RSPX_BLOCKED(DD, BB) hipLaunchKernelGGL((blocked::blocked_kernel<DD, BB>), grid, dim3(64), 0, s, a)
#define RSPX_BLOCKED_BN(DD)             \
  if (BN == 32) RSPX_BLOCKED(DD, 32);    \
  else if (BN == 64) RSPX_BLOCKED(DD, 64); \
  else RSPX_BLOCKED(DD, 128);
  if (D == 128) { RSPX_BLOCKED_BN(128) }
  else if (D == 64) { RSPX_BLOCKED_BN(64) }
  else if (D == 32) { RSPX_BLOCKED_BN(32) }
  else { RSPX_BLOCKED_BN(256) }
#undef RSPX_BLOCKED_BN
#undef RSPX_BLOCKED
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
