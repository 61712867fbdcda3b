// Trie-verification attention for gfx950 (MI355X).
//
// Replaces the Triton kernel _attn_hyb / fused_attn_hyb of
// respect/kernels/attention.py:15-96.  Semantics per (head, query row):
// softmax(q . k * scale) . v over the P prompt keys (never masked) and over
// the node slots the row's mask allows, fp32 accumulation, bf16 output.
//
// Reduction tree, fixed by P and by the row's allowed node slots only:
//
//   step   32 prompt keys.  Scores from bf16 MFMA 16x16x32 (fp32 accumulate,
//          head_dim reduced by a fixed chain of MFMAs), base-2 exponent with
//          the scale folded into log2(e).  Probabilities are rounded to bf16
//          before the PV MFMA, as the reference rounds p before tl.dot
//          (attention.py:48).
//   group  RL consecutive prompt keys (a whole number of steps; NG <= 16
//          groups), online softmax over its steps in key order.  The running
//          reference maximum of a row is moved only when a step's maximum
//          exceeds it by more than 2^8 (then the accumulator is rescaled);
//          otherwise probabilities are taken against the old reference and may
//          reach 2^8.  The rule looks at the row's own scores only.
//   final  the NG groups left to right, then the node partial.
//   node   the row's allowed node slots, one at a time in slot order, fp32
//          probabilities (the reference's node loop, attention.py:52-67).
//          Masked slots are skipped; in the reference they are exact no-ops,
//          so only the sequence of allowed slots matters.
//
// RL and NG depend on P only.  Which wavefront computes what changes with the
// number of rows, never the arithmetic of a row, so a row's bits are the same
// whether it is verified alone (1-token decoding) or inside a 128-node trie,
// and wherever its allowed slots sit in the node segment.
//
// Two launches on the caller's stream, no host synchronisation:
//   A  prompt_kernel: workgroup = (kv head g, 64 or 128 GQA rows, group).
//      The four waves issue the group's K/V straight from HBM into an LDS ring
//      (global_load_lds, up to 8 steps in flight, no registers held), laid
//      out so that each lane's MFMA fragment is one conflict-free ds_read;
//      then each wave consumes the steps for its 16 or 32 rows (V transposed
//      in registers for the PV B operand) and stores its group partials.
//   B  node_merge_kernel: one wave per (query row, head).  It lists the
//      allowed node slots (ballot + mbcnt), folds them in order (dot products
//      reduced with DPP / permlane butterflies), combines the group partials
//      of kernel A in group order and the node partial last, writes bf16.
//   Rows are packed GQA-wise (row = query * GQA + head-in-group), so a kv
//   head's K/V is read once for all query heads that share it.  With 8 kv
//   heads, workgroup g of either kernel lands on XCD g (round-robin dispatch),
//   so a head's K/V and partials stay in one XCD's L2.

#include "common.h"
#include "respect_amd.h"

namespace rspx {

constexpr int kNGTarget = 16;   // maximum number of key groups per kv head
constexpr int kStep = 32;       // keys per online-softmax step
constexpr float kLazyTau = 8.f; // log2 headroom before the reference max moves
constexpr int kMaxNodeSlots = 4096;

struct TrieAttnArgs {
  const uint16_t* q;  int64_t sqh, sqm;
  const uint16_t* kp; int64_t skph, skpn;
  const uint16_t* vp; int64_t svph, svpn;
  const uint16_t* kn; int64_t sknh, sknn;
  const uint16_t* vn; int64_t svnh, svnn;
  const uint8_t* msk; int64_t smm, smn;
  uint16_t* out;      int64_t soh, som;
  int HK, GQA, M, P, NN;
  int R, NT, NG, RL;
  float c;        // sm_scale * log2(e)
  float* gp_ml;   // [HK][R][NG][2]  group partial (m, l)
  float* gp_acc;  // [HK][R][NG][D]
};

template <int D> struct VRow;
template <> struct VRow<128> { typedef u32x4 T; };
template <> struct VRow<64> { typedef u32x2 T; };

// state (m, l, acc) <- state (+) incoming.  An incoming partial with m = -inf
// is empty and left out (it would be an exact no-op).  From the empty state
// (-inf, 0, 0) the first combine reproduces the incoming partial exactly.
template <int N>
__device__ __forceinline__ void combine(float& m, float& l, float* acc, float m2, float l2,
                                        const float* acc2) {
  if (m2 == kNegInf) return;
  const float mn = fmaxf(m, m2);
  const float a = fexp2(m - mn);
  const float b = fexp2(m2 - mn);
  l = __builtin_fmaf(l2, b, l * a);
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = __builtin_fmaf(acc2[i], b, acc[i] * a);
  m = mn;
}

// Sum / max over the four 16-lane rows of a wave, the same operand order in
// every lane: v_permlane16_swap pairs rows (0,1) and (2,3), then
// v_permlane32_swap pairs the halves.
__device__ __forceinline__ float rows4_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  const float s = __int_as_float(r[0]) + __int_as_float(r[1]);
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_int(s), __float_as_int(s), false, false);
  return __int_as_float(t[0]) + __int_as_float(t[1]);
}
__device__ __forceinline__ float rows4_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  const float s = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
  auto t = __builtin_amdgcn_permlane32_swap(__float_as_int(s), __float_as_int(s), false, false);
  return fmaxf(__int_as_float(t[0]), __int_as_float(t[1]));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of L consecutive lanes; every lane of a group gets
// bitwise the same value (each butterfly level adds the same two operands).
template <int L>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (L >= 2) x = x + dpp<0xB1>(x);    // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (L >= 4) x = x + dpp<0x4E>(x);    // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (L >= 8) x = x + dpp<0x141>(x);   // row_half_mirror: quads of an 8-lane half
  if constexpr (L >= 16) x = x + dpp<0x140>(x);  // row_mirror: halves of a 16-lane row
  if constexpr (L >= 32) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
    x = __int_as_float(r[0]) + __int_as_float(r[1]);
  }
  if constexpr (L >= 64) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    x = __int_as_float(r[0]) + __int_as_float(r[1]);
  }
  return x;
}

// Load n bf16 values (n in {1,2,4,8,16,32}) starting at p and widen to fp32.
template <int N>
__device__ __forceinline__ void load_row_f32(const uint16_t* p, float* dst) {
  if constexpr (N == 1) {
    dst[0] = bf16_to_f32(*p);
  } else if constexpr (N == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    dst[0] = bf16_lo(w); dst[1] = bf16_hi(w);
  } else if constexpr (N == 4) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) { dst[2 * i] = bf16_lo(w[i]); dst[2 * i + 1] = bf16_hi(w[i]); }
  } else {
#pragma unroll
    for (int c = 0; c < N / 8; ++c) {
      const u32x4 w = reinterpret_cast<const u32x4*>(p)[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) { dst[8 * c + 2 * i] = bf16_lo(w[i]); dst[8 * c + 2 * i + 1] = bf16_hi(w[i]); }
    }
  }
}

// Geometry of one 32-key step of K/V in LDS.  A step is cut into 1 KB (or
// 256 B) chunks, one per wave-wide direct-to-LDS load: lane l's bytes land at
// chunk base + l * lane_bytes, which is exactly the MFMA fragment lane l reads
// back with one conflict-free ds_read.
template <int D>
struct StepGeom {
  static constexpr int DQ = D / 32;              // QK k-steps over head_dim
  static constexpr int DPL = D / 16;             // PV MFMAs per step
  static constexpr int KCH = 2 * DQ;             // K chunks: (key block, k-step), 16 B per lane
  static constexpr int VB = 2 * DPL;             // V bytes per lane per PV k-slot (16 or 8)
  static constexpr int VS = VB == 16 ? 16 : 4;   // bytes per lane of one V load (DMA sizes: 4, 12, 16)
  static constexpr int VPER = VB / VS;           // V loads per PV k-slot
  static constexpr int VCH = 8 * VPER;           // V chunks
  static constexpr int KBYTES = KCH * 1024;
  static constexpr int SLOT = KBYTES + VCH * 64 * VS;
  static constexpr int CH = KCH + VCH;           // chunks (= loads) per step
};

constexpr int kWaves = 4;     // waves per prompt workgroup
constexpr int kRing = 7;      // LDS ring slots (steps in flight)

__device__ __forceinline__ void wait_vm(int n) {
  // s_waitcnt vmcnt(n); the count must be an immediate, hence the switch.
#define RSPX_VM(v) __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | 0x70 | 0xF00)
  switch (n) {
    case 0: RSPX_VM(0); break;
    case 1: RSPX_VM(1); break;
    case 2: RSPX_VM(2); break;
    case 3: RSPX_VM(3); break;
    case 4: RSPX_VM(4); break;
    case 5: RSPX_VM(5); break;
    case 6: RSPX_VM(6); break;
    case 7: RSPX_VM(7); break;
    case 8: RSPX_VM(8); break;
    case 9: RSPX_VM(9); break;
    case 10: RSPX_VM(10); break;
    case 11: RSPX_VM(11); break;
    case 12: RSPX_VM(12); break;
    case 13: RSPX_VM(13); break;
    case 14: RSPX_VM(14); break;
    case 15: RSPX_VM(15); break;
    case 16: RSPX_VM(16); break;
    case 17: RSPX_VM(17); break;
    case 18: RSPX_VM(18); break;
    case 19: RSPX_VM(19); break;
    case 20: RSPX_VM(20); break;
    case 21: RSPX_VM(21); break;
    case 22: RSPX_VM(22); break;
    case 23: RSPX_VM(23); break;
    case 24: RSPX_VM(24); break;
    case 25: RSPX_VM(25); break;
    case 26: RSPX_VM(26); break;
    case 27: RSPX_VM(27); break;
    case 28: RSPX_VM(28); break;
    case 29: RSPX_VM(29); break;
    case 30: RSPX_VM(30); break;
    case 31: RSPX_VM(31); break;
    case 32: RSPX_VM(32); break;
    case 33: RSPX_VM(33); break;
    case 34: RSPX_VM(34); break;
    case 35: RSPX_VM(35); break;
    case 36: RSPX_VM(36); break;
    case 37: RSPX_VM(37); break;
    case 38: RSPX_VM(38); break;
    case 39: RSPX_VM(39); break;
    case 40: RSPX_VM(40); break;
    case 41: RSPX_VM(41); break;
    case 42: RSPX_VM(42); break;
    case 43: RSPX_VM(43); break;
    case 44: RSPX_VM(44); break;
    case 45: RSPX_VM(45); break;
    case 46: RSPX_VM(46); break;
    case 47: RSPX_VM(47); break;
    case 48: RSPX_VM(48); break;
    case 49: RSPX_VM(49); break;
    case 50: RSPX_VM(50); break;
    case 51: RSPX_VM(51); break;
    case 52: RSPX_VM(52); break;
    case 53: RSPX_VM(53); break;
    case 54: RSPX_VM(54); break;
    case 55: RSPX_VM(55); break;
    case 56: RSPX_VM(56); break;
    case 57: RSPX_VM(57); break;
    case 58: RSPX_VM(58); break;
    case 59: RSPX_VM(59); break;
    case 60: RSPX_VM(60); break;
    case 61: RSPX_VM(61); break;
    case 62: RSPX_VM(62); break;
    case 63: RSPX_VM(63); break;
    default: RSPX_VM(0); break;
  }
#undef RSPX_VM
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

// Direct-to-LDS loads: lane l's bytes land at dst + l * size.  Non-template
// wrappers: the host compilation pass rejects these builtins inside templates.
__device__ __forceinline__ void dma16(const void* src, lds_char* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
}
// Raw buffer variant: byte offset `voff` from the descriptor base; reads past
// the descriptor's size return zeros.
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, int voff, lds_char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void bdma4(__amdgpu_buffer_rsrc_t r, int voff, lds_char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 4, voff, 0, 0, 0);
}
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw-buffer descriptor dword 3
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, kBufWord3);
}

// This wave's share of the chunks of one step into the ring slot at `dst`.
// The descriptors start at the step's first key and end at key P, so keys past
// P read zeros.  Chunk j of wave w is c = w + 4 j: K chunk (kb, i) gives lane
// (n16, g4) K[key 16 kb + n16][32 i + 8 g4, +8); V chunk ii (VPER parts) gives
// V[key(ii)][DPL n16, +DPL), key(ii) = 4 g4 + ii (ii < 4) or 12 + 4 g4 + ii.
// voff[j] holds the lane's byte offset of chunk j within a step.
template <int D>
__device__ __forceinline__ void issue_step(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                           const int* voff, lds_char* dst, int w) {
  using G = StepGeom<D>;
  constexpr int L = G::CH / kWaves;
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int c = w + j * kWaves;
    if (c < G::KCH) {
      bdma16(rk, voff[j], dst + c * 1024);
    } else {
      const int vc = c - G::KCH;
      if constexpr (G::VS == 16) bdma16(rv, voff[j], dst + G::KBYTES + vc * 1024);
      else bdma4(rv, voff[j], dst + G::KBYTES + vc * 256);
    }
  }
}

// ------------------------------------------------------------------ kernel A
// Workgroup (g, rb, q): kv head g, rows [64 kRT rb, +64 kRT) (4 waves x kRT
// 16-row tiles), key group q = steps [q NS, q NS + NS).  Every wave issues its share
// of the group's K/V chunks straight into an LDS ring (up to 8 steps in
// flight, no registers held), then all waves consume the steps in order.
template <int D, int kRT>
__global__ __launch_bounds__(256) void prompt_kernel(TrieAttnArgs A) {
  using G = StepGeom<D>;
  constexpr int DQ = G::DQ, DPL = G::DPL;
  static_assert(G::CH % kWaves == 0, "chunks must split evenly over the waves");
  __shared__ __attribute__((aligned(16))) char ring[kRing * G::SLOT + kWaves * kRT * DQ * 1024];

  const int lane = __lane_id();
  const int w = threadIdx.x >> 6;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int g = blockIdx.x % A.HK;
  const int rest = blockIdx.x / A.HK;
  const int q = rest % A.NG;
  const int t0 = (rest / A.NG) * (kWaves * kRT) + w * kRT;   // this wave's first tile
  const int P = A.P;
  const int kbeg = q * A.RL;
  const int ns = min(A.RL, P - kbeg + kStep - 1) / kStep;      // steps with >= 1 valid key
  const bool has_rows = 16 * t0 < A.R;

  // Q^T fragments (B operand of S^T = K Q^T): row n16 of each tile, head_dim
  // [32 i + 8 g4, +8).  They travel through LDS like K/V (issued before the
  // K/V ring, so the step-0 wait covers them).  Rows past R read row 0 and
  // are never stored.
  lds_char* qreg = (lds_char*)ring + kRing * G::SLOT + w * (kRT * DQ * 1024);
#pragma unroll
  for (int t = 0; t < kRT; ++t) {
    const int r = 16 * (t0 + t) + n16;
    const int rc = r < A.R ? r : 0;
    const int mq = rc / A.GQA, jh = rc - mq * A.GQA;
    const uint16_t* base = A.q + (g * A.GQA + jh) * A.sqh + (int64_t)mq * A.sqm + 8 * g4;
#pragma unroll
    for (int i = 0; i < DQ; ++i)
      dma16(base + 32 * i, qreg + (t * DQ + i) * 1024);
  }
  bf16x8 qop[kRT][DQ];

  const uint16_t* kpg = A.kp + g * A.skph;
  const uint16_t* vpg = A.vp + g * A.svph;
  lds_char* ringp = (lds_char*)ring;
  constexpr int L = G::CH / kWaves;
  int voff[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int c = w + j * kWaves;
    if (c < G::KCH) {
      const int kb = c / DQ, i = c - kb * DQ;
      voff[j] = 2 * ((16 * kb + n16) * (int)A.skpn + 32 * i + 8 * g4);
    } else {
      const int vc = c - G::KCH;
      const int ii = vc / G::VPER, part = vc - ii * G::VPER;
      const int key = ii < 4 ? 4 * g4 + ii : 12 + 4 * g4 + ii;
      voff[j] = 2 * (key * (int)A.svpn + DPL * n16) + part * G::VS;
    }
  }
  // Descriptors covering keys [ks, P) of this kv head.
#define RSPX_RK(ks) buffer_rsrc(kpg + (int64_t)(ks) * A.skpn, 2 * ((int64_t)(P - (ks) - 1) * A.skpn + D))
#define RSPX_RV(ks) buffer_rsrc(vpg + (int64_t)(ks) * A.svpn, 2 * ((int64_t)(P - (ks) - 1) * A.svpn + D))

  float mref[kRT], lrow[kRT];
  f32x4 acc[kRT][DPL];
#pragma unroll
  for (int t = 0; t < kRT; ++t) {
    mref[t] = kNegInf;
    lrow[t] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int pro = min(ns, kRing);
  for (int s = 0; s < pro; ++s)
    issue_step<D>(RSPX_RK(kbeg + s * kStep), RSPX_RV(kbeg + s * kStep), voff, ringp + s * G::SLOT, w);
  // The Q chunks were issued first, so they are done once at most the K/V
  // chunks are outstanding; each wave reads only its own Q region.
  wait_vm(L * pro);
  if (has_rows) {
#pragma unroll
    for (int t = 0; t < kRT; ++t)
#pragma unroll
      for (int i = 0; i < DQ; ++i)
        qop[t][i] = __builtin_bit_cast(
            bf16x8, *(const __attribute__((address_space(3))) u32x4*)(qreg + (t * DQ + i) * 1024 + 16 * lane));
  }

  for (int s = 0; s < ns; ++s) {
    // Own chunks of step s have landed: allow the later steps already issued.
    const int hi = s == 0 ? pro - 1 : min(ns - 1, s + kRing - 2);
    wait_vm(L * (hi - s));
    // Every wave's chunks of step s are in LDS and step s-1 is consumed.  A raw
    // s_barrier: __syncthreads() would also wait for every LDS DMA in flight.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of step s-1 are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s >= 1 && s + kRing - 1 < ns) {
      const int kn = kbeg + (s + kRing - 1) * kStep;
      issue_step<D>(RSPX_RK(kn), RSPX_RV(kn), voff, ringp + ((s - 1) % kRing) * G::SLOT, w);
    }
    if (!has_rows) continue;

    const lds_char* slot = ringp + (s % kRing) * G::SLOT;
    const int ks = kbeg + s * kStep;
    u32x4 kf[2][DQ];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < DQ; ++i)
        kf[kb][i] = *(const __attribute__((address_space(3))) u32x4*)(slot + (kb * DQ + i) * 1024 + 16 * lane);
    typename VRow<D>::T vf[8];
#pragma unroll
    for (int ii = 0; ii < 8; ++ii) {
      if constexpr (G::VPER == 1) {
        vf[ii] = *(const __attribute__((address_space(3))) typename VRow<D>::T*)(
            slot + G::KBYTES + ii * 1024 + 16 * lane);
      } else {
#pragma unroll
        for (int part = 0; part < G::VPER; ++part)
          vf[ii][part] = *(const __attribute__((address_space(3))) uint32_t*)(
              slot + G::KBYTES + (ii * G::VPER + part) * 256 + 4 * lane);
      }
    }

    // S^T = K Q^T for two blocks of 16 keys.
    f32x4 sc[kRT][2];
#pragma unroll
    for (int t = 0; t < kRT; ++t)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[kb][i]), qop[t][i], sv,
                                                       0, 0, 0);
        sc[t][kb] = sv;
      }

    // Lane (n16, g4) holds row n16, keys 16 kb + 4 g4 + e of the step.  Raw
    // scores; keys past P (only in a group's last step) are masked to -inf.
    // Since scale > 0, max(s) * c is exactly the max of the scaled scores.
    bf16x8 pop[kRT];
    float mx[kRT];
    float s8[kRT][8];
    bool any_move = false;
    const bool full = ks + kStep <= P;
#pragma unroll
    for (int t = 0; t < kRT; ++t) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) s8[t][4 * kb + e] = sc[t][kb][e];
      if (!full) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (ks + 16 * kb + 4 * g4 + e >= P) s8[t][4 * kb + e] = kNegInf;
      }
      float m8 = s8[t][0];
#pragma unroll
      for (int i = 1; i < 8; ++i) m8 = fmaxf(m8, s8[t][i]);
      mx[t] = rows4_max(m8) * A.c;
      any_move |= mx[t] > mref[t] + kLazyTau;
    }
    // Move the reference maximum of rows that outgrew it (wave-uniform branch;
    // rows that did not move get alpha = 2^0 = 1 exactly).
    if (__builtin_amdgcn_ballot_w64(any_move) != 0) {
#pragma unroll
      for (int t = 0; t < kRT; ++t) {
        const float mn = mx[t] > mref[t] + kLazyTau ? mx[t] : mref[t];
        const float alpha = fexp2(mref[t] - mn);
        lrow[t] = lrow[t] * alpha;
        mref[t] = mn;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ae = shfl_idx(alpha, 4 * g4 + e);
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[t][j][e] = acc[t][j][e] * ae;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kRT; ++t) {
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = fexp2(__builtin_fmaf(s8[t][i], A.c, -mref[t]));
      float rs = p[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) rs = rs + p[i];
      lrow[t] = lrow[t] + rows4_sum(rs);
      u32x4 pw;
#pragma unroll
      for (int i = 0; i < 4; ++i) pw[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
      pop[t] = __builtin_bit_cast(bf16x8, pw);
    }

    // O += bf16(P) V.  B operand of MFMA j: lane (n16, g4) supplies
    // V[key(8 g4 + ii)][DPL n16 + j], ii = 0..7 -- a register transpose of the
    // 8 rows it holds.  Output lane: rows 4 g4 + e, head_dim DPL n16 + j.
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      u32x4 bj;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t wa = vf[2 * pp][j >> 1];
        const uint32_t wb = vf[2 * pp + 1][j >> 1];
        bj[pp] = (j & 1) ? ((wa >> 16) | (wb & 0xffff0000u)) : ((wa & 0xffffu) | (wb << 16));
      }
      const bf16x8 vop = __builtin_bit_cast(bf16x8, bj);
#pragma unroll
      for (int t = 0; t < kRT; ++t)
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[t], vop, acc[t][j], 0, 0, 0);
    }
  }
  if (!has_rows) return;

  // Group partial of each row straight from the MFMA layout.
#pragma unroll
  for (int t = 0; t < kRT; ++t) {
    if (g4 == 0) {
      const int r = 16 * (t0 + t) + n16;
      if (r < A.R) {
        const size_t idx = ((size_t)g * A.R + r) * A.NG + q;
        A.gp_ml[idx * 2] = mref[t];
        A.gp_ml[idx * 2 + 1] = lrow[t];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 16 * (t0 + t) + 4 * g4 + e;
      if (r < A.R) {
        float* dst = A.gp_acc + (((size_t)g * A.R + r) * A.NG + q) * D + DPL * n16;
#pragma unroll
        for (int j = 0; j < DPL; j += 4)
          *reinterpret_cast<f32x4*>(dst + j) = f32x4{acc[t][j][e], acc[t][j + 1][e], acc[t][j + 2][e], acc[t][j + 3][e]};
      }
    }
  }
}

#undef RSPX_RK
#undef RSPX_RV

// ------------------------------------------------------------------ kernel B
// One wave per (query row mq, head h); a workgroup holds 4 consecutive heads of
// the same row (they share the node list and, for GQA >= 4, the kv head).
// Lanes split head_dim (DN = D / 64 values each).  Node fold, then the final
// combine (groups in order, node partial last) and the bf16 store.
template <int D>
__global__ __launch_bounds__(256) void node_merge_kernel(TrieAttnArgs A) {
  constexpr int DN = D / 64;
  constexpr int kB = 8;            // node slots per load batch
  constexpr int kMaxG = 16;        // groups per kv head (NG <= 16 by construction)
  __shared__ int16_t lds_list[4][kMaxNodeSlots];

  const int lane = __lane_id();
  const int w = threadIdx.x >> 6;
  const int HB = (A.HK * A.GQA + 3) / 4;
  const int hb = blockIdx.x % HB;
  const int mq = blockIdx.x / HB;
  const int h = hb * 4 + w;
  if (h >= A.HK * A.GQA) return;
  const int g = h / A.GQA;
  const int r = mq * A.GQA + (h - g * A.GQA);
  const int NG = A.NG;
  const int d0 = lane * DN;

  float qf[DN];
  load_row_f32<DN>(A.q + h * A.sqh + (int64_t)mq * A.sqm + d0, qf);

  // List the allowed node slots in slot order.
  int16_t* list = lds_list[w];
  const uint8_t* mrow = A.msk + (int64_t)mq * A.smm;
  int T = 0;
  for (int c0 = 0; c0 < A.NN; c0 += 64) {
    const int t = c0 + lane;
    const bool allowed = (t < A.NN) && (mrow[(int64_t)t * A.smn] != 0);
    const uint64_t bits = __builtin_amdgcn_ballot_w64(allowed);
    const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bits >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0));
    if (allowed) list[T + pos] = (int16_t)t;
    T += __builtin_popcountll(bits);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the list writes are visible to the wave
  __builtin_amdgcn_wave_barrier();

  float m = kNegInf, l = 0.f, acc[DN];
#pragma unroll
  for (int i = 0; i < DN; ++i) acc[i] = 0.f;
  const uint16_t* kb = A.kn + g * A.sknh + d0;
  const uint16_t* vb = A.vn + g * A.svnh + d0;

  uint32_t kr[2][kB], vr[2][kB];   // DN bf16 per lane: one packed word (DN = 2) or a half (DN = 1)
  auto ld = [&](const uint16_t* p) -> uint32_t {
    if constexpr (DN == 2) return *reinterpret_cast<const uint32_t*>(p);
    else return *p;
  };
  auto load_batch = [&](int b0, int buf) {
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int tt = list[min(b0 + u, T - 1)];
      kr[buf][u] = ld(kb + (int64_t)tt * A.sknn);
      vr[buf][u] = ld(vb + (int64_t)tt * A.svnn);
    }
  };
  if (T > 0) load_batch(0, 0);
  // Group partials of this row, requested after the first K/V batch (loads
  // complete in order) and consumed after the fold.
  float gm[kMaxG], gl[kMaxG], ga[kMaxG][DN];
  const size_t gbase = ((size_t)g * A.R + r) * NG;
#pragma unroll
  for (int qq = 0; qq < kMaxG; ++qq) {
    if (qq < NG) {
      gm[qq] = A.gp_ml[(gbase + qq) * 2];
      gl[qq] = A.gp_ml[(gbase + qq) * 2 + 1];
      const float* src = A.gp_acc + (gbase + qq) * D + d0;
      if constexpr (DN == 2) {
        const float2 v2 = *reinterpret_cast<const float2*>(src);
        ga[qq][0] = v2.x; ga[qq][1] = v2.y;
      } else {
        ga[qq][0] = src[0];
      }
    }
  }

  for (int b0 = 0; b0 < T; b0 += 2 * kB) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int bb = b0 + half * kB;
      if (bb >= T) break;
      if (bb + kB < T) load_batch(bb + kB, half ^ 1);
      float s[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        float dot = __builtin_fmaf(qf[0], bf16_lo(kr[half][u]), 0.f);
        if constexpr (DN == 2) dot = __builtin_fmaf(qf[1], bf16_hi(kr[half][u]), dot);
        s[u] = group_sum<64>(dot) * A.c;
      }
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        if (bb + u >= T) break;
        const float mn = fmaxf(m, s[u]);
        const float a = fexp2(m - mn);
        const float p = fexp2(s[u] - mn);
        l = __builtin_fmaf(l, a, p);
        acc[0] = __builtin_fmaf(p, bf16_lo(vr[half][u]), acc[0] * a);
        if constexpr (DN == 2) acc[1] = __builtin_fmaf(p, bf16_hi(vr[half][u]), acc[1] * a);
        m = mn;
      }
    }
  }

  // Final: groups in order, then the node partial.
  float fm = kNegInf, fl = 0.f, facc[DN];
#pragma unroll
  for (int i = 0; i < DN; ++i) facc[i] = 0.f;
#pragma unroll
  for (int qq = 0; qq < kMaxG; ++qq)
    if (qq < NG) combine<DN>(fm, fl, facc, gm[qq], gl[qq], ga[qq]);
  combine<DN>(fm, fl, facc, m, l, acc);

  uint16_t* o = A.out + h * A.soh + (int64_t)mq * A.som + d0;
  if constexpr (DN == 2) *reinterpret_cast<uint32_t*>(o) = pack_bf16x2(facc[0] / fl, facc[1] / fl);
  else o[0] = f32_to_bf16_rne(facc[0] / fl);
}

// ------------------------------------------------------------------ host side

struct Plan {
  int GQA, R, NT, RT, NG, RL, prompt_wgs, node_wgs;
  size_t off_gp_ml, off_gp_acc, total;
};

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Group length RL (keys) and count NG depend on P only: NG <= 16 groups of a
// whole number of 32-key steps.
static int make_plan(int H, int HK, int M, int P, int NN, int D, int rows_per_wave, Plan* pl) {
  if (H <= 0 || HK <= 0 || M < 0 || P < 0 || NN < 0 || H % HK != 0) return RSPX_EINVAL;
  if (NN > kMaxNodeSlots) return RSPX_EINVAL;
  if (D != 64 && D != 128) return RSPX_EUNSUPPORTED;
  const int GQA = H / HK;
  if (GQA != 1 && GQA != 2 && GQA != 4 && GQA != 8 && GQA != 16) return RSPX_EUNSUPPORTED;
  pl->GQA = GQA;
  pl->R = M * GQA;
  pl->NT = (pl->R + 15) / 16;
  if (P > 0) {
    const int steps = (P + kStep - 1) / kStep;
    const int ns = (steps + kNGTarget - 1) / kNGTarget;
    pl->RL = ns * kStep;
    pl->NG = (P + pl->RL - 1) / pl->RL;
  } else {
    pl->RL = kStep;
    pl->NG = 0;
  }
  const int rt = rows_per_wave == 0 ? 2 : rows_per_wave;
  if (rt != 1 && rt != 2) return RSPX_EINVAL;
  pl->RT = rt;
  const int rows_per_wg = kWaves * rt * 16;
  pl->prompt_wgs = HK * ((pl->R + rows_per_wg - 1) / rows_per_wg) * pl->NG;
  pl->node_wgs = M * ((H + 3) / 4);
  const size_t parts = (size_t)HK * pl->R * pl->NG;
  size_t off = 0;
  pl->off_gp_ml = off;  off = align256(off + parts * 2 * sizeof(float));
  pl->off_gp_acc = off; off = align256(off + parts * D * sizeof(float));
  pl->total = off;
  return RSPX_OK;
}

template <int D>
static void launch_all(const TrieAttnArgs& a, const Plan& pl, hipStream_t s) {
  if (pl.prompt_wgs > 0) {
    if (pl.RT == 1) hipLaunchKernelGGL((prompt_kernel<D, 1>), dim3(pl.prompt_wgs), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prompt_kernel<D, 2>), dim3(pl.prompt_wgs), dim3(256), 0, s, a);
  }
  hipLaunchKernelGGL((node_merge_kernel<D>), dim3(pl.node_wgs), dim3(256), 0, s, a);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace rspx

using namespace rspx;

extern "C" int64_t rspx_trie_attn_workspace_bytes(int H, int HK, int M, int P, int D) {
  Plan pl;
  if (make_plan(H, HK, M, P, 0, D, 1, &pl) != RSPX_OK) return -1;
  return (int64_t)pl.total;  // independent of NN and rows_per_wave
}

extern "C" int rspx_trie_attn(const void* q, int64_t sqh, int64_t sqm,
                              const void* kp, int64_t skph, int64_t skpn,
                              const void* vp, int64_t svph, int64_t svpn,
                              const void* kn, int64_t sknh, int64_t sknn,
                              const void* vn, int64_t svnh, int64_t svnn,
                              const uint8_t* msk, int64_t smm, int64_t smn,
                              void* out, int64_t soh, int64_t som,
                              int H, int HK, int M, int P, int NN, int D, float sm_scale,
                              void* workspace, int64_t workspace_bytes, int rows_per_wave,
                              void* stream) {
  Plan pl;
  int rc = make_plan(H, HK, M, P, NN, D, rows_per_wave, &pl);
  if (rc != RSPX_OK) return rc;
  if (!(sm_scale > 0.f) || sm_scale == __builtin_huge_valf()) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!q || !out || (P > 0 && (!kp || !vp)) || (NN > 0 && (!kn || !vn || !msk)))
    return RSPX_EINVAL;
  if (pl.total > 0 && (!workspace || workspace_bytes < (int64_t)pl.total)) return RSPX_EWORKSPACE;
  const void* ptrs[] = {q, kp, vp, kn, vn, out, workspace};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return RSPX_EALIGN;
  const int64_t strides[] = {sqh, sqm, skph, skpn, svph, svpn, sknh, sknn, svnh, svnn, soh, som};
  for (int64_t s : strides)
    if (s % 8 != 0) return RSPX_EALIGN;

  TrieAttnArgs a;
  a.q = static_cast<const uint16_t*>(q);   a.sqh = sqh;   a.sqm = sqm;
  a.kp = static_cast<const uint16_t*>(kp); a.skph = skph; a.skpn = skpn;
  a.vp = static_cast<const uint16_t*>(vp); a.svph = svph; a.svpn = svpn;
  a.kn = static_cast<const uint16_t*>(kn); a.sknh = sknh; a.sknn = sknn;
  a.vn = static_cast<const uint16_t*>(vn); a.svnh = svnh; a.svnn = svnn;
  a.msk = msk; a.smm = smm; a.smn = smn;
  a.out = static_cast<uint16_t*>(out); a.soh = soh; a.som = som;
  a.HK = HK; a.GQA = pl.GQA; a.M = M; a.P = P; a.NN = NN;
  a.R = pl.R; a.NT = pl.NT; a.NG = pl.NG; a.RL = pl.RL;
  a.c = (float)((double)sm_scale * 1.4426950408889634);
  char* ws = static_cast<char*>(workspace);
  a.gp_ml = reinterpret_cast<float*>(ws + pl.off_gp_ml);
  a.gp_acc = reinterpret_cast<float*>(ws + pl.off_gp_acc);

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) launch_all<128>(a, pl, s);
  else launch_all<64>(a, pl, s);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
