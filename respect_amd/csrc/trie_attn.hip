// Trie-verification attention for gfx950 (MI355X).
//
// Replaces the Triton kernel _attn_hyb / fused_attn_hyb of
// respect/kernels/attention.py:15-96.  Semantics per (head, query row):
// softmax(q . k * scale) . v over the P prompt keys (never masked) and over
// the node slots the row's mask allows, fp32 accumulation, bf16 output.
//
// Reduction tree, fixed by P and by the row's allowed node slots only:
//
//   step     32 prompt keys.  Scores from bf16 MFMA 16x16x32 (fp32
//            accumulate, head_dim reduced by a fixed chain of MFMAs),
//            base-2 exponent with the scale folded into log2(e).
//            Probabilities are rounded to bf16 before the PV MFMA, as the
//            reference rounds p before tl.dot (attention.py:48).
//   quarter  steps 4i + k (i = 0, 1, ...) of a group, online softmax in step
//            order.  The running reference maximum of a row moves only when
//            a step's maximum exceeds it by more than 2^8 (then the
//            accumulator is rescaled); otherwise probabilities are taken
//            against the old reference and may reach 2^8.
//   group    S = 4 NR consecutive steps (NG <= 8 groups): its quarters
//            scaled to the row's maximum M over them (2^(m_k - M), 0 for an
//            empty quarter) and summed as (q0 + q1) + (q2 + q3), l likewise.
//   node     score q.k c from a bf16 MFMA chain; m = the maximum over the
//            row's allowed node slots; p = 2^(s - m) in fp32, split as
//            hi = bf16(p) and lo = bf16(p - hi); the allowed slots taken in
//            slot order (rank r = the r-th allowed slot) in tiles of 32
//            ranks, each tile summed on the MFMA as acc += V^T hi, then
//            acc += V^T lo (l likewise with V = 1).  The reference's node loop
//            (attention.py:52-67) forms the same sums with an online maximum.
//            Masked slots are skipped; in the reference they are exact
//            no-ops, so only the sequence of allowed slots matters.
//   final    the NG groups left to right, then the node partial.
//
// S and NG depend on P only.  Which wave computes what changes with the number
// of rows, never the arithmetic of a row, so a row's bits are the same whether
// it is verified alone (1-token decoding) or inside a 128-node trie, and
// wherever its allowed slots sit in the node segment.
//
// Launches on the caller's stream, no host synchronisation.  Normally one,
// fused_kernel: workgroup = (kv head g, block of 32 RT GQA rows, key group),
// 8 waves = 2 row halves x 4 key quarters, all resident at once.  The waves
// issue the group's K/V straight from HBM into an LDS ring (buffer_load ...
// lds, a round of 4 steps per ring slot), laid out so that K fragments are one
// conflict-free ds_read_b128 and V fragments one ds_read_b64_tr_b16 (the
// transposing LDS read of gfx950) per MFMA operand half.  Wave (h, k) computes
// step 4i + k of round i for its 16 RT rows; the four quarters are combined
// through LDS and the group partial (m, l, acc) is stored; the workgroup then
// counts itself, computes the node partials of its share of the block's rows
// (MFMA scores and rank-tiled MFMA sums) and, once the block's groups are all
// counted, merges its rows.  A grid up to twice what the device holds at once
// runs as fused2_kernel (two row blocks per workgroup, one after the other);
// a larger one as prompt_kernel then node_merge_kernel -- the same bits.
//   Rows are packed GQA-wise (row = query * GQA + head-in-group), so a kv
//   head's K/V is read once from HBM for all query heads that share it.  With
//   8 kv heads, workgroup g of kernel A lands on XCD g (round-robin dispatch),
//   so the row blocks that share a head's K/V meet in one XCD's L2.
//   head_dim 32, 64, 128 or 256, the arithmetic the same function of D.  The
//   LDS budget sets the rest: a round of four steps takes 16 / 64 / 128 KB at
//   D = 32 / 128 / 256, so the ring holds 4 / 2 / 1 rounds; a resident node
//   segment holds 3 chunks (1 at D = 256), and D = 256 runs one 16-row tile
//   per wave (two would not fit the registers).

#include <mutex>
#include <type_traits>

#include "common.h"
#include "respect_amd.h"

namespace rspx {

constexpr int kStep = 32;        // keys per online-softmax step
constexpr int kQuarters = 4;     // key quarters (waves) per row half
constexpr int kGroupTarget = 8;  // maximum number of key groups per kv head
constexpr float kLazyTau = 8.f;  // log2 headroom before the reference max moves
constexpr int kMaxNodeSlots = 4096;
constexpr int kWavesA = 8;       // waves per prompt workgroup

// Strides are in elements; the host checks that every element offset of a
// tensor fits 30 bits, so offsets (and byte offsets) are 32-bit arithmetic.
// Kept at 184 bytes: one more int field (192 bytes of kernel arguments) made
// the compiler read pointers of this struct from memory as generic pointers,
// so the group-partial stores became flat stores, whose counters forced
// extra waits everywhere (the 8B-shape call 18.4 -> 34 us, same bits).
struct TrieAttnArgs {
  const uint16_t* q;  int sqh, sqm;
  const uint16_t* kp; int skph, skpn;
  const uint16_t* vp; int svph, svpn;
  const uint16_t* kn; int sknh, sknn;
  const uint16_t* vn; int svnh, svnn;
  const uint8_t* msk; int smm, smn;
  uint16_t* out;      int soh, som;   // soh < 0: out is [M, H D] in the tiled activation layout
  int HK, GQS, M, P, NN;   // GQS = log2(query heads per kv head)
  int R, NRB, NG, S;  // rows per kv head, row blocks, groups, steps per group
  float c;            // sm_scale * log2(e)
  float* gp_ml;       // [HK][R][NG][2]  group partial (m, l)
  float* gp_acc;      // [HK][R][NG][D]
  int* sync;          // fused launch: a timeout flag, then [HK][NRB][2] counters
  int spin;           // fused launch: polls of a block's counter before the wait gives up
  int deadline;       // fused launch: s_memrealtime ticks a wait may last before it gives up
};
static_assert(sizeof(TrieAttnArgs) == 184, "kernel argument struct stays at 184 bytes");

__device__ __forceinline__ int wg_index(const TrieAttnArgs& A, int g, int rb, int q) {
  return g + A.HK * (rb + A.NRB * q);
}

// Phase timestamps (built only with -DRSPX_PHASE_TRACE, into a separate
// library; the product library has none of this): wave w of workgroup b
// records the device's real-time counter (s_memrealtime, 100 MHz) at mark k
// of the one-launch kernel into g_phase[(b 8 + w) kPhaseMarks + k], read back
// with rspx_trie_attn_phase_trace.  Marks: 0 start; 1 + 2 r / 2 + 2 r round
// r (r < 3) landed / computed; 7 node loads issued and quarter (m, l)
// exchanged; 8 scaled quarters written; 9 quarter sums read; 10 node chunk
// written into LDS (the hook); 11 group partial stored and counted; 12 node
// partials done; 13 wait over; 14 merged; 15 end.
constexpr int kPhaseMarks = 16;
constexpr int kPhaseWgs = 1024;
// Dispatch-order index of workgroup (g, rb, q) of the one-launch grid
// (kv head fastest, then row block, then group), from values every mark's
// scope holds: no grid-size loads in the traced kernel.
#ifdef RSPX_PHASE_TRACE
__device__ uint64_t g_phase[kPhaseWgs * kWavesA * kPhaseMarks];
#define RSPX_MARK(k)                                                                                   \
  do {                                                                                                 \
    if (__lane_id() == 0 && wg_index(A, g, rb, q) < kPhaseWgs)                                         \
      g_phase[(wg_index(A, g, rb, q) * kWavesA + (threadIdx.x >> 6)) * kPhaseMarks + (k)] =            \
          __builtin_amdgcn_s_memrealtime();                                                            \
  } while (0)
#else
#define RSPX_MARK(k) \
  do {               \
  } while (0)
#endif

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

// state (m, l, acc) <- state (+) incoming.  An incoming partial with m = -inf
// is empty and left out (it would be an exact no-op).  From the empty state
// (-inf, 0, 0) the first combine reproduces the incoming partial exactly.
// Selects instead of a branch: the values are the same, and a branch here
// let the compiler sink the incoming partial's loads into it, after the
// other loads' wait.
template <int N>
__device__ __forceinline__ void combine(float& m, float& l, float* acc, float m2, float l2,
                                        const float* acc2) {
  const bool skip = m2 == kNegInf;
  const float mn = fmaxf(m, m2);
  const float a = fexp2(m - mn);
  const float b = fexp2(m2 - mn);
  l = skip ? l : __builtin_fmaf(l2, b, l * a);
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = skip ? acc[i] : __builtin_fmaf(acc2[i], b, acc[i] * a);
  m = skip ? m : mn;
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

// Sum over aligned groups of 16 lanes; every lane of a group gets bitwise the
// same value (each butterfly level adds the same two operands in every lane).
__device__ __forceinline__ float sum16(float x) {
  x = x + dpp<0xB1>(x);    // quad_perm [1,0,3,2]: lane ^ 1
  x = x + dpp<0x4E>(x);    // quad_perm [2,3,0,1]: lane ^ 2
  x = x + dpp<0x141>(x);   // row_half_mirror: quads of an 8-lane half
  x = x + dpp<0x140>(x);   // row_mirror: halves of a 16-lane row
  return x;
}

// Geometry of one 32-key step of K/V in LDS.  A step is cut into 1 KB chunks,
// one per wave-wide direct-to-LDS load (lane l's 16 bytes land at chunk base
// + 16 l).  K chunk (kb, i): lane (n16, g4) <- K[16 kb + n16][32 i + 8 g4, +8),
// exactly the A fragment lane l reads back with one ds_read_b128.  V: key rows
// of U = D / 8 16-byte units; unit b of key t sits at position b ^ f(t) of the
// row (f even), so the 16 lanes of one transposing read (4 keys x 32 bytes)
// hit distinct banks.
template <int D>
struct StepGeom {
  static constexpr int DQ = D / 32;          // QK MFMAs per 16x16 tile (k = 32 each)
  static constexpr int DT = D / 16;          // PV MFMAs per tile (16 head_dim columns each)
  static constexpr int U = D / 8;            // 16-byte units per key row
  static constexpr int KCH = 2 * DQ;         // K chunks per step
  static constexpr int VCH = D / 16;         // V chunks per step (32 keys x 2D bytes / 1 KB)
  static constexpr int CH = KCH + VCH;       // chunks per step
  static constexpr int KPV = 1024 / (16 * U);  // keys per V chunk
  static constexpr int KBYTES = KCH * 1024;
  static constexpr int SLOT = CH * 1024;     // bytes per step
  static constexpr int ROUND = kQuarters * SLOT;
  static constexpr int RING = D == 256 ? 1 : D == 128 ? 2 : 4;  // rounds in flight (LDS-bound)
  static constexpr int OWN = kQuarters * CH / kWavesA;  // chunks one wave issues per round
};

// K rows in LDS: 16-byte unit u of key row `key` holds the row's unit
// u ^ kswz(key), so the 16 lanes of an MFMA A-fragment read (keys n16 of a
// 16-key block, one 16-byte unit each) fall on 16 different bank groups of
// the 256-byte bank row, while each direct-to-LDS load still copies whole
// rows (KPV of them, 1 KB).  Rows of at least 256 bytes start in bank group
// 0, so the key alone picks the group; shorter rows share a bank row with
// 256 / (2 D) - 1 neighbours and the swizzle changes every 16 / U keys.
template <int D>
__device__ __forceinline__ int kswz(int key) {
  constexpr int U = D / 8;
  if constexpr (U >= 16) return key % 16;
  else return (key / (16 / U)) % U;
}

// V rows: an even swizzle (units 2 j and 2 j + 1 stay adjacent), so that the
// 32 lanes of one pass of a transposing read (8 keys x 32 bytes) hit distinct
// 32-byte bank ranges.
template <int D>
__device__ __forceinline__ int vswz(int key) {
  constexpr int U = D / 8;
  if constexpr (U >= 16) return 2 * (key % 8);
  else return 2 * ((key / (16 / U)) % (U / 2));
}

// s_waitcnt vmcnt(v) for an immediate v.
#define RSPX_VM(v) __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | 0x70 | 0xF00)

// Waits until at most `younger` rounds of OWN loads each (younger < RING) are
// still in flight: vmcnt(OWN younger), the count as an immediate.
template <int OWN, int RING>
__device__ __forceinline__ void wait_rounds(int younger) {
  static_assert(OWN * (RING - 1) < 64, "vmcnt range");
  if constexpr (RING > 1) {
    if (younger >= RING - 1) {
      RSPX_VM(OWN * (RING - 1));
      return;
    }
    wait_rounds<OWN, RING - 1>(younger);
  } else {
    RSPX_VM(0);
  }
}

// Direct-to-LDS loads: lane l's bytes land at dst + 16 l.  Non-template
// wrappers: the host compilation pass rejects these builtins inside templates.
__device__ __forceinline__ void dma16(const void* src, lds_char* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
}
// Raw buffer variant: byte offset `voff` from the descriptor base; reads past
// the descriptor's size return zeros and touch no memory.
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, int voff, lds_char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, 0, 0, 0);
}
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw-buffer descriptor dword 3
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(nbytes > 0 ? nbytes : 0), kBufWord3);
}

// The transposing LDS read: within each 16-lane row, lane i receives
// element (i % 4) of the 8 bytes addressed by lane 4 e + i / 4, for e = 0..3.
__device__ __forceinline__ s16x4 lds_read_tr(const lds_char* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
}

// lds_read_tr pair without the compiler's fence: the intrinsic's memory
// operand carries no alias information, so the compiler puts s_waitcnt
// vmcnt(0) in front of it -- a wait for every vector-memory operation in
// flight, the group partial's counter add included.  For LDS data that is
// known to be in place (its loads waited for), read the two halves in asm and
// wait for them (lgkmcnt) inside the asm that hands them out.
__device__ __forceinline__ void lds_read_tr2_nofence(const lds_char* p0, const lds_char* p1, s16x4& lo, s16x4& hi) {
  asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(lo), "=&v"(hi)
               : "v"(p0), "v"(p1)
               : "memory");
}

__device__ __forceinline__ void lds_barrier() {
  // Every wave's LDS reads issued so far are complete, then a raw s_barrier:
  // __syncthreads() would also wait for every direct-to-LDS load in flight.
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// This wave's chunks of one round (4 steps from step `sfirst` of the group)
// into the ring slot at `dst`: chunk c = w + 8 j is chunk c % CH of
// step-in-round c / CH.  voff[t] is the lane's byte offset of chunk
// (w + 8 t) % CH relative to its step's first key; kstep / vstep are the bytes
// per step.  The descriptors rk / rv start at the group's first key and end at
// key P of the kv head, so keys past P (and whole steps past P) read zeros
// without touching memory.
template <int D, int NV>
__device__ __forceinline__ void issue_round(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int kstep,
                                            int vstep, int sfirst, const int (&voff)[NV], lds_char* dst, int w) {
  using G = StepGeom<D>;
#pragma unroll
  for (int j = 0; j < G::OWN; ++j) {
    const int c = w + kWavesA * j;
    const int sr = c / G::CH, cc = c % G::CH;
    const int st = sfirst + sr;
    if (cc < G::KCH) bdma16(rk, voff[j % NV] + st * kstep, dst + sr * G::SLOT + cc * 1024);
    else bdma16(rv, voff[j % NV] + st * vstep, dst + sr * G::SLOT + cc * 1024);
  }
}

// ------------------------------------------------------------------ kernel A
// LDS of a prompt workgroup: the K/V ring, then the Q fragments.
template <int D, int kRT>
struct PromptLds {
  using G = StepGeom<D>;
  static constexpr int QBYTES = 2 * kRT * G::DQ * 1024;
  static constexpr int RINGBYTES = G::RING * G::ROUND;
  static constexpr int BYTES = RINGBYTES + QBYTES;
  // The quarters' (m, l) of the combine, past the Q fragments (KEEP_Q).
  static constexpr int MLBYTES = 8 * kRT * 16 * 8;
  static_assert(BYTES + MLBYTES <= 160 * 1024, "LDS budget");
};

// The prompt work of workgroup (g, rb, q) -- kv head g, rows [32 kRT rb,
// +32 kRT), key group q = steps [q S, q S + S) -- up to its group partial in
// memory.  Wave w: row half h = w / 4 (kRT tiles of 16 rows), key quarter
// k = w % 4 (steps 4 i + k of the group).  ATOMIC: the partial is stored with
// agent-scope atomic stores (write-through) for a merge inside the same launch.
// KEEP_Q: the combine's (m, l) go past the Q fragments (PromptLds::MLBYTES more
// LDS), which stay in place for the hook and after it.
// after_loop runs once every wave is past its last step, before the combine;
// first_round once every wave's round 0 (and every memory operation the
// workgroup issued before it) is complete.
template <int D, int kRT, bool ATOMIC, bool EARLY_STORES = false, bool KEEP_Q = false, class Hook, class Hook0,
          class Hook1>
__device__ __forceinline__ void prompt_block(const TrieAttnArgs& A, char* lds, int g, int rb, int q,
                                             const Hook& before_stores, const Hook0& after_loop,
                                             const Hook1& first_round) {
  using G = StepGeom<D>;
  using L = PromptLds<D, kRT>;
  constexpr int DQ = G::DQ, DT = G::DT;
  constexpr int RINGBYTES = L::RINGBYTES;

  const int lane = __lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int h = w >> 2, k = w & 3;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int P = A.P;
  const int steps = (P + kStep - 1) / kStep;
  const int s0 = q * A.S;                       // first step of the group
  const int ns = min(A.S, steps - s0);          // steps of the group (>= 1)
  const int nr = (ns + kQuarters - 1) / kQuarters;
  const int row0 = rb * 32 * kRT;               // first row of the block
  const int trow = row0 + 16 * kRT * h;         // first row of this wave's tiles
  const bool has_rows = trow < A.R;

  lds_char* ring = (lds_char*)lds;
  lds_char* qreg = ring + RINGBYTES;

  // Q^T fragments (B operand of S^T = K Q^T): chunk (tile T, i) holds, for
  // lane (n16, g4), row 16 T + n16 of the block, head_dim [32 i + 8 g4, +8).
  // Rows past R read row 0 and are never stored.
  for (int c = w; c < 2 * kRT * DQ; c += kWavesA) {
    const int T = c / DQ, i = c - T * DQ;
    const int r = row0 + 16 * T + n16;
    const int rc = r < A.R ? r : 0;
    const int mq = rc >> A.GQS, jh = rc & ((1 << A.GQS) - 1);
    dma16(A.q + (((g << A.GQS) + jh) * A.sqh + mq * A.sqm + 32 * i + 8 * g4), qreg + c * 1024);
  }

  // This wave's chunks of a round: c = w + 8 j, step-in-round c / CH, chunk
  // c % CH.  voff[t] is the lane's byte offset of chunk w + 8 t (mod CH)
  // relative to the step's first key.
  constexpr int NV = G::CH >= kWavesA ? G::CH / kWavesA : 1;
  int voff[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const int cc = (w + kWavesA * t) % G::CH;
    if (cc < G::KCH) {
      const int key = G::KPV * cc + lane / G::U;
      const int b = (lane % G::U) ^ kswz<D>(key);
      voff[t] = 2 * key * A.skpn + 16 * b;
    } else {
      const int key = G::KPV * (cc - G::KCH) + lane / G::U;
      const int b = (lane % G::U) ^ vswz<D>(key);
      voff[t] = 2 * key * A.svpn + 16 * b;
    }
  }
  const uint16_t* kpg = A.kp + g * A.skph;
  const uint16_t* vpg = A.vp + g * A.svph;

  // Transposing-read addresses of the V operand halves (keys 4 g4 + e and
  // 16 + 4 g4 + e) for head_dim tile j, relative to a step slot.
  int trv[2][DT];
  {
    const int e = n16 >> 2, c4 = n16 & 3;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int key = 16 * kh + 4 * g4 + e;
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        const int b = 2 * j + (c4 >> 1);
        trv[kh][j] = G::KBYTES + 16 * (key * G::U + (b ^ vswz<D>(key))) + 8 * (c4 & 1);
      }
    }
  }

  // A-fragment addresses of the K operand: lane (n16, g4) reads key
  // 16 kb + n16, head_dim [32 i + 8 g4, +8) = 16-byte unit 4 i + g4.
  int kro[2][DQ];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int key = 16 * kb + n16;
      kro[kb][i] = 16 * (key * G::U + ((4 * i + g4) ^ kswz<D>(key)));
    }

  float mref[kRT], lrow[kRT];
  f32x4 acc[kRT][DT];
#pragma unroll
  for (int t = 0; t < kRT; ++t) {
    mref[t] = kNegInf;
    lrow[t] = 0.f;
#pragma unroll
    for (int j = 0; j < DT; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int ks0 = s0 * kStep;   // the group's first key
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kpg + ks0 * A.skpn, 2 * ((P - ks0 - 1) * A.skpn + D));
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(vpg + ks0 * A.svpn, 2 * ((P - ks0 - 1) * A.svpn + D));
  const int kstep = 2 * kStep * A.skpn, vstep = 2 * kStep * A.svpn;
  // Round 0 alone first: requested together with the next rounds, it shared
  // the memory path with them and landed later; rounds 1 .. RING - 1 are
  // requested once round 0 is in, and land while it is computed.
  issue_round<D>(rk, rv, kstep, vstep, 0, voff, ring, w);

  bf16x8 qop[kRT][DQ];
  for (int r = 0; r < nr; ++r) {
    // Own chunks of round r (and the Q chunks, issued first) have landed.
    wait_rounds<G::OWN, G::RING>(r == 0 ? 0 : min(nr - 1 - r, G::RING - 1));
    lds_barrier();   // every wave's chunks of round r are in LDS
    if (r == 0) {
      first_round();
      for (int rr = 1; rr < min(nr, G::RING); ++rr)
        issue_round<D>(rk, rv, kstep, vstep, kQuarters * rr, voff, ring + rr * G::ROUND, w);
    }
    if (r < 3) RSPX_MARK(1 + 2 * r);
    if (r == 0 && has_rows) {
#pragma unroll
      for (int t = 0; t < kRT; ++t)
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          qop[t][i] = __builtin_bit_cast(
              bf16x8, *(const __attribute__((address_space(3))) u32x4*)(
                          qreg + ((kRT * h + t) * DQ + i) * 1024 + 16 * lane));
    }
    const int sl = kQuarters * r + k;  // step of this wave within the group
    if (has_rows && sl < ns) {

    const lds_char* slot = ring + (r % G::RING) * G::ROUND + k * G::SLOT;
    const int ks = (s0 + sl) * kStep;
    u32x4 kf[2][DQ];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < DQ; ++i)
        kf[kb][i] = *(const __attribute__((address_space(3))) u32x4*)(slot + kro[kb][i]);

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
    // scores; keys past P (only in the last step) are masked to -inf.  Since
    // scale > 0, max(s) * c is exactly the max of the scaled scores.
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
        for (int j = 0; j < DT; ++j) acc[t][j] = acc[t][j] * alpha;
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

    // O^T += V^T bf16(P)^T.  B operand: lane (n16, g4) holds row n16's p at
    // k-slots 8 g4 + i <-> keys 4 g4 + i (i < 4) and 12 + 4 g4 + i.  A operand
    // of head_dim tile j: V[key(k-slot)][16 j + n16], two transposing reads.
    // Output lane: row n16, head_dim 16 j + 4 g4 + e -- each lane holds four
    // consecutive head_dim columns of the row whose softmax state it keeps.
#pragma unroll
    for (int j = 0; j < DT; ++j) {
      const s16x4 lo = lds_read_tr(slot + trv[0][j]);
      const s16x4 hi = lds_read_tr(slot + trv[1][j]);
      const bf16x8 vop = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int t = 0; t < kRT; ++t)
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[t], acc[t][j], 0, 0, 0);
    }
    }
    if (r < 3) RSPX_MARK(2 + 2 * r);
    // Round r is consumed by every wave: its ring slot takes round r + RING.
    if (r + G::RING < nr) {
      lds_barrier();
      issue_round<D>(rk, rv, kstep, vstep, kQuarters * (r + G::RING), voff,
                     ring + (r % G::RING) * G::ROUND, w);
    }
  }

  after_loop();
  // Quarter partials combined in one step (the ring and the Q area are free
  // once every wave is past its last step).  Each wave writes (m, l) of its
  // rows, then scales its accumulators by s_k = exp2(m_k - M), M the row's
  // maximum over the four quarters k (s_k = 0 for an empty quarter), and
  // writes them row-major into the ring; every wave then sums a share of the
  // block's rows over the quarters as (q0 + q1) + (q2 + q3) and stores it, with
  // l = (l0 s0 + l1 s1) + (l2 s2 + l3 s3) beside M.
  typedef __attribute__((address_space(3))) float lds_float;
  typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
  typedef __attribute__((address_space(3))) f32x2 lds_f32x2;
  constexpr int BR = 32 * kRT;  // rows of the block
  static_assert(4 * BR * D * 4 <= RINGBYTES, "the four scaled quarters fit the ring");
  static_assert(L::MLBYTES <= L::QBYTES, "quarter (m, l) fit the Q area");
  lds_float* qml = (lds_float*)(KEEP_Q ? qreg + L::QBYTES : qreg);    // [h][k][t][16 rows] (m, l)
  lds_float* qacc = (lds_float*)ring;   // [k][BR rows][D], 16-byte units swizzled by row
  lds_barrier();
  if (g4 == 0) {
#pragma unroll
    for (int t = 0; t < kRT; ++t)
      *(lds_f32x2*)(qml + (((4 * h + k) * kRT + t) * 16 + n16) * 2) = f32x2{mref[t], lrow[t]};
  }
  lds_barrier();
  RSPX_MARK(7);
  float Mr[kRT], Lr[kRT];
#pragma unroll
  for (int t = 0; t < kRT; ++t) {
    float mk[4], lk[4], sk[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const f32x2 v = *(const lds_f32x2*)(qml + (((4 * h + kk) * kRT + t) * 16 + n16) * 2);
      mk[kk] = v.x;
      lk[kk] = v.y;
    }
    const float M = fmaxf(fmaxf(mk[0], mk[1]), fmaxf(mk[2], mk[3]));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) sk[kk] = mk[kk] == kNegInf ? 0.f : fexp2(mk[kk] - M);
    Mr[t] = M;
    Lr[t] = (lk[0] * sk[0] + lk[1] * sk[1]) + (lk[2] * sk[2] + lk[3] * sk[3]);
    const float own = k == 0 ? sk[0] : k == 1 ? sk[1] : k == 2 ? sk[2] : sk[3];
    // Row 16 t + n16 of this half, 16-byte units 4 j + g4, unit index XOR (row & 7).
    const int row = 16 * kRT * h + 16 * t + n16;
    lds_float* dst = qacc + (k * BR + row) * D;
#pragma unroll
    for (int j = 0; j < DT; ++j)
      *(lds_f32x4*)(dst + 4 * ((4 * j + g4) ^ (row & 7))) = acc[t][j] * own;
  }
  lds_barrier();
  RSPX_MARK(8);
  // Group partial: rows RPI x + lane / (D / 4), columns [4 c4, +4): 1 KB per
  // store instruction; ATOMIC: with the coherence of an agent-scope atomic store.
  // With fewer pieces than waves (D = 32, one row tile) waves past the last
  // piece store nothing.
  constexpr int RPI = 1024 / (4 * D);
  constexpr int NST = BR / RPI;
  static_assert(NST % kWavesA == 0 || NST < kWavesA, "every storing wave stores the same number of pieces");
  constexpr int NSW = (NST + kWavesA - 1) / kWavesA;
  const bool stores = NST >= kWavesA || w < NST;
  const int c4 = lane % (D / 4);
  f32x4 sv[NSW];
#pragma unroll
  for (int jj = 0; jj < NSW; ++jj) {
    sv[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!stores) continue;
    const int rl = (w + kWavesA * jj) * RPI + lane / (D / 4);
    const lds_float* src = qacc + rl * D + 4 * (c4 ^ (rl & 7));
    const f32x4 a0 = *(const lds_f32x4*)(src);
    const f32x4 a1 = *(const lds_f32x4*)(src + BR * D);
    const f32x4 a2 = *(const lds_f32x4*)(src + 2 * BR * D);
    const f32x4 a3 = *(const lds_f32x4*)(src + 3 * BR * D);
    sv[jj] = (a0 + a1) + (a2 + a3);
  }
  const __amdgpu_buffer_rsrc_t racc = buffer_rsrc(A.gp_acc, 0x7fffffff);
  auto store_partial = [&] {
    if (has_rows && k == 0 && g4 == 0) {
#pragma unroll
      for (int t = 0; t < kRT; ++t) {
        const int r = trow + 16 * t + n16;
        if (r < A.R) {
          const size_t mo = ((size_t)g * A.R + r) * A.NG + q;   // (m, l) pair index
          if constexpr (ATOMIC) {
            // One 8-byte store with the coherence of an agent-scope atomic store
            // (sc1), instead of two 4-byte atomic stores.
            __builtin_amdgcn_raw_buffer_store_b64(f32x2{Mr[t], Lr[t]}, buffer_rsrc(A.gp_ml, 0x7fffffff),
                                                  (int)(mo * 8), 0, 16);
          } else {
            A.gp_ml[2 * mo] = Mr[t];
            A.gp_ml[2 * mo + 1] = Lr[t];
          }
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < NSW; ++jj) {
      const int r = row0 + (w + kWavesA * jj) * RPI + lane / (D / 4);
      if (stores && r < A.R) {
        const size_t off = (((size_t)g * A.R + r) * A.NG + q) * D + 4 * c4;
        if constexpr (ATOMIC) __builtin_amdgcn_raw_buffer_store_b128(sv[jj], racc, (int)(off * 4), 0, 16);
        else *reinterpret_cast<f32x4*>(A.gp_acc + off) = sv[jj];
      }
    }
  };
  // EARLY_STORES (callers with no hook): the stores go out before the
  // barrier (128-node tries at 8B heads: 33.1 -> 32.7 us).  A hook that
  // writes node data into the ring goes first: issued after the stores, the
  // compiler's wait for the registers it writes from would also wait for
  // the stores' write-through, and further chunks' loads land while the
  // stores drain.
  if constexpr (EARLY_STORES) store_partial();
  // Every wave's ring reads are complete: `before_stores` may issue
  // direct-to-LDS loads into the ring.
  lds_barrier();
  RSPX_MARK(9);
  before_stores();
  RSPX_MARK(10);
  if constexpr (!EARLY_STORES) store_partial();
}

template <int D, int kRT>
__global__ __launch_bounds__(512) void prompt_kernel(TrieAttnArgs A) {
  __shared__ __attribute__((aligned(16))) char lds[PromptLds<D, kRT>::BYTES];
  prompt_block<D, kRT, false, true>(A, lds, blockIdx.x, blockIdx.y, blockIdx.z, [] {}, [] {}, [] {});
}

// ------------------------------------------------------------------ node partials and merge
constexpr int kChunk = 64;       // node slots staged in LDS at a time
constexpr int kNodeTile = 32;    // ranks per MFMA tile of the node sums
constexpr int kNodeRows = 16;    // rows of one node_rows call (at most one MFMA tile of columns)
constexpr int kRankTab = 128;    // entries of a wave's rolling rank -> slot table
static_assert(kMaxNodeSlots % kChunk == 0, "whole mask words");

// Node LDS, for at most kNodeRows rows:
//   KB   RES chunks of K as score fragments -- 1 KB per 16-slot tile kt and
//        32-wide head_dim step i; lane (n16, g4)'s 16 bytes are K[16 kt + n16][32 i +
//        8 g4, +8), one ds_read_b128;
//   VB   RES chunks of V rows, 2 D bytes per slot; 16-byte unit u of row r holds
//        the row's unit u ^ vswz(r), so the transposing reads of four rows hit
//        distinct banks.  When the segment streams, KB and VB hold instead
//        STAGES double-buffered V stages of kNodeTile rows (same row layout);
//   S    fp32 scores (times c) of the rows x the resident slots (or one chunk);
//   NP   the node partial of each row: m, l, pad, pad, acc[D];
//   MW   per group of rows, the 64-bit allowed-slot mask word of every chunk;
//   TAB  per wave, kRankTab int16: the slot of rank r at r % kRankTab;
//   Z    2 D bytes of zeros (the V row of a rank past the row's allowed count);
//   CNT  per group, the number of allowed slots.
//   RES chunks (192 slots up to D = 128, 64 at D = 256) make a resident
//   segment; STAGES waves stream a longer one.
template <int D> struct NodeLds {
  static constexpr int RES = D <= 128 ? 3 : 1;        // chunks a resident node segment holds
  static constexpr int STAGES = D <= 128 ? 6 : 2;     // waves with a double-buffered V stage when streaming
  static constexpr int CB = kChunk * 2 * D;   // one chunk's K (or V)
  static constexpr int KOFF = 0;
  static constexpr int VOFF = RES * CB;
  static constexpr int STAGE = 2 * kNodeTile * 2 * D;   // one wave's double-buffered V stage
  static_assert(STAGES * STAGE <= 2 * RES * CB, "stages fit KB + VB");
  static constexpr int SR = RES * kChunk + 4;      // floats per score row
  static constexpr int SOFF = 2 * RES * CB;
  static constexpr int NPROW = D + 4;
  static constexpr int NPOFF = SOFF + kNodeRows * SR * 4;
  static constexpr int MWOFF = NPOFF + kNodeRows * NPROW * 4;
  // A resident segment uses MW instead as each group's rank -> slot table (int16).
  static_assert(kNodeRows * RES * kChunk * 2 <= kNodeRows * (kMaxNodeSlots / kChunk) * 8, "rank tables fit MW");
  static constexpr int TOFF = MWOFF + kNodeRows * (kMaxNodeSlots / kChunk) * 8;
  static constexpr int ZOFF = TOFF + kWavesA * kRankTab * 2;
  static constexpr int CNTOFF = ZOFF + 2 * D;
  static constexpr int BYTES = CNTOFF + kNodeRows * 4;
  static constexpr int TGOFF = MWOFF;             // rank -> slot tables of a resident segment
  static __device__ __forceinline__ lds_char* kbuf(lds_char* kv, int b) { return kv + KOFF + b * CB; }
  static __device__ __forceinline__ lds_char* vbuf(lds_char* kv, int b) { return kv + VOFF + b * CB; }
};

template <int D> struct VResLds;

// Node LDS of a V-resident segment (RES < chunks <= VRES): only V stays in
// LDS (VRES chunks), the scores come from K fragments loaded into registers.
// The same roles and row layouts as NodeLds with VRES resident chunks.
template <int D> struct VResLds {
  static constexpr int RES = D <= 128 ? 5 : 1;    // chunks of the segment (320 slots up to D = 128; none at 256)
  static constexpr int CB = kChunk * 2 * D;
  static constexpr int VOFF = 0;
  static constexpr int SR = RES * kChunk + 4;
  static constexpr int SOFF = RES * CB;
  static constexpr int NPROW = D + 4;
  static constexpr int NPOFF = SOFF + kNodeRows * SR * 4;
  static constexpr int TGOFF = NPOFF + kNodeRows * NPROW * 4;
  static constexpr int ZOFF = TGOFF + kNodeRows * RES * kChunk * 2;
  static constexpr int CNTOFF = ZOFF + 2 * D;
  static constexpr int BYTES = CNTOFF + kNodeRows * 4;
  // Unused by a resident segment (streaming only), kept for node_task's signature.
  static constexpr int MWOFF = 0, TOFF = 0, KOFF = 0, STAGE = 0;
  static __device__ __forceinline__ lds_char* vbuf(lds_char* kv, int b) { return kv + VOFF + b * CB; }
};

// Bytes of LDS the node phase may use (either layout).
template <int D> constexpr int node_area_bytes() {
  return NodeLds<D>::BYTES > VResLds<D>::BYTES ? NodeLds<D>::BYTES : VResLds<D>::BYTES;
}

// Where a row's result goes: row r of kv head g is query r / GQA of head
// g GQA + r % GQA.  Rows past R shadow a valid row and are never stored.
struct RowRef {
  int rr, mq, hd;
  bool live;
};
__device__ __forceinline__ RowRef row_ref(const TrieAttnArgs& A, int g, int r, int fallback) {
  RowRef x;
  x.live = r < A.R;
  x.rr = x.live ? r : fallback;
  x.mq = x.rr >> A.GQS;
  x.hd = (g << A.GQS) + (x.rr & ((1 << A.GQS) - 1));
  return x;
}

// Element offset of (head R.hd, query R.mq, head_dim d) in out: strided, or
// column R.hd D + d of row R.mq of the tiled [M, H D] matrix (d a multiple
// of 4, so a lane's 2 or 4 elements stay contiguous in either layout).
template <int D>
__device__ __forceinline__ int64_t out_offset(int soh, int som, int heads, int hd, int mq, int d) {
  return soh < 0 ? tiled_offset(mq, hd * D + d, heads * D) : (int64_t)hd * soh + (int64_t)mq * som + d;
}

typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) int16_t lds_i16;
typedef __attribute__((address_space(3))) uint32_t lds_u32;

constexpr int kNodeRounds = kNodeRows / kWavesA;  // rows per wave in one node_rows call

// Loads a caller may issue ahead of node_rows for a resident node segment (at
// most NodeLds<D>::RES chunks): every chunk's K/V in LDS, the score fragment of the
// wave's first task and the mask bytes of the wave's rows.
template <int D> struct NodePre {
  bf16x8 qf[D / 32];
  // Raw mask bytes of chunk c and round i (m<c><i>), loaded without branches
  // from clamped addresses; node_rows zeroes the ones out of range and packs
  // them.  Nothing here is combined at issue time, so issuing them makes no
  // wave wait for its loads (a use right after the loads would wait for every
  // load in flight, the node K/V included, before the group partial is
  // stored).  Named scalars read with constant indices only: a run-time choice
  // between them can fold into one indexed load, which puts the whole struct
  // in scratch.
  uint32_t m00 = 0, m01 = 0, m10 = 0, m11 = 0, m20 = 0, m21 = 0;
};
static_assert(kNodeRounds == 2, "NodePre holds the mask bytes of two rounds");
// node_masks of chunk c from node_prefetch's raw bytes (r0: round 0, r1: round 1).
// The empty asm pins the packing here: hoisted up to the loads, it made the
// wave wait for them before the group partial's stores.
__device__ __forceinline__ uint32_t pre_masks(const TrieAttnArgs& A, int nrd, int c, uint32_t r0, uint32_t r1) {
  asm volatile("" : "+v"(r0), "+v"(r1));
  const bool in = c * kChunk + __lane_id() < A.NN;
  return (in && nrd > 0 ? r0 : 0u) | ((in && nrd > 1 ? r1 : 0u) << 8);
}

// Chunk c0 of kv head g's node K (score fragments) and V rows (16-byte units
// swizzled by row) into LDS buffer b: 1 KB pieces x = w + 8 j of the chunk's
// D / 8 K pieces, then its D / 8 V pieces.  Slots past NN read zeros.  Piece
// x + 8 lies a fixed distance further on than piece x, in memory and in LDS
// (8 is a multiple of the D / 32 K pieces per 16 slots, and V rows move by a
// multiple of the swizzle's 8-row period), so each wave computes its first K
// and V offsets once and steps them: straight-line issue, no per-piece
// divisions.
// Pieces of node_issue per wave.
template <int D> constexpr int node_pieces() {
  constexpr int KX = NodeLds<D>::CB / 1024;
  return KX % kWavesA == 0 ? 2 * KX / kWavesA : 1;
}

// f(j, rsrc, byte offset, LDS offset from kv) for piece j of this wave.
template <int D, class F>
__device__ __forceinline__ void node_each_piece(const TrieAttnArgs& A, int g, int c0, int b, int w, const F& f) {
  using LY = NodeLds<D>;
  constexpr int DQ = D / 32, RB = 2 * D;
  constexpr int KX = LY::CB / 1024;        // K pieces (and V pieces) of a chunk
  constexpr int NJ = 2 * KX / kWavesA;     // pieces per wave
  static_assert(8 % DQ == 0 && 1024 % RB == 0 && (KX % kWavesA == 0 || 2 * KX == kWavesA), "piece stepping");
  const int lane = __lane_id();
  const int left = A.NN - c0 - 1;
  const __amdgpu_buffer_rsrc_t rk =
      buffer_rsrc(A.kn + (g * A.sknh + c0 * A.sknn), 2 * (left * A.sknn + D));
  const __amdgpu_buffer_rsrc_t rv =
      buffer_rsrc(A.vn + (g * A.svnh + c0 * A.svnn), 2 * (left * A.svnn + D));
  // First K piece of the wave: w (at D = 32, one piece per wave: K for w < 4).
  const int koff = 2 * ((16 * (w / DQ) + (lane & 15)) * A.sknn + 32 * (w % DQ) + 8 * (lane >> 4));
  const int kstep = 2 * 16 * (8 / DQ) * A.sknn;
  // First V piece: w, or w - KX at D = 32.
  const int y0 = KX % kWavesA == 0 ? w : w - KX;
  const int row = y0 * (1024 / RB) + 16 * lane / RB;
  const int voff = 2 * row * A.svnn + 16 * (((16 * lane) % RB) / 16 ^ vswz<D>(row));
  const int vstep = 2 * kWavesA * (1024 / RB) * A.svnn;
  if constexpr (KX % kWavesA == 0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j < KX / kWavesA) f(j, rk, koff + j * kstep, LY::KOFF + b * LY::CB + (w + kWavesA * j) * 1024);
      else f(j, rv, voff + (j - KX / kWavesA) * vstep, LY::VOFF + b * LY::CB + (w + kWavesA * (j - KX / kWavesA)) * 1024);
    }
  } else {
    const bool isk = w < KX;
    f(0, isk ? rk : rv, isk ? koff : voff, isk ? LY::KOFF + b * LY::CB + w * 1024 : LY::VOFF + b * LY::CB + y0 * 1024);
  }
}

template <int D>
__device__ __forceinline__ void node_issue(const TrieAttnArgs& A, int g, int c0, lds_char* kv, int b, int w) {
  node_each_piece<D>(A, g, c0, b, w, [&](int, __amdgpu_buffer_rsrc_t r, int off, int lo) { bdma16(r, off, kv + lo); });
}

// node_issue's pieces of chunk c0 into registers (lane i: the 16 bytes its
// direct-to-LDS load would have written at the piece's LDS offset + 16 i), and
// their LDS stores into buffer b: the loads can then be in flight while the
// LDS is still in other use, with no LDS-DMA fence on the LDS accesses between.
template <int D>
__device__ __forceinline__ void node_load(const TrieAttnArgs& A, int g, int c0, u32x4 (&pc)[node_pieces<D>()], int w) {
  node_each_piece<D>(A, g, c0, 0, w, [&](int j, __amdgpu_buffer_rsrc_t r, int off, int) {
    pc[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  });
}
template <int D>
__device__ __forceinline__ void node_put(const TrieAttnArgs& A, int g, int c0, lds_char* kv, int b,
                                         const u32x4 (&pc)[node_pieces<D>()], int w) {
  const int lane = __lane_id();
  node_each_piece<D>(A, g, c0, b, w, [&](int j, __amdgpu_buffer_rsrc_t, int, int lo) {
    *(lds_u32x4*)(kv + lo + 16 * lane) = pc[j];
  });
}

// Score fragment of the rows starting at p0: lane (n16, g4) holds head_dim
// [32 i + 8 g4, +8) of row p0 + n16 (rows at or past rend shadow row p0).
template <int D>
__device__ __forceinline__ void node_q(const TrieAttnArgs& A, int g, int p0, int rend, bf16x8 (&qf)[D / 32]) {
  const int lane = __lane_id();
  const int r = p0 + (lane & 15);
  const RowRef R = row_ref(A, g, r < rend ? r : p0, p0);
  const uint16_t* qp = A.q + (R.hd * A.sqh + R.mq * A.sqm + 8 * (lane >> 4));
#pragma unroll
  for (int i = 0; i < D / 32; ++i) qf[i] = *reinterpret_cast<const bf16x8*>(qp + 32 * i);
}

// node_q's fragment from a prompt workgroup's Q fragments in LDS (prompt_block
// with KEEP_Q: chunk (tile T, i) at qreg + 1 KB (T DQ + i), lane (n16, g4)
// holding row 16 T + n16 of the block from row0, head_dim [32 i + 8 g4, +8)),
// for rows p0 .. rend - 1 of that block.  The asm read and its own lgkmcnt
// wait keep the compiler from fencing it behind the direct-to-LDS loads in
// flight.
template <int D>
__device__ __forceinline__ void node_q_lds(const lds_char* qreg, int row0, int p0, int rend, bf16x8 (&qf)[D / 32]) {
  constexpr int DQ = D / 32;
  const int lane = __lane_id();
  const int r = p0 + (lane & 15);
  const int br = (r < rend ? r : p0) - row0;
  const lds_char* src = qreg + (br >> 4) * DQ * 1024 + 16 * ((br & 15) + 16 * (lane >> 4));
  if constexpr (DQ == 4) {
    u32x4 v0, v1, v2, v3;
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
        : "v"(src)
        : "memory");
    qf[0] = __builtin_bit_cast(bf16x8, v0);
    qf[1] = __builtin_bit_cast(bf16x8, v1);
    qf[2] = __builtin_bit_cast(bf16x8, v2);
    qf[3] = __builtin_bit_cast(bf16x8, v3);
  } else {
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      u32x4 v;
      asm volatile("ds_read_b128 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(src), "i"(1024 * i) : "memory");
      qf[i] = __builtin_bit_cast(bf16x8, v);
    }
  }
}

// Mask byte of row r (below R) for slot c0 + lane; 0 past NN.
__device__ __forceinline__ uint8_t node_mask(const TrieAttnArgs& A, int r, int c0) {
  const int t = c0 + __lane_id();
  return t < A.NN ? A.msk[(r >> A.GQS) * A.smm + t * A.smn] : (uint8_t)0;
}

// Mask bytes of the wave's rounds for chunk c0: byte i for row p0 + w + 8 i.
__device__ __forceinline__ uint32_t node_masks(const TrieAttnArgs& A, int p0, int nrd, int w, int c0) {
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < kNodeRounds; ++i)
    if (i < nrd) mb |= (uint32_t)node_mask(A, p0 + w + kWavesA * i, c0) << (8 * i);
  return mb;
}

// Scores q.k times A.c of rows [p0, rend) (at most kNodeRows) and chunk c0's
// slots into S ([row - p0][SR], fp32): one 16x16x32 MFMA chain per 16-slot
// tile, waves 0..3 one tile each; qf is the score fragment of rows p0 + n16.
// Each score depends only on its row's q and its slot's k (the chain over
// head_dim is the same in every tile and lane): no position changes its bits.
template <int D, int SR>
__device__ __forceinline__ void node_scores(const TrieAttnArgs& A, int c0, const lds_char* kb, lds_float* S, int w,
                                            const bf16x8 (&qf)[D / 32]) {
  constexpr int DQ = D / 32;
  const int lane = __lane_id();
  const int kt = w;
  if (kt >= 4 || 16 * kt >= A.NN - c0) return;
  f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    const bf16x8 a = *(const __attribute__((address_space(3))) bf16x8*)(kb + (kt * DQ + i) * 1024 + 16 * lane);
    sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[i], sv, 0, 0, 0);
  }
  // Lane (n16, g4), element j: slot 16 kt + 4 g4 + j of row p0 + n16.
  *(lds_f32x4*)(S + (lane & 15) * SR + 16 * kt + 4 * (lane >> 4)) = sv * A.c;
}

__device__ __forceinline__ float max64(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return rows4_max(x);
}

__device__ __forceinline__ int lanes_below(uint64_t mm) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0));
}
__device__ __forceinline__ uint64_t lds_u64_uniform(const lds_char* p) {
  const u32x2 v = *(const __attribute__((address_space(3))) u32x2*)p;
  return ((uint64_t)__builtin_amdgcn_readfirstlane(v[1]) << 32) | (uint32_t)__builtin_amdgcn_readfirstlane(v[0]);
}

// The rank -> slot table of one wave for one group: mask words are consumed in
// slot order, each allowed slot written at its rank % kRankTab, until the ranks
// below `upto` are all in the table (or the words run out).  Entries of ranks in
// [upto - 64, upto + 63] never alias each other.
// rc: next mask word, rbase: ranks before word rc (wave-uniform).
__device__ __forceinline__ void rank_fill(int& rc, int& rbase, int upto, int nch, const lds_char* mw, lds_i16* tab) {
  const int lane = __lane_id();
  while (rbase < upto && rc < nch) {
    const uint64_t mm = lds_u64_uniform(mw + 8 * rc);
    if ((mm >> lane) & 1) tab[(rbase + lanes_below(mm)) & (kRankTab - 1)] = (int16_t)(kChunk * rc + lane);
    rbase += __builtin_popcountll(mm);
    ++rc;
  }
}

// The node sums of one group of rows (the rows of query mq among [p0, rend);
// MFMA column n16 is row p0 + n16, whose score fragment is qf, and columns of
// rows outside the group carry p = 0) over d-tiles [NJ sl, NJ sl + NJ) of
// head_dim, and l when sl = 0.  Ranks in tiles of kNodeTile: per tile the p of
// the tile's ranks (0 past the group's allowed count n), hi = bf16(p),
// lo = bf16(p - hi), then acc <- MFMA(V^T, hi, acc), acc <- MFMA(V^T, lo, acc),
// l likewise with V = 1 -- k-slot 8 g4 + i of the B operand is rank 4 g4 + i
// (i < 4) or 16 + 4 g4 + i - 4, as the prompt's PV product.  RES: p comes by
// rank from the score area (node_rows wrote it there) and V rows are gathered
// from the resident chunks through the group's rank -> slot table.  Otherwise
// the ranks come from the query's mask words, S^T = K Q^T is recomputed for
// the tile's slots (the chain of node_scores: the same bits) with K straight
// from memory, p = 2^(s - m), and the tile's 32 V rows are copied by rank into
// this wave's stage.
template <int D, bool RES, int NJ, class LY = NodeLds<D>>
__device__ __forceinline__ void node_task(const TrieAttnArgs& A, int g, int p0, int rend, int mq, int gl, int sl,
                                          lds_char* kv, int w, int nch, const bf16x8 (&qf)[D / 32]) {
  constexpr int DQ = D / 32, RB = 2 * D;
  const int lane = __lane_id();
  const int n16 = lane & 15, g4 = lane >> 4, e4 = n16 >> 2, c4 = n16 & 3;
  const int row = p0 + n16;                            // column n16: row p0 + n16 (qf's rows)
  const bool col = row < rend && (row >> A.GQS) == mq;
  const int rl = col ? n16 : 0;                        // its local row
  lds_float* NP = (lds_float*)(kv + LY::NPOFF);
  const lds_char* mw = kv + LY::MWOFF + gl * (kMaxNodeSlots / kChunk) * 8;
  lds_i16* tab = (lds_i16*)(kv + LY::TOFF) + w * kRankTab;
  const lds_char* zrow = kv + LY::ZOFF;
  const int n = __builtin_amdgcn_readfirstlane(*(const lds_u32*)(kv + LY::CNTOFF + 4 * gl));
  const float mcol = NP[rl * LY::NPROW];

  const __amdgpu_buffer_rsrc_t rk =
      buffer_rsrc(A.kn + g * A.sknh, 2 * ((A.NN - 1) * A.sknn + D));
  const __amdgpu_buffer_rsrc_t rv =
      buffer_rsrc(A.vn + g * A.svnh, 2 * ((A.NN - 1) * A.svnn + D));
  lds_char* stage = kv + LY::KOFF + w * LY::STAGE;

  const uint32_t one2 = 0x3f803f80u;   // two bf16 1.0
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{one2, one2, one2, one2});
  f32x4 acc[NJ], lacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jj = 0; jj < NJ; ++jj) acc[jj] = f32x4{0.f, 0.f, 0.f, 0.f};

  int rc = 0, rbase = 0;
  const int ntile = (n + kNodeTile - 1) / kNodeTile;
  const lds_float* Srow = (const lds_float*)(kv + LY::SOFF) + rl * LY::SR;
  for (int t = 0; t < ntile; ++t) {
    const int r0 = kNodeTile * t;
    if constexpr (!RES) rank_fill(rc, rbase, r0 + kNodeTile, nch, mw, tab);
    float pv[8];   // p of ranks r0 + 16 kb + 4 g4 + j (the B operand's k-slots)
    const lds_char *vrow0, *vrow1;
    int vsw0, vsw1;
    if constexpr (RES) {
      // p of the row by rank (node_rows wrote them over the row's scores) and
      // the group's rank -> slot table: four consecutive ranks per read.
      const f32x4 pa = *(const lds_f32x4*)(Srow + r0 + 4 * g4);
      const f32x4 pb = *(const lds_f32x4*)(Srow + r0 + 16 + 4 * g4);
      const lds_i16* tg = (const lds_i16*)(kv + LY::TGOFF) + gl * LY::RES * kChunk;
      uint64_t t4[2];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
        t4[kh] = *(const __attribute__((address_space(3))) uint64_t*)(tg + r0 + 16 * kh + 4 * g4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = col && r0 + 4 * g4 + j < n ? pa[j] : 0.f;
        pv[4 + j] = col && r0 + 16 + 4 * g4 + j < n ? pb[j] : 0.f;
      }
      // V rows of ranks r0 + 16 kh + 4 g4 + e4 (entry e4 of t4[kh]); ranks past
      // n read the zero row.
      auto vsrc = [&](int kh, const lds_char*& vr, int& sw) {
        const bool on = r0 + 16 * kh + 4 * g4 + e4 < n;
        const int s = (int)((t4[kh] >> (16 * e4)) & 0xffff);
        vr = on ? LY::vbuf(kv, s >> 6) + (s & 63) * RB : zrow;
        sw = on ? vswz<D>(s & 63) : 0;
      };
      vsrc(0, vrow0, vsw0);
      vsrc(1, vrow1, vsw1);
    } else {
      // K fragments of the tile's two 16-rank blocks (lane (n16, g4): rank
      // r0 + 16 kb + n16) straight from memory; the 32 V rows copied by rank into
      // this wave's stage (rows past n read zeros).
      u32x4 kf[2][DQ];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int rk_ = r0 + 16 * kb + n16;
        const int s = rk_ < n ? tab[rk_ & (kRankTab - 1)] : 0;
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          kf[kb][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rk, 2 * (s * A.sknn + 32 * i + 8 * g4), 0, 0));
      }
      lds_char* st = stage + (t & 1) * (kNodeTile * RB);
#pragma unroll
      for (int x = 0; x < kNodeTile * RB / 1024; ++x) {
        const int byte = x * 1024 + 16 * lane;
        const int rr = byte / RB, u = (byte % RB) / 16;
        const int rv_ = r0 + rr;
        const int s = rv_ < n ? tab[rv_ & (kRankTab - 1)] : -1;
        bdma16(rv, s >= 0 ? 2 * s * A.svnn + 16 * (u ^ vswz<D>(rr)) : 0x7ffffff0, st + x * 1024);
      }
      const int rr0 = 4 * g4 + e4, rr1 = 16 + 4 * g4 + e4;
      vrow0 = st + rr0 * RB;
      vrow1 = st + rr1 * RB;
      vsw0 = vswz<D>(rr0);
      vsw1 = vswz<D>(rr1);
      __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): K fragments and this wave's stage rows
      // Scores (the chain of node_scores: the same bits as the resident form).
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[kb][i]), qf[i], sv, 0, 0, 0);
        const f32x4 sc = sv * A.c;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool on = col && r0 + 16 * kb + 4 * g4 + j < n;
          pv[4 * kb + j] = on ? fexp2(sc[j] - mcol) : 0.f;
        }
      }
    }
    u32x4 hw, lw;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hw[i] = pack_bf16x2(pv[2 * i], pv[2 * i + 1]);
      lw[i] = pack_bf16x2(pv[2 * i] - bf16_lo(hw[i]), pv[2 * i + 1] - bf16_hi(hw[i]));
    }
    const bf16x8 hop = __builtin_bit_cast(bf16x8, hw), lop = __builtin_bit_cast(bf16x8, lw);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const int b = 2 * (NJ * sl + jj) + (c4 >> 1);
      s16x4 lo, hi;
      if constexpr (RES) {
        // V rows resident since before the caller's wait: no fence needed.
        lds_read_tr2_nofence(vrow0 + 16 * (b ^ vsw0) + 8 * (c4 & 1), vrow1 + 16 * (b ^ vsw1) + 8 * (c4 & 1), lo, hi);
      } else {
        lo = lds_read_tr(vrow0 + 16 * (b ^ vsw0) + 8 * (c4 & 1));
        hi = lds_read_tr(vrow1 + 16 * (b ^ vsw1) + 8 * (c4 & 1));
      }
      const bf16x8 vop = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, hop, acc[jj], 0, 0, 0);
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, lop, acc[jj], 0, 0, 0);
    }
    if (sl == 0) {
      lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, hop, lacc, 0, 0, 0);
      lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, lop, lacc, 0, 0, 0);
    }
  }
  // Lane (n16, g4) holds head_dim 16 j + 4 g4 + e of column n16.
  if (col) {
    lds_float* np = NP + rl * LY::NPROW;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) *(lds_f32x4*)(np + 4 + 16 * (NJ * sl + jj) + 4 * g4) = acc[jj];
    if (sl == 0 && g4 == 0) np[1] = lacc[0];
  }
}

// The per-row pass of a resident segment, rows p0 + w + 8 i (i < nrd) of this
// wave, after the scores S of every resident chunk are in LDS: m (the exact
// maximum over the row's allowed slots) into NP, then p = 2^(s - m) of the
// allowed slots written by rank over the row's own scores (rank <= slot: every
// score is in registers first); the group's first row writes its rank -> slot
// table and count.  mb[c]: the rows' mask bytes of chunk c (byte i: round i).
template <int D, class LY>
__device__ __forceinline__ void node_rank_rows(const TrieAttnArgs& A, int p0, int nrd, lds_char* kv, int w, int nch,
                                               const uint32_t (&mb)[LY::RES]) {
  constexpr int nw = kWavesA;
  const int lane = __lane_id();
  const int GQA = 1 << A.GQS;
  const int q0 = p0 >> A.GQS;
  lds_float* S = (lds_float*)(kv + LY::SOFF);
  lds_float* NP = (lds_float*)(kv + LY::NPOFF);
  lds_i16* TG = (lds_i16*)(kv + LY::TGOFF);
#pragma unroll 1
  for (int i = 0; i < nrd; ++i) {
    const int row = w + nw * i;
    const int r = p0 + row;
    const bool lead = r == p0 || (r & (GQA - 1)) == 0;
    const int gl = (r >> A.GQS) - q0;
    float sc[LY::RES];
    bool ok[LY::RES];
    float x = kNegInf;
#pragma unroll
    for (int c = 0; c < LY::RES; ++c) {
      ok[c] = c < nch && ((mb[c] >> (8 * i)) & 0xff) != 0;
      sc[c] = c < nch ? S[row * LY::SR + kChunk * c + lane] : 0.f;
      x = fmaxf(x, ok[c] ? sc[c] : kNegInf);
    }
    const float m = max64(x);
    if (lane == 0) NP[row * LY::NPROW] = m;
    int base = 0;
#pragma unroll
    for (int c = 0; c < LY::RES; ++c) {
      if (c < nch) {
        const uint64_t mm = __builtin_amdgcn_ballot_w64(ok[c]);
        const int rk = base + lanes_below(mm);
        if (ok[c]) {
          S[row * LY::SR + rk] = fexp2(sc[c] - m);
          if (lead) TG[gl * LY::RES * kChunk + rk] = (int16_t)(kChunk * c + lane);
        }
        base += __builtin_popcountll(mm);
      }
    }
    if (lead && lane == 0) *(lds_u32*)(kv + LY::CNTOFF + 4 * gl) = (uint32_t)base;
  }
}

// The node sums of a resident segment for rows [p0, rend): (group, d-slice)
// tasks over the waves, at most two per wave.
template <int D, class LY>
__device__ __forceinline__ void node_res_tasks(const TrieAttnArgs& A, int g, int p0, int rend, lds_char* kv, int w,
                                               int nch, const bf16x8 (&qf)[D / 32]) {
  constexpr int nw = kWavesA;
  constexpr int DT = D / 16;
  const int q0 = p0 >> A.GQS;
  const int ng = ((rend - 1) >> A.GQS) - q0 + 1;  // groups of rows (one query each)
  const int ds = ng >= 8 ? 1 : ng >= 4 ? 2 : ng >= 2 ? 4 : 8;
  const int dsl = ds < DT ? ds : DT;
  for (int task = w; task < ng * dsl; task += nw) {
    const int gl = task / dsl, sl = task - gl * dsl;
    const int nj = DT / dsl;
    if (nj == DT) node_task<D, true, DT, LY>(A, g, p0, rend, q0 + gl, gl, sl, kv, w, nch, qf);
    else if (nj * 2 == DT) node_task<D, true, (DT >= 2 ? DT / 2 : 1), LY>(A, g, p0, rend, q0 + gl, gl, sl, kv, w, nch, qf);
    else if (nj * 4 == DT) node_task<D, true, (DT >= 4 ? DT / 4 : 1), LY>(A, g, p0, rend, q0 + gl, gl, sl, kv, w, nch, qf);
    else node_task<D, true, (DT >= 8 ? DT / 8 : 1), LY>(A, g, p0, rend, q0 + gl, gl, sl, kv, w, nch, qf);
  }
}

// Node partials of rows [p0, rend) of kv head g (at most kNodeRows) over each
// row's allowed node slots (attention.py:52-67): m is the exact maximum score
// over the allowed slots; the sums run over the allowed slots in slot order
// (rank r = the r-th allowed slot), in MFMA tiles of kNodeTile ranks (node_task),
// so every bit depends only on the ordered list of the row's allowed (k, v),
// not on where in the node segment they sit.  Every wave of the workgroup
// calls it; the partial (m, l, acc) of row p0 + i is left in the node-partial
// area of LDS, row i, after the closing barrier.
//   have_pre: the caller issued a resident segment (at most RES chunks,
// chunk c into buffer c) and `pre` (node_prefetch), has since waited for those
// loads (vmcnt 0) and passed a workgroup barrier.  A resident segment the
// caller did not issue is loaded here; a longer one streams: its maxima come
// from a pass over K chunk by chunk, its sums from K and V gathered by rank.
template <int D>
__device__ __forceinline__ const lds_float* node_rows(const TrieAttnArgs& A, int g, int p0, int rend, lds_char* kv,
                                                     int w, const NodePre<D>& pre, bool have_pre) {
  using LY = NodeLds<D>;
  constexpr int nw = kWavesA;
  constexpr int DT = D / 16;
  const int lane = __lane_id();
  const int NN = A.NN;
  if (NN == 0) return (const lds_float*)(kv + LY::NPOFF);
  const int nrd = (rend - p0 - w + nw - 1) / nw;   // rows of this wave: p0 + w + 8 i
  const int nch = (NN + kChunk - 1) / kChunk;
  const bool res = NN <= LY::RES * kChunk;
  constexpr bool kVRes = VResLds<D>::RES > LY::RES;
  const bool vres = kVRes && !res && NN <= VResLds<D>::RES * kChunk;
  lds_float* S = (lds_float*)(kv + LY::SOFF);
  lds_float* NP = (lds_float*)(kv + LY::NPOFF);
  const int GQA = 1 << A.GQS;
  const int q0 = p0 >> A.GQS;
  const int ng = ((rend - 1) >> A.GQS) - q0 + 1;  // groups of rows (one query each)
  bf16x8 qf[D / 32];                               // score fragment of rows p0 + n16
  if (have_pre) {
#pragma unroll
    for (int i = 0; i < D / 32; ++i) qf[i] = pre.qf[i];
  } else {
    node_q<D>(A, g, p0, rend, qf);
  }

  // Maxima, mask words, allowed counts.  The first row of each group in
  // [p0, rend) records the group's mask words and count.
  auto row_words = [&](int i, int c, uint32_t mb, float x) {
    const int r = p0 + w + nw * i;
    const bool lead = r == p0 || (r & (GQA - 1)) == 0;
    const uint64_t mm = __builtin_amdgcn_ballot_w64(((mb >> (8 * i)) & 0xff) != 0);
    if (lead && lane == 0) {
      const int gl = (r >> A.GQS) - q0;
      *(__attribute__((address_space(3))) uint64_t*)(kv + LY::MWOFF + (gl * (kMaxNodeSlots / kChunk) + c) * 8) = mm;
      lds_u32* cnt = (lds_u32*)(kv + LY::CNTOFF + 4 * gl);
      *cnt = (c == 0 ? 0u : *cnt) + (uint32_t)__builtin_popcountll(mm);
    }
    (void)x;
  };
  if (res) {
    uint32_t mb[LY::RES];
    if (have_pre) {
      static_assert(LY::RES <= 3, "NodePre holds the mask bytes of three chunks");
      mb[0] = pre_masks(A, nrd, 0, pre.m00, pre.m01);
      if constexpr (LY::RES > 1) mb[1] = pre_masks(A, nrd, 1, pre.m10, pre.m11);
      if constexpr (LY::RES > 2) mb[2] = pre_masks(A, nrd, 2, pre.m20, pre.m21);
    } else {
#pragma unroll
      for (int c = 0; c < LY::RES; ++c) {
        mb[c] = 0;
        if (c < nch) {
          node_issue<D>(A, g, kChunk * c, kv, c, w);
          mb[c] = node_masks(A, p0, nrd, w, kChunk * c);
        }
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      lds_barrier();
    }
#pragma unroll
    for (int c = 0; c < LY::RES; ++c)
      if (c < nch) node_scores<D, LY::SR>(A, kChunk * c, LY::kbuf(kv, c), S + kChunk * c, w, qf);
    if (w == 0) {
      // The zero V row (2 D bytes).
      for (int b = 4 * lane; b < 2 * D; b += 256) *(lds_u32*)(kv + LY::ZOFF + b) = 0u;
    }
    lds_barrier();
    node_rank_rows<D, LY>(A, p0, nrd, kv, w, nch, mb);
  } else if (kVRes && vres) {
    using VL = VResLds<D>;
    // V-resident: every chunk's V rows DMA'd into LDS, the scores of the
    // wave's 16-slot tiles (w, w + 8, ...) from K fragments loaded into
    // registers -- all loads issued before the first wait.
    constexpr int DQ = D / 32, RB = 2 * D, VX = VL::CB / 1024;
    constexpr int MT = (VL::RES * kChunk / 16 + nw - 1) / nw;   // tiles per wave
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(A.kn + g * A.sknh, 2 * ((NN - 1) * A.sknn + D));
    const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(A.vn + g * A.svnh, 2 * ((NN - 1) * A.svnn + D));
    const int n16 = lane & 15, g4 = lane >> 4;
    const int nt = (NN + 15) / 16;
    u32x4 kf[MT][DQ];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int slot = 16 * (w + nw * j) + n16;   // slots past NN read zeros
#pragma unroll
      for (int i = 0; i < DQ; ++i)
        kf[j][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rk, w + nw * j < nt ? 2 * (slot * A.sknn + 32 * i + 8 * g4) : 0x7ffffff0,
                                                  0, 0));
    }
    for (int x = w; x < nch * VX; x += nw) {
      const int c = x / VX;
      const int byte = (x - c * VX) * 1024 + 16 * lane;
      const int row = byte / RB, u = (byte % RB) / 16;
      bdma16(rv, 2 * (kChunk * c + row) * A.svnn + 16 * (u ^ vswz<D>(row)), VL::vbuf(kv, c) + (x - c * VX) * 1024);
    }
    uint32_t mb[VL::RES];
#pragma unroll
    for (int c = 0; c < VL::RES; ++c) mb[c] = c < nch ? node_masks(A, p0, nrd, w, kChunk * c) : 0u;
    lds_float* SV = (lds_float*)(kv + VL::SOFF);
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int tt = w + nw * j;
      if (tt < nt) {
        f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[j][i]), qf[i], sv, 0, 0, 0);
        // Lane (n16, g4), element j: slot 16 tt + 4 g4 + j of row p0 + n16 (the chain of node_scores).
        *(lds_f32x4*)(SV + n16 * VL::SR + 16 * tt + 4 * g4) = sv * A.c;
      }
    }
    if (w == 0) {
      for (int b = 4 * lane; b < 2 * D; b += 256) *(lds_u32*)(kv + VL::ZOFF + b) = 0u;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's V rows
    lds_barrier();
    node_rank_rows<D, VL>(A, p0, nrd, kv, w, nch, mb);
  } else {
    // Streaming: the scores of up to SUP slots at a time into the KB / VB area
    // ([row][SUP + 4] fp32), from K fragments loaded straight into registers
    // (16-slot tiles, waves w, w + 8, ...), the rows' mask bits beside them; then
    // each row's maximum, mask words and count.
    constexpr int DQ = D / 32;
    constexpr int SUP = ((2 * LY::RES * LY::CB) / (kNodeRows * 4) - 4) / kChunk * kChunk;
    constexpr int SRS = SUP + 4;
    static_assert(kNodeRows * SRS * 4 <= 2 * LY::RES * LY::CB && SUP / kChunk <= 32, "super-chunk scores fit KB + VB");
    lds_float* SS = (lds_float*)(kv + LY::KOFF);
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(A.kn + g * A.sknh, 2 * ((NN - 1) * A.sknn + D));
    const int n16 = lane & 15, g4 = lane >> 4;
    for (int s0 = 0; s0 < NN; s0 += SUP) {
      const int ns = min(SUP, NN - s0);
      if (s0 > 0) lds_barrier();   // every wave is done with the previous super-chunk's scores
      uint32_t mbits[kNodeRounds] = {};
      for (int c = 0; c < ns / kChunk + (ns % kChunk != 0); ++c) {
        const uint32_t mb = node_masks(A, p0, nrd, w, s0 + kChunk * c);
#pragma unroll
        for (int i = 0; i < kNodeRounds; ++i) mbits[i] |= (uint32_t)(((mb >> (8 * i)) & 0xff) != 0) << c;
      }
      const int nt = (ns + 15) / 16;
      for (int tt = w; tt < nt; tt += nw) {
        const int slot = s0 + 16 * tt + n16;
        const int sr = slot < NN ? slot : 0;
        u32x4 kf[DQ];
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          kf[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rk, 2 * (sr * A.sknn + 32 * i + 8 * g4), 0, 0));
        f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < DQ; ++i)
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[i]), qf[i], sv, 0, 0, 0);
        // Lane (n16, g4), element j: slot s0 + 16 tt + 4 g4 + j of row p0 + n16.
        *(lds_f32x4*)(SS + n16 * SRS + 16 * tt + 4 * g4) = sv * A.c;
      }
      lds_barrier();
#pragma unroll 1
      for (int i = 0; i < nrd; ++i) {
        const int row = w + nw * i;
        float x = kNegInf;
        for (int c = 0; c * kChunk < ns; ++c) {
          const bool ok = (mbits[i] >> c) & 1;
          x = fmaxf(x, ok ? SS[row * SRS + kChunk * c + lane] : kNegInf);
          row_words(i, (s0 / kChunk) + c, ok ? 0xffu << (8 * i) : 0u, x);
        }
        const float m = max64(x);
        if (lane == 0) NP[row * LY::NPROW] = s0 == 0 ? m : fmaxf(NP[row * LY::NPROW], m);
      }
    }
  }
  lds_barrier();   // scores, maxima, mask words and counts visible; KB / VB free when streaming

  if (res) {
    node_res_tasks<D, LY>(A, g, p0, rend, kv, w, nch, qf);
  } else if (kVRes && vres) {
    node_res_tasks<D, VResLds<D>>(A, g, p0, rend, kv, w, nch, qf);
  } else if (w < LY::STAGES) {
    // D = 256: two d-slices per group (each recomputes the same scores), so a
    // task's accumulators and K fragments fit the registers.
    constexpr int SL = D >= 256 ? 2 : 1;
    for (int task = w; task < ng * SL; task += LY::STAGES)
      node_task<D, false, DT / SL>(A, g, p0, rend, q0 + task / SL, task / SL, task % SL, kv, w, nch, qf);
  }
  lds_barrier();   // every row's partial is in NP
  return (const lds_float*)(kv + (vres ? VResLds<D>::NPOFF : LY::NPOFF));
}

// Issues node_rows' loads of a resident segment (0 < NN <= RES kChunk,
// p0 < rend): chunk c into buffer c, the mask bytes and the score fragment.
// qreg (not null): the score fragment from prompt_block's Q fragments in LDS
// (KEEP_Q), rows from row0, instead of from memory.
// The mask bytes of node_prefetch.
template <int D>
__device__ __forceinline__ void node_prefetch_masks(const TrieAttnArgs& A, int p0, int rend, int w, NodePre<D>& pre) {
  constexpr int nw = kWavesA;
  const int nrd = (rend - p0 - w + nw - 1) / nw;
  // Mask byte of round i, chunk c: row p0 + w + 8 i (p0 past the wave's rows),
  // slot c kChunk + lane clamped into [0, NN); node_rows zeroes what is out of range.
  auto raw = [&](int c, int i) -> uint32_t {
    const int t = min(c * kChunk + (int)__lane_id(), A.NN - 1);
    const int r = i < nrd ? p0 + w + kWavesA * i : p0;
    return A.msk[(r >> A.GQS) * A.smm + t * A.smn];
  };
  pre.m00 = raw(0, 0);
  pre.m01 = raw(0, 1);
  if constexpr (NodeLds<D>::RES > 1) {
    pre.m10 = raw(1, 0);
    pre.m11 = raw(1, 1);
  }
  if constexpr (NodeLds<D>::RES > 2) {
    pre.m20 = raw(2, 0);
    pre.m21 = raw(2, 1);
  }
}

template <int D>
__device__ __forceinline__ void node_prefetch(const TrieAttnArgs& A, int g, int p0, int rend, lds_char* kv, int w,
                                              NodePre<D>& pre, const lds_char* qreg = nullptr, int row0 = 0) {
  for (int b = 0; b < NodeLds<D>::RES && b * kChunk < A.NN; ++b) node_issue<D>(A, g, b * kChunk, kv, b, w);
  node_prefetch_masks<D>(A, p0, rend, w, pre);
  if (qreg) node_q_lds<D>(qreg, row0, p0, rend, pre.qf);
  else node_q<D>(A, g, p0, rend, pre.qf);
}


// Columns per lane when one wave merges one row (D = 32: half the wave).
template <int D> constexpr int merge_cols() { return D >= 64 ? D / 64 : 1; }

// Final result of row r of kv head g, one row over the wave (lane l < D / DL:
// head_dim [DL l, +DL)): the group partials combined in group order, then the
// node partial (m, l, acc); bf16 store.
template <int D, bool COH = false>
__device__ __forceinline__ void merge_row(const TrieAttnArgs& A, int g, int r, float m, float l,
                                          const float (&acc)[merge_cols<D>()]) {
  constexpr int DL = merge_cols<D>();
  const int lane = __lane_id();
  const bool on = DL * lane < D;
  const int ln = on ? lane : 0;   // lanes past the row read lane 0's columns and store nothing
  const RowRef R = row_ref(A, g, r, r);
  const int NG = A.NG;
  float gm[kGroupTarget], gl[kGroupTarget], ga[kGroupTarget][DL];
  const size_t gbase = ((size_t)g * A.R + r) * NG;
  // Byte offsets of the partials fit 31 bits (checked by the host for COH).
  const __amdgpu_buffer_rsrc_t rml = buffer_rsrc(A.gp_ml, 0x7fffffff);
  const __amdgpu_buffer_rsrc_t racc = buffer_rsrc(A.gp_acc, 0x7fffffff);
  // Every group slot loads, with no branch around a load (groups past NG
  // re-read group NG - 1 and are not combined): a load under a branch makes
  // the compiler wait for the loads before it at the branch's join, which
  // split these loads into several memory round trips.
#pragma unroll
  for (int qq = 0; qq < kGroupTarget; ++qq) {
    {
      const int qc = qq < NG ? qq : NG - 1;
      const size_t ao = (gbase + qc) * D + DL * ln;
      if constexpr (COH) {
        // sc1 (cache policy 16): the coherence of an agent-scope atomic load.
        const f32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(rml, (int)((gbase + qc) * 8), 0, 16);
        gm[qq] = ml.x;
        gl[qq] = ml.y;
        if constexpr (DL == 4) {
          const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(racc, (int)(ao * 4), 0, 16));
#pragma unroll
          for (int k = 0; k < 4; ++k) ga[qq][k] = a[k];
        } else if constexpr (DL == 2) {
          const f32x2 a = __builtin_amdgcn_raw_buffer_load_b64(racc, (int)(ao * 4), 0, 16);
          ga[qq][0] = a.x;
          ga[qq][1] = a.y;
        } else {
          ga[qq][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(racc, (int)(ao * 4), 0, 16));
        }
      } else {
        const float2 ml = *reinterpret_cast<const float2*>(A.gp_ml + (gbase + qc) * 2);
        gm[qq] = ml.x;
        gl[qq] = ml.y;
#pragma unroll
        for (int k = 0; k < DL; ++k) ga[qq][k] = A.gp_acc[ao + k];
      }
    }
  }
  float fm = kNegInf, fl = 0.f, facc[DL];
#pragma unroll
  for (int k = 0; k < DL; ++k) facc[k] = 0.f;
#pragma unroll
  for (int qq = 0; qq < kGroupTarget; ++qq)
    combine<DL>(fm, fl, facc, qq < NG ? gm[qq] : kNegInf, gl[qq], ga[qq]);   // past NG: left out
  combine<DL>(fm, fl, facc, m, l, acc);
  if (!on) return;
  uint16_t* o = A.out + out_offset<D>(A.soh, A.som, A.HK << A.GQS, R.hd, R.mq, DL * lane);
  if constexpr (DL == 4)
    *reinterpret_cast<u32x2*>(o) = u32x2{pack_bf16x2(facc[0] / fl, facc[1] / fl), pack_bf16x2(facc[2] / fl, facc[3] / fl)};
  else if constexpr (DL == 2) *reinterpret_cast<uint32_t*>(o) = pack_bf16x2(facc[0] / fl, facc[1] / fl);
  else *o = f32_to_bf16_rne(facc[0] / fl);
}

// The node partial of wave w's round i, left in LDS by node_rows in the rows
// NP[i][D + 4] = (m, l, pad, pad, acc) (empty when there are no node slots),
// merged into row p0 + w + 8 i.
template <int D, bool COH>
__device__ __forceinline__ void merge_rounds(const TrieAttnArgs& A, int g, int p0, int rend, const lds_float* NP,
                                             int w) {
  constexpr int DL = merge_cols<D>();
  const int lane = __lane_id();
  const int ln = DL * lane < D ? lane : 0;
  const int nrd = (rend - p0 - w + kWavesA - 1) / kWavesA;
  using LY = NodeLds<D>;
#pragma unroll 1
  for (int i = 0; i < nrd; ++i) {
    const int row = w + kWavesA * i;
    float m = kNegInf, l = 0.f, acc[DL];
#pragma unroll
    for (int k = 0; k < DL; ++k) acc[k] = 0.f;
    if (A.NN > 0) {
      const lds_float* np = NP + row * LY::NPROW;
      m = np[0];
      l = np[1];
#pragma unroll
      for (int k = 0; k < DL; ++k) acc[k] = np[4 + DL * ln + k];
    }
    merge_row<D, COH>(A, g, p0 + row, m, l, acc);
  }
}

// ------------------------------------------------------------------ kernel B
// Workgroup (g, c8): rows [8 c8, 8 c8 + 8) of kv head g, row 8 c8 + w on
// wave w: node partial, then merge.  A node segment of at most RES chunks
// is loaded whole up front; a longer one streams.
template <int D>
__global__ __launch_bounds__(64 * kWavesA) void node_merge_kernel(TrieAttnArgs A) {
  using LY = NodeLds<D>;
  static_assert(8 <= kNodeRows, "a workgroup's rows fit the node areas");
  __shared__ __attribute__((aligned(16))) char kv[node_area_bytes<D>()];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int RC8 = (A.R + 7) / 8;
  const int g = blockIdx.x / RC8;
  const int p0 = 8 * (blockIdx.x - g * RC8);
  const int rend = min(p0 + 8, A.R);
  NodePre<D> pre;
  const bool pf = A.NN > 0 && A.NN <= LY::RES * kChunk;
  if (pf) {
    node_prefetch<D>(A, g, p0, rend, (lds_char*)kv, w, pre);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's part of the segment is in LDS
    lds_barrier();                       // and every other wave's part
  }
  const lds_float* np = node_rows<D>(A, g, p0, rend, (lds_char*)kv, w, pre, pf);
  merge_rounds<D, false>(A, g, p0, rend, np, w);
}

// NaN in every element of rows [p0, rend) of kv head g (row p0 + w + 8 i on
// wave w): the output of a workgroup whose wait for the group partials gave up.
template <int D>
__device__ __forceinline__ void nan_rows(const TrieAttnArgs& A, int g, int p0, int rend, int w) {
  constexpr int DL = merge_cols<D>();
  const int lane = __lane_id();
  if (DL * lane >= D) return;
  for (int r = p0 + w; r < rend; r += kWavesA) {
    const RowRef R = row_ref(A, g, r, r);
    uint16_t* o = A.out + out_offset<D>(A.soh, A.som, A.HK << A.GQS, R.hd, R.mq, DL * lane);
    if constexpr (DL == 4) *reinterpret_cast<u32x2*>(o) = u32x2{0x7fc07fc0u, 0x7fc07fc0u};
    else if constexpr (DL == 2) *reinterpret_cast<uint32_t*>(o) = 0x7fc07fc0u;
    else *o = (uint16_t)0x7fc0;
  }
}

// ------------------------------------------------------------------ fused kernel
// One launch: workgroup (g, rb, q) runs prompt_block, counts itself in
// cnt[g][rb], computes the node partials of its share of the block's rows --
// rows q RPW .. q RPW + RPW - 1 of the block, row r0 + w + 8 i on wave w --
// and, once all NG groups of the block are counted, merges those rows.  Every
// workgroup of the grid is resident at once (the host launches this kernel
// only when the grid fits), so the wait always ends; it is also bounded
// (A.spin polls), and a workgroup whose wait gives up stores NaN in every
// element of the rows it would merge -- the failure reaches the caller's
// output without a host synchronisation -- and raises a flag the host can
// read.  Counters are never reset: every call moves each block's counter by
// exactly kCountUnit, whether or not a wait gave up (see kCountUnit).
//
// The wait is bounded in time: kWaitMs milliseconds of the device's
// constant-rate real-time counter (s_memrealtime, hipDeviceAttributeWallClockRate
// kHz), far beyond a call's normal length (tens of microseconds), short enough
// that a broken co-residency surfaces as a failed call instead of a stall.
//
// Visibility without cache-wide fences: every word that crosses workgroups
// (group partials, counters) is written by an agent-scope atomic store or
// read-modify-write and read by a load with the same coherence bit (sc1) as an
// agent-scope atomic load, so no access depends on an L2 write-back or
// invalidate.  Order: each wave waits for its own partial stores to complete
// (vmcnt 0) before the workgroup barrier that precedes the counter increment;
// the partial loads are issued only after the counter load that released the
// wait has returned.  A release/acquire pair at agent scope (buffer_wbl2 and
// buffer_inv of the whole L2) would order the same accesses at several
// microseconds per workgroup.
constexpr int kSpinLimit = 0x7fffffff;   // no poll bound of its own: the deadline ends a wait
constexpr int kWaitMs = 4;
// Polls before a fused launch's wait gives up (rspx_trie_attn_set_spin_limit
// lowers it so tests can exercise the give-up path with every kernel exiting).
static int g_spin_limit = kSpinLimit;

// kWaitMs in s_memrealtime ticks of the current device (100 MHz if the rate
// cannot be queried).
static int wait_deadline_ticks() {
  static int ticks[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kWaitMs * 100000;
  if (ticks[dev] == 0) {
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) khz = 100000;
    const int64_t t = (int64_t)khz * kWaitMs;
    ticks[dev] = (int)(t < 0x7fffffff ? t : 0x7fffffff);
  }
  return ticks[dev];
}
constexpr int kSyncWords = 4096;   // timeout flag + [HK][NRB][2] counters (the second word of each pair unused)
// Every one-launch call adds exactly kCountUnit to the counter of each row
// block it computes: the block's NG workgroups add kCountUnit / NG each, the
// first kCountUnit % NG of them one more (NG <= kGroupTarget = kCountUnit).
// So between calls every counter is a multiple of kCountUnit, and a workgroup
// of call k that reads its block's counter before adding its own share sees a
// value in [kCountUnit k, kCountUnit (k + 1)): no call ever resets a counter,
// and calls of any shapes may share the words in turn.
constexpr uint32_t kCountUnit = kGroupTarget;
static_assert((kCountUnit & (kCountUnit - 1)) == 0, "2^32 is a multiple of the unit: wrap-around keeps the invariant");

// Rows [r0, rend) merged by workgroup (g, rb, q) of a fused launch: its share
// of the row block, a multiple of 4 rows.
template <int kRT>
__device__ __forceinline__ void merge_share(const TrieAttnArgs& A, int rb, int q, int& r0, int& rend) {
  const int rows_blk = 32 * kRT;
  // ceil(rows_blk / 4 / NG) for NG = 1 .. kGroupTarget, 5 bits each: no division.
  constexpr int a = rows_blk / 4;
  constexpr uint64_t tab = [] {
    uint64_t t = 0;
    for (int n = 1; n <= kGroupTarget; ++n) t |= (uint64_t)((a + n - 1) / n) << (5 * n);
    return t;
  }();
  static_assert(a < 32, "5-bit table entries");
  const int rpw = 4 * (int)((tab >> (5 * A.NG)) & 31);
  r0 = rb * rows_blk + q * rpw;
  rend = min(rb * rows_blk + min(rows_blk, (q + 1) * rpw), A.R);
}

// After workgroup (g, rb, q) has counted its group partial of row block rb:
// the node partials of its merge rows [r0, rend) of that block in batches of
// at most kNodeRows (the first batch while the block's other workgroups
// finish, then the bounded wait), then the merge.  pre / pf: node_rows'
// first batch.  old: the counter before this workgroup's share
// (counter_before), so the block is complete once the counter has moved
// kCountUnit past the multiple of kCountUnit below it.
template <int D, int kRT>
__device__ __forceinline__ void block_tail(const TrieAttnArgs& A, char* lds, int g, int rb, int q, int r0, int rend,
                                           const NodePre<D>& pre, bool pf, int old) {
  const int lane = __lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int* cnt = A.sync + 1 + 2 * (g * A.NRB + rb);
  const int rend0 = min(rend, r0 + kNodeRows);
  int* gave_up = reinterpret_cast<int*>(lds + node_area_bytes<D>());  // one LDS word past the node areas
  if (r0 < rend) {
    const lds_float* np = node_rows<D>(A, g, r0, rend0, (lds_char*)lds, w, pre, pf);
    RSPX_MARK(12);
    if (w == 0) {
      // Bounded in time (A.deadline ticks of the constant-rate real-time
      // counter) and in polls (A.spin, lowered only by a test hook).
      const uint32_t base = (uint32_t)__builtin_amdgcn_readfirstlane(old) & ~(kCountUnit - 1);
      uint32_t v = base;
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (int it = 0; it < A.spin; ++it) {
        v = (uint32_t)__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v - base >= kCountUnit) break;
        if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)A.deadline) break;
        __builtin_amdgcn_s_sleep(2);
      }
      const bool short_ = v - base < kCountUnit;
      if (lane == 0) {
        *gave_up = short_;
        if (short_) __hip_atomic_store(A.sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    lds_barrier();
    RSPX_MARK(13);
    const bool bad = __builtin_amdgcn_readfirstlane(*gave_up);
    if (bad) nan_rows<D>(A, g, r0, rend0, w);
    else merge_rounds<D, true>(A, g, r0, rend0, np, w);
    RSPX_MARK(14);
    // Further batches (short prompts: few key groups, many rows per workgroup).
    for (int b0 = rend0; b0 < rend; b0 += kNodeRows) {
      const int be = min(rend, b0 + kNodeRows);
      NodePre<D> none;
      const lds_float* npb = node_rows<D>(A, g, b0, be, (lds_char*)lds, w, none, false);
      if (bad) nan_rows<D>(A, g, b0, be, w);
      else merge_rounds<D, true>(A, g, b0, be, npb, w);
    }
  }
  RSPX_MARK(15);
}

// Adds workgroup q's share of kCountUnit to row block rb's counter, from the
// last wave (waves 0-3 score the node slots next, and a wave with the add in
// flight would wait for it at its first vmcnt wait).  Every wave's stores of
// the group partial must be complete (each wave's vmcnt(0), then a barrier).
__device__ __forceinline__ void count_add(const TrieAttnArgs& A, int g, int rb, int q) {
  if (threadIdx.x == 64 * (kWavesA - 1)) {
    const int share = (int)kCountUnit / A.NG + (q < (int)kCountUnit % A.NG ? 1 : 0);
    __hip_atomic_fetch_add(A.sync + 1 + 2 * (g * A.NRB + rb), share, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The group partial is complete in memory (each wave waited for its own
// stores): add workgroup q's share of kCountUnit to the row block's counter.
__device__ __forceinline__ void count_partial(const TrieAttnArgs& A, int g, int rb, int q) {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are complete
  lds_barrier();
  RSPX_MARK(11);
  count_add(A, g, rb, q);
}

// The row block's counter as this workgroup finds it before adding its own
// share (read at the kernel's start): in [kCountUnit k, kCountUnit (k + 1))
// during call k.  Every lane loads it, with no branch around the load, so the
// value is waited for only where block_tail uses it (a value merged from a
// branch is copied, and the copy waits for the load).
__device__ __forceinline__ int counter_before(const TrieAttnArgs& A, int g, int rb) {
  return __hip_atomic_load(A.sync + 1 + 2 * (g * A.NRB + rb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int kRT>
__global__ __launch_bounds__(512) void fused_kernel(TrieAttnArgs A) {
  using LY = NodeLds<D>;
  using PL = PromptLds<D, kRT>;
  constexpr int NB = node_area_bytes<D>() + 16;
  constexpr int LB = PL::BYTES + PL::MLBYTES > NB ? PL::BYTES + PL::MLBYTES : NB;
  static_assert(NB <= PL::RINGBYTES, "node LDS and the wait flag inside the ring (the Q fragments stay)");
  __shared__ __attribute__((aligned(16))) char lds[LB];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x, rb = blockIdx.y, q = blockIdx.z;
  RSPX_MARK(0);
  // Every argument the prologue needs, requested in one batch: left to the
  // compiler, they came in three dependent scalar-load round trips before the
  // first K/V request.
  asm volatile("" ::"s"(A.q), "s"(A.kp), "s"(A.vp), "s"(A.sync), "s"(A.sqh), "s"(A.sqm), "s"(A.skph), "s"(A.skpn),
               "s"(A.svph), "s"(A.svpn), "s"(A.P), "s"(A.NRB), "s"(A.NG), "s"(A.S), "s"(A.R), "s"(A.GQS));
  int r0, rend;
  merge_share<kRT>(A, rb, q, r0, rend);
  const int rend0 = min(rend, r0 + kNodeRows);               // the first batch of node rows
  const int old = counter_before(A, g, rb);

  // A resident node segment (K/V, score fragment, mask bytes of the first
  // batch) is loaded while the group partial is being stored.  Up to
  // D = 128 the first chunk's K/V and the mask bytes are requested into
  // registers before the quarter combine (whose LDS traffic they then
  // overlap) and written into the ring after it.
  const bool pf = A.NN > 0 && A.NN <= LY::RES * kChunk && r0 < rend;
  constexpr bool kEarly = D <= 128;
  NodePre<D> pre;
  u32x4 pc[node_pieces<D>()];
  const lds_char* qreg = (const lds_char*)lds + PL::RINGBYTES;
  prompt_block<D, kRT, true, false, true>(
      A, lds, g, rb, q,
      [&] {
        if constexpr (kEarly) {
          // Unconditional, so that no path leaves the register loads pending
          // (without a prefetch the node phase overwrites these bytes).
          node_put<D>(A, g, 0, (lds_char*)lds, 0, pc, w);
          if (!pf) return;
          for (int b = 1; b < LY::RES && b * kChunk < A.NN; ++b) node_issue<D>(A, g, b * kChunk, (lds_char*)lds, b, w);
          node_q_lds<D>(qreg, rb * 32 * kRT, r0, rend0, pre.qf);
        } else {
          if (pf) node_prefetch<D>(A, g, r0, rend0, (lds_char*)lds, w, pre, qreg, rb * 32 * kRT);
        }
      },
      [&] {
        if constexpr (kEarly) {
          if (pf) {
            node_load<D>(A, g, 0, pc, w);
            node_prefetch_masks<D>(A, r0, rend0, w, pre);
          }
        }
      },
      [] {});
  count_partial(A, g, rb, q);
  block_tail<D, kRT>(A, lds, g, rb, q, r0, rend, pre, pf, old);
}

// The same work as fused_kernel for grids twice as large as the device holds
// at once (e.g. 128-node tries at 8B heads: 512 rows per kv head): workgroup
// (g, rbw, q) runs the prompt groups of row blocks rbw and rbw + NRBW
// (NRBW = ceil(NRB / 2)) one after the other, counting each, then the node
// partials and merges of its merge rows (its shares of both blocks, or with
// NG = 2, 4 or 8 twice a share of one block).  Every count precedes every
// wait, so the waits end as in fused_kernel; the arithmetic of every row is
// the same: the same bits.
template <int D, int kRT>
__global__ __launch_bounds__(512) void fused2_kernel(TrieAttnArgs A) {
  using LY = NodeLds<D>;
  using PL = PromptLds<D, kRT>;
  constexpr int NB = node_area_bytes<D>() + 16;
  constexpr int LB = PL::BYTES + PL::MLBYTES > NB ? PL::BYTES + PL::MLBYTES : NB;
  static_assert(NB <= PL::RINGBYTES, "node LDS and the wait flag inside the ring (the Q fragments stay)");
  __shared__ __attribute__((aligned(16))) char lds[LB];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x, rbw = blockIdx.y, q = blockIdx.z;
  // Every argument the prologue needs, requested in one batch.
  asm volatile("" ::"s"(A.q), "s"(A.kp), "s"(A.vp), "s"(A.sync), "s"(A.sqh), "s"(A.sqm), "s"(A.skph), "s"(A.skpn),
               "s"(A.svph), "s"(A.svpn), "s"(A.P), "s"(A.NRB), "s"(A.NG), "s"(A.S), "s"(A.R), "s"(A.GQS));
  const int NRBW = (A.NRB + 1) / 2;
  const int nb = rbw + NRBW < A.NRB ? 2 : 1;
  const int rb1 = nb > 1 ? rbw + NRBW : rbw;
  const int old[2] = {counter_before(A, g, rbw), counter_before(A, g, rb1)};
  // With two blocks and NG = 2, 4 or 8 the merges are split by workgroup, not
  // by block: workgroup q merges 2 (32 kRT) / NG consecutive rows of one block
  // (block rbw for q < NG / 2, block rb1 above), so it has one node phase, one
  // wait and one merge for twice the rows of a block's share.  With a resident
  // node segment (up to D = 128) its node data is requested during the second
  // block's prompt part: the first chunk's K/V into registers before that
  // block's quarter combine (written into the ring after it, further chunks as
  // direct-to-LDS loads) with the rows' mask bytes, and the score fragment from
  // memory (rows of block rbw) or from the second block's Q fragments, kept in
  // LDS (rows of block rb1).
  constexpr bool kEarly = D <= 128;
  const int rows_blk = 32 * kRT;
  const bool pairs = nb > 1 && (A.NG == 2 || A.NG == 4 || A.NG == 8);
  const bool second = pairs && q >= (A.NG >> 1);
  const int mrb = second ? rb1 : rbw;            // the block whose rows this workgroup merges (pairs)
  int m0 = 0, mend = 0;
  if (pairs) {
    const int rpw2 = 2 * rows_blk / A.NG;        // 16 .. 64 rows, a multiple of 4 dividing the block
    m0 = mrb * rows_blk + (second ? q - (A.NG >> 1) : q) * rpw2;
    mend = min(m0 + rpw2, A.R);
  }
  const int mend0 = min(mend, m0 + kNodeRows);
  const bool pf = kEarly && pairs && A.NN > 0 && A.NN <= LY::RES * kChunk && m0 < mend;
  NodePre<D> pre;
  u32x4 pc[node_pieces<D>()];
  const lds_char* qreg = (const lds_char*)lds + PL::RINGBYTES;
  prompt_block<D, kRT, true, true>(A, lds, g, rbw, q, [] {}, [] {}, [] {});
  // With a second block the first block's count waits for nothing: it is added
  // once the second block's round 0 has landed, by when the first block's
  // stores (issued before that round's loads) are complete in every wave.
  if (nb == 1) count_partial(A, g, rbw, q);
  if (nb > 1) {
    prompt_block<D, kRT, true, false, true>(
        A, lds, g, rb1, q,
        [&] {
          if constexpr (kEarly) {
            // Unconditional, so that no path leaves the register loads pending.
            node_put<D>(A, g, 0, (lds_char*)lds, 0, pc, w);
            if (!pf) return;
            for (int b = 1; b < LY::RES && b * kChunk < A.NN; ++b) node_issue<D>(A, g, b * kChunk, (lds_char*)lds, b, w);
          }
        },
        [&] {
          if constexpr (kEarly) {
            if (pf) {
              node_load<D>(A, g, 0, pc, w);
              node_prefetch_masks<D>(A, m0, mend0, w, pre);
              if (!second) node_q<D>(A, g, m0, mend0, pre.qf);
            }
          }
        },
        [&] { count_add(A, g, rbw, q); });
    count_partial(A, g, rb1, q);
    if constexpr (kEarly)
      if (pf && second) node_q_lds<D>(qreg, rb1 * rows_blk, m0, mend0, pre.qf);
  }
  if (pairs) {
    block_tail<D, kRT>(A, lds, g, mrb, q, m0, mend, pre, pf, second ? old[1] : old[0]);
  } else {
    NodePre<D> none;
    int r0, rend;
    merge_share<kRT>(A, rbw, q, r0, rend);
    block_tail<D, kRT>(A, lds, g, rbw, q, r0, rend, none, false, old[0]);
    if (nb > 1) {
      merge_share<kRT>(A, rb1, q, r0, rend);
      block_tail<D, kRT>(A, lds, g, rb1, q, r0, rend, none, false, old[1]);
    }
  }
}

// ------------------------------------------------------------------ host side

struct Plan {
  int GQA, R, RT, NRB, NG, S, prompt_wgs, node_wgs;
  size_t off_gp_ml, off_gp_acc, off_sync, total;
};

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

template <int D, int RT, bool TWO = false>
static int fused_capacity();

// Steps per group S = 4 NR and the group count NG <= 8 depend on P only.
static int make_plan(int H, int HK, int M, int P, int NN, int D, int rows_per_wave, Plan* pl) {
  if (H <= 0 || HK <= 0 || M < 0 || P < 0 || NN < 0 || H % HK != 0) return RSPX_EINVAL;
  if (NN > kMaxNodeSlots) return RSPX_EINVAL;
  if (D != 32 && D != 64 && D != 128 && D != 256) return RSPX_EUNSUPPORTED;
  const int GQA = H / HK;
  if (GQA != 1 && GQA != 2 && GQA != 4 && GQA != 8 && GQA != 16) return RSPX_EUNSUPPORTED;
  pl->GQA = GQA;
  pl->R = M * GQA;
  if (P > 0) {
    const int steps = (P + kStep - 1) / kStep;
    const int nr = (steps + kQuarters * kGroupTarget - 1) / (kQuarters * kGroupTarget);
    pl->S = kQuarters * nr;
    pl->NG = (steps + pl->S - 1) / pl->S;
  } else {
    pl->S = kQuarters;
    pl->NG = 0;
  }
  int rt = rows_per_wave;
  if (rt == 0) {
    // One 16-row tile per wave while that grid (twice as many row blocks)
    // still fits on the device at once, else two: the same bits either way.
    // D = 256 always takes one (two tiles of 256 columns exceed the registers).
    const int nrb1 = (pl->R + 31) / 32;
    const int cap1 = D == 256 ? 0
                     : D == 128 ? fused_capacity<128, 1>()
                     : D == 64  ? fused_capacity<64, 1>()
                                : fused_capacity<32, 1>();
    rt = (D == 256 || (pl->NG > 0 && HK * nrb1 * pl->NG <= cap1)) ? 1 : 2;
  }
  if (rt != 1 && rt != 2) return RSPX_EINVAL;
  if (D == 256 && rt != 1) return RSPX_EUNSUPPORTED;
  pl->RT = rt;
  pl->NRB = (pl->R + 32 * rt - 1) / (32 * rt);
  if (pl->NRB > 65535) return RSPX_EUNSUPPORTED;   // the grid's y dimension (row blocks)
  pl->prompt_wgs = HK * pl->NRB * pl->NG;
  pl->node_wgs = HK * ((pl->R + 7) / 8);
  const size_t parts = (size_t)HK * pl->R * pl->NG;
  // The synchronisation words sit at the start, at the same place for every
  // shape, so a workspace shared by calls of different shapes never holds
  // another call's partials where a call expects zero counters.
  size_t off = 0;
  pl->off_sync = off;   off = align256(off + kSyncWords * sizeof(int));
  pl->off_gp_ml = off;  off = align256(off + parts * 2 * sizeof(float));
  pl->off_gp_acc = off; off = align256(off + parts * D * sizeof(float));
  pl->total = off;
  return RSPX_OK;
}

// Workgroups of fused_kernel<D, RT> (TWO: fused2_kernel<D, RT>) the device
// holds at once (0 if unknown).
template <int D, int RT, bool TWO>
static int fused_capacity() {
  static int cap[64];
  static bool done[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!done[dev]) {
    int a = 0, cus = 0;
    hipError_t e;
    if constexpr (TWO) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, fused2_kernel<D, RT>, 64 * kWavesA, 0);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, fused_kernel<D, RT>, 64 * kWavesA, 0);
    if (e != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      a = cus = 0;
    }
    cap[dev] = a * cus;
    done[dev] = true;
  }
  return cap[dev];
}


template <int D, int RT>
static void launch_rt(const TrieAttnArgs& a, const Plan& pl, hipStream_t s, int mode) {
  const bool one = pl.NG > 0 && mode != 2 && 1 + 2 * pl.NRB * a.HK <= kSyncWords &&
                   (size_t)a.HK * pl.R * pl.NG * D * sizeof(float) < (size_t(1) << 31);
  const int cap = one ? fused_capacity<D, RT>() : 0;
  if (one && pl.prompt_wgs <= cap) {
    hipLaunchKernelGGL((fused_kernel<D, RT>), dim3(a.HK, pl.NRB, pl.NG), dim3(64 * kWavesA), 0, s, a);
    return;
  }
  // Two row blocks per workgroup (fused2_kernel) when that grid fits.
  const int wgs2 = a.HK * ((pl.NRB + 1) / 2) * pl.NG;
  if (one && pl.NRB > 1 && wgs2 <= fused_capacity<D, RT, true>()) {
    hipLaunchKernelGGL((fused2_kernel<D, RT>), dim3(a.HK, (pl.NRB + 1) / 2, pl.NG), dim3(64 * kWavesA), 0, s, a);
    return;
  }
  if (pl.prompt_wgs > 0) hipLaunchKernelGGL((prompt_kernel<D, RT>), dim3(a.HK, pl.NRB, pl.NG), dim3(64 * kWavesA), 0, s, a);
  hipLaunchKernelGGL((node_merge_kernel<D>), dim3(pl.node_wgs), dim3(64 * kWavesA), 0, s, a);
}

template <int D>
static void launch_all(const TrieAttnArgs& a, const Plan& pl, hipStream_t s, int mode) {
  if constexpr (D == 256) launch_rt<D, 1>(a, pl, s, mode);
  else if (pl.RT == 1) launch_rt<D, 1>(a, pl, s, mode);
  else launch_rt<D, 2>(a, pl, s, mode);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace rspx

using namespace rspx;

extern "C" int64_t rspx_trie_attn_workspace_bytes(int H, int HK, int M, int P, int D) {
  Plan pl;
  if (make_plan(H, HK, M, P, 0, D, 1, &pl) != RSPX_OK) return -1;
  return (int64_t)pl.total;  // independent of NN and rows_per_wave
}

static int trie_attn_impl(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                          const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh, int64_t sknn,
                          const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk, int64_t smm, int64_t smn,
                          void* out, int64_t soh, int64_t som, int H, int HK, int M, int P, int NN, int D,
                          float sm_scale, void* workspace, int64_t workspace_bytes, int rows_per_wave, void* stream,
                          int mode) {
  Plan pl;
  int rc = make_plan(H, HK, M, P, NN, D, rows_per_wave, &pl);
  if (rc != RSPX_OK) return rc;
  if (!(sm_scale > 0.f) || sm_scale == __builtin_huge_valf()) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!q || !out || (P > 0 && (!kp || !vp)) || (NN > 0 && (!kn || !vn || !msk)))
    return RSPX_EINVAL;
  if (!workspace || workspace_bytes < (int64_t)pl.total) return RSPX_EWORKSPACE;
  const void* ptrs[] = {q, kp, vp, kn, vn, out, workspace};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return RSPX_EALIGN;
  // som == RSPX_TILED: out is the [M, H D] matrix (query m, column h D + d)
  // in the tiled activation layout, ceil(M / 64) 64 H D elements; soh must
  // then be D.
  const bool out_tiled = som == kTiled;
  if (out_tiled && soh != D) return RSPX_EINVAL;
  const int64_t strides[] = {sqh, sqm, skph, skpn, svph, svpn, sknh, sknn, svnh, svnn, soh, out_tiled ? 8 : som};
  for (int64_t s : strides) {
    if (s < 0) return RSPX_EINVAL;
    if (s % 8 != 0) return RSPX_EALIGN;
  }
  if (smm < 0 || smn < 0) return RSPX_EINVAL;
  // The kernels address every tensor with 32-bit offsets: the largest element
  // offset of each must stay below 2^30 (byte offsets below 2^31).
  const int64_t lim = int64_t(1) << 30;
  auto span = [](int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t last) {
    return (n0 > 0 ? (n0 - 1) * s0 : 0) + (n1 > 0 ? (n1 - 1) * s1 : 0) + last;
  };
  if (span(H, sqh, M, sqm, D) >= lim) return RSPX_EUNSUPPORTED;
  if (out_tiled ? (int64_t)((M + 63) / 64) * 64 * H * D >= lim : span(H, soh, M, som, D) >= lim)
    return RSPX_EUNSUPPORTED;
  if (P > 0 && (span(HK, skph, P, skpn, D) >= lim || span(HK, svph, P, svpn, D) >= lim)) return RSPX_EUNSUPPORTED;
  if (NN > 0 && (span(HK, sknh, NN, sknn, D) >= lim || span(HK, svnh, NN, svnn, D) >= lim ||
                 span(M, smm, NN, smn, 1) >= lim))
    return RSPX_EUNSUPPORTED;
  // The group partials too ([HK][R][NG][D] fp32, addressed with 32-bit byte offsets).
  if ((int64_t)(pl.total - pl.off_gp_acc) >= 2 * lim) return RSPX_EUNSUPPORTED;

  TrieAttnArgs a;
  a.q = static_cast<const uint16_t*>(q);   a.sqh = (int)sqh;   a.sqm = (int)sqm;
  a.kp = static_cast<const uint16_t*>(kp); a.skph = (int)skph; a.skpn = (int)skpn;
  a.vp = static_cast<const uint16_t*>(vp); a.svph = (int)svph; a.svpn = (int)svpn;
  a.kn = static_cast<const uint16_t*>(kn); a.sknh = (int)sknh; a.sknn = (int)sknn;
  a.vn = static_cast<const uint16_t*>(vn); a.svnh = (int)svnh; a.svnn = (int)svnn;
  a.msk = msk; a.smm = (int)smm; a.smn = (int)smn;
  a.out = static_cast<uint16_t*>(out); a.soh = out_tiled ? -1 : (int)soh; a.som = out_tiled ? 0 : (int)som;
  a.HK = HK; a.GQS = __builtin_ctz(pl.GQA); a.M = M; a.P = P; a.NN = NN;
  a.R = pl.R; a.NRB = pl.NRB; a.NG = pl.NG; a.S = pl.S;
  a.c = (float)((double)sm_scale * 1.4426950408889634);
  char* ws = static_cast<char*>(workspace);
  a.gp_ml = reinterpret_cast<float*>(ws + pl.off_gp_ml);
  a.gp_acc = reinterpret_cast<float*>(ws + pl.off_gp_acc);
  a.sync = reinterpret_cast<int*>(ws + pl.off_sync);
  a.spin = g_spin_limit;
  a.deadline = wait_deadline_ticks();

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 32: launch_all<32>(a, pl, s, mode); break;
    case 64: launch_all<64>(a, pl, s, mode); break;
    case 128: launch_all<128>(a, pl, s, mode); break;
    default: launch_all<256>(a, pl, s, mode); break;
  }
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_trie_attn(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                              const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh, int64_t sknn,
                              const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk, int64_t smm,
                              int64_t smn, void* out, int64_t soh, int64_t som, int H, int HK, int M, int P, int NN,
                              int D, float sm_scale, void* workspace, int64_t workspace_bytes, int rows_per_wave,
                              void* stream) {
  return trie_attn_impl(q, sqh, sqm, kp, skph, skpn, vp, svph, svpn, kn, sknh, sknn, vn, svnh, svnn, msk, smm, smn,
                        out, soh, som, H, HK, M, P, NN, D, sm_scale, workspace, workspace_bytes, rows_per_wave,
                        stream, 0);
}

// ------------------------------------------------------------------ allocation-free variant
// A workspace that lives in the code object: one per GPU the library runs on,
// held until the process ends.  Its first kSyncWords ints are the one-launch
// synchronisation words; the group partials follow, as in a caller's
// workspace.  The array has static storage with no initialiser, so the code
// object's loader hands it over zero-filled on every device before any call
// (no fill kernel, nothing to order against the first call's stream); every
// call leaves the counters at zero again and rspx_trie_attn_status(NULL, ...)
// clears the timeout flag it reports.  In host code the array's name is only a
// stand-in: the device address comes from hipGetSymbolAddress, once per
// device, and is what kernels are given.
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// Device address of the current device's scratch (looked up on the first call
// on that device; no device work is queued).
static int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return RSPX_ELAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RSPX_ELAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return RSPX_OK;
}

extern "C" int rspx_trie_attn_noalloc(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph,
                                      int64_t skpn, const void* vp, int64_t svph, int64_t svpn, const void* kn,
                                      int64_t sknh, int64_t sknn, const void* vn, int64_t svnh, int64_t svnn,
                                      const uint8_t* msk, int64_t smm, int64_t smn, void* out, int64_t soh,
                                      int64_t som, int H, int HK, int M, int P, int NN, int D, float sm_scale,
                                      int rows_per_wave, void* stream) {
  Plan pl;
  const int rc = make_plan(H, HK, M, P, NN, D, rows_per_wave, &pl);
  if (rc != RSPX_OK) return rc;
  if (pl.total > kStaticScratchBytes) return RSPX_EWORKSPACE;
  if (M == 0) return RSPX_OK;
  void* ws = nullptr;
  const int sr = static_scratch(&ws);
  if (sr != RSPX_OK) return sr;
  return trie_attn_impl(q, sqh, sqm, kp, skph, skpn, vp, svph, svpn, kn, sknh, sknn, vn, svnh, svnn, msk, smm, smn,
                        out, soh, som, H, HK, M, P, NN, D, sm_scale, ws, (int64_t)kStaticScratchBytes, rows_per_wave,
                        stream, 0);
}

extern "C" int rspx_trie_attn_launches(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph,
                                       int64_t skpn, const void* vp, int64_t svph, int64_t svpn, const void* kn,
                                       int64_t sknh, int64_t sknn, const void* vn, int64_t svnh, int64_t svnn,
                                       const uint8_t* msk, int64_t smm, int64_t smn, void* out, int64_t soh,
                                       int64_t som, int H, int HK, int M, int P, int NN, int D, float sm_scale,
                                       void* workspace, int64_t workspace_bytes, int rows_per_wave, int launches,
                                       void* stream) {
  if (launches != 1 && launches != 2) return RSPX_EINVAL;
  return trie_attn_impl(q, sqh, sqm, kp, skph, skpn, vp, svph, svpn, kn, sknh, sknn, vn, svnh, svnn, msk, smm, smn,
                        out, soh, som, H, HK, M, P, NN, D, sm_scale, workspace, workspace_bytes, rows_per_wave,
                        stream, launches);
}

extern "C" int rspx_trie_attn_set_spin_limit(int polls) {
  const int prev = g_spin_limit;
  g_spin_limit = polls < 0 ? kSpinLimit : polls;
  return prev;
}

extern "C" int rspx_trie_attn_status(void* workspace, int H, int HK, int M, int P, int D, void* stream) {
  Plan pl;
  if (make_plan(H, HK, M, P, 0, D, 1, &pl) != RSPX_OK) return RSPX_EINVAL;
  void* ws = workspace;
  if (!ws && static_scratch(&ws) != RSPX_OK) return RSPX_ELAUNCH;
  int* flag = reinterpret_cast<int*>(static_cast<char*>(ws) + pl.off_sync);
  int v = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&v, flag, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return RSPX_ELAUNCH;
  if (v != 0) {
    // Read and clear: the flag reports each failure once.
    static const int zero = 0;
    if (hipMemcpyAsync(flag, &zero, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return RSPX_ELAUNCH;
  }
  return v ? 1 : 0;
}

#ifdef RSPX_PHASE_TRACE
// Trace builds only (not in the product library): copies the phase marks of
// the last one-launch call, kPhaseWgs x 8 waves x kPhaseMarks uint64, to host.
extern "C" int rspx_trie_attn_phase_trace(uint64_t* host, int64_t n) {
  const size_t bytes = sizeof(uint64_t) * (size_t)kPhaseWgs * kWavesA * kPhaseMarks;
  if (!host || n < (int64_t)(bytes / sizeof(uint64_t))) return RSPX_EINVAL;
  if (hipDeviceSynchronize() != hipSuccess) return RSPX_ELAUNCH;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase), bytes) == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}
#endif
