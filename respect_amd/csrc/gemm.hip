// Row-invariant linear layer for gfx950: C[M, N] = X[M, K] . W[N, K]^T.
//
// Replaces linear / _gemm of respect/kernels/gemm.py:11-41 (FixedLinear,
// respect/kernels/patch.py:26-37): bf16 inputs, fp32 accumulation, output in
// bf16 (the layers) or fp32 (the vocabulary projection, patch.py:23).
//
// Reduction order of every output element, fixed by (N, K) only:
//   K is cut into S equal chunks (S from splits(N, K), never from M); each
//   chunk is a chain of v_mfma_f32_16x16x32_bf16 over its 32-wide k-blocks in
//   increasing k; the chunk results are added in chunk order,
//   ((c0 + c1) + c2) + ..., then rounded once to the output type.
// So a row's output bits do not depend on how many rows the call carries.
//
// Work split: workgroup = (16 W output columns, chunk s, 64-row tile), W = 4,
// 6 or 8 waves of 16 columns each (the host picks W per shape for speed; the
// chunk count S comes from 64-column tiles whatever W is, so W never changes
// a bit of the result).  W -- the large operand, read exactly once -- goes
// straight from HBM into the MFMA A operand registers (lane (n16, g4) loads
// W[col n16][k + 8 g4, +8): 16 contiguous bytes), in rounds of 8 k-blocks
// requested 3 rounds ahead.  X (at most 64 rows) is shared by the block's
// waves: each round of it is copied into LDS with direct-to-LDS loads laid
// out as MFMA B fragments (one conflict-free ds_read_b128 per 16-row tile and
// k-block).  The output tile D[n][m] comes back as 4 consecutive columns per
// lane.
//
// x may also come in the tiled layout (row stride RSPX_TILED, tiled_offset in
// common.h): a 64-row block's k-block is then four 1 KB operand tiles, and
// each direct-to-LDS load copies one whole tile instead of 16 rows x 64 B
// (gate/up [64 x 4096] . [24576 x 4096]^T on MI355X: 46 instead of 53 us).
// The LDS image, and so every result bit, is the same in both layouts.  The
// SwiGLU epilogue can write its output tiled for the next layer.
//
// S > 1 writes fp32 chunk partials [S][M][N] into the caller's workspace and
// a second kernel sums them in chunk order and rounds.
//
// W may also come in a tiled layout (row stride RSPX_TILED; written by
// rspx_linear_tile_weight from the row-major matrix): 16-row slabs of
// 16 K + kWSlabPad elements, slab n / 16 holding the K / 32 tiles of its rows
// one after the other, tile k / 32 holding element (n, k) at
// (n % 16 + 16 ((k % 32) / 8)) 8 + k % 8 -- lane n % 16 + 16 g of a wave
// loads its MFMA A operand (row n % 16, k 8 g .. 8 g + 7) as 16 contiguous
// bytes of one 1 KB tile.  The TCP (vector L1) then handles one 8 KB piece per
// wave and round instead of 16 rows of 512 bytes on 16 pages (q/k/v, o,
// gate/up, down at 64 rows: 14.1 / 10.4 / 40.2 / 23.4 us instead of 14.6 /
// 11.1 / 42.0 / 24.6; one row 11.0 / 7.9 / 34.9 / 18.7 instead of 11.3 / 8.5 /
// 34.4 / 19.5).  The same bits as the row-major W.

#include "common.h"
#include "respect_amd.h"

namespace rspx {

namespace gemm {

constexpr int kSplitCols = 64;  // column tile the chunk count S is derived from
constexpr int kRows = 64;       // rows per workgroup (4 MFMA tiles)
constexpr int kRoundKB = 8;    // k-blocks of 32 per round
constexpr int kRoundK = 32 * kRoundKB;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) char lds_char_t;

__device__ __forceinline__ void x_dma16(__amdgpu_buffer_rsrc_t r, int voff, lds_char_t* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)dst, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(nbytes > 0 ? nbytes : 0), 0x00020000);
}

struct Args {
  const uint16_t* x; int64_t sx;  // [M, K]
  const uint16_t* w; int64_t sw;  // [N, K]
  void* out; int64_t so;          // [M, N]: bf16 or fp32 (S == 1)
  float* part;                    // [S][M][N] fp32 (S > 1)
  int M, N, K, S, KC, out_fp32;
  int to_part;                    // write chunk partials even when S == 1
  int silu;                       // S == 1: columns (2i, 2i + 1) are (gate_i, up_i); out[m][i] = SwiGLU
  int x_tiled;                    // x in the tiled layout (sx unused)
  int out_tiled;                  // silu: out in the tiled layout of [M, N / 2] (so unused)
};

constexpr int kXResRounds = 4;   // X-resident blocks: K chunks of at most 4 rounds (128 KB of LDS)
// Elements after each 16-row slab of a tiled W.  Slabs of 4096 or 12288
// columns are a multiple of 128 KB long, so without it every wave's stream
// starts at the same offset modulo the memory-channel interleave; 128 bytes
// spread them (on MI355X, 64 rows: gate/up [24576, 4096] 40.2 instead of 41.7
// us with no pad, down [4096, 12288] 23.4 vs 24.1, vocabulary 238 vs 250; pads
// of 32, 128, 256, 512, 1024 and 2048 elements measured no better).
constexpr int kWSlabPad = 64;
constexpr int kOOB = 0x7ffffff0;  // a buffer offset past any descriptor: loads return 0, touch nothing
constexpr int kOOBRow = 0x40000000;  // the same for a whole lane chunk (k-block steps added stay below 2^31)

__device__ __forceinline__ void vm_wait0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ void raw_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// acc[t] += W . X^T over one round: X B-fragments of row tile t, k-block kb
// from LDS buffer xb, W A-fragments from registers wf.
template <int MT>
__device__ __forceinline__ void round_compute(const lds_char_t* xb, const u32x4 (&wf)[kRoundKB], f32x4 (&acc)[4],
                                              int lane) {
#pragma unroll
  for (int kb = 0; kb < kRoundKB; ++kb) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const u32x4 xf = *(const __attribute__((address_space(3))) u32x4*)(xb + (kb * 4 + t) * 1024 + 16 * lane);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[kb]),
                                                       __builtin_bit_cast(bf16x8, xf), acc[t], 0, 0, 0);
    }
  }
}

// X chunks of round rr into LDS buffer xb: the NC = 8 MT chunks c of a round
// (k-block kb = c / MT, row tile t = c % MT: rows 16 t + n16, k [8 g4, +8) of
// the block; only the MT row tiles the block computes) are spread over the W
// waves, wave w taking c = w, w + W, ...; chunk (kb, t) lands at
// (4 kb + t) KB of the buffer whatever MT is; xo[t] is this lane's offset of
// row tile t.  Rounds past the chunk and rows past M use out-of-range
// offsets: zeros, no memory traffic.  Wave w issues the same
// ceil((NC - w) / W) X chunks and 8 W loads per round on every path, so the
// waits below are exact counts.  xkb: bytes between consecutive k-blocks of
// one lane's chunk (64 row-major, 4096 tiled).
template <int W, int MT>
__device__ __forceinline__ void issue_x(__amdgpu_buffer_rsrc_t rx, const int (&xo)[4], int xkb, int rr, int nr,
                                        lds_char_t* xb, int w) {
  constexpr int NC = 8 * MT;
  const bool live = rr < nr;
  if constexpr (NC % W == 0 && W % MT == 0) {
    // Every chunk of wave w is row tile w % MT, whose offset the caller put in xo[0].
#pragma unroll
    for (int j = 0; j < NC / W; ++j) {
      const int kb = w / MT + (W / MT) * j;
      x_dma16(rx, live ? xo[0] + xkb * (rr * kRoundKB + kb) : kOOB, xb + (kb * 4 + w % MT) * 1024);
    }
  } else {
#pragma unroll
    for (int j = 0; j < (NC + W - 1) / W; ++j) {
      const int c = w + W * j;
      const int kb = c / MT, t = c % MT;
      if (c < NC) x_dma16(rx, live ? xo[t] + xkb * (rr * kRoundKB + kb) : kOOB, xb + (kb * 4 + t) * 1024);
    }
  }
  asm volatile("" ::: "memory");
}

// WKB: bytes between a lane's consecutive k-blocks of W (64 row-major, 1024
// tiled).
template <int WKB>
__device__ __forceinline__ void issue_w(__amdgpu_buffer_rsrc_t rw, int woff, int rr, int nr, u32x4 (&wf)[kRoundKB]) {
  const bool live = rr < nr;
#pragma unroll
  for (int kb = 0; kb < kRoundKB; ++kb)
    wf[kb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rw, live ? woff + WKB * (rr * kRoundKB + kb) : kOOB, 0, 0));
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n), 0 <= n <= 63 (a compile-time constant for 4 and 8
// waves, where one case remains; a per-wave value for 6 waves).
#define RSPX_VMW(v) __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | 0x70 | 0xF00)
__device__ __forceinline__ void vm_wait_n(int n) {
  switch (n) {
    case 0: RSPX_VMW(0); break;
    case 1: RSPX_VMW(1); break;
    case 2: RSPX_VMW(2); break;
    case 3: RSPX_VMW(3); break;
    case 4: RSPX_VMW(4); break;
    case 5: RSPX_VMW(5); break;
    case 6: RSPX_VMW(6); break;
    case 7: RSPX_VMW(7); break;
    case 8: RSPX_VMW(8); break;
    case 9: RSPX_VMW(9); break;
    case 10: RSPX_VMW(10); break;
    case 11: RSPX_VMW(11); break;
    case 12: RSPX_VMW(12); break;
    case 13: RSPX_VMW(13); break;
    case 14: RSPX_VMW(14); break;
    case 15: RSPX_VMW(15); break;
    case 16: RSPX_VMW(16); break;
    case 17: RSPX_VMW(17); break;
    case 18: RSPX_VMW(18); break;
    case 19: RSPX_VMW(19); break;
    case 20: RSPX_VMW(20); break;
    case 21: RSPX_VMW(21); break;
    case 22: RSPX_VMW(22); break;
    case 23: RSPX_VMW(23); break;
    case 24: RSPX_VMW(24); break;
    case 25: RSPX_VMW(25); break;
    case 26: RSPX_VMW(26); break;
    case 27: RSPX_VMW(27); break;
    case 28: RSPX_VMW(28); break;
    case 29: RSPX_VMW(29); break;
    case 30: RSPX_VMW(30); break;
    case 31: RSPX_VMW(31); break;
    case 32: RSPX_VMW(32); break;
    case 33: RSPX_VMW(33); break;
    case 34: RSPX_VMW(34); break;
    case 35: RSPX_VMW(35); break;
    case 36: RSPX_VMW(36); break;
    case 37: RSPX_VMW(37); break;
    case 38: RSPX_VMW(38); break;
    case 39: RSPX_VMW(39); break;
    case 40: RSPX_VMW(40); break;
    case 41: RSPX_VMW(41); break;
    case 42: RSPX_VMW(42); break;
    case 43: RSPX_VMW(43); break;
    case 44: RSPX_VMW(44); break;
    case 45: RSPX_VMW(45); break;
    case 46: RSPX_VMW(46); break;
    case 47: RSPX_VMW(47); break;
    case 48: RSPX_VMW(48); break;
    case 49: RSPX_VMW(49); break;
    case 50: RSPX_VMW(50); break;
    case 51: RSPX_VMW(51); break;
    case 52: RSPX_VMW(52); break;
    case 53: RSPX_VMW(53); break;
    case 54: RSPX_VMW(54); break;
    case 55: RSPX_VMW(55); break;
    case 56: RSPX_VMW(56); break;
    case 57: RSPX_VMW(57); break;
    case 58: RSPX_VMW(58); break;
    case 59: RSPX_VMW(59); break;
    case 60: RSPX_VMW(60); break;
    case 61: RSPX_VMW(61); break;
    case 62: RSPX_VMW(62); break;
    default: RSPX_VMW(63); break;
  }
}
#undef RSPX_VMW

// Pipeline: W (the HBM stream) is requested 3 rounds ahead into a ring of 4
// register buffers, X (L2-resident) 1 round ahead into 2 LDS buffers.  Round
// r issues X(r + 1) and W(r + 3), then waits until X(r) and W(r) have landed.
// NR > 0: the NR rounds are unrolled at compile time, so every wait count is
// exact and the compiler's own waits for the W registers never drain the
// prefetch; NR == 0: a run-time loop (any round count, shallower prefetch).
//
// XRES (NR <= kXResRounds): the block's whole X chunk is copied into LDS up
// front (NR x 32 KB), so the main loop streams W with no X loads and no
// barriers.  The LDS image and the MFMA chain are those of the two-buffer
// form: the same bits.
//
// WT: W in the tiled layout (w row stride RSPX_TILED): a wave's 16 bytes per
// lane of a k-block are one 1 KB tile and its k-blocks follow each other, so
// a round of W is 8 KB in one piece instead of 16 rows x 512 bytes.  The MFMA
// operands, and so every bit, are the same.
template <int MT, int NR, int W, bool XRES = false, bool WT = false>
__global__ __launch_bounds__(64 * W) void gemm_kernel(Args A) {
  constexpr int WKB = WT ? 1024 : 64;
  static_assert(!XRES || (NR > 0 && NR <= kXResRounds), "X-resident blocks hold at most kXResRounds rounds");
  constexpr int kCols = 16 * W;
  __shared__ __attribute__((aligned(16))) char xs[XRES ? NR : 2][kRoundKB * 4 * 1024];  // 32 KB each
  constexpr int XB = kRoundKB * 4 * 1024;
  const int lane = __lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // X chunks this wave issues per round: a constant when W divides 8 MT, so
  // every wait count below is one too (a run-time count leaves the compiler's
  // own waits for the W registers conservative).
  constexpr int NC = 8 * MT;
  const int XPW = NC % W == 0 ? NC / W : (NC - w + W - 1) / W;
  const int n16 = lane & 15, g4 = lane >> 4;
  // Grid (column tile, K chunk, 64-row tile): no index divisions.  The
  // arguments the prologue needs are requested in one batch.
  const int nt = blockIdx.x, s = blockIdx.y, mt = blockIdx.z;
  asm volatile("" ::"s"(A.x), "s"(A.w), "s"(A.sx), "s"(A.sw), "s"(A.M), "s"(A.N), "s"(A.K), "s"(A.KC),
               "s"(A.x_tiled));
  const int col = nt * kCols + 16 * w;        // this wave's first column
  const int row0 = mt * kRows;
  const int k0 = s * A.KC;
  const int nr = NR > 0 ? NR : A.KC / kRoundK;
  const bool has_cols = col < A.N;            // N % 16 == 0: whole tiles only

  // X: rows [row0, M) from column k0.  W: this wave's 16 rows, columns
  // [k0, k0 + KC) (no bytes at all for a wave past N).
  // Tiled x: this block's chunk is (K - k0) / 32 k-blocks of four 1 KB tiles;
  // a wave whose tile lies past M loads nothing (rows past M inside a tile are
  // read but only reach output rows that are never stored).
  const int mrows = min(kRows, A.M - row0);
  // xoff[t]: this lane's offset of row tile t; when every chunk of a wave is
  // one row tile (issue_x), only its offset, kept in xoff[0].
  __amdgpu_buffer_rsrc_t rx;
  int xoff[4], xkb;
  auto tile_off = [&](int t) {
    return A.x_tiled ? (16 * t < mrows ? 1024 * t + 16 * lane : kOOBRow)
                     : 2 * ((16 * t + n16) * (int)A.sx + 8 * g4);
  };
  if (A.x_tiled) {
    rx = rsrc(A.x + (int64_t)mt * kRows * A.K + (int64_t)(k0 / 32) * 2048, (int64_t)(A.K - k0) * 128);
    xkb = 4096;
  } else {
    rx = rsrc(A.x + (int64_t)row0 * A.sx + k0, 2 * ((int64_t)(mrows - 1) * A.sx + (A.K - k0)));
    xkb = 64;
  }
  if constexpr (NC % W == 0 && W % MT == 0) {
    xoff[0] = tile_off(w % MT);
    xoff[1] = xoff[2] = xoff[3] = 0;
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) xoff[t] = tile_off(t);
  }
  const __amdgpu_buffer_rsrc_t rw =
      WT ? rsrc(A.w + (int64_t)(has_cols ? col / 16 : 0) * ((A.K / 32) * 512 + kWSlabPad) + (k0 / 32) * 512,
                has_cols ? A.KC * 32 : 0)
         : rsrc(A.w + (int64_t)(has_cols ? col : 0) * A.sw + k0, has_cols ? 2 * (15 * A.sw + A.KC) : 0);
  const int woff = WT ? 16 * lane : 2 * (n16 * (int)A.sw + 8 * g4);

  lds_char_t* xl = (lds_char_t*)xs[0];
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (XRES) {
    u32x4 wbuf[4][kRoundKB];
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) issue_x<W, MT>(rx, xoff, xkb, rr, nr, xl + rr * XB, w);
    issue_w<WKB>(rw, woff, 0, nr, wbuf[0]);
    if constexpr (NR > 1) issue_w<WKB>(rw, woff, 1, nr, wbuf[1]);
    if constexpr (NR > 2) issue_w<WKB>(rw, woff, 2, nr, wbuf[2]);
    vm_wait_n(8 * (1 + (1 < NR) + (2 < NR)));  // every X chunk (issued before the W rounds) landed
    raw_barrier();
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (r + 3 < NR) issue_w<WKB>(rw, woff, r + 3, nr, wbuf[(r + 3) & 3]);
      vm_wait_n(8 * ((r + 1 < NR) + (r + 2 < NR) + (r + 3 < NR)));  // W(r) landed
      round_compute<MT>(xl + r * XB, wbuf[r & 3], acc, lane);
    }
  } else if constexpr (NR > 0) {
    // Only loads whose data is used are issued (the compiler would drop the
    // others and the counts below would be off).  Exact wait per round: the
    // loads issued after the later of X(r) and W(r).
    u32x4 wbuf[4][kRoundKB];
    issue_x<W, MT>(rx, xoff, xkb, 0, nr, xl, w);
    issue_w<WKB>(rw, woff, 0, nr, wbuf[0]);
    if constexpr (NR > 1) issue_w<WKB>(rw, woff, 1, nr, wbuf[1]);
    if constexpr (NR > 2) issue_w<WKB>(rw, woff, 2, nr, wbuf[2]);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (r + 1 < NR) issue_x<W, MT>(rx, xoff, xkb, r + 1, nr, xl + ((r + 1) & 1) * XB, w);
      if (r + 3 < NR) issue_w<WKB>(rw, woff, r + 3, nr, wbuf[(r + 3) & 3]);
      const int younger = r == 0 ? 8 * ((1 < NR) + (2 < NR) + (3 < NR)) + XPW * (1 < NR)
                                 : 8 * ((r + 2 < NR) + (r + 3 < NR)) + XPW * (r + 1 < NR);
      vm_wait_n(younger);
      raw_barrier();
      round_compute<MT>(xl + (r & 1) * XB, wbuf[r & 3], acc, lane);
      raw_barrier();
    }
  } else {
    u32x4 wa[kRoundKB], wb[kRoundKB];
    issue_x<W, MT>(rx, xoff, xkb, 0, nr, xl, w);
    issue_w<WKB>(rw, woff, 0, nr, wa);
    for (int r = 0; r < nr; r += 2) {
      issue_x<W, MT>(rx, xoff, xkb, r + 1, nr, xl + XB, w);
      issue_w<WKB>(rw, woff, r + 1, nr, wb);
      vm_wait_n(8 + XPW);
      raw_barrier();
      round_compute<MT>(xl, wa, acc, lane);
      raw_barrier();
      if (r + 1 >= nr) break;
      issue_x<W, MT>(rx, xoff, xkb, r + 2, nr, xl, w);
      issue_w<WKB>(rw, woff, r + 2, nr, wa);
      vm_wait_n(8 + XPW);
      raw_barrier();
      round_compute<MT>(xl + XB, wb, acc, lane);
      raw_barrier();
    }
  }
  vm_wait0();
  if (!has_cols) return;

  // D[n][m]: lane (n16, g4) holds columns col + 4 g4 + e of row 16 t + n16.
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = row0 + 16 * t + n16;
    if (m >= A.M) continue;
    const int n = col + 4 * g4;
    if (A.S > 1 || A.to_part) {
      *reinterpret_cast<f32x4*>(A.part + ((size_t)s * A.M + m) * A.N + n) = acc[t];
    } else if (A.out_fp32) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(A.out) + (int64_t)m * A.so + n) = acc[t];
    } else if (A.silu) {
      // The bf16 gate/up values rspx_linear would store, then rspx_silu_mul's
      // arithmetic: bf16(bf16(silu(g)) * u) for columns n / 2 and n / 2 + 1.
      const uint32_t p0 = pack_bf16x2(acc[t][0], acc[t][1]);
      const uint32_t p1 = pack_bf16x2(acc[t][2], acc[t][3]);
      const float a0 = round_bf16(silu_f32(bf16_lo(p0))), a1 = round_bf16(silu_f32(bf16_lo(p1)));
      uint16_t* dst = static_cast<uint16_t*>(A.out) +
                      (A.out_tiled ? tiled_offset(m, n / 2, A.N / 2) : (int64_t)m * A.so + n / 2);
      *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(a0 * bf16_hi(p0), a1 * bf16_hi(p1));
    } else {
      u32x2 o;
      o[0] = pack_bf16x2(acc[t][0], acc[t][1]);
      o[1] = pack_bf16x2(acc[t][2], acc[t][3]);
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(A.out) + (int64_t)m * A.so + n) = o;
    }
  }
}

// out[m][n] = round(((p0 + p1) + p2) + ...), 4 columns per thread.  Grid:
// x = 256-thread blocks along a row, y = rows from row0 (at most 65535 per
// launch), so no thread divides to find its row.
template <int SC>
__global__ __launch_bounds__(256) void reduce_kernel(const float* part, int S, int M, int N, void* out, int64_t so,
                                                     int out_fp32, int row0) {
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  const int m = row0 + blockIdx.y;
  const f32x4 v = sum_parts4<SC>(part + (int64_t)m * N + n, S, (int64_t)M * N);
  if (out_fp32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + (int64_t)m * so + n) = v;
  } else {
    u32x2 o;
    o[0] = pack_bf16x2(v[0], v[1]);
    o[1] = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + (int64_t)m * so + n) = o;
  }
}

// Any shape outside gemm_kernel's (N % 16 != 0 or K % 256 != 0): one chain
// of v_mfma_f32_16x16x32_bf16 over the 32-wide k-blocks of K in increasing k,
// rounded once -- an order fixed by K alone, so a row's bits never depend on
// M.  Workgroup = 4 waves on adjacent 16-column groups of a 64-column tile,
// times one 64-row tile (MT row tiles of 16).  Operands go from memory
// straight into the MFMA registers through bounded buffer loads: rows past M,
// columns past N and k past K get an out-of-range offset and read as zero, so
// they add exact zeros to the chain.  V16 (every row 16-byte aligned, K % 8
// == 0): a lane's 8 consecutive k come in one 16-byte load, else in eight
// 2-byte loads; both give the same operand values.
struct AnyArgs {
  const uint16_t* x; int64_t sx;  // [M, K]
  const uint16_t* w; int64_t sw;  // [N, K]
  void* out; int64_t so;          // [M, N], bf16 or fp32
  int M, N, K, out_fp32;
};

// The MFMA operand of one lane: row `row` (element offset roff from the
// descriptor's base; ok = the row exists), k .. k + 7.
template <bool V16>
__device__ __forceinline__ u32x4 any_frag(__amdgpu_buffer_rsrc_t r, int roff, bool ok, int k, int K) {
  if constexpr (V16) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, ok && k < K ? (roff + k) * 2 : kOOB, 0, 0));
  } else {
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      h[j] = __builtin_amdgcn_raw_buffer_load_b16(r, ok && k + j < K ? (roff + k + j) * 2 : kOOB, 0, 0);
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  }
}

template <int MT, bool V16>
__global__ __launch_bounds__(256) void gemm_any_kernel(AnyArgs A) {
  const int lane = __lane_id(), wv = threadIdx.x >> 6;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * 64 + wv * 16, m0 = blockIdx.y * kRows;
  if (n0 >= A.N) return;  // whole wave; no barriers below
  const int nw = min(16, A.N - n0), mw = min(kRows, A.M - m0);
  // Descriptors start at the wave's first column and the tile's first row,
  // so every offset fits 31 bits (the host checks 64 rows of x and 16 of w).
  const __amdgpu_buffer_rsrc_t rw = rsrc(A.w + (int64_t)n0 * A.sw, ((int64_t)(nw - 1) * A.sw + A.K) * 2);
  const __amdgpu_buffer_rsrc_t rx = rsrc(A.x + (int64_t)m0 * A.sx, ((int64_t)(mw - 1) * A.sx + A.K) * 2);
  const bool wok = n16 < nw;
  const int woff = n16 * (int)A.sw;
  int xoff[MT];
  bool xok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    xok[t] = 16 * t + n16 < mw;
    xoff[t] = (16 * t + n16) * (int)A.sx;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nkb = (A.K + 31) >> 5;
  for (int kb = 0; kb < nkb; ++kb) {
    const int k = 32 * kb + 8 * g4;
    const u32x4 wf = any_frag<V16>(rw, woff, wok, k, A.K);
    u32x4 xf[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) xf[t] = any_frag<V16>(rx, xoff[t], xok[t], k, A.K);
#pragma unroll
    for (int t = 0; t < MT; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf), __builtin_bit_cast(bf16x8, xf[t]),
                                                       acc[t], 0, 0, 0);
  }
  // acc[t][e] = D[column 4 g4 + e][row 16 t + n16] of the wave's tile.
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + 16 * t + n16;
    if (m >= A.M) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = n0 + 4 * g4 + e;
      if (n >= A.N) continue;
      if (A.out_fp32)
        static_cast<float*>(A.out)[(int64_t)m * A.so + n] = acc[t][e];
      else
        static_cast<uint16_t*>(A.out)[(int64_t)m * A.so + n] = f32_to_bf16_rne(acc[t][e]);
    }
  }
}

}  // namespace gemm

// Chunk count of the K reduction: a function of (N, K) only.  More chunks
// until the grid has >= 256 workgroups per 64-row tile, at most 8, each chunk
// a whole number of 256-wide rounds.
static int linear_splits(int N, int K) {
  const int nt = (N + gemm::kSplitCols - 1) / gemm::kSplitCols;
  int S = 1;
  while (nt * S < 256 && S < 8 && K % (gemm::kRoundK * 2 * S) == 0) S *= 2;
  return S;
}

// W [N, K] (row stride sw) into the tiled layout: one thread per 16 bytes of
// the output, the slab pads written as zeros.
__global__ __launch_bounds__(256) void tile_weight_kernel(const uint16_t* w, int64_t sw, int N, int K,
                                                         uint16_t* out) {
  const int64_t slab = (int64_t)K * 16 + gemm::kWSlabPad;   // elements per slab
  const int64_t per = slab / 8;                              // 16-byte units per slab
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= (int64_t)(N / 16) * per) return;
  const int s = (int)(u / per);
  const int64_t j = u - s * per;                             // unit inside the slab
  u32x4 v = {0u, 0u, 0u, 0u};
  if (j < (int64_t)K * 2) {
    const int t = (int)(j >> 6), lane = (int)(j & 63);
    const int n = 16 * s + (lane & 15), k = 32 * t + 8 * (lane >> 4);
    v = *reinterpret_cast<const u32x4*>(w + (int64_t)n * sw + k);
  }
  *reinterpret_cast<u32x4*>(out + u * 8) = v;
}

}  // namespace rspx

using namespace rspx;

extern "C" int64_t rspx_linear_tiled_weight_elems(int N, int K) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % 32 != 0) return -1;
  return (int64_t)(N / 16) * ((int64_t)K * 16 + gemm::kWSlabPad);
}

extern "C" int rspx_linear_tile_weight(const void* w, int64_t sw, int N, int K, void* out, void* stream) {
  if (N <= 0 || K <= 0 || !w || !out || sw < K) return RSPX_EINVAL;
  if (N % 16 != 0 || K % 32 != 0) return RSPX_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u) || sw % 8)
    return RSPX_EALIGN;
  const int64_t units = rspx_linear_tiled_weight_elems(N, K) / 8;
  if ((units + 255) / 256 > 0x7fffffff) return RSPX_EUNSUPPORTED;
  hipLaunchKernelGGL(tile_weight_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), sw, N, K,
                     static_cast<uint16_t*>(out));
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

// Shapes gemm_kernel takes; every other (N, K) runs gemm_any_kernel (one
// K chain).  The choice depends on (N, K) only.
static bool linear_fast_shape(int N, int K) { return N % 16 == 0 && K % gemm::kRoundK == 0; }

extern "C" int rspx_linear_splits(int N, int K) {
  if (N <= 0 || K <= 0) return -1;
  return linear_fast_shape(N, K) ? linear_splits(N, K) : 1;
}

extern "C" int64_t rspx_linear_workspace_bytes(int M, int N, int K) {
  if (M < 0 || N <= 0 || K <= 0) return -1;
  const int S = rspx_linear_splits(N, K);
  return S > 1 ? (int64_t)S * M * N * (int64_t)sizeof(float) : 0;
}

namespace rspx {
static int linear_launch(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M, int N,
                         int K, int out_fp32, float* part, int to_part, hipStream_t s, int silu = 0) {
  const int S = linear_splits(N, K);
  gemm::Args a;
  a.x = static_cast<const uint16_t*>(x); a.sx = sx;
  a.w = static_cast<const uint16_t*>(w); a.sw = sw;
  a.out = out; a.so = so;
  a.part = part;
  a.M = M; a.N = N; a.K = K; a.S = S; a.KC = K / S; a.out_fp32 = out_fp32 ? 1 : 0; a.to_part = to_part;
  a.silu = silu;
  a.x_tiled = sx == kTiled;
  a.out_tiled = silu && so == kTiled;
  const int MTILES = (M + gemm::kRows - 1) / gemm::kRows;
  // 8 waves (128 columns) share each X round between twice the columns; worth
  // it while the grid keeps >= 192 workgroups, and for the widest layers
  // (the vocabulary head) only when the X block is large (many rows).
  const int wg8 = (N + 127) / 128 * S;
  // An 8-wave grid that leaves CUs idle: 6 waves (96 columns) fill them
  // (gate/up [64 x 4096] . [24576 x 4096]^T: 192 -> 256 workgroups, 47.7 ->
  // 42.2 us, one row 38.9 -> 34.8 us; q/k/v [6144 x 4096], 4 K chunks: 15.4 ->
  // 14.8 us with X resident).  The vocabulary head gained nothing from it.
  const int wg6 = (N + 95) / 96 * S;
  const int waves = (N % 96 == 0 && wg8 < 256 && wg6 >= 256 && wg6 <= 512) ? 6
                    : (wg8 >= 192 && (M >= 32 || wg8 < 1024)) ? 8 : 4;
  const int NT = (N + 16 * waves - 1) / (16 * waves);
  if (MTILES > 65535) return RSPX_EUNSUPPORTED;
  const int mt = (MTILES > 1 || M >= 64) ? 4 : (M + 15) / 16;  // row tiles per 64-row tile
  // X-resident blocks pay where X is large against each block's W slice and
  // the grid is one wave of 6- or 8-wave blocks (q/k/v [64 x 4096] .
  // [6144 x 4096]^T: 17.5 -> 16.7 us at 8 waves); for 4-wave blocks and for
  // one row they cost a little.
  const bool xres = waves >= 6 && M >= 32;
  const int nr = a.KC / gemm::kRoundK;
  const dim3 g((unsigned)NT, (unsigned)S, (unsigned)MTILES), b(64 * waves);
#define RSPX_GEMM_NR(MTV, WV, WTV)                                                                       \
  switch (nr) {                                                                                          \
    case 1: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 1, WV, false, WTV>), g, b, 0, s, a); break;       \
    case 2: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 2, WV, false, WTV>), g, b, 0, s, a); break;       \
    case 3: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 3, WV, false, WTV>), g, b, 0, s, a); break;       \
    case 4:                                                                                              \
      if (xres) hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 4, WV, true, WTV>), g, b, 0, s, a);           \
      else hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 4, WV, false, WTV>), g, b, 0, s, a);               \
      break;                                                                                             \
    case 6: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 6, WV, false, WTV>), g, b, 0, s, a); break;       \
    case 8: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 8, WV, false, WTV>), g, b, 0, s, a); break;       \
    case 12: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 12, WV, false, WTV>), g, b, 0, s, a); break;     \
    case 16: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 16, WV, false, WTV>), g, b, 0, s, a); break;     \
    default: hipLaunchKernelGGL((gemm::gemm_kernel<MTV, 0, WV, false, WTV>), g, b, 0, s, a); break;      \
  }
#define RSPX_GEMM_MT(WV, WTV)                                                                            \
  if (mt == 4) { RSPX_GEMM_NR(4, WV, WTV) }                                                              \
  else if (mt == 3) { RSPX_GEMM_NR(3, WV, WTV) }                                                         \
  else if (mt == 2) { RSPX_GEMM_NR(2, WV, WTV) }                                                         \
  else { RSPX_GEMM_NR(1, WV, WTV) }
#define RSPX_GEMM_W(WV)                                                                                  \
  if (sw == kTiled) { RSPX_GEMM_MT(WV, true) }                                                           \
  else { RSPX_GEMM_MT(WV, false) }
  if (waves == 6) { RSPX_GEMM_W(6) }
  else if (waves == 8) { RSPX_GEMM_W(8) }
  else { RSPX_GEMM_W(4) }
#undef RSPX_GEMM_W
#undef RSPX_GEMM_MT
#undef RSPX_GEMM_NR
  if (S > 1 && !to_part) {
    const unsigned bx = (unsigned)((N / 4 + 255) / 256);
    for (int row0 = 0; row0 < M; row0 += 65535) {
      const dim3 rg(bx, (unsigned)min(M - row0, 65535));
      RSPX_WITH_SPLITS(S, SC,
                       hipLaunchKernelGGL((gemm::reduce_kernel<SC>), rg, dim3(256), 0, s, part, S, M, N, out, so,
                                          a.out_fp32, row0));
    }
  }
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

static int linear_check(const void* x, int64_t sx, const void* w, int64_t sw, int M, int N, int K) {
  if (M < 0 || N <= 0 || K <= 0) return RSPX_EINVAL;
  if (N % 16 != 0 || K % gemm::kRoundK != 0) return RSPX_EUNSUPPORTED;
  if (M == 0) return RSPX_OK;
  if (!x || !w) return RSPX_EINVAL;
  const bool xt = sx == kTiled, wt = sw == kTiled;
  if ((!xt && sx < K) || (!wt && sw < K)) return RSPX_EINVAL;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!al(x) || !al(w) || (!xt && sx % 8) || (!wt && sw % 8)) return RSPX_EALIGN;
  if ((!xt && (int64_t)64 * sx * 2 >= (1ll << 31)) || (!wt && (int64_t)16 * sw * 2 >= (1ll << 31)) ||
      (int64_t)K * 128 >= (1ll << 30))
    return RSPX_EUNSUPPORTED;
  return RSPX_OK;
}
}  // namespace rspx

// Any (N, K): row-major x and w with rows of at least K elements (2-byte
// aligned, any stride below 2^24 elements), out [M, N] with row stride so.
static int linear_any(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M, int N,
                      int K, int out_fp32, hipStream_t s) {
  if (M < 0 || N <= 0 || K <= 0) return RSPX_EINVAL;
  if (M == 0) return RSPX_OK;
  if (!x || !w || !out) return RSPX_EINVAL;
  if (sx == kTiled || sw == kTiled) return RSPX_EUNSUPPORTED;  // the tiled layouts need N % 16, K % 32
  if (sx < K || sw < K || so < N) return RSPX_EINVAL;
  auto al = [](const void* p, unsigned a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (!al(x, 2) || !al(w, 2) || !al(out, out_fp32 ? 4 : 2)) return RSPX_EALIGN;
  // 31-bit byte offsets inside one 64-row tile of x and one 16-row slice of w.
  if (((int64_t)gemm::kRows * sx + K) * 2 >= (1ll << 31) - 64 || ((int64_t)16 * sw + K) * 2 >= (1ll << 31) - 64)
    return RSPX_EUNSUPPORTED;
  const int64_t gx = (N + 63) / 64, gy = (M + gemm::kRows - 1) / gemm::kRows;
  if (gy > 65535) return RSPX_EUNSUPPORTED;
  gemm::AnyArgs a{static_cast<const uint16_t*>(x), sx, static_cast<const uint16_t*>(w), sw, out, so, M, N, K,
                  out_fp32 ? 1 : 0};
  const bool v16 = K % 8 == 0 && sx % 8 == 0 && sw % 8 == 0 && al(x, 16) && al(w, 16);
  const int mt = M >= gemm::kRows ? 4 : (M + 15) / 16;
  const dim3 g((unsigned)gx, (unsigned)gy), b(256);
#define RSPX_ANY_MT(V)                                                                   \
  if (mt == 4) hipLaunchKernelGGL((gemm::gemm_any_kernel<4, V>), g, b, 0, s, a);         \
  else if (mt == 3) hipLaunchKernelGGL((gemm::gemm_any_kernel<3, V>), g, b, 0, s, a);    \
  else if (mt == 2) hipLaunchKernelGGL((gemm::gemm_any_kernel<2, V>), g, b, 0, s, a);    \
  else hipLaunchKernelGGL((gemm::gemm_any_kernel<1, V>), g, b, 0, s, a);
  if (v16) { RSPX_ANY_MT(true) }
  else { RSPX_ANY_MT(false) }
#undef RSPX_ANY_MT
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_linear(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M, int N,
                           int K, int out_fp32, void* workspace, int64_t workspace_bytes, void* stream) {
  if (N > 0 && K > 0 && !linear_fast_shape(N, K))
    return linear_any(x, sx, w, sw, out, so, M, N, K, out_fp32, static_cast<hipStream_t>(stream));
  int rc = linear_check(x, sx, w, sw, M, N, K);
  if (rc != RSPX_OK || M == 0) return rc;
  if (!out) return RSPX_EINVAL;
  if (so < N) return RSPX_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out) & 15u) || so % 4) return RSPX_EALIGN;
  const int S = linear_splits(N, K);
  const int64_t need = S > 1 ? (int64_t)S * M * N * (int64_t)sizeof(float) : 0;
  if (need > 0 && (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u)))
    return RSPX_EWORKSPACE;
  return linear_launch(x, sx, w, sw, out, so, M, N, K, out_fp32, static_cast<float*>(workspace), 0,
                       static_cast<hipStream_t>(stream));
}

extern "C" int rspx_linear_silu(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M,
                                int N, int K, void* stream) {
  int rc = linear_check(x, sx, w, sw, M, N, K);
  if (rc != RSPX_OK || M == 0) return rc;
  const bool ot = so == kTiled;
  if (!out || N % 32 != 0 || (!ot && so < N / 2) || (ot && (N / 2) % 32 != 0)) return RSPX_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out) & 15u) || (!ot && so % 8)) return RSPX_EALIGN;
  if (linear_splits(N, K) != 1) return RSPX_EUNSUPPORTED;
  return linear_launch(x, sx, w, sw, out, so, M, N, K, 0, nullptr, 0, static_cast<hipStream_t>(stream), 1);
}

extern "C" int rspx_linear_partials(const void* x, int64_t sx, const void* w, int64_t sw, float* part, int M, int N,
                                    int K, void* stream) {
  int rc = linear_check(x, sx, w, sw, M, N, K);
  if (rc != RSPX_OK || M == 0) return rc;
  if (!part || (reinterpret_cast<uintptr_t>(part) & 15u)) return RSPX_EINVAL;
  return linear_launch(x, sx, w, sw, nullptr, N, M, N, K, 1, part, 1, static_cast<hipStream_t>(stream));
}
