// Row-invariant RMSNorm, RoPE, and the fused q/k RMSNorm + RoPE of a decoder
// layer, for gfx950.
//
// RMSNorm (respect/kernels/rmsnorm.py:12-32, HF Qwen3VLTextRMSNorm):
//   x32 = float(x); var = sum(x32^2) / N; xh = bf16(x32 * rsqrt(var + eps));
//   y = bf16(float(w) * float(xh)).
// The sum of squares of a row is always taken in the same order -- each lane
// folds its 8-element vectors sequentially, lanes are combined by a fixed DPP /
// permlane butterfly, waves in wave order -- and the work split depends on N
// only, so a row's bits never depend on how many rows a call carries.
//
// RoPE (respect/system/fused.py:45-75, HF apply_rotary_pos_emb):
//   y = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)),
//   rotate_half(x)[d] = -x[d + D/2] (d < D/2) or x[d - D/2].
// Every multiply and add is an IEEE fp32 operation rounded once to bf16, the
// rounding points of PyTorch bf16 arithmetic (no FMA contraction), so results
// match PyTorch's elementwise ops bit for bit.
//
// Vectors of 8 bf16 (16-byte loads/stores) throughout; N and D must be
// multiples of 8.

#include "common.h"
#include "respect_amd.h"

namespace rspx {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of L lanes (L a power of two <= 64); every lane of a
// group gets bitwise the same value.
template <int L>
__device__ __forceinline__ float lane_group_sum(float x) {
  if constexpr (L >= 2) x = x + dpp_f<0xB1>(x);    // lane ^ 1
  if constexpr (L >= 4) x = x + dpp_f<0x4E>(x);    // lane ^ 2
  if constexpr (L >= 8) x = x + dpp_f<0x141>(x);   // half-row mirror
  if constexpr (L >= 16) x = x + dpp_f<0x140>(x);  // row mirror
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

// A 16-byte store; NT: non-temporal (not kept in L2).  Stand-alone element-wise
// calls whose output is not read right away gain from it (it shortens the
// write-back at the kernel's end); inside the decoder step, where the next
// kernel reads the output, cached stores measured faster.
template <bool NT>
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
  else *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ void unpack8(const u32x4& w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) { f[2 * i] = bf16_lo(w[i]); f[2 * i + 1] = bf16_hi(w[i]); }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return w;
}

// 1 / sqrt(v): correctly rounded square root, then a correctly rounded divide.
__device__ __forceinline__ float rsqrt_rn(float v) { return 1.0f / __builtin_sqrtf(v); }

// Input of a normalised row.  MODE 0: x.  MODE 1: the residual sum
// bf16(x + h) with h bf16 (one fp32 add rounded once, as PyTorch's bf16 add),
// also stored to xo.  MODE 2: the same with h the output of a K-split linear
// layer given by its fp32 chunk partials (h = bf16(((p0 + p1) + ...)), the
// value rspx_linear would have stored).
struct RowIn {
  const uint16_t* x; int64_t sx;
  const uint16_t* h; int64_t sh;
  const float* hp; int64_t shp, sps; int S;
  uint16_t* xo; int64_t sxo;
};

// The arguments a row kernel needs before its loads, requested in one batch
// (left to the compiler they come in two or three dependent scalar-load round
// trips, each in front of the loads that use them).
__device__ __forceinline__ void pin_row_args(const RowIn& in, const uint16_t* w, const uint16_t* y, int64_t sy,
                                             int n, float eps) {
  asm volatile("" ::"s"(in.x), "s"(in.sx), "s"(in.h), "s"(in.sh), "s"(in.hp), "s"(in.shp), "s"(in.sps), "s"(in.S),
               "s"(in.xo), "s"(in.sxo), "s"(w), "s"(y), "s"(sy), "s"(n), "s"(eps));
}

template <int MODE, int SC>
__device__ __forceinline__ void load_row_vec(const RowIn& in, int row, int c, float* v) {
  unpack8(*reinterpret_cast<const u32x4*>(in.x + row * in.sx + c), v);
  if constexpr (MODE >= 1) {
    float hv[8];
    if constexpr (MODE == 1) {
      unpack8(*reinterpret_cast<const u32x4*>(in.h + row * in.sh + c), hv);
    } else {
      const float* hp = in.hp + row * in.shp + c;
      f32x4 a, b;
      sum_parts8<SC>(hp, in.S, in.sps, a, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) { hv[e] = round_bf16(a[e]); hv[4 + e] = round_bf16(b[e]); }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_bf16(v[i] + hv[i]);
    *reinterpret_cast<u32x4*>(in.xo + row * in.sxo + c) = pack8(v);
  }
}

// Normalise a row held by TPR lanes (TPR <= 64, all in one wave), VPL
// 8-element vectors per lane.
// Where the 8 outputs (row, c .. c + 7) go: row stride sy, or the tiled
// layout (tiled_offset) when sy == kTiled.
__device__ __forceinline__ uint16_t* out_at(uint16_t* y, int64_t sy, int row, int c, int n) {
  return y + (sy == kTiled ? tiled_offset(row, c, n) : row * sy + c);
}

template <int TPR, int VPL, int MODE, int SC, bool NT = false>
__device__ __forceinline__ void rms_row_wave(const RowIn& in, int row, const uint16_t* w, uint16_t* y, int64_t sy,
                                             int sub, int n, float eps) {
  // The weights are requested first: after the row's stores and the
  // reduction they would be one more dependent memory round trip.
  u32x4 wraw[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TPR + sub) * 8;
    wraw[v] = c < n ? *reinterpret_cast<const u32x4*>(w + c) : u32x4{0u, 0u, 0u, 0u};
  }
  float xv[VPL][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TPR + sub) * 8;
    if (c < n) {
      load_row_vec<MODE, SC>(in, row, c, xv[v]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[v][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xv[v][i], xv[v][i], ss);
  }
  ss = lane_group_sum<TPR>(ss);
  const float r = rsqrt_rn(ss / (float)n + eps);
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TPR + sub) * 8;
    if (c < n) {
      float wv[8], o[8];
      unpack8(wraw[v], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = wv[i] * round_bf16(xv[v][i] * r);
      st16<NT>(out_at(y, sy, row, c, n), pack8(o));
    }
  }
}

}  // namespace

// Rows of up to 64*8*VPL elements: one row per TPR lanes of a wave.
template <int TPR, int VPL, int MODE, int SC>
__global__ __launch_bounds__(256) void rmsnorm_small_kernel(RowIn in, const uint16_t* w, uint16_t* y, int64_t sy,
                                                            int rows, int n, float eps) {
  pin_row_args(in, w, y, sy, n, eps);
  const int lane = __lane_id();
  const int row = (blockIdx.x * 256 + threadIdx.x) / TPR;
  const int sub = lane % TPR;
  if (row >= rows) return;   // whole lane groups leave together (TPR divides 64)
  rms_row_wave<TPR, VPL, MODE, SC>(in, row, w, y, sy, sub, n, eps);
}

// Long rows: one TH-thread workgroup per row, VPL 8-element vectors per
// thread.  Wave sums are combined in wave order through LDS.
template <int VPL, int MODE, int SC, int TH, bool NT = false>
__device__ __forceinline__ void rms_row_block(const RowIn& in, const uint16_t* w, uint16_t* y, int64_t sy, int row,
                                              int n, float eps) {
  constexpr int NW = TH / 64;
  __shared__ float part[NW];
  const int t = threadIdx.x, lane = __lane_id(), wv = t >> 6;
  // The weights are requested first (see rms_row_wave).
  u32x4 wraw[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TH + t) * 8;
    wraw[v] = c < n ? *reinterpret_cast<const u32x4*>(w + c) : u32x4{0u, 0u, 0u, 0u};
  }
  float xv[VPL][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TH + t) * 8;
    if (c < n) {
      load_row_vec<MODE, SC>(in, row, c, xv[v]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[v][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xv[v][i], xv[v][i], ss);
  }
  ss = lane_group_sum<64>(ss);
  if (lane == 0) part[wv] = ss;
  __syncthreads();
  float tot = part[0];
#pragma unroll
  for (int k = 1; k < NW; ++k) tot = tot + part[k];
  const float r = rsqrt_rn(tot / (float)n + eps);
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = (v * TH + t) * 8;
    if (c < n) {
      float wvv[8], o[8];
      unpack8(wraw[v], wvv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = wvv[i] * round_bf16(xv[v][i] * r);
      st16<NT>(out_at(y, sy, row, c, n), pack8(o));
    }
  }
}

template <int VPL, int MODE, int SC, int TH = 256>
__global__ __launch_bounds__(TH) void rmsnorm_row_kernel(RowIn in, const uint16_t* w, uint16_t* y, int64_t sy, int n,
                                                         float eps) {
  pin_row_args(in, w, y, sy, n, eps);
  rms_row_block<VPL, MODE, SC, TH>(in, w, y, sy, blockIdx.x, n, eps);
}

// Rows of any length (n % 8 != 0, or n > 16384) at any 2-byte alignment:
// one 256-thread workgroup per row, element c on thread c % 256, each thread
// folding its elements in increasing c, lanes combined by the butterfly and
// waves in wave order -- an order fixed by n.  The second pass reads the row
// again (MODE 1: the xo the same thread wrote, so xo may alias the residual),
// so the length is unbounded.
template <int MODE>
__global__ __launch_bounds__(256) void rmsnorm_any_kernel(RowIn in, const uint16_t* w, uint16_t* y, int64_t sy, int n,
                                                          float eps) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const uint16_t* xr = in.x + row * in.sx;
  float ss = 0.f;
  for (int c = t; c < n; c += 256) {
    float v = bf16_to_f32(xr[c]);
    if constexpr (MODE == 1) {
      v = round_bf16(v + bf16_to_f32(in.h[row * in.sh + c]));
      in.xo[row * in.sxo + c] = f32_to_bf16_rne(v);
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = lane_group_sum<64>(ss);
  if (__lane_id() == 0) part[t >> 6] = ss;
  __syncthreads();
  const float r = rsqrt_rn((((part[0] + part[1]) + part[2]) + part[3]) / (float)n + eps);
  const uint16_t* xs = MODE == 1 ? in.xo + row * in.sxo : xr;
  for (int c = t; c < n; c += 256)
    y[row * sy + c] = f32_to_bf16_rne(bf16_to_f32(w[c]) * round_bf16(bf16_to_f32(xs[c]) * r));
}

namespace {

// RoPE on one row of D = 16 * 8 elements held by 16 lanes (8 each).  The
// partner half comes from the lane 8 positions away (DPP row rotate by 8).
__device__ __forceinline__ void rope_vec(const float* xv, const float* cs, const float* sn, int sub, float* o) {
  float part[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    part[i] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(xv[i]), 0x128, 0xF, 0xF, false));  // row_ror:8
  const bool first_half = sub < 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float rh = first_half ? -part[i] : part[i];
    const float a = round_bf16(xv[i] * cs[i]);
    const float b = round_bf16(rh * sn[i]);
    o[i] = a + b;   // rounded to bf16 by the store
  }
}

}  // namespace

// RoPE for D = 128: x [B, H, L, D] (any strides, D contiguous), cos/sin
// [B, L, D] with row stride scl and batch stride scb; y [B, H, L, D] contiguous.
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* x, int64_t sxb, int64_t sxh, int64_t sxl,
                                                   const uint16_t* cosb, const uint16_t* sinb, int64_t scb,
                                                   int64_t scl, uint16_t* y, int B, int H, int L) {
  constexpr int D = 128;
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int rowid = gid >> 4;      // (b, h, l) row
  const int sub = gid & 15;
  const int nrows = B * H * L;
  if (rowid >= nrows) return;      // 16-lane groups leave together
  const int l = rowid % L;
  const int h = (rowid / L) % H;
  const int b = rowid / (L * H);
  float xv[8], cs[8], sn[8], o[8];
  unpack8(*reinterpret_cast<const u32x4*>(x + b * sxb + h * sxh + (int64_t)l * sxl + sub * 8), xv);
  unpack8(*reinterpret_cast<const u32x4*>(cosb + b * scb + (int64_t)l * scl + sub * 8), cs);
  unpack8(*reinterpret_cast<const u32x4*>(sinb + b * scb + (int64_t)l * scl + sub * 8), sn);
  rope_vec(xv, cs, sn, sub, o);
  *reinterpret_cast<u32x4*>(y + (int64_t)rowid * D + sub * 8) = pack8(o);
}

// RoPE for any D with D % 16 == 0 and D <= 512: a row's D elements sit on
// TPR = D / 8 consecutive lanes of a wave (8 each; 64 / TPR rows per wave, the
// remaining lanes idle), and the rotate-half partner -- D / 2 elements away,
// TPR / 2 lanes -- comes through ds_bpermute.  The arithmetic of rope_kernel:
// bf16(x cos) + bf16(rotate_half(x) sin), rounded to bf16 by the store.
__global__ __launch_bounds__(256) void rope_any_kernel(const uint16_t* x, int64_t sxb, int64_t sxh, int64_t sxl,
                                                       const uint16_t* cosb, const uint16_t* sinb, int64_t scb,
                                                       int64_t scl, uint16_t* y, int B, int H, int L, int D) {
  const int lane = __lane_id();
  const int TPR = D >> 3, half = TPR >> 1, rpw = 64 / TPR;
  const int rin = lane / TPR, sub = lane - rin * TPR;
  const int64_t rowid = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw + rin;
  const int64_t nrows = (int64_t)B * H * L;
  const bool act = rin < rpw && rowid < nrows;
  float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, cs[8], sn[8];
  int64_t yo = 0;
  if (act) {
    const int l = (int)(rowid % L);
    const int h = (int)((rowid / L) % H);
    const int b = (int)(rowid / ((int64_t)L * H));
    unpack8(*reinterpret_cast<const u32x4*>(x + b * sxb + h * sxh + (int64_t)l * sxl + sub * 8), xv);
    unpack8(*reinterpret_cast<const u32x4*>(cosb + b * scb + (int64_t)l * scl + sub * 8), cs);
    unpack8(*reinterpret_cast<const u32x4*>(sinb + b * scb + (int64_t)l * scl + sub * 8), sn);
    yo = rowid * D + sub * 8;
  }
  // Every lane takes part in the exchange; idle lanes send zeros.
  const int partner = lane - sub + (sub < half ? sub + half : sub - half);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float p = __int_as_float(__builtin_amdgcn_ds_bpermute(partner << 2, __float_as_int(xv[i])));
    const float rh = sub < half ? -p : p;
    o[i] = round_bf16(xv[i] * cs[i]) + round_bf16(rh * sn[i]);
  }
  if (act) *reinterpret_cast<u32x4*>(y + yo) = pack8(o);
}

// q/k RMSNorm over head_dim followed by RoPE, one launch for q and k.
// q [T, HQ, D] (token stride sqt, head stride sqh), k [T, HK, D]; wq, wk [D];
// cos/sin rows per token (stride scs); outputs qo [T, HQ, D], ko [T, HK, D]
// contiguous.  Equal, bit for bit, to rmsnorm followed by rope.
struct QKArgs {
  const uint16_t* q; int64_t sqt, sqh;
  const uint16_t* k; int64_t skt, skh;
  const uint16_t* wq; const uint16_t* wk;
  const uint16_t* cosb; const uint16_t* sinb; int64_t scs;
  uint16_t* qo; uint16_t* ko;
  int T, HQ, HK, D;
  float eps;
};

// D = 128: row gid / 16 of the q rows then the k rows, on 16 lanes.  Row
// indices are 32-bit (the host keeps 16 T (HQ + HK) below 2^31): a 64-bit
// division in front of the address arithmetic would delay every load.
template <bool NT = false>
__device__ __forceinline__ void qk_norm_rope_row(const QKArgs& a, int gid) {
  constexpr int D = 128;
  const int rowid = gid >> 4;
  const int sub = gid & 15;
  const int nq = a.T * a.HQ;
  if (rowid >= nq + a.T * a.HK) return;
  const bool isq = rowid < nq;
  const int r = isq ? rowid : rowid - nq;
  const int HH = isq ? a.HQ : a.HK;
  const int t = r / HH, hh = r - t * HH;
  const uint16_t* src = isq ? a.q + (int64_t)t * a.sqt + hh * a.sqh : a.k + (int64_t)t * a.skt + hh * a.skh;
  const uint16_t* w = isq ? a.wq : a.wk;
  float xv[8];
  unpack8(*reinterpret_cast<const u32x4*>(src + sub * 8), xv);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xv[i], xv[i], ss);
  ss = lane_group_sum<16>(ss);
  const float rr = rsqrt_rn(ss / (float)D + a.eps);
  float wv[8], nv[8], cs[8], sn[8], o[8];
  unpack8(*reinterpret_cast<const u32x4*>(w + sub * 8), wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) nv[i] = round_bf16(wv[i] * round_bf16(xv[i] * rr));
  unpack8(*reinterpret_cast<const u32x4*>(a.cosb + (int64_t)t * a.scs + sub * 8), cs);
  unpack8(*reinterpret_cast<const u32x4*>(a.sinb + (int64_t)t * a.scs + sub * 8), sn);
  rope_vec(nv, cs, sn, sub, o);
  uint16_t* dst = (isq ? a.qo : a.ko) + (int64_t)r * D;
  st16<NT>(dst + sub * 8, pack8(o));
}

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QKArgs a) {
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.sqt), "s"(a.sqh), "s"(a.skt), "s"(a.skh), "s"(a.wq), "s"(a.wk),
               "s"(a.cosb), "s"(a.sinb), "s"(a.scs), "s"(a.qo), "s"(a.ko), "s"(a.T), "s"(a.HQ), "s"(a.HK),
               "s"(a.eps));   // one argument batch
  qk_norm_rope_row<false>(a, blockIdx.x * 256 + threadIdx.x);
}

// One decoder layer's q/k/v epilogue for T tokens, one launch: from the packed
// projection row qkv[t] = [q (HQ D) | k (HK D) | v (HK D)], q and k get the
// q_norm / k_norm RMSNorm and RoPE (the arithmetic of qk_norm_rope_kernel);
// q goes to qo [T, HQ, D], k and v are written straight into the KV cache at
// the token's physical slot: cache[h][slot[t]][:] (head stride sh, slot
// stride sn).  A slot outside [0, cap) writes no K/V and makes the token's q
// NaN, so the error shows in every output that token reaches.
template <int SC>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(const uint16_t* qkv, int64_t sqkv, const float* qp,
                                                             int S, int64_t sps, const uint16_t* wq,
                                                             const uint16_t* wk, const uint16_t* cosb,
                                                             const uint16_t* sinb, int64_t scs, const int* slots,
                                                             int cap, uint16_t* ck, int64_t skh, int64_t skn, uint16_t* cv,
                                                             int64_t svh, int64_t svn, uint16_t* qo, int t0, int HQ,
                                                             int HK, float eps) {
  // Grid (blocks of 16 head rows, token t0 + y): token t's q heads, then its
  // k heads, then its v heads; no index division.  The arguments the loads
  // need are requested in one batch (left to the compiler: three dependent
  // scalar-load round trips).
  asm volatile("" ::"s"(qkv), "s"(sqkv), "s"(qp), "s"(S), "s"(sps), "s"(wq), "s"(wk), "s"(cosb), "s"(sinb),
               "s"(scs), "s"(slots), "s"(t0), "s"(HQ), "s"(HK));
  constexpr int D = 128;
  const int rowid = (blockIdx.x * 256 + threadIdx.x) >> 4;   // head row of the token
  const int sub = threadIdx.x & 15;
  if (rowid >= HQ + 2 * HK) return;
  const int t = t0 + blockIdx.y;
  const int kind = rowid < HQ ? 0 : rowid < HQ + HK ? 1 : 2;
  const int hh = kind == 0 ? rowid : kind == 1 ? rowid - HQ : rowid - HQ - HK;
  const int col = (kind == 0 ? hh * D : kind == 1 ? (HQ + hh) * D : (HQ + HK + hh) * D) + sub * 8;
  // Norm weights and rotary rows are requested with the projection values
  // (v rows load them unused): after the reduction they would be one more
  // dependent memory round trip.
  const u32x4 wraw = *reinterpret_cast<const u32x4*>((kind == 0 ? wq : wk) + sub * 8);
  const u32x4 craw = *reinterpret_cast<const u32x4*>(cosb + (int64_t)t * scs + sub * 8);
  const u32x4 sraw = *reinterpret_cast<const u32x4*>(sinb + (int64_t)t * scs + sub * 8);
  u32x4 raw;
  if (qp) {  // the projection's fp32 chunk partials, summed and rounded as rspx_linear would
    const float* p = qp + (int64_t)t * sqkv + col;
    f32x4 a, b;
    sum_parts8<SC>(p, S, sps, a, b);
    raw[0] = pack_bf16x2(a[0], a[1]); raw[1] = pack_bf16x2(a[2], a[3]);
    raw[2] = pack_bf16x2(b[0], b[1]); raw[3] = pack_bf16x2(b[2], b[3]);
  } else {
    raw = *reinterpret_cast<const u32x4*>(qkv + (int64_t)t * sqkv + col);
  }
  const int slot = slots[t];
  const bool slot_ok = slot >= 0 && slot < cap;
  if (kind != 0 && !slot_ok) return;
  if (kind == 2) {
    *reinterpret_cast<u32x4*>(cv + hh * svh + (int64_t)slot * svn + sub * 8) = raw;
    return;
  }
  float xv[8];
  unpack8(raw, xv);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xv[i], xv[i], ss);
  ss = lane_group_sum<16>(ss);
  const float rr = rsqrt_rn(ss / (float)D + eps);
  float wv[8], nv[8], cs[8], sn[8], o[8];
  unpack8(wraw, wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) nv[i] = round_bf16(wv[i] * round_bf16(xv[i] * rr));
  unpack8(craw, cs);
  unpack8(sraw, sn);
  rope_vec(nv, cs, sn, sub, o);
  uint16_t* dst = kind == 0 ? qo + ((int64_t)t * HQ + hh) * D : ck + hh * skh + (int64_t)slot * skn;
  if (!slot_ok) {
    *reinterpret_cast<u32x4*>(dst + sub * 8) = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
    return;
  }
  *reinterpret_cast<u32x4*>(dst + sub * 8) = pack8(o);
}

namespace {

// RoPE of one row held by TPR lanes, 8 elements per lane (lanes with
// sub >= D / 8 idle); the rotate-half partner -- D / 2 elements, D / 16 lanes
// away -- comes through ds_bpermute.  The arithmetic of rope_vec.
__device__ __forceinline__ void rope_lanes(const float* xv, const float* cs, const float* sn, int lane, int sub, int D,
                                           float* o) {
  const int half = D >> 4;
  const int partner = lane - sub + (sub < half ? sub + half : sub - half);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float p = __int_as_float(__builtin_amdgcn_ds_bpermute(partner << 2, __float_as_int(xv[i])));
    const float rh = sub < half ? -p : p;
    o[i] = round_bf16(xv[i] * cs[i]) + round_bf16(rh * sn[i]);
  }
}

// RMSNorm of one D-element row on TPR lanes (the split rmsnorm_small_kernel
// uses for n = D: TPR 16 up to D = 128, else 64), then RoPE: nv = the
// normalised row, o = its rotation.
template <int TPR>
__device__ __forceinline__ void norm_rope_lanes(const float* xv, const u32x4& wraw, const u32x4& craw,
                                                const u32x4& sraw, int lane, int sub, int D, float eps, float* o) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xv[i], xv[i], ss);
  ss = lane_group_sum<TPR>(ss);
  const float rr = rsqrt_rn(ss / (float)D + eps);
  float wv[8], nv[8], cs[8], sn[8];
  unpack8(wraw, wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) nv[i] = round_bf16(wv[i] * round_bf16(xv[i] * rr));
  unpack8(craw, cs);
  unpack8(sraw, sn);
  rope_lanes(nv, cs, sn, lane, sub, D, o);
}

__device__ __forceinline__ u32x4 load8_or_zero(const uint16_t* p, bool ok) {
  return ok ? *reinterpret_cast<const u32x4*>(p) : u32x4{0u, 0u, 0u, 0u};
}

}  // namespace

// qk_norm_rope_row for head dims other than 128 (D % 16 == 0, D <= 512): a
// row on TPR lanes, 64 / TPR rows per wave.  Bitwise equal to rmsnorm
// followed by rope at the same D.
template <int TPR, bool NT = false>
__device__ __forceinline__ void qk_norm_rope_any_row(const QKArgs& a, int gid) {
  const int lane = __lane_id(), sub = lane % TPR;
  const int rowid = gid / TPR;
  const int nq = a.T * a.HQ;
  if (rowid >= nq + a.T * a.HK) return;   // whole lane groups leave together
  const bool isq = rowid < nq;
  const int r = isq ? rowid : rowid - nq;
  const int HH = isq ? a.HQ : a.HK;
  const int t = r / HH, hh = r - t * HH;
  const uint16_t* src = isq ? a.q + (int64_t)t * a.sqt + hh * a.sqh : a.k + (int64_t)t * a.skt + hh * a.skh;
  const bool act = sub * 8 < a.D;
  const u32x4 wraw = load8_or_zero((isq ? a.wq : a.wk) + sub * 8, act);
  const u32x4 craw = load8_or_zero(a.cosb + (int64_t)t * a.scs + sub * 8, act);
  const u32x4 sraw = load8_or_zero(a.sinb + (int64_t)t * a.scs + sub * 8, act);
  float xv[8], o[8];
  unpack8(load8_or_zero(src + sub * 8, act), xv);
  norm_rope_lanes<TPR>(xv, wraw, craw, sraw, lane, sub, a.D, a.eps, o);
  if (act) st16<NT>((isq ? a.qo : a.ko) + (int64_t)r * a.D + sub * 8, pack8(o));
}

template <int TPR>
__global__ __launch_bounds__(256) void qk_norm_rope_any_kernel(QKArgs a) {
  qk_norm_rope_any_row<TPR>(a, blockIdx.x * 256 + threadIdx.x);
}

// qkv_rope_cache_kernel for head dims other than 128 (D % 16 == 0,
// D <= 512), rows on TPR lanes as in qk_norm_rope_any_kernel; the same slot
// rules.
template <int SC, int TPR>
__global__ __launch_bounds__(256) void qkv_rope_cache_any_kernel(const uint16_t* qkv, int64_t sqkv, const float* qp,
                                                                 int S, int64_t sps, const uint16_t* wq,
                                                                 const uint16_t* wk, const uint16_t* cosb,
                                                                 const uint16_t* sinb, int64_t scs, const int* slots,
                                                                 int cap, uint16_t* ck, int64_t skh, int64_t skn,
                                                                 uint16_t* cv, int64_t svh, int64_t svn, uint16_t* qo,
                                                                 int T, int HQ, int HK, int D, float eps) {
  const int lane = __lane_id(), sub = lane % TPR;
  const int rowid = (blockIdx.x * 256 + threadIdx.x) / TPR;   // 32-bit: the host keeps the thread count below 2^31
  const int nq = T * HQ, nk = T * HK;
  if (rowid >= nq + 2 * nk) return;   // whole lane groups leave together
  int kind, t, hh;
  if (rowid < nq) { kind = 0; t = rowid / HQ; hh = rowid - t * HQ; }
  else if (rowid < nq + nk) { kind = 1; t = (rowid - nq) / HK; hh = rowid - nq - t * HK; }
  else { kind = 2; t = (rowid - nq - nk) / HK; hh = rowid - nq - nk - t * HK; }
  const int col = (kind == 0 ? hh : kind == 1 ? HQ + hh : HQ + HK + hh) * D + sub * 8;
  const bool act = sub * 8 < D;
  const u32x4 wraw = load8_or_zero((kind == 0 ? wq : wk) + sub * 8, act);
  const u32x4 craw = load8_or_zero(cosb + (int64_t)t * scs + sub * 8, act);
  const u32x4 sraw = load8_or_zero(sinb + (int64_t)t * scs + sub * 8, act);
  u32x4 raw = {0u, 0u, 0u, 0u};
  if (act) {
    if (qp) {  // the projection's fp32 chunk partials, summed and rounded as rspx_linear would
      f32x4 a, b;
      sum_parts8<SC>(qp + (int64_t)t * sqkv + col, S, sps, a, b);
      raw[0] = pack_bf16x2(a[0], a[1]); raw[1] = pack_bf16x2(a[2], a[3]);
      raw[2] = pack_bf16x2(b[0], b[1]); raw[3] = pack_bf16x2(b[2], b[3]);
    } else {
      raw = *reinterpret_cast<const u32x4*>(qkv + (int64_t)t * sqkv + col);
    }
  }
  const int slot = slots[t];
  const bool slot_ok = slot >= 0 && slot < cap;
  if (kind != 0 && !slot_ok) return;   // the whole row's group (same token) leaves
  if (kind == 2) {
    if (act) *reinterpret_cast<u32x4*>(cv + hh * svh + (int64_t)slot * svn + sub * 8) = raw;
    return;
  }
  float xv[8], o[8];
  unpack8(raw, xv);
  norm_rope_lanes<TPR>(xv, wraw, craw, sraw, lane, sub, D, eps, o);
  uint16_t* dst = kind == 0 ? qo + ((int64_t)t * HQ + hh) * D : ck + hh * skh + (int64_t)slot * skn;
  if (!act) return;
  if (!slot_ok) {
    *reinterpret_cast<u32x4*>(dst + sub * 8) = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
    return;
  }
  *reinterpret_cast<u32x4*>(dst + sub * 8) = pack8(o);
}

// RMSNorm of `rows` rows of n and the q/k RMSNorm + RoPE of T tokens in one
// launch, for a caller with both inputs ready: workgroups [0, nb) run the
// RMSNorm split rspx_rmsnorm uses for n (NK: 0 / 1 rows on 16 / 64 lanes,
// 2 .. 5 one workgroup per row with VPL 1, 1, 4, 8), the rest the q/k rows
// (QK: 0 for D = 128, else the lanes per row of the other head dims).  Each
// part runs the very code of its own kernel, so every output is bitwise what
// the two separate calls give; the stores are non-temporal (3.72 -> 3.39-3.50
// us for RMSNorm [64, 4096] + q/k [64, 40, 128] on MI355X).
template <int NK, int QK, int TH>
__global__ __launch_bounds__(TH) void rmsnorm_qk_norm_rope_kernel(RowIn in, const uint16_t* w, uint16_t* y,
                                                                  int64_t sy, int rows, int n, float eps, int nb,
                                                                  QKArgs a) {
  // The arguments either kind of workgroup needs before its loads, requested
  // in one batch (left to the compiler: three or four dependent scalar-load
  // round trips).
  asm volatile("" ::"s"(nb), "s"(in.x), "s"(in.sx), "s"(w), "s"(rows), "s"(n), "s"(a.q), "s"(a.k), "s"(a.sqt),
               "s"(a.sqh), "s"(a.skt), "s"(a.skh), "s"(a.wq), "s"(a.wk), "s"(a.cosb), "s"(a.sinb), "s"(a.scs),
               "s"(a.qo), "s"(a.ko), "s"(a.T), "s"(a.HQ), "s"(a.HK), "s"(a.D), "s"(a.eps), "s"(y), "s"(sy), "s"(eps));
  if ((int)blockIdx.x < nb) {
    if constexpr (NK <= 1) {
      constexpr int TPR = NK == 0 ? 16 : 64;
      const int row = (blockIdx.x * TH + threadIdx.x) / TPR;
      if (row < rows) rms_row_wave<TPR, 1, 0, 1, true>(in, row, w, y, sy, __lane_id() % TPR, n, eps);
    } else {
      constexpr int VPL = NK <= 3 ? 1 : NK == 4 ? 4 : 8;
      rms_row_block<VPL, 0, 1, TH, true>(in, w, y, sy, blockIdx.x, n, eps);
    }
    return;
  }
  const int gid = (blockIdx.x - nb) * TH + threadIdx.x;
  if constexpr (QK == 0) qk_norm_rope_row<true>(a, gid);
  else qk_norm_rope_any_row<QK, true>(a, gid);
}

}  // namespace rspx

using namespace rspx;

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

namespace rspx {
// The split depends on n only (never on rows), for every input mode.
template <int MODE, int SC>
static void launch_rmsnorm(const RowIn& in, const uint16_t* W, uint16_t* Y, int64_t sy, int rows, int n, float eps,
                           hipStream_t s) {
  const int vec = n / 8;
  if (vec <= 16) {
    hipLaunchKernelGGL((rmsnorm_small_kernel<16, 1, MODE, SC>), dim3((rows * 16 + 255) / 256), dim3(256), 0, s, in, W, Y,
                       sy, rows, n, eps);
  } else if (vec <= 64) {
    hipLaunchKernelGGL((rmsnorm_small_kernel<64, 1, MODE, SC>), dim3((rows * 64 + 255) / 256), dim3(256), 0, s, in, W, Y,
                       sy, rows, n, eps);
  } else if (vec <= 256) {
    hipLaunchKernelGGL((rmsnorm_row_kernel<1, MODE, SC>), dim3(rows), dim3(256), 0, s, in, W, Y, sy, n, eps);
  } else if (vec <= 512) {
    hipLaunchKernelGGL((rmsnorm_row_kernel<1, MODE, SC, 512>), dim3(rows), dim3(512), 0, s, in, W, Y, sy, n, eps);
  } else if (vec <= 1024) {
    hipLaunchKernelGGL((rmsnorm_row_kernel<4, MODE, SC>), dim3(rows), dim3(256), 0, s, in, W, Y, sy, n, eps);
  } else {
    hipLaunchKernelGGL((rmsnorm_row_kernel<8, MODE, SC>), dim3(rows), dim3(256), 0, s, in, W, Y, sy, n, eps);
  }
}
}  // namespace rspx

static int norm_args_ok(int rows, int n) {
  if (rows < 0 || n <= 0 || n % 8 != 0 || n > 16384) return n % 8 ? RSPX_EUNSUPPORTED : RSPX_EINVAL;
  return RSPX_OK;
}

// Row lengths the vector kernels take; every other n runs rmsnorm_any_kernel.
// The choice depends on n only.
static bool norm_fast(int n) { return n > 0 && n % 8 == 0 && n <= 16384; }

static bool al2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

// Any n (row-major output only): MODE 0 rmsnorm, MODE 1 residual add + rmsnorm.
template <int MODE>
static int rmsnorm_any(const RowIn& in, const void* w, void* y, int64_t sy, int rows, int n, float eps, void* stream) {
  if (rows < 0 || n <= 0) return RSPX_EINVAL;
  if (rows == 0) return RSPX_OK;
  if (!in.x || !w || !y || (MODE == 1 && (!in.h || !in.xo))) return RSPX_EINVAL;
  if (sy == kTiled) return RSPX_EUNSUPPORTED;   // the tiled layout needs n % 32 == 0
  if (sy < 0 || in.sx < 0) return RSPX_EINVAL;
  if (!al2(in.x) || !al2(w) || !al2(y) || (MODE == 1 && (!al2(in.h) || !al2(in.xo)))) return RSPX_EALIGN;
  hipLaunchKernelGGL((rmsnorm_any_kernel<MODE>), dim3((unsigned)rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     in, static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), sy, n, eps);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

// Output row stride: a multiple of 8 elements, or kTiled (then n % 32 == 0).
static int norm_out_ok(int64_t sy, int n) {
  if (sy == kTiled) return n % 32 == 0 ? RSPX_OK : RSPX_EUNSUPPORTED;
  if (sy < 0) return RSPX_EINVAL;
  return sy % 8 ? RSPX_EALIGN : RSPX_OK;
}

extern "C" int rspx_rmsnorm(const void* x, int64_t sx, const void* w, void* y, int64_t sy, int rows, int n,
                            float eps, void* stream) {
  if (!norm_fast(n)) {
    RowIn in{static_cast<const uint16_t*>(x), sx, nullptr, 0, nullptr, 0, 0, 1, nullptr, 0};
    return rmsnorm_any<0>(in, w, y, sy, rows, n, eps, stream);
  }
  int rc = norm_args_ok(rows, n);
  if (rc != RSPX_OK || rows == 0) return rc;
  if (!x || !w || !y) return RSPX_EINVAL;
  if (!al16(x) || !al16(w) || !al16(y) || sx % 8) return RSPX_EALIGN;
  if ((rc = norm_out_ok(sy, n)) != RSPX_OK) return rc;
  RowIn in{static_cast<const uint16_t*>(x), sx, nullptr, 0, nullptr, 0, 0, 1, nullptr, 0};
  launch_rmsnorm<0, 1>(in, static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), sy, rows, n, eps,
                    static_cast<hipStream_t>(stream));
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_add_rmsnorm(const void* r, int64_t sr, const void* h, int64_t sh, const void* w, void* xo,
                                int64_t sxo, void* y, int64_t sy, int rows, int n, float eps, void* stream) {
  if (!norm_fast(n)) {
    RowIn in{static_cast<const uint16_t*>(r), sr, static_cast<const uint16_t*>(h), sh, nullptr, 0, 0, 1,
             static_cast<uint16_t*>(xo), sxo};
    return rmsnorm_any<1>(in, w, y, sy, rows, n, eps, stream);
  }
  int rc = norm_args_ok(rows, n);
  if (rc != RSPX_OK || rows == 0) return rc;
  if (!r || !h || !w || !xo || !y) return RSPX_EINVAL;
  if (!al16(r) || !al16(h) || !al16(w) || !al16(xo) || !al16(y) || sr % 8 || sh % 8 || sxo % 8) return RSPX_EALIGN;
  if ((rc = norm_out_ok(sy, n)) != RSPX_OK) return rc;
  RowIn in{static_cast<const uint16_t*>(r), sr, static_cast<const uint16_t*>(h), sh, nullptr, 0, 0, 1,
           static_cast<uint16_t*>(xo), sxo};
  launch_rmsnorm<1, 1>(in, static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), sy, rows, n, eps,
                    static_cast<hipStream_t>(stream));
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_add_rmsnorm_partials(const void* r, int64_t sr, const float* hp, int S, const void* w, void* xo,
                                         int64_t sxo, void* y, int64_t sy, int rows, int n, float eps, void* stream) {
  int rc = norm_args_ok(rows, n);
  if (rc != RSPX_OK || rows == 0) return rc;
  if (S < 1 || S > kMaxSplits) return RSPX_EINVAL;
  if (!r || !hp || !w || !xo || !y) return RSPX_EINVAL;
  if (!al16(r) || !al16(hp) || !al16(w) || !al16(xo) || !al16(y) || sr % 8 || sxo % 8) return RSPX_EALIGN;
  if ((rc = norm_out_ok(sy, n)) != RSPX_OK) return rc;
  RowIn in{static_cast<const uint16_t*>(r), sr, nullptr, 0, hp, n, (int64_t)rows * n, S, static_cast<uint16_t*>(xo),
           sxo};
  RSPX_WITH_SPLITS(S, SC, launch_rmsnorm<2, SC>(in, static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), sy,
                                                  rows, n, eps, static_cast<hipStream_t>(stream)));
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxl, const void* cosb, const void* sinb,
                         int64_t scb, int64_t scl, void* y, int B, int H, int L, int D, void* stream) {
  if (B < 0 || H < 0 || L < 0 || D <= 0) return RSPX_EINVAL;
  if (D % 16 != 0 || D > 512) return RSPX_EUNSUPPORTED;
  const int64_t rows = (int64_t)B * H * L;
  if (rows == 0) return RSPX_OK;
  if (!x || !cosb || !sinb || !y) return RSPX_EINVAL;
  if (!al16(x) || !al16(cosb) || !al16(sinb) || !al16(y) || sxb % 8 || sxh % 8 || sxl % 8 || scb % 8 || scl % 8)
    return RSPX_EALIGN;
  if (D != 128) {
    const int64_t waves = (rows + 64 / (D / 8) - 1) / (64 / (D / 8));
    if ((waves + 3) / 4 > 0x7fffffff) return RSPX_EUNSUPPORTED;
    hipLaunchKernelGGL(rope_any_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), sxb, sxh, sxl,
                       static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb), scb, scl,
                       static_cast<uint16_t*>(y), B, H, L, D);
    return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
  }
  const int64_t threads = rows * 16;
  if (threads + 255 >= 0x7fffff00) return RSPX_EUNSUPPORTED;   // 32-bit thread indices
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), sxb, sxh, sxl,
                     static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb), scb, scl,
                     static_cast<uint16_t*>(y), B, H, L);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

// The q/k part's checks; fills a.
static int qk_args(const void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt, int64_t skh, const void* wq,
                   const void* wk, const void* cosb, const void* sinb, int64_t scs, void* qo, void* ko, int T, int HQ,
                   int HK, int D, float eps, QKArgs& a) {
  if (T < 0 || HQ < 0 || HK < 0 || D <= 0) return RSPX_EINVAL;
  if (D % 16 != 0 || D > 512) return RSPX_EUNSUPPORTED;
  a = QKArgs{static_cast<const uint16_t*>(q), sqt, sqh, static_cast<const uint16_t*>(k), skt, skh,
             static_cast<const uint16_t*>(wq), static_cast<const uint16_t*>(wk), static_cast<const uint16_t*>(cosb),
             static_cast<const uint16_t*>(sinb), scs, static_cast<uint16_t*>(qo), static_cast<uint16_t*>(ko), T, HQ,
             HK, D, eps};
  if ((int64_t)T * (HQ + HK) == 0) return RSPX_OK;
  if (!q || !k || !wq || !wk || !cosb || !sinb || !qo || !ko) return RSPX_EINVAL;
  const void* ps[] = {q, k, wq, wk, cosb, sinb, qo, ko};
  for (const void* p : ps)
    if (!al16(p)) return RSPX_EALIGN;
  if (sqt % 8 || sqh % 8 || skt % 8 || skh % 8 || scs % 8) return RSPX_EALIGN;
  return RSPX_OK;
}

// Lanes per q/k row: 16 (D = 128 on its own code, or D < 128), 64 above.
static int qk_lanes(int D) { return D <= 128 ? 16 : 64; }

extern "C" int rspx_qk_norm_rope(const void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt,
                                 int64_t skh, const void* wq, const void* wk, const void* cosb,
                                 const void* sinb, int64_t scs, void* qo, void* ko, int T, int HQ, int HK,
                                 int D, float eps, void* stream) {
  QKArgs a;
  int rc = qk_args(q, sqt, sqh, k, skt, skh, wq, wk, cosb, sinb, scs, qo, ko, T, HQ, HK, D, eps, a);
  const int64_t rows = (int64_t)T * (HQ + HK);
  if (rc != RSPX_OK || rows == 0) return rc;
  if (rows * qk_lanes(D) >= 0x7fffff00) return RSPX_EUNSUPPORTED;   // 32-bit thread indices
  const int64_t blocks = (rows * qk_lanes(D) + 255) / 256;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else if (D < 128) hipLaunchKernelGGL((qk_norm_rope_any_kernel<16>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((qk_norm_rope_any_kernel<64>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_rmsnorm_qk_norm_rope(const void* x, int64_t sx, const void* w, void* y, int64_t sy, int rows,
                                         int n, float eps, const void* q, int64_t sqt, int64_t sqh, const void* k,
                                         int64_t skt, int64_t skh, const void* wq, const void* wk, const void* cosb,
                                         const void* sinb, int64_t scs, void* qo, void* ko, int T, int HQ, int HK,
                                         int D, float qk_eps, void* stream) {
  // The RMSNorm part: the rules of rspx_rmsnorm's vector kernels.
  if (rows < 0 || n <= 0) return RSPX_EINVAL;
  if (!norm_fast(n)) return RSPX_EUNSUPPORTED;
  if (rows > 0) {
    if (!x || !w || !y) return RSPX_EINVAL;
    if (!al16(x) || !al16(w) || !al16(y) || sx % 8) return RSPX_EALIGN;
    const int rc = norm_out_ok(sy, n);
    if (rc != RSPX_OK) return rc;
  }
  QKArgs a;
  const int rc = qk_args(q, sqt, sqh, k, skt, skh, wq, wk, cosb, sinb, scs, qo, ko, T, HQ, HK, D, qk_eps, a);
  if (rc != RSPX_OK) return rc;
  const int vec = n / 8;
  const int nk = vec <= 16 ? 0 : vec <= 64 ? 1 : vec <= 256 ? 2 : vec <= 512 ? 3 : vec <= 1024 ? 4 : 5;
  const int th = nk == 3 ? 512 : 256;
  const int64_t nb = nk == 0 ? ((int64_t)rows * 16 + 255) / 256 : nk == 1 ? ((int64_t)rows * 64 + 255) / 256 : rows;
  const int64_t qrows = (int64_t)T * (HQ + HK);
  const int64_t blocks = nb + (qrows * qk_lanes(D) + th - 1) / th;
  if (blocks == 0) return RSPX_OK;
  if (qrows * qk_lanes(D) >= 0x7fffff00 || blocks > 0x7fffffff) return RSPX_EUNSUPPORTED;
  RowIn in{static_cast<const uint16_t*>(x), sx, nullptr, 0, nullptr, 0, 0, 1, nullptr, 0};
  const uint16_t* W = static_cast<const uint16_t*>(w);
  uint16_t* Y = static_cast<uint16_t*>(y);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)blocks);
#define RSPX_NQR(NK, TH)                                                                                        \
  if (D == 128)                                                                                                 \
    hipLaunchKernelGGL((rmsnorm_qk_norm_rope_kernel<NK, 0, TH>), g, dim3(TH), 0, s, in, W, Y, sy, rows, n, eps, \
                       (int)nb, a);                                                                             \
  else if (D < 128)                                                                                             \
    hipLaunchKernelGGL((rmsnorm_qk_norm_rope_kernel<NK, 16, TH>), g, dim3(TH), 0, s, in, W, Y, sy, rows, n, eps,\
                       (int)nb, a);                                                                             \
  else                                                                                                          \
    hipLaunchKernelGGL((rmsnorm_qk_norm_rope_kernel<NK, 64, TH>), g, dim3(TH), 0, s, in, W, Y, sy, rows, n, eps,\
                       (int)nb, a);
  switch (nk) {
    case 0: RSPX_NQR(0, 256) break;
    case 1: RSPX_NQR(1, 256) break;
    case 2: RSPX_NQR(2, 256) break;
    case 3: RSPX_NQR(3, 512) break;
    case 4: RSPX_NQR(4, 256) break;
    default: RSPX_NQR(5, 256) break;
  }
#undef RSPX_NQR
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

static int qkv_rope_cache_launch(const uint16_t* qkv, int64_t sqkv, const float* qp, int S, int64_t sps,
                                 const void* wq, const void* wk, const void* cosb, const void* sinb, int64_t scs,
                                 const int32_t* slots, int cap, void* cache_k, int64_t skh, int64_t skn, void* cache_v,
                                 int64_t svh, int64_t svn, void* qo, int T, int HQ, int HK, int D, float eps,
                                 void* stream) {
  if (T < 0 || HQ <= 0 || HK <= 0 || cap < 0 || D <= 0) return RSPX_EINVAL;
  if (D % 16 != 0 || D > 512) return RSPX_EUNSUPPORTED;
  if (T == 0) return RSPX_OK;
  if ((!qkv && !qp) || !wq || !wk || !cosb || !sinb || !slots || !cache_k || !cache_v || !qo) return RSPX_EINVAL;
  const void* ps[] = {wq, wk, cosb, sinb, cache_k, cache_v, qo};
  for (const void* p : ps)
    if (!al16(p)) return RSPX_EALIGN;
  if ((qkv && !al16(qkv)) || (qp && !al16(qp))) return RSPX_EALIGN;
  if (sqkv % 8 || scs % 8 || skh % 8 || skn % 8 || svh % 8 || svn % 8) return RSPX_EALIGN;
  if (sqkv < (int64_t)(HQ + 2 * HK) * D) return RSPX_EINVAL;
  if (D != 128) {
    const int tpr = D <= 128 ? 16 : 64;
    const int64_t blocks = ((int64_t)T * (HQ + 2 * HK) * tpr + 255) / 256;
    if (blocks * 256 >= 0x7fffff00) return RSPX_EUNSUPPORTED;   // 32-bit thread indices
#define RSPX_QKVC_ANY(TPR)                                                                                      \
  RSPX_WITH_SPLITS(qp ? S : 1, SC,                                                                              \
                   hipLaunchKernelGGL((qkv_rope_cache_any_kernel<SC, TPR>), dim3((unsigned)blocks), dim3(256), 0, \
                                      static_cast<hipStream_t>(stream), qkv, sqkv, qp, S, sps,                  \
                                      static_cast<const uint16_t*>(wq), static_cast<const uint16_t*>(wk),       \
                                      static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb),   \
                                      scs, slots, cap, static_cast<uint16_t*>(cache_k), skh, skn,               \
                                      static_cast<uint16_t*>(cache_v), svh, svn, static_cast<uint16_t*>(qo), T, \
                                      HQ, HK, D, eps))
    if (tpr == 16) RSPX_QKVC_ANY(16);
    else RSPX_QKVC_ANY(64);
#undef RSPX_QKVC_ANY
    return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
  }
  const int64_t per_token = (int64_t)(HQ + 2 * HK) * 16;
  if (per_token + 255 >= 0x7fffff00) return RSPX_EUNSUPPORTED;   // 32-bit thread indices
  const unsigned bx = (unsigned)((per_token + 255) / 256);
  for (int t0 = 0; t0 < T; t0 += 65535) {   // one launch per 65535 tokens
    const dim3 grid(bx, (unsigned)min(T - t0, 65535));
    RSPX_WITH_SPLITS(qp ? S : 1, SC,
                     hipLaunchKernelGGL((qkv_rope_cache_kernel<SC>), grid, dim3(256), 0,
                                        static_cast<hipStream_t>(stream), qkv, sqkv, qp, S, sps,
                                        static_cast<const uint16_t*>(wq), static_cast<const uint16_t*>(wk),
                                        static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb), scs,
                                        slots, cap, static_cast<uint16_t*>(cache_k), skh, skn,
                                        static_cast<uint16_t*>(cache_v), svh, svn, static_cast<uint16_t*>(qo), t0, HQ,
                                        HK, eps));
  }
  return hipGetLastError() == hipSuccess ? RSPX_OK : RSPX_ELAUNCH;
}

extern "C" int rspx_qkv_rope_cache(const void* qkv, int64_t sqkv, const void* wq, const void* wk, const void* cosb,
                                   const void* sinb, int64_t scs, const int32_t* slots, int cap, void* cache_k,
                                   int64_t skh, int64_t skn, void* cache_v, int64_t svh, int64_t svn, void* qo, int T,
                                   int HQ, int HK, int D, float eps, void* stream) {
  if (!qkv) return RSPX_EINVAL;
  return qkv_rope_cache_launch(static_cast<const uint16_t*>(qkv), sqkv, nullptr, 1, 0, wq, wk, cosb, sinb, scs, slots,
                               cap, cache_k, skh, skn, cache_v, svh, svn, qo, T, HQ, HK, D, eps, stream);
}

extern "C" int rspx_qkv_rope_cache_partials(const float* qkvp, int S, const void* wq, const void* wk,
                                            const void* cosb, const void* sinb, int64_t scs, const int32_t* slots,
                                            int cap, void* cache_k, int64_t skh, int64_t skn, void* cache_v, int64_t svh,
                                            int64_t svn, void* qo, int T, int HQ, int HK, int D, float eps,
                                            void* stream) {
  if (!qkvp || S < 1 || S > kMaxSplits) return RSPX_EINVAL;
  const int64_t n = (int64_t)(HQ + 2 * HK) * D;
  return qkv_rope_cache_launch(nullptr, n, qkvp, S, (int64_t)T * n, wq, wk, cosb, sinb, scs, slots, cap, cache_k, skh,
                               skn, cache_v, svh, svn, qo, T, HQ, HK, D, eps, stream);
}
