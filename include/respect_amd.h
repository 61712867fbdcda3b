/* respect_amd.h -- C ABI of the MI355X (gfx950) deterministic verification
 * kernels.
 *
 * Every entry point takes device pointers, element strides and sizes, and a
 * hipStream_t passed as void*.  Work is enqueued on that stream; nothing
 * blocks the host.  Tensors are bf16 (passed as uint16_t bit patterns) unless
 * stated otherwise; the innermost (feature) dimension must be contiguous.
 * The return value is RSPX_OK or a negative RSPX_E* code; no exception or
 * abort ever crosses this boundary.
 *
 * Reference interfaces replaced (soonhong99/respect, file:line):
 *   rspx_trie_attn      respect/kernels/attention.py:74  fused_attn_hyb(q, kp, vp, kn, vn, msk, sm_scale)
 *   rspx_rmsnorm        respect/kernels/rmsnorm.py:25    rmsnorm(x, w, eps)
 *   rspx_rope           respect/system/fused.py:67       rope(x, cos, sin)
 *   rspx_qk_norm_rope   respect/kernels/rmsnorm.py:25 followed by the RoPE of
 *                       HF apply_rotary_pos_emb (q_norm/k_norm + RoPE of one decoder layer)
 *   rspx_silu_mul       respect/system/fused.py:116      silu_mul(g, u)
 */
#ifndef RESPECT_AMD_H
#define RESPECT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RSPX_OK 0
#define RSPX_EINVAL (-1)       /* bad size, stride or null pointer */
#define RSPX_EUNSUPPORTED (-2) /* head_dim / GQA ratio / dtype not built */
#define RSPX_EWORKSPACE (-3)   /* workspace missing or too small */
#define RSPX_EALIGN (-4)       /* pointer or stride not 16-byte aligned */
#define RSPX_ELAUNCH (-5)      /* HIP launch error */

/* Human-readable text for an RSPX_* code (static storage). */
const char* rspx_strerror(int code);

/* Library version, e.g. "respect_amd 0.1.0 gfx950". */
const char* rspx_version(void);

/* ---------------------------------------------------------------- attention
 * Trie-verification attention (replaces respect/kernels/attention.py:74-96).
 *
 *   q   [H, M, D]    query rows (M = query tokens / trie nodes)
 *   kp  [HK, P, D]   prompt keys   (slots [0, P) of the cache; never masked)
 *   vp  [HK, P, D]   prompt values
 *   kn  [HK, NN, D]  node keys     (slots P.. of the cache: committed tokens and trie nodes)
 *   vn  [HK, NN, D]  node values
 *   msk [M, NN]      uint8/bool, nonzero = row may attend to that node slot
 *   out [H, M, D]    bf16 result
 *
 * P is explicit (in the reference it is kp.shape[1]).  Strides are in
 * elements; the D axis must have stride 1.  q/k/v/out base pointers and
 * head/row strides must be 16-byte aligned (strides multiple of 8 elements).
 * Head h reads kv head h / (H / HK).  D in {64, 128}; H / HK in {1,2,4,8,16}.
 *
 * Result per (head, row): softmax over the P prompt keys and the allowed node
 * slots, fp32 accumulation, one bf16 rounding at the end.  The reduction
 * order is a fixed function of P and of the row's allowed node slots taken
 * in slot order: it does not depend on M, on where the allowed slots sit in
 * [0, NN), on masked slots, or on the other rows.
 *
 * workspace: device memory of at least rspx_trie_attn_workspace_bytes(...)
 * bytes (16-byte aligned, contents irrelevant) that holds the per-group
 * partial results between the two kernels of a call.  A workspace must not be
 * used by two calls that can run at the same time (different streams).
 * NN <= 4096 (the node-slot limit of the reference dispatcher, NMAX).
 *
 * rows_per_wave: 0 = automatic, else 1 or 2 (16-row tiles per wave).  It
 * changes only the work distribution, never the result.
 */

int64_t rspx_trie_attn_workspace_bytes(int H, int HK, int M, int P, int D);

int rspx_trie_attn(const void* q, int64_t sqh, int64_t sqm,
                   const void* kp, int64_t skph, int64_t skpn,
                   const void* vp, int64_t svph, int64_t svpn,
                   const void* kn, int64_t sknh, int64_t sknn,
                   const void* vn, int64_t svnh, int64_t svnn,
                   const uint8_t* msk, int64_t smm, int64_t smn,
                   void* out, int64_t soh, int64_t som,
                   int H, int HK, int M, int P, int NN, int D, float sm_scale,
                   void* workspace, int64_t workspace_bytes, int rows_per_wave,
                   void* stream);

/* ---------------------------------------------------------------- RMSNorm
 * y[r] = bf16(w * bf16(x[r] * rsqrt(mean(x[r]^2) + eps))), fp32 statistics
 * (replaces respect/kernels/rmsnorm.py:25 rmsnorm(x, w, eps)).
 * x, y: [rows, n] with row strides sx, sy (elements); w: [n].  n % 8 == 0,
 * n <= 16384.  The sum of squares of a row is taken in an order fixed by n,
 * so a row's output does not depend on `rows`.
 */
int rspx_rmsnorm(const void* x, int64_t sx, const void* w, void* y, int64_t sy, int rows, int n, float eps,
                 void* stream);

/* ---------------------------------------------------------------- RoPE
 * y = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin))   (replaces
 * respect/system/fused.py:67 rope(x, cos, sin) for bf16 inputs).
 * x: [B, H, L, D] with strides sxb, sxh, sxl; cos/sin: [B, L, D] with strides
 * scb, scl; y: [B, H, L, D] contiguous.  D == 128.  Bitwise equal to PyTorch's
 * bf16 elementwise ops.
 */
int rspx_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxl, const void* cos, const void* sin,
              int64_t scb, int64_t scl, void* y, int B, int H, int L, int D, void* stream);

/* ---------------------------------------------------------------- q/k norm + RoPE
 * The q_norm / k_norm RMSNorm over head_dim followed by RoPE, for all query
 * and key heads of T tokens in one launch (replaces rmsnorm
 * respect/kernels/rmsnorm.py:25 on q/k heads followed by HF
 * apply_rotary_pos_emb).  q: [T, HQ, D] (strides sqt, sqh), k: [T, HK, D]
 * (skt, skh), wq/wk: [D], cos/sin: [T, D] (row stride scs), qo: [T, HQ, D],
 * ko: [T, HK, D] contiguous.  D == 128.  Bitwise equal to rspx_rmsnorm
 * followed by rspx_rope.
 */
int rspx_qk_norm_rope(const void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt, int64_t skh,
                      const void* wq, const void* wk, const void* cos, const void* sin, int64_t scs, void* qo,
                      void* ko, int T, int HQ, int HK, int D, float eps, void* stream);

/* ---------------------------------------------------------------- SwiGLU
 * y = bf16(bf16(g / (1 + exp(-g))) * u)  (replaces respect/system/fused.py:116
 * silu_mul(g, u)).  g, u, y: [rows, cols] with row strides sg, su, sy; views
 * into one packed gate/up tensor are fine.  cols % 8 == 0.
 */
int rspx_silu_mul(const void* g, int64_t sg, const void* u, int64_t su, void* y, int64_t sy, int rows, int cols,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RESPECT_AMD_H */
