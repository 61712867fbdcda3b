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
 *   rspx_rmsnorm_qk_norm_rope  rspx_rmsnorm and rspx_qk_norm_rope in one launch (no counterpart)
 *   rspx_silu_mul       respect/system/fused.py:116      silu_mul(g, u)
 *   rspx_linear         respect/kernels/gemm.py:30       linear(x, w, ..., out_dtype)
 *   rspx_add_rmsnorm    residual add (HF decoder layer) followed by rmsnorm, rmsnorm.py:25
 *   rspx_qkv_rope_cache q_norm/k_norm + RoPE + KV write of one decoder layer
 *                       (rmsnorm.py:25, HF apply_rotary_pos_emb, kv_buffer.py:32-36 update)
 *   rspx_trie_mask      respect/decoding/verify.py:22-41 mask + dispatch.py:94-115 padding
 *   rspx_kv_compact     respect/decoding/kv_buffer.py:93 compact(cache, prompt_len, base, slots)
 *   rspx_argmax_rows    respect/decoding/acceptance.py:20 greedy_token(logits, offset, size)
 *   rspx_square         respect/system/fused.py:126 _sq_k (the squares of rmsnorm, fused.py:176)
 *   rspx_add_sq         respect/system/fused.py:185 add_sq(r, h)
 *   rspx_norm_apply     respect/system/fused.py:148 _norm_apply_k (norm_from, fused.py:165)
 *   rspx_rope_vision    respect/system/fused.py:97  rope_vision(x, cos, sin)
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

/* Tiled activation layout.  Passed as the row stride of a bf16 activation
 * matrix A[M, K] with K % 32 == 0 -- x of rspx_linear, rspx_linear_silu and
 * rspx_linear_partials; y of rspx_rmsnorm, rspx_add_rmsnorm and
 * rspx_add_rmsnorm_partials; out of rspx_linear_silu; out of rspx_trie_attn
 * as the [M, H D] matrix (som = RSPX_TILED, soh = D) -- RSPX_TILED names
 * this layout instead of row-major: element (m, k) sits at
 *   ((((m / 64) * (K / 32) + k / 32) * 4 + (m % 64) / 16) * 64
 *      + m % 16 + 16 * ((k % 32) / 8)) * 8 + k % 8,
 * i.e. for each 64-row block and 32-wide k-block the four 16 x 32 MFMA
 * operand tiles of that block, 1 KB each.  The buffer must hold
 * ceil(M / 64) * 64 * K elements; what rows M .. of the last block hold never
 * reaches a result.  The linear layers load a tiled x a whole tile per
 * instruction and give bit for bit the results of the same x row-major.  No
 * counterpart in the reference: an activation layout of the decoder step.
 */
#define RSPX_TILED ((int64_t)-1)

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
 * Head h reads kv head h / (H / HK).  D in {32, 64, 128, 256} (the head_dims
 * of reference_blocked.py:89); H / HK in {1,2,4,8,16}.
 *
 * Result per (head, row): softmax over the P prompt keys and the allowed node
 * slots, fp32 accumulation, one bf16 rounding at the end.  The reduction
 * order is a fixed function of P and of the row's allowed node slots taken
 * in slot order: it does not depend on M, on where the allowed slots sit in
 * [0, NN), on masked slots, or on the other rows.
 *
 * workspace: device memory of at least rspx_trie_attn_workspace_bytes(...)
 * bytes, 16-byte aligned and zero-filled before its first use; every call
 * moves each per-row-block counter it uses (in the first 16 KiB, at the same
 * place for every shape) by exactly 8, so they stay multiples of 8 between
 * calls and calls of any shapes may share one workspace in turn.  It holds those words (per-row-block counters of the one-launch
 * path) and the per-group partial results.  A workspace must not be used by
 * two calls that can run at the same time.
 * NN <= 4096 (the node-slot limit of the reference dispatcher, NMAX).
 *
 * Launches: one (prompt groups, node partials and merge in one kernel whose
 * workgroups wait for each other; used when the grid, or half of it with two
 * row blocks per workgroup, fits on the device at once) or two (prompt
 * groups, then node partials and merge).  All give the same bits.
 *
 * rows_per_wave: 0 = automatic (one 16-row tile per wave when that grid
 * fits on the device at once, e.g. 1-token calls; two otherwise), else 1 or
 * 2.  It changes only the work distribution, never the result.  D = 256
 * always runs one (2 returns RSPX_EUNSUPPORTED).
 *
 * out: element (head h, row m, d) at h soh + m som + d; or, with som =
 * RSPX_TILED and soh = D (no counterpart in the reference), column h D + d of
 * row m of the [M, H D] matrix in the tiled activation layout (ceil(M / 64) 64
 * H D elements), the x the o projection of the decoder step reads fastest.
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

/* rspx_trie_attn with the launch count forced: launches = 1 (the one-kernel
 * path; falls back to two when the grid does not fit) or 2.  For tests and
 * measurements; the result is the same either way.
 */
int rspx_trie_attn_launches(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                            const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh, int64_t sknn,
                            const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk, int64_t smm, int64_t smn,
                            void* out, int64_t soh, int64_t som, int H, int HK, int M, int P, int NN, int D,
                            float sm_scale, void* workspace, int64_t workspace_bytes, int rows_per_wave, int launches,
                            void* stream);

/* 1 if a one-launch call on this workspace ran out of its bounded wait since
 * the flag was last cleared, 0 if not, < 0 on error; a set flag is cleared
 * (each failure is reported once).  workspace NULL: the static scratch of
 * rspx_trie_attn_noalloc on the current device.  Synchronises the stream, so
 * it cannot be called under graph capture.  A workgroup whose wait runs out
 * (after 4 ms of the device's real-time counter) stores NaN in every element
 * of the output rows it merges, so such a call's output carries the failure
 * without this query.  The flag is the workspace's first int
 * (RSPX_ATTN_STATUS_WORD): a caller may copy it to the host with a copy it
 * already makes instead of calling this function, and zero it itself.
 */
#define RSPX_ATTN_STATUS_WORD 0
int rspx_trie_attn_status(void* workspace, int H, int HK, int M, int P, int D, void* stream);

/* rspx_trie_attn without a workspace argument: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * scratch is a 32 MiB array in the library's code object, one per GPU,
 * held until the process ends; the call allocates nothing.  Calls whose
 * rspx_trie_attn_workspace_bytes(H, HK, M, P, D) exceeds 32 MiB return
 * RSPX_EWORKSPACE (the 8B shape holds up to 251 query rows at 3072 prompt
 * keys).  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two host threads) race and give invalid results.
 * The array is zero when the library is loaded (static storage), so no call
 * needs a fill first, on any stream; its timeout flag is read and cleared by
 * rspx_trie_attn_status(NULL, ...).  Same results, bit for bit, as
 * rspx_trie_attn.
 */
int rspx_trie_attn_noalloc(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                           const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh, int64_t sknn,
                           const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk, int64_t smm, int64_t smn,
                           void* out, int64_t soh, int64_t som, int H, int HK, int M, int P, int NN, int D,
                           float sm_scale, int rows_per_wave, void* stream);

/* ---------------------------------------------------------------- tile-wise (blocked) attention
 * The negative control of the slot-layout experiment, replacing
 * respect/kernels/reference_blocked.py:83 fused_attn(q, kp, vp, kn, vn, msk,
 * sm_scale, BM, BN, ...): the same arguments as rspx_trie_attn (no
 * workspace), but node slots reduced tile by tile (BN in {32, 64, 128}) like
 * the prompt, one online-softmax update per tile, bf16 probabilities in every
 * PV product -- so the result depends on where the node slots sit.  D in
 * {32, 64, 128, 256}.  Output row stride and base 8-byte aligned.
 */
int rspx_blocked_attn(const void* q, int64_t sqh, int64_t sqm, const void* kp, int64_t skph, int64_t skpn,
                      const void* vp, int64_t svph, int64_t svpn, const void* kn, int64_t sknh, int64_t sknn,
                      const void* vn, int64_t svnh, int64_t svnn, const uint8_t* msk, int64_t smm, int64_t smn,
                      void* out, int64_t soh, int64_t som, int H, int HK, int M, int P, int NN, int D, int BN,
                      float sm_scale, void* stream);

/* Test hook, no counterpart in the reference: sets how many times a one-launch
 * workgroup polls its row block's counter before its wait gives up (a
 * negative value restores the default: no poll bound, the 4 ms deadline
 * alone ends a wait); returns the previous value.  Lets a test drive the
 * give-up path (0 polls: every wait gives up at once) while every kernel still
 * exits normally.  Process-wide, not thread-safe; read at each launch.
 */
int rspx_trie_attn_set_spin_limit(int polls);

/* ---------------------------------------------------------------- RMSNorm
 * y[r] = bf16(w * bf16(x[r] * rsqrt(mean(x[r]^2) + eps))), fp32 statistics
 * (replaces respect/kernels/rmsnorm.py:25 rmsnorm(x, w, eps)).
 * x, y: [rows, n] with row strides sx, sy (elements; sy may be RSPX_TILED,
 * then n % 32 == 0); w: [n].  Any n > 0 (the reference's rmsnorm masks any
 * N, rmsnorm.py:25-32): n % 8 == 0 and n <= 16384 take vectorised kernels
 * (pointers and strides 16-byte aligned, RSPX_EALIGN otherwise); every other
 * n a one-workgroup-per-row kernel with 2-byte element loads (2-byte
 * alignment; row-major y only).  The sum of squares of a row is taken in an
 * order fixed by n, so a row's output does not depend on `rows`.
 */
int rspx_rmsnorm(const void* x, int64_t sx, const void* w, void* y, int64_t sy, int rows, int n, float eps,
                 void* stream);

/* ---------------------------------------------------------------- RoPE
 * y = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin))   (replaces
 * respect/system/fused.py:67 rope(x, cos, sin) for bf16 inputs).
 * x: [B, H, L, D] with strides sxb, sxh, sxl; cos/sin: [B, L, D] with strides
 * scb, scl; y: [B, H, L, D] contiguous.  Any D with D % 16 == 0 and
 * D <= 512 (RSPX_EUNSUPPORTED otherwise; the reference's kernel masks a
 * power-of-two tile, fused.py:47-75).  Bitwise equal to PyTorch's bf16
 * elementwise ops.
 */
int rspx_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxl, const void* cos, const void* sin,
              int64_t scb, int64_t scl, void* y, int B, int H, int L, int D, void* stream);

/* ---------------------------------------------------------------- q/k norm + RoPE
 * The q_norm / k_norm RMSNorm over head_dim followed by RoPE, for all query
 * and key heads of T tokens in one launch (replaces rmsnorm
 * respect/kernels/rmsnorm.py:25 on q/k heads followed by HF
 * apply_rotary_pos_emb).  q: [T, HQ, D] (strides sqt, sqh), k: [T, HK, D]
 * (skt, skh), wq/wk: [D], cos/sin: [T, D] (row stride scs), qo: [T, HQ, D],
 * ko: [T, HK, D] contiguous.  D % 16 == 0, D <= 512 (the head dims
 * rspx_rope takes; RSPX_EUNSUPPORTED otherwise).  Bitwise equal to
 * rspx_rmsnorm followed by rspx_rope at the same D.
 */
int rspx_qk_norm_rope(const void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt, int64_t skh,
                      const void* wq, const void* wk, const void* cos, const void* sin, int64_t scs, void* qo,
                      void* ko, int T, int HQ, int HK, int D, float eps, void* stream);

/* rspx_rmsnorm (x, w, y over rows x n, eps) and rspx_qk_norm_rope (q .. D,
 * qk_eps) in one launch, for a caller whose two inputs are both ready: the
 * RMSNorm rows and the q/k rows run in disjoint workgroups of one grid, each
 * on the code of its own kernel, so every output is bitwise what the two
 * calls give.  The size rules of both, with n % 8 == 0 and n <= 16384
 * (RSPX_EUNSUPPORTED otherwise).  No counterpart in the reference, whose
 * RMSNorm (rmsnorm.py:25) and RoPE (fused.py:67) are separate launches: it
 * saves one launch where both stages are due together, as in the
 * RMSNorm [64, 4096] + q/k RoPE workload of the element-wise benchmark.
 */
int rspx_rmsnorm_qk_norm_rope(const void* x, int64_t sx, const void* w, void* y, int64_t sy, int rows, int n,
                              float eps, const void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt,
                              int64_t skh, const void* wq, const void* wk, const void* cos, const void* sin,
                              int64_t scs, void* qo, void* ko, int T, int HQ, int HK, int D, float qk_eps,
                              void* stream);

/* ---------------------------------------------------------------- SwiGLU
 * y = bf16(bf16(g / (1 + exp(-g))) * u)  (replaces respect/system/fused.py:116
 * silu_mul(g, u)).  g, u, y: [rows, cols] with row strides sg, su, sy; views
 * into one packed gate/up tensor are fine.  Any cols; 2-byte alignment (two
 * elements per thread where cols, the strides and the pointers are even).
 */
int rspx_silu_mul(const void* g, int64_t sg, const void* u, int64_t su, void* y, int64_t sy, int rows, int cols,
                  void* stream);

/* ---------------------------------------------------------------- linear
 * out[M, N] = x[M, K] . w[N, K]^T, bf16 inputs, fp32 accumulation, output
 * bf16 (out_fp32 = 0) or fp32 (out_fp32 = 1) (replaces
 * respect/kernels/gemm.py:30 linear(x, w, ..., out_dtype); bias is the
 * caller's, as in the reference).  Row strides sx, sw, so in elements; rows
 * 16-byte aligned; sx may be RSPX_TILED, and so may sw: w is then in the
 * tiled weight layout rspx_linear_tile_weight writes (same results, bit for
 * bit).  Any M, N, K (the reference's kernel masks every edge,
 * gemm.py:19-27): with N % 16 == 0 and K % 256 == 0 the streaming kernel
 * runs; any other (N, K) runs one bounded-load MFMA chain per output tile,
 * row-major operands only (RSPX_EUNSUPPORTED for RSPX_TILED), 2-byte
 * alignment (4-byte for an fp32 out), row strides below 2^24 elements.
 *
 * Reduction order: K is cut into rspx_linear_splits(N, K) equal chunks (a
 * function of N and K only; 1 outside N % 16 == 0, K % 256 == 0); each chunk
 * is a fixed chain of bf16 MFMAs over 32-wide k-blocks in increasing k (k
 * past K reads as zero); chunk results are added in chunk order and rounded
 * once.  A row's output bits therefore do not depend on M.  With more than
 * one chunk the fp32 chunk partials go through `workspace`
 * (rspx_linear_workspace_bytes(M, N, K) bytes, 16-byte aligned; 0 with one
 * chunk).
 */
int rspx_linear_splits(int N, int K);
int64_t rspx_linear_workspace_bytes(int M, int N, int K);
int rspx_linear(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M, int N, int K,
                int out_fp32, void* workspace, int64_t workspace_bytes, void* stream);

/* Gate/up projection with SwiGLU in its epilogue: w holds the gate and up
 * rows interleaved (row 2i = gate row i, row 2i + 1 = up row i, N = 2F), and
 * out[m][i] (F columns, row stride so >= F) = bf16(bf16(silu(g)) * u) of the
 * bf16 g = (x.w^T)[m][2i], u = (x.w^T)[m][2i + 1] -- bit for bit rspx_linear
 * followed by rspx_silu_mul on the de-interleaved halves.  so == RSPX_TILED
 * writes out in the tiled layout of [M, N / 2] (then N % 64 == 0).  Needs a single
 * K chunk (rspx_linear_splits(N, K) == 1; RSPX_EUNSUPPORTED otherwise) and
 * N % 32 == 0.  No counterpart in the reference: it fuses linear
 * (respect/kernels/gemm.py:30) with silu_mul (respect/system/fused.py:116)
 * for the decoder step.
 */
int rspx_linear_silu(const void* x, int64_t sx, const void* w, int64_t sw, void* out, int64_t so, int M, int N, int K,
                     void* stream);

/* The same product, left as its fp32 chunk partials part[S][M][N] (S =
 * rspx_linear_splits(N, K), also when S == 1) for a consumer that adds them
 * in chunk order and rounds -- rspx_add_rmsnorm_partials,
 * rspx_qkv_rope_cache_partials -- so the sum never takes a launch of its own.
 * N % 16 == 0 and K % 256 == 0 (RSPX_EUNSUPPORTED otherwise), as for
 * rspx_linear_silu.
 */
int rspx_linear_partials(const void* x, int64_t sx, const void* w, int64_t sw, float* part, int M, int N, int K,
                         void* stream);

/* The tiled weight layout (no counterpart in the reference, whose weights stay
 * nn.Linear's row-major [N, K]): w [N, K] (row stride sw >= K, a multiple of
 * 8; 16-byte aligned) copied into out, which holds
 * rspx_linear_tiled_weight_elems(N, K) bf16 elements: 16-row slabs of
 * 16 K + 64 elements (the last 64 zero), slab n / 16 holding the K / 32
 * tiles of 16 x 32 elements of its rows in order of k, element (n, k) at
 * (n % 16 + 16 ((k % 32) / 8)) 8 + k % 8 inside its tile.  Pass out with row
 * stride RSPX_TILED as the w of rspx_linear, rspx_linear_silu and
 * rspx_linear_partials: each wave then reads one 1 KB tile per k-block, in
 * one piece per round.  N % 16 == 0, K % 32 == 0 (-1 / RSPX_EUNSUPPORTED
 * otherwise).
 */
int64_t rspx_linear_tiled_weight_elems(int N, int K);
int rspx_linear_tile_weight(const void* w, int64_t sw, int N, int K, void* out, void* stream);

/* ---------------------------------------------------------------- residual add + RMSNorm
 * xo[r] = bf16(r[r] + h[r]) (PyTorch's bf16 add), y[r] = rmsnorm(xo[r], w, eps)
 * bit for bit as rspx_rmsnorm would give on xo.  Same size rules as
 * rspx_rmsnorm; xo may alias r.
 */
int rspx_add_rmsnorm(const void* r, int64_t sr, const void* h, int64_t sh, const void* w, void* xo, int64_t sxo,
                     void* y, int64_t sy, int rows, int n, float eps, void* stream);

/* The same with h given as the fp32 chunk partials hp[S][rows][n] of a
 * linear layer (rspx_linear_partials; 1 <= S <= 8, the most
 * rspx_linear_splits gives): h = bf16 of their chunk-order sum,
 * bit for bit the h rspx_linear would have produced.  n % 8 == 0 and
 * n <= 16384 (RSPX_EUNSUPPORTED otherwise).
 */
int rspx_add_rmsnorm_partials(const void* r, int64_t sr, const float* hp, int S, const void* w, void* xo, int64_t sxo,
                              void* y, int64_t sy, int rows, int n, float eps, void* stream);

/* ---------------------------------------------------------------- q/k/v epilogue of a decoder layer
 * qkv: [T, (HQ + 2 HK) D] packed projection rows [q | k | v] (row stride
 * sqkv).  q and k get RMSNorm over head_dim (wq / wk) and RoPE (cos/sin rows
 * per token, stride scs) with the arithmetic of rspx_qk_norm_rope; q goes to
 * qo [T, HQ, D] (contiguous); k and v are written into the KV cache of the
 * layer: cache_k[h * skh + slots[t] * skn + d] (likewise v).  D % 16 == 0,
 * D <= 512.
 * cap: slots per head of the cache.  A token whose slot lies outside
 * [0, cap) writes no K/V and gets a NaN q row (the reference's index_copy_
 * would raise a device-side assert; here the error reaches every output the
 * token feeds, without a host synchronisation).
 */
int rspx_qkv_rope_cache(const void* qkv, int64_t sqkv, const void* wq, const void* wk, const void* cos,
                        const void* sin, int64_t scs, const int32_t* slots, int cap, void* cache_k, int64_t skh,
                        int64_t skn, void* cache_v, int64_t svh, int64_t svn, void* qo, int T, int HQ, int HK, int D,
                        float eps, void* stream);

/* The same with the projection given as fp32 chunk partials
 * qkvp[S][T][(HQ + 2 HK) D] (rspx_linear_partials; 1 <= S <= 8).
 */
int rspx_qkv_rope_cache_partials(const float* qkvp, int S, const void* wq, const void* wk, const void* cos,
                                 const void* sin, int64_t scs, const int32_t* slots, int cap, void* cache_k,
                                 int64_t skh, int64_t skn, void* cache_v, int64_t svh, int64_t svn, void* qo, int T,
                                 int HQ, int HK, int D, float eps, void* stream);

/* ---------------------------------------------------------------- trie mask from a parent array
 * parent: [N] int32 (parent index, -1 for a root; parents precede children).
 * msk: [M, NN] uint8 (row stride smm): row i < N opens slots [0, base) (the
 * committed tokens) and base + a for every ancestor a of i and i itself;
 * rows N..M-1 (query padding) open slot 0 only.  depth: [N] int32 out.
 * base + N <= NN.
 */
int rspx_trie_mask(const int32_t* parent, int N, int base, int M, int NN, uint8_t* msk, int64_t smm, int32_t* depth,
                   void* stream);

/* The row inputs of one forward from a step descriptor in device memory, so a
 * captured forward takes a new trie (or a new token) from one host-to-device
 * copy:  desc = [n, base, tok[0..T), parent[0..T)] (int32; parents precede
 * children, -1 for a root).  Row i < n: ids[i] = tok[i] (0 if outside
 * [0, vocab)), slots[i] = P + base + i, pos[i] = P + base + depth(i), and the
 * mask row rspx_trie_mask gives node i; rows n..T-1: ids 0, slots pad0 + i,
 * pos 0, slot 0 only.  A descriptor with n outside [0, T], base < 0 or
 * base + n > NN is taken as n = 0.  ids, slots, pos: [T] int32; msk: [T, NN]
 * uint8 (row stride smm).  No counterpart in the reference: it is
 * respect/decoding/verify.py:22-41's mask and slot/position set-up moved onto
 * the device for the decoder's captured forwards (also the 1-token path: a
 * one-node trie at base = committed count).
 */
int rspx_step_inputs(const int32_t* desc, int T, int P, int NN, int pad0, int vocab, int32_t* ids, int32_t* slots,
                     int32_t* pos, uint8_t* msk, int64_t smm, void* stream);

/* ---------------------------------------------------------------- KV compaction
 * For each of n_tensors cache tensors (device array `bases` of base
 * addresses, each [HK][cap][D] bf16 with head stride sh and slot stride sn)
 * and each head: rows src[0..n) are moved to rows dst0 .. dst0 + n - 1.  All
 * sources are read before any destination is written.  n <= 128, D <= 128.
 */
int rspx_kv_compact(const uint64_t* bases, int n_tensors, int HK, int D, int64_t sh, int64_t sn, int cap, int dst0,
                    const int32_t* src, int n, void* stream);

/* ---------------------------------------------------------------- greedy token per row
 * out[m] = argmax over j of logits[m][j] (fp32, row stride sl, 16-byte
 * aligned rows), columns [off, off + size) counted as -inf; NaN is the
 * largest value; ties go to the lowest index.  workspace: at least
 * rspx_argmax_workspace_bytes(M, V) bytes.
 */
int64_t rspx_argmax_workspace_bytes(int M, int V);
int rspx_argmax_rows(const float* logits, int64_t sl, int M, int V, int off, int size, int64_t* out, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- Prefill / Flow element-wise
 * The kernels the reference's Prefill and Flow patches use, at PyTorch's
 * rounding points (every multiply and add a separate fp32 operation):
 *
 * rspx_square: q = float(x)^2.  x [rows, n] bf16 (row stride sx), q [rows, n]
 *   fp32 (row stride sq).  Replaces _sq_k, respect/system/fused.py:126.
 * rspx_add_sq: x = bf16(float(r) + float(h)), q = float(x)^2.  Replaces
 *   add_sq(r, h), respect/system/fused.py:185 (bf16 inputs and output).
 * rspx_norm_apply: y = bf16(float(w) * bf16(float(x) * rsqrt(var[row] + eps)))
 *   with var [rows] fp32 (the mean of q, taken by the caller as the reference
 *   takes it with PyTorch) and w [n].  rsqrt is a correctly rounded square
 *   root and divide.  Replaces _norm_apply_k / norm_from(xs, sq, w, eps),
 *   respect/system/fused.py:148-173.
 * rspx_rope_vision: y = bf16(x * cos + rotate_half(x) * sin) in fp32 with one
 *   final rounding; x [L, NH, D] bf16 (strides sxl, sxh), cos/sin [L, D] fp32
 *   (row stride scl), y [L, NH, D] contiguous.  D % 16 == 0.  Replaces
 *   rope_vision(x, cos, sin), respect/system/fused.py:97.
 * n % 8 == 0; pointers and row strides 16-byte aligned.
 */
int rspx_square(const void* x, int64_t sx, float* q, int64_t sq, int rows, int n, void* stream);
int rspx_add_sq(const void* r, int64_t sr, const void* h, int64_t sh, void* x, int64_t sx, float* q, int64_t sq,
                int rows, int n, void* stream);
int rspx_norm_apply(const void* x, int64_t sx, const float* var, const void* w, void* y, int64_t sy, int rows, int n,
                    float eps, void* stream);
int rspx_rope_vision(const void* x, int64_t sxl, int64_t sxh, const float* cos, const float* sin, int64_t scl,
                     void* y, int L, int NH, int D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RESPECT_AMD_H */
