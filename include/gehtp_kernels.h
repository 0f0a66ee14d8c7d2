/* gehtp_kernels.h — kernel-level C entry points of libgehtp (gfx950).
 *
 * These have no single counterpart in the reference ABI: they expose the kernels
 * behind individual runlist ops so a caller (this library's tests and benchmark,
 * or an integrator that keeps its own memory) can run one op on device buffers
 * without building a blob. Each names the reference routine whose result it
 * reproduces.
 *
 * Conventions: every pointer is a DEVICE pointer; `stream` is a hipStream_t
 * (NULL = the legacy default stream); the call only enqueues work. Return 0 on
 * success, GEHTP_EINVAL for a rejected shape/alignment, GEHTP_E2BIG for a request beyond
 * a fixed scratch, GEHTP_ENOTSUP for a form an entry point does not take, or a positive
 * hipError_t.
 */
#ifndef GEHTP_KERNELS_H
#define GEHTP_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEHTP_EINVAL (-22)
#define GEHTP_E2BIG (-7)   /* request larger than a fixed-size scratch */

/* y[M, ldy] = x[M, ldx] . dequant(W)^T, W4G int4 group-64 (OP_MATMUL_W4G_F16):
 * M <= 4 runs the GEMV, larger M the MFMA GEMM. Mirrors exec_matmul_f16's scalar
 * arithmetic (oplist_exec.c:1802-1811) on dequant(W) = fp16(q*s) with fp32
 * accumulation (summation order differs).
 * K % 64 == 0, ldx % 8 == 0, x and wq 16-byte aligned. */
int gehtp_w4g_matmul(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y,
                     uint32_t ldy, uint32_t M, uint32_t N, uint32_t K, void* stream);
/* Force one implementation (for measurement): GEMV needs M <= 4. */
int gehtp_w4g_gemv(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y,
                   uint32_t ldy, uint32_t M, uint32_t N, uint32_t K, void* stream);
int gehtp_w4g_gemm(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y,
                   uint32_t ldy, uint32_t M, uint32_t N, uint32_t K, void* stream);
/* OP_W4G_FUSED_F16 on device buffers: gamma (NULL = none) RMSNorm of x first (GEMV
 * sizes only), mode 1 = SwiGLU over interleaved gate/up rows (N/2 outputs), res (NULL =
 * none) added with row stride ldr. Same roundings as the separate runlist ops. */
int gehtp_w4g_fused(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y,
                    uint32_t ldy, uint32_t M, uint32_t N, uint32_t K, const void* gamma,
                    const void* res, uint32_t ldr, uint32_t mode, void* stream);
/* gehtp_w4g_fused with an fp32 workspace (16-byte aligned) that lets the GEMM split K for
 * narrow-N shapes (fewer 128 x 128 tiles than two per CU): in three parts (K >= 48 * 64)
 * when the 128 x 256 grid of three parts fits one round at two workgroups per CU (on
 * that tile when the grid also reaches half the CUs, else on 128-column tiles of 128,
 * 64 or 32 rows), else in two (K >= 32 * 64) on the 128-column tiles; each part writes
 * its sums there and a second pass adds them in part order and applies the epilogue. Needs
 * gehtp_w4g_split_bytes(M, N, K) bytes (0: this shape does not split; work may be NULL
 * or smaller, and the GEMM then runs in one pass). Calls sharing a workspace must not
 * overlap. No counterpart in the reference (its matmul runs on the NPU's own engine). */
size_t gehtp_w4g_split_bytes(uint32_t M, uint32_t N, uint32_t K);
int gehtp_w4g_fused_ws(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y,
                       uint32_t ldy, uint32_t M, uint32_t N, uint32_t K, const void* gamma,
                       const void* res, uint32_t ldr, uint32_t mode, void* work, size_t work_bytes,
                       void* stream);
/* OP_QK_ROPE_KV_F16 on device buffers: qkv [n_tok, (H+2KVH)*128], H + KVH <= 64; ring of state_bytes;
 * count_dev = device uint32 auto-position counter (read, then advanced by n_tok);
 * k_out / v_out may be NULL. */
int gehtp_qk_rope_kv(const void* qkv, uint32_t n_tok, uint32_t H, uint32_t KVH,
                     const void* q_gamma, const void* k_gamma, float theta, void* q_out,
                     void* k_out, void* v_out, void* ring, uint32_t state_bytes,
                     void* count_dev, void* stream);
/* w[N, K] fp16 = fp16(q * s): the dequant, bit-exact. */
int gehtp_w4g_dequant(const void* wq, const void* ws, void* w, uint32_t N, uint32_t K, void* stream);

/* OP_MATMUL_F16 / _SPLIT semantics (oplist_exec.c:1709-1813), flags as in the op. */
int gehtp_matmul_f16(const void* a, const void* w, void* y, uint32_t M, uint32_t K,
                     uint32_t N_full, uint32_t n0, uint32_t N, uint32_t flags, void* stream);

/* OP_RMSNORM2_F16 (oplist_exec.c:1817-1872): rows x rw, b may be NULL. */
int gehtp_rmsnorm2(const void* x, const void* gamma, const void* beta, void* y, uint32_t rows,
                   uint32_t rw, void* stream);
/* OP_SOFTMAX_F16 (oplist_exec.c:1163-1194). */
int gehtp_softmax(const void* x, void* y, uint32_t rows, uint32_t n, void* stream);

/* Fused causal GQA attention (OP_ATTN_F16): q [S,H,128], k/v [S,KVH,128] -> out [S,H,128].
 * scale > 0 and finite, else GEHTP_EINVAL. */
int gehtp_attn_prefill(const void* q, const void* k, const void* v, void* out, uint32_t S,
                       uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal, void* stream);
/* Decode attention (OP_ATTN_DECODE_F16) over positions [0, n_kv) of a KV ring of
 * state_bytes (slot = [K | V], each KVH*hd fp16): q [H,128] -> out [H,128].
 * work: 16-byte aligned device float buffer of gehtp_attn_decode_work_floats(n_kv, H, hd)
 * for per-chunk partials (no initial contents needed). */
int gehtp_attn_decode(const void* q, const void* ring, uint32_t state_bytes, void* out,
                      uint32_t n_kv, uint32_t H, uint32_t KVH, uint32_t hd, float scale,
                      void* work, uint32_t work_floats, void* stream);
uint32_t gehtp_attn_decode_work_floats(uint32_t n_kv, uint32_t H, uint32_t hd);
/* gehtp_attn_decode without a workspace argument, allocating nothing. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The per-chunk
 * partials live in a fixed scratch array of GEHTP_ATTN_DECODE_NOALLOC_MAX_FLOATS floats
 * (4 MiB) that each GPU holds until the process ends: a call needing more than that
 * (gehtp_attn_decode_work_floats(n_kv, H, hd) > the maximum, e.g. n_kv > 15872 at H = 32)
 * returns GEHTP_E2BIG and launches nothing. Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other threads) race. Same
 * arguments, checks and results as gehtp_attn_decode; call it with the stream's device
 * current. */
#define GEHTP_ATTN_DECODE_NOALLOC_MAX_FLOATS (1u << 20)
int gehtp_attn_decode_noalloc(const void* q, const void* ring, uint32_t state_bytes, void* out,
                              uint32_t n_kv, uint32_t H, uint32_t KVH, uint32_t hd, float scale,
                              void* stream);
/* OP_ATTN_DECODE_QKV_F16 on device buffers: qkv = raw [q | k | v] row of the new token
 * ((H + 2*KVH)*128 fp16); q/k RMSNorm (gammas [128]) and RoPE (theta) at position
 * *count_dev, k/v written to the ring, attention over positions 0..*count_dev, then
 * *count_dev += 1. work: 16-byte aligned, gehtp_attn_decode_work_floats(ring slots, H,
 * 128) floats, zeroed before its first use; its head then carries the RoPE cos/sin of
 * the current and next position from call to call (one work buffer may serve every
 * layer, or one per layer). */
int gehtp_attn_decode_qkv(const void* qkv, uint32_t H, uint32_t KVH, const void* q_gamma,
                          const void* k_gamma, float theta, float scale, void* ring,
                          uint32_t state_bytes, void* count_dev, void* out, void* work,
                          uint32_t work_floats, void* stream);
/* OP_W4G_FUSED_F16's GEMV (M = 1; gamma = RMSNorm weights or NULL; no residual, no
 * SwiGLU) writing qkv ((H + 2*KVH)*128 rows of K) followed by gehtp_attn_decode_qkv on
 * that row, in one launch plus the merge pass, with the bits of the two calls. Returns
 * GEHTP_ENOTSUP, launching nothing, for what the one-launch form does not take (K = 512 C
 * with C in {2, 4, 5} or 1024 C with C in {3, 4}; H / KVH in {1, 2, 4, 8}; a grid the
 * device cannot hold at once). work: 16-byte aligned,
 * gehtp_attn_qkv_fused_work_floats(ring slots, H, KVH) floats, zeroed before its first
 * use; gehtp_attn_decode_qkv may share it. No counterpart in the reference: the engine
 * performs its OP_W4G_FUSED_F16 -> OP_ATTN_DECODE_QKV_F16 pairs this way. */
#define GEHTP_ENOTSUP (-95)
uint32_t gehtp_attn_qkv_fused_work_floats(uint32_t nslots, uint32_t H, uint32_t KVH);
int gehtp_qkv_attn_decode(const void* x, const void* wq, const void* ws, const void* gamma, uint32_t K,
                          void* qkv, uint32_t H, uint32_t KVH, const void* q_gamma, const void* k_gamma,
                          float theta, float scale, void* ring, uint32_t state_bytes, void* count_dev,
                          void* out, void* work, uint32_t work_floats, void* stream);
/* gehtp_qkv_attn_decode followed by the o-proj GEMV that reads its output (wo_q / wo_s:
 * W4G weights of N rows of K = H*128; res: residual [N] or NULL; y: [N]), in two launches:
 * the GEMV + chunk pass, then the merge pass + the o-proj GEMV. The bits of the three
 * separate calls (out holds the attention output as well). GEHTP_ENOTSUP, launching
 * nothing, for what either launch does not take. work: as gehtp_qkv_attn_decode. No
 * counterpart in the reference: the engine performs its OP_W4G_FUSED_F16 ->
 * OP_ATTN_DECODE_QKV_F16 -> OP_W4G_FUSED_F16 runs this way. */
int gehtp_qkv_attn_oproj_decode(const void* x, const void* wq, const void* ws, const void* gamma, uint32_t K,
                                void* qkv, uint32_t H, uint32_t KVH, const void* q_gamma, const void* k_gamma,
                                float theta, float scale, void* ring, uint32_t state_bytes, void* count_dev,
                                void* out, const void* wo_q, const void* wo_s, void* y, uint32_t N,
                                const void* res, void* work, uint32_t work_floats, void* stream);
/* Append n_tok tokens (k/v [n_tok, KVH*hd]) at positions pos..pos+n_tok-1 of the ring. */
int gehtp_kv_append(void* ring, uint32_t state_bytes, const void* k, const void* v,
                    uint32_t kv_elems, uint32_t n_tok, uint32_t pos, void* stream);
/* OP_ROPE_F16 with an explicit start position. */
int gehtp_rope(const void* x, void* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd,
               uint32_t pos0, float theta, uint32_t row_stride, void* stream);
/* OP_ARGMAX_F16: out (device int32) = first index of the maximum. */
int gehtp_argmax(const void* x, uint32_t n, void* out, void* stream);

/* crouton16_row4 surfaces (kernels/src/runtime/gemm_dispatch.c:38-72): rows, cols
 * multiples of 32; surf 4-byte aligned. Bit copies of u16 elements. */
int gehtp_crouton_encode(const void* lin, void* surf, uint32_t rows, uint32_t cols, void* stream);
int gehtp_crouton_decode(const void* surf, void* lin, uint32_t rows, uint32_t cols, void* stream);
/* OP_MATMUL_W4A16 (opcode 1, exec_matmul oplist_exec.c:438-529; formula
 * kernels/docs/api_v22_w4a16.md:11): out_surf[M,N] (crouton u16) =
 * clip(nearest(sum_k (A[m,k] - 32768) * W[k,n] / 7) + 32768), act_surf [M,K] crouton u16,
 * w = [N][K/2] bytes, low nibble = even k, value = nibble - 8. M, K, N multiples of 32. */
int gehtp_matmul_w4a16(const void* act_surf, const void* w, void* out_surf, uint32_t M, uint32_t K,
                       uint32_t N, void* stream);
/* OP_RMSNORM_F16 (opcode 2, exec_rmsnorm oplist_exec.c:559-591): y [m,n] fp16 row-major
 * from a crouton u16 surface (value - 32768) and weights w [n] fp16. */
int gehtp_rmsnorm_crouton(const void* x_surf, const void* w, void* y, uint32_t m, uint32_t n,
                          void* stream);

/* Library identification: "gehtp-gfx950 <version>". */
const char* gehtp_version(void);

#ifdef __cplusplus
}
#endif
#endif
