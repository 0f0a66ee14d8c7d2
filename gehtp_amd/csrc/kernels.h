// kernels.h — host-side launchers of the gfx950 kernels (internal to libgehtp).
//
// Every launcher enqueues on the given stream and returns hipSuccess or the launch
// error; shapes are validated by the caller (engine ops or the C-ABI entry points)
// before a launcher is reached, so every launch stays inside its buffers.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace gehtp {

// Number of compute units of the current device (cached).
int device_cu_count();

// ---- W4G (int4, group 64, fp16 scales) ----
// Outputs of OP_QK_ROPE_KV_F16 for a q|k|v GEMM that performs that op in its epilogue.
struct W4gRope {
    uint32_t H = 0, KVH = 0;
    const __half* q_gamma = nullptr;
    const __half* k_gamma = nullptr;
    const void* table = nullptr;   // launch_rope_table's output for this call (n_tok = M)
    __half* q_out = nullptr;
    __half* k_out = nullptr;
    __half* v_out = nullptr;
    uint8_t* ring = nullptr;
    uint32_t slot_bytes = 0, nslots = 0;
};
// Optional fused parts of a W4A16 linear (OP_W4G_FUSED_F16), each reproducing the
// runlist op it replaces with that op's roundings:
//   gamma  RMSNorm of the input rows first (RMSNORM2_F16 with a zero bias; GEMV only —
//          callers of the GEMM normalize into a buffer first)
//   res    y = f16(f16(acc) + res[m*ldr + n])                  (ADD_F16 after the matmul)
//   swiglu weight rows interleaved (2j = gate j, 2j+1 = up j); output column j =
//          f16(f16(silu(f16(acc_g))) * f16(acc_u))            (UNARY silu, BINARY mul)
struct W4gEpilogue {
    const __half* gamma = nullptr;
    const __half* res = nullptr;
    uint32_t ldr = 0;
    bool swiglu = false;
    // GEMM only: fp32 workspace for a K split (w4g_gemm_split_bytes); without one, or
    // when too small, the GEMM runs unsplit. Calls that share it must not overlap.
    float* split_ws = nullptr;
    size_t split_ws_bytes = 0;
    // GEMM with a K split, plain epilogue: when set, the split's finishing pass also
    // writes RMSNORM2_F16(y rows, norm_gamma, no bias) to norm_out (M x N, dense) and
    // sets *norm_done; shapes it cannot take leave *norm_done false.
    const __half* norm_gamma = nullptr;
    __half* norm_out = nullptr;
    bool* norm_done = nullptr;
    // GEMM only: the q|k|v GEMM of OP_QK_ROPE_KV_F16 (N = (H + 2 KVH) * 128, plain
    // epilogue): when set, its epilogue also performs that op — per-head RMSNorm + RoPE
    // of the q and k heads at the positions of a table built by launch_rope_table (which
    // advances the counter), k and v appended to the ring, q_out [M][H*128] and the
    // optional k_out / v_out [M][KVH*128] written — with the rows kernel's arithmetic.
    const W4gRope* rope = nullptr;
};
// y[m*ldy + n] = f16( sum_k x[m*ldx + k] * fp16(q[n,k] * s[n, k/64]) ), m < M, n < N,
// each dequantized weight rounded to fp16 as the reference does, fp32 accumulation
// (N = weight rows; with swiglu the output has N/2 columns).
hipError_t launch_w4g_gemv(const __half* x, uint32_t ldx, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi = W4gEpilogue());
hipError_t launch_w4g_gemm(const __half* a, uint32_t lda, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi = W4gEpilogue());
// K parts the GEMM uses for (M, N, K) when given a workspace, and the workspace bytes
// (0 when it runs unsplit).
uint32_t w4g_gemm_split_parts(uint32_t M, uint32_t N, uint32_t K);
size_t w4g_gemm_split_bytes(uint32_t M, uint32_t N, uint32_t K);
// w[n*K + k] = fp16(q * s) (bit-exact dequant; used by tests and the fp16 fallback).
hipError_t launch_w4g_dequant(const uint8_t* wq, const __half* ws, __half* w,
                              uint32_t N, uint32_t K, hipStream_t st);
// Largest M the GEMV handles; larger M goes to the MFMA GEMM.
constexpr uint32_t kW4gGemvMaxM = 4;
// True when launch_w4g_gemv runs the GEMV itself for (M, K) (otherwise it hands the
// call to the GEMM, which cannot take an RMSNorm prologue).
bool w4g_gemv_supported(uint32_t M, uint32_t K);

// ---- fp16 x fp16 matmul, reference OP_MATMUL_F16 semantics ----
// y[b][m][n0+n] over batch b < Bn; a [Bn][M][K] (or [K][M] when t0), w [Bn][K][N_full]
// (or [Bn][N_full][K] when t1); f32 accumulate, f16 out.
hipError_t launch_matmul_f16(const __half* a, const __half* w, __half* y,
                             uint32_t M, uint32_t K, uint32_t N_full, uint32_t n0, uint32_t N,
                             bool t0, bool t1, uint32_t Bn, hipStream_t st);

// ---- row ops ----
// One wavefront per row: y = f16(x / (float)sqrt(mean(x^2) + 1e-6) * g + b); b may be null.
hipError_t launch_rmsnorm2(const __half* x, const __half* g, const __half* b, __half* y,
                           uint32_t rows, uint32_t rw, hipStream_t st);
// Row softmax with exec_softmax's dispatch (vector path when n % 32 == 0).
hipError_t launch_softmax(const __half* x, __half* y, uint32_t rows, uint32_t n, hipStream_t st);
hipError_t launch_binary(const __half* a, const __half* b, __half* y, uint32_t n, uint32_t subtype,
                         hipStream_t st);
// SELECT: y[i] = c[i%cn]!=0 ? t[i%tn] : f[i%fn] (scalar operands broadcast), n = max counts.
hipError_t launch_select(const __half* c, uint32_t cn, const __half* t, uint32_t tn,
                         const __half* f, uint32_t fn, __half* y, uint32_t n, hipStream_t st);
hipError_t launch_unary(const __half* x, __half* y, uint32_t n, uint32_t subtype, hipStream_t st);
hipError_t launch_argmax(const __half* x, uint32_t n, int32_t* out, hipStream_t st);
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t st);
hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t st);
hipError_t launch_broadcast(const __half* x, __half* y, uint32_t n, const uint32_t in_d[4],
                            const uint32_t out_d[4], hipStream_t st);
hipError_t launch_transpose_gen(const __half* x, __half* y, uint32_t rank, const uint32_t dims[4],
                                uint32_t perm, hipStream_t st);
hipError_t launch_slice(const __half* x, __half* y, uint32_t n_out, uint32_t rank,
                        const uint32_t b[3], const uint32_t s[3], const uint32_t d[3],
                        const uint32_t od[3], hipStream_t st);
// Rotary embedding, half-split layout; position of token t = base + t where
// base = pos0 or, when pos_dev is non-null, *pos_dev (device counter) + pos0.
hipError_t launch_rope(const __half* x, __half* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd,
                       uint32_t pos0, const uint32_t* pos_dev, float theta, uint32_t row_stride,
                       hipStream_t st);

// ---- KV ring (slot-major, slot = [K face | V face], each KVH*hd fp16) ----
// Writes k, v (kv_elems each) into slot (*count_dev or pos) % nslots and, for the
// automatic form, increments *count_dev. pos == UINT32_MAX selects the counter.
hipError_t launch_kv_append(uint8_t* ring, uint32_t slot_bytes, uint32_t nslots, const __half* k,
                            const __half* v, uint32_t kv_elems, uint32_t pos, uint32_t* count_dev,
                            hipStream_t st);
// n_tok tokens (row stride kv_elems) at positions base..base+n_tok-1, base = pos or,
// when pos == UINT32_MAX, *count_dev (then advanced by n_tok).
hipError_t launch_kv_append_n(uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                              const __half* k, const __half* v, uint32_t kv_elems, uint32_t n_tok,
                              uint32_t pos, uint32_t* count_dev, hipStream_t st);
// OP_QK_ROPE_KV_F16: per token t of qkv [n_tok][(H+2KVH)*128] (= [q | k | v]):
// q_out[t] = rope(rmsnorm_128(q, q_gamma)), k = rope(rmsnorm_128(k, k_gamma)) and v go to
// ring slot (*count_dev + t) % nslots (and to k_out / v_out when non-null); then
// *count_dev += n_tok. Positions for RoPE are *count_dev + t. head_dim is 128.
// done_dev (optional): a device counter, zero between launches, with which the
// multi-token kernel advances *count_dev itself (no separate add launch).
hipError_t launch_qk_rope_kv(const __half* qkv, uint32_t n_tok, uint32_t H, uint32_t KVH,
                             const __half* q_gamma, const __half* k_gamma, float theta, __half* q_out,
                             __half* k_out, __half* v_out, uint8_t* ring, uint32_t slot_bytes,
                             uint32_t nslots, uint32_t* count_dev, hipStream_t st,
                             uint32_t* done_dev = nullptr);
// RoPE table of an n_tok-token call at the counter's position for the fused q|k|v GEMM
// epilogue: f16 cos [n_tok][64], f16 sin [n_tok][64], then the start position (uint32);
// w4g_rope_table_bytes(n_tok) bytes, 16-byte aligned. Advances *count_dev by n_tok
// (done_dev: a zero counter of the state, left zero).
inline size_t w4g_rope_table_bytes(uint32_t n_tok) { return (size_t)n_tok * 256 + 16; }
hipError_t launch_rope_table(uint32_t* count_dev, uint32_t* done_dev, float theta, uint32_t n_tok, void* table,
                             hipStream_t st);
// kT [H][hd][pstride], v [H][pstride][hd]; positions >= n_kv of the pstride are zero.
hipError_t launch_kv_gather(const uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                            __half* kT, __half* vo, uint32_t n_kv, uint32_t pstride, uint32_t H,
                            uint32_t KVH, uint32_t hd, hipStream_t st);

// ---- attention ----
// Flash prefill: q [S][H][hd] (row stride ldq), k/v [S][KVH][hd] (row stride ldkv),
// out [S][H][hd] (row stride ldo); hd == 128.
hipError_t launch_attn_prefill(const __half* q, uint32_t ldq, const __half* k, const __half* v,
                               uint32_t ldkv, __half* out, uint32_t ldo, uint32_t S, uint32_t H,
                               uint32_t KVH, uint32_t hd, float scale, bool causal,
                               hipStream_t st);
// The same with head strides (elements between heads h and h+1 of q, k/v and out; the
// plain form uses 128, token-major [S, H, 128]); head-major [H, S, 128] operands pass
// ld = 128 and head stride S*128.
hipError_t launch_attn_prefill_hs(const __half* q, uint32_t ldq, uint32_t qhs, const __half* k, const __half* v,
                                  uint32_t ldkv, uint32_t kvhs, __half* out, uint32_t ldo, uint32_t ohs, uint32_t S,
                                  uint32_t H, uint32_t KVH, uint32_t hd, float scale, bool causal, hipStream_t st);
// Split-KV decode: q [H][hd]; K/V read from the ring for positions [0, n_kv) where
// n_kv = n_kv_host, or *count_dev when count_dev is non-null. mask (optional): additive
// fp16 mask rows [H][P] (mask_shared: one row [P] for every head) over a gathered layout
// of P >= n_kv positions (P <= nslots) whose
// positions past n_kv hold zero K and V, as KV_GATHER with an automatic count lays out
// (those positions then score their mask value alone). n_kv_known: a count the device
// counter is known to have reached (K/V of the chunks below it are requested before the
// counter is read; a wrong value costs time, never correctness).
hipError_t launch_attn_decode(const __half* q, const uint8_t* ring, uint32_t slot_bytes,
                              uint32_t nslots, __half* out, uint32_t n_kv_host,
                              const uint32_t* count_dev, uint32_t H, uint32_t KVH, uint32_t hd,
                              float scale, float* work, uint32_t work_floats, hipStream_t st,
                              const __half* mask = nullptr, uint32_t P = 0, uint32_t n_kv_known = 0,
                              bool mask_shared = false);
// Fused decode step (OP_ATTN_DECODE_QKV_F16): QK-RMSNorm + RoPE of the raw [q | k | v]
// row at position *count_dev, k/v appended to the ring, attention over positions
// 0..*count_dev, then *count_dev += 1. work's head must be zero before the first call
// (the engine clears a new workspace).
hipError_t launch_attn_decode_qkv(const __half* qkv, const __half* q_gamma, const __half* k_gamma,
                                  float theta, uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                                  uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH,
                                  float scale, float* work, uint32_t work_floats, hipStream_t st,
                                  uint32_t n_kv_known = 0);
// Floats of workspace launch_attn_decode needs for n_kv positions.
uint32_t attn_decode_work_floats(uint32_t max_kv, uint32_t H, uint32_t hd);
// OP_W4G_FUSED_F16's GEMV (M = 1; RMSNorm gamma optional; no residual, no SwiGLU) that
// writes the [q | k | v] row qkv (N = (H + 2 KVH) * 128 rows of K) and the
// OP_ATTN_DECODE_QKV_F16 reading it next, in one launch plus the merge pass: the bits of
// launch_w4g_gemv followed by launch_attn_decode_qkv. Returns hipErrorNotSupported and
// launches nothing for what it does not take (K = 512 C with C in {2, 4, 5} or K = 1024 C
// with C in {3, 4}; group size 1, 2, 4 or 8; a grid that does not fit on the device at
// once; invalid arguments give hipErrorInvalidValue). work:
// attn_qkv_fused_work_floats(nslots, H, KVH) floats, head zero before the first call,
// shared with launch_attn_decode_qkv.
hipError_t launch_qkv_attn_decode(const __half* x, const uint8_t* wq, const __half* wsc, const __half* gamma,
                                  uint32_t K, __half* qkv, const __half* q_gamma, const __half* k_gamma,
                                  float theta, uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                                  uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, float scale,
                                  float* work, uint32_t work_floats, hipStream_t st, uint32_t n_kv_known = 0,
                                  bool defer_merge = false);
uint32_t attn_qkv_fused_work_floats(uint32_t nslots, uint32_t H, uint32_t KVH);
// After launch_qkv_attn_decode(defer_merge = true): its merge pass and the o-proj GEMV that
// reads the attention output (OP_W4G_FUSED_F16, M = 1, K = H * 128, N rows, optional
// residual res, no RMSNorm, no SwiGLU; y = its output) in one launch, the bits of the
// merge pass followed by launch_w4g_gemv. hipErrorNotSupported (nothing launched) where
// merge_oproj_supported is false; then launch_attn_merge_deferred runs the merge alone.
bool merge_oproj_supported(uint32_t H, uint32_t N);
hipError_t launch_merge_oproj(uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, uint32_t nslots,
                              float theta, float* work, uint32_t work_floats, const uint8_t* wq, const __half* wsc,
                              __half* y, uint32_t N, const __half* res, hipStream_t st);
hipError_t launch_attn_merge_deferred(uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, uint32_t nslots,
                                      float theta, float* work, hipStream_t st);
// Whether launch_qkv_attn_decode takes this shape (16-byte aligned operands aside).
bool qkv_attn_decode_supported(uint32_t K, uint32_t H, uint32_t KVH, uint32_t nslots);

// ---- crouton16_row4 surfaces, opcode 1 / 2, data ops (k_data.hip) ----
hipError_t launch_crouton_encode(const uint16_t* lin, uint16_t* surf, uint32_t rows, uint32_t cols,
                                 hipStream_t st);
hipError_t launch_crouton_decode(const uint16_t* surf, uint16_t* lin, uint32_t rows, uint32_t cols,
                                 hipStream_t st);
// OP_MATMUL_W4A16: act / out are crouton16_row4 u16 surfaces, w = [N][K/2] +8 nibbles.
hipError_t launch_matmul_w4a16(const uint16_t* act, const uint8_t* w, uint16_t* out, uint32_t M, uint32_t K,
                               uint32_t N, hipStream_t st);
hipError_t launch_rmsnorm_crouton(const uint16_t* x, const __half* w, __half* y, uint32_t m, uint32_t n,
                                  hipStream_t st);
hipError_t launch_concat(const uint16_t* const* xs, const uint32_t* sizes, uint32_t n_seg, uint16_t* y,
                         uint32_t n_elems, hipStream_t st);
hipError_t launch_split(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t total, uint32_t off,
                        uint32_t size, hipStream_t st);
hipError_t launch_pad(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t in_inner, uint32_t out_inner,
                      uint32_t before, uint16_t pv, hipStream_t st);
hipError_t launch_reduce(const __half* x, __half* y, uint32_t outer, uint32_t L, uint32_t inner,
                         uint32_t subtype, hipStream_t st);
hipError_t launch_cumsum(const __half* x, __half* y, uint32_t rows, uint32_t n, uint32_t exclusive,
                         uint32_t reverse, hipStream_t st);
hipError_t launch_gather(const uint16_t* tbl, const int32_t* idx, uint16_t* y, uint32_t n, uint32_t axis,
                         uint32_t xrank, uint32_t irank, const uint32_t* td, const uint32_t* xd,
                         hipStream_t st);
hipError_t launch_transpose4(const uint16_t* x, uint16_t* y, uint32_t Hh, uint32_t W, uint32_t Cc,
                             uint32_t perm, hipStream_t st);

}  // namespace gehtp
