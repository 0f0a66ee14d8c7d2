// capi.cpp — kernel-level C entry points (include/gehtp_kernels.h).
// Shapes and alignment are checked here so every launch stays inside its buffers.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "gehtp_kernels.h"
#include "kernels.h"

using namespace gehtp;

namespace {

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }
inline int rc(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline const __half* H(const void* p) { return static_cast<const __half*>(p); }
inline __half* Hm(void* p) { return static_cast<__half*>(p); }

bool w4g_args_ok(const void* x, uint32_t ldx, const void* wq, const void* ws, const void* y,
                 uint32_t ldy, uint32_t N, uint32_t K) {
    return x && wq && ws && y && K && K % 64 == 0 && ldx >= K && ldx % 8 == 0 && ldy >= N &&
           al16(x) && al16(wq) && ((reinterpret_cast<uintptr_t>(ws) & 1u) == 0);
}

// Scratch of gehtp_attn_decode_noalloc: the decode attention's per-chunk partial records
// in a file-scope device array instead of a caller's or an allocated workspace. Every GPU
// the library runs on holds its own copy from code-object load until the process ends,
// and every call on that GPU shares it (calls that overlap on one GPU race). In host code
// `scratch` is only a stand-in for the symbol, not a device address: the address is
// looked up once per device with hipGetSymbolAddress and only that pointer is handed to
// kernels. Nothing in it needs to start at zero: each chunk workgroup writes its whole
// record before the merge pass reads it, and the merge reads only the chunks of n_kv.
__device__ __align__(256) float scratch[GEHTP_ATTN_DECODE_NOALLOC_MAX_FLOATS];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's address of `scratch` (looked up on the first call per device,
// with that device current). 0 on success, else a hipError_t / GEHTP_EINVAL.
int noalloc_scratch(float** out) {
    int dev = -1;
    if (const hipError_t e = hipGetDevice(&dev)) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return GEHTP_EINVAL;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" {

int gehtp_w4g_gemv(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y, uint32_t ldy,
                   uint32_t M, uint32_t N, uint32_t K, void* stream) {
    if (!w4g_args_ok(x, ldx, wq, ws, y, ldy, N, K) || M > kW4gGemvMaxM) return GEHTP_EINVAL;
    return rc(launch_w4g_gemv(H(x), ldx, static_cast<const uint8_t*>(wq), H(ws), Hm(y), ldy, M, N, K, S(stream)));
}

int gehtp_w4g_gemm(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y, uint32_t ldy,
                   uint32_t M, uint32_t N, uint32_t K, void* stream) {
    if (!w4g_args_ok(x, ldx, wq, ws, y, ldy, N, K)) return GEHTP_EINVAL;
    return rc(launch_w4g_gemm(H(x), ldx, static_cast<const uint8_t*>(wq), H(ws), Hm(y), ldy, M, N, K, S(stream)));
}

int gehtp_w4g_matmul(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y, uint32_t ldy,
                     uint32_t M, uint32_t N, uint32_t K, void* stream) {
    return M <= kW4gGemvMaxM ? gehtp_w4g_gemv(x, ldx, wq, ws, y, ldy, M, N, K, stream)
                             : gehtp_w4g_gemm(x, ldx, wq, ws, y, ldy, M, N, K, stream);
}

int gehtp_w4g_fused(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y, uint32_t ldy,
                    uint32_t M, uint32_t N, uint32_t K, const void* gamma, const void* res, uint32_t ldr,
                    uint32_t mode, void* stream) {
    return gehtp_w4g_fused_ws(x, ldx, wq, ws, y, ldy, M, N, K, gamma, res, ldr, mode, nullptr, 0, stream);
}

size_t gehtp_w4g_split_bytes(uint32_t M, uint32_t N, uint32_t K) {
    return (M > kW4gGemvMaxM && K && K % 64 == 0) ? w4g_gemm_split_bytes(M, N, K) : 0;
}

int gehtp_w4g_fused_ws(const void* x, uint32_t ldx, const void* wq, const void* ws, void* y, uint32_t ldy,
                       uint32_t M, uint32_t N, uint32_t K, const void* gamma, const void* res, uint32_t ldr,
                       uint32_t mode, void* work, size_t work_bytes, void* stream) {
    const uint32_t n_out = mode == 1 ? N / 2 : N;
    if (mode > 1 || (mode == 1 && (N & 1)) || !w4g_args_ok(x, ldx, wq, ws, y, ldy, n_out, K) ||
        (gamma && !al16(gamma)) || (res && ldr < n_out) || (work && !al16(work)))
        return GEHTP_EINVAL;
    W4gEpilogue epi;
    epi.gamma = H(gamma);
    epi.res = H(res);
    epi.ldr = ldr;
    epi.swiglu = mode == 1;
    epi.split_ws = static_cast<float*>(work);
    epi.split_ws_bytes = work ? work_bytes : 0;
    if (w4g_gemv_supported(M, K))
        return rc(launch_w4g_gemv(H(x), ldx, static_cast<const uint8_t*>(wq), H(ws), Hm(y), ldy, M, N, K,
                                  S(stream), epi));
    if (gamma) return GEHTP_EINVAL;   // GEMM path: normalize with gehtp_rmsnorm2 first
    return rc(launch_w4g_gemm(H(x), ldx, static_cast<const uint8_t*>(wq), H(ws), Hm(y), ldy, M, N, K, S(stream), epi));
}

int gehtp_qk_rope_kv(const void* qkv, uint32_t n_tok, uint32_t Hh, uint32_t KVH, const void* q_gamma,
                     const void* k_gamma, float theta, void* q_out, void* k_out, void* v_out, void* ring,
                     uint32_t state_bytes, void* count_dev, void* stream) {
    const uint32_t slot_bytes = KVH * 128u * 4u;
    if (!qkv || !q_gamma || !k_gamma || !q_out || !ring || !count_dev || !Hh || !KVH ||
        state_bytes % slot_bytes)
        return GEHTP_EINVAL;
    return rc(launch_qk_rope_kv(H(qkv), n_tok, Hh, KVH, H(q_gamma), H(k_gamma), theta, Hm(q_out), Hm(k_out),
                                Hm(v_out), static_cast<uint8_t*>(ring), slot_bytes, state_bytes / slot_bytes,
                                static_cast<uint32_t*>(count_dev), S(stream)));
}

int gehtp_w4g_dequant(const void* wq, const void* ws, void* w, uint32_t N, uint32_t K, void* stream) {
    if (!wq || !ws || !w || K % 64 || !al16(wq) || !al16(w)) return GEHTP_EINVAL;
    return rc(launch_w4g_dequant(static_cast<const uint8_t*>(wq), H(ws), Hm(w), N, K, S(stream)));
}

int gehtp_matmul_f16(const void* a, const void* w, void* y, uint32_t M, uint32_t K, uint32_t N_full,
                     uint32_t n0, uint32_t N, uint32_t flags, void* stream) {
    if (!a || !w || !y || (uint64_t)n0 + N > N_full) return GEHTP_EINVAL;
    uint32_t Bn = flags >> 16;
    if (!Bn || !(flags & 4u)) Bn = 1;
    return rc(launch_matmul_f16(H(a), H(w), Hm(y), M, K, N_full, n0, N, flags & 1u, flags & 2u, Bn, S(stream)));
}

int gehtp_rmsnorm2(const void* x, const void* gamma, const void* beta, void* y, uint32_t rows, uint32_t rw,
                   void* stream) {
    if (!x || !gamma || !y || !rw || (rw % 8 == 0 && !al16(x))) return GEHTP_EINVAL;
    return rc(launch_rmsnorm2(H(x), H(gamma), H(beta), Hm(y), rows, rw, S(stream)));
}

int gehtp_softmax(const void* x, void* y, uint32_t rows, uint32_t n, void* stream) {
    if (!x || !y) return GEHTP_EINVAL;
    return rc(launch_softmax(H(x), Hm(y), rows, n, S(stream)));
}

int gehtp_attn_prefill(const void* q, const void* k, const void* v, void* out, uint32_t S_, uint32_t Hh,
                       uint32_t KVH, uint32_t hd, float scale, int causal, void* stream) {
    if (!q || !k || !v || !out || hd != 128 || !KVH || Hh % KVH || !al16(q) || !al16(k) || !al16(v) ||
        (reinterpret_cast<uintptr_t>(out) & 7u))
        return GEHTP_EINVAL;
    return rc(launch_attn_prefill(H(q), Hh * hd, H(k), H(v), KVH * hd, Hm(out), Hh * hd, S_, Hh, KVH, hd, scale,
                                  causal != 0, S(stream)));
}

uint32_t gehtp_attn_decode_work_floats(uint32_t n_kv, uint32_t Hh, uint32_t hd) {
    return attn_decode_work_floats(n_kv, Hh, hd);
}

int gehtp_attn_decode(const void* q, const void* ring, uint32_t state_bytes, void* out, uint32_t n_kv,
                      uint32_t Hh, uint32_t KVH, uint32_t hd, float scale, void* work, uint32_t work_floats,
                      void* stream) {
    const uint32_t slot_bytes = KVH * hd * 4u;
    if (!q || !ring || !out || !work || hd != 128 || !KVH || Hh % KVH || !slot_bytes ||
        state_bytes % slot_bytes || !al16(q) || !al16(ring) || !al16(work))
        return GEHTP_EINVAL;
    const uint32_t nslots = state_bytes / slot_bytes;
    if (!n_kv || n_kv > nslots) return GEHTP_EINVAL;
    return rc(launch_attn_decode(H(q), static_cast<const uint8_t*>(ring), slot_bytes, nslots, Hm(out), n_kv,
                                 nullptr, Hh, KVH, hd, scale, static_cast<float*>(work), work_floats, S(stream)));
}

int gehtp_attn_decode_qkv(const void* qkv, uint32_t Hh, uint32_t KVH, const void* q_gamma, const void* k_gamma,
                          float theta, float scale, void* ring, uint32_t state_bytes, void* count_dev, void* out,
                          void* work, uint32_t work_floats, void* stream) {
    const uint32_t slot_bytes = KVH * 128u * 4u;
    if (!qkv || !q_gamma || !k_gamma || !ring || !count_dev || !out || !work || !KVH || Hh % KVH ||
        state_bytes % slot_bytes || !state_bytes || !al16(ring) || !al16(work) || (reinterpret_cast<uintptr_t>(out) & 7u))
        return GEHTP_EINVAL;
    return rc(launch_attn_decode_qkv(H(qkv), H(q_gamma), H(k_gamma), theta, static_cast<uint8_t*>(ring), slot_bytes,
                                     state_bytes / slot_bytes, static_cast<uint32_t*>(count_dev), Hm(out), Hh, KVH,
                                     scale, static_cast<float*>(work), work_floats, S(stream)));
}

uint32_t gehtp_attn_qkv_fused_work_floats(uint32_t nslots, uint32_t Hh, uint32_t KVH) {
    return attn_qkv_fused_work_floats(nslots, Hh, KVH);
}

int gehtp_qkv_attn_decode(const void* x, const void* wq, const void* ws, const void* gamma, uint32_t K, void* qkv,
                          uint32_t Hh, uint32_t KVH, const void* q_gamma, const void* k_gamma, float theta,
                          float scale, void* ring, uint32_t state_bytes, void* count_dev, void* out, void* work,
                          uint32_t work_floats, void* stream) {
    const uint32_t slot_bytes = KVH * 128u * 4u;
    if (!x || !wq || !ws || !qkv || !q_gamma || !k_gamma || !ring || !count_dev || !out || !work || !KVH ||
        Hh % KVH || !K || K % 64 || state_bytes % slot_bytes || !state_bytes || !al16(x) || !al16(wq) ||
        (gamma && !al16(gamma)) || (reinterpret_cast<uintptr_t>(ws) & 1u) || !al16(ring) || !al16(work) ||
        (reinterpret_cast<uintptr_t>(out) & 7u))
        return GEHTP_EINVAL;
    const hipError_t e = launch_qkv_attn_decode(H(x), static_cast<const uint8_t*>(wq), H(ws), H(gamma), K, Hm(qkv),
                                                H(q_gamma), H(k_gamma), theta, static_cast<uint8_t*>(ring),
                                                slot_bytes, state_bytes / slot_bytes,
                                                static_cast<uint32_t*>(count_dev), Hm(out), Hh, KVH, scale,
                                                static_cast<float*>(work), work_floats, S(stream));
    return e == hipErrorNotSupported ? GEHTP_ENOTSUP : rc(e);
}

int gehtp_qkv_attn_oproj_decode(const void* x, const void* wq, const void* ws, const void* gamma, uint32_t K,
                                void* qkv, uint32_t Hh, uint32_t KVH, const void* q_gamma, const void* k_gamma,
                                float theta, float scale, void* ring, uint32_t state_bytes, void* count_dev,
                                void* out, const void* wo_q, const void* wo_s, void* y, uint32_t N,
                                const void* res, void* work, uint32_t work_floats, void* stream) {
    const uint32_t slot_bytes = KVH * 128u * 4u;
    if (!x || !wq || !ws || !qkv || !q_gamma || !k_gamma || !ring || !count_dev || !out || !wo_q || !wo_s || !y ||
        !work || !KVH || Hh % KVH || !K || K % 64 || state_bytes % slot_bytes || !state_bytes || !al16(x) ||
        !al16(wq) || !al16(wo_q) || (gamma && !al16(gamma)) || (reinterpret_cast<uintptr_t>(ws) & 1u) ||
        (reinterpret_cast<uintptr_t>(wo_s) & 1u) || !al16(ring) || !al16(work) || !al16(out))
        return GEHTP_EINVAL;
    const uint32_t nslots = state_bytes / slot_bytes;
    if (!qkv_attn_decode_supported(K, Hh, KVH, nslots) || !merge_oproj_supported(Hh, N)) return GEHTP_ENOTSUP;
    hipError_t e = launch_qkv_attn_decode(H(x), static_cast<const uint8_t*>(wq), H(ws), H(gamma), K, Hm(qkv),
                                          H(q_gamma), H(k_gamma), theta, static_cast<uint8_t*>(ring), slot_bytes,
                                          nslots, static_cast<uint32_t*>(count_dev), Hm(out), Hh, KVH, scale,
                                          static_cast<float*>(work), work_floats, S(stream), 0u, true);
    if (e == hipSuccess)
        e = launch_merge_oproj(static_cast<uint32_t*>(count_dev), Hm(out), Hh, KVH, nslots, theta,
                               static_cast<float*>(work), work_floats, static_cast<const uint8_t*>(wo_q), H(wo_s),
                               Hm(y), N, H(res), S(stream));
    return e == hipErrorNotSupported ? GEHTP_ENOTSUP : rc(e);
}

int gehtp_attn_decode_noalloc(const void* q, const void* ring, uint32_t state_bytes, void* out, uint32_t n_kv,
                              uint32_t Hh, uint32_t KVH, uint32_t hd, float scale, void* stream) {
    const uint32_t slot_bytes = KVH * hd * 4u;
    if (!q || !ring || !out || hd != 128 || !KVH || Hh % KVH || !slot_bytes || state_bytes % slot_bytes ||
        !al16(q) || !al16(ring))
        return GEHTP_EINVAL;
    const uint32_t nslots = state_bytes / slot_bytes;
    if (!n_kv || n_kv > nslots) return GEHTP_EINVAL;
    if (attn_decode_work_floats(n_kv, Hh, hd) > GEHTP_ATTN_DECODE_NOALLOC_MAX_FLOATS) return GEHTP_E2BIG;
    float* work = nullptr;
    if (const int e = noalloc_scratch(&work)) return e;
    return rc(launch_attn_decode(H(q), static_cast<const uint8_t*>(ring), slot_bytes, nslots, Hm(out), n_kv, nullptr,
                                 Hh, KVH, hd, scale, work, GEHTP_ATTN_DECODE_NOALLOC_MAX_FLOATS, S(stream)));
}

int gehtp_kv_append(void* ring, uint32_t state_bytes, const void* k, const void* v, uint32_t kv_elems,
                    uint32_t n_tok, uint32_t pos, void* stream) {
    const uint32_t slot_bytes = kv_elems * 4u;
    if (!ring || !k || !v || !kv_elems || state_bytes % slot_bytes || pos == 0xFFFFFFFFu) return GEHTP_EINVAL;
    return rc(launch_kv_append_n(static_cast<uint8_t*>(ring), slot_bytes, state_bytes / slot_bytes, H(k), H(v),
                                 kv_elems, n_tok, pos, nullptr, S(stream)));
}

int gehtp_rope(const void* x, void* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd, uint32_t pos0,
               float theta, uint32_t row_stride, void* stream) {
    if (!x || !y || !hd || hd % 2 || row_stride < n_heads * hd) return GEHTP_EINVAL;
    return rc(launch_rope(H(x), Hm(y), n_tok, n_heads, hd, pos0, nullptr, theta, row_stride, S(stream)));
}

int gehtp_argmax(const void* x, uint32_t n, void* out, void* stream) {
    if (!x || !out) return GEHTP_EINVAL;
    return rc(launch_argmax(H(x), n, static_cast<int32_t*>(out), S(stream)));
}

int gehtp_crouton_encode(const void* lin, void* surf, uint32_t rows, uint32_t cols, void* stream) {
    if (!lin || !surf || rows % 32 || cols % 32 || (reinterpret_cast<uintptr_t>(surf) & 3u)) return GEHTP_EINVAL;
    return rc(launch_crouton_encode(static_cast<const uint16_t*>(lin), static_cast<uint16_t*>(surf), rows, cols,
                                    S(stream)));
}

int gehtp_crouton_decode(const void* surf, void* lin, uint32_t rows, uint32_t cols, void* stream) {
    if (!lin || !surf || rows % 32 || cols % 32 || (reinterpret_cast<uintptr_t>(surf) & 3u)) return GEHTP_EINVAL;
    return rc(launch_crouton_decode(static_cast<const uint16_t*>(surf), static_cast<uint16_t*>(lin), rows, cols,
                                    S(stream)));
}

int gehtp_matmul_w4a16(const void* act_surf, const void* w, void* out_surf, uint32_t M, uint32_t K, uint32_t N,
                       void* stream) {
    if (!act_surf || !w || !out_surf || !M || !K || !N || M % 32 || K % 32 || N % 32 || !al16(act_surf) ||
        !al16(w) || (reinterpret_cast<uintptr_t>(out_surf) & 1u))
        return GEHTP_EINVAL;
    return rc(launch_matmul_w4a16(static_cast<const uint16_t*>(act_surf), static_cast<const uint8_t*>(w),
                                  static_cast<uint16_t*>(out_surf), M, K, N, S(stream)));
}

int gehtp_rmsnorm_crouton(const void* x_surf, const void* w, void* y, uint32_t m, uint32_t n, void* stream) {
    if (!x_surf || !w || !y || !m || m % 32 || n % 32) return GEHTP_EINVAL;
    return rc(launch_rmsnorm_crouton(static_cast<const uint16_t*>(x_surf), H(w), Hm(y), m, n, S(stream)));
}

const char* gehtp_version(void) { return "gehtp-gfx950 0.1"; }

}  // extern "C"
