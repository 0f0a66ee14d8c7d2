/* gehtp_oracle.h — CPU restatement of GEHTP's scalar golden path (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP engine. Only tests/, the smoke check
 * and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Each function restates one reference routine (file:line in the .c file) with
 * the same arithmetic order, so results are bit-identical to the reference's
 * scalar path when compiled with -O2 -ffp-contract=off and no fast-math.
 */
#ifndef GEHTP_ORACLE_H
#define GEHTP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE binary16 conversion ---- */
float go_f16_to_f32(uint16_t h);
uint16_t go_f32_to_f16(float f);
void go_f16_to_f32_n(const uint16_t* in, float* out, size_t n);
void go_f32_to_f16_n(const float* in, uint16_t* out, size_t n);

/* ---- int4 group-quantized weights (the W4G format of OP_MATMUL_W4G_F16) ---- */
void go_w4g_pack(const int8_t* q, uint32_t N, uint32_t K, uint8_t* wq);
void go_w4g_unpack(const uint8_t* wq, uint32_t N, uint32_t K, int8_t* q);
int  go_w4g_dequant(const uint8_t* wq, const uint16_t* ws, uint32_t N, uint32_t K,
                    uint32_t group, uint16_t* w /* [N,K] fp16 */);

/* ---- linears ---- */
int go_matmul_f16(const uint16_t* a, const uint16_t* w, uint16_t* y,
                  uint32_t M, uint32_t K, uint32_t N_full, uint32_t n0, uint32_t N,
                  uint32_t flags);
/* y[M,N] = a[M,K] . dequant(W)^T with the OP_MATMUL_F16 scalar arithmetic.
 * n_threads > 1 splits the N outputs over OpenMP threads; every output keeps
 * the sequential k order, so the result is identical for any thread count. */
int go_matmul_w4g(const uint16_t* a, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                  uint32_t M, uint32_t K, uint32_t N, uint32_t group, int n_threads);
/* Same for fp16 weights stored [N,K] (the lm_head). */
int go_matmul_f16_nk_mt(const uint16_t* a, const uint16_t* w, uint16_t* y,
                        uint32_t M, uint32_t K, uint32_t N, int n_threads);
/* Scalar forms of the two above (go_matmul_w4g / go_matmul_f16_nk_mt are the
 * vectorised forms in gehtp_oracle_fast.c, bit-identical for NaN-free results). */
int go_matmul_w4g_ref(const uint16_t* a, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                      uint32_t M, uint32_t K, uint32_t N, uint32_t group, int n_threads);
int go_matmul_f16_nk_ref(const uint16_t* a, const uint16_t* w, uint16_t* y,
                         uint32_t M, uint32_t K, uint32_t N, int n_threads);
/* 1 when the vector forms run (AVX2 + F16C present); go_fast_disable(1) forces the
 * scalar forms, go_fast_disable(0) re-enables detection. */
int go_fast_available(void);
void go_fast_disable(int off);
/* Summation order of the vector forms (linears, attention): 0 = the scalar restatement's
 * sequential order (default); 1 = 32-wide slices combined pairwise; 2 = 16-wide slices
 * combined in sequence (attention's P.V: 64-key chunks). Same products and f16 rounding
 * points; for measuring order-only spread. Returns -1 for an unknown mode or when the
 * vector forms are unavailable. */
int go_set_order(int mode);

/* ---- row ops ---- */
int  go_rmsnorm2(const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                 uint16_t* y, uint32_t n, uint32_t rw);
void go_softmax_scalar(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n);
void go_softmax_host(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n);
void go_softmax(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n);
int  go_binary(const uint16_t* a, const uint16_t* b, uint16_t* y, uint32_t n, uint32_t subtype);
int  go_unary(const uint16_t* x, uint16_t* y, uint32_t n, uint32_t subtype);
int32_t go_argmax(const uint16_t* x, uint32_t n);

/* ---- KV ring state (OP_KV_APPEND_F16 / OP_KV_GATHER_F16) ---- */
struct go_kv {
    uint8_t* buf;         /* nslots * slot_bytes, slot = [K face | V face] */
    uint32_t slot_bytes;  /* 2 * kv_elems * 2 */
    uint32_t nslots;
    uint32_t count;       /* auto-position counter */
    uint32_t* posmap;     /* nslots entries, 0xFFFFFFFF = empty */
};
int go_kv_init(struct go_kv* c, uint8_t* buf, uint32_t state_bytes, uint32_t kv_elems,
               uint32_t* posmap);
int go_kv_append(struct go_kv* c, const uint16_t* k, const uint16_t* v, uint32_t pos);
int go_kv_gather(struct go_kv* c, uint16_t* kT, uint16_t* vo, uint32_t n_kv,
                 uint32_t n_heads, uint32_t kv_heads, uint32_t hd);

/* ---- attention as the reference runlist composes it (f16 at every op) ----
 * q [S,H,hd], k/v [S,KVH,hd] -> out [S,H,hd]. scale is applied as the fp16
 * value f16(scale) (it arrives as an f16 constant slot in reference blobs). */
int go_attn_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                    uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal);
/* The same over n_threads OpenMP threads (heads in parallel; each head's arithmetic
 * unchanged), and its scalar form (go_attn_prefill is the vectorised one). */
int go_attn_prefill_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                       uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal,
                       int n_threads);
int go_attn_prefill_ref(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                        uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal);
/* One query token against the ring: q [H,hd] -> out [H,hd]. */
int go_attn_decode(struct go_kv* c, const uint16_t* q, uint16_t* out, uint32_t n_kv,
                   uint32_t H, uint32_t KVH, uint32_t hd, float scale);
/* go_attn_decode over a ring given as raw bytes + posmap (oracle.KVRing's state):
 * positions [0, n_kv) must be present (else -2). Vectorised; the arithmetic of
 * go_attn_decode. */
int go_attn_decode_ring(const uint8_t* buf, const uint32_t* posmap, uint32_t nslots, uint32_t slot_bytes,
                        const uint16_t* q, uint16_t* out, uint32_t n_kv, uint32_t H, uint32_t KVH,
                        uint32_t hd, float scale);
/* Rotary embedding as the runlist's mul/slice/neg/concat/add chain computes it. */
int go_rope(const uint16_t* x, uint16_t* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd,
            uint32_t pos0, float theta, uint32_t row_stride);

/* ---- remaining runlist ops (gehtp_oracle_ops.c) ---- */
int go_crouton_encode(const uint16_t* lin, uint16_t* surf, uint32_t rows, uint32_t cols);
int go_crouton_decode(const uint16_t* surf, uint16_t* lin, uint32_t rows, uint32_t cols);
int go_matmul_w4a16(const uint16_t* act_surf, const uint8_t* w, uint16_t* out_surf,
                    uint32_t M, uint32_t K, uint32_t N);
int go_rmsnorm_crouton(const uint16_t* x_surf, const uint16_t* w16, uint16_t* y, uint32_t m, uint32_t n);
int go_concat(const uint16_t* const* xs, uint16_t* y, uint32_t n_seg, uint32_t n_elems,
              const uint32_t* sizes);
int go_split(const uint16_t* x, uint32_t x_elems, uint16_t* y, uint32_t n_seg, const uint32_t* sizes,
             uint32_t split_index);
int go_reduce(const uint16_t* x, uint16_t* y, uint32_t n, uint32_t axis, uint32_t subtype,
              const uint32_t* d);
int go_pad(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t in_inner, uint32_t out_inner,
           uint32_t pad_before, uint16_t pv);
int go_cumsum(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n, uint32_t exclusive,
              uint32_t reverse);
int go_gather(const uint16_t* tbl, const int32_t* idx, uint16_t* y, uint32_t n, uint32_t packed,
              const uint32_t* td, const uint32_t* xd);
int go_transpose4(const uint16_t* x, uint16_t* y, uint32_t Hh, uint32_t W, uint32_t Cc, uint32_t perm);
int go_broadcast(const uint16_t* x, uint16_t* y, uint32_t n, const uint32_t* in_d, const uint32_t* out_d);
int go_transpose_gen(const uint16_t* x, uint16_t* y, uint32_t rk, const uint32_t* dims, uint32_t perm);
int go_slice(const uint16_t* x, uint16_t* y, uint32_t n_out, uint32_t rk, const uint32_t* b, const uint32_t* e,
             const uint32_t* s, const uint32_t* d);

#ifdef __cplusplus
}
#endif
#endif
