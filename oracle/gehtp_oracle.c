/* gehtp_oracle.c — CPU restatement of GEHTP's scalar golden path (TEST INFRASTRUCTURE).
 *
 * Loaded only by tests/, the smoke check and bench.py's cpu_baseline leg. The HIP
 * engine never links or calls it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp, no fast-math).
 *
 * Parity pins (what checks each function; "unpinned" where nothing does):
 *   f16 conversions   exhaustive vs numpy's IEEE casts (tests/test_oracle.py)
 *   w4g pack/dequant  closed form fp16(q*s) per element vs numpy; round trip.
 *                     The g64 format has no reference implementation.
 *   matmul_f16        identity / one-hot weights give exact copies; float64 brute
 *                     force within accumulated-rounding bound; index invariants of
 *                     kernels/host/test_gemv_f16.c (t0/t1/batched/split)
 *   rmsnorm2          closed forms (constant row, zero row) and numpy float64
 *   softmax           rows sum to 1, shift invariance, one-hot limit
 *   kv ring           byte-exact vs the reference kvcache.c built from source
 *                     (oracle/_ref) and the GQA gather round trip
 *   attention         one-key rows return V exactly; decode step t == prefill row t
 *   rope              position 0 is the identity; norm preservation per pair
 */
#include "gehtp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32, RNE with correct subnormals.
 * Reference: kernels/src/runtime/oplist_exec.c:371-418. */
float go_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* normalise the subnormal mantissa */
            int e = 0;
            while (!(man & 0x400u)) { man <<= 1; e++; }
            bits = sign | ((uint32_t)(113 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t go_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t fexp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    int32_t exp = (int32_t)fexp - 112;   /* rebias 127 -> 15 */
    /* NaN and Inf both map to Inf of the same sign (the reference keeps no payload). */
    if (fexp == 0xffu || exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t sub = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (sub & 1u))) sub++;
        return (uint16_t)(sign | sub);
    }
    uint32_t h = sign | ((uint32_t)exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* carry may reach Inf: correct */
    return (uint16_t)h;
}

void go_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = go_f16_to_f32(in[i]);
}
void go_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = go_f32_to_f16(in[i]);
}

#define F(h) go_f16_to_f32(h)
#define H(f) go_f32_to_f16(f)

/* binary64 -> binary16 with a single RNE rounding (numpy's float64 -> float16 cast). */
static uint16_t f64_to_f16(double d) {
    uint64_t x;
    memcpy(&x, &d, 8);
    uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    int32_t dexp = (int32_t)((x >> 52) & 0x7ffu);
    uint64_t man = x & ((1ull << 52) - 1);
    if (dexp == 0x7ff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int32_t exp = dexp - 1008;   /* rebias 1023 -> 15 */
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    uint64_t kept, rem, halfway;
    if (exp <= 0) {
        if (exp < -10) return sign;
        uint64_t m = man | (1ull << 52);
        uint32_t shift = (uint32_t)(43 - exp);
        kept = m >> shift;
        rem = m & ((1ull << shift) - 1);
        halfway = 1ull << (shift - 1);
    } else {
        kept = ((uint64_t)exp << 10) | (man >> 42);
        rem = man & ((1ull << 42) - 1);
        halfway = 1ull << 41;
    }
    if (rem > halfway || (rem == halfway && (kept & 1u))) kept++;
    return (uint16_t)(sign | kept);
}

/* ------------------------------------------------------------------------- */
/* W4G: row n of wq holds K/2 bytes; byte j = (k=2j) low nibble | (k=2j+1) high
 * nibble; stored nibble = q + 8 (offset binary, as ggml Q4_0,
 * kernels/host/vendor/weight_pack.h:52-58). dequant = fp16(q * s), RNE, like the
 * reference's Q4_0 -> fp16 tile dequant (kernels/include/internal/hmx-mm-kernels-tiled.h:38-135). */
void go_w4g_pack(const int8_t* q, uint32_t N, uint32_t K, uint8_t* wq) {
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t j = 0; j < K / 2; j++) {
            uint32_t lo = (uint32_t)(q[(size_t)n * K + 2 * j] + 8) & 0xFu;
            uint32_t hi = (uint32_t)(q[(size_t)n * K + 2 * j + 1] + 8) & 0xFu;
            wq[(size_t)n * (K / 2) + j] = (uint8_t)(lo | (hi << 4));
        }
}

void go_w4g_unpack(const uint8_t* wq, uint32_t N, uint32_t K, int8_t* q) {
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t j = 0; j < K / 2; j++) {
            uint8_t b = wq[(size_t)n * (K / 2) + j];
            q[(size_t)n * K + 2 * j] = (int8_t)((b & 0xF) - 8);
            q[(size_t)n * K + 2 * j + 1] = (int8_t)((b >> 4) - 8);
        }
}

int go_w4g_dequant(const uint8_t* wq, const uint16_t* ws, uint32_t N, uint32_t K,
                   uint32_t group, uint16_t* w) {
    if (!group || K % group || K % 2) return -1;
    const uint32_t G = K / group;
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t k = 0; k < K; k++) {
            uint8_t b = wq[(size_t)n * (K / 2) + k / 2];
            int q = (int)((k & 1) ? (b >> 4) : (b & 0xF)) - 8;
            float s = F(ws[(size_t)n * G + k / group]);
            w[(size_t)n * K + k] = H((float)q * s);   /* q*s is exact in f32 */
        }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* OP_MATMUL_F16 / OP_MATMUL_F16_SPLIT scalar path:
 * kernels/src/runtime/oplist_exec.c:1709-1813 (scalar branch 1785-1812).
 * y[m, n0+n] = f16(sum_k f32(a) * f32(w)), k ascending, float accumulator. */
int go_matmul_f16(const uint16_t* a, const uint16_t* w, uint16_t* y,
                  uint32_t M, uint32_t K, uint32_t N_full, uint32_t n0, uint32_t N,
                  uint32_t flags) {
    int t0 = (int)(flags & 1u), t1 = (int)(flags & 2u), batched = (int)(flags & 4u);
    uint32_t Bn = flags >> 16;
    if (Bn == 0) Bn = 1;
    if (batched) {
        for (uint32_t bb = 0; bb < Bn; bb++)
            for (uint32_t m = 0; m < M; m++)
                for (uint32_t n = 0; n < N; n++) {
                    float acc = 0.0f;
                    for (uint32_t k = 0; k < K; k++) {
                        float av = F(a[((size_t)bb * M + m) * K + k]);
                        float wv = F(w[t1 ? ((size_t)bb * N_full + n0 + n) * K + k
                                          : ((size_t)bb * K + k) * N_full + (n0 + n)]);
                        acc += av * wv;
                    }
                    y[((size_t)bb * M + m) * N_full + (n0 + n)] = H(acc);
                }
        return 0;
    }
    for (uint32_t m = 0; m < M; m++)
        for (uint32_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; k++) {
                float av = F(a[t0 ? (size_t)k * M + m : (size_t)m * K + k]);
                float wv = F(w[t1 ? (size_t)(n0 + n) * K + k : (size_t)k * N_full + (n0 + n)]);
                acc += av * wv;
            }
            y[(size_t)m * N_full + (n0 + n)] = H(acc);
        }
    return 0;
}

/* The flags=2 ([N,K] weights) case of go_matmul_f16, restructured so that the
 * inner loop runs across output columns (vectorisable) while each output still
 * accumulates k = 0,1,2,... in order: bit-identical to go_matmul_f16. */
static void matmul_nk_core(const uint16_t* a, const float* wT /* [K][N] f32 */,
                           uint16_t* y, uint32_t M, uint32_t K, uint32_t N,
                           uint32_t n_begin, uint32_t n_end, float* acc) {
    for (uint32_t m = 0; m < M; m++) {
        for (uint32_t n = n_begin; n < n_end; n++) acc[n - n_begin] = 0.0f;
        for (uint32_t k = 0; k < K; k++) {
            const float av = F(a[(size_t)m * K + k]);
            const float* wr = wT + (size_t)k * N;
            for (uint32_t n = n_begin; n < n_end; n++) acc[n - n_begin] += av * wr[n];
        }
        for (uint32_t n = n_begin; n < n_end; n++) y[(size_t)m * N + n] = H(acc[n - n_begin]);
    }
}

static int matmul_nk_mt(const uint16_t* a, const uint16_t* w_nk, uint16_t* y,
                        uint32_t M, uint32_t K, uint32_t N, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (M <= 4) {
        /* decode sizes: the reference's own loop order (row n of w streamed once per m) */
        float* af = (float*)malloc((size_t)M * K * sizeof(float));
        if (!af) return -1;
        for (size_t i = 0; i < (size_t)M * K; i++) af[i] = F(a[i]);
#pragma omp parallel for num_threads(n_threads) schedule(static)
        for (uint32_t n = 0; n < N; n++) {
            const uint16_t* wr = w_nk + (size_t)n * K;
            for (uint32_t m = 0; m < M; m++) {
                float acc = 0.0f;
                for (uint32_t k = 0; k < K; k++) acc += af[(size_t)m * K + k] * F(wr[k]);
                y[(size_t)m * N + n] = H(acc);
            }
        }
        free(af);
        return 0;
    }
    float* wT = (float*)malloc((size_t)K * N * sizeof(float));
    if (!wT) return -1;
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t k = 0; k < K; k++) wT[(size_t)k * N + n] = F(w_nk[(size_t)n * K + k]);
    if (n_threads < 1) n_threads = 1;
    const uint32_t chunk = 256;
    const uint32_t n_chunks = (N + chunk - 1) / chunk;
    int rc = 0;
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 1)
    for (uint32_t c = 0; c < n_chunks; c++) {
        float acc[256];
        uint32_t nb = c * chunk, ne = nb + chunk < N ? nb + chunk : N;
        matmul_nk_core(a, wT, y, M, K, N, nb, ne, acc);
    }
    free(wT);
    return rc;
}

/* Scalar forms of the two linears (the vector forms in gehtp_oracle_fast.c fall back
 * to these on CPUs without AVX2/F16C; tests compare both with go_matmul_f16). */
int go_matmul_w4g_ref(const uint16_t* a, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                      uint32_t M, uint32_t K, uint32_t N, uint32_t group, int n_threads) {
    uint16_t* w = (uint16_t*)malloc((size_t)N * K * 2);
    if (!w) return -1;
    if (go_w4g_dequant(wq, ws, N, K, group, w)) { free(w); return -1; }
    int rc = matmul_nk_mt(a, w, y, M, K, N, n_threads);
    free(w);
    return rc;
}

int go_matmul_f16_nk_ref(const uint16_t* a, const uint16_t* w, uint16_t* y,
                         uint32_t M, uint32_t K, uint32_t N, int n_threads) {
    return matmul_nk_mt(a, w, y, M, K, N, n_threads);
}

/* ------------------------------------------------------------------------- */
/* OP_RMSNORM2_F16: kernels/src/runtime/oplist_exec.c:1859-1871 (scalar path).
 * Sum of squares in double, rms = (float)sqrt(mean + 1e-6), divide, scale, bias. */
int go_rmsnorm2(const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                uint16_t* y, uint32_t n, uint32_t rw) {
    if (rw == 0 || n % rw) return -1;
    uint32_t m = n / rw;
#pragma omp parallel for schedule(static) if (n >= (1u << 16))
    for (uint32_t r = 0; r < m; r++) {
        const uint16_t* xr = x + (size_t)r * rw;
        double acc = 0.0;
        for (uint32_t i = 0; i < rw; i++) {
            float v = F(xr[i]);
            acc += (double)v * (double)v;
        }
        float rms = (float)sqrt(acc / (double)rw + 1e-6);
        for (uint32_t i = 0; i < rw; i++) {
            float v = F(xr[i]) / rms;
            v = v * F(gamma[i]) + (beta ? F(beta[i]) : 0.0f);
            y[(size_t)r * rw + i] = H(v);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Softmax, scalar form: kernels/src/runtime/oplist_exec.c:1184-1192.
 * e rounded to f16 first, float sum, then f16(f16(e) / sum). */
void go_softmax_scalar(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n) {
    for (uint32_t r = 0; r < rows; r++) {
        const uint16_t* xr = x + (size_t)r * n;
        uint16_t* yr = y + (size_t)r * n;
        float mx = F(xr[0]);
        for (uint32_t i = 1; i < n; i++) mx = fmaxf(mx, F(xr[i]));
        float sum = 0.0f;
        for (uint32_t i = 0; i < n; i++) {
            float e = expf(F(xr[i]) - mx);
            yr[i] = H(e);
            sum += e;
        }
        for (uint32_t i = 0; i < n; i++) yr[i] = H(F(yr[i]) / sum);
    }
}

/* Softmax as exec_softmax runs it on a host build when n % 32 == 0
 * (oplist_exec.c:1171-1182 -> kernels/src/hvx/hvx_softmax.c:81-93 scalar body):
 * f32 exponentials, double sum, multiply by (float)(1/sum). */
void go_softmax_host(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n) {
    for (uint32_t r = 0; r < rows; r++) {
        const uint16_t* xr = x + (size_t)r * n;
        uint16_t* yr = y + (size_t)r * n;
        float mx = -FLT_MAX;
        for (uint32_t i = 0; i < n; i++) { float v = F(xr[i]); if (v > mx) mx = v; }
        double sum = 0.0;
        float* e = (float*)malloc((size_t)n * sizeof(float));
        for (uint32_t i = 0; i < n; i++) { e[i] = expf(F(xr[i]) - mx); sum += e[i]; }
        float inv = (sum > 0.0) ? (float)(1.0 / sum) : 0.0f;
        for (uint32_t i = 0; i < n; i++) yr[i] = H(e[i] * inv);
        free(e);
    }
}

/* exec_softmax's dispatch (oplist_exec.c:1171): the vector path whenever
 * n % 32 == 0 and rows*n >= 32, the scalar loop otherwise. */
void go_softmax(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n) {
    if (rows >= 1 && n % 32 == 0 && (size_t)rows * n >= 32) go_softmax_host(x, y, rows, n);
    else go_softmax_scalar(x, y, rows, n);
}

/* OP_BINARY_F16 element-wise subtypes 0..5: oplist_exec.c:1143-1158, with exec_binary's
 * dispatch (:1126-1145): for n >= 32, subtypes 0..3 run hvhx_v2_{add,sub,mul,div}_f32
 * between the f16 conversions of hvx_binary.c; on a host build those are the plain f32
 * ops (hvx_binary.c:38-86), so division is NOT guarded against a zero divisor there. */
int go_binary(const uint16_t* a, const uint16_t* b, uint16_t* y, uint32_t n, uint32_t subtype) {
    if (subtype > 5) return -1;
    const int vec = n >= 32u;
#pragma omp parallel for schedule(static) if (n >= (1u << 16))
    for (uint32_t i = 0; i < n; i++) {
        float x0 = F(a[i]), x1 = F(b[i]), r = x0;
        switch (subtype) {
        case 0: r = x0 + x1; break;
        case 1: r = x0 - x1; break;
        case 2: r = x0 * x1; break;
        case 3: r = vec ? x0 / x1 : ((x1 != 0) ? x0 / x1 : 0.0f); break;
        case 4: r = (x0 == x1) ? 1.0f : 0.0f; break;
        case 5: r = ((uint32_t)x0 & (uint32_t)x1) ? 1.0f : 0.0f; break;
        }
        y[i] = H(r);
    }
    return 0;
}

/* OP_UNARY_F16 scalar subtypes: oplist_exec.c:1047-1078, with exec_unary's dispatch
 * (:1021-1045): for n >= 32, subtypes 1/8/9/12 run hvhx_v2_{exp,sigmoid,tanh,silu}_f32,
 * whose host bodies are the same f32 formulas (hvx_unary.c:44-156), and COPY (14) is a
 * bit copy (NaN payloads kept) instead of the f16 -> f32 -> f16 round trip. */
int go_unary(const uint16_t* x, uint16_t* y, uint32_t n, uint32_t subtype) {
    if (subtype > 16) return -1;
    if (subtype == 14 && n >= 32u) {
        memcpy(y, x, (size_t)n * 2u);
        return 0;
    }
#pragma omp parallel for schedule(static) if (n >= (1u << 16))
    for (uint32_t i = 0; i < n; i++) {
        float v = F(x[i]), r = v;
        switch (subtype) {
        case 0: r = -v; break;
        case 1: r = expf(v); break;
        case 2: r = (v >= 0) ? sqrtf(v) : 0.0f; break;
        case 3: r = (v > 0) ? 1.0f / sqrtf(v) : 0.0f; break;
        case 4: r = (v > 0) ? logf(v) : 0.0f; break;
        case 5: r = fabsf(v); break;
        case 6: r = sinf(v); break;
        case 7: r = cosf(v); break;
        case 8: r = 1.0f / (1.0f + expf(-v)); break;
        case 9: r = tanhf(v); break;
        case 10: r = 0.5f * v * (1.0f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v))); break;
        case 11: r = fmaxf(0.0f, v); break;
        case 12: r = v / (1.0f + expf(-v)); break;
        case 13: r = (v > 30.0f) ? v : (v < -30.0f ? expf(v) : log1pf(expf(v))); break;
        case 14: r = v; break;
        case 15: r = (v != v) ? 1.0f : 0.0f; break;
        case 16: r = (v == v && (v > 3.4e38f || v < -3.4e38f)) ? 1.0f : 0.0f; break;
        }
        y[i] = H(r);
    }
    return 0;
}

/* OP_ARGMAX_F16: first strict maximum, start value -1e30 (oplist_exec.c:1990-2004). */
int32_t go_argmax(const uint16_t* x, uint32_t n) {
    int32_t best = 0;
    float bv = -1e30f;
    for (uint32_t i = 0; i < n; i++) {
        float v = F(x[i]);
        if (v > bv) { bv = v; best = (int32_t)i; }
    }
    return best;
}

/* ------------------------------------------------------------------------- */
/* KV ring: slot = pos % nslots, posmap[slot] = pos, face = [K | V].
 * Reference: kernels/src/runtime/kvcache.c:49-68 and the geometry rule of
 * state_kvc, oplist_exec.c:2119-2151. */
int go_kv_init(struct go_kv* c, uint8_t* buf, uint32_t state_bytes, uint32_t kv_elems,
               uint32_t* posmap) {
    uint32_t slot_bytes = kv_elems * 4u;
    if (slot_bytes < 256u || (slot_bytes & 127u) || state_bytes % slot_bytes) return -1;
    c->buf = buf;
    c->slot_bytes = slot_bytes;
    c->nslots = state_bytes / slot_bytes;
    c->count = 0;
    c->posmap = posmap;
    for (uint32_t i = 0; i < c->nslots; i++) posmap[i] = 0xFFFFFFFFu;
    memset(buf, 0, state_bytes);
    return 0;
}

/* OP_KV_APPEND_F16: oplist_exec.c:2154-2176. pos == 0xFFFFFFFA uses the counter. */
int go_kv_append(struct go_kv* c, const uint16_t* k, const uint16_t* v, uint32_t pos) {
    if (pos == 0xFFFFFFFAu) {
        if (c->count >= c->nslots) return -1;
        pos = c->count++;
    }
    uint32_t slot = pos % c->nslots;
    uint32_t half = c->slot_bytes / 2;
    memcpy(c->buf + (size_t)slot * c->slot_bytes, k, half);
    memcpy(c->buf + (size_t)slot * c->slot_bytes + half, v, half);
    c->posmap[slot] = pos;
    return (int)slot;
}

/* OP_KV_GATHER_F16: oplist_exec.c:2183-2231. kT [H, hd, pstride], v [H, pstride, hd];
 * n_kv == AUTO reads the counter and pads the outputs to nslots with zeros. */
int go_kv_gather(struct go_kv* c, uint16_t* kT, uint16_t* vo, uint32_t n_kv,
                 uint32_t n_heads, uint32_t kv_heads, uint32_t hd) {
    if (!n_heads || !kv_heads || !hd || n_heads % kv_heads) return -1;
    if (kv_heads * hd * 4u != c->slot_bytes) return -1;
    uint32_t pstride = n_kv;
    if (n_kv == 0xFFFFFFFAu) {
        if (c->count == 0 || c->count > c->nslots) return -1;
        n_kv = c->count;
        pstride = c->nslots;
    }
    if (pstride > n_kv) {
        if (kT) memset(kT, 0, (size_t)n_heads * hd * pstride * 2);
        if (vo) memset(vo, 0, (size_t)n_heads * pstride * hd * 2);
    }
    uint32_t rep = n_heads / kv_heads;
    for (uint32_t p = 0; p < n_kv; p++) {
        uint32_t slot = p % c->nslots;
        if (c->posmap[slot] != p) return -2;   /* lookup miss is a hard error */
        const uint16_t* kf = (const uint16_t*)(c->buf + (size_t)slot * c->slot_bytes);
        const uint16_t* vf = (const uint16_t*)(c->buf + (size_t)slot * c->slot_bytes + c->slot_bytes / 2);
        for (uint32_t h = 0; h < n_heads; h++) {
            const uint16_t* ks = kf + (h / rep) * hd;
            const uint16_t* vs = vf + (h / rep) * hd;
            if (kT) for (uint32_t d = 0; d < hd; d++) kT[((size_t)h * hd + d) * pstride + p] = ks[d];
            if (vo) memcpy(vo + ((size_t)h * pstride + p) * hd, vs, (size_t)hd * 2);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Prefill attention as reference runlists compose it (see
 * test_models/transformer32/gen_transformer.py:146-194 for the f16 discipline and
 * scripts/export_layer_onnx.py:39-55 for the causal mask): per head h with kv head
 * h / (H/KVH):
 *   s = MATMUL_F16(q_h, K_kv^T)            f16 out, k ascending
 *   s = BINARY mul (s, f16(scale))          f16 out
 *   s = BINARY add (s, mask)  mask 0 / -inf f16 out
 *   p = SOFTMAX(s) over S keys              exec_softmax dispatch
 *   o = MATMUL_F16(p, V_kv)                 f16 out, j ascending */
int go_attn_prefill_ref(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                        uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal) {
    if (!S || !H || !KVH || H % KVH) return -1;
    const uint32_t rep = H / KVH;
    const float sc = F(H(scale));
    const uint16_t neg_inf = 0xFC00u;
    uint16_t* s = (uint16_t*)malloc((size_t)S * S * 2);
    uint16_t* p = (uint16_t*)malloc((size_t)S * S * 2);
    if (!s || !p) { free(s); free(p); return -1; }
    for (uint32_t h = 0; h < H; h++) {
        const uint32_t kv = h / rep;
        for (uint32_t i = 0; i < S; i++)
            for (uint32_t j = 0; j < S; j++) {
                float acc = 0.0f;
                for (uint32_t d = 0; d < hd; d++)
                    acc += F(q[((size_t)i * H + h) * hd + d]) * F(k[((size_t)j * KVH + kv) * hd + d]);
                uint16_t t = H(acc);
                t = H(F(t) * sc);
                uint16_t mask = (causal && j > i) ? neg_inf : 0;
                s[(size_t)i * S + j] = H(F(t) + F(mask));
            }
        go_softmax(s, p, S, S);
        for (uint32_t i = 0; i < S; i++)
            for (uint32_t d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (uint32_t j = 0; j < S; j++)
                    acc += F(p[(size_t)i * S + j]) * F(v[((size_t)j * KVH + kv) * hd + d]);
                out[((size_t)i * H + h) * hd + d] = H(acc);
            }
    }
    free(s);
    free(p);
    return 0;
}

/* Decode attention as the persistent decode graph runs it (scripts/surgery_decode_graph.py:
 * KV_GATHER -> batched MATMUL_F16 -> scale -> additive mask -> SOFTMAX -> MATMUL_F16),
 * over exactly the n_kv valid positions. */
int go_attn_decode(struct go_kv* c, const uint16_t* q, uint16_t* out, uint32_t n_kv,
                   uint32_t H, uint32_t KVH, uint32_t hd, float scale) {
    if (n_kv == 0xFFFFFFFAu) n_kv = c->count;
    if (!n_kv || !H || !KVH || H % KVH) return -1;
    uint16_t* kT = (uint16_t*)malloc((size_t)H * hd * n_kv * 2);
    uint16_t* vo = (uint16_t*)malloc((size_t)H * n_kv * hd * 2);
    uint16_t* s = (uint16_t*)malloc((size_t)n_kv * 2);
    uint16_t* p = (uint16_t*)malloc((size_t)n_kv * 2);
    int rc = -1;
    if (!kT || !vo || !s || !p) goto done;
    if (go_kv_gather(c, kT, vo, n_kv, H, KVH, hd)) goto done;
    {
        const float sc = F(H(scale));
        for (uint32_t h = 0; h < H; h++) {
            for (uint32_t j = 0; j < n_kv; j++) {
                float acc = 0.0f;
                for (uint32_t d = 0; d < hd; d++)
                    acc += F(q[(size_t)h * hd + d]) * F(kT[((size_t)h * hd + d) * n_kv + j]);
                uint16_t t = H(acc);
                t = H(F(t) * sc);
                s[j] = H(F(t) + 0.0f);
            }
            go_softmax(s, p, 1, n_kv);
            for (uint32_t d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (uint32_t j = 0; j < n_kv; j++)
                    acc += F(p[j]) * F(vo[((size_t)h * n_kv + j) * hd + d]);
                out[(size_t)h * hd + d] = H(acc);
            }
        }
        rc = 0;
    }
done:
    free(kT); free(vo); free(s); free(p);
    return rc;
}

/* RoPE (half split) as the runlist computes it with f16 cos/sin tables built in
 * float64 (scripts/persistent_runtime.py:43-55: inv = 1/theta^(2j/d), cos/sin of
 * position * inv, each duplicated over both halves, cast to f16):
 *   y = BINARY add( BINARY mul(x, cos), BINARY mul(rotate_half(x), sin) )
 * rotate_half(x) = [-x2, x1] is exact in f16. */
int go_rope(const uint16_t* x, uint16_t* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd,
            uint32_t pos0, float theta, uint32_t row_stride) {
    if (hd % 2 || row_stride < n_heads * hd) return -1;
    const uint32_t half = hd / 2;
#pragma omp parallel for schedule(static) if (n_tok >= 64)
    for (uint32_t t = 0; t < n_tok; t++) {
        const double pos = (double)(pos0 + t);
        for (uint32_t i = 0; i < half; i++) {
            double inv = 1.0 / pow((double)theta, (double)(2 * i) / (double)hd);
            float c = F(f64_to_f16(cos(pos * inv)));
            float s = F(f64_to_f16(sin(pos * inv)));
            for (uint32_t h = 0; h < n_heads; h++) {
                const uint16_t* xr = x + (size_t)t * row_stride + (size_t)h * hd;
                uint16_t* yr = y + (size_t)t * row_stride + (size_t)h * hd;
                float x1 = F(xr[i]), x2 = F(xr[i + half]);
                float a1 = F(H(x1 * c)), b1 = F(H(-x2 * s));
                float a2 = F(H(x2 * c)), b2 = F(H(x1 * s));
                yr[i] = H(a1 + b1);
                yr[i + half] = H(a2 + b2);
            }
        }
    }
    return 0;
}
