/* gehtp_oracle_fast.c — vectorised forms of the oracle's heavy loops (TEST INFRASTRUCTURE).
 *
 * Loaded only by tests/, the smoke check and bench.py's cpu_baseline leg; the HIP
 * engine never links or calls it.
 *
 * Every function here computes what a scalar restatement in gehtp_oracle.c computes
 * (in summation order 0, the default; go_set_order below), with the same per-output
 * arithmetic: each output keeps its own sequential
 * accumulation order (k = 0, 1, 2, ... for the linears, d for attention scores, j for
 * attention values), with an f32 product rounded before the f32 add (no FMA: the file
 * is built with -ffp-contract=off), and the same f16 rounding points. Only the
 * iteration ORDER ACROSS outputs changes: eight (AVX2) neighbouring outputs advance
 * together, several rows share one pass over the weights, and output blocks run on
 * OpenMP threads. So results are bit-identical to the scalar forms for every input
 * that produces no NaN (NaN outputs still become the same-signed Inf of go_f32_to_f16,
 * but which NaN operand propagates — hence that sign — may differ).
 * tests/test_oracle_fast.py checks each function against its scalar form.
 *
 * f16 <-> f32 use the F16C conversions, which are IEEE binary16 with round-to-nearest
 * -even and gradual underflow (MXCSR's FTZ/DAZ stay off in this process); NaN lanes of
 * f32 -> f16 are redone by go_f32_to_f16 (NaN -> Inf, as oplist_exec.c:401 does).
 * On a CPU without AVX2/F16C every entry point runs its scalar form instead.
 */
#include "gehtp_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <float.h>
#include <stdlib.h>
#include <string.h>

#define TGT __attribute__((target("avx2,f16c")))
#define NB 16u    /* output columns per weight block: two 8-lane vectors */

typedef float v8f __attribute__((vector_size(32)));

static int g_fast = -1;

int go_fast_available(void) {
    if (g_fast < 0) {
        __builtin_cpu_init();
        g_fast = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("f16c");
    }
    return g_fast;
}

/* Force the scalar forms (1) or allow the vector forms again (0); for tests. */
void go_fast_disable(int off) { g_fast = off ? 0 : -1; }

/* Summation order of the vector forms' long sums (go_set_order). Mode 0 is the scalar
 * restatement's sequential order, bit-identical to it. Modes 1 and 2 are other valid
 * fp32 orders of the same products, with the same f16 rounding points, used only to
 * measure how far a correct implementation's results may move with the order alone:
 *   1: each sum cut into 32-wide slices (linears: k; attention scores: d), each slice
 *      summed in sequence from zero, the slice sums combined pairwise (a tree:
 *      (s0 + s1) + (s2 + s3) ...); attention's P.V sum over keys in 64-key chunks,
 *      combined pairwise;
 *   2: 16-wide slices summed from zero, their sums added in sequence
 *      (((s0 + s1) + s2) + ...); P.V in 64-key chunks added in sequence. */
static int g_order = 0;

int go_set_order(int mode) {
    if (mode < 0 || mode > 2 || (mode && !go_fast_available())) return -1;
    g_order = mode;
    return 0;
}

static inline uint32_t order_width(void) { return g_order == 1 ? 32u : 16u; }

/* Combine n slice sums (vectors at stride st) into v[0] in the mode's order. */
static inline void combine_slices(v8f* v, uint32_t n, uint32_t st) {
    if (g_order == 1) {
        for (uint32_t w = 1; w < n; w *= 2)
            for (uint32_t i = 0; i + w < n; i += 2 * w) v[(size_t)i * st] = v[(size_t)i * st] + v[(size_t)(i + w) * st];
    } else {
        for (uint32_t i = 1; i < n; i++) v[0] = v[0] + v[(size_t)i * st];
    }
}

TGT static inline v8f ld8(const float* p) { v8f v; memcpy(&v, p, sizeof v); return v; }
TGT static inline void st8(float* p, v8f v) { memcpy(p, &v, sizeof v); }
TGT static inline v8f bc8(float x) { return (v8f){x, x, x, x, x, x, x, x}; }

TGT static inline v8f h2f8(const uint16_t* p) {
    return (v8f)_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)p));
}

/* 8 floats -> 8 binary16, RNE; NaN lanes as go_f32_to_f16. */
TGT static inline void f2h8(uint16_t* p, v8f x) {
    __m128i h = _mm256_cvtps_ph((__m256)x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    _mm_storeu_si128((__m128i*)p, h);
    if (_mm256_movemask_ps(_mm256_cmp_ps((__m256)x, (__m256)x, _CMP_UNORD_Q))) {
        float t[8];
        memcpy(t, &x, sizeof t);
        for (int i = 0; i < 8; i++)
            if (t[i] != t[i]) p[i] = go_f32_to_f16(t[i]);
    }
}

/* F(H(x)): the value after an f16 rounding point (NaN lanes: go_f32_to_f16's Inf). */
TGT static inline v8f rt16(v8f x) {
    uint16_t h[8];
    f2h8(h, x);
    return h2f8(h);
}

/* ------------------------------------------------------------------------- */
/* Linears. A block holds NB weight rows (output columns) transposed to [K][NB] f32,
 * each value the f32 of the fp16 weight the scalar form multiplies by. */

/* W4G rows n0..n0+nb-1: fp16(q * s) (go_w4g_dequant), zero rows past nb. */
TGT static void block_w4g(const uint8_t* wq, const uint16_t* ws, uint32_t K, uint32_t group,
                          uint32_t n0, uint32_t nb, float* blk, float* tmp) {
    static const float nib[16] = {-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7};
    const uint32_t G = K / group;
    for (uint32_t r = 0; r < NB; r++) {
        if (r >= nb) {
            for (uint32_t k = 0; k < K; k++) blk[(size_t)k * NB + r] = 0.0f;
            continue;
        }
        const uint8_t* row = wq + (size_t)(n0 + r) * (K / 2);
        const uint16_t* srow = ws + (size_t)(n0 + r) * G;
        for (uint32_t k = 0; k < K; k += 8) {
            const v8f s = bc8(go_f16_to_f32(srow[k / group]));   /* group % 8 == 0 (checked) */
            const uint8_t* b = row + k / 2;
            v8f q = {nib[b[0] & 15], nib[b[0] >> 4], nib[b[1] & 15], nib[b[1] >> 4],
                     nib[b[2] & 15], nib[b[2] >> 4], nib[b[3] & 15], nib[b[3] >> 4]};
            st8(tmp + k, rt16(q * s));   /* q*s exact in f32, then one RNE to fp16 */
        }
        for (uint32_t k = 0; k < K; k++) blk[(size_t)k * NB + r] = tmp[k];
    }
}

/* fp16 rows [N][K] n0..n0+nb-1. */
TGT static void block_f16(const uint16_t* w, uint32_t K, uint32_t n0, uint32_t nb, float* blk,
                          float* tmp) {
    for (uint32_t r = 0; r < NB; r++) {
        if (r >= nb) {
            for (uint32_t k = 0; k < K; k++) blk[(size_t)k * NB + r] = 0.0f;
            continue;
        }
        const uint16_t* row = w + (size_t)(n0 + r) * K;
        uint32_t k = 0;
        for (; k + 8 <= K; k += 8) st8(tmp + k, h2f8(row + k));
        for (; k < K; k++) tmp[k] = go_f16_to_f32(row[k]);
        for (k = 0; k < K; k++) blk[(size_t)k * NB + r] = tmp[k];
    }
}

TGT static inline void store_row(uint16_t* y, v8f lo, v8f hi, uint32_t nb) {
    uint16_t h[NB];
    f2h8(h, lo);
    f2h8(h + 8, hi);
    memcpy(y, h, (size_t)nb * 2);
}

/* y[m, n0 + r] = f16(sum_k af[m,k] * blk[k][r]), k ascending, for all m < M. */
TGT static void mm_block(const float* af, uint32_t M, uint32_t K, const float* blk, uint16_t* y,
                         uint32_t ldy, uint32_t n0, uint32_t nb) {
    uint32_t m = 0;
    for (; m + 4 <= M; m += 4) {
        const float* a0 = af + (size_t)m * K;
        const float* a1 = a0 + K;
        const float* a2 = a1 + K;
        const float* a3 = a2 + K;
        v8f c00 = bc8(0.0f), c01 = c00, c10 = c00, c11 = c00, c20 = c00, c21 = c00, c30 = c00, c31 = c00;
        for (uint32_t k = 0; k < K; k++) {
            const v8f w0 = ld8(blk + (size_t)k * NB), w1 = ld8(blk + (size_t)k * NB + 8);
            const v8f x0 = bc8(a0[k]), x1 = bc8(a1[k]), x2 = bc8(a2[k]), x3 = bc8(a3[k]);
            c00 = c00 + x0 * w0; c01 = c01 + x0 * w1;
            c10 = c10 + x1 * w0; c11 = c11 + x1 * w1;
            c20 = c20 + x2 * w0; c21 = c21 + x2 * w1;
            c30 = c30 + x3 * w0; c31 = c31 + x3 * w1;
        }
        store_row(y + (size_t)m * ldy + n0, c00, c01, nb);
        store_row(y + (size_t)(m + 1) * ldy + n0, c10, c11, nb);
        store_row(y + (size_t)(m + 2) * ldy + n0, c20, c21, nb);
        store_row(y + (size_t)(m + 3) * ldy + n0, c30, c31, nb);
    }
    for (; m < M; m++) {
        const float* a0 = af + (size_t)m * K;
        v8f c0 = bc8(0.0f), c1 = c0;
        for (uint32_t k = 0; k < K; k++) {
            const v8f x0 = bc8(a0[k]);
            c0 = c0 + x0 * ld8(blk + (size_t)k * NB);
            c1 = c1 + x0 * ld8(blk + (size_t)k * NB + 8);
        }
        store_row(y + (size_t)m * ldy + n0, c0, c1, nb);
    }
}

/* mm_block in the order of g_order (1 or 2): per row, the two 8-column accumulators
 * restart at each slice of order_width() k values; part holds 2 * ceil(K / width)
 * vectors. */
TGT static void mm_block_ordered(const float* af, uint32_t M, uint32_t K, const float* blk, uint16_t* y,
                                 uint32_t ldy, uint32_t n0, uint32_t nb, v8f* part) {
    const uint32_t W = order_width(), ns = (K + W - 1) / W;
    for (uint32_t m = 0; m < M; m++) {
        const float* a0 = af + (size_t)m * K;
        for (uint32_t sl = 0; sl < ns; sl++) {
            v8f c0 = bc8(0.0f), c1 = c0;
            const uint32_t ke = (sl + 1) * W < K ? (sl + 1) * W : K;
            for (uint32_t k = sl * W; k < ke; k++) {
                const v8f x0 = bc8(a0[k]);
                c0 = c0 + x0 * ld8(blk + (size_t)k * NB);
                c1 = c1 + x0 * ld8(blk + (size_t)k * NB + 8);
            }
            part[2 * sl] = c0;
            part[2 * sl + 1] = c1;
        }
        combine_slices(part, ns, 2);
        combine_slices(part + 1, ns, 2);
        store_row(y + (size_t)m * ldy + n0, part[0], part[1], nb);
    }
}

TGT static float* to_f32(const uint16_t* a, size_t n) {
    float* f = (float*)malloc(n * sizeof(float) + 32);
    if (!f) return NULL;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) st8(f + i, h2f8(a + i));
    for (; i < n; i++) f[i] = go_f16_to_f32(a[i]);
    return f;
}

/* Shared driver: wq/ws (W4G) or w (fp16 [N][K]) -> y[M][N]. */
TGT static int linear_fast(const uint16_t* a, const uint8_t* wq, const uint16_t* ws,
                           const uint16_t* w, uint16_t* y, uint32_t M, uint32_t K, uint32_t N,
                           uint32_t group, int n_threads) {
    float* af = to_f32(a, (size_t)M * K);
    if (!af) return -1;
    const uint32_t nblk = (N + NB - 1) / NB;
    int fail = 0;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
    {
        float* blk = (float*)malloc((size_t)K * NB * sizeof(float));
        float* tmp = (float*)malloc((size_t)K * sizeof(float) + 64);
        v8f* part = (v8f*)aligned_alloc(32, ((size_t)2 * (K / 16 + 1) * sizeof(v8f) + 31) / 32 * 32);
        if (!blk || !tmp || !part) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (uint32_t b = 0; b < nblk; b++) {
                const uint32_t n0 = b * NB, nb = N - n0 < NB ? N - n0 : NB;
                if (wq) block_w4g(wq, ws, K, group, n0, nb, blk, tmp);
                else block_f16(w, K, n0, nb, blk, tmp);
                if (g_order) mm_block_ordered(af, M, K, blk, y, N, n0, nb, part);
                else mm_block(af, M, K, blk, y, N, n0, nb);
            }
        }
        free(blk);
        free(tmp);
        free(part);
    }
    free(af);
    return fail ? -1 : 0;
}

int go_matmul_w4g(const uint16_t* a, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                  uint32_t M, uint32_t K, uint32_t N, uint32_t group, int n_threads) {
    if (!group || K % group || K % 2) return -1;
    if (!go_fast_available() || group % 8) return go_matmul_w4g_ref(a, wq, ws, y, M, K, N, group, n_threads);
    return linear_fast(a, wq, ws, NULL, y, M, K, N, group, n_threads);
}

int go_matmul_f16_nk_mt(const uint16_t* a, const uint16_t* w, uint16_t* y,
                        uint32_t M, uint32_t K, uint32_t N, int n_threads) {
    if (!go_fast_available()) return go_matmul_f16_nk_ref(a, w, y, M, K, N, n_threads);
    return linear_fast(a, NULL, NULL, w, y, M, K, N, 0, n_threads);
}

/* ------------------------------------------------------------------------- */
/* Attention. Scores of one query row i against keys j (vectorised over j) follow
 * go_attn_prefill's chain: t = f16(sum_d q*k), t = f16(t * f16(scale)),
 * s = f16(t + mask); the causal mask's -inf keys (j > i) are not computed: their
 * softmax terms are exact zeros in both softmax forms (exp(-inf) = 0 adds nothing
 * to the sum, and p = f16(0 * inv) = 0), and 0 * v adds nothing to an output sum
 * that starts at +0 (p >= 0, so the sum never holds -0) as long as v is finite:
 * with a non-finite V row the masked keys are computed too. */

/* scores srow[j] for j in [0, jn) of query qrow against kt [hd][ldk] (f32 of K^T). */
TGT static void attn_scores(const float* qrow, const float* kt, uint32_t ldk, uint32_t hd,
                            uint32_t jn, float sc, float* srow) {
    const v8f vsc = bc8(sc), zero = bc8(0.0f);
    uint32_t j0 = 0;
    if (g_order) {   /* d in slices of order_width(), combined in the mode's order */
        const uint32_t W = order_width(), ns = (hd + W - 1) / W;
        v8f part[256 / 16];
        for (; j0 < jn; j0 += 8) {   /* kt rows are padded to a multiple of 8 keys */
            for (uint32_t sl = 0; sl < ns; sl++) {
                v8f c0 = zero;
                const uint32_t de = (sl + 1) * W < hd ? (sl + 1) * W : hd;
                for (uint32_t d = sl * W; d < de; d++) c0 = c0 + bc8(qrow[d]) * ld8(kt + (size_t)d * ldk + j0);
                part[sl] = c0;
            }
            combine_slices(part, ns, 1);
            st8(srow + j0, rt16(rt16(rt16(part[0]) * vsc) + zero));
        }
        return;
    }
    for (; j0 + 32 <= jn; j0 += 32) {
        v8f c0 = zero, c1 = zero, c2 = zero, c3 = zero;
        for (uint32_t d = 0; d < hd; d++) {
            const v8f x = bc8(qrow[d]);
            const float* kr = kt + (size_t)d * ldk + j0;
            c0 = c0 + x * ld8(kr);
            c1 = c1 + x * ld8(kr + 8);
            c2 = c2 + x * ld8(kr + 16);
            c3 = c3 + x * ld8(kr + 24);
        }
        st8(srow + j0, rt16(rt16(rt16(c0) * vsc) + zero));
        st8(srow + j0 + 8, rt16(rt16(rt16(c1) * vsc) + zero));
        st8(srow + j0 + 16, rt16(rt16(rt16(c2) * vsc) + zero));
        st8(srow + j0 + 24, rt16(rt16(rt16(c3) * vsc) + zero));
    }
    for (; j0 < jn; j0 += 8) {   /* kt rows are padded to a multiple of 8 keys */
        v8f c0 = zero;
        for (uint32_t d = 0; d < hd; d++) c0 = c0 + bc8(qrow[d]) * ld8(kt + (size_t)d * ldk + j0);
        st8(srow + j0, rt16(rt16(rt16(c0) * vsc) + zero));
    }
}

/* p[0..jn) from scores s[0..jn) of a row of n keys (the others -inf), with
 * exec_softmax's dispatch on (rows, n) (go_softmax): returns the f32 of the f16 p. */
static void attn_softmax(const float* s, float* p, uint32_t jn, uint32_t rows, uint32_t n) {
    if (rows >= 1 && n % 32 == 0 && (size_t)rows * n >= 32) {   /* go_softmax_host */
        float mx = -FLT_MAX;
        for (uint32_t j = 0; j < jn; j++) if (s[j] > mx) mx = s[j];
        double sum = 0.0;
        for (uint32_t j = 0; j < jn; j++) { p[j] = expf(s[j] - mx); sum += p[j]; }
        const float inv = (sum > 0.0) ? (float)(1.0 / sum) : 0.0f;
        for (uint32_t j = 0; j < jn; j++) p[j] = go_f16_to_f32(go_f32_to_f16(p[j] * inv));
    } else {                                                      /* go_softmax_scalar */
        float mx = s[0];
        for (uint32_t j = 1; j < jn; j++) mx = fmaxf(mx, s[j]);
        float sum = 0.0f;
        for (uint32_t j = 0; j < jn; j++) {
            const float e = expf(s[j] - mx);
            p[j] = go_f16_to_f32(go_f32_to_f16(e));
            sum += e;
        }
        for (uint32_t j = 0; j < jn; j++) p[j] = go_f16_to_f32(go_f32_to_f16(p[j] / sum));
    }
}

/* out[d] = f16(sum_j p[j] * v[j][d]), j ascending, hd % 8 == 0, hd <= 256. */
TGT static void attn_values(const float* p, const float* vf, uint32_t hd, uint32_t jn, uint16_t* out) {
    v8f acc[32];
    const uint32_t nv = hd / 8;
    if (g_order) {   /* keys in 64-key chunks, each from zero, combined in the mode's order */
        const uint32_t nc = (jn + 63) / 64;
        v8f* part = (v8f*)aligned_alloc(32, (size_t)(nc ? nc : 1) * nv * sizeof(v8f));
        if (part) {
            for (uint32_t c = 0; c < nc; c++) {
                for (uint32_t i = 0; i < nv; i++) acc[i] = bc8(0.0f);
                const uint32_t je = (c + 1) * 64 < jn ? (c + 1) * 64 : jn;
                for (uint32_t j = c * 64; j < je; j++) {
                    const v8f pb = bc8(p[j]);
                    const float* vr = vf + (size_t)j * hd;
                    for (uint32_t i = 0; i < nv; i++) acc[i] = acc[i] + pb * ld8(vr + 8 * i);
                }
                for (uint32_t i = 0; i < nv; i++) part[(size_t)c * nv + i] = acc[i];
            }
            for (uint32_t i = 0; i < nv; i++) {
                if (nc) combine_slices(part + i, nc, nv);
                f2h8(out + 8 * i, nc ? part[i] : bc8(0.0f));
            }
            free(part);
            return;
        }
    }
    for (uint32_t i = 0; i < nv; i++) acc[i] = bc8(0.0f);
    for (uint32_t j = 0; j < jn; j++) {
        const v8f pb = bc8(p[j]);
        const float* vr = vf + (size_t)j * hd;
        for (uint32_t i = 0; i < nv; i++) acc[i] = acc[i] + pb * ld8(vr + 8 * i);
    }
    for (uint32_t i = 0; i < nv; i++) f2h8(out + 8 * i, acc[i]);
}

static int all_finite(const float* v, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!(v[i] - v[i] == 0.0f)) return 0;
    return 1;
}

TGT static int attn_prefill_fast(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                                 uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale,
                                 int causal, int n_threads) {
    const uint32_t rep = H / KVH;
    const float sc = go_f16_to_f32(go_f32_to_f16(scale));
    const uint32_t ldk = (S + 7) / 8 * 8;
    int fail = 0;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
    {
        float* kt = (float*)calloc((size_t)hd * ldk, sizeof(float));
        float* vf = (float*)malloc((size_t)S * hd * sizeof(float));
        float* qf = (float*)malloc((size_t)hd * sizeof(float));
        float* srow = (float*)malloc((size_t)ldk * sizeof(float));
        float* prow = (float*)malloc((size_t)ldk * sizeof(float));
        if (!kt || !vf || !qf || !srow || !prow) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (uint32_t h = 0; h < H; h++) {
                const uint32_t g = h / rep;
                for (uint32_t j = 0; j < S; j++)
                    for (uint32_t d = 0; d < hd; d++) {
                        kt[(size_t)d * ldk + j] = go_f16_to_f32(k[((size_t)j * KVH + g) * hd + d]);
                        vf[(size_t)j * hd + d] = go_f16_to_f32(v[((size_t)j * KVH + g) * hd + d]);
                    }
                const int skip = causal && all_finite(vf, (size_t)S * hd);
                for (uint32_t i = 0; i < S; i++) {
                    for (uint32_t d = 0; d < hd; d++) qf[d] = go_f16_to_f32(q[((size_t)i * H + h) * hd + d]);
                    const uint32_t jn = skip ? i + 1 : S;
                    attn_scores(qf, kt, ldk, hd, jn, sc, srow);
                    if (causal && !skip)
                        for (uint32_t j = i + 1; j < S; j++) srow[j] = -INFINITY;
                    attn_softmax(srow, prow, jn, S, S);
                    attn_values(prow, vf, hd, jn, out + ((size_t)i * H + h) * hd);
                }
            }
        }
        free(kt); free(vf); free(qf); free(srow); free(prow);
    }
    return fail ? -1 : 0;
}

int go_attn_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                    uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal) {
    return go_attn_prefill_mt(q, k, v, out, S, H, KVH, hd, scale, causal, 1);
}

int go_attn_prefill_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                       uint32_t S, uint32_t H, uint32_t KVH, uint32_t hd, float scale, int causal,
                       int n_threads) {
    if (!S || !H || !KVH || H % KVH) return -1;
    if (!go_fast_available() || hd % 8 || hd > 256)
        return go_attn_prefill_ref(q, k, v, out, S, H, KVH, hd, scale, causal);
    return attn_prefill_fast(q, k, v, out, S, H, KVH, hd, scale, causal, n_threads);
}

/* One query token against positions [0, n_kv) of a KV ring held as raw bytes + posmap
 * (the state go_kv and oracle.KVRing keep), as go_attn_decode computes it. */
TGT static int attn_ring_fast(const uint8_t* buf, const uint32_t* posmap, uint32_t nslots,
                              uint32_t slot_bytes, const uint16_t* q, uint16_t* out, uint32_t n_kv,
                              uint32_t H, uint32_t KVH, uint32_t hd, float scale) {
    const uint32_t rep = H / KVH;
    const float sc = go_f16_to_f32(go_f32_to_f16(scale));
    const uint32_t ldk = (n_kv + 7) / 8 * 8;
    float* kt = (float*)calloc((size_t)hd * ldk, sizeof(float));
    float* vf = (float*)malloc((size_t)n_kv * hd * sizeof(float));
    float* qf = (float*)malloc((size_t)hd * sizeof(float));
    float* srow = (float*)malloc((size_t)ldk * sizeof(float));
    float* prow = (float*)malloc((size_t)ldk * sizeof(float));
    int rc = -1;
    if (!kt || !vf || !qf || !srow || !prow) goto done;
    for (uint32_t g = 0; g < KVH; g++) {
        for (uint32_t j = 0; j < n_kv; j++) {
            const uint16_t* kf = (const uint16_t*)(buf + (size_t)(j % nslots) * slot_bytes) + (size_t)g * hd;
            const uint16_t* vv = (const uint16_t*)(buf + (size_t)(j % nslots) * slot_bytes + slot_bytes / 2) +
                                 (size_t)g * hd;
            for (uint32_t d = 0; d < hd; d++) {
                kt[(size_t)d * ldk + j] = go_f16_to_f32(kf[d]);
                vf[(size_t)j * hd + d] = go_f16_to_f32(vv[d]);
            }
        }
        for (uint32_t r = 0; r < rep; r++) {
            const uint32_t h = g * rep + r;
            for (uint32_t d = 0; d < hd; d++) qf[d] = go_f16_to_f32(q[(size_t)h * hd + d]);
            attn_scores(qf, kt, ldk, hd, n_kv, sc, srow);
            attn_softmax(srow, prow, n_kv, 1, n_kv);
            attn_values(prow, vf, hd, n_kv, out + (size_t)h * hd);
        }
    }
    rc = 0;
done:
    free(kt); free(vf); free(qf); free(srow); free(prow);
    return rc;
}

int go_attn_decode_ring(const uint8_t* buf, const uint32_t* posmap, uint32_t nslots, uint32_t slot_bytes,
                        const uint16_t* q, uint16_t* out, uint32_t n_kv, uint32_t H, uint32_t KVH,
                        uint32_t hd, float scale) {
    if (!n_kv || !H || !KVH || H % KVH || !nslots || KVH * hd * 4u != slot_bytes) return -1;
    for (uint32_t p = 0; p < n_kv; p++)
        if (posmap[p % nslots] != p) return -2;   /* lookup miss, as go_kv_gather */
    if (!go_fast_available() || hd % 8 || hd > 256) {
        struct go_kv c = {(uint8_t*)buf, slot_bytes, nslots, n_kv, (uint32_t*)posmap};
        return go_attn_decode(&c, q, out, n_kv, H, KVH, hd, scale);
    }
    return attn_ring_fast(buf, posmap, nslots, slot_bytes, q, out, n_kv, H, KVH, hd, scale);
}
