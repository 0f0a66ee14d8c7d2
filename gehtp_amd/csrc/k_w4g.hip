// k_w4g.hip — W4A16 group-64 kernels for gfx950: decode GEMV, prefill GEMM (MFMA), dequant.
//
// Weight format (OP_MATMUL_W4G_F16): wq row n = K/2 bytes, byte j holds k=2j in the
// low nibble and k=2j+1 in the high nibble, stored as q+8; ws[n][k/64] fp16.
// Dequant is fp16(q*s), RNE — computed as two exact packed-fp16 steps:
//   h = half(0x6400 | nib) = 1024 + nib;  q = h - 1032 (exact);  w = q * s (one RNE).
//
// One 32-bit word of weights = 8 consecutive k. Masking (w >> 4i) & 0x000F000F gives
// the half pairs (k0,k4), (k1,k5), (k2,k6), (k3,k7); activations are staged in the
// same pair order so each pair feeds one v_dot2_f32_f16 (fp32 accumulate).
#include "kernels.h"

namespace gehtp {

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16x_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Four dequantized pairs (k0,k4),(k1,k5),(k2,k6),(k3,k7) of one weight word.
__device__ __forceinline__ void dequant_word(uint32_t w, h2_t s2, h2_t out[4]) {
    const h2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t m = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
        const h2_t q = as_h2(m) - bias;   // exact: integers below 2048
        out[i] = q * s2;                  // one RNE rounding: fp16(q*s)
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// GEMV: each workgroup streams the contiguous weight rows [r0, r0+RB) as a flat
// sequence of 32-byte groups (j = row*G + g), so consecutive threads read
// consecutive 32-byte pieces regardless of K. Activations sit in LDS as
// xs[m][c][g] (16 bytes each, pair order) so that threads working on consecutive
// groups read consecutive 16-byte LDS words. Group partial sums land in LDS and
// one wavefront per row (or row pair, for SwiGLU) adds them up and applies the
// epilogue.
struct GemvArgs {
    const __half* x;
    uint32_t ldx;
    const u32x4* wq;
    const __half* ws;
    __half* y;
    uint32_t ldy;
    uint32_t N, G, rows_per_wg;
    const __half* gamma;
    const __half* res;
    uint32_t ldr;
    int swiglu;
};

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2hb(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

template <int MR>
__global__ __launch_bounds__(256) void w4g_gemv_kernel(GemvArgs A) {
    extern __shared__ uint4 smem[];
    const uint32_t G = A.G;
    uint4* xs = smem;                                   // [MR][8][G]
    float* red = reinterpret_cast<float*>(smem + MR * 8 * G);   // [MR][RB*G]
    __shared__ double s_ss[4][MR];
    __shared__ float s_rms[MR];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t r0 = blockIdx.x * A.rows_per_wg;
    const uint32_t RB = min(A.rows_per_wg, A.N - r0);
    const uint32_t T = RB * G;
    const u32x4* wrow = A.wq + (size_t)r0 * G * 2;
    const __half* srow = A.ws + (size_t)r0 * G;

    constexpr int U = 4;
    // Issue the first batch of weight loads before staging activations.
    u32x4 wv[U][2];
    __half sv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t j = tid + 256u * u;
        if (j < T) {
            wv[u][0] = __builtin_nontemporal_load(&wrow[2 * j]);
            wv[u][1] = __builtin_nontemporal_load(&wrow[2 * j + 1]);
            sv[u] = srow[j];
        }
    }

    // Optional RMSNorm prologue: every workgroup computes the rows' sums of squares
    // (in double, as RMSNORM2_F16 does) from its own reads of x.
    if (A.gamma) {
        double ss[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) ss[m] = 0.0;
        for (uint32_t i = tid; i < 8 * G; i += 256) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint4 v = *reinterpret_cast<const uint4*>(A.x + (size_t)m * A.ldx + i * 8);
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const double lo = (double)h2f((uint16_t)(w4[e] & 0xFFFFu));
                    const double hi = (double)h2f((uint16_t)(w4[e] >> 16));
                    ss[m] += lo * lo;
                    ss[m] += hi * hi;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const double t = wave_sum_d(ss[m]);
            if (lane == 0) s_ss[wave][m] = t;
        }
        __syncthreads();
        if (tid < MR) {
            const double t = s_ss[0][tid] + s_ss[1][tid] + s_ss[2][tid] + s_ss[3][tid];
            s_rms[tid] = (float)sqrt(t / (double)(G * 64) + 1e-6);
        }
        __syncthreads();
    }

    for (uint32_t i = tid; i < MR * 8 * G; i += 256) {
        const uint32_t m = i / (8 * G);
        const uint32_t rem = i - m * 8 * G;
        const uint32_t g = rem >> 3, c = rem & 7;
        uint4 v = *reinterpret_cast<const uint4*>(A.x + (size_t)m * A.ldx + g * 64 + c * 8);
        if (A.gamma) {
            // h = f16(f16-exact x / rms * gamma + 0), the RMSNORM2_F16 arithmetic
            const uint4 gv = *reinterpret_cast<const uint4*>(A.gamma + g * 64 + c * 8);
            const float rms = s_rms[m];
            uint32_t w4[4] = {v.x, v.y, v.z, v.w};
            const uint32_t g4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float lo = __fdiv_rn(h2f((uint16_t)(w4[e] & 0xFFFFu)), rms);
                float hi = __fdiv_rn(h2f((uint16_t)(w4[e] >> 16)), rms);
                lo = __fadd_rn(__fmul_rn(lo, h2f((uint16_t)(g4[e] & 0xFFFFu))), 0.0f);
                hi = __fadd_rn(__fmul_rn(hi, h2f((uint16_t)(g4[e] >> 16))), 0.0f);
                w4[e] = (uint32_t)f2hb(lo) | ((uint32_t)f2hb(hi) << 16);
            }
            v = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        uint4 p;
        p.x = (v.x & 0xFFFFu) | (v.z << 16);
        p.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
        p.z = (v.y & 0xFFFFu) | (v.w << 16);
        p.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
        xs[(m * 8 + c) * G + g] = p;
    }
    __syncthreads();

    const uint32_t step = 256u % G;
    uint32_t g0 = tid % G;
    for (uint32_t jb = tid; jb < T; jb += 256u * U) {
        uint32_t g = g0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = jb + 256u * u;
            if (j < T) {
                const _Float16 s = __builtin_bit_cast(_Float16, sv[u]);
                const h2_t s2 = {s, s};
                float acc[MR];
#pragma unroll
                for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
                const uint32_t words[8] = {wv[u][0].x, wv[u][0].y, wv[u][0].z, wv[u][0].w,
                                           wv[u][1].x, wv[u][1].y, wv[u][1].z, wv[u][1].w};
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    h2_t d[4];
                    dequant_word(words[c], s2, d);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        const uint4 xv = xs[(m * 8 + c) * G + g];
                        acc[m] = __builtin_amdgcn_fdot2(d[0], as_h2(xv.x), acc[m], false);
                        acc[m] = __builtin_amdgcn_fdot2(d[1], as_h2(xv.y), acc[m], false);
                        acc[m] = __builtin_amdgcn_fdot2(d[2], as_h2(xv.z), acc[m], false);
                        acc[m] = __builtin_amdgcn_fdot2(d[3], as_h2(xv.w), acc[m], false);
                    }
                }
#pragma unroll
                for (int m = 0; m < MR; ++m) red[m * T + j] = acc[m];
            }
            g += step;
            if (g >= G) g -= G;
        }
        g0 = g;
        // Next batch of loads.
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = jb + 256u * U + 256u * u;
            if (j < T) {
                wv[u][0] = __builtin_nontemporal_load(&wrow[2 * j]);
                wv[u][1] = __builtin_nontemporal_load(&wrow[2 * j + 1]);
                sv[u] = srow[j];
            }
        }
    }
    __syncthreads();

    if (!A.swiglu) {
        for (uint32_t r = wave; r < RB; r += 4) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float s = 0.0f;
                for (uint32_t i = lane; i < G; i += 64) s += red[m * T + r * G + i];
                s = wave_sum(s);
                if (lane == 0) {
                    uint16_t v = f2hb(s);
                    if (A.res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, A.res[(size_t)m * A.ldr + r0 + r]))));
                    reinterpret_cast<uint16_t*>(A.y)[(size_t)m * A.ldy + r0 + r] = v;
                }
            }
        }
    } else {
        // rows (2p, 2p+1) = (gate, up) of output column (r0 + 2p) / 2; r0 and RB are even
        for (uint32_t p = wave; 2 * p < RB; p += 4) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float sg = 0.0f, su = 0.0f;
                for (uint32_t i = lane; i < G; i += 64) {
                    sg += red[m * T + (2 * p) * G + i];
                    su += red[m * T + (2 * p + 1) * G + i];
                }
                sg = wave_sum(sg);
                su = wave_sum(su);
                if (lane == 0) {
                    const float gv = h2f(f2hb(sg)), uv = h2f(f2hb(su));
                    const float act = h2f(f2hb(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv)))));
                    uint16_t v = f2hb(__fmul_rn(act, uv));
                    const uint32_t col = (r0 >> 1) + p;
                    if (A.res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, A.res[(size_t)m * A.ldr + col]))));
                    reinterpret_cast<uint16_t*>(A.y)[(size_t)m * A.ldy + col] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Bit-exact dequant: one thread per 32 weights (16 bytes in, 64 bytes out).
__global__ __launch_bounds__(256) void w4g_dequant_kernel(const uint4* __restrict__ wq,
                                                          const __half* __restrict__ ws,
                                                          uint4* __restrict__ w, uint32_t n_chunks,
                                                          uint32_t G) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;   // chunk of 32 weights
    if (i >= n_chunks) return;
    const uint4 v = wq[i];
    const _Float16 s = __builtin_bit_cast(_Float16, ws[i >> 1]);   // 2 chunks per group
    const h2_t s2 = {s, s};
    (void)G;
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        h2_t d[4];
        dequant_word(words[c], s2, d);
        // back to natural order k0..k7
        uint4 o;
        o.x = (as_u32(d[0]) & 0xFFFFu) | (as_u32(d[1]) << 16);
        o.y = (as_u32(d[2]) & 0xFFFFu) | (as_u32(d[3]) << 16);
        o.z = (as_u32(d[0]) >> 16) | (as_u32(d[1]) & 0xFFFF0000u);
        o.w = (as_u32(d[2]) >> 16) | (as_u32(d[3]) & 0xFFFF0000u);
        w[(size_t)i * 4 + c] = o;
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM: C[M,N] = A[M,K] . dequant(W)^T on v_mfma_f32_32x32x16_f16.
// Workgroup tile 128x128, BK = 64 (one scale group), 4 waves in a 2x2 layout, each
// wave 64x64 = 2x2 MFMA tiles. A and the dequantized W tile are staged in LDS with
// a 16-byte row pad; the next K step's global loads are issued before the MFMAs.
constexpr int BM = 128, BN = 128, BK = 64, LDS_STRIDE = BK + 8;   // halves

__global__ __launch_bounds__(256) void w4g_gemm_kernel(
    const __half* __restrict__ a, uint32_t lda, const uint4* __restrict__ wq,
    const __half* __restrict__ ws, __half* __restrict__ y, uint32_t ldy, uint32_t M, uint32_t N,
    uint32_t K, const __half* __restrict__ res, uint32_t ldr, int swiglu) {
    __shared__ __align__(16) _Float16 As[BM * LDS_STRIDE];
    __shared__ __align__(16) _Float16 Bs[BN * LDS_STRIDE];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t G = K / 64;

    // Global load assignment. A: 4 x 16 bytes per thread (rows tid/8 + 32i, chunk tid%8).
    // W: row n0 + tid/2, half tid%2 (32 weights = 16 bytes) plus its scale.
    const uint32_t a_chunk = tid & 7, a_row = tid >> 3;
    const uint32_t w_row = tid >> 1, w_half = tid & 1;
    const bool w_ok = n0 + w_row < N;

    uint4 ra[4];
    uint4 rw = make_uint4(0, 0, 0, 0);
    __half rs = __float2half(0.0f);

    auto load_k = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = m0 + a_row + 32u * i;
            ra[i] = r < M ? *reinterpret_cast<const uint4*>(a + (size_t)r * lda + kb * 64 + a_chunk * 8)
                          : make_uint4(0, 0, 0, 0);
        }
        if (w_ok) {
            rw = wq[((size_t)(n0 + w_row) * G + kb) * 2 + w_half];
            rs = ws[(size_t)(n0 + w_row) * G + kb];
        }
    };

    f16x_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const uint32_t wm = wave >> 1, wn = wave & 1;
    load_k(0);
    for (uint32_t kb = 0; kb < G; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(&As[(a_row + 32 * i) * LDS_STRIDE + a_chunk * 8]) = ra[i];
        {
            const _Float16 s = __builtin_bit_cast(_Float16, rs);
            const h2_t s2 = {s, s};
            const uint32_t words[4] = {rw.x, rw.y, rw.z, rw.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                h2_t d[4];
                dequant_word(words[c], s2, d);
                uint4 o;
                o.x = (as_u32(d[0]) & 0xFFFFu) | (as_u32(d[1]) << 16);
                o.y = (as_u32(d[2]) & 0xFFFFu) | (as_u32(d[3]) << 16);
                o.z = (as_u32(d[0]) >> 16) | (as_u32(d[1]) & 0xFFFF0000u);
                o.w = (as_u32(d[2]) >> 16) | (as_u32(d[3]) & 0xFFFF0000u);
                *reinterpret_cast<uint4*>(&Bs[w_row * LDS_STRIDE + w_half * 32 + c * 8]) = o;
            }
        }
        __syncthreads();
        if (kb + 1 < G) load_k(kb + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            h8_t af[2], bf[2];
            const uint32_t kof = kk * 16 + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const h8_t*>(&As[(wm * 64 + i * 32 + (lane & 31)) * LDS_STRIDE + kof]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const h8_t*>(&Bs[(wn * 64 + j * 32 + (lane & 31)) * LDS_STRIDE + kof]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // Accumulator layout (32x32): lane l, reg r -> col l%32, row 8*(r/4) + 4*(l/32) + r%4.
    // With SwiGLU, columns 2c / 2c+1 (gate / up of output c) sit in lanes l, l^1.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float partner = __shfl_xor(acc[i][j][r], 1, 64);
                if (col >= N || row >= M) continue;
                uint16_t v;
                uint32_t oc = col;
                if (swiglu) {
                    if (lane & 1) continue;
                    const float gv = h2f(f2hb(acc[i][j][r])), uv = h2f(f2hb(partner));
                    const float act = h2f(f2hb(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv)))));
                    v = f2hb(__fmul_rn(act, uv));
                    oc = col >> 1;
                } else {
                    v = f2hb(acc[i][j][r]);
                }
                if (res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, res[(size_t)row * ldr + oc]))));
                reinterpret_cast<uint16_t*>(y)[(size_t)row * ldy + oc] = v;
            }
        }
}

}  // namespace

hipError_t launch_w4g_gemv(const __half* x, uint32_t ldx, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi) {
    if (M == 0 || N == 0) return hipSuccess;
    if (epi.swiglu && (N & 1)) return hipErrorInvalidValue;
    const uint32_t G = K / 64;
    const uint32_t target_wgs = 2u * (uint32_t)device_cu_count();
    const uint32_t t_max = M == 1 ? 2048u : 1024u;
    uint32_t rb = (N + target_wgs - 1) / target_wgs;
    const uint32_t rb_cap = t_max / G > 0 ? t_max / G : 1;
    if (rb > rb_cap) rb = rb_cap;
    if (rb < 1) rb = 1;
    if (epi.swiglu) rb = (rb + 1) & ~1u;   // gate/up pairs never straddle workgroups
    const uint32_t grid = (N + rb - 1) / rb;
    const size_t lds = (size_t)M * K * 2 + (size_t)M * rb * G * 4;
    // Activations live in LDS: beyond the 64 KiB dynamic-LDS budget use the GEMM.
    if (lds > 65536) {
        if (epi.gamma) return hipErrorInvalidValue;   // the engine normalizes before a GEMM
        return launch_w4g_gemm(x, ldx, wq, ws, y, ldy, M, N, K, st, epi);
    }
    GemvArgs A{x, ldx, reinterpret_cast<const u32x4*>(wq), ws, y, ldy, N, G, rb,
               epi.gamma, epi.res, epi.ldr, epi.swiglu ? 1 : 0};
    switch (M) {
    case 1: hipLaunchKernelGGL(w4g_gemv_kernel<1>, dim3(grid), dim3(256), lds, st, A); break;
    case 2: hipLaunchKernelGGL(w4g_gemv_kernel<2>, dim3(grid), dim3(256), lds, st, A); break;
    case 3: hipLaunchKernelGGL(w4g_gemv_kernel<3>, dim3(grid), dim3(256), lds, st, A); break;
    case 4: hipLaunchKernelGGL(w4g_gemv_kernel<4>, dim3(grid), dim3(256), lds, st, A); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_w4g_gemm(const __half* a, uint32_t lda, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi) {
    if (M == 0 || N == 0) return hipSuccess;
    if (epi.gamma || (epi.swiglu && (N & 1))) return hipErrorInvalidValue;
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(w4g_gemm_kernel, grid, dim3(256), 0, st, a, lda,
                       reinterpret_cast<const uint4*>(wq), ws, y, ldy, M, N, K, epi.res, epi.ldr,
                       epi.swiglu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_w4g_dequant(const uint8_t* wq, const __half* ws, __half* w, uint32_t N,
                              uint32_t K, hipStream_t st) {
    const uint32_t n_chunks = N * (K / 32);
    if (!n_chunks) return hipSuccess;
    hipLaunchKernelGGL(w4g_dequant_kernel, dim3((n_chunks + 255) / 256), dim3(256), 0, st,
                       reinterpret_cast<const uint4*>(wq), ws, reinterpret_cast<uint4*>(w), n_chunks,
                       K / 64);
    return hipGetLastError();
}

}  // namespace gehtp
