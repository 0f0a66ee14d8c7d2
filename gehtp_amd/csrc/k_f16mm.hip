// k_f16mm.hip — fp16 x fp16 -> fp16 matmul with the reference OP_MATMUL_F16 contract
// (oplist_exec.c:1709-1813): flags t0 (a stored [K,M]), t1 (w stored [N,K]), batched
// (Bn in flags >> 16), and the SPLIT column window [n0, n0+N) of an N_full-wide output.
//
//   M <= 4, t1:   GEMV, one wavefront per output column n streaming w's row n (the
//                 lm_head path); activations staged once per workgroup in LDS.
//   M <= 4, !t1:  GEMV over columns, one thread per n (w rows are contiguous in n).
//   otherwise:    MFMA 32x32x16 tiles with element-guarded loads (any shape/flags).
#include "kernels.h"

namespace gehtp {

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f16x_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Reinterpret a 32-bit word as two halves. Takes the word BY VALUE: a bit cast applied
// directly to an ext_vector element (v[e]) miscompiles to always reading element 0.
__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// --- GEMV, w stored [N][K] ---------------------------------------------------
// 16 output columns per workgroup (4 per wave). vec: K % 8 == 0 and 16-byte alignment.
template <int MR>
__global__ __launch_bounds__(256) void gemv_nk_kernel(const __half* __restrict__ a,
                                                      const __half* __restrict__ w,
                                                      __half* __restrict__ y, uint32_t K,
                                                      uint32_t N_full, uint32_t n0, uint32_t N,
                                                      uint32_t M) {
    extern __shared__ u32x4 xs[];   // [MR][K/8]
    const uint32_t bb = blockIdx.y;
    const __half* ab = a + (size_t)bb * M * K;
    const __half* wb = w + (size_t)bb * N_full * K;
    __half* yb = y + (size_t)bb * M * N_full;
    const uint32_t kc = K / 8;
    for (uint32_t i = threadIdx.x; i < MR * kc; i += 256)
        xs[i] = reinterpret_cast<const u32x4*>(ab)[(i / kc) * kc + (i % kc)];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t r = 0; r < 4; ++r) {
        const uint32_t n = blockIdx.x * 16 + wave * 4 + r;
        if (n >= N) break;
        const u32x4* wr = reinterpret_cast<const u32x4*>(wb + (size_t)(n0 + n) * K);
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
        for (uint32_t c = lane; c < kc; c += 64) {
            const u32x4 wv = __builtin_nontemporal_load(&wr[c]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const u32x4 xv = xs[m * kc + c];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[m] = __builtin_amdgcn_fdot2(as_h2(wv[e]),
                                                    as_h2(xv[e]), acc[m], false);
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float s = wave_sum(acc[m]);
            if (lane == 0) yb[(size_t)m * N_full + n0 + n] = __float2half(s);
        }
    }
}

// The same GEMV for M = 1 when each lane owns NC = K / 512 16-byte chunks of a row (the
// lm_head: K = 2560, NC = 5): the activation chunks are requested first, then every
// weight chunk of the wave's 4 rows, and only then x is staged in LDS and the rows are
// computed, so a wave waits on one memory round trip instead of one per row. Each lane
// accumulates chunks lane, lane + 64, ... in the order of gemv_nk_kernel and the row sum
// is the same wave reduction: the same bits.
template <int NC>
__global__ __launch_bounds__(256) void gemv_nk_pre_kernel(const __half* __restrict__ a,
                                                          const __half* __restrict__ w,
                                                          __half* __restrict__ y, uint32_t K,
                                                          uint32_t N_full, uint32_t n0, uint32_t N) {
    constexpr uint32_t kc = 64 * NC, XC = (kc + 255) / 256;
    extern __shared__ u32x4 xs[];   // [K/8]
    const uint32_t bb = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32x4* ab = reinterpret_cast<const u32x4*>(a + (size_t)bb * K);
    const __half* wb = w + (size_t)bb * N_full * K;
    __half* yb = y + (size_t)bb * N_full;
    u32x4 xr[XC];
#pragma unroll
    for (uint32_t i = 0; i < XC; ++i) xr[i] = ab[min(tid + 256 * i, kc - 1)];
    const uint32_t nb = blockIdx.x * 16 + wave * 4;
    u32x4 wv[4][NC];
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
        const u32x4* wr = reinterpret_cast<const u32x4*>(wb + (size_t)(n0 + min(nb + r, N - 1)) * K);
#pragma unroll
        for (int j = 0; j < NC; ++j) wv[r][j] = __builtin_nontemporal_load(&wr[lane + 64 * j]);
    }
#pragma unroll
    for (uint32_t i = 0; i < XC; ++i)
        if (tid + 256 * i < kc) xs[tid + 256 * i] = xr[i];
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const u32x4 xv = xs[lane + 64 * j];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_fdot2(as_h2(wv[r][j][e]), as_h2(xv[e]), acc, false);
        }
        const float sum = wave_sum(acc);
        if (lane == 0 && nb + r < N) yb[n0 + nb + r] = __float2half(sum);
    }
}

// --- GEMV, w stored [K][N_full] --------------------------------------------------
__global__ __launch_bounds__(256) void gemv_kn_kernel(const __half* __restrict__ a,
                                                      const __half* __restrict__ w,
                                                      __half* __restrict__ y, uint32_t M,
                                                      uint32_t K, uint32_t N_full, uint32_t n0,
                                                      uint32_t N, int t0) {
    const uint32_t bb = blockIdx.y;
    const uint32_t n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const __half* ab = a + (size_t)bb * M * K;
    const __half* wb = w + (size_t)bb * K * N_full;
    __half* yb = y + (size_t)bb * M * N_full;
    for (uint32_t m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (uint32_t k = 0; k < K; ++k) {
            const float av = __half2float(ab[t0 ? (size_t)k * M + m : (size_t)m * K + k]);
            acc = fmaf(av, __half2float(wb[(size_t)k * N_full + n0 + n]), acc);
        }
        yb[(size_t)m * N_full + n0 + n] = __float2half(acc);
    }
}

// --- general MFMA GEMM ------------------------------------------------------------
// 64x64 output tile per workgroup, BK = 32, 4 waves each owning one 32x32 MFMA tile.
constexpr int TM = 64, TN = 64, TK = 32, TS = TK + 8;

__global__ __launch_bounds__(256) void gemm_f16_kernel(const __half* __restrict__ a,
                                                       const __half* __restrict__ w,
                                                       __half* __restrict__ y, uint32_t M,
                                                       uint32_t K, uint32_t N_full, uint32_t n0,
                                                       uint32_t N, int t0, int t1, int batched) {
    __shared__ __align__(16) _Float16 As[TM * TS];
    __shared__ __align__(16) _Float16 Bs[TN * TS];
    const uint32_t bb = blockIdx.z;
    const __half* ab = a + (size_t)bb * M * K;
    const __half* wb = w + (size_t)bb * K * N_full;
    __half* yb = y + (size_t)bb * M * N_full;
    if (batched) t0 = 0;   // the reference's batched form ignores t0
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * TM, nt0 = blockIdx.x * TN;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    f16x_t acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    for (uint32_t kb = 0; kb < K; kb += TK) {
        // 64x32 elements per operand tile, 8 per thread.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t idx = tid + 256u * e;           // 0..2047
            uint32_t r, k;
            if (t0) { k = idx / TM; r = idx % TM; } else { r = idx / TK; k = idx % TK; }
            const uint32_t gm = m0 + r, gk = kb + k;
            _Float16 v = (_Float16)0.0f;
            if (gm < M && gk < K)
                v = __builtin_bit_cast(_Float16, ab[t0 ? (size_t)gk * M + gm : (size_t)gm * K + gk]);
            As[r * TS + k] = v;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t idx = tid + 256u * e;
            uint32_t c, k;
            if (t1) { c = idx / TK; k = idx % TK; } else { k = idx / TN; c = idx % TN; }
            const uint32_t gn = nt0 + c, gk = kb + k;
            _Float16 v = (_Float16)0.0f;
            if (gn < N && gk < K)
                v = __builtin_bit_cast(_Float16,
                                       wb[t1 ? (size_t)(n0 + gn) * K + gk : (size_t)gk * N_full + n0 + gn]);
            Bs[c * TS + k] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK / 16; ++kk) {
            const uint32_t kof = kk * 16 + 8 * (lane >> 5);
            const h8_t af = *reinterpret_cast<const h8_t*>(&As[(wm * 32 + (lane & 31)) * TS + kof]);
            const h8_t bf = *reinterpret_cast<const h8_t*>(&Bs[(wn * 32 + (lane & 31)) * TS + kof]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    const uint32_t col = nt0 + wn * 32 + (lane & 31);
    if (col < N) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row < M) yb[(size_t)row * N_full + n0 + col] = __float2half(acc[r]);
        }
    }
}

}  // namespace

hipError_t launch_matmul_f16(const __half* a, const __half* w, __half* y, uint32_t M, uint32_t K,
                             uint32_t N_full, uint32_t n0, uint32_t N, bool t0, bool t1,
                             uint32_t Bn, hipStream_t st) {
    if (!M || !N || !Bn) return hipSuccess;
    const bool batched = Bn > 1;
    const bool aligned = ((uintptr_t)a % 16 == 0) && ((uintptr_t)w % 16 == 0) && K % 8 == 0;
    if (M <= 4 && t1 && !t0 && aligned && (size_t)M * K * 2 <= 65536) {
        const size_t lds = (size_t)M * K * 2;
        dim3 grid((N + 15) / 16, Bn);
        if (M == 1 && K % 512 == 0 && K / 512 <= 8) {
            switch (K / 512) {
            case 1: hipLaunchKernelGGL(gemv_nk_pre_kernel<1>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 2: hipLaunchKernelGGL(gemv_nk_pre_kernel<2>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 3: hipLaunchKernelGGL(gemv_nk_pre_kernel<3>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 4: hipLaunchKernelGGL(gemv_nk_pre_kernel<4>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 5: hipLaunchKernelGGL(gemv_nk_pre_kernel<5>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 6: hipLaunchKernelGGL(gemv_nk_pre_kernel<6>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            case 7: hipLaunchKernelGGL(gemv_nk_pre_kernel<7>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            default: hipLaunchKernelGGL(gemv_nk_pre_kernel<8>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N); break;
            }
            return hipGetLastError();
        }
        switch (M) {
        case 1: hipLaunchKernelGGL(gemv_nk_kernel<1>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N, M); break;
        case 2: hipLaunchKernelGGL(gemv_nk_kernel<2>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N, M); break;
        case 3: hipLaunchKernelGGL(gemv_nk_kernel<3>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N, M); break;
        default: hipLaunchKernelGGL(gemv_nk_kernel<4>, grid, dim3(256), lds, st, a, w, y, K, N_full, n0, N, M); break;
        }
        return hipGetLastError();
    }
    if (M <= 4 && !t1) {
        dim3 grid((N + 255) / 256, Bn);
        hipLaunchKernelGGL(gemv_kn_kernel, grid, dim3(256), 0, st, a, w, y, M, K, N_full, n0, N,
                           (int)(t0 && !batched));
        return hipGetLastError();
    }
    dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM, Bn);
    hipLaunchKernelGGL(gemm_f16_kernel, grid, dim3(256), 0, st, a, w, y, M, K, N_full, n0, N,
                       (int)t0, (int)t1, (int)batched);
    return hipGetLastError();
}

}  // namespace gehtp
