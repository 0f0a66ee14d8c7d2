// k_data.hip — crouton16_row4 surfaces, OP_MATMUL_W4A16 (opcode 1), OP_RMSNORM_F16
// (opcode 2) and the runlist's data-movement / reduction ops, for gfx950.
//
// crouton16_row4 (kernels/src/runtime/gemm_dispatch.c:38-72): element (r, c) of a
// rows x cols u16 surface sits at
//   chunk = ((phase * n_kt + kt) * n_m32 + g) * 2 + rp,   pos = 64 * chunk + 2 * (c % 32) + (r & 1)
// with g = r / 32, phase = (r % 32) / 4, rp = (r % 4) / 2, kt = c / 32.
#include "kernels.h"

namespace gehtp {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ size_t crouton_pos(uint32_t r, uint32_t c, uint32_t n_m32, uint32_t n_kt) {
    const uint32_t rr = r & 31u;
    const size_t chunk = ((size_t)((rr >> 2) * n_kt + (c >> 5)) * n_m32 + (r >> 5)) * 2 + ((rr >> 1) & 1u);
    return chunk * 64 + 2 * (c & 31u) + (r & 1u);
}

// One thread per surface pair (two rows of one column): surface words are written in
// order, the linear side reads two rows.
__global__ void crouton_encode_kernel(const uint16_t* __restrict__ lin, uint32_t* __restrict__ surf,
                                      uint32_t rows, uint32_t cols) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t n_m32 = rows >> 5, n_kt = cols >> 5;
    if (q >= (size_t)rows * cols / 2) return;
    const uint32_t ci = (uint32_t)(q & 31u);
    size_t rest = q >> 5;
    const uint32_t rp = (uint32_t)(rest & 1u);
    rest >>= 1;
    const uint32_t g = (uint32_t)(rest % n_m32);
    rest /= n_m32;
    const uint32_t kt = (uint32_t)(rest % n_kt), phase = (uint32_t)(rest / n_kt);
    const uint32_t row0 = g * 32 + phase * 4 + rp * 2, c = kt * 32 + ci;
    surf[q] = (uint32_t)lin[(size_t)row0 * cols + c] | ((uint32_t)lin[(size_t)(row0 + 1) * cols + c] << 16);
}

__global__ void crouton_decode_kernel(const uint32_t* __restrict__ surf, uint16_t* __restrict__ lin,
                                      uint32_t rows, uint32_t cols) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t n_m32 = rows >> 5, n_kt = cols >> 5;
    if (q >= (size_t)rows * cols / 2) return;
    const uint32_t ci = (uint32_t)(q & 31u);
    size_t rest = q >> 5;
    const uint32_t rp = (uint32_t)(rest & 1u);
    rest >>= 1;
    const uint32_t g = (uint32_t)(rest % n_m32);
    rest /= n_m32;
    const uint32_t kt = (uint32_t)(rest % n_kt), phase = (uint32_t)(rest / n_kt);
    const uint32_t row0 = g * 32 + phase * 4 + rp * 2, c = kt * 32 + ci;
    const uint32_t v = surf[q];
    lin[(size_t)row0 * cols + c] = (uint16_t)(v & 0xFFFFu);
    lin[(size_t)(row0 + 1) * cols + c] = (uint16_t)(v >> 16);
}

// ---------------------------------------------------------------------------
// OP_MATMUL_W4A16: Y[m,n] = clip(nearest((sum_k (A[m,k]-32768) W[k,n]) / 7) + 32768).
// Workgroup tile 64 (m) x 64 (n), K step 32. A comes straight from the crouton act
// surface: the (kt, g) 32x32 block is 16 contiguous 128-byte chunks (8 phases x 2 row
// pairs); A - 32768 as int16 is A ^ 0x8000. W rows ([N][K/2], +8 nibbles) unpack to
// int16 in LDS. Products accumulate with v_dot2_i32_i16 in int32 per K step (at most
// 32 * 2^15 * 8 = 2^23) and in int64 across steps. Results go to the crouton out surface.
constexpr int WA_BM = 64, WA_BN = 64, WA_BK = 32, WA_LD = WA_BK + 2;   // int16 row stride (pairs stay aligned)

__device__ __forceinline__ int64_t round_div7(int64_t s) { return s >= 0 ? (s + 3) / 7 : -((-s + 3) / 7); }

__global__ __launch_bounds__(256) void w4a16_gemm_kernel(const uint16_t* __restrict__ act,
                                                         const uint8_t* __restrict__ w,
                                                         uint16_t* __restrict__ out, uint32_t M,
                                                         uint32_t K, uint32_t N) {
    __shared__ __align__(16) int16_t As[WA_BM * WA_LD];
    __shared__ __align__(16) int16_t Ws[WA_BN * WA_LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t m0 = blockIdx.y * WA_BM, n0 = blockIdx.x * WA_BN;
    const uint32_t n_m32 = M >> 5, n_kt = K >> 5;
    const uint32_t tm = tid >> 4, tn = tid & 15;   // 4 x 4 outputs: rows tm*4.., cols tn*4..
    int64_t tot[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = 0;

    for (uint32_t kt = 0; kt < n_kt; ++kt) {
        // A: 2 row groups x 16 chunks x 8 pieces of 16 bytes = 256 pieces, one per thread.
        {
            const uint32_t gl = tid >> 7, u = tid & 127, ch = u >> 3, piece = u & 7;
            const uint32_t phase = ch >> 1, rp = ch & 1;
            const uint32_t g = (m0 >> 5) + gl;
            if (g < n_m32) {
                const size_t chunk = ((size_t)(phase * n_kt + kt) * n_m32 + g) * 2 + rp;
                const u32x4 v = *reinterpret_cast<const u32x4*>(act + chunk * 64 + piece * 8);
                const uint32_t r0 = gl * 32 + phase * 4 + rp * 2;   // local row of the pair
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t col = piece * 4 + e;
                    const uint32_t x = v[e] ^ 0x80008000u;
                    As[r0 * WA_LD + col] = (int16_t)(x & 0xFFFFu);
                    As[(r0 + 1) * WA_LD + col] = (int16_t)(x >> 16);
                }
            }
        }
        // W: 64 rows x 16 bytes (32 nibbles) of this K step.
        if (tid < WA_BN) {
            const uint32_t n = n0 + tid;
            u32x4 v = {0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};   // q = 0 past N
            if (n < N) v = *reinterpret_cast<const u32x4*>(w + (size_t)n * (K / 2) + kt * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    Ws[tid * WA_LD + e * 8 + b] = (int16_t)((int32_t)((v[e] >> (4 * b)) & 0xFu) - 8);
        }
        __syncthreads();
        int32_t acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = 0;
#pragma unroll
        for (int kk = 0; kk < WA_BK; kk += 2) {
            s2_t a2[4], w2[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a2[i] = *reinterpret_cast<const s2_t*>(&As[(tm * 4 + i) * WA_LD + kk]);
#pragma unroll
            for (int j = 0; j < 4; ++j) w2[j] = *reinterpret_cast<const s2_t*>(&Ws[(tn * 4 + j) * WA_LD + kk]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_sdot2(a2[i], w2[j], acc[i][j], false);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][j] += acc[i][j];
        __syncthreads();
    }
    const uint32_t on_m32 = M >> 5, on_kt = N >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t m = m0 + tm * 4 + i, n = n0 + tn * 4 + j;
            if (m >= M || n >= N) continue;
            int64_t v = round_div7(tot[i][j]) + 32768;
            v = v < 0 ? 0 : (v > 65535 ? 65535 : v);
            out[crouton_pos(m, n, on_m32, on_kt)] = (uint16_t)v;
        }
}

// OP_RMSNORM_F16 (oplist_exec.c:559-591), one wavefront per row of the crouton surface:
// x = float(u16 - 32768), squares summed in double, rms = (float)sqrt(acc/n + 1e-6),
// y = f16((x / rms) * w) row-major.
__global__ __launch_bounds__(256) void rmsnorm_crouton_kernel(const uint16_t* __restrict__ x,
                                                              const __half* __restrict__ wt,
                                                              __half* __restrict__ y, uint32_t m,
                                                              uint32_t n) {
    const uint32_t lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= m) return;
    const uint32_t n_m32 = m >> 5, n_kt = n >> 5;
    double acc = 0.0;
    for (uint32_t c = lane; c < n; c += 64) {
        const float xf = (float)((int32_t)x[crouton_pos(r, c, n_m32, n_kt)] - 32768);
        acc += (double)xf * (double)xf;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float rms = (float)sqrt(acc / (double)n + 1e-6);
    for (uint32_t c = lane; c < n; c += 64) {
        const float xf = (float)((int32_t)x[crouton_pos(r, c, n_m32, n_kt)] - 32768);
        y[(size_t)r * n + c] = __float2half(__fmul_rn(__fdiv_rn(xf, rms), __half2float(wt[c])));
    }
}

// ---------------------------------------------------------------------------
// Data movement (bit copies of f16 words) and reductions.
struct Seg4 {
    const uint16_t* x[4];
    uint32_t size[4];
};

__global__ void concat_kernel(Seg4 s, uint16_t* __restrict__ y, uint32_t n_seg, uint32_t total, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t o = i / total;
    uint32_t c = i - o * total;
    for (uint32_t k = 0; k < n_seg; ++k) {
        if (c < s.size[k]) { y[i] = s.x[k][(size_t)o * s.size[k] + c]; return; }
        c -= s.size[k];
    }
}

__global__ void split_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, uint32_t total,
                             uint32_t off, uint32_t size, uint32_t n) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const uint32_t o = j / size, c = j - o * size;
    y[j] = x[(size_t)o * total + off + c];
}

__global__ void pad_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, uint32_t outer,
                           uint32_t in_inner, uint32_t out_inner, uint32_t before, uint16_t pv) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)outer * out_inner) return;
    const uint32_t r = (uint32_t)(i / out_inner), c = (uint32_t)(i - (size_t)r * out_inner);
    y[i] = (c >= before && c < before + in_inner) ? x[(size_t)r * in_inner + (c - before)] : pv;
}

// OP_REDUCE_F16 (oplist_exec.c:1258-1299): thread per output, the reference's order.
__global__ void reduce_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t outer,
                              uint32_t L, uint32_t inner, uint32_t subtype) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= outer * inner) return;
    const uint32_t o = t / inner, i = t - o * inner;
    const __half* base = x + ((size_t)o * L) * inner + i;
    float acc = subtype == 2 ? -3.0e38f : subtype == 3 ? 3.0e38f : 0.0f;
    for (uint32_t l = 0; l < L; ++l) {
        const float v = __half2float(base[(size_t)l * inner]);
        if (subtype == 2) acc = v > acc ? v : acc;
        else if (subtype == 3) acc = v < acc ? v : acc;
        else acc = __fadd_rn(acc, v);
    }
    if (subtype == 1) acc = __fdiv_rn(acc, (float)L);
    y[(size_t)o * inner + i] = __float2half(acc);
}

// OP_CUMSUM_F32 (oplist_exec.c:1320-1347): thread per row, sequential f32 sum.
__global__ void cumsum_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t rows,
                              uint32_t n, uint32_t exclusive, uint32_t reverse) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float acc = 0.0f;
    for (uint32_t s = 0; s < n; ++s) {
        const size_t idx = (size_t)r * n + (reverse ? n - 1 - s : s);
        const float v = __half2float(x[idx]);
        y[idx] = __float2half(exclusive ? acc : __fadd_rn(acc, v));
        acc = __fadd_rn(acc, v);
    }
}

// OP_GATHER_F16 (oplist_exec.c:1378-1436), thread per output element.
struct GatherGeom {
    uint32_t axis, xrank, irank;
    uint32_t td[5], xd[5];
    uint64_t os[5], ts[5], xs[5];
};

__global__ void gather_kernel(const uint16_t* __restrict__ tbl, const int32_t* __restrict__ idx,
                              uint16_t* __restrict__ y, uint32_t n, GatherGeom G) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint64_t rem = i;
    uint32_t oc[5];
#pragma unroll
    for (int d = 0; d < 5; ++d) { oc[d] = (uint32_t)(rem / G.os[d]); rem %= G.os[d]; }
    uint64_t il = 0;
    for (uint32_t k = 0; k < G.xrank && k < 5; ++k) il += (uint64_t)(oc[G.axis + k] % G.xd[k]) * G.xs[k];
    int32_t r = idx[il];
    if (r < 0) r += (int32_t)G.td[G.axis];
    if (r < 0 || r >= (int32_t)G.td[G.axis]) { y[i] = 0; return; }
    uint64_t src = 0;
    for (uint32_t d = 0; d < G.axis && d < 5; ++d) src += (uint64_t)oc[d] * G.ts[d];
    src += (uint64_t)r * G.ts[G.axis];
    for (uint32_t d = G.axis + 1; d < G.irank && d < 5; ++d) {
        const uint32_t ocd = d + G.xrank - 1;
        src += (uint64_t)(ocd < 5 ? oc[ocd] : 0) * G.ts[d];
    }
    y[i] = tbl[src];
}

// OP_TRANSPOSE_F16 (oplist_exec.c:983-1011): (1, H, W, C) with perm[output axis] = input axis.
__global__ void transpose4_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, uint32_t Hh,
                                  uint32_t W, uint32_t Cc, uint32_t perm) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)Hh * W * Cc) return;
    const uint32_t dims[4] = {1, Hh, W, Cc};
    const uint32_t p[4] = {perm & 0xFF, (perm >> 8) & 0xFF, (perm >> 16) & 0xFF, (perm >> 24) & 0xFF};
    const uint64_t si[4] = {(uint64_t)Hh * W * Cc, (uint64_t)W * Cc, Cc, 1};
    uint64_t rem = i;
    uint32_t ic[4] = {0, 0, 0, 0};
    for (int ax = 3; ax >= 0; --ax) {
        const uint32_t d = dims[p[ax]];
        ic[p[ax]] = (uint32_t)(rem % d);
        rem /= d;
    }
    y[i] = x[ic[0] * si[0] + ic[1] * si[1] + ic[2] * si[2] + ic[3] * si[3]];
}

inline uint32_t nblk(size_t n, uint32_t bs) { return (uint32_t)((n + bs - 1) / bs); }

}  // namespace

hipError_t launch_crouton_encode(const uint16_t* lin, uint16_t* surf, uint32_t rows, uint32_t cols,
                                 hipStream_t st) {
    if (rows % 32 || cols % 32) return hipErrorInvalidValue;
    const size_t pairs = (size_t)rows * cols / 2;
    if (!pairs) return hipSuccess;
    hipLaunchKernelGGL(crouton_encode_kernel, dim3(nblk(pairs, 256)), dim3(256), 0, st, lin,
                       reinterpret_cast<uint32_t*>(surf), rows, cols);
    return hipGetLastError();
}

hipError_t launch_crouton_decode(const uint16_t* surf, uint16_t* lin, uint32_t rows, uint32_t cols,
                                 hipStream_t st) {
    if (rows % 32 || cols % 32) return hipErrorInvalidValue;
    const size_t pairs = (size_t)rows * cols / 2;
    if (!pairs) return hipSuccess;
    hipLaunchKernelGGL(crouton_decode_kernel, dim3(nblk(pairs, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t*>(surf), lin, rows, cols);
    return hipGetLastError();
}

hipError_t launch_matmul_w4a16(const uint16_t* act, const uint8_t* w, uint16_t* out, uint32_t M, uint32_t K,
                               uint32_t N, hipStream_t st) {
    if (M % 32 || K % 32 || N % 32) return hipErrorInvalidValue;
    if (!M || !N || !K) return hipSuccess;
    hipLaunchKernelGGL(w4a16_gemm_kernel, dim3((N + WA_BN - 1) / WA_BN, (M + WA_BM - 1) / WA_BM), dim3(256), 0, st,
                       act, w, out, M, K, N);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_crouton(const uint16_t* x, const __half* w, __half* y, uint32_t m, uint32_t n,
                                  hipStream_t st) {
    if (!m || m % 32 || n % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_crouton_kernel, dim3((m + 3) / 4), dim3(256), 0, st, x, w, y, m, n);
    return hipGetLastError();
}

hipError_t launch_concat(const uint16_t* const* xs, const uint32_t* sizes, uint32_t n_seg, uint16_t* y,
                         uint32_t n_elems, hipStream_t st) {
    Seg4 s{};
    uint32_t total = 0;
    for (uint32_t k = 0; k < n_seg && k < 4; ++k) {
        s.x[k] = xs[k];
        s.size[k] = sizes[k];
        total += sizes[k];
    }
    if (!total || n_elems % total) return hipErrorInvalidValue;
    if (!n_elems) return hipSuccess;
    hipLaunchKernelGGL(concat_kernel, dim3(nblk(n_elems, 256)), dim3(256), 0, st, s, y, n_seg < 4 ? n_seg : 4,
                       total, n_elems);
    return hipGetLastError();
}

hipError_t launch_split(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t total, uint32_t off,
                        uint32_t size, hipStream_t st) {
    const size_t n = (size_t)outer * size;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(split_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, x, y, total, off, size, (uint32_t)n);
    return hipGetLastError();
}

hipError_t launch_pad(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t in_inner, uint32_t out_inner,
                      uint32_t before, uint16_t pv, hipStream_t st) {
    const size_t n = (size_t)outer * out_inner;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(pad_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, x, y, outer, in_inner, out_inner,
                       before, pv);
    return hipGetLastError();
}

hipError_t launch_reduce(const __half* x, __half* y, uint32_t outer, uint32_t L, uint32_t inner,
                         uint32_t subtype, hipStream_t st) {
    const size_t n = (size_t)outer * inner;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(reduce_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, x, y, outer, L, inner, subtype);
    return hipGetLastError();
}

hipError_t launch_cumsum(const __half* x, __half* y, uint32_t rows, uint32_t n, uint32_t exclusive,
                         uint32_t reverse, hipStream_t st) {
    if (!rows) return hipSuccess;
    hipLaunchKernelGGL(cumsum_kernel, dim3(nblk(rows, 64)), dim3(64), 0, st, x, y, rows, n, exclusive, reverse);
    return hipGetLastError();
}

hipError_t launch_gather(const uint16_t* tbl, const int32_t* idx, uint16_t* y, uint32_t n, uint32_t axis,
                         uint32_t xrank, uint32_t irank, const uint32_t* td, const uint32_t* xd,
                         hipStream_t st) {
    if (axis >= irank || irank > 5 || xrank > 5 || xrank == 0) return hipErrorInvalidValue;
    GatherGeom G{};
    G.axis = axis;
    G.xrank = xrank;
    G.irank = irank;
    for (int d = 0; d < 5; ++d) { G.td[d] = td[d]; G.xd[d] = xd[d]; }
    uint32_t od[5] = {1, 1, 1, 1, 1};
    for (uint32_t d = 0; d < axis && d < 5; ++d) od[d] = td[d];
    for (uint32_t k = 0; k < xrank && axis + k < 5; ++k) od[axis + k] = xd[k];
    for (uint32_t d = axis + 1; d < irank && d < 5; ++d)
        if (d + xrank - 1 < 5) od[d + xrank - 1] = td[d];
    for (int d = 0; d < 5; ++d) { G.os[d] = 1; G.ts[d] = 1; G.xs[d] = 1; }
    for (int d = 3; d >= 0; --d) {
        G.os[d] = G.os[d + 1] * od[d + 1];
        G.ts[d] = G.ts[d + 1] * td[d + 1];
        G.xs[d] = G.xs[d + 1] * xd[d + 1];
    }
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, tbl, idx, y, n, G);
    return hipGetLastError();
}

hipError_t launch_transpose4(const uint16_t* x, uint16_t* y, uint32_t Hh, uint32_t W, uint32_t Cc,
                             uint32_t perm, hipStream_t st) {
    for (int s = 0; s < 32; s += 8)
        if (((perm >> s) & 0xFF) > 3) return hipErrorInvalidValue;
    const size_t n = (size_t)Hh * W * Cc;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(transpose4_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, x, y, Hh, W, Cc, perm);
    return hipGetLastError();
}

}  // namespace gehtp
