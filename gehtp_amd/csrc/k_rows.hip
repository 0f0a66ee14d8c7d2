// k_rows.hip — row-wise and element-wise runlist ops for gfx950.
//
// Arithmetic that the reference rounds through f16 at op boundaries is done here
// with explicitly rounded operations (__fmul_rn / __fadd_rn / __fdiv_rn) so no
// FMA contraction changes a result the reference's scalar path defines exactly.
#include "kernels.h"
#include "dev_rope.h"

#include <algorithm>
#include <cmath>

namespace gehtp {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }
__device__ __forceinline__ __half f2h(float f) { return __float2half(f); }   // RNE

// Wave-wide reductions over DPP (dev_reduce.h); every lane gets the result.
__device__ __forceinline__ float wave_sum_f(float v) { return dev::wave_sum(v); }
__device__ __forceinline__ double wave_sum_d(double v) { return dev::wave_sum(v); }
__device__ __forceinline__ float wave_max_f(float v) { return dev::wave_max(v); }

using dev::f64_to_f16_bits;

// ---------------------------------------------------------------------------
// RMSNorm, one wavefront per row (reference exec_rmsnorm2, oplist_exec.c:1859-1871):
// squares summed in double (each f32 square is exact in double), rms =
// (float)sqrt(mean + 1e-6) in double, then f16(x / rms * g + b) with each step rounded.
__global__ __launch_bounds__(256) void rmsnorm2_kernel(const __half* __restrict__ x,
                                                       const __half* __restrict__ g,
                                                       const __half* __restrict__ b,
                                                       __half* __restrict__ y, uint32_t rows,
                                                       uint32_t rw) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const __half* xr = x + (size_t)row * rw;
    __half* yr = y + (size_t)row * rw;
    double acc = 0.0;
    const bool vec = (rw % 8 == 0);
    if (vec) {
        for (uint32_t i = lane * 8; i < rw; i += 512) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(xr + i);
            const __half* hv = reinterpret_cast<const __half*>(&v);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double f = (double)h2f(hv[e]);
                acc += f * f;
            }
        }
    } else {
        for (uint32_t i = lane; i < rw; i += 64) {
            const double f = (double)h2f(xr[i]);
            acc += f * f;
        }
    }
    acc = wave_sum_d(acc);
    const float rms = (float)sqrt(acc / (double)rw + 1e-6);
    const float rcp = __fdiv_rn(1.0f, rms);   // x / rms via dev::div_markstein (exact)
    const bool vec_out = vec && ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(b) |
                                  reinterpret_cast<uintptr_t>(yr)) & 15u) == 0;
    if (vec_out) {
        for (uint32_t i = lane * 8; i < rw; i += 512) {
            const u32x4 xv = *reinterpret_cast<const u32x4*>(xr + i);
            const u32x4 gv = *reinterpret_cast<const u32x4*>(g + i);
            const u32x4 bv = b ? *reinterpret_cast<const u32x4*>(b + i) : u32x4{0u, 0u, 0u, 0u};
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const uint32_t sh = 16 * hh;
                    const float xf = dev::bits_f((uint16_t)(xv[e] >> sh));
                    const float q = dev::div_markstein(xf, rms, rcp);
                    v[hh] = __fadd_rn(__fmul_rn(q, dev::bits_f((uint16_t)(gv[e] >> sh))),
                                      dev::bits_f((uint16_t)(bv[e] >> sh)));
                }
                o[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[0]) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[1]) << 16);
            }
            *reinterpret_cast<u32x4*>(yr + i) = o;
        }
    } else {
        for (uint32_t i = lane; i < rw; i += 64) {
            float v = dev::div_markstein(h2f(xr[i]), rms, rcp);
            v = __fadd_rn(__fmul_rn(v, h2f(g[i])), b ? h2f(b[i]) : 0.0f);
            yr[i] = f2h(v);
        }
    }
}

// Same arithmetic with the whole row in registers: lane l owns the 16-byte chunks
// l, l+64, ..., l+64(C-1) of x, gamma and bias, all loaded before any arithmetic
// (chunk indices past the row are clamped to its last chunk and not used), so a row
// costs one memory round trip instead of one per loop trip. Needs rw % 8 == 0,
// rw <= 512*C and 16-byte aligned x, gamma, bias and y.
template <int C, bool HAS_B>
__global__ __launch_bounds__(256) void rmsnorm2_reg_kernel(const __half* __restrict__ x,
                                                           const __half* __restrict__ g,
                                                           const __half* __restrict__ b,
                                                           __half* __restrict__ y, uint32_t rows,
                                                           uint32_t rw) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t nch = rw / 8;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + (size_t)row * rw);
    const u32x4* g4 = reinterpret_cast<const u32x4*>(g);
    const u32x4* b4 = reinterpret_cast<const u32x4*>(b);
    u32x4 xv[C], gv[C], bv[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const uint32_t i = min(lane + 64u * j, nch - 1);
        xv[j] = xr[i];
        gv[j] = g4[i];
        bv[j] = HAS_B ? b4[i] : u32x4{0u, 0u, 0u, 0u};
    }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const bool valid = lane + 64u * j < nch;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const double f = valid ? (double)dev::bits_f((uint16_t)(xv[j][e / 2] >> (16 * (e & 1)))) : 0.0;
            acc += f * f;
        }
    }
    acc = wave_sum_d(acc);
    const float rms = (float)sqrt(acc / (double)rw + 1e-6);
    const float rcp = __fdiv_rn(1.0f, rms);   // x / rms via dev::div_markstein (exact)
    u32x4* yr = reinterpret_cast<u32x4*>(y + (size_t)row * rw);
#pragma unroll
    for (int j = 0; j < C; ++j) {
        if (lane + 64u * j >= nch) continue;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint32_t sh = 16 * hh;
                const float q = dev::div_markstein(dev::bits_f((uint16_t)(xv[j][e] >> sh)), rms, rcp);
                v[hh] = __fadd_rn(__fmul_rn(q, dev::bits_f((uint16_t)(gv[j][e] >> sh))),
                                  dev::bits_f((uint16_t)(bv[j][e] >> sh)));
            }
            o[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[0]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[1]) << 16);
        }
        yr[lane + 64u * j] = o;
    }
}

// ---------------------------------------------------------------------------
// Softmax, one workgroup per row, following exec_softmax's two forms
// (oplist_exec.c:1163-1194 and kernels/src/hvx/hvx_softmax.c:81-93).
__global__ __launch_bounds__(256) void softmax_kernel(const __half* __restrict__ x,
                                                      __half* __restrict__ y, uint32_t n,
                                                      int vector_form) {
    __shared__ float red_f[4];
    __shared__ double red_d[4];
    const uint32_t row = blockIdx.x;
    const __half* xr = x + (size_t)row * n;
    __half* yr = y + (size_t)row * n;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    float mx = -INFINITY;
    for (uint32_t i = tid; i < n; i += 256) mx = fmaxf(mx, h2f(xr[i]));
    mx = wave_max_f(mx);
    if (lane == 0) red_f[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    __syncthreads();

    if (vector_form) {
        double s = 0.0;
        for (uint32_t i = tid; i < n; i += 256) s += (double)expf(__fsub_rn(h2f(xr[i]), mx));
        s = wave_sum_d(s);
        if (lane == 0) red_d[wave] = s;
        __syncthreads();
        const double sum = red_d[0] + red_d[1] + red_d[2] + red_d[3];
        const float inv = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
        for (uint32_t i = tid; i < n; i += 256)
            yr[i] = f2h(__fmul_rn(expf(__fsub_rn(h2f(xr[i]), mx)), inv));
    } else {
        float s = 0.0f;
        for (uint32_t i = tid; i < n; i += 256) s += expf(__fsub_rn(h2f(xr[i]), mx));
        s = wave_sum_f(s);
        if (lane == 0) red_f[wave] = s;
        __syncthreads();
        const float sum = red_f[0] + red_f[1] + red_f[2] + red_f[3];
        for (uint32_t i = tid; i < n; i += 256) {
            const __half e = f2h(expf(__fsub_rn(h2f(xr[i]), mx)));
            yr[i] = f2h(__fdiv_rn(h2f(e), sum));
        }
    }
}

// ---------------------------------------------------------------------------
// f16 store of the element-wise ops: RNE, with a NaN stored as the Inf of its sign, as
// the reference's converters do (oplist_exec.c:401, hvx_binary.c hb_f32_to_f16).
__device__ __forceinline__ __half f2h_ew(float f) {
    return f != f ? __ushort_as_half((uint16_t)((__float_as_uint(f) >> 16 & 0x8000u) | 0x7C00u)) : f2h(f);
}

// Element-wise binary ops, subtypes 0..5 (oplist_exec.c:1143-1158). exec_binary's
// dispatch: for n >= 32 the division runs hvhx_v2_div_f32, which has no zero test
// (hvx_binary.c:66-86, oplist_exec.c:1126-1145); below 32 elements x / 0 gives 0.
__global__ void binary_kernel(const __half* __restrict__ a, const __half* __restrict__ b,
                              __half* __restrict__ y, uint32_t n, uint32_t subtype) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x0 = h2f(a[i]), x1 = h2f(b[i]);
    float r = x0;
    switch (subtype) {
    case 0: r = __fadd_rn(x0, x1); break;
    case 1: r = __fsub_rn(x0, x1); break;
    case 2: r = __fmul_rn(x0, x1); break;
    case 3: r = (n >= 32u || x1 != 0.0f) ? __fdiv_rn(x0, x1) : 0.0f; break;
    case 4: r = (x0 == x1) ? 1.0f : 0.0f; break;
    case 5: r = ((uint32_t)x0 & (uint32_t)x1) ? 1.0f : 0.0f; break;
    default: break;
    }
    y[i] = f2h_ew(r);
}

__global__ void select_kernel(const __half* __restrict__ c, uint32_t cn, const __half* __restrict__ t,
                              uint32_t tn, const __half* __restrict__ f, uint32_t fn,
                              __half* __restrict__ y, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float cv = h2f(c[cn <= 1 ? 0 : (cn < n ? i % cn : i)]);
    const float r = cv != 0.0f ? h2f(t[tn <= 1 ? 0 : (tn < n ? i % tn : i)])
                               : h2f(f[fn <= 1 ? 0 : (fn < n ? i % fn : i)]);
    y[i] = f2h_ew(r);
}

// Element-wise unary ops, subtypes 0..16 (oplist_exec.c:1047-1078); COPY (14) over 32
// or more elements is a bit copy, as exec_unary's memcpy (oplist_exec.c:1042-1044).
__global__ void unary_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t n,
                             uint32_t subtype) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (subtype == 14u && n >= 32u) {
        y[i] = x[i];
        return;
    }
    const float v = h2f(x[i]);
    float r = v;
    switch (subtype) {
    case 0: r = -v; break;
    case 1: r = expf(v); break;
    case 2: r = v >= 0.0f ? __fsqrt_rn(v) : 0.0f; break;
    case 3: r = v > 0.0f ? __fdiv_rn(1.0f, __fsqrt_rn(v)) : 0.0f; break;
    case 4: r = v > 0.0f ? logf(v) : 0.0f; break;
    case 5: r = fabsf(v); break;
    case 6: r = sinf(v); break;
    case 7: r = cosf(v); break;
    case 8: r = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v))); break;
    case 9: r = tanhf(v); break;
    case 10: {
        const float v3 = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, v), v), v);
        const float t = tanhf(__fmul_rn(0.7978845608f, __fadd_rn(v, v3)));
        r = __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, t));
        break;
    }
    case 11: r = fmaxf(0.0f, v); break;
    case 12: r = __fdiv_rn(v, __fadd_rn(1.0f, expf(-v))); break;
    case 13: r = v > 30.0f ? v : (v < -30.0f ? expf(v) : log1pf(expf(v))); break;
    case 14: r = v; break;
    case 15: r = (v != v) ? 1.0f : 0.0f; break;
    case 16: r = (v == v && (v > 3.4e38f || v < -3.4e38f)) ? 1.0f : 0.0f; break;
    default: break;
    }
    y[i] = f2h_ew(r);
}

// ---------------------------------------------------------------------------
// Argmax: first index of the strict maximum above -1e30 (oplist_exec.c:1990-2004).
// Pass 1: each workgroup reduces its part to (value, first index) and folds it into one
// device-wide 64-bit key with atomicMax: the high word orders the value (-0 folded to
// +0, so equal values tie), the low word is ~index, so the larger key is the larger
// value and, among equal values, the smaller index. Pass 2 writes the index (0 when no
// value exceeds -1e30) and clears the key for the next call; the kernel boundary
// between the passes makes every atomic visible. Calls on one device must not overlap.
__device__ unsigned long long g_argmax_key;   // 0 between calls

__device__ __forceinline__ unsigned long long argmax_pack(float v, int32_t i) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (uint32_t)~(uint32_t)i;
}

constexpr uint32_t kArgmaxChunks = 4;   // 16-byte chunks per thread in pass 1

__global__ __launch_bounds__(256) void argmax_part_kernel(const __half* __restrict__ x, uint32_t n,
                                                          uint32_t n8) {
    __shared__ float sv[4];
    __shared__ int32_t si[4];
    float bv = -1e30f;
    int32_t bi = 0;
    const uint32_t tid = threadIdx.x;
    // This thread's chunks c = blockIdx.x*1024 + 256u + tid (u = 0..3), all loads first
    // (indices past the end clamped and not used), scanned in increasing index order.
    if (n8) {
        const u32x4* xv = reinterpret_cast<const u32x4*>(x);
        const uint32_t c0 = blockIdx.x * (256 * kArgmaxChunks) + tid;
        u32x4 v[kArgmaxChunks];
#pragma unroll
        for (uint32_t u = 0; u < kArgmaxChunks; ++u) v[u] = xv[min(c0 + 256 * u, n8 - 1)];
#pragma unroll
        for (uint32_t u = 0; u < kArgmaxChunks; ++u) {
            if (c0 + 256 * u >= n8) break;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = h2f(__ushort_as_half((uint16_t)(v[u][e / 2] >> (16 * (e & 1)))));
                if (f > bv) { bv = f; bi = (int32_t)((c0 + 256 * u) * 8 + e); }
            }
        }
    }
    // Elements past the 16-byte chunks (all of them when x is not 16-byte aligned).
    for (uint32_t j = n8 * 8 + blockIdx.x * 256 + tid; j < n; j += gridDim.x * 256) {
        const float f = h2f(x[j]);
        if (f > bv) { bv = f; bi = (int32_t)j; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int32_t oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    const uint32_t wave = tid >> 6;
    if ((tid & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
        if (bv > -1e30f) atomicMax(&g_argmax_key, argmax_pack(bv, bi));
    }
}

__global__ void argmax_final_kernel(int32_t* __restrict__ out) {
    const unsigned long long k = g_argmax_key;
    out[0] = k ? (int32_t)~(uint32_t)k : 0;
    g_argmax_key = 0ull;
}

__global__ void copy_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (((uintptr_t)dst | (uintptr_t)src | n) % 16 == 0) {
        for (; i < n / 16; i += stride)
            reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(src)[i];
    } else {
        for (; i < n; i += stride) dst[i] = src[i];
    }
}

__global__ void fill_zero_kernel(uint8_t* __restrict__ dst, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (((uintptr_t)dst | n) % 16 == 0) {
        for (; i < n / 16; i += stride) reinterpret_cast<u32x4*>(dst)[i] = u32x4{0, 0, 0, 0};
    } else {
        for (; i < n; i += stride) dst[i] = 0;
    }
}

// numpy broadcast with the reference's rank rules (oplist_exec.c:1876-1907).
struct Dims4 { uint32_t v[4]; };
__global__ void broadcast_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t n,
                                 Dims4 in_d, Dims4 ostr, Dims4 istr, uint32_t r, uint32_t lead) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t rem = i, in_lin = 0;
    for (uint32_t d = 0; d < r; ++d) {
        const uint32_t c = rem / ostr.v[d];
        rem -= c * ostr.v[d];
        if (d < lead) continue;
        const uint32_t idim = in_d.v[d - lead];
        if (idim > 1) in_lin += (c % idim) * istr.v[d - lead];
    }
    y[i] = x[in_lin];
}

// General C-order transpose, rank 2..4 (oplist_exec.c:1910-1948): input linear t
// maps to output offset sum_ax ic[perm[ax]] * so[ax].
__global__ void transpose_gen_kernel(const __half* __restrict__ x, __half* __restrict__ y,
                                     uint32_t n, uint32_t rk, Dims4 si, Dims4 so, Dims4 perm) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    uint32_t rem = t, ic[4] = {0, 0, 0, 0};
    for (uint32_t i = 0; i < rk; ++i) { ic[i] = rem / si.v[i]; rem -= ic[i] * si.v[i]; }
    uint32_t ot = 0;
    for (uint32_t ax = 0; ax < rk; ++ax) ot += ic[perm.v[ax]] * so.v[ax];
    y[ot] = x[t];
}

// Strided slice, rank <= 3 (oplist_exec.c:1950-1988).
__global__ void slice_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t n_out,
                             uint32_t rk, Dims4 bb, Dims4 ss, Dims4 istr, Dims4 ostr) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_out) return;
    uint32_t rem = i, in_lin = 0;
    for (uint32_t ax = 0; ax < rk; ++ax) {
        const uint32_t c = rem / ostr.v[ax];
        rem -= c * ostr.v[ax];
        in_lin += (bb.v[ax] + c * ss.v[ax]) * istr.v[ax];
    }
    y[i] = x[in_lin];
}

// RoPE, half split: for pair (i, i+hd/2) of each head,
//   y_i = f16(f16(x_i c) + f16(-x_{i+h} s)),  y_{i+h} = f16(f16(x_{i+h} c) + f16(x_i s)),
// with c, s = f16(cos/sin(pos * theta^(-2i/hd))) computed in double, as the
// reference's mul/neg/concat/add chain with f16 tables does.
__global__ void rope_kernel(const __half* __restrict__ x, __half* __restrict__ y, uint32_t n_tok,
                            uint32_t n_heads, uint32_t hd, uint32_t pos0,
                            const uint32_t* __restrict__ pos_dev, float theta, uint32_t row_stride) {
    const uint32_t half = hd / 2;
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;   // (t, i)
    if (idx >= n_tok * half) return;
    const uint32_t t = idx / half, i = idx - t * half;
    const uint32_t base = pos_dev ? *pos_dev + pos0 : pos0;
    const double pos = (double)(base + t);
    const double inv = 1.0 / pow((double)theta, (double)(2 * i) / (double)hd);
    const float c = __half2float(__ushort_as_half(f64_to_f16_bits(cos(pos * inv))));
    const float s = __half2float(__ushort_as_half(f64_to_f16_bits(sin(pos * inv))));
    for (uint32_t h = 0; h < n_heads; ++h) {
        const size_t o = (size_t)t * row_stride + (size_t)h * hd;
        const float x1 = h2f(x[o + i]), x2 = h2f(x[o + i + half]);
        const float a1 = h2f(f2h(__fmul_rn(x1, c))), b1 = h2f(f2h(__fmul_rn(-x2, s)));
        const float a2 = h2f(f2h(__fmul_rn(x2, c))), b2 = h2f(f2h(__fmul_rn(x1, s)));
        y[o + i] = f2h(__fadd_rn(a1, b1));
        y[o + i + half] = f2h(__fadd_rn(a2, b2));
    }
}

// ---------------------------------------------------------------------------
// KV ring append of n_tok tokens: workgroup t copies token t. The base position is
// read by every workgroup before the last one to finish advances the device counter:
// the counter is advanced by a separate single-thread kernel launched afterwards.
__global__ __launch_bounds__(256) void kv_append_kernel(uint8_t* __restrict__ ring,
                                                        uint32_t slot_bytes, uint32_t nslots,
                                                        const __half* __restrict__ k,
                                                        const __half* __restrict__ v,
                                                        uint32_t kv_elems, uint32_t pos,
                                                        const uint32_t* __restrict__ count) {
    const uint32_t t = blockIdx.x;
    const uint32_t base = (pos == 0xFFFFFFFFu) ? *count : pos;
    const uint32_t slot = (base + t) % nslots;
    __half* kf = reinterpret_cast<__half*>(ring + (size_t)slot * slot_bytes);
    __half* vf = kf + kv_elems;
    const __half* ks = k + (size_t)t * kv_elems;
    const __half* vs = v + (size_t)t * kv_elems;
    for (uint32_t i = threadIdx.x; i < kv_elems; i += 256) {
        kf[i] = ks[i];
        vf[i] = vs[i];
    }
}

__global__ void counter_add_kernel(uint32_t* count, uint32_t n) { *count += n; }

// Fused per-token QK-norm + RoPE + KV append (OP_QK_ROPE_KV_F16). Workgroup t handles
// token t of a [q | k | v] row; each wavefront takes whole 128-dim heads, lane l owning
// the RoPE pair (l, l+64). Arithmetic = RMSNORM2_F16 (rw 128, zero bias) then the RoPE
// chain of rope_kernel, so results equal the separate ops bit for bit.
struct QkRopeKvArgs {
    const __half* qkv;
    uint32_t ld, H, KVH;
    const __half* qg;
    const __half* kg;
    float theta;
    __half* q_out;
    __half* k_out;
    __half* v_out;
    uint8_t* ring;
    uint32_t slot_bytes, nslots;
    uint32_t* count;
    int advance;    // single-workgroup launch: advance the counter in-kernel
    uint32_t* done;      // rows kernel: workgroups-finished counter (zero between launches);
                         // the last workgroup to finish advances *count (all have read it)
};

// One workgroup per token: wave 0 computes the token's RoPE table (64 frequency pairs,
// evaluated in double) into LDS once; each wave then loads the inputs of all its heads
// (heads wave, wave+4, ...; loads unconditional with clamped head indices so they are
// all in flight together) before normalizing and rotating them one by one.
constexpr uint32_t kQkMaxHeadsPerWave = 16;   // H + KVH <= 64

__global__ __launch_bounds__(256) void qk_rope_kv_kernel(QkRopeKvArgs A) {
    constexpr uint32_t HD = 128;
    __shared__ uint32_t s_pos;
    __shared__ float s_c[64], s_s[64];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) s_pos = *A.count;
    __syncthreads();
    const uint32_t pos = s_pos + t;
    if (wave == 0) {
        float c, s;
        dev::rope_cs(pos, lane, A.theta, c, s);
        s_c[lane] = c;
        s_s[lane] = s;
    }
    const uint32_t slot = pos % A.nslots;
    const __half* row = A.qkv + (size_t)t * A.ld;
    __half* kface = reinterpret_cast<__half*>(A.ring + (size_t)slot * A.slot_bytes);
    __half* vface = kface + A.KVH * HD;
    const uint32_t nh = A.H + A.KVH;
    float x1[kQkMaxHeadsPerWave], x2[kQkMaxHeadsPerWave];
#pragma unroll
    for (uint32_t j = 0; j < kQkMaxHeadsPerWave; ++j) {
        const uint32_t r = min(wave + 4 * j, nh - 1);   // k heads follow the q heads
        x1[j] = h2f(row[(size_t)r * HD + lane]);
        x2[j] = h2f(row[(size_t)r * HD + lane + 64]);
    }
    const float qg1 = h2f(A.qg[lane]), qg2 = h2f(A.qg[lane + 64]);
    const float kg1 = h2f(A.kg[lane]), kg2 = h2f(A.kg[lane + 64]);
    __syncthreads();
    const float c = s_c[lane], s = s_s[lane];
#pragma unroll
    for (uint32_t j = 0; j < kQkMaxHeadsPerWave; ++j) {
        const uint32_t r = wave + 4 * j;
        if (r >= nh) break;   // wave-uniform
        const bool is_q = r < A.H;
        float y1f, y2f;
        dev::head_norm_rope(x1[j], x2[j], is_q ? qg1 : kg1, is_q ? qg2 : kg2, c, s, y1f, y2f);
        const __half y1 = f2h(y1f), y2 = f2h(y2f);
        if (is_q) {
            __half* qo = A.q_out + (size_t)t * A.H * HD + (size_t)r * HD;
            qo[lane] = y1;
            qo[lane + 64] = y2;
        } else {
            const uint32_t kh = r - A.H;
            kface[kh * HD + lane] = y1;
            kface[kh * HD + lane + 64] = y2;
            if (A.k_out) {
                __half* ko = A.k_out + (size_t)t * A.KVH * HD + (size_t)kh * HD;
                ko[lane] = y1;
                ko[lane + 64] = y2;
            }
        }
    }
    const __half* v = row + (size_t)nh * HD;
    for (uint32_t i = tid; i < A.KVH * HD; i += 256) {
        vface[i] = v[i];
        if (A.v_out) A.v_out[(size_t)t * A.KVH * HD + i] = v[i];
    }
    if (A.advance) {
        __syncthreads();
        if (tid == 0) *A.count = s_pos + 1;
    }
}

// Prefill form of qk_rope_kv_kernel: TOK tokens per workgroup, one 128-dim head row per
// 8-lane group, lane g owning elements [8g, 8g+8) and [64+8g, 64+8g+8) — both halves of
// its RoPE pairs, so the rotation needs no lane exchange. The per-head work (sum of
// squares reduced over 8 lanes instead of 64, the rms and its reciprocal) is shared by
// 8 heads per instruction. The token's RoPE table (64 cos / sin pairs, evaluated in
// double) is built in LDS by one thread per entry while the head rows are in flight.
// RoPE runs on packed f16 operations: each product and sum of two f16 values rounded
// once to f16 equals the f32 operation rounded to f16 (24 >= 2*11 + 1 bits, so the
// double rounding is innocuous), the arithmetic of rope_kernel. Pointers, row stride and
// ring slot size must be 16-byte aligned; the counter is not advanced here.
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2v u2h2(uint32_t w) { return __builtin_bit_cast(h2v, w); }
__device__ __forceinline__ uint32_t h22u(h2v v) { return __builtin_bit_cast(uint32_t, v); }

template <uint32_t TOK>
__global__ __launch_bounds__(256) void qk_rope_kv_rows_kernel(QkRopeKvArgs A, uint32_t n_tok) {
    constexpr uint32_t HD = 128, IT = TOK * 64 / 32;   // head rows per lane group, at most
    __shared__ uint32_t s_pos;
    __shared__ __align__(16) _Float16 s_cos[TOK][64], s_sin[TOK][64];
    const uint32_t tid = threadIdx.x, t0 = blockIdx.x * TOK;
    const uint32_t nt = min(TOK, n_tok - t0), nh = A.H + A.KVH, nrows = nt * nh;
    const uint32_t grp = tid >> 3, g = tid & 7;
    if (tid == 0) s_pos = *A.count;
    // Head rows grp, grp + 32, ...; loads of rows past the workgroup's are skipped by a
    // workgroup-uniform test, the last group of a partial pass loads a clamped row.
    u32x4 xl[IT], xh[IT];
#pragma unroll
    for (uint32_t it = 0; it < IT; ++it) {
        if (32 * it >= nrows) break;
        const uint32_t hr = min(grp + 32 * it, nrows - 1), tk = hr / nh, r = hr - tk * nh;
        const __half* row = A.qkv + (size_t)(t0 + tk) * A.ld + (size_t)r * HD;
        xl[it] = *reinterpret_cast<const u32x4*>(row + 8 * g);
        xh[it] = *reinterpret_cast<const u32x4*>(row + 64 + 8 * g);
    }
    const u32x4 qgl = *reinterpret_cast<const u32x4*>(A.qg + 8 * g), qgh = *reinterpret_cast<const u32x4*>(A.qg + 64 + 8 * g);
    const u32x4 kgl = *reinterpret_cast<const u32x4*>(A.kg + 8 * g), kgh = *reinterpret_cast<const u32x4*>(A.kg + 64 + 8 * g);
    __syncthreads();
    const uint32_t pos0 = s_pos + t0;
    for (uint32_t e = tid; e < TOK * 64; e += 256) {
        const uint32_t tk = e >> 6, i = e & 63;
        const uint32_t w = dev::rope_cs_bits(pos0 + tk, dev::rope_inv(i, A.theta));
        s_cos[tk][i] = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
        s_sin[tk][i] = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    }
    __syncthreads();

#pragma unroll
    for (uint32_t it = 0; it < IT; ++it) {
        if (32 * it >= nrows) break;
        const uint32_t hr = grp + 32 * it, hc = min(hr, nrows - 1), tk = hc / nh, r = hc - tk * nh;
        const bool is_q = r < A.H;
        const u32x4 gl = is_q ? qgl : kgl, gh = is_q ? qgh : kgh;
        const u32x4 cw = *reinterpret_cast<const u32x4*>(&s_cos[tk][8 * g]);
        const u32x4 sw = *reinterpret_cast<const u32x4*>(&s_sin[tk][8 * g]);
        u32x4 yl, yh;
        dev::qk_row8_norm_rope(xl[it], xh[it], gl, gh, cw, sw, yl, yh);
        if (hr >= nrows) continue;
        const uint32_t tok = t0 + tk;
        if (is_q) {
            __half* qo = A.q_out + (size_t)tok * A.H * HD + (size_t)r * HD;
            *reinterpret_cast<u32x4*>(qo + 8 * g) = yl;
            *reinterpret_cast<u32x4*>(qo + 64 + 8 * g) = yh;
        } else {
            const uint32_t kh = r - A.H;
            __half* kf = reinterpret_cast<__half*>(A.ring + (size_t)((pos0 + tk) % A.nslots) * A.slot_bytes) + kh * HD;
            *reinterpret_cast<u32x4*>(kf + 8 * g) = yl;
            *reinterpret_cast<u32x4*>(kf + 64 + 8 * g) = yh;
            if (A.k_out) {
                __half* ko = A.k_out + (size_t)tok * A.KVH * HD + (size_t)kh * HD;
                *reinterpret_cast<u32x4*>(ko + 8 * g) = yl;
                *reinterpret_cast<u32x4*>(ko + 64 + 8 * g) = yh;
            }
        }
    }
    // V rows: 16-byte chunks copied to the ring (and v_out).
    const uint32_t vc = A.KVH * HD / 8;
    for (uint32_t i = tid; i < nt * vc; i += 256) {
        const uint32_t tk = i / vc, c = i - tk * vc;
        const u32x4 v = *reinterpret_cast<const u32x4*>(A.qkv + (size_t)(t0 + tk) * A.ld + (size_t)nh * HD + 8 * c);
        __half* vf = reinterpret_cast<__half*>(A.ring + (size_t)((pos0 + tk) % A.nslots) * A.slot_bytes) + A.KVH * HD;
        *reinterpret_cast<u32x4*>(vf + 8 * c) = v;
        if (A.v_out) *reinterpret_cast<u32x4*>(A.v_out + (size_t)(t0 + tk) * A.KVH * HD + 8 * c) = v;
    }
    // Counter advance by the last workgroup to finish: every workgroup read *count at its
    // start (thread 0, waited for before the first barrier), so once all have counted
    // themselves done nobody reads it again in this launch.
    if (A.done && tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(A.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == gridDim.x - 1) {
            *A.done = 0u;
            *A.count = s_pos + n_tok;
        }
    }
}
constexpr uint32_t kQkRowsTok = 4;

// RoPE table of one prefill call for the q|k|v GEMM's fused QK-norm/RoPE epilogue:
// f16 cos and sin planes [n_tok][64] at positions *count + t (the entries the rows
// kernel builds in LDS), the start position in hdr[0]; the last workgroup to finish
// advances *count by n_tok, as the rows kernel does.
__global__ __launch_bounds__(256) void rope_table_kernel(uint32_t* count, uint32_t* done, float theta,
                                                         uint32_t n_tok, _Float16* cosp, _Float16* sinp,
                                                         uint32_t* hdr) {
    __shared__ uint32_t s_pos;
    __shared__ double s_inv[64];   // the 64 frequencies, once per workgroup
    const uint32_t tid = threadIdx.x, e = blockIdx.x * 256 + tid;
    if (tid == 0) s_pos = *count;
    if (tid < 64) s_inv[tid] = dev::rope_inv(tid, theta);
    __syncthreads();
    if (e < n_tok * 64) {
        const uint32_t w = dev::rope_cs_bits(s_pos + (e >> 6), s_inv[e & 63]);
        cosp[e] = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
        sinp[e] = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    }
    if (blockIdx.x == 0 && tid == 0) hdr[0] = s_pos;
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == gridDim.x - 1) {
            *done = 0u;
            *count = s_pos + n_tok;
        }
    }
}

// KV gather with GQA expansion (oplist_exec.c:2183-2231): kT[h][d][p], v[h][p][d].
__global__ void kv_gather_kernel(const uint8_t* __restrict__ ring, uint32_t slot_bytes,
                                 uint32_t nslots, __half* __restrict__ kT, __half* __restrict__ vo,
                                 uint32_t n_kv, uint32_t pstride, uint32_t H, uint32_t KVH,
                                 uint32_t hd) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;   // (h, p, d)
    const uint32_t total = H * pstride * hd;
    if (idx >= total) return;
    const uint32_t d = idx % hd;
    const uint32_t p = (idx / hd) % pstride;
    const uint32_t h = idx / (hd * pstride);
    const uint32_t rep = H / KVH;
    __half kval = __ushort_as_half(0), vval = __ushort_as_half(0);
    if (p < n_kv) {
        const uint32_t slot = p % nslots;
        const __half* kf = reinterpret_cast<const __half*>(ring + (size_t)slot * slot_bytes);
        kval = kf[(h / rep) * hd + d];
        vval = kf[KVH * hd + (h / rep) * hd + d];
    }
    if (kT) kT[((size_t)h * hd + d) * pstride + p] = kval;
    if (vo) vo[((size_t)h * pstride + p) * hd + d] = vval;
}

inline uint32_t blocks_for(size_t n, uint32_t bs) { return (uint32_t)((n + bs - 1) / bs); }

}  // namespace

namespace {
template <int C>
void rmsnorm2_reg(const __half* x, const __half* g, const __half* b, __half* y, uint32_t rows, uint32_t rw,
                  hipStream_t st) {
    if (b)
        hipLaunchKernelGGL((rmsnorm2_reg_kernel<C, true>), dim3(blocks_for(rows, 4)), dim3(256), 0, st, x, g, b, y,
                           rows, rw);
    else
        hipLaunchKernelGGL((rmsnorm2_reg_kernel<C, false>), dim3(blocks_for(rows, 4)), dim3(256), 0, st, x, g, b,
                           y, rows, rw);
}
}  // namespace

hipError_t launch_rmsnorm2(const __half* x, const __half* g, const __half* b, __half* y,
                           uint32_t rows, uint32_t rw, hipStream_t st) {
    if (!rows || !rw) return hipSuccess;
    const bool al = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                      reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
    const uint32_t c = (rw + 511) / 512;   // 16-byte chunks per lane
    if (al && rw % 8 == 0 && c <= 16) {
        if (c <= 1) rmsnorm2_reg<1>(x, g, b, y, rows, rw, st);
        else if (c <= 2) rmsnorm2_reg<2>(x, g, b, y, rows, rw, st);
        else if (c <= 4) rmsnorm2_reg<4>(x, g, b, y, rows, rw, st);
        else if (c <= 5) rmsnorm2_reg<5>(x, g, b, y, rows, rw, st);
        else if (c <= 8) rmsnorm2_reg<8>(x, g, b, y, rows, rw, st);
        else if (c <= 10) rmsnorm2_reg<10>(x, g, b, y, rows, rw, st);
        else rmsnorm2_reg<16>(x, g, b, y, rows, rw, st);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(rmsnorm2_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, st, x, g, b, y,
                       rows, rw);
    return hipGetLastError();
}

hipError_t launch_softmax(const __half* x, __half* y, uint32_t rows, uint32_t n, hipStream_t st) {
    if (!rows || !n) return hipSuccess;
    const int vector_form = (n % 32 == 0 && (size_t)rows * n >= 32) ? 1 : 0;
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, st, x, y, n, vector_form);
    return hipGetLastError();
}

hipError_t launch_binary(const __half* a, const __half* b, __half* y, uint32_t n, uint32_t subtype,
                         hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(binary_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, a, b, y, n, subtype);
    return hipGetLastError();
}

hipError_t launch_select(const __half* c, uint32_t cn, const __half* t, uint32_t tn,
                         const __half* f, uint32_t fn, __half* y, uint32_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(select_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, c, cn, t, tn, f,
                       fn, y, n);
    return hipGetLastError();
}

hipError_t launch_unary(const __half* x, __half* y, uint32_t n, uint32_t subtype, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(unary_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n, subtype);
    return hipGetLastError();
}

hipError_t launch_argmax(const __half* x, uint32_t n, int32_t* out, hipStream_t st) {
    const uint32_t n8 = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) ? n / 8 : 0;
    const uint32_t tail = n - 8 * n8;
    const uint32_t blocks = std::max({1u, (n8 + 256 * kArgmaxChunks - 1) / (256 * kArgmaxChunks),
                                      std::min(1024u, (tail + 4095) / 4096)});
    hipLaunchKernelGGL(argmax_part_kernel, dim3(blocks), dim3(256), 0, st, x, n, n8);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1), 0, st, out);
    return hipGetLastError();
}

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (!bytes) return hipSuccess;
    const size_t units = bytes % 16 == 0 ? bytes / 16 : bytes;
    uint32_t grid = blocks_for(units, 256);
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(256), 0, st, static_cast<uint8_t*>(dst),
                       static_cast<const uint8_t*>(src), bytes);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t st) {
    if (!bytes) return hipSuccess;
    const size_t units = bytes % 16 == 0 ? bytes / 16 : bytes;
    uint32_t grid = blocks_for(units, 256);
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, st, static_cast<uint8_t*>(dst), bytes);
    return hipGetLastError();
}

hipError_t launch_broadcast(const __half* x, __half* y, uint32_t n, const uint32_t in_d[4],
                            const uint32_t out_d[4], hipStream_t st) {
    if (!n) return hipSuccess;
    uint32_t r = 4;
    while (r > 0 && out_d[r - 1] == 1) r--;
    if (r == 0) r = 1;
    uint32_t ir = 4;
    if (ir > r) ir = r;
    Dims4 istr{{1, 1, 1, 1}}, ostr{{1, 1, 1, 1}}, ind{{in_d[0], in_d[1], in_d[2], in_d[3]}};
    for (int i = (int)ir - 2; i >= 0; --i) istr.v[i] = istr.v[i + 1] * in_d[i + 1];
    for (int i = (int)r - 2; i >= 0; --i) ostr.v[i] = ostr.v[i + 1] * out_d[i + 1];
    hipLaunchKernelGGL(broadcast_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n, ind,
                       ostr, istr, r, r - ir);
    return hipGetLastError();
}

hipError_t launch_transpose_gen(const __half* x, __half* y, uint32_t rk, const uint32_t dims[4],
                                uint32_t perm, hipStream_t st) {
    uint32_t p[4] = {perm & 0xFFu, (perm >> 8) & 0xFFu, (perm >> 16) & 0xFFu, (perm >> 24) & 0xFFu};
    Dims4 si{{1, 1, 1, 1}}, so{{1, 1, 1, 1}}, pm{{p[0], p[1], p[2], p[3]}};
    size_t n = 1;
    for (uint32_t i = 0; i < rk; ++i) n *= dims[i];
    for (int i = (int)rk - 2; i >= 0; --i) {
        si.v[i] = si.v[i + 1] * dims[i + 1];
        const uint32_t pd = p[i + 1] >= rk ? 1u : dims[p[i + 1]];
        so.v[i] = so.v[i + 1] * pd;
    }
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(transpose_gen_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y,
                       (uint32_t)n, rk, si, so, pm);
    return hipGetLastError();
}

hipError_t launch_slice(const __half* x, __half* y, uint32_t n_out, uint32_t rank,
                        const uint32_t b[3], const uint32_t s[3], const uint32_t d[3],
                        const uint32_t od[3], hipStream_t st) {
    if (!n_out) return hipSuccess;
    Dims4 bb{{b[0], b[1], b[2], 0}}, ss{{s[0], s[1], s[2], 1}}, istr{{1, 1, 1, 1}}, ostr{{1, 1, 1, 1}};
    for (int i = (int)rank - 2; i >= 0; --i) {
        istr.v[i] = istr.v[i + 1] * d[i + 1];
        ostr.v[i] = ostr.v[i + 1] * od[i + 1];
    }
    hipLaunchKernelGGL(slice_kernel, dim3(blocks_for(n_out, 256)), dim3(256), 0, st, x, y, n_out,
                       rank, bb, ss, istr, ostr);
    return hipGetLastError();
}

hipError_t launch_rope(const __half* x, __half* y, uint32_t n_tok, uint32_t n_heads, uint32_t hd,
                       uint32_t pos0, const uint32_t* pos_dev, float theta, uint32_t row_stride,
                       hipStream_t st) {
    const size_t n = (size_t)n_tok * (hd / 2);
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n_tok, n_heads,
                       hd, pos0, pos_dev, theta, row_stride);
    return hipGetLastError();
}

hipError_t launch_kv_append_n(uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                              const __half* k, const __half* v, uint32_t kv_elems, uint32_t n_tok,
                              uint32_t pos, uint32_t* count_dev, hipStream_t st) {
    if (!n_tok) return hipSuccess;
    hipLaunchKernelGGL(kv_append_kernel, dim3(n_tok), dim3(256), 0, st, ring, slot_bytes, nslots, k,
                       v, kv_elems, pos, count_dev);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pos != 0xFFFFFFFFu) return e;
    hipLaunchKernelGGL(counter_add_kernel, dim3(1), dim3(1), 0, st, count_dev, n_tok);
    return hipGetLastError();
}

hipError_t launch_kv_append(uint8_t* ring, uint32_t slot_bytes, uint32_t nslots, const __half* k,
                            const __half* v, uint32_t kv_elems, uint32_t pos, uint32_t* count_dev,
                            hipStream_t st) {
    return launch_kv_append_n(ring, slot_bytes, nslots, k, v, kv_elems, 1, pos, count_dev, st);
}

hipError_t launch_qk_rope_kv(const __half* qkv, uint32_t n_tok, uint32_t H, uint32_t KVH,
                             const __half* q_gamma, const __half* k_gamma, float theta, __half* q_out,
                             __half* k_out, __half* v_out, uint8_t* ring, uint32_t slot_bytes,
                             uint32_t nslots, uint32_t* count_dev, hipStream_t st, uint32_t* done_dev) {
    if (!H || !KVH || H + KVH > 4 * kQkMaxHeadsPerWave) return hipErrorInvalidValue;
    if (!n_tok) return hipSuccess;
    QkRopeKvArgs A{qkv, (H + 2 * KVH) * 128u, H, KVH, q_gamma, k_gamma, theta, q_out, k_out, v_out,
                   ring, slot_bytes, nslots, count_dev, n_tok == 1 ? 1 : 0, nullptr};
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const bool rows = n_tok > 1 && al16(qkv) && al16(q_gamma) && al16(k_gamma) && al16(q_out) && al16(k_out) &&
                      al16(v_out) && al16(ring) && slot_bytes % 16 == 0;
    if (rows) {
        A.done = done_dev;
        hipLaunchKernelGGL(qk_rope_kv_rows_kernel<kQkRowsTok>, dim3((n_tok + kQkRowsTok - 1) / kQkRowsTok), dim3(256),
                           0, st, A, n_tok);
    } else {
        hipLaunchKernelGGL(qk_rope_kv_kernel, dim3(n_tok), dim3(256), 0, st, A);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_tok == 1 || (rows && done_dev)) return e;
    hipLaunchKernelGGL(counter_add_kernel, dim3(1), dim3(1), 0, st, count_dev, n_tok);
    return hipGetLastError();
}

hipError_t launch_rope_table(uint32_t* count_dev, uint32_t* done_dev, float theta, uint32_t n_tok, void* table,
                             hipStream_t st) {
    if (!n_tok || !count_dev || !done_dev || !table || ((uintptr_t)table & 15u)) return hipErrorInvalidValue;
    _Float16* cosp = static_cast<_Float16*>(table);
    hipLaunchKernelGGL(rope_table_kernel, dim3((n_tok * 64 + 255) / 256), dim3(256), 0, st, count_dev, done_dev, theta,
                       n_tok, cosp, cosp + (size_t)n_tok * 64, reinterpret_cast<uint32_t*>(cosp + (size_t)n_tok * 128));
    return hipGetLastError();
}

hipError_t launch_kv_gather(const uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                            __half* kT, __half* vo, uint32_t n_kv, uint32_t pstride, uint32_t H,
                            uint32_t KVH, uint32_t hd, hipStream_t st) {
    const size_t n = (size_t)H * pstride * hd;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(kv_gather_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, ring, slot_bytes,
                       nslots, kT, vo, n_kv, pstride, H, KVH, hd);
    return hipGetLastError();
}

}  // namespace gehtp
