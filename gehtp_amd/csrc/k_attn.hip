// k_attn.hip — causal GQA attention for gfx950: flash prefill (MFMA) and split-KV decode.
//
// Prefill computes S^T = K . Q^T instead of Q . K^T so that each lane of a 32x32
// MFMA accumulator owns ONE query and 16 keys: the online-softmax row statistics
// then need a single cross-lane exchange (lane l <-> l^32) instead of a 32-lane
// reduction, and the rescale of the output accumulator is a per-lane scalar.
// O^T = V^T . P^T reuses P straight from the accumulator registers as the MFMA B
// operand; V is staged transposed in LDS so the A operand reads 8-byte runs.
#include "kernels.h"

#include <cmath>

namespace gehtp {

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f16x_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Reinterpret a 32-bit word as two halves. Takes the word BY VALUE: a bit cast applied
// directly to an ext_vector element (v[e]) miscompiles to always reading element 0.
__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

constexpr int HD = 128;          // head dim this kernel is built for
constexpr int QT = 128;          // queries per workgroup (4 waves x 32)
constexpr int KT = 64;           // keys per LDS stage
constexpr int KS = HD + 8;       // K tile row stride (halves)
constexpr int VS = KT + 8;       // V^T tile row stride (halves)
constexpr float kLog2e = 1.4426950408889634f;

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const __half* __restrict__ q, uint32_t ldq, const __half* __restrict__ k,
    const __half* __restrict__ v, uint32_t ldkv, __half* __restrict__ out, uint32_t ldo,
    uint32_t S, uint32_t H, uint32_t KVH, float scale_log2) {
    __shared__ __align__(16) _Float16 Ks[KT * KS];
    __shared__ __align__(16) _Float16 Vt[HD * VS];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n_qt = (S + QT - 1) / QT;
    const uint32_t qtile = n_qt - 1 - blockIdx.x;      // heaviest causal tiles first
    const uint32_t h = blockIdx.y;
    const uint32_t kvh = h / (H / KVH);
    const uint32_t q0 = qtile * QT;
    const uint32_t qw = q0 + wave * 32;                 // this wave's first query
    const uint32_t my_q = qw + (lane & 31);
    const uint32_t hl = lane >> 5;

    // Q^T fragments (MFMA B operand): query my_q, dims 16*kk + 8*hl + [0,8).
    h8_t qf[HD / 16];
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
        if (my_q < S)
            qf[kk] = *reinterpret_cast<const h8_t*>(q + (size_t)my_q * ldq + h * HD + kk * 16 + hl * 8);
        else
            qf[kk] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }

    f16x_t o[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    const uint32_t kend = CAUSAL ? min(S, q0 + QT) : S;
    for (uint32_t kb = 0; kb < kend; kb += KT) {
        __syncthreads();
        // Stage K (row-major) and V (transposed) for keys [kb, kb+64).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = (tid >> 4) + 16 * i, ch = tid & 15;
            u32x4 kv4 = {0, 0, 0, 0}, vv4 = {0, 0, 0, 0};
            if (kb + key < S) {
                const size_t off = (size_t)(kb + key) * ldkv + kvh * HD + ch * 8;
                kv4 = *reinterpret_cast<const u32x4*>(k + off);
                vv4 = *reinterpret_cast<const u32x4*>(v + off);
            }
            *reinterpret_cast<u32x4*>(&Ks[key * KS + ch * 8]) = kv4;
            const _Float16* ve = reinterpret_cast<const _Float16*>(&vv4);
#pragma unroll
            for (int e = 0; e < 8; ++e) Vt[(ch * 8 + e) * VS + key] = ve[e];
        }
        __syncthreads();

#pragma unroll
        for (int sub = 0; sub < KT / 32; ++sub) {
            const uint32_t kt0 = kb + sub * 32;
            if (CAUSAL && kt0 > qw + 31) continue;   // whole 32x32 block masked for this wave
            if (kt0 >= S) continue;
            f16x_t s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < HD / 16; ++kk) {
                const h8_t kf = *reinterpret_cast<const h8_t*>(&Ks[(sub * 32 + (lane & 31)) * KS + kk * 16 + hl * 8]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], s, 0, 0, 0);
            }
            // s[r]: key kt0 + 8*(r/4) + 4*hl + r%4, query my_q.
            float mloc = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t key = kt0 + 8 * (r >> 2) + 4 * hl + (r & 3);
                float x = s[r] * scale_log2;
                if (key >= S || (CAUSAL && key > my_q)) x = -INFINITY;
                s[r] = x;
                mloc = fmaxf(mloc, x);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const float m_new = fmaxf(m_run, mloc);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f(m_run - m_use);
            float lsum = 0.0f;
            h8_t pb[2];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2f(s[r] - m_use);
                lsum += p;
                pb[r >> 3][r & 7] = (_Float16)p;
            }
            lsum += __shfl_xor(lsum, 32, 64);
            l_run = l_run * alpha + lsum;
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            // O^T[d][q] += sum_key V^T[d][key] P^T[key][q]. k-slot 8*hl+i of half j maps to
            // key 16*j + 8*(i/4) + 4*hl + i%4 — the key held in pb[j][i].
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt) {
                const uint32_t d = dt * 32 + (lane & 31);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t kl = sub * 32 + 16 * j + 4 * hl;
                    const u32x2 lo = *reinterpret_cast<const u32x2*>(&Vt[d * VS + kl]);
                    const u32x2 hi = *reinterpret_cast<const u32x2*>(&Vt[d * VS + kl + 8]);
                    const u32x4 packed = {lo[0], lo[1], hi[0], hi[1]};
                    const h8_t vf = __builtin_bit_cast(h8_t, packed);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pb[j], o[dt], 0, 0, 0);
                }
            }
        }
    }

    if (my_q < S) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        __half* orow = out + (size_t)my_q * ldo + h * HD;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                h4_t v4;
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = (_Float16)(o[dt][rb * 4 + e] * inv);
                *reinterpret_cast<h4_t*>(orow + dt * 32 + rb * 8 + 4 * hl) = v4;
            }
    }
}

// ---------------------------------------------------------------------------
// Decode: workgroup (chunk c, kv head g) handles keys [64c, 64c+64) for the rep query
// heads of g, reading each K/V row once. Partial (max, sum, O) go to the workspace
// and a second kernel merges the chunks with the log-sum-exp rule.
constexpr int DC = 64;          // keys per chunk
constexpr int MAX_REP = 8;

template <int REP>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const __half* __restrict__ q, const uint8_t* __restrict__ ring, uint32_t slot_bytes,
    uint32_t nslots, uint32_t n_kv_host, const uint32_t* __restrict__ count_dev, uint32_t KVH,
    float scale_log2, float* __restrict__ work, uint32_t* __restrict__ done, uint32_t max_chunks,
    __half* __restrict__ out) {
    __shared__ float sc[REP][DC];
    __shared__ float red[4][REP][HD];
    __shared__ float s_M[REP], s_L[REP];
    __shared__ uint32_t s_last;
    const uint32_t n_kv = count_dev ? *count_dev : n_kv_host;
    const uint32_t c = blockIdx.x, g = blockIdx.y;
    if (c * DC >= n_kv) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t ch = lane & 15;   // 8-dim chunk of the head

    u32x4 qv[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r)
        qv[r] = *reinterpret_cast<const u32x4*>(q + (size_t)(g * REP + r) * HD + ch * 8);

    // Phase 1: scores. 4 keys per wave per step (16 lanes per key).
#pragma unroll
    for (int it = 0; it < DC / 16; ++it) {
        const uint32_t kl = it * 16 + wave * 4 + (lane >> 4);
        const uint32_t key = c * DC + kl;
        float acc[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) acc[r] = 0.0f;
        if (key < n_kv) {
            const uint32_t slot = key % nslots;
            const u32x4 kv4 = *reinterpret_cast<const u32x4*>(
                ring + (size_t)slot * slot_bytes + ((size_t)g * HD + ch * 8) * 2);
#pragma unroll
            for (int r = 0; r < REP; ++r)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[r] = __builtin_amdgcn_fdot2(as_h2(kv4[e]),
                                                    as_h2(qv[r][e]), acc[r], false);
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float a = acc[r];
            a += __shfl_xor(a, 8, 64);
            a += __shfl_xor(a, 4, 64);
            a += __shfl_xor(a, 2, 64);
            a += __shfl_xor(a, 1, 64);
            if (ch == 0) sc[r][kl] = key < n_kv ? a * scale_log2 : -INFINITY;
        }
    }
    __syncthreads();

    // Phase 2: per-head max and exponentials over the chunk (one wave per head).
    float* wchunk = work + ((size_t)g * max_chunks + c) * REP * (HD + 2);
    for (uint32_t r = wave; r < REP; r += 4) {
        const float x = sc[r][lane];
        float m = x;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        const float p = exp2f(x - m);
        float l = p;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
        sc[r][lane] = p;
        if (lane == 0) { wchunk[r * (HD + 2)] = m; wchunk[r * (HD + 2) + 1] = l; }
    }
    __syncthreads();

    // Phase 3: O[r][d] = sum_key p[r][key] V[key][d]; 16 key streams x 16 dim chunks.
    float acc[REP][8];
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
    const uint32_t stream = tid >> 4;
#pragma unroll
    for (int it = 0; it < DC / 16; ++it) {
        const uint32_t kl = stream + 16 * it;
        const uint32_t key = c * DC + kl;
        if (key < n_kv) {
            const uint32_t slot = key % nslots;
            const u32x4 vv4 = *reinterpret_cast<const u32x4*>(
                ring + (size_t)slot * slot_bytes + slot_bytes / 2 + ((size_t)g * HD + ch * 8) * 2);
            const _Float16* ve = reinterpret_cast<const _Float16*>(&vv4);
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float p = sc[r][kl];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r][e] = fmaf(p, (float)ve[e], acc[r][e]);
            }
        }
    }
    // Reduce the 4 streams inside the wave (lanes l, l^16, l^32, l^48), then across waves.
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float a = acc[r][e];
            a += __shfl_xor(a, 16, 64);
            a += __shfl_xor(a, 32, 64);
            acc[r][e] = a;
        }
    if (lane < 16) {
#pragma unroll
        for (int r = 0; r < REP; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e) red[wave][r][ch * 8 + e] = acc[r][e];
    }
    __syncthreads();
    for (uint32_t i = tid; i < REP * HD; i += 256) {
        const uint32_t r = i / HD, d = i % HD;
        wchunk[r * (HD + 2) + 2 + d] = red[0][r][d] + red[1][r][d] + red[2][r][d] + red[3][r][d];
    }

    // The last workgroup of this kv head to finish merges the chunks (log-sum-exp) and
    // resets the completion counter for the next call.
    const uint32_t nc = (n_kv + DC - 1) / DC;
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&done[g], 1u) == nc - 1) ? 1u : 0u;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float* wg = work + (size_t)g * max_chunks * REP * (HD + 2);
    for (uint32_t r = wave; r < REP; r += 4) {
        float M = -INFINITY;
        for (uint32_t cc = lane; cc < nc; cc += 64) M = fmaxf(M, wg[(size_t)cc * REP * (HD + 2) + r * (HD + 2)]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        float L = 0.0f;
        for (uint32_t cc = lane; cc < nc; cc += 64) {
            const float* w = wg + (size_t)cc * REP * (HD + 2) + r * (HD + 2);
            L += w[1] * exp2f(w[0] - M);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off, 64);
        if (lane == 0) { s_M[r] = M; s_L[r] = L; }
    }
    __syncthreads();
    for (uint32_t i = tid; i < REP * HD; i += 256) {
        const uint32_t r = i / HD, d = i % HD;
        const float M = s_M[r];
        float O = 0.0f;
        for (uint32_t cc = 0; cc < nc; ++cc) {
            const float* w = wg + (size_t)cc * REP * (HD + 2) + r * (HD + 2);
            O += w[2 + d] * exp2f(w[0] - M);
        }
        out[(size_t)(g * REP + r) * HD + d] = __float2half(s_L[r] > 0.0f ? O / s_L[r] : 0.0f);
    }
    if (tid == 0) done[g] = 0;
}

}  // namespace

hipError_t launch_attn_prefill(const __half* q, uint32_t ldq, const __half* k, const __half* v,
                               uint32_t ldkv, __half* out, uint32_t ldo, uint32_t S, uint32_t H,
                               uint32_t KVH, uint32_t hd, float scale, bool causal,
                               hipStream_t st) {
    if (hd != HD || !KVH || H % KVH) return hipErrorInvalidValue;
    if (!S || !H) return hipSuccess;
    dim3 grid((S + QT - 1) / QT, H);
    const float sl2 = scale * kLog2e;
    if (causal)
        hipLaunchKernelGGL(attn_prefill_kernel<true>, grid, dim3(256), 0, st, q, ldq, k, v, ldkv,
                           out, ldo, S, H, KVH, sl2);
    else
        hipLaunchKernelGGL(attn_prefill_kernel<false>, grid, dim3(256), 0, st, q, ldq, k, v, ldkv,
                           out, ldo, S, H, KVH, sl2);
    return hipGetLastError();
}

// Workspace: KVH completion counters (64 floats reserved, zero before the first call;
// every call leaves them zero) followed by the per-chunk partials.
constexpr uint32_t kDoneSlots = 64;

uint32_t attn_decode_work_floats(uint32_t max_kv, uint32_t H, uint32_t hd) {
    return kDoneSlots + ((max_kv + DC - 1) / DC) * H * (hd + 2);
}

hipError_t launch_attn_decode(const __half* q, const uint8_t* ring, uint32_t slot_bytes,
                              uint32_t nslots, __half* out, uint32_t n_kv_host,
                              const uint32_t* count_dev, uint32_t H, uint32_t KVH, uint32_t hd,
                              float scale, float* work, uint32_t work_floats, hipStream_t st) {
    if (hd != HD || !KVH || H % KVH || KVH > kDoneSlots) return hipErrorInvalidValue;
    const uint32_t rep = H / KVH;
    if (rep > MAX_REP || slot_bytes != KVH * HD * 4) return hipErrorInvalidValue;
    // Chunks cover every position the ring can hold, so a device-side count never
    // exceeds the grid.
    const uint32_t max_kv = count_dev ? nslots : n_kv_host;
    const uint32_t max_chunks = (max_kv + DC - 1) / DC;
    if (attn_decode_work_floats(max_kv, H, hd) > work_floats) return hipErrorInvalidValue;
    if (!max_chunks) return hipSuccess;
    const float sl2 = scale * kLog2e;
    uint32_t* done = reinterpret_cast<uint32_t*>(work);
    float* part = work + kDoneSlots;
    dim3 grid(max_chunks, KVH);
    switch (rep) {
    case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(256), 0, st, q, ring, slot_bytes, nslots, n_kv_host, count_dev, KVH, sl2, part, done, max_chunks, out); break;
    case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(256), 0, st, q, ring, slot_bytes, nslots, n_kv_host, count_dev, KVH, sl2, part, done, max_chunks, out); break;
    case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, dim3(256), 0, st, q, ring, slot_bytes, nslots, n_kv_host, count_dev, KVH, sl2, part, done, max_chunks, out); break;
    case 8: hipLaunchKernelGGL(attn_decode_kernel<8>, grid, dim3(256), 0, st, q, ring, slot_bytes, nslots, n_kv_host, count_dev, KVH, sl2, part, done, max_chunks, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gehtp
