// dev_w4g.h — W4A16 device helpers shared by the GEMV kernels (k_w4g.hip) and the
// fused q|k|v GEMV + decode attention kernel (k_attn.hip): the exact group-64 dequant,
// fp16 bit conversions and the row-in-wave GEMV body.
//
// Weight format (OP_MATMUL_W4G_F16): wq row n = K/2 bytes, byte j holds k=2j in the
// low nibble and k=2j+1 in the high nibble, stored as q+8; ws[n][k/64] fp16.
#pragma once

#include "dev_reduce.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <cstdint>

namespace gehtp {

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16x_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// (w & mask) | magic in one VALU op. Written out because with both constants as
// literals the compiler emits a separate AND and OR (gfx9 VOP3 takes no literal, so
// the mask goes in an SGPR and the magic in a VGPR).
template <uint32_t MASK>
__device__ __forceinline__ uint32_t nib_magic(uint32_t w, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(MASK), "v"(magic));
    return r;
}

// Four dequantized pairs (k0,k4),(k1,k5),(k2,k6),(k3,k7) of one weight word.
__device__ __forceinline__ void dequant_word(uint32_t w, h2_t s2, h2_t out[4]) {
    const h2_t b_lo = {(_Float16)1032.0f, (_Float16)1032.0f};   // 1024 + 8
    const h2_t b_hi = {(_Float16)72.0f, (_Float16)72.0f};       // 64 + 8
    const uint32_t w8 = w >> 8;
    // q = h - bias is exact (small integers); q * s is the one RNE rounding: fp16(q*s)
    out[0] = (as_h2(nib_magic<0x000F000Fu>(w, 0x64006400u)) - b_lo) * s2;
    out[1] = (as_h2(nib_magic<0x00F000F0u>(w, 0x54005400u)) - b_hi) * s2;
    out[2] = (as_h2(nib_magic<0x000F000Fu>(w8, 0x64006400u)) - b_lo) * s2;
    out[3] = (as_h2(nib_magic<0x00F000F0u>(w8, 0x54005400u)) - b_hi) * s2;
}

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2hb(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// UNARY silu on an fp16 input: f16(h / (1 + exp(-h))) with each fp32 op correctly rounded.
__device__ __forceinline__ uint16_t silu_f16_expr(uint16_t hb) {
    const float h = h2f(hb);
    return f2hb(__fdiv_rn(h, __fadd_rn(1.0f, expf(-h))));
}

// ---------------------------------------------------------------------------
// GEMV for M = 1 with whole rows inside a wave. P = 16 or 32 lanes share a row, each
// owning C of its 16-byte slices (lane p: slices p, p + P, ...; K = 32 * C * P, so each
// load instruction reads P consecutive slices of a row), and a wave holds RW = 64 / P
// rows per pass and a row's partial sums meet in DPP / row-swap steps inside the wave:
// no workgroup barrier follows the passes, and each wave stores its rows as soon as its
// own loads have landed (w4g_gemv_kernel waits at a barrier for the workgroup's slowest
// wave before its LDS row sums). Every weight load is issued up front, slice-major (the
// order the arithmetic consumes them), behind the activation loads. The workgroup stages
// x once in LDS, in the dequant's pair order, normalized first when gamma is given (the
// RMSNorm prologue of w4g_gemv_kernel: same arithmetic and bits), chunk i at slot
// i ^ ((i >> 4) & 3) so that the 16 lanes of a read hit 16 distinct bank groups. Per row
// the C slices of a lane are summed in order, then the P lanes by the butterfly of
// dev::row_sum16 (and dev::pair_row_sum for P = 32).
//
// With REC (no SwiGLU), each pair of rows (2i, 2i + 1) is also published as one 8-byte
// record rec[i] = y[2i] | y[2i + 1] << 16 | tag << 32, stored with one agent-scope atomic
// store: a reader on any XCD that polls rec[i] with agent-scope atomic loads until it
// sees the tag has both values, with no fence on either side (a kernel that runs this
// body next to the rows' readers hands them over that way).
//
// With XREC, x is not read from A.x but from such records, xrec[i] = x[2i] | x[2i + 1] <<
// 16 | xtag << 32, which other workgroups of the same launch publish: the weight loads
// are issued first, then one thread waits for the last record and every thread reads
// (and checks) its own.

// Bound on the polls of one hand-off record: a wait that reaches it writes 1 to *err and
// goes on with two fp16 NaNs in place of the values (so the call's outputs show it), so
// that every wave ends. ~1 us per poll, so tens of ms.
constexpr uint32_t kHandoffSpins = 1u << 15;
constexpr uint32_t kHandoffNaN2 = 0x7E007E00u;

// The low 32 bits of record p once its high half carries tag: agent-scope atomic loads,
// s_sleep(NAP) between them.
template <int NAP>
__device__ __forceinline__ uint32_t handoff_wait(const unsigned long long* p, uint32_t tag, uint32_t* err) {
    unsigned long long v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t spin = 0; (uint32_t)(v >> 32) != tag; ++spin) {
        if (spin == kHandoffSpins) {
            *err = 1u;
            return kHandoffNaN2;
        }
        __builtin_amdgcn_s_sleep(NAP);
        v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return (uint32_t)v;
}
__device__ __forceinline__ void handoff_store(unsigned long long* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, (unsigned long long)tag << 32 | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemvRwArgs {
    const __half* x;
    const uint8_t* wq;
    const __half* ws;
    __half* y;
    uint32_t N, K;
    const __half* gamma;
    const __half* res;
    int swiglu;
};

// Workgroup wg of the launch, nt threads (nt / 64 waves); xn: K / 8 16-byte LDS slots
// (x in pair order, padded layout), s_ss: 8 doubles of LDS.
template <int C, int P, int NP, int PRE, bool REC = false, bool XREC = false>
__device__ __forceinline__ void gemv_rw_body(const GemvRwArgs& A, uint32_t wg, uint32_t nt, u32x4* xn,
                                             double* s_ss, unsigned long long* rec = nullptr,
                                             uint32_t tag = 0u, const unsigned long long* xrec = nullptr,
                                             uint32_t xtag = 0u, uint32_t* err = nullptr) {
    constexpr int RW = 64 / P;
    static_assert(P == 16 || P == 32, "lanes per row");
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t p = lane % P, g = lane / P;
    const uint32_t R = (nt / 64) * RW, rows_wg = R * NP;
    // As in w4g_gemv_kernel: N >= rows_wg, and the last workgroup is moved back to end at
    // row N, recomputing (not storing) the rows its predecessor covers.
    const uint32_t r0n = wg * rows_wg;
    const uint32_t r0 = min(r0n, A.N - rows_wg);
    const uint32_t skip = r0n - r0;
    const uint32_t rowbytes = A.K / 2, G = A.K / 64, K8 = A.K / 8;
    const uint32_t lrow = wave * RW + g;   // this lane's row within a pass
    auto slice = [&](int c) -> uint32_t { return (uint32_t)c * P + p; };   // this lane's slices

    // x (and gamma) chunks this thread stages: t, t + nt, ... (clamped; K8 <= PRE nt is
    // checked on the host).
    u32x4 xv[PRE], gv[PRE];
#pragma unroll
    for (int k = 0; k < PRE; ++k) {
        const uint32_t i = min(t + k * nt, K8 - 1);
        if constexpr (!XREC) xv[k] = reinterpret_cast<const u32x4*>(A.x)[i];
        if (A.gamma) gv[k] = reinterpret_cast<const u32x4*>(A.gamma)[i];
    }
    uint16_t resv[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const uint32_t r = r0 + i * R + lrow;
        resv[i] = A.res ? __builtin_bit_cast(uint16_t, A.res[A.swiglu ? r / 2 : r]) : (uint16_t)0;
    }
    const uint8_t* wq0 = A.wq + (size_t)r0 * rowbytes;
    const uint16_t* ws0 = reinterpret_cast<const uint16_t*>(A.ws) + (size_t)r0 * G;
    u32x4 w[C][NP];
    uint16_t sc[C][NP];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const uint32_t lr = i * R + lrow;
            w[c][i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(wq0 + (size_t)(lr * rowbytes + slice(c) * 16)));
            sc[c][i] = ws0[(size_t)lr * G + (slice(c) >> 1)];
        }
    if constexpr (XREC) {
        if (t == 0) handoff_wait<2>(xrec + (K8 * 4 - 1), xtag, err);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PRE; ++k) {
            const uint32_t i = min(t + k * nt, K8 - 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[k][e] = handoff_wait<1>(xrec + 4 * i + e, xtag, err);
        }
    }

    float rms = 1.0f, rcp = 1.0f;
    if (A.gamma) {
        // RMSNorm of w4g_gemv_kernel (M = 1): sum of squares in double over the row.
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < PRE; ++k) {
            if (t + k * nt >= K8) break;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double lo = (double)h2f((uint16_t)(xv[k][e] & 0xFFFFu));
                const double hi = (double)h2f((uint16_t)(xv[k][e] >> 16));
                ss = __builtin_fma(lo, lo, ss);
                ss = __builtin_fma(hi, hi, ss);
            }
        }
        {
            const double wsum = dev::wave_sum(ss);
            if (lane == 0) s_ss[wave] = wsum;
        }
        __syncthreads();
        double tot = 0.0;
        for (uint32_t v = 0; v < nt / 64; ++v) tot += s_ss[v];
        rms = (float)sqrt(tot / (double)A.K + 1e-6);
        rcp = __fdiv_rn(1.0f, rms);
    }
    auto div_rms = [&](float a) {
        const float q = a * rcp;
        return __builtin_fmaf(__builtin_fmaf(-q, rms, a), rcp, q);
    };
    auto xslot = [](uint32_t i) -> uint32_t { return i ^ ((i >> 4) & 3u); };
#pragma unroll
    for (int k = 0; k < PRE; ++k) {
        const uint32_t i = t + k * nt;
        if (i >= K8) break;
        u32x4 o = xv[k];
        if (A.gamma) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float lo = div_rms(h2f((uint16_t)(o[e] & 0xFFFFu)));
                float hi = div_rms(h2f((uint16_t)(o[e] >> 16)));
                // RN(y * g + 0) in one fma: the exact product plus +0 rounded once is the
                // separate multiply's rounding, with -0 mapped to +0 as by the "+ 0". The
                // empty asm keeps the f32 result as it is before the fp16 conversion (a
                // mixed-precision fma rounding straight to fp16 would skip that rounding).
                lo = __builtin_fmaf(lo, h2f((uint16_t)(gv[k][e] & 0xFFFFu)), 0.0f);
                hi = __builtin_fmaf(hi, h2f((uint16_t)(gv[k][e] >> 16)), 0.0f);
                asm volatile("" : "+v"(lo), "+v"(hi));
                o[e] = (uint32_t)f2hb(lo) | ((uint32_t)f2hb(hi) << 16);
            }
        }
        // pair order (x0,x4) (x1,x5) (x2,x6) (x3,x7)
        xn[xslot(i)] = u32x4{(o[0] & 0xFFFFu) | (o[2] << 16), (o[0] >> 16) | (o[2] & 0xFFFF0000u),
                             (o[1] & 0xFFFFu) | (o[3] << 16), (o[1] >> 16) | (o[3] & 0xFFFF0000u)};
    }
    __syncthreads();

    float acc[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        u32x4 xp[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) xp[e] = xn[xslot(4 * slice(c) + e)];
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const _Float16 sh = __builtin_bit_cast(_Float16, sc[c][i]);
            const h2_t s2 = {sh, sh};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h2_t d[4];
                dequant_word(w[c][i][e], s2, d);
                acc[i] = __builtin_amdgcn_fdot2(d[0], as_h2(xp[e][0]), acc[i], false);
                acc[i] = __builtin_amdgcn_fdot2(d[1], as_h2(xp[e][1]), acc[i], false);
                acc[i] = __builtin_amdgcn_fdot2(d[2], as_h2(xp[e][2]), acc[i], false);
                acc[i] = __builtin_amdgcn_fdot2(d[3], as_h2(xp[e][3]), acc[i], false);
            }
        }
        // one slice's x pairs in registers at a time (the compiler would otherwise hoist
        // every slice's LDS reads and hold them all)
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        float sum = dev::row_sum16(acc[i]);
        if constexpr (P == 32) sum = dev::pair_row_sum(sum);
        const uint32_t lr = i * R + lrow;
        if constexpr (REC) {   // no SwiGLU: rows 2k (group g even) and 2k + 1 (group g + 1) as one record
            uint16_t v = f2hb(sum);
            if (A.res) v = f2hb(__fadd_rn(h2f(v), h2f(resv[i])));
            if (p == 0 && lr >= skip) reinterpret_cast<uint16_t*>(A.y)[r0 + lr] = v;
            uint32_t a = v, b = a;
            if constexpr (P == 16) dev::permlane16_swap(a, b);
            else dev::permlane32_swap(a, b);
            if (p == 0 && !(g & 1) && lr >= skip)
                __hip_atomic_store(rec + ((r0 + lr) >> 1),
                                   (unsigned long long)tag << 32 | (uint32_t)v | (b & 0xFFFFu) << 16,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (!A.swiglu) {
            if (p == 0 && lr >= skip) {
                uint16_t v = f2hb(sum);
                if (A.res) v = f2hb(__fadd_rn(h2f(v), h2f(resv[i])));
                reinterpret_cast<uint16_t*>(A.y)[r0 + lr] = v;
            }
        } else {
            // gate = row 2k (group g even), up = row 2k + 1 (group g + 1): the partner's
            // sum arrives in the even group's lanes through the row swap pairing them.
            uint32_t a = __builtin_bit_cast(uint32_t, sum), b = a;
            if constexpr (P == 16) dev::permlane16_swap(a, b);
            else dev::permlane32_swap(a, b);
            const float up = __builtin_bit_cast(float, b);
            if (p == 0 && !(g & 1) && lr >= skip) {
                const float gvf = h2f(f2hb(sum)), uv = h2f(f2hb(up));
                const float act = h2f(silu_f16_expr(f2hb(gvf)));
                uint16_t v = f2hb(__fmul_rn(act, uv));
                if (A.res) v = f2hb(__fadd_rn(h2f(v), h2f(resv[i])));
                reinterpret_cast<uint16_t*>(A.y)[(r0 + lr) >> 1] = v;
            }
        }
    }
}

}  // namespace

}  // namespace gehtp
