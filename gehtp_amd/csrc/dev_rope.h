// dev_rope.h — device helpers shared by the QK-norm/RoPE kernels (k_rows.hip) and the
// fused decode attention (k_attn.hip), so both produce the same bits.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dev_reduce.h"

namespace gehtp {
namespace dev {

// binary64 -> binary16, one RNE rounding (the reference builds RoPE tables this way).
__device__ __forceinline__ uint16_t f64_to_f16_bits(double d) {
    const uint64_t x = __builtin_bit_cast(uint64_t, d);
    const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    const int32_t dexp = (int32_t)((x >> 52) & 0x7ffu);
    const uint64_t man = x & ((1ull << 52) - 1);
    if (dexp == 0x7ff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    const int32_t exp = dexp - 1008;
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    uint64_t kept, rem, halfway;
    if (exp <= 0) {
        if (exp < -10) return sign;
        const uint64_t m = man | (1ull << 52);
        const uint32_t shift = (uint32_t)(43 - exp);
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

__device__ __forceinline__ float bits_f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float rne_f16(float f) { return (float)(_Float16)f; }

// RoPE table entry of pair i of a 128-dim head at position pos:
// c, s = f16(cos / sin(pos * theta^(-2i/128))) evaluated in double.
__device__ __forceinline__ double rope_inv(uint32_t i, float theta) {
    return 1.0 / pow((double)theta, (double)(2 * i) / 128.0);
}
// The pair as f16 bits: cos in bits 0-15, sin in bits 16-31.
__device__ __forceinline__ uint32_t rope_cs_bits(uint32_t pos, double inv) {
    double s, c;
    sincos((double)pos * inv, &s, &c);   // one argument reduction, the bits of cos() and sin()
    return (uint32_t)f64_to_f16_bits(c) | ((uint32_t)f64_to_f16_bits(s) << 16);
}
__device__ __forceinline__ void rope_cs_inv(uint32_t pos, double inv, float& c, float& s) {
    const uint32_t w = rope_cs_bits(pos, inv);
    c = bits_f((uint16_t)(w & 0xFFFFu));
    s = bits_f((uint16_t)(w >> 16));
}
__device__ __forceinline__ void rope_cs(uint32_t pos, uint32_t i, float theta, float& c, float& s) {
    rope_cs_inv(pos, rope_inv(i, theta), c, s);
}

// One 128-dim head held by a full wavefront, lane l owning (x[l], x[l+64]):
// h = RMSNORM2_F16(x, gamma, zero bias) (squares summed in double), then the RoPE
// chain y_l = f16(f16(h_l c) + f16(-h_{l+64} s)), y_{l+64} = f16(f16(h_{l+64} c) + f16(h_l s)).
// Every lane of the wavefront must call it (cross-lane sum).
// x / rms is RN(x * y) corrected once with y = RN(1 / rms) (Markstein): q = RN(x * y),
// r = fma(-q, rms, x) (exact), RN(q + r * y) — the correctly rounded quotient, the same
// as IEEE division for every finite fp16 x (a signed zero may differ, which the + 0
// below maps to +0 either way).
__device__ __forceinline__ float div_markstein(float a, float b, float y) {
    const float q = a * y;
    return __builtin_fmaf(__builtin_fmaf(-q, b, a), y, q);
}

__device__ __forceinline__ void head_norm_rope(float x1, float x2, float g1, float g2, float c, float s,
                                               float& y1, float& y2) {
    const double ss = wave_sum((double)x1 * (double)x1 + (double)x2 * (double)x2);
    const float rms = (float)sqrt(ss / 128.0 + 1e-6);
    const float y = __fdiv_rn(1.0f, rms);
    const float h1 = rne_f16(__fadd_rn(__fmul_rn(div_markstein(x1, rms, y), g1), 0.0f));
    const float h2 = rne_f16(__fadd_rn(__fmul_rn(div_markstein(x2, rms, y), g2), 0.0f));
    const float a1 = rne_f16(__fmul_rn(h1, c)), b1 = rne_f16(__fmul_rn(-h2, s));
    const float a2 = rne_f16(__fmul_rn(h2, c)), b2 = rne_f16(__fmul_rn(h1, s));
    y1 = rne_f16(__fadd_rn(a1, b1));
    y2 = rne_f16(__fadd_rn(a2, b2));
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2_pk __attribute__((ext_vector_type(2)));
// A word as two f16 lanes. Words are passed by value: __builtin_bit_cast applied directly
// to an element of an ext_vector reads element 0 whatever the index.
__device__ __forceinline__ h2_pk h2_of(uint32_t w) { return __builtin_bit_cast(h2_pk, w); }

// One 128-dim q or k head row held by an aligned group of 8 lanes: lane g owns halves
// [8g, 8g+8) (xl) and [64+8g, 64+8g+8) (xh) — both halves of its RoPE pairs — with the
// gamma halves at the same places (gl, gh) and the token's RoPE table entries 8g..8g+7
// as f16 cos (cw) and sin (sw). RMSNORM2_F16 without bias: squares in double, summed in
// the lane's element order, then over the group as ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7));
// x / rms as Markstein's corrected quotient, times gamma, + 0, rounded to f16. RoPE on
// packed f16: each product and sum of two f16 values rounded once to f16 equals the f32
// operation rounded to f16 (24 >= 2*11 + 1 bits, so the double rounding is innocuous),
// the arithmetic of the reference's rope op. All 8 lanes of the group must call it.
__device__ __forceinline__ void qk_row8_norm_rope(const u32x4_t& xl, const u32x4_t& xh, const u32x4_t& gl,
                                                  const u32x4_t& gh, const u32x4_t& cw, const u32x4_t& sw,
                                                  u32x4_t& yl, u32x4_t& yh) {
    float x[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        x[2 * k] = bits_f((uint16_t)(xl[k] & 0xFFFFu));
        x[2 * k + 1] = bits_f((uint16_t)(xl[k] >> 16));
        x[8 + 2 * k] = bits_f((uint16_t)(xh[k] & 0xFFFFu));
        x[8 + 2 * k + 1] = bits_f((uint16_t)(xh[k] >> 16));
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k) ss += (double)x[k] * (double)x[k];
    ss += dpp<kDppQuadSwap1>(ss);
    ss += dpp<kDppQuadSwap2>(ss);
    ss += dpp<kDppRowHalfMirror>(ss);
    const float rms = (float)sqrt(ss / 128.0 + 1e-6);
    const float y = __fdiv_rn(1.0f, rms);
    uint32_t hw[8];   // normalized halves as f16 pairs: [0,4) low half, [4,8) high half
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t gw = k < 4 ? gl[k] : gh[k - 4];
        const float h0 = __fadd_rn(__fmul_rn(div_markstein(x[2 * k], rms, y), bits_f((uint16_t)(gw & 0xFFFFu))), 0.0f);
        const float h1 = __fadd_rn(__fmul_rn(div_markstein(x[2 * k + 1], rms, y), bits_f((uint16_t)(gw >> 16))), 0.0f);
        hw[k] = __builtin_bit_cast(uint32_t, h2_pk{(_Float16)h0, (_Float16)h1});
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const h2_pk a = h2_of(hw[k]), b = h2_of(hw[4 + k]), c = h2_of(cw[k]), sn = h2_of(sw[k]);
        const h2_pk ac = a * c, bs = b * sn, bc = b * c, as = a * sn;
        yl[k] = __builtin_bit_cast(uint32_t, ac - bs);
        yh[k] = __builtin_bit_cast(uint32_t, bc + as);
    }
}

}  // namespace dev
}  // namespace gehtp
