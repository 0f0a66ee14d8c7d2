// k_w4g.hip — W4A16 group-64 kernels for gfx950: decode GEMV, prefill GEMM (MFMA), dequant.
//
// Weight format (OP_MATMUL_W4G_F16): wq row n = K/2 bytes, byte j holds k=2j in the
// low nibble and k=2j+1 in the high nibble, stored as q+8; ws[n][k/64] fp16.
// Dequant is fp16(q*s), RNE — computed as two exact packed-fp16 steps:
//   h = half(magic | nibble bits) = base + nib;  q = h - (base + 8) (exact);  w = q * s
// (one RNE). A nibble in mantissa bits 0-3 takes magic 0x6400 (base 1024, ulp 1); one
// in bits 4-7 takes 0x5400 (base 64, ulp 1/16), so it needs no shift.
//
// One 32-bit word of weights = 8 consecutive k. With w8 = w >> 8, masking w and w8
// with 0x000F000F and 0x00F000F0 gives the half pairs (k0,k4), (k1,k5), (k2,k6),
// (k3,k7); activations are staged in the same pair order so each pair feeds one
// v_dot2_f32_f16 (fp32 accumulate).
#include "dev_reduce.h"
#include "dev_rope.h"
#include "dev_w4g.h"
#include "kernels.h"

#include <algorithm>
#include <atomic>
#include <cmath>

namespace gehtp {

namespace {

// ---------------------------------------------------------------------------
// GEMV (M <= 4). A weight row is S = K/32 slices of 16 bytes (32 weights, half a
// scale group). P = S threads share a row, each owning one slice; R = nthreads/P rows
// are processed per pass and a workgroup runs np passes over its R*np contiguous rows.
// A thread's activation slice stays in registers (pair order) for the whole kernel,
// so the inner loop is global loads + dequant + v_dot2 with no LDS traffic. With up to
// 4 passes all weight loads are issued up front and each pass is computed when its own
// load lands; with more, the passes run in batches (of 4, or 5 for 10 passes) with the
// next batch's loads in flight while the current one is computed. Pass partials go to
// LDS and teams of 16, 32 or 64 lanes sum each row before the epilogue.
struct GemvArgs {
    const __half* x;
    uint32_t ldx;
    const uint8_t* wq;
    const __half* ws;
    __half* y;
    uint32_t ldy;
    uint32_t N, K, P, R, np;
    uint32_t red_floats;   // size of the partials region; normalized rows follow it
    const __half* gamma;
    const __half* res;
    uint32_t ldr;
    int swiglu;
};

// SwiGLU's silu (silu_f16_expr): its input is always an fp16 value, so the whole function
// is a table of 65536 fp16 results, filled once per device by silu_table_kernel with that
// same expression: a lookup gives the expression's bits for a fraction of its VALU work
// (the correctly rounded exp and division were ~5 % of the gate/up GEMM).
__device__ uint16_t g_silu_tab[65536];
__device__ __forceinline__ float silu_of(float gate_f16) { return h2f(g_silu_tab[f2hb(gate_f16)]); }

__global__ __launch_bounds__(256) void silu_table_kernel() {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    g_silu_tab[i] = silu_f16_expr((uint16_t)i);
}

constexpr int kGemvU = 4;   // passes per load batch (5 for the 10-pass form)
// Pass counts with a fully unrolled batch schedule; other counts above kGemvU run the
// batch loop and must be multiples of kGemvU.
__host__ __device__ constexpr bool gemv_static_np(uint32_t np) { return np == 8 || np == 10 || np == 12; }

template <int MR, int NP>
__global__ __launch_bounds__(512) void w4g_gemv_kernel(GemvArgs A) {
    constexpr int U = NP == 10 ? 5 : kGemvU;
    // Dynamic LDS: red = [np][MR][nt] pass partials, then (with gamma) the normalized
    // rows [MR][K] halves at a 16-byte aligned offset.
    extern __shared__ __align__(16) float red[];
    __shared__ double s_ss[8][MR];
    const uint32_t nt = blockDim.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t P = A.P, R = A.R;
    const uint32_t p = t % P, rr = t / P;
    const bool active = rr < R;
    const uint32_t rows_wg = R * A.np;
    // The host guarantees N >= rows_wg. The last workgroup is moved back to end at row N:
    // it overlaps its predecessor by `skip` rows, which it computes again (same bits) and
    // does not store. Every workgroup thus covers rows_wg rows and no load needs a
    // clamped index.
    const uint32_t r0n = blockIdx.x * rows_wg;
    const uint32_t r0 = min(r0n, A.N - rows_wg);
    const uint32_t skip = r0n - r0;
    const uint32_t RB = rows_wg;
    const uint32_t rowbytes = A.K / 2, G = A.K / 64, K8 = A.K / 8;
    const uint32_t nb = (A.np + U - 1) / U;

    // Every global load below is unconditional: a load under a divergent branch with a
    // zeroing else-path makes the compiler wait for each load before issuing the next.
    // Lanes past the workgroup's R rows per pass load row rr = 0; the reduction never
    // reads their partial sums. Each load is a workgroup-uniform base (advanced by a
    // uniform step per pass, scalar arithmetic) plus this thread's fixed 32-bit offset
    // (the host checks that one weight matrix spans less than 4 GiB). A scale is loaded
    // as its own 16-bit value and only widened to a pair where it is used.
    const uint32_t rrc = active ? rr : 0u;
    const uint8_t* wq0 = A.wq + (size_t)r0 * rowbytes;
    const uint16_t* ws0 = reinterpret_cast<const uint16_t*>(A.ws) + (size_t)r0 * G;
    const uint32_t w_off = rrc * rowbytes + p * 16, s_off = rrc * G + (p >> 1);
    auto load_pass = [&](uint32_t i, u32x4& w, uint32_t& s) {
        w = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(wq0 + (size_t)(i * R) * rowbytes + w_off));
        s = ws0[(size_t)(i * R) * G + s_off];
    };
    auto scale_of = [&](uint32_t word) -> _Float16 { return __builtin_bit_cast(_Float16, (uint16_t)word); };
    auto load_batch = [&](uint32_t b, u32x4 (&w)[U], uint32_t (&s)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) load_pass(b * U + u, w[u], s[u]);
    };

    // Activations first: loads complete in order, so the prologue waits only for these
    // (L2-resident) and not for the weight loads queued behind them.
    constexpr int PRE = 2;   // chunks of x and gamma per thread fetched up front
    u32x4 xr[MR][4];         // this thread's activation slice (32 values per row m)
    u32x4 xv[PRE][MR], gv[PRE];
    if (A.gamma) {
#pragma unroll
        for (int k = 0; k < PRE; ++k) {
            const uint32_t i = min(t + k * nt, K8 - 1);
#pragma unroll
            for (int m = 0; m < MR; ++m) xv[k][m] = reinterpret_cast<const u32x4*>(A.x + (size_t)m * A.ldx)[i];
            gv[k] = reinterpret_cast<const u32x4*>(A.gamma)[i];
        }
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                xr[m][c] = reinterpret_cast<const u32x4*>(A.x + (size_t)m * A.ldx)[p * 4 + c];
    }

    // Epilogue teams: TG 16-lane groups (1, 2 or 4, within one wave) sum each output
    // row, TG > 1 when the workgroup has fewer rows than groups; with SwiGLU a group sums
    // one gate/up pair. Team `team` writes output `team` first: its residual is fetched
    // now so the epilogue does not wait on a fresh global load.
    const uint32_t grp = t >> 4, ngrp = nt >> 4;
    const uint32_t n_out_wg = A.swiglu ? RB / 2 : RB, out0 = A.swiglu ? r0 / 2 : r0;
    const uint32_t TG = A.swiglu ? 1u : ngrp >= 4 * RB ? 4u : ngrp >= 2 * RB ? 2u : 1u;
    const uint32_t team = grp / TG, nteam = ngrp / TG, tl = t % (16 * TG), gl = t & 15;
    uint16_t res0[MR];
    if (A.res) {
        const uint32_t j = team < n_out_wg ? team : 0u;
#pragma unroll
        for (int m = 0; m < MR; ++m) res0[m] = __builtin_bit_cast(uint16_t, A.res[(size_t)m * A.ldr + out0 + j]);
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) res0[m] = 0;
    }

    // NP in 1..4: straight-line, every load issued here. NP = k*U (k > 1): k batches in a
    // fully unrolled ping-pong, so every wait counts exactly the loads it needs; NP = 0:
    // the same ping-pong as a loop over np / U batches.
    constexpr bool STRAIGHT = NP > 0 && NP <= U;
    constexpr int NB = NP > U ? NP / U : 0;
    constexpr int NPA = STRAIGHT ? NP : 1;
    u32x4 wa[U], wb[U], wall[NPA];
    uint32_t sa[U], sb[U], sall[NPA];
    if constexpr (STRAIGHT) {
#pragma unroll
        for (int i = 0; i < NP; ++i) load_pass(i, wall[i], sall[i]);
    } else {
        load_batch(0, wa, sa);
    }

    if (A.gamma) {
        // RMSNorm prologue, cooperative: sum of squares in double (as RMSNORM2_F16), then
        // h = f16(x / rms * gamma + 0) for the whole row into LDS.
        auto chunk_x = [&](int k, uint32_t i, int m) -> u32x4 {
            return k < PRE ? xv[k][m] : reinterpret_cast<const u32x4*>(A.x + (size_t)m * A.ldx)[i];
        };
        double ss[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) ss[m] = 0.0;
        for (uint32_t k = 0, i = t; i < K8; ++k, i += nt) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const u32x4 v = chunk_x((int)min(k, (uint32_t)PRE), i, m);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const double lo = (double)h2f((uint16_t)(v[e] & 0xFFFFu));
                    const double hi = (double)h2f((uint16_t)(v[e] >> 16));
                    ss[m] = __builtin_fma(lo, lo, ss[m]);   // lo*lo is exact: same bits as * then +
                    ss[m] = __builtin_fma(hi, hi, ss[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const double w = dev::wave_sum(ss[m]);
            if (lane == 0) s_ss[wave][m] = w;
        }
        __syncthreads();
        // Every thread adds the wave sums itself (same order everywhere), so no second
        // barrier is needed. x / rms is computed as Markstein's correction of x * y with
        // y = RN(1/rms): q = RN(x*y), r = fma(-q, rms, x) (exact), RN(q + r*y) — the
        // correctly rounded quotient, checked against IEEE division for every finite
        // fp16 x over thousands of divisors (signed zeros aside, which the + 0 below
        // maps to +0 either way).
        float rms[MR], rcp[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            double tot = 0.0;
            for (uint32_t w = 0; w < nt / 64; ++w) tot += s_ss[w][m];
            rms[m] = (float)sqrt(tot / (double)A.K + 1e-6);
            rcp[m] = __fdiv_rn(1.0f, rms[m]);
        }
        auto div_rms = [&](float a, int m) {
            const float q = a * rcp[m];
            return __builtin_fmaf(__builtin_fmaf(-q, rms[m], a), rcp[m], q);
        };
        u32x4* xn = reinterpret_cast<u32x4*>(red + A.red_floats);
        // 16-byte chunk i of a row sits at slot i ^ ((i >> 4) & 3): the reads below (lane p
        // takes chunks 4p .. 4p+3, one per instruction) then hit 64 distinct banks per 16
        // lanes instead of 4-way conflicting, and the writes (consecutive chunks) stay
        // conflict-free; K8 is a multiple of 8, so a row's slots stay in the row.
        auto xslot = [](uint32_t i) -> uint32_t { return i ^ ((i >> 4) & 3u); };
        for (uint32_t k = 0, i = t; i < K8; ++k, i += nt) {
            const u32x4 g4 = k < PRE ? gv[k] : reinterpret_cast<const u32x4*>(A.gamma)[i];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const u32x4 v = chunk_x((int)min(k, (uint32_t)PRE), i, m);
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float lo = div_rms(h2f((uint16_t)(v[e] & 0xFFFFu)), m);
                    float hi = div_rms(h2f((uint16_t)(v[e] >> 16)), m);
                    // RN(y * g) with -0 -> +0 as one fma with a +0 addend (see below)
                    lo = __builtin_fmaf(lo, h2f((uint16_t)(g4[e] & 0xFFFFu)), 0.0f);
                    hi = __builtin_fmaf(hi, h2f((uint16_t)(g4[e] >> 16)), 0.0f);
                    asm volatile("" : "+v"(lo), "+v"(hi));
                    o[e] = (uint32_t)f2hb(lo) | ((uint32_t)f2hb(hi) << 16);
                }
                xn[m * K8 + xslot(i)] = o;
            }
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < 4; ++c) xr[m][c] = xn[m * K8 + xslot(p * 4 + c)];
        if (A.red_floats == 0) __syncthreads();   // xn shares LDS with red
    }

    // Pair order of dequant_word: (x0,x4) (x1,x5) (x2,x6) (x3,x7) per 8-value word.
    uint32_t xs[MR][16];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4 v = xr[m][c];
            xs[m][4 * c + 0] = (v[0] & 0xFFFFu) | (v[2] << 16);
            xs[m][4 * c + 1] = (v[0] >> 16) | (v[2] & 0xFFFF0000u);
            xs[m][4 * c + 2] = (v[1] & 0xFFFFu) | (v[3] << 16);
            xs[m][4 * c + 3] = (v[1] >> 16) | (v[3] & 0xFFFF0000u);
        }

    auto compute_pass = [&](uint32_t i, const u32x4& wc, uint32_t sc) {
        const _Float16 sh = scale_of(sc);
        const h2_t s2 = {sh, sh};
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            h2_t d[4];
            dequant_word(wc[c], s2, d);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                acc[m] = __builtin_amdgcn_fdot2(d[0], as_h2(xs[m][4 * c + 0]), acc[m], false);
                acc[m] = __builtin_amdgcn_fdot2(d[1], as_h2(xs[m][4 * c + 1]), acc[m], false);
                acc[m] = __builtin_amdgcn_fdot2(d[2], as_h2(xs[m][4 * c + 2]), acc[m], false);
                acc[m] = __builtin_amdgcn_fdot2(d[3], as_h2(xs[m][4 * c + 3]), acc[m], false);
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) red[(i * MR + m) * nt + t] = acc[m];
    };
    auto compute_batch = [&](uint32_t b, const u32x4 (&wc)[U], const uint32_t (&sc)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) compute_pass(b * U + u, wc[u], sc[u]);
    };
    if constexpr (STRAIGHT) {
#pragma unroll
        for (int i = 0; i < NP; ++i) compute_pass(i, wall[i], sall[i]);
    } else if constexpr (NB > 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b & 1) {
                if (b + 1 < NB) load_batch(b + 1, wa, sa);
                compute_batch(b, wb, sb);
            } else {
                if (b + 1 < NB) load_batch(b + 1, wb, sb);
                compute_batch(b, wa, sa);
            }
        }
    } else {
        // Ping-pong over two register buffers: the next batch is in flight while one computes.
        for (uint32_t b = 0; b < nb; b += 2) {
            if (b + 1 < nb) load_batch(b + 1, wb, sb);
            compute_batch(b, wa, sa);
            if (b + 1 >= nb) break;
            if (b + 2 < nb) load_batch(b + 2, wa, sa);
            compute_batch(b + 1, wb, sb);
        }
    }
    __syncthreads();

    // Row sums over the teams, then the epilogue.
    auto res_at = [&](int m, uint32_t j) -> float {   // residual of output j of this workgroup
        return h2f(j == team ? res0[m] : __builtin_bit_cast(uint16_t, A.res[(size_t)m * A.ldr + out0 + j]));
    };
    if (!A.swiglu) {
        for (uint32_t lr = team; lr < RB; lr += nteam) {
            const uint32_t i = lr / R, base = (lr % R) * P;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float s = 0.0f;
                for (uint32_t k = tl; k < P; k += 16 * TG) s += red[(i * MR + m) * nt + base + k];
                s = dev::row_sum16(s);
                if (TG == 2) s = dev::pair_row_sum(s);
                if (TG == 4) s = dev::cross_row_sum(s);
                if (tl == 0 && lr >= skip) {
                    uint16_t v = f2hb(s);
                    if (A.res) v = f2hb(__fadd_rn(h2f(v), res_at(m, lr)));
                    reinterpret_cast<uint16_t*>(A.y)[(size_t)m * A.ldy + r0 + lr] = v;
                }
            }
        }
    } else {
        // rows (2k, 2k+1) = (gate, up) of output column (r0 + 2k) / 2; r0 and RB are even
        for (uint32_t k2 = grp; 2 * k2 < RB; k2 += ngrp) {
            const uint32_t lg = 2 * k2, lu = lg + 1;
            const uint32_t ig = lg / R, bg = (lg % R) * P, iu = lu / R, bu = (lu % R) * P;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float sg = 0.0f, su = 0.0f;
                for (uint32_t k = gl; k < P; k += 16) {
                    sg += red[(ig * MR + m) * nt + bg + k];
                    su += red[(iu * MR + m) * nt + bu + k];
                }
                sg = dev::row_sum16(sg);
                su = dev::row_sum16(su);
                if (gl == 0 && 2 * k2 >= skip) {
                    const float gv = h2f(f2hb(sg)), uv = h2f(f2hb(su));
                    // the expression rather than the table: a table read right after
                    // the kernel boundary would sit on this epilogue's short tail
                    const float act = h2f(silu_f16_expr(f2hb(gv)));
                    uint16_t v = f2hb(__fmul_rn(act, uv));
                    const uint32_t col = (r0 >> 1) + k2;
                    if (A.res) v = f2hb(__fadd_rn(h2f(v), res_at(m, k2)));
                    reinterpret_cast<uint16_t*>(A.y)[(size_t)m * A.ldy + col] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV for M = 1 with whole rows inside a wave: gemv_rw_body (dev_w4g.h), one workgroup
// per block of rows, x staged in dynamic LDS.
template <int C, int P, int NP, int PRE>
__global__ __launch_bounds__(512) void w4g_gemv_rw_kernel(GemvRwArgs A) {
    extern __shared__ __align__(16) float lds_rw[];   // x in pair order, padded layout
    __shared__ double s_ss[8];
    gemv_rw_body<C, P, NP, PRE>(A, blockIdx.x, blockDim.x, reinterpret_cast<u32x4*>(lds_rw), s_ss);
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
// Prefill GEMM: C[M,N] = A[M,K] . dequant(W)^T on v_mfma_f32_32x32x16_f16, with the B
// operand dequantized straight from global memory into registers. Lane l of a wave
// supplies B[k][n] for n = l%32 and 8 k's; with lane half h = l/32 owning bytes
// 16h..16h+15 of a weight row's 32-byte K step (64 k), one 16-byte load gives the 4
// words of the step's 4 MFMAs (word q: k = 32h + 8q + 0..7, dequantized in pair order
// (k0,k4)(k1,k5)(k2,k6)(k3,k7)). A goes through LDS with the same k assignment: each
// 16-byte chunk of an A row is stored in that pair order, so lane (row m = l%32, half h)
// reads the chunk at k = 32h + 8q for MFMA q. W never touches LDS.
// Workgroup tile 128 x 128, K step 64 (one scale group), 4 waves side by side in N,
// each 128 x 32 = 4 x 1 MFMA tiles (16 MFMAs per K step): every weight is dequantized
// once per workgroup, and the LDS carries only A (16 KiB written, 64 KiB read per K step).
// Three workgroups per CU (168 VGPRs); their barriers are independent, so one's LDS and
// load phases overlap another's MFMAs. Pipeline: global loads two K steps ahead in two
// register stages; during the MFMAs of step k, the dequantized B of step k+1 is built
// in the other B register set and the A chunks of step k+1 are written to the other LDS
// buffer; one barrier per K step. Loads are unconditional with clamped rows (rows past
// M or N are computed, never stored), which keeps the compiler from waiting on each
// load in turn.
// The 1-D grid runs m tiles fastest: workgroup i goes to XCD i % 8, so with 16 m tiles
// (M = 2048) every XCD keeps two bands of A in its L2 while W streams.
constexpr int WI = 4, GB_M = 32 * WI, GB_N = 128, GB_K = 64, GB_LDS = GB_K + 8;

// Output of one GEMM element pair: plain (two columns, each rounded to fp16, plus the
// residual) or SwiGLU (gate = column 2c, up = column 2c+1 -> output column c), the
// roundings of MATMUL_W4G followed by UNARY silu, BINARY mul and ADD.
__device__ __forceinline__ void w4g_store(__half* __restrict__ y, uint32_t ldy, const __half* __restrict__ res,
                                          uint32_t ldr, uint32_t row, uint32_t col, float acc) {
    uint16_t v = f2hb(acc);
    if (res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, res[(size_t)row * ldr + col]))));
    reinterpret_cast<uint16_t*>(y)[(size_t)row * ldy + col] = v;
}
__device__ __forceinline__ void w4g_store_swiglu(__half* __restrict__ y, uint32_t ldy, const __half* __restrict__ res,
                                                 uint32_t ldr, uint32_t row, uint32_t oc, float gate, float up) {
    const float gv = h2f(f2hb(gate)), uv = h2f(f2hb(up));
    const float act = silu_of(gv);
    uint16_t v = f2hb(__fmul_rn(act, uv));
    if (res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, res[(size_t)row * ldr + oc]))));
    reinterpret_cast<uint16_t*>(y)[(size_t)row * ldy + oc] = v;
}

// SwiGLU epilogue of a wave's WI x WJ accumulator tiles. Accumulator layout (32x32):
// lane l, reg r -> col l%32, row 8*(r/4) + 4*(l/32) + r%4. Columns 2c / 2c+1 (gate / up
// of output c) sit in lanes l, l^1; registers r, r+1 (r even) hold rows q, q+1. One
// exchange per register pair (the even lane hands over its row-(q+1) gate, the odd lane
// its row-q up, a DPP quad swap) lets the even lane finish row q and the odd lane row
// q+1. All silu
// lookups are issued before any store (a store through y could alias the table for the
// compiler, which would otherwise wait for each store before the next lookup).
template <int WI_, int WJ>
__device__ __forceinline__ void w4g_swiglu_tiles(f16x_t (&acc)[WI_][WJ], uint32_t lane, uint32_t m0, uint32_t col0,
                                                 uint32_t M, uint32_t N, __half* __restrict__ y, uint32_t ldy,
                                                 const __half* __restrict__ res, uint32_t ldr) {
    const bool odd = lane & 1;
    const uint32_t half = lane >> 5, l32 = lane & 31;
    uint16_t tb[WI_][WJ][8];
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const float got = dev::dpp<dev::kDppQuadSwap1>(odd ? acc[i][j][r] : acc[i][j][r + 1]);
                const float gate = odd ? got : acc[i][j][r];
                const float up = odd ? acc[i][j][r + 1] : got;
                acc[i][j][r] = gate;
                acc[i][j][r + 1] = up;
                tb[i][j][r / 2] = g_silu_tab[f2hb(gate)];
            }
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const uint32_t col = col0 + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const uint32_t rr = r + (odd ? 1 : 0);
                const uint32_t row = m0 + i * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
                if (col >= N || row >= M) continue;   // N is even: both lanes of a pair agree
                const uint32_t oc = col >> 1;
                uint16_t v = f2hb(__fmul_rn(h2f(tb[i][j][r / 2]), h2f(f2hb(acc[i][j][r + 1]))));
                if (res) v = f2hb(__fadd_rn(h2f(v), h2f(__builtin_bit_cast(uint16_t, res[(size_t)row * ldr + oc]))));
                reinterpret_cast<uint16_t*>(y)[(size_t)row * ldy + oc] = v;
            }
        }
}

// Plain epilogue of a wave's WI x WJ accumulator tiles: fp16 outputs (plus the residual)
// or, with `part`, fp32 split-K partials, one value per store (a lane-pair exchange that
// stores two adjacent columns at once measured 3-5 % slower on the 4B shapes).
template <int WI_, int WJ>
__device__ __forceinline__ void w4g_plain_tiles(const f16x_t (&acc)[WI_][WJ], uint32_t lane, uint32_t m0,
                                                uint32_t col0, uint32_t M, uint32_t N, __half* __restrict__ y,
                                                uint32_t ldy, const __half* __restrict__ res, uint32_t ldr,
                                                float* __restrict__ part, uint32_t split) {
    const uint32_t half = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const uint32_t col = col0 + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (col >= N || row >= M) continue;
                if (part) part[((size_t)split * M + row) * N + col] = acc[i][j][r];
                else w4g_store(y, ldy, res, ldr, row, col, acc[i][j][r]);
            }
        }
}

// Epilogue of the q|k|v GEMM that also performs OP_QK_ROPE_KV_F16 (W4gRope): the
// workgroup's 32 WT x 128 tile is head n0 / 128 of tokens m0 .. m0 + 32 WT - 1. Its fp16 outputs
// are staged in LDS (the A tiles' space) so that each 8-lane group holds one token's head
// row as the rows kernel's groups do, then finished with that kernel's arithmetic
// (dev::qk_row8_norm_rope, RoPE entries from the call's table): q heads to q_out, k
// heads (normalized, rotated) and v heads (as they are) to the ring slot of the token's
// position and to k_out / v_out; y is written as well, 16 bytes per store.
constexpr uint32_t kRopeSR = 128 + 8;   // staging row stride (halves)
template <int WT>
__device__ __forceinline__ void w4g_rope_tile(const f16x_t (&acc)[WT][1], uint32_t tid, uint32_t m0, uint32_t n0,
                                              uint32_t M, __half* __restrict__ y, uint32_t ldy, const W4gRope& R,
                                              _Float16* __restrict__ st) {
    const uint32_t lane = tid & 63, wave = tid >> 6, half = lane >> 5, l32 = lane & 31;
    __syncthreads();   // every wave's last MFMAs have read the A tiles
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            st[(i * 32 + 8 * (r >> 2) + 4 * half + (r & 3)) * kRopeSR + 32 * wave + l32] = (_Float16)acc[i][0][r];
    const uint32_t grp = tid >> 3, g = tid & 7, hh = n0 >> 7;
    const bool is_q = hh < R.H, is_k = !is_q && hh < R.H + R.KVH;
    u32x4 gl = {0u, 0u, 0u, 0u}, gh = {0u, 0u, 0u, 0u};
    if (is_q || is_k) {
        const __half* gm = is_q ? R.q_gamma : R.k_gamma;
        gl = *reinterpret_cast<const u32x4*>(gm + 8 * g);
        gh = *reinterpret_cast<const u32x4*>(gm + 64 + 8 * g);
    }
    const _Float16* cosp = static_cast<const _Float16*>(R.table);
    const _Float16* sinp = cosp + (size_t)M * 64;
    const uint32_t pos0 = *reinterpret_cast<const uint32_t*>(cosp + (size_t)M * 128);
    __syncthreads();
#pragma unroll
    for (uint32_t it = 0; it < WT; ++it) {
        const uint32_t r = grp + 32 * it, tok = m0 + r;
        if (tok >= M) break;   // the same for the 8 lanes of a group
        const u32x4 xl = *reinterpret_cast<const u32x4*>(&st[r * kRopeSR + 8 * g]);
        const u32x4 xh = *reinterpret_cast<const u32x4*>(&st[r * kRopeSR + 64 + 8 * g]);
        __half* yr = y + (size_t)tok * ldy + n0;
        *reinterpret_cast<u32x4*>(yr + 8 * g) = xl;
        *reinterpret_cast<u32x4*>(yr + 64 + 8 * g) = xh;
        __half* face = reinterpret_cast<__half*>(R.ring + (size_t)((pos0 + tok) % R.nslots) * R.slot_bytes);
        __half *d0, *d1;   // ring / q_out row, k_out / v_out row
        u32x4 ol = xl, oh = xh;
        if (is_q || is_k) {
            const u32x4 cw = *reinterpret_cast<const u32x4*>(cosp + (size_t)tok * 64 + 8 * g);
            const u32x4 sw = *reinterpret_cast<const u32x4*>(sinp + (size_t)tok * 64 + 8 * g);
            dev::qk_row8_norm_rope(xl, xh, gl, gh, cw, sw, ol, oh);
        }
        if (is_q) {
            d0 = R.q_out + ((size_t)tok * R.H + hh) * 128;
            d1 = nullptr;
        } else if (is_k) {
            const uint32_t kh = hh - R.H;
            d0 = face + kh * 128;
            d1 = R.k_out ? R.k_out + ((size_t)tok * R.KVH + kh) * 128 : nullptr;
        } else {
            const uint32_t vh = hh - R.H - R.KVH;
            d0 = face + (R.KVH + vh) * 128;
            d1 = R.v_out ? R.v_out + ((size_t)tok * R.KVH + vh) * 128 : nullptr;
        }
        *reinterpret_cast<u32x4*>(d0 + 8 * g) = ol;
        *reinterpret_cast<u32x4*>(d0 + 64 + 8 * g) = oh;
        if (d1) {
            *reinterpret_cast<u32x4*>(d1 + 8 * g) = ol;
            *reinterpret_cast<u32x4*>(d1 + 64 + 8 * g) = oh;
        }
    }
}

__device__ __forceinline__ u32x4 pair_order16(u32x4 v) {   // k0..k7 -> (k0,k4)(k1,k5)(k2,k6)(k3,k7)
    return u32x4{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                 __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
}

template <bool ROPE, int WT>
__global__ __launch_bounds__(256, 3) void w4g_gemm_kernel(
    const __half* __restrict__ a, uint32_t lda, const uint8_t* __restrict__ wq,
    const __half* __restrict__ ws, __half* __restrict__ y, uint32_t ldy, uint32_t M, uint32_t N,
    uint32_t K, const __half* __restrict__ res, uint32_t ldr, int swiglu, uint32_t mtiles, uint32_t ntiles,
    uint32_t split_steps, float* __restrict__ part, W4gRope rope) {
    constexpr int BM = 32 * WT;                    // workgroup tile rows (WT MFMA tiles per wave)
    constexpr int CA = BM * (GB_K / 8) / 256;      // 16-byte A chunks per thread per K step
    static_assert(!ROPE || (GB_N == 128 && kRopeSR <= 2 * GB_LDS), "rope staging tile");
    __shared__ __align__(16) _Float16 As[2][BM * GB_LDS];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Workgroup -> (m tile, n tile, K part): m fastest, K part slowest. With `part`,
    // K part s covers K steps [s*split_steps, (s+1)*split_steps) and its fp32 sums go to
    // part[s][M][N] for w4g_splitk_reduce_kernel; otherwise one part covers all of K.
    const uint32_t m0 = (blockIdx.x % mtiles) * BM, n0 = (blockIdx.x / mtiles % ntiles) * GB_N;
    const uint32_t split = blockIdx.x / (mtiles * ntiles);
    const uint32_t G = K / 64, rowbytes = K / 2;
    const uint32_t kbase = split * split_steps, nsteps = min(split_steps, K / GB_K - kbase);
    constexpr int WJ = 1;   // MFMA tiles per wave: WT (M) x WJ (N)
    const uint32_t wn = wave, half = lane >> 5, l32 = lane & 31;
    size_t wrow[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) wrow[j] = min(n0 + wn * 32 * WJ + j * 32 + l32, N - 1);
    const uint32_t arow = tid / 8, apiece = tid % 8;   // A chunk: rows arow + 32i, piece apiece

    u32x4 ra[2][CA], rw[2][WJ];
    uint16_t rs[2][WJ];
    auto load = [&](int st, uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const size_t r = min(m0 + arow + 32u * i, M - 1);
            ra[st][i] = *reinterpret_cast<const u32x4*>(a + r * lda + (kbase + kb) * GB_K + apiece * 8);
        }
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            rw[st][j] = *reinterpret_cast<const u32x4*>(wq + wrow[j] * rowbytes + (kbase + kb) * 32 + 16 * half);
            rs[st][j] = __builtin_bit_cast(uint16_t, ws[wrow[j] * G + kbase + kb]);
        }
    };
    auto store_a = [&](int st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CA; ++i)
            *reinterpret_cast<u32x4*>(&As[buf][(arow + 32 * i) * GB_LDS + apiece * 8]) = pair_order16(ra[st][i]);
    };
    h8_t bop[2][WJ][4];   // [B set][n block][MFMA q]
    auto dequant_b = [&](int st, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const _Float16 sh = __builtin_bit_cast(_Float16, rs[st][j]);
            const h2_t s2 = {sh, sh};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                h2_t d[4];
                dequant_word(rw[st][j][q], s2, d);
                bop[set][j][q] = h8_t{d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
            }
        }
    };

    f16x_t acc[WT][WJ];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto mfma = [&](int buf, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h8_t af[WT];
#pragma unroll
            for (int i = 0; i < WT; ++i)
                af[i] = *reinterpret_cast<const h8_t*>(&As[buf][(i * 32 + l32) * GB_LDS + 32 * half + 8 * q]);
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bop[set][j][q], acc[i][j], 0, 0, 0);
        }
    };

    // Step k: MFMAs on LDS buffer k%2 and B set k%2; loads of step k+2 into register
    // stage k%2 (its previous contents, step k, were consumed during step k-1); A and B
    // of step k+1 (register stage (k+1)%2) into LDS buffer / B set (k+1)%2. Past the
    // end the last step is loaded and stored again, unread (nothing conditional).
    const uint32_t last = nsteps - 1;
    load(0, 0);
    load(1, min(1u, last));
    store_a(0, 0);
    dequant_b(0, 0);
    __syncthreads();
    uint32_t kb = 0;
    for (; kb + 1 < nsteps; kb += 2) {
        load(0, min(kb + 2, last));
        __builtin_amdgcn_sched_barrier(0);
        mfma(0, 0);
        store_a(1, 1);
        dequant_b(1, 1);
        __syncthreads();
        load(1, min(kb + 3, last));
        __builtin_amdgcn_sched_barrier(0);
        mfma(1, 1);
        store_a(0, 0);
        dequant_b(0, 0);
        __syncthreads();
    }
    if (kb < nsteps) mfma(0, 0);   // odd step count: the last step is in buffer / set 0

    // Accumulator layout (32x32): lane l, reg r -> col l%32, row 8*(r/4) + 4*(l/32) + r%4.
    if constexpr (ROPE) {   // launched only for an unsplit plain q|k|v GEMM
        w4g_rope_tile(acc, tid, m0, n0, M, y, ldy, rope, &As[0][0]);
        return;
    }
    if (!part && swiglu) {
        w4g_swiglu_tiles(acc, lane, m0, n0 + wn * 32 * WJ, M, N, y, ldy, res, ldr);
        return;
    }
    w4g_plain_tiles(acc, lane, m0, n0 + wn * 32 * WJ, M, N, y, ldy, res, ldr, part, split);
}

// Wide variant for the wide-N shapes: a 128 x 256 workgroup tile, each wave 128 x 64
// (4 x 2 MFMA tiles), so every A fragment read from LDS feeds two MFMAs (half the LDS
// read traffic per MFMA of the 128 x 128 tile, whose A reads keep LDS as busy as the
// MFMAs keep the matrix pipes) while each weight is still dequantized once per 128
// rows. To fit two workgroups per CU (256 registers per lane, 128 of them
// accumulators), B is dequantized just before the MFMAs of each 16-deep sub-step
// instead of a whole K step ahead, raw W is held in three register stages (loaded two
// steps ahead) and A one step (loaded at the start of a step, stored to LDS after its
// MFMAs). The K order, operand layouts and MFMA sequence per output are those of
// w4g_gemm_kernel, so both kernels give the same bits.
constexpr int GW_WJ = 2;
constexpr uint32_t GW_N = 4 * 32 * GW_WJ;   // workgroup tile width

__global__ __launch_bounds__(256, 2) void w4g_gemm_wide_kernel(
    const __half* __restrict__ a, uint32_t lda, const uint8_t* __restrict__ wq,
    const __half* __restrict__ ws, __half* __restrict__ y, uint32_t ldy, uint32_t M, uint32_t N,
    uint32_t K, const __half* __restrict__ res, uint32_t ldr, int swiglu, uint32_t mtiles, uint32_t ntiles,
    uint32_t split_steps, float* __restrict__ part) {
    constexpr int CA = GB_M * (GB_K / 8) / 256;
    constexpr int WJ = GW_WJ;
    __shared__ __align__(16) _Float16 As[2][GB_M * GB_LDS];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = (blockIdx.x % mtiles) * GB_M, n0 = (blockIdx.x / mtiles % ntiles) * GW_N;
    const uint32_t split = blockIdx.x / (mtiles * ntiles);
    const uint32_t G = K / 64, rowbytes = K / 2;
    const uint32_t kbase = split * split_steps, nsteps = min(split_steps, K / GB_K - kbase);
    const uint32_t half = lane >> 5, l32 = lane & 31;
    size_t wrow[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) wrow[j] = min(n0 + wave * 32 * WJ + j * 32 + l32, N - 1);
    const uint32_t arow = tid / 8, apiece = tid % 8;
    const uint32_t last = nsteps - 1;

    u32x4 ra[CA], rw[3][WJ];
    uint16_t rs[3][WJ];
    auto load_a = [&](uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const size_t r = min(m0 + arow + 32u * i, M - 1);
            ra[i] = *reinterpret_cast<const u32x4*>(a + r * lda + (kbase + kb) * GB_K + apiece * 8);
        }
    };
    auto load_w = [&](int st, uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            rw[st][j] = *reinterpret_cast<const u32x4*>(wq + wrow[j] * rowbytes + (kbase + kb) * 32 + 16 * half);
            rs[st][j] = __builtin_bit_cast(uint16_t, ws[wrow[j] * G + kbase + kb]);
        }
    };
    auto store_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CA; ++i)
            *reinterpret_cast<u32x4*>(&As[buf][(arow + 32 * i) * GB_LDS + apiece * 8]) = pair_order16(ra[i]);
    };

    f16x_t acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Step kb: MFMAs on LDS buffer kb % 2 with the raw W of stage kb % 3; A of step kb + 1
    // and W of step kb + 2 (into stage (kb + 2) % 3, free since step kb - 1) are requested
    // first. Past the end the last step is loaded again, unread.
    auto step = [&](int buf, int st, int st2, uint32_t kb) __attribute__((always_inline)) {
        load_a(min(kb + 1, last));
        load_w(st2, min(kb + 2, last));
        __builtin_amdgcn_sched_barrier(0);
        h2_t s2[WJ];
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const _Float16 sh = __builtin_bit_cast(_Float16, rs[st][j]);
            s2[j] = h2_t{sh, sh};
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h8_t af[WI], bf[WJ];
#pragma unroll
            for (int i = 0; i < WI; ++i)
                af[i] = *reinterpret_cast<const h8_t*>(&As[buf][(i * 32 + l32) * GB_LDS + 32 * half + 8 * q]);
#pragma unroll
            for (int j = 0; j < WJ; ++j) {
                h2_t d[4];
                dequant_word(rw[st][j][q], s2[j], d);
                bf[j] = h8_t{d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
            }
#pragma unroll
            for (int i = 0; i < WI; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        store_a(buf ^ 1);
        __syncthreads();
    };

    load_w(0, 0);
    load_w(1, min(1u, last));
    load_a(0);
    store_a(0);
    __syncthreads();
    // Whole rounds of six steps (buffer and stage indices static, no exit inside a round,
    // so no load is moved past a branch), then up to five more.
    uint32_t kb = 0;
    for (; kb + 6 <= nsteps; kb += 6) {
#pragma unroll
        for (int u = 0; u < 6; ++u) step(u % 2, u % 3, (u + 2) % 3, kb + u);
    }
#pragma unroll
    for (int u = 0; u < 5; ++u)
        if (kb + u < nsteps) step(u % 2, u % 3, (u + 2) % 3, kb + u);
    if (!part && swiglu) {
        w4g_swiglu_tiles(acc, lane, m0, n0 + wave * 32 * WJ, M, N, y, ldy, res, ldr);
        return;
    }
    w4g_plain_tiles(acc, lane, m0, n0 + wave * 32 * WJ, M, N, y, ldy, res, ldr, part, split);
}

// Split-K finish, vector form (N, ldy, ldr multiples of 8, 16-byte aligned rows): a
// thread sums 8 consecutive fp32 columns over the parts in part order (two 16-byte loads
// per part) and stores 8 (plain) or 4 (SwiGLU) outputs at once, with the arithmetic of
// w4g_store / w4g_store_swiglu.
__global__ __launch_bounds__(256) void w4g_splitk_reduce8_kernel(const float* __restrict__ part, uint32_t parts,
                                                                 __half* __restrict__ y, uint32_t ldy, uint32_t M,
                                                                 uint32_t N, const __half* __restrict__ res,
                                                                 uint32_t ldr, int swiglu) {
    const uint32_t n8 = N / 8;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * n8) return;
    const uint32_t row = (uint32_t)(i / n8), c = 8 * (uint32_t)(i % n8);
    const float* p = part + (size_t)row * N + c;
    float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    for (uint32_t k = 1; k < parts; ++k) {
        p += (size_t)M * N;
        const float4 u = *reinterpret_cast<const float4*>(p), v = *reinterpret_cast<const float4*>(p + 4);
        a.x = __fadd_rn(a.x, u.x); a.y = __fadd_rn(a.y, u.y); a.z = __fadd_rn(a.z, u.z); a.w = __fadd_rn(a.w, u.w);
        b.x = __fadd_rn(b.x, v.x); b.y = __fadd_rn(b.y, v.y); b.z = __fadd_rn(b.z, v.z); b.w = __fadd_rn(b.w, v.w);
    }
    const float sum[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (!swiglu) {
        u32x4 rv = {0u, 0u, 0u, 0u};
        if (res) rv = *reinterpret_cast<const u32x4*>(res + (size_t)row * ldr + c);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint16_t lo = f2hb(sum[2 * e]), hi = f2hb(sum[2 * e + 1]);
            if (res) {
                lo = f2hb(__fadd_rn(h2f(lo), h2f((uint16_t)(rv[e] & 0xFFFFu))));
                hi = f2hb(__fadd_rn(h2f(hi), h2f((uint16_t)(rv[e] >> 16))));
            }
            o[e] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<u32x4*>(y + (size_t)row * ldy + c) = o;
    } else {
        const uint32_t oc = c / 2;
        uint32_t rv[2] = {0u, 0u};
        if (res) {
            const uint2 r2 = *reinterpret_cast<const uint2*>(res + (size_t)row * ldr + oc);
            rv[0] = r2.x; rv[1] = r2.y;
        }
        uint16_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float gv = h2f(f2hb(sum[2 * j])), uv = h2f(f2hb(sum[2 * j + 1]));
            const float act = silu_of(gv);
            uint16_t v = f2hb(__fmul_rn(act, uv));
            if (res) v = f2hb(__fadd_rn(h2f(v), h2f((uint16_t)(rv[j >> 1] >> (16 * (j & 1))))));
            o[j] = v;
        }
        *reinterpret_cast<uint2*>(y + (size_t)row * ldy + oc) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
    }
}

// Split-K finish fused with the RMSNorm of the finished rows (the next op's input): one
// workgroup per row, each thread finishing 8-column groups as w4g_splitk_reduce8_kernel
// does (plain epilogue) and keeping them in registers; then RMSNORM2_F16 without bias
// over the row as the decode GEMV's prologue computes it (squares of the fp16 row in
// double, rms = sqrt(sum / N + 1e-6) rounded to float, x / rms as Markstein's corrected
// quotient, times gamma, + 0, rounded to fp16) into xn [M, N].
constexpr uint32_t kRedNormG = 2;   // 8-column groups per thread: N <= 4096
__global__ __launch_bounds__(256) void w4g_splitk_reduce_norm_kernel(
    const float* __restrict__ part, uint32_t parts, __half* __restrict__ y, uint32_t ldy, uint32_t M, uint32_t N,
    const __half* __restrict__ res, uint32_t ldr, const __half* __restrict__ gamma, __half* __restrict__ xn) {
    __shared__ double s_ss;
    __shared__ __align__(16) u32x4 s_row[256 * kRedNormG];
    const uint32_t row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6, n8 = N / 8;
    u32x4 xv[kRedNormG];
#pragma unroll
    for (uint32_t j = 0; j < kRedNormG; ++j) {
        const uint32_t q = t + 256 * j;
        xv[j] = u32x4{0u, 0u, 0u, 0u};
        if (q >= n8) continue;
        const float* p = part + (size_t)row * N + 8 * q;
        float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
        for (uint32_t k = 1; k < parts; ++k) {
            p += (size_t)M * N;
            const float4 u = *reinterpret_cast<const float4*>(p), v = *reinterpret_cast<const float4*>(p + 4);
            a.x = __fadd_rn(a.x, u.x); a.y = __fadd_rn(a.y, u.y); a.z = __fadd_rn(a.z, u.z); a.w = __fadd_rn(a.w, u.w);
            b.x = __fadd_rn(b.x, v.x); b.y = __fadd_rn(b.y, v.y); b.z = __fadd_rn(b.z, v.z); b.w = __fadd_rn(b.w, v.w);
        }
        const float sum[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        u32x4 rv = {0u, 0u, 0u, 0u};
        if (res) rv = *reinterpret_cast<const u32x4*>(res + (size_t)row * ldr + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint16_t lo = f2hb(sum[2 * e]), hi = f2hb(sum[2 * e + 1]);
            if (res) {
                lo = f2hb(__fadd_rn(h2f(lo), h2f((uint16_t)(rv[e] & 0xFFFFu))));
                hi = f2hb(__fadd_rn(h2f(hi), h2f((uint16_t)(rv[e] >> 16))));
            }
            xv[j][e] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<u32x4*>(y + (size_t)row * ldy + 8 * q) = xv[j];
        s_row[q] = xv[j];
    }
    __syncthreads();
    // The sum of squares in exactly the order of the standalone RMSNORM2 kernel
    // (rmsnorm2_reg_kernel: lane l takes 8-value chunks l, l + 64, ... in turn, each value
    // squared and added in double, then the same wave reduction), so a row normalized here
    // and the same row normalized by that kernel are bit-identical.
    if (wave == 0) {
        double ss = 0.0;
        for (uint32_t q = lane; q < n8; q += 64) {
            const u32x4 v = s_row[q];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double f = (double)h2f((uint16_t)(v[e / 2] >> (16 * (e & 1))));
                ss += f * f;
            }
        }
        ss = dev::wave_sum(ss);
        if (lane == 0) s_ss = ss;
    }
    __syncthreads();
    const double tot = s_ss;
    const float rms = (float)sqrt(tot / (double)N + 1e-6);
    const float rcp = __fdiv_rn(1.0f, rms);
    auto norm = [&](uint16_t xb, uint16_t gb) {
        const float x = h2f(xb), qt = x * rcp;
        const float d = __builtin_fmaf(__builtin_fmaf(-qt, rms, x), rcp, qt);
        return f2hb(__fadd_rn(__fmul_rn(d, h2f(gb)), 0.0f));
    };
#pragma unroll
    for (uint32_t j = 0; j < kRedNormG; ++j) {
        const uint32_t q = t + 256 * j;
        if (q >= n8) continue;
        const u32x4 g4 = *reinterpret_cast<const u32x4*>(gamma + 8 * q);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)norm((uint16_t)(xv[j][e] & 0xFFFFu), (uint16_t)(g4[e] & 0xFFFFu)) |
                   ((uint32_t)norm((uint16_t)(xv[j][e] >> 16), (uint16_t)(g4[e] >> 16)) << 16);
        *reinterpret_cast<u32x4*>(xn + (size_t)row * N + 8 * q) = o;
    }
}

// Split-K finish: element pair (row, 2p..2p+1) sums the fp32 parts in part order and
// stores through the GEMM's own epilogue.
__global__ __launch_bounds__(256) void w4g_splitk_reduce_kernel(const float* __restrict__ part, uint32_t parts,
                                                                __half* __restrict__ y, uint32_t ldy, uint32_t M,
                                                                uint32_t N, const __half* __restrict__ res,
                                                                uint32_t ldr, int swiglu) {
    const uint32_t np = (N + 1) / 2;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * np) return;
    const uint32_t row = (uint32_t)(i / np), c = 2 * (uint32_t)(i % np);
    const bool two = c + 1 < N;
    const float* p = part + (size_t)row * N + c;
    float s0 = p[0], s1 = two ? p[1] : 0.0f;
    for (uint32_t k = 1; k < parts; ++k) {
        p += (size_t)M * N;
        s0 = __fadd_rn(s0, p[0]);
        if (two) s1 = __fadd_rn(s1, p[1]);
    }
    if (swiglu) {
        w4g_store_swiglu(y, ldy, res, ldr, row, c >> 1, s0, s1);
    } else {
        w4g_store(y, ldy, res, ldr, row, c, s0);
        if (two) w4g_store(y, ldy, res, ldr, row, c + 1, s1);
    }
}

}  // namespace

namespace {

// Fills this device's silu table before its first SwiGLU epilogue: the filling kernel
// goes on the caller's stream ahead of the GEMM / GEMV; outside stream capture the call
// then waits for it once, so launches on any stream find the table filled afterwards.
// Under capture the fill stays in the captured work (ordered before the epilogue there)
// and a later call fills it again. Concurrent first calls both write the same values.
hipError_t silu_table_ready(hipStream_t st) {
    static std::atomic<uint64_t> ready{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if ((ready.load(std::memory_order_acquire) >> dev) & 1u) return hipSuccess;
    hipLaunchKernelGGL(silu_table_kernel, dim3(65536 / 256), dim3(256), 0, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return hipSuccess;
    e = hipStreamSynchronize(st);
    if (e == hipSuccess) ready.fetch_or(1ull << dev, std::memory_order_release);
    return e;
}

// Launch shape of the GEMV for (M, K); see w4g_gemv_kernel.
struct GemvPlan {
    uint32_t nt = 0, P = 0, R = 0;
    bool ok = false;
};

GemvPlan gemv_plan(uint32_t M, uint32_t K) {
    GemvPlan best;
    if (M == 0 || M > kW4gGemvMaxM || K == 0 || K % 64 || (size_t)M * K * 2 > 65536) return best;
    const uint32_t P = K / 32;
    if (P > 512) return best;
    double best_score = -1.0;
    for (uint32_t nt = 64; nt <= 512; nt += 64) {
        if (nt < P) continue;
        const uint32_t R = nt / P;
        // fill of the thread block first, then blocks near 256 threads
        const double score = (double)(R * P) / nt * 1000.0 - std::abs((int)nt - 256) / 64.0;
        if (score > best_score) {
            best_score = score;
            best.nt = nt; best.P = P; best.R = R; best.ok = true;
        }
    }
    return best;
}

// Up to 4 passes per thread run the straight-line form (all weight loads issued before
// the RMSNorm prologue, each pass computed as soon as its own load has landed; measured
// 12.0 against 10.6 us for batches at the gate/up shape's 5-10 passes); 8, 10 and 12
// passes run unrolled two-buffer batch schedules, other counts the same as a loop.
template <int MR>
hipError_t gemv_dispatch(dim3 g3, dim3 b3, size_t lds, hipStream_t st, const GemvArgs& A) {
    if (A.np > (uint32_t)kGemvU && !gemv_static_np(A.np) && A.np % kGemvU) return hipErrorInvalidValue;
    switch (A.np <= 4 || gemv_static_np(A.np) ? A.np : 0u) {
    case 1: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 1>), g3, b3, lds, st, A); break;
    case 2: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 2>), g3, b3, lds, st, A); break;
    case 3: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 3>), g3, b3, lds, st, A); break;
    case 4: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 4>), g3, b3, lds, st, A); break;
    case 8: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 8>), g3, b3, lds, st, A); break;
    case 10: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 10>), g3, b3, lds, st, A); break;
    case 12: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 12>), g3, b3, lds, st, A); break;
    default: hipLaunchKernelGGL((w4g_gemv_kernel<MR, 0>), g3, b3, lds, st, A); break;
    }
    return hipGetLastError();
}

}  // namespace

bool w4g_gemv_supported(uint32_t M, uint32_t K) { return gemv_plan(M, K).ok; }

// Row-in-wave GEMV (M = 1): lanes per row P and slices per lane C for K, and the launch.
// Returns false (nothing launched) for the shapes it does not take.
template <int C, int P, int PRE = 2>
hipError_t gemv_rw_dispatch(uint32_t np, dim3 g3, dim3 b3, size_t lds, hipStream_t st, const GemvRwArgs& A) {
    if constexpr (C > 5) {   // one pass: two would not fit the registers
        if (np != 1) return hipErrorInvalidValue;
        hipLaunchKernelGGL((w4g_gemv_rw_kernel<C, P, 1, PRE>), g3, b3, lds, st, A);
    } else if (np == 1) {
        hipLaunchKernelGGL((w4g_gemv_rw_kernel<C, P, 1, PRE>), g3, b3, lds, st, A);
    } else {
        hipLaunchKernelGGL((w4g_gemv_rw_kernel<C, P, 2, PRE>), g3, b3, lds, st, A);
    }
    return hipGetLastError();
}

bool gemv_rw_launch(const GemvRwArgs& A, hipStream_t st, hipError_t* err) {
    if (A.K % 32) return false;
    const uint32_t S = A.K / 32, K8 = A.K / 8;
    uint32_t C, P;
    // (K = 9728 as 19 slices on 16 lanes ran the 4B down-projection in 6.50 us against
    // 5.87 us for the cross-wave kernel's three single-row workgroups per CU.)
    if (S % 16 == 0 && (S / 16 == 2 || S / 16 == 4 || S / 16 == 5)) { C = S / 16; P = 16; }
    else if (S % 32 == 0 && (S / 32 == 3 || S / 32 == 4)) { C = S / 32; P = 32; }
    else return false;
    const uint32_t pre = 2;   // chunks of x each thread stages
    // Workgroups of W waves (W = 5 and 7 leave one SIMD with an extra wave) running NP
    // passes of W * RW rows. The busiest CU sets the time, so the choice minimizes the
    // rows on the busiest CU (workgroups spread evenly), then the workgroup count (each
    // stages x, and normalizes it). Graph-timed on the 4B decode shapes against the
    // cross-wave kernel: q|k|v (N 6144, K 2560, RMSNorm; 256 workgroups of 3 waves, 2
    // passes) 4.31 against 5.43 us, o-proj (N 2560, K 4096, residual; 214 of 6 waves)
    // 3.58 against 3.90 us, gate/up (N 19456, K 2560, RMSNorm + SwiGLU; 1216 of 4 waves)
    // 8.89 against 10.09 us.
    const uint32_t RW = 64 / P, cus = (uint32_t)device_cu_count();
    uint32_t bW = 0, bNP = 0;
    uint64_t best_cu = ~0ull, best_wg = ~0ull;
    for (uint32_t W : {2u, 3u, 4u, 6u, 8u})
        for (uint32_t np = 1; np <= (C > 5 ? 1u : 2u); ++np) {
            const uint32_t rows = W * RW * np;
            if (rows > A.N || K8 > pre * 64 * W) continue;
            const uint64_t nwg = (A.N + rows - 1) / rows, per_cu = (nwg + cus - 1) / cus * rows;
            if (per_cu < best_cu || (per_cu == best_cu && nwg < best_wg)) {
                best_cu = per_cu; best_wg = nwg; bW = W; bNP = np;
            }
        }
    if (!bW) return false;
    const uint32_t rows_wg = bW * RW * bNP;
    const size_t lds = (size_t)K8 * 16;
    const dim3 g3((A.N + rows_wg - 1) / rows_wg), b3(64 * bW);
    if (P == 16)
        *err = C == 2 ? gemv_rw_dispatch<2, 16>(bNP, g3, b3, lds, st, A)
             : C == 4 ? gemv_rw_dispatch<4, 16>(bNP, g3, b3, lds, st, A)
                      : gemv_rw_dispatch<5, 16>(bNP, g3, b3, lds, st, A);
    else
        *err = C == 3 ? gemv_rw_dispatch<3, 32>(bNP, g3, b3, lds, st, A) : gemv_rw_dispatch<4, 32>(bNP, g3, b3, lds, st, A);
    return true;
}

hipError_t launch_w4g_gemv(const __half* x, uint32_t ldx, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi) {
    if (M == 0 || N == 0) return hipSuccess;
    if (epi.swiglu && (N & 1)) return hipErrorInvalidValue;
    const GemvPlan pl = gemv_plan(M, K);
    if (!pl.ok) {
        if (epi.gamma) return hipErrorInvalidValue;   // the engine normalizes before a GEMM
        return launch_w4g_gemm(x, ldx, wq, ws, y, ldy, M, N, K, st, epi);
    }
    // The kernel addresses weights by 32-bit offsets from a workgroup's first row.
    if ((uint64_t)N * (K / 2) >= (1ull << 32)) return hipErrorInvalidValue;
    if (M == 1) {
        hipError_t e = hipSuccess;
        if (gemv_rw_launch(GemvRwArgs{x, wq, ws, y, N, K, epi.gamma, epi.res, epi.swiglu ? 1 : 0}, st, &e)) return e;
    }
    // Rows per workgroup: about two workgroups per CU (three when one workgroup holds a
    // single row per pass, as for K = 9728: measured 11 % faster there, slower for the
    // multi-row shapes), partial sums within 32 KiB.
    const uint32_t target = (pl.R == 1 ? 3u : 2u) * (uint32_t)device_cu_count();
    uint32_t R = std::min(pl.R, N);   // rows per pass; a workgroup never spans more than N rows
    uint32_t np = (N + R * target - 1) / (R * target);
    const uint32_t np_max = std::max(1u, 8192u / (M * pl.nt));
    const uint32_t np_fit = std::min(np_max, N / R);
    np = std::max(1u, std::min(np, np_fit));
    // Other counts above kGemvU run the batch loop in whole batches of kGemvU. (The row
    // split matters more than wasted work: the busiest CUs set the time, so the gate/up
    // shape keeps 10 passes, 80 rows on a CU holding two workgroups, not 8 or 12 with 96.)
    if (np > (uint32_t)kGemvU && !gemv_static_np(np)) {
        const uint32_t up = (np + kGemvU - 1) / kGemvU * kGemvU;
        np = up <= np_fit ? up : np / kGemvU * kGemvU;
    }
    if (epi.swiglu && ((R * np) & 1)) {   // gate/up pairs never straddle workgroups (N is even)
        if (np > 1) --np;
        else if (2 * R <= N && 2 <= np_max) np = 2;
        else --R;                         // R odd >= 3 here
    }
    // Normalized rows after the partials when both fit in 64 KiB; otherwise they share
    // the start of LDS (red_floats = 0) and the kernel adds a barrier between them.
    const size_t red_b = ((size_t)np * M * pl.nt * 4 + 15) & ~(size_t)15;
    const size_t xn_b = epi.gamma ? (size_t)M * K * 2 : 0;
    const bool split = red_b + xn_b <= 65536;
    const size_t lds = split ? red_b + xn_b : std::max(red_b, xn_b);
    const uint32_t grid = (N + R * np - 1) / (R * np);
    GemvArgs A{x, ldx, wq, ws, y, ldy, N, K, pl.P, R, np, split ? (uint32_t)(red_b / 4) : 0u,
               epi.gamma, epi.res, epi.ldr, epi.swiglu ? 1 : 0};
    const dim3 g3(grid), b3(pl.nt);
    switch (M) {
    case 1: return gemv_dispatch<1>(g3, b3, lds, st, A);
    case 2: return gemv_dispatch<2>(g3, b3, lds, st, A);
    case 3: return gemv_dispatch<3>(g3, b3, lds, st, A);
    case 4: return gemv_dispatch<4>(g3, b3, lds, st, A);
    default: return hipErrorInvalidValue;
    }
}

// MFMA row tiles per wave (rows per workgroup / 32) of the 128-column kernel (nt counts
// a split's parts as further column tiles): 128-row tiles while that grid covers the CUs, else 64-row tiles while their grid
// exceeds half of them, else 32-row tiles. Each output's K order and MFMA sequence do
// not depend on the tile height, so all three give the same bits. Measured with idle
// CUs (M x N x K, us for 128 / 64 / 32 rows): 512 x 3072 x 1024 16.0 / 10.0 / 12.3,
// 512 x 4096 x 1024 16.0 / 10.0 / 12.3, 64 x 4096 x 1024 14.4 / 9.2 / 7.4; K in two
// parts, 512 x 1024 x 2048 (128 or 256 workgroups at 64 or 32 rows): 13.2 / 11.6.
static uint32_t narrow_tile_wt(uint32_t M, uint32_t nt) {
    const size_t cus = (size_t)device_cu_count();
    if ((size_t)((M + 127) / 128) * nt >= cus) return 4u;
    return (size_t)((M + 63) / 64) * nt * 2 > cus ? 2u : 1u;
}

hipError_t launch_w4g_gemm(const __half* a, uint32_t lda, const uint8_t* wq, const __half* ws,
                           __half* y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                           hipStream_t st, const W4gEpilogue& epi) {
    if (M == 0 || N == 0) return hipSuccess;
    if (epi.gamma || (epi.swiglu && (N & 1))) return hipErrorInvalidValue;
    if (epi.rope) {   // the q|k|v GEMM of OP_QK_ROPE_KV_F16: 128 x 128 tiles (one head each), unsplit
        const W4gRope& R = *epi.rope;
        auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
        if (epi.swiglu || epi.res || !R.H || !R.KVH || N != (R.H + 2 * R.KVH) * 128u || ldy % 8 || !al16(y) ||
            !al16(R.q_gamma) || !al16(R.k_gamma) || !al16(R.table) || !al16(R.q_out) || !al16(R.k_out) ||
            !al16(R.v_out) || !al16(R.ring) || R.slot_bytes % 16 || !R.nslots ||
            R.slot_bytes < R.KVH * 128u * 4u)
            return hipErrorInvalidValue;
        const uint32_t nt = N / GB_N, wt = narrow_tile_wt(M, nt);
        const uint32_t mt = (M + 32 * wt - 1) / (32 * wt);
        const auto kern = wt == 4 ? w4g_gemm_kernel<true, 4> : wt == 2 ? w4g_gemm_kernel<true, 2> : w4g_gemm_kernel<true, 1>;
        hipLaunchKernelGGL(kern, dim3(mt * nt), dim3(256), 0, st, a, lda, wq, ws, y, ldy, M, N, K, nullptr, 0u, 0, mt,
                           nt, K / GB_K, nullptr, R);
        return hipGetLastError();
    }
    if (epi.swiglu) {
        const hipError_t te = silu_table_ready(st);
        if (te != hipSuccess) return te;
    }
    const uint32_t mt = (M + GB_M - 1) / GB_M, nt = (N + GB_N - 1) / GB_N, steps = K / GB_K;
    const uint32_t ntw = (N + GW_N - 1) / GW_N;
    const uint32_t parts = w4g_gemm_split_parts(M, N, K);
    const size_t need = (size_t)parts * M * N * sizeof(float);
    const bool split = parts > 1 && epi.split_ws && epi.split_ws_bytes >= need;
    const uint32_t per = split ? (steps + parts - 1) / parts : steps;
    // Both tile shapes give the same bits. The wide one when its grid fills two rounds of
    // two workgroups per CU (measured at M = 2048: gate/up N = 19456 256 vs 263 us; with
    // fewer tiles, qkv N = 6144 and a two-part split of N = 2560, the 128 x 128 tile at
    // three per CU is 5-9 % faster) and for a three-part split, sized for it.
    const size_t cus = (size_t)device_cu_count();
    const bool wide = (size_t)mt * ntw * (split ? parts : 1u) >= 4 * cus ||
                      (split && parts == 3 && (size_t)6 * mt * ntw >= cus);
    // A split on the 128 x 128 kernel counts its parts as further column tiles.
    const uint32_t wt = wide ? 4u : narrow_tile_wt(M, split ? nt * parts : nt);
    auto narrow = [&](auto kern, uint32_t rows, float* pw) {
        const uint32_t mtn = (M + rows - 1) / rows;
        hipLaunchKernelGGL(kern, dim3(mtn * nt * (pw ? parts : 1u)), dim3(256), 0, st, a, lda, wq, ws, y, ldy, M, N, K,
                           epi.res, epi.ldr, epi.swiglu ? 1 : 0, mtn, nt, per, pw, W4gRope{});
    };
    auto gemm = [&](float* pw) {
        if (wide)
            hipLaunchKernelGGL(w4g_gemm_wide_kernel, dim3(mt * ntw * (pw ? parts : 1u)), dim3(256), 0, st, a, lda, wq,
                               ws, y, ldy, M, N, K, epi.res, epi.ldr, epi.swiglu ? 1 : 0, mt, ntw, per, pw);
        else if (wt == 4)
            narrow(w4g_gemm_kernel<false, 4>, 128u, pw);
        else if (wt == 2)
            narrow(w4g_gemm_kernel<false, 2>, 64u, pw);
        else
            narrow(w4g_gemm_kernel<false, 1>, 32u, pw);
    };
    if (split) {
        gemm(epi.split_ws);
        const uint32_t oal = epi.swiglu ? 4u : 8u;   // output elements per vector store
        const bool vec = N % 8 == 0 && ldy % oal == 0 && (uintptr_t)y % (2 * oal) == 0 &&
                         (!epi.res || (epi.ldr % oal == 0 && (uintptr_t)epi.res % (2 * oal) == 0)) &&
                         (uintptr_t)epi.split_ws % 16 == 0;
        const bool fuse_norm = vec && !epi.swiglu && epi.norm_gamma && epi.norm_out && N <= 256 * 8 * kRedNormG &&
                               (uintptr_t)epi.norm_gamma % 16 == 0 && (uintptr_t)epi.norm_out % 16 == 0;
        if (fuse_norm) {
            hipLaunchKernelGGL(w4g_splitk_reduce_norm_kernel, dim3(M), dim3(256), 0, st, epi.split_ws, parts, y, ldy,
                               M, N, epi.res, epi.ldr, epi.norm_gamma, epi.norm_out);
            if (epi.norm_done) *epi.norm_done = true;
        } else if (vec) {
            const size_t n8 = (size_t)M * (N / 8);
            hipLaunchKernelGGL(w4g_splitk_reduce8_kernel, dim3((uint32_t)((n8 + 255) / 256)), dim3(256), 0, st,
                               epi.split_ws, parts, y, ldy, M, N, epi.res, epi.ldr, epi.swiglu ? 1 : 0);
        } else {
            const size_t pairs = (size_t)M * ((N + 1) / 2);
            hipLaunchKernelGGL(w4g_splitk_reduce_kernel, dim3((uint32_t)((pairs + 255) / 256)), dim3(256), 0, st,
                               epi.split_ws, parts, y, ldy, M, N, epi.res, epi.ldr, epi.swiglu ? 1 : 0);
        }
        return hipGetLastError();
    }
    gemm(nullptr);
    return hipGetLastError();
}

// K is split when the 128 x 128 tile grid alone would give fewer than two workgroups
// per CU (three fit at once): the narrow-N projections (N = hidden) otherwise run one
// latency-bound workgroup on most CUs. Three parts of 16+ K steps when the 128 x 256
// grid of three parts fits one round at two workgroups per CU: on that tile when it
// also reaches half the CUs (M = 2048, N = 2560: 160 tiles, 480 workgroups; the o- and
// down-projections measured 2.4 % faster per prefill than two parts on the 128 x 128
// tile, whose A reads from LDS take as long as its MFMAs; M = 1024: 240 workgroups,
// 74.1 against 75.4 us on 128-row narrow tiles), else on the 128 x 128 kernel's shorter
// tiles (graph-timed, wide against narrow: M = 512, N = 1024, K = 3072 29.6 -> 15.0 us;
// M = 128, N = 2560, K = 9728 58.2 -> 24.6 us);
// otherwise two parts of 16+ steps on the 128 x 128 kernel.
uint32_t w4g_gemm_split_parts(uint32_t M, uint32_t N, uint32_t K) {
    const size_t mt = (M + GB_M - 1) / GB_M, cus = (size_t)device_cu_count();
    if (mt * ((N + GB_N - 1) / GB_N) >= 2 * cus) return 1u;
    if (K / GB_K >= 48 && 3 * mt * ((N + GW_N - 1) / GW_N) <= 2 * cus) return 3u;
    return K / GB_K >= 32 ? 2u : 1u;
}

size_t w4g_gemm_split_bytes(uint32_t M, uint32_t N, uint32_t K) {
    const uint32_t parts = w4g_gemm_split_parts(M, N, K);
    return parts > 1 ? (size_t)parts * M * N * sizeof(float) : 0;
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
