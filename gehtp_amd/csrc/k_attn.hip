// k_attn.hip — causal GQA attention for gfx950: flash prefill (MFMA) and split-KV decode.
//
// Prefill computes S^T = K . Q^T instead of Q . K^T so that each lane of a 32x32
// MFMA accumulator owns ONE query and 16 keys: the online-softmax row statistics
// then need a single cross-lane exchange (lane l <-> l^32) instead of a 32-lane
// reduction, and the rescale of the output accumulator is a per-lane scalar.
// O^T = V^T . P^T reuses P straight from the accumulator registers as the MFMA B
// operand; V is staged transposed in LDS so the A operand reads 8-byte runs.
#include "kernels.h"
#include "dev_reduce.h"
#include "dev_rope.h"
#include "dev_w4g.h"

#include <algorithm>
#include <atomic>
#include <cmath>

namespace gehtp {

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f16x_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int HD = 128;          // head dim this kernel is built for
constexpr int KT = 64;           // keys per LDS stage
constexpr int KS = HD + 8;       // K tile row stride (halves)
constexpr int VSR = HD + 32;     // V tile row stride (halves): 80 dwords, so the 4 rows x 64 bytes
                                 // that 32 lanes of a transposed read take hit 64 distinct banks
constexpr float kLog2e = 1.4426950408889634f;
// Buffer resource word 3 for raw dword loads on gfx9-family parts: data format 32
// (bits 15..18 = 4); a raw load past the resource's byte count returns zeros.
constexpr int kBufDword3 = 0x00020000;

typedef short s4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, output lane l receives
// element l%4 of the 8-byte chunks addressed by lanes l/4, l/4+4, l/4+8, l/4+12.
__device__ __forceinline__ u32x2 lds_read_tr16(const _Float16* p) {
    const s4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4_t*)(const_cast<_Float16*>(p)));
    return __builtin_bit_cast(u32x2, r);
}

// Flash attention forward. A workgroup owns 32 WPH queries of one head (wave w of a
// half: queries 32w..32w+31; WPH = 4 normally, 2 when 128-query tiles would leave CUs
// idle, 1 when 64-query tiles would too); per 64-key stage, K and V are staged row-major in LDS (the next stage's
// loads are in flight during the compute). Scores are computed transposed,
// S^T = K Q^T (MFMA A = K rows, B = Q^T held in registers), so each lane owns one query
// and its 32 scores of a stage; the online-softmax statistics need one exchange with
// lane l^32. O^T = V^T P^T: the V^T operand comes from the row-major V tile through the
// transposing LDS read, P^T straight from the score registers.
//
// The online softmax keeps a lazily moved reference max (see the stage code) and sums
// the fp16 weights P.V consumes; K / V stage rows come in through buffer loads.
//
// Two halves of WPH waves split a tile's key stages: half p runs stages
// [p*ns0, min(ns, (p+1)*ns0)) (ns0 = ceil(ns/2)) on its own LDS tiles, both halves in
// lockstep (the shorter one idles through its last step), and half 1 hands its partial
// (O, max, sum) to half 0 through LDS at the end. A causal tile then costs half its
// stages: the heaviest tiles no longer set the kernel's time (the grid runs the heavy
// tiles of every head first, one 8-wave workgroup per CU, the light ones behind them).
constexpr uint32_t KV_HALF = KT * KS + KT * VSR;   // halves of one LDS K + V stage

template <bool CAUSAL, int WPH>
__global__ __launch_bounds__(128 * WPH) void attn_prefill_kernel(
    const __half* __restrict__ q, uint32_t ldq, uint32_t qhs, const __half* __restrict__ k,
    const __half* __restrict__ v, uint32_t ldkv, uint32_t kvhs, __half* __restrict__ out, uint32_t ldo,
    uint32_t ohs, uint32_t S, uint32_t H, uint32_t KVH, float scale_log2) {
    // 8-wave tiles double-buffer the stages (one workgroup per CU either way); smaller
    // workgroups keep one buffer, so that two of them still fit a CU's LDS.
    constexpr bool DB = WPH == 4;
    __shared__ __align__(16) _Float16 kvbuf[(DB ? 2 : 1) * 2 * KV_HALF];   // [stage buffer][half]
    constexpr uint32_t QT = 32 * WPH, NT = 64 * WPH;   // queries per tile, threads per half
    constexpr int KR = KT * 16 / NT;                     // K / V rows per thread per stage
    const uint32_t part = __builtin_amdgcn_readfirstlane(threadIdx.x / NT), tid = threadIdx.x % NT, lane = tid & 63,
                   wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    _Float16* const Ks0 = kvbuf + part * KV_HALF;   // stage buffer b at + 2 * b * KV_HALF
    const uint32_t n_qt = (S + QT - 1) / QT;
    const uint32_t qtile = n_qt - 1 - blockIdx.y;      // heaviest causal tiles first
    const uint32_t h = blockIdx.x;
    const uint32_t kvh = h / (H / KVH);
    const uint32_t q0 = qtile * QT;
    const uint32_t qw = q0 + wave * 32;                 // this wave's first query
    const uint32_t my_q = qw + (lane & 31);
    const uint32_t hl = lane >> 5;

    // Q^T fragments (MFMA B operand): query my_q, dims 16*kk + 8*hl + [0,8). Queries past
    // S read row S-1 (their outputs are not stored).
    h8_t qf[HD / 16];
    {
        const size_t qrow = min(my_q, S - 1);
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk)
            qf[kk] = *reinterpret_cast<const h8_t*>(q + qrow * ldq + (size_t)h * qhs + kk * 16 + hl * 8);
    }

    f16x_t o[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    const uint32_t kend = CAUSAL ? min(S, q0 + QT) : S;
    // K and V rows of this thread's KR keys (stage-local key (tid>>4) + (NT/16)i, dims 8*ch..),
    // read as buffer loads whose resource spans the stage's rows below S: rows past S
    // read as zeros (their scores are masked), and the per-thread byte offsets are fixed,
    // so a stage's addresses cost scalar instructions only (kb < S, and the resource's
    // byte count, at most KT rows, fits 32 bits for any row pitch below 2^25 halves).
    const uint32_t ch = tid & 15;
    u32x4 kv4[KR], vv4[KR];
    const __half* const kh = k + (size_t)kvh * kvhs;
    const __half* const vh = v + (size_t)kvh * kvhs;
    uint32_t voff[KR];
#pragma unroll
    for (int i = 0; i < KR; ++i) voff[i] = (((tid >> 4) + (NT / 16) * i) * ldkv + ch * 8) * 2;
    auto load_kv = [&](uint32_t kb) {
        const uint32_t nrec = min(S - kb, (uint32_t)KT) * ldkv * 2;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kh + (size_t)kb * ldkv), 0, nrec, kBufDword3);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void*)(vh + (size_t)kb * ldkv), 0, nrec, kBufDword3);
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            kv4[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, voff[i], 0, 0));
            vv4[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff[i], 0, 0));
        }
    };
    // This lane's address pattern for the transposed V reads (see lds_read_tr16): source
    // row 4*hl + (lane%16)/4 (+ 16j, + 8 for the second half), column
    // 16*((lane/16)%2) + 4*(lane%4) (+ 32*dt).
    const uint32_t tr_row = 4 * hl + ((lane & 15) >> 2);
    const uint32_t tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    const uint32_t ns = (kend + KT - 1) / KT, ns0 = (ns + 1) / 2;
    const uint32_t st0 = part * ns0, st1 = min(ns, st0 + ns0);   // this half's stages
    const uint32_t klast = st1 > st0 ? min(st1 * KT, kend) - 1 : kend - 1;
    // With two LDS stage buffers, stage it is computed from buffer it % 2 while the
    // registers hold stage it + 1, written to the other buffer after the compute: one
    // barrier per stage (the other buffer was last read in stage it - 1, before the
    // previous barrier). With one buffer, a barrier before the write as well.
    auto stage_kv = [&](uint32_t b) __attribute__((always_inline)) {
        _Float16* const Kd = Ks0 + 2 * b * KV_HALF;
        _Float16* const Vd = Kd + KT * KS;
#pragma unroll
        for (int i = 0; i < KR; ++i) {
            const uint32_t key = (tid >> 4) + (NT / 16) * i;
            *reinterpret_cast<u32x4*>(&Kd[key * KS + ch * 8]) = kv4[i];
            *reinterpret_cast<u32x4*>(&Vd[key * VSR + ch * 8]) = vv4[i];
        }
    };
    load_kv(min(st0 * KT, kend - 1));
    // One stage of this wave: keys kb .. kb + KT - 1 from the K / V tiles at Ks / Vs.
    auto stage_compute = [&](const _Float16* Ks, const _Float16* Vs, uint32_t kb) __attribute__((always_inline)) {
        // Scores of the stage's two 32-key halves: two independent MFMA chains, all K
        // fragments read first.
        f16x_t s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) { s0[r] = 0.0f; s1[r] = 0.0f; }
        // K fragments are requested two MFMA pairs ahead (the group barriers below hold
        // the scheduler to that order).
        h8_t kf0[HD / 16], kf1[HD / 16];
        auto kread = [&](int kk) __attribute__((always_inline)) {
            kf0[kk] = *reinterpret_cast<const h8_t*>(&Ks[(lane & 31) * KS + kk * 16 + hl * 8]);
            kf1[kk] = *reinterpret_cast<const h8_t*>(&Ks[(32 + (lane & 31)) * KS + kk * 16 + hl * 8]);
        };
        kread(0);
        kread(1);
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
            if (kk + 2 < HD / 16) kread(kk + 2);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf0[kk], qf[kk], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf1[kk], qf[kk], s1, 0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        // s0[r] / s1[r]: key kb (+32) + 8*(r/4) + 4*hl + r%4, query my_q. Scores stay raw
        // (the launcher guarantees scale > 0, so max commutes with the scaling); a stage
        // wholly below the diagonal and inside S skips the mask (a wave-uniform test).
        // The first P.V group's V^T operands are requested before the softmax runs.
        u32x4 vpre[HD / 32];
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt) {
            const _Float16* base = &Vs[tr_row * VSR + 32 * dt + tr_col];
            const u32x2 lo = lds_read_tr16(base);
            const u32x2 hi = lds_read_tr16(base + 8 * VSR);
            vpre[dt] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
        const bool full = kb + KT <= S && (!CAUSAL || kb + KT - 1 <= qw);
        // (scores are finite or -inf: the max is three-input v_max3 without NaN quieting)
        float mloc = -INFINITY;
        if (!full) {   // key kb + 4*hl + c is valid iff c <= lim
            const int lim = (int)(CAUSAL ? min(my_q, S - 1) : S - 1) - (int)(kb + 4 * hl);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int c = 8 * (r >> 2) + (r & 3);
                if (c > lim) s0[r] = -INFINITY;
                if (c + 32 > lim) s1[r] = -INFINITY;
            }
        }
        {   // a max3 tree over the 32 scores (depth 4 instead of a 16-long chain)
            float t1[12];
#pragma unroll
            for (int i = 0; i < 10; ++i) {
                const int a = 3 * i, b = 3 * i + 1, c = 3 * i + 2;
                t1[i] = dev::max3_nonan(a < 16 ? s0[a] : s1[a - 16], b < 16 ? s0[b] : s1[b - 16], c < 16 ? s0[c] : s1[c - 16]);
            }
            t1[10] = s1[14];
            t1[11] = s1[15];
            const float u0 = dev::max3_nonan(t1[0], t1[1], t1[2]), u1 = dev::max3_nonan(t1[3], t1[4], t1[5]);
            const float u2 = dev::max3_nonan(t1[6], t1[7], t1[8]), u3 = dev::max3_nonan(t1[9], t1[10], t1[11]);
            mloc = dev::max3_nonan(dev::max3_nonan(u0, u1, u2), u3, mloc);
        }
        {   // the other half of this query's keys sits in lane l ^ 32
            uint32_t x0 = __builtin_bit_cast(uint32_t, mloc), x1 = x0;
            dev::permlane32_swap(x0, x1);
            mloc = fmaxf(__builtin_bit_cast(float, x0), __builtin_bit_cast(float, x1));
        }
        const float m_top = fmaxf(m_run, mloc);
        // Lazy rescaling: the reference max m_run moves only when this stage's max exceeds
        // it by more than 8 in log2 units, so P stays below 2^8 (fp16 holds it) and O is
        // rescaled in a few stages instead of almost every one. (m_top - m_run is NaN when
        // both are -inf: no move.) The sum and O share the reference, so it cancels in O / l.
        const bool grow = (m_top - m_run) * scale_log2 > 8.0f;
        const float m_new = grow ? m_top : m_run;
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float neg_ms = -m_use * scale_log2;
        // v_exp_f32 directly: results below 2^-126 flush to 0, which a softmax weight can
        // afford. p = 2^((s - m) * scale_log2) with the scaling folded into one fma.
        const float alpha = grow ? __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, scale_log2, neg_ms)) : 1.0f;
        // P^T operand j (keys 16j .. 16j+15 of the stage): k-slot i of lane-half hl holds
        // key 16j + 8*(i/4) + 4*hl + i%4, i.e. score register 8*(j%2) + i of s0 / s1.
        // The row sum adds the fp16 weights that P.V uses, two per v_dot2_f32_f16.
        typedef _Float16 h2v_t __attribute__((ext_vector_type(2)));
        typedef float f2v_t __attribute__((ext_vector_type(2)));
        const h2v_t ones = {(_Float16)1.0f, (_Float16)1.0f};
        h8_t pb[4];
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 8 * (j & 1) + 2 * e;
                const float a = j < 2 ? s0[r] : s1[r], b = j < 2 ? s0[r + 1] : s1[r + 1];
                const f2v_t f = {__builtin_amdgcn_exp2f(__builtin_fmaf(a, scale_log2, neg_ms)),
                                 __builtin_amdgcn_exp2f(__builtin_fmaf(b, scale_log2, neg_ms))};
                const h2v_t hp = __builtin_convertvector(f, h2v_t);
                ls[j] = __builtin_amdgcn_fdot2(hp, ones, ls[j], false);
                w[e] = __builtin_bit_cast(uint32_t, hp);
            }
            pb[j] = __builtin_bit_cast(h8_t, w);
        }
        float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
        {
            uint32_t x0 = __builtin_bit_cast(uint32_t, lsum), x1 = x0;
            dev::permlane32_swap(x0, x1);
            lsum = __builtin_bit_cast(float, x0) + __builtin_bit_cast(float, x1);
        }
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        if (__any(grow)) {
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        // O^T[d][q] += sum_key V^T[d][key] P^T[key][q]: for each 32-dim block and each
        // 16-key group j, two transposed reads give keys 16j + 4*hl + [0,4) and +8.
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16* base = &Vs[(16 * j + tr_row) * VSR + 32 * dt + tr_col];
                u32x4 packed;
                if (j == 0) {
                    packed = vpre[dt];
                } else {
                    const u32x2 lo = lds_read_tr16(base);
                    const u32x2 hi = lds_read_tr16(base + 8 * VSR);
                    packed = u32x4{lo[0], lo[1], hi[0], hi[1]};
                }
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, packed), pb[j], o[dt], 0, 0, 0);
            }
        }
    };
    // A stage runs unless it is the shorter half's idle step or wholly masked for this wave.
    auto active = [&](uint32_t it, uint32_t kb) { return st0 + it < st1 && !(CAUSAL && kb > qw + 31); };
    if constexpr (DB) {
        stage_kv(0);
        load_kv(min(st0 * KT + KT, klast));
        __syncthreads();
        for (uint32_t it = 0; it < ns0; ++it) {
            const uint32_t kb = (st0 + it) * KT;
            const _Float16* const Ks = Ks0 + 2 * (it & 1) * KV_HALF;
            if (active(it, kb)) stage_compute(Ks, Ks + KT * KS, kb);
            if (it + 1 < ns0) {
                stage_kv((it + 1) & 1);
                load_kv(min(kb + 2 * KT, klast));
            }
            __syncthreads();
        }
    } else {
        for (uint32_t it = 0; it < ns0; ++it) {
            const uint32_t kb = (st0 + it) * KT;
            __syncthreads();
            stage_kv(0);
            __syncthreads();
            load_kv(min(kb + KT, klast));
            if (active(it, kb)) stage_compute(Ks0, Ks0 + KT * KS, kb);
        }
    }

    // Half 1 hands (O, max, sum) to half 0 through the K/V tiles (lane-major floats: 66
    // per lane, 64 lanes x WPH waves); half 0 rescales both to the common max.
    __syncthreads();
    float* xch = reinterpret_cast<float*>(kvbuf);
    const uint32_t xl = wave * 64 + lane;
    if (part == 1) {
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) xch[(dt * 16 + r) * NT + xl] = o[dt][r];
        xch[64 * NT + xl] = m_run;
        xch[65 * NT + xl] = l_run;
    }
    __syncthreads();
    if (part == 1) return;
    {
        const float m1 = xch[64 * NT + xl], l1 = xch[65 * NT + xl];
        const float m = fmaxf(m_run, m1);
        const float a0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - m) * scale_log2);
        const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m1 - m) * scale_log2);
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * a0 + xch[(dt * 16 + r) * NT + xl] * a1;
        l_run = l_run * a0 + l1 * a1;
    }
    if (my_q < S) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        __half* orow = out + (size_t)my_q * ldo + (size_t)h * ohs;
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
// Decode, pass 1: workgroup (chunk c, kv head g) handles keys [64c, 64c+64) for the REP
// query heads of g, reading each K/V row once; all K and V loads of the chunk are
// issued before any arithmetic, so a chunk costs one memory round trip. Partials
// (O[128], max, sum) go to the workspace. Pass 2 (attn_merge_kernel) combines the
// chunks of each query head with the log-sum-exp rule. Two launches instead of a
// "last workgroup merges" scheme: on gfx950 the device-scope fence that scheme needs
// writes back and invalidates the whole L2 in every workgroup.
//
// FUSED (OP_ATTN_DECODE_QKV_F16): q, k and v of the new token come raw from the fused
// QKV row. Each workgroup applies QK-RMSNorm + RoPE to its REP query heads itself (the
// arithmetic of qk_rope_kv_kernel, so the bits match), and the workgroup whose chunk
// holds the new position also normalizes/rotates k of head g, writes k and v into the
// ring slot and uses them for that key. The position is the state's device counter;
// the merge pass advances it. The RoPE cos/sin (fp64 pow, cos, sin per lane) are the
// slow part of that prologue, so an extra workgroup of the merge pass computes them
// for this call's position and the next one into two workspace records, each tagged
// with (position + 1, theta): the next layer of the same step (one workspace serves
// every layer) or the next step of the same layer (one workspace per layer) finds its
// values there; a call that finds neither (the first after a prefill or a reset)
// computes its own. A record is a pure function of its tag, so the bits are the same
// either way.
constexpr int DC = 64;          // keys per chunk
constexpr int MAX_REP = 8;
constexpr int PS = HD + 4;      // partial record: O[HD], m, l, 2 pad (16-byte aligned)
// Workspace head (uint32 words): [0] second call sequence number of the fused calls
// (advanced by qkv_attn_decode_kernel; tags the attention-output records of
// merge_oproj_kernel); [1] n_kv of the last fused call; [2] call sequence number of the
// fused calls (advanced by their merge pass; tags the q|k|v hand-off records, see
// qkv_attn_decode_kernel); [3] nonzero once a hand-off wait gave up;
// RoPE records j = 0, 1: [4 + j] position + 1 (0 = empty), [6 + j] theta bits,
// [8 + 64j + i] pair i as f16 cos | f16 sin << 16. Partials follow the head.
constexpr uint32_t kWsSeqB = 0, kWsSnap = 1, kWsSeq = 2, kWsErr = 3, kWsRopeTag = 4, kWsRopeTheta = 6, kWsRope = 8;
constexpr uint32_t kWsHead = kWsRope + HD;

struct DecodeArgs {
    const __half* q;         // [H, HD] ready queries (plain op)
    const __half* qkv;       // fused: [q | k | v] row of the new token
    const __half* qg;        // fused: q / k RMSNorm gammas [HD]
    const __half* kg;
    float theta;             // fused: RoPE base
    uint8_t* ring;
    uint32_t slot_bytes, nslots, KVH, H;
    uint32_t n_kv_host;      // used when count is null
    uint32_t* count;         // device position counter (plain op: n_kv = *count)
    float scale_log2;
    float* part;             // partials [KVH][max_chunks][REP][PS]
    uint32_t max_chunks;
    uint32_t* ws;            // fused: workspace head (snapshot, RoPE records)
    // Additive mask (plain op only, may be null): row h (query head) at mask + h * mask_hs
    // (mask_hs = P, or 0 for one row shared by every head), one value per position of a
    // gathered layout of P positions; positions [n_kv, P) hold zero K/V there, so they
    // score the mask value alone (added by the merge pass).
    const __half* mask;
    uint32_t P;
    uint32_t mask_hs;
    uint32_t spec_chunks;    // chunks whose keys are known to lie below the count
    uint32_t kv_naps;        // hand-off form: s_sleep(4) steps before the K/V rows are requested
};

// MFMA operand layouts of v_mfma_f32_16x16x32_f16 (lane l, column lc = l % 16, row group
// lr = l / 16): A (16 x 32) row lc, k = 8lr .. 8lr+7; B (32 x 16) column lc, the same k;
// D (16 x 16, four floats) rows 4lr .. 4lr+3, column lc.
//
// The four waves stage the chunk's K and V rows (16 keys each) in LDS and apply the
// query heads' norm + RoPE; then one wave does the arithmetic and the others leave.
// Scores S^T = K . Q^T: the 64 keys as four 16-row A tiles, the REP query heads as B
// columns (zero past REP), four dims steps of 32. Each lane then holds the 16 scores
// (keys 16t + 4lr + i) of head lc, so the chunk's max and sum take two cross-row steps.
// P . V runs transposed, O^T = V^T . P^T: step j's B operand is the probabilities of
// tiles 2j and 2j+1 as the registers hold them, rounded to fp16 (k index 8lr + i <->
// key 32j + 4lr + i, 8lr + 4 + i <-> key 32j + 16 + 4lr + i); the A operand (dim 16u +
// lc, the same keys) comes from the row-major V tile through the transposing LDS read,
// each lane pointing at the 8-byte piece (key 32j + 4lr + lc/4, dims 16u + 4(lc%4) ..)
// so that lane lc receives element lc%4 of the pieces of lanes lc/4 + 4i.
constexpr int VSD = HD + 16;   // V tile row stride (halves): a 32-lane transposed read hits 64 banks
constexpr int KSD = HD + 8;    // K tile row stride (halves): 16 rows of a 16-byte access hit 64 banks
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float cross_row_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    dev::permlane32_swap(a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = __builtin_bit_cast(uint32_t, v);
    b = a;
    dev::permlane16_swap(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// LDS of one chunk workgroup. raw: the new token's REP q rows, then its k and v rows of
// head g, as f16 pairs (hand-off form only).
template <int REP>
struct DecodeSmem {
    __align__(16) _Float16 v[DC * VSD];
    __align__(16) _Float16 kt[DC * KSD];
    __align__(16) _Float16 q[REP][HD];
    __align__(16) _Float16 k[HD];
    __align__(16) uint32_t raw[(REP + 2) * HD / 2];
};

// Chunk c of kv head g. HO (hand-off, FUSED only): the new token's q|k|v row is not read
// from A.qkv but from the row-pair records rec[] that the q|k|v GEMV workgroups of the
// same launch publish with the call's tag (workspace word kWsSeq + 1).
template <int REP, bool FUSED, bool HO>
__device__ __forceinline__ void attn_decode_body(const DecodeArgs& A, uint32_t c, uint32_t g, DecodeSmem<REP>& sm,
                                                 const unsigned long long* rec) {
    static_assert(FUSED || !HO, "the hand-off form is the fused op's");
    _Float16* const s_v = sm.v;
    _Float16* const s_kt = sm.kt;
    auto& s_q = sm.q;
    _Float16* const s_k = sm.k;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lc = lane & 15, lr = lane >> 4;
    uint32_t rtag[2] = {0u, 0u}, rtheta[2] = {0u, 0u}, rw[2] = {0u, 0u};
    if constexpr (FUSED) {   // issued with the counter load: neither depends on it
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            rtag[j] = A.ws[kWsRopeTag + j];
            rtheta[j] = A.ws[kWsRopeTheta + j];
            rw[j] = A.ws[kWsRope + HD / 2 * j + lane];
        }
    }
    // Wave w's 16 K and V rows (key 16w + lc, dims 32s + 8lr .. +8) for the LDS tiles.
    // Chunks below spec_chunks (see spec_chunks on the host) request them before the
    // count arrives; the others after it, for keys inside the count only. Rows of slots
    // past the count are stale and masked below.
    u32x4 kr[4], vr[4];
    auto row = [&](uint32_t key, uint32_t lim) -> const uint8_t* {
        const uint32_t slot = (key < lim ? key : c * DC) % A.nslots;
        return A.ring + (size_t)slot * A.slot_bytes + ((size_t)g * HD + 8 * lr) * 2;
    };
    auto load_kv = [&](uint32_t lim) {
        const uint8_t* kb = row(c * DC + 16 * wave + lc, lim);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            kr[s] = *reinterpret_cast<const u32x4*>(kb + 64 * s);
            vr[s] = *reinterpret_cast<const u32x4*>(kb + A.slot_bytes / 2 + 64 * s);
        }
    };
    // Load order = wait order (loads return in order): the counter first, then the new
    // token's q rows (and its k / v rows and gammas, FUSED), the plain op's q, and only
    // then the K/V rows of the chunks below spec_chunks. Waiting for the counter and the
    // q rows does not wait for the K/V rows, so the queries' norm + RoPE run while those
    // are in flight.
    const uint32_t cnt = (FUSED || A.count) ? *A.count : A.n_kv_host;
    uint32_t tag = 0u;
    if constexpr (HO) tag = A.ws[kWsSeq] + 1u;
    constexpr int QW = (REP + 3) / 4;   // query heads per wave
    const uint32_t kwave = (REP < 4 ? (uint32_t)REP : 0u) % 4;   // the wave that handles k of head g
    uint16_t qx1[QW] = {}, qx2[QW] = {}, kx1 = 0, kx2 = 0, kg1 = 0, kg2 = 0, vx1 = 0, vx2 = 0, qg1 = 0, qg2 = 0;
    u32x4 vn[4] = {};
    h8_t qpl[4] = {};
    const uint32_t qh = min(lc, (uint32_t)REP - 1u);
    if constexpr (HO) {   // the rows themselves arrive through the records, below
        qg1 = __half_as_ushort(A.qg[lane]);
        qg2 = __half_as_ushort(A.qg[lane + 64]);
        if (wave == kwave) {
            kg1 = __half_as_ushort(A.kg[lane]);
            kg2 = __half_as_ushort(A.kg[lane + 64]);
        }
    } else if constexpr (FUSED) {
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const uint32_t r = wave + 4 * j;
            if (r < (uint32_t)REP) {
                const __half* src = A.qkv + (size_t)(g * REP + r) * HD;
                qx1[j] = __half_as_ushort(src[lane]);
                qx2[j] = __half_as_ushort(src[lane + 64]);
            }
        }
        qg1 = __half_as_ushort(A.qg[lane]);
        qg2 = __half_as_ushort(A.qg[lane + 64]);
        if (wave == kwave) {
            const __half* ksrc = A.qkv + (size_t)(A.H + g) * HD;
            const __half* vsrc = A.qkv + (size_t)(A.H + A.KVH + g) * HD;
            kx1 = __half_as_ushort(ksrc[lane]);
            kx2 = __half_as_ushort(ksrc[lane + 64]);
            kg1 = __half_as_ushort(A.kg[lane]);
            kg2 = __half_as_ushort(A.kg[lane + 64]);
            vx1 = __half_as_ushort(vsrc[lane]);
            vx2 = __half_as_ushort(vsrc[lane + 64]);
        }
        const __half* vnew = A.qkv + (size_t)(A.H + A.KVH + g) * HD + 8 * lr;
#pragma unroll
        for (int s = 0; s < 4; ++s) vn[s] = *reinterpret_cast<const u32x4*>(vnew + 32 * s);
    } else if (wave == 0) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            qpl[s] = *reinterpret_cast<const h8_t*>(A.q + (size_t)(g * REP + qh) * HD + 32 * s + 8 * lr);
    }
    const bool early = c < A.spec_chunks;
    if constexpr (HO) {
        // The K/V rows are not needed before the GEMV's records arrive: requested ~1 us in
        // (for the 4B q|k|v weights), they leave the memory system to the GEMV's weight
        // stream first (the 4B layer 13.5 -> 13.05 us; 2 us in: 13.8).
        for (uint32_t k = 0; k < A.kv_naps; ++k) __builtin_amdgcn_s_sleep(4);
    }
    if (early) load_kv(0xFFFFFFFFu);
    asm volatile("" ::: "memory");
    const uint32_t pos = FUSED ? cnt : 0u;   // position of the new token
    const uint32_t n_kv = FUSED ? pos + 1 : cnt;
    if (c * DC >= n_kv) return;
    if (FUSED && c == 0 && g == 0 && tid == 0) A.ws[kWsSnap] = n_kv;
    if (!early) load_kv(n_kv);
    const bool owns_new = FUSED && pos / DC == c;
    // K and V tiles. The new token's V row comes from the QKV row (its ring slot was read
    // before this launch wrote it; its K row is replaced below). V rows past n_kv are
    // zero, since slots not yet written may hold anything and p = 0 times a non-finite
    // value would reach the sums; their scores are -inf whatever K holds. In the
    // hand-off form the tiles are staged before the records are waited for (the K/V
    // loads are the older ones in flight), the new token's V row once its record is in.
    const uint32_t trow = 16 * wave + lc, tkey = c * DC + trow;   // this lane's tile row
    auto stage_tiles = [&]() {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x4 v = vr[s];
            if (!HO && FUSED && tkey == pos) v = vn[s];
            if (tkey >= n_kv) v = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(&s_v[trow * VSD + 32 * s + 8 * lr]) = v;
            *reinterpret_cast<u32x4*>(&s_kt[trow * KSD + 32 * s + 8 * lr]) = kr[s];
        }
    };
    if constexpr (HO) {
        stage_tiles();
        // Wait for the records of this group's q rows and of k and v of head g (record i
        // of row block b: rows 2i, 2i + 1 of head b), then take the values from LDS as
        // the other form takes them from the q|k|v row. One thread first waits for the
        // last v record (the v rows are the GEMV's last row blocks), then every thread
        // reads and checks its own records, so that the polls do not load the memory
        // system while the GEMV streams its weights.
        constexpr uint32_t NREC = (REP + 2) * HD / 2;
        auto rec_at = [&](uint32_t i) {
            const uint32_t b = i / (HD / 2);
            const uint32_t head = b < (uint32_t)REP ? g * REP + b : b == (uint32_t)REP ? A.H + g : A.H + A.KVH + g;
            return rec + (size_t)head * (HD / 2) + i % (HD / 2);
        };
        if (tid == 0) handoff_wait<2>(rec_at(NREC - 1), tag, A.ws + kWsErr);
        __syncthreads();
        for (uint32_t i = tid; i < NREC; i += 256) sm.raw[i] = handoff_wait<1>(rec_at(i), tag, A.ws + kWsErr);
        __syncthreads();
        const uint16_t* raw16 = reinterpret_cast<const uint16_t*>(sm.raw);
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const uint32_t r = wave + 4 * j;
            if (r < (uint32_t)REP) {
                qx1[j] = raw16[r * HD + lane];
                qx2[j] = raw16[r * HD + lane + 64];
            }
        }
        if (wave == kwave) {
            kx1 = raw16[REP * HD + lane];
            kx2 = raw16[REP * HD + lane + 64];
            vx1 = raw16[(REP + 1) * HD + lane];
            vx2 = raw16[(REP + 1) * HD + lane + 64];
        }
        if (tkey == pos) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                *reinterpret_cast<u32x4*>(&s_v[trow * VSD + 32 * s + 8 * lr]) =
                    *reinterpret_cast<const u32x4*>(&raw16[(REP + 1) * HD + 32 * s + 8 * lr]);
        }
    }

    if constexpr (FUSED) {
        float cr, sr;
        const uint32_t tb = __float_as_uint(A.theta);
        const bool hit0 = rtag[0] == pos + 1 && rtheta[0] == tb, hit1 = rtag[1] == pos + 1 && rtheta[1] == tb;
        if (hit0 || hit1) {   // wave-uniform
            const uint32_t w = hit0 ? rw[0] : rw[1];
            cr = dev::bits_f((uint16_t)(w & 0xFFFFu));
            sr = dev::bits_f((uint16_t)(w >> 16));
        } else {
            dev::rope_cs_inv(pos, dev::rope_inv(lane, A.theta), cr, sr);
        }
        auto hf = [](uint16_t b) { return __half2float(__ushort_as_half(b)); };
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const uint32_t r = wave + 4 * j;
            if (r >= (uint32_t)REP) break;
            float y1, y2;
            dev::head_norm_rope(hf(qx1[j]), hf(qx2[j]), hf(qg1), hf(qg2), cr, sr, y1, y2);
            s_q[r][lane] = (_Float16)y1;
            s_q[r][lane + 64] = (_Float16)y2;
        }
        if (owns_new && wave == kwave) {
            // k of head g: norm + RoPE; v raw. Written to the ring; k kept for this chunk.
            float y1, y2;
            dev::head_norm_rope(hf(kx1), hf(kx2), hf(kg1), hf(kg2), cr, sr, y1, y2);
            s_k[lane] = (_Float16)y1;
            s_k[lane + 64] = (_Float16)y2;
            _Float16* kface = reinterpret_cast<_Float16*>(A.ring + (size_t)(pos % A.nslots) * A.slot_bytes);
            _Float16* vface = kface + A.KVH * HD;
            kface[g * HD + lane] = (_Float16)y1;
            kface[g * HD + lane + 64] = (_Float16)y2;
            vface[g * HD + lane] = __builtin_bit_cast(_Float16, vx1);
            vface[g * HD + lane + 64] = __builtin_bit_cast(_Float16, vx2);
        }
    }
    if constexpr (!HO) stage_tiles();
    __syncthreads();
    if (wave != 0) return;

    // Queries as B columns; K rows as A tiles (key 16t + lc), the new token's k in place
    // of its stale ring row.
    h8_t qb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const h8_t v = FUSED ? *reinterpret_cast<const h8_t*>(&s_q[qh][32 * s + 8 * lr]) : qpl[s];
        qb[s] = lc < (uint32_t)REP ? v : h8_t{};
    }
    u32x4 kf[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) kf[t][s] = *reinterpret_cast<const u32x4*>(&s_kt[(16 * t + lc) * KSD + 32 * s + 8 * lr]);
    if (owns_new) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (c * DC + 16 * t + lc == pos) {
#pragma unroll
                for (int s = 0; s < 4; ++s) kf[t][s] = *reinterpret_cast<const u32x4*>(&s_k[32 * s + 8 * lr]);
            }
    }
    f4_t sa[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        sa[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
            sa[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, kf[t][s]), qb[s], sa[t], 0, 0, 0);
    }

    // Scores in log2 units plus the mask; this lane: head lc, keys 16t + 4lr + i.
    float x[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = c * DC + 16 * t + 4 * lr + i;
            float mk = 0.0f;
            if (!FUSED && A.mask) mk = __half2float(A.mask[(size_t)(g * REP + qh) * A.mask_hs + min(key, n_kv - 1u)]) * kLog2e;
            x[t][i] = key < n_kv ? sa[t][i] * A.scale_log2 + mk : -INFINITY;
        }
    float mx = -INFINITY;   // scores are finite or -inf: v_max3 without NaN quieting
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        mx = dev::max3_nonan(mx, x[t][0], x[t][1]);
        mx = dev::max3_nonan(mx, x[t][2], x[t][3]);
    }
    const float m = cross_row_max(mx);
    float p[4][4], ls = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[t][i] = m == -INFINITY ? 0.0f : exp2f(x[t][i] - m);   // a chunk whose keys are all masked
            ls += p[t][i];
        }
    const float l = dev::cross_row_sum(ls);
    float* wchunk = A.part + ((size_t)g * A.max_chunks + c) * REP * PS;
    if (lr == 0 && lc < (uint32_t)REP) {
        wchunk[lc * PS + HD] = m;
        wchunk[lc * PS + HD + 1] = l;
    }

    f4_t oa[HD / 16];
#pragma unroll
    for (int u = 0; u < HD / 16; ++u) oa[u] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const h8_t pb = {(_Float16)p[2 * j][0], (_Float16)p[2 * j][1], (_Float16)p[2 * j][2], (_Float16)p[2 * j][3],
                         (_Float16)p[2 * j + 1][0], (_Float16)p[2 * j + 1][1], (_Float16)p[2 * j + 1][2],
                         (_Float16)p[2 * j + 1][3]};
        const _Float16* r0 = &s_v[(32 * j + 4 * lr + lc / 4) * VSD + 4 * (lc % 4)];
#pragma unroll
        for (int u = 0; u < HD / 16; ++u) {
            const u32x2 lo = lds_read_tr16(r0 + 16 * u);
            const u32x2 hi = lds_read_tr16(r0 + 16 * VSD + 16 * u);
            const h8_t af = __builtin_bit_cast(h8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
            oa[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, pb, oa[u], 0, 0, 0);
        }
    }
    if (lc < (uint32_t)REP) {
#pragma unroll
        for (int u = 0; u < HD / 16; ++u)
            *reinterpret_cast<float4*>(wchunk + lc * PS + 16 * u + 4 * lr) =
                make_float4(oa[u][0], oa[u][1], oa[u][2], oa[u][3]);
    }
}

template <int REP, bool FUSED>
__global__ __launch_bounds__(256) void attn_decode_kernel(DecodeArgs A) {
    __shared__ DecodeSmem<REP> sm;
    attn_decode_body<REP, FUSED, false>(A, blockIdx.x, blockIdx.y, sm, nullptr);
}

// The fused op's q|k|v GEMV and its chunk pass in one launch. Workgroups [0, n_gemv)
// run the row-in-wave GEMV (gemv_rw_body: 4 waves, one pass, C slices of P lanes per
// row) and, besides writing the q|k|v row, publish it as tagged row-pair records; the
// chunk workgroups (c, g) behind them request their K/V rows at once and take the new
// token's q, k and v from the records when they arrive, so the K/V stream of the chunk
// pass overlaps the GEMV instead of following it. Waits go one way only, chunk
// workgroups on GEMV workgroups, which never wait; the host launches this only when
// the whole grid fits on the device at once, so every waited-for workgroup is running.
// Tags are the workspace's call sequence number + 1 (the merge pass advances it after
// each call), so a record left by an earlier call never matches.
struct QkvAttnArgs {
    GemvRwArgs G;
    DecodeArgs D;
    unsigned long long* rec;   // (H + 2 KVH) * HD / 2 records
    uint32_t n_gemv;
};

template <int REP, int C, int P>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void qkv_attn_decode_kernel(QkvAttnArgs QA) {
    __shared__ DecodeSmem<REP> sm;
    __shared__ double s_ss[8];
    if (blockIdx.x < QA.n_gemv) {
        const uint32_t tag = QA.D.ws[kWsSeq] + 1u;
        // merge_oproj_kernel's tags: no workgroup of this launch reads that word
        if (blockIdx.x == 0 && threadIdx.x == 0) QA.D.ws[kWsSeqB] = QA.D.ws[kWsSeqB] + 1u;
        gemv_rw_body<C, P, 1, 2, true>(QA.G, blockIdx.x, 256u, reinterpret_cast<u32x4*>(sm.v), s_ss, QA.rec, tag);
        return;
    }
    const uint32_t b = blockIdx.x - QA.n_gemv;
    attn_decode_body<REP, true, true>(QA.D, b % QA.D.max_chunks, b / QA.D.max_chunks, sm, QA.rec);
}

// Decode, pass 2: one workgroup per query head h = g*rep + r merges its chunks:
// M = max m_c, L = sum l_c 2^(m_c - M), O = sum O_c 2^(m_c - M) / L, in one pass:
// thread (grp, d4) merges chunks grp, grp+8, ... of dims 4*d4..4*d4+3 online (running
// max, rescaling its sums when the max grows), then the 8 groups are merged in LDS.
// With `advance` (fused), n_kv is the chunk pass's snapshot (the counter + 1): query
// head 0 stores it as the new counter value (no other workgroup of this pass reads the
// counter), and the extra last workgroup writes the two RoPE records.
// With a mask over a gathered layout of P > n_kv positions, positions [n_kv, P) (zero K
// and V) add their mask values to the softmax denominator: one more partial (m, l) with
// O = 0, reduced over the workgroup.
// Workgroup h of the pass (rope_wg: the extra one). With orec, the head's output is also
// published as tagged row-pair records orec[h * HD / 2 + i] (see merge_oproj_kernel).
struct MergeSmem {
    __align__(16) float4 o[256];
    float m[8], l[8], t[4];
};
__device__ __forceinline__ void attn_merge_body(const float* __restrict__ part, uint32_t n_kv_host,
                                                uint32_t* __restrict__ count, int advance, uint32_t rep,
                                                uint32_t max_chunks, __half* __restrict__ out,
                                                uint32_t* __restrict__ ws, float theta,
                                                const __half* __restrict__ mask, uint32_t P, uint32_t mask_hs,
                                                uint32_t h, bool rope_wg, MergeSmem& lds,
                                                unsigned long long* orec, uint32_t otag) {
    float4* const s_o = lds.o;
    float* const s_m = lds.m;
    float* const s_l = lds.l;
    float* const s_t = lds.t;
    const uint32_t g = h / rep, r = h % rep;
    const uint32_t tid = threadIdx.x;
    if (rope_wg) {
        if (tid == 0) ws[kWsSeq] = ws[kWsSeq] + 1u;   // this call's records are all read
        const uint32_t n_kv = ws[kWsSnap];
        // RoPE records for positions n_kv - 1 (wave 0) and n_kv (wave 1).
        const uint32_t j = tid >> 6, i = tid & 63;
        if (j < 2) {
            ws[kWsRope + HD / 2 * j + i] = dev::rope_cs_bits(n_kv - 1 + j, dev::rope_inv(i, theta));
            if (i == 0) {
                ws[kWsRopeTag + j] = n_kv + j;
                ws[kWsRopeTheta + j] = __float_as_uint(theta);
            }
        }
        return;
    }
    const float* base = part + ((size_t)g * max_chunks * rep + r) * PS;   // chunk c at + c*rep*PS
    const size_t cstride = (size_t)rep * PS;

    const uint32_t d4 = tid & 31, grp = tid >> 5;
    float mg = -INFINITY, lg = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto merge_one = [&](float mc, float lc, const float4& v) {
        if (mc > mg) {   // 2^-inf = 0 on the first chunk
            const float sc = exp2f(mg - mc);
            o.x *= sc; o.y *= sc; o.z *= sc; o.w *= sc;
            lg *= sc;
            mg = mc;
        }
        const float wt = mc == -INFINITY ? 0.0f : exp2f(mc - mg);   // a chunk whose keys are all masked
        o.x = fmaf(wt, v.x, o.x);
        o.y = fmaf(wt, v.y, o.y);
        o.z = fmaf(wt, v.z, o.z);
        o.w = fmaf(wt, v.w, o.w);
        lg = fmaf(wt, lc, lg);
    };
    // The first kSpec records of each thread group are loaded whatever n_kv turns out to
    // be (records of chunks past it hold stale values and are never merged), so their
    // loads overlap the counter's instead of waiting for it; chunks beyond, if any, follow.
    constexpr uint32_t kSpec = 8;
    float sm[kSpec], sl[kSpec];
    float4 sv[kSpec];
#pragma unroll
    for (uint32_t k = 0; k < kSpec; ++k) {
        const float* w = base + (size_t)min(grp + 8 * k, max_chunks - 1) * cstride;
        sm[k] = w[HD];
        sl[k] = w[HD + 1];
        sv[k] = *reinterpret_cast<const float4*>(w + 4 * d4);
    }
    asm volatile("" ::: "memory");   // the count is read after the records are requested
    const uint32_t n_kv = advance ? ws[kWsSnap] : count ? *count : n_kv_host;
    const uint32_t nc = (n_kv + DC - 1) / DC;
#pragma unroll
    for (uint32_t k = 0; k < kSpec; ++k)
        if (grp + 8 * k < nc) merge_one(sm[k], sl[k], sv[k]);
    for (uint32_t c = grp + 8 * kSpec; c < nc; c += 8) {
        const float* w = base + c * cstride;
        merge_one(w[HD], w[HD + 1], *reinterpret_cast<const float4*>(w + 4 * d4));
    }
    s_o[tid] = o;
    if (d4 == 0) { s_m[grp] = mg; s_l[grp] = lg; }
    // Tail of a masked gathered layout: max, then sum of 2^(mask - max), over the workgroup.
    float tm = -INFINITY, tl = 0.0f;
    const bool tail = mask && P > n_kv;
    if (tail) {
        const __half* mrow = mask + (size_t)h * mask_hs;
        for (uint32_t j = n_kv + tid; j < P; j += 256) tm = fmaxf(tm, __half2float(mrow[j]) * kLog2e);
        tm = dev::wave_max(tm);
        if ((tid & 63) == 0) s_t[tid >> 6] = tm;
        __syncthreads();
        tm = fmaxf(fmaxf(s_t[0], s_t[1]), fmaxf(s_t[2], s_t[3]));
        if (tm != -INFINITY)
            for (uint32_t j = n_kv + tid; j < P; j += 256) tl += exp2f(__half2float(mrow[j]) * kLog2e - tm);
        tl = dev::wave_sum(tl);
        __syncthreads();
        if ((tid & 63) == 0) s_t[tid >> 6] = tl;
        __syncthreads();
        tl = s_t[0] + s_t[1] + s_t[2] + s_t[3];
    }
    __syncthreads();
    if (tid < 32) {
        float M = s_m[0];
        for (uint32_t k = 1; k < 8; ++k) M = fmaxf(M, s_m[k]);
        M = fmaxf(M, tm);
        float L = tm == -INFINITY ? 0.0f : exp2f(tm - M) * tl;
        o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t k = 0; k < 8; ++k) {
            const float wk = s_m[k] == -INFINITY ? 0.0f : exp2f(s_m[k] - M);   // 0 for a group without chunks
            const float4 p = s_o[tid + 32 * k];
            o.x = fmaf(wk, p.x, o.x);
            o.y = fmaf(wk, p.y, o.y);
            o.z = fmaf(wk, p.z, o.z);
            o.w = fmaf(wk, p.w, o.w);
            L = fmaf(wk, s_l[k], L);
        }
        h4_t hv = {(_Float16)(L > 0.0f ? o.x / L : 0.0f), (_Float16)(L > 0.0f ? o.y / L : 0.0f),
                   (_Float16)(L > 0.0f ? o.z / L : 0.0f), (_Float16)(L > 0.0f ? o.w / L : 0.0f)};
        *reinterpret_cast<h4_t*>(out + (size_t)h * HD + 4 * tid) = hv;
        if (orec) {
            const u32x2 w = __builtin_bit_cast(u32x2, hv);
            handoff_store(orec + (size_t)h * (HD / 2) + 2 * tid, otag, w[0]);
            handoff_store(orec + (size_t)h * (HD / 2) + 2 * tid + 1, otag, w[1]);
        }
    }
    if (advance && h == 0 && tid == 0) *count = n_kv;
}

__global__ __launch_bounds__(256) void attn_merge_kernel(
    const float* __restrict__ part, uint32_t n_kv_host, uint32_t* __restrict__ count, int advance,
    uint32_t rep, uint32_t max_chunks, __half* __restrict__ out, uint32_t* __restrict__ ws, float theta,
    const __half* __restrict__ mask, uint32_t P, uint32_t mask_hs) {
    __shared__ MergeSmem sm;
    attn_merge_body(part, n_kv_host, count, advance, rep, max_chunks, out, ws, theta, mask, P, mask_hs, blockIdx.x,
                    advance && blockIdx.x == gridDim.x - 1, sm, nullptr, 0u);
}

// The fused op's merge pass and the o-proj GEMV reading its output (an OP_W4G_FUSED_F16
// with M = 1, no RMSNorm, no SwiGLU) in one launch. Workgroups [0, H) merge a query
// head each and, besides writing the attention output, publish it as tagged row-pair
// records (tag: workspace word kWsSeqB + 1); workgroup H writes the RoPE records; the
// GEMV workgroups behind them (gemv_rw_body, 4 waves, 2 passes) request their weights
// at once and take x from those records. (Dequantizing the weights while x is on its
// way, with one pass per workgroup, was slower: 17.4 against 17.0 us for the 4B
// q|k|v + attention + o-proj.) Waits go one way (GEMV on merge workgroups,
// which never wait) and the host launches this only when the grid fits on the device
// at once.
struct MergeOprojArgs {
    const float* part;
    uint32_t* count;
    uint32_t rep, max_chunks, H;
    __half* out;
    uint32_t* ws;
    float theta;
    GemvRwArgs G;               // the o-proj; x = out
    unsigned long long* xrec;   // H * HD / 2 records of out
};

template <int C, int P>
__global__ __launch_bounds__(256) void merge_oproj_kernel(MergeOprojArgs M) {
    __shared__ MergeSmem ms;
    __shared__ __align__(16) u32x4 xs[C * P * 4];   // x in pair order (K / 8 slots)
    __shared__ double s_ss[8];
    const uint32_t tag = M.ws[kWsSeqB] + 1u;
    if (blockIdx.x <= M.H) {
        attn_merge_body(M.part, 0u, M.count, 1, M.rep, M.max_chunks, M.out, M.ws, M.theta, nullptr, 0u, 0u,
                        blockIdx.x, blockIdx.x == M.H, ms, M.xrec, tag);
        return;
    }
    gemv_rw_body<C, P, 2, 2, false, true>(M.G, blockIdx.x - (M.H + 1), 256u, xs, s_ss, nullptr, 0u, M.xrec, tag,
                                          M.ws + kWsErr);
}

}  // namespace

hipError_t launch_attn_prefill(const __half* q, uint32_t ldq, const __half* k, const __half* v,
                               uint32_t ldkv, __half* out, uint32_t ldo, uint32_t S, uint32_t H,
                               uint32_t KVH, uint32_t hd, float scale, bool causal,
                               hipStream_t st) {
    return launch_attn_prefill_hs(q, ldq, HD, k, v, ldkv, HD, out, ldo, HD, S, H, KVH, hd, scale, causal, st);
}

hipError_t launch_attn_prefill_hs(const __half* q, uint32_t ldq, uint32_t qhs, const __half* k, const __half* v,
                                  uint32_t ldkv, uint32_t kvhs, __half* out, uint32_t ldo, uint32_t ohs, uint32_t S,
                                  uint32_t H, uint32_t KVH, uint32_t hd, float scale, bool causal, hipStream_t st) {
    if (hd != HD || !KVH || H % KVH) return hipErrorInvalidValue;
    if (!(scale > 0.0f && scale < INFINITY)) return hipErrorInvalidValue;   // the kernel's max needs scale > 0
    if ((uint64_t)ldkv * 2u * KT > 0xFFFFFFFFull) return hipErrorInvalidValue;   // a stage's K / V bytes: 32-bit offsets
    if (!S || !H) return hipSuccess;
    // 128-query tiles (8-wave workgroups) while they give every CU one; else 64-query
    // tiles (4-wave workgroups) while those do; else 32-query tiles (2-wave workgroups).
    const size_t cus = (size_t)device_cu_count();
    const uint32_t wph = (size_t)H * ((S + 127) / 128) >= cus ? 4u : (size_t)H * ((S + 63) / 64) >= cus ? 2u : 1u;
    const uint32_t qt = 32 * wph;
    dim3 grid(H, (S + qt - 1) / qt);   // heads fastest: the heavy tiles of every head go first
    const float sl2 = scale * kLog2e;
    const auto kern = causal ? (wph == 4   ? attn_prefill_kernel<true, 4>
                                : wph == 2 ? attn_prefill_kernel<true, 2>
                                           : attn_prefill_kernel<true, 1>)
                             : (wph == 4   ? attn_prefill_kernel<false, 4>
                                : wph == 2 ? attn_prefill_kernel<false, 2>
                                           : attn_prefill_kernel<false, 1>);
    hipLaunchKernelGGL(kern, grid, dim3(4 * qt), 0, st, q, ldq, qhs, k, v, ldkv, kvhs, out, ldo, ohs, S, H, KVH,
                       sl2);
    return hipGetLastError();
}

// Workspace: the head (fused-call snapshot and RoPE records; zero before the first fused
// call) then per (kv head, chunk, query head) partial records of PS floats.
uint32_t attn_decode_work_floats(uint32_t max_kv, uint32_t H, uint32_t hd) {
    (void)hd;
    return kWsHead + ((max_kv + DC - 1) / DC) * H * PS;
}

namespace {

template <bool FUSED>
hipError_t decode_launch(const DecodeArgs& A, uint32_t rep, int advance, __half* out, float* work,
                         hipStream_t st) {
    dim3 grid(A.max_chunks, A.KVH);
    switch (rep) {
    case 1: hipLaunchKernelGGL((attn_decode_kernel<1, FUSED>), grid, dim3(256), 0, st, A); break;
    case 2: hipLaunchKernelGGL((attn_decode_kernel<2, FUSED>), grid, dim3(256), 0, st, A); break;
    case 4: hipLaunchKernelGGL((attn_decode_kernel<4, FUSED>), grid, dim3(256), 0, st, A); break;
    case 8: hipLaunchKernelGGL((attn_decode_kernel<8, FUSED>), grid, dim3(256), 0, st, A); break;
    default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(attn_merge_kernel, dim3(A.H + (advance ? 1 : 0)), dim3(256), 0, st, A.part, A.n_kv_host,
                       A.count, advance, rep, A.max_chunks, out, reinterpret_cast<uint32_t*>(work), A.theta,
                       A.mask, A.P, A.mask_hs);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_decode(const __half* q, const uint8_t* ring, uint32_t slot_bytes,
                              uint32_t nslots, __half* out, uint32_t n_kv_host,
                              const uint32_t* count_dev, uint32_t H, uint32_t KVH, uint32_t hd,
                              float scale, float* work, uint32_t work_floats, hipStream_t st,
                              const __half* mask, uint32_t P, uint32_t n_kv_known, bool mask_shared) {
    if (hd != HD || !KVH || H % KVH) return hipErrorInvalidValue;
    if (mask && (P == 0 || P > nslots || (!count_dev && n_kv_host > P))) return hipErrorInvalidValue;
    const uint32_t rep = H / KVH;
    if (rep > MAX_REP || slot_bytes != KVH * HD * 4) return hipErrorInvalidValue;
    // Chunks cover every position the ring can hold, so a device-side count never
    // exceeds the grid.
    const uint32_t max_kv = count_dev ? nslots : n_kv_host;
    const uint32_t max_chunks = (max_kv + DC - 1) / DC;
    if (attn_decode_work_floats(max_kv, H, hd) > work_floats) return hipErrorInvalidValue;
    if (!max_chunks) return hipSuccess;
    DecodeArgs A{q, nullptr, nullptr, nullptr, 0.0f, const_cast<uint8_t*>(ring), slot_bytes, nslots, KVH, H,
                 n_kv_host, const_cast<uint32_t*>(count_dev), scale * kLog2e, work + kWsHead, max_chunks, nullptr,
                 mask, mask ? P : 0u, mask && !mask_shared ? P : 0u,
                 (count_dev ? std::min(n_kv_known, nslots) : n_kv_host) / DC};
    return decode_launch<false>(A, rep, 0, out, work, st);
}

hipError_t launch_attn_decode_qkv(const __half* qkv, const __half* q_gamma, const __half* k_gamma,
                                  float theta, uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                                  uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH,
                                  float scale, float* work, uint32_t work_floats, hipStream_t st,
                                  uint32_t n_kv_known) {
    if (!KVH || H % KVH || !count_dev) return hipErrorInvalidValue;
    const uint32_t rep = H / KVH;
    if (rep > MAX_REP || slot_bytes != KVH * HD * 4 || !nslots) return hipErrorInvalidValue;
    const uint32_t max_chunks = (nslots + DC - 1) / DC;
    if (attn_decode_work_floats(nslots, H, HD) > work_floats) return hipErrorInvalidValue;
    DecodeArgs A{nullptr, qkv, q_gamma, k_gamma, theta, ring, slot_bytes, nslots, KVH, H,
                 0u, count_dev, scale * kLog2e, work + kWsHead, max_chunks,
                 reinterpret_cast<uint32_t*>(work), nullptr, 0u, 0u, std::min(n_kv_known, nslots) / DC};
    return decode_launch<true>(A, rep, 1, out, work, st);
}

namespace {

// Workgroups per CU of the one-launch kernel (0 if unknown), once per instance.
template <int REP, int C, int P>
int qkv_attn_occupancy() {
    static std::atomic<int> occ{-1};
    int o = occ.load(std::memory_order_relaxed);
    if (o < 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, qkv_attn_decode_kernel<REP, C, P>, 256, 0) !=
            hipSuccess)
            nb = 0;
        occ.store(nb, std::memory_order_relaxed);
        o = nb;
    }
    return o;
}

// The instance for (rep, C, P): its occupancy query (launch == false) or its launch.
template <int REP>
int qkv_attn_instance(uint32_t C, uint32_t P, bool launch, const QkvAttnArgs* QA, uint32_t grid, hipStream_t st) {
#define GEHTP_QKV_ATTN(CC, PP)                                                                     \
    if (C == CC && P == PP) {                                                                     \
        if (!launch) return qkv_attn_occupancy<REP, CC, PP>();                                    \
        hipLaunchKernelGGL((qkv_attn_decode_kernel<REP, CC, PP>), dim3(grid), dim3(256), 0, st, *QA); \
        return 1;                                                                                 \
    }
    GEHTP_QKV_ATTN(2, 16)
    GEHTP_QKV_ATTN(4, 16)
    GEHTP_QKV_ATTN(5, 16)
    GEHTP_QKV_ATTN(3, 32)
    GEHTP_QKV_ATTN(4, 32)
#undef GEHTP_QKV_ATTN
    return 0;
}

int qkv_attn_call(uint32_t rep, uint32_t C, uint32_t P, bool launch, const QkvAttnArgs* QA, uint32_t grid,
                  hipStream_t st) {
    switch (rep) {
    case 1: return qkv_attn_instance<1>(C, P, launch, QA, grid, st);
    case 2: return qkv_attn_instance<2>(C, P, launch, QA, grid, st);
    case 4: return qkv_attn_instance<4>(C, P, launch, QA, grid, st);
    case 8: return qkv_attn_instance<8>(C, P, launch, QA, grid, st);
    default: return 0;
    }
}

struct QkvAttnPlan {
    bool ok = false;
    uint32_t C = 0, P = 0, rep = 0, N = 0, n_gemv = 0, max_chunks = 0, grid = 0;
};

// Shape rules of the one-launch form; ok only when the whole grid fits on the device at
// once (the waits need every GEMV workgroup resident or done while a chunk workgroup
// waits, which holds in any dispatch order when all are resident together; at most
// 128 VGPRs, amdgpu_waves_per_eu(4), gives four 4-wave workgroups per CU). (GEMV
// workgroups of three working waves and 12 rows, two per CU, ran the 4B layer slower:
// 14.2 against 13.6 us, each of the 512 workgroups staging and normalizing x.)
QkvAttnPlan qkv_attn_plan(uint32_t K, uint32_t H, uint32_t KVH, uint32_t nslots) {
    QkvAttnPlan pl;
    if (!KVH || H % KVH || !nslots) return pl;
    pl.rep = H / KVH;
    if (pl.rep != 1 && pl.rep != 2 && pl.rep != 4 && pl.rep != 8) return pl;
    if (K % 512 == 0 && (K / 512 == 2 || K / 512 == 4 || K / 512 == 5)) { pl.C = K / 512; pl.P = 16; }
    else if (K % 1024 == 0 && (K / 1024 == 3 || K / 1024 == 4)) { pl.C = K / 1024; pl.P = 32; }
    else return pl;
    pl.N = (H + 2 * KVH) * HD;
    if ((uint64_t)pl.N * (K / 2) >= (1ull << 32)) return pl;   // 32-bit row offsets
    const uint32_t rows_wg = 4u * (64u / pl.P);               // 4 waves, one pass
    pl.n_gemv = (pl.N + rows_wg - 1) / rows_wg;
    pl.max_chunks = (nslots + DC - 1) / DC;
    const uint64_t grid = (uint64_t)pl.n_gemv + (uint64_t)pl.max_chunks * KVH;
    const int occ = qkv_attn_call(pl.rep, pl.C, pl.P, false, nullptr, 0, nullptr);
    if (occ <= 0 || grid > (uint64_t)occ * (uint64_t)device_cu_count()) return pl;
    pl.grid = (uint32_t)grid;
    pl.ok = true;
    return pl;
}

uint32_t qkv_rec_offset(uint32_t nslots, uint32_t H) { return (attn_decode_work_floats(nslots, H, HD) + 1u) & ~1u; }

}  // namespace

// Records (8 bytes, 2 values each) after the partials: the q|k|v row, then the attention
// output (merge_oproj_kernel).
uint32_t attn_qkv_fused_work_floats(uint32_t nslots, uint32_t H, uint32_t KVH) {
    return qkv_rec_offset(nslots, H) + (H + 2 * KVH) * HD + H * HD;
}

namespace {

unsigned long long* out_recs(float* work, uint32_t nslots, uint32_t H, uint32_t KVH) {
    return reinterpret_cast<unsigned long long*>(work + qkv_rec_offset(nslots, H) + (H + 2 * KVH) * HD);
}

template <int C, int P>
int merge_oproj_occupancy() {
    static std::atomic<int> occ{-1};
    int o = occ.load(std::memory_order_relaxed);
    if (o < 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, merge_oproj_kernel<C, P>, 256, 0) != hipSuccess) nb = 0;
        occ.store(nb, std::memory_order_relaxed);
        o = nb;
    }
    return o;
}

struct MergeOprojPlan {
    bool ok = false;
    uint32_t C = 0, P = 0, n_gemv = 0;
};

// The o-proj GEMV of merge_oproj_kernel: K = H * 128 as 16 lanes x {2, 4, 5} or 32 lanes
// x {3, 4} slices per row, 4 waves of 2 passes per workgroup; the grid must fit at once.
MergeOprojPlan merge_oproj_plan(uint32_t H, uint32_t N) {
    MergeOprojPlan pl;
    const uint32_t K = H * HD;
    if (K % 512 == 0 && (K / 512 == 2 || K / 512 == 4 || K / 512 == 5)) { pl.C = K / 512; pl.P = 16; }
    else if (K % 1024 == 0 && (K / 1024 == 3 || K / 1024 == 4)) { pl.C = K / 1024; pl.P = 32; }
    else return pl;
    const uint32_t rows_wg = 4u * (64u / pl.P) * 2u;
    if (N < rows_wg || (uint64_t)N * (K / 2) >= (1ull << 32)) return pl;
    pl.n_gemv = (N + rows_wg - 1) / rows_wg;
    int occ = 0;
    if (pl.P == 16) occ = pl.C == 2 ? merge_oproj_occupancy<2, 16>() : pl.C == 4 ? merge_oproj_occupancy<4, 16>()
                                                                             : merge_oproj_occupancy<5, 16>();
    else occ = pl.C == 3 ? merge_oproj_occupancy<3, 32>() : merge_oproj_occupancy<4, 32>();
    if (occ <= 0 || (uint64_t)H + 1 + pl.n_gemv > (uint64_t)occ * (uint64_t)device_cu_count()) return pl;
    pl.ok = true;
    return pl;
}

}  // namespace

bool merge_oproj_supported(uint32_t H, uint32_t N) { return merge_oproj_plan(H, N).ok; }

hipError_t launch_attn_merge_deferred(uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, uint32_t nslots,
                                      float theta, float* work, hipStream_t st) {
    if (!KVH || H % KVH || !nslots) return hipErrorInvalidValue;
    const uint32_t max_chunks = (nslots + DC - 1) / DC;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(H + 1), dim3(256), 0, st, work + kWsHead, 0u, count_dev, 1, H / KVH,
                       max_chunks, out, reinterpret_cast<uint32_t*>(work), theta, nullptr, 0u, 0u);
    return hipGetLastError();
}

hipError_t launch_merge_oproj(uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, uint32_t nslots,
                              float theta, float* work, uint32_t work_floats, const uint8_t* wq, const __half* wsc,
                              __half* y, uint32_t N, const __half* res, hipStream_t st) {
    if (!KVH || H % KVH || !nslots || attn_qkv_fused_work_floats(nslots, H, KVH) > work_floats)
        return hipErrorInvalidValue;
    if (((uintptr_t)wq | (uintptr_t)work | (uintptr_t)out) % 16) return hipErrorInvalidValue;
    const MergeOprojPlan pl = merge_oproj_plan(H, N);
    if (!pl.ok) return hipErrorNotSupported;
    MergeOprojArgs M;
    M.part = work + kWsHead;
    M.count = count_dev;
    M.rep = H / KVH;
    M.max_chunks = (nslots + DC - 1) / DC;
    M.H = H;
    M.out = out;
    M.ws = reinterpret_cast<uint32_t*>(work);
    M.theta = theta;
    M.G = GemvRwArgs{out, wq, wsc, y, N, H * HD, nullptr, res, 0};
    M.xrec = out_recs(work, nslots, H, KVH);
    const dim3 grid(H + 1 + pl.n_gemv), blk(256);
    if (pl.P == 16) {
        if (pl.C == 2) hipLaunchKernelGGL((merge_oproj_kernel<2, 16>), grid, blk, 0, st, M);
        else if (pl.C == 4) hipLaunchKernelGGL((merge_oproj_kernel<4, 16>), grid, blk, 0, st, M);
        else hipLaunchKernelGGL((merge_oproj_kernel<5, 16>), grid, blk, 0, st, M);
    } else {
        if (pl.C == 3) hipLaunchKernelGGL((merge_oproj_kernel<3, 32>), grid, blk, 0, st, M);
        else hipLaunchKernelGGL((merge_oproj_kernel<4, 32>), grid, blk, 0, st, M);
    }
    return hipGetLastError();
}

bool qkv_attn_decode_supported(uint32_t K, uint32_t H, uint32_t KVH, uint32_t nslots) {
    return qkv_attn_plan(K, H, KVH, nslots).ok;
}

hipError_t launch_qkv_attn_decode(const __half* x, const uint8_t* wq, const __half* wsc, const __half* gamma,
                                  uint32_t K, __half* qkv, const __half* q_gamma, const __half* k_gamma,
                                  float theta, uint8_t* ring, uint32_t slot_bytes, uint32_t nslots,
                                  uint32_t* count_dev, __half* out, uint32_t H, uint32_t KVH, float scale,
                                  float* work, uint32_t work_floats, hipStream_t st, uint32_t n_kv_known,
                                  bool defer_merge) {
    if (!KVH || H % KVH || !count_dev || !nslots || slot_bytes != KVH * HD * 4) return hipErrorInvalidValue;
    if (attn_qkv_fused_work_floats(nslots, H, KVH) > work_floats) return hipErrorInvalidValue;
    if (((uintptr_t)x | (uintptr_t)wq | (uintptr_t)gamma | (uintptr_t)work) % 16) return hipErrorInvalidValue;
    const QkvAttnPlan pl = qkv_attn_plan(K, H, KVH, nslots);
    if (!pl.ok) return hipErrorNotSupported;
    QkvAttnArgs QA;
    QA.G = GemvRwArgs{x, wq, wsc, qkv, pl.N, K, gamma, nullptr, 0};
    // ~1.07 us of s_sleep(4) steps (256 clocks each) per 7.9 MB of q|k|v weights
    const uint32_t naps = (uint32_t)std::min<uint64_t>(20u, ((uint64_t)pl.N * (K / 2) * 10u + 3932160u) / 7864320u);
    QA.D = DecodeArgs{nullptr, qkv, q_gamma, k_gamma, theta, ring, slot_bytes, nslots, KVH, H,
                      0u, count_dev, scale * kLog2e, work + kWsHead, pl.max_chunks,
                      reinterpret_cast<uint32_t*>(work), nullptr, 0u, 0u, std::min(n_kv_known, nslots) / DC, naps};
    QA.rec = reinterpret_cast<unsigned long long*>(work + qkv_rec_offset(nslots, H));
    QA.n_gemv = pl.n_gemv;
    qkv_attn_call(pl.rep, pl.C, pl.P, true, &QA, pl.grid, st);
    if (defer_merge) return hipGetLastError();
    hipLaunchKernelGGL(attn_merge_kernel, dim3(H + 1), dim3(256), 0, st, QA.D.part, 0u, count_dev, 1, pl.rep,
                       pl.max_chunks, out, reinterpret_cast<uint32_t*>(work), theta, nullptr, 0u, 0u);
    return hipGetLastError();
}

}  // namespace gehtp
