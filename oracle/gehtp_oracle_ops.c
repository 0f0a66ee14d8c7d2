/* gehtp_oracle_ops.c — CPU restatement of the reference's remaining runlist ops
 * (TEST INFRASTRUCTURE: loaded only by tests/, the smoke check and bench.py's
 * cpu_baseline leg, never by the product).
 *
 * Each function cites the reference routine it restates; arithmetic order and
 * rounding points follow it (f16 <-> f32 through go_f16_to_f32 / go_f32_to_f16,
 * the reference's RNE conversion).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gehtp_oracle.h"

#define F(h) go_f16_to_f32(h)
#define H(f) go_f32_to_f16(f)

/* ---- crouton16_row4 surface (kernels/src/runtime/gemm_dispatch.c:38-72,
 * oplist_exec.c:421-436): surface order phase(8) -> kt(cols/32) -> g(rows/32) ->
 * row pair(2) -> 32 columns x (row0, row0+1), row0 = 32g + 4*phase + 2*rp. */
int go_crouton_encode(const uint16_t* lin, uint16_t* surf, uint32_t rows, uint32_t cols) {
    if (rows % 32 || cols % 32) return -1;
    const uint32_t n_m32 = rows / 32, n_kt = cols / 32;
    size_t out = 0;
    for (uint32_t phase = 0; phase < 8; phase++)
        for (uint32_t kt = 0; kt < n_kt; kt++)
            for (uint32_t g = 0; g < n_m32; g++)
                for (uint32_t rp = 0; rp < 2; rp++) {
                    const uint32_t row0 = g * 32 + phase * 4 + rp * 2;
                    uint16_t* p = surf + out;
                    for (uint32_t c = kt * 32; c < kt * 32 + 32; c++) {
                        p[0] = lin[(size_t)row0 * cols + c];
                        p[1] = lin[(size_t)(row0 + 1) * cols + c];
                        p += 2;
                    }
                    out += 64;
                }
    return 0;
}

int go_crouton_decode(const uint16_t* surf, uint16_t* lin, uint32_t rows, uint32_t cols) {
    if (rows % 32 || cols % 32) return -1;
    const uint32_t n_m32 = rows / 32, n_kt = cols / 32;
    size_t out = 0;
    for (uint32_t phase = 0; phase < 8; phase++)
        for (uint32_t kt = 0; kt < n_kt; kt++)
            for (uint32_t g = 0; g < n_m32; g++)
                for (uint32_t rp = 0; rp < 2; rp++) {
                    const uint32_t row0 = g * 32 + phase * 4 + rp * 2;
                    const uint16_t* p = surf + out;
                    for (uint32_t c = kt * 32; c < kt * 32 + 32; c++) {
                        lin[(size_t)row0 * cols + c] = p[0];
                        lin[(size_t)(row0 + 1) * cols + c] = p[1];
                        p += 2;
                    }
                    out += 64;
                }
    return 0;
}

/* ---- OP_MATMUL_W4A16 (opcode 1): the reference's closed form
 * (kernels/docs/api_v22_w4a16.md:11, kernels/assets/s2560/Y_gold.json "formula"):
 *   Y[m,n] = clip(round_div7(sum_k (A[m,k] - 32768) * W[k,n]) + 32768, 0, 65535)
 * A: u16 crouton16_row4 surface [M,K]; Y: u16 crouton16_row4 surface [M,N].
 * W: 4-bit values in [-8, 7]. The HMX tile packing of the reference's weight slot is
 * defined only inside its device kernel; this build reads the K*N/2-byte slot as
 * [N][K/2], byte j of row n = k 2j (low nibble) and 2j+1 (high nibble), stored +8
 * (the OP_MATMUL_W4G_F16 / Q4_0 nibble convention).
 * round_div7 = nearest integer to s/7 (s is an integer, so s/7 is never a tie). */
static int64_t round_div7(int64_t s) { return s >= 0 ? (s + 3) / 7 : -((-s + 3) / 7); }

int go_matmul_w4a16(const uint16_t* act_surf, const uint8_t* w, uint16_t* out_surf,
                    uint32_t M, uint32_t K, uint32_t N) {
    if (M % 32 || K % 32 || N % 32) return -1;
    uint16_t* a = malloc((size_t)M * K * 2);
    uint16_t* y = malloc((size_t)M * N * 2);
    if (!a || !y) { free(a); free(y); return -1; }
    go_crouton_decode(act_surf, a, M, K);
    for (uint32_t m = 0; m < M; m++)
        for (uint32_t n = 0; n < N; n++) {
            int64_t s = 0;
            const uint8_t* wr = w + (size_t)n * (K / 2);
            for (uint32_t k = 0; k < K; k++) {
                const int32_t q = (int32_t)((wr[k / 2] >> (4 * (k & 1))) & 0xF) - 8;
                s += (int64_t)((int32_t)a[(size_t)m * K + k] - 32768) * q;
            }
            int64_t v = round_div7(s) + 32768;
            if (v < 0) v = 0;
            if (v > 65535) v = 65535;
            y[(size_t)m * N + n] = (uint16_t)v;
        }
    go_crouton_encode(y, out_surf, M, N);
    free(a);
    free(y);
    return 0;
}

/* ---- OP_RMSNORM_F16 (opcode 2) on a crouton u16 surface (oplist_exec.c:559-591):
 * x = (float)(u16 - 32768); acc = sum double(x)^2; rms = (float)sqrt(acc/n + 1e-6);
 * y[r, i] = f16(x / rms * w[i]) row-major. */
int go_rmsnorm_crouton(const uint16_t* x_surf, const uint16_t* w16, uint16_t* y, uint32_t m, uint32_t n) {
    if (!m || m % 32 || n % 32) return -1;
    uint16_t* rows = malloc((size_t)m * n * 2);
    float* w = malloc((size_t)n * 4);
    float* xf = malloc((size_t)n * 4);
    if (!rows || !w || !xf) { free(rows); free(w); free(xf); return -1; }
    go_crouton_decode(x_surf, rows, m, n);
    for (uint32_t i = 0; i < n; i++) w[i] = F(w16[i]);
    for (uint32_t r = 0; r < m; r++) {
        const uint16_t* row = rows + (size_t)r * n;
        double acc = 0.0;
        for (uint32_t i = 0; i < n; i++) {
            xf[i] = (float)((int32_t)row[i] - 32768);
            acc += (double)xf[i] * (double)xf[i];
        }
        const float rms = (float)sqrt(acc / (double)n + 1e-6);
        for (uint32_t i = 0; i < n; i++) y[(size_t)r * n + i] = H(xf[i] / rms * w[i]);
    }
    free(rows);
    free(w);
    free(xf);
    return 0;
}

/* ---- OP_CONCAT_F16 (oplist_exec.c:1196-1220): last-axis concat of up to 4 segments,
 * segment k = (outer, sizes[k]) row-major at columns [start_k, start_k + sizes[k]). */
int go_concat(const uint16_t* const* xs, uint16_t* y, uint32_t n_seg, uint32_t n_elems,
              const uint32_t* sizes) {
    uint32_t total = 0;
    for (uint32_t i = 0; i < n_seg && i < 4; i++) total += sizes[i];
    if (total == 0 || n_elems % total) return -1;
    const uint32_t outer = n_elems / total;
    uint32_t start = 0;
    for (uint32_t k = 0; k < n_seg && k < 4; k++) {
        for (uint32_t o = 0; o < outer; o++)
            memcpy(y + (size_t)o * total + start, xs[k] + (size_t)o * sizes[k], sizes[k] * 2u);
        start += sizes[k];
    }
    return 0;
}

/* ---- OP_SPLIT_F16 (oplist_exec.c:1222-1256): segment split_index of a last-axis split;
 * x holds x_elems values, outer = x_elems / sum(sizes). */
int go_split(const uint16_t* x, uint32_t x_elems, uint16_t* y, uint32_t n_seg, const uint32_t* sizes,
             uint32_t split_index) {
    uint32_t total = 0;
    for (uint32_t i = 0; i < n_seg && i < 4; i++) total += sizes[i];
    if (total == 0 || x_elems == 0) return -1;
    const uint32_t outer = x_elems / total;
    uint32_t off = 0;
    for (uint32_t k = 0; k < n_seg && k < 4; k++) {
        if (k == split_index)
            for (uint32_t o = 0; o < outer; o++)
                memcpy(y + (size_t)o * sizes[k], x + (size_t)o * total + off, sizes[k] * 2u);
        off += sizes[k];
    }
    return 0;
}

/* ---- OP_REDUCE_F16 (oplist_exec.c:1258-1299): single-axis reduce over d[axis] with
 * inner = prod d[axis+1..3]; subtype 0 sum, 1 mean, 2 max, 3 min; f32 accumulate. */
int go_reduce(const uint16_t* x, uint16_t* y, uint32_t n, uint32_t axis, uint32_t subtype,
              const uint32_t* d) {
    if (axis >= 4 || subtype > 3) return -1;
    uint32_t L = d[axis] ? d[axis] : 1, inner = 1;
    for (uint32_t a = axis + 1; a < 4; a++) inner *= d[a];
    if ((uint64_t)L * inner == 0 || n % (L * inner)) return -1;
    const uint32_t outer = n / (L * inner);
    for (uint32_t o = 0; o < outer; o++)
        for (uint32_t i = 0; i < inner; i++) {
            const uint16_t* base = x + ((size_t)o * L) * inner + i;
            float acc = subtype == 2 ? -3.0e38f : subtype == 3 ? 3.0e38f : 0.0f;
            for (uint32_t l = 0; l < L; l++) {
                const float v = F(base[(size_t)l * inner]);
                if (subtype == 2) acc = v > acc ? v : acc;
                else if (subtype == 3) acc = v < acc ? v : acc;
                else acc += v;
            }
            if (subtype == 1) acc /= (float)L;
            y[(size_t)o * inner + i] = H(acc);
        }
    return 0;
}

/* ---- OP_PAD_F16 (oplist_exec.c:1301-1318): rows of in_inner -> out_inner with
 * pad_before values of pv, the row, then pv to the end. */
int go_pad(const uint16_t* x, uint16_t* y, uint32_t outer, uint32_t in_inner, uint32_t out_inner,
           uint32_t pad_before, uint16_t pv) {
    if (pad_before + in_inner > out_inner) return -1;
    for (uint32_t i = 0; i < outer; i++) {
        uint16_t* dst = y + (size_t)i * out_inner;
        for (uint32_t j = 0; j < pad_before; j++) dst[j] = pv;
        memcpy(dst + pad_before, x + (size_t)i * in_inner, (size_t)in_inner * 2u);
        for (uint32_t j = pad_before + in_inner; j < out_inner; j++) dst[j] = pv;
    }
    return 0;
}

/* ---- OP_CUMSUM_F32 (oplist_exec.c:1320-1347): per row, f32 running sum of f16
 * values, f16 out (exclusive: the sum before the element; reverse: from the end). */
int go_cumsum(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t n, uint32_t exclusive,
              uint32_t reverse) {
    for (uint32_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (uint32_t s = 0; s < n; s++) {
            const uint32_t i = reverse ? n - 1 - s : s;
            const size_t idx = (size_t)r * n + i;
            const float v = F(x[idx]);
            y[idx] = H(exclusive ? acc : acc + v);
            acc += v;
        }
    }
    return 0;
}

/* ---- OP_GATHER_F16 (oplist_exec.c:1378-1436): out shape od = td with axis replaced by
 * the index shape xd[0..xrank); out element i takes r = idx[il] (negative wraps once)
 * along axis of tbl, out-of-range r gives 0. packed = axis | xrank << 8 | irank << 16. */
int go_gather(const uint16_t* tbl, const int32_t* idx, uint16_t* y, uint32_t n, uint32_t packed,
              const uint32_t* td, const uint32_t* xd) {
    const uint32_t axis = packed & 0xFF, xrank = (packed >> 8) & 0xFF, irank = (packed >> 16) & 0xFF;
    if (axis >= irank || irank > 5 || xrank > 5 || xrank == 0) return -1;
    uint32_t od[5] = {1, 1, 1, 1, 1};
    for (uint32_t d = 0; d < axis && d < 5; d++) od[d] = td[d];
    for (uint32_t k = 0; k < xrank && axis + k < 5; k++) od[axis + k] = xd[k];
    for (uint32_t d = axis + 1; d < irank && d < 5; d++) {
        const uint32_t ocd = d + xrank - 1;
        if (ocd < 5) od[ocd] = td[d];
    }
    size_t os[5] = {1, 1, 1, 1, 1}, ts[5] = {1, 1, 1, 1, 1}, xs[5] = {1, 1, 1, 1, 1};
    for (int d = 3; d >= 0; d--) {
        os[d] = os[d + 1] * od[d + 1];
        ts[d] = ts[d + 1] * td[d + 1];
        xs[d] = xs[d + 1] * xd[d + 1];
    }
    for (uint32_t i = 0; i < n; i++) {
        size_t rem = i;
        uint32_t oc[5];
        for (int d = 0; d < 5; d++) { oc[d] = (uint32_t)(rem / os[d]); rem %= os[d]; }
        size_t il = 0;
        for (uint32_t k = 0; k < xrank && k < 5; k++) il += (oc[axis + k] % xd[k]) * xs[k];
        int32_t r = idx[il];
        if (r < 0) r += (int32_t)td[axis];
        if (r < 0 || r >= (int32_t)td[axis]) { y[i] = 0; continue; }
        size_t src = 0;
        for (uint32_t d = 0; d < axis && d < 5; d++) src += (size_t)oc[d] * ts[d];
        src += (size_t)r * ts[axis];
        for (uint32_t d = axis + 1; d < irank && d < 5; d++) {
            const uint32_t ocd = d + xrank - 1;
            src += (size_t)(ocd < 5 ? oc[ocd] : 0) * ts[d];
        }
        y[i] = tbl[src];
    }
    return 0;
}

/* ---- OP_TRANSPOSE_F16 (oplist_exec.c:983-1011): 4-D (1, H, W, C) permutation, perm
 * one byte per output axis (the input axis it takes). */
int go_transpose4(const uint16_t* x, uint16_t* y, uint32_t Hh, uint32_t W, uint32_t Cc, uint32_t perm) {
    const uint32_t p[4] = {perm & 0xFF, (perm >> 8) & 0xFF, (perm >> 16) & 0xFF, (perm >> 24) & 0xFF};
    for (int i = 0; i < 4; i++)
        if (p[i] > 3) return -1;
    const uint32_t dims[4] = {1, Hh, W, Cc};
    const size_t si[4] = {(size_t)Hh * W * Cc, (size_t)W * Cc, Cc, 1};
    for (uint32_t o0 = 0; o0 < dims[p[0]]; o0++)
        for (uint32_t o1 = 0; o1 < dims[p[1]]; o1++)
            for (uint32_t o2 = 0; o2 < dims[p[2]]; o2++)
                for (uint32_t o3 = 0; o3 < dims[p[3]]; o3++) {
                    const uint32_t oc[4] = {o0, o1, o2, o3};
                    uint32_t ic[4] = {0, 0, 0, 0};
                    for (int ax = 0; ax < 4; ax++) ic[p[ax]] = oc[ax];
                    const size_t src = ic[0] * si[0] + ic[1] * si[1] + ic[2] * si[2] + ic[3] * si[3];
                    y[(((size_t)o0 * dims[p[1]] + o1) * dims[p[2]] + o2) * dims[p[3]] + o3] = x[src];
                }
    return 0;
}

/* ---- OP_BROADCAST_F16 (oplist_exec.c:1876-1907): right-aligned broadcast of b [in_d]
 * to [out_d] (4 dims each, trailing 1s of out_d trimmed, in_d taken to the same rank);
 * an input dim of 1 repeats, any other dim d indexes (coordinate mod d). */
int go_broadcast(const uint16_t* x, uint16_t* y, uint32_t n, const uint32_t* in_d, const uint32_t* out_d) {
    uint32_t r = 4;
    while (r > 0 && out_d[r - 1] == 1) r--;
    uint32_t ir = 4;
    if (r == 0) r = 1;
    if (ir > r) ir = r;
    uint32_t istr[4] = {1, 1, 1, 1}, ostr[4] = {1, 1, 1, 1};
    for (int i = (int)ir - 2; i >= 0; i--) istr[i] = istr[i + 1] * in_d[i + 1];
    for (int i = (int)r - 2; i >= 0; i--) ostr[i] = ostr[i + 1] * out_d[i + 1];
    const uint32_t lead = r - ir;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t rem = i, in_lin = 0;
        for (uint32_t d = 0; d < r; d++) {
            const uint32_t c = rem / ostr[d];
            rem %= ostr[d];
            if (d < lead) continue;
            const uint32_t idim = in_d[d - lead];
            if (idim > 1) in_lin += (c % idim) * istr[d - lead];
        }
        y[i] = x[in_lin];
    }
    return 0;
}

/* ---- OP_TRANSPOSE_GEN_F16 (oplist_exec.c:1910-1948): C-order rank-2..4 transpose of
 * x [dims], output axis i = input axis perm byte i. */
int go_transpose_gen(const uint16_t* x, uint16_t* y, uint32_t rk, const uint32_t* dims, uint32_t perm) {
    if (rk < 2 || rk > 4) return -1;
    const uint32_t p[4] = {perm & 0xFF, (perm >> 8) & 0xFF, (perm >> 16) & 0xFF, (perm >> 24) & 0xFF};
    size_t n = 1;
    for (uint32_t i = 0; i < rk; i++) n *= dims[i];
    uint32_t si[4], so[4];
    si[rk - 1] = 1;
    so[rk - 1] = 1;
    for (int i = (int)rk - 2; i >= 0; i--) {
        si[i] = si[i + 1] * dims[i + 1];
        so[i] = so[i + 1] * (p[i + 1] >= rk ? 1u : dims[p[i + 1]]);
    }
    for (size_t t = 0; t < n; t++) {
        uint32_t rem = (uint32_t)t, ic[4] = {0, 0, 0, 0};
        for (uint32_t i = 0; i < rk; i++) { ic[i] = rem / si[i]; rem %= si[i]; }
        uint32_t ot = 0;
        for (uint32_t ax = 0; ax < rk; ax++) ot += ic[p[ax]] * so[ax];
        y[ot] = x[t];
    }
    return 0;
}

/* ---- OP_STRIDED_SLICE_F16 (oplist_exec.c:1950-1988): rank 1..3, output element i at
 * input coordinates b[ax] + c[ax] * s[ax] (c = C-order coordinates of i over the slice
 * extents ceil((e - b) / s)); stride 0 reads as 1. */
int go_slice(const uint16_t* x, uint16_t* y, uint32_t n_out, uint32_t rk, const uint32_t* b, const uint32_t* e,
             const uint32_t* s, const uint32_t* d) {
    if (rk < 1 || rk > 3) return -1;
    uint32_t ss[3], od[3] = {1, 1, 1}, istr[3], ostr[3];
    for (uint32_t ax = 0; ax < rk; ax++) {
        ss[ax] = s[ax] ? s[ax] : 1u;
        const uint32_t span = e[ax] > b[ax] ? e[ax] - b[ax] : 0;
        od[ax] = (span + ss[ax] - 1) / ss[ax];
    }
    istr[rk - 1] = 1;
    ostr[rk - 1] = 1;
    for (int i = (int)rk - 2; i >= 0; i--) {
        istr[i] = istr[i + 1] * d[i + 1];
        ostr[i] = ostr[i + 1] * od[i + 1];
    }
    for (uint32_t i = 0; i < n_out; i++) {
        uint32_t rem = i, in_lin = 0;
        for (uint32_t ax = 0; ax < rk; ax++) {
            const uint32_t c = rem / ostr[ax];
            rem %= ostr[ax];
            in_lin += (b[ax] + c * ss[ax]) * istr[ax];
        }
        y[i] = x[in_lin];
    }
    return 0;
}
