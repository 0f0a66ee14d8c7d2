/* oplist_parse.h — WTOP runlist blob: wire format, limits, opcodes, parser ABI.
 *
 * Drop-in for GEHTP's parser header (reference: kernels/include/oplist_parse.h).
 * Every constant, enum value and struct layout below is byte-compatible with the
 * reference so that a blob written by the reference emitter parses unchanged and
 * callers compiled against the reference header link against this library.
 *
 * Wire format (all little-endian):
 *   +0   "WTOP"
 *   +4   u16 version   (1: 16-byte slot records, 2: 24-byte slot records)
 *   +6   u16 0x1234    (endianness check)
 *   +8   u32 n_slots   (1..WT_MAX_SLOTS)
 *   +12  u32 n_ops     (1..WT_MAX_OPS)
 *   +16  slot records  v1 {len, count, offset32, addr}
 *                      v2 {len, count, offset_lo, offset_hi, addr, reserved}
 *   then op records    {u16 opcode, u16 n_args, u32 args[n_args]}
 *   then weight region, starting at the first 128-byte boundary after the ops;
 *        each slot's offset (relative to the region) is 128-byte aligned.
 *
 * Argument references (reference: oplist_exec.c:175-213):
 *   0x8000|s  slot s            0x6000|i  persistent state i
 *   0x4000|t  "VTCM-resident" temp t (here: a separate HBM sub-arena)
 *   t         ordinary temp t
 *
 * Opcodes 40..42 are additions of this library (no counterpart in the
 * reference); see their comments.
 */
#ifndef OPLIST_PARSE_H
#define OPLIST_PARSE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format constants (reference oplist_parse.h:42-58). */
#define WT_BLOB_VER 1u
#define WT_BLOB_VER_2 2u
#define WT_SLOT_SIZE_V2 24u
#define WT_ENDIAN_CHK 0x1234u
#define WT_SLOT_SIZE 16u
#define WT_WEIGHT_ALIGN 128u
#define WT_MAX_SLOTS 4096u
#define WT_MAX_OPS 65536u
#define WT_MAX_ARGS 16u

/* Slot address sentinels (reference oplist_parse.h:59-92). */
#define WT_SLOT_EXT_IN  0xFFFFFFFFu  /* data comes from run_io's in_ptr          */
#define WT_SLOT_EXT_OUT 0xFFFFFFFEu  /* output copy target marker                */
#define WT_SLOT_TEMPOFF 0xFFFFFFFDu  /* static temp plan: [cap][reserve][n][n*{tid,off,size}] */
#define WT_SLOT_EXT_WGT 0xFFFFFFFCu  /* weights live in the external weight image */
#define WT_REF_VTCM_FLAG 0x4000u
#define WT_SLOT_STATE 0xFFFFFFFBu    /* persistent states: [n][n*{bytes}]          */
#define WT_REF_STATE_FLAG 0x6000u
#define WT_MAX_STATES 64u
#define WT_KV_POS_AUTO 0xFFFFFFFAu   /* KV position driven by the state's counter  */
#define WT_REF_ENG_FLAG 0xC000u      /* OP_DMA only: engine surface reference      */
#define WT_ENG_ACT 0u
#define WT_ENG_OUT 1u
#define WT_ENG_WT 2u
#define WT_ENG_BIAS 3u
#define WT_DMA_FENCE_NONE 0xFFu

/* Opcodes (reference oplist_parse.h:103-215). */
enum {
    OP_NOP = 0,
    OP_MATMUL_W4A16 = 1,
    OP_RMSNORM_F16 = 2,
    OP_PIN = 3,
    OP_SILU_F16 = 4,
    OP_IM2COL = 5,
    OP_CONV2D_F16 = 6,
    OP_ADD_F16 = 7,
    OP_SPILL = 8,
    OP_FILL = 9,
    OP_TRANSPOSE_F16 = 10,
    OP_UNARY_F16 = 11,
    OP_BINARY_F16 = 12,
    OP_SOFTMAX_F16 = 13,
    OP_CONCAT_F16 = 14,
    OP_STRIDED_SLICE_F16 = 15,
    OP_SPLIT_F16 = 16,
    OP_REDUCE_F16 = 17,
    OP_CUMSUM_F32 = 18,
    OP_CONV1D_SSM_F16 = 19,
    OP_GATHER_F16 = 20,
    OP_ARGMAX_F16 = 21,
    OP_KV_APPEND_F16 = 22,
    OP_KV_GATHER_F16 = 23,
    OP_MATMUL_F16 = 24,
    OP_RMSNORM2_F16 = 25,
    OP_BROADCAST_F16 = 26,
    OP_TRANSPOSE_GEN_F16 = 27,
    OP_SCATTER_ND_F16 = 28,
    OP_CONV1D_SSM_STEP_F16 = 29,
    OP_DELTA_CHUNK_F16 = 30,
    OP_DMA = 33,
    OP_PAD_F16 = 34,
    OP_MATMUL_F16_SPLIT = 35,

    /* ---- additions (no reference counterpart) ----
     * OP_MATMUL_W4G_F16: y[M,N] = a[M,K] . dequant(W)^T, fp16 in/out, fp32 accumulate.
     *   args [a_ref, wq_ref, ws_ref, out_t, M, K, N, group, flags]
     *   wq: N*K/2 bytes, row n holds K/2 bytes; byte j = k=2j in the low nibble,
     *       k=2j+1 in the high nibble; value = nibble - 8 (offset binary, like Q4_0).
     *   ws: N*(K/group) fp16 scales, row-major.  dequant(W)[n,k] = fp16(q * s).
     *   flags: bit1 must be set (W stored [N,K]); bits 16..31 = row stride of the
     *   output in elements when nonzero (lets several linears write one buffer).
     *   group must be 64 in this build; K % 64 == 0. */
    OP_MATMUL_W4G_F16 = 40,
    /* OP_ATTN_F16: fused causal GQA attention over a prefill chunk.
     *   args [q_ref, k_ref, v_ref, out_t, S, H, KVH, hd, scale_f32_bits, flags]
     *   q [S, H, hd], k/v [S, KVH, hd] token-major, out [S, H, hd].
     *   flags bit0 = causal. q head h reads kv head h / (H / KVH). scale must be
     *   positive and finite (the chain form below takes any scale).
     *   Replaces the runlist chain MATMUL_F16(batched) -> BINARY mul -> BINARY add
     *   (mask) -> SOFTMAX -> MATMUL_F16 (reference oplist_exec.c:1081-1194,1709-1813). */
    OP_ATTN_F16 = 41,
    /* OP_ATTN_DECODE_F16: attention of one new token against a KV ring state.
     *   args [q_ref, state_ref, out_t, n_kv, H, KVH, hd, scale_f32_bits]
     *   q [H, hd]; state = KV ring written by OP_KV_APPEND_F16 (slot-major,
     *   K face | V face, each [KVH, hd]); n_kv may be WT_KV_POS_AUTO.
     *   Replaces KV_GATHER -> MATMUL_F16 -> BINARY add -> SOFTMAX -> MATMUL_F16. */
    OP_ATTN_DECODE_F16 = 42,
    /* OP_ROPE_F16: rotary embedding (half-split, NeoX/Qwen layout) in place of the
     *   runlist's slice/mul/add chain.
     *   args [x_ref, y_t, n_tok, n_heads, hd, pos0, theta_f32_bits, row_stride]
     *   x/y [n_tok, row_stride] fp16, heads at column h*hd; position of token t is
     *   pos0 + t, or (state counter of 0x6000|i) + t when pos0 == 0x6000|i. */
    OP_ROPE_F16 = 43,
    /* OP_KV_APPEND_N_F16: append n_tok consecutive tokens to a KV ring state.
     *   args [k_ref, v_ref, state_ref, pos, n_tok, kv_elems]
     *   k/v [n_tok, kv_elems]; token t goes to position pos + t (pos may be
     *   WT_KV_POS_AUTO: the state's counter, advanced by n_tok). Same ring as
     *   OP_KV_APPEND_F16, which appends exactly one token. */
    OP_KV_APPEND_N_F16 = 44,
    /* OP_W4G_FUSED_F16: OP_MATMUL_W4G_F16 with the ops around a decoder linear folded in.
     *   args [a_ref, wq_ref, ws_ref, out_t, M, K, N, gamma_ref, res_ref, mode, flags]
     *   gamma_ref != WT_REF_NONE: a := RMSNORM2_F16(a, gamma, zero bias) first.
     *   mode 0: y = a.dequant(W)^T (N output columns).
     *   mode 1 (SwiGLU): weight rows interleaved, row 2j = gate j, row 2j+1 = up j;
     *          y[:, j] = f16(f16(silu(f16(gate))) * f16(up)), N/2 output columns
     *          (= UNARY_F16 silu then BINARY_F16 mul).
     *   res_ref != WT_REF_NONE: y = f16(y + res) (= ADD_F16), res [M, N_out].
     *   flags: bit1 must be set; bits 16..31 = output row stride (0 = N_out).
     *   Each fused step rounds exactly where the op it replaces does. */
    OP_W4G_FUSED_F16 = 45,
    /* OP_QK_ROPE_KV_F16: per-head QK RMSNorm + RoPE + KV append for a fused QKV row.
     *   args [qkv_ref, q_out_t, k_out_t, v_out_t, state_ref, n_tok, H, KVH, hd,
     *         q_gamma_ref, k_gamma_ref, theta_f32_bits]
     *   qkv [n_tok, (H + 2*KVH)*hd] rows [q | k | v]; hd == 128; H + KVH <= 64.
     *   q_out[t] = ROPE(RMSNORM2(q_t, q_gamma)), k_t = ROPE(RMSNORM2(k_t, k_gamma)) and
     *   v_t are appended to the ring at the state's counter (advanced by n_tok);
     *   k_out_t / v_out_t (WT_REF_NONE to skip) receive k_t / v_t token-major.
     *   RoPE positions = counter + t. Replaces RMSNORM2 x2, ROPE x2, KV_APPEND_N. */
    OP_QK_ROPE_KV_F16 = 46,
    /* OP_ATTN_DECODE_QKV_F16: one decode step of a layer's attention from the raw fused
     *   QKV row: OP_QK_ROPE_KV_F16 (n_tok 1) then OP_ATTN_DECODE_F16 at n_kv = counter + 1.
     *   args [qkv_ref, state_ref, out_t, H, KVH, hd, q_gamma_ref, k_gamma_ref,
     *         theta_f32_bits, scale_f32_bits]
     *   qkv [(H + 2*KVH)*hd] = [q | k | v]; hd == 128; the new k/v go to the ring at the
     *   state's counter, which is then advanced by one. out [H, hd]. */
    OP_ATTN_DECODE_QKV_F16 = 47,
};

/* "No reference" argument value of the added opcodes. */
#define WT_REF_NONE 0xFFFFFFFFu

/* Arities (reference oplist_parse.h:218-251). */
#define WT_ARITY_NOP 0
#define WT_ARITY_MATMUL 6
#define WT_ARITY_RMSNORM 4
#define WT_ARITY_PIN 1
#define WT_ARITY_SILU 3
#define WT_ARITY_IM2COL 15
#define WT_ARITY_CONV2D_F16 13
#define WT_ARITY_ADD_F16 4
#define WT_ARITY_SPILL 4
#define WT_ARITY_FILL 4
#define WT_ARITY_TRANSPOSE_F16 6
#define WT_ARITY_UNARY_F16 4
#define WT_ARITY_BINARY_F16 5
#define WT_ARITY_SOFTMAX_F16 4
#define WT_ARITY_CONCAT_F16 16
#define WT_ARITY_STRIDED_SLICE_F16 16
#define WT_ARITY_SPLIT_F16 16
#define WT_ARITY_REDUCE_F16 9
#define WT_ARITY_CUMSUM_F32 7
#define WT_ARITY_CONV1D_SSM_F16 6
#define WT_ARITY_GATHER_F16 15
#define WT_ARITY_ARGMAX_F16 3
#define WT_ARITY_KV_APPEND_F16 4
#define WT_ARITY_KV_GATHER_F16 7
#define WT_ARITY_MATMUL_F16 7
#define WT_ARITY_RMSNORM2_F16 5
#define WT_ARITY_BROADCAST_F16 12
#define WT_ARITY_TRANSPOSE_GEN_F16 8
#define WT_ARITY_SCATTER_ND_F16 14
#define WT_ARITY_DMA 8
#define WT_ARITY_PAD_F16 7
#define WT_ARITY_MATMUL_F16_SPLIT 9
#define WT_ARITY_CONV1D_SSM_STEP_F16 6
#define WT_ARITY_DELTA_CHUNK_F16 12
#define WT_ARITY_MATMUL_W4G_F16 9
#define WT_ARITY_ATTN_F16 10
#define WT_ARITY_ATTN_DECODE_F16 8
#define WT_ARITY_ROPE_F16 8
#define WT_ARITY_KV_APPEND_N_F16 6
#define WT_ARITY_W4G_FUSED_F16 11
#define WT_ARITY_QK_ROPE_KV_F16 12
#define WT_ARITY_ATTN_DECODE_QKV_F16 10

/* In-memory records (reference oplist_parse.h:253-275); layouts are ABI. */
struct wt_slot {
    uint32_t len;
    uint32_t count;
    uint64_t offset;   /* byte offset in the weight region (or external image) */
    uint32_t addr;     /* 0 or one of the WT_SLOT_* sentinels */
};

struct wt_op {
    uint16_t opcode;
    uint16_t n_args;
    uint32_t args[WT_MAX_ARGS];
};

struct wt_blob {
    uint16_t ver;
    uint32_t n_slots;
    uint32_t n_ops;
    uint32_t weight_off;
    struct wt_slot slots[WT_MAX_SLOTS];
    struct wt_op ops[WT_MAX_OPS];
    const uint8_t* weight_base;   /* points into the caller's blob buffer */
    size_t weight_bytes;
};

/* Error codes (reference oplist_parse.h:277-292). */
enum {
    WT_OK = 0,
    WT_ERR_SHORT = -1,
    WT_ERR_MAGIC = -2,
    WT_ERR_VER = -3,
    WT_ERR_ENDIAN = -4,
    WT_ERR_NSLOTS = -5,
    WT_ERR_NOPS = -6,
    WT_ERR_SLOTS_OVERRUN = -7,
    WT_ERR_WEIGHT_OVERRUN = -8,
    WT_ERR_OP_TRUNC = -9,
    WT_ERR_OPCODE = -10,
    WT_ERR_ARITY = -11,
    WT_ERR_BAD_REF = -12,
    WT_ERR_ALIGN = -13,
};

/* Parse and bounds-check a blob (reference oplist_parse.c:86-169).
 * Returns WT_OK or a negative WT_ERR_*; *out is valid only on WT_OK. */
int wt_parse(const uint8_t* buf, size_t size, struct wt_blob* out);

/* Human-readable text for a wt_parse return code (reference oplist_parse.c:171-189). */
const char* wt_err_str(int rc);

static inline uint32_t wt_rd_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) |
           ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline uint16_t wt_rd_u16(const uint8_t* p) {
    return (uint16_t)((uint16_t)p[0] | ((uint16_t)p[1] << 8));
}

#ifdef __cplusplus
}
#endif

#endif /* OPLIST_PARSE_H */
