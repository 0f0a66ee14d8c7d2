// wt_parse.cpp — WTOP blob parser and the W3 inspect report.
//
// Behaviour follows the reference parser (kernels/src/runtime/oplist_parse.c:86-169):
// the same checks in the same order, so every malformed blob yields the same
// WT_ERR_* code. The op metadata (arity, which argument positions are slot
// references) lives in one table instead of two switch statements.
#include <atomic>
#include <cstdio>
#include <cstring>

#include "oplist_parse.h"

namespace {

// Per-opcode metadata: arity, and a bit mask of argument positions that may hold a
// slot reference (reference oplist_parse.c:10-84). arity < 0 = unknown opcode.
struct OpInfo {
    int arity;
    uint32_t slot_args;
};

constexpr uint32_t bits(std::initializer_list<int> idx) {
    uint32_t m = 0;
    for (int i : idx) m |= 1u << i;
    return m;
}

struct OpTable {
    OpInfo info[64];
    constexpr OpTable() : info{} {
        for (auto& i : info) i = {-1, 0};
        info[OP_NOP] = {WT_ARITY_NOP, 0};
        info[OP_MATMUL_W4A16] = {WT_ARITY_MATMUL, bits({0, 1})};
        info[OP_RMSNORM_F16] = {WT_ARITY_RMSNORM, bits({1})};
        info[OP_PIN] = {WT_ARITY_PIN, bits({0})};
        info[OP_SILU_F16] = {WT_ARITY_SILU, 0};
        info[OP_IM2COL] = {WT_ARITY_IM2COL, 0};
        info[OP_CONV2D_F16] = {WT_ARITY_CONV2D_F16, bits({1, 2})};
        info[OP_ADD_F16] = {WT_ARITY_ADD_F16, 0};
        info[OP_SPILL] = {WT_ARITY_SPILL, bits({1})};
        info[OP_FILL] = {WT_ARITY_FILL, bits({0})};
        info[OP_TRANSPOSE_F16] = {WT_ARITY_TRANSPOSE_F16, 0};
        info[OP_UNARY_F16] = {WT_ARITY_UNARY_F16, bits({0})};
        info[OP_BINARY_F16] = {WT_ARITY_BINARY_F16, bits({0, 1})};
        info[OP_SOFTMAX_F16] = {WT_ARITY_SOFTMAX_F16, bits({0})};
        info[OP_CONCAT_F16] = {WT_ARITY_CONCAT_F16, bits({0, 1, 2, 3, 4, 5, 6, 7})};
        info[OP_STRIDED_SLICE_F16] = {WT_ARITY_STRIDED_SLICE_F16, bits({0})};
        info[OP_SPLIT_F16] = {WT_ARITY_SPLIT_F16, bits({0})};
        info[OP_REDUCE_F16] = {WT_ARITY_REDUCE_F16, bits({0})};
        info[OP_CUMSUM_F32] = {WT_ARITY_CUMSUM_F32, bits({0})};
        info[OP_CONV1D_SSM_F16] = {WT_ARITY_CONV1D_SSM_F16, bits({0, 1})};
        info[OP_GATHER_F16] = {WT_ARITY_GATHER_F16, bits({0, 1})};
        info[OP_ARGMAX_F16] = {WT_ARITY_ARGMAX_F16, bits({0})};
        info[OP_KV_APPEND_F16] = {WT_ARITY_KV_APPEND_F16, bits({0, 1, 2})};
        info[OP_KV_GATHER_F16] = {WT_ARITY_KV_GATHER_F16, bits({0, 1})};
        info[OP_MATMUL_F16] = {WT_ARITY_MATMUL_F16, bits({0, 1})};
        info[OP_RMSNORM2_F16] = {WT_ARITY_RMSNORM2_F16, bits({1, 2})};
        info[OP_BROADCAST_F16] = {WT_ARITY_BROADCAST_F16, bits({0})};
        info[OP_TRANSPOSE_GEN_F16] = {WT_ARITY_TRANSPOSE_GEN_F16, bits({0})};
        info[OP_SCATTER_ND_F16] = {WT_ARITY_SCATTER_ND_F16, bits({0, 1, 2})};
        info[OP_CONV1D_SSM_STEP_F16] = {WT_ARITY_CONV1D_SSM_STEP_F16, bits({0, 1})};
        info[OP_DELTA_CHUNK_F16] = {WT_ARITY_DELTA_CHUNK_F16, bits({0, 1, 2, 3, 4})};
        info[OP_DMA] = {WT_ARITY_DMA, bits({0, 1})};
        info[OP_PAD_F16] = {WT_ARITY_PAD_F16, bits({0})};
        info[OP_MATMUL_F16_SPLIT] = {WT_ARITY_MATMUL_F16_SPLIT, bits({0, 1})};
        // additions of this library
        info[OP_MATMUL_W4G_F16] = {WT_ARITY_MATMUL_W4G_F16, bits({0, 1, 2})};
        info[OP_ATTN_F16] = {WT_ARITY_ATTN_F16, bits({0, 1, 2})};
        info[OP_ATTN_DECODE_F16] = {WT_ARITY_ATTN_DECODE_F16, bits({0})};
        info[OP_ROPE_F16] = {WT_ARITY_ROPE_F16, bits({0})};
        info[OP_KV_APPEND_N_F16] = {WT_ARITY_KV_APPEND_N_F16, bits({0, 1})};
        info[OP_W4G_FUSED_F16] = {WT_ARITY_W4G_FUSED_F16, bits({0, 1, 2, 7, 8})};
        info[OP_QK_ROPE_KV_F16] = {WT_ARITY_QK_ROPE_KV_F16, bits({0, 9, 10})};
        info[OP_ATTN_DECODE_QKV_F16] = {WT_ARITY_ATTN_DECODE_QKV_F16, bits({0, 6, 7})};
    }
};

constexpr OpTable kOps{};

inline const OpInfo* op_info(uint16_t opcode) {
    if (opcode >= 64 || kOps.info[opcode].arity < 0) return nullptr;
    return &kOps.info[opcode];
}

}  // namespace

namespace gehtp {
// Bumped by every successful wt_parse: the engine's per-blob caches (fused op chains)
// are keyed by it, so a re-parsed blob, even at the same address, is analysed afresh.
std::atomic<uint64_t> g_parse_epoch{0};
}  // namespace gehtp

extern "C" int wt_parse(const uint8_t* buf, size_t size, struct wt_blob* out) {
    if (!buf || !out || size < 16u) return WT_ERR_SHORT;
    if (std::memcmp(buf, "WTOP", 4) != 0) return WT_ERR_MAGIC;
    out->ver = wt_rd_u16(buf + 4);
    if (out->ver != WT_BLOB_VER && out->ver != WT_BLOB_VER_2) return WT_ERR_VER;
    if (wt_rd_u16(buf + 6) != WT_ENDIAN_CHK) return WT_ERR_ENDIAN;
    out->n_slots = wt_rd_u32(buf + 8);
    out->n_ops = wt_rd_u32(buf + 12);
    if (out->n_slots == 0 || out->n_slots > WT_MAX_SLOTS) return WT_ERR_NSLOTS;
    if (out->n_ops == 0 || out->n_ops > WT_MAX_OPS) return WT_ERR_NOPS;

    const bool v2 = out->ver >= WT_BLOB_VER_2;
    const size_t rec = v2 ? WT_SLOT_SIZE_V2 : WT_SLOT_SIZE;
    const size_t slots_end = 16u + (size_t)out->n_slots * rec;
    if (size < slots_end) return WT_ERR_SLOTS_OVERRUN;
    for (uint32_t i = 0; i < out->n_slots; ++i) {
        const uint8_t* r = buf + 16u + (size_t)i * rec;
        wt_slot& s = out->slots[i];
        s.len = wt_rd_u32(r);
        s.count = wt_rd_u32(r + 4);
        if (v2) {
            s.offset = (uint64_t)wt_rd_u32(r + 8) | ((uint64_t)wt_rd_u32(r + 12) << 32);
            s.addr = wt_rd_u32(r + 16);
        } else {
            s.offset = wt_rd_u32(r + 8);
            s.addr = wt_rd_u32(r + 12);
        }
        if (s.len == 0) return WT_ERR_WEIGHT_OVERRUN;
        if (s.offset % WT_WEIGHT_ALIGN) return WT_ERR_ALIGN;
        // v1 offsets are 32-bit: the slot must end below 4 GiB.
        if (!v2 && s.offset + s.len > 0xFFFFFFFFull) return WT_ERR_WEIGHT_OVERRUN;
    }

    size_t p = slots_end;
    for (uint32_t i = 0; i < out->n_ops; ++i) {
        if (size < p + 4u) return WT_ERR_OP_TRUNC;
        const uint16_t opcode = wt_rd_u16(buf + p);
        const uint16_t n_args = wt_rd_u16(buf + p + 2);
        const OpInfo* info = op_info(opcode);
        if (!info) return WT_ERR_OPCODE;
        if (n_args != (uint16_t)info->arity) return WT_ERR_ARITY;
        if (size < p + 4u + (size_t)n_args * 4u) return WT_ERR_OP_TRUNC;
        wt_op& op = out->ops[i];
        op.opcode = opcode;
        op.n_args = n_args;
        for (uint16_t a = 0; a < n_args; ++a) op.args[a] = wt_rd_u32(buf + p + 4u + 4u * a);
        p += 4u + 4u * (size_t)n_args;
    }

    // The weight region starts at the first 128-byte boundary after the op table;
    // the reference computes this in 32 bits.
    const uint32_t p32 = (uint32_t)p;
    out->weight_off = WT_WEIGHT_ALIGN * ((p32 + WT_WEIGHT_ALIGN - 1u) / WT_WEIGHT_ALIGN);
    if ((size_t)out->weight_off > size) return WT_ERR_WEIGHT_OVERRUN;
    out->weight_base = buf + out->weight_off;
    out->weight_bytes = size - out->weight_off;

    for (uint32_t i = 0; i < out->n_slots; ++i) {
        const wt_slot& s = out->slots[i];
        if (s.addr == WT_SLOT_EXT_WGT) continue;  // lives in the external image
        if (s.offset + (uint64_t)s.len > out->weight_bytes) return WT_ERR_WEIGHT_OVERRUN;
    }
    for (uint32_t i = 0; i < out->n_ops; ++i) {
        const wt_op& op = out->ops[i];
        const uint32_t mask = op_info(op.opcode)->slot_args;
        for (uint16_t a = 0; a < op.n_args; ++a) {
            if (!(mask & (1u << a))) continue;
            const uint32_t v = op.args[a];
            // OP_DMA may name an engine surface (0xC000|id) instead of a slot.
            if (op.opcode == OP_DMA && (v & 0xC000u) == 0xC000u) continue;
            // Optional references of the added fused opcodes.
            if (v == WT_REF_NONE && op.opcode >= OP_W4G_FUSED_F16) continue;
            // Only 0x8000-tagged values address slot space; bare ids are temps.
            if ((v & 0x8000u) && (v & 0x7FFFu) >= out->n_slots) return WT_ERR_BAD_REF;
        }
    }
    gehtp::g_parse_epoch.fetch_add(1, std::memory_order_relaxed);
    return WT_OK;
}

extern "C" const char* wt_err_str(int rc) {
    switch (rc) {
    case WT_OK: return "OK";
    case WT_ERR_SHORT: return "buffer shorter than header";
    case WT_ERR_MAGIC: return "bad magic";
    case WT_ERR_VER: return "unsupported version";
    case WT_ERR_ENDIAN: return "endian check failed";
    case WT_ERR_NSLOTS: return "n_slots out of range";
    case WT_ERR_NOPS: return "n_ops out of range";
    case WT_ERR_SLOTS_OVERRUN: return "slot table overruns buffer";
    case WT_ERR_WEIGHT_OVERRUN: return "slot offset+len overruns weight region";
    case WT_ERR_OP_TRUNC: return "op table truncated";
    case WT_ERR_OPCODE: return "unknown opcode";
    case WT_ERR_ARITY: return "n_args mismatch for opcode";
    case WT_ERR_BAD_REF: return "op arg references missing slot";
    case WT_ERR_ALIGN: return "slot offset not 128B aligned";
    default: return "unknown";
    }
}

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4), used only by the W3 report below.
namespace {

struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t blk[64];
    size_t fill = 0;
    uint64_t total = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void compress(const uint8_t* p) {
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
            0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
            0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
            0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
            0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
            0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
            0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
            0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
            0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
            0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
            0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
                   (uint32_t)p[4 * i + 2] << 8 | (uint32_t)p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }

    void update(const uint8_t* p, size_t n) {
        total += n;
        while (n) {
            size_t take = 64 - fill < n ? 64 - fill : n;
            std::memcpy(blk + fill, p, take);
            fill += take; p += take; n -= take;
            if (fill == 64) { compress(blk); fill = 0; }
        }
    }

    void hex(char out[65]) {
        const uint64_t bitlen = total * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t lenb[8];
        for (int i = 0; i < 8; ++i) lenb[i] = (uint8_t)(bitlen >> (56 - 8 * i));
        update(lenb, 8);
        for (int i = 0; i < 8; ++i) std::snprintf(out + 8 * i, 9, "%08x", h[i]);
    }
};

void sha256_hex(const uint8_t* p, size_t n, char out[65]) {
    Sha256 s;
    if (p && n) s.update(p, n);
    s.hex(out);
}

}  // namespace

// W3 report lines (reference kernels/src/runtime/wt_w3.c:8-47): same keys and order.
extern "C" void wt_w3_report(const char* blob_name, const uint8_t* buf, size_t size,
                             const struct wt_blob* w,
                             void (*emit)(const char* line, void* ud), void* ud) {
    char line[1024], sha[65], wsha[65];
    sha256_hex(buf, size, sha);
    sha256_hex(w->weight_base, w->weight_bytes, wsha);
    std::snprintf(line, sizeof line,
                  "{\"t\":\"W3\",\"mode\":\"parse\",\"blob\":\"%s\",\"ver\":%u,\"endian_chk\":%u,"
                  "\"n_slots\":%u,\"n_ops\":%u,\"blob_bytes\":%zu,\"blob_sha256\":\"%s\","
                  "\"weight_off\":%u,\"weight_bytes\":%zu,\"weight_sha256\":\"%s\"}",
                  blob_name, (unsigned)w->ver, (unsigned)WT_ENDIAN_CHK, w->n_slots, w->n_ops, size,
                  sha, w->weight_off, w->weight_bytes, wsha);
    emit(line, ud);
    for (uint32_t i = 0; i < w->n_slots; ++i) {
        const wt_slot& s = w->slots[i];
        const bool inline_data = s.addr != WT_SLOT_EXT_WGT && s.offset + s.len <= w->weight_bytes;
        sha256_hex(inline_data ? w->weight_base + s.offset : nullptr, inline_data ? s.len : 0, sha);
        // The reference prints the (in-memory 64-bit) offset through %u.
        std::snprintf(line, sizeof line,
                      "{\"t\":\"W3\",\"slot\":%u,\"len\":%u,\"count\":%u,\"offset\":%u,\"addr\":%u,"
                      "\"sha256\":\"%s\"}",
                      i, s.len, s.count, (unsigned)s.offset, s.addr, sha);
        emit(line, ud);
    }
    for (uint32_t i = 0; i < w->n_ops; ++i) {
        char args[200] = "";
        int off = 0;
        for (uint16_t a = 0; a < w->ops[i].n_args && off < (int)sizeof args; ++a)
            off += std::snprintf(args + off, sizeof args - off, "%s%u", a ? "," : "", w->ops[i].args[a]);
        std::snprintf(line, sizeof line,
                      "{\"t\":\"W3\",\"op\":%u,\"opcode\":%u,\"n_args\":%u,\"args\":[%s]}",
                      i, (unsigned)w->ops[i].opcode, (unsigned)w->ops[i].n_args, args);
        emit(line, ud);
    }
    emit("{\"t\":\"W3\",\"verdict\":\"PASS\"}", ud);
}
