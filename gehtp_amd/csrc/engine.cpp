// engine.cpp — the runlist engine: GEHTP's wt_exec_* ABI on one HIP device.
//
// Structure follows the reference engine (kernels/src/runtime/oplist_exec.c): a
// process-wide singleton, temps addressed by id, the TEMPOFF static plan with a
// bump fallback, persistent states, EXT_IN / EXT_WGT slots, and table dispatch by
// opcode. What differs is where data lives and who computes:
//   - the blob's weight region (and the external weight image) is copied to HBM
//     once per blob; temps, states and the "VTCM" pool are HBM allocations;
//   - each op enqueues gfx950 kernels on the engine stream; a run drains the stream
//     before returning; there is no CPU compute path for any op;
//   - KV ring bookkeeping (positions, counters) is mirrored on the host for the
//     reference's hard-error checks, and on the device so kernels read positions;
//   - a run repeated with the same ops and the same device buffers (a decode step)
//     is replayed as a HIP graph, which halves the per-kernel launch cost.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.h"
#include "oplist_exec.h"
#include "oplist_parse.h"

namespace gehtp {

int device_cu_count() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return cus;
}

extern std::atomic<uint64_t> g_parse_epoch;   // wt_parse.cpp

}  // namespace gehtp

using namespace gehtp;

namespace {

constexpr uint32_t kMaxTemps = WT_EXEC_MAX_TEMPS;
constexpr uint32_t kNone = 0xFFFFFFFFu;

struct State {
    uint8_t* dev = nullptr;
    uint32_t bytes = 0;
    uint32_t count = 0;            // host mirror of the auto-position counter
    bool kv_ready = false;
    uint32_t slot_bytes = 0, nslots = 0;
    std::vector<uint32_t> posmap;  // slot -> absolute position (kNone = empty)
    uint32_t valid_prefix = 0;     // positions 0..valid_prefix-1 all present in their slots
};

struct Engine {
    bool ready = false;
    hipStream_t stream = nullptr;

    uint8_t* temps[kMaxTemps] = {};
    uint32_t temp_bytes[kMaxTemps] = {};
    uint32_t last_bytes[kMaxTemps] = {};
    std::vector<uint8_t> mirror[kMaxTemps];

    uint8_t* pool = nullptr;
    uint32_t pool_cap = 0, pool_used = 0;
    bool pool_owned = false;
    std::vector<void*> retired_pools;   // earlier bump pools stay valid until shutdown
    const uint32_t* static_offsets = nullptr;
    bool plan_from_blob = false;          // static_offsets come from a blob's TEMPOFF slot
    std::vector<uint8_t> plan_payload;    // that slot's bytes
    uint32_t static_off_arr[kMaxTemps];
    uint8_t* vtcm_pool = nullptr;
    uint32_t vtcm_pool_size = 0;
    uint32_t vtcm_off_arr[kMaxTemps];

    uint32_t n_states = 0;
    State st[WT_MAX_STATES];
    bool states_loaded = false;
    uint32_t* counters_dev = nullptr;   // per state: auto-position counter, then [WT_MAX_STATES + i] a
                                        // workgroups-finished counter of the prefill QK/RoPE kernel

    // Device copy of the blob's weight region and its identity.
    uint8_t* w_dev = nullptr;
    size_t w_cap = 0;
    uint64_t w_key = 0;
    // External weight image.
    const uint8_t* ext_host = nullptr;
    uint8_t* ext_dev = nullptr;
    size_t ext_cap = 0;
    uint64_t ext_key = 0;
    // Injected input for EXT_IN slots: staged through pinned host memory into in_dev,
    // or a caller-bound device buffer (in_bound); in_src is the one the current run reads.
    uint8_t* in_dev = nullptr;
    uint8_t* in_host = nullptr;
    size_t in_cap = 0;
    bool in_active = false;
    uint8_t* in_bound = nullptr;
    size_t in_bound_bytes = 0;
    uint8_t* in_src = nullptr;
    // Pinned buffer for wt_exec_run_io's output: the copy is queued behind the run so one
    // wait covers both (out_pending = bytes queued by the current run, 0 if none).
    uint8_t* out_host = nullptr;
    size_t out_cap = 0;
    size_t out_pending = 0;

    float* attn_work = nullptr;
    uint32_t attn_work_floats = 0;
    uint8_t* norm_buf = nullptr;   // normalized rows for OP_W4G_FUSED_F16 on the GEMM path
    size_t norm_cap = 0;
    uint8_t* split_buf = nullptr;  // fp32 K-split partials of the W4G GEMM
    size_t split_cap = 0;
    uint8_t* rope_buf = nullptr;   // RoPE table of a q|k|v GEMM performing OP_QK_ROPE_KV_F16
    size_t rope_cap = 0;

    // OP_MATMUL_W4A16 engine surfaces (the reference's HMX engine: shape, act, out,
    // weights, bias), read by OP_DMA's 0xC000 references; engine_m reports w4_m.
    bool w4_ready = false;
    uint32_t w4_m = 0, w4_k = 0, w4_n = 0;
    uint8_t* w4_out = nullptr;
    size_t w4_out_cap = 0;
    uint8_t* w4_act = nullptr;
    const uint8_t* w4_wt = nullptr;
    const uint8_t* w4_bias = nullptr;

    // Graph replay. `epoch` changes whenever a device pointer that kernels receive may
    // have changed (any allocation or free, a temp moving, a new pool or weight image).
    uint64_t epoch = 1;
    bool replay = false;    // host pass of a graph replay: device work is not enqueued
    bool variant = false;   // an op of this run passed host-side step state to a kernel
    int graphs = -1;        // -1: not yet read from the environment; 0 off; 1 on
    int fusion = -1;        // attention-chain fusion: -1 not yet read from the environment
    uint64_t chains_found = 0, fused_runs = 0, fused_alias_runs = 0;
    uint8_t* fuse_scratch = nullptr;       // fused attention output when it overlaps an input
    uint64_t fuse_scratch_cap = 0;
    uint64_t qkv_rope_fused = 0;   // OP_QK_ROPE_KV_F16 ops performed by their GEMM's epilogue
    uint64_t qkv_attn_fused = 0;   // OP_ATTN_DECODE_QKV_F16 ops performed in their GEMV's launch
    uint64_t merge_oproj_fused = 0;   // o-proj GEMVs run in one launch with the merge pass before them
    bool graphs_broken = false;
    uint32_t n_captures = 0, n_replays = 0;

    wt_exec_stats stats{};
    wt_op_ts* ts = nullptr;
    uint32_t ts_cap = 0;
    bool trace = false;
    const char* hook = nullptr;
    std::vector<hipEvent_t> events;

    Engine() {
        std::fill(std::begin(static_off_arr), std::end(static_off_arr), kNone);
        std::fill(std::begin(vtcm_off_arr), std::end(vtcm_off_arr), kNone);
    }
};

Engine g;

// ---- load-time fusion of the reference attention chains: observation log ----
// The first full run of a blob runs its attention chains op by op and logs, per op,
// every temp it reads (with the op that last wrote that temp in this run) and every
// temp it writes (with the device bytes written). A chain qualifies for fusion only if
// the log shows that running it as one kernel at its last op gives what the op chain
// gives (fusion_validate). ref_ptr reports reads, temp_get writes.
struct ObsRead { uint32_t op, id, writer; uintptr_t p; uint64_t n; };
struct ObsWrite { uint32_t op, id; uintptr_t p; uint64_t n; };
struct FuseObs {
    bool on = false;
    uint32_t op = 0;                  // op being run
    std::vector<uint32_t> writer;     // temp id -> op that last wrote it in this run
    std::vector<ObsRead> reads;
    std::vector<ObsWrite> writes;
};
FuseObs g_obs;
// Temps a fused chain left unwritten (its intermediates) since their last write:
// wt_exec_temp returns NULL for them.
std::vector<uint8_t> g_unmat;
uint32_t g_run_out_temp = 0xFFFFFFFFu;   // run_io's output temp (read after the run)
bool g_defer_wait = false;               // wt_exec_run_steps: a replayed run returns unwaited

inline void obs_read(uint32_t arg) {
    if (!g_obs.on || (arg & 0x8000u) || (arg & 0xE000u) == WT_REF_STATE_FLAG) return;
    const uint32_t t = arg & 0x3FFFu;
    if (t >= kMaxTemps) return;
    const uint8_t* p = (arg & 0x4000u) ? (g.vtcm_pool && g.vtcm_off_arr[t] != kNone ? g.vtcm_pool + g.vtcm_off_arr[t]
                                                                                   : nullptr)
                                       : g.temps[t];
    g_obs.reads.push_back({g_obs.op, t, g_obs.writer[t], reinterpret_cast<uintptr_t>(p), g.last_bytes[t]});
}
inline void obs_write(uint32_t id, const uint8_t* p, uint64_t n) {
    if (!g_obs.on || id >= kMaxTemps || !p) return;
    g_obs.writer[id] = g_obs.op;
    g_obs.writes.push_back({g_obs.op, id, reinterpret_cast<uintptr_t>(p), n});
}

#define ERR(...) (std::snprintf(err, errn, __VA_ARGS__), -1)

// Every device allocation and free of the engine goes through these two, so that a
// captured graph is never replayed against moved buffers.
hipError_t dev_malloc(void** p, size_t bytes) {
    ++g.epoch;
    return hipMalloc(p, bytes);
}
void dev_free(void* p) {
    ++g.epoch;
    if (p) hipFree(p);
}

int ensure_ready(char* err, size_t errn) {
    if (g.ready) return 0;
    if (const char* t = std::getenv("GEHTP_TRACE"); t && t[0] && t[0] != '0') g.trace = true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return ERR("no HIP device visible");
    if (hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking) != hipSuccess)
        return ERR("hipStreamCreate failed");
    if (dev_malloc(reinterpret_cast<void**>(&g.counters_dev), 2 * WT_MAX_STATES * sizeof(uint32_t)) != hipSuccess)
        return ERR("counter alloc failed");
    if (launch_fill_zero(g.counters_dev, 2 * WT_MAX_STATES * sizeof(uint32_t), g.stream) != hipSuccess)
        return ERR("counter clear failed");
    g.ready = true;
    return 0;
}

// 64-bit FNV-1a over a byte range.
uint64_t fnv(uint64_t h, const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    for (size_t i = 0; i < n; ++i) { h ^= b[i]; h *= 0x100000001b3ull; }
    return h;
}

// Change-detection hash of a byte range: FNV-style multiply-xor on 8-byte words in
// four independent lanes (a run checks its images every call, so this stays cheap:
// about 7 GB/s against FNV-1a's 0.7 GB/s).
uint64_t hash_bytes(uint64_t h, const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    uint64_t l[4] = {h, h ^ 0x9e3779b97f4a7c15ull, h ^ 0xc2b2ae3d27d4eb4full, h ^ 0x165667b19e3779f9ull};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int k = 0; k < 4; ++k) {
            uint64_t w;
            std::memcpy(&w, b + i + 8 * k, 8);
            l[k] = (l[k] ^ w) * 0x100000001b3ull;
            l[k] ^= l[k] >> 29;
        }
    uint64_t r = l[0];
    for (int k = 1; k < 4; ++k) r = (r ^ l[k]) * 0x9e3779b97f4a7c15ull;
    return fnv(r, b + i, n - i);
}

// Identity of a host byte image: pointer, size and content (all of it up to 64 KiB,
// else 64 evenly spaced 1 KiB windows), so a new blob that reuses an old buffer
// address is still recognised as new.
uint64_t image_key(const uint8_t* p, size_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    h = fnv(h, &p, sizeof p);
    h = fnv(h, &n, sizeof n);
    if (n <= (64u << 10)) return hash_bytes(h, p, n);
    for (int i = 0; i < 64; ++i) {
        const size_t off = (n - 1024) / 63 * (size_t)i;
        h = hash_bytes(h, p + off, 1024);
    }
    return h;
}

int upload(uint8_t** dev, size_t* cap, const uint8_t* host, size_t bytes, char* err, size_t errn) {
    if (bytes > *cap) {
        if (*dev) dev_free(*dev);
        *dev = nullptr;
        *cap = 0;
        if (dev_malloc(reinterpret_cast<void**>(dev), bytes) != hipSuccess)
            return ERR("device alloc of %zu bytes failed", bytes);
        *cap = bytes;
    }
    // On the engine's stream (created non-blocking: null-stream copies and memsets are
    // not ordered with its kernels), then drained so the host image may change after.
    if (bytes && (hipMemcpyAsync(*dev, host, bytes, hipMemcpyHostToDevice, g.stream) != hipSuccess ||
                  hipStreamSynchronize(g.stream) != hipSuccess))
        return ERR("weight upload failed");
    return 0;
}

int ensure_weights(const wt_blob* b, char* err, size_t errn) {
    uint64_t key = image_key(b->weight_base, b->weight_bytes);
    key = hash_bytes(key, b->slots, sizeof(wt_slot) * b->n_slots);
    if (key != g.w_key || !g.w_dev) {
        if (upload(&g.w_dev, &g.w_cap, b->weight_base, std::max<size_t>(b->weight_bytes, 16), err, errn))
            return -1;
        g.w_key = key;
    }
    size_t ext_need = 0;
    for (uint32_t i = 0; i < b->n_slots; ++i)
        if (b->slots[i].addr == WT_SLOT_EXT_WGT)
            ext_need = std::max<size_t>(ext_need, b->slots[i].offset + b->slots[i].len);
    if (ext_need && g.ext_host) {
        const uint64_t ek = image_key(g.ext_host, ext_need);
        if (ek != g.ext_key || !g.ext_dev) {
            if (upload(&g.ext_dev, &g.ext_cap, g.ext_host, ext_need, err, errn)) return -1;
            g.ext_key = ek;
        }
    }
    return 0;
}

// ---- reference decoding (oplist_exec.c:175-213), returning DEVICE pointers ----
uint8_t* slot_ptr(const wt_blob* b, uint32_t s) {
    if (s >= b->n_slots) return nullptr;
    const wt_slot& sl = b->slots[s];
    if (sl.addr == WT_SLOT_EXT_IN && g.in_active) return g.in_src;
    if (sl.addr == WT_SLOT_EXT_WGT) return (g.ext_dev && g.ext_host) ? g.ext_dev + sl.offset : nullptr;
    return g.w_dev + sl.offset;
}

uint8_t* ref_ptr(const wt_blob* b, uint32_t arg) {
    obs_read(arg);
    if (arg & 0x8000u) return slot_ptr(b, arg & 0x7FFFu);
    if ((arg & 0xE000u) == WT_REF_STATE_FLAG) {
        const uint32_t s = arg & 0x1FFFu;
        return s < g.n_states ? g.st[s].dev : nullptr;
    }
    if (arg & 0x4000u) {
        const uint32_t t = arg & 0x3FFFu;
        if (t < kMaxTemps && g.vtcm_pool && g.vtcm_off_arr[t] != kNone) return g.vtcm_pool + g.vtcm_off_arr[t];
        return nullptr;
    }
    return arg < kMaxTemps ? g.temps[arg] : nullptr;
}

// f16 element count of a reference (oplist_exec.c:221-225).
uint32_t ref_elem_count(const wt_blob* b, uint32_t arg) {
    if (arg & 0x8000u) {
        const uint32_t s = arg & 0x7FFFu;
        return s < b->n_slots ? b->slots[s].count : 0;
    }
    if (arg & 0x4000u) return 0;
    return arg < kMaxTemps ? g.last_bytes[arg] / 2u : 0;
}

// Byte capacity behind a reference, when known (0 = unknown).
size_t ref_bytes(const wt_blob* b, uint32_t arg) {
    if (arg & 0x8000u) {
        const uint32_t s = arg & 0x7FFFu;
        return s < b->n_slots ? b->slots[s].len : 0;
    }
    if ((arg & 0xE000u) == WT_REF_STATE_FLAG) {
        const uint32_t s = arg & 0x1FFFu;
        return s < g.n_states ? g.st[s].bytes : 0;
    }
    if (arg & 0x4000u) return 0;
    return arg < kMaxTemps ? g.temp_bytes[arg] : 0;
}

// Temp allocation (oplist_exec.c:257-335): VTCM-plan temps, static-plan temps, then
// a 128-byte aligned bump that only grows; earlier pools are kept alive.
uint8_t* temp_get_at(uint32_t id, uint32_t bytes) {
    if (id >= kMaxTemps) return nullptr;
    if (!g_unmat.empty()) g_unmat[id] = 0;
    if (g.vtcm_off_arr[id] != kNone) {
        const uint32_t off = g.vtcm_off_arr[id];
        if (!g.vtcm_pool || (uint64_t)off + bytes > g.vtcm_pool_size) return nullptr;
        g.temps[id] = g.vtcm_pool + off;
        g.temp_bytes[id] = bytes;
        g.last_bytes[id] = bytes;
        return g.temps[id];
    }
    if (g.static_offsets && g.pool) {
        const uint32_t off = g.static_offsets[id];
        if (off != kNone) {
            if ((uint64_t)off + bytes > g.pool_used) return nullptr;
            g.temps[id] = g.pool + off;
            g.temp_bytes[id] = bytes;
            g.last_bytes[id] = bytes;
            return g.temps[id];
        }
    }
    if (!g.temps[id] || g.temp_bytes[id] < bytes) {
        const uint32_t aligned = (bytes + 127u) & ~127u;
        if ((uint64_t)g.pool_used + aligned > g.pool_cap) {
            if (g.static_offsets) return nullptr;   // static plan: reserve exhausted
            uint64_t ncap = g.pool_cap ? g.pool_cap : (64u << 20);
            while (ncap < (uint64_t)g.pool_used + aligned) ncap *= 2;
            if (ncap > 0xFFFFFFFFull) return nullptr;
            void* np = nullptr;
            if (dev_malloc(&np, ncap) != hipSuccess) return nullptr;
            if (g.pool && g.pool_owned) g.retired_pools.push_back(g.pool);
            g.pool = static_cast<uint8_t*>(np);
            g.pool_cap = (uint32_t)ncap;
            g.pool_used = 0;
            g.pool_owned = true;
        }
        g.temps[id] = g.pool + g.pool_used;
        g.pool_used += aligned;
        g.temp_bytes[id] = bytes;
        ++g.epoch;
    }
    g.last_bytes[id] = bytes;
    return g.temps[id];
}

uint8_t* temp_get(uint32_t id, uint32_t bytes) {
    uint8_t* p = temp_get_at(id, bytes);
    obs_write(id, p, bytes);
    return p;
}

// Drops a static plan loaded from a blob's TEMPOFF slot: the temps living in its pools
// are forgotten (a later write allocates them again), the pools are freed once the
// stream is idle, and captured graphs (which hold their addresses) are dropped.
void drop_graphs();
void drop_blob_plan() {
    if (g.stream) hipStreamSynchronize(g.stream);
    drop_graphs();
    auto inside = [](const uint8_t* p, const uint8_t* base, uint64_t n) { return base && p >= base && p < base + n; };
    for (uint32_t t = 0; t < kMaxTemps; ++t)
        if (g.temps[t] && (inside(g.temps[t], g.pool, g.pool_cap) || inside(g.temps[t], g.vtcm_pool, g.vtcm_pool_size))) {
            g.temps[t] = nullptr;
            g.temp_bytes[t] = 0;
        }
    if (g.pool && g.pool_owned) dev_free(g.pool);
    if (g.vtcm_pool) dev_free(g.vtcm_pool);
    std::fill(std::begin(g.static_off_arr), std::end(g.static_off_arr), kNone);
    std::fill(std::begin(g.vtcm_off_arr), std::end(g.vtcm_off_arr), kNone);
    g.pool = nullptr;
    g.pool_cap = g.pool_used = 0;
    g.pool_owned = false;
    g.vtcm_pool = nullptr;
    g.vtcm_pool_size = 0;
    g.static_offsets = nullptr;
    g.plan_payload.clear();
    g.plan_from_blob = false;
    ++g.epoch;
}

// TEMPOFF slot (oplist_exec.c:2012-2066): [cap][reserve: lo16 bump KB | hi16 VTCM KB][n][n x {tid,off,size}].
// The reference parses the first TEMPOFF slot it meets and keeps that plan until
// shutdown, so a second blob with another plan (a model's decode blob after its prefill
// blob) would run on the first blob's offsets, whose sizes and sharing belong to other
// temps. Here each blob runs with its own plan: a different TEMPOFF payload replaces the
// loaded one, a blob without one drops it (bump allocation); a plan installed by the
// caller through wt_exec_pool_init is kept, as in the reference.
int load_tempoff(const wt_blob* b, char* err, size_t errn) {
    const uint8_t* tp = nullptr;
    uint32_t tlen = 0;
    for (uint32_t s = 0; s < b->n_slots; ++s)
        if (b->slots[s].addr == WT_SLOT_TEMPOFF) {
            tp = b->weight_base + b->slots[s].offset;
            tlen = b->slots[s].len;
            break;
        }
    if (g.static_offsets && !g.plan_from_blob) return 0;   // the caller's plan
    if (!tp) {
        if (g.plan_from_blob) drop_blob_plan();
        return 0;
    }
    if (g.plan_from_blob && g.plan_payload.size() == tlen && std::memcmp(g.plan_payload.data(), tp, tlen) == 0)
        return 0;   // this blob's plan is loaded
    if (g.plan_from_blob) drop_blob_plan();
    std::fill(std::begin(g.static_off_arr), std::end(g.static_off_arr), kNone);
    std::fill(std::begin(g.vtcm_off_arr), std::end(g.vtcm_off_arr), kNone);
    {
        const uint8_t* p = tp;
        const uint32_t len = tlen;
        if (len < 12u) return ERR("tempoff slot short");
        uint32_t cap, reserve, n;
        std::memcpy(&cap, p, 4);
        std::memcpy(&reserve, p + 4, 4);
        std::memcpy(&n, p + 8, 4);
        if ((uint64_t)len < 12u + (uint64_t)n * 12u) return ERR("tempoff table short");
        if (cap == 0 || cap > 0x80000000u) return ERR("tempoff cap bad");
        const uint32_t vtcm_cap = (reserve >> 16) * 1024u;
        reserve = (reserve & 0xFFFFu) * 1024u;
        uint32_t tmp_static[kMaxTemps], tmp_vtcm[kMaxTemps];
        std::fill(std::begin(tmp_static), std::end(tmp_static), kNone);
        std::fill(std::begin(tmp_vtcm), std::end(tmp_vtcm), kNone);
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t tid, off, sz;
            std::memcpy(&tid, p + 12 + 12 * i, 4);
            std::memcpy(&off, p + 16 + 12 * i, 4);
            std::memcpy(&sz, p + 20 + 12 * i, 4);
            const uint32_t t = tid & 0x3FFFu;
            if (t >= kMaxTemps) return ERR("tempoff tid bad %u", t);
            if (tid & WT_REF_VTCM_FLAG) {
                if (vtcm_cap == 0 || (uint64_t)off + sz > vtcm_cap)
                    return ERR("tempoff vtcm entry bad (tid %u off %u sz %u vtcm_cap %u)", t, off, sz, vtcm_cap);
                tmp_vtcm[t] = off;
            } else {
                if ((uint64_t)off + sz > cap)
                    return ERR("tempoff entry bad (tid %u off %u sz %u cap %u)", t, off, sz, cap);
                tmp_static[t] = off;
            }
        }
        void* pool = nullptr;
        if (dev_malloc(&pool, (size_t)cap + reserve) != hipSuccess) return ERR("tempoff pool alloc");
        if (g.pool && g.pool_owned) g.retired_pools.push_back(g.pool);
        std::memcpy(g.static_off_arr, tmp_static, sizeof tmp_static);
        std::memcpy(g.vtcm_off_arr, tmp_vtcm, sizeof tmp_vtcm);
        g.pool = static_cast<uint8_t*>(pool);
        g.pool_cap = cap + reserve;
        g.pool_used = cap;
        g.pool_owned = true;
        g.static_offsets = g.static_off_arr;
        if (vtcm_cap) {
            void* vp = nullptr;
            if (dev_malloc(&vp, vtcm_cap) != hipSuccess) return ERR("vtcm pool alloc");
            g.vtcm_pool = static_cast<uint8_t*>(vp);
            g.vtcm_pool_size = vtcm_cap;
        }
        g.plan_payload.assign(tp, tp + tlen);
        g.plan_from_blob = true;
    }
    return 0;
}

// STATE slot (oplist_exec.c:2071-2102): [n][n x bytes], zeroed, process lifetime.
// The reference loads the table once per process. Here a blob whose STATE table
// differs from the loaded one (another model in the same process) replaces it with
// fresh zeroed states; a blob with the same table, or with none, keeps the states,
// so a prefill blob and a decode blob of one model share their KV rings.
int load_states(const wt_blob* b, char* err, size_t errn) {
    for (uint32_t s = 0; s < b->n_slots; ++s) {
        if (b->slots[s].addr != WT_SLOT_STATE) continue;
        const uint8_t* p = b->weight_base + b->slots[s].offset;
        const uint32_t len = b->slots[s].len;
        if (len < 4u) return ERR("state slot short");
        uint32_t n;
        std::memcpy(&n, p, 4);
        if (n == 0 || n > WT_MAX_STATES || len < 4u + n * 4u)
            return ERR("state slot table bad (n=%u len=%u)", n, len);
        bool same = g.states_loaded && g.n_states == n;
        for (uint32_t i = 0; same && i < n; ++i) {
            uint32_t bytes;
            std::memcpy(&bytes, p + 4 + 4 * i, 4);
            same = g.st[i].bytes == bytes;
        }
        if (same) return 0;
        for (uint32_t i = 0; i < g.n_states; ++i) {
            if (g.st[i].dev) dev_free(g.st[i].dev);
            g.st[i] = State{};
        }
        g.n_states = 0;
        // Clears go on the engine's stream: a null-stream memset is not ordered with the
        // kernels of a non-blocking stream and could land after the first KV append.
        if (g.counters_dev && launch_fill_zero(g.counters_dev, 2 * WT_MAX_STATES * sizeof(uint32_t), g.stream) != hipSuccess)
            return ERR("counter clear failed");
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t bytes;
            std::memcpy(&bytes, p + 4 + 4 * i, 4);
            if (bytes == 0 || bytes > (1u << 30)) return ERR("state %u bytes bad %u", i, bytes);
            void* d = nullptr;
            if (dev_malloc(&d, bytes) != hipSuccess) return ERR("state %u alloc %u", i, bytes);
            if (launch_fill_zero(d, bytes, g.stream) != hipSuccess) return ERR("state %u clear", i);
            g.st[i] = State{};
            g.st[i].dev = static_cast<uint8_t*>(d);
            g.st[i].bytes = bytes;
        }
        g.n_states = n;
        break;
    }
    g.states_loaded = true;
    return 0;
}

// KV geometry from the op's shape (oplist_exec.c:2119-2151).
State* state_kv(uint32_t ref, uint32_t kv_elems, char* err, size_t errn) {
    if ((ref & 0xE000u) != WT_REF_STATE_FLAG) {
        std::snprintf(err, errn, "kv state_ref not 0x6000|idx (0x%X)", ref);
        return nullptr;
    }
    const uint32_t i = ref & 0x1FFFu;
    if (i >= g.n_states) { std::snprintf(err, errn, "kv state idx %u oob", i); return nullptr; }
    State& s = g.st[i];
    const uint32_t slot_bytes = kv_elems * 4u;
    if (!s.kv_ready) {
        if (slot_bytes < 256u || (slot_bytes & 127u) || s.bytes % slot_bytes) {
            std::snprintf(err, errn, "kv state %u geometry bad (slot=%u total=%u)", i, slot_bytes, s.bytes);
            return nullptr;
        }
        s.slot_bytes = slot_bytes;
        s.nslots = s.bytes / slot_bytes;
        s.posmap.assign(s.nslots, kNone);
        s.kv_ready = true;
    } else if (s.slot_bytes != slot_bytes) {
        std::snprintf(err, errn, "kv state %u slot_bytes mismatch (%u vs %u)", i, s.slot_bytes, slot_bytes);
        return nullptr;
    }
    return &s;
}

// Host-side lookup check for positions [0, n_kv) (kvcache.c:64-68): a miss is a hard error.
// Record that position p now occupies its ring slot, keeping valid_prefix exact:
// it grows over consecutive present positions and shrinks when a wrapped append
// overwrites one of them.
void kv_mark(State& s, uint32_t p) {
    const uint32_t slot = p % s.nslots;
    s.posmap[slot] = p;
    if (slot < s.valid_prefix && p != slot) s.valid_prefix = slot;
    while (s.valid_prefix < s.nslots && s.posmap[s.valid_prefix] == s.valid_prefix) ++s.valid_prefix;
}

int attn_workspace(uint32_t need, char* err, size_t errn);
int gemm_split_ws(W4gEpilogue& epi, uint32_t M, uint32_t N, uint32_t K, char* err, size_t errn);

int kv_check(const State& s, uint32_t n_kv, char* err, size_t errn) {
    if (n_kv > s.valid_prefix) return ERR("kv gather miss pos %u (state bug)", s.valid_prefix);
    return 0;
}

float f32_from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// ---- op implementations ----
struct Ctx {
    const wt_blob* b;
    const wt_op* op;
    uint32_t* engine_m;
    char* err;
    size_t errn;
};

// Enqueue device work; skipped in the host pass of a graph replay, whose kernels
// the graph already carries.
#define CHECK_LAUNCH(expr)                                                             \
    do {                                                                               \
        if (!g.replay) {                                                               \
            hipError_t e_ = (expr);                                                    \
            if (e_ != hipSuccess) return ERR("launch failed: %s", hipGetErrorString(e_)); \
        }                                                                              \
    } while (0)

hipError_t copy_d2d(void* dst, const void* src, size_t bytes) {
    if (g.replay || !bytes) return hipSuccess;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g.stream);
}

#define A(i) (cx.op->args[i])

int op_nop(Ctx& cx) { (void)cx; g.stats.nop++; return 0; }

int op_pin(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    if (A(0) >= cx.b->n_slots) return ERR("pin slot oob");
    // Weights are resident in HBM from the first run: pinning is bookkeeping only.
    g.stats.pin++;
    g.stats.pin_skipped++;
    return 0;
}

int op_matmul_f16(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const bool split = cx.op->opcode == OP_MATMUL_F16_SPLIT;
    const uint32_t M = A(3), K = A(4);
    const uint32_t N_full = A(5), n0 = split ? A(6) : 0, N = split ? A(7) : A(5);
    const uint32_t flags = split ? A(8) : A(6);
    uint32_t Bn = flags >> 16;
    if (!Bn) Bn = 1;
    const bool t0 = flags & 1u, t1 = flags & 2u, batched = flags & 4u;
    if (!batched) Bn = 1;
    if ((uint64_t)n0 + N > N_full) return ERR("matmul_f16 chunk [%u,+%u) beyond N_full %u", n0, N, N_full);
    const __half* a = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* w = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    const uint64_t ybytes = (uint64_t)M * N_full * Bn * 2u;
    if (ybytes > 0xFFFFFFFFull) return ERR("matmul_f16 output too large");
    // SPLIT chunks share the output temp: keep earlier chunks' columns.
    __half* y = reinterpret_cast<__half*>(temp_get(A(2), (uint32_t)ybytes));
    if (!a || !w || !y) return ERR("matmul_f16 ref fail");
    const size_t abytes = ref_bytes(cx.b, A(0)), wbytes = ref_bytes(cx.b, A(1));
    if (abytes && abytes < (uint64_t)M * K * Bn * 2u) return ERR("matmul_f16 a smaller than M*K");
    if (wbytes && wbytes < (uint64_t)K * N_full * Bn * 2u) return ERR("matmul_f16 w smaller than K*N");
    CHECK_LAUNCH(launch_matmul_f16(a, w, y, M, K, N_full, n0, N, t0, t1, Bn, g.stream));
    return 0;
}

int op_matmul_w4g(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t M = A(4), K = A(5), N = A(6), group = A(7), flags = A(8);
    if (group != 64) return ERR("w4g group %u unsupported (64 only)", group);
    if (!(flags & 2u) || (flags & 0xFFFDu)) return ERR("w4g flags 0x%X unsupported (need t1)", flags);
    if (K == 0 || K % 64) return ERR("w4g K=%u not a multiple of 64", K);
    const uint32_t ldy = (flags >> 16) ? (flags >> 16) : N;
    if (ldy < N) return ERR("w4g output stride %u < N %u", ldy, N);
    const __half* a = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const uint8_t* wq = ref_ptr(cx.b, A(1));
    const __half* ws = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(2)));
    const uint64_t ybytes = ((uint64_t)(M ? M - 1 : 0) * ldy + N) * 2u;
    __half* y = reinterpret_cast<__half*>(temp_get(A(3), (uint32_t)ybytes));
    if (!a || !wq || !ws || !y) return ERR("w4g ref fail");
    const size_t ab = ref_bytes(cx.b, A(0)), qb = ref_bytes(cx.b, A(1)), sb = ref_bytes(cx.b, A(2));
    if (ab && ab < (uint64_t)M * K * 2u) return ERR("w4g activation smaller than M*K");
    if (qb && qb < (uint64_t)N * K / 2u) return ERR("w4g weight slot %zu < N*K/2", qb);
    if (sb && sb < (uint64_t)N * (K / 64) * 2u) return ERR("w4g scale slot %zu < N*K/64*2", sb);
    if (((uintptr_t)a | (uintptr_t)wq) % 16) return ERR("w4g operands not 16-byte aligned");
    g.stats.matmul++;
    if (M <= kW4gGemvMaxM) {
        CHECK_LAUNCH(launch_w4g_gemv(a, K, wq, ws, y, ldy, M, N, K, g.stream));
    } else {
        W4gEpilogue epi;
        if (gemm_split_ws(epi, M, N, K, err, errn)) return -1;
        CHECK_LAUNCH(launch_w4g_gemm(a, K, wq, ws, y, ldy, M, N, K, g.stream, epi));
    }
    return 0;
}

int op_rmsnorm2(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t w_s = A(1) & 0x7FFFu, b_s = A(2) & 0x7FFFu, n = A(4);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* gw = reinterpret_cast<const __half*>(slot_ptr(cx.b, w_s));
    const __half* bv = reinterpret_cast<const __half*>(slot_ptr(cx.b, b_s));
    __half* y = reinterpret_cast<__half*>(temp_get(A(3), n * 2u));
    if (!x || !gw || !y) return ERR("rmsnorm2 ref fail");
    const uint32_t rw = cx.b->slots[w_s].len / 2u;
    if (rw == 0 || n % rw) return ERR("rmsnorm2 shape n%u rw%u", n, rw);
    if (bv && cx.b->slots[b_s].len < rw * 2u) return ERR("rmsnorm2 bias slot shorter than row");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)n * 2u) return ERR("rmsnorm2 input smaller than n");
    g.stats.rmsnorm++;
    CHECK_LAUNCH(launch_rmsnorm2(x, gw, bv, y, n / rw, rw, g.stream));
    return 0;
}

int op_softmax(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t rows = A(2), n = A(3);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), rows * n * 2u));
    if (!x || !y) return ERR("softmax ref fail");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)rows * n * 2u) return ERR("softmax input smaller than rows*n");
    CHECK_LAUNCH(launch_softmax(x, y, rows, n, g.stream));
    return 0;
}

int op_binary(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    if (A(4) == 8) {   // SELECT [c, t, f, out, 8]
        const __half* c = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
        const __half* t = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
        const __half* f = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(2)));
        const uint32_t cn = ref_elem_count(cx.b, A(0)), tn = ref_elem_count(cx.b, A(1));
        const uint32_t fn = ref_elem_count(cx.b, A(2));
        const uint32_t n = std::max(std::max(cn, tn), fn);
        __half* y = reinterpret_cast<__half*>(temp_get(A(3), n * 2u));
        if (!c || !t || !f || !y || n == 0) return ERR("select ref fail");
        CHECK_LAUNCH(launch_select(c, cn, t, tn, f, fn, y, n, g.stream));
        return 0;
    }
    const uint32_t n = A(3), sub = A(4);
    const __half* a = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* bb = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(2), n * 2u));
    if (!a || !bb || !y) return ERR("binary ref fail");
    const size_t ab = ref_bytes(cx.b, A(0)), bbytes = ref_bytes(cx.b, A(1));
    if ((ab && ab < (uint64_t)n * 2u) || (bbytes && bbytes < (uint64_t)n * 2u))
        return ERR("binary operand smaller than n");
    CHECK_LAUNCH(launch_binary(a, bb, y, n, sub, g.stream));
    return 0;
}

int op_add(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(3);
    const __half* a = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* bb = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(2), n * 2u));
    if (!a || !bb) return ERR("add ref empty");
    if (!y) return ERR("add temp alloc");
    const size_t ab = ref_bytes(cx.b, A(0)), bbytes = ref_bytes(cx.b, A(1));
    if ((ab && ab < (uint64_t)n * 2u) || (bbytes && bbytes < (uint64_t)n * 2u))
        return ERR("add operand smaller than n");
    g.stats.add++;
    CHECK_LAUNCH(launch_binary(a, bb, y, n, 0, g.stream));
    return 0;
}

int op_unary(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(2), sub = A(3);
    if (sub > 16) return ERR("unary unknown subtype %u", sub);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), n * 2u));
    if (!x || !y) return ERR("unary ref fail");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)n * 2u) return ERR("unary input smaller than n");
    CHECK_LAUNCH(launch_unary(x, y, n, sub, g.stream));
    return 0;
}

int op_silu(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t x_t = A(0), n = A(2);
    obs_read(x_t);
    if (x_t >= kMaxTemps || !g.temps[x_t]) return ERR("silu src temp %u empty", x_t);
    if (g.temp_bytes[x_t] != n * 2u)
        return ERR("silu n_elem mismatch (%u vs face %u)", n, g.temp_bytes[x_t] / 2u);
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), n * 2u));
    if (!y) return ERR("silu temp %u alloc", A(1));
    g.stats.silu++;
    CHECK_LAUNCH(launch_unary(reinterpret_cast<const __half*>(g.temps[x_t]), y, n, 12, g.stream));
    return 0;
}

int op_argmax(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(2);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    int32_t* y = reinterpret_cast<int32_t*>(temp_get(A(1), 4u));
    if (!x || !y) return ERR("argmax ref fail");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)n * 2u) return ERR("argmax input smaller than n");
    CHECK_LAUNCH(launch_argmax(x, n, y, g.stream));
    return 0;
}

int op_broadcast(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(2), b_elems = A(3);
    const uint32_t in_d[4] = {A(4), A(5), A(6), A(7)}, out_d[4] = {A(8), A(9), A(10), A(11)};
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), n * 2u));
    if (!x || !y || b_elems == 0) return ERR("broadcast ref fail");
    CHECK_LAUNCH(launch_broadcast(x, y, n, in_d, out_d, g.stream));
    return 0;
}

int op_transpose_gen(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t rk = A(2);
    const uint32_t dims[4] = {A(3), A(4), A(5), A(6)};
    if (rk < 2 || rk > 4) return ERR("transpose_gen rank %u", rk);
    uint64_t n = 1;
    for (uint32_t i = 0; i < rk; ++i) n *= dims[i];
    for (uint32_t i = 0; i < rk; ++i)
        if (((A(7) >> (8 * i)) & 0xFFu) >= rk) return ERR("transpose_gen perm bad");
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), (uint32_t)n * 2u));
    if (!x || !y) return ERR("transpose_gen ref fail");
    CHECK_LAUNCH(launch_transpose_gen(x, y, rk, dims, A(7), g.stream));
    return 0;
}

int op_slice(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n_out = A(2), rk = A(3);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), n_out * 2u));
    if (!x || !y) return ERR("slice ref fail");
    if (rk < 1 || rk > 3) return ERR("slice rank %u", rk);
    uint32_t bb[3] = {A(4), A(5), A(6)}, ee[3] = {A(7), A(8), A(9)}, ss[3] = {A(10), A(11), A(12)};
    uint32_t dd[3] = {A(13), A(14), A(15)}, od[3] = {1, 1, 1};
    uint64_t prod = 1;
    for (uint32_t ax = 0; ax < rk; ++ax) {
        if (ss[ax] == 0) ss[ax] = 1;
        const uint32_t span = ee[ax] > bb[ax] ? ee[ax] - bb[ax] : 0;
        od[ax] = (span + ss[ax] - 1) / ss[ax];
        prod *= od[ax];
        if (od[ax] && (uint64_t)bb[ax] + (uint64_t)(od[ax] - 1) * ss[ax] >= dd[ax])
            return ERR("slice axis %u reads beyond dim %u", ax, dd[ax]);
    }
    if (n_out > prod) return ERR("slice n_out %u exceeds slice size", n_out);
    CHECK_LAUNCH(launch_slice(x, y, n_out, rk, bb, ss, dd, od, g.stream));
    return 0;
}

int op_kv_append(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const __half* k = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* v = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    const uint32_t kn = ref_elem_count(cx.b, A(0)), vn = ref_elem_count(cx.b, A(1));
    if (!k || !v || !kn || kn != vn) return ERR("kv append ref fail");
    State* s = state_kv(A(2), kn, err, errn);
    if (!s) return -1;
    const uint32_t si = A(2) & 0x1FFFu;
    uint32_t pos = A(3), dev_pos = A(3);
    if (pos == WT_KV_POS_AUTO) {
        if (s->count >= s->nslots)
            return ERR("kv append state %u count=%u >= nslots=%u (context too long)", si, s->count, s->nslots);
        pos = s->count++;
        dev_pos = 0xFFFFFFFFu;
    }
    kv_mark(*s, pos);
    CHECK_LAUNCH(launch_kv_append(s->dev, s->slot_bytes, s->nslots, k, v, kn, dev_pos,
                                  g.counters_dev + si, g.stream));
    return 0;
}

int op_kv_append_n(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n_tok = A(4), kv_elems = A(5);
    const __half* k = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* v = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    if (!k || !v || !kv_elems || !n_tok) return ERR("kv append_n ref fail");
    const size_t kb = ref_bytes(cx.b, A(0)), vb = ref_bytes(cx.b, A(1));
    if ((kb && kb < (uint64_t)n_tok * kv_elems * 2u) || (vb && vb < (uint64_t)n_tok * kv_elems * 2u))
        return ERR("kv append_n k/v smaller than n_tok*kv_elems");
    State* s = state_kv(A(2), kv_elems, err, errn);
    if (!s) return -1;
    const uint32_t si = A(2) & 0x1FFFu;
    uint32_t pos = A(3), dev_pos = A(3);
    if (pos == WT_KV_POS_AUTO) {
        if ((uint64_t)s->count + n_tok > s->nslots)
            return ERR("kv append_n state %u count=%u + %u > nslots=%u", si, s->count, n_tok, s->nslots);
        pos = s->count;
        s->count += n_tok;
        dev_pos = 0xFFFFFFFFu;
    }
    for (uint32_t t = 0; t < n_tok; ++t) kv_mark(*s, pos + t);
    CHECK_LAUNCH(launch_kv_append_n(s->dev, s->slot_bytes, s->nslots, k, v, kv_elems, n_tok, dev_pos,
                                    g.counters_dev + si, g.stream));
    return 0;
}

int op_kv_gather(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    uint32_t n_kv = A(3);
    const uint32_t H = A(4), KVH = A(5), hd = A(6);
    if (!H || !KVH || !hd || H % KVH) return ERR("kv gather gqa bad (h=%u kvh=%u hd=%u)", H, KVH, hd);
    State* s = state_kv(A(0), KVH * hd, err, errn);
    if (!s) return -1;
    uint32_t pstride = n_kv;
    if (n_kv == WT_KV_POS_AUTO) {
        if (s->count == 0 || s->count > s->nslots)
            return ERR("kv gather state %u count=%u bad (append first?)", A(0) & 0x1FFFu, s->count);
        n_kv = s->count;
        pstride = s->nslots;
        g.variant = true;   // the position count is a kernel argument
    }
    if (kv_check(*s, n_kv, err, errn)) return -1;
    const uint64_t bytes = (uint64_t)H * hd * pstride * 2u;
    if (bytes > 0xFFFFFFFFull) return ERR("kv gather output too large");
    __half* kT = A(1) ? reinterpret_cast<__half*>(temp_get(A(1), (uint32_t)bytes)) : nullptr;
    __half* vo = A(2) ? reinterpret_cast<__half*>(temp_get(A(2), (uint32_t)bytes)) : nullptr;
    if ((!kT && A(1)) || (!vo && A(2))) return ERR("kv gather out alloc");
    CHECK_LAUNCH(launch_kv_gather(s->dev, s->slot_bytes, s->nslots, kT, vo, n_kv, pstride, H, KVH, hd,
                                  g.stream));
    return 0;
}

int op_attn(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t S = A(4), H = A(5), KVH = A(6), hd = A(7), flags = A(9);
    const float scale = f32_from_bits(A(8));
    if (hd != 128) return ERR("attn head_dim %u unsupported (128 only)", hd);
    if (!KVH || H % KVH) return ERR("attn heads %u not a multiple of kv heads %u", H, KVH);
    if (!(scale > 0.0f && scale < INFINITY)) return ERR("attn scale %g must be positive and finite", scale);
    const __half* q = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const __half* k = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(1)));
    const __half* v = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(2)));
    __half* o = reinterpret_cast<__half*>(temp_get(A(3), S * H * hd * 2u));
    if (!q || !k || !v || !o) return ERR("attn ref fail");
    const size_t qb = ref_bytes(cx.b, A(0)), kb = ref_bytes(cx.b, A(1)), vb = ref_bytes(cx.b, A(2));
    if ((qb && qb < (uint64_t)S * H * hd * 2u) || (kb && kb < (uint64_t)S * KVH * hd * 2u) ||
        (vb && vb < (uint64_t)S * KVH * hd * 2u))
        return ERR("attn operand smaller than its shape");
    CHECK_LAUNCH(launch_attn_prefill(q, H * hd, k, v, KVH * hd, o, H * hd, S, H, KVH, hd, scale,
                                     flags & 1u, g.stream));
    return 0;
}

int op_attn_decode(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    uint32_t n_kv = A(3);
    const uint32_t H = A(4), KVH = A(5), hd = A(6);
    const float scale = f32_from_bits(A(7));
    if (hd != 128) return ERR("attn_decode head_dim %u unsupported (128 only)", hd);
    if (!KVH || H % KVH) return ERR("attn_decode heads %u not a multiple of kv heads %u", H, KVH);
    const uint32_t rep = H / KVH;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return ERR("attn_decode group size %u unsupported", rep);
    State* s = state_kv(A(1), KVH * hd, err, errn);
    if (!s) return -1;
    const bool autopos = n_kv == WT_KV_POS_AUTO;
    if (autopos) n_kv = s->count;
    if (n_kv == 0 || n_kv > s->nslots) return ERR("attn_decode n_kv %u bad (nslots %u)", n_kv, s->nslots);
    if (kv_check(*s, n_kv, err, errn)) return -1;
    const __half* q = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* o = reinterpret_cast<__half*>(temp_get(A(2), H * hd * 2u));
    if (!q || !o) return ERR("attn_decode ref fail");
    const size_t qb = ref_bytes(cx.b, A(0));
    if (qb && qb < (uint64_t)H * hd * 2u) return ERR("attn_decode q smaller than H*hd");
    if (attn_workspace(attn_decode_work_floats(autopos ? s->nslots : n_kv, H, hd), err, errn)) return -1;
    CHECK_LAUNCH(launch_attn_decode(q, s->dev, s->slot_bytes, s->nslots, o, autopos ? 0u : n_kv,
                                    autopos ? g.counters_dev + (A(1) & 0x1FFFu) : nullptr, H, KVH, hd,
                                    scale, g.attn_work, g.attn_work_floats, g.stream, nullptr, 0u, n_kv));
    return 0;
}

// Engine-private device scratch (grown on demand, freed at shutdown).
int scratch(uint8_t** p, size_t* cap, size_t bytes, char* err, size_t errn) {
    if (bytes <= *cap) return 0;
    if (*p) dev_free(*p);
    *p = nullptr;
    *cap = 0;
    if (dev_malloc(reinterpret_cast<void**>(p), bytes) != hipSuccess) return ERR("scratch alloc %zu", bytes);
    *cap = bytes;
    return 0;
}

// Attach the engine's K-split workspace to a W4G GEMM epilogue (grown on demand).
int gemm_split_ws(W4gEpilogue& epi, uint32_t M, uint32_t N, uint32_t K, char* err, size_t errn) {
    const size_t need = w4g_gemm_split_bytes(M, N, K);
    if (!need) return 0;
    if (scratch(&g.split_buf, &g.split_cap, need, err, errn)) return -1;
    epi.split_ws = reinterpret_cast<float*>(g.split_buf);
    epi.split_ws_bytes = g.split_cap;
    return 0;
}

// Normalized rows that a K-split GEMM's finishing pass already wrote into norm_buf for
// the next op (an OP_W4G_FUSED_F16 whose RMSNorm input is that GEMM's output).
struct PreNorm {
    const wt_op* op = nullptr;   // the op they are for
    const void* src = nullptr;
    const void* gamma = nullptr;
    uint32_t M = 0, K = 0;
};
PreNorm g_prenorm;
// An OP_QK_ROPE_KV_F16 that the q|k|v GEMM before it performed in its epilogue.
const wt_op* g_rope_pre = nullptr;
// OP_QK_ROPE_KV_F16's operands, checked, with its outputs allocated.
struct QkRope {
    const __half* qkv = nullptr;
    const __half* qg = nullptr;
    const __half* kg = nullptr;
    float theta = 0.0f;
    uint32_t n_tok = 0, H = 0, KVH = 0, si = 0;
    State* s = nullptr;
    __half* q_out = nullptr;
    __half* k_out = nullptr;
    __half* v_out = nullptr;
};
int qk_rope_prep(const wt_blob* b, const wt_op* op, QkRope& r, char* err, size_t errn);
void qk_rope_commit(const QkRope& r);
// An OP_ATTN_DECODE_QKV_F16 that the q|k|v GEMV before it performed in the same launch.
const wt_op* g_attn_pre = nullptr;
// OP_ATTN_DECODE_QKV_F16's operands, checked, with its output and workspace allocated.
struct AttnQkv {
    const __half* qkv = nullptr;
    const __half* qg = nullptr;
    const __half* kg = nullptr;
    float theta = 0.0f, scale = 0.0f;
    uint32_t H = 0, KVH = 0, si = 0;
    State* s = nullptr;
    __half* o = nullptr;
};
int attn_qkv_prep(const wt_blob* b, const wt_op* op, AttnQkv& r, char* err, size_t errn);
void attn_qkv_commit(const AttnQkv& r);
// The merge pass that such a launch left to the o-proj GEMV op after it (op), which runs
// both in one launch; any other next op, or the end of the run, runs it alone first.
struct MergePending {
    const wt_op* op = nullptr;
    uint32_t* count = nullptr;
    __half* out = nullptr;
    uint32_t H = 0, KVH = 0, nslots = 0;
    float theta = 0.0f;
};
MergePending g_merge_pending;
int flush_merge_pending(char* err, size_t errn);
bool fusion_on();
extern uint32_t g_run_end;

int op_w4g_fused(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t M = A(4), K = A(5), N = A(6), mode = A(9), flags = A(10);
    const bool swiglu = mode == 1;
    if (mode > 1) return ERR("w4g_fused mode %u unknown", mode);
    if (!(flags & 2u) || (flags & 0xFFFDu)) return ERR("w4g_fused flags 0x%X unsupported (need t1)", flags);
    if (K == 0 || K % 64) return ERR("w4g_fused K=%u not a multiple of 64", K);
    if (swiglu && (N & 1)) return ERR("w4g_fused SwiGLU needs an even row count, got %u", N);
    const uint32_t n_out = swiglu ? N / 2 : N;
    const uint32_t ldy = (flags >> 16) ? (flags >> 16) : n_out;
    if (ldy < n_out) return ERR("w4g_fused output stride %u < %u", ldy, n_out);
    const __half* a = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const uint8_t* wq = ref_ptr(cx.b, A(1));
    const __half* ws = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(2)));
    const __half* gamma = A(7) == WT_REF_NONE ? nullptr : reinterpret_cast<const __half*>(ref_ptr(cx.b, A(7)));
    const __half* res = A(8) == WT_REF_NONE ? nullptr : reinterpret_cast<const __half*>(ref_ptr(cx.b, A(8)));
    if (!a || !wq || !ws || (A(7) != WT_REF_NONE && !gamma) || (A(8) != WT_REF_NONE && !res))
        return ERR("w4g_fused ref fail");
    const size_t ab = ref_bytes(cx.b, A(0)), qb = ref_bytes(cx.b, A(1)), sb = ref_bytes(cx.b, A(2));
    if (ab && ab < (uint64_t)M * K * 2u) return ERR("w4g_fused activation smaller than M*K");
    if (qb && qb < (uint64_t)N * K / 2u) return ERR("w4g_fused weight slot %zu < N*K/2", qb);
    if (sb && sb < (uint64_t)N * (K / 64) * 2u) return ERR("w4g_fused scale slot %zu < N*K/64*2", sb);
    if (gamma) {
        const size_t gb = ref_bytes(cx.b, A(7));
        if (gb && gb < (uint64_t)K * 2u) return ERR("w4g_fused gamma shorter than K");
    }
    if (res) {
        const size_t rb = ref_bytes(cx.b, A(8));
        if (rb && rb < (uint64_t)M * n_out * 2u) return ERR("w4g_fused residual smaller than M*N_out");
    }
    if (((uintptr_t)a | (uintptr_t)wq | (uintptr_t)gamma) % 16) return ERR("w4g_fused operands not 16-byte aligned");
    const uint64_t ybytes = ((uint64_t)(M ? M - 1 : 0) * ldy + n_out) * 2u;
    __half* y = reinterpret_cast<__half*>(temp_get(A(3), (uint32_t)ybytes));
    if (!y) return ERR("w4g_fused out alloc");
    g.stats.matmul++;
    W4gEpilogue epi;
    epi.res = res;
    epi.ldr = n_out;
    epi.swiglu = swiglu;
    const bool gemv_fits = w4g_gemv_supported(M, K);
    if (g_merge_pending.op == cx.op) {   // left by the q|k|v GEMV two ops back
        const MergePending mp = g_merge_pending;
        g_merge_pending = MergePending{};
        // In that launch the merge workgroups store the attention output while the GEMV
        // workgroups read the residual and store y: neither may share its bytes (a
        // memory plan may place y over the attention output, dead after this op).
        auto apart = [](const void* p, size_t np, const void* q, size_t nq) {
            const uint8_t* a0 = static_cast<const uint8_t*>(p);
            const uint8_t* b0 = static_cast<const uint8_t*>(q);
            return a0 + np <= b0 || b0 + nq <= a0;
        };
        const size_t ob = (size_t)mp.H * 128u * 2u;
        if (gemv_fits && M == 1 && a == mp.out && !gamma && !swiglu && ldy == N && ((uintptr_t)ws & 1u) == 0 &&
            apart(y, (size_t)N * 2u, mp.out, ob) && (!res || apart(res, (size_t)N * 2u, mp.out, ob))) {
            CHECK_LAUNCH(launch_merge_oproj(mp.count, mp.out, mp.H, mp.KVH, mp.nslots, mp.theta, g.attn_work,
                                            g.attn_work_floats, wq, ws, y, N, res, g.stream));
            g.merge_oproj_fused++;
            return 0;
        }
        CHECK_LAUNCH(launch_attn_merge_deferred(mp.count, mp.out, mp.H, mp.KVH, mp.nslots, mp.theta, g.attn_work,
                                                g.stream));
    }
    if (gemv_fits) {
        epi.gamma = gamma;
        // The OP_ATTN_DECODE_QKV_F16 that reads this q|k|v row next, in the same run:
        // one launch runs the GEMV and that op's chunk pass side by side (the chunk
        // workgroups' K/V loads overlap the GEMV), then its merge pass; that op then finds
        // its work done. Shapes the launch does not take leave the op to run alone.
        const wt_op* rx = cx.op + 1;
        if (fusion_on() && M == 1 && !swiglu && !res && ldy == N && (uint32_t)(rx - cx.b->ops) < g_run_end &&
            rx->opcode == OP_ATTN_DECODE_QKV_F16 && rx->n_args >= 10 && rx->args[0] == A(3) && rx->args[5] == 128 &&
            rx->args[4] && rx->args[3] % rx->args[4] == 0 &&
            (uint64_t)(rx->args[3] + 2ull * rx->args[4]) * 128u == N) {
            AttnQkv r;
            char rerr[8];
            if (attn_qkv_prep(cx.b, rx, r, rerr, sizeof rerr) == 0) {
                // The launch's GEMV reads x while its chunk workgroups write the ring, and
                // writes y while they read the ring: both must be apart.
                const uint8_t* rb = r.s->dev;
                const uint64_t rn = (uint64_t)r.s->nslots * r.s->slot_bytes;
                auto apart = [&](const void* p, uint64_t n) {
                    const uint8_t* q = static_cast<const uint8_t*>(p);
                    return q + n <= rb || q >= rb + rn;
                };
                auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
                if (apart(a, (uint64_t)K * 2u) && apart(y, (uint64_t)N * 2u) && apart(gamma ? gamma : a, K * 2u) &&
                    al16(g.attn_work) && al16(r.o) && qkv_attn_decode_supported(K, r.H, r.KVH, r.s->nslots)) {
                    // The o-proj GEMV reading the attention output right after (M = 1, no
                    // RMSNorm, no SwiGLU, output stride N) takes the merge pass into its
                    // own launch, where its weight loads overlap the merge.
                    const wt_op* ox = cx.op + 2;
                    const bool defer = (uint32_t)(ox - cx.b->ops) < g_run_end && ox->opcode == OP_W4G_FUSED_F16 &&
                                       ox->n_args >= 11 && ox->args[0] == rx->args[2] && ox->args[4] == 1 &&
                                       ox->args[5] == r.H * 128u && ox->args[7] == WT_REF_NONE && ox->args[9] == 0 &&
                                       ox->args[10] == 2u && merge_oproj_supported(r.H, ox->args[6]);
                    CHECK_LAUNCH(launch_qkv_attn_decode(a, wq, ws, gamma, K, y, r.qg, r.kg, r.theta, r.s->dev,
                                                        r.s->slot_bytes, r.s->nslots, g.counters_dev + r.si, r.o,
                                                        r.H, r.KVH, r.scale, g.attn_work, g.attn_work_floats,
                                                        g.stream, r.s->count + 1, defer));
                    if (defer)
                        g_merge_pending = MergePending{ox, g.counters_dev + r.si, r.o, r.H, r.KVH, r.s->nslots, r.theta};
                    attn_qkv_commit(r);
                    g_attn_pre = rx;
                    g.qkv_attn_fused++;
                    return 0;
                }
            }
        }
        CHECK_LAUNCH(launch_w4g_gemv(a, K, wq, ws, y, ldy, M, N, K, g.stream, epi));
        return 0;
    }
    const __half* src = a;
    const PreNorm pre = g_prenorm;
    g_prenorm = PreNorm{};
    if (gamma) {   // normalize the rows into scratch (unless the previous op did), then the GEMM
        const bool done = pre.op == cx.op && pre.src == a && pre.gamma == gamma && pre.M == M && pre.K == K &&
                          g.norm_buf && g.norm_cap >= (size_t)M * K * 2;
        if (!done) {
            if (scratch(&g.norm_buf, &g.norm_cap, (size_t)M * K * 2, err, errn)) return -1;
            CHECK_LAUNCH(launch_rmsnorm2(a, gamma, nullptr, reinterpret_cast<__half*>(g.norm_buf), M, K, g.stream));
        }
        src = reinterpret_cast<const __half*>(g.norm_buf);
    }
    // The OP_QK_ROPE_KV_F16 that reads this q|k|v output next, in the same run: the
    // GEMM's epilogue performs it (after a table kernel that fixes the positions and
    // advances the counter), writing y as well, and that op then finds its work done.
    // Shapes or operands the epilogue cannot take leave the op to run (or fail) alone.
    const wt_op* rx = cx.op + 1;
    if (fusion_on() && !swiglu && !res && ldy == N && (uint32_t)(rx - cx.b->ops) < g_run_end &&
        rx->opcode == OP_QK_ROPE_KV_F16 && rx->n_args >= 12 && rx->args[0] == A(3) && rx->args[5] == M &&
        rx->args[8] == 128 && (uint64_t)(rx->args[6] + 2ull * rx->args[7]) * 128u == N) {
        QkRope r;
        char rerr[8];
        auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
        if (qk_rope_prep(cx.b, rx, r, rerr, sizeof rerr) == 0 && al16(y) && ldy % 8 == 0 && al16(r.qg) &&
            al16(r.kg) && al16(r.q_out) && al16(r.k_out) && al16(r.v_out) && al16(r.s->dev) &&
            r.s->slot_bytes % 16 == 0) {
            if (scratch(&g.rope_buf, &g.rope_cap, w4g_rope_table_bytes(M), err, errn)) return -1;
            W4gRope R;
            R.H = r.H;
            R.KVH = r.KVH;
            R.q_gamma = r.qg;
            R.k_gamma = r.kg;
            R.table = g.rope_buf;
            R.q_out = r.q_out;
            R.k_out = r.k_out;
            R.v_out = r.v_out;
            R.ring = r.s->dev;
            R.slot_bytes = r.s->slot_bytes;
            R.nslots = r.s->nslots;
            epi.rope = &R;
            CHECK_LAUNCH(launch_rope_table(g.counters_dev + r.si, g.counters_dev + WT_MAX_STATES + r.si, r.theta, M,
                                           g.rope_buf, g.stream));
            CHECK_LAUNCH(launch_w4g_gemm(src, K, wq, ws, y, ldy, M, N, K, g.stream, epi));
            qk_rope_commit(r);
            g_rope_pre = rx;
            g.qkv_rope_fused++;
            return 0;
        }
    }
    if (gemm_split_ws(epi, M, N, K, err, errn)) return -1;
    // The next op normalizing this output for its own GEMM: the split's finishing pass
    // writes those rows too (one pass over the output instead of two).
    bool norm_done = false;
    const wt_op* nx = cx.op + 1;
    const __half* ngamma = nullptr;
    if (!gamma && !swiglu && ldy == n_out && epi.split_ws && nx < cx.b->ops + cx.b->n_ops &&
        nx->opcode == OP_W4G_FUSED_F16 && nx->n_args >= 11 && nx->args[0] == A(3) && nx->args[4] == M &&
        nx->args[5] == n_out && !w4g_gemv_supported(M, n_out) && (nx->args[7] & 0x8000u) &&
        (nx->args[7] & 0x7FFFu) < cx.b->n_slots && cx.b->slots[nx->args[7] & 0x7FFFu].len >= (uint64_t)n_out * 2u) {
        ngamma = reinterpret_cast<const __half*>(slot_ptr(cx.b, nx->args[7] & 0x7FFFu));
        if (ngamma) {
            if (scratch(&g.norm_buf, &g.norm_cap, (size_t)M * n_out * 2, err, errn)) return -1;
            epi.norm_gamma = ngamma;
            epi.norm_out = reinterpret_cast<__half*>(g.norm_buf);
            epi.norm_done = &norm_done;
        }
    }
    CHECK_LAUNCH(launch_w4g_gemm(src, K, wq, ws, y, ldy, M, N, K, g.stream, epi));
    if (norm_done) g_prenorm = PreNorm{nx, y, ngamma, M, n_out};
    return 0;
}

int qk_rope_prep(const wt_blob* b, const wt_op* op, QkRope& r, char* err, size_t errn) {
    const uint32_t* a = op->args;
    const uint32_t n_tok = a[5], H = a[6], KVH = a[7], hd = a[8];
    if (hd != 128) return ERR("qk_rope_kv head_dim %u unsupported (128 only)", hd);
    if (!n_tok || !H || !KVH) return ERR("qk_rope_kv empty shape");
    if (H + KVH > 64) return ERR("qk_rope_kv supports at most 64 q + kv heads (got %u)", H + KVH);
    r.qkv = reinterpret_cast<const __half*>(ref_ptr(b, a[0]));
    r.qg = reinterpret_cast<const __half*>(ref_ptr(b, a[9]));
    r.kg = reinterpret_cast<const __half*>(ref_ptr(b, a[10]));
    if (!r.qkv || !r.qg || !r.kg) return ERR("qk_rope_kv ref fail");
    const uint64_t row = (uint64_t)(H + 2 * KVH) * hd;
    const size_t xb = ref_bytes(b, a[0]);
    if (xb && xb < n_tok * row * 2u) return ERR("qk_rope_kv input smaller than n_tok rows");
    const size_t qgb = ref_bytes(b, a[9]), kgb = ref_bytes(b, a[10]);
    if ((qgb && qgb < hd * 2u) || (kgb && kgb < hd * 2u)) return ERR("qk_rope_kv gamma shorter than head_dim");
    r.s = state_kv(a[4], KVH * hd, err, errn);
    if (!r.s) return -1;
    r.si = a[4] & 0x1FFFu;
    if ((uint64_t)r.s->count + n_tok > r.s->nslots)
        return ERR("qk_rope_kv state %u count=%u + %u > nslots=%u", r.si, r.s->count, n_tok, r.s->nslots);
    r.q_out = reinterpret_cast<__half*>(temp_get(a[1], n_tok * H * hd * 2u));
    r.k_out = a[2] == WT_REF_NONE ? nullptr : reinterpret_cast<__half*>(temp_get(a[2], n_tok * KVH * hd * 2u));
    r.v_out = a[3] == WT_REF_NONE ? nullptr : reinterpret_cast<__half*>(temp_get(a[3], n_tok * KVH * hd * 2u));
    if (!r.q_out || (a[2] != WT_REF_NONE && !r.k_out) || (a[3] != WT_REF_NONE && !r.v_out))
        return ERR("qk_rope_kv out alloc");
    r.theta = f32_from_bits(a[11]);
    r.n_tok = n_tok;
    r.H = H;
    r.KVH = KVH;
    return 0;
}
// Host side of the op once its device work is queued: the positions it appends.
void qk_rope_commit(const QkRope& r) {
    const uint32_t pos = r.s->count;
    r.s->count += r.n_tok;
    for (uint32_t t = 0; t < r.n_tok; ++t) kv_mark(*r.s, pos + t);
}

int op_qk_rope_kv(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    if (g_rope_pre == cx.op) {   // the previous op's GEMM epilogue did it (op_w4g_fused)
        g_rope_pre = nullptr;
        return 0;
    }
    QkRope r;
    if (qk_rope_prep(cx.b, cx.op, r, err, errn)) return -1;
    CHECK_LAUNCH(launch_qk_rope_kv(r.qkv, r.n_tok, r.H, r.KVH, r.qg, r.kg, r.theta, r.q_out, r.k_out, r.v_out,
                                   r.s->dev, r.s->slot_bytes, r.s->nslots, g.counters_dev + r.si, g.stream,
                                   g.counters_dev + WT_MAX_STATES + r.si));
    qk_rope_commit(r);
    return 0;
}

// Attention workspace shared by the decode ops (grown on demand). Zeroed when
// allocated: the fused op's RoPE records must start empty (tag 0).
int attn_workspace(uint32_t need, char* err, size_t errn) {
    if (need <= g.attn_work_floats) return 0;
    if (g.attn_work) dev_free(g.attn_work);
    g.attn_work = nullptr;
    g.attn_work_floats = 0;
    if (dev_malloc(reinterpret_cast<void**>(&g.attn_work), (size_t)need * 4u) != hipSuccess)
        return ERR("attn_decode workspace alloc");
    if (launch_fill_zero(g.attn_work, (size_t)need * 4u, g.stream) != hipSuccess)
        return ERR("attn_decode workspace clear");
    g.attn_work_floats = need;
    return 0;
}

int op_attn_decode_qkv(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    if (g_attn_pre == cx.op) {   // the q|k|v GEMV before it ran it in its own launch (op_w4g_fused)
        g_attn_pre = nullptr;
        return 0;
    }
    AttnQkv r;
    if (attn_qkv_prep(cx.b, cx.op, r, err, errn)) return -1;
    attn_qkv_commit(r);
    CHECK_LAUNCH(launch_attn_decode_qkv(r.qkv, r.qg, r.kg, r.theta, r.s->dev, r.s->slot_bytes, r.s->nslots,
                                        g.counters_dev + r.si, r.o, r.H, r.KVH, r.scale, g.attn_work,
                                        g.attn_work_floats, g.stream, r.s->count));
    return 0;
}

int attn_qkv_prep(const wt_blob* b, const wt_op* op, AttnQkv& r, char* err, size_t errn) {
    const uint32_t* a = op->args;
    const uint32_t H = a[3], KVH = a[4], hd = a[5];
    const float theta = f32_from_bits(a[8]), scale = f32_from_bits(a[9]);
    if (hd != 128) return ERR("attn_decode_qkv head_dim %u unsupported (128 only)", hd);
    if (!KVH || H % KVH) return ERR("attn_decode_qkv heads %u not a multiple of kv heads %u", H, KVH);
    const uint32_t rep = H / KVH;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return ERR("attn_decode_qkv group size %u unsupported", rep);
    const __half* qkv = reinterpret_cast<const __half*>(ref_ptr(b, a[0]));
    const __half* qg = reinterpret_cast<const __half*>(ref_ptr(b, a[6]));
    const __half* kg = reinterpret_cast<const __half*>(ref_ptr(b, a[7]));
    if (!qkv || !qg || !kg) return ERR("attn_decode_qkv ref fail");
    const size_t xb = ref_bytes(b, a[0]);
    if (xb && xb < (uint64_t)(H + 2 * KVH) * hd * 2u) return ERR("attn_decode_qkv input smaller than one qkv row");
    const size_t qgb = ref_bytes(b, a[6]), kgb = ref_bytes(b, a[7]);
    if ((qgb && qgb < hd * 2u) || (kgb && kgb < hd * 2u)) return ERR("attn_decode_qkv gamma shorter than head_dim");
    State* s = state_kv(a[1], KVH * hd, err, errn);
    if (!s) return -1;
    const uint32_t si = a[1] & 0x1FFFu;
    if (s->count >= s->nslots)
        return ERR("attn_decode_qkv state %u count=%u >= nslots=%u (context too long)", si, s->count, s->nslots);
    if (kv_check(*s, s->count, err, errn)) return -1;
    __half* o = reinterpret_cast<__half*>(temp_get(a[2], H * hd * 2u));
    if (!o) return ERR("attn_decode_qkv out alloc");
    // sized for the one-launch form too (launch_qkv_attn_decode), which the plain form
    // shares
    if (attn_workspace(attn_qkv_fused_work_floats(s->nslots, H, KVH), err, errn)) return -1;
    r.qkv = qkv;
    r.qg = qg;
    r.kg = kg;
    r.theta = theta;
    r.scale = scale;
    r.H = H;
    r.KVH = KVH;
    r.si = si;
    r.s = s;
    r.o = o;
    return 0;
}

void attn_qkv_commit(const AttnQkv& r) {
    kv_mark(*r.s, r.s->count);
    r.s->count += 1;
}

int flush_merge_pending(char* err, size_t errn) {
    if (!g_merge_pending.op) return 0;
    const MergePending mp = g_merge_pending;
    g_merge_pending = MergePending{};
    CHECK_LAUNCH(launch_attn_merge_deferred(mp.count, mp.out, mp.H, mp.KVH, mp.nslots, mp.theta, g.attn_work,
                                            g.stream));
    return 0;
}

// Host bytes of constant slot s (in-blob weights or the external image), or null.
const uint8_t* slot_host_bytes(const wt_blob* b, uint32_t s) {
    if (s >= b->n_slots) return nullptr;
    const wt_slot& sl = b->slots[s];
    if (sl.addr == WT_SLOT_EXT_WGT) return g.ext_host ? g.ext_host + sl.offset : nullptr;
    if (sl.addr >= WT_SLOT_STATE || (uint64_t)sl.offset + sl.len > b->weight_bytes) return nullptr;
    return b->weight_base + sl.offset;
}

// ---- OP_MATMUL_W4A16 (opcode 1, oplist_exec.c:438-529) ----
// Supply slots (folded bias, act/out tables) are located by length in slot order as
// the reference does; the math is the closed form of kernels/docs/api_v22_w4a16.md:11.
// The folded bias term (+ bias_fold[n], (N/32) x 512 bytes) is stored in the HMX
// engine's own packing, which only the engine's kernel defines (no readable source
// gives the value of bias_fold[n] from those bytes), so only an all-zero bias slot is
// accepted and any other fails the op with an error instead of being dropped.
// The result always lands in the engine's out surface (OP_DMA's ENG_OUT); with a slot
// activation it is also copied to the out temp, with a VTCM-staged activation
// (0x4000|temp) it stays in the engine surface, as in the reference.
int op_matmul_w4a16(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const wt_blob* b = cx.b;
    const uint32_t act_s = A(0), w_s = A(1), out_t = A(2), M = A(3), K = A(4), N = A(5);
    const uint64_t act_b = (uint64_t)M * K * 2u, wt_b = (uint64_t)K * N / 2u, out_b = (uint64_t)M * N * 2u;
    const uint64_t bias_b = (uint64_t)(N / 32u) * 512u, tbl_b = 8ull * (K / 32u) * 4u;
    g.stats.matmul++;
    const uint8_t *bias = nullptr, *atbl = nullptr, *otbl = nullptr;
    uint32_t bias_s = 0;
    for (uint32_t i = 0; i < b->n_slots; ++i) {
        const uint8_t* p = slot_ptr(b, i);
        const uint32_t L = b->slots[i].len;
        if (!bias && L == bias_b) { bias = p; bias_s = i; }
        else if (!atbl && L == tbl_b) atbl = p;
        else if (!otbl && L == tbl_b) otbl = p;
    }
    if (!bias || !atbl || !otbl) return ERR("supply slots missing (bias/atbl/otbl)");
    {
        const uint8_t* hb = slot_host_bytes(b, bias_s);
        if (!hb) return ERR("w4a16 folded bias slot %u not readable on the host", bias_s);
        for (uint64_t i = 0; i < bias_b; ++i)
            if (hb[i])
                return ERR("w4a16 folded bias slot %u is non-zero (byte %llu): its HMX packing is not supported, "
                           "only an all-zero bias runs", bias_s, (unsigned long long)i);
    }
    if (!M || M % 32u || K % 32u || N % 32u || !K || !N)
        return ERR("w4a16 shape m%u k%u n%u (multiples of 32 needed)", M, K, N);
    if (out_b > 0xFFFFFFFFull) return ERR("w4a16 output too large");
    const uint8_t* act = nullptr;
    if (act_s & WT_REF_VTCM_FLAG) {
        act = ref_ptr(b, act_s);
        if (!act) return ERR("dma-prestaged act bad (temp %u not in the VTCM pool)", act_s & 0x3FFFu);
        if (g.vtcm_off_arr[act_s & 0x3FFFu] + act_b > g.vtcm_pool_size) return ERR("dma-prestaged act beyond the pool");
    } else {
        if (act_s >= b->n_slots || b->slots[act_s].len != act_b) return ERR("act slot size mismatch");
        act = slot_ptr(b, act_s);
    }
    if (w_s >= b->n_slots || b->slots[w_s].len != wt_b) return ERR("w slot size mismatch");
    const uint8_t* w = slot_ptr(b, w_s);
    if (!act || !w) return ERR("w4a16 ref fail");
    uint8_t* out = temp_get(out_t, (uint32_t)out_b);
    if (!out) return ERR("temp %u alloc", out_t);
    if (scratch(&g.w4_out, &g.w4_out_cap, out_b, err, errn)) return -1;
    CHECK_LAUNCH(launch_matmul_w4a16(reinterpret_cast<const uint16_t*>(act), w, reinterpret_cast<uint16_t*>(g.w4_out),
                                     M, K, N, g.stream));
    if (!(act_s & WT_REF_VTCM_FLAG) && copy_d2d(out, g.w4_out, out_b) != hipSuccess)
        return ERR("w4a16 out copy");
    g.w4_ready = true;
    g.w4_m = M; g.w4_k = K; g.w4_n = N;
    g.w4_act = const_cast<uint8_t*>(act);
    g.w4_wt = w;
    g.w4_bias = bias;
    *cx.engine_m = M;
    return 0;
}

// ---- OP_RMSNORM_F16 (opcode 2, oplist_exec.c:559-591): rows = the W4A16 engine's M ----
int op_rmsnorm_crouton(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t x_t = A(0), w_s = A(1), y_t = A(2), n = A(3), m = *cx.engine_m;
    g.stats.rmsnorm++;
    obs_read(x_t);
    if (x_t >= kMaxTemps || !g.temps[x_t]) return ERR("rmsnorm src temp %u empty", x_t);
    if (w_s >= cx.b->n_slots || cx.b->slots[w_s].len != n * 2u) return ERR("rms w slot len mismatch");
    if (!m || m % 32u || n % 32u) return ERR("rms shape m%u n%u", m, n);
    if ((uint64_t)m * n * 2u > g.temp_bytes[x_t]) return ERR("rmsnorm src temp %u smaller than m*n", x_t);
    __half* y = reinterpret_cast<__half*>(temp_get(y_t, m * n * 2u));
    const __half* w = reinterpret_cast<const __half*>(slot_ptr(cx.b, w_s));
    if (!y || !w) return ERR("rms alloc");
    CHECK_LAUNCH(launch_rmsnorm_crouton(reinterpret_cast<const uint16_t*>(g.temps[x_t]), w, y, m, n, g.stream));
    return 0;
}

// ---- OP_FILL (opcode 9, oplist_exec.c:864-885): n f16 from a pool slot at byte offset ----
int op_fill(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t pool_s = A(0), off = A(1), dst = A(2), n = A(3);
    const uint64_t bytes = (uint64_t)n * 2u;
    g.stats.fill++;
    if (pool_s >= cx.b->n_slots || cx.b->slots[pool_s].len < (uint64_t)off + bytes) return ERR("fill pool oob");
    const uint8_t* src = slot_ptr(cx.b, pool_s) + off;
    uint8_t* d = nullptr;
    if (dst & 0x8000u) {
        const uint32_t s2 = dst & 0x7FFFu;
        if (s2 >= cx.b->n_slots || cx.b->slots[s2].len < bytes) return ERR("fill dst empty");
        d = slot_ptr(cx.b, s2);
    } else {
        d = temp_get(dst, (uint32_t)bytes);
    }
    if (!d) return ERR("fill dst empty");
    if (copy_d2d(d, src, bytes) != hipSuccess) return ERR("fill copy");
    return 0;
}

// ---- OP_TRANSPOSE_F16 (opcode 10, oplist_exec.c:983-1011): (1, H, W, C), perm per byte ----
int op_transpose4(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t Hh = A(2), W = A(3), Cc = A(4), perm = A(5);
    g.stats.transpose++;
    const uint64_t n = (uint64_t)Hh * W * Cc;
    const uint8_t* src = ref_ptr(cx.b, A(0));
    if (!src) return ERR("transpose src ref empty");
    const size_t sb = ref_bytes(cx.b, A(0));
    if (sb && sb < n * 2u) return ERR("transpose source smaller than H*W*C");
    for (int i = 0; i < 32; i += 8)
        if (((perm >> i) & 0xFFu) > 3u) return ERR("transpose perm 0x%08X bad", perm);
    uint8_t* dst = temp_get(A(1), (uint32_t)(n * 2u));
    if (!dst) return ERR("transpose temp alloc");
    CHECK_LAUNCH(launch_transpose4(reinterpret_cast<const uint16_t*>(src), reinterpret_cast<uint16_t*>(dst), Hh, W, Cc,
                                   perm, g.stream));
    return 0;
}

// ---- OP_CONCAT_F16 (opcode 14, oplist_exec.c:1196-1220) ----
int op_concat(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t out_t = A(8), n_seg = std::min<uint32_t>(A(10), 4u), n_elems = A(11);
    uint32_t sizes[4] = {A(12), A(13), A(14), A(15)}, total = 0;
    for (uint32_t i = 0; i < n_seg; ++i) total += sizes[i];
    if (total == 0 || n_elems % total != 0) return ERR("concat shape");
    const uint32_t outer = n_elems / total;
    uint16_t* y = reinterpret_cast<uint16_t*>(temp_get(out_t, n_elems * 2u));
    if (!y) return ERR("concat out fail");
    const uint16_t* xs[4] = {nullptr, nullptr, nullptr, nullptr};
    for (uint32_t k = 0; k < n_seg; ++k) {
        xs[k] = reinterpret_cast<const uint16_t*>(ref_ptr(cx.b, A(k)));
        if (!xs[k]) return ERR("concat in fail");
        const size_t xb = ref_bytes(cx.b, A(k));
        if (xb && xb < (uint64_t)outer * sizes[k] * 2u) return ERR("concat segment %u smaller than its span", k);
    }
    CHECK_LAUNCH(launch_concat(xs, sizes, n_seg, y, n_elems, g.stream));
    return 0;
}

// ---- OP_SPLIT_F16 (opcode 16, oplist_exec.c:1222-1256): writes segment split_index ----
int op_split(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t x_t = A(0), n_seg = std::min<uint32_t>(A(10), 4u), idx = A(15);
    uint32_t sizes[4] = {A(11), A(12), A(13), A(14)}, total = 0;
    const uint16_t* x = reinterpret_cast<const uint16_t*>(ref_ptr(cx.b, x_t));
    if (!x) return ERR("split in fail");
    for (uint32_t i = 0; i < n_seg; ++i) total += sizes[i];
    if (total == 0) return ERR("split shape");
    uint32_t x_elems = 0;
    if ((x_t & 0x8000u) == 0 && x_t < kMaxTemps) x_elems = g.temp_bytes[x_t] / 2u;
    if (x_elems == 0) return ERR("split x size");
    const uint32_t outer = x_elems / total;
    uint32_t off = 0;
    for (uint32_t k = 0; k < n_seg; ++k) {
        if (k == idx) {
            uint16_t* y = reinterpret_cast<uint16_t*>(temp_get(A(1), outer * sizes[k] * 2u));
            if (!y) return ERR("split out fail");
            CHECK_LAUNCH(launch_split(x, y, outer, total, off, sizes[k], g.stream));
        }
        off += sizes[k];
    }
    return 0;
}

// ---- OP_REDUCE_F16 (opcode 17, oplist_exec.c:1258-1299) ----
int op_reduce(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(2), axis = A(3), subtype = A(4);
    const uint32_t d[4] = {A(5), A(6), A(7), A(8)};
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    if (!x) return ERR("reduce in fail");
    if (axis >= 4 || subtype > 3) return ERR("reduce axis/subtype bad (axis=%u sub=%u)", axis, subtype);
    const uint32_t L = d[axis] ? d[axis] : 1u;
    uint64_t inner = 1;
    for (uint32_t a = axis + 1; a < 4; ++a) inner *= d[a];
    if (inner * L == 0 || inner * L > 0xFFFFFFFFull || n % (uint32_t)(inner * L) != 0)
        return ERR("reduce geom (n=%u L=%u inner=%llu)", n, L, (unsigned long long)inner);
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)n * 2u) return ERR("reduce input smaller than n");
    const uint32_t outer = n / (uint32_t)(inner * L);
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), (uint32_t)(outer * inner * 2u)));
    if (!y) return ERR("reduce out fail");
    CHECK_LAUNCH(launch_reduce(x, y, outer, L, (uint32_t)inner, subtype, g.stream));
    return 0;
}

// ---- OP_CUMSUM_F32 (opcode 18, oplist_exec.c:1320-1347) ----
int op_cumsum(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t rows = A(2), n = A(3), excl = A(5), rev = A(6);
    const uint64_t bytes = (uint64_t)rows * n * 2u;
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), (uint32_t)bytes));
    if (!x || !y || bytes > 0xFFFFFFFFull) return ERR("cumsum ref fail");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < bytes) return ERR("cumsum input smaller than rows*n");
    CHECK_LAUNCH(launch_cumsum(x, y, rows, n, excl, rev, g.stream));
    return 0;
}

// ---- OP_GATHER_F16 (opcode 20, oplist_exec.c:1378-1436) ----
int op_gather(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n = A(3), packed = A(4);
    const uint32_t axis = packed & 0xFFu, xrank = (packed >> 8) & 0xFFu, irank = (packed >> 16) & 0xFFu;
    const uint32_t td[5] = {A(5), A(6), A(7), A(8), A(9)}, xd[5] = {A(10), A(11), A(12), A(13), A(14)};
    const uint16_t* tbl = reinterpret_cast<const uint16_t*>(ref_ptr(cx.b, A(0)));
    const int32_t* idx = reinterpret_cast<const int32_t*>(ref_ptr(cx.b, A(1)));
    uint16_t* y = reinterpret_cast<uint16_t*>(temp_get(A(2), n * 2u));
    if (!tbl || !idx || !y) return ERR("gather ref fail");
    if (axis >= irank || irank > 5 || xrank > 5 || xrank == 0)
        return ERR("gather axis/rank bad (a=%u x=%u i=%u)", axis, xrank, irank);
    uint64_t tn = 1, xn = 1;
    for (int i = 0; i < 5; ++i) {
        if (!td[i] || !xd[i]) return ERR("gather zero dimension");
        tn *= td[i];
        xn *= xd[i];
    }
    const size_t tb = ref_bytes(cx.b, A(0)), ib = ref_bytes(cx.b, A(1));
    if ((tb && tb < tn * 2u) || (ib && ib < xn * 4u)) return ERR("gather table or index smaller than its dims");
    CHECK_LAUNCH(launch_gather(tbl, idx, y, n, axis, xrank, irank, td, xd, g.stream));
    return 0;
}

// ---- OP_DMA (opcode 33, oplist_exec.c:887-981): a device copy between references ----
uint8_t* dma_resolve(const wt_blob* b, uint32_t ref, uint32_t off, uint32_t bytes, bool is_dst) {
    if ((ref & 0xC000u) == WT_REF_ENG_FLAG) {
        if (!g.w4_ready) return nullptr;
        uint8_t* p = nullptr;
        uint64_t cap = 0;
        switch (ref & 0xFFu) {
        case WT_ENG_ACT: p = g.w4_act; cap = (uint64_t)g.w4_m * g.w4_k * 2u; break;
        case WT_ENG_OUT: p = g.w4_out; cap = (uint64_t)g.w4_m * g.w4_n * 2u; break;
        case WT_ENG_WT: p = const_cast<uint8_t*>(g.w4_wt); cap = (uint64_t)g.w4_k * g.w4_n / 2u; break;
        case WT_ENG_BIAS: p = const_cast<uint8_t*>(g.w4_bias); cap = (uint64_t)(g.w4_n / 32u) * 512u; break;
        default: return nullptr;
        }
        if (!p || (uint64_t)off + bytes > cap) return nullptr;
        return p + off;
    }
    if (ref & 0x8000u) {
        const uint32_t s = ref & 0x7FFFu;
        if (s >= b->n_slots || (uint64_t)off + bytes > b->slots[s].len) return nullptr;
        uint8_t* p = slot_ptr(b, s);
        return p ? p + off : nullptr;
    }
    if (!is_dst) obs_read(ref);
    if (ref & 0x4000u) {
        const uint32_t t = ref & 0x3FFFu;
        if (t >= kMaxTemps || g.vtcm_off_arr[t] == kNone || !g.vtcm_pool) return nullptr;
        if ((uint64_t)g.vtcm_off_arr[t] + off + bytes > g.vtcm_pool_size) return nullptr;
        return g.vtcm_pool + g.vtcm_off_arr[t] + off;
    }
    if (ref >= kMaxTemps) return nullptr;
    if (is_dst) {
        uint8_t* p = temp_get(ref, off + bytes);
        return p ? p + off : nullptr;
    }
    if (!g.temps[ref] || (uint64_t)off + bytes > g.temp_bytes[ref]) return nullptr;
    return g.temps[ref] + off;
}

int op_dma(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t bytes = A(2), f_src = A(6), f_dst = A(7);
    if (bytes == 0) return 0;
    if ((f_src > 3u && f_src != WT_DMA_FENCE_NONE) || (f_dst > 3u && f_dst != WT_DMA_FENCE_NONE))
        return ERR("dma fence arg bad");
    if ((uint64_t)A(4) + bytes > 0xFFFFFFFFull) return ERR("dma ref fail");
    const uint8_t* src = dma_resolve(cx.b, A(0), A(3), bytes, false);
    uint8_t* dst = dma_resolve(cx.b, A(1), A(4), bytes, true);
    if (!src || !dst) return ERR("dma ref fail");
    if (copy_d2d(dst, src, bytes) != hipSuccess) return ERR("dma copy");
    return 0;
}

// ---- OP_PAD_F16 (opcode 34, oplist_exec.c:1301-1318) ----
int op_pad(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t outer = A(2), in_inner = A(3), out_inner = A(4), before = A(5);
    const uint16_t pv = (uint16_t)A(6);
    const uint64_t ob = (uint64_t)outer * out_inner * 2u;
    const uint16_t* x = reinterpret_cast<const uint16_t*>(ref_ptr(cx.b, A(0)));
    uint16_t* y = ob <= 0xFFFFFFFFull ? reinterpret_cast<uint16_t*>(temp_get(A(1), (uint32_t)ob)) : nullptr;
    if (!x || !y) return ERR("pad ref fail");
    if ((uint64_t)before + in_inner > out_inner) return ERR("pad geom");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < (uint64_t)outer * in_inner * 2u) return ERR("pad input smaller than outer*in_inner");
    CHECK_LAUNCH(launch_pad(x, y, outer, in_inner, out_inner, before, pv, g.stream));
    return 0;
}

int op_rope(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    const uint32_t n_tok = A(2), H = A(3), hd = A(4), pos0 = A(5), row_stride = A(7);
    const float theta = f32_from_bits(A(6));
    if (hd == 0 || hd % 2) return ERR("rope head_dim %u must be even", hd);
    if (row_stride < H * hd) return ERR("rope row stride %u < heads*hd %u", row_stride, H * hd);
    const __half* x = reinterpret_cast<const __half*>(ref_ptr(cx.b, A(0)));
    const uint64_t bytes = (uint64_t)n_tok * row_stride * 2u;
    __half* y = reinterpret_cast<__half*>(temp_get(A(1), (uint32_t)bytes));
    if (!x || !y) return ERR("rope ref fail");
    const size_t xb = ref_bytes(cx.b, A(0));
    if (xb && xb < bytes) return ERR("rope input smaller than n_tok*row_stride");
    const uint32_t* pos_dev = nullptr;
    uint32_t base = pos0;
    if ((pos0 & 0xFFFFE000u) == WT_REF_STATE_FLAG) {
        const uint32_t si = pos0 & 0x1FFFu;
        if (si >= g.n_states) return ERR("rope state %u oob", si);
        pos_dev = g.counters_dev + si;
        base = 0;
    }
    CHECK_LAUNCH(launch_rope(x, y, n_tok, H, hd, base, pos_dev, theta, row_stride, g.stream));
    return 0;
}

int op_unsupported(Ctx& cx) {
    char* err = cx.err; size_t errn = cx.errn;
    return ERR("opcode %u has no HIP kernel in this build", (unsigned)cx.op->opcode);
}

typedef int (*OpFn)(Ctx&);

struct Table {
    OpFn fn[64];
    Table() {
        for (auto& f : fn) f = op_unsupported;
        fn[OP_NOP] = op_nop;
        fn[OP_MATMUL_W4A16] = op_matmul_w4a16;
        fn[OP_RMSNORM_F16] = op_rmsnorm_crouton;
        fn[OP_FILL] = op_fill;
        fn[OP_TRANSPOSE_F16] = op_transpose4;
        fn[OP_CONCAT_F16] = op_concat;
        fn[OP_SPLIT_F16] = op_split;
        fn[OP_REDUCE_F16] = op_reduce;
        fn[OP_CUMSUM_F32] = op_cumsum;
        fn[OP_GATHER_F16] = op_gather;
        fn[OP_DMA] = op_dma;
        fn[OP_PAD_F16] = op_pad;
        fn[OP_PIN] = op_pin;
        fn[OP_SILU_F16] = op_silu;
        fn[OP_ADD_F16] = op_add;
        fn[OP_UNARY_F16] = op_unary;
        fn[OP_BINARY_F16] = op_binary;
        fn[OP_SOFTMAX_F16] = op_softmax;
        fn[OP_STRIDED_SLICE_F16] = op_slice;
        fn[OP_ARGMAX_F16] = op_argmax;
        fn[OP_KV_APPEND_F16] = op_kv_append;
        fn[OP_KV_GATHER_F16] = op_kv_gather;
        fn[OP_MATMUL_F16] = op_matmul_f16;
        fn[OP_MATMUL_F16_SPLIT] = op_matmul_f16;
        fn[OP_RMSNORM2_F16] = op_rmsnorm2;
        fn[OP_BROADCAST_F16] = op_broadcast;
        fn[OP_TRANSPOSE_GEN_F16] = op_transpose_gen;
        fn[OP_MATMUL_W4G_F16] = op_matmul_w4g;
        fn[OP_ATTN_F16] = op_attn;
        fn[OP_ATTN_DECODE_F16] = op_attn_decode;
        fn[OP_ROPE_F16] = op_rope;
        fn[OP_KV_APPEND_N_F16] = op_kv_append_n;
        fn[OP_W4G_FUSED_F16] = op_w4g_fused;
        fn[OP_QK_ROPE_KV_F16] = op_qk_rope_kv;
        fn[OP_ATTN_DECODE_QKV_F16] = op_attn_decode_qkv;
    }
};
const Table kTable;

// Tensor dump hook "opidx:temp,..." (oplist_exec.c:108-166): host files /tmp/hook_<i>_<t>.f16.raw.
const char* hook_spec() {
    static const char* env_hook = nullptr;
    static bool env_tried = false;
    if (g.hook) return g.hook;
    if (!env_tried) { env_hook = std::getenv("GEHTP_HOOK"); env_tried = true; }
    return env_hook;
}

void hook_dump(uint32_t ii) {
    const char* hook = hook_spec();
    if (!hook || !hook[0]) return;
    const char* tok = hook;
    while (*tok) {
        const char* comma = std::strchr(tok, ',');
        const size_t len = comma ? (size_t)(comma - tok) : std::strlen(tok);
        std::string item(tok, len);
        const size_t colon = item.find(':');
        if (colon != std::string::npos) {
            const uint32_t hi = (uint32_t)std::strtoul(item.substr(0, colon).c_str(), nullptr, 0);
            const uint32_t ht = (uint32_t)std::strtoul(item.substr(colon + 1).c_str(), nullptr, 0);
            if (hi == ii && ht < kMaxTemps && g.temps[ht]) {
                std::vector<uint8_t> host(g.last_bytes[ht]);
                if (hipStreamSynchronize(g.stream) == hipSuccess &&
                    hipMemcpy(host.data(), g.temps[ht], host.size(), hipMemcpyDeviceToHost) == hipSuccess) {
                    char fn[128];
                    std::snprintf(fn, sizeof fn, "/tmp/hook_%u_%u.f16.raw", hi, ht);
                    if (FILE* f = std::fopen(fn, "wb")) {
                        std::fwrite(host.data(), 1, host.size(), f);
                        std::fclose(f);
                    }
                }
            }
        }
        if (!comma) break;
        tok = comma + 1;
    }
}


// ---- graph replay of repeated runs ----
// A decode step runs the same ops on the same buffers every time, and its kernels
// read positions from the device counters, so its launches (kernel, grid, arguments)
// repeat exactly. Once one direct run of a range has shown that (no device buffer
// moved during it, no op passed host-side step state to a kernel), the next identical
// run is captured into a HIP graph. Later identical runs launch the graph and then
// walk the ops on the host with device work suppressed, which keeps the host-side
// bookkeeping (KV position mirrors, temp sizes, stats) exactly as a direct run
// leaves it. A preflight of the KV capacity checks comes first, so a run that would
// fail its host-side checks takes the direct path and fails at the same op.
// Host state a handler may read that an earlier run left behind: element counts of
// temps (ref_elem_count) and the opcode-1 engine surfaces (OP_DMA's 0xC000 refs).
struct HostIn {   // no padding: compared with memcmp
    uint32_t last_bytes[kMaxTemps];
    uint32_t w4_ready, w4_m, w4_k, w4_n;
    const void* w4p[4];
};
static_assert(sizeof(HostIn) == kMaxTemps * 4 + 16 + 4 * sizeof(void*), "HostIn has padding");
void host_in(HostIn& h) {
    std::memset(&h, 0, sizeof h);
    std::memcpy(h.last_bytes, g.last_bytes, sizeof h.last_bytes);
    h.w4_ready = g.w4_ready ? 1u : 0u;
    h.w4_m = g.w4_m; h.w4_k = g.w4_k; h.w4_n = g.w4_n;
    h.w4p[0] = g.w4_out; h.w4p[1] = g.w4_act; h.w4p[2] = g.w4_wt; h.w4p[3] = g.w4_bias;
}

struct RunSig {
    const wt_blob* b = nullptr;
    uint32_t first = 0, count = 0;
    bool in_active = false;
    const uint8_t* in_src = nullptr;
    uint64_t epoch = 0, w_key = 0, ext_key = 0;
    std::vector<wt_op> ops;
    HostIn in{};   // at the start of the run

    bool same(const wt_blob* bb, uint32_t f, uint32_t c, const HostIn& now) const {
        return b == bb && first == f && count == c && in_active == g.in_active && in_src == g.in_src && epoch == g.epoch &&
               w_key == g.w_key && ext_key == g.ext_key && ops.size() == c &&
               std::memcmp(ops.data(), bb->ops + f, sizeof(wt_op) * c) == 0 &&
               std::memcmp(&in, &now, sizeof in) == 0;
    }
    void set(const wt_blob* bb, uint32_t f, uint32_t c, const HostIn& start) {
        b = bb; first = f; count = c;
        in_active = g.in_active;
        in_src = g.in_src;
        epoch = g.epoch; w_key = g.w_key; ext_key = g.ext_key;
        ops.assign(bb->ops + f, bb->ops + f + c);
        in = start;
    }
};

struct RunGraph {
    RunSig sig;
    hipGraphExec_t exec = nullptr;
    std::vector<std::pair<uint32_t, uint32_t>> adv;   // (state, positions the run appends)
    uint64_t used = 0;
};

constexpr size_t kMaxGraphs = 4;
std::vector<RunGraph> g_graphs;
RunSig g_stable;            // last direct run that qualified for capture
bool g_stable_ok = false;
uint64_t g_use_tick = 0;

bool graphs_on() {
    if (g.graphs < 0) {
        const char* e = std::getenv("GEHTP_NO_GRAPH");
        g.graphs = (e && e[0] && e[0] != '0') ? 0 : 1;
    }
    return g.graphs == 1 && !g.graphs_broken;
}

// Callers hold the stream idle (runs drain it before returning).
void drop_graphs() {
    if (!g_graphs.empty() && g.stream) hipStreamSynchronize(g.stream);
    for (RunGraph& r : g_graphs)
        if (r.exec) hipGraphExecDestroy(r.exec);
    g_graphs.clear();
    g_stable_ok = false;
}

RunGraph* find_graph(const wt_blob* b, uint32_t first, uint32_t count, const HostIn& now) {
    for (RunGraph& r : g_graphs)
        if (r.sig.same(b, first, count, now)) return &r;
    return nullptr;
}

bool preflight(const RunGraph& r) {
    for (const auto& a : r.adv) {
        if (a.first >= g.n_states) return false;
        const State& s = g.st[a.first];
        if (!s.kv_ready || (uint64_t)s.count + a.second > s.nslots || s.valid_prefix < s.count) return false;
    }
    return true;
}

void keep_graph(const wt_blob* b, uint32_t first, uint32_t count, hipGraphExec_t exec, const uint32_t* counts0,
                const HostIn& start) {
    if (g_graphs.size() >= kMaxGraphs) {
        auto lru = std::min_element(g_graphs.begin(), g_graphs.end(),
                                    [](const RunGraph& x, const RunGraph& y) { return x.used < y.used; });
        hipGraphExecDestroy(lru->exec);
        g_graphs.erase(lru);
    }
    RunGraph r;
    r.sig.set(b, first, count, start);
    r.exec = exec;
    r.used = ++g_use_tick;
    for (uint32_t i = 0; i < g.n_states; ++i)
        if (g.st[i].count != counts0[i]) r.adv.emplace_back(i, g.st[i].count - counts0[i]);
    g_graphs.push_back(std::move(r));
}

// ---- load-time fusion of the reference attention chains ----
// The reference composes attention from runlist ops (oplist_exec.c:1081-1194,
// 1709-1813, 1876-1907, 2183-2231) in the forms its emitter writes
// (compiler/tools/wtop_ops/op_matmul.cpp:36-98, op_eltwise_binary.cpp:9-67,
// op_softmax.cpp:9-21, op_decode_state.cpp:66-80):
//   prefill: [q = BINARY mul(q0, scale)] -> MATMUL_F16 q.k^T with the heads in the batch
//     dimension ([H, S, 128]; k given with flags bit1, or as k^T [H, 128, S] written by
//     a TRANSPOSE_GEN of k; one unbatched head likewise) -> [BINARY mul by a scale] ->
//     [BINARY add or ADD_F16 of an additive mask: causal 0 / -inf, or all zero] ->
//     SOFTMAX over rows -> MATMUL_F16 p.v;
//   decode (scripts/surgery_decode_graph.py:143-168): KV_GATHER of a state (one op with
//     both faces, or one op per face: kT [H, hd, P], v [H, P, hd]) -> [pre-scale] ->
//     MATMUL_F16 q.kT -> [BINARY mul by a scale] -> [add of a mask operand of H rows of
//     P, or of one row BROADCAST over the heads] -> SOFTMAX -> MATMUL_F16 p.v.
// A scale is a constant slot of equal positive values or a BROADCAST of one; a prefill
// mask is a constant slot or a BROADCAST of one over the heads. BROADCAST and
// TRANSPOSE_GEN ops that feed the chain are members of it. Members are found by
// dataflow (for each operand, the op that last wrote it), not by adjacency: other ops
// may stand between them, and temp ids the emitter recycles are followed
// (compiler/tools/wtop_ops/wtop_ops.hpp:131-146). The chain runs as one kernel at its
// last member (the flash prefill kernel, or the split-KV decode kernel reading the ring
// in place), each input's device pointer taken where the member reading it stands; the
// other members are skipped.
//
// A blob's first full run executes every chain op by op and logs reads and writes; a
// chain is fused on later runs only if the log shows (fusion_validate):
//  - each member read the value the matcher expects (nothing rewrote it in between);
//  - no other op read an intermediate of the chain (inside its window, or after it
//    before the temp is written again, or as run_io's output), and no member read one
//    carried over from a previous run; a BROADCAST, TRANSPOSE_GEN or KV_GATHER member
//    whose output other ops read still runs (it is kept, not skipped);
//  - no other op that still runs wrote over an input's bytes between the member's read
//    and the last member (under a TEMPOFF plan, temps of other ids may share them).
// When the output's bytes overlap an input's at run time (a plan may place the output
// over k, dead after the first matmul in op order), the kernel writes engine scratch
// and the result is copied to the output. Fused results are within the fp16 tolerance
// of the chain, not its per-op roundings.
constexpr uint32_t kChainMax = 12;   // member ops of one chain
constexpr uint32_t kWindow = 48;     // ops searched before / after a member for its neighbours

struct ChainEdge { uint32_t op, id, from; };   // member `op` reads temp `id` last written by op `from` (kNone: an input)

struct AttnChain {
    uint32_t mem[kChainMax] = {};
    uint32_t n_mem = 0;
    uint32_t head = 0, last = 0;          // first and last member (the kernel runs at `last`)
    uint32_t S = 0, H = 0;
    float scale = 1.0f;
    bool causal = false;
    bool decode = false;
    // Kernel inputs: each reference and the member op where its pointer is taken.
    uint32_t q = 0, k = 0, v = 0, mask = kNone;
    uint32_t q_at = 0, k_at = 0, v_at = 0, mask_at = 0;
    bool mask_shared = false;             // decode: one mask row for every head
    uint32_t out = 0;                     // the last member's output temp
    uint32_t state = 0, KVH = 0, P = 0, n_kv = 0;   // decode: gathered state, kv heads, layout, n_kv arg
    ChainEdge edge[2 * kChainMax] = {};
    uint32_t n_edge = 0;
};
struct FusionPlan {
    const wt_blob* b = nullptr;
    uint32_t n_ops = 0;
    uint64_t parse_epoch = 0;
    bool observed = false;
    std::vector<AttnChain> chains;
    std::vector<uint8_t> blocked;          // per chain: the observed run ruled fusion out
    std::vector<uint32_t> keep;            // per chain: members (bit k = mem[k]) that run when fused
    std::vector<uint8_t> aliased;          // per chain: observed output bytes overlapping an input's
    std::vector<int32_t> member_of;        // op index -> chain index (-1: none)
    uint64_t used = 0;
};
struct FusedIn { const uint8_t* q = nullptr; const uint8_t* k = nullptr; const uint8_t* v = nullptr;
                 const uint8_t* mask = nullptr; };
constexpr size_t kMaxPlans = 8;
std::vector<FusionPlan> g_plans;
uint64_t g_plan_tick = 0;
const FusionPlan* g_fplan = nullptr;   // plan applied to the current run (observed, fusion on)
FusionPlan* g_obs_plan = nullptr;      // plan being observed during the current run
std::vector<uint8_t> g_active;         // per chain of g_fplan: running fused in the current run
std::vector<FusedIn> g_fin;            // per chain: input pointers taken so far in the current run
uint32_t g_run_end = 0;                // one past the current run's last op

bool fusion_on() {
    if (g.fusion < 0) {
        const char* e = std::getenv("GEHTP_NO_FUSE");
        g.fusion = (e && e[0] && e[0] != '0') ? 0 : 1;
    }
    return g.fusion == 1;
}

bool is_temp_ref(uint32_t r) {
    return !(r & 0x8000u) && (r & 0xE000u) != WT_REF_STATE_FLAG && (r & 0x3FFFu) < kMaxTemps;
}
bool same_temp(uint32_t a, uint32_t b) { return is_temp_ref(a) && is_temp_ref(b) && (a & 0x3FFFu) == (b & 0x3FFFu); }

// Host bytes of a constant slot reference (in-blob or external weights), or null.
const uint16_t* slot_host_f16(const wt_blob* b, uint32_t ref, uint64_t n) {
    if (!(ref & 0x8000u)) return nullptr;
    const uint32_t s = ref & 0x7FFFu;
    if (s >= b->n_slots) return nullptr;
    const wt_slot& sl = b->slots[s];
    if ((uint64_t)sl.len < n * 2u) return nullptr;
    const uint8_t* p = nullptr;
    if (sl.addr == WT_SLOT_EXT_WGT) {
        p = g.ext_host ? g.ext_host + sl.offset : nullptr;
    } else if (sl.addr < WT_SLOT_STATE) {
        if ((uint64_t)sl.offset + sl.len > b->weight_bytes) return nullptr;
        p = b->weight_base + sl.offset;
    }
    return (p && (reinterpret_cast<uintptr_t>(p) & 1u) == 0) ? reinterpret_cast<const uint16_t*>(p) : nullptr;
}

// Whether op o writes temp ref t, for the opcodes a chain is made of.
bool writes_temp(const wt_op& o, uint32_t t) {
    switch (o.opcode) {
    case OP_MATMUL_F16: case OP_BINARY_F16: case OP_ADD_F16:
        return o.n_args >= 3 && same_temp(o.args[2], t);
    case OP_BROADCAST_F16: case OP_TRANSPOSE_GEN_F16: case OP_SOFTMAX_F16:
        return o.n_args >= 2 && same_temp(o.args[1], t);
    case OP_KV_GATHER_F16:
        return o.n_args >= 3 && ((o.args[1] && same_temp(o.args[1], t)) || (o.args[2] && same_temp(o.args[2], t)));
    default:
        return false;
    }
}

// The latest op in [lo, y) of those opcodes that writes temp t (kNone if none). Other
// ops that may write t in between are found by the observed run's log.
uint32_t writer_before(const wt_blob* b, uint32_t y, uint32_t t, uint32_t lo) {
    if (!is_temp_ref(t)) return kNone;
    for (uint32_t j = y; j-- > lo;)
        if (writes_temp(b->ops[j], t)) return j;
    return kNone;
}

// The first op in (x, x + kWindow] of those opcodes that reads temp t as an input;
// *pos = the argument position.
bool next_reader(const wt_blob* b, uint32_t x, uint32_t t, uint32_t* at, uint32_t* pos) {
    const uint32_t hi = (uint32_t)std::min<uint64_t>((uint64_t)x + kWindow, b->n_ops - 1u);
    for (uint32_t j = x + 1; j <= hi; ++j) {
        const wt_op& o = b->ops[j];
        uint32_t np = 0;
        switch (o.opcode) {
        case OP_MATMUL_F16: case OP_BINARY_F16: case OP_ADD_F16: np = 2; break;
        case OP_SOFTMAX_F16: case OP_BROADCAST_F16: case OP_TRANSPOSE_GEN_F16: np = 1; break;
        default: break;
        }
        for (uint32_t p = 0; p < np && p < o.n_args; ++p)
            if (same_temp(o.args[p], t)) { *at = j; *pos = p; return true; }
    }
    return false;
}

// A BROADCAST that repeats its n_in-element input `reps` times back to back (numpy
// broadcast of one leading axis of 1; dims of 4, left- or right-aligned).
bool bcast_tiles(const wt_op& B, uint64_t n_in, uint32_t reps) {
    if (B.n_args < 12 || B.args[3] != n_in || (uint64_t)B.args[2] != n_in * reps) return false;
    const uint32_t* id = &B.args[4];
    const uint32_t* od = &B.args[8];
    uint32_t j = 0;
    while (j < 4 && id[j] == od[j]) ++j;
    if (j == 4) return reps == 1;
    uint64_t outer = 1;
    for (uint32_t i = 0; i < j; ++i) outer *= od[i];
    if (outer != 1 || id[j] != 1 || od[j] != reps) return false;
    for (uint32_t i = j + 1; i < 4; ++i)
        if (id[i] != od[i]) return false;
    return true;
}

struct Matcher {
    const wt_blob* b;
    const std::vector<int32_t>& member_of;   // ops claimed by earlier chains
    AttnChain c;
    uint32_t lo = 0;                         // lowest op index searched for a member

    bool add(uint32_t op) {
        for (uint32_t k = 0; k < c.n_mem; ++k)
            if (c.mem[k] == op) return true;
        if (c.n_mem >= kChainMax || member_of[op] >= 0) return false;
        c.mem[c.n_mem++] = op;
        return true;
    }
    bool edge(uint32_t op, uint32_t ref, uint32_t from) {
        if (!is_temp_ref(ref)) return true;
        if (c.n_edge >= 2 * kChainMax) return false;
        c.edge[c.n_edge++] = {op, ref & 0x3FFFu, from};
        return true;
    }
    // A BROADCAST written into operand `ref` of op `at`: made a member (if no earlier
    // chain holds it) and recorded as the operand's writer.
    bool bcast_member(uint32_t at, uint32_t ref, uint32_t j) {
        if (member_of[j] < 0 && !add(j)) return false;
        return edge(at, ref, j);
    }
    // The positive scale of operand `ref` (n elements) of op `at`: a slot of n equal
    // values, or a BROADCAST of a slot of equal values.
    bool scale_source(uint32_t at, uint32_t ref, uint64_t n, float* sc) {
        const uint16_t* p = nullptr;
        uint64_t m = n;
        uint32_t j = kNone;
        if (ref & 0x8000u) {
            p = slot_host_f16(b, ref, n);
        } else if (is_temp_ref(ref)) {
            j = writer_before(b, at, ref, lo);
            if (j == kNone) return false;
            const wt_op& B = b->ops[j];
            if (B.opcode != OP_BROADCAST_F16 || B.n_args < 12 || B.args[2] != n || !B.args[3]) return false;
            m = B.args[3];
            p = slot_host_f16(b, B.args[0], m);
        }
        if (!p) return false;
        for (uint64_t e = 1; e < m; ++e)
            if (p[e] != p[0]) return false;
        const float v = (float)__builtin_bit_cast(_Float16, p[0]);
        if (!(v > 0.0f && v < INFINITY)) return false;
        *sc = v;
        return j == kNone || bcast_member(at, ref, j);
    }
    // q, or a pre-scaled q: BINARY mul of q0 by a constant scale (written before `at`).
    bool query(uint32_t at, uint32_t qref, uint64_t nq, bool* pre) {
        *pre = false;
        c.q = qref;
        c.q_at = at;
        const uint32_t j = writer_before(b, at, qref, lo);
        if (j != kNone && member_of[j] < 0) {
            const wt_op& P = b->ops[j];
            if (P.opcode == OP_BINARY_F16 && P.n_args >= 5 && P.args[4] == 2u && P.args[3] == nq) {
                for (uint32_t side = 0; side < 2 && !*pre; ++side) {
                    const uint32_t q0 = P.args[side], sref = P.args[1 - side];
                    if (!is_temp_ref(q0) && !(q0 & 0x8000u)) continue;
                    const uint32_t n0 = c.n_mem, e0 = c.n_edge;
                    float sc;
                    if (scale_source(j, sref, nq, &sc)) {
                        *pre = true;
                        c.scale = sc;
                        c.q = q0;
                        c.q_at = j;
                        if (!add(j) || !edge(j, q0, kNone)) return false;
                    } else {
                        c.n_mem = n0;
                        c.n_edge = e0;
                    }
                }
            }
        }
        return edge(at, qref, *pre ? j : kNone);
    }
    // Window bounds and ops that would invalidate the chain's inputs unseen by the log.
    bool finish() {
        c.head = c.last = c.mem[0];
        for (uint32_t k = 1; k < c.n_mem; ++k) {
            c.head = std::min(c.head, c.mem[k]);
            c.last = std::max(c.last, c.mem[k]);
        }
        // The kernel reads the ring at the last member; the gathers read it where they
        // stand: no op between them may append to a ring.
        uint32_t ring0 = c.last;
        for (uint32_t k = 0; k < c.n_mem; ++k)
            if (b->ops[c.mem[k]].opcode == OP_KV_GATHER_F16) ring0 = std::min(ring0, c.mem[k]);
        for (uint32_t o = c.head; o <= c.last; ++o) {
            const uint16_t oc = b->ops[o].opcode;
            if (oc == OP_DMA || oc == OP_SPILL || oc == OP_FILL) return false;
            if (c.decode && o > ring0 && (oc == OP_KV_APPEND_F16 || oc == OP_KV_APPEND_N_F16 ||
                                          oc == OP_QK_ROPE_KV_F16 || oc == OP_ATTN_DECODE_QKV_F16))
                return false;
        }
        return true;
    }
};

// Prefill chain whose q.k^T MATMUL_F16 is op i.
bool match_attn_chain(Matcher& m, uint32_t i) {
    const wt_blob* b = m.b;
    AttnChain& c = m.c;
    const wt_op& A = b->ops[i];
    if (A.opcode != OP_MATMUL_F16 || A.n_args < 7) return false;
    const uint32_t S = A.args[3], fl = A.args[6];
    const bool batched = (fl & 4u) != 0;
    const uint32_t H = batched ? fl >> 16 : 1u;
    if (!S || A.args[4] != 128 || A.args[5] != S || !H || (fl & 1u) || (!batched && (fl >> 16))) return false;
    const uint64_t n = (uint64_t)H * S * S;
    if (n > 0xFFFFFFFFull || !is_temp_ref(A.args[2])) return false;
    c = AttnChain{};
    c.S = S; c.H = H;
    m.lo = i > kWindow ? i - kWindow : 0;
    if (!m.add(i)) return false;
    // k: [H, S, 128] read transposed (flags bit1), or k^T [H, 128, S] from a TRANSPOSE_GEN
    if (fl & 2u) {
        if (!is_temp_ref(A.args[1]) && !(A.args[1] & 0x8000u)) return false;
        c.k = A.args[1];
        c.k_at = i;
        if (!m.edge(i, A.args[1], kNone)) return false;
    } else {
        const uint32_t j = writer_before(b, i, A.args[1], m.lo);
        if (j == kNone) return false;
        const wt_op& T = b->ops[j];
        if (T.opcode != OP_TRANSPOSE_GEN_F16 || T.n_args < 8) return false;
        const uint32_t rk = T.args[2], perm = T.args[7];
        const bool ok3 = rk == 3 && T.args[3] == H && T.args[4] == S && T.args[5] == 128 &&
                         (perm & 0xFFFFFFu) == (0u | (2u << 8) | (1u << 16));
        const bool ok2 = rk == 2 && H == 1 && T.args[3] == S && T.args[4] == 128 && (perm & 0xFFFFu) == (1u | (0u << 8));
        if (!(ok3 || ok2) || (!is_temp_ref(T.args[0]) && !(T.args[0] & 0x8000u))) return false;
        if (!m.add(j) || !m.edge(j, T.args[0], kNone) || !m.edge(i, A.args[1], j)) return false;
        c.k = T.args[0];
        c.k_at = j;
    }
    bool pre = false;
    if (!is_temp_ref(A.args[0]) && !(A.args[0] & 0x8000u)) return false;
    if (!m.query(i, A.args[0], (uint64_t)H * S * 128u, &pre)) return false;
    // scale and mask, in either order, then SOFTMAX
    uint32_t prev = A.args[2], at = i, j = 0, pos = 0;
    bool post = false, masked = false;
    for (;;) {
        if (!next_reader(b, at, prev, &j, &pos)) return false;
        const wt_op& X = b->ops[j];
        if (X.opcode == OP_SOFTMAX_F16) break;
        if (pos > 1 || X.args[3] != n || !is_temp_ref(X.args[2])) return false;
        const uint32_t other = X.args[1 - pos];
        if (X.opcode == OP_BINARY_F16 && X.n_args >= 5 && X.args[4] == 2u && !post && !pre) {
            if (!m.scale_source(j, other, n, &c.scale)) return false;
            post = true;
        } else if (((X.opcode == OP_BINARY_F16 && X.n_args >= 5 && X.args[4] == 0u) ||
                    (X.opcode == OP_ADD_F16 && X.n_args >= 4)) && !masked) {
            // additive mask [H, S, S]: a slot, or a BROADCAST of an [S, S] slot over the heads
            const uint16_t* mk = nullptr;
            if (other & 0x8000u) {
                mk = slot_host_f16(b, other, n);
            } else {
                const uint32_t bj = writer_before(b, j, other, m.lo);
                if (bj == kNone || b->ops[bj].opcode != OP_BROADCAST_F16 || !bcast_tiles(b->ops[bj], (uint64_t)S * S, H))
                    return false;
                mk = slot_host_f16(b, b->ops[bj].args[0], (uint64_t)S * S);
                if (mk && !m.bcast_member(j, other, bj)) return false;
            }
            if (!mk) return false;
            const uint64_t nm = (other & 0x8000u) ? n : (uint64_t)S * S;
            bool causal = true, zeros = true;
            for (uint64_t e = 0; e < nm && (causal || zeros); ++e) {
                const uint32_t row = (uint32_t)((e / S) % S), col = (uint32_t)(e % S);
                const bool zero = (mk[e] & 0x7FFFu) == 0;
                zeros = zeros && zero;
                causal = causal && (col <= row ? zero : mk[e] == 0xFC00u);
            }
            if (!causal && !zeros) return false;
            c.causal = causal && S > 1;
            masked = true;
        } else {
            return false;
        }
        if (!m.add(j) || !m.edge(j, prev, at)) return false;
        prev = X.args[2];
        at = j;
    }
    const wt_op& D = b->ops[j];
    if (D.n_args < 4 || D.args[0] != prev || D.args[2] != H * S || D.args[3] != S || !is_temp_ref(D.args[1]))
        return false;
    if (!m.add(j) || !m.edge(j, prev, at)) return false;
    prev = D.args[1];
    at = j;
    if (!next_reader(b, at, prev, &j, &pos)) return false;
    const wt_op& E = b->ops[j];
    if (E.opcode != OP_MATMUL_F16 || E.n_args < 7 || pos != 0 || E.args[3] != S || E.args[4] != S ||
        E.args[5] != 128 || E.args[6] != (batched ? ((H << 16) | 4u) : 0u) || !is_temp_ref(E.args[2]) ||
        (!is_temp_ref(E.args[1]) && !(E.args[1] & 0x8000u)))
        return false;
    if (!m.add(j) || !m.edge(j, prev, at) || !m.edge(j, E.args[1], kNone)) return false;
    c.v = E.args[1];
    c.v_at = j;
    c.out = E.args[2];
    return m.finish() && c.last == j;
}

// Bytes of state idx in the blob's STATE table (0 if absent).
uint32_t blob_state_bytes(const wt_blob* b, uint32_t idx) {
    for (uint32_t s = 0; s < b->n_slots; ++s) {
        const wt_slot& sl = b->slots[s];
        if (sl.addr != WT_SLOT_STATE || (uint64_t)sl.offset + sl.len > b->weight_bytes || sl.len < 4u) continue;
        const uint8_t* p = b->weight_base + sl.offset;
        uint32_t n;
        std::memcpy(&n, p, 4);
        if (idx >= n || sl.len < 4u + 4u * (idx + 1u)) return 0;
        uint32_t bytes;
        std::memcpy(&bytes, p + 4 + 4 * idx, 4);
        return bytes;
    }
    return 0;
}

// Decode chain whose q.kT MATMUL_F16 (one query row) is op i.
bool match_decode_chain(Matcher& m, uint32_t i) {
    const wt_blob* b = m.b;
    AttnChain& c = m.c;
    const wt_op& A = b->ops[i];
    if (A.opcode != OP_MATMUL_F16 || A.n_args < 7 || A.args[3] != 1u || A.args[4] != 128u) return false;
    const uint32_t P = A.args[5], H = A.args[6] >> 16, hd = 128;
    if (!P || !H || A.args[6] != ((H << 16) | 4u) || !is_temp_ref(A.args[1]) || !is_temp_ref(A.args[2])) return false;
    c = AttnChain{};
    c.decode = true;
    c.S = 1; c.H = H; c.P = P;
    m.lo = i > kWindow ? i - kWindow : 0;
    if (!m.add(i)) return false;
    // the kT face: a KV_GATHER of a state
    const uint32_t gk = writer_before(b, i, A.args[1], m.lo);
    if (gk == kNone) return false;
    const wt_op& G = b->ops[gk];
    if (G.opcode != OP_KV_GATHER_F16 || G.n_args < 7 || !G.args[1] || !same_temp(G.args[1], A.args[1])) return false;
    const uint32_t st = G.args[0], n_kv = G.args[3], KVH = G.args[5];
    if ((st & 0xE000u) != WT_REF_STATE_FLAG || G.args[4] != H || G.args[6] != hd || !KVH || H % KVH ||
        H > 0xFFFFu)
        return false;
    const uint32_t rep = H / KVH;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return false;
    uint32_t Pg = n_kv;
    if (n_kv == WT_KV_POS_AUTO) {
        const uint32_t bytes = blob_state_bytes(b, st & 0x1FFFu), slot = KVH * hd * 4u;
        if (!bytes || bytes % slot) return false;
        Pg = bytes / slot;
    }
    if (Pg != P) return false;
    c.state = st; c.KVH = KVH; c.n_kv = n_kv;
    if (!m.add(gk) || !m.edge(i, A.args[1], gk)) return false;
    const uint64_t n = (uint64_t)H * P;
    bool pre = false;
    if (!is_temp_ref(A.args[0]) && !(A.args[0] & 0x8000u)) return false;
    if (!m.query(i, A.args[0], (uint64_t)H * hd, &pre)) return false;
    uint32_t prev = A.args[2], at = i, j = 0, pos = 0;
    bool post = false, masked = false;
    for (;;) {
        if (!next_reader(b, at, prev, &j, &pos)) return false;
        const wt_op& X = b->ops[j];
        if (X.opcode == OP_SOFTMAX_F16) break;
        if (pos > 1 || X.args[3] != n || !is_temp_ref(X.args[2])) return false;
        const uint32_t other = X.args[1 - pos];
        if (X.opcode == OP_BINARY_F16 && X.n_args >= 5 && X.args[4] == 2u && !post && !pre) {
            if (!m.scale_source(j, other, n, &c.scale)) return false;
            post = true;
        } else if (((X.opcode == OP_BINARY_F16 && X.n_args >= 5 && X.args[4] == 0u) ||
                    (X.opcode == OP_ADD_F16 && X.n_args >= 4)) && !masked) {
            // the mask: one row of P BROADCAST over the heads after q.kT (read in place), or
            // H rows (a broadcast written earlier, e.g. once for every layer, is read as it
            // stands: its input row need not outlive it)
            const uint32_t bj = is_temp_ref(other) ? writer_before(b, j, other, m.lo) : kNone;
            if (bj != kNone && bj > i && m.member_of[bj] < 0 && b->ops[bj].opcode == OP_BROADCAST_F16 &&
                bcast_tiles(b->ops[bj], P, H) && (is_temp_ref(b->ops[bj].args[0]) || (b->ops[bj].args[0] & 0x8000u))) {
                if (!m.bcast_member(j, other, bj) || !m.edge(bj, b->ops[bj].args[0], kNone)) return false;
                c.mask = b->ops[bj].args[0];
                c.mask_at = bj;
                c.mask_shared = true;
            } else {
                if (!is_temp_ref(other) && !(other & 0x8000u)) return false;
                if (!m.edge(j, other, kNone)) return false;
                c.mask = other;
                c.mask_at = j;
            }
            masked = true;
        } else {
            return false;
        }
        if (!m.add(j) || !m.edge(j, prev, at)) return false;
        prev = X.args[2];
        at = j;
    }
    if (n_kv == WT_KV_POS_AUTO && P > 1 && !masked) return false;   // the zero-filled tail would take part
    const wt_op& D = b->ops[j];
    if (D.n_args < 4 || D.args[0] != prev || D.args[2] != H || D.args[3] != P || !is_temp_ref(D.args[1]))
        return false;
    if (!m.add(j) || !m.edge(j, prev, at)) return false;
    prev = D.args[1];
    at = j;
    if (!next_reader(b, at, prev, &j, &pos)) return false;
    const wt_op& E = b->ops[j];
    if (E.opcode != OP_MATMUL_F16 || E.n_args < 7 || pos != 0 || E.args[3] != 1u || E.args[4] != P ||
        E.args[5] != hd || E.args[6] != ((H << 16) | 4u) || !is_temp_ref(E.args[2]) || !is_temp_ref(E.args[1]))
        return false;
    // the v face: the same gather, or a second KV_GATHER of the same state and layout
    const uint32_t gv = writer_before(b, j, E.args[1], m.lo);
    if (gv == kNone) return false;
    const wt_op& V = b->ops[gv];
    if (V.opcode != OP_KV_GATHER_F16 || V.n_args < 7 || !V.args[2] || !same_temp(V.args[2], E.args[1]) ||
        V.args[0] != st || V.args[3] != n_kv || V.args[4] != H || V.args[5] != KVH || V.args[6] != hd)
        return false;
    if (!m.add(gv) || !m.edge(j, E.args[1], gv) || !m.add(j) || !m.edge(j, prev, at)) return false;
    c.v = E.args[1];
    c.v_at = j;
    c.out = E.args[2];
    return m.finish() && c.last == j;
}

// The attention chains of a blob, in op order (each op a member of at most one chain).
std::vector<AttnChain> scan_chains(const wt_blob* b, std::vector<int32_t>& member_of) {
    std::vector<AttnChain> chains;
    member_of.assign(b->n_ops, -1);
    for (uint32_t i = 0; i < b->n_ops; ++i) {
        Matcher m{b, member_of, AttnChain{}};
        if (!match_attn_chain(m, i)) {
            Matcher d{b, member_of, AttnChain{}};
            if (!match_decode_chain(d, i)) continue;
            m.c = d.c;
        }
        for (uint32_t k = 0; k < m.c.n_mem; ++k) member_of[m.c.mem[k]] = (int32_t)chains.size();
        chains.push_back(m.c);
    }
    return chains;
}

// The plan of a blob (created, with its chains detected, on first sight of the blob as
// parsed; a new plan drops the captured graphs, which may hold the blob's old form).
FusionPlan* fusion_plan(const wt_blob* b) {
    const uint64_t ep = g_parse_epoch.load(std::memory_order_relaxed);
    for (FusionPlan& p : g_plans)
        if (p.b == b && p.n_ops == b->n_ops && p.parse_epoch == ep) {
            p.used = ++g_plan_tick;
            return &p;
        }
    for (auto it = g_plans.begin(); it != g_plans.end();)   // stale plans of this blob
        it = it->b == b ? g_plans.erase(it) : it + 1;
    if (g_plans.size() >= kMaxPlans)
        g_plans.erase(std::min_element(g_plans.begin(), g_plans.end(),
                                       [](const FusionPlan& x, const FusionPlan& y) { return x.used < y.used; }));
    drop_graphs();
    FusionPlan p;
    p.b = b; p.n_ops = b->n_ops; p.parse_epoch = ep; p.used = ++g_plan_tick;
    p.chains = scan_chains(b, p.member_of);
    p.blocked.assign(p.chains.size(), 0);
    p.keep.assign(p.chains.size(), 0);
    p.aliased.assign(p.chains.size(), 0);
    g.chains_found += p.chains.size();
    g_plans.push_back(std::move(p));
    return &g_plans.back();
}

int member_index(const AttnChain& c, uint32_t op) {
    for (uint32_t k = 0; k < c.n_mem; ++k)
        if (c.mem[k] == op) return (int)k;
    return -1;
}

bool ranges_overlap(uintptr_t a, uint64_t na, uintptr_t b, uint64_t nb) {
    return na && nb && a < b + nb && b < a + na;
}

// Decides, from the observed run's log, which chains may run fused and which of their
// members still run then (the rules above fusion's matchers).
void fusion_validate(FusionPlan& p) {
    for (size_t ci = 0; ci < p.chains.size(); ++ci) {
        const AttnChain& c = p.chains[ci];
        bool blocked = false;
        uint32_t keep = 0;
        // 1. each member read what the matcher expects
        for (const ObsRead& r : g_obs.reads) {
            if (r.op < c.head || r.op > c.last || member_index(c, r.op) < 0) continue;
            const ChainEdge* e = nullptr;
            for (uint32_t k = 0; k < c.n_edge && !e; ++k)
                if (c.edge[k].op == r.op && c.edge[k].id == r.id) e = &c.edge[k];
            if (!e) { blocked = true; break; }
            if (e->from != kNone ? r.writer != e->from : (r.writer != kNone && member_index(c, r.writer) >= 0)) {
                blocked = true;
                break;
            }
        }
        // 2. members' outputs read elsewhere (the last member's output excepted)
        for (const ObsRead& r : g_obs.reads) {
            if (blocked) break;
            if (r.writer == kNone || r.writer == c.last) continue;
            const int mw = member_index(c, r.writer);
            if (mw < 0 || member_index(c, r.op) >= 0) continue;
            const uint16_t oc = p.b->ops[r.writer].opcode;
            if (oc == OP_BROADCAST_F16 || oc == OP_TRANSPOSE_GEN_F16 || oc == OP_KV_GATHER_F16) keep |= 1u << mw;
            else blocked = true;
        }
        // 3. inputs' bytes intact from their read to the last member, and the output's
        //    overlap with them (then the kernel writes scratch)
        bool aliased = false;
        for (uint32_t k = 0; k < c.n_edge && !blocked; ++k) {
            const ChainEdge& e = c.edge[k];
            if (e.from != kNone) continue;
            const ObsRead* r = nullptr;
            for (const ObsRead& x : g_obs.reads)
                if (x.op == e.op && x.id == e.id) { r = &x; break; }
            if (!r || !r->p) { blocked = true; break; }
            for (const ObsWrite& w : g_obs.writes) {
                if (w.op <= e.op || w.op > c.last || !ranges_overlap(w.p, w.n, r->p, r->n)) continue;
                if (w.op == c.last) { aliased = true; continue; }
                const int mw = member_index(c, w.op);
                if (mw >= 0 && !((keep >> mw) & 1u)) continue;   // a skipped member writes nothing when fused
                blocked = true;
                break;
            }
        }
        p.blocked[ci] = blocked;
        p.keep[ci] = keep;
        p.aliased[ci] = aliased;
    }
}

// The fused kernel's output: the chain's output temp, or, when its bytes overlap an
// input's, engine scratch copied to it after the kernel.
struct FusedOut { __half* dst = nullptr; __half* kernel = nullptr; uint64_t bytes = 0; };
int fused_out(const AttnChain& c, uint64_t bytes, const std::pair<const uint8_t*, uint64_t>* in, int n_in,
              FusedOut& o, char* err, size_t errn) {
    if (bytes > 0xFFFFFFFFull) return ERR("fused attention output too large");
    o.dst = reinterpret_cast<__half*>(temp_get(c.out, (uint32_t)bytes));
    if (!o.dst) return ERR("fused attention output alloc");
    o.kernel = o.dst;
    o.bytes = bytes;
    bool alias = false;
    for (int k = 0; k < n_in; ++k)
        alias = alias || ranges_overlap(reinterpret_cast<uintptr_t>(o.dst), bytes,
                                        reinterpret_cast<uintptr_t>(in[k].first), in[k].second);
    if (!alias) return 0;
    if (g.fuse_scratch_cap < bytes) {
        if (g.fuse_scratch) dev_free(g.fuse_scratch);
        g.fuse_scratch = nullptr;
        g.fuse_scratch_cap = 0;
        if (dev_malloc(reinterpret_cast<void**>(&g.fuse_scratch), bytes) != hipSuccess)
            return ERR("fused attention scratch alloc");
        g.fuse_scratch_cap = bytes;
    }
    o.kernel = reinterpret_cast<__half*>(g.fuse_scratch);
    g.fused_alias_runs++;
    return 0;
}

int fused_out_done(const FusedOut& o, char* err, size_t errn) {
    if (o.kernel == o.dst) return 0;
    if (copy_d2d(o.dst, o.kernel, o.bytes) != hipSuccess) return ERR("fused attention output copy");
    return 0;
}

int run_fused_decode(const wt_blob* b, const AttnChain& c, const FusedIn& in, char* err, size_t errn) {
    const uint32_t H = c.H, KVH = c.KVH, hd = 128, P = c.P;
    State* s = state_kv(c.state, KVH * hd, err, errn);
    if (!s) return -1;
    const uint32_t si = c.state & 0x1FFFu;
    const bool autopos = c.n_kv == WT_KV_POS_AUTO;
    uint32_t n_kv = c.n_kv;
    if (autopos) {   // the gather's checks (oplist_exec.c:2199-2205)
        if (s->count == 0 || s->count > s->nslots)
            return ERR("kv gather state %u count=%u bad (append first?)", si, s->count);
        if (s->nslots != P) return ERR("fused decode attention: state %u has %u slots, chain %u", si, s->nslots, P);
        n_kv = s->count;
    } else if (n_kv > s->nslots) {
        return ERR("kv gather n_kv %u > nslots %u", n_kv, s->nslots);
    }
    if (kv_check(*s, n_kv, err, errn)) return -1;
    const __half* q = reinterpret_cast<const __half*>(in.q);
    const __half* mask = c.mask != kNone ? reinterpret_cast<const __half*>(in.mask) : nullptr;
    if (!q || (c.mask != kNone && !mask)) return ERR("fused decode attention ref fail");
    const uint64_t qn = (uint64_t)H * hd * 2u, mn = c.mask != kNone ? (uint64_t)(c.mask_shared ? 1u : H) * P * 2u : 0;
    const size_t qb = ref_bytes(b, c.q), mb = c.mask != kNone ? ref_bytes(b, c.mask) : 0;
    if ((qb && qb < qn) || (mb && mb < mn)) return ERR("fused decode attention operand too small");
    const std::pair<const uint8_t*, uint64_t> ins[2] = {{in.q, qn}, {in.mask, mn}};
    if (attn_workspace(attn_decode_work_floats(autopos ? s->nslots : n_kv, H, hd), err, errn)) return -1;
    FusedOut o;
    if (fused_out(c, (uint64_t)H * hd * 2u, ins, 2, o, err, errn)) return -1;
    CHECK_LAUNCH(launch_attn_decode(q, s->dev, s->slot_bytes, s->nslots, o.kernel, autopos ? 0u : n_kv,
                                    autopos ? g.counters_dev + si : nullptr, H, KVH, hd, c.scale, g.attn_work,
                                    g.attn_work_floats, g.stream, mask, mask ? P : 0u, n_kv, c.mask_shared));
    return fused_out_done(o, err, errn);
}

int run_fused_attn(const wt_blob* b, const AttnChain& c, const FusedIn& in, char* err, size_t errn) {
    if (c.decode) return run_fused_decode(b, c, in, err, errn);
    const uint32_t S = c.S, H = c.H;
    const uint64_t bytes = (uint64_t)S * H * 128u * 2u;
    const __half* q = reinterpret_cast<const __half*>(in.q);
    const __half* k = reinterpret_cast<const __half*>(in.k);
    const __half* v = reinterpret_cast<const __half*>(in.v);
    if (!q || !k || !v) return ERR("fused attention ref fail");
    const size_t qb = ref_bytes(b, c.q), kb = ref_bytes(b, c.k), vb = ref_bytes(b, c.v);
    if ((qb && qb < bytes) || (kb && kb < bytes) || (vb && vb < bytes)) return ERR("fused attention operand too small");
    const std::pair<const uint8_t*, uint64_t> ins[3] = {{in.q, bytes}, {in.k, bytes}, {in.v, bytes}};
    FusedOut o;
    if (fused_out(c, bytes, ins, 3, o, err, errn)) return -1;
    CHECK_LAUNCH(launch_attn_prefill_hs(q, 128, S * 128, k, v, 128, S * 128, o.kernel, 128, S * 128, S, H, H, 128,
                                        c.scale, c.causal, g.stream));
    return fused_out_done(o, err, errn);
}

// Marks the outputs of a skipped member as not materialized.
void unmat_member(const wt_op& o, const AttnChain& c) {
    if (g_unmat.empty()) g_unmat.assign(kMaxTemps, 0);
    uint32_t outs[2] = {kNone, kNone};
    switch (o.opcode) {
    case OP_MATMUL_F16: case OP_BINARY_F16: case OP_ADD_F16: outs[0] = o.args[2]; break;
    case OP_BROADCAST_F16: case OP_TRANSPOSE_GEN_F16: case OP_SOFTMAX_F16: outs[0] = o.args[1]; break;
    case OP_KV_GATHER_F16: outs[0] = o.args[1] ? o.args[1] : kNone; outs[1] = o.args[2] ? o.args[2] : kNone; break;
    default: break;
    }
    for (uint32_t t : outs)
        if (t != kNone && is_temp_ref(t) && !same_temp(t, c.out)) g_unmat[t & 0x3FFFu] = 1;
}

// Fused-run handling of op i of a chain: returns 1 when the op is done (skipped, or the
// chain's kernel launched at its last member: *rc holds the status), 0 to run it.
int fused_member(const wt_blob* b, uint32_t i, int* rc, char* err, size_t errn) {
    const int32_t ci = g_fplan->member_of[i];
    if (ci < 0) return 0;
    const AttnChain& c = g_fplan->chains[ci];
    if (i == c.head) {
        g_active[ci] = !g_fplan->blocked[ci] && c.last < g_run_end;
        g_fin[ci] = FusedIn{};
    }
    if (!g_active[ci]) return 0;
    FusedIn& in = g_fin[ci];
    if (i == c.q_at) in.q = ref_ptr(b, c.q);
    if (i == c.k_at && !c.decode) in.k = ref_ptr(b, c.k);
    if (i == c.v_at && !c.decode) in.v = ref_ptr(b, c.v);
    if (c.mask != kNone && i == c.mask_at) in.mask = ref_ptr(b, c.mask);
    if (i == c.last) {
        *rc = run_fused_attn(b, c, in, err, errn);
        g.fused_runs++;
        g.stats.ops++;
        return 1;
    }
    const int mk = member_index(c, i);
    if (mk >= 0 && ((g_fplan->keep[ci] >> mk) & 1u)) return 0;
    unmat_member(b->ops[i], c);
    *rc = 0;
    return 1;
}

// One op through its handler; returns the handler's status.
int run_op(const wt_blob* b, uint32_t i, uint32_t ii, uint32_t* engine_m, char* err, size_t errn) {
    const wt_op* op = &b->ops[i];
    if (g_prenorm.op != op) g_prenorm = PreNorm{};   // only ever for the very next op
    if (g_rope_pre != op) g_rope_pre = nullptr;
    if (g_attn_pre != op) g_attn_pre = nullptr;
    if (g_merge_pending.op && g_merge_pending.op != op && g_attn_pre != op && flush_merge_pending(err, errn))
        return -1;
    if (g_fplan) {
        int frc = 0;
        if (fused_member(b, i, &frc, err, errn)) return frc;
    }
    if (g_obs.on) g_obs.op = i;
    Ctx cx{b, op, engine_m, err, errn};
    const int rc = op->opcode < 64 ? kTable.fn[op->opcode](cx) : op_unsupported(cx);
    if (g.trace)
        std::fprintf(stderr, "[gehtp] op%u code=%u a=%u,%u,%u,%u rc=%d pool=%u%s\n", ii, (unsigned)op->opcode,
                     op->args[0], op->args[1], op->args[2], op->args[3], rc, g.pool_used,
                     g.replay ? " (graph)" : "");
    g.stats.ops++;
    return rc;
}

// Waits for a run's work. When wt_exec_run_io asked for an output that fits the pinned
// output buffer, its device-to-host copy is queued first, so the one wait covers both
// (wt_exec_run_steps queues its own copies).
hipError_t end_run_sync() {
    g.out_pending = 0;
    const uint32_t t = g_run_out_temp;
    if (!g_defer_wait && t < kMaxTemps && g.temps[t] && g.last_bytes[t] && g.last_bytes[t] <= g.out_cap &&
        hipMemcpyAsync(g.out_host, g.temps[t], g.last_bytes[t], hipMemcpyDeviceToHost, g.stream) == hipSuccess)
        g.out_pending = g.last_bytes[t];
    return hipStreamSynchronize(g.stream);
}

int replay_graph(RunGraph& r, const wt_blob* b, uint32_t first, uint32_t count, uint32_t* engine_m, char* err,
                 size_t errn) {
    const hipError_t le = hipGraphLaunch(r.exec, g.stream);
    if (le != hipSuccess) return ERR("graph launch failed: %s", hipGetErrorString(le));
    r.used = ++g_use_tick;
    const uint64_t ep0 = g.epoch;
    g.variant = false;
    g.replay = true;
    int fail = 0;
    for (uint32_t ii = 0; ii < count && !fail; ++ii)
        if (run_op(b, first + ii, ii, engine_m, err, errn)) fail = (int)(first + ii) + 1;
    if (flush_merge_pending(err, errn) && !fail) fail = (int)(first + count);
    g.replay = false;
    const hipError_t e = g_defer_wait && !fail ? hipSuccess : end_run_sync();
    if (e != hipSuccess) return ERR("device error: %s", hipGetErrorString(e));
    if (fail || g.epoch != ep0 || g.variant) {
        if (g_defer_wait) hipStreamSynchronize(g.stream);
        // The preflight makes this unreachable for the ops this engine implements; if
        // the host pass ever disagrees with the capture, stop using graphs.
        g.graphs_broken = true;
        drop_graphs();
        if (fail) return fail;
        return ERR("graph replay diverged from its capture");
    }
    g.n_replays++;
    return 0;
}

}  // namespace

extern "C" {

int wt_exec_run_range(const struct wt_blob* b, uint32_t first, uint32_t count, uint32_t* engine_m,
                      int64_t* op_us, char* err, size_t errn) {
    g_prenorm = PreNorm{};
    g_rope_pre = nullptr;
    g_attn_pre = nullptr;
    g_merge_pending = MergePending{};
    char dummy_err[8];
    if (!err || !errn) { err = dummy_err; errn = sizeof dummy_err; }
    uint32_t dummy_m = 0;
    if (!engine_m) engine_m = &dummy_m;
    *engine_m = g.w4_ready ? g.w4_m : 0;   // oplist_exec.c:2503
    if (!b) return ERR("null blob");
    if ((uint64_t)first + count > b->n_ops) return ERR("range oob");
    if (ensure_ready(err, errn)) return -1;
    if (ensure_weights(b, err, errn)) return -1;
    if (load_tempoff(b, err, errn)) return -1;
    if (load_states(b, err, errn)) return -1;

    const bool timed = op_us || (g.ts && g.ts_cap);
    if (timed && g.events.size() < 2 * (size_t)count + 1) {
        const size_t have = g.events.size();
        g.events.resize(2 * (size_t)count + 1);
        for (size_t i = have; i < g.events.size(); ++i)
            if (hipEventCreate(&g.events[i]) != hipSuccess) return ERR("event create failed");
    }
    const bool sync_each = std::getenv("GEHTP_SYNC_EACH_OP") != nullptr;
    const char* hk = hook_spec();
    const bool hooked = hk && hk[0];
    // Attention-chain fusion: a blob's first full run is observed (ops run one by one);
    // later runs launch the chains that qualified as single fused kernels. Per-op tensor
    // hooks see every op's output, so they run without fusion.
    g_fplan = nullptr;
    g_obs_plan = nullptr;
    g_run_end = first + count;
    bool observing = false;
    if (fusion_on() && !hooked) {
        FusionPlan* fp = fusion_plan(b);
        if (fp->observed) {
            g_fplan = fp;
            g_active.assign(fp->chains.size(), 0);
            g_fin.assign(fp->chains.size(), FusedIn{});
        } else if (!fp->chains.empty() && first == 0 && count == b->n_ops) {
            observing = true;
            g_obs_plan = fp;
            g_obs.writer.assign(kMaxTemps, kNone);
            g_obs.reads.clear();
            g_obs.writes.clear();
            g_obs.op = 0;
            g_obs.on = true;
        }
    }
    // The observed run neither replays nor qualifies a graph: the next run differs from it.
    const bool can_graph = count && !timed && !sync_each && !hooked && graphs_on() && !observing;
    static HostIn hin;   // one engine per process; runs are not reentrant
    if (can_graph) {
        host_in(hin);
        RunGraph* r = find_graph(b, first, count, hin);
        if (r && preflight(*r)) return replay_graph(*r, b, first, count, engine_m, err, errn);
    }
    bool capture = can_graph && g_stable_ok && g_stable.same(b, first, count, hin);
    uint32_t counts0[WT_MAX_STATES];
    for (uint32_t i = 0; i < g.n_states; ++i) counts0[i] = g.st[i].count;
    const uint64_t ep0 = g.epoch;
    g.variant = false;
    if (capture && hipStreamBeginCapture(g.stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
        (void)hipGetLastError();
        capture = false;
    }

    if (timed && hipEventRecord(g.events[2 * (size_t)count], g.stream) != hipSuccess)
        return ERR("event record failed");
    int fail = 0;
    for (uint32_t ii = 0; ii < count && !fail; ++ii) {
        const uint32_t i = first + ii;
        if (timed) hipEventRecord(g.events[2 * ii], g.stream);
        int rc = run_op(b, i, ii, engine_m, err, errn);
        if (timed) hipEventRecord(g.events[2 * ii + 1], g.stream);
        if (rc == 0 && sync_each) {
            const hipError_t e = hipStreamSynchronize(g.stream);
            if (e != hipSuccess) { std::snprintf(err, errn, "op %u: %s", i, hipGetErrorString(e)); rc = -1; }
        }
        if (rc == 0) hook_dump(ii);
        if (rc) fail = (int)i + 1;
    }
    // a merge pass still left over (its GEMV op failed or lies past the run) runs alone
    if (flush_merge_pending(err, errn) && !fail) fail = (int)(first + count);
    if (observing) {
        g_obs.op = b->n_ops;   // run_io's output copy reads after every op
        if (g_run_out_temp != kNone) obs_read(g_run_out_temp);
        g_obs.on = false;
        if (!fail) {
            fusion_validate(*g_obs_plan);
            g_obs_plan->observed = true;
        }
        g_obs.reads.clear();
        g_obs.writes.clear();
        g_obs_plan = nullptr;
    }
    if (capture) {
        // The captured work of this run (all of it, or the ops before a failing one)
        // is launched once from the graph; it is kept for replay only if this run
        // matched the direct run that qualified it.
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipError_t ce = hipStreamEndCapture(g.stream, &graph);
        if (ce == hipSuccess) ce = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (graph) hipGraphDestroy(graph);
        if (ce == hipSuccess) ce = hipGraphLaunch(exec, g.stream);
        if (ce != hipSuccess) {
            g.graphs_broken = true;
            hipStreamSynchronize(g.stream);
            if (exec) hipGraphExecDestroy(exec);
            drop_graphs();
            return ERR("graph capture of ops %u..%u failed: %s", first, first + count - 1, hipGetErrorString(ce));
        }
        const bool keep = !fail && !g.variant && g.epoch == ep0;
        if (keep) {
            keep_graph(b, first, count, exec, counts0, hin);
            g.n_captures++;
            g_stable_ok = false;
        } else {
            hipStreamSynchronize(g.stream);
            hipGraphExecDestroy(exec);
        }
    } else if (can_graph && !fail) {
        g_stable_ok = !g.variant && g.epoch == ep0;
        if (g_stable_ok) g_stable.set(b, first, count, hin);
    }
    if (fail) {
        hipStreamSynchronize(g.stream);
        return fail;
    }
    const hipError_t e = end_run_sync();
    if (e != hipSuccess) return ERR("device error: %s", hipGetErrorString(e));
    if (timed) {
        for (uint32_t ii = 0; ii < count; ++ii) {
            float ms = 0.0f, st_ms = 0.0f;
            hipEventElapsedTime(&ms, g.events[2 * ii], g.events[2 * ii + 1]);
            hipEventElapsedTime(&st_ms, g.events[2 * (size_t)count], g.events[2 * ii]);
            if (op_us) op_us[ii] = (int64_t)std::llround(ms * 1000.0);
            const uint32_t i = first + ii;
            if (g.ts && i < g.ts_cap) {
                g.ts[i].start_us = (uint32_t)std::llround(st_ms * 1000.0);
                g.ts[i].dur_us = (uint32_t)std::llround(ms * 1000.0);
                g.ts[i].dma_us = 0;
                g.ts[i].dma_bytes = 0;
                g.ts[i].engine = WT_ENG_HMX;
            }
        }
    }
    return 0;
}

int wt_exec_run(const struct wt_blob* b, uint32_t* engine_m, int64_t* op_us, char* err, size_t errn) {
    g.stats = wt_exec_stats{};
    return wt_exec_run_range(b, 0, b ? b->n_ops : 0, engine_m, op_us, err, errn);
}

}  // extern "C"

namespace {

// Bytes of the blob's EXT_IN input slot (0 if it has none).
size_t input_bytes(const wt_blob* b) {
    size_t need = 0;
    for (uint32_t i = 0; i < b->n_slots; ++i)
        if (b->slots[i].addr == WT_SLOT_EXT_IN) need = std::max<size_t>(need, b->slots[i].len);
    return need;
}

// Host input of `need` bytes staged through pinned memory into in_dev (the previous run
// drained the stream, so the staging buffer is free); the runs that follow read in_dev.
int stage_input(const void* in_ptr, size_t need, char* err, size_t errn) {
    if (ensure_ready(err, errn)) return -1;
    if (!need) return 0;
    if (need > g.in_cap) {
        if (g.in_dev) dev_free(g.in_dev);
        if (g.in_host) hipHostFree(g.in_host);
        g.in_dev = g.in_host = nullptr;
        g.in_cap = 0;
        if (dev_malloc(reinterpret_cast<void**>(&g.in_dev), need) != hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&g.in_host), need, hipHostMallocDefault) != hipSuccess)
            return ERR("input buffer alloc");
        g.in_cap = need;
    }
    std::memcpy(g.in_host, in_ptr, need);
    if (hipMemcpyAsync(g.in_dev, g.in_host, need, hipMemcpyHostToDevice, g.stream) != hipSuccess)
        return ERR("input upload failed");
    g.in_active = true;
    g.in_src = g.in_dev;
    return 0;
}

}  // namespace

extern "C" {

int wt_exec_run_io(const struct wt_blob* b, const void* in_ptr, void* out_ptr, uint32_t out_temp,
                   uint32_t* engine_m, int64_t* op_us, char* err, size_t errn) {
    char dummy_err[8];
    if (!err || !errn) { err = dummy_err; errn = sizeof dummy_err; }
    if (!b) return ERR("null blob");
    g.in_active = false;
    g.in_src = nullptr;
    const size_t need = input_bytes(b);
    if (!in_ptr && g.in_bound && need) {
        // Device-resident input bound by wt_exec_set_input_device: no host staging.
        if (need > g.in_bound_bytes)
            return ERR("bound device input holds %zu bytes, the blob's input slot needs %zu", g.in_bound_bytes, need);
        g.in_active = true;
        g.in_src = g.in_bound;
    }
    if (in_ptr && stage_input(in_ptr, need, err, errn)) return -1;
    g_run_out_temp = out_ptr ? out_temp : kNone;
    g.out_pending = 0;
    int rc = wt_exec_run(b, engine_m, op_us, err, errn);
    g_run_out_temp = kNone;
    if (rc == 0 && out_ptr && out_temp < kMaxTemps && g.temps[out_temp]) {
        const size_t n = g.last_bytes[out_temp];
        if (n && g.out_pending == n) {
            std::memcpy(out_ptr, g.out_host, n);   // copied during the run's final wait
        } else {
            if (hipMemcpy(out_ptr, g.temps[out_temp], n, hipMemcpyDeviceToHost) != hipSuccess)
                rc = ERR("output copy failed");
            // Size the pinned output buffer for the next run (outputs up to 4 MiB).
            constexpr size_t kOutPinnedMax = 4u << 20;
            if (rc == 0 && n > g.out_cap && n <= kOutPinnedMax) {
                if (g.out_host) hipHostFree(g.out_host);
                g.out_host = nullptr;
                g.out_cap = 0;
                if (hipHostMalloc(reinterpret_cast<void**>(&g.out_host), n, hipHostMallocDefault) == hipSuccess)
                    g.out_cap = n;
            }
        }
    }
    g.out_pending = 0;
    g.in_active = false;
    g.in_src = nullptr;
    return rc;
}

int wt_exec_run_steps(const struct wt_blob* b, uint32_t steps, const void* in_ptr, void* out_ptr, uint32_t out_temp,
                      uint32_t* engine_m, char* err, size_t errn) {
    char dummy_err[8];
    if (!err || !errn) { err = dummy_err; errn = sizeof dummy_err; }
    if (!b || !in_ptr || !out_ptr) return ERR("run_steps: null blob, input or output");
    if (!steps) return 0;
    if (out_temp >= kMaxTemps) return ERR("run_steps: out_temp %u out of range", out_temp);
    const size_t need = input_bytes(b);
    if (!need || need > 4096) return ERR("run_steps: the blob's input slot holds %zu bytes (1..4096)", need);
    constexpr size_t kStepsOutMax = 64u << 20;   // pinned bytes for the steps' outputs
    if ((size_t)steps * need > kStepsOutMax)
        return ERR("run_steps: %u steps x %zu bytes exceed the %zu-byte output limit", steps, need, kStepsOutMax);
    g.in_active = false;
    g.in_src = nullptr;
    if (stage_input(in_ptr, need, err, errn)) return -1;
    // One pinned row per step for the outputs, read back after the final wait.
    if ((size_t)steps * need > g.out_cap) {
        if (g.out_host) hipHostFree(g.out_host);
        g.out_host = nullptr;
        g.out_cap = 0;
        if (hipHostMalloc(reinterpret_cast<void**>(&g.out_host), (size_t)steps * need, hipHostMallocDefault) !=
            hipSuccess)
            return ERR("run_steps: output buffer alloc");
        g.out_cap = (size_t)steps * need;
    }
    int rc = 0;
    for (uint32_t s = 0; s < steps && rc == 0; ++s) {
        g.in_active = true;
        g.in_src = g.in_dev;
        g_run_out_temp = out_temp;
        g_defer_wait = true;
        rc = wt_exec_run(b, engine_m, nullptr, err, errn);
        g_defer_wait = false;
        g_run_out_temp = kNone;
        if (rc) break;
        if (!g.temps[out_temp] || g.last_bytes[out_temp] != need) {
            hipStreamSynchronize(g.stream);
            rc = ERR("run_steps: output temp %u holds %u bytes, the input slot %zu", out_temp,
                     g.last_bytes[out_temp], need);
            break;
        }
        // This step's output is the next step's input, and one row of the result.
        if (hipMemcpyAsync(g.in_dev, g.temps[out_temp], need, hipMemcpyDeviceToDevice, g.stream) != hipSuccess ||
            hipMemcpyAsync(g.out_host + (size_t)s * need, g.temps[out_temp], need, hipMemcpyDeviceToHost,
                           g.stream) != hipSuccess) {
            hipStreamSynchronize(g.stream);
            rc = ERR("run_steps: output copy failed");
        }
    }
    const hipError_t e = hipStreamSynchronize(g.stream);
    if (rc == 0 && e != hipSuccess) rc = ERR("device error: %s", hipGetErrorString(e));
    if (rc == 0) std::memcpy(out_ptr, g.out_host, (size_t)steps * need);
    g.in_active = false;
    g.in_src = nullptr;
    return rc;
}

void wt_exec_set_input_device(const void* dev_ptr, size_t bytes) {
    uint8_t* p = dev_ptr ? static_cast<uint8_t*>(const_cast<void*>(dev_ptr)) : nullptr;
    if (p != g.in_bound || (p ? bytes : 0) != g.in_bound_bytes) ++g.epoch;
    g.in_bound = p;
    g.in_bound_bytes = p ? bytes : 0;
}

uint8_t* wt_exec_temp(uint32_t id) {
    if (id >= kMaxTemps || !g.temps[id]) return nullptr;
    if (!g_unmat.empty() && g_unmat[id]) return nullptr;   // intermediate of a fused chain
    std::vector<uint8_t>& m = g.mirror[id];
    m.resize(std::max<uint32_t>(g.temp_bytes[id], 1));
    if (g.stream) hipStreamSynchronize(g.stream);
    if (hipMemcpy(m.data(), g.temps[id], g.temp_bytes[id], hipMemcpyDeviceToHost) != hipSuccess) return nullptr;
    return m.data();
}

uint32_t wt_exec_temp_bytes(uint32_t id) { return id < kMaxTemps ? g.temp_bytes[id] : 0; }
uint32_t wt_exec_temp_last_bytes(uint32_t id) { return id < kMaxTemps ? g.last_bytes[id] : 0; }

void wt_exec_shutdown(void) {
    if (g.stream) hipStreamSynchronize(g.stream);
    g.stats = wt_exec_stats{};
    drop_graphs();
    g_plans.clear();
    g_fplan = nullptr;
    g.in_bound = nullptr;   // the caller's buffer may not outlive the engine's use of it
    g.in_bound_bytes = 0;
    if (g.pool && g.pool_owned) dev_free(g.pool);
    for (void* p : g.retired_pools) dev_free(p);
    g.retired_pools.clear();
    g.pool = nullptr;
    g.pool_cap = g.pool_used = 0;
    g.pool_owned = false;
    g.static_offsets = nullptr;
    g.plan_from_blob = false;
    g.plan_payload.clear();
    if (g.vtcm_pool) dev_free(g.vtcm_pool);
    g.vtcm_pool = nullptr;
    g.vtcm_pool_size = 0;
    std::fill(std::begin(g.static_off_arr), std::end(g.static_off_arr), kNone);
    std::fill(std::begin(g.vtcm_off_arr), std::end(g.vtcm_off_arr), kNone);
    for (uint32_t i = 0; i < kMaxTemps; ++i) {
        g.temps[i] = nullptr;
        g.temp_bytes[i] = 0;
        g.last_bytes[i] = 0;
        std::vector<uint8_t>().swap(g.mirror[i]);
    }
    if (g.attn_work) dev_free(g.attn_work);
    g.attn_work = nullptr;
    g.attn_work_floats = 0;
    if (g.fuse_scratch) dev_free(g.fuse_scratch);
    g.fuse_scratch = nullptr;
    g.fuse_scratch_cap = 0;
    if (g.norm_buf) dev_free(g.norm_buf);
    g.norm_buf = nullptr;
    g.norm_cap = 0;
    if (g.split_buf) dev_free(g.split_buf);
    g.split_buf = nullptr;
    g.split_cap = 0;
    if (g.rope_buf) dev_free(g.rope_buf);
    g.rope_buf = nullptr;
    g.rope_cap = 0;
    if (g.w4_out) dev_free(g.w4_out);
    g.w4_out = nullptr;
    g.w4_out_cap = 0;
    g.w4_ready = false;
    g.w4_m = g.w4_k = g.w4_n = 0;
    g.w4_act = nullptr;
    g.w4_wt = g.w4_bias = nullptr;
    // Weights stay resident (keyed by content); states persist until state_reset.
}

void wt_exec_state_reset(void) {
    for (uint32_t i = 0; i < g.n_states; ++i) {
        State& s = g.st[i];
        if (s.dev) launch_fill_zero(s.dev, s.bytes, g.stream);   // ordered before the next run's kernels
        s.count = 0;
        if (s.kv_ready) std::fill(s.posmap.begin(), s.posmap.end(), kNone);
        s.valid_prefix = 0;
    }
    if (g.counters_dev) launch_fill_zero(g.counters_dev, 2 * WT_MAX_STATES * sizeof(uint32_t), g.stream);
}

void wt_exec_pool_init(uint8_t* base, uint32_t total_cap, uint32_t static_cap, const uint32_t* offsets) {
    ++g.epoch;
    if (g.plan_from_blob) drop_blob_plan();   // the caller's plan replaces a blob's
    if (base) {
        if (g.pool && g.pool_owned) g.retired_pools.push_back(g.pool);
        g.pool = base;
        g.pool_cap = total_cap;
        g.pool_used = static_cap ? static_cap : total_cap;
        g.pool_owned = false;
    }
    g.static_offsets = offsets;
}

void wt_exec_get_stats(struct wt_exec_stats* st) {
    if (st) *st = g.stats;
}

void wt_exec_set_ext_weights(const void* wgt_ptr) {
    if (wgt_ptr != g.ext_host) ++g.epoch;
    g.ext_host = static_cast<const uint8_t*>(wgt_ptr);
}

void wt_exec_set_ts(struct wt_op_ts* buf, uint32_t cap) {
    g.ts = buf;
    g.ts_cap = buf ? cap : 0;
}

void wt_exec_set_trace(int on) { g.trace = on != 0; }

int wt_exec_set_graphs(int on) {
    const int prev = graphs_on() ? 1 : 0;
    if (!on) drop_graphs();
    g.graphs = on ? 1 : 0;
    if (on) g.graphs_broken = false;
    return prev;
}

void wt_exec_graph_stats(uint32_t* captures, uint32_t* replays) {
    if (captures) *captures = g.n_captures;
    if (replays) *replays = g.n_replays;
}

int wt_exec_set_fusion(int on) {
    const int prev = fusion_on() ? 1 : 0;
    if ((on ? 1 : 0) != prev) {
        drop_graphs();   // graphs hold whichever form the runs that made them used
        g_plans.clear();
    }
    g.fusion = on ? 1 : 0;
    return prev;
}

void wt_exec_fusion_stats(uint64_t* chains_found, uint64_t* fused_runs) {
    if (chains_found) *chains_found = g.chains_found;
    if (fused_runs) *fused_runs = g.fused_runs;
}

void wt_exec_fusion_detail(const struct wt_blob* b, uint32_t* chains, uint32_t* blocked, uint32_t* aliased,
                           uint64_t* alias_runs) {
    uint32_t n = 0, nb = 0, na = 0;
    bool planned = false;
    const uint64_t ep = g_parse_epoch.load(std::memory_order_relaxed);
    for (const FusionPlan& p : g_plans) {
        if (!b || p.b != b || p.n_ops != b->n_ops || p.parse_epoch != ep) continue;
        planned = true;
        n = (uint32_t)p.chains.size();
        for (size_t c = 0; c < p.chains.size(); ++c) {
            nb += p.observed && p.blocked[c];
            na += p.observed && p.aliased[c];
        }
    }
    if (!planned && b && b->n_ops) {   // not run yet: the chains the matchers find (no device work)
        std::vector<int32_t> member_of;
        n = (uint32_t)scan_chains(b, member_of).size();
    }
    if (chains) *chains = n;
    if (blocked) *blocked = nb;
    if (aliased) *aliased = na;
    if (alias_runs) *alias_runs = g.fused_alias_runs;
}

uint64_t wt_exec_qkv_rope_fused(void) { return g.qkv_rope_fused; }
uint64_t wt_exec_qkv_attn_fused(void) { return g.qkv_attn_fused; }
uint64_t wt_exec_merge_oproj_fused(void) { return g.merge_oproj_fused; }

void wt_exec_set_hook(const char* spec) { g.hook = spec; }

}  // extern "C"
