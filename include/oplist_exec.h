/* oplist_exec.h — runlist engine ABI (HIP/gfx950 implementation).
 *
 * Drop-in for GEHTP's engine header (reference: kernels/include/oplist_exec.h).
 * Same functions, same struct layouts, same return conventions:
 *   run*  -> 0 on success, the 1-based index of the failing op, or -1 on a
 *            setup failure; a human-readable reason is written to err.
 *
 * Differences a caller can observe, all forced by the device being a GPU:
 *   - Every op runs as HIP kernels on one stream of the current device; the run
 *     functions return after that stream has drained.
 *   - wt_exec_temp() returns a host mirror of the temp's device buffer, copied
 *     back at the time of the call (valid until the next run or shutdown).
 *   - An opcode without a gfx950 kernel fails the run with "no HIP kernel"; there
 *     is no silent CPU fallback.
 */
#ifndef GEHTP_OPLIST_EXEC_H
#define GEHTP_OPLIST_EXEC_H

#include <stddef.h>
#include <stdint.h>
#include "oplist_parse.h"

#ifdef __cplusplus
extern "C" {
#endif

#define WT_EXEC_MAX_TEMPS 4096

/* Run every op of b (reference oplist_exec.c:2573). */
int wt_exec_run(const struct wt_blob* b, uint32_t* engine_m,
                int64_t* op_us, char* err, size_t errn);

/* Host view of temp id (reference oplist_exec.h:34-38). */
uint8_t*  wt_exec_temp(uint32_t id);
uint32_t  wt_exec_temp_bytes(uint32_t id);
uint32_t  wt_exec_temp_last_bytes(uint32_t id);

/* Free temps and pools; persistent states survive (reference oplist_exec.c:531). */
void wt_exec_shutdown(void);

/* Zero every persistent state and its KV counters (reference oplist_exec.c:2104). */
void wt_exec_state_reset(void);

/* Caller-provided temp pool (reference oplist_exec.c:351-359). base is a DEVICE
 * pointer in this implementation; base=NULL && offsets=NULL restores bump mode. */
void wt_exec_pool_init(uint8_t* base, uint32_t total_cap, uint32_t static_cap,
                       const uint32_t* offsets);

struct wt_exec_stats {
    uint32_t ops, nop, matmul, rmsnorm, silu, pin, pin_skipped;
    uint32_t im2col, conv2d, add, spill, fill, transpose;
};

/* Run ops[first, first+count) (reference oplist_exec.c:2499-2565). */
int  wt_exec_run_range(const struct wt_blob* b, uint32_t first, uint32_t count,
                       uint32_t* engine_m, int64_t* op_us, char* err, size_t errn);
void wt_exec_get_stats(struct wt_exec_stats* st);

/* Run with injected input and copied-back output (reference oplist_exec.c:2587-2602).
 * in_ptr/out_ptr are HOST pointers; out receives wt_exec_temp_last_bytes(out_temp). */
int  wt_exec_run_io(const struct wt_blob* b, const void* in_ptr, void* out_ptr,
                    uint32_t out_temp,
                    uint32_t* engine_m, int64_t* op_us, char* err, size_t errn);

/* Extension: `steps` runs of a blob whose output feeds its own input, chained on the
 * device: in_ptr (HOST, the blob's EXT_IN slot bytes) is the first step's input; after
 * each step, out_temp's bytes (they must be as many as the input slot's) become the next
 * step's input and row s of out_ptr (HOST, steps * input bytes). Steps replayed from the
 * blob's captured HIP graph are queued without waiting for the one before, and one wait
 * at the end covers them all; an error stops at the failing step; steps * input bytes
 * is at most 64 MiB (input slot 1..4096 bytes). For greedy decoding
 * with a token-id input (the blob gathers the embedding row itself): the reference has
 * no counterpart (its host loop feeds one step at a time, oplist_exec.c:2587-2602,
 * scripts/persistent_runtime.py:43-62). */
int  wt_exec_run_steps(const struct wt_blob* b, uint32_t steps, const void* in_ptr, void* out_ptr,
                       uint32_t out_temp, uint32_t* engine_m, char* err, size_t errn);

/* Extension: bind a caller-owned DEVICE buffer of `bytes` bytes as the EXT_IN input of
 * the following wt_exec_run_io calls made with in_ptr NULL (a non-NULL in_ptr still
 * stages that host input). No host copy is made: the caller keeps the buffer alive and
 * unchanged while runs may read it, and writes it in order with the engine's stream
 * (e.g. finished before the call). A run whose input slot needs more than `bytes`
 * fails. NULL unbinds. The reference has no counterpart: its input always comes from
 * host memory (oplist_exec.c:2587-2602); this lets a caller time or chain runs with
 * inputs already resident in HBM. */
void wt_exec_set_input_device(const void* dev_ptr, size_t bytes);

/* External weight image for WT_SLOT_EXT_WGT slots (host pointer; uploaded to
 * HBM on the next run, once per (pointer, blob)). NULL disables. */
void wt_exec_set_ext_weights(const void* wgt_ptr);

enum wt_engine { WT_ENG_SCALAR = 0, WT_ENG_HVX = 1, WT_ENG_HMX = 2 };
/* In this implementation every op's engine is reported as WT_ENG_HMX (= "matrix
 * device") and dma_us/dma_bytes carry host->device copy time/bytes of the op. */
struct wt_op_ts {
    uint32_t start_us;
    uint32_t dur_us;
    uint32_t dma_us;
    uint32_t dma_bytes;
    uint32_t engine;
};
void wt_exec_set_ts(struct wt_op_ts* buf, uint32_t cap);

/* Per-op trace lines to stderr when on (default off here: no device log path). */
void wt_exec_set_trace(int on);

/* Tensor dump hook "opidx:temp,..." -> /tmp/hook_<idx>_<temp>.f16.raw
 * (reference oplist_exec.c:108-166); falls back to env GEHTP_HOOK. */
void wt_exec_set_hook(const char* spec);

/* Graph replay of repeated runs. No counterpart in the reference engine, whose ops
 * have no kernel-launch cost to amortise. When a run of ops[first, first+count) is
 * repeated with the same ops and the same device buffers (a decode step: positions
 * come from device-side counters), the engine captures it into a HIP graph on the
 * second identical run and replays the graph afterwards; results, return codes and
 * host-side state are those of a direct run. Runs with per-op timing, a tensor
 * hook or GEHTP_SYNC_EACH_OP always launch directly. Default on unless the
 * environment sets GEHTP_NO_GRAPH=1. wt_exec_set_graphs returns the previous
 * setting; wt_exec_graph_stats reports how many graphs were captured and replayed. */
int  wt_exec_set_graphs(int on);
void wt_exec_graph_stats(uint32_t* captures, uint32_t* replays);

/* Extension: load-time fusion of the reference attention op chains. Prefill: [BINARY
 * mul of q by a constant scale] -> MATMUL_F16 q.k^T (heads in the batch dimension, head
 * dim 128; k read transposed, or k^T written by a TRANSPOSE_GEN of k) -> [BINARY mul by
 * a constant scale] -> [BINARY add or ADD_F16 of a causal (0 / -inf) or all-zero mask]
 * -> SOFTMAX -> MATMUL_F16 p.v runs as one flash-attention kernel; decode: KV_GATHER of
 * a state (one op, or one per face) -> [pre-scale] -> MATMUL_F16 q.kT -> [scale] ->
 * [mask add: H rows, or one row BROADCAST over the heads] -> SOFTMAX -> MATMUL_F16 p.v
 * runs as the split-KV decode kernel on the ring. Scales and masks may be constant
 * slots or BROADCASTs of them. Members are found by dataflow (other ops may stand
 * between them; recycled temp ids are followed); the kernel runs at the last member.
 * A blob's first full run executes the chains op by op and logs reads and writes; a
 * chain is fused on later runs only if no other op read its intermediates and no op
 * that still runs wrote over its inputs' bytes before the kernel's turn. Results are
 * within the fp16 tolerance of the op-by-op chain. Default on unless the environment
 * sets GEHTP_NO_FUSE=1; wt_exec_set_fusion returns the previous setting;
 * wt_exec_fusion_stats reports chains found in the blobs seen and chain executions run
 * fused. After a fused run, wt_exec_temp returns NULL for the chain's intermediate
 * temps (they were not computed). */
int  wt_exec_set_fusion(int on);
void wt_exec_fusion_stats(uint64_t* chains_found, uint64_t* fused_runs);
/* Extension: the fusion plan of a parsed blob (after its first full run): attention
 * chains found in it, those its observed run ruled out of fusion, those whose output
 * bytes overlapped an input's in that run; and, process-wide, fused executions whose
 * output overlapped an input (the kernel then writes engine scratch, copied to the
 * output after it). For a blob not yet run, chains is what the matchers find in it
 * (host work only, no device call) and the other counts 0. */
void wt_exec_fusion_detail(const struct wt_blob* b, uint32_t* chains, uint32_t* blocked, uint32_t* aliased,
                           uint64_t* alias_runs);
/* Extension, under the same switch: an OP_W4G_FUSED_F16 q|k|v GEMM (GEMM path, plain
 * epilogue) followed in the same run by the OP_QK_ROPE_KV_F16 that reads its output
 * performs that op in its epilogue (same bits; the GEMM's own output is written too);
 * this counts such executions. */
uint64_t wt_exec_qkv_rope_fused(void);
/* Extension, under the same switch: an OP_W4G_FUSED_F16 q|k|v GEMV (M = 1, no residual,
 * no SwiGLU) followed in the same run by the OP_ATTN_DECODE_QKV_F16 that reads its
 * output runs in one launch with that op's chunk pass (same bits; the GEMV's own output
 * is written too), where the shape allows; this counts such executions. */
uint64_t wt_exec_qkv_attn_fused(void);
/* Extension, same switch: after such a launch, the o-proj OP_W4G_FUSED_F16 GEMV that reads
 * the attention output next (M = 1, no RMSNorm, no SwiGLU) runs in one launch with the
 * attention op's merge pass (same bits); this counts such executions. */
uint64_t wt_exec_merge_oproj_fused(void);

/* W3 inspect report: one JSON line per call of emit (reference wt_w3.c). */
void wt_w3_report(const char* blob_name, const uint8_t* buf, size_t size,
                  const struct wt_blob* w,
                  void (*emit)(const char* line, void* ud), void* ud);

#ifdef __cplusplus
}
#endif
#endif /* GEHTP_OPLIST_EXEC_H */
