"""Qwen3-style W4A16 runlists written in the reference runlist's own op chain.

gehtp_amd.qwen3 writes this build's fused opcodes (45/46/47/41); this module writes the
same model the way the reference front-end lowers it (the op sequence of a compiled
Qwen decoder layer: compiler/tools/wtop_ops/op_matmul.cpp:36-98 for the batched
attention matmuls, scripts/surgery_decode_graph.py:143-168 for the decode step), with
only the linears as this build's W4A16 opcode 40 (the reference has no int4 g64 format):

    h     = RMSNORM2(x, g_attn)                        25
    q,k,v = MATMUL_W4G(h, Wq / Wk / Wv)               40 x 3
    qn,kn = RMSNORM2 per 128-wide head row            25 x 2
    RoPE  = x*cos + rotate_half(x)*sin                15 x 2 (halves), 11 (neg), 14 (concat),
                                                        12 mul x 2, 12 add   (per q and k)
  decode (one token, positions from the KV state's counter):
    KV_APPEND(k, v) ; KV_GATHER -> kT [H,hd,P], v [H,P,hd]         22, 23
    s = MATMUL_F16(q, kT) batched ; *scale ; +mask ; SOFTMAX ; MATMUL_F16(p, v)   24 12 12 13 24
  prefill (S tokens, no state):
    q/k/v to head-major [., S, hd]; k/v repeated to H heads     27, 26
    s = MATMUL_F16(q, k^T) batched ; *scale ; +causal mask ; SOFTMAX ; MATMUL_F16(p, v) ; back to [S, H, hd]
    o     = MATMUL_W4G(a, Wo) ; x1 = ADD(x, o)                 40, 7
    m     = SLICE(gate/up rows) -> UNARY silu -> BINARY mul    40, 15 x 2, 11, 12
    x     = BINARY add(x1, MATMUL_W4G(m, Wd))                  40, 12
then RMSNORM2, the fp16 lm_head (MATMUL_F16) and ARGMAX.

The decode blob's input is the reference persistent runner's step body
(scripts/persistent_runtime.py:43-62): token id (int32) then the face [cos | sin | mask]
in fp16: cos / sin of position * 1/theta^(2j/hd) in float64, each half duplicated, and
the additive mask over the P = max_pos ring positions (0 up to the token's position,
-inf after). The embedding row is gathered in-graph (GATHER, 20) and the face is carved
with STRIDED_SLICE. The prefill blob's input is the prompt's token ids (int32 [S]).

`lowering` selects how the attention chain is written:
  "chain"    : as above (scale and mask as full-size constant slots, one KV_GATHER with
               both faces, fresh temp ids);
  "ref_post" : the forms the reference emitter writes for a scale after q.k^T
               (test_models/transformer32: MatMul -> BROADCAST -> BINARY mul): k^T by
               TRANSPOSE_GEN and MATMUL_F16 flags 4, the scale a 1-value slot BROADCAST
               to the scores' shape and multiplied, the mask a BROADCAST of one [S, S] (or,
               in decode, the step input's [P] row) over the heads added with ADD_F16,
               one KV_GATHER per face (compiler/tools/wtop_ops/op_decode_state.cpp:66-80);
  "ref_pre"  : the same with the scale applied to q before the matmul and k read
               transposed (flags 6) (qwen35_08b manifest ops 2722-2728: BROADCAST, BINARY,
               MATMUL, BROADCAST, ADD_F16, SOFTMAX, MATMUL).
`recycle` renumbers temps with the reference emitter's free list (gehtp_amd.tempplan),
and `tempoff` adds a static temp plan (TEMPOFF slot) whose temps share bytes wherever
their spans do not meet.

Weights are the same external image as gehtp_amd.qwen3.Weights: q/k/v are contiguous
row ranges of the stored q|k|v matrix; gate/up stay interleaved in one matrix and are
separated by two strided slices after the linear.
"""
from __future__ import annotations

import numpy as np

from .abi import WT_KV_POS_AUTO, WT_SLOT_EXT_WGT, opcodes as OP
from .qwen3 import Qwen3Config, Weights
from .runlist import BlobBuilder, _Slot

NEG, SILU = 0, 12                   # UNARY subtypes (oplist_exec.c:1056-1068)
ADD, MUL = 0, 2                     # BINARY subtypes (oplist_exec.c:1146-1150)
F16_NEG_INF = 0xFC00


def rope_tables(pos: np.ndarray, hd: int, theta: float):
    """fp16 cos / sin rows [len(pos), hd] as the reference host builds them
    (scripts/persistent_runtime.py:43-55): float64 angles, each half duplicated."""
    inv = 1.0 / (float(theta) ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    return (np.concatenate([c, c], axis=1).astype(np.float16),
            np.concatenate([s, s], axis=1).astype(np.float16))


def face_elems(cfg: Qwen3Config, max_pos: int) -> int:
    """fp16 elements of the decode step input: id (2) + cos + sin + mask."""
    return 2 + 2 * cfg.head_dim + max_pos


def decode_input(cfg: Qwen3Config, token: int, pos: int, max_pos: int) -> bytes:
    """The decode blob's step body for `token` at position `pos`."""
    if not 0 <= pos < max_pos:
        raise ValueError(f"position {pos} outside [0, {max_pos})")
    c, s = rope_tables(np.array([pos]), cfg.head_dim, cfg.theta)
    mask = np.zeros(max_pos, np.float16)
    mask[pos + 1:] = -np.inf
    return (np.array([token], np.int32).tobytes() + c.tobytes() + s.tobytes() + mask.tobytes())


class _ChainEmitter:
    def __init__(self, cfg: Qwen3Config, w: Weights):
        self.cfg, self.w = cfg, w
        self.bb = BlobBuilder()
        self.slot = {}
        c = cfg
        D = c.hidden
        for name, (off, nb) in w.layout.items():
            if ".wqkv." in name:
                continue
            count = nb * 2 if name.endswith(".q") else nb // 2
            self.slot[name] = self._ext(off, nb, count)
        # q, k, v: contiguous row ranges of the stored q|k|v matrix
        for l in range(c.layers):
            qo, _ = w.layout[f"{l}.wqkv.q"]
            so, _ = w.layout[f"{l}.wqkv.s"]
            r0 = 0
            for nm, rows in (("wq", c.q_dim), ("wk", c.kv_dim), ("wv", c.kv_dim)):
                self.slot[f"{l}.{nm}.q"] = self._ext(qo + r0 * D // 2, rows * D // 2, rows * D)
                self.slot[f"{l}.{nm}.s"] = self._ext(so + r0 * (D // c.group) * 2, rows * (D // c.group) * 2,
                                                     rows * (D // c.group))
                r0 += rows
        self.zero_d = self.bb.add_slot(np.zeros(D, np.float16))
        self.zero_hd = self.bb.add_slot(np.zeros(c.head_dim, np.float16))

    def _ext(self, off, nb, count):
        if off % 128:
            raise ValueError("external weight slot offsets must be 128-byte aligned")
        self.bb.slots.append(_Slot(None, nb, count, WT_SLOT_EXT_WGT, off))
        return len(self.bb.slots) - 1

    def ref(self, name):
        return self.bb.slot_ref(self.slot[name])

    def T(self):
        return self.bb.temp()

    # ---- op helpers ----
    def rmsnorm(self, x, gamma_ref, zero_slot, n):
        y = self.T()
        self.bb.op(OP.RMSNORM2_F16, x, gamma_ref, self.bb.slot_ref(zero_slot), y, n)
        return y

    def w4g(self, a, l, nm, M, K, N):
        y = self.T()
        self.bb.op(OP.MATMUL_W4G_F16, a, self.ref(f"{l}.{nm}.q"), self.ref(f"{l}.{nm}.s"), y, M, K, N,
                   self.cfg.group, 2)
        return y

    def slice1(self, x, n_in, b0, e0, s0=1):
        y = self.T()
        n = (e0 - b0 + s0 - 1) // s0
        self.bb.op(OP.STRIDED_SLICE_F16, x, y, n, 1, b0, 0, 0, e0, 0, 0, s0, 1, 1, n_in, 1, 1)
        return y

    def slice2(self, x, rows, cols, c0, c1, cs=1):
        """x [rows, cols] -> x[:, c0:c1:cs]."""
        y = self.T()
        n = rows * ((c1 - c0 + cs - 1) // cs)
        self.bb.op(OP.STRIDED_SLICE_F16, x, y, n, 2, 0, c0, 0, rows, c1, 0, 1, cs, 1, rows, cols, 1)
        return y

    def binary(self, a, b, n, sub):
        y = self.T()
        self.bb.op(OP.BINARY_F16, a, b, y, n, sub)
        return y

    def add_f16(self, a, b, n):
        y = self.T()
        self.bb.op(OP.ADD_F16, a, b, y, n)
        return y

    def unary(self, x, n, sub):
        y = self.T()
        self.bb.op(OP.UNARY_F16, x, y, n, sub)
        return y

    def concat2(self, a, b, rows, ca, cb):
        y = self.T()
        self.bb.op(OP.CONCAT_F16, a, b, 0, 0, 0, 0, 0, 0, y, 0, 2, rows * (ca + cb), ca, cb, 0, 0)
        return y

    def broadcast(self, x, in_d, out_d):
        y = self.T()
        n = int(np.prod(out_d))
        ind = list(in_d) + [1] * (4 - len(in_d))
        outd = list(out_d) + [1] * (4 - len(out_d))
        self.bb.op(OP.BROADCAST_F16, x, y, n, int(np.prod(in_d)), *ind, *outd)
        return y

    def transpose3(self, x, dims, perm):
        y = self.T()
        self.bb.op(OP.TRANSPOSE_GEN_F16, x, y, 3, dims[0], dims[1], dims[2], 1,
                   perm[0] | (perm[1] << 8) | (perm[2] << 16))
        return y

    def rope(self, x, rows, cos_b, sin_b):
        """rows x hd (one head per row): x*cos + [-x2, x1]*sin."""
        hd = self.cfg.head_dim
        half = hd // 2
        n = rows * hd
        x1 = self.slice2(x, rows, hd, 0, half)
        x2 = self.slice2(x, rows, hd, half, hd)
        rot = self.concat2(self.unary(x2, rows * half, NEG), x1, rows, half, half)
        return self.binary(self.binary(x, cos_b, n, MUL), self.binary(rot, sin_b, n, MUL), n, ADD)

    def ffn(self, x, l, S):
        c = self.cfg
        D, F = c.hidden, c.ffn
        h2 = self.rmsnorm(x, self.ref(f"{l}.g_ffn"), self.zero_d, S * D)
        gu = self.w4g(h2, l, "wgu", S, D, 2 * F)
        g = self.slice2(gu, S, 2 * F, 0, 2 * F, 2)
        u = self.slice2(gu, S, 2 * F, 1, 2 * F, 2)
        m = self.binary(self.unary(g, S * F, SILU), u, S * F, MUL)
        return self.binary(x, self.w4g(m, l, "wd", S, F, D), S * D, ADD)

    def head(self, x, S):
        c, bb = self.cfg, self.bb
        n = S * c.hidden
        hn = self.rmsnorm(x, self.ref("g_final"), self.zero_d, n)
        last = hn if S == 1 else self.slice1(hn, n, n - c.hidden, n)
        logits, tok = self.T(), self.T()
        bb.op(OP.MATMUL_F16, last, self.ref("embed"), logits, 1, c.hidden, c.vocab, 2)
        bb.op(OP.ARGMAX_F16, logits, tok, c.vocab)
        return logits, tok

    def gather_rows(self, ids_ref, n_ids):
        c = self.cfg
        x = self.T()
        self.bb.op(OP.GATHER_F16, self.ref("embed"), ids_ref, x, n_ids * c.hidden, 0 | (1 << 8) | (2 << 16),
                   c.vocab, c.hidden, 1, 1, 1, n_ids, 1, 1, 1, 1)
        return x


LOWERINGS = ("chain", "ref_post", "ref_pre")


def _finish(bb, keep, recycle: bool, tempoff: bool):
    """Renumber temps (reference free list) and add a TEMPOFF plan, as asked; returns
    the renumbered ids of `keep`."""
    from .tempplan import recycle as _recycle, tempoff_plan
    ids = list(keep)
    if recycle:
        m = _recycle(bb, keep=ids)
        ids = [m[t] for t in ids]
    if tempoff:
        cap, entries = tempoff_plan(bb, keep=ids)
        bb.set_tempoff(cap, entries)
    return ids


def _scale_ref(e, lowering, n, dims):
    """The scale operand for a BINARY mul over n values: a full-size slot ("chain") or
    a 1-value slot BROADCAST to `dims`."""
    c, bb = e.cfg, e.bb
    if lowering == "chain":
        return bb.slot_ref(bb.add_slot(np.full(n, np.float16(c.scale), np.float16)))
    if not hasattr(e, "scale1"):
        e.scale1 = bb.slot_ref(bb.add_slot(np.array([c.scale], np.float16)))
    return e.broadcast(e.scale1, [1] * len(dims), dims)


def emit_decode_chain(cfg: Qwen3Config, w: Weights, max_pos: int, lowering: str = "chain",
                      recycle: bool = False, tempoff: bool = False):
    """(blob, temps) of one decode step in the reference op chain. Input: the step body
    of decode_input(); KV rings of max_pos positions (one STATE per layer)."""
    if lowering not in LOWERINGS:
        raise ValueError(f"lowering {lowering!r} not in {LOWERINGS}")
    e = _ChainEmitter(cfg, w)
    c, bb = cfg, e.bb
    H, KVH, hd, P, D = c.heads, c.kv_heads, c.head_dim, max_pos, c.hidden
    nface = face_elems(cfg, max_pos)
    face = bb.slot_ref(bb.add_input_slot(nface * 2))
    states = [bb.add_state(max_pos * c.kv_dim * 4) for _ in range(c.layers)]
    scale_full = _scale_ref(e, "chain", H * P, None) if lowering == "chain" else None
    x = e.gather_rows(face, 1)
    cos = e.slice1(face, nface, 2, 2 + hd)
    sin = e.slice1(face, nface, 2 + hd, 2 + 2 * hd)
    mask = e.slice1(face, nface, 2 + 2 * hd, 2 + 2 * hd + P)
    cos_q, sin_q = e.broadcast(cos, [1, hd], [H, hd]), e.broadcast(sin, [1, hd], [H, hd])
    cos_k, sin_k = e.broadcast(cos, [1, hd], [KVH, hd]), e.broadcast(sin, [1, hd], [KVH, hd])
    mask_h = e.broadcast(mask, [1, P], [H, P]) if lowering == "chain" else None
    for l in range(c.layers):
        h = e.rmsnorm(x, e.ref(f"{l}.g_attn"), e.zero_d, D)
        q = e.w4g(h, l, "wq", 1, D, c.q_dim)
        k = e.w4g(h, l, "wk", 1, D, c.kv_dim)
        v = e.w4g(h, l, "wv", 1, D, c.kv_dim)
        qr = e.rope(e.rmsnorm(q, e.ref(f"{l}.q_norm"), e.zero_hd, c.q_dim), H, cos_q, sin_q)
        kr = e.rope(e.rmsnorm(k, e.ref(f"{l}.k_norm"), e.zero_hd, c.kv_dim), KVH, cos_k, sin_k)
        bb.op(OP.KV_APPEND_F16, kr, v, states[l], WT_KV_POS_AUTO)
        if lowering == "chain":
            kT, vv = e.T(), e.T()
            bb.op(OP.KV_GATHER_F16, states[l], kT, vv, WT_KV_POS_AUTO, H, KVH, hd)
            s = e.T()
            bb.op(OP.MATMUL_F16, qr, kT, s, 1, hd, P, 4 | (H << 16))
            s2 = e.binary(e.binary(s, scale_full, H * P, MUL), mask_h, H * P, ADD)
        else:
            kT = e.T()
            bb.op(OP.KV_GATHER_F16, states[l], kT, 0, WT_KV_POS_AUTO, H, KVH, hd)
            vv = e.T()
            bb.op(OP.KV_GATHER_F16, states[l], 0, vv, WT_KV_POS_AUTO, H, KVH, hd)
            if lowering == "ref_pre":
                qr = e.binary(qr, _scale_ref(e, lowering, H * hd, [H, hd]), H * hd, MUL)
            s = e.T()
            bb.op(OP.MATMUL_F16, qr, kT, s, 1, hd, P, 4 | (H << 16))
            if lowering == "ref_post":
                s = e.binary(s, _scale_ref(e, lowering, H * P, [H, P]), H * P, MUL)
            s2 = e.add_f16(s, e.broadcast(mask, [1, P], [H, P]), H * P)
        p, a = e.T(), e.T()
        bb.op(OP.SOFTMAX_F16, s2, p, H, P)
        bb.op(OP.MATMUL_F16, p, vv, a, 1, P, hd, 4 | (H << 16))
        o = e.w4g(a, l, "wo", 1, c.q_dim, D)
        x1 = e.T()
        bb.op(OP.ADD_F16, x, o, x1, D)
        x = e.ffn(x1, l, 1)
    logits, tok = e.head(x, 1)
    logits, tok = _finish(bb, [logits, tok], recycle, tempoff)
    return bb.build(), {"logits": logits, "tok": tok}


def emit_prefill_chain(cfg: Qwen3Config, w: Weights, S: int, lowering: str = "chain", recycle: bool = False,
                       tempoff: bool = False):
    """(blob, temps) of a causal prefill of S tokens in the reference op chain (no KV
    state: the reference serves a prompt through its decode graph). Input: the prompt's
    token ids, int32 [S]."""
    if lowering not in LOWERINGS:
        raise ValueError(f"lowering {lowering!r} not in {LOWERINGS}")
    e = _ChainEmitter(cfg, w)
    c, bb = cfg, e.bb
    H, KVH, hd, D = c.heads, c.kv_heads, c.head_dim, c.hidden
    rep = H // KVH
    ids = bb.slot_ref(bb.add_input_slot(S * 4, count=S))
    cos_t, sin_t = rope_tables(np.arange(S), hd, c.theta)
    cos_s, sin_s = bb.slot_ref(bb.add_slot(cos_t)), bb.slot_ref(bb.add_slot(sin_t))
    n = H * S * S
    causal = np.where(np.arange(S)[None, :] <= np.arange(S)[:, None], np.float16(0), np.float16(-np.inf))
    if lowering == "chain":
        scale = _scale_ref(e, lowering, n, None)
        mask = bb.slot_ref(bb.add_slot(np.broadcast_to(causal, (H, S, S)).astype(np.float16)))
    else:
        mask_ss = bb.slot_ref(bb.add_slot(causal.astype(np.float16)))
    x = e.gather_rows(ids, S)
    cos_q, sin_q = e.broadcast(cos_s, [S, 1, hd], [S, H, hd]), e.broadcast(sin_s, [S, 1, hd], [S, H, hd])
    cos_k, sin_k = e.broadcast(cos_s, [S, 1, hd], [S, KVH, hd]), e.broadcast(sin_s, [S, 1, hd], [S, KVH, hd])
    for l in range(c.layers):
        h = e.rmsnorm(x, e.ref(f"{l}.g_attn"), e.zero_d, S * D)
        q = e.w4g(h, l, "wq", S, D, c.q_dim)
        k = e.w4g(h, l, "wk", S, D, c.kv_dim)
        v = e.w4g(h, l, "wv", S, D, c.kv_dim)
        qr = e.rope(e.rmsnorm(q, e.ref(f"{l}.q_norm"), e.zero_hd, S * c.q_dim), S * H, cos_q, sin_q)
        kr = e.rope(e.rmsnorm(k, e.ref(f"{l}.k_norm"), e.zero_hd, S * c.kv_dim), S * KVH, cos_k, sin_k)
        qh = e.transpose3(qr, (S, H, hd), (1, 0, 2))
        kh = e.broadcast(e.transpose3(kr, (S, KVH, hd), (1, 0, 2)), [KVH, 1, S, hd], [KVH, rep, S, hd])
        vh = e.broadcast(e.transpose3(v, (S, KVH, hd), (1, 0, 2)), [KVH, 1, S, hd], [KVH, rep, S, hd])
        s = e.T()
        if lowering == "chain":
            bb.op(OP.MATMUL_F16, qh, kh, s, S, hd, S, 6 | (H << 16))
            s2 = e.binary(e.binary(s, scale, n, MUL), mask, n, ADD)
        elif lowering == "ref_post":
            kT = e.transpose3(kh, (H, S, hd), (0, 2, 1))
            bb.op(OP.MATMUL_F16, qh, kT, s, S, hd, S, 4 | (H << 16))
            s1 = e.binary(s, _scale_ref(e, lowering, n, [H, S, S]), n, MUL)
            s2 = e.add_f16(s1, e.broadcast(mask_ss, [1, S, S], [H, S, S]), n)
        else:
            qs = e.binary(qh, _scale_ref(e, lowering, H * S * hd, [H, S, hd]), H * S * hd, MUL)
            bb.op(OP.MATMUL_F16, qs, kh, s, S, hd, S, 6 | (H << 16))
            s2 = e.add_f16(s, e.broadcast(mask_ss, [1, S, S], [H, S, S]), n)
        p, ah = e.T(), e.T()
        bb.op(OP.SOFTMAX_F16, s2, p, H * S, S)
        bb.op(OP.MATMUL_F16, p, vh, ah, S, S, hd, 4 | (H << 16))
        a = e.transpose3(ah, (H, S, hd), (1, 0, 2))
        o = e.w4g(a, l, "wo", S, c.q_dim, D)
        x1 = e.T()
        bb.op(OP.ADD_F16, x, o, x1, S * D)
        x = e.ffn(x1, l, S)
    logits, tok = e.head(x, S)
    logits, tok = _finish(bb, [logits, tok], recycle, tempoff)
    return bb.build(), {"logits": logits, "tok": tok}
