"""Runlist emitter for Qwen3-style decoder models with W4A16 (int4 g64) linears.

Writes WTOP blobs for prefill and for one decode step, in the reference engine's
terms: weights as EXT_WGT slots of one external image (so a multi-GB model is not
inlined into the blob), one persistent KV-ring STATE per layer, activations in
temps, the token embeddings arriving through the EXT_IN slot.

Per layer (pre-norm, eps 1e-6), four fused linears and two attention ops:
    qkv = W4G_FUSED(x, Wqkv, norm=g_attn)            RMSNORM2 + q|k|v linears
    q   = QK_ROPE_KV(qkv)                            Qwen3 QK-norm, RoPE, KV append
    a   = ATTN (prefill, causal)
  (decode: a = ATTN_DECODE_QKV(qkv), the two ops above over the layer's ring in one)
    x1  = W4G_FUSED(a, Wo, residual=x)               o-proj + ADD
    m   = W4G_FUSED(x1, Wgu, norm=g_ffn, SwiGLU)     RMSNORM2 + gate|up + silu * up
    x   = W4G_FUSED(m, Wd, residual=x1)              down-proj + ADD
then RMSNORM2(x, g_final), the fp16 lm_head (MATMUL_F16, w stored [V, D]) on the
last token and ARGMAX. Each fused op rounds where the separate runlist ops it replaces
round, so the oracle composition of the separate ops (oracle/qwen3_ref.py) is the
checker. RoPE positions come from the layer state's counter, so the decode blob is
identical for every step.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .abi import WT_KV_POS_AUTO, WT_REF_NONE, opcodes as OP
from .runlist import BlobBuilder, f32_bits


@dataclass(frozen=True)
class Qwen3Config:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    ffn: int
    vocab: int
    head_dim: int = 128
    theta: float = 1e6
    group: int = 64

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def scale(self) -> float:
        # the attention scale as an fp16 constant, as reference runlists carry it
        return float(np.float16(1.0 / math.sqrt(self.head_dim)))

    def linears(self):
        """(name, N, K) of the per-layer W4A16 linears."""
        D, F = self.hidden, self.ffn
        return [("wq", self.q_dim, D), ("wk", self.kv_dim, D), ("wv", self.kv_dim, D),
                ("wo", D, self.q_dim), ("wg", F, D), ("wu", F, D), ("wd", D, F)]

    def fused_linears(self):
        """(name, rows, K) of the stored (fused) matrices: q|k|v rows, o, gate/up rows
        interleaved, down."""
        D, F = self.hidden, self.ffn
        return [("wqkv", self.q_dim + 2 * self.kv_dim, D), ("wo", D, self.q_dim),
                ("wgu", 2 * F, D), ("wd", D, F)]

    def decode_weight_bytes(self) -> int:
        """Algorithmic HBM bytes of one decode token: int4 weights + fp16 scales of every
        linear, plus the fp16 lm_head."""
        per_layer = sum(n * k // 2 + n * (k // self.group) * 2 for _, n, k in self.linears())
        return self.layers * per_layer + self.vocab * self.hidden * 2

    def prefill_flops(self, S: int) -> float:
        lin = sum(2.0 * S * n * k for _, n, k in self.linears()) * self.layers
        attn = 2 * 2.0 * self.heads * (S * (S + 1) / 2) * self.head_dim * self.layers
        return lin + attn + 2.0 * self.vocab * self.hidden   # lm_head on the last token


# BASELINE configs 4 and 5.
CONFIG_08B_LAYER = Qwen3Config(layers=1, hidden=1024, heads=16, kv_heads=8, ffn=3072, vocab=151936)
CONFIG_4B = Qwen3Config(layers=36, hidden=2560, heads=32, kv_heads=8, ffn=9728, vocab=151936)


# Random-init int4 values for the model configs: each uniform nibble is mapped through
# this zero-mean, symmetric table (std 2.98) instead of taking q uniform on [-8, 7].
# Uniform [-8, 7] has mean -0.5: across 36 layers that common-mode bias makes the fp16
# residual stream overflow (measured: inf by layer 4 of the 4B-class model).
INT4_INIT_TABLE = np.array([-6, -4, -3, -2, -2, -1, -1, 0, 0, 1, 1, 2, 2, 3, 4, 6], np.int8)
_BYTE_LUT = np.array([((INT4_INIT_TABLE[b & 15] + 8) | ((INT4_INIT_TABLE[b >> 4] + 8) << 4))
                      for b in range(256)], np.uint8)


class Weights:
    """Random-init weights laid out in ONE external image (numpy uint8), plus views.

    int4 values: uniform random nibbles mapped through INT4_INIT_TABLE (zero mean);
    scales U[0.005, 0.02]; norm gammas U(0.8, 1.2); embeddings ~N(0, 1) (tied lm_head)."""

    def __init__(self, cfg: Qwen3Config, seed: int = 0, embed_std: float = 1.0):
        self.cfg = cfg
        rng = np.random.default_rng(seed)
        layout, off = {}, 0

        def reserve(name, nbytes):
            nonlocal off
            off = (off + 127) // 128 * 128
            layout[name] = (off, nbytes)
            off += nbytes

        for l in range(cfg.layers):
            for nm, n, k in cfg.fused_linears():
                reserve(f"{l}.{nm}.q", n * k // 2)
                reserve(f"{l}.{nm}.s", n * (k // cfg.group) * 2)
            for nm, n in (("g_attn", cfg.hidden), ("g_ffn", cfg.hidden), ("q_norm", cfg.head_dim),
                          ("k_norm", cfg.head_dim)):
                reserve(f"{l}.{nm}", n * 2)
        reserve("g_final", cfg.hidden * 2)
        reserve("embed", cfg.vocab * cfg.hidden * 2)
        self.layout = layout
        self.image = np.zeros((off + 127) // 128 * 128, np.uint8)
        for name, (o, nb) in layout.items():
            view = self.image[o:o + nb]
            if name.endswith(".q"):
                view[:] = _BYTE_LUT[np.frombuffer(rng.bytes(nb), np.uint8)]
            elif name.endswith(".s"):
                view.view(np.float16)[:] = rng.uniform(0.005, 0.02, nb // 2).astype(np.float16)
            elif name == "embed":
                e = view.view(np.float16).reshape(cfg.vocab, cfg.hidden)
                for r0 in range(0, cfg.vocab, 8192):
                    r1 = min(cfg.vocab, r0 + 8192)
                    e[r0:r1] = (rng.standard_normal((r1 - r0, cfg.hidden), np.float32) * embed_std).astype(np.float16)
            else:
                view.view(np.float16)[:] = rng.uniform(0.8, 1.2, nb // 2).astype(np.float16)

    def get(self, name: str) -> np.ndarray:
        o, nb = self.layout[name]
        return self.image[o:o + nb]

    def f16(self, name: str) -> np.ndarray:
        return self.get(name).view(np.float16)

    def fused(self, layer: int, nm: str):
        """(wq uint8 [rows, K/2], scales fp16 [rows, K/64]) of a stored fused matrix."""
        n, k = {x[0]: (x[1], x[2]) for x in self.cfg.fused_linears()}[nm]
        return (self.get(f"{layer}.{nm}.q").reshape(n, k // 2),
                self.f16(f"{layer}.{nm}.s").reshape(n, k // self.cfg.group))

    def linear(self, layer: int, nm: str):
        """(wq packed uint8 [N, K/2], scales fp16 [N, K/64]) of a logical linear
        (wq, wk, wv, wo, wg, wu, wd), cut out of the fused storage."""
        c = self.cfg
        if nm in ("wq", "wk", "wv"):
            q, s = self.fused(layer, "wqkv")
            lo = {"wq": 0, "wk": c.q_dim, "wv": c.q_dim + c.kv_dim}[nm]
            hi = lo + (c.q_dim if nm == "wq" else c.kv_dim)
            return q[lo:hi], s[lo:hi]
        if nm in ("wg", "wu"):
            q, s = self.fused(layer, "wgu")
            r = 0 if nm == "wg" else 1
            return np.ascontiguousarray(q[r::2]), np.ascontiguousarray(s[r::2])
        return self.fused(layer, nm)

    def embed(self) -> np.ndarray:
        return self.f16("embed").reshape(self.cfg.vocab, self.cfg.hidden)


class _Emitter:
    def __init__(self, cfg: Qwen3Config, w: Weights, max_pos: int, fused_decode: bool = True):
        self.cfg, self.w, self.max_pos = cfg, w, max_pos
        self.fused_decode = fused_decode
        self.bb = BlobBuilder()
        self.slot = {}
        # EXT_WGT slots pointing into the external image (descriptors only).
        for name, (off, nb) in w.layout.items():
            count = nb * 2 if name.endswith(".q") else nb // 2
            self.slot[name] = self._ext_slot(off, nb, count)
        self.zero_bias = self.bb.add_slot(np.zeros(max(cfg.hidden, cfg.head_dim), np.float16))
        self.states = [self.bb.add_state(max_pos * cfg.kv_dim * 4) for _ in range(cfg.layers)]
        self.t = {n: self.bb.temp() for n in
                  ("x", "x1", "h", "qkv", "qr", "kr", "v", "a", "m", "last", "logits", "tok")}

    def _ext_slot(self, off, nb, count):
        from .abi import WT_SLOT_EXT_WGT
        from .runlist import _Slot
        self.bb.slots.append(_Slot(None, nb, count, WT_SLOT_EXT_WGT, off))
        return len(self.bb.slots) - 1

    def ref(self, name):
        return self.bb.slot_ref(self.slot[name])

    def norm(self, x, gamma, y, n):
        bb = self.bb
        bb.op(OP.RMSNORM2_F16, x, self.ref(gamma), bb.slot_ref(self.zero_bias), y, n)

    def w4g(self, a, l, nm, y, M, norm=None, res=None, swiglu=False):
        n, k = {x[0]: (x[1], x[2]) for x in self.cfg.fused_linears()}[nm]
        self.bb.op(OP.W4G_FUSED_F16, a, self.ref(f"{l}.{nm}.q"), self.ref(f"{l}.{nm}.s"), y, M, k, n,
                   self.ref(norm) if norm else WT_REF_NONE, res if res is not None else WT_REF_NONE,
                   1 if swiglu else 0, 2)

    def layer(self, l: int, S: int, x_in: int, decode: bool):
        c, bb, t = self.cfg, self.bb, self.t
        st = self.states[l]
        self.w4g(x_in, l, "wqkv", t["qkv"], S, norm=f"{l}.g_attn")
        if decode and self.fused_decode:
            bb.op(OP.ATTN_DECODE_QKV_F16, t["qkv"], st, t["a"], c.heads, c.kv_heads, c.head_dim,
                  self.ref(f"{l}.q_norm"), self.ref(f"{l}.k_norm"), f32_bits(c.theta), f32_bits(c.scale))
        else:
            bb.op(OP.QK_ROPE_KV_F16, t["qkv"], t["qr"], WT_REF_NONE if decode else t["kr"],
                  WT_REF_NONE if decode else t["v"], st, S, c.heads, c.kv_heads, c.head_dim,
                  self.ref(f"{l}.q_norm"), self.ref(f"{l}.k_norm"), f32_bits(c.theta))
        if decode and self.fused_decode:
            pass   # attention already emitted
        elif decode:
            bb.op(OP.ATTN_DECODE_F16, t["qr"], st, t["a"], WT_KV_POS_AUTO, c.heads, c.kv_heads, c.head_dim,
                  f32_bits(c.scale))
        else:
            bb.op(OP.ATTN_F16, t["qr"], t["kr"], t["v"], t["a"], S, c.heads, c.kv_heads, c.head_dim,
                  f32_bits(c.scale), 1)
        self.w4g(t["a"], l, "wo", t["x1"], S, res=x_in)
        self.w4g(t["x1"], l, "wgu", t["m"], S, norm=f"{l}.g_ffn", swiglu=True)
        self.w4g(t["m"], l, "wd", t["x"], S, res=t["x1"])

    def head(self, S: int):
        c, bb, t = self.cfg, self.bb, self.t
        self.norm(t["x"], "g_final", t["h"], S * c.hidden)
        src = t["h"]
        if S > 1:   # lm_head on the last token only
            n = S * c.hidden
            bb.op(OP.STRIDED_SLICE_F16, t["h"], t["last"], c.hidden, 1, n - c.hidden, 0, 0, n, 1, 1,
                  1, 1, 1, n, 1, 1)
            src = t["last"]
        bb.op(OP.MATMUL_F16, src, self.ref("embed"), t["logits"], 1, c.hidden, c.vocab, 2)
        bb.op(OP.ARGMAX_F16, t["logits"], t["tok"], c.vocab)

    def finish(self, recycle: bool, tempoff: bool) -> bytes:
        """Build the blob; with `recycle` its temps renumbered by the reference emitter's
        free list, with `tempoff` a TEMPOFF static plan added (gehtp_amd.tempplan). The
        logits and token temps are kept live to the end (read after the run)."""
        from .tempplan import recycle as _recycle, tempoff_plan
        keep = [self.t["logits"], self.t["tok"]]
        if recycle:
            m = _recycle(self.bb, keep=keep)
            self.t = {k: m[v] for k, v in self.t.items() if v in m}
            keep = [self.t["logits"], self.t["tok"]]
        if tempoff:
            cap, entries = tempoff_plan(self.bb, keep=keep)
            self.bb.set_tempoff(cap, entries)
        return self.bb.build()

    def emit(self, S: int, decode: bool, token_input: bool = False, recycle: bool = False,
             tempoff: bool = False) -> bytes:
        c, bb = self.cfg, self.bb
        if token_input:   # int32 token ids in; the embedding rows gathered in-graph
            ids = bb.add_input_slot(S * 4)
            x0 = bb.temp()
            self.t["x0"] = x0
            bb.op(OP.GATHER_F16, self.ref("embed"), bb.slot_ref(ids), x0, S * c.hidden, 0 | (1 << 8) | (2 << 16),
                  c.vocab, c.hidden, 1, 1, 1, S, 1, 1, 1, 1)
            x_in = x0
        else:
            x_in = bb.slot_ref(bb.add_input_slot(S * c.hidden * 2))
        for l in range(c.layers):
            self.layer(l, S, x_in if l == 0 else self.t["x"], decode)
        self.head(S)
        return self.finish(recycle, tempoff)


def emit_prefill(cfg: Qwen3Config, w: Weights, S: int, max_pos: int, recycle: bool = False,
                 tempoff: bool = False):
    """(blob bytes, temp ids): a prefill of S tokens; input = embeddings [S, hidden] fp16.
    recycle / tempoff: temp ids from the reference emitter's free list / a TEMPOFF plan."""
    e = _Emitter(cfg, w, max_pos)
    blob = e.emit(S, decode=False, recycle=recycle, tempoff=tempoff)
    return blob, dict(e.t)


def emit_decode(cfg: Qwen3Config, w: Weights, max_pos: int, fused: bool = True, token_input: bool = False,
                recycle: bool = False, tempoff: bool = False):
    """(blob bytes, temp ids): one decode step; input = the token's embedding [hidden],
    or with token_input its int32 id (the row gathered in-graph from the lm_head / embedding
    table, so the step's ARGMAX output can feed the next step: wt_exec_run_steps).
    fused: attention as one OP_ATTN_DECODE_QKV_F16 per layer instead of
    OP_QK_ROPE_KV_F16 + OP_ATTN_DECODE_F16. recycle / tempoff as for emit_prefill."""
    e = _Emitter(cfg, w, max_pos, fused_decode=fused)
    blob = e.emit(1, decode=True, token_input=token_input, recycle=recycle, tempoff=tempoff)
    return blob, dict(e.t)
