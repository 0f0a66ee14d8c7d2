"""The Qwen3-style W4A16 model composed from the oracle's restated ops (TEST INFRASTRUCTURE).

Follows the same op sequence as gehtp_amd.qwen3's runlists, but every op is the
reference's scalar arithmetic with f16 rounding at op boundaries, and attention is
the reference runlist chain (batched matmul, scale, mask, softmax, matmul; see
oracle/gehtp_oracle.c go_attn_prefill and KVRing.attn_decode).
"""
from __future__ import annotations

import numpy as np

from . import oracle as o


class RefModel:
    def __init__(self, cfg, weights, max_pos: int, threads: int = 8):
        self.cfg, self.w, self.threads = cfg, weights, threads
        self.rings = [o.KVRing(max_pos * cfg.kv_dim * 4, cfg.kv_dim) for _ in range(cfg.layers)]
        self.pos = 0

    def _lin(self, x, l, nm):
        wq, ws = self.w.linear(l, nm)
        return o.matmul_w4g(x, wq, ws, self.threads)

    def _qk(self, h, l, S):
        c = self.cfg
        q = self._lin(h, l, "wq")
        k = self._lin(h, l, "wk")
        v = self._lin(h, l, "wv")
        qn = o.rmsnorm2(q.reshape(S * c.heads, c.head_dim), self.w.f16(f"{l}.q_norm")).reshape(S, c.q_dim)
        kn = o.rmsnorm2(k.reshape(S * c.kv_heads, c.head_dim), self.w.f16(f"{l}.k_norm")).reshape(S, c.kv_dim)
        qr = o.rope(qn, c.heads, c.head_dim, self.pos, c.theta)
        kr = o.rope(kn, c.kv_heads, c.head_dim, self.pos, c.theta)
        return qr, kr, v

    def _ffn(self, x, l):
        h2 = o.rmsnorm2(x, self.w.f16(f"{l}.g_ffn"))
        g = self._lin(h2, l, "wg")
        u = self._lin(h2, l, "wu")
        m = o.binary(o.unary(g, 12), u, 2)
        return o.binary(x, self._lin(m, l, "wd"), 0)

    def _head(self, x_last):
        hn = o.rmsnorm2(x_last, self.w.f16("g_final"))
        return o.matmul_f16_nk(hn, self.w.embed(), self.threads)[0]

    def prefill(self, x: np.ndarray) -> np.ndarray:
        """x [S, hidden] fp16 embeddings -> logits of the last token [vocab]."""
        c = self.cfg
        S = x.shape[0]
        for l in range(c.layers):
            h = o.rmsnorm2(x, self.w.f16(f"{l}.g_attn"))
            qr, kr, v = self._qk(h, l, S)
            for t in range(S):
                self.rings[l].append(kr[t], v[t])
            a = o.attn_prefill(qr.reshape(S, c.heads, c.head_dim), kr.reshape(S, c.kv_heads, c.head_dim),
                               v.reshape(S, c.kv_heads, c.head_dim), c.scale, True,
                               threads=self.threads).reshape(S, c.q_dim)
            x1 = o.binary(x, self._lin(a, l, "wo"), 0)
            x = self._ffn(x1, l)
        self.pos += S
        return self._head(x[-1:])

    def decode(self, x: np.ndarray) -> np.ndarray:
        """x [hidden] fp16 embedding of the next token -> logits [vocab]."""
        c = self.cfg
        x = x.reshape(1, c.hidden)
        for l in range(c.layers):
            h = o.rmsnorm2(x, self.w.f16(f"{l}.g_attn"))
            qr, kr, v = self._qk(h, l, 1)
            self.rings[l].append(kr[0], v[0])
            a = self.rings[l].attn_decode(qr[0], self.pos + 1, c.heads, c.kv_heads, c.head_dim,
                                          c.scale).reshape(1, c.q_dim)
            x1 = o.binary(x, self._lin(a, l, "wo"), 0)
            x = self._ffn(x1, l)
        self.pos += 1
        return self._head(x)
