"""numpy front end of the C oracle (TEST INFRASTRUCTURE — the checker, never the product).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
Arrays in and out are numpy float16 (bit-identical to the C uint16 buffers).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF = HERE / "_ref"

_lib = None


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        _p = C.c_void_p
        u = C.c_uint32
        sig = {
            "go_f16_to_f32": (C.c_float, [C.c_uint16]),
            "go_f32_to_f16": (C.c_uint16, [C.c_float]),
            "go_f16_to_f32_n": (None, [_p, _p, C.c_size_t]),
            "go_f32_to_f16_n": (None, [_p, _p, C.c_size_t]),
            "go_w4g_pack": (None, [_p, u, u, _p]),
            "go_w4g_unpack": (None, [_p, u, u, _p]),
            "go_w4g_dequant": (C.c_int, [_p, _p, u, u, u, _p]),
            "go_matmul_f16": (C.c_int, [_p, _p, _p, u, u, u, u, u, u]),
            "go_matmul_w4g": (C.c_int, [_p, _p, _p, _p, u, u, u, u, C.c_int]),
            "go_matmul_f16_nk_mt": (C.c_int, [_p, _p, _p, u, u, u, C.c_int]),
            "go_matmul_w4g_ref": (C.c_int, [_p, _p, _p, _p, u, u, u, u, C.c_int]),
            "go_matmul_f16_nk_ref": (C.c_int, [_p, _p, _p, u, u, u, C.c_int]),
            "go_fast_available": (C.c_int, []),
            "go_fast_disable": (None, [C.c_int]),
            "go_set_order": (C.c_int, [C.c_int]),
            "go_attn_prefill_mt": (C.c_int, [_p, _p, _p, _p, u, u, u, u, C.c_float, C.c_int, C.c_int]),
            "go_attn_prefill_ref": (C.c_int, [_p, _p, _p, _p, u, u, u, u, C.c_float, C.c_int]),
            "go_attn_decode_ring": (C.c_int, [_p, _p, u, u, _p, _p, u, u, u, u, C.c_float]),
            "go_rmsnorm2": (C.c_int, [_p, _p, _p, _p, u, u]),
            "go_softmax_scalar": (None, [_p, _p, u, u]),
            "go_softmax_host": (None, [_p, _p, u, u]),
            "go_softmax": (None, [_p, _p, u, u]),
            "go_binary": (C.c_int, [_p, _p, _p, u, u]),
            "go_unary": (C.c_int, [_p, _p, u, u]),
            "go_argmax": (C.c_int32, [_p, u]),
            "go_attn_prefill": (C.c_int, [_p, _p, _p, _p, u, u, u, u, C.c_float, C.c_int]),
            "go_rope": (C.c_int, [_p, _p, u, u, u, u, C.c_float, u]),
            "go_crouton_encode": (C.c_int, [_p, _p, u, u]),
            "go_crouton_decode": (C.c_int, [_p, _p, u, u]),
            "go_matmul_w4a16": (C.c_int, [_p, _p, _p, u, u, u]),
            "go_rmsnorm_crouton": (C.c_int, [_p, _p, _p, u, u]),
            "go_concat": (C.c_int, [_p, _p, u, u, _p]),
            "go_split": (C.c_int, [_p, u, _p, u, _p, u]),
            "go_reduce": (C.c_int, [_p, _p, u, u, u, _p]),
            "go_pad": (C.c_int, [_p, _p, u, u, u, u, C.c_uint16]),
            "go_cumsum": (C.c_int, [_p, _p, u, u, u, u]),
            "go_gather": (C.c_int, [_p, _p, _p, u, u, _p, _p]),
            "go_transpose4": (C.c_int, [_p, _p, u, u, u, u]),
            "go_broadcast": (C.c_int, [_p, _p, u, _p, _p]),
            "go_transpose_gen": (C.c_int, [_p, _p, u, _p, u]),
            "go_slice": (C.c_int, [_p, _p, u, u, _p, _p, _p, _p]),
        }
        for name, (res, args) in sig.items():
            f = getattr(_lib, name)
            f.restype, f.argtypes = res, args
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return a.ctypes.data


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


# ---- conversions ----
def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().go_f16_to_f32_n(_p(bits), _p(out), bits.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().go_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


# ---- W4G ----
def w4g_pack(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    N, K = q.shape
    out = np.empty((N, K // 2), np.uint8)
    lib().go_w4g_pack(_p(q), N, K, _p(out))
    return out


def w4g_unpack(wq: np.ndarray, K: int) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    N = wq.shape[0]
    out = np.empty((N, K), np.int8)
    lib().go_w4g_unpack(_p(wq), N, K, _p(out))
    return out


def w4g_dequant(wq: np.ndarray, ws: np.ndarray, K: int, group: int = 64) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    ws = _h(ws)
    N = wq.shape[0]
    out = np.empty((N, K), np.float16)
    if lib().go_w4g_dequant(_p(wq), _p(ws), N, K, group, _p(out)):
        raise ValueError("bad w4g shape")
    return out


# ---- linears ----
def matmul_f16(a, w, M, K, N_full, n0=0, N=None, flags=0, out=None) -> np.ndarray:
    a, w = _h(a), _h(w)
    N = N_full if N is None else N
    Bn = max(flags >> 16, 1) if flags & 4 else 1
    y = _h(out) if out is not None else np.zeros(Bn * M * N_full, np.float16)
    lib().go_matmul_f16(_p(a), _p(w), _p(y), M, K, N_full, n0, N, flags)
    return y


def matmul_w4g(a, wq, ws, threads: int = 1, form: str = "fast") -> np.ndarray:
    """y = a . dequant(W)^T (OP_MATMUL_F16 scalar arithmetic on fp16(q*s)); form "ref"
    runs the scalar restatement, "fast" its vectorised, bit-identical form."""
    a = _h(a)
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    ws = _h(ws)
    M, K = a.shape
    N = wq.shape[0]
    y = np.empty((M, N), np.float16)
    fn = lib().go_matmul_w4g if form == "fast" else lib().go_matmul_w4g_ref
    if fn(_p(a), _p(wq), _p(ws), _p(y), M, K, N, 64, threads):
        raise ValueError("bad w4g shape")
    return y


def matmul_f16_nk(a, w, threads: int = 1, form: str = "fast") -> np.ndarray:
    """y = a . w^T with w [N, K] fp16 (the lm_head form), sequential-k arithmetic."""
    a, w = _h(a), _h(w)
    M, K = a.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float16)
    fn = lib().go_matmul_f16_nk_mt if form == "fast" else lib().go_matmul_f16_nk_ref
    if fn(_p(a), _p(w), _p(y), M, K, N, threads):
        raise MemoryError("matmul_f16_nk")
    return y


def fast_available() -> bool:
    return bool(lib().go_fast_available())


class summation_order:
    """Context manager: run the vector forms in fp32 summation order `mode` (0 = the
    scalar restatement's sequential order; 1 = 32-wide slices combined pairwise; 2 =
    16-wide slices combined in sequence; attention's P.V in 64-key chunks) with the same
    f16 rounding points, to measure how far a correct implementation may move with the
    order alone. Raises when the vector forms are unavailable."""

    def __init__(self, mode: int):
        self.mode = mode

    def __enter__(self):
        if lib().go_set_order(self.mode):
            raise RuntimeError(f"summation order {self.mode} unavailable (needs the AVX2/F16C forms)")
        return self

    def __exit__(self, *exc):
        lib().go_set_order(0)
        return False


# ---- rows ----
def rmsnorm2(x, gamma, beta=None) -> np.ndarray:
    x, gamma = _h(x), _h(gamma)
    rw = gamma.size
    y = np.empty(x.shape, np.float16)
    b = _h(beta) if beta is not None else None
    if lib().go_rmsnorm2(_p(x), _p(gamma), _p(b) if b is not None else None, _p(y), x.size, rw):
        raise ValueError("bad rmsnorm shape")
    return y


def softmax(x, rows, n, form: str = "dispatch") -> np.ndarray:
    x = _h(x)
    y = np.empty(x.shape, np.float16)
    fn = {"dispatch": lib().go_softmax, "scalar": lib().go_softmax_scalar,
          "host": lib().go_softmax_host}[form]
    fn(_p(x), _p(y), rows, n)
    return y


def binary(a, b, subtype: int) -> np.ndarray:
    a, b = _h(a), _h(b)
    y = np.empty(a.shape, np.float16)
    lib().go_binary(_p(a), _p(b), _p(y), a.size, subtype)
    return y


def unary(x, subtype: int) -> np.ndarray:
    x = _h(x)
    y = np.empty(x.shape, np.float16)
    lib().go_unary(_p(x), _p(y), x.size, subtype)
    return y


def argmax(x) -> int:
    x = _h(x)
    return int(lib().go_argmax(_p(x), x.size))


def attn_prefill(q, k, v, scale: float, causal: bool = True, threads: int = 1,
                 form: str = "fast") -> np.ndarray:
    """q [S,H,hd], k/v [S,KVH,hd] -> [S,H,hd], reference runlist composition
    (form "ref": the scalar restatement; "fast": vectorised, heads over threads)."""
    q, k, v = _h(q), _h(k), _h(v)
    S, H, hd = q.shape
    KVH = k.shape[1]
    out = np.empty_like(q)
    if form == "fast":
        rc = lib().go_attn_prefill_mt(_p(q), _p(k), _p(v), _p(out), S, H, KVH, hd, scale, int(causal), threads)
    else:
        rc = lib().go_attn_prefill_ref(_p(q), _p(k), _p(v), _p(out), S, H, KVH, hd, scale, int(causal))
    if rc:
        raise ValueError("bad attention shape")
    return out


def rope(x, n_heads: int, hd: int, pos0: int, theta: float, row_stride: int | None = None) -> np.ndarray:
    x = _h(x)
    n_tok = x.shape[0]
    row_stride = row_stride or n_heads * hd
    y = x.copy()
    lib().go_rope(_p(x), _p(y), n_tok, n_heads, hd, pos0, theta, row_stride)
    return y


class KVRing:
    """The reference KV ring (kvcache.c) restated: slot = pos % nslots, [K | V] faces."""

    def __init__(self, state_bytes: int, kv_elems: int):
        self.slot_bytes = kv_elems * 4
        if self.slot_bytes < 256 or self.slot_bytes % 128 or state_bytes % self.slot_bytes:
            raise ValueError("kv geometry bad")
        self.kv_elems = kv_elems
        self.nslots = state_bytes // self.slot_bytes
        self.buf = np.zeros(state_bytes, np.uint8)
        self.posmap = np.full(self.nslots, 0xFFFFFFFF, np.uint32)
        self.count = 0

    def append(self, k, v, pos: int | None = None) -> int:
        if pos is None:
            if self.count >= self.nslots:
                raise OverflowError("kv ring full")
            pos = self.count
            self.count += 1
        slot = pos % self.nslots
        half = self.slot_bytes // 2
        base = slot * self.slot_bytes
        self.buf[base:base + half] = _h(k).view(np.uint8).ravel()
        self.buf[base + half:base + 2 * half] = _h(v).view(np.uint8).ravel()
        self.posmap[slot] = pos
        return slot

    def gather(self, n_kv: int, H: int, KVH: int, hd: int, pstride: int | None = None):
        """(kT [H, hd, pstride], v [H, pstride, hd]) with GQA expansion kv = h // (H/KVH)."""
        pstride = pstride or n_kv
        kT = np.zeros((H, hd, pstride), np.float16)
        vo = np.zeros((H, pstride, hd), np.float16)
        rep = H // KVH
        for p in range(n_kv):
            slot = p % self.nslots
            if self.posmap[slot] != p:
                raise KeyError(f"kv gather miss pos {p}")
            face = self.buf[slot * self.slot_bytes:(slot + 1) * self.slot_bytes].view(np.float16)
            kf = face[:KVH * hd].reshape(KVH, hd)
            vf = face[KVH * hd:].reshape(KVH, hd)
            for h in range(H):
                kT[h, :, p] = kf[h // rep]
                vo[h, p, :] = vf[h // rep]
        return kT, vo

    def attn_decode(self, q, n_kv: int, H: int, KVH: int, hd: int, scale: float) -> np.ndarray:
        """One-token attention over positions [0, n_kv) as the reference decode chain
        computes it (go_attn_decode's arithmetic, vectorised in C)."""
        q = _h(q).reshape(H, hd)
        out = np.empty((H, hd), np.float16)
        rc = lib().go_attn_decode_ring(_p(self.buf), _p(self.posmap), self.nslots, self.slot_bytes, _p(q),
                                       _p(out), n_kv, H, KVH, hd, scale)
        if rc == -2:
            raise KeyError("kv gather miss")
        if rc:
            raise ValueError("bad decode attention shape")
        return out

    def attn_decode_chain(self, q, n_kv: int, H: int, KVH: int, hd: int, scale: float) -> np.ndarray:
        """The same, op by op: KV_GATHER, MATMUL_F16, BINARY mul, SOFTMAX, MATMUL_F16
        (scripts/surgery_decode_graph.py:143-168), each an oracle op with f16 output."""
        kT, vo = self.gather(n_kv, H, KVH, hd)
        q = _h(q).reshape(H, hd)
        out = np.empty((H, hd), np.float16)
        sc = np.float16(scale)
        for h in range(H):
            s = matmul_f16(q[h], kT[h], 1, hd, n_kv)
            s = binary(s, np.full(n_kv, sc, np.float16), 2)
            p = softmax(s, 1, n_kv)
            out[h] = matmul_f16(p, vo[h], 1, n_kv, hd)
        return out


# ---- remaining runlist ops (gehtp_oracle_ops.c) ----
def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def crouton_encode(lin) -> np.ndarray:
    """crouton16_row4 surface (flat u16) of a row-major [rows, cols] u16 array."""
    lin = _u16(lin)
    rows, cols = lin.shape
    out = np.empty(rows * cols, np.uint16)
    if lib().go_crouton_encode(_p(lin), _p(out), rows, cols):
        raise ValueError("crouton shape must be multiples of 32")
    return out


def crouton_decode(surf, rows: int, cols: int) -> np.ndarray:
    surf = _u16(surf).ravel()
    out = np.empty((rows, cols), np.uint16)
    if lib().go_crouton_decode(_p(surf), _p(out), rows, cols):
        raise ValueError("crouton shape must be multiples of 32")
    return out


def w4a16_pack(w_nk) -> np.ndarray:
    """W [N, K] int values in [-8, 7] -> the K*N/2-byte slot ([N][K/2], +8 nibbles)."""
    return w4g_pack(np.asarray(w_nk, np.int8)).ravel()


def matmul_w4a16(act_surf, w_slot, M: int, K: int, N: int) -> np.ndarray:
    """OP_MATMUL_W4A16: crouton u16 surface [M,N] from crouton act [M,K] and the W slot."""
    a = _u16(act_surf).ravel()
    w = np.ascontiguousarray(w_slot, np.uint8).ravel()
    out = np.empty(M * N, np.uint16)
    if lib().go_matmul_w4a16(_p(a), _p(w), _p(out), M, K, N):
        raise ValueError("matmul_w4a16 shape")
    return out


def rmsnorm_crouton(x_surf, w, m: int, n: int) -> np.ndarray:
    """OP_RMSNORM_F16 on a crouton u16 surface: row-major f16 [m, n]."""
    x = _u16(x_surf).ravel()
    wv = _h(w)
    y = np.empty((m, n), np.float16)
    if lib().go_rmsnorm_crouton(_p(x), _p(wv), _p(y), m, n):
        raise ValueError("rmsnorm shape")
    return y


def concat(segs, outer: int) -> np.ndarray:
    segs = [_h(s) for s in segs]
    sizes = (C.c_uint32 * 4)(*([s.size // outer for s in segs] + [0] * (4 - len(segs))))
    ptrs = (C.c_void_p * 4)(*([_p(s) for s in segs] + [None] * (4 - len(segs))))
    n = sum(s.size for s in segs)
    y = np.empty(n, np.float16)
    if lib().go_concat(C.cast(ptrs, C.c_void_p), _p(y), len(segs), n, C.cast(sizes, C.c_void_p)):
        raise ValueError("concat shape")
    return y


def split(x, sizes, index: int) -> np.ndarray:
    x = _h(x).ravel()
    sz = (C.c_uint32 * 4)(*(list(sizes) + [0] * (4 - len(sizes))))
    outer = x.size // sum(sizes)
    y = np.empty(outer * sizes[index], np.float16)
    if lib().go_split(_p(x), x.size, _p(y), len(sizes), C.cast(sz, C.c_void_p), index):
        raise ValueError("split shape")
    return y


def reduce(x, dims, axis: int, subtype: int) -> np.ndarray:
    x = _h(x).ravel()
    d = (C.c_uint32 * 4)(*dims)
    if not 0 <= axis < 4:
        raise ValueError("reduce axis")
    L = dims[axis] or 1
    inner = int(np.prod(dims[axis + 1:])) if axis < 3 else 1
    y = np.empty(x.size // (L * inner) * inner, np.float16)
    if lib().go_reduce(_p(x), _p(y), x.size, axis, subtype, C.cast(d, C.c_void_p)):
        raise ValueError("reduce geometry")
    return y


def pad(x, outer: int, in_inner: int, out_inner: int, before: int, value) -> np.ndarray:
    x = _h(x).ravel()
    y = np.empty(outer * out_inner, np.float16)
    pv = int(np.float16(value).view(np.uint16))
    if lib().go_pad(_p(x), _p(y), outer, in_inner, out_inner, before, pv):
        raise ValueError("pad geometry")
    return y


def cumsum(x, rows: int, n: int, exclusive: bool = False, reverse: bool = False) -> np.ndarray:
    x = _h(x).ravel()
    y = np.empty(rows * n, np.float16)
    lib().go_cumsum(_p(x), _p(y), rows, n, int(exclusive), int(reverse))
    return y


def gather(tbl, idx, td, xd, axis: int) -> np.ndarray:
    """OP_GATHER_F16 with tbl dims td (irank = len(td)) and index dims xd."""
    tbl = _h(tbl).ravel()
    idx = np.ascontiguousarray(idx, np.int32).ravel()
    irank, xrank = len(td), len(xd)
    tdv = (C.c_uint32 * 5)(*(list(td) + [1] * (5 - irank)))
    xdv = (C.c_uint32 * 5)(*(list(xd) + [1] * (5 - xrank)))
    od = list(td[:axis]) + list(xd) + list(td[axis + 1:])
    n = int(np.prod(od))
    y = np.empty(n, np.float16)
    packed = axis | (xrank << 8) | (irank << 16)
    if lib().go_gather(_p(tbl), _p(idx), _p(y), n, packed, C.cast(tdv, C.c_void_p), C.cast(xdv, C.c_void_p)):
        raise ValueError("gather rank/axis")
    return y


def transpose4(x, Hh: int, W: int, Cc: int, perm) -> np.ndarray:
    x = _h(x).ravel()
    y = np.empty(x.size, np.float16)
    pv = perm[0] | (perm[1] << 8) | (perm[2] << 16) | (perm[3] << 24)
    if lib().go_transpose4(_p(x), _p(y), Hh, W, Cc, pv):
        raise ValueError("transpose perm")
    return y


def _u32v(vals, n):
    v = list(vals) + [1] * (n - len(vals))
    return (C.c_uint32 * n)(*v)


def broadcast(x, in_d, out_d) -> np.ndarray:
    """OP_BROADCAST_F16: x (in_d elements) -> out_d (up to 4 dims each)."""
    x = _h(x)
    n = int(np.prod(out_d))
    y = np.empty(n, np.float16)
    lib().go_broadcast(_p(x), _p(y), n, C.cast(_u32v(in_d, 4), C.c_void_p), C.cast(_u32v(out_d, 4), C.c_void_p))
    return y


def transpose_gen(x, dims, perm) -> np.ndarray:
    """OP_TRANSPOSE_GEN_F16: x [dims] (rank 2..4), output axis i = input axis perm[i]."""
    x = _h(x)
    rk = len(dims)
    pv = sum(int(p) << (8 * i) for i, p in enumerate(perm))
    y = np.empty(int(np.prod(dims)), np.float16)
    if lib().go_transpose_gen(_p(x), _p(y), rk, C.cast(_u32v(dims, 4), C.c_void_p), pv):
        raise ValueError("transpose_gen rank")
    return y


def strided_slice(x, n_out, b, e, s, d) -> np.ndarray:
    """OP_STRIDED_SLICE_F16 (rank len(d) <= 3)."""
    x = _h(x)
    rk = len(d)
    y = np.empty(n_out, np.float16)
    args = [C.cast(_u32v(v, 3), C.c_void_p) for v in (b, e, s, d)]
    if lib().go_slice(_p(x), _p(y), n_out, rk, *args):
        raise ValueError("slice rank")
    return y
