"""Pins of the CPU oracle: each restated function is checked against something that
fixes its result independently — numpy's IEEE casts, closed forms, brute force,
or the reference's own C sources compiled as they lie (oracle/_ref)."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from helpers import cosine, normal_f16, w4g_weights
from oracle.oracle import REF as _REF


# ---------------------------------------------------------------- f16 --------
def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_f32_to_f16_rne(oracle):
    rng = np.random.default_rng(0)
    # every exponent, random mantissas, plus exact halfway points and the carry cases
    exps = np.arange(0, 255, dtype=np.uint32)
    man = rng.integers(0, 1 << 23, size=(255, 600), dtype=np.uint32)
    man[:, :8] = [0, 0x1000, 0x3000, 0x2000, 0x7FFFFF, 0x7FF000, 0x1FFF, 0x800000 - 0x1000]
    bits = (exps[:, None] << 23) | (man & 0x7FFFFF)
    bits = np.concatenate([bits.ravel(), bits.ravel() | 0x80000000])
    x = bits.view(np.float32)
    got = oracle.f32_to_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_nan_maps_to_inf(oracle):
    """The reference drops NaN payloads and returns Inf (oplist_exec.c:401)."""
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 1e9, -1e9], np.float32)
    got = oracle.f32_to_f16(x)
    assert list(got) == [0x7C00, 0xFC00, 0x7C00, 0xFC00, 0x7C00, 0xFC00]


# ---------------------------------------------------------------- W4G --------
def test_w4g_pack_layout_and_round_trip(oracle):
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(32, 128), dtype=np.int8)
    wq = oracle.w4g_pack(q)
    # byte j of row n: low nibble k=2j, high nibble k=2j+1, stored q+8
    lo = (q[:, 0::2].astype(np.int32) + 8)
    hi = (q[:, 1::2].astype(np.int32) + 8)
    assert np.array_equal(wq, (lo | (hi << 4)).astype(np.uint8))
    assert np.array_equal(oracle.w4g_unpack(wq, 128), q)


def test_w4g_dequant_closed_form(oracle):
    rng = np.random.default_rng(2)
    N, K = 48, 256
    q, wq, ws = w4g_weights(rng, N, K)
    ws[0] = np.float16(6.1e-5)      # products in the f16 subnormal range
    ws[1] = np.float16(9000.0)      # products that overflow to inf (q*s > 65504)
    ws[2] = np.float16(-0.0)
    got = oracle.w4g_dequant(wq, ws, K)
    s = np.repeat(ws.astype(np.float32), 64, axis=1)
    ref = (q.astype(np.float32) * s).astype(np.float16)     # q*s exact in f32, one RNE
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


# ---------------------------------------------------------------- matmul -----
def test_matmul_f16_identity_and_one_hot(oracle):
    rng = np.random.default_rng(3)
    M, K = 5, 64
    a = normal_f16(rng, M, K)
    eye = np.eye(K, dtype=np.float16)
    for flags in (0, 2):   # w stored [K,N] or [N,K]; identity is symmetric
        y = oracle.matmul_f16(a.ravel(), eye.ravel(), M, K, K, flags=flags).reshape(M, K)
        assert np.array_equal(y, a)
    # one-hot column picks one input column exactly
    w = np.zeros((K, 3), np.float16)
    w[[7, 0, 63], [0, 1, 2]] = 1
    y = oracle.matmul_f16(a.ravel(), w.ravel(), M, K, 3).reshape(M, 3)
    assert np.array_equal(y, a[:, [7, 0, 63]])


def test_matmul_f16_layouts_vs_float64(oracle):
    """t0/t1/batched/SPLIT index formulas (kernels/host/test_gemv_f16.c:73-175) against
    a float64 product, within the accumulated-rounding bound."""
    rng = np.random.default_rng(4)
    M, K, N = 7, 96, 40
    a = normal_f16(rng, M, K)
    w = normal_f16(rng, K, N)
    ref = a.astype(np.float64) @ w.astype(np.float64)
    bound = 2 * K * 2**-24 * (np.abs(a).astype(np.float64) @ np.abs(w).astype(np.float64)) + np.abs(ref) * 2**-11
    cases = {0: (a, w), 1: (a.T.copy(), w), 2: (a, w.T.copy()), 3: (a.T.copy(), w.T.copy())}
    for flags, (aa, ww) in cases.items():
        y = oracle.matmul_f16(aa.ravel(), ww.ravel(), M, K, N, flags=flags).reshape(M, N)
        assert (np.abs(y.astype(np.float64) - ref) <= bound + 1e-12).all(), flags
    # batched (Bn=3) == three separate products
    Bn = 3
    ab = normal_f16(rng, Bn, M, K)
    wb = normal_f16(rng, Bn, N, K)
    yb = oracle.matmul_f16(ab.ravel(), wb.ravel(), M, K, N, flags=(Bn << 16) | 4 | 2).reshape(Bn, M, N)
    for b in range(Bn):
        yy = oracle.matmul_f16(ab[b].ravel(), wb[b].ravel(), M, K, N, flags=2).reshape(M, N)
        assert np.array_equal(yb[b], yy)
    # SPLIT: chunks [0,16) + [16,40) == the whole op, byte for byte (test_wtop_emit.cpp:556-596)
    whole = oracle.matmul_f16(a.ravel(), w.ravel(), M, K, N).reshape(M, N)
    y = np.zeros(M * N, np.float16)
    y = oracle.matmul_f16(a.ravel(), w.ravel(), M, K, N, 0, 16, 0, out=y)
    y = oracle.matmul_f16(a.ravel(), w.ravel(), M, K, N, 16, 24, 0, out=y)
    assert np.array_equal(y.reshape(M, N), whole)


def test_matmul_w4g_threads_bit_identical(oracle):
    rng = np.random.default_rng(5)
    _, wq, ws = w4g_weights(rng, 300, 256)
    a = normal_f16(rng, 3, 256)
    y1 = oracle.matmul_w4g(a, wq, ws, threads=1)
    y8 = oracle.matmul_w4g(a, wq, ws, threads=8)
    assert np.array_equal(y1.view(np.uint16), y8.view(np.uint16))
    # and equals the plain OP_MATMUL_F16 scalar loop on the dequantized weights
    w = oracle.w4g_dequant(wq, ws, 256)
    y = oracle.matmul_f16(a.ravel(), w.ravel(), 3, 256, 300, flags=2).reshape(3, 300)
    assert np.array_equal(y1.view(np.uint16), y.view(np.uint16))


# ---------------------------------------------------------------- rmsnorm ----
def test_rmsnorm2_closed_forms(oracle):
    rw = 256
    gamma = np.linspace(0.8, 1.2, rw).astype(np.float16)
    beta = np.linspace(-0.1, 0.1, rw).astype(np.float16)
    x = np.zeros((3, rw), np.float16)
    x[1] = np.float16(2.0)
    x[2] = np.float16(-0.5)
    y = oracle.rmsnorm2(x, gamma, beta).astype(np.float64)
    assert np.array_equal(y[0], beta.astype(np.float64))          # zero row -> bias
    for r, c in ((1, 2.0), (2, -0.5)):                             # constant row
        expect = np.sign(c) / math.sqrt(1 + 1e-6 / (c * c)) * gamma.astype(np.float64) + beta
        assert np.abs(y[r] - expect).max() <= 2e-3


def test_rmsnorm2_vs_float64(oracle):
    rng = np.random.default_rng(6)
    x = normal_f16(rng, 64, 1024)
    g = rng.uniform(0.8, 1.2, 1024).astype(np.float16)
    y = oracle.rmsnorm2(x, g).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * g.astype(np.float64)
    ulp = np.abs(ref) * 2**-10 + 2**-24
    assert (np.abs(y - ref) <= ulp).all()


# ---------------------------------------------------------------- softmax ----
def test_softmax_properties(oracle):
    rng = np.random.default_rng(7)
    for n in (64, 100):
        x = (rng.standard_normal((8, n)) * 4).astype(np.float16)
        y = oracle.softmax(x, 8, n).astype(np.float64)
        assert np.allclose(y.sum(1), 1.0, atol=3e-3)
        ys = oracle.softmax((x.astype(np.float32) + 3).astype(np.float16), 8, n)
        assert np.abs(ys.astype(np.float64) - y).max() <= 2e-3     # shift invariance
    one = np.full((1, 64), -60000, np.float16)
    one[0, 17] = 0
    assert np.array_equal(oracle.softmax(one, 1, 64)[0], np.eye(64, dtype=np.float16)[17])


@pytest.mark.skipif(not (_REF / "libref_softmax.so").exists(),
                    reason="oracle/_ref not built (reference tree absent)")
def test_softmax_host_form_matches_reference_source(oracle):
    """go_softmax_host == the reference's hvhx_v2_softmax_f32 host body (hvx_softmax.c:81-93)
    compiled from its own source, wrapped in exec_softmax's f16->f32->f16 conversions."""
    ref = C.CDLL(str(oracle.REF / "libref_softmax.so"))
    ref.hvhx_v2_softmax_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
    rng = np.random.default_rng(8)
    rows, n = 16, 256
    x = (rng.standard_normal((rows, n)) * 5).astype(np.float16)
    got = oracle.softmax(x, rows, n, form="host")
    xf = oracle.f16_to_f32(x.view(np.uint16))
    out = np.empty_like(xf)
    pad = np.empty(n, np.float32)
    for r in range(rows):
        src = np.ascontiguousarray(xf[r])
        dst = np.empty(n, np.float32)
        ref.hvhx_v2_softmax_f32(src.ctypes.data, dst.ctypes.data, pad.ctypes.data, n)
        out[r] = dst
    expect = oracle.f32_to_f16(out)
    assert np.array_equal(got.view(np.uint16), expect)


# ---------------------------------------------------------------- KV ring ----
@pytest.mark.skipif(not (_REF / "libref_kvcache.so").exists(),
                    reason="oracle/_ref not built (reference tree absent)")
def test_kv_ring_matches_reference_kvcache(oracle):
    """The oracle ring == kvcache.c (compiled from the reference source) byte for byte,
    including wrap-around: slot = pos % nslots, lookup hit iff posmap[slot] == pos."""

    class Kvc(C.Structure):
        _fields_ = [("base", C.c_void_p), ("slot_bytes", C.c_uint32), ("nslots", C.c_uint32),
                    ("posmap", C.c_void_p), ("consumer", C.c_int), ("mem", C.c_int),
                    ("n_append", C.c_uint32), ("n_evict", C.c_uint32)]

    ref = C.CDLL(str(oracle.REF / "libref_kvcache.so"))
    ref.kvc_init.argtypes = [C.POINTER(Kvc), C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
    ref.kvc_append.argtypes = [C.POINTER(Kvc), C.c_void_p, C.c_void_p, C.c_uint32]
    ref.kvc_lookup.argtypes = [C.POINTER(Kvc), C.c_uint32]
    kv_elems, nslots = 256, 6
    state = nslots * kv_elems * 4
    buf = np.zeros(state + 128, np.uint8)
    base = (buf.ctypes.data + 127) // 128 * 128
    off = base - buf.ctypes.data
    posmap = np.zeros(nslots, np.uint32)
    c = Kvc()
    assert ref.kvc_init(C.byref(c), base, kv_elems * 4, nslots, posmap.ctypes.data) == 0
    ring = oracle.KVRing(state, kv_elems)
    rng = np.random.default_rng(9)
    for pos in [0, 1, 2, 3, 4, 5, 6, 7, 9, 3]:
        k, v = normal_f16(rng, kv_elems), normal_f16(rng, kv_elems)
        assert ref.kvc_append(C.byref(c), k.ctypes.data, v.ctypes.data, pos) == ring.append(k, v, pos)
        assert np.array_equal(buf[off:off + state], ring.buf)
        assert np.array_equal(posmap, ring.posmap)
        for p in range(12):
            hit = ref.kvc_lookup(C.byref(c), p)
            assert (hit >= 0) == (ring.posmap[p % nslots] == p)


def test_kv_gather_gqa_round_trip(oracle):
    rng = np.random.default_rng(10)
    H, KVH, hd, n = 8, 2, 128, 5
    ring = oracle.KVRing(16 * KVH * hd * 4, KVH * hd)
    ks = normal_f16(rng, n, KVH, hd)
    vs = normal_f16(rng, n, KVH, hd)
    for t in range(n):
        ring.append(ks[t].ravel(), vs[t].ravel())
    kT, vo = ring.gather(n, H, KVH, hd, pstride=16)
    for h in range(H):
        assert np.array_equal(kT[h, :, :n], ks[:, h // 4, :].T)
        assert np.array_equal(vo[h, :n], vs[:, h // 4, :])
    assert not kT[:, :, n:].any() and not vo[:, n:].any()


# ---------------------------------------------------------------- attention --
def test_attention_one_key_rows_and_decode_equivalence(oracle):
    rng = np.random.default_rng(11)
    S, H, KVH, hd = 24, 4, 2, 128
    scale = float(np.float16(1 / math.sqrt(hd)))
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, KVH, hd), normal_f16(rng, S, KVH, hd)
    out = oracle.attn_prefill(q, k, v, scale, True)
    for h in range(H):
        assert np.array_equal(out[0, h], v[0, h // 2])     # causal row 0 sees one key
    ring = oracle.KVRing(32 * KVH * hd * 4, KVH * hd)
    for t in range(S):
        ring.append(k[t].ravel(), v[t].ravel())
    for t in (5, S - 1):
        dec = ring.attn_decode(q[t], t + 1, H, KVH, hd, scale)
        assert cosine(dec, out[t]) >= 0.9999
        assert np.abs(dec.astype(np.float32) - out[t].astype(np.float32)).max() <= 2e-2


def test_attention_vs_float64(oracle):
    rng = np.random.default_rng(12)
    S, H, KVH, hd = 40, 2, 1, 128
    scale = float(np.float16(1 / math.sqrt(hd)))
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, KVH, hd), normal_f16(rng, S, KVH, hd)
    out = oracle.attn_prefill(q, k, v, scale, True).astype(np.float64)
    for h in range(H):
        s = q[:, h].astype(np.float64) @ k[:, 0].astype(np.float64).T * scale
        s[np.triu(np.ones((S, S), bool), 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref = p @ v[:, 0].astype(np.float64)
        assert np.abs(out[:, h] - ref).max() <= 2e-2
        assert cosine(out[:, h], ref) >= 0.9999


# ---------------------------------------------------------------- rope -------
def test_rope_identity_at_zero_and_pair_norm(oracle):
    rng = np.random.default_rng(13)
    x = normal_f16(rng, 1, 4 * 128)
    assert np.array_equal(oracle.rope(x, 4, 128, 0, 1e6), x)
    y = oracle.rope(np.repeat(x, 3, 0), 4, 128, 77, 1e6).astype(np.float64)
    xr = x.astype(np.float64).reshape(4, 2, 64)
    yr = y[0].reshape(4, 2, 64)
    assert np.abs(np.hypot(yr[:, 0], yr[:, 1]) - np.hypot(xr[:, 0], xr[:, 1])).max() <= 1e-2
    # hand-rolled float64 rotation of one pair
    inv = 1.0 / 1e6 ** (2 * 5 / 128)
    c, s = np.float16(math.cos(77 * inv)), np.float16(math.sin(77 * inv))
    x1, x2 = x[0, 5], x[0, 5 + 64]
    e1 = np.float16(np.float16(x1 * np.float32(c)) + np.float16(-x2 * np.float32(s)))
    assert y[0, 5] == e1


def test_argmax_first_max(oracle):
    x = np.array([1, 3, 3, -np.inf, 2], np.float16)
    assert oracle.argmax(x) == 1
    assert oracle.argmax(np.full(4, -np.inf, np.float16)) == 0
