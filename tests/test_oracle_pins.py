"""Pins of the oracle functions the E2E and epilogue checks rest on (CPU only):

- go_unary / go_binary against the reference's own element-wise kernels, hvx_unary.c and
  hvx_binary.c, compiled from source as they lie (oracle/_ref), on the path exec_unary /
  exec_binary take for n >= 32 (oplist_exec.c:1021-1045, 1126-1145), exhaustively over
  every f16 input for the unary subtypes that path covers; and every subtype of the
  scalar path (n < 32, oplist_exec.c:1047-1078, 1143-1158) against float64 closed forms;
- the vectorised oracle linears (go_matmul_w4g, go_matmul_f16_nk_mt) against the scalar
  OP_MATMUL_F16 restatement go_matmul_f16 (oplist_exec.c:1802-1811) at M = 1 ... 512,
  including the M > 4 shapes of every prefill check;
- vectorised prefill / decode attention against the scalar op-chain forms;
- go_softmax_scalar's rounding point of e (oplist_exec.c:1184-1192) on a hand-computed row.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from oracle import oracle as O

_REF = O.REF
ALL_F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
FINITE_F16 = ALL_F16[(ALL_F16 & 0x7C00) != 0x7C00]


def _bits(a) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint16)


def _ref_lib(name):
    lib = C.CDLL(str(_REF / name))
    return lib


needs_ref = pytest.mark.skipif(not (_REF / "libref_unary.so").exists() or not (_REF / "libref_binary.so").exists(),
                               reason="oracle/_ref not built (reference tree absent)")


def _ref_cvt():
    b = _ref_lib("libref_binary.so")
    b.hvhx_v2_cvt_f16_to_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    b.hvhx_v2_cvt_f32_to_f16.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    return b


def _ref_unary(x_bits: np.ndarray, fn_name: str) -> np.ndarray:
    """exec_unary's n >= 32 path built from the reference's functions: cvt, kernel, cvt."""
    b, u = _ref_cvt(), _ref_lib("libref_unary.so")
    fn = getattr(u, fn_name)
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    n = x_bits.size
    xf = np.empty(n, np.float32)
    b.hvhx_v2_cvt_f16_to_f32(xf.ctypes.data, x_bits.ctypes.data, n)
    fn(xf.ctypes.data, xf.ctypes.data, n)
    y = np.empty(n, np.uint16)
    b.hvhx_v2_cvt_f32_to_f16(y.ctypes.data, xf.ctypes.data, n)
    return y


@needs_ref
@pytest.mark.parametrize("subtype,fn", [(1, "hvhx_v2_exp_f32"), (8, "hvhx_v2_sigmoid_f32"),
                                        (9, "hvhx_v2_tanh_f32"), (12, "hvhx_v2_silu_f32")])
def test_unary_vector_path_matches_reference_source(oracle, subtype, fn):
    x = np.ascontiguousarray(ALL_F16)
    got = _bits(oracle.unary(x.view(np.float16), subtype))
    assert np.array_equal(got, _ref_unary(x, fn)), f"unary {subtype}"


def test_unary_copy_vector_path_is_a_bit_copy(oracle):
    """COPY (14) with n >= 32 is memcpy (oplist_exec.c:1042-1044): NaN payloads survive;
    below 32 elements it is the f16 -> f32 -> f16 round trip (NaN -> Inf)."""
    x = np.ascontiguousarray(ALL_F16)
    assert np.array_equal(_bits(oracle.unary(x.view(np.float16), 14)), x)
    nan = np.array([0x7E01, 0xFD00, 0x3C00], np.uint16)
    assert list(_bits(oracle.unary(nan.view(np.float16), 14))) == [0x7C00, 0xFC00, 0x3C00]


@needs_ref
@pytest.mark.parametrize("subtype,fn", [(0, "hvhx_v2_add_f32"), (1, "hvhx_v2_sub_f32"),
                                        (2, "hvhx_v2_mul_f32"), (3, "hvhx_v2_div_f32")])
def test_binary_vector_path_matches_reference_source(oracle, subtype, fn):
    rng = np.random.default_rng(40 + subtype)
    n = 1 << 18
    a = rng.choice(ALL_F16, n).astype(np.uint16)
    b = rng.choice(ALL_F16, n).astype(np.uint16)
    b[:4096] = rng.choice(np.array([0x0000, 0x8000, 0x7C00, 0xFC00, 0x0001, 0x8001, 0x7BFF], np.uint16), 4096)
    got = _bits(oracle.binary(a.view(np.float16), b.view(np.float16), subtype))
    cv, lib = _ref_cvt(), _ref_lib("libref_binary.so")
    f = getattr(lib, fn)
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
    af, bf, yf = np.empty(n, np.float32), np.empty(n, np.float32), np.empty(n, np.float32)
    cv.hvhx_v2_cvt_f16_to_f32(af.ctypes.data, a.ctypes.data, n)
    cv.hvhx_v2_cvt_f16_to_f32(bf.ctypes.data, b.ctypes.data, n)
    f(yf.ctypes.data, af.ctypes.data, bf.ctypes.data, n)
    want = np.empty(n, np.uint16)
    cv.hvhx_v2_cvt_f32_to_f16(want.ctypes.data, yf.ctypes.data, n)
    assert np.array_equal(got, want), f"binary {subtype}: {int((got != want).sum())} differ"


@needs_ref
def test_reference_f16_conversions_match_oracle(oracle):
    """hvx_binary.c's own f16 <-> f32 conversions (hb_f16_to_f32 / hb_f32_to_f16, host path)
    equal the oracle's (oplist_exec.c:371-418): every f16, and f32 values around every
    f16 rounding boundary."""
    cv = _ref_cvt()
    x = np.ascontiguousarray(ALL_F16)
    want = np.empty(65536, np.float32)
    cv.hvhx_v2_cvt_f16_to_f32(want.ctypes.data, x.ctypes.data, 65536)
    got = oracle.f16_to_f32(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    f = FINITE_F16.view(np.float16).astype(np.float32).view(np.uint32).astype(np.int64)
    probes = np.concatenate([f + d for d in (-1, 0, 1, 0x0FFF, 0x1000, 0x1001, 0x2000)]).astype(np.uint32)
    pf = np.ascontiguousarray(probes.view(np.float32))
    want16 = np.empty(pf.size, np.uint16)
    cv.hvhx_v2_cvt_f32_to_f16(want16.ctypes.data, pf.ctypes.data, pf.size)
    assert np.array_equal(oracle.f32_to_f16(pf), want16)


def _closed(subtype: int, v: np.ndarray) -> np.ndarray:
    """float64 value of each scalar unary subtype (oplist_exec.c:1047-1078)."""
    with np.errstate(all="ignore"):
        return {
            0: -v, 1: np.exp(v), 2: np.where(v >= 0, np.sqrt(np.maximum(v, 0)), 0.0),
            3: np.where(v > 0, 1 / np.sqrt(np.maximum(v, 1e-300)), 0.0),
            4: np.where(v > 0, np.log(np.maximum(v, 1e-300)), 0.0), 5: np.abs(v), 6: np.sin(v), 7: np.cos(v),
            8: 1 / (1 + np.exp(-v)), 9: np.tanh(v),
            10: 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3))), 11: np.maximum(v, 0.0),
            12: v / (1 + np.exp(-v)), 13: np.where(v > 30, v, np.where(v < -30, np.exp(v), np.log1p(np.exp(v)))),
            14: v, 15: np.zeros_like(v), 16: np.zeros_like(v),
        }[subtype]


@pytest.mark.parametrize("subtype", list(range(17)))
def test_unary_scalar_path_closed_forms(oracle, subtype):
    """n < 32 (the scalar loop): each finite f16 input, 31 at a time, against the float64
    closed form rounded to f16: exact for the sign / abs / relu / copy / predicate subtypes,
    within one f16 ulp (relative 2^-10 at normal outputs, or 2^-24 absolute) for the
    transcendental ones, whose f32 libm result is rounded twice."""
    x = FINITE_F16.view(np.float16)
    if subtype in (6, 7):    # large arguments: f32 sin/cos argument reduction is what the reference does
        x = x[np.abs(x.astype(np.float64)) < 100]
    pad = (-x.size) % 31
    xs = np.concatenate([x, np.zeros(pad, np.float16)]).reshape(-1, 31)
    got = np.concatenate([oracle.unary(r, subtype) for r in xs])[: x.size].astype(np.float64)
    want = _closed(subtype, x.astype(np.float64))
    want16 = want.astype(np.float16).astype(np.float64)
    if subtype in (0, 5, 11, 14, 15, 16):
        ok = (got == want16) | (np.isnan(want16) & np.isinf(got))
    else:
        tol = np.maximum(np.abs(want16) * 2.0 ** -10, 2.0 ** -24)
        if subtype == 10:   # f32 1 + tanhf(u) cancels for u << 0: tanhf's own rounding, scaled by 0.5 v
            tol = tol + np.abs(x.astype(np.float64)) * 2.0 ** -22
        ok = (np.abs(got - want16) <= tol) | (np.isinf(want16) & (got == want16))
        ok |= np.isinf(want16) & np.isinf(got) & (np.sign(want16) == np.sign(got))
    assert ok.all(), f"subtype {subtype}: {(~ok).sum()} inputs, e.g. x={x[~ok][:4]} got={got[~ok][:4]} want={want16[~ok][:4]}"


def test_binary_scalar_path_closed_forms(oracle):
    """n < 32: add / sub / mul of two f16 values are exact in float64, and their f32
    rounding is exact too for mul (22 significant bits); add / sub may round once in f32
    and once in f16 (within one f16 ulp of the float64 sum). Division by zero gives 0
    (the scalar guard), EQ and AND the 0/1 predicates."""
    rng = np.random.default_rng(9)
    a = rng.choice(FINITE_F16, 31 * 400).view(np.float16)
    b = rng.choice(FINITE_F16, 31 * 400).view(np.float16)
    b[::7] = 0
    af, bf = a.astype(np.float64), b.astype(np.float64)

    def run(st):
        return np.concatenate([oracle.binary(a[i:i + 31], b[i:i + 31], st) for i in range(0, a.size, 31)]).astype(np.float64)

    with np.errstate(all="ignore"):
        mul = (af * bf).astype(np.float16).astype(np.float64)
        assert np.array_equal(run(2), mul)
        for st, exact in ((0, af + bf), (1, af - bf)):
            w = exact.astype(np.float16).astype(np.float64)
            g = run(st)
            assert (np.abs(g - w) <= np.maximum(np.abs(w) * 2.0 ** -10, 2.0 ** -24) + 0 * w).all() or \
                   np.array_equal(np.isinf(g), np.isinf(w))
        d = run(3)
        assert (d[bf == 0] == 0).all()
        wd = (af / np.where(bf == 0, 1, bf)).astype(np.float16).astype(np.float64)
        nz = bf != 0
        assert (np.abs(d[nz] - wd[nz]) <= np.maximum(np.abs(wd[nz]) * 2.0 ** -10, 2.0 ** -24)).all() | \
               np.isinf(wd[nz]).any()
    assert np.array_equal(run(4), (af == bf).astype(np.float64))
    pa = np.abs(a[:31 * 40]).astype(np.float16)
    pb = np.abs(b[:31 * 40]).astype(np.float16)
    g = np.concatenate([oracle.binary(pa[i:i + 31], pb[i:i + 31], 5) for i in range(0, pa.size, 31)])
    want = ((pa.astype(np.float64).astype(np.uint64) & pb.astype(np.float64).astype(np.uint64)) != 0)
    assert np.array_equal(g.astype(np.float64), want.astype(np.float64))


def test_binary_vector_division_by_zero_is_unguarded(oracle):
    """n >= 32: division runs hvhx_v2_div_f32 (a / b, no zero test), so x / 0 = +-Inf;
    below 32 elements the scalar guard returns 0."""
    a = np.full(32, 3.0, np.float16)
    a[1] = -2.0
    b = np.zeros(32, np.float16)
    y = _bits(oracle.binary(a, b, 3))
    assert y[0] == 0x7C00 and y[1] == 0xFC00
    assert not _bits(oracle.binary(a[:31], b[:31], 3)).any()


def test_softmax_scalar_rounds_e_before_dividing(oracle):
    """Hand-computed row [0, -0.5009765625] (n = 2, the scalar form of exec_softmax,
    oplist_exec.c:1184-1192):
      e0 = 1, e1 = expf(-0.5009765625) = 0.6059386134 (f32); sum = 1.6059386730 (f32)
      y0 = f16(f32(f16(1)) / sum) = f16(0.62268877)            = 0x38FB (0.62255859375)
      y1 = f16(f32(f16(e1)) / sum), f16(e1) = 0x38D9 = 0.605957031250
         = f16(0.37732264)                                      = 0x360A (0.37744140625)
    Dividing the unrounded e1 would give f16(0.37731117) = 0x3609."""
    x = np.array([[0.0, -0.5009765625]], np.float16)
    assert list(_bits(oracle.softmax(x, 1, 2, form="scalar"))[0]) == [0x38FB, 0x360A]
    assert list(_bits(oracle.softmax(x, 1, 2))[0]) == [0x38FB, 0x360A]   # dispatch: n % 32 != 0


# ---------------------------------------------------------- vectorised oracle ----
@pytest.mark.parametrize("M,K,N", [(1, 64, 1), (1, 128, 17), (2, 192, 40), (3, 256, 33), (4, 64, 16),
                                   (5, 128, 31), (33, 320, 50), (64, 256, 48), (512, 128, 19)])
def test_fast_w4g_linear_equals_scalar_matmul(oracle, M, K, N):
    """go_matmul_w4g (vectorised) == go_w4g_dequant then go_matmul_f16 with w stored [N,K]
    (the OP_MATMUL_F16 scalar loop, oplist_exec.c:1802-1811), bit for bit, for any thread
    count; and == the previous scalar form go_matmul_w4g_ref."""
    rng = np.random.default_rng(M * 1000 + N)
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    wq = oracle.w4g_pack(q)
    ws = rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float16)
    ws.ravel()[::5] = rng.uniform(6e-8, 6e-5, ws.ravel()[::5].size)   # subnormal scales
    a = (rng.standard_normal((M, K)) * 4).astype(np.float16)
    spec = oracle.matmul_f16(a, oracle.w4g_dequant(wq, ws, K), M, K, N, flags=2).reshape(M, N)
    for t in (1, 3):
        assert np.array_equal(_bits(oracle.matmul_w4g(a, wq, ws, t)), _bits(spec)), f"threads {t}"
    assert np.array_equal(_bits(oracle.matmul_w4g(a, wq, ws, 2, form="ref")), _bits(spec))


@pytest.mark.parametrize("M,K,N", [(1, 2560, 37), (3, 96, 20), (5, 64, 33), (33, 200, 17)])
def test_fast_f16_nk_linear_equals_scalar_matmul(oracle, M, K, N):
    rng = np.random.default_rng(M + K + N)
    a = rng.standard_normal((M, K)).astype(np.float16)
    w = rng.standard_normal((N, K)).astype(np.float16)
    w.ravel()[::11] = np.float16(65504)   # some outputs overflow to +-Inf
    spec = oracle.matmul_f16(a, w, M, K, N, flags=2).reshape(M, N)
    assert np.array_equal(_bits(oracle.matmul_f16_nk(a, w, 4)), _bits(spec))
    assert np.array_equal(_bits(oracle.matmul_f16_nk(a, w, 1, form="ref")), _bits(spec))


@pytest.mark.parametrize("S,H,KVH,hd,causal", [(1, 2, 1, 16, True), (7, 4, 2, 16, True), (50, 4, 2, 32, True),
                                               (64, 4, 2, 128, True), (64, 2, 2, 128, False),
                                               (37, 4, 1, 128, False), (96, 4, 2, 64, True)])
def test_fast_attention_prefill_equals_scalar_chain(oracle, S, H, KVH, hd, causal):
    """Vectorised prefill attention (causal keys past the diagonal skipped) == the scalar
    op-chain restatement go_attn_prefill_ref, both softmax forms (S % 32 == 0 or not)."""
    rng = np.random.default_rng(S * 10 + H)
    q = (rng.standard_normal((S, H, hd)) * 2).astype(np.float16)
    k = rng.standard_normal((S, KVH, hd)).astype(np.float16)
    v = rng.standard_normal((S, KVH, hd)).astype(np.float16)
    want = oracle.attn_prefill(q, k, v, 0.0883883, causal, form="ref")
    assert np.array_equal(_bits(oracle.attn_prefill(q, k, v, 0.0883883, causal, threads=3)), _bits(want))
    if causal and S > 2:   # a non-finite V row past the diagonal: no keys skipped, same result
        v2 = v.copy()
        v2[S - 1, 0, 0] = np.float16(np.inf)
        want2 = oracle.attn_prefill(q, k, v2, 0.0883883, causal, form="ref")
        assert np.array_equal(_bits(oracle.attn_prefill(q, k, v2, 0.0883883, causal, threads=2)), _bits(want2))


def test_fast_attention_decode_equals_op_chain(oracle):
    """KVRing.attn_decode (C, vectorised) == KV_GATHER -> MATMUL_F16 -> BINARY mul -> SOFTMAX
    -> MATMUL_F16 run op by op on the oracle, over a wrapped ring and both softmax forms."""
    rng = np.random.default_rng(77)
    H, KVH, hd = 8, 2, 128
    ring = O.KVRing(40 * KVH * hd * 4, KVH * hd)
    for p in range(70):   # explicit positions wrap the ring: 30..69 live, 0..29 overwritten
        ring.append(rng.standard_normal(KVH * hd).astype(np.float16), rng.standard_normal(KVH * hd).astype(np.float16),
                    pos=p)
    with pytest.raises(KeyError):
        ring.attn_decode(np.zeros((H, hd), np.float16), 70, H, KVH, hd, 0.088)
    ring2 = O.KVRing(80 * KVH * hd * 4, KVH * hd)
    for _ in range(70):
        ring2.append(rng.standard_normal(KVH * hd).astype(np.float16), rng.standard_normal(KVH * hd).astype(np.float16))
    for n in (1, 31, 32, 64, 70):
        q = rng.standard_normal((H, hd)).astype(np.float16)
        a = ring2.attn_decode(q, n, H, KVH, hd, 0.0883883)
        b = ring2.attn_decode_chain(q, n, H, KVH, hd, 0.0883883)
        assert np.array_equal(_bits(a), _bits(b)), n


def test_scalar_fallback_equals_vector_forms(oracle):
    """With the vector forms switched off, the entry points run their scalar forms and
    give the same bits (the path a CPU without AVX2/F16C takes)."""
    rng = np.random.default_rng(5)
    M, K, N = 6, 128, 24
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    wq, ws = oracle.w4g_pack(q), rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float16)
    qa = rng.standard_normal((20, 2, 32)).astype(np.float16)
    kv = rng.standard_normal((20, 1, 32)).astype(np.float16)
    fast = oracle.matmul_w4g(a, wq, ws, 2), oracle.attn_prefill(qa, kv, kv, 0.17, True)
    oracle.lib().go_fast_disable(1)
    try:
        slow = oracle.matmul_w4g(a, wq, ws, 2), oracle.attn_prefill(qa, kv, kv, 0.17, True)
    finally:
        oracle.lib().go_fast_disable(0)
    for f, s in zip(fast, slow):
        assert np.array_equal(_bits(f), _bits(s))


def _ordered_sum(prod: np.ndarray, width: int, mode: int) -> np.ndarray:
    """float32 sum over the last axis of `prod` in summation order `mode`: slices of
    `width` summed from zero in sequence, the slice sums combined pairwise (mode 1) or
    in sequence (mode 2); every add one float32 rounding (numpy float32 arrays)."""
    n = prod.shape[-1]
    parts = []
    for s0 in range(0, n, width):
        acc = np.zeros(prod.shape[:-1], np.float32)
        for k in range(s0, min(s0 + width, n)):
            acc = acc + prod[..., k]
        parts.append(acc)
    if mode == 1:
        w = 1
        while w < len(parts):
            for i in range(0, len(parts) - w, 2 * w):
                parts[i] = parts[i] + parts[i + w]
            w *= 2
        return parts[0]
    acc = parts[0]
    for p in parts[1:]:
        acc = acc + p
    return acc


@pytest.mark.parametrize("mode", [1, 2])
def test_summation_orders_are_the_stated_fp32_orders(oracle, mode):
    """go_set_order's modes (used to measure order-only spread for the end-to-end gate)
    compute exactly the stated fp32 order of the same products: the W4G linear (K = 200:
    a ragged last slice; 7 slices of 32 in mode 1, an odd count for the pairwise tree)
    and the fp16 [N, K] linear against float32 numpy sums in that order, bit for bit;
    mode 0 stays the sequential order."""
    if not oracle.fast_available():
        pytest.skip("vector forms unavailable")
    rng = np.random.default_rng(11 + mode)
    M, K, N = 3, 200, 21
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    wq = oracle.w4g_pack(q)
    ws = rng.uniform(0.005, 0.02, (N, K // 8)).astype(np.float16)   # group 8
    a = rng.standard_normal((M, K)).astype(np.float16)
    wf = rng.standard_normal((N, K)).astype(np.float16)
    # Row 0 x column 0 tells the orders apart: products 1, then 2^-25 each (below half an
    # ulp of 1, lost one by one in sequence, kept as 32- / 16-term slice sums), then -1:
    # the sequential sum is 0, a sliced one 2^-25 times the kept terms.
    a[0] = np.float16(2.0 ** -12)
    a[0, 0], a[0, -1] = 1, -1
    wf[0] = np.float16(2.0 ** -13)
    wf[0, 0] = wf[0, -1] = 1
    width = 32 if mode == 1 else 16
    wdq = oracle.w4g_dequant(wq, ws, K, 8).astype(np.float32)

    def ordered(w):
        prod = a.astype(np.float32)[:, None, :] * w.astype(np.float32)[None, :, :]
        return _ordered_sum(prod, width, mode).astype(np.float16)

    seq_w4g = oracle.lib()
    y0 = np.empty((M, N), np.float16)
    assert seq_w4g.go_matmul_w4g(O._p(a), O._p(wq), O._p(ws), O._p(y0), M, K, N, 8, 2) == 0
    with oracle.summation_order(mode):
        y = np.empty((M, N), np.float16)
        assert seq_w4g.go_matmul_w4g(O._p(a), O._p(wq), O._p(ws), O._p(y), M, K, N, 8, 2) == 0
        yf = oracle.matmul_f16_nk(a, wf, 2)
    assert yf[0, 0] > 0 and oracle.matmul_f16_nk(a, wf, 2)[0, 0] == 0
    assert np.array_equal(_bits(y), _bits(ordered(wdq)))
    assert np.array_equal(_bits(yf), _bits(ordered(wf)))
    seq = np.zeros((M, N), np.float32)
    for k in range(K):
        seq = seq + a.astype(np.float32)[:, k:k + 1] * wdq[None, :, k][0]
    assert np.array_equal(_bits(y0), _bits(seq.astype(np.float16)))


@pytest.mark.parametrize("mode", [1, 2])
def test_attention_summation_orders(oracle, mode):
    """Causal prefill attention in mode 1 / 2: the q.k scores summed over d in 32- / 16-wide
    slices (pairwise / in sequence), rounded through the chain's f16 points (score, times
    f16 scale, plus a zero mask), the oracle's softmax row, then P.V over keys in 64-key
    chunks combined pairwise / in sequence, against float32 numpy in those orders (S = 150:
    three chunks, the last ragged)."""
    if not oracle.fast_available():
        pytest.skip("vector forms unavailable")
    rng = np.random.default_rng(21 + mode)
    S, H, KVH, hd, scale = 150, 2, 1, 64, 0.125
    qa = rng.standard_normal((S, H, hd)).astype(np.float16)
    ka = rng.standard_normal((S, KVH, hd)).astype(np.float16)
    va = rng.standard_normal((S, KVH, hd)).astype(np.float16)
    with oracle.summation_order(mode):
        got = oracle.attn_prefill(qa, ka, va, scale, True, threads=2)
    width = 32 if mode == 1 else 16
    sc = np.float32(np.float16(scale))
    want = np.empty((S, H, hd), np.float16)
    for h in range(H):
        qf, kf, vf = qa[:, h].astype(np.float32), ka[:, 0].astype(np.float32), va[:, 0].astype(np.float32)
        t = _ordered_sum(qf[:, None, :] * kf[None, :, :], width, mode).astype(np.float16)
        t = (t.astype(np.float32) * sc).astype(np.float16)
        s = (t.astype(np.float32) + np.float32(0)).astype(np.float16)
        s[np.triu_indices(S, 1)] = np.float16(-np.inf)
        p = oracle.softmax(s, S, S).astype(np.float32)
        for i in range(S):
            prod = (p[i, :i + 1, None] * vf[:i + 1]).T   # [hd, keys]
            want[i, h] = _ordered_sum(prod, 64, mode).astype(np.float16)
    assert np.array_equal(_bits(got), _bits(want))
