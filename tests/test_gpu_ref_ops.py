"""GPU parity, through the engine, of the reference runlist ops that compiled blobs carry
most (qwen35_08b manifest: UNARY 5305, STRIDED_SLICE 3507, BROADCAST 1476, ADD 1291,
TRANSPOSE_GEN 175) plus SILU and the chunked fp16 linear (opcode 35), against the oracle
(oracle/gehtp_oracle*.c restating oplist_exec.c:594-614, 807-848, 1013-1079, 1709-1813,
1876-1988).

Bars: data movement (broadcast, transpose, slice) and exact arithmetic (neg, abs, relu,
copy, sqrt, the f32 add of ADD, the NaN / Inf tests) bit-exact (relu up to the sign of a
zero result, which C's fmaxf leaves unspecified); the transcendental UNARY
subtypes and SILU, whose f32 libm results may differ from the device's by an f32 ulp
before the f16 rounding, within one fp16 ulp (and >= 99 % exact); opcode 35 chunks
byte-identical to the whole opcode-24 product (the reference's SPLIT invariant,
compiler/tests/test_wtop_emit.cpp:556-596) and within the fp16 bar of the oracle."""
from __future__ import annotations

import itertools

import numpy as np
import pytest

from helpers import assert_close, normal_f16

from gehtp_amd.abi import opcodes as OP
from gehtp_amd.runlist import BlobBuilder

pytestmark = pytest.mark.gpu

EXACT_UNARY = {0, 2, 5, 11, 14, 15, 16}


@pytest.fixture(autouse=True)
def fresh_engine(engine, torch_dev):
    engine.shutdown()
    engine.state_reset()
    yield
    engine.shutdown()


def _ulps(a, b):
    ai = a.view(np.int16).astype(np.int32)
    bi = b.view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def _special_inputs(rng, n):
    x = (rng.standard_normal(n) * 3).astype(np.float16)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504, -65504, 1e-7, -6e-8, 0.5, 31.0, -31.0, 88.0,
                   -88.0, 1.0, -1.0], np.float16)
    x[:min(n, sp.size)] = sp[:min(n, sp.size)]
    return x


def _run(engine, bb, temps):
    engine.run(engine.parse(bb.build()))
    return {k: np.frombuffer(engine.temp(t), np.float16).copy() for k, t in temps.items()}


@pytest.mark.parametrize("n", [20, 1000], ids=["scalar-form", "n>=32-form"])
def test_unary_all_subtypes(engine, oracle, n):
    rng = np.random.default_rng(n)
    x = _special_inputs(rng, n)
    pos = np.abs(x)
    bb = BlobBuilder()
    sx, sp = bb.add_slot(x), bb.add_slot(pos)
    temps = {}
    for sub in range(17):
        temps[sub] = bb.temp()
        bb.op(OP.UNARY_F16, bb.slot_ref(sp if sub in (2, 3, 4) else sx), temps[sub], n, sub)
    out = _run(engine, bb, temps)
    for sub in range(17):
        want = oracle.unary(pos if sub in (2, 3, 4) else x, sub)
        got = out[sub][:n]
        if sub in EXACT_UNARY:
            same = got.view(np.uint16) == want.view(np.uint16)
            if sub == 11:   # fmaxf(0, -0): C leaves the sign of the zero unspecified
                same |= (got.astype(np.float32) == 0) & (want.astype(np.float32) == 0)
            bad = np.flatnonzero(~same)
            assert bad.size == 0, (f"subtype {sub}: x={x[bad[:4]]} got={got[bad[:4]].view(np.uint16)} "
                                   f"want={want[bad[:4]].view(np.uint16)}")
            continue
        fin = np.isfinite(want.astype(np.float32)) | np.isfinite(got.astype(np.float32))
        same_special = (got.view(np.uint16) == want.view(np.uint16)) | ~fin
        assert same_special.all(), f"subtype {sub}: non-finite results differ"
        u = _ulps(got[fin], want[fin])
        assert (u <= 1).all(), f"subtype {sub}: {int(u.max())} ulps"
        assert (u == 0).mean() >= 0.99, f"subtype {sub}: only {(u == 0).mean():.3f} exact"


@pytest.mark.parametrize("n", [40, 3000])
def test_add_and_silu(engine, oracle, n):
    """ADD (op 7): f16(f32(a) + f32(b)) bit-exact; SILU (op 4) against UNARY silu."""
    rng = np.random.default_rng(n + 1)
    a, b = _special_inputs(rng, n), normal_f16(rng, n)
    bb = BlobBuilder()
    sa, sb = bb.add_slot(a), bb.add_slot(b)
    t_add, t_in, t_silu = bb.temp(), bb.temp(), bb.temp()
    bb.op(OP.ADD_F16, bb.slot_ref(sa), bb.slot_ref(sb), t_add, n)
    bb.op(OP.UNARY_F16, bb.slot_ref(sb), t_in, n, 14)          # SILU reads a temp (oplist_exec.c:596)
    bb.op(OP.SILU_F16, t_in, t_silu, n)
    out = _run(engine, bb, {"add": t_add, "silu": t_silu})
    want = oracle.binary(a, b, 0)
    assert np.array_equal(out["add"][:n].view(np.uint16), want.view(np.uint16))
    ws = oracle.unary(b, 12)
    u = _ulps(out["silu"][:n], ws)
    assert (u <= 1).all() and (u == 0).mean() >= 0.99


@pytest.mark.parametrize("in_d,out_d", [
    ([1, 128], [32, 128]), ([1, 4096], [16, 4096]), ([5, 1, 128], [5, 4, 128]),
    ([8, 1, 40, 128], [8, 4, 40, 128]), ([3, 1], [3, 7]), ([1, 1, 6], [2, 5, 6]), ([1], [9]),
])
def test_broadcast(engine, oracle, in_d, out_d):
    rng = np.random.default_rng(int(np.prod(out_d)) % 1000)
    x = normal_f16(rng, int(np.prod(in_d)))
    bb = BlobBuilder()
    sx = bb.add_slot(x)
    t = bb.temp()
    n = int(np.prod(out_d))
    bb.op(OP.BROADCAST_F16, bb.slot_ref(sx), t, n, x.size, *(list(in_d) + [1] * (4 - len(in_d))),
          *(list(out_d) + [1] * (4 - len(out_d))))
    got = _run(engine, bb, {"y": t})["y"][:n]
    want = oracle.broadcast(x, in_d, out_d)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("dims", [(40, 128), (64, 8, 128), (2, 3, 4, 5), (7, 1, 6), (128, 16, 64)])
def test_transpose_gen(engine, oracle, dims):
    rng = np.random.default_rng(sum(dims))
    x = normal_f16(rng, int(np.prod(dims)))
    perms = list(itertools.permutations(range(len(dims))))
    bb = BlobBuilder()
    sx = bb.add_slot(x)
    temps = {}
    for p in perms:
        temps[p] = bb.temp()
        d4 = list(dims) + [1] * (4 - len(dims))
        bb.op(OP.TRANSPOSE_GEN_F16, bb.slot_ref(sx), temps[p], len(dims), *d4, sum(v << (8 * i) for i, v in enumerate(p)))
    out = _run(engine, bb, temps)
    for p in perms:
        want = oracle.transpose_gen(x, dims, p)
        assert np.array_equal(out[p][:x.size].view(np.uint16), want.view(np.uint16)), p


@pytest.mark.parametrize("d,b,e,s", [
    ((40,), (3,), (37,), (1,)), ((4096,), (1,), (4096,), (2,)),
    ((32, 128), (0, 0), (32, 64), (1, 1)), ((32, 128), (0, 64), (32, 128), (1, 1)),
    ((64, 2048), (0, 1), (64, 2048), (1, 2)), ((5, 20), (1, 0), (5, 20), (2, 3)),
    ((3, 4, 10), (1, 0, 2), (3, 4, 9), (1, 2, 3)), ((16, 32, 128), (0, 0, 64), (16, 32, 128), (1, 1, 1)),
])
def test_strided_slice(engine, oracle, d, b, e, s):
    rng = np.random.default_rng(sum(d))
    x = normal_f16(rng, int(np.prod(d)))
    n = x.reshape(d)[tuple(slice(bb_, ee, ss) for bb_, ee, ss in zip(b, e, s))].size
    bb = BlobBuilder()
    sx = bb.add_slot(x)
    t = bb.temp()
    pad = lambda v: list(v) + [0] * (3 - len(v))   # noqa: E731
    bb.op(OP.STRIDED_SLICE_F16, bb.slot_ref(sx), t, n, len(d), *pad(b), *pad(e), *pad(s), *(list(d) + [1] * (3 - len(d))))
    got = _run(engine, bb, {"y": t})["y"][:n]
    want = oracle.strided_slice(x, n, b, e, s, d)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("M,K,N,t1", [(1, 2560, 4096, True), (7, 512, 960, True), (64, 256, 384, False)])
def test_matmul_f16_split_chunks(engine, oracle, M, K, N, t1):
    """Opcode 35: three chunks [n0, n0 + N_chunk) of one output; byte-identical to the
    whole opcode-24 product, and within the fp16 bar of the oracle."""
    rng = np.random.default_rng(M * N)
    a = (normal_f16(rng, M, K) * np.float16(0.25)).astype(np.float16)
    w = (normal_f16(rng, N, K) if t1 else normal_f16(rng, K, N)) * np.float16(0.25)
    w = w.astype(np.float16)
    flags = 2 if t1 else 0
    cuts = [0, N // 3 // 32 * 32, 2 * N // 3 // 32 * 32, N]
    bb = BlobBuilder()
    sa, sw = bb.add_slot(a), bb.add_slot(w)
    t_whole, t_split = bb.temp(), bb.temp()
    bb.op(OP.MATMUL_F16, bb.slot_ref(sa), bb.slot_ref(sw), t_whole, M, K, N, flags)
    for c0, c1 in zip(cuts[:-1], cuts[1:]):
        bb.op(OP.MATMUL_F16_SPLIT, bb.slot_ref(sa), bb.slot_ref(sw), t_split, M, K, N, c0, c1 - c0, flags)
    out = _run(engine, bb, {"w": t_whole, "s": t_split})
    whole, split = out["w"][:M * N], out["s"][:M * N]
    assert np.array_equal(whole.view(np.uint16), split.view(np.uint16))
    want = oracle.matmul_f16(a, w, M, K, N, flags=flags)
    assert_close(split.reshape(M, N), want.reshape(M, N), what=f"split M{M} K{K} N{N}")
