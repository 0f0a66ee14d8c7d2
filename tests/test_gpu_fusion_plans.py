"""Load-time fusion of the attention chain under static temp plans (TEMPOFF) whose temps
share device bytes, in the reference emitter's lowerings
(compiler/tools/wtop_ops/op_matmul.cpp:36-98, op_eltwise_binary.cpp:9-67; a scale after
q.k^T as in test_models/transformer32, or on q before it as in the qwen35_08b manifest's
ops 2722-2728; the mask BROADCAST over the heads and added with ADD_F16).

A plan may legally give the chain's output the bytes of k (dead after q.k^T when the
chain runs op by op): fused, the kernel would write over its own input, so it writes
engine scratch and the result is copied over (wt_exec_fusion_detail counts it). A plan
may also give a temp written by another op inside the chain's window the bytes of q
(dead after q.k^T in op order): the kernel, which runs at the chain's last op, would read
the overwritten q, so the observed run rules the chain out and it keeps running op by op.
Either way the results are the op chain's: fused within the fp16 tolerance of the chain
and of the oracle, unfused bit-identical to the fusion-off run."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_close, normal_f16

from gehtp_amd.abi import WT_KV_POS_AUTO, opcodes as OP
from gehtp_amd.runlist import BlobBuilder
from gehtp_amd.tempplan import out_bytes, _roles

pytestmark = pytest.mark.gpu

HD = 128


def _slice(bb, src, n_in, b0, n):
    y = bb.temp()
    bb.op(OP.STRIDED_SLICE_F16, src, y, n, 1, b0, 0, 0, b0 + n, 0, 0, 1, 1, 1, n_in, 1, 1)
    return y


def _bcast(bb, x, in_d, out_d):
    y = bb.temp()
    ind = list(in_d) + [1] * (4 - len(in_d))
    outd = list(out_d) + [1] * (4 - len(out_d))
    bb.op(OP.BROADCAST_F16, x, y, int(np.prod(out_d)), int(np.prod(in_d)), *ind, *outd)
    return y


def _prefill_blob(H, S, form, late_v):
    """q | k | v [H, S, 128] from the input slot, then the attention chain in `form`;
    with late_v the slice producing v stands between SOFTMAX and p.v (another op inside
    the chain's window)."""
    bb = BlobBuilder()
    n = H * S * HD
    x = bb.slot_ref(bb.add_input_slot(3 * n * 2))
    scale1 = bb.slot_ref(bb.add_slot(np.array([1.0 / np.sqrt(HD)], np.float16)))
    causal = np.where(np.arange(S)[None, :] <= np.arange(S)[:, None], np.float16(0), np.float16(-np.inf))
    mask = bb.slot_ref(bb.add_slot(causal.astype(np.float16)))
    q, k = _slice(bb, x, 3 * n, 0, n), _slice(bb, x, 3 * n, n, n)
    v = None if late_v else _slice(bb, x, 3 * n, 2 * n, n)
    s = bb.temp()
    if form == "ref_pre":
        qs = bb.temp()
        bb.op(OP.BINARY_F16, q, _bcast(bb, scale1, [1, 1, 1], [H, S, HD]), qs, n, 2)
        bb.op(OP.MATMUL_F16, qs, k, s, S, HD, S, 6 | (H << 16))
    else:
        kT = bb.temp()
        bb.op(OP.TRANSPOSE_GEN_F16, k, kT, 3, H, S, HD, 1, 0 | (2 << 8) | (1 << 16))
        bb.op(OP.MATMUL_F16, q, kT, s, S, HD, S, 4 | (H << 16))
        s1 = bb.temp()
        bb.op(OP.BINARY_F16, s, _bcast(bb, scale1, [1, 1, 1], [H, S, S]), s1, H * S * S, 2)
        s = s1
    s2, p, o = bb.temp(), bb.temp(), bb.temp()
    bb.op(OP.ADD_F16, s, _bcast(bb, mask, [1, S, S], [H, S, S]), s2, H * S * S)
    bb.op(OP.SOFTMAX_F16, s2, p, H * S, S)
    if late_v:
        v = _slice(bb, x, 3 * n, 2 * n, n)
    bb.op(OP.MATMUL_F16, p, v, o, S, S, HD, 4 | (H << 16))
    return bb, {"q": q, "k": k, "v": v, "o": o}


def _plan(bb, same=()):
    """Every temp its own bytes, except each (a, b) in `same`: b takes a's offset."""
    size = {}
    for opc, args in bb.ops:
        for t in _roles(opc, args)[1]:
            size[t] = max(size.get(t, 0), out_bytes(bb, opc, args))
    off, cap = {}, 0
    for t in sorted(size):
        off[t] = cap
        cap += (size[t] + 127) // 128 * 128
    for a, b in same:
        assert size[b] <= size[a]
        off[b] = off[a]
    bb.set_tempoff(cap, [(t, off[t], size[t]) for t in sorted(size)])


def _run(engine, blob, inp, out_t, fusion, runs=2):
    prev = engine.set_fusion(fusion)
    try:
        engine.shutdown()
        pb = engine.parse(blob)
        f0, r0 = engine.fusion_stats()
        a0 = engine.fusion_detail(pb)["alias_runs"]
        outs = [np.frombuffer(engine.run_io(pb, inp, out_t)[0], np.float16).copy() for _ in range(runs)]
        f1, r1 = engine.fusion_stats()
        d = engine.fusion_detail(pb)
        engine.shutdown()
    finally:
        engine.set_fusion(prev)
    d["fused_runs"] = r1 - r0
    d["alias_runs"] -= a0
    return outs, d


def _oracle_prefill(oracle, qkv, H, S):
    q, k, v = (a.reshape(H, S, HD).transpose(1, 0, 2).copy() for a in np.split(qkv, 3))
    return oracle.attn_prefill(q, k, v, 1.0 / np.sqrt(HD), True).transpose(1, 0, 2).ravel()


@pytest.mark.parametrize("form", ["ref_post", "ref_pre"])
def test_prefill_chain_output_over_k(engine, oracle, form):
    """TEMPOFF gives the chain's output k's bytes: the fused run writes scratch and
    copies, the observed run flags the overlap; results equal the chain's within the
    fp16 tolerance, and the oracle's."""
    H, S = 4, 128
    rng = np.random.default_rng(7)
    qkv = normal_f16(rng, 3 * H * S * HD)
    bb, t = _prefill_blob(H, S, form, late_v=False)
    _plan(bb, same=[(t["k"], t["o"])])
    blob = bb.build()
    (ref0, ref1), d0 = _run(engine, blob, qkv.tobytes(), t["o"], fusion=False)
    assert np.array_equal(ref0.view(np.uint16), ref1.view(np.uint16)) and d0["fused_runs"] == 0
    (obs, fused), d = _run(engine, blob, qkv.tobytes(), t["o"], fusion=True)
    assert d["chains"] == 1 and d["blocked"] == 0 and d["aliased"] == 1, d
    assert d["fused_runs"] == 1 and d["alias_runs"] == 1, d
    assert np.array_equal(obs.view(np.uint16), ref0.view(np.uint16))   # the observed run is op by op
    assert_close(fused, ref0, what=f"{form} fused over k vs chain")
    assert_close(fused, _oracle_prefill(oracle, qkv, H, S), what=f"{form} fused vs oracle")


@pytest.mark.parametrize("form", ["ref_post", "ref_pre"])
def test_prefill_chain_input_overwritten_in_window_stays_unfused(engine, form):
    """v is produced between SOFTMAX and p.v and the plan gives it q's bytes (q is dead
    by then in op order): the kernel would read the overwritten q at the chain's last op,
    so the chain is ruled out and runs op by op, bit-identical to fusion off."""
    H, S = 4, 64
    rng = np.random.default_rng(8)
    qkv = normal_f16(rng, 3 * H * S * HD)
    bb, t = _prefill_blob(H, S, form, late_v=True)
    _plan(bb, same=[(t["q"], t["v"])])
    blob = bb.build()
    (ref0, _), _ = _run(engine, blob, qkv.tobytes(), t["o"], fusion=False)
    (a, b), d = _run(engine, blob, qkv.tobytes(), t["o"], fusion=True)
    assert d["chains"] == 1 and d["blocked"] == 1 and d["fused_runs"] == 0, d
    for r in (a, b):
        assert np.array_equal(r.view(np.uint16), ref0.view(np.uint16))


@pytest.mark.parametrize("form", ["ref_post", "ref_pre"])
def test_prefill_chain_late_v_fuses(engine, oracle, form):
    """The same window (v produced between SOFTMAX and p.v, as transformer32's second
    layer computes v after the softmax) with every temp in its own bytes fuses: the
    kernel runs at p.v, where v exists."""
    H, S = 4, 64
    rng = np.random.default_rng(9)
    qkv = normal_f16(rng, 3 * H * S * HD)
    bb, t = _prefill_blob(H, S, form, late_v=True)
    _plan(bb)
    blob = bb.build()
    (ref0, _), _ = _run(engine, blob, qkv.tobytes(), t["o"], fusion=False)
    (_, fused), d = _run(engine, blob, qkv.tobytes(), t["o"], fusion=True)
    assert d["chains"] == 1 and d["blocked"] == 0 and d["aliased"] == 0 and d["fused_runs"] == 1, d
    assert_close(fused, ref0, what=f"{form} late v fused vs chain")
    assert_close(fused, _oracle_prefill(oracle, qkv, H, S), what=f"{form} late v vs oracle")


def test_decode_chain_output_over_q(engine):
    """Decode in the reference emitter's form (two single-face KV_GATHERs, q pre-scaled,
    the step's mask row BROADCAST over the heads and added with ADD_F16) under a plan
    giving the output q's bytes: fused steps write scratch and copy, and equal the op
    chain within the fp16 tolerance at every step."""
    H, KVH, P, steps = 8, 2, 96, 12
    bb = BlobBuilder()
    kv = KVH * HD
    n_in = H * HD + 2 * kv + P
    x = bb.slot_ref(bb.add_input_slot(n_in * 2))
    st = bb.add_state(P * kv * 4)
    scale1 = bb.slot_ref(bb.add_slot(np.array([1.0 / np.sqrt(HD)], np.float16)))
    q = _slice(bb, x, n_in, 0, H * HD)
    k = _slice(bb, x, n_in, H * HD, kv)
    v = _slice(bb, x, n_in, H * HD + kv, kv)
    mrow = _slice(bb, x, n_in, H * HD + 2 * kv, P)
    bb.op(OP.KV_APPEND_F16, k, v, st, WT_KV_POS_AUTO)
    kT, vv = bb.temp(), bb.temp()
    bb.op(OP.KV_GATHER_F16, st, kT, 0, WT_KV_POS_AUTO, H, KVH, HD)
    bb.op(OP.KV_GATHER_F16, st, 0, vv, WT_KV_POS_AUTO, H, KVH, HD)
    qs, s, s2, p, o = (bb.temp() for _ in range(5))
    bb.op(OP.BINARY_F16, q, _bcast(bb, scale1, [1, 1], [H, HD]), qs, H * HD, 2)
    bb.op(OP.MATMUL_F16, qs, kT, s, 1, HD, P, 4 | (H << 16))
    bb.op(OP.ADD_F16, s, _bcast(bb, mrow, [1, P], [H, P]), s2, H * P)
    bb.op(OP.SOFTMAX_F16, s2, p, H, P)
    bb.op(OP.MATMUL_F16, p, vv, o, 1, P, HD, 4 | (H << 16))
    _plan(bb, same=[(q, o)])
    blob = bb.build()
    rng = np.random.default_rng(10)
    inputs = []
    for pos in range(steps):
        mask = np.zeros(P, np.float16)
        mask[pos + 1:] = -np.inf
        inputs.append(np.concatenate([normal_f16(rng, H * HD + 2 * kv), mask]).tobytes())
    res = {}
    for fusion in (False, True):
        prev = engine.set_fusion(fusion)
        try:
            engine.shutdown()
            pb = engine.parse(blob)
            engine.state_reset()
            a0 = engine.fusion_detail(pb)["alias_runs"]
            res[fusion] = [np.frombuffer(engine.run_io(pb, inp, o)[0], np.float16).copy() for inp in inputs]
            d = engine.fusion_detail(pb)
            engine.shutdown()
        finally:
            engine.set_fusion(prev)
    assert d["chains"] == 1 and d["blocked"] == 0 and d["aliased"] == 1, d
    assert d["alias_runs"] - a0 == steps - 1, d
    for t_, (a, b) in enumerate(zip(res[False], res[True])):
        assert_close(b, a, what=f"decode step {t_} fused over q vs chain")
