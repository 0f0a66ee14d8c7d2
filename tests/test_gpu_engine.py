"""The runlist engine through the reference ABI (wt_parse / wt_exec_run_io / temps /
states) on hand-built WTOP blobs, checked against the CPU oracle."""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest

from helpers import assert_close, normal_f16, w4g_weights

from gehtp_amd import WtExecError
from gehtp_amd.abi import WT_KV_POS_AUTO, WT_REF_NONE, opcodes as OP
from gehtp_amd.runlist import BlobBuilder, f32_bits

pytestmark = pytest.mark.gpu

SCALE = float(np.float16(1.0 / math.sqrt(128)))


@pytest.fixture(autouse=True)
def fresh_engine(engine, torch_dev):
    engine.shutdown()
    engine.state_reset()
    yield
    engine.shutdown()


def _h(b: bytes, shape=None):
    a = np.frombuffer(b, np.float16)
    return a.reshape(shape) if shape else a


def test_w4g_op_via_run_io(engine, oracle):
    rng = np.random.default_rng(1)
    M, N, K = 1, 3072, 1024
    _, wq, ws = w4g_weights(rng, N, K)
    x = normal_f16(rng, M, K)
    bb = BlobBuilder()
    xs = bb.add_input_slot(M * K * 2)
    sq = bb.add_slot(wq, count=N * K)
    ss = bb.add_slot(ws)
    t = bb.temp()
    bb.op(OP.MATMUL_W4G_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t, M, K, N, 64, 2)
    pb = engine.parse(bb.build())
    out, us = engine.run_io(pb, x.tobytes(), t, timing=True)
    assert_close(_h(out, (M, N)), oracle.matmul_w4g(x, wq, ws), what="run_io w4g")
    assert len(us) == 1 and us[0] >= 0
    assert engine.stats().matmul == 1 and engine.stats().ops == 1
    # second call with a different input re-uses the resident weights
    x2 = normal_f16(rng, M, K)
    out2, _ = engine.run_io(pb, x2.tobytes(), t)
    assert_close(_h(out2, (M, N)), oracle.matmul_w4g(x2, wq, ws), what="run_io w4g #2")


def test_run_io_device_bound_input(engine, oracle, torch_dev):
    """wt_exec_set_input_device: runs read the bound HBM buffer in place (no staging),
    through direct runs, graph capture and replays, each seeing the buffer's current
    contents; a host input still takes precedence; a too-small binding is an error."""
    import torch
    rng = np.random.default_rng(3)
    M, N, K = 1, 3072, 1024
    _, wq, ws = w4g_weights(rng, N, K)
    bb = BlobBuilder()
    xs = bb.add_input_slot(M * K * 2)
    sq = bb.add_slot(wq, count=N * K)
    ss = bb.add_slot(ws)
    t = bb.temp()
    bb.op(OP.MATMUL_W4G_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t, M, K, N, 64, 2)
    pb = engine.parse(bb.build())
    xd = torch.empty(M * K, dtype=torch.float16, device=torch_dev)
    try:
        engine.set_input_device(xd.data_ptr(), M * K * 2)
        xs_, outs = [], []
        for i in range(6):   # identical runs: direct, then captured, then graph replays
            x = normal_f16(rng, M, K)
            xd.copy_(torch.from_numpy(x.reshape(-1)))
            torch.cuda.synchronize()
            out, _ = engine.run_io(pb, None, t)
            xs_.append(x)
            outs.append(out)
        for i, (x, out) in enumerate(zip(xs_, outs)):
            assert_close(_h(out, (M, N)), oracle.matmul_w4g(x, wq, ws), what=f"bound input run {i}")
            ref, _ = engine.run_io(pb, x.tobytes(), t)   # host input wins over the binding
            assert _h(out).tobytes() == _h(ref).tobytes(), f"run {i}"
        engine.set_input_device(xd.data_ptr(), M * K * 2 - 2)
        with pytest.raises(WtExecError, match="bound device input"):
            engine.run_io(pb, None, t)
    finally:
        engine.set_input_device(None)


@pytest.mark.parametrize("mode", [0, 1])
def test_split_k_finish_normalizes_next_op(engine, oracle, mode):
    """OP_W4G_FUSED_F16 with a K split and a residual (o-proj-like), then OP_W4G_FUSED_F16
    normalizing that output (RMSNORM2 -> linear, SwiGLU for mode 1): the split's
    finishing pass also writes the normalized rows the second op's GEMM reads. Both
    outputs match the oracle's op chain, and the second op run alone (normalizing by
    itself) gives the same output."""
    rng = np.random.default_rng(70 + mode)
    M, K1, N1, N2 = 256, 4096, 1024, 1024 if mode else 512
    _, wq1, ws1 = w4g_weights(rng, N1, K1)
    _, wq2, ws2 = w4g_weights(rng, N2, N1)
    a = normal_f16(rng, M, K1) * np.float16(0.25)
    r = normal_f16(rng, M, N1)
    gam = rng.uniform(0.8, 1.2, N1).astype(np.float16)
    bb = BlobBuilder()
    xs = bb.add_input_slot(M * K1 * 2)
    q1, s1 = bb.add_slot(wq1, count=N1 * K1), bb.add_slot(ws1)
    q2, s2 = bb.add_slot(wq2, count=N2 * N1), bb.add_slot(ws2)
    rs, gs = bb.add_slot(r), bb.add_slot(gam)
    t1, t2 = bb.temp(), bb.temp()
    n_out = N2 // 2 if mode else N2
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(q1), bb.slot_ref(s1), t1, M, K1, N1, WT_REF_NONE,
          bb.slot_ref(rs), 0, 2)
    bb.op(OP.W4G_FUSED_F16, t1, bb.slot_ref(q2), bb.slot_ref(s2), t2, M, N1, N2, bb.slot_ref(gs), WT_REF_NONE,
          mode, 2)
    pb = engine.parse(bb.build())
    out, _ = engine.run_io(pb, a.tobytes(), t2, out_bytes=M * n_out * 2)
    y1 = _h(engine.temp(t1), (M, N1))
    y1_ref = oracle.binary(oracle.matmul_w4g(a, wq1, ws1, threads=8), r, 0)
    assert_close(y1, y1_ref, what="split-K output")
    acc = oracle.matmul_w4g(oracle.rmsnorm2(y1, gam, np.zeros(N1, np.float16)), wq2, ws2, threads=8)
    ref = oracle.binary(oracle.unary(acc[:, 0::2].copy(), 12), acc[:, 1::2].copy(), 2) if mode else acc
    fused = _h(out, (M, n_out))
    assert_close(fused, ref, what="next op on the pre-normalized rows")
    engine.run(pb, first=1, count=1)   # the second op alone normalizes its input itself
    alone = _h(engine.temp(t2), (M, n_out))
    # the fused finish sums the squares in the standalone RMSNORM2 kernel's order
    assert np.array_equal(fused.view(np.uint16), alone.view(np.uint16))


@pytest.mark.parametrize("M,H,KVH,runs,kv_outs", [(256, 16, 8, 3, True), (200, 32, 8, 2, True),
                                                  (2048, 32, 8, 1, True), (320, 16, 4, 2, False)])
def test_qkv_gemm_performs_rope_op(engine, oracle, M, H, KVH, runs, kv_outs):
    """OP_W4G_FUSED_F16 (RMSNorm + q|k|v GEMM) followed by the OP_QK_ROPE_KV_F16 reading
    its output: with fusion on, the GEMM's epilogue performs that op (after a table
    kernel that fixes the positions and advances the counter). Over `runs` prefill calls
    in a row (positions continuing, later calls replayed from a HIP graph) the q / k / v
    outputs, the GEMM output, the ring read back by KV_GATHER and the positions are
    bit-identical to the op-by-op runs; a ragged M leaves a partial token tile. The q
    output also matches the oracle's RMSNorm + RoPE of the GEMM output. Without k / v
    outputs the ring alone receives them."""
    rng = np.random.default_rng(90 + M + H)
    K, hd, theta = 1024, 128, 1e6
    N, kv = (H + 2 * KVH) * hd, KVH * hd
    max_pos = runs * M
    _, wq, ws = w4g_weights(rng, N, K)
    gam = rng.uniform(0.8, 1.2, K).astype(np.float16)
    qg = rng.uniform(0.8, 1.2, hd).astype(np.float16)
    kg = rng.uniform(0.8, 1.2, hd).astype(np.float16)
    bb = BlobBuilder()
    st = bb.add_state(max_pos * kv * 4)
    xs = bb.add_input_slot(M * K * 2)
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    sg, sqg, skg = bb.add_slot(gam), bb.add_slot(qg), bb.add_slot(kg)
    t_qkv, t_q, t_k, t_v, t_kT, t_vo = (bb.temp() for _ in range(6))
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_qkv, M, K, N, bb.slot_ref(sg),
          WT_REF_NONE, 0, 2)
    bb.op(OP.QK_ROPE_KV_F16, t_qkv, t_q, t_k if kv_outs else WT_REF_NONE, t_v if kv_outs else WT_REF_NONE, st, M,
          H, KVH, hd, bb.slot_ref(sqg), bb.slot_ref(skg), f32_bits(theta))
    bb.op(OP.KV_GATHER_F16, st, t_kT, t_vo, WT_KV_POS_AUTO, H, KVH, hd)
    pb = engine.parse(bb.build())
    xs_in = [normal_f16(rng, M, K) for _ in range(runs)]
    got = {}
    for fusion in (False, True):
        prev = engine.set_fusion(fusion)
        try:
            engine.state_reset()
            n0 = engine.qkv_rope_fused()
            res = []
            for x in xs_in:
                engine.run_io(pb, x.tobytes(), t_q, out_bytes=M * H * hd * 2)
                temps = (t_qkv, t_q, t_k, t_v, t_kT, t_vo) if kv_outs else (t_qkv, t_q, t_kT, t_vo)
                res.append([engine.temp(t) for t in temps])
            assert engine.qkv_rope_fused() - n0 == (runs if fusion else 0)
            got[fusion] = res
        finally:
            engine.set_fusion(prev)
    names = ("qkv", "q", "k", "v", "kT", "v gathered") if kv_outs else ("qkv", "q", "kT", "v gathered")
    for r in range(runs):
        for name, a, b in zip(names, got[False][r], got[True][r]):
            assert a == b, f"call {r}: {name} differs between the fused and the op-by-op run"
    qkv0 = _h(got[True][0][0], (M, N))
    qn = oracle.rmsnorm2(np.ascontiguousarray(qkv0[:, :H * hd]).reshape(-1, hd), qg, np.zeros(hd, np.float16))
    q_ref = oracle.rope(qn.reshape(M, -1), H, hd, 0, theta)
    d = np.abs(_h(got[True][0][1]).view(np.int16).astype(np.int32) - q_ref.reshape(-1).view(np.int16).astype(np.int32))
    assert d.max() <= 1 and (d == 0).mean() > 0.999   # RMSNorm's double sum order may flip 1 ulp


def test_qkv_gemm_rope_op_error_keeps_its_index(engine):
    """A q|k|v GEMM + OP_QK_ROPE_KV_F16 pair whose state cannot take the call (256 tokens
    into 64 slots) is not fused: the GEMM runs alone and the second op fails with its
    own 1-based index and the reference's message."""
    rng = np.random.default_rng(97)
    M, H, KVH, K, hd = 256, 16, 8, 1024, 128
    N = (H + 2 * KVH) * hd
    _, wq, ws = w4g_weights(rng, N, K)
    bb = BlobBuilder()
    st = bb.add_state(64 * KVH * hd * 4)
    xs = bb.add_input_slot(M * K * 2)
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    sqg = bb.add_slot(rng.uniform(0.8, 1.2, hd).astype(np.float16))
    t_qkv, t_q = bb.temp(), bb.temp()
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_qkv, M, K, N, WT_REF_NONE,
          WT_REF_NONE, 0, 2)
    bb.op(OP.QK_ROPE_KV_F16, t_qkv, t_q, WT_REF_NONE, WT_REF_NONE, st, M, H, KVH, hd, bb.slot_ref(sqg),
          bb.slot_ref(sqg), f32_bits(1e6))
    pb = engine.parse(bb.build())
    prev = engine.set_fusion(True)
    try:
        n0 = engine.qkv_rope_fused()
        with pytest.raises(WtExecError) as ei:
            engine.run_io(pb, normal_f16(rng, M, K).tobytes(), t_q)
        assert ei.value.rc == 2 and "nslots" in str(ei.value)
        assert engine.qkv_rope_fused() == n0
    finally:
        engine.set_fusion(prev)


def test_rmsnorm_then_w4g_gemm_runlist(engine, oracle):
    """Config 2 as a two-op runlist: RMSNORM2_F16 -> MATMUL_W4G_F16 (M=512)."""
    rng = np.random.default_rng(2)
    M, N, K = 512, 3072, 1024
    x = normal_f16(rng, M, K)
    gamma = rng.uniform(0.8, 1.2, K).astype(np.float16)
    _, wq, ws = w4g_weights(rng, N, K)
    bb = BlobBuilder()
    xs = bb.add_input_slot(M * K * 2)
    gs = bb.add_slot(gamma)
    zs = bb.add_slot(np.zeros(K, np.float16))
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    h, y = bb.temp(), bb.temp()
    bb.op(OP.RMSNORM2_F16, bb.slot_ref(xs), bb.slot_ref(gs), bb.slot_ref(zs), h, M * K)
    bb.op(OP.MATMUL_W4G_F16, h, bb.slot_ref(sq), bb.slot_ref(ss), y, M, K, N, 64, 2)
    pb = engine.parse(bb.build())
    out, _ = engine.run_io(pb, x.tobytes(), y, out_bytes=M * N * 2)
    h_ref = oracle.rmsnorm2(x, gamma, np.zeros(K, np.float16))
    h_got = _h(engine.temp(h), (M, K))
    assert np.abs(h_got.astype(np.float32) - h_ref.astype(np.float32)).max() <= 2e-3
    assert_close(_h(out, (M, N)), oracle.matmul_w4g(h_ref, wq, ws, threads=8), what="rms+gemm")


def _attention_chain_blob(S, H, KVH, hd, q, k, v):
    """Reference-style prefill attention: per kv-group batched MATMUL_F16 (q . k^T),
    BINARY mul (scale), BINARY add (causal mask), SOFTMAX, batched MATMUL_F16 (p . v).
    Heads are laid out [H, S, hd] (the reference chain's batched layout)."""
    rep = H // KVH
    bb = BlobBuilder()
    qh = np.ascontiguousarray(q.transpose(1, 0, 2))                       # [H,S,hd]
    kx = np.ascontiguousarray(np.repeat(k.transpose(1, 0, 2), rep, 0))     # [H,S,hd] (GQA expanded)
    vx = np.ascontiguousarray(np.repeat(v.transpose(1, 0, 2), rep, 0))
    sq, sk, sv = bb.add_slot(qh), bb.add_slot(kx), bb.add_slot(vx)
    scale = bb.add_slot(np.full(H * S * S, np.float16(SCALE), np.float16))
    mask = np.where(np.tril(np.ones((S, S), bool)), 0.0, -np.inf).astype(np.float16)
    smask = bb.add_slot(np.ascontiguousarray(np.broadcast_to(mask, (H, S, S))))
    t_s, t_sc, t_m, t_p, t_o = (bb.temp() for _ in range(5))
    bb.op(OP.MATMUL_F16, bb.slot_ref(sq), bb.slot_ref(sk), t_s, S, hd, S, (H << 16) | 4 | 2)
    bb.op(OP.BINARY_F16, t_s, bb.slot_ref(scale), t_sc, H * S * S, 2)
    bb.op(OP.BINARY_F16, t_sc, bb.slot_ref(smask), t_m, H * S * S, 0)
    bb.op(OP.SOFTMAX_F16, t_m, t_p, H * S, S)
    bb.op(OP.MATMUL_F16, t_p, bb.slot_ref(sv), t_o, S, S, hd, (H << 16) | 4)
    # fused op on the same data, token-major
    sq2, sk2, sv2 = bb.add_slot(q), bb.add_slot(k), bb.add_slot(v)
    t_f = bb.temp()
    bb.op(OP.ATTN_F16, bb.slot_ref(sq2), bb.slot_ref(sk2), bb.slot_ref(sv2), t_f, S, H, KVH, hd,
          f32_bits(SCALE), 1)
    return bb, t_o, t_f


def test_attention_chain_vs_fused_vs_oracle(engine, oracle):
    rng = np.random.default_rng(4)
    S, H, KVH, hd = 160, 4, 2, 128
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, KVH, hd), normal_f16(rng, S, KVH, hd)
    bb, t_chain, t_fused = _attention_chain_blob(S, H, KVH, hd, q, k, v)
    pb = engine.parse(bb.build())
    engine.run(pb)
    chain = _h(engine.temp(t_chain), (H, S, hd)).transpose(1, 0, 2)
    fused = _h(engine.temp(t_fused), (S, H, hd))
    ref = oracle.attn_prefill(q, k, v, SCALE, True)
    assert_close(chain, ref, what="runlist chain vs oracle")
    assert_close(fused, ref, what="fused vs oracle")


def test_attention_chain_fusion(engine, oracle):
    """Load-time fusion: the blob's first full run executes the reference chain op by op
    and finds its intermediates unread elsewhere; later runs execute it as one flash
    attention kernel (the third as a graph capture, the fourth as a replay). Every run
    stays within the parity tolerance of the oracle and of the op-by-op chain, and the
    chain's intermediates are no longer readable once it ran fused."""
    rng = np.random.default_rng(14)
    S, H, KVH, hd = 192, 4, 2, 128
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, KVH, hd), normal_f16(rng, S, KVH, hd)
    bb, t_chain, _ = _attention_chain_blob(S, H, KVH, hd, q, k, v)
    ref = oracle.attn_prefill(q, k, v, SCALE, True)
    prev = engine.set_fusion(True)
    try:
        pb = engine.parse(bb.build())
        found0, fused0 = engine.fusion_stats()
        outs = []
        for _ in range(4):
            engine.run(pb)
            outs.append(_h(engine.temp(t_chain), (H, S, hd)).transpose(1, 0, 2).copy())
        found1, fused1 = engine.fusion_stats()
        with pytest.raises(KeyError):
            engine.temp(3)   # the softmax output (temps 0..4 are the chain's), not computed
    finally:
        engine.set_fusion(prev)
    assert found1 - found0 == 1
    assert fused1 - fused0 == 3
    for i, o in enumerate(outs):
        assert_close(o, ref, what=f"run {i}")
    assert_close(outs[1], outs[0], what="fused vs op-by-op chain")
    assert np.array_equal(outs[3].view(np.uint16), outs[2].view(np.uint16))   # replay == capture
    assert np.array_equal(outs[2].view(np.uint16), outs[1].view(np.uint16))   # capture == direct


def test_attention_chain_unfused_when_intermediate_read(engine):
    """A later op reading the softmax output keeps the chain op by op: every run gives
    bit-identical results and the probabilities stay readable."""
    rng = np.random.default_rng(15)
    S, H, KVH, hd = 96, 2, 1, 128
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, KVH, hd), normal_f16(rng, S, KVH, hd)
    bb, t_chain, _ = _attention_chain_blob(S, H, KVH, hd, q, k, v)
    t_x = bb.temp()
    bb.op(OP.BINARY_F16, 3, 3, t_x, H * S * S, 0)   # p + p, after the chain
    pb = engine.parse(bb.build())
    found0, fused0 = engine.fusion_stats()
    outs = []
    for _ in range(3):
        engine.run(pb)
        outs.append(engine.temp(t_chain))
    p = _h(engine.temp(3), (H, S, S)).astype(np.float32)
    found1, fused1 = engine.fusion_stats()
    assert found1 - found0 == 1 and fused1 == fused0
    assert outs[0] == outs[1] == outs[2]
    assert np.allclose(p.sum(-1), 1.0, atol=2e-2)
    x = _h(engine.temp(t_x), (H, S, S)).astype(np.float32)
    assert np.array_equal(x, 2 * p)


@pytest.mark.parametrize("zero_mask", [True, False])
def test_attention_chain_fusion_noncausal(engine, oracle, zero_mask):
    """Chains with an all-zero mask op, or without a mask op, fuse as non-causal
    attention; with fusion switched off the same blob runs op by op."""
    rng = np.random.default_rng(16 + zero_mask)
    S, H, hd = 130, 2, 128
    q, k, v = normal_f16(rng, S, H, hd), normal_f16(rng, S, H, hd), normal_f16(rng, S, H, hd)
    bb = BlobBuilder()
    sq = bb.add_slot(np.ascontiguousarray(q.transpose(1, 0, 2)))
    sk = bb.add_slot(np.ascontiguousarray(k.transpose(1, 0, 2)))
    sv = bb.add_slot(np.ascontiguousarray(v.transpose(1, 0, 2)))
    scale = bb.add_slot(np.full(H * S * S, np.float16(SCALE), np.float16))
    t_s, t_sc, t_m, t_p, t_o = (bb.temp() for _ in range(5))
    bb.op(OP.MATMUL_F16, bb.slot_ref(sq), bb.slot_ref(sk), t_s, S, hd, S, (H << 16) | 4 | 2)
    bb.op(OP.BINARY_F16, t_s, bb.slot_ref(scale), t_sc, H * S * S, 2)
    src = t_sc
    if zero_mask:
        smask = bb.add_slot(np.zeros(H * S * S, np.float16))
        bb.op(OP.BINARY_F16, t_sc, bb.slot_ref(smask), t_m, H * S * S, 0)
        src = t_m
    bb.op(OP.SOFTMAX_F16, src, t_p, H * S, S)
    bb.op(OP.MATMUL_F16, t_p, bb.slot_ref(sv), t_o, S, S, hd, (H << 16) | 4)
    ref = oracle.attn_prefill(q, k, v, SCALE, False)
    found0, fused0 = engine.fusion_stats()
    prev = engine.set_fusion(False)
    try:
        pb = engine.parse(bb.build())
        for _ in range(2):
            engine.run(pb)
        chain = _h(engine.temp(t_o), (H, S, hd)).transpose(1, 0, 2).copy()
        assert engine.fusion_stats()[1] == fused0
    finally:
        engine.set_fusion(prev)
    pb = engine.parse(bb.build())
    for _ in range(2):
        engine.run(pb)
    fused = _h(engine.temp(t_o), (H, S, hd)).transpose(1, 0, 2)
    found1, fused1 = engine.fusion_stats()
    assert found1 - found0 == 1 and fused1 - fused0 == 1
    assert_close(chain, ref, what="op-by-op non-causal chain")
    assert_close(fused, ref, what="fused non-causal chain")


def _decode_blob(H, KVH, hd, max_pos):
    bb = BlobBuilder()
    kv_elems = KVH * hd
    st = bb.add_state(max_pos * kv_elems * 4)
    qs = bb.add_input_slot((H * hd + 2 * kv_elems) * 2)
    # the input face is [q | k | v]; three slices split it (STRIDED_SLICE, rank 1)
    tq, tk, tv, to = bb.temp(), bb.temp(), bb.temp(), bb.temp()
    n_in = H * hd + 2 * kv_elems
    for t, b0, n in ((tq, 0, H * hd), (tk, H * hd, kv_elems), (tv, H * hd + kv_elems, kv_elems)):
        bb.op(OP.STRIDED_SLICE_F16, bb.slot_ref(qs), t, n, 1, b0, 0, 0, b0 + n, 1, 1, 1, 1, 1, n_in, 1, 1)
    bb.op(OP.KV_APPEND_F16, tk, tv, st, WT_KV_POS_AUTO)
    bb.op(OP.ATTN_DECODE_F16, tq, st, to, WT_KV_POS_AUTO, H, KVH, hd, f32_bits(SCALE))
    return bb, to


def test_decode_loop_auto_positions(engine, oracle):
    """KV_APPEND (auto position) + ATTN_DECODE over 40 steps vs the reference ring + chain."""
    rng = np.random.default_rng(5)
    H, KVH, hd, max_pos = 16, 8, 128, 64
    bb, to = _decode_blob(H, KVH, hd, max_pos)
    pb = engine.parse(bb.build())
    ring = oracle.KVRing(max_pos * KVH * hd * 4, KVH * hd)
    for step in range(40):
        q, k, v = normal_f16(rng, H * hd), normal_f16(rng, KVH * hd), normal_f16(rng, KVH * hd)
        out, _ = engine.run_io(pb, np.concatenate([q, k, v]).tobytes(), to)
        ring.append(k, v)
        ref = ring.attn_decode(q, step + 1, H, KVH, hd, SCALE)
        assert_close(_h(out, (H, hd)), ref, what=f"decode step {step}")


@pytest.mark.parametrize("graphs", [False, True])
def test_decode_overflow_same_with_graphs(engine, oracle, graphs):
    """Filling the ring and appending once more fails at the KV_APPEND op with the
    reference's context error whether the steps ran direct or from a replayed graph;
    outputs of the steps before match the oracle either way."""
    rng = np.random.default_rng(8)
    H, KVH, hd, max_pos = 8, 4, 128, 12
    bb, to = _decode_blob(H, KVH, hd, max_pos)
    pb = engine.parse(bb.build())
    ring = oracle.KVRing(max_pos * KVH * hd * 4, KVH * hd)
    prev = engine.set_graphs(graphs)
    try:
        r0 = engine.graph_stats()[1]
        for step in range(max_pos):
            q, k, v = normal_f16(rng, H * hd), normal_f16(rng, KVH * hd), normal_f16(rng, KVH * hd)
            out, _ = engine.run_io(pb, np.concatenate([q, k, v]).tobytes(), to)
            ring.append(k, v)
            assert_close(_h(out, (H, hd)), ring.attn_decode(q, step + 1, H, KVH, hd, SCALE),
                         what=f"decode step {step}")
        replays = engine.graph_stats()[1] - r0
        assert (replays >= max_pos - 4) if graphs else replays == 0
        with pytest.raises(WtExecError) as ei:
            engine.run_io(pb, normal_f16(rng, H * hd + 2 * KVH * hd).tobytes(), to)
        assert ei.value.rc == 4 and "context too long" in str(ei.value)
    finally:
        engine.set_graphs(prev)


def test_kv_gather_and_overflow(engine, oracle):
    """KV_GATHER output layout (kT [H,hd,nslots] zero tail, v [H,nslots,hd]) is byte-exact;
    appending past nslots is the reference's hard error."""
    rng = np.random.default_rng(6)
    H, KVH, hd, max_pos = 4, 2, 128, 8
    kv = KVH * hd
    bb = BlobBuilder()
    st = bb.add_state(max_pos * kv * 4)
    ks, vs = bb.add_input_slot(kv * 2), bb.add_slot(np.zeros(kv, np.float16))
    bb.temp()                     # temp id 0 means "skip this face" in KV_GATHER
    tkT, tvo = bb.temp(), bb.temp()
    bb.op(OP.KV_APPEND_F16, bb.slot_ref(ks), bb.slot_ref(vs), st, WT_KV_POS_AUTO)
    bb.op(OP.KV_GATHER_F16, st, tkT, tvo, WT_KV_POS_AUTO, H, KVH, hd)
    pb = engine.parse(bb.build())
    ring = oracle.KVRing(max_pos * kv * 4, kv)
    for step in range(max_pos):
        k = normal_f16(rng, kv)
        engine.run_io(pb, k.tobytes(), tkT)
        ring.append(k, np.zeros(kv, np.float16))
        kT_ref, v_ref = ring.gather(step + 1, H, KVH, hd, pstride=max_pos)
        assert np.array_equal(_h(engine.temp(tkT)), kT_ref.ravel())
        assert np.array_equal(_h(engine.temp(tvo)), v_ref.ravel())
    with pytest.raises(WtExecError) as ei:
        engine.run_io(pb, normal_f16(rng, kv).tobytes(), tkT)
    assert ei.value.rc == 1 and "nslots" in str(ei.value)
    engine.state_reset()
    engine.run_io(pb, normal_f16(rng, kv).tobytes(), tkT)   # fresh sequence works again


def test_unported_opcode_fails_loudly(engine):
    bb = BlobBuilder()
    s = bb.add_slot(np.zeros(64, np.float16))
    t = bb.temp()
    bb.op(OP.NOP)
    bb.op(OP.SCATTER_ND_F16, bb.slot_ref(s), bb.slot_ref(s), bb.slot_ref(s), t, *([1] * 10))
    pb = engine.parse(bb.build())
    with pytest.raises(WtExecError) as ei:
        engine.run(pb)
    assert ei.value.rc == 2 and "no HIP kernel" in str(ei.value)


def test_tempoff_static_plan_matches_bump(engine, oracle):
    """The same two-op blob with and without a TEMPOFF plan gives identical bytes."""
    rng = np.random.default_rng(8)
    M, N, K = 4, 640, 256
    x = normal_f16(rng, M, K)
    gamma = rng.uniform(0.8, 1.2, K).astype(np.float16)
    _, wq, ws = w4g_weights(rng, N, K)

    def blob(static):
        bb = BlobBuilder()
        xs = bb.add_input_slot(M * K * 2)
        gs, zs = bb.add_slot(gamma), bb.add_slot(np.zeros(K, np.float16))
        sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
        bb.op(OP.RMSNORM2_F16, bb.slot_ref(xs), bb.slot_ref(gs), bb.slot_ref(zs), 0, M * K)
        bb.op(OP.MATMUL_W4G_F16, 0, bb.slot_ref(sq), bb.slot_ref(ss), 1, M, K, N, 64, 2)
        if static:
            bb.set_tempoff(1 << 20, [(0, 0, M * K * 2), (1, 65536, M * N * 2)], bump_kb=64)
        return bb.build()

    outs = []
    for static in (False, True):
        engine.shutdown()
        pb = engine.parse(blob(static))
        out, _ = engine.run_io(pb, x.tobytes(), 1)
        outs.append(out)
    assert outs[0] == outs[1]


@pytest.mark.parametrize("M,N,K", [(2048, 16384, 512), (256, 1024, 512), (3, 2048, 512), (1, 2048, 512)],
                         ids=["gemm-wide", "gemm", "gemv-m3", "gemv-m1"])
def test_swiglu_epilogue_matches_op_chain(engine, M, N, K):
    """OP_W4G_FUSED_F16 with SwiGLU (its silu read from the per-device table) gives the bits
    of the same linear without SwiGLU followed by the reference's own ops: STRIDED_SLICE of
    the gate and up columns, UNARY silu, BINARY mul. Covers the 128x256 and 128x128 GEMM
    tiles and the GEMV."""
    rng = np.random.default_rng(M + N)
    _, wq, ws = w4g_weights(rng, N, K)
    x = normal_f16(rng, M, K) * np.float16(2.0)
    bb = BlobBuilder()
    xs = bb.add_input_slot(M * K * 2)
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    t_f, t_p, t_g, t_u, t_a, t_y = (bb.temp() for _ in range(6))
    n = M * (N // 2)
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_f, M, K, N, WT_REF_NONE,
          WT_REF_NONE, 1, 2)
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_p, M, K, N, WT_REF_NONE,
          WT_REF_NONE, 0, 2)
    for t, c0 in ((t_g, 0), (t_u, 1)):
        bb.op(OP.STRIDED_SLICE_F16, t_p, t, n, 2, 0, c0, 0, M, N, 0, 1, 2, 0, M, N, 1)
    bb.op(OP.UNARY_F16, t_g, t_a, n, 12)
    bb.op(OP.BINARY_F16, t_a, t_u, t_y, n, 2)
    pb = engine.parse(bb.build())
    engine.run_io(pb, x.tobytes(), t_f)
    fused = _h(engine.temp(t_f))[:n]
    chain = _h(engine.temp(t_y))[:n]
    assert np.isfinite(fused.astype(np.float32)).all()
    assert np.array_equal(fused.view(np.uint16), chain.view(np.uint16))
