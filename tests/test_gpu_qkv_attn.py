"""The decode step's q|k|v GEMV and its attention op in one launch (GPU): the chunk
workgroups take the new token's q / k / v rows from tagged records that the GEMV
workgroups of the same launch publish. Bit-identical to the two separate kernels and to
the op-by-op engine runs."""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import from_dev, normal_f16, ptr, stream_ptr, to_dev, w4g_weights

from gehtp_amd import WtExecError
from gehtp_amd.abi import WT_REF_NONE, opcodes as OP
from gehtp_amd.runlist import BlobBuilder, f32_bits

pytestmark = pytest.mark.gpu

SCALE = float(np.float16(1.0 / math.sqrt(128)))
GEHTP_ENOTSUP = -95


def _sync():
    import torch
    torch.cuda.synchronize()


@pytest.mark.parametrize("H,KVH,K,nslots,pos0", [
    (32, 8, 2560, 4096, 2059),   # the 4B decode shape at ~2k keys (spec chunks, 33 active)
    (32, 8, 2560, 4608, 3000),   # a grid too large for GEMV workgroups of three waves
    (32, 8, 2560, 256, 0),       # first position
    (16, 8, 1024, 256, 62),      # 0.8B-class; crosses a 64-key chunk boundary
    (16, 8, 4096, 512, 127),     # 32 lanes per row, 4 slices
    (8, 8, 2048, 128, 5),        # one query head per kv head
    (32, 4, 3072, 256, 191),     # eight query heads per kv head, 32 lanes x 3 slices
])
def test_qkv_attn_one_launch_matches_two_kernels(lib, oracle, torch_dev, H, KVH, K, nslots, pos0):
    """gehtp_qkv_attn_decode against gehtp_w4g_fused (RMSNorm + GEMV) followed by
    gehtp_attn_decode_qkv over three consecutive steps: the q|k|v row, the ring, the
    counter and the attention output bit-identical, and the hand-off never gave up
    (workspace word 3) while the call sequence number (word 2) advanced once per call."""
    import torch
    rng = np.random.default_rng(H * 7 + K + pos0)
    hd = 128
    N, kv_elems = (H + 2 * KVH) * hd, KVH * hd
    state_bytes = nslots * kv_elems * 4
    _, wq, ws = w4g_weights(rng, N, K)
    wq_d, ws_d = to_dev(wq, torch_dev), to_dev(ws, torch_dev)
    gam = to_dev(rng.uniform(0.2, 0.3, K).astype(np.float16), torch_dev)
    qg = to_dev(rng.uniform(0.8, 1.2, hd).astype(np.float16), torch_dev)
    kg = to_dev(rng.uniform(0.8, 1.2, hd).astype(np.float16), torch_dev)
    ring_ref = oracle.KVRing(state_bytes, kv_elems)
    for _ in range(pos0):
        ring_ref.append(normal_f16(rng, kv_elems), normal_f16(rng, kv_elems))
    ring_a = torch.from_numpy(ring_ref.buf.copy()).to(torch_dev)
    ring_b = ring_a.clone()
    count_a = torch.tensor([pos0], dtype=torch.int32, device=torch_dev)
    count_b = count_a.clone()
    wf_a = lib.gehtp_attn_decode_work_floats(nslots, H, hd)
    wf_b = lib.gehtp_attn_qkv_fused_work_floats(nslots, H, KVH)
    assert wf_b > wf_a
    work_a = torch.zeros(wf_a, dtype=torch.float32, device=torch_dev)
    work_b = torch.zeros(wf_b, dtype=torch.float32, device=torch_dev)
    qkv_a = torch.empty(N, dtype=torch.float16, device=torch_dev)
    qkv_b = torch.empty(N, dtype=torch.float16, device=torch_dev)
    out_a = torch.empty((H, hd), dtype=torch.float16, device=torch_dev)
    out_b = torch.empty((H, hd), dtype=torch.float16, device=torch_dev)
    for step in range(3):
        x = to_dev((normal_f16(rng, 1, K) * np.float16(2)).astype(np.float16), torch_dev)
        assert lib.gehtp_w4g_fused(ptr(x), K, ptr(wq_d), ptr(ws_d), ptr(qkv_a), N, 1, N, K, ptr(gam), None, N, 0,
                                   stream_ptr()) == 0
        assert lib.gehtp_attn_decode_qkv(ptr(qkv_a), H, KVH, ptr(qg), ptr(kg), 1e6, SCALE, ptr(ring_a), state_bytes,
                                         ptr(count_a), ptr(out_a), ptr(work_a), wf_a, stream_ptr()) == 0
        rc = lib.gehtp_qkv_attn_decode(ptr(x), ptr(wq_d), ptr(ws_d), ptr(gam), K, ptr(qkv_b), H, KVH, ptr(qg),
                                       ptr(kg), 1e6, SCALE, ptr(ring_b), state_bytes, ptr(count_b), ptr(out_b),
                                       ptr(work_b), wf_b, stream_ptr())
        assert rc == 0
        _sync()
        n_kv = pos0 + step + 1
        assert int(count_a.item()) == int(count_b.item()) == n_kv
        assert torch.equal(qkv_a, qkv_b), f"step {step}: q|k|v rows differ"
        assert torch.equal(ring_a, ring_b), f"step {step}: rings differ"
        assert np.array_equal(from_dev(out_a).view(np.int16), from_dev(out_b).view(np.int16)), f"step {step}"
        head = work_b[:4].cpu().view(torch.int32).numpy()
        assert head[3] == 0, "a hand-off wait gave up"
        assert head[2] == step + 1


@pytest.mark.parametrize("H,KVH,K,nslots,pos0,with_res", [(32, 8, 2560, 4096, 2059, True),
                                                          (16, 8, 1024, 256, 63, False),
                                                          (8, 8, 2048, 128, 0, True)])
def test_qkv_attn_oproj_two_launches_match_separate_calls(lib, torch_dev, H, KVH, K, nslots, pos0, with_res):
    """gehtp_qkv_attn_oproj_decode (the q|k|v GEMV + chunk pass, then the merge pass + the
    o-proj GEMV reading the attention output from the merge workgroups' records) against
    gehtp_w4g_fused -> gehtp_attn_decode_qkv -> gehtp_w4g_fused over three steps: the
    q|k|v row, the attention output, the o-proj output, the ring and the counter
    bit-identical; no hand-off wait gave up."""
    import torch
    rng = np.random.default_rng(H * 11 + K + pos0)
    hd = 128
    N, kv_elems, Ko = (H + 2 * KVH) * hd, KVH * hd, H * hd
    state_bytes = nslots * kv_elems * 4
    _, wq, ws = w4g_weights(rng, N, K)
    _, woq, wos = w4g_weights(rng, K, Ko)
    wq_d, ws_d, woq_d, wos_d = (to_dev(a, torch_dev) for a in (wq, ws, woq, wos))
    gam = to_dev(rng.uniform(0.2, 0.3, K).astype(np.float16), torch_dev)
    qg = to_dev(rng.uniform(0.8, 1.2, hd).astype(np.float16), torch_dev)
    kg = to_dev(rng.uniform(0.8, 1.2, hd).astype(np.float16), torch_dev)
    ring_a = torch.from_numpy(normal_f16(rng, state_bytes // 2)).to(torch_dev)
    ring_b = ring_a.clone()
    count_a = torch.tensor([pos0], dtype=torch.int32, device=torch_dev)
    count_b = count_a.clone()
    wf = lib.gehtp_attn_qkv_fused_work_floats(nslots, H, KVH)
    work_a = torch.zeros(wf, dtype=torch.float32, device=torch_dev)
    work_b = torch.zeros(wf, dtype=torch.float32, device=torch_dev)
    qkv_a, qkv_b = (torch.empty(N, dtype=torch.float16, device=torch_dev) for _ in range(2))
    out_a, out_b = (torch.empty((H, hd), dtype=torch.float16, device=torch_dev) for _ in range(2))
    y_a, y_b = (torch.empty(K, dtype=torch.float16, device=torch_dev) for _ in range(2))
    for step in range(3):
        x = to_dev((normal_f16(rng, 1, K) * np.float16(2)).astype(np.float16), torch_dev)
        res = ptr(x) if with_res else None
        assert lib.gehtp_w4g_fused(ptr(x), K, ptr(wq_d), ptr(ws_d), ptr(qkv_a), N, 1, N, K, ptr(gam), None, N, 0,
                                   stream_ptr()) == 0
        assert lib.gehtp_attn_decode_qkv(ptr(qkv_a), H, KVH, ptr(qg), ptr(kg), 1e6, SCALE, ptr(ring_a), state_bytes,
                                         ptr(count_a), ptr(out_a), ptr(work_a), wf, stream_ptr()) == 0
        assert lib.gehtp_w4g_fused(ptr(out_a), Ko, ptr(woq_d), ptr(wos_d), ptr(y_a), K, 1, K, Ko, None, res, K, 0,
                                   stream_ptr()) == 0
        rc = lib.gehtp_qkv_attn_oproj_decode(ptr(x), ptr(wq_d), ptr(ws_d), ptr(gam), K, ptr(qkv_b), H, KVH, ptr(qg),
                                             ptr(kg), 1e6, SCALE, ptr(ring_b), state_bytes, ptr(count_b), ptr(out_b),
                                             ptr(woq_d), ptr(wos_d), ptr(y_b), K, res, ptr(work_b), wf, stream_ptr())
        assert rc == 0
        _sync()
        assert int(count_a.item()) == int(count_b.item()) == pos0 + step + 1
        for name, a, b in (("q|k|v", qkv_a, qkv_b), ("attention", out_a, out_b), ("o-proj", y_a, y_b),
                           ("ring", ring_a, ring_b)):
            assert torch.equal(a, b), f"step {step}: {name} differs"
        assert int(work_b[:4].cpu().view(torch.int32).numpy()[3]) == 0, "a hand-off wait gave up"


def test_qkv_attn_one_launch_rejects_other_shapes(lib, torch_dev):
    """Shapes the one-launch form does not take return GEHTP_ENOTSUP and launch nothing
    (K = 1536 has no row-in-wave layout; a group of 3 query heads per kv head is not
    built); a workspace smaller than gehtp_attn_qkv_fused_work_floats is an argument
    error."""
    import torch
    dev = torch_dev
    buf = torch.zeros(1 << 22, dtype=torch.float16, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    work = torch.zeros(1 << 20, dtype=torch.float32, device=dev)
    p = ptr(buf)
    for (H, KVH, K) in [(16, 8, 1536), (24, 8, 2560)]:
        wf = lib.gehtp_attn_qkv_fused_work_floats(64, H, KVH)
        rc = lib.gehtp_qkv_attn_decode(p, p, p, p, K, p, H, KVH, p, p, 1e6, SCALE, p, 64 * KVH * 512, ptr(count),
                                       p, ptr(work), wf, stream_ptr())
        assert rc == GEHTP_ENOTSUP, (H, KVH, K, rc)
    wf = lib.gehtp_attn_qkv_fused_work_floats(64, 32, 8)
    rc = lib.gehtp_qkv_attn_decode(p, p, p, p, 2560, p, 32, 8, p, p, 1e6, SCALE, p, 64 * 8 * 512, ptr(count), p,
                                   ptr(work), wf - 2, stream_ptr())
    assert rc not in (0, GEHTP_ENOTSUP)
    _sync()
    assert int(count.item()) == 0


def _decode_blob(rng, H, KVH, K, nslots, with_gamma=True):
    hd = 128
    N, kv = (H + 2 * KVH) * hd, KVH * hd
    _, wq, ws = w4g_weights(rng, N, K)
    bb = BlobBuilder()
    st = bb.add_state(nslots * kv * 4)
    xs = bb.add_input_slot(K * 2)
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    sg = bb.add_slot(rng.uniform(0.2, 0.3, K).astype(np.float16))
    sqg = bb.add_slot(rng.uniform(0.8, 1.2, hd).astype(np.float16))
    skg = bb.add_slot(rng.uniform(0.8, 1.2, hd).astype(np.float16))
    t_qkv, t_o = bb.temp(), bb.temp()
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_qkv, 1, K, N,
          bb.slot_ref(sg) if with_gamma else WT_REF_NONE, WT_REF_NONE, 0, 2)
    bb.op(OP.ATTN_DECODE_QKV_F16, t_qkv, st, t_o, H, KVH, hd, bb.slot_ref(sqg), bb.slot_ref(skg), f32_bits(1e6),
          f32_bits(SCALE))
    return bb.build(), t_qkv, t_o


@pytest.mark.parametrize("H,KVH,K,nslots,steps,with_gamma", [(32, 8, 2560, 512, 70, True),
                                                              (16, 8, 1024, 128, 5, False)])
def test_engine_runs_decode_pair_in_one_launch(engine, torch_dev, H, KVH, K, nslots, steps, with_gamma):
    """OP_W4G_FUSED_F16 (M = 1) followed by the OP_ATTN_DECODE_QKV_F16 reading its output:
    with fusion on the engine runs both in one launch (later steps replayed from a HIP
    graph); over `steps` decode steps (crossing 64-key chunk boundaries) the q|k|v temp
    and the attention output are bit-identical to the op-by-op runs, and the counter of
    such executions advances once per step."""
    rng = np.random.default_rng(H + K + steps)
    blob, t_qkv, t_o = _decode_blob(rng, H, KVH, K, nslots, with_gamma)
    pb = engine.parse(blob)
    xs = [(normal_f16(rng, 1, K) * np.float16(2)).astype(np.float16) for _ in range(steps)]
    got = {}
    for fusion in (False, True):
        prev = engine.set_fusion(fusion)
        try:
            engine.state_reset()
            n0 = engine.qkv_attn_fused()
            res = []
            for x in xs:
                out, _ = engine.run_io(pb, x.tobytes(), t_o, out_bytes=H * 128 * 2)
                res.append((engine.temp(t_qkv), out))
            assert engine.qkv_attn_fused() - n0 == (steps if fusion else 0)
            got[fusion] = res
        finally:
            engine.set_fusion(prev)
    for s in range(steps):
        assert got[False][s][0] == got[True][s][0], f"step {s}: q|k|v differs"
        assert got[False][s][1] == got[True][s][1], f"step {s}: attention output differs"


def _decode_block_blob(rng, H, KVH, K, nslots, res_kind, plan_o_over_a=False):
    """q|k|v GEMV -> ATTN_DECODE_QKV -> o-proj GEMV (res_kind: 'x' = the block input as the
    residual, 'none'), then a second GEMV reading the o-proj output. plan_o_over_a: a
    TEMPOFF plan with the o-proj output at the attention output's offset."""
    hd = 128
    N, kv, Ko = (H + 2 * KVH) * hd, KVH * hd, H * hd
    _, wq, ws = w4g_weights(rng, N, K)
    _, woq, wos = w4g_weights(rng, K, Ko)
    bb = BlobBuilder()
    st = bb.add_state(nslots * kv * 4)
    xs = bb.add_input_slot(K * 2)
    sq, ss = bb.add_slot(wq, count=N * K), bb.add_slot(ws)
    soq, sos = bb.add_slot(woq, count=K * Ko), bb.add_slot(wos)
    sg = bb.add_slot(rng.uniform(0.2, 0.3, K).astype(np.float16))
    sqg = bb.add_slot(rng.uniform(0.8, 1.2, hd).astype(np.float16))
    skg = bb.add_slot(rng.uniform(0.8, 1.2, hd).astype(np.float16))
    t_qkv, t_a, t_o, t_y = bb.temp(), bb.temp(), bb.temp(), bb.temp()
    bb.op(OP.W4G_FUSED_F16, bb.slot_ref(xs), bb.slot_ref(sq), bb.slot_ref(ss), t_qkv, 1, K, N, bb.slot_ref(sg),
          WT_REF_NONE, 0, 2)
    bb.op(OP.ATTN_DECODE_QKV_F16, t_qkv, st, t_a, H, KVH, hd, bb.slot_ref(sqg), bb.slot_ref(skg), f32_bits(1e6),
          f32_bits(SCALE))
    bb.op(OP.W4G_FUSED_F16, t_a, bb.slot_ref(soq), bb.slot_ref(sos), t_o, 1, Ko, K, WT_REF_NONE,
          bb.slot_ref(xs) if res_kind == "x" else WT_REF_NONE, 0, 2)
    bb.op(OP.W4G_FUSED_F16, t_o, bb.slot_ref(sq), bb.slot_ref(ss), t_y, 1, K, N, bb.slot_ref(sg), WT_REF_NONE, 0, 2)
    if plan_o_over_a:
        sizes = {t_qkv: N * 2, t_a: Ko * 2, t_o: K * 2, t_y: N * 2}
        off, cap = {}, 0
        for t in (t_qkv, t_a, t_y):
            off[t] = cap
            cap += (sizes[t] + 127) // 128 * 128
        off[t_o] = off[t_a]
        bb.set_tempoff(cap, [(t, off[t], sizes[t]) for t in sorted(sizes)])
    return bb.build(), (t_qkv, t_a, t_o, t_y)


@pytest.mark.parametrize("H,KVH,K,nslots,steps,res_kind", [(32, 8, 2560, 512, 67, "x"), (16, 8, 1024, 256, 9, "none"),
                                                            (16, 8, 2048, 128, 4, "x")])
def test_engine_runs_merge_with_oproj(engine, torch_dev, H, KVH, K, nslots, steps, res_kind):
    """q|k|v GEMV -> ATTN_DECODE_QKV -> o-proj GEMV: with fusion on, the first launch runs
    the GEMV and the chunk pass, the second the merge pass and the o-proj GEMV (x taken
    from the merge workgroups' records; later steps replayed from a HIP graph). Every temp
    bit-identical to the op-by-op runs over `steps` decode steps; a run that ends right
    after the attention op (ops 0-1) still gets its merge pass; counters advance once
    per fused step (step 1 runs ops 0-1 and 2-3 as two runs on the previous step's input)."""
    rng = np.random.default_rng(H + K + steps + 7)
    blob, temps = _decode_block_blob(rng, H, KVH, K, nslots, res_kind)
    pb = engine.parse(blob)
    xs = [(normal_f16(rng, 1, K) * np.float16(2)).astype(np.float16) for _ in range(steps)]
    got = {}
    for fusion in (False, True):
        prev = engine.set_fusion(fusion)
        try:
            engine.state_reset()
            n0, m0 = engine.qkv_attn_fused(), engine.merge_oproj_fused()
            res = []
            for s, x in enumerate(xs):
                if s == 1:   # a run of the first two ops only (the last step's input), then the rest
                    engine.run(pb, first=0, count=2)
                    engine.run(pb, first=2, count=2)
                else:
                    engine.run_io(pb, x.tobytes(), temps[3])
                res.append([engine.temp(t) for t in temps])
            if fusion:
                assert engine.qkv_attn_fused() - n0 == steps
                assert engine.merge_oproj_fused() - m0 == steps - 1
            else:
                assert engine.qkv_attn_fused() == n0 and engine.merge_oproj_fused() == m0
            got[fusion] = res
        finally:
            engine.set_fusion(prev)
    names = ("qkv", "attention", "o-proj", "next GEMV")
    for s in range(steps):
        for name, a, b in zip(names, got[False][s], got[True][s]):
            assert a == b, f"step {s}: {name} differs between the fused and the op-by-op run"


def test_engine_merge_oproj_not_fused_when_output_overlaps(engine, torch_dev):
    """A TEMPOFF plan that places the o-proj output over the attention output (dead after
    the o-proj reads it; op by op that is legal): the merge pass may not share a launch
    with that GEMV (its workgroups store the attention output while the GEMV's store y),
    so the engine runs it alone; every temp equals the op-by-op run, the q|k|v GEMV +
    chunk pass launch is still taken."""
    rng = np.random.default_rng(41)
    H, KVH, K, nslots, steps = 32, 8, 2560, 256, 3
    blob_plain, temps = _decode_block_blob(rng, H, KVH, K, nslots, "x")
    rng = np.random.default_rng(41)
    bb_blob, temps2 = _decode_block_blob(rng, H, KVH, K, nslots, "x", plan_o_over_a=True)
    assert temps == temps2
    xs = [(normal_f16(rng, 1, K) * np.float16(2)).astype(np.float16) for _ in range(steps)]
    got = {}
    for name, blob, fusion in (("plain", blob_plain, False), ("aliased", bb_blob, True)):
        prev = engine.set_fusion(fusion)
        try:
            engine.shutdown()
            engine.state_reset()
            pb = engine.parse(blob)
            n0, m0 = engine.qkv_attn_fused(), engine.merge_oproj_fused()
            res = []
            for x in xs:
                engine.run_io(pb, x.tobytes(), temps[3])
                res.append([engine.temp(t) for t in (temps[0], temps[2], temps[3])])
            if fusion:
                assert engine.qkv_attn_fused() - n0 == steps
                assert engine.merge_oproj_fused() == m0
            got[name] = res
            engine.shutdown()
        finally:
            engine.set_fusion(prev)
    for s in range(steps):
        for what, a, b in zip(("qkv", "o-proj", "next GEMV"), got["plain"][s], got["aliased"][s]):
            assert a == b, f"step {s}: {what} differs"


def test_engine_decode_pair_error_keeps_its_index(engine, torch_dev):
    """A decode pair whose state is full (2 slots, third step) is not run in one launch:
    the GEMV runs alone and the attention op fails with its own 1-based index and the
    reference's message."""
    rng = np.random.default_rng(5)
    blob, t_qkv, t_o = _decode_blob(rng, 16, 8, 1024, 2)
    pb = engine.parse(blob)
    prev = engine.set_fusion(True)
    try:
        engine.state_reset()
        for _ in range(2):
            engine.run_io(pb, normal_f16(rng, 1, 1024).tobytes(), t_o)
        n0 = engine.qkv_attn_fused()
        with pytest.raises(WtExecError) as ei:
            engine.run_io(pb, normal_f16(rng, 1, 1024).tobytes(), t_o)
        assert ei.value.rc == 2 and "nslots" in str(ei.value)
        assert engine.qkv_attn_fused() == n0
    finally:
        engine.set_fusion(prev)
