"""The chain-form runlist emitter (gehtp_amd.qwen3_chain) on the CPU: its blobs parse,
carry the reference chain's opcodes (and none of this build's fused ones), and the
decode step body is the reference runner's (scripts/persistent_runtime.py:43-62)."""
from __future__ import annotations

import collections

import numpy as np

from gehtp_amd import Engine
from gehtp_amd.qwen3 import Qwen3Config, Weights
from gehtp_amd.qwen3_chain import decode_input, emit_decode_chain, emit_prefill_chain, face_elems, rope_tables

SMALL = Qwen3Config(layers=2, hidden=512, heads=4, kv_heads=2, ffn=1024, vocab=3000)


def _hist(blob):
    pb = Engine().parse(blob)
    return collections.Counter(pb.blob.ops[i].opcode for i in range(pb.n_ops)), pb.n_ops


def test_decode_chain_opcodes():
    w = Weights(SMALL, seed=1)
    hist, n = _hist(emit_decode_chain(SMALL, w, 64)[0])
    L = SMALL.layers
    # per layer: 22, 23, 24 x 2, 13, 7; RoPE 15 x 2 + 11 + 14 per q and k; 40 x 6
    assert hist[22] == L and hist[23] == L and hist[24] == 2 * L + 1 and hist[13] == L and hist[7] == L
    assert hist[40] == 6 * L and hist[14] == 2 * L and hist[20] == 1 and hist[21] == 1
    assert hist[15] == 3 + 6 * L and hist[26] == 5 and hist[11] == 3 * L
    assert not ({41, 42, 43, 44, 45, 46, 47} & set(hist)), "the chain form uses no fused opcode"


def test_prefill_chain_opcodes():
    w = Weights(SMALL, seed=1)
    hist, _ = _hist(emit_prefill_chain(SMALL, w, 16)[0])
    L = SMALL.layers
    assert hist[27] == 4 * L and hist[26] == 4 + 2 * L and hist[24] == 2 * L + 1 and hist[13] == L
    assert 22 not in hist and 23 not in hist


def test_decode_input_face():
    P = 16
    body = decode_input(SMALL, 1234, 0, P)
    assert len(body) == face_elems(SMALL, P) * 2
    assert np.frombuffer(body[:4], np.int32)[0] == 1234
    f = np.frombuffer(body[4:], np.float16)
    cos, sin, mask = f[:128], f[128:256], f[256:]
    assert (cos == 1).all() and (sin == 0).all()                # position 0
    assert mask[0] == 0 and np.isneginf(mask[1:]).all()
    body = decode_input(SMALL, 7, 5, P)
    f = np.frombuffer(body[4:], np.float16)
    c, s = rope_tables(np.array([5]), 128, SMALL.theta)
    assert np.array_equal(f[:128], c[0]) and np.array_equal(f[128:256], s[0])
    assert np.array_equal(f[:64], f[64:128])                     # each half duplicated
    # pair 0 rotates by exactly the position (inv_freq 1)
    assert f[0] == np.float16(np.cos(5.0)) and f[128] == np.float16(np.sin(5.0))
    assert (f[256:256 + 6] == 0).all() and np.isneginf(f[256 + 6:]).all()


def _detail(blob):
    eng = Engine()
    return eng.fusion_detail(eng.parse(blob))


def test_attention_chains_found_in_every_lowering():
    """The engine's fusion matchers (host code; no device call before a run) find one
    attention chain per layer in every lowering of the prefill and decode blobs: this
    build's chain form, the reference emitter's post-scale form (TRANSPOSE_GEN k^T,
    BROADCAST scale, BROADCAST mask + ADD_F16, one KV_GATHER per face) and its pre-scale
    form (q scaled before q.k^T), with fresh or recycled temp ids and with a TEMPOFF plan."""
    w = Weights(SMALL, seed=1)
    for lowering in ("chain", "ref_post", "ref_pre"):
        for recycle, tempoff in ((False, False), (True, False), (True, True)):
            pre = emit_prefill_chain(SMALL, w, 16, lowering=lowering, recycle=recycle, tempoff=tempoff)[0]
            dec = emit_decode_chain(SMALL, w, 64, lowering=lowering, recycle=recycle, tempoff=tempoff)[0]
            assert _detail(pre)["chains"] == SMALL.layers, (lowering, recycle, tempoff, "prefill")
            assert _detail(dec)["chains"] == SMALL.layers, (lowering, recycle, tempoff, "decode")


def test_reference_lowering_opcodes():
    """ref_pre writes BROADCAST -> BINARY -> MATMUL -> BROADCAST -> ADD_F16 -> SOFTMAX ->
    MATMUL around each prefill attention (qwen35_08b manifest ops 2722-2728), and the
    decode blob two single-face KV_GATHERs per layer."""
    w = Weights(SMALL, seed=1)
    pb = Engine().parse(emit_prefill_chain(SMALL, w, 16, lowering="ref_pre")[0])
    seq = [pb.blob.ops[i].opcode for i in range(pb.n_ops)]
    assert sum(seq[i:i + 7] == [26, 12, 24, 26, 7, 13, 24] for i in range(len(seq))) == SMALL.layers
    pb = Engine().parse(emit_decode_chain(SMALL, w, 64, lowering="ref_post")[0])
    gathers = [pb.blob.ops[i] for i in range(pb.n_ops) if pb.blob.ops[i].opcode == 23]
    assert len(gathers) == 2 * SMALL.layers
    assert all((g.args[1] == 0) != (g.args[2] == 0) for g in gathers)


def test_recycled_ids_and_tempoff_plan():
    """Recycling reuses ids the way the reference emitter's free list does (far fewer ids
    than ops), never hands an op's output the id of one of its own inputs, and the
    TEMPOFF plan gives ids busy at the same time disjoint bytes, while the run's values
    share them (the plan is far smaller than all outputs side by side)."""
    from gehtp_amd.runlist import BlobBuilder  # noqa: F401
    from gehtp_amd.qwen3_chain import _ChainEmitter  # noqa: F401
    from gehtp_amd import tempplan
    w = Weights(SMALL, seed=1)
    blob, t = emit_prefill_chain(SMALL, w, 16, lowering="ref_post", recycle=True, tempoff=True)
    pb = Engine().parse(blob)
    bb_like = type("B", (), {"state_bytes": []})()
    ops = [(pb.blob.ops[i].opcode, list(pb.blob.ops[i].args[:pb.blob.ops[i].n_args])) for i in range(pb.n_ops)]
    ids = set()
    spans = {}   # id -> [write, last read] of each of its values
    for i, (opc, args) in enumerate(ops):
        ins, outs = tempplan._roles(opc, args)
        assert not set(ins) & set(outs), f"op {i} writes over its own input"
        ids.update(ins + outs)
        for x in ins:
            spans[x][-1][1] = i
        for x in outs:
            spans.setdefault(x, []).append([i, i])
    for x in (t["logits"], t["tok"]):
        spans[x][-1][1] = len(ops)
    assert len(ids) < len(ops) // 3
    # the TEMPOFF slot's entries
    import struct
    from gehtp_amd.abi import WT_SLOT_TEMPOFF
    sl = [pb.blob.slots[i] for i in range(pb.n_slots) if pb.blob.slots[i].addr == WT_SLOT_TEMPOFF]
    assert len(sl) == 1
    raw = blob[pb.blob.weight_off + sl[0].offset:][:sl[0].len]
    cap, _, n = struct.unpack_from("<III", raw)
    ent = [struct.unpack_from("<III", raw, 12 + 12 * k) for k in range(n)]
    assert {e[0] for e in ent} == set(spans)
    for a in ent:
        assert a[1] + a[2] <= cap and a[1] % 128 == 0
        for b in ent:
            live_together = any(not (x[1] < y[0] or y[1] < x[0]) for x in spans[a[0]] for y in spans[b[0]])
            if a[0] < b[0] and live_together:
                assert a[1] + a[2] <= b[1] or b[1] + b[2] <= a[1], (a, b)
    # values share bytes: the plan is a fraction of every op output held apart
    total = sum(tempplan.out_bytes(bb_like, opc, args) * len(tempplan._roles(opc, args)[1]) for opc, args in ops)
    assert cap < total / 4
