"""Temp-id recycling and TEMPOFF plans (gehtp_amd.tempplan) on the CPU, for the chain-form
emitter and this build's fused-opcode emitter: recycling keeps every read bound to the
same write (the blob computes the same dataflow with fewer ids), and a plan gives ids that
are live at the same time disjoint bytes inside its cap."""
from __future__ import annotations

import struct

import pytest

from gehtp_amd import Engine
from gehtp_amd.abi import WT_SLOT_TEMPOFF
from gehtp_amd.qwen3 import Qwen3Config, Weights, emit_decode, emit_prefill
from gehtp_amd.qwen3_chain import emit_decode_chain, emit_prefill_chain
from gehtp_amd import tempplan

SMALL = Qwen3Config(layers=2, hidden=512, heads=4, kv_heads=2, ffn=1024, vocab=3000)


def _ops(blob):
    pb = Engine().parse(blob)
    ops = [(pb.blob.ops[i].opcode, list(pb.blob.ops[i].args[:pb.blob.ops[i].n_args])) for i in range(pb.n_ops)]
    return pb, ops


def _dataflow(ops):
    """For each op and input position: the index of the op whose write it reads."""
    writer, flow = {}, []
    for i, (opc, args) in enumerate(ops):
        pin, pout = tempplan._positions(opc, args)
        flow.append(tuple(writer.get(args[p], -1) for p in pin))
        for p in pout:
            writer[args[p]] = i
    return flow


def _spans(ops, keep):
    spans = {}
    for i, (opc, args) in enumerate(ops):
        pin, pout = tempplan._positions(opc, args)
        for p in pin:
            spans[args[p]][-1][1] = i
        for p in pout:
            spans.setdefault(args[p], []).append([i, i])
    for t in keep:
        spans[t][-1][1] = len(ops)
    return spans


def _plan(blob, pb):
    sl = [pb.blob.slots[i] for i in range(pb.n_slots) if pb.blob.slots[i].addr == WT_SLOT_TEMPOFF]
    assert len(sl) == 1
    raw = blob[pb.blob.weight_off + sl[0].offset:][:sl[0].len]
    cap, _, n = struct.unpack_from("<III", raw)
    return cap, [struct.unpack_from("<III", raw, 12 + 12 * k) for k in range(n)]


def _check_plan(blob, keep):
    pb, ops = _ops(blob)
    cap, ent = _plan(blob, pb)
    spans = _spans(ops, keep)
    assert {e[0] for e in ent} == set(spans)
    for a in ent:
        assert a[1] % 128 == 0 and a[1] + a[2] <= cap
        for b in ent:
            if a[0] < b[0] and any(not (x[1] < y[0] or y[1] < x[0]) for x in spans[a[0]] for y in spans[b[0]]):
                assert a[1] + a[2] <= b[1] or b[1] + b[2] <= a[1], (a, b)
    return cap, ent


EMITTERS = [
    ("fused prefill", lambda w, **k: emit_prefill(SMALL, w, 24, 64, **k)),
    ("fused decode", lambda w, **k: emit_decode(SMALL, w, 64, **k)),
    ("fused decode, token input", lambda w, **k: emit_decode(SMALL, w, 64, token_input=True, **k)),
    ("chain prefill ref_post", lambda w, **k: emit_prefill_chain(SMALL, w, 16, lowering="ref_post", **k)),
    ("chain decode ref_pre", lambda w, **k: emit_decode_chain(SMALL, w, 64, lowering="ref_pre", **k)),
]


@pytest.mark.parametrize("name,emit", EMITTERS, ids=[e[0] for e in EMITTERS])
def test_recycling_keeps_the_dataflow(name, emit):
    w = Weights(SMALL, seed=2)
    plain, _ = emit(w)
    rec, t = emit(w, recycle=True)
    _, ops0 = _ops(plain)
    _, ops1 = _ops(rec)
    assert [o[0] for o in ops0] == [o[0] for o in ops1]
    assert _dataflow(ops0) == _dataflow(ops1)
    ids0 = {a for opc, args in ops0 for p in sum(tempplan._positions(opc, args), ()) for a in [args[p]]}
    ids1 = {a for opc, args in ops1 for p in sum(tempplan._positions(opc, args), ()) for a in [args[p]]}
    assert len(ids1) <= len(ids0) and 0 not in ids1
    for opc, args in ops1:   # no op writes over its own input
        ins, outs = tempplan._roles(opc, args)
        assert not set(ins) & set(outs)


@pytest.mark.parametrize("name,emit", EMITTERS, ids=[e[0] for e in EMITTERS])
@pytest.mark.parametrize("recycle", [False, True])
def test_tempoff_plans_are_disjoint_where_live(name, emit, recycle):
    w = Weights(SMALL, seed=2)
    blob, t = emit(w, recycle=recycle, tempoff=True)
    _check_plan(blob, [t["logits"], t["tok"]])


def test_fused_prefill_plan_shares_bytes():
    """This build's prefill blob reuses one id per tensor role in every layer; its plan
    lets the roles whose values never meet (the SwiGLU activation and the attention
    tensors) share bytes."""
    w = Weights(SMALL, seed=2)
    blob, t = emit_prefill(SMALL, w, 24, 64, tempoff=True)
    cap, ent = _check_plan(blob, [t["logits"], t["tok"]])
    assert cap < sum((e[2] + 127) // 128 * 128 for e in ent)
