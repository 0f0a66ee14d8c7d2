"""Temp-id recycling and a static temp plan (TEMPOFF) for emitted runlists.

The reference emitter hands out temp ids from a free list: after each op, the temps
whose last consumer it was go back on the list, and the next output takes the id
released last (compiler/tools/wtop_ops/wtop_ops.hpp:131-146, released after each op in
compiler/tools/wtop_emit.cpp:562-565; an op's output is allocated before its inputs
are released, so no op writes over its own input). Its compiler also fixes each temp's
device offset ahead of time, reusing the bytes of temps no longer live, and the emitter
writes that plan into the TEMPOFF slot (compiler/tools/wtop_emit.cpp:569-602):
[cap][reserve: lo16 bump KB | hi16 VTCM KB][n][n x {tid, offset, size}].

`recycle` renumbers a BlobBuilder's temps the same way, and `tempoff_plan` builds a
plan over the renumbered ids: one offset per id, held from the id's first write to its
last read, first fit at the lowest offset free over that span, so temps whose spans do
not meet share bytes.
"""
from __future__ import annotations

import numpy as np

from .abi import WT_KV_POS_AUTO, WT_REF_STATE_FLAG, opcodes as OP

# Temp roles per opcode: (input argument positions, output argument positions).
_ROLES = {
    OP.ADD_F16: ((0, 1), (2,)),
    OP.UNARY_F16: ((0,), (1,)),
    OP.BINARY_F16: ((0, 1), (2,)),
    OP.SOFTMAX_F16: ((0,), (1,)),
    OP.CONCAT_F16: ((0, 1), (8,)),
    OP.STRIDED_SLICE_F16: ((0,), (1,)),
    OP.GATHER_F16: ((0, 1), (2,)),
    OP.ARGMAX_F16: ((0,), (1,)),
    OP.KV_APPEND_F16: ((0, 1), ()),
    OP.KV_GATHER_F16: ((), (1, 2)),
    OP.MATMUL_F16: ((0, 1), (2,)),
    OP.RMSNORM2_F16: ((0,), (3,)),
    OP.BROADCAST_F16: ((0,), (1,)),
    OP.TRANSPOSE_GEN_F16: ((0,), (1,)),
    OP.MATMUL_W4G_F16: ((0,), (3,)),
}


def _is_temp(a: int) -> bool:
    return not (a & 0x8000) and (a & 0xE000) != WT_REF_STATE_FLAG


def _roles(opc: int, args):
    if opc not in _ROLES:
        raise ValueError(f"recycle: no temp roles for opcode {opc}")
    ins, outs = _ROLES[opc]
    if opc == OP.KV_GATHER_F16:   # a face argument of 0 means no output
        outs = tuple(p for p in outs if args[p] != 0)
    if opc == OP.CONCAT_F16:
        ins = tuple(p for p in range(8) if p < 2 or args[p] != 0)
    return ([args[p] for p in ins if _is_temp(args[p])], [args[p] for p in outs if _is_temp(args[p])])


def recycle(bb, keep=()) -> dict:
    """Renumber the temps of bb's ops in place with the reference emitter's free list;
    temps in `keep` (read after the run, e.g. logits) are never released. Returns the
    map old id -> new id."""
    last = {}
    for i, (opc, args) in enumerate(bb.ops):
        for t in _roles(opc, args)[0]:
            last[t] = i
    for t in keep:
        last[t] = len(bb.ops)
    # Ids start at 1: a KV_GATHER face argument of 0 means "no face", so id 0 could not
    # name a gathered face.
    free, nxt, new = [], 1, {}
    for i, (opc, args) in enumerate(bb.ops):
        ins, outs = _roles(opc, args)
        ins_new = [new[t] for t in ins]   # an input is always written before it is read
        for t in outs:
            if t in new and last.get(t, -1) > i:
                raise ValueError(f"recycle: temp {t} written again while live (op {i})")
            if free:
                new[t] = free.pop()
            else:
                new[t] = nxt
                nxt += 1
        amap = dict(zip(ins, ins_new))
        amap.update({t: new[t] for t in outs})
        p_ins, p_outs = _ROLES[opc]
        for p in set(p_ins) | set(p_outs):
            if p < len(args) and _is_temp(args[p]) and args[p] in amap:
                args[p] = amap[args[p]]
        released = []
        for t in ins:
            if last.get(t) == i and t not in released:
                released.append(t)
                free.append(new[t])
    bb.next_temp = nxt
    return new


def _state_slots(bb, st_ref: int, kv_elems: int) -> int:
    return bb.state_bytes[st_ref & 0x1FFF] // (kv_elems * 4)


def out_bytes(bb, opc: int, args) -> int:
    """Bytes an op writes to its output temp(s) (per face for KV_GATHER)."""
    a = args
    if opc in (OP.ADD_F16, OP.BINARY_F16):
        return a[3] * 2
    if opc == OP.UNARY_F16:
        return a[2] * 2
    if opc == OP.SOFTMAX_F16:
        return a[2] * a[3] * 2
    if opc == OP.CONCAT_F16:
        return a[11] * 2
    if opc in (OP.STRIDED_SLICE_F16, OP.BROADCAST_F16):
        return a[2] * 2
    if opc == OP.GATHER_F16:
        return a[3] * 2
    if opc == OP.ARGMAX_F16:
        return 4
    if opc == OP.MATMUL_F16:
        bn = (a[6] >> 16) if a[6] & 4 else 1
        return a[3] * a[5] * max(bn, 1) * 2
    if opc == OP.RMSNORM2_F16:
        return a[4] * 2
    if opc == OP.TRANSPOSE_GEN_F16:
        return int(np.prod(a[3:3 + a[2]])) * 2
    if opc == OP.MATMUL_W4G_F16:
        return a[4] * a[6] * 2
    if opc == OP.KV_GATHER_F16:
        P = a[3] if a[3] != WT_KV_POS_AUTO else _state_slots(bb, a[0], a[5] * a[6])
        return a[4] * a[6] * P * 2
    return 0


def tempoff_plan(bb, keep=(), align: int = 128):
    """(cap, [(tid, offset, size)]) for bb's (recycled) temps: each id holds one offset,
    busy over the spans of its values (each from its write to its last read; temps in
    `keep` to the end of the run); ids placed first fit at the lowest offset whose bytes
    no id busy at the same time holds."""
    spans, size = {}, {}
    for i, (opc, args) in enumerate(bb.ops):
        ins, outs = _roles(opc, args)
        for t in ins:
            spans[t][-1][1] = i
        nb = out_bytes(bb, opc, args)
        for t in outs:
            spans.setdefault(t, []).append([i, i])
            size[t] = max(size.get(t, 0), nb)
    for t in keep:
        spans[t][-1][1] = len(bb.ops)

    def meet(a, b):
        return any(not (x[1] < y[0] or y[1] < x[0]) for x in a for y in b)

    placed = []   # (id, off, end)
    entries, cap = [], 0
    for t in sorted(spans, key=lambda x: (spans[x][0][0], x)):
        sz = (size[t] + align - 1) // align * align
        busy = sorted((o, e) for u, o, e in placed if meet(spans[u], spans[t]))
        off = 0
        for o, e in busy:
            if off + sz <= o:
                break
            off = max(off, e)
        placed.append((t, off, off + sz))
        entries.append((t, off, size[t]))
        cap = max(cap, off + sz)
    return cap, entries
