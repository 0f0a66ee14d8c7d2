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
    # this build's fused opcodes (include/oplist_parse.h)
    OP.W4G_FUSED_F16: ((0, 8), (3,)),
    OP.QK_ROPE_KV_F16: ((0,), (1, 2, 3)),
    OP.ATTN_DECODE_QKV_F16: ((0,), (2,)),
    OP.ATTN_F16: ((0, 1, 2), (3,)),
    OP.ATTN_DECODE_F16: ((0,), (2,)),
}


def _is_temp(a: int) -> bool:   # WT_REF_NONE (0xFFFFFFFF) carries bit 15: no temp
    return not (a & 0x8000) and (a & 0xE000) != WT_REF_STATE_FLAG


def _positions(opc: int, args):
    """(input, output) argument positions holding temps."""
    if opc not in _ROLES:
        raise ValueError(f"recycle: no temp roles for opcode {opc}")
    ins, outs = _ROLES[opc]
    if opc == OP.KV_GATHER_F16:   # a face argument of 0 means no output
        outs = tuple(p for p in outs if args[p] != 0)
    if opc == OP.CONCAT_F16:
        ins = tuple(p for p in range(8) if p < 2 or args[p] != 0)
    return (tuple(p for p in ins if _is_temp(args[p])), tuple(p for p in outs if _is_temp(args[p])))


def _roles(opc: int, args):
    ins, outs = _positions(opc, args)
    return ([args[p] for p in ins], [args[p] for p in outs])


def recycle(bb, keep=()) -> dict:
    """Renumber the temps of bb's ops in place with the reference emitter's free list.
    Every write of a temp starts a new value (an emitter may write one id once per layer);
    a value's id returns to the list after its last read. Temps in `keep` (read after the
    run, e.g. logits) keep their last value to the end. Returns the map old id -> the new
    id of its last value."""
    # values: one per write; last read of each
    cur, last, n_val = {}, {}, 0
    vals_in, vals_out = [], []
    for i, (opc, args) in enumerate(bb.ops):
        ins, outs = _roles(opc, args)
        vin = []
        for t in ins:
            if t not in cur:
                raise ValueError(f"recycle: op {i} reads temp {t} before any write")
            vin.append(cur[t])
            last[cur[t]] = i
        vout = []
        for t in outs:
            cur[t] = n_val
            last.setdefault(n_val, i)
            vout.append(n_val)
            n_val += 1
        vals_in.append(vin)
        vals_out.append(vout)
    for t in keep:
        last[cur[t]] = len(bb.ops)
    # Ids start at 1: a KV_GATHER face argument of 0 means "no face", so id 0 could not
    # name a gathered face.
    free, nxt, vid = [], 1, {}
    for i, (opc, args) in enumerate(bb.ops):
        ins, outs = _roles(opc, args)
        amap = {t: vid[v] for t, v in zip(ins, vals_in[i])}
        for t, v in zip(outs, vals_out[i]):
            if free:
                vid[v] = free.pop()
            else:
                vid[v] = nxt
                nxt += 1
        omap = {t: vid[v] for t, v in zip(outs, vals_out[i])}
        p_in, p_out = _positions(opc, args)
        for p in p_in:
            args[p] = amap[args[p]]
        for p in p_out:
            args[p] = omap[args[p]]
        released = []
        for v in vals_in[i]:
            if last[v] == i and v not in released:
                released.append(v)
                free.append(vid[v])
        for v in vals_out[i]:   # written, never read (and not kept): free at once
            if last[v] == i and v not in vals_in[i] and v not in released:
                released.append(v)
                free.append(vid[v])
    bb.next_temp = nxt
    return {t: vid[v] for t, v in cur.items()}


def _state_slots(bb, st_ref: int, kv_elems: int) -> int:
    return bb.state_bytes[st_ref & 0x1FFF] // (kv_elems * 4)


def out_bytes(bb, opc: int, args, pos: int | None = None) -> int:
    """Bytes an op writes to its output temp at argument position `pos` (default: its
    first output; every KV_GATHER face has the same size)."""
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
    if opc == OP.W4G_FUSED_F16:   # [a, wq, ws, y, M, K, N, gamma, res, swiglu, flags]
        return a[4] * (a[6] // 2 if a[9] else a[6]) * 2
    if opc == OP.QK_ROPE_KV_F16:  # [qkv, q_out, k_out, v_out, state, S, H, KVH, hd, ...]
        heads = a[6] if (pos or 1) == 1 else a[7]
        return a[5] * heads * a[8] * 2
    if opc == OP.ATTN_DECODE_QKV_F16:   # [qkv, state, out, H, KVH, hd, ...]
        return a[3] * a[5] * 2
    if opc == OP.ATTN_F16:        # [q, k, v, out, S, H, KVH, hd, ...]
        return a[4] * a[5] * a[7] * 2
    if opc == OP.ATTN_DECODE_F16:  # [q, state, out, n_kv, H, KVH, hd, scale]
        return a[4] * a[6] * 2
    return 0


def tempoff_plan(bb, keep=(), align: int = 128):
    """(cap, [(tid, offset, size)]) for bb's (recycled) temps: each id holds one offset,
    busy over the spans of its values (each from its write to its last read; temps in
    `keep` to the end of the run); ids placed first fit at the lowest offset whose bytes
    no id busy at the same time holds."""
    spans, size = {}, {}
    for i, (opc, args) in enumerate(bb.ops):
        pin, pout = _positions(opc, args)
        for p in pin:
            spans[args[p]][-1][1] = i
        for p in pout:
            t = args[p]
            spans.setdefault(t, []).append([i, i])
            size[t] = max(size.get(t, 0), out_bytes(bb, opc, args, p))
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
