"""Writes the golden fixtures in tests/golden/ (run from the repo root; needs oracle/_ref).

Reference-derived vectors come from the reference's own C sources compiled as they lie
(oracle/_ref: kernels/src/runtime/oplist_parse.c, kvcache.c, kernels/src/hvx/hvx_softmax.c),
run on fixed seeded inputs. Oracle-derived vectors (file names starting with oracle_)
freeze this repository's restatement for paths no reference function covers (the W4G
group-64 format), so any later change to it shows up.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from gehtp_amd.abi import WtBlob, opcodes as OP  # noqa: E402
from gehtp_amd.runlist import BlobBuilder  # noqa: E402
from oracle import oracle as o  # noqa: E402

OUT = Path(__file__).resolve().parent


def ref_softmax():
    ref = C.CDLL(str(o.REF / "libref_softmax.so"))
    ref.hvhx_v2_softmax_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
    rng = np.random.default_rng(101)
    x = (rng.standard_normal((8, 256)) * 4).astype(np.float16)
    xf = o.f16_to_f32(x.view(np.uint16))
    y = np.empty_like(xf)
    pad = np.empty(256, np.float32)
    for r in range(8):
        src = np.ascontiguousarray(xf[r])
        dst = np.empty(256, np.float32)
        ref.hvhx_v2_softmax_f32(src.ctypes.data, dst.ctypes.data, pad.ctypes.data, 256)
        y[r] = dst
    np.savez(OUT / "ref_softmax_host.npz", x=x, y_f32=y, y_f16=o.f32_to_f16(y).view(np.float16))


def ref_kvcache():
    class Kvc(C.Structure):
        _fields_ = [("base", C.c_void_p), ("slot_bytes", C.c_uint32), ("nslots", C.c_uint32),
                    ("posmap", C.c_void_p), ("consumer", C.c_int), ("mem", C.c_int),
                    ("n_append", C.c_uint32), ("n_evict", C.c_uint32)]
    ref = C.CDLL(str(o.REF / "libref_kvcache.so"))
    ref.kvc_init.argtypes = [C.POINTER(Kvc), C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
    ref.kvc_append.argtypes = [C.POINTER(Kvc), C.c_void_p, C.c_void_p, C.c_uint32]
    kv_elems, nslots = 256, 6
    state = nslots * kv_elems * 4
    buf = np.zeros(state + 128, np.uint8)
    base = (buf.ctypes.data + 127) // 128 * 128
    off = base - buf.ctypes.data
    posmap = np.zeros(nslots, np.uint32)
    c = Kvc()
    assert ref.kvc_init(C.byref(c), base, kv_elems * 4, nslots, posmap.ctypes.data) == 0
    rng = np.random.default_rng(102)
    pos = np.array([0, 1, 2, 3, 4, 5, 6, 7, 9, 3], np.uint32)
    ks = rng.standard_normal((len(pos), kv_elems)).astype(np.float16)
    vs = rng.standard_normal((len(pos), kv_elems)).astype(np.float16)
    slots = []
    for i, p in enumerate(pos):
        slots.append(ref.kvc_append(C.byref(c), ks[i].ctypes.data, vs[i].ctypes.data, int(p)))
    np.savez(OUT / "ref_kvcache.npz", pos=pos, k=ks, v=vs, slots=np.array(slots, np.int32),
             ring=buf[off:off + state].copy(), posmap=posmap.copy(), kv_elems=kv_elems, nslots=nslots)


def ref_parse():
    ref = C.CDLL(str(o.REF / "libref_parse.so"))
    ref.wt_parse.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.POINTER(WtBlob)]
    bb = BlobBuilder()
    x = bb.add_input_slot(256)
    w = bb.add_slot(np.arange(3000, dtype=np.uint16).astype(np.uint8).tobytes())
    s = bb.add_slot(np.ones(64, np.float16))
    bb.add_state(8 * 1024)
    bb.op(OP.NOP)
    bb.op(OP.PIN, bb.slot_ref(w))
    bb.op(OP.RMSNORM2_F16, bb.slot_ref(x), bb.slot_ref(s), bb.slot_ref(s), 0, 128)
    bb.op(OP.MATMUL_F16, 0, bb.slot_ref(w), 1, 2, 64, 3, 2)
    good = bb.build(1)
    rng = np.random.default_rng(103)
    blobs, codes = [good], []
    for _ in range(63):
        bad = bytearray(good)
        i = int(rng.integers(0, 300))
        bad[i] = int(rng.integers(0, 256))
        cut = int(rng.integers(16, len(bad) + 1)) if rng.random() < 0.2 else len(bad)
        blobs.append(bytes(bad[:cut]))
    for b in blobs:
        buf = C.create_string_buffer(b, len(b))
        codes.append(ref.wt_parse(C.cast(buf, C.POINTER(C.c_uint8)), len(b), C.byref(WtBlob())))
    lens = np.array([len(b) for b in blobs], np.int64)
    np.savez(OUT / "ref_parse.npz", data=np.frombuffer(b"".join(blobs), np.uint8), lens=lens,
             codes=np.array(codes, np.int32))


def oracle_w4g():
    rng = np.random.default_rng(104)
    N, K, M = 96, 256, 3
    q = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    wq = o.w4g_pack(q)
    ws = rng.uniform(0.005, 0.02, size=(N, K // 64)).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    np.savez(OUT / "oracle_w4g_small.npz", wq=wq, ws=ws, x=x, w=o.w4g_dequant(wq, ws, K),
             y=o.matmul_w4g(x, wq, ws))


if __name__ == "__main__":
    if not (o.REF / "libref_parse.so").exists():
        sys.exit("oracle/_ref is not built (needs the reference tree): run `make -C oracle`")
    ref_softmax()
    ref_kvcache()
    ref_parse()
    oracle_w4g()
    print("fixtures written to", OUT)
