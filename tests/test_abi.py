"""The C-ABI boundary on the CPU: the library loads, exports every function the
headers declare, and wt_parse behaves exactly like the reference parser (compiled
from kernels/src/runtime/oplist_parse.c into oracle/_ref) on valid and corrupted
blobs. No GPU calls are made here."""
from __future__ import annotations

import ctypes as C
import hashlib
import re
import struct
from pathlib import Path

import numpy as np
import pytest

from gehtp_amd import abi
from gehtp_amd.abi import WtBlob, opcodes as OP
from gehtp_amd.runlist import BlobBuilder

ROOT = Path(__file__).resolve().parents[1]
REF_PARSE = ROOT / "oracle" / "_ref" / "libref_parse.so"


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"static inline[^{]*\{[^}]*\}", "", text)
        for m in re.finditer(r"\b(wt_\w+|gehtp_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_function(lib):
    declared = _declared_functions()
    assert {"wt_parse", "wt_exec_run_io", "gehtp_w4g_matmul", "gehtp_attn_decode"} <= declared
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert set(abi.EXPORTS) == declared, set(abi.EXPORTS) ^ declared
    assert lib.gehtp_version().startswith(b"gehtp-gfx950")


def test_struct_layouts():
    assert C.sizeof(abi.WtSlot) == 24 and abi.WtSlot.offset.offset == 8 and abi.WtSlot.addr.offset == 16
    assert C.sizeof(abi.WtOp) == 68
    assert abi.WtBlob.slots.offset == 16
    assert C.sizeof(abi.WtOpTs) == 20 and C.sizeof(abi.WtExecStats) == 52


def _sample_blob(rng, version=None):
    bb = BlobBuilder()
    x = bb.add_input_slot(256)
    w = bb.add_slot(rng.integers(0, 255, 3000, dtype=np.uint8).tobytes())
    s = bb.add_slot(np.ones(64, np.float16))
    st = bb.add_state(8 * 1024)
    bb.op(OP.NOP)
    bb.op(OP.PIN, bb.slot_ref(w))
    bb.op(OP.RMSNORM2_F16, bb.slot_ref(x), bb.slot_ref(s), bb.slot_ref(s), 0, 128)
    bb.op(OP.MATMUL_F16, 0, bb.slot_ref(w), 1, 2, 64, 3, 2)
    bb.op(OP.KV_APPEND_F16, 0, 1, st, abi.WT_KV_POS_AUTO)
    bb.op(OP.DMA, 0xC001, bb.slot_ref(w), 64, 0, 0, 0, 0xFF, 0xFF)
    return bb.build(version)


def _parse_both(lib, ref, data: bytes):
    buf = C.create_string_buffer(data, len(data))
    a, b = WtBlob(), WtBlob()
    ra = lib.wt_parse(C.cast(buf, C.POINTER(C.c_uint8)), len(data), C.byref(a))
    rb = ref.wt_parse(C.cast(buf, C.POINTER(C.c_uint8)), len(data), C.byref(b))
    return ra, rb, a, b


@pytest.fixture(scope="module")
def ref_parser():
    if not REF_PARSE.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ref = C.CDLL(str(REF_PARSE))
    ref.wt_parse.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.POINTER(WtBlob)]
    ref.wt_parse.restype = C.c_int
    return ref


def _same_blob(a: WtBlob, b: WtBlob):
    assert (a.ver, a.n_slots, a.n_ops, a.weight_off, a.weight_bytes) == \
           (b.ver, b.n_slots, b.n_ops, b.weight_off, b.weight_bytes)
    for i in range(a.n_slots):
        sa, sb = a.slots[i], b.slots[i]
        assert (sa.len, sa.count, sa.offset, sa.addr) == (sb.len, sb.count, sb.offset, sb.addr)
    for i in range(a.n_ops):
        oa, ob = a.ops[i], b.ops[i]
        assert (oa.opcode, oa.n_args) == (ob.opcode, ob.n_args)
        assert list(oa.args)[:oa.n_args] == list(ob.args)[:ob.n_args]


def test_parse_matches_reference_on_valid_blobs(lib, ref_parser):
    rng = np.random.default_rng(0)
    for ver in (1, 2):
        data = _sample_blob(rng, ver)
        ra, rb, a, b = _parse_both(lib, ref_parser, data)
        assert ra == rb == 0
        _same_blob(a, b)


def test_parse_error_codes_match_reference(lib, ref_parser):
    """The negative cases of kernels/examples/21_oplist_exec and compiler/tests/test_wtop_emit.cpp,
    plus random single-byte corruptions and truncations, all give the reference's code."""
    rng = np.random.default_rng(1)
    good = bytearray(_sample_blob(rng, 1))
    cases = {
        "short": bytes(good[:10]),
        "magic": b"WTOQ" + bytes(good[4:]),
        "ver": bytes(good[:4]) + struct.pack("<H", 3) + bytes(good[6:]),
        "endian": bytes(good[:6]) + struct.pack("<H", 0x3412) + bytes(good[8:]),
        "nslots0": bytes(good[:8]) + struct.pack("<I", 0) + bytes(good[12:]),
        "nslots_big": bytes(good[:8]) + struct.pack("<I", 4097) + bytes(good[12:]),
        "nops0": bytes(good[:12]) + struct.pack("<I", 0) + bytes(good[16:]),
        "slots_overrun": bytes(good[:40]),
    }
    expect = {"short": -1, "magic": -2, "ver": -3, "endian": -4, "nslots0": -5, "nslots_big": -5,
              "nops0": -6, "slots_overrun": -7}
    for name, data in cases.items():
        ra, rb, _, _ = _parse_both(lib, ref_parser, data)
        assert ra == rb == expect[name], (name, ra, rb)
    # op table: bad arity, unknown opcode, bad slot ref, misaligned slot offset
    n_slots = struct.unpack_from("<I", good, 8)[0]
    op0 = 16 + 16 * n_slots
    bad = bytearray(good); struct.pack_into("<H", bad, op0 + 2, 1)          # NOP with 1 arg
    assert _parse_both(lib, ref_parser, bytes(bad))[:2] == (-11, -11)
    bad = bytearray(good); struct.pack_into("<H", bad, op0, 31)             # unused opcode
    assert _parse_both(lib, ref_parser, bytes(bad))[:2] == (-10, -10)
    bad = bytearray(good); struct.pack_into("<I", bad, op0 + 4 + 4, 0x8000 | 99)   # PIN slot 99
    assert _parse_both(lib, ref_parser, bytes(bad))[:2] == (-12, -12)
    bad = bytearray(good); struct.pack_into("<I", bad, 16 + 16 + 8, 130)    # slot 1 offset % 128
    assert _parse_both(lib, ref_parser, bytes(bad))[:2] == (-13, -13)
    for cut in (op0 + 2, op0 + 6, len(good) - 1):
        ra, rb, _, _ = _parse_both(lib, ref_parser, bytes(good[:cut]))
        assert ra == rb, cut
    for _ in range(400):
        bad = bytearray(good)
        i = int(rng.integers(0, min(len(bad), op0 + 120)))
        bad[i] = int(rng.integers(0, 256))
        ra, rb, a, b = _parse_both(lib, ref_parser, bytes(bad))
        assert ra == rb, (i, ra, rb)
        if ra == 0:
            _same_blob(a, b)


def test_parse_accepts_added_opcodes_reference_rejects(lib, ref_parser):
    """Opcodes 40..44 are this library's additions: the reference parser rejects them."""
    bb = BlobBuilder()
    s = bb.add_slot(np.zeros(64, np.float16))
    bb.op(OP.MATMUL_W4G_F16, 0, bb.slot_ref(s), bb.slot_ref(s), 1, 1, 64, 2, 64, 2)
    ra, rb, _, _ = _parse_both(lib, ref_parser, bb.build())
    assert (ra, rb) == (0, -10)


def test_w3_report(lib):
    rng = np.random.default_rng(2)
    data = _sample_blob(rng, 1)
    buf = C.create_string_buffer(data, len(data))
    blob = WtBlob()
    assert lib.wt_parse(C.cast(buf, C.POINTER(C.c_uint8)), len(data), C.byref(blob)) == 0
    lines = []
    cb = C.CFUNCTYPE(None, C.c_char_p, C.c_void_p)(lambda s, ud: lines.append(s.decode()))
    lib.wt_w3_report(b"t.wtop", C.cast(buf, C.POINTER(C.c_uint8)), len(data), C.byref(blob), cb, None)
    assert len(lines) == 1 + blob.n_slots + blob.n_ops + 1
    assert f'"blob_sha256":"{hashlib.sha256(data).hexdigest()}"' in lines[0]
    w = data[blob.weight_off:]
    assert f'"weight_sha256":"{hashlib.sha256(w).hexdigest()}"' in lines[0]
    s1 = blob.slots[1]
    assert hashlib.sha256(w[s1.offset:s1.offset + s1.len]).hexdigest() in lines[2]
    assert lines[-1] == '{"t":"W3","verdict":"PASS"}'


def test_builder_layout_rules():
    bb = BlobBuilder()
    bb.add_slot(b"\x01" * 3)
    bb.add_slot(b"\x02" * 200)
    bb.op(OP.NOP)
    data = bb.build()
    n_slots, n_ops = struct.unpack_from("<II", data, 8)
    assert (n_slots, n_ops) == (2, 1)
    offs = [struct.unpack_from("<I", data, 16 + 16 * i + 8)[0] for i in range(2)]
    assert offs == [0, 128]
    woff = (16 + 32 + 4 + 127) // 128 * 128
    assert data[woff:woff + 3] == b"\x01" * 3 and data[woff + 128:woff + 328] == b"\x02" * 200


def test_python_io_buffers_sized_from_the_input_slot():
    """wt_exec_run_io / wt_exec_run_steps read the EXT_IN slot's length from the host input
    and run_steps writes steps times that length: the Python mirror checks the caller's
    bytes against the slot before any call (no GPU call is made: each raises first)."""
    from gehtp_amd import Engine
    bb = BlobBuilder()
    x = bb.add_input_slot(64)
    bb.op(OP.ARGMAX_F16, bb.slot_ref(x), 0, 32)
    eng = Engine()
    pb = eng.parse(bb.build())
    assert pb.input_bytes == 64
    with pytest.raises(ValueError, match="input slot 64"):
        eng.run_steps(pb, 4, b"\0" * 4, 0)
    with pytest.raises(ValueError, match="input slot 64"):
        eng.run_steps(pb, 4, b"\0" * 128, 0)
    with pytest.raises(ValueError, match="64 MiB"):
        eng.run_steps(pb, (64 << 20) // 64 + 1, b"\0" * 64, 0)
    with pytest.raises(ValueError, match="input slot 64"):
        eng.run_io(pb, b"\0" * 32, 0)
