"""gehtp_amd — GEHTP's runlist engine on MI355X (gfx950), from Python.

The product is ``libgehtp.so`` (C ABI in ``include/``). This module loads it with
ctypes and mirrors the reference's host interface (``wt_parse``, ``wt_exec_run*``,
``wt_exec_temp*`` ...; reference ``kernels/include/oplist_exec.h``) so Python code
and tests drive the same entry points a C caller would.

Loading fails loudly when the library has not been built: there is no fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

from . import abi
from .abi import (WT_ERR, WtBlob, WtExecStats, WtOpTs, load_library, opcodes)

__all__ = ["abi", "WtBlob", "WtExecStats", "WtOpTs", "Engine", "ParsedBlob",
           "WtParseError", "WtExecError", "load_library", "opcodes", "lib_path"]

lib_path = Path(__file__).resolve().parent / "libgehtp.so"


class WtParseError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"wt_parse: {msg} ({rc})")
        self.rc = rc


class WtExecError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"wt_exec: rc={rc}: {msg}")
        self.rc = rc


class ParsedBlob:
    """A parsed blob: owns the byte buffer the wt_blob's weight_base points into."""

    def __init__(self, lib, data: bytes):
        self._buf = C.create_string_buffer(bytes(data), len(data))
        self.size = len(data)
        self.blob = WtBlob()
        rc = lib.wt_parse(C.cast(self._buf, C.POINTER(C.c_uint8)), C.c_size_t(len(data)),
                          C.byref(self.blob))
        if rc != 0:
            raise WtParseError(rc, lib.wt_err_str(rc).decode())
        ins = [self.blob.slots[i].len for i in range(self.blob.n_slots)
               if self.blob.slots[i].addr == abi.WT_SLOT_EXT_IN]
        self._input_bytes = max(ins, default=0)

    @property
    def n_ops(self) -> int:
        return self.blob.n_ops

    @property
    def n_slots(self) -> int:
        return self.blob.n_slots

    @property
    def input_bytes(self) -> int:
        """Bytes of the blob's EXT_IN input slot (the largest one; 0 if it has none): what
        wt_exec_run_io and wt_exec_run_steps read from their host input pointer."""
        return self._input_bytes


class Engine:
    """Process-wide engine (the library keeps one global instance, like the reference)."""

    def __init__(self, path: str | Path | None = None):
        self.lib = load_library(path or lib_path)
        self._obuf = None

    def parse(self, data: bytes) -> ParsedBlob:
        return ParsedBlob(self.lib, data)

    def _check(self, rc: int, err) -> None:
        if rc != 0:
            raise WtExecError(rc, err.value.decode(errors="replace"))

    def run(self, pb: ParsedBlob, first: int = 0, count: int | None = None, timing: bool = False):
        """wt_exec_run / wt_exec_run_range. Returns (engine_m, op_us list or None)."""
        count = pb.n_ops - first if count is None else count
        err = C.create_string_buffer(512)
        m = C.c_uint32(0)
        us = (C.c_int64 * max(count, 1))() if timing else None
        if first == 0 and count == pb.n_ops:
            rc = self.lib.wt_exec_run(C.byref(pb.blob), C.byref(m), us, err, 512)
        else:
            rc = self.lib.wt_exec_run_range(C.byref(pb.blob), first, count, C.byref(m), us, err, 512)
        self._check(rc, err)
        return m.value, (list(us) if timing else None)

    def run_io(self, pb: ParsedBlob, inp: bytes | None, out_temp: int, out_bytes: int | None = None,
               timing: bool = False):
        """wt_exec_run_io: returns (output bytes, op_us or None)."""
        err = C.create_string_buffer(512)
        m = C.c_uint32(0)
        us = (C.c_int64 * max(pb.n_ops, 1))() if timing else None
        # The library copies the input slot's length from in_ptr, whatever the caller
        # passed: a shorter buffer would be read past its end.
        if inp is not None and len(inp) < pb.input_bytes:
            raise ValueError(f"run_io: input holds {len(inp)} bytes, the blob's input slot {pb.input_bytes}")
        ibuf = C.c_char_p(bytes(inp)) if inp is not None else None
        # run_io copies the output temp's last-written bytes into out_ptr, so the buffer
        # must hold the largest output the caller expects (out_bytes, default 64 MiB).
        # One buffer per engine, allocated once: a fresh 64 MiB buffer per decode step
        # would cost more than the step.
        cap = max(out_bytes or 0, 64 << 20)
        if self._obuf is None or len(self._obuf) < cap:
            self._obuf = C.create_string_buffer(cap)
        rc = self.lib.wt_exec_run_io(C.byref(pb.blob), ibuf, self._obuf, out_temp, C.byref(m), us, err, 512)
        self._check(rc, err)
        n = self.lib.wt_exec_temp_last_bytes(out_temp)
        return C.string_at(self._obuf, n), (list(us) if timing else None)

    def run_steps(self, pb: ParsedBlob, steps: int, inp: bytes, out_temp: int) -> bytes:
        """wt_exec_run_steps: `steps` runs chained on the device (each run's out_temp bytes
        become the next run's input); returns the steps' outputs concatenated."""
        err = C.create_string_buffer(512)
        m = C.c_uint32(0)
        # The library reads the input slot's length from inp and writes steps times that
        # many bytes to the output: both buffers are sized from the slot, not from inp.
        n = pb.input_bytes
        if len(inp) != n:
            raise ValueError(f"run_steps: input holds {len(inp)} bytes, the blob's input slot {n}")
        if steps * n > (64 << 20):
            raise ValueError(f"run_steps: {steps} steps x {n} bytes exceed the 64 MiB output limit")
        obuf = C.create_string_buffer(max(steps * n, 1))
        rc = self.lib.wt_exec_run_steps(C.byref(pb.blob), steps, C.c_char_p(bytes(inp)), obuf, out_temp, C.byref(m),
                                        err, 512)
        self._check(rc, err)
        return obuf.raw[:steps * n]

    def temp(self, tid: int) -> bytes:
        """Bytes last written to temp tid (host copy)."""
        n = self.lib.wt_exec_temp_last_bytes(tid)
        p = self.lib.wt_exec_temp(tid)
        if not p:
            raise KeyError(f"temp {tid} not allocated, or an intermediate of an attention chain that ran fused")
        return C.string_at(p, n)

    def temp_bytes(self, tid: int) -> int:
        return self.lib.wt_exec_temp_bytes(tid)

    def temp_last_bytes(self, tid: int) -> int:
        return self.lib.wt_exec_temp_last_bytes(tid)

    def stats(self) -> WtExecStats:
        st = WtExecStats()
        self.lib.wt_exec_get_stats(C.byref(st))
        return st

    def shutdown(self) -> None:
        self.lib.wt_exec_shutdown()

    def state_reset(self) -> None:
        self.lib.wt_exec_state_reset()

    def set_ext_weights(self, buf) -> None:
        self._ext = buf
        self.lib.wt_exec_set_ext_weights(buf)

    def set_trace(self, on: bool) -> None:
        self.lib.wt_exec_set_trace(1 if on else 0)

    def set_graphs(self, on: bool) -> bool:
        """Graph replay of repeated runs on/off; returns the previous setting."""
        return bool(self.lib.wt_exec_set_graphs(1 if on else 0))

    def graph_stats(self) -> tuple[int, int]:
        """(graphs captured, graph replays) since the library was loaded."""
        c, r = C.c_uint32(0), C.c_uint32(0)
        self.lib.wt_exec_graph_stats(C.byref(c), C.byref(r))
        return c.value, r.value

    def set_input_device(self, ptr: int | None, nbytes: int = 0) -> None:
        """Bind a device buffer (address, bytes) as the input of later run_io calls made
        with inp=None; None unbinds. The buffer must stay alive and unchanged meanwhile."""
        self.lib.wt_exec_set_input_device(C.c_void_p(ptr) if ptr else None, nbytes if ptr else 0)

    def set_fusion(self, on: bool) -> bool:
        """Fuse the reference attention op chain into one kernel (default on);
        returns the previous setting."""
        return bool(self.lib.wt_exec_set_fusion(1 if on else 0))

    def fusion_stats(self) -> tuple[int, int]:
        """(attention chains found in the blobs seen, chain executions run fused)."""
        f, r = C.c_uint64(0), C.c_uint64(0)
        self.lib.wt_exec_fusion_stats(C.byref(f), C.byref(r))
        return f.value, r.value

    def fusion_detail(self, pb: ParsedBlob) -> dict:
        """The fusion plan of a blob after its first full run: chains found, chains the
        observed run ruled out, chains whose output overlapped an input in that run, and
        (process-wide) fused executions that wrote scratch because of such an overlap."""
        n, blk, al, runs = C.c_uint32(0), C.c_uint32(0), C.c_uint32(0), C.c_uint64(0)
        self.lib.wt_exec_fusion_detail(C.byref(pb.blob), C.byref(n), C.byref(blk), C.byref(al), C.byref(runs))
        return {"chains": n.value, "blocked": blk.value, "aliased": al.value, "alias_runs": runs.value}

    def qkv_rope_fused(self) -> int:
        """QK-norm/RoPE/KV-append ops performed by their q|k|v GEMM's epilogue so far."""
        return int(self.lib.wt_exec_qkv_rope_fused())

    def qkv_attn_fused(self) -> int:
        """Decode attention ops run in their q|k|v GEMV's launch so far."""
        return int(self.lib.wt_exec_qkv_attn_fused())

    def merge_oproj_fused(self) -> int:
        """o-proj GEMVs run in one launch with the decode attention's merge pass so far."""
        return int(self.lib.wt_exec_merge_oproj_fused())


WT_ERR = WT_ERR
