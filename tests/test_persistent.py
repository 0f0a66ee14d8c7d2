"""The resident decode server (gehtp_amd/gehtp_persistent) and its client: the
request/response protocol of the reference's persistent runner
(kernels/examples/42_gehtp_persistent/main.c:14-31) over local files. These requests
never reach the GPU (ping, reset, shutdown, malformed frames); decode runs through the
server are checked in tests/test_gpu_model.py."""
from __future__ import annotations

import json
import struct
import time

import numpy as np
import pytest

from gehtp_amd.abi import opcodes as OP
from gehtp_amd.persistent import SERVER, PersistentRuntime, PersistentRuntimeError
from gehtp_amd.runlist import BlobBuilder

pytestmark = pytest.mark.skipif(not SERVER.exists(), reason="server not built (python -m gehtp_amd.build)")


def _blob(tmp_path):
    bb = BlobBuilder()
    bb.add_input_slot(64 * 2)
    t = bb.temp()
    bb.op(OP.NOP)
    p = tmp_path / "tiny.wtop"
    p.write_bytes(bb.build())
    return p, t


def test_server_lifecycle_and_errors(tmp_path):
    blob, t = _blob(tmp_path)
    rt = PersistentRuntime(tmp_path / "persist", timeout=20.0)
    info = rt.start_server(blob, out_temp=t, in_bytes=128, idle_exit_s=60)
    try:
        assert info["pid"] > 0 and rt.server_running()
        assert rt.ping() == {"rc": 0, "pong": 1}
        assert rt.reset() == {"rc": 0, "reset": 1}
        with pytest.raises(PersistentRuntimeError, match="bad_op"):
            rt._rpc({"op": "explode"})
        # a frame longer than the header says (op != run: no body expected)
        j = json.dumps({"op": "ping"}).encode()
        rt.req.write_bytes(struct.pack("!I", len(j)) + j + b"extra")
        deadline = time.monotonic() + 20
        while not rt.resp.exists() and time.monotonic() < deadline:
            time.sleep(0.005)
        data = rt.resp.read_bytes()
        rt.resp.unlink()
        n = struct.unpack("!I", data[:4])[0]
        assert json.loads(data[4:4 + n]) == {"rc": -1, "err": "req_oversize"}
        assert not rt.req.exists()          # the server claimed (removed) the request
        assert rt.ping()["pong"] == 1       # and keeps serving
        with pytest.raises(ValueError):
            rt.run(b"short")                # client-side size check
    finally:
        rc = rt.stop_server()
    assert rc == 0 and not rt.server_running()
    assert "[stop] served" in rt.server_log()


def test_server_rejects_bad_job(tmp_path):
    rt = PersistentRuntime(tmp_path / "persist", timeout=5.0)
    with pytest.raises(PersistentRuntimeError, match="exited during startup"):
        rt.start_server(tmp_path / "missing.wtop", out_temp=0, in_bytes=4)
    assert "read blob" in rt.server_log()
