"""Client of the resident decode server (gehtp_amd/gehtp_persistent).

The reference drives its device-resident runner through files pushed over adb
(scripts/persistent_runtime.py: PersistentDeviceRuntime, start_server / _rpc /
stop_server, protocol kernels/examples/42_gehtp_persistent/main.c:14-31). The server
here runs on the GPU host itself, so the same protocol goes through local files:

  job file   "key value" lines: blob, out_temp, in_bytes, req, resp, out, idle_exit_s,
             optional weights_size (<blob stem>.weights.bin) and trace
  request    4-byte big-endian header length + JSON header (+ in_bytes of input for
             "run"), written to a temporary name and renamed into place
  response   4-byte big-endian length + JSON; rc != 0 raises PersistentRuntimeError
"""
from __future__ import annotations

import json
import os
import struct
import subprocess
import time
from pathlib import Path
from typing import Any, Optional

SERVER = Path(__file__).resolve().parent / "gehtp_persistent"


class PersistentRuntimeError(RuntimeError):
    """A failed request or a server that did not start or answer."""


class PersistentRuntime:
    POLL_INTERVAL = 0.002
    STARTUP_TIMEOUT = 120.0

    def __init__(self, persist_dir: str | Path, timeout: float = 60.0):
        self.dir = Path(persist_dir)
        self.timeout = timeout
        self.proc: Optional[subprocess.Popen] = None
        self.in_bytes = 0

    @property
    def req(self) -> Path:
        return self.dir / "req.bin"

    @property
    def resp(self) -> Path:
        return self.dir / "resp.bin"

    @property
    def out(self) -> Path:
        return self.dir / "out.f16.raw"

    # ---- server lifecycle ----
    def start_server(self, blob: str | Path, out_temp: int, in_bytes: int, *,
                     weights_size: Optional[int] = None, idle_exit_s: int = 600,
                     trace: bool = False) -> dict[str, Any]:
        """Write the job file, start the server and wait until it answers a ping.
        With weights_size, the external weight image is <blob stem>.weights.bin."""
        if not SERVER.exists():
            raise PersistentRuntimeError(f"{SERVER} not built (python -m gehtp_amd.build)")
        self.dir.mkdir(parents=True, exist_ok=True)
        lines = [f"blob {Path(blob).resolve()}", f"out_temp {out_temp}", f"in_bytes {in_bytes}",
                 f"req {self.req}", f"resp {self.resp}", f"out {self.out}", f"idle_exit_s {idle_exit_s}",
                 f"trace {1 if trace else 0}"]
        if weights_size:
            lines.append(f"weights_size {weights_size}")
        job = self.dir / "job.txt"
        job.write_text("\n".join(lines) + "\n")
        self.in_bytes = in_bytes
        log = open(self.dir / "server.log", "wb")
        self.proc = subprocess.Popen([str(SERVER), str(job)], stdout=log, stderr=subprocess.STDOUT,
                                     stdin=subprocess.DEVNULL)
        log.close()
        t0 = time.monotonic()
        last: Optional[Exception] = None
        while time.monotonic() - t0 < self.STARTUP_TIMEOUT:
            if self.proc.poll() is not None:
                raise PersistentRuntimeError(
                    f"server exited during startup (rc {self.proc.returncode}):\n{self.server_log()}")
            try:
                self._rpc({"op": "ping"}, timeout=5.0)
                return {"pid": self.proc.pid, "blob": str(blob), "out_temp": out_temp, "in_bytes": in_bytes}
            except PersistentRuntimeError as e:
                last = e
        self.kill()
        raise PersistentRuntimeError(f"server not ready in {self.STARTUP_TIMEOUT}s: {last}")

    def server_log(self) -> str:
        p = self.dir / "server.log"
        return p.read_text(errors="replace")[-4000:] if p.exists() else ""

    def server_running(self) -> bool:
        return self.proc is not None and self.proc.poll() is None

    def stop_server(self, timeout: float = 30.0) -> int:
        """Ask the server to shut down (it releases the engine itself) and wait."""
        if not self.server_running():
            return self.proc.returncode if self.proc else 0
        try:
            self._rpc({"op": "shutdown"}, timeout=timeout)
        except PersistentRuntimeError:
            pass
        try:
            return self.proc.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            self.kill()
            return -9

    def kill(self) -> None:
        if self.proc is not None and self.proc.poll() is None:
            self.proc.kill()
            self.proc.wait()

    # ---- file-queue RPC ----
    def _rpc(self, hdr: dict[str, Any], body: bytes = b"", timeout: Optional[float] = None) -> dict[str, Any]:
        timeout = timeout or self.timeout
        if self.resp.exists():
            self.resp.unlink()
        j = json.dumps(hdr, separators=(",", ":")).encode("utf-8")
        tmp = self.req.with_name(self.req.name + ".tmp")
        tmp.write_bytes(struct.pack("!I", len(j)) + j + body)
        os.replace(tmp, self.req)
        deadline = time.monotonic() + timeout
        while time.monotonic() < deadline:
            if self.resp.exists():
                data = self.resp.read_bytes()
                self.resp.unlink()
                if len(data) < 4:
                    raise PersistentRuntimeError(f"short resp ({len(data)}B)")
                n = struct.unpack("!I", data[:4])[0]
                if len(data) < 4 + n:
                    raise PersistentRuntimeError(f"truncated resp ({len(data)}B < {4 + n})")
                out = json.loads(data[4:4 + n].decode("utf-8"))
                if out.get("rc", 0) != 0:
                    raise PersistentRuntimeError(f"server rc={out.get('rc')}: {out.get('err', 'unknown')}")
                return out
            if self.proc is not None and self.proc.poll() is not None:
                raise PersistentRuntimeError(f"server exited (rc {self.proc.returncode}):\n{self.server_log()}")
            time.sleep(self.POLL_INTERVAL)
        raise PersistentRuntimeError(f"rpc timeout after {timeout}s (op={hdr.get('op')})")

    # ---- requests ----
    def ping(self) -> dict[str, Any]:
        return self._rpc({"op": "ping"})

    def reset(self) -> dict[str, Any]:
        """Zero every persistent state (KV rings and position counters)."""
        return self._rpc({"op": "reset"})

    def run(self, body: bytes, *, want_out: bool = False) -> tuple[int, dict[str, Any], Optional[bytes]]:
        """One run of the blob on `body` (in_bytes of input). Returns (token, response,
        the out temp's bytes when want_out). The token is the first maximum of the out
        temp read as f16."""
        if len(body) != self.in_bytes:
            raise ValueError(f"body is {len(body)} bytes, the server expects {self.in_bytes}")
        r = self._rpc({"op": "run", "want_out": 1 if want_out else 0}, body)
        out = self.out.read_bytes() if want_out else None
        return int(r["token"]), r, out
