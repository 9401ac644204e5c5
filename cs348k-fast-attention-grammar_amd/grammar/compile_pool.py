"""hiprtc compiles in worker processes, each with a wall-clock limit.

The descent compiles the candidates of a coordinate concurrently (the
reference compiles one at a time inside its SIGALRM-guarded import,
grammar/optimization.py:262-283). A hiprtc call that hangs cannot be
interrupted in the process that made it, so every compile runs in a worker
process (grammar/compile_worker.py, which loads only libgrammar_rtc.so and
never opens the GPU). One dispatcher thread per worker sends it a job and
waits for the reply up to the limit; past it the worker is killed (its exact
PID), the job fails with CompileTimeout, and the next job starts a fresh
worker. So a hung compile costs one limit of wall time and never a worker.

    pool = CompilePool(workers=4, timeout=60)
    fut = pool.submit(src)          # concurrent.futures.Future -> code bytes
    code = fut.result()             # or raises CompileTimeout / CompileError
"""
from __future__ import annotations

import atexit
import json
import os
import queue
import select
import subprocess
import sys
import threading
import time
import weakref
from concurrent.futures import Future

from . import runtime as rt
from .compile_worker import write_frame

WORKER_SCRIPT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "compile_worker.py")
RTC_LIB_PATH = os.path.join(os.path.dirname(rt.LIB_PATH), "libgrammar_rtc.so")


class CompileTimeout(Exception):
    """A compile that ran past the pool's wall-clock limit (its worker was killed)."""


class WorkerDied(rt.CompileError):
    """The worker process ended without answering (crash of the compiler)."""


def default_worker_cmd() -> list:
    if not os.path.exists(RTC_LIB_PATH):
        raise RuntimeError(f"{RTC_LIB_PATH} is missing: build it with `python __graft_entry__.py` "
                           "or build_native.py before compiling")
    return [sys.executable, "-u", WORKER_SCRIPT, RTC_LIB_PATH, rt.CSRC_DIR]


class _Deadline(Exception):
    pass


class _Worker:
    """One worker process and the reads of its replies against a deadline."""

    def __init__(self, cmd: list):
        self.proc = subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, bufsize=0,
                                     close_fds=True)
        self.fin = self.proc.stdin.fileno()
        self.fout = self.proc.stdout.fileno()

    def _read_exact(self, n: int, deadline: float | None) -> bytes:
        parts, got = [], 0
        while got < n:
            wait = None if deadline is None else deadline - time.monotonic()
            if wait is not None and wait <= 0:
                raise _Deadline()
            ready, _, _ = select.select([self.fout], [], [], wait)
            if not ready:
                raise _Deadline()
            b = os.read(self.fout, n - got)
            if not b:
                raise EOFError("compile worker closed its output")
            parts.append(b)
            got += len(b)
        return b"".join(parts)

    def _frame(self, deadline) -> bytes:
        n = int.from_bytes(self._read_exact(4, deadline), "little")
        return self._read_exact(n, deadline)

    def request(self, meta: dict, src: bytes, timeout: float) -> tuple:
        deadline = time.monotonic() + timeout if timeout and timeout > 0 else None
        write_frame(self.fin, json.dumps(meta).encode())
        write_frame(self.fin, src)
        status = json.loads(self._frame(deadline))
        code = self._frame(deadline)
        return status, code

    def kill(self) -> None:
        try:
            self.proc.kill()
        except OSError:
            pass
        try:
            self.proc.wait(timeout=10)
        except subprocess.TimeoutExpired:
            pass
        for f in (self.proc.stdin, self.proc.stdout):
            try:
                f.close()
            except OSError:
                pass


_pools = weakref.WeakSet()


class CompilePool:
    def __init__(self, workers: int = 4, timeout: float = 60.0, worker_cmd: list | None = None):
        self.timeout = float(timeout or 0.0)
        self._cmd = list(worker_cmd) if worker_cmd is not None else None
        self._jobs: queue.Queue = queue.Queue()
        self._workers: list = [None] * max(1, int(workers))
        self._closed = False
        self.timeouts = 0          # compiles killed at the limit
        self.spawned = 0           # worker processes started
        self._lock = threading.Lock()
        self._threads = [threading.Thread(target=self._serve, args=(i,), daemon=True, name=f"gr-compile-{i}")
                         for i in range(len(self._workers))]
        for t in self._threads:
            t.start()
        _pools.add(self)

    def submit(self, src: str, name: str = "gr_module.hip", opts: list | None = None) -> Future:
        if self._closed:
            raise RuntimeError("CompilePool is closed")
        fut: Future = Future()
        self._jobs.put((fut, {"name": name, "opts": list(opts or [])}, src.encode()))
        return fut

    def compile(self, src: str, **kw) -> bytes:
        return self.submit(src, **kw).result()

    def _worker(self, i: int) -> _Worker:
        w = self._workers[i]
        if w is None or w.proc.poll() is not None:
            if w is not None:
                w.kill()
            w = _Worker(self._cmd or default_worker_cmd())
            self._workers[i] = w
            with self._lock:
                self.spawned += 1
        return w

    def _serve(self, i: int) -> None:
        while True:
            job = self._jobs.get()
            if job is None:
                return
            fut, meta, src = job
            if not fut.set_running_or_notify_cancel():
                continue
            w = None
            try:
                w = self._worker(i)
                status, code = w.request(meta, src, self.timeout)
            except _Deadline:
                w.kill()
                self._workers[i] = None
                with self._lock:
                    self.timeouts += 1
                fut.set_exception(CompileTimeout(f"hiprtc compile exceeded {self.timeout:.0f}s (worker killed)"))
                continue
            except (EOFError, OSError, ValueError) as e:
                if w is not None:
                    w.kill()
                    self._workers[i] = None
                fut.set_exception(WorkerDied(rt.GR_E_COMPILE, f"compile worker failed: {e}"))
                continue
            except BaseException as e:     # never leave a future unresolved
                fut.set_exception(e)
                continue
            if status.get("ok"):
                fut.set_result(code)
            else:
                fut.set_exception(rt.CompileError(rt.GR_E_COMPILE, status.get("error", "compile failed")))

    def close(self) -> None:
        if self._closed:
            return
        self._closed = True
        for _ in self._threads:
            self._jobs.put(None)
        for i, w in enumerate(self._workers):
            if w is not None:
                w.kill()
                self._workers[i] = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@atexit.register
def _close_all() -> None:
    for p in list(_pools):
        p.close()
