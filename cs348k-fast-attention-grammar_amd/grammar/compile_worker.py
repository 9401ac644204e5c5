"""A hiprtc compile worker process (run as a script by grammar.compile_pool).

It loads lib/libgrammar_rtc.so -- gr_compile and nothing of the HIP runtime --
so the process never opens the GPU and may be killed at any moment, which is
how a compile that runs past its wall-clock limit is ended (the reference
scores such a compile as a penalty after SIGALRM,
grammar/optimization.py:262-283; a hiprtc call cannot be interrupted inside
the process that made it).

Protocol on stdin/stdout, every frame a little-endian u32 length and that
many bytes:
  request:  frame(JSON {"name": str, "opts": [str]}), frame(source text)
  reply:    frame(JSON {"ok": bool, "error": str}), frame(code object bytes)
The worker serves requests until stdin closes.

    python compile_worker.py <path of libgrammar_rtc.so> <include dir>
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
import sys


def read_frame(fd: int) -> bytes | None:
    head = _read_exact(fd, 4)
    if head is None:
        return None
    (n,) = struct.unpack("<I", head)
    body = _read_exact(fd, n)
    if body is None:
        raise EOFError("truncated frame")
    return body


def _read_exact(fd: int, n: int) -> bytes | None:
    parts, got = [], 0
    while got < n:
        b = os.read(fd, n - got)
        if not b:
            if got == 0:
                return None
            raise EOFError("truncated frame")
        parts.append(b)
        got += len(b)
    return b"".join(parts)


def write_frame(fd: int, data: bytes) -> None:
    buf = struct.pack("<I", len(data)) + data
    view = memoryview(buf)
    while view:
        n = os.write(fd, view)
        view = view[n:]


def _compiler(lib_path: str):
    L = ctypes.CDLL(lib_path)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    L.gr_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                             ctypes.POINTER(vp), ctypes.POINTER(sz), ctypes.c_char_p, sz]
    L.gr_free_code.argtypes = [vp]
    L.gr_free_code.restype = None
    L.gr_last_error.restype = ctypes.c_char_p

    def compile_one(src: bytes, name: str, opts: list) -> tuple:
        arr = (ctypes.c_char_p * max(1, len(opts)))(*[o.encode() for o in opts])
        code, size = vp(), sz()
        log = ctypes.create_string_buffer(16384)
        rc = L.gr_compile(src, name.encode(), arr, len(opts), ctypes.byref(code), ctypes.byref(size), log, len(log))
        if rc != 0:
            msg = log.value.decode(errors="replace") or L.gr_last_error().decode(errors="replace")
            return False, f"[gr {rc}] {msg}", b""
        try:
            return True, "", ctypes.string_at(code, size.value)
        finally:
            L.gr_free_code(code)
    return compile_one


def main(argv: list) -> int:
    lib_path, include_dir = argv[1], argv[2]
    compile_one = _compiler(lib_path)
    fin, fout = sys.stdin.fileno(), sys.stdout.fileno()
    while True:
        meta = read_frame(fin)
        if meta is None:
            return 0
        src = read_frame(fin)
        req = json.loads(meta)
        ok, err, code = compile_one(src, req.get("name", "gr_module.hip"), ["-I" + include_dir] + req.get("opts", []))
        write_frame(fout, json.dumps({"ok": ok, "error": err}).encode())
        write_frame(fout, code)


if __name__ == "__main__":
    sys.exit(main(sys.argv))
