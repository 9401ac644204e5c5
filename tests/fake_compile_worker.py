"""A stand-in compile worker for the CPU tests of grammar.compile_pool: it
speaks the worker protocol of grammar/compile_worker.py but compiles nothing.
A source containing HANG makes it sleep far past any test's limit, FAIL makes
it report a compile error, CRASH makes it exit without answering; any other
source comes back as b"CODE:" + source."""
import json
import os
import sys
import time

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "cs348k-fast-attention-grammar_amd"))
from grammar.compile_worker import read_frame, write_frame  # noqa: E402


def main() -> int:
    fin, fout = sys.stdin.fileno(), sys.stdout.fileno()
    while True:
        meta = read_frame(fin)
        if meta is None:
            return 0
        src = read_frame(fin)
        if b"HANG" in src:
            time.sleep(600)
        if b"CRASH" in src:
            os._exit(3)
        if b"FAIL" in src:
            write_frame(fout, json.dumps({"ok": False, "error": "error: fake compile failure"}).encode())
            write_frame(fout, b"")
            continue
        write_frame(fout, json.dumps({"ok": True, "error": ""}).encode())
        write_frame(fout, b"CODE:" + src)


if __name__ == "__main__":
    sys.exit(main())
