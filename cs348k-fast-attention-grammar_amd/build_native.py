"""Build libgrammar_rt.so (the C-ABI runtime + hand-written gfx950 kernels)
and libgrammar_rtc.so (the hiprtc compile entry points alone).

Every .hip / .cpp source under csrc/ is compiled with hipcc for gfx950 only,
with packed FP32 instructions disabled, and linked into lib/libgrammar_rt.so
next to this file. gr_rtc.cpp (hiprtc compilation and the error slot, no HIP
runtime call) is host C++ built with g++; it is linked into libgrammar_rt.so
and, on its own, into lib/libgrammar_rtc.so, the library the compile worker
processes load (they never open the GPU). The objects are compiled in
parallel.

    python build_native.py            # build (always recompiles)
"""
from __future__ import annotations

import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "lib", "obj")
LIB = os.path.join(LIBDIR, "libgrammar_rt.so")
RTC_LIB = os.path.join(LIBDIR, "libgrammar_rtc.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ROCM = "/opt/rocm"
HOST_ONLY = ("gr_rtc.cpp",)   # host C++ (hiprtc only), built with CXX

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", os.path.join(REPO, "include"),
    "-Wno-unused-result",
]


# Per-source extra flags. The backward's d = 128 dK/dV kernel runs one wave
# per SIMD; left to its heuristics the backend then puts every MFMA
# accumulator in AGPRs and copies the score accumulators to VGPRs (and back)
# for the softmax arithmetic on every tile. With VGPR-form MFMAs the score
# accumulators stay in VGPRs, and the dK/dV accumulators, pinned to AGPRs by
# inline assembly, need no copies either (the d = 64 kernels are faster with
# the heuristics).
EXTRA = {"gr_attn_bwd128.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    if os.path.basename(src) in HOST_ONLY:
        cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
               "-I", CSRC, "-I", os.path.join(REPO, "include"), "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    t0 = time.time()
    srcs = _sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    rtc_objs = [o for o in objs if os.path.basename(o)[:-2] in HOST_ONLY]
    links = ((LIB, [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs]),
             (RTC_LIB, [CXX, "-shared", "-fPIC", *rtc_objs]))
    for out, cmd in links:
        tmp = out + ".tmp"
        r = subprocess.run(cmd + ["-o", tmp, f"-L{ROCM}/lib", "-lhiprtc", f"-Wl,-rpath,{ROCM}/lib"],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link of {out} failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, out)
    if verbose:
        print(f"[build_native] {LIB}, {RTC_LIB} ({len(srcs)} sources, {time.time() - t0:.1f}s)", flush=True)
    return LIB


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
