// gr_rtc.cpp -- the host-only part of the C ABI: hiprtc compilation of
// rendered modules, toolchain identification and the per-thread error slot.
//
// It stands in for the cuTile JIT of a generated module (reference
// grammar/optimization.py:262-283, grammar/kernel_ast.py:1228-1229). The file
// uses no HIP runtime call, so it is linked twice: into libgrammar_rt.so (the
// full ABI) and on its own into libgrammar_rtc.so, which the compile worker
// processes load. A worker therefore never opens the GPU, and a hung compile
// can be ended by killing its process.
#include <hip/hiprtc.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gr_err.h"
#include "grammar_rt.h"

namespace gr {

static thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace gr

extern "C" {

const char* gr_last_error(void) { return gr::g_err.c_str(); }

const char* gr_version(void) {
  static std::string v;
  if (v.empty()) {
    int maj = 0, min = 0;
    hiprtcVersion(&maj, &min);
    v = "gfx950 hiprtc " + std::to_string(maj) + "." + std::to_string(min);
  }
  return v.c_str();
}

int gr_compile(const char* src, const char* name, const char* const* opts, int nopts, void** code,
               size_t* code_size, char* log, size_t loglen) {
  if (!src || !code || !code_size) return gr::fail(GR_E_ARG, "gr_compile: null argument");
  if (nopts < 0 || (nopts && !opts)) return gr::fail(GR_E_ARG, "gr_compile: bad option list");
  if (log && loglen) log[0] = 0;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, src, name ? name : "gr_module.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return gr::fail(GR_E_COMPILE, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  // Packed FP32 instructions stay disabled in every kernel this library builds.
  std::vector<const char*> o = {"--offload-arch=gfx950", "-O3", "-std=c++17",
                                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  for (int i = 0; i < nopts; ++i) o.push_back(opts[i]);
  r = hiprtcCompileProgram(prog, (int)o.size(), o.data());
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(prog, &ls);
    std::string lg(ls + 1, '\0');
    if (ls) hiprtcGetProgramLog(prog, &lg[0]);
    if (log && loglen) {
      strncpy(log, lg.c_str(), loglen - 1);
      log[loglen - 1] = 0;
    }
    hiprtcDestroyProgram(&prog);
    return gr::fail(GR_E_COMPILE, "hiprtc compile failed: %.1500s", lg.c_str());
  }
  size_t cs = 0;
  hiprtcGetCodeSize(prog, &cs);
  void* buf = malloc(cs);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return gr::fail(GR_E_RUNTIME, "gr_compile: out of host memory");
  }
  hiprtcGetCode(prog, (char*)buf);
  hiprtcDestroyProgram(&prog);
  *code = buf;
  *code_size = cs;
  return GR_OK;
}

void gr_free_code(void* code) { free(code); }

}  // extern "C"
