// gr_runtime.cpp -- code-object loading, launch plans and hipEvent timing
// behind the C ABI in include/grammar_rt.h (hiprtc compilation and the error
// slot live in gr_rtc.cpp).
//
// This is the MI355X replacement for the part of the reference that cupy
// provides: loading the JIT-compiled module, ct.launch of each stage
// (grammar/kernel_ast.py:1268-1276) and the cp.cuda.Event timing loops
// (grammar/optimization.py:284-300, bench.py:49-74).
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gr_host.h"
#include "grammar_rt.h"

namespace gr {

int hip_check(hipError_t e, int code, const char* what) {
  if (e == hipSuccess) return GR_OK;
  return fail(code, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

}  // namespace gr

struct gr_module {
  hipModule_t mod;
  std::vector<gr_kernel*> kernels;
};

struct gr_kernel {
  hipFunction_t fn;
};

struct gr_plan_step {
  gr_kernel* k = nullptr;
  uint32_t grid[3] = {1, 1, 1};
  uint32_t block[3] = {1, 1, 1};
  uint32_t lds = 0;
  std::vector<uint64_t> args;
  std::vector<void*> argp;
};

struct gr_plan {
  std::vector<gr_plan_step> steps;
};

namespace {

// A bounded device spin launched ahead of a timed region: it holds the stream
// (about 28 us: 8 sleeps of 127 x 64 clocks) while the host enqueues the
// first event and the launches behind it, so the event pair brackets GPU
// time only, not the host's launch latency of the first launch.
__global__ void gr_hold_kernel(int rounds) {
  for (int i = 0; i < rounds; ++i) __builtin_amdgcn_s_sleep(127);
}

int hold_stream(hipStream_t st) {
  hipLaunchKernelGGL(gr_hold_kernel, dim3(1), dim3(64), 0, st, 8);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_plan_time hold launch");
}

}  // namespace

extern "C" {

int gr_device_info(int device, long long* out5) {
  if (!out5) return gr::fail(GR_E_ARG, "gr_device_info: null output");
  hipDeviceProp_t p;
  int rc = gr::hip_check(hipGetDeviceProperties(&p, device), GR_E_RUNTIME, "hipGetDeviceProperties");
  if (rc) return rc;
  out5[0] = p.multiProcessorCount;
  out5[1] = (long long)p.sharedMemPerBlock;
  out5[2] = p.warpSize;
  out5[3] = p.clockRate;
  out5[4] = p.l2CacheSize;
  return GR_OK;
}

int gr_module_load(const void* code, size_t code_size, gr_module** out) {
  if (!code || !code_size || !out) return gr::fail(GR_E_ARG, "gr_module_load: null argument");
  hipModule_t m;
  int rc = gr::hip_check(hipModuleLoadData(&m, code), GR_E_LOAD, "hipModuleLoadData");
  if (rc) return rc;
  *out = new gr_module{m, {}};
  return GR_OK;
}

void gr_module_free(gr_module* mod) {
  if (!mod) return;
  for (gr_kernel* k : mod->kernels) delete k;
  hipModuleUnload(mod->mod);
  delete mod;
}

int gr_get_kernel(gr_module* mod, const char* name, gr_kernel** out) {
  if (!mod || !name || !out) return gr::fail(GR_E_ARG, "gr_get_kernel: null argument");
  hipFunction_t f;
  hipError_t e = hipModuleGetFunction(&f, mod->mod, name);
  if (e != hipSuccess) return gr::fail(GR_E_LOAD, "hipModuleGetFunction(%s): %s", name, hipGetErrorString(e));
  gr_kernel* k = new gr_kernel{f};
  mod->kernels.push_back(k);
  *out = k;
  return GR_OK;
}

static int launch_raw(gr_kernel* k, const uint32_t grid[3], const uint32_t block[3], uint32_t lds,
                      hipStream_t st, void** argp) {
  // gfx950 accepts up to 160 KiB of dynamic LDS per workgroup without an opt-in;
  // a request beyond the device limit fails the launch and is reported below.
  hipError_t e = hipModuleLaunchKernel(k->fn, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                       lds, st, argp, nullptr);
  if (e != hipSuccess) return gr::fail(GR_E_LAUNCH, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
  return GR_OK;
}

int gr_launch(gr_kernel* k, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes, void* stream,
              const uint64_t* args, int nargs) {
  if (!k || !grid || !block || (nargs && !args) || nargs < 0)
    return gr::fail(GR_E_ARG, "gr_launch: bad argument");
  std::vector<uint64_t> vals(args, args + nargs);
  std::vector<void*> ptrs(nargs);
  for (int i = 0; i < nargs; ++i) ptrs[i] = &vals[i];
  return launch_raw(k, grid, block, lds_bytes, (hipStream_t)stream, nargs ? ptrs.data() : nullptr);
}

int gr_plan_create(int nsteps, gr_plan** out) {
  if (nsteps < 0 || !out) return gr::fail(GR_E_ARG, "gr_plan_create: bad argument");
  gr_plan* p = new gr_plan;
  p->steps.resize(nsteps);
  *out = p;
  return GR_OK;
}

int gr_plan_set_step(gr_plan* p, int i, gr_kernel* k, const uint32_t grid[3], const uint32_t block[3],
                     uint32_t lds_bytes, const uint64_t* args, int nargs) {
  if (!p || i < 0 || i >= (int)p->steps.size() || !k || !grid || !block || nargs < 0 || (nargs && !args))
    return gr::fail(GR_E_ARG, "gr_plan_set_step: bad argument");
  for (int d = 0; d < 3; ++d)
    if (grid[d] == 0 || block[d] == 0) return gr::fail(GR_E_ARG, "gr_plan_set_step: zero grid/block dim");
  if ((uint64_t)block[0] * block[1] * block[2] > 1024) return gr::fail(GR_E_ARG, "gr_plan_set_step: block > 1024");
  gr_plan_step& s = p->steps[i];
  s.k = k;
  for (int d = 0; d < 3; ++d) {
    s.grid[d] = grid[d];
    s.block[d] = block[d];
  }
  s.lds = lds_bytes;
  s.args.assign(args, args + nargs);
  s.argp.resize(nargs);
  for (int a = 0; a < nargs; ++a) s.argp[a] = &s.args[a];
  return GR_OK;
}

int gr_plan_run(gr_plan* p, void* stream) {
  if (!p) return gr::fail(GR_E_ARG, "gr_plan_run: null plan");
  for (size_t i = 0; i < p->steps.size(); ++i) {
    gr_plan_step& s = p->steps[i];
    if (!s.k) return gr::fail(GR_E_ARG, "gr_plan_run: step %zu not set", i);
    int rc = launch_raw(s.k, s.grid, s.block, s.lds, (hipStream_t)stream, s.argp.empty() ? nullptr : s.argp.data());
    if (rc) return rc;
  }
  return GR_OK;
}

void gr_plan_free(gr_plan* p) { delete p; }

int gr_plan_time(gr_plan* p, void* stream, int warmup, int iters, int mode, float* ms_out) {
  if (!p || iters <= 0 || warmup < 0 || !ms_out || (mode != GR_TIME_BATCH && mode != GR_TIME_MIN))
    return gr::fail(GR_E_ARG, "gr_plan_time: bad argument");
  hipStream_t st = (hipStream_t)stream;
  int rc;
  for (int i = 0; i < warmup; ++i)
    if ((rc = gr_plan_run(p, stream))) return rc;
  hipEvent_t e0, e1;
  if ((rc = gr::hip_check(hipEventCreate(&e0), GR_E_RUNTIME, "hipEventCreate"))) return rc;
  if ((rc = gr::hip_check(hipEventCreate(&e1), GR_E_RUNTIME, "hipEventCreate"))) {
    hipEventDestroy(e0);
    return rc;
  }
  float result = 0.f;
  if (mode == GR_TIME_BATCH) {
    rc = hold_stream(st);
    if (!rc) rc = gr::hip_check(hipEventRecord(e0, st), GR_E_RUNTIME, "hipEventRecord");
    for (int i = 0; !rc && i < iters; ++i) rc = gr_plan_run(p, stream);
    if (!rc) rc = gr::hip_check(hipEventRecord(e1, st), GR_E_RUNTIME, "hipEventRecord");
    if (!rc) rc = gr::hip_check(hipEventSynchronize(e1), GR_E_RUNTIME, "hipEventSynchronize");
    float ms = 0.f;
    if (!rc) rc = gr::hip_check(hipEventElapsedTime(&ms, e0, e1), GR_E_RUNTIME, "hipEventElapsedTime");
    result = ms / (float)iters;
  } else {
    float best = 3.0e38f;
    for (int i = 0; !rc && i < iters; ++i) {
      rc = hold_stream(st);
      if (!rc) rc = gr::hip_check(hipEventRecord(e0, st), GR_E_RUNTIME, "hipEventRecord");
      if (!rc) rc = gr_plan_run(p, stream);
      if (!rc) rc = gr::hip_check(hipEventRecord(e1, st), GR_E_RUNTIME, "hipEventRecord");
      if (!rc) rc = gr::hip_check(hipEventSynchronize(e1), GR_E_RUNTIME, "hipEventSynchronize");
      float ms = 0.f;
      if (!rc) rc = gr::hip_check(hipEventElapsedTime(&ms, e0, e1), GR_E_RUNTIME, "hipEventElapsedTime");
      if (!rc && ms < best) best = ms;
    }
    result = best;
  }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (rc) return rc;
  *ms_out = result;
  return GR_OK;
}

}  // extern "C"
