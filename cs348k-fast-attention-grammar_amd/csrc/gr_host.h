// gr_host.h -- host-side helpers shared by the translation units of
// libgrammar_rt.so: the per-thread error slot behind gr_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <cstdarg>
#include <cstdio>

namespace gr {

// Record a failure message for gr_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Map a HIP status to GR_OK / `code` with a message naming `what`.
int hip_check(hipError_t e, int code, const char* what);

}  // namespace gr
