// gr_host.h -- host-side helpers shared by the HIP translation units of
// libgrammar_rt.so: the error slot and HIP status mapping.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdarg>
#include <cstdio>

#include "gr_err.h"

namespace gr {

// Map a HIP status to GR_OK / `code` with a message naming `what`.
int hip_check(hipError_t e, int code, const char* what);

}  // namespace gr
