// gr_err.h -- the per-thread error slot behind gr_last_error(), shared by the
// host-only compile unit and the HIP translation units of libgrammar_rt.so.
#pragma once

namespace gr {

// Record a failure message for gr_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace gr
