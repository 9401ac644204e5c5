// gr_attn_bwd.hip -- the attention backward (gr_flash_bwd.h) behind
// gr_attn_bwd(), and its d = 64 instances. The d = 128 instances live in
// gr_attn_bwd128.hip, which build_native.py compiles with MFMAs in VGPR form.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gr_flash_bwd.h"
#include "gr_host.h"
#include "grammar_rt.h"

#include "gr_attn_bwd_launch.h"

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" size_t gr_attn_bwd_workspace(int B, int H, int N, int D) {
  if (B <= 0 || H <= 0 || N <= 0 || D <= 0) return 0;
  return (size_t)B * H * N * sizeof(float);
}

extern "C" int gr_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                           const float* lse, void* dq, void* dk, void* dv, int dtype, int B, int H, int N, int D,
                           const long long* strides, int causal, float scale, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv || !strides)
    return gr::fail(GR_E_ARG, "gr_attn_bwd: null argument");
  if (B <= 0 || H <= 0 || N <= 0) return gr::fail(GR_E_ARG, "gr_attn_bwd: B, H, N must be positive");
  const void* ptrs[10] = {q, k, v, o, dout, dq, dk, dv, workspace, lse};
  for (int i = 0; i < 9; ++i)
    if (!aligned16(ptrs[i])) return gr::fail(GR_E_ARG, "gr_attn_bwd: tensors and workspace must be 16-byte aligned");
  if ((uintptr_t)lse & 3) return gr::fail(GR_E_ARG, "gr_attn_bwd: lse must be 4-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (strides[i] < 0 || strides[i] % 8 != 0)
      return gr::fail(GR_E_ARG, "gr_attn_bwd: strides must be non-negative multiples of 8 elements");
  if (!(scale > 0.f)) return gr::fail(GR_E_ARG, "gr_attn_bwd: scale must be positive");
  const size_t need = gr_attn_bwd_workspace(B, H, N, D);
  if (!workspace || workspace_bytes < need)
    return gr::fail(GR_E_ARG, "gr_attn_bwd: workspace of %zu bytes needed", need);
  gr_attn_bwd_args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dout = dout;
  a.lse = lse;
  a.delta = static_cast<float*>(workspace);
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.sb = strides[0];
  a.sh = strides[1];
  a.sn = strides[2];
  a.B = B;
  a.H = H;
  a.N = N;
  a.scale = scale;
  hipStream_t st = (hipStream_t)stream;
  const bool c = causal != 0;
  if (dtype != GR_F16 && dtype != GR_BF16)
    return gr::fail(GR_E_ARG, "gr_attn_bwd: dtype %d unsupported (GR_F16 or GR_BF16)", dtype);
  if (D == 128) return gr_attn_bwd_launch_d128(a, dtype == GR_BF16, c, st);
  if (D != 64) return gr::fail(GR_E_ARG, "gr_attn_bwd: head dim D=%d unsupported (64 or 128)", D);
  return dtype == GR_BF16 ? launch_bwd<__bf16, 64, 128, 128>(a, c, st) : launch_bwd<_Float16, 64, 128, 128>(a, c, st);
}

