// gr_attn_bwd_launch.h -- launchers of the attention backward kernels
// (host side, included by the translation units that instantiate them).
#pragma once
#include <hip/hip_runtime.h>

#include "gr_flash_bwd.h"
#include "gr_host.h"
#include "grammar_rt.h"

namespace {

// fp16 with scale log2(e) <= 1: the kernels' pre-scaled forms (PRE), whose
// scores come out of the MFMAs in log2 units relative to the row's L.
template <class T>
bool bwd_prescale(const gr_attn_bwd_args& a) {
  return gr_is_same<T, _Float16>::value && a.scale * 1.4426950408889634f <= 1.0f;
}

// Backward tiles. dK/dV: (queries per tile, keys per workgroup) = (128, 128),
// one wave per 32 keys. dQ: key tiles of 128 at d = 64, 64 at d = 128, 8 waves
// (256 queries) per workgroup when N allows it, else 4. (At C2 the 128-deep
// tiles took dQ from 28.7 to 28.0 us and dK/dV from 35.5 to 34.8 us: half the
// tile barriers and loads per MFMA; at C3 the dK/dV kernel's 128-query tiles
// ran 661 against 682 us for 64.)
template <class T, int D, int NW>
void launch_bwd_dq(const gr_attn_bwd_args& a, bool causal, hipStream_t st) {
  constexpr int DQ_BN = D <= 64 ? 128 : 64;
  const dim3 grid((unsigned)((long long)a.B * a.H * (a.N / (NW * 32))));
  constexpr int LDS = gr_attn_bwd_dq_lds<D, DQ_BN>::BYTES;
  const bool pre = bwd_prescale<T>(a);
  if (causal && pre)
    hipLaunchKernelGGL((gr_attn_bwd_dq_kernel<T, D, NW, DQ_BN, true, true>), grid, dim3(NW * 64), LDS, st, a);
  else if (causal)
    hipLaunchKernelGGL((gr_attn_bwd_dq_kernel<T, D, NW, DQ_BN, true, false>), grid, dim3(NW * 64), LDS, st, a);
  else if (pre)
    hipLaunchKernelGGL((gr_attn_bwd_dq_kernel<T, D, NW, DQ_BN, false, true>), grid, dim3(NW * 64), LDS, st, a);
  else
    hipLaunchKernelGGL((gr_attn_bwd_dq_kernel<T, D, NW, DQ_BN, false, false>), grid, dim3(NW * 64), LDS, st, a);
}

template <class T, int D, int BM, int BN>
int launch_bwd(const gr_attn_bwd_args& a, bool causal, hipStream_t st) {
  if (a.N % BN != 0 || a.N % BM != 0 || a.N % 128 != 0)
    return gr::fail(GR_E_ARG, "gr_attn_bwd: N=%d must be a multiple of %d at D=%d", a.N, BN > 128 ? BN : 128, D);
  // dQ first: it also writes delta, which the dK/dV kernel reads
  if (a.N % 256 == 0) launch_bwd_dq<T, D, 8>(a, causal, st);
  else launch_bwd_dq<T, D, 4>(a, causal, st);
  int rc = gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_bwd dQ launch");
  if (rc) return rc;
  const dim3 grid((unsigned)((long long)a.B * a.H * (a.N / BN)));
  constexpr int LDS = gr_attn_bwd_lds<D, BM, BN>::BYTES;
  const bool pre = bwd_prescale<T>(a);
  const dim3 blk(BN / 32 * 64);
  if constexpr (D == 128) {
    if (causal && pre) hipLaunchKernelGGL((gr_attn_bwd128_kernel<T, BM, BN, true, true>), grid, blk, LDS, st, a);
    else if (causal) hipLaunchKernelGGL((gr_attn_bwd128_kernel<T, BM, BN, true, false>), grid, blk, LDS, st, a);
    else if (pre) hipLaunchKernelGGL((gr_attn_bwd128_kernel<T, BM, BN, false, true>), grid, blk, LDS, st, a);
    else hipLaunchKernelGGL((gr_attn_bwd128_kernel<T, BM, BN, false, false>), grid, blk, LDS, st, a);
  } else {
    if (causal && pre) hipLaunchKernelGGL((gr_attn_bwd_kernel<T, D, BM, BN, true, true>), grid, blk, LDS, st, a);
    else if (causal) hipLaunchKernelGGL((gr_attn_bwd_kernel<T, D, BM, BN, true, false>), grid, blk, LDS, st, a);
    else if (pre) hipLaunchKernelGGL((gr_attn_bwd_kernel<T, D, BM, BN, false, true>), grid, blk, LDS, st, a);
    else hipLaunchKernelGGL((gr_attn_bwd_kernel<T, D, BM, BN, false, false>), grid, blk, LDS, st, a);
  }
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_bwd dK/dV launch");
}

}  // namespace

// The d = 128 launches (gr_attn_bwd128.hip).
int gr_attn_bwd_launch_d128(const gr_attn_bwd_args& a, bool bf16, bool causal, hipStream_t st);
