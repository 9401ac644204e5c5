// gr_attn_bwd128.hip -- the d = 128 instances of the attention backward.
// Compiled with MFMAs in VGPR form (build_native.py): the dK/dV kernel runs
// one wave per SIMD, and left to its heuristics the backend puts every MFMA
// accumulator in AGPRs and copies the score accumulators to VGPRs (and back)
// for the softmax arithmetic on every tile. In VGPR form the score and dP
// MFMAs write VGPRs, while dK^T and dV^T stay in AGPRs through inline
// assembly (gr_bwd_mfma_agpr).
#include "gr_attn_bwd_launch.h"

int gr_attn_bwd_launch_d128(const gr_attn_bwd_args& a, bool bf16, bool causal, hipStream_t st) {
  return bf16 ? launch_bwd<__bf16, 128, 128, 128>(a, causal, st) : launch_bwd<_Float16, 128, 128, 128>(a, causal, st);
}
