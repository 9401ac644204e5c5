#include "gr_gemm_f32.h"
#include "gr_flash_f32.h"

// generated from a grammar program: 1 stage(s), storage fp32

// stage O: fp32 flash attention on the fp32 matrix cores (32 queries x 4 chunk(s) of 32 keys
// per workgroup, one chunk per wave, merged in LDS; 4 workgroup(s) per query block)
// partials of the 4 workgroups of each query block, merged by t_O_merge_kernel;
// they are this module's, so two launches of it must not overlap
__device__ float gr_ws_t_O[131072];
__device__ float gr_ml_t_O[4096];
extern "C" __global__ __launch_bounds__(256)
void t_O_kernel(const float* __restrict__ t_KT, const float* __restrict__ t_Q, const float* __restrict__ t_V, float* __restrict__ t_O) {
  extern __shared__ __attribute__((aligned(16))) char gr_flash_smem[];
  gr_attn_args a;
  a.q = t_Q; a.k = t_KT; a.v = t_V; a.o = t_O;
  a.q_sb = 32768LL; a.q_sh = 0; a.q_sn = 64;
  a.k_sb = 32768LL; a.k_sh = 0; a.k_sn = 512;
  a.v_sb = 32768LL; a.v_sh = 0; a.v_sn = 64;
  a.o_sb = 32768LL; a.o_sh = 0; a.o_sn = 64;
  a.B = 1; a.H = 1; a.N = 512; a.Nq = 512;
  a.scale_log2 = 0.18033688011112042f;
  gr_flash32_fwd_body<64, 32, 4, true, 4>(a, gr_flash_smem, gr_ws_t_O, gr_ml_t_O);
}
extern "C" __global__ __launch_bounds__(256)
void t_O_merge_kernel(const float* __restrict__ t_KT, const float* __restrict__ t_Q, const float* __restrict__ t_V, float* __restrict__ t_O) {
  gr_attn_args a;
  a.q = t_Q; a.k = t_KT; a.v = t_V; a.o = t_O;
  a.q_sb = 32768LL; a.q_sh = 0; a.q_sn = 64;
  a.k_sb = 32768LL; a.k_sh = 0; a.k_sn = 512;
  a.v_sb = 32768LL; a.v_sh = 0; a.v_sn = 64;
  a.o_sb = 32768LL; a.o_sh = 0; a.o_sn = 64;
  a.B = 1; a.H = 1; a.N = 512; a.Nq = 512;
  a.scale_log2 = 0.18033688011112042f;
  gr_flash32_merge_body<64, 4>(a, gr_ws_t_O, gr_ml_t_O);
}

/*GR_PLAN {"dtype": "fp32", "fn": "fn", "inputs": ["KT", "Q", "V"], "intermediates": [], "meta": {"dtype": "fp32", "flops": 68681728, "flops_exact": true, "inputs": [["KT", [64, 512]], ["Q", [512, 64]], ["V", [512, 64]]], "output": ["O", [512, 64]]}, "outputs": ["O"], "steps": [{"args": ["KT", "Q", "V", "O"], "block": [256, 1, 1], "grid": [64, 1, 1], "kernel": "t_O_kernel", "lds": 35840, "lowering": "flash", "tiles": {"block_m": 128, "block_n": 32, "parts": 4, "waves": 4}}, {"args": ["KT", "Q", "V", "O"], "block": [256, 1, 1], "grid": [16, 1, 1], "kernel": "t_O_merge_kernel", "lds": 0, "lowering": "flash", "merge": true}], "tensors": {"KT": [64, 512], "O": [512, 64], "Q": [512, 64], "V": [512, 64]}} GR_PLAN*/
