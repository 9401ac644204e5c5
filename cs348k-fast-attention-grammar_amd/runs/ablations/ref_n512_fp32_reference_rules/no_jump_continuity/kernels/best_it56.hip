#include "gr_gemm_f32.h"

// generated from a grammar program: 3 stage(s), storage fp32

// stage Ss: fp32 MFMA GEMM 512x512x64 (x1), tile 32x64x32
extern "C" __global__ __launch_bounds__(128)
void t_Ss_kernel(const float* __restrict__ t_KT, const float* __restrict__ t_Q, float* __restrict__ t_Ss) {
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = t_Q; a.b = t_KT; a.c = t_Ss;
  a.a_sb = 32768LL; a.a_sm = 64;
  a.b_sb = 32768LL; a.b_s = 512;
  a.c_sb = 262144LL; a.c_sm = 512;
  a.M = 512; a.N = 512; a.K = 64;
  a.alpha = 0.125f;
  gr_gemm_f32_body<32, 64, 32, 1, 2, false, 0>(a, gr_gemm_smem);
}


// stage P: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_P_kernel(const float* __restrict__ t_Ss, float* __restrict__ t_P) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  float r3 = -GR_INF;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x2[8]; gr_row_load<8>(x2, t_Ss + (row / 1LL) * 512LL + c0);
  #pragma unroll
    for (int k = 0; k < 8; ++k) {
      r3 = fmaxf(r3, x2[k]);
    }
  }
  r3 = gr_wave_max(r3);
  float r5 = 0.f;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x4[8]; gr_row_load<8>(x4, t_Ss + (row / 1LL) * 512LL + c0);
  #pragma unroll
    for (int k = 0; k < 8; ++k) {
      r5 += (__expf((x4[k] - r3)));
    }
  }
  r5 = gr_wave_sum(r5);
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_Ss + (row / 1LL) * 512LL + c0);
    float y[8];
  #pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = ((__expf((x1[k] - r3))) / r5);
    gr_row_store<8>(t_P + (row / 1LL) * 512LL + c0, y);
  }
}


// stage O: fp32 MFMA GEMM 512x64x512 (x1), tile 32x32x32, K split over
// 8 workgroups; their partial products live in this module's workspace between the two launches,
// so two runs of the module must not overlap
__device__ float gr_ws_t_O[262144];
extern "C" __global__ __launch_bounds__(64)
void t_O_kernel(const float* __restrict__ t_P, const float* __restrict__ t_V, float* __restrict__ t_O) {
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = t_P; a.b = t_V; a.c = t_O;
  a.a_sb = 262144LL; a.a_sm = 512;
  a.b_sb = 32768LL; a.b_s = 64;
  a.c_sb = 32768LL; a.c_sm = 64;
  a.M = 512; a.N = 64; a.K = 512;
  a.alpha = 1.0f;
  a.c = gr_ws_t_O; a.c_sb = 32768LL; a.alpha = 1.0f; a.r = nullptr;
  a.ksplit = 8; a.c_sz = 32768LL;
  gr_gemm_f32_body<32, 32, 32, 1, 1, false, 0>(a, gr_gemm_smem);
}
extern "C" __global__ __launch_bounds__(256)
void t_O_reduce_kernel(const float* __restrict__ t_P, const float* __restrict__ t_V, float* __restrict__ t_O) {
  gr_gemm_args a;
  a.a = t_P; a.b = t_V; a.c = t_O;
  a.a_sb = 262144LL; a.a_sm = 512;
  a.b_sb = 32768LL; a.b_s = 64;
  a.c_sb = 32768LL; a.c_sm = 64;
  a.M = 512; a.N = 64; a.K = 512;
  a.alpha = 1.0f;
  gr_gemm_f32_reduce_body<0>(a, gr_ws_t_O, 8, 32768LL, 1);
}

/*GR_PLAN {"dtype": "fp32", "fn": "fn", "inputs": ["KT", "Q", "V"], "intermediates": ["P", "Ss"], "meta": {"dtype": "fp32", "flops": 68681728, "flops_exact": true, "inputs": [["KT", [64, 512]], ["Q", [512, 64]], ["V", [512, 64]]], "output": ["O", [512, 64]]}, "outputs": ["O"], "steps": [{"args": ["KT", "Q", "Ss"], "block": [128, 1, 1], "grid": [128, 1, 1], "kernel": "t_Ss_kernel", "lds": 27648, "lowering": "gemm", "tiles": {"block_k": 32, "block_m": 32, "block_n": 64}}, {"args": ["Ss", "P"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_P_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["P", "V", "O"], "block": [64, 1, 1], "grid": [32, 1, 8], "kernel": "t_O_kernel", "lds": 19456, "lowering": "gemm", "tiles": {"block_k": 32, "block_m": 32, "block_n": 32, "ksplit": 8}}, {"args": ["P", "V", "O"], "block": [256, 1, 1], "grid": [32, 1, 1], "kernel": "t_O_reduce_kernel", "lds": 0, "lowering": "gemm", "merge": true}], "tensors": {"KT": [64, 512], "O": [512, 64], "P": [512, 512], "Q": [512, 64], "Ss": [512, 512], "V": [512, 64]}} GR_PLAN*/
