#include "gr_gemm_f32.h"

// generated from a grammar program: 8 stage(s), storage fp32

// stage S: fp32 MFMA GEMM 512x512x64 (x1), tile 64x32x32
extern "C" __global__ __launch_bounds__(128)
void t_S_kernel(const float* __restrict__ t_Q, const float* __restrict__ t_KT, float* __restrict__ t_S) {
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = t_Q; a.b = t_KT; a.c = t_S;
  a.a_sb = 32768LL; a.a_sm = 64;
  a.b_sb = 32768LL; a.b_s = 512;
  a.c_sb = 262144LL; a.c_sm = 512;
  a.M = 512; a.N = 512; a.K = 64;
  a.alpha = 1.0f;
  gr_gemm_f32_body<64, 32, 32, 2, 1, false, 0>(a, gr_gemm_smem);
}


// stage Ss: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_Ss_kernel(const float* __restrict__ t_S, float* __restrict__ t_Ss) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_S + (row / 1LL) * 512LL + c0);
    float y[8];
  #pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (x1[k] * 0.125f);
    gr_row_store<8>(t_Ss + (row / 1LL) * 512LL + c0, y);
  }
}


// stage mx: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_mx_kernel(const float* __restrict__ t_Ss, float* __restrict__ t_mx) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  float r2 = -GR_INF;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_Ss + (row / 1LL) * 512LL + c0);
  #pragma unroll
    for (int k = 0; k < 8; ++k) {
      r2 = fmaxf(r2, x1[k]);
    }
  }
  r2 = gr_wave_max(r2);
  if (lane == 0) t_mx[(row / 1LL) * 1LL] = (float)r2;
}


// stage sb: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_sb_kernel(const float* __restrict__ t_Ss, const float* __restrict__ t_mx, float* __restrict__ t_sb) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  const float s2 = (float)t_mx[(row / 1LL) * 1LL];
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_Ss + (row / 1LL) * 512LL + c0);
    float y[8];
  #pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (x1[k] - s2);
    gr_row_store<8>(t_sb + (row / 1LL) * 512LL + c0, y);
  }
}


// stage e: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_e_kernel(const float* __restrict__ t_sb, float* __restrict__ t_e) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_sb + (row / 1LL) * 512LL + c0);
    float y[8];
  #pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (__expf(x1[k]));
    gr_row_store<8>(t_e + (row / 1LL) * 512LL + c0, y);
  }
}


// stage sm: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_sm_kernel(const float* __restrict__ t_e, float* __restrict__ t_sm) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  float r2 = 0.f;
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_e + (row / 1LL) * 512LL + c0);
  #pragma unroll
    for (int k = 0; k < 8; ++k) {
      r2 += x1[k];
    }
  }
  r2 = gr_wave_sum(r2);
  if (lane == 0) t_sm[(row / 1LL) * 1LL] = (float)r2;
}


// stage P: row lowering (512 rows x 512, one wave per row, 8-wide accesses)
extern "C" __global__ __launch_bounds__(256)
void t_P_kernel(const float* __restrict__ t_e, const float* __restrict__ t_sm, float* __restrict__ t_P) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= 512LL) return;
  const float s2 = (float)t_sm[(row / 1LL) * 1LL];
  for (int c0 = lane * 8; c0 < 512; c0 += 512) {
    float x1[8]; gr_row_load<8>(x1, t_e + (row / 1LL) * 512LL + c0);
    float y[8];
  #pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (x1[k] / s2);
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

/*GR_PLAN {"dtype": "fp32", "fn": "fn", "inputs": ["KT", "Q", "V"], "intermediates": ["P", "S", "Ss", "e", "mx", "sb", "sm"], "meta": {"dtype": "fp32", "flops": 68681728, "flops_exact": true, "inputs": [["KT", [64, 512]], ["Q", [512, 64]], ["V", [512, 64]]], "output": ["O", [512, 64]]}, "outputs": ["O"], "steps": [{"args": ["Q", "KT", "S"], "block": [128, 1, 1], "grid": [128, 1, 1], "kernel": "t_S_kernel", "lds": 28672, "lowering": "gemm", "tiles": {"block_k": 32, "block_m": 64, "block_n": 32}}, {"args": ["S", "Ss"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_Ss_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["Ss", "mx"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_mx_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["Ss", "mx", "sb"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_sb_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["sb", "e"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_e_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["e", "sm"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_sm_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["e", "sm", "P"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_P_kernel", "lds": 0, "lowering": "rows", "tiles": {"vec": 8}}, {"args": ["P", "V", "O"], "block": [64, 1, 1], "grid": [32, 1, 8], "kernel": "t_O_kernel", "lds": 19456, "lowering": "gemm", "tiles": {"block_k": 32, "block_m": 32, "block_n": 32, "ksplit": 8}}, {"args": ["P", "V", "O"], "block": [256, 1, 1], "grid": [32, 1, 1], "kernel": "t_O_reduce_kernel", "lds": 0, "lowering": "gemm", "merge": true}], "tensors": {"KT": [64, 512], "O": [512, 64], "P": [512, 512], "Q": [512, 64], "S": [512, 512], "Ss": [512, 512], "V": [512, 64], "e": [512, 512], "mx": [512, 1], "sb": [512, 512], "sm": [512, 1]}} GR_PLAN*/
