#include "gr_gemm.h"

// generated from a grammar program: 2 stage(s), storage fp32
// stage Ss: generic LDS-tile kernel, tile (16, 16), 9216 B LDS
extern "C" __global__ __launch_bounds__(256) void t_Ss_kernel(const float* __restrict__ t_Q, const float* __restrict__ t_KT, float* __restrict__ t_Ss) {
  extern __shared__ __attribute__((aligned(16))) float gr_lds[];
  constexpr int B0 = 0;
  constexpr int B1 = 1024;
  constexpr int B2 = 2048;
  constexpr int B3 = 0;
  int bid = blockIdx.x;
  const int b_t_j = bid % 32; bid /= 32;
  const int b_t_i = bid % 32; bid /= 32;
  for (int e = threadIdx.x; e < 1024; e += 256) {
    const int i0 = (e / 64);
    const int i1 = e % 64;
    gr_lds[B0 + e] = (float)t_Q[(long long)((b_t_i)*16 + i0)*64 + (long long)(i1)];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 1024; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    gr_lds[B1 + e] = (float)t_KT[(long long)(i0)*512 + (long long)((b_t_j)*16 + i1)];
  }
  __syncthreads();
  // matmul: C = A @ B (K = 64)
  for (int e = threadIdx.x; e < 256; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    float s = 0.f;
    for (int k = 0; k < 64; ++k) s = fmaf(gr_lds[B0 + (i0)*64 + (k)], gr_lds[B1 + (k)*16 + (i1)], s);
    gr_lds[B2 + e] = s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    gr_lds[B3 + e] = gr_lds[B2 + (i0)*16 + (i1)] * 0.125f;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    t_Ss[(long long)((b_t_i)*16 + i0)*512 + (long long)((b_t_j)*16 + i1)] = (float)gr_lds[B3 + (i0)*16 + (i1)];
  }
  __syncthreads();
}

// stage O: generic LDS-tile kernel, tile (16, 16), 66560 B LDS
extern "C" __global__ __launch_bounds__(256) void t_O_kernel(const float* __restrict__ t_Ss, const float* __restrict__ t_V, float* __restrict__ t_O) {
  extern __shared__ __attribute__((aligned(16))) float gr_lds[];
  constexpr int B0 = 0;
  constexpr int B1 = 8192;
  constexpr int B2 = 16384;
  int bid = blockIdx.x;
  const int b_t_dd = bid % 4; bid /= 4;
  const int b_t_i = bid % 32; bid /= 32;
  for (int e = threadIdx.x; e < 8192; e += 256) {
    const int i0 = (e / 512);
    const int i1 = e % 512;
    gr_lds[B0 + e] = (float)t_Ss[(long long)((b_t_i)*16 + i0)*512 + (long long)(i1)];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 8192; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    gr_lds[B1 + e] = (float)t_V[(long long)(i0)*64 + (long long)((b_t_dd)*16 + i1)];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    float m = -GR_INF;
    for (int k = 0; k < 512; ++k) m = fmaxf(m, gr_lds[B0 + (i0)*512 + (k)]);
    if (m == -GR_INF) m = 0.f;
    float l = 0.f, s = 0.f;
    for (int k = 0; k < 512; ++k) { const float p = __expf(gr_lds[B0 + (i0)*512 + (k)] - m); l += p; s = fmaf(p, gr_lds[B1 + (k)*16 + (i1)], s); }
    gr_lds[B2 + e] = s / l;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 256) {
    const int i0 = (e / 16);
    const int i1 = e % 16;
    t_O[(long long)((b_t_i)*16 + i0)*64 + (long long)((b_t_dd)*16 + i1)] = (float)gr_lds[B2 + (i0)*16 + (i1)];
  }
  __syncthreads();
}

/*GR_PLAN {"dtype": "fp32", "fn": "fn", "inputs": ["KT", "Q", "V"], "intermediates": ["Ss"], "meta": {"dtype": "fp32", "flops": 68681728, "flops_exact": true, "inputs": [["KT", [64, 512]], ["Q", [512, 64]], ["V", [512, 64]]], "output": ["O", [512, 64]]}, "outputs": ["O"], "steps": [{"args": ["Q", "KT", "Ss"], "block": [256, 1, 1], "grid": [1024, 1, 1], "kernel": "t_Ss_kernel", "lds": 9216, "lowering": "generic"}, {"args": ["Ss", "V", "O"], "block": [256, 1, 1], "grid": [128, 1, 1], "kernel": "t_O_kernel", "lds": 66560, "lowering": "generic"}], "tensors": {"KT": [64, 512], "O": [512, 64], "Q": [512, 64], "Ss": [512, 512], "V": [512, 64]}} GR_PLAN*/
