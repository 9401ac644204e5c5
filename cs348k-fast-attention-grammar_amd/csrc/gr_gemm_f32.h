// gr_gemm_f32.h -- batched fp32 GEMM with a fused epilogue on the fp32 matrix
// cores of gfx950 (v_mfma_f32_32x32x2_f32), for the grammar's fp32 programs.
//
//   C[z] = act(alpha * A[z] @ B[z]) [+ R[z]]   A [M, K], B [K, N] or K-major [N, K],
//                                              C, R [M, N]
//
// The reference's programs are fp32 end to end; without this their matmul
// stages would run on the generic LDS lowering's scalar FMAs.
//
// Design (one workgroup = WGM x WGN waves = a BM x BN tile of C):
//  * Transposed form C^T = B^T A^T, as in gr_gemm.h: the MFMA "A" operand is
//    a 32-column block of B (one n per lane), the "B" operand a 32-row block
//    of A (one m per lane); the accumulators give each lane one row m of C
//    with runs of 4 consecutive n, stored as 16-byte writes.
//  * A 32x32x2 MFMA contracts two k, one per half-wave. A lane reads 4
//    consecutive k of its row of A in one 16-byte LDS read and feeds them to 4
//    MFMAs; half-wave g takes k = kb + 4g + t in MFMA t. The B operand pairs
//    the same k: 16-byte reads of a K-major B, else four 4-byte reads down a
//    column of the [BK][BN] tile.
//  * Tiles go global -> registers -> LDS (16-byte accesses), two LDS stages,
//    the next tile's loads issued before the current tile's MFMAs and one
//    barrier per k tile. Rows are padded (A and K-major B by 4 floats, a
//    [BK][BN] B by 8) so the fragment reads of the 16 or 32 lanes that the
//    LDS serves together fall on distinct banks.
//  * M, N multiples of the tile, K of BK; row strides multiples of 4 floats.
#pragma once
#include "gr_gemm.h"

template <int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR>
struct gr_gemm_f32_cfg {
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int A_LD = BK + 4;                          // floats per LDS row of A
  static constexpr int B_LD = B_KMAJOR ? BK + 4 : BN + 8;      // of B^T [BN][BK] or B [BK][BN]
  static constexpr int A_FLOATS = BM * A_LD;
  static constexpr int B_FLOATS = (B_KMAJOR ? BN : BK) * B_LD;
  static constexpr int STAGE = (A_FLOATS + B_FLOATS) * 4;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int A_VEC = BM * BK / 4;                    // 16-byte pieces per tile
  static constexpr int B_VEC = BN * BK / 4;
  static constexpr int A_PER = (A_VEC + NT - 1) / NT;
  static constexpr int B_PER = (B_VEC + NT - 1) / NT;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "each wave owns whole 32x32 blocks");
  static_assert(BK % 8 == 0, "k tile: whole groups of 8 (4 MFMAs of 2)");
};

template <int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI>
__device__ __forceinline__ void gr_gemm_f32_body(const gr_gemm_args& a, char* lds) {
  typedef gr_gemm_f32_cfg<BM, BN, BK, WGM, WGN, B_KMAJOR> G;
  constexpr int NT = G::NT, TM = G::TM, TN = G::TN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = a.N / BN;
  const int bid = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int tm = bid / tiles_n, tn = bid % tiles_n;
  const long long z = blockIdx.y;
  // split K (ksplit > 1): this workgroup's part of the contraction, its
  // partial product written to its own C slice (gr_gemm_f32_reduce_body sums them)
  const int kpart = a.K / a.ksplit, k0 = (int)blockIdx.z * kpart;
  const float* A = static_cast<const float*>(a.a) + z * a.a_sb + (long long)tm * BM * a.a_sm + k0;
  const float* B = static_cast<const float*>(a.b) + z * a.b_sb +
                   (B_KMAJOR ? (long long)tn * BN * a.b_s + k0 : (long long)tn * BN + (long long)k0 * a.b_s);
  float* C = static_cast<float*>(a.c) + blockIdx.z * a.c_sz + z * a.c_sb + (long long)tm * BM * a.c_sm +
             (long long)tn * BN;

  gr_f32x16 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = (gr_f32x16)(0.f);

  // global -> register staging of one k tile, then register -> LDS
  gr_f32x4 ra[G::A_PER], rb[G::B_PER];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < G::A_PER; ++i) {
      const int v = tid + i * NT;
      if (G::A_VEC % NT == 0 || v < G::A_VEC) {
        const int row = v / (BK / 4), c4 = v % (BK / 4);
        ra[i] = *reinterpret_cast<const gr_f32x4*>(A + (long long)row * a.a_sm + (long long)kt * BK + c4 * 4);
      }
    }
#pragma unroll
    for (int i = 0; i < G::B_PER; ++i) {
      const int v = tid + i * NT;
      if (G::B_VEC % NT == 0 || v < G::B_VEC) {
        if constexpr (B_KMAJOR) {
          const int row = v / (BK / 4), c4 = v % (BK / 4);          // row = n
          rb[i] = *reinterpret_cast<const gr_f32x4*>(B + (long long)row * a.b_s + (long long)kt * BK + c4 * 4);
        } else {
          const int row = v / (BN / 4), c4 = v % (BN / 4);          // row = k
          rb[i] = *reinterpret_cast<const gr_f32x4*>(B + ((long long)kt * BK + row) * a.b_s + c4 * 4);
        }
      }
    }
  };
  auto sstore = [&](char* st) {
    float* la = reinterpret_cast<float*>(st);
    float* lb = la + G::A_FLOATS;
#pragma unroll
    for (int i = 0; i < G::A_PER; ++i) {
      const int v = tid + i * NT;
      if (G::A_VEC % NT == 0 || v < G::A_VEC)
        *reinterpret_cast<gr_f32x4*>(la + (v / (BK / 4)) * G::A_LD + (v % (BK / 4)) * 4) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < G::B_PER; ++i) {
      const int v = tid + i * NT;
      if (G::B_VEC % NT == 0 || v < G::B_VEC) {
        constexpr int CPR = B_KMAJOR ? BK / 4 : BN / 4;
        *reinterpret_cast<gr_f32x4*>(lb + (v / CPR) * G::B_LD + (v % CPR) * 4) = rb[i];
      }
    }
  };
  auto mma_tile = [&](const char* st) {
    const float* la = reinterpret_cast<const float*>(st);
    const float* lb = la + G::A_FLOATS;
#pragma unroll
    for (int kb = 0; kb < BK; kb += 8) {
      gr_f32x4 af[TM], bf[TN];
#pragma unroll
      for (int j = 0; j < TM; ++j)
        af[j] = *reinterpret_cast<const gr_f32x4*>(la + (wm * G::WM + j * 32 + l32) * G::A_LD + kb + 4 * g);
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int n = wn * G::WN + i * 32 + l32;
        if constexpr (B_KMAJOR) {
          bf[i] = *reinterpret_cast<const gr_f32x4*>(lb + n * G::B_LD + kb + 4 * g);
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) bf[i][t] = lb[(kb + 4 * g + t) * G::B_LD + n];
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int j = 0; j < TM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[i][t], af[j][t], acc[i][j], 0, 0, 0);
    }
  };

  const int nk = kpart / BK;
  gload(0);
  sstore(lds);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload(kt + 1);
    mma_tile(lds + (kt & 1) * G::STAGE);
    if (kt + 1 < nk) sstore(lds + ((kt + 1) & 1) * G::STAGE);
    __syncthreads();
  }

  // lane (l32, g) of block (i, j): row m = wm*WM + 32j + l32, columns
  // n = wn*WN + 32i + 8q + 4g + (0..3) in accumulators 4q..4q+3
  // (a null residual adds nothing: a split stage whose sum is taken by its
  // consumer adds R in its first K part only)
  const float* R = ((EPI & GR_EPI_RES) && a.r) ? static_cast<const float*>(a.r) + z * a.r_sb +
                                                     (long long)tm * BM * a.r_sm + (long long)tn * BN
                                               : nullptr;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = wm * G::WM + j * 32 + l32;
    float* crow = C + (long long)row * a.c_sm;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wn * G::WN + i * 32 + 8 * q + 4 * g;
        gr_f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + e]);
        if constexpr ((EPI & GR_EPI_RES) != 0) {
          if (R) w += *reinterpret_cast<const gr_f32x4*>(R + (long long)row * a.r_sm + col);
        }
        *reinterpret_cast<gr_f32x4*>(crow + col) = w;
      }
  }
}

// The second launch of a split-K GEMM: C = act(alpha * sum_s P_s) [+ R] over
// the ksplit partial products P_s (at ws + s * ws_sz, laid out as C with
// row stride N, batch stride M N). One thread per 4 consecutive columns of
// one row; the grid covers batch * M * N / 4 threads in workgroups of 256.
template <int EPI>
__device__ __forceinline__ void gr_gemm_f32_reduce_body(const gr_gemm_args& a, const float* ws, int ksplit,
                                                        long long ws_sz, int batch) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long per = (long long)a.M * a.N / 4;
  if (idx >= per * batch) return;
  const long long z = idx / per, e4 = (idx % per) * 4;
  const int row = (int)(e4 / a.N), col = (int)(e4 % a.N);
  gr_f32x4 sum = (gr_f32x4)(0.f);
  for (int s = 0; s < ksplit; ++s)
    sum += *reinterpret_cast<const gr_f32x4*>(ws + s * ws_sz + z * a.M * (long long)a.N + e4);
  gr_f32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = gr_epilogue<EPI>(a.alpha * sum[e]);
  if constexpr ((EPI & GR_EPI_RES) != 0)
    w += *reinterpret_cast<const gr_f32x4*>(static_cast<const float*>(a.r) + z * a.r_sb + (long long)row * a.r_sm + col);
  *reinterpret_cast<gr_f32x4*>(static_cast<float*>(a.c) + z * a.c_sb + (long long)row * a.c_sm + col) = w;
}

template <int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI>
__global__ __launch_bounds__(WGM * WGN * 64) void gr_gemm_f32_kernel(gr_gemm_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_gemm_f32_body<BM, BN, BK, WGM, WGN, B_KMAJOR, EPI>(a, gr_lds);
}
