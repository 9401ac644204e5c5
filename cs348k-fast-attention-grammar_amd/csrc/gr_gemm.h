// gr_gemm.h -- batched MFMA GEMM with a fused elementwise epilogue, gfx950.
//
//   C[z] = act(alpha * A[z] @ B[z])      A [M, K] (unit stride on K)
//                                        B [K, N] (unit stride on N), or K-major [N, K]
//                                        C [M, N] (unit stride on N), fp32 accumulate
//
// This is the grammar's matmul stage (Compute("matmul") over a contraction
// axis, optionally followed by mulc and relu/silu) and the two GEMMs of the
// MLP block (silu after the first).
//
// Design (one workgroup = WGM x WGN waves = a BM x BN tile of C):
//  * The contraction runs on v_mfma_f32_32x32x16 in the transposed form
//    C^T = B^T A^T: the MFMA "A" operand is a 32-row block of B^T and the "B"
//    operand a 32-row block of A, both read from LDS as one 16-byte load per
//    lane (8 consecutive k). The accumulators then give each lane one row m of
//    C with 4-element runs along n, which are written as 8-byte stores.
//  * LDS holds A as [BM][BK] (k contiguous). A K-major B is held as [BN][BK];
//    a [K, N] B as it is in memory, [BK][BN], its fragments read with
//    gfx950's transposing LDS read (gr_tr_frag). 16-byte chunks are
//    XOR-swizzled by row so the MFMA operand reads and the tile writes are
//    conflict free.
//  * Two LDS stages: the next k tile goes straight from global memory into
//    one stage (global_load_lds, no staging registers) while the current one
//    feeds the MFMAs; one barrier per k tile.
//  * Tiles are walked in groups of GROUP_M tile rows (B columns reused from
//    L2), and the group order is remapped so consecutive groups run on one XCD.
//  * M and N need not be multiples of the tile (N a multiple of 8): edge
//    tiles read their last valid row / 16-byte column chunk in place of the
//    missing ones and store only the valid part. K is a multiple of BK.
#pragma once
#include "gr_flash_fwd.h"

#ifndef GR_EPI_NONE
#define GR_EPI_NONE 0
#define GR_EPI_RELU 1
#define GR_EPI_SILU 2
#endif

struct gr_gemm_args {
  const void* a;
  const void* b;
  void* c;
  long long a_sb, a_sm;   // batch stride, row stride of A
  long long b_sb, b_s;    // batch stride; row stride of B ([K,N]: over k; K-major: over n)
  long long c_sb, c_sm;   // batch stride, row stride of C
  int M, N, K;
  float alpha;
};

template <int EPI>
__device__ __forceinline__ float gr_epilogue(float v) {
  if constexpr (EPI == GR_EPI_RELU) return v > 0.f ? v : 0.f;
  else if constexpr (EPI == GR_EPI_SILU)
    return v * __builtin_amdgcn_rcpf(1.f + gr_exp2(v * -1.4426950408889634f));
  else return v;
}

template <int BM, int BN, int BK, int WGM, int WGN>
struct gr_gemm_cfg {
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = NW * 64;
  static constexpr int WM = BM / WGM;
  static constexpr int WN = BN / WGN;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static constexpr int A_BYTES = BM * BK * 2;
  static constexpr int B_BYTES = BN * BK * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int C_BYTES = BM * BN * 2;     // the output tile, staged for coalesced stores
  static constexpr int LDS = 2 * STAGE > C_BYTES ? 2 * STAGE : C_BYTES;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "each wave owns whole 32x32 blocks");
  static_assert(BK % 16 == 0 && BK >= 16, "k tile");
  // 16-byte operand reads use chunk pairs (2*ks + lane/32): a row needs >= 2 chunks
  static_assert(BK / 8 >= 2, "k tile");
};

template <class T, int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI>
__device__ __forceinline__ void gr_gemm_body(const gr_gemm_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN> G;
  constexpr int NT = G::NT, TM = G::TM, TN = G::TN, CPR = BK / 8;
  constexpr int GROUP_M = 8;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / WGN, wn = wave % WGN;

  // tile walk: grouped rows, XCD-local groups
  const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
  const int ntile = tiles_m * tiles_n;
  const int bid = gr_xcd_remap(blockIdx.x, ntile);
  const int per_group = GROUP_M * tiles_n;
  const int grp = bid / per_group;
  const int first_m = grp * GROUP_M;
  const int gsz = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const int in_grp = bid - grp * per_group;
  const int tm = first_m + in_grp % gsz;
  const int tn = in_grp / gsz;
  const long long z = blockIdx.y;

  const T* A = static_cast<const T*>(a.a) + z * a.a_sb + (long long)tm * BM * a.a_sm;
  const T* B = static_cast<const T*>(a.b) + z * a.b_sb +
               (B_KMAJOR ? (long long)tn * BN * a.b_s : (long long)tn * BN);
  T* C = static_cast<T*>(a.c) + z * a.c_sb + (long long)tm * BM * a.c_sm + (long long)tn * BN;

  const long long b_step = B_KMAJOR ? (long long)BK : (long long)BK * a.b_s;
  // valid rows of this tile of C and valid 16-byte chunks of its rows
  const int rows_ok = a.M - tm * BM < BM ? a.M - tm * BM : BM;
  const int cols_ok = a.N - tn * BN < BN ? a.N - tn * BN : BN;

  gr_f32x16 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = (gr_f32x16)(0.f);

  // one k tile of MFMAs from an LDS stage
  // one k tile of MFMAs from an LDS stage
  auto frags = [&](const char* cur, int ks, vec8 (&bt)[TN], vec8 (&am)[TM]) {
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int row = wn * G::WN + i * 32 + l32;
      if constexpr (B_KMAJOR)
        bt[i] = gr_as<vec8>(gr_ld16(cur + G::A_BYTES + row * (BK * 2) + gr_swz<CPR>(row, 2 * ks + g) * 16));
      else
        bt[i] = gr_tr_frag<T, BN, false>(cur + G::A_BYTES, ks * 16, wn * G::WN + i * 32, lane);
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int row = wm * G::WM + j * 32 + l32;
      am[j] = gr_as<vec8>(gr_ld16(cur + row * (BK * 2) + gr_swz<CPR>(row, 2 * ks + g) * 16));
    }
  };
  auto mma_tile = [&](const char* cur) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      vec8 bt[TN], am[TM];
      frags(cur, ks, bt, am);
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = MF::mma32(bt[i], am[j], acc[i][j]);
    }
  };

  // tiles go straight from global memory into the next LDS stage while the
  // current one feeds the MFMAs; the stage is published after vmcnt drains
  const int nk = a.K / BK;
  gr_lds_loader<T, BM, BK, NT> la;
  // A [K, N] B is copied into LDS as laid out in memory ([BK][BN], swizzled for
  // transposing reads) and its fragments are read back with gr_tr_frag; a
  // K-major B is already [BN][BK].
  typename gr_cond<B_KMAJOR, gr_lds_loader<T, BN, BK, NT>, gr_lds_loader<T, BK, BN, NT, true>>::type lb;
  la.init(tid, a.a_sm, rows_ok);
  if constexpr (B_KMAJOR) lb.init(tid, a.b_s, cols_ok);
  else lb.init(tid, a.b_s, BK, cols_ok / 8);
  la.load(A, lds);
  lb.load(B, lds + G::A_BYTES);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const char* cur = lds + (kt & 1) * G::STAGE;
    char* nxt = lds + ((kt + 1) & 1) * G::STAGE;
    if (kt + 1 < nk) {
      la.load(A + (long long)(kt + 1) * BK, nxt);
      lb.load(B + (long long)(kt + 1) * b_step, nxt + G::A_BYTES);
    }
    mma_tile(cur);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // epilogue: lane (l32, g) of block (i, j) holds row m = wm*WM + 32j + l32 and
  // columns n = wn*WN + 32i + 8q + 4g + (0..3) in registers 4q..4q+3. The tile
  // goes through LDS (16-byte chunks XOR-swizzled by row, as the operand
  // tiles) so that the global stores are whole 16-byte chunks of contiguous
  // row segments. The main loop's final barrier has retired every operand read.
  constexpr int OCPR = BN / 8;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = wm * G::WM + j * 32 + l32;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int chunk = (wn * G::WN + i * 32 + 8 * q) >> 3;
        gr_u32x2 w;
        w[0] = gr_pack2f<T>(gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + 0]),
                            gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + 1]));
        w[1] = gr_pack2f<T>(gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + 2]),
                            gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + 3]));
        *reinterpret_cast<gr_u32x2*>(lds + row * (BN * 2) + gr_swz<OCPR>(row, chunk) * 16 + g * 8) = w;
      }
  }
  __syncthreads();
  constexpr int CHUNKS = BM * OCPR;
#pragma unroll
  for (int it = 0; it < (CHUNKS + NT - 1) / NT; ++it) {
    const int cidx = tid + it * NT;
    if (CHUNKS % NT == 0 || cidx < CHUNKS) {
      const int row = cidx / OCPR, cc = cidx % OCPR;
      const gr_u32x4 v = gr_ld16(lds + row * (BN * 2) + gr_swz<OCPR>(row, cc) * 16);
      if (row < rows_ok && cc * 8 < cols_ok) gr_st16(C + (long long)row * a.c_sm + cc * 8, v);
    }
  }
}

// Waves per SIMD that the register budget allows for a wave tile of TN x TM
// 32x32 blocks: 16*TN*TM accumulators plus 4*(TN+TM) operand registers,
// loader offsets and addressing.
template <int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR>
struct gr_gemm_wpe {
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN> G;
  static constexpr int LOADER = (BM * BK / 8 + G::NT - 1) / G::NT + (BN * BK / 8 + G::NT - 1) / G::NT;
  static constexpr int EST = 16 * G::TN * G::TM + 4 * (G::TN + G::TM) + LOADER + 40;
  static constexpr int value = EST > 240 ? 1 : 2;
};

template <class T, int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI>
__global__ __launch_bounds__(WGM * WGN * 64)
__attribute__((amdgpu_waves_per_eu(gr_gemm_wpe<BM, BN, BK, WGM, WGN, B_KMAJOR>::value)))
void gr_gemm_kernel(gr_gemm_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_gemm_body<T, BM, BN, BK, WGM, WGN, B_KMAJOR, EPI>(a, gr_lds);
}
