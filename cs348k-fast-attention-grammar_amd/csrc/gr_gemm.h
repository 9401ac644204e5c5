// gr_gemm.h -- batched MFMA GEMM with a fused elementwise epilogue, gfx950.
//
//   C[z] = act(alpha * A[z] @ B[z]) [+ R[z]]   A [M, K] (unit stride on K)
//                                              B [K, N] (unit stride on N), or K-major [N, K]
//                                              C, R [M, N] (unit stride on N), fp32 accumulate
//
// This is the grammar's matmul stage (Compute("matmul") over a contraction
// axis, optionally followed by mulc, relu/silu and the add of a loaded
// residual tensor) and the two GEMMs of the MLP block (silu after the first).
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
//  * A ring of STAGES LDS stages: k tiles go straight from global memory into
//    LDS (global_load_lds, no staging registers) STAGES - 1 tiles ahead of the
//    one feeding the MFMAs; one barrier per k tile, and each wave waits only
//    for the next tile's loads before it.
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
#define GR_EPI_RES 4     // flag: + R after the activation (residual add, in fp32 before the rounding)
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
  const void* r = nullptr;        // residual R (GR_EPI_RES), laid out like C
  long long r_sb = 0, r_sm = 0;   // its batch and row strides
  int ksplit = 1;                 // fp32 GEMM: blockIdx.z takes K part blockIdx.z of ksplit ...
  long long c_sz = 0;             // ... and writes it at C + blockIdx.z * c_sz
};

template <int EPI>
__device__ __forceinline__ float gr_epilogue(float v) {
  if constexpr ((EPI & 3) == GR_EPI_RELU) return v > 0.f ? v : 0.f;
  else if constexpr ((EPI & 3) == GR_EPI_SILU)
    return v * __builtin_amdgcn_rcpf(1.f + gr_exp2(v * -1.4426950408889634f));
  else return v;
}

// s_waitcnt that waits only until at most N vector memory operations of this
// wave are outstanding (expcnt and lgkmcnt left at their "no wait" maxima).
template <int N>
__device__ __forceinline__ void gr_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES = 2>
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
  static constexpr int LDS = STAGES * STAGE > C_BYTES ? STAGES * STAGE : C_BYTES;
  static_assert(STAGES >= 2, "at least a double-buffered ring");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "each wave owns whole 32x32 blocks");
  static_assert(BK % 16 == 0 && BK >= 16, "k tile");
  // 16-byte operand reads use chunk pairs (2*ks + lane/32): a row needs >= 2 chunks
  static_assert(BK / 8 >= 2, "k tile");
};

template <class T, int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI, int STAGES = 2>
__device__ __forceinline__ void gr_gemm_body(const gr_gemm_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN, STAGES> G;
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

  // Tiles go straight from global memory into a ring of STAGES LDS stages,
  // STAGES - 1 k tiles ahead of the one feeding the MFMAs. Before the barrier
  // that publishes tile kt + 1, each wave waits only for its own loads of that
  // tile (the loads of the later tiles stay in flight; a wave's vector memory
  // operations complete in order). The stage a load overwrites held tile
  // kt - 1, whose last reads finished before the previous barrier.
  const int nk = a.K / BK;
  gr_lds_loader<T, BM, BK, NT> la;
  // A [K, N] B is copied into LDS as laid out in memory ([BK][BN], swizzled for
  // transposing reads) and its fragments are read back with gr_tr_frag; a
  // K-major B is already [BN][BK].
  typedef typename gr_cond<B_KMAJOR, gr_lds_loader<T, BN, BK, NT>, gr_lds_loader<T, BK, BN, NT, true>>::type LB;
  LB lb;
  la.init(tid, a.a_sm, rows_ok);
  if constexpr (B_KMAJOR) lb.init(tid, a.b_s, cols_ok);
  else lb.init(tid, a.b_s, BK, cols_ok / 8);
  // vector memory operations per thread and k tile (every thread issues the same count)
  constexpr int PER_TILE = gr_lds_loader<T, BM, BK, NT>::PER + LB::PER;
  // partial waits count loads: every thread must issue the same number per tile
  static_assert(STAGES == 2 || ((BM * BK / 8) % NT == 0 && (BN * BK / 8) % NT == 0),
                "a ring deeper than two stages needs whole 16-byte chunks per thread");
  auto load_tile = [&](int kt) {
    char* dst = lds + (kt % STAGES) * G::STAGE;
    la.load(A + (long long)kt * BK, dst);
    lb.load(B + (long long)kt * b_step, dst + G::A_BYTES);
  };
  // wait until tile `next` has landed, with `ahead` later tiles in flight
  auto wait_for = [&](int ahead) {
    if constexpr (STAGES >= 4) {
      if (ahead >= 2) { gr_wait_vmcnt<2 * PER_TILE>(); return; }
    }
    if constexpr (STAGES >= 3) {
      if (ahead >= 1) { gr_wait_vmcnt<PER_TILE>(); return; }
    }
    gr_wait_vmcnt<0>();
  };
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) load_tile(s);
  {
    const int issued = nk < STAGES - 1 ? nk : STAGES - 1;
    wait_for(issued - 1);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + STAGES - 1 < nk) load_tile(kt + STAGES - 1);
    mma_tile(lds + (kt % STAGES) * G::STAGE);
    // tiles issued beyond kt + 1
    const int last = kt + STAGES - 1 < nk ? kt + STAGES - 1 : nk - 1;
    wait_for(last - (kt + 1) > 0 ? last - (kt + 1) : 0);
    __syncthreads();
  }

  // epilogue: lane (l32, g) of block (i, j) holds row m = wm*WM + 32j + l32 and
  // columns n = wn*WN + 32i + 8q + 4g + (0..3) in registers 4q..4q+3. The tile
  // goes through LDS (16-byte chunks XOR-swizzled by row, as the operand
  // tiles) so that the global stores are whole 16-byte chunks of contiguous
  // row segments. The main loop's final barrier has retired every operand read.
  constexpr int OCPR = BN / 8;
  const T* R = (EPI & GR_EPI_RES)
                   ? static_cast<const T*>(a.r) + z * a.r_sb + (long long)tm * BM * a.r_sm + (long long)tn * BN
                   : nullptr;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = wm * G::WM + j * 32 + l32;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wn * G::WN + i * 32 + 8 * q + 4 * g;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gr_epilogue<EPI>(a.alpha * acc[i][j][4 * q + e]);
        if constexpr ((EPI & GR_EPI_RES) != 0) {
          // the residual's 4 values of this lane (rows and columns past the
          // edge of C are never stored, and not read)
          if (row < rows_ok && col < cols_ok) {
            const gr_u32x2 rw = *reinterpret_cast<const gr_u32x2*>(R + (long long)row * a.r_sm + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const unsigned short h = (unsigned short)(rw[e >> 1] >> (16 * (e & 1)));
              v[e] += (float)__builtin_bit_cast(T, h);
            }
          }
        }
        gr_u32x2 w;
        w[0] = gr_pack2f<T>(v[0], v[1]);
        w[1] = gr_pack2f<T>(v[2], v[3]);
        *reinterpret_cast<gr_u32x2*>(lds + row * (BN * 2) + gr_swz<OCPR>(row, col >> 3) * 16 + g * 8) = w;
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
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN, 2> G;
  static constexpr int LOADER = (BM * BK / 8 + G::NT - 1) / G::NT + (BN * BK / 8 + G::NT - 1) / G::NT;
  static constexpr int EST = 16 * G::TN * G::TM + 4 * (G::TN + G::TM) + LOADER + 40;
  static constexpr int value = EST > 240 ? 1 : 2;
};

template <class T, int BM, int BN, int BK, int WGM, int WGN, bool B_KMAJOR, int EPI, int STAGES = 2>
__global__ __launch_bounds__(WGM * WGN * 64)
__attribute__((amdgpu_waves_per_eu(gr_gemm_wpe<BM, BN, BK, WGM, WGN, B_KMAJOR>::value)))
void gr_gemm_kernel(gr_gemm_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_gemm_body<T, BM, BN, BK, WGM, WGN, B_KMAJOR, EPI, STAGES>(a, gr_lds);
}
