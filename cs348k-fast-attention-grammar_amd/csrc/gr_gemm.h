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

// Epilogue of a BM x BN tile of C: act(alpha * acc) [+ R], through LDS so
// that the global stores are whole 16-byte chunks of contiguous row segments.
// Lane (l32, g) of accumulator block (i, j) holds row m = m0 + 32j + l32 and
// columns n = n0 + 32i + 8q + 4g + (0..3) in registers 4q..4q+3 (the wave's
// block of C starts at (m0, n0)); the staged tile is XOR-swizzled by row as
// the operand tiles are. The caller has retired every LDS operand read of
// the workgroup (a barrier) before the call.
template <class T, int BM, int BN, int TM, int TN, int NT, int EPI>
__device__ __forceinline__ void gr_gemm_store_tile(const gr_gemm_args& a, const gr_f32x16 (&acc)[TN][TM], char* lds,
                                                   int m0, int n0, int tm, int tn, long long z, int rows_ok,
                                                   int cols_ok) {
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  T* C = static_cast<T*>(a.c) + z * a.c_sb + (long long)tm * BM * a.c_sm + (long long)tn * BN;
  constexpr int OCPR = BN / 8;
  const T* R = (EPI & GR_EPI_RES)
                   ? static_cast<const T*>(a.r) + z * a.r_sb + (long long)tm * BM * a.r_sm + (long long)tn * BN
                   : nullptr;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = m0 + j * 32 + l32;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + i * 32 + 8 * q + 4 * g;
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

  // epilogue: the main loop's final barrier has retired every operand read
  gr_gemm_store_tile<T, BM, BN, TM, TN, NT, EPI>(a, acc, lds, wm * G::WM, wn * G::WN, tm, tn, z, rows_ok, cols_ok);
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

// ---------------------------------------------------------------------------
// The 256 x 256 tile at one wave per SIMD (gr_gemm_w4_body): four waves, each
// owning a 128 x 128 block of C in AGPR accumulators (16 blocks of 32 x 32:
// all 256 AGPRs). The main loop's order is fixed by hand: per 16-deep k step
// 16 MFMAs (inline assembly, so that the compiler neither reorders them nor
// moves the accumulators), the next k step's 12 fragment reads after the
// first eight of them, in the order the next step first uses the fragments
// (fragments double-buffered in VGPRs). k tiles go straight from global
// memory into a ring of STAGES LDS stages: the barrier that publishes tile
// t + 1 sits before tile t's last k step, whose fragments are already in
// registers, and during that step the tile's stage is refilled with tile
// t + STAGES, one direct load after each MFMA rather than all at once (a
// burst of loads keeps the wave from issuing its MFMAs). The loop is peeled
// so that no slot carries a branch. Against the two-waves-per-SIMD body on
// the C4 GEMMs this takes H*W2 from 0.623 to 0.574 ms and X*W1 + SiLU from
// 0.692 to 0.636 ms (one box, warm), with bit-identical results (the same
// k order per accumulator).
// ---------------------------------------------------------------------------
template <class V>
__device__ __forceinline__ void gr_mfma32_acc(gr_f32x16& acc, V a, V b) {
  if constexpr (gr_is_same<V, gr_f16x8>::value)
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// k tile -> ring depth of the one-wave body (LDS: two 64-deep or four 32-deep stages)
template <int BK> struct gr_gemm_w4_stages { static constexpr int value = BK == 64 ? 2 : 4; };

// BNT: the tile's columns, 256 (waves of 128 x 128) or 128 (waves of 128 x 64).
template <class T, bool B_KMAJOR, int EPI, int BK = 64, int BNT = 256>
__device__ __forceinline__ void gr_gemm_w4_body(const gr_gemm_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int BM = 256, BN = BNT, WGM = 2, WGN = 2, STAGES = gr_gemm_w4_stages<BK>::value;
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN, STAGES> G;
  constexpr int NT = G::NT, TM = G::TM, TN = G::TN, CPR = BK / 8, KS = BK / 16;
  constexpr int NMF = TN * TM;                       // MFMAs per 16-deep k step
  constexpr int GROUP_M = 8;
  static_assert(NT == 256 && TM == 4 && (TN == 4 || TN == 2), "four waves of 128 x 128 or 128 x 64");
  static_assert(BK == 32 || BK == 64, "32- or 64-deep k tiles");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / WGN, wn = wave % WGN;

  // tile walk: grouped rows, XCD-local groups (as gr_gemm_body)
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
  const long long b_step = B_KMAJOR ? (long long)BK : (long long)BK * a.b_s;
  const int rows_ok = a.M - tm * BM < BM ? a.M - tm * BM : BM;
  const int cols_ok = a.N - tn * BN < BN ? a.N - tn * BN : BN;

  gr_f32x16 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = (gr_f32x16)(0.f);
  // wait states between vector writes of the accumulators and the MFMAs that
  // read them (or back): the compiler counts none into inline assembly
  auto acc_guard = [&]() {
    if constexpr (TN == 4)
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                   : "+a"(acc[0][0]), "+a"(acc[0][1]), "+a"(acc[0][2]), "+a"(acc[0][3]), "+a"(acc[1][0]),
                     "+a"(acc[1][1]), "+a"(acc[1][2]), "+a"(acc[1][3]), "+a"(acc[2][0]), "+a"(acc[2][1]),
                     "+a"(acc[2][2]), "+a"(acc[2][3]), "+a"(acc[3][0]), "+a"(acc[3][1]), "+a"(acc[3][2]),
                     "+a"(acc[3][3]));
    else
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                   : "+a"(acc[0][0]), "+a"(acc[0][1]), "+a"(acc[0][2]), "+a"(acc[0][3]), "+a"(acc[1][0]),
                     "+a"(acc[1][1]), "+a"(acc[1][2]), "+a"(acc[1][3]));
  };
  // the zeroing moves retire before the first MFMA reads them as its
  // accumulator (without this the last-zeroed register of a block was read
  // stale)
  acc_guard();

  const int nk = a.K / BK;
  typedef gr_lds_loader<T, BM, BK, NT> LA;
  typedef typename gr_cond<B_KMAJOR, gr_lds_loader<T, BN, BK, NT>, gr_lds_loader<T, BK, BN, NT, true>>::type LB;
  LA la;
  LB lb;
  la.init(tid, a.a_sm, rows_ok);
  if constexpr (B_KMAJOR) lb.init(tid, a.b_s, cols_ok);
  else lb.init(tid, a.b_s, BK, cols_ok / 8);
  constexpr int PER_A = LA::PER, PER_TILE = LA::PER + LB::PER;   // direct loads per thread and tile
  static_assert((BM * BK / 8) % NT == 0 && (BN * BK / 8) % NT == 0, "whole chunks per thread");
  constexpr int LPS = (PER_TILE + NMF - 1) / NMF;   // direct loads per MFMA slot of a refilling k step
  static_assert(LPS <= 2 && (STAGES - 1) * PER_TILE < 64, "at most two loads per MFMA slot; vmcnt range");
  auto stage = [&](int t) -> char* { return lds + (t % STAGES) * G::STAGE; };
  auto load_tile = [&](int t) {
    if (t < nk) {
      la.load(A + (long long)t * BK, stage(t));
      lb.load(B + (long long)t * b_step, stage(t) + G::A_BYTES);
    }
  };
  auto load_one = [&](int t, int idx) {    // direct load idx of tile t (A's first, then B's)
    char* dst = stage(t);
    if (idx < PER_A) gr_g2lds16(A + (long long)t * BK + la.goff[idx], gr_lds_addr(dst) + idx * NT * 16 + la.lwave);
    else gr_g2lds16(B + (long long)t * b_step + lb.goff[idx - PER_A],
                    gr_lds_addr(dst + G::A_BYTES) + (idx - PER_A) * NT * 16 + lb.lwave);
  };
  auto bfrag = [&](const char* cur, int ks, int i) -> vec8 {
    if constexpr (B_KMAJOR) {
      const int row = wn * G::WN + i * 32 + l32;
      return gr_as<vec8>(gr_ld16(cur + G::A_BYTES + row * (BK * 2) + gr_swz<CPR>(row, 2 * ks + g) * 16));
    } else {
      return gr_tr_frag<T, BN, false>(cur + G::A_BYTES, ks * 16, wn * G::WN + i * 32, lane);
    }
  };
  auto afrag = [&](const char* cur, int ks, int j) -> vec8 {
    const int row = wm * G::WM + j * 32 + l32;
    return gr_as<vec8>(gr_ld16(cur + row * (BK * 2) + gr_swz<CPR>(row, 2 * ks + g) * 16));
  };

  // prologue: the first STAGES tiles in flight, tile 0 published, its first fragments read
#pragma unroll
  for (int s = 0; s < STAGES; ++s) load_tile(s);
  if (nk >= STAGES) gr_wait_vmcnt<(STAGES - 1) * PER_TILE>(); else gr_wait_vmcnt<0>();
  __syncthreads();
  vec8 bt[2][TN], am[2][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i) bt[0][i] = bfrag(stage(0), 0, i);
#pragma unroll
  for (int j = 0; j < TM; ++j) am[0][j] = afrag(stage(0), 0, j);

  // One k step: TN * TM MFMAs from fragment buffer CB. MORE: the next step's
  // fragments (from `nxt`, depth nks) into buffer 1 - CB, one read after each
  // of the first TM + TN MFMAs in the order of their first use (am[0], bt[0],
  // am[1..3], bt[1..TN-1]). LOAD: the direct loads of tile load_t, LPS after
  // each MFMA.
  auto kstep = [&](auto cb_tag, auto more_tag, auto load_tag, const char* nxt, int nks, int load_t) {
    constexpr int CB = decltype(cb_tag)::value, NB = 1 - CB;
    constexpr bool MORE = decltype(more_tag)::value, LOAD = decltype(load_tag)::value;
#pragma unroll
    for (int idx = 0; idx < NMF; ++idx) {
      gr_mfma32_acc(acc[idx >> 2][idx & 3], bt[CB][idx >> 2], am[CB][idx & 3]);
      if constexpr (MORE) {
        if (idx == 0) am[NB][0] = afrag(nxt, nks, 0);
        else if (idx == 1) bt[NB][0] = bfrag(nxt, nks, 0);
        else if (idx < 5) am[NB][idx - 1] = afrag(nxt, nks, idx - 1);
        else if (idx < 4 + TN) bt[NB][idx - 4] = bfrag(nxt, nks, idx - 4);
      }
      if constexpr (LOAD) {
#pragma unroll
        for (int l = 0; l < LPS; ++l)
          if (idx * LPS + l < PER_TILE) load_one(load_t, idx * LPS + l);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // a tile: its first KS - 1 k steps, then (unless it is the last tile) the
  // barrier that publishes tile t + 1 and the last k step, which reads tile
  // t + 1's first fragments and (LOAD) refills this stage with tile t + STAGES
  auto tile = [&](int t, auto load_tag, auto last_tag) {
    constexpr bool LOAD = decltype(load_tag)::value, LASTTILE = decltype(last_tag)::value;
    char* const cur = stage(t);
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) {
      if (ks & 1) kstep(gr_ic<1>{}, gr_ic<1>{}, gr_ic<0>{}, cur, ks + 1, 0);
      else kstep(gr_ic<0>{}, gr_ic<1>{}, gr_ic<0>{}, cur, ks + 1, 0);
    }
    if constexpr (LASTTILE) {
      kstep(gr_ic<(KS - 1) & 1>{}, gr_ic<0>{}, gr_ic<0>{}, cur, 0, 0);
    } else {
      // tile t + 1 must have landed; with LOAD the later tiles up to t + STAGES - 1 stay in flight
      if constexpr (LOAD && STAGES > 2) gr_wait_vmcnt<(STAGES - 2) * PER_TILE>(); else gr_wait_vmcnt<0>();
      // this wave's fragment reads of tile t are done; also a compiler memory fence
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      kstep(gr_ic<(KS - 1) & 1>{}, gr_ic<1>{}, gr_ic<LOAD ? 1 : 0>{}, stage(t + 1), 0, t + STAGES);
    }
  };
  static_assert(KS % 2 == 0, "an even number of k steps per tile keeps the fragment buffers in step");
  int t = 0;
  for (; t + STAGES < nk; ++t) tile(t, gr_ic<1>{}, gr_ic<0>{});
  for (; t + 1 < nk; ++t) tile(t, gr_ic<0>{}, gr_ic<0>{});
  tile(t, gr_ic<0>{}, gr_ic<1>{});

  // the MFMA results before any vector read of the accumulators (the compiler
  // does not count wait states after inline assembly), then every wave past
  // its operand reads before the output tile overwrites the stages
  acc_guard();
  __syncthreads();
  gr_gemm_store_tile<T, BM, BN, TM, TN, NT, EPI>(a, acc, lds, wm * G::WM, wn * G::WN, tm, tn, z, rows_ok, cols_ok);
}

// LDS bytes of the one-wave body: the operand ring or the staged output tile
template <int BK, int BNT = 256>
struct gr_gemm_w4_lds {
  typedef gr_gemm_cfg<256, BNT, BK, 2, 2, gr_gemm_w4_stages<BK>::value> G;
  static constexpr int value = G::LDS;
};

template <class T, bool B_KMAJOR, int EPI, int BK = 64, int BNT = 256>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void gr_gemm_w4_kernel(gr_gemm_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_gemm_w4_body<T, B_KMAJOR, EPI, BK, BNT>(a, gr_lds);
}
