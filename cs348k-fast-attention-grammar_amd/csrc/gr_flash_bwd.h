// gr_flash_bwd.h -- attention backward (dQ, dK, dV) for gfx950 (CDNA4).
//
// Given Q, K, V, O, dO [B, H, N, D] (common strides, unit stride on D) and
// the forward's row log-sum-exp L (natural log of sum_j exp(scale q.k_j)),
// computes dV = P^T dO, dK = scale dS^T Q, dQ = scale dS K with
// P = exp(scale Q K^T - L) [causal mask], dS = P * (dO V^T - delta),
// delta = rowsum(dO * O). Two kernels (the dQ one runs first):
//  * gr_attn_bwd_kernel (dK, dV; gr_attn_bwd128_kernel at d = 128): one
//    workgroup per block of BN keys of one head, one wave per 32 of them. K
//    and V of the wave are MFMA operands held in registers; dK^T and dV^T
//    accumulate in registers (at d = 128 in AGPRs, by inline-assembly MFMAs)
//    over all query tiles. Per tile of BM queries (Q and dO double-buffered in LDS, loaded
//    straight from global memory): S = Q K^T and dP = dO V^T with one key per
//    lane (Q and dO rows read with bits 2 and 3 of the row index swapped, so
//    each half-wave's accumulators hold 8 consecutive queries: they are
//    directly the B operand of dV^T += dO^T P and dK^T += Q^T dS, whose dO^T
//    and Q^T fragments come from transposing LDS reads of the same tiles).
//  * gr_attn_bwd_dq_kernel (dQ): the forward's structure -- one wave per 32
//    queries, Q and dO in registers, K and V tiles streamed through LDS --
//    recomputing S^T = K Q^T and dP^T = V dO^T with one query per lane, then
//    dQ^T += K^T dS^T with K^T read transposed from the K tile. Recomputing
//    the two products costs less here than adding every key block's dQ into
//    an fp32 accumulator with float atomics (which took over half the time).
//    It runs first and also forms delta = rowsum(dO * O) of its queries from
//    the dO fragments it holds, storing it for the dK/dV kernel.
// Causal: a key block meets only the query tiles at or after its first key
// (and a query tile only the key tiles up to its last query); the mask is
// applied on the 32-row blocks that straddle the diagonal (the d = 128 dK/dV
// kernel runs those query tiles first, then the rest with no mask code).
// Outputs are staged through the free LDS and stored as whole rows
// (gr_store_block_t).
#pragma once
#include "gr_flash_fwd.h"

struct gr_attn_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;     // [b*H+h][N], natural log
  float* delta;         // [b*H+h][N]: rowsum(dO * O), written by the dQ kernel
  void* dq;
  void* dk;
  void* dv;
  long long sb, sh, sn;   // strides of all nine [B, H, N, D] tensors
  int B, H, N;
  float scale;
};

// Store a wave's 32 x D block whose transpose sits in MFMA accumulators
// (acc[db] register r: row l32, column db*32 + 8(r/4) + 4g + r%4), times mul,
// as rows of T: staged through this wave's 32*D*2 bytes of free LDS, so the
// global stores are whole 16-byte chunks of consecutive rows (row r at
// dst + r*ld), streamed past the caches (nontemporal).
template <class T, int D>
__device__ __forceinline__ void gr_store_block_t(const gr_f32x16 (&acc)[D / 32], float mul, char* stage, T* dst,
                                                 long long ld, int lane) {
  constexpr int CPR = D / 8;
  const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      gr_u32x2 w;
      w[0] = gr_pack2f<T>(acc[db][4 * rr] * mul, acc[db][4 * rr + 1] * mul);
      w[1] = gr_pack2f<T>(acc[db][4 * rr + 2] * mul, acc[db][4 * rr + 3] * mul);
      *reinterpret_cast<gr_u32x2*>(stage + l32 * (D * 2) + gr_swz<CPR>(l32, db * 4 + rr) * 16 + g * 8) = w;
    }
  __builtin_amdgcn_wave_barrier();   // LDS writes and reads of one wave stay in order
#pragma unroll
  for (int it = 0; it < 32 * CPR / 64; ++it) {
    const int j = it * 64 + lane, row = j / CPR, ch = j % CPR;
    __builtin_nontemporal_store(gr_ld16(stage + row * (D * 2) + gr_swz<CPR>(row, ch) * 16),
                                reinterpret_cast<gr_u32x4*>(dst + (long long)row * ld + ch * 8));
  }
}

// LDS of the dK/dV kernel: two stages of (Q, dO, L, delta) tiles.
template <int D, int BM, int BN>
struct gr_attn_bwd_lds {
  static constexpr int QT = BM * D * 2;          // one Q or dO tile
  static constexpr int STAGE = 2 * QT + 2 * BM * 4;   // Q, dO, then log2-domain L and delta
  static constexpr int RING = 2 * STAGE;
  static constexpr int BYTES = RING;
};

// dK^T / dV^T += A B with the accumulator pinned in AGPRs (the d = 128
// kernel: its score and dP accumulators, read by the vector ALU, stay in
// VGPRs). The compiler counts no wait states into inline assembly: s_nop 1
// covers the two the MFMA needs after a vector write of its A / B operands,
// which the packing of P and dS has just done.
template <class T>
__device__ __forceinline__ void gr_bwd_mfma_agpr(gr_f32x16& acc, typename gr_mfma<T>::vec8 a,
                                                 typename gr_mfma<T>::vec8 b) {
  if constexpr (gr_is_same<T, _Float16>::value)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// PRE (fp16 with scale log2(e) <= 1, K held in registers): K pre-scaled by
// c = scale log2(e) (one more fp16 rounding, relative 2^-11) so that S comes
// out in log2 units, and the S accumulators start from the queries' -L
// log2(e): p = 2^S with no vector multiply-add per score. The dP
// accumulators always start from -delta, so dS = p dP. Both statistics sit
// negated in LDS and are read straight into the accumulators.
template <class T, int D, int BM, int BN, bool CAUSAL, bool PRE = false>
__global__ __launch_bounds__(BN / 32 * 64) __attribute__((amdgpu_waves_per_eu(2)))
void gr_attn_bwd_kernel(gr_attn_bwd_args a) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int NW = BN / 32, NT = NW * 64;
  constexpr int DS = D / 16, DB = D / 32, QJ = BM / 32;
  typedef gr_attn_bwd_lds<D, BM, BN> L;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && D == 64, "tile shape (d = 128: gr_attn_bwd128_kernel)");
  static_assert(2 * BM <= NT, "one thread per statistic of a query tile");
  extern __shared__ __attribute__((aligned(16))) char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nkb = a.N / BN;
  int bh, kb;                                   // causal: key block 0 has the most queries
  if constexpr (CAUSAL) {
    gr_causal_order((int)blockIdx.x, (int)gridDim.x, nkb, bh, kb);
  } else {
    const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    bh = logical / nkb;
    kb = logical % nkb;
  }
  const long long base = (bh / a.H) * a.sb + (bh % a.H) * a.sh;
  const T* Q = static_cast<const T*>(a.q) + base;
  const T* K = static_cast<const T*>(a.k) + base;
  const T* V = static_cast<const T*>(a.v) + base;
  const T* dO = static_cast<const T*>(a.dout) + base;
  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32;
  const float c = a.scale * 1.4426950408889634f;

  // this wave's 32 keys as MFMA B operands (8 consecutive d per lane)
  vec8 kf[DS], vf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    kf[ds] = gr_as<vec8>(gr_ld16(K + (long long)(kw0 + l32) * a.sn + ds * 16 + 8 * g));
    vf[ds] = gr_as<vec8>(gr_ld16(V + (long long)(kw0 + l32) * a.sn + ds * 16 + 8 * g));
  }
  if constexpr (PRE) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[ds][e] = (T)((float)kf[ds][e] * c);
  }
  gr_f32x16 dkt[DB], dvt[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkt[db] = (gr_f32x16)(0.f);
    dvt[db] = (gr_f32x16)(0.f);
  }

  gr_lds_loader<T, BM, D, NT, false, false, true> ql;   // Q / dO tiles: row reads and transposing reads
  ql.init(tid, a.sn);
  const int qt0 = CAUSAL ? key0 / BM : 0;
  const int nqt = a.N / BM;
  auto load_tile = [&](int qt, int st) {
    char* s = lds + st * L::STAGE;
    ql.load(Q + (long long)qt * BM * a.sn, s);
    ql.load(dO + (long long)qt * BM * a.sn, s + L::QT);
    float* stat = reinterpret_cast<float*>(s + 2 * L::QT);
    const long long r0 = (long long)bh * a.N + (long long)qt * BM;
    if (tid < BM) stat[tid] = a.lse[r0 + tid] * -1.4426950408889634f;
    else if (tid < 2 * BM) stat[tid] = -a.delta[r0 + tid - BM];
  };
  load_tile(qt0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int qt = qt0; qt < nqt; ++qt) {
    const int st = (qt - qt0) & 1;
    // the other stage was last read before the previous iteration's closing barrier
    if (qt + 1 < nqt) load_tile(qt + 1, st ^ 1);
    const char* qs = lds + st * L::STAGE;
    const char* dos = qs + L::QT;
    const float* nlse2 = reinterpret_cast<const float*>(qs + 2 * L::QT);   // -L log2(e)
    const float* ndlt = nlse2 + BM;                                          // -delta
    const int q0 = qt * BM;

    vec8 pb[QJ][2], dsb[QJ][2];
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      // S and dP for queries j*32..+32 (row permuted) and this wave's keys,
      // from the queries' statistics (register r: query j*32 + 16(r/8) + 8g + r%8)
      gr_f32x16 sa, dpa;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql_ = j * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
        sa[r] = PRE ? nlse2[ql_] : 0.f;
        dpa[r] = ndlt[ql_];
      }
      const int row = j * 32 + gr_perm32(l32);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const int ch = gr_swz_rt<D / 8>(row, 2 * ds + g);
        const vec8 qa = gr_as<vec8>(gr_ld16(qs + row * (D * 2) + ch * 16));
        const vec8 da = gr_as<vec8>(gr_ld16(dos + row * (D * 2) + ch * 16));
        sa = MF::mma32(qa, kf[ds], sa);
        dpa = MF::mma32(da, vf[ds], dpa);
      }
      // register r holds query j*32 + 8g + r (r < 8) or j*32 + 16 + 8g + r - 8.
      // Causal: only a block whose queries start below the wave's last key
      // is masked (a wave-uniform branch; p = 2^-inf = 0 where key > query).
      if (CAUSAL && kw0 + 31 > q0 + j * 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kw0 + l32 > q0 + j * 32 + 16 * (r >> 3) + 8 * g + (r & 7)) sa[r] = -GR_INF;
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        gr_u32x4 pw, dw;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float p2[2], d2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int r = 8 * hf + e + u;
            const int ql_ = j * 32 + 16 * hf + 8 * g + e + u;
            const float p = PRE ? gr_exp2(sa[r]) : gr_exp2(fmaf(sa[r], c, nlse2[ql_]));
            p2[u] = p;
            d2[u] = p * dpa[r];
          }
          pw[e >> 1] = gr_pack2f<T>(p2[0], p2[1]);
          dw[e >> 1] = gr_pack2f<T>(d2[0], d2[1]);
        }
        pb[j][hf] = gr_as<vec8>(pw);
        dsb[j][hf] = gr_as<vec8>(dw);
      }
      // dV^T += dO^T P and dK^T += Q^T dS over these 32 queries (2 MFMA k-steps)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const vec8 dot = gr_tr_frag<T, D, false, true>(dos, j * 32 + 16 * hf, db * 32, lane);
          const vec8 qtr = gr_tr_frag<T, D, false, true>(qs, j * 32 + 16 * hf, db * 32, lane);
          dvt[db] = MF::mma32(dot, pb[j][hf], dvt[db]);
          dkt[db] = MF::mma32(qtr, dsb[j][hf], dkt[db]);
        }
    }
    // the backend's interleaving of LDS reads and MFMAs for this region
    // (dK/dV at C2: 36.0 against 37.3-37.6 us)
    __builtin_amdgcn_iglp_opt(0);
    __builtin_amdgcn_s_waitcnt(0);   // the next stage has landed
    __syncthreads();
  }

  // dK = scale dK^T^T, dV = dV^T^T for keys kw0.. (the LDS stages are free
  // after the last tile's barrier: 2 * 32 * D * 2 bytes per wave)
  static_assert(NW * 2 * 32 * D * 2 <= L::BYTES, "dK/dV staging fits the LDS stages");
  char* const stage = lds + wave * (2 * 32 * D * 2);
  gr_store_block_t<T, D>(dkt, a.scale, stage, static_cast<T*>(a.dk) + base + (long long)kw0 * a.sn, a.sn, lane);
  gr_store_block_t<T, D>(dvt, 1.0f, stage + 32 * D * 2, static_cast<T*>(a.dv) + base + (long long)kw0 * a.sn, a.sn,
                         lane);
}

// The d = 128 dK/dV kernel: gr_attn_bwd_kernel's math on one wave per SIMD,
// K and V of the wave in registers, dK^T and dV^T in AGPRs by inline-assembly
// MFMAs (gr_bwd_mfma_agpr) while the S and dP accumulators stay in VGPRs for
// the vector ALU (this unit is compiled with VGPR-form MFMAs). The tile body
// is one lambda run first on the query tiles that straddle the diagonal, with
// the mask, then on the rest, whose schedule the backend interleaves
// (iglp_opt). At C3 (B2 H32 N4096 causal bf16) the kernel took 616 against
// 653-667 us for the same math with K and V read from LDS, the accumulators
// in VGPRs and the mask test in every tile; at N = 4,096 non-causal 1,120
// against 1,372 us. (The d = 64 kernel keeps its plain loop: as a lambda its
// body took 22 more VGPRs and ran 1 % slower at C2.)
template <class T, int BM, int BN, bool CAUSAL, bool PRE = false>
__global__ __launch_bounds__(BN / 32 * 64) __attribute__((amdgpu_waves_per_eu(1)))
void gr_attn_bwd128_kernel(gr_attn_bwd_args a) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int D = 128;
  constexpr int NW = BN / 32, NT = NW * 64;
  constexpr int DS = D / 16, DB = D / 32, QJ = BM / 32;
  typedef gr_attn_bwd_lds<D, BM, BN> L;
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert(2 * BM <= NT, "one thread per statistic of a query tile");
  extern __shared__ __attribute__((aligned(16))) char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nkb = a.N / BN;
  int bh, kb;                                   // causal: key block 0 has the most queries
  if constexpr (CAUSAL) {
    gr_causal_order((int)blockIdx.x, (int)gridDim.x, nkb, bh, kb);
  } else {
    const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    bh = logical / nkb;
    kb = logical % nkb;
  }
  const long long base = (bh / a.H) * a.sb + (bh % a.H) * a.sh;
  const T* Q = static_cast<const T*>(a.q) + base;
  const T* K = static_cast<const T*>(a.k) + base;
  const T* V = static_cast<const T*>(a.v) + base;
  const T* dO = static_cast<const T*>(a.dout) + base;
  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32;
  const float c = a.scale * 1.4426950408889634f;

  // this wave's 32 keys as MFMA B operands (8 consecutive d per lane)
  vec8 kf[DS], vf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    kf[ds] = gr_as<vec8>(gr_ld16(K + (long long)(kw0 + l32) * a.sn + ds * 16 + 8 * g));
    vf[ds] = gr_as<vec8>(gr_ld16(V + (long long)(kw0 + l32) * a.sn + ds * 16 + 8 * g));
  }
  if constexpr (PRE) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[ds][e] = (T)((float)kf[ds][e] * c);
  }
  gr_f32x16 dkt[DB], dvt[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkt[db] = (gr_f32x16)(0.f);
    dvt[db] = (gr_f32x16)(0.f);
  }
  // the vector writes of the accumulators (zeroing) retire before the first
  // MFMA reads them, and the MFMA results before the epilogue reads them: the
  // compiler counts no wait states across inline assembly
  auto acc_guard = [&]() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                   : "+a"(dkt[0]), "+a"(dkt[1]), "+a"(dkt[2]), "+a"(dkt[3]), "+a"(dvt[0]), "+a"(dvt[1]),
                     "+a"(dvt[2]), "+a"(dvt[3]));
  };
  acc_guard();

  gr_lds_loader<T, BM, D, NT, false, false, true> ql;   // Q / dO tiles: row reads and transposing reads
  ql.init(tid, a.sn);
  const int qt0 = CAUSAL ? key0 / BM : 0;
  const int nqt = a.N / BM;
  auto load_tile = [&](int qt, int st) {
    char* s = lds + st * L::STAGE;
    ql.load(Q + (long long)qt * BM * a.sn, s);
    ql.load(dO + (long long)qt * BM * a.sn, s + L::QT);
    float* stat = reinterpret_cast<float*>(s + 2 * L::QT);
    const long long r0 = (long long)bh * a.N + (long long)qt * BM;
    if (tid < BM) stat[tid] = a.lse[r0 + tid] * -1.4426950408889634f;
    else if (tid < 2 * BM) stat[tid] = -a.delta[r0 + tid - BM];
  };
  load_tile(qt0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // one query tile; MASK: the tile straddles the diagonal (causal)
  auto tile = [&](int qt, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value != 0;
    const int st = (qt - qt0) & 1;
    // the other stage was last read before the previous tile's closing barrier
    if (qt + 1 < nqt) load_tile(qt + 1, st ^ 1);
    const char* qs = lds + st * L::STAGE;
    const char* dos = qs + L::QT;
    const float* nlse2 = reinterpret_cast<const float*>(qs + 2 * L::QT);   // -L log2(e)
    const float* ndlt = nlse2 + BM;                                          // -delta
    const int q0 = qt * BM;

    vec8 pb[QJ][2], dsb[QJ][2];
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      // S and dP for queries j*32..+32 (row permuted) and this wave's keys,
      // from the queries' statistics (register r: query j*32 + 16(r/8) + 8g + r%8)
      gr_f32x16 sa, dpa;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql_ = j * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
        sa[r] = PRE ? nlse2[ql_] : 0.f;
        dpa[r] = ndlt[ql_];
      }
      const int row = j * 32 + gr_perm32(l32);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const int ch = gr_swz_rt<D / 8>(row, 2 * ds + g);
        const vec8 qa = gr_as<vec8>(gr_ld16(qs + row * (D * 2) + ch * 16));
        const vec8 da = gr_as<vec8>(gr_ld16(dos + row * (D * 2) + ch * 16));
        sa = MF::mma32(qa, kf[ds], sa);
        dpa = MF::mma32(da, vf[ds], dpa);
      }
      // register r holds query j*32 + 8g + r (r < 8) or j*32 + 16 + 8g + r - 8.
      // Only a block whose queries start below the wave's last key is masked
      // (a wave-uniform branch; p = 2^-inf = 0 where key > query).
      if (MASK && kw0 + 31 > q0 + j * 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kw0 + l32 > q0 + j * 32 + 16 * (r >> 3) + 8 * g + (r & 7)) sa[r] = -GR_INF;
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        gr_u32x4 pw, dw;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float p2[2], d2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int r = 8 * hf + e + u;
            const int ql_ = j * 32 + 16 * hf + 8 * g + e + u;
            const float p = PRE ? gr_exp2(sa[r]) : gr_exp2(fmaf(sa[r], c, nlse2[ql_]));
            p2[u] = p;
            d2[u] = p * dpa[r];
          }
          pw[e >> 1] = gr_pack2f<T>(p2[0], p2[1]);
          dw[e >> 1] = gr_pack2f<T>(d2[0], d2[1]);
        }
        pb[j][hf] = gr_as<vec8>(pw);
        dsb[j][hf] = gr_as<vec8>(dw);
      }
      // dV^T += dO^T P and dK^T += Q^T dS over these 32 queries (2 MFMA k-steps)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const vec8 dot = gr_tr_frag<T, D, false, true>(dos, j * 32 + 16 * hf, db * 32, lane);
          const vec8 qtr = gr_tr_frag<T, D, false, true>(qs, j * 32 + 16 * hf, db * 32, lane);
          gr_bwd_mfma_agpr<T>(dvt[db], dot, pb[j][hf]);
          gr_bwd_mfma_agpr<T>(dkt[db], qtr, dsb[j][hf]);
        }
    }
    // the backend's interleaving of LDS reads and MFMAs for the unmasked
    // tiles (N = 4,096 non-causal: 1.12 against 1.22 ms)
    if constexpr (!MASK) __builtin_amdgcn_iglp_opt(0);
    __builtin_amdgcn_s_waitcnt(0);   // the next stage has landed
    __syncthreads();
  };
  // causal: the query tiles that straddle this block's keys first, then the
  // rest without the mask code
  int qt = qt0;
  if constexpr (CAUSAL) {
    const int qd = (key0 + BN - 1) / BM + 1 < nqt ? (key0 + BN - 1) / BM + 1 : nqt;
    for (; qt < qd; ++qt) tile(qt, gr_ic<1>{});
  }
  for (; qt < nqt; ++qt) tile(qt, gr_ic<0>{});
  acc_guard();

  // dK = scale dK^T^T, dV = dV^T^T for keys kw0.. (the LDS stages are free
  // after the last tile's barrier: 2 * 32 * D * 2 bytes per wave)
  static_assert(NW * 2 * 32 * D * 2 <= L::BYTES, "dK/dV staging fits the LDS stages");
  char* const stage = lds + wave * (2 * 32 * D * 2);
  gr_store_block_t<T, D>(dkt, a.scale, stage, static_cast<T*>(a.dk) + base + (long long)kw0 * a.sn, a.sn, lane);
  gr_store_block_t<T, D>(dvt, 1.0f, stage + 32 * D * 2, static_cast<T*>(a.dv) + base + (long long)kw0 * a.sn, a.sn,
                         lane);
}

template <int D, int BN>
struct gr_attn_bwd_dq_lds {
  static constexpr int TILE = BN * D * 2;
  static constexpr int BYTES = 2 * 2 * TILE;   // two stages of K and V
};

// dQ: one workgroup per NW*32 queries of one head, one wave per 32 (one query
// per lane); key tiles of BN stream through LDS with their rows stored in the
// gr_perm32 order, which makes each half-wave's S^T / dP^T accumulators 8
// consecutive keys -- the B operand of dQ^T += K^T dS^T.
// PRE (fp16 with scale log2(e) <= 1): Q pre-scaled by c = scale log2(e) in
// registers (one more fp16 rounding, relative 2^-11) so that S^T comes out in
// log2 units, and the S^T accumulators start from -L log2(e): p = 2^S^T with
// no vector multiply-add per score. The dP^T accumulators always start from
// -delta, so dS = p dP^T.
template <class T, int D, int NW, int BN, bool CAUSAL, bool PRE = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
void gr_attn_bwd_dq_kernel(gr_attn_bwd_args a) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int BM = NW * 32, NT = NW * 64;
  constexpr int KB = BN / 32, DS = D / 16, DB = D / 32;
  typedef gr_attn_bwd_dq_lds<D, BN> L;
  extern __shared__ __attribute__((aligned(16))) char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nqt = a.N / BM;
  int bh, qt;
  if constexpr (CAUSAL) {
    gr_causal_order((int)blockIdx.x, (int)gridDim.x, nqt, bh, qt);
    qt = nqt - 1 - qt;                        // the longest query tiles first
  } else {
    const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    bh = logical / nqt;
    qt = logical % nqt;
  }
  const long long base = (bh / a.H) * a.sb + (bh % a.H) * a.sh;
  const T* Q = static_cast<const T*>(a.q) + base;
  const T* K = static_cast<const T*>(a.k) + base;
  const T* V = static_cast<const T*>(a.v) + base;
  const T* dO = static_cast<const T*>(a.dout) + base;
  const int q0 = qt * BM;
  const int qw = q0 + wave * 32;
  const int myq = qw + l32;
  const float c = a.scale * 1.4426950408889634f;

  vec8 qf[DS], df[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    qf[ds] = gr_as<vec8>(gr_ld16(Q + (long long)myq * a.sn + ds * 16 + 8 * g));
    df[ds] = gr_as<vec8>(gr_ld16(dO + (long long)myq * a.sn + ds * 16 + 8 * g));
  }
  const float lse2 = a.lse[(long long)bh * a.N + myq] * 1.4426950408889634f;
  // delta of this lane's query: its half of the row (d = ds*16 + 8g + e), then
  // the other half from lane ^ 32
  float dlt = 0.f;
  {
    const T* O = static_cast<const T*>(a.o) + base + (long long)myq * a.sn;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const vec8 ov = gr_as<vec8>(gr_ld16(O + ds * 16 + 8 * g));
#pragma unroll
      for (int e = 0; e < 8; ++e) dlt = fmaf((float)ov[e], (float)df[ds][e], dlt);
    }
    dlt += gr_xor32(dlt);
    if (g == 0) a.delta[(long long)bh * a.N + myq] = dlt;
  }
  if constexpr (PRE) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ds][e] = (T)((float)qf[ds][e] * c);
  }
  // the accumulators' starting values: this lane's query's -L log2(e) (PRE)
  // and -delta, the same in all 16 registers
  const gr_f32x16 s_init = (gr_f32x16)(PRE ? -lse2 : 0.f), dp_init = (gr_f32x16)(-dlt);
  gr_f32x16 dqt[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqt[db] = (gr_f32x16)(0.f);

  gr_lds_loader<T, BN, D, NT, false, true, true> kl;   // rows in gr_perm32 order, gr_swz_rt
  kl.init(tid, a.sn);
  const int ntile = CAUSAL ? (q0 + BM + BN - 1) / BN : a.N / BN;
  auto load_tile = [&](int t, int st) {
    char* s = lds + st * 2 * L::TILE;
    kl.load(K + (long long)t * BN * a.sn, s);
    kl.load(V + (long long)t * BN * a.sn, s + L::TILE);
  };
  load_tile(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int t = 0; t < ntile; ++t) {
    const int st = t & 1;
    if (t + 1 < ntile) load_tile(t + 1, st ^ 1);
    const char* ks = lds + st * 2 * L::TILE;
    const char* vs = ks + L::TILE;
    const int k0 = t * BN;
    if (!CAUSAL || k0 <= qw + 31) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        // S^T and dP^T for keys kb*32.. (LDS rows kb*32 + l32) against this lane's query
        gr_f32x16 sa = s_init, dpa = dp_init;
        const int row = kb * 32 + l32;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          const int ch = gr_swz_rt<D / 8>(row, 2 * ds + g);
          sa = MF::mma32(gr_as<vec8>(gr_ld16(ks + row * (D * 2) + ch * 16)), qf[ds], sa);
          dpa = MF::mma32(gr_as<vec8>(gr_ld16(vs + row * (D * 2) + ch * 16)), df[ds], dpa);
        }
        // register r: key k0 + kb*32 + 8g + r (r < 8) or + 16 + 8g + r - 8;
        // causal: only a key block that reaches past the wave's first query
        // is masked (wave-uniform branch)
        if (CAUSAL && k0 + kb * 32 + 31 > qw) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (k0 + kb * 32 + 16 * (r >> 3) + 8 * g + (r & 7) > myq) sa[r] = -GR_INF;
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          gr_u32x4 dw;
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            float d2[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int r = 8 * hf + e + u;
              const float p = PRE ? gr_exp2(sa[r]) : gr_exp2(fmaf(sa[r], c, -lse2));
              d2[u] = p * dpa[r];
            }
            dw[e >> 1] = gr_pack2f<T>(d2[0], d2[1]);
          }
          const vec8 dsb = gr_as<vec8>(dw);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const vec8 kt = gr_tr_frag<T, D, false, true, true>(ks, kb * 32 + 16 * hf, db * 32, lane);
            dqt[db] = MF::mma32(kt, dsb, dqt[db]);
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);   // the next stage has landed
    __syncthreads();
  }

  // dQ = scale dQ^T^T for queries qw.. (staged in the free LDS stages)
  static_assert(NW * 32 * D * 2 <= L::BYTES, "dQ staging fits the LDS stages");
  gr_store_block_t<T, D>(dqt, a.scale, lds + wave * (32 * D * 2), static_cast<T*>(a.dq) + base + (long long)qw * a.sn,
                         a.sn, lane);
}
