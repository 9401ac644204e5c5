// gr_flash_fwd.h -- tiled flash-style attention forward for gfx950 (CDNA4).
//
// Computes O = softmax(scale * Q K^T [+ causal mask]) V for Q/K/V/O laid out as
// [B, H, N, D] with arbitrary batch/head/sequence strides (unit stride on D).
// K may instead be given transposed (KT [B, H, D, N]), which is the layout the
// reference grammar's attention program reads (run_attention_search.py:82-84).
//
// Design (one workgroup = NW waves = BM = NW*QB*32 queries of one head):
//  * Both contractions run on the 32x32x16 MFMA with the *transposed*
//    formulation S^T = K Q^T and O^T = V^T P^T. The accumulator layout then
//    gives every lane a single query column, so the online-softmax row max,
//    rescale and row sum are lane-local; only the max needs one exchange with
//    the lane 32 positions away per key tile, and the row sum is combined once
//    at the end.
//  * K rows are written to LDS with bits 2 and 3 of the row swapped, which
//    makes the S^T accumulators of each half-wave hold 8 *consecutive* keys;
//    those registers are then exactly the B operand of the P*V MFMA, and V^T
//    can be read with one 16-byte LDS load per MFMA.
//  * Q stays in registers for the whole kernel. K and V tiles are double
//    buffered in LDS (one barrier per key tile) and prefetched one tile
//    ahead: with DIRECT straight from global memory into LDS
//    (global_load_lds_dwordx4), else through registers. 16-byte LDS chunks
//    are XOR-swizzled by row so both the tile writes and the MFMA operand
//    reads are bank-conflict free.
//  * With TR (the default in every launch path) V, and K when it comes
//    transposed (KT), are copied into LDS as laid out in memory and the MFMA
//    fragments are read back with gfx950's transposing LDS read, so no tile is
//    transposed in registers on its way in.
//  * Causal: key tiles past the block's last query are never visited; waves
//    whose queries all precede a tile skip its math; the mask is applied only
//    on diagonal tiles. Heavy query tiles are scheduled first.
//  * Workgroups of one head are mapped to one XCD so K/V are shared in its L2.
//  * Nq (queries) may differ from N (keys) for non-causal launches (decode
//    shapes): query rows past Nq are computed from a copy of the last row and
//    not stored. SPLIT: the workgroups of a query tile split the keys and
//    leave partial results that a second kernel merges.
#pragma once
#include "gr_common.h"

struct gr_attn_args {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  long long q_sb, q_sh, q_sn;
  long long k_sb, k_sh, k_sn;   // for KT layout: k_sn is the stride of the D axis
  long long v_sb, v_sh, v_sn;
  long long o_sb, o_sh, o_sn;
  int B, H, N;                  // N: keys
  int Nq;                       // queries (== N unless a decode-shape launch)
  float scale_log2;             // softmax scale * log2(e)
  // key-split launches (SPLIT): blockIdx.y = s takes keys [s*kchunk, (s+1)*kchunk)
  // and writes its unnormalised partial O [s][b*H+h][q][D] and (m, l)
  // [s][b*H+h][q] in fp32 for gr_attn_combine_kernel
  int kchunk = 0;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  // training forward: the row log-sum-exp of the scaled scores (natural log),
  // [b*H+h][q] fp32, kept for the backward pass; nullptr = not written
  float* lse = nullptr;
};

// The online softmax moves its exponent base only when a row's max grows by
// more than this many powers of two (p then stays <= 2^8, exact in fp16/bf16).
#ifndef GR_RESCALE_LOG2
#define GR_RESCALE_LOG2 8.0f
#endif

// GR_FLASH_OPT (on unless built with -DGR_FLASH_OPT=0; the pipelined and
// register-transposing variants always take the max pass): after the first
// key tile P is computed with the current base and no max pass; only when
// some p overflowed the P type (the row max grew by more than ~16 powers of
// two in fp16) is the tile redone with the max pass and a rescale. Q is
// pre-scaled by scale log2(e) and the score MFMAs start from -base, so p is
// one exp2 of the accumulator. The score MFMAs of a tile then need not all
// finish before its first exponentials, and ~100 VALU instructions per
// 128-key tile and wave drop out.
#ifndef GR_FLASH_OPT
#define GR_FLASH_OPT 1
#endif

template <int V> struct gr_ic { static constexpr int value = V; };
template <bool C, class X, class Y> struct gr_cond { typedef X type; };
template <class X, class Y> struct gr_cond<false, X, Y> { typedef Y type; };
template <class X, class Y> struct gr_is_same { static constexpr bool value = false; };
template <class X> struct gr_is_same<X, X> { static constexpr bool value = true; };

// Swap bits 2 and 3 of a row index inside a 32-row MFMA block.
__device__ __forceinline__ int gr_perm32(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// XOR swizzle of the 16-byte chunk index inside an LDS row of CPR chunks.
// A 16-byte LDS access by a wavefront is served 8 lanes (32 banks) or 16 lanes
// (64 banks) at a time; the MFMA operand reads put consecutive rows of an
// aligned 16-row group on consecutive lanes, all at the same logical chunk.
// Each mapping below gives those rows distinct bank groups under both bank
// counts, and is a bit-linear (XOR) function of the row.
template <int CPR>
__device__ __forceinline__ int gr_swz(int row, int chunk) {
  if constexpr (CPR >= 16) return chunk ^ (row & 15);                         // 256+ B rows
  else if constexpr (CPR == 8) return chunk ^ ((row ^ (row >> 3)) & 7);       // 128 B rows
  else if constexpr (CPR == 4) return chunk ^ (((row >> 1) ^ (row >> 3)) & 3);  // 64 B rows
  else if constexpr (CPR == 2) return chunk ^ (((row >> 2) ^ (row >> 3)) & 1);  // 32 B rows
  else return chunk;
}

// Swizzle of tiles that are read back only through gr_tr_frag (transposing
// reads): a fragment read touches 4 consecutive rows x 4 consecutive 16-byte
// chunks per half-wave, and these XOR patterns put those 16 chunks on 16
// distinct 4-bank groups for every row length; the 16-byte tile writes of a
// row (or of two 128-byte rows) stay conflict free as well.
template <int CPR>
__device__ __forceinline__ int gr_swz_tr(int row, int chunk) {
  if constexpr (CPR >= 16) return chunk ^ ((row & 3) << 2);
  else if constexpr (CPR == 8) return chunk ^ (((row >> 1) & 1) << 2);
  else return chunk;
}

// Swizzle of tiles read both ways: by 16-byte row reads (16 consecutive rows,
// one chunk) and by gr_tr_frag (4 consecutive rows x 4 consecutive chunks per
// 32 lanes). With 64 four-byte banks both touch 16 distinct 16-byte bank
// groups: h(row) is a bijection of the row's low four bits (bits 1-3 at
// 128-byte rows, where bit 0 already selects the half of the banks), and its
// top two bits differ between the four rows of an aligned group (bit 2 for
// the two rows of equal parity at 128-byte rows).
template <int CPR>
__device__ __forceinline__ int gr_swz_rt(int row, int chunk) {
  if constexpr (CPR >= 16) return chunk ^ (((row & 3) << 2) | ((row >> 2) & 3));     // 256+ B rows
  else if constexpr (CPR == 8) return chunk ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));  // 128 B rows
  else return gr_swz<CPR>(row, chunk);
}

// Global [ROWS][COLS] tile (row stride ld elements) -> LDS rows, same shape.
// Per-thread global and LDS offsets are computed once (init) and reused for
// every tile, so the main loop spends no VALU on address arithmetic. TRSWZ
// selects the swizzle of tiles read through gr_tr_frag.
template <class T, int ROWS, int COLS, int NT, bool PERM, bool TRSWZ = false>
struct gr_row_loader {
  static constexpr int CPR = COLS / 8;
  static constexpr int CHUNKS = ROWS * CPR;
  static constexpr int PER = (CHUNKS + NT - 1) / NT;
  gr_u32x4 r[PER];
  int goff[PER];
  int loff[PER];
  __device__ __forceinline__ void init(int tid, long long ld) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, cc = c % CPR;
      const int prow = PERM ? gr_perm32(row) : row;
      goff[i] = (int)(row * ld) + cc * 8;
      loff[i] = prow * (COLS * 2) + (TRSWZ ? gr_swz_tr<CPR>(prow, cc) : gr_swz<CPR>(prow, cc)) * 16;
    }
  }
  __device__ __forceinline__ bool live(int i, int tid) const { return CHUNKS % NT == 0 || tid + i * NT < CHUNKS; }
  __device__ __forceinline__ void gload(const T* src, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (live(i, tid)) r[i] = gr_ld16(src + goff[i]);
  }
  __device__ __forceinline__ void sstore(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (live(i, tid)) gr_st16(dst + loff[i], r[i]);
  }
};

// Global [ROWS][COLS] tile -> LDS rows, same shape and swizzle as
// gr_row_loader, but loaded straight into LDS (gfx950 global_load_lds_dwordx4):
// no staging registers and no LDS write instructions. Each such load writes
// its 64 lanes' 16-byte chunks to 1 KiB of LDS at a wave-uniform base, lane l
// at base + 16 l, so the swizzle is applied on the global side: the lane that
// lands on LDS slot (row, physical chunk) fetches logical chunk swz(row,
// physical chunk) (the XOR swizzles are involutions); with PERM, LDS row r
// holds global row gr_perm32(r) (also an involution). RTSWZ: gr_swz_rt
// instead of gr_swz / gr_swz_tr. The data is in LDS once the wave's vmcnt
// drains; callers wait on it before the publishing barrier.
template <class T, int ROWS, int COLS, int NT, bool TRSWZ = false, bool PERM = false, bool RTSWZ = false>
struct gr_lds_loader {
  static constexpr int CPR = COLS / 8;
  static constexpr int CHUNKS = ROWS * CPR;
  static constexpr int PER = (CHUNKS + NT - 1) / NT;
  int goff[PER];
  unsigned int lwave;   // wave-uniform
  // rows_valid / chunks_valid (edge tiles): source rows and 16-byte chunks
  // past them are read from the last valid one instead (the LDS tile is full,
  // its extra rows / columns hold copies that the caller never stores).
  __device__ __forceinline__ void init(int tid, long long ld, int rows_valid = ROWS, int chunks_valid = CPR) {
    lwave = __builtin_amdgcn_readfirstlane((tid >> 6) * 64 * 16);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, pc = c % CPR;
      const int lc = RTSWZ ? gr_swz_rt<CPR>(row, pc) : TRSWZ ? gr_swz_tr<CPR>(row, pc) : gr_swz<CPR>(row, pc);
      const int srow = PERM ? gr_perm32(row) : row;
      goff[i] = (int)((srow < rows_valid ? srow : rows_valid - 1) * ld) + (lc < chunks_valid ? lc : chunks_valid - 1) * 8;
    }
  }
  __device__ __forceinline__ void load(const T* src, char* dst) const {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (CHUNKS % NT == 0 || (int)threadIdx.x + i * NT < CHUNKS)   // idle lanes write nothing
        gr_g2lds16(src + goff[i], gr_lds_addr(dst) + i * NT * 16 + lwave);
  }
};

// Global [SR][SC] tile (row stride ld) -> LDS [SC][SR] (transposed). Each unit
// takes two source rows x 8 columns and writes 8 dwords, each holding the pair
// of source-row values for one destination row.
//
// LDS address of (destination row, source-row pair p): row * SR*2 | chunk*16 |
// (p & 3)*4 with chunk = (p >> 2) ^ h(row) -- three bit-disjoint fields that are
// linear over GF(2) in the bits of (unit, e). Hence addr(unit, e) =
// addr(unit, 0) ^ addr(0, e): one base register per unit and a compile-time
// constant per destination row e.
template <class T, int SR, int SC, int NT, bool PERM>
struct gr_tr_loader {
  static constexpr int PAIRS = SR / 2;
  static constexpr int SCPR = SC / 8;
  static constexpr int UNITS = PAIRS * SCPR;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int DCPR = SR / 8;
  static_assert((SR & (SR - 1)) == 0 && SR >= 16, "SR must be a power of two");
  gr_u32x4 r0[PER], r1[PER];
  int goff[PER];
  int ld1;
  int lbase[PER];
  static __device__ __forceinline__ int addr(int drow, int p) {
    const int prow = PERM ? gr_perm32(drow) : drow;
    return prow * (SR * 2) + gr_swz<DCPR>(prow, p >> 2) * 16 + (p & 3) * 4;
  }
  __device__ __forceinline__ void init(int tid, long long ld) {
    ld1 = (int)ld;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      const int p = u % PAIRS, cc = u / PAIRS;
      goff[i] = (int)(2 * p * ld) + cc * 8;
      lbase[i] = addr(cc * 8, p);
    }
  }
  __device__ __forceinline__ bool live(int i, int tid) const { return UNITS % NT == 0 || tid + i * NT < UNITS; }
  __device__ __forceinline__ void gload(const T* src, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (live(i, tid)) {
        r0[i] = gr_ld16(src + goff[i]);
        r1[i] = gr_ld16(src + goff[i] + ld1);
      }
  }
  __device__ __forceinline__ void sstore(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (live(i, tid)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const unsigned int w0 = r0[i][e >> 1], w1 = r1[i][e >> 1];
          const unsigned int w = (e & 1) ? __builtin_amdgcn_perm(w1, w0, 0x07060302u)
                                         : __builtin_amdgcn_perm(w1, w0, 0x05040100u);
          *reinterpret_cast<unsigned int*>(dst + (lbase[i] ^ addr(e, 0))) = w;
        }
      }
  }
};

// MFMA operand fragment (8 consecutive k for one m/n per lane, as the 16-byte
// reads of k-contiguous tiles give) from an LDS tile laid out the other way:
// [K rows][COLS] with the m/n index contiguous, swizzled by gr_swz_tr. Two
// gfx950 transposing reads (ds_read_b64_tr_b16): within each 16-lane group,
// lane 4a+b receives element b of the 4-element vectors addressed by lanes
// a, a+4, a+8, a+12. Lane l addresses row k0 + 8(l/32) + 4h + (l/4)%4 and
// column n0 + 16((l/16)%2) + 4c, so that it receives rows k0 + 8(l/32) +
// 4h + 0..3 of column n0 + perm(l%32), where c = l%4 (PERM: its two bits
// swapped, i.e. column bits 2 and 3 swapped, as gr_perm32 does to K rows).
// RTSWZ: the tile is swizzled with gr_swz_rt (a tile that 16-byte row reads
// use as well) instead of gr_swz_tr. PERMROW: the tile's rows are stored with bits 2
// and 3 swapped (gr_perm32 within 32-row blocks, k0 a multiple of 16); the
// lane still receives logical rows k0 + 8(l/32) + 0..7.
template <class T, int COLS, bool PERM, bool RTSWZ = false, bool PERMROW = false>
__device__ __forceinline__ typename gr_mfma<T>::vec8 gr_tr_frag(const char* tile, int k0, int n0, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  const int c = lane & 3;
  const int cc = PERM ? (((c & 1) << 1) | (c >> 1)) : c;
  const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * cc;
  gr_u32x4 r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = k0 + (PERMROW ? 4 * (lane >> 5) + 8 * h : 8 * (lane >> 5) + 4 * h) + ((lane >> 2) & 3);
    const int chunk = RTSWZ ? gr_swz_rt<COLS / 8>(row, col >> 3) : gr_swz_tr<COLS / 8>(row, col >> 3);
    const char* p = tile + row * (COLS * 2) + chunk * 16 + (col & 7) * 2;
    const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(__attribute__((address_space(3))) char*)(char*)p);
    const gr_u32x2 w = __builtin_bit_cast(gr_u32x2, v);
    r[2 * h] = w[0];
    r[2 * h + 1] = w[1];
  }
  return gr_as<typename gr_mfma<T>::vec8>(r);
}

template <int D, int BN>
struct gr_flash_lds {
  static constexpr int KS = BN * D * 2;
  static constexpr int VT = D * BN * 2;
  static constexpr int BYTES = 2 * (KS + VT);
};

// One key tile of S^T = K Q^T for this wave: s[kb][qb] (32 keys x 32 queries
// per block). K rows sit in LDS with the row permutation gr_perm32.
template <class T, int D, int BN, int QB, bool KTR = false>
__device__ __forceinline__ void gr_flash_qk(gr_f32x16 (&s)[BN / 32][QB], const char* ks,
                                            const typename gr_mfma<T>::vec8 (&qf)[QB][D / 16], int l32, int g) {
  typedef typename gr_mfma<T>::vec8 vec8;
#pragma unroll
  for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) s[kb][qb] = (gr_f32x16)(0.f);
  // the key blocks' accumulator chains interleaved: consecutive MFMAs are
  // independent
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds)
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      const int row = kb * 32 + l32;
      // KTR: K^T tile [D][BN] read transposed; else K rows [BN][D] (rows bit-permuted)
      const vec8 af = KTR ? gr_tr_frag<T, BN, true>(ks, ds * 16, kb * 32, l32 + 32 * g)
                          : gr_as<vec8>(gr_ld16(ks + row * (D * 2) + gr_swz<D / 8>(row, 2 * ds + g) * 16));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[kb][qb] = gr_mfma<T>::mma32(af, qf[qb][ds], s[kb][qb]);
    }
}

// gr_flash_qk with the accumulators starting from ci[qb] instead of zero: each
// score comes out as q.k - base in one MFMA chain.
template <class T, int D, int BN, int QB, bool KTR = false>
__device__ __forceinline__ void gr_flash_qk_from(gr_f32x16 (&s)[BN / 32][QB], const char* ks,
                                                 const typename gr_mfma<T>::vec8 (&qf)[QB][D / 16],
                                                 const gr_f32x16 (&ci)[QB], int l32, int g) {
  typedef typename gr_mfma<T>::vec8 vec8;
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds)
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      const int row = kb * 32 + l32;
      const vec8 af = KTR ? gr_tr_frag<T, BN, true>(ks, ds * 16, kb * 32, l32 + 32 * g)
                          : gr_as<vec8>(gr_ld16(ks + row * (D * 2) + gr_swz<D / 8>(row, 2 * ds + g) * 16));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[kb][qb] = gr_mfma<T>::mma32(af, qf[qb][ds], ds == 0 ? ci[qb] : s[kb][qb]);
    }
}

// PRESCALE = false keeps fp16 Q as given and scales every score on the VALU
// instead (as bf16 does): the launch path for fp16 with scale log2(e) > 1,
// where the pre-scaled Q could overflow.
template <class T, int D, int BN, int NW, int QB, bool CAUSAL, bool KT_LAYOUT, bool PIPE, bool TR = false,
          bool DIRECT = false, bool SPLIT = false, bool PRESCALE = true>
__device__ __forceinline__ void gr_flash_fwd_body(const gr_attn_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  typedef typename MF::vec2 vec2;
  constexpr int BM = NW * QB * 32;
  constexpr int NT = NW * 64;
  constexpr int KB = BN / 32;      // 32-key blocks per tile
  constexpr int DB = D / 32;       // 32-wide head-dim blocks
  constexpr int DS = D / 16;       // 16-deep contraction steps over D
  typedef gr_flash_lds<D, BN> L;
  static_assert(BN % 32 == 0 && D % 32 == 0, "tile shape");
  static_assert(!(SPLIT && (CAUSAL || PIPE)), "key split: non-causal, straight schedule");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int Nq = a.Nq;
  const int nqt = (Nq + BM - 1) / BM;
  int bh, qt;
  if constexpr (CAUSAL) {
    gr_causal_order((int)blockIdx.x, (int)gridDim.x, nqt, bh, qt);
    qt = nqt - 1 - qt;                        // the longest query tiles first
  } else {
    const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    bh = logical / nqt;
    qt = logical % nqt;
  }
  const int b = bh / a.H, h = bh % a.H;

  // this workgroup's keys: all of them, or (SPLIT) part blockIdx.y
  const int key0 = SPLIT ? (int)blockIdx.y * a.kchunk : 0;
  const int nkeys = SPLIT ? (a.N - key0 < a.kchunk ? a.N - key0 : a.kchunk) : a.N;
  const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
  const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh + key0 * (KT_LAYOUT ? 1LL : a.k_sn);
  const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh + key0 * a.v_sn;
  T* Op = (T*)a.o + b * a.o_sb + h * a.o_sh;

  const int q0 = qt * BM;
  const int qw = q0 + wave * (QB * 32);
  const float c = a.scale_log2;

  // Q fragments (8 consecutive d of one query per lane). STAGE_Q: each wave
  // loads its 32-query blocks straight into the LDS slots the second key tile
  // will use (whole rows, 16 bytes per lane) and reads its fragments from
  // there before the prologue barrier; else a lane loads its fragments from
  // global memory directly (every load then touches 32 rows).
  constexpr int QBLK = 32 * D * 2;
  constexpr bool STAGE_Q = DIRECT && !PIPE && NW * QB <= 2 * KB;
  vec8 qf[QB][DS];
  if constexpr (!STAGE_Q) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        qf[qb][ds] = gr_as<vec8>(gr_ld16(Qp + (long long)gr_imin(qw + qb * 32 + l32, Nq - 1) * a.q_sn + ds * 16 + 8 * g));
  }
  auto q_stage = [&](int qb) -> char* {
    // K slot 1, then V slot 1, KB blocks each; wave-uniform (an SGPR for the
    // direct loads' LDS base)
    const int idx = __builtin_amdgcn_readfirstlane(wave) * QB + qb;
    return (idx < KB ? lds + L::KS : lds + 2 * L::KS + L::VT) + (idx % KB) * QBLK;
  };
  if constexpr (STAGE_Q) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      gr_lds_loader<T, 32, D, 64> ql;
      const int rows = Nq - (qw + qb * 32);
      ql.init(lane, a.q_sn, rows < 1 ? 1 : (rows > 32 ? 32 : rows));
      ql.load(Qp + (long long)(qw + qb * 32 < Nq ? qw + qb * 32 : Nq - 1) * a.q_sn, q_stage(qb));
    }
  }
  // CI (transposing reads, GR_FLASH_OPT): Q is pre-scaled by c = scale
  // log2(e) (rounded to T once: relative 2^-11 in fp16, 2^-8 in bf16) and the
  // score MFMAs start from -base, so the scores come out as exponents of 2
  // relative to the base and p = 2^s needs no VALU multiply-add per score. m
  // then holds the base in those units (scale log2(e) q.k). fp16 only: bf16
  // keeps Q as given.
  constexpr bool CI = GR_FLASH_OPT && PRESCALE && TR && gr_is_same<T, _Float16>::value;
  gr_f32x16 cinit[QB];
  auto prescale_q = [&]() {
    if constexpr (CI) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        cinit[qb] = (gr_f32x16)(0.f);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[qb][ds][e] = (T)((float)qf[qb][ds][e] * a.scale_log2);
      }
    }
  };

  gr_f32x16 o[DB][QB];
  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -GR_INF;
    l[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db][qb] = (gr_f32x16)(0.f);
  }

  char* ks0 = lds;
  char* vt0 = lds + 2 * L::KS;

  // K tile source: natural rows [BN keys][D] or transposed [D][BN keys].
  // TR: V and (KT layout) K^T tiles land in LDS as they are in memory and the
  // MFMA fragments are read back transposed (gr_tr_frag).
  constexpr bool KTR = TR && KT_LAYOUT;
  typedef gr_row_loader<T, BN, D, NT, true> KRows;
  typedef typename gr_cond<KTR, gr_row_loader<T, D, BN, NT, false, true>, gr_tr_loader<T, D, BN, NT, true>>::type KCols;
  typedef typename gr_cond<TR, gr_row_loader<T, BN, D, NT, false, true>, gr_tr_loader<T, BN, D, NT, false>>::type VLoad;
  // DIRECT (needs TR): the same tiles, loaded straight into LDS.
  static_assert(!DIRECT || TR, "direct-to-LDS tiles are read through gr_tr_frag");
  typedef typename gr_cond<KT_LAYOUT, gr_lds_loader<T, D, BN, NT, true>, gr_lds_loader<T, BN, D, NT, false, true>>::type
      KDirect;
  typedef gr_lds_loader<T, BN, D, NT, true> VDirect;
  typename gr_cond<DIRECT, KDirect, typename gr_cond<KT_LAYOUT, KCols, KRows>::type>::type kl;
  typename gr_cond<DIRECT, VDirect, VLoad>::type vl;
  kl.init(tid, a.k_sn);
  vl.init(tid, a.v_sn);
  // Element offset of key tile t in K (KT layout: a column offset).
  const long long k_tile = KT_LAYOUT ? (long long)BN : (long long)BN * a.k_sn;
  const long long v_tile = (long long)BN * a.v_sn;

  const int ntile = CAUSAL ? (q0 + BM + BN - 1) / BN : nkeys / BN;
  const int wq_last = qw + QB * 32 - 1;        // this wave's last query
  auto wave_active = [&](int t) { return !CAUSAL || t * BN <= wq_last; };

  // LDS ring: K_j and V_j live in slot j & 1. With PIPE the scores of tile
  // t+1 are computed during iteration t (on the matrix cores, while tile t's
  // softmax runs on the vector ALUs): iteration t reads K_{t+1} and V_t and then
  // stores K_{t+2}, V_{t+1} into the slots K_t and V_{t-1} occupied. Without
  // PIPE iteration t reads K_t, V_t and stores K_{t+1}, V_{t+1}.
  constexpr int KAHEAD = PIPE ? 2 : 1;
  if constexpr (DIRECT) {
    kl.load(Kp, ks0);
    vl.load(Vp, vt0);
    if (PIPE && ntile > 1) kl.load(Kp + k_tile, ks0 + L::KS);
  } else {
    kl.gload(Kp, tid);
    vl.gload(Vp, tid);
    kl.sstore(ks0, tid);
    vl.sstore(vt0, tid);
    if (PIPE && ntile > 1) {
      kl.gload(Kp + k_tile, tid);
      kl.sstore(ks0 + L::KS, tid);
    }
  }
  // Retire every prologue load (the Q fragments in particular) before the
  // loop: the compiler's wait-counter tracking cannot see through the loop
  // back edge that they completed, and would otherwise wait on the vmcnt of
  // the in-flight next-tile prefetch at the first score MFMA of every tile.
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (STAGE_Q) {
    // this wave's own Q blocks (its loads have landed: vmcnt is 0); the
    // barrier below orders these reads before the next tile's prefetch
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        qf[qb][ds] = gr_as<vec8>(gr_ld16(q_stage(qb) + l32 * (D * 2) + gr_swz<D / 8>(l32, 2 * ds + g) * 16));
  }
  __syncthreads();
  prescale_q();
  // Two score buffers used in turn (the loop is unrolled by two), so handing
  // the next tile's scores over costs no register moves.
  gr_f32x16 sA[KB][QB], sB[PIPE ? KB : 1][QB];
  // CI with PIPE: the base (in exponent units) each score buffer's MFMAs
  // started from; slot j & 1 holds tile j's
  float sbase[2][QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) sbase[0][qb] = sbase[1][qb] = 0.f;
  if (PIPE) {
    gr_flash_qk<T, D, BN, QB, KTR>(sA, ks0, qf, l32, g);
    if constexpr (CI && !CAUSAL) {
      // the first tile's max pass here, so that every tile takes the fast
      // path: the base moves to the row max and the first scores follow it
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mt = -GR_INF;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sA[kb][qb][r]);
        mt = fmaxf(mt, gr_xor32(mt));
        m[qb] = mt;
        sbase[0][qb] = mt;
        cinit[qb] = (gr_f32x16)(-mt);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sA[kb][qb] -= mt;
      }
    }
    __syncthreads();   // every wave is done with slot 0 of K before K_2 lands there
  }

  // One key tile. s: this tile's scores; sn: next tile's (PIPE only).
  // Slots are compile-time in each unrolled copy (ODD = t & 1).
  auto tile = [&](const int t, auto odd_tag, auto& s, auto& sn) {
    constexpr int ODD = decltype(odd_tag)::value;
    const bool pf_k = t + KAHEAD < ntile, pf_v = t + 1 < ntile;
    // The slots the next tiles go to were last read before the previous
    // iteration's closing barrier.
    char* const k_next = ks0 + (PIPE ? ODD : (ODD ^ 1)) * L::KS;
    char* const v_next = vt0 + (ODD ^ 1) * L::VT;
    if constexpr (DIRECT) {
      if (pf_k) kl.load(Kp + (t + KAHEAD) * k_tile, k_next);
      if (pf_v) vl.load(Vp + (t + 1) * v_tile, v_next);
    } else {
      if (pf_k) kl.gload(Kp + (t + KAHEAD) * k_tile, tid);
      if (pf_v) vl.gload(Vp + (t + 1) * v_tile, tid);
    }
    const int k0 = t * BN;
    if (wave_active(t)) {
      // this tile's scores (with PIPE they were computed in the previous
      // iteration) and, on the diagonal of a causal block, the mask
      auto mask = [&]() {
        if (CAUSAL && k0 + BN - 1 > qw) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              const int query = qw + qb * 32 + l32;
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int key = k0 + kb * 32 + ((r < 8) ? (8 * g + r) : (16 + 8 * g + r - 8));
                if (key > query) s[kb][qb][r] = -GR_INF;
              }
            }
        }
      };
      auto scores = [&]() {
        if constexpr (!PIPE) gr_flash_qk<T, D, BN, QB, KTR>(s, ks0 + ODD * L::KS, qf, l32, g);
        mask();
      };
#if GR_FLASH_OPT
      if constexpr (CI) {
        // P of the whole tile with the current base and no max pass; the max
        // pass runs only on the first tile and when some p overflowed (then
        // the base moves to the true max and P is recomputed, shifted).
        vec8 pt[KB][2][QB];
        float lt[QB];
        auto make_p = [&](auto shift_tag, const float (&sh)[QB]) {
          constexpr bool SHIFT = decltype(shift_tag)::value;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) lt[qb] = 0.f;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
              for (int qb = 0; qb < QB; ++qb) {
                gr_u32x4 pw;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                  const float x0 = SHIFT ? s[kb][qb][8 * hf + e] + sh[qb] : s[kb][qb][8 * hf + e];
                  const float x1 = SHIFT ? s[kb][qb][8 * hf + e + 1] + sh[qb] : s[kb][qb][8 * hf + e + 1];
                  const vec2 pp = __builtin_convertvector((gr_f32x2){gr_exp2(x0), gr_exp2(x1)}, vec2);
                  lt[qb] = MF::sum2(pp, lt[qb]);
                  pw[e >> 1] = __builtin_bit_cast(unsigned int, pp);
                }
                pt[kb][hf][qb] = gr_as<vec8>(pw);
              }
        };
        bool fresh = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) fresh |= m[qb] == -GR_INF;
        bool ok = false;
        if constexpr (PIPE) {
          // This tile's scores were computed in the previous iteration from
          // the base of that time (sbase). In one basic block, so that the
          // scheduler can put the exponentials between the matrix ops: the
          // next tile's score MFMAs from the current base, and P of this tile
          // taken as if its base were still current. A tile whose base has
          // moved since (a rescale in between), the first tile and a tile
          // with an overflowed p take the slow path below.
          mask();
          bool stale = false;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            stale |= sbase[ODD][qb] != -cinit[qb][0];
            sbase[ODD ^ 1][qb] = -cinit[qb][0];
          }
          gr_flash_qk_from<T, D, BN, QB, KTR>(sn, ks0 + (ODD ^ 1) * L::KS, qf, cinit, l32, g);
          const float z[QB] = {};
          make_p(gr_ic<0>{}, z);
          bool bad = fresh || stale;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) bad |= !(lt[qb] <= 3.0e38f);   // an inf (or NaN) p
          ok = !gr_any(bad);
          // the next tile's K fragment reads first (their latency hides
          // behind the first exponentials), then per 32-key half block of
          // this tile its share of the score MFMAs and the exponentials,
          // packing and sums of its 16 scores per query block
          constexpr int NQK = KB * DS * QB;
          constexpr int NRD = KB * DS * (KTR ? 2 : 1);
          constexpr int GROUPS = KB * 2;
          __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);              // K fragment reads (t+1)
#pragma unroll
          for (int i = 0; i < GROUPS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, NQK / GROUPS, 0);   // score MFMAs (t+1)
            __builtin_amdgcn_sched_group_barrier(0x002, 16 * QB, 0);        // softmax VALU (t)
          }
        } else {
          gr_flash_qk_from<T, D, BN, QB, KTR>(s, ks0 + ODD * L::KS, qf, cinit, l32, g);
          mask();
          if (!gr_any(fresh)) {
            const float z[QB] = {};
            make_p(gr_ic<0>{}, z);
            bool bad = false;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) bad |= !(lt[qb] <= 3.0e38f);   // an inf (or NaN) p
            ok = !gr_any(bad);
          }
        }
        if (!ok) {
          float sh[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            // the base these scores are relative to
            const float bt = PIPE ? sbase[ODD][qb] : ((m[qb] == -GR_INF) ? 0.f : m[qb]);
            float mt = -GR_INF;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
              for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][qb][r]);
            mt = fmaxf(mt, gr_xor32(mt));
            const float mn = fmaxf(m[qb], mt + bt);
            if (gr_any(mn > m[qb])) {
              const float alpha = gr_exp2(m[qb] - mn);   // m = -inf -> 0
              l[qb] *= alpha;
#pragma unroll
              for (int db = 0; db < DB; ++db) o[db][qb] *= alpha;
              m[qb] = mn;
            }
            const float nb = (m[qb] == -GR_INF) ? 0.f : m[qb];
            sh[qb] = bt - nb;
            cinit[qb] = (gr_f32x16)(-nb);
          }
          make_p(gr_ic<1>{}, sh);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) l[qb] += lt[qb];
        const char* vt = vt0 + ODD * L::VT;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              const vec8 vf = gr_tr_frag<T, D, false>(vt, kb * 32 + 16 * hf, db * 32, l32 + 32 * g);
#pragma unroll
              for (int qb = 0; qb < QB; ++qb) o[db][qb] = MF::mma32(vf, pt[kb][hf][qb], o[db][qb]);
            }
      } else
      if constexpr (!PIPE && TR) {
        // bf16: Q is not pre-scaled (its rounding would cost 2^-8), one
        // multiply-add per score instead
        // P of the whole tile with the current base; the max pass runs only on
        // the first tile and when some p overflowed (then the base moves to
        // the true max and P is recomputed).
        vec8 pt[KB][2][QB];
        float lt[QB];
        auto make_p = [&](const float (&nmc)[QB]) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) lt[qb] = 0.f;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
              for (int qb = 0; qb < QB; ++qb) {
                gr_u32x4 pw;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                  const float p0 = gr_exp2(fmaf(s[kb][qb][8 * hf + e], c, nmc[qb]));
                  const float p1 = gr_exp2(fmaf(s[kb][qb][8 * hf + e + 1], c, nmc[qb]));
                  const vec2 pp = __builtin_convertvector((gr_f32x2){p0, p1}, vec2);
                  lt[qb] = MF::sum2(pp, lt[qb]);
                  pw[e >> 1] = __builtin_bit_cast(unsigned int, pp);
                }
                pt[kb][hf][qb] = gr_as<vec8>(pw);
              }
        };
        bool fresh = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) fresh |= m[qb] == -GR_INF;
        bool ok = false;
        if (gr_any(fresh)) {
          scores();
        } else {
          // the scores and their exponentials in one block, so the first
          // blocks' exponentials can run while the last score MFMAs do
          scores();
          float nmc[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) nmc[qb] = -m[qb] * c;
          make_p(nmc);
          bool bad = false;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) bad |= !(lt[qb] <= 3.0e38f);   // an inf (or NaN) p
          ok = !gr_any(bad);
        }
        if (!ok) {
          float nmc[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            float mt = -GR_INF;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
              for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][qb][r]);
            mt = fmaxf(mt, gr_xor32(mt));
            const float mn = fmaxf(m[qb], mt);
            if (gr_any(mn > m[qb])) {
              const float alpha = gr_exp2((m[qb] - mn) * c);   // m = -inf -> 0
              l[qb] *= alpha;
#pragma unroll
              for (int db = 0; db < DB; ++db) o[db][qb] *= alpha;
              m[qb] = mn;
            }
            nmc[qb] = -((m[qb] == -GR_INF) ? 0.f : m[qb]) * c;
          }
          make_p(nmc);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) l[qb] += lt[qb];
        const char* vt = vt0 + ODD * L::VT;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              const vec8 vf = gr_tr_frag<T, D, false>(vt, kb * 32 + 16 * hf, db * 32, l32 + 32 * g);
#pragma unroll
              for (int qb = 0; qb < QB; ++qb) o[db][qb] = MF::mma32(vf, pt[kb][hf][qb], o[db][qb]);
            }
      } else
#endif
      {
      scores();
      // Running reference max m. The exponent base is only moved (and the
      // accumulators rescaled) when some lane's true max exceeds m by more
      // than 2^GR_RESCALE_LOG2 in p; otherwise p = 2^((s - m) c) may reach
      // that bound, which fp16/bf16 P, the fp32 row sum and fp32 O absorb
      // exactly as well: O = sum p v / sum p does not depend on the base.
      float nmc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mt = -GR_INF;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][qb][r]);
        mt = fmaxf(mt, gr_xor32(mt));
        const float mn = fmaxf(m[qb], mt);
        if (gr_any(mn > m[qb] + GR_RESCALE_LOG2 / c)) {    // m = -inf: any finite score moves it
          const float alpha = gr_exp2((m[qb] - mn) * c);   // m = -inf -> 0
          l[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[db][qb] *= alpha;
          m[qb] = mn;
        }
        nmc[qb] = -((m[qb] == -GR_INF) ? 0.f : m[qb]) * c;
      }
      // PIPE: the next tile's scores, issued unconditionally so they share one
      // basic block with this tile's softmax and P*V and can be interleaved
      // with them (after the last tile this reads a stale but valid K slot and
      // the result is dropped).
      if constexpr (PIPE) gr_flash_qk<T, D, BN, QB, KTR>(sn, ks0 + (ODD ^ 1) * L::KS, qf, l32, g);
      const char* vt = vt0 + ODD * L::VT;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          vec8 pf[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            gr_u32x4 pw;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              const float p0 = gr_exp2(fmaf(s[kb][qb][8 * hf + e], c, nmc[qb]));
              const float p1 = gr_exp2(fmaf(s[kb][qb][8 * hf + e + 1], c, nmc[qb]));
              const vec2 pp = __builtin_convertvector((gr_f32x2){p0, p1}, vec2);
              l[qb] = MF::sum2(pp, l[qb]);
              pw[e >> 1] = __builtin_bit_cast(unsigned int, pp);
            }
            pf[qb] = gr_as<vec8>(pw);
          }
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int row = db * 32 + l32;
            const vec8 vf = TR ? gr_tr_frag<T, D, false>(vt, kb * 32 + 16 * hf, db * 32, l32 + 32 * g)
                               : gr_as<vec8>(gr_ld16(vt + row * (BN * 2) + gr_swz<BN / 8>(row, 4 * kb + 2 * hf + g) * 16));
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) o[db][qb] = MF::mma32(vf, pf[qb], o[db][qb]);
          }
        }
      }
      if constexpr (PIPE && !CI) {
        // Interleave: per 32-key half block, the next tile's K reads and score
        // MFMAs between this tile's exponentials and its P*V MFMAs, so the
        // matrix cores run while the VALU works on the softmax.
        constexpr int NQK = KB * DS * QB;          // next-tile score MFMAs
        constexpr int NPV = KB * 2 * DB * QB;      // this tile's P*V MFMAs
        constexpr int GROUPS = KB * 2;
#pragma unroll
        for (int i = 0; i < GROUPS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, NQK / GROUPS, 0);   // K fragment reads
          __builtin_amdgcn_sched_group_barrier(0x008, NQK / GROUPS, 0);   // score MFMAs (t+1)
          __builtin_amdgcn_sched_group_barrier(0x002, 12 * QB, 0);        // softmax VALU
          __builtin_amdgcn_sched_group_barrier(0x100, DB, 0);             // V^T fragment reads
          __builtin_amdgcn_sched_group_barrier(0x008, NPV / GROUPS, 0);   // P*V MFMAs (t)
        }
      }
    }
    if constexpr (DIRECT) {
      __builtin_amdgcn_s_waitcnt(0);   // this wave's tile loads have landed in LDS
    } else {
      if (pf_k) kl.sstore(k_next, tid);
      if (pf_v) vl.sstore(v_next, tid);
    }
    __syncthreads();
  };

  for (int t = 0; t < ntile; t += 2) {
    if constexpr (PIPE) {
      tile(t, gr_ic<0>{}, sA, sB);
      if (t + 1 < ntile) tile(t + 1, gr_ic<1>{}, sB, sA);
    } else {
      tile(t, gr_ic<0>{}, sA, sB);
      if (t + 1 < ntile) tile(t + 1, gr_ic<1>{}, sA, sB);
    }
  }

  if constexpr (SPLIT) {
    // unnormalised partial O and the (reference max, row sum) it is based on
    const long long part = (long long)blockIdx.y * a.B * a.H + bh;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q = qw + qb * 32 + l32;
      const float lt = l[qb] + gr_xor32(l[qb]);
      if (q < Nq) {
        float* po = a.part_o + (part * Nq + q) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const gr_f32x4 w = {o[db][qb][4 * rr], o[db][qb][4 * rr + 1], o[db][qb][4 * rr + 2], o[db][qb][4 * rr + 3]};
            *reinterpret_cast<gr_f32x4*>(po + db * 32 + 8 * rr + 4 * g) = w;
          }
        // m in units of q.k (the merge kernel scales by c)
        if (g == 0) *reinterpret_cast<gr_f32x2*>(a.part_ml + (part * Nq + q) * 2) = (gr_f32x2){CI ? m[qb] / c : m[qb], lt};
      }
    }
    return;
  }
  // O = O^T^T / l. A lane holds 4 x 8 bytes of its query's row per 32 head
  // dims; written as they are, every store instruction touches 32 rows. When
  // the LDS ring can hold the workgroup's O tile (it is free after the last
  // tile's barrier), each wave stages its 32 x D block there and stores whole
  // 16-byte chunks of consecutive rows instead (8 rows of 128 bytes per
  // instruction at d = 64).
  constexpr int CPR = D / 8;
  constexpr bool STAGE_O = L::BYTES >= NW * QB * 32 * D * 2;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = l[qb] + gr_xor32(l[qb]);
    const float inv = 1.0f / lt;
    const bool live = qw + qb * 32 + l32 < Nq;
    // log-sum-exp of scale * s: p = 2^((s - m) c) with c = scale log2(e)
    if (live && a.lse && g == 0)
      a.lse[(long long)bh * Nq + qw + qb * 32 + l32] = ((CI ? m[qb] : m[qb] * c) + __builtin_amdgcn_logf(lt)) * 0.6931471805599453f;
    char* const stage = lds + (wave * QB + qb) * (32 * D * 2);
    T* orow = Op + (long long)(qw + qb * 32 + l32) * a.o_sn;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const unsigned int w0 = gr_pack2f<T>(o[db][qb][4 * rr + 0] * inv, o[db][qb][4 * rr + 1] * inv);
        const unsigned int w1 = gr_pack2f<T>(o[db][qb][4 * rr + 2] * inv, o[db][qb][4 * rr + 3] * inv);
        gr_u32x2 w = {w0, w1};
        if constexpr (STAGE_O)
          *reinterpret_cast<gr_u32x2*>(stage + l32 * (D * 2) + gr_swz<CPR>(l32, db * 4 + rr) * 16 + g * 8) = w;
        else if (live)
          *reinterpret_cast<gr_u32x2*>(orow + db * 32 + 8 * rr + 4 * g) = w;
      }
    if constexpr (STAGE_O) {
      __builtin_amdgcn_wave_barrier();   // this wave's LDS writes precede its reads (in order per wave)
#pragma unroll
      for (int it = 0; it < 32 * CPR / 64; ++it) {
        const int j = it * 64 + lane, row = j / CPR, ch = j % CPR;
        const gr_u32x4 v = gr_ld16(stage + row * (D * 2) + gr_swz<CPR>(row, ch) * 16);
        if (qw + qb * 32 + row < Nq)   // streamed past the caches: nothing here reads O back
          __builtin_nontemporal_store(v, reinterpret_cast<gr_u32x4*>(Op + (long long)(qw + qb * 32 + row) * a.o_sn + ch * 8));
      }
    }
  }
}

// Waves per SIMD the kernel is compiled for. Two caps it at 256 VGPRs, which
// lets the backend keep every MFMA operand and accumulator in VGPRs (no AGPR
// round trips around the softmax arithmetic); configurations whose estimated
// live state exceeds that ask for one wave (and use AGPRs) instead of spilling.
// Estimate (VGPRs/lane): two score buffers QB*BN, output QB*D/2, Q fragments
// QB*D/4, prefetch registers + offsets of the K and V tile loaders, ~40 misc.
template <int D, int BN, int NW, int QB, bool KT, bool PIPE>
struct gr_flash_wpe {
  static constexpr int NT = NW * 64;
  static constexpr int K_UNITS = KT ? (D / 2) * (BN / 8) : BN * D / 8;
  static constexpr int K_REGS = (KT ? 10 : 6) * ((K_UNITS + NT - 1) / NT);
  static constexpr int V_REGS = 10 * (((BN / 2) * (D / 8) + NT - 1) / NT);
  static constexpr int EST = (PIPE ? 2 : 1) * QB * BN / 2 + QB * D / 2 + QB * D / 4 + K_REGS + V_REGS + 40;
  static constexpr int value = EST > 224 ? 1 : 2;
};

// Kernel wrapper used by the prebuilt library; the grammar renderer emits its
// own wrappers with baked-in shapes around the same body.
template <class T, int D, int BN, int NW, int QB, bool CAUSAL, bool KT_LAYOUT, bool PIPE, bool TR = false,
          bool DIRECT = false, bool SPLIT = false, bool PRESCALE = true>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(gr_flash_wpe<D, BN, NW, QB, KT_LAYOUT, PIPE>::value)))
void gr_flash_fwd_kernel(gr_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash_fwd_body<T, D, BN, NW, QB, CAUSAL, KT_LAYOUT, PIPE, TR, DIRECT, SPLIT, PRESCALE>(a, gr_lds);
}
