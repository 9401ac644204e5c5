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
//  * Q stays in registers for the whole kernel. K and V^T tiles are double
//    buffered in LDS (one barrier per key tile) and prefetched from global
//    into registers one tile ahead. 16-byte LDS chunks are XOR-swizzled by row
//    so both the tile writes and the MFMA operand reads are bank-conflict free.
//  * Causal: key tiles past the block's last query are never visited; waves
//    whose queries all precede a tile skip its math; the mask is applied only
//    on diagonal tiles. Heavy query tiles are scheduled first.
//  * Workgroups of one head are mapped to one XCD so K/V are shared in its L2.
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
  int B, H, N;
  float scale_log2;             // softmax scale * log2(e)
};

template <bool C, class X, class Y> struct gr_cond { typedef X type; };
template <class X, class Y> struct gr_cond<false, X, Y> { typedef Y type; };

// Swap bits 2 and 3 of a row index inside a 32-row MFMA block.
__device__ __forceinline__ int gr_perm32(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// XOR swizzle of the 16-byte chunk index inside an LDS row of CPR chunks, so
// that 8 consecutive rows read at the same logical chunk hit distinct banks.
template <int CPR>
__device__ __forceinline__ int gr_swz(int row, int chunk) {
  if constexpr (CPR >= 8) return chunk ^ (row & 7);
  else if constexpr (CPR == 4) return chunk ^ ((row >> 1) & 3);
  else if constexpr (CPR == 2) return chunk ^ ((row >> 2) & 1);
  else return chunk;
}

// Global [ROWS][COLS] tile (row stride ld elements) -> LDS rows, same shape.
template <class T, int ROWS, int COLS, int NT, bool PERM>
struct gr_row_loader {
  static constexpr int CPR = COLS / 8;
  static constexpr int CHUNKS = ROWS * CPR;
  static constexpr int PER = (CHUNKS + NT - 1) / NT;
  gr_u32x4 r[PER];
  __device__ __forceinline__ void gload(const T* src, long long ld, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) {
        const int row = c / CPR, cc = c % CPR;
        r[i] = gr_ld16(src + (long long)row * ld + cc * 8);
      }
    }
  }
  __device__ __forceinline__ void sstore(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) {
        const int row = c / CPR, cc = c % CPR;
        const int prow = PERM ? gr_perm32(row) : row;
        gr_st16(dst + prow * (COLS * 2) + gr_swz<CPR>(prow, cc) * 16, r[i]);
      }
    }
  }
};

// Global [SR][SC] tile (row stride ld) -> LDS [SC][SR] (transposed). Each unit
// takes two source rows x 8 columns and writes 8 dwords, each holding the pair
// of source-row values for one destination row.
template <class T, int SR, int SC, int NT, bool PERM>
struct gr_tr_loader {
  static constexpr int PAIRS = SR / 2;
  static constexpr int SCPR = SC / 8;
  static constexpr int UNITS = PAIRS * SCPR;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int DCPR = SR / 8;
  gr_u32x4 r0[PER], r1[PER];
  __device__ __forceinline__ void gload(const T* src, long long ld, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int p = u % PAIRS, cc = u / PAIRS;
        r0[i] = gr_ld16(src + (long long)(2 * p) * ld + cc * 8);
        r1[i] = gr_ld16(src + (long long)(2 * p + 1) * ld + cc * 8);
      }
    }
  }
  __device__ __forceinline__ void sstore(char* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int p = u % PAIRS, cc = u / PAIRS;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const unsigned int w0 = r0[i][e >> 1], w1 = r1[i][e >> 1];
          const unsigned int w = (e & 1) ? ((w0 >> 16) | (w1 & 0xffff0000u))
                                         : ((w0 & 0xffffu) | (w1 << 16));
          const int drow = cc * 8 + e;
          const int prow = PERM ? gr_perm32(drow) : drow;
          *reinterpret_cast<unsigned int*>(dst + prow * (SR * 2) +
                                           gr_swz<DCPR>(prow, p >> 2) * 16 + (p & 3) * 4) = w;
        }
      }
    }
  }
};

template <int D, int BN>
struct gr_flash_lds {
  static constexpr int KS = BN * D * 2;
  static constexpr int VT = D * BN * 2;
  static constexpr int BYTES = 2 * (KS + VT);
};

template <class T, int D, int BN, int NW, int QB, bool CAUSAL, bool KT_LAYOUT>
__device__ __forceinline__ void gr_flash_fwd_body(const gr_attn_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int BM = NW * QB * 32;
  constexpr int NT = NW * 64;
  constexpr int KB = BN / 32;      // 32-key blocks per tile
  constexpr int DB = D / 32;       // 32-wide head-dim blocks
  constexpr int DS = D / 16;       // 16-deep contraction steps over D
  typedef gr_flash_lds<D, BN> L;
  static_assert(BN % 32 == 0 && D % 32 == 0, "tile shape");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nqt = a.N / BM;
  const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / nqt;
  int qt = logical % nqt;
  if (CAUSAL) qt = nqt - 1 - qt;
  const int b = bh / a.H, h = bh % a.H;

  const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
  const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
  const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
  T* Op = (T*)a.o + b * a.o_sb + h * a.o_sh;

  const int q0 = qt * BM;
  const int qw = q0 + wave * (QB * 32);
  const float c = a.scale_log2;

  vec8 qf[QB][DS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qf[qb][ds] = gr_as<vec8>(gr_ld16(Qp + (long long)(qw + qb * 32 + l32) * a.q_sn + ds * 16 + 8 * g));

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
  typedef gr_row_loader<T, BN, D, NT, true> KRows;
  typedef gr_tr_loader<T, D, BN, NT, true> KCols;
  typedef gr_tr_loader<T, BN, D, NT, false> VLoad;
  typename gr_cond<KT_LAYOUT, KCols, KRows>::type kl;
  VLoad vl;

  const int ntile = CAUSAL ? (q0 + BM + BN - 1) / BN : a.N / BN;

  auto gload = [&](int t) {
    if constexpr (KT_LAYOUT) kl.gload(Kp + t * BN, a.k_sn, tid);
    else kl.gload(Kp + (long long)t * BN * a.k_sn, a.k_sn, tid);
    vl.gload(Vp + (long long)t * BN * a.v_sn, a.v_sn, tid);
  };
  auto sstore = [&](int buf) {
    kl.sstore(ks0 + buf * L::KS, tid);
    vl.sstore(vt0 + buf * L::VT, tid);
  };

  gload(0);
  sstore(0);
  for (int t = 0; t < ntile; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntile) gload(t + 1);
    __syncthreads();
    const int k0 = t * BN;
    const bool active = !CAUSAL || (k0 <= qw + QB * 32 - 1);
    if (active) {
      const char* ks = ks0 + cur * L::KS;
      const char* vt = vt0 + cur * L::VT;
      gr_f32x16 s[KB][QB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[kb][qb] = (gr_f32x16)(0.f);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int row = kb * 32 + l32;
          const vec8 af = gr_as<vec8>(gr_ld16(ks + row * (D * 2) + gr_swz<D / 8>(row, 2 * ds + g) * 16));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) s[kb][qb] = MF::mma32(af, qf[qb][ds], s[kb][qb]);
        }
      }
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
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mt = -GR_INF;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][qb][r]);
        mt = fmaxf(mt, gr_xor32(mt));
        const float mn = fmaxf(m[qb], mt);
        const float ms = (mn == -GR_INF) ? 0.f : mn;
        const float alpha = gr_exp2((m[qb] - ms) * c);
        const float nmc = -ms * c;
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = gr_exp2(fmaf(s[kb][qb][r], c, nmc));
            s[kb][qb][r] = p;
            ls += p;
          }
        l[qb] = l[qb] * alpha + ls;
        m[qb] = mn;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db][qb] *= alpha;
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          vec8 pf[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int e = 0; e < 8; ++e) pf[qb][e] = (T)s[kb][qb][8 * hf + e];
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int row = db * 32 + l32;
            const vec8 vf = gr_as<vec8>(gr_ld16(vt + row * (BN * 2) + gr_swz<BN / 8>(row, 4 * kb + 2 * hf + g) * 16));
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) o[db][qb] = MF::mma32(vf, pf[qb], o[db][qb]);
          }
        }
    }
    if (t + 1 < ntile) sstore(cur ^ 1);
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = l[qb] + gr_xor32(l[qb]);
    const float inv = 1.0f / lt;
    T* orow = Op + (long long)(qw + qb * 32 + l32) * a.o_sn;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const unsigned int w0 = gr_pack2<T>((T)(o[db][qb][4 * rr + 0] * inv), (T)(o[db][qb][4 * rr + 1] * inv));
        const unsigned int w1 = gr_pack2<T>((T)(o[db][qb][4 * rr + 2] * inv), (T)(o[db][qb][4 * rr + 3] * inv));
        gr_u32x2 w = {w0, w1};
        *reinterpret_cast<gr_u32x2*>(orow + db * 32 + 8 * rr + 4 * g) = w;
      }
  }
}

// Kernel wrapper used by the prebuilt library; the grammar renderer emits its
// own wrappers with baked-in shapes around the same body.
template <class T, int D, int BN, int NW, int QB, bool CAUSAL, bool KT_LAYOUT>
__global__ __launch_bounds__(NW * 64) void gr_flash_fwd_kernel(gr_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash_fwd_body<T, D, BN, NW, QB, CAUSAL, KT_LAYOUT>(a, gr_lds);
}
