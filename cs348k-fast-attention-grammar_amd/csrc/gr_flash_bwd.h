// gr_flash_bwd.h -- attention backward (dQ, dK, dV) for gfx950 (CDNA4).
//
// Given Q, K, V, O, dO [B, H, N, D] (common strides, unit stride on D) and
// the forward's row log-sum-exp L (natural log of sum_j exp(scale q.k_j)),
// computes dV = P^T dO, dK = scale dS^T Q, dQ = scale dS K with
// P = exp(scale Q K^T - L) [causal mask], dS = P * (dO V^T - delta),
// delta = rowsum(dO * O). Three kernels:
//  * gr_attn_bwd_pre_kernel: delta per row, and the fp32 dQ accumulator
//    cleared (a kernel, not a memset, so a captured graph replays it).
//  * gr_attn_bwd_kernel: one workgroup per block of BN keys of one head,
//    one wave per 32 of them. K and V of the wave stay in registers as MFMA
//    operands; dK^T and dV^T accumulate in registers over all query tiles.
//    Per tile of BM queries (Q and dO double-buffered in LDS, loaded straight
//    from global memory): S = Q K^T and dP = dO V^T with one key per lane (Q
//    and dO rows read with bits 2 and 3 of the row index swapped, so each
//    half-wave's accumulators hold 8 consecutive queries: they are directly
//    the B operand of dV^T += dO^T P and dK^T += Q^T dS, whose dO^T and Q^T
//    fragments come from transposing LDS reads of the same tiles). dS^T goes
//    to LDS and the workgroup forms dQ_tile = dS K from it and a K tile,
//    added into the fp32 accumulator with hardware float atomics.
//  * gr_attn_bwd_post_kernel: dQ = scale * accumulator in the storage type.
// Causal: a key block meets only the query tiles at or after its first key;
// the mask is applied on the tiles that straddle the diagonal.
#pragma once
#include "gr_flash_fwd.h"

struct gr_attn_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;     // [b*H+h][N], natural log
  float* delta;         // [b*H+h][N]
  float* dq_acc;        // [b*H+h][N][D]
  void* dq;
  void* dk;
  void* dv;
  long long sb, sh, sn;   // strides of all nine [B, H, N, D] tensors
  int B, H, N;
  float scale;
};

template <class T, int D>
__global__ __launch_bounds__(256) void gr_attn_bwd_pre_kernel(gr_attn_bwd_args a) {
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long rows = (long long)a.B * a.H * a.N;
  if (row >= rows) return;
  const int n = (int)(row % a.N);
  const int bh = (int)(row / a.N);
  const long long off = (bh / a.H) * a.sb + (bh % a.H) * a.sh + (long long)n * a.sn;
  const T* o = static_cast<const T*>(a.o) + off;
  const T* dout = static_cast<const T*>(a.dout) + off;
  float acc = 0.f;
  float* dq = a.dq_acc + row * D;
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const gr_u32x4 x = gr_ld16(o + 8 * c), y = gr_ld16(dout + 8 * c);
    const typename gr_mfma<T>::vec8 xv = gr_as<typename gr_mfma<T>::vec8>(x);
    const typename gr_mfma<T>::vec8 yv = gr_as<typename gr_mfma<T>::vec8>(y);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)xv[e] * (float)yv[e];
    *reinterpret_cast<gr_f32x4*>(dq + 8 * c) = (gr_f32x4)(0.f);
    *reinterpret_cast<gr_f32x4*>(dq + 8 * c + 4) = (gr_f32x4)(0.f);
  }
  a.delta[row] = acc;
}

template <class T, int D>
__global__ __launch_bounds__(256) void gr_attn_bwd_post_kernel(gr_attn_bwd_args a) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // one 8-element chunk
  const long long chunks = (long long)a.B * a.H * a.N * (D / 8);
  if (idx >= chunks) return;
  const long long row = idx / (D / 8);
  const int c = (int)(idx % (D / 8));
  const int n = (int)(row % a.N);
  const int bh = (int)(row / a.N);
  const float* src = a.dq_acc + row * D + 8 * c;
  const gr_f32x4 v0 = *reinterpret_cast<const gr_f32x4*>(src);
  const gr_f32x4 v1 = *reinterpret_cast<const gr_f32x4*>(src + 4);
  gr_u32x4 w;
  w[0] = gr_pack2<T>((T)(v0[0] * a.scale), (T)(v0[1] * a.scale));
  w[1] = gr_pack2<T>((T)(v0[2] * a.scale), (T)(v0[3] * a.scale));
  w[2] = gr_pack2<T>((T)(v1[0] * a.scale), (T)(v1[1] * a.scale));
  w[3] = gr_pack2<T>((T)(v1[2] * a.scale), (T)(v1[3] * a.scale));
  T* dst = static_cast<T*>(a.dq) + (bh / a.H) * a.sb + (bh % a.H) * a.sh + (long long)n * a.sn + 8 * c;
  gr_st16(dst, w);
}

template <int D, int BM, int BN>
struct gr_attn_bwd_lds {
  static constexpr int QT = BM * D * 2;          // one Q or dO tile
  static constexpr int STAGE = 2 * QT + 2 * BM * 4;   // Q, dO, then log2-domain L and delta
  static constexpr int KTILE = BN * D * 2;
  static constexpr int DST = BN * BM * 2;        // dS^T
  static constexpr int BYTES = 2 * STAGE + KTILE + DST;
};

template <class T, int D, int BM, int BN, bool CAUSAL>
__global__ __launch_bounds__(BN / 32 * 64) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
void gr_attn_bwd_kernel(gr_attn_bwd_args a) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  constexpr int NW = BN / 32, NT = NW * 64;
  constexpr int DS = D / 16, DB = D / 32, QJ = BM / 32;
  typedef gr_attn_bwd_lds<D, BM, BN> L;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && D % 32 == 0, "tile shape");
  static_assert(2 * BM <= NT, "one thread per statistic of a query tile");
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* const k_tile = lds + 2 * L::STAGE;
  char* const dst_tile = k_tile + L::KTILE;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nkb = a.N / BN;
  const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / nkb, kb = logical % nkb;
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
  gr_f32x16 dkt[DB], dvt[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkt[db] = (gr_f32x16)(0.f);
    dvt[db] = (gr_f32x16)(0.f);
  }

  gr_lds_loader<T, BN, D, NT, true> kl;     // K tile, read back transposed (dQ)
  gr_lds_loader<T, BM, D, NT> ql;           // Q / dO tiles: row reads and transposing reads
  kl.init(tid, a.sn);
  ql.init(tid, a.sn);
  const int qt0 = CAUSAL ? key0 / BM : 0;
  const int nqt = a.N / BM;
  auto load_tile = [&](int qt, int st) {
    char* s = lds + st * L::STAGE;
    ql.load(Q + (long long)qt * BM * a.sn, s);
    ql.load(dO + (long long)qt * BM * a.sn, s + L::QT);
    float* stat = reinterpret_cast<float*>(s + 2 * L::QT);
    const long long r0 = (long long)bh * a.N + (long long)qt * BM;
    if (tid < BM) stat[tid] = a.lse[r0 + tid] * 1.4426950408889634f;
    else if (tid < 2 * BM) stat[tid] = a.delta[r0 + tid - BM];
  };
  kl.load(K + (long long)key0 * a.sn, k_tile);
  load_tile(qt0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int qt = qt0; qt < nqt; ++qt) {
    const int st = (qt - qt0) & 1;
    // the other stage was last read before the previous iteration's closing barrier
    if (qt + 1 < nqt) load_tile(qt + 1, st ^ 1);
    const char* qs = lds + st * L::STAGE;
    const char* dos = qs + L::QT;
    const float* lse2 = reinterpret_cast<const float*>(qs + 2 * L::QT);
    const float* dlt = lse2 + BM;
    const int q0 = qt * BM;

    vec8 pb[QJ][2], dsb[QJ][2];
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      // S and dP for queries j*32..+32 (row permuted) and this wave's keys
      gr_f32x16 sa = (gr_f32x16)(0.f), dpa = (gr_f32x16)(0.f);
      const int row = j * 32 + gr_perm32(l32);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const int ch = gr_swz<D / 8>(row, 2 * ds + g);
        const vec8 qa = gr_as<vec8>(gr_ld16(qs + row * (D * 2) + ch * 16));
        const vec8 da = gr_as<vec8>(gr_ld16(dos + row * (D * 2) + ch * 16));
        sa = MF::mma32(qa, kf[ds], sa);
        dpa = MF::mma32(da, vf[ds], dpa);
      }
      // register r holds query j*32 + 8g + r (r < 8) or j*32 + 16 + 8g + r - 8
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
            float p = gr_exp2(sa[r] * c - lse2[ql_]);
            if (CAUSAL && kw0 + l32 > q0 + ql_) p = 0.f;
            p2[u] = p;
            d2[u] = p * (dpa[r] - dlt[ql_]);
          }
          pw[e >> 1] = gr_pack2<T>((T)p2[0], (T)p2[1]);
          dw[e >> 1] = gr_pack2<T>((T)d2[0], (T)d2[1]);
        }
        pb[j][hf] = gr_as<vec8>(pw);
        dsb[j][hf] = gr_as<vec8>(dw);
        // dS^T row (this lane's key), queries j*32 + 16hf + 8g .. +8: one 16-byte chunk
        const int krow = wave * 32 + l32;
        *reinterpret_cast<gr_u32x4*>(dst_tile + krow * (BM * 2) + gr_swz_tr<BM / 8>(krow, 4 * j + 2 * hf + g) * 16) = dw;
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
    __syncthreads();   // dS^T complete
    // dQ tile (BM x D) = dS K over this block's BN keys; the waves share its 32x32 blocks
#pragma unroll
    for (int bi = wave; bi < QJ * DB; bi += NW) {
      const int qj = bi / DB, db = bi % DB;
      gr_f32x16 acc = (gr_f32x16)(0.f);
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        const vec8 dsa = gr_tr_frag<T, BM, false>(dst_tile, ks * 16, qj * 32, lane);
        const vec8 kb_ = gr_tr_frag<T, D, false>(k_tile, ks * 16, db * 32, lane);
        acc = MF::mma32(dsa, kb_, acc);
      }
      float* dq = a.dq_acc + ((long long)bh * a.N + q0 + qj * 32) * D + db * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) unsafeAtomicAdd(dq + (8 * (r >> 2) + 4 * g + (r & 3)) * D, acc[r]);
    }
    __builtin_amdgcn_s_waitcnt(0);   // the next stage has landed
    __syncthreads();
  }

  // dK = scale dK^T^T, dV = dV^T^T: lane holds key kw0 + l32, d rows 8(r/4) + 4g + r%4 of block db
  T* dk = static_cast<T*>(a.dk) + base + (long long)(kw0 + l32) * a.sn;
  T* dv = static_cast<T*>(a.dv) + base + (long long)(kw0 + l32) * a.sn;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d = db * 32 + 8 * rr + 4 * g;
      gr_u32x2 wk, wv;
      wk[0] = gr_pack2<T>((T)(dkt[db][4 * rr] * a.scale), (T)(dkt[db][4 * rr + 1] * a.scale));
      wk[1] = gr_pack2<T>((T)(dkt[db][4 * rr + 2] * a.scale), (T)(dkt[db][4 * rr + 3] * a.scale));
      wv[0] = gr_pack2<T>((T)dvt[db][4 * rr], (T)dvt[db][4 * rr + 1]);
      wv[1] = gr_pack2<T>((T)dvt[db][4 * rr + 2], (T)dvt[db][4 * rr + 3]);
      *reinterpret_cast<gr_u32x2*>(dk + d) = wk;
      *reinterpret_cast<gr_u32x2*>(dv + d) = wv;
    }
}
