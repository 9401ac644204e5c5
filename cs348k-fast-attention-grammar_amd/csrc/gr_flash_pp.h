// gr_flash_pp.h -- "ping-pong" schedule of the flash attention forward, gfx950.
//
// Same math and data layout as gr_flash_fwd_body (transposed S^T = K Q^T and
// O^T = V^T P^T on the 32x32x16 MFMA, K rows bit-permuted in LDS, V^T tiles,
// XOR-swizzled LDS, XCD-local heads), but one workgroup is 8 waves = 256
// queries split into two groups of four that run half a key tile apart:
//
//   phase 2u   : group A  P_{u-1} V_{u-1} + S_u = K_u Q^T   (matrix cores)
//                group B  softmax of S_{u-1}                 (vector ALUs)
//   phase 2u+1 : group A  softmax of S_u                     (vector ALUs)
//                group B  P_{u-1} V_{u-1} + S_u              (matrix cores)
//
// Wave w and wave w+4 share a SIMD, so in every phase one of them keeps the
// matrix core busy while the other works through the exponentials; without
// the offset both waves of a SIMD reach the same phase together and the two
// units take turns. One barrier closes each phase. K_t and V_t live in
// two-slot LDS rings: K_{u+1} and V_u are fetched into registers in phase 2u
// and written in phase 2u+1, after their slots' previous tiles were last read
// (K_{u-1} in phase 2u-1, V_{u-2} in phase 2u-1).
//
// Non-causal only; the softmax moves its base lazily as in gr_flash_fwd_body.
#pragma once
#include "gr_flash_fwd.h"

template <class T, int D, int BN, bool KT_LAYOUT>
__device__ __forceinline__ void gr_flash_pp_body(const gr_attn_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  typedef typename MF::vec2 vec2;
  constexpr int NT = 512;          // 8 waves
  constexpr int BM = 256;
  constexpr int KB = BN / 32;
  constexpr int DB = D / 32;
  constexpr int DS = D / 16;
  typedef gr_flash_lds<D, BN> L;
  static_assert(BN % 32 == 0 && D % 32 == 0, "tile shape");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int grp = wave >> 2;
  const int nqt = a.N / BM;
  const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / nqt, qt = logical % nqt;
  const int b = bh / a.H, h = bh % a.H;

  const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
  const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
  const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
  T* Op = (T*)a.o + b * a.o_sb + h * a.o_sh;
  const int qw = qt * BM + wave * 32;
  const float c = a.scale_log2;

  vec8 qf[1][DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
    qf[0][ds] = gr_as<vec8>(gr_ld16(Qp + (long long)(qw + l32) * a.q_sn + ds * 16 + 8 * g));

  gr_f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (gr_f32x16)(0.f);
  float m = -GR_INF, l = 0.f;
  gr_f32x16 s[KB][1];
  vec8 pf[KB][2];

  char* ks0 = lds;
  char* vt0 = lds + 2 * L::KS;
  typedef gr_row_loader<T, BN, D, NT, true> KRows;
  typedef gr_tr_loader<T, D, BN, NT, true> KCols;
  typedef gr_tr_loader<T, BN, D, NT, false> VLoad;
  typename gr_cond<KT_LAYOUT, KCols, KRows>::type kl;
  VLoad vl;
  kl.init(tid, a.k_sn);
  vl.init(tid, a.v_sn);
  const long long k_tile = KT_LAYOUT ? (long long)BN : (long long)BN * a.k_sn;
  const long long v_tile = (long long)BN * a.v_sn;
  const int ntile = a.N / BN;

  kl.gload(Kp, tid);
  kl.sstore(ks0, tid);
  __syncthreads();

  const int nph = 2 * ntile + 2;
  for (int ph = 0; ph < nph; ++ph) {
    const int u = ph >> 1;
    if ((ph & 1) == 0) {
      if (u + 1 < ntile) kl.gload(Kp + (u + 1) * k_tile, tid);
      if (u < ntile) vl.gload(Vp + u * v_tile, tid);
    }
    const int my = ph - grp;            // this group's own phase
    if (my >= 0) {
      const int t = my >> 1;
      if ((my & 1) == 0) {
        // matrix phase: P_{t-1} V_{t-1}, then S_t
        if (t >= 1) {
          const char* vt = vt0 + ((t - 1) & 1) * L::VT;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
              for (int db = 0; db < DB; ++db) {
                const int row = db * 32 + l32;
                const vec8 vf = gr_as<vec8>(gr_ld16(vt + row * (BN * 2) + gr_swz<BN / 8>(row, 4 * kb + 2 * hf + g) * 16));
                o[db] = MF::mma32(vf, pf[kb][hf], o[db]);
              }
        }
        if (t < ntile) gr_flash_qk<T, D, BN, 1>(s, ks0 + (t & 1) * L::KS, qf, l32, g);
      } else if (t < ntile) {
        // vector phase: online softmax of S_t into P_t (registers)
        float mt = -GR_INF;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][0][r]);
        mt = fmaxf(mt, gr_xor32(mt));
        const float mn = fmaxf(m, mt);
        if (gr_any(mn > m + GR_RESCALE_LOG2 / c)) {
          const float alpha = gr_exp2((m - mn) * c);
          l *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[db] *= alpha;
          m = mn;
        }
        const float nmc = -((m == -GR_INF) ? 0.f : m) * c;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            gr_u32x4 pw;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              const float p0 = gr_exp2(fmaf(s[kb][0][8 * hf + e], c, nmc));
              const float p1 = gr_exp2(fmaf(s[kb][0][8 * hf + e + 1], c, nmc));
              const vec2 pp = __builtin_convertvector((gr_f32x2){p0, p1}, vec2);
              l = MF::sum2(pp, l);
              pw[e >> 1] = __builtin_bit_cast(unsigned int, pp);
            }
            pf[kb][hf] = gr_as<vec8>(pw);
          }
      }
    }
    if (ph & 1) {
      if (u + 1 < ntile) kl.sstore(ks0 + ((u + 1) & 1) * L::KS, tid);
      if (u < ntile) vl.sstore(vt0 + (u & 1) * L::VT, tid);
    }
    __syncthreads();
  }

  const float lt = l + gr_xor32(l);
  const float inv = 1.0f / lt;
  T* orow = Op + (long long)(qw + l32) * a.o_sn;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const unsigned int w0 = gr_pack2<T>((T)(o[db][4 * rr + 0] * inv), (T)(o[db][4 * rr + 1] * inv));
      const unsigned int w1 = gr_pack2<T>((T)(o[db][4 * rr + 2] * inv), (T)(o[db][4 * rr + 3] * inv));
      gr_u32x2 w = {w0, w1};
      *reinterpret_cast<gr_u32x2*>(orow + db * 32 + 8 * rr + 4 * g) = w;
    }
}

template <class T, int D, int BN, bool KT_LAYOUT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void gr_flash_pp_kernel(gr_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash_pp_body<T, D, BN, KT_LAYOUT>(a, gr_lds);
}
