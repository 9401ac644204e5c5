// gr_flash_decode.h -- attention for a few queries per head (decode steps):
// a streaming kernel that reads K and V once, straight into registers.
//
// With one to four queries the MFMA tiles of the flash body would compute 32
// query rows for every real one, and its LDS-staged key tiles cap the bytes in
// flight per compute unit. Here a step is HBM-bound (K and V are read once), so
// the kernel is shaped for bandwidth instead:
//  * D/8 lanes hold one key row (16 bytes each), so a wave reads 64/(D/8)
//    consecutive rows -- 1 KiB of contiguous memory -- per load instruction;
//    U such loads of K and U of V per iteration, and the next iteration's are
//    issued before this one is used (two register buffers).
//  * Scores are dot products on the VALU in fp32 (the query pre-scaled into
//    exponent units, c = scale log2(e)), reduced across a row's lanes by
//    shuffles; the online softmax runs per iteration of 64/(D/8)*U keys.
//  * A workgroup (NWV waves) takes one head and one part of the keys (grid.y
//    = key parts); its waves take consecutive slices of the part and merge
//    through LDS. With more than one part each writes its unnormalised O and
//    (max, row sum) and gr_attn_combine_kernel merges them, as for the flash
//    body's key split.
#pragma once
#include "gr_flash_fwd.h"

// NWV waves per workgroup, NQ >= a.Nq query slots, U key-row loads of K and
// of V per lane and iteration.
template <class T, int D, int NQ, int U, int NWV>
__device__ __forceinline__ void gr_attn_decode_stream_body(const gr_attn_args& a) {
  constexpr int LPK = D / 8;        // lanes per key row
  constexpr int KPR = 64 / LPK;     // key rows per wave load
  constexpr int KPI = KPR * U;      // keys per wave iteration
  typedef T t8 __attribute__((ext_vector_type(8)));
  typedef float f8 __attribute__((ext_vector_type(8)));
  __shared__ float xm[NWV][NQ][D + 2];   // per wave: O (D), then max and row sum

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ch = lane % LPK, grp = lane / LPK;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int Nq = a.Nq;
  const int key0 = blockIdx.y * a.kchunk;
  const int kend = gr_imin(a.N, key0 + a.kchunk);
  const T* Qp = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* Kp = static_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh;
  const T* Vp = static_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;
  const float c = a.scale_log2;

  f8 qv[NQ], o[NQ];
  float m[NQ], l[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const int qrow = qi < Nq ? qi : Nq - 1;
    qv[qi] = __builtin_convertvector(gr_as<t8>(gr_ld16(Qp + (long long)qrow * a.q_sn + ch * 8)), f8) * c;
    o[qi] = (f8)(0.f);
    m[qi] = -GR_INF;
    l[qi] = 0.f;
  }

  // this wave's keys: a 1/NWV slice of the part, a whole number of iterations
  const int per = ((kend - key0 + NWV * KPI - 1) / (NWV * KPI)) * KPI;
  const int kw0 = key0 + wave * per;
  const int kw1 = gr_imin(kend, kw0 + per);

  auto load = [&](int kw, gr_u32x4 (&kr)[U], gr_u32x4 (&vr)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long key = gr_imin(kw + u * KPR + grp, kend - 1);   // rows past the part: a copy, masked
      kr[u] = gr_ld16(Kp + key * a.k_sn + ch * 8);
      vr[u] = gr_ld16(Vp + key * a.v_sn + ch * 8);
    }
  };
  auto process = [&](int kw, const gr_u32x4 (&kr)[U], const gr_u32x4 (&vr)[U]) {
    float s[NQ][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f8 kf = __builtin_convertvector(gr_as<t8>(kr[u]), f8);
      const bool live = kw + u * KPR + grp < kw1;
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qv[qi][e], kf[e], d);
#pragma unroll
        for (int off = 1; off < LPK; off <<= 1) d += __shfl_xor(d, off, 64);
        s[qi][u] = live ? d : -GR_INF;
      }
    }
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      float mx = s[qi][0];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[qi][u]);
#pragma unroll
      for (int off = LPK; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float mn = fmaxf(m[qi], mx);
      const float base = mn == -GR_INF ? 0.f : mn;   // no live key yet: p and alpha are 0
      const float alpha = gr_exp2(m[qi] - base);
      l[qi] *= alpha;
      o[qi] *= alpha;
      m[qi] = mn;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = gr_exp2(s[qi][u] - base);
        l[qi] += p;
        o[qi] += p * __builtin_convertvector(gr_as<t8>(vr[u]), f8);
      }
    }
  };

  gr_u32x4 ka[U], va[U], kb[U], vb[U];
  if (kw0 < kw1) load(kw0, ka, va);
  for (int kw = kw0; kw < kw1; kw += 2 * KPI) {
    if (kw + KPI < kw1) load(kw + KPI, kb, vb);
    process(kw, ka, va);
    if (kw + KPI < kw1) {
      if (kw + 2 * KPI < kw1) load(kw + 2 * KPI, ka, va);
      process(kw + KPI, kb, vb);
    }
  }

  // merge the wave's key rows (lane groups), then the workgroup's waves
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
      l[qi] += __shfl_xor(l[qi], off, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[qi][e] += __shfl_xor(o[qi][e], off, 64);
    }
    if (grp == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xm[wave][qi][ch * 8 + e] = o[qi][e];
      if (ch == 0) {
        xm[wave][qi][D] = m[qi];
        xm[wave][qi][D + 1] = l[qi];
      }
    }
  }
  __syncthreads();
  // thread t: query t / LPK, 8 head dims (t % LPK) * 8
  const int t = threadIdx.x, qi = t / LPK, c8 = (t % LPK) * 8;
  if (qi >= Nq || qi >= NQ) return;
  float M = -GR_INF;
#pragma unroll
  for (int w = 0; w < NWV; ++w) M = fmaxf(M, xm[w][qi][D]);
  const float mb = M == -GR_INF ? 0.f : M;
  float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    const float wt = gr_exp2(xm[w][qi][D] - mb);
    L += wt * xm[w][qi][D + 1];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += wt * xm[w][qi][c8 + e];
  }
  if (gridDim.y == 1) {
    const float inv = 1.0f / L;
    gr_u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = gr_pack2f<T>(acc[2 * e] * inv, acc[2 * e + 1] * inv);
    T* orow = static_cast<T*>(a.o) + b * a.o_sb + h * a.o_sh + (long long)qi * a.o_sn;
    gr_st16(orow + c8, out);
  } else {
    // partial of key part blockIdx.y: unnormalised O and (max in q.k units, row sum)
    const long long row = (long long)bh * Nq + qi;
    const long long part = (long long)blockIdx.y * a.B * a.H * Nq + row;
    float* po = a.part_o + part * D + c8;
    *reinterpret_cast<gr_f32x4*>(po) = (gr_f32x4){acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<gr_f32x4*>(po + 4) = (gr_f32x4){acc[4], acc[5], acc[6], acc[7]};
    if (c8 == 0) *reinterpret_cast<gr_f32x2*>(a.part_ml + part * 2) = (gr_f32x2){M / c, L};
  }
}

template <class T, int D, int NQ, int U, int NWV = 4>
__global__ __launch_bounds__(NWV * 64) void gr_attn_decode_stream_kernel(gr_attn_args a) {
  gr_attn_decode_stream_body<T, D, NQ, U, NWV>(a);
}
