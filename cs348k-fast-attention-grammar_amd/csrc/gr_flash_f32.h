// gr_flash_f32.h -- fp32 attention forward on the fp32 matrix cores of gfx950
// (v_mfma_f32_32x32x2_f32), for the grammar's fp32 programs: one launch,
// keys split over waves, partials merged by the last wave of each query block.
//
//   O = softmax(scale * Q K^T) V      Q, V, O [B, H, N, D], K natural or K^T
//
// The reference's own attention workload is fp32 and small (one head,
// N = 512, d = 64: 67 MFLOP). At the fp32 matrix cores' rate one wave takes
// about 2 us per 32 x 32 block of queries x keys, so the work is spread as
// wide as the problem allows: every wave owns one 32-query block and one
// chunk of BN keys, runs the online softmax over that chunk's 32-key blocks
// with its operands read straight from global memory (no LDS, no barrier),
// and leaves an unnormalised partial (O, m, l). The last wave to finish a
// query block (a device-scope counter) merges the block's partials,
//   O = sum_s 2^((m_s - M) c) O_s / sum_s 2^((m_s - M) c) l_s,  M = max_s m_s,
// writes O and resets the counter for the next launch. Workspace and counters
// are module-scope device arrays the renderer sizes for the stage (zero at
// load); two launches of one module must not overlap.
//
//  * Transposed form as in gr_flash_fwd_body: S^T = K Q^T, O^T = V^T P^T. A
//    32x32x2 MFMA contracts one index per half-wave: for d the lane of half g
//    takes d = 8 dg + 4 g + t in MFMA t of group dg (one 16-byte load of Q and
//    of a natural K row per group); for the keys the score accumulators are
//    the P operand as they stand (accumulator r is key 8 (r / 4) + 4 g + r % 4,
//    MFMA t takes r = t), and V's row of that key is read at d = lane % 32.
//  * Lane-local softmax (each lane owns one query and half the block's keys):
//    one exchange with the other half-wave per block for the max.
#pragma once
#include "gr_flash_fwd.h"

template <int D, int BN, int NW, bool KT_LAYOUT>
__device__ __forceinline__ void gr_flash32_fwd_body(const gr_attn_args& a, float* ws_o, float* ws_ml,
                                                    unsigned int* cnt) {
  constexpr int KB = BN / 32;      // 32-key blocks per wave
  constexpr int DB = D / 32;       // 32-wide head-dim blocks of O^T
  constexpr int DG = D / 8;        // groups of 8 d (4 MFMAs of 2)
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int lead = a.B * a.H;
  const int nqb = a.N / 32, parts = a.N / BN, qgroups = nqb / NW;
  const int wg = blockIdx.x;
  const int bh = wg / (parts * qgroups);
  const int rem = wg % (parts * qgroups);
  const int part = rem / qgroups;
  const int qblk = (rem % qgroups) * NW + wave;
  const int b = bh / a.H, h = bh % a.H;
  const float* Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
  const float* Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
  const float* Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
  float* Op = (float*)a.o + b * a.o_sb + h * a.o_sh;
  const int q0 = qblk * 32, k0 = part * BN;
  const float c = a.scale_log2;

  gr_f32x4 qf[DG];
#pragma unroll
  for (int dg = 0; dg < DG; ++dg)
    qf[dg] = *reinterpret_cast<const gr_f32x4*>(Qp + (long long)(q0 + l32) * a.q_sn + 8 * dg + 4 * g);

  gr_f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (gr_f32x16)(0.f);
  float m = -GR_INF, l = 0.f;
#pragma unroll 1
  for (int kb = 0; kb < KB; ++kb) {
    const int kr = k0 + 32 * kb;
    gr_f32x16 s = (gr_f32x16)(0.f);
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) {
      gr_f32x4 kf;
      if constexpr (KT_LAYOUT) {
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[t] = Kp[(long long)(8 * dg + 4 * g + t) * a.k_sn + kr + l32];
      } else {
        kf = *reinterpret_cast<const gr_f32x4*>(Kp + (long long)(kr + l32) * a.k_sn + 8 * dg + 4 * g);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[t], qf[dg][t], s, 0, 0, 0);
    }
    // s[r]: key kr + 8 (r / 4) + 4 g + r % 4 of query q0 + l32
    float mt = -GR_INF;
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = fmaxf(mt, gr_xor32(mt));
    const float mn = fmaxf(m, mt);
    const float alpha = gr_exp2((m - mn) * c);   // m = -inf -> 0
    l *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;
    m = mn;
    const float mc = m * c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = gr_exp2(fmaf(s[r], c, -mc));
      l += s[r];
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float vf = Vp[(long long)(kr + 8 * (t >> 2) + 4 * g + (t & 3)) * a.v_sn + 32 * db + l32];
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf, s[t], o[db], 0, 0, 0);
      }
  }
  l += gr_xor32(l);

  // this wave's partial: O^T lane (query l32, half g) holds d = 32 db +
  // 8 (r / 4) + 4 g + r % 4
  const long long row = (long long)(part * lead + bh) * a.N + q0 + l32;
  float* wo = ws_o + row * D;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      *reinterpret_cast<gr_f32x4*>(wo + 32 * db + 8 * rr + 4 * g) =
          (gr_f32x4){o[db][4 * rr], o[db][4 * rr + 1], o[db][4 * rr + 2], o[db][4 * rr + 3]};
  if (g == 0) *reinterpret_cast<gr_f32x2*>(ws_ml + row * 2) = (gr_f32x2){m, l};
  __threadfence();   // the partial is visible device-wide before it is counted
  unsigned int arrived = 0u;
  if (lane == 0) arrived = atomicAdd(cnt + (long long)bh * nqb + qblk, 1u);
  arrived = __shfl(arrived, 0, 64);
  if (arrived != (unsigned int)(parts - 1)) return;
  __threadfence();   // every counted partial is visible to this wave

  // merge: lane (query l32, half g) builds d in [D/2 g, D/2 (g + 1))
  constexpr int HD = D / 2;
  float mx = -GR_INF;
  for (int s = 0; s < parts; ++s) mx = fmaxf(mx, ws_ml[((long long)(s * lead + bh) * a.N + q0 + l32) * 2]);
  float acc[HD];
#pragma unroll
  for (int i = 0; i < HD; ++i) acc[i] = 0.f;
  float L = 0.f;
  for (int s = 0; s < parts; ++s) {
    const long long r2 = (long long)(s * lead + bh) * a.N + q0 + l32;
    const gr_f32x2 ml = *reinterpret_cast<const gr_f32x2*>(ws_ml + r2 * 2);
    const float w = gr_exp2((ml[0] - mx) * c);
    L = fmaf(w, ml[1], L);
    const float* src = ws_o + r2 * D + HD * g;
#pragma unroll
    for (int i = 0; i < HD; i += 4) {
      const gr_f32x4 v = *reinterpret_cast<const gr_f32x4*>(src + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i + e] = fmaf(w, v[e], acc[i + e]);
    }
  }
  const float inv = 1.0f / L;
  float* dst = Op + (long long)(q0 + l32) * a.o_sn + HD * g;
#pragma unroll
  for (int i = 0; i < HD; i += 4)
    *reinterpret_cast<gr_f32x4*>(dst + i) = (gr_f32x4){acc[i] * inv, acc[i + 1] * inv, acc[i + 2] * inv, acc[i + 3] * inv};
  if (lane == 0) cnt[(long long)bh * nqb + qblk] = 0u;   // ready for the next launch
}
