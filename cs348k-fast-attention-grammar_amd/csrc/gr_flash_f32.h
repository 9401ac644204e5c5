// gr_flash_f32.h -- fp32 attention forward on the fp32 matrix cores of gfx950
// (v_mfma_f32_32x32x2_f32), for the grammar's fp32 programs: keys split over
// the waves of a workgroup (merged in LDS) and, optionally, over workgroups
// (merged by a second launch).
//
//   O = softmax(scale * Q K^T) V      Q, V, O [B, H, N, D], K natural or K^T
//
// The reference's own attention workload is fp32 and small (one head,
// N = 512, d = 64: 67 MFLOP). At the fp32 matrix cores' rate one wave takes
// about 2 us per 32 x 32 block of queries x keys, so the work is spread as
// wide as the problem allows. A workgroup owns one 32-query block and NW
// consecutive chunks of BN keys, one per wave; a wave runs the online softmax
// over its chunk's 32-key blocks with its operands read straight from global
// memory into registers (the next block's loads in flight during this
// block's MFMAs). The NW partials (O, m, l) are merged through LDS, each wave
// merging a D / NW slice. With PARTS = N / (NW BN) > 1 workgroups per query
// block, each leaves its merged partial in a workspace and a second launch
// (gr_flash32_merge_body) combines them,
//   O = sum_s 2^((m_s - M) c) O_s / sum_s 2^((m_s - M) c) l_s,  M = max_s m_s.
// The workspace is module-scope device arrays the renderer sizes for the
// stage (two launches of one module must not overlap), or, behind
// gr_attn_fwd, a buffer the library keeps per (device, stream).
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

template <int D, int NW>
struct gr_flash32_lds {
  static constexpr int LD = D + 4;                       // padded row of a wave's O partial (floats)
  static constexpr int O_FLOATS = NW * 32 * LD;
  static constexpr int BYTES = (O_FLOATS + NW * 32 * 2) * 4;
};

// nkb: 32-key blocks per wave when the chunk length is only known at run time
// (the library launches: nkb = N / (32 NW PARTS)); 0 takes BN / 32.
template <int D, int BN, int NW, bool KT_LAYOUT, int PARTS>
__device__ __forceinline__ void gr_flash32_fwd_body(const gr_attn_args& a, char* lds, float* ws_o, float* ws_ml,
                                                    int nkb = 0) {
  const int KB = nkb > 0 ? nkb : BN / 32;   // 32-key blocks per wave
  constexpr int DB = D / 32;       // 32-wide head-dim blocks of O^T
  constexpr int DG = D / 8;        // groups of 8 d (4 MFMAs of 2)
  constexpr int SL = D / NW;       // head dims each wave merges
  typedef gr_flash32_lds<D, NW> L;
  static_assert(D % 32 == 0 && BN % 32 == 0 && SL % 16 == 0, "tile shape: D / NW a multiple of 16");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int lead = a.B * a.H;
  const int nqb = a.N / 32;
  const int wg = blockIdx.x;
  const int bh = wg / (nqb * PARTS);
  const int rem = wg % (nqb * PARTS);
  const int qblk = rem / PARTS, part = rem % PARTS;
  const int b = bh / a.H, h = bh % a.H;
  const float* Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
  const float* Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
  const float* Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
  float* Op = (float*)a.o + b * a.o_sb + h * a.o_sh;
  const int q0 = qblk * 32, k0 = (part * NW + wave) * 32 * KB;
  const float c = a.scale_log2;

  gr_f32x4 qf[DG];
#pragma unroll
  for (int dg = 0; dg < DG; ++dg)
    qf[dg] = *reinterpret_cast<const gr_f32x4*>(Qp + (long long)(q0 + l32) * a.q_sn + 8 * dg + 4 * g);

  // operands of one 32-key block: K (MFMA A of the scores) and V (MFMA A of P V).
  // Each lane keeps one base pointer per operand; the rest of every address
  // is wave-uniform (scalar arithmetic when the strides are run-time values).
  const float* const k_lane = KT_LAYOUT ? Kp + (long long)(4 * g) * a.k_sn + l32 : Kp + (long long)l32 * a.k_sn + 4 * g;
  const float* const v_lane = Vp + (long long)(4 * g) * a.v_sn + l32;
  auto load_k = [&](int kr, gr_f32x4 (&kf)[DG]) {
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) {
      if constexpr (KT_LAYOUT) {
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[dg][t] = k_lane[(long long)(8 * dg + t) * a.k_sn + kr];
      } else {
        kf[dg] = *reinterpret_cast<const gr_f32x4*>(k_lane + (long long)kr * a.k_sn + 8 * dg);
      }
    }
  };
  auto load_v = [&](int kr, float (&vf)[DB][16]) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int t = 0; t < 16; ++t) vf[db][t] = v_lane[(long long)(kr + 8 * (t >> 2) + (t & 3)) * a.v_sn + 32 * db];
  };

  gr_f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (gr_f32x16)(0.f);
  float m = -GR_INF, l = 0.f;
  gr_f32x4 kf[DG];
  float vf[DB][16];
  load_k(k0, kf);
  load_v(k0, vf);
#pragma unroll 1
  for (int kb = 0; kb < KB; ++kb) {
    gr_f32x4 kn[DG];
    float vn[DB][16];
    if (kb + 1 < KB) {
      load_k(k0 + 32 * (kb + 1), kn);
      load_v(k0 + 32 * (kb + 1), vn);
    }
    gr_f32x16 s = (gr_f32x16)(0.f);
#pragma unroll
    for (int dg = 0; dg < DG; ++dg)
#pragma unroll
      for (int t = 0; t < 4; ++t) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[dg][t], qf[dg][t], s, 0, 0, 0);
    // s[r]: key 8 (r / 4) + 4 g + r % 4 of the block, query q0 + l32
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
      for (int t = 0; t < 16; ++t) o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[db][t], s[t], o[db], 0, 0, 0);
    if (kb + 1 < KB) {
#pragma unroll
      for (int dg = 0; dg < DG; ++dg) kf[dg] = kn[dg];
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int t = 0; t < 16; ++t) vf[db][t] = vn[db][t];
    }
  }
  l += gr_xor32(l);

  // the NW wave partials -> LDS: O^T lane (query l32, half g) holds d =
  // 32 db + 8 (r / 4) + 4 g + r % 4; rows padded so the 16-byte writes of 16
  // consecutive queries fall on distinct banks
  float* lo = reinterpret_cast<float*>(lds);
  float* lml = lo + L::O_FLOATS;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      *reinterpret_cast<gr_f32x4*>(lo + (wave * 32 + l32) * L::LD + 32 * db + 8 * rr + 4 * g) =
          (gr_f32x4){o[db][4 * rr], o[db][4 * rr + 1], o[db][4 * rr + 2], o[db][4 * rr + 3]};
  if (g == 0) *reinterpret_cast<gr_f32x2*>(lml + (wave * 32 + l32) * 2) = (gr_f32x2){m, l};
  __syncthreads();

  // merge of the workgroup's chunks: wave w, lane (query l32, half g) takes
  // head dims SL w + 16 p + 8 g + 0..7 of its slice
  const int d0 = SL * wave + 8 * g;
  float mx = -GR_INF;
#pragma unroll
  for (int w = 0; w < NW; ++w) mx = fmaxf(mx, lml[(w * 32 + l32) * 2]);
  constexpr int PER = SL / 16;                         // 8-wide pieces per lane
  float acc[PER][8];
#pragma unroll
  for (int p = 0; p < PER; ++p)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[p][e] = 0.f;
  float L_ = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const gr_f32x2 ml = *reinterpret_cast<const gr_f32x2*>(lml + (w * 32 + l32) * 2);
    const float e = gr_exp2((ml[0] - mx) * c);
    L_ = fmaf(e, ml[1], L_);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const float* src = lo + (w * 32 + l32) * L::LD + d0 + 16 * p;
      const gr_f32x4 v0 = *reinterpret_cast<const gr_f32x4*>(src);
      const gr_f32x4 v1 = *reinterpret_cast<const gr_f32x4*>(src + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[p][i] = fmaf(e, v0[i], acc[p][i]);
        acc[p][4 + i] = fmaf(e, v1[i], acc[p][4 + i]);
      }
    }
  }
  auto store_o = [&](float Lv) {
    const float inv = 1.0f / Lv;
    float* dst = Op + (long long)(q0 + l32) * a.o_sn + d0;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      *reinterpret_cast<gr_f32x4*>(dst + 16 * p) =
          (gr_f32x4){acc[p][0] * inv, acc[p][1] * inv, acc[p][2] * inv, acc[p][3] * inv};
      *reinterpret_cast<gr_f32x4*>(dst + 16 * p + 4) =
          (gr_f32x4){acc[p][4] * inv, acc[p][5] * inv, acc[p][6] * inv, acc[p][7] * inv};
    }
  };
  if constexpr (PARTS == 1) {
    store_o(L_);
  } else {
    // this workgroup's merged partial -> workspace, for gr_flash32_merge_body
    const long long row = (long long)(part * lead + bh) * a.N + q0 + l32;
    float* wo = ws_o + row * D + d0;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      *reinterpret_cast<gr_f32x4*>(wo + 16 * p) = (gr_f32x4){acc[p][0], acc[p][1], acc[p][2], acc[p][3]};
      *reinterpret_cast<gr_f32x4*>(wo + 16 * p + 4) = (gr_f32x4){acc[p][4], acc[p][5], acc[p][6], acc[p][7]};
    }
    if (wave == 0 && g == 0) *reinterpret_cast<gr_f32x2*>(ws_ml + row * 2) = (gr_f32x2){mx, L_};
  }
}

// The second launch of a split stage: O from the PARTS partials of every
// query, O = sum_s 2^((m_s - M) c) O_s / sum_s 2^((m_s - M) c) l_s with
// M = max_s m_s. One thread per (query row, 8 head dims); the grid covers
// lead * N * D / 8 threads in workgroups of 256.
template <int D, int PARTS>
__device__ __forceinline__ void gr_flash32_merge_body(const gr_attn_args& a, const float* ws_o, const float* ws_ml) {
  constexpr int CH = D / 8;
  const int lead = a.B * a.H;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long rows = (long long)lead * a.N;
  if (idx >= rows * CH) return;
  const int ch = (int)(idx % CH);
  const long long r = idx / CH;                     // bh * N + q
  const int bh = (int)(r / a.N), q = (int)(r % a.N);
  const float c = a.scale_log2;
  float mx = -GR_INF;
#pragma unroll
  for (int s = 0; s < PARTS; ++s) mx = fmaxf(mx, ws_ml[((long long)s * rows + r) * 2]);
  float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < PARTS; ++s) {
    const gr_f32x2 ml = *reinterpret_cast<const gr_f32x2*>(ws_ml + ((long long)s * rows + r) * 2);
    const float w = gr_exp2((ml[0] - mx) * c);
    L = fmaf(w, ml[1], L);
    const float* src = ws_o + ((long long)s * rows + r) * D + ch * 8;
    const gr_f32x4 v0 = *reinterpret_cast<const gr_f32x4*>(src);
    const gr_f32x4 v1 = *reinterpret_cast<const gr_f32x4*>(src + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = fmaf(w, v0[e], acc[e]);
      acc[4 + e] = fmaf(w, v1[e], acc[4 + e]);
    }
  }
  const float inv = 1.0f / L;
  const int b = bh / a.H, h = bh % a.H;
  float* dst = (float*)a.o + b * a.o_sb + h * a.o_sh + (long long)q * a.o_sn + ch * 8;
  *reinterpret_cast<gr_f32x4*>(dst) = (gr_f32x4){acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  *reinterpret_cast<gr_f32x4*>(dst + 4) = (gr_f32x4){acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
}
