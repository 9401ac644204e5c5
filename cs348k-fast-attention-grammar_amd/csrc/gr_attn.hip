// gr_attn.hip -- prebuilt instances of the hand-written CDNA4 attention
// forward (gr_flash_fwd.h) behind gr_attn_fwd(), plus the MFMA layout self-test.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gr_flash_fwd.h"
#include "gr_host.h"
#include "grammar_rt.h"

namespace {

template <class T, int D, int BN, int NW, int QB, bool CAUSAL, bool KT, bool PIPE = false>
int launch_flash(const gr_attn_args& a, hipStream_t st) {
  constexpr int BM = NW * QB * 32;
  constexpr int LDS = gr_flash_lds<D, BN>::BYTES;
  // K/V tiles go straight into LDS when they give every thread the same
  // number of 16-byte chunks (D * BN / 8 per tile), else through registers.
  constexpr bool DIRECT = (D * BN / 8) % (NW * 64) == 0;
  if (a.N % BM != 0 || a.N % BN != 0)
    return gr::fail(GR_E_ARG, "gr_attn_fwd: N=%d must be a multiple of block_m=%d and block_n=%d", a.N, BM, BN);
  const long long nblk = (long long)a.B * a.H * (a.N / BM);
  if (nblk <= 0 || nblk > 0x7fffffffLL) return gr::fail(GR_E_ARG, "gr_attn_fwd: grid size %lld out of range", nblk);
  hipLaunchKernelGGL((gr_flash_fwd_kernel<T, D, BN, NW, QB, CAUSAL, KT, PIPE, true, DIRECT>), dim3((unsigned)nblk),
                     dim3(NW * 64), LDS, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd launch");
}

// Tile configurations compiled into the library: (block_m, block_n) ->
// (waves, query blocks per wave, key tile). One wave per 32 queries.
// block_m 0 / block_n 0 pick the largest tiles that divide N (256 x 128 at
// D = 64, 256 x 64 at D = 128).
template <class T, int D, bool CAUSAL, bool KT>
int dispatch_tiles(const gr_attn_args& a, int bm, int bn, hipStream_t st) {
  if (bm == 0) bm = a.N % 256 == 0 ? 256 : a.N % 128 == 0 ? 128 : 64;
  if (bn == 0) bn = (D == 64 && a.N % 128 == 0) ? 128 : a.N % 64 == 0 ? 64 : 32;
  if (bm == 256 && bn == 64) return launch_flash<T, D, 64, 8, 1, CAUSAL, KT>(a, st);
  if (bm == 256 && bn == 32) return launch_flash<T, D, 32, 8, 1, CAUSAL, KT>(a, st);
  if (bm == 128 && bn == 64) return launch_flash<T, D, 64, 4, 1, CAUSAL, KT>(a, st);
  if (bm == 128 && bn == 32) return launch_flash<T, D, 32, 4, 1, CAUSAL, KT>(a, st);
  if (bm == 64 && bn == 64) return launch_flash<T, D, 64, 2, 1, CAUSAL, KT>(a, st);
  if (bm == 64 && bn == 32) return launch_flash<T, D, 32, 2, 1, CAUSAL, KT>(a, st);
  // block_m = 129 / 257 select the software-pipelined schedule (128 / 256 queries).
  if (bm == 129 && bn == 64) return launch_flash<T, D, 64, 4, 1, CAUSAL, KT, true>(a, st);
  if (bm == 129 && bn == 32) return launch_flash<T, D, 32, 4, 1, CAUSAL, KT, true>(a, st);
  if (bm == 257 && bn == 64) return launch_flash<T, D, 64, 8, 1, CAUSAL, KT, true>(a, st);
  if (bm == 257 && bn == 32) return launch_flash<T, D, 32, 8, 1, CAUSAL, KT, true>(a, st);
  if constexpr (D == 64) {
    if (bm == 256 && bn == 128) return launch_flash<T, D, 128, 8, 1, CAUSAL, KT>(a, st);
    if (bm == 128 && bn == 128) return launch_flash<T, D, 128, 4, 1, CAUSAL, KT>(a, st);
    if (bm == 129 && bn == 128) return launch_flash<T, D, 128, 4, 1, CAUSAL, KT, true>(a, st);
  }
  return gr::fail(GR_E_ARG, "gr_attn_fwd: unsupported tile (block_m=%d, block_n=%d) for D=%d", bm, bn, D);
}

template <class T>
int dispatch_shape(const gr_attn_args& a, int D, bool causal, bool kt, int bm, int bn, hipStream_t st) {
#define GR_CASE(DD, C, K)                                                          \
  if (D == DD && causal == C && kt == K) return dispatch_tiles<T, DD, C, K>(a, bm, bn, st);
  GR_CASE(64, false, false)
  GR_CASE(64, false, true)
  GR_CASE(64, true, false)
  GR_CASE(64, true, true)
  GR_CASE(128, false, false)
  GR_CASE(128, false, true)
  GR_CASE(128, true, false)
  GR_CASE(128, true, true)
#undef GR_CASE
  return gr::fail(GR_E_ARG, "gr_attn_fwd: head dim D=%d unsupported (64 or 128)", D);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

__global__ void gr_selftest_mfma32_kernel(const _Float16* A, const _Float16* B, float* Dm) {
  const int l = threadIdx.x, l32 = l & 31, g = l >> 5;
  gr_f16x8 a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = A[l32 * 16 + 8 * g + e];       // A[m][k], m = l % 32, k in group l / 32
    b[e] = B[(8 * g + e) * 32 + l32];     // B[k][n], n = l % 32
  }
  gr_f32x16 acc = (gr_f32x16)(0.f);
  acc = gr_mfma<_Float16>::mma32(a, b, acc);
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r / 4) + 4 * g + (r % 4);
    Dm[m * 32 + l32] = acc[r];
  }
}

}  // namespace

extern "C" int gr_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int N,
                           int D, const long long* qs, const long long* ks, const long long* vs, const long long* os,
                           int k_transposed, int causal, float scale, int block_m, int block_n, void* stream) {
  if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return gr::fail(GR_E_ARG, "gr_attn_fwd: null argument");
  if (B <= 0 || H <= 0 || N <= 0) return gr::fail(GR_E_ARG, "gr_attn_fwd: B, H, N must be positive");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return gr::fail(GR_E_ARG, "gr_attn_fwd: base pointers must be 16-byte aligned");
  const long long* all[4] = {qs, ks, vs, os};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      if (all[t][i] < 0 || (all[t][i] % 8) != 0)
        return gr::fail(GR_E_ARG, "gr_attn_fwd: strides must be non-negative multiples of 8 elements");
  if (!(scale > 0.f)) return gr::fail(GR_E_ARG, "gr_attn_fwd: scale must be positive");
  gr_attn_args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.q_sb = qs[0]; a.q_sh = qs[1]; a.q_sn = qs[2];
  a.k_sb = ks[0]; a.k_sh = ks[1]; a.k_sn = ks[2];
  a.v_sb = vs[0]; a.v_sh = vs[1]; a.v_sn = vs[2];
  a.o_sb = os[0]; a.o_sh = os[1]; a.o_sn = os[2];
  a.B = B;
  a.H = H;
  a.N = N;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GR_F16) return dispatch_shape<_Float16>(a, D, causal != 0, k_transposed != 0, block_m, block_n, st);
  if (dtype == GR_BF16) return dispatch_shape<__bf16>(a, D, causal != 0, k_transposed != 0, block_m, block_n, st);
  return gr::fail(GR_E_ARG, "gr_attn_fwd: dtype %d unsupported (GR_F16 or GR_BF16)", dtype);
}

extern "C" int gr_selftest_mfma32(const void* a, const void* b, float* d, void* stream) {
  if (!a || !b || !d) return gr::fail(GR_E_ARG, "gr_selftest_mfma32: null argument");
  hipLaunchKernelGGL(gr_selftest_mfma32_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const _Float16*)a,
                     (const _Float16*)b, d);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_selftest_mfma32 launch");
}
