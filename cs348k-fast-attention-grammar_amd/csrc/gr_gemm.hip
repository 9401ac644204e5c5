// gr_gemm.hip -- prebuilt instances of the MFMA GEMM with fused epilogue
// (gr_gemm.h) behind gr_gemm(), and the two-GEMM MLP block gr_mlp_fwd().
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gr_gemm.h"
#include "gr_gemm_f32.h"
#include "gr_host.h"
#include "grammar_rt.h"

namespace {

template <class T, int BM, int BN, int BK, int WGM, int WGN, bool KM, int EPI>
int launch_gemm(const gr_gemm_args& a, int batch, hipStream_t st) {
  typedef gr_gemm_cfg<BM, BN, BK, WGM, WGN> G;
  if (a.K % BK)
    return gr::fail(GR_E_ARG, "gr_gemm: K=%d must be a multiple of the k tile %d", a.K, BK);
  const long long nblk = (long long)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (nblk <= 0 || nblk > 0x7fffffffLL || batch > 65535)
    return gr::fail(GR_E_ARG, "gr_gemm: grid (%lld tiles, batch %d) out of range", nblk, batch);
  hipLaunchKernelGGL((gr_gemm_kernel<T, BM, BN, BK, WGM, WGN, KM, EPI>), dim3((unsigned)nblk, (unsigned)batch),
                     dim3(G::NT), G::LDS, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_gemm launch");
}

// Compute units of the current device (0 if unknown), read once per device.
int cu_count() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cache[dev] = n;
  }
  return cache[dev];
}

// The 256 x 256 tile: four waves (one per SIMD) of 128 x 128, the
// hand-ordered main loop of gr_gemm_w4_body, one workgroup per CU. When the
// last round of workgroups would leave more than half of the CUs idle (X W1
// of the C4 MLP: 1,376 tiles on 256 CUs, a sixth round of 96), the columns
// past the whole rounds go to a second launch of the same body on 256 x 128
// tiles (waves of 128 x 64), if those fit in one round: 1,280 + 192 there.
template <class T, bool KM, int EPI, int BK>
int launch_gemm_w4(const gr_gemm_args& a, int batch, hipStream_t st) {
  if (a.K % BK)
    return gr::fail(GR_E_ARG, "gr_gemm: K=%d must be a multiple of the k tile %d", a.K, BK);
  const int mt = (a.M + 255) / 256, nt = (a.N + 255) / 256;
  const long long nblk = (long long)mt * nt;
  if (nblk <= 0 || nblk > 0x7fffffffLL || batch > 65535)
    return gr::fail(GR_E_ARG, "gr_gemm: grid (%lld tiles, batch %d) out of range", nblk, batch);
  const int cus = cu_count();
  if (batch == 1 && cus > 0 && nblk > cus) {
    const long long rounds = (nblk + cus - 1) / cus;
    const long long last = nblk - (rounds - 1) * cus;            // workgroups of the last round
    const int nt_main = (int)((rounds - 1) * cus / mt);          // column tiles of the whole rounds
    const int col0 = nt_main * 256;
    const long long rest = (long long)mt * ((a.N - col0 + 127) / 128);
    if (2 * last <= cus && nt_main > 0 && nt_main < nt && rest <= cus) {
      gr_gemm_args m = a, r = a;
      m.N = col0;
      r.N = a.N - col0;
      r.b = static_cast<const T*>(a.b) + (KM ? (long long)col0 * a.b_s : (long long)col0);
      r.c = static_cast<T*>(a.c) + col0;
      if (a.r) r.r = static_cast<const T*>(a.r) + col0;
      hipLaunchKernelGGL((gr_gemm_w4_kernel<T, KM, EPI, BK>), dim3((unsigned)((long long)mt * nt_main)), dim3(256),
                         gr_gemm_w4_lds<BK>::value, st, m);
      const int rc = gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_gemm launch");
      if (rc) return rc;
      hipLaunchKernelGGL((gr_gemm_w4_kernel<T, KM, EPI, BK, 128>), dim3((unsigned)rest), dim3(256),
                         (gr_gemm_w4_lds<BK, 128>::value), st, r);
      return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_gemm launch");
    }
  }
  hipLaunchKernelGGL((gr_gemm_w4_kernel<T, KM, EPI, BK>), dim3((unsigned)nblk, (unsigned)batch), dim3(256),
                     gr_gemm_w4_lds<BK>::value, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_gemm launch");
}

// (block_m, block_n) -> (k tile, wave grid) compiled into the library; the
// 128x128 and 256x256 tiles take 64-deep k tiles when K allows, else 32.
template <class T, bool KM, int EPI>
int dispatch_tile(const gr_gemm_args& a, int batch, int bm, int bn, hipStream_t st) {
  if (bm == 0) bm = 256;
  if (bn == 0) bn = 256;
  const bool k64 = a.K % 64 == 0;
  if (bm == 128 && bn == 128)
    return k64 ? launch_gemm<T, 128, 128, 64, 2, 2, KM, EPI>(a, batch, st)
               : launch_gemm<T, 128, 128, 32, 2, 2, KM, EPI>(a, batch, st);
  if (bm == 256 && bn == 128) return launch_gemm<T, 256, 128, 32, 2, 2, KM, EPI>(a, batch, st);
  if (bm == 128 && bn == 256) return launch_gemm<T, 128, 256, 32, 2, 2, KM, EPI>(a, batch, st);
  if (bm == 256 && bn == 256)
    return k64 ? launch_gemm_w4<T, KM, EPI, 64>(a, batch, st) : launch_gemm_w4<T, KM, EPI, 32>(a, batch, st);
  return gr::fail(GR_E_ARG, "gr_gemm: unsupported tile (block_m=%d, block_n=%d)", bm, bn);
}

template <class T>
int dispatch(const gr_gemm_args& a, int batch, bool km, int epi, int bm, int bn, hipStream_t st) {
#define GR_CASE(K, E) \
  if (km == K && epi == E) return dispatch_tile<T, K, E>(a, batch, bm, bn, st);
  GR_CASE(false, GR_EPI_NONE)
  GR_CASE(false, GR_EPI_RELU)
  GR_CASE(false, GR_EPI_SILU)
  GR_CASE(true, GR_EPI_NONE)
  GR_CASE(true, GR_EPI_RELU)
  GR_CASE(true, GR_EPI_SILU)
#undef GR_CASE
  return gr::fail(GR_E_ARG, "gr_gemm: epilogue %d unsupported", epi);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// fp32 on the fp32 matrix cores (gr_gemm_f32.h): (block_m, block_n) in
// {32, 64, 128}^2, one wave per 32 rows / columns up to 2 x 2 waves; k tile 32
// when K allows, else 16 or 8. M and N must be multiples of the tile.
template <int BM, int BN, bool KM, int EPI>
int launch_gemm_f32(const gr_gemm_args& a, int batch, hipStream_t st) {
  constexpr int WGM = BM >= 64 ? 2 : 1, WGN = BN >= 64 ? 2 : 1;
  if (a.M % BM || a.N % BN)
    return gr::fail(GR_E_ARG, "gr_gemm: fp32 needs M=%d, N=%d multiples of the tile %dx%d", a.M, a.N, BM, BN);
  const long long nblk = (long long)(a.M / BM) * (a.N / BN);
  if (nblk > 0x7fffffffLL || batch > 65535) return gr::fail(GR_E_ARG, "gr_gemm: grid out of range");
#define GR_F32K(BK)                                                                                        \
  hipLaunchKernelGGL((gr_gemm_f32_kernel<BM, BN, BK, WGM, WGN, KM, EPI>), dim3((unsigned)nblk, (unsigned)batch), \
                     dim3(WGM * WGN * 64), (gr_gemm_f32_cfg<BM, BN, BK, WGM, WGN, KM>::LDS), st, a)
  if (a.K % 32 == 0) GR_F32K(32);
  else if (a.K % 16 == 0) GR_F32K(16);
  else if (a.K % 8 == 0) GR_F32K(8);
  else return gr::fail(GR_E_ARG, "gr_gemm: fp32 needs K=%d a multiple of 8", a.K);
#undef GR_F32K
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_gemm launch");
}

template <bool KM, int EPI>
int dispatch_f32_tile(const gr_gemm_args& a, int batch, int bm, int bn, hipStream_t st) {
  if (bm == 0) bm = a.M % 128 == 0 ? 128 : a.M % 64 == 0 ? 64 : 32;
  if (bn == 0) bn = a.N % 128 == 0 ? 128 : a.N % 64 == 0 ? 64 : 32;
#define GR_T(M_, N_) \
  if (bm == M_ && bn == N_) return launch_gemm_f32<M_, N_, KM, EPI>(a, batch, st);
  GR_T(32, 32) GR_T(32, 64) GR_T(32, 128) GR_T(64, 32) GR_T(64, 64) GR_T(64, 128)
  GR_T(128, 32) GR_T(128, 64) GR_T(128, 128)
#undef GR_T
  return gr::fail(GR_E_ARG, "gr_gemm: unsupported fp32 tile (block_m=%d, block_n=%d)", bm, bn);
}

int dispatch_f32(const gr_gemm_args& a, int batch, bool km, int epi, int bm, int bn, hipStream_t st) {
#define GR_CASE(K, E) \
  if (km == K && epi == E) return dispatch_f32_tile<K, E>(a, batch, bm, bn, st);
  GR_CASE(false, GR_EPI_NONE)
  GR_CASE(false, GR_EPI_RELU)
  GR_CASE(false, GR_EPI_SILU)
  GR_CASE(true, GR_EPI_NONE)
  GR_CASE(true, GR_EPI_RELU)
  GR_CASE(true, GR_EPI_SILU)
#undef GR_CASE
  return gr::fail(GR_E_ARG, "gr_gemm: epilogue %d unsupported", epi);
}

}  // namespace

extern "C" int gr_gemm(const void* a, const void* b, void* c, int dtype, int batch, int M, int N, int K,
                       const long long* a_strides, const long long* b_strides, const long long* c_strides,
                       int b_kmajor, int epilogue, float alpha, int block_m, int block_n, void* stream) {
  if (!a || !b || !c || !a_strides || !b_strides || !c_strides) return gr::fail(GR_E_ARG, "gr_gemm: null argument");
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0) return gr::fail(GR_E_ARG, "gr_gemm: sizes must be positive");
  if (dtype != GR_F32 && (N % 8 != 0 || K % 32 != 0))
    return gr::fail(GR_E_ARG, "gr_gemm: N=%d must be a multiple of 8 and K=%d a multiple of 32", N, K);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return gr::fail(GR_E_ARG, "gr_gemm: base pointers must be 16-byte aligned");
  const long long* all[3] = {a_strides, b_strides, c_strides};
  const int sq = dtype == GR_F32 ? 4 : 8;    // elements per 16 bytes
  for (int t = 0; t < 3; ++t)
    for (int i = 0; i < 2; ++i)
      if (all[t][i] < 0 || (all[t][i] % sq) != 0)
        return gr::fail(GR_E_ARG, "gr_gemm: strides must be non-negative multiples of 16 bytes");
  // 32-bit per-thread offsets inside one tile walk: the rows a tile spans
  if (a_strides[1] > 0x3fffffffLL / 256 || b_strides[1] > 0x3fffffffLL / 256)
    return gr::fail(GR_E_ARG, "gr_gemm: row strides too large");
  gr_gemm_args g;
  g.a = a;
  g.b = b;
  g.c = c;
  g.a_sb = a_strides[0]; g.a_sm = a_strides[1];
  g.b_sb = b_strides[0]; g.b_s = b_strides[1];
  g.c_sb = c_strides[0]; g.c_sm = c_strides[1];
  g.M = M;
  g.N = N;
  g.K = K;
  g.alpha = alpha;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GR_F16) return dispatch<_Float16>(g, batch, b_kmajor != 0, epilogue, block_m, block_n, st);
  if (dtype == GR_BF16) return dispatch<__bf16>(g, batch, b_kmajor != 0, epilogue, block_m, block_n, st);
  if (dtype == GR_F32) return dispatch_f32(g, batch, b_kmajor != 0, epilogue, block_m, block_n, st);
  return gr::fail(GR_E_ARG, "gr_gemm: dtype %d unsupported (GR_F32, GR_F16 or GR_BF16)", dtype);
}

extern "C" int gr_mlp_fwd(const void* x, const void* w1, const void* w2, void* h, void* y, int dtype, int M,
                          int D, int F, int block_m, int block_n, void* stream) {
  const long long xs[2] = {0, D}, w1s[2] = {0, F}, hs[2] = {0, F}, w2s[2] = {0, D}, ys[2] = {0, D};
  int rc = gr_gemm(x, w1, h, dtype, 1, M, F, D, xs, w1s, hs, 0, GR_EPI_SILU, 1.0f, block_m, block_n, stream);
  if (rc != 0) return rc;
  return gr_gemm(h, w2, y, dtype, 1, M, D, F, hs, w2s, ys, 0, GR_EPI_NONE, 1.0f, block_m, block_n, stream);
}
