// gr_attn.hip -- prebuilt instances of the hand-written CDNA4 attention
// forward (gr_flash_fwd.h) behind gr_attn_fwd(), plus the MFMA layout self-test.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <thread>
#include <vector>

#include "gr_flash_decode.h"
#include "gr_flash_f32.h"
#include "gr_flash_w2.h"
#include "gr_flash_w2h.h"
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

// fp16, D = 64, non-causal, 256 x 64 tiles (with or without the training
// forward's log-sum-exp): two waves per SIMD with the hand-ordered main loop
// (gr_flash_w2.h); N a multiple of 256.
template <bool KT>
int launch_w2(const gr_attn_args& a, hipStream_t st) {
  const long long nblk = (long long)a.B * a.H * (a.N / 256);
  if (nblk <= 0 || nblk > 0x7fffffffLL) return gr::fail(GR_E_ARG, "gr_attn_fwd: grid size %lld out of range", nblk);
  hipLaunchKernelGGL((gr_flash_w2_kernel<KT>), dim3((unsigned)nblk), dim3(512), GR_FLASH_W2_LDS, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd launch");
}

// fp16 or bf16, D = 128, K transposed, causal or not, 256 x 64 tiles without
// the training forward's log-sum-exp: two waves per SIMD with the
// hand-ordered main loop (gr_flash_w2h.h); N a multiple of 256.
template <class T, bool CAUSAL>
int launch_w2h(const gr_attn_args& a, hipStream_t st) {
  const long long nblk = (long long)a.B * a.H * (a.N / 256);
  if (nblk <= 0 || nblk > 0x7fffffffLL) return gr::fail(GR_E_ARG, "gr_attn_fwd: grid size %lld out of range", nblk);
  hipLaunchKernelGGL((gr_flash_w2h_kernel<T, CAUSAL>), dim3((unsigned)nblk), dim3(512), GR_FLASH_W2H_LDS, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd launch");
}

// Tile configurations compiled into the library: (block_m, block_n) ->
// (waves, query blocks per wave, key tile). One wave per 32 queries.
// block_m 0 / block_n 0 pick the largest tiles that divide N (256 x 128 at
// D = 64, 256 x 64 at D = 128), except 256 x 64 where the two-wave body of
// gr_flash_w2.h applies (fp16, D = 64, non-causal, N a multiple of 256).
template <class T, int D, bool CAUSAL, bool KT>
int dispatch_tiles(const gr_attn_args& a, int bm, int bn, hipStream_t st) {
  if (bm == 0) bm = a.N % 256 == 0 ? 256 : a.N % 128 == 0 ? 128 : 64;
  constexpr bool W2 = gr_is_same<T, _Float16>::value && D == 64 && !CAUSAL;
  if (bn == 0) bn = (W2 && bm == 256 && a.N % 256 == 0) ? 64 : (D == 64 && a.N % 128 == 0) ? 128 : a.N % 64 == 0 ? 64 : 32;
  if constexpr (W2)
    if (bm == 256 && bn == 64 && a.N % 256 == 0 && a.Nq == a.N) return launch_w2<KT>(a, st);
  if constexpr (D == 128 && KT)
    if (bm == 256 && bn == 64 && a.lse == nullptr && a.N % 256 == 0 && a.Nq == a.N) return launch_w2h<T, CAUSAL>(a, st);
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

// fp16 with scale log2(e) > 1 (Q as given, every score scaled on the VALU):
// one tile, 64 queries x 32 keys (two waves).
template <int D, bool CAUSAL, bool KT>
int launch_unscaled_q(const gr_attn_args& a, hipStream_t st) {
  constexpr int BM = 64, BN = 32, NW = 2;
  constexpr bool DIRECT = (D * BN / 8) % (NW * 64) == 0;
  constexpr int LDS = gr_flash_lds<D, BN>::BYTES;
  if (a.N % BM != 0)
    return gr::fail(GR_E_ARG, "gr_attn_fwd: fp16 with scale * log2(e) > 1 needs N=%d a multiple of 64", a.N);
  const long long nblk = (long long)a.B * a.H * (a.N / BM);
  if (nblk <= 0 || nblk > 0x7fffffffLL) return gr::fail(GR_E_ARG, "gr_attn_fwd: grid size %lld out of range", nblk);
  hipLaunchKernelGGL((gr_flash_fwd_kernel<_Float16, D, BN, NW, 1, CAUSAL, KT, false, true, DIRECT, false, false>),
                     dim3((unsigned)nblk), dim3(NW * 64), LDS, st, a);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd launch");
}

int dispatch_unscaled_q(const gr_attn_args& a, int D, bool causal, bool kt, int bm, int bn, hipStream_t st) {
  if ((bm != 0 && bm != 64) || (bn != 0 && bn != 32))
    return gr::fail(GR_E_ARG, "gr_attn_fwd: fp16 with scale * log2(e) > 1 runs the 64 x 32 tile only (asked for %d x %d)",
                    bm, bn);
#define GR_CASE(DD, C, K) \
  if (D == DD && causal == C && kt == K) return launch_unscaled_q<DD, C, K>(a, st);
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

// Merge of the key-split partials: one thread per (head, query, 8 of D).
// m_s are the parts' reference maxima (score units), l_s their row sums:
// O = sum_s w_s O_s / sum_s w_s l_s with w_s = 2^((m_s - max_s m_s) c).
template <class T, int D>
__global__ __launch_bounds__(256) void gr_attn_combine_kernel(const float* __restrict__ po, const float* __restrict__ pml,
                                                              T* o, long long o_sb, long long o_sh, long long o_sn,
                                                              int B, int H, int Nq, int S, float c) {
  constexpr int CH = D / 8;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long rows = (long long)B * H * Nq;
  if (idx >= rows * CH) return;
  const int ch = (int)(idx % CH);
  const long long row = idx / CH;              // (b*H + h) * Nq + q
  const int q = (int)(row % Nq);
  const int bh = (int)(row / Nq);
  const long long stride = rows;               // rows per split
  float mx = -GR_INF;
  for (int s = 0; s < S; ++s) mx = fmaxf(mx, pml[(s * stride + row) * 2]);
  float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const float* ml = pml + (s * stride + row) * 2;
    const float w = gr_exp2((ml[0] - mx) * c);
    L += w * ml[1];
    const float* src = po + (s * stride + row) * D + ch * 8;
    const gr_f32x4 v0 = *reinterpret_cast<const gr_f32x4*>(src);
    const gr_f32x4 v1 = *reinterpret_cast<const gr_f32x4*>(src + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] += w * v0[e];
      acc[4 + e] += w * v1[e];
    }
  }
  const float inv = 1.0f / L;
  gr_u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = gr_pack2f<T>(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  const int b = bh / H, h = bh % H;
  gr_st16(o + b * o_sb + h * o_sh + (long long)q * o_sn + ch * 8, out);
}

template <class T, int D, int BN, int NW, bool SPLIT, bool PRESCALE = true>
void decode_kernel(const gr_attn_args& a, dim3 grid, hipStream_t st) {
  constexpr int LDS = gr_flash_lds<D, BN>::BYTES;
  hipLaunchKernelGGL((gr_flash_fwd_kernel<T, D, BN, NW, 1, false, false, false, true, true, SPLIT, PRESCALE>), grid,
                     dim3(NW * 64), LDS, st, a);
}

template <class T, int D, int BN, bool SPLIT>
void decode_nw(const gr_attn_args& a, int nw, dim3 grid, hipStream_t st) {
  if (nw == 1) decode_kernel<T, D, BN, 1, SPLIT>(a, grid, st);
  else if (nw == 2) decode_kernel<T, D, BN, 2, SPLIT>(a, grid, st);
  else decode_kernel<T, D, BN, 4, SPLIT>(a, grid, st);
}

template <class T, int D, int NQ>
void decode_stream(const gr_attn_args& a, int S, hipStream_t st) {
  constexpr int U = NQ == 1 ? 8 : 4;   // key-row loads of K and of V per lane and iteration
  hipLaunchKernelGGL((gr_attn_decode_stream_kernel<T, D, NQ, U>), dim3((unsigned)(a.B * a.H), (unsigned)S),
                     dim3(256), 0, st, a);
}

// Decode-shape launch: Nq queries (any count) against N keys, non-causal, K in
// [B, H, N, D]. Up to 4 queries: the streaming kernel (gr_flash_decode.h),
// one workgroup per head and key part. More: the flash body with 32 queries
// per wave, up to 4 waves, 64-key tiles (32 when N is not a multiple of 64).
// S > 1 splits the keys over S workgroups per head (or query tile) and merges
// their partials through the workspace.
// Message for a workspace smaller than the key split needs: the caller's
// buffer (gr_attn_decode) or the library's fixed scratch array
// (gr_attn_decode_noalloc).
int workspace_short(bool fixed, size_t need, int S, size_t have) {
  if (fixed)
    return gr::fail(GR_E_ARG, "gr_attn_decode_noalloc: %d key parts need %zu bytes of scratch, more than the "
                    "%zu-byte maximum (ask for fewer splits or use gr_attn_decode with a workspace)", S, need, have);
  return gr::fail(GR_E_ARG, "gr_attn_decode: workspace of %zu bytes needed for %d key parts", need, S);
}

template <class T, int D>
int launch_decode(gr_attn_args a, int S, void* ws, size_t ws_bytes, bool fixed_ws, hipStream_t st) {
  if (a.Nq <= 4) {
    if (S < 1) S = 1;
    if (S > a.N / 32) S = a.N / 32;
    a.kchunk = ((a.N / 32 + S - 1) / S) * 32;
    S = (a.N + a.kchunk - 1) / a.kchunk;         // every part gets keys
    if ((long long)a.B * a.H > 0x7fffffffLL || S > 65535) return gr::fail(GR_E_ARG, "gr_attn_decode: grid out of range");
    if (S > 1) {
      const size_t need = gr_attn_decode_workspace(a.B, a.H, a.Nq, D, S);
      if (!ws || ws_bytes < need) return workspace_short(fixed_ws, need, S, ws_bytes);
      a.part_o = static_cast<float*>(ws);
      a.part_ml = a.part_o + (size_t)S * a.B * a.H * a.Nq * D;
    }
    if (a.Nq == 1) decode_stream<T, D, 1>(a, S, st);
    else if (a.Nq == 2) decode_stream<T, D, 2>(a, S, st);
    else decode_stream<T, D, 4>(a, S, st);
    int rc = gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_decode launch");
    if (rc != 0 || S == 1) return rc;
    const long long threads = (long long)a.B * a.H * a.Nq * (D / 8);
    hipLaunchKernelGGL((gr_attn_combine_kernel<T, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       a.part_o, a.part_ml, static_cast<T*>(a.o), a.o_sb, a.o_sh, a.o_sn, a.B, a.H, a.Nq, S,
                       a.scale_log2);
    return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_decode combine launch");
  }
  // fp16 with scale log2(e) > 1: Q as given (one wave per query tile, 32-key tiles)
  const bool unscaled = gr_is_same<T, _Float16>::value && a.scale_log2 > 1.0f;
  const int nw = unscaled ? 1 : a.Nq <= 32 ? 1 : a.Nq <= 64 ? 2 : 4;
  const long long nqt = (a.Nq + 32 * nw - 1) / (32 * nw);
  const bool bn64 = !unscaled && a.N % 64 == 0;
  const int bn = bn64 ? 64 : 32;
  const int tiles = a.N / bn;
  if (S < 1) S = 1;
  if (S > tiles) S = tiles;
  a.kchunk = ((tiles + S - 1) / S) * bn;
  S = (a.N + a.kchunk - 1) / a.kchunk;         // every part gets keys
  const long long nblk = (long long)a.B * a.H * nqt;
  if (nblk > 0x7fffffffLL || S > 65535) return gr::fail(GR_E_ARG, "gr_attn_decode: grid out of range");
  if (S > 1) {
    const size_t need = gr_attn_decode_workspace(a.B, a.H, a.Nq, D, S);
    if (!ws || ws_bytes < need) return workspace_short(fixed_ws, need, S, ws_bytes);
    a.part_o = static_cast<float*>(ws);
    a.part_ml = a.part_o + (size_t)S * a.B * a.H * a.Nq * D;
  }
  const dim3 grid((unsigned)nblk, (unsigned)S);
  if (unscaled) {
    if constexpr (gr_is_same<T, _Float16>::value) {
      if (S > 1) decode_kernel<T, D, 32, 1, true, false>(a, grid, st);
      else decode_kernel<T, D, 32, 1, false, false>(a, grid, st);
    }
  } else if (S > 1) {
    if (bn64) decode_nw<T, D, 64, true>(a, nw, grid, st);
    else decode_nw<T, D, 32, true>(a, nw, grid, st);
  } else {
    if (bn64) decode_nw<T, D, 64, false>(a, nw, grid, st);
    else decode_nw<T, D, 32, false>(a, nw, grid, st);
  }
  int rc = gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_decode launch");
  if (rc != 0 || S == 1) return rc;
  const long long threads = (long long)a.B * a.H * a.Nq * (D / 8);
  hipLaunchKernelGGL((gr_attn_combine_kernel<T, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     a.part_o, a.part_ml, static_cast<T*>(a.o), a.o_sb, a.o_sh, a.o_sn, a.B, a.H, a.Nq, S,
                     a.scale_log2);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_decode combine launch");
}

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

namespace {

// fp32 (the reference's own dtype) on the fp32 matrix cores: a workgroup owns
// 32 queries and splits its keys over its NW waves (merged through LDS). When
// the query blocks alone would leave most CUs idle, the keys of each query
// block are also split over PARTS workgroups (PARTS = 1: one launch, no
// workspace).
template <int D, int NW, bool KT>
__global__ __launch_bounds__(NW * 64) void gr_flash32_kernel(gr_attn_args a, int nkb) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash32_fwd_body<D, 32, NW, KT, 1>(a, gr_lds, nullptr, nullptr, nkb);
}

// ONE: one 32-key block per wave, known at compile time (no block loop and no
// prefetch registers); else nkb blocks per wave.
template <int D, bool KT, int PARTS, bool ONE>
__global__ __launch_bounds__(256) void gr_flash32_split_kernel(gr_attn_args a, int nkb, float* ws_o, float* ws_ml) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash32_fwd_body<D, 32, 4, KT, PARTS>(a, gr_lds, ws_o, ws_ml, ONE ? 0 : nkb);
}

template <int D, int PARTS>
__global__ __launch_bounds__(256) void gr_flash32_merge_kernel(gr_attn_args a, const float* ws_o, const float* ws_ml) {
  gr_flash32_merge_body<D, PARTS>(a, ws_o, ws_ml);
}

// Workspace of the fp32 key split: one buffer per (device, stream), grown on
// demand. Calls on one stream run in order, so they can share it; a buffer
// that grew is kept (queued work may still read it) until the process ends.
// hipStreamPerThread names a different stream in every host thread, so its
// buffers are kept per thread as well (one per host thread that ever split
// on it, none freed before the process ends). A split launch has at most
// kF32SplitTarget workgroups of 32 query rows (query blocks x parts), so a
// buffer stays below 256 * 32 * (D + 2) floats (4.3 MB at D = 128).
struct F32Workspace {
  int dev;
  hipStream_t st;
  std::thread::id thread;
  void* p;
  size_t bytes;
};
std::mutex g_f32_ws_lock;
std::vector<F32Workspace> g_f32_ws;
std::vector<void*> g_f32_ws_retired;

int f32_workspace(hipStream_t st, size_t bytes, void** out) {
  int dev = 0;
  int rc = gr::hip_check(hipGetDevice(&dev), GR_E_RUNTIME, "gr_attn_fwd: hipGetDevice");
  if (rc) return rc;
  const std::thread::id thread = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
  std::lock_guard<std::mutex> hold(g_f32_ws_lock);
  F32Workspace* w = nullptr;
  for (auto& e : g_f32_ws)
    if (e.dev == dev && e.st == st && e.thread == thread) w = &e;
  if (w && w->bytes >= bytes) {
    *out = w->p;
    return GR_OK;
  }
  void* p = nullptr;
  rc = gr::hip_check(hipMalloc(&p, bytes), GR_E_RUNTIME, "gr_attn_fwd: fp32 key-split workspace");
  if (rc) return rc;
  if (w) {
    g_f32_ws_retired.push_back(w->p);
    w->p = p;
    w->bytes = bytes;
  } else {
    g_f32_ws.push_back({dev, st, thread, p, bytes});
  }
  *out = p;
  return GR_OK;
}

template <int D, bool KT, int PARTS>
int launch_flash32_split(const gr_attn_args& a, long long nblk, hipStream_t st) {
  const long long rows = (long long)a.B * a.H * a.N;
  const size_t o_floats = (size_t)PARTS * rows * D;
  void* ws = nullptr;
  int rc = f32_workspace(st, (o_floats + (size_t)PARTS * rows * 2) * sizeof(float), &ws);
  if (rc) return rc;
  float* ws_o = static_cast<float*>(ws);
  float* ws_ml = ws_o + o_floats;
  const int nkb = a.N / (32 * 4 * PARTS);
  if (nkb == 1)
    hipLaunchKernelGGL((gr_flash32_split_kernel<D, KT, PARTS, true>), dim3((unsigned)(nblk * PARTS)), dim3(256),
                       (gr_flash32_lds<D, 4>::BYTES), st, a, nkb, ws_o, ws_ml);
  else
    hipLaunchKernelGGL((gr_flash32_split_kernel<D, KT, PARTS, false>), dim3((unsigned)(nblk * PARTS)), dim3(256),
                       (gr_flash32_lds<D, 4>::BYTES), st, a, nkb, ws_o, ws_ml);
  rc = gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd fp32 key-split launch");
  if (rc) return rc;
  const long long threads = rows * (D / 8);
  hipLaunchKernelGGL((gr_flash32_merge_kernel<D, PARTS>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     a, (const float*)ws_o, (const float*)ws_ml);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd fp32 merge launch");
}

// Workgroups a split launch aims for: one per CU of an MI355X.
constexpr long long kF32SplitTarget = 256;

template <int D, bool KT>
int launch_flash32(const gr_attn_args& a, hipStream_t st) {
  const int nw = a.N % 128 == 0 ? 4 : (a.N % 64 == 0 ? 2 : 1);
  const int nkb = a.N / (32 * nw);
  const long long nblk = (long long)a.B * a.H * (a.N / 32);
  if (nblk <= 0 || nblk > 0x7fffffffLL) return gr::fail(GR_E_ARG, "gr_attn_fwd: grid size %lld out of range", nblk);
  // the most key parts (8, 4 or 2, dividing the 32-key blocks of a wave)
  // that keep the launch within one workgroup per CU
  if (nw == 4) {
    if (nkb % 8 == 0 && nblk * 8 <= kF32SplitTarget) return launch_flash32_split<D, KT, 8>(a, nblk, st);
    if (nkb % 4 == 0 && nblk * 4 <= kF32SplitTarget) return launch_flash32_split<D, KT, 4>(a, nblk, st);
    if (nkb % 2 == 0 && nblk * 2 <= kF32SplitTarget) return launch_flash32_split<D, KT, 2>(a, nblk, st);
  }
  if (nw == 4)
    hipLaunchKernelGGL((gr_flash32_kernel<D, 4, KT>), dim3((unsigned)nblk), dim3(256), (gr_flash32_lds<D, 4>::BYTES),
                       st, a, nkb);
  else if (nw == 2)
    hipLaunchKernelGGL((gr_flash32_kernel<D, 2, KT>), dim3((unsigned)nblk), dim3(128), (gr_flash32_lds<D, 2>::BYTES),
                       st, a, nkb);
  else
    hipLaunchKernelGGL((gr_flash32_kernel<D, 1, KT>), dim3((unsigned)nblk), dim3(64), (gr_flash32_lds<D, 1>::BYTES),
                       st, a, nkb);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_attn_fwd fp32 launch");
}

int attn_fwd_f32(const gr_attn_args& a, int D, bool causal, bool k_transposed, bool train, hipStream_t st) {
  if (causal) return gr::fail(GR_E_ARG, "gr_attn_fwd: fp32 is non-causal only (the reference's fp32 workload)");
  if (train) return gr::fail(GR_E_ARG, "gr_attn_fwd_train: fp32 has no training path (GR_F16 or GR_BF16)");
  if (a.N % 32) return gr::fail(GR_E_ARG, "gr_attn_fwd: fp32 needs N a multiple of 32 (got %d)", a.N);
  if (D == 64) return k_transposed ? launch_flash32<64, true>(a, st) : launch_flash32<64, false>(a, st);
  if (D == 128) return k_transposed ? launch_flash32<128, true>(a, st) : launch_flash32<128, false>(a, st);
  return gr::fail(GR_E_ARG, "gr_attn_fwd: head dim %d unsupported (64 or 128)", D);
}

int attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int dtype, int B, int H, int N, int D,
             const long long* qs, const long long* ks, const long long* vs, const long long* os, int k_transposed,
             int causal, float scale, int block_m, int block_n, void* stream) {
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
  a.Nq = N;
  a.kchunk = N;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.lse = lse;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  // fp16 pre-scales Q by scale * log2(e) in fp16; above 1 a finite q could
  // overflow, so such calls take the kernels that keep Q as given
  if (dtype == GR_F16 && a.scale_log2 > 1.0f)
    return dispatch_unscaled_q(a, D, causal != 0, k_transposed != 0, block_m, block_n, st);
  if (dtype == GR_F16) return dispatch_shape<_Float16>(a, D, causal != 0, k_transposed != 0, block_m, block_n, st);
  if (dtype == GR_BF16) return dispatch_shape<__bf16>(a, D, causal != 0, k_transposed != 0, block_m, block_n, st);
  if (dtype == GR_F32) return attn_fwd_f32(a, D, causal != 0, k_transposed != 0, lse != nullptr, st);
  return gr::fail(GR_E_ARG, "gr_attn_fwd: dtype %d unsupported (GR_F16, GR_BF16 or GR_F32)", dtype);
}

}  // namespace

extern "C" int gr_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int N,
                           int D, const long long* qs, const long long* ks, const long long* vs, const long long* os,
                           int k_transposed, int causal, float scale, int block_m, int block_n, void* stream) {
  return attn_fwd(q, k, v, o, nullptr, dtype, B, H, N, D, qs, ks, vs, os, k_transposed, causal, scale, block_m,
                  block_n, stream);
}

extern "C" int gr_attn_fwd_train(const void* q, const void* k, const void* v, void* o, float* lse, int dtype, int B,
                                 int H, int N, int D, const long long* qs, const long long* ks, const long long* vs,
                                 const long long* os, int k_transposed, int causal, float scale, int block_m,
                                 int block_n, void* stream) {
  if (!lse || ((uintptr_t)lse & 3)) return gr::fail(GR_E_ARG, "gr_attn_fwd_train: lse must be a 4-byte aligned buffer");
  return attn_fwd(q, k, v, o, lse, dtype, B, H, N, D, qs, ks, vs, os, k_transposed, causal, scale, block_m, block_n,
                  stream);
}

extern "C" int gr_selftest_mfma32(const void* a, const void* b, float* d, void* stream) {
  if (!a || !b || !d) return gr::fail(GR_E_ARG, "gr_selftest_mfma32: null argument");
  hipLaunchKernelGGL(gr_selftest_mfma32_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const _Float16*)a,
                     (const _Float16*)b, d);
  return gr::hip_check(hipGetLastError(), GR_E_LAUNCH, "gr_selftest_mfma32 launch");
}

extern "C" size_t gr_attn_decode_workspace(int B, int H, int Nq, int D, int splits) {
  if (B <= 0 || H <= 0 || Nq <= 0 || D <= 0 || splits <= 1) return 0;
  return (size_t)splits * B * H * Nq * (D + 2) * sizeof(float);
}

namespace {

int attn_decode(const char* who, const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                int Nq, int N, int D, const long long* qs, const long long* ks, const long long* vs,
                const long long* os, float scale, int splits, void* workspace, size_t workspace_bytes, bool fixed_ws,
                void* stream) {
  if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return gr::fail(GR_E_ARG, "%s: null argument", who);
  if (B <= 0 || H <= 0 || Nq <= 0 || N <= 0) return gr::fail(GR_E_ARG, "%s: B, H, Nq, N must be positive", who);
  if (N % 32 != 0) return gr::fail(GR_E_ARG, "%s: N=%d keys must be a multiple of 32", who, N);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || ((uintptr_t)workspace & 15))
    return gr::fail(GR_E_ARG, "%s: base pointers must be 16-byte aligned", who);
  const long long* all[4] = {qs, ks, vs, os};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      if (all[t][i] < 0 || (all[t][i] % 8) != 0)
        return gr::fail(GR_E_ARG, "%s: strides must be non-negative multiples of 8 elements", who);
  if (!(scale > 0.f)) return gr::fail(GR_E_ARG, "%s: scale must be positive", who);
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
  a.Nq = Nq;
  a.kchunk = N;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
#define GR_DT(TT)                                                                                  \
  if (D == 64) return launch_decode<TT, 64>(a, splits, workspace, workspace_bytes, fixed_ws, st);  \
  if (D == 128) return launch_decode<TT, 128>(a, splits, workspace, workspace_bytes, fixed_ws, st); \
  return gr::fail(GR_E_ARG, "%s: head dim D=%d unsupported (64 or 128)", who, D);
  if (dtype == GR_F16) { GR_DT(_Float16) }
  if (dtype == GR_BF16) { GR_DT(__bf16) }
#undef GR_DT
  return gr::fail(GR_E_ARG, "%s: dtype %d unsupported (GR_F16 or GR_BF16)", who, dtype);
}

// The key-split partials of gr_attn_decode_noalloc live in this array, one
// copy per device, held until the process ends. The kernels only ever see
// its device address (g_scratch), which hipGetSymbolAddress returns for the
// device current at the first call on it; the array's name is a host-side
// stand-in and never goes to a kernel.
constexpr size_t kDecodeScratch = (size_t)GR_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kDecodeScratch];
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_lock;

int scratch_address(void** out) {
  int dev = 0;
  int rc = gr::hip_check(hipGetDevice(&dev), GR_E_RUNTIME, "gr_attn_decode_noalloc: hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices) return gr::fail(GR_E_ARG, "gr_attn_decode_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    rc = gr::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), GR_E_RUNTIME,
                       "gr_attn_decode_noalloc: hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    if (!p) return gr::fail(GR_E_RUNTIME, "gr_attn_decode_noalloc: no device address for the scratch array");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return GR_OK;
}

}  // namespace

extern "C" int gr_attn_decode(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int Nq,
                              int N, int D, const long long* qs, const long long* ks, const long long* vs,
                              const long long* os, float scale, int splits, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return attn_decode("gr_attn_decode", q, k, v, o, dtype, B, H, Nq, N, D, qs, ks, vs, os, scale, splits, workspace,
                     workspace_bytes, false, stream);
}

extern "C" int gr_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                                      int Nq, int N, int D, const long long* qs, const long long* ks,
                                      const long long* vs, const long long* os, float scale, int splits,
                                      void* stream) {
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return attn_decode("gr_attn_decode_noalloc", q, k, v, o, dtype, B, H, Nq, N, D, qs, ks, vs, os, scale, splits, ws,
                     kDecodeScratch, true, stream);
}
