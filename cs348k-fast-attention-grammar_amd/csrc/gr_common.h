// gr_common.h -- device-side vocabulary shared by the hand-written CDNA4 kernels
// and by every HIP translation unit the grammar renderer emits (hiprtc includes
// this file by name). gfx950 only: 64-lane wavefronts, the double-K MFMA family
// (v_mfma_f32_32x32x16_{f16,bf16}), 160 KiB of LDS per CU.
//
// Self-contained on purpose: hiprtc compiles it without the C++ standard
// library, so nothing here includes a system header beyond what hiprtc provides.
#pragma once
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

#ifndef GR_INF
#define GR_INF __builtin_inff()
#endif

// Marks, in generated code, the per-iteration offset of a sub-tile read from a
// value materialised outside a ReductionLoop (an extract bridge).
#define GR_SUBTILE(x) (x)

typedef _Float16 gr_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 gr_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 gr_f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 gr_bf16x4 __attribute__((ext_vector_type(4)));
typedef float gr_f32x16 __attribute__((ext_vector_type(16)));
typedef float gr_f32x4 __attribute__((ext_vector_type(4)));
typedef float gr_f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int gr_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int gr_u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Element traits: storage type T (fp16 or bf16) -> MFMA operand vector and the
// 32x32x16 matrix-core op. Operand layout (A: M x K, B: K x N, lane l):
//   A[m][k]: m = l % 32, k in the 8-wide group (l / 32)
//   B[k][n]: n = l % 32, k in the 8-wide group (l / 32)
//   D[m][n]: n = l % 32, m = 8*(r/4) + 4*(l/32) + (r%4) for accumulator r
// Only the pairing of k between A and B matters for a contraction, so callers
// may assign any 8 contraction indices to a lane group as long as A and B agree.
// ---------------------------------------------------------------------------
template <class T> struct gr_mfma;

typedef _Float16 gr_f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 gr_bf16x2 __attribute__((ext_vector_type(2)));

template <> struct gr_mfma<_Float16> {
  typedef gr_f16x8 vec8;
  typedef gr_f16x4 vec4;
  typedef gr_f16x2 vec2;
  // acc + a.x + a.y, products exact, fp32 accumulate (v_dot2c_f32_f16).
  static __device__ __forceinline__ float sum2(vec2 a, float acc) {
    const vec2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(a, one, acc, false);
  }
  static __device__ __forceinline__ gr_f32x16 mma32(vec8 a, vec8 b, gr_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ gr_f32x4 mma16(vec8 a, vec8 b, gr_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct gr_mfma<__bf16> {
  typedef gr_bf16x8 vec8;
  typedef gr_bf16x4 vec4;
  typedef gr_bf16x2 vec2;
  static __device__ __forceinline__ float sum2(vec2 a, float acc) {
    const vec2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(a, one, acc, false);
  }
  static __device__ __forceinline__ gr_f32x16 mma32(vec8 a, vec8 b, gr_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ gr_f32x4 mma16(vec8 a, vec8 b, gr_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// 16-byte and 8-byte raw moves. The bit casts keep the vector registers intact.
template <class V>
__device__ __forceinline__ V gr_as(gr_u32x4 x) { return __builtin_bit_cast(V, x); }
template <class V>
__device__ __forceinline__ gr_u32x4 gr_raw(V x) { return __builtin_bit_cast(gr_u32x4, x); }

__device__ __forceinline__ int gr_imin(int a, int b) { return a < b ? a : b; }

__device__ __forceinline__ gr_u32x4 gr_ld16(const void* p) {
  return *reinterpret_cast<const gr_u32x4*>(p);
}
__device__ __forceinline__ void gr_st16(void* p, gr_u32x4 v) {
  *reinterpret_cast<gr_u32x4*>(p) = v;
}

// 16 bytes per lane from global memory straight into LDS (gfx950
// global_load_lds_dwordx4): lane l's bytes land at LDS address lds + 16 l,
// where lds must be wave-uniform (it goes through M0; gr_lds_addr gives the
// LDS address of a pointer into shared memory). Written as inline assembly so
// that the compiler does not treat the load as an LDS store it must wait for
// before every later LDS read (it cannot tell the slot being filled from the
// slot being read); callers wait on vmcnt themselves before publishing the
// tile. M0 is saved and restored around the load, and one wait state
// separates the M0 write from the load that reads it.
__device__ __forceinline__ void gr_g2lds16(const void* g, unsigned int lds) {
  unsigned int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds)
      : "memory");
}
// LDS address of a (generic) pointer into shared memory: the low 32 bits of a
// flat address in the LDS aperture.
__device__ __forceinline__ unsigned int gr_lds_addr(const void* p) {
  return (unsigned int)(unsigned long long)p;
}

// Exchange with the lane 32 positions away (the other half of the wavefront).
__device__ __forceinline__ float gr_xor32(float v) {
  return __shfl_xor(v, 32, 64);
}

// 2^x on the transcendental unit (v_exp_f32); overflows to +inf, -inf gives 0.
__device__ __forceinline__ float gr_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Round two floats to the storage type and pack them into one dword (low = a,
// high = b): one v_cvt_pk_{f16,bf16}_f32 on gfx950.
template <class T>
__device__ __forceinline__ unsigned int gr_pack2f(float a, float b) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(unsigned int, __builtin_convertvector((gr_f32x2){a, b}, t2));
}

// Pack two storage-type values into one dword (low = a, high = b).
template <class T>
__device__ __forceinline__ unsigned int gr_pack2(T a, T b) {
  unsigned short lo = __builtin_bit_cast(unsigned short, a);
  unsigned short hi = __builtin_bit_cast(unsigned short, b);
  return (unsigned int)lo | ((unsigned int)hi << 16);
}

// Workgroup index remap so that consecutive logical blocks land on the same
// XCD (MI355X dispatches workgroups round-robin over its 8 XCDs, each with its
// own L2). Blocks that share K/V (same head) then share an L2.
__device__ __forceinline__ int gr_xcd_remap(int bid, int nblk) {
  if ((nblk & 7) != 0) return bid;
  return (bid & 7) * (nblk >> 3) + (bid >> 3);
}

// Causal grids, where a head's blocks have unequal work that falls with their
// rank r (0 = longest): block index -> (head bh, rank r) such that each XCD
// runs the blocks of its heads longest-first across all of them, rather than
// head after head. With nper blocks per head and heads in multiples of 8,
// XCD x holds heads [x per, (x + 1) per), as gr_xcd_remap groups them, taken
// rank by rank; otherwise the whole grid goes rank by rank. List scheduling
// in head-major order leaves the shortest blocks of the last heads and the
// longest of others unevenly spread: a 20 % longer makespan at B2 H32 N4096
// against none for longest-first.
__device__ __forceinline__ void gr_causal_order(int bid, int nblk, int nper, int& bh, int& r) {
  const int nbh = nblk / nper;
  if ((nbh & 7) == 0) {
    const int logical = gr_xcd_remap(bid, nblk);
    const int per = nbh >> 3, span = nblk >> 3;
    const int x = logical / span, m = logical % span;
    bh = x * per + m % per;
    r = m / per;
  } else {
    bh = bid % nbh;
    r = bid / nbh;
  }
}

// Wave-uniform "any lane" vote.
__device__ __forceinline__ bool gr_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// ---------------------------------------------------------------------------
// Row-lowering helpers: VEC consecutive elements of a row to/from fp32
// registers with one vector access (the offset is a multiple of VEC), and
// reductions across the 64 lanes of a wavefront.
// ---------------------------------------------------------------------------
template <int VEC, class T>
__device__ __forceinline__ void gr_row_load(float (&d)[VEC], const T* p) {
  if constexpr (VEC == 1) {
    d[0] = (float)p[0];
  } else {
    typedef T vec_t __attribute__((ext_vector_type(VEC)));
    const vec_t v = *reinterpret_cast<const vec_t*>(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) d[k] = (float)v[k];
  }
}

// VEC consecutive elements of a row of a tensor that a split-K GEMM stage
// left as `parts` fp32 partial products `part_stride` floats apart: their sum.
template <int VEC>
__device__ __forceinline__ void gr_row_load_parts(float (&d)[VEC], const float* p, long long part_stride,
                                                  int parts) {
  gr_row_load<VEC>(d, p);
  for (int s = 1; s < parts; ++s) {
    float e[VEC];
    gr_row_load<VEC>(e, p + s * part_stride);
#pragma unroll
    for (int k = 0; k < VEC; ++k) d[k] += e[k];
  }
}

template <int VEC, class T>
__device__ __forceinline__ void gr_row_store(T* p, const float (&y)[VEC]) {
  if constexpr (VEC == 1) {
    p[0] = (T)y[0];
  } else {
    typedef T vec_t __attribute__((ext_vector_type(VEC)));
    vec_t v;
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = (T)y[k];
    *reinterpret_cast<vec_t*>(p) = v;
  }
}

__device__ __forceinline__ float gr_wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float gr_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
