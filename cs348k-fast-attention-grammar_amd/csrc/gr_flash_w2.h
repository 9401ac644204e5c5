// gr_flash_w2.h -- flash attention forward, two waves per SIMD, each running
// a hand-ordered main loop (gfx950, fp16, head dim 64, non-causal).
//
// Same contract and tile layouts as gr_flash_fwd_body (O = softmax(scale Q
// K^T) V, K natural or transposed, [B, H, N, D] with free batch/head/row
// strides), for N a multiple of 256 with as many queries as keys and
// scale log2(e) <= 1 (Q is pre-scaled in fp16).
//
// A workgroup is 8 waves of 32 queries (two per SIMD, 256 queries). Each
// 64-key tile is one step of 16 "slots" of one MFMA plus the vector work of
// one score pair (two exponentials, a pack, a packed row-sum add): the score MFMAs
// of tile j + 1 (two 32-key halves, four 16-deep MFMAs each) and the P.V MFMAs
// of tile j - 1 (two 32-wide head-dim blocks, four 16-key chunks each)
// alternate, and between them the exponentials of tile j's scores. The order
// inside a slot is fixed in inline assembly. One wave cannot hide the other
// per-tile work (fragment reads, barrier, loads) behind its own slots, whose
// vector work already fills the MFMA time; the second wave of the SIMD fills
// those gaps. All operands stay in VGPRs, fewer than 256, which fits two waves.
//
// K and V tiles go straight from global memory into two rings of 8 LDS slots
// of 8 KiB (128 KiB), loaded 4 to 6 tiles ahead; one barrier per tile. Each
// wave stages its Q rows, and at the end its O rows, in 4 KiB of its own
// (32 KiB more). Operand fragments are read from LDS just in time, at a
// per-lane base plus an immediate: the step loop is unrolled over the ring's
// eight slots so that every slot offset is a constant.
//
// Against gr_flash_fwd_body's 256 x 128 tile, interleaved on one box: B4 H16
// N1024 d64 (the C2 shape) 17.45 us against 19.1-19.4 us, B1 H16 N4096 61.0 us
// against 66.6 us. A straight-line fit over 7 to 63 steps per workgroup gives
// 0.91 us per 64-key step (0.99) and 3.9 us per workgroup (4.1): the first Q
// and tile loads, the O store and the launch.
//
// Softmax in exponent units, as the fp16 path of gr_flash_fwd_body: Q is
// pre-scaled by scale log2(e) and the score MFMAs start from -base, so
// p = 2^s. The base is the first tile's row max; a step with a p or a row-sum
// half past the fp16 range (a row max that grew by more than ~2^10) is redone
// on a slow path that moves the base, rescales the accumulators and shifts
// the next tile's scores. Row sums add the packed fp16 P of a step in fp16
// (16 values per half, one packed add per pair) and go into the fp32 sum once
// per step: two fp32 adds per pair would cost more vector time than the pack.
//
// Hazards the compiler does not see through inline assembly are kept apart
// by construction: every score register is read by the vector unit at least
// four slots after the MFMA that wrote it, every P register is read by an
// MFMA at least eight slots after the vector op that wrote it, and the slow
// path and the end of the loop are fenced with s_nop.
#pragma once
#include "gr_gemm.h"

#define GR_W2_GUARD "s_nop 7\n\ts_nop 7\n\ts_nop 3"

// The vector half of a slot: scores x0, x1 to 2^x in t0, t1, packed to fp16
// into pk; the previous pair's pack pp is added into the packed row sums la.
// A vector op that reads the result of a transcendental op (v_exp_f32) must
// issue at least one instruction after it (the compiler does not insert that
// wait state inside inline assembly), so the row-sum add sits between the
// second exponential and the pack.
#define GR_W2_VALU                               \
  "v_exp_f32 %[t0], %[x0]\n\t"                   \
  "v_exp_f32 %[t1], %[x1]\n\t"                   \
  "v_pk_add_f16 %[la], %[la], %[pp]\n\t"         \
  "v_cvt_pk_f16_f32 %[pk], %[t0], %[t1]\n\t"

template <bool KT>
__device__ __forceinline__ void gr_flash_w2_body(const gr_attn_args& a, char* lds) {
  typedef _Float16 T;
  typedef gr_mfma<T> MF;
  typedef MF::vec8 vec8;
  constexpr int D = 64, BNT = 64, BM = 256, NT = 512, NSLOT = 8;
  constexpr int TILE_K = BNT * D * 2;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int N = a.N, nqt = N / BM;
  const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / nqt, qt = logical % nqt;
  const int b = bh / a.H, h = bh % a.H;
  const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
  const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
  const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
  T* Op = (T*)a.o + b * a.o_sb + h * a.o_sh;
  const int qw = qt * BM + wave * 32;       // this wave's 32 queries
  const float c = a.scale_log2;

  // K and V tiles of 64 keys (K rows in the perm32 order that makes the score
  // accumulators the P.V MFMAs' operand), straight into the ring
  typedef typename gr_cond<KT, gr_lds_loader<T, D, BNT, NT, true>, gr_lds_loader<T, BNT, D, NT, false, true>>::type KL;
  typedef gr_lds_loader<T, BNT, D, NT, true> VL;
  constexpr int PER_TILE = KL::PER + VL::PER;    // direct loads per thread and tile
  static_assert((D * BNT / 8) % NT == 0, "whole chunks per thread");
  KL kl;
  VL vl;
  kl.init(tid, a.k_sn);
  vl.init(tid, a.v_sn);
  const long long k_tile = KT ? (long long)BNT : (long long)BNT * a.k_sn;
  const long long v_tile = (long long)BNT * a.v_sn;
  const int ntile = N / BNT;
  // LDS: K tiles in the first NSLOT * 8 KiB, V tiles in the next, so that a
  // fragment's address is a per-lane base plus an immediate (< 64 KiB) for its
  // slot, chunk and half; with the step loop unrolled over the ring, every
  // slot index is a compile-time constant.
  constexpr int VOFF = NSLOT * TILE_K, QOFF = 2 * NSLOT * TILE_K;
  // A tile is one direct load of K and one of V per thread, from a wave-uniform
  // (scalar) tile base plus the lane's constant byte offset, so that moving to
  // the next tile costs scalar arithmetic only; M0 (the LDS destination) is
  // saved and restored once for both.
  static_assert(KL::PER == 1 && VL::PER == 1 && KL::CHUNKS == NT && VL::CHUNKS == NT, "one chunk per thread");
  const unsigned kgo = (unsigned)kl.goff[0] * 2u, vgo = (unsigned)vl.goff[0] * 2u;
  const unsigned lbase = gr_lds_addr(lds) + kl.lwave;
  auto load_tile = [&](int t, int slot) {
    if (t < ntile) {
      const T* kb = Kp + t * k_tile;
      const T* vb = Vp + t * v_tile;
      unsigned saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %3\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %2, %1\n\t"
          "s_mov_b32 m0, %6\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %5, %4\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(kb), "v"(kgo), "s"(lbase + slot * TILE_K), "s"(vb), "v"(vgo), "s"(lbase + VOFF + slot * TILE_K)
          : "memory");
    }
  };
  // lane base of two transposing reads (gr_tr_frag) of a tile with 128-byte
  // rows at k0 = 0; rows k0 + 4h lie (k0 + 4h) * 128 bytes further on, as the
  // swizzle depends on row bit 1 only
  auto tr_base = [&](int n0, bool perm) -> int {
    const int cq = lane & 3;
    const int cc = perm ? (((cq & 1) << 1) | (cq >> 1)) : cq;
    const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * cc;
    const int row = 8 * (lane >> 5) + ((lane >> 2) & 3);
    return row * 128 + gr_swz_tr<8>(row, col >> 3) * 16 + (col & 7) * 2;
  };
  auto tr2 = [&](int off) -> vec8 {
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    gr_u32x4 r;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const char* p = lds + off + hh * 512;
      const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(__attribute__((address_space(3))) char*)(char*)p);
      const gr_u32x2 w = __builtin_bit_cast(gr_u32x2, v);
      r[2 * hh] = w[0];
      r[2 * hh + 1] = w[1];
    }
    return gr_as<vec8>(r);
  };
  // K fragment (32-key half kb, depth block ds) and V fragment (16-key chunk
  // cc, head-dim block db) of the tile in ring slot `slot`
  int kbase[KT ? 2 : 8], vbase[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if constexpr (KT) {
      kbase[kb] = tr_base(kb * 32, true);
    } else {
      const int row = kb * 32 + l32;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) kbase[kb * 4 + ds] = row * (D * 2) + gr_swz<D / 8>(row, 2 * ds + g) * 16;
    }
  }
#pragma unroll
  for (int db = 0; db < 2; ++db) vbase[db] = VOFF + tr_base(db * 32, false);
  auto kfrag = [&](int slot, int kb, int ds) -> vec8 {
    if constexpr (KT) return tr2(kbase[kb] + slot * TILE_K + ds * 16 * 128);
    return gr_as<vec8>(gr_ld16(lds + kbase[kb * 4 + ds] + slot * TILE_K));
  };
  auto vfrag = [&](int slot, int cc, int db) -> vec8 { return tr2(vbase[db] + slot * TILE_K + cc * 16 * 128); };

  // prologue: each wave's 32 Q rows into its own 4 KiB of the Q area (after
  // the ring), then the first NSLOT tiles, all as direct loads. Q goes first,
  // so that the wait for tiles 0 to 2 covers it; its fragments are then read
  // from LDS (a value loaded into registers by assembly would be copied by the
  // compiler before any wait of ours).
  char* const qarea = lds + QOFF + wave * (32 * D * 2);
  {
    gr_lds_loader<T, 32, D, 64> ql;
    ql.init(lane, a.q_sn);
    ql.load(Qp + (long long)qw * a.q_sn, qarea);
  }
#pragma unroll
  for (int t = 0; t < NSLOT; ++t) load_tile(t, t);
  // Q and tiles 0, 1 and 2 landed (later tiles may stay in flight)
  if (ntile >= NSLOT) gr_wait_vmcnt<(NSLOT - 3) * PER_TILE>(); else gr_wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // Q fragments pre-scaled by scale log2(e)
  vec8 qf[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    vec8 v = gr_as<vec8>(gr_ld16(qarea + l32 * (D * 2) + gr_swz<D / 8>(l32, 2 * ds + g) * 16));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (T)((float)v[e] * c);
    qf[ds] = v;
  }

  // tile 0: scores from zero, the base from their row max, P(0)
  gr_f32x16 sA[2], sB[2], cinit;
  float lsum;
  {
    gr_f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = (gr_f32x16)(0.f);
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) s[kb] = MF::mma32(kfrag(0, kb, ds), qf[ds], s[kb]);
    }
    float mt = s[0][0];
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(s[0][r], s[1][r]));
    mt = fmaxf(mt, gr_xor32(mt));
    cinit = (gr_f32x16)(-mt);
    sB[0] = s[0] - mt;                       // tile 0's scores, relative to the base
    sB[1] = s[1] - mt;
  }
  gr_u32x4 pA[4], pB[4];                     // P of a tile, [16-key chunk]
  {
    float l = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float p0 = gr_exp2(sB[kb][8 * hf + e]), p1 = gr_exp2(sB[kb][8 * hf + e + 1]);
          pB[2 * kb + hf][e >> 1] = gr_pack2f<T>(p0, p1);
          l += p0 + p1;
        }
    lsum = l;
  }
  // tile 1's scores (from -base)
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    gr_f32x16 s = MF::mma32(kfrag(1, kb, 0), qf[0], cinit);
#pragma unroll
    for (int ds = 1; ds < 4; ++ds) s = MF::mma32(kfrag(1, kb, ds), qf[ds], s);
    sA[kb] = s;
  }
  gr_f32x16 o[2];                            // O^T accumulators [head-dim block]
  o[0] = (gr_f32x16)(0.f);
  o[1] = (gr_f32x16)(0.f);
  // Operand fragments are read just in time into two-deep rings: the score
  // MFMA of slot 2q (q = 0..7: half kb = q % 2, depth ds = q / 2) takes K
  // fragment kq[q % 2], the P.V MFMA of slot 2p + 1 (p = 0..7: chunk cc =
  // p / 2, head-dim block db = p % 2) V fragment vp[p % 2]; each is refilled
  // right after the slot that used it with the fragment two such slots ahead
  // (the last two of a step with the next step's first two).
  auto kfq = [&](int t, int q) -> vec8 { return kfrag(t, q & 1, q >> 1); };
  auto vfp = [&](int t, int p) -> vec8 { return vfrag(t, p >> 1, p & 1); };
  vec8 kq[2], vp[2];
  kq[0] = kfq(2, 0);   // tile t sits in ring slot t here
  kq[1] = kfq(2, 1);
  vp[0] = vfp(0, 0);
  vp[1] = vfp(0, 1);

  // Step j (j = I mod 8, so that every ring slot is a constant): S_next =
  // scores of tile j + 1, P_cur = P of tile j (from S_cur), O += V^T P_prev
  // (tile j - 1). Reads K of tile j + 1 (and the first two fragments of tile
  // j + 2) and V of tile j - 1 (and the first two of tile j).
  auto step = [&](auto ic, gr_f32x16 (&S_cur)[2], gr_f32x16 (&S_next)[2], gr_u32x4 (&P_cur)[4], gr_u32x4 (&P_prev)[4]) {
    constexpr int I = decltype(ic)::value;
    constexpr int SK1 = (I + 1) & (NSLOT - 1), SK2 = (I + 2) & (NSLOT - 1);
    constexpr int SV0 = (I + NSLOT - 1) & (NSLOT - 1), SV1 = I & (NSLOT - 1);
    // row sums of the step's packed P, pair by pair in fp16 (each half adds
    // 16 values), one slot behind the pack that wrote them
    unsigned lt = 0u, zero = 0u;
    float t0, t1;
#define GR_W2_OUT(I) [t0] "=&v"(t0), [t1] "=&v"(t1), [pk] "=&v"(P_cur[(I) / 4][(I) % 4]), [la] "+v"(lt)
#define GR_W2_X(I)                                                                                  \
  [x0] "v"(S_cur[(I) / 8][2 * ((I) % 8)]), [x1] "v"(S_cur[(I) / 8][2 * ((I) % 8) + 1]),             \
      [pp] "v"((I) == 0 ? zero : P_cur[((I) - 1) / 4][((I) - 1) % 4])
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int q = s >> 1;
      if ((s & 1) == 0) {
        // score MFMA: half kb = q % 2, depth ds = q / 2 (the first of each chain from -base)
        if (q < 2)
          asm volatile("v_mfma_f32_32x32x16_f16 %[d], %[ka], %[qb], %[ci]\n\t" GR_W2_VALU
                       : [d] "=&v"(S_next[q & 1]), GR_W2_OUT(s)
                       : [ka] "v"(kq[q & 1]), [qb] "v"(qf[0]), [ci] "v"(cinit), GR_W2_X(s));
        else
          asm volatile("v_mfma_f32_32x32x16_f16 %[d], %[ka], %[qb], %[d]\n\t" GR_W2_VALU
                       : [d] "+v"(S_next[q & 1]), GR_W2_OUT(s)
                       : [ka] "v"(kq[q & 1]), [qb] "v"(qf[q >> 1]), GR_W2_X(s));
        kq[q & 1] = q + 2 < 8 ? kfq(SK1, q + 2) : kfq(SK2, q - 6);
      } else {
        // P.V MFMA: chunk cc = q / 2, head-dim block db = q % 2
        asm volatile("v_mfma_f32_32x32x16_f16 %[d], %[va], %[pb], %[d]\n\t" GR_W2_VALU
                     : [d] "+v"(o[q & 1]), GR_W2_OUT(s)
                     : [va] "v"(vp[q & 1]), [pb] "v"(P_prev[q >> 1]), GR_W2_X(s));
        vp[q & 1] = q + 2 < 8 ? vfp(SV0, q + 2) : vfp(SV1, q - 6);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#undef GR_W2_X
#undef GR_W2_OUT
    asm volatile("v_pk_add_f16 %0, %0, %1" : "+v"(lt) : "v"(P_cur[3][3]));
    float ltq;
    {
      const gr_f16x2 hsum = __builtin_bit_cast(gr_f16x2, lt);
      ltq = (float)hsum[0] + (float)hsum[1];
    }
    // a p past fp16's range, or a half-sum that overflowed, reads as inf (or NaN)
    if (__builtin_expect(gr_any(!(ltq <= 3.0e38f)), 0)) {
      asm volatile(GR_W2_GUARD : "+v"(S_next[0]), "+v"(S_next[1]), "+v"(o[0]), "+v"(o[1]));
      // Slow path: the base moves to the true row max of tile j (whose scores
      // are still in S_cur, relative to the old base), O and the row sum are
      // rescaled, P of tile j is recomputed and tile j + 1's scores are
      // shifted to the new base.
      float mt = S_cur[0][0];
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(S_cur[0][r], S_cur[1][r]));
      mt = fmaxf(mt, gr_xor32(mt));
      const float sh = mt > 0.f ? mt : 0.f;   // the base moves up by sh (exponent units)
      const float alpha = gr_exp2(-sh);
      lsum *= alpha;
      o[0] *= alpha;
      o[1] *= alpha;
      cinit -= sh;
      S_next[0] -= sh;
      S_next[1] -= sh;
      float l = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const float p0 = gr_exp2(S_cur[kb][8 * hf + e] - sh), p1 = gr_exp2(S_cur[kb][8 * hf + e + 1] - sh);
            P_cur[2 * kb + hf][e >> 1] = gr_pack2f<T>(p0, p1);
            l += p0 + p1;
          }
      ltq = l;
      asm volatile(GR_W2_GUARD : "+v"(S_next[0]), "+v"(S_next[1]), "+v"(o[0]), "+v"(o[1]), "+v"(P_cur[0]),
                   "+v"(P_cur[1]), "+v"(P_cur[2]), "+v"(P_cur[3]));
    }
    lsum += ltq;
  };

  asm volatile(GR_W2_GUARD : "+v"(sA[0]), "+v"(sA[1]), "+v"(sB[0]), "+v"(sB[1]), "+v"(cinit), "+v"(pB[0]),
               "+v"(pB[1]), "+v"(pB[2]), "+v"(pB[3]), "+v"(o[0]), "+v"(o[1]));
  // The loop. The barrier before step j publishes tile j + 2 (later tiles may
  // stay in flight) and frees tile j - 2's slot for tile j + NSLOT - 2.
  auto publish = [&](auto ic, int j) {
    constexpr int I = decltype(ic)::value;
    if (j + NSLOT - 3 < ntile) gr_wait_vmcnt<(NSLOT - 5) * PER_TILE>(); else gr_wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (j >= 2) load_tile(j + NSLOT - 2, (I + NSLOT - 2) & (NSLOT - 1));
  };
  // steps 1 .. ntile - 1: whole groups of eight (the ring's period; the
  // score and P buffers alternate with the step's parity), then the rest,
  // three or seven steps (ntile - 1 is 3 mod 4), in straight code
#define GR_W2_STEP(I, SC, SN, PC, PP) \
  publish(gr_ic<I>{}, m + (I));       \
  step(gr_ic<I>{}, SC, SN, PC, PP);
  int m = 0;
  for (; m + 8 < ntile; m += 8) {
    GR_W2_STEP(1, sA, sB, pA, pB)
    GR_W2_STEP(2, sB, sA, pB, pA)
    GR_W2_STEP(3, sA, sB, pA, pB)
    GR_W2_STEP(4, sB, sA, pB, pA)
    GR_W2_STEP(5, sA, sB, pA, pB)
    GR_W2_STEP(6, sB, sA, pB, pA)
    GR_W2_STEP(7, sA, sB, pA, pB)
    GR_W2_STEP(8, sB, sA, pB, pA)
  }
  GR_W2_STEP(1, sA, sB, pA, pB)
  GR_W2_STEP(2, sB, sA, pB, pA)
  GR_W2_STEP(3, sA, sB, pA, pB)
  if (m + 4 < ntile) {
    GR_W2_STEP(4, sB, sA, pB, pA)
    GR_W2_STEP(5, sA, sB, pA, pB)
    GR_W2_STEP(6, sB, sA, pB, pA)
    GR_W2_STEP(7, sA, sB, pA, pB)
  }
#undef GR_W2_STEP
  // P.V of the last tile (its P in pA: ntile - 1 is odd)
  {
    gr_u32x4 (&pl)[4] = pA;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(o[p & 1]) : "v"(vp[p & 1]), "v"(gr_as<vec8>(pl[p >> 1])));
      if (p + 2 < 8) vp[p & 1] = vfp((ntile - 1) & (NSLOT - 1), p + 2);
    }
  }
  asm volatile(GR_W2_GUARD : "+v"(o[0]), "+v"(o[1]));

  // O = O^T^T / l, staged through this wave's own Q area (no other wave
  // touches it) as whole 16-byte row chunks
  constexpr int CPR = D / 8;
  const float lrow = lsum + gr_xor32(lsum);
  const float inv = 1.0f / lrow;
  // the training forward's row log-sum-exp (natural log): the base is -cinit
  // in the pre-scaled (log2) units of the scores
  if (a.lse && g == 0)
    a.lse[(long long)bh * a.Nq + qw + l32] = (__builtin_amdgcn_logf(lrow) - cinit[0]) * 0.6931471805599453f;
  char* const stage = qarea;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      gr_u32x2 w;
      w[0] = gr_pack2f<T>(o[db][4 * rr + 0] * inv, o[db][4 * rr + 1] * inv);
      w[1] = gr_pack2f<T>(o[db][4 * rr + 2] * inv, o[db][4 * rr + 3] * inv);
      *reinterpret_cast<gr_u32x2*>(stage + l32 * (D * 2) + gr_swz<CPR>(l32, db * 4 + rr) * 16 + g * 8) = w;
    }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < 32 * CPR / 64; ++it) {
    const int jj = it * 64 + lane, row = jj / CPR, ch = jj % CPR;
    const gr_u32x4 v = gr_ld16(stage + row * (D * 2) + gr_swz<CPR>(row, ch) * 16);
    __builtin_nontemporal_store(v, reinterpret_cast<gr_u32x4*>(Op + (long long)(qw + row) * a.o_sn + ch * 8));
  }
}

// LDS bytes: eight K tile slots and eight V tile slots of 8 KiB, then 4 KiB of
// Q (and later O) per wave: 160 KiB, all of a CU's LDS
constexpr int GR_FLASH_W2_LDS = 8 * (2 * 64 * 64 * 2) + 8 * 32 * 64 * 2;

template <bool KT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void gr_flash_w2_kernel(gr_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash_w2_body<KT>(a, gr_lds);
}
