// gr_flash_w2h.h -- flash attention forward at head dim 128, two waves per
// SIMD, each running a hand-ordered main loop (gfx950, bf16 or fp16, causal or
// not, K given transposed).
//
// Same contract as gr_flash_fwd_body with the K^T layout (O = softmax(scale Q
// K^T) V; Q, V, O [B, H, N, D], K^T [B, H, D, N], free batch/head/row
// strides), for N a multiple of 256 with as many queries as keys. Q is kept as
// given: every score is scaled on the vector unit (one multiply-add before its
// exponential), so any scale is exact and the score MFMAs start from zero.
//
// A workgroup is 8 waves of 32 queries (two per SIMD, 256 queries). Each
// 64-key tile is one step of 32 "slots" of one MFMA plus the vector work of
// one score (multiply-add, exponential, row-sum add, and on every second slot
// the pack of the pair): the score MFMAs of tile j + 1 (two 32-key halves,
// eight 16-deep MFMAs each) and the P.V MFMAs of tile j - 1 (four 32-wide
// head-dim blocks, four 16-key chunks each) alternate, and between them the
// vector work of tile j's scores. At head dim 128 a slot's vector work is about
// half the MFMA's 32 cycles, so the MFMA pipe can stay busy; the second wave of
// the SIMD hides each wave's per-tile work (fragment reads at the start of a
// step, the barrier, the tile loads). All operands stay in VGPRs.
//
// Causal: a query block visits the key tiles up to its diagonal, the four of
// the diagonal 256 x 256 block first, in a step variant that masks each score
// by comparing its key with the lane's query, then the others unmasked: two
// straight runs of steps with no join between masked and unmasked code (a
// join made the compiler copy the accumulators and spill). Each XCD runs the
// query blocks of its heads longest-first (gr_causal_order).
//
// LDS: K^T tiles [128][64] and V tiles [64][128] of 16 KiB in two 5-slot
// rings (160 KiB, all of a CU's LDS); tiles are loaded two steps ahead, one
// barrier per tile. Q is staged through two ring slots before the first tiles
// fill them, and O through the ring at the end.
//
// Softmax: the base m of a row is the max of its first tile's scaled scores;
// p = 2^(s c - m). A step with a row sum past the P type's range (a row max
// that grew by about 2^16 for fp16; an fp32 overflow for bf16) is redone on a
// slow path that moves the base and rescales the accumulators.
//
// Hazards the compiler does not see through inline assembly are kept apart
// by construction: every score register is read by the vector unit at least
// four slots after the MFMA that wrote it, every P register is read by an
// MFMA at least eight slots after the vector op that wrote it, and the slow
// path and the end of the loop are fenced with s_nop.
#pragma once
#include "gr_gemm.h"

#define GR_W2H_GUARD "s_nop 7\n\ts_nop 7\n\ts_nop 3"

template <class T>
struct gr_w2h_ops;
template <>
struct gr_w2h_ops<_Float16> {
  static constexpr const char* mfma = "v_mfma_f32_32x32x16_f16";
  static constexpr const char* pack = "v_cvt_pk_f16_f32";
  static constexpr float sum_max = 65504.f;     // a p past this overflows the packed fp16
};
template <>
struct gr_w2h_ops<__bf16> {
  static constexpr const char* mfma = "v_mfma_f32_32x32x16_bf16";
  static constexpr const char* pack = "v_cvt_pk_bf16_f32";
  static constexpr float sum_max = 3.0e38f;     // only an fp32 overflow
};

// The vector work of one slot on score x: t = 2^(x c + nm), the previous
// slot's t (tp) added into the row sum. A vector op that reads the result of
// a transcendental op (v_exp_f32) must issue at least one instruction after
// it (the compiler does not insert that wait state inside inline assembly):
// the add of tp sits between the exponential and the pack that reads t.
#define GR_W2H_V0 "v_fma_f32 %[t], %[x], %[c], %[nm]\n\tv_exp_f32 %[t], %[t]\n\tv_add_f32 %[la], %[la], %[tp]\n\t"
// masked: the score is dropped (-inf) unless its key offset kc <= delta
#define GR_W2H_V0M                                           \
  "v_fma_f32 %[t], %[x], %[c], %[nm]\n\t"                    \
  "v_cmp_ge_i32 vcc, %[dl], %[kc]\n\t"                       \
  "v_cndmask_b32 %[t], %[ninf], %[t], vcc\n\t"               \
  "v_exp_f32 %[t], %[t]\n\t"                                 \
  "v_add_f32 %[la], %[la], %[tp]\n\t"

template <class T, bool CAUSAL>
__device__ __forceinline__ void gr_flash_w2h_body(const gr_attn_args& a, char* lds) {
  typedef gr_mfma<T> MF;
  typedef typename MF::vec8 vec8;
  typedef gr_w2h_ops<T> OP;
  constexpr int D = 128, BNT = 64, BM = 256, NT = 512, NSLOT = 5;
  constexpr int TILE = BNT * D * 2;                 // bytes of a K^T or a V tile
  constexpr int VOFF = NSLOT * TILE;                // V ring after the K^T ring

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int N = a.N, nqt = N / BM;
  int bh, qt;
  if constexpr (CAUSAL) {
    // the query blocks nearest the end (the most key tiles) first
    gr_causal_order((int)blockIdx.x, (int)gridDim.x, nqt, bh, qt);
    qt = nqt - 1 - qt;
  } else {
    const int logical = gr_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    bh = logical / nqt;
    qt = logical % nqt;
  }
  const int b = bh / a.H, h = bh % a.H;
  const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
  const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
  const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
  T* Op = (T*)a.o + b * a.o_sb + h * a.o_sh;
  const int qw = qt * BM + wave * 32;               // this wave's 32 queries
  const float c = a.scale_log2;
  const int ntile = CAUSAL ? 4 * (qt + 1) : N / BNT;
  // key block of the t-th tile processed: causal takes the four diagonal
  // (masked) blocks first, then blocks 0 .. 4 qt - 1, so that every masked
  // step comes before every unmasked one
  auto kblk = [&](int t) -> int { return CAUSAL ? (t < 4 ? 4 * qt + t : t - 4) : t; };

  // K^T [128][64] and V [64][128] tiles, straight into the two rings
  typedef gr_lds_loader<T, D, BNT, NT, true> KL;
  typedef gr_lds_loader<T, BNT, D, NT, true> VL;
  static_assert(KL::PER == 2 && VL::PER == 2 && KL::CHUNKS == 2 * NT && VL::CHUNKS == 2 * NT, "two chunks per thread");
  constexpr int PER_TILE = KL::PER + VL::PER;       // direct loads per thread and tile
  KL kl;
  VL vl;
  kl.init(tid, a.k_sn);
  vl.init(tid, a.v_sn);
  const unsigned kgo0 = (unsigned)kl.goff[0] * 2u, kgo1 = (unsigned)kl.goff[1] * 2u;
  const unsigned vgo0 = (unsigned)vl.goff[0] * 2u, vgo1 = (unsigned)vl.goff[1] * 2u;
  const unsigned lbase = gr_lds_addr(lds) + kl.lwave;
  auto slot_of = [&](int t) -> int { return t % NSLOT; };
  // one tile: two direct loads of K^T and two of V per thread, from wave-uniform
  // (scalar) tile bases plus the lane's constant byte offsets; M0 (the LDS
  // destination) is saved and restored once for the four
  auto load_tile = [&](int t) {
    if (t < ntile) {
      const T* kb = Kp + (long long)kblk(t) * BNT;
      const T* vb = Vp + (long long)kblk(t) * BNT * a.v_sn;
      const unsigned kd = lbase + slot_of(t) * TILE, vd = kd + VOFF;
      unsigned saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %3\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %2, %1\n\t"
          "s_mov_b32 m0, %5\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %4, %1\n\t"
          "s_mov_b32 m0, %8\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %7, %6\n\t"
          "s_mov_b32 m0, %10\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %9, %6\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(kb), "v"(kgo0), "s"(kd), "v"(kgo1), "s"(kd + NT * 16), "s"(vb), "v"(vgo0), "s"(vd), "v"(vgo1),
            "s"(vd + NT * 16)
          : "memory");
    }
  };
  // Lane base of two transposing reads (gr_tr_frag) of a tile with ROWB-byte
  // rows at k0 = 0, swizzled by gr_swz_tr: rows k0 + 4h lie (k0 + 4h) * ROWB
  // bytes further on, as the swizzle depends on row bits 0-1 only
  auto tr_base = [&](int n0, bool perm, auto rowb_tag) -> int {
    constexpr int ROWB = decltype(rowb_tag)::value;
    const int cq = lane & 3;
    const int cc = perm ? (((cq & 1) << 1) | (cq >> 1)) : cq;
    const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * cc;
    const int row = 8 * (lane >> 5) + ((lane >> 2) & 3);
    return row * ROWB + gr_swz_tr<ROWB / 16>(row, col >> 3) * 16 + (col & 7) * 2;
  };
  auto tr2 = [&](int off, auto rowb_tag) -> vec8 {
    constexpr int ROWB = decltype(rowb_tag)::value;
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    gr_u32x4 r;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const char* p = lds + off + hh * 4 * ROWB;
      const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(__attribute__((address_space(3))) char*)(char*)p);
      const gr_u32x2 w = __builtin_bit_cast(gr_u32x2, v);
      r[2 * hh] = w[0];
      r[2 * hh + 1] = w[1];
    }
    return gr_as<vec8>(r);
  };
  // K fragment (32-key half kb, depth block ds: keys in perm32 order, so that
  // the score accumulators are the P.V MFMAs' operand) and V fragment (16-key
  // chunk cc, head-dim block db) of the tile in ring slot `slot`
  int kbase[2], vbase[4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) kbase[kb] = tr_base(kb * 32, true, gr_ic<BNT * 2>{});
#pragma unroll
  for (int db = 0; db < 4; ++db) vbase[db] = VOFF + tr_base(db * 32, false, gr_ic<D * 2>{});
  auto kfrag = [&](int slot, int kb, int ds) -> vec8 { return tr2(kbase[kb] + slot * TILE + ds * 16 * (BNT * 2), gr_ic<BNT * 2>{}); };
  auto vfrag = [&](int slot, int cc, int db) -> vec8 { return tr2(vbase[db] + slot * TILE + cc * 16 * (D * 2), gr_ic<D * 2>{}); };

  // Prologue: each wave's 32 Q rows into 8 KiB of ring slots 3 and 4 (before
  // tiles 3 and 4 fill them), tiles 0, 1 and 2. Once Q and tile 0 have
  // landed, Q goes into registers and tile 0's scores are computed while
  // tiles 1 and 2 are still in flight; tile 3 is loaded once tile 1 has
  // landed and every wave has read its Q.
  char* const qstage = lds + (wave < 4 ? 3 * TILE + wave * 8192 : VOFF + 3 * TILE + (wave - 4) * 8192);
  {
    gr_lds_loader<T, 32, D, 64> ql;
    ql.init(lane, a.q_sn);
    ql.load(Qp + (long long)qw * a.q_sn, qstage);
  }
  load_tile(0);
  load_tile(1);
  load_tile(2);
  gr_wait_vmcnt<2 * PER_TILE>();                  // Q and tile 0 (every tile exists: ntile >= 4)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  vec8 qf[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) qf[ds] = gr_as<vec8>(gr_ld16(qstage + l32 * (D * 2) + gr_swz<D / 8>(l32, 2 * ds + g) * 16));

  // a score's key offset within its tile (perm32 order): element r of half kb
  // is key 32 kb + 16 (r / 8) + 8 g + r % 8; the lane's query is qw + l32
  const float ninf = -__builtin_inff();
  auto visible = [&](int t, int kb, int r) -> bool {
    return 64 * kblk(t) + 32 * kb + 16 * (r >> 3) + 8 * g + (r & 7) <= qw + l32;
  };

  // tile 0: scores from zero, the base from their (scaled) row max, P(0)
  gr_f32x16 sA[2], sB[2];
  float nm, lsum;
  gr_u32x4 pA[4], pB[4];                     // P of a tile, [16-key chunk]
  {
    gr_f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = (gr_f32x16)(0.f);
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) s[kb] = MF::mma32(kfrag(0, kb, ds), qf[ds], s[kb]);
    }
    float mt = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = s[kb][r] * c;
        s[kb][r] = (!CAUSAL || visible(0, kb, r)) ? v : ninf;
        mt = fmaxf(mt, s[kb][r]);
      }
    mt = fmaxf(mt, gr_xor32(mt));
    nm = -mt;
    float l = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float p0 = gr_exp2(s[kb][8 * hf + e] - mt), p1 = gr_exp2(s[kb][8 * hf + e + 1] - mt);
          pB[2 * kb + hf][e >> 1] = gr_pack2f<T>(p0, p1);
          l += p0 + p1;
        }
    lsum = l;
  }
  // tile 1 landed, and every wave has read its Q (slots 3 and 4 are free)
  gr_wait_vmcnt<PER_TILE>();
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  load_tile(3);
  // tile 1's scores (unscaled, from zero)
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    gr_f32x16 s = MF::mma32(kfrag(1, kb, 0), qf[0], (gr_f32x16)(0.f));
#pragma unroll
    for (int ds = 1; ds < 8; ++ds) s = MF::mma32(kfrag(1, kb, ds), qf[ds], s);
    sA[kb] = s;
  }
  gr_f32x16 o[4];                            // O^T accumulators [head-dim block]
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = (gr_f32x16)(0.f);

  // Step j: S_next = scores of tile j + 1 (unscaled, from zero), P_cur = P of
  // tile j (from S_cur, masked on diagonal tiles), O += V^T P_prev (tile j - 1).
  // K fragments of tile j + 1 and V fragments of tile j - 1 are read just in
  // time into two-deep rings: the score MFMA of slot 2q (q = 0..15: half kb =
  // q % 2, depth ds = q / 2) takes kq[q % 2], the P.V MFMA of slot 2p + 1 (p =
  // 0..15: head-dim block db = p % 4, chunk cc = p / 4) vp[p % 2]; each is
  // refilled after the slot that used it, the first two at the step's start.
  // The vector work of slot s is score s of tile j (half s / 16, element
  // s % 16); odd slots pack their pair into P_cur.
  auto step = [&](int j, auto mask_tag, gr_f32x16 (&S_cur)[2], gr_f32x16 (&S_next)[2], gr_u32x4 (&P_cur)[4],
                  gr_u32x4 (&P_prev)[4]) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int sk = slot_of(j + 1), sv = slot_of(j + NSLOT - 1);
    // this step's fragment bases, opaque to the compiler: each read is then a
    // base plus an immediate, rather than one hoisted address per fragment
    int ka[2], va[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) ka[kb] = kbase[kb] + sk * TILE;
#pragma unroll
    for (int db = 0; db < 4; ++db) va[db] = vbase[db] + sv * TILE;
    asm volatile("" : "+v"(ka[0]), "+v"(ka[1]), "+v"(va[0]), "+v"(va[1]), "+v"(va[2]), "+v"(va[3]));
    auto kf = [&](int kb, int ds) -> vec8 { return tr2(ka[kb] + ds * 16 * (BNT * 2), gr_ic<BNT * 2>{}); };
    auto vf = [&](int cc, int db) -> vec8 { return tr2(va[db] + cc * 16 * (D * 2), gr_ic<D * 2>{}); };
    vec8 kq[2], vp[2];
    kq[0] = kf(0, 0);
    kq[1] = kf(1, 0);
    vp[0] = vf(0, 0);
    vp[1] = vf(0, 1);
    // masking: score (kb, r) of tile j is kept iff 16 (r / 8) + r % 8 <=
    // delta - 32 kb, with delta = qw + l32 - 64 j - 8 g
    const int delta = qw + l32 - 64 * kblk(j) - 8 * g;
    float la = 0.f, tA = 0.f, tB = 0.f;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      const int kb = s >> 4, r = s & 15, q = s >> 1;
      float& t = (s & 1) ? tB : tA;            // this slot's p
      float& tp = (s & 1) ? tA : tB;           // the previous slot's (0 at s = 0)
      const int dl = delta - 32 * kb;
#define GR_W2H_VIN [x] "v"(S_cur[kb][r]), [c] "s"(c), [nm] "v"(nm), [tp] "v"(tp)
#define GR_W2H_MIN [dl] "v"(dl), [kc] "n"(16 * (r >> 3) + (r & 7)), [ninf] "v"(ninf)
      // one slot: MFMA text MT with its operand lists MO (outputs) and MI
      // (inputs), then the slot's vector work (masked or not, packing or not)
#define GR_W2H_SLOT(MT, PK, MO, MI)                                                                                   \
  if constexpr (MASK) {                                                                                               \
    if (s & 1)                                                                                                        \
      asm volatile(MT GR_W2H_V0M PK " %[pk], %[tp], %[t]\n\t"                                                         \
                   : MO, [t] "=&v"(t), [la] "+v"(la), [pk] "=&v"(P_cur[s >> 3][(s >> 1) & 3]) : MI, GR_W2H_VIN, GR_W2H_MIN : "vcc");          \
    else                                                                                                              \
      asm volatile(MT GR_W2H_V0M : MO, [t] "=&v"(t), [la] "+v"(la) : MI, GR_W2H_VIN, GR_W2H_MIN : "vcc");            \
  } else {                                                                                                            \
    if (s & 1)                                                                                                        \
      asm volatile(MT GR_W2H_V0 PK " %[pk], %[tp], %[t]\n\t"                                                          \
                   : MO, [t] "=&v"(t), [la] "+v"(la), [pk] "=&v"(P_cur[s >> 3][(s >> 1) & 3]) : MI, GR_W2H_VIN);                               \
    else                                                                                                              \
      asm volatile(MT GR_W2H_V0 : MO, [t] "=&v"(t), [la] "+v"(la) : MI, GR_W2H_VIN);                                 \
  }
#define GR_W2H_KINDS(MFMA, PK)                                                                                        \
  if ((s & 1) == 0 && q < 2) {                                                                                        \
    GR_W2H_SLOT(MFMA " %[d], %[ka], %[qb], 0\n\t", PK, [d] "=&v"(S_next[q & 1]),                                     \
                [ka] "v"(kq[q & 1]) GR_W2H_COMMA [qb] "v"(qf[q >> 1]))                                                \
  } else if ((s & 1) == 0) {                                                                                          \
    GR_W2H_SLOT(MFMA " %[d], %[ka], %[qb], %[d]\n\t", PK, [d] "+v"(S_next[q & 1]),                                   \
                [ka] "v"(kq[q & 1]) GR_W2H_COMMA [qb] "v"(qf[q >> 1]))                                                \
  } else {                                                                                                            \
    GR_W2H_SLOT(MFMA " %[d], %[va], %[pb], %[d]\n\t", PK, [d] "+v"(o[q & 3]),                                        \
                [va] "v"(vp[q & 1]) GR_W2H_COMMA [pb] "v"(gr_as<vec8>(P_prev[q >> 2])))                               \
  }
#define GR_W2H_COMMA ,
      if constexpr (gr_is_same<T, __bf16>::value) {
        GR_W2H_KINDS("v_mfma_f32_32x32x16_bf16", "v_cvt_pk_bf16_f32")
      } else {
        GR_W2H_KINDS("v_mfma_f32_32x32x16_f16", "v_cvt_pk_f16_f32")
      }
#undef GR_W2H_COMMA
#undef GR_W2H_KINDS
#undef GR_W2H_SLOT
#undef GR_W2H_MIN
#undef GR_W2H_VIN
      // refill the ring entry this slot used with the fragment two such slots ahead
      if ((s & 1) == 0) {
        if (q + 2 < 16) kq[q & 1] = kf(q & 1, (q + 2) >> 1);
      } else {
        if (q + 2 < 16) vp[q & 1] = vf((q + 2) >> 2, (q + 2) & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the last score's p joins the sum; the step's row sums to fp32 lsum
    asm volatile("v_add_f32 %0, %0, %1" : "+v"(la) : "v"(tB));
    float ltq = la;
    // a p (or a row sum) past the P type's range reads as > sum_max (or NaN)
    if (__builtin_expect(gr_any(!(ltq <= OP::sum_max)), 0)) {
      asm volatile(GR_W2H_GUARD : "+v"(S_next[0]), "+v"(S_next[1]), "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
      // Slow path: the base moves to the true (scaled) row max of tile j,
      // O and the row sum are rescaled, and P of tile j is recomputed.
      float mt = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!MASK || visible(j, kb, r)) mt = fmaxf(mt, S_cur[kb][r] * c);
      mt = fmaxf(mt, gr_xor32(mt));
      const float sh = fmaxf(mt + nm, 0.f);   // the base moves up by sh
      const float alpha = gr_exp2(-sh);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      nm -= sh;
      float l = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const int r = 8 * hf + e;
            const float p0 = (!MASK || visible(j, kb, r)) ? gr_exp2(fmaf(S_cur[kb][r], c, nm)) : 0.f;
            const float p1 = (!MASK || visible(j, kb, r + 1)) ? gr_exp2(fmaf(S_cur[kb][r + 1], c, nm)) : 0.f;
            P_cur[2 * kb + hf][e >> 1] = gr_pack2f<T>(p0, p1);
            l += p0 + p1;
          }
      ltq = l;
      asm volatile(GR_W2H_GUARD : "+v"(S_next[0]), "+v"(S_next[1]), "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]),
                   "+v"(P_cur[0]), "+v"(P_cur[1]), "+v"(P_cur[2]), "+v"(P_cur[3]));
    }
    lsum += ltq;
  };

  asm volatile(GR_W2H_GUARD : "+v"(sA[0]), "+v"(sA[1]), "+v"(pB[0]), "+v"(pB[1]), "+v"(pB[2]), "+v"(pB[3]), "+v"(o[0]),
               "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
  // The barrier before step j publishes tile j + 1 (tile j + 2 may stay in
  // flight) and frees tile j - 2's slot for tile j + 3.
  auto publish = [&](int j) {
    if (j + 2 < ntile) gr_wait_vmcnt<PER_TILE>(); else gr_wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    load_tile(j + 3);
  };
  // Steps 1 .. ntile - 1 (an odd count), the score and P buffers alternating
  // with the step's parity: step 1, then pairs; causal: steps 1 - 3 (the rest
  // of the diagonal block) masked, every later step unmasked.
  publish(1);
  step(1, gr_ic<CAUSAL>{}, sA, sB, pA, pB);
  int j = 2;
  if constexpr (CAUSAL) {
    publish(2);
    step(2, gr_ic<1>{}, sB, sA, pB, pA);
    publish(3);
    step(3, gr_ic<1>{}, sA, sB, pA, pB);
    j = 4;
  }
  for (; j < ntile; j += 2) {
    publish(j);
    step(j, gr_ic<0>{}, sB, sA, pB, pA);
    publish(j + 1);
    step(j + 1, gr_ic<0>{}, sA, sB, pA, pB);
  }
  // P.V of the last tile (its P in pA: ntile - 1 is odd)
  {
    const int sv = slot_of(ntile - 1);
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const vec8 vf = vfrag(sv, p >> 2, p & 3);
      if constexpr (gr_is_same<T, __bf16>::value)
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(o[p & 3]) : "v"(vf), "v"(gr_as<vec8>(pA[p >> 2])));
      else
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(o[p & 3]) : "v"(vf), "v"(gr_as<vec8>(pA[p >> 2])));
    }
  }
  asm volatile(GR_W2H_GUARD : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
  gr_wait_vmcnt<0>();
  __syncthreads();   // every wave past its last ring reads: the O staging reuses the ring

  // O = O^T^T / l, staged through this wave's 8 KiB of the ring (where its Q
  // was) as whole 16-byte row chunks
  constexpr int CPR = D / 8;
  const float inv = 1.0f / (lsum + gr_xor32(lsum));
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      gr_u32x2 w;
      w[0] = gr_pack2f<T>(o[db][4 * rr + 0] * inv, o[db][4 * rr + 1] * inv);
      w[1] = gr_pack2f<T>(o[db][4 * rr + 2] * inv, o[db][4 * rr + 3] * inv);
      *reinterpret_cast<gr_u32x2*>(qstage + l32 * (D * 2) + gr_swz<CPR>(l32, db * 4 + rr) * 16 + g * 8) = w;
    }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < 32 * CPR / 64; ++it) {
    const int jj = it * 64 + lane, row = jj / CPR, ch = jj % CPR;
    const gr_u32x4 v = gr_ld16(qstage + row * (D * 2) + gr_swz<CPR>(row, ch) * 16);
    __builtin_nontemporal_store(v, reinterpret_cast<gr_u32x4*>(Op + (long long)(qw + row) * a.o_sn + ch * 8));
  }
}

// LDS bytes: five K^T tile slots and five V tile slots of 16 KiB (all 160 KiB)
constexpr int GR_FLASH_W2H_LDS = 2 * 5 * 64 * 128 * 2;

template <class T, bool CAUSAL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void gr_flash_w2h_kernel(gr_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) char gr_lds[];
  gr_flash_w2h_body<T, CAUSAL>(a, gr_lds);
}
