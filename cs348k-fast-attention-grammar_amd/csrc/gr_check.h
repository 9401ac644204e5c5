// gr_check.h -- the checking build of the generic LDS-tile lowering.
//
// A module rendered with check=True routes every LDS access of its generic
// stages through GR_LR (read) / GR_LW (write), every global index through
// GR_GI, and every workgroup barrier through GR_SYNC. Nothing faults: an
// out-of-range index is counted and replaced by 0 (in range), and every
// finding is counted in a small device buffer (the stage's last argument) that
// the host reads back after the run.
//
// Races: the generic lowering separates its statements by barriers; two
// accesses to one LDS word by different threads between the same two
// barriers, at least one of them a write, are a race. Each LDS float has two
// shadow words behind the stage's tiles (so the checking build needs three
// times the LDS): the stamp (barrier interval, thread) of its last write and
// of its last read. A read finds a write of another thread in the current
// interval (RAW); a write finds a read (WAR) or write (WAW) of another thread.
// The shadow updates are themselves unsynchronised, so a race can go
// unreported when several threads touch one word in one interval (the last
// reader's stamp hides earlier ones); a reported race is always real.
#pragma once
#include "gr_common.h"

enum {
  GR_CHK_LDS_RANGE = 0,      // LDS index outside the stage's tiles
  GR_CHK_GLOBAL_RANGE = 1,   // global index outside the tensor
  GR_CHK_RAW = 2,            // read of a word another thread wrote since the last barrier
  GR_CHK_WAR = 3,            // write of a word another thread read since the last barrier
  GR_CHK_WAW = 4,            // write of a word another thread wrote since the last barrier
  GR_CHK_FIRST = 8,          // kind + 1 of the first finding (0: none)
  GR_CHK_FIRST_LINE = 9,     // its source line in the rendered module
  GR_CHK_FIRST_INDEX = 10,   // its index
  GR_CHK_WORDS = 16
};

__device__ __forceinline__ void gr_chk_note(unsigned int* chk, int kind, int line, long long idx) {
  atomicAdd(chk + kind, 1u);
  if (atomicCAS(chk + GR_CHK_FIRST, 0u, (unsigned int)kind + 1u) == 0u) {
    chk[GR_CHK_FIRST_LINE] = (unsigned int)line;
    chk[GR_CHK_FIRST_INDEX] = (unsigned int)idx;
  }
}

// stamp: barrier interval (low 20 bits) above the thread index + 1
__device__ __forceinline__ unsigned int gr_chk_stamp(unsigned int epoch) {
  return (epoch << 12) | (threadIdx.x + 1u);
}

__device__ __forceinline__ bool gr_chk_other(unsigned int stamp, unsigned int me) {
  return (stamp >> 12) == (me >> 12) && stamp != me;
}

__device__ __forceinline__ int gr_chk_lds_r(unsigned int* chk, unsigned int* sh, int i, int n, unsigned int epoch,
                                            int line) {
  if (i < 0 || i >= n) {
    gr_chk_note(chk, GR_CHK_LDS_RANGE, line, i);
    return 0;
  }
  const unsigned int me = gr_chk_stamp(epoch);
  if (gr_chk_other(sh[2 * i], me)) gr_chk_note(chk, GR_CHK_RAW, line, i);
  sh[2 * i + 1] = me;
  return i;
}

__device__ __forceinline__ int gr_chk_lds_w(unsigned int* chk, unsigned int* sh, int i, int n, unsigned int epoch,
                                            int line) {
  if (i < 0 || i >= n) {
    gr_chk_note(chk, GR_CHK_LDS_RANGE, line, i);
    return 0;
  }
  const unsigned int me = gr_chk_stamp(epoch);
  if (gr_chk_other(sh[2 * i], me)) gr_chk_note(chk, GR_CHK_WAW, line, i);
  if (gr_chk_other(sh[2 * i + 1], me)) gr_chk_note(chk, GR_CHK_WAR, line, i);
  sh[2 * i] = me;
  return i;
}

__device__ __forceinline__ long long gr_chk_g(unsigned int* chk, long long i, long long n, int line) {
  if (i < 0 || i >= n) {
    gr_chk_note(chk, GR_CHK_GLOBAL_RANGE, line, i);
    return 0;
  }
  return i;
}

// The instrumented kernel defines gr_chk (the buffer), gr_sh (the shadow
// words), gr_nfl (LDS floats of its tiles) and gr_epoch (barrier interval).
#define GR_LR(i) gr_lds[gr_chk_lds_r(gr_chk, gr_sh, (i), gr_nfl, gr_epoch, __LINE__)]
#define GR_LW(i) gr_lds[gr_chk_lds_w(gr_chk, gr_sh, (i), gr_nfl, gr_epoch, __LINE__)]
#define GR_GI(i, n) gr_chk_g(gr_chk, (long long)(i), (n), __LINE__)
#define GR_SYNC()    \
  do {               \
    __syncthreads(); \
    ++gr_epoch;      \
  } while (0)
