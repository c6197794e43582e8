// Within-cluster top-q: for every (row, cluster) with quota q_c > 0, the q_c tail members of the
// cluster with the highest QGS score (ties to the lower position) become exact reads.
//
// Reference semantics: the per-token rank within its bin by the selector score
// (multibin.py:2522-2558, trunc_keep = rank < quota) with the deployed tie order of
// ours_graph.py:93-135 / ours_fused.py:228-282 (score, then members before generated tokens,
// then position -- i.e. position order, since every generated token follows the prefix).
// Selected, sink, local and unwritten positions carry a -inf score and never qualify.
//
// exp_idx row layout: cluster c owns slots [base_c, base_c + q_c), base_c = sum_{c'<c} q_c';
// a segment lists its chosen members in position order and is -1 past them; slots past sum q
// are -1.  Only E slots exist: a segment straddling E keeps its best E - base_c members.
//
// gfx950 decomposition: one 1024-thread workgroup per row.  About 40 of 64 clusters carry a
// quota and their members cover most of the row, so the row is streamed (scores S and byte
// cluster ids asg8, coalesced) into registers -- 1024 * PPT positions at a time, PPT per
// thread -- and every selection step works on those registers and on LDS.  Scores are
// compared through their order-preserving 32-bit key, whose bits are taken LB at a time (LB =
// 8, 7 or 6 for C <= 64, 128, 256) by successive histogram levels:
//   L1  per-cluster histogram of the top LB key bits (LDS atomics).  Histogram rows carry one
//       pad word after every NB/16 bins, so the 16 threads that scan a row read 16 banks;
//   T1  16 threads per cluster: t = min(q_c, members, E - base_c) and the level-1 bin holding
//       the t-th best member; every cluster now has a boundary bin [klo, khi] of keys.  Members
//       above it are chosen; a cluster whose whole bin completes t is done, the others are split;
//   G   every member at or above its cluster's boundary bin (a few thousand of the row's
//       members) is gathered into an LDS list: per-thread hit masks, one scan per wave and one
//       LDS atomic per wave, no per-member atomics;
//   refinement levels, while any cluster is split: the histogram of the next LB key bits of
//       each split cluster's boundary-bin members (built from the list, about 5 entries per
//       thread), then the bin holding its t-th member.  A cluster whose new bin fits in the LDS
//       staging space is staged; one that does not stays split for the next level; at full key
//       depth (only equal keys left) it is resolved block-wide in P5.  When the level-1 set
//       does not fit the list, the levels run over the registers instead and G follows them,
//       with the final bins;
//   F   one pass over the list: members above the boundary bin are chosen (written straight into
//       their cluster's segment of the chosen-word list), members inside a staged cluster's bin
//       become unique 64-bit keys (score key << 32 | ~position);
//   P5  one wave per staged cluster picks the `need` best staged keys (repeated wave maxima for
//       small `need`, an MSB-first bitwise search on ballot counts otherwise, over the key bits
//       the bin leaves open); equal keys beyond the staging space are ranked by position in a
//       block-wide bitwise search that streams the row again.  (The linear-bin kernel below
//       ranks the keys of clusters with at most 128 staged keys one thread per key instead);
//   P6  every chosen (cluster << 24 | position) word gets its rank among its cluster's words by
//       position (counting, or a bitonic sort when one cluster has more than 1024), lands in an
//       LDS copy of the exp_idx row, and the row is written out once (-1 where a segment is
//       short).
// Rows longer than 1024 * PPT positions are processed in segments that are re-read from
// global memory (L2 / Infinity Cache) in each pass.  Rows are read in groups of four
// positions, so both row strides are multiples of 4 and hold round_up(Lmax, 4) entries.
#include <algorithm>

#include "oa_common.h"
#include "oa_score.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxC = 256;
constexpr int kMaxE = 4096;
constexpr int kMaxPos = 1 << 24;               // positions (< 2^24 - 1) are packed into 24 bits
constexpr int kExtractMax = 40;                // need above this: bitwise threshold search
constexpr int kUCapMax = 16384;                // gathered members (u64)
constexpr int kRankTMax = 1024;                // a cluster with more chosen words: bitonic sort
constexpr int kUPT = 8;                        // gathered entries per thread handled together
constexpr unsigned kNegInfKey = 0x007fffffu;   // float_key(-inf)
constexpr unsigned kNoGather = 0xffffffffu;    // gathering bound of a cluster with no quota
constexpr int kLdsLimit = 160 * 1024;
constexpr int kSmallRows = 256;               // below: oa_topq_heads path 0 in one launch
constexpr int32_t kRowMarked = -2;              // exp_idx[row][0] of a row left to the key-prefix kernel
constexpr int kTileLd = 3;                      // tile extremes per thread (linear-bin kernel)
constexpr int kRowGrid = 64;                    // key-prefix kernel over marked rows: workgroups

enum : int { kModeNone = 0, kModeAll = 1, kModeStaged = 2, kModeBlock = 3, kModeSplit = 4 };

struct TopqArgs {
  const float* S; long s_stride;
  const uint8_t* asg8; long a_stride;
  const float* quota; int C; int E; const int* n_dev;
  int32_t* exp_idx;
  int lb;          // bits per histogram level (8, 7 or 6)
  int ucap;        // gathered-member list capacity (entries; 64 per-lane trash slots follow)
  int hwords;      // ints of the area holding the histogram, then the staged keys, then the row
  int gcap;        // staged-key capacity (u64 entries)
  int cpow;        // power of two >= E: chosen-word list and the P6 sort
  int marked_only; // key-prefix kernel: only rows the linear-bin kernel marked kRowMarked
  int rows;        // rows of the launch (the marked-only grid walks them)
  // linear-bin kernel over 16-bit key heads (oa_topq_heads): the head rows, and what recomputes
  // exact scores (the staged members', and a whole row into S32 when it is left to the
  // key-prefix kernel, which then reads S32 as its S)
  const uint16_t* H; long h_stride;
  const int8_t* codes; long lmax_codes; const int8_t* limbs; const int* fexp;
  float* S32; long s32_stride;
  int force_mark;  // tests: every row is left to the key-prefix kernel
  // optional (linear-bin kernel over heads): each 64-position tile's greatest score (TM) and
  // least finite score (TMn) from the scan; then the row's range comes from them instead of a
  // pass over the row, and every group of positions is binned as soon as it arrives
  const float* TM; const float* TMn; long tm_stride;
};

// the largest t = head - 0x7f of a finite float (head 0xff7f): the linear-bin kernel caps t here
constexpr uint16_t kTopT = 0xff00;

__device__ __forceinline__ unsigned long long key64(uint32_t key, int pos) {
  return ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - (unsigned)pos);
}

// The staged keys of one cluster lie in its boundary bin [klo, khi] of score keys (khi = klo |
// (2^w - 1)): they share klo's top 32 - w bits and, since positions are below 2^24, bits 24..31
// of the inverted position.  A bitwise threshold search starts from those bits (bin_floor) and
// decides only the others, from bit 31 + w down, skipping 31..24.
__device__ __forceinline__ unsigned long long bin_floor(uint32_t klo, uint32_t top8 = 0xffu) {
  return ((unsigned long long)klo << 32) | ((unsigned long long)top8 << 24);
}
// the linear-bin kernel's staged keys carry 255 - cluster in bits 24..31 instead (constant within
// a cluster, so the order of one cluster's keys is unchanged): one thread can then rank a key
// against the rest of its cluster's keys
__device__ __forceinline__ unsigned long long staged_key(uint32_t key, int c, int pos) {
  return ((unsigned long long)key << 32) | ((uint32_t)(255 - c) << 24) | (0xffffffu - (uint32_t)pos);
}
__device__ __forceinline__ uint32_t key_pos(unsigned long long x) {
  return 0xffffffu - (uint32_t)(x & 0xffffffull);
}
__device__ __forceinline__ int bin_top_bit(uint32_t klo, uint32_t khi) {
  const int w = __popc(klo ^ khi);
  return w > 0 ? 31 + w : 23;
}
__device__ __forceinline__ int next_free_bit(int bit) { return bit == 32 ? 23 : bit - 1; }

// append one chosen (cluster << 24 | position) word per taking lane, one LDS atomic per wave
__device__ __forceinline__ void append_chosen(bool take, uint32_t word, uint32_t* cst, int* ctr,
                                              int lane) {
  const unsigned long long bal = __ballot(take);
  if (bal == 0ull) return;
  const int leader = __ffsll((long long)bal) - 1;
  int off = 0;
  if (lane == leader) off = atomicAdd(ctr, __popcll(bal));
  off = __builtin_amdgcn_readlane(off, leader);   // the leader is uniform
  if (take) cst[off + __popcll(bal & ((1ull << lane) - 1ull))] = word;
}

// P5 on one staged cluster: the `need` largest of cnt unique keys, held KR per lane
template <int KR>
__device__ void select_staged(const unsigned long long* src, int cnt, int need, int c,
                              unsigned long long floor, int top, uint32_t* cst, int* ctr, int lane) {
  if (KR == 1) {
    // at most 64 keys, one per lane: each key's rank is the number of larger keys (the keys are
    // distinct), counted over broadcast LDS reads; the `need` best have rank < need
    const unsigned long long x = src[min(lane, cnt - 1)];
    int rank = 0;
    for (int m = 0; m < cnt; ++m) rank += src[m] > x ? 1 : 0;
    const bool take = lane < cnt && rank < need;
    append_chosen(take, ((uint32_t)c << 24) | key_pos(x), cst, ctr, lane);
    return;
  }
  unsigned long long x[KR];
#pragma unroll
  for (int j = 0; j < KR; ++j) x[j] = src[min(j * 64 + lane, cnt - 1)];
#pragma unroll
  for (int j = 0; j < KR; ++j) x[j] = j * 64 + lane < cnt ? x[j] : 0ull;
  unsigned long long T = 0ull;
  if (need <= kExtractMax) {
    unsigned taken = 0u;
    for (int k = 0; k < need; ++k) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int j = 0; j < KR; ++j)
        if (!((taken >> j) & 1u) && x[j] > best) best = x[j];
      best = oa::wave_max_u64(best);
#pragma unroll
      for (int j = 0; j < KR; ++j)
        if (x[j] == best) taken |= 1u << j;
      T = best;
    }
  } else {
    T = floor;
    for (int bit = top; bit >= 0; bit = next_free_bit(bit)) {
      const unsigned long long cnd = T | (1ull << bit);
      int k = 0;
#pragma unroll
      for (int j = 0; j < KR; ++j) k += __popcll(__ballot(x[j] >= cnd));
      if (k >= need) T = cnd;
    }
  }
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const bool take = x[j] != 0ull && x[j] >= T;
    append_chosen(take, ((uint32_t)c << 24) | key_pos(x[j]), cst, ctr, lane);
  }
}

// the same from LDS in a loop, for more than 512 staged keys
__device__ void select_staged_loop(const unsigned long long* src, int cnt, int need, int c,
                                   unsigned long long floor, int top, uint32_t* cst, int* ctr,
                                   int lane) {
  unsigned long long T = floor;
  for (int bit = top; bit >= 0; bit = next_free_bit(bit)) {
    const unsigned long long cnd = T | (1ull << bit);
    int k = 0;
    for (int b0 = 0; b0 < cnt; b0 += 64) {
      const int j = b0 + lane;
      k += __popcll(__ballot(j < cnt && src[min(j, cnt - 1)] >= cnd));
    }
    if (k >= need) T = cnd;
  }
  for (int b0 = 0; b0 < cnt; b0 += 64) {
    const int j = b0 + lane;
    const unsigned long long x = src[min(j, cnt - 1)];
    const bool take = j < cnt && x >= T;
    append_chosen(take, ((uint32_t)c << 24) | key_pos(x), cst, ctr, lane);
  }
}

// the float of the key head t + 0x7f (low 16 key bits 0): k & 0x7fffffff for a key with its top
// bit set, ~k otherwise, as an arithmetic shift and one 3-input bit operation
__device__ __forceinline__ float head_float(uint32_t t) {
  uint32_t k = (t + oa::kNegInfHead) << 16;
  asm("" : "+v"(k));      // one key feeds both operands (not a key and its complement)
  uint32_t m = (uint32_t)((int32_t)k >> 31);
  asm("" : "+v"(m));      // keeps the shift (not a compare and select) feeding the bit operation
  return __uint_as_float(~(k ^ (m & 0x7fffffffu)));
}

// 16 threads (one DPP row) scan one padded histogram row of NB = 16 * BPT bins from the top:
// thread j holds bins [j*BPT, (j+1)*BPT) in x[], ls = their sum, sfx = members in its bins and
// all bins above (a suffix scan on row_shl DPP moves: lanes past the row's end read 0)
template <int BPT>
struct RowScan {
  int x[BPT];
  int ls, sfx;
};
template <int BPT>
__device__ __forceinline__ void scan_row(const int* row, int j, RowScan<BPT>& r) {
  const int* h = row + j * (BPT + 1);
  r.ls = 0;
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    r.x[b] = h[b];
    r.ls += r.x[b];
  }
  int v = r.ls;
  v += __builtin_amdgcn_update_dpp(0, v, 0x101, 0xf, 0xf, false);   // row_shl:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x102, 0xf, 0xf, false);   // row_shl:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x104, 0xf, 0xf, false);   // row_shl:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x108, 0xf, 0xf, false);   // row_shl:8
  r.sfx = v;
}
// the same over one of the linear-bin kernel's rows of 16 * BPT bins without pad words: thread j
// holds bins [j*BPT, (j+1)*BPT); bin 0 (non-members) counts nothing
template <int BPT>
__device__ __forceinline__ void scan_row_dense(const int* row, int j, RowScan<BPT>& r) {
  const int* h = row + j * BPT;
  r.ls = 0;
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    r.x[b] = (b == 0 && j == 0) ? 0 : h[b];
    r.ls += r.x[b];
  }
  int v = r.ls;
  v += __builtin_amdgcn_update_dpp(0, v, 0x101, 0xf, 0xf, false);   // row_shl:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x102, 0xf, 0xf, false);   // row_shl:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x104, 0xf, 0xf, false);   // row_shl:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x108, 0xf, 0xf, false);   // row_shl:8
  r.sfx = v;
}
// on the thread whose bins hold the t-th best member (sfx >= t > sfx - ls): the bin (local
// index), the members above it, and the members in it
template <int BPT>
__device__ __forceinline__ void find_bin(const RowScan<BPT>& r, int t, int& bin, int& acc,
                                         int& cnt) {
  acc = r.sfx - r.ls;
  bin = 0;
  cnt = 0;
#pragma unroll
  for (int b = BPT - 1; b >= 0; --b) {
    if (cnt == 0 && acc + r.x[b] >= t) { bin = b; cnt = r.x[b]; }
    else if (cnt == 0) acc += r.x[b];
  }
}


// wave 0: exp_idx segment of each cluster (s_base, exclusive prefix of the quotas) and its
// E-capped quota s_w = min(q_c, E - base_c), clamped at 0
__device__ __forceinline__ void quota_load(const float* qrow, int C, int lane, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = qrow[min(lane * 4 + i, C - 1)];
}
__device__ __forceinline__ void quota_scan(const float* qv, int C, int E, int lane, int* s_base,
                                           int* s_w) {
  int v[4], loc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (int)qv[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = lane * 4 + i < C ? v[i] : 0;
    loc += v[i];
  }
  const int incl = oa::wave_incl_scan_i32(loc);
  int run = incl - loc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane * 4 + i;     // 0..255
    s_base[c] = run;
    s_w[c] = c < C ? max(0, min(v[i], E - run)) : 0;
    run += v[i];
  }
  if (lane == 63) s_base[kMaxC] = incl;
}
__device__ __forceinline__ void quota_prefix(const float* qrow, int C, int E, int lane, int* s_base,
                                             int* s_w) {
  float qv[4];
  quota_load(qrow, C, lane, qv);
  quota_scan(qv, C, E, lane, s_base, s_w);
}

// wave 0: chosen-word segment of each cluster (exclusive prefix of s_t)
__device__ __forceinline__ void chosen_prefix(const int* s_t, int* s_tpre, int lane) {
  int v[4], loc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[i] = s_t[lane * 4 + i]; loc += v[i]; }
  const int incl = oa::wave_incl_scan_i32(loc);
  int run = incl - loc;
#pragma unroll
  for (int i = 0; i < 4; ++i) { s_tpre[lane * 4 + i] = run; run += v[i]; }
  const int mx = (int)oa::wave_max_u32((unsigned)max(max(v[0], v[1]), max(v[2], v[3])));
  if (lane == 63) { s_tpre[kMaxC] = incl; s_tpre[kMaxC + 1] = mx; }
}

// P5 for every staged cluster, one wave per cluster: the `need` best of its staged keys join
// its chosen words
__device__ __forceinline__ void select_all_staged(int C, int wave, int lane, const int* s_mode,
                                                  const int* s_bcnt, const int* s_t,
                                                  const int* s_above,
                                                  const unsigned long long* s_g, const int* s_goff,
                                                  uint32_t* s_cst, const int* s_tpre,
                                                  const unsigned* s_klo, const unsigned* s_khi,
                                                  int* s_ccur, bool tagged = false,
                                                  int min_cnt = -1) {
  for (int c = wave; c < C; c += kWaves) {
    if (s_mode[c] != kModeStaged) continue;
    const int cnt = s_bcnt[c];
    if (cnt <= min_cnt) continue;
    const int need = s_t[c] - s_above[c];
    const unsigned long long* src = s_g + s_goff[c];
    uint32_t* dst = s_cst + s_tpre[c];
    const unsigned long long fl = bin_floor(s_klo[c], tagged ? 255u - (unsigned)c : 0xffu);
    const int top = bin_top_bit(s_klo[c], s_khi[c]);
    if (cnt <= 64) select_staged<1>(src, cnt, need, c, fl, top, dst, &s_ccur[c], lane);
    else if (cnt <= 256) select_staged<4>(src, cnt, need, c, fl, top, dst, &s_ccur[c], lane);
    else if (cnt <= 512) select_staged<8>(src, cnt, need, c, fl, top, dst, &s_ccur[c], lane);
    else select_staged_loop(src, cnt, need, c, fl, top, dst, &s_ccur[c], lane);
  }
}

// P5 for the staged clusters of at most kP5Thread keys, one thread per staged key (keys tagged
// with their cluster, staged_key): a key's rank is the number of larger keys of its cluster
// (the keys are distinct), counted over LDS reads that the lanes of a wave mostly share; the
// `need` best (rank < need) join the cluster's chosen words.  Balanced over the block however
// the keys fall into clusters.
constexpr int kP5Thread = 128;
__device__ __forceinline__ void select_small_staged(int tid, int gused, const int* s_bcnt,
                                                    const int* s_t, const int* s_above,
                                                    const unsigned long long* s_g,
                                                    const int* s_goff, uint32_t* s_cst,
                                                    const int* s_tpre, int* s_ccur) {
  for (int j = tid; j < gused; j += kThreads) {
    const unsigned long long x = s_g[j];
    const int c = 255 - (int)(((uint32_t)x) >> 24);
    const int cnt = s_bcnt[c];
    if (cnt > kP5Thread) continue;
    const unsigned long long* src = s_g + s_goff[c];
    int rank = 0, m = 0;
    for (; m + 4 <= cnt; m += 4) {
      const unsigned long long y0 = src[m], y1 = src[m + 1], y2 = src[m + 2], y3 = src[m + 3];
      rank += (y0 > x) + (y1 > x) + (y2 > x) + (y3 > x);
    }
    for (; m < cnt; ++m) rank += src[m] > x ? 1 : 0;
    if (rank < s_t[c] - s_above[c])
      s_cst[s_tpre[c] + atomicAdd(&s_ccur[c], 1)] = ((uint32_t)c << 24) | key_pos(x);
  }
}

// P6 and the write: each chosen word's rank inside its cluster (by position) places it in an
// LDS copy of the exp_idx row (-1 where a segment is short), which is then written out once.
// Starts and ends with a barrier; s_out may alias the staged keys (dead by then).
__device__ __forceinline__ void rank_and_write(int E, int tid, const int* s_base, const int* s_t,
                                               const int* s_tpre, uint32_t* s_cst, int* s_out,
                                               int32_t* erow) {
  oa::lds_barrier();
  for (int sl = tid; sl < E; sl += kThreads) s_out[sl] = -1;
  oa::lds_barrier();
  const int total = s_tpre[kMaxC];   // == sum_c t_c; every cluster's segment is full
  // rank by counting costs each word its cluster's t reads (broadcast within a wave: words of
  // one cluster read the same entries); only a cluster of more than kRankTMax words sorts
  if (s_tpre[kMaxC + 1] <= kRankTMax) {
    for (int j = tid; j < total; j += kThreads) {
      const uint32_t w = s_cst[j];
      const int c = (int)(w >> 24);
      const int b = s_tpre[c], t = s_t[c];
      int rank = 0, k = b;
      for (; k + 8 <= b + t; k += 8) {
        uint32_t y[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) y[u] = s_cst[k + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) rank += y[u] < w ? 1 : 0;
      }
      for (; k < b + t; ++k) rank += s_cst[k] < w ? 1 : 0;
      s_out[s_base[c] + rank] = (int)(w & 0xffffffu);
    }
  } else {
    int P = 1;
    while (P < total) P <<= 1;
    for (int i = total + tid; i < P; i += kThreads) s_cst[i] = 0xffffffffu;
    oa::lds_barrier();
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < P; i += kThreads) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const uint32_t x = s_cst[i], y = s_cst[ixj];
            const bool up = (i & k) == 0;
            if ((x > y) == up) { s_cst[i] = y; s_cst[ixj] = x; }
          }
        }
        oa::lds_barrier();
      }
    }
    for (int j = tid; j < total; j += kThreads) {
      const uint32_t w = s_cst[j];
      const int c = (int)(w >> 24);
      s_out[s_base[c] + (j - s_tpre[c])] = (int)(w & 0xffffffu);
    }
  }
  oa::lds_barrier();
  for (int sl = tid; sl < E; sl += kThreads) erow[sl] = s_out[sl];
}

template <int PPT, int LB>
__device__ __forceinline__ void topq_row_body(const TopqArgs& a, int row, unsigned long long* dyn) {
  __shared__ int s_w[kMaxC];              // min(q_c, E - base_c), clamped at 0
  __shared__ int s_base[kMaxC + 1];       // first exp_idx slot of each cluster
  __shared__ int s_t[kMaxC];              // members chosen
  __shared__ int s_above[kMaxC];          // members with a prefix above the boundary prefix
  __shared__ int s_bcnt[kMaxC];           // members in the boundary prefix bin
  __shared__ unsigned s_klo[kMaxC];       // boundary bin [klo, khi] of score keys of each cluster
  __shared__ unsigned s_khi[kMaxC];
  __shared__ unsigned s_pref[kMaxC];      // refinement: boundary-bin prefix of a split cluster, or ~0
  __shared__ unsigned s_lo[kMaxC];        // members whose key is > s_lo[c] are gathered
  __shared__ int s_mode[kMaxC];
  __shared__ int s_goff[kMaxC], s_gcur[kMaxC];   // staged keys: segment start, fill count
  __shared__ int s_ccur[kMaxC];           // chosen words written per cluster
  __shared__ int s_tpre[kMaxC + 2];       // chosen-word segment start per cluster; total, max
  __shared__ int s_fbl[kMaxC];
  __shared__ int s_gused, s_nfb, s_nsplit, s_hits1, s_ucnt, s_fbcnt[3];
  constexpr int NB = 1 << LB;
  constexpr int HS = NB + 16;             // histogram row: a pad word after every NB/16 bins
  constexpr int sb = LB - 4;              // bin b sits at word b + (b >> sb) of its row
  constexpr int bpt = NB >> 4;            // bins per scanning thread
  uint32_t* s_uw = reinterpret_cast<uint32_t*>(dyn);                         // ucap + 64
  uint32_t* s_uk = s_uw + a.ucap + 64;                                        // ucap + 64
  int* s_hist = reinterpret_cast<int*>(dyn + a.ucap + 64);                    // hwords
  unsigned long long* s_g = reinterpret_cast<unsigned long long*>(s_hist);    // after T2
  int* s_out = s_hist;                                                        // after P5
  uint32_t* s_cst = reinterpret_cast<uint32_t*>(s_hist + a.hwords);           // cpow

  // an opaque copy of the thread index: in topq_marked_kernel's row loop, nothing derived from it
  // is hoisted out of the loop to stay live across the body (that spills at the register cap)
  int tid_v = (int)threadIdx.x;
  asm volatile("" : "+v"(tid_v));
  const int tid = tid_v;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int C = a.C, E = a.E;
  constexpr int sh1 = 32 - LB;
  constexpr int sh1p = sh1 + sb;          // shift giving a level-1 bin's pad-word count
  const int trash = C * HS + lane;        // per-lane histogram slot for non-members
  const int n = *a.n_dev;
  const float* srow = a.S + (long)row * a.s_stride;
  const uint8_t* arow = a.asg8 + (long)row * a.a_stride;
  int32_t* erow = a.exp_idx + (long)row * E;

  // register i of a thread holds position sg*SEG + (i/4)*4096 + 4*tid + i%4: each group of four
  // consecutive positions arrives as one float4 of scores and one u32 of cluster ids
  constexpr int SEG = kThreads * PPT;
  constexpr int NG = PPT / 4;
  constexpr int CH = 12;         // positions whose per-cluster lookups are issued together
  static_assert(PPT % 4 == 0, "PPT must be a multiple of 4");
  const int nseg = n > 0 ? (n + SEG - 1) / SEG : 0;
  uint32_t kk[PPT];              // score key of a qualifying member, else 0
  uint32_t cp[NG];               // cluster ids, 4 per register
  auto pos_of = [&](int sg, int i) -> int { return sg * SEG + (i >> 2) * 4096 + 4 * tid + (i & 3); };

  // stream segment sg of the row into registers (clamped loads: all of them in flight); rows
  // are read up to the multiple of 4 that follows n - 1.  issue() only starts the loads, keys()
  // turns the arrived scores into keys (0 for a position that does not qualify)
  auto issue = [&](int sg) {
    const int last4 = (n - 1) & ~3;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int p = min(sg * SEG + g * 4096 + 4 * tid, last4);
      const float4 v = *reinterpret_cast<const float4*>(srow + p);
      cp[g] = *reinterpret_cast<const uint32_t*>(arow + p);
      kk[4 * g] = __float_as_uint(v.x);
      kk[4 * g + 1] = __float_as_uint(v.y);
      kk[4 * g + 2] = __float_as_uint(v.z);
      kk[4 * g + 3] = __float_as_uint(v.w);
    }
  };
  auto keys = [&](int sg) {
    const int lim = n - sg * SEG - 4 * tid;   // register i is in the row iff (i/4)*4096 + i%4 < lim
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const uint32_t key = oa::float_key(__uint_as_float(kk[i]));
      const bool q = (i >> 2) * 4096 + (i & 3) < lim && key > kNegInfKey;
      kk[i] = q ? key : 0u;
    }
  };
  auto load = [&](int sg) {
    issue(sg);
    keys(sg);
  };
  auto cid = [&](int i) -> int { return (int)((cp[i >> 2] >> (8 * (i & 3))) & 0xffu); };

  // append the members flagged in hb (bit i = register i) to the gathered list: an exclusive
  // scan of the per-thread counts inside the wave, one LDS atomic per wave for its base.  Every
  // register is written: a member to the next list slot, anything else to the lane's trash slot
  // (the histograms bound the list size, so the slots never run past ucap)
  auto gather = [&](int sg, unsigned long long hb) {
    const int cnt = __popcll(hb);
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    const int tot = __shfl(incl, 63, 64);
    int wbase = 0;
    if (lane == 0 && tot > 0) wbase = atomicAdd(&s_ucnt, tot);
    wbase = __shfl(wbase, 0, 64);
    const int tr = a.ucap + lane;
    int d = wbase + incl - cnt - tr;           // next list slot, relative to the trash slot
    const int pbase = sg * SEG + 4 * tid;
    const uint32_t hlo = (uint32_t)hb, hhi = (uint32_t)(hb >> 32);
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      // 0 or -1: bit i of hb, sign-extended
      const int m = __builtin_amdgcn_sbfe((int)(i < 32 ? hlo : hhi), i & 31, 1);
      const int dst = tr + (d & m);
      s_uw[dst] = ((uint32_t)cid(i) << 24) | (uint32_t)(pbase + (i >> 2) * 4096 + (i & 3));
      s_uk[dst] = kk[i];
      d -= m;
    }
  };

  auto clear_hist = [&]() {
    for (int i = tid; i < (C * HS) / 4; i += kThreads) reinterpret_cast<int4*>(s_hist)[i] = make_int4(0, 0, 0, 0);
  };

  // the first segment's loads are in flight while P0 runs (its barriers order LDS only)
  if (nseg > 0) issue(0);

  // ---- P0: quota prefix, per-cluster state, histogram clear
  if (wave == 0) quota_prefix(a.quota + (long)row * C, C, E, lane, s_base, s_w);
  for (int c = tid; c < kMaxC; c += kThreads) {
    s_t[c] = 0; s_above[c] = 0; s_bcnt[c] = 0; s_klo[c] = 0u; s_khi[c] = 0u; s_pref[c] = ~0u;
    s_lo[c] = kNoGather;
    s_mode[c] = kModeNone; s_goff[c] = 0; s_gcur[c] = 0; s_ccur[c] = 0;
  }
  for (int i = tid; i < (C * HS) / 4; i += kThreads) reinterpret_cast<int4*>(s_hist)[i] = make_int4(0, 0, 0, 0);
  if (tid == 0) {
    s_gused = 0; s_nfb = 0; s_nsplit = 0; s_hits1 = 0; s_ucnt = 0;
    s_fbcnt[0] = 0; s_fbcnt[1] = 0; s_fbcnt[2] = 0;
  }
  oa::lds_barrier();

  // ---- L1: histogram of the top LB key bits per cluster
  for (int sg = 0; sg < nseg; ++sg) {
    if (sg > 0) issue(sg);
    keys(sg);
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const uint32_t k = kk[i];
      int slot = (int)__umul24(cid(i), HS) + (int)(k >> sh1) + (int)(k >> sh1p);
      asm volatile("" : "+v"(slot));   // computed in every lane: a select, not a branch
      atomicAdd(&s_hist[k ? slot : trash], 1);
    }
  }
  oa::lds_barrier();

  // ---- T1: level-1 bin of the t-th best member, 16 threads per cluster
  for (int cb = 0; cb < C; cb += kThreads / 16) {
    const int c = cb + (tid >> 4);
    const int j = tid & 15;
    const int w = c < C ? s_w[c] : 0;
    RowScan<bpt> r;
    scan_row(s_hist + min(c, C - 1) * HS, j, r);
    const int m = __shfl(r.sfx, 0, 16);
    if (c < C && w > 0) {
      const int t = min(w, m);
      if (t > 0 && t == m) {     // every member is chosen
        if (j == 0) {
          s_t[c] = t; s_mode[c] = kModeAll; s_klo[c] = 0u; s_khi[c] = ~0u;
          s_lo[c] = kNegInfKey;              // gathering bound - 1: every member
          atomicAdd(&s_hits1, t);
        }
      } else if (t > 0 && r.sfx >= t && r.sfx - r.ls < t) {
        int b, acc, cnt;
        find_bin(r, t, b, acc, cnt);
        const unsigned b1 = (unsigned)(j * bpt + b);
        s_t[c] = t;
        s_above[c] = acc;
        s_bcnt[c] = cnt;
        s_klo[c] = b1 << sh1;
        s_khi[c] = (b1 << sh1) | ((1u << sh1) - 1u);
        s_lo[c] = max(b1 << sh1, kNegInfKey + 1u) - 1u;   // gathering bound - 1 (members only)
        if (t - acc == cnt) {    // the whole level-1 bin completes t: no split
          s_mode[c] = kModeAll;
        } else {
          s_mode[c] = kModeSplit;
          atomicAdd(&s_nsplit, 1);
        }
        atomicAdd(&s_hits1, acc + cnt);
      }
    }
  }
  oa::lds_barrier();
  const bool fits = s_hits1 <= a.ucap;   // block-uniform: the level-1 set fits in the list
  int ucnt = 0;

  // One more histogram level for every split cluster: the next LB key bits of its boundary
  // bin's members (from the gathered list, or from the registers when the list does not hold
  // the level-1 set), then the bin of the t-th member.  A cluster whose new boundary bin fits
  // in the staging space is staged, one at full key depth that does not is resolved
  // block-wide in P5, the others stay split for the next level.
  int depth = 1;
  auto refine = [&](bool from_list) {
    ++depth;
    const int shp = max(32 - LB * (depth - 1), 0);   // the split bins' prefix shift (> 0)
    const int shd = max(32 - LB * depth, 0);         // this level's bin shift
    for (int c = tid; c < kMaxC; c += kThreads)
      s_pref[c] = c < C && s_mode[c] == kModeSplit ? s_klo[c] >> shp : ~0u;
    clear_hist();
    oa::lds_barrier();
    // every thread has read s_nsplit for its loop test before the barrier above; the count is
    // rebuilt in the scan below, after the next barrier
    if (tid == 0) s_nsplit = 0;
    if (from_list) {
      for (int j0 = 0; j0 < ucnt; j0 += kThreads * kUPT) {
        int cc[kUPT];
        uint32_t k[kUPT];
#pragma unroll
        for (int u = 0; u < kUPT; ++u) {
          const int j = min(j0 + u * kThreads + tid, ucnt - 1);
          cc[u] = (int)(s_uw[j] >> 24);
          k[u] = s_uk[j];
        }
#pragma unroll
        for (int u = 0; u < kUPT; ++u) {
          const bool in = j0 + u * kThreads + tid < ucnt && (k[u] >> shp) == s_pref[cc[u]];
          const uint32_t bn = (k[u] >> shd) & (NB - 1);
          atomicAdd(&s_hist[in ? cc[u] * HS + (int)bn + (int)(bn >> sb) : trash], 1);
        }
      }
    } else {
      for (int sg = 0; sg < nseg; ++sg) {
        if (nseg > 1) load(sg);
#pragma unroll
        for (int i0 = 0; i0 < PPT; i0 += CH) {
          unsigned pv[CH];
#pragma unroll
          for (int j = 0; j < CH; ++j)
            if (i0 + j < PPT) pv[j] = s_pref[cid(i0 + j)];
#pragma unroll
          for (int j = 0; j < CH; ++j) {
            if (i0 + j < PPT) {
              const int i = i0 + j;
              const uint32_t k = kk[i];
              const bool in = k && (k >> shp) == pv[j];
              const uint32_t bn = (k >> shd) & (NB - 1);
              int slot = (int)__umul24(cid(i), HS) + (int)bn + (int)(bn >> sb);
              asm volatile("" : "+v"(slot));
              atomicAdd(&s_hist[in ? slot : trash], 1);
            }
          }
        }
      }
    }
    oa::lds_barrier();
    for (int cb = 0; cb < C; cb += kThreads / 16) {
      const int c = cb + (tid >> 4);
      const int j = tid & 15;
      if (c >= C || s_pref[c] == ~0u) continue;     // uniform over the cluster's 16 threads
      RowScan<bpt> r;
      scan_row(s_hist + c * HS, j, r);
      const int t2 = s_t[c] - s_above[c];           // rank of the t-th member inside the bin
      if (r.sfx >= t2 && r.sfx - r.ls < t2) {
        int b, acc, cnt;
        find_bin(r, t2, b, acc, cnt);
        // at the last level the bin index may repeat bits of the prefix: OR leaves them as is
        const unsigned klo = s_klo[c] | ((unsigned)(j * bpt + b) << shd);
        const int need = t2 - acc;
        s_klo[c] = klo;
        s_khi[c] = klo | ((1u << shd) - 1u);
        s_above[c] = s_above[c] + acc;
        s_bcnt[c] = cnt;
        int mode = kModeAll;
        if (need < cnt) {
          // reserve [off, off + cnt) of the staging space only if it fits (compare-and-swap:
          // a reservation taken back after the fact could overlap one made meanwhile)
          int off = s_gused;
          bool got = false;
          while (off + cnt <= a.gcap) {
            const int prev = atomicCAS(&s_gused, off, off + cnt);
            if (prev == off) { got = true; break; }
            off = prev;
          }
          if (got) {
            mode = kModeStaged;
            s_goff[c] = off;
          } else {
            if (shd == 0) {      // equal keys beyond the staging space: block-wide search in P5
              mode = kModeBlock;
              s_fbl[atomicAdd(&s_nfb, 1)] = c;
            } else {
              mode = kModeSplit;
              atomicAdd(&s_nsplit, 1);
            }
          }
        }
        s_mode[c] = mode;
      }
    }
    oa::lds_barrier();
  };

  if (!fits) {
    while (s_nsplit > 0) refine(false);       // block-uniform loop: s_nsplit read after a barrier
    // final gathering bounds, stored as bound - 1 for a strict test (no key exceeds ~0, so a
    // cluster without quota gathers nothing): the boundary bin and above (members only: keys
    // > kNegInfKey), only the members above the bin for a block-wide cluster
    for (int c = tid; c < kMaxC; c += kThreads) {
      const int mode = c < C ? s_mode[c] : kModeNone;
      s_lo[c] = mode == kModeNone ? kNoGather
                : (mode == kModeBlock ? s_khi[c] : max(s_klo[c], kNegInfKey + 1u) - 1u);
    }
    oa::lds_barrier();
  }

  if (wave == 0) chosen_prefix(s_t, s_tpre, lane);   // chosen-word segment of each cluster

  // ---- G: gather every member whose key reaches its cluster's bound
  for (int sg = 0; sg < nseg; ++sg) {
    if (nseg > 1) load(sg);
    unsigned long long hb = 0ull;
#pragma unroll
    for (int i0 = 0; i0 < PPT; i0 += CH) {
      unsigned lov[CH];
#pragma unroll
      for (int j = 0; j < CH; ++j)
        if (i0 + j < PPT) lov[j] = s_lo[cid(i0 + j)];
#pragma unroll
      for (int j = 0; j < CH; ++j)
        if (i0 + j < PPT && kk[i0 + j] > lov[j]) hb |= 1ull << (i0 + j);
    }
    gather(sg, hb);
  }
  oa::lds_barrier();
  ucnt = min(s_ucnt, a.ucap);

  if (fits)
    while (s_nsplit > 0) refine(true);

  // ---- F: gathered members above the boundary bin are chosen (all of a whole-bin cluster's
  // from klo up), members inside a staged cluster's bin are staged
  for (int j0 = 0; j0 < ucnt; j0 += kThreads * kUPT) {
    uint32_t e[kUPT], key[kUPT], lo[kUPT], hi[kUPT];
    int mode[kUPT];
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int j = min(j0 + u * kThreads + tid, ucnt - 1);
      e[u] = s_uw[j];
      key[u] = s_uk[j];
    }
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int c = (int)(e[u] >> 24);
      lo[u] = s_klo[c];
      hi[u] = s_khi[c];
      mode[u] = j0 + u * kThreads + tid < ucnt ? s_mode[c] : kModeNone;
    }
#pragma unroll
    for (int u = 0; u < kUPT; ++u) {
      const int c = (int)(e[u] >> 24);
      if (mode[u] != kModeNone && (key[u] > hi[u] || (mode[u] == kModeAll && key[u] >= lo[u])))
        s_cst[s_tpre[c] + atomicAdd(&s_ccur[c], 1)] = e[u];
      else if (mode[u] == kModeStaged && key[u] >= lo[u] && key[u] <= hi[u])
        s_g[s_goff[c] + atomicAdd(&s_gcur[c], 1)] = key64(key[u], (int)(e[u] & 0xffffffu));
    }
  }
  oa::lds_barrier();

  // ---- P5: the `need` best of each staged cluster's boundary bin, one wave per cluster
  select_all_staged(C, wave, lane, s_mode, s_bcnt, s_t, s_above, s_g, s_goff, s_cst, s_tpre, s_klo,
                    s_khi, s_ccur);
  // clusters whose boundary bin holds more equal keys than the staging space: block-wide
  // bitwise search over the positions, re-streaming the row (rare)
  const int nfb = s_nfb;         // final since the last refinement barrier
  for (int f = 0; f < nfb; ++f) {
    const int c = s_fbl[f];
    const uint32_t K0 = s_klo[c];   // the boundary key (khi == klo at full depth)
    const int need = s_t[c] - s_above[c];
    unsigned long long T = bin_floor(K0);
    for (int bit = 23, it = 0; bit >= 0; --bit, ++it) {
      const unsigned long long cnd = T | (1ull << bit);
      int k = 0;
      for (int sg = 0; sg < nseg; ++sg) {
        load(sg);
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
          const int p = pos_of(sg, i);
          const bool in = kk[i] == K0 && cid(i) == c && key64(kk[i], p) >= cnd;
          k += __popcll(__ballot(in));
        }
      }
      // three counters in rotation: the one cleared here is next added to two barriers later
      if (lane == 0 && k) atomicAdd(&s_fbcnt[it % 3], k);
      oa::lds_barrier();
      if (s_fbcnt[it % 3] >= need) T = cnd;
      if (tid == 0) s_fbcnt[(it + 2) % 3] = 0;
    }
    for (int sg = 0; sg < nseg; ++sg) {
      load(sg);
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int p = pos_of(sg, i);
        const bool take = kk[i] == K0 && cid(i) == c && key64(kk[i], p) >= T;
        append_chosen(take, ((uint32_t)c << 24) | (uint32_t)p, s_cst + s_tpre[c], &s_ccur[c], lane);
      }
    }
    oa::lds_barrier();
    if (tid == 0) { s_fbcnt[0] = 0; s_fbcnt[1] = 0; s_fbcnt[2] = 0; }
    oa::lds_barrier();
  }
  // ---- P6: each chosen word's rank inside its cluster (by position), then the row write
  rank_and_write(E, tid, s_base, s_t, s_tpre, s_cst, s_out, erow);
}

template <int PPT, int LB>
__global__ void __launch_bounds__(kThreads) topq_row_kernel(TopqArgs a) {
  extern __shared__ unsigned long long dyn[];
  topq_row_body<PPT, LB>(a, blockIdx.x, dyn);
}

// After the linear-bin kernel: a grid of at most kRowGrid workgroups runs the rows it marked
// (usually none), so an empty pass dispatches 64 workgroups, not one per row.  Wave 0
// reads the marks of 64 of the workgroup's rows (blockIdx.x + j * gridDim.x) at once; their
// ballot reaches every wave through LDS.
template <int PPT, int LB>
__global__ void __launch_bounds__(kThreads) topq_marked_kernel(TopqArgs a) {
  extern __shared__ unsigned long long dyn[];
  __shared__ unsigned long long s_marks;
  bool ran = false;
  for (int base = 0; base < a.rows; base += 64 * gridDim.x) {
    if (threadIdx.x < 64) {
      const int row = base + blockIdx.x + (int)threadIdx.x * gridDim.x;
      const unsigned long long m = __ballot(row < a.rows && a.exp_idx[(long)row * a.E] == kRowMarked);
      if (threadIdx.x == 0) s_marks = m;
    }
    __syncthreads();
    // uniform (read at full exec): the rows and their pointers stay in scalar registers
    const unsigned long long m = s_marks;
    unsigned long long mk = ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(m >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)m);
    __syncthreads();                     // every wave holds the mask before the next batch's
    while (mk) {
      const int j = __ffsll((long long)mk) - 1;
      mk &= mk - 1;
      if (ran) __syncthreads();          // the previous row's LDS is dead before P0 reuses it
      topq_row_body<PPT, LB>(a, base + blockIdx.x + j * gridDim.x, dyn);
      ran = true;
    }
  }
}

// The linear-bin kernel: the common path.  Scores are binned linearly over the row's range of
// qualifying (head-truncated) scores, [smin, smax]: bin(s) = 1 + (int)((s - smin) * (HS - 2) /
// (smax - smin)), bin 0 for a position that is no member; any binning non-decreasing in s keeps
// the selection exact, since a member in a higher bin beats every member in a lower one, and
// the boundary bin of a cluster (the bin of its t-th best member) holds a handful of members
// where the key-prefix bins hold hundreds.  One pass builds the per-cluster histograms (R, L1),
// 16 threads per cluster find the boundary bins (T1), and one more pass over the registers (G)
// sends members above the boundary straight to their cluster's chosen words and boundary-bin
// members to the staged keys; P5 and P6 are shared with the key-prefix kernel.  A row whose
// staged members do not fit the staging space is marked (exp_idx[row][0] = kRowMarked) and left
// to the key-prefix kernel, launched next over the marked rows only.
//
// HEADS: the score rows hold 16-bit key heads (oa_qgs_scan_heads), which are all the kernel
// keeps of a score anyway; exact scores come from the codes (oa::qgs_score).
// Returns true for a row it leaves to the key-prefix algorithm (marked kRowMarked).
template <int PPT, int LB, bool HEADS, bool TILE>
__device__ __forceinline__ bool topq_linear_body(const TopqArgs& a, int row, unsigned long long* dyn) {
  static_assert(HEADS || !TILE, "the tile range comes with the head rows");
  __shared__ int s_w[kMaxC];
  __shared__ int s_base[kMaxC + 1];
  __shared__ int s_t[kMaxC];
  __shared__ int s_above[kMaxC];
  __shared__ int s_bcnt[kMaxC];
  __shared__ unsigned s_klo[kMaxC], s_khi[kMaxC];   // 0, ~0: P5 searches all 32 key bits
  __shared__ unsigned s_sel[kMaxC];       // lowest gathered bin (low half), first chosen bin (high half)
  __shared__ int s_mode[kMaxC];
  __shared__ int s_goff[kMaxC], s_gcur[kMaxC];
  __shared__ int s_ccur[kMaxC];
  __shared__ int s_tpre[kMaxC + 2];
  __shared__ int s_gused, s_fail;
  __shared__ uint32_t s_rlo[kWaves], s_rhi[kWaves];
  __shared__ int s_lw[HEADS ? 32 : 1];    // the row's limb words (exact scores)
  // a cluster's histogram row holds HS = 2^LB + 16 bins: bin 0 counts the positions that are no
  // member (ignored), a member's bin is 1 .. HS - 1; 16 threads scan a row, HS / 16 bins each
  // (HS / 16 is odd, so the 16 threads' first bins lie in 16 different banks)
  constexpr int NB = 1 << LB;
  constexpr int HS = NB + 16;
  constexpr int bpt = HS / 16;
  int* s_hist = reinterpret_cast<int*>(dyn);                                  // hwords
  unsigned long long* s_g = reinterpret_cast<unsigned long long*>(s_hist);    // after T1
  int* s_out = s_hist;                                                        // after P5
  uint32_t* s_cst = reinterpret_cast<uint32_t*>(s_hist + a.hwords);           // cpow

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int C = a.C, E = a.E;
  const int n = *a.n_dev;
  const float* srow = a.S + (long)row * a.s_stride;
  const uint16_t* hrow = a.H + (long)row * a.h_stride;
  const uint8_t* arow = a.asg8 + (long)row * a.a_stride;
  int32_t* erow = a.exp_idx + (long)row * E;
  const int kvr = row / 4;

  constexpr int SEG = kThreads * PPT;
  constexpr int NG = PPT / 4;
  constexpr int CH = 18;          // cluster lookups in flight per G batch (36 spills)
  // the single-segment instantiations (PPT <= 36) are launched only for Lmax <= SEG
  constexpr bool kMulti = PPT > 36;
  const int nseg = n > 0 ? (kMulti ? (n + SEG - 1) / SEG : 1) : 0;
  // Only the top 16 bits of each key stay in registers (two per register), as t = h - 0x7f for a
  // member (h = key >> 16 >= 0x80 for every finite score) and 0 for anything else, with t capped
  // at kTopT (the head of the largest finite floats: +inf and NaN share their bin, so every
  // member's t stands for a finite float): t is non-decreasing in the score, so bins of t order
  // members as their scores do, and the few members of a staged bin get their exact keys from S
  // again
  uint32_t kk[PPT];             // the loaded scores, until keys() packs them
  uint32_t kh[PPT / 2];         // 16-bit key heads of positions 2j (low half) and 2j + 1
  uint32_t cp[NG];
  auto pos_of = [&](int sg, int i) -> int { return sg * SEG + (i >> 2) * 4096 + 4 * tid + (i & 3); };
  auto issue = [&](int sg) {
    const int last4 = (n - 1) & ~3;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int p = min(sg * SEG + g * 4096 + 4 * tid, last4);
      cp[g] = *reinterpret_cast<const uint32_t*>(arow + p);
      if (HEADS) {
        const uint2 v = *reinterpret_cast<const uint2*>(hrow + p);
        kh[2 * g] = v.x;
        kh[2 * g + 1] = v.y;
      } else {
        const float4 v = *reinterpret_cast<const float4*>(srow + p);
        kk[4 * g] = __float_as_uint(v.x);
        kk[4 * g + 1] = __float_as_uint(v.y);
        kk[4 * g + 2] = __float_as_uint(v.z);
        kk[4 * g + 3] = __float_as_uint(v.w);
      }
    }
  };
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  // t of the four positions of group g of segment sg (two registers), in place
  auto key_group = [&](int sg, int g) {
    const int lim = n - sg * SEG - 4 * tid;
    {
      if (HEADS && g * 4096 + 3 < lim) {
        // the group lies inside the row: a saturating subtract of 0x7f maps the heads of -inf
        // (0x7f) to 0 and a member's head h to h - 0x7f, two positions per instruction
#pragma unroll
        for (int w = 0; w < 2; ++w)
          kh[2 * g + w] = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(
                              __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, kh[2 * g + w]),
                                                            (u16x2){0x7f, 0x7f}),
                              (u16x2){kTopT, kTopT}));
        return;
      }
#pragma unroll
      for (int j = 2 * g; j < 2 * g + 2; ++j) {
        uint32_t h2 = 0u;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i = 2 * j + u;
          if (HEADS) {
            const uint32_t h = (kh[j] >> (16 * u)) & 0xffffu;
            const bool q = (i >> 2) * 4096 + (i & 3) < lim && h > oa::kNegInfHead;
            h2 |= (q ? min(h - (uint32_t)oa::kNegInfHead, (uint32_t)kTopT) : 0u) << (16 * u);
          } else {
            const uint32_t key = oa::float_key(__uint_as_float(kk[i]));
            const bool q = (i >> 2) * 4096 + (i & 3) < lim && key > kNegInfKey;
            h2 |= (q ? min((key >> 16) - (uint32_t)oa::kNegInfHead, (uint32_t)kTopT) : 0u) << (16 * u);
          }
        }
        kh[j] = h2;
      }
    }
  };
  auto keys = [&](int sg) {
#pragma unroll
    for (int g = 0; g < NG; ++g) key_group(sg, g);
  };
  auto load = [&](int sg) { issue(sg); keys(sg); };
  auto hd = [&](int i) -> uint32_t { return (kh[i >> 1] >> (16 * (i & 1))) & 0xffffu; };
  auto cid = [&](int i) -> int { return (int)((cp[i >> 2] >> (8 * (i & 3))) & 0xffu); };

  // the quotas and the limb words are requested ahead of the row (loads return in order, so
  // the prefix would otherwise wait for the whole row); so are (TILE) the row's tile extremes --
  // the tiles holding a position below n; a single-segment row has at most 16 PPT <= kThreads of
  // them, one per thread.  With them no pass over the row precedes the binning (a row of several
  // segments is then read twice, not three times)
  float qv[4];
  if (wave == 0) quota_load(a.quota + (long)row * C, C, lane, qv);
  int lwv = 0;
  if (HEADS && tid < 32) lwv = oa::limb_words(a.limbs, kvr, row % 4)[tid];
  const int ntu = (n + 63) / 64;
  constexpr int TL = kMulti ? kTileLd : 1;
  float tx[TL], tn[TL];
  if (TILE) {
    const float* tm_row = a.TM + (long)row * a.tm_stride;
    const float* tmn_row = a.TMn + (long)row * a.tm_stride;
#pragma unroll
    for (int u = 0; u < TL; ++u) {
      const int j = max(min(tid + u * kThreads, ntu - 1), 0);
      tx[u] = tm_row[j];
      tn[u] = tmn_row[j];
    }
  }
  if (nseg > 0) issue(0);       // in flight while P0 runs

  // ---- P0: quota prefix, per-cluster state, histogram clear
  if (wave == 0) quota_scan(qv, C, E, lane, s_base, s_w);
  for (int c = tid; c < kMaxC; c += kThreads) {
    s_t[c] = 0; s_above[c] = 0; s_bcnt[c] = 0; s_klo[c] = 0u; s_khi[c] = ~0u;
    s_sel[c] = 0xffffffffu; s_mode[c] = kModeNone; s_goff[c] = 0; s_gcur[c] = 0; s_ccur[c] = 0;
  }
  for (int i = tid; i < (C * HS) / 4; i += kThreads) reinterpret_cast<int4*>(s_hist)[i] = make_int4(0, 0, 0, 0);
  if (tid == 0) { s_gused = 0; s_fail = a.force_mark; }
  if (HEADS && tid < 32) s_lw[tid] = lwv;

  // ---- R: the range of the qualifying members' score keys
  // two heads per register on the packed 16-bit ALU: a non-member (head 0) becomes 0xffff after
  // the wrapping - 1, so it never wins the minimum of the members' heads - 1
  // (with the tile extremes: the t of the least and greatest finite score below n, a range that
  // holds every member's t -- the selected positions' scores only widen it)
  uint32_t khi = 0u, klo = 0xffffffffu;
  if (TILE) {
    float tmx = -INFINITY, tmn = INFINITY;
#pragma unroll
    for (int u = 0; u < TL; ++u) {
      if (tid + u * kThreads < ntu) {
        tmx = fmaxf(tmx, tx[u]);
        tmn = fminf(tmn, tn[u]);
      }
    }
    if (tmx > -INFINITY) {
      khi = min((oa::float_key(tmx) >> 16) - (uint32_t)oa::kNegInfHead, (uint32_t)kTopT);
      klo = min((oa::float_key(tmn) >> 16) - (uint32_t)oa::kNegInfHead, (uint32_t)kTopT);
    }
  } else {
    u16x2 vlo = {0xffff, 0xffff}, vhi = {0, 0};
    for (int sg = 0; sg < nseg; ++sg) {
      if (sg == 0) keys(0); else load(sg);
#pragma unroll
      for (int j = 0; j < PPT / 2; ++j) {
        const u16x2 h = __builtin_bit_cast(u16x2, kh[j]);
        vhi = __builtin_elementwise_max(vhi, h);
        vlo = __builtin_elementwise_min(vlo, (u16x2)(h - (u16x2){1, 1}));
      }
    }
    khi = max((uint32_t)vhi.x, (uint32_t)vhi.y);
    klo = min((uint32_t)vlo.x, (uint32_t)vlo.y) + 1u;   // with no member khi is 0
  }
  klo = ~oa::wave_max_u32(~klo);
  khi = oa::wave_max_u32(khi);
  if (lane == 0) { s_rlo[wave] = klo; s_rhi[wave] = khi; }
  oa::lds_barrier();
  klo = 0xffffffffu;
  khi = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) { klo = min(klo, s_rlo[w]); khi = max(khi, s_rhi[w]); }
  // bin of a member's t: 1 + (x - smin) * (HS - 2) / (smax - smin), truncated, with x the float
  // of the head (t + 0x7f) << 16 -- in one fma, rounded once, so non-decreasing in t and inside
  // [1, HS - 1] (the heads carry 8 significant bits, so |smin| * scale stays below 2^15 and
  // the fma's error far below 1/2).  A non-member's t = 0 gives a NaN float (below -inf's key):
  // the fma keeps it NaN and fmaxf(NaN, 0) = 0, bin 0.  With one distinct member head (or a span
  // that overflows) scale is 0 and every member lands in bin 1
  float scale = 0.f, off = 1.5f;
  if (khi != 0u) {
    const float smin = head_float(klo);
    const float span = head_float(khi) - smin;
    if (span > 0.f && span < INFINITY) {
      scale = (float)(HS - 2) / span;
      off = 1.5f - smin * scale;
    }
  }
  // (clamped into the row as well: a member outside the range -- only if the caller's tile
  // extremes do not hold its score -- stays inside the cluster's histogram row)
  auto fbin = [&](uint32_t t) -> int {
    return (int)fminf(fmaxf(fmaf(head_float(t), scale, off), 0.f), (float)(HS - 1));
  };

  // ---- L1: per-cluster histogram of the linear bins.  A single-segment row keeps each
  // position's bin in place of its t for G (0 still marks a non-member).  Groups of four
  // positions wholly past n are skipped (uniform); in the group holding n the positions past it
  // (clamped loads: copies of one cluster id) count in per-lane trash words, not all in one bin 0
  const int trash = C * HS + lane;
  for (int sg = 0; sg < nseg; ++sg) {
    // with the tile range the row's t are formed here, group by group as the loads arrive
    if (TILE ? sg > 0 : nseg > 1) issue(sg);
    if (!TILE && nseg > 1) keys(sg);
    const int lim0 = n - sg * SEG;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g * 4096 >= lim0) continue;
      if (TILE) key_group(sg, g);
      const bool full = (g + 1) * 4096 <= lim0;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const int j = 2 * g + w;
        const int b0 = fbin(kh[j] & 0xffffu);
        const int b1 = fbin(kh[j] >> 16);
        int a0 = (int)__umul24(cid(2 * j), HS) + b0;
        int a1 = (int)__umul24(cid(2 * j + 1), HS) + b1;
        if (!full) {
          a0 = b0 ? a0 : trash;
          a1 = b1 ? a1 : trash;
        }
        atomicAdd(&s_hist[a0], 1);
        atomicAdd(&s_hist[a1], 1);
        if (!kMulti) kh[j] = (uint32_t)b0 | ((uint32_t)b1 << 16);
      }
    }
  }
  oa::lds_barrier();

  // ---- T1: boundary bin b1 of every cluster with quota; bins above it are chosen, b1 itself
  // is chosen whole when it completes t, else its members are staged
  for (int cb = 0; cb < C; cb += kThreads / 16) {
    const int c = cb + (tid >> 4);
    const int j = tid & 15;
    const int w = c < C ? s_w[c] : 0;
    RowScan<bpt> r;
    scan_row_dense(s_hist + min(c, C - 1) * HS, j, r);
    const int m = __shfl(r.sfx, 0, 16);
    if (c < C && w > 0) {
      const int t = min(w, m);
      if (t > 0 && t == m) {     // every member is chosen (bins 1 and up: no non-member)
        if (j == 0) { s_t[c] = t; s_mode[c] = kModeAll; s_sel[c] = 0x00010001u; }
      } else if (t > 0 && r.sfx >= t && r.sfx - r.ls < t) {
        int b, acc, cnt;
        find_bin(r, t, b, acc, cnt);
        const unsigned b1 = (unsigned)(j * bpt + b);
        s_t[c] = t;
        s_above[c] = acc;
        s_bcnt[c] = cnt;
        if (t - acc == cnt) {
          s_mode[c] = kModeAll;
          s_sel[c] = (b1 << 16) | b1;
        } else {
          const int off = atomicAdd(&s_gused, cnt);
          if (off + cnt <= a.gcap) {
            s_mode[c] = kModeStaged;
            s_goff[c] = off;
            s_sel[c] = ((b1 + 1u) << 16) | b1;
          } else {
            s_fail = 1;
          }
        }
      }
    }
  }
  oa::lds_barrier();
  if (s_fail) {                  // uniform: the key-prefix kernel takes the row
    if (HEADS) {                 // ... from exact fp32 scores: the row is recomputed into S32
      const double inv = ldexp(1.0, -a.fexp[row]);
      float* orow = a.S32 + (long)row * a.s32_stride;
      for (int p = tid; p < n; p += kThreads)
        orow[p] = hrow[p] > oa::kNegInfHead ? oa::qgs_score_lds(a.codes, a.lmax_codes, kvr, p, s_lw, inv)
                                            : -INFINITY;
    }
    if (tid == 0) erow[0] = kRowMarked;
    return true;
  }
  if (wave == 0) chosen_prefix(s_t, s_tpre, lane);
  oa::lds_barrier();

  // ---- G: members in the chosen bins to their cluster's chosen words, members in a staged
  // bin to its staged keys (the histogram is dead: the staged keys reuse it)
  for (int sg = 0; sg < nseg; ++sg) {
    if (nseg > 1) load(sg);
    const int lim0 = n - sg * SEG;       // groups of four positions wholly past n are skipped
#pragma unroll
    for (int i0 = 0; i0 < PPT; i0 += CH) {
      unsigned sv[CH];
#pragma unroll
      for (int j = 0; j < CH; ++j)
        if (i0 + j < PPT && ((i0 + j) >> 2) * 4096 < lim0) sv[j] = s_sel[cid(i0 + j)];
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        if (i0 + j < PPT && ((i0 + j) >> 2) * 4096 < lim0) {
          const int i = i0 + j;
          // the bin (single segment) or t; a non-member's bin 0 is below every chosen or staged
          // bin (those are 1 or more)
          // bin (one compare, rarely true); a gathered member at or above the first chosen bin is
          // chosen, one below it sits in the staged bin
          const int bn = kMulti ? fbin(hd(i)) : (int)hd(i);
          if (bn >= (int)(sv[j] & 0xffffu)) {
            const int c = cid(i);
            if (bn >= (int)(sv[j] >> 16))
              s_cst[s_tpre[c] + atomicAdd(&s_ccur[c], 1)] = ((uint32_t)c << 24) | (uint32_t)pos_of(sg, i);
            else
              s_g[s_goff[c] + atomicAdd(&s_gcur[c], 1)] = staged_key(0u, c, pos_of(sg, i));
          }
        }
      }
    }
  }
  oa::lds_barrier();
  // the staged members' exact keys, from S or recomputed from the codes (they fill [0, s_gused)
  // of the staged keys)
  {
    const double inv = HEADS ? ldexp(1.0, -a.fexp[row]) : 0.0;
    for (int j = tid; j < s_gused; j += kThreads) {
      const unsigned long long e = s_g[j];
      const int p = (int)key_pos(e);
      const float sc = HEADS ? oa::qgs_score_lds(a.codes, a.lmax_codes, kvr, p, s_lw, inv) : srow[p];
      s_g[j] = ((unsigned long long)oa::float_key(sc) << 32) | (e & 0xffffffffull);
    }
  }
  oa::lds_barrier();

  // ---- P5 (small staged clusters one thread per key, the others one wave each), P6
  select_small_staged(tid, s_gused, s_bcnt, s_t, s_above, s_g, s_goff, s_cst, s_tpre, s_ccur);
  select_all_staged(C, wave, lane, s_mode, s_bcnt, s_t, s_above, s_g, s_goff, s_cst, s_tpre, s_klo,
                    s_khi, s_ccur, true, kP5Thread);
  rank_and_write(E, tid, s_base, s_t, s_tpre, s_cst, s_out, erow);
  return false;
}

template <int PPT, int LB, bool HEADS, bool TILE>
// up to 64 VGPRs for the single-segment instantiations: two workgroups (rows) per unit
__global__ void __launch_bounds__(kThreads, PPT <= 36 ? 8 : 4) topq_linear_kernel(TopqArgs a) {
  extern __shared__ unsigned long long dyn[];
  topq_linear_body<PPT, LB, HEADS, TILE>(a, blockIdx.x, dyn);
}

// Fewer rows than compute units (one workgroup per unit, so its LDS and registers are free):
// the linear-bin algorithm and, on a row it cannot finish, the key-prefix algorithm in the same
// workgroup, instead of a second launch over every row.  lin and pre are the two algorithms'
// arguments (LDS layouts); the dynamic LDS holds either's.
template <int PPT, int LB, int PLB, bool TILE>
__global__ void __launch_bounds__(kThreads) topq_small_kernel(TopqArgs lin, TopqArgs pre) {
  extern __shared__ unsigned long long dyn[];
  if (topq_linear_body<PPT, LB, true, TILE>(lin, blockIdx.x, dyn)) {   // uniform
    // the row's exact scores (S32) written above are read back by every wave
    __threadfence();
    __syncthreads();
    topq_row_body<PPT, PLB>(pre, blockIdx.x, dyn);
  }
}

template <int PPT, int LB>
int launch_row(const TopqArgs& a, int rows, size_t lds, hipStream_t s) {
  const void* fn = a.marked_only ? (const void*)topq_marked_kernel<PPT, LB> : (const void*)topq_row_kernel<PPT, LB>;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return (int)e;
  if (a.marked_only)
    hipLaunchKernelGGL((topq_marked_kernel<PPT, LB>), dim3(std::min(rows, kRowGrid)), dim3(kThreads), lds, s, a);
  else
    hipLaunchKernelGGL((topq_row_kernel<PPT, LB>), dim3(rows), dim3(kThreads), lds, s, a);
  return OA_LAUNCH_STATUS();
}

template <int LB>
int launch_lb(const TopqArgs& a, int rows, int Lmax, size_t lds, hipStream_t s) {
  if (Lmax <= kThreads * 8) return launch_row<8, LB>(a, rows, lds, s);
  if (Lmax <= kThreads * 16) return launch_row<16, LB>(a, rows, lds, s);
  if (Lmax <= kThreads * 36) return launch_row<36, LB>(a, rows, lds, s);
  return launch_row<44, LB>(a, rows, lds, s);
}

template <int PPT, int LB, bool HEADS, bool TILE>
int launch_linear(const TopqArgs& a, int rows, size_t lds, hipStream_t s) {
  const hipError_t e = hipFuncSetAttribute((const void*)topq_linear_kernel<PPT, LB, HEADS, TILE>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((topq_linear_kernel<PPT, LB, HEADS, TILE>), dim3(rows), dim3(kThreads), lds, s, a);
  return OA_LAUNCH_STATUS();
}

template <int LB, bool HEADS, bool TILE>
int launch_linear_lb(const TopqArgs& a, int rows, int Lmax, size_t lds, hipStream_t s) {
  if (Lmax <= kThreads * 8) return launch_linear<8, LB, HEADS, TILE>(a, rows, lds, s);
  if (Lmax <= kThreads * 16) return launch_linear<16, LB, HEADS, TILE>(a, rows, lds, s);
  if (Lmax <= kThreads * 36) return launch_linear<36, LB, HEADS, TILE>(a, rows, lds, s);
  return launch_linear<44, LB, HEADS, TILE>(a, rows, lds, s);
}

// The one-launch kernel holds both algorithms' static LDS; the key-prefix algorithm's gathered
// list takes what the unit's LDS leaves beside it, sized from the compiled kernel's own static
// LDS (hipFuncGetAttributes).  Returns kNotLaunched when the list would be too short to run the
// key-prefix algorithm in the same workgroup: the caller then takes two launches.
constexpr int kNotLaunched = -1001;
template <int PPT, int LB, int PLB, bool TILE>
int launch_small(const TopqArgs& lin, TopqArgs pre, int rows, size_t lds_lin, hipStream_t s) {
  const void* fn = (const void*)topq_small_kernel<PPT, LB, PLB, TILE>;
  hipFuncAttributes fa;
  const hipError_t ea = hipFuncGetAttributes(&fa, fn);
  if (ea != hipSuccess) return (int)ea;
  const long room = (long)kLdsLimit - (long)fa.sharedSizeBytes - 4L * pre.hwords - 4L * pre.cpow - 8L * 64;
  pre.ucap = (int)std::min<long>(kUCapMax, std::max<long>(room, 0) / 8) & ~3;
  pre.gcap = std::min(pre.hwords / 2, pre.ucap - pre.E);
  if (pre.gcap < 64) return kNotLaunched;
  const size_t lds_pre = 8 * (size_t)(pre.ucap + 64) + 4 * (size_t)pre.hwords + 4 * (size_t)pre.cpow;
  const size_t lds = std::max(lds_lin, lds_pre);
  if ((long)lds + (long)fa.sharedSizeBytes > kLdsLimit) return kNotLaunched;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((topq_small_kernel<PPT, LB, PLB, TILE>), dim3(rows), dim3(kThreads), lds, s, lin, pre);
  return OA_LAUNCH_STATUS();
}
template <int LB, int PLB, bool TILE>
int launch_small_ppt(const TopqArgs& lin, const TopqArgs& pre, int rows, int Lmax, size_t lds_lin,
                     hipStream_t s) {
  if (Lmax <= kThreads * 8) return launch_small<8, LB, PLB, TILE>(lin, pre, rows, lds_lin, s);
  if (Lmax <= kThreads * 16) return launch_small<16, LB, PLB, TILE>(lin, pre, rows, lds_lin, s);
  return launch_small<36, LB, PLB, TILE>(lin, pre, rows, lds_lin, s);
}

}  // namespace

namespace {

// the launch sequence shared by oa_topq_path and oa_topq_heads: `a` carries the pointers; the
// sizes are set here.  lin: run the linear-bin kernel (heads: its 16-bit variant); pre: run
// the key-prefix kernel (after lin: on the rows lin marked only)
int topq_launch(TopqArgs a, int rows, int C, int Lmax, int E, bool lin, bool heads, bool pre,
                hipStream_t s) {
  // bits per histogram level: 8, 7 or 6, so that C * (2^lb + 16) ints stay near 64 KiB
  a.lb = C <= 64 ? 8 : (C <= 128 ? 7 : 6);
  a.cpow = 4;                   // >= 4: the LDS rows are cleared and scanned 4 words at a time
  while (a.cpow < E) a.cpow <<= 1;
  // key-prefix kernel, dynamic LDS: gathered list (ucap + 64 trash entries: a word array and a
  // key array) | histogram -> staged keys -> output row (hwords ints) | chosen words (cpow u32)
  const long hist = (long)C * ((1 << a.lb) + 16) + 64;
  a.hwords = (int)((std::max<long>(hist, a.cpow) + 3) & ~3L);
  const long static_lds = (long)sizeof(int) * (16 * kMaxC + 8);
  const long room = (long)kLdsLimit - static_lds - 4L * a.hwords - 4L * a.cpow - 8L * 64;
  a.ucap = (int)std::min<long>(kUCapMax, room / 8) & ~3;   // keeps the histogram 16-byte aligned
  a.gcap = std::min(a.hwords / 2, a.ucap - E);             // the final gathering fits in ucap
  if (a.gcap < 64) return OA_EINVAL;
  const size_t lds = 8 * (size_t)(a.ucap + 64) + 4 * (size_t)a.hwords + 4 * (size_t)a.cpow;
  a.marked_only = 0;
  a.rows = rows;
  // the tile range: head rows with the scan's tile extremes, at most kTileLd tiles per thread
  const bool tile = heads && a.TM != nullptr && (Lmax + 63) / 64 <= kTileLd * kThreads;
  if (lin) {
    // linear-bin kernel, dynamic LDS: histogram -> staged keys -> output row | chosen words.
    // 7 bits for C <= 64, 6 for C <= 128, else 5: two workgroups' LDS fits one unit.  Rows
    // longer than one register segment run one workgroup per unit anyway (their VGPRs), and
    // keep 6 bits (smaller boundary bins: fewer rows overflow the staging space)
    TopqArgs al = a;
    al.lb = C <= 64 ? 7 : (C <= 128 || Lmax > kThreads * 36 ? 6 : 5);
    al.hwords = (int)((std::max<long>((long)C * ((1 << al.lb) + 16) + 64, a.cpow) + 3) & ~3L);
    al.gcap = al.hwords / 2;
    const size_t lds_lin = 4 * (size_t)al.hwords + 4 * (size_t)a.cpow;
    if (heads && pre && rows < kSmallRows && Lmax <= kThreads * 36) {
      // one launch: the key-prefix algorithm's gathered list shrinks by the linear-bin
      // algorithm's static LDS, which the same workgroup holds (path 3, every row marked, then
      // runs every row through the key-prefix algorithm in this kernel)
      int st1 = kNotLaunched;
      if (tile) {
        if (al.lb == 7 && a.lb == 8) st1 = launch_small_ppt<7, 8, true>(al, a, rows, Lmax, lds_lin, s);
        else if (al.lb == 6 && a.lb == 7) st1 = launch_small_ppt<6, 7, true>(al, a, rows, Lmax, lds_lin, s);
        else if (al.lb == 5 && a.lb == 6) st1 = launch_small_ppt<5, 6, true>(al, a, rows, Lmax, lds_lin, s);
      } else {
        if (al.lb == 7 && a.lb == 8) st1 = launch_small_ppt<7, 8, false>(al, a, rows, Lmax, lds_lin, s);
        else if (al.lb == 6 && a.lb == 7) st1 = launch_small_ppt<6, 7, false>(al, a, rows, Lmax, lds_lin, s);
        else if (al.lb == 5 && a.lb == 6) st1 = launch_small_ppt<5, 6, false>(al, a, rows, Lmax, lds_lin, s);
      }
      if (st1 != kNotLaunched) return st1;
    }
    int st;
    if (tile) st = al.lb == 7 ? launch_linear_lb<7, true, true>(al, rows, Lmax, lds_lin, s)
                   : al.lb == 6 ? launch_linear_lb<6, true, true>(al, rows, Lmax, lds_lin, s)
                                : launch_linear_lb<5, true, true>(al, rows, Lmax, lds_lin, s);
    else if (heads) st = al.lb == 7 ? launch_linear_lb<7, true, false>(al, rows, Lmax, lds_lin, s)
                    : al.lb == 6 ? launch_linear_lb<6, true, false>(al, rows, Lmax, lds_lin, s)
                                 : launch_linear_lb<5, true, false>(al, rows, Lmax, lds_lin, s);
    else st = al.lb == 7 ? launch_linear_lb<7, false, false>(al, rows, Lmax, lds_lin, s)
              : al.lb == 6 ? launch_linear_lb<6, false, false>(al, rows, Lmax, lds_lin, s)
                           : launch_linear_lb<5, false, false>(al, rows, Lmax, lds_lin, s);
    if (st || !pre) return st;
    a.marked_only = 1;
  }
  if (a.lb == 8) return launch_lb<8>(a, rows, Lmax, lds, s);
  if (a.lb == 7) return launch_lb<7>(a, rows, Lmax, lds, s);
  return launch_lb<6>(a, rows, Lmax, lds, s);
}

bool topq_sizes_ok(int rows, int C, int E, int Lmax) {
  return rows > 0 && C > 0 && C <= kMaxC && E >= 0 && E <= kMaxE && Lmax > 0 && Lmax < kMaxPos;
}

}  // namespace

// path 0: the linear-bin kernel on every row, then the key-prefix kernel on the rows it
// marked; path 1: the key-prefix kernel on every row; path 2: the linear-bin kernel alone (a
// row it leaves to the key-prefix kernel keeps the mark kRowMarked in exp_idx[row][0])
extern "C" int oa_topq_path(const float* S, long s_stride, const uint8_t* asg8, long asg8_stride,
                            const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
                            const int* n_dev, int path, void* stream) {
  const long lmax4 = ((long)Lmax + 3) & ~3L;
  if (!topq_sizes_ok(rows, C, E, Lmax) || !S || !asg8 || !quota || !n_dev ||
      (E > 0 && !exp_idx) || s_stride % 4 || asg8_stride % 4 || s_stride < lmax4 ||
      asg8_stride < lmax4 || (reinterpret_cast<uintptr_t>(S) & 15) ||
      (reinterpret_cast<uintptr_t>(asg8) & 3) || path < 0 || path > 2)
    return OA_EINVAL;
  if (E == 0) return 0;
  TopqArgs a = {};
  a.S = S; a.s_stride = s_stride; a.asg8 = asg8; a.a_stride = asg8_stride; a.quota = quota;
  a.C = C; a.E = E; a.n_dev = n_dev; a.exp_idx = exp_idx;
  return topq_launch(a, rows, C, Lmax, E, path != 1, false, path != 2, (hipStream_t)stream);
}

extern "C" int oa_topq(const float* S, long s_stride, const uint8_t* asg8, long asg8_stride,
                       const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
                       const int* n_dev, void* stream) {
  return oa_topq_path(S, s_stride, asg8, asg8_stride, quota, rows, C, Lmax, exp_idx, E, n_dev, 0,
                      stream);
}

// over 16-bit key heads (oa_qgs_scan_heads + oa_topk_select_heads).  path 0: as oa_topq (rows
// the linear-bin kernel leaves are recomputed into S32 and selected by the key-prefix kernel);
// path 2: the linear-bin kernel alone; path 3: every row is left to the key-prefix kernel
extern "C" int oa_topq_heads(const uint16_t* H, long h_stride, const uint8_t* asg8,
                             long asg8_stride, const float* quota, int rows, int C, int Lmax,
                             int32_t* exp_idx, int E, const int* n_dev, const int8_t* codes,
                             int kv_rows, const int8_t* limbs, const int* fexp, float* S32,
                             long s32_stride, const float* TM, const float* TMn, long tm_stride,
                             int path, void* stream) {
  const long lmax4 = ((long)Lmax + 3) & ~3L;
  if (!topq_sizes_ok(rows, C, E, Lmax) || !H || !asg8 || !quota || !n_dev || !codes || !limbs ||
      !fexp || !S32 || (E > 0 && !exp_idx) || kv_rows <= 0 || rows != kv_rows * 4 ||
      (!TM != !TMn) || (TM && tm_stride < ((long)Lmax + 63) / 64) ||
      h_stride % 4 || asg8_stride % 4 || s32_stride % 4 || h_stride < lmax4 ||
      asg8_stride < lmax4 || s32_stride < lmax4 || (reinterpret_cast<uintptr_t>(H) & 7) ||
      (reinterpret_cast<uintptr_t>(S32) & 15) || (reinterpret_cast<uintptr_t>(asg8) & 3) ||
      (reinterpret_cast<uintptr_t>(codes) & 15) || (reinterpret_cast<uintptr_t>(limbs) & 3) ||
      !(path == 0 || path == 2 || path == 3))
    return OA_EINVAL;
  if (E == 0) return 0;
  TopqArgs a = {};
  a.S = S32; a.s_stride = s32_stride; a.asg8 = asg8; a.a_stride = asg8_stride; a.quota = quota;
  a.C = C; a.E = E; a.n_dev = n_dev; a.exp_idx = exp_idx;
  a.H = H; a.h_stride = h_stride; a.codes = codes; a.lmax_codes = Lmax; a.limbs = limbs;
  a.fexp = fexp; a.S32 = S32; a.s32_stride = s32_stride; a.force_mark = path == 3;
  a.TM = TM; a.TMn = TMn; a.tm_stride = tm_stride;
  return topq_launch(a, rows, C, Lmax, E, true, true, path != 2, (hipStream_t)stream);
}
