// Exact top-k of one query-head row by one wave, register variant (rows of at most 64 * TPL
// score tiles, k <= KR), shared by the top-k launch and the small-batch top-k + gate + fill launch.
//
// Reference semantics: StaticTopKMasker.add_mask (static_top_k.py:221-262: top-k over positions
// not already taken by the sink/local maskers), deployed select kernel graph_runner.py:100-159;
// ties break to the lower position (graph_runner.py:127-151).
#pragma once
#include "oa_common.h"
#include "oa_score.h"

namespace oa_sel {

constexpr int GQ = 4;    // query heads per KV head (limb rows = GQ * 4 = 16)
constexpr int kMaxTop = 64;

__device__ __forceinline__ unsigned long long tile_key(float v, int t) {
  return ((unsigned long long)oa::float_key(v) << 32) | (0xffffffffu - (unsigned)t);
}

// With HEADS the score rows hold 16-bit key heads: the candidate tiles' exact scores are
// recomputed from the codes (oa::qgs_score, the scan's arithmetic), and the selected tokens'
// heads are set to that of -inf.
struct Rescore {
  const int8_t* codes; long lmax;   // (BH, Lmax, 32)
  const int8_t* limbs;              // (BH, 16, 32)
  const int* fexp;                  // (R,)
};

// candidate score of position pos of a query-head row (sink, local and unwritten: -inf)
template <bool HEADS>
__device__ __forceinline__ float cand_score(const void* Sv, long s_stride, int row, int pos, int ns,
                                            int dead_hi, const Rescore& rs, const int* lw,
                                            double inv) {
  if (!HEADS) return static_cast<const float*>(Sv)[(long)row * s_stride + pos];
  if (pos < ns || pos >= dead_hi) return -INFINITY;
  return oa::qgs_score(rs.codes, rs.lmax, row / GQ, pos, lw, inv);
}
template <bool HEADS>
__device__ __forceinline__ void mark_selected(void* Sv, long s_stride, int row, int pos) {
  if (HEADS) static_cast<uint16_t*>(Sv)[(long)row * s_stride + pos] = oa::kNegInfHead;
  else static_cast<float*>(Sv)[(long)row * s_stride + pos] = -INFINITY;
}
// the row's limb words (HEADS only) and 2^-F
template <bool HEADS>
__device__ __forceinline__ double load_limbs(const Rescore& rs, int row, int* lw) {
  if (!HEADS) return 0.0;
  const int* p = oa::limb_words(rs.limbs, row / GQ, row % GQ);
#pragma unroll
  for (int w = 0; w < 32; ++w) lw[w] = p[w];
  return ldexp(1.0, -rs.fexp[row]);
}

// Lane l keeps the keys of tiles l, l+64, ... and later of column l of the k chosen tiles in
// registers; every extraction step is one wave maximum (DPP) and an in-register update by the
// owning lane.  Writes sel = [0..ns) ++ [n-nl..n) ++ top and marks the selected scores.
// lds_sel, when not null, receives the same sel row (for the rest of the workgroup).
template <int TPL, int KR, bool HEADS>
__device__ __forceinline__ void topk_reg_row(void* __restrict__ Sv, long s_stride,
                                             const float* __restrict__ TM, long tm_stride,
                                             int ntiles, int32_t* __restrict__ sel, long sel_stride,
                                             int n, int ns, int nl, int k_top, const Rescore& rs,
                                             int row, int lane, int32_t* lds_sel = nullptr) {
  int lw[HEADS ? 32 : 1];
  const double inv = load_limbs<HEADS>(rs, row, lw);
  unsigned long long tk[TPL];
  float tv[TPL];
#pragma unroll
  for (int j = 0; j < TPL; ++j) tv[j] = TM[(long)row * tm_stride + min(j * 64 + lane, ntiles - 1)];
  unsigned long long mine = 0ull;
#pragma unroll
  for (int j = 0; j < TPL; ++j) {
    const int t = j * 64 + lane;
    tk[j] = t < ntiles ? tile_key(tv[j], t) : 0ull;
    mine = tk[j] > mine ? tk[j] : mine;
  }
  int my_tile = 0;               // lane i < k_top: the i-th chosen tile
  unsigned long long kth = 0ull; // the key of the k-th chosen tile's maximum
  for (int i = 0; i < k_top; ++i) {
    const unsigned long long best = oa::wave_max_u64(mine);
    const int t = (int)(0xffffffffu - (unsigned)(best & 0xffffffffull));
    if (lane == i) my_tile = t;
    kth = best;
    if (best == mine) {          // the owner lane drops the tile and refreshes its maximum
      mine = 0ull;
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        tk[j] = tk[j] == best ? 0ull : tk[j];
        mine = tk[j] > mine ? tk[j] : mine;
      }
    }
  }
  // candidates: lane l holds column l of the k chosen tiles
  unsigned long long ck[KR];
  float cv[KR];
  if (HEADS) {
    // only candidates whose key head reaches that of the k-th chosen tile maximum can be in the
    // top k (heads are non-decreasing in the score): their exact scores are recomputed, the
    // others count as -inf
    // (the heads and every candidate's code are loaded in one round)
    const uint16_t* Hrow = static_cast<const uint16_t*>(Sv) + (long)row * s_stride;
    const int kvr = row / GQ;
    const int dead_hi = n - nl;
    uint32_t hv[KR];
    uint4 cw[KR][2];
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int tj = __builtin_amdgcn_readlane(my_tile, min(j, max(k_top - 1, 0)));   // uniform lane
      const int pos = tj * 64 + lane;
      hv[j] = j < k_top ? Hrow[pos] : 0u;
      const uint4* cp = reinterpret_cast<const uint4*>(rs.codes + ((long)kvr * rs.lmax +
                                                                   max(min(pos, dead_hi - 1), 0)) * 32);
      cw[j][0] = cp[0];
      cw[j][1] = cp[1];
    }
    // each chosen tile holds a token scoring at least the k-th chosen tile maximum, so the k-th
    // best score reaches it, and so does every top-k token's head
    const uint32_t T = (uint32_t)(kth >> 48);
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int tj = __builtin_amdgcn_readlane(my_tile, min(j, max(k_top - 1, 0)));   // uniform lane
      const int pos = tj * 64 + lane;
      cv[j] = -INFINITY;
      if (j < k_top && hv[j] >= T && pos >= ns && pos < dead_hi)
        cv[j] = oa::qgs_score_words(cw[j][0], cw[j][1], lw, inv);
    }
  } else {
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int tj = __builtin_amdgcn_readlane(my_tile, min(j, max(k_top - 1, 0)));   // uniform lane
      cv[j] = cand_score<HEADS>(Sv, s_stride, row, tj * 64 + lane, ns, n - nl, rs, lw, inv);
    }
  }
  mine = 0ull;
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const int tj = __builtin_amdgcn_readlane(my_tile, min(j, max(k_top - 1, 0)));   // uniform lane
    ck[j] = j < k_top ? tile_key(cv[j], tj * 64 + lane) : 0ull;
    mine = ck[j] > mine ? ck[j] : mine;
  }
  int my_pos = 0;                // lane i < k_top: the i-th selected position
  for (int i = 0; i < k_top; ++i) {
    const unsigned long long best = oa::wave_max_u64(mine);
    const int pos = (int)(0xffffffffu - (unsigned)(best & 0xffffffffull));
    if (lane == i) my_pos = pos;
    if (best == mine) {
      mine = 0ull;
#pragma unroll
      for (int j = 0; j < KR; ++j) {
        ck[j] = ck[j] == best ? 0ull : ck[j];
        mine = ck[j] > mine ? ck[j] : mine;
      }
    }
  }
  int32_t* sr = sel + (long)row * sel_stride;
  if (lane < ns) sr[lane] = lane;
  if (lane < nl) sr[ns + lane] = n - nl + lane;
  if (lane < k_top) {
    sr[ns + nl + lane] = my_pos;
    mark_selected<HEADS>(Sv, s_stride, row, my_pos);
  }
  if (lds_sel) {
    if (lane < ns) lds_sel[lane] = lane;
    if (lane < nl) lds_sel[ns + lane] = n - nl + lane;
    if (lane < k_top) lds_sel[ns + nl + lane] = my_pos;
  }
}

}  // namespace oa_sel
