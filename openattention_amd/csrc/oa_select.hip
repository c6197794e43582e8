// QGS selection on gfx950: query projection, int8 code scan, exact top-k.
//
// Reference semantics: StaticTopKMasker._scores (static_top_k.py:197-218: zq = (q U) * scale,
// score_i = zq . code_i), add_mask (static_top_k.py:221-262: top-k over positions not already
// taken by the sink/local maskers), deployed scan/select kernels graph_runner.py:100-159.
//
// Exactness.  The reference's fp32 matmul has no defined summation order, so this library
// fixes one that any implementation can reproduce bit for bit:
//   F_row   = 30 - e, where max_r |zq_r| = m * 2^e with m in [0.5, 1)
//   Z_r     = rint(zq_r * 2^F_row)              (|Z_r| < 2^30, an int32)
//   S_i     = sum_r Z_r * code_{i,r}            (exact integer, |S_i| < 2^43)
//   score_i = fp32(S_i * 2^-F_row)              (one rounding)
// The integer sum is order independent, so it is evaluated on the int8 matrix cores:
// Z_r is split into four signed 8-bit limbs and one v_mfma_i32_16x16x32_i8 multiplies the
// 16 limb rows (4 query heads x 4 limbs) of a KV head with the 32-byte codes of 16 tokens.
// Each output lane then holds the four limb partials of one (token, head) and recombines
// them exactly in fp64 (all values are integers below 2^53).
// Top-k ties break to the lower position (graph_runner.py:127-151 rule).
#include "oa_common.h"
#include "oa_score.h"
#include "oa_prep.h"
#include "oa_topk_row.h"
#include "oa_gate_row.h"

typedef int oa_v4i __attribute__((ext_vector_type(4)));

namespace {

using namespace oa_sel;

constexpr int RQ = 32;   // QGS rank (bytes of code per token)

// ------------------------------------------------------------------------------------------
// prep: one wave per query-head row (body in oa_prep.h, shared with the fused index+prep kernel)
__global__ void __launch_bounds__(64) qgs_prep_kernel(const uint16_t* __restrict__ q, long q_stride,
                                                      const float* __restrict__ U,
                                                      const float* __restrict__ scale, int G,
                                                      int8_t* __restrict__ limbs,
                                                      int* __restrict__ fexp,
                                                      float* __restrict__ zq_out) {
  oa::qgs_prep_row(q, q_stride, U, scale, G, limbs, fexp, zq_out, blockIdx.x, threadIdx.x);
}

// ------------------------------------------------------------------------------------------
// scan: grid (token chunks of kTokWG, BH).  4 waves; each wave owns kTilesPerWave 64-token
// tiles, four MFMA blocks of 16 tokens per tile, and requests all of their codes before the
// first MFMA.  Writes the score of every position (sink/local and positions >= n as -inf) and
// the maximum of every 64-token tile per query-head row.  The codes are read once per step, so
// they are loaded non-temporally (and so are the head rows stored).
constexpr int kScanThreads = 256;
constexpr int kTilesPerWave = 2;
constexpr int kTokWG = kScanThreads / 64 * kTilesPerWave * 64;

struct ScanArgs {
  const int8_t* codes; int Lmax; const int8_t* limbs; const int* fexp;
  void* Sv; long s_stride; float* TM; long tm_stride;
  const int* n_dev; int ns; int nl;
  float* TMn;      // optional: each tile's least finite score (+inf for a tile without one)
};

// HEADS: the score rows hold 16-bit key heads (oa::score_head) instead of fp32 scores.
// One block: token chunk `chunk` (kTokWG tokens) of KV row kvr.
// MIN: the tile minima of the finite scores too (sa.TMn)
template <bool HEADS, bool MIN = false>
__device__ __forceinline__ void scan_block(const ScanArgs& sa, int chunk, int kvr) {
  const int8_t* __restrict__ codes = sa.codes;
  const int Lmax = sa.Lmax;
  const int8_t* __restrict__ limbs = sa.limbs;
  const int* __restrict__ fexp = sa.fexp;
  void* __restrict__ Sv = sa.Sv;
  const long s_stride = sa.s_stride;
  float* __restrict__ TM = sa.TM;
  float* __restrict__ TMn = sa.TMn;
  const long tm_stride = sa.tm_stride;
  const int ns = sa.ns, nl = sa.nl;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4;        // k-group for the operands; head g for the output
  const int nn = lane & 15;        // token inside a 16-token block; limb row for A
  const int tile_begin = chunk * (kTokWG / 64) + wave * kTilesPerWave;
  const int ntile_total = (Lmax + 63) / 64;
  const int8_t* cb = codes + (long)kvr * Lmax * RQ;
  // every code of the wave's tiles in flight at once (addresses clamped to the last token;
  // tokens past Lmax are zeroed below)
  long b_op[kTilesPerWave][4];
#pragma unroll
  for (int t = 0; t < kTilesPerWave; ++t)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int tok = (tile_begin + t) * 64 + b * 16 + nn;
      b_op[t][b] = __builtin_nontemporal_load(
          reinterpret_cast<const long*>(cb + (long)min(tok, Lmax - 1) * RQ + kg * 8));
    }
  const int n = *sa.n_dev;
  const int dead_hi = n - nl;      // positions >= dead_hi are local or not yet written
  const long a_op = *reinterpret_cast<const long*>(limbs + (long)kvr * 16 * RQ + nn * RQ + kg * 8);
  const int row = kvr * GQ + kg;
  const double inv = ldexp(1.0, -fexp[row]);
  float* Srow = static_cast<float*>(Sv) + (long)row * s_stride;
  uint16_t* Hrow = static_cast<uint16_t*>(Sv) + (long)row * s_stride;

  // heads: each wave stages its tile's 4 x 64 heads in LDS and writes them back as 8-byte words
  // (four consecutive positions per lane: whole 128-byte lines per store)
  __shared__ uint16_t s_h[HEADS ? kScanThreads / 64 : 1][GQ][64];
  // the block's tile maxima, written out together at the end (consecutive lanes, consecutive
  // tiles of a row: one store instead of four-lane scattered ones per tile)
  constexpr int kTB = kTokWG / 64;
  __shared__ float s_tm[GQ][kTB];
  __shared__ float s_tmn[GQ][kTB];
#pragma unroll
  for (int t = 0; t < kTilesPerWave; ++t) {
    const int tile = tile_begin + t;
    if (tile >= ntile_total) break;
    float tmax = -INFINITY, tmin = INFINITY;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int tok = tile * 64 + b * 16 + nn;
      oa_v4i zero = {0, 0, 0, 0};
      oa_v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_op, tok < Lmax ? b_op[t][b] : 0L,
                                                         zero, 0, 0, 0);
      // the exact integer sum: limb partials are below 2^19 in magnitude, so each pair joins
      // exactly in int32 (< 2^28) and the two pairs exactly in fp64 (< 2^44)
      const int xh = acc[3] * 256 + acc[2];
      const int xl = acc[1] * 256 + acc[0];
      const double s = fma((double)xh, 65536.0, (double)xl);
      float sc = (float)(s * inv);
      const bool dead = tok < ns || tok >= dead_hi;
      if (MIN) tmin = fminf(tmin, dead ? INFINITY : sc);
      if (dead) sc = -INFINITY;
      if (HEADS) s_h[wave][kg][b * 16 + nn] = oa::score_head(sc);
      else Srow[tok] = sc;
      tmax = fmaxf(tmax, sc);
    }
    if (HEADS) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      const uint2 hv = *reinterpret_cast<const uint2*>(&s_h[wave][kg][4 * nn]);
      uint32_t* hp = reinterpret_cast<uint32_t*>(Hrow + (long)tile * 64 + 4 * nn);
      __builtin_nontemporal_store(hv.x, hp);
      __builtin_nontemporal_store(hv.y, hp + 1);
      // the staged heads are read before the next tile overwrites them
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
    // one 16-lane DPP row per head: the tile maximum in every lane of the row
    tmax = oa::group16_max(tmax);
    if (nn == 0) s_tm[kg][wave * kTilesPerWave + t] = tmax;
    if (MIN) {
      tmin = oa::group16_min(tmin);
      if (nn == 0) s_tmn[kg][wave * kTilesPerWave + t] = tmin;
    }
  }
  oa::lds_barrier();
  if (threadIdx.x < GQ * kTB) {
    const int g = threadIdx.x / kTB;
    const int tile = chunk * kTB + threadIdx.x % kTB;
    if (tile < ntile_total) {
      TM[(long)(kvr * GQ + g) * tm_stride + tile] = s_tm[g][threadIdx.x % kTB];
      if (MIN) TMn[(long)(kvr * GQ + g) * tm_stride + tile] = s_tmn[g][threadIdx.x % kTB];
    }
  }
}

template <bool HEADS, bool MIN>
__global__ void __launch_bounds__(kScanThreads) qgs_scan_kernel(ScanArgs sa) {
  scan_block<HEADS, MIN>(sa, blockIdx.x, blockIdx.y);
}

// The scan over heads and the pooled part of the ErrorGate in one launch: n_scan blocks of
// scan_block<true> (chunk-fastest order, as qgs_scan_kernel's grid) and n_gate blocks of
// gate_pooled_unit (row r, clusters 16 u .. 16 u + 15), spread evenly through the block order
// so that the gate's short dependent chains run under the scan's code stream.  Both read state
// the index update left (codes, limbs; Sk, Sk2, n) and write disjoint outputs.
template <bool MIN>
__global__ void __launch_bounds__(kScanThreads) qgs_scan_gate_kernel(ScanArgs sa, oa_gate::GateArgs ga,
                                                                     int nchunks, int n_scan, int n_gate) {
  const long b = blockIdx.x;
  const long tot = (long)n_scan + n_gate;
  const long g0 = b * n_gate / tot;
  const long g1 = (b + 1) * n_gate / tot;
  if (g1 > g0) {                                    // uniform: gate unit g0
    __shared__ float s_zb[oa_gate::kPoolClusters], s_s2[oa_gate::kPoolClusters],
        s_nt[oa_gate::kPoolClusters];
    const int units = (ga.C + oa_gate::kPoolClusters - 1) / oa_gate::kPoolClusters;
    const int row = (int)(g0 / units);
    oa_gate::gate_pooled_unit(ga, row, (int)(g0 % units) * oa_gate::kPoolClusters, s_zb, s_s2, s_nt);
  } else {
    const long si = b - g0;                         // scan blocks before this one
    scan_block<true, MIN>(sa, (int)(si % nchunks), (int)(si / nchunks));
  }
}

// ------------------------------------------------------------------------------------------
// select: one wave per query-head row.  The k tiles with the largest maxima (ties to the
// lower tile) hold every top-k token, the lowest-position tied ones included; the row top-k
// is taken among their scores (ties to the lower position).  Then
// sel = [0..ns) ++ [n-nl..n) ++ top, and the selected tokens' scores are set to -inf so the
// within-cluster top-q ranks them last.
constexpr int kMaxTilesLds = 4096;   // Lmax <= 262144
__device__ __forceinline__ int lanes_below(unsigned long long m, int lane) {
  return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
}

// Radix-select variant for rows of at most 64*TPL tiles and k_top <= kMaxTop.  The k-th largest
// tile key T is found bit by bit from ballot counts over the tile keys held in registers (lane
// l: tiles l, l + 64, ...); the chosen tiles are those above T and the lowest-index ones equal
// to it.  Every top-k token scores at least T (k chosen tiles each hold a token that does), so
// only candidates whose key reaches T join the candidate list (with HEADS: whose head reaches
// T's head, exact scores then recomputed for the list alone).  The k-th largest candidate key
// (score key << 32 | ~position: distinct) is found the same way, and the k winners are written
// in descending key order, as repeated wave maxima would give them.
// Sink, local and unwritten positions are candidates scoring -inf (the register variant's and
// graph_runner.py:145-151's rule): a row with fewer than k_top live positions is filled with the
// lowest such positions, so the list always holds at least k_top candidates, each below
// ntiles * 64.
template <int TPL, bool HEADS>
__global__ void __launch_bounds__(64) topk_select_kernel(void* __restrict__ Sv, long s_stride,
                                                         const float* __restrict__ TM, long tm_stride,
                                                         int ntiles, int32_t* __restrict__ sel,
                                                         long sel_stride, const int* __restrict__ n_dev,
                                                         int ns, int nl, int k_top, Rescore rs) {
  __shared__ int s_tile[kMaxTop];
  __shared__ unsigned long long s_ck[kMaxTop * 64];   // candidate positions, then their keys
  __shared__ unsigned long long s_win[kMaxTop];
  const int row = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2
  const int lane = threadIdx.x;
  const int n = *n_dev;
  const int dead_hi = n - nl;
  if (k_top == 0) {                                     // uniform: sink and local only
    int32_t* sr = sel + (long)row * sel_stride;
    if (lane < ns) sr[lane] = lane;
    if (lane < nl) sr[ns + lane] = n - nl + lane;
    return;
  }
  int lw[HEADS ? 32 : 1];
  const double inv = load_limbs<HEADS>(rs, row, lw);
  uint32_t tk[TPL];
  float tv[TPL];
#pragma unroll
  for (int j = 0; j < TPL; ++j) tv[j] = TM[(long)row * tm_stride + min(j * 64 + lane, ntiles - 1)];
#pragma unroll
  for (int j = 0; j < TPL; ++j) tk[j] = j * 64 + lane < ntiles ? oa::float_key(tv[j]) : 0u;
  // ---- T: the largest key value reached by at least k tiles
  uint32_t T = 0u;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < TPL; ++j) cnt += __popcll(__ballot(tk[j] >= cand));
    if (cnt >= k_top) T = cand;
  }
  int need = k_top;
#pragma unroll
  for (int j = 0; j < TPL; ++j) need -= __popcll(__ballot(tk[j] > T));
  // ---- the chosen tiles, in tile order: above T, then equal to T while need lasts
  int nt = 0;
#pragma unroll
  for (int j = 0; j < TPL; ++j) {
    const unsigned long long meq = __ballot(tk[j] == T);
    const bool take = tk[j] > T || (tk[j] == T && lanes_below(meq, lane) < need);
    need -= min(need, __popcll(meq));
    const unsigned long long mt = __ballot(take);
    if (take) s_tile[nt + lanes_below(mt, lane)] = j * 64 + lane;
    nt += __popcll(mt);
  }
  __syncthreads();
  // ---- candidates: column lane of every chosen tile whose key (head) reaches T's (every
  // tile's value is requested before any is used: one round of loads)
  uint32_t cv[kMaxTop];
#pragma unroll
  for (int j = 0; j < kMaxTop; ++j) {
    const int pos = s_tile[min(j, k_top - 1)] * 64 + lane;     // past k_top: a repeat, unused
    cv[j] = HEADS ? (uint32_t)static_cast<const uint16_t*>(Sv)[(long)row * s_stride + pos]
                  : __float_as_uint(static_cast<const float*>(Sv)[(long)row * s_stride + pos]);
  }
  int nc = 0;
#pragma unroll
  for (int j = 0; j < kMaxTop; ++j) {
    if (j >= k_top) continue;                       // uniform
    const int pos = s_tile[j] * 64 + lane;
    const bool live = pos >= ns && pos < dead_hi;
    bool q;
    unsigned long long key = 0ull;
    if (HEADS) {
      // a dead position's head is that of -inf: it qualifies only when T is -inf itself
      q = cv[j] >= (T >> 16);
    } else {
      key = tile_key(live ? __uint_as_float(cv[j]) : -INFINITY, pos);
      q = (uint32_t)(key >> 32) >= T;
    }
    const unsigned long long m = __ballot(q);
    if (q) s_ck[nc + lanes_below(m, lane)] = HEADS ? (unsigned long long)pos : key;
    nc += __popcll(m);
  }
  __syncthreads();
  if (HEADS) {
    // exact scores of the list, four candidates' codes in flight per lane (a dead candidate
    // scores -inf; its code address is clamped into the row's written positions)
    const int kvr = row / GQ;
    for (int i0 = 0; i0 < nc; i0 += 256) {
      int pos[4];
      uint4 c0[4], c1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = min(i0 + u * 64 + lane, nc - 1);
        pos[u] = (int)s_ck[i];
        const long cpos = max(min(pos[u], dead_hi - 1), 0);
        const uint4* cp = reinterpret_cast<const uint4*>(rs.codes + ((long)kvr * rs.lmax + cpos) * 32);
        c0[u] = cp[0];
        c1[u] = cp[1];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * 64 + lane;
        const bool live = pos[u] >= ns && pos[u] < dead_hi;
        if (i < nc)
          s_ck[i] = tile_key(live ? oa::qgs_score_words(c0[u], c1[u], lw, inv) : -INFINITY, pos[u]);
      }
    }
    __syncthreads();
  }
  // ---- the k-th largest candidate key: 32 score bits, then the position bits (positions are
  // below 2^24, so bits 24..31 of ~position are all ones)
  unsigned long long T2 = 0xff000000ull;
  for (int bit = 63; bit >= 0; bit = bit == 32 ? 23 : bit - 1) {
    const unsigned long long cand = T2 | (1ull << bit);
    int cnt = 0;
    for (int i0 = 0; i0 < nc; i0 += 64) cnt += __popcll(__ballot(i0 + lane < nc && s_ck[i0 + lane] >= cand));
    if (cnt >= k_top) T2 = cand;
  }
  // ---- the k winners (keys >= T2), then each one's rank among them (descending keys)
  int nw = 0;
  for (int i0 = 0; i0 < nc; i0 += 64) {
    const bool w = i0 + lane < nc && s_ck[i0 + lane] >= T2;
    const unsigned long long m = __ballot(w);
    if (w) s_win[nw + lanes_below(m, lane)] = s_ck[i0 + lane];
    nw += __popcll(m);
  }
  __syncthreads();
  int32_t* sr = sel + (long)row * sel_stride;
  if (lane < ns) sr[lane] = lane;
  if (lane < nl) sr[ns + lane] = n - nl + lane;
  if (lane < k_top) {
    const unsigned long long x = s_win[lane];
    int rank = 0;
    for (int i = 0; i < k_top; ++i) rank += s_win[i] > x ? 1 : 0;
    const int pos = (int)(0xffffffffu - (unsigned)(x & 0xffffffffull));
    sr[ns + nl + rank] = pos;
    mark_selected<HEADS>(Sv, s_stride, row, pos);
  }
}

// Register variant for rows of at most 64*TPL tiles and k_top <= KR, one wave per row (the row
// body, topk_reg_row, is shared with the small-batch top-k + gate + fill launch)
template <int TPL, int KR, bool HEADS>
__global__ void __launch_bounds__(64) topk_select_reg_kernel(void* __restrict__ Sv, long s_stride,
                                                             const float* __restrict__ TM,
                                                             long tm_stride, int ntiles,
                                                             int32_t* __restrict__ sel,
                                                             long sel_stride,
                                                             const int* __restrict__ n_dev, int ns,
                                                             int nl, int k_top, Rescore rs) {
  const int row = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2
  topk_reg_row<TPL, KR, HEADS>(Sv, s_stride, TM, tm_stride, ntiles, sel, sel_stride, *n_dev, ns,
                               nl, k_top, rs, row, threadIdx.x);
}

}  // namespace

extern "C" int oa_qgs_prep(const void* q, long q_stride, const float* U, const float* scale,
                           int rows, int kv_rows, int head_dim, int rank, int8_t* limbs, int* fexp,
                           float* zq_out, void* stream) {
  if (head_dim != OA_D || rank != RQ || kv_rows <= 0 || rows != kv_rows * GQ) return OA_EINVAL;
  hipLaunchKernelGGL(qgs_prep_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream,
                     (const uint16_t*)q, q_stride, U, scale, GQ, limbs, fexp, zq_out);
  return OA_LAUNCH_STATUS();
}

namespace {
template <bool HEADS>
int launch_scan(const int8_t* codes, int kv_rows, int Lmax, int rank, const int8_t* limbs,
                const int* fexp, void* S, long s_stride, float* TM, long tm_stride, float* TMn,
                const int* n_dev, int ns, int nl, void* stream) {
  if (rank != RQ || kv_rows <= 0 || Lmax <= 0) return OA_EINVAL;
  const int ntile = (Lmax + 63) / 64;
  if (s_stride < (long)ntile * 64 || tm_stride < ntile || ns < 0 || nl < 0) return OA_EINVAL;
  dim3 grid((Lmax + kTokWG - 1) / kTokWG, kv_rows);
  const ScanArgs sa{codes, Lmax, limbs, fexp, S, s_stride, TM, tm_stride, n_dev, ns, nl, TMn};
  if (TMn)
    hipLaunchKernelGGL((qgs_scan_kernel<HEADS, true>), grid, dim3(kScanThreads), 0, (hipStream_t)stream, sa);
  else
    hipLaunchKernelGGL((qgs_scan_kernel<HEADS, false>), grid, dim3(kScanThreads), 0, (hipStream_t)stream, sa);
  return OA_LAUNCH_STATUS();
}

template <bool HEADS>
int launch_topk(void* S, long s_stride, const float* TM, long tm_stride, int rows, int ntiles,
                int32_t* sel, long sel_stride, const int* n_dev, int ns, int nl, int k_top,
                Rescore rs, void* stream) {
  if (rows <= 0 || ntiles <= 0 || ntiles > kMaxTilesLds || k_top < 0 || k_top > kMaxTop ||
      k_top > ntiles || ns < 0 || nl < 0 || ns > 64 || nl > 64 || sel_stride < ns + nl + k_top)
    return OA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  // register variants sized to the row: TPL tiles per lane, KR candidate columns
#define OA_TOPK_REG(T, KK)                                                                     \
  hipLaunchKernelGGL((topk_select_reg_kernel<T, KK, HEADS>), dim3(rows), dim3(64), 0, st, S,    \
                     s_stride, TM, tm_stride, ntiles, sel, sel_stride, n_dev, ns, nl, k_top, rs)
  const int tpl = (ntiles + 63) / 64;
  if (k_top <= 9 && tpl <= 9) OA_TOPK_REG(9, 9);
  else if (k_top <= 16 && tpl <= 16) OA_TOPK_REG(16, 16);
  else if (k_top <= 16 && tpl <= 32) OA_TOPK_REG(32, 16);
  else {
    // the radix-select variant, sized to the row's tiles
#define OA_TOPK_RS(T)                                                                          \
  hipLaunchKernelGGL((topk_select_kernel<T, HEADS>), dim3(rows), dim3(64), 0, st, S, s_stride,  \
                     TM, tm_stride, ntiles, sel, sel_stride, n_dev, ns, nl, k_top, rs)
    if (tpl <= 16) OA_TOPK_RS(16);
    else if (tpl <= 32) OA_TOPK_RS(32);
    else OA_TOPK_RS(64);
#undef OA_TOPK_RS
  }
#undef OA_TOPK_REG
  return OA_LAUNCH_STATUS();
}
}  // namespace

extern "C" int oa_qgs_scan(const int8_t* codes, int kv_rows, int Lmax, int rank, const int8_t* limbs,
                           const int* fexp, float* S, long s_stride, float* TM, long tm_stride,
                           const int* n_dev, int ns, int nl, void* stream) {
  return launch_scan<false>(codes, kv_rows, Lmax, rank, limbs, fexp, S, s_stride, TM, tm_stride,
                            nullptr, n_dev, ns, nl, stream);
}

extern "C" int oa_qgs_scan_heads(const int8_t* codes, int kv_rows, int Lmax, int rank,
                                 const int8_t* limbs, const int* fexp, uint16_t* H, long h_stride,
                                 float* TM, long tm_stride, float* TMn, const int* n_dev, int ns,
                                 int nl, void* stream) {
  if (!H || (reinterpret_cast<uintptr_t>(H) & 7) || h_stride % 4) return OA_EINVAL;
  return launch_scan<true>(codes, kv_rows, Lmax, rank, limbs, fexp, H, h_stride, TM, tm_stride,
                           TMn, n_dev, ns, nl, stream);
}

extern "C" int oa_topk_select(float* S, long s_stride, const float* TM, long tm_stride, int rows,
                              int ntiles, int32_t* sel, long sel_stride, const int* n_dev, int ns,
                              int nl, int k_top, void* stream) {
  return launch_topk<false>(S, s_stride, TM, tm_stride, rows, ntiles, sel, sel_stride, n_dev, ns,
                            nl, k_top, Rescore{nullptr, 0, nullptr, nullptr}, stream);
}

extern "C" int oa_topk_select_heads(uint16_t* H, long h_stride, const float* TM, long tm_stride,
                                    int rows, int ntiles, int32_t* sel, long sel_stride,
                                    const int* n_dev, int ns, int nl, int k_top,
                                    const int8_t* codes, int kv_rows, int Lmax,
                                    const int8_t* limbs, const int* fexp, void* stream) {
  if (!H || !codes || !limbs || !fexp || kv_rows <= 0 || rows != kv_rows * GQ || Lmax <= 0 ||
      (reinterpret_cast<uintptr_t>(codes) & 15) || (reinterpret_cast<uintptr_t>(limbs) & 3))
    return OA_EINVAL;
  return launch_topk<true>(H, h_stride, TM, tm_stride, rows, ntiles, sel, sel_stride, n_dev, ns,
                           nl, k_top, Rescore{codes, (long)Lmax, limbs, fexp}, stream);
}

extern "C" int oa_qgs_scan_gate(const int8_t* codes, int kv_rows, int Lmax, int rank,
                                const int8_t* limbs, const int* fexp, uint16_t* H, long h_stride,
                                float* TM, long tm_stride, float* TMn, const int* n_dev, int ns,
                                int nl, const void* q, long q_stride, const float* Sk, const float* Sk2,
                                const float* nb, int C, float sm_scale, float sm_scale_sq,
                                float* score, float* n_t, float* qsk, void* stream) {
  if (!H || (reinterpret_cast<uintptr_t>(H) & 7) || h_stride % 4 || rank != RQ || kv_rows <= 0 ||
      Lmax <= 0 || !q || !Sk || !Sk2 || !nb || !score || !n_t || C <= 0 || C > 256)
    return OA_EINVAL;
  const int ntile = (Lmax + 63) / 64;
  if (h_stride < (long)ntile * 64 || tm_stride < ntile || ns < 0 || nl < 0) return OA_EINVAL;
  const ScanArgs sa{codes, Lmax, limbs, fexp, H, h_stride, TM, tm_stride, n_dev, ns, nl, TMn};
  oa_gate::GateArgs ga{};
  ga.q = (const uint16_t*)q; ga.q_stride = q_stride;
  ga.Sk = Sk; ga.Sk2 = Sk2; ga.st_stride_r = (long)C * OA_D;
  ga.nb = nb; ga.nb_stride = C;
  ga.score = score; ga.n_t = n_t; ga.out_stride = C; ga.qsk = qsk;
  ga.C = C; ga.sc = sm_scale; ga.sc2 = sm_scale_sq;
  const int rows = kv_rows * GQ;
  const int nchunks = (Lmax + kTokWG - 1) / kTokWG;
  const long n_scan = (long)nchunks * kv_rows;
  const long n_gate = (long)rows * ((C + oa_gate::kPoolClusters - 1) / oa_gate::kPoolClusters);
  if (n_scan + n_gate > 0x7fffffffL) return OA_EINVAL;
  hipLaunchKernelGGL(TMn ? qgs_scan_gate_kernel<true> : qgs_scan_gate_kernel<false>,
                     dim3((unsigned)(n_scan + n_gate)), dim3(kScanThreads), 0,
                     (hipStream_t)stream, sa, ga, nchunks, (int)n_scan, (int)n_gate);
  return OA_LAUNCH_STATUS();
}
