// ErrorGate (wl1 cluster score) and hierarchical water-filling of the exact-read budget E.
//
// ErrorGate follows the accuracy-path estimator: tail statistics of every QGC cluster are the
// cached pooled sums minus the selected tokens (methods_eager.py:612-627, ours_fused.py:122-154),
// moments as UTAMultiBinAttention._moments_from_key_stats (multibin.py:605-644) with
// s2 = 0 for clusters of fewer than two tail tokens (multibin.py:734-738), and the wl1 score
// zbar + log n + s2/2 + log max(erf(sqrt(s2)/sqrt2), 1e-30) (multibin.py:2370-2389).
//
// Water-filling is UTAMultiBinAttention._hier_quota_impl (multibin.py:1385-1422): fp64,
// w_b = exp(s_b - max s), 64 bisection steps on log(lambda) for sum_b min(n_b, lambda w_b) = E,
// q_b = floor(min(n_b, lambda w_b)) (q = n when the tail is smaller than E), leftover tokens one
// each to the highest-score live clusters with room, in score order (ties to the lower
// cluster id).  Sums that feed comparisons use a fixed order (lane-strided partials, then the
// wave butterfly) and the elementary functions come from oa_detmath.h, so the integer quotas
// are reproducible bit for bit on the CPU.
#include "oa_common.h"
#include "oa_detmath.h"
#include "oa_topk_row.h"
#include "oa_gate_row.h"

namespace {

using namespace oa_gate;

constexpr int kGateThreads = 512;
constexpr int kGateWaves = kGateThreads / 64;
constexpr int kMaxSel = 64;
constexpr int kMaxC = 256;
constexpr int kFuseRows = 256;       // oa_gate_fill: one fused launch below this many rows

// ErrorGate of one row by a 512-thread workgroup into LDS rows (score, n_t).  The wave-wide dot
// products run six clusters per wave at a time with all their loads in flight; the scalar tails (erf, logs)
// then run one cluster per thread.  Dynamic LDS: n_sel * 128 floats of selected keys.
__device__ __forceinline__ void gate_row(const GateArgs& a, int row, float* s_score, float* s_nt) {
  extern __shared__ float s_k[];
  __shared__ unsigned long long s_selmask[kMaxC];
  __shared__ float s_zbar[kMaxC], s_s2[kMaxC], s_qsk[kMaxC];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int kvr = row / a.G;
  constexpr int kBatch = 4;     // larger batches spill at the 64-VGPR cap
  float sk[kBatch][2], s2[kBatch][2], nbv[kBatch];
  auto issue = [&](int c0) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = min(c0 + kGateWaves * i, a.C - 1);
      const long base = (long)row * a.st_stride_r + (long)c * OA_D;
      sk[i][0] = a.Sk[base + lane];
      sk[i][1] = a.Sk[base + lane + 64];
      s2[i][0] = a.Sk2[base + lane];
      s2[i][1] = a.Sk2[base + lane + 64];
      nbv[i] = a.nb[(long)row * a.nb_stride + c];
    }
  };
  for (int c = tid; c < a.C; c += kGateThreads) s_selmask[c] = 0ull;
  __syncthreads();
  if (wave < a.C) issue(wave);
  // the selected positions (one per thread for the cluster masks, up to two 16-byte key words per
  // thread for the staged keys), then their cluster ids and key words, all requested before the
  // first batch is computed
  constexpr int kW = OA_D / 8;
  const long srow = (long)row * a.sel_stride;
  const int n_sel = a.n_sel;
  const int e0 = tid, e1 = tid + kGateThreads;
  const int tokm = tid < n_sel ? a.sel[srow + tid] : -1;
  const int tok0 = e0 < n_sel * kW ? a.sel[srow + e0 / kW] : -1;
  const int tok1 = e1 < n_sel * kW ? a.sel[srow + e1 / kW] : -1;
  const float q_lo = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane]);
  const float q_hi = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane + 64]);
  const float qq_lo = q_lo * q_lo, qq_hi = q_hi * q_hi;
  const int cm = tokm >= 0 ? a.asg[(long)row * a.asg_stride + tokm] : -1;
  uint4 kw0 = make_uint4(0u, 0u, 0u, 0u), kw1 = kw0;
  if (tok0 >= 0)
    kw0 = *reinterpret_cast<const uint4*>(a.K + (long)kvr * a.k_sb + (long)tok0 * a.k_ss + (e0 % kW) * 8);
  if (tok1 >= 0)
    kw1 = *reinterpret_cast<const uint4*>(a.K + (long)kvr * a.k_sb + (long)tok1 * a.k_ss + (e1 % kW) * 8);
  auto dots = [&](float k0, float k1, float t0, float t1, float nbc, int c,
                  unsigned long long mask) {
    float zb, sv, nt, qs;
    gate_dots(a, k0, k1, t0, t1, nbc, q_lo, q_hi, qq_lo, qq_hi, mask, s_k, lane, &zb, &sv, &nt, &qs);
    if (lane == 0) {
      s_zbar[c] = zb;
      s_s2[c] = sv;
      s_nt[c] = nt;
      s_qsk[c] = qs;
    }
  };
  // ---- the first batch as if its clusters held no selected token (most do not) while the
  // selected keys arrive; a cluster that holds one is done again below
#pragma unroll
  for (int i = 0; i < kBatch; ++i) {
    const int c = wave + kGateWaves * i;
    if (c < a.C) dots(sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], c, 0ull);
  }
  // ---- selected keys into LDS; per cluster, the mask of its selected tokens
  if (cm >= 0) atomicOr(&s_selmask[cm], 1ull << tid);
  if (e0 < n_sel * kW) {
    float x[8];
    oa::unpack8(kw0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_k[(e0 / kW) * OA_D + (e0 % kW) * 8 + j] = x[j];
  }
  if (e1 < n_sel * kW) {
    float x[8];
    oa::unpack8(kw1, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_k[(e1 / kW) * OA_D + (e1 % kW) * 8 + j] = x[j];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kBatch; ++i) {
    const int c = wave + kGateWaves * i;
    if (c < a.C && s_selmask[c]) dots(sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], c, s_selmask[c]);
  }
  // ---- the other batches, all loads of a batch in flight
  for (int c0 = wave + kGateWaves * kBatch; c0 < a.C; c0 += kGateWaves * kBatch) {
    issue(c0);
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = c0 + kGateWaves * i;
      if (c < a.C) dots(sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], c, s_selmask[c]);
    }
  }
  __syncthreads();
  // ---- scalar tails, one cluster per thread
  for (int c = tid; c < a.C; c += kGateThreads) {
    s_score[c] = gate_score(s_zbar[c], s_s2[c], s_nt[c]);
    if (a.qsk) a.qsk[(long)row * a.C + c] = s_qsk[c];
  }
  __syncthreads();
}

// 8 waves per SIMD (<= 64 VGPRs): every row of a B=32 batch is resident at once
__global__ void __launch_bounds__(kGateThreads, 8) errorgate_kernel(GateArgs a) {
  __shared__ float s_score[kMaxC], s_nt[kMaxC];
  const int row = blockIdx.x;
  gate_row(a, row, s_score, s_nt);
  for (int c = threadIdx.x; c < a.C; c += kGateThreads) {
    a.score[(long)row * a.out_stride + c] = s_score[c];
    a.n_t[(long)row * a.out_stride + c] = s_nt[c];
  }
}

// one wave per row; cluster c lives in lane c % 64, slot c / 64 (NS slots per lane)
template <int NS>
__device__ __forceinline__ double canon_sum(const double* x, int C, int lane) {
  double p = 0.0;
  bool first = true;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    int c = lane + 64 * j;
    if (c < C) {
      p = first ? x[j] : p + x[j];
      first = false;
    }
  }
  return oa::wave_sum(p);
}

// the wave maximum on the DPP / permlane-swap network (no LDS round trips; the maximum does not
// depend on the order, and a zero's sign does not matter where it is used)
__device__ __forceinline__ double swap_max(unsigned lo0, unsigned hi0, unsigned lo1, unsigned hi1) {
  const double x = __longlong_as_double((long long)(((unsigned long long)hi0 << 32) | lo0));
  const double y = __longlong_as_double((long long)(((unsigned long long)hi1 << 32) | lo1));
  return fmax(x, y);
}
__device__ __forceinline__ double wave_max_f64(double v) {
  v = fmax(v, oa::dpp_f64<0xB1>(v));
  v = fmax(v, oa::dpp_f64<0x4E>(v));
  v = fmax(v, oa::dpp_f64<0x141>(v));
  v = fmax(v, oa::dpp_f64<0x140>(v));
  unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const auto l16 = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
  const auto h16 = __builtin_amdgcn_permlane16_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
  v = swap_max(l16[0], h16[0], l16[1], h16[1]);
  b = (unsigned long long)__double_as_longlong(v);
  const auto l32 = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
  const auto h32 = __builtin_amdgcn_permlane32_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
  return swap_max(l32[0], h32[0], l32[1], h32[1]);
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)b, l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// f = sum_b min(cap_b, em w_b) in the canonical order, em = exp(mid)
template <int NS>
__device__ __forceinline__ double fill_em(double em, const double* cap, const double* w, int C,
                                          int lane) {
  double part[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) part[j] = fmin(cap[j], em * w[j]);
  return canon_sum<NS>(part, C, lane);
}

// Water-filling, split so that the one-wave kernel and the workgroup-wide variant run the same
// arithmetic.  Cluster c lives in lane c % 64, slot c / 64 of a wave.
template <int NS>
struct FillState {
  double sv[NS], w[NS], cap[NS];
  bool ok[NS];
  double lo, hi, tot;
};

// live clusters, weights w_b = exp(s_b - max s), total tail, and the bracket of log(lambda)
template <int NS>
__device__ __forceinline__ void fill_prologue(const float* score_row, const float* nt_row, int C,
                                              int lane, FillState<NS>& f) {
  const double NEG = __longlong_as_double((long long)0xfff0000000000000ULL);
  double smax = NEG;
  for (int j = 0; j < NS; ++j) {
    int c = lane + 64 * j;
    f.sv[j] = NEG; f.w[j] = 0.0; f.cap[j] = 0.0; f.ok[j] = false;
    if (c < C) {
      float nt = nt_row[c];
      f.ok[j] = nt > 1.0f;
      if (f.ok[j]) {
        f.sv[j] = (double)score_row[c];
        f.cap[j] = (double)nt;
      }
      smax = fmax(smax, f.sv[j]);
    }
  }
  smax = wave_max_f64(smax);
  if (!(smax > NEG && smax < -NEG)) smax = 0.0;
  double rmax = 0.0;
  for (int j = 0; j < NS; ++j) {
    if (f.ok[j]) f.w[j] = oa::det_exp(f.sv[j] - smax);
    double ratio = (f.w[j] > 0.0) ? f.cap[j] / fmax(f.w[j], 1e-300) : 0.0;
    if (lane + 64 * j < C) rmax = fmax(rmax, ratio);
  }
  rmax = wave_max_f64(rmax);
  // the butterfly leaves one value on every lane; lane 0's copy lets the compiler branch on it
  // as a wave-uniform value
  f.tot = readlane_f64(canon_sum<NS>(f.cap, C, lane), 0);
  f.lo = -3.0 * 2.302585092994046;
  f.hi = readlane_f64(oa::det_log(fmax(rmax, 1e-3)) + 1.0, 0);
}

// quotas floor(min(n_b, lambda w_b)) at the final lo, leftover tokens one each to the live
// clusters with room in score order (dead clusters as -inf), ties to the lower id.
//
// The leftover order: every cluster with room has the distinct 40-bit key (order-preserving key
// of its score << 8) | (255 - id), larger = earlier, and the rem largest keys take one more
// token.  With one cluster per lane (C <= 64) each lane counts the keys above its own (every
// lane's key staged in s_key, keys of clusters without room as 0, which no key is below); with
// more, the rem-th largest key is found bit by bit from the top (40 wave-wide counts).  Both
// give the set that ranking every cluster against every other gives.
template <int NS>
__device__ __forceinline__ void fill_epilogue(const FillState<NS>& f, int C, double budget, int lane,
                                              float* quota_row, unsigned long long* s_key) {
  double qv[NS];
  const double el = oa::det_exp(f.lo);
  for (int j = 0; j < NS; ++j) {
    qv[j] = floor(fmin(f.cap[j], el * f.w[j]));
    if (f.tot <= budget) qv[j] = f.cap[j];
  }
  const double qsum = readlane_f64(canon_sum<NS>(qv, C, lane), 0);
  double rem = fmin(f.tot, budget) - qsum;
  rem = rint(rem > 0.0 ? rem : 0.0);
  unsigned long long u[NS];
  bool room[NS];
  int total = 0;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int c = lane + 64 * j;
    // dead clusters rank below every live one (key 0; they have no room anyway); -0 and +0 are
    // one score (a tie, settled by the id)
    const float sf = (float)f.sv[j];
    const unsigned kf = f.ok[j] ? oa::float_key(sf == 0.f ? 0.f : sf) : 0u;
    room[j] = c < C && qv[j] < f.cap[j] && kf != 0xffffffffu;
    u[j] = ((unsigned long long)kf << 8) | (unsigned long long)(255 - (c & 255));
    if (NS > 1) total += __popcll(__ballot(room[j]));
  }
  const bool any = rem > 0.0;
  if (NS == 1) {
    const unsigned long long mk = room[0] ? u[0] : 0ull;
    s_key[lane] = mk;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const ulonglong2* kp = reinterpret_cast<const ulonglong2*>(s_key);
    int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll 2
    for (int i = 0; i < 32; i += 2) {
      const ulonglong2 x = kp[i], y = kp[i + 1];
      c0 += x.x > mk ? 1 : 0;
      c1 += x.y > mk ? 1 : 0;
      c2 += y.x > mk ? 1 : 0;
      c3 += y.y > mk ? 1 : 0;
    }
    const double rank = (double)((c0 + c1) + (c2 + c3));
    if (lane < C) quota_row[lane] = (float)(qv[0] + ((any && room[0] && rank < rem) ? 1.0 : 0.0));
    return;
  }
  unsigned long long t = 0ull;                      // keys >= t get one more
  if (any && rem < (double)total) {
    int need = (int)rem;
    for (int bit = 39; bit >= 0; --bit) {
      const unsigned long long cand = t | (1ull << bit);
      int cnt = 0;
#pragma unroll
      for (int j = 0; j < NS; ++j) cnt += __popcll(__ballot(room[j] && (u[j] >> bit) == (cand >> bit)));
      if (cnt >= need) t = cand;
      else need -= cnt;
    }
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int c = lane + 64 * j;
    if (c < C) quota_row[c] = (float)(qv[j] + ((any && room[j] && u[j] >= t) ? 1.0 : 0.0));
  }
}

// water-filling of one row by one wave (lane = threadIdx.x % 64); score/n_t rows may be in LDS.
//
// The 64 bisection steps run as rounds of DEPTH steps.  A round evaluates, in parallel, every
// midpoint the next DEPTH sequential steps could visit: the probe tree in heap order (node 1 =
// mid of (lo, hi); node 2n takes the left half (f > E: hi = mid), node 2n+1 the right half),
// P lanes per node, node n in lanes [nP, nP + P).  Each node's interval is rebuilt from
// (lo, hi) by the same 0.5 * (lo + hi) operations the sequential steps perform, so its midpoint
// is the one the sequential bisection would probe if it reached that node.  f at a node is the
// canonical sum: the lane partial of canonical lane l is its clusters l, l + 64, ... added in
// slot order, the 64 lane partials are added by the balanced pairwise tree of the xor butterfly
// (m = 1, 2, ..., 32; IEEE addition is commutative, so every lane of the butterfly holds that
// tree's value).  Here each of a node's P lanes adds 64 / P consecutive lane partials by the
// lower levels of that tree and the node's lanes add the P subtotals by its top levels.  The
// walk down the tree then takes the sequential path from the ballot of f > E.
//
// Most steps need no probe.  The computed f is a non-decreasing function F of em = exp(mid)
// (min(cap, RN(em w)) with w >= 0, and IEEE sums of non-negative terms in a fixed order, are
// monotone), and det_exp is within 2^-51 of exp, so det_exp(x) <= det_exp(a) (1 + 2^-49.9) for
// every x <= a.  One round probes F at em = det_exp(x) (1 + 2^-47) for points x = a below the
// water level's estimate and at det_exp(x) (1 - 2^-47) for points x = b above it: F <= E there
// proves f(mid) <= E for every mid <= a, F > E proves f(mid) > E for every mid >= b.  The
// sequential steps whose midpoint lies outside (a, b) then take their branch without a probe,
// and a step whose midpoint is a bound already probed changes nothing (neither can any later
// one).  The estimate is the fixed point of lambda = (E - sum of the capped n_b) / (sum of the
// other w_b); a bracket not proven leaves every step to the probes.
template <int NS>
__device__ __forceinline__ void waterfill_row(const float* score_row, const float* nt_row,
                                              float* quota_row, int C, double budget, int lane,
                                              double2* s_cw) {
  // ---- live clusters, weights and the bracket of log(lambda)
  FillState<NS> f;
  fill_prologue<NS>(score_row, nt_row, C, lane, f);
  // the tail fits the budget: every quota is its cap, the bisection's result is not used
  if (!(f.tot > budget)) {
    fill_epilogue<NS>(f, C, budget, lane, quota_row, reinterpret_cast<unsigned long long*>(s_cw));
    return;
  }
  // 8 lanes per probe node: each lane then adds only 8 canonical lane partials, and a round's
  // fp64 work (not its latency) is what the lane count trades against the round count
  constexpr int P = 8;                       // lanes per probe node
  constexpr int NL = 64 / P;                 // canonical lane partials per lane (= nodes + 1)
  constexpr int DEPTH = 3;                   // log2(NL): nodes 1 .. NL - 1
  static_assert((1 << DEPTH) == NL, "probe tree shape");
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int c = lane + 64 * j;
    if (c < C) s_cw[c] = make_double2(f.cap[j], f.w[j]);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // this lane's share: canonical lane partials l = sub * NL + i, clusters l + 64 j (zero past C:
  // min(0, em * 0) = +0 leaves a sum of non-negative terms unchanged)
  const int sub = lane % P;
  const int node = lane / P;
  double cp[NL][NS], wp[NL][NS];
#pragma unroll
  for (int i = 0; i < NL; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int c = sub * NL + i + 64 * j;
      const double2 v = c < C ? s_cw[c] : make_double2(0.0, 0.0);
      cp[i][j] = v.x;
      wp[i][j] = v.y;
    }
  // f at em for this lane's node (the same value on the node's P lanes)
  auto probe = [&](double em) {
    double part[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      double p = fmin(cp[i][0], em * wp[i][0]);
#pragma unroll
      for (int j = 1; j < NS; ++j) p = p + fmin(cp[i][j], em * wp[i][j]);
      part[i] = p;
    }
#pragma unroll
    for (int st = 1; st < NL; st <<= 1)
#pragma unroll
      for (int i = 0; i < NL; i += 2 * st) part[i] = part[i] + part[i + st];
    double fv = part[0];
    fv = fv + oa::dpp_f64<0xB1>(fv);                   // node lanes xor 1
    if (P >= 4) fv = fv + oa::dpp_f64<0x4E>(fv);       // xor 2
    if (P >= 8) fv = fv + oa::dpp_f64<0x141>(fv);      // xor 4 (4-lane groups are uniform)
    return fv;
  };
  // ---- the proven bracket (a, b)
  const double INF = __longlong_as_double(0x7ff0000000000000LL);
  double a = -INF, b = INF;
  {
    bool capped[NS];
    double lam = 0.0;
#pragma unroll
    for (int j = 0; j < NS; ++j) capped[j] = false;
    for (int it = 0; it < 16; ++it) {
      double sc = 0.0, sw = 0.0;
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        if (capped[j]) sc += f.cap[j];
        else sw += f.w[j];
      }
      sc = readlane_f64(oa::wave_sum(sc), 0);
      sw = readlane_f64(oa::wave_sum(sw), 0);
      const double l = (budget - sc) / sw;
      if (!(l > 0.0 && l < INF)) break;
      lam = l;
      bool changed = false;
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const bool cj = f.cap[j] <= l * f.w[j];
        changed = changed || cj != capped[j];
        capped[j] = cj;
      }
      if (!__any(changed)) break;
    }
    const double x0 = oa::det_log(lam);
    if (x0 > -600.0 && x0 < 600.0) {
      // nodes 0-3 probe below x0, nodes 4-7 above, nearest first
      const int rung = node & 3;
      const bool up = node >= 4;
      const double dl = fmax(fabs(x0), 0.0625) *
                        (rung == 0 ? 0x1p-46 : rung == 1 ? 0x1p-43 : rung == 2 ? 0x1p-38 : 0x1p-26);
      const double xk = up ? x0 + dl : x0 - dl;
      const double em = oa::det_exp(xk) * (up ? 1.0 - 0x1p-47 : 1.0 + 0x1p-47);
      const unsigned long long gt = __ballot(probe(em) > budget);
      for (int k = 0; k < 4; ++k)
        if (!((gt >> (k * P)) & 1ull)) { a = readlane_f64(xk, k * P); break; }
      for (int k = 4; k < 8; ++k)
        if ((gt >> (k * P)) & 1ull) { b = readlane_f64(xk, k * P); break; }
    }
  }
  const int lev = node > 0 ? 31 - __clz(node) : 0;   // depth of this lane's node (root 0)
  // ---- 64 bisection steps: decided by the bracket, or DEPTH per round of probes
  double lo = f.lo, hi = f.hi;
  bool lo_probed = false, hi_probed = false;          // f at lo (hi) known to be <= E (> E)
  int done = 0;
  while (done < 64) {
    double m = 0.5 * (lo + hi);
    if ((m == lo && lo_probed) || (m == hi && hi_probed)) break;   // a fixed point
    // steps the bracket decides, 8 at a time and without branches: a step it cannot decide
    // changes nothing, so every step after it stays undecided as well.  The bounds are carried
    // halved: 0.5 lo + 0.5 hi is 0.5 (lo + hi) exactly (halving is exact and commutes with
    // rounding), and the halving of a new bound then runs beside its comparisons
    if (64 - done >= 8) {
      double lh = 0.5 * lo, hh = 0.5 * hi;
      int dec = 0;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const double mm = lh + hh;
        const double mh = 0.5 * mm;
        const bool L = mm <= a;
        const bool H = mm >= b;
        lh = L ? mh : lh;
        hh = H ? mh : hh;
        lo_probed = lo_probed || L;
        hi_probed = hi_probed || H;
        dec += (L || H) ? 1 : 0;
      }
      lo = 2.0 * lh;
      hi = 2.0 * hh;
      done += dec;
      if (dec == 8) continue;
    } else if (m <= a || m >= b) {
      if (m <= a) { lo = m; lo_probed = true; } else { hi = m; hi_probed = true; }
      ++done;
      continue;
    }
    m = 0.5 * (lo + hi);
    if ((m == lo && lo_probed) || (m == hi && hi_probed)) break;
    // the next step needs a probe: one round of DEPTH steps
    const int d = min(DEPTH, 64 - done);
    double nlo = lo, nhi = hi;
    double mid = m;
#pragma unroll
    for (int bt = DEPTH - 2; bt >= 0; --bt) {
      if (bt < lev) {
        if ((node >> bt) & 1) nlo = mid; else nhi = mid;
        mid = 0.5 * (nlo + nhi);
      }
    }
    const unsigned long long gt = __ballot(probe(oa::det_exp_v(mid)) > budget);
    int nd = 1, lo_nd = 0, hi_nd = 0;
    for (int k = 0; k < d; ++k) {
      if ((gt >> (nd * P)) & 1ull) { hi_nd = nd; nd = 2 * nd; }
      else { lo_nd = nd; nd = 2 * nd + 1; }
    }
    if (lo_nd) { lo = readlane_f64(mid, lo_nd * P); lo_probed = true; }
    if (hi_nd) { hi = readlane_f64(mid, hi_nd * P); hi_probed = true; }
    done += d;
  }
  f.lo = lo;
  f.hi = hi;
  // ---- quotas, leftover tokens by score order
  fill_epilogue<NS>(f, C, budget, lane, quota_row, reinterpret_cast<unsigned long long*>(s_cw));
}

// one row per wave: the fill is a serial chain, so rows (not lanes) carry the parallelism
template <int NS>
__global__ void __launch_bounds__(64) waterfill_kernel(const float* __restrict__ score,
                                                       const float* __restrict__ n_t, long in_stride,
                                                       float* __restrict__ quota, long q_stride, int C,
                                                       double budget) {
  __shared__ double2 s_cw[kMaxC];
  const int row = blockIdx.x;
  waterfill_row<NS>(score + (long)row * in_stride, n_t + (long)row * in_stride,
                    quota + (long)row * q_stride, C, budget, threadIdx.x, s_cw);
}

// fewer rows than compute units: the gate and the fill of a row in one workgroup.  The launch
// saved is worth more than the gate's workgroup slots the fill holds when every row is resident
// anyway; the fill reads the gate's scores and n_t from LDS (the same fp32 values it would read
// back from the outputs, which are still written)
template <int NS>
__global__ void __launch_bounds__(kGateThreads) gate_fill_kernel(GateArgs a, float* __restrict__ quota,
                                                                 double budget) {
  __shared__ float s_score[kMaxC], s_nt[kMaxC];
  __shared__ double2 s_cw[kMaxC];
  const int row = blockIdx.x;
  gate_row(a, row, s_score, s_nt);
  for (int c = threadIdx.x; c < a.C; c += kGateThreads) {
    a.score[(long)row * a.out_stride + c] = s_score[c];
    a.n_t[(long)row * a.out_stride + c] = s_nt[c];
  }
  if (threadIdx.x < 64)
    waterfill_row<NS>(s_score, s_nt, quota + (long)row * a.C, a.C, budget, threadIdx.x, s_cw);
}

// the row's top-k arguments (the register top-k of oa_topk_row.h over key heads)
struct TopkArgs {
  uint16_t* H; long h_stride;
  const float* TM; long tm_stride; int ntiles;
  const int* n_dev; int ns, nl, k_top;
  oa_sel::Rescore rs;
};

// ---- the ErrorGate finished after the selection, with the water-fill ------------------------
// oa_qgs_scan_gate left every cluster's score and n_t as if no token were selected (and q . Sk).
// Once sel is known only the clusters holding a selected token change: they are computed again
// from the pooled sums minus their selected keys, in selection order (gate_dots with the
// cluster's mask: the arithmetic of gate_row), and the fill runs on the completed rows.
constexpr int kFixThreads = 256;

struct FixLds {
  float score[kMaxC], nt[kMaxC];
  double2 cw[kMaxC];
  unsigned long long selmask[kMaxC];
  int sel[kMaxSel];
  int hit[kMaxSel];
  float zb[kMaxSel], s2[kMaxSel], hnt[kMaxSel];
  int nhit;
};

// the pooled score and n_t rows into LDS, the masks cleared (threads [t0, t0 + nthreads)); with
// load_sel the row's sel from global memory as well (else the top-k leaves it in L.sel)
__device__ __forceinline__ void fix_load(const GateArgs& a, int row, FixLds& L, int t0, int nthreads,
                                         bool load_sel) {
  const int t = (int)threadIdx.x - t0;
  for (int c = t; c < a.C; c += nthreads) {
    L.score[c] = a.score[(long)row * a.out_stride + c];
    L.nt[c] = a.n_t[(long)row * a.out_stride + c];
    L.selmask[c] = 0ull;
  }
  if (load_sel && t < a.n_sel) L.sel[t] = a.sel[(long)row * a.sel_stride + t];
  if (t == 0) L.nhit = 0;
}

// after fix_load (and the top-k) and a barrier: the clusters holding a selected token done again,
// then the fill (wave 0).  Dynamic LDS: n_sel * 128 floats of selected keys.
template <int NS, int kThr = kFixThreads>
__device__ __forceinline__ void fix_finish(const GateArgs& a, int row, FixLds& L, float* quota_row,
                                           double budget) {
  constexpr int kWv = kThr / 64;
  extern __shared__ float s_k[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int kvr = row / a.G;
  constexpr int kW = OA_D / 8;
  const int n_sel = a.n_sel;
  // selected tokens: cluster ids (one per thread) and key words (16 bytes each, up to four per
  // thread), all requested together
  const int tokm = tid < n_sel ? L.sel[tid] : -1;
  const int cm = tokm >= 0 ? a.asg[(long)row * a.asg_stride + tokm] : -1;
  uint4 kw[4];
  int ke[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = tid + u * kThr;
    ke[u] = e < n_sel * kW ? e : -1;
    kw[u] = make_uint4(0u, 0u, 0u, 0u);
    if (ke[u] >= 0)
      kw[u] = *reinterpret_cast<const uint4*>(a.K + (long)kvr * a.k_sb + (long)L.sel[e / kW] * a.k_ss +
                                              (e % kW) * 8);
  }
  const float q_lo = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane]);
  const float q_hi = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane + 64]);
  if (cm >= 0) {
    const unsigned long long old = atomicOr(&L.selmask[cm], 1ull << tid);
    if (old == 0ull) L.hit[atomicAdd(&L.nhit, 1)] = cm;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (ke[u] < 0) continue;
    float x[8];
    oa::unpack8(kw[u], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_k[(ke[u] / kW) * OA_D + (ke[u] % kW) * 8 + j] = x[j];
  }
  __syncthreads();
  // the hit clusters' dot products: wave w takes hits w, w + 4, ..., kBatch of them with all
  // their loads in flight at a time
  const int nhit = L.nhit;
  const float qq_lo = q_lo * q_lo, qq_hi = q_hi * q_hi;
  constexpr int kBatch = 4;
  for (int h0 = wave; h0 < nhit; h0 += kWv * kBatch) {
    float sk[kBatch][2], s2[kBatch][2], nbv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int h = min(h0 + kWv * i, nhit - 1);
      const int c = L.hit[h];
      const long base = (long)row * a.st_stride_r + (long)c * OA_D;
      sk[i][0] = a.Sk[base + lane];
      sk[i][1] = a.Sk[base + lane + 64];
      s2[i][0] = a.Sk2[base + lane];
      s2[i][1] = a.Sk2[base + lane + 64];
      nbv[i] = a.nb[(long)row * a.nb_stride + c];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int h = h0 + kWv * i;
      if (h < nhit) {
        float zb, sv, nt, qs;
        gate_dots(a, sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], q_lo, q_hi, qq_lo, qq_hi,
                  L.selmask[L.hit[h]], s_k, lane, &zb, &sv, &nt, &qs);
        if (lane == 0) {
          L.zb[h] = zb;
          L.s2[h] = sv;
          L.hnt[h] = nt;
        }
      }
    }
  }
  __syncthreads();
  // the scalar tails, one hit cluster per thread
  if (tid < nhit) {
    const int c = L.hit[tid];
    const float sc = gate_score(L.zb[tid], L.s2[tid], L.hnt[tid]);
    L.score[c] = sc;
    L.nt[c] = L.hnt[tid];
    a.score[(long)row * a.out_stride + c] = sc;
    a.n_t[(long)row * a.out_stride + c] = L.hnt[tid];
  }
  __syncthreads();
  if (wave == 0) waterfill_row<NS>(L.score, L.nt, quota_row, a.C, budget, lane, L.cw);
}

template <int NS>
__global__ void __launch_bounds__(kFixThreads) fix_fill_kernel(GateArgs a, float* __restrict__ quota,
                                                               double budget) {
  __shared__ FixLds L;
  const int row = blockIdx.x;
  fix_load(a, row, L, 0, kFixThreads, true);
  __syncthreads();
  fix_finish<NS>(a, row, L, quota + (long)row * a.C, budget);
}

// the row's register top-k (wave 0, its sel row also into LDS) while the other waves stage the
// pooled rows, then the correction and the fill
template <int NS, int TPL, int KR>
__global__ void __launch_bounds__(kFixThreads) topk_fix_fill_kernel(TopkArgs t, GateArgs a, int32_t* sel,
                                                                    float* __restrict__ quota,
                                                                    double budget) {
  __shared__ FixLds L;
  const int row = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2
  if (threadIdx.x < 64)
    oa_sel::topk_reg_row<TPL, KR, true>(t.H, t.h_stride, t.TM, t.tm_stride, t.ntiles, sel,
                                        a.sel_stride, *t.n_dev, t.ns, t.nl, t.k_top, t.rs, row,
                                        threadIdx.x, L.sel);
  else
    fix_load(a, row, L, 64, kFixThreads - 64, false);
  __syncthreads();
  fix_finish<NS>(a, row, L, quota + (long)row * a.C, budget);
}

// ---- top-k, ErrorGate and water-fill of a row in one workgroup, the gate's pooled part
// concurrent with the top-k -----------------------------------------------------------------
// Wave 0 runs the row's register top-k while waves 1 .. W-1 compute the clusters' pooled
// ErrorGate dot products (gate_dots with an empty mask): wave w takes the batches of kPoolBatch
// consecutive clusters w - 1, w - 1 + (W - 1), ... (a fixed split: every loop bound depends on
// the wave index and C only), all of a batch's loads in flight.  Then every cluster's scalar
// tail (one per thread), the clusters holding a selected token done again with their masks
// (fix_finish), and the fill on wave 0.  Every cluster's score and n_t, and q . Sk, are
// written out.
constexpr int kPoolBatch = 8;
struct Gate2Lds {
  FixLds f;
  float zb[kMaxC], s2[kMaxC], nt[kMaxC];
};

template <int W>
__device__ __forceinline__ void pooled_batches(const GateArgs& a, int row, Gate2Lds& L) {
  constexpr int nGW = W - 1;
  const int gw = (int)(threadIdx.x >> 6) - 1;       // 0 .. W-2
  const int lane = threadIdx.x & 63;
  const float q_lo = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane]);
  const float q_hi = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane + 64]);
  const float qq_lo = q_lo * q_lo, qq_hi = q_hi * q_hi;
  for (int c0 = gw * kPoolBatch; c0 < a.C; c0 += nGW * kPoolBatch) {
    float sk[kPoolBatch][2], s2[kPoolBatch][2], nbv[kPoolBatch];
#pragma unroll
    for (int i = 0; i < kPoolBatch; ++i) {
      const int c = min(c0 + i, a.C - 1);
      const long base = (long)row * a.st_stride_r + (long)c * OA_D;
      sk[i][0] = a.Sk[base + lane];
      sk[i][1] = a.Sk[base + lane + 64];
      s2[i][0] = a.Sk2[base + lane];
      s2[i][1] = a.Sk2[base + lane + 64];
      nbv[i] = a.nb[(long)row * a.nb_stride + c];
    }
#pragma unroll
    for (int i = 0; i < kPoolBatch; ++i) {
      const int c = c0 + i;
      if (c < a.C) {
        float zb, sv, nt, qs;
        gate_dots(a, sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], q_lo, q_hi, qq_lo, qq_hi, 0ull,
                  nullptr, lane, &zb, &sv, &nt, &qs);
        if (lane == 0) {
          L.zb[c] = zb;
          L.s2[c] = sv;
          L.nt[c] = nt;
          if (a.qsk) a.qsk[(long)row * a.C + c] = qs;
        }
      }
    }
  }
}

template <int NS, int TPL, int KR, int W>
__global__ void __launch_bounds__(64 * W) topk_gate2_fill_kernel(TopkArgs t, GateArgs a, int32_t* sel,
                                                                  float* __restrict__ quota, double budget) {
  __shared__ Gate2Lds L;
  constexpr int kThr = 64 * W;
  const int row = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2
  const int tid = threadIdx.x;
  if (tid < 64)
    oa_sel::topk_reg_row<TPL, KR, true>(t.H, t.h_stride, t.TM, t.tm_stride, t.ntiles, sel,
                                        a.sel_stride, *t.n_dev, t.ns, t.nl, t.k_top, t.rs, row, tid,
                                        L.f.sel);
  else
    pooled_batches<W>(a, row, L);
  if (tid == 0) L.f.nhit = 0;
  __syncthreads();
  for (int c = tid; c < a.C; c += kThr) {
    L.f.score[c] = gate_score(L.zb[c], L.s2[c], L.nt[c]);
    L.f.nt[c] = L.nt[c];
    L.f.selmask[c] = 0ull;
  }
  __syncthreads();
  fix_finish<NS, kThr>(a, row, L.f, quota + (long)row * a.C, budget);
  // the rows' pooled values of the clusters no selected token touched (fix_finish wrote the others)
  for (int c = tid; c < a.C; c += kThr) {
    if (L.f.selmask[c]) continue;
    a.score[(long)row * a.out_stride + c] = L.f.score[c];
    a.n_t[(long)row * a.out_stride + c] = L.f.nt[c];
  }
}

int launch_fill(const float* score, const float* n_t, int rows, int C, int budget, float* quota,
                hipStream_t s) {
  const int ns = (C + 63) / 64;
  if (ns == 1)
    hipLaunchKernelGGL(waterfill_kernel<1>, dim3(rows), dim3(64), 0, s, score, n_t, (long)C, quota,
                       (long)C, C, (double)budget);
  else if (ns == 2)
    hipLaunchKernelGGL(waterfill_kernel<2>, dim3(rows), dim3(64), 0, s, score, n_t, (long)C, quota,
                       (long)C, C, (double)budget);
  else if (ns == 3)
    hipLaunchKernelGGL(waterfill_kernel<3>, dim3(rows), dim3(64), 0, s, score, n_t, (long)C, quota,
                       (long)C, C, (double)budget);
  else
    hipLaunchKernelGGL(waterfill_kernel<4>, dim3(rows), dim3(64), 0, s, score, n_t, (long)C, quota,
                       (long)C, C, (double)budget);
  return OA_LAUNCH_STATUS();
}

}  // namespace

extern "C" int oa_errorgate(const void* q, long q_stride, const void* K, long k_stride_b,
                            long k_stride_s, int rows, int kv_rows, int head_dim,
                            const int32_t* asg, long asg_stride, const int32_t* sel, long sel_stride,
                            int n_sel, const float* Sk, const float* Sk2, const float* nb, int C,
                            float sm_scale, float sm_scale_sq, float* score, float* n_t,
                            void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows % kv_rows != 0 || n_sel < 0 || n_sel > kMaxSel ||
      C <= 0 || C > kMaxC || k_stride_b % 8 || k_stride_s % 8 ||
      (reinterpret_cast<uintptr_t>(K) & 15))
    return OA_EINVAL;
  GateArgs a;
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.k_sb = k_stride_b; a.k_ss = k_stride_s; a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.Sk = Sk; a.Sk2 = Sk2; a.st_stride_r = (long)C * OA_D;
  a.nb = nb; a.nb_stride = C;
  a.score = score; a.n_t = n_t; a.out_stride = C; a.qsk = nullptr;
  a.C = C; a.sc = sm_scale;
  a.sc2 = sm_scale_sq;
  hipLaunchKernelGGL(errorgate_kernel, dim3(rows), dim3(kGateThreads),
                     sizeof(float) * (size_t)n_sel * OA_D, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_gate_fill(const void* q, long q_stride, const void* K, long k_stride_b,
                            long k_stride_s, int rows, int kv_rows, int head_dim,
                            const int32_t* asg, long asg_stride, const int32_t* sel, long sel_stride,
                            int n_sel, const float* Sk, const float* Sk2, const float* nb, int C,
                            float sm_scale, float sm_scale_sq, int budget, float* score, float* n_t,
                            float* quota, float* qsk, void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows % kv_rows != 0 || n_sel < 0 || n_sel > kMaxSel ||
      C <= 0 || C > kMaxC || budget < 0 || k_stride_b % 8 || k_stride_s % 8 ||
      (reinterpret_cast<uintptr_t>(K) & 15))
    return OA_EINVAL;
  GateArgs a;
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.k_sb = k_stride_b; a.k_ss = k_stride_s; a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.Sk = Sk; a.Sk2 = Sk2; a.st_stride_r = (long)C * OA_D;
  a.nb = nb; a.nb_stride = C;
  a.score = score; a.n_t = n_t; a.out_stride = C; a.qsk = qsk;
  a.C = C; a.sc = sm_scale; a.sc2 = sm_scale_sq;
  const size_t lds = sizeof(float) * (size_t)n_sel * OA_D;
  if (rows < kFuseRows) {
    const int ns = (C + 63) / 64;
    const dim3 g(rows), blk(kGateThreads);
    hipStream_t s = (hipStream_t)stream;
    if (ns == 1) hipLaunchKernelGGL(gate_fill_kernel<1>, g, blk, lds, s, a, quota, (double)budget);
    else if (ns == 2) hipLaunchKernelGGL(gate_fill_kernel<2>, g, blk, lds, s, a, quota, (double)budget);
    else if (ns == 3) hipLaunchKernelGGL(gate_fill_kernel<3>, g, blk, lds, s, a, quota, (double)budget);
    else hipLaunchKernelGGL(gate_fill_kernel<4>, g, blk, lds, s, a, quota, (double)budget);
    return OA_LAUNCH_STATUS();
  }
  // the gate is wide and short, the fill one serial chain per row: as two launches every row of
  // each is resident at once instead of the fill holding the gate's workgroup slots
  hipLaunchKernelGGL(errorgate_kernel, dim3(rows), dim3(kGateThreads), lds, (hipStream_t)stream, a);
  const int st = OA_LAUNCH_STATUS();
  if (st) return st;
  return launch_fill(score, n_t, rows, C, budget, quota, (hipStream_t)stream);
}

extern "C" int oa_topk_gate_fill(uint16_t* H, long h_stride, const float* TM, long tm_stride,
                                 int ntiles, const int* n_dev, int ns, int nl, int k_top,
                                 const int8_t* codes, int Lmax, const int8_t* limbs,
                                 const int* fexp, const void* q, long q_stride, const void* K,
                                 long k_stride_b, long k_stride_s, int rows, int kv_rows,
                                 int head_dim, const int32_t* asg, long asg_stride, int32_t* sel,
                                 long sel_stride, const float* Sk, const float* Sk2,
                                 const float* nb, int C, float sm_scale, float sm_scale_sq,
                                 int budget, float* score, float* n_t, float* quota, float* qsk,
                                 void* stream) {
  const int n_sel = ns + nl + k_top;
  const int tpl = (ntiles + 63) / 64;
  const int reg = (k_top <= 9 && tpl <= 9) ? 1 : (k_top <= 16 && tpl <= 16) ? 2 : (k_top <= 16 && tpl <= 32) ? 3 : 0;
  // one launch needs the register top-k; at kFuseRows rows or more also a single cluster slot per
  // lane (C <= 64): the fill's slots take 130-214 VGPRs at C = 65..256, which would leave half of
  // a B = 32 batch's rows waiting for a workgroup slot (measured slower than two launches)
  if (!reg || (rows >= kFuseRows && C > 64)) {
    // two launches: the top-k the row needs, then the gate and fill
    int st = oa_topk_select_heads(H, h_stride, TM, tm_stride, rows, ntiles, sel, sel_stride, n_dev,
                                  ns, nl, k_top, codes, kv_rows, Lmax, limbs, fexp, stream);
    if (st) return st;
    return oa_gate_fill(q, q_stride, K, k_stride_b, k_stride_s, rows, kv_rows, head_dim, asg,
                        asg_stride, sel, sel_stride, n_sel, Sk, Sk2, nb, C, sm_scale, sm_scale_sq,
                        budget, score, n_t, quota, qsk, stream);
  }
  // the checks of both launches it replaces
  if (!H || !codes || !limbs || !fexp || !q || !K || !asg || (!sel && n_sel > 0) || !Sk || !Sk2 ||
      !nb || !score || !n_t || !quota || kv_rows <= 0 || rows != kv_rows * oa_sel::GQ ||
      Lmax <= 0 || (reinterpret_cast<uintptr_t>(codes) & 15) ||
      (reinterpret_cast<uintptr_t>(limbs) & 3) || ntiles <= 0 || k_top < 0 || k_top > ntiles ||
      ns < 0 || nl < 0 || ns > 64 || nl > 64 || sel_stride < n_sel || head_dim != OA_D ||
      n_sel > kMaxSel || C <= 0 || C > kMaxC || budget < 0 || k_stride_b % 8 || k_stride_s % 8 ||
      (reinterpret_cast<uintptr_t>(K) & 15))
    return OA_EINVAL;
  TopkArgs t;
  t.H = H; t.h_stride = h_stride; t.TM = TM; t.tm_stride = tm_stride; t.ntiles = ntiles;
  t.n_dev = n_dev; t.ns = ns; t.nl = nl; t.k_top = k_top;
  t.rs = oa_sel::Rescore{codes, (long)Lmax, limbs, fexp};
  GateArgs a{};
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.k_sb = k_stride_b; a.k_ss = k_stride_s; a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.Sk = Sk; a.Sk2 = Sk2; a.st_stride_r = (long)C * OA_D;
  a.nb = nb; a.nb_stride = C;
  a.score = score; a.n_t = n_t; a.out_stride = C; a.qsk = qsk;
  a.C = C; a.sc = sm_scale; a.sc2 = sm_scale_sq;
  const size_t lds = sizeof(float) * (size_t)n_sel * OA_D;
  const int nsl = (C + 63) / 64;
  hipStream_t s = (hipStream_t)stream;
  const double bd = (double)budget;
  // waves per row: every row stays resident (4 at B = 32); with few rows, enough waves that each
  // takes one batch of kPoolBatch clusters (16 up to 64 rows, 8 up to kFuseRows)
  const int wv = rows <= 64 ? 16 : rows < kFuseRows ? 8 : 4;
  const dim3 g(rows);
#define OA_TG2(NS, T, KK)                                                                       \
  do {                                                                                          \
    if (wv == 16)                                                                               \
      hipLaunchKernelGGL((topk_gate2_fill_kernel<NS, T, KK, 16>), g, dim3(1024), lds, s, t, a, sel, quota, bd); \
    else if (wv == 8)                                                                           \
      hipLaunchKernelGGL((topk_gate2_fill_kernel<NS, T, KK, 8>), g, dim3(512), lds, s, t, a, sel, quota, bd); \
    else                                                                                        \
      hipLaunchKernelGGL((topk_gate2_fill_kernel<NS, T, KK, 4>), g, dim3(256), lds, s, t, a, sel, quota, bd); \
  } while (0)
#define OA_TG2_NS(NS)                                                                           \
  do {                                                                                          \
    if (reg == 1) OA_TG2(NS, 9, 9);                                                             \
    else if (reg == 2) OA_TG2(NS, 16, 16);                                                      \
    else OA_TG2(NS, 32, 16);                                                                    \
  } while (0)
  if (nsl == 1) OA_TG2_NS(1);
  else if (nsl == 2) OA_TG2_NS(2);
  else if (nsl == 3) OA_TG2_NS(3);
  else OA_TG2_NS(4);
#undef OA_TG2_NS
#undef OA_TG2
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_waterfill(const float* score, const float* n_t, int rows, int C, int budget,
                            float* quota, void* stream) {
  if (rows <= 0 || C <= 0 || C > kMaxC || budget < 0) return OA_EINVAL;
  return launch_fill(score, n_t, rows, C, budget, quota, (hipStream_t)stream);
}

extern "C" int oa_topk_fix_fill(uint16_t* H, long h_stride, const float* TM, long tm_stride,
                                int ntiles, const int* n_dev, int ns, int nl, int k_top,
                                const int8_t* codes, int Lmax, const int8_t* limbs, const int* fexp,
                                const void* q, long q_stride, const void* K, long k_stride_b,
                                long k_stride_s, int rows, int kv_rows, int head_dim,
                                const int32_t* asg, long asg_stride, int32_t* sel, long sel_stride,
                                const float* Sk, const float* Sk2, const float* nb, int C,
                                float sm_scale, float sm_scale_sq, int budget, float* score,
                                float* n_t, float* quota, void* stream) {
  const int n_sel = ns + nl + k_top;
  if (!H || !codes || !limbs || !fexp || !q || !K || !asg || (!sel && n_sel > 0) || !Sk || !Sk2 || !nb || !score ||
      !n_t || !quota || kv_rows <= 0 || rows != kv_rows * oa_sel::GQ || Lmax <= 0 ||
      (reinterpret_cast<uintptr_t>(codes) & 15) || (reinterpret_cast<uintptr_t>(limbs) & 3) ||
      ntiles <= 0 || k_top < 0 || k_top > ntiles || ns < 0 || nl < 0 || ns > 64 || nl > 64 ||
      sel_stride < n_sel || head_dim != OA_D || n_sel > kMaxSel || C <= 0 || C > kMaxC ||
      budget < 0 || k_stride_b % 8 || k_stride_s % 8 || (reinterpret_cast<uintptr_t>(K) & 15))
    return OA_EINVAL;
  GateArgs a{};
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.k_sb = k_stride_b; a.k_ss = k_stride_s; a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.Sk = Sk; a.Sk2 = Sk2; a.st_stride_r = (long)C * OA_D;
  a.nb = nb; a.nb_stride = C;
  a.score = score; a.n_t = n_t; a.out_stride = C; a.qsk = nullptr;
  a.C = C; a.sc = sm_scale; a.sc2 = sm_scale_sq;
  const size_t lds = sizeof(float) * (size_t)n_sel * OA_D;
  const int nsl = (C + 63) / 64;
  const int tpl = (ntiles + 63) / 64;
  const dim3 g(rows), blk(kFixThreads);
  hipStream_t s = (hipStream_t)stream;
  const double bd = (double)budget;
  const int reg = (k_top <= 9 && tpl <= 9) ? 1 : (k_top <= 16 && tpl <= 16) ? 2 : (k_top <= 16 && tpl <= 32) ? 3 : 0;
  if (!reg) {
    // the radix-select top-k the row needs, then the correction and the fill
    const int st = oa_topk_select_heads(H, h_stride, TM, tm_stride, rows, ntiles, sel, sel_stride,
                                        n_dev, ns, nl, k_top, codes, kv_rows, Lmax, limbs, fexp, stream);
    if (st) return st;
    if (nsl == 1) hipLaunchKernelGGL(fix_fill_kernel<1>, g, blk, lds, s, a, quota, bd);
    else if (nsl == 2) hipLaunchKernelGGL(fix_fill_kernel<2>, g, blk, lds, s, a, quota, bd);
    else if (nsl == 3) hipLaunchKernelGGL(fix_fill_kernel<3>, g, blk, lds, s, a, quota, bd);
    else hipLaunchKernelGGL(fix_fill_kernel<4>, g, blk, lds, s, a, quota, bd);
    return OA_LAUNCH_STATUS();
  }
  TopkArgs t;
  t.H = H; t.h_stride = h_stride; t.TM = TM; t.tm_stride = tm_stride; t.ntiles = ntiles;
  t.n_dev = n_dev; t.ns = ns; t.nl = nl; t.k_top = k_top;
  t.rs = oa_sel::Rescore{codes, (long)Lmax, limbs, fexp};
#define OA_TFF(NS)                                                                              \
  do {                                                                                          \
    if (reg == 1)                                                                               \
      hipLaunchKernelGGL((topk_fix_fill_kernel<NS, 9, 9>), g, blk, lds, s, t, a, sel, quota, bd); \
    else if (reg == 2)                                                                          \
      hipLaunchKernelGGL((topk_fix_fill_kernel<NS, 16, 16>), g, blk, lds, s, t, a, sel, quota, bd); \
    else                                                                                        \
      hipLaunchKernelGGL((topk_fix_fill_kernel<NS, 32, 16>), g, blk, lds, s, t, a, sel, quota, bd); \
  } while (0)
  if (nsl == 1) OA_TFF(1);
  else if (nsl == 2) OA_TFF(2);
  else if (nsl == 3) OA_TFF(3);
  else OA_TFF(4);
#undef OA_TFF
  return OA_LAUNCH_STATUS();
}
