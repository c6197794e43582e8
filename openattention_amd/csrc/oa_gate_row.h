// ErrorGate (wl1 cluster score) arithmetic of one cluster, shared by the ErrorGate launches
// (oa_gate.hip) and the scan launch that computes the pooled part (oa_select.hip).
//
// Reference semantics: tail statistics of a QGC cluster = the cached pooled sums minus the
// selected tokens (methods_eager.py:612-627, ours_fused.py:122-154), moments as
// UTAMultiBinAttention._moments_from_key_stats (multibin.py:605-644) with s2 = 0 for clusters of
// fewer than two tail tokens (multibin.py:734-738), and the wl1 score
// zbar + log n + s2/2 + log max(erf(sqrt(s2)/sqrt2), 1e-30) (multibin.py:2370-2389).
#pragma once
#include "oa_common.h"
#include "oa_detmath.h"

namespace oa_gate {

struct GateArgs {
  const uint16_t* q; long q_stride;
  const uint16_t* K; long k_sb; long k_ss; int G;
  const int32_t* asg; long asg_stride;
  const int32_t* sel; long sel_stride; int n_sel;
  const float* Sk; const float* Sk2; long st_stride_r;   // (R, C, D): row stride in floats
  const float* nb; long nb_stride;
  float* score; float* n_t; long out_stride;
  float* qsk;                                         // optional: q . Sk_c of every cluster
  int C; float sc; float sc2;
};

// x / den for den >= 1, given r = 1 / den correctly rounded: q = RN(x r) lies within one ulp of
// x / den and r within half an ulp of 1 / den, so fma(fma(-q, den, x), r, q) is x / den correctly
// rounded (Markstein's theorem; the residual fma(-q, den, x) is exact) as long as nothing
// underflows or overflows.  Zeros (whose sign the residual step loses), tiny, huge and
// non-finite x take the division itself.
__device__ __forceinline__ bool div_fast_ok(float x) {
  const float ax = fabsf(x);
  return ax >= 0x1p-100f && ax <= 0x1p100f;
}
__device__ __forceinline__ float div_den(float x, float den, float r) {
  const float q = x * r;
  return fmaf(fmaf(-q, den, x), r, q);
}

// the two wave-wide parts of one cluster's score (lane holds dims lane and lane+64): the tail
// sums minus the selected tokens, then zbar = sc q.kbar and the raw sc2 (q*q).var
__device__ __forceinline__ void gate_dots(const GateArgs& a, float sk_lo, float sk_hi,
                                          float s2_lo, float s2_hi, float nt, float q_lo,
                                          float q_hi, float qq_lo, float qq_hi,
                                          unsigned long long selmask, const float* s_k, int lane,
                                          float* zbar_out, float* s2_out, float* nt_out,
                                          float* qsk_out) {
  // q . Sk of the pooled sums (before the selected tokens leave them), for the residual pass
  *qsk_out = oa::dot128_canon(q_lo, sk_lo, q_hi, sk_hi);
  // the cluster's selected tokens, in selection order (bit i = selected token i)
  while (selmask) {
    const int i = __ffsll((long long)selmask) - 1;
    selmask &= selmask - 1ull;
    {
      const float k_lo = s_k[i * OA_D + lane], k_hi = s_k[i * OA_D + lane + 64];
      sk_lo = sk_lo - k_lo;
      sk_hi = sk_hi - k_hi;
      s2_lo = s2_lo - k_lo * k_lo;
      s2_hi = s2_hi - k_hi * k_hi;
      nt = nt - 1.0f;
    }
  }
  const float den = fmaxf(nt, 1.0f);
  float kb_lo, kb_hi, ks_lo, ks_hi;
  if (__all(div_fast_ok(sk_lo) && div_fast_ok(sk_hi) && div_fast_ok(s2_lo) && div_fast_ok(s2_hi))) {
    const float r = 1.0f / den;          // uniform: one division per cluster
    kb_lo = div_den(sk_lo, den, r); kb_hi = div_den(sk_hi, den, r);
    ks_lo = div_den(s2_lo, den, r); ks_hi = div_den(s2_hi, den, r);
  } else {
    kb_lo = sk_lo / den; kb_hi = sk_hi / den;
    ks_lo = s2_lo / den; ks_hi = s2_hi / den;
  }
  const float v_lo = fmaxf(ks_lo - kb_lo * kb_lo, 0.f);
  const float v_hi = fmaxf(ks_hi - kb_hi * kb_hi, 0.f);
  *zbar_out = a.sc * oa::dot128_canon(q_lo, kb_lo, q_hi, kb_hi);
  *s2_out = a.sc2 * oa::dot128_canon(qq_lo, v_lo, qq_hi, v_hi);
  *nt_out = nt;
}

// the scalar tail of one cluster's wl1 score
__device__ __forceinline__ float gate_score(float zbar, float s2, float nt) {
  if (!(nt >= 2.0f)) s2 = 0.f;
  const float s2c = fmaxf(s2, 0.f);
  const float sig = sqrtf(s2c);
  const float er = oa::det_erff(sig * 0.70710677f);
  const float log_d = 0.5f * s2c + oa::det_logf(fmaxf(er, 1e-30f));
  return (zbar + oa::det_logf(fmaxf(nt, 1.0f))) + log_d;
}

// The pooled part of the ErrorGate of one row: clusters [c0, c0 + kPoolClusters) as if none of
// them held a selected token (the tail sums are the pooled ones), by one 256-thread block.
// Each wave takes kPoolClusters / 4 clusters with all of their loads in flight, then one
// thread per cluster forms the wl1 score.  Writes score, n_t (= n_c) and, when asked, q . Sk_c.
// For a cluster that holds no selected token this is the final ErrorGate output bit for bit
// (gate_dots with an empty mask is the same arithmetic); the others are done again once the
// selection is known.
constexpr int kPoolClusters = 16;
constexpr int kPoolThreads = 256;
__device__ __forceinline__ void gate_pooled_unit(const GateArgs& a, int row, int c0, float* s_zb,
                                                 float* s_s2, float* s_nt) {
  constexpr int kPer = kPoolClusters / (kPoolThreads / 64);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  float sk[kPer][2], s2[kPer][2], nbv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = min(c0 + wave + 4 * i, a.C - 1);
    const long base = (long)row * a.st_stride_r + (long)c * OA_D;
    sk[i][0] = a.Sk[base + lane];
    sk[i][1] = a.Sk[base + lane + 64];
    s2[i][0] = a.Sk2[base + lane];
    s2[i][1] = a.Sk2[base + lane + 64];
    nbv[i] = a.nb[(long)row * a.nb_stride + c];
  }
  const float q_lo = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane]);
  const float q_hi = oa::bf16_to_f32(a.q[(long)row * a.q_stride + lane + 64]);
  const float qq_lo = q_lo * q_lo, qq_hi = q_hi * q_hi;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = wave + 4 * i;                 // the cluster's slot in the unit
    const int c = c0 + j;
    if (c < a.C) {
      float zb, sv, nt, qs;
      gate_dots(a, sk[i][0], sk[i][1], s2[i][0], s2[i][1], nbv[i], q_lo, q_hi, qq_lo, qq_hi, 0ull,
                nullptr, lane, &zb, &sv, &nt, &qs);
      if (lane == 0) {
        s_zb[j] = zb;
        s_s2[j] = sv;
        s_nt[j] = nt;
        if (a.qsk) a.qsk[(long)row * a.C + c] = qs;
      }
    }
  }
  __syncthreads();
  if (tid < kPoolClusters && c0 + tid < a.C) {
    const long o = (long)row * a.out_stride + c0 + tid;
    a.score[o] = gate_score(s_zb[tid], s_s2[tid], s_nt[tid]);
    a.n_t[o] = s_nt[tid];
  }
}

}  // namespace oa_gate
