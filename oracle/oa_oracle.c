/*
 * CPU restatement of the OpenAttention sparse decode step -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the gfx950 kernels of openattention_amd.  It is compiled by
 * oracle/build.py with gcc (-O2 -ffp-contract=off) and called from tests/, from
 * __graft_entry__.smoke() and from the cpu_baseline leg of bench.py.  Nothing in the product
 * path loads it.
 *
 * Every function restates the reference algorithm (file:line cited at each function) with the
 * arithmetic order this project defines for reproducibility (see the "canonical" helpers):
 * the decision path (codes, cluster ids, QGS scores, top-k, ErrorGate scores, quotas, top-q)
 * is replayed bit for bit; the floating outputs (residual proxies, attention output) are
 * computed in fp64 and compared with a tolerance.
 *
 * Layouts (row-major, matching the device buffers):
 *   K, V      (BH, Lmax, D)  bf16 as uint16          codes (BH, Lmax, RQ) int8
 *   U         (BH, D, RQ)    f32                     scale (BH, RQ) f32
 *   W         (R, D, RC)     bf16                    colmean (R, RC), cent (R, C, RC) f32
 *   asg       (R, Lmax)      i32                     nb (R, C) f32
 *   Sk,Sk2,Sv (R, C, D)      f32                     q (R, D) bf16
 * with R = BH * G query-head rows, row r reading KV row r / G.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define D 128
#define RQ 32
#define RC 16

/* ------------------------------------------------------------------ scalar helpers */
static float bf2f(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf_round(float f) { return bf2f(f2bf(f)); }

static uint32_t fkey(float s) {
  uint32_t b;
  memcpy(&b, &s, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* fixed-order 128-term dot product: p_l = fma(a[l+64], b[l+64], a[l]*b[l]), then the xor
 * butterfly over 64 partials (m = 1, 2, ..., 32).  Same order as the device helper. */
static float dot128_canon(const float* a, const float* b) {
  float p[64], t[64];
  for (int l = 0; l < 64; ++l) p[l] = fmaf(a[l + 64], b[l + 64], a[l] * b[l]);
  for (int m = 1; m <= 32; m <<= 1) {
    for (int l = 0; l < 64; ++l) t[l] = p[l] + p[l ^ m];
    memcpy(p, t, sizeof p);
  }
  return p[0];
}

/* butterfly sum of 64 double partials (m = 1, 2, ..., 32) */
static double bfly64(const double* x) {
  double p[64], t[64];
  memcpy(p, x, sizeof p);
  for (int m = 1; m <= 32; m <<= 1) {
    for (int l = 0; l < 64; ++l) t[l] = p[l] + p[l ^ m];
    memcpy(p, t, sizeof p);
  }
  return p[0];
}

/* cluster c lives in slot (c % 64, c / 64): lane partial = x_l (+ x_{l+64} (+ ...)) */
static double canon_sum_c(const double* x, int C) {
  double part[64];
  for (int l = 0; l < 64; ++l) {
    double p = 0.0;
    int first = 1;
    for (int j = 0; j < 4; ++j) {
      int c = l + 64 * j;
      if (c < C) {
        p = first ? x[c] : p + x[c];
        first = 0;
      }
    }
    part[l] = p;
  }
  return bfly64(part);
}

/* ------------------------------------------------------------------ deterministic libm
 * Same published algorithms, constants and term counts as the device header:
 * exp  Cody-Waite (fdlibm ln2 split) + Taylor to r^13; log  2 atanh((m-1)/(m+1)) series to
 * f^23; erf  (2/sqrt(pi)) x sum_n (-1)^n x^(2n) / (n!(2n+1)), 72 terms in Horner form for
 * |x| < 4 (coefficients rounded to double), +-1 beyond. */
double oa_det_exp(double x) {
  if (x != x) return x;
  if (x > 709.782712893384) return INFINITY;
  if (x < -745.2) return 0.0;
  const double k = rint(x * 0x1.71547652b82fep+0);
  double r = fma(-k, 0x1.62e42fee00000p-1, x);
  r = fma(-k, 0x1.a39ef35793c76p-33, r);
  static const double c[] = {0x1.6124613a86d09p-33, 0x1.1eed8eff8d898p-29, 0x1.ae64567f544e4p-26,
                             0x1.27e4fb7789f5cp-22, 0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-16,
                             0x1.a01a01a01a01ap-13, 0x1.6c16c16c16c17p-10, 0x1.1111111111111p-7,
                             0x1.5555555555555p-5,  0x1.5555555555555p-3,  0.5, 1.0, 1.0};
  double p = c[0];
  for (int i = 1; i < 14; ++i) p = fma(p, r, c[i]);
  return ldexp(p, (int)k);
}

double oa_det_log(double x) {
  if (x != x) return x;
  if (x < 0.0) return NAN;
  if (x == 0.0) return -INFINITY;
  if (isinf(x)) return x;
  int e;
  double m = frexp(x, &e);
  if (m < 0x1.6a09e667f3bcdp-1) {
    m = m * 2.0;
    e = e - 1;
  }
  const double f = (m - 1.0) / (m + 1.0);
  const double s = f * f;
  double p = 1.0 / 23.0;
  for (int k = 21; k >= 1; k -= 2) p = fma(p, s, 1.0 / (double)k);
  const double lm = 2.0 * f * p;
  const double de = (double)e;
  return fma(de, 0x1.62e42fee00000p-1, fma(de, 0x1.a39ef35793c76p-33, lm));
}

float oa_det_logf(float x) { return (float)oa_det_log((double)x); }

static const double kErfC[72] = {
    0x1.0000000000000p+0, -0x1.5555555555555p-2, 0x1.999999999999ap-4,
    -0x1.8618618618618p-6, 0x1.2f684bda12f68p-8, -0x1.8d3018d3018d3p-11,
    0x1.c01c01c01c01cp-14, -0x1.bbd779334ef0bp-17, 0x1.87a00187a0018p-20,
    -0x1.3777c55568ccdp-23, 0x1.c2e3054870b38p-27, -0x1.2b67310aa9f3ap-30,
    0x1.6f448e13e85e1p-34, -0x1.a289ee7e40f74p-38, 0x1.bd577e658d020p-42,
    -0x1.bc6250fb14231p-46, 0x1.a173a167fba4dp-50, -0x1.7271cbe5863ecp-54,
    0x1.377c2110f2083p-58, -0x1.f1b4073b34a68p-63, 0x1.7abd72258fb6ep-67,
    -0x1.13246abce1bddp-71, 0x1.7e6b81382cd42p-76, -0x1.fd6bebd65107ap-81,
    0x1.45c0a838efe59p-85, -0x1.909c9de3a31c5p-90, 0x1.da7460554e5dbp-95,
    -0x1.0eef30fa10d2cp-99, 0x1.2ac65385f79acp-104, -0x1.3e81bb5701ac5p-109,
    0x1.4899fcdef0a8dp-114, -0x1.486eea20c2656p-119, 0x1.3e53defc4e233p-124,
    -0x1.2b778acc3dedfp-129, 0x1.11ae81077a49ep-134, -0x1.e6597092ccbf0p-140,
    0x1.a47767f2a3c32p-145, -0x1.61f30bc3acd1ap-150, 0x1.22521d98f98a9p-155,
    -0x1.d05cc9e3507c9p-161, 0x1.6a513f56f8a2fp-166, -0x1.13f85fc9e143ep-171,
    0x1.9aa19d4d16643p-177, -0x1.2a8fa59ffec31p-182, 0x1.a8830736a5123p-188,
    -0x1.273d8edcec957p-193, 0x1.91ef82b367a95p-199, -0x1.0be5a4cd94283p-204,
    0x1.5dd4c9219115ap-210, -0x1.bfb10e0f68c50p-216, 0x1.18d952ef00889p-221,
    -0x1.59982b2e94840p-227, 0x1.a13ec00b39f6fp-233, -0x1.ee6cefaa5a158p-239,
    0x1.1f9dec94da5f8p-244, -0x1.48a6b3820b441p-250, 0x1.70f41ac13e2a1p-256,
    -0x1.970f1cb2ad53fp-262, 0x1.b97d90d3e603bp-268, -0x1.d6db2a7c68dcbp-274,
    0x1.edf1e6e4658a9p-280, -0x1.fdcf88bbf71dbp-286, 0x1.02eb04e5f82f5p-291,
    -0x1.02e2bc1b5790ep-297, 0x1.fdbe706576d5dp-304, -0x1.ee3d33862f55bp-310,
    0x1.d80e20102c46ep-316, -0x1.bc3cf47bca3afp-322, 0x1.9c00b17fe33c8p-328,
    -0x1.78a61f51a767fp-334, 0x1.537ae8ecb0688p-340, -0x1.2dbafa5779b80p-346,
};

float oa_det_erff(float xf) {
  const double x = (double)xf;
  if (x != x) return xf;
  const double ax = x < 0.0 ? -x : x;
  if (ax >= 4.0) return x < 0.0 ? -1.0f : 1.0f;
  const double x2 = ax * ax;
  double s = kErfC[71];
  for (int n = 70; n >= 0; --n) s = fma(s, x2, kErfC[n]);
  const float rf = (float)((ax * s) * 0x1.20dd750429b6dp+0);
  return x < 0.0 ? -rf : rf;
}

/* ------------------------------------------------------------------ QGS projection
 * StaticTopKMasker._scores (static_top_k.py:203-213): zq = (q U) * scale (per KV-head U and
 * scale shared by its G query heads), then the fixed-point form used for exact scores:
 * F = 30 - e with max|zq| = m 2^e (m in [0.5,1)), Z_r = rint(zq_r 2^F). */
void oa_ref_qgs_prep(const uint16_t* q, const float* U, const float* scale, int R, int G, float* zq,
                     int* fexp, int32_t* Z) {
  float qa[D], ua[D];
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    for (int d = 0; d < D; ++d) qa[d] = bf2f(q[(long)r * D + d]);
    float emax = 0.f;
    for (int j = 0; j < RQ; ++j) {
      for (int d = 0; d < D; ++d) ua[d] = U[((long)kvr * D + d) * RQ + j];
      const float z = dot128_canon(qa, ua) * scale[(long)kvr * RQ + j];
      zq[(long)r * RQ + j] = z;
      if (fabsf(z) > emax) emax = fabsf(z);
    }
    int F = 0;
    const int usable = emax > 0.f && isfinite(emax);
    if (usable) {
      int ex;
      (void)frexpf(emax, &ex);
      F = 30 - ex;
    }
    fexp[r] = F;
    for (int j = 0; j < RQ; ++j)
      Z[(long)r * RQ + j] = usable ? (int32_t)rint(ldexp((double)zq[(long)r * RQ + j], F)) : 0;
  }
}

/* score_i = fp32( sum_r Z_r code_{i,r} * 2^-F ), exact integer sum, one rounding.
 * Positions < ns or >= n - nl (sink, local, not yet written) get -inf. */
void oa_ref_qgs_scores(const int8_t* codes, int Lmax, const int32_t* Z, const int* fexp, int R, int G,
                       int n, int ns, int nl, int ncols, float* S) {
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    const double inv = ldexp(1.0, -fexp[r]);
    const int32_t* z = Z + (long)r * RQ;
    for (int i = 0; i < ncols; ++i) {
      float sc;
      if (i < ns || i >= n - nl || i >= Lmax) {
        sc = -INFINITY;
      } else {
        const int8_t* c = codes + ((long)kvr * Lmax + i) * RQ;
        int64_t s = 0;
        for (int j = 0; j < RQ; ++j) s += (int64_t)z[j] * (int64_t)c[j];
        sc = (float)((double)s * inv);
      }
      S[(long)r * ncols + i] = sc;
    }
  }
}

/* ------------------------------------------------------------------ top-k + sink/local
 * SinkMasker (basic_fixed.py:354-363), LocalMasker.update_core (basic_fixed.py:48-67) and
 * TopKMasker._get_topk_indices_from_inactive_positions (fixed/base.py:74-85): the k highest
 * scores among positions [ns, n - nl), ties to the lower position (the deployed rule,
 * graph_runner.py:127-151).  The masker sets the sink and local positions to -inf before its
 * torch.topk (fixed/base.py:80-81) and the deployed kernel keeps them, and positions past n, as
 * -inf candidates (graph_runner.py:133,145-151): a row with fewer than k live positions takes the
 * lowest-position -inf ones after every live one.  sel row = [0..ns) ++ [n-nl..n) ++ top in
 * rank order. */
static int cmp_desc_key(const void* a, const void* b) {
  const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

void oa_ref_topk_select(const float* S, int ncols, int R, int n, int ns, int nl, int k, int32_t* sel) {
  const int NS = ns + nl + k;
  if (k < 0 || k > 256 || k > ncols) abort();
  for (int r = 0; r < R; ++r) {
    int32_t* out = sel + (long)r * NS;
    for (int i = 0; i < ns; ++i) out[i] = i;
    for (int i = 0; i < nl; ++i) out[ns + i] = n - nl + i;
    /* partial selection over every position of the row: keep the best k with an insertion
     * buffer (distinct keys: the low word is ~position) */
    uint64_t best[256];
    int nb = 0;
    for (int i = 0; i < ncols; ++i) {
      const int live = i >= ns && i < n - nl;
      const uint64_t x = ((uint64_t)fkey(live ? S[(long)r * ncols + i] : -INFINITY) << 32) |
                         (uint64_t)(0xffffffffu - (uint32_t)i);
      if (nb < k) {
        int p = nb++;
        while (p > 0 && best[p - 1] < x) { best[p] = best[p - 1]; --p; }
        best[p] = x;
      } else if (k > 0 && x > best[k - 1]) {
        int p = k - 1;
        while (p > 0 && best[p - 1] < x) { best[p] = best[p - 1]; --p; }
        best[p] = x;
      }
    }
    for (int i = 0; i < k; ++i) out[ns + nl + i] = (int32_t)(0xffffffffu - (uint32_t)(best[i] & 0xffffffffu));
  }
}

/* ------------------------------------------------------------------ ErrorGate (wl1)
 * Tail statistics = pooled sums minus the selected tokens, subtracted in sel-list order
 * (methods_eager.py:612-627); moments as _moments_from_key_stats (multibin.py:605-644) with
 * s2 = 0 below two tail tokens (multibin.py:734-738); wl1 score (multibin.py:2370-2389):
 * score = (zbar + log max(n,1)) + (s2/2 + log max(erf(sqrt(s2) * 0.70710677), 1e-30)). */
void oa_ref_errorgate(const uint16_t* q, const uint16_t* K, int Lmax, const int32_t* asg,
                      const int32_t* sel, int n_sel, const float* Sk, const float* Sk2, const float* nb,
                      int R, int G, int C, float sc, float sc2, float* score, float* n_t) {
  float qa[D], qq[D], sk[D], s2[D], kb[D], var[D], kk[D];
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    for (int d = 0; d < D; ++d) {
      qa[d] = bf2f(q[(long)r * D + d]);
      qq[d] = qa[d] * qa[d];
    }
    for (int c = 0; c < C; ++c) {
      const long base = ((long)r * C + c) * D;
      for (int d = 0; d < D; ++d) { sk[d] = Sk[base + d]; s2[d] = Sk2[base + d]; }
      float nt = nb[(long)r * C + c];
      for (int i = 0; i < n_sel; ++i) {
        const int tok = sel[(long)r * n_sel + i];
        if (tok < 0 || asg[(long)r * Lmax + tok] != c) continue;
        for (int d = 0; d < D; ++d) {
          kk[d] = bf2f(K[((long)kvr * Lmax + tok) * D + d]);
          sk[d] = sk[d] - kk[d];
          s2[d] = s2[d] - kk[d] * kk[d];
        }
        nt = nt - 1.0f;
      }
      const float den = fmaxf(nt, 1.0f);
      for (int d = 0; d < D; ++d) {
        kb[d] = sk[d] / den;
        const float ks = s2[d] / den;
        var[d] = fmaxf(ks - kb[d] * kb[d], 0.f);
      }
      const float zbar = sc * dot128_canon(qa, kb);
      float sv = sc2 * dot128_canon(qq, var);
      if (!(nt >= 2.0f)) sv = 0.f;
      const float s2c = fmaxf(sv, 0.f);
      const float sig = sqrtf(s2c);
      const float er = oa_det_erff(sig * 0.70710677f);
      const float log_d = 0.5f * s2c + oa_det_logf(fmaxf(er, 1e-30f));
      score[(long)r * C + c] = (zbar + oa_det_logf(fmaxf(nt, 1.0f))) + log_d;
      n_t[(long)r * C + c] = nt;
    }
  }
}

/* ------------------------------------------------------------------ water-filling
 * UTAMultiBinAttention._hier_quota_impl (multibin.py:1385-1422), gamma = 1, fp64, 64
 * bisection steps; order = live scores descending (multibin.py:2471-2472), ties to the
 * lower cluster id.  Sums use the canonical cluster order of the device kernel. */
void oa_ref_waterfill(const float* score, const float* n_t, int R, int C, double B, float* quota) {
  double sv[256], w[256], cap[256], qv[256], part[256];
  int ok[256];
  for (int r = 0; r < R; ++r) {
    double smax = -INFINITY;
    for (int c = 0; c < C; ++c) {
      const float nt = n_t[(long)r * C + c];
      ok[c] = nt > 1.0f;
      sv[c] = ok[c] ? (double)score[(long)r * C + c] : -INFINITY;
      cap[c] = ok[c] ? (double)nt : 0.0;
      if (sv[c] > smax) smax = sv[c];
    }
    if (!isfinite(smax)) smax = 0.0;
    double rmax = 0.0;
    for (int c = 0; c < C; ++c) {
      w[c] = ok[c] ? oa_det_exp(sv[c] - smax) : 0.0;
      const double ratio = w[c] > 0.0 ? cap[c] / fmax(w[c], 1e-300) : 0.0;
      if (ratio > rmax) rmax = ratio;
    }
    const double tot = canon_sum_c(cap, C);
    double lo = -3.0 * 2.302585092994046;
    double hi = oa_det_log(fmax(rmax, 1e-3)) + 1.0;
    for (int it = 0; it < 64; ++it) {
      const double mid = 0.5 * (lo + hi);
      const double em = oa_det_exp(mid);
      for (int c = 0; c < C; ++c) part[c] = fmin(cap[c], em * w[c]);
      const double f = canon_sum_c(part, C);
      if (f > B) hi = mid; else lo = mid;
    }
    const double el = oa_det_exp(lo);
    for (int c = 0; c < C; ++c) {
      qv[c] = floor(fmin(cap[c], el * w[c]));
      if (tot <= B) qv[c] = cap[c];
    }
    const double qsum = canon_sum_c(qv, C);
    double rem = fmin(tot, B) - qsum;
    rem = rint(rem > 0.0 ? rem : 0.0);
    for (int c = 0; c < C; ++c) {
      double add = 0.0;
      if (qv[c] < cap[c]) {
        int rank = 0;
        for (int c2 = 0; c2 < C; ++c2) {
          if (!(qv[c2] < cap[c2])) continue;
          if (sv[c2] > sv[c] || (sv[c2] == sv[c] && c2 < c)) ++rank;
        }
        if ((double)rank < rem) add = 1.0;
      }
      quota[(long)r * C + c] = (float)(qv[c] + add);
    }
  }
}

/* ------------------------------------------------------------------ within-cluster top-q
 * Per-token rank within its bin by the selector score, trunc_keep = rank < quota
 * (multibin.py:2522-2558); ties to the lower position (ours_graph.py:93-135).  Members are
 * derived from asg over [0, n) minus the selected tokens -- independent of the device's CSR
 * and generated-token lists.  Segment layout: cluster c at [base_c, base_c + q_c), its chosen
 * members in position order.  Slots past sum q are -1. */
void oa_ref_topq(const float* S, int ncols, const int32_t* asg, int Lmax, const int32_t* sel, int n_sel,
                 const float* quota, int R, int C, int n, int E, int32_t* exp_idx) {
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(n > 0 ? n : 1));
  int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
  char* is_sel = (char*)malloc((size_t)(n > 0 ? n : 1));
  for (int r = 0; r < R; ++r) {
    int32_t* out = exp_idx + (long)r * E;
    for (int j = 0; j < E; ++j) out[j] = -1;
    memset(is_sel, 0, (size_t)n);
    for (int i = 0; i < n_sel; ++i) {
      const int t = sel[(long)r * n_sel + i];
      if (t >= 0 && t < n) is_sel[t] = 1;
    }
    int base = 0;
    for (int c = 0; c < C; ++c) {
      const int qc = (int)quota[(long)r * C + c];
      if (qc <= 0) continue;
      int m = 0;
      for (int i = 0; i < n; ++i) {
        if (is_sel[i] || asg[(long)r * Lmax + i] != c) continue;
        keys[m++] = ((uint64_t)fkey(S[(long)r * ncols + i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
      }
      qsort(keys, (size_t)m, sizeof(uint64_t), cmp_desc_key);
      /* the row holds E slots: a segment that would run past E keeps its best E - base members
       * (the reference never overflows, as its water-filling keeps sum q <= E) */
      int take = qc < m ? qc : m;
      if (take > E - base) take = E - base > 0 ? E - base : 0;
      /* the chosen members, listed in position order */
      for (int j = 0; j < take; ++j) tmp[j] = (int32_t)(0xffffffffu - (uint32_t)(keys[j] & 0xffffffffu));
      for (int a = 1; a < take; ++a) {
        int32_t x = tmp[a];
        int b = a - 1;
        while (b >= 0 && tmp[b] > x) { tmp[b + 1] = tmp[b]; --b; }
        tmp[b + 1] = x;
      }
      for (int j = 0; j < take; ++j) out[base + j] = tmp[j];
      base += qc;
    }
  }
  free(keys);
  free(tmp);
  free(is_sel);
}

/* ------------------------------------------------------------------ residual proxies
 * multibin.py:2598-2642 (residual_stats="full"); ours_fused.py:366-407.  fp64. */
void oa_ref_residual(const uint16_t* K, const uint16_t* V, int Lmax, const int32_t* asg, const int32_t* sel,
                     int n_sel, const int32_t* exp_idx, int E, const float* quota, const float* n_t,
                     const float* Sk, const float* Sv, int R, int G, int C, double* kbar_r, double* vbar_r,
                     double* log_n) {
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    for (int c = 0; c < C; ++c) {
      double* kb = kbar_r + ((long)r * C + c) * D;
      double* vb = vbar_r + ((long)r * C + c) * D;
      for (int d = 0; d < D; ++d) {
        kb[d] = Sk[((long)r * C + c) * D + d];
        vb[d] = Sv[((long)r * C + c) * D + d];
      }
    }
    for (int pass = 0; pass < 2; ++pass) {
      const int cnt = pass == 0 ? n_sel : E;
      const int32_t* lst = pass == 0 ? sel + (long)r * n_sel : exp_idx + (long)r * E;
      for (int i = 0; i < cnt; ++i) {
        const int tok = lst[i];
        if (tok < 0) continue;
        const int c = asg[(long)r * Lmax + tok];
        double* kb = kbar_r + ((long)r * C + c) * D;
        double* vb = vbar_r + ((long)r * C + c) * D;
        for (int d = 0; d < D; ++d) {
          kb[d] -= bf2f(K[((long)kvr * Lmax + tok) * D + d]);
          vb[d] -= bf2f(V[((long)kvr * Lmax + tok) * D + d]);
        }
      }
    }
    for (int c = 0; c < C; ++c) {
      const double nr = (double)n_t[(long)r * C + c] - (double)quota[(long)r * C + c];
      const double den = nr > 1.0 ? nr : 1.0;
      double* kb = kbar_r + ((long)r * C + c) * D;
      double* vb = vbar_r + ((long)r * C + c) * D;
      for (int d = 0; d < D; ++d) { kb[d] /= den; vb[d] /= den; }
      log_n[(long)r * C + c] = nr > 0.5 ? log(den) : -INFINITY;
    }
  }
}

/* ------------------------------------------------------------------ merge softmax
 * One softmax over {selected} U {expanded} U {proxies} (multibin.py:2727-2747;
 * methods_eager.py:708-720).  fp64.  kbar/vbar rows: per query-head row (pkv = 0) or per KV
 * head (pkv = 1, triton_expand_decode.py).  -1 indices and -inf log_n are skipped; a row with
 * nothing valid returns 0. */
void oa_ref_flash(const uint16_t* q, const uint16_t* K, const uint16_t* V, int Lmax, const int32_t* sel,
                  int n_sel, const int32_t* exp_idx, int n_exp, const double* kbar, const double* vbar,
                  const double* log_n, int n_bins, int pkv, int R, int G, double sm, double* out) {
  double* z = (double*)malloc(sizeof(double) * (size_t)(n_sel + n_exp + n_bins + 1));
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    double qa[D];
    for (int d = 0; d < D; ++d) qa[d] = bf2f(q[(long)r * D + d]);
    double mx = -INFINITY;
    const int T = n_sel + n_exp + n_bins;
    for (int t = 0; t < T; ++t) {
      z[t] = -INFINITY;
      if (t < n_sel + n_exp) {
        const int tok = t < n_sel ? sel[(long)r * n_sel + t] : exp_idx[(long)r * n_exp + (t - n_sel)];
        if (tok < 0) continue;
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += qa[d] * bf2f(K[((long)kvr * Lmax + tok) * D + d]);
        z[t] = s * sm;
      } else {
        const int b = t - n_sel - n_exp;
        const double ln = log_n[(long)r * n_bins + b];
        if (!(ln > -INFINITY)) continue;
        const long pr = pkv ? kvr : r;
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += qa[d] * kbar[((long)pr * n_bins + b) * D + d];
        z[t] = s * sm + ln;
      }
      if (z[t] > mx) mx = z[t];
    }
    double den = 0.0, acc[D];
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    if (mx > -INFINITY) {
      for (int t = 0; t < T; ++t) {
        if (!(z[t] > -INFINITY)) continue;
        const double p = exp(z[t] - mx);
        den += p;
        if (t < n_sel + n_exp) {
          const int tok = t < n_sel ? sel[(long)r * n_sel + t] : exp_idx[(long)r * n_exp + (t - n_sel)];
          for (int d = 0; d < D; ++d) acc[d] += p * bf2f(V[((long)kvr * Lmax + tok) * D + d]);
        } else {
          const int b = t - n_sel - n_exp;
          const long pr = pkv ? kvr : r;
          for (int d = 0; d < D; ++d) acc[d] += p * vbar[((long)pr * n_bins + b) * D + d];
        }
      }
    }
    for (int d = 0; d < D; ++d) out[(long)r * D + d] = den > 0.0 ? acc[d] / den : 0.0;
  }
  free(z);
}

/* dense attention over positions [0, n), fp64 (comparator check) */
void oa_ref_dense(const uint16_t* q, const uint16_t* K, const uint16_t* V, int Lmax, int n, int R, int G,
                  double sm, double* out) {
  double* z = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    double qa[D], acc[D], mx = -INFINITY, den = 0.0;
    for (int d = 0; d < D; ++d) { qa[d] = bf2f(q[(long)r * D + d]); acc[d] = 0.0; }
    for (int t = 0; t < n; ++t) {
      double s = 0.0;
      for (int d = 0; d < D; ++d) s += qa[d] * bf2f(K[((long)kvr * Lmax + t) * D + d]);
      z[t] = s * sm;
      if (z[t] > mx) mx = z[t];
    }
    for (int t = 0; t < n; ++t) {
      const double p = exp(z[t] - mx);
      den += p;
      for (int d = 0; d < D; ++d) acc[d] += p * bf2f(V[((long)kvr * Lmax + t) * D + d]);
    }
    for (int d = 0; d < D; ++d) out[(long)r * D + d] = acc[d] / den;
  }
  free(z);
}

/* ------------------------------------------------------------------ index update
 * _k_index_update_d2 (ours_graph.py:43-90), methods_eager.py:586-601, static_top_k.py:166-183,
 * multibin.py:2062-2096.  Mutates codes, asg, nb, Sk, Sk2, Sv, reclist, reccnt in place. */
void oa_ref_index_update(const uint16_t* K, const uint16_t* V, int Lmax, int pos, int R, int G, int C,
                         int8_t* codes, const float* U, const float* scale, const uint16_t* W,
                         const float* colmean, const float* cent, int32_t* asg, float* nb, float* Sk,
                         float* Sk2, float* Sv, int32_t* reclist, int32_t* reccnt, int rmax) {
  float ka[D], va[D], ua[D];
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    for (int d = 0; d < D; ++d) {
      ka[d] = bf2f(K[((long)kvr * Lmax + pos) * D + d]);
      va[d] = bf2f(V[((long)kvr * Lmax + pos) * D + d]);
    }
    if (r % G == 0) {
      for (int j = 0; j < RQ; ++j) {
        for (int d = 0; d < D; ++d) ua[d] = U[((long)kvr * D + d) * RQ + j];
        const float zc = dot128_canon(ka, ua);
        float code = rintf(zc / scale[(long)kvr * RQ + j]);
        code = fminf(fmaxf(code, -127.f), 127.f);
        codes[((long)kvr * Lmax + pos) * RQ + j] = (int8_t)(int)code;
      }
    }
    float zp[RC];
    for (int j = 0; j < RC; ++j) {
      for (int d = 0; d < D; ++d) ua[d] = bf2f(W[((long)r * D + d) * RC + j]);
      zp[j] = bf_round(dot128_canon(ka, ua)) - colmean[(long)r * RC + j];
    }
    int best_c = 0;
    float best = -INFINITY;
    for (int c = 0; c < C; ++c) {
      const float* cc = cent + ((long)r * C + c) * RC;
      float sim = zp[0] * cc[0];
      float h = cc[0] * cc[0];
      for (int j = 1; j < RC; ++j) {
        sim = fmaf(zp[j], cc[j], sim);
        h = fmaf(cc[j], cc[j], h);
      }
      const float dist = sim - 0.5f * h;
      if (c == 0 || dist > best) { best = dist; best_c = c; }
    }
    const int c = best_c;
    const long sb = ((long)r * C + c) * D;
    for (int d = 0; d < D; ++d) {
      Sk[sb + d] += ka[d];
      Sk2[sb + d] += ka[d] * ka[d];
      Sv[sb + d] += va[d];
    }
    asg[(long)r * Lmax + pos] = c;
    nb[(long)r * C + c] += 1.0f;
    const long rc = (long)r * C + c;
    if (reccnt[rc] < rmax) reclist[rc * rmax + reccnt[rc]] = pos;
    reccnt[rc] += 1;
  }
}

/* Removal of the token at pos from every query row's cluster statistics, in the fp32 terms of
 * oa_ref_index_update's statistics step (n_c -= 1, Sk_c -= k, Sk2_c -= k*k, Sv_c -= v with
 * c = asg[r][pos]).  A multi-row call's causal row i keeps only the keys before
 * n_i = K - Q + i + 1 in its tail (valid = raw > NEG with the causal mask added,
 * multibin.py:2210-2218); the statistics of [0, n_i) are those of [0, K) with the keys
 * K-1, ..., n_i taken back in that order. */
void oa_ref_index_downdate(const uint16_t* K, const uint16_t* V, int Lmax, int pos, int R, int G,
                           int C, const int32_t* asg, float* nb, float* Sk, float* Sk2, float* Sv) {
  for (int r = 0; r < R; ++r) {
    const int kvr = r / G;
    const int c = asg[(long)r * Lmax + pos];
    if (c < 0 || c >= C) continue;
    const long sb = ((long)r * C + c) * D;
    for (int d = 0; d < D; ++d) {
      const float k = bf2f(K[((long)kvr * Lmax + pos) * D + d]);
      const float v = bf2f(V[((long)kvr * Lmax + pos) * D + d]);
      Sk[sb + d] -= k;
      Sk2[sb + d] -= k * k;
      Sv[sb + d] -= v;
    }
    nb[(long)r * C + c] -= 1.0f;
  }
}

/* ==================================================================================== prefill
 * Index build of one request (KV rows h < HKV of K, V: (HKV, Lmax, 128) bf16; query rows
 * r < R = G * HKV).  Orders as fixed by the device build (openattention_amd/csrc/oa_build.hip).
 */

/* QGS codes: ours_fastbuild.py:256-261, StaticTopKMasker._extend (static_top_k.py:174-181).
 * zc_r = fma chain over d = 0..127 from 0; scale = max(max_t |zc| / 127, 1e-12);
 * codes = clamp(rint(zc / scale), -127, 127).  codes (HKV, Lmax, 32), scale (HKV, 32). */
void oa_ref_qgs_codes(const uint16_t* K, int Lmax, int HKV, int T, const float* U, int8_t* codes,
                      float* scale) {
  float* zc = (float*)malloc(sizeof(float) * (size_t)T * RQ);
  for (int h = 0; h < HKV; ++h) {
    const float* Uh = U + (long)h * D * RQ;
    float amax[RQ];
    for (int r = 0; r < RQ; ++r) amax[r] = 0.f;
    for (int t = 0; t < T; ++t) {
      const uint16_t* kr = K + ((long)h * Lmax + t) * D;
      for (int r = 0; r < RQ; ++r) {
        float z = 0.f;
        for (int d = 0; d < D; ++d) z = fmaf(bf2f(kr[d]), Uh[d * RQ + r], z);
        zc[(long)t * RQ + r] = z;
        if (fabsf(z) > amax[r]) amax[r] = fabsf(z);
      }
    }
    for (int r = 0; r < RQ; ++r) scale[h * RQ + r] = fmaxf(amax[r] / 127.0f, 1e-12f);
    for (int t = 0; t < T; ++t)
      for (int r = 0; r < RQ; ++r) {
        const float q = fminf(fmaxf(rintf(zc[(long)t * RQ + r] / scale[h * RQ + r]), -127.f), 127.f);
        codes[((long)h * Lmax + t) * RQ + r] = (int8_t)(int)q;
      }
  }
  free(zc);
}

/* QGC projection before centring: zraw = bf16(k W) with the product's sum taken exactly and
 * rounded once to fp32 (the device's bf16 matrix cores round their fp32 partials themselves, so
 * the device agrees with this up to rare bf16 ties).  zraw (R, T, 16) bf16 bits. */
void oa_ref_qgc_zraw(const uint16_t* K, int Lmax, int R, int G, int T, const uint16_t* W,
                     uint16_t* zraw) {
  for (int r = 0; r < R; ++r) {
    const uint16_t* Wr = W + (long)r * D * RC;
    for (int t = 0; t < T; ++t) {
      const uint16_t* kr = K + ((long)(r / G) * Lmax + t) * D;
      for (int j = 0; j < RC; ++j) {
        long double s = 0.0L;
        for (int d = 0; d < D; ++d) s += (long double)bf2f(kr[d]) * (long double)bf2f(Wr[d * RC + j]);
        zraw[((long)r * T + t) * RC + j] = f2bf((float)s);
      }
    }
  }
}

/* colmean and centring in the device's order: per 64-token tile and column, four lane partials
 * g = 0..3 (tokens 64k + 16b + 4g + i, b then i ascending, fp64), combined (g0+g1)+(g2+g3);
 * tiles summed in order; colmean = fp32(sum / T); zP = zraw - colmean (fp32). */
void oa_ref_qgc_center(const uint16_t* zraw, int R, int T, float* zP, float* colmean) {
  const int ntiles = (T + 63) / 64;
  for (int r = 0; r < R; ++r) {
    for (int j = 0; j < RC; ++j) {
      double s = 0.0;
      for (int k = 0; k < ntiles; ++k) {
        double c[4];
        for (int g = 0; g < 4; ++g) {
          c[g] = 0.0;
          for (int b = 0; b < 4; ++b)
            for (int i = 0; i < 4; ++i) {
              const int t = 64 * k + 16 * b + 4 * g + i;
              if (t < T) c[g] += (double)bf2f(zraw[((long)r * T + t) * RC + j]);
            }
        }
        s += (c[0] + c[1]) + (c[2] + c[3]);
      }
      colmean[r * RC + j] = (float)(s / (double)T);
    }
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < RC; ++j)
        zP[((long)r * T + t) * RC + j] = bf2f(zraw[((long)r * T + t) * RC + j]) - colmean[r * RC + j];
  }
}

/* k-means assignment (ours_fastbuild.py:52-82, methods_eager.py:536-540): a_t = argmax_c
 * bf16(bf16(bf16(zP_t) . bf16(c)) - bf16(|c|^2 / 2)), the dot taken exactly and rounded once to
 * fp32 (see oa_ref_qgc_zraw), |c|^2 = sequential fp32 sum of the rounded squares; ties to the
 * lower cluster.  zP (R, T, 16); cent (R, C, 16); asg (R, T). */
void oa_ref_kmeans_assign(const float* zP, int R, int T, const float* cent, int C, int32_t* asg) {
  float* cb = (float*)malloc(sizeof(float) * (size_t)C * RC);
  float* half = (float*)malloc(sizeof(float) * (size_t)C);
  for (int r = 0; r < R; ++r) {
    for (int c = 0; c < C; ++c) {
      const float* cc = cent + ((long)r * C + c) * RC;
      float s = 0.f;
      for (int j = 0; j < RC; ++j) {
        cb[c * RC + j] = bf_round(cc[j]);
        s = s + cc[j] * cc[j];
      }
      half[c] = bf_round(0.5f * s);
    }
    for (int t = 0; t < T; ++t) {
      float zb[RC];
      for (int j = 0; j < RC; ++j) zb[j] = bf_round(zP[((long)r * T + t) * RC + j]);
      int best_c = 0;
      float best = 0.f;
      for (int c = 0; c < C; ++c) {
        double s = 0.0;   /* 16 products of bf16 values: exact in fp64 */
        for (int j = 0; j < RC; ++j) s += (double)zb[j] * (double)cb[c * RC + j];
        const float dist = bf_round(bf_round((float)s) - half[c]);
        if (c == 0 || dist > best) { best = dist; best_c = c; }
      }
      asg[(long)r * T + t] = best_c;
    }
  }
  free(cb);
  free(half);
}

/* k-means update (ours_fastbuild.py:85-108, methods_eager.py:541-547): centroid = fp32(fp64 sum
 * of the members' zP rows in position order / count); an empty cluster takes zP[init[c]].
 * cnt (R, C) member counts. */
void oa_ref_kmeans_update(const float* zP, int R, int T, const int32_t* asg, int C,
                          const int32_t* init, float* cent, float* cnt) {
  double* acc = (double*)malloc(sizeof(double) * (size_t)C * RC);
  int* n = (int*)malloc(sizeof(int) * (size_t)C);
  for (int r = 0; r < R; ++r) {
    memset(acc, 0, sizeof(double) * (size_t)C * RC);
    memset(n, 0, sizeof(int) * (size_t)C);
    for (int t = 0; t < T; ++t) {
      const int c = asg[(long)r * T + t];
      n[c] += 1;
      for (int j = 0; j < RC; ++j) acc[c * RC + j] += (double)zP[((long)r * T + t) * RC + j];
    }
    for (int c = 0; c < C; ++c) {
      for (int j = 0; j < RC; ++j)
        cent[((long)r * C + c) * RC + j] =
            n[c] > 0 ? (float)(acc[c * RC + j] / (double)n[c]) : zP[((long)r * T + init[c]) * RC + j];
      cnt[r * C + c] = (float)n[c];
    }
  }
  free(acc);
  free(n);
}

/* Cluster statistics and CSR lists (ours_fastbuild.py:111-139, 293-301): per cluster the
 * members in position order; nb = count; Sk, Sk2, Sv = fp32 of the fp64 sums of k, k*k, v in that
 * order; mem = members grouped by cluster (stable argsort), cstart = exclusive prefix, clen.
 * nb (R, C); Sk, Sk2, Sv (R, C, 128); mem (R, T). */
void oa_ref_cluster_build(const uint16_t* K, const uint16_t* V, int Lmax, int R, int G, int T,
                          const int32_t* asg, int C, float* nb, float* Sk, float* Sk2, float* Sv,
                          int32_t* mem, int32_t* cstart, int32_t* clen) {
  double* acc = (double*)malloc(sizeof(double) * (size_t)C * D * 3);
  int* n = (int*)malloc(sizeof(int) * (size_t)C);
  int* fill = (int*)malloc(sizeof(int) * (size_t)C);
  for (int r = 0; r < R; ++r) {
    const int32_t* ar = asg + (long)r * T;
    memset(acc, 0, sizeof(double) * (size_t)C * D * 3);
    memset(n, 0, sizeof(int) * (size_t)C);
    for (int t = 0; t < T; ++t) n[ar[t]] += 1;
    int run = 0;
    for (int c = 0; c < C; ++c) {
      cstart[r * C + c] = run;
      clen[r * C + c] = n[c];
      nb[r * C + c] = (float)n[c];
      fill[c] = run;
      run += n[c];
    }
    for (int t = 0; t < T; ++t) {
      const int c = ar[t];
      mem[(long)r * T + fill[c]++] = t;
      const uint16_t* kr = K + ((long)(r / G) * Lmax + t) * D;
      const uint16_t* vr = V + ((long)(r / G) * Lmax + t) * D;
      double* a = acc + (long)c * D * 3;
      for (int d = 0; d < D; ++d) {
        const double k = (double)bf2f(kr[d]);
        a[d] += k;
        a[D + d] += k * k;
        a[2 * D + d] += (double)bf2f(vr[d]);
      }
    }
    for (int c = 0; c < C; ++c)
      for (int d = 0; d < D; ++d) {
        const long o = ((long)r * C + c) * D + d;
        Sk[o] = (float)acc[(long)c * D * 3 + d];
        Sk2[o] = (float)acc[(long)c * D * 3 + D + d];
        Sv[o] = (float)acc[(long)c * D * 3 + 2 * D + d];
      }
  }
  free(acc);
  free(n);
  free(fill);
}
