// Residual cluster proxies and the fused decode softmax of the deployed step.
//
// Residual (multibin.py:2598-2642, residual_stats="full"; deployed ours_fused.py:366-407):
// every token read exactly (selected or expanded) leaves its cluster's proxy:
//   n'_c    = n_t,c - q_c
//   kbar'_c = (Sk_c - sum_{read tokens in c} k) / max(n'_c, 1)
//   vbar'_c = (Sv_c - sum_{read tokens in c} v) / max(n'_c, 1)
//   ln n'_c if n'_c > 0.5, else -inf (the proxy leaves the softmax)
// Softmax merge (multibin.py:2727-2747): one softmax over {selected} U {expanded} U {proxies},
// proxy logit s q.kbar'_c + ln n'_c.
//
// gfx950 decomposition: one 256-thread workgroup per query-head row.  Each of its four waves
// owns clusters c = w, w+4, ...: it walks the cluster's own contiguous segment of exp_idx
// (written grouped by cluster by the top-q kernel) plus the cluster's selected tokens,
// accumulating the residual sums in registers while folding the same K,V rows into the
// wave's online softmax, then folds the cluster's proxy.  Every K/V row is read once, the
// sums are owned by one wave (no atomics, run-to-run deterministic), and the proxies never
// leave registers.  A lane holds dims (2l, 2l+1), so a row is one 4-byte load per lane.
// Wave 0 also folds the selected tokens.  The four wave states are merged at the end.
//
// oa_residual writes kbar', vbar' (bf16) and ln n' instead of the softmax (the operator
// surface of the reference's residual kernels), for use with oa_flash_decode.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxC = 256;
constexpr int kMaxSel = 64;
constexpr float kLog2e = 1.4426950408889634f;

struct ResArgs {
  const uint16_t* q; long q_stride;
  const uint16_t* K; const uint16_t* V; long kv_sb; long kv_ss; int G;
  const int32_t* asg; long asg_stride;
  const int32_t* sel; long sel_stride; int n_sel;
  const int32_t* exq; int E;
  const float* quota; const float* n_t;
  const float* Sk; const float* Sv;
  int C; float sm_scale;
  uint16_t* out; long out_stride;               // fused variant
  uint16_t* kbar_r; uint16_t* vbar_r; float* logn;  // residual-only variant
};

struct Soft {
  float m, l, a0, a1;
  __device__ __forceinline__ void init() { m = -INFINITY; l = 0.f; a0 = 0.f; a1 = 0.f; }
  __device__ __forceinline__ void add(float z, float v0, float v1) {
    const float mn = fmaxf(m, z);
    const float al = exp2f(m - mn);
    const float p = exp2f(z - mn);
    a0 = fmaf(p, v0, a0 * al);
    a1 = fmaf(p, v1, a1 * al);
    l = fmaf(l, al, p);
    m = mn;
  }
};

__device__ __forceinline__ float2 ld_bf16x2(const uint16_t* p) {
  const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
  return make_float2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

template <bool FUSED>
__global__ void __launch_bounds__(kThreads) residual_kernel(ResArgs a) {
  __shared__ int s_base[kMaxC + 1];
  __shared__ int s_q[kMaxC];
  __shared__ int s_scid[kMaxSel];
  __shared__ float s_m[kWaves], s_l[kWaves];
  __shared__ float s_acc[kWaves][OA_D];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int kvr = row / a.G;
  const int d0 = 2 * lane;
  const uint16_t* Kb = a.K + (long)kvr * a.kv_sb + d0;
  const uint16_t* Vb = a.V + (long)kvr * a.kv_sb + d0;

  if (tid == 0) {
    int acc = 0;
    for (int c = 0; c < a.C; ++c) {
      const int qc = (int)a.quota[(long)row * a.C + c];
      s_q[c] = qc;
      s_base[c] = acc;
      acc += qc;
    }
    s_base[a.C] = acc;
  }
  for (int i = tid; i < a.n_sel; i += kThreads) {
    const int tok = a.sel[(long)row * a.sel_stride + i];
    s_scid[i] = tok >= 0 ? a.asg[(long)row * a.asg_stride + tok] : -1;
  }
  __syncthreads();

  const float2 qv = ld_bf16x2(a.q + (long)row * a.q_stride + d0);
  const float zs = a.sm_scale * kLog2e;
  Soft sm;
  sm.init();
  if (FUSED && wave == 0) {
    for (int i = 0; i < a.n_sel; ++i) {
      const int tok = a.sel[(long)row * a.sel_stride + i];
      if (tok < 0) continue;
      const float2 k = ld_bf16x2(Kb + (long)tok * a.kv_ss);
      const float2 v = ld_bf16x2(Vb + (long)tok * a.kv_ss);
      const float z = oa::wave_sum(fmaf(qv.y, k.y, qv.x * k.x)) * zs;
      sm.add(z, v.x, v.y);
    }
  }
  const int32_t* erow = a.exq + (long)row * a.E;
  for (int c = wave; c < a.C; c += kWaves) {
    float dk0 = 0.f, dk1 = 0.f, dv0 = 0.f, dv1 = 0.f;
    for (int i = 0; i < a.n_sel; ++i) {
      if (s_scid[i] != c) continue;
      const int tok = a.sel[(long)row * a.sel_stride + i];
      const float2 k = ld_bf16x2(Kb + (long)tok * a.kv_ss);
      const float2 v = ld_bf16x2(Vb + (long)tok * a.kv_ss);
      dk0 += k.x; dk1 += k.y; dv0 += v.x; dv1 += v.y;
    }
    const int b0 = s_base[c];
    const int b1 = min(s_base[c] + s_q[c], a.E);
    int j = b0;
    for (; j + 4 <= b1; j += 4) {
      int t[4];
      float2 k[4], v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = erow[j + u];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long off = (long)(t[u] >= 0 ? t[u] : 0) * a.kv_ss;
        k[u] = ld_bf16x2(Kb + off);
        v[u] = ld_bf16x2(Vb + off);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (t[u] < 0) continue;
        dk0 += k[u].x; dk1 += k[u].y; dv0 += v[u].x; dv1 += v[u].y;
        if (FUSED) {
          const float z = oa::wave_sum(fmaf(qv.y, k[u].y, qv.x * k[u].x)) * zs;
          sm.add(z, v[u].x, v[u].y);
        }
      }
    }
    for (; j < b1; ++j) {
      const int tok = erow[j];
      if (tok < 0) continue;
      const float2 k = ld_bf16x2(Kb + (long)tok * a.kv_ss);
      const float2 v = ld_bf16x2(Vb + (long)tok * a.kv_ss);
      dk0 += k.x; dk1 += k.y; dv0 += v.x; dv1 += v.y;
      if (FUSED) {
        const float z = oa::wave_sum(fmaf(qv.y, k.y, qv.x * k.x)) * zs;
        sm.add(z, v.x, v.y);
      }
    }
    const long sb = ((long)row * a.C + c) * OA_D + d0;
    const float2 sk = *reinterpret_cast<const float2*>(a.Sk + sb);
    const float2 sv = *reinterpret_cast<const float2*>(a.Sv + sb);
    const float nr = a.n_t[(long)row * a.C + c] - (float)s_q[c];
    const float den = fmaxf(nr, 1.0f);
    const float kb0 = (sk.x - dk0) / den, kb1 = (sk.y - dk1) / den;
    const float vb0 = (sv.x - dv0) / den, vb1 = (sv.y - dv1) / den;
    const bool live = nr > 0.5f;
    const float ln = live ? logf(den) : -INFINITY;
    if (FUSED) {
      if (live) {
        const float z = (oa::wave_sum(fmaf(qv.y, kb1, qv.x * kb0)) * a.sm_scale + ln) * kLog2e;
        sm.add(z, vb0, vb1);
      }
    } else {
      const long ob = ((long)row * a.C + c) * OA_D + d0;
      const uint32_t kw = (uint32_t)oa::f32_to_bf16(kb0) | ((uint32_t)oa::f32_to_bf16(kb1) << 16);
      const uint32_t vw = (uint32_t)oa::f32_to_bf16(vb0) | ((uint32_t)oa::f32_to_bf16(vb1) << 16);
      *reinterpret_cast<uint32_t*>(a.kbar_r + ob) = kw;
      *reinterpret_cast<uint32_t*>(a.vbar_r + ob) = vw;
      if (lane == 0) a.logn[(long)row * a.C + c] = ln;
    }
  }
  if (!FUSED) return;
  if (lane == 0) { s_m[wave] = sm.m; s_l[wave] = sm.l; }
  s_acc[wave][d0] = sm.a0;
  s_acc[wave][d0 + 1] = sm.a1;
  __syncthreads();
  if (tid < OA_D) {
    float M = -INFINITY;
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w]);
    float L = 0.f, A = 0.f;
    if (M > -INFINITY) {
      for (int w = 0; w < kWaves; ++w) {
        if (s_m[w] > -INFINITY) {
          const float wt = exp2f(s_m[w] - M);
          L = fmaf(s_l[w], wt, L);
          A = fmaf(s_acc[w][tid], wt, A);
        }
      }
    }
    const float o = L > 0.f ? A / L : 0.f;
    a.out[(long)row * a.out_stride + tid] = oa::f32_to_bf16(o);
  }
}

int launch(bool fused, const void* q, long q_stride, const void* K, const void* V, long kv_sb,
           long kv_ss, int rows, int kv_rows, int head_dim, const int32_t* asg, long asg_stride,
           const int32_t* sel, long sel_stride, int n_sel, const int32_t* exp_idx, int E,
           const float* quota, const float* n_t, const float* Sk, const float* Sv, int C,
           float sm_scale, void* out, long out_stride, void* kbar_r, void* vbar_r, float* logn,
           void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows % kv_rows != 0 || C <= 0 || C > kMaxC ||
      n_sel < 0 || n_sel > kMaxSel || E < 0 || (kv_ss % 2) != 0)
    return OA_EINVAL;
  ResArgs a;
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.kv_sb = kv_sb; a.kv_ss = kv_ss;
  a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.exq = exp_idx; a.E = E; a.quota = quota; a.n_t = n_t; a.Sk = Sk; a.Sv = Sv;
  a.C = C; a.sm_scale = sm_scale;
  a.out = (uint16_t*)out; a.out_stride = out_stride;
  a.kbar_r = (uint16_t*)kbar_r; a.vbar_r = (uint16_t*)vbar_r; a.logn = logn;
  if (fused)
    hipLaunchKernelGGL(residual_kernel<true>, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(residual_kernel<false>, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}

}  // namespace

extern "C" int oa_residual_flash(const void* q, long q_stride, const void* K, const void* V,
                                 long kv_stride_b, long kv_stride_s, int rows, int kv_rows,
                                 int head_dim, const int32_t* asg, long asg_stride,
                                 const int32_t* sel, long sel_stride, int n_sel,
                                 const int32_t* exp_idx, int E, const float* quota,
                                 const float* n_t, const float* Sk, const float* Sv, int C,
                                 float sm_scale, void* out, long out_stride, void* stream) {
  if (!out) return OA_EINVAL;
  return launch(true, q, q_stride, K, V, kv_stride_b, kv_stride_s, rows, kv_rows, head_dim, asg,
                asg_stride, sel, sel_stride, n_sel, exp_idx, E, quota, n_t, Sk, Sv, C, sm_scale,
                out, out_stride, nullptr, nullptr, nullptr, stream);
}

extern "C" int oa_residual(const void* K, const void* V, long kv_stride_b, long kv_stride_s,
                           int rows, int kv_rows, int head_dim, const int32_t* asg,
                           long asg_stride, const int32_t* sel, long sel_stride, int n_sel,
                           const int32_t* exp_idx, int E, const float* quota, const float* n_t,
                           const float* Sk, const float* Sv, int C, void* kbar_r, void* vbar_r,
                           float* log_n, void* stream) {
  if (!kbar_r || !vbar_r || !log_n) return OA_EINVAL;
  // the query is not read by the residual-only variant; pass K so the pointer is valid
  return launch(false, K, 0, K, V, kv_stride_b, kv_stride_s, rows, kv_rows, head_dim, asg,
                asg_stride, sel, sel_stride, n_sel, exp_idx, E, quota, n_t, Sk, Sv, C, 0.f,
                nullptr, 0, kbar_r, vbar_r, log_n, stream);
}
