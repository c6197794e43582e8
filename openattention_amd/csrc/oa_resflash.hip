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
// Fused kernel (oa_residual_flash), gfx950 decomposition.  The proxy logit needs only
//   q.kbar'_c = (q.Sk_c - sum_{read i in c} q.k_i) / max(n'_c, 1),
// scalars the softmax computes anyway, and the merged numerator regroups as
//   sum_i (p_i - w_c(i) / den_c(i)) v_i + sum_c (w_c / den_c) Sv_c
// (w_c the proxy weight, den_c = max(n'_c, 1)), so no per-cluster vector sums are formed.
// One 512-thread workgroup per query-head row, 32 lane groups of 16 lanes (8 dims per lane):
//   pass 1  every read token's q.k and every cluster's q.Sk as independent units, spread
//           round-robin over the lane groups, eight loads in flight per group;
//   scalars one thread per cluster sums its read tokens' dots in list order (selected tokens,
//           then its exp_idx segment), forms the proxy logit; block max and weights;
//   pass 2  every read token's V row and every cluster's Sv row scaled by its coefficient,
//           accumulated per lane group and reduced over the groups in a fixed order.
// Every K/V and statistics row is read once; all sums have a fixed order (deterministic).
// exp_idx must list each cluster's tokens inside that cluster's quota segment (an expanded
// token's cluster is the owner of its slot), which is the layout oa_topq writes.
//
// oa_residual writes kbar', vbar' (bf16) and ln n' instead of the softmax (the operator
// surface of the reference's residual kernels), for use with oa_flash_decode.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;
constexpr int kMaxC = 256;
constexpr int kMaxSel = 64;
constexpr int kMaxE = 4096;
constexpr float kLog2e = 1.4426950408889634f;

struct ResArgs {
  const uint16_t* q; long q_stride;
  const uint16_t* K; const uint16_t* V; long kv_sb; long kv_ss; int G;
  const int32_t* asg; long asg_stride;
  const int32_t* sel; long sel_stride; int n_sel;
  const int32_t* exq; int E;
  const float* quota; const float* n_t;
  const float* Sk; const float* Sv;
  const float* qsk;                             // optional: q . Sk_c from the gate
  int C; float sm_scale;
  void* out; long out_stride; int out_f32;      // fused variant
  uint16_t* kbar_r; uint16_t* vbar_r; float* logn;  // residual-only variant
};

struct Soft {
  float m, l, a[8];
  __device__ __forceinline__ void init() {
    m = -INFINITY; l = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = 0.f;
  }
  __device__ __forceinline__ void add(float z, const float* v) {
    const float mn = fmaxf(m, z);
    const float al = exp2f(m - mn);
    const float p = exp2f(z - mn);
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = fmaf(p, v[i], a[i] * al);
    l = fmaf(l, al, p);
    m = mn;
  }
};

__device__ __forceinline__ float dot8(const float* a, const float* b) {
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) p = fmaf(a[i], b[i], p);
  return p;
}

template <bool FUSED>
__global__ void __launch_bounds__(kThreads) residual_kernel(ResArgs a) {
  __shared__ int s_base[kMaxC + 1];
  __shared__ int s_q[kMaxC];
  __shared__ int s_stok[kMaxSel];
  __shared__ int s_scid[kMaxSel];
  __shared__ int s_exp[kMaxE];
  __shared__ float s_m[kGroups], s_l[kGroups];
  __shared__ float s_acc[kGroups][OA_D];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;
  const int sub = tid & 15;
  const int d0 = sub * 8;
  const int kvr = row / a.G;
  const uint16_t* Kb = a.K + (long)kvr * a.kv_sb + d0;
  const uint16_t* Vb = a.V + (long)kvr * a.kv_sb + d0;

  if (tid < 64) {
    // quotas -> segment bases: lane l owns clusters 4l..4l+3, exclusive scan over lanes
    int v[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid * 4 + i;
      v[i] = c < a.C ? (int)a.quota[(long)row * a.C + c] : 0;
      loc += v[i];
    }
    const int incl = oa::wave_incl_scan_i32(loc);
    int run = incl - loc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid * 4 + i;
      if (c < a.C) { s_q[c] = v[i]; s_base[c] = run; }
      run += v[i];
    }
    if (tid == 63) s_base[a.C] = incl;
  }
  for (int i = tid; i < a.n_sel; i += kThreads) {
    const int tok = a.sel[(long)row * a.sel_stride + i];
    s_stok[i] = tok;
    s_scid[i] = tok >= 0 ? a.asg[(long)row * a.asg_stride + tok] : -1;
  }
  for (int j = tid; j < a.E; j += kThreads) s_exp[j] = a.exq[(long)row * a.E + j];
  __syncthreads();

  float qv[8];
  oa::unpack8(*reinterpret_cast<const uint4*>(a.q + (long)row * a.q_stride + d0), qv);
  const float zs = a.sm_scale * kLog2e;
  Soft sm;
  sm.init();
  for (int c = grp; c < a.C; c += kGroups) {
    float dk[8], dv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { dk[i] = 0.f; dv[i] = 0.f; }
    // the selected tokens of this cluster (each selected token lies in exactly one cluster, so
    // the softmax sees it exactly once)
    for (int i = 0; i < a.n_sel; ++i) {
      if (s_scid[i] != c) continue;
      const long off = (long)s_stok[i] * a.kv_ss;
      float kx[8], vx[8];
      oa::unpack8(*reinterpret_cast<const uint4*>(Kb + off), kx);
      oa::unpack8(*reinterpret_cast<const uint4*>(Vb + off), vx);
#pragma unroll
      for (int e = 0; e < 8; ++e) { dk[e] += kx[e]; dv[e] += vx[e]; }
      if (FUSED) sm.add(oa::group16_sum(dot8(qv, kx)) * zs, vx);
    }
    // the cluster's segment of expanded tokens, four in flight
    const int qc = s_q[c];
    const int b0 = s_base[c];
    const int b1 = min(b0 + qc, a.E);
    for (int j = b0; j < b1; j += 4) {
      uint4 kw[4], vw[4];
      int tk[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        tk[u] = (j + u < b1) ? s_exp[j + u] : -1;
        const long off = (long)(tk[u] >= 0 ? tk[u] : 0) * a.kv_ss;
        kw[u] = *reinterpret_cast<const uint4*>(Kb + off);
        vw[u] = *reinterpret_cast<const uint4*>(Vb + off);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (tk[u] < 0) continue;
        float kx[8], vx[8];
        oa::unpack8(kw[u], kx);
        oa::unpack8(vw[u], vx);
#pragma unroll
        for (int e = 0; e < 8; ++e) { dk[e] += kx[e]; dv[e] += vx[e]; }
        if (FUSED) sm.add(oa::group16_sum(dot8(qv, kx)) * zs, vx);
      }
    }
    // the proxy of the members still unread
    const long sb = ((long)row * a.C + c) * OA_D + d0;
    const float4 k0 = *reinterpret_cast<const float4*>(a.Sk + sb);
    const float4 k1 = *reinterpret_cast<const float4*>(a.Sk + sb + 4);
    const float4 v0 = *reinterpret_cast<const float4*>(a.Sv + sb);
    const float4 v1 = *reinterpret_cast<const float4*>(a.Sv + sb + 4);
    const float sk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float svv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    const float nr = a.n_t[(long)row * a.C + c] - (float)qc;
    const float den = fmaxf(nr, 1.0f);
    float kb[8], vb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kb[e] = (sk[e] - dk[e]) / den;
      vb[e] = (svv[e] - dv[e]) / den;
    }
    const bool live = nr > 0.5f;
    const float ln = live ? logf(den) : -INFINITY;
    if (FUSED) {
      const float dot = oa::group16_sum(dot8(qv, kb));
      if (live) sm.add((dot * a.sm_scale + ln) * kLog2e, vb);
    } else {
      const long ob = ((long)row * a.C + c) * OA_D + d0;
      uint4 kw, vw;
      kw.x = (uint32_t)oa::f32_to_bf16(kb[0]) | ((uint32_t)oa::f32_to_bf16(kb[1]) << 16);
      kw.y = (uint32_t)oa::f32_to_bf16(kb[2]) | ((uint32_t)oa::f32_to_bf16(kb[3]) << 16);
      kw.z = (uint32_t)oa::f32_to_bf16(kb[4]) | ((uint32_t)oa::f32_to_bf16(kb[5]) << 16);
      kw.w = (uint32_t)oa::f32_to_bf16(kb[6]) | ((uint32_t)oa::f32_to_bf16(kb[7]) << 16);
      vw.x = (uint32_t)oa::f32_to_bf16(vb[0]) | ((uint32_t)oa::f32_to_bf16(vb[1]) << 16);
      vw.y = (uint32_t)oa::f32_to_bf16(vb[2]) | ((uint32_t)oa::f32_to_bf16(vb[3]) << 16);
      vw.z = (uint32_t)oa::f32_to_bf16(vb[4]) | ((uint32_t)oa::f32_to_bf16(vb[5]) << 16);
      vw.w = (uint32_t)oa::f32_to_bf16(vb[6]) | ((uint32_t)oa::f32_to_bf16(vb[7]) << 16);
      *reinterpret_cast<uint4*>(a.kbar_r + ob) = kw;
      *reinterpret_cast<uint4*>(a.vbar_r + ob) = vw;
      if (sub == 0) a.logn[(long)row * a.C + c] = ln;
    }
  }
  if (!FUSED) return;
  if (sub == 0) { s_m[grp] = sm.m; s_l[grp] = sm.l; }
#pragma unroll
  for (int i = 0; i < 8; ++i) s_acc[grp][d0 + i] = sm.a[i];
  __syncthreads();
  if (tid < OA_D) {
    float M = -INFINITY;
    for (int g = 0; g < kGroups; ++g) M = fmaxf(M, s_m[g]);
    float L = 0.f, A = 0.f;
    if (M > -INFINITY) {
      for (int g = 0; g < kGroups; ++g) {
        if (s_m[g] > -INFINITY) {
          const float wt = exp2f(s_m[g] - M);
          L = fmaf(s_l[g], wt, L);
          A = fmaf(s_acc[g][tid], wt, A);
        }
      }
    }
    const float o = L > 0.f ? A / L : 0.f;
    oa::store_out(a.out, a.out_f32, (long)row * a.out_stride + tid, o);
  }
}

constexpr int kRFThreads = 512;
constexpr int kRFGroups = kRFThreads / 16;
constexpr int kRFWaves = kRFThreads / 64;
constexpr int kBatch = 4;

// fixed-order sum / max over the workgroup (thread partials -> wave butterfly -> waves in order)
__device__ __forceinline__ float block_sum(float v, float* s_red, int tid) {
  v = oa::wave_sum(v);
  __syncthreads();
  if ((tid & 63) == 0) s_red[tid >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kRFWaves; ++w) t += s_red[w];
  return t;
}
__device__ __forceinline__ float block_max(float v, float* s_red, int tid) {
  v = oa::wave_max(v);
  __syncthreads();
  if ((tid & 63) == 0) s_red[tid >> 6] = v;
  __syncthreads();
  float t = -INFINITY;
#pragma unroll
  for (int w = 0; w < kRFWaves; ++w) t = fmaxf(t, s_red[w]);
  return t;
}

// 8 waves per SIMD (<= 64 VGPRs): every row of a B=32 batch is resident at once
__global__ void __launch_bounds__(kRFThreads, 8) resflash_kernel(ResArgs a) {
  extern __shared__ int dyn_rf[];
  __shared__ int s_base[kMaxC + 1];
  __shared__ int s_q[kMaxC];
  __shared__ float s_nt[kMaxC];
  __shared__ float s_qsk[kMaxC], s_l2[kMaxC], s_cw[kMaxC];
  __shared__ float s_red[kRFWaves];
  __shared__ float s_acc[kRFGroups][OA_D];
  const int NI = a.n_sel + a.E;
  int* s_tok = dyn_rf;                                        // NI
  int* s_cid = s_tok + NI;                                    // NI
  float* s_z = reinterpret_cast<float*>(s_cid + NI);          // NI: q.k, later the coefficient
  const int row = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2
  const int tid = threadIdx.x;
  const int grp = tid >> 4;
  const int sub = tid & 15;
  const int d0 = sub * 8;
  const int C = a.C;
  const int kvr = row / a.G;
  const uint16_t* Kb = a.K + (long)kvr * a.kv_sb + d0;
  const uint16_t* Vb = a.V + (long)kvr * a.kv_sb + d0;

  // ---- phase 0: read lists, quota segments and tail counts (one round of loads: every
  // thread issues its first quota, tail-count and list loads before using any of them)
  int qv4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qv4[i] = (int)a.quota[(long)row * C + min((tid & 63) * 4 + i, C - 1)];
  const float ntv = a.n_t[(long)row * C + min(tid, C - 1)];
  int tok0 = -1;
  if (NI > 0) {
    const int i = min(tid, NI - 1);
    tok0 = i < a.n_sel ? a.sel[(long)row * a.sel_stride + i] : a.exq[(long)row * a.E + (i - a.n_sel)];
  }
  if (tid < 64) {
    int loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qv4[i] = tid * 4 + i < C ? qv4[i] : 0;
      loc += qv4[i];
    }
    const int incl = oa::wave_incl_scan_i32(loc);
    int run = incl - loc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid * 4 + i;
      if (c < C) { s_q[c] = qv4[i]; s_base[c] = run; }
      run += qv4[i];
    }
  }
  if (tid < C) s_nt[tid] = ntv;
  for (int c = tid + kRFThreads; c < C; c += kRFThreads) s_nt[c] = a.n_t[(long)row * C + c];
  if (a.qsk)                       // q . Sk from the gate: no pass over Sk below
    for (int c = tid; c < C; c += kRFThreads) s_qsk[c] = a.qsk[(long)row * C + c];
  if (tid < NI) s_tok[tid] = tok0;
  for (int i = tid + kRFThreads; i < NI; i += kRFThreads) {
    const int tok = i < a.n_sel ? a.sel[(long)row * a.sel_stride + i]
                                : a.exq[(long)row * a.E + (i - a.n_sel)];
    s_tok[i] = tok;
  }
  float qv[8];
  oa::unpack8(*reinterpret_cast<const uint4*>(a.q + (long)row * a.q_stride + d0), qv);
  __syncthreads();

  // ---- pass 1: q.k of every read token, q.Sk of every cluster; cluster ids of the read
  // tokens (expanded tokens: the owner of their quota segment; selected tokens: asg).  The
  // first batch of every stream is issued before any of them is used.
  auto load_k = [&](int u0, uint4* w) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int u = min(u0 + j * kRFGroups, NI - 1);
      const int tok = max(s_tok[u], 0);
      w[j] = *reinterpret_cast<const uint4*>(Kb + (long)tok * a.kv_ss);
    }
  };
  auto load_stat = [&](const float* base, int c0, float4 (*x)[2]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = min(c0 + j * kRFGroups, C - 1);
      const float* p = base + ((long)row * C + c) * OA_D + d0;
      x[j][0] = *reinterpret_cast<const float4*>(p);
      x[j][1] = *reinterpret_cast<const float4*>(p + 4);
    }
  };
  auto dots_k = [&](int u0, const uint4* w) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int u = u0 + j * kRFGroups;
      float kx[8];
      oa::unpack8(w[j], kx);
      const float z = oa::group16_sum(dot8(qv, kx));
      if (u < NI && sub == 0) s_z[u] = z;
    }
  };
  auto dots_sk = [&](int c0, float4 (*x)[2]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = c0 + j * kRFGroups;
      const float sk[8] = {x[j][0].x, x[j][0].y, x[j][0].z, x[j][0].w,
                           x[j][1].x, x[j][1].y, x[j][1].z, x[j][1].w};
      const float z = oa::group16_sum(dot8(qv, sk));
      if (c < C && sub == 0) s_qsk[c] = z;
    }
  };
  float4 skx[4][2];
  uint4 kw[kBatch];
  if (!a.qsk) load_stat(a.Sk, grp, skx);
  if (NI > 0) load_k(grp, kw);
  int scid = -1;
  const int stok = a.n_sel > 0 ? s_tok[min(tid, a.n_sel - 1)] : -1;
  if (a.n_sel > 0) {
    const int c = a.asg[(long)row * a.asg_stride + max(stok, 0)];
    scid = stok >= 0 ? c : -1;
  }
  for (int i = tid; i < NI; i += kRFThreads) {
    if (i < a.n_sel) continue;
    int c = -1;
    if (s_tok[i] >= 0) {
      const int j = i - a.n_sel;
      int lo = 0, hi = C - 1;                    // last cluster with base <= j
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_base[mid] <= j) lo = mid; else hi = mid - 1;
      }
      c = lo;
    }
    s_cid[i] = c;
  }
  if (tid < a.n_sel) s_cid[tid] = scid;
  if (NI > 0) dots_k(grp, kw);
  for (int u0 = grp + kRFGroups * kBatch; u0 < NI; u0 += kRFGroups * kBatch) {
    load_k(u0, kw);
    dots_k(u0, kw);
  }
  if (!a.qsk) {
    dots_sk(grp, skx);
    for (int c0 = grp + kRFGroups * 4; c0 < C; c0 += kRFGroups * 4) {
      load_stat(a.Sk, c0, skx);
      dots_sk(c0, skx);
    }
  }
  __syncthreads();

  // ---- scalars: proxy logits (log2 units), block max, weights, coefficients
  // Z_c = sum of q.k over the cluster's read tokens (its selected tokens and its expanded
  // segment), one 16-lane group per cluster: lanes take every 16th token, a fixed DPP tree adds
  // the 16 partials (a segment can hold hundreds of tokens)
  const float zs = a.sm_scale * kLog2e;
  for (int c = grp; c < C; c += kRFGroups) {
    float Z = 0.f;
    for (int i = sub; i < a.n_sel; i += 16)
      if (s_cid[i] == c) Z += s_z[i];
    const int b1 = min(s_base[c] + s_q[c], a.E);
    for (int j = s_base[c] + sub; j < b1; j += 16) {
      const int i = a.n_sel + j;
      if (s_cid[i] == c) Z += s_z[i];
    }
    Z = oa::group16_sum(Z);
    if (sub == 0) {
      const float nr = s_nt[c] - (float)s_q[c];
      const float den = fmaxf(nr, 1.0f);
      const bool live = nr > 0.5f;
      s_l2[c] = live ? (((s_qsk[c] - Z) / den) * a.sm_scale + logf(den)) * kLog2e : -INFINITY;
      s_cw[c] = den;
    }
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int i = tid; i < NI; i += kRFThreads)
    if (s_cid[i] >= 0) mx = fmaxf(mx, s_z[i] * zs);
  for (int c = tid; c < C; c += kRFThreads) mx = fmaxf(mx, s_l2[c]);
  const float M = block_max(mx, s_red, tid);
  float lsum = 0.f;
  for (int c = tid; c < C; c += kRFThreads) {
    const float wc = M > -INFINITY && s_l2[c] > -INFINITY ? exp2f(s_l2[c] - M) : 0.f;
    lsum += wc;
    s_cw[c] = wc / s_cw[c];                 // w_c / den_c (0 for a dead proxy)
  }
  __syncthreads();
  for (int i = tid; i < NI; i += kRFThreads) {
    const int c = s_cid[i];
    float coef = 0.f;
    if (c >= 0) {
      const float p = exp2f(s_z[i] * zs - M);
      lsum += p;
      coef = p - s_cw[c];
    }
    s_z[i] = coef;
  }
  const float L = block_sum(lsum, s_red, tid);   // its barriers also publish s_z

  // ---- pass 2: coefficient-weighted V rows and Sv rows
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int u0 = grp; u0 < NI; u0 += kRFGroups * kBatch) {
    uint4 w[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int u = min(u0 + j * kRFGroups, NI - 1);
      const int tok = max(s_tok[u], 0);
      w[j] = *reinterpret_cast<const uint4*>(Vb + (long)tok * a.kv_ss);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int u = u0 + j * kRFGroups;
      const float cf = u < NI ? s_z[u] : 0.f;
      float vx[8];
      oa::unpack8(w[j], vx);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(cf, vx[e], acc[e]);
    }
  }
  for (int c0 = grp; c0 < C; c0 += kRFGroups * 4) {
    float4 x[4][2];
    load_stat(a.Sv, c0, x);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = c0 + j * kRFGroups;
      const float cf = c < C ? s_cw[c] : 0.f;
      const float sv[8] = {x[j][0].x, x[j][0].y, x[j][0].z, x[j][0].w,
                           x[j][1].x, x[j][1].y, x[j][1].z, x[j][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(cf, sv[e], acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_acc[grp][d0 + e] = acc[e];
  __syncthreads();
  if (tid < OA_D) {
    float A = 0.f;
    for (int g = 0; g < kRFGroups; ++g) A += s_acc[g][tid];
    const float o = L > 0.f ? A / L : 0.f;
    oa::store_out(a.out, a.out_f32, (long)row * a.out_stride + tid, o);
  }
}

int launch(bool fused, const void* q, long q_stride, const void* K, const void* V, long kv_sb,
           long kv_ss, int rows, int kv_rows, int head_dim, const int32_t* asg, long asg_stride,
           const int32_t* sel, long sel_stride, int n_sel, const int32_t* exp_idx, int E,
           const float* quota, const float* n_t, const float* Sk, const float* Sv, int C,
           float sm_scale, void* out, long out_stride, int out_f32, void* kbar_r, void* vbar_r,
           float* logn, const float* qsk, void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows % kv_rows != 0 || C <= 0 || C > kMaxC ||
      n_sel < 0 || n_sel > kMaxSel || E < 0 || E > kMaxE || (kv_ss % 8) != 0 || (kv_sb % 8) != 0)
    return OA_EINVAL;
  ResArgs a;
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.kv_sb = kv_sb; a.kv_ss = kv_ss;
  a.G = rows / kv_rows;
  a.asg = asg; a.asg_stride = asg_stride;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.exq = exp_idx; a.E = E; a.quota = quota; a.n_t = n_t; a.Sk = Sk; a.Sv = Sv; a.qsk = qsk;
  a.C = C; a.sm_scale = sm_scale;
  a.out = out; a.out_stride = out_stride; a.out_f32 = out_f32 ? 1 : 0;
  a.kbar_r = (uint16_t*)kbar_r; a.vbar_r = (uint16_t*)vbar_r; a.logn = logn;
  if (fused) {
    const size_t lds = sizeof(int) * 3 * (size_t)(n_sel + E);
    if (lds > 65536) {
      const hipError_t e = hipFuncSetAttribute((const void*)resflash_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(resflash_kernel, dim3(rows), dim3(kRFThreads), lds, (hipStream_t)stream, a);
  } else
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
                                 float sm_scale, void* out, long out_stride, int out_is_f32,
                                 const float* qsk, void* stream) {
  if (!out || (q_stride % 8) != 0) return OA_EINVAL;
  return launch(true, q, q_stride, K, V, kv_stride_b, kv_stride_s, rows, kv_rows, head_dim, asg,
                asg_stride, sel, sel_stride, n_sel, exp_idx, E, quota, n_t, Sk, Sv, C, sm_scale,
                out, out_stride, out_is_f32, nullptr, nullptr, nullptr, qsk, stream);
}

extern "C" int oa_residual(const void* K, const void* V, long kv_stride_b, long kv_stride_s,
                           int rows, int kv_rows, int head_dim, const int32_t* asg,
                           long asg_stride, const int32_t* sel, long sel_stride, int n_sel,
                           const int32_t* exp_idx, int E, const float* quota, const float* n_t,
                           const float* Sk, const float* Sv, int C, void* kbar_r, void* vbar_r,
                           float* log_n, void* stream) {
  if (!kbar_r || !vbar_r || !log_n) return OA_EINVAL;
  // the residual-only variant reads no query; K stands in so the pointer is valid
  return launch(false, K, 0, K, V, kv_stride_b, kv_stride_s, rows, kv_rows, head_dim, asg,
                asg_stride, sel, sel_stride, n_sel, exp_idx, E, quota, n_t, Sk, Sv, C, 0.f,
                nullptr, 0, 0, kbar_r, vbar_r, log_n, nullptr, stream);
}
