// Dense bf16 decode attention (the comparator of the sparse stage), split-K over the keys
// with the length n read from device memory.
//
// Reference comparator: _k_dense_split + _k_dense_combine (inference/graph_runner.py:259-312)
// and torch SDPA over the whole cache (bench_flash_latency.py:93-97).
//
// gfx950 decomposition: grid (splits, B*HKV); a 256-thread workgroup streams one contiguous
// key chunk of one KV head for all G=4 query heads of that head, so every K/V byte is read
// once per KV head.  16 lane groups of 16 lanes each take four keys per round (one 16-byte K
// and one 16-byte V load per lane and key, all eight issued first; q.k on the packed bf16 dot
// instructions, fp32 accumulation), keep four online softmaxes
// (one per query head, rescaled once per round), and merge in a fixed order; partial
// (m, l, acc) go to the caller's workspace and a combine kernel finishes the rows.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;
constexpr int GQ = 4;
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 __attribute__((ext_vector_type(2))) bf16x2;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (read once: non-temporal)
__device__ __forceinline__ uint4 load_nt16(const uint16_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// dot of 8 bf16 pairs held as four packed words (v_dot2_f32_bf16, fp32 accumulation)
__device__ __forceinline__ float dot8_bf16(const uint4 a, const uint4 b) {
  float p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.x), __builtin_bit_cast(bf16x2, b.x),
                                            0.f, false);
  p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.y), __builtin_bit_cast(bf16x2, b.y), p, false);
  p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.z), __builtin_bit_cast(bf16x2, b.z), p, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.w), __builtin_bit_cast(bf16x2, b.w), p, false);
}

__global__ void __launch_bounds__(kThreads) dense_split_kernel(
    const uint16_t* __restrict__ q, long q_stride, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, long kv_sb, long kv_ss, const int* __restrict__ n_dev,
    int chunk, int nsplit, float sm_scale, float* __restrict__ ws_m, float* __restrict__ ws_l,
    float* __restrict__ ws_acc) {
  const int split = blockIdx.x;
  const int kvr = blockIdx.y;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;
  const int sub = tid & 15;
  const int d0 = sub * 8;
  const int n = *n_dev;
  const int t0 = split * chunk;
  const int t1 = min(n, t0 + chunk);
  uint4 qv[GQ];                       // the four query heads' 8 dims, packed bf16 pairs
#pragma unroll
  for (int g = 0; g < GQ; ++g)
    qv[g] = *reinterpret_cast<const uint4*>(q + (long)(kvr * GQ + g) * q_stride + d0);
  const float zs = sm_scale * kLog2e;
  float m[GQ], l[GQ], acc[GQ][8];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    m[g] = -INFINITY; l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }
  const uint16_t* Kb = K + (long)kvr * kv_sb + d0;
  const uint16_t* Vb = V + (long)kvr * kv_sb + d0;
  // each lane group takes kKeys keys per round (keys t, t + 16, ...): all their K and V loads
  // are issued before any arithmetic, and the running maximum is rescaled once per round
  constexpr int kKeys = 4;
  for (int tb = t0 + grp; tb < t1; tb += kGroups * kKeys) {
    uint4 kw[kKeys], vw[kKeys];
    bool ok[kKeys];
#pragma unroll
    for (int u = 0; u < kKeys; ++u) {
      const int t = tb + u * kGroups;
      ok[u] = t < t1;
      const long off = (long)(ok[u] ? t : t0) * kv_ss;
      kw[u] = load_nt16(Kb + off);
      vw[u] = load_nt16(Vb + off);
    }
    float z[GQ][kKeys];
#pragma unroll
    for (int u = 0; u < kKeys; ++u) {
#pragma unroll
      for (int g = 0; g < GQ; ++g)
        z[g][u] = ok[u] ? oa::group16_sum(dot8_bf16(qv[g], kw[u])) * zs : -INFINITY;
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      float mn = m[g];
#pragma unroll
      for (int u = 0; u < kKeys; ++u) mn = fmaxf(mn, z[g][u]);
      const float al = exp2f(m[g] - mn);
      l[g] *= al;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] *= al;
      m[g] = mn;
    }
#pragma unroll
    for (int u = 0; u < kKeys; ++u) {
      float vx[8];
      oa::unpack8(vw[u], vx);
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        // key u = 0 of a round is always valid, so m[g] is finite here; masked keys weigh 0
        const float pe = ok[u] ? exp2f(z[g][u] - m[g]) : 0.f;
        l[g] += pe;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(pe, vx[i], acc[g][i]);
      }
    }
  }
  __shared__ float s_m[GQ][kGroups], s_l[GQ][kGroups];
  __shared__ float s_acc[GQ][kGroups][OA_D];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    if (sub == 0) { s_m[g][grp] = m[g]; s_l[g][grp] = l[g]; }
#pragma unroll
    for (int i = 0; i < 8; ++i) s_acc[g][grp][d0 + i] = acc[g][i];
  }
  __syncthreads();
  for (int e = tid; e < GQ * OA_D; e += kThreads) {
    const int g = e / OA_D, d = e % OA_D;
    float M = -INFINITY;
    for (int j = 0; j < kGroups; ++j) M = fmaxf(M, s_m[g][j]);
    float L = 0.f, A = 0.f;
    if (M > -INFINITY) {
      for (int j = 0; j < kGroups; ++j) {
        if (s_m[g][j] > -INFINITY) {
          const float w = exp2f(s_m[g][j] - M);
          L = fmaf(s_l[g][j], w, L);
          A = fmaf(s_acc[g][j][d], w, A);
        }
      }
    }
    const long pr = (long)(kvr * GQ + g) * nsplit + split;
    if (d == 0) { ws_m[pr] = M; ws_l[pr] = L; }
    ws_acc[pr * OA_D + d] = A;
  }
}

__global__ void __launch_bounds__(OA_D) dense_combine_kernel(const float* ws_m, const float* ws_l,
                                                             const float* ws_acc, int nsplit,
                                                             uint16_t* out, long out_stride) {
  const int row = blockIdx.x;
  const int d = threadIdx.x;
  const long base = (long)row * nsplit;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ws_m[base + s]);
  float L = 0.f, A = 0.f;
  if (M > -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ms = ws_m[base + s];
      if (ms > -INFINITY) {
        const float w = exp2f(ms - M);
        L = fmaf(ws_l[base + s], w, L);
        A = fmaf(ws_acc[(base + s) * OA_D + d], w, A);
      }
    }
  }
  out[(long)row * out_stride + d] = oa::f32_to_bf16(L > 0.f ? A / L : 0.f);
}

}  // namespace

extern "C" int oa_dense_decode(const void* q, long q_stride, const void* K, const void* V,
                               long kv_stride_b, long kv_stride_s, int rows, int kv_rows,
                               int head_dim, int Lmax, const int* n_dev, float sm_scale, int nsplit,
                               float* ws_m, float* ws_l, float* ws_acc, void* out, long out_stride,
                               void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows != kv_rows * GQ || nsplit < 1 || Lmax <= 0 ||
      !ws_m || !ws_l || !ws_acc)
    return OA_EINVAL;
  const int chunk = (Lmax + nsplit - 1) / nsplit;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(dense_split_kernel, dim3(nsplit, kv_rows), dim3(kThreads), 0, s,
                     (const uint16_t*)q, q_stride, (const uint16_t*)K, (const uint16_t*)V,
                     kv_stride_b, kv_stride_s, n_dev, chunk, nsplit, sm_scale, ws_m, ws_l, ws_acc);
  int st = OA_LAUNCH_STATUS();
  if (st) return st;
  hipLaunchKernelGGL(dense_combine_kernel, dim3(rows), dim3(OA_D), 0, s, ws_m, ws_l, ws_acc, nsplit,
                     (uint16_t*)out, out_stride);
  return OA_LAUNCH_STATUS();
}
