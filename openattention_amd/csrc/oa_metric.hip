// The a10 query metric of every query-head row of a build, on the device: the moment of the
// row's question rows advanced to the decode position, trace-normalised and blended with the
// (per head) rotated static metric, and each KV row's group mean (methods_eager.py:510-519;
// static_top_k.py:185-194).  For question row q_p (p over the picked rows, P of them), advanced
// by its own RoPE angle,
//   r_p = s (cos_p * q_p + sin_p * rotate_half(q_p))                     (fp64)
//   Mq  = fp32((sum_p r_p r_p^T) / P)                                    (fp64 sums over p in order)
//   M   = mst_half + 0.5 (Mq / max(tr Mq, 1e-12))                        (fp32; tr summed in order)
//   Mg  = (M_0 + M_1 + ... + M_{G-1}) / G over a KV row's G query rows   (fp32, in order)
// mst_half = 1/2 nt(the rotated static metric) is formed once per layer on the host side.
// One 256-thread workgroup per KV row: the picked rows of one query row at a time in LDS (fp64),
// each thread an 8 x 8 block of the 128 x 128 moment.
#include "oa_common.h"

namespace {

constexpr int kN = 128;
constexpr int kMaxP = 64;
constexpr int kThreads = 256;

template <bool BF16>
__device__ __forceinline__ double q_at(const void* q, long idx) {
  if (BF16) return (double)oa::bf16_to_f32(static_cast<const uint16_t*>(q)[idx]);
  return (double)static_cast<const float*>(q)[idx];
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void query_metric_kernel(
    const void* __restrict__ q, long q_sr, long q_sp, int G, const int* __restrict__ pick, int P,
    const double* __restrict__ cosv, const double* __restrict__ sinv, double scaling,
    const float* __restrict__ mst_half, int heads, float* __restrict__ gm_out,
    float* __restrict__ m_out) {
  __shared__ __align__(16) double s_r[kMaxP * kN];
  __shared__ float s_diag[kN];
  __shared__ float s_tr;
  const int kvr = blockIdx.x;
  const int t = threadIdx.x;
  const int i0 = (t >> 4) * 8, j0 = (t & 15) * 8;
  float gm[8][8];
  for (int h = 0; h < G; ++h) {
    const int row = kvr * G + h;
    if (h) __syncthreads();             // the previous row's reads of s_r and s_tr are done
    for (int e = t; e < P * kN; e += kThreads) {
      const int p = e / kN, d = e % kN;
      const long base = (long)row * q_sr + (long)pick[p] * q_sp;
      const double x = q_at<BF16>(q, base + d);
      const double xh = d < kN / 2 ? -q_at<BF16>(q, base + d + kN / 2) : q_at<BF16>(q, base + d - kN / 2);
      const double c = cosv[p * kN + d] * x;
      const double sn = sinv[p * kN + d] * xh;
      s_r[e] = scaling * (c + sn);
    }
    __syncthreads();
    double acc[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[a][b] = 0.0;
    for (int p = 0; p < P; ++p) {
      double ra[8], rb[8];
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        const double2 x = *reinterpret_cast<const double2*>(&s_r[p * kN + i0 + k]);
        const double2 y = *reinterpret_cast<const double2*>(&s_r[p * kN + j0 + k]);
        ra[k] = x.x; ra[k + 1] = x.y;
        rb[k] = y.x; rb[k + 1] = y.y;
      }
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[a][b] = fma(ra[a], rb[b], acc[a][b]);
    }
    float mq[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) mq[a][b] = (float)(acc[a][b] / (double)P);
    if (i0 == j0) {
#pragma unroll
      for (int a = 0; a < 8; ++a) s_diag[i0 + a] = mq[a][a];
    }
    __syncthreads();
    if (t == 0) {
      float tr = 0.f;
      for (int i = 0; i < kN; ++i) tr = tr + s_diag[i];
      s_tr = fmaxf(tr, 1e-12f);
    }
    __syncthreads();
    const float tr = s_tr;
    const float* ms = mst_half + (long)(row % heads) * kN * kN;
    float* mo = m_out + (long)row * kN * kN;
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      float v[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        v[b] = ms[(i0 + a) * kN + j0 + b] + 0.5f * (mq[a][b] / tr);
        gm[a][b] = h ? gm[a][b] + v[b] : v[b];
      }
      float4* dst = reinterpret_cast<float4*>(mo + (i0 + a) * kN + j0);
      dst[0] = make_float4(v[0], v[1], v[2], v[3]);
      dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  float* go = gm_out + (long)kvr * kN * kN;
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    float v[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = gm[a][b] / (float)G;
    float4* dst = reinterpret_cast<float4*>(go + (i0 + a) * kN + j0);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

}  // namespace

extern "C" int oa_query_metric(const void* q, int q_bf16, long q_stride_row, long q_stride_pos, int rows,
                               int G, const int32_t* pick, int P, const double* cosv, const double* sinv,
                               double scaling, const float* mst_half, int heads, float* gm_out,
                               float* m_out, void* stream) {
  if (rows <= 0 || G <= 0 || G > 8 || rows % G || P < 1 || P > kMaxP || heads <= 0 || !q || !pick ||
      !cosv || !sinv || !mst_half || !gm_out || !m_out || q_stride_pos < kN ||
      (reinterpret_cast<uintptr_t>(gm_out) & 15) || (reinterpret_cast<uintptr_t>(m_out) & 15))
    return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (q_bf16)
    hipLaunchKernelGGL(query_metric_kernel<true>, dim3(rows / G), dim3(kThreads), 0, s, q, q_stride_row,
                       q_stride_pos, G, pick, P, cosv, sinv, scaling, mst_half, heads, gm_out, m_out);
  else
    hipLaunchKernelGGL(query_metric_kernel<false>, dim3(rows / G), dim3(kThreads), 0, s, q, q_stride_row,
                       q_stride_pos, G, pick, P, cosv, sinv, scaling, mst_half, heads, gm_out, m_out);
  return OA_LAUNCH_STATUS();
}
