// Top eigenpairs of symmetric positive semi-definite 128 x 128 fp32 matrices: the a10 bases at
// prefill (U = the top-32 eigenvectors of each KV head's group-mean metric, W from the top-16
// eigenpairs of each query head's metric), which the reference obtains from torch.linalg.eigh
// (inference/methods_eager.py:519-528).
//
// Method: one-sided (Hestenes) Jacobi.  Pairs of columns (a, b) of A are rotated,
//   [a b] <- [a b] [[c, s], [-s, c]],  tan = t, t^2 + 2 zeta t - 1 = 0 (the smaller root),
//   zeta = (|b|^2 - |a|^2) / (2 a.b),
// which makes the pair orthogonal.  Repeated over every pair until each is orthogonal to a
// relative tolerance, A V = B holds with mutually orthogonal columns.  For A = Q diag(lambda) Q^T
// positive semi-definite, B = Q diag(lambda) (the columns are lambda_j q_j): the eigenvalues are
// the column norms and the eigenvectors the normalised columns, so V is never formed.  Only the
// lower triangle of M is read (torch.linalg.eigh's default).
//
// Layout: one workgroup of 256 threads per matrix.  A quad of lanes holds one column pair, each
// lane 32 rows of both columns in registers; one step rotates the 64 pairs at once.  A sweep of
// 127 steps meets every two columns once, by recursive halving: at level l = 0..6 the columns
// form 2^l blocks, each split into halves H0 | H1 held as (a, b) by h = 64 >> l quads, and the
// block meets H0 x H1 in h steps, its b columns moving one quad along (through LDS) after each
// step.  Between levels the first h/2 quads of a block hand their b column to quad i + h/2 for
// its a column, so each new block again holds one column of each of its halves per quad.
// Each column's squared norm travels with it (recomputed at every sweep start), so a step forms
// one dot product, a.b, per pair; a pair counts as orthogonal when |a.b| <= kTol |a| |b| or when
// both columns are below 1e-6 |A|_F (numerically in the null space, where fp32 cannot resolve
// their angle).  Sweeps repeat until one applies no rotation (at most kMaxSweeps).  Every matrix
// runs the same fixed schedule on its own workgroup: results do not depend on the batch a
// matrix is in.
#include "oa_common.h"

namespace {

constexpr int kN = 128;
constexpr int kQuads = 64;
constexpr int kRows = 32;                      // rows of each column held by one lane
constexpr int kThreads = kQuads * 4;
constexpr int kSubStride = kRows + 4;          // floats per lane chunk in LDS (padded)
constexpr int kSlotStride = 4 * kSubStride;    // floats per column slot
constexpr int kMaxSweeps = 40;
constexpr int kMaxK = 64;
constexpr float kTol = 1e-5f;                  // |a.b| <= kTol |a| |b| counts as orthogonal

static_assert(kN * kMaxK <= kQuads * kSlotStride, "output staging fits the exchange buffer");

__device__ __forceinline__ float quad_sum(float v) {
  v = v + oa::dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + oa::dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  return v;
}
__device__ __forceinline__ double quad_sum(double v) {
  v = v + oa::dpp_f64<0xB1>(v);
  v = v + oa::dpp_f64<0x4E>(v);
  return v;
}
__device__ __forceinline__ int quad_sum(int v) {
  v += __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false);
  return v;
}

// squared norm of the column part a lane holds, summed over the quad
__device__ __forceinline__ float quad_norm2(const float (&a)[kRows]) {
  float x0 = 0.f, x1 = 0.f;
#pragma unroll
  for (int j = 0; j < kRows; j += 2) {
    x0 = fmaf(a[j], a[j], x0);
    x1 = fmaf(a[j + 1], a[j + 1], x1);
  }
  return quad_sum(x0 + x1);
}

// one Jacobi rotation of the quad's column pair, whose squared norms al, be are carried along
// (recomputed at every sweep start) and updated as al - t ga, be + t ga (the rotated pair's Gram
// diagonal); true if the pair was not yet orthogonal.  The rotation itself is skipped when no
// pair of the wave needs one.
__device__ __forceinline__ bool rotate_pair(float (&a)[kRows], float (&b)[kRows], float& al,
                                            float& be, float floor2) {
  float ga0 = 0.f, ga1 = 0.f;
#pragma unroll
  for (int j = 0; j < kRows; j += 2) {
    ga0 = fmaf(a[j], b[j], ga0);
    ga1 = fmaf(a[j + 1], b[j + 1], ga1);
  }
  // the quad's sum: every lane of the quad ends with the same bits
  const float ga = quad_sum(ga0 + ga1);
  // orthogonal to the tolerance, or both columns negligible against the matrix (their norms
  // below 1e-6 |A|_F: they cannot move the leading eigenvectors)
  const bool on = ga * ga > (kTol * kTol) * (al * be) && al + be > floor2;
  if (__ballot(on) == 0ull) return false;
  // the angle from the hardware reciprocal and square roots (about 1 ulp): an error there only
  // changes which orthogonal rotation is applied (c^2 + s^2 = 1 to about 2 ulp either way); for
  // ga = 0 the quotients are inf or NaN and the pair is not rotated
  const float zeta = (be - al) * __builtin_amdgcn_rcpf(2.f * ga);
  const float t = copysignf(
      __builtin_amdgcn_rcpf(fabsf(zeta) + __builtin_amdgcn_sqrtf(fmaf(zeta, zeta, 1.f))), zeta);
  const float cr = __builtin_amdgcn_rsqf(fmaf(t, t, 1.f));
  const float c = on ? cr : 1.f;
  const float s = on ? cr * t : 0.f;
  const float tg = on ? t * ga : 0.f;
  al = fmaxf(al - tg, 0.f);
  be = be + tg;
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const float x = a[j], y = b[j];
    a[j] = fmaf(c, x, -(s * y));
    b[j] = fmaf(s, x, c * y);
  }
  return on;
}

// a lane's part of a column and the column's squared norm (in the chunk's padding)
__device__ __forceinline__ void put32(float* p, const float (&v)[kRows], float n2) {
#pragma unroll
  for (int j = 0; j < kRows; j += 4)
    *reinterpret_cast<float4*>(p + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  p[kRows] = n2;
}
__device__ __forceinline__ float get32(const float* p, float (&v)[kRows]) {
#pragma unroll
  for (int j = 0; j < kRows; j += 4) {
    const float4 x = *reinterpret_cast<const float4*>(p + j);
    v[j] = x.x; v[j + 1] = x.y; v[j + 2] = x.z; v[j + 3] = x.w;
  }
  return p[kRows];
}

// element (r, c) of the symmetric matrix from the lower triangle of row-major M
__device__ __forceinline__ float sym_at(const float* M, int r, int c) {
  return r >= c ? M[r * kN + c] : M[c * kN + r];
}

__global__ __launch_bounds__(kThreads, 4) void sym_eig_top_kernel(const float* __restrict__ M,
                                                               long m_stride, int k,
                                                               float* __restrict__ ev,
                                                               float* __restrict__ evec,
                                                               int* __restrict__ sweeps_out) {
  __shared__ __align__(16) float s_x[kQuads * kSlotStride];
  __shared__ double s_nrm[2 * kQuads];
  __shared__ int s_flag[kThreads / OA_WAVE];
  __shared__ float s_fro[kThreads / OA_WAVE];
  const int m = blockIdx.x;
  const int tid = threadIdx.x, g = tid >> 2, sub = tid & 3;
  const float* A = M + (long)m * m_stride;
  const int r0 = sub * kRows;

  float a[kRows], b[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    a[j] = sym_at(A, r0 + j, g);
    b[j] = sym_at(A, r0 + j, g + kQuads);
  }
  float* mine = s_x + g * kSlotStride + sub * kSubStride;
  // |A|_F^2 (each quad's two columns, summed over the wave and then the four waves)
  {
    float f = 0.f;
#pragma unroll
    for (int j = 0; j < kRows; ++j) f = fmaf(a[j], a[j], fmaf(b[j], b[j], f));
    f = oa::wave_sum(f);
    if ((tid & (OA_WAVE - 1)) == 0) s_fro[tid / OA_WAVE] = f;
  }
  __syncthreads();
  const float floor2 = 1e-12f * ((s_fro[0] + s_fro[1]) + (s_fro[2] + s_fro[3]));

  int sweep = 0;
  bool more = true;
  while (more && sweep < kMaxSweeps) {
    unsigned long long any = 0;
    float al = quad_norm2(a), be = quad_norm2(b);
    for (int lev = 0; lev < 7; ++lev) {
      const int h = kQuads >> lev;
      const int i = g & (h - 1), g0 = g - i;
      const float* next = s_x + (g0 + ((i + 1) & (h - 1))) * kSlotStride + sub * kSubStride;
      for (int t = 0; t < h; ++t) {
        any |= __ballot(rotate_pair(a, b, al, be, floor2));
        if (t + 1 < h) {
          // quad i takes the b column of quad i + 1 (within the block)
          put32(mine, b, be);
          __syncthreads();
          be = get32(next, b);
          __syncthreads();
        }
      }
      if (lev < 6) {
        const int hb = h >> 1;
        const float* partner = s_x + (i < hb ? g + hb : g - hb) * kSlotStride + sub * kSubStride;
        if (i < hb)
          put32(mine, b, be);
        else
          put32(mine, a, al);
        __syncthreads();
        if (i < hb)
          be = get32(partner, b);
        else
          al = get32(partner, a);
        __syncthreads();
      }
    }
    ++sweep;
    if ((tid & (OA_WAVE - 1)) == 0) s_flag[tid / OA_WAVE] = any != 0ull;
    __syncthreads();
    more = (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) != 0;
  }

  // column norms in fp64 (slot g: the quad's a column, slot 64 + g: its b column)
  // (scheduling barriers every 8 rows keep the fp64 conversions from being hoisted all at once)
  double pa = 0.0, pb = 0.0;
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    pa = fma((double)a[j], (double)a[j], pa);
    pb = fma((double)b[j], (double)b[j], pb);
    if ((j & 7) == 7) __builtin_amdgcn_sched_barrier(0);
  }
  const double na = sqrt(quad_sum(pa)), nb = sqrt(quad_sum(pb));
  if (sub == 0) {
    s_nrm[g] = na;
    s_nrm[kQuads + g] = nb;
  }
  __syncthreads();
  // rank in descending norm, ties to the lower slot: each lane counts over a quarter of the slots
  int ra = 0, rb = 0;
#pragma unroll 4
  for (int j = sub * 32; j < sub * 32 + 32; ++j) {
    const double x = s_nrm[j];
    ra += (x > na) || (x == na && j < g);
    rb += (x > nb) || (x == nb && j < kQuads + g);
  }
  ra = quad_sum(ra);
  rb = quad_sum(rb);
  // the k largest, ascending (the largest in position k - 1), staged one output column per slot
  // for a coalesced store; a zero column (a zero eigenvalue among the k) is stored as zeros
  if (ra < k) {
    const int p = k - 1 - ra;
    const float inv = na > 0.0 ? (float)(1.0 / na) : 0.f;
#pragma unroll
    for (int j = 0; j < kRows; ++j) a[j] *= inv;
    put32(s_x + p * kSlotStride + sub * kSubStride, a, 0.f);
    if (sub == 0) ev[(long)m * k + p] = (float)na;
  }
  if (rb < k) {
    const int p = k - 1 - rb;
    const float inv = nb > 0.0 ? (float)(1.0 / nb) : 0.f;
#pragma unroll
    for (int j = 0; j < kRows; ++j) b[j] *= inv;
    put32(s_x + p * kSlotStride + sub * kSubStride, b, 0.f);
    if (sub == 0) ev[(long)m * k + p] = (float)nb;
  }
  __syncthreads();
  float* out = evec + (long)m * kN * k;
  for (int e = tid; e < kN * k; e += kThreads) {
    const int row = e / k, p = e - row * k;
    out[e] = s_x[p * kSlotStride + (row / kRows) * kSubStride + row % kRows];
  }
  if (sweeps_out && tid == 0) sweeps_out[m] = more ? -sweep : sweep;
}

}  // namespace

extern "C" int oa_sym_eig_top(const float* M, long m_stride, int batch, int n, int k, float* evals,
                              float* evecs, int* sweeps, void* stream) {
  if (batch < 0 || n != kN || k < 1 || k > kMaxK || m_stride < (long)kN * kN || !M || !evals ||
      !evecs)
    return OA_EINVAL;
  if (batch == 0) return 0;
  hipLaunchKernelGGL(sym_eig_top_kernel, dim3(batch), dim3(kThreads), 0, (hipStream_t)stream, M,
                     m_stride, k, evals, evecs, sweeps);
  return OA_LAUNCH_STATUS();
}
