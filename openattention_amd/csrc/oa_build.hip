// Prefill index build on gfx950: QGS codes, QGC projection, k-means (assign / update), and the
// cluster statistics with their CSR member lists.  One request (batch row) at a time: kv_rows
// KV-head rows and rows = G * kv_rows query-head rows; query row r reads KV row r / G.
//
// Reference: the fast build of inference/ours_fastbuild.py:236-304 and the eager build of
// inference/methods_eager.py:505-555, with the accuracy-path semantics where they differ:
//   codes    zc = k U (fp32), scale = max(max_t |zc| / 127, 1e-12) per (KV head, coordinate),
//            codes = clamp(rint(zc / scale), -127, 127)  (static_top_k.py:174-181)
//   project  zP = bf16(k W) - colmean, colmean = mean_t bf16(k W)  (methods_eager.py:526-531,
//            ours_fastbuild.py:264-275)
//   assign   a_t = argmax_c bf16(bf16(bf16(zP_t) . bf16(c)) - bf16(|c|^2 / 2)), ties to the lower
//            cluster  (ours_fastbuild.py:52-82, methods_eager.py:536-540)
//   update   c = mean of the members, an empty cluster keeps its initial point
//            (ours_fastbuild.py:85-108, methods_eager.py:541-547)
//   sums     n_c, Sk_c = sum k, Sk2_c = sum k*k, Sv_c = sum v over the members; member lists =
//            stable argsort of the assignment  (ours_fastbuild.py:111-139, 293-301)
//
// Orders.  The reference leaves every summation order to its libraries.  This build fixes one
// wherever a CPU restatement has to match it bit for bit:
//   codes    zc_r = fma chain over d = 0..127 in fp32 (z = fma(k_d, U_dr, z), from z = 0);
//   colmean  per 64-token tile an fp64 sum in a fixed lane order, the tiles summed in order,
//            then one rounding of sum / T to fp32;
//   update   per cluster an fp64 sum of the members in position order, one rounding of
//            sum / count to fp32;
//   sums     per cluster fp64 sums of k, k*k and v over the members in position order, one
//            rounding to fp32.
// The two matrix products of the QGC step (k W and zP . c) run on the bf16 matrix cores with
// fp32 accumulation, as the reference's bf16 matmuls do; their fp32 partial rounding is the
// hardware's, so the CPU restatement matches them up to an agreement rate (ties of the bf16
// result), not bit for bit.
#include <algorithm>

#include "oa_common.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short short4v;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float float4v;

constexpr int kD = 128;
constexpr int kRQ = 32;       // QGS rank
constexpr int kRC = 16;       // QGC rank
constexpr int kMaxC = 256;

__device__ __forceinline__ __bf16 bits_bf16(uint16_t h) { return __builtin_bit_cast(__bf16, h); }

// ---------------------------------------------------------------------------------- codes
// zc of one token (one lane) against U in LDS (U[d][r], 128 x 32 floats): fma chain over d
__device__ __forceinline__ void token_zc(const uint16_t* krow, const float* sU, float z[kRQ]) {
#pragma unroll
  for (int r = 0; r < kRQ; ++r) z[r] = 0.f;
  for (int d0 = 0; d0 < kD; d0 += 8) {
    const uint4 w = *reinterpret_cast<const uint4*>(krow + d0);
    float kv[8];
    oa::unpack8(w, kv);
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const float4* u4 = reinterpret_cast<const float4*>(sU + (d0 + dd) * kRQ);
#pragma unroll
      for (int r4 = 0; r4 < kRQ / 4; ++r4) {
        const float4 u = u4[r4];
        z[4 * r4] = fmaf(kv[dd], u.x, z[4 * r4]);
        z[4 * r4 + 1] = fmaf(kv[dd], u.y, z[4 * r4 + 1]);
        z[4 * r4 + 2] = fmaf(kv[dd], u.z, z[4 * r4 + 2]);
        z[4 * r4 + 3] = fmaf(kv[dd], u.w, z[4 * r4 + 3]);
      }
    }
  }
}

constexpr int kCodeThreads = 256;

__global__ void __launch_bounds__(64) clear_u32_kernel(uint32_t* p, int n) {
  for (int i = threadIdx.x + blockIdx.x * 64; i < n; i += 64 * gridDim.x) p[i] = 0u;
}

// pass 1: per (KV row, coordinate) the maximum |zc| over the tokens, as float bits (|zc| >= 0,
// so the unsigned maximum of the bits is the float maximum); zc itself into zc_ws when given
// (128 bytes per token), so that pass 2 quantizes without a second fma chain
// The block's 256 key rows are staged through LDS, 64 dims at a time (coalesced 128-byte row
// segments, rows padded to 144 bytes so that a 16-lane phase of row reads hits distinct banks):
// a lane walking its own row straight from memory touched 64 lines per load and lost them to
// the other rows before its next step (5.5x the keys' bytes fetched).  U's rows come through
// scalar loads (the same for every lane; the fmas take them from SGPRs) rather than LDS
// broadcasts, which bounded the pass by LDS bandwidth.  The fma chain over d is token_zc's, in
// the same order.
constexpr int kZcDims = 64;                    // dims staged per pass
constexpr int kZcRowQ = kZcDims / 8 + 1;       // uint4 per staged row (8 + 1 pad)

__global__ void __launch_bounds__(kCodeThreads) codes_amax_kernel(const uint16_t* __restrict__ K, long ksh,
                                                                  long kst, int T,
                                                                  const float* __restrict__ U,
                                                                  uint32_t* __restrict__ amax,
                                                                  float* __restrict__ zc_ws) {
  __shared__ uint32_t s_m[kRQ];
  __shared__ uint4 s_k[kCodeThreads * kZcRowQ];
  const int h = blockIdx.y;
  const float* __restrict__ Uh = U + (long)h * kD * kRQ;
  if (threadIdx.x < kRQ) s_m[threadIdx.x] = 0u;
  const int t0 = blockIdx.x * kCodeThreads;
  const int t = t0 + threadIdx.x;
  const uint16_t* kh = K + (long)h * ksh;
  float z[kRQ];
#pragma unroll
  for (int r = 0; r < kRQ; ++r) z[r] = 0.f;
  for (int d0 = 0; d0 < kD; d0 += kZcDims) {
    if (d0) __syncthreads();   // every lane has read the previous dims
#pragma unroll
    for (int j = 0; j < kZcDims / 8; ++j) {
      const int i = threadIdx.x + j * kCodeThreads;
      const int r = i / (kZcDims / 8), c = i % (kZcDims / 8);
      s_k[r * kZcRowQ + c] =
          *reinterpret_cast<const uint4*>(kh + (long)min(t0 + r, T - 1) * kst + d0 + 8 * c);
    }
    __syncthreads();
    for (int c = 0; c < kZcDims / 8; ++c) {
      float kv[8];
      oa::unpack8(s_k[threadIdx.x * kZcRowQ + c], kv);
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        const float* ud = Uh + (d0 + 8 * c + dd) * kRQ;
#pragma unroll
        for (int r = 0; r < kRQ; ++r) z[r] = fmaf(kv[dd], ud[r], z[r]);
      }
    }
  }
  const bool in = t < T;
  if (zc_ws && in) {
    float4* zo = reinterpret_cast<float4*>(zc_ws + ((long)h * T + t) * kRQ);
#pragma unroll
    for (int r4 = 0; r4 < kRQ / 4; ++r4) zo[r4] = make_float4(z[4 * r4], z[4 * r4 + 1], z[4 * r4 + 2], z[4 * r4 + 3]);
  }
#pragma unroll
  for (int r = 0; r < kRQ; ++r) {
    const unsigned m = oa::wave_max_u32(in ? __float_as_uint(fabsf(z[r])) : 0u);
    if ((threadIdx.x & 63) == 0) atomicMax(&s_m[r], m);
  }
  __syncthreads();
  if (threadIdx.x < kRQ) atomicMax(&amax[h * kRQ + threadIdx.x], s_m[threadIdx.x]);
}

// pass 2: the codes (32 bytes per token) and, from the first block of each KV row, the scale
__global__ void __launch_bounds__(kCodeThreads) codes_write_kernel(const uint16_t* K, long ksh, long kst,
                                                                   int T, const float* U,
                                                                   const uint32_t* amax, int8_t* codes,
                                                                   long csh, float* scale,
                                                                   const float* zc_ws) {
  __shared__ float sU[kD * kRQ];
  __shared__ float s_sc[kRQ];
  const int h = blockIdx.y;
  for (int i = threadIdx.x; i < kD * kRQ; i += kCodeThreads) sU[i] = U[(long)h * kD * kRQ + i];
  if (threadIdx.x < kRQ) {
    const float sc = fmaxf(__uint_as_float(amax[h * kRQ + threadIdx.x]) / 127.0f, 1e-12f);
    s_sc[threadIdx.x] = sc;
    if (blockIdx.x == 0) scale[h * kRQ + threadIdx.x] = sc;
  }
  __syncthreads();
  const int t = blockIdx.x * kCodeThreads + threadIdx.x;
  if (t >= T) return;
  float z[kRQ];
  if (zc_ws) {
    const float4* zi = reinterpret_cast<const float4*>(zc_ws + ((long)h * T + t) * kRQ);
#pragma unroll
    for (int r4 = 0; r4 < kRQ / 4; ++r4) {
      const float4 v = zi[r4];
      z[4 * r4] = v.x; z[4 * r4 + 1] = v.y; z[4 * r4 + 2] = v.z; z[4 * r4 + 3] = v.w;
    }
  } else {
    token_zc(K + (long)h * ksh + (long)t * kst, sU, z);
  }
  uint32_t packed[kRQ / 4];
#pragma unroll
  for (int r4 = 0; r4 < kRQ / 4; ++r4) {
    uint32_t w = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = fminf(fmaxf(rintf(z[4 * r4 + j] / s_sc[4 * r4 + j]), -127.f), 127.f);
      w |= ((uint32_t)(uint8_t)(int8_t)(int)q) << (8 * j);
    }
    packed[r4] = w;
  }
  uint4* dst = reinterpret_cast<uint4*>(codes + (long)h * csh + (long)t * kRQ);
  dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// ---------------------------------------------------------------------------------- projection
constexpr int kProjTiles = 8;    // 64-token tiles per wave (the row's W operands loaded once)
// One wave per (8 64-token tiles, query row or KV row).  Four 16-token blocks, each 16 tokens x 16 columns
// from four v_mfma_f32_16x16x32_bf16 over d = 0..127 (A: token rows of K, B: the row's W).
// Output layout of a 16x16 block: lane l holds tokens 4*(l/16) + i (i = 0..3) of column l % 16.
// zraw = bf16(acc) is written (as fp32) into zP, and the tile's column sums (fp64, lane order
// below) into tsum[row][tile][16].
// NG query rows per wave (NG == G: a KV row's query rows, whose K blocks are then loaded once for
// all of them; NG == 1: blockIdx.y is the query row).
template <int NG>
__global__ void __launch_bounds__(64) qgc_project_kernel(const uint16_t* K, long ksh, long kst, int G,
                                                         int T, const uint16_t* W, float* zP,
                                                         long zps, uint16_t* zraw_out, double* tsum,
                                                         int ntiles) {
  __shared__ uint4 s_z[NG][64 * kRC / 8];         // the tile's bf16(k W), token rows of 32 bytes
  const int lane = threadIdx.x;
  const int row0 = NG == 1 ? (int)blockIdx.y : (int)blockIdx.y * G;
  const uint16_t* krow = K + (long)(row0 / G) * ksh;
  // B operand of chunk ch: column j = lane % 16, dims ch*32 + 8*(lane/16) + e, e = 0..7
  bf16x8 bw[NG][4];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        bw[g][ch][e] = bits_bf16(W[(long)(row0 + g) * kD * kRC + (ch * 32 + 8 * (lane >> 4) + e) * kRC + (lane & 15)]);
  const int tend = min(ntiles, (int)(blockIdx.x + 1) * kProjTiles);
#pragma unroll 1
  for (int tile = blockIdx.x * kProjTiles; tile < tend; ++tile) {
  double cs[NG];   // this lane's column (lane % 16) partial over its tokens, in block order
#pragma unroll
  for (int g = 0; g < NG; ++g) cs[g] = 0.0;
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int t0 = tile * 64 + blk * 16;
    const int ta = min(t0 + (lane & 15), T - 1);          // A row: token t0 + lane % 16
    uint4 av[4];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
      av[ch] = *reinterpret_cast<const uint4*>(krow + (long)ta * kst + ch * 32 + 8 * (lane >> 4));
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ch = 0; ch < 4; ++ch)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[ch]), bw[g][ch], acc, 0, 0, 0);
      uint16_t* s_zh = reinterpret_cast<uint16_t*>(s_z[g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 4 * (lane >> 4) + i;
        const uint16_t hb = oa::f32_to_bf16_rn(acc[i]);
        const float v = oa::bf16_to_f32(hb);
        s_zh[(blk * 16 + 4 * (lane >> 4) + i) * kRC + (lane & 15)] = hb;
        if (t < T) {
          if (zP) zP[(long)(row0 + g) * zps + (long)t * kRC + (lane & 15)] = v;
          cs[g] += (double)v;
        }
      }
    }
  }
  // the tile's rows out through LDS: lane l writes token l's 32 bytes
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (zraw_out) {
    const int t = tile * 64 + lane;
    if (t < T) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        uint4* dst = reinterpret_cast<uint4*>(zraw_out + (long)(row0 + g) * zps + (long)t * kRC);
        dst[0] = s_z[g][lane * 2];
        dst[1] = s_z[g][lane * 2 + 1];
      }
    }
  }
  // lanes j, 16 + j, 32 + j, 48 + j hold column j: ((g0 + g1) + (g2 + g3))
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    double c = cs[g];
    c += __shfl_xor(c, 16, 64);
    c += __shfl_xor(c, 32, 64);
    if (lane < 16) tsum[((long)(row0 + g) * ntiles + tile) * kRC + lane] = c;
  }
  // the next tile's stores to s_z wait for these reads
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  }
}

// colmean from the tile sums (tiles in order, fp64): one wave per row, lane j < 16 a column; the
// sums of 16 tiles are requested together and then added in tile order (one load in flight at a
// time left the pass bound by memory latency: 0.21 ms at 512 tiles, 0.44 ms at 2048)
__global__ void __launch_bounds__(64) qgc_colmean_kernel(int T, const double* tsum, int ntiles,
                                                         float* colmean) {
  constexpr int kBatch = 16;
  const int row = blockIdx.x;
  const int j = threadIdx.x;
  if (j < kRC) {
    const double* p = tsum + (long)row * ntiles * kRC + j;
    double s = 0.0;
    int k = 0;
    for (; k + kBatch <= ntiles; k += kBatch) {
      double x[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) x[u] = p[(long)(k + u) * kRC];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) s += x[u];
    }
    for (; k < ntiles; ++k) s += p[(long)k * kRC];
    colmean[row * kRC + j] = (float)(s / (double)T);
  }
}

// zP -= colmean in place (float4 per thread: four columns of one token)
__global__ void __launch_bounds__(256) qgc_center_kernel(float* zP, long zps, int T,
                                                         const float* colmean) {
  const int row = blockIdx.y;
  const float* cm = colmean + row * kRC;
  float4* z = reinterpret_cast<float4*>(zP + (long)row * zps);
  const long n4 = (long)T * (kRC / 4);
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
    const int c4 = (int)(i & 3) * 4;
    float4 v = z[i];
    v.x = v.x - cm[c4];
    v.y = v.y - cm[c4 + 1];
    v.z = v.z - cm[c4 + 2];
    v.w = v.w - cm[c4 + 3];
    z[i] = v;
  }
}

// ---------------------------------------------------------------------------------- k-means
// two fp32 values rounded to bf16 (nearest even) in one conversion: a in the low half
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2v;
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}

// One 256-thread workgroup per (kAsgTiles 64-token tiles, query row): the row's centroids (bf16,
// B operands: centroid lane % 16 of a 16-centroid block, dims 4*(lane/16)..+3) and
// bf16(|c|^2 / 2) are staged in LDS once and every wave then takes every fourth tile.
// Per 16-token block and centroid block one v_mfma_f32_16x16x16bf16_1k gives 16 x 16 dots;
// the distance bf16(bf16(dot) - half) is ranked through the key (bf16 key << 16 | 255 - c), so the
// maximum over the 16 centroid lanes (a DPP row) and over the blocks is the argmax with ties to
// the lower cluster.
constexpr int kAsgThreads = 256;
constexpr int kAsgTiles = 32;
__global__ void __launch_bounds__(kAsgThreads) kmeans_assign_kernel(const uint16_t* zraw,
                                                                    const float* colmean, long zps, int T,
                                                                    const float* cent, int C,
                                                                    int32_t* asg, long as,
                                                                    uint8_t* asg8, long a8s) {
  __shared__ uint16_t s_cb[kMaxC * kRC];
  __shared__ uint16_t s_half[kMaxC];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.y;
  const int CB = (C + 15) / 16;
  const int ntiles = (T + 63) / 64;
  const float* cr = cent + (long)row * C * kRC;
  // four centroid values per thread and iteration (C * kRC is a multiple of 4)
  for (int i = 4 * threadIdx.x; i < CB * 16 * kRC; i += 4 * kAsgThreads) {
    if (i < C * kRC) {
      const float4 x = *reinterpret_cast<const float4*>(cr + i);
      s_cb[i] = oa::f32_to_bf16(x.x);
      s_cb[i + 1] = oa::f32_to_bf16(x.y);
      s_cb[i + 2] = oa::f32_to_bf16(x.z);
      s_cb[i + 3] = oa::f32_to_bf16(x.w);
    } else {
      s_cb[i] = s_cb[i + 1] = s_cb[i + 2] = s_cb[i + 3] = 0;
    }
  }
  int zero_half = 0;          // this thread staged a real centroid with bf16(|c|^2 / 2) = +0
  for (int c = threadIdx.x; c < CB * 16; c += kAsgThreads) {
    uint16_t hv = 0x7f80u;   // padding centroids: +inf, a distance of -inf ranks below every real one
    if (c < C) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < kRC; ++j) {
        const float x = cr[c * kRC + j];
        s = s + x * x;
      }
      hv = oa::f32_to_bf16(0.5f * s);
      zero_half |= hv == 0;
    }
    s_half[c] = hv;
  }
  // bf16(x - half) is -0 only for half = +0 (x - x rounds to +0): without such a centroid the
  // distances need no -0 -> +0 step, and their keys are formed two at a time from the packed pair
  const bool fast = __syncthreads_or(zero_half) == 0;
  // zP = bf16(k W) - colmean, formed from the stored bf16 projection (the same fp32 values)
  float cm[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) cm[e] = colmean[row * kRC + 4 * (lane >> 4) + e];
  const int tend = min(ntiles, (blockIdx.x + 1) * kAsgTiles);
  for (int tile = blockIdx.x * kAsgTiles + wave; tile < tend; tile += kAsgThreads / 64) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int t0 = tile * 64 + blk * 16;
      const int ta = min(t0 + (lane & 15), T - 1);
      const uint2 zr =
          *reinterpret_cast<const uint2*>(zraw + (long)row * zps + (long)ta * kRC + 4 * (lane >> 4));
      short4v a;
      a[0] = (short)oa::f32_to_bf16_rn(__uint_as_float(zr.x << 16) - cm[0]);
      a[1] = (short)oa::f32_to_bf16_rn(__uint_as_float(zr.x & 0xffff0000u) - cm[1]);
      a[2] = (short)oa::f32_to_bf16_rn(__uint_as_float(zr.y << 16) - cm[2]);
      a[3] = (short)oa::f32_to_bf16_rn(__uint_as_float(zr.y & 0xffff0000u) - cm[3]);
      uint32_t best[4] = {0u, 0u, 0u, 0u};
      for (int cb = 0; cb < CB; ++cb) {
        const int c = cb * 16 + (lane & 15);
        const uint16_t* bp = s_cb + c * kRC + 4 * (lane >> 4);
        short4v b;
        b[0] = (short)bp[0]; b[1] = (short)bp[1]; b[2] = (short)bp[2]; b[3] = (short)bp[3];
        float4v acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
        const float hf = oa::bf16_to_f32(s_half[c]);
        // bf16(bf16(dot) - half), two values per conversion; + 0 turns -0 into +0 (one score); the
        // key is the distance's order-preserving key (its top 16 bits: the bf16 key) with the tag
        // 255 - c below it
        const uint32_t tag = (uint32_t)(255 - c);
        const uint32_t p01 = cvt_pk_bf16(acc[0], acc[1]), p23 = cvt_pk_bf16(acc[2], acc[3]);
        const uint32_t q01 = cvt_pk_bf16(__uint_as_float(p01 << 16) - hf, __uint_as_float(p01 & 0xffff0000u) - hf);
        const uint32_t q23 = cvt_pk_bf16(__uint_as_float(p23 << 16) - hf, __uint_as_float(p23 & 0xffff0000u) - hf);
        if (fast) {
          // the order-preserving key of each bf16 half (negative: every bit flipped; otherwise
          // the sign bit set), two halves per instruction, then key << 16 | tag per distance
          const uint32_t k01 = q01 ^ (((q01 >> 15) & 0x00010001u) * 0x7fffu | 0x80008000u);
          const uint32_t k23 = q23 ^ (((q23 >> 15) & 0x00010001u) * 0x7fffu | 0x80008000u);
          best[0] = max(best[0], (k01 << 16) | tag);
          best[1] = max(best[1], (k01 & 0xffff0000u) | tag);
          best[2] = max(best[2], (k23 << 16) | tag);
          best[3] = max(best[3], (k23 & 0xffff0000u) | tag);
        } else {
          const float e[4] = {__uint_as_float(q01 << 16) + 0.f, __uint_as_float(q01 & 0xffff0000u) + 0.f,
                              __uint_as_float(q23 << 16) + 0.f, __uint_as_float(q23 & 0xffff0000u) + 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) best[i] = max(best[i], (oa::float_key(e[i]) & 0xffff0000u) | tag);
        }
      }
      // maximum over the 16 lanes of each DPP row (the 16 centroids of one block column set)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v = best[i];
        v = max(v, oa::dpp_u32<0xB1, 0xf>(v));
        v = max(v, oa::dpp_u32<0x4E, 0xf>(v));
        v = max(v, oa::dpp_u32<0x141, 0xf>(v));
        v = max(v, oa::dpp_u32<0x140, 0xf>(v));
        best[i] = v;
      }
      if ((lane & 15) < 4) {
        const int i = lane & 15;
        const int t = t0 + 4 * (lane >> 4) + i;
        // lane (16g + i) holds token 4g + i of the block: best[i] of its row
        uint32_t v = i == 0 ? best[0] : (i == 1 ? best[1] : (i == 2 ? best[2] : best[3]));
        if (t < T) {
          const int cid = 255 - (int)(v & 0xffu);   // (every real distance key exceeds 0)
          asg[(long)row * as + t] = cid;
          asg8[(long)row * a8s + t] = (uint8_t)cid;
        }
      }
    }
  }
}

constexpr int kMemBuf = 2048;   // member positions staged in LDS at a time

// a wave copies 1 <= n <= (the LDS array's size) member positions into LDS, eight loads per lane
// in flight at a time (one at a time, each copy waited on its load)
__device__ __forceinline__ void stage_members(int* s_pos, const int32_t* ml, int n, int lane) {
  for (int b = 0; b < n; b += 512) {
    int v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ml[min(b + lane + 64 * u, n - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (b + lane + 64 * u < n) s_pos[b + lane + 64 * u] = v[u];
  }
}

// One wave per (cluster, query row): the members in position order (the row's member lists of
// csr_sort_kernel), their zP rows staged kUB at a time through LDS (the next batch requested
// while one is summed) and summed in fp64 by lanes 0..15 (one column each) in that order;
// centroid = fp32(sum / count), or the initial point when the cluster is empty.
__global__ void __launch_bounds__(64) kmeans_update_kernel(const uint16_t* zraw, const float* colmean,
                                                           long zps, int C, const int32_t* mem, long ms,
                                                           const int32_t* cstart, const int32_t* clen,
                                                           const int32_t* init_idx, float* cent,
                                                           float* cnt_out) {
  constexpr int kUB = 64;                      // members per staged batch
  constexpr int kUpdBuf = 512;                 // member positions staged at a time (6 KB of LDS
                                               // per wave: about 26 waves per compute unit)
  __shared__ int s_pos[kUpdBuf];
  __shared__ float4 s_stage[kUB * (kRC / 4)];
  const int lane = threadIdx.x;
  // the C workgroups of a row run on one XCD (workgroups are dealt to the 8 XCDs in turn), so the
  // row's projection lines, each holding the rows of members of several clusters, are fetched
  // into that XCD's L2 once rather than by every XCD
  int c, row;
  {
    const int b = blockIdx.x, rows = gridDim.x / C;
    if (rows % 8 == 0) {
      const int k = b >> 3;
      row = (k / C) * 8 + (b & 7);
      c = k % C;
    } else {
      row = b / C;
      c = b % C;
    }
  }
  const int32_t* ml = mem + (long)row * ms + cstart[row * C + c];
  const int cl = clen[row * C + c];
  const uint16_t* zr = zraw + (long)row * zps;
  // zP = bf16(k W) - colmean from the stored bf16 projection: this lane's quarter of a row
  float cq[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) cq[e] = colmean[row * kRC + 4 * (lane & 3) + e];
  double acc = 0.0;
  int cnt = 0;
  // lane l reads member quarter l % 4 of members l / 4 + 16 b of a batch; a slot past the last
  // member reads the last member's row again (never summed), so the loads issue without branches
  auto load = [&](uint2* w, int k0, int n) {
#pragma unroll
    for (int b = 0; b < kUB / 16; ++b) {
      const int m = min(k0 + (lane >> 2) + 16 * b, n - 1);
      w[b] = *reinterpret_cast<const uint2*>(zr + (long)s_pos[m] * kRC + 4 * (lane & 3));
    }
  };
  for (int i0 = 0; i0 < cl; i0 += kUpdBuf) {
    const int n = min(kUpdBuf, cl - i0);
    stage_members(s_pos, ml + i0, n, lane);
    __syncthreads();
    uint2 w[kUB / 16];
    if (n > 0) load(w, 0, n);
    for (int k0 = 0; k0 < n; k0 += kUB) {
#pragma unroll
      for (int b = 0; b < kUB / 16; ++b)
        s_stage[((lane >> 2) + 16 * b) * 4 + (lane & 3)] =
            make_float4(__uint_as_float(w[b].x << 16) - cq[0], __uint_as_float(w[b].x & 0xffff0000u) - cq[1],
                        __uint_as_float(w[b].y << 16) - cq[2], __uint_as_float(w[b].y & 0xffff0000u) - cq[3]);
      __syncthreads();
      // the next batch's rows are requested while this one is summed
      if (k0 + kUB < n) load(w, k0 + kUB, n);
      if (lane < kRC) {
        // 16 staged values read together, then added in member order (a slot past the last
        // member adds +0, which leaves the sum as it is: it is never -0 starting from +0)
        const float* st = reinterpret_cast<const float*>(s_stage);
        const int mm = min(kUB, n - k0);
        for (int m0 = 0; m0 < mm; m0 += 16) {
          float v[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] = st[(m0 + u) * kRC + lane];   // m0 + u < kUB
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] = m0 + u < mm ? v[u] : 0.f;
#pragma unroll
          for (int u = 0; u < 16; ++u) acc += (double)v[u];
        }
      }
      __syncthreads();
    }
    cnt += n;
  }
  if (lane < kRC) {
    const float v = cnt > 0 ? (float)(acc / (double)cnt)
                            : oa::bf16_to_f32(zr[(long)init_idx[c] * kRC + lane]) - colmean[row * kRC + lane];
    cent[((long)row * C + c) * kRC + lane] = v;
  }
  if (lane == 0 && cnt_out) cnt_out[row * C + c] = (float)cnt;
}

// ---------------------------------------------------------------------------------- sums + CSR
// One 1024-thread workgroup per query row: nb, clen (member counts), cstart (exclusive prefix)
// and mem, every cluster's members in position order (a stable counting sort of the row's ids).
// The row is taken 1024 positions at a time, wave w holding positions 64 w .. 64 w + 63 of the
// step.  A lane's equal-id lanes are the AND over the 8 id bits of that bit's ballot (or its
// complement); its rank among them orders it, their count goes to LDS per (cluster, wave), and
// a 16-lane scan per cluster turns the counts into the waves' starts in wave order -- so equal
// ids keep their position order inside a step, and the steps follow each other.
constexpr int kSortThreads = 1024;
constexpr int kSortStage = 32768;   // rows of at most this many ids are staged in LDS by the sort
constexpr int kSortWaves = kSortThreads / 64;
__global__ void __launch_bounds__(kSortThreads) csr_sort_kernel(int T, const uint8_t* asg8, long a8s, int C,
                                                               float* nb, int32_t* cstart, int32_t* clen,
                                                               int32_t* mem, long ms, int staged) {
  __shared__ int s_base[kMaxC];
  __shared__ int s_wcnt[kMaxC][kSortWaves];
  __shared__ __align__(16) uint8_t s_ids[kSortStage];   // the row's ids when staged (T <= kSortStage)
  const int row = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint8_t* ar = asg8 + (long)row * a8s;
  int32_t* mr = mem + (long)row * ms;
  for (int c = tid; c < kMaxC; c += kSortThreads) s_base[c] = 0;
  __syncthreads();
  if (staged) {
    // 16 ids per thread and load (rows 16-byte aligned, their stride a multiple of 16), kept in
    // LDS for the scatter pass
    const int T16 = (T + 15) / 16;
    for (int i = tid; i < T16; i += kSortThreads) {
      const uint4 w = reinterpret_cast<const uint4*>(ar)[i];
      *reinterpret_cast<uint4*>(s_ids + 16 * i) = w;
      const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int b = 0; b < 16; ++b)
        if (16 * i + b < T) atomicAdd(&s_base[(q[b >> 2] >> (8 * (b & 3))) & 0xffu], 1);
    }
  } else {
    for (int t = tid; t < T; t += kSortThreads) atomicAdd(&s_base[ar[t]], 1);
  }
  __syncthreads();
  if (wave == 0) {
    int v[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = s_base[lane * 4 + i]; loc += v[i]; }
    const int incl = oa::wave_incl_scan_i32(loc);
    int run = incl - loc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane * 4 + i;
      if (c < C) {
        cstart[row * C + c] = run;
        clen[row * C + c] = v[i];
        if (nb) nb[row * C + c] = (float)v[i];
      }
      s_base[c] = run;
      run += v[i];
    }
  }
  const unsigned long long lower = (1ull << lane) - 1ull;
  for (int p0 = 0; p0 < T; p0 += kSortThreads) {
    for (int i = tid; i < kSortWaves * kMaxC; i += kSortThreads) (&s_wcnt[0][0])[i] = 0;
    __syncthreads();
    const int p = p0 + tid;
    const bool valid = p < T;
    const int x = valid ? (int)(staged ? s_ids[p] : ar[p]) : 0;
    unsigned long long m = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const unsigned long long bb = __ballot((x >> bit) & 1);
      m &= ((x >> bit) & 1) ? bb : ~bb;
    }
    const int rank = __popcll(m & lower);
    if (valid && rank == 0) s_wcnt[x][wave] = __popcll(m);
    __syncthreads();
    // the waves' starts per cluster: thread (c, w) of 16-lane groups, an inclusive scan over w
    for (int e = tid; e < C * kSortWaves; e += kSortThreads) {
      const int c = e >> 4, w = e & 15;
      const int v = s_wcnt[c][w];
      int incl = v;
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, true);   // row_shr:1
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, true);   // row_shr:2
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, true);   // row_shr:4
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, true);   // row_shr:8
      const int base = s_base[c];
      s_wcnt[c][w] = base + incl - v;
      if (w == kSortWaves - 1) s_base[c] = base + incl;
    }
    __syncthreads();
    if (valid) mr[s_wcnt[x][wave] + rank] = p;
    __syncthreads();
  }
}

// One wave per (cluster, query row): the fp64 sums of k, k*k and v over the members in position
// order (mem, written by csr_sort_kernel; lane l: dims 2l, 2l + 1), the K and V words of 16
// members requested together.
__global__ void __launch_bounds__(64) cluster_sums_kernel(const uint16_t* K, const uint16_t* V, long ksh,
                                                          long kst, int G, int C, const int32_t* cstart,
                                                          const int32_t* clen, float* Sk, float* Sk2,
                                                          float* Sv, const int32_t* mem, long ms,
                                                          float* nb) {
  __shared__ int s_pos[kMemBuf];
  const int lane = threadIdx.x;
  // every token's K and V rows are read once per query row of its KV row (each query row has its
  // own clusters).  The G * C workgroups of a KV row run on one XCD, its query rows interleaved,
  // so that they walk the KV row's positions together and the later reads of a row hit that
  // XCD's L2 (workgroups are dealt to the 8 XCDs in turn)
  int c, row;
  {
    const int b = blockIdx.x, rows = gridDim.x / C, kv_rows = rows / G;
    if (kv_rows % 8 == 0) {
      const int k = b >> 3, per = G * C;
      const int j = k % per;
      row = ((k / per) * 8 + (b & 7)) * G + j % G;
      c = j / G;
    } else {
      row = b / C;
      c = b % C;
    }
  }
  const uint16_t* kr = K + (long)(row / G) * ksh + 2 * lane;
  const uint16_t* vr = V + (long)(row / G) * ksh + 2 * lane;
  const int32_t* ml = mem + (long)row * ms + cstart[row * C + c];
  const int cl = clen[row * C + c];
  if (nb && lane == 0) nb[row * C + c] = (float)cl;   // (when the sort did not write it)
  double k0 = 0.0, k1 = 0.0, q0 = 0.0, q1 = 0.0, v0 = 0.0, v1 = 0.0;
  constexpr int U = 16;
  for (int i0 = 0; i0 < cl; i0 += kMemBuf) {
    const int n = min(kMemBuf, cl - i0);
    stage_members(s_pos, ml + i0, n, lane);
    __syncthreads();
    for (int k = 0; k < n; k += U) {
      uint32_t kw[U], vw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long off = (long)s_pos[min(k + u, n - 1)] * kst;
        kw[u] = *reinterpret_cast<const uint32_t*>(kr + off);
        vw[u] = *reinterpret_cast<const uint32_t*>(vr + off);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (k + u < n) {
          const double a0 = (double)__uint_as_float(kw[u] << 16);
          const double a1 = (double)__uint_as_float(kw[u] & 0xffff0000u);
          k0 += a0; k1 += a1; q0 += a0 * a0; q1 += a1 * a1;
          v0 += (double)__uint_as_float(vw[u] << 16);
          v1 += (double)__uint_as_float(vw[u] & 0xffff0000u);
        }
      }
    }
    __syncthreads();
  }
  const long o = ((long)row * C + c) * kD + 2 * lane;
  Sk[o] = (float)k0; Sk[o + 1] = (float)k1;
  Sk2[o] = (float)q0; Sk2[o + 1] = (float)q1;
  Sv[o] = (float)v0; Sv[o + 1] = (float)v1;
}

}  // namespace

extern "C" int oa_qgs_codes(const void* K, long k_stride_h, long k_stride_t, int kv_rows, int T,
                            const float* U, int8_t* codes, long codes_stride_h, float* scale,
                            uint32_t* amax_ws, float* zc_ws, void* stream) {
  if (kv_rows <= 0 || T <= 0 || !K || !U || !codes || !scale || !amax_ws || k_stride_t < kD ||
      k_stride_t % 8 || k_stride_h % 8 || codes_stride_h < (long)T * kRQ || codes_stride_h % 16 ||
      (reinterpret_cast<uintptr_t>(K) & 15) || (reinterpret_cast<uintptr_t>(codes) & 15) ||
      (reinterpret_cast<uintptr_t>(zc_ws) & 15))
    return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* k = reinterpret_cast<const uint16_t*>(K);
  hipLaunchKernelGGL(clear_u32_kernel, dim3(std::min(64, (kv_rows * kRQ + 63) / 64)), dim3(64), 0, s,
                     amax_ws, kv_rows * kRQ);
  const dim3 grid((T + kCodeThreads - 1) / kCodeThreads, kv_rows);
  hipLaunchKernelGGL(codes_amax_kernel, grid, dim3(kCodeThreads), 0, s, k, k_stride_h, k_stride_t, T, U,
                     amax_ws, zc_ws);
  hipLaunchKernelGGL(codes_write_kernel, grid, dim3(kCodeThreads), 0, s, k, k_stride_h, k_stride_t, T, U,
                     amax_ws, codes, codes_stride_h, scale, zc_ws);
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_qgc_project(const void* K, long k_stride_h, long k_stride_t, int rows, int G, int T,
                              const void* W, float* zP, long zp_stride, float* colmean,
                              double* tile_ws, uint16_t* zraw_out, void* stream) {
  if (rows <= 0 || G <= 0 || rows % G || T <= 0 || !K || !W || (!zP && !zraw_out) || !colmean ||
      !tile_ws || k_stride_t < kD || k_stride_t % 8 || k_stride_h % 8 || zp_stride < (long)T * kRC ||
      zp_stride % 4 || (reinterpret_cast<uintptr_t>(K) & 15) || (reinterpret_cast<uintptr_t>(zP) & 15) ||
      (reinterpret_cast<uintptr_t>(zraw_out) & 15) || (zraw_out && zp_stride % 8))
    return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const int ntiles = (T + 63) / 64;
  const int nx = (ntiles + kProjTiles - 1) / kProjTiles;
  if (G == 4)   // a KV row's four query rows per wave: each K block loaded once for all four
    hipLaunchKernelGGL(qgc_project_kernel<4>, dim3(nx, rows / 4), dim3(64), 0, s,
                       reinterpret_cast<const uint16_t*>(K), k_stride_h, k_stride_t, G, T,
                       reinterpret_cast<const uint16_t*>(W), zP, zp_stride, zraw_out, tile_ws, ntiles);
  else
    hipLaunchKernelGGL(qgc_project_kernel<1>, dim3(nx, rows), dim3(64), 0, s,
                       reinterpret_cast<const uint16_t*>(K), k_stride_h, k_stride_t, G, T,
                       reinterpret_cast<const uint16_t*>(W), zP, zp_stride, zraw_out, tile_ws, ntiles);
  hipLaunchKernelGGL(qgc_colmean_kernel, dim3(rows), dim3(64), 0, s, T, tile_ws, ntiles, colmean);
  if (zP) {
    const int nb = std::min(16, (T * (kRC / 4) + 255) / 256);
    hipLaunchKernelGGL(qgc_center_kernel, dim3(nb, rows), dim3(256), 0, s, zP, zp_stride, T, colmean);
  }
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_kmeans_assign(const uint16_t* zraw, const float* colmean, long z_stride, int rows,
                                int T, const float* cent, int C, int32_t* asg, long asg_stride,
                                uint8_t* asg8, long asg8_stride, void* stream) {
  if (rows <= 0 || T <= 0 || C <= 0 || C > kMaxC || !zraw || !colmean || !cent || !asg || !asg8 ||
      z_stride < (long)T * kRC || z_stride % 4 || asg_stride < T || asg8_stride < T ||
      (reinterpret_cast<uintptr_t>(zraw) & 7))
    return OA_EINVAL;
  const int ntiles = (T + 63) / 64;
  hipLaunchKernelGGL(kmeans_assign_kernel, dim3((ntiles + kAsgTiles - 1) / kAsgTiles, rows),
                     dim3(kAsgThreads), 0, (hipStream_t)stream, zraw, colmean, z_stride, T, cent, C, asg,
                     asg_stride, asg8, asg8_stride);
  return OA_LAUNCH_STATUS();
}

// the sort stages a row's ids in LDS with 16-byte loads when the row fits and its rows are
// 16-byte aligned with a stride that is a multiple of 16 (it then reads up to the next multiple of
// 16 of T, inside the row's stride)
static int sort_staged(int T, const uint8_t* asg8, long asg8_stride) {
  return T <= kSortStage && asg8_stride % 16 == 0 && (reinterpret_cast<uintptr_t>(asg8) & 15) == 0;
}

extern "C" int oa_kmeans_update(const uint16_t* zraw, const float* colmean, long z_stride, int rows,
                                int T, const uint8_t* asg8, long asg8_stride, int C,
                                const int32_t* init_idx, float* cent, float* cnt_out, int32_t* mem_ws,
                                long mem_stride, int32_t* cstart_ws, int32_t* clen_ws, void* stream) {
  if (rows <= 0 || T <= 0 || C <= 0 || C > kMaxC || !zraw || !colmean || !asg8 || !init_idx || !cent ||
      !mem_ws || !cstart_ws || !clen_ws || mem_stride < T || z_stride < (long)T * kRC ||
      z_stride % 4 || (reinterpret_cast<uintptr_t>(zraw) & 7) || asg8_stride < T)
    return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(csr_sort_kernel, dim3(rows), dim3(kSortThreads), 0, s, T, asg8, asg8_stride, C,
                     nullptr, cstart_ws, clen_ws, mem_ws, mem_stride, sort_staged(T, asg8, asg8_stride));
  hipLaunchKernelGGL(kmeans_update_kernel, dim3(C * rows), dim3(64), 0, s, zraw, colmean, z_stride, C,
                     mem_ws, mem_stride, cstart_ws, clen_ws, init_idx, cent, cnt_out);
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_cluster_build(const void* K, const void* V, long kv_stride_h, long kv_stride_t, int rows,
                                int G, int T, const uint8_t* asg8, long asg8_stride, int C, float* nb,
                                float* Sk, float* Sk2, float* Sv, int32_t* mem, long mem_stride,
                                int32_t* cstart, int32_t* clen, void* stream) {
  if (rows <= 0 || G <= 0 || rows % G || T <= 0 || C <= 0 || C > kMaxC || !K || !V || !asg8 || !nb ||
      !Sk || !Sk2 || !Sv || !mem || !cstart || !clen || kv_stride_t < kD || kv_stride_t % 2 ||
      kv_stride_h % 2 || asg8_stride < T || mem_stride < T || (reinterpret_cast<uintptr_t>(K) & 3) ||
      (reinterpret_cast<uintptr_t>(V) & 3))
    return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(csr_sort_kernel, dim3(rows), dim3(kSortThreads), 0, s, T, asg8, asg8_stride, C, nb,
                     cstart, clen, mem, mem_stride, sort_staged(T, asg8, asg8_stride));
  hipLaunchKernelGGL(cluster_sums_kernel, dim3(C * rows), dim3(64), 0, s,
                     reinterpret_cast<const uint16_t*>(K), reinterpret_cast<const uint16_t*>(V),
                     kv_stride_h, kv_stride_t, G, C, cstart, clen, Sk, Sk2, Sv, mem, mem_stride,
                     static_cast<float*>(nullptr));
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_cluster_sums(const void* K, const void* V, long kv_stride_h, long kv_stride_t, int rows,
                               int G, int T, int C, float* nb, float* Sk, float* Sk2, float* Sv,
                               const int32_t* mem, long mem_stride, const int32_t* cstart,
                               const int32_t* clen, void* stream) {
  if (rows <= 0 || G <= 0 || rows % G || T <= 0 || C <= 0 || C > kMaxC || !K || !V || !nb || !Sk ||
      !Sk2 || !Sv || !mem || !cstart || !clen || kv_stride_t < kD || kv_stride_t % 2 ||
      kv_stride_h % 2 || mem_stride < T || (reinterpret_cast<uintptr_t>(K) & 3) ||
      (reinterpret_cast<uintptr_t>(V) & 3))
    return OA_EINVAL;
  hipLaunchKernelGGL(cluster_sums_kernel, dim3(C * rows), dim3(64), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint16_t*>(K), reinterpret_cast<const uint16_t*>(V),
                     kv_stride_h, kv_stride_t, G, C, cstart, clen, Sk, Sk2, Sv, mem, mem_stride, nb);
  return OA_LAUNCH_STATUS();
}
