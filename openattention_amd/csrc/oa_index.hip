// Index update of the token written at position n-1 (device-side n).
//
// Reference: _k_index_update_d2 (inference/ours_graph.py:43-90) and the eager step 1 of
// Ours.decode (methods_eager.py:586-601); accuracy-path counterparts StaticTopKMasker._extend
// (static_top_k.py:166-183) and UTAMultiBinAttention._profile_extend (multibin.py:2062-2096).
//   code_r  = clamp(rint((k . U[:, r]) / scale_r), -127, 127)        (KV-head row only)
//   zp_j    = bf16(k . W[:, j]) - colmean_j                            (per query-head row)
//   cluster = argmax_c (zp . cent_c - 0.5 |cent_c|^2), ties to the lower id
//   n_c += 1; Sk_c += k; Sk2_c += k*k; Sv_c += v; append n-1 to the cluster's generated list;
//   the cluster id is stored as int32 (asg) and as uint8 (asg8, the byte stream top-q reads)
// Dot products use the canonical order of oa_common.h; zp . cent and |cent|^2 are sequential
// fma chains over j = 0..15 -- the CPU restatement replays both.
#include "oa_common.h"
#include "oa_prep.h"

namespace {

constexpr int RQ = 32;
constexpr int RC = 16;

struct IdxArgs {
  const uint16_t* K; const uint16_t* V; long kv_sb; long kv_ss;
  int8_t* codes; int Lmax_codes;
  const float* U; const float* scale;
  const uint16_t* W; const float* colmean; const float* cent;
  int32_t* asg; long asg_stride;
  uint8_t* asg8; long asg8_stride;
  float* nb; float* Sk; float* Sk2; float* Sv;
  int32_t* reclist; int32_t* reccnt; int rmax;
  const int* n_dev; int C; int G;
};

// the int8 QGS code of the token at n-1 of KV row r / G (written by query row r % G == 0)
__device__ __forceinline__ void index_codes_row(const IdxArgs& a, int r, int lane) {
  const int kvr = r / a.G;
  const int pos = *a.n_dev - 1;
  const uint16_t* kp = a.K + (long)kvr * a.kv_sb + (long)pos * a.kv_ss;
  const float k_lo = oa::bf16_to_f32(kp[lane]), k_hi = oa::bf16_to_f32(kp[lane + 64]);
  if (r % a.G == 0) {
    const float* Ub = a.U + (long)kvr * OA_D * RQ;
    float ul[RQ], uh[RQ];
#pragma unroll
    for (int j = 0; j < RQ; j += 4) {
      const float4 x = *reinterpret_cast<const float4*>(Ub + lane * RQ + j);
      const float4 y = *reinterpret_cast<const float4*>(Ub + (lane + 64) * RQ + j);
      ul[j] = x.x; ul[j + 1] = x.y; ul[j + 2] = x.z; ul[j + 3] = x.w;
      uh[j] = y.x; uh[j + 1] = y.y; uh[j + 2] = y.z; uh[j + 3] = y.w;
    }
    int8_t mycode = 0;
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      const float zc = oa::dot128_canon(k_lo, ul[j], k_hi, uh[j]);
      float code = rintf(zc / a.scale[(long)kvr * RQ + j]);
      code = fminf(fmaxf(code, -127.f), 127.f);
      if (lane == j) mycode = (int8_t)(int)code;
    }
    if (lane < RQ) a.codes[((long)kvr * a.Lmax_codes + pos) * RQ + lane] = mycode;
  }
}

// the token at n-1 joins query row r's nearest centroid: its asg / asg8 entry, the cluster's
// Sk, Sk2, Sv, nb and recent-token list
__device__ __forceinline__ void index_assign_row(const IdxArgs& a, int r, int lane) {
  const int kvr = r / a.G;
  const int pos = *a.n_dev - 1;
  const uint16_t* kp = a.K + (long)kvr * a.kv_sb + (long)pos * a.kv_ss;
  const uint16_t* vp = a.V + (long)kvr * a.kv_sb + (long)pos * a.kv_ss;
  const float k_lo = oa::bf16_to_f32(kp[lane]), k_hi = oa::bf16_to_f32(kp[lane + 64]);
  const float v_lo = oa::bf16_to_f32(vp[lane]), v_hi = oa::bf16_to_f32(vp[lane + 64]);
  // lane l holds rows l and l+64 of W (16 bf16 each, 32 contiguous bytes)
  const uint16_t* Wb = a.W + (long)r * OA_D * RC;
  float wl[RC], wh[RC];
  oa::unpack8(*reinterpret_cast<const uint4*>(Wb + lane * RC), wl);
  oa::unpack8(*reinterpret_cast<const uint4*>(Wb + lane * RC + 8), wl + 8);
  oa::unpack8(*reinterpret_cast<const uint4*>(Wb + (lane + 64) * RC), wh);
  oa::unpack8(*reinterpret_cast<const uint4*>(Wb + (lane + 64) * RC + 8), wh + 8);
  // the lane's first centroid is requested with W (its distance needs zp only later)
  const float* cb = a.cent + (long)r * a.C * RC;
  float c0[RC];
#pragma unroll
  for (int j = 0; j < RC; j += 4) {
    const float4 x = *reinterpret_cast<const float4*>(cb + (long)min(lane, a.C - 1) * RC + j);
    c0[j] = x.x; c0[j + 1] = x.y; c0[j + 2] = x.z; c0[j + 3] = x.w;
  }
  float zp[RC];
#pragma unroll
  for (int j = 0; j < RC; ++j) {
    const float d = oa::dot128_canon(k_lo, wl[j], k_hi, wh[j]);
    zp[j] = oa::bf16_round(d) - a.colmean[(long)r * RC + j];
  }
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int c = lane; c < a.C; c += 64) {
    float cc[RC];
    if (c == lane) {
#pragma unroll
      for (int j = 0; j < RC; ++j) cc[j] = c0[j];
    } else {
#pragma unroll
      for (int j = 0; j < RC; j += 4) {
        const float4 x = *reinterpret_cast<const float4*>(cb + (long)c * RC + j);
        cc[j] = x.x; cc[j + 1] = x.y; cc[j + 2] = x.z; cc[j + 3] = x.w;
      }
    }
    float sim = zp[0] * cc[0];
    float h = cc[0] * cc[0];
#pragma unroll
    for (int j = 1; j < RC; ++j) {
      sim = fmaf(zp[j], cc[j], sim);
      h = fmaf(cc[j], cc[j], h);
    }
    const float dist = sim - 0.5f * h;
    if (dist > best || bidx == 0x7fffffff) { best = dist; bidx = c; }
  }
  // the argmax (ties to the lower id) on the DPP / permlane network: the pairing of the xor
  // butterfly (m = 1, 2, 4, 8, 16, 32; the mirrors pair groups that are uniform by then); the
  // larger distance, then the lower id, is an order-free pick, so every lane ends with the winner
  auto take = [&](float ob, int oi) {
    if (ob > best || (ob == best && oi < bidx)) { best = ob; bidx = oi; }
  };
  take(oa::dpp_f32<0xB1>(best), __builtin_amdgcn_update_dpp(bidx, bidx, 0xB1, 0xf, 0xf, false));
  take(oa::dpp_f32<0x4E>(best), __builtin_amdgcn_update_dpp(bidx, bidx, 0x4E, 0xf, 0xf, false));
  take(oa::dpp_f32<0x141>(best), __builtin_amdgcn_update_dpp(bidx, bidx, 0x141, 0xf, 0xf, false));
  take(oa::dpp_f32<0x140>(best), __builtin_amdgcn_update_dpp(bidx, bidx, 0x140, 0xf, 0xf, false));
  // (a permlane swap returns the lane's own pair and its partner's; the pick is symmetric)
  {
    const auto b16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(best), __float_as_uint(best), false, false);
    const auto i16 = __builtin_amdgcn_permlane16_swap((unsigned)bidx, (unsigned)bidx, false, false);
    best = __uint_as_float(b16[0]);
    bidx = (int)i16[0];
    take(__uint_as_float(b16[1]), (int)i16[1]);
  }
  {
    const auto b32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(best), __float_as_uint(best), false, false);
    const auto i32 = __builtin_amdgcn_permlane32_swap((unsigned)bidx, (unsigned)bidx, false, false);
    best = __uint_as_float(b32[0]);
    bidx = (int)i32[0];
    take(__uint_as_float(b32[1]), (int)i32[1]);
  }
  const int c = bidx;
  const long sb = ((long)r * a.C + c) * OA_D;
  a.Sk[sb + lane] += k_lo;
  a.Sk[sb + lane + 64] += k_hi;
  a.Sk2[sb + lane] += k_lo * k_lo;
  a.Sk2[sb + lane + 64] += k_hi * k_hi;
  a.Sv[sb + lane] += v_lo;
  a.Sv[sb + lane + 64] += v_hi;
  if (lane == 0) {
    a.asg[(long)r * a.asg_stride + pos] = c;
    a.asg8[(long)r * a.asg8_stride + pos] = (uint8_t)c;
    a.nb[(long)r * a.C + c] += 1.0f;
    const long rc = (long)r * a.C + c;
    const int cnt = a.reccnt[rc];
    if (cnt < a.rmax) a.reclist[rc * a.rmax + cnt] = pos;
    a.reccnt[rc] = cnt + 1;
  }
}

__global__ void __launch_bounds__(64) index_update_kernel(IdxArgs a) {
  index_codes_row(a, blockIdx.x, threadIdx.x);
  index_assign_row(a, blockIdx.x, threadIdx.x);
}

struct PrepArgs {
  const uint16_t* q; long q_stride; int8_t* limbs; int* fexp;
};

// one query-head row per 192-thread workgroup: wave 0 adds the token at n-1 to the row's
// clustering, wave 1 projects the row's query, wave 2 (of the first row of each KV row) writes
// the token's code; the three touch disjoint data
__global__ void __launch_bounds__(192) index_prep_kernel(IdxArgs a, PrepArgs p) {
  const int w = threadIdx.x >> 6;
  const int r = oa::xcd_row(blockIdx.x, gridDim.x);   // a KV row's query rows share one L2 (U)
  if (w == 0)
    index_assign_row(a, r, threadIdx.x);
  else if (w == 1)
    oa::qgs_prep_row(p.q, p.q_stride, a.U, a.scale, a.G, p.limbs, p.fexp, nullptr, r,
                     threadIdx.x - 64);
  else if (r % a.G == 0)
    index_codes_row(a, r, threadIdx.x - 128);
}

// The token at position n-1 leaves every query row's cluster statistics: the inverse of the
// statistics part of the index update, in the same fp32 terms (n_c -= 1, Sk_c -= k,
// Sk2_c -= k*k, Sv_c -= v; c = asg[row][n-1]).  Codes, cluster ids and lists stay as they are:
// every decode stage reads positions below n only.  A multi-row call takes its later keys back
// this way, so that each causal row sees the statistics of the keys before it.
struct DownArgs {
  const uint16_t* K; const uint16_t* V; long kv_sb; long kv_ss;
  const int32_t* asg; long asg_stride;
  float* nb; float* Sk; float* Sk2; float* Sv;
  const int* n_dev; int C; int G;
};

__global__ void __launch_bounds__(64) index_downdate_kernel(DownArgs a) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  const int kvr = r / a.G;
  const int pos = *a.n_dev - 1;
  if (pos < 0) return;                                        // uniform
  const int c = a.asg[(long)r * a.asg_stride + pos];
  if (c < 0 || c >= a.C) return;                              // uniform
  const uint16_t* kp = a.K + (long)kvr * a.kv_sb + (long)pos * a.kv_ss;
  const uint16_t* vp = a.V + (long)kvr * a.kv_sb + (long)pos * a.kv_ss;
  const float k_lo = oa::bf16_to_f32(kp[lane]), k_hi = oa::bf16_to_f32(kp[lane + 64]);
  const float v_lo = oa::bf16_to_f32(vp[lane]), v_hi = oa::bf16_to_f32(vp[lane + 64]);
  const long sb = ((long)r * a.C + c) * OA_D;
  a.Sk[sb + lane] -= k_lo;
  a.Sk[sb + lane + 64] -= k_hi;
  a.Sk2[sb + lane] -= k_lo * k_lo;
  a.Sk2[sb + lane + 64] -= k_hi * k_hi;
  a.Sv[sb + lane] -= v_lo;
  a.Sv[sb + lane + 64] -= v_hi;
  if (lane == 0) a.nb[(long)r * a.C + c] -= 1.0f;
}

}  // namespace

extern "C" int oa_index_update(const void* K, const void* V, long kv_stride_b, long kv_stride_s,
                               int rows, int kv_rows, int head_dim, int8_t* codes, int codes_lmax,
                               int rank_q, const float* U, const float* scale, const void* W,
                               const float* colmean, int rank_c, const float* cent, int C,
                               int32_t* asg, long asg_stride, uint8_t* asg8, long asg8_stride,
                               float* nb, float* Sk, float* Sk2,
                               float* Sv, int32_t* reclist, int32_t* reccnt, int rmax,
                               const int* n_dev, void* stream) {
  if (head_dim != OA_D || rank_q != RQ || rank_c != RC || kv_rows <= 0 || rows % kv_rows != 0 ||
      C <= 0 || C > 256 || rmax < 0 || !asg8)
    return OA_EINVAL;
  IdxArgs a;
  a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.kv_sb = kv_stride_b; a.kv_ss = kv_stride_s;
  a.codes = codes; a.Lmax_codes = codes_lmax; a.U = U; a.scale = scale;
  a.W = (const uint16_t*)W; a.colmean = colmean; a.cent = cent;
  a.asg = asg; a.asg_stride = asg_stride; a.asg8 = asg8; a.asg8_stride = asg8_stride; a.nb = nb; a.Sk = Sk; a.Sk2 = Sk2; a.Sv = Sv;
  a.reclist = reclist; a.reccnt = reccnt; a.rmax = rmax; a.n_dev = n_dev; a.C = C;
  a.G = rows / kv_rows;
  hipLaunchKernelGGL(index_update_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_index_prep(const void* K, const void* V, long kv_stride_b, long kv_stride_s,
                             int rows, int kv_rows, int head_dim, int8_t* codes, int codes_lmax,
                             int rank_q, const float* U, const float* scale, const void* W,
                             const float* colmean, int rank_c, const float* cent, int C,
                             int32_t* asg, long asg_stride, uint8_t* asg8, long asg8_stride,
                             float* nb, float* Sk, float* Sk2, float* Sv, int32_t* reclist,
                             int32_t* reccnt, int rmax, const int* n_dev, const void* q,
                             long q_stride, int8_t* limbs, int* fexp, void* stream) {
  if (head_dim != OA_D || rank_q != RQ || rank_c != RC || kv_rows <= 0 || rows % kv_rows != 0 ||
      rows / kv_rows != 4 || C <= 0 || C > 256 || rmax < 0 || !asg8 || !q || !limbs || !fexp)
    return OA_EINVAL;
  IdxArgs a;
  a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.kv_sb = kv_stride_b; a.kv_ss = kv_stride_s;
  a.codes = codes; a.Lmax_codes = codes_lmax; a.U = U; a.scale = scale;
  a.W = (const uint16_t*)W; a.colmean = colmean; a.cent = cent;
  a.asg = asg; a.asg_stride = asg_stride; a.asg8 = asg8; a.asg8_stride = asg8_stride; a.nb = nb;
  a.Sk = Sk; a.Sk2 = Sk2; a.Sv = Sv;
  a.reclist = reclist; a.reccnt = reccnt; a.rmax = rmax; a.n_dev = n_dev; a.C = C;
  a.G = rows / kv_rows;
  PrepArgs p;
  p.q = (const uint16_t*)q; p.q_stride = q_stride; p.limbs = limbs; p.fexp = fexp;
  hipLaunchKernelGGL(index_prep_kernel, dim3(rows), dim3(192), 0, (hipStream_t)stream, a, p);
  return OA_LAUNCH_STATUS();
}

extern "C" int oa_index_downdate(const void* K, const void* V, long kv_stride_b, long kv_stride_s,
                                 int rows, int kv_rows, int head_dim, const int32_t* asg,
                                 long asg_stride, float* nb, float* Sk, float* Sk2, float* Sv, int C,
                                 const int* n_dev, void* stream) {
  if (head_dim != OA_D || kv_rows <= 0 || rows % kv_rows != 0 || C <= 0 || C > 256 || !K || !V ||
      !asg || !nb || !Sk || !Sk2 || !Sv || !n_dev)
    return OA_EINVAL;
  DownArgs a;
  a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.kv_sb = kv_stride_b; a.kv_ss = kv_stride_s;
  a.asg = asg; a.asg_stride = asg_stride; a.nb = nb; a.Sk = Sk; a.Sk2 = Sk2; a.Sv = Sv;
  a.n_dev = n_dev; a.C = C; a.G = rows / kv_rows;
  hipLaunchKernelGGL(index_downdate_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}
