// QGS query projection of one query-head row by one wave (used by qgs_prep_kernel and by the
// fused index-update + prep kernel).
//
// Reference: zq = (q U) * scale (StaticTopKMasker._scores, static_top_k.py:203-213).
// zq_r = (q . U[:, r]) * scale_r in the canonical dot order; then the fixed-point exponent
// F = 30 - e (max_r |zq_r| = m 2^e, m in [0.5, 1)) and Z_r = rint(zq_r 2^F) split into four
// signed 8-bit limbs (Z = l0 + 256 l1 + 65536 l2 + 2^24 l3), the int8 MFMA operand of the scan.
#pragma once
#include "oa_common.h"

namespace oa {

constexpr int kPrepRQ = 32;   // QGS rank (bytes of code per token)

__device__ __forceinline__ void qgs_prep_row(const uint16_t* __restrict__ q, long q_stride,
                                             const float* __restrict__ U,      // (BH, D, RQ)
                                             const float* __restrict__ scale,  // (BH, RQ)
                                             int G, int8_t* __restrict__ limbs, // (BH, 16, RQ)
                                             int* __restrict__ fexp, float* __restrict__ zq_out,
                                             int row, int lane) {
  constexpr int RQ = kPrepRQ;
  const int kvr = row / G;
  const int g = row % G;
  const float q_lo = bf16_to_f32(q[(long)row * q_stride + lane]);
  const float q_hi = bf16_to_f32(q[(long)row * q_stride + lane + 64]);
  const float* Ub = U + (long)kvr * OA_D * RQ;
  // lane l holds rows l and l+64 of U (32 contiguous floats each)
  float ul[RQ], uh[RQ], sc[RQ];
#pragma unroll
  for (int j = 0; j < RQ; j += 4) {
    const float4 a = *reinterpret_cast<const float4*>(Ub + lane * RQ + j);
    const float4 b = *reinterpret_cast<const float4*>(Ub + (lane + 64) * RQ + j);
    ul[j] = a.x; ul[j + 1] = a.y; ul[j + 2] = a.z; ul[j + 3] = a.w;
    uh[j] = b.x; uh[j + 1] = b.y; uh[j + 2] = b.z; uh[j + 3] = b.w;
  }
#pragma unroll
  for (int j = 0; j < RQ; ++j) sc[j] = scale[(long)kvr * RQ + j];
  float myz = 0.f;
#pragma unroll
  for (int j = 0; j < RQ; ++j) {
    const float d = dot128_canon(q_lo, ul[j], q_hi, uh[j]);
    const float z = d * sc[j];
    if (lane == j) myz = z;
  }
  float a = (lane < RQ) ? fabsf(myz) : 0.f;
  float emax = wave_max(a);
  int F = 0;
  int Z = 0;
  if (emax > 0.f && emax < INFINITY) {
    int ex;
    (void)frexpf(emax, &ex);
    F = 30 - ex;
    if (lane < RQ) Z = (int)rint(ldexp((double)myz, F));
  }
  if (lane < RQ) {
    int l0 = (int)(int8_t)(Z & 0xff);
    int z1 = (Z - l0) >> 8;
    int l1 = (int)(int8_t)(z1 & 0xff);
    int z2 = (z1 - l1) >> 8;
    int l2 = (int)(int8_t)(z2 & 0xff);
    int l3 = (z2 - l2) >> 8;
    int8_t* Lb = limbs + (long)kvr * 16 * RQ;
    Lb[(g * 4 + 0) * RQ + lane] = (int8_t)l0;
    Lb[(g * 4 + 1) * RQ + lane] = (int8_t)l1;
    Lb[(g * 4 + 2) * RQ + lane] = (int8_t)l2;
    Lb[(g * 4 + 3) * RQ + lane] = (int8_t)l3;
    if (zq_out) zq_out[(long)row * RQ + lane] = myz;
  }
  if (lane == 0) fexp[row] = F;
}

}  // namespace oa
