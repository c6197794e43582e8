// Exact QGS score of one token, recomputed from its int8 code with the scan's arithmetic.
//
// The scan multiplies a KV head's 16 limb rows (4 query heads x 4 signed 8-bit limbs of
// Z_r = rint(zq_r 2^F)) by the 32-byte codes of 16 tokens on the int8 matrix cores, recombines
// the four exact int32 limb dots in fp64 and rounds once: score = fp32(S_int 2^-F).  The same
// integers come out of four v_dot4_i32_i8 chains, so a score recomputed here is bit for bit the
// scan's.  Kernels that keep only 16-bit key heads of the scores use this for the few tokens
// whose exact order matters.
#pragma once

#include "oa_common.h"

namespace oa {

// the four limb rows of query head g of KV row kvr as 8 packed words each: lw[k*8 + w] holds
// limb k of QGS dims 4w .. 4w+3 (limbs laid out (BH, 16, 32), rows g*4 + k)
__device__ __forceinline__ const int* limb_words(const int8_t* limbs, int kvr, int g) {
  return reinterpret_cast<const int*>(limbs + ((long)kvr * 16 + g * 4) * 32);
}

// the exact score of a token from its 32-byte code (two 16-byte words c0, c1); lw as above,
// inv = 2^-F of the query row
__device__ __forceinline__ float qgs_score_words(uint4 c0, uint4 c1, const int* lw, double inv) {
  const int cw[8] = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w,
                     (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
  int acc[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int w = 0; w < 8; ++w) acc[k] = __builtin_amdgcn_sdot4(cw[w], lw[k * 8 + w], acc[k], false);
  double s = (double)acc[3];
  s = fma(s, 256.0, (double)acc[2]);
  s = fma(s, 256.0, (double)acc[1]);
  s = fma(s, 256.0, (double)acc[0]);
  return (float)(s * inv);
}

// the exact score of token pos of KV row kvr (codes laid out (BH, Lmax, 32))
__device__ __forceinline__ float qgs_score(const int8_t* codes, long lmax, int kvr, int pos,
                                           const int* lw, double inv) {
  const uint4* cp = reinterpret_cast<const uint4*>(codes + ((long)kvr * lmax + pos) * 32);
  const uint4 c0 = cp[0], c1 = cp[1];
  const int cw[8] = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w,
                     (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
  int acc[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int w = 0; w < 8; ++w) acc[k] = __builtin_amdgcn_sdot4(cw[w], lw[k * 8 + w], acc[k], false);
  double s = (double)acc[3];
  s = fma(s, 256.0, (double)acc[2]);
  s = fma(s, 256.0, (double)acc[1]);
  s = fma(s, 256.0, (double)acc[0]);
  return (float)(s * inv);
}

// the same with the limb words read from LDS one limb row at a time (few registers: for
// kernels running close to their register budget)
__device__ __forceinline__ float qgs_score_lds(const int8_t* codes, long lmax, int kvr, int pos,
                                               const int* s_lw, double inv) {
  const uint4* cp = reinterpret_cast<const uint4*>(codes + ((long)kvr * lmax + pos) * 32);
  const uint4 c0 = cp[0], c1 = cp[1];
  const int cw[8] = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w,
                     (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
  int acc[4];
#pragma unroll 1
  for (int k = 0; k < 4; ++k) {
    int a = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) a = __builtin_amdgcn_sdot4(cw[w], s_lw[k * 8 + w], a, false);
    acc[k] = a;
  }
  double s = (double)acc[3];
  s = fma(s, 256.0, (double)acc[2]);
  s = fma(s, 256.0, (double)acc[1]);
  s = fma(s, 256.0, (double)acc[0]);
  return (float)(s * inv);
}

// 16-bit head of a score's order-preserving key (non-decreasing in the score; -inf -> 0x007f,
// the least finite score -> 0x0080)
__device__ __forceinline__ uint16_t score_head(float s) { return (uint16_t)(float_key(s) >> 16); }
constexpr uint16_t kNegInfHead = 0x007f;

}  // namespace oa
