// Shared device helpers for the OpenAttention sparse-decode kernels (gfx950, wave64).
//
// Conventions used by every kernel in this library:
//   * head_dim D is 128 (Llama-3.1-8B shapes); the host entry points reject anything else.
//   * one wavefront is 64 lanes; a "lane group" is 16 consecutive lanes.
//   * all reductions that feed a discrete decision (top-k, quota, argmax) use a fixed
//     butterfly order (xor 1,2,4,8,16,32 over the 64 lanes), so every lane ends with the
//     same bits and the CPU restatement can replay the exact order.
//   * the library is compiled with -ffp-contract=off: a fused multiply-add only happens
//     where the source calls fmaf()/fma() explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "openattention_amd.h"

#define OA_D 128
#define OA_WAVE 64

namespace oa {

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// round-to-nearest-even fp32 -> bf16 (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// the same rounding by the gfx950 conversion instruction (v_cvt_pk_bf16_f32): equal to
// f32_to_bf16 for every input that is not a NaN (checked on the device over 2^24 values with
// denormals and exact ties); for finite-or-infinite operands only
__device__ __forceinline__ uint16_t f32_to_bf16_rn(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// one output element: fp32 as is, or rounded to bf16
__device__ __forceinline__ void store_out(void* out, int out_f32, long idx, float v) {
  if (out_f32)
    static_cast<float*>(out)[idx] = v;
  else
    static_cast<uint16_t*>(out)[idx] = f32_to_bf16(v);
}

// unpack 8 bf16 (one 16-byte load) into floats
__device__ __forceinline__ void unpack8(const uint4 w, float* x) {
  x[0] = __uint_as_float(w.x << 16); x[1] = __uint_as_float(w.x & 0xffff0000u);
  x[2] = __uint_as_float(w.y << 16); x[3] = __uint_as_float(w.y & 0xffff0000u);
  x[4] = __uint_as_float(w.z << 16); x[5] = __uint_as_float(w.z & 0xffff0000u);
  x[6] = __uint_as_float(w.w << 16); x[7] = __uint_as_float(w.w & 0xffff0000u);
}

// ---- butterfly reductions over the full wave (every lane gets the result) -------------------
// Canonical order: the xor butterfly with m = 1, 2, 4, 8, 16, 32 (lane l adds the value of lane
// l ^ m at each level).  Each level maps onto a cross-lane primitive that delivers exactly the
// partner's value: quad_perm [1,0,3,2] (m=1) and [2,3,0,1] (m=2); row_half_mirror (m=4) and
// row_mirror (m=8), whose sources lie in the partner's quad / 8-lane group, which is uniform by
// then; v_permlane16_swap / v_permlane32_swap (m=16, 32), whose two results are the lane's own
// value and its partner's.  Addition is commutative, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xf,
                                                    0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp((int)b, (int)b, CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp((int)(b >> 32), (int)(b >> 32), CTRL, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ float swap16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ double swap16_sum(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
  const double x = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0]));
  const double y = __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  return x + y;
}
__device__ __forceinline__ double swap32_sum(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
  const double x = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0]));
  const double y = __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  return x + y;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_f32<0xB1>(v);     // m = 1
  v = v + dpp_f32<0x4E>(v);     // m = 2
  v = v + dpp_f32<0x141>(v);    // m = 4
  v = v + dpp_f32<0x140>(v);    // m = 8
  v = swap16_sum(v);            // m = 16
  return swap32_sum(v);         // m = 32
}
__device__ __forceinline__ double wave_sum(double v) {
  v = v + dpp_f64<0xB1>(v);
  v = v + dpp_f64<0x4E>(v);
  v = v + dpp_f64<0x141>(v);
  v = v + dpp_f64<0x140>(v);
  v = swap16_sum(v);
  return swap32_sum(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ int wave_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(v, v, 0x140, 0xf, 0xf, false);
  const auto r16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = (int)(r16[0] + r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return (int)(r32[0] + r32[1]);
}
// inclusive prefix sum over the wave's lanes on the DPP network (row shifts inside each 16-lane
// row, then row_bcast15 / row_bcast31 carry the row totals upward); integers, so exact
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return v;
}
// sum inside each aligned 16-lane group (a DPP row), order m = 1, 2, 4, 8
__device__ __forceinline__ float group16_sum(float v) {
  v = v + dpp_f32<0xB1>(v);
  v = v + dpp_f32<0x4E>(v);
  v = v + dpp_f32<0x141>(v);
  return v + dpp_f32<0x140>(v);
}
// the maximum of each 16-lane row, in every lane of the row (the same DPP folds)
__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  return fmaxf(v, dpp_f32<0x140>(v));
}
__device__ __forceinline__ float group16_min(float v) {
  v = fminf(v, dpp_f32<0xB1>(v));
  v = fminf(v, dpp_f32<0x4E>(v));
  v = fminf(v, dpp_f32<0x141>(v));
  return fminf(v, dpp_f32<0x140>(v));
}

// ---- order-independent reductions on the DPP network (no LDS round trips) ------------------
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror fold each 16-lane row;
// row_bcast15 (rows 1, 3) and row_bcast31 (rows 2, 3) fold the rows into lane 63, which is then
// read into a scalar: every lane returns the wave's maximum.  Lanes a DPP step does not write
// keep their own value (old = src), so max() leaves them unchanged.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWMASK, 0xf, false);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ unsigned long long dpp_max_u64_step(unsigned long long v) {
  const unsigned lo = dpp_u32<CTRL, ROWMASK>((unsigned)v);
  const unsigned hi = dpp_u32<CTRL, ROWMASK>((unsigned)(v >> 32));
  const unsigned long long o = ((unsigned long long)hi << 32) | lo;
  return o > v ? o : v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  v = dpp_max_u64_step<0xB1, 0xf>(v);    // quad_perm [1,0,3,2]
  v = dpp_max_u64_step<0x4E, 0xf>(v);    // quad_perm [2,3,0,1]
  v = dpp_max_u64_step<0x141, 0xf>(v);   // row_half_mirror
  v = dpp_max_u64_step<0x140, 0xf>(v);   // row_mirror
  v = dpp_max_u64_step<0x142, 0xa>(v);   // row_bcast15
  v = dpp_max_u64_step<0x143, 0xc>(v);   // row_bcast31
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, 63);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), 63);
  return ((unsigned long long)hi << 32) | lo;
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ unsigned dpp_max_u32_step(unsigned v) {
  const unsigned o = dpp_u32<CTRL, ROWMASK>(v);
  return o > v ? o : v;
}
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
  v = dpp_max_u32_step<0xB1, 0xf>(v);
  v = dpp_max_u32_step<0x4E, 0xf>(v);
  v = dpp_max_u32_step<0x141, 0xf>(v);
  v = dpp_max_u32_step<0x140, 0xf>(v);
  v = dpp_max_u32_step<0x142, 0xa>(v);
  v = dpp_max_u32_step<0x143, 0xc>(v);
  return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}


// Canonical 128-term fp32 dot product used wherever the result feeds a discrete decision:
// lane l holds elements l and l+64; p_l = fma(a[l+64], b[l+64], a[l]*b[l]); then the wave
// butterfly (m = 1, 2, ..., 32).  Every lane returns the same value.
__device__ __forceinline__ float dot128_canon(float a_lo, float b_lo, float a_hi, float b_hi) {
  float p = fmaf(a_hi, b_hi, a_lo * b_lo);
  return wave_sum(p);
}

// workgroup barrier that orders LDS only: waits for this wave's LDS operations, not for its
// global loads still in flight (__syncthreads() also drains those)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// XCD-aware row of a one-row-per-workgroup launch: workgroups go to the 8 XCDs round-robin
// (workgroup b to XCD b % 8), each XCD with its own L2; this bijection gives XCD x the rows
// [x rows/8, (x+1) rows/8), so the query-head rows of one KV row (consecutive rows) share an L2.
// Identity when rows is not a multiple of 8.
__device__ __forceinline__ int xcd_row(int b, int rows) {
  return (rows & 7) ? b : (b & 7) * (rows >> 3) + (b >> 3);
}

// order-preserving uint32 image of a float (larger float -> larger key, -inf lowest)
__device__ __forceinline__ uint32_t float_key(float s) {
  const uint32_t b = __float_as_uint(s);
  // negative: flip every bit; non-negative: set the sign bit
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

}  // namespace oa

// host-side launch status helper: the last launch error as an int
#define OA_LAUNCH_STATUS() ((int)hipGetLastError())
