// Deterministic elementary functions for the decision path of the decode stage.
//
// The ErrorGate cluster score (log, erf) and the water-filling weights (exp, log) decide
// integer quotas through floor(lambda * w_b) and comparisons, so the GPU result must be the
// same bits as the CPU restatement.  Vendor libm/ocml implementations differ from glibc, so
// these functions are written with IEEE-exact primitives only (+, -, *, /, explicit fma,
// ldexp, frexp, rint) and fixed term counts.  Accuracy is ~1 ulp in double; the fp32
// wrappers evaluate in double and round once.
//
//   exp  : Cody-Waite reduction x = k ln2 + r (fdlibm split of ln2), Taylor to r^13 on
//          |r| <= ln2/2 (truncation < 4e-18), scaled by 2^k with ldexp.
//   log  : x = m 2^e, m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(f), f = (m-1)/(m+1),
//          series in f^2 to f^23 (|f| <= 0.1716, truncation < 1e-18).
//   erf  : Maclaurin series erf(x) = (2/sqrt(pi)) x sum_n c_n x^(2n), c_n = (-1)^n/(n!(2n+1))
//          rounded to double, 72 terms in Horner form (truncation < 2e-18 at |x| = 4), for
//          |x| < 4; erf(x) = sign(x) beyond (erf(4) rounds to 1.0f).
#pragma once
#include <hip/hip_runtime.h>

namespace oa {

__device__ __forceinline__ double det_exp(double x) {
  if (x != x) return x;
  if (x > 709.782712893384) return __longlong_as_double(0x7ff0000000000000LL);
  if (x < -745.2) return 0.0;
  const double k = rint(x * 0x1.71547652b82fep+0);
  double r = fma(-k, 0x1.62e42fee00000p-1, x);
  r = fma(-k, 0x1.a39ef35793c76p-33, r);
  double p = 0x1.6124613a86d09p-33;          // 1/13!
  p = fma(p, r, 0x1.1eed8eff8d898p-29);      // 1/12!
  p = fma(p, r, 0x1.ae64567f544e4p-26);      // 1/11!
  p = fma(p, r, 0x1.27e4fb7789f5cp-22);      // 1/10!
  p = fma(p, r, 0x1.71de3a556c734p-19);      // 1/9!
  p = fma(p, r, 0x1.a01a01a01a01ap-16);      // 1/8!
  p = fma(p, r, 0x1.a01a01a01a01ap-13);      // 1/7!
  p = fma(p, r, 0x1.6c16c16c16c17p-10);      // 1/6!
  p = fma(p, r, 0x1.1111111111111p-7);       // 1/5!
  p = fma(p, r, 0x1.5555555555555p-5);       // 1/4!
  p = fma(p, r, 0x1.5555555555555p-3);       // 1/3!
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  return ldexp(p, (int)k);
}

// det_exp without branches, the same bits for every input: the polynomial runs on x clamped into
// the finite range (x itself there) and the out-of-range results are selected afterwards, so the
// lanes of a wave that hold different x never split the wave
__device__ __forceinline__ double det_exp_v(double x) {
  const double xc = fmin(fmax(x, -745.2), 709.782712893384);
  const double k = rint(xc * 0x1.71547652b82fep+0);
  double r = fma(-k, 0x1.62e42fee00000p-1, xc);
  r = fma(-k, 0x1.a39ef35793c76p-33, r);
  double p = 0x1.6124613a86d09p-33;
  p = fma(p, r, 0x1.1eed8eff8d898p-29);
  p = fma(p, r, 0x1.ae64567f544e4p-26);
  p = fma(p, r, 0x1.27e4fb7789f5cp-22);
  p = fma(p, r, 0x1.71de3a556c734p-19);
  p = fma(p, r, 0x1.a01a01a01a01ap-16);
  p = fma(p, r, 0x1.a01a01a01a01ap-13);
  p = fma(p, r, 0x1.6c16c16c16c17p-10);
  p = fma(p, r, 0x1.1111111111111p-7);
  p = fma(p, r, 0x1.5555555555555p-5);
  p = fma(p, r, 0x1.5555555555555p-3);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  double e = ldexp(p, (int)k);
  e = x > 709.782712893384 ? __longlong_as_double(0x7ff0000000000000LL) : e;
  e = x < -745.2 ? 0.0 : e;
  return x != x ? x : e;
}

__device__ __forceinline__ double det_log(double x) {
  if (x != x) return x;
  if (x < 0.0) return __longlong_as_double(0x7ff8000000000000LL);
  if (x == 0.0) return __longlong_as_double((long long)0xfff0000000000000ULL);
  if (x == __longlong_as_double(0x7ff0000000000000LL)) return x;
  int e;
  double m = frexp(x, &e);                   // m in [0.5, 1)
  if (m < 0x1.6a09e667f3bcdp-1) {            // sqrt(1/2)
    m = m * 2.0;
    e = e - 1;
  }
  const double f = (m - 1.0) / (m + 1.0);
  const double s = f * f;
  double p = 1.0 / 23.0;
  p = fma(p, s, 1.0 / 21.0);
  p = fma(p, s, 1.0 / 19.0);
  p = fma(p, s, 1.0 / 17.0);
  p = fma(p, s, 1.0 / 15.0);
  p = fma(p, s, 1.0 / 13.0);
  p = fma(p, s, 1.0 / 11.0);
  p = fma(p, s, 1.0 / 9.0);
  p = fma(p, s, 1.0 / 7.0);
  p = fma(p, s, 1.0 / 5.0);
  p = fma(p, s, 1.0 / 3.0);
  p = fma(p, s, 1.0);
  const double lm = 2.0 * f * p;
  const double de = (double)e;
  return fma(de, 0x1.62e42fee00000p-1, fma(de, 0x1.a39ef35793c76p-33, lm));
}

__device__ __forceinline__ float det_logf(float x) { return (float)det_log((double)x); }

__device__ __constant__ const double kErfC[72] = {
    0x1.0000000000000p+0, -0x1.5555555555555p-2, 0x1.999999999999ap-4,
    -0x1.8618618618618p-6, 0x1.2f684bda12f68p-8, -0x1.8d3018d3018d3p-11,
    0x1.c01c01c01c01cp-14, -0x1.bbd779334ef0bp-17, 0x1.87a00187a0018p-20,
    -0x1.3777c55568ccdp-23, 0x1.c2e3054870b38p-27, -0x1.2b67310aa9f3ap-30,
    0x1.6f448e13e85e1p-34, -0x1.a289ee7e40f74p-38, 0x1.bd577e658d020p-42,
    -0x1.bc6250fb14231p-46, 0x1.a173a167fba4dp-50, -0x1.7271cbe5863ecp-54,
    0x1.377c2110f2083p-58, -0x1.f1b4073b34a68p-63, 0x1.7abd72258fb6ep-67,
    -0x1.13246abce1bddp-71, 0x1.7e6b81382cd42p-76, -0x1.fd6bebd65107ap-81,
    0x1.45c0a838efe59p-85, -0x1.909c9de3a31c5p-90, 0x1.da7460554e5dbp-95,
    -0x1.0eef30fa10d2cp-99, 0x1.2ac65385f79acp-104, -0x1.3e81bb5701ac5p-109,
    0x1.4899fcdef0a8dp-114, -0x1.486eea20c2656p-119, 0x1.3e53defc4e233p-124,
    -0x1.2b778acc3dedfp-129, 0x1.11ae81077a49ep-134, -0x1.e6597092ccbf0p-140,
    0x1.a47767f2a3c32p-145, -0x1.61f30bc3acd1ap-150, 0x1.22521d98f98a9p-155,
    -0x1.d05cc9e3507c9p-161, 0x1.6a513f56f8a2fp-166, -0x1.13f85fc9e143ep-171,
    0x1.9aa19d4d16643p-177, -0x1.2a8fa59ffec31p-182, 0x1.a8830736a5123p-188,
    -0x1.273d8edcec957p-193, 0x1.91ef82b367a95p-199, -0x1.0be5a4cd94283p-204,
    0x1.5dd4c9219115ap-210, -0x1.bfb10e0f68c50p-216, 0x1.18d952ef00889p-221,
    -0x1.59982b2e94840p-227, 0x1.a13ec00b39f6fp-233, -0x1.ee6cefaa5a158p-239,
    0x1.1f9dec94da5f8p-244, -0x1.48a6b3820b441p-250, 0x1.70f41ac13e2a1p-256,
    -0x1.970f1cb2ad53fp-262, 0x1.b97d90d3e603bp-268, -0x1.d6db2a7c68dcbp-274,
    0x1.edf1e6e4658a9p-280, -0x1.fdcf88bbf71dbp-286, 0x1.02eb04e5f82f5p-291,
    -0x1.02e2bc1b5790ep-297, 0x1.fdbe706576d5dp-304, -0x1.ee3d33862f55bp-310,
    0x1.d80e20102c46ep-316, -0x1.bc3cf47bca3afp-322, 0x1.9c00b17fe33c8p-328,
    -0x1.78a61f51a767fp-334, 0x1.537ae8ecb0688p-340, -0x1.2dbafa5779b80p-346,
};

__device__ __forceinline__ float det_erff(float xf) {
  const double x = (double)xf;
  if (x != x) return xf;
  const double ax = x < 0.0 ? -x : x;
  if (ax >= 4.0) return x < 0.0 ? -1.0f : 1.0f;
  const double x2 = ax * ax;
  // the coefficients through vector loads (returned in order), so that the compiler keeps a
  // few ahead of the fma chain instead of waiting on each batch of scalar loads
  const double* tb = kErfC;
  asm volatile("" : "+v"(tb));
  double s = tb[71];
#pragma unroll
  for (int n = 70; n >= 0; --n) s = fma(s, x2, tb[n]);
  const double r = (ax * s) * 0x1.20dd750429b6dp+0;  // 2/sqrt(pi)
  const float rf = (float)r;
  return x < 0.0 ? -rf : rf;
}

}  // namespace oa
