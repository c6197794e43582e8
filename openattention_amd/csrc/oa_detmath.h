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
//   erf  : Maclaurin series (2/sqrt(pi)) sum (-1)^n x^(2n+1) / (n! (2n+1)), 80 terms, for
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

__device__ __forceinline__ float det_erff(float xf) {
  const double x = (double)xf;
  if (x != x) return xf;
  const double ax = x < 0.0 ? -x : x;
  if (ax >= 4.0) return x < 0.0 ? -1.0f : 1.0f;
  const double mx2 = -(ax * ax);
  double t = ax, sum = ax;
  for (int n = 1; n <= 80; ++n) {
    t = (t * mx2) / (double)n;
    sum = sum + t / (double)(2 * n + 1);
  }
  const double r = sum * 0x1.20dd750429b6dp+0;  // 2/sqrt(pi)
  const float rf = (float)r;
  return x < 0.0 ? -rf : rf;
}

}  // namespace oa
