// e^x in float64 with few registers, for the SiLU gate's
// float32(exp(-float64(g))) (stablelm.go:371-373, model.go:463-470), where
// only the float32 rounding of the result is used.
//
// Method (Cody-Waite reduction, Taylor kernel): k = rint(x / ln 2),
// r = x - k ln 2 with ln 2 split in a 32-bit head (k * head is exact) and a
// tail, both steps fused; e^r by the Taylor series to r^13 / 13!
// (|r| <= ln2/2: the first dropped term is below 4e-18 relative), Horner
// with fused multiply-adds; then the exact scaling by 2^k (ldexp also
// rounds once into the subnormal range). Within 2 ulp of e^x in float64,
// so its float32 rounding equals the correctly rounded float32 of e^x
// except where e^x lies within ~2 float64 ulp of a float32 rounding
// boundary. Overflow gives +inf, underflow 0, NaN stays NaN.
//
// Plain C++ (fma, rint, ldexp) so the host test suite checks the same
// arithmetic against the C library; every operation is an IEEE operation
// with one rounding, identical on the host and on gfx950.
#pragma once

#include <cmath>

#ifdef __HIPCC__
#define TINYOAI_HD __host__ __device__
#else
#define TINYOAI_HD
#endif

TINYOAI_HD inline double exp_f64(double x) {
  if (x != x) return x;
  if (x > 709.782712893384) return INFINITY;  // e^x > DBL_MAX
  if (x < -745.1332191019412) return 0.0;     // e^x below half the smallest subnormal
  const double kLn2Hi = 0x1.62e42fee00000p-1, kLn2Lo = 0x1.a39ef35793c76p-33, kInvLn2 = 0x1.71547652b82fep+0;
  const double k = rint(x * kInvLn2);
  double r = fma(-k, kLn2Hi, x);
  r = fma(-k, kLn2Lo, r);
  // 1 / n! for n = 13 .. 0
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
  return ldexp(p, (int)k);
}
