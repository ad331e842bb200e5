// Directed rounding by error-free transformations, for gfx950 device code.
//
// AMDGCN has no per-instruction rounding mode, so the checkers' "round upward" operations are
// built from round-to-nearest ones:
//   add_up(a, b): s = RN(a + b) and its exact error e = (a + b) - s by Knuth's TwoSum (exact
//                 whenever s is finite); RU(a + b) = next_up(s) if e > 0, else s.
//   mul_up(a, b): p = RN(a b) and its error e = fma(a, b, -p), exact unless a b is near the
//                 underflow range; RU(a b) = next_up(p) if e > 0, else p.  Below 2^-960 the
//                 residual may be inexact, so p is raised unconditionally, which still bounds
//                 a b from above (RU(a b) <= next_up(RN(a b)) always).
// Both return exactly the round-upward result except in that tiny-product case, where they
// may return one ulp more; every result is an upper bound of the exact value, which is all the
// thresholds need (every part of tau rounded up, the hypothesis of the reference's T3).
// The library is compiled with -ffp-contract=off so the compiler cannot fuse or reassociate
// these sequences.

#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pck {

__device__ __forceinline__ double next_up(double v) {
  if (v != v || v == __builtin_inf()) return v;
  if (v == 0.0) return 0x1p-1074;  // from +-0 to the smallest subnormal
  const int64_t bits = __double_as_longlong(v);
  return __longlong_as_double(v > 0.0 ? bits + 1 : bits - 1);
}

__device__ __forceinline__ double add_up(double a, double b) {
  const double s = a + b;
  if (s == -__builtin_inf() && a != -__builtin_inf() && b != -__builtin_inf())
    return -__DBL_MAX__;  // negative overflow rounds up to the most negative finite
  if (s != s || s == __builtin_inf() || s == -__builtin_inf()) return s;
  const double bv = s - a;
  const double err = (a - (s - bv)) + (b - bv);
  return err > 0.0 ? next_up(s) : s;
}

__device__ __forceinline__ double mul_up(double a, double b) {
  const double p = a * b;
  if (p != p || p == __builtin_inf()) return p;
  if (p == -__builtin_inf()) {
    return (a == -__builtin_inf() || b == -__builtin_inf() || a == __builtin_inf() ||
            b == __builtin_inf())
               ? p
               : -__DBL_MAX__;
  }
  if (p == 0.0) {
    if (a == 0.0 || b == 0.0) return p;  // exact zero
    return next_up(p);                    // a nonzero product that underflowed
  }
  if (__builtin_fabs(p) < 0x1p-960) return next_up(p);
  const double err = __builtin_fma(a, b, -p);
  return err > 0.0 ? next_up(p) : p;
}

}  // namespace pck

namespace pck {

// RU(a + b) for a, b >= 0 without branches (the checkers' sums of magnitudes): the TwoSum
// error decides whether the round-to-nearest sum is raised by one ulp; +inf stays +inf (its
// error is NaN, which compares false); 0 + 0 stays +0.
__device__ __forceinline__ double add_up_nonneg(double a, double b) {
  const double s = a + b;
  const double bv = s - a;
  const double err = (a - (s - bv)) + (b - bv);
  const double raised = __longlong_as_double(__double_as_longlong(s) + 1);
  return err > 0.0 ? raised : s;
}

// mul_up(a, b) for a, b >= +0 without branches, with the same result there: a zero factor
// keeps +0; a product of nonzero factors below 2^-960 (an underflow to 0 included) is raised
// one ulp from its round-to-nearest value, any other when the FMA residual is positive; +inf
// and NaN pass through (their residual is NaN).
__device__ __forceinline__ double mul_up_pos(double a, double b) {
  const double p = a * b;
  const double err = __builtin_fma(a, b, -p);
  const bool tiny = p < 0x1p-960 && a != 0.0 && b != 0.0;
  const double raised = __longlong_as_double(__double_as_longlong(p) + 1);
  return (err > 0.0 || tiny) ? raised : p;
}

// RU(a b) for a, b >= 0 without branches: raised by one ulp when the FMA residual is positive
// or the product is below 2^-960 (where the residual may be inexact; raising still bounds a b
// from above); +inf stays +inf (its residual is -inf or NaN) and NaN stays NaN.
__device__ __forceinline__ double mul_up_nonneg(double a, double b) {
  const double p = a * b;
  const double err = __builtin_fma(a, b, -p);
  const double raised = __longlong_as_double(__double_as_longlong(p) + 1);
  return (err > 0.0 || p < 0x1p-960) ? raised : p;
}

}  // namespace pck
