// Directed rounding by error-free transformations, for gfx950 device code.
//
// AMDGCN has no per-instruction rounding mode, so the checkers' "round upward" operations are
// built from round-to-nearest ones (the hot upward sums of non-negative terms instead switch
// the wave's rounding mode around their adds: add_up_rm2 / add_up_rm4 below):
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

// In-hardware upward additions for the checkers' inner loops and reductions: every a_i becomes
// RU(a_i + b_i), one v_add_f64 each, issued while the wave's FP64 rounding mode (MODE bits 3:2,
// which FP16 shares) is round toward +inf.  The mode write, the adds and the write that sets
// the mode back to round to nearest even (the kernel's mode) form one asm block, so no
// instruction the compiler schedules runs under the upward mode; each mode write is followed
// by two wait states (s_nop 1) before anything that may depend on it.  The result is the
// correctly rounded upward sum for any operands (NaN propagates as in any add), so for
// a, b >= 0 it has add_up_nonneg's bits.  It replaces a TwoSum of seven dependent operations
// by one add.
__device__ __forceinline__ void add_up_rm2(double& a0, double b0, double& a1, double b1) {
  __asm__ volatile(
      "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 1\n\t"
      "s_nop 1\n\t"
      "v_add_f64 %0, %0, %2\n\t"
      "v_add_f64 %1, %1, %3\n\t"
      "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 0\n\t"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(b0), "v"(b1));
}

__device__ __forceinline__ void add_up_rm4(double (&a)[4], double b0, double b1, double b2,
                                           double b3) {
  __asm__ volatile(
      "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 1\n\t"
      "s_nop 1\n\t"
      "v_add_f64 %0, %0, %4\n\t"
      "v_add_f64 %1, %1, %5\n\t"
      "v_add_f64 %2, %2, %6\n\t"
      "v_add_f64 %3, %3, %7\n\t"
      "s_setreg_imm32_b32 hwreg(HW_REG_MODE, 2, 2), 0\n\t"
      "s_nop 1"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3])
      : "v"(b0), "v"(b1), "v"(b2), "v"(b3));
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
