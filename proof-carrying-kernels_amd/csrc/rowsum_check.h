// The row-sum check: the blocked checker's relation evaluated from the per-row FP64 sums
// (d_i, s_i) that an in-pass GEMV launch wrote, with no checksum bank.  Shared by the
// standalone launch (checker.hip) and by GEMV launches that carry checks of earlier outputs
// (gemv.hip), so both give bit-identical rho, tau and verdicts.
//
// For check k and row block beta of `block` rows (reference relation:
// src/pck/cuda/csrc/checker_kernel.cu:115-183, with c . x = (r^T W) x evaluated as r^T (W x)):
//   rho = sum_i r_i d_i - sum_i r_i y_i           FP64, round to nearest
//   s   = s_factor * (sum_i s_i rounded up), rounded up, then up to FP32
//   tau = coef s + geps ((1 + u32) s + sum |y_i|) + tau_floor, every operation rounded up
// and the block passes only if every y_i is finite, tau is finite and |rho| <= tau.
//
// Why the threshold is sound.  The products p_j are exact in FP32 (barring underflow, at most
// 2^-150 each, which tau_floor's 2 b n 2^-150 term covers for d and s).  d_i adds them in pairs
// in FP32, each pair within u32 (|p0| + |p1|), so sum_i |r_i (d_i - (W x)_i)| <= u32 S + (FP64
// error) with S = sum_{i, j} |W_ij x_j|: the same u32 S that coef = gamma_h + u32 reserves in
// the bank checker for c's FP32 rounding.  s_i is the FP32 RN sum of |p_j| of depth D (a lane's
// (T / min(T, 64)) ceil(ceil(n / V) / T) V terms plus the butterfly's levels), so
// S_i <= s_i / (1 - gamma_D(u32)) <= s_i s_factor.  The FP64 sums (d's pair sums, the check's
// per-lane sums and butterfly, the final subtraction) are within gamma_H(u64) (S + sum |y|) for
// H >= D + ceil(b / 64) + 7, which geps covers.  gamma_h s covers the GEMV tree's own error as
// in the bank checker (T2/T3); s here bounds the exact S, where the bank's a . |x| carries the
// BF16 rounding of a on top.

// Order (fixed, so results do not depend on scheduling): lane l of the wave adds rows
// l, l + 64, l + 128, ... in increasing order into cx, r.y (round to nearest) and s, sum |y|
// (round up, error-free), then the lanes combine by an xor butterfly over offsets 32, 16, ..., 1
// (each combination is symmetric, so every lane ends with the same value).

#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace rowsum {

constexpr int kWave = 64;
constexpr double kOnePlusU32 = 1.0 + 0x1p-24;  // exact in FP64

// The smallest FP32 value >= v (v >= 0), widened back to FP64; +inf beyond the FP32 range.
__device__ __forceinline__ double up_to_f32(double v) {
  float f = static_cast<float>(v);
  if (static_cast<double>(f) < v) f = __uint_as_float(__float_as_uint(f) + 1u);
  return static_cast<double>(f);
}

// Checks work item `item` of `batch` (one (check, block) pair) with the calling wave; lane 0
// writes passed, rho and tau.  Every lane of the wave must call it (the butterfly).
__device__ __forceinline__ void check_item(const PckRowSumBatch& batch, int64_t item) {
  int g = 0;
  while (g + 1 < batch.count && item >= batch.start[g + 1]) ++g;
  const PckRowSumCheckDesc& d = batch.desc[g];
  const int64_t pair = item - batch.start[g];  // k * num_blocks + beta
  const int64_t beta = pair % d.num_blocks;
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const double2* sums = reinterpret_cast<const double2*>(d.sums) + beta * d.block;
  const float* y = d.y + beta * d.block;
  const int8_t* r = d.r + pair * d.block;

  double cx = 0.0, ry = 0.0, s = 0.0, ya = 0.0;
  for (int64_t i = lane; i < d.block; i += kWave) {
    const double2 ds = sums[i];
    const double yi = static_cast<double>(y[i]);
    const bool neg = r[i] < 0;
    cx = cx + (neg ? -ds.x : ds.x);
    ry = ry + (neg ? -yi : yi);
    s = add_up_nonneg(s, ds.y);
    ya = add_up_nonneg(ya, __builtin_fabs(yi));
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) {
    const double ocx = __shfl_xor(cx, off, kWave);
    const double ory = __shfl_xor(ry, off, kWave);
    const double os = __shfl_xor(s, off, kWave);
    const double oya = __shfl_xor(ya, off, kWave);
    cx = cx + ocx;
    ry = ry + ory;
    s = add_up_nonneg(s, os);
    ya = add_up_nonneg(ya, oya);
  }
  if (lane == 0) {
    const double s_up = up_to_f32(mul_up_nonneg(s, d.s_factor));
    const double rho = cx - ry;
    const double cabs_up = mul_up(kOnePlusU32, s_up);
    const double eps = mul_up(d.geps, add_up(cabs_up, ya));
    const double tau = add_up(add_up(mul_up(d.coef, s_up), eps), d.tau_floor);
    // Non-finite outputs, weights or activations (s or tau non-finite) fail closed; NaN
    // compares false.
    d.passed[pair] =
        __builtin_isfinite(ya) && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
    d.rho[pair] = rho;
    d.tau[pair] = tau;
  }
}

// Host-side validation: every descriptor's shape, non-negative finite constants, 16-byte
// aligned sums, and the work-item prefix sums (one item per (check, block) pair).
inline hipError_t validate(const PckRowSumBatch& batch) {
  if (batch.count < 0 || batch.count > PCK_MAX_BATCH || batch.start[0] != 0)
    return hipErrorInvalidValue;
  for (int g = 0; g < batch.count; ++g) {
    const PckRowSumCheckDesc& d = batch.desc[g];
    const bool finite = __builtin_isfinite(d.coef) && __builtin_isfinite(d.geps) &&
                        __builtin_isfinite(d.tau_floor) && __builtin_isfinite(d.s_factor);
    if (d.num_blocks < 1 || d.checks < 1 || d.block < 1 || !d.sums || !d.y || !d.r ||
        !d.passed || !d.rho || !d.tau || (reinterpret_cast<uintptr_t>(d.sums) & 15) != 0 ||
        !finite || d.coef < 0 || d.geps < 0 || d.tau_floor < 0 || d.s_factor < 1.0 ||
        batch.start[g + 1] - batch.start[g] != static_cast<int64_t>(d.checks) * d.num_blocks)
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

__host__ __device__ inline int64_t items(const PckRowSumBatch& batch) {
  return batch.start[batch.count];
}

}  // namespace rowsum
}  // namespace pck
