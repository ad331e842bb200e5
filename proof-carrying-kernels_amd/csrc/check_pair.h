// The blocked checker's work for one (check, block) pair, by one 256-lane workgroup.  Shared by
// the standalone checker kernel (checker.hip) and by GEMV launches that carry checks of outputs
// produced by earlier launches (gemv.hip), so both give bit-identical rho, tau and verdicts.
//
// Bank (built at weight load by pck.cuda.checker, reference src/pck/cuda/checker.py:72-129):
//   c[k, beta, :] = r[k, beta, :]^T W_beta     FP32, rounded to nearest
//   a[beta, :]    = sum_{i in beta} |W_i|       BF16, rounded up
//   r[k, beta, :] in {-1, +1}                   int8, secret
// For every check k and row block beta (reference src/pck/cuda/csrc/checker_kernel.cu:49-91):
//   rho = c . x - r . y_beta
//   s   = a . |x|                               every operation rounded up
//   tau = coef s + geps ((1 + u32) s + sum |y_beta|) + tau_floor, every operation rounded up
// and the block passes only if every y in it is finite, tau is finite and |rho| <= tau.
//
// Arithmetic.  FP64 runs at the FP32 (non-packed) rate on MI355X, so rho is evaluated entirely
// in FP64: each c_j x_j (24 + 8 significand bits) is exact in FP64 and every addition is one
// FP64 operation, so rho's rounding error is at most gamma_H(u64) (sum |c_j x_j| + sum |y_i|)
// for the depth H <= n + b + 1 of its evaluation, which the host's geps (reference formula,
// which also carries the reference's FP32 Dot2 term) covers.  s and the sums of |y| add exact
// non-negative terms (a_j |x_j| has 16 significand bits) with upward-rounded FP64 additions:
// in the bank loop and the workgroup reduction one add each under the wave's upward rounding
// mode (add_up_rm4 / add_up_rm2), elsewhere the TwoSum form add_up_nonneg, the same bits.  The reference adds the same terms in FP32, rounding up, and then in FP64; since every
// FP32 partial it forms is at least the exact sum, and the FP64 sums here are exact whenever
// its FP32 ones are, this s is at most the reference's (equal on typical inputs), and so is
// tau.  An s beyond the FP32 range becomes +inf (tau = inf, a failed block), as the
// reference's FP32 sum would overflow.  tau's products and sums use the general round-up
// operations.
//
// Order.  Lane t accumulates the y terms of rows t, t + 256, ..., then the bank quads t,
// t + 256, t + 512, ... in increasing order (four accumulators per quantity, one per column of a
// quad); the workgroup reduction is a fixed wave64 butterfly over lane distances 1, 2, 4, 8, 16,
// 32 (so lane 0 holds ((v0 + v1) + (v2 + v3)) + ...) and a fixed halving over the four waves.
// The result does not depend on scheduling or on kAhead (loads issued ahead per lane).

#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace check {

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr double kOnePlusU32 = 1.0 + 0x1p-24;  // exact in FP64

__device__ __forceinline__ double bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ double bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ double bf16_at(const uint16_t* p, int64_t j) {
  return __uint_as_float(static_cast<uint32_t>(p[j]) << 16);
}

// Raw buffer resources for the batched checker: a lane offset at or past `bytes` reads zero.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// The smallest FP32 value >= v (v >= 0), widened back to FP64; +inf beyond the FP32 range
// (the batched checker's bound on s).
__device__ __forceinline__ double round_up_to_f32(double v) {
  float f = static_cast<float>(v);
  if (static_cast<double>(f) < v) f = __uint_as_float(__float_as_uint(f) + 1u);  // v >= 0
  return static_cast<double>(f);
}

// v (>= 0) if it lies within the FP32 range, else +inf: the threshold fails closed where the
// reference's FP32 sum of |a x| would overflow.
__device__ __forceinline__ double within_f32_range(double v) {
  return v <= static_cast<double>(__FLT_MAX__) ? v : __builtin_inf();
}

// The four per-lane quantities: c.x and r.y round to nearest, s and sum |y| round up.
struct Quad {
  double cx, s, ry, yabs;
};

__device__ __forceinline__ Quad combine(const Quad& a, const Quad& b) {
  double s = a.s, yabs = a.yabs;
  add_up_rm2(s, b.s, yabs, b.yabs);  // RU, as add_up_nonneg
  return Quad{a.cx + b.cx, s, a.ry + b.ry, yabs};
}

// v in the lane that DPP pattern kCtrl names (every lane has a source for the patterns used).
template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      0, static_cast<int>(static_cast<uint32_t>(u)), kCtrl, 0xF, 0xF, false));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      0, static_cast<int>(static_cast<uint32_t>(u >> 32)), kCtrl, 0xF, 0xF, false));
  return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}
template <int kCtrl>
__device__ __forceinline__ Quad dpp_quad(const Quad& v) {
  return Quad{dpp_f64<kCtrl>(v.cx), dpp_f64<kCtrl>(v.s), dpp_f64<kCtrl>(v.ry),
              dpp_f64<kCtrl>(v.yabs)};
}
__device__ __forceinline__ double lane_f64(double v, int lane) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), lane));
  const uint64_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), lane));
  return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}
__device__ __forceinline__ Quad lane_quad(const Quad& v, int lane) {
  return Quad{lane_f64(v.cx, lane), lane_f64(v.s, lane), lane_f64(v.ry, lane),
              lane_f64(v.yabs, lane)};
}

// Workgroup sums of the four quantities in one exchange, valid in every lane.  Inside each
// 16-lane row the partners are the lanes at distance 1 and 2 (quad_perm), then the mirror lanes
// in the other quad (row_half_mirror) and the other half-row (row_mirror); every lane of a group
// holds the same value after each level (combine is symmetric in its operands), so this is the
// butterfly over distances 1, 2, 4 and 8.  The rows then combine as (r0 + r1) + (r2 + r3),
// the butterfly's distances 16 and 32, read from lanes 0, 16, 32 and 48.
__device__ __forceinline__ Quad group_sum(Quad v, Quad* lds) {
  v = combine(v, dpp_quad<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = combine(v, dpp_quad<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = combine(v, dpp_quad<0x141>(v));  // row_half_mirror
  v = combine(v, dpp_quad<0x140>(v));  // row_mirror
  v = combine(combine(lane_quad(v, 0), lane_quad(v, 16)),
              combine(lane_quad(v, 32), lane_quad(v, 48)));
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
  __syncthreads();
  Quad w[kWaves];
#pragma unroll
  for (int i = 0; i < kWaves; ++i) w[i] = lds[i];
#pragma unroll
  for (int half = kWaves / 2; half > 0; half /= 2)
#pragma unroll
    for (int i = 0; i < half; ++i) w[i] = combine(w[i], w[i + half]);
  return w[0];
}

// One column: c.x with the exact product (one rounding, the add's) and a.|x| rounded up.
__device__ __forceinline__ void column(double& cx, double& s, double cj, double aj, double xj) {
  cx = __builtin_fma(cj, xj, cx);
  s = add_up_nonneg(s, aj * __builtin_fabs(xj));
}

// The descriptor that owns work item `item`: the number of boundaries start[1 .. count - 1]
// at or below it (start increases), from independent loads rather than a chain of them.
__device__ __forceinline__ int owner(const PckCheckBatch& batch, int64_t item) {
  int g = 0;
#pragma unroll
  for (int j = 1; j < PCK_MAX_BATCH; ++j) g += (j < batch.count && item >= batch.start[j]) ? 1 : 0;
  return g;
}

// Checks work item `item` of `batch` (one (check, block) pair, owned by descriptor g) with the
// calling workgroup of kThreads lanes; `lds` holds kWaves Quads.  Lane 0 writes passed, rho and
// tau.
template <int kAhead>
__device__ __forceinline__ void check_pair(const PckCheckBatch& batch, int64_t item, int g,
                                           Quad* lds) {
  const PckCheckDesc& d = batch.desc[g];
  const int64_t pair = item - batch.start[g];  // k * num_blocks + beta
  const int64_t beta = pair % d.num_blocks;
  const int64_t n = d.n;
  const int t = static_cast<int>(threadIdx.x);
  const float* c_row = d.c + pair * n;
  const uint16_t* a_row = static_cast<const uint16_t*>(d.a) + beta * n;
  const uint16_t* x = static_cast<const uint16_t*>(d.x);
  const int8_t* r_row = d.r + pair * d.block;
  const float* y_blk = d.y + beta * d.block;

  // The y terms.  A block of at most kThreads rows is one value per lane, requested here with
  // unconditional loads (row 0 for lanes past the block, dropped at use: a branch around the
  // loads would make its merge wait for them) and used after the bank's loads are issued;
  // longer blocks loop.  A non-finite y makes sum |y| non-finite (FP32 values cannot overflow
  // an FP64 sum of at most 2^31 of them).
  Quad q{0.0, 0.0, 0.0, 0.0};
  const bool one_y = d.block <= kThreads;
  const int yi = t < d.block ? t : 0;
  const float y_mine = y_blk[yi];
  const int8_t r_mine = r_row[yi];
  if (!one_y) {
    for (int i = t; i < d.block; i += kThreads) {
      const double yd = static_cast<double>(y_blk[i]);
      q.ry = q.ry + (r_row[i] > 0 ? yd : -yd);
      q.yabs = add_up_nonneg(q.yabs, __builtin_fabs(yd));
    }
  }

  // Bank terms: kAhead quads per lane are loaded before any is consumed; indices past the row
  // load quad 0 and their columns are zeroed (c = x = 0 adds exactly nothing), so the loop has
  // no data-dependent branches.
  double cx[4] = {0.0, 0.0, 0.0, 0.0};
  double sa[4] = {0.0, 0.0, 0.0, 0.0};
  int64_t done = 0;
  const bool quads = n % 4 == 0 && (reinterpret_cast<uintptr_t>(c_row) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a_row) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(x) & 7) == 0;
  if (quads) {
    const float4* c4 = reinterpret_cast<const float4*>(c_row);
    const uint2* a4 = reinterpret_cast<const uint2*>(a_row);
    const uint2* x4 = reinterpret_cast<const uint2*>(x);
    const int64_t nq = n / 4;
    for (int64_t q0 = t; q0 < nq; q0 += kAhead * kThreads) {
      float4 cv[kAhead];
      uint2 av[kAhead];
      uint2 xv[kAhead];
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        const int64_t qk = q0 + static_cast<int64_t>(k) * kThreads;
        const int64_t at = qk < nq ? qk : 0;
        cv[k] = c4[at];
        av[k] = a4[at];
        xv[k] = x4[at];
      }
      // All kAhead quads are requested before the first is used (the scheduler would otherwise
      // move loads next to their uses for occupancy, one round trip after another).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        // Columns past the row are zeroed by masking their bits with a word the compiler
        // cannot see through (an empty asm): a select on the loaded value would be compiled
        // into a branch around its load, followed by a wait for every load in flight.
        uint32_t keep = q0 + static_cast<int64_t>(k) * kThreads < nq ? 0xFFFFFFFFu : 0u;
        __asm__("" : "+v"(keep));
        const float4 c = make_float4(__uint_as_float(__float_as_uint(cv[k].x) & keep),
                                     __uint_as_float(__float_as_uint(cv[k].y) & keep),
                                     __uint_as_float(__float_as_uint(cv[k].z) & keep),
                                     __uint_as_float(__float_as_uint(cv[k].w) & keep));
        const uint2 xx = make_uint2(xv[k].x & keep, xv[k].y & keep);
        const double x0 = bf16_lo(xx.x), x1 = bf16_hi(xx.x), x2 = bf16_lo(xx.y),
                     x3 = bf16_hi(xx.y);
        cx[0] = __builtin_fma(static_cast<double>(c.x), x0, cx[0]);
        cx[1] = __builtin_fma(static_cast<double>(c.y), x1, cx[1]);
        cx[2] = __builtin_fma(static_cast<double>(c.z), x2, cx[2]);
        cx[3] = __builtin_fma(static_cast<double>(c.w), x3, cx[3]);
        // a_j |x_j| is exact (16 significand bits); the four sums round upward in hardware
        add_up_rm4(sa, bf16_lo(av[k].x) * __builtin_fabs(x0), bf16_hi(av[k].x) * __builtin_fabs(x1),
                   bf16_lo(av[k].y) * __builtin_fabs(x2), bf16_hi(av[k].y) * __builtin_fabs(x3));
      }
    }
    done = nq * 4;
  }
  for (int64_t j = done + t; j < n; j += kThreads) {
    column(cx[j & 3], sa[j & 3], static_cast<double>(c_row[j]), bf16_at(a_row, j), bf16_at(x, j));
  }
  if (one_y && t < d.block) {
    const double yd = static_cast<double>(y_mine);
    q.ry = r_mine > 0 ? yd : -yd;
    q.yabs = __builtin_fabs(yd);
  }
  q.cx = (cx[0] + cx[2]) + (cx[1] + cx[3]);
  q.s = add_up_nonneg(add_up_nonneg(sa[0], sa[2]), add_up_nonneg(sa[1], sa[3]));

  const Quad total = group_sum(q, lds);
  if (t == 0) {
    const double s_up = within_f32_range(total.s);
    const double rho = total.cx - total.ry;
    double tau;
    if (d.coef >= 0.0 && d.geps >= 0.0 && d.tau_floor >= 0.0) {
      // every operand is >= +0 (or +inf / NaN), where these branch-free forms give the
      // general operations' results
      const double cabs_up = mul_up_pos(kOnePlusU32, s_up);
      const double eps = mul_up_pos(d.geps, add_up_nonneg(cabs_up, total.yabs));
      tau = add_up_nonneg(add_up_nonneg(mul_up_pos(d.coef, s_up), eps), d.tau_floor);
    } else {
      const double cabs_up = mul_up(kOnePlusU32, s_up);
      const double eps = mul_up(d.geps, add_up(cabs_up, total.yabs));
      tau = add_up(add_up(mul_up(d.coef, s_up), eps), d.tau_floor);
    }
    // Non-finite outputs and an overflowing threshold (tau = inf) fail closed; NaN compares
    // false.
    d.passed[pair] =
        __builtin_isfinite(total.yabs) && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
    d.rho[pair] = rho;
    d.tau[pair] = tau;
  }
}

// Host-side validation of a batch: the shape of every descriptor and the work-item prefix sums
// (one item per (check, block) pair).  Returns hipSuccess or hipErrorInvalidValue.
inline hipError_t validate(const PckCheckBatch& batch) {
  if (batch.count < 1 || batch.count > PCK_MAX_BATCH || batch.start[0] != 0)
    return hipErrorInvalidValue;
  for (int g = 0; g < batch.count; ++g) {
    const PckCheckDesc& d = batch.desc[g];
    if (d.num_blocks < 1 || d.checks < 1 || d.block < 1 || d.n < 1 || !d.c || !d.a || !d.r ||
        !d.x || !d.y || !d.passed || !d.rho || !d.tau ||
        batch.start[g + 1] - batch.start[g] != static_cast<int64_t>(d.checks) * d.num_blocks)
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace check
}  // namespace pck
