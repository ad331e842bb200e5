// Trusted blocked checksum checker for y = W x on gfx950.
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
// Arithmetic on gfx950.  FP64 runs at the FP32 rate on MI355X, so rho is evaluated entirely in
// FP64: each c_j x_j (24 + 8 significand bits) and each a_j |x_j| (8 + 8) is exact in FP64, and
// every addition is one FP64 operation.  rho's rounding error is therefore at most
// gamma_H(u64) (sum |c_j x_j| + sum |y_i|) for the depth H <= n + b + 1 of its evaluation,
// which the host's geps >= gamma_H(u64) + ... already covers (the reference's per-thread FP32
// Dot2 error term is not needed, only bounded from above).  s and tau use the error-free
// round-up operations of rounding.h.
//
// Parallelism: the n columns of each (check, block) pair are split into `segments` workgroups
// so the grid fills the 256 CUs.  Each workgroup publishes its partial c.x and s, then takes a
// ticket on the pair's counter; the last one merges the partials in segment order (a fixed
// order, so results do not depend on scheduling), evaluates the y terms and the verdict, and
// resets the counter.  MI355X has one L2 per XCD, so publication uses an agent-scope
// acquire-release atomic (the compiler emits the L2 write-back and invalidate it needs), not a
// bare fence.  One launch checks up to PCK_MAX_BATCH outputs.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr double kOnePlusU32 = 1.0 + 0x1p-24;  // exact in FP64

__device__ __forceinline__ float bf16_to_float(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

template <bool kUp>
__device__ __forceinline__ double combine(double a, double b) {
  return kUp ? add_up(a, b) : a + b;
}

// Sum over the workgroup; every thread returns the same value.  A wave64 xor butterfly
// (symmetric in its operands, so all lanes agree), then the four wave sums in fixed order.
template <bool kUp>
__device__ double group_sum(double v, double* lds) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) v = combine<kUp>(v, __shfl_xor(v, off, kWave));
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
  __syncthreads();
  const double total = combine<kUp>(combine<kUp>(lds[0], lds[2]), combine<kUp>(lds[1], lds[3]));
  __syncthreads();
  return total;
}

__global__ void __launch_bounds__(kThreads) blocked_check_kernel(const PckCheckBatch batch) {
  __shared__ double lds[kWaves];
  __shared__ int last;

  const int64_t item = blockIdx.x;
  int g = 0;
  while (g + 1 < batch.count && item >= batch.start[g + 1]) ++g;
  const PckCheckDesc& d = batch.desc[g];
  const int64_t local = item - batch.start[g];
  const int64_t pair = local / d.segments;  // k * num_blocks + beta
  const int64_t seg = local % d.segments;
  const int64_t beta = pair % d.num_blocks;
  const int64_t n = d.n;
  const int t = static_cast<int>(threadIdx.x);
  const float* c_row = d.c + pair * n;
  const uint16_t* a_row = static_cast<const uint16_t*>(d.a) + beta * n;
  const uint16_t* x = static_cast<const uint16_t*>(d.x);

  // Phase 1 (every segment): partial c . x (FP64, exact products) and a . |x| (rounded up).
  const int64_t j_end = min(n, (seg + 1) * d.seg_len);
  double cx = 0.0;
  double s = 0.0;
  for (int64_t j = seg * d.seg_len + t; j < j_end; j += kThreads) {
    const double xj = static_cast<double>(bf16_to_float(x[j]));
    const double cj = static_cast<double>(c_row[j]);
    cx = __builtin_fma(cj, xj, cx);  // the product is exact: one rounding, the add's
    const double aj = static_cast<double>(bf16_to_float(a_row[j]));
    s = add_up(s, aj * __builtin_fabs(xj));  // exact product, sum rounded up
  }
  cx = group_sum<false>(cx, lds);
  s = group_sum<true>(s, lds);
  if (t == 0) {
    d.partial_cx[pair * d.segments + seg] = cx;
    d.partial_s[pair * d.segments + seg] = s;
    const unsigned ticket = __hip_atomic_fetch_add(&d.counters[pair], 1u, __ATOMIC_ACQ_REL,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    last = ticket == static_cast<unsigned>(d.segments) - 1;
  }
  __syncthreads();
  if (!last) return;

  // Phase 2 (the last segment to finish): the y terms, the merge and the verdict.
  const int8_t* r_row = d.r + pair * d.block;
  const float* y_blk = d.y + beta * d.block;
  double ry = 0.0;
  double yabs = 0.0;
  int bad = 0;
  for (int i = t; i < d.block; i += kThreads) {
    const float yi = y_blk[i];
    bad |= !__builtin_isfinite(yi);
    const double yd = static_cast<double>(yi);
    ry = ry + (r_row[i] > 0 ? yd : -yd);
    yabs = add_up(yabs, __builtin_fabs(yd));
  }
  const int nonfinite = __syncthreads_or(bad);
  ry = group_sum<false>(ry, lds);
  yabs = group_sum<true>(yabs, lds);

  if (t == 0) {
    const double* pcx = d.partial_cx + pair * d.segments;
    const double* ps = d.partial_s + pair * d.segments;
    double cx_total = 0.0;
    double s_total = 0.0;
    for (int i = 0; i < d.segments; ++i) {  // fixed order: a deterministic result
      cx_total = cx_total + pcx[i];
      s_total = add_up(s_total, ps[i]);
    }
    __hip_atomic_store(&d.counters[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    const double rho = cx_total - ry;
    const double cabs_up = mul_up(kOnePlusU32, s_total);
    const double eps = mul_up(d.geps, add_up(cabs_up, yabs));
    const double tau = add_up(add_up(mul_up(d.coef, s_total), eps), d.tau_floor);
    // An overflowing threshold (tau = inf) fails closed; NaN compares false.
    d.passed[pair] = nonfinite == 0 && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
    d.rho[pair] = rho;
    d.tau[pair] = tau;
  }
}

}  // namespace
}  // namespace pck

extern "C" int pck_blocked_check(const PckCheckBatch* batch, void* stream) {
  if (batch == nullptr || batch->count < 1 || batch->count > PCK_MAX_BATCH)
    return hipErrorInvalidValue;
  for (int g = 0; g < batch->count; ++g) {
    const PckCheckDesc& d = batch->desc[g];
    if (d.segments < 1 || d.num_blocks < 1 || d.checks < 1 || d.block < 1 || d.n < 1 ||
        d.seg_len < 1 || d.seg_len * d.segments < d.n ||
        batch->start[g + 1] - batch->start[g] !=
            static_cast<int64_t>(d.checks) * d.num_blocks * d.segments)
      return hipErrorInvalidValue;
  }
  const int64_t items = batch->start[batch->count];
  if (batch->start[0] != 0 || items < 1 || items * pck::kThreads > 0xFFFFFFFFll)
    return hipErrorInvalidValue;  // the dispatch size is 32-bit in work-items
  pck::blocked_check_kernel<<<dim3(static_cast<unsigned>(items)), dim3(pck::kThreads), 0,
                              static_cast<hipStream_t>(stream)>>>(*batch);
  return hipGetLastError();
}
