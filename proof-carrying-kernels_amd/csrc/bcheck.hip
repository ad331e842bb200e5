// Blocked checker for a batch of activation rows: every column b of Y = X W^T is checked the way
// the single-vector checker checks y = W x (check_pair.h), with the same bank and constants:
//   rho[k, beta, b] = c[k, beta] . X[b] - r[k, beta] . Y[b, beta rows]
//   s               = a[beta] . |X[b]|, bounded above and rounded up to FP32
//   tau             = coef s + geps ((1 + u32) s + sum |Y[b, beta rows]|) + tau_floor, every
//                     operation rounded up
// and (k, beta, b) passes only if every Y in the block's rows of column b is finite, tau is
// finite and |rho| <= tau.  The reference checks one GEMV output per descriptor
// (src/pck/cuda/csrc/checker_kernel.cu:87-196); its batched use at B > 1 is one check per
// column, which is what this kernel computes, reading the bank once for all B columns.
//
// Arithmetic (bounds as in check_pair.h):
//   c.x: c_j x_j has 24 + 8 significand bits, exact in FP64; each is added with one fma, so
//        the error of rho stays within the gamma_H(u64) term of the host's geps.
//   s:   a_j |x_j| (8 + 8 bits) is exact in FP64 and never below 2^-266, so a round-to-nearest
//        FP64 sum s^ of n <= 2^20 of them (any order) has s <= s^ (1 + 2^-32); the kernel
//        raises s^ by 2^-31 (the product's own rounding included) and rounds up to FP32.
//   sum |y|: error-free round-up additions, as in check_pair.h.
//
// Work item: 4 (check, block) pairs x 16 batch columns, one 256-lane workgroup.  The bank rows
// and X columns pass through LDS as FP64 in chunks of 64 columns (two buffers); wave w adds
// columns 16w .. 16w + 15 of each chunk for all 64 outputs; the four wave sums meet in LDS in a
// fixed order, so the result does not depend on scheduling.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "check_pair.h"
#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace {

constexpr int kThreads = 256;
constexpr int kPairs = 4;    // (check, block) pairs per work item
constexpr int kCols = 16;    // batch columns per work item
constexpr int kChunk = 64;   // bank columns per LDS chunk
constexpr double kSumSlack = 1.0 + 0x1p-31;

struct BatchCheckSet {
  PckBatchCheckDesc desc[PCK_MAX_BATCH];
  int64_t start[PCK_MAX_BATCH + 1];  // work-item prefix sums
  int64_t pair_tiles[PCK_MAX_BATCH];
  int count;
};

struct Staged {
  float c;
  uint32_t a;   // BF16 bits
  uint2 x;      // four BF16
};

__device__ __forceinline__ double bf16_bits(uint32_t h) { return __uint_as_float(h << 16); }

__global__ void __launch_bounds__(kThreads) batch_check_kernel(const BatchCheckSet set) {
  __shared__ double cs[2][kPairs][kChunk];
  __shared__ double as[2][kPairs][kChunk];
  __shared__ double xs[2][kChunk][kCols];
  __shared__ double red[4][4][kPairs * kCols];  // [wave][quantity][output]

  const int64_t item = blockIdx.x;
  int g = 0;
  while (g + 1 < set.count && item >= set.start[g + 1]) ++g;
  const PckBatchCheckDesc& d = set.desc[g];
  const int64_t local = item - set.start[g];
  const int64_t pair0 = (local % set.pair_tiles[g]) * kPairs;
  const int64_t col0 = (local / set.pair_tiles[g]) * kCols;
  const int64_t pairs = d.checks * d.num_blocks;
  const int64_t n = d.n;
  const int64_t m = d.num_blocks * d.block;

  const int t = static_cast<int>(threadIdx.x);
  const int wave = t / 64;
  const int o = t % 64;  // output of this lane: pair p, column b
  const int p = o / kCols;
  const int b = o % kCols;

  // Staging roles: lane t loads bank element (t / 64, t % 64) of the chunk and X columns
  // 4 (t % 16) .. + 3 of batch row t / 16.
  const int sp = t / kChunk, sj = t % kChunk;
  const int xr = t / 16, xj = (t % 16) * 4;
  const int64_t s_pair = pair0 + sp;
  const bool s_pair_ok = s_pair < pairs;
  const float* c_row = d.c + (s_pair_ok ? s_pair : 0) * n;
  const uint16_t* a_row =
      static_cast<const uint16_t*>(d.a) + (s_pair_ok ? s_pair % d.num_blocks : 0) * n;
  const int64_t x_col = col0 + xr;
  const bool x_ok = x_col < d.batch;
  const uint16_t* x_row = static_cast<const uint16_t*>(d.X) + (x_ok ? x_col : 0) * n;
  const bool x_vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(d.X) & 7) == 0;

  auto fetch = [&](int64_t j0) {
    Staged v{0.f, 0u, make_uint2(0u, 0u)};
    const int64_t j = j0 + sj;
    if (s_pair_ok && j < n) {
      v.c = c_row[j];
      v.a = a_row[j];
    }
    if (x_ok) {
      const int64_t jx = j0 + xj;
      if (x_vec && jx + 3 < n) {
        v.x = *reinterpret_cast<const uint2*>(x_row + jx);
      } else {
        uint32_t e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) e[k] = jx + k < n ? x_row[jx + k] : 0u;
        v.x = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
      }
    }
    return v;
  };
  auto stage = [&](int buf, const Staged& v) {
    cs[buf][sp][sj] = static_cast<double>(v.c);
    as[buf][sp][sj] = bf16_bits(v.a);
    xs[buf][xj + 0][xr] = bf16_bits(v.x.x & 0xFFFFu);
    xs[buf][xj + 1][xr] = bf16_bits(v.x.x >> 16);
    xs[buf][xj + 2][xr] = bf16_bits(v.x.y & 0xFFFFu);
    xs[buf][xj + 3][xr] = bf16_bits(v.x.y >> 16);
  };

  double cx = 0.0, s = 0.0;
  const int64_t chunks = (n + kChunk - 1) / kChunk;
  stage(0, fetch(0));
  __syncthreads();
  for (int64_t ch = 0; ch < chunks; ++ch) {
    const int buf = static_cast<int>(ch & 1);
    const bool more = ch + 1 < chunks;
    Staged next{};
    if (more) next = fetch((ch + 1) * kChunk);  // in flight while this chunk is added
#pragma unroll
    for (int jj = 16 * wave; jj < 16 * wave + 16; ++jj) {
      const double x = xs[buf][jj][b];
      cx = __builtin_fma(cs[buf][p][jj], x, cx);
      s = __builtin_fma(as[buf][p][jj], __builtin_fabs(x), s);
    }
    if (more) stage(buf ^ 1, next);
    __syncthreads();
  }

  // The block's outputs of this column: r . y (round to nearest) and sum |y| (round up); the
  // four waves take rows w, w + 4, ...
  const int64_t pair = pair0 + p;
  const int64_t col = col0 + b;
  double ry = 0.0, yabs = 0.0;
  if (pair < pairs && col < d.batch) {
    const int64_t beta = pair % d.num_blocks;
    const int8_t* r_row = d.r + pair * d.block;
    const float* y_blk = d.Y + col * m + beta * d.block;
    for (int64_t i = wave; i < d.block; i += 4) {
      const double yd = static_cast<double>(y_blk[i]);
      ry = ry + (r_row[i] > 0 ? yd : -yd);
      yabs = add_up_nonneg(yabs, __builtin_fabs(yd));
    }
  }
  red[wave][0][o] = cx;
  red[wave][1][o] = s;
  red[wave][2][o] = ry;
  red[wave][3][o] = yabs;
  __syncthreads();
  if (wave != 0 || pair >= pairs || col >= d.batch) return;
  const double cx_t = (red[0][0][o] + red[1][0][o]) + (red[2][0][o] + red[3][0][o]);
  const double s_t = (red[0][1][o] + red[1][1][o]) + (red[2][1][o] + red[3][1][o]);
  const double ry_t = (red[0][2][o] + red[1][2][o]) + (red[2][2][o] + red[3][2][o]);
  const double yabs_t = add_up_nonneg(add_up_nonneg(red[0][3][o], red[1][3][o]),
                                      add_up_nonneg(red[2][3][o], red[3][3][o]));
  const double s_up = check::round_up_to_f32(mul_up(s_t, kSumSlack));
  const double rho = cx_t - ry_t;
  const double cabs_up = mul_up(check::kOnePlusU32, s_up);
  const double eps = mul_up(d.geps, add_up(cabs_up, yabs_t));
  const double tau = add_up(add_up(mul_up(d.coef, s_up), eps), d.tau_floor);
  const int64_t at = pair * d.batch + col;
  d.passed[at] =
      __builtin_isfinite(yabs_t) && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
  d.rho[at] = rho;
  d.tau[at] = tau;
}

}  // namespace
}  // namespace pck

extern "C" int pck_batch_check(const PckBatchCheckDesc* descs, int count, void* stream) {
  using namespace pck;
  if (count < 1 || count > PCK_MAX_BATCH || descs == nullptr) return hipErrorInvalidValue;
  BatchCheckSet set{};
  set.count = count;
  for (int g = 0; g < count; ++g) {
    const PckBatchCheckDesc& d = descs[g];
    if (d.num_blocks < 1 || d.checks < 1 || d.block < 1 || d.n < 1 || d.batch < 1 || !d.c ||
        !d.a || !d.r || !d.X || !d.Y || !d.passed || !d.rho || !d.tau || d.n > (1 << 20))
      return hipErrorInvalidValue;
    set.desc[g] = d;
    set.pair_tiles[g] = (d.checks * d.num_blocks + kPairs - 1) / kPairs;
    const int64_t col_tiles = (d.batch + kCols - 1) / kCols;
    set.start[g + 1] = set.start[g] + set.pair_tiles[g] * col_tiles;
  }
  const int64_t items = set.start[count];
  if (items > 0x7FFFFFFF / kThreads) return hipErrorInvalidValue;
  batch_check_kernel<<<dim3(static_cast<unsigned>(items)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream)>>>(set);
  return hipGetLastError();
}
