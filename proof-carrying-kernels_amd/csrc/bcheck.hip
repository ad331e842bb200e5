// Blocked checker for a batch of activation rows: every column b of Y = X W^T is checked the way
// the single-vector checker checks y = W x (check_pair.h), with the same bank and constants:
//   rho[k, beta, b] = c[k, beta] . X[b] - r[k, beta] . Y[b, beta rows]
//   s               = a[beta] . |X[b]|, bounded above and rounded up to FP32
//   tau             = coef s + geps ((1 + u32) s + sum |Y[b, beta rows]|) + tau_floor, every
//                     operation rounded up
// and (k, beta, b) passes only if every Y in the block's rows of column b is finite, tau is
// finite and |rho| <= tau.  The reference checks one GEMV output per descriptor
// (src/pck/cuda/csrc/checker_kernel.cu:87-196); its batched use at B > 1 is one check per
// column, which is what this computes, reading the bank once per 32 columns.
//
// Arithmetic.
//   c.x: on the FP64 matrix cores (v_mfma_f64_16x16x4_f64; measured on MI355X with the probe
//        library: each output is four IEEE FMAs in K order, each rounded once to nearest even,
//        continued through the accumulator).  c_j x_j has 24 + 8 significand bits, exact in
//        FP64, so every FMA is one rounded addition and the error of rho stays within the
//        gamma_H(u64) term of the host's geps: a product passes through at most seg_len / 4
//        additions in its wave's K quarter, 2 for the workgroup's quarters, one per later
//        segment of its subset and 2 for the subsets, and the subtraction of r . y (itself at
//        most block / 16 + 4 deep), below H >= n + b + 1.
//   s:   on the BF16 matrix cores (v_mfma_f32_16x16x32_bf16, zero accumulator: one step adds 32
//        exact products a_j |x_j| into an FP32 result) with every step result added in FP64.  A
//        step's result is below the exact sum of its non-negative products by at most 2^-18
//        (32 products truncated below 2^-23 of the largest) plus one FP32 rounding (2^-24),
//        relative, and by at most 33 x 2^-126 absolute when products or the result fall below
//        the FP32 normal range; the FP64 additions are far below either.  Operands are raised to
//        at least 2^-126 first (a zero or subnormal a_j or |x_j| becomes 2^-126, which only
//        raises s), so no subnormal input reaches the matrix core.  The finish raises s by
//        n 2^-124 and then by the factor 1 + 2^-16, rounding up, and rounds up to FP32: tau is
//        never below its exact value and at most (1 + 2^-15) above it when no a_j or x_j is
//        below 2^-100.  (The reference's s adds FP32 round-up partial sums of about n / 256
//        terms each, within a few 2^-20 relative of exact.)
//   sum |y|: a round-to-nearest FP64 sum of the |y| (FP32, exact in FP64) at most b / 16 + 4
//        additions deep, raised by the factor 1 + (b + 4) 2^-52 with upward rounding: at least
//        the exact sum, since each addition loses at most 2^-53 of the non-negative partial sum.
//
// Two launches.  Partial: a workgroup owns 32 (check, block) pairs x 32 batch columns x one K
// segment; its four waves take the segment's K quarters and each computes the whole 32 x 32
// tile (2 x 2 matrix-core tiles) from operands loaded straight into registers: per 32 columns
// lane l reads 32 contiguous bytes of bank row l % 16 of each row tile (c) and 16 of a and of X
// row l % 16 of each column tile, the K order inside each group of 32 chosen so; the next kRing
// groups are in flight per lane.  The quarters meet in LDS in a fixed order and the segment's
// (c.x, a.|x|) tile goes to the workspace as whole rows of 32 columns.  Finish: a workgroup per
// (block, 64 batch columns): rows of 16 lanes read the block's outputs (r . y per check, rounded
// to nearest, and sum |y|, rounded up) with a fixed DPP butterfly per column, the partials are
// added in a fixed order with loads across 64 columns, and one lane per column forms rho, tau
// and the verdict.  Nothing depends on scheduling.

#include <hip/hip_runtime.h>

#include <atomic>

#include <climits>
#include <cstdint>
#include <utility>

#include "check_pair.h"
#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;            // K quarters of a workgroup's segment
constexpr int kTile = 16;            // matrix-core tile (rows and columns)
constexpr int kPairsWG = 2 * kTile;  // pairs per workgroup tile
constexpr int kColsWG = 2 * kTile;   // batch columns per workgroup tile
constexpr int kStep = 32;            // K columns per step: 8 FP64 + 1 BF16 MFMA per tile
constexpr int kRing = 2;             // steps of loads in flight per lane
constexpr int kTargetGroups = 256;   // one workgroup per CU on MI355X
constexpr int kFinishLanes = 16;    // finish: lanes per block's outputs (a DPP row)
constexpr int kFinishCols = 64;     // finish: batch columns per workgroup
constexpr double kSumSlack = 1.0 + 0x1p-16;
constexpr double kSubnormalSlack = 0x1p-124;  // per column of the reduction

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// What a partial workgroup needs of its descriptor, in 64 bytes that load together (every
// count fits in 32 bits: the plan bounds pairs x n x 4 and batch x n x 2 below 2^31).
struct PartialDesc {
  const float* c;
  const void* a;
  const void* X;
  int64_t slot;        // the descriptor's first workspace entry
  int32_t start;       // its first partial workgroup
  int32_t segments;    // K segments
  int32_t pair_tiles;  // tiles of kPairsWG pairs
  int32_t pairs;       // checks x num_blocks
  int32_t num_blocks;
  int32_t n;
  int32_t batch;
  int32_t unused;
};
static_assert(sizeof(PartialDesc) == 64, "one 64-byte record per descriptor");

// What a finish workgroup needs of its descriptor for its loads, in 64 bytes.
struct FinishDesc {
  const float* Y;
  const int8_t* r;
  int64_t slot;     // the descriptor's first workspace entry
  int64_t outs;     // checks x num_blocks x batch: the stride of one segment's partials
  int32_t start;    // its first finish workgroup
  int32_t num_blocks;
  int32_t block;
  int32_t checks;
  int32_t batch;
  int32_t segments;
  int32_t n;
  int32_t unused;
};
static_assert(sizeof(FinishDesc) == 64, "one 64-byte record per descriptor");

struct Plan {
  PartialDesc part[PCK_MAX_BATCH];
  FinishDesc fin[PCK_MAX_BATCH];
  // The descriptor searches' bounds in 32 bits (one load each; the launch checks both grids
  // are below 2^31): the first partial and finish workgroup of descriptors 1 .. count - 1,
  // INT32_MAX past the count.
  int32_t part_first[PCK_MAX_BATCH];
  int32_t fin_first[PCK_MAX_BATCH];
  PckBatchCheckDesc desc[PCK_MAX_BATCH];
  int64_t start[PCK_MAX_BATCH + 1];   // partial workgroups, prefix sums
  int64_t finish[PCK_MAX_BATCH + 1];  // finish workgroups (blocks x column groups), prefix
  int64_t slots[PCK_MAX_BATCH + 1];   // partial entries (segments x outputs), prefix sums
  int64_t pair_tiles[PCK_MAX_BATCH];
  int64_t segments[PCK_MAX_BATCH];
  int64_t seg_len;
  int count;
  double* part_cx;  // (slots): c.x of one segment, at seg * pairs * batch + pair * batch + col
  double* part_s;   // (slots): a.|x| of one segment, same index
};

// One lane's operands for one step: eight consecutive columns of bank rows (c and a) of both
// row tiles and of batch rows (X) of both column tiles.
struct Staged {
  u32x4 c[2][2];  // [row tile][half]: eight FP32
  u32x4 a[2];     // [row tile]: eight BF16
  u32x4 x[2];     // [column tile]: eight BF16
};

__device__ __forceinline__ u32x4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ double bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ double bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// max(|v|, 2^-126) for eight packed BF16 values (0x0080 is 2^-126).
__device__ __forceinline__ bf16x8 abs_floor8(u32x4 v) {
  u32x4 a = v & 0x7FFF7FFFu;
  // the AND stays one 32-bit instruction per pair (without the empty asm the compiler splits
  // it per 16-bit value and repacks)
  __asm__("" : "+v"(a));
  const u16x8 f = __builtin_elementwise_max(__builtin_bit_cast(u16x8, a), (u16x8)(0x80));
  return __builtin_bit_cast(bf16x8, f);
}

__global__ void __launch_bounds__(kThreads) partial_kernel(const Plan plan) {
  __shared__ double red[2][kWaves][kPairsWG][kColsWG + 1];  // [c.x, a.|x|][quarter][pair][col]

  const int item = static_cast<int>(blockIdx.x);  // the launch checks the grid is < 2^31
  // The descriptor: every bound compared at once (not a chain of dependent loads), then its
  // whole record.  Every value below is needed before the first operand load; empty asm
  // statements that read them make the compiler request them together, the plan's own fields
  // with the bounds and then the record: two round trips instead of one per use.
  double* const part_cx = plan.part_cx;
  double* const part_s = plan.part_s;
  const int seg_len = static_cast<int>(plan.seg_len);  // at most n rounded up to the quantum
  int g = 0;
#pragma unroll
  for (int i = 1; i < PCK_MAX_BATCH; ++i) g += item >= plan.part_first[i] ? 1 : 0;
  __asm__ volatile("" ::"s"(part_cx), "s"(part_s), "s"(seg_len));
  const PartialDesc p = plan.part[g];
  __asm__ volatile("" ::"s"(p.c), "s"(p.a), "s"(p.X), "s"(p.slot), "s"(p.start), "s"(p.segments),
                   "s"(p.pair_tiles), "s"(p.pairs), "s"(p.num_blocks), "s"(p.n), "s"(p.batch));
  const int local = item - p.start;
  const int seg = local % p.segments;
  const int tile = local / p.segments;
  const int pair0 = (tile % p.pair_tiles) * kPairsWG;
  const int col0 = (tile / p.pair_tiles) * kColsWG;
  const int pairs = p.pairs;
  const int n = p.n;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / 64);
  const int quarter = seg_len / kWaves;
  const int j_seg_hi = (seg + 1) * seg_len < n ? (seg + 1) * seg_len : n;
  const int j_lo = seg * seg_len + wave * quarter;
  const int j_hi = j_lo + quarter < j_seg_hi ? j_lo + quarter : j_seg_hi;
  const int steps = j_hi > j_lo ? (j_hi - j_lo + kStep - 1) / kStep : 0;

  // Lane l = 16 q + i supplies row i of the A tiles (bank rows) and column i of the B tiles
  // (batch rows) at the step's columns 8 q .. 8 q + 7: FP64 step e takes column 8 q + e as its
  // K slot q, the BF16 step takes all eight as its K slots of lane group q.  Raw buffer loads,
  // issued unconditionally (so the loads in flight are counted exactly): rows and columns past
  // the operands or past the quarter point past the buffer and read zero (n % 8 == 0 and every
  // bound is a multiple of 8: a lane's eight columns are all in or all out).
  const int lane = static_cast<int>(threadIdx.x) % 64;
  const int li = lane % 16, lq = lane / 16;
  const __amdgpu_buffer_rsrc_t rc = check::make_rsrc(p.c, static_cast<uint32_t>(pairs * n * 4));
  const __amdgpu_buffer_rsrc_t ra =
      check::make_rsrc(p.a, static_cast<uint32_t>(p.num_blocks * n * 2));
  const __amdgpu_buffer_rsrc_t rx = check::make_rsrc(p.X, static_cast<uint32_t>(p.batch * n * 2));
  const int j_lane = j_lo + 8 * lq;
  uint32_t c_voff[2], a_voff[2], x_voff[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int pair = pair0 + kTile * t + li;
    const int col = col0 + kTile * t + li;
    // unsigned: a lane past n (a wave with no steps) stays below 2^32
    const uint32_t jl = static_cast<uint32_t>(j_lane), un = static_cast<uint32_t>(n);
    c_voff[t] = pair < pairs ? (static_cast<uint32_t>(pair) * un + jl) * 4u : check::kOutOfRange;
    a_voff[t] = pair < pairs ? (static_cast<uint32_t>(pair % p.num_blocks) * un + jl) * 2u
                             : check::kOutOfRange;
    x_voff[t] = col < p.batch ? (static_cast<uint32_t>(col) * un + jl) * 2u : check::kOutOfRange;
  }

  auto fetch = [&](int step) {
    const int st = step < steps ? step : (steps > 0 ? steps - 1 : 0);  // past the end: unused
    const uint32_t at = static_cast<uint32_t>(st) * kStep;
    // A lane past the quarter's end sets the offset's top bit, which puts every load past its
    // buffer (below 2^31 bytes), so it reads zero.  The bit is opaque to the compiler (an empty
    // asm), so the loads stay unconditional: a select between two offsets compiles into
    // branches, with each load behind a wait for every load in flight.
    uint32_t out = j_lane + st * kStep < j_hi ? 0u : check::kOutOfRange;
    __asm__("" : "+v"(out));
    Staged v;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v.c[t][0] = load_b128(rc, (c_voff[t] + at * 4) | out);
      v.c[t][1] = load_b128(rc, (c_voff[t] + at * 4 + 16) | out);
      v.a[t] = load_b128(ra, (a_voff[t] + at * 2) | out);
      v.x[t] = load_b128(rx, (x_voff[t] + at * 2) | out);
    }
    return v;
  };

  // cx[t][u] register r: pair 16 t + 4 r + lq, column 16 u + li (FP64 16 x 16 D layout);
  // s[t][u][r]: pair 16 t + 4 lq + r, column 16 u + li (FP32 16 x 16 D layout).
  f64x4 cx[2][2];
  double s[2][2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      cx[t][u] = (f64x4){0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int r = 0; r < 4; ++r) s[t][u][r] = 0.0;
    }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  auto consume = [&](const Staged& v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      double xe[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
        xe[u] = (e & 1) ? bf16_hi(v.x[u][e / 2]) : bf16_lo(v.x[u][e / 2]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const double ce = static_cast<double>(__uint_as_float(v.c[t][e / 4][e % 4]));
#pragma unroll
        for (int u = 0; u < 2; ++u)
          cx[t][u] = __builtin_amdgcn_mfma_f64_16x16x4f64(ce, xe[u], cx[t][u], 0, 0, 0);
      }
    }
    bf16x8 af[2], xf[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) af[t] = abs_floor8(v.a[t]);
#pragma unroll
    for (int u = 0; u < 2; ++u) xf[u] = abs_floor8(v.x[u]);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], xf[u], zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[t][u][r] = s[t][u][r] + static_cast<double>(p[r]);
      }
  };

  // Step q is consumed from ring slot q % kRing, which is then refilled with step q + kRing.
  // Whole ring passes have no exit inside, so the loads in flight are the same on every entry
  // to the loop head.  A scheduling barrier after each refill keeps its loads ahead of the next
  // slot's products (the scheduler otherwise sinks them to the end of the pass, leaving no
  // load in flight while the last slot is consumed).
  Staged ring[kRing];
#pragma unroll
  for (int k = 0; k < kRing; ++k) ring[k] = fetch(k);
  const int full = steps / kRing * kRing;
  for (int base = 0; base < full; base += kRing) {
    [&]<int... K>(std::integer_sequence<int, K...>) {
      ((consume(ring[K]), ring[K] = fetch(base + K + kRing), __builtin_amdgcn_sched_barrier(0)),
       ...);
    }(std::make_integer_sequence<int, kRing>{});
  }
  [&]<int... K>(std::integer_sequence<int, K...>) {
    ((full + K < steps ? (consume(ring[K]), 0) : 0), ...);
  }(std::make_integer_sequence<int, kRing>{});

  // The quarters meet in LDS: ((q0 + q1) + (q2 + q3)) per output, then whole rows of 32
  // columns go to the workspace.
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[0][wave][kTile * t + 4 * r + lq][kTile * u + li] = cx[t][u][r];
        red[1][wave][kTile * t + 4 * lq + r][kTile * u + li] = s[t][u][r];
      }
  __syncthreads();
  const int64_t outs = static_cast<int64_t>(pairs) * p.batch;
  double* dst_cx = part_cx + p.slot + seg * outs;
  double* dst_s = part_s + p.slot + seg * outs;
  const int t = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < kPairsWG * kColsWG / kThreads; ++i) {
    const int o = t + kThreads * i;
    const int pr = o / kColsWG, cl = o % kColsWG;
    const int pair = pair0 + pr, col = col0 + cl;
    if (pair < pairs && col < p.batch) {
      const int64_t at = static_cast<int64_t>(pair) * p.batch + col;
      dst_cx[at] =
          (red[0][0][pr][cl] + red[0][1][pr][cl]) + (red[0][2][pr][cl] + red[0][3][pr][cl]);
      dst_s[at] =
          (red[1][0][pr][cl] + red[1][1][pr][cl]) + (red[1][2][pr][cl] + red[1][3][pr][cl]);
    }
  }
}

// A double moved across lanes by a DPP pattern within rows of 16 lanes.
template <int kCtrl>
__device__ __forceinline__ double dpp_double(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b & 0xFFFFFFFFu), kCtrl, 0xF, 0xF,
                                             false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), kCtrl, 0xF, 0xF, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}

// Sum over a row of 16 lanes, the same bits on every lane: the partner at each level holds the
// sum of the other half of the current group (quad_perm 1032, quad_perm 2301, half mirror,
// mirror), and a + b = b + a.
__device__ __forceinline__ double row_sum(double v) {
  v = v + dpp_double<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = v + dpp_double<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = v + dpp_double<0x141>(v);  // row_half_mirror: the other quad of the 8
  return v + dpp_double<0x140>(v);  // row_mirror: the other 8 of the 16
}

// A workgroup per (block beta, 64 batch columns).
//   Outputs: row r = t / 16 of 16 lanes takes columns r, r + 16, r + 32, r + 48; lane q reads
//   the float4 groups q, q + 16, ... (rows 64 i + 4 q .. + 3) of the block in each of them, all
//   loads of a pass in flight (the block's signs once for the four columns); DPP row sums.
//   Partials: lane t takes column t % 64 and segments t / 64, t / 64 + 4, ... in order (one load
//   instruction reads 64 consecutive columns of one segment), four of them in flight per pass
//   (a layer's plan gives a subset 1-4 segments; more in flight would re-read the last one);
//   the four subsets meet in LDS as (p0 + p1) + (p2 + p3).
//   Lanes 0 .. 63 then form rho, tau and the verdict of one column each; every operand of tau is
//   non-negative (the plan checks the constants), so the branch-free round-up operations apply.
__global__ void __launch_bounds__(kThreads) finish_kernel(const Plan plan) {
  constexpr int kRowCols = kFinishCols / kFinishLanes;  // columns per row of 16 lanes
  constexpr int kSubsets = kThreads / kFinishCols;      // segment subsets
  constexpr int kPass = 2;                              // float4 groups per lane per pass
  __shared__ double red_ry[kFinishCols], red_yabs[kFinishCols];
  __shared__ double red_cx[kSubsets][kFinishCols], red_s[kSubsets][kFinishCols];

  const int item = static_cast<int>(blockIdx.x);  // the launch checks the grid is < 2^31
  // The plan's fields with the search bounds, then the record: two round trips (see the
  // partial kernel).
  const double* const part_cx = plan.part_cx;
  const double* const part_s = plan.part_s;
  int g = 0;
#pragma unroll
  for (int i = 1; i < PCK_MAX_BATCH; ++i) g += item >= plan.fin_first[i] ? 1 : 0;
  __asm__ volatile("" ::"s"(part_cx), "s"(part_s));
  const FinishDesc f = plan.fin[g];
  __asm__ volatile("" ::"s"(f.Y), "s"(f.r), "s"(f.slot), "s"(f.outs), "s"(f.start),
                   "s"(f.num_blocks), "s"(f.block), "s"(f.checks), "s"(f.batch), "s"(f.segments));
  const int local = item - f.start;
  const int nb = f.num_blocks;
  const int beta = local % nb;
  const int col0 = (local / nb) * kFinishCols;
  const int t = static_cast<int>(threadIdx.x);
  const int row = t / kFinishLanes, q = t % kFinishLanes;
  const int64_t m = static_cast<int64_t>(nb) * f.block;
  const int groups = f.block / 4;  // block % 4 == 0
  const int segments = f.segments;
  const int cols = f.batch - col0 < kFinishCols ? f.batch - col0 : kFinishCols;  // >= 1
  // Every load below is an unconditional raw buffer load at a valid address: a uniform base
  // and a 32-bit lane offset (the plan bounds every range below 2^31 bytes).  A column past
  // the batch reads the last column, a group or segment past the end reads the last one, and
  // data that is not needed is dropped where it is used, by a select on the value: a
  // conditional load would be followed by a wait for it before the next one could be issued.
  // The sums of columns past the batch are computed and never read.
  //   Outputs: from the workgroup's first column of the block; column j of row r at
  //   (min(r + 16 j, cols - 1) m) x 4 bytes.
  const __amdgpu_buffer_rsrc_t y_rsrc = check::make_rsrc(
      f.Y + static_cast<int64_t>(col0) * m + static_cast<int64_t>(beta) * f.block,
      static_cast<uint32_t>(((cols - 1) * m + f.block) * 4));
  uint32_t y_off[kRowCols];
#pragma unroll
  for (int j = 0; j < kRowCols; ++j) {
    const int c = row + kFinishLanes * j < cols ? row + kFinishLanes * j : cols - 1;
    y_off[j] = static_cast<uint32_t>(c * m * 4);
  }

  // sum |y| to nearest, at most block / 16 + 4 additions deep, then raised by 1 + (b + 4) 2^-52
  // (the factor is exact in FP64)
  const double yabs_slack = 1.0 + static_cast<double>(f.block + 4) * 0x1p-52;
  double yabs[kRowCols] = {};
  const int pc = t % kFinishCols;  // partials: this lane's column
  const int sub = __builtin_amdgcn_readfirstlane(t / kFinishCols);  // and its segment subset
  const uint32_t p_off = static_cast<uint32_t>((pc < cols ? pc : cols - 1) * 8);
  const uint32_t seg_bytes = static_cast<uint32_t>(f.outs * 8);  // one segment's partials
  constexpr int kAhead = 4;
  int k = 0;
  do {  // checks >= 1 (the plan rejects fewer)
    const int64_t pair = static_cast<int64_t>(k) * nb + beta;
    const __amdgpu_buffer_rsrc_t r_rsrc =
        check::make_rsrc(f.r + pair * f.block, static_cast<uint32_t>(f.block));
    // One pass of outputs: float4 groups i0, i0 + 16 of the block in each of the row's columns,
    // and their signs.
    f32x4 v[kRowCols][kPass];
    uint32_t sg[kPass];
    auto load_pass = [&](int i0) {
#pragma unroll
      for (int e = 0; e < kPass; ++e) {
        const int i = i0 + kFinishLanes * e < groups ? i0 + kFinishLanes * e : groups - 1;
        sg[e] = __builtin_amdgcn_raw_buffer_load_b32(r_rsrc, i * 4, 0, 0);
#pragma unroll
        for (int j = 0; j < kRowCols; ++j)
          v[j][e] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(y_rsrc, y_off[j] + i * 16, 0, 0));
      }
    };
    double ry[kRowCols] = {};
    const bool first = k == 0;  // sum |y| once, over the first check's pass
    auto use_pass = [&](int i0) {
#pragma unroll
      for (int e = 0; e < kPass; ++e) {
        const bool in = i0 + kFinishLanes * e < groups;  // groups past the end add nothing
#pragma unroll
        for (int j = 0; j < kRowCols; ++j) {
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            // A skipped term adds +0.0, which leaves the sum unchanged: it starts at +0 and
            // never becomes -0 under round-to-nearest.
            const double yd = static_cast<double>(v[j][e][h]);
            const bool plus = static_cast<int8_t>((sg[e] >> (8 * h)) & 0xFFu) > 0;
            ry[j] = ry[j] + (in ? (plus ? yd : -yd) : 0.0);
            yabs[j] = yabs[j] + (in && first ? __builtin_fabs(yd) : 0.0);
          }
        }
      }
    };
    // The first pass of outputs is requested first, then this lane's first pass of partials
    // (column t % 64, segments t / 64, t / 64 + 4, ...): loads complete in the order they are
    // issued, so the outputs, used first, wait for nothing behind them.
    load_pass(q);
    const __amdgpu_buffer_rsrc_t cx_rsrc = check::make_rsrc(
        part_cx + f.slot + pair * f.batch + col0,
        static_cast<uint32_t>((segments - 1) * f.outs * 8 + cols * 8));
    const __amdgpu_buffer_rsrc_t s_rsrc = check::make_rsrc(
        part_s + f.slot + pair * f.batch + col0,
        static_cast<uint32_t>((segments - 1) * f.outs * 8 + cols * 8));
    auto load_partial = [&](const __amdgpu_buffer_rsrc_t& rs, int sgi) {
      return __builtin_bit_cast(
          double, __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(p_off),
                                                       static_cast<int>(sgi * seg_bytes), 0));
    };
    double vc[kAhead], vs[kAhead];
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      const int sgi = sub + kSubsets * e < segments ? sub + kSubsets * e : segments - 1;
      vc[e] = load_partial(cx_rsrc, sgi);
      vs[e] = load_partial(s_rsrc, sgi);
    }
    __builtin_amdgcn_sched_barrier(0);
    use_pass(q);
    for (int i0 = q + kPass * kFinishLanes; i0 < groups; i0 += kPass * kFinishLanes) {
      load_pass(i0);
      use_pass(i0);
    }
#pragma unroll
    for (int j = 0; j < kRowCols; ++j) {
      ry[j] = row_sum(ry[j]);
      if (first) yabs[j] = mul_up_nonneg(row_sum(yabs[j]), yabs_slack);
      if (q == 0) {
        red_ry[row + kFinishLanes * j] = ry[j];
        red_yabs[row + kFinishLanes * j] = yabs[j];
      }
    }

    // Partials, in the order of the segments: the first pass loaded above, later passes here.
    {
      double cx = 0.0, s = 0.0;
      for (int s0 = sub;;) {
#pragma unroll
        for (int e = 0; e < kAhead; ++e) {
          const bool in = s0 + kSubsets * e < segments;  // past the end: + 0.0, as above
          cx = cx + (in ? vc[e] : 0.0);
          s = s + (in ? vs[e] : 0.0);
        }
        s0 += kAhead * kSubsets;
        if (s0 >= segments) break;
#pragma unroll
        for (int e = 0; e < kAhead; ++e) {
          const int sgi = s0 + kSubsets * e < segments ? s0 + kSubsets * e : segments - 1;
          vc[e] = load_partial(cx_rsrc, sgi);
          vs[e] = load_partial(s_rsrc, sgi);
        }
      }
      red_cx[sub][pc] = cx;
      red_s[sub][pc] = s;
    }
    __syncthreads();
    if (t < kFinishCols && col0 + t < f.batch) {
      const PckBatchCheckDesc& d = plan.desc[g];
      const double cx = (red_cx[0][t] + red_cx[1][t]) + (red_cx[2][t] + red_cx[3][t]);
      const double s = (red_s[0][t] + red_s[1][t]) + (red_s[2][t] + red_s[3][t]);
      const double ya = red_yabs[t];
      const double s_bound = add_up_nonneg(s, static_cast<double>(f.n) * kSubnormalSlack);
      const double s_up = check::round_up_to_f32(mul_up_nonneg(s_bound, kSumSlack));
      const double rho = cx - red_ry[t];
      const double cabs_up = mul_up_nonneg(check::kOnePlusU32, s_up);
      const double eps = mul_up_nonneg(d.geps, add_up_nonneg(cabs_up, ya));
      const double tau =
          add_up_nonneg(add_up_nonneg(mul_up_nonneg(d.coef, s_up), eps), d.tau_floor);
      const int64_t at = pair * f.batch + col0 + t;
      d.passed[at] = __builtin_isfinite(ya) && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
      d.rho[at] = rho;
      d.tau[at] = tau;
    }
    __syncthreads();  // the LDS sums are rewritten for the next check
  } while (++k < f.checks);
}

// Fills the plan's counts; returns the workspace bytes, or -1 for an invalid descriptor.
int64_t make_plan(const PckBatchCheckDesc* descs, int count, Plan& plan) {
  if (count < 1 || count > PCK_MAX_BATCH || descs == nullptr) return -1;
  plan.count = count;
  int64_t tile_columns = 0;  // sum of pair tiles x column tiles x n
  int64_t max_n = 0;
  for (int g = 0; g < count; ++g) {
    const PckBatchCheckDesc& d = descs[g];
    if (d.num_blocks < 1 || d.checks < 1 || d.block < 4 || d.block % 4 != 0 ||
        d.block >= (int64_t{1} << 30) || d.n < 8 ||
        d.n % 8 != 0 || d.batch < 1 || !d.c || !d.a || !d.r || !d.X || !d.Y || !d.passed ||
        !d.rho || !d.tau || d.n > (1 << 20) || reinterpret_cast<uintptr_t>(d.X) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d.c) % 16 != 0 || reinterpret_cast<uintptr_t>(d.a) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d.Y) % 16 != 0 || reinterpret_cast<uintptr_t>(d.r) % 4 != 0 ||
        d.checks * d.num_blocks * d.n * 4 >= 0x80000000ll || d.batch * d.n * 2 >= 0x80000000ll ||
        d.num_blocks * ((d.batch + kFinishCols - 1) / kFinishCols) >= 0x80000000ll ||
        d.num_blocks * d.block * kFinishCols * 4 >= 0x80000000ll ||  // one finish's outputs
        !(d.coef >= 0.0 && d.geps >= 0.0 && d.tau_floor >= 0.0) ||  // NaN fails too
        !__builtin_isfinite(d.coef + d.geps + d.tau_floor))
      return -1;
    plan.desc[g] = d;
    const int64_t pairs = d.checks * d.num_blocks;
    plan.pair_tiles[g] = (pairs + kPairsWG - 1) / kPairsWG;
    tile_columns += plan.pair_tiles[g] * ((d.batch + kColsWG - 1) / kColsWG) * d.n;
    max_n = d.n > max_n ? d.n : max_n;
  }
  // Segment length: the shortest multiple of (quarters x kRing steps) that keeps the grid within
  // kTargetGroups workgroups, so that every CU holds at most one and no CU waits for a second
  // (longest rows when no length does).
  constexpr int64_t kQuantum = kWaves * kRing * kStep;
  int64_t seg = (tile_columns / kTargetGroups + kQuantum - 1) / kQuantum * kQuantum;
  seg = seg < kQuantum ? kQuantum : seg;
  for (;; seg += kQuantum) {
    int64_t groups = 0;
    for (int g = 0; g < count; ++g)
      groups += plan.pair_tiles[g] * ((descs[g].batch + kColsWG - 1) / kColsWG) *
                ((descs[g].n + seg - 1) / seg);
    if (groups <= kTargetGroups || seg >= max_n) break;
  }
  plan.seg_len = seg;
  plan.start[0] = 0;
  plan.finish[0] = 0;
  plan.slots[0] = 0;
  for (int g = 0; g < count; ++g) {
    const PckBatchCheckDesc& d = plan.desc[g];
    const int64_t pairs = d.checks * d.num_blocks;
    plan.segments[g] = (d.n + seg - 1) / seg;
    const int64_t col_tiles = (d.batch + kColsWG - 1) / kColsWG;
    plan.start[g + 1] = plan.start[g] + plan.pair_tiles[g] * col_tiles * plan.segments[g];
    plan.finish[g + 1] =
        plan.finish[g] + d.num_blocks * ((d.batch + kFinishCols - 1) / kFinishCols);
    plan.slots[g + 1] = plan.slots[g] + pairs * d.batch * plan.segments[g];
    PartialDesc& p = plan.part[g];
    p.c = d.c;
    p.a = d.a;
    p.X = d.X;
    p.slot = plan.slots[g];
    p.start = static_cast<int32_t>(plan.start[g]);
    p.segments = static_cast<int32_t>(plan.segments[g]);
    p.pair_tiles = static_cast<int32_t>(plan.pair_tiles[g]);
    p.pairs = static_cast<int32_t>(pairs);
    p.num_blocks = static_cast<int32_t>(d.num_blocks);
    p.n = static_cast<int32_t>(d.n);
    p.batch = static_cast<int32_t>(d.batch);
    p.unused = 0;
    FinishDesc& f = plan.fin[g];
    f.Y = d.Y;
    f.r = d.r;
    f.slot = plan.slots[g];
    f.outs = pairs * d.batch;
    f.start = static_cast<int32_t>(plan.finish[g]);
    f.num_blocks = static_cast<int32_t>(d.num_blocks);
    f.block = static_cast<int32_t>(d.block);
    f.checks = static_cast<int32_t>(d.checks);
    f.batch = static_cast<int32_t>(d.batch);
    f.segments = static_cast<int32_t>(plan.segments[g]);
    f.n = static_cast<int32_t>(d.n);
    f.unused = 0;
  }
  for (int g = 0; g < PCK_MAX_BATCH; ++g) {
    const bool live = g < count && plan.start[g] <= INT32_MAX && plan.finish[g] <= INT32_MAX;
    plan.part_first[g] = live ? static_cast<int32_t>(plan.start[g]) : INT32_MAX;
    plan.fin_first[g] = live ? static_cast<int32_t>(plan.finish[g]) : INT32_MAX;
  }
  // one descriptor's partials are addressed with 32-bit byte offsets
  if (plan.slots[count] * static_cast<int64_t>(sizeof(double)) >= 0x80000000ll) return -1;
  return 2 * plan.slots[count] * static_cast<int64_t>(sizeof(double));
}

}  // namespace
}  // namespace pck

extern "C" int pck_batch_check_workspace(const PckBatchCheckDesc* descs, int count,
                                         int64_t* bytes) {
  pck::Plan plan{};
  const int64_t need = pck::make_plan(descs, count, plan);
  if (need < 0 || bytes == nullptr) return hipErrorInvalidValue;
  *bytes = need;
  return hipSuccess;
}

namespace pck {
namespace {

// Both launches of a planned check, with the partial sums in `workspace` (at least the plan's
// bytes, 8-byte aligned; every slot is written by the partial launch before the finish reads
// it, so it needs no clearing).
hipError_t launch_planned(Plan& plan, void* workspace, hipStream_t s) {
  const int count = plan.count;
  plan.part_cx = static_cast<double*>(workspace);
  plan.part_s = plan.part_cx + plan.slots[count];
  const int64_t groups = plan.start[count];
  const int64_t finishers = plan.finish[count];
  if (groups > 0x7FFFFFFF || finishers > 0x7FFFFFFF) return hipErrorInvalidValue;
  partial_kernel<<<dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0, s>>>(plan);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  finish_kernel<<<dim3(static_cast<unsigned>(finishers)), dim3(kThreads), 0, s>>>(plan);
  return hipGetLastError();
}

// The allocation-free entry's workspace: file-scope device memory, one copy on every GPU the
// library runs on, held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address): each device's address
// comes from hipGetSymbolAddress, once per device, with that device current.
constexpr int64_t kScratchBytes = int64_t{16} << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) double scratch[kScratchBytes / sizeof(double)];
std::atomic<void*> g_scratch_address[kMaxDevices];

// The current device's address of `scratch` (looked up on this device's first call), or null
// with the error in `err`.
void* scratch_address(hipError_t& err) {
  int device = -1;
  err = hipGetDevice(&device);
  if (err != hipSuccess) return nullptr;
  if (device < 0 || device >= kMaxDevices) {
    err = hipErrorInvalidDevice;
    return nullptr;
  }
  void* known = g_scratch_address[device].load(std::memory_order_acquire);
  if (known != nullptr) return known;
  void* address = nullptr;
  err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
  if (err != hipSuccess || address == nullptr) {
    if (err == hipSuccess) err = hipErrorInvalidSymbol;
    return nullptr;
  }
  g_scratch_address[device].store(address, std::memory_order_release);  // same value if raced
  return address;
}

}  // namespace
}  // namespace pck

extern "C" int pck_batch_check(const PckBatchCheckDesc* descs, int count, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  pck::Plan plan{};
  const int64_t need = pck::make_plan(descs, count, plan);
  if (need < 0 || workspace == nullptr || workspace_bytes < need ||
      reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
    return hipErrorInvalidValue;
  return pck::launch_planned(plan, workspace, static_cast<hipStream_t>(stream));
}

extern "C" int64_t pck_batch_check_static_bytes(void) { return pck::kScratchBytes; }

extern "C" int pck_batch_check_static_init(void) {
  hipError_t err = hipSuccess;
  return pck::scratch_address(err) != nullptr ? hipSuccess : err;
}

extern "C" int pck_batch_check_static(const PckBatchCheckDesc* descs, int count, void* stream) {
  pck::Plan plan{};
  const int64_t need = pck::make_plan(descs, count, plan);
  if (need < 0) return hipErrorInvalidValue;
  if (need > pck::kScratchBytes) return hipErrorOutOfMemory;  // beyond the static scratch
  hipError_t err = hipSuccess;
  void* workspace = pck::scratch_address(err);
  if (workspace == nullptr) return err;
  return pck::launch_planned(plan, workspace, static_cast<hipStream_t>(stream));
}
