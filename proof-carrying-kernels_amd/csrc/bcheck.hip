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
constexpr int kTargetGroups = 512;   // about two workgroups per CU on MI355X
constexpr int kFinishLanes = 16;    // finish: lanes per block's outputs (a DPP row)
constexpr int kFinishCols = 64;     // finish: batch columns per workgroup
constexpr double kSumSlack = 1.0 + 0x1p-16;
constexpr double kSubnormalSlack = 0x1p-124;  // per column of the reduction

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct Plan {
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
  const u16x8 h = __builtin_bit_cast(u16x8, v & 0x7FFF7FFFu);
  const u16x8 f = __builtin_elementwise_max(h, (u16x8)(0x80));
  return __builtin_bit_cast(bf16x8, f);
}

__global__ void __launch_bounds__(kThreads) partial_kernel(const Plan plan) {
  __shared__ double red[2][kWaves][kPairsWG][kColsWG + 1];  // [c.x, a.|x|][quarter][pair][col]

  const int64_t item = blockIdx.x;
  // The descriptor: every comparison at once, so its loads are not a chain of dependent ones.
  int g = 0;
#pragma unroll
  for (int i = 1; i < PCK_MAX_BATCH; ++i) g += (i < plan.count && item >= plan.start[i]) ? 1 : 0;
  const PckBatchCheckDesc& d = plan.desc[g];
  const int64_t local = item - plan.start[g];
  const int64_t segments = plan.segments[g];
  const int64_t seg = local % segments;
  const int64_t tile = local / segments;
  const int64_t pair0 = (tile % plan.pair_tiles[g]) * kPairsWG;
  const int64_t col0 = (tile / plan.pair_tiles[g]) * kColsWG;
  const int64_t pairs = d.checks * d.num_blocks;
  const int64_t n = d.n;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / 64);
  const int64_t quarter = plan.seg_len / kWaves;
  const int64_t j_seg_hi = (seg + 1) * plan.seg_len < n ? (seg + 1) * plan.seg_len : n;
  const int64_t j_lo = seg * plan.seg_len + wave * quarter;
  const int64_t j_hi = j_lo + quarter < j_seg_hi ? j_lo + quarter : j_seg_hi;
  const int steps = j_hi > j_lo ? static_cast<int>((j_hi - j_lo + kStep - 1) / kStep) : 0;

  // Lane l = 16 q + i supplies row i of the A tiles (bank rows) and column i of the B tiles
  // (batch rows) at the step's columns 8 q .. 8 q + 7: FP64 step e takes column 8 q + e as its
  // K slot q, the BF16 step takes all eight as its K slots of lane group q.  Raw buffer loads,
  // issued unconditionally (so the loads in flight are counted exactly): rows and columns past
  // the operands or past the quarter point past the buffer and read zero (n % 8 == 0 and every
  // bound is a multiple of 8: a lane's eight columns are all in or all out).
  const int lane = static_cast<int>(threadIdx.x) % 64;
  const int li = lane % 16, lq = lane / 16;
  const __amdgpu_buffer_rsrc_t rc = check::make_rsrc(d.c, static_cast<uint32_t>(pairs * n * 4));
  const __amdgpu_buffer_rsrc_t ra =
      check::make_rsrc(d.a, static_cast<uint32_t>(d.num_blocks * n * 2));
  const __amdgpu_buffer_rsrc_t rx = check::make_rsrc(d.X, static_cast<uint32_t>(d.batch * n * 2));
  const int64_t j_lane = j_lo + 8 * lq;
  uint32_t c_voff[2], a_voff[2], x_voff[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t pair = pair0 + kTile * t + li;
    const int64_t col = col0 + kTile * t + li;
    c_voff[t] = pair < pairs ? static_cast<uint32_t>((pair * n + j_lane) * 4) : check::kOutOfRange;
    a_voff[t] = pair < pairs ? static_cast<uint32_t>(((pair % d.num_blocks) * n + j_lane) * 2)
                             : check::kOutOfRange;
    x_voff[t] = col < d.batch ? static_cast<uint32_t>((col * n + j_lane) * 2) : check::kOutOfRange;
  }

  auto fetch = [&](int step) {
    const int st = step < steps ? step : (steps > 0 ? steps - 1 : 0);  // past the end: unused
    const uint32_t at = static_cast<uint32_t>(st) * kStep;
    // the select is on the offset, so nothing waits for the load here
    const bool in = j_lane + static_cast<int64_t>(st) * kStep < j_hi;
    Staged v;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v.c[t][0] = load_b128(rc, in ? c_voff[t] + at * 4 : check::kOutOfRange);
      v.c[t][1] = load_b128(rc, in ? c_voff[t] + at * 4 + 16 : check::kOutOfRange);
      v.a[t] = load_b128(ra, in ? a_voff[t] + at * 2 : check::kOutOfRange);
      v.x[t] = load_b128(rx, in ? x_voff[t] + at * 2 : check::kOutOfRange);
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
  // to the loop head.
  Staged ring[kRing];
#pragma unroll
  for (int k = 0; k < kRing; ++k) ring[k] = fetch(k);
  const int full = steps / kRing * kRing;
  for (int base = 0; base < full; base += kRing) {
    [&]<int... K>(std::integer_sequence<int, K...>) {
      ((consume(ring[K]), ring[K] = fetch(base + K + kRing)), ...);
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
  const int64_t outs = pairs * d.batch;
  double* dst_cx = plan.part_cx + plan.slots[g] + seg * outs;
  double* dst_s = plan.part_s + plan.slots[g] + seg * outs;
  const int t = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < kPairsWG * kColsWG / kThreads; ++i) {
    const int o = t + kThreads * i;
    const int pr = o / kColsWG, cl = o % kColsWG;
    const int64_t pair = pair0 + pr, col = col0 + cl;
    if (pair < pairs && col < d.batch) {
      dst_cx[pair * d.batch + col] =
          (red[0][0][pr][cl] + red[0][1][pr][cl]) + (red[0][2][pr][cl] + red[0][3][pr][cl]);
      dst_s[pair * d.batch + col] =
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
//   instruction reads 64 consecutive columns of one segment); the four subsets meet in LDS as
//   (p0 + p1) + (p2 + p3).
//   Lanes 0 .. 63 then form rho, tau and the verdict of one column each; every operand of tau is
//   non-negative (the plan checks the constants), so the branch-free round-up operations apply.
__global__ void __launch_bounds__(kThreads) finish_kernel(const Plan plan) {
  constexpr int kRowCols = kFinishCols / kFinishLanes;  // columns per row of 16 lanes
  constexpr int kSubsets = kThreads / kFinishCols;      // segment subsets
  constexpr int kPass = 2;                              // float4 groups per lane per pass
  __shared__ double red_ry[kFinishCols], red_yabs[kFinishCols];
  __shared__ double red_cx[kSubsets][kFinishCols], red_s[kSubsets][kFinishCols];

  const int64_t item = blockIdx.x;
  int g = 0;
#pragma unroll
  for (int i = 1; i < PCK_MAX_BATCH; ++i) g += (i < plan.count && item >= plan.finish[i]) ? 1 : 0;
  const PckBatchCheckDesc& d = plan.desc[g];
  const int local = static_cast<int>(item - plan.finish[g]);  // < 2^31
  const int nb = static_cast<int>(d.num_blocks);
  const int beta = local % nb;
  const int64_t col0 = static_cast<int64_t>(local / nb) * kFinishCols;
  const int t = static_cast<int>(threadIdx.x);
  const int row = t / kFinishLanes, q = t % kFinishLanes;
  const int64_t m = d.num_blocks * d.block;
  const int groups = static_cast<int>(d.block / 4);  // block % 4 == 0
  const int segments = static_cast<int>(plan.segments[g]);
  const int64_t outs = d.checks * d.num_blocks * d.batch;
  // Every load below is unconditional, at a valid address (a column past the batch reads
  // column 0, a group or segment past the end reads the last one), and data that is not needed
  // is dropped where it is used: a conditional load would be followed by a wait for it before
  // the next one could be issued.  The sums of columns past the batch are computed and never
  // read.
  const float4* ycol[kRowCols];
#pragma unroll
  for (int j = 0; j < kRowCols; ++j) {
    const int64_t col = col0 + row + kFinishLanes * j;
    ycol[j] = reinterpret_cast<const float4*>(d.Y + (col < d.batch ? col : 0) * m + beta * d.block);
  }

  // sum |y| to nearest, at most block / 16 + 4 additions deep, then raised by 1 + (b + 4) 2^-52
  // (the factor is exact in FP64)
  const double yabs_slack = 1.0 + static_cast<double>(d.block + 4) * 0x1p-52;
  double yabs[kRowCols] = {};
  const int pc = t % kFinishCols, sub = t / kFinishCols;  // partials: column, segment subset
  const bool pin = col0 + pc < d.batch;
  constexpr int kAhead = 8;
  for (int64_t k = 0; k < d.checks; ++k) {
    const int64_t pair = k * d.num_blocks + beta;
    const uint32_t* sign = reinterpret_cast<const uint32_t*>(d.r + pair * d.block);
    // The first pass of this lane's partials (column t % 64, segments t / 64, t / 64 + 4, ...)
    // is requested before the outputs, so both reads are in flight together.
    const int64_t pat = pair * d.batch + (pin ? col0 + pc : 0);
    const double* pcx = plan.part_cx + plan.slots[g] + pat;
    const double* ps = plan.part_s + plan.slots[g] + pat;
    double vc[kAhead], vs[kAhead];
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      const int sgi = sub + kSubsets * e < segments ? sub + kSubsets * e : segments - 1;
      vc[e] = pcx[sgi * outs];
      vs[e] = ps[sgi * outs];
    }
    double ry[kRowCols] = {};
    for (int i0 = q; i0 < groups; i0 += kPass * kFinishLanes) {
      float4 v[kRowCols][kPass];
      uint32_t sg[kPass];
#pragma unroll
      for (int e = 0; e < kPass; ++e) {
        const int i = i0 + kFinishLanes * e < groups ? i0 + kFinishLanes * e : groups - 1;
        sg[e] = sign[i];
#pragma unroll
        for (int j = 0; j < kRowCols; ++j) v[j][e] = ycol[j][i];
      }
#pragma unroll
      for (int e = 0; e < kPass; ++e) {
        if (i0 + kFinishLanes * e >= groups) break;
#pragma unroll
        for (int j = 0; j < kRowCols; ++j) {
          const float f[4] = {v[j][e].x, v[j][e].y, v[j][e].z, v[j][e].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const double yd = static_cast<double>(f[h]);
            const bool plus = static_cast<int8_t>((sg[e] >> (8 * h)) & 0xFFu) > 0;
            ry[j] = ry[j] + (plus ? yd : -yd);
            if (k == 0) yabs[j] = yabs[j] + __builtin_fabs(yd);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kRowCols; ++j) {
      ry[j] = row_sum(ry[j]);
      if (k == 0) yabs[j] = mul_up_nonneg(row_sum(yabs[j]), yabs_slack);
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
          if (s0 + kSubsets * e >= segments) break;
          cx = cx + vc[e];
          s = s + vs[e];
        }
        s0 += kAhead * kSubsets;
        if (s0 >= segments) break;
#pragma unroll
        for (int e = 0; e < kAhead; ++e) {
          const int sgi = s0 + kSubsets * e < segments ? s0 + kSubsets * e : segments - 1;
          vc[e] = pcx[sgi * outs];
          vs[e] = ps[sgi * outs];
        }
      }
      red_cx[sub][pc] = cx;
      red_s[sub][pc] = s;
    }
    __syncthreads();
    if (t < kFinishCols && col0 + t < d.batch) {
      const double cx = (red_cx[0][t] + red_cx[1][t]) + (red_cx[2][t] + red_cx[3][t]);
      const double s = (red_s[0][t] + red_s[1][t]) + (red_s[2][t] + red_s[3][t]);
      const double ya = red_yabs[t];
      const double s_bound = add_up_nonneg(s, static_cast<double>(d.n) * kSubnormalSlack);
      const double s_up = check::round_up_to_f32(mul_up_nonneg(s_bound, kSumSlack));
      const double rho = cx - red_ry[t];
      const double cabs_up = mul_up_nonneg(check::kOnePlusU32, s_up);
      const double eps = mul_up_nonneg(d.geps, add_up_nonneg(cabs_up, ya));
      const double tau =
          add_up_nonneg(add_up_nonneg(mul_up_nonneg(d.coef, s_up), eps), d.tau_floor);
      const int64_t at = pair * d.batch + col0 + t;
      d.passed[at] = __builtin_isfinite(ya) && __builtin_isfinite(tau) && __builtin_fabs(rho) <= tau;
      d.rho[at] = rho;
      d.tau[at] = tau;
    }
    __syncthreads();  // the LDS sums are rewritten for the next check
  }
}

// Fills the plan's counts; returns the workspace bytes, or -1 for an invalid descriptor.
int64_t make_plan(const PckBatchCheckDesc* descs, int count, Plan& plan) {
  if (count < 1 || count > PCK_MAX_BATCH || descs == nullptr) return -1;
  plan.count = count;
  int64_t tile_columns = 0;  // sum of pair tiles x column tiles x n
  for (int g = 0; g < count; ++g) {
    const PckBatchCheckDesc& d = descs[g];
    if (d.num_blocks < 1 || d.checks < 1 || d.block < 4 || d.block % 4 != 0 || d.n < 8 ||
        d.n % 8 != 0 || d.batch < 1 || !d.c || !d.a || !d.r || !d.X || !d.Y || !d.passed ||
        !d.rho || !d.tau || d.n > (1 << 20) || reinterpret_cast<uintptr_t>(d.X) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d.c) % 16 != 0 || reinterpret_cast<uintptr_t>(d.a) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d.Y) % 16 != 0 || reinterpret_cast<uintptr_t>(d.r) % 4 != 0 ||
        d.checks * d.num_blocks * d.n * 4 >= 0x80000000ll || d.batch * d.n * 2 >= 0x80000000ll ||
        d.num_blocks * ((d.batch + kFinishCols - 1) / kFinishCols) >= 0x80000000ll ||
        !(d.coef >= 0.0 && d.geps >= 0.0 && d.tau_floor >= 0.0) ||  // NaN fails too
        !__builtin_isfinite(d.coef + d.geps + d.tau_floor))
      return -1;
    plan.desc[g] = d;
    const int64_t pairs = d.checks * d.num_blocks;
    plan.pair_tiles[g] = (pairs + kPairsWG - 1) / kPairsWG;
    tile_columns += plan.pair_tiles[g] * ((d.batch + kColsWG - 1) / kColsWG) * d.n;
  }
  // Segment length: a multiple of (quarters x kRing steps) giving about kTargetGroups
  // workgroups.
  constexpr int64_t kQuantum = kWaves * kRing * kStep;
  int64_t seg = (tile_columns / kTargetGroups + kQuantum - 1) / kQuantum * kQuantum;
  seg = seg < kQuantum ? kQuantum : seg;
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
  }
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
