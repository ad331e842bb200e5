// GEMV y = W x for the decode hot path on gfx950: BF16 or OCP FP8 E4M3FN weights, BF16 x,
// FP32 accumulation and output.
//
// Numerics are defined by the summation tree, not by the hardware mapping.  The coalesced tree
// of `threads` = T virtual lanes (reference src/pck/cuda/csrc/gemv_kernel.cu:139-178, model
// src/pck/gemv.py:71-101): virtual lane t owns the 16-byte vectors t, t + T, t + 2T, ... of a
// row (8 BF16 or 16 FP8 columns each) and adds their products one at a time in column order,
// starting from its first product, with columns past n contributing +0; each virtual warp of
// 32 lanes is reduced by halving, then the T / 32 warp sums are reduced by halving.
//
// Hardware mapping (MI355X, wave64): one wave computes one row (two rows when T = 32).  Lane l
// of the wave runs the T / 64 chains l, l + 64, l + 128, ... so that for every vector index the
// wave reads 64 consecutive 16-byte vectors (1 KiB, fully coalesced), and all of a lane's loads
// for U vector positions are issued before any product is consumed, which keeps enough bytes in
// flight per CU to stream HBM.  The two halves of a wave are the two virtual warps 2j and
// 2j + 1 of chain slot j, so the in-warp halving is a width-32 xor butterfly (lane 0 of each
// half ends with exactly the halving order's value), and the warp sums are combined in the
// halving order from uniform registers.  No LDS and no barrier are needed.
//
// Products: BF16 x BF16 (8 + 8 significand bits) and E4M3 x BF16 (4 + 8) are exact in FP32
// except under underflow; they are formed with a separate v_mul_f32 and added with v_add_f32 (the
// library is built with -ffp-contract=off), exactly the reference's __fmul_rn / __fadd_rn.  The
// chain accumulator starts at -0.0, the additive identity of IEEE round-to-nearest, so
// "-0 + p0" equals "start from p0" bit for bit, signed zero included.
//
// The naive tree (reference model src/pck/gemv.py:14-57) fixes a different order: virtual lane
// t sums the contiguous chunk [t c, (t + 1) c) of a row, then neighbour pairs combine level by
// level.  Its kernel maps the levels of stride below 64 onto DPP / permlane moves inside a wave
// and meets only the wave sums in LDS (gemv_naive_kernel below).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "check_pair.h"
#include "pck_hip.h"
#include "rowsum_check.h"

namespace pck {
namespace {

constexpr int kWave = 64;
constexpr int kWarp = 32;
constexpr int kWavesPerGroup = 4;
constexpr int kGroupThreads = kWave * kWavesPerGroup;

struct GemvItem {
  const void* W;
  const uint16_t* x;
  float* y;
  double* sums;  // (m, 2) FP64 row sums (d_i, s_i) of the in-pass path; unused otherwise
  int64_t m;
  int64_t n;
  int64_t per_lane;  // vectors per virtual lane: ceil(ceil(n / vec) / T)
  const float* scale = nullptr;  // (m,) FP32 row scales of an FP8 weight, with y_scaled
  float* y_scaled = nullptr;     // (m,) scale[i] * y[i], rounded to nearest; or null
};

// Writes row `row` of an item: the tree's sum, and the dequantised output `scale * value` when
// the item has row scales (one FP32 multiply, as y = s z would round it).
__device__ __forceinline__ void store_row(const GemvItem& it, int64_t row, float value,
                                          float scale) {
  it.y[row] = value;
  if (it.y_scaled != nullptr) it.y_scaled[row] = scale * value;
}

struct GemvBatch {
  GemvItem item[PCK_MAX_GROUP];
  int64_t first_group[PCK_MAX_GROUP + 1];  // workgroup prefix sums
  int count;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Two E4M3FN codes (bytes 0-1, or 2-3 with kHigh) of `w` to FP32, exactly (hardware OCP decode).
template <bool kHigh>
__device__ __forceinline__ float2 fp8_pair(uint32_t w) {
  auto v = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), kHigh);
  return make_float2(v[0], v[1]);
}

__device__ __forceinline__ float fp8_one(uint8_t code) { return fp8_pair<false>(code).x; }

// Row sums of the in-pass path, from the FP32 products the tree already forms (exact: 8 + 8 or
// 4 + 8 significand bits, barring FP32 underflow).  Each pair of consecutive products is added
// in FP32 (rounding error at most u32 (|p0| + |p1|)), widened and added to d in FP64; |p| is
// added to s in FP32, one product at a time in column order.
struct RowSums {
  double d = 0.0;
  float s = 0.0f;
};

template <bool kSums>
__device__ __forceinline__ void add_pair(RowSums& rs, float p0, float p1) {
  if constexpr (kSums) {
    rs.d = rs.d + static_cast<double>(p0 + p1);
    rs.s = rs.s + __builtin_fabsf(p0);
    rs.s = rs.s + __builtin_fabsf(p1);
  }
}

// Adds the products of one vector to `acc` (and, with kSums, to the row sums), in column order.
template <bool kFp8, bool kSums = false>
__device__ __forceinline__ void add_products(float& acc, RowSums& rs, const uint4& w,
                                             const uint4& xa, const uint4& xb) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  if constexpr (!kFp8) {
    const uint32_t xd[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float p0 = bf16_lo(wd[k]) * bf16_lo(xd[k]);
      const float p1 = bf16_hi(wd[k]) * bf16_hi(xd[k]);
      acc = acc + p0;
      acc = acc + p1;
      add_pair<kSums>(rs, p0, p1);
    }
  } else {
    const uint32_t xd[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float2 f01 = fp8_pair<false>(wd[k]);
      const float2 f23 = fp8_pair<true>(wd[k]);
      const float p0 = f01.x * bf16_lo(xd[2 * k]);
      const float p1 = f01.y * bf16_hi(xd[2 * k]);
      const float p2 = f23.x * bf16_lo(xd[2 * k + 1]);
      const float p3 = f23.y * bf16_hi(xd[2 * k + 1]);
      acc = acc + p0;
      acc = acc + p1;
      acc = acc + p2;
      acc = acc + p3;
      add_pair<kSums>(rs, p0, p1);
      add_pair<kSums>(rs, p2, p3);
    }
  }
}

// Element loads for rows that cannot take 16-byte vectors (n not a multiple of the vector width
// or a misaligned pointer): the same products in the same order, +0 past n.
template <bool kFp8, bool kSums = false>
__device__ __forceinline__ void add_products_scalar(float& acc, RowSums& rs, const void* w_row,
                                                    const uint16_t* x, int64_t col, int64_t n) {
  constexpr int V = kFp8 ? 16 : 8;
  float p[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t j = col + k;
    p[k] = 0.0f;
    if (j < n) {
      const float xv = __uint_as_float(static_cast<uint32_t>(x[j]) << 16);
      float wv;
      if constexpr (kFp8) {
        wv = fp8_one(static_cast<const uint8_t*>(w_row)[j]);
      } else {
        wv = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(w_row)[j]) << 16);
      }
      p[k] = wv * xv;
    }
    acc = acc + p[k];
  }
#pragma unroll
  for (int k = 0; k < V; k += 2) add_pair<kSums>(rs, p[k], p[k + 1]);
}

// a[i] += a[i + 16] ... a[0] += a[1] inside each 32-lane half of the wave, the halving order of
// the reference's 32-lane shuffle-down reduction, with lane 0 (and lane 32) ending on a[0].
// Step 16 moves whole rows of 16 lanes with gfx950's v_permlane16_swap (the second result holds
// each even row's partner row); steps 8 and 4 rotate inside a row (row_ror:8 gives lane i the
// value of lane i ^ 8, row_ror:12 that of lane i + 4 for the lanes i < 4 that matter); steps 2
// and 1 are quad permutes.  Everything stays in VALU instructions (DPP folds into the adds).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float halve32(float v) {
  const auto swapped = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false,
                                                        false);
  v = v + __int_as_float(swapped[1]);  // lanes 0-15 (32-47) receive lanes 16-31 (48-63)
  v = v + dpp_move<0x128>(v);          // row_ror:8
  v = v + dpp_move<0x12C>(v);          // row_ror:12
  v = v + dpp_move<0x4E>(v);           // quad_perm [2,3,0,1]
  v = v + dpp_move<0xB1>(v);           // quad_perm [1,0,3,2]
  return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// T virtual lanes per row, R rows per wave slot, U vector positions loaded ahead, kNt:
// non-temporal weight loads (streamed once, so they need not displace x in the caches).
// kPad: some vectors of a chain lie past n (n is not a multiple of T * vec), so loads of those
// are redirected to column 0 and their data replaced by zeros.  kVector: 16-byte loads (n is a
// multiple of vec and the pointers are aligned); otherwise element loads.
template <bool kNt>
__device__ __forceinline__ uint4 load_w(const unsigned char* p) {
  if constexpr (kNt) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

template <int T, int R, int U, bool kFp8, bool kVector, bool kPad, bool kNt, bool kSums = false>
__device__ __forceinline__ void gemv_rows(const GemvBatch& batch, int64_t group) {
  constexpr int V = kFp8 ? 16 : 8;
  constexpr int kLanesPerRow = T >= kWave ? kWave : T;
  constexpr int kSlots = kWave / kLanesPerRow;  // rows side by side in one wave (2 if T = 32)
  constexpr int kChains = T / kLanesPerRow;     // chains per lane
  constexpr int kElemBytes = kFp8 ? 1 : 2;

  int g = 0;
  while (g + 1 < batch.count && group >= batch.first_group[g + 1]) ++g;
  const GemvItem& it = batch.item[g];
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int64_t wave =
      (group - batch.first_group[g]) * kWavesPerGroup + (static_cast<int>(threadIdx.x) >> 6);
  const int slot = lane / kLanesPerRow;
  const int chain0 = lane % kLanesPerRow;
  const int64_t n = it.n;
  const int64_t P = it.per_lane;
  const uint16_t* __restrict__ x = it.x;

  // Rows past m compute on row m - 1 (a valid address) and are not stored.
  const unsigned char* w_rows[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = (wave * kSlots + slot) * R + r;
    live[r] = row < it.m;
    w_rows[r] =
        static_cast<const unsigned char*>(it.W) + (live[r] ? row : it.m - 1) * n * kElemBytes;
  }

  // Row scales of a scaled FP8 item, loaded ahead of the weight stream so that their latency
  // is hidden behind it instead of adding a dependent load to the launch's tail.
  float scale[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = (wave * kSlots + slot) * R + r;
    scale[r] = (kFp8 && it.y_scaled != nullptr) ? it.scale[live[r] ? row : it.m - 1] : 1.0f;
  }

  float acc[R][kChains];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[r][j] = -0.0f;
  RowSums rs[R][kChains];  // per row and chain: the lane's d and s (kSums only)

  for (int64_t v0 = 0; v0 < P; v0 += U) {
    if constexpr (kVector) {
      uint4 wb[U][R][kChains];
      uint4 xa[U][kChains];
      uint4 xb[U][kChains];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (U > 1 && v0 + u >= P) break;  // uniform: the tail of the last block
#pragma unroll
        for (int j = 0; j < kChains; ++j) {
          const int64_t col = ((v0 + u) * T + chain0 + kLanesPerRow * j) * V;
          const int64_t at = (!kPad || col < n) ? col : 0;
          xa[u][j] = *reinterpret_cast<const uint4*>(x + at);
          if constexpr (kFp8) xb[u][j] = *reinterpret_cast<const uint4*>(x + at + 8);
#pragma unroll
          for (int r = 0; r < R; ++r)
            wb[u][r][j] = load_w<kNt>(w_rows[r] + at * kElemBytes);
          if constexpr (kPad) {
            if (col >= n) {  // a padding vector: +0 products (0 x 0)
              xa[u][j] = make_uint4(0, 0, 0, 0);
              xb[u][j] = make_uint4(0, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < R; ++r) wb[u][r][j] = make_uint4(0, 0, 0, 0);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (U > 1 && v0 + u >= P) break;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int j = 0; j < kChains; ++j)
            add_products<kFp8, kSums>(acc[r][j], rs[r][j], wb[u][r][j], xa[u][j],
                                      kFp8 ? xb[u][j] : xa[u][j]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int j = 0; j < kChains; ++j) {
          const int64_t col = (v0 * T + chain0 + kLanesPerRow * j) * V;
          add_products_scalar<kFp8, kSums>(acc[r][j], rs[r][j], w_rows[r], x, col, n);
        }
      }
    }
  }

  if constexpr (kSums) {
    // Each lane combines its chains' sums in halving order (chain i += chain i + half), then
    // the row's lanes combine theirs by an xor butterfly (symmetric, so every lane of the row
    // ends with the same pair); the row's first lane stores it as one 16-byte write.
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int half = kChains / 2; half > 0; half /= 2)
#pragma unroll
        for (int i = 0; i < half; ++i) {
          rs[r][i].d = rs[r][i].d + rs[r][i + half].d;
          rs[r][i].s = rs[r][i].s + rs[r][i + half].s;
        }
      RowSums t = rs[r][0];
#pragma unroll
      for (int off = kLanesPerRow / 2; off > 0; off /= 2) {
        const double od = __shfl_xor(t.d, off, kWave);
        const float os = __shfl_xor(t.s, off, kWave);
        t.d = t.d + od;
        t.s = t.s + os;
      }
      const int64_t row = (wave * kSlots + slot) * R + r;
      if (chain0 == 0 && live[r])
        reinterpret_cast<double2*>(it.sums)[row] = make_double2(t.d, static_cast<double>(t.s));
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    // Halving inside each 32-lane virtual warp.
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[r][j] = halve32(acc[r][j]);
    const int64_t row = (wave * kSlots + slot) * R + r;
    if constexpr (kSlots == 2) {
      // T = 32: one virtual warp per row; lanes 0 and 32 hold the two rows' sums.
      if (chain0 == 0 && live[r]) store_row(it, row, acc[r][0], scale[r]);
    } else {
      // Warp w = 2j + h is half h of chain slot j; reduce the T / 32 warp sums by halving.
      constexpr int kWarps = 2 * kChains;
      float ws[kWarps];
#pragma unroll
      for (int j = 0; j < kChains; ++j) {
        ws[2 * j] = lane_value(acc[r][j], 0);
        ws[2 * j + 1] = lane_value(acc[r][j], kWarp);
      }
#pragma unroll
      for (int half = kWarps / 2; half > 0; half /= 2)
#pragma unroll
        for (int i = 0; i < half; ++i) ws[i] = ws[i] + ws[i + half];
      if (lane == 0 && live[r]) store_row(it, row, ws[0], scale[r]);
    }
  }
}

template <int T, int R, int U, bool kFp8, bool kVector, bool kPad, bool kNt>
__global__ void __launch_bounds__(kGroupThreads) gemv_tree_kernel(const GemvBatch batch) {
  gemv_rows<T, R, U, kFp8, kVector, kPad, kNt>(batch, blockIdx.x);
}

// A GEMV launch that also checks outputs of earlier launches: the first workgroups of the grid
// each run one (check, block) pair of `ride` (the standalone checker's code, so rho, tau and the
// verdicts are bit-identical to pck_blocked_check), the rest compute the GEMV rows.  The checked
// y were written by launches that finished before this one started (stream order), and the
// checker workgroups are separate wavefronts that read them from memory; their latency hides
// behind the GEMV's streaming, and the bank reads add about 2.3% (BF16, b = 128) to the bytes.
// Rows longer than 4,096 columns keep 8 quads per lane in flight (a 14,336-column row in two
// round trips instead of four); more would push the kernel past 128 VGPRs and halve the GEMV
// waves a SIMD holds.
template <int T, int R, int U, bool kFp8, bool kPad, bool kNt>
__global__ void __launch_bounds__(kGroupThreads)
    gemv_ride_kernel(const GemvBatch batch, const PckCheckBatch ride) {
  __shared__ check::Quad lds[check::kWaves];
  const int64_t items = ride.start[ride.count];
  if (static_cast<int64_t>(blockIdx.x) < items) {
    const int g = check::owner(ride, blockIdx.x);
    if (ride.desc[g].n > 4 * 4 * check::kThreads)
      check::check_pair<8>(ride, blockIdx.x, g, lds);
    else
      check::check_pair<4>(ride, blockIdx.x, g, lds);
    return;
  }
  gemv_rows<T, R, U, kFp8, true, kPad, kNt>(batch, static_cast<int64_t>(blockIdx.x) - items);
}

// The in-pass GEMV: the tree's outputs plus each row's sums (d_i, s_i), and in the first
// workgroups of the grid the row-sum checks of `ride` (outputs of earlier launches on the stream,
// read from memory; one wave per (check, block) pair, the code of pck_rowsum_check, so the
// results are bit-identical to it).  A check never reads anything this launch writes.
template <int T, int R, int U, bool kFp8, bool kVector, bool kPad, bool kNt>
__global__ void __launch_bounds__(kGroupThreads)
    gemv_rowsum_kernel(const GemvBatch batch, const PckRowSumBatch ride) {
  const int64_t items = rowsum::items(ride);
  const int64_t ride_groups = (items + kWavesPerGroup - 1) / kWavesPerGroup;
  const int64_t group = static_cast<int64_t>(blockIdx.x);
  if (group < ride_groups) {
    const int64_t item = group * kWavesPerGroup + (static_cast<int>(threadIdx.x) >> 6);
    if (item < items) rowsum::check_item(ride, item);  // uniform per wave
    return;
  }
  gemv_rows<T, R, U, kFp8, kVector, kPad, kNt, true>(batch, group - ride_groups);
}

// Naive tree (order of the reference model src/pck/gemv.py:14-57): `threads` = T virtual lanes
// per row, lane t owning the contiguous chunk [t c, (t + 1) c), c = ceil(n / T), summed in
// column order from its first product (columns past n add +0), then the T chain sums combined
// by neighbour pairs, stride 1, 2, 4, ...: a[t] += a[t + s] for t a multiple of 2s.
//
// One workgroup of max(T, 64) lanes per row, lane t of the workgroup being virtual lane t (lanes
// t >= T, present only when T < 64, own chunks wholly past n and feed no level below T).  The
// levels of stride 1 .. 32 run inside each wave: every lane adds the value of its partner lane
// t + s, moved by DPP (quad permutes for 1 and 2, row rotations for 4 and 8), permlane16_swap
// (16) or a read of lane 32 (32); the lanes that matter at a level read only lanes that
// mattered at the level before, so lane 0 ends with the wave's subtree.  The levels of stride 64
// and up combine the T / 64 wave sums, which meet in LDS behind one barrier, in the same pair
// order.  kVector: 16-byte loads of W and x (c and n multiples of 8, aligned pointers), every
// vector wholly before or wholly past n.
template <bool kVector>
__global__ void __launch_bounds__(1024)
    gemv_naive_kernel(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                      float* __restrict__ y, int64_t n, int64_t chunk, int threads) {
  __shared__ float wave_sum[1024 / kWave];
  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);
  const uint16_t* row = W + static_cast<int64_t>(blockIdx.x) * n;
  const int64_t first = static_cast<int64_t>(t) * chunk;

  float acc = 0.0f;
  if constexpr (kVector) {
    for (int64_t v = 0; v < chunk; v += 8) {
      const int64_t col = first + v;
      uint4 wv = make_uint4(0, 0, 0, 0), xv = make_uint4(0, 0, 0, 0);  // past n: +0 products
      if (col < n) {
        wv = *reinterpret_cast<const uint4*>(row + col);
        xv = *reinterpret_cast<const uint4*>(x + col);
      }
      const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
      const uint32_t xd[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float p0 = bf16_lo(wd[k]) * bf16_lo(xd[k]);
        const float p1 = bf16_hi(wd[k]) * bf16_hi(xd[k]);
        acc = (v == 0 && k == 0) ? p0 : acc + p0;
        acc = acc + p1;
      }
    }
  } else {
    for (int64_t j = first; j < first + chunk; ++j) {
      float p = 0.0f;
      if (j < n) p = __uint_as_float(static_cast<uint32_t>(row[j]) << 16) *
                     __uint_as_float(static_cast<uint32_t>(x[j]) << 16);
      acc = j == first ? p : acc + p;
    }
  }

  // Levels inside the wave (uniform bounds: `threads` is the same for every lane).
  if (threads > 1) acc = acc + dpp_move<0xB1>(acc);   // stride 1: quad_perm [1,0,3,2]
  if (threads > 2) acc = acc + dpp_move<0x4E>(acc);   // stride 2: quad_perm [2,3,0,1]
  if (threads > 4) acc = acc + dpp_move<0x12C>(acc);  // stride 4: row_ror:12, lane i <- i + 4
  if (threads > 8) acc = acc + dpp_move<0x128>(acc);  // stride 8: row_ror:8, lane i <- i + 8
  if (threads > 16) {                                  // stride 16: lanes 0-15 <- 16-31
    const auto swapped =
        __builtin_amdgcn_permlane16_swap(__float_as_int(acc), __float_as_int(acc), false, false);
    acc = acc + __int_as_float(swapped[1]);
  }
  if (threads > 32) acc = lane_value(acc, 0) + lane_value(acc, 32);  // stride 32

  if (threads <= kWave) {
    if (t == 0) y[blockIdx.x] = acc;
    return;
  }
  // Levels across waves: wave w's subtree is a[64 w]; pairs of stride 64, 128, ...
  if (lane == 0) wave_sum[t / kWave] = acc;
  __syncthreads();
  if (t == 0) {
    const int waves = threads / kWave;
    float a[1024 / kWave];
#pragma unroll
    for (int w = 0; w < 1024 / kWave; ++w) a[w] = w < waves ? wave_sum[w] : 0.0f;
#pragma unroll
    for (int s = 1; s < 1024 / kWave; s *= 2)
#pragma unroll
      for (int w = 0; w + s < 1024 / kWave; w += 2 * s)
        if (s < waves) a[w] = a[w] + a[w + s];
    y[blockIdx.x] = a[0];
  }
}

// Launch shape of the coalesced kernel: rows per wave slot, vector positions loaded ahead and
// non-temporal weight loads.  T = 256 (the reference's default tree) has every combination
// instantiated for tuning; other thread counts use one shape per padding / weight type.
struct TreeShape {
  int rows;
  int unroll;
  int nt;
};

TreeShape g_shape_override = {0, 0, 0};

// Defaults from sweeps of every shape over each Llama-3-8B decode launch on MI355X.  BF16:
// non-temporal weight loads won everywhere.  FP8 rows are half as long, so two rows per wave
// keep as many bytes in flight as one BF16 row, except for a launch of at most 4096 rows (o),
// where one row per wave and two positions ahead give twice the waves (4.9 against 5.4 us).
// The sweeps replay each launch over weight copies that do not fit the Infinity Cache (with
// four copies of FP8 down, 235 MB, plain loads won from the cache; streamed from HBM, as in a
// decode pass, non-temporal loads take 13.1 against 14.6 us).
TreeShape choose_shape(int64_t per_lane, int64_t rows, bool fp8) {
  if (g_shape_override.rows > 0) return g_shape_override;
  if (fp8) return per_lane <= 2 && rows <= 4096 ? TreeShape{1, 2, 1} : TreeShape{2, 1, 1};
  return per_lane > 2 ? TreeShape{2, 2, 1} : TreeShape{1, 2, 1};
}

// Fills the workgroup prefix sums for rows_per_group rows per workgroup; returns the total.
int64_t plan_groups(GemvBatch& batch, int64_t rows_per_group) {
  batch.first_group[0] = 0;
  for (int g = 0; g < batch.count; ++g) {
    batch.first_group[g + 1] =
        batch.first_group[g] + (batch.item[g].m + rows_per_group - 1) / rows_per_group;
  }
  return batch.first_group[batch.count];
}

// kSums: the in-pass kernel, with `rs` the row-sum checks it carries; otherwise the plain tree.
template <int T, int R, int U, bool kFp8, bool kVector, bool kPad, bool kNt, bool kSums>
hipError_t launch_tree(GemvBatch& batch, const PckRowSumBatch* rs, hipStream_t stream) {
  constexpr int kLanesPerRow = T >= kWave ? kWave : T;
  const int64_t groups = plan_groups(batch, (kWave / kLanesPerRow) * R * kWavesPerGroup);
  if constexpr (kSums) {
    const int64_t total = groups + (rowsum::items(*rs) + kWavesPerGroup - 1) / kWavesPerGroup;
    if (total == 0) return hipSuccess;
    if (total * kGroupThreads > 0xFFFFFFFFll) return hipErrorInvalidValue;  // 32-bit dispatch
    gemv_rowsum_kernel<T, R, U, kFp8, kVector, kPad, kNt>
        <<<dim3(static_cast<unsigned>(total)), dim3(kGroupThreads), 0, stream>>>(batch, *rs);
  } else {
    (void)rs;
    if (groups == 0) return hipSuccess;
    if (groups * kGroupThreads > 0xFFFFFFFFll) return hipErrorInvalidValue;  // 32-bit dispatch
    gemv_tree_kernel<T, R, U, kFp8, kVector, kPad, kNt>
        <<<dim3(static_cast<unsigned>(groups)), dim3(kGroupThreads), 0, stream>>>(batch);
  }
  return hipGetLastError();
}

template <int T, int R, bool kFp8, bool kPad, bool kNt, bool kSums>
hipError_t launch_unroll(GemvBatch& batch, int unroll, const PckRowSumBatch* rs, hipStream_t s) {
  if (unroll >= 4) return launch_tree<T, R, 4, kFp8, true, kPad, kNt, kSums>(batch, rs, s);
  if (unroll == 2) return launch_tree<T, R, 2, kFp8, true, kPad, kNt, kSums>(batch, rs, s);
  return launch_tree<T, R, 1, kFp8, true, kPad, kNt, kSums>(batch, rs, s);
}

template <int T, bool kFp8, bool kPad, bool kSums>
hipError_t launch_vector(GemvBatch& batch, TreeShape shape, const PckRowSumBatch* rs,
                         hipStream_t s) {
  if constexpr (T == 256) {
    const bool nt = shape.nt != 0;
    const int u = shape.unroll;
    switch (shape.rows) {
      case 4:
        return nt ? launch_unroll<T, 4, kFp8, kPad, true, kSums>(batch, u, rs, s)
                  : launch_unroll<T, 4, kFp8, kPad, false, kSums>(batch, u, rs, s);
      case 2:
        return nt ? launch_unroll<T, 2, kFp8, kPad, true, kSums>(batch, u, rs, s)
                  : launch_unroll<T, 2, kFp8, kPad, false, kSums>(batch, u, rs, s);
      default:
        return nt ? launch_unroll<T, 1, kFp8, kPad, true, kSums>(batch, u, rs, s)
                  : launch_unroll<T, 1, kFp8, kPad, false, kSums>(batch, u, rs, s);
    }
  } else {
    (void)shape;
    return launch_tree<T, 1, 2, kFp8, true, kPad, false, kSums>(batch, rs, s);
  }
}

template <int T, bool kFp8, bool kSums = false>
hipError_t launch_for_threads(GemvBatch& batch, bool vector, bool pad, TreeShape shape,
                              hipStream_t s, const PckRowSumBatch* rs = nullptr) {
  if (!vector) return launch_tree<T, 1, 1, kFp8, false, true, false, kSums>(batch, rs, s);
  return pad ? launch_vector<T, kFp8, true, kSums>(batch, shape, rs, s)
             : launch_vector<T, kFp8, false, kSums>(batch, shape, rs, s);
}

template <int R, int U, bool kFp8, bool kPad, bool kNt = true>
hipError_t launch_ride_shape(GemvBatch& batch, const PckCheckBatch& ride, hipStream_t stream) {
  const int64_t groups = plan_groups(batch, static_cast<int64_t>(R) * kWavesPerGroup);
  const int64_t total = groups + ride.start[ride.count];
  if (total * kGroupThreads > 0xFFFFFFFFll) return hipErrorInvalidValue;  // 32-bit dispatch size
  gemv_ride_kernel<256, R, U, kFp8, kPad, kNt>
      <<<dim3(static_cast<unsigned>(total)), dim3(kGroupThreads), 0, stream>>>(batch, ride);
  return hipGetLastError();
}

// The carried-check launch uses the built-in shape of the T = 256 vector path for long rows
// (choose_shape's), the launches a layer's checks ride in.
template <bool kFp8>
hipError_t launch_ride(GemvBatch& batch, bool pad, int64_t per_lane, const PckCheckBatch& ride,
                       hipStream_t stream) {
  if constexpr (kFp8) {
    (void)per_lane;
    return pad ? launch_ride_shape<2, 1, true, true>(batch, ride, stream)
               : launch_ride_shape<2, 1, true, false>(batch, ride, stream);
  } else {
    if (per_lane > 2) {
      return pad ? launch_ride_shape<2, 2, false, true>(batch, ride, stream)
                 : launch_ride_shape<2, 2, false, false>(batch, ride, stream);
    }
    return pad ? launch_ride_shape<1, 2, false, true>(batch, ride, stream)
               : launch_ride_shape<1, 2, false, false>(batch, ride, stream);
  }
}

// The launch plan of a group: validated items, whether every row takes 16-byte vectors, whether
// any chain has padding vectors, the longest chain and the total rows.
struct GroupPlan {
  GemvBatch batch{};
  bool vector = true;
  bool pad = false;
  int64_t max_per_lane = 1;
  int64_t rows = 0;
};

template <bool kFp8>
hipError_t plan_group(const PckGemv* gemvs, double* const* sums, int count, int threads,
                      GroupPlan& plan, const float* const* scales = nullptr,
                      float* const* scaled = nullptr) {
  constexpr int V = kFp8 ? 16 : 8;
  if (count < 1 || count > PCK_MAX_GROUP || gemvs == nullptr) return hipErrorInvalidValue;
  if (threads < kWarp || threads > 1024 || (threads & (threads - 1)) != 0)
    return hipErrorInvalidValue;
  plan.batch.count = count;
  for (int g = 0; g < count; ++g) {
    const PckGemv& d = gemvs[g];
    if (d.m < 0 || d.m > 0x7FFFFFFF || (d.m > 0 && (d.n < 1 || !d.W || !d.x || !d.y)))
      return hipErrorInvalidValue;
    double* rs = sums != nullptr ? sums[g] : nullptr;
    if (sums != nullptr && d.m > 0 && (rs == nullptr || reinterpret_cast<uintptr_t>(rs) % 16 != 0))
      return hipErrorInvalidValue;
    const int64_t n = d.m > 0 ? d.n : 1;
    const int64_t per_lane = ((n + V - 1) / V + threads - 1) / threads;
    plan.batch.item[g] =
        GemvItem{d.W, static_cast<const uint16_t*>(d.x), d.y, rs, d.m, n, per_lane};
    if (scaled != nullptr && d.m > 0) {
      if (scales == nullptr || scales[g] == nullptr || scaled[g] == nullptr)
        return hipErrorInvalidValue;
      plan.batch.item[g].scale = scales[g];
      plan.batch.item[g].y_scaled = scaled[g];
    }
    plan.rows += d.m;
    if (d.m > 0) {
      plan.vector = plan.vector && n % V == 0 && reinterpret_cast<uintptr_t>(d.W) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d.x) % 16 == 0;
      plan.max_per_lane = per_lane > plan.max_per_lane ? per_lane : plan.max_per_lane;
      plan.pad = plan.pad || n % (static_cast<int64_t>(threads) * V) != 0;
    }
  }
  return hipSuccess;
}

template <bool kFp8>
hipError_t launch_group(const PckGemv* gemvs, int count, int threads, const PckCheckBatch* ride,
                        hipStream_t stream, const float* const* scales = nullptr,
                        float* const* scaled = nullptr) {
  GroupPlan plan;
  if (plan_group<kFp8>(gemvs, nullptr, count, threads, plan, scales, scaled) != hipSuccess)
    return hipErrorInvalidValue;
  GemvBatch& batch = plan.batch;
  const bool vector = plan.vector, pad = plan.pad;
  const int64_t max_per_lane = plan.max_per_lane;
  if (ride != nullptr) {
    if (check::validate(*ride) != hipSuccess) return hipErrorInvalidValue;
    if (threads == 256 && vector) {
      bool any_rows = false;
      for (int g = 0; g < count; ++g) any_rows = any_rows || batch.item[g].m > 0;
      if (any_rows) return launch_ride<kFp8>(batch, pad, max_per_lane, *ride, stream);
    }
    // Other configurations: the same check as its own launch first (identical results).
    const int64_t items = ride->start[ride->count];
    if (items * check::kThreads > 0xFFFFFFFFll) return hipErrorInvalidValue;
    const int err = pck_blocked_check(ride, stream);
    if (err != 0) return static_cast<hipError_t>(err);
  }
  const TreeShape shape = choose_shape(max_per_lane, plan.rows, kFp8);
  switch (threads) {
    case 32: return launch_for_threads<32, kFp8>(batch, vector, pad, shape, stream);
    case 64: return launch_for_threads<64, kFp8>(batch, vector, pad, shape, stream);
    case 128: return launch_for_threads<128, kFp8>(batch, vector, pad, shape, stream);
    case 256: return launch_for_threads<256, kFp8>(batch, vector, pad, shape, stream);
    case 512: return launch_for_threads<512, kFp8>(batch, vector, pad, shape, stream);
    default: return launch_for_threads<1024, kFp8>(batch, vector, pad, shape, stream);
  }
}

// Launch shape of the in-pass kernel (pck_gemv_set_shape overrides it as for the plain tree).
TreeShape choose_rowsum_shape(int64_t per_lane, int64_t rows, bool fp8) {
  return choose_shape(per_lane, rows, fp8);
}

template <bool kFp8>
hipError_t launch_group_rowsums(const PckGemv* gemvs, double* const* sums, int count, int threads,
                                const PckRowSumBatch* ride, hipStream_t stream) {
  if (sums == nullptr) return hipErrorInvalidValue;
  GroupPlan plan;
  if (plan_group<kFp8>(gemvs, sums, count, threads, plan) != hipSuccess)
    return hipErrorInvalidValue;
  PckRowSumBatch none{};
  const PckRowSumBatch* rs = ride != nullptr ? ride : &none;
  if (rowsum::validate(*rs) != hipSuccess) return hipErrorInvalidValue;
  GemvBatch& b = plan.batch;
  const TreeShape shape = choose_rowsum_shape(plan.max_per_lane, plan.rows, kFp8);
  const bool v = plan.vector, p = plan.pad;

  switch (threads) {
    case 32: return launch_for_threads<32, kFp8, true>(b, v, p, shape, stream, rs);
    case 64: return launch_for_threads<64, kFp8, true>(b, v, p, shape, stream, rs);
    case 128: return launch_for_threads<128, kFp8, true>(b, v, p, shape, stream, rs);
    case 256: return launch_for_threads<256, kFp8, true>(b, v, p, shape, stream, rs);
    case 512: return launch_for_threads<512, kFp8, true>(b, v, p, shape, stream, rs);
    default: return launch_for_threads<1024, kFp8, true>(b, v, p, shape, stream, rs);
  }
}

}  // namespace
}  // namespace pck

extern "C" {

int pck_gemv_bf16_coalesced(const void* W, const void* x, float* y, int64_t m, int64_t n,
                            int threads, void* stream) {
  const PckGemv one{W, x, y, m, n};
  return pck::launch_group<false>(&one, 1, threads, nullptr, static_cast<hipStream_t>(stream));
}

int pck_gemv_fp8_coalesced(const void* Q, const void* x, float* z, int64_t m, int64_t n,
                           int threads, void* stream) {
  const PckGemv one{Q, x, z, m, n};
  return pck::launch_group<true>(&one, 1, threads, nullptr, static_cast<hipStream_t>(stream));
}

int pck_gemv_group_check(int weight_kind, const PckGemv* gemvs, int count, int threads,
                         const PckCheckBatch* ride, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (weight_kind == 0) return pck::launch_group<false>(gemvs, count, threads, ride, s);
  if (weight_kind == 1) return pck::launch_group<true>(gemvs, count, threads, ride, s);
  return hipErrorInvalidValue;
}

int pck_gemv_group_rowsums(int weight_kind, const PckGemv* gemvs, double* const* sums, int count,
                           int threads, const PckRowSumBatch* ride, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (weight_kind == 0) return pck::launch_group_rowsums<false>(gemvs, sums, count, threads, ride, s);
  if (weight_kind == 1) return pck::launch_group_rowsums<true>(gemvs, sums, count, threads, ride, s);
  return hipErrorInvalidValue;
}

int pck_gemv_group(int weight_kind, const PckGemv* gemvs, int count, int threads, void* stream) {
  return pck_gemv_group_check(weight_kind, gemvs, count, threads, nullptr, stream);
}

int pck_gemv_group_fp8_scaled(const PckGemv* gemvs, const float* const* scales,
                              float* const* scaled, int count, int threads,
                              const PckCheckBatch* ride, void* stream) {
  if (scales == nullptr || scaled == nullptr) return hipErrorInvalidValue;
  return pck::launch_group<true>(gemvs, count, threads, ride, static_cast<hipStream_t>(stream),
                                 scales, scaled);
}

int pck_gemv_bf16_naive(const void* W, const void* x, float* y, int64_t m, int64_t n, int threads,
                        void* stream) {
  if (threads < 1 || threads > 1024 || (threads & (threads - 1)) != 0) return hipErrorInvalidValue;
  const int64_t lanes = threads < 64 ? 64 : threads;  // workgroup size of the launch
  if (m < 0 || m > 0x7FFFFFFF || m * lanes > 0xFFFFFFFFll) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (n < 1 || !W || !x || !y) return hipErrorInvalidValue;
  const int64_t chunk = (n + threads - 1) / threads;
  const bool vector = chunk % 8 == 0 && n % 8 == 0 && reinterpret_cast<uintptr_t>(W) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(x) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(m)), group(static_cast<unsigned>(lanes));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* w16 = static_cast<const uint16_t*>(W);
  const auto* x16 = static_cast<const uint16_t*>(x);
  if (vector)
    pck::gemv_naive_kernel<true><<<grid, group, 0, s>>>(w16, x16, y, n, chunk, threads);
  else
    pck::gemv_naive_kernel<false><<<grid, group, 0, s>>>(w16, x16, y, n, chunk, threads);
  return hipGetLastError();
}

int pck_gemv_set_shape(int rows_per_wave, int unroll, int nontemporal) {
  if (rows_per_wave < 0 || rows_per_wave > 4 || rows_per_wave == 3 || unroll < 0 || unroll > 4 ||
      (rows_per_wave > 0 && unroll < 1))
    return hipErrorInvalidValue;
  pck::g_shape_override = pck::TreeShape{rows_per_wave, unroll, nontemporal != 0};
  return hipSuccess;
}

const char* pck_error_string(int err) { return hipGetErrorString(static_cast<hipError_t>(err)); }

}  // extern "C"
