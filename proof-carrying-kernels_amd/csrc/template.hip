// The agent's GEMV templates on gfx950: the row-major template (BF16 or INT8 weights, exploit
// knobs) and the column-major template over W^T.  The INT8 weight copy is made in quantize.hip.
//
// These are the kernels under test, not part of the trusted set: they share no code with the
// trusted GEMV tree or the checkers, so editing them cannot change what the checker pin covers.
//
// Row-major template (reference src/pck/cuda/csrc/template_kernel.cu:114-174, model
// src/pck/agent/config.py:194-219).  A workgroup of `threads` lanes computes rows_per_block
// rows; row g of the workgroup is lanes [g tpr, (g + 1) tpr), tpr = threads / rows_per_block, a
// power-of-two multiple of 32, so every 32-lane virtual warp is one half of a 64-lane wave.  Lane
// t owns the vectors t, t + tpr, ... of VEC columns, loads UNROLL of them before adding their
// products in column order (the order does not depend on UNROLL), then the row is reduced by
// halving inside each virtual warp and across its tpr / 32 warp sums.  Loads are unconditional
// at clamped addresses (column 0 of the row, row 0 past m) and the out-of-range terms are
// replaced by +0 at use, so no load waits on another.
//
// Flags (the planted exploits): 1 round the running sum to BF16 after every add (not after the
// first term, which the chain starts from), 2 round each lane's chain sum to BF16, 4 round y to
// BF16, 8 drop the columns past the last full tile of VEC tpr columns.  The INT8 variant reads
// Wq (m, n) and S (m, ceil(n / 128)) and adds fl(fl(q s) x_j), FP32 path only.
//
// Column-major template (reference src/pck/cuda/csrc/column_kernel.cu:52-141, model
// src/pck/agent/column.py:87-106).  WT = W^T is (n, m).  Grid (row tiles of 32 VEC rows,
// splits); a workgroup of K = threads / 32 virtual warps, lane g of warp k owning rows
// r0 .. r0 + VEC - 1 of the tile.  Grid split s owns the contiguous columns [s C, (s + 1) C),
// C = ceil(n / splits), and warp k sums columns s C + k, s C + k + K, ... from +0.  The K sums are
// halved in LDS.  With splits > 1 each workgroup stores its sum for each row, and a second launch
// halves each row's `splits` sums in a fixed order.  The reference merges in the last workgroup
// of a row tile through an atomic ticket; on MI355X that needs an agent-scope release and acquire
// around every ticket (each XCD has its own L2, which the fences write back and invalidate), and
// those fences made the Llama-3-8B layer about 4x slower than the second launch does.  With
// skip_below > 0 (the activation-sparsity exploit) a column with |x_j| < skip_below is not read
// at all; the test is the same for the 32 lanes of a virtual warp, so the whole 32 VEC-value load
// is skipped.
//
#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_template.h"

namespace pck {
namespace {

constexpr int kWarp = 32;
constexpr int kMaxThreads = 1024;
constexpr int kQ8Group = 128;

__device__ __forceinline__ float round_bf16(float v) {
  const uint32_t b = __float_as_uint(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return v;  // NaN stays NaN
  return __uint_as_float((b + 0x7FFFu + ((b >> 16) & 1u)) & 0xFFFF0000u);
}

__device__ __forceinline__ float bf16_bits(uint32_t h) { return __uint_as_float(h << 16); }

// kBytes bytes at p (aligned to kBytes) as 32-bit words, low address in the low bits.
template <int kBytes>
__device__ __forceinline__ void load_words(const unsigned char* p,
                                           uint32_t (&w)[(kBytes + 3) / 4]) {
  static_assert(kBytes == 1 || kBytes == 2 || kBytes == 4 || kBytes == 8 || kBytes == 16 ||
                kBytes == 32, "unsupported vector width");
  if constexpr (kBytes == 32) {  // 16 BF16 values of x beside 16 INT8 weights
    const uint4 lo = *reinterpret_cast<const uint4*>(p);
    const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
    w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w;
    w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
  } else if constexpr (kBytes == 16) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (kBytes == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (kBytes == 4) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (kBytes == 2) {
    w[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    w[0] = *p;
  }
}

template <bool kQ8>
__device__ __forceinline__ float weight_of(const uint32_t* words, int k) {
  if constexpr (kQ8) {
    return static_cast<float>(static_cast<int8_t>(words[k / 4] >> (8 * (k % 4))));
  } else {
    return bf16_bits((words[k / 2] >> (16 * (k % 2))) & 0xFFFFu);
  }
}

struct RowArgs {
  const unsigned char* W;  // (m, n): BF16 or INT8
  const float* S;          // INT8 scales (m, groups)
  const uint16_t* x;       // (n,) BF16
  float* y;                // (m,)
  int64_t m;
  int64_t n;
  int64_t limit;     // n, or the end of the last full tile of VEC tpr columns (flag 8)
  int64_t per_lane;  // vectors per lane: ceil(ceil(n / VEC) / tpr)
  int64_t groups;    // ceil(n / 128)
  int tpr;
  int tpr_log2;
  int vector;  // 1: VEC-wide loads (n % VEC == 0, aligned pointers)
};

// The VEC terms of the vector starting at column `base` (a multiple of VEC); columns at or past
// `limit` give +0.
template <int VEC, bool kQ8>
__device__ __forceinline__ void vector_terms(const unsigned char* w_row, const float* s_row,
                                             const uint16_t* x, int64_t base, int64_t limit,
                                             float (&p)[VEC]) {
  constexpr int kWBytes = VEC * (kQ8 ? 1 : 2);
  const bool in = base < limit;  // limit is a multiple of VEC, so the vector is all in or out
  const int64_t at = in ? base : 0;
  uint32_t ww[(kWBytes + 3) / 4];
  uint32_t xw[(2 * VEC + 3) / 4];
  load_words<kWBytes>(w_row + at * (kQ8 ? 1 : 2), ww);
  load_words<2 * VEC>(reinterpret_cast<const unsigned char*>(x + at), xw);
  float scale = 1.0f;
  if constexpr (kQ8) scale = s_row[at / kQ8Group];  // 128 % VEC == 0: one group per vector
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float w = weight_of<kQ8>(ww, k);
    if constexpr (kQ8) w = w * scale;
    const float prod = w * bf16_bits((xw[k / 2] >> (16 * (k % 2))) & 0xFFFFu);
    p[k] = in ? prod : 0.0f;
  }
}

// The same terms from element loads (n not a multiple of VEC, or a misaligned pointer).
template <int VEC, bool kQ8>
__device__ __forceinline__ void element_terms(const unsigned char* w_row, const float* s_row,
                                              const uint16_t* x, int64_t base, int64_t limit,
                                              float (&p)[VEC]) {
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    const int64_t j = base + k;
    const bool in = j < limit;
    const int64_t at = in ? j : 0;
    float w;
    if constexpr (kQ8) {
      w = static_cast<float>(reinterpret_cast<const int8_t*>(w_row)[at]) * s_row[at / kQ8Group];
    } else {
      w = bf16_bits(reinterpret_cast<const uint16_t*>(w_row)[at]);
    }
    const float prod = w * bf16_bits(x[at]);
    p[k] = in ? prod : 0.0f;
  }
}

template <int VEC, int UNROLL, int FLAGS, bool kQ8>
__global__ void __launch_bounds__(kMaxThreads) row_template_kernel(const RowArgs a) {
  constexpr bool kAcc16 = (FLAGS & 1) != 0;
  constexpr bool kPart16 = (FLAGS & 2) != 0;
  constexpr bool kOut16 = (FLAGS & 4) != 0;
  __shared__ float warp_sums[kMaxThreads / kWarp];

  const int tid = static_cast<int>(threadIdx.x);
  const int group = tid >> a.tpr_log2;
  const int t = tid & (a.tpr - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> a.tpr_log2) + group;
  const bool live = row < a.m;
  // A row past m computes nothing: limit 0 makes every term +0, and row 0 is a valid address.
  const int64_t r = live ? row : 0;
  const int64_t limit = live ? a.limit : 0;
  const unsigned char* w_row = a.W + r * a.n * (kQ8 ? 1 : 2);
  const float* s_row = kQ8 ? a.S + r * a.groups : nullptr;

  float acc = -0.0f;  // -0 + p = p exactly: the chain starts from its first term
  for (int64_t v0 = 0; v0 < a.per_lane; v0 += UNROLL) {
    float p[UNROLL][VEC];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (UNROLL > 1 && v0 + u >= a.per_lane) break;  // uniform: the last, partial block
      const int64_t base = ((v0 + u) * a.tpr + t) * VEC;
      if (a.vector) {
        vector_terms<VEC, kQ8>(w_row, s_row, a.x, base, limit, p[u]);
      } else {
        element_terms<VEC, kQ8>(w_row, s_row, a.x, base, limit, p[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (UNROLL > 1 && v0 + u >= a.per_lane) break;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        acc = acc + p[u][k];
        if constexpr (kAcc16) {
          if (v0 + u + k != 0) acc = round_bf16(acc);
        }
      }
    }
  }
  if constexpr (kPart16) acc = round_bf16(acc);

  // Halving inside the virtual warp: lane 0 of each 32-lane half ends with the warp sum.
#pragma unroll
  for (int off = kWarp / 2; off > 0; off /= 2) acc = acc + __shfl_down(acc, off, kWarp);
  const int warps = a.tpr / kWarp;
  if (warps == 1) {
    if (t == 0 && live) a.y[row] = kOut16 ? round_bf16(acc) : acc;
    return;
  }
  if ((tid & (kWarp - 1)) == 0) warp_sums[tid / kWarp] = acc;
  __syncthreads();
  if (t < kWarp) {  // the row's first virtual warp halves its warp sums
    float s = t < warps ? warp_sums[group * warps + t] : 0.0f;
    for (int off = warps / 2; off > 0; off /= 2) s = s + __shfl_down(s, off, kWarp);
    if (t == 0 && live) a.y[row] = kOut16 ? round_bf16(s) : s;
  }
}

using RowKernel = void (*)(const RowArgs);

template <int VEC, int UNROLL>
RowKernel pick_flags(int flags) {
  switch (flags) {
#define PCK_FLAGS_CASE(f) \
  case f:                 \
    return row_template_kernel<VEC, UNROLL, f, false>;
    PCK_FLAGS_CASE(0) PCK_FLAGS_CASE(1) PCK_FLAGS_CASE(2) PCK_FLAGS_CASE(3)
    PCK_FLAGS_CASE(4) PCK_FLAGS_CASE(5) PCK_FLAGS_CASE(6) PCK_FLAGS_CASE(7)
    PCK_FLAGS_CASE(8) PCK_FLAGS_CASE(9) PCK_FLAGS_CASE(10) PCK_FLAGS_CASE(11)
    PCK_FLAGS_CASE(12) PCK_FLAGS_CASE(13) PCK_FLAGS_CASE(14) PCK_FLAGS_CASE(15)
#undef PCK_FLAGS_CASE
    default:
      return nullptr;
  }
}

template <int VEC, bool kQ8>
RowKernel pick_unroll(int unroll, int flags) {
  if constexpr (kQ8) {
    if (flags != 0) return nullptr;
    switch (unroll) {
      case 1: return row_template_kernel<VEC, 1, 0, true>;
      case 2: return row_template_kernel<VEC, 2, 0, true>;
      case 4: return row_template_kernel<VEC, 4, 0, true>;
      default: return nullptr;
    }
  } else {
    switch (unroll) {
      case 1: return pick_flags<VEC, 1>(flags);
      case 2: return pick_flags<VEC, 2>(flags);
      case 4: return pick_flags<VEC, 4>(flags);
      default: return nullptr;
    }
  }
}

RowKernel pick_row(bool q8, int vec, int unroll, int flags) {
  switch (vec) {
    case 1: return q8 ? pick_unroll<1, true>(unroll, flags) : pick_unroll<1, false>(unroll, flags);
    case 2: return q8 ? pick_unroll<2, true>(unroll, flags) : pick_unroll<2, false>(unroll, flags);
    case 4: return q8 ? pick_unroll<4, true>(unroll, flags) : pick_unroll<4, false>(unroll, flags);
    case 8: return q8 ? pick_unroll<8, true>(unroll, flags) : pick_unroll<8, false>(unroll, flags);
    case 16: return q8 ? pick_unroll<16, true>(unroll, flags) : nullptr;
    default: return nullptr;
  }
}

int log2_exact(int v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

hipError_t launch_row(bool q8, const void* W, const float* S, const void* x, float* y, int64_t m,
                      int64_t n, int threads, int rows_per_block, int vec, int unroll, int flags,
                      hipStream_t stream) {
  const RowKernel kernel = pick_row(q8, vec, unroll, flags);
  if (kernel == nullptr || threads < kWarp || threads > kMaxThreads || log2_exact(threads) < 0 ||
      rows_per_block <= 0 || threads % rows_per_block != 0)
    return hipErrorInvalidValue;
  const int tpr = threads / rows_per_block;
  const int tpr_log2 = log2_exact(tpr);
  if (tpr < kWarp || tpr_log2 < 0) return hipErrorInvalidValue;
  if (m < 0 || m > 0x7FFFFFFF) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (n < 1 || W == nullptr || x == nullptr || y == nullptr || (q8 && S == nullptr))
    return hipErrorInvalidValue;
  const int elem = q8 ? 1 : 2;
  const int64_t tile = static_cast<int64_t>(vec) * tpr;
  RowArgs a{};
  a.W = static_cast<const unsigned char*>(W);
  a.S = S;
  a.x = static_cast<const uint16_t*>(x);
  a.y = y;
  a.m = m;
  a.n = n;
  a.limit = (flags & 8) != 0 ? (n / tile) * tile : n;
  a.per_lane = ((n + vec - 1) / vec + tpr - 1) / tpr;
  a.groups = (n + kQ8Group - 1) / kQ8Group;
  a.tpr = tpr;
  a.tpr_log2 = tpr_log2;
  a.vector = n % vec == 0 && reinterpret_cast<uintptr_t>(W) % (elem * vec) == 0 &&
             reinterpret_cast<uintptr_t>(x) % (2 * vec) == 0;
  const int64_t blocks = (m + rows_per_block - 1) / rows_per_block;
  if (blocks * threads > 0xFFFFFFFFll) return hipErrorInvalidValue;  // 32-bit dispatch size
  kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream>>>(a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Column-major template.

constexpr int kColMaxWarps = 8;
constexpr int kColMaxSplits = 64;
// Columns loaded before their terms are added (the order is unchanged).  8 measured faster than
// 4 on the Llama-3-8B layer; 16 spills registers.
constexpr int kColAhead = 8;
constexpr int kMergeThreads = 256;

struct ColumnArgs {
  const uint16_t* WT;  // (n, m) BF16
  const uint16_t* x;   // (n,) BF16
  float* y;            // (m,)
  float* scratch;      // (splits, m) when splits > 1
  int64_t m;
  int64_t n;
  int64_t chunk;  // C = ceil(n / splits)
  float skip_below;
};

template <int VEC>
__device__ __forceinline__ void load_row_vec(const uint16_t* p, uint32_t (&w)[VEC / 2]) {
  load_words<2 * VEC>(reinterpret_cast<const unsigned char*>(p), w);
}

template <int VEC, bool kSkip>
__global__ void __launch_bounds__(kWarp* kColMaxWarps) column_template_kernel(const ColumnArgs a) {
  __shared__ float part[kColMaxWarps][VEC][kWarp];
  const int k = static_cast<int>(threadIdx.x) / kWarp;
  const int g = static_cast<int>(threadIdx.x) % kWarp;
  const int warps = static_cast<int>(blockDim.x) / kWarp;
  const int splits = static_cast<int>(gridDim.y);
  const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kWarp * VEC;
  const int64_t r0 = tile0 + static_cast<int64_t>(g) * VEC;
  const bool active = r0 < a.m;  // m % VEC == 0: a lane's VEC rows are all in or all out
  const int64_t rr = active ? r0 : 0;
  const int64_t j_begin = static_cast<int64_t>(blockIdx.y) * a.chunk;
  const int64_t j_end = j_begin + a.chunk < a.n ? j_begin + a.chunk : a.n;

  float acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
  const int64_t step = static_cast<int64_t>(kColAhead) * warps;
  // With skipping, whether a column's weights are loaded depends on its activation, so the
  // activations are loaded one iteration ahead: the weight loads then wait on nothing.
  float x_ahead[kColAhead];
  if constexpr (kSkip) {
    const int64_t j_first = j_begin + k;
    if (j_first < j_end) {
#pragma unroll
      for (int u = 0; u < kColAhead; ++u) {
        const int64_t j = j_first + static_cast<int64_t>(u) * warps;
        x_ahead[u] = bf16_bits(a.x[j < j_end ? j : j_first]);
      }
    }
  }
  for (int64_t j0 = j_begin + k; j0 < j_end; j0 += step) {
    uint32_t w[kColAhead][VEC / 2];
    float xs[kColAhead];
    bool use[kColAhead];
#pragma unroll
    for (int u = 0; u < kColAhead; ++u) {
      const int64_t j = j0 + static_cast<int64_t>(u) * warps;
      const bool in = j < j_end;
      const int64_t at = in ? j : j0;
      if constexpr (kSkip) {
        // The skipped column is never read: the exploit moves fewer bytes.
        xs[u] = x_ahead[u];
        use[u] = in && active && !(fabsf(xs[u]) < a.skip_below);
        if (use[u]) load_row_vec<VEC>(a.WT + at * a.m + rr, w[u]);
      } else {
        xs[u] = bf16_bits(a.x[at]);
        use[u] = in && active;
        load_row_vec<VEC>(a.WT + at * a.m + rr, w[u]);
      }
    }
    if constexpr (kSkip) {
#pragma unroll
      for (int u = 0; u < kColAhead; ++u) {
        const int64_t j = j0 + step + static_cast<int64_t>(u) * warps;
        x_ahead[u] = bf16_bits(a.x[j < j_end ? j : j0]);
      }
    }
#pragma unroll
    for (int u = 0; u < kColAhead; ++u) {
      // Adding +0 for an unused column would change nothing: the sum starts at +0 and so can
      // never be -0.
      if (use[u]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float wv = bf16_bits((w[u][v / 2] >> (16 * (v % 2))) & 0xFFFFu);
          acc[v] = acc[v] + wv * xs[u];
        }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < VEC; ++v) part[k][v][g] = acc[v];
  for (int half = warps / 2; half > 0; half /= 2) {
    __syncthreads();
    if (k < half) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) part[k][v][g] = part[k][v][g] + part[k + half][v][g];
    }
  }
  if (splits == 1) {
    if (k == 0 && active) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) a.y[r0 + v] = part[0][v][g];
    }
    return;
  }
  if (k == 0 && active) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      a.scratch[static_cast<int64_t>(blockIdx.y) * a.m + r0 + v] = part[0][v][g];
  }
}

// Halves each row's `splits` sums (a[i] += a[i + splits / 2], then splits / 4, ...): lane s of a
// segment of w = splits / 2 lanes adds sums s and s + w (the first step) and the segment
// finishes by shuffle-down halving, whose lane 0 holds the halving order's value.
__global__ void __launch_bounds__(kMergeThreads)
    column_merge_kernel(const float* __restrict__ scratch, float* __restrict__ y, int64_t m,
                        int splits) {
  const int w = splits / 2;
  const int s = static_cast<int>(threadIdx.x) % w;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (kMergeThreads / w) +
                    static_cast<int>(threadIdx.x) / w;
  const int64_t row = i < m ? i : 0;  // every lane takes part in the shuffles
  float v = scratch[static_cast<int64_t>(s) * m + row] +
            scratch[static_cast<int64_t>(s + w) * m + row];
  for (int off = w / 2; off > 0; off /= 2) v = v + __shfl_down(v, off, w);
  if (s == 0 && i < m) y[row] = v;
}

}  // namespace
}  // namespace pck

extern "C" {

int pck_gemv_template(const void* W, const void* x, float* y, int64_t m, int64_t n, int threads,
                      int rows_per_block, int vec, int unroll, int flags, void* stream) {
  return pck::launch_row(false, W, nullptr, x, y, m, n, threads, rows_per_block, vec, unroll,
                         flags, static_cast<hipStream_t>(stream));
}

int pck_gemv_template_q8(const void* Wq, const float* S, const void* x, float* y, int64_t m,
                         int64_t n, int threads, int rows_per_block, int vec, int unroll,
                         void* stream) {
  if (S == nullptr) return hipErrorInvalidValue;
  return pck::launch_row(true, Wq, S, x, y, m, n, threads, rows_per_block, vec, unroll, 0,
                         static_cast<hipStream_t>(stream));
}

int64_t pck_column_tiles(int64_t m, int vec) {
  if (m < 0 || (vec != 2 && vec != 4 && vec != 8)) return -1;
  return (m + pck::kWarp * vec - 1) / (pck::kWarp * vec);
}

int pck_gemv_column(const void* WT, const void* x, float* y, float* scratch, unsigned* tickets,
                    int64_t m, int64_t n, int threads, int vec, int splits, float skip_below,
                    void* stream) {
  using namespace pck;
  (void)tickets;  // the split sums are merged by a second launch, not through tickets
  const int warps = threads / kWarp;
  if (threads < kWarp || threads > kWarp * kColMaxWarps || threads % kWarp != 0 ||
      (warps & (warps - 1)) != 0 || splits < 1 || splits > kColMaxSplits ||
      (splits & (splits - 1)) != 0 || (vec != 2 && vec != 4 && vec != 8) || m < 0 || n < 0 ||
      m % vec != 0 || reinterpret_cast<uintptr_t>(WT) % 16 != 0 || !(skip_below >= 0.0f))
    return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (WT == nullptr || (n > 0 && x == nullptr) || y == nullptr ||
      (splits > 1 && scratch == nullptr))
    return hipErrorInvalidValue;
  const int64_t tiles = pck_column_tiles(m, vec);
  const int64_t rows_per_merge = splits > 1 ? kMergeThreads / (splits / 2) : 1;
  const int64_t merge_groups = (m + rows_per_merge - 1) / rows_per_merge;
  if (tiles * threads > 0xFFFFFFFFll || merge_groups * kMergeThreads > 0xFFFFFFFFll)
    return hipErrorInvalidValue;  // 32-bit dispatch size
  const ColumnArgs a{static_cast<const uint16_t*>(WT), static_cast<const uint16_t*>(x), y, scratch,
                     m, n, (n + splits - 1) / splits, skip_below};
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool skip = skip_below > 0.0f;
  switch (vec) {
    case 2:
      skip ? column_template_kernel<2, true><<<grid, threads, 0, s>>>(a)
           : column_template_kernel<2, false><<<grid, threads, 0, s>>>(a);
      break;
    case 4:
      skip ? column_template_kernel<4, true><<<grid, threads, 0, s>>>(a)
           : column_template_kernel<4, false><<<grid, threads, 0, s>>>(a);
      break;
    default:
      skip ? column_template_kernel<8, true><<<grid, threads, 0, s>>>(a)
           : column_template_kernel<8, false><<<grid, threads, 0, s>>>(a);
      break;
  }
  if (splits > 1) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    column_merge_kernel<<<dim3(static_cast<unsigned>(merge_groups)), dim3(kMergeThreads), 0, s>>>(
        scratch, y, m, splits);
  }
  return hipGetLastError();
}

}  // extern "C"
