// Set-sampling checker: checks that a sampler's selected set is a valid top-k set, or a valid
// minimal top-p nucleus, of each row of FP32 logits.  The GPU form of the CPU checker
// (reference src/pck/sampling.py:91-122); the reference's kernel is
// src/pck/cuda/csrc/sampling_kernel.cu:38-229.
//
// For row b with selection sel[b, 0 .. len[b]) over V logits:
//   top-k passes iff the selection is well formed (every index in range, none twice, length k),
//     no logit is NaN and min(selected) >= max(rejected) (-inf when nothing is rejected);
//   top-p also needs mass >= p - slack and mass_without_smallest < p + slack, where
//     mass = sum_sel e / sum_all e and mass_without_smallest drops e of the smallest selected
//     logit, e = exp((l - M) / T), M the row maximum.  `slack` comes from the host: the
//     sampler's declared error plus the bound below for this kernel's own rounding.
// min(selected) and max(rejected) are exact (FP32 comparisons).  Each e is FP32 expf on the
// split argument d = (l - m) / T = hi + lo (d in FP64, hi = fp32(d), lo = fp32(d - hi)):
// e = fma(expf(hi), lo, expf(hi)), within a few FP32 ulps of e^d for every |d| (an FP32
// argument alone would lose |d| ulps), 0 for d < -128 (masked -inf logits among them); the
// sums are FP64.
//
// Launches on the caller's stream; nothing depends on scheduling:
//   mark:    (selections longer than kLdsSelect only) one lane per selected entry sets its bit
//            in the row's bitmap (caller-zeroed scratch) with a device-scope atomic OR.  An
//            index out of range, or one whose bit was already set, marks the row malformed (a
//            plain store of 1 to the row's flag).
//   segment: a workgroup per (row, segment of ceil(V / S) logits).  For selections of at most
//            kLdsSelect entries it first builds its segment's bitmap in LDS from the selection
//            itself (LDS atomic OR: a bit already set is a duplicate; segment 0 also flags
//            indices out of range), so those calls need no scratch and no mark launch.  It then
//            forms the exact min over the selected, max over the rejected and over all logits,
//            a NaN flag and, for top-p, the FP64 sums of e^((l - m_s) / T) over all and over
//            the selected logits relative to the segment's own maximum m_s, in a fixed order
//            (lane, then wave butterfly, then waves in order).
//   finish:  a wave per row; lane i merges segments i, i + 64, ... in order (M = max m_s,
//            z_s e^((m_s - M) / T) with FP64 exp, multiply and add), the lanes meet in a fixed
//            butterfly, and lane 0 decides.
// The reference merges in the last segment to finish through an atomic ticket; here a third
// launch does it, so no workgroup waits on another's writes across the per-XCD L2 caches.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "pck_hip.h"

namespace pck {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kAhead = 8;  // logits in flight per lane
constexpr int64_t kLdsSelect = 4096;      // selections up to this length are read per segment
constexpr int64_t kLdsBits = 1 << 18;     // the largest segment bitmap kept in LDS (32 KiB)
constexpr uint32_t kNanFlag = 1u, kMalformedFlag = 2u;

struct Partial {
  float min_sel, max_rej, max_all;
  uint32_t flags;  // kNanFlag, kMalformedFlag
  double z, z_sel;
};
static_assert(sizeof(Partial) == 32, "partial layout");

struct Args {
  const float* logits;
  const int64_t* sel;
  const int64_t* len;  // (rows,), or NULL: every row is max_len long
  int64_t rows, vocab, max_len, k;
  int top_p;
  double p, temperature, slack;
  int64_t segments, seg_len, words;
  uint32_t* bitmap;  // (rows, words); unused when the selection bitmap is built in LDS
  uint32_t* flags;   // (rows,): nonzero = malformed
  Partial* partials; // (rows, segments)
  uint8_t* passed;
  float* min_sel;
  float* max_rej;
  double* mass;
  double* without;
};

// The selection length of a row (every row is max_len long without a lengths array).
__device__ __forceinline__ int64_t row_length(const Args& a, int64_t row) {
  return a.len ? a.len[row] : a.max_len;
}

__global__ void __launch_bounds__(kThreads) mark_kernel(const Args a) {
  const int64_t row = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t n = row_length(a, row) < a.max_len ? row_length(a, row) : a.max_len;
  if (i >= n) return;
  const int64_t idx = a.sel[row * a.max_len + i];
  if (idx < 0 || idx >= a.vocab) {
    a.flags[row] = 1u;
    return;
  }
  const uint32_t bit = 1u << (idx & 31);
  if (atomicOr(&a.bitmap[row * a.words + (idx >> 5)], bit) & bit) a.flags[row] = 1u;
}

__device__ __forceinline__ bool selected(const uint32_t* bits, int64_t j) {
  return (bits[j >> 5] >> (j & 31)) & 1u;
}

// Builds the segment's selection bitmap in LDS from the row's selection (bit j - j0 for index
// j in [j0, j1)); returns this lane's malformed finding (a duplicate in the segment, or, in
// segment 0, an index out of range).
__device__ bool build_lds_bitmap(const Args& a, int64_t row, int64_t seg, int64_t j0,
                                 int64_t j1, uint32_t* lds) {
  const int t = static_cast<int>(threadIdx.x);
  const int64_t words = (j1 - j0 + 31) / 32;
  for (int64_t w = t; w < words; w += kThreads) lds[w] = 0u;
  __syncthreads();
  const int64_t n = row_length(a, row) < a.max_len ? row_length(a, row) : a.max_len;
  const int64_t* sel = a.sel + row * a.max_len;
  bool bad = false;
  // kAhead entries per lane in flight; an entry past the end reads the last one (never used)
  for (int64_t i0 = t; i0 < n; i0 += kAhead * kThreads) {
    int64_t v[kAhead];
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      const int64_t i = i0 + static_cast<int64_t>(e) * kThreads;
      v[e] = sel[i < n ? i : n - 1];
    }
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      if (i0 + static_cast<int64_t>(e) * kThreads >= n) break;
      const int64_t idx = v[e];
      if (idx < 0 || idx >= a.vocab) {
        bad |= seg == 0;
      } else if (idx >= j0 && idx < j1) {
        const int64_t off = idx - j0;
        const uint32_t bit = 1u << (off & 31);
        bad |= (atomicOr(&lds[off >> 5], bit) & bit) != 0u;
      }
    }
  }
  __syncthreads();
  return bad;
}

// e^d for d = (l - m) / T formed in FP64: FP32 expf of the rounded argument, corrected by the
// argument's rounding error lo (e^(hi + lo) = e^hi (1 + lo + ...), |lo| <= 2^-24 |hi|).
__device__ __forceinline__ double term(float l, double m, double temperature) {
  const double d = (static_cast<double>(l) - m) / temperature;
  if (!(d >= -128.0)) return 0.0;  // below e^-128 (and -inf logits); NaN is flagged elsewhere
  const float hi = static_cast<float>(d);
  const float lo = static_cast<float>(d - static_cast<double>(hi));
  const float eh = expf(hi);
  return static_cast<double>(__builtin_fmaf(eh, lo, eh));
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v = fminf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// The same bits on every lane: at each level both partners add the same two values.
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v = v + __shfl_xor(v, o, kWave);
  return v;
}

template <bool kLds>
__global__ void __launch_bounds__(kThreads) segment_kernel(const Args a) {
  extern __shared__ uint32_t lds_bits[];  // kLds: the segment's bitmap
  __shared__ float fred[3][kWaves];
  __shared__ double dred[2][kWaves];
  __shared__ uint32_t any_flag;
  const int t = static_cast<int>(threadIdx.x);
  const int wave = t / kWave, lane = t % kWave;
  const int64_t row = blockIdx.y, seg = blockIdx.x;
  const float* l = a.logits + row * a.vocab;
  const int64_t j0 = seg * a.seg_len < a.vocab ? seg * a.seg_len : a.vocab;
  const int64_t j1 = j0 + a.seg_len < a.vocab ? j0 + a.seg_len : a.vocab;
  if (t == 0) any_flag = 0u;
  bool malformed = false;
  if constexpr (kLds) malformed = build_lds_bitmap(a, row, seg, j0, j1, lds_bits);
  // bit of logit j: kLds, bit j - j0 of the LDS bitmap; else bit j of the row's bitmap
  const uint32_t* bits = kLds ? lds_bits : a.bitmap + row * a.words;
  const int64_t base = kLds ? j0 : 0;

  float mn = INFINITY, mx_rej = -INFINITY, mx = -INFINITY;
  bool nan = false;
  for (int64_t jb = j0 + t; jb < j1; jb += kAhead * kThreads) {
    float x[kAhead];
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      const int64_t j = jb + static_cast<int64_t>(e) * kThreads;
      x[e] = l[j < j1 ? j : j1 - 1];  // past the segment: a valid address, never used
    }
#pragma unroll
    for (int e = 0; e < kAhead; ++e) {
      const int64_t j = jb + static_cast<int64_t>(e) * kThreads;
      if (j >= j1) break;
      nan |= x[e] != x[e];
      mx = fmaxf(mx, x[e]);
      if (selected(bits, j - base)) mn = fminf(mn, x[e]);
      else mx_rej = fmaxf(mx_rej, x[e]);
    }
  }
  mn = wave_min(mn);
  mx_rej = wave_max(mx_rej);
  mx = wave_max(mx);
  const bool wave_nan = __any(nan);
  const bool wave_bad = __any(malformed);
  __syncthreads();  // any_flag is cleared before any wave sets it
  if (lane == 0) {
    fred[0][wave] = mn;
    fred[1][wave] = mx_rej;
    fred[2][wave] = mx;
    if (wave_nan) atomicOr(&any_flag, kNanFlag);
    if (wave_bad) atomicOr(&any_flag, kMalformedFlag);
  }
  __syncthreads();
  mn = fred[0][0], mx_rej = fred[1][0], mx = fred[2][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    mn = fminf(mn, fred[0][w]);
    mx_rej = fmaxf(mx_rej, fred[1][w]);
    mx = fmaxf(mx, fred[2][w]);
  }

  double z = 0.0, z_sel = 0.0;
  if (a.top_p && mx > -INFINITY) {  // uniform
    const double m = static_cast<double>(mx);
    for (int64_t jb = j0 + t; jb < j1; jb += kAhead * kThreads) {
      float x[kAhead];
#pragma unroll
      for (int e = 0; e < kAhead; ++e) {
        const int64_t j = jb + static_cast<int64_t>(e) * kThreads;
        x[e] = l[j < j1 ? j : j1 - 1];  // past the segment: a valid address, never used
      }
#pragma unroll
      for (int e = 0; e < kAhead; ++e) {
        const int64_t j = jb + static_cast<int64_t>(e) * kThreads;
        if (j >= j1) break;
        const double v = term(x[e], m, a.temperature);
        z = z + v;
        if (selected(bits, j - base)) z_sel = z_sel + v;
      }
    }
    z = wave_sum(z);
    z_sel = wave_sum(z_sel);
    if (lane == 0) {
      dred[0][wave] = z;
      dred[1][wave] = z_sel;
    }
    __syncthreads();
    z = (dred[0][0] + dred[0][1]) + (dred[0][2] + dred[0][3]);
    z_sel = (dred[1][0] + dred[1][1]) + (dred[1][2] + dred[1][3]);
  }
  if (t == 0) a.partials[row * a.segments + seg] = Partial{mn, mx_rej, mx, any_flag, z, z_sel};
}

__global__ void __launch_bounds__(kThreads) finish_kernel(const Args a, int lds_select) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  if (row >= a.rows) return;  // whole waves
  const Partial* ps = a.partials + row * a.segments;
  float min_sel = INFINITY, max_rej = -INFINITY, mx = -INFINITY;
  uint32_t flags = 0u;
  for (int64_t s = lane; s < a.segments; s += kWave) {
    min_sel = fminf(min_sel, ps[s].min_sel);
    max_rej = fmaxf(max_rej, ps[s].max_rej);
    mx = fmaxf(mx, ps[s].max_all);
    flags |= ps[s].flags;
  }
  min_sel = wave_min(min_sel);
  max_rej = wave_max(max_rej);
  mx = wave_max(mx);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) flags |= __shfl_xor(flags, o, kWave);
  const int64_t n_sel = row_length(a, row);
  const bool malformed = lds_select ? (flags & kMalformedFlag) != 0u : a.flags[row] != 0u;
  const bool well_formed = !malformed && n_sel >= 1 && n_sel <= a.max_len && n_sel <= a.vocab &&
                           (a.top_p || n_sel == a.k);
  bool ok = well_formed && (flags & kNanFlag) == 0u && min_sel >= max_rej;
  double mass = 0.0, without = 0.0;
  if (a.top_p && ok) {  // uniform over the wave
    const double big_m = static_cast<double>(mx);
    double big_z = 0.0, big_z_sel = 0.0;
    for (int64_t s = lane; s < a.segments; s += kWave) {  // this lane's segments in order
      if (ps[s].max_all > -INFINITY) {
        const double scale = exp((static_cast<double>(ps[s].max_all) - big_m) / a.temperature);
        big_z = big_z + ps[s].z * scale;
        big_z_sel = big_z_sel + ps[s].z_sel * scale;
      }
    }
    big_z = wave_sum(big_z);
    big_z_sel = wave_sum(big_z_sel);
    const double e_min = exp((static_cast<double>(min_sel) - big_m) / a.temperature);
    mass = big_z_sel / big_z;
    without = (big_z_sel - e_min) / big_z;
    ok = mass >= a.p - a.slack && without < a.p + a.slack;
  }
  if (lane != 0) return;
  a.passed[row] = ok ? 1u : 0u;
  a.min_sel[row] = min_sel;
  a.max_rej[row] = max_rej;
  a.mass[row] = mass;
  a.without[row] = without;
}

}  // namespace
}  // namespace pck

extern "C" int pck_sampling_needs_scratch(int64_t vocab, int64_t max_len, int64_t segments) {
  if (vocab < 1 || max_len < 1 || segments < 1 || segments > vocab) return -1;
  const int64_t seg_len = (vocab + segments - 1) / segments;
  return max_len <= pck::kLdsSelect && seg_len <= pck::kLdsBits ? 0 : 1;
}

extern "C" int64_t pck_sampling_scratch_words(int64_t vocab) {
  return vocab < 1 ? -1 : (vocab + 31) / 32 + 1;
}

extern "C" int64_t pck_sampling_partial_bytes(void) {
  return static_cast<int64_t>(sizeof(pck::Partial));
}

extern "C" int pck_sampling_check(const float* logits, const int64_t* selected,
                                  const int64_t* lengths, int64_t rows, int64_t vocab,
                                  int64_t max_len, int64_t k, int top_p, double p,
                                  double temperature, double slack, int64_t segments,
                                  uint32_t* scratch, void* partials, uint8_t* passed,
                                  float* min_selected, float* max_rejected, double* mass,
                                  double* mass_without_smallest, void* stream) {
  using namespace pck;
  const int64_t seg_len = (vocab + segments - 1) / segments;
  const bool lds_select = max_len <= kLdsSelect && seg_len <= kLdsBits;
  if (!logits || !selected || (!scratch && !lds_select) || !partials || !passed ||
      !min_selected ||
      !max_rejected || !mass || !mass_without_smallest || rows < 1 || rows > 65535 ||
      vocab < 1 || max_len < 1 || segments < 1 || segments > vocab ||
      segments > 0x7FFFFFFF || !(temperature > 0.0) || !(slack >= 0.0) ||
      (max_len + kThreads - 1) / kThreads > 0x7FFFFFFF ||
      reinterpret_cast<uintptr_t>(partials) % 8 != 0)
    return hipErrorInvalidValue;
  Args a{};
  a.logits = logits;
  a.sel = selected;
  a.len = lengths;
  a.rows = rows;
  a.vocab = vocab;
  a.max_len = max_len;
  a.k = k;
  a.top_p = top_p != 0;
  a.p = p;
  a.temperature = temperature;
  a.slack = slack;
  a.segments = segments;
  a.seg_len = seg_len;
  a.words = (vocab + 31) / 32;
  a.bitmap = scratch;
  a.flags = scratch ? scratch + rows * a.words : nullptr;
  a.partials = static_cast<Partial*>(partials);
  a.passed = passed;
  a.min_sel = min_selected;
  a.max_rej = max_rejected;
  a.mass = mass;
  a.without = mass_without_smallest;
  auto s = static_cast<hipStream_t>(stream);
  const dim3 seg_grid(static_cast<unsigned>(segments), static_cast<unsigned>(rows));
  hipError_t err;
  if (lds_select) {
    const size_t lds = static_cast<size_t>((seg_len + 31) / 32) * sizeof(uint32_t);
    segment_kernel<true><<<seg_grid, dim3(kThreads), lds, s>>>(a);
  } else {
    const dim3 mark_grid(static_cast<unsigned>((max_len + kThreads - 1) / kThreads),
                         static_cast<unsigned>(rows));
    mark_kernel<<<mark_grid, dim3(kThreads), 0, s>>>(a);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    segment_kernel<false><<<seg_grid, dim3(kThreads), 0, s>>>(a);
  }
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  finish_kernel<<<dim3(static_cast<unsigned>((rows + kWaves - 1) / kWaves)), dim3(kThreads), 0,
                  s>>>(a, lds_select ? 1 : 0);
  return hipGetLastError();
}
