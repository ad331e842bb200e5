// Sampled-token membership check (top-k / top-p / greedy) for a batch of rows, on gfx950.
//
// Semantics: reference src/pck/member.py:118-197 (`check_members`), per row with logits l,
// token t, k = top_k (vocab if none), p = top_p (1 if none):
//   above   = #{j : l_j > l_t}                                  exact FP32 compares
//   ok      = no NaN in l  and  0 <= t < vocab  and  above < (greedy ? 1 : k)
//   top-p   kept = {j : l_j >= kth} where kth is the k_eff-th largest logit, k_eff =
//           min(k, k_lim) (k_lim = largest host top-k below vocab: a stale host copy is
//           clamped, reference member.py:170,175); every logit is kept for a row without a
//           top-k, unless all_k (reference's top-(max k) path) says every row has one.
//           r = sum_{kept, l_j > l_t} e_j / sum_{kept} e_j with e_j the FP32 term
//           expf(hi) + expf(hi) lo of the exact split l_j - max = hi + lo (TwoSum), 0 when
//           hi < -128 (reference member.py:105-115), summed in FP64.
//           ok &= p >= 1 or greedy or r < next_up(p + slack); mass_above = p < 1 ? r : 0.
// The sums are order-free within member_eps32 (reference member.py:84-102); ok and above are
// exact.  For a token below kth (already rejected by the top-k test) r counts every kept
// logit above it, where the reference's top-(max k) path leaves out ties beyond max k; the
// verdict is the same (false).
//
// Kernel: one workgroup of 1024 lanes per row.
//   Prefix (the first kPrefix logits): count above, NaN flag and each lane's
//   maximum.  For a top-p row with a top-k, a 16-bit radix select over the 1024 lane maxima
//   gives L0, a value at or below the k_eff-th largest lane maximum, so at least k_eff logits of
//   the prefix are >= L0 and L0 is a lower bound of the row's kth (the k-th largest of a part
//   never exceeds that of the whole).
//   Stream (the rest of the row, read from HBM once, non-temporal): count above, NaN flag, row
//   maximum, and the logits >= L0 compacted into LDS, each wave into its own segment of kSeg
//   slots (a ballot per step; the wave's count is uniform, so no atomics); then the prefix,
//   held in registers (or re-read from L2 for unaligned or short rows), is compacted too.  For
//   LLM logits that is a few hundred values (a few dozen per wave); kth and both sums come from
//   LDS with no further pass over the row, each wave reading back its own segment (into
//   registers, one candidate per lane, when no wave holds more than 64).
//   Tail: one exchange for the counts, flags and maximum; kth by an exact radix select over the
//   candidates, four 8-bit rounds of one barrier each (every wave scans the histogram itself
//   and finds the digit in scalar registers); the two FP64 sums; the verdict.
//   Fallbacks: if more than kSeg values qualify in one wave (flat or adversarial rows), an
//   exact 4-pass radix select over the row and a summing pass take over.  Rows without a top-k
//   sum over the whole row in a second pass.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"
#include "rounding.h"

namespace pck {
namespace {

constexpr int kThreads = 1024;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kCap = 4096;  // candidates held in LDS
constexpr int kSeg = kCap / kWaves;  // candidates each wave holds, in its own segment
constexpr int64_t kPrefix = 16 * kThreads;  // logits that set the candidate threshold

using MemberArgs = PckMemberArgs;

// Order-preserving 64-bit key of an FP64 value (a larger value has a larger key), for the
// totals' running maximum of r - p, kept with an unsigned atomic maximum.
__device__ __forceinline__ unsigned long long order_key64(double v) {
  const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// Order-preserving key: a larger float has a larger key; -0 and +0 share the key of +0.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u << 1) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// FP32 e^(x - m) from the exact split x - m = hi + lo (Knuth's TwoSum), 0 where hi < -128 or
// NaN; the operation order of reference member.py:110-115.
__device__ __forceinline__ float split_term(float x, float m) {
  const float nm = -m;
  const float hi = x + nm;
  const float bv = hi - x;
  const float lo = (x - (hi - bv)) + (nm - bv);
  const float eh = expf(hi);
  const float prod = eh * lo;
  return hi >= -128.0f ? eh + prod : 0.0f;
}

struct Scratch {
  alignas(16) float cand[kCap];
  alignas(16) uint32_t hist[3][256];
  double red_d[2][kWaves];
  int64_t red_i[kWaves];
  float red_f[kWaves];
  int red_flag[kWaves];
};

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return static_cast<int>(threadIdx.x) / kWave; }

// The value of v in the lane kCtrl's DPP pattern names (every lane has a source here).
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __uint_as_float(dpp<kCtrl>(__float_as_uint(v)));
}
template <int kCtrl>
__device__ __forceinline__ double dpp(double v) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = dpp<kCtrl>(static_cast<uint32_t>(u));
  const uint64_t hi = dpp<kCtrl>(static_cast<uint32_t>(u >> 32));
  return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}

__device__ __forceinline__ uint32_t read_lane(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ float read_lane(float v, int lane) {
  return __uint_as_float(read_lane(__float_as_uint(v), lane));
}
__device__ __forceinline__ double read_lane(double v, int lane) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = read_lane(static_cast<uint32_t>(u), lane);
  const uint64_t hi = read_lane(static_cast<uint32_t>(u >> 32), lane);
  return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}

// op over the wave's 64 lanes, returned in every lane, in a fixed order: inside each 16-lane
// row, partners at quad_perm [1,0,3,2] and [2,3,0,1], then row_ror 4 and row_ror 8 (every
// lane then holds its row's result; for a non-associative op the lanes may differ in how it
// was grouped, and only lanes 0, 16, 32 and 48 are read), then (r0 op r1) op (r2 op r3).
// Every lane must be active.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  v = op(v, dpp<0xB1>(v));
  v = op(v, dpp<0x4E>(v));
  v = op(v, dpp<0x124>(v));
  v = op(v, dpp<0x128>(v));
  return op(op(read_lane(v, 0), read_lane(v, 16)), op(read_lane(v, 32), read_lane(v, 48)));
}

// Workgroup sum of `count`, OR of `flag` and max of `v` (one barrier; the exchange slots are
// not reused afterwards).  A lane's count and the wave's sum fit in 32 bits.
__device__ void group_reduce(uint32_t lane_count, int64_t& count, int& flag, float& v,
                             Scratch& s) {
  const uint32_t c = wave_reduce(lane_count, [](uint32_t x, uint32_t y) { return x + y; });
  const uint32_t f =
      wave_reduce(static_cast<uint32_t>(flag), [](uint32_t x, uint32_t y) { return x | y; });
  const float mx = wave_reduce(v, [](float x, float y) { return fmaxf(x, y); });
  if (lane_id() == 0) {
    s.red_i[wave_id()] = c;
    s.red_flag[wave_id()] = static_cast<int>(f);
    s.red_f[wave_id()] = mx;
  }
  __syncthreads();
  count = 0;
  flag = 0;
  v = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    count += s.red_i[w];
    flag |= s.red_flag[w];
    v = fmaxf(v, s.red_f[w]);
  }
}

// Two FP64 sums at once (the kept mass and the mass above the token), in a fixed order (one
// barrier; the exchange slots are not reused afterwards).
__device__ void group_sum2(double& a, double& b, Scratch& s) {
  const auto add = [](double x, double y) { return x + y; };
  a = wave_reduce(a, add);
  b = wave_reduce(b, add);
  if (lane_id() == 0) {
    s.red_d[0][wave_id()] = a;
    s.red_d[1][wave_id()] = b;
  }
  __syncthreads();
  a = 0.0;
  b = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    a += s.red_d[0][w];
    b += s.red_d[1][w];
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool kNt>
__device__ __forceinline__ f32x4 load_quad(const f32x4* p) {
  if constexpr (kNt) return __builtin_nontemporal_load(p);
  else return *p;
}

// Calls f4(quad) for the 16-byte quads and f1(value) for the remaining logits of row[begin,
// end), each logit exactly once (begin % 4 == 0); four quads in flight per lane when the row is
// aligned, element loads otherwise.  kNt: non-temporal loads (data read once that need not stay
// in the caches).  pre() runs once, by every lane, after the first quads are requested and
// before any is used, so workgroup-wide work placed there overlaps their latency.
template <bool kNt, typename F4, typename F1, typename P>
__device__ __forceinline__ void for_each4(const float* __restrict__ row, int64_t begin,
                                          int64_t end, F4&& f4, F1&& f1, P&& pre) {
  const int t = static_cast<int>(threadIdx.x);
  int64_t done = begin;
  if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const f32x4* quads = reinterpret_cast<const f32x4*>(row);
    const int64_t q1 = end / 4;
    int64_t q = begin / 4 + t;
    const bool first = q + 3 * kThreads < q1;
    f32x4 a, b, c, d;
    if (first) {
      a = load_quad<kNt>(quads + q);
      b = load_quad<kNt>(quads + q + kThreads);
      c = load_quad<kNt>(quads + q + 2 * kThreads);
      d = load_quad<kNt>(quads + q + 3 * kThreads);
    }
    pre();
    if (first) {
      f4(a), f4(b), f4(c), f4(d);
      q += 4 * kThreads;
    }
    for (; q + 3 * kThreads < q1; q += 4 * kThreads) {
      a = load_quad<kNt>(quads + q);
      b = load_quad<kNt>(quads + q + kThreads);
      c = load_quad<kNt>(quads + q + 2 * kThreads);
      d = load_quad<kNt>(quads + q + 3 * kThreads);
      f4(a), f4(b), f4(c), f4(d);
    }
    for (; q < q1; q += kThreads) f4(load_quad<kNt>(quads + q));
    done = end > begin ? (q1 * 4 > begin ? q1 * 4 : begin) : end;
  } else {
    pre();
  }
  for (int64_t i = done + t; i < end; i += kThreads) f1(row[i]);
}

template <bool kNt, typename F4, typename F1>
__device__ __forceinline__ void for_each4(const float* __restrict__ row, int64_t begin,
                                          int64_t end, F4&& f4, F1&& f1) {
  for_each4<kNt>(row, begin, end, f4, f1, [] {});
}

// Calls f(value) for every logit of row[begin, end), each exactly once (begin % 4 == 0).
template <bool kNt, typename F>
__device__ __forceinline__ void for_each(const float* __restrict__ row, int64_t begin,
                                         int64_t end, F&& f) {
  for_each4<kNt>(row, begin, end, [&](const f32x4& v) { f(v[0]), f(v[1]), f(v[2]), f(v[3]); }, f);
}

// Inclusive prefix sum over the 64 lanes in VALU cross-lane moves: Hillis-Steele steps of
// 1, 2, 4 and 8 inside each 16-lane row (row_shr, lanes without a source read 0), then each
// row's total is carried into the next (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows
// 2 and 3).
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
  const int x = static_cast<int>(v);
  int a = x + __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  a += __builtin_amdgcn_update_dpp(0, a, 0x112, 0xF, 0xF, true);         // row_shr:2
  a += __builtin_amdgcn_update_dpp(0, a, 0x114, 0xF, 0xF, true);         // row_shr:4
  a += __builtin_amdgcn_update_dpp(0, a, 0x118, 0xF, 0xF, true);         // row_shr:8
  a += __builtin_amdgcn_update_dpp(0, a, 0x142, 0xA, 0xF, false);        // row_bcast:15
  a += __builtin_amdgcn_update_dpp(0, a, 0x143, 0xC, 0xF, false);        // row_bcast:31
  return static_cast<uint32_t>(a);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Adds the digits (k >> shift) & 255 of the keys with (k & mask) == prefix into hist.  Keys
// bunch into a few buckets (one exponent byte for every candidate): a wave whose counted lanes
// share one digit adds them with one atomic instead of serialising them.
__device__ __forceinline__ void radix_count(uint32_t k, uint32_t prefix, uint32_t mask,
                                            int shift, uint32_t* hist) {
  const bool hit = (k & mask) == prefix;
  const uint32_t digit = (k >> shift) & 255u;
  const uint64_t counted = __ballot(hit);
  const int first = counted ? __builtin_ctzll(counted) : 0;
  const uint32_t d0 = read_lane(digit, first);
  if (__ballot(hit && digit != d0) == 0) {
    if (counted != 0 && lane_id() == first)
      atomicAdd(&hist[d0], static_cast<uint32_t>(__builtin_popcountll(counted)));
  } else if (hit) {
    atomicAdd(&hist[digit], 1u);
  }
}

// The digit of a complete 256-bin histogram that holds the want-th largest key, with want
// turned into the rank within that digit; every wave computes it itself.  Lane l owns digits
// 255 - 4l ... 252 - 4l (descending; h[3] is digit 255 - 4l).  The first lane whose inclusive
// count reaches want owns the digit; its four counts and the count before them are read into
// scalar registers and the descent runs once per wave.
__device__ __forceinline__ uint32_t radix_find(const uint32_t* hist, uint32_t& want) {
  const u32x4 h = *reinterpret_cast<const u32x4*>(hist + 252 - 4 * lane_id());
  const uint32_t own = h[0] + h[1] + h[2] + h[3];
  const uint32_t incl = wave_inclusive_sum(own);
  const uint64_t reach = __ballot(incl >= want);
  const int src = reach ? __builtin_ctzll(reach) : kWave - 1;
  uint32_t rest = want - read_lane(incl - own, src);  // rank within the owner's four digits
  uint32_t digit = static_cast<uint32_t>(255 - 4 * src);
  const uint32_t c3 = read_lane(h[3], src);
  const uint32_t c2 = read_lane(h[2], src);
  const uint32_t c1 = read_lane(h[1], src);
  if (rest > c3) {
    rest -= c3, --digit;
    if (rest > c2) {
      rest -= c2, --digit;
      if (rest > c1) rest -= c1, --digit;
    }
  }
  want = rest;
  return digit;
}

// Key of the rank-th largest (1-based) of the workgroup's keys, by an exact radix select over
// 8-bit digits with LDS histograms.  visit(f) calls f(key) for each key a lane holds, the same
// way on every round (each key by one lane).  Every lane returns the same key.  With kRounds < 4
// only the top 8 kRounds bits are selected and the rest are zero: the result is the smallest key
// of the bucket that holds the rank-th largest.  The caller clears hist[0], with a barrier
// between that and the call.
template <int kRounds = 4, typename V>
__device__ uint32_t radix_select(int64_t rank, V&& visit, Scratch& s) {
  const int t = static_cast<int>(threadIdx.x);
  uint32_t prefix = 0;
  uint32_t mask = 0;
  uint32_t want = static_cast<uint32_t>(rank);  // counts fit in 32 bits (vocab < 2^31)
#pragma unroll
  for (int round = 0; round < kRounds; ++round) {
    const int shift = 24 - 8 * round;
    uint32_t* const hist = s.hist[round % 3];
    // Round r counts into hist[r % 3] and clears hist[(r + 1) % 3], last read by the scans of
    // round r - 2, which every wave finished before the barrier of round r - 1; every wave
    // scans the histogram itself, so a round takes one barrier.
    if (t < 256) s.hist[(round + 1) % 3][t] = 0;
    visit([&](uint32_t k) { radix_count(k, prefix, mask, shift, hist); });
    __syncthreads();
    prefix |= radix_find(hist, want) << shift;
    mask |= 255u << shift;
  }
  return prefix;
}

__global__ void __launch_bounds__(kThreads) member_kernel(const MemberArgs A) {
  __shared__ Scratch s;
  const int64_t r = blockIdx.x;
  const int t = static_cast<int>(threadIdx.x);
  const int64_t vocab = A.vocab;
  const float* __restrict__ row = A.logits + r * vocab;

  const int64_t token = A.tokens[r];
  const bool in_range = token >= 0 && token < vocab;
  const float lt = row[in_range ? token : (token < 0 ? 0 : vocab - 1)];
  // a requested top-k is clamped to [1, vocab] (reference src/pck/member.py:153)
  const int64_t k_req = A.top_k ? A.top_k[r] : vocab;
  const int64_t k_row = k_req < 1 ? 1 : (k_req > vocab ? vocab : k_req);
  // Greedy rows: the caller's flags, or temperature 0 of the row's request (vLLM's sampling
  // state, read through the row's request index).  A request index outside the temperature
  // array rejects the row without reading it.
  const int64_t request = A.temperature ? A.temperature_index[r] : 0;
  const bool request_ok = !A.temperature || (request >= 0 && request < A.temperature_count);
  const bool greedy = A.temperature ? request_ok && A.temperature[request_ok ? request : 0] == 0.0f
                                    : (A.greedy ? A.greedy[r] != 0 : false);
  const bool has_p = A.top_p != nullptr;
  const double p = !has_p ? 1.0
                   : A.top_p_fp32 ? static_cast<double>(static_cast<const float*>(A.top_p)[r])
                                  : static_cast<const double*>(A.top_p)[r];

  const bool want_mass = has_p && p < 1.0;
  const bool use_kth = A.all_k || (A.k_lim > 0 && k_row < vocab);
  const int64_t k_eff = k_row < A.k_lim ? k_row : A.k_lim;
  const bool fused = want_mass && use_kth && k_eff <= kThreads;
  const int64_t prefix = vocab < kPrefix ? vocab : kPrefix;

  // Exact count above the token, NaN flag and lane maxima over the prefix (kept in L2).
  uint32_t above_lane = 0;
  int nan = 0;
  float lane_max = -__builtin_inff();
  auto scan = [&](float l) {
    above_lane += l > lt;
    nan |= l != l;
    lane_max = fmaxf(lane_max, l);
  };
  // An aligned row with a full prefix keeps its prefix quads in registers for the compaction.
  const bool held = (reinterpret_cast<uintptr_t>(row) & 15) == 0 && prefix == kPrefix;
  constexpr int kHeld = kPrefix / (4 * kThreads);
  f32x4 pq[kHeld];
  if (held) {
    const f32x4* quads = reinterpret_cast<const f32x4*>(row);
#pragma unroll
    for (int j = 0; j < kHeld; ++j) pq[j] = quads[t + j * kThreads];
#pragma unroll
    for (int j = 0; j < kHeld; ++j) scan(pq[j][0]), scan(pq[j][1]), scan(pq[j][2]), scan(pq[j][3]);
  } else {
    for_each<false>(row, 0, prefix, scan);
  }

  // Candidate threshold: the smallest value of the 16-bit key bucket that holds the k_eff-th
  // largest lane maximum of the prefix (a NaN bit pattern there means -inf: keep everything).
  // It is selected while the stream's first loads are in flight.
  float low = -__builtin_inff();
  auto threshold = [&] {
    const uint32_t key = order_key(lane_max);
    if (t < 256) s.hist[0][t] = 0;
    __syncthreads();
    low = key_value(radix_select<2>(k_eff, [&](auto&& f) { f(key); }, s));
    if (low != low) low = -__builtin_inff();
  };
  // Compacts every logit >= low into the wave's LDS segment.  The wave's count follows the
  // ballots, so no atomic is needed.  Lanes may diverge at the end of a range: the lanes that
  // run a step are then always a prefix of the wave from its lane 0 (a lane's trip count never
  // exceeds that of a lower lane), so lane 0 runs every step and holds the wave's count, and
  // each step takes the count from the first active lane.
  float* const seg = s.cand + wave_id() * kSeg;
  int wcount = 0;
  auto compact = [&](float l) {
    const bool take = l >= low;
    const uint64_t want = __ballot(take);
    if (want != 0) {
      const int first = __builtin_amdgcn_readfirstlane(wcount);
      if (take) {
        const uint64_t below = lane_id() ? want & (~0ull >> (kWave - lane_id())) : 0ull;
        const int at = first + __builtin_popcountll(below);
        if (at < kSeg) seg[at] = l;
      }
      wcount = first + __builtin_popcountll(want);
    }
  };
  // Most quads hold no candidate: one ballot per quad decides whether any lane needs compact.
  auto compact4 = [&](const f32x4& v) {
    const bool any = (v[0] >= low) | (v[1] >= low) | (v[2] >= low) | (v[3] >= low);
    if (__ballot(any) != 0) compact(v[0]), compact(v[1]), compact(v[2]), compact(v[3]);
  };
  // The rest of the row, streamed from HBM once.
  if (fused) {
    for_each4<true>(
        row, prefix, vocab,
        [&](const f32x4& v) {
          scan(v[0]), scan(v[1]), scan(v[2]), scan(v[3]);
          compact4(v);
        },
        [&](float l) {
          scan(l);
          compact(l);
        },
        threshold);
    if (held) {
#pragma unroll
      for (int j = 0; j < kHeld; ++j) compact4(pq[j]);
    } else {
      for_each4<false>(row, 0, prefix, compact4, compact);
    }
  } else {
    for_each<true>(row, prefix, vocab, scan);
  }
  // bit 0: a NaN in the row; bit 1: a wave's segment overflowed; bit 2: a wave holds more
  // candidates than lanes (every lane runs here, so the first active lane is lane 0)
  wcount = __builtin_amdgcn_readfirstlane(wcount);
  int64_t above = 0;
  int flags = nan | (wcount > kSeg ? 2 : 0) | (wcount > kWave ? 4 : 0);
  float m = lane_max;
  // hist[0] is cleared for the select below; its last readers (the threshold's first round)
  // are done, and the barrier of group_reduce orders the clear before the select
  if (t < 256) s.hist[0][t] = 0;
  group_reduce(above_lane, above, flags, m, s);
  const bool any_nan = flags & 1;
  const bool overflow = flags & 2;

  bool ok = request_ok && !any_nan && in_range && above < (greedy ? 1 : k_row);
  double mass = 0.0;
  if (want_mass) {
    double z = 0.0;
    double a = 0.0;
    if (!use_kth) {
      for_each<false>(row, 0, vocab, [&](float l) {
        const float e = split_term(l, m);
        z += e;
        a += l > lt ? e : 0.0;
      });
    } else if (fused && !(flags & 4)) {
      // At most one candidate per lane (the common case): each lane keeps its candidate, key
      // and term in registers for every round of the select.
      const bool have = lane_id() < wcount;
      const float c = have ? seg[lane_id()] : 0.0f;
      const uint32_t key = order_key(c);
      const float e = have ? split_term(c, m) : 0.0f;
      const float kth = key_value(radix_select(k_eff, [&](auto&& f) {
        if (have) f(key);
      }, s));
      if (have && c >= kth) {
        z = e;
        a = c > lt ? e : 0.0;
      }
    } else if (fused && !overflow) {
      // each wave reads back its own segment (LDS is in order within a wave)
      const float kth = key_value(radix_select(k_eff, [&](auto&& f) {
        for (int j = lane_id(); j < wcount; j += kWave) f(order_key(seg[j]));
      }, s));
      for (int j = lane_id(); j < wcount; j += kWave) {
        const float l = seg[j];
        if (l >= kth) {
          const float e = split_term(l, m);
          z += e;
          a += l > lt ? e : 0.0;
        }
      }
    } else {
      const float kth = key_value(radix_select(k_eff, [&](auto&& f) {
        for (int64_t i = t; i < vocab; i += kThreads) f(order_key(row[i]));
      }, s));
      for_each<false>(row, 0, vocab, [&](float l) {
        if (l >= kth) {
          const float e = split_term(l, m);
          z += e;
          a += l > lt ? e : 0.0;
        }
      });
    }
    group_sum2(z, a, s);
    const double ratio = a / z;
    mass = ratio;
    const double high = next_up(p + A.slack);  // the bound rounded outward
    ok = ok && (greedy || ratio < high);
  }
  if (t == 0) {
    if (A.ok) A.ok[r] = ok;
    if (A.above) A.above[r] = above;
    if (A.mass_above) A.mass_above[r] = mass;
    if (A.totals) {
      // Running totals (integer atomics, so the sums do not depend on the order of rows):
      // rows, rejected, injected, caught (rejected and injected), false alarms (rejected, not
      // injected), and the maximum of r - p over accepted top-p rows not greedy (the key of
      // -1 is the host's initial value: no such row yet).
      unsigned long long* tot = A.totals;
      const bool injected = A.injected ? A.injected[r] != 0 : false;
      atomicAdd(&tot[0], 1ull);
      if (!ok) atomicAdd(&tot[1], 1ull);
      if (injected) atomicAdd(&tot[2], 1ull);
      if (!ok && injected) atomicAdd(&tot[3], 1ull);
      if (!ok && !injected) atomicAdd(&tot[4], 1ull);
      if (ok && want_mass && !greedy) atomicMax(&tot[5], order_key64(mass - p));
    }
  }
}

}  // namespace
}  // namespace pck

extern "C" int pck_check_members_ex(const PckMemberArgs* args, void* stream) {
  if (args == nullptr) return hipErrorInvalidValue;
  const PckMemberArgs& a = *args;
  if (a.rows < 0 || a.rows * pck::kThreads > 0xFFFFFFFFll || a.vocab < 1 ||
      a.vocab > 0x7FFFFFFF || a.k_lim < 0 || a.k_lim > a.vocab)
    return hipErrorInvalidValue;
  if (a.rows == 0) return hipSuccess;
  if (!a.logits || !a.tokens ||
      (a.temperature && (!a.temperature_index || a.temperature_count < 1)))
    return hipErrorInvalidValue;
  if (a.all_k && a.k_lim < 1) return hipErrorInvalidValue;
  pck::member_kernel<<<dim3(static_cast<unsigned>(a.rows)), dim3(pck::kThreads), 0,
                       static_cast<hipStream_t>(stream)>>>(a);
  return hipGetLastError();
}

extern "C" int pck_check_members(const float* logits, int64_t rows, int64_t vocab,
                                 const int64_t* tokens, const int64_t* top_k, const double* top_p,
                                 const uint8_t* greedy, double slack, int64_t k_lim, int all_k,
                                 uint8_t* ok, int64_t* above, double* mass_above, void* stream) {
  if (rows > 0 && (!ok || !above || !mass_above)) return hipErrorInvalidValue;
  PckMemberArgs a{};
  a.logits = logits;
  a.rows = rows;
  a.vocab = vocab;
  a.tokens = tokens;
  a.top_k = top_k;
  a.top_p = top_p;
  a.greedy = greedy;
  a.slack = slack;
  a.k_lim = k_lim;
  a.all_k = all_k;
  a.ok = ok;
  a.above = above;
  a.mass_above = mass_above;
  return pck_check_members_ex(&a, stream);
}
