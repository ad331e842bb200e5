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
//   Pass 1 (HBM): count above, NaN flag, row max, and each lane's own maximum.
//   The k_eff-th largest of the 1024 lane maxima, L0, is a lower bound of kth (k_eff lanes hold
//   a value >= L0), so every kept logit is >= L0.
//   Pass 2 (the row is now in L2/MALL): compact the logits >= L0 into LDS (ballot + one LDS
//   atomic per wave).  For LLM logits that is a few dozen values; kth and both sums then come
//   from LDS without another pass.  If more than kCap values qualify (flat or adversarial
//   rows), an exact 4-pass radix select over the row and a summing pass take over.
//   Rows without a top-k sum over the whole row in pass 2.

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

struct MemberArgs {
  const float* logits;
  int64_t rows;
  int64_t vocab;
  const int64_t* tokens;
  const int64_t* top_k;
  const double* top_p;
  const uint8_t* greedy;
  double slack;
  int64_t k_lim;
  int all_k;
  uint8_t* ok;
  int64_t* above;
  double* mass_above;
};

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
  float cand[kCap];
  uint32_t lane_key[kThreads];
  uint32_t hist[256];
  double red_d[2][kWaves];
  int64_t red_i[kWaves];
  float red_f[kWaves];
  int red_flag[kWaves];
  int count;
  uint32_t digit;
  int64_t rank;
};

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return static_cast<int>(threadIdx.x) / kWave; }

__device__ int64_t group_sum_i64(int64_t v, Scratch& s) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) v += __shfl_xor(v, off, kWave);
  if (lane_id() == 0) s.red_i[wave_id()] = v;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total += s.red_i[w];
  __syncthreads();
  return total;
}

__device__ float group_max(float v, Scratch& s) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) v = fmaxf(v, __shfl_xor(v, off, kWave));
  if (lane_id() == 0) s.red_f[wave_id()] = v;
  __syncthreads();
  float total = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total = fmaxf(total, s.red_f[w]);
  __syncthreads();
  return total;
}

// Two FP64 sums at once (the kept mass and the mass above the token).
__device__ void group_sum2(double& a, double& b, Scratch& s) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) {
    a += __shfl_xor(a, off, kWave);
    b += __shfl_xor(b, off, kWave);
  }
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
  __syncthreads();
}

// Calls f(value) for every logit of the row, each exactly once; float4 loads when aligned.
template <typename F>
__device__ __forceinline__ void for_each(const float* __restrict__ row, int64_t vocab, F&& f) {
  const int t = static_cast<int>(threadIdx.x);
  int64_t done = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const float4* quads = reinterpret_cast<const float4*>(row);
    const int64_t nq = vocab / 4;
    int64_t q = t;
    for (; q + 3 * kThreads < nq; q += 4 * kThreads) {
      const float4 a = quads[q];
      const float4 b = quads[q + kThreads];
      const float4 c = quads[q + 2 * kThreads];
      const float4 d = quads[q + 3 * kThreads];
      f(a.x), f(a.y), f(a.z), f(a.w);
      f(b.x), f(b.y), f(b.z), f(b.w);
      f(c.x), f(c.y), f(c.z), f(c.w);
      f(d.x), f(d.y), f(d.z), f(d.w);
    }
    for (; q < nq; q += kThreads) {
      const float4 a = quads[q];
      f(a.x), f(a.y), f(a.z), f(a.w);
    }
    done = nq * 4;
  }
  for (int64_t i = done + t; i < vocab; i += kThreads) f(row[i]);
}

// Key of the rank-th largest (1-based) of `count` keys given by key_of(i), by an exact radix
// select over 8-bit digits with an LDS histogram.  Every lane returns the same key.
template <typename K>
__device__ uint32_t radix_select(int64_t count, int64_t rank, K&& key_of, Scratch& s) {
  const int t = static_cast<int>(threadIdx.x);
  uint32_t prefix = 0;
  uint32_t mask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (t < 256) s.hist[t] = 0;
    __syncthreads();
    for (int64_t i = t; i < count; i += kThreads) {
      const uint32_t k = key_of(i);
      if ((k & mask) == prefix) atomicAdd(&s.hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave_id() == 0) {
      // lane l owns digits 255 - 4l ... 252 - 4l (descending); scan lanes in order
      const int l = lane_id();
      uint32_t h[4];
      int64_t own = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        h[q] = s.hist[255 - 4 * l - q];
        own += h[q];
      }
      int64_t incl = own;
#pragma unroll
      for (int off = 1; off < kWave; off *= 2) {
        const int64_t up = __shfl_up(incl, off, kWave);
        if (l >= off) incl += up;
      }
      const int64_t excl = incl - own;
      if (excl < rank && rank <= incl) {
        int64_t cum = excl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (cum + h[q] >= rank) {
            s.digit = static_cast<uint32_t>(255 - 4 * l - q);
            s.rank = rank - cum;
            break;
          }
          cum += h[q];
        }
      }
    }
    __syncthreads();
    prefix |= s.digit << shift;
    mask |= 255u << shift;
    rank = s.rank;
    __syncthreads();
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
  const int64_t k_row = A.top_k ? A.top_k[r] : vocab;
  const bool greedy = A.greedy ? A.greedy[r] != 0 : false;
  const double p = A.top_p ? A.top_p[r] : 1.0;

  // Pass 1: exact count above the token, NaN flag, row maximum and lane maxima.
  uint32_t above_lane = 0;
  int nan = 0;
  float lane_max = -__builtin_inff();
  for_each(row, vocab, [&](float l) {
    above_lane += l > lt;
    nan |= l != l;
    lane_max = fmaxf(lane_max, l);
  });
  const int64_t above = group_sum_i64(above_lane, s);
  const int any_nan = __syncthreads_or(nan);
  const float m = group_max(lane_max, s);

  bool ok = !any_nan && in_range && above < (greedy ? 1 : k_row);
  double mass = 0.0;
  if (A.top_p != nullptr && p < 1.0) {
    const bool use_kth = A.all_k || (A.k_lim > 0 && k_row < vocab);
    double z = 0.0;
    double a = 0.0;
    if (!use_kth) {
      for_each(row, vocab, [&](float l) {
        const float e = split_term(l, m);
        z += e;
        a += l > lt ? e : 0.0;
      });
    } else {
      const int64_t k_eff = k_row < A.k_lim ? k_row : A.k_lim;
      bool in_lds = false;
      if (k_eff <= kThreads) {
        s.lane_key[t] = order_key(lane_max);
        if (t == 0) s.count = 0;
        __syncthreads();
        const float low =
            key_value(radix_select(kThreads, k_eff, [&](int64_t i) { return s.lane_key[i]; }, s));
        // Pass 2: compact every logit >= low into LDS.
        for_each(row, vocab, [&](float l) {
          const bool take = l >= low;
          const uint64_t want = __ballot(take);
          if (want != 0) {
            const uint64_t active = __ballot(1);
            const int leader = __builtin_ctzll(active);
            int base = 0;
            if (lane_id() == leader) base = atomicAdd(&s.count, __builtin_popcountll(want));
            base = __shfl(base, leader, kWave);
            if (take) {
              const uint64_t below = lane_id() ? want & (~0ull >> (kWave - lane_id())) : 0ull;
              const int at = base + __builtin_popcountll(below);
              if (at < kCap) s.cand[at] = l;
            }
          }
        });
        __syncthreads();
        in_lds = s.count <= kCap;
      }
      if (in_lds) {
        const int64_t count = s.count;
        const float kth = key_value(
            radix_select(count, k_eff, [&](int64_t i) { return order_key(s.cand[i]); }, s));
        for (int64_t i = t; i < count; i += kThreads) {
          const float l = s.cand[i];
          if (l >= kth) {
            const float e = split_term(l, m);
            z += e;
            a += l > lt ? e : 0.0;
          }
        }
      } else {
        const float kth = key_value(
            radix_select(vocab, k_eff, [&](int64_t i) { return order_key(row[i]); }, s));
        for_each(row, vocab, [&](float l) {
          if (l >= kth) {
            const float e = split_term(l, m);
            z += e;
            a += l > lt ? e : 0.0;
          }
        });
      }
    }
    group_sum2(z, a, s);
    const double ratio = a / z;
    mass = ratio;
    const double high = next_up(p + A.slack);  // the bound rounded outward
    ok = ok && (greedy || ratio < high);
  }
  if (t == 0) {
    A.ok[r] = ok;
    A.above[r] = above;
    A.mass_above[r] = mass;
  }
}

}  // namespace
}  // namespace pck

extern "C" int pck_check_members(const float* logits, int64_t rows, int64_t vocab,
                                 const int64_t* tokens, const int64_t* top_k, const double* top_p,
                                 const uint8_t* greedy, double slack, int64_t k_lim, int all_k,
                                 uint8_t* ok, int64_t* above, double* mass_above, void* stream) {
  if (rows < 0 || rows * pck::kThreads > 0xFFFFFFFFll || vocab < 1 || k_lim < 0 || k_lim > vocab)
    return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!logits || !tokens || !ok || !above || !mass_above) return hipErrorInvalidValue;
  if (all_k && k_lim < 1) return hipErrorInvalidValue;
  const pck::MemberArgs args{logits, rows,  vocab, tokens, top_k, top_p, greedy,
                             slack,  k_lim, all_k, ok,     above, mass_above};
  pck::member_kernel<<<dim3(static_cast<unsigned>(rows)), dim3(pck::kThreads), 0,
                       static_cast<hipStream_t>(stream)>>>(args);
  return hipGetLastError();
}
