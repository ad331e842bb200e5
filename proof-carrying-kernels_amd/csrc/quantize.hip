// The INT8 weight copy read by the row-major template's INT8 variant (template.hip).
//
// Reference src/pck/agent/config.py:163-175 (NumPy on the CPU there, called by
// src/pck/cuda/gemv.py:95-102).  One wave per (row, 128-column group) finds max |w| by a wave
// reduction, sets scale = max / 127 (1 for an all-zero group) and q = round-half-even(w / scale)
// clipped to [-127, 127].  Both divisions are correctly rounded (__fdiv_rn, the IEEE division
// sequence), and rintf rounds ties to even, so the copy equals NumPy's bit for bit.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_template.h"

namespace pck {
namespace {

constexpr int kWave = 64;
constexpr int kQ8Group = 128;

__device__ __forceinline__ float bf16_bits(uint32_t h) { return __uint_as_float(h << 16); }

// One wave per (row, group), two columns per lane.

template <bool kF32>
__global__ void __launch_bounds__(256)
    quantize_rows_kernel(const void* __restrict__ W, int8_t* __restrict__ Wq,
                         float* __restrict__ S, int64_t m, int64_t n, int64_t groups) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
  if (item >= m * groups) return;  // uniform per wave
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int64_t row = item / groups;
  const int64_t c0 = (item % groups) * kQ8Group + 2 * lane;
  float w[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int64_t c = c0 + e;
    const int64_t at = row * n + (c < n ? c : 0);
    const float v = kF32 ? static_cast<const float*>(W)[at]
                         : bf16_bits(static_cast<const uint16_t*>(W)[at]);
    w[e] = c < n ? v : 0.0f;  // the padded tail of the last group is zero
  }
  float amax = fmaxf(fabsf(w[0]), fabsf(w[1]));
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float scale = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float q = fminf(fmaxf(rintf(__fdiv_rn(w[e], scale)), -127.0f), 127.0f);
    if (c0 + e < n) Wq[row * n + c0 + e] = static_cast<int8_t>(q);
  }
  if (lane == 0) S[item] = scale;
}

}  // namespace
}  // namespace pck

extern "C" {

int pck_quantize_rows_q8(const void* W, int w_kind, int8_t* Wq, float* S, int64_t m, int64_t n,
                         void* stream) {
  using namespace pck;
  if ((w_kind != 0 && w_kind != 1) || m < 0 || n < 0 || m > 0x7FFFFFFF) return hipErrorInvalidValue;
  if (m == 0 || n == 0) return hipSuccess;
  if (W == nullptr || Wq == nullptr || S == nullptr) return hipErrorInvalidValue;
  const int64_t groups = (n + kQ8Group - 1) / kQ8Group;
  const int64_t blocks = (m * groups + 3) / 4;
  if (blocks * 256 > 0xFFFFFFFFll) return hipErrorInvalidValue;  // 32-bit dispatch size
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (w_kind == 1) {
    quantize_rows_kernel<true><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        W, Wq, S, m, n, groups);
  } else {
    quantize_rows_kernel<false><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        W, Wq, S, m, n, groups);
  }
  return hipGetLastError();
}

}  // extern "C"
