// Probes of the device arithmetic that the library's error bounds assume, built into their own
// library (libpck_probe.so) with the same flags as libpck_hip.so.  Nothing in the product
// calls them; tests run them on the GPU and compare the results with exact host arithmetic.
//
//   pck_probe_expf            y = expf(x), the FP32 exponential the membership and sampling
//                             kernels call (same header, same flags, same code);
//   pck_probe_mfma_f64        v_mfma_f64_16x16x4_f64 chains, as the batched checker runs c . x;
//   pck_probe_mfma_bf16       v_mfma_f32_32x32x16_bf16 chains;
//   pck_probe_mfma_bf16_k8    v_mfma_f32_32x32x8_bf16 chains (the batched product's step: one
//                             group of 8 K-slots split over the two lane halves, 4 per lane);
//   pck_probe_mfma_bf16_16x16 v_mfma_f32_16x16x32_bf16 chains (the batched checker's a . |x|);
//   pck_probe_round_up        rounding.h's upward products and sums, general and branch-free.
//   pck_probe_round_up_mode   rounding.h's upward sums under the wave's rounding mode, and an
//                             add the compiler places after them (round to nearest again).
//
// Operands are passed in lane order, so the probes embed no matrix layout: tile t, step s,
// lane l reads its A and B operands at [(t * steps + s) * 64 + l] (8 or 4 BF16 values or one
// FP64 value each) and its accumulator registers at [t * 64 + l] (16, 4 or 4 values), and writes
// the result registers after the last step in the same place of D.  One wave per tile; every
// tile index below `tiles`, so each access stays inside buffers of the documented sizes.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_probe.h"
#include "rounding.h"

namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

__global__ void __launch_bounds__(256) expf_kernel(const float* x, float* y, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = expf(x[i]);
}

__global__ void __launch_bounds__(kWave) mfma_f64_kernel(const double* a, const double* b,
                                                         const double* c, double* d, int steps) {
  const int64_t t = blockIdx.x;
  const int l = static_cast<int>(threadIdx.x);
  f64x4 acc;
  for (int v = 0; v < 4; ++v) acc[v] = c[(t * kWave + l) * 4 + v];
  for (int s = 0; s < steps; ++s) {
    const int64_t o = (t * steps + s) * kWave + l;
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[o], b[o], acc, 0, 0, 0);
  }
  for (int v = 0; v < 4; ++v) d[(t * kWave + l) * 4 + v] = acc[v];
}

__device__ inline bf16x8 load_bf16x8(const uint16_t* p) {
  const u16x8 bits = *reinterpret_cast<const u16x8*>(p);
  return __builtin_bit_cast(bf16x8, bits);
}

template <int kRegs>
__global__ void __launch_bounds__(kWave) mfma_bf16_kernel(const uint16_t* a, const uint16_t* b,
                                                          const float* c, float* d, int steps) {
  using acc_t = float __attribute__((ext_vector_type(kRegs)));
  const int64_t t = blockIdx.x;
  const int l = static_cast<int>(threadIdx.x);
  acc_t acc;
  for (int v = 0; v < kRegs; ++v) acc[v] = c[(t * kWave + l) * kRegs + v];
  for (int s = 0; s < steps; ++s) {
    const int64_t o = ((t * steps + s) * kWave + l) * 8;
    const bf16x8 av = load_bf16x8(a + o);
    const bf16x8 bv = load_bf16x8(b + o);
    if constexpr (kRegs == 16)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    else
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  }
  for (int v = 0; v < kRegs; ++v) d[(t * kWave + l) * kRegs + v] = acc[v];
}

// Four BF16 operands per lane (8 bytes): v_mfma_f32_32x32x8_bf16, the instruction the batched
// product issues.
__global__ void __launch_bounds__(kWave) mfma_bf16_k8_kernel(const uint16_t* a, const uint16_t* b,
                                                             const float* c, float* d, int steps) {
  const int64_t t = blockIdx.x;
  const int l = static_cast<int>(threadIdx.x);
  f32x16 acc;
  for (int v = 0; v < 16; ++v) acc[v] = c[(t * kWave + l) * 16 + v];
  for (int s = 0; s < steps; ++s) {
    const int64_t o = ((t * steps + s) * kWave + l) * 4;
    const s16x4 av = *reinterpret_cast<const s16x4*>(a + o);
    const s16x4 bv = *reinterpret_cast<const s16x4*>(b + o);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(av, bv, acc, 0, 0, 0);
  }
  for (int v = 0; v < 16; ++v) d[(t * kWave + l) * 16 + v] = acc[v];
}

__global__ void __launch_bounds__(256) round_up_kernel(const double* a, const double* b,
                                                       double* out, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    out[4 * i] = pck::mul_up(a[i], b[i]);
    out[4 * i + 1] = pck::mul_up_pos(a[i], b[i]);
    out[4 * i + 2] = pck::add_up(a[i], b[i]);
    out[4 * i + 3] = pck::add_up_nonneg(a[i], b[i]);
  }
}

// out[3 i] = add_up_rm2's and out[3 i + 1] = add_up_rm4's RU(a + b) (one slot of each, the
// others busy with other sums); out[3 i + 2] = (a + 0, rounded upward) + b as the compiler
// issues it after the blocks, which must be the round-to-nearest a + b (the mode restored).
__global__ void __launch_bounds__(256) round_up_mode_kernel(const double* a, const double* b,
                                                            double* out, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    double s0 = a[i], s1 = a[i];
    pck::add_up_rm2(s0, b[i], s1, 0.0);
    double q[4] = {1.0, 0x1p-60, a[i], 3.0};
    pck::add_up_rm4(q, 0x1p-60, 1.0, b[i], 0x1p-70);
    out[3 * i] = s0;
    out[3 * i + 1] = q[2];
    out[3 * i + 2] = s1 + b[i];
  }
}

bool tiles_ok(int64_t tiles, int steps) {
  return tiles >= 1 && tiles <= (1 << 20) && steps >= 1 && steps <= 64;
}

}  // namespace

extern "C" int pck_probe_expf(const float* x, float* y, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (x == nullptr || y == nullptr))) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  expf_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                static_cast<hipStream_t>(stream)>>>(x, y, n);
  return hipGetLastError();
}

extern "C" int pck_probe_mfma_f64(const double* a, const double* b, const double* c, double* d,
                                  int64_t tiles, int steps, void* stream) {
  if (!tiles_ok(tiles, steps) || !a || !b || !c || !d) return hipErrorInvalidValue;
  mfma_f64_kernel<<<dim3(static_cast<unsigned>(tiles)), dim3(kWave), 0,
                    static_cast<hipStream_t>(stream)>>>(a, b, c, d, steps);
  return hipGetLastError();
}

extern "C" int pck_probe_mfma_bf16(const uint16_t* a, const uint16_t* b, const float* c, float* d,
                                   int64_t tiles, int steps, void* stream) {
  if (!tiles_ok(tiles, steps) || !a || !b || !c || !d) return hipErrorInvalidValue;
  mfma_bf16_kernel<16><<<dim3(static_cast<unsigned>(tiles)), dim3(kWave), 0,
                         static_cast<hipStream_t>(stream)>>>(a, b, c, d, steps);
  return hipGetLastError();
}

extern "C" int pck_probe_mfma_bf16_16x16(const uint16_t* a, const uint16_t* b, const float* c,
                                         float* d, int64_t tiles, int steps, void* stream) {
  if (!tiles_ok(tiles, steps) || !a || !b || !c || !d) return hipErrorInvalidValue;
  mfma_bf16_kernel<4><<<dim3(static_cast<unsigned>(tiles)), dim3(kWave), 0,
                        static_cast<hipStream_t>(stream)>>>(a, b, c, d, steps);
  return hipGetLastError();
}

extern "C" int pck_probe_mfma_bf16_k8(const uint16_t* a, const uint16_t* b, const float* c,
                                      float* d, int64_t tiles, int steps, void* stream) {
  if (!tiles_ok(tiles, steps) || !a || !b || !c || !d) return hipErrorInvalidValue;
  mfma_bf16_k8_kernel<<<dim3(static_cast<unsigned>(tiles)), dim3(kWave), 0,
                        static_cast<hipStream_t>(stream)>>>(a, b, c, d, steps);
  return hipGetLastError();
}

extern "C" int pck_probe_round_up(const double* a, const double* b, double* out, int64_t n,
                                  void* stream) {
  if (n < 0 || (n > 0 && (a == nullptr || b == nullptr || out == nullptr)))
    return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  round_up_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                    static_cast<hipStream_t>(stream)>>>(a, b, out, n);
  return hipGetLastError();
}

extern "C" int pck_probe_round_up_mode(const double* a, const double* b, double* out, int64_t n,
                                       void* stream) {
  if (n < 0 || (n > 0 && (a == nullptr || b == nullptr || out == nullptr)))
    return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  round_up_mode_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                         static_cast<hipStream_t>(stream)>>>(a, b, out, n);
  return hipGetLastError();
}
