// Read-only streaming kernel: the practical HBM read ceiling the GEMV bandwidth is compared with.
//
// Every lane reads 16-byte vectors in a grid-stride loop (eight non-temporal loads in flight per iteration) and folds
// them with XOR; one value per workgroup is stored so the loads cannot be removed.  No reference
// counterpart: the reference compares with a device-to-device copy (read + write,
// src/pck/cuda/timing.py:50-55), which on MI355X understates a read-only stream.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"

namespace pck {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
    read_stream_kernel(const uint4* __restrict__ src, int64_t vectors, uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  constexpr int kAhead = 8;
  for (; i + (kAhead - 1) * stride < vectors; i += kAhead * stride) {
    uint4 v[kAhead];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + i + k * stride));
      v[k] = make_uint4(w[0], w[1], w[2], w[3]);
    }
#pragma unroll
    for (int k = 0; k < kAhead; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < vectors; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  for (int off = 32; off > 0; off /= 2) acc ^= __shfl_xor(acc, off, 64);
  __shared__ uint32_t waves[kThreads / 64];
  if ((threadIdx.x & 63) == 0) waves[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = waves[0] ^ waves[1] ^ waves[2] ^ waves[3];
}

}  // namespace
}  // namespace pck

extern "C" int pck_read_stream(const void* src, int64_t bytes, uint32_t* sink, int groups,
                               void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || groups < 1 ||
      reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return hipErrorInvalidValue;
  pck::read_stream_kernel<<<dim3(static_cast<unsigned>(groups)), dim3(pck::kThreads), 0,
                            static_cast<hipStream_t>(stream)>>>(static_cast<const uint4*>(src),
                                                                bytes / 16, sink);
  return hipGetLastError();
}
