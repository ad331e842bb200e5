// Read-only streaming kernel: the practical HBM read ceiling the GEMV bandwidth is compared with.
//
// Every lane reads 16-byte vectors in a grid-stride loop (four in flight per iteration) and folds
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
  for (; i + 3 * stride < vectors; i += 4 * stride) {
    const uint4 a = src[i];
    const uint4 b = src[i + stride];
    const uint4 c = src[i + 2 * stride];
    const uint4 d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    acc ^= c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
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
