// Read-only streaming kernel: the practical HBM read ceiling the GEMV bandwidth is compared with.
//
// Workgroup g reads one contiguous chunk of 16-byte vectors (ceil(vectors / groups) rounded up to
// whole passes of 2048 vectors, so trailing workgroups may read nothing); each lane
// keeps eight non-temporal loads in flight (lane t reads vectors t, t + 256, ... of the chunk)
// and folds them with XOR; each wave stores one value, so the loads cannot be removed and no
// wave waits for another at the end.
// Contiguous 64 KiB chunks per workgroup measured fastest on MI355X (7.13 TB/s over 2 GiB, against
// 5.8 TB/s for a grid-stride walk).  No reference counterpart: the reference compares with a
// device-to-device copy (read + write, src/pck/cuda/timing.py:50-55), which on MI355X understates
// a read-only stream.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pck_hip.h"

namespace pck {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
    read_stream_kernel(const uint4* __restrict__ src, int64_t vectors, int64_t per_group,
                       uint32_t* __restrict__ sink) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* base = reinterpret_cast<const u32x4*>(src);
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * per_group;
  const int64_t hi = lo + per_group < vectors ? lo + per_group : vectors;
  uint32_t acc = 0;
  constexpr int kAhead = 8;
  int64_t i = lo + threadIdx.x;
  for (; i + (kAhead - 1) * kThreads < hi; i += kAhead * kThreads) {
    u32x4 v[kAhead];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) v[k] = __builtin_nontemporal_load(base + i + k * kThreads);
#pragma unroll
    for (int k = 0; k < kAhead; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  for (; i < hi; i += kThreads) {
    const u32x4 a = base[i];
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  for (int off = 32; off > 0; off /= 2) acc ^= __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0)
    sink[static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64] = acc;
}

}  // namespace
}  // namespace pck

extern "C" int pck_read_stream(const void* src, int64_t bytes, uint32_t* sink, int groups,
                               void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || groups < 1 ||
      reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return hipErrorInvalidValue;
  const int64_t vectors = bytes / 16;
  // whole passes of the unrolled loop per chunk: a ragged chunk would leave a few lanes of every
  // workgroup in the one-load-at-a-time tail loop (about 2 us per launch)
  constexpr int64_t kPass = 8 * pck::kThreads;
  const int64_t per_group = ((vectors + groups - 1) / groups + kPass - 1) / kPass * kPass;
  pck::read_stream_kernel<<<dim3(static_cast<unsigned>(groups)), dim3(pck::kThreads), 0,
                            static_cast<hipStream_t>(stream)>>>(static_cast<const uint4*>(src),
                                                                vectors, per_group, sink);
  return hipGetLastError();
}
