/* TEST INFRASTRUCTURE — scalar C restatement of the GEMV summation trees.
 *
 * An independent, loop-by-loop model of the kernels' trees, written without the reshapes of
 * oracle/gemv.py, so that tests can cross-check the two restatements bit for bit (the role
 * `loop_reference_coalesced` plays in the reference's tests/test_gemv.py:93-122).  It is
 * also the all-core CPU baseline that bench.py times beside the GPU.
 *
 * Trees (reference src/pck/gemv.py:14-101, src/pck/cuda/csrc/gemv_kernel.cu:27-178):
 *   coalesced: lane t of `threads` sums vectors t, t + threads, ... of `vec` columns in
 *              column order (first product as the start value, columns past n are +0), then
 *              halving within each 32-lane warp, then halving across warp sums;
 *   naive:     lane t sums the contiguous chunk [t c, (t + 1) c), c = ceil(n / threads),
 *              then a pairwise tree (stride 1, 2, 4, ...).
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast math, so every float
 * operation is one IEEE round-to-nearest SSE operation with subnormals kept).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WARP 32

static void halve(float* a, int len) {
  for (int half = len / 2; half > 0; half /= 2) {
    for (int i = 0; i < half; ++i) a[i] = a[i] + a[i + half];
  }
}

/* y[i] = row i of W (m x n, row-major, values already rounded to the kernel's input type)
 * times x, in the coalesced kernel's order.  threads is a power of two >= 32, vec >= 1. */
void oracle_gemv_coalesced(const float* W, const float* x, float* y, int64_t m, int64_t n,
                           int threads, int vec) {
  const int64_t vectors = (n + vec - 1) / vec;
  const int64_t per_lane = (vectors + threads - 1) / threads;
#pragma omp parallel
  {
    float* lane = (float*)malloc(sizeof(float) * (size_t)threads);
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      const float* row = W + i * n;
      for (int t = 0; t < threads; ++t) {
        float acc = 0.0f;
        int first = 1;
        for (int64_t v = 0; v < per_lane; ++v) {
          const int64_t base = (v * threads + t) * (int64_t)vec;
          for (int k = 0; k < vec; ++k) {
            const int64_t j = base + k;
            const float p = j < n ? row[j] * x[j] : 0.0f;
            if (first) {
              acc = p;
              first = 0;
            } else {
              acc = acc + p;
            }
          }
        }
        lane[t] = acc;
      }
      for (int w = 0; w < threads / WARP; ++w) {
        halve(lane + w * WARP, WARP);
        lane[w] = lane[w * WARP]; /* warp sums move to the front, in warp order */
      }
      halve(lane, threads / WARP);
      y[i] = lane[0];
    }
    free(lane);
  }
}

/* The naive kernel's order: contiguous chunks, then a neighbour-pair tree. */
void oracle_gemv_naive(const float* W, const float* x, float* y, int64_t m, int64_t n,
                       int threads) {
  const int64_t chunk = (n + threads - 1) / threads;
#pragma omp parallel
  {
    float* lane = (float*)malloc(sizeof(float) * (size_t)threads);
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      const float* row = W + i * n;
      for (int t = 0; t < threads; ++t) {
        const int64_t begin = t * chunk;
        float acc = begin < n ? row[begin] * x[begin] : 0.0f;
        for (int64_t j = begin + 1; j < begin + chunk; ++j) {
          acc = acc + (j < n ? row[j] * x[j] : 0.0f);
        }
        lane[t] = acc;
      }
      for (int stride = 1; stride < threads; stride *= 2) {
        for (int t = 0; t + stride < threads; t += 2 * stride) lane[t] = lane[t] + lane[t + stride];
      }
      y[i] = lane[0];
    }
    free(lane);
  }
}
