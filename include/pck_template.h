/* C ABI of the agent's GEMV templates in libpck_hip.so (gfx950).
 *
 * These are the kernels the checker is run against, not part of the trusted set: the row-major
 * template with its exploit knobs, its INT8-weight variant, the column-major template over
 * W^T, and the INT8 weight copy.  Like every entry point of libpck_hip.so, each only enqueues
 * work on `stream` (a hipStream_t as void*; NULL is the null stream), returns a hipError_t value
 * (0 = hipSuccess) and allocates nothing: outputs, scratch and tickets belong to the caller.
 * All pointers are device pointers to contiguous arrays; x and the weights are BF16 unless
 * stated.
 */
#ifndef PCK_TEMPLATE_H
#define PCK_TEMPLATE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Row-major template, y = W x, W (m, n) BF16, y (m,) FP32.  A workgroup of `threads` lanes
 * (a power of two in [32, 1024]) computes `rows_per_block` rows, so a row has
 * tpr = threads / rows_per_block lanes, which must be a power of two >= 32.  vec in {1, 2, 4, 8}
 * columns per vector, unroll in {1, 2, 4} vectors loaded ahead; flags: 1 accumulator BF16,
 * 2 partials BF16, 4 output BF16, 8 skip the columns past the last full tile of vec * tpr.
 * Vector loads when n % vec == 0 and W, x are aligned to vec elements; the bits are the same
 * either way.  Returns hipErrorInvalidValue for any other knob, m > INT32_MAX or n < 1 (m > 0).
 * Replaces pck::gemv_template, reference src/pck/cuda/csrc/template_kernel.cu:293-298
 * (bound at src/pck/cuda/csrc/bindings.cpp:85-96). */
int pck_gemv_template(const void* W, const void* x, float* y, int64_t m, int64_t n, int threads,
                      int rows_per_block, int vec, int unroll, int flags, void* stream);

/* The row-major template over an INT8 copy of W: Wq (m, n) int8 and S (m, ceil(n / 128)) FP32
 * (from pck_quantize_rows_q8); the term for column j is fl(fl(q_ij S[i, j / 128]) x_j).  The FP32
 * path (no flags); vec may also be 16.
 * Replaces pck::gemv_template_q8, reference src/pck/cuda/csrc/template_kernel.cu:300-306
 * (bound at src/pck/cuda/csrc/bindings.cpp:98-125). */
int pck_gemv_template_q8(const void* Wq, const float* S, const void* x, float* y, int64_t m,
                         int64_t n, int threads, int rows_per_block, int vec, int unroll,
                         void* stream);

/* Row tiles of the column-major template: ceil(m / (32 vec)); -1 for m < 0 or vec not in
 * {2, 4, 8}.  Replaces pck::column_tiles, reference src/pck/cuda/csrc/column_kernel.cu:154. */
int64_t pck_column_tiles(int64_t m, int vec);

/* Column-major template, y = W x from WT = W^T, (n, m) BF16, 16-byte aligned, m % vec == 0.
 * threads = 32 K with K a power of two <= 8; vec in {2, 4, 8}; splits a power of two <= 64;
 * skip_below >= 0 skips (and never reads) every column with |x_j| < skip_below.  With
 * splits > 1, scratch holds splits * m floats and a second launch on `stream` merges them, so
 * calls may overlap when their scratch buffers differ.  `tickets` is not read (the reference
 * merges through zeroed tickets; here the merge is a launch of its own) and may be NULL.
 * Replaces pck::gemv_column, reference src/pck/cuda/csrc/column_kernel.cu:158-184 (bound at
 * src/pck/cuda/csrc/bindings.cpp:127-151). */
int pck_gemv_column(const void* WT, const void* x, float* y, float* scratch, unsigned* tickets,
                    int64_t m, int64_t n, int threads, int vec, int splits, float skip_below,
                    void* stream);

/* The INT8 copy read by pck_gemv_template_q8: W (m, n), BF16 (w_kind 0) or FP32 (w_kind 1) and
 * finite; Wq (m, n) int8; S (m, ceil(n / 128)) FP32.  Per row and group of 128 columns (the last
 * one zero-padded): S = max |w| / 127 (1 for an all-zero group), q = round-half-even(w / S)
 * clipped to [-127, 127], divisions correctly rounded.
 * Replaces pck.agent.config.quantize_rows, a NumPy function in the reference
 * (src/pck/agent/config.py:163-175) called by src/pck/cuda/gemv.py:95-102. */
int pck_quantize_rows_q8(const void* W, int w_kind, int8_t* Wq, float* S, int64_t m, int64_t n,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCK_TEMPLATE_H */
