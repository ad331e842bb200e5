/* Probes of device arithmetic (libpck_probe.so).  No counterpart in the reference: the
 * reference's error bounds assume a device expf within 2 ulp (src/pck/member.py:84-102), and
 * this build's batched kernels assume properties of the gfx950 matrix cores; these entry
 * points let tests measure both.  Nothing in the product calls them.
 *
 * Operands are in lane order (no matrix layout is built in): for tile t < tiles and step
 * s < steps, lane l < 64 reads A and B at element [(t * steps + s) * 64 + l] (one FP64 value,
 * or 8 or 4 BF16 values given as their 16-bit patterns) and its accumulator registers at
 * [t * 64 + l] (4 FP64, 16 or 4 FP32 values); after the last step it writes its result
 * registers to D at the same place.  1 <= tiles <= 2^20 and 1 <= steps <= 64, else
 * hipErrorInvalidValue before anything is enqueued.  Returns a hipError_t. */
#ifndef PCK_PROBE_H
#define PCK_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[i] = expf(x[i]) for i < n, compiled as the membership and sampling kernels compile it. */
int pck_probe_expf(const float* x, float* y, int64_t n, void* stream);

/* Chains of v_mfma_f64_16x16x4_f64: a, b (tiles * steps * 64) doubles, c, d (tiles * 64 * 4). */
int pck_probe_mfma_f64(const double* a, const double* b, const double* c, double* d,
                       int64_t tiles, int steps, void* stream);

/* Chains of v_mfma_f32_32x32x16_bf16: a, b (tiles * steps * 64 * 8) BF16 patterns, c, d
 * (tiles * 64 * 16) floats. */
int pck_probe_mfma_bf16(const uint16_t* a, const uint16_t* b, const float* c, float* d,
                        int64_t tiles, int steps, void* stream);

/* Chains of v_mfma_f32_16x16x32_bf16: a, b as above, c, d (tiles * 64 * 4) floats. */
int pck_probe_mfma_bf16_16x16(const uint16_t* a, const uint16_t* b, const float* c, float* d,
                              int64_t tiles, int steps, void* stream);

/* Chains of v_mfma_f32_32x32x8_bf16 (the batched product's instruction): a, b (tiles * steps *
 * 64 * 4) BF16 patterns, 4 per lane (lane l + 32 h holds row / column l, K-slots 4h .. 4h + 3),
 * c, d (tiles * 64 * 16) floats. */
int pck_probe_mfma_bf16_k8(const uint16_t* a, const uint16_t* b, const float* c, float* d,
                           int64_t tiles, int steps, void* stream);

/* The checkers' directed roundings (csrc/rounding.h) for n pairs: out[4 i .. 4 i + 3] =
 * mul_up(a[i], b[i]), mul_up_pos(a[i], b[i]), add_up(a[i], b[i]), add_up_nonneg(a[i], b[i]).
 * The branch-free forms are meant for non-negative operands, where they must give the
 * general forms' bits. */
int pck_probe_round_up(const double* a, const double* b, double* out, int64_t n, void* stream);

/* The checkers' in-hardware upward sums (csrc/rounding.h add_up_rm2 / add_up_rm4, one add each
 * under the wave's round-toward-+inf mode) for n pairs: out[3 i] and out[3 i + 1] = RU(a[i] +
 * b[i]) from each form; out[3 i + 2] = an ordinary add issued after them, RN(a[i] + b[i]) when
 * the forms leave the rounding mode as they found it. */
int pck_probe_round_up_mode(const double* a, const double* b, double* out, int64_t n,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCK_PROBE_H */
