/* C ABI of libpck_hip.so: the MI355X (gfx950) decode hot path of proof-carrying-kernels.
 *
 * Every entry point only enqueues work on `stream` (a hipStream_t passed as void*; NULL is the
 * device's null stream) and returns a hipError_t value (0 = hipSuccess).  None allocates, frees,
 * synchronises or reads device memory on the host.  All pointers are device pointers to
 * contiguous arrays; the caller owns every buffer (outputs, scratch and banks included).
 *
 * Numerics (what the tests pin):
 *   - the GEMVs reproduce the reference's summation trees bit for bit: lane t of `threads` virtual
 *     lanes sums vectors t, t + threads, ... of 8 (BF16) or 16 (FP8) columns, starting from its
 *     first product with columns past n as +0, then halving within 32-lane virtual warps and
 *     across warp sums (tree height (vec * ceil(ceil(n / vec) / threads) - 1) + log2 threads);
 *   - the checker evaluates rho = c.x - r.y and the threshold tau with every operation of tau
 *     rounded up, and passes a block only if its outputs are finite, tau is finite and
 *     |rho| <= tau;
 *   - the membership check compares logits exactly in FP32 and sums split-argument FP32
 *     softmax terms in FP64.
 */
#ifndef PCK_HIP_H
#define PCK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------
 * GEMV y = W x: W (m, n) row-major, x (n,) BF16, y (m,) FP32.  1 <= threads <= 1024, a power of
 * two (>= 32 for the coalesced kernels).  Vector (16-byte) loads are used when n is a multiple of
 * the vector width and W and x are 16-byte aligned; otherwise element loads with identical bits.
 * -------------------------------------------------------------------------------------------*/

/* BF16 weights, naive tree (contiguous chunk per lane, then neighbour pairs).
 * Replaces pck::gemv_bf16_naive, reference src/pck/cuda/csrc/gemv_kernel.cu:204-211. */
int pck_gemv_bf16_naive(const void* W, const void* x, float* y, int64_t m, int64_t n, int threads,
                        void* stream);

/* BF16 weights, coalesced tree with 8-column vectors.
 * Replaces pck::gemv_bf16_coalesced, reference src/pck/cuda/csrc/gemv_kernel.cu:182-191. */
int pck_gemv_bf16_coalesced(const void* W, const void* x, float* y, int64_t m, int64_t n,
                            int threads, void* stream);

/* OCP FP8 E4M3FN weights (unscaled codes), coalesced tree with 16-column vectors: z = Q x.
 * Replaces pck::gemv_fp8_coalesced, reference src/pck/cuda/csrc/gemv_kernel.cu:193-202. */
int pck_gemv_fp8_coalesced(const void* Q, const void* x, float* z, int64_t m, int64_t n,
                           int threads, void* stream);

#define PCK_MAX_GROUP 8

typedef struct PckGemv {
  const void* W; /* (m, n) BF16 or E4M3FN */
  const void* x; /* (n,) BF16 */
  float* y;      /* (m,) FP32 */
  int64_t m;
  int64_t n;
} PckGemv;

/* Up to PCK_MAX_GROUP independent GEMVs of one weight type in one launch (e.g. q, k and v of a
 * decode layer, which share x).  Each output has exactly the bits of its single-GEMV call.
 * weight_kind: 0 = BF16 (coalesced tree), 1 = FP8 E4M3FN.  No reference counterpart: the
 * reference fuses such GEMVs by concatenating weights (harness/bench_decode_layer.py:48-53);
 * a grouped launch gives the same one-launch cost without the copy. */
int pck_gemv_group(int weight_kind, const PckGemv* gemvs, int count, int threads, void* stream);

struct PckCheckBatch;

/* pck_gemv_group plus the blocked checks of `ride` (NULL: none) in the same launch: the first
 * workgroups of the grid run the checker's per-(check, block) work, the rest the GEMVs.  The
 * checked outputs must come from launches earlier on `stream` (not from this one).  rho, tau
 * and the verdicts are bit-identical to pck_blocked_check(ride); the checker workgroups are
 * separate wavefronts reading y from memory, so a check never trusts the launch it rides in.
 * At threads = 256 with vector loads the checks share the launch; otherwise they run as their
 * own launch just before the GEMVs.  No reference counterpart: it hides the checker launch's
 * fixed latency behind the GEMV stream (the reference's check_many is a separate launch). */
int pck_gemv_group_check(int weight_kind, const PckGemv* gemvs, int count, int threads,
                         const struct PckCheckBatch* ride, void* stream);

/* FP8 grouped launch (optionally with carried checks, as pck_gemv_group_check) whose epilogue
 * also dequantises: for item g, besides z = Q x in gemvs[g].y (the tree's exact bits, which the
 * checker verifies against Q), it writes scaled[g][i] = scales[g][i] * z_i, one FP32 multiply
 * rounded to nearest (the same bits as a separate y = s z).  scales[g] and scaled[g] are (m,)
 * FP32 and must be non-null for every item with rows.  No reference counterpart: the reference
 * applies the row scales of its quantizer (src/pck/cuda/gemv.py:41-58) in a separate op after
 * gemv_fp8. */
int pck_gemv_group_fp8_scaled(const PckGemv* gemvs, const float* const* scales,
                              float* const* scaled, int count, int threads,
                              const struct PckCheckBatch* ride, void* stream);

/* Launch-shape knob of the coalesced kernels at threads = 256, for tuning sweeps: rows per wave
 * slot (1, 2 or 4), vector positions loaded ahead per lane (1, 2 or 4) and non-temporal weight
 * loads (0 or 1); rows_per_wave = 0 restores the built-in choice.  Changes only speed: outputs
 * keep the same bits for every shape.  Process-wide and not thread-safe; no reference
 * counterpart. */
int pck_gemv_set_shape(int rows_per_wave, int unroll, int nontemporal);



/* ---------------------------------------------------------------------------------------------
 * Batched decode product Y (batch, m) FP32 = X (batch, n) BF16 times W^T, W (m, n) BF16
 * (weight_kind 0) or E4M3FN codes (weight_kind 1), on the matrix cores.  Each matrix-core
 * step carries one 8-column chunk with a zero accumulator: pck_bgemm issues
 * v_mfma_f32_32x32x16_bf16 with lanes 0-31 populated, pck_bgemm_packed issues
 * v_mfma_f32_32x32x8_bf16 (its one group of 8 K-slots spread over both lane halves).  Both
 * round RNE_fp32(sum of the 8 exact products, each truncated toward zero to 2^(em - 24),
 * em = max floor(log2|w|) + floor(log2|x|)), as recorded on MI355X by the probe library for
 * each instruction.  Chunk results are summed in FP32: 8 K segments of
 * P = ceil(ceil(n / 8) / 8) chunks; inside a segment, groups of 16 chunks are each summed from
 * -0.0 in chunk order and the group sums added in group order from -0.0; then
 * ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)).  Tree height
 * 9 + min(P, 16) + ceil(P / 16) + 3.
 * No reference counterpart on the hot path: the reference's nearest code is the diagnostic
 * harness/csrc/batched_gemv.cu:25-117 (batch <= 8, FP32 cores).
 * -------------------------------------------------------------------------------------------*/
int pck_bgemm(int weight_kind, const void* W, const void* X, float* Y, int64_t m, int64_t n,
              int64_t batch, void* stream);

/* The same product on operands packed into 32-row tiles, the layout the matrix cores read with
 * one 16-byte load per lane (8 for E4M3FN weights) per two K-steps: step pair p of tile
 * `tile`, lane L = 32 h + l holds row 32 tile + l, columns 16p + 4h .. + 3 then
 * 16p + 8 + 4h .. + 3, at byte ((tile * n / 16 + p) * 64 + L) * Q (Q = 16 for BF16, 8 for
 * E4M3FN); rows past the end are zero.  pck_bgemm_pack writes that layout from (rows, n)
 * row-major (kind 0: BF16, kind 1: E4M3FN; dst holds ceil(rows / 32) * 32 * n elements);
 * weights are packed once at load time, activations per call.  pck_bgemm_packed needs
 * n % 128 == 0, m % 4 == 0 and 16-byte aligned Wp, Xp and Y, and gives the same bits as
 * pck_bgemm.  No reference counterpart. */
int pck_bgemm_pack(int kind, const void* src, void* dst, int64_t rows, int64_t n, void* stream);
int pck_bgemm_packed(int weight_kind, const void* Wp, const void* Xp, float* Y, int64_t m,
                     int64_t n, int64_t batch, void* stream);

/* Tuning knob of pck_bgemm_packed: 32-row weight tiles and 32-row batch tiles per workgroup,
 * (1, 1), (1, 2), (1, 4) or (2, 2); (0, 0) restores the built-in choice.
 * Changes only speed: outputs keep the same bits.  Process-wide and not thread-safe; no
 * reference counterpart. */
int pck_bgemm_set_shape(int rows, int tiles);

/* ---------------------------------------------------------------------------------------------
 * Blocked checksum checker.  Field for field the reference's CheckDesc / CheckBatch
 * (src/pck/cuda/csrc/checker.h:13-44); replaces pck::blocked_check
 * (src/pck/cuda/csrc/checker_kernel.cu:189-196).
 * -------------------------------------------------------------------------------------------*/

#define PCK_MAX_BATCH 8

typedef struct PckCheckDesc {
  const float* c;          /* (K, nb, n) FP32 checksums r^T W_beta                    */
  const void* a;           /* (nb, n) BF16 column sums of |W| per block, rounded up   */
  const int8_t* r;         /* (K, nb, b) secret signs in {-1, +1}                     */
  const void* x;           /* (n,) BF16                                               */
  const float* y;          /* (nb * b,) FP32 output under check                       */
  double* partial_cx;      /* (K, nb, segments) scratch (unused by this kernel)         */
  double* partial_s;       /* (K, nb, segments) scratch (unused by this kernel)         */
  unsigned int* counters;  /* (K, nb) zero on entry; left zero on exit                */
  uint8_t* passed;         /* (K, nb) outputs: bool, rho, tau                         */
  double* rho;
  double* tau;
  int64_t n;
  int64_t seg_len;         /* ceil(n / segments)                                      */
  int32_t block;
  int32_t num_blocks;
  int32_t checks;
  int32_t segments;
  double coef;             /* >= gamma_h + u32, rounded up                            */
  double geps;             /* >= gamma_H(u64) + gamma_2L(u32)^2 + their product       */
  double tau_floor;        /* >= n 2^-148                                             */
} PckCheckDesc;

typedef struct PckCheckBatch {
  PckCheckDesc desc[PCK_MAX_BATCH];
  int64_t start[PCK_MAX_BATCH + 1]; /* work item i belongs to check g if start[g] <= i < start[g+1] */
  int32_t count;                    /* 1 .. PCK_MAX_BATCH */
} PckCheckBatch;

/* One launch checks every described output, one work item (a 256-lane workgroup) per
 * (check, block) pair: start[g + 1] - start[g] = checks * num_blocks.  The scratch fields
 * (partial_cx, partial_s, counters) and `segments` keep the reference's descriptor; the
 * kernel reads and writes neither (counters stay zero).  With more pairs than compute units
 * the launch deals the descriptors in another order (the longest rows where no second-round
 * workgroup joins them); each descriptor's results do not depend on the order. */
int pck_blocked_check(const PckCheckBatch* batch, void* stream);

/* ---------------------------------------------------------------------------------------------
 * In-pass checksums: the blocked check without a bank.  A GEMV launch that also writes, for
 * every output row i, an FP64 pair from the FP32 products p_j = W_ij x_j its tree forms anyway:
 *   d_i  consecutive products added in pairs in FP32, the pair sums widened and added in FP64
 *   s_i  sum_j |p_j| in FP32 (stored widened)
 * Lane l of the row's min(threads, 64) lanes keeps one (d, s) per chain (l, l + 64, ...),
 * from +0, and takes each chain's columns in the tree's own order (vector positions, then the
 * columns of a vector); the chains combine in halving order (chain i += chain i + half), then
 * the lanes by an xor butterfly (offsets 32 .. 1, or 16 .. 1 at threads = 32).  The rows' y
 * keep the bits of pck_gemv_group.
 * A row-sum check then needs only (d, s), y and the signs of each block:
 *   rho = sum_i r_i d_i - sum_i r_i y_i                       FP64, round to nearest
 *   s   = s_factor * sum_i s_i, rounded up, then up to FP32    (s_factor bounds the FP32 sums)
 *   tau = coef s + geps ((1 + u32) s + sum |y_i|) + tau_floor  every operation rounded up
 * and the block passes only if its y are finite, tau is finite and |rho| <= tau: the blocked
 * checker's relation (reference src/pck/cuda/csrc/checker_kernel.cu:115-183) with c . x
 * replaced by r^T (W x) from the pair sums (their FP32 rounding, at most u32 sum |p|, is the
 * budget coef's u32 term gives c's FP32 rounding there) and s = a . |x| by a bound on the exact
 * sum of |W_ij x_j| (the bank's a carries BF16 rounding up to 2^-8 on top).
 * One wave per (check, block) pair: lane l takes rows l, l + 64, ... in order, then an xor
 * butterfly (cx and r.y round to nearest, s and sum |y| round up).  No reference
 * counterpart: the reference always reads a precomputed bank (src/pck/cuda/checker.py:91-104),
 * 2.3% (BF16) / 4.7% (FP8) of the layer's bytes at b = 128.
 * -------------------------------------------------------------------------------------------*/
typedef struct PckRowSumCheckDesc {
  const double* sums; /* (nb * b, 2) FP64 (d_i, s_i), 16-byte aligned                    */
  const float* y;     /* (nb * b,) FP32 output under check                               */
  const int8_t* r;    /* (K, nb, b) secret signs in {-1, +1}                             */
  uint8_t* passed;    /* (K, nb) outputs: bool, rho, tau                                 */
  double* rho;
  double* tau;
  int32_t block;
  int32_t num_blocks;
  int32_t checks;
  int32_t reserved;   /* 0 */
  double coef;        /* >= gamma_h + u32, rounded up                                    */
  double geps;        /* >= gamma_H(u64), H >= D + ceil(b / 64) + 7                      */
  double tau_floor;   /* >= n 2^-148 + 2 b n 2^-150 (FP32 product underflow)             */
  double s_factor;    /* >= 1 / (1 - gamma_D(u32)), D >= the row sums' depth: the max    */
                      /* over threads T and vector width V of                             */
                      /* (T / min(T, 64)) ceil(ceil(n / V) / T) V + log2 min(T, 64)       */
} PckRowSumCheckDesc;

typedef struct PckRowSumBatch {
  PckRowSumCheckDesc desc[PCK_MAX_BATCH];
  int64_t start[PCK_MAX_BATCH + 1]; /* work item i belongs to check g if start[g] <= i < start[g+1] */
  int32_t count;                    /* 0 .. PCK_MAX_BATCH (0: no checks) */
} PckRowSumBatch;

/* pck_gemv_group plus the row sums: sums[g] is GEMV g's (m, 2) FP64 output, 16-byte aligned.
 * `ride` (NULL: none) holds row-sum checks of outputs that launches earlier on `stream`
 * produced; their waves run in the first workgroups of the grid (one wave per (check, block)
 * pair), and their results are bit-identical to pck_rowsum_check(ride). */
int pck_gemv_group_rowsums(int weight_kind, const PckGemv* gemvs, double* const* sums, int count,
                           int threads, const PckRowSumBatch* ride, void* stream);

/* The row-sum checks of `batch` as one launch (four pairs per 256-lane workgroup). */
int pck_rowsum_check(const PckRowSumBatch* batch, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Blocked checker for a batch of activation rows (Y = X W^T, B >= 1): every column of Y is
 * checked as pck_blocked_check checks one GEMV output, against the same bank, signs and
 * constants (rho = c . X[b] - r . Y[b, beta rows] in FP64; tau as for pck_blocked_check with
 * s = a . |X[b]| bounded above, at most a factor 1 + 2^-15 over the exact value for
 * normal-range inputs, and rounded up to FP32).  Outputs (K, nb, batch): index
 * (k * nb + beta) * batch + b.  One launch checks up to PCK_MAX_BATCH outputs (a whole decode
 * layer).  The reference checks one vector per descriptor (checker_kernel.cu:87-196); this is
 * that check for every column, reading the bank once.
 * -------------------------------------------------------------------------------------------*/
typedef struct PckBatchCheckDesc {
  const float* c;      /* (K, nb, n) FP32 checksums r^T W_beta                    */
  const void* a;       /* (nb, n) BF16 column sums of |W| per block, rounded up   */
  const int8_t* r;     /* (K, nb, b) secret signs in {-1, +1}                     */
  const void* X;       /* (batch, n) BF16                                         */
  const float* Y;      /* (batch, nb * b) FP32 outputs under check                */
  uint8_t* passed;     /* (K, nb, batch)                                          */
  double* rho;         /* (K, nb, batch)                                          */
  double* tau;         /* (K, nb, batch)                                          */
  int64_t n;           /* columns of W, at most 2^20                              */
  int64_t block;
  int64_t num_blocks;
  int64_t checks;
  int64_t batch;
  double coef;
  double geps;
  double tau_floor;
} PckBatchCheckDesc;

/* Two launches (matrix-core partial sums per K segment; then a launch that reads the outputs
 * and adds the segments in a fixed order) with a caller-allocated workspace of
 * pck_batch_check_workspace bytes (8-byte aligned); the library allocates nothing.  The
 * workspace is not shared between calls that overlap.  Needs n % 8 == 0, block % 4 == 0,
 * c, a, X, Y 16-byte and r 4-byte aligned, and coef, geps, tau_floor finite and >= 0; the
 * kernels address with 32-bit byte offsets, so each output needs nb * b * 256 < 2^31 (fewer
 * than 2^23 rows) and each of the workspace's two partial arrays stays below 2^31 bytes;
 * otherwise hipErrorInvalidValue before anything is enqueued. */
int pck_batch_check_workspace(const PckBatchCheckDesc* descs, int count, int64_t* bytes);
int pck_batch_check(const PckBatchCheckDesc* descs, int count, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* pck_batch_check without a caller workspace and without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc).  The partial sums go to a file-scope device
 * array of pck_batch_check_static_bytes() bytes (16 MiB), one per GPU the library runs on,
 * held until the process ends.  Its address on a device is looked up once, by
 * pck_batch_check_static_init() called with that device current, or else by the first
 * pck_batch_check_static call with that device current.  The lookup is a HIP runtime call
 * (hipGetSymbolAddress), so a caller whose first call on a device may be under HIP graph
 * capture calls pck_batch_check_static_init() on that device beforehand, outside the capture;
 * after that no call makes a runtime call other than its two kernel launches.  init returns a
 * hipError_t and may be called again (it then does nothing).  A plan that needs more than that
 * returns hipErrorOutOfMemory
 * (a Llama-3-8B decode layer needs 6.5 MiB at batch 128 or 256); invalid descriptors return
 * hipErrorInvalidValue as for pck_batch_check; in both cases nothing is enqueued.  Every
 * call on one GPU shares its array: calls that overlap on one GPU (different streams, or
 * different host threads) race.  Nothing in the array needs clearing between calls. */
int64_t pck_batch_check_static_bytes(void);
int pck_batch_check_static_init(void);
int pck_batch_check_static(const PckBatchCheckDesc* descs, int count, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Sampled-token membership check for a batch of rows (top-k / top-p / greedy), the native
 * kernel behind pck.member.check_members (reference src/pck/member.py:118-197).
 *   logits (rows, vocab) FP32, 1 <= vocab < 2^31; tokens (rows,) int64 (any value:
 *   out-of-range ids reject);
 *   top_k (rows,) int64 or NULL (clamped to [1, vocab] here; vocab = no top-k);
 *   top_p (rows,) FP64 or NULL (1 = no top-p); greedy (rows,) uint8 or NULL;
 *   slack = next_up(tol + member_eps32(vocab)) from the host;
 *   k_lim = largest host-side top-k below vocab (0 if none); all_k = every host top-k < vocab;
 *   outputs ok (rows,) uint8, above (rows,) int64, mass_above (rows,) FP64.
 * -------------------------------------------------------------------------------------------*/
int pck_check_members(const float* logits, int64_t rows, int64_t vocab, const int64_t* tokens,
                      const int64_t* top_k, const double* top_p, const uint8_t* greedy,
                      double slack, int64_t k_lim, int all_k, uint8_t* ok, int64_t* above,
                      double* mass_above, void* stream);

/* The same check with the options a sampler hook needs in one launch (the reference's plugin
 * builds these with torch ops around its check, src/pck/vllm_plugin.py:146-186):
 *   top_p            FP64, or FP32 when top_p_fp32 = 1 (widened exactly), or NULL;
 *   temperature      (temperature_count,) FP32 with temperature_index (rows,) int64: row r is
 *                    greedy iff temperature[temperature_index[r]] == 0 (vLLM's per-request
 *                    sampling state); a row whose index lies outside [0, temperature_count)
 *                    is rejected (ok = 0, counted as rejected) and the array is not read for
 *                    it; NULL: greedy as in pck_check_members (temperature_count unused);
 *   injected         (rows,) uint8 faults the caller planted, or NULL;
 *   ok, above, mass_above   outputs as in pck_check_members; each may be NULL;
 *   totals           NULL, or 6 words the kernel adds each row into (64-bit atomics):
 *                    [0] rows, [1] rejected, [2] injected, [3] rejected and injected,
 *                    [4] rejected and not injected, [5] maximum of K(r - p) over accepted,
 *                    non-greedy rows with p < 1, where K is the order-preserving key of an FP64
 *                    value v: bits(v) | 2^63 for v >= 0, ~bits(v) for v < 0.  The caller
 *                    initialises the buffer (word 5 to K(-1) for "none yet") and may keep
 *                    adding to it across calls.
 * No reference counterpart as a native entry; pck_check_members is this with every option
 * off. */
typedef struct PckMemberArgs {
  const float* logits;
  int64_t rows;
  int64_t vocab;
  const int64_t* tokens;
  const int64_t* top_k;
  const void* top_p;
  const uint8_t* greedy;
  const float* temperature;
  const int64_t* temperature_index;
  int64_t temperature_count;
  const uint8_t* injected;
  double slack;
  int64_t k_lim;
  int32_t all_k;
  int32_t top_p_fp32;
  uint8_t* ok;
  int64_t* above;
  double* mass_above;
  unsigned long long* totals;
} PckMemberArgs;

int pck_check_members_ex(const PckMemberArgs* args, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Set-sampling checker (top-k / top-p): is sel[b, 0 .. len[b]) a valid top-k set (top_p = 0,
 * length k) or a valid minimal top-p nucleus (top_p = 1) of row b of logits (rows, vocab) FP32?
 * Replaces pck::sampling_check (reference src/pck/cuda/csrc/sampling_kernel.cu:211-229) with
 * the same arguments and outputs:
 *   passed (rows,) uint8; min_selected, max_rejected (rows,) FP32, exact; mass and
 *   mass_without_smallest (rows,) FP64 (0 unless top-p and the set checks passed).
 * slack is the host's: the sampler's declared error plus this kernel's own rounding.
 * lengths (rows,) int64, or NULL: every row's selection is all max_len entries (a top-k call;
 * the reference passes a tensor filled with k).
 * scratch: rows * pck_sampling_scratch_words(vocab) uint32, zero on entry (the caller zeroes it;
 * it holds the selection bitmaps and a malformed flag per row), needed only when
 * pck_sampling_needs_scratch(vocab, max_len, segments) returns 1 (selections longer than 4096,
 * or segments of more than 2^18 logits); otherwise it may be NULL and the segment workgroups
 * build their bitmaps in LDS.  partials: rows * segments * pck_sampling_partial_bytes(),
 * 8-byte aligned.  1 <= segments <= vocab, rows <= 65535, temperature > 0, slack >= 0.
 * Launches: (mark,) segment, finish.  pck_sampling_needs_scratch has no reference counterpart:
 * the reference always builds the bitmap in zeroed global scratch.
 * -------------------------------------------------------------------------------------------*/
int pck_sampling_needs_scratch(int64_t vocab, int64_t max_len, int64_t segments);
int64_t pck_sampling_scratch_words(int64_t vocab);
int64_t pck_sampling_partial_bytes(void);
int pck_sampling_check(const float* logits, const int64_t* selected, const int64_t* lengths,
                       int64_t rows, int64_t vocab, int64_t max_len, int64_t k, int top_p,
                       double p, double temperature, double slack, int64_t segments,
                       uint32_t* scratch, void* partials, uint8_t* passed, float* min_selected,
                       float* max_rejected, double* mass, double* mass_without_smallest,
                       void* stream);

/* Measurement: reads `bytes` (a multiple of 16, 16-byte aligned) from `src`, workgroup g of
 * `groups` (256 lanes, 4 waves each) one contiguous chunk of ceil(bytes / 16 / groups) 16-byte
 * vectors rounded up to a multiple of 2048, and stores one word per wave into sink[4 * groups]
 * (their XOR is the XOR of every 32-bit word read).  The practical HBM read ceiling for the GEMV
 * roofline (use 64 KiB per workgroup); no reference counterpart (the reference measures a
 * device-to-device copy, src/pck/cuda/timing.py:50-55). */
int pck_read_stream(const void* src, int64_t bytes, uint32_t* sink, int groups, void* stream);

/* Text for a value returned by any entry point. */
const char* pck_error_string(int err);

#ifdef __cplusplus
}
#endif

#endif /* PCK_HIP_H */
