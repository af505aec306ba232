/*
 * torchpairwise_amd — C ABI of the gfx950 (MI355X) pairwise-metric kernels.
 *
 * The reference (inspiros/torchpairwise v0.3.0) exposes its kernels only through
 * PyTorch dispatcher registrations (TORCH_LIBRARY_IMPL(torchpairwise, CPU/CUDA, m));
 * it has no C ABI of its own.  Each entry point below replaces one of those
 * registered L1 kernels (the reference file:line is given beside it), with plain
 * device pointers and sizes instead of at::Tensor, so that any host language can
 * bind it.  The PyTorch extension in torchpairwise_amd/csrc/ops is one such host;
 * ctypes (tests) is another.
 *
 * Conventions shared by every entry point:
 *   - all pointers are device pointers (HBM) unless stated otherwise;
 *   - tensors are dense and row-major: x1 is [batch, n, d], x2 is [batch, m, d],
 *     pairwise outputs are [batch, n, m];
 *   - `stream` is a hipStream_t (NULL = the null stream); work is only enqueued,
 *     nothing synchronises;
 *   - the return value is TPW_OK or an error code; tpw_last_error() gives the
 *     message of the last failure on the calling thread.
 *   - no entry point allocates device memory; scratch memory, where a kernel needs
 *     it, is passed in by the caller (its size is given by a *_workspace_size call).
 */
#ifndef TORCHPAIRWISE_AMD_H_
#define TORCHPAIRWISE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TPW_OK 0
#define TPW_ERR_INVALID 1 /* bad argument (shape, dtype, alignment, null pointer) */
#define TPW_ERR_LAUNCH 2  /* the HIP runtime rejected a launch */

/* element types (TPW_F32 / TPW_BF16 for the floating-point kernels; all of them for
 * tpw_compare_reduce) */
#define TPW_F32 0
#define TPW_BF16 1
#define TPW_F16 2
#define TPW_F64 3
#define TPW_I8 4
#define TPW_U8 5
#define TPW_I16 6
#define TPW_I32 7
#define TPW_I64 8

/* Message of the last failed call on this thread ("" if none). */
const char *tpw_last_error(void);

/* HIP runtime version the library was built against, as hipRuntimeGetVersion
 * reports it.  Replaces `_cuda_version()` (torchpairwise/csrc/torchpairwise.cpp:28-40),
 * which returned CUDA_VERSION or -1. */
int tpw_runtime_version(void);

/* Launch timer (measurement support; no counterpart in the reference).  Arms HIP event
 * pairs around every launch of one kernel family ("inner_tile_kernel",
 * "pairwise_inner_kernel", "lp_forward_kernel", "bool_reduce_kernel",
 * "bool_bits_tile_kernel") made on the current device, at most `capacity` launches (later ones
 * are counted as dropped).  Events are recorded on the stream each launch goes to, so a caller
 * reads the device duration of the launches inside its own timed loop.  Creates events the
 * first time (no device memory).  Not for concurrent use from several threads. */
int tpw_launch_timer_arm(const char *family, int capacity);
/* Disarms the timer, waits for the recorded events and writes the first min(count,
 * capacity) launch durations in ms to ms[]; *count = launches recorded, *dropped (may be
 * NULL) = launches past the armed capacity. */
int tpw_launch_timer_read(float *ms, int capacity, int *count, int *dropped);

/* Launches `count` empty kernels (one wave each) back to back on `stream` (measurement
 * support; no counterpart in the reference): the floor a chain of that many dependent launches
 * costs on the device, against which a multi-launch operation can be measured. */
int tpw_empty_launches(int count, void *stream);

/* ------------------------------------------------------------------------- */
/* Bit-packed boolean family (hamming, jaccard, pw*_sum / pw*_mean on bool)   */
/* ------------------------------------------------------------------------- */

/* binary ops of the reference's common/binary_ops.h:9-20 that act on bool */
#define TPW_BIT_AND 0
#define TPW_BIT_OR 1
#define TPW_BIT_XOR 2
#define TPW_BIT_EQ 3
#define TPW_BIT_NE 4
/* the ordering comparisons of the same header (tpw_pairwise_binary only) */
#define TPW_CMP_LT 5
#define TPW_CMP_GT 6
#define TPW_CMP_LE 7
#define TPW_CMP_GE 8
/* reductions of common/reduction_ops.h:8-12 that produce float32 */
#define TPW_RED_SUM 0
#define TPW_RED_MEAN 1

/* Number of uint32 words per packed row of `d` booleans: ceil(d/32) rounded up
 * to a multiple of 4 so that rows are 16-byte aligned.  Padding bits are zero. */
int64_t tpw_packed_words(int64_t d);

/* Pack `rows` rows of `d` bool bytes (0/1, torch.bool layout) into
 * rows x tpw_packed_words(d) uint32 words, bit k of row r at word k/32, bit k%32.
 * If `row_popcounts` is not NULL it receives the number of set bits of each row.
 * Replaces the bool-byte input path of pairwise_binary_reduction_forward_kernel
 * (csrc/ops/cuda/pairwise_binary_kernels.cu:144-220), which read the bytes
 * directly for every output. */
int tpw_pack_bool_rows(const uint8_t *x, int64_t rows, int64_t d, uint32_t *words,
                       int32_t *row_popcounts, void *stream);

/* out[b,i,j] = reduction_k op(x1[b,i,k], x2[b,j,k]) over packed rows, as float32.
 * `op` is a TPW_BIT_* code, `reduction` TPW_RED_SUM (count) or TPW_RED_MEAN
 * (count / d).  Counts are exact integers; the result is the reference's float
 * accumulator (exact below 2^24, saturating at 2^24) and its `val /= d`.
 * Replaces pairwise_binary_reduction_forward_kernel<op, Sum|Mean> for bool inputs
 * (csrc/ops/cuda/pairwise_binary_kernels.cu:32-53,144-220;
 *  CPU: csrc/ops/cpu/pairwise_binary_kernels.cpp:28-49,118-171).
 * hamming_distances on bool is (TPW_BIT_NE, TPW_RED_MEAN)
 * (csrc/ops/pairwise_metrics.cpp:206-213). */
int tpw_bool_pairwise_reduce(const uint32_t *x1_words, const uint32_t *x2_words,
                             int64_t batch, int64_t n, int64_t m, int64_t d, int op,
                             int reduction, float *out, void *stream);

/* The same reduction given the rows' popcounts (tpw_pack_bool_rows' row_popcounts):
 * for rows of more than 256 features every op's count follows from the AND count
 * and the popcounts (or = pa + pb - and, xor = ne = pa + pb - 2 and,
 * eq = d - xor), which the matrix cores form; results equal
 * tpw_bool_pairwise_reduce's bit for bit.  Replaces the same reference kernels
 * (csrc/ops/cuda/pairwise_binary_kernels.cu:32-53,144-220). */
int tpw_bool_pairwise_reduce_counted(const uint32_t *x1_words, const uint32_t *x2_words,
                                     const int32_t *x1_popcounts, const int32_t *x2_popcounts,
                                     int64_t batch, int64_t n, int64_t m, int64_t d, int op,
                                     int reduction, float *out, void *stream);

/* jaccard_distances on bool: out = prf_div(xor_count, or_count, "zero"), i.e.
 * or == 0 ? 0 : fl32(xor) / fl32(or), from AND counts and row popcounts
 * (xor = pa + pb - 2 and, or = pa + pb - and).  Replaces the three passes
 * pwxor_sum + pwor_sum + prf_div of csrc/ops/pairwise_metrics.cpp:215-222. */
int tpw_jaccard_bool(const uint32_t *x1_words, const uint32_t *x2_words,
                     const int32_t *x1_popcounts, const int32_t *x2_popcounts,
                     int64_t batch, int64_t n, int64_t m, int64_t d, float *out,
                     void *stream);

/* Kernel functions of tpw_pairwise_kernel (POLYNOMIAL, SIGMOID) and tpw_pairwise_exp_kernel
 * (RBF, LAPLACIAN) */
#define TPW_KER_POLYNOMIAL 0
#define TPW_KER_SIGMOID 1
#define TPW_KER_RBF 2
#define TPW_KER_LAPLACIAN 3

/* out = (x1 . x2^T * gamma + coef0)^degree (POLYNOMIAL) or tanh(x1 . x2^T * gamma + coef0)
 * (SIGMOID) on the MFMA kernel, the function applied to the fp32 accumulators before the one
 * write of out.  Replaces the matmul + mul_ + add_ + pow_ / tanh_ passes of polynomial_kernel
 * and sigmoid_kernel (pairwise_metrics.cpp:67-78,80-90); degree k = 2, 3 as products, otherwise
 * powf, as ATen's pow with a scalar exponent.  dtype TPW_F32 or TPW_BF16. */
int tpw_pairwise_kernel(const void *x1, const void *x2, int dtype, int64_t batch, int64_t n,
                        int64_t m, int64_t d, int kind, float gamma, float coef0, int degree,
                        void *out, void *stream);

/* Gradients of tpw_pairwise_kernel, the autograd of the reference's composite: the per-pair
 * weight grad * degree * (S gamma + coef0)^(degree - 1) * gamma (S recomputed on the MFMA
 * path) or grad * (1 - out^2) * gamma, then grad_x1 = W . x2, grad_x2 = W^T . x1 on the
 * matrix cores.  Workspace: tpw_inner_backward_workspace_size(batch, n, m, d) bytes; `out`
 * (the forward result) is needed for SIGMOID. */
int tpw_pairwise_kernel_backward(const void *grad, const void *x1, const void *x2,
                                 const void *out, int dtype, int64_t batch, int64_t n, int64_t m,
                                 int64_t d, int kind, float gamma, float coef0, int degree,
                                 void *grad_x1, void *grad_x2, void *workspace, void *stream);

/* out = exp(-gamma * sum_k (x1 - x2)^2) (RBF, the reference's sqeuclidean = _ppminkowski
 * p = 2, then mul_(-gamma).exp_()) or exp(-gamma * sum_k |x1 - x2|) (LAPLACIAN, cdist p = 1)
 * on the VALU tile kernel with the exponential in its epilogue: one write of out instead of
 * three passes.  fp32 [batch, n, d] x [batch, m, d].  Replaces rbf_kernel / laplacian_kernel
 * (pairwise_metrics.cpp:92-110); their gradients are the reference's exp backward (grad * out
 * * -gamma) fed to the _ppminkowski / cdist p = 1 backward entry points above. */
int tpw_pairwise_exp_kernel(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                            int64_t d, int kind, float gamma, float *out, void *stream);

/* grad_x1 [batch, n, d] and grad_x2 [batch, m, d] of tpw_pairwise_exp_kernel's out, given the
 * upstream grad and that out (fp32 [batch, n, m]).  Each pair's gradient of the distance is
 * (grad * out) * (-gamma), the reference's exp_ backward and then mul_(-gamma)'s, one rounding
 * each, followed by the _ppminkowski p = 2 (RBF) or cdist p = 1 (LAPLACIAN) backward.  It is
 * formed while the backward kernel stages its pairs (no N x M array written): RBF always,
 * LAPLACIAN where d > 64 and n, m, d are multiples of 4 with 16-byte aligned arrays (elsewhere
 * one elementwise pass into the workspace, one N x M write instead of two).  Results equal those
 * two ATen multiplies followed by tpw_ppminkowski_backward (p = 2) or tpw_lp_distances_backward2
 * (p = 1) bit for bit.  workspace: tpw_pairwise_exp_kernel_backward_workspace_size(kind, ...)
 * bytes.  Replaces the autograd chain of the reference's rbf_kernel / laplacian_kernel
 * composites (pairwise_metrics.cpp:92-110): the backward of exp_ and mul_, then
 * _ppminkowski_backward (ppminkowski_kernel.cpp:125-160) or PyTorch's _cdist_backward. */
size_t tpw_pairwise_exp_kernel_backward_workspace_size(int kind, int64_t batch, int64_t n, int64_t m,
                                                       int64_t d);
int tpw_pairwise_exp_kernel_backward(const float *grad, const float *out, const float *x1,
                                     const float *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                                     int kind, float gamma, float *grad_x1, float *grad_x2,
                                     void *workspace, void *stream);

/* Boolean count metrics of tpw_bool_count_metric */
#define TPW_BMET_HAMMING 0
#define TPW_BMET_JACCARD 1
#define TPW_BMET_DICE 2
#define TPW_BMET_KULCZYNSKI1 3
#define TPW_BMET_KULSINSKI 4
#define TPW_BMET_ROGERSTANIMOTO 5
#define TPW_BMET_RUSSELLRAO 6
#define TPW_BMET_SOKALMICHENER 7
#define TPW_BMET_SOKALSNEATH 8
#define TPW_BMET_YULE 9

/* One pass for any boolean count metric of packed rows with their popcounts (both from
 * tpw_pack_bool_rows): the tile counts and = popcount(a & b) per pair; xor = pa + pb - 2 and,
 * or = pa + pb - and, eq = d - xor, a & ~b = pa - and, ~a & b = pb - and,
 * ~a & ~b = d - pa - pb + and.  Each count is then what the reference's float32 pw*_sum
 * accumulator holds (exact below 2^24, then 2^24), and the output follows the reference's
 * float32 composite over those counts in its operation order, without contraction:
 *   HAMMING        pwne_mean                       (pairwise_metrics.cpp:206-213)
 *   JACCARD        prf_div(xor, or, "zero")        (:215-222)
 *   KULSINSKI      (xor - and + d) / (xor + d)     (:224-234)
 *   KULCZYNSKI1    and / xor                       (:236-243)
 *   YULE           prf_div(2 hR, and nor + hR), hR = (a & ~b)(~a & b)   (:339-347)
 *   DICE           xor / (2 and + xor)             (:349-357)
 *   ROGERSTANIMOTO, SOKALMICHENER  2 xor / (eq + 2 xor)   (:359-368, :379-388)
 *   RUSSELLRAO     (d - and) * fl(1 / d): the reference's GPU route, where ATen divides a
 *                  tensor by a CPU scalar as a multiply by the float reciprocal (:370-377)
 *   SOKALSNEATH    2 xor / (and + 2 xor)           (:390-399)
 * Replaces the 2-4 pw*_sum passes and the elementwise passes of each composite. */
int tpw_bool_count_metric(const uint32_t *x1_words, const uint32_t *x2_words,
                          const int32_t *x1_popcounts, const int32_t *x2_popcounts,
                          int64_t batch, int64_t n, int64_t m, int64_t d, int metric, float *out,
                          void *stream);

/* Set bytes per row of a [rows, d] bool matrix (torch.bool layout, bytes 0/1), as int32:
 * the row popcounts of the byte entry points below.  Replaces nothing in the reference (its
 * kernels count per output pair). */
int tpw_bool_row_counts(const uint8_t *x, int64_t rows, int64_t d, int32_t *counts, void *stream);

/* The bool reductions and count metrics straight from bool bytes (0/1, torch.bool layout,
 * [batch, n, d] and [batch, m, d], any alignment) and their row counts
 * (tpw_bool_row_counts), on the int8 matrix cores: the AND count of two rows is their int8
 * dot product (v_mfma_i32_32x32x32_i8, int32 accumulation), and or / xor / ne / eq follow
 * from it and the row counts as listed for tpw_bool_count_metric.  Outputs equal those of
 * tpw_bool_pairwise_reduce / tpw_bool_count_metric on the packed rows bit for bit, without
 * the pack pass.  Replaces pairwise_binary_reduction_forward_kernel<op, Sum|Mean> for bool
 * inputs (csrc/ops/cuda/pairwise_binary_kernels.cu:32-53,144-220; CPU:
 * csrc/ops/cpu/pairwise_binary_kernels.cpp:28-49,118-171) and the boolean metric composites
 * of csrc/ops/pairwise_metrics.cpp:206-243,339-399. */
int tpw_bool_bytes_reduce(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                          const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m, int64_t d,
                          int op, int reduction, float *out, void *stream);
int tpw_bool_bytes_count_metric(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                                const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m,
                                int64_t d, int metric, float *out, void *stream);

/* Bool rows as fp4 (e2m1) values 0.0 / 1.0: nibble 0x0 or 0x2, feature 2j in the low nibble of
 * byte j, each row zero-padded to tpw_bool_fp4_row_bytes(d) = ceil(d / 256) * 128 bytes.
 * tpw_pack_bool_fp4 converts [rows, d] bool bytes (0/1, any alignment) into that layout
 * (16-byte aligned output) and writes the row counts, in one pass; d < 2^24.
 * tpw_bool_fp4_reduce / tpw_bool_fp4_count_metric then take the AND counts as fp4 dot products
 * on the gfx950 scaled matrix cores (v_mfma_scale_f32_32x32x64_f8f6f4, exact: integer partial
 * sums below 2^24) and finish exactly as tpw_bool_bytes_reduce / tpw_bool_bytes_count_metric,
 * bit for bit, at half their operand bytes and matrix-core cycles.  x1 / x2 are the packed
 * [batch, n, row_bytes] / [batch, m, row_bytes] operands; per batch, rows x row bytes < 2^31.
 * Replace the same reference kernels as the byte entry points above
 * (csrc/ops/cuda/pairwise_binary_kernels.cu:32-53,144-220;
 * csrc/ops/pairwise_metrics.cpp:206-243,339-399). */
int64_t tpw_bool_fp4_row_bytes(int64_t d);
int tpw_pack_bool_fp4(const uint8_t *x, int64_t rows, int64_t d, uint8_t *fp4, int32_t *counts,
                      void *stream);
int tpw_bool_fp4_reduce(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                        const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m, int64_t d,
                        int op, int reduction, float *out, void *stream);
int tpw_bool_fp4_count_metric(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                              const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m,
                              int64_t d, int metric, float *out, void *stream);

/* Self-check of the quotient the bit and fp4 tile kernels use for rows of at most 2^20
 * features (reciprocal, one Newton step, one residual correction), which must equal the IEEE
 * divide for integer numerators in [0, 2^22] and denominators in [1, 2^21].  For every
 * o in [o_lo, o_hi] and the x_count numerators x = phase(o) + k x_step, adds to *mismatches
 * the number of quotients whose bits differ from __fdiv_rn's (both the sequence from the
 * hardware reciprocal and the one from RN(1 / o)).  No counterpart in the reference: a
 * diagnostic of this library's arithmetic for its tests. */
int tpw_count_division_check(int64_t o_lo, int64_t o_hi, int64_t x_step, int64_t x_count,
                             unsigned long long *mismatches, void *stream);

/* Equal / not-equal counts (TPW_BIT_EQ / TPW_BIT_NE, TPW_RED_SUM / TPW_RED_MEAN) of
 * non-bool inputs of element type `elem_type` (TPW_F32 ... TPW_I64), compared by value
 * like C++ ==; output float32 [batch, n, m] as tpw_bool_pairwise_reduce.
 * Replaces pairwise_binary_reduction_forward_kernel<Equal|NotEqual, Sum|Mean> for
 * non-bool dtypes (csrc/ops/cuda/pairwise_binary_kernels.cu:32-53,144-220), which
 * hamming_distances reaches without a bool coercion (csrc/ops/pairwise_metrics.cpp:206-213). */
int tpw_compare_reduce(const void *x1, const void *x2, int elem_type, int64_t batch,
                       int64_t n, int64_t m, int64_t d, int op, int reduction, float *out,
                       void *stream);

/* ------------------------------------------------------------------------- */
/* Inner-product family (MFMA): euclidean, sqeuclidean, cosine, linear        */
/* ------------------------------------------------------------------------- */

#define TPW_EPI_DOT 0         /* s = x1 . x2                                  */
#define TPW_EPI_EUCLIDEAN 1   /* sqrt(max(0, |x1|^2 + |x2|^2 - 2 s))          */
#define TPW_EPI_SQEUCLIDEAN 2 /* max(0, |x1|^2 + |x2|^2 - 2 s)                */
#define TPW_EPI_COSINE_SIM 3  /* prf_div(s, |x1| |x2|, "identity")            */
#define TPW_EPI_COSINE_DIST 4 /* clip(1 - prf_div(s, |x1||x2|, identity), 0, 2) */
#define TPW_EPI_CORRELATION 5 /* 1 - prf_div(s, |x1||x2|, identity), no clip     */

/* norms[r] = sum_k x[r,k]^2 (squared != 0) or its square root, in float32.
 * Replaces x.pow(2).sum(-1) / x.norm(2, -1) feeding _euclidean_dist
 * (torch/_decomp/decompositions.py:691-701) and cosine_similarity
 * (csrc/ops/pairwise_metrics.cpp:118-119). */
int tpw_row_norms(const void *x, int dtype, int64_t rows, int64_t d, int squared,
                  float *norms, void *stream);

/* out[b,i,j] = epilogue(x1[b,i,:] . x2[b,j,:], aux1[b*n+i], aux2[b*m+j]) with the
 * contraction on the matrix cores (fp32: v_mfma_f32_32x32x2_f32; bf16:
 * v_mfma_f32_32x32x16_bf16, fp32 accumulation).  aux1/aux2 are the squared norms
 * for EUCLIDEAN/SQEUCLIDEAN, the norms for COSINE_*, unused (may be NULL) for DOT.
 * `out` has the element type of the inputs.
 * Replaces at::cdist(x1, x2, 2) on its matrix-product path (_euclidean_dist,
 * csrc/ops/pairwise_metrics.cpp:24-31), matmul + prf_div (+ 1 - s, clip) of
 * cosine_similarity / cosine_distances (csrc/ops/pairwise_metrics.cpp:51-56,112-122), the
 * matmul of linear_kernel (DOT, :58-65) and, on centred rows, correlation_distances'
 * matmul + prf_div + neg_ + add_(1) (CORRELATION, :190-204). */
int tpw_pairwise_inner(const void *x1, const void *x2, int dtype, int64_t batch,
                       int64_t n, int64_t m, int64_t d, const float *aux1,
                       const float *aux2, int epilogue, void *out, void *stream);

/* ------------------------------------------------------------------------- */
/* Non-GEMM reductions (VALU): manhattan, chebyshev, minkowski                */
/* ------------------------------------------------------------------------- */

/* out[b,i,j] = (sum_k |x1[b,i,k] - x2[b,j,k]|^p)^(1/p); p = 0 counts non-zero
 * differences, p = 1 manhattan, p = +inf chebyshev (max).  fp32 only.
 * Replaces at::_cdist_forward (reached from at::cdist for p != 2, and for p = 2
 * when both row counts are <= 25) used by manhattan / minkowski / chebyshev
 * (csrc/ops/pairwise_metrics.cpp:42-49,160-168,299-306). */
int tpw_lp_distances(const float *x1, const float *x2, int64_t batch, int64_t n,
                     int64_t m, int64_t d, double p, float *out, void *stream);

/* tpw_lp_distances with a bf16 output [batch,n,m] (uint16 bits): the fp32 result rounded once
 * to nearest even (NaN to 0x7fc0), written directly, where a float output would be written,
 * read back and converted.  x1, x2 are fp32 (bf16 inputs widened by the caller).  Replaces
 * at::cdist on bf16 tensors for p != 2 (csrc/ops/pairwise_metrics.cpp:42-49,160-168,299-306). */
int tpw_lp_distances_bf16(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                          int64_t d, double p, uint16_t *out, void *stream);

/* out[b,i,j] = v1[b,i] / sum_k (a[b,i,k] - b[b,j,k])^2 (an IEEE divide) for rows a, b
 * centred by the caller and v1 = sum_k a^2: the forward of _snr as one pass, where the
 * reference's GPU route writes the squared distances and divides in a second pass
 * (csrc/ops/cpu/snr_kernel.cpp:13-33, cuda/snr_kernel.cu:100-105).  fp32. */
int tpw_snr_centered(const float *a, const float *b, const float *v1, int64_t batch, int64_t n,
                     int64_t m, int64_t d, float *out, void *stream);

/* Workspace (bytes) of tpw_lp_distances_backward (either direction: the same size serves
 * the transposed call) and tpw_lp_distances_backward2 for these sizes. */
size_t tpw_lp_backward_workspace_size(int64_t batch, int64_t n, int64_t m, int64_t d);

/* grad_x1[b,i,k] = sum_j dD[b,i,j]/dx1[b,i,k] * grad[b,i,j] for the Lp distance
 * `dist` produced by tpw_lp_distances (same p), with torch's per-p formulas
 * (p = 0: zero; 1: g sign(diff); p < 2: sign(diff) |diff|^(p-1) g / dist^(p-1), 0 where
 * dist == 0 or (diff == 0 and p < 1); 2: g diff / dist; inf: g sign(diff) [|diff| == dist];
 * other: diff |diff|^(p-2) g / dist^(p-1)).  Here n is the row count of `x1` and m that
 * of `x2`.  With `transposed` != 0 the same call yields grad_x2: pass x2 as `x1`, x1 as
 * `x2`, and the original grad and dist, which are then read transposed (as [batch,m,n]).
 * Replaces at::_cdist_backward (derivatives.yaml:1338-1340: x1 -> _cdist_backward
 * (grad, x1, x2, p, result); x2 -> _cdist_backward(grad.mT, x2, x1, p, result.mT)). */
int tpw_lp_distances_backward(const float *grad, const float *x1, const float *x2,
                              const float *dist, int64_t batch, int64_t n, int64_t m,
                              int64_t d, double p, int transposed, float *grad_x1,
                              void *workspace, void *stream);

/* Both gradients of tpw_lp_distances in one call (grad_x1 [batch,n,d], grad_x2
 * [batch,m,d]), sharing the per-pair weight pass; same formulas as above.  Replaces the
 * pair of _cdist_backward calls of derivatives.yaml:1338-1340. */
int tpw_lp_distances_backward2(const float *grad, const float *x1, const float *x2,
                               const float *dist, int64_t batch, int64_t n, int64_t m,
                               int64_t d, double p, float *grad_x1, float *grad_x2,
                               void *workspace, void *stream);

/* ------------------------------------------------------------------------- */
/* The reference's own VALU metric kernels (fp32; x1 [batch,n,d], x2 [batch,m,d]) */
/* ------------------------------------------------------------------------- */

#define TPW_FAM_PPMINKOWSKI 0
#define TPW_FAM_WMINKOWSKI 1
#define TPW_FAM_CANBERRA 2
#define TPW_FAM_BRAYCURTIS 3
#define TPW_FAM_CHI2 4
#define TPW_FAM_JS 5

/* out = sum_k |x1 - x2|^p with no root (p = 0: d, as the reference fills; p = +-inf: max /
 * min of |diff|).  Replaces _ppminkowski (torchpairwise/csrc/ops/ppminkowski.cpp:32-34,
 * cpu/ppminkowski_kernel.cpp:58-118); sqeuclidean_distances is p = 2. */
int tpw_ppminkowski(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                    int64_t d, double p, float *out, void *stream);

/* out = (sum_k w[b,k] |x1 - x2|^p)^(1/p) (p = 0: d; p = +-inf: max / min of w |diff|),
 * w [batch, d].  Replaces _wminkowski (wminkowski.cpp:34-36,
 * cpu/wminkowski_kernel.cpp:63-128); seuclidean is w = 1 / V, p = 2. */
int tpw_wminkowski(const float *x1, const float *x2, const float *w, int64_t batch, int64_t n,
                   int64_t m, int64_t d, double p, float *out, void *stream);

/* out = sum_k |x1 - x2| / (|x1| + |x2|), terms with a zero denominator skipped.  Replaces
 * _canberra (canberra.cpp:30-32, cpu/canberra_kernel.cpp:13-82). */
int tpw_canberra(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                 int64_t d, float *out, void *stream);

/* out = sum_k |x1 - x2| / sum_k |x1 + x2|.  Replaces _braycurtis (braycurtis.cpp:30-32,
 * cpu/braycurtis_kernel.cpp:13-81). */
int tpw_braycurtis(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                   int64_t d, float *out, void *stream);

/* out = -sum_k (x1 - x2)^2 / (x1 + x2), terms with x1 + x2 == 0 skipped.  Replaces
 * _additive_chi2_kernel (additive_chi2_kernel.cpp:30-32, cpu/additive_chi2_kernel.cpp:13-33,35-70). */
int tpw_additive_chi2(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                      int64_t d, float *out, void *stream);

/* out = sum_k (rel_entr(x1, mid) + rel_entr(x2, mid)) / divisor, mid = (x1 + x2) / 2, with
 * rel_entr of cpu/rel_entr.h; divisor = 2, or 2 ln(base).  Replaces _sqjensenshannon
 * (sqjensenshannon.cpp:33-35, cpu/sqjensenshannon_kernel.cpp:13-31,33-80). */
int tpw_sqjensenshannon(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                        int64_t d, double divisor, float *out, void *stream);

/* Workspace (bytes) of the backward of family member `metric` (TPW_FAM_*). */
size_t tpw_family_backward_workspace_size(int metric, int64_t batch, int64_t n, int64_t m,
                                          int64_t d);

/* Gradients of the four members above with the reference's formulas, summed over pairs in
 * a fixed order (the reference's GPU kernels use atomics).  p = 0 gives zero gradients, as
 * in the reference; p = +-inf is rejected (TPW_ERR_INVALID).  `out` is the forward result.
 * Replace __ppminkowski_backward (ppminkowski.cpp:35-37, cpu/ppminkowski_kernel.cpp:121-
 * 289), __wminkowski_backward (wminkowski.cpp:37-39, cpu/wminkowski_kernel.cpp:
 * 131-379; grad_w [batch, d]), __canberra_backward (canberra.cpp:33-35,
 * cpu/canberra_kernel.cpp:85-179; no guard: a zero |x1| + |x2| gives NaN, as there) and
 * __braycurtis_backward (braycurtis.cpp:33-35, cpu/braycurtis_kernel.cpp:84-226). */
int tpw_ppminkowski_backward(const float *grad, const float *x1, const float *x2, int64_t batch,
                             int64_t n, int64_t m, int64_t d, double p, float *grad_x1,
                             float *grad_x2, void *workspace, void *stream);
int tpw_wminkowski_backward(const float *grad, const float *x1, const float *x2, const float *w,
                            const float *out, int64_t batch, int64_t n, int64_t m, int64_t d,
                            double p, float *grad_x1, float *grad_x2, float *grad_w,
                            void *workspace, void *stream);
int tpw_canberra_backward(const float *grad, const float *x1, const float *x2, int64_t batch,
                          int64_t n, int64_t m, int64_t d, float *grad_x1, float *grad_x2,
                          void *workspace, void *stream);
int tpw_braycurtis_backward(const float *grad, const float *x1, const float *x2,
                            const float *out, int64_t batch, int64_t n, int64_t m, int64_t d,
                            float *grad_x1, float *grad_x2, void *workspace, void *stream);

/* Gradients of tpw_additive_chi2 and tpw_sqjensenshannon with the reference's formulas
 * (__additive_chi2_kernel_backward, additive_chi2_kernel.cpp:33-35,
 * cpu/additive_chi2_kernel.cpp:72-183; __sqjensenshannon_backward, sqjensenshannon.cpp:36-38,
 * cpu/sqjensenshannon_kernel.cpp:82-197), summed over pairs in a fixed order. */
int tpw_additive_chi2_backward(const float *grad, const float *x1, const float *x2,
                               int64_t batch, int64_t n, int64_t m, int64_t d, float *grad_x1,
                               float *grad_x2, void *workspace, void *stream);
int tpw_sqjensenshannon_backward(const float *grad, const float *x1, const float *x2,
                                 int64_t batch, int64_t n, int64_t m, int64_t d, double divisor,
                                 float *grad_x1, float *grad_x2, void *workspace, void *stream);

/* float64 forms of the six members above (metric = TPW_FAM_*; w [batch, d] for
 * TPW_FAM_WMINKOWSKI, else ignored; p is the exponent for the Minkowski members, the divisor
 * for TPW_FAM_JS, unused otherwise).  Same per-pair expressions as the reference's loops, summed
 * over k in order, in double.  Replace the double dispatch of the reference's CUDA kernels:
 * _ppminkowski (cuda/ppminkowski_kernel.cu:102), _wminkowski (cuda/wminkowski_kernel.cu:113),
 * _canberra (cuda/canberra_kernel.cu:74), _braycurtis (cuda/braycurtis_kernel.cu:73),
 * _additive_chi2_kernel (cuda/additive_chi2_kernel.cu:75), _sqjensenshannon
 * (cuda/sqjensenshannon_kernel.cu:74). */
int tpw_family_f64(int metric, const double *x1, const double *x2, const double *w, int64_t batch,
                   int64_t n, int64_t m, int64_t d, double p, double *out, void *stream);

/* Workspace (bytes) of tpw_family_f64_backward. */
size_t tpw_family_f64_backward_workspace_size(int metric, int64_t batch, int64_t n, int64_t m,
                                              int64_t d, double p);

/* Gradients of tpw_family_f64 with the reference's formulas (p = +-inf included: the first
 * arg-extremum feature per pair), summed over pairs in a fixed order, in double; grad_w
 * [batch, d] for TPW_FAM_WMINKOWSKI.  Replace the double dispatch of the reference's
 * __*_backward CUDA kernels (cuda/ppminkowski_kernel.cu:247, cuda/wminkowski_kernel.cu:299,
 * cuda/canberra_kernel.cu:162, cuda/braycurtis_kernel.cu:191, cuda/additive_chi2_kernel.cu:167,
 * cuda/sqjensenshannon_kernel.cu:178). */
int tpw_family_f64_backward(int metric, const double *grad, const double *x1, const double *x2,
                            const double *w, int64_t batch, int64_t n, int64_t m, int64_t d,
                            double p, double *grad_x1, double *grad_x2, double *grad_w,
                            void *workspace, void *stream);

/* Unreduced pairwise binary op: out[b,i,j,k] = op(x1[b,i,k], x2[b,j,k]) as bool bytes (0/1),
 * out [batch, n, m, d] 16-byte aligned; x1 [batch, n, d], x2 [batch, m, d] of element type
 * dtype (TPW_U8 for bool).  op: TPW_BIT_AND / OR / XOR (bool elements only, as the reference
 * dispatches them), TPW_BIT_EQ / NE, TPW_CMP_LT / GT / LE / GE (float16 and bfloat16 compared
 * as float).  Replaces pairwise_binary_forward_kernel (cuda/pairwise_binary_kernels.cu:16-30,
 * 61-141; cpu/pairwise_binary_kernels.cpp:12-26) behind pwand, pwor, pwxor, pweq, pwne, pwlt,
 * pwgt, pwle, pwge (pairwise_binary.cpp:34-89). */
int tpw_pairwise_binary(const void *x1, const void *x2, int dtype, int op, int64_t batch, int64_t n,
                        int64_t m, int64_t d, uint8_t *out, void *stream);

/* Workspace (bytes) of tpw_haversine / tpw_haversine_backward. */
size_t tpw_haversine_workspace_size(int64_t batch, int64_t n, int64_t m);

/* Workspace (bytes) of tpw_sqmahalanobis for these sizes (dtype TPW_F32 or TPW_F64). */
size_t tpw_sqmahalanobis_workspace_size(int dtype, int64_t batch, int64_t n, int64_t m, int64_t d);

/* out[b,i,j] = d^T VI[b] d with d = x1[b,i,:] - x2[b,j,:] (x1 [batch,n,d], x2 [batch,m,d],
 * VI [batch,d,d], dtype TPW_F32 or TPW_F64).  Computed as sum_k d_k (P1[i,k] - P2[j,k]) with
 * the per-row projections P = x VI^T formed once (in double, carried as two floats for
 * TPW_F32): O(d) per pair instead of the reference's O(d^2), and, as there, the difference
 * comes first, so identical rows give exactly 0.  x2 may be x1 (n == m): the projection is
 * then formed once.  Replaces _sqmahalanobis_forward_kernel
 * (csrc/ops/cpu/sqmahalanobis_kernel.cpp:11-88; CUDA cuda/sqmahalanobis_kernel.cu:16-100). */
int tpw_sqmahalanobis(const void *x1, const void *x2, const void *VI, int dtype, int64_t batch,
                      int64_t n, int64_t m, int64_t d, void *out, void *workspace, void *stream);

/* out[b,i,j] = 2 asin(sqrt(sin^2(dlat/2) + cos lat_i cos lat_j sin^2(dlon/2))) for points
 * x1 [batch, n, 2], x2 [batch, m, 2] given as (latitude, longitude) in radians.  Replaces
 * _haversine (haversine.cpp:30-32, cpu/haversine_kernel.cpp:13-27,29-75). */
int tpw_haversine(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                  float *out, void *workspace, void *stream);

/* Gradients of tpw_haversine with the reference's formulas (__haversine_backward,
 * haversine.cpp:33-35, cpu/haversine_kernel.cpp:78-217; no guard: a zero or antipodal pair
 * gives inf/NaN, as there), grad_x1 [batch, n, 2], grad_x2 [batch, m, 2]. */
int tpw_haversine_backward(const float *grad, const float *x1, const float *x2, int64_t batch,
                           int64_t n, int64_t m, float *grad_x1, float *grad_x2,
                           void *workspace, void *stream);

/* float64 forms of tpw_haversine / tpw_haversine_backward (no workspace): the reference's
 * double dispatch of _haversine and __haversine_backward (cuda/haversine_kernel.cu:69,185). */
int tpw_haversine_f64(const double *x1, const double *x2, int64_t batch, int64_t n, int64_t m,
                      double *out, void *stream);
int tpw_haversine_f64_backward(const double *grad, const double *x1, const double *x2,
                               int64_t batch, int64_t n, int64_t m, double *grad_x1,
                               double *grad_x2, void *stream);

/* ------------------------------------------------------------------------- */
/* Backward of the inner-product family                                       */
/* ------------------------------------------------------------------------- */

/* Workspace (bytes) needed by tpw_euclidean_backward / tpw_cosine_backward: an fp32
 * [batch, n, m] pair-weight matrix plus small per-row buffers. */
size_t tpw_inner_backward_workspace_size(int64_t batch, int64_t n, int64_t m, int64_t d);

/* _euclidean_dist_backward: ratio = grad / res (0 where res == 0);
 * grad_x1 = x1 * sum_j ratio - ratio @ x2, grad_x2 = x2 * sum_i ratio - ratio^T @ x1.
 * grad and res are [batch,n,m] of the input type; both gradient products run on the
 * matrix cores.  When x2 is x1 (x2=None upstream), the caller adds the two halves.
 * Replaces _euclidean_dist_backward (derivatives.yaml:1335-1336) under at::cdist(p=2). */
int tpw_euclidean_backward(const void *grad, const void *x1, const void *x2,
                           const void *res, int dtype, int64_t batch, int64_t n,
                           int64_t m, int64_t d, void *grad_x1, void *grad_x2,
                           void *workspace, void *stream);

/* Backward of sqeuclidean_distances (sum_k (x1 - x2)^2): grad_x1 = x1 * sum_j 2 grad -
 * (2 grad) @ x2, grad_x2 = x2 * sum_i 2 grad - (2 grad)^T @ x1, i.e. the p = 2 case of
 * _ppminkowski's backward g p |d|^(p-1) sign(d) (csrc/ops/cpu/ppminkowski_kernel.cpp:122-169)
 * summed over the other operand. */
int tpw_sqeuclidean_backward(const void *grad, const void *x1, const void *x2, int dtype,
                             int64_t batch, int64_t n, int64_t m, int64_t d, void *grad_x1,
                             void *grad_x2, void *workspace, void *stream);

/* Backward of linear_kernel (x1 . x2^T): grad_x1 = grad . x2, grad_x2 = grad^T . x1 on the
 * matrix cores (the autograd of the reference's matmul, pairwise_metrics.cpp:58-65).
 * Workspace: tpw_inner_backward_workspace_size(batch, n, m, d) bytes. */
int tpw_linear_backward(const void *grad, const void *x1, const void *x2, int dtype,
                        int64_t batch, int64_t n, int64_t m, int64_t d, void *grad_x1,
                        void *grad_x2, void *workspace, void *stream);

/* Backward of cosine_distances = clip(1 - prf_div(x1 x2^T, n1 n2^T, identity), 0, 2):
 * the autograd graph of csrc/ops/pairwise_metrics.cpp:51-56,112-122 with the prf_div
 * backward of csrc/ops/cpu/prf_div_kernel.cpp:258-277, the clamp mask of
 * derivatives.yaml (grad where min <= x <= max) and torch's 2-norm backward (0 where the
 * norm is 0).  `norms1`/`norms2` are the fp32 row norms of x1/x2.  `similarity` = 1: the
 * op is cosine_similarity (no 1 - s, no clip); 2: correlation_distances' 1 - s without the
 * clip (pairwise_metrics.cpp:190-204, neg_ then add_(1)) of rows the caller has centred.
 * `out` (may be NULL): the forward's output [batch,n,m] of the input type.  Given, the
 * weights come from it (s = out, or 1 - out) with no recomputed x1 x2^T; a distance output
 * of exactly 0 or 2 then counts as clipped.  NULL: x1 x2^T is recomputed on the matrix cores.
 * When x2 is x1 (x2=None upstream), the caller adds the two halves. */
int tpw_cosine_backward(const void *grad, const void *x1, const void *x2,
                        const float *norms1, const float *norms2, const void *out, int dtype,
                        int64_t batch, int64_t n, int64_t m, int64_t d, int similarity,
                        void *grad_x1, void *grad_x2, void *workspace, void *stream);

/* ------------------------------------------------------------------------- */
/* prf_div (guarded divide)                                                   */
/* ------------------------------------------------------------------------- */

/* out = y != 0 ? x / y : (identity ? x : 0), elementwise over `numel` elements of type
 * TPW_F32 / TPW_F64 / TPW_F16 / TPW_BF16 (half types round after each operation).  `out`
 * may be `x` or `y` (the in-place forms); prf_ldiv(a, b) is this with x = b, y = a.
 * Replaces prf_div_forward_kernel (csrc/ops/cpu/prf_div_kernel.cpp:14-24,58-103;
 * CUDA csrc/ops/cuda/prf_div_kernel.cu:24-36,76-133) with mode "zero" / "identity", and the
 * in-place prf_div__forward_kernel (cpu/prf_div_kernel.cpp:153-207; cuda :190-256). */
int tpw_prf_div(const void *x, const void *y, int dtype, int64_t numel, int identity,
                void *out, void *stream);

/* The scalar forms.  scalar_first == 0: out = c != 0 ? x / c : (identity ? x : 0)
 * (prf_div.Scalar, prf_ldiv.rScalar); scalar_first != 0: out = x != 0 ? c / x :
 * (identity ? c : 0) (prf_ldiv.Scalar, prf_div.rScalar).  c is rounded to the element type
 * first (to float, then to the half type, as c10::Scalar::to does).  `out` may be `x`.
 * Replaces the scalar overloads of prf_div_forward_kernel_impl and the Scalar / rScalar /
 * in-place Scalar kernels (csrc/ops/cpu/prf_div_kernel.cpp:25-54,106-151,210-255;
 * CUDA csrc/ops/cuda/prf_div_kernel.cu:39-70,136-188,259-306). */
int tpw_prf_div_scalar(const void *x, double c, int dtype, int64_t numel, int identity,
                       int scalar_first, void *out, void *stream);

/* grad_x = y != 0 ? g / y : (identity ? g : 0); grad_y = y != 0 ? (g / y) * -x / y : 0.
 * Replaces prf_div_backward_kernel (csrc/ops/cpu/prf_div_kernel.cpp:258-277;
 * CUDA csrc/ops/cuda/prf_div_kernel.cu:315-368). */
int tpw_prf_div_backward(const void *grad, const void *x, const void *y, int dtype,
                         int64_t numel, int identity, void *grad_x, void *grad_y,
                         void *stream);

/* Backward of the scalar forms, into grad_x (every element written).  scalar_first == 0
 * (z = x / c): grad_x = c != 0 ? g / c : (identity ? g : 0), x unused (may be NULL);
 * scalar_first != 0 (z = c / x): grad_x = x != 0 ? (g * -c) / (x * x) : 0.
 * Replaces the scalar overloads of prf_div_backward_kernel_impl and the Scalar / rScalar
 * backward kernels (csrc/ops/cpu/prf_div_kernel.cpp:279-311,363-450;
 * CUDA csrc/ops/cuda/prf_div_kernel.cu:336-368,426-525). */
int tpw_prf_div_scalar_backward(const void *grad, const void *x, double c, int dtype,
                                int64_t numel, int identity, int scalar_first, void *grad_x,
                                void *stream);

/* ------------------------------------------------------------------------- */
/* Directed Hausdorff                                                         */
/* ------------------------------------------------------------------------- */

/* Workspace (bytes) for tpw_directed_hausdorff with these sizes. */
size_t tpw_hausdorff_workspace_size(int64_t batch, int64_t b1, int64_t p1, int64_t b2,
                                    int64_t p2, int64_t d);

/* out[b,i,j] = sqrt(max_m min_n |x1[b,i,m,:] - x2[b,j,n,:]|^2), x1 [batch,b1,p1,d],
 * x2 [batch,b2,p2,d] fp32, with the reference's indices: idx1 = the last m (in
 * iteration order) reaching the maximum, idx2 = the first n reaching that m's
 * minimum.  Squared distances are summed k = 0..d-1 in fp32 without contraction,
 * as the reference CPU loop does.  perm1 [batch,p1] / perm2 [batch,p2] give the
 * iteration order (shuffle=True) or are NULL for natural order; reported indices
 * are the permuted values.  The full p1 x p2 distance matrix is never formed.
 * Replaces _directed_hausdorff_forward_kernel
 * (csrc/ops/cpu/hausdorff_kernel.cpp:12-185; CUDA csrc/ops/cuda/hausdorff_kernel.cu:17-195). */
int tpw_directed_hausdorff(const float *x1, const float *x2, int64_t batch, int64_t b1,
                           int64_t p1, int64_t b2, int64_t p2, int64_t d,
                           const int64_t *perm1, const int64_t *perm2, float *out,
                           int64_t *idx1, int64_t *idx2, void *workspace, void *stream);

/* Work counters of tpw_directed_hausdorff (measurement support; no counterpart in the
 * reference).  arm != 0: waits for the current device, zeroes the counters and starts counting
 * the calls made on that device (out is not used).  arm == 0: waits for the device, stops
 * counting and writes out[0] = point pairs whose squared distance the kernels evaluated,
 * out[1] = cell-box tests of the sorted mode's cell scan (one box against one x2 point),
 * out[2] = kernel launches, summed over the calls since arming.  Pairs are counted on the
 * cell-grid paths (d <= 3); the d >= 4 kernels do not count.  Not for concurrent use from
 * several threads. */
int tpw_hausdorff_counters(int arm, unsigned long long *out);

/* Size of the static scratch buffer of tpw_directed_hausdorff_noalloc, in MiB (per GPU). */
#define TPW_HAUSDORFF_NOALLOC_SCRATCH_MIB 96

/* tpw_directed_hausdorff without a workspace argument: the same kernels and results, with
 * their scratch in a static device array of TPW_HAUSDORFF_NOALLOC_SCRATCH_MIB MiB that each
 * GPU holds until the process ends.  It has no counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): it calls no hipMalloc / hipFree.  Sizes whose
 * tpw_hausdorff_workspace_size exceeds the buffer are rejected with TPW_ERR_INVALID (the
 * [16, 65536, 3] x [16, 65536, 3] case needs 45 MiB).  The array is in a code object of its
 * own: a GPU holds it from this entry point's first call there, and processes that never call
 * it hold none.  Every call on one GPU shares that GPU's buffer, so calls are serialised: each
 * call's stream waits for the previous call's work on that GPU (one event per device, created
 * at the first call) before its own.  Under HIP graph capture that wait is left out and the
 * graph's order is the caller's to give: captured calls that overlap on one GPU race. */
int tpw_directed_hausdorff_noalloc(const float *x1, const float *x2, int64_t batch, int64_t b1,
                                   int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                   const int64_t *perm1, const int64_t *perm2, float *out,
                                   int64_t *idx1, int64_t *idx2, void *stream);

/* grad_x1[b,i,idx1,k] += grad * (x1[idx1,k] - x2[idx2,k]) / out summed over j in
 * order; grad_x2[b,j,idx2,k] += grad * (x2[idx2,k] - x1[idx1,k]) / out summed over
 * i in order, starting from zero: grad_x1/grad_x2 are overwritten (every element
 * written; no fill by the caller is needed).
 * Replaces the scatter half of _directed_hausdorff_backward_kernel
 * (csrc/ops/cpu/hausdorff_kernel.cpp:187-235,308-336;
 *  CUDA csrc/ops/cuda/hausdorff_kernel.cu:199-246). */
int tpw_directed_hausdorff_backward(const float *grad, const float *x1, const float *x2,
                                    const float *out, const int64_t *idx1,
                                    const int64_t *idx2, int64_t batch, int64_t b1,
                                    int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                    float *grad_x1, float *grad_x2, void *stream);

/* Directed Hausdorff for dtype TPW_F64 or TPW_F16 (TPW_F32 also accepted: it gives the
 * pruned pipeline's results bit for bit): the reference's early-exit loop run in its own order,
 * one wave per cloud pair, with the element type's arithmetic (float16: each difference,
 * square and sum computed in float and rounded to half, as c10::Half does).  Same arguments
 * and outputs as tpw_directed_hausdorff, out in the input dtype, no workspace.  Replaces the
 * double and half dispatch of _directed_hausdorff_forward_kernel (cuda/hausdorff_kernel.cu:
 * 16-105,150; cpu/hausdorff_kernel.cpp:12-100). */
int tpw_directed_hausdorff_exact(int dtype, const void *x1, const void *x2, int64_t batch,
                                 int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                 const int64_t *perm1, const int64_t *perm2, void *out,
                                 int64_t *idx1, int64_t *idx2, void *stream);

/* Gradients for tpw_directed_hausdorff_exact's dtypes, from its outputs and indices (which
 * must lie in [0, p1) and [0, p2)): grad_x1 and grad_x2 are overwritten (zero-filled here),
 * then the same scatter as tpw_directed_hausdorff_backward in the element type's arithmetic.
 * Replaces the double and half dispatch of _directed_hausdorff_backward_kernel
 * (cuda/hausdorff_kernel.cu:199-246,283; cpu/hausdorff_kernel.cpp:187-235). */
int tpw_directed_hausdorff_exact_backward(int dtype, const void *grad, const void *x1,
                                          const void *x2, const void *out, const int64_t *idx1,
                                          const int64_t *idx2, int64_t batch, int64_t b1,
                                          int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                          void *grad_x1, void *grad_x2, void *stream);

/* ------------------------------------------------------------------------- */
/* Neighbour masks                                                            */
/* ------------------------------------------------------------------------- */

/* mask [rows, cols] (bool bytes, 0/1) = 1 at the `count` smallest entries of each row of
 * dist [rows, cols] (all entries when count >= cols), 0 elsewhere.  Ascending order with
 * NaN after +inf and -0 == +0; ties broken by the lower column index, i.e. the first
 * `count` positions of a stable argsort.  dtype: TPW_F32, TPW_BF16 or TPW_F16;
 * rows, cols < 2^31.  With count = k + 1 this replaces the argsort + slice + index_put_ of
 * k_neighbors_mask (torchpairwise/csrc/ops/neighbors.cpp:29-34), which materialises a
 * full sort of every row; the reference's argsort is unstable, so on ties across the
 * selection boundary its choice is implementation-defined. */
int tpw_row_smallest_mask(const void *dist, int dtype, int64_t rows, int64_t cols,
                          int64_t count, void *mask, void *stream);

/* radius_neighbors_mask with the euclidean metric in one pass: out[b,i,j] (bool bytes) = 1
 * where the euclidean distance of x1[b,i] and x2[b,j] -- the value tpw_pairwise_inner
 * (TPW_EPI_EUCLIDEAN) stores for the same inputs, rounded to bf16 for bf16 -- is <= eps,
 * 0 elsewhere (NaN: 0).  aux1 / aux2: the squared row norms (tpw_row_norms, squared = 1).
 * eps is the radius as the inputs' dtype holds it (float32, or the bf16 value of the
 * float).  The distance matrix is never written.  Replaces cdist(x1, x2, metric).le(epsilon)
 * of radius_neighbors_mask (torchpairwise/csrc/ops/neighbors.cpp:37-60) for the euclidean
 * metric on its matrix-product path. */
int tpw_radius_mask_euclidean(const void *x1, const void *x2, int dtype, int64_t batch,
                              int64_t n, int64_t m, int64_t d, const float *aux1,
                              const float *aux2, float eps, uint8_t *out, void *stream);

/* k_neighbors_mask with the euclidean metric without the distance matrix: mask [n, m] (bool
 * bytes) = 1 at each row's `count` smallest distances between x1 [n, d] and x2 [m, d] (float32 or
 * bfloat16; aux1 / aux2 the squared row norms as for TPW_EPI_EUCLIDEAN), in the order of
 * tpw_row_smallest_mask (ascending, -0 == +0, NaN after +inf, ties to the lower column) over the
 * distances the euclidean op stores (bfloat16: rounded to bfloat16), so the mask equals that of
 * tpw_pairwise_inner (TPW_EPI_EUCLIDEAN) followed by tpw_row_smallest_mask bit for bit.  The
 * tile kernel keeps each row's C >= count smallest (distance, column) keys per 128 columns in
 * the workspace (tpw_knn_mask_workspace_size bytes, 16-byte aligned); a select kernel merges
 * them and writes the mask rows.  Sizes: tpw_knn_mask_euclidean_supported (count 1..16 and <= m,
 * m a multiple of 16, d * element size a multiple of 128 bytes); inputs and mask 16-byte aligned.
 * Replaces cdist + argsort + index_put_ of k_neighbors_mask (torchpairwise/csrc/ops/
 * neighbors.cpp:10-35) for the euclidean metric. */
int tpw_knn_mask_euclidean_supported(int dtype, int64_t n, int64_t m, int64_t d, int64_t count);
size_t tpw_knn_mask_workspace_size(int64_t n, int64_t m, int64_t count);
int tpw_knn_mask_euclidean(const void *x1, const void *x2, int dtype, int64_t n, int64_t m, int64_t d,
                           const float *aux1, const float *aux2, int64_t count, uint8_t *mask,
                           void *workspace, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHPAIRWISE_AMD_H_ */
