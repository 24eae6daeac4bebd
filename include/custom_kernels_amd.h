/*
 * C ABI of the MI355X (gfx950) activation-path library libcustom_kernels_amd.so.
 *
 * Conventions (same as the reference's csrc/includes/<op>.h launchers):
 *   - every launcher returns a hipError_t as int32_t: 0 == success;
 *     hipErrorInvalidValue (1) for an unknown dtype / format / mode tag,
 *     returned before any device call; otherwise the launch status;
 *   - all tensors are caller-allocated, contiguous, row-major device
 *     buffers; the library never allocates, frees, copies or synchronises;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t; NULL is the
 *     null stream);
 *   - empty work (a dimension <= 0) returns 0 without touching the device;
 *   - unaligned pointers and sizes that are not a multiple of the 16-byte
 *     vector width are accepted (scalar kernels handle them).
 *
 * The reference declares its launchers with cudaError_t / cudaStream_t; both
 * are 32-bit-enum / pointer sized, so these declarations are ABI-compatible
 * with its Rust `extern "C"` blocks (src/kernels/<op>.rs declare `-> i32` and
 * `stream: *mut c_void`).
 */
#ifndef CUSTOM_KERNELS_AMD_H_
#define CUSTOM_KERNELS_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dtype tags. Replaces KernelDType (reference csrc/includes/common.cuh:28-34,
 * src/kernels/dtype.rs:5-25); same values. */
enum {
  CCK_DTYPE_F32 = 0,
  CCK_DTYPE_F16 = 1,
  CCK_DTYPE_BF16 = 2,
  CCK_DTYPE_F8E4M3 = 3, /* OCP e4m3fn (torch.float8_e4m3fn) */
  CCK_DTYPE_F8E5M2 = 4  /* OCP e5m2 (torch.float8_e5m2) */
};

/* Scale modes of the fused FP8 launchers. */
enum {
  CCK_SCALE_TOKEN = 0, /* dynamic, one scale per row, written to scale[rows] */
  CCK_SCALE_STATIC = 1 /* caller-given static_scale; `scale` is not used */
};

/* residual_out = x + residual; y = rmsnorm(residual_out) * weight.
 * x, residual, y, residual_out: [rows, cols]; weight: [cols]; one dtype.
 * Replaces reference csrc/includes/rmsnorm_residual.h:17-27. */
int32_t launch_rmsnorm_residual_fwd(const void* x, const void* residual, const void* weight,
                                    void* y, void* residual_out, int64_t rows, int64_t cols,
                                    float eps, int32_t dtype, void* stream);

/* y = silu(gate) * up over n elements.
 * Replaces reference csrc/includes/swiglu.h:16-22. */
int32_t launch_swiglu_fwd(const void* gate, const void* up, void* y, int64_t n, int32_t dtype,
                          void* stream);

/* Half-split RoPE. q: [batch, seq_len, n_q_heads, head_dim], k: [batch, seq_len,
 * n_kv_heads, head_dim], cos/sin: float32 [seq_len, head_dim/2]. q_out may equal
 * q and k_out may equal k (in place). head_dim must be even.
 * Replaces reference csrc/includes/rope.h:23-36. */
int32_t launch_rope_fwd(const void* q, const void* k, const void* cos_table, const void* sin_table,
                        void* q_out, void* k_out, int64_t batch, int64_t seq_len,
                        int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim, int32_t dtype,
                        void* stream);

/* Dynamic FP8, one scale per 128x128 tile; scale: float32 [ceil(m/128), ceil(n/128)].
 * fp8_format: CCK_DTYPE_F8E4M3 or CCK_DTYPE_F8E5M2.
 * Replaces reference csrc/includes/fp8_quant.h:41-49. */
int32_t launch_fp8_quant_block_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                   int64_t n, int32_t dtype, int32_t fp8_format, void* stream);

/* Dynamic FP8, one scale for the matrix; scale: float32 [1]; amax_scratch:
 * int32 [1], caller-zeroed before every call, left holding the bits of
 * max |x| (atomically max-ed in, as in the reference; a nonzero initial value
 * takes part in the maximum and so in the scale). amax_scratch may be NULL
 * (an addition): then no amax word is written. While the call runs, x_fp8
 * and scale also hold its exchange of per-workgroup maxima, which the codes
 * and the final scale overwrite; the call keeps no other state, so calls on
 * different streams may overlap. Inputs of 2^20 or more 16-byte vectors that
 * fit in the registers of a grid the GPU holds at once (up to 64 MiB of x on
 * MI355X) are read from HBM once; larger aligned inputs are read once plus
 * the part the registers do not hold. Where such a grid is not resident at
 * once (other work holding CUs), its waiting workgroups give up after about
 * 2 ms and each reads all of x itself: slower (one more read of x per such
 * workgroup, at most 511), never wrong. Replaces reference
 * csrc/includes/fp8_quant.h:51-60. */
int32_t launch_fp8_quant_tensor_fwd(const void* x, uint8_t* x_fp8, float* scale,
                                    int32_t* amax_scratch, int64_t m, int64_t n, int32_t dtype,
                                    int32_t fp8_format, void* stream);

/* ---- Additive entry points (no reference counterpart; they implement the
 * per-token / static / fused FP8 modes by composing the reference's eager
 * formulas: baselines/fp8_quant.py:162-178 per row, baselines/rmsnorm_residual.py:123-136,
 * baselines/swiglu.py:107-112). ---- */

/* Dynamic FP8, one scale per row; scale: float32 [m]. */
int32_t launch_fp8_quant_token_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                   int64_t n, int32_t dtype, int32_t fp8_format, void* stream);

/* As launch_fp8_quant_tensor_fwd (same codes and scale), with no caller
 * memory beyond x, x_fp8 and scale: no counterpart in the reference. For
 * callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc); it calls no allocating routine, and none
 * of its kernels needs scratch memory. Inputs that take the one-pass form
 * (as launch_fp8_quant_tensor_fwd, with x_fp8 and scale holding the exchange)
 * keep no state between calls. The others take a two-pass form whose
 * per-workgroup maxima live in a 2048-byte device array owned by the
 * library, one per GPU, held until the process ends: such calls that overlap
 * on one GPU race on it (each call rewrites every word it reads, so later
 * calls are unaffected). Any m * n that fits int64 works (else
 * hipErrorInvalidValue, before any device call). */
int32_t launch_fp8_quant_tensor_noalloc_fwd(const void* x, uint8_t* x_fp8, float* scale, int64_t m,
                                            int64_t n, int32_t dtype, int32_t fp8_format, void* stream);

/* FP8 with a caller-given scale: x_fp8 = fp8(x / scale). scale_out may be
 * NULL; otherwise the launch also stores scale into scale_out[0] (the scale
 * tensor a caller returns), so a static call is a single kernel. */
int32_t launch_fp8_quant_static_fwd(const void* x, uint8_t* x_fp8, float scale, float* scale_out, int64_t m,
                                    int64_t n, int32_t dtype, int32_t fp8_format, void* stream);

/* residual_out = x + residual, and the FP8 codes of y = rmsnorm(residual_out) * weight
 * (y rounded to dtype first; y itself is not written). scale_mode CCK_SCALE_TOKEN
 * writes scale[rows]; CCK_SCALE_STATIC uses static_scale and, when scale is not
 * NULL, stores it into scale[0]. */
int32_t launch_rmsnorm_residual_fp8_fwd(const void* x, const void* residual, const void* weight,
                                        uint8_t* y_fp8, float* scale, void* residual_out,
                                        int64_t rows, int64_t cols, float eps, float static_scale,
                                        int32_t scale_mode, int32_t dtype, int32_t fp8_format,
                                        void* stream);

/* FP8 codes of y = silu(gate) * up (y rounded to dtype first), rows of length cols.
 * scale_mode as above. */
int32_t launch_swiglu_fp8_fwd(const void* gate, const void* up, uint8_t* y_fp8, float* scale,
                              int64_t rows, int64_t cols, float static_scale, int32_t scale_mode,
                              int32_t dtype, int32_t fp8_format, void* stream);

/* ---- MoE dispatch path (the two memory-bound steps beside an FP8 MoE FFN). ---- */

/* Row gather: dst[i] = src[indices[i]]. src: [S, hidden_dim], indices: int64
 * [n_dst_rows], dst: [n_dst_rows, hidden_dim]; dtype F32/F16/BF16, or
 * F8E4M3/F8E5M2 codes (the rows are moved as bytes; FP8 is an addition to
 * the reference's three). A negative index yields a zero row; indices must be
 * < S (this launcher is not told S, as in the reference).
 * Replaces reference csrc/includes/token_permute.h:17-24. */
int32_t launch_token_gather_fwd(const void* src, const int64_t* indices, void* dst, int64_t n_dst_rows,
                                int64_t hidden_dim, int32_t dtype, void* stream);

/* Weighted combine: combined[t] = sum_j weights[t,j] * expert_output[unpermute_index[t,j]],
 * products rounded to fp32 and summed in torch-CPU's order for (x.float() * w).sum(dim=1)
 * (j order, in ATen's 16-step blocks beyond k = 16, on the leading 32 * floor(h / 32)
 * columns; ATen's four-slot order on the rest; a row sum when hidden_dim == 1), the
 * sum rounded to dtype. Two launches when hidden_dim is not a multiple of 32.
 * expert_output: [N, hidden_dim], unpermute_index: int64 [n_tokens, k], weights:
 * float32 [n_tokens, k], combined: [n_tokens, hidden_dim]. A negative index
 * drops its term.
 * Replaces reference csrc/includes/token_permute.h:32-41. */
int32_t launch_token_combine_fwd(const void* expert_output, const int64_t* unpermute_index,
                                 const float* weights, void* combined, int64_t n_tokens, int64_t k,
                                 int64_t hidden_dim, int32_t dtype, void* stream);

/* As launch_token_gather_fwd / launch_token_combine_fwd, told the source row
 * count: an index outside [0, n_src_rows) (resp. [0, n_expert_rows)) yields a
 * zero row (resp. drops its term) instead of reading out of bounds. No
 * reference counterpart; the Python binding calls these. */
int32_t launch_token_gather_checked_fwd(const void* src, const int64_t* indices, void* dst,
                                        int64_t n_src_rows, int64_t n_dst_rows, int64_t hidden_dim,
                                        int32_t dtype, void* stream);
int32_t launch_token_combine_checked_fwd(const void* expert_output, const int64_t* unpermute_index,
                                         const float* weights, void* combined, int64_t n_expert_rows,
                                         int64_t n_tokens, int64_t k, int64_t hidden_dim, int32_t dtype,
                                         void* stream);

/* Softmax top-k router: per token, probs = softmax(float(logits)) in torch-CPU's
 * float32 order on an AVX-512 host (SLEEF's expf, 16-lane sums, the reciprocal's
 * product); the k largest (descending; ties to the lower expert index) into topk_weights float32
 * [num_tokens, k] and topk_indices int64 [num_tokens, k], renormalised to sum
 * to 1 when renormalize != 0 (ATen's row-sum order, an IEEE division). num_experts <= 256 and k <= num_experts, else
 * hipErrorInvalidValue.
 * Replaces reference csrc/includes/moe_router.h:20-29. */
int32_t launch_moe_router_fwd(const void* logits, float* topk_weights, int64_t* topk_indices,
                              int64_t num_tokens, int64_t num_experts, int64_t k, int32_t dtype,
                              int32_t renormalize, void* stream);

/* The index bookkeeping between the router and the gather: with i indexing
 * topk_indices int64 [n_tokens, k] flat and entries ordered by (expert id, i),
 * permute_index int64 [n_tokens * k] gets i / k of the p-th entry and
 * unpermute_index int64 [n_tokens, k] gets each entry's position p. This is a
 * stable argsort of the expert ids and its inverse. Ids outside
 * [0, num_experts) are ordered after every expert, by i. 1 <= num_experts <= 256
 * and n_tokens * k <= INT32_MAX, else hipErrorInvalidValue. From 65536
 * entries the call enqueues three kernels on stream and keeps intermediate
 * counts in permute_index until the last one; the three buffers must not
 * overlap.
 * No reference launcher: replaces the torch ops of reference
 * baselines/token_permute.py:55-70 (compute_permutation). */
int32_t launch_moe_permutation_fwd(const int64_t* topk_indices, int64_t* permute_index, int64_t* unpermute_index,
                                   int64_t n_tokens, int64_t k, int64_t num_experts, void* stream);

/* ---- Diagnostics (no reference counterpart): device-side checks of the
 * arithmetic shortcuts used on the FP8 fast path. ---- */

/* Compares the hardware fp32->fp8 conversion with the exact encoder for every
 * fp32 bit pattern in [start, start + count). counters: 8 x u64, zeroed, with
 * [4..7] preset to UINT64_MAX; see csrc/selftest.hip for the layout. */
int32_t cck_fp8_cvt_selftest(uint64_t start, uint64_t count, int32_t fp8_format,
                             unsigned long long* counters, void* stream);

/* Compares the three-op division with IEEE x / s for every (x, s) pair inside
 * the fast-path domain. counters: 5 x u64, zeroed, with [3] preset to
 * UINT64_MAX; see csrc/selftest.hip for the layout. */
int32_t cck_div_selftest(const float* xs, int64_t nx, const float* ss, int64_t ns,
                         unsigned long long* counters, void* stream);

/* Compares the dynamic-scale computation with clamp(amax / FP8_MAX, 1e-12) in
 * IEEE division for amax = every non-negative fp32 pattern in [start,
 * start + count) (sign bit cleared). counters: 2 x u64, [0] zeroed, [1] preset
 * to UINT64_MAX. */
int32_t cck_scale_selftest(uint64_t start, uint64_t count, int32_t fp8_format,
                           unsigned long long* counters, void* stream);

/* Checks the bf16 SiLU table of the SwiGLU+FP8 kernels: both fills against the
 * arithmetic SiLU for every entry, and the table lookup against the arithmetic
 * path for all 2^16 bf16 gates. counters: 6 x u64, zeroed, with [2] preset to
 * UINT64_MAX; [0], [1], [3] are mismatch counts; see csrc/selftest.hip for the
 * layout. */
int32_t cck_silu_table_selftest(unsigned long long* counters, void* stream);

/* Checks the fp32 SwiGLU's sigmoid (torch-CPU's: SLEEF's expf, 1 + e, a
 * division) as the kernels evaluate it against the operation-for-operation
 * form, for every fp32 bit pattern g in [start, start + count) (at most
 * 2^32 - start): counters, 7 x u64, zeroed, with [4..6] preset to
 * UINT64_MAX: [0] expf mismatches, [1] sigmoid mismatches, [2] reciprocal
 * mismatches against IEEE 1 / g on [1, 2^64), [3] patterns checked in [2],
 * [4..6] the lowest mismatching pattern of [0..2]. */
int32_t cck_sigmoid_selftest(uint64_t start, uint64_t count, unsigned long long* counters, void* stream);

/* Test hook (no reference counterpart): sets the number of polls (about
 * 1 us each) a waiting workgroup of the one-pass per-tensor FP8 form
 * (launch_fp8_quant_tensor_fwd and launch_fp8_quant_tensor_noalloc_fwd) makes
 * for the scale before it reads all of x and takes the maximum itself
 * (default 2048); polls < 0 only queries. Returns the previous value. Takes
 * effect for later launches. */
int32_t cck_fp8_tensor_noalloc_poll_limit(int32_t polls);

/* HBM calibration stream (no reference counterpart): one launch of a pure
 * traffic pattern on 16-byte nontemporal vectors, to measure the practical
 * bandwidth ceiling of the ops' access patterns. n_vec counts the 16-byte
 * vectors of one input stream. pattern 0: copy a -> c; 1: two reads, one
 * write (a, b -> c); 2: rows of 512 vectors, two reads and two writes with a
 * workgroup barrier between the stores (a, b -> c, d; n_vec % 512 == 0);
 * 3: read 16 bytes, write 8 (a -> c, c holds 8 * n_vec bytes); 4: rows of
 * 1792 vectors, two 16-byte reads and one 8-byte write per vector (a, b -> c,
 * c holds 8 * n_vec bytes; n_vec % 1792 == 0); 5: rows of 512 vectors, two
 * 16-byte reads, a 16-byte write and an 8-byte write per vector (a, b -> c,
 * d; d holds 8 * n_vec bytes; n_vec % 512 == 0). Unused pointers may be
 * null. hipErrorInvalidValue for an unknown pattern or a partial row. */
int32_t cck_hbm_stream(int32_t pattern, const void* a, const void* b, void* c, void* d, int64_t n_vec,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CUSTOM_KERNELS_AMD_H_ */
