/*
 * efla_hip.h -- C ABI of the MI355X (gfx950) EFLA hot path.
 *
 * Drop-in for the reference's kernel ABI (kernels/cuda/include/kernels.h):
 * same argument order, meaning, tensor layouts and error behaviour, with
 * hipStream_t in place of cudaStream_t.  Every entry returns a hipError_t code
 * as int; the codes the reference returns keep their numbers
 * (0 success, 1 invalid value, 2 out of memory, 9 invalid configuration).
 * Pointers are caller-owned device pointers to contiguous row-major buffers;
 * calls are asynchronous on `stream`.  No entry point allocates per call: the
 * Mode Q entries take a caller workspace, or use scratch the library caches
 * per (device, stream), allocated once and grown only when a larger problem
 * arrives; callers on different streams never share it, and calls on one
 * stream from several host threads take turns while they queue their work.
 *
 * Layouts:
 *   tokens      (B, T, H, D) row-major, i.e. token-major with heads interleaved
 *   Mode R state (B*H, d, d) bf16, row index = key dim, column = value dim
 *   Mode Q state (N, H, d_k, d_v) fp32
 *   beta        (B, T, H), same dtype as q/k/v
 *   cu_seqlens  int32 (N+1) device array of packed sequence offsets, or NULL
 */
#ifndef EFLA_HIP_H
#define EFLA_HIP_H

#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: hipDataType values, equal to the reference's cudaDataType codes */
#define EFLA_DTYPE_F32 0
#define EFLA_DTYPE_F16 2
#define EFLA_DTYPE_BF16 14

/* ========================================================================
 * EFLA, reference ABI ("Mode R")
 * ======================================================================== */

/*
 * Replaces efla_forward_cuda (kernels/cuda/include/kernels.h:35-47,
 * kernels/cuda/efla.cu:482-541).  Per (b, h), token-sequential:
 *   lambda = |k_t|^2, c = (1 - exp(-beta lambda)) / lambda,
 *   S <- bf16(S + c k_t (v_t - S^T k_t)^T), o_t = S k_t   (requires d_k == d_v)
 * k, v, output: (B, T, H, d) bf16.  state: (B*H, d, d) bf16, read as S_0 and
 * overwritten with S_T.  chunk_size (ignored by the reference) is a tuning
 * hint: for d = 64 / 128 the number of tokens staged in LDS at once (16, 32 or
 * 64: the largest not above it, at least 16; 0 -> 32); the results do not
 * depend on it.  Validation order: B, H or d == 0 -> 1; T == 0 -> 0; any null
 * pointer -> 1; B*H or sizes overflowing -> 9.
 * Scratch comes from the stream's cached workspace (leased per call): 4 bytes
 * per (b, t, h) for the coefficients, and for d = 64 / 128 with B*H at most
 * half the device's CU count (two workgroups per (b, h), each owning half of
 * the state's columns) 4 bytes per output element more: one fp32 buffer of
 * row sums both workgroups add into (cfg3's B=4, T=8192, H=32, d=128:
 * 0.54 GB).  `efla_rt_workspace_release_stream` frees a stream's share.
 */
int efla_forward_hip(const void* k, const void* v, void* state, void* output,
                     size_t batch_size, size_t seq_len, size_t num_heads, size_t head_dim,
                     float beta, size_t chunk_size, hipStream_t stream);

/*
 * Replaces efla_backward_cuda (kernels.h:52-66, efla.cu:543-709).  `state` is
 * S_0.  Outputs grad_k, grad_v (B, T, H, d) bf16 and grad_state = dL/dS_0
 * (B*H, d, d) bf16 for the loss sum(output * grad_output).  T == 0 zeroes
 * grad_state and returns 0.  State history is recomputed from checkpoints in a
 * cached workspace instead of the reference's per-call (T+1)*d*d allocation:
 * one bf16 d*d checkpoint per 32 tokens (64 on the LDS-resident path) and one
 * segment's states per (b, h), 8 bytes per (b, t, h) of coefficients, and with
 * the column split (as efla_forward_hip) 4 bytes per grad_k element for the
 * fp32 row sums.
 */
int efla_backward_hip(const void* grad_output, const void* k, const void* v, const void* state,
                      void* grad_k, void* grad_v, void* grad_state, size_t batch_size,
                      size_t seq_len, size_t num_heads, size_t head_dim, float beta,
                      hipStream_t stream);

/*
 * Replaces efla_chunked_scan_cuda (kernels.h:71-77, efla.cu:711-748).
 * chunk_states is a HOST array of num_chunks device pointers, each to H*d*d
 * bf16 values; chunk_states[i] <- bf16(chunk_states[i-1] + chunk_states[i])
 * for i = 1..num_chunks-1 (an inclusive prefix sum, as in the reference).
 */
int efla_chunked_scan_hip(void** chunk_states, size_t num_chunks, size_t num_heads,
                          size_t head_dim, hipStream_t stream);

/* ========================================================================
 * EFLA, chunked query-readout form ("Mode Q")
 *
 * No reference counterpart: the benchmark configurations need a query
 * readout o_t = S_t^T q_t, per-token beta, d_k != d_v, dq, dbeta and varlen
 * packing, none of which the reference ABI expresses.  The state recurrence
 * is the reference's (efla.cu:154-233) with beta per token.
 *
 * q, k (B, T, H, d_k); v, output (B, T, H, d_v); beta (B, T, H); all of
 * `dtype` (EFLA_DTYPE_BF16 or EFLA_DTYPE_F32), fp32 accumulation.  With
 * cu_seqlens != NULL the batch must be 1 and `seq_len` is the packed token
 * count; num_seqs gives the number of sequences (cu_seqlens has num_seqs+1
 * entries); otherwise num_seqs must equal batch_size.  initial_state /
 * final_state (num_seqs, H, d_k, d_v) fp32, either may be NULL.
 * Supported: chunk_size 64 (0 selects 64); (d_k, d_v) in
 * {64,128} x {64,128,256} for bf16, d_k = d_v = 64 for fp32.
 * Workspace: pass NULL to use the library's cached buffer for `stream`, or
 * a buffer of at least efla_chunk_*_workspace_size() bytes.
 * ======================================================================== */
size_t efla_chunk_fwd_workspace_size(size_t batch_size, size_t seq_len, size_t num_seqs,
                                     size_t num_heads, size_t head_dim_k, size_t head_dim_v,
                                     int dtype);

/* flags of efla_chunk_fwd_hip */
/* Also write each chunk's start state (bf16) and, on the bf16 path, its
 * P = tril(Q K^T) (bf16) into the caller-owned `workspace`, where a backward
 * call with EFLA_BWD_REUSE_STATES reads them instead of recomputing the state
 * scan and the P tiles.  Requires a non-NULL workspace of at least
 * efla_chunk_bwd_workspace_size() bytes (the one the backward will get). */
#define EFLA_FWD_SAVE_STATES 1u

/* flags: 0 or EFLA_FWD_SAVE_STATES (other bits -> 1). */
int efla_chunk_fwd_hip(const void* q, const void* k, const void* v, const void* beta,
                       const float* initial_state, void* output, float* final_state,
                       const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                       size_t num_seqs, size_t num_heads, size_t head_dim_k,
                       size_t head_dim_v, size_t chunk_size, int dtype, void* workspace,
                       size_t workspace_bytes, unsigned flags, hipStream_t stream);

size_t efla_chunk_bwd_workspace_size(size_t batch_size, size_t seq_len, size_t num_seqs,
                                     size_t num_heads, size_t head_dim_k, size_t head_dim_v,
                                     int dtype);

/* flags of efla_chunk_bwd_hip */
/* The caller-owned `workspace` is the one the forward call on these exact
 * inputs (same q, k, v, beta, cu_seqlens, shapes) used, and nothing has
 * written to it since: the backward takes the forward's per-chunk WY factors
 * (W, U, T) and per-token coefficients (b, dc/dlambda, dc/dbeta) from it
 * instead of recomputing them.  The chunk states are
 * recomputed unless EFLA_BWD_REUSE_STATES is also set.  Requires a non-NULL
 * workspace of at least efla_chunk_bwd_workspace_size() bytes, also passed to
 * the forward. */
#define EFLA_BWD_REUSE_FORWARD 1u
/* With EFLA_BWD_REUSE_FORWARD only: the forward also ran with
 * EFLA_FWD_SAVE_STATES on this workspace, so the chunk states and P are read
 * from it too and the backward runs no forward recompute at all (bf16; the
 * fp32 path accepts the flag and recomputes the states). */
#define EFLA_BWD_REUSE_STATES 2u

/* Gradients of sum(output * grad_output) + sum(final_state * grad_final_state);
 * grad_final_state and grad_initial_state may be NULL.  flags: 0,
 * EFLA_BWD_REUSE_FORWARD or EFLA_BWD_REUSE_FORWARD | EFLA_BWD_REUSE_STATES
 * (anything else -> 1). */
int efla_chunk_bwd_hip(const void* q, const void* k, const void* v, const void* beta,
                       const float* initial_state, const void* grad_output,
                       const float* grad_final_state, void* grad_q, void* grad_k,
                       void* grad_v, void* grad_beta, float* grad_initial_state,
                       const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                       size_t num_seqs, size_t num_heads, size_t head_dim_k,
                       size_t head_dim_v, size_t chunk_size, int dtype, void* workspace,
                       size_t workspace_bytes, unsigned flags, hipStream_t stream);

/*
 * No reference counterpart (the reference slices its projections into
 * separate buffers).  efla_chunk_fwd_hip / efla_chunk_bwd_hip with explicit
 * token strides, so q, k, v (and grad_q, grad_k, grad_v) can be column slices
 * of one fused projection row, [q | k | v | beta-logit] per token, read and
 * written in place without copies.  token_strides[i] is the number of
 * elements from one token's row to the next's: q, k, v for the forward;
 * q, k, v, grad_q, grad_k, grad_v for the backward; NULL means packed
 * (H*d_k, H*d_k, H*d_v, ...).  Within a row, heads stay packed (head h at
 * h*d).  output, grad_output and beta stay packed.  A non-packed stride must
 * be at least the packed one, a multiple of 8 elements and below 2^24, with
 * its pointer 16-byte aligned (else 1); non-packed strides with the fp32
 * path return 801.  Everything else is as in the packed entry points.
 */
int efla_chunk_fwd_strided_hip(const void* q, const void* k, const void* v, const void* beta,
                               const float* initial_state, void* output, float* final_state,
                               const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                               size_t num_seqs, size_t num_heads, size_t head_dim_k,
                               size_t head_dim_v, size_t chunk_size, int dtype,
                               void* workspace, size_t workspace_bytes, unsigned flags,
                               const int64_t* token_strides, hipStream_t stream);

int efla_chunk_bwd_strided_hip(const void* q, const void* k, const void* v, const void* beta,
                               const float* initial_state, const void* grad_output,
                               const float* grad_final_state, void* grad_q, void* grad_k,
                               void* grad_v, void* grad_beta, float* grad_initial_state,
                               const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                               size_t num_seqs, size_t num_heads, size_t head_dim_k,
                               size_t head_dim_v, size_t chunk_size, int dtype,
                               void* workspace, size_t workspace_bytes, unsigned flags,
                               const int64_t* token_strides, hipStream_t stream);

/*
 * No reference counterpart.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): efla_chunk_fwd_hip with no workspace argument and no flags,
 * whose per-chunk factors go to a fixed device array of
 * EFLA_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends.  The call allocates nothing.  A problem whose
 * forward workspace (efla_chunk_fwd_workspace_size) exceeds that size returns
 * 2 (out of memory) before any work is queued; every other argument and
 * return code is as in efla_chunk_fwd_hip, and the results are identical to
 * its.  All calls on one GPU share the array: calls that overlap on one GPU
 * (on different streams, or from different host threads) race and must be
 * serialised by the caller.
 */
#define EFLA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

int efla_chunk_fwd_noalloc_hip(const void* q, const void* k, const void* v, const void* beta,
                               const float* initial_state, void* output, float* final_state,
                               const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                               size_t num_seqs, size_t num_heads, size_t head_dim_k,
                               size_t head_dim_v, size_t chunk_size, int dtype,
                               hipStream_t stream);

/* No reference counterpart; the affine combine efla_chunked_scan_hip does not
 * do (efla.cu:711-748 sums states; src/model/efla.zig:473-484 is empty).
 * In place over consecutive segments of the same sequences:
 *   states[i] = transitions[i] * states[i-1] + states[i],  i = 1 .. n-1,
 * where states[i] (num_states, d_k, d_v) fp32 holds on entry the segment's
 * final state from a zero start (B_i) and transitions[i] (num_states, d_k,
 * d_k) fp32 its state transition A_i = prod_t (I - c_t k_t k_t^T) (the final
 * state of efla_chunk_fwd_hip on the segment with S_0 = I and v = 0).  On
 * return states[i] is the true state after segment i.  Host arrays of device
 * pointers; transitions[0] is not read.  Zero sizes or NULL -> 1;
 * d_k > 256 -> 9. */
int efla_affine_state_scan_hip(const float* const* transitions, float* const* states,
                               size_t num_chunks, size_t num_states, size_t head_dim_k,
                               size_t head_dim_v, hipStream_t stream);

/* ========================================================================
 * LayerNorm
 * ======================================================================== */

/* Replaces layernorm_forward_cuda (kernels.h:153-162, layernorm.cu:359-383):
 * rows = numel / normalized_shape; y = (x - mean) * rsqrt(var + eps) * w + b,
 * bias may be NULL.  bf16 in/out, fp32 statistics. */
int layernorm_forward_hip(const void* input, const void* weight, const void* bias, void* output,
                          size_t numel, size_t normalized_shape, float eps, hipStream_t stream);

/* No reference counterpart (the reference has no LayerNorm backward): the
 * forward above that also stores per-row fp32 mean and rstd for the backward. */
int layernorm_forward_stats_hip(const void* input, const void* weight, const void* bias,
                                void* output, float* mean, float* rstd, size_t numel,
                                size_t normalized_shape, float eps, hipStream_t stream);

/* No reference counterpart.  grad_input bf16; grad_weight / grad_bias fp32
 * (either may be NULL).  Uses the cached workspace for per-block partials. */
int layernorm_backward_hip(const void* grad_output, const void* input, const void* weight,
                           const float* mean, const float* rstd, void* grad_input,
                           float* grad_weight, float* grad_bias, size_t numel,
                           size_t normalized_shape, hipStream_t stream);

/* No reference counterpart: layernorm_backward_hip with grad_input =
 * LayerNorm's input gradient + residual (bf16, same shape), the add a
 * pre-LN residual block does after each LayerNorm backward, fused into the
 * row pass.  residual NULL (with rows to do) -> 1. */
int layernorm_backward_residual_hip(const void* grad_output, const void* input,
                                    const void* weight, const float* mean, const float* rstd,
                                    const void* residual, void* grad_input, float* grad_weight,
                                    float* grad_bias, size_t numel, size_t normalized_shape,
                                    hipStream_t stream);

/* No reference counterpart: the general LayerNorm backward.  residual (added
 * to grad_input) may be NULL; grad_weight, grad_bias and grad_input_colsum
 * may each be NULL.  grad_weight / grad_bias are fp32, or bf16 when
 * param_grads_bf16 is non-zero (written straight into a bf16 gradient
 * buffer, the sums still taken in fp32).  grad_input_colsum receives the
 * column sums of grad_input as written (bf16, normalized_shape values): the
 * gradient of a bias of the product whose output gradient grad_input is,
 * summed in the same row pass (D a multiple of 512 up to 2048, 16-byte
 * aligned rows) or in a pass of its own. */
int layernorm_backward_ex_hip(const void* grad_output, const void* input, const void* weight,
                              const float* mean, const float* rstd, const void* residual,
                              void* grad_input, void* grad_weight, void* grad_bias,
                              void* grad_input_colsum, size_t numel, size_t normalized_shape,
                              int param_grads_bf16, hipStream_t stream);

/* ========================================================================
 * RMSNorm
 * ======================================================================== */

/* Replaces rmsnorm_forward_cuda (kernels.h:125-133, layernorm.cu:15-48,
 * 307-329): rows = numel / normalized_shape; y = x * rsqrt(mean(x^2) + eps)
 * * w.  bf16 in/out, fp32 statistics.  normalized_shape == 0 or a NULL
 * pointer -> 1; no whole row -> 0 with nothing launched. */
int rmsnorm_forward_hip(const void* input, const void* weight, void* output, size_t numel,
                        size_t normalized_shape, float eps, hipStream_t stream);

/* Replaces rmsnorm_backward_cuda (kernels.h:138-148, layernorm.cu:51-127,
 * 331-357) with the exact gradient, rs = rsqrt(mean(x^2) + eps), g = dy * w:
 *   grad_input = rs g - x rs^3 mean(g x)    (bf16)
 *   grad_weight += sum over rows of dy x rs (fp32, may be NULL).
 * The reference scales the second term by rs instead of rs^3 and adds fp32
 * values through a float pointer into a bf16 buffer; both are corrected here
 * and grad_weight is an fp32 accumulator.  grad_weight with normalized_shape
 * > 16384 -> 9.  Uses the cached workspace for per-block partials. */
int rmsnorm_backward_hip(const void* grad_output, const void* input, const void* weight,
                         void* grad_input, float* grad_weight, size_t numel,
                         size_t normalized_shape, float eps, hipStream_t stream);

/* ========================================================================
 * ShortConv and PRISM (the consumer of the EFLA output in the reference's
 * TransformerBlock, src/model/model.zig:169-176)
 * ======================================================================== */

/* Replaces shortconv_forward_cuda (kernels.h:107-116, declared only), with the
 * semantics of ShortConv.forwardCpu (src/model/prism.zig:448-473): a causal
 * depthwise convolution over (batch, seq_len, hidden_dim) bf16 with weight
 * (hidden_dim, window_size) bf16,
 *   y[b,t,c] = bf16(sum_{w < W, t-w >= 0} x[b,t-w,c] * weight[c,w]),
 * the fp32 terms added in increasing w, bit-identical to that loop (a bf16
 * product is exact in fp32 unless it falls below fp32's normal range).  No
 * element -> 0; a NULL pointer -> 1. */
int shortconv_forward_hip(const void* input, const void* weight, void* output,
                          size_t batch_size, size_t seq_len, size_t hidden_dim,
                          size_t window_size, hipStream_t stream);

/* Replaces shortConvBackwardCuda (src/kernels/prism_kernels.zig:50-60,
 * declared only): grad_input (bf16, may be NULL) and grad_weight (fp32
 * (hidden_dim, window_size), added into, may be NULL). */
int shortconv_backward_hip(const void* grad_output, const void* input, const void* weight,
                           void* grad_input, float* grad_weight, size_t batch_size,
                           size_t seq_len, size_t hidden_dim, size_t window_size,
                           hipStream_t stream);

/* Replaces prism_forward_cuda (kernels.h:86-102, declared only), with the
 * semantics of PrismLayer.prismForwardCpu (src/model/prism.zig:251-323): for
 * every row and channel d < head_dim, r = v - u and for each of the
 * num_iterations steps l: delta = GELU_tanh(w_p[l][d] * r),
 * o = bf16(o + 0.5 delta), r -= delta; channels >= head_dim are 0.  w_p is a
 * host array of num_iterations device pointers (bf16, at least head_dim
 * values each).  As in that path, prev_state, w_beta, w_k and alpha are not
 * read; new_state (head_dim x head_dim bf16) is zero-filled when non-NULL.
 * head_dim == 0 or > hidden_dim, or a NULL pointer -> 1; more than 16
 * iterations -> 9. */
int prism_forward_hip(const void* u, const void* v, const void* prev_state, void* new_state,
                      void* output, const void** w_beta, const void** w_k, const void** w_p,
                      size_t batch_size, size_t seq_len, size_t hidden_dim, size_t head_dim,
                      size_t num_iterations, float alpha, hipStream_t stream);

/* No usable reference counterpart (prismBackwardCuda, prism_kernels.zig:24-37,
 * takes no weights; PrismLayer.backward, prism.zig:326-356, returns zeros):
 * the gradient of prism_forward_hip with the bf16 rounding of o passed
 * straight through.  grad_u, grad_v bf16 (full rows; 0 beyond head_dim);
 * grad_w_p a host array of num_iterations fp32 device pointers, each added
 * into over its first head_dim values (may be NULL).  When hidden_dim and
 * head_dim are multiples of 8, head_dim / 8 divides 256, the activations are
 * 16-byte aligned and num_iterations <= 4, the sums run in a fixed order
 * through a cached workspace of 4 * num_iterations * head_dim bytes per 16
 * rows; otherwise they are added with float atomics and their order varies
 * between runs. */
int prism_backward_hip(const void* grad_output, const void* u, const void* v, const void** w_p,
                       void* grad_u, void* grad_v, float** grad_w_p, size_t batch_size,
                       size_t seq_len, size_t hidden_dim, size_t head_dim,
                       size_t num_iterations, hipStream_t stream);

/* ========================================================================
 * GEMM (row-major)
 *
 * Hand-written MFMA kernels: bf16 / fp16 problems whose k, output columns
 * and strides are multiples of 8 elements (16-byte rows) run a 256 x 256 x 64
 * tile kernel; everything else (fp32, mixed dtypes, other shapes) a generic
 * 128 x 128 one (efla_rt_set_gemm_backend(1) forces it).  No vendor BLAS
 * is linked.
 * ======================================================================== */

/* Replaces gemm_forward_cuda (kernels.h:211-223, gemm.cu:303-398):
 * c[m x n] = a[m x k] * b[k x n] (+ bias[n]), fp32 accumulation; dtypes are
 * EFLA_DTYPE_* codes for each operand.  m or n == 0 -> 0; k == 0 -> c = bias
 * (or 0). */
int gemm_forward_hip(const void* a, const void* b, const void* bias, void* c, size_t m,
                     size_t k, size_t n, int dtype_a, int dtype_b, int dtype_c,
                     hipStream_t stream);

/* Replaces gemm_backward_cuda (kernels.h:228-239, gemm.cu:400-548), bf16:
 * grad_a = grad_c * b^T, grad_b = a^T * grad_c, grad_bias = column sums of
 * grad_c; a NULL gradient pointer skips that product. */
int gemm_backward_hip(const void* grad_c, const void* a, const void* b, void* grad_a,
                      void* grad_b, void* grad_bias, size_t m, size_t k, size_t n,
                      hipStream_t stream);

/* No reference counterpart as an entry point (gemm.cu:182-234 keeps its
 * strided helper gemm_row_major_ex internal): the strided, accumulating
 * product the training step's projections use,
 *   D[m x n] = alpha op(A) op(B) (+ bias[n]) + beta C,
 * row-major with row strides lda, ldb, ldc, ldd; op(A) is A (stored m x k) or,
 * with trans_a, A^T (A stored k x m); op(B) likewise (k x n or, transposed,
 * n x k).  One dtype for every operand, fp32 accumulation.  C is read only
 * when beta != 0 and may be D; k == 0 gives D = bias + beta C without
 * reading A or B (they may be NULL, their strides are not checked).  m or
 * n == 0 -> 0; bad strides or pointers -> 1. */
int gemm_ex_hip(int trans_a, int trans_b, size_t m, size_t n, size_t k, float alpha,
                const void* a, size_t lda, const void* b, size_t ldb, const void* bias,
                float beta, const void* c, size_t ldc, void* d, size_t ldd, int dtype,
                hipStream_t stream);

/* No reference counterpart: the MLP's first product with the GELU fused into
 * its epilogue (bf16, row-major, contiguous),
 *   pre[m x n] = a[m x k] b[k x n] + bias[n]   (bias may be NULL)
 *   out        = GELU_tanh(pre)                 (computed from bf16(pre))
 * pre is written for the backward.  Same codes as gemm_forward_hip. */
int gemm_gelu_forward_hip(const void* a, const void* b, const void* bias, void* pre, void* out,
                          size_t m, size_t k, size_t n, hipStream_t stream);

/* No reference counterpart: gemm_backward_hip for c = GELU_tanh(pre) b + bias
 * with the GELU derivative fused into grad_a's epilogue,
 *   grad_pre      = bf16(grad_c b^T) * GELU'(pre)   (m x k; NULL skips it)
 *   grad_b        = a^T grad_c                      (k x n, a = GELU(pre); NULL skips it)
 *   grad_bias     = column sums of grad_c           (n; NULL skips it)
 *   grad_pre_bias = column sums of grad_pre         (k; NULL skips it; needs
 *                   grad_pre): the gradient of the bias of the product that
 *                   made pre, summed in grad_pre's epilogue
 * bf16, row-major, contiguous.  Same codes as gemm_backward_hip. */
int gemm_gelu_backward_hip(const void* grad_c, const void* a, const void* b, const void* pre,
                           void* grad_pre, void* grad_b, void* grad_bias, void* grad_pre_bias,
                           size_t m, size_t k, size_t n, hipStream_t stream);

/* ========================================================================
 * GELU and AdamW (the config-4 training step around EFLA)
 * ======================================================================== */

/* Replaces gelu_forward_cuda (kernels.h:171-177, layernorm.cu:189-214,
 * 385-403): y = GELU(x), bf16 in / out, fp32 math; approximate selects the
 * tanh form 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), otherwise
 * x Phi(x).  numel == 0 -> 9 (the reference launches an empty grid); a NULL
 * pointer -> 1. */
int gelu_forward_hip(const void* input, void* output, size_t numel, bool approximate,
                     hipStream_t stream);

/* Replaces gelu_backward_cuda (kernels.h:182-189, layernorm.cu:216-250,
 * 405-425): grad_input = grad_output * GELU'(input), bf16.  Same return codes
 * as gelu_forward_hip. */
int gelu_backward_hip(const void* grad_output, const void* input, void* grad_input,
                      size_t numel, bool approximate, hipStream_t stream);

/* Replaces adamw_step_cuda (kernels.h:309-322, optim.cu:147-178, 657-709):
 * bf16 param, grad, exp_avg, exp_avg_sq updated in place with fp32 math,
 *   m = b1 m + (1 - b1) g,  v = b2 v + (1 - b2) g^2,
 *   p = p (1 - lr wd) - lr (m / bc1) / (sqrt(v / bc2) + eps),
 * bc = 1 - beta^step in double.  numel == 0 -> 0; a NULL pointer -> 1;
 * non-finite hyper-parameters, beta outside [0, 1), eps <= 0 or step == 0
 * -> 1. */
int adamw_step_hip(void* param, const void* grad, void* exp_avg, void* exp_avg_sq, size_t numel,
                   float lr, float beta1, float beta2, float eps, float weight_decay, size_t step,
                   hipStream_t stream);

/* No reference counterpart (the reference keeps bf16 optimizer state): the
 * same step on fp32 master weights and fp32 moments with a bf16 gradient;
 * param_bf16, if not NULL, receives the new weights rounded to bf16.  Same
 * return codes as adamw_step_hip. */
int adamw_step_master_hip(float* param, const void* grad, float* exp_avg, float* exp_avg_sq,
                          void* param_bf16, size_t numel, float lr, float beta1, float beta2,
                          float eps, float weight_decay, size_t step, hipStream_t stream);

/* No reference counterpart: the per-token beta gate of a model whose fused
 * projection row ends in `cols` beta logits (the config-4 model, one logit
 * per head).  beta[r*cols + c] = bf16(sigmoid(float(logits[r*ld + c]))) for
 * r < rows, c < cols; fp32 math.  rows or cols == 0 -> 0; a NULL pointer or
 * ld < cols -> 1; ld >= 2^24 or rows > 2^40 -> 9. */
int sigmoid_gate_forward_hip(const void* logits, size_t ld, void* beta, size_t rows,
                             size_t cols, hipStream_t stream);

/* Its gradient: grad_logits[r*ld + c] = bf16((float(grad_beta[i]) * b) * (1 - b))
 * with i = r*cols + c and b = float(beta[i]); grad_beta and beta packed
 * (rows, cols).  Same return codes as sigmoid_gate_forward_hip. */
int sigmoid_gate_backward_hip(const void* grad_beta, const void* beta, void* grad_logits,
                              size_t ld, size_t rows, size_t cols, hipStream_t stream);

/* ========================================================================
 * Token embedding and cross-entropy (the ends of the config-4 step)
 * ======================================================================== */

/* Replaces embedding_forward_cuda (kernels.h:366-373; declared only in the
 * reference, semantics of Embedding.forward, layers.zig:658-686):
 * output[i, :] = weight[indices[i], :], bf16, indices int32.  Like the
 * reference entry it cannot range-check (no vocabulary size): every index
 * must be valid.  num_indices == 0 -> 0; NULL or embedding_dim == 0 -> 1. */
int embedding_forward_hip(const int32_t* indices, const void* weight, void* output,
                          size_t num_indices, size_t embedding_dim, hipStream_t stream);

/* No reference counterpart: embedding_forward_hip with the vocabulary size;
 * an index outside [0, num_embeddings) gives a zero row. */
int embedding_forward_checked_hip(const int32_t* indices, const void* weight, void* output,
                                  size_t num_indices, size_t num_embeddings,
                                  size_t embedding_dim, hipStream_t stream);

/* No reference counterpart: grad_weight[indices[i], :] += grad_output[i, :]
 * in fp32 (grad_weight is accumulated into, not cleared; duplicate indices
 * add in no fixed order); indices out of range are skipped. */
int embedding_backward_hip(const void* grad_output, const int32_t* indices, float* grad_weight,
                           size_t num_indices, size_t num_embeddings, size_t embedding_dim,
                           hipStream_t stream);

/* Replaces cross_entropy_forward_cuda (kernels.h:248-256; declared only,
 * semantics of crossEntropyForwardCpu, nn_kernels.zig:200-246): logits
 * (batch, vocab) bf16, targets int32, loss (batch,) fp32 with
 *   loss[i] = ((1 - eps) (logsumexp(z_i) - z_i,t) + eps log vocab) / batch,
 * so sum(loss) is the mean loss.  A target outside [0, vocab) gives NaN.
 * batch == 0 -> 0; NULL, vocab == 0 or eps outside [0, 1) -> 1. */
int cross_entropy_forward_hip(const void* logits, const int32_t* targets, void* loss,
                              size_t batch_size, size_t vocab_size, float label_smoothing,
                              hipStream_t stream);

/* Replaces cross_entropy_backward_cuda (kernels.h:261-270): grad_loss
 * (batch,) fp32 is dL/dloss[i]; grad_logits (batch, vocab) bf16 =
 * grad_loss[i] (1 - eps) (softmax(z_i) - onehot(t_i)) / batch.  Same return
 * codes as the forward. */
int cross_entropy_backward_hip(const void* grad_loss, const void* logits, const int32_t* targets,
                               void* grad_logits, size_t batch_size, size_t vocab_size,
                               float label_smoothing, hipStream_t stream);

/* No reference counterpart: cross_entropy_forward_hip and
 * cross_entropy_backward_hip from one read of the logits.  loss[i] as the
 * forward; grad_logits as the backward with dL/dloss[i] = grad_loss[i]
 * (grad_loss NULL: 1 for every row, the gradient of the summed rows).
 * grad_logits may be logits itself (overwritten in place).  Same codes as
 * the two entries. */
int cross_entropy_forward_backward_hip(const void* logits, const int32_t* targets,
                                       const float* grad_loss, float* loss, void* grad_logits,
                                       size_t batch_size, size_t vocab_size,
                                       float label_smoothing, hipStream_t stream);

/* ========================================================================
 * Sequence packing (host, no GPU)
 * ======================================================================== */

/* Replaces packSequences (src/data/dataset.zig:421-465): the sequences are
 * given concatenated in `tokens` with their `lengths`; each is packed in
 * order if it fits in what is left of max_length and skipped otherwise.
 * Outputs (each may be NULL): packed_tokens, positions (index within its
 * sequence) and sequence_ids, max_length entries each; cu_seqlens int32, at
 * most num_sequences_in + 1 entries, starting at 0 (the reference's
 * cumulative_lengths are cu_seqlens[1..]).  Host memory; returns 0, 1 for a
 * NULL count pointer or NULL inputs, 9 when max_length exceeds INT32_MAX. */
int efla_pack_sequences(const uint32_t* tokens, const size_t* lengths, size_t num_sequences_in,
                        size_t max_length, uint32_t* packed_tokens, size_t* positions,
                        size_t* sequence_ids, int32_t* cu_seqlens, size_t* num_tokens_out,
                        size_t* num_sequences_out);

#ifdef __cplusplus
}
#endif

#endif /* EFLA_HIP_H */
