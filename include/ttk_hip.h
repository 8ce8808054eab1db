/*
 * ttk_hip.h - C ABI of the MI355X (gfx950) fused attention, fused
 * residual-add + LayerNorm and exact-GELU kernels.
 *
 * Plain C: no HIP, no torch types.  Every tensor is a raw device pointer plus
 * element strides.  The caller owns all memory (inputs and outputs); the
 * library never allocates, frees, retains a pointer past the call, or
 * synchronises.  Each call enqueues its kernel(s) on `stream` (a hipStream_t
 * passed as void*; NULL is the legacy default stream), so calls are legal
 * inside hipGraph stream capture.
 *
 * Errors: every entry point returns a ttk_status.  On failure the message is
 * available from ttk_last_error() on the calling thread (thread-local).  No
 * entry point falls back to another implementation.
 *
 * Library: libttk_hip.so, built by triton-transformer-kernels_amd/build.py.
 */
#ifndef TTK_HIP_H
#define TTK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTK_ABI_VERSION 9

/* Bytes of the arrival-counter block that leads every attention workspace
 * (and the library's static scratch): the same for every launch shape. */
#define TTK_ATTENTION_WS_COUNTER_BYTES 16384

typedef enum {
  TTK_OK = 0,
  TTK_EINVAL = 1,       /* malformed arguments: null pointer, bad size/stride */
  TTK_EUNSUPPORTED = 2, /* well-formed but outside the kernels' envelope     */
  TTK_ELAUNCH = 3       /* the HIP runtime rejected the launch               */
} ttk_status;

typedef enum { TTK_F32 = 0, TTK_BF16 = 1, TTK_F16 = 2 } ttk_dtype;

/* Activation applied by ttk_linear_fwd to the rounded linear output. */
typedef enum { TTK_ACT_NONE = 0, TTK_ACT_GELU = 1 } ttk_activation;

/* Version of this ABI (TTK_ABI_VERSION of the built library). */
int ttk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ttk_last_error(void);

/*
 * Fused forward attention over the [B, S, H, D] ("BSHD") layout:
 *
 *   out[b,s,h,:] = sum_t P[s,t] * v[b,t,h,:],
 *   P[s,:] = softmax_t( scale * <q[b,s,h,:], k[b,t,h,:]> ) over allowed t,
 *   allowed(s,t) = key_valid[b,t] (if given) && (!causal || t <= s).
 *
 * Softmax statistics and the output accumulator are fp32; the score matrix is
 * never materialised.  A query row with no allowed key produces exact zeros.
 * Causal launches never visit key tiles past the query tile's diagonal.
 *
 * q/k/v/out: device pointers of dtype `dtype` (TTK_F32, TTK_BF16, TTK_F16).
 * *_strides[3]: element strides of the B, S and H axes; the D axis has
 *   stride 1.  Rows must be 16-byte aligned (pointer and every stride times
 *   the element size a multiple of 16 bytes) - otherwise TTK_EUNSUPPORTED.
 * key_valid: NULL, or a [B, S] byte mask (nonzero = valid) with element
 *   strides mask_strides[2] (mask_strides may be NULL when key_valid is).
 * D must be one of 8, 16, 32, 64, 128.
 * Limits (TTK_EUNSUPPORTED beyond them): S <= 2^24; B * H * ceil(S / 128)
 * <= 16777215 (2^32 - 1 work-items of 256-thread workgroups, the HIP grid
 * limit); K and V sequence strides below 2^25 elements.
 *
 * Replaces the launch of `_attention_fwd` inside `triton_attention`
 * (reference transformer_opt/kernels/attention.py:268-360, kernel :103-265);
 * the argument meaning (BSHD strides, optional [B,S] key mask, causal flag,
 * softmax scale) is that launch's.
 */
ttk_status ttk_attention_fwd(const void* q, const void* k, const void* v,
                             const uint8_t* key_valid, void* out, int dtype,
                             int64_t B, int64_t S, int64_t H, int64_t D,
                             const int64_t q_strides[3],
                             const int64_t k_strides[3],
                             const int64_t v_strides[3],
                             const int64_t mask_strides[2],
                             const int64_t o_strides[3], float scale,
                             int causal, void* stream);

/*
 * Workspace bytes ttk_attention_fwd_ws uses for this launch on the current
 * device; 0 when the launch needs none (every launch but a causal bf16/fp16
 * one whose heaviest query tile outweighs 1.5 average workgroup slots).
 * Also 0 for arguments ttk_attention_fwd would reject.
 *
 * No counterpart in the reference (its Triton launch has no workspace); it
 * sizes the buffer of the key-split schedule below.
 */
size_t ttk_attention_workspace_size(int dtype, int64_t B, int64_t S, int64_t H,
                                    int64_t D, int causal);

/*
 * ttk_attention_fwd with a caller-owned workspace (256-byte aligned,
 * workspace_bytes long).  The workspace starts with the schedule's arrival
 * counters, a block of TTK_ATTENTION_WS_COUNTER_BYTES whatever the shape;
 * those must be zero before the first call, and every call leaves them zero,
 * so one workspace serves launches of any shapes in any order.  The rest
 * needs no initialisation.
 *
 * With at least ttk_attention_workspace_size() bytes, a causal bf16/fp16
 * launch whose heaviest query tile outweighs 1.5 average workgroup slots
 * cuts each query tile that sees more key tiles than the average slot
 * carries into key chunks, run as separate workgroups whose partial softmax
 * states (integer reference exponent, row sum, accumulators) are merged by
 * the chunk that finishes last - the launch no longer lasts as long as its
 * heaviest query tile.  With less (or NULL), the call equals
 * ttk_attention_fwd.  Calls that share a workspace must not overlap (same
 * stream, or ordered by events).
 *
 * Replaces the same launch as ttk_attention_fwd (reference
 * transformer_opt/kernels/attention.py:306-360); the workspace is this
 * build's addition.
 */
ttk_status ttk_attention_fwd_ws(const void* q, const void* k, const void* v,
                                const uint8_t* key_valid, void* out, int dtype,
                                int64_t B, int64_t S, int64_t H, int64_t D,
                                const int64_t q_strides[3],
                                const int64_t k_strides[3],
                                const int64_t v_strides[3],
                                const int64_t mask_strides[2],
                                const int64_t o_strides[3], float scale,
                                int causal, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * ttk_attention_fwd_ws without a caller workspace and without any device
 * allocation: the key-split schedule keeps its counters and partial states
 * in a static 32 MiB device array of the library (one per GPU, held until
 * the process ends), whose address is looked up once per device.  A launch
 * whose schedule needs more than that (ttk_attention_workspace_size() >
 * 33554432) is rejected with TTK_EUNSUPPORTED; launches that need no
 * workspace run as ttk_attention_fwd.  All calls on one GPU share the array:
 * calls that overlap on one GPU (different streams, unordered) race.  Each
 * launch leaves the array's counters zero, as they start.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory or pass a workspace: code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc.
 */
ttk_status ttk_attention_fwd_noalloc(const void* q, const void* k, const void* v,
                                     const uint8_t* key_valid, void* out, int dtype,
                                     int64_t B, int64_t S, int64_t H, int64_t D,
                                     const int64_t q_strides[3],
                                     const int64_t k_strides[3],
                                     const int64_t v_strides[3],
                                     const int64_t mask_strides[2],
                                     const int64_t o_strides[3], float scale,
                                     int causal, void* stream);

/*
 * Fused residual add + LayerNorm over `rows` contiguous rows of width N:
 *
 *   r = x + u                        (u == NULL means r = x)
 *   if zero_invalid_residual:   r[row] = 0 where row_valid[row] == 0
 *   y = (r - mean(r)) * rsqrt(var(r) + eps) * w + b   (biased variance)
 *   if zero_invalid_normalized: y[row] = 0 where row_valid[row] == 0
 *
 * Writes r to residual_out (skipped when residual_out == NULL) and y to
 * normalized_out.  Statistics are fp32; r is rounded to `dtype` before the
 * statistics are taken, exactly as an eager `x + u` followed by a LayerNorm.
 * x, u, residual_out, normalized_out: rows*N contiguous elements of `dtype`;
 * w: N elements; b: N elements or NULL; row_valid: `rows` bytes or NULL
 * (required when either zeroing flag is set).
 * Limits (TTK_EUNSUPPORTED beyond them): N <= 65536; the launch grid at most
 * 16777215 workgroups - rows <= 16777215 for widths that take the
 * one-workgroup-per-row path (N not a multiple of 16 bytes, unaligned
 * buffers, or more than 16 vectors per lane), and 4 * 64 / lanes_per_row
 * times that for the others (at least 4 * 16777215 rows).
 *
 * Replaces the launch of `_residual_layer_norm_fwd` inside
 * `fused_residual_layer_norm` (reference
 * transformer_opt/kernels/residual_layer_norm.py:159-237, kernel :73-126).
 */
ttk_status ttk_residual_layernorm_fwd(const void* x, const void* u,
                                      const void* w, const void* b,
                                      const uint8_t* row_valid,
                                      void* residual_out, void* normalized_out,
                                      int dtype, int64_t rows, int64_t N,
                                      float eps, int zero_invalid_residual,
                                      int zero_invalid_normalized,
                                      void* stream);

/*
 * Exact (erf) GELU, elementwise: y[i] = x[i] * Phi(x[i]) for i < n, computed
 * in fp32 and rounded once to `dtype` (TTK_F32, TTK_BF16 or TTK_F16).  x and
 * y are contiguous; y == x (in place) is allowed, any other overlap is
 * TTK_EINVAL.  16-byte aligned buffers take the vector path.  n <=
 * 4294967040 (2^32 - 256: an unaligned buffer runs one element per
 * work-item), else TTK_EUNSUPPORTED.
 *
 * Replaces the separate GELU pass of the encoder's FFN,
 * `F.gelu(layer.ffn_in(ffn_input), approximate="none")` (reference
 * transformer_opt/submission.py:507; benchmarks/torch_transformer_benchmark.py:
 * 95-97), on the library GEMM's output.
 */
ttk_status ttk_gelu_fwd(const void* x, void* y, int dtype, int64_t n, void* stream);

/*
 * Linear layer with an optional exact (erf) GELU, bf16 / fp16:
 *
 *   Y = act( round( X W^T + bias ) )
 *
 * X [M, K] (row stride ldx elements), W [N, K] (the nn.Linear weight, row
 * stride ldw), bias [N] or NULL, Y [M, N] (row stride ldy), all of `dtype`.
 * The product accumulates in fp32 and bias is added in fp32; the sum is
 * rounded to dtype (round to nearest even), and with TTK_ACT_GELU the GELU of
 * that rounded value is rounded again - the dtype boundaries of
 * F.gelu(F.linear(x, W, b)) in 16-bit torch.  The bf16 GELU is exact: every
 * result equals the correctly rounded x * Phi(x) of its input.
 *
 * Requirements (TTK_EUNSUPPORTED otherwise): dtype TTK_BF16 or TTK_F16; K a
 * multiple of 128 and at least 256; N a multiple of 32; x, w and y 16-byte
 * aligned, ldx, ldw and ldy multiples of 8 with ldx, ldw >= K and ldy >= N;
 * bias 4-byte aligned; ((M - 1) * ldx + K) * 2 and ((N - 1) * ldw + K) * 2
 * below 2^32 and M * ldy * 2 below 2^31.  y must not overlap x, w or bias
 * (TTK_EINVAL).  M == 0 is a no-op.
 *
 * Replaces the FFN input projection and its separate GELU pass,
 * `F.gelu(layer.ffn_in(h))` (reference transformer_opt/submission.py:507;
 * benchmarks/torch_transformer_benchmark.py:95-97; the fused Linear + GELU
 * candidate of benchmarks/experiments/c15_components.py:131-166), with the
 * GELU applied in the GEMM's epilogue.
 */
ttk_status ttk_linear_fwd(const void* x, const void* w, const void* bias, void* y, int dtype,
                          int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                          int64_t ldy, int activation, void* stream);

/* Bytes of the counter block that leads every ttk_linear_residual_ln_fwd
 * workspace: the same for every M (one counter per 64 rows of the largest M
 * the entry point takes). */
#define TTK_LINEAR_LN_WS_COUNTER_BYTES 65536

/*
 * Bytes of the workspace ttk_linear_residual_ln_fwd needs for M rows: the
 * counter block (TTK_LINEAR_LN_WS_COUNTER_BYTES) followed by 1 KB of row
 * statistics per 64-row block (0 for M <= 0).
 */
int64_t ttk_linear_residual_ln_workspace_size(int64_t M);

/*
 * W [N, K] (16-bit, row stride ldw elements) into the MFMA fragment order
 * ttk_linear_residual_ln_fwd reads (N * K elements, contiguous): 16-byte
 * chunk (fb * K/16 + q) * 64 + l holds W[32 fb + l % 32][16 q + 8 (l / 32) .. + 7].
 * One 1 KB block per (32 rows, 16 k) fragment, so each fragment is one
 * coalesced load.  Requirements (TTK_EUNSUPPORTED otherwise): dtype TTK_BF16
 * or TTK_F16, N a multiple of 32, K of 16, w and w_packed 16-byte aligned,
 * ldw a multiple of 8 and >= K; w_packed must not overlap w (TTK_EINVAL).
 * A weight that does not change is packed once.
 */
ttk_status ttk_linear_pack_weight(const void* w, void* w_packed, int dtype, int64_t N, int64_t K,
                                  int64_t ldw, void* stream);

/*
 * Output projection + residual add + LayerNorm in one kernel, bf16 / fp16,
 * rows of N = 1024:
 *
 *   attn_out = round( A W^T + bias )
 *   r        = round( x + attn_out )                (the residual output)
 *   y        = round( (r - mean) * rsqrt(var + eps) * gamma + beta )
 *
 * A [M, K] (row stride lda), W [N, K] packed by ttk_linear_pack_weight,
 * bias [N] or NULL, x, r, y [M, N] (row strides ldx, ldr, ldy), gamma [N],
 * beta [N] or NULL; mean and the biased variance are those of the rounded r
 * over its N features, in fp32.  These are the dtype boundaries of the
 * reference's `self._fused_residual_norm(x, out_proj(context), norm2)` in
 * 16-bit torch.  r equals the eager 16-bit `x + F.linear(A, W, bias)` bit for
 * bit whenever the projection does; y is deterministic (independent of
 * scheduling) and agrees with ttk_residual_layernorm_fwd on the same r to
 * the last rounding step.
 *
 * Two workgroups share each 64-row block (one per half of the features) and
 * exchange their half-row statistics through the workspace; the first to
 * finish polls for the other at most max_polls times (a negative value takes
 * the library default, 4096) and otherwise hands its half to the other,
 * which then normalises the whole block.  Both routes give the same bits.
 *
 * workspace: ttk_linear_residual_ln_workspace_size(M) bytes, 4-byte aligned,
 * its counter block zero before the call; every completed call leaves it
 * zero and the block sits at the same bytes for every M, so one zero-filled
 * buffer serves every later call of any shape on one stream.  Calls that
 * share a workspace must not run concurrently.
 *
 * Requirements (TTK_EUNSUPPORTED otherwise): dtype TTK_BF16 or TTK_F16;
 * N == 1024; K a positive multiple of 128; a, w_packed, x, gamma, beta, r
 * and y 16-byte aligned, bias 2-byte aligned; lda, ldx, ldr, ldy multiples
 * of 8 with lda >= K and ldx, ldr, ldy >= N; M * ld * 2 below 2^31 for x, r
 * and y.  r and y must not overlap each other, an input or the workspace
 * (TTK_EINVAL).  M == 0 is a no-op.
 *
 * Replaces the attention output projection and the first fused residual +
 * LayerNorm of an encoder block (reference transformer_opt/submission.py:
 * 497-505 with fused_residual_layer_norm, transformer_opt/kernels/
 * residual_layer_norm.py:159-237): the projection's output never goes
 * through HBM and the LayerNorm launch is gone.
 */
ttk_status ttk_linear_residual_ln_fwd(const void* a, const void* w_packed, const void* bias,
                                      const void* x, const void* gamma, const void* beta, void* r,
                                      void* y, void* workspace, int64_t workspace_bytes, int dtype,
                                      int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldx,
                                      int64_t ldr, int64_t ldy, float eps, int max_polls,
                                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TTK_HIP_H */
