/*
 * theorem_mi355x.h — C ABI of libtheorem_mi355x.so, the MI355X (gfx950) HIP
 * implementation of Theorem's four hot kernels.
 *
 * Every entry point:
 *   - takes raw device pointers, sizes and dtype codes (no framework types);
 *   - launches asynchronously on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronises, allocates or frees device memory;
 *   - validates its arguments on the host BEFORE any launch and returns a
 *     negative thm_status for an invalid call (nothing is launched), a positive
 *     hipError_t if the launch itself failed, and THM_OK (0) otherwise;
 *   - reads its inputs and writes only its outputs; each output element is
 *     written by exactly one lane, so results are bitwise deterministic.
 *
 * Tensor layouts are dense row-major ("contiguous" in PyTorch terms) exactly
 * as the reference's Python kernels lay them out:
 *   conv:     x, out [batch, dim, seqlen]; weight [dim, width]; bias [dim]
 *   DeltaNet: per-token tensors [B, T, H, D] (D = K or V); gates/beta [B, T, H];
 *             A [B, T, H, chunk_size]; per-chunk states [B, T/chunk_size, H, K, V].
 */
#ifndef THEOREM_MI355X_H
#define THEOREM_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define THM_ABI_VERSION 1

/* Status codes (negative = rejected on the host before any launch). */
#define THM_OK 0
#define THM_ERR_NULL_POINTER (-1) /* a required pointer is NULL                */
#define THM_ERR_BAD_SHAPE (-2)    /* negative/zero/overflowing size, T % BT     */
#define THM_ERR_BAD_DTYPE (-3)    /* unknown or unsupported dtype code          */
#define THM_ERR_UNSUPPORTED (-4)  /* valid but not implemented (K, V, width)    */
#define THM_ERR_MISALIGNED (-5)   /* pointer not aligned to its element size    */
#define THM_ERR_BAD_ARGUMENT (-6) /* flag/activation/chunk_size out of range    */

/* Element type codes. */
#define THM_DTYPE_F32 0
#define THM_DTYPE_BF16 1

/* Activation codes for thm_causal_conv1d_fwd. */
#define THM_ACT_NONE 0 /* the reference's behaviour (no activation)          */
#define THM_ACT_SILU 1 /* x * sigmoid(x); extension, not in the reference    */

/* Gate transforms for thm_chunk_local_cumsum. */
#define THM_GATE_IDENTITY 0   /* g = chunk-local cumsum of a              */
#define THM_GATE_LOGSIGMOID 1 /* g = chunk-local cumsum of log(sigmoid(a)) */

/* Flags for thm_chunk_fwd_h. */
#define THM_H_DELTA 1 /* delta-rule form: v_new = u - w.S, h[c] stored BEFORE the
                         update of chunk c, optional v_new / final-state output.
                         Without it: the reference's form (v used as is, h[c]
                         stored AFTER the update of chunk c). */

/* Library ABI version (THM_ABI_VERSION of the build). */
int thm_abi_version(void);

/* Human-readable text for a status code (static storage, never NULL). */
const char* thm_status_string(int status);

/*
 * Depthwise causal 1-D convolution.
 *   out[b,d,t] = act( bias[d] + sum_{k<width} weight[d,k] * x[b,d,t-width+1+k] ),
 *   x[b,d,t<0] = 0, fp32 accumulation.
 * Replaces the launcher `custom_kernel((x, weight, bias))` of
 * kernels/causal_conv1d/kernel.py:170-230 and its Triton kernel
 * `causal_conv1d_kernel` (kernel.py:44-117); math of reference.py:55-81.
 *   x_dtype: dtype of x and out (F32 or BF16); w_dtype: dtype of weight and bias.
 *   bias may be NULL (treated as zeros; the reference always passes one).
 *   1 <= width <= 8.
 */
int thm_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, void* out,
                          int64_t batch, int64_t dim, int64_t seqlen, int32_t width,
                          int32_t x_dtype, int32_t w_dtype, int32_t activation,
                          void* stream);

/*
 * Channels-last variant of thm_causal_conv1d_fwd: x, out [batch, seqlen, dim]
 * with dim contiguous (in PyTorch terms, a [batch, dim, seqlen] tensor that is
 * a transposed view of a contiguous [batch, seqlen, dim] one).  Same math,
 * arguments and status codes as thm_causal_conv1d_fwd.  No counterpart in the
 * reference, whose conv asserts the [batch, dim, seqlen] layout
 * (kernels/causal_conv1d/kernel.py:184); this is the layout a Mamba-2 block
 * holds its activations in.
 */
int thm_causal_conv1d_fwd_channels_last(const void* x, const void* weight, const void* bias,
                                        void* out, int64_t batch, int64_t seqlen, int64_t dim,
                                        int32_t width, int32_t x_dtype, int32_t w_dtype,
                                        int32_t activation, void* stream);

/*
 * Decode step of the causal conv with a rolling state, per (b, d):
 *   window = conv_state[b, d, 0..state_len) ++ x[b, d, 0..seqlen)
 *   out[b, d, t] = act( bias[d] + sum_{k<width} weight[d,k] * window[state_len - width + 1 + t + k] )
 *   conv_state[b, d, :] = the last state_len samples of window   (updated in place)
 * x, out [batch, dim, seqlen]; conv_state [batch, dim, state_len] in x_dtype,
 * state_len >= width - 1.  Running it token by token from a zero state gives
 * thm_causal_conv1d_fwd of the whole sequence.  No counterpart in the
 * reference (which has no decode path); it is the incremental form of the
 * reference's conv (kernels/causal_conv1d/reference.py:55-81).
 */
int thm_causal_conv1d_update(const void* x, void* conv_state, const void* weight, const void* bias,
                             void* out, int64_t batch, int64_t dim, int64_t seqlen,
                             int64_t state_len, int32_t width, int32_t x_dtype, int32_t w_dtype,
                             int32_t activation, void* stream);

/*
 * Gated DeltaNet WY recompute, per chunk c of chunk_size = 64 tokens:
 *   w_c = A_c . (k_c * (beta_c * exp(g_c)))      [64 x K]
 *   u_c = A_c . (v_c * beta_c)                   [64 x V]
 * with A_c[r, j] = A[b, c*64 + r, h, j] (the full 64x64 block is applied).
 * Replaces `custom_kernel(Data)` / `_launch` of
 * kernels/recompute_w_u/kernel.py:192-248 and `recompute_w_u_kernel`
 * (kernel.py:73-186); math of reference.py:118-149.
 *   kv_dtype: dtype of k, v, w, u (F32 or BF16). beta, A, g are fp32.
 *   g may be NULL (no gate: exp(g) = 1).
 *   K, V in {64, 128}; T % 64 == 0.
 */
int thm_recompute_w_u_fwd(const void* k, const void* v, const void* beta, const void* A,
                          const void* g, void* w, void* u,
                          int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                          int32_t chunk_size, int32_t kv_dtype, void* stream);

/*
 * Gated DeltaNet inter-chunk state recurrence over chunks c = 0..T/64-1 of one
 * (b, head), state S [K x V] fp32 (S = h0 or 0 at c = 0), g_last = g at the
 * chunk's last token:
 *   reference form (flags = 0; `vu` = v):
 *     S <- exp(g_last) S + k_c^T (v_c * exp(g_last - g_c));  h[c] = S
 *   delta form (flags = THM_H_DELTA; `vu` = u, `w` required):
 *     h[c] = S;  v_new_c = u_c - w_c . S;
 *     S <- exp(g_last) S + (k_c * exp(g_last - g_c))^T v_new_c
 *   ht (optional) receives the final S; v_new (optional, delta form only)
 *   receives v_new in kv_dtype.
 * Replaces `custom_kernel(dict)` of kernels/chunk_fwd_h/kernel.py:141-191 and
 * `chunk_fwd_h_kernel` (kernel.py:61-138); reference form = reference.py:50-97.
 *   kv_dtype: dtype of k, w, vu, v_new (F32 or BF16). g, h0, h, ht are fp32.
 *   g may be NULL (no gate). K, V in {64, 128}; T % 64 == 0.
 *   k, w, vu, h and v_new must be 16-byte aligned; g, h0 and ht 4-byte.
 */
int thm_chunk_fwd_h(const void* k, const void* w, const void* vu, const void* g,
                    const void* h0, void* h, void* v_new, void* ht,
                    int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                    int32_t chunk_size, int32_t kv_dtype, int32_t flags, void* stream);

/*
 * Gated DeltaNet chunkwise output, per chunk c and token i of the chunk:
 *   o[i] = scale * ( sum_{j<=i in chunk} (q_i . k_j) exp(g_i - g_j) v_j
 *                    + exp(g_i) q_i . h[c] )
 * (causal mask includes the diagonal). Replaces `custom_kernel(dict)` of
 * kernels/chunk_fwd_o/kernel.py:146-212 and `_chunk_fwd_o_kernel`
 * (kernel.py:52-136); math of reference.py:80-142 (there in the equivalent
 * factored form q*exp(g), v*exp(-g)).
 *   qkv_dtype: dtype of q, k, v and o (F32 or BF16). g and h are fp32.
 *   g may be NULL (no gate). K, V in {64, 128}; T % 64 == 0.
 *   Allocates nothing.  Large bf16 grids (at least twice as many tiles as
 *   2 workgroups per CU) hand their tiles out at run time from counter slots
 *   of a static device array (256 per device), which each launch resets.
 *   The host gives a slot only to a launch whose slot's previous launch has
 *   completed (an event per slot, recorded behind each launch), so launches
 *   in flight on any streams never share one; with every slot busy, a launch
 *   takes the fixed walk of its tiles.  A launch on a stream that is being
 *   captured into a graph always takes the fixed walk and touches no counter:
 *   the captured graph holds no state and may be replayed any number of
 *   times, on any streams.  Outputs are the same on either walk.
 */
int thm_chunk_fwd_o(const void* q, const void* k, const void* v, const void* g,
                    const void* h, void* o, float scale,
                    int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                    int32_t chunk_size, int32_t qkv_dtype, void* stream);

/*
 * Fused chunked Gated DeltaNet forward (delta form): per (b, head) and chunk c,
 *   v_new = u_c - w_c S;
 *   o_c = scale * ( exp(g_i) q_i . S + sum_{j<=i} (q_i . k_j) exp(g_i - g_j) v_new_j );
 *   S <- exp(g_last) S + (k_c * exp(g_last - g_c))^T v_new
 * i.e. thm_chunk_fwd_h (flags = THM_H_DELTA) followed by thm_chunk_fwd_o with
 * h[c] = the state before chunk c, without writing the per-chunk states.
 * Replaces the composition of kernels/chunk_fwd_h/kernel.py:141-191 and
 * kernels/chunk_fwd_o/kernel.py:146-212 in the chunked forward; no single
 * reference function does this.
 *   bf16 only (qkv_dtype = THM_DTYPE_BF16): q, k, w, u, o, v_new bf16;
 *   g, h0, ht fp32.  g, h0, v_new, ht may be NULL.  K, V in {64, 128};
 *   T % 64 == 0.
 */
int thm_chunk_gated_delta_fwd(const void* q, const void* k, const void* w, const void* u,
                              const void* g, const void* h0, void* o, void* v_new, void* ht,
                              float scale, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                              int32_t chunk_size, int32_t qkv_dtype, void* stream);

/*
 * The same recurrence and output from the WY matrix instead of w and u: per
 * chunk c,
 *   v_new = A_c (beta_c * (v_c - exp(g_c) * (k_c S)))
 * which equals u_c - w_c S for w_c = A_c (k_c beta_c exp(g_c)), u_c =
 * A_c (v_c beta_c) (recompute_w_u, kernels/recompute_w_u/reference.py:118-149),
 * so w and u are never formed; o, v_new and ht as thm_chunk_gated_delta_fwd.
 * A is thm_wy_build_A's output (sign = +1 for the gated delta rule).
 * Replaces recompute_w_u, chunk_fwd_h (delta form) and chunk_fwd_o in the
 * chunked forward (kernels/recompute_w_u/kernel.py:192-248,
 * kernels/chunk_fwd_h/kernel.py:141-191, kernels/chunk_fwd_o/kernel.py:146-212);
 * no single reference function does this.
 *   bf16 only: q, k, v, o, v_new bf16; beta [B, T, H], A [B, T, H, 64], g, h0,
 *   ht fp32.  g, h0, v_new, ht may be NULL.  K, V in {64, 128}; T % 64 == 0.
 *   q, k, v and A 16-byte aligned, o and v_new 8-byte, beta, g, h0, ht 4-byte.
 */
int thm_chunk_gated_delta_fwd_a(const void* q, const void* k, const void* v, const void* beta,
                                const void* A, const void* g, const void* h0, void* o, void* v_new,
                                void* ht, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                                int64_t V, int32_t chunk_size, int32_t qkv_dtype, void* stream);

/*
 * WY matrix of the chunked Gated DeltaNet forward, per chunk c of
 * chunk_size = 64 tokens:
 *   M[i][j] = beta_i (k_i . k_j) exp(g_i - g_j) for j < i (0 on and above the diagonal),
 *   A_c = (I + sign M)^{-1}
 * with A_c[r, :] stored at A[b, c*64 + r, h, :] (the layout recompute_w_u reads).
 * sign = -1 is the reference's (I - M)^{-1}: replaces `_build_A` of
 * kernels/recompute_w_u/reference.py:48-91 (torch matmul + solve_triangular);
 * sign = +1 is the gated delta rule's (I + M)^{-1}.
 *   k_dtype: dtype of k (F32 or BF16). beta, g and A are fp32.
 *   g may be NULL (no gate). K in {64, 128}; T % 64 == 0.
 */
int thm_wy_build_A(const void* k, const void* beta, const void* g, void* A,
                   int64_t B, int64_t T, int64_t H, int64_t K,
                   int32_t chunk_size, int32_t k_dtype, int32_t sign, void* stream);

/*
 * Fused WY forward: the WY matrix A_c of thm_wy_build_A (same sign convention)
 * and the recompute_w_u products with it, in one pass, per chunk c:
 *   w_c = A_c (k_c * beta_c exp(g_c)),   u_c = A_c (v_c * beta_c)
 * A is never written.  Replaces `_build_A` followed by the recompute_w_u
 * kernel (kernels/recompute_w_u/reference.py:48-91 and :118-149) for callers
 * that need only w and u; w and u equal thm_wy_build_A + thm_recompute_w_u_fwd.
 *   bf16 only (kv_dtype = THM_DTYPE_BF16): k, v, w, u bf16; beta, g fp32.
 *   g may be NULL (no gate). K, V in {64, 128}; T % 64 == 0.
 */
int thm_wy_fwd(const void* k, const void* v, const void* beta, const void* g, void* w, void* u,
               int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
               int32_t chunk_size, int32_t kv_dtype, int32_t sign, void* stream);

/*
 * Gate preprocessing: per 64-token chunk, the inclusive cumulative sum of the
 * per-token log decay,
 *   g[b, t, h] = sum_{t' in chunk(t), t' <= t} f(a[b, t', h]),
 * f = identity (THM_GATE_IDENTITY) or log(sigmoid(.)) (THM_GATE_LOGSIGMOID).
 * This is the chunk-local cumulative gate g that every chunk kernel above
 * takes; the reference forms it inside its input generators
 * (kernels/chunk_fwd_h/reference.py:15-47, kernels/recompute_w_u/reference.py:94-115,
 * `reshape(B, T/BT, BT, H).cumsum(dim=2)`).
 *   a_dtype: dtype of a (F32 or BF16); g is fp32 [B, T, H]. T % 64 == 0.
 */
int thm_chunk_local_cumsum(const void* a, void* g, int64_t B, int64_t T, int64_t H,
                           int32_t chunk_size, int32_t a_dtype, int32_t mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* THEOREM_MI355X_H */
