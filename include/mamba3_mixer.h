/*
 * mamba3_mixer.h -- C ABI of the token-parallel operations of the Mamba-3
 * mixer and language model around the scan (gfx950, bf16 activations).
 *
 * With m3_scan / m3_step (mamba3_ssm.h) these compose Mamba3Mixer::apply,
 * ::apply_with_state and ::step and the Mamba3Lm forward:
 *
 *   m3_rms_norm                 RmsNorm::apply            src/nn/norm.rs:95-105
 *                               (fused rms_norm_kernel    src/tensor/ops/fused.rs:140-185)
 *   m3_quantize_int8_columns    Quantizer::quantize, QuantConfig::int8_weights
 *                                                         src/nn/quant.rs:95-103, 231-245, 282-330
 *   m3_linear, m3_linear_nt     Linear::apply (+ the stack's residual add)
 *                                                         src/nn/linear.rs:155-185,
 *                                                         src/models/hybrid.rs:446-456
 *   m3_mixer_prologue           Mamba3Mixer::project after in_proj
 *                                                         src/models/mamba3.rs:376-466
 *   m3_mixer_prologue_conv      the same with the causal convolution and its history
 *                                                         src/models/mamba3.rs:386-400,
 *                                                         src/nn/conv.rs:143-225,
 *                                                         src/tensor/ops/fused.rs:780-865
 *   m3_mixer_gate               Mamba3Mixer::finish before out_proj
 *                                                         src/models/mamba3.rs:468-477
 *   m3_embedding_lookup         Embedding::lookup         src/nn/embedding.rs
 *   m3_mixer_step               Mamba3Mixer::step between in_proj and out_proj in
 *                               one launch (prologue, mamba3_step, gate)
 *                                                         src/models/mamba3.rs:569-630
 *   m3_mixer_step_conv          the same with the convolution's history step
 *                               (one launch) and the post-gate norm (+1)
 *                                                         src/models/mamba3.rs:569-630,
 *                                                         src/tensor/ops/fused.rs:833-865
 *
 * Conventions are those of mamba3_ssm.h: caller-allocated contiguous device
 * buffers, asynchronous on `stream`, status codes with m3_last_error().
 * Activations are bf16 (raw 16-bit words); weights of norms and biases, and
 * dt / lambda, are f32.
 */
#ifndef MAMBA3_MIXER_H
#define MAMBA3_MIXER_H

#include <stddef.h>
#include <stdint.h>

#include "mamba3_ssm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * weight, rows of `dim` bf16
 * elements at strides x_stride / y_stride (elements); weight [dim] f32 or
 * NULL (no gain). */
m3_status m3_rms_norm(size_t rows, size_t dim, const void *x, size_t x_stride, const float *weight,
                      float eps, void *y, size_t y_stride, void *stream);

/* Symmetric per-output-channel int8 fake quantization of a Linear weight
 * w [in_features, out_features] (f32, row-major as the reference stores it):
 * scale_j = max(max_i |w_ij|, 1e-12) / 127, code_ij = clamp(round(w_ij /
 * scale_j), -127, 127).  codes [in, out] are written as bf16 (whole numbers,
 * exact), scales [out] as f32; w' = code * scale is the fake-quantized
 * weight. */
m3_status m3_quantize_int8_columns(size_t in_features, size_t out_features, const float *w,
                                   void *codes, float *scales, void *stream);

/* y[m, n] = (x[m, k] @ w[k, n]) * col_scale[n] + residual[m, n], bf16 with f32
 * accumulation (hipBLASLt).  col_scale and residual may be NULL; residual may
 * alias y.  The workspace (up to m3_linear_workspace_bytes(), 256-byte
 * aligned, or NULL) widens the kernels hipBLASLt may pick.  The first call
 * for a (m, k, n, scaled, workspace) shape times hipBLASLt's candidate
 * algorithms on the caller's inputs into a scratch output, each run after a
 * 512 MB cache-evicting write (both buffers allocated and freed by the call),
 * and blocks on `stream` while it reads the timings; later calls are
 * asynchronous.  The
 * reference tunes its matmul plans once per shape the same way
 * (src/tensor/matmul.rs:1636-1943).  M3_LINEAR_TUNE=0 in the environment
 * keeps hipBLASLt's first choice instead, as does a first call made while
 * `stream` is being captured into a graph. */
size_t m3_linear_workspace_bytes(void);
m3_status m3_linear(size_t m, size_t k, size_t n, const void *x, const void *w,
                    const float *col_scale, const void *residual, void *y, void *workspace,
                    size_t workspace_bytes, void *stream);

/* m3_linear with the weight given transposed, w_t [n, k] (row-major): the
 * same product, y[m, n] = (x[m, k] @ w_t[n, k]^T) * col_scale[n] +
 * residual[m, n].  hipBLASLt's kernels for this layout are the faster ones
 * at large m; a caller that holds the weight only for the product (the
 * int8 codes) keeps it this way.  Up to 512 rows and 4096 columns (k a
 * multiple of 128, n of 8, 16-byte aligned buffers) both forms run on the
 * library's own few-row kernel instead of hipBLASLt. */
m3_status m3_linear_nt(size_t m, size_t k, size_t n, const void *x, const void *w_t,
                       const float *col_scale, const void *residual, void *y, void *workspace,
                       size_t workspace_bytes, void *stream);

/* Shapes of one mixer (SsmConfig fields, config.rs:84-128). */
typedef struct m3_mixer_dims {
    size_t tokens;            /* batch * seq */
    size_t heads, head_dim, d_state, rank, groups;
    int32_t discretization;   /* m3_discretization: learned -> lambda piece present */
    int32_t dynamics;         /* m3_dynamics: rotational -> theta piece present */
    float norm_eps;           /* RmsNorm eps of bc_norm (1e-5) */
} m3_mixer_dims;

/* Width of the in_proj output row (SsmConfig::in_proj_width). */
size_t m3_mixer_in_proj_width(const m3_mixer_dims *d);

/* From the in_proj output `projected` [tokens, in_proj_width] (bf16) to the
 * scan inputs: x [tokens, H, P, R], b and c [tokens, H, N, R] (bf16), dt and
 * lambda [tokens, H] (f32), theta [tokens, H, N/2] (bf16, rotational only).
 * theta is a copy of the row's last H*N/2 columns: NULL skips the copy, for
 * a caller that reads theta in place (m3_scan_gated's theta_stride).
 * b_bias / c_bias [H, N] and bc_norm [N] (RMSNorm gain) are f32 or NULL when
 * the config has no bias / no norm.  No convolution (conv_kernel None). */
m3_status m3_mixer_prologue(const m3_mixer_dims *d, const void *projected, const float *dt_bias,
                            const float *b_bias, const float *c_bias, const float *bc_norm,
                            void *x, void *b, void *c, float *dt, float *lambda, void *theta,
                            void *stream);

/* The depthwise causal convolution of a mixer with conv_kernel = k
 * (CausalConv1d, src/nn/conv.rs:60-225) over the channels [x | B | C] of the
 * projection, channels = d_inner + 2 * G * N * R.  With the window
 * w = history ++ input along the sequence (history: the k-1 positions before
 * it), out[s, ch] = bias[ch] + sum_j weight[j, ch] * w[s + j, ch]
 * (src/tensor/ops/fused.rs:780-832): tap j multiplies the input delayed by
 * k-1-j positions.  The new history is the window's last k-1 positions
 * (fused.rs:833-865). */
typedef struct m3_conv1d {
    size_t kernel_size;        /* k >= 2 */
    size_t seq_len;            /* positions per sequence: tokens = batch * seq_len */
    const float *weight;       /* [k, channels] f32 */
    const float *bias;         /* [channels] f32, or NULL (no bias) */
    const void *history;       /* bf16 [batch, k-1, channels], or NULL (zeros) */
    void *new_history;         /* bf16 [batch, k-1, channels], or NULL (not written) */
} m3_conv1d;

/* Mamba3Mixer::project with the convolution (src/models/mamba3.rs:386-400):
 * m3_mixer_prologue with x, B and C taken from the convolution's output
 * before the silu.  conv NULL is m3_mixer_prologue.  new_history may equal
 * history when seq_len is 1 (the decode step updates its cache in place);
 * otherwise the two must not overlap (the history is read by other
 * positions' workgroups while the new one is written). */
m3_status m3_mixer_prologue_conv(const m3_mixer_dims *d, const m3_conv1d *conv,
                                 const void *projected, const float *dt_bias,
                                 const float *b_bias, const float *c_bias, const float *bc_norm,
                                 void *x, void *b, void *c, float *dt, float *lambda, void *theta,
                                 void *stream);

/* out[t] = [RMSNorm(y[t]) * norm_weight] * silu(z[t]) over rows of d_inner;
 * z rows are z_stride elements apart (the z piece of the projection);
 * norm_weight NULL skips the post-gate norm. */
m3_status m3_mixer_gate(size_t tokens, size_t d_inner, const void *y, const void *z,
                        size_t z_stride, const float *norm_weight, float eps, void *out,
                        void *stream);

/* Mamba3Mixer::step between its two projections (src/models/mamba3.rs:569-630,
 * after in_proj and before out_proj) in one launch, for one token per
 * sequence (d->tokens is the batch): m3_mixer_prologue on `projected`
 * [batch, in_proj_width], then m3_step on `state` (or m3_step_factored on
 * `factored`; exactly one is non-NULL) in place with a_log [H] and d_skip [H]
 * (or NULL), then m3_mixer_gate without a post-gate norm into out
 * [batch, d_inner] (bf16).  The results equal those three calls bit for bit;
 * the scan inputs and y never go through memory.  No reference counterpart
 * as one call (the reference issues the three pieces).  No convolution and
 * no post-gate norm: m3_mixer_step_conv takes those.  Shapes: d_state a multiple
 * of 8 up to 128 with d_state / 8 a power of two, head_dim * rank a multiple
 * of 8 up to 512, rank 1, 2, 4 or 8 (else M3_ERR_UNSUPPORTED). */
m3_status m3_mixer_step(const m3_mixer_dims *d, const void *projected, const float *dt_bias,
                        const float *b_bias, const float *c_bias, const float *bc_norm,
                        const float *a_log, const float *d_skip, m3_ssm_state *state,
                        m3_ssm_state_factored *factored, void *out, void *stream);

/* m3_mixer_step for a mixer with the causal convolution and/or the post-gate
 * norm, such as the reference's default mixer (conv_kernel Some(4),
 * src/ssm/config.rs:143) stepped by Mamba3Mixer::step
 * (src/models/mamba3.rs:569-630) with its history update
 * (src/tensor/ops/fused.rs:833-865).  conv (or NULL) has seq_len 1 and at
 * most 4 taps (more: M3_ERR_UNSUPPORTED, compose the calls): x, B and
 * C come from the convolution over history ++ this token, as
 * m3_mixer_prologue_conv computes them, and new_history receives the last
 * k-1 positions.  new_history may be history itself (the cache updated in
 * place) when groups == heads, where every channel belongs to one
 * (sequence, head); with groups < heads an in-place history is
 * M3_ERR_UNSUPPORTED (pass a separate buffer, or compose the calls).  The
 * weight, bias and histories are 16-byte aligned.  post_norm_weight
 * [d_inner] (or NULL) is the post-gate RMSNorm gain (eps post_norm_eps): the
 * norm spans every head of a row, so the step writes y to out and
 * m3_mixer_gate with the norm follows on out in place (two launches; one
 * without the norm).  The results equal m3_mixer_prologue_conv, m3_step (or
 * m3_step_factored) and m3_mixer_gate bit for bit.  Shapes as m3_mixer_step. */
m3_status m3_mixer_step_conv(const m3_mixer_dims *d, const m3_conv1d *conv, const void *projected,
                             const float *dt_bias, const float *b_bias, const float *c_bias,
                             const float *bc_norm, const float *a_log, const float *d_skip,
                             const float *post_norm_weight, float post_norm_eps,
                             m3_ssm_state *state, m3_ssm_state_factored *factored, void *out,
                             void *stream);

/* out[i] = table[ids[i]] for bf16 rows of dim (table [vocab, dim]).  The
 * ids live on the device, so they are not checked on the host: an id outside
 * [0, vocab) reads nothing and yields a zero row. */
m3_status m3_embedding_lookup(size_t n, size_t dim, const int32_t *ids, size_t vocab,
                              const void *table, void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_MIXER_H */
