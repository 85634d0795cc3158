// Host-side launcher declarations shared by the C ABI (m3_api.cpp) and the
// kernel translation units.  Shapes have been validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace m3 {

// Decode step: one token per sequence, state updated in place.
struct StepLaunch {
    size_t batch, heads, head_dim, d_state, rank;
    int bf16;                       // storage of x, b, c, theta, y
    const void *x, *b, *c;          // [B,H,P,R], [B,H,N,R], [B,H,N,R]
    const float *dt, *lambda;       // [B,H]
    const float *a_log;             // [H]
    const void *theta;              // [B,H,N/2] or null
    const float *d_skip;            // [H] or null
    float *h, *last_u, *angle;      // [B,H,P,N] x2, [B,H,N/2] (null without theta)
    void *y;                        // [B,H,P,R]
    // Factored last_u (last_u null): the previous token's x [B,H,P,R] and
    // unrotated b [B,H,N,R] in the storage type, overwritten with this step's.
    void *x_prev, *b_prev;
    // 0: x, b, c, theta, dt, lambda and y in the [B,H,...] layout above.
    // Otherwise the token rows between consecutive batch entries of those
    // (entry (b, h) at row b * in_bstride * H + h, as one token of a
    // [B,T,H,...] window with in_bstride = T); such launches take the
    // generic body.
    size_t in_bstride;
};
hipError_t launch_step(const StepLaunch &a, hipStream_t stream);
// Shapes the factored form (last_u null) covers: the vector body's.
bool step_factored_supported(size_t d_state, size_t rank);
// Several layers' steps in one launch: per-layer buffers in a table passed by
// value (kernel arguments), the shapes shared.
struct StepLayer {
    const void *x, *b, *c;
    const float *dt, *lambda, *a_log;
    const void *theta;
    const float *d_skip;
    float *h, *last_u, *angle;
    void *y;
    void *x_prev, *b_prev;
};
// The mixer's decode step between its two projections in one launch
// (decode_step.hip): the 16-byte prologue's arithmetic on the projection row
// of each sequence, the SSM step on the state in place, and the gate without
// a post-gate norm.  `s` carries the shapes, a_log, d_skip and the state
// buffers; its x, b, c, dt, lambda, theta and y are not used.
struct MixerStepLaunch {
    StepLaunch s;
    size_t groups, width;
    int learned_lambda;
    float fixed_lambda, norm_eps;
    const void *projected;          // bf16 [B, width]
    const float *dt_bias;           // [H]
    const float *b_bias, *c_bias;   // [H, N] or null
    const float *bc_norm;           // [N] or null
    void *out;                      // bf16 [B, H*P*R]: silu(z) * y, or y when !gate
    int gate;                       // 0: y alone (a post-gate norm and the gate follow)
    // the causal convolution over [x | B | C] (conv_k 0: none), one position
    // per sequence: taps 0 .. k-2 from the history, k-1 from the row
    size_t conv_k;
    const float *conv_w, *conv_b;   // [k, C] and [C] (or null), C = d_inner + 2 G R N
    const void *hist;               // bf16 [B, k-1, C], or null (zeros)
    void *new_hist;                 // bf16 [B, k-1, C], or null; may be hist when G == H
};
// Shapes the fused step covers: the 16-byte prologue's (d_state a multiple
// of 8 with d_state / 8 a power of two, head_dim * rank and the row width
// multiples of 8) and the vector step body's (rank 1, 2, 4 or 8).
bool mixer_step_supported(size_t head_dim, size_t d_state, size_t rank, size_t width);
// Convolution taps the fused step holds in registers (the reference default is 4).
constexpr size_t kMixerStepConvTaps = 4;
hipError_t launch_mixer_step(const MixerStepLaunch &a, hipStream_t stream);
constexpr size_t kStepLayersPerLaunch = 24;
struct StepLayerTable {
    StepLayer layer[kStepLayersPerLaunch];
};
bool step_layers_supported(size_t d_state, size_t rank);
// last_u [B,H,P,N] = x_prev (R(-angle) b_prev)^T (angle null: no rotation).
hipError_t launch_unfactor(size_t batch, size_t heads, size_t P, size_t N, size_t R, bool bf16,
                           const void *x_prev, const void *b_prev, const float *angle,
                           float *last_u, hipStream_t s);
hipError_t launch_step_layers(const StepLaunch &a, const StepLayerTable &t, size_t n,
                              hipStream_t stream);

// Chunked scan.  `mode_raw` selects the mamba3_scan prologue (a, g, w built
// from dt, lambda, a_log) versus ssd_chunked's precomputed a, g, w.
struct ScanLaunch {
    size_t batch, seq, heads, head_dim, d_state, rank;
    int bf16;
    int mode_raw;
    const void *x, *b, *c;          // [B,T,H,P,R], [B,T,H,N,R] x2
    const float *dt, *lambda, *a_log;   // raw mode
    const float *a, *g, *w;             // ssd_chunked mode
    const void *theta;              // [B,T,H,N/2] or null (raw mode only)
    // elements between consecutive tokens' theta rows; 0 is H*N/2 (the
    // contiguous layout).  Taken by the specialised kernels only
    // (scan_fast_supported), e.g. theta read in place from the in_proj rows.
    size_t theta_stride;
    const float *d_skip;            // [H] or null
    const float *h0, *last_u0;      // incoming state or null (raw: both or neither)
    const float *angle0;            // [B,H,N/2] or null
    const float *init_state;        // ssd_chunked's initial_state or null
    void *y;                        // [B,T,H,P,R]
    // Optional gate on y (Mamba3Mixer::finish, models/mamba3.rs:468-477),
    // taken by the bf16 rank-1 chunk-parallel path only: y = bf16(y) *
    // silu(z), z bf16 at gate_z + token * gate_stride + h * head_dim + p.
    const void *gate_z;
    size_t gate_stride;
    float *h_out, *last_u_out, *angle_out;  // null when not wanted
    // the caller's chunk_size (tokens; 0 = 64): the chunk-parallel path passes
    // the state between segments of at least this many tokens
    size_t chunk_size;
    // chunk-parallel form: 0 the fused single launch where it covers the
    // shape (bf16, rank 1), 1 the three launches
    int path;
    // the fused launch's look-back: lb_mode 1 gives up at once (tests);
    // lb_spin polls of one flag before giving up (0: the default)
    int lb_mode, lb_spin;
};
hipError_t launch_scan(const ScanLaunch &a, hipStream_t stream);
// The specialised kernel (head_dim 64, d_state 64/128, rank 1/2/4, 16-byte
// aligned x/b/c/theta/y); hipErrorNotSupported for anything else.
bool scan_fast_supported(const ScanLaunch &a);
hipError_t launch_scan_fast(const ScanLaunch &a, hipStream_t stream);
// The chunk-parallel form of the same shapes (chunk states, an elementwise
// state pass, chunk outputs: three launches over a 256-byte aligned caller
// workspace): the workspace bytes it needs (0 when the shape is not covered),
// and the launch.
size_t scan_chunked_workspace(const ScanLaunch &a);
hipError_t launch_scan_chunked(const ScanLaunch &a, void *workspace, hipStream_t stream);
// Kernel launches the chunk-parallel form makes for these inputs: 1 for the
// fused single launch (bf16, rank 1, up to three rounds of its workgroups), 3
// otherwise.
int scan_chunked_launches(const ScanLaunch &a);
// Rows (token, rank) per chunk of the backward: 32, or 64 for bf16 storage
// with d_state 64 (whose 16-byte staging needs the longer chunk).
inline int scan_backward_rows(const ScanLaunch &a) { return (a.bf16 && a.d_state == 64) ? 64 : 32; }

// Backward of the scan (mamba3_scan mode, the chunk-parallel shapes): the
// gradients of the loss given dL/dy (and optionally dL/dh, dL/dangle of the
// outgoing state).  Outputs in the storage type where the input has it.
struct ScanGrads {
    const void *dy;                 // [B,T,H,P,R]
    const float *dh_out;            // [B,H,P,N] or null
    const float *dangle_out;        // [B,H,N/2] or null
    const float *dlast_u_out;       // [B,H,P,N] or null
    void *dx, *db, *dc;             // like x, b, c
    float *ddt, *dlambda;           // [B,T,H]
    float *da_log;                  // [H]
    void *dtheta;                   // like theta, or null
    float *dd_skip;                 // [H] or null
    float *dh0, *dlast_u0;          // [B,H,P,N] or null
    float *dangle0;                 // [B,H,N/2] or null
};
bool scan_backward_supported(const ScanLaunch &a);
size_t scan_backward_workspace(const ScanLaunch &a);
hipError_t launch_scan_backward(const ScanLaunch &a, const ScanGrads &g, void *workspace,
                                hipStream_t stream);
// The same gradients for any other shape whose per-token vectors fit 64 KB
// of LDS (2 P R + 4 N R + 3 N/2 floats): the reverse mode of the recurrence,
// token by token, one workgroup per sequence (ssd_scan_backward_generic.hip).
bool scan_backward_generic_supported(const ScanLaunch &a);
size_t scan_backward_generic_workspace(const ScanLaunch &a);
hipError_t launch_scan_backward_generic(const ScanLaunch &a, const ScanGrads &g, void *workspace,
                                        hipStream_t stream);

// Largest head_dim / d_state the scan kernels are instantiated for.
constexpr size_t kScanMaxHeadDim = 128;
constexpr size_t kScanMaxState = 256;
constexpr size_t kScanMaxRank = 64;

// MFMA lane-layout self test (writes 0 on success, else a failure code).
hipError_t launch_mfma_selftest(int *result_host);

// ---------------------------------------------------------------- mixer ops
// Row-wise RMSNorm over bf16 rows (y = x * rsqrt(mean(x^2) + eps) * w).
hipError_t launch_rms_norm(size_t rows, size_t dim, const void *x, size_t x_stride,
                           const float *w, float eps, void *y, size_t y_stride, hipStream_t s);
// Symmetric per-output-channel int8 codes (as exact bf16) and f32 scales of
// a [k, n] f32 weight.
hipError_t launch_quantize_columns(size_t k, size_t n, const float *w, void *codes, float *scales,
                                   hipStream_t s);
// Mamba3Mixer::project after the input projection.
struct PrologueLaunch {
    size_t tokens, heads, head_dim, d_state, rank, groups;
    size_t width;                   // row width of `projected`
    int learned_lambda;             // lambda piece present (else fixed_lambda)
    float fixed_lambda;
    int has_theta;
    float norm_eps;
    const void *projected;          // bf16 [tokens, width]
    const float *dt_bias;           // [H]
    const float *b_bias, *c_bias;   // [H, N] or null
    const float *bc_norm;           // [N] RMSNorm gain or null (no norm)
    void *x, *b, *c;                // bf16 [tokens, H, P, R], [tokens, H, N, R] x2
    float *dt, *lambda;             // [tokens, H]
    void *theta;                    // bf16 [tokens, H, N/2] (has_theta)
    // Causal convolution over [x | B | C] (conv_k 0: none).  Token t is
    // position t % seq_len of sequence t / seq_len.
    size_t conv_k, seq_len;
    const float *conv_w;            // [conv_k, channels]
    const float *conv_b;            // [channels] or null
    const void *hist;               // bf16 [batch, conv_k-1, channels] or null (zeros)
    void *new_hist;                 // bf16 [batch, conv_k-1, channels] or null
};
hipError_t launch_mixer_prologue(const PrologueLaunch &a, hipStream_t s);
// out = [RMSNorm(y)] * silu(z), rows of d_inner.
hipError_t launch_mixer_gate(size_t tokens, size_t d_inner, const void *y, const void *z,
                             size_t z_stride, const float *norm_w, float eps, void *out,
                             hipStream_t s);
// out[i] = table[ids[i]], bf16 rows of dim (zero rows for ids outside vocab).
hipError_t launch_embedding(size_t n, size_t dim, const int32_t *ids, size_t vocab, const void *table,
                            void *out, hipStream_t s);
// y = (x @ w) * col_scale + residual through hipBLASLt (bf16, f32 accumulate).
// The few-row product (skinny_gemm.hip): up to 512 rows, K a multiple of
// 128, N a multiple of 8 below 4096, 16-byte aligned buffers.
bool skinny_gemm_supported(size_t m, size_t k, size_t n, const void *x, const void *w,
                           const float *scale, const void *res, const void *y);
hipError_t launch_skinny_gemm(size_t m, size_t k, size_t n, const void *x, const void *w,
                              bool w_transposed, const float *scale, const void *res, void *y,
                              hipStream_t s);
hipError_t launch_linear(size_t m, size_t k, size_t n, const void *x, const void *w,
                         bool w_transposed, const float *col_scale, const void *residual, void *y,
                         void *workspace, size_t workspace_bytes, hipStream_t s);
constexpr size_t kLinearWorkspace = size_t(32) << 20;

}  // namespace m3
