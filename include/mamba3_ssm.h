/*
 * mamba3_ssm.h -- C ABI of the MI355X (gfx950) Mamba-3 SSD scan and decode step.
 *
 * This is the boundary a host in any language binds (the reference crate's
 * Rust host would bind it through a thin `extern "C"` -sys crate that
 * declares these functions and structs 1:1).  It replaces the reference's
 * generic Rust API over a CubeCL runtime (BectorVoom/mamba-trainer):
 *
 *   m3_ssm_config / m3_config_*   SsmConfig and its enums   src/ssm/config.rs:19-347
 *   m3_ssm_state                  SsmState                  src/ssm/scan.rs:293-358
 *   m3_scan_inputs / m3_scan      ScanInputs, mamba3_scan   src/ssm/scan.rs:360-618
 *   m3_scan_gated                 mamba3_scan then Mamba3Mixer::finish's gate
 *                                                           src/models/mamba3.rs:468-477
 *   m3_scan_output                ScanOutput                src/ssm/scan.rs:445-452
 *   m3_scan_grads / m3_scan_backward
 *                                 gradient of mamba3_scan   src/ssm/scan.rs:458-638 under
 *                                 autodiff (src/autodiff/), with the hand-written adjoints
 *                                 src/tensor/ops/fused.rs:2080-2138, 2326-2382, 2513-2549
 *   m3_ssd_args / m3_ssd_chunked  ssd_chunked               src/ssm/scan.rs:98-291
 *   m3_step_inputs / m3_step      mamba3_step               src/ssm/scan.rs:640-712
 *   m3_step_factored              the same on a cache with last_u factored (no
 *                                 reference counterpart; see its declaration)
 *   m3_step_layers                several layers' steps in one launch (no
 *                                 reference counterpart; see its declaration)
 *   m3_state_unfactor             the full last_u of a factored state
 *   m3_status / m3_last_error     Error / Result            src/error.rs:5-61
 *
 * Conventions
 *   - All tensors are caller-allocated, contiguous, row-major device buffers
 *     with the reference's layouts (rank-last x/b/c, N contiguous in the state).
 *   - `dtype` selects the storage of x, b, c, theta and y (f32, bf16 or f16,
 *     the 16-bit forms as raw words).  dt, lambda, a_log, d_skip and the state
 *     are f32.  f16 storage (FloatElem for half::f16, src/backend.rs:86-98)
 *     runs the f32 kernels on f32 copies: the call widens its f16 inputs into
 *     temporaries allocated in stream order (hipMallocAsync) on `stream`,
 *     narrows its f16 outputs back (round to nearest even) and frees the
 *     temporaries in stream order, so its results are exactly the f32 call's
 *     on the widened inputs, rounded to f16.  m3_scan_no_alloc,
 *     m3_scan_gated and m3_step_layers take f32 or bf16 only.
 *   - Calls are asynchronous on `stream` (a hipStream_t; NULL = the default
 *     stream) and never synchronise the host.  No call allocates device memory
 *     except those with f16 storage (above) and an m3_scan beyond the scan
 *     kernels' tiles without want_state (m3_scan).
 *   - Errors return a status; m3_last_error() gives this thread's message.
 *     Validation mirrors the reference's rules and messages.
 *   - Deviations from the reference, by design:
 *       * m3_step updates the state in place (the reference returns a new
 *         SsmState each step, scan.rs:704-711);
 *       * seq == 0 returns an empty y and passes the state through (the
 *         reference's mamba3_scan would underflow `seq - 1` there).
 */
#ifndef MAMBA3_SSM_H
#define MAMBA3_SSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3_ABI_VERSION 1

/* Error taxonomy of src/error.rs:9-49; M3_ERR_HIP / M3_ERR_ARGUMENT have no
 * reference counterpart (device failures and NULL/invalid pointers). */
typedef enum m3_status {
    M3_OK = 0,
    M3_ERR_CONFIG = 1,       /* Error::Config      */
    M3_ERR_SHAPE = 2,        /* Error::Shape       */
    M3_ERR_RANK = 3,         /* Error::Rank        */
    M3_ERR_UNSUPPORTED = 4,  /* Error::Unsupported */
    M3_ERR_HIP = 5,
    M3_ERR_ARGUMENT = 6,
    M3_ERR_STATE_DICT = 7,   /* Error::StateDict   */
    M3_ERR_IO = 8,           /* Error::Io          */
    M3_ERR_JSON = 9          /* Error::Json        */
} m3_status;

typedef enum m3_dtype { M3_F32 = 0, M3_BF16 = 1, M3_F16 = 2 } m3_dtype;

/* src/ssm/config.rs:19-26 */
typedef enum m3_discretization {
    M3_EULER = 0,
    M3_TRAPEZOID = 1,
    M3_LEARNED_TRAPEZOID = 2
} m3_discretization;

/* src/ssm/config.rs:46-55 */
typedef enum m3_dynamics { M3_REAL = 0, M3_ROTATIONAL = 1 } m3_dynamics;

/* SsmConfig, src/ssm/config.rs:84-128.  `rank` is SsmMode (1 = Siso,
 * R > 1 = Mimo{rank: R}; 0 is invalid); `conv_kernel` 0 means None. */
typedef struct m3_ssm_config {
    size_t d_model, n_heads, head_dim, d_state, n_groups;
    int32_t discretization;   /* m3_discretization */
    int32_t dynamics;         /* m3_dynamics */
    size_t rank;
    size_t chunk_size;
    size_t conv_kernel;
    int32_t bc_norm, bc_bias, post_gate_norm, skip_connection;
    float dt_min, dt_max, dt_init_floor, a_init_min, a_init_max;
    int32_t bias;
} m3_ssm_config;

/* Default::default() (config.rs:130-156). */
m3_status m3_config_default(m3_ssm_config *out);
/* SsmConfig::validate (config.rs:203-245). */
m3_status m3_config_validate(const m3_ssm_config *cfg);
/* Widths, config.rs:164-200. */
size_t m3_config_d_inner(const m3_ssm_config *cfg);
size_t m3_config_bc_width(const m3_ssm_config *cfg);
size_t m3_config_theta_width(const m3_ssm_config *cfg);
size_t m3_config_lambda_width(const m3_ssm_config *cfg);
size_t m3_config_in_proj_width(const m3_ssm_config *cfg);
/* Discretization::fixed_lambda (config.rs:29-36): 1, 0.5, or NaN if learned. */
float m3_discretization_fixed_lambda(int32_t discretization);

/* SsmState, src/ssm/scan.rs:294-302. */
typedef struct m3_ssm_state {
    float *h;       /* [B, H, P, N] */
    float *last_u;  /* [B, H, P, N] */
    float *angle;   /* [B, H, N/2], NULL for real dynamics */
} m3_ssm_state;

/* ScanInputs, src/ssm/scan.rs:361-385. */
typedef struct m3_scan_inputs {
    size_t batch, seq, heads, head_dim, d_state, rank;
    int32_t dtype;            /* m3_dtype of x, b, c, theta, y */
    const void *x;            /* [B, T, H, P, R] */
    const void *b;            /* [B, T, H, N, R] */
    const void *c;            /* [B, T, H, N, R] */
    const float *dt;          /* [B, T, H], positive */
    const float *a_log;       /* [H], A = -exp(a_log) */
    const float *lambda;      /* [B, T, H], in [0, 1] */
    const void *theta;        /* [B, T, H, N/2] or NULL (real dynamics) */
    const float *d_skip;      /* [H] or NULL */
    const m3_ssm_state *state;/* carried-in state or NULL */
    size_t chunk_size;        /* > 0; the three-launch chunk-parallel form passes
                               * the state between segments of at least this many
                               * tokens (tiles inside a segment are the kernel's
                               * own); the fused single launch always uses
                               * segments of 128 tokens */
    int32_t want_state;       /* ScanInputs::want_state */
    /* Device scratch for the chunk-parallel scan (no reference counterpart:
     * the reference allocates its intermediates per call): 256-byte aligned,
     * at least m3_scan_workspace_bytes() bytes.  NULL, a smaller or unaligned
     * buffer selects the single-pass kernel, which gives the same results to
     * rounding and needs no scratch.  The contents need no initialisation;
     * calls that share a workspace must be ordered on one stream.
     *
     * The chunk-parallel scan takes one of two forms.  The fused single
     * launch (bf16 storage, rank 1, d_state 64 or 128, while its grid of one
     * workgroup per 128-token segment fits three rounds of two workgroups per
     * CU) reads every input once: each segment publishes its contribution to
     * the state in the workspace and takes the state entering it from the
     * segments before it by a bounded wait on their flags.  A segment whose
     * wait gives up (about a second without an answer, which needs the GPU to
     * stop running the earlier segments' workgroups) takes NaN as its entering
     * state, so its outputs, those of the later segments of its sequence and
     * the sequence's boundary state are NaN, never stale.  Results do not
     * depend on the order in which workgroups run.  Other shapes take three
     * launches (segment states, a state pass, segment outputs). */
    void *workspace;
    size_t workspace_bytes;
} m3_scan_inputs;

/* ScanOutput, src/ssm/scan.rs:446-452.  `state` is written when want_state
 * (angle when theta is given).  Outputs must not alias inputs. */
typedef struct m3_scan_output {
    void *y;                  /* [B, T, H, P, R] */
    m3_ssm_state state;
} m3_scan_output;

/* mamba3_scan (scan.rs:458-618): trapezoid weights, rotating frame, MIMO
 * fold, carried state, skip path and boundary state in one launch.  Shapes
 * beyond the scan kernels' tiles (head_dim over 128, d_state over 256, rank
 * over a chunk's rows: 64 for bf16, 32 for f32, halved above d_state 128)
 * run as the recurrence, token by token, on the step kernel: one launch per
 * token, the carried state in the output state buffers (in temporaries
 * allocated and freed in stream order when want_state is 0).  Only shapes
 * beyond that kernel too (2 d_state rank + head_dim rank > 16384) return
 * M3_ERR_UNSUPPORTED, before any device work. */
m3_status m3_scan(const m3_scan_inputs *in, const m3_scan_output *out, void *stream);

/* m3_scan, then the mixer's gate on its y in place (Mamba3Mixer::finish
 * without a post-gate norm, src/models/mamba3.rs:468-477):
 * y = bf16(y) * silu(z), z bf16 [B*T rows of z_stride, the first
 * heads*head_dim*rank columns].  The same bytes as m3_scan followed by
 * m3_mixer_gate(..., norm_weight = NULL, out = y).  bf16 storage only
 * (else M3_ERR_UNSUPPORTED); z_stride < heads*head_dim*rank is M3_ERR_SHAPE.
 * Where the chunk-parallel form runs at rank 1 the gate rides on its output
 * kernel (no y round trip); elsewhere it is a second launch.
 * theta_stride: elements between consecutive tokens' theta rows, so theta
 * may be read in place from the in_proj output (theta_stride = its row
 * width); 0 is the contiguous [B, T, H, N/2] layout.  A stride under
 * heads*d_state/2 is M3_ERR_SHAPE; one other than 0 needs the specialised
 * kernels' shapes (head_dim 64, d_state 64 or 128, rank 1, 2 or 4, 16-byte
 * aligned buffers, rows of whole 16-byte pieces), else M3_ERR_UNSUPPORTED. */
m3_status m3_scan_gated(const m3_scan_inputs *in, const m3_scan_output *out, const void *z,
                        size_t z_stride, size_t theta_stride, void *stream);

/* Workspace bytes the chunk-parallel scan needs for these inputs (shapes and
 * dtype are read; pointers are not); 0 when the shape runs single-pass only.
 * No reference counterpart (see m3_scan_inputs.workspace). */
size_t m3_scan_workspace_bytes(const m3_scan_inputs *in);

/* Size of the static device scratch m3_scan_no_alloc uses, in MiB. */
#define M3_NO_ALLOC_SCRATCH_MIB 32

/* m3_scan without any allocation.  No reference counterpart: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  The chunk-parallel path's workspace
 * is a file-scope device array of M3_NO_ALLOC_SCRATCH_MIB MiB instead of the
 * caller's buffer (in->workspace and in->workspace_bytes are ignored).  Each GPU
 * holds its own copy of that array from the moment the library's code object is
 * loaded on that device (the first launch of any of its kernels there) until
 * the process ends, so every process that uses the library on a GPU holds those
 * M3_NO_ALLOC_SCRATCH_MIB MiB there whether or not it calls this function.
 * Where the fused launch's workspace (m3_scan_workspace_bytes) exceeds it and
 * the three launches' fits, the three launches run (results equal to rounding);
 * shapes whose workspace exceeds it on either form return M3_ERR_UNSUPPORTED
 * before any device work.  Otherwise results are those of m3_scan with a
 * caller workspace, bit for bit.  Every call on a GPU shares that GPU's
 * array, so calls on one GPU must not overlap.  An eager call on a stream
 * other than the previous eager call's, while that call may still run (its
 * completion event, recorded after it, is pending), returns M3_ERR_ARGUMENT
 * before any device work instead of racing; order such calls on one stream or
 * with an event.  Calls captured into a HIP graph, and the graph's replays,
 * are not tracked: overlapping them races and gives wrong results.  The
 * scratch needs no clearing: the chunk-parallel kernels write every byte they
 * later read within one call.  It calls no hipMalloc, hipFree or allocating
 * library routine (the guard's event is created once per device). */
m3_status m3_scan_no_alloc(const m3_scan_inputs *in, const m3_scan_output *out, void *stream);

/* Gradients of mamba3_scan for the loss L, given dL/dy.  The reference gets
 * them by reverse-mode autodiff through the composed scan (Var::backward over
 * scan.rs:458-638; its own adjoint kernels are ssd_band_backward fused.rs:
 * 2080-2138, exp_decay_backward 2326-2382 and trapezoid_weights_backward
 * 2513-2549).  Layouts as m3_scan_inputs; dx, db, dc and dtheta are in the
 * inputs' dtype, the rest f32.  Upstream gradients of the outgoing state (h,
 * last_u, angle) are optional; last_u's flows into x, b and the angle of the
 * last token (last_u = sum_r x_{L-1,r} B~_{L-1,r}^T, scan.rs:599-618), which is
 * how a window chained to the next one through SsmState is differentiated. */
typedef struct m3_scan_grads {
    const void *dy;           /* [B, T, H, P, R]: dL/dy (required) */
    const float *dh;          /* [B, H, P, N]: dL/d(output state h), or NULL */
    const float *dangle;      /* [B, H, N/2]: dL/d(output state angle), or NULL */
    void *dx;                 /* [B, T, H, P, R] (required) */
    void *db;                 /* [B, T, H, N, R] (required) */
    void *dc;                 /* [B, T, H, N, R] (required) */
    float *ddt;               /* [B, T, H] (required) */
    float *dlambda;           /* [B, T, H] (required) */
    float *da_log;            /* [H] (required), summed over the batch */
    void *dtheta;             /* [B, T, H, N/2], required when theta is given */
    float *dd_skip;           /* [H] or NULL (written when d_skip is given) */
    float *dh0;               /* [B, H, P, N] or NULL (carried-in state only) */
    float *dlast_u0;          /* [B, H, P, N] or NULL (carried-in state only) */
    float *dangle0;           /* [B, H, N/2] or NULL (carried-in angle only) */
    const float *dlast_u;     /* [B, H, P, N]: dL/d(output state last_u), or NULL */
} m3_scan_grads;

/* Backward of m3_scan on the same inputs (`in`, whose workspace must hold
 * m3_scan_backward_workspace_bytes(in) bytes, 256-byte aligned).  The forward
 * chunk states are recomputed; the forward outputs are not needed.  The
 * chunk kernels take head_dim 64, d_state 64/128, rank 1/2/4 with aligned
 * buffers; their partial sums inside a workgroup are accumulated with LDS
 * atomics, so repeated calls agree to f32 rounding, not bit for bit.  Other
 * shapes (and alignments) take the reverse mode of the recurrence token by
 * token, one workgroup per sequence with states recomputed from checkpoints
 * every 32 tokens (deterministic, and slow: a fallback), up to per-token
 * vectors of 64 KB (2 head_dim rank + 4 d_state rank + 3 d_state/2 floats;
 * beyond that M3_ERR_UNSUPPORTED, before any device work). */
m3_status m3_scan_backward(const m3_scan_inputs *in, const m3_scan_grads *grads, void *stream);

/* Workspace bytes m3_scan_backward needs for these inputs (0 when the shape
 * is not covered).  No reference counterpart. */
size_t m3_scan_backward_workspace_bytes(const m3_scan_inputs *in);

/* ssd_chunked arguments (scan.rs:100-126): one input/output channel. */
typedef struct m3_ssd_args {
    size_t batch, seq, heads, head_dim, d_state;
    int32_t dtype;            /* m3_dtype of x, b, c, y */
    const void *x;            /* [B, T, H, P] */
    const void *b;            /* [B, T, H, N] */
    const void *c;            /* [B, T, H, N] */
    const float *a;           /* [B, T, H], log decay dt*A (non-positive) */
    const float *g;           /* [B, T, H], diagonal weight */
    const float *w;           /* [B, T, H], off-diagonal weight */
    const float *initial_state; /* [B, H, P, N] or NULL */
    size_t chunk_size;
    int32_t want_state;
} m3_ssd_args;

/* ssd_chunked (scan.rs:116-291).  final_state [B,H,P,N] is written when
 * want_state (it may be NULL otherwise). */
m3_status m3_ssd_chunked(const m3_ssd_args *args, void *y, float *final_state, void *stream);

/* mamba3_step arguments (scan.rs:646-659): one token per sequence. */
typedef struct m3_step_inputs {
    size_t batch, heads, head_dim, d_state, rank;
    int32_t dtype;            /* m3_dtype of x, b, c, theta, y */
    const void *x;            /* [B, H, P, R] */
    const void *b;            /* [B, H, N, R] */
    const void *c;            /* [B, H, N, R] */
    const float *dt;          /* [B, H] */
    const float *lambda;      /* [B, H] */
    const float *a_log;       /* [H] */
    const void *theta;        /* [B, H, N/2] or NULL */
    const float *d_skip;      /* [H] or NULL */
} m3_step_inputs;

/* mamba3_step (scan.rs:649-712), in place: `state` (h, last_u and, with
 * theta, angle) is read and overwritten; y [B, H, P, R] is written. */
m3_status m3_step(const m3_step_inputs *in, m3_ssm_state *state, void *y, void *stream);

/* A second decode-cache format with last_u factored.  No reference
 * counterpart: the reference's SsmState.last_u is a full [B,H,P,N] tensor
 * (scan.rs:293-303).  It is, after any window or step, the last token's
 * rank-R outer product sum_r x_r B~_r^T with B~ = R(-angle) B
 * (scan.rs:599-618, 683-691), so carrying that token's x and unrotated B
 * with the angle holds the same information, and a step streams h alone:
 * 8 bytes per state element instead of 16. */
typedef struct m3_ssm_state_factored {
    float *h;        /* [B, H, P, N] f32 */
    void *x_prev;    /* [B, H, P, R] in the step inputs' dtype */
    void *b_prev;    /* [B, H, N, R] in the step inputs' dtype, unrotated */
    float *angle;    /* [B, H, N/2], NULL for real dynamics */
} m3_ssm_state_factored;

/* mamba3_step on the factored state, in place: h, x_prev, b_prev and angle
 * are read and overwritten (x_prev and b_prev take this step's x and b).
 * y and the new h equal m3_step's, bit for bit, on the full state whose
 * last_u = x_prev B~_prev^T as m3_step itself stored it.  A state from a
 * window of m3_scan starts with the window's last x and b (and the scan's h
 * and angle); a zero state has zero x_prev and b_prev.  Covers d_state a
 * multiple of 4 with d_state / 4 a power of two up to 64 and rank 1, 2, 3,
 * 4 or 8 (else M3_ERR_UNSUPPORTED); x_prev and b_prev must not overlap the
 * inputs. */
m3_status m3_step_factored(const m3_step_inputs *in, m3_ssm_state_factored *state, void *y,
                           void *stream);

/* The last_u [B, H, P, N] a factored state stands for:
 * last_u = sum_r x_prev_r (R(-angle) b_prev_r)^T, with the roundings
 * m3_step_factored uses (angle NULL: no rotation).  Callers that hand a
 * factored cache to m3_scan (a window after decoding) rebuild the full state
 * with it.  dtype is that of x_prev and b_prev. */
m3_status m3_state_unfactor(size_t batch, size_t heads, size_t head_dim, size_t d_state,
                            size_t rank, int32_t dtype, const void *x_prev, const void *b_prev,
                            const float *angle, float *last_u, void *stream);

/* n_layers steps in one launch (up to 24 layers a launch; more are split):
 * layer l is m3_step(&inputs[l], &states[l], ys[l]) or, with `factored`
 * instead of `states`, m3_step_factored(&inputs[l], &factored[l], ys[l]),
 * with the same results bit for bit.  No reference counterpart (the
 * reference steps each layer by itself): for callers that hold every
 * layer's inputs at once, such as a benchmark over a whole cache.  All
 * layers share batch, heads, head_dim, d_state, rank, dtype and whether
 * theta and d_skip are given (else M3_ERR_SHAPE); the shapes are the
 * factored step's (else M3_ERR_UNSUPPORTED).  Exactly one of states and
 * factored is non-NULL. */
m3_status m3_step_layers(size_t n_layers, const m3_step_inputs *inputs, m3_ssm_state *states,
                         m3_ssm_state_factored *factored, void *const *ys, void *stream);

/* Status name and this thread's last error message ("" after success). */
const char *m3_status_string(m3_status status);
const char *m3_last_error(void);

/* Kernel launches issued by this library since load (the reference's
 * launch counter, src/backend.rs:231-281). */
uint64_t m3_launch_count(void);

/* Test and benchmark settings of the chunk-parallel scan, process-wide.  No
 * reference counterpart.  path 0 (the default) runs the fused single launch
 * where it covers the shape (bf16 storage, rank 1) and the three launches
 * elsewhere; path 1 runs the three launches everywhere (m3_scan_workspace_bytes
 * follows the setting).  lookback_mode 1 makes every fused-launch segment after
 * a sequence's first give up its look-back at once, as a segment does after
 * lookback_spin unanswered polls (0: the default, about a second): its outputs,
 * those of the sequence's later segments and the sequence's boundary state
 * come out NaN.  Returns M3_ERR_ARGUMENT for values outside those ranges. */
m3_status m3_debug_scan_options(int32_t path, int32_t lookback_mode, int32_t lookback_spin);

/* Runs the MFMA lane-layout self test on the current device: *result is 0
 * when the layouts the kernels assume hold.  Synchronous; allocates 4 bytes. */
m3_status m3_selftest_mfma(int32_t *result);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_SSM_H */
