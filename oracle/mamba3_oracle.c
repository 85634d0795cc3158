/*
 * mamba3_oracle.c -- CPU restatement of the Mamba-3 SSD scan and decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP path
 * and the CPU baseline that bench.py reports beside it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links, calls or falls back to it.
 *
 * Three families of functions live here; every one cites the reference code
 * it restates (paths are relative to the reference crate BectorVoom/mamba-trainer):
 *
 *   1. m3o_noise / m3o_test_reference_f32
 *        the reference test-suite's own input generator and its own direct
 *        recurrence oracle (tests/ssm.rs:26-34, 58-106), restated verbatim in
 *        f32 with the same loop order.
 *   2. m3o_scan_recurrence_f64 (and its reverse mode, m3o_scan_backward_f64)
 *        the exponential-trapezoidal recurrence (src/ssm/scan.rs:5-45) evaluated
 *        token by token in double precision, extended with everything the scan
 *        API carries: MIMO rank (scan.rs:538-589), the rotating frame
 *        (scan.rs:482-519), an incoming SsmState (scan.rs:521-535), the skip
 *        path (scan.rs:593-597) and the outgoing state (scan.rs:599-638).
 *   3. the composed f32 algorithm, stage for stage:
 *        m3o_ssd_chunked_f32   src/ssm/scan.rs:116-291
 *        m3o_scan_composed_f32 src/ssm/scan.rs:458-638
 *        m3o_step_f32          src/ssm/scan.rs:649-712
 *      and the fused forward kernels those stages call (src/tensor/ops/fused.rs,
 *      src/tensor/ops/scan.rs, src/tensor/ops/elemwise.rs:349).
 *
 * Pinning (what checks each function; the tests live in tests/test_oracle_*.py):
 *   - m3o_noise: bit-exact LCG; known first values are asserted.
 *   - cumsum family: the literal known answers of tests/tensor.rs:183-200.
 *   - trapezoid / band / exp_decay / coefficients / angle / rotation: the
 *     reference's own known-answer inputs from tests/autograd.rs:518-823 and
 *     tests/tensor.rs:510-537, plus closed forms (Euler collapse w == g,
 *     quarter-turn rotation of a unit vector).
 *   - m3o_test_reference_f32: it is the reference's own oracle; it is checked
 *     against m3o_scan_recurrence_f64 and a scalar (P = N = 1) hand evaluation.
 *   - m3o_scan_recurrence_f64: against m3o_test_reference_f32 on the reference
 *     cases, against the composed algorithm on every case of tests/ssm.rs,
 *     against closed forms (one token, pure rotation e^{i*theta*t}, pure decay),
 *     and against the invariants split-window == single pass, stepwise ==
 *     parallel, MIMO == sum of SISO systems, Euler == Mamba-2.
 *   - m3o_scan_backward_f64: against central finite differences of
 *     m3o_scan_recurrence_f64 on every input (x, b, c, dt, lambda, a_log,
 *     theta, d_skip, h0, last_u0, angle0) through random directional
 *     derivatives, with and without upstream state gradients; and against the
 *     reference's scan_is_differentiable case (tests/ssm.rs:382-426).
 *   - m3o_ssd_chunked_f32 / m3o_scan_composed_f32 / m3o_step_f32: against the
 *     f64 recurrence at the reference's own tolerances (2e-4 / 3e-4).
 *   - fault injection (m3o_set_fault) plants a mistake in this file on the
 *     CPU and the tests assert that the checks above catch every planted one.
 *
 * Layouts (row-major, contiguous; rank is the last axis, as in ScanInputs):
 *   x [B,T,H,P,R]   b, c [B,T,H,N,R]   dt, lambda [B,T,H]   a_log, d_skip [H]
 *   theta [B,T,H,N/2]   h, last_u [B,H,P,N]   angle [B,H,N/2]   y [B,T,H,P,R]
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define M3O_LOG_DECAY_FLOOR (-60.0f) /* src/ssm/scan.rs:57 */

/* ---------------------------------------------------------------------------
 * Fault injection (test infrastructure): a planted mistake per code.
 * ------------------------------------------------------------------------- */
enum {
    M3O_FAULT_NONE = 0,
    M3O_FAULT_DROP_BETA = 1,        /* trapezoid one-step-behind term removed */
    M3O_FAULT_ROT_SIGN = 2,         /* frame rotated by +phi instead of -phi */
    M3O_FAULT_TRANSPOSE_U = 3,      /* u[p][n] built as x[n] * b[p] (P == N) */
    M3O_FAULT_LAMBDA_INDEX = 4,     /* f_j reads lambda_j instead of lambda_{j+1} */
    M3O_FAULT_DECAY_SIGN = 5,       /* alpha = exp(-dt*A) */
    M3O_FAULT_MIMO_DIAG = 6,        /* MIMO cross terms i != j dropped */
    M3O_FAULT_SKIP_SIGN = 7,        /* y -= D*x */
    M3O_FAULT_CARRY_BETA = 8,       /* incoming last_u ignored */
    M3O_FAULT_CHUNK_STATE_W = 9,    /* chunk summary weighted by g instead of w */
    M3O_FAULT_BWD_ROT_SIGN = 10,    /* backward: dB, dC rotated by -phi instead of +phi */
};
static int g_fault = 0;
void m3o_set_fault(int code) { g_fault = code; }
int m3o_get_fault(void) { return g_fault; }

int m3o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------------------
 * 1. The reference test suite's generator and direct oracle.
 * ------------------------------------------------------------------------- */

/* tests/ssm.rs:26-34: deterministic values in [-1, 1). */
void m3o_noise(size_t n, uint64_t seed, float *out) {
    uint64_t s = seed * 6364136223846793005ULL + 1ULL;
    for (size_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        out[i] = ((float)(s >> 33) / (float)(1ULL << 31)) - 1.0f;
    }
}

/* tests/ssm.rs:58-106, verbatim in f32: SISO, no rotation, zero initial state.
 * x [B,T,H,P], b, c [B,T,H,N], dt, lambda [B,T,H], a_head [H] (= A, negative).
 * Writes y [B,T,H,P] and the final h [B,H,P,N]. */
void m3o_test_reference_f32(size_t batch, size_t seq, size_t heads, size_t head_dim,
                            size_t state, const float *x, const float *b, const float *c,
                            const float *dt, const float *lambda, const float *a_head,
                            float *y, float *h) {
    size_t hs = batch * heads * head_dim * state;
    float *prev_u = (float *)calloc(hs ? hs : 1, sizeof(float));
    memset(h, 0, hs * sizeof(float));
    for (size_t tt = 0; tt < seq; ++tt)
        for (size_t bb = 0; bb < batch; ++bb)
            for (size_t hh = 0; hh < heads; ++hh) {
                size_t idx = (bb * seq + tt) * heads + hh;
                float step = dt[idx];
                float lam = lambda[idx];
                float alpha = expf(step * a_head[hh]);
                float beta = (1.0f - lam) * step * alpha;
                float gamma = lam * step;
                size_t x_off = idx * head_dim;
                size_t bc_off = idx * state;
                size_t h_off = (bb * heads + hh) * head_dim * state;
                for (size_t p = 0; p < head_dim; ++p) {
                    float xv = x[x_off + p];
                    float acc = 0.0f;
                    for (size_t n = 0; n < state; ++n) {
                        float u = xv * b[bc_off + n];
                        size_t slot = h_off + p * state + n;
                        float nw = alpha * h[slot] + beta * prev_u[slot] + gamma * u;
                        h[slot] = nw;
                        prev_u[slot] = u;
                        acc += c[bc_off + n] * nw;
                    }
                    y[x_off + p] = acc;
                }
            }
    free(prev_u);
}

/* ---------------------------------------------------------------------------
 * 2. The f64 recurrence.
 * ------------------------------------------------------------------------- */

static double wrap_pi_f64(double v) {
    const double two_pi = 6.283185307179586476925286766559;
    return v - nearbyint(v / two_pi) * two_pi;
}

/* Rotate the half-split pair (v1, v2) by -phi (src/tensor/ops/fused.rs:610-617
 * with from_angle: c = cos(phi), s = -sin(phi)). */
static void rot_neg_f64(double phi, double v1, double v2, double *o1, double *o2) {
    double cs = cos(phi), sn = sin(phi);
    if (g_fault == M3O_FAULT_ROT_SIGN) sn = -sn;
    *o1 = v1 * cs + v2 * sn;
    *o2 = -v1 * sn + v2 * cs;
}

/*
 * h_t = alpha_t h_{t-1} + beta_t u_{t-1} + gamma_t u_t,  y_t = C~_t^T h_t (+ D x_t)
 *   alpha = exp(dt A), beta = (1 - lambda) dt alpha, gamma = lambda dt
 *   u_t[p][n] = sum_r x_t[p][r] B~_t[n][r]      (src/ssm/scan.rs:5-25, 683-690)
 *   B~_t, C~_t = B_t, C_t rotated by -phi_t, phi_t = angle0 + sum_{s<=t} dt_s theta_s
 * h0 / last_u0 may be NULL (zero state); angle0 may be NULL (zero angle).
 * Outputs: y [B,T,H,P,R]; h_out, last_u_out [B,H,P,N]; angle_out [B,H,N/2]
 * (wrapped to [-pi, pi]) when theta is given.  Any output may be NULL.
 */
void m3o_scan_recurrence_f64(size_t B, size_t T, size_t H, size_t P, size_t N, size_t R,
                             const float *x, const float *b, const float *c,
                             const float *dt, const float *a_log, const float *lambda,
                             const float *theta, const float *d_skip, const float *h0,
                             const float *last_u0, const float *angle0, double *y,
                             double *h_out, double *last_u_out, double *angle_out) {
    size_t half = N / 2;
    #pragma omp parallel for collapse(2) schedule(static)
    for (size_t bb = 0; bb < B; ++bb)
        for (size_t hh = 0; hh < H; ++hh) {
            double *h = (double *)calloc(P * N + 1, sizeof(double));
            double *lu = (double *)calloc(P * N + 1, sizeof(double));
            double *u = (double *)calloc(P * N + 1, sizeof(double));
            double *phi = (double *)calloc(half + 1, sizeof(double));
            double *bt = (double *)calloc(N * R + 1, sizeof(double));
            double *ct = (double *)calloc(N * R + 1, sizeof(double));
            size_t so = (bb * H + hh) * P * N;
            if (h0)
                for (size_t i = 0; i < P * N; ++i) h[i] = h0[so + i];
            if (last_u0 && g_fault != M3O_FAULT_CARRY_BETA)
                for (size_t i = 0; i < P * N; ++i) lu[i] = last_u0[so + i];
            if (angle0)
                for (size_t i = 0; i < half; ++i) phi[i] = angle0[(bb * H + hh) * half + i];
            double A = -exp((double)a_log[hh]);
            if (g_fault == M3O_FAULT_DECAY_SIGN) A = -A;
            for (size_t t = 0; t < T; ++t) {
                size_t idx = (bb * T + t) * H + hh;
                double step = dt[idx], lam = lambda[idx];
                double alpha = exp(step * A);
                double beta = (1.0 - lam) * step * alpha;
                double gamma = lam * step;
                if (g_fault == M3O_FAULT_DROP_BETA) beta = 0.0;
                if (g_fault == M3O_FAULT_LAMBDA_INDEX) {
                    /* planted: b_t reads lambda_{t-1} instead of lambda_t */
                    double lp = t ? lambda[(bb * T + t - 1) * H + hh] : lam;
                    beta = (1.0 - lp) * step * alpha;
                }
                const float *bs = b + idx * N * R;
                const float *cs = c + idx * N * R;
                for (size_t i = 0; i < N * R; ++i) { bt[i] = bs[i]; ct[i] = cs[i]; }
                if (theta) {
                    for (size_t i = 0; i < half; ++i) {
                        phi[i] += step * (double)theta[idx * half + i];
                        for (size_t r = 0; r < R; ++r) {
                            double o1, o2;
                            rot_neg_f64(phi[i], bs[i * R + r], bs[(i + half) * R + r], &o1, &o2);
                            bt[i * R + r] = o1; bt[(i + half) * R + r] = o2;
                            rot_neg_f64(phi[i], cs[i * R + r], cs[(i + half) * R + r], &o1, &o2);
                            ct[i * R + r] = o1; ct[(i + half) * R + r] = o2;
                        }
                    }
                }
                const float *xs = x + idx * P * R;
                for (size_t p = 0; p < P; ++p)
                    for (size_t n = 0; n < N; ++n) {
                        double acc = 0.0;
                        for (size_t r = 0; r < R; ++r) {
                            if (g_fault == M3O_FAULT_TRANSPOSE_U && P == N)
                                acc += (double)xs[n * R + r] * bt[p * R + r];
                            else
                                acc += (double)xs[p * R + r] * bt[n * R + r];
                        }
                        u[p * N + n] = acc;
                    }
                for (size_t i = 0; i < P * N; ++i) {
                    h[i] = alpha * h[i] + beta * lu[i] + gamma * u[i];
                    lu[i] = u[i];
                }
                if (y) {
                    double *ys = y + idx * P * R;
                    for (size_t p = 0; p < P; ++p)
                        for (size_t r = 0; r < R; ++r) {
                            double acc = 0.0;
                            for (size_t n = 0; n < N; ++n) acc += ct[n * R + r] * h[p * N + n];
                            double skip = 0.0;
                            if (d_skip) skip = (double)d_skip[hh] * (double)xs[p * R + r];
                            if (g_fault == M3O_FAULT_SKIP_SIGN) skip = -skip;
                            ys[p * R + r] = acc + skip;
                        }
                }
            }
            if (h_out) for (size_t i = 0; i < P * N; ++i) h_out[so + i] = h[i];
            if (last_u_out) {
                if (T == 0 && last_u0)
                    for (size_t i = 0; i < P * N; ++i) last_u_out[so + i] = last_u0[so + i];
                else
                    for (size_t i = 0; i < P * N; ++i) last_u_out[so + i] = T ? lu[i] : 0.0;
            }
            if (angle_out)
                for (size_t i = 0; i < half; ++i)
                    angle_out[(bb * H + hh) * half + i] = T ? wrap_pi_f64(phi[i]) : phi[i];
            free(h); free(lu); free(u); free(phi); free(bt); free(ct);
        }
}

/*
 * Reverse mode of m3o_scan_recurrence_f64 (the gradient the reference gets by
 * autodiff through mamba3_scan, src/ssm/scan.rs:458-638, whose hand-written
 * pieces are ssd_band_backward fused.rs:2080-2138, exp_decay_backward
 * 2326-2382 and trapezoid_weights_backward 2513-2549), evaluated token by
 * token in double precision.
 *
 * Forward, per (batch, head):  h_t = alpha_t h_{t-1} + beta_t u_{t-1} + gamma_t u_t,
 * u_t = sum_r x_t[:, r] B~_t[:, r]^T, y_t = C~_t^T h_t + D x_t, with
 * phi_t = angle0 + sum_{s<=t} dt_s theta_s (the angle is wrapped only where it
 * is output, so its derivative is 1).  Backward walks t = T-1 .. 0 carrying
 * dh = dL/dh_t, dlu = dL/du_t (through beta_{t+1}) and the running sum of
 * dL/dphi over t' >= t; states are recomputed from checkpoints every
 * M3O_BWD_SEG tokens.
 *
 * Inputs as m3o_scan_recurrence_f64, plus dy [B,T,H,P,R] and the optional
 * upstream gradients of the outgoing state dh_out, dlast_u_out [B,H,P,N],
 * dangle_out [B,H,N/2] (NULL = zero).  Outputs (any may be NULL): dx, db, dc,
 * ddt, dlambda, dtheta (theta's layout), da_log [H], dd_skip [H] (summed over
 * the batch), dh0, dlast_u0 [B,H,P,N], dangle0 [B,H,N/2].
 */
#define M3O_BWD_SEG 32

void m3o_scan_backward_f64(size_t B, size_t T, size_t H, size_t P, size_t N, size_t R,
                           const float *x, const float *b, const float *c, const float *dt,
                           const float *a_log, const float *lambda, const float *theta,
                           const float *d_skip, const float *h0, const float *last_u0,
                           const float *angle0, const double *dy, const double *dh_out,
                           const double *dlast_u_out, const double *dangle_out, double *dx,
                           double *db, double *dc, double *ddt, double *dlambda,
                           double *dtheta, double *da_log, double *dd_skip, double *dh0,
                           double *dlast_u0, double *dangle0) {
    const size_t half = N / 2, PN = P * N, NR = N * R;
    double *part_a = (double *)calloc(B * H + 1, sizeof(double));
    double *part_d = (double *)calloc(B * H + 1, sizeof(double));
    #pragma omp parallel for collapse(2) schedule(static)
    for (size_t bb = 0; bb < B; ++bb)
        for (size_t hh = 0; hh < H; ++hh) {
            const size_t nseg = (T + M3O_BWD_SEG - 1) / M3O_BWD_SEG;
            double *alpha = (double *)calloc(T + 1, sizeof(double));
            double *beta = (double *)calloc(T + 1, sizeof(double));
            double *gamma = (double *)calloc(T + 1, sizeof(double));
            double *phi = (double *)calloc(T * half + 1, sizeof(double));
            double *bt = (double *)calloc(T * NR + 1, sizeof(double));
            double *ct = (double *)calloc(T * NR + 1, sizeof(double));
            double *hck = (double *)calloc((nseg + 1) * PN + 1, sizeof(double));
            double *luck = (double *)calloc((nseg + 1) * PN + 1, sizeof(double));
            double *hs = (double *)calloc(M3O_BWD_SEG * PN + 1, sizeof(double));
            double *us = (double *)calloc(M3O_BWD_SEG * PN + 1, sizeof(double));
            double *h = (double *)calloc(PN + 1, sizeof(double));
            double *lu = (double *)calloc(PN + 1, sizeof(double));
            double *dh = (double *)calloc(PN + 1, sizeof(double));
            double *dlu = (double *)calloc(PN + 1, sizeof(double));
            double *du = (double *)calloc(PN + 1, sizeof(double));
            double *dbt = (double *)calloc(NR + 1, sizeof(double));
            double *dct = (double *)calloc(NR + 1, sizeof(double));
            double *dphi = (double *)calloc(half + 1, sizeof(double));
            const size_t so = (bb * H + hh) * PN;
            const double A = -exp((double)a_log[hh]);
            const double D = d_skip ? (double)d_skip[hh] : 0.0;
            double dA = 0.0, dD = 0.0;

            /* per-token coefficients and rotated B, C (as the forward) */
            for (size_t i = 0; i < half; ++i) dphi[i] = angle0 ? angle0[(bb * H + hh) * half + i] : 0.0;
            for (size_t t = 0; t < T; ++t) {
                const size_t idx = (bb * T + t) * H + hh;
                const double step = dt[idx], lam = lambda[idx];
                alpha[t] = exp(step * A);
                beta[t] = (1.0 - lam) * step * alpha[t];
                gamma[t] = lam * step;
                if (g_fault == M3O_FAULT_DROP_BETA) beta[t] = 0.0;
                const float *bs = b + idx * NR, *cs = c + idx * NR;
                for (size_t i = 0; i < NR; ++i) { bt[t * NR + i] = bs[i]; ct[t * NR + i] = cs[i]; }
                if (theta)
                    for (size_t i = 0; i < half; ++i) {
                        dphi[i] += step * (double)theta[idx * half + i];
                        phi[t * half + i] = dphi[i];
                        for (size_t r = 0; r < R; ++r) {
                            double o1, o2;
                            rot_neg_f64(dphi[i], bs[i * R + r], bs[(i + half) * R + r], &o1, &o2);
                            bt[t * NR + i * R + r] = o1; bt[t * NR + (i + half) * R + r] = o2;
                            rot_neg_f64(dphi[i], cs[i * R + r], cs[(i + half) * R + r], &o1, &o2);
                            ct[t * NR + i * R + r] = o1; ct[t * NR + (i + half) * R + r] = o2;
                        }
                    }
            }
            /* forward with a checkpoint of (h, last_u) at every segment start */
            if (h0) for (size_t i = 0; i < PN; ++i) h[i] = h0[so + i];
            if (last_u0) for (size_t i = 0; i < PN; ++i) lu[i] = last_u0[so + i];
            for (size_t t = 0; t < T; ++t) {
                if (t % M3O_BWD_SEG == 0) {
                    memcpy(hck + (t / M3O_BWD_SEG) * PN, h, PN * sizeof(double));
                    memcpy(luck + (t / M3O_BWD_SEG) * PN, lu, PN * sizeof(double));
                }
                const float *xs = x + ((bb * T + t) * H + hh) * P * R;
                for (size_t p = 0; p < P; ++p)
                    for (size_t n = 0; n < N; ++n) {
                        double acc = 0.0;
                        for (size_t r = 0; r < R; ++r) acc += (double)xs[p * R + r] * bt[t * NR + n * R + r];
                        h[p * N + n] = alpha[t] * h[p * N + n] + beta[t] * lu[p * N + n] + gamma[t] * acc;
                        lu[p * N + n] = acc;
                    }
            }

            /* backward */
            for (size_t i = 0; i < PN; ++i) {
                dh[i] = dh_out ? dh_out[so + i] : 0.0;
                dlu[i] = dlast_u_out ? dlast_u_out[so + i] : 0.0;
            }
            for (size_t i = 0; i < half; ++i)
                dphi[i] = dangle_out ? dangle_out[(bb * H + hh) * half + i] : 0.0;
            for (size_t sg = nseg; sg-- > 0;) {
                const size_t t0 = sg * M3O_BWD_SEG;
                const size_t t1 = (t0 + M3O_BWD_SEG < T) ? t0 + M3O_BWD_SEG : T;
                memcpy(h, hck + sg * PN, PN * sizeof(double));
                memcpy(lu, luck + sg * PN, PN * sizeof(double));
                for (size_t t = t0; t < t1; ++t) {
                    const float *xs = x + ((bb * T + t) * H + hh) * P * R;
                    double *hv = hs + (t - t0) * PN, *uv = us + (t - t0) * PN;
                    for (size_t p = 0; p < P; ++p)
                        for (size_t n = 0; n < N; ++n) {
                            double acc = 0.0;
                            for (size_t r = 0; r < R; ++r) acc += (double)xs[p * R + r] * bt[t * NR + n * R + r];
                            h[p * N + n] = alpha[t] * h[p * N + n] + beta[t] * lu[p * N + n] + gamma[t] * acc;
                            lu[p * N + n] = acc;
                            hv[p * N + n] = h[p * N + n];
                            uv[p * N + n] = acc;
                        }
                }
                for (size_t t = t1; t-- > t0;) {
                    const size_t idx = (bb * T + t) * H + hh;
                    const float *xs = x + idx * P * R;
                    const double *hv = hs + (t - t0) * PN, *uv = us + (t - t0) * PN;
                    const double *hp = (t > t0) ? hs + (t - 1 - t0) * PN : hck + sg * PN;
                    const double *up = (t > t0) ? us + (t - 1 - t0) * PN : luck + sg * PN;
                    double ddt_t = 0.0, dlam_t = 0.0;
                    for (size_t i = 0; i < NR; ++i) { dbt[i] = 0.0; dct[i] = 0.0; }
                    /* y_t = C~_t^T h_t + D x_t */
                    for (size_t p = 0; p < P; ++p)
                        for (size_t r = 0; r < R; ++r) {
                            const double g = dy[idx * P * R + p * R + r];
                            dD += g * (double)xs[p * R + r];
                            if (dx) dx[idx * P * R + p * R + r] = D * g;
                            for (size_t n = 0; n < N; ++n) {
                                dh[p * N + n] += g * ct[t * NR + n * R + r];
                                dct[n * R + r] += g * hv[p * N + n];
                            }
                        }
                    /* h_t = alpha h_{t-1} + beta u_{t-1} + gamma u_t */
                    double dal = 0.0, dbe = 0.0, dga = 0.0;
                    for (size_t i = 0; i < PN; ++i) {
                        dal += dh[i] * hp[i];
                        dbe += dh[i] * up[i];
                        dga += dh[i] * uv[i];
                        du[i] = gamma[t] * dh[i] + dlu[i];
                        dlu[i] = beta[t] * dh[i];
                        dh[i] = alpha[t] * dh[i];
                    }
                    /* u_t = sum_r x_t[:, r] B~_t[:, r]^T */
                    for (size_t p = 0; p < P; ++p)
                        for (size_t r = 0; r < R; ++r) {
                            double acc = 0.0;
                            for (size_t n = 0; n < N; ++n) acc += du[p * N + n] * bt[t * NR + n * R + r];
                            if (dx) dx[idx * P * R + p * R + r] += acc;
                        }
                    for (size_t n = 0; n < N; ++n)
                        for (size_t r = 0; r < R; ++r) {
                            double acc = 0.0;
                            for (size_t p = 0; p < P; ++p) acc += du[p * N + n] * (double)xs[p * R + r];
                            dbt[n * R + r] = acc;
                        }
                    /* alpha = exp(dt A), beta = (1 - lambda) dt alpha, gamma = lambda dt */
                    const double step = dt[idx], lam = lambda[idx], al = alpha[t];
                    ddt_t += dal * al * A;
                    dA += dal * al * step;
                    if (g_fault != M3O_FAULT_DROP_BETA) {
                        dlam_t -= dbe * step * al;
                        ddt_t += dbe * (1.0 - lam) * (al + step * al * A);
                        dA += dbe * (1.0 - lam) * step * al * step;
                    }
                    dlam_t += dga * step;
                    ddt_t += dga * lam;
                    /* rotation by -phi: dB = R(phi) dB~, dphi = dB~1 B~2 - dB~2 B~1 (and C) */
                    if (theta) {
                        for (size_t i = 0; i < half; ++i) {
                            const double ph = phi[t * half + i], cs = cos(ph);
                            const double sn = (g_fault == M3O_FAULT_BWD_ROT_SIGN) ? -sin(ph) : sin(ph);
                            double dp = 0.0;
                            for (size_t r = 0; r < R; ++r) {
                                const size_t i1 = i * R + r, i2 = (i + half) * R + r;
                                const double b1 = bt[t * NR + i1], b2 = bt[t * NR + i2];
                                const double c1 = ct[t * NR + i1], c2 = ct[t * NR + i2];
                                dp += dbt[i1] * b2 - dbt[i2] * b1 + dct[i1] * c2 - dct[i2] * c1;
                                const double db1 = dbt[i1] * cs - dbt[i2] * sn;
                                const double db2 = dbt[i1] * sn + dbt[i2] * cs;
                                const double dc1 = dct[i1] * cs - dct[i2] * sn;
                                const double dc2 = dct[i1] * sn + dct[i2] * cs;
                                dbt[i1] = db1; dbt[i2] = db2; dct[i1] = dc1; dct[i2] = dc2;
                            }
                            dphi[i] += dp;
                            if (dtheta) dtheta[idx * half + i] = step * dphi[i];
                            ddt_t += (double)theta[idx * half + i] * dphi[i];
                        }
                    }
                    if (db) for (size_t i = 0; i < NR; ++i) db[idx * NR + i] = dbt[i];
                    if (dc) for (size_t i = 0; i < NR; ++i) dc[idx * NR + i] = dct[i];
                    if (ddt) ddt[idx] = ddt_t;
                    if (dlambda) dlambda[idx] = dlam_t;
                }
            }
            if (dh0) for (size_t i = 0; i < PN; ++i) dh0[so + i] = dh[i];
            if (dlast_u0) for (size_t i = 0; i < PN; ++i) dlast_u0[so + i] = dlu[i];
            if (dangle0)
                for (size_t i = 0; i < half; ++i) dangle0[(bb * H + hh) * half + i] = theta ? dphi[i] : 0.0;
            part_a[bb * H + hh] = dA * A;
            part_d[bb * H + hh] = dD;
            free(alpha); free(beta); free(gamma); free(phi); free(bt); free(ct); free(hck);
            free(luck); free(hs); free(us); free(h); free(lu); free(dh); free(dlu); free(du);
            free(dbt); free(dct); free(dphi);
        }
    for (size_t hh = 0; hh < H; ++hh) {
        double sa = 0.0, sd = 0.0;
        for (size_t bb = 0; bb < B; ++bb) { sa += part_a[bb * H + hh]; sd += part_d[bb * H + hh]; }
        if (da_log) da_log[hh] = sa;
        if (dd_skip) dd_skip[hh] = sd;
    }
    free(part_a);
    free(part_d);
}

/* ---------------------------------------------------------------------------
 * 3a. The fused forward kernels, restated elementwise.
 * ------------------------------------------------------------------------- */

/* src/tensor/ops/scan.rs:18-51 -- one lane walks the axis serially; `outer`
 * rows, `len` along the axis, `inner` lanes beside it. */
void m3o_cumsum(const float *in, float *out, size_t outer, size_t len, size_t inner,
                int reverse, int exclusive) {
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < inner; ++i) {
            size_t base = o * len * inner + i;
            float acc = 0.0f;
            for (size_t step = 0; step < len; ++step) {
                size_t idx = reverse ? len - 1 - step : step;
                float v = in[base + idx * inner];
                if (exclusive) { out[base + idx * inner] = acc; acc += v; }
                else { acc += v; out[base + idx * inner] = acc; }
            }
        }
}

/* src/tensor/ops/elemwise.rs:349: x - round(x / a) * a. */
float m3o_wrap_to(float x, float a) { return x - roundf(x / a) * a; }

/* src/tensor/ops/fused.rs:2483-2503: g = lambda*dt; w = g + (1-lambda_{t+1}) dt_{t+1},
 * the shifted term zero at t = seq-1.  Layout [outer, seq, inner]. */
void m3o_trapezoid_weights(const float *lambda, const float *dt, float *g, float *w,
                           size_t outer, size_t seq, size_t inner) {
    size_t n = outer * seq * inner;
    for (size_t pos = 0; pos < n; ++pos) {
        size_t t = (pos / inner) % seq;
        float gv = lambda[pos] * dt[pos];
        float f = 0.0f;
        if (t + 1 < seq) {
            size_t next = pos + inner;
            float lam = (g_fault == M3O_FAULT_LAMBDA_INDEX) ? lambda[pos] : lambda[next];
            f = (1.0f - lam) * dt[next];
        }
        if (g_fault == M3O_FAULT_DROP_BETA) f = 0.0f;
        g[pos] = gv;
        w[pos] = gv + f;
    }
}

static float clamp_decay(float d) {
    /* .max(floor).min(0) as in fused.rs:2064 / 2310 */
    float v = d < M3O_LOG_DECAY_FLOOR ? M3O_LOG_DECAY_FLOOR : d;
    return v > 0.0f ? 0.0f : v;
}

/* src/tensor/ops/fused.rs:2044-2070: band[row][t][s]. */
void m3o_ssd_band(const float *acum, const float *w, const float *g, float *out, size_t rows,
                  size_t chunk) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t t = 0; t < chunk; ++t)
            for (size_t s = 0; s < chunk; ++s) {
                float v = 0.0f;
                if (s <= t) {
                    float d = clamp_decay(acum[r * chunk + t] - acum[r * chunk + s]);
                    float scale = (s == t) ? g[r * chunk + s] : w[r * chunk + s];
                    v = scale * expf(d);
                }
                out[(r * chunk + t) * chunk + s] = v;
            }
}

/* src/tensor/ops/fused.rs:2281-2318 for one element: exp(clamp(a - b)) * m. */
float m3o_exp_decay1(float a, float b, float m) { return expf(clamp_decay(a - b)) * m; }

/* src/tensor/ops/fused.rs:1679-1697, packed [3, B*H]. */
void m3o_ssm_coefficients(const float *a_log, const float *dt, const float *lambda,
                          float *out, size_t heads, size_t lanes) {
    for (size_t i = 0; i < lanes; ++i) {
        float a = 0.0f - expf(a_log[i % heads]);
        if (g_fault == M3O_FAULT_DECAY_SIGN) a = -a;
        float step = dt[i], lam = lambda[i];
        float alpha = expf(step * a);
        out[i] = alpha;
        out[lanes + i] = (g_fault == M3O_FAULT_DROP_BETA) ? 0.0f : (1.0f - lam) * step * alpha;
        out[2 * lanes + i] = lam * step;
    }
}

static const float M3O_TWO_PI = 6.28318530717958647692f; /* 2.0 * f32::consts::PI */

/* src/tensor/ops/fused.rs:1534-1555: phi = wrap(prev + dt*theta); `inner` angles
 * per (batch, head) lane. */
void m3o_ssm_angle(const float *dt, const float *theta, const float *prev, float *phi,
                   size_t inner, size_t lanes) {
    const float inv_two_pi = 1.0f / M3O_TWO_PI;
    for (size_t i = 0; i < lanes; ++i) {
        float raw = theta[i] * dt[i / inner];
        if (prev) raw += prev[i];
        float turns = roundf(raw * inv_two_pi);
        phi[i] = raw - turns * M3O_TWO_PI;
    }
}

/* src/tensor/ops/fused.rs:588-619 with from_angle: rows of length 2*half; row r
 * reads table row (r / repeat) % table_rows.  Rotates by -phi. */
void m3o_rotate_by_angle(const float *x, const float *phi, float *out, size_t rows,
                         size_t half, size_t repeat, size_t table_rows) {
    for (size_t row = 0; row < rows; ++row)
        for (size_t i = 0; i < half; ++i) {
            size_t base = row * half * 2;
            size_t tab = ((row / repeat) % table_rows) * half + i;
            float x1 = x[base + i], x2 = x[base + half + i];
            float cs = cosf(phi[tab]);
            float sn = -sinf(phi[tab]);
            if (g_fault == M3O_FAULT_ROT_SIGN) sn = -sn;
            out[base + i] = x1 * cs - x2 * sn;
            out[base + half + i] = x1 * sn + x2 * cs;
        }
}

/* ---------------------------------------------------------------------------
 * 3b. ssd_chunked, stage for stage (src/ssm/scan.rs:116-291).
 * x [B,T,H,P], b, c [B,T,H,N], a, g, w [B,T,H], init [B,H,P,N] or NULL.
 * Everything in ssd_chunked is independent across (batch, head): the permutes
 * only reorder, so each (b, h) pair is computed on its own, in parallel.
 * ------------------------------------------------------------------------- */
void m3o_ssd_chunked_f32(size_t B, size_t T, size_t H, size_t P, size_t N,
                         const float *x, const float *b, const float *c, const float *a,
                         const float *g, const float *w, const float *init,
                         size_t chunk_size, int want_state, float *y, float *final_state) {
    if (T == 0) { /* scan.rs:134-144 */
        if (want_state && final_state) {
            size_t n = B * H * P * N;
            if (init) memcpy(final_state, init, n * sizeof(float));
            else memset(final_state, 0, n * sizeof(float));
        }
        return;
    }
    size_t chunk = chunk_size < 1 ? 1 : (chunk_size > T ? T : chunk_size); /* 146 */
    size_t pad = (chunk - T % chunk) % chunk;
    size_t L = T + pad, C = L / chunk;

    #pragma omp parallel for collapse(2) schedule(dynamic)
    for (size_t bb = 0; bb < B; ++bb)
        for (size_t hh = 0; hh < H; ++hh) {
            /* zero-padded per-(b,h) sequences (scan.rs:151-165) */
            float *xs = (float *)calloc(L * P, sizeof(float));
            float *bs = (float *)calloc(L * N, sizeof(float));
            float *cs = (float *)calloc(L * N, sizeof(float));
            float *as = (float *)calloc(L, sizeof(float));
            float *gs = (float *)calloc(L, sizeof(float));
            float *ws = (float *)calloc(L, sizeof(float));
            for (size_t t = 0; t < T; ++t) {
                size_t idx = (bb * T + t) * H + hh;
                memcpy(xs + t * P, x + idx * P, P * sizeof(float));
                memcpy(bs + t * N, b + idx * N, N * sizeof(float));
                memcpy(cs + t * N, c + idx * N, N * sizeof(float));
                as[t] = a[idx]; gs[t] = g[idx]; ws[t] = w[idx];
            }
            /* acum = cumsum within each chunk (scan.rs:169) */
            float *acum = (float *)malloc(L * sizeof(float));
            m3o_cumsum(as, acum, C, chunk, 1, 0, 0);

            float *band = (float *)malloc(chunk * chunk * sizeof(float));
            float *yd = (float *)calloc(L * P, sizeof(float));
            float *cst = (float *)calloc(C * P * N, sizeof(float)); /* chunk_state [C][P][N] */
            float *wx = (float *)malloc(chunk * P * sizeof(float));
            for (size_t k = 0; k < C; ++k) {
                const float *ak = acum + k * chunk;
                /* 1. intra-chunk: band (fused.rs:2044-2070), cb = C B^T, (cb*band) X */
                m3o_ssd_band(ak, ws + k * chunk, gs + k * chunk, band, 1, chunk);
                for (size_t t = 0; t < chunk; ++t) {
                    float *yrow = yd + (k * chunk + t) * P;
                    for (size_t s = 0; s < chunk; ++s) {
                        float cb = 0.0f;
                        for (size_t n = 0; n < N; ++n)
                            cb += cs[(k * chunk + t) * N + n] * bs[(k * chunk + s) * N + n];
                        band[t * chunk + s] = cb * band[t * chunk + s]; /* mixing, in place */
                    }
                    for (size_t p = 0; p < P; ++p) {
                        float acc = 0.0f;
                        for (size_t s = 0; s < chunk; ++s)
                            acc += band[t * chunk + s] * xs[(k * chunk + s) * P + p];
                        yrow[p] = acc;
                    }
                }
                /* 2. chunk summary (scan.rs:207-216) */
                float last = ak[chunk - 1];
                for (size_t s = 0; s < chunk; ++s) {
                    float wt = (g_fault == M3O_FAULT_CHUNK_STATE_W) ? gs[k * chunk + s]
                                                                    : ws[k * chunk + s];
                    float d2e = m3o_exp_decay1(last, ak[s], wt);
                    for (size_t p = 0; p < P; ++p) wx[s * P + p] = xs[(k * chunk + s) * P + p] * d2e;
                }
                for (size_t p = 0; p < P; ++p)
                    for (size_t n = 0; n < N; ++n) {
                        float acc = 0.0f;
                        for (size_t s = 0; s < chunk; ++s)
                            acc += wx[s * P + p] * bs[(k * chunk + s) * N + n];
                        cst[(k * P + p) * N + n] = acc;
                    }
            }
            /* 3. inter-chunk recurrence as the O(C^2) masked product (scan.rs:218-251) */
            float *cdec = (float *)malloc(C * sizeof(float));
            float *before = (float *)malloc(C * sizeof(float));
            float *through = (float *)malloc(C * sizeof(float));
            for (size_t k = 0; k < C; ++k) cdec[k] = acum[k * chunk + chunk - 1];
            m3o_cumsum(cdec, before, 1, C, 1, 0, 1);
            m3o_cumsum(cdec, through, 1, C, 1, 0, 0);
            float *carry = (float *)calloc(C * P * N, sizeof(float));
            for (size_t k = 0; k < C; ++k)
                for (size_t e = 0; e < P * N; ++e) {
                    float acc = 0.0f;
                    for (size_t j = 0; j < C; ++j) {
                        float mask = j < k ? 1.0f : 0.0f; /* strict_causal_mask, base.rs:239-247 */
                        acc += m3o_exp_decay1(before[k], through[j], mask) * cst[j * P * N + e];
                    }
                    carry[k * P * N + e] = acc;
                }
            if (init) {
                const float *is = init + (bb * H + hh) * P * N;
                for (size_t k = 0; k < C; ++k) {
                    float sc = m3o_exp_decay1(before[k], 0.0f, 1.0f);
                    for (size_t e = 0; e < P * N; ++e) carry[k * P * N + e] += is[e] * sc;
                }
            }
            /* 4. carry-in contribution (scan.rs:253-268) */
            for (size_t k = 0; k < C; ++k)
                for (size_t t = 0; t < chunk; ++t) {
                    size_t tt = k * chunk + t;
                    float dec = m3o_exp_decay1(acum[tt], 0.0f, 1.0f);
                    for (size_t p = 0; p < P; ++p) {
                        float acc = 0.0f;
                        for (size_t n = 0; n < N; ++n)
                            acc += (cs[tt * N + n] * dec) * carry[(k * P + p) * N + n];
                        if (tt < T) y[((bb * T + tt) * H + hh) * P + p] = yd[tt * P + p] + acc;
                    }
                }
            /* boundary state (scan.rs:270-288) */
            if (want_state && final_state) {
                float tail = m3o_exp_decay1(cdec[C - 1], 0.0f, 1.0f);
                float *fs = final_state + (bb * H + hh) * P * N;
                for (size_t e = 0; e < P * N; ++e)
                    fs[e] = carry[(C - 1) * P * N + e] * tail + cst[(C - 1) * P * N + e];
            }
            free(xs); free(bs); free(cs); free(as); free(gs); free(ws); free(acum);
            free(band); free(yd); free(cst); free(wx); free(cdec); free(before);
            free(through); free(carry);
        }
}

/* ---------------------------------------------------------------------------
 * 3c. mamba3_scan, stage for stage (src/ssm/scan.rs:458-638).
 * Output pointers h_out / last_u_out / angle_out are written when want_state.
 * ------------------------------------------------------------------------- */
void m3o_scan_composed_f32(size_t B, size_t T, size_t H, size_t P, size_t N, size_t R,
                           const float *x, const float *b, const float *c, const float *dt,
                           const float *a_log, const float *lambda, const float *theta,
                           const float *d_skip, const float *h0, const float *last_u0,
                           const float *angle0, size_t chunk_size, int want_state, float *y,
                           float *h_out, float *last_u_out, float *angle_out) {
    size_t BTH = B * T * H, half = N / 2, SN = B * H * P * N;
    /* decay: a = dt * (-exp(a_log)) (scan.rs:468-475) */
    float *a = (float *)malloc((BTH + 1) * sizeof(float));
    for (size_t i = 0; i < BTH; ++i) {
        float ah = -expf(a_log[i % H]);
        if (g_fault == M3O_FAULT_DECAY_SIGN) ah = -ah;
        a[i] = dt[i] * ah;
    }
    /* trapezoid weights (scan.rs:477-479) */
    float *g = (float *)malloc((BTH + 1) * sizeof(float));
    float *w = (float *)malloc((BTH + 1) * sizeof(float));
    m3o_trapezoid_weights(lambda, dt, g, w, B, T, H);

    /* rotation (scan.rs:481-519): phi = wrap(cumsum_t(dt*theta) + prev) */
    size_t bcn = B * T * H * N * R;
    float *brot = (float *)malloc((bcn + 1) * sizeof(float));
    float *crot = (float *)malloc((bcn + 1) * sizeof(float));
    memcpy(brot, b, bcn * sizeof(float));
    memcpy(crot, c, bcn * sizeof(float));
    float *phi = NULL;
    if (theta && half) {
        size_t np = B * T * H * half;
        float *stepv = (float *)malloc(np * sizeof(float));
        phi = (float *)malloc(np * sizeof(float));
        for (size_t i = 0; i < np; ++i) stepv[i] = dt[i / half] * theta[i];
        m3o_cumsum(stepv, phi, B, T, H * half, 0, 0);
        if (angle0)
            for (size_t bb = 0; bb < B; ++bb)
                for (size_t t = 0; t < T; ++t)
                    for (size_t e = 0; e < H * half; ++e)
                        phi[(bb * T + t) * H * half + e] += angle0[bb * H * half + e];
        for (size_t i = 0; i < np; ++i) phi[i] = m3o_wrap_to(phi[i], 2.0f * 3.14159265358979323846f);
        /* [b,t,h,n,r] -> [b,t,h,r,n], rotate rows of length N sharing one table row
         * per (b,t,h) across the rank, then back. */
        float *moved = (float *)malloc(bcn * sizeof(float));
        float *done = (float *)malloc(bcn * sizeof(float));
        for (int which = 0; which < 2; ++which) {
            float *dst = which ? crot : brot;
            const float *src = which ? c : b;
            for (size_t row = 0; row < BTH; ++row)
                for (size_t n = 0; n < N; ++n)
                    for (size_t r = 0; r < R; ++r)
                        moved[(row * R + r) * N + n] = src[(row * N + n) * R + r];
            m3o_rotate_by_angle(moved, phi, done, BTH * R, half, R, BTH);
            for (size_t row = 0; row < BTH; ++row)
                for (size_t n = 0; n < N; ++n)
                    for (size_t r = 0; r < R; ++r)
                        dst[(row * N + n) * R + r] = done[(row * R + r) * N + n];
        }
        free(moved); free(done); free(stepv);
    }

    /* carry S = h + (1 - lambda_0) dt_0 last_u (scan.rs:521-535) */
    float *carry = NULL;
    if (h0 && last_u0) {
        carry = (float *)malloc((SN + 1) * sizeof(float));
        for (size_t bb = 0; bb < B; ++bb)
            for (size_t hh = 0; hh < H; ++hh) {
                float first = 0.0f;
                if (T > 0) {
                    size_t i0 = (bb * T) * H + hh;
                    first = (1.0f - lambda[i0]) * dt[i0];
                }
                if (g_fault == M3O_FAULT_CARRY_BETA || g_fault == M3O_FAULT_DROP_BETA) first = 0.0f;
                size_t so = (bb * H + hh) * P * N;
                for (size_t e = 0; e < P * N; ++e) carry[so + e] = h0[so + e] + last_u0[so + e] * first;
            }
    }

    /* R^2 SISO scans (scan.rs:537-589) */
    size_t xn = B * T * H * P, sn = B * T * H * N;
    float *xj = (float *)malloc((xn + 1) * sizeof(float));
    float *bj = (float *)malloc((sn + 1) * sizeof(float));
    float *ci = (float *)malloc((sn + 1) * sizeof(float));
    float *yij = (float *)malloc((xn + 1) * sizeof(float));
    float *acc = (float *)malloc((xn + 1) * sizeof(float));
    float *stj = (float *)malloc((SN + 1) * sizeof(float));
    float *total = want_state ? (float *)calloc(SN + 1, sizeof(float)) : NULL;
    int have_total = 0;
    for (size_t i = 0; i < R; ++i) {
        for (size_t e = 0; e < sn; ++e) ci[e] = crot[e * R + i];
        for (size_t j = 0; j < R; ++j) {
            if (g_fault == M3O_FAULT_MIMO_DIAG && i != j) continue;
            for (size_t e = 0; e < sn; ++e) bj[e] = brot[e * R + j];
            for (size_t e = 0; e < xn; ++e) xj[e] = x[e * R + j];
            m3o_ssd_chunked_f32(B, T, H, P, N, xj, bj, ci, a, g, w, j == 0 ? carry : NULL,
                                chunk_size, want_state, yij, stj);
            if (j == 0 || (g_fault == M3O_FAULT_MIMO_DIAG && j == i))
                memcpy(acc, yij, xn * sizeof(float));
            else
                for (size_t e = 0; e < xn; ++e) acc[e] += yij[e];
            if (i == 0 && want_state) {
                if (!have_total) { memcpy(total, stj, SN * sizeof(float)); have_total = 1; }
                else for (size_t e = 0; e < SN; ++e) total[e] += stj[e];
            }
        }
        for (size_t e = 0; e < xn; ++e) y[e * R + i] = acc[e];
    }
    /* skip path (scan.rs:593-597) */
    if (d_skip)
        for (size_t e = 0; e < xn * R; ++e) {
            size_t hh = (e / (P * R)) % H;
            float s = x[e] * d_skip[hh];
            y[e] = (g_fault == M3O_FAULT_SKIP_SIGN) ? y[e] - s : y[e] + s;
        }
    /* state to carry (scan.rs:599-638) */
    if (want_state) {
        if (h_out) memcpy(h_out, total, SN * sizeof(float));
        if (last_u_out) {
            if (T == 0) {
                if (last_u0) memcpy(last_u_out, last_u0, SN * sizeof(float));
                else memset(last_u_out, 0, SN * sizeof(float));
            } else
                for (size_t bb = 0; bb < B; ++bb)
                    for (size_t hh = 0; hh < H; ++hh) {
                        size_t idx = (bb * T + T - 1) * H + hh;
                        const float *xl = x + idx * P * R;
                        const float *bl = brot + idx * N * R;
                        float *lu = last_u_out + (bb * H + hh) * P * N;
                        for (size_t p = 0; p < P; ++p)
                            for (size_t n = 0; n < N; ++n) {
                                float s = 0.0f;
                                for (size_t r = 0; r < R; ++r) s += xl[p * R + r] * bl[n * R + r];
                                lu[p * N + n] = s;
                            }
                    }
        }
        if (angle_out && theta && half) {
            if (T == 0) {
                for (size_t e = 0; e < B * H * half; ++e) angle_out[e] = angle0 ? angle0[e] : 0.0f;
            } else
                for (size_t bb = 0; bb < B; ++bb)
                    memcpy(angle_out + bb * H * half, phi + (bb * T + T - 1) * H * half,
                           H * half * sizeof(float));
        }
    }
    free(a); free(g); free(w); free(brot); free(crot); free(phi); free(carry); free(xj);
    free(bj); free(ci); free(yij); free(acc); free(stj); free(total);
}

/* ---------------------------------------------------------------------------
 * 3d. mamba3_step (src/ssm/scan.rs:649-712), state updated in place.
 * x [B,H,P,R], b, c [B,H,N,R], dt, lambda [B,H], theta [B,H,N/2] or NULL,
 * h, last_u [B,H,P,N] (in/out), angle [B,H,N/2] (in/out; required with theta),
 * y [B,H,P,R].
 * ------------------------------------------------------------------------- */
void m3o_step_f32(size_t B, size_t H, size_t P, size_t N, size_t R, const float *x,
                  const float *b, const float *c, const float *dt, const float *lambda,
                  const float *a_log, const float *theta, const float *d_skip, float *h,
                  float *last_u, float *angle, float *y) {
    size_t BH = B * H, half = N / 2;
    float *coef = (float *)malloc(3 * (BH + 1) * sizeof(float));
    m3o_ssm_coefficients(a_log, dt, lambda, coef, H, BH);
    #pragma omp parallel for schedule(static)
    for (size_t bh = 0; bh < BH; ++bh) {
        float *bt = (float *)malloc((N * R + 1) * sizeof(float));
        float *ct = (float *)malloc((N * R + 1) * sizeof(float));
        float *u = (float *)malloc((P * N + 1) * sizeof(float));
        float *mv = (float *)malloc((N * R + 1) * sizeof(float));
        float *dn = (float *)malloc((N * R + 1) * sizeof(float));
        const float *bs = b + bh * N * R, *cs = c + bh * N * R;
        memcpy(bt, bs, N * R * sizeof(float));
        memcpy(ct, cs, N * R * sizeof(float));
        if (theta && half) {
            float *phi = angle + bh * half;
            float *nphi = (float *)malloc(half * sizeof(float));
            m3o_ssm_angle(dt + bh, theta + bh * half, phi, nphi, half, half);
            memcpy(phi, nphi, half * sizeof(float));
            free(nphi);
            for (int which = 0; which < 2; ++which) {
                const float *src = which ? cs : bs;
                float *dst = which ? ct : bt;
                for (size_t n = 0; n < N; ++n)
                    for (size_t r = 0; r < R; ++r) mv[r * N + n] = src[n * R + r];
                m3o_rotate_by_angle(mv, phi, dn, R, half, R, 1);
                for (size_t n = 0; n < N; ++n)
                    for (size_t r = 0; r < R; ++r) dst[n * R + r] = dn[r * N + n];
            }
        }
        const float *xs = x + bh * P * R;
        for (size_t p = 0; p < P; ++p)
            for (size_t n = 0; n < N; ++n) {
                float s = 0.0f;
                for (size_t r = 0; r < R; ++r) {
                    if (g_fault == M3O_FAULT_TRANSPOSE_U && P == N) s += xs[n * R + r] * bt[p * R + r];
                    else s += xs[p * R + r] * bt[n * R + r];
                }
                u[p * N + n] = s;
            }
        float al = coef[bh], be = coef[BH + bh], ga = coef[2 * BH + bh];
        float *hs = h + bh * P * N, *ls = last_u + bh * P * N;
        for (size_t e = 0; e < P * N; ++e) {
            hs[e] = hs[e] * al + ls[e] * be + u[e] * ga; /* fused.rs:1360-1362 */
            ls[e] = u[e];
        }
        float *ys = y + bh * P * R;
        for (size_t r = 0; r < R; ++r)
            for (size_t p = 0; p < P; ++p) {
                float s = 0.0f;
                for (size_t n = 0; n < N; ++n) s += ct[n * R + r] * hs[p * N + n];
                float sk = d_skip ? xs[p * R + r] * d_skip[bh % H] : 0.0f;
                if (g_fault == M3O_FAULT_SKIP_SIGN) sk = -sk;
                ys[p * R + r] = s + sk;
            }
        free(bt); free(ct); free(u); free(mv); free(dn);
    }
    free(coef);
}
