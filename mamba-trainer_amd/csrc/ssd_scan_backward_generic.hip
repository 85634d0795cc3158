// Backward of mamba3_scan for shapes the chunk kernels do not cover (any
// head_dim, d_state and rank whose per-token vectors fit 64 KB of LDS): the
// reverse mode of the recurrence itself, token by token, as the reference's
// autodiff differentiates its composed scan (scan.rs:458-638) and as the f64
// reference of the tests does it.  Per (batch, head) sequence, with
// u_t = sum_r x_t[:, r] B~_t[:, r]^T, alpha_t = exp(dt_t A),
// beta_t = (1 - lambda_t) dt_t alpha_t, gamma_t = lambda_t dt_t:
//   h_t = alpha_t h_{t-1} + beta_t u_{t-1} + gamma_t u_t,   y_t = C~_t^T h_t + D x_t,
// with h_{-1} = h0, u_{-1} = last_u0 and B~, C~ rotated by the running angle
// phi_t = wrap(phi_{t-1} + dt_t theta_t) (phi_{-1} = angle0), the angle the
// token-by-token forward (the step kernel) keeps.  The reverse walk carries
// dL/dh_t, dL/du_t (through beta_{t+1}) and the running dL/dphi; the states it
// needs are recomputed from checkpoints every kSeg tokens.  One workgroup per
// sequence, f32 throughout; slow by design (no BASELINE shape takes it).
#include "m3_device.hpp"
#include "m3_internal.hpp"

namespace m3 {

namespace {

constexpr int kGT = 256;     // threads of a workgroup
constexpr size_t kSeg = 32;  // tokens between state checkpoints

template <typename T>
__device__ __forceinline__ float ldg_(const void *p, size_t i) {
    return to_f32(static_cast<const T *>(p)[i]);
}
template <typename T>
__device__ __forceinline__ void stg_(void *p, size_t i, float v) {
    static_cast<T *>(p)[i] = from_f32<T>(v);
}

// rotation of a pair by -phi, (x1 cos + x2 sin, -x1 sin + x2 cos), with the
// step kernel's fused multiply-adds
__device__ __forceinline__ float rlo(float x1, float x2, float cs, float sn) {
    return __builtin_fmaf(x1, cs, x2 * sn);
}
__device__ __forceinline__ float rhi(float x1, float x2, float cs, float sn) {
    return __builtin_fmaf(x2, cs, -(x1 * sn));
}

// Per-sequence slices of the workspace (floats).
struct GenWs {
    float *phi;          // [T][N/2]: the angle after each token
    float *hck, *luck;   // [nseg][P N]: h and last_u entering each kSeg-token segment
    float *hs, *us;      // [kSeg][P N]: h_t and u_t of the segment being walked
    float *h, *lu;       // [P N]: running forward state
    float *dh, *dlu, *du;// [P N]
    float *part;         // [2]: dA * A and dD of this sequence
};

struct GenLayout {
    size_t per_seq;      // floats per sequence, 64-float aligned
    size_t phi, hck, luck, hs, us, h, lu, dh, dlu, du, part;
};

GenLayout gen_layout(const ScanLaunch &a) {
    const size_t PN = a.head_dim * a.d_state, nseg = (a.seq + kSeg - 1) / kSeg;
    auto up = [](size_t v) { return (v + 63) / 64 * 64; };
    GenLayout l;
    size_t o = 0;
    l.phi = o;  o += up(a.seq * (a.d_state / 2) + 1);
    l.hck = o;  o += up(nseg * PN);
    l.luck = o; o += up(nseg * PN);
    l.hs = o;   o += up(kSeg * PN);
    l.us = o;   o += up(kSeg * PN);
    l.h = o;    o += up(PN);
    l.lu = o;   o += up(PN);
    l.dh = o;   o += up(PN);
    l.dlu = o;  o += up(PN);
    l.du = o;   o += up(PN);
    l.part = o; o += 64;
    l.per_seq = o;
    return l;
}

size_t gen_lds_floats(const ScanLaunch &a) {
    const size_t PR = a.head_dim * a.rank, NR = a.d_state * a.rank, NH = a.d_state / 2;
    return 2 * PR + 4 * NR + 3 * NH + 8;
}

// Sum of v over the workgroup; every thread gets it.  red holds kGT / 64
// floats; the call begins and ends with a barrier of its own.
__device__ __forceinline__ float block_sum4(float v, float *red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < kGT / 64; ++w) s += red[w];
    __syncthreads();
    return s;
}

template <typename T>
__global__ void __launch_bounds__(kGT)
bwd_generic_kernel(ScanLaunch a, ScanGrads g, float *ws, GenLayout lay) {
    extern __shared__ float sm[];
    const size_t H = a.heads, L = a.seq, P = a.head_dim, N = a.d_state, R = a.rank;
    const size_t NH = N / 2, PN = P * N, NR = N * R, PR = P * R;
    const size_t bh = blockIdx.x, bb = bh / H, hh = bh % H;
    const int tid = threadIdx.x;
    const bool rot = a.theta != nullptr;
    float *xs = sm, *dys = xs + PR, *bt = dys + PR, *ct = bt + NR, *dbt = ct + NR;
    float *dct = dbt + NR, *cs = dct + NR, *sn = cs + NH, *dphr = sn + NH, *red = dphr + NH;
    float *base = ws + bh * lay.per_seq;
    GenWs w;
    w.phi = base + lay.phi;
    w.hck = base + lay.hck;
    w.luck = base + lay.luck;
    w.hs = base + lay.hs;
    w.us = base + lay.us;
    w.h = base + lay.h;
    w.lu = base + lay.lu;
    w.dh = base + lay.dh;
    w.dlu = base + lay.dlu;
    w.du = base + lay.du;
    w.part = base + lay.part;
    const float A = 0.0f - expf(a.a_log[hh]);
    const float D = a.d_skip ? a.d_skip[hh] : 0.0f;
    auto row = [&](size_t t) { return (bb * L + t) * H + hh; };

    // ---- the angle after each token, per pair (the step kernel's recurrence)
    if (rot) {
        for (size_t i = tid; i < NH; i += kGT) {
            float ph = a.angle0 ? a.angle0[bh * NH + i] : 0.0f;
            for (size_t t = 0; t < L; ++t) {
                const size_t ix = row(t);
                ph = wrap_angle(ldg_<T>(a.theta, ix * NH + i) * a.dt[ix] + ph);
                w.phi[t * NH + i] = ph;
            }
        }
    }
    __syncthreads();

    // token t's x (and dy) and its rotated B (and C) into LDS
    auto stage = [&](size_t t, bool back) {
        const size_t ix = row(t);
        if (rot)
            for (size_t i = tid; i < NH; i += kGT) {
                float s1, c1;
                sincosf(w.phi[t * NH + i], &s1, &c1);
                sn[i] = s1;
                cs[i] = c1;
            }
        __syncthreads();
        for (size_t e = tid; e < NR; e += kGT) {
            const size_t n = e / R, r = e % R;
            auto rotated = [&](const void *src) {
                const float v = ldg_<T>(src, ix * NR + e);
                if (!rot) return v;
                const size_t i = n < NH ? n : n - NH;
                const float v1 = ldg_<T>(src, ix * NR + i * R + r);
                const float v2 = ldg_<T>(src, ix * NR + (i + NH) * R + r);
                return n < NH ? rlo(v1, v2, cs[i], sn[i]) : rhi(v1, v2, cs[i], sn[i]);
            };
            bt[e] = rotated(a.b);
            if (back) ct[e] = rotated(a.c);
        }
        for (size_t e = tid; e < PR; e += kGT) {
            xs[e] = ldg_<T>(a.x, ix * PR + e);
            if (back) dys[e] = ldg_<T>(g.dy, ix * PR + e);
        }
        __syncthreads();
    };
    auto coeffs = [&](size_t t, float &al, float &be, float &ga) {
        const size_t ix = row(t);
        const float step = a.dt[ix], lam = a.lambda[ix];
        al = expf(step * A);
        be = (1.0f - lam) * step * al;
        ga = lam * step;
    };
    // one forward token on the running state; optionally keep h_t and u_t
    auto forward = [&](size_t t, float *hkeep, float *ukeep) {
        stage(t, false);
        float al, be, ga;
        coeffs(t, al, be, ga);
        for (size_t e = tid; e < PN; e += kGT) {
            const size_t p = e / N, n = e % N;
            float u = 0.0f;
            for (size_t r = 0; r < R; ++r) u = __builtin_fmaf(xs[p * R + r], bt[n * R + r], u);
            const float hn = al * w.h[e] + be * w.lu[e] + ga * u;
            w.h[e] = hn;
            w.lu[e] = u;
            if (hkeep) {
                hkeep[e] = hn;
                ukeep[e] = u;
            }
        }
        __syncthreads();
    };

    // ---- forward, with a checkpoint of (h, last_u) entering every segment
    for (size_t e = tid; e < PN; e += kGT) {
        w.h[e] = a.h0 ? a.h0[bh * PN + e] : 0.0f;
        w.lu[e] = a.last_u0 ? a.last_u0[bh * PN + e] : 0.0f;
    }
    for (size_t t = 0; t < L; ++t) {
        if (t % kSeg == 0)
            for (size_t e = tid; e < PN; e += kGT) {
                w.hck[(t / kSeg) * PN + e] = w.h[e];
                w.luck[(t / kSeg) * PN + e] = w.lu[e];
            }
        forward(t, nullptr, nullptr);
    }

    // ---- reverse
    for (size_t e = tid; e < PN; e += kGT) {
        w.dh[e] = g.dh_out ? g.dh_out[bh * PN + e] : 0.0f;
        w.dlu[e] = g.dlast_u_out ? g.dlast_u_out[bh * PN + e] : 0.0f;
    }
    for (size_t i = tid; i < NH; i += kGT) dphr[i] = (rot && g.dangle_out) ? g.dangle_out[bh * NH + i] : 0.0f;
    float dA = 0.0f, dD = 0.0f;   // thread 0's running sums
    const size_t nseg = (L + kSeg - 1) / kSeg;
    for (size_t sg = nseg; sg-- > 0;) {
        const size_t t0 = sg * kSeg, t1 = t0 + kSeg < L ? t0 + kSeg : L;
        for (size_t e = tid; e < PN; e += kGT) {
            w.h[e] = w.hck[sg * PN + e];
            w.lu[e] = w.luck[sg * PN + e];
        }
        for (size_t t = t0; t < t1; ++t) forward(t, w.hs + (t - t0) * PN, w.us + (t - t0) * PN);
        for (size_t t = t1; t-- > t0;) {
            stage(t, true);
            const size_t ix = row(t);
            const float *hv = w.hs + (t - t0) * PN, *uv = w.us + (t - t0) * PN;
            const float *hp = t > t0 ? w.hs + (t - 1 - t0) * PN : w.hck + sg * PN;
            const float *upv = t > t0 ? w.us + (t - 1 - t0) * PN : w.luck + sg * PN;
            float al, be, ga;
            coeffs(t, al, be, ga);
            // dC~ = h_t^T dy_t
            for (size_t e = tid; e < NR; e += kGT) {
                const size_t n = e / R, r = e % R;
                float acc = 0.0f;
                for (size_t p = 0; p < P; ++p) acc = __builtin_fmaf(dys[p * R + r], hv[p * N + n], acc);
                dct[e] = acc;
            }
            // dh_t += dy_t C~_t; the coefficient sums; du_t, then dL/du_{t-1}, dL/dh_{t-1}
            float pal = 0.0f, pbe = 0.0f, pga = 0.0f, pdd = 0.0f;
            for (size_t e = tid; e < PN; e += kGT) {
                const size_t p = e / N, n = e % N;
                float gy = 0.0f;
                for (size_t r = 0; r < R; ++r) gy = __builtin_fmaf(dys[p * R + r], ct[n * R + r], gy);
                const float dhv = w.dh[e] + gy;
                pal = __builtin_fmaf(dhv, hp[e], pal);
                pbe = __builtin_fmaf(dhv, upv[e], pbe);
                pga = __builtin_fmaf(dhv, uv[e], pga);
                w.du[e] = ga * dhv + w.dlu[e];
                w.dlu[e] = be * dhv;
                w.dh[e] = al * dhv;
            }
            for (size_t e = tid; e < PR; e += kGT) pdd = __builtin_fmaf(dys[e], xs[e], pdd);
            const float dal = block_sum4(pal, red), dbe = block_sum4(pbe, red);
            const float dga = block_sum4(pga, red), ddd = block_sum4(pdd, red);
            // dx_t = D dy_t + du_t B~_t; dB~_t = du_t^T x_t
            for (size_t e = tid; e < PR; e += kGT) {
                const size_t p = e / R, r = e % R;
                float acc = D * dys[e];
                for (size_t n = 0; n < N; ++n) acc = __builtin_fmaf(w.du[p * N + n], bt[n * R + r], acc);
                stg_<T>(g.dx, ix * PR + e, acc);
            }
            for (size_t e = tid; e < NR; e += kGT) {
                const size_t n = e / R, r = e % R;
                float acc = 0.0f;
                for (size_t p = 0; p < P; ++p) acc = __builtin_fmaf(w.du[p * N + n], xs[p * R + r], acc);
                dbt[e] = acc;
            }
            __syncthreads();
            // the rotation back (dB = R(phi) dB~) and the angle's gradient
            float pth = 0.0f;
            const float step = a.dt[ix], lam = a.lambda[ix];
            if (rot) {
                for (size_t i = tid; i < NH; i += kGT) {
                    float dp = 0.0f;
                    for (size_t r = 0; r < R; ++r) {
                        const size_t i1 = i * R + r, i2 = (i + NH) * R + r;
                        dp += dbt[i1] * bt[i2] - dbt[i2] * bt[i1] + dct[i1] * ct[i2] - dct[i2] * ct[i1];
                        const float b1 = dbt[i1], b2 = dbt[i2], c1 = dct[i1], c2 = dct[i2];
                        dbt[i1] = b1 * cs[i] - b2 * sn[i];
                        dbt[i2] = b1 * sn[i] + b2 * cs[i];
                        dct[i1] = c1 * cs[i] - c2 * sn[i];
                        dct[i2] = c1 * sn[i] + c2 * cs[i];
                    }
                    const float run = dphr[i] + dp;
                    dphr[i] = run;
                    stg_<T>(g.dtheta, ix * NH + i, step * run);
                    pth = __builtin_fmaf(ldg_<T>(a.theta, ix * NH + i), run, pth);
                }
            }
            const float dth = block_sum4(pth, red);
            for (size_t e = tid; e < NR; e += kGT) {
                stg_<T>(g.db, ix * NR + e, dbt[e]);
                stg_<T>(g.dc, ix * NR + e, dct[e]);
            }
            if (tid == 0) {
                // alpha = exp(dt A), beta = (1 - lambda) dt alpha, gamma = lambda dt
                float ddt = dal * al * A + dbe * (1.0f - lam) * (al + step * al * A) + dga * lam + dth;
                const float dlam = dga * step - dbe * step * al;
                dA += dal * al * step + dbe * (1.0f - lam) * step * al * step;
                dD += ddd;
                g.ddt[ix] = ddt;
                g.dlambda[ix] = dlam;
            }
            __syncthreads();   // LDS is restaged by the next token
        }
    }
    for (size_t e = tid; e < PN; e += kGT) {
        if (g.dh0) g.dh0[bh * PN + e] = w.dh[e];
        if (g.dlast_u0) g.dlast_u0[bh * PN + e] = w.dlu[e];
    }
    if (g.dangle0)
        for (size_t i = tid; i < NH; i += kGT) g.dangle0[bh * NH + i] = rot ? dphr[i] : 0.0f;
    if (tid == 0) {
        w.part[0] = dA * A;
        w.part[1] = dD;
    }
}

// da_log and dd_skip: the sequences' partial sums over the batch, in order.
__global__ void bwd_generic_head_kernel(ScanLaunch a, ScanGrads g, const float *ws, size_t per_seq,
                                        size_t part) {
    const size_t H = a.heads;
    for (size_t h = threadIdx.x; h < H; h += blockDim.x) {
        float sa = 0.0f, sd = 0.0f;
        for (size_t b = 0; b < a.batch; ++b) {
            const float *pp = ws + (b * H + h) * per_seq + part;
            sa += pp[0];
            sd += pp[1];
        }
        g.da_log[h] = sa;
        if (g.dd_skip) g.dd_skip[h] = sd;
    }
}

}  // namespace

bool scan_backward_generic_supported(const ScanLaunch &a) {
    return a.mode_raw && a.seq > 0 && a.head_dim > 0 && a.d_state > 0 && a.rank > 0 &&
           gen_lds_floats(a) * sizeof(float) <= 65536 &&
           (a.theta == nullptr || a.d_state % 2 == 0);
}

size_t scan_backward_generic_workspace(const ScanLaunch &a) {
    if (!scan_backward_generic_supported(a)) return 0;
    return a.batch * a.heads * gen_layout(a).per_seq * sizeof(float);
}

hipError_t launch_scan_backward_generic(const ScanLaunch &a, const ScanGrads &g, void *workspace,
                                        hipStream_t stream) {
    if (!scan_backward_generic_supported(a)) return hipErrorNotSupported;
    const GenLayout lay = gen_layout(a);
    float *ws = static_cast<float *>(workspace);
    const size_t lds = gen_lds_floats(a) * sizeof(float);
    const dim3 grid(static_cast<unsigned>(a.batch * a.heads));
    if (a.bf16)
        hipLaunchKernelGGL((bwd_generic_kernel<bf16_t>), grid, dim3(kGT), lds, stream, a, g, ws, lay);
    else
        hipLaunchKernelGGL((bwd_generic_kernel<float>), grid, dim3(kGT), lds, stream, a, g, ws, lay);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_generic_head_kernel, dim3(1), dim3(256), 0, stream, a, g,
                       static_cast<const float *>(ws), lay.per_seq, lay.part);
    return hipGetLastError();
}

}  // namespace m3
