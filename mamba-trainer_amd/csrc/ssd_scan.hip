// Chunked SSD scan of the Mamba-3 SSM for gfx950 (MI355X).
//
// Restates src/ssm/scan.rs:116-291 (ssd_chunked) and 458-638 (mamba3_scan):
// the trapezoidal two-band mask, the rotating frame, the MIMO fold, the carried
// state and the boundary state -- as ONE kernel per call instead of the
// reference's ~25-30 materialising launches per SISO system (and R^2 systems
// for MIMO).
//
// Design (one workgroup per (batch, head); wave w owns head_dim columns
// p in [16w, 16w+16)):
//   The sequence is walked chunk by chunk.  A chunk holds ROWS rows; a row is
//   a (token, rank) pair rho = t*R + r, so the MIMO fold is the same code as
//   SISO with R > 1 (scan.rs:537-589 become one rank-R contraction).
//   Per chunk:
//   S1  the per-token scalars -- log decay a = dt*A, trapezoid weights
//       g = lambda*dt, w = g + (1-lambda_{t+1}) dt_{t+1} (fused.rs:2483-2503),
//       their in-chunk prefix acum (ops/scan.rs:18-51), the decay-to-end
//       weights w*exp(clamp(acum_end - acum)) (fused.rs:2281-2318) -- with a
//       wave-level scan; and a blocked prefix of dt*theta for the frame angle.
//   S2  B and C rotated by -phi (fused.rs:588-619) straight into LDS as MFMA
//       operands, B a second time transposed and pre-scaled by the decay-to-
//       end weights, X transposed.  The angle stays chunk-relative on top of a
//       running wrapped angle, so it never grows past 2*pi (the reference
//       accumulates it absolutely in f32, scan.rs:490-497).
//   S3  MFMA: the masked C B^T band (ssd_band, fused.rs:2044-2070) is built in
//       registers from G^T = B~ C~^T and written to LDS; the carry-in output
//       (C~ exp(acum)) S^T (scan.rs:253-263) is accumulated straight from the
//       state registers; the state is advanced S = exp(dA) S + (w-decayed B~)^T X
//       (scan.rs:207-251 as an O(C) walk, not the O(C^2) transfer matrix).
//   S4  MFMA: y += (C B^T o band) X, skip D*x, store.
//   The state S (f32) never leaves the registers of the wave that owns it.
//
// Storage: bf16 inputs use bf16 MFMA operands with f32 accumulation; f32
// inputs use f32 MFMA (16x16x4) throughout.
#include "m3_device.hpp"
#include "m3_internal.hpp"

namespace m3 {

namespace {

// LDS-only barrier: waits for this wave's LDS traffic, not for in-flight
// global loads (the next chunk's prefetch stays in flight across it).
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0), vmcnt/expcnt untouched
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T> struct OpTraits;
template <> struct OpTraits<float> {
    using op_t = float;
    static constexpr int KB = 16;   // k per mma_kblock
};
template <> struct OpTraits<bf16_t> {
    using op_t = __bf16;
    static constexpr int KB = 32;
};

__device__ __forceinline__ float op_to_f32(float v) { return v; }
__device__ __forceinline__ float op_to_f32(__bf16 v) { return static_cast<float>(v); }
template <typename O> __device__ __forceinline__ O f32_to_op(float v);
template <> __device__ __forceinline__ float f32_to_op<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 f32_to_op<__bf16>(float v) {
    return static_cast<__bf16>(v);
}

// One K block of a 16x16 tile: `ar` is this lane's A row, `br` its B column
// (both k-contiguous in LDS), already offset to the block start.
__device__ __forceinline__ f32x4 mma_kblock(const __bf16 *ar, const __bf16 *br, f32x4 acc,
                                            int g) {
    bf16x8 av = *reinterpret_cast<const bf16x8 *>(ar + 8 * g);
    bf16x8 bv = *reinterpret_cast<const bf16x8 *>(br + 8 * g);
    return mfma_bf16(av, bv, acc);
}
__device__ __forceinline__ f32x4 mma_kblock(const float *ar, const float *br, f32x4 acc,
                                            int g) {
    f32x4 av = *reinterpret_cast<const f32x4 *>(ar + 4 * g);
    f32x4 bv = *reinterpret_cast<const f32x4 *>(br + 4 * g);
    acc = mfma_f32(av[0], bv[0], acc);
    acc = mfma_f32(av[1], bv[1], acc);
    acc = mfma_f32(av[2], bv[2], acc);
    acc = mfma_f32(av[3], bv[3], acc);
    return acc;
}

template <typename T>
__device__ __forceinline__ float ldg(const void *p, size_t i) {
    return to_f32(static_cast<const T *>(p)[i]);
}

__device__ __forceinline__ void fast_or_exact_sincos(float x, float *s, float *c, bool exact) {
    if (exact) {
        sincosf(x, s, c);
    } else {
        *s = __sinf(x);
        *c = __cosf(x);
    }
}

template <typename T, int NP, int PT, int ROWS>
struct ScanSmem {
    using op_t = typename OpTraits<T>::op_t;
    static constexpr int PAD = 16 / sizeof(op_t);
    static constexpr int LDN = NP + PAD;     // pitch of [row][n] operands
    static constexpr int LDR = ROWS + PAD;   // pitch of [*][row] operands
    static constexpr int NH = NP / 2;
    op_t Bs[ROWS * LDN];        // B~[rho][n]
    op_t Cs[ROWS * LDN];        // C~[rho][n]
    op_t Bwt[NP * LDR];         // (B~ * decay-to-end * w)^T [n][rho]
    op_t Xt[PT * 16 * LDR];     // X^T [p][rho]
    op_t Ms[ROWS * LDR];        // masked band (C~ B~^T o L)[rho_t][rho_s]
    float psi[ROWS * NH];       // in-block prefix of dt*theta [token][pair]
    float tot[PT * NH];         // per-block totals [block][pair]
    float phi0[NH];             // running wrapped angle entering the chunk
    float acum[ROWS], gw[ROWS], ww[ROWS], wdec[ROWS], eac[ROWS];
};

template <typename T, int NP, int PT, int ROWS>
__global__ void __launch_bounds__(64 * PT, 1)
ssd_scan_kernel(ScanLaunch a, int qtok, int nchunks) {
    using S = ScanSmem<T, NP, PT, ROWS>;
    using op_t = typename S::op_t;
    constexpr int KB = OpTraits<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int NT = ROWS / 16;          // row tiles per chunk
    constexpr int NTN = NP / 16;           // state-column tiles
    constexpr int THREADS = 64 * PT;
    constexpr bool kBf16 = sizeof(op_t) == 2;

    extern __shared__ __align__(16) unsigned char smem_raw[];
    S &sm = *reinterpret_cast<S *>(smem_raw);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq, P = a.head_dim, N = a.d_state, R = a.rank;
    const size_t bb = blockIdx.x / H, hh = blockIdx.x % H;
    const int NHr = static_cast<int>(N / 2);   // runtime pairs
    const bool rot = a.theta != nullptr;
    const int rows_live = qtok * static_cast<int>(R);
    const bool exact = !kBf16;

    // ---- zero every operand buffer once (pads, dead rows, upper band tiles)
    {
        uint32_t *z = reinterpret_cast<uint32_t *>(smem_raw);
        const int words = static_cast<int>(sizeof(S) / 4);
        for (int i = tid; i < words; i += THREADS) z[i] = 0u;
    }

    // ---- state registers: S^T[n][p] tiles, lane holds n = 16i + 4g + r, p = 16w + c
    f32x4 st[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int pcol = 16 * wave + c;
    {
        const size_t sbase = (bb * H + hh) * P * N;
        float first = 0.0f;
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        if (l0 != nullptr && L > 0) {
            // carry S = h + (1 - lambda_0) dt_0 last_u   (scan.rs:521-535)
            const size_t i0 = (bb * L) * H + hh;
            first = (1.0f - a.lambda[i0]) * a.dt[i0];
        }
        if (h0 != nullptr && pcol < static_cast<int>(P)) {
#pragma unroll
            for (int i = 0; i < NTN; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = 16 * i + 4 * g + r;
                    if (n < static_cast<int>(N)) {
                        float v = h0[sbase + pcol * N + n];
                        if (l0 != nullptr) v = v + l0[sbase + pcol * N + n] * first;
                        st[i][r] = v;
                    }
                }
        }
    }
    __syncthreads();
    if (rot) {
        for (int i = tid; i < NHr; i += THREADS)
            sm.phi0[i] = a.angle0 ? a.angle0[(bb * H + hh) * NHr + i] : 0.0f;
    }

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const int tb = (qtok + PT - 1) / PT;   // tokens per angle block

    __syncthreads();

    for (int ck = 0; ck < nchunks; ++ck) {
        const size_t tau0 = static_cast<size_t>(ck) * qtok;

        // ================= S1: per-token scalars + angle block prefix
        if (wave == 0) {
            const int t = lane;
            const size_t tau = tau0 + t;
            const bool live = t < qtok && tau < L;
            float av = 0.f, gv = 0.f, wv = 0.f;
            if (live) {
                const size_t idx = (bb * L + tau) * H + hh;
                if (a.mode_raw) {
                    const float d = a.dt[idx], l = a.lambda[idx];
                    av = d * A;
                    gv = l * d;                                  // fused.rs:2494
                    float f = 0.0f;
                    if (tau + 1 < L) {
                        const size_t nx = idx + H;
                        f = (1.0f - a.lambda[nx]) * a.dt[nx];    // fused.rs:2497-2498
                    }
                    wv = gv + f;
                } else {
                    av = a.a[idx];
                    gv = a.g[idx];
                    wv = a.w[idx];
                }
            }
            const float acum = wave_inclusive_scan(av, lane);
            const float last = __shfl(acum, qtok - 1, 64);
            if (t < qtok) {
                sm.acum[t] = acum;
                sm.gw[t] = gv;
                sm.ww[t] = wv;
                sm.wdec[t] = decay_exp(last - acum) * wv;   // exp_decay(last, acum, w)
                sm.eac[t] = decay_exp(acum);                // exp_decay(acum)
            }
        }
        if (rot) {
            const int t0 = wave * tb;
            const int t1 = min(t0 + tb, qtok);
            for (int i = lane; i < NHr; i += 64) {
                float acc = 0.0f;
                for (int t = t0; t < t1; ++t) {
                    const size_t tau = tau0 + t;
                    float inc = 0.0f;
                    if (tau < L) {
                        const size_t idx = (bb * L + tau) * H + hh;
                        inc = a.dt[idx] * ldg<T>(a.theta, idx * NHr + i);
                    }
                    acc += inc;
                    sm.psi[t * NHr + i] = acc;
                }
                sm.tot[wave * NHr + i] = acc;
            }
        }
        lds_barrier();

        // ================= S2: rotate / stage B~, C~, (B~ w decay)^T, X^T
        {
            const int npairs = rot ? NHr : static_cast<int>(N);
            const int items = rows_live * npairs;
            for (int it = tid; it < items; it += THREADS) {
                const int rho = it / npairs;
                const int i = it - rho * npairs;
                const int t = rho / static_cast<int>(R);
                const int r = rho - t * static_cast<int>(R);
                const size_t tau = tau0 + t;
                const bool live = tau < L;
                const size_t bcb = ((bb * L + (live ? tau : 0)) * H + hh) * N * R;
                const float wd = sm.wdec[t];
                if (rot) {
                    float b1 = 0.f, b2 = 0.f, c1 = 0.f, c2 = 0.f, phi = 0.f;
                    if (live) {
                        b1 = ldg<T>(a.b, bcb + i * R + r);
                        b2 = ldg<T>(a.b, bcb + (i + NHr) * R + r);
                        c1 = ldg<T>(a.c, bcb + i * R + r);
                        c2 = ldg<T>(a.c, bcb + (i + NHr) * R + r);
                        const int blk = t / tb;
                        float base = sm.phi0[i];
                        for (int k = 0; k < blk; ++k) base += sm.tot[k * NHr + i];
                        phi = wrap_angle(base + sm.psi[t * NHr + i]);
                        if (a.angle_out && tau == L - 1 && r == 0)
                            a.angle_out[(bb * H + hh) * NHr + i] = phi;
                    }
                    float sn, cs;
                    fast_or_exact_sincos(phi, &sn, &cs, exact);
                    const float rb1 = b1 * cs + b2 * sn, rb2 = -b1 * sn + b2 * cs;
                    const float rc1 = c1 * cs + c2 * sn, rc2 = -c1 * sn + c2 * cs;
                    sm.Bs[rho * LDN + i] = f32_to_op<op_t>(rb1);
                    sm.Bs[rho * LDN + i + NHr] = f32_to_op<op_t>(rb2);
                    sm.Cs[rho * LDN + i] = f32_to_op<op_t>(rc1);
                    sm.Cs[rho * LDN + i + NHr] = f32_to_op<op_t>(rc2);
                    sm.Bwt[i * LDR + rho] = f32_to_op<op_t>(rb1 * wd);
                    sm.Bwt[(i + NHr) * LDR + rho] = f32_to_op<op_t>(rb2 * wd);
                } else {
                    float bv = 0.f, cv = 0.f;
                    if (live) {
                        bv = ldg<T>(a.b, bcb + i * R + r);
                        cv = ldg<T>(a.c, bcb + i * R + r);
                    }
                    sm.Bs[rho * LDN + i] = f32_to_op<op_t>(bv);
                    sm.Cs[rho * LDN + i] = f32_to_op<op_t>(cv);
                    sm.Bwt[i * LDR + rho] = f32_to_op<op_t>(bv * wd);
                }
            }
            const int xitems = rows_live * static_cast<int>(P);
            for (int it = tid; it < xitems; it += THREADS) {
                const int rho = it / static_cast<int>(P);
                const int p = it - rho * static_cast<int>(P);
                const int t = rho / static_cast<int>(R);
                const int r = rho - t * static_cast<int>(R);
                const size_t tau = tau0 + t;
                float xv = 0.f;
                if (tau < L) xv = ldg<T>(a.x, (((bb * L + tau) * H + hh) * P + p) * R + r);
                sm.Xt[p * LDR + rho] = f32_to_op<op_t>(xv);
            }
        }
        lds_barrier();

        // ================= S3: band -> Ms, carry-in output, state advance
        f32x4 yacc[NT];
        {
            // (a) G^T tiles, masked, into Ms[t][s].  An s-tile is needed when its
            // first row's token is not after the last token of the t-tile; for a
            // rank that does not divide 16 a token's rows straddle two tiles, so
            // that includes the tile just above the diagonal.
            int idx = 0;
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const int tlast = (16 * tj + 15) / static_cast<int>(R);
#pragma unroll
                for (int si = 0; si < NT; ++si) {
                    if ((16 * si) / static_cast<int>(R) > tlast) continue;
                    if ((idx++) % PT != wave) continue;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *ar = &sm.Bs[(16 * si + c) * LDN];
                    const op_t *br = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
                    for (int kb = 0; kb < NP / KB; ++kb)
                        acc = mma_kblock(ar + kb * KB, br + kb * KB, acc, g);
                    const int trow = 16 * tj + c;
                    const int tt = trow / static_cast<int>(R);
                    float vals[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int srow = 16 * si + 4 * g + r;
                        const int ts = srow / static_cast<int>(R);
                        float v = 0.0f;
                        if (ts <= tt && tt < qtok) {
                            const float wgt = (ts == tt) ? sm.gw[ts] : sm.ww[ts];
                            v = acc[r] * wgt * decay_exp(sm.acum[tt] - sm.acum[ts]);
                        }
                        vals[r] = v;
                    }
                    op_t *dst = &sm.Ms[trow * LDR + 16 * si + 4 * g];
#pragma unroll
                    for (int r = 0; r < 4; ++r) dst[r] = f32_to_op<op_t>(vals[r]);
                }
            }

            // (b) carry-in output: y^T[p][t] = exp(acum_t) * sum_n S[p][n] C~[t][n]
            if constexpr (kBf16) {
                bf16x8 sa[NP / 32];
#pragma unroll
                for (int kb = 0; kb < NP / 32; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        sa[kb][j] = to_bf16(st[2 * kb][j]);
                        sa[kb][4 + j] = to_bf16(st[2 * kb + 1][j]);
                    }
#pragma unroll
                for (int tj = 0; tj < NT; ++tj) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *cr = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
                    for (int kb = 0; kb < NP / 32; ++kb) {
                        bf16x4 lo = *reinterpret_cast<const bf16x4 *>(cr + 32 * kb + 4 * g);
                        bf16x4 hi = *reinterpret_cast<const bf16x4 *>(cr + 32 * kb + 16 + 4 * g);
                        bf16x8 bv;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            bv[j] = lo[j];
                            bv[4 + j] = hi[j];
                        }
                        acc = mfma_bf16(sa[kb], bv, acc);
                    }
                    const int tt = (16 * tj + c) / static_cast<int>(R);
                    const float sc = tt < qtok ? sm.eac[tt] : 0.0f;
                    yacc[tj] = acc * sc;
                }
            } else {
#pragma unroll
                for (int tj = 0; tj < NT; ++tj) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *cr = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
                    for (int i = 0; i < NTN; ++i) {
                        f32x4 bv = *reinterpret_cast<const f32x4 *>(cr + 16 * i + 4 * g);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc = mfma_f32(st[i][r], bv[r], acc);
                    }
                    const int tt = (16 * tj + c) / static_cast<int>(R);
                    const float sc = tt < qtok ? sm.eac[tt] : 0.0f;
                    yacc[tj] = acc * sc;
                }
            }

            // (c) state advance: S^T = exp(dA) S^T + (B~ w decay)^T X
            const float edA = decay_exp(sm.acum[qtok - 1]);
            const op_t *xr = &sm.Xt[(16 * wave + c) * LDR];
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                f32x4 acc = st[i] * edA;
                const op_t *ar = &sm.Bwt[(16 * i + c) * LDR];
#pragma unroll
                for (int kb = 0; kb < ROWS / KB; ++kb)
                    acc = mma_kblock(ar + kb * KB, xr + kb * KB, acc, g);
                st[i] = acc;
            }

            // running frame angle for the next chunk
            if (rot && wave == 0) {
                for (int i = lane; i < NHr; i += 64) {
                    float base = sm.phi0[i];
                    for (int k = 0; k < PT; ++k)
                        if (k * tb < qtok) base += sm.tot[k * NHr + i];
                    sm.phi0[i] = wrap_angle(base);
                }
            }
        }
        lds_barrier();

        // ================= S4: y += (band o C B^T) X, skip, store
        {
            const op_t *xr = &sm.Xt[(16 * wave + c) * LDR];
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const op_t *mr = &sm.Ms[(16 * tj + c) * LDR];
                // s-rows past the last token of this t-tile are masked to zero
                const int tlast = (16 * tj + 15) / static_cast<int>(R);
                const int send = min(ROWS, (tlast + 1) * static_cast<int>(R));
                const int nkb = (send + KB - 1) / KB;
#pragma unroll
                for (int kb = 0; kb < (ROWS / KB); ++kb)
                    if (kb < nkb) yacc[tj] = mma_kblock(xr + kb * KB, mr + kb * KB, yacc[tj], g);
            }
            T *y = static_cast<T *>(a.y);
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const int rho = 16 * tj + c;
                const int t = rho / static_cast<int>(R);
                const int rr = rho - t * static_cast<int>(R);
                const size_t tau = tau0 + t;
                if (rho < rows_live && tau < L) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int p = 16 * wave + 4 * g + r;
                        if (p < static_cast<int>(P)) {
                            float v = yacc[tj][r];
                            if (a.d_skip) v += dskip * op_to_f32(sm.Xt[p * LDR + rho]);
                            y[(((bb * L + tau) * H + hh) * P + p) * R + rr] = from_f32<T>(v);
                        }
                    }
                }
            }
        }
        if (ck + 1 < nchunks) lds_barrier();
    }

    // ---- boundary state (scan.rs:270-288, 599-638)
    if (a.h_out != nullptr && pcol < static_cast<int>(P)) {
        const size_t sbase = (bb * H + hh) * P * N;
#pragma unroll
        for (int i = 0; i < NTN; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = 16 * i + 4 * g + r;
                if (n < static_cast<int>(N)) a.h_out[sbase + pcol * N + n] = st[i][r];
            }
    }
    if (a.last_u_out != nullptr && L > 0) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T, from the final chunk's LDS tiles.
        const int tl = static_cast<int>((L - 1) - static_cast<size_t>(nchunks - 1) * qtok);
        const size_t sbase = (bb * H + hh) * P * N;
        const int items = static_cast<int>(P * N);
        for (int it = tid; it < items; it += THREADS) {
            const int p = it / static_cast<int>(N);
            const int n = it - p * static_cast<int>(N);
            float acc = 0.0f;
            for (int r = 0; r < static_cast<int>(R); ++r) {
                const int rho = tl * static_cast<int>(R) + r;
                acc += op_to_f32(sm.Xt[p * LDR + rho]) * op_to_f32(sm.Bs[rho * LDN + n]);
            }
            a.last_u_out[sbase + it] = acc;
        }
    }
}

template <typename T, int NP, int PT, int ROWS>
hipError_t launch_cfg(const ScanLaunch &a, hipStream_t s) {
    using Sm = ScanSmem<T, NP, PT, ROWS>;
    const int qtok = static_cast<int>(ROWS / a.rank);
    const int nchunks = static_cast<int>((a.seq + qtok - 1) / qtok);
    const size_t smem = sizeof(Sm);
    auto kern = ssd_scan_kernel<T, NP, PT, ROWS>;
    // opt in to more than 64 KiB of dynamic LDS once per instantiation
    static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(smem));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(a.batch * a.heads), dim3(64 * PT), smem, s, a, qtok, nchunks);
    return hipGetLastError();
}

template <typename T, int NP, int ROWS>
hipError_t launch_np(const ScanLaunch &a, hipStream_t s) {
    // one wave per 16 head_dim columns; waves past head_dim idle on zero tiles
    const size_t pt = (a.head_dim + 15) / 16;
    if (pt <= 1) return launch_cfg<T, NP, 1, ROWS>(a, s);
    if (pt <= 2) return launch_cfg<T, NP, 2, ROWS>(a, s);
    if (pt <= 4) return launch_cfg<T, NP, 4, ROWS>(a, s);
    if (pt <= 8) return launch_cfg<T, NP, 8, ROWS>(a, s);
    return hipErrorInvalidValue;
}

template <typename T, int ROWS_SMALL_N, int ROWS_LARGE_N>
hipError_t launch_t(const ScanLaunch &a, hipStream_t s) {
    const size_t n = a.d_state;
    if (n <= 32) return launch_np<T, 32, ROWS_SMALL_N>(a, s);
    if (n <= 64) return launch_np<T, 64, ROWS_SMALL_N>(a, s);
    if (n <= 128) return launch_np<T, 128, ROWS_SMALL_N>(a, s);
    return launch_np<T, 256, ROWS_LARGE_N>(a, s);
}

}  // namespace

hipError_t launch_scan(const ScanLaunch &a, hipStream_t stream) {
    if (a.batch * a.heads == 0 || a.seq == 0) return hipSuccess;
    if (scan_fast_supported(a)) return launch_scan_fast(a, stream);
    // the generic kernel reads theta in the contiguous layout only
    if (a.theta != nullptr && a.theta_stride != 0) return hipErrorNotSupported;
    if (a.bf16) return launch_t<bf16_t, 64, 32>(a, stream);
    return launch_t<float, 32, 16>(a, stream);
}

}  // namespace m3
