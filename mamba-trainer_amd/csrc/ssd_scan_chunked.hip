// Chunked SSD scan for gfx950 as three chunk-parallel launches over a caller
// workspace.  Same shapes as ssd_scan_fast.hip (head_dim 64, d_state 64/128,
// rank 1/2/4, aligned operands) and the same algorithm, src/ssm/scan.rs:116-291
// (ssd_chunked) and 458-638 (mamba3_scan), regrouped so that only an
// elementwise recurrence runs in sequence:
//
//   chunk_state_kernel  one workgroup per (batch, head, chunk).  In the chunk's
//       own rotating frame (angles relative to the chunk start, so nothing from
//       earlier chunks is needed) it forms U_k = sum_s (B_s w_s decay_s)^T x_s,
//       the chunk's contribution to the state (scan.rs:207-251), together with
//       the chunk decay exp(sum dt A) and, per rotation pair, the chunk's angle
//       total Phi_k with its cosine and sine.
//   state_pass_kernel   one thread per (batch, head, p, four state pairs):
//       S_0 = R(angle0) h0 and S_{k+1} = R(Phi_k) (decay_k S_k + U_k), the state
//       entering each chunk expressed in that chunk's frame, written as MFMA
//       operand fragments; at the end the boundary state in the global frame
//       (scan.rs:270-288, 599-638).
//   chunk_scan_kernel   one workgroup per (batch, head, chunk):
//       y = (C~ B~^T o L) X + exp(acum) C~ S_k  (ssd_band fused.rs:2044-2070,
//       scan.rs:253-263), the skip D on the band's diagonal (scan.rs:593-597).
//
// Frames.  With phi_t the running angle and phi^s_k its value entering chunk k,
// B~_t = R(-phi_t) B_t = R(-phi^s_k) B^(k)_t where B^(k)_t is B_t rotated by the
// in-chunk angle only.  The state in chunk k's frame is S = R(phi^s_k) h, so
// C~_t . h = C^(k)_t . S, and moving to the next frame is a rotation of every
// (n, n + N/2) pair by the chunk total Phi_k.
//
// Why three launches: a batch x head count of ~100 sequences fills under half
// of the chip's 256 CUs when each sequence is walked by one workgroup, and
// every chunk's rotation (a sine and cosine per token and pair), decay weights
// and band are latency-bound there.  Here both heavy passes spread over every
// chunk of every sequence; the sequential pass is a few FMAs per element and
// streams U_k from HBM.
#include <type_traits>

#include "scan_common.hpp"

namespace m3 {

namespace {

using namespace scan;

constexpr int kP = 64;   // head_dim of these kernels

// Workspace sections, byte offsets from the base.  U and S are stored in the
// operand type: bf16 for bf16 storage (the state itself is carried in f32 by
// the state pass), f32 otherwise.
struct ChunkedLayout {
    size_t u, s, eda, phi, cph, sph, total;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

ChunkedLayout chunked_layout(size_t bhk, size_t n, bool bf16) {
    ChunkedLayout l;
    size_t o = 0;
    l.u = o;
    o = align256(o + bhk * kP * n * (bf16 ? 2 : 4));
    l.s = o;
    o = align256(o + bhk * kP * n * (bf16 ? 2 : 4));
    l.eda = o;
    o = align256(o + bhk * 4);
    l.phi = o;
    o = align256(o + bhk * (n / 2) * 4);
    l.cph = o;
    o = align256(o + bhk * (n / 2) * 4);
    l.sph = o;
    o = align256(o + bhk * (n / 2) * 4);
    l.total = o;
    return l;
}

struct ChunkWs {
    void *u;        // [bhk][p-tile][n-tile][lane][4]: U^T tiles in MFMA D layout
    void *s;        // as u: S^T tiles of the state entering each chunk
    float *eda;     // [bhk] exp(clamp(sum of dt A over the chunk))
    float *phi;     // [bhk][N/2] angle total of the chunk per pair
    float *cph;     // [bhk][N/2] cos Phi
    float *sph;     // [bhk][N/2] sin Phi
};

ChunkWs chunk_ws(char *base, const ChunkedLayout &l) {
    ChunkWs w;
    w.u = base + l.u;
    w.s = base + l.s;
    w.eda = reinterpret_cast<float *>(base + l.eda);
    w.phi = reinterpret_cast<float *>(base + l.phi);
    w.cph = reinterpret_cast<float *>(base + l.cph);
    w.sph = reinterpret_cast<float *>(base + l.sph);
    return w;
}

// Four consecutive values of U (element index e, a multiple of four).
template <bool BF>
__device__ __forceinline__ void store_u(void *u, size_t e, const f32x4 v) {
    if constexpr (BF) {
        bf16x4 q;
#pragma unroll
        for (int r = 0; r < 4; ++r) q[r] = to_bf16(v[r]);
        *reinterpret_cast<bf16x4 *>(static_cast<__bf16 *>(u) + e) = q;
    } else {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(u) + e) = v;
    }
}
template <bool BF>
__device__ __forceinline__ f32x4 load_u(const void *u, size_t e) {
    if constexpr (BF) {
        const bf16x4 q = *reinterpret_cast<const bf16x4 *>(static_cast<const __bf16 *>(u) + e);
        return f32x4{static_cast<float>(q[0]), static_cast<float>(q[1]), static_cast<float>(q[2]),
                     static_cast<float>(q[3])};
    } else {
        return *reinterpret_cast<const f32x4 *>(static_cast<const float *>(u) + e);
    }
}

// ================================================================ chunk state
template <typename T, int N, int R, int ROWS>
struct StateSmem {
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDR = ROWS + PAD;
    op_t Bwt[N * LDR];      // (B^(k) * w * decay-to-end)^T [n][rho]
    op_t Xt[kP * LDR];      // X^T [p][rho]
    float phi_tot[N / 2];   // the sub-chunk's angle total per pair
    float phi_acc[N / 2];   // the chunk's so far
};

// A chunk here is HALF sub-chunks of ROWS rows (the MIMO ranks take HALF = R,
// so that a chunk spans ROWS tokens whatever the rank), staged one after the
// other.  With U_h, e_h, Phi_h those of sub-chunk h in its own frame, the
// chunk's are accumulated as U = e_h U + R(-Phi) U_h, e = e e_h,
// Phi = Phi + Phi_h: the state recurrence S' = R(Phi)(e S + U) composed over
// the sub-chunks (the per-pair rotations commute).
template <typename T, int N, int R, int ROWS, int HALF>
__global__ void __launch_bounds__(kThreads, 2)
chunk_state_kernel(ScanLaunch a, ChunkWs ws, int nck) {
    constexpr int P = kP;
    using G = Geo<T, N, P, R, ROWS, 4>;
    using S = StateSmem<T, N, R, ROWS>;
    using RawT = Raw<T, N, P, R, ROWS, 4, false>;
    using op_t = typename S::op_t;
    constexpr int KB = sizeof(typename S::op_t) == 2 ? 32 : 16;
    constexpr int LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL;
    constexpr int NTN = N / 16;
    constexpr bool kBf16 = sizeof(op_t) == 2;

    __shared__ S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t bhk = blockIdx.x;
    const int ck = static_cast<int>(bhk % nck);
    const size_t bh = bhk / nck;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)

    // U^T[n][p] of this wave's p-tile, accumulated over the sub-chunks
    f32x4 uacc[NTN];
    float eacc = 1.0f;
#pragma unroll 1
    for (int h = 0; h < HALF; ++h) {
        const int sck = ck * HALF + h;
        RawT cur;
        load_chunk<T, N, P, R, ROWS, 4, false>(rs, sck, wave, lane, cur);

        const size_t tau = static_cast<size_t>(sck) * QT + my_t;
        const bool live = tok_lane && tau < L;
        float av, gv, wv;
        token_scalars(a, cur, A, live, av, gv, wv);
        const float acum = seg_scan<G::SW>(av);
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        const float wd = dexp<kBf16>(last - acum) * wv;   // exp_decay(last, acum, w)
        const float eh = dexp<kBf16>(last);

        // in-chunk angle (inclusive cumsum of dt * theta), rotation by its negative
        float cs[PPL], sn[PPL];
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            cs[j] = 1.0f;
            sn[j] = 0.0f;
        }
        if (rot) {
            const float dtt = live ? cur.s0 : 0.0f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const float pre = seg_scan<G::SW>(dtt * welem<T>(cur.th, j));
                if (my_t == QT - 1) sm.phi_tot[i0 + j] = pre;
                const float psi = wrap_angle(pre);
                if constexpr (kBf16) {
                    // the hardware sine takes revolutions; |psi| <= pi
                    const float rev = psi * 0.15915494309189533577f;
                    sn[j] = __builtin_amdgcn_sinf(rev);
                    cs[j] = __builtin_amdgcn_cosf(rev);
                } else {
                    sincosf(psi, &sn[j], &cs[j]);
                }
            }
        }
        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / 4) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                sm.Xt[p * LDR + my_t * R + r] = to_op<op_t>(elem<T>(cur.x, e));
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = my_t * R + r;
#pragma unroll
                for (int j = 0; j < PPL; ++j) {
                    const float b1 = elem<T>(cur.b[0], j * R + r);
                    const float b2 = elem<T>(cur.b[1], j * R + r);
                    const float w1 = (b1 * cs[j] + b2 * sn[j]) * wd;    // fused.rs:610-617
                    const float w2 = (-b1 * sn[j] + b2 * cs[j]) * wd;
                    sm.Bwt[(i0 + j) * LDR + rho] = to_op<op_t>(w1);
                    sm.Bwt[(i0 + NH + j) * LDR + rho] = to_op<op_t>(w2);
                }
            }
        }
        __syncthreads();

        if constexpr (HALF == 1) {
            // the chunk's angle total per pair, with its cosine and sine
            if (tid < NH) {
                const float tot = rot ? sm.phi_tot[tid] : 0.0f;
                float ts = 0.0f, tc = 1.0f;
                if (rot) sincosf(tot, &ts, &tc);
                ws.phi[bhk * NH + tid] = tot;
                ws.cph[bhk * NH + tid] = tc;
                ws.sph[bhk * NH + tid] = ts;
            }
            if (tid == 0) ws.eda[bhk] = eh;
        }
        // U_h^T[n][p] = sum_rho Bwt[n][rho] X^T[p][rho]; wave w takes p-tile w
        const op_t *xr = &sm.Xt[(16 * wave + c) * LDR];
        const size_t uo = (bhk * 4 + wave) * NTN * 256 + lane * 4;
        f32x4 uh[NTN];
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const op_t *ar = &sm.Bwt[(16 * i + c) * LDR];
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb) acc = mma_kb(ar + kb * KB, xr + kb * KB, acc, g);
            if constexpr (HALF == 1) store_u<kBf16>(ws.u, uo + i * 256, acc);
            uh[i] = acc;
        }
        if constexpr (HALF > 1) {
            if (h == 0) {
#pragma unroll
                for (int i = 0; i < NTN; ++i) uacc[i] = uh[i];
            } else {
                // U = e_h U + R(-Phi) U_h over the pairs (n, n + N/2): tiles i, i + NTN/2
#pragma unroll
                for (int i = 0; i < NTN / 2; ++i) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float ps = 0.0f, pc = 1.0f;
                        if (rot) sincosf(sm.phi_acc[16 * i + 4 * g + r], &ps, &pc);
                        const float lo = uh[i][r], hi = uh[i + NTN / 2][r];
                        uacc[i][r] = eh * uacc[i][r] + lo * pc + hi * ps;
                        uacc[i + NTN / 2][r] = eh * uacc[i + NTN / 2][r] - lo * ps + hi * pc;
                    }
                }
            }
            eacc *= eh;
            __syncthreads();   // every read of this sub-chunk's LDS is done
            if (tid < NH)
                sm.phi_acc[tid] = (h == 0 ? 0.0f : sm.phi_acc[tid]) + (rot ? sm.phi_tot[tid] : 0.0f);
            __syncthreads();
        }
    }

    if constexpr (HALF > 1) {
        const size_t uo = (bhk * 4 + wave) * NTN * 256 + lane * 4;
#pragma unroll
        for (int i = 0; i < NTN; ++i) store_u<kBf16>(ws.u, uo + i * 256, uacc[i]);
        if (tid == 0) ws.eda[bhk] = eacc;
        // the chunk's angle total per pair, with its cosine and sine
        if (tid < NH) {
            const float tot = sm.phi_acc[tid];
            float ts = 0.0f, tc = 1.0f;
            if (rot) sincosf(tot, &ts, &tc);
            ws.phi[bhk * NH + tid] = tot;
            ws.cph[bhk * NH + tid] = tc;
            ws.sph[bhk * NH + tid] = ts;
        }
    }
}

// ================================================================ state pass
__device__ __forceinline__ void sincos4(const f32x4 t, f32x4 &sn, f32x4 &cs) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float s, c;
        sincosf(t[r], &s, &c);
        sn[r] = s;
        cs[r] = c;
    }
}

// v1 = element n, v2 = element n + N/2 of a pair; R(t) (v1, v2) =
// (v1 cos t - v2 sin t, v1 sin t + v2 cos t)
__device__ __forceinline__ void rotate_pairs(f32x4 &lo, f32x4 &hi, const f32x4 cs, const f32x4 sn) {
    const f32x4 l = lo;
    lo = l * cs - hi * sn;
    hi = l * sn + hi * cs;
}

template <typename T, int N>
__global__ void __launch_bounds__(kThreads)
state_pass_kernel(ScanLaunch a, ChunkWs ws, int nck) {
    constexpr int P = kP;
    constexpr int NTN = N / 16;
    constexpr int HT = NTN / 2;   // n-tiles per half
    constexpr int NH = N / 2;
    constexpr bool kBf16 = sizeof(T) == 2;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int pt = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;
    const size_t H = a.heads, L = a.seq;
    const int i1 = static_cast<int>(blockIdx.x % HT);
    const size_t bh = blockIdx.x / HT;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int p = 16 * pt + c;
    const int nlo = 16 * i1 + 4 * g;   // my pairs are (nlo + r, nlo + r + N/2), r < 4
    const size_t sbase = bh * P * N + static_cast<size_t>(p) * N;

    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    {
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        if (h0 != nullptr) {
            lo = *reinterpret_cast<const f32x4 *>(h0 + sbase + nlo);
            hi = *reinterpret_cast<const f32x4 *>(h0 + sbase + nlo + NH);
            if (l0 != nullptr) {
                // carry S = h + (1 - lambda_0) dt_0 last_u   (scan.rs:521-535)
                const size_t i0s = (bb * L) * H + hh;
                const float first = (1.0f - a.lambda[i0s]) * a.dt[i0s];
                lo += *reinterpret_cast<const f32x4 *>(l0 + sbase + nlo) * first;
                hi += *reinterpret_cast<const f32x4 *>(l0 + sbase + nlo + NH) * first;
            }
        }
    }
    // running wrapped angle of my pairs; the carried state into chunk 0's frame
    f32x4 phi = {0.f, 0.f, 0.f, 0.f};
    if (rot && a.angle0 != nullptr) {
        phi = *reinterpret_cast<const f32x4 *>(a.angle0 + bh * NH + nlo);
        f32x4 cs, sn;
        sincos4(phi, sn, cs);
        rotate_pairs(lo, hi, cs, sn);
    }

    const size_t bhk0 = bh * nck;
    struct In {
        f32x4 ulo, uhi, cs, sn, ph;
        float e;
    };
    auto load = [&](int k, In &d) {
        const int kk = k < nck ? k : nck - 1;   // past the end: re-read the last chunk, unused
        const size_t bhk = bhk0 + kk;
        const size_t u = (bhk * 4 + pt) * NTN * 256 + lane * 4;
        d.ulo = load_u<kBf16>(ws.u, u + i1 * 256);
        d.uhi = load_u<kBf16>(ws.u, u + (i1 + HT) * 256);
        d.e = ws.eda[bhk];
        if (rot) {
            d.cs = *reinterpret_cast<const f32x4 *>(ws.cph + bhk * NH + nlo);
            d.sn = *reinterpret_cast<const f32x4 *>(ws.sph + bhk * NH + nlo);
            d.ph = *reinterpret_cast<const f32x4 *>(ws.phi + bhk * NH + nlo);
        }
    };
    auto step = [&](int k, const In &d) {
        const size_t so = ((bhk0 + k) * 4 + pt) * NTN * 256 + lane * 4;
        store_u<kBf16>(ws.s, so + i1 * 256, lo);
        store_u<kBf16>(ws.s, so + (i1 + HT) * 256, hi);
        lo = lo * d.e + d.ulo;
        hi = hi * d.e + d.uhi;
        if (rot) {
            rotate_pairs(lo, hi, d.cs, d.sn);
#pragma unroll
            for (int r = 0; r < 4; ++r) phi[r] = wrap_angle(phi[r] + d.ph[r]);
        }
    };
    // eight chunks in flight ahead of the one being applied
    constexpr int D = 8;
    In d[D];
#pragma unroll
    for (int j = 0; j < D; ++j) load(j, d[j]);
    for (int k = 0; k < nck; k += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (k + j < nck) step(k + j, d[j]);
            load(k + D + j, d[j]);
        }
    }

    // ---- boundary state in the global frame (scan.rs:270-288, 599-638)
    f32x4 ce = {1.f, 1.f, 1.f, 1.f}, se = {0.f, 0.f, 0.f, 0.f};
    if (rot) sincos4(phi, se, ce);
    if (a.h_out != nullptr) {
        f32x4 hl = lo, hh2 = hi;
        rotate_pairs(hl, hh2, ce, -se);   // R(-phi_end)
        *reinterpret_cast<f32x4 *>(a.h_out + sbase + nlo) = hl;
        *reinterpret_cast<f32x4 *>(a.h_out + sbase + nlo + NH) = hh2;
    }
    if (a.angle_out != nullptr && pt == 0 && c == 0)
        *reinterpret_cast<f32x4 *>(a.angle_out + bh * NH + nlo) = phi;
    if (a.last_u_out != nullptr) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T with B~ = R(-phi_end) B  (scan.rs:599-618)
        const size_t tl = (bb * L + (L - 1)) * H + hh;
        const T *bp = static_cast<const T *>(a.b) + tl * N * a.rank;
        const T *xp = static_cast<const T *>(a.x) + (tl * P + static_cast<size_t>(p)) * a.rank;
        f32x4 ul = {0.f, 0.f, 0.f, 0.f}, uh = ul;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            if (m >= static_cast<int>(a.rank)) break;
            const float xv = to_f32(xp[m]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float b1 = to_f32(bp[(nlo + r) * a.rank + m]);
                const float b2 = to_f32(bp[(nlo + r + NH) * a.rank + m]);
                ul[r] += xv * (b1 * ce[r] + b2 * se[r]);
                uh[r] += xv * (-b1 * se[r] + b2 * ce[r]);
            }
        }
        *reinterpret_cast<f32x4 *>(a.last_u_out + sbase + nlo) = ul;
        *reinterpret_cast<f32x4 *>(a.last_u_out + sbase + nlo + NH) = uh;
    }
}

// ================================================================ chunk scan
template <typename T, int N, int R, int ROWS, int HALF>
struct ScanSmem {
    using G = Geo<T, N, kP, R, ROWS, 4>;
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;
    static constexpr int LDR = ROWS + PAD;
    op_t Bs[ROWS * LDN];    // B^(k)[rho][npos(n)]
    op_t Cs[ROWS * LDN];    // C^(k)[rho][npos(n)]
    op_t Xt[kP * LDR];      // X^T [p][rho]
    op_t Ms[ROWS * LDR];    // masked band (C B^T o L)[rho_t][rho_s]
    float acum[G::QT], gw[G::QT], ww[G::QT], eac[G::QT];
    // with sub-chunks: the sub-chunk's angle total per pair, w x decay to its end per token
    float phi_tot[HALF > 1 ? N / 2 : 1];
    float wdv[HALF > 1 ? G::QT : 1];
};

// HALF sub-chunks of ROWS rows per chunk, one after the other: between them
// the state advances in registers, S' = R(Phi_h)(e_h S + U_h), with U_h formed
// from the sub-chunk's staged B~ and X^T.
template <typename T, int N, int R, int ROWS, int HALF>
__global__ void __launch_bounds__(kThreads, HALF > 1 ? 2 : 3)
chunk_scan_kernel(ScanLaunch a, ChunkWs ws, int nck) {
    constexpr int P = kP;
    using G = Geo<T, N, P, R, ROWS, 4>;
    using S = ScanSmem<T, N, R, ROWS, HALF>;
    using RawT = Raw<T, N, P, R, ROWS, 4, true>;
    using op_t = typename S::op_t;
    constexpr int KB = Op<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL;
    constexpr int NT = ROWS / 16;
    constexpr int NTN = N / 16;
    constexpr bool kBf16 = sizeof(op_t) == 2;
    constexpr uint32_t SZ = sizeof(T);

    __shared__ S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t bhk = blockIdx.x;
    const int ck = static_cast<int>(bhk % nck);
    const size_t bh = bhk / nck;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;
    const int pcol = 16 * wave + c;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);
    // The (first sub-)chunk's inputs go first: the stage waits for them while
    // the state fragments below are still in flight.  bf16 sub-chunks then load
    // the next sub-chunk's inputs behind the current one's work (f32 lacks the
    // registers for it).
    constexpr bool kPrefetch = HALF > 1 && sizeof(T) == 2;
    RawT cur, nxt;
    if constexpr (HALF == 1 || kPrefetch)
        load_chunk<T, N, P, R, ROWS, 4, true>(rs, ck * HALF, wave, lane, HALF == 1 ? cur : nxt);

    // the state entering this chunk, in its frame, as carry-in A operands
    // (bf16: n-tiles 2kb and 2kb + 1 form k-block kb, matching npos)
    using frag_t = typename std::conditional<kBf16, bf16x8, f32x4>::type;
    constexpr int NF = kBf16 ? N / 32 : NTN;
    frag_t sf[NF];
    if constexpr (kBf16) {
        const bf16x4 *src = static_cast<const bf16x4 *>(ws.s) + (bhk * 4 + wave) * NTN * 64 + lane;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const bf16x4 lo = src[(2 * f) * 64], hi = src[(2 * f + 1) * 64];
            sf[f] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    } else {
        const f32x4 *src = static_cast<const f32x4 *>(ws.s) + (bhk * 4 + wave) * NTN * 64 + lane;
#pragma unroll
        for (int f = 0; f < NF; ++f) sf[f] = src[f * 64];
    }

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const bool skip = a.d_skip != nullptr;

#pragma unroll 1
    for (int h = 0; h < HALF; ++h) {
    const int sck = ck * HALF + h;
    if constexpr (kPrefetch) {
        cur = nxt;
        if (h + 1 < HALF) load_chunk<T, N, P, R, ROWS, 4, true>(rs, sck + 1, wave, lane, nxt);
    } else if constexpr (HALF > 1) {
        load_chunk<T, N, P, R, ROWS, 4, true>(rs, sck, wave, lane, cur);
    }
    // ---- stage: per-token scalars, in-chunk angles, rotated B and C, X^T
    {
        const size_t tau = static_cast<size_t>(sck) * QT + my_t;
        const bool live = tok_lane && tau < L;
        float av, gv, wv;
        token_scalars(a, cur, A, live, av, gv, wv);
        const float acum = seg_scan<G::SW>(av);
        if (wave == 0 && sub == 0 && tok_lane) {
            sm.acum[my_t] = acum;
            sm.gw[my_t] = gv;
            sm.ww[my_t] = wv;
            sm.eac[my_t] = dexp<kBf16>(acum);             // exp_decay(acum)
            if (HALF > 1) {
                const float last = __int_as_float(
                    __builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
                sm.wdv[my_t] = dexp<kBf16>(last - acum) * wv;   // w x decay to the end
            }
        }
        float cs[PPL], sn[PPL];
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            cs[j] = 1.0f;
            sn[j] = 0.0f;
        }
        if (rot) {
            const float dtt = live ? cur.s0 : 0.0f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const float pre = seg_scan<G::SW>(dtt * welem<T>(cur.th, j));
                if (HALF > 1 && my_t == QT - 1) sm.phi_tot[i0 + j] = pre;
                const float psi = wrap_angle(pre);
                if constexpr (kBf16) {
                    const float rev = psi * 0.15915494309189533577f;
                    sn[j] = __builtin_amdgcn_sinf(rev);
                    cs[j] = __builtin_amdgcn_cosf(rev);
                } else {
                    sincosf(psi, &sn[j], &cs[j]);
                }
            }
        }
        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / 4) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                sm.Xt[p * LDR + my_t * R + r] = to_op<op_t>(elem<T>(cur.x, e));
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = my_t * R + r;
                float rb[2][PPL], rc[2][PPL];
#pragma unroll
                for (int j = 0; j < PPL; ++j) {
                    const float b1 = elem<T>(cur.b[0], j * R + r);
                    const float b2 = elem<T>(cur.b[1], j * R + r);
                    const float c1 = elem<T>(cur.c[0], j * R + r);
                    const float c2 = elem<T>(cur.c[1], j * R + r);
                    rb[0][j] = b1 * cs[j] + b2 * sn[j];
                    rb[1][j] = -b1 * sn[j] + b2 * cs[j];
                    rc[0][j] = c1 * cs[j] + c2 * sn[j];
                    rc[1][j] = -c1 * sn[j] + c2 * cs[j];
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if constexpr (PPL % 4 == 0) {
#pragma unroll
                        for (int q = 0; q < PPL; q += 4) {
                            const int n = i0 + h * NH + q;
                            st4(&sm.Bs[rho * LDN + npos<kBf16>(n)], &rb[h][q]);
                            st4(&sm.Cs[rho * LDN + npos<kBf16>(n)], &rc[h][q]);
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < PPL; ++j) {
                            const int n = i0 + h * NH + j;
                            sm.Bs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rb[h][j]);
                            sm.Cs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rc[h][j]);
                        }
                    }
                }
            }
        }
    }
    lds_barrier();

    // ---- masked band into Ms; tiles above the band that the y product
    //      still reads (k-blocks wider than a tile) are zeroed
    {
        int idx = 0;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            const int tlast = (16 * tj + 15) / R;
            const int send = (tlast + 1) * R < ROWS ? (tlast + 1) * R : ROWS;
            const int ncol = ((send + KB - 1) / KB) * KB;
#pragma unroll
            for (int si = 0; si < NT; ++si) {
                if (16 * si >= ncol) continue;
                if ((idx++) % 4 != wave) continue;
                const int trow = 16 * tj + c;
                float vals[4] = {0.f, 0.f, 0.f, 0.f};
                if ((16 * si) / R <= tlast) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *ar = &sm.Bs[(16 * si + c) * LDN];
                    const op_t *br = &sm.Cs[trow * LDN];
#pragma unroll
                    for (int kb = 0; kb < N / KB; ++kb)
                        acc = mma_kb(ar + kb * KB, br + kb * KB, acc, g);
                    const int tt = trow / R;
                    const float at = sm.acum[tt];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int srow = 16 * si + 4 * g + r;
                        const int ts = srow / R;
                        float v = 0.0f;
                        if (ts <= tt) {
                            const float wgt = (ts == tt) ? sm.gw[ts] : sm.ww[ts];
                            v = acc[r] * wgt * dexp<kBf16>(at - sm.acum[ts]);
                        }
                        if (skip && srow == trow) v += dskip;   // scan.rs:593-597
                        vals[r] = v;
                    }
                }
                st4(&sm.Ms[trow * LDR + 16 * si + 4 * g], vals);
            }
        }
    }
    lds_barrier();

    // ---- y^T[p][t] = exp(acum_t) sum_n S[p][n] C[t][n] + sum_s X^T[p][s] M[t][s]
    const op_t *xr = &sm.Xt[pcol * LDR];
    const uint32_t tau0 = static_cast<uint32_t>(sck) * QT;
#pragma unroll
    for (int tj = 0; tj < NT; ++tj) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const op_t *cr = &sm.Cs[(16 * tj + c) * LDN];
        if constexpr (kBf16) {
#pragma unroll
            for (int kb = 0; kb < N / 32; ++kb)
                acc = mfma_bf16(sf[kb], *reinterpret_cast<const bf16x8 *>(cr + 32 * kb + 8 * g), acc);
        } else {
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                const f32x4 bv = *reinterpret_cast<const f32x4 *>(cr + 16 * i + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc = mfma_f32(sf[i][r], bv[r], acc);
            }
        }
        acc = acc * sm.eac[(16 * tj + c) / R];
        const op_t *mr = &sm.Ms[(16 * tj + c) * LDR];
        const int tlast = (16 * tj + 15) / R;
        const int send = (tlast + 1) * R < ROWS ? (tlast + 1) * R : ROWS;
        const int nkb = (send + KB - 1) / KB;
#pragma unroll
        for (int kb = 0; kb < ROWS / KB; ++kb)
            if (kb < nkb) acc = mma_kb(xr + kb * KB, mr + kb * KB, acc, g);

        const int rho = 16 * tj + c;
        const int rr = rho % R;
        const uint32_t tau = tau0 + rho / R;
        // rows past the sequence end fall outside the buffer: dropped
        const uint32_t oy = tau * rs.tok_x + ((16 * wave + 4 * g) * R + rr) * SZ;
        if constexpr (R == 1) {
            if constexpr (kBf16) {
                u32x2 pk;
                pk[0] = static_cast<unsigned int>(from_f32<bf16_t>(acc[0]).bits) |
                        (static_cast<unsigned int>(from_f32<bf16_t>(acc[1]).bits) << 16);
                pk[1] = static_cast<unsigned int>(from_f32<bf16_t>(acc[2]).bits) |
                        (static_cast<unsigned int>(from_f32<bf16_t>(acc[3]).bits) << 16);
                bst8(pk, rs.y, oy);
            } else {
                bst16(u32x4{__float_as_uint(acc[0]), __float_as_uint(acc[1]),
                            __float_as_uint(acc[2]), __float_as_uint(acc[3])},
                      rs.y, oy);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kBf16)
                    bst2(from_f32<bf16_t>(acc[r]).bits, rs.y, oy + r * R * SZ);
                else
                    bst4(__float_as_uint(acc[r]), rs.y, oy + r * R * SZ);
            }
        }
    }

    if (h + 1 < HALF) {
        // ---- the state entering the next sub-chunk: S' = R(Phi_h)(e_h S + U_h),
        // U_h^T[n][p] = sum_rho (B~ w decay-to-end)[rho][n] X^T[p][rho] over
        // this wave's p-tile; the D tiles of U line up with the S fragments
        const float eh = dexp<kBf16>(sm.acum[QT - 1]);
        f32x4 uh[NTN];
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const int n = 16 * i + c;
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb) {
                if constexpr (kBf16) {
                    bf16x8 av;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int rho = 32 * kb + 8 * g + j;
                        av[j] = static_cast<__bf16>(
                            static_cast<float>(sm.Bs[rho * LDN + npos<kBf16>(n)]) * sm.wdv[rho / R]);
                    }
                    acc = mfma_bf16(av, *reinterpret_cast<const bf16x8 *>(xr + 32 * kb + 8 * g), acc);
                } else {
                    const f32x4 bv = *reinterpret_cast<const f32x4 *>(xr + 16 * kb + 4 * g);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int rho = 16 * kb + 4 * g + j;
                        acc = mfma_f32(static_cast<float>(sm.Bs[rho * LDN + n]) * sm.wdv[rho / R],
                                       bv[j], acc);
                    }
                }
            }
            uh[i] = acc;
        }
        // S (this lane: p = 16 wave + c, n = 16 i + 4 g + r) in f32, advanced and rotated
        f32x4 st[NTN];
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            if constexpr (kBf16) {
                const bf16x8 f = sf[i / 2];
#pragma unroll
                for (int r = 0; r < 4; ++r) st[i][r] = static_cast<float>(f[(i & 1) * 4 + r]);
            } else {
                st[i] = sf[i];
            }
            st[i] = st[i] * eh + uh[i];
        }
        if (rot) {
#pragma unroll
            for (int i = 0; i < NTN / 2; ++i) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float ps, pc;
                    sincosf(sm.phi_tot[16 * i + 4 * g + r], &ps, &pc);
                    const float lo = st[i][r], hi = st[i + NTN / 2][r];
                    st[i][r] = lo * pc - hi * ps;                  // R(Phi_h)
                    st[i + NTN / 2][r] = lo * ps + hi * pc;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            if constexpr (kBf16) {
#pragma unroll
                for (int r = 0; r < 4; ++r) sf[i / 2][(i & 1) * 4 + r] = static_cast<__bf16>(st[i][r]);
            } else {
                sf[i] = st[i];
            }
        }
        lds_barrier();   // the next sub-chunk's staging reuses the LDS
    }
    }   // sub-chunks
}

// Sub-chunks per chunk of the three launches: one per rank, so that a chunk
// spans ROWS tokens whatever the rank and the U / S records and the state
// pass stay per ROWS tokens (the MIMO ranks would otherwise multiply them).
constexpr int half_for(int r) { return r; }

size_t chunk_count(const ScanLaunch &a, int rows) {
    const size_t qt = static_cast<size_t>(rows) / a.rank;
    const size_t nsub = (a.seq + qt - 1) / qt;
    const size_t half = static_cast<size_t>(half_for(static_cast<int>(a.rank)));
    return (nsub + half - 1) / half;
}

template <typename T, int N, int R, int ROWS>
hipError_t launch_three(const ScanLaunch &a, char *base, hipStream_t s) {
    constexpr int HALF = half_for(R);
    const int nck = static_cast<int>(chunk_count(a, ROWS));
    const size_t bh = a.batch * a.heads;
    const size_t bhk = bh * nck;
    const ChunkWs ws = chunk_ws(base, chunked_layout(bhk, N, sizeof(T) == 2));
    hipLaunchKernelGGL((chunk_state_kernel<T, N, R, ROWS, HALF>), dim3(bhk), dim3(kThreads), 0, s,
                       a, ws, nck);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((state_pass_kernel<T, N>), dim3(bh * (N / 32)), dim3(kThreads), 0, s, a, ws,
                       nck);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_scan_kernel<T, N, R, ROWS, HALF>), dim3(bhk), dim3(kThreads), 0, s,
                       a, ws, nck);
    return hipGetLastError();
}

template <typename T, int ROWS>
hipError_t launch_t(const ScanLaunch &a, char *ws, hipStream_t s) {
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_three<T, 128, 1, ROWS>(a, ws, s);
        if (r == 2) return launch_three<T, 128, 2, ROWS>(a, ws, s);
        if (r == 4) return launch_three<T, 128, 4, ROWS>(a, ws, s);
    } else if (n == 64) {
        if (r == 1) return launch_three<T, 64, 1, ROWS>(a, ws, s);
        if (r == 2) return launch_three<T, 64, 2, ROWS>(a, ws, s);
        if (r == 4) return launch_three<T, 64, 4, ROWS>(a, ws, s);
    }
    return hipErrorNotSupported;
}

int rows_for(const ScanLaunch &a) { return a.bf16 ? 64 : 32; }

}  // namespace

// The single pass walks each (batch, head) sequence with one workgroup per CU,
// so its time goes in whole rounds of one sequence per CU; the three
// chunk-parallel launches cost about the same per sequence at any count.  The
// single pass is the faster form once the last round fills ~70 % of the chip
// (measured on MI355X at L = 2048, H = 12, N = 128, bf16, in us chunked vs
// single pass: 96 sequences 107 vs 191, 192: 239 vs 222, 240: 299 vs 227,
// 288: 367 vs 434, 384: 482 vs 442).  The workspace is asked for only where
// the chunked form wins.
static size_t device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return static_cast<size_t>(cus);
}

size_t scan_chunked_workspace(const ScanLaunch &a) {
    if (!scan_fast_supported(a) || a.seq == 0) return 0;
    const size_t seqs = a.batch * a.heads, cus = device_cus();
    const size_t rounds = (seqs + cus - 1) / cus;
    if (seqs * 10 >= rounds * cus * 7) return 0;
    return chunked_layout(a.batch * a.heads * chunk_count(a, rows_for(a)), a.d_state, a.bf16 != 0)
        .total;
}

hipError_t launch_scan_chunked(const ScanLaunch &a, void *workspace, hipStream_t stream) {
    if (!scan_fast_supported(a) || a.seq == 0) return hipErrorNotSupported;
    char *ws = static_cast<char *>(workspace);
    if (a.bf16) return launch_t<bf16_t, 64>(a, ws, stream);
    return launch_t<float, 32>(a, ws, stream);
}

}  // namespace m3
