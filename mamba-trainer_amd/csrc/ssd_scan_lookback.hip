// Chunked SSD scan for gfx950 in one launch, with a decoupled look-back for
// the state recurrence.  Shapes as the chunk-parallel kernels: bf16 storage,
// head_dim 64, d_state 64/128, rank 1/2/4, aligned operands.  It restates
// src/ssm/scan.rs:116-291 (ssd_chunked) and 458-638 (mamba3_scan).
//
// One workgroup per (batch, head, chunk).  Workgroups take a ticket from a
// counter as they start; ticket t is chunk t / S of sequence t % S (S =
// batch x heads), so every workgroup a ticket holder waits for holds a smaller
// ticket and is already running: the waits always end.
//
// Per chunk k of a sequence:
//   stage    lane = token: the log-decay prefix and the in-chunk angle prefix
//            (DPP scans), trapezoid weights (fused.rs:2483-2503), B and C
//            rotated by the in-chunk angle (fused.rs:588-619) into LDS as
//            B~^T [n][row] and C~ [row][n], X^T [p][row].
//   local    MFMA: U_k^T = B~^T diag(w decay-to-end) X, the chunk's share of
//            the state (scan.rs:207-216), and the masked band
//            (C~ B~^T o L) with the skip D on its diagonal (fused.rs:2044-2070,
//            scan.rs:593-597).
//   record   A chunk whose predecessor has not yet published its prefix
//            publishes its aggregate A_k = (U_k, decay e_k, angle total
//            Phi_k); the map it stands for is T_k(S) = R(Phi_k)(e_k S + U_k).
//   look-back  Walking back from chunk k-1, aggregates are folded into one
//            map G(S) = R(Theta)(E S) + V until a chunk whose prefix S_{j+1}
//            (the state entering chunk j+1, in that chunk's frame) is
//            published: S_k = G(S_{j+1}).  Chunk 0 starts from the carried-in
//            state (scan.rs:521-535).
//   prefix   S_{k+1} = T_k(S_k) and the wrapped global angle entering chunk
//            k+1 are published (not by the last chunk, which instead writes
//            the boundary state h, last_u and angle, scan.rs:270-288, 599-638).
//   output   y = band X + exp(acum) C~ S_k (scan.rs:253-263).
//
// This replaces the O(C^2) inter-chunk transfer of scan.rs:218-251 with the
// elementwise recurrence S_{k+1} = T_k(S_k), evaluated where it is needed.
// Records are f32 and move through device-coherent loads and stores (sc1); a
// record is complete before its flag is set (s_waitcnt vmcnt(0), then the
// flag), and read only after its flag has been seen.  Inputs are read once.
#include <algorithm>
#include <cstdlib>

#include "scan_common.hpp"

namespace m3 {

namespace {

using namespace scan;

constexpr int kP = 64;
constexpr int kRows = 64;   // rows (token, rank) per chunk

constexpr unsigned kAgg = 1u;
constexpr unsigned kPrefix = 2u;
// Polls of one flag before a wait is abandoned.  A predecessor holds a smaller
// ticket and publishes within microseconds; the limit only bounds the kernel
// if that invariant is ever broken (counted in the control word, see below).
constexpr unsigned kSpinLimit = 1u << 20;

// Workspace sections, byte offsets from the base (each 256-byte aligned):
//   ctl     [64] u32: [0] ticket counter, [1] abandoned waits
//   flag    [S * C] u32, 0 empty / kAgg / kPrefix
//   agg_u   [S * C][P * N] f32, U_k^T in MFMA D layout [p-tile][n-tile][lane][4]
//   agg_e   [S * C] f32 chunk decay exp(sum dt A)
//   agg_phi [S * C][N/2] f32 chunk angle total per pair
//   pre_s   [S * C][P * N] f32, S_{k+1} in the layout of agg_u
//   pre_phi [S * C][N/2] f32 wrapped angle entering chunk k+1
// ctl and flag are cleared by lookback_clear_kernel before every scan.
struct LbLayout {
    size_t ctl, flag, agg_u, agg_e, agg_phi, pre_s, pre_phi, total;
};

size_t lb_align(size_t v) { return (v + 255) & ~size_t(255); }

LbLayout lb_layout(size_t bhk, size_t n) {
    LbLayout l;
    size_t o = 0;
    l.ctl = o;
    o = lb_align(o + 64 * 4);
    l.flag = o;
    o = lb_align(o + bhk * 4);
    l.agg_u = o;
    o = lb_align(o + bhk * kP * n * 4);
    l.agg_e = o;
    o = lb_align(o + bhk * 4);
    l.agg_phi = o;
    o = lb_align(o + bhk * (n / 2) * 4);
    l.pre_s = o;
    o = lb_align(o + bhk * kP * n * 4);
    l.pre_phi = o;
    o = lb_align(o + bhk * (n / 2) * 4);
    l.total = o;
    return l;
}

struct LbWs {
    unsigned *ctl;
    unsigned *flag;
    float *agg_u, *agg_e, *agg_phi, *pre_s, *pre_phi;
};

LbWs lb_ws(char *base, const LbLayout &l) {
    LbWs w;
    w.ctl = reinterpret_cast<unsigned *>(base + l.ctl);
    w.flag = reinterpret_cast<unsigned *>(base + l.flag);
    w.agg_u = reinterpret_cast<float *>(base + l.agg_u);
    w.agg_e = reinterpret_cast<float *>(base + l.agg_e);
    w.agg_phi = reinterpret_cast<float *>(base + l.agg_phi);
    w.pre_s = reinterpret_cast<float *>(base + l.pre_s);
    w.pre_phi = reinterpret_cast<float *>(base + l.pre_phi);
    return w;
}

__global__ void lookback_clear_kernel(unsigned *p, size_t n) {
    for (size_t i = blockIdx.x * size_t(256) + threadIdx.x; i < n; i += gridDim.x * size_t(256))
        p[i] = 0u;
}

// Every store this thread issued has completed before the workgroup barrier
// that precedes a flag store (order-only workgroup fence plus vmcnt(0); the
// records themselves were written device-coherent).
__device__ __forceinline__ void records_done() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));   // vmcnt(0)
}

__device__ __forceinline__ unsigned flag_load(const unsigned *f) {
    return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned wait_flag(const unsigned *f, unsigned *abandoned) {
    unsigned v;
    unsigned n = 0;
    while ((v = flag_load(f)) == 0u) {
        if (++n == kSpinLimit) {
            __hip_atomic_fetch_add(abandoned, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return kPrefix;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return v;
}

// sin and cos of an angle through the hardware units, which take revolutions:
// the angle is first wrapped into [-pi, pi] (bf16 storage bounds the accuracy
// this path needs far above their error).
__device__ __forceinline__ void hw_sincos(float x, float *sv, float *cv) {
    const float rev = wrap_angle(x) * 0.15915494309189533577f;
    *sv = __builtin_amdgcn_sinf(rev);
    *cv = __builtin_amdgcn_cosf(rev);
}

__device__ __forceinline__ u32x4 as_u4(f32x4 v) {
    return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                 __float_as_uint(v[3])};
}
__device__ __forceinline__ f32x4 as_f4(u32x4 v) {
    return f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                 __uint_as_float(v[3])};
}

// v1 = element n, v2 = element n + N/2 of a pair; R(t) (v1, v2) =
// (v1 cos t - v2 sin t, v1 sin t + v2 cos t)
__device__ __forceinline__ void rot_pairs(f32x4 &lo, f32x4 &hi, const f32x4 cs, const f32x4 sn) {
    const f32x4 l = lo;
    lo = l * cs - hi * sn;
    hi = l * sn + hi * cs;
}

// The band tiles (t-tile tj, s-tile si) the output product reads, in order:
// every tile on or below the diagonal of 16-row tiles, plus the zero tiles
// above it that a 32-row k-block still covers.  tile(i) = tj << 8 | si.
template <int R>
struct BandTiles {
    static constexpr int NT = kRows / 16;
    static constexpr int ncol(int tj) {
        const int tlast = (16 * tj + 15) / R;
        const int send = (tlast + 1) * R < kRows ? (tlast + 1) * R : kRows;
        return ((send + 31) / 32) * 32;
    }
    static constexpr int count() {
        int n = 0;
        for (int tj = 0; tj < NT; ++tj) n += ncol(tj) / 16;
        return n;
    }
    static constexpr int COUNT = count();
    static constexpr int SLOTS = (COUNT + 3) / 4;
    static __device__ __forceinline__ int tile(int i) {
        int tj = 0;
        while (i >= ncol(tj) / 16) {
            i -= ncol(tj) / 16;
            ++tj;
        }
        return (tj << 8) | i;
    }
};

template <int N, int R>
struct LbSmem {
    using G = Geo<bf16_t, N, kP, R, kRows, 4>;
    static constexpr int LDN = N + 8;       // C~ rows, 16-byte aligned
    static constexpr int LDR = kRows + 8;   // X^T and band rows, 16-byte aligned
    // B~^T rows of 2*LDB = 136 bytes (34 banks): the eight rows an MFMA lane
    // gathers for one operand are four apart and fall eight banks apart
    static constexpr int LDB = kRows + 4;
    __bf16 Cs[kRows * LDN];   // C~[rho][npos(n)]
    __bf16 Xt[kP * LDR];      // X^T [p][rho]
    union {
        __bf16 Bt[N * LDB];       // B~^T [n][rho] (stage, local products)
        __bf16 Ms[kRows * LDR];   // masked band [rho_t][rho_s] (outputs)
    } u;
    float acum[G::QT], gw[G::QT], ww[G::QT], eac[G::QT], wd[G::QT];
    float phi_tot[N / 2];   // in-chunk angle at the last token, per pair
    float cph[N / 2], sph[N / 2];   // cos, sin of the chunk total Phi_k
    float cth[N / 2], sth[N / 2];   // cos, sin of the folded rotation / final angle
    float eda;
    unsigned ticket, flag, hint;
};

template <int N, int R>
// d_state 128 holds the chunk share U, the fold V and a record in registers
// at once: two workgroups per CU; d_state 64 fits four.
__global__ void __launch_bounds__(kThreads, N == 128 ? 2 : 4)
ssd_scan_lookback_kernel(ScanLaunch a, LbWs ws, int nck, int min_fold) {
    using T = bf16_t;
    constexpr int P = kP, ROWS = kRows;
    using G = Geo<T, N, P, R, ROWS, 4>;
    using S = LbSmem<N, R>;
    using RawT = Raw<T, N, P, R, ROWS, 4, true>;
    constexpr int KB = 32;
    constexpr int LDN = S::LDN, LDR = S::LDR, LDB = S::LDB;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL;
    constexpr int NT = ROWS / 16;
    constexpr int NTN = N / 16;
    constexpr int HT = NTN / 2;
    constexpr uint32_t SZ = 2;
    constexpr uint32_t REC = P * N * 4;   // bytes of one state record

    __shared__ S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t nseq = a.batch * H;

    if (tid == 0)
        sm.ticket = __hip_atomic_fetch_add(ws.ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    // the ticket is uniform: keep it (and all that derives from it) scalar
    const size_t tk = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(sm.ticket)));
    const int ck = static_cast<int>(tk / nseq);
    const size_t bh = tk % nseq;
    const size_t bb = bh / H, hh = bh % H;
    const size_t rec = bh * nck + ck;
    const bool rot = a.theta != nullptr;
    const bool last_chunk = ck == nck - 1;

    // the predecessor's flag as a hint: a chunk whose predecessor already has
    // its prefix skips publishing an aggregate
    unsigned hint = 0u;
    if (tid == 0 && ck > 0) hint = flag_load(ws.flag + rec - 1);

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;
    const int pcol = 16 * wave + c;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);
    RawT cur;
    load_chunk<T, N, P, R, ROWS, 4, true>(rs, ck, wave, lane, cur);

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const bool skip = a.d_skip != nullptr;

    // ---- stage
    {
        const size_t tau = static_cast<size_t>(ck) * QT + my_t;
        const bool live = tok_lane && tau < L;
        float av, gv, wv;
        token_scalars(a, cur, A, live, av, gv, wv);
        const float acum = seg_scan<G::SW>(av);
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        if (wave == 0 && sub == 0 && tok_lane) {
            sm.acum[my_t] = acum;
            sm.gw[my_t] = gv;
            sm.ww[my_t] = wv;
            sm.eac[my_t] = dexp<true>(acum);                  // exp_decay(acum)
            sm.wd[my_t] = dexp<true>(last - acum) * wv;       // exp_decay(last, acum, w)
        }
        if (tid == 0) sm.eda = dexp<true>(last);
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
                // the hardware sine takes revolutions; |psi| <= pi
                const float rev = wrap_angle(pre) * 0.15915494309189533577f;
                sn[j] = __builtin_amdgcn_sinf(rev);
                cs[j] = __builtin_amdgcn_cosf(rev);
            }
        }
        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / 4) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                sm.Xt[p * LDR + my_t * R + r] = to_op<__bf16>(elem<T>(cur.x, e));
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = my_t * R + r;
                float rc[2][PPL];
#pragma unroll
                for (int j = 0; j < PPL; ++j) {
                    const float b1 = elem<T>(cur.b[0], j * R + r);
                    const float b2 = elem<T>(cur.b[1], j * R + r);
                    const float c1 = elem<T>(cur.c[0], j * R + r);
                    const float c2 = elem<T>(cur.c[1], j * R + r);
                    sm.u.Bt[(i0 + j) * LDB + rho] = to_op<__bf16>(b1 * cs[j] + b2 * sn[j]);
                    sm.u.Bt[(i0 + NH + j) * LDB + rho] = to_op<__bf16>(-b1 * sn[j] + b2 * cs[j]);
                    rc[0][j] = c1 * cs[j] + c2 * sn[j];
                    rc[1][j] = -c1 * sn[j] + c2 * cs[j];
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if constexpr (PPL % 4 == 0) {
#pragma unroll
                        for (int q = 0; q < PPL; q += 4)
                            st4(&sm.Cs[rho * LDN + npos<true>(i0 + h * NH + q)], &rc[h][q]);
                    } else {
#pragma unroll
                        for (int j = 0; j < PPL; ++j)
                            sm.Cs[rho * LDN + npos<true>(i0 + h * NH + j)] = to_op<__bf16>(rc[h][j]);
                    }
                }
            }
        }
    }
    lds_barrier();

    // ---- chunk aggregate: cos and sin of the angle total (precise)
    float my_phi = 0.0f;   // tid < NH: Phi_k of pair tid
    if (tid < NH) {
        float ts = 0.0f, tc = 1.0f;
        if (rot) {
            my_phi = sm.phi_tot[tid];
            hw_sincos(my_phi, &ts, &tc);
        }
        sm.cph[tid] = tc;
        sm.sph[tid] = ts;
    }

    // ---- U^T[n][p] = sum_rho B~^T[n][rho] (w decay X)[rho][p]; wave w: p-tile w.
    //      B operand: X^T row p, k-slots 8g..8g+7 of each k-block, weighted.
    bf16x8 xw[ROWS / KB];
#pragma unroll
    for (int kb = 0; kb < ROWS / KB; ++kb) {
        const bf16x8 xv = *reinterpret_cast<const bf16x8 *>(&sm.Xt[pcol * LDR + KB * kb + 8 * g]);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            xw[kb][j] = to_bf16(static_cast<float>(xv[j]) * sm.wd[(KB * kb + 8 * g + j) / R]);
    }
    f32x4 u[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < ROWS / KB; ++kb) {
            const __bf16 *ar = &sm.u.Bt[(16 * i + c) * LDB + KB * kb + 8 * g];   // 8-byte aligned
            const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(ar);
            const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(ar + 4);
            const bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc = mfma_bf16(av, xw[kb], acc);
        }
        u[i] = acc;
    }

    // ---- masked band tiles (transposed: D[s][t], lane holds four s of one t).
    //      A operand: B~ rows s gathered from B~^T in the k order of C~'s
    //      columns (position 32kb + 8g + 4h + r holds n = 32kb + 16h + 4g + r).
    //      Band tile 4q + w goes to wave w, register slot q.
    using BT = BandTiles<R>;
    float band[BT::SLOTS][4];
#pragma unroll
    for (int q = 0; q < BT::SLOTS; ++q) {
#pragma unroll
        for (int r = 0; r < 4; ++r) band[q][r] = 0.0f;
        const int idx = 4 * q + wave;
        if (idx >= BT::COUNT) continue;
        const int tj = BT::tile(idx) >> 8, si = BT::tile(idx) & 255;
        const int trow = 16 * tj + c;
        const int tlast = (16 * tj + 15) / R;
        if ((16 * si) / R > tlast) continue;   // above the band: zeros
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < N / KB; ++kb) {
            bf16x8 av;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    av[4 * h + r] = sm.u.Bt[(KB * kb + 16 * h + 4 * g + r) * LDB + 16 * si + c];
            const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(&sm.Cs[trow * LDN + KB * kb + 8 * g]);
            acc = mfma_bf16(av, bv, acc);
        }
        const int tt = trow / R;
        const float at = sm.acum[tt];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int srow = 16 * si + 4 * g + r;
            const int ts = srow / R;
            float v = 0.0f;
            if (ts <= tt) {
                const float wgt = (ts == tt) ? sm.gw[ts] : sm.ww[ts];
                v = acc[r] * wgt * dexp<true>(at - sm.acum[ts]);
            }
            if (skip && srow == trow) v += dskip;   // scan.rs:593-597
            band[q][r] = v;
        }
    }
    if (tid == 0) sm.hint = hint;
    __syncthreads();   // B~^T is dead from here: its space becomes the band
#pragma unroll
    for (int q = 0; q < BT::SLOTS; ++q) {
        const int idx = 4 * q + wave;
        if (idx >= BT::COUNT) continue;
        const int tj = BT::tile(idx) >> 8, si = BT::tile(idx) & 255;
        st4(&sm.u.Ms[(16 * tj + c) * LDR + 16 * si + 4 * g], band[q]);
    }

    const float eda = sm.eda;
    // this lane's state elements: p = pcol, n = 16i + 4g + r; pairs (i, i + HT)
    const uint32_t soff = static_cast<uint32_t>(((wave * NTN) * 64 + lane) * 16);

    // ---- publish the aggregate when the predecessor's prefix was not ready
    if (ck > 0 && (min_fold > 0 ||
                   __builtin_amdgcn_readfirstlane(static_cast<int>(sm.hint)) != static_cast<int>(kPrefix))) {
        const rsrc_t ru = make_rsrc(ws.agg_u + rec * (P * N), REC);
#pragma unroll
        for (int i = 0; i < NTN; ++i) bst16_coh(as_u4(u[i]), ru, soff + i * 64 * 16);
        if (tid < NH) bstf_coh(my_phi, make_rsrc(ws.agg_phi + rec * NH, NH * 4), tid * 4);
        if (tid == 0) bstf_coh(eda, make_rsrc(ws.agg_e + rec, 4), 0);
        records_done();
        __syncthreads();
        if (tid == 0)
            __hip_atomic_store(ws.flag + rec, kAgg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- the state entering this chunk, in its frame
    f32x4 st[NTN];
    float phi0 = 0.0f;   // tid < NH: wrapped global angle entering this chunk
    if (ck == 0) {
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        const size_t sbase = bh * P * N + static_cast<size_t>(pcol) * N;
#pragma unroll
        for (int i = 0; i < NTN; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (h0 != nullptr) {
            float first = 0.0f;
            if (l0 != nullptr) {
                // carry S = h + (1 - lambda_0) dt_0 last_u   (scan.rs:521-535)
                const size_t i0s = (bb * L) * H + hh;
                first = (1.0f - a.lambda[i0s]) * a.dt[i0s];
            }
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                st[i] = *reinterpret_cast<const f32x4 *>(h0 + sbase + 16 * i + 4 * g);
                if (l0 != nullptr)
                    st[i] += *reinterpret_cast<const f32x4 *>(l0 + sbase + 16 * i + 4 * g) * first;
            }
        }
        if (rot && a.angle0 != nullptr) {
            // into chunk 0's frame: S_0 = R(angle0) h
#pragma unroll
            for (int i = 0; i < HT; ++i) {
                const f32x4 ph = *reinterpret_cast<const f32x4 *>(a.angle0 + bh * NH + 16 * i + 4 * g);
                f32x4 cs4, sn4;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float sv, cv;
                    hw_sincos(ph[r], &sv, &cv);
                    sn4[r] = sv;
                    cs4[r] = cv;
                }
                rot_pairs(st[i], st[i + HT], cs4, sn4);
            }
            if (tid < NH) phi0 = a.angle0[bh * NH + tid];
        }
    } else {
        // fold aggregates until a published prefix: S_k = R(Theta)(E S_{j+1}) + V
        float E = 1.0f;
        f32x4 v[NTN];
#pragma unroll
        for (int i = 0; i < NTN; ++i) v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        float tsum = 0.0f;   // tid < NH: Theta of pair tid
        bool folded = false;
        int j = ck - 1;
        for (;;) {
            const size_t rj = bh * nck + j;
            if (tid == 0) sm.flag = wait_flag(ws.flag + rj, ws.ctl + 1);
            __syncthreads();
            // with min_fold > 0 (a verification mode) every chunk publishes its
            // aggregate and the first min_fold steps fold aggregates even
            // where a prefix is already out
            const bool pre = __builtin_amdgcn_readfirstlane(static_cast<int>(sm.flag)) >=
                                 static_cast<int>(kPrefix) &&
                             (ck - 1 - j >= min_fold || j == 0);
            // one record per step: the prefix S_{j+1}, or the aggregate U_j
            const rsrc_t rr = make_rsrc((pre ? ws.pre_s : ws.agg_u) + rj * (P * N), REC);
            f32x4 rv[NTN];
#pragma unroll
            for (int i = 0; i < NTN; ++i) rv[i] = as_f4(bld16_coh(rr, soff + i * 64 * 16));
            if (pre) {
                if (tid < NH) phi0 = bldf_coh(make_rsrc(ws.pre_phi + rj * NH, NH * 4), tid * 4) + tsum;
                // S_k = G(S_{j+1})
                if (rot && folded) {
#pragma unroll
                    for (int i = 0; i < HT; ++i) {
                        const f32x4 cs4 = *reinterpret_cast<const f32x4 *>(&sm.cth[16 * i + 4 * g]);
                        const f32x4 sn4 = *reinterpret_cast<const f32x4 *>(&sm.sth[16 * i + 4 * g]);
                        f32x4 lo = rv[i] * E, hi = rv[i + HT] * E;
                        rot_pairs(lo, hi, cs4, sn4);
                        st[i] = lo + v[i];
                        st[i + HT] = hi + v[i + HT];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < NTN; ++i) st[i] = rv[i] * E + v[i];
                }
                break;
            }
            // aggregate of chunk j: G <- G o T_j
            const float ej = bldf_coh(make_rsrc(ws.agg_e + rj, 4), 0);
            if (rot && tid < NH) {
                tsum += bldf_coh(make_rsrc(ws.agg_phi + rj * NH, NH * 4), tid * 4);
                float ts, tc;
                hw_sincos(tsum, &ts, &tc);
                sm.cth[tid] = tc;
                sm.sth[tid] = ts;
            }
            __syncthreads();
            if (rot) {
#pragma unroll
                for (int i = 0; i < HT; ++i) {
                    const f32x4 cs4 = *reinterpret_cast<const f32x4 *>(&sm.cth[16 * i + 4 * g]);
                    const f32x4 sn4 = *reinterpret_cast<const f32x4 *>(&sm.sth[16 * i + 4 * g]);
                    f32x4 lo = rv[i], hi = rv[i + HT];
                    rot_pairs(lo, hi, cs4, sn4);
                    v[i] += lo * E;
                    v[i + HT] += hi * E;
                }
            } else {
#pragma unroll
                for (int i = 0; i < NTN; ++i) v[i] += rv[i] * E;
            }
            folded = true;
            E *= ej;
            --j;
        }
    }

    // ---- S_{k+1} = R(Phi_k)(e_k S_k + U_k), and the angle entering chunk k+1
    const float phi_next = wrap_angle(phi0 + my_phi);   // tid < NH
    const bool want_state = a.h_out != nullptr || a.last_u_out != nullptr || a.angle_out != nullptr;
    if (last_chunk && want_state && tid < NH) {
        float ts = 0.0f, tc = 1.0f;
        if (rot) hw_sincos(phi_next, &ts, &tc);
        sm.cth[tid] = tc;   // the look-back is over: the fold's rotation is dead
        sm.sth[tid] = ts;
        if (a.angle_out != nullptr) a.angle_out[bh * NH + tid] = phi_next;
    }
    if (!last_chunk || want_state) {
        f32x4 nx[NTN];
#pragma unroll
        for (int i = 0; i < HT; ++i) {
            f32x4 lo = st[i] * eda + u[i], hi = st[i + HT] * eda + u[i + HT];
            if (rot) {
                const f32x4 cs4 = *reinterpret_cast<const f32x4 *>(&sm.cph[16 * i + 4 * g]);
                const f32x4 sn4 = *reinterpret_cast<const f32x4 *>(&sm.sph[16 * i + 4 * g]);
                rot_pairs(lo, hi, cs4, sn4);
            }
            nx[i] = lo;
            nx[i + HT] = hi;
        }
        if (!last_chunk) {
            const rsrc_t rp = make_rsrc(ws.pre_s + rec * (P * N), REC);
#pragma unroll
            for (int i = 0; i < NTN; ++i) bst16_coh(as_u4(nx[i]), rp, soff + i * 64 * 16);
            if (tid < NH) bstf_coh(phi_next, make_rsrc(ws.pre_phi + rec * NH, NH * 4), tid * 4);
            records_done();
        } else {
            // boundary state in the global frame (scan.rs:270-288, 599-638)
            __syncthreads();
            const size_t sbase = bh * P * N + static_cast<size_t>(pcol) * N;
            const size_t tl = (bb * L + (L - 1)) * H + hh;
            const T *bp = static_cast<const T *>(a.b) + tl * N * R;
            const T *xp = static_cast<const T *>(a.x) + (tl * P + static_cast<size_t>(pcol)) * R;
#pragma unroll
            for (int i = 0; i < HT; ++i) {
                const int nlo = 16 * i + 4 * g;
                const f32x4 ce = *reinterpret_cast<const f32x4 *>(&sm.cth[nlo]);
                const f32x4 se = *reinterpret_cast<const f32x4 *>(&sm.sth[nlo]);
                if (a.h_out != nullptr) {
                    f32x4 hl = nx[i], hh2 = nx[i + HT];
                    rot_pairs(hl, hh2, ce, -se);   // R(-phi_end)
                    *reinterpret_cast<f32x4 *>(a.h_out + sbase + nlo) = hl;
                    *reinterpret_cast<f32x4 *>(a.h_out + sbase + nlo + NH) = hh2;
                }
                if (a.last_u_out != nullptr) {
                    // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T, B~ = R(-phi_end) B  (scan.rs:599-618)
                    f32x4 ul = {0.f, 0.f, 0.f, 0.f}, uh = ul;
#pragma unroll
                    for (int m = 0; m < R; ++m) {
                        const float xv = to_f32(xp[m]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float b1 = to_f32(bp[(nlo + r) * R + m]);
                            const float b2 = to_f32(bp[(nlo + r + NH) * R + m]);
                            ul[r] += xv * (b1 * ce[r] + b2 * se[r]);
                            uh[r] += xv * (-b1 * se[r] + b2 * ce[r]);
                        }
                    }
                    *reinterpret_cast<f32x4 *>(a.last_u_out + sbase + nlo) = ul;
                    *reinterpret_cast<f32x4 *>(a.last_u_out + sbase + nlo + NH) = uh;
                }
            }
        }
    }
    __syncthreads();   // also orders the band stores before the output products
    if (!last_chunk && tid == 0)
        __hip_atomic_store(ws.flag + rec, kPrefix, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- y^T[p][t] = exp(acum_t) sum_n S[p][n] C~[t][n] + sum_s X^T[p][s] M[t][s]
    {
        bf16x8 sf[N / 32];
#pragma unroll
        for (int f = 0; f < N / 32; ++f) {
            const f32x4 lo = st[2 * f], hi = st[2 * f + 1];
            sf[f] = bf16x8{to_bf16(lo[0]), to_bf16(lo[1]), to_bf16(lo[2]), to_bf16(lo[3]),
                           to_bf16(hi[0]), to_bf16(hi[1]), to_bf16(hi[2]), to_bf16(hi[3])};
        }
        const __bf16 *xr = &sm.Xt[pcol * LDR];
        const uint32_t tau0 = static_cast<uint32_t>(ck) * QT;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const __bf16 *cr = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
            for (int kb = 0; kb < N / 32; ++kb)
                acc = mfma_bf16(sf[kb], *reinterpret_cast<const bf16x8 *>(cr + 32 * kb + 8 * g), acc);
            acc = acc * sm.eac[(16 * tj + c) / R];
            const __bf16 *mr = &sm.u.Ms[(16 * tj + c) * LDR];
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
                u32x2 pk;
                pk[0] = static_cast<unsigned int>(from_f32<bf16_t>(acc[0]).bits) |
                        (static_cast<unsigned int>(from_f32<bf16_t>(acc[1]).bits) << 16);
                pk[1] = static_cast<unsigned int>(from_f32<bf16_t>(acc[2]).bits) |
                        (static_cast<unsigned int>(from_f32<bf16_t>(acc[3]).bits) << 16);
                bst8(pk, rs.y, oy);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) bst2(from_f32<bf16_t>(acc[r]).bits, rs.y, oy + r * R * SZ);
            }
        }
    }
}

// M3_SCAN_LOOKBACK_FOLD=m (verification only): every chunk folds at least m
// predecessor aggregates before it takes a published prefix.
int min_fold() {
    const char *e = std::getenv("M3_SCAN_LOOKBACK_FOLD");
    return e != nullptr ? std::max(0, std::atoi(e)) : 0;
}

template <int N, int R>
hipError_t launch_lb(const ScanLaunch &a, char *base, hipStream_t s) {
    constexpr int QT = kRows / R;
    const int nck = static_cast<int>((a.seq + QT - 1) / QT);
    const size_t bhk = a.batch * a.heads * nck;
    const LbLayout l = lb_layout(bhk, N);
    const LbWs ws = lb_ws(base, l);
    const size_t nclear = (l.agg_u - l.ctl) / 4;   // ctl and flag sections
    const unsigned cblocks = static_cast<unsigned>(std::min<size_t>((nclear + 255) / 256, 1024));
    hipLaunchKernelGGL(lookback_clear_kernel, dim3(cblocks), dim3(256), 0, s, ws.ctl, nclear);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((ssd_scan_lookback_kernel<N, R>), dim3(bhk), dim3(kThreads), 0, s, a, ws,
                       nck, min_fold());
    return hipGetLastError();
}

}  // namespace

bool scan_lookback_supported(const ScanLaunch &a) {
    return a.bf16 && a.mode_raw && scan_fast_supported(a) && a.seq > 0 &&
           (a.d_state == 64 || a.d_state == 128) &&
           (a.rank == 1 || a.rank == 2 || a.rank == 4);
}

size_t scan_lookback_workspace(const ScanLaunch &a) {
    if (!scan_lookback_supported(a)) return 0;
    const size_t qt = kRows / a.rank;
    const size_t nck = (a.seq + qt - 1) / qt;
    return lb_layout(a.batch * a.heads * nck, a.d_state).total;
}

hipError_t launch_scan_lookback(const ScanLaunch &a, void *workspace, hipStream_t stream) {
    if (!scan_lookback_supported(a)) return hipErrorNotSupported;
    char *ws = static_cast<char *>(workspace);
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_lb<128, 1>(a, ws, stream);
        if (r == 2) return launch_lb<128, 2>(a, ws, stream);
        if (r == 4) return launch_lb<128, 4>(a, ws, stream);
    } else if (n == 64) {
        if (r == 1) return launch_lb<64, 1>(a, ws, stream);
        if (r == 2) return launch_lb<64, 2>(a, ws, stream);
        if (r == 4) return launch_lb<64, 4>(a, ws, stream);
    }
    return hipErrorNotSupported;
}

}  // namespace m3
