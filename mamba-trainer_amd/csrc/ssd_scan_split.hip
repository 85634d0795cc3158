// Chunked SSD scan for gfx950 as two kernels: a chunk-parallel pass that does
// all the per-token elementwise work, and a sequential walk that only carries
// the state.  Same shapes as ssd_scan_fast.hip (head_dim 64, d_state 64/128,
// rank 1/2/4, aligned operands); restates src/ssm/scan.rs:116-291, 458-638.
//
// Why two kernels: per chunk, the rotation of B and C (one sine and cosine per
// (token, pair), fused.rs:588-619), the decay and trapezoid weights and the
// band mask are several thousand VALU instructions, while a batch x head count
// of ~100 sequences fills under half of the chip's 256 CUs.  The chunk pass
// spreads that work over every chunk of every sequence at once; the walk keeps
// only what truly depends on the previous chunk.
//
// ssd_chunk_kernel -- one workgroup per (chunk, batch, head).  Everything is
//   expressed in the chunk's own rotating frame (angles relative to the chunk
//   start, so the pass needs nothing from earlier chunks).  It writes, per
//   chunk, into the caller's workspace:
//     M   [ROWS][ROWS]  masked band  (C~ B~^T o L)   (ssd_band, fused.rs:2044-2070)
//                       with the skip D on the diagonal (scan.rs:593-597)
//     Ce  [ROWS][N]     C~_t * exp(acum_t)            (scan.rs:253-263)
//     Bwt [N][ROWS]     (B~_s * w_s * exp(acum_end - acum_s))^T   (scan.rs:207-216)
//     decay exp(acum_end), and per pair the chunk's angle total Phi with its
//     cosine and sine.
// ssd_walk_kernel -- one workgroup per (batch, head), four waves, the f32
//   state S in registers.  Per chunk: y = M X + Ce S (MFMA), S = decay * S +
//   Bwt X (MFMA), then S is turned into the next chunk's frame by rotating
//   its (n, n + N/2) pairs by Phi.  Inputs of chunk k+2 are requested while
//   chunk k+1 is staged into the second LDS operand set.
//
// The workspace is sized so that it stays resident in the MI355X's memory-side
// (infinity) cache between the two launches at the benchmark shapes.
#include "scan_common.hpp"

namespace m3 {

namespace {

using namespace scan;

// Offsets (bytes) of the workspace sections for one launch.
struct SplitLayout {
    size_t m, ce, bwt, cdec, phi, cphi, sphi, total;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

SplitLayout split_layout(size_t bh, size_t nchunks, size_t rows, size_t n, size_t esz) {
    SplitLayout l{};
    const size_t ch = bh * nchunks;
    size_t o = 0;
    l.m = o;
    o = align256(o + ch * rows * rows * esz);
    l.ce = o;
    o = align256(o + ch * rows * n * esz);
    l.bwt = o;
    o = align256(o + ch * n * rows * esz);
    l.cdec = o;
    o = align256(o + ch * 4);
    l.phi = o;
    o = align256(o + ch * (n / 2) * 4);
    l.cphi = o;
    o = align256(o + ch * (n / 2) * 4);
    l.sphi = o;
    o = align256(o + ch * (n / 2) * 4);
    l.total = o;
    return l;
}

struct SplitWs {
    char *base;
    SplitLayout l;
};

// ============================================================== chunk pass
template <typename T, int N, int R, int ROWS>
struct ChunkSmem {
    using G = Geo<T, N, 64, R, ROWS>;
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;
    static constexpr int LDR = ROWS + PAD;
    op_t Bs[ROWS * LDN];
    op_t Cs[ROWS * LDN];
    op_t Bwt[N * LDR];
    float acum[G::QT], gw[G::QT], ww[G::QT];
    float phi_tot[G::NH];
};

template <typename T, int N, int R, int ROWS>
__global__ void __launch_bounds__(kThreads)
ssd_chunk_kernel(ScanLaunch a, SplitWs ws, int nchunks) {
    constexpr int P = 64;
    using G = Geo<T, N, P, R, ROWS>;
    using S = ChunkSmem<T, N, R, ROWS>;
    using op_t = typename S::op_t;
    constexpr int KB = Op<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL;
    constexpr int NT = ROWS / 16;
    constexpr bool kBf16 = sizeof(op_t) == 2;
    constexpr uint32_t SZ = sizeof(T);

    __shared__ __align__(16) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t BH = a.batch * H;
    const size_t bh = blockIdx.x % BH;
    const int ck = static_cast<int>(blockIdx.x / BH);
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const size_t chunk_id = bh * nchunks + ck;

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;

    // ---- this lane's token: B and C pair slices, theta slice, dt / lambda
    const size_t row0 = bb * L * H + hh;
    const size_t rows = L * H - hh;
    auto mk = [&](const void *base, size_t row_bytes) {
        return make_rsrc(static_cast<const char *>(base) + row0 * row_bytes,
                         static_cast<uint32_t>(rows * row_bytes));
    };
    const uint32_t tok = static_cast<uint32_t>(ck) * QT + my_t;
    const uint32_t tok_bc = static_cast<uint32_t>(H * N * R * SZ);
    const uint32_t tok_s = static_cast<uint32_t>(H * 4);
    u32x4 vb[2][G::HV], vc[2][G::HV];
    {
        const rsrc_t rb = mk(a.b, N * R * SZ), rc = mk(a.c, N * R * SZ);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < G::HV; ++v) {
                const uint32_t off = tok * tok_bc + ((i0 + h * NH) * R + v * G::E) * SZ;
                vb[h][v] = bld16(rb, off);
                vc[h][v] = bld16(rc, off);
            }
    }
    unsigned int th[G::TW];
    if (rot) {
        const rsrc_t rt = mk(a.theta, NH * SZ);
        const uint32_t ot = tok * static_cast<uint32_t>(H * NH * SZ) + i0 * SZ;
        if constexpr (G::THB >= 16) {
#pragma unroll
            for (int v = 0; v < G::THB / 16; ++v) {
                const u32x4 q = bld16(rt, ot + 16 * v);
#pragma unroll
                for (int j = 0; j < 4; ++j) th[4 * v + j] = q[j];
            }
        } else if constexpr (G::THB == 8) {
            const u32x2 q = bld8(rt, ot);
            th[0] = q[0];
            th[1] = q[1];
        } else {
            th[0] = bld4(rt, ot);
        }
    }
    float s0, s1, s2, s3;
    if (a.mode_raw) {
        const rsrc_t rdt = mk(a.dt, 4), rl = mk(a.lambda, 4);
        s0 = bldf(rdt, tok * tok_s);
        s1 = bldf(rl, tok * tok_s);
        s2 = bldf(rdt, (tok + 1) * tok_s);   // next token (the trapezoid's halo)
        s3 = bldf(rl, (tok + 1) * tok_s);
    } else {
        s0 = bldf(mk(a.a, 4), tok * tok_s);
        s1 = bldf(mk(a.g, 4), tok * tok_s);
        s2 = bldf(mk(a.w, 4), tok * tok_s);
        s3 = 0.0f;
    }

    // ---- per-token scalars: log decay, trapezoid weights, in-chunk cumsum
    const bool live = tok_lane && tok < L;
    float av, gv, wv;
    if (a.mode_raw) {
        const float A = 0.0f - expf(a.a_log[hh]);    // a_log.exp().neg() (scan.rs:470-474)
        av = s0 * A;
        gv = s1 * s0;                                // fused.rs:2494
        wv = gv + (1.0f - s3) * s2;                  // fused.rs:2496-2498
    } else {
        av = s0;
        gv = s1;
        wv = s2;
    }
    if (!live) av = gv = wv = 0.f;
    const float acum = seg_scan<G::SW>(av);
    const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
    const float wd = dexp<kBf16>(last - acum) * wv;   // exp_decay(last, acum, w)
    const float eac = dexp<kBf16>(acum);              // exp_decay(acum)
    if (wave == 0 && sub == 0 && tok_lane) {
        sm.acum[my_t] = acum;
        sm.gw[my_t] = gv;
        sm.ww[my_t] = wv;
        if (my_t == QT - 1)
            reinterpret_cast<float *>(ws.base + ws.l.cdec)[chunk_id] = dexp<kBf16>(acum);
    }

    // ---- frame angle relative to the chunk start, and the chunk's total
    float cs[PPL], sn[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        cs[j] = 1.0f;
        sn[j] = 0.0f;
    }
    if (rot) {
        const float dtt = live ? s0 : 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const float pre = seg_scan<G::SW>(dtt * welem<T>(th, j));
            // the lane of the chunk's last token holds the chunk total
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

    // ---- rotate B and C by -psi (fused.rs:610-617); stage the band operands,
    //      write C~ exp(acum) and stage (B~ w decay)^T
    if (tok_lane) {
        op_t *ce_o = reinterpret_cast<op_t *>(ws.base + ws.l.ce) + chunk_id * ROWS * N;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int rho = my_t * R + r;
            float rb[2][PPL], rc[2][PPL];
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const float b1 = elem<T>(vb[0], j * R + r);
                const float b2 = elem<T>(vb[1], j * R + r);
                const float c1 = elem<T>(vc[0], j * R + r);
                const float c2 = elem<T>(vc[1], j * R + r);
                rb[0][j] = b1 * cs[j] + b2 * sn[j];
                rb[1][j] = -b1 * sn[j] + b2 * cs[j];
                rc[0][j] = c1 * cs[j] + c2 * sn[j];
                rc[1][j] = -c1 * sn[j] + c2 * cs[j];
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float ce[PPL];
#pragma unroll
                for (int j = 0; j < PPL; ++j) ce[j] = rc[h][j] * eac;
                if constexpr (PPL % 4 == 0) {
#pragma unroll
                    for (int q = 0; q < PPL; q += 4) {
                        const int n = i0 + h * NH + q;
                        st4(&sm.Bs[rho * LDN + npos<kBf16>(n)], &rb[h][q]);
                        st4(&sm.Cs[rho * LDN + npos<kBf16>(n)], &rc[h][q]);
                        st4(&ce_o[rho * N + npos<kBf16>(n)], &ce[q]);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < PPL; ++j) {
                        const int n = i0 + h * NH + j;
                        sm.Bs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rb[h][j]);
                        sm.Cs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rc[h][j]);
                        ce_o[rho * N + npos<kBf16>(n)] = to_op<op_t>(ce[j]);
                    }
                }
#pragma unroll
                for (int j = 0; j < PPL; ++j)
                    sm.Bwt[(i0 + h * NH + j) * LDR + rho] = to_op<op_t>(rb[h][j] * wd);
            }
        }
    }
    __syncthreads();

    // ---- the chunk's angle total per pair, with its cosine and sine (one
    //      pair per thread)
    if (tid < NH) {
        const float tot = rot ? sm.phi_tot[tid] : 0.0f;
        float ts = 0.0f, tc = 1.0f;
        if (rot) sincosf(tot, &ts, &tc);
        reinterpret_cast<float *>(ws.base + ws.l.phi)[chunk_id * NH + tid] = tot;
        reinterpret_cast<float *>(ws.base + ws.l.cphi)[chunk_id * NH + tid] = tc;
        reinterpret_cast<float *>(ws.base + ws.l.sphi)[chunk_id * NH + tid] = ts;
    }

    // ---- masked band, every tile (the upper ones as zeros), into M
    {
        op_t *m_o = reinterpret_cast<op_t *>(ws.base + ws.l.m) + chunk_id * ROWS * ROWS;
        const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
        const bool skip = a.d_skip != nullptr;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            const int tlast = (16 * tj + 15) / R;
#pragma unroll
            for (int si = 0; si < NT; ++si) {
                if ((tj * NT + si) % 4 != wave) continue;
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
                        if (skip && srow == trow) v += dskip;
                        vals[r] = v;
                    }
                }
                st4(&m_o[trow * ROWS + 16 * si + 4 * g], vals);
            }
        }
    }

    // ---- (B~ w decay)^T rows, coalesced
    {
        op_t *b_o = reinterpret_cast<op_t *>(ws.base + ws.l.bwt) + chunk_id * N * ROWS;
        constexpr int EOP = 16 / static_cast<int>(sizeof(op_t));
        constexpr int PER_ROW = ROWS / EOP;
        for (int v = tid; v < N * PER_ROW; v += kThreads) {
            const int n = v / PER_ROW, q = (v % PER_ROW) * EOP;
            *reinterpret_cast<u32x4 *>(&b_o[n * ROWS + q]) =
                *reinterpret_cast<const u32x4 *>(&sm.Bwt[n * LDR + q]);
        }
    }
}

// ============================================================== state walk
template <typename T, int N, int R, int ROWS>
struct WalkSmem {
    using G = Geo<T, N, 64, R, ROWS>;
    using op_t = typename Op<T>::t;
    static constexpr int P = 64;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;
    static constexpr int LDR = ROWS + PAD;
    struct Set {
        op_t Xt[P * LDR];
        op_t Ms[ROWS * LDR];
        op_t Ce[ROWS * LDN];
        op_t Bwt[N * LDR];
        float cdec;
        float phi[G::NH], cph[G::NH], sph[G::NH];
    };
    Set set[2];
    float fin_c[G::NH], fin_s[G::NH];
};

template <typename T, int N, int R, int ROWS>
struct WalkRaw {
    using G = Geo<T, N, 64, R, ROWS>;
    static constexpr int SZ = sizeof(T);
    static constexpr int MV = ROWS * ROWS * SZ / 16 / kThreads;
    static constexpr int CV = ROWS * N * SZ / 16 / kThreads;
    static_assert(MV >= 1 && CV >= 1, "whole vectors per thread");
    u32x4 x[G::XV];
    u32x4 m[MV], ce[CV], bw[CV];
    float cdec, phi, cph, sph;
};

template <typename T, int N, int R, int ROWS>
__global__ void __launch_bounds__(kThreads, 1)
ssd_walk_kernel(ScanLaunch a, SplitWs ws, int nchunks) {
    constexpr int P = 64;
    using G = Geo<T, N, P, R, ROWS>;
    using S = WalkSmem<T, N, R, ROWS>;
    using RawT = WalkRaw<T, N, R, ROWS>;
    using op_t = typename S::op_t;
    constexpr int KB = Op<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH;
    constexpr int NT = ROWS / 16;
    constexpr int NTN = N / 16;
    constexpr bool kBf16 = sizeof(op_t) == 2;
    constexpr uint32_t SZ = sizeof(T);
    constexpr int EOP = 16 / static_cast<int>(sizeof(op_t));

    extern __shared__ __align__(16) unsigned char smem_raw[];
    S &sm = *reinterpret_cast<S *>(smem_raw);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t bh = blockIdx.x;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;

    // x of this sequence, and this sequence's workspace sections
    const size_t row0 = bb * L * H + hh;
    const size_t rows = L * H - hh;
    const rsrc_t rx = make_rsrc(static_cast<const char *>(a.x) + row0 * P * R * SZ,
                                static_cast<uint32_t>(rows * P * R * SZ));
    const rsrc_t ry = make_rsrc(static_cast<const char *>(a.y) + row0 * P * R * SZ,
                                static_cast<uint32_t>(rows * P * R * SZ));
    const uint32_t tok_x = static_cast<uint32_t>(H * P * R * SZ);
    const size_t c0 = bh * nchunks;
    auto sec = [&](size_t off, size_t per_chunk) {
        return make_rsrc(ws.base + off + c0 * per_chunk,
                         static_cast<uint32_t>(nchunks * per_chunk));
    };
    const rsrc_t rm = sec(ws.l.m, ROWS * ROWS * SZ);
    const rsrc_t rce = sec(ws.l.ce, ROWS * N * SZ);
    const rsrc_t rbw = sec(ws.l.bwt, N * ROWS * SZ);
    const rsrc_t rcd = sec(ws.l.cdec, 4);
    const rsrc_t rph = sec(ws.l.phi, NH * 4);
    const rsrc_t rcp = sec(ws.l.cphi, NH * 4);
    const rsrc_t rsp = sec(ws.l.sphi, NH * 4);

    auto load = [&](int ck, RawT &raw) {
        const uint32_t tok = static_cast<uint32_t>(ck) * QT + my_t;
        const uint32_t ox = tok * tok_x + (wave * 16 * R + sub * G::XE) * SZ;
#pragma unroll
        for (int v = 0; v < G::XV; ++v) raw.x[v] = bld16(rx, ox + 16 * v);
        const uint32_t cm = static_cast<uint32_t>(ck) * (ROWS * ROWS * SZ);
#pragma unroll
        for (int v = 0; v < RawT::MV; ++v) raw.m[v] = bld16(rm, cm + (tid + kThreads * v) * 16);
        const uint32_t cc = static_cast<uint32_t>(ck) * (ROWS * N * SZ);
#pragma unroll
        for (int v = 0; v < RawT::CV; ++v) {
            raw.ce[v] = bld16(rce, cc + (tid + kThreads * v) * 16);
            raw.bw[v] = bld16(rbw, cc + (tid + kThreads * v) * 16);
        }
        raw.cdec = bldf(rcd, static_cast<uint32_t>(ck) * 4);
        const uint32_t cp = static_cast<uint32_t>(ck) * (NH * 4) + (tid % NH) * 4;
        raw.phi = bldf(rph, cp);
        raw.cph = bldf(rcp, cp);
        raw.sph = bldf(rsp, cp);
    };

    auto stage = [&](const RawT &raw, typename S::Set &ss) {
        // X^T from my head_dim slice of x (lane = token)
        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * 16 * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                ss.Xt[p * LDR + my_t * R + r] = to_op<op_t>(elem<T>(raw.x, e));
            }
        }
        // M, Ce, Bwt rows into their padded LDS rows
#pragma unroll
        for (int v = 0; v < RawT::MV; ++v) {
            const int e = (tid + kThreads * v) * EOP;
            *reinterpret_cast<u32x4 *>(&ss.Ms[(e / ROWS) * LDR + e % ROWS]) = raw.m[v];
        }
#pragma unroll
        for (int v = 0; v < RawT::CV; ++v) {
            const int e = (tid + kThreads * v) * EOP;
            *reinterpret_cast<u32x4 *>(&ss.Ce[(e / N) * LDN + e % N]) = raw.ce[v];
            *reinterpret_cast<u32x4 *>(&ss.Bwt[(e / ROWS) * LDR + e % ROWS]) = raw.bw[v];
        }
        if (tid == 0) ss.cdec = raw.cdec;
        if (tid < NH) {
            ss.phi[tid] = raw.phi;
            ss.cph[tid] = raw.cph;
            ss.sph[tid] = raw.sph;
        }
    };

    RawT raw0, raw1;
    load(0, raw0);
    load(1, raw1);

    // state registers: S^T[n][p] tiles, lane holds n = 16i + 4g + r, p = 16w + c;
    // S is kept in the current chunk's frame
    f32x4 st[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int pcol = 16 * wave + c;
    const size_t sbase = (bb * H + hh) * P * N;
    // running wrapped angle of my state pairs n = 16i + 4g + r (i < NTN / 2)
    float phe[NTN / 2][4];
#pragma unroll
    for (int i = 0; i < NTN / 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            phe[i][r] = (rot && a.angle0) ? a.angle0[bh * NH + 16 * i + 4 * g + r] : 0.0f;
    {
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        if (h0 != nullptr) {
            float first = 0.0f;
            if (l0 != nullptr) {
                // carry S = h + (1 - lambda_0) dt_0 last_u   (scan.rs:521-535)
                const size_t i0s = (bb * L) * H + hh;
                first = (1.0f - a.lambda[i0s]) * a.dt[i0s];
            }
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                const size_t o = sbase + pcol * N + 16 * i + 4 * g;
                f32x4 v = *reinterpret_cast<const f32x4 *>(h0 + o);
                if (l0 != nullptr) v += *reinterpret_cast<const f32x4 *>(l0 + o) * first;
                st[i] = v;
            }
            if (rot && a.angle0) {
                // into the first chunk's frame: rotate every pair by angle0
#pragma unroll
                for (int i = 0; i < NTN / 2; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sa, ca;
                        sincosf(phe[i][r], &sa, &ca);
                        const float v1 = st[i][r], v2 = st[i + NTN / 2][r];
                        st[i][r] = v1 * ca - v2 * sa;
                        st[i + NTN / 2][r] = v1 * sa + v2 * ca;
                    }
            }
        }
    }
    for (int i = tid; i < static_cast<int>(sizeof(S) / 4); i += kThreads)
        reinterpret_cast<uint32_t *>(smem_raw)[i] = 0u;
    __syncthreads();

    auto compute = [&](int ck, const typename S::Set &ss) {
        // y^T[p][t] = sum_s X^T[p][s] M[t][s] + sum_n S[p][n] Ce[t][n]
        f32x4 yacc[NT];
        const op_t *xr = &ss.Xt[(16 * wave + c) * LDR];
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            yacc[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
            const op_t *mr = &ss.Ms[(16 * tj + c) * LDR];
            const int tlast = (16 * tj + 15) / R;
            const int send = (tlast + 1) * R < ROWS ? (tlast + 1) * R : ROWS;
            const int nkb = (send + KB - 1) / KB;
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb)
                if (kb < nkb) yacc[tj] = mma_kb(xr + kb * KB, mr + kb * KB, yacc[tj], g);
        }
        if constexpr (kBf16) {
            bf16x8 sa[N / 32];
#pragma unroll
            for (int kb = 0; kb < N / 32; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sa[kb][j] = to_bf16(st[2 * kb][j]);
                    sa[kb][4 + j] = to_bf16(st[2 * kb + 1][j]);
                }
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const op_t *cr = &ss.Ce[(16 * tj + c) * LDN];
#pragma unroll
                for (int kb = 0; kb < N / 32; ++kb)
                    yacc[tj] = mfma_bf16(sa[kb],
                                         *reinterpret_cast<const bf16x8 *>(cr + 32 * kb + 8 * g),
                                         yacc[tj]);
            }
        } else {
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const op_t *cr = &ss.Ce[(16 * tj + c) * LDN];
#pragma unroll
                for (int i = 0; i < NTN; ++i) {
                    const f32x4 bv = *reinterpret_cast<const f32x4 *>(cr + 16 * i + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) yacc[tj] = mfma_f32(st[i][r], bv[r], yacc[tj]);
                }
            }
        }
        const uint32_t tau0 = static_cast<uint32_t>(ck) * QT;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            const int rho = 16 * tj + c;
            const int rr = rho % R;
            const uint32_t tau = tau0 + rho / R;
            const f32x4 v = yacc[tj];
            // rows past the sequence end fall outside the buffer: dropped
            const uint32_t oy = tau * tok_x + ((16 * wave + 4 * g) * R + rr) * SZ;
            if constexpr (R == 1) {
                if constexpr (kBf16) {
                    u32x2 pk;
                    pk[0] = static_cast<unsigned int>(from_f32<bf16_t>(v[0]).bits) |
                            (static_cast<unsigned int>(from_f32<bf16_t>(v[1]).bits) << 16);
                    pk[1] = static_cast<unsigned int>(from_f32<bf16_t>(v[2]).bits) |
                            (static_cast<unsigned int>(from_f32<bf16_t>(v[3]).bits) << 16);
                    bst8(pk, ry, oy);
                } else {
                    bst16(u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                __float_as_uint(v[2]), __float_as_uint(v[3])},
                          ry, oy);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (kBf16)
                        bst2(from_f32<bf16_t>(v[r]).bits, ry, oy + r * R * SZ);
                    else
                        bst4(__float_as_uint(v[r]), ry, oy + r * R * SZ);
                }
            }
        }
        // S = decay * S + Bwt X, then into the next chunk's frame
        const float dec = ss.cdec;
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            f32x4 acc = st[i] * dec;
            const op_t *ar = &ss.Bwt[(16 * i + c) * LDR];
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb) acc = mma_kb(ar + kb * KB, xr + kb * KB, acc, g);
            st[i] = acc;
        }
        if (rot) {
#pragma unroll
            for (int i = 0; i < NTN / 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = 16 * i + 4 * g + r;
                    const float cp = ss.cph[n], sp = ss.sph[n];
                    const float v1 = st[i][r], v2 = st[i + NTN / 2][r];
                    st[i][r] = v1 * cp - v2 * sp;
                    st[i + NTN / 2][r] = v1 * sp + v2 * cp;
                    phe[i][r] = wrap_angle(phe[i][r] + ss.phi[n]);
                }
        }
    };

    stage(raw0, sm.set[0]);
    __syncthreads();
    auto step = [&](int ck, typename S::Set &cur, typename S::Set &nxt, RawT &mine,
                    const RawT &next_raw) {
        load(ck + 2, mine);   // past the last chunk this reads zeros
        compute(ck, cur);
        if (ck + 1 < nchunks) stage(next_raw, nxt);
        lds_barrier();
    };
    for (int ck = 0; ck < nchunks; ck += 2) {
        step(ck, sm.set[0], sm.set[1], raw0, raw1);
        if (ck + 1 < nchunks) step(ck + 1, sm.set[1], sm.set[0], raw1, raw0);
    }

    // ---- boundary state in the global frame (scan.rs:270-288, 599-638)
    if (rot && wave == 0 && c == 0) {
#pragma unroll
        for (int i = 0; i < NTN / 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = 16 * i + 4 * g + r;
                float sa, ca;
                sincosf(phe[i][r], &sa, &ca);
                sm.fin_c[n] = ca;
                sm.fin_s[n] = sa;
                if (a.angle_out) a.angle_out[bh * NH + n] = phe[i][r];
            }
    }
    if (!rot) {
        for (int n = tid; n < NH; n += kThreads) {
            sm.fin_c[n] = 1.0f;
            sm.fin_s[n] = 0.0f;
        }
    }
    __syncthreads();
    if (a.h_out != nullptr) {
        if (rot) {
#pragma unroll
            for (int i = 0; i < NTN / 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = 16 * i + 4 * g + r;
                    const float ca = sm.fin_c[n], sa = sm.fin_s[n];
                    const float v1 = st[i][r], v2 = st[i + NTN / 2][r];
                    st[i][r] = v1 * ca + v2 * sa;
                    st[i + NTN / 2][r] = -v1 * sa + v2 * ca;
                }
        }
#pragma unroll
        for (int i = 0; i < NTN; ++i)
            *reinterpret_cast<f32x4 *>(a.h_out + sbase + pcol * N + 16 * i + 4 * g) = st[i];
    }
    if (a.last_u_out != nullptr) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T with B~ rotated by the final angle
        const typename S::Set &ls = sm.set[(nchunks - 1) & 1];
        const int tl = static_cast<int>((L - 1) - static_cast<size_t>(nchunks - 1) * QT);
        const T *bl = static_cast<const T *>(a.b) + ((bb * L + (L - 1)) * H + hh) * N * R;
        for (int it = tid; it < P * N; it += kThreads) {
            const int p = it / N;
            const int n = it - p * N;
            const int i = n % NH;
            const float ca = sm.fin_c[i], sa = sm.fin_s[i];
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v1 = to_f32(bl[i * R + r]), v2 = to_f32(bl[(i + NH) * R + r]);
                const float bt = n < NH ? v1 * ca + v2 * sa : -v1 * sa + v2 * ca;
                acc += op_f32(ls.Xt[p * LDR + tl * R + r]) * bt;
            }
            a.last_u_out[sbase + it] = acc;
        }
    }
}

template <typename T, int N, int R, int ROWS>
hipError_t launch_pair(const ScanLaunch &a, char *ws_base, hipStream_t s) {
    using G = Geo<T, N, 64, R, ROWS>;
    const int nchunks = static_cast<int>((a.seq + G::QT - 1) / G::QT);
    const size_t bh = a.batch * a.heads;
    SplitWs ws{ws_base, split_layout(bh, nchunks, ROWS, N, sizeof(T))};
    hipLaunchKernelGGL((ssd_chunk_kernel<T, N, R, ROWS>), dim3(bh * nchunks), dim3(kThreads), 0,
                       s, a, ws, nchunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    using Sm = WalkSmem<T, N, R, ROWS>;
    auto kern = ssd_walk_kernel<T, N, R, ROWS>;
    static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(sizeof(Sm)));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(bh), dim3(kThreads), sizeof(Sm), s, a, ws, nchunks);
    return hipGetLastError();
}

template <typename T, int ROWS>
hipError_t launch_t(const ScanLaunch &a, char *ws, hipStream_t s) {
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_pair<T, 128, 1, ROWS>(a, ws, s);
        if (r == 2) return launch_pair<T, 128, 2, ROWS>(a, ws, s);
        if (r == 4) return launch_pair<T, 128, 4, ROWS>(a, ws, s);
    } else if (n == 64) {
        if (r == 1) return launch_pair<T, 64, 1, ROWS>(a, ws, s);
        if (r == 2) return launch_pair<T, 64, 2, ROWS>(a, ws, s);
        if (r == 4) return launch_pair<T, 64, 4, ROWS>(a, ws, s);
    }
    return hipErrorNotSupported;
}

}  // namespace

size_t scan_split_workspace(const ScanLaunch &a) {
    if (!scan_fast_supported(a)) return 0;
    const size_t rows = a.bf16 ? 64 : 32;
    const size_t qt = rows / a.rank;
    const size_t nchunks = (a.seq + qt - 1) / qt;
    return split_layout(a.batch * a.heads, nchunks, rows, a.d_state, a.bf16 ? 2 : 4).total;
}

hipError_t launch_scan_split(const ScanLaunch &a, void *workspace, hipStream_t stream) {
    if (!scan_fast_supported(a)) return hipErrorNotSupported;
    char *ws = static_cast<char *>(workspace);
    if (a.bf16) return launch_t<bf16_t, 64>(a, ws, stream);
    return launch_t<float, 32>(a, ws, stream);
}

}  // namespace m3
