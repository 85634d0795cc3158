// Chunked SSD scan for gfx950, specialised for the common shapes:
// head_dim 64, d_state 64 or 128, MIMO rank 1, 2 or 4, f32 or bf16 storage,
// 16-byte aligned operands.  Other shapes take the generic kernel in
// ssd_scan.hip.  Both restate src/ssm/scan.rs:116-291 (ssd_chunked) and
// 458-638 (mamba3_scan) and are checked against the same oracle.
//
// One workgroup per (batch, head) walks the sequence chunk by chunk; the f32
// state S never leaves registers.  Per chunk:
//
//   stage  Lane = token.  Wave w loads, for its token, its rotation pairs of
//          B and C, the matching theta slice, its head_dim slice of x, and
//          dt/lambda of the token and the next one (raw buffer loads: past the
//          sequence end they read as zeros).  The in-chunk prefixes -- the
//          log-decay cumsum (ops/scan.rs:18-51) and the frame angle cumsum of
//          dt*theta -- are DPP scans across the wave's lanes, so each lane ends
//          up with its own token's decay weights, trapezoid weights
//          (fused.rs:2483-2503) and wrapped angle (elemwise.rs:349).  B and C
//          are rotated by -phi in registers (fused.rs:588-619) and written to
//          LDS as MFMA operands; so are (B~ * w * decay-to-end)^T and X^T.  The
//          inputs of the chunk after next are requested before the stage.
//   P4     MFMA: the masked C B^T band (ssd_band, fused.rs:2044-2070) into LDS,
//          and the state advance S = exp(dA) S + (w-decayed B~)^T X
//          (scan.rs:207-251, an O(C) walk in place of the O(C^2) transfer).
//   P5     MFMA: y = exp(acum) (C~ S) + (band o C B^T) X (scan.rs:253-263;
//          the skip D rides on the band's diagonal), then the store.
//
// Two shapes of workgroup:
//   NW = 4  wave w owns head_dim columns [16w, 16w+16) and the whole state of
//           those columns.
//   NW = 8  (bf16, d_state 128) wave w = (p-tile w%4, half w/4) owns n-tiles
//           [4*half, 4*half+4) of the state of its sixteen columns, produces y
//           for t-tiles {2*half, 2*half+1}, and gets the other half of the
//           state it needs for the carry-in product as bf16 through LDS.  Two
//           waves per SIMD hide each other's LDS and MFMA latency.
//
// The LDS operand set is double-buffered, so the stage of chunk k+1 runs in
// the same phase as P5 of chunk k: two workgroup barriers per chunk.
#include "scan_common.hpp"

namespace m3 {

namespace {

using namespace scan;

template <typename T, int N, int P, int R, int ROWS, int NW>
struct Smem {
    using G = Geo<T, N, P, R, ROWS, NW>;
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;    // pitch of [row][n] operands
    static constexpr int LDR = ROWS + PAD; // pitch of [*][row] operands
    struct Set {
        op_t Bs[ROWS * LDN];    // B~[rho][npos(n)]
        op_t Cs[ROWS * LDN];    // C~[rho][npos(n)]
        op_t Bwt[N * LDR];      // (B~ * w * decay-to-end)^T [n][rho]
        op_t Xt[P * LDR];       // X^T [p][rho]
        float acum[G::QT], gw[G::QT], ww[G::QT], eac[G::QT];
    };
    Set set[2];
    op_t Ms[ROWS * LDR];        // masked band (C~ B~^T o L)[rho_t][rho_s]
    // NW = 8: each wave's half of S_k as bf16 MFMA A-operand slices,
    // [p-tile][half][k-block within the half][lane]
    bf16x8 xchg[NW == 8 ? 4 * 2 * (N / 64) * 64 : 1];
};

template <typename T, int N, int P, int R, int ROWS, int NW>
__global__ void __launch_bounds__(64 * NW, 1)
ssd_scan_fast_kernel(ScanLaunch a, int nchunks) {
    using G = Geo<T, N, P, R, ROWS, NW>;
    using S = Smem<T, N, P, R, ROWS, NW>;
    using RawT = Raw<T, N, P, R, ROWS, NW>;
    using op_t = typename S::op_t;
    constexpr int THREADS = 64 * NW;
    constexpr int KB = Op<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL;
    constexpr int NT = ROWS / 16;    // row tiles per chunk
    constexpr int NTN = N / 16;      // state-column tiles
    constexpr bool kBf16 = sizeof(op_t) == 2;
    constexpr uint32_t SZ = sizeof(T);
    static_assert(NW == 4 || (NW == 8 && kBf16), "eight waves split the bf16 state in halves");
    // state n-tiles held by a wave, and the t-tiles of y it produces
    constexpr int SNT = NW == 8 ? NTN / 2 : NTN;
    constexpr int YT = NW == 8 ? NT / 2 : NT;

    extern __shared__ __align__(16) unsigned char smem_raw[];
    S &sm = *reinterpret_cast<S *>(smem_raw);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int pt = wave & 3;                       // my p-tile (columns [16pt, 16pt+16))
    const int hf = NW == 8 ? (wave >> 2) : 0;      // my state half / y half
    const int n0 = hf * SNT;                       // my first state n-tile
    const int t0 = hf * YT;                        // my first y t-tile

    const size_t H = a.heads, L = a.seq;
    const size_t bb = blockIdx.x / H, hh = blockIdx.x % H;
    const bool rot = a.theta != nullptr;

    // lane = token: my token within the chunk, my pairs [i0, i0 + PPL)
    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);

    RawT raw0, raw1;
    load_chunk<T, N, P, R, ROWS, NW>(rs, 0, wave, lane, raw0);
    load_chunk<T, N, P, R, ROWS, NW>(rs, 1, wave, lane, raw1);

    // zero the operand buffers once: pads and the never-written upper band tiles
    {
        uint32_t *z = reinterpret_cast<uint32_t *>(smem_raw);
        const int words = static_cast<int>(sizeof(S) / 4);
        for (int i = tid; i < words; i += THREADS) z[i] = 0u;
    }

    // state registers: S^T[n][p] tiles n-tile n0 + i, lane holds
    // n = 16(n0 + i) + 4g + r, p = 16pt + c
    f32x4 st[SNT];
#pragma unroll
    for (int i = 0; i < SNT; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int pcol = 16 * pt + c;
    const size_t sbase = (bb * H + hh) * P * N;
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
            for (int i = 0; i < SNT; ++i) {
                const size_t o = sbase + pcol * N + 16 * (n0 + i) + 4 * g;
                f32x4 v = *reinterpret_cast<const f32x4 *>(h0 + o);
                if (l0 != nullptr) v += *reinterpret_cast<const f32x4 *>(l0 + o) * first;
                st[i] = v;
            }
        }
    }
    // running wrapped frame angle entering the chunk, for my pairs
    float phi0[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j)
        phi0[j] = (rot && a.angle0) ? a.angle0[(bb * H + hh) * NH + i0 + j] : 0.0f;

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const bool skip = a.d_skip != nullptr;
    __syncthreads();

    // ---------------------------------------------------------------- stage
    auto stage = [&](int ck, const RawT &cur, typename S::Set &ss) {
        const size_t tau = static_cast<size_t>(ck) * QT + my_t;
        const bool live = tok_lane && tau < L;
        // per-token scalars: log decay, trapezoid weights, in-chunk cumsum
        float av, gv, wv;
        if (a.mode_raw) {
            av = cur.s0 * A;
            gv = cur.s1 * cur.s0;                        // fused.rs:2494
            wv = gv + (1.0f - cur.s3) * cur.s2;          // fused.rs:2496-2498
        } else {
            av = cur.s0;
            gv = cur.s1;
            wv = cur.s2;
        }
        if (!live) av = gv = wv = 0.f;
        const float acum = seg_scan<G::SW>(av);
        const float last =
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        const float wd = dexp<kBf16>(last - acum) * wv;   // exp_decay(last, acum, w)
        if (wave == 0 && sub == 0 && tok_lane) {
            ss.acum[my_t] = acum;
            ss.gw[my_t] = gv;
            ss.ww[my_t] = wv;
            ss.eac[my_t] = dexp<kBf16>(acum);             // exp_decay(acum)
        }
        // frame angle: cumsum of dt*theta within the chunk on top of the
        // running wrapped angle (the reference cumsums it absolutely in f32
        // and wraps afterwards, scan.rs:490-497)
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
                const float phi = wrap_angle(phi0[j] + pre);
                const float tot = __shfl(pre, sub * G::SW + QT - 1, 64);
                phi0[j] = wrap_angle(phi0[j] + tot);
                if (a.angle_out && tok_lane && tau == L - 1)
                    a.angle_out[(bb * H + hh) * NH + i0 + j] = phi;
                if constexpr (kBf16) {
                    // the hardware sine takes revolutions; |phi| <= pi
                    const float rev = phi * 0.15915494309189533577f;
                    sn[j] = __builtin_amdgcn_sinf(rev);
                    cs[j] = __builtin_amdgcn_cosf(rev);
                } else {
                    sincosf(phi, &sn[j], &cs[j]);
                }
            }
        }
        if (tok_lane) {
            // X^T from my head_dim slice of x
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / NW) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                ss.Xt[p * LDR + my_t * R + r] = to_op<op_t>(elem<T>(cur.x, e));
            }
            // rotate B and C by -phi (fused.rs:610-617); identity without theta
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
                        // groups of four consecutive columns stay contiguous under npos
#pragma unroll
                        for (int q = 0; q < PPL; q += 4) {
                            const int n = i0 + h * NH + q;
                            st4(&ss.Bs[rho * LDN + npos<kBf16>(n)], &rb[h][q]);
                            st4(&ss.Cs[rho * LDN + npos<kBf16>(n)], &rc[h][q]);
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < PPL; ++j) {
                            const int n = i0 + h * NH + j;
                            ss.Bs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rb[h][j]);
                            ss.Cs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rc[h][j]);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < PPL; ++j)
                        ss.Bwt[(i0 + h * NH + j) * LDR + rho] = to_op<op_t>(rb[h][j] * wd);
                }
            }
        }
    };

    // ---------------------------------------------------------------- P4
    // the band into Ms; my half of S_k to the exchange (NW = 8) or as the
    // carry-in A operand (kept in registers); the state advance
    auto p4 = [&](const typename S::Set &ss, bf16x8 *sa, f32x4 *ycar) {
        int idx = 0;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            const int tlast = (16 * tj + 15) / R;
#pragma unroll
            for (int si = 0; si < NT; ++si) {
                if ((16 * si) / R > tlast) continue;
                if ((idx++) % NW != wave) continue;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const op_t *ar = &ss.Bs[(16 * si + c) * LDN];
                const op_t *br = &ss.Cs[(16 * tj + c) * LDN];
#pragma unroll
                for (int kb = 0; kb < N / KB; ++kb)
                    acc = mma_kb(ar + kb * KB, br + kb * KB, acc, g);
                const int trow = 16 * tj + c;
                const int tt = trow / R;
                const float at = ss.acum[tt];
                float vals[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int srow = 16 * si + 4 * g + r;
                    const int ts = srow / R;
                    float v = 0.0f;
                    if (ts <= tt) {
                        const float wgt = (ts == tt) ? ss.gw[ts] : ss.ww[ts];
                        v = acc[r] * wgt * dexp<kBf16>(at - ss.acum[ts]);
                    }
                    // the skip D x rides on the band's diagonal (scan.rs:593-597)
                    if (skip && srow == trow) v += dskip;
                    vals[r] = v;
                }
                st4(&sm.Ms[trow * LDR + 16 * si + 4 * g], vals);
            }
        }

        // S_k for the carry-in product.  bf16: as MFMA A-operand slices (k = n
        // in the npos column order), for eight waves also to the exchange;
        // f32: the product itself, before the advance overwrites S_k.
        if constexpr (kBf16) {
#pragma unroll
            for (int kb = 0; kb < SNT / 2; ++kb) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sa[kb][j] = to_bf16(st[2 * kb][j]);
                    sa[kb][4 + j] = to_bf16(st[2 * kb + 1][j]);
                }
                if constexpr (NW == 8) sm.xchg[((pt * 2 + hf) * (SNT / 2) + kb) * 64 + lane] = sa[kb];
            }
        } else {
#pragma unroll
            for (int q = 0; q < YT; ++q) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const op_t *cr = &ss.Cs[(16 * (t0 + q) + c) * LDN];
#pragma unroll
                for (int i = 0; i < NTN; ++i) {
                    const f32x4 bv = *reinterpret_cast<const f32x4 *>(cr + 16 * i + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc = mfma_f32(st[i][r], bv[r], acc);
                }
                ycar[q] = acc;
            }
        }

        // state advance: S^T = exp(dA) S^T + (B~ w decay)^T X
        const float edA = dexp<kBf16>(ss.acum[QT - 1]);
        const op_t *xr = &ss.Xt[pcol * LDR];
#pragma unroll
        for (int i = 0; i < SNT; ++i) {
            f32x4 acc = st[i] * edA;
            const op_t *ar = &ss.Bwt[(16 * (n0 + i) + c) * LDR];
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb)
                acc = mma_kb(ar + kb * KB, xr + kb * KB, acc, g);
            st[i] = acc;
        }
    };

    // ---------------------------------------------------------------- P5
    // y^T[p][t] = exp(acum_t) sum_n S_k[p][n] C~[t][n] + sum_s X^T[p][s] M[t][s]
    auto p5 = [&](int ck, const typename S::Set &ss, const bf16x8 *sa, const f32x4 *ycar) {
        constexpr int KH = kBf16 ? SNT / 2 : 1;   // 32-wide k-blocks of one state half
        f32x4 yacc[YT];
#pragma unroll
        for (int q = 0; q < YT; ++q) {
            const int tj = t0 + q;
            f32x4 acc;
            if constexpr (kBf16) {
                acc = f32x4{0.f, 0.f, 0.f, 0.f};
                const op_t *cr = &ss.Cs[(16 * tj + c) * LDN + 8 * g];
#pragma unroll
                for (int kb = 0; kb < KH; ++kb)
                    acc = mfma_bf16(sa[kb], *reinterpret_cast<const bf16x8 *>(cr + 32 * (hf * KH + kb)),
                                    acc);
                if constexpr (NW == 8) {
                    const int oh = 1 - hf;   // the partner wave's half
#pragma unroll
                    for (int kb = 0; kb < KH; ++kb)
                        acc = mfma_bf16(sm.xchg[((pt * 2 + oh) * KH + kb) * 64 + lane],
                                        *reinterpret_cast<const bf16x8 *>(cr + 32 * (oh * KH + kb)), acc);
                }
            } else {
                acc = ycar[q];
            }
            acc = acc * ss.eac[(16 * tj + c) / R];
            const op_t *mr = &sm.Ms[(16 * tj + c) * LDR];
            const op_t *xr = &ss.Xt[pcol * LDR];
            const int tlast = (16 * tj + 15) / R;
            const int send = (tlast + 1) * R < ROWS ? (tlast + 1) * R : ROWS;
            const int nkb = (send + KB - 1) / KB;
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb)
                if (kb < nkb) acc = mma_kb(xr + kb * KB, mr + kb * KB, acc, g);
            yacc[q] = acc;
        }
        const uint32_t tau0 = static_cast<uint32_t>(ck) * QT;
#pragma unroll
        for (int q = 0; q < YT; ++q) {
            const int rho = 16 * (t0 + q) + c;
            const int rr = rho % R;
            const uint32_t tau = tau0 + rho / R;
            const f32x4 v = yacc[q];
            // rows past the sequence end fall outside the buffer: dropped
            const uint32_t oy = tau * rs.tok_x + ((16 * pt + 4 * g) * R + rr) * SZ;
            if constexpr (R == 1) {
                if constexpr (kBf16) {
                    u32x2 pk;
                    pk[0] = pack_bf16x2(v[0], v[1]);
                    pk[1] = pack_bf16x2(v[2], v[3]);
                    bst8(pk, rs.y, oy);
                } else {
                    bst16(u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                __float_as_uint(v[2]), __float_as_uint(v[3])},
                          rs.y, oy);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (kBf16)
                        bst2(from_f32<bf16_t>(v[r]).bits, rs.y, oy + r * R * SZ);
                    else
                        bst4(__float_as_uint(v[r]), rs.y, oy + r * R * SZ);
                }
            }
        }
    };

    // chunk ck uses operand set ck % 2 and raw registers ck % 2; the inputs of
    // chunk ck + 2 are requested while chunk ck + 1 is staged
    stage(0, raw0, sm.set[0]);
    lds_barrier();
    auto step = [&](int ck, typename S::Set &cur, typename S::Set &nxt, RawT &mine,
                    const RawT &next_raw) {
        bf16x8 sa[kBf16 ? SNT / 2 : 1];
        f32x4 ycar[kBf16 ? 1 : YT];
        p4(cur, sa, ycar);
        lds_barrier();
        p5(ck, cur, sa, ycar);
        load_chunk<T, N, P, R, ROWS, NW>(rs, ck + 2, wave, lane, mine);   // zeros past the end
        if (ck + 1 < nchunks) stage(ck + 1, next_raw, nxt);
        lds_barrier();
    };
    for (int ck = 0; ck < nchunks; ck += 2) {
        step(ck, sm.set[0], sm.set[1], raw0, raw1);
        if (ck + 1 < nchunks) step(ck + 1, sm.set[1], sm.set[0], raw1, raw0);
    }

    // ---- boundary state (scan.rs:270-288, 599-638)
    if (a.h_out != nullptr) {
#pragma unroll
        for (int i = 0; i < SNT; ++i)
            *reinterpret_cast<f32x4 *>(a.h_out + sbase + pcol * N + 16 * (n0 + i) + 4 * g) = st[i];
    }
    if (a.last_u_out != nullptr) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T, from the final chunk's LDS tiles
        const typename S::Set &ls = sm.set[(nchunks - 1) & 1];
        const int tl = static_cast<int>((L - 1) - static_cast<size_t>(nchunks - 1) * QT);
        for (int it = tid; it < P * N; it += THREADS) {
            const int p = it / N;
            const int n = it - p * N;
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = tl * R + r;
                acc += op_f32(ls.Xt[p * LDR + rho]) * op_f32(ls.Bs[rho * LDN + npos<kBf16>(n)]);
            }
            a.last_u_out[sbase + it] = acc;
        }
    }
}

template <typename T, int N, int R, int ROWS, int NW>
hipError_t launch_one(const ScanLaunch &a, hipStream_t s) {
    constexpr int P = 64;
    using Sm = Smem<T, N, P, R, ROWS, NW>;
    using G = Geo<T, N, P, R, ROWS, NW>;
    const int nchunks = static_cast<int>((a.seq + G::QT - 1) / G::QT);
    const size_t smem = sizeof(Sm);
    auto kern = ssd_scan_fast_kernel<T, N, P, R, ROWS, NW>;
    static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(smem));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(a.batch * a.heads), dim3(64 * NW), smem, s, a, nchunks);
    return hipGetLastError();
}

template <typename T, int ROWS, int NW128>
hipError_t launch_t(const ScanLaunch &a, hipStream_t s) {
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_one<T, 128, 1, ROWS, NW128>(a, s);
        if (r == 2) return launch_one<T, 128, 2, ROWS, NW128>(a, s);
        if (r == 4) return launch_one<T, 128, 4, ROWS, NW128>(a, s);
    } else if (n == 64) {
        if (r == 1) return launch_one<T, 64, 1, ROWS, 4>(a, s);
        if (r == 2) return launch_one<T, 64, 2, ROWS, 4>(a, s);
        if (r == 4) return launch_one<T, 64, 4, ROWS, 4>(a, s);
    }
    return hipErrorNotSupported;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool scan_fast_supported(const ScanLaunch &a) {
    if (a.head_dim != 64) return false;
    if (a.d_state != 64 && a.d_state != 128) return false;
    if (a.rank != 1 && a.rank != 2 && a.rank != 4) return false;
    if (!aligned16(a.x) || !aligned16(a.b) || !aligned16(a.c) || !aligned16(a.y)) return false;
    if (a.theta != nullptr && !aligned16(a.theta)) return false;
    // the state is read and written as 16-byte vectors
    for (const float *p : {a.h0, a.last_u0, a.init_state, static_cast<const float *>(a.h_out)})
        if (p != nullptr && !aligned16(p)) return false;
    // buffer offsets are 32-bit: a batch's rows, plus two chunks of overrun,
    // must stay below 2 GiB for the widest per-token row (b and c)
    const size_t esz = a.bf16 ? 2 : 4;
    const size_t row = a.d_state * a.rank * esz;
    if ((a.seq + 128) * a.heads * row >= (size_t(1) << 31)) return false;
    // theta rows at their own token stride: whole 16-byte pieces, rows that
    // do not overlap, the same 32-bit bound
    if (a.theta != nullptr && a.theta_stride != 0 &&
        (a.theta_stride * esz % 16 != 0 || a.theta_stride < a.heads * (a.d_state / 2) ||
         (a.seq + 128) * a.theta_stride * esz >= (size_t(1) << 31)))
        return false;
    return true;
}

hipError_t launch_scan_fast(const ScanLaunch &a, hipStream_t stream) {
    if (!scan_fast_supported(a)) return hipErrorNotSupported;
    if (a.bf16) return launch_t<bf16_t, 64, 8>(a, stream);
    return launch_t<float, 32, 4>(a, stream);
}

}  // namespace m3
