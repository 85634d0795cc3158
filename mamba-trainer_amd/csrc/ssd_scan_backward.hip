// Backward of the chunked SSD scan (mamba3_scan, src/ssm/scan.rs:458-638) for
// gfx950: the gradient the reference obtains by autodiff through the composed
// scan, whose hand-written adjoints are ssd_band_backward
// (src/tensor/ops/fused.rs:2080-2138), exp_decay_backward (2326-2382) and
// trapezoid_weights_backward (2513-2549).  Shapes as the chunk-parallel
// forward: head_dim 64, d_state 64/128, rank 1/2/4; f32 or bf16 storage,
// f32 arithmetic (MFMA f32 16x16x4 over f32 operands in LDS).
//
// Chunks of 32 rows (token, rank); 64 for bf16 storage with d_state 64.  In
// chunk k's own rotating frame, with alpha the in-chunk inclusive cumsum of a = dt A, K_ts = W_ts e^{alpha_t -
// alpha_s} (W = g on the token diagonal, w below it), CB = C~ B~^T, M = CB o K,
// wbar_s = e^{alpha_E - alpha_s} w_s, S_k the state entering the chunk and
// Gh_k = dL/d(e_k S_k + U_k) = R(-Phi_k) G_{k+1}:
//
//   dX       = M^T dY + D dY + diag(wbar) B~ Gh^T
//   dC~      = (dY X^T o K) B~ + diag(e^alpha) dY S
//   dB~      = (dY X^T o K)^T C~ + diag(wbar) X Gh
//   G_k      = e_k Gh_k + (diag(e^alpha) dY)^T C~            (reverse state pass)
//   dalpha_t = sum_{s<t} L_ts - sum_{t'>t} L_t't + e^{alpha_t} dy_t . (S C~_t)
//              - wbar_t x_t . (Gh B~_t)   (+ the alpha_E terms on the last row),
//              L = dM o M;  da = in-chunk reverse cumsum of dalpha
//   dphi_t   = sum_pairs dB~1 B~2 - dB~2 B~1 + dC~1 C~2 - dC~2 C~1, invariant
//              under the frame rotation, so the global angle gradient is its
//              reverse cumsum over the whole sequence.
//
// Launches: bwd_passes_kernel (the forward recurrence giving S_k, each
// chunk's U_k, the forward's chunk state, formed in place with f32 operands;
// and the reverse one giving G and Gh per chunk, with each chunk's V_k, its
// direct share of G, and dh0 / dlast_u0; side by side), bwd_chunk_kernel (dx, db, dc and
// the per-token da, dg, dw and angle sums), bwd_angle_kernel (the angle sums
// of later chunks), bwd_token_kernel (dtheta, ddt, dlambda: trapezoid_weights
// backward, the decay and angle chains) and bwd_head_kernel (da_log, dD).
#include <algorithm>

#include "scan_common.hpp"

namespace m3 {

namespace {

constexpr int kP = 64;
constexpr int kWaves = 16;
constexpr int kBT = 64 * kWaves;

struct BwdArgs {
    const void *dy;           // [B,T,H,P,R]
    const float *dh_out;      // [B,H,P,N] or null
    const float *dangle_out;  // [B,H,N/2] or null
    const float *dlast_u_out; // [B,H,P,N] or null
    void *dx, *db, *dc;       // storage type
    float *ddt, *dlambda;     // [B,T,H]
    float *da_log;            // [H]
    void *dtheta;             // [B,T,H,N/2] or null
    float *dd_skip;           // [H] or null
    float *dh0, *dlast_u0;    // [B,H,P,N] or null
    float *dangle0;           // [B,H,N/2] or null
};

// Backward workspace, 256-byte aligned sections.  Per (batch, head, chunk):
// S_k and Gh_k as f32 [p-tile][n-tile][lane][4] MFMA D-layout records of the
// [P][N] state and the chunk decay e_k.
// With an upstream gradient of the outgoing last_u: the angle seed (that
// gradient's angle term plus dL/dangle) and the last token's dx and db terms.
struct BwdLayout {
    size_t s, gh, eda, cin, ctot, off, da, dg, dw, pd, pa, pfirst;
    size_t seed, lux, lub, total;
};

size_t balign(size_t v) { return (v + 255) & ~size_t(255); }

BwdLayout bwd_layout(size_t bh, size_t nck, size_t seq, size_t n, size_t r) {
    const size_t bhk = bh * nck, rec = bhk * kP * n * 4, pairs = bhk * (n / 2) * 4;
    BwdLayout l;
    size_t o = 0;
    l.s = o;      o = balign(o + rec);
    l.gh = o;     o = balign(o + rec);
    l.eda = o;    o = balign(o + bhk * 4);
    l.cin = o;    o = balign(o + bh * seq * (n / 2) * 4);
    l.ctot = o;   o = balign(o + pairs);
    l.off = o;    o = balign(o + pairs);
    l.da = o;     o = balign(o + bh * seq * 4);
    l.dg = o;     o = balign(o + bh * seq * 4);
    l.dw = o;     o = balign(o + bh * seq * 4);
    l.pd = o;     o = balign(o + bhk * 4);
    l.pa = o;     o = balign(o + bhk * 4);
    l.pfirst = o; o = balign(o + bh * (n / 32) * 4);
    l.seed = o;   o = balign(o + bh * (n / 2) * 4);
    l.lux = o;    o = balign(o + bh * kP * r * 4);
    l.lub = o;    o = balign(o + bh * n * r * 4);
    l.total = o;
    return l;
}

struct BwdWs {
    float *s, *gh, *eda;
    float *cin, *ctot, *off, *da, *dg, *dw, *pd, *pa, *pfirst;
    float *seed, *lux, *lub;
};

// element access in the storage type
template <typename T> __device__ __forceinline__ float ldv(const void *p, size_t i);
template <> __device__ __forceinline__ float ldv<float>(const void *p, size_t i) {
    return static_cast<const float *>(p)[i];
}
template <> __device__ __forceinline__ float ldv<bf16_t>(const void *p, size_t i) {
    return to_f32(static_cast<const bf16_t *>(p)[i]);
}
template <typename T> __device__ __forceinline__ void stv(void *p, size_t i, float v);
template <> __device__ __forceinline__ void stv<float>(void *p, size_t i, float v) {
    static_cast<float *>(p)[i] = v;
}
template <> __device__ __forceinline__ void stv<bf16_t>(void *p, size_t i, float v) {
    static_cast<bf16_t *>(p)[i] = from_f32<bf16_t>(v);
}

// Four elements i, i + R, i + 2R, i + 3R in the storage type: one 16-byte
// (f32) or 8-byte (bf16) store when they are adjacent (rank 1; i is then a
// multiple of 4 in a 16-byte aligned buffer), else four scalar stores.
template <typename T, int R>
__device__ __forceinline__ void st4(void *p, size_t i, f32x4 v) {
    if constexpr (R == 1) {
        if constexpr (sizeof(T) == 4) {
            *reinterpret_cast<f32x4 *>(static_cast<float *>(p) + i) = v;
        } else {
            bf16x4 h;
#pragma unroll
            for (int r = 0; r < 4; ++r) h[r] = to_bf16(v[r]);
            *reinterpret_cast<bf16x4 *>(static_cast<bf16_t *>(p) + i) = h;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) stv<T>(p, i + r * R, v[r]);
    }
}

// (p, n) of element e of a [p-tile][n-tile][lane][4] MFMA D-layout record
__device__ __forceinline__ void dl_pn(int e, int ntn, int &p, int &n) {
    const int r = e & 3, lane = (e >> 2) & 63, tile = e >> 8;
    const int i = tile % ntn, pt = tile / ntn;
    p = 16 * pt + (lane & 15);
    n = 16 * i + 4 * (lane >> 4) + r;
}

__device__ __forceinline__ float clamp_exp(float d) {
    return expf(fminf(fmaxf(d, -60.0f), 0.0f));
}

template <bool PRECISE>
__device__ __forceinline__ void sincos_any(float x, float &s, float &c) {
    if constexpr (PRECISE) {
        sincosf(x, &s, &c);
    } else {
        const float rev = wrap_angle(x) * 0.15915494309189533577f;
        s = __builtin_amdgcn_sinf(rev);
        c = __builtin_amdgcn_cosf(rev);
    }
}

// D(16x16) += A(16 x K) B(K x 16) in f32: A(m, k) = a[m * am + k * ak],
// B(k, n) = b[k * bk + n * bn]; lane (c, g) supplies A(c, k0+g), B(k0+g, c).
// The operands of up to sixteen MFMAs are read from LDS together and the
// MFMAs then issue back to back (one LDS wait per batch, not per MFMA).
template <int K>
__device__ __forceinline__ f32x4 mma_f32(const float *a, int am, int ak, const float *b, int bk,
                                         int bn, f32x4 acc, int c, int g) {
    static_assert(K % 4 == 0, "K");
    constexpr int KB = K / 4 < 16 ? K / 4 : 16;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 4 * KB) {
        float av[KB], bv[KB];
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const int k = k0 + 4 * j + g;
            av[j] = a[c * am + k * ak];
            bv[j] = b[k * bk + c * bn];
        }
#pragma unroll
        for (int j = 0; j < KB; ++j) acc = mfma_f32(av[j], bv[j], acc);
    }
    return acc;
}

// Two products sharing the B operand: D0 += A0 B, D1 += A1 B.
template <int K>
__device__ __forceinline__ void mma2_f32(const float *a0, const float *a1, int am, int ak,
                                         const float *b, int bk, int bn, f32x4 &d0, f32x4 &d1,
                                         int c, int g) {
    static_assert(K % 4 == 0, "K");
    constexpr int KB = K / 4 < 16 ? K / 4 : 16;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 4 * KB) {
        float av[KB], aw[KB], bv[KB];
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const int k = k0 + 4 * j + g;
            av[j] = a0[c * am + k * ak];
            aw[j] = a1[c * am + k * ak];
            bv[j] = b[k * bk + c * bn];
        }
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            d0 = mfma_f32(av[j], bv[j], d0);
            d1 = mfma_f32(aw[j], bv[j], d1);
        }
    }
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

// ---------------------------------------------------------------- staging
template <int N, int R, int kRows>
struct Smem {
    static constexpr int QT = kRows / R, NH = N / 2, NTN = N / 16;
    // Row pitches = 12 (mod 64 words) where LDS allows: an MFMA operand read
    // as A(c, k0 + g) = m[c * pitch + k] then touches each bank at most once
    // (64 banks) or twice (32), and read transposed, m[c + k * pitch], at most
    // twice (three times).  The 64-row chunk keeps 4 (mod 64) to fit.
    static constexpr int kPad = kRows == 64 ? 4 : 12;
    static constexpr int LB = N + kPad;     // B~, C~ rows
    static constexpr int LX = kP + kPad;    // X, dY rows
    static constexpr int LM = kRows + kPad; // M, dCB rows
    static constexpr int LS = N + kPad;     // S, Gh rows
    // staged element (row rho, column n / p)
    __device__ static int bi(int rho, int n) { return rho * LB + n; }
    __device__ static int xi(int rho, int p) { return rho * LX + p; }
    float Bs[kRows * LB], Cs[kRows * LB];
    float Xs[kRows * LX], Ys[kRows * LX];
    float Ms[kRows * LM], Ds[kRows * LM];
    float Ss[kP * LS], Gs[kP * LS];
    // per token and pair, rows of AP = NH + 3 words: a row-strided access by
    // sixteen lanes then spreads over the banks instead of landing on one.
    // cos and sin of the in-chunk angle; once every reader holds its values
    // they take the two halves of the angle sums
    static constexpr int AP = NH + 3;
    float acs[QT * AP], asn[QT * AP];
    float phi_end[NH];      // the chunk's angle total per pair
    float dtv[QT], lamv[QT], acum[QT], gw[QT], ww[QT], eac[QT], ebar[QT], wbar[QT];
    float rin[kRows], cinx[kRows], dwi[kRows], qv[kRows], rcr[kRows];
    float dgv[QT], dal[QT];
    float red[32];
    float gs, pdsum;
};

// Per-token scalars, the in-chunk angles, and (X, dY) / (B~, C~) as asked.
// Every global load of the chunk is issued before the first use of any of
// them (NTH threads, the workgroup size): a wave then waits once for its
// whole share instead of once per staged element.
template <typename T, int N, int R, int kRows, bool WANT_B, bool WANT_X, int NTH, typename S>
__device__ void stage(const ScanLaunch &a, const BwdArgs &g, S &sm, size_t bh, int ck) {
    constexpr int QT = S::QT, NH = S::NH, NW = NTH / 64;
    constexpr int TI = NH / NW;                 // angle pairs per wave
    // chunks of at most 32 tokens scan two pairs per wave scan (lanes [0, 32)
    // and [32, 64)); lane -> token tl of pair wave + (PK j + hl) NW
    constexpr bool PACK = QT <= 32;
    constexpr int PK = PACK ? 2 : 1, TS = TI / PK;
    static_assert(TI % PK == 0, "paired angle scans");
    constexpr int JB = (QT * NH + NTH - 1) / NTH;   // (token, pair) items per thread
    constexpr int JX = kRows * kP / NTH;        // (row, p) items per thread
    static_assert(NH % NW == 0 && (kRows * kP) % NTH == 0, "stage split");
    constexpr bool kPrecise = true;   // precise sines whatever the storage
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const float A = 0.0f - expf(a.a_log[hh]);
    const size_t t0 = static_cast<size_t>(ck) * QT;

    // ---- loads
    float dt = 0.0f, lam = 0.0f, dtn = 0.0f, lamn = 0.0f;
    if (tid < QT) {
        const size_t t = t0 + tid;
        const size_t ix = (bb * L + t) * H + hh;
        if (t < L) {
            dt = a.dt[ix];
            lam = a.lambda[ix];
        }
        if (t + 1 < L) {
            dtn = a.dt[ix + H];
            lamn = a.lambda[ix + H];
        }
    }
    const int tl = PACK ? (lane & 31) : lane, hl = PACK ? (lane >> 5) : 0;
    const size_t tgl = t0 + tl;
    const bool tlive = tl < QT && tgl < L;
    // Loads are unconditional at clamped (in-bounds) indices and the dead
    // lanes zeroed afterwards, so no load sits behind a branch (which would
    // make each one wait for its data before the next is issued).
    float th[TS];
    if (rot) {
        const size_t th0 = ((bb * L + (tlive ? tgl : 0)) * H + hh) * NH;
#pragma unroll
        for (int j = 0; j < TS; ++j) {
            const float v = ldv<T>(a.theta, th0 + wave + (PK * j + hl) * NW);
            th[j] = tlive ? v : 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < TS; ++j) th[j] = 0.0f;
    }
    float b1[JB][R], b2[JB][R], c1[JB][R], c2[JB][R];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int e = tid + j * NTH, t = e / NH;
        const int i = e < QT * NH ? e % NH : 0;
        const size_t tg = t0 + t;
        const bool live = e < QT * NH && tg < L;
        const size_t base = ((bb * L + (live ? tg : 0)) * H + hh) * N * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            b1[j][r] = b2[j][r] = 0.0f;
            if constexpr (WANT_B) {
                const float u1 = ldv<T>(a.b, base + i * R + r);
                const float u2 = ldv<T>(a.b, base + (i + NH) * R + r);
                b1[j][r] = live ? u1 : 0.0f;
                b2[j][r] = live ? u2 : 0.0f;
            }
            const float v1 = ldv<T>(a.c, base + i * R + r);
            const float v2 = ldv<T>(a.c, base + (i + NH) * R + r);
            c1[j][r] = live ? v1 : 0.0f;
            c2[j][r] = live ? v2 : 0.0f;
        }
    }
    float yv[JX], xv[JX];
#pragma unroll
    for (int j = 0; j < JX; ++j) {
        const int e = tid + j * NTH, rho = e / kP, p = e % kP;
        const int t = rho / R, r = rho % R;
        const size_t tg = t0 + t;
        const bool live = tg < L;
        const size_t ix = (((bb * L + (live ? tg : 0)) * H + hh) * kP + p) * R + r;
        const float vy = ldv<T>(g.dy, ix);
        yv[j] = live ? vy : 0.0f;
        xv[j] = 0.0f;
        if constexpr (WANT_X) {
            const float vx = ldv<T>(a.x, ix);
            xv[j] = live ? vx : 0.0f;
        }
    }

    // ---- per-token scalars and the in-chunk prefixes (wave scans, lane = token)
    if (tid < QT) {
        sm.dtv[tid] = dt;
        sm.lamv[tid] = lam;
        sm.gw[tid] = lam * dt;                          // fused.rs:2494
        sm.ww[tid] = lam * dt + (1.0f - lamn) * dtn;    // fused.rs:2496-2498
    }
    if (wave == 0) {
        const float v = seg_scan<64>(tid < QT ? dt * A : 0.0f);
        if (lane < QT) sm.acum[lane] = v;
    }
    __syncthreads();
    if (rot) {
        // the in-chunk angle (inclusive cumsum of dt theta) and its cos / sin
        const float dtl = tlive ? sm.dtv[tl] : 0.0f;
#pragma unroll
        for (int j = 0; j < TS; ++j) {
            const int i = wave + (PK * j + hl) * NW;
            const float v = PACK ? seg_scan<32>(dtl * th[j]) : seg_scan<64>(dtl * th[j]);
            if (tl < QT) {
                float sv, cv;
                sincos_any<kPrecise>(v, sv, cv);
                sm.acs[tl * S::AP + i] = cv;
                sm.asn[tl * S::AP + i] = sv;
            }
            if (tl == QT - 1) sm.phi_end[i] = v;
        }
    }
#pragma unroll
    for (int j = 0; j < JX; ++j) {
        const int e = tid + j * NTH, rho = e / kP, p = e % kP;
        sm.Ys[S::xi(rho, p)] = yv[j];
        if constexpr (WANT_X) sm.Xs[S::xi(rho, p)] = xv[j];
    }
    __syncthreads();
    if (tid < QT) {
        const float e = sm.acum[QT - 1];
        sm.eac[tid] = clamp_exp(sm.acum[tid]);
        sm.ebar[tid] = clamp_exp(e - sm.acum[tid]);
        sm.wbar[tid] = sm.ebar[tid] * sm.ww[tid];
    }
    // ---- rotation by the negative in-chunk angle (fused.rs:610-617) into LDS
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int e = tid + j * NTH, t = e / NH, i = e % NH;
        if (e >= QT * NH) break;
        float sn = 0.0f, cs = 1.0f;
        if (rot) {
            cs = sm.acs[t * S::AP + i];
            sn = sm.asn[t * S::AP + i];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int rho = t * R + r;
            if constexpr (WANT_B) {
                sm.Bs[S::bi(rho, i)] = b1[j][r] * cs + b2[j][r] * sn;
                sm.Bs[S::bi(rho, i + NH)] = -b1[j][r] * sn + b2[j][r] * cs;
            }
            sm.Cs[S::bi(rho, i)] = c1[j][r] * cs + c2[j][r] * sn;
            sm.Cs[S::bi(rho, i + NH)] = -c1[j][r] * sn + c2[j][r] * cs;
        }
    }
}

// ---------------------------------------------------------------- state passes
// The recompute's sequential parts, each with its chunk term formed in place:
//   forward: S_0 = R(angle0)(h0 + (1 - lambda_0) dt_0 last_u0) (scan.rs:521-535),
//     S_{k+1} = R(Phi_k)(e_k S_k + U_k), S_k written for every chunk
//     (scan.rs:244-251 in chunk frames), with
//     U_k^T[n][p] = sum_rho wbar B~[rho][n] X[rho][p], the chunk's contribution
//     to the state (the forward's chunk state, scan.rs:207-251), f32 operands;
//   reverse: G_C = R(phi_end) dh_out (or 0); for k = C-1 .. 0: Gh_k =
//     R(-Phi_k) G_{k+1}, G_k = e_k Gh_k + V_k, with V_k^T[n][p] =
//     sum_rho C~[rho][n] e^{alpha} dY[rho][p], the chunk's direct share of
//     dL/dS_k (the carry-in product y += e^alpha C~ S, scan.rs:253-263); then
//     dh0, dlast_u0 and the gradient of (1 - lambda_0) dt_0.
// One workgroup per (batch, head, 16 rotation pairs) and direction; thread =
// (p, four pairs): the state's 32 columns of those pairs stay in registers.
// Per chunk the workgroup stages the token scalars and its pairs' in-chunk
// angles (the scans of the chunk kernel's stage, so every value is the
// same), rotates its 32 columns of B (or C) into LDS scaled by wbar (or not),
// stages X (or e^alpha dY), and forms U^T (or V^T) by f32 MFMA directly in the
// state's lane layout.  The raw inputs of the next chunks are loaded ahead
// into registers; no per-chunk record but S_k (Gh_k) leaves the workgroup.
template <int R, int kRows>
struct PassSmem {
    static constexpr int QT = kRows / R, LDR = kRows + 4, AP = 17;
    float As[32 * LDR];      // rotated columns: [column][rho], lo pairs then hi
    float Xs[kP * LDR];      // X or e^alpha dY: [p][rho]
    // per chunk parity: cos / sin of the in-chunk angle [token][pair], the
    // token scalars, the decay prefix and the per-token scale
    float acs[2][QT * AP], asn[2][QT * AP];
    float dtv[2][QT], acum[2][QT], ww[2][QT], scal[2][QT];
    float phi[16];           // the sequence's angle total per pair (reverse pass)
    float red[16];
};

template <typename T, int N, int R, int kRows, bool FWD>
__device__ void state_pass(const ScanLaunch &a, const BwdArgs &g, const BwdWs &w, int nck,
                           size_t blk, PassSmem<R, kRows> &sm) {
    using S = PassSmem<R, kRows>;
    constexpr int NTN = N / 16, HT = NTN / 2, NH = N / 2, QT = S::QT, LDR = S::LDR, AP = S::AP;
    constexpr int NW = 4;                       // waves
    constexpr int TI = 16 / NW;                 // pairs per wave in the angle scans
    constexpr bool PACK = QT <= 32;             // two 32-token scans per wave
    constexpr int PK = PACK ? 2 : 1, TS = TI / PK;
    constexpr int JB = 16 * kRows / 256;        // (row, pair) items per thread
    constexpr int JX = kP * kRows / 256;        // (row, p) items per thread
    constexpr int D = kRows == 32 ? 3 : 2;      // chunks loaded ahead
    static_assert(TI % PK == 0 && JB >= 1 && JX >= 1, "pass split");
    const int tid = threadIdx.x, lane = tid & 63, pt = tid >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(pt);
    const int c = lane & 15, gq = lane >> 4;
    const int i1 = static_cast<int>(blk % HT);
    const size_t bh = blk / HT;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const float A = 0.0f - expf(a.a_log[hh]);
    const int p = 16 * pt + c, nlo = 16 * i1 + 4 * gq;
    const size_t sbase = bh * kP * N + static_cast<size_t>(p) * N;
    const int tl = PACK ? (lane & 31) : lane, hl = PACK ? (lane >> 5) : 0;
    auto rot4 = [](f32x4 &lo, f32x4 &hi, f32x4 cs, f32x4 sn) {
        const f32x4 l = lo;
        lo = l * cs - hi * sn;
        hi = l * sn + hi * cs;
    };
    auto sincos4 = [](f32x4 t, f32x4 &sn, f32x4 &cs) {
        for (int r = 0; r < 4; ++r) {
            float s, cc;
            sincosf(t[r], &s, &cc);
            sn[r] = s;
            cs[r] = cc;
        }
    };

    struct In {
        float dt, lam, dtn, lamn;
        float th[TS];
        float b1[JB], b2[JB];
        float xv[JX];
    };
    // Chunk k's raw inputs, by buffer loads over this sequence's tokens: a
    // token at or past the sequence end reads as zero, as the chunk kernel's
    // stage zeroes it.  A thread's items sit at fixed byte offsets from its
    // chunk-0 offsets (256 threads cover whole tokens of every array).
    constexpr uint32_t SZ = sizeof(T);
    const scan::SeqBufs rs = scan::seq_bufs<T, N, kP, R>(a, bb, hh);
    const rsrc_t rbc = FWD ? rs.b : rs.c;
    const rsrc_t rxy = FWD ? rs.x
                           : make_rsrc(static_cast<const char *>(g.dy) + (bb * L * H + hh) * kP * R * SZ,
                                       static_cast<uint32_t>((L * H - hh) * kP * R * SZ));
    auto ld = [](rsrc_t r, uint32_t off) -> float {
        if constexpr (sizeof(T) == 4)
            return bldf(r, off);
        else
            return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)) << 16);
    };
    const int ts = tid < QT ? tid : 0;
    const uint32_t o_s = ts * rs.tok_s;
    const uint32_t o_th = tl * rs.tok_th + (16 * i1) * SZ;
    const int tb = tid / (16 * R), qr = tid % (16 * R);
    const uint32_t o_bc = tb * rs.tok_bc + (16 * i1 * R + qr) * SZ;
    const uint32_t bc_j = (16 / R) * rs.tok_bc;
    const int tx = tid / (kP * R), pr = tid % (kP * R);
    const uint32_t o_xy = tx * rs.tok_x + pr * SZ;
    const uint32_t xy_j = (256 / (kP * R)) * rs.tok_x;
    auto load = [&](int k, In &d) {
        const int kk = k < 0 ? 0 : (k < nck ? k : nck - 1);   // outside: re-read, unused
        const uint32_t t0 = static_cast<uint32_t>(kk) * QT;
        d.dt = bldf(rs.s0, o_s + t0 * rs.tok_s);
        d.lam = bldf(rs.s1, o_s + t0 * rs.tok_s);
        d.dtn = bldf(rs.s0, o_s + (t0 + 1) * rs.tok_s);
        d.lamn = bldf(rs.s1, o_s + (t0 + 1) * rs.tok_s);
        if (rot) {
            const uint32_t o = o_th + t0 * rs.tok_th;
#pragma unroll
            for (int j = 0; j < TS; ++j) {
                const float v = ld(rs.th, o + (wave + (PK * j + hl) * NW) * SZ);
                d.th[j] = tl < QT ? v : 0.0f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < TS; ++j) d.th[j] = 0.0f;
        }
        const uint32_t ob = o_bc + t0 * rs.tok_bc;
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            d.b1[j] = ld(rbc, ob + j * bc_j);
            d.b2[j] = ld(rbc, ob + j * bc_j + NH * R * SZ);
        }
        const uint32_t ox = o_xy + t0 * rs.tok_x;
#pragma unroll
        for (int j = 0; j < JX; ++j) d.xv[j] = ld(rxy, ox + j * xy_j);
    };
    // Chunk k's term of this lane's state columns (acc), its decay e and the
    // rotation by its angle totals (pc, ps).
    // The chunk's work in four pieces, software-pipelined over two sets of
    // the per-chunk tables (sb = chunk parity): the scalars and decay prefix
    // (p1) and the angles (p2) of chunk k + 1 run in the same two barrier
    // phases as the staging (p3) and the products (p4) of chunk k.
    //   phase X: p3(k), p1(k + 1);  barrier;  phase Y: p4(k), p2(k + 1);  barrier
    // token scalars, the decay prefix (fused.rs:2494-2498)
    auto p1 = [&](const In &d, int sb) {
        if (tid < QT) {
            sm.dtv[sb][tid] = d.dt;
            sm.ww[sb][tid] = d.lam * d.dt + (1.0f - d.lamn) * d.dtn;
        }
        if (wave == 0) {
            const float v = seg_scan<64>(tid < QT ? d.dt * A : 0.0f);
            if (lane < QT) sm.acum[sb][lane] = v;
        }
    };
    // the in-chunk angle of this workgroup's pairs and its cos / sin; per
    // token wbar (B~'s scale) or e^alpha (dY's)
    auto p2 = [&](int k, const In &d, int sb) {
        if (rot) {
            const size_t t0 = static_cast<size_t>(k) * QT;
            const float dtl = (tl < QT && t0 + tl < L) ? sm.dtv[sb][tl] : 0.0f;
#pragma unroll
            for (int j = 0; j < TS; ++j) {
                const int i = wave + (PK * j + hl) * NW;
                const float v = PACK ? seg_scan<32>(dtl * d.th[j]) : seg_scan<64>(dtl * d.th[j]);
                if (tl < QT) {
                    float sv, cv;
                    sincos_any<true>(v, sv, cv);
                    sm.acs[sb][tl * AP + i] = cv;
                    sm.asn[sb][tl * AP + i] = sv;
                }
            }
        }
        if (tid < QT) {
            const float et = sm.acum[sb][QT - 1];
            sm.scal[sb][tid] = FWD ? clamp_exp(et - sm.acum[sb][tid]) * sm.ww[sb][tid]
                                   : clamp_exp(sm.acum[sb][tid]);
        }
    };
    // rotation by the negative in-chunk angle (fused.rs:610-617) into LDS;
    // the chunk decay
    auto p3 = [&](const In &d, int sb, float &e) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            const int ee = tid + 256 * j, t = ee / (16 * R), qr = ee % (16 * R);
            const int q = qr / R, rho = t * R + qr % R;
            float sn = 0.0f, cs = 1.0f;
            if (rot) {
                cs = sm.acs[sb][t * AP + q];
                sn = sm.asn[sb][t * AP + q];
            }
            float lo = d.b1[j] * cs + d.b2[j] * sn;
            float hi = -d.b1[j] * sn + d.b2[j] * cs;
            if constexpr (FWD) {
                lo *= sm.scal[sb][t];
                hi *= sm.scal[sb][t];
            }
            sm.As[q * LDR + rho] = lo;
            sm.As[(16 + q) * LDR + rho] = hi;
        }
#pragma unroll
        for (int j = 0; j < JX; ++j) {
            const int ee = tid + 256 * j, t = ee / (kP * R), pr = ee % (kP * R);
            float v = d.xv[j];
            if constexpr (!FWD) v *= sm.scal[sb][t];
            sm.Xs[(pr / R) * LDR + t * R + pr % R] = v;
        }
        e = clamp_exp(sm.acum[sb][QT - 1]);
    };
    // U^T (V^T) at this lane's (n, p): A(m = n, k = rho), B(k = rho, col = p);
    // the rotation by the chunk's angle totals, the in-chunk angles of its
    // last row
    auto p4 = [&](int sb, f32x4 &alo, f32x4 &ahi, f32x4 &pc, f32x4 &ps) {
        alo = f32x4{0.f, 0.f, 0.f, 0.f};
        ahi = alo;
        const float *br = sm.Xs + p * LDR;
#pragma unroll
        for (int kb = 0; kb < kRows / 16; ++kb) {
            alo = scan::mma_kb(sm.As + c * LDR + 16 * kb, br + 16 * kb, alo, gq);
            ahi = scan::mma_kb(sm.As + (16 + c) * LDR + 16 * kb, br + 16 * kb, ahi, gq);
        }
        pc = f32x4{1.f, 1.f, 1.f, 1.f};
        ps = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rot) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pc[r] = sm.acs[sb][(QT - 1) * AP + 4 * gq + r];
                ps[r] = sm.asn[sb][(QT - 1) * AP + 4 * gq + r];
            }
        }
    };
    auto offs = [&](int k, size_t &o, size_t &oh) {
        const size_t bhk = bh * nck + k;
        o = bhk * kP * N + ((pt * NTN + i1) * 64 + lane) * 4;
        oh = bhk * kP * N + ((pt * NTN + i1 + HT) * 64 + lane) * 4;
    };

    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    if constexpr (FWD) {
        if (a.h0 != nullptr) {
            lo = *reinterpret_cast<const f32x4 *>(a.h0 + sbase + nlo);
            hi = *reinterpret_cast<const f32x4 *>(a.h0 + sbase + nlo + NH);
            if (a.last_u0 != nullptr) {
                const size_t i0 = (bb * L) * H + hh;
                const float first = (1.0f - a.lambda[i0]) * a.dt[i0];
                lo += *reinterpret_cast<const f32x4 *>(a.last_u0 + sbase + nlo) * first;
                hi += *reinterpret_cast<const f32x4 *>(a.last_u0 + sbase + nlo + NH) * first;
            }
        }
        if (rot && a.angle0 != nullptr) {
            f32x4 sn, cs;
            sincos4(*reinterpret_cast<const f32x4 *>(a.angle0 + bh * NH + nlo), sn, cs);
            rot4(lo, hi, cs, sn);
        }
        In d[D];
#pragma unroll
        for (int j = 0; j < D; ++j) load(j, d[j]);
        p1(d[0], 0);
        __syncthreads();
        p2(0, d[0], 0);
        __syncthreads();
        for (int k = 0; k < nck; k += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const int kc = k + j;
                if (kc < nck) {
                    const int sb = kc & 1;
                    const bool more = kc + 1 < nck;
                    float e;
                    p3(d[j], sb, e);
                    if (more) p1(d[(j + 1) % D], sb ^ 1);
                    __syncthreads();
                    f32x4 ulo, uhi, pc, ps;
                    p4(sb, ulo, uhi, pc, ps);
                    if (more) p2(kc + 1, d[(j + 1) % D], sb ^ 1);
                    size_t o, oh;
                    offs(kc, o, oh);
                    *reinterpret_cast<f32x4 *>(w.s + o) = lo;
                    *reinterpret_cast<f32x4 *>(w.s + oh) = hi;
                    lo = lo * e + ulo;
                    hi = hi * e + uhi;
                    if (rot) rot4(lo, hi, pc, ps);   // R(Phi_k)
                    if (i1 == 0 && tid == 0) w.eda[bh * nck + kc] = e;
                    __syncthreads();
                }
                load(kc + D, d[j]);
            }
        }
    } else {
        if (g.dh_out != nullptr) {
            lo = *reinterpret_cast<const f32x4 *>(g.dh_out + sbase + nlo);
            hi = *reinterpret_cast<const f32x4 *>(g.dh_out + sbase + nlo + NH);
            if (rot) {
                // phi_end = angle0 + sum_k Phi_k: the final frame, S_C = R(phi_end) h_out.
                // Each Phi_k is the in-chunk scan's last value, summed in chunk order.
                constexpr int DT = 8;
                float ph[TS], dq[DT], tq[DT][TS];
#pragma unroll
                for (int j = 0; j < TS; ++j) {
                    const int i = wave + (PK * j + hl) * NW;
                    ph[j] = a.angle0 != nullptr ? a.angle0[bh * NH + 16 * i1 + i] : 0.0f;
                }
                auto tload = [&](int k, float &dv, float (&tv)[TS]) {
                    const int kk = k < nck ? k : nck - 1;
                    const size_t tg = static_cast<size_t>(kk) * QT + tl;
                    const bool tlive = tl < QT && tg < L;
                    const size_t row = (bb * L + (tlive ? tg : 0)) * H + hh;
                    const float v = a.dt[row];
                    dv = tlive ? v : 0.0f;
#pragma unroll
                    for (int j = 0; j < TS; ++j) {
                        const float u = ldv<T>(a.theta, row * NH + 16 * i1 + wave + (PK * j + hl) * NW);
                        tv[j] = tlive ? u : 0.0f;
                    }
                };
#pragma unroll
                for (int q = 0; q < DT; ++q) tload(q, dq[q], tq[q]);
                for (int k = 0; k < nck; k += DT) {
#pragma unroll
                    for (int q = 0; q < DT; ++q) {
                        if (k + q < nck) {
#pragma unroll
                            for (int j = 0; j < TS; ++j) {
                                const float v = PACK ? seg_scan<32>(dq[q] * tq[q][j])
                                                     : seg_scan<64>(dq[q] * tq[q][j]);
                                ph[j] += v;
                            }
                        }
                        tload(k + DT + q, dq[q], tq[q]);
                    }
                }
                if (tl == QT - 1) {
#pragma unroll
                    for (int j = 0; j < TS; ++j) sm.phi[wave + (PK * j + hl) * NW] = ph[j];
                }
                __syncthreads();
                f32x4 pe;
#pragma unroll
                for (int r = 0; r < 4; ++r) pe[r] = sm.phi[4 * gq + r];
                __syncthreads();
                f32x4 sn, cs;
                sincos4(pe, sn, cs);
                rot4(lo, hi, cs, sn);
            }
        }
        In d[D];
#pragma unroll
        for (int j = 0; j < D; ++j) load(nck - 1 - j, d[j]);
        p1(d[0], (nck - 1) & 1);
        __syncthreads();
        p2(nck - 1, d[0], (nck - 1) & 1);
        __syncthreads();
        for (int k = nck - 1; k >= 0; k -= D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const int kc = k - j;
                if (kc >= 0) {
                    const int sb = kc & 1;
                    const bool more = kc > 0;
                    float e;
                    p3(d[j], sb, e);
                    if (more) p1(d[(j + 1) % D], sb ^ 1);
                    __syncthreads();
                    f32x4 vlo, vhi, pc, ps;
                    p4(sb, vlo, vhi, pc, ps);
                    if (more) p2(kc - 1, d[(j + 1) % D], sb ^ 1);
                    if (rot) rot4(lo, hi, pc, -ps);   // R(-Phi_k)
                    size_t o, oh;
                    offs(kc, o, oh);
                    *reinterpret_cast<f32x4 *>(w.gh + o) = lo;
                    *reinterpret_cast<f32x4 *>(w.gh + oh) = hi;
                    lo = lo * e + vlo;
                    hi = hi * e + vhi;
                    __syncthreads();
                }
                load(kc - D, d[j]);
            }
        }
        // into the global frame: dZ0 = R(-angle0) G_0
        if (rot && a.angle0 != nullptr) {
            f32x4 sn, cs;
            sincos4(*reinterpret_cast<const f32x4 *>(a.angle0 + bh * NH + nlo), sn, cs);
            rot4(lo, hi, cs, -sn);
        }
        float dfirst = 0.0f;
        if (a.h0 != nullptr) {
            if (g.dh0 != nullptr) {
                *reinterpret_cast<f32x4 *>(g.dh0 + sbase + nlo) = lo;
                *reinterpret_cast<f32x4 *>(g.dh0 + sbase + nlo + NH) = hi;
            }
            if (a.last_u0 != nullptr) {
                const size_t i0 = (bb * L) * H + hh;
                const float first = (1.0f - a.lambda[i0]) * a.dt[i0];
                const f32x4 ul = *reinterpret_cast<const f32x4 *>(a.last_u0 + sbase + nlo);
                const f32x4 uh = *reinterpret_cast<const f32x4 *>(a.last_u0 + sbase + nlo + NH);
                for (int r = 0; r < 4; ++r) dfirst += lo[r] * ul[r] + hi[r] * uh[r];
                if (g.dlast_u0 != nullptr) {
                    *reinterpret_cast<f32x4 *>(g.dlast_u0 + sbase + nlo) = lo * first;
                    *reinterpret_cast<f32x4 *>(g.dlast_u0 + sbase + nlo + NH) = hi * first;
                }
            }
        }
        dfirst = block_sum(dfirst, sm.red);
        if (tid == 0) w.pfirst[blk] = dfirst;
    }
}

// Both sequential passes in one launch (they are independent): workgroups
// [0, nb) run the forward recurrence, [nb, 2 nb) the reverse one.
template <typename T, int N, int R, int kRows>
__global__ void __launch_bounds__(256) bwd_passes_kernel(ScanLaunch a, BwdArgs g, BwdWs w,
                                                         int nck) {
    __shared__ __attribute__((aligned(16))) PassSmem<R, kRows> sm;
    const size_t nb = a.batch * a.heads * (N / 32);
    if (blockIdx.x < nb)
        state_pass<T, N, R, kRows, true>(a, g, w, nck, blockIdx.x, sm);
    else
        state_pass<T, N, R, kRows, false>(a, g, w, nck, blockIdx.x - nb, sm);
}

// ---------------------------------------------------------------- chunk gradients
template <typename T, int N, int R, int kRows>
__global__ void __launch_bounds__(kBT, 1) bwd_chunk_kernel(ScanLaunch a, BwdArgs g, BwdWs w,
                                                           int nck) {
    using S = Smem<N, R, kRows>;
    constexpr int NT = kRows / 16;
    constexpr int QT = S::QT, NH = S::NH, NTN = N / 16;
    constexpr int LB = S::LB, LX = S::LX, LM = S::LM, LS = S::LS;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    S &sm = *reinterpret_cast<S *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, gq = lane >> 4;
    const size_t bhk = blockIdx.x;
    const int ck = static_cast<int>(bhk % nck);
    const size_t bh = bhk / nck;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const float D = a.d_skip ? a.d_skip[hh] : 0.0f;

    stage<T, N, R, kRows, true, true, kBT>(a, g, sm, bh, ck);
    // the state entering the chunk and Gh, [p][n]: four consecutive n per
    // 16-byte record piece, all loads in flight together
    {
        constexpr int JS = kP * N / 4 / kBT;
        static_assert(JS * 4 * kBT == kP * N, "state copy split");
        f32x4 sv[JS], gv[JS];
        const f32x4 *s4 = reinterpret_cast<const f32x4 *>(w.s +
                                                          bhk * kP * N);
        const f32x4 *g4 = reinterpret_cast<const f32x4 *>(w.gh + bhk * kP * N);
#pragma unroll
        for (int j = 0; j < JS; ++j) {
            sv[j] = s4[tid + j * kBT];
            gv[j] = g4[tid + j * kBT];
        }
#pragma unroll
        for (int j = 0; j < JS; ++j) {
            int p, n;
            dl_pn(4 * (tid + j * kBT), NTN, p, n);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sm.Ss[p * LS + n + r] = sv[j][r];
                sm.Gs[p * LS + n + r] = gv[j][r];
            }
        }
    }
    if (tid < kRows) {
        sm.rin[tid] = sm.cinx[tid] = sm.dwi[tid] = sm.qv[tid] = sm.rcr[tid] = 0.0f;
    }
    if (tid < QT) sm.dgv[tid] = 0.0f;
    __syncthreads();

    // Three phases.  Phase 1 is everything that does not need the band: the
    // band products themselves, the Gh B~^T half of dX, the S dY / Gh X half of
    // each dC~ / dB~ job with its row sums, and the jobs' sines.  Phase 2 is
    // the band, elementwise.  Phase 3 finishes dX and the jobs with M and dCB.
    // Work per wave: at most one dX tile and one job (accumulators stay in
    // registers across the barriers); band products go to the waves from
    // kWaves / 2 on first, which carry no dX tile.
    constexpr int NB = NT * (NT + 1) / 2;
    constexpr int PT = NTN / 2, NJ = NT * PT;
    static_assert(2 * NJ <= kWaves && 4 * NT <= kWaves, "one job and one dX tile per wave");
    const bool rot = a.theta != nullptr;

    // ---- phase 1a: band products, raw: CB[t][s] = sum_n C~[t][n] B~[s][n]
    // into Ms and dM[t][s] = sum_p dY[t][p] X[s][p] into Ds, for the tiles on
    // and below the diagonal (the tiles above lie above the token diagonal)
    for (int job = (wave + kWaves / 2) % kWaves; job < 2 * NB; job += kWaves) {
        int q = job >> 1, tj = 0;
        while (q > tj) {
            q -= tj + 1;
            ++tj;
        }
        const int si = q;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float *dst;
        if ((job & 1) == 0) {
            acc = mma_f32<N>(sm.Cs + 16 * tj * LB, LB, 1, sm.Bs + 16 * si * LB, 1, LB, acc, c, gq);
            dst = sm.Ms;
        } else {
            acc = mma_f32<kP>(sm.Ys + 16 * tj * LX, LX, 1, sm.Xs + 16 * si * LX, 1, LX, acc, c, gq);
            dst = sm.Ds;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(16 * tj + 4 * gq + r) * LM + 16 * si + c] = acc[r];
    }

    // ---- phase 1b: dX^T[p][s] = wbar_s sum_n Gh[p][n] B~[s][n] (+ phase 3)
    const bool has_dx = wave < 4 * NT;
    const int xpt = wave & 3, xst = wave >> 2;
    f32x4 xacc = {0.f, 0.f, 0.f, 0.f};
    if (has_dx)
        xacc = mma_f32<N>(sm.Gs + 16 * xpt * LS, LS, 1, sm.Bs + 16 * xst * LB, 1, LB, xacc, c, gq);

    // ---- phase 1c: dC~ and dB~ as [n][row] tiles; job = (which, pair tile i,
    // row tile); a job writes the gradient of C (which = 0) or B
    const bool has_job = wave < 2 * NJ, isb = wave >= NJ;
    const int jj = isb ? wave - NJ : wave;
    const int ji = jj % PT, rt = jj / PT;
    const int row = 16 * rt + c, tr = row / R, rr = row % R;
    const int n0 = 16 * ji + 4 * gq;
    // the job's own rotated operand (C~ for dC~, B~ for dB~) at its elements
    const float *own = isb ? sm.Bs : sm.Cs;
    float sn[4], cs[4], o1[4], o2[4];
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    if (has_job) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sn[r] = 0.0f;
            cs[r] = 1.0f;
            if (rot) {
                cs[r] = sm.acs[tr * S::AP + n0 + r];
                sn[r] = sm.asn[tr * S::AP + n0 + r];
            }
            o1[r] = own[row * LB + n0 + r];
            o2[r] = own[row * LB + n0 + r + NH];
        }
        if (!isb) {
            // dC~^T[n][t] = e^{alpha_t} sum_p S[p][n] dY[t][p] + (phase 3)
            mma2_f32<kP>(sm.Ss + 16 * ji, sm.Ss + 16 * (ji + PT), 1, LS, sm.Ys + 16 * rt * LX, 1,
                         LX, lo, hi, c, gq);
            const float ea = sm.eac[tr];
            lo = lo * ea;
            hi = hi * ea;
        } else {
            // dB~^T[n][s] = wbar_s sum_p Gh[p][n] X[s][p] + (phase 3)
            mma2_f32<kP>(sm.Gs + 16 * ji, sm.Gs + 16 * (ji + PT), 1, LS, sm.Xs + 16 * rt * LX, 1,
                         LX, lo, hi, c, gq);
        }
        // row . (S or Gh part): the e^alpha dy.(S C~) and wbar x.(Gh B~) terms
        float q = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) q += lo[r] * o1[r] + hi[r] * o2[r];
        q += __shfl_xor(q, 16, 64);
        q += __shfl_xor(q, 32, 64);
        if (gq == 0) atomicAdd(isb ? &sm.qv[row] : &sm.rcr[row], q);
        if (isb) {
            const float wb = sm.wbar[tr];
            lo = lo * wb;
            hi = hi * wb;
        }
    }
    __syncthreads();

    // ---- phase 2: the band, elementwise (one (t, s) per thread in turn, s
    // fastest): K = W e^{alpha_t - alpha_s}, M = CB o K, dCB = dM o K; the
    // diagonal's dg sums, and off it L = dM o M (row sums, column sums) and
    // the dw sums
    static_assert(kRows == 32 || kRows == 64, "band rows");
    for (int e0 = 0; e0 < kRows * kRows; e0 += kBT) {
        const int e = e0 + tid, t = e / kRows, s = e % kRows;
        const int tt = t / R, ts = s / R;
        float lam = 0.0f, dwe = 0.0f;
        if (e < kRows * kRows) {
            float m = 0.0f, d = 0.0f;
            if (tt >= ts) {
                const float cb = sm.Ms[t * LM + s], dm = sm.Ds[t * LM + s];
                const float E = clamp_exp(sm.acum[tt] - sm.acum[ts]);
                const float K = (tt == ts ? sm.gw[ts] : sm.ww[ts]) * E;
                m = cb * K;
                d = dm * K;
                if (tt == ts) {
                    atomicAdd(&sm.dgv[ts], dm * cb);
                } else {
                    lam = dm * m;
                    dwe = dm * cb * E;
                }
            }
            sm.Ms[t * LM + s] = m;
            sm.Ds[t * LM + s] = d;
        }
        // row sums: a row is kRows consecutive lanes of one wave
        float rs = lam;
        for (int off = 1; off < kRows; off <<= 1) rs += __shfl_xor(rs, off, 64);
        if (s == 0 && e < kRows * kRows) sm.rin[t] = rs;
        // column sums: add the wave's rows first, then one atomic per column
        float cl = lam, cw = dwe;
        if constexpr (kRows == 32) {
            cl += __shfl_xor(cl, 32, 64);
            cw += __shfl_xor(cw, 32, 64);
        }
        if (lane < kRows && e < kRows * kRows) {
            atomicAdd(&sm.cinx[s], cl);
            atomicAdd(&sm.dwi[s], cw);
        }
    }
    __syncthreads();

    // ---- phase 3a: dX^T[p][s] += sum_t dY[t][p] M[t][s] + D dY[s][p]
    if (has_dx) {
        const int s = 16 * xst + c, ts = s / R, rs = s % R;
        f32x4 acc = xacc * sm.wbar[ts];
        acc = mma_f32<kRows>(sm.Ys + 16 * xpt, 1, LX, sm.Ms + 16 * xst, LM, 1, acc, c, gq);
        const size_t tg = static_cast<size_t>(ck) * QT + ts;
        if (tg < L) {
            const size_t base = ((bb * L + tg) * H + hh) * kP * R;
            const int p0 = 16 * xpt + 4 * gq;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += D * sm.Ys[s * LX + p0 + r];
            st4<T, R>(g.dx, base + p0 * R + rs, acc);
        }
    }
    // ---- phase 3b: the band halves of dC~ and dB~
    //   dC~^T[n][t] += sum_s B~[s][n] dCB[t][s],  dB~^T[n][s] += sum_t C~[t][n] dCB[t][s]
    // then the angle sums (every cos / sin was read in phase 1: asn receives
    // the dB~ half, acs the dC~ half, one lane per (token, pair)) and the
    // rotation back, d = R(psi) d~ (the transpose of fused.rs:610-617)
    if (has_job) {
        if (!isb)
            mma2_f32<kRows>(sm.Bs + 16 * ji, sm.Bs + 16 * (ji + PT), 1, LB, sm.Ds + 16 * rt * LM,
                            1, LM, lo, hi, c, gq);
        else
            mma2_f32<kRows>(sm.Cs + 16 * ji, sm.Cs + 16 * (ji + PT), 1, LB, sm.Ds + 16 * rt, LM, 1,
                            lo, hi, c, gq);
        if (rot) {
            float *half = isb ? sm.asn : sm.acs;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float cr = lo[r] * o2[r] - hi[r] * o1[r];
                // the R rows of a token sit in adjacent lanes
                if constexpr (R >= 2) cr += __shfl_xor(cr, 1, 64);
                if constexpr (R >= 4) cr += __shfl_xor(cr, 2, 64);
                if (rr == 0) half[tr * S::AP + n0 + r] = cr;
            }
        }
        f32x4 v1, v2;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            v1[r] = lo[r] * cs[r] - hi[r] * sn[r];
            v2[r] = lo[r] * sn[r] + hi[r] * cs[r];
        }
        const size_t tg = static_cast<size_t>(ck) * QT + tr;
        if (tg < L) {
            void *dst = isb ? g.db : g.dc;
            const size_t base = ((bb * L + tg) * H + hh) * N * R;
            st4<T, R>(dst, base + n0 * R + rr, v1);
            st4<T, R>(dst, base + (n0 + NH) * R + rr, v2);
        }
    }

    // ---- <Gh, S> and the skip's sum dY . X, one block reduction for both
    {
        float gsum = 0.0f, dsum = 0.0f;
        for (int e = tid; e < kP * N; e += kBT) {
            const int p = e / N, n = e % N;
            gsum += sm.Gs[p * LS + n] * sm.Ss[p * LS + n];
        }
        for (int e = tid; e < kRows * kP; e += kBT) {
            const int rho = e / kP, p = e % kP;
            dsum += sm.Ys[rho * LX + p] * sm.Xs[rho * LX + p];
        }
        gsum = group_sum(gsum, 64);
        dsum = group_sum(dsum, 64);
        if (lane == 0) {
            sm.red[wave] = gsum;
            sm.red[16 + wave] = dsum;
        }
    }
    static_assert(kWaves <= 16, "block reduction slots");
    __syncthreads();

    // ---- per-token scalars: dalpha, then da = in-chunk reverse cumsum
    if (wave == 0) {
        const float gs = group_sum(lane < kWaves ? sm.red[lane] : 0.0f, 64);
        const float ds = group_sum(lane < kWaves ? sm.red[16 + lane] : 0.0f, 64);
        if (lane == 0) w.pd[bhk] = ds;
        // the alpha_E terms of the last row: sum over rows of wbar q
        const float e = group_sum(lane < kRows ? sm.qv[lane] * sm.wbar[lane / R] : 0.0f, 64);
        float d = 0.0f, dw = 0.0f;
        if (tid < QT) {
            for (int r = 0; r < R; ++r) {
                const int row = tid * R + r;
                d += sm.rin[row] - sm.cinx[row] + sm.rcr[row] - sm.qv[row] * sm.wbar[tid];
                dw += sm.dwi[row] + sm.qv[row] * sm.ebar[tid];
            }
        }
        if (tid == QT - 1) d += e + w.eda[bhk] * gs;
        if (tid < QT) sm.dal[tid] = d;
        const size_t tg = static_cast<size_t>(ck) * QT + tid;
        if (tid < QT && tg < L) {
            w.dg[bh * L + tg] = sm.dgv[tid];
            w.dw[bh * L + tg] = dw;
        }
    }
    __syncthreads();
    // in-chunk reverse cumsums as wave scans over lanes in reverse token order
    // (lane l holds token QT-1-l): da from dalpha (wave 0), and per rotation
    // pair the angle sums (pairs spread over the waves, written back to acs)
    {
        const int t = QT - 1 - lane;
        const size_t tg = static_cast<size_t>(ck) * QT + t;
        const bool live = lane < QT && tg < L;
        if (wave == 0) {
            const float v = seg_scan<64>(lane < QT ? sm.dal[t] : 0.0f);
            if (live) w.da[bh * L + tg] = v;
        }
        if (a.theta != nullptr) {
            for (int i = wave; i < NH; i += kWaves) {
                const float v = seg_scan<64>(
                    lane < QT ? sm.acs[t * S::AP + i] + sm.asn[t * S::AP + i] : 0.0f);
                if (lane < QT) sm.acs[t * S::AP + i] = v;
                if (lane == QT - 1) w.ctot[bhk * NH + i] = v;
            }
        }
    }
    if (a.theta != nullptr) {
        __syncthreads();
        // token-major rows of pairs, stored whole
        for (int e = tid; e < QT * NH; e += kBT) {
            const int t = e / NH, i = e % NH;
            const size_t tg = static_cast<size_t>(ck) * QT + t;
            if (tg < L) w.cin[(bh * L + tg) * NH + i] = sm.acs[t * S::AP + i];
        }
    }
}

// ---------------------------------------------------------------- angle sums of later chunks
template <int N>
__global__ void bwd_angle_kernel(ScanLaunch a, BwdArgs g, BwdWs w, int nck) {
    constexpr int NH = N / 2, D = 8;
    const size_t bh = blockIdx.x;
    const int i = threadIdx.x;
    if (i >= NH) return;
    float run = g.dangle_out ? g.dangle_out[bh * NH + i] : 0.0f;
    // eight chunk totals in flight ahead of the running sum
    for (int k0 = nck - 1; k0 >= 0; k0 -= D) {
        float v[D];
#pragma unroll
        for (int j = 0; j < D; ++j) v[j] = k0 - j >= 0 ? w.ctot[(bh * nck + k0 - j) * NH + i] : 0.0f;
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (k0 - j < 0) break;
            w.off[(bh * nck + k0 - j) * NH + i] = run;
            run += v[j];
        }
    }
    if (g.dangle0 != nullptr) g.dangle0[bh * NH + i] = run;
}

// ---------------------------------------------------------------- per token
// dtheta_t = dt_t dphi_t, ddt_t = theta_t . dphi_t + A da_t
//   + lambda_t (dg_t + dw_t) + (1 - lambda_t) dw_{t-1},
// dlambda_t = dt_t (dg_t + dw_t) - dt_t dw_{t-1}    (trapezoid_weights_backward,
// fused.rs:2513-2549), plus the carried-in boundary term at t = 0.
// One workgroup per chunk, one wave per token, lane = rotation pair.
template <typename T, int N, int R, int kRows>
__global__ void __launch_bounds__(256) bwd_token_kernel(ScanLaunch a, BwdArgs g, BwdWs w, int nck) {
    constexpr int NH = N / 2, QT = kRows / R;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t bhk = blockIdx.x;
    const int ck = static_cast<int>(bhk % nck);
    const size_t bh = bhk / nck;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const float A = 0.0f - expf(a.a_log[hh]);
    const bool rot = a.theta != nullptr;
    constexpr int TW = (QT + 3) / 4;   // tokens per wave: wave + 4 j
    static_assert(TW <= 64, "tokens per wave");
    // the per-token scalars of the second part (lane j = token wave + 4 j)
    // go out first: they depend on nothing below
    const int tk = wave + 4 * lane;
    const size_t tkg = static_cast<size_t>(ck) * QT + tk;
    const bool tk_live = lane < TW && tk < QT && tkg < L;
    const size_t tkc = tk_live ? tkg : 0;
    const size_t tkx = (bb * L + tkc) * H + hh;
    const float dt = a.dt[tkx], lam = a.lambda[tkx];
    const float da = w.da[bh * L + tkc];
    const float dgw = w.dg[bh * L + tkc] + w.dw[bh * L + tkc];
    const float dwv = w.dw[bh * L + (tkc > 0 ? tkc - 1 : 0)];
    // per pair (lane = pair): dtheta and the angle part of ddt, with every
    // load issued first (unconditional at clamped indices)
    float cin[TW], th[TW];
    const int pl = lane < NH ? lane : 0;
#pragma unroll
    for (int j = 0; j < TW; ++j) {
        const int t = wave + 4 * j;
        const size_t tg = static_cast<size_t>(ck) * QT + t;
        const bool live = t < QT && tg < L && lane < NH;
        const size_t tc = live ? tg : 0;
        const size_t ix = (bb * L + tc) * H + hh;
        float u = 0.0f, v = 0.0f;
        if (rot) {
            u = w.cin[(bh * L + tc) * NH + pl];
            v = ldv<T>(a.theta, ix * NH + pl);
        }
        cin[j] = live ? u : 0.0f;
        th[j] = live ? v : 0.0f;
    }
    const float off = rot ? w.off[bhk * NH + pl] : 0.0f;
    float mine = 0.0f;   // lane j keeps token wave + 4 j's angle part
#pragma unroll
    for (int j = 0; j < TW; ++j) {
        const int t = wave + 4 * j;
        const size_t tg = static_cast<size_t>(ck) * QT + t;
        float part = 0.0f;
        if (rot && t < QT && tg < L && lane < NH) {
            const size_t ix = (bb * L + tg) * H + hh;
            const float dphi = cin[j] + off;
            if (g.dtheta != nullptr) stv<T>(g.dtheta, ix * NH + lane, a.dt[ix] * dphi);
            part = th[j] * dphi;
        }
        part = group_sum(part, 64);
        if (lane == j) mine = part;
    }
    // per token (lane j = token wave + 4 j): trapezoid and decay chains
    const float dwp = tkc > 0 ? dwv : 0.0f;
    float ddt = mine + A * da + lam * dgw + (1.0f - lam) * dwp;
    float dlam = dt * dgw - dt * dwp;
    if (tk_live && tkg == 0 && a.h0 != nullptr && a.last_u0 != nullptr) {
        float dfirst = 0.0f;
        for (int q = 0; q < N / 32; ++q) dfirst += w.pfirst[bh * (N / 32) + q];
        ddt += (1.0f - lam) * dfirst;
        dlam -= dt * dfirst;
    }
    if (tk_live) {
        g.ddt[tkx] = ddt;
        g.dlambda[tkx] = dlam;
    }
    float asum = tk_live ? dt * da : 0.0f;
    __shared__ float red[16];
    asum = block_sum(asum, red);
    if (threadIdx.x == 0) w.pa[bhk] = asum;
}

// ---------------------------------------------------------------- per head
__global__ void __launch_bounds__(256) bwd_head_kernel(ScanLaunch a, BwdArgs g, BwdWs w, int nck) {
    __shared__ float red[16];
    const size_t hh = blockIdx.x;
    const size_t H = a.heads;
    const float A = 0.0f - expf(a.a_log[hh]);
    float sa = 0.0f, sd = 0.0f;
    const size_t n = a.batch * static_cast<size_t>(nck);
    for (size_t j = threadIdx.x; j < n; j += blockDim.x) {
        const size_t bb = j / nck, k = j % nck;
        const size_t bhk = (bb * H + hh) * nck + k;
        sa += w.pa[bhk];
        sd += w.pd[bhk];
    }
    sa = block_sum(sa, red);
    sd = block_sum(sd, red + 8);
    if (threadIdx.x == 0) {
        g.da_log[hh] = A * sa;     // A = -exp(a_log): dA/da_log = A
        if (g.dd_skip != nullptr) g.dd_skip[hh] = sd;
    }
}

// ---------------------------------------------------------------- outgoing last_u
// last_u = sum_r x_{L-1,r} (R(-phi_{L-1}) B_{L-1,r})^T (scan.rs:599-618), so an
// upstream gradient G of it adds, at the last token,
//   dx[p][r]  += sum_n G[p][n] B~[n][r]
//   dB~[n][r]  = sum_p G[p][n] x[p][r],   dB = R(+phi) dB~
//   dphi_i    += sum_r dB~_1 B~_2 - dB~_2 B~_1   (d B~_1/dphi = B~_2, d B~_2/dphi = -B~_1)
// The angle term joins dL/dangle as the seed of the angle gradient's reverse
// cumsum (bwd_angle_kernel); the dx and db terms wait in the workspace for
// bwd_last_add_kernel.  One workgroup per (batch, head).
template <typename T, int N, int R>
__global__ void __launch_bounds__(256) bwd_last_u_kernel(ScanLaunch a, BwdArgs g, BwdWs w) {
    constexpr int NH = N / 2, P = kP;
    __shared__ float sphi[4][NH];
    __shared__ float sx[P * R];
    __shared__ float sb[N * R];      // B~ of the last token
    __shared__ float sdb[N * R];     // dB~
    const int tid = threadIdx.x;
    const size_t bh = blockIdx.x;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const size_t tl = (bb * L + (L - 1)) * H + hh;   // (b, L-1, h)
    // phi_{L-1} = angle0 + sum_t dt_t theta_t, four token stripes per pair
    if (rot) {
        const int i = tid % NH, q = tid / NH;        // NH <= 64: q < 4 covers 256 threads
        float acc = 0.0f;
        if (i < NH && q < 4) {
            for (size_t t = q; t < L; t += 4) {
                const size_t row = (bb * L + t) * H + hh;
                acc += a.dt[row] * ldv<T>(a.theta, row * NH + i);
            }
            sphi[q][i] = acc;
        }
    }
    for (int e = tid; e < P * R; e += 256) sx[e] = ldv<T>(a.x, tl * P * R + e);
    __syncthreads();
    for (int i = tid; i < NH; i += 256) {
        float phi = 0.0f, cs = 1.0f, sn = 0.0f;
        if (rot) {
            phi = sphi[0][i] + sphi[1][i] + sphi[2][i] + sphi[3][i];
            if (a.angle0 != nullptr) phi += a.angle0[bh * NH + i];
            sincosf(wrap_angle(phi), &sn, &cs);
        }
        sphi[0][i] = cs;
        sphi[1][i] = sn;
        for (int r = 0; r < R; ++r) {
            const float b1 = ldv<T>(a.b, (tl * N + i) * R + r);
            const float b2 = ldv<T>(a.b, (tl * N + i + NH) * R + r);
            sb[i * R + r] = b1 * cs + b2 * sn;              // fused.rs:610-617
            sb[(i + NH) * R + r] = -b1 * sn + b2 * cs;
        }
    }
    __syncthreads();
    const float *G = g.dlast_u_out + bh * P * N;
    // dB~[n][r] = sum_p G[p][n] x[p][r]
    for (int e = tid; e < N * R; e += 256) {
        const int n = e / R, r = e % R;
        float acc = 0.0f;
        for (int p = 0; p < P; ++p) acc += G[p * N + n] * sx[p * R + r];
        sdb[e] = acc;
    }
    // dx[p][r] = sum_n G[p][n] B~[n][r]
    for (int e = tid; e < P * R; e += 256) {
        const int p = e / R, r = e % R;
        float acc = 0.0f;
        for (int n = 0; n < N; ++n) acc += G[p * N + n] * sb[n * R + r];
        w.lux[bh * P * R + e] = acc;
    }
    __syncthreads();
    for (int i = tid; i < NH; i += 256) {
        const float cs = sphi[0][i], sn = sphi[1][i];
        float dphi = 0.0f;
        for (int r = 0; r < R; ++r) {
            const float d1 = sdb[i * R + r], d2 = sdb[(i + NH) * R + r];
            dphi += d1 * sb[(i + NH) * R + r] - d2 * sb[i * R + r];
            w.lub[(bh * N + i) * R + r] = d1 * cs - d2 * sn;          // R(+phi) dB~
            w.lub[(bh * N + i + NH) * R + r] = d1 * sn + d2 * cs;
        }
        if (rot) w.seed[bh * NH + i] = (g.dangle_out ? g.dangle_out[bh * NH + i] : 0.0f) + dphi;
    }
}

// The last token's dx and db terms of the outgoing last_u, added to the
// gradients the main passes wrote (in their storage type).
template <typename T, int N, int R>
__global__ void __launch_bounds__(256) bwd_last_add_kernel(ScanLaunch a, BwdArgs g, BwdWs w) {
    constexpr int P = kP;
    const size_t bh = blockIdx.x;
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    const size_t tl = (bb * L + (L - 1)) * H + hh;
    for (int e = threadIdx.x; e < P * R; e += 256)
        stv<T>(g.dx, tl * P * R + e, ldv<T>(g.dx, tl * P * R + e) + w.lux[bh * P * R + e]);
    for (int e = threadIdx.x; e < N * R; e += 256)
        stv<T>(g.db, tl * N * R + e, ldv<T>(g.db, tl * N * R + e) + w.lub[bh * N * R + e]);
}

template <typename K>
hipError_t set_lds(K kern, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

template <typename T, int N, int R, int RW>
hipError_t launch_bwd(const ScanLaunch &a, const BwdArgs &g, char *base, hipStream_t s) {
    const int nck = static_cast<int>((a.seq + RW / R - 1) / (RW / R));
    const size_t bh = a.batch * a.heads, bhk = bh * nck;
    const BwdLayout l = bwd_layout(bh, nck, a.seq, N, R);
    BwdWs w;
    auto f = [base](size_t off) { return reinterpret_cast<float *>(base + off); };
    w.s = f(l.s);
    w.gh = f(l.gh);
    w.eda = f(l.eda);
    w.cin = f(l.cin);
    w.ctot = f(l.ctot);
    w.off = f(l.off);
    w.da = f(l.da);
    w.dg = f(l.dg);
    w.dw = f(l.dw);
    w.pd = f(l.pd);
    w.pa = f(l.pa);
    w.pfirst = f(l.pfirst);
    w.seed = f(l.seed);
    w.lux = f(l.lux);
    w.lub = f(l.lub);

    static_assert(sizeof(Smem<N, R, RW>) <= 160 * 1024, "chunk kernel LDS over 160 KB");
    const size_t lds = sizeof(Smem<N, R, RW>);
    static const hipError_t a2 = set_lds(bwd_chunk_kernel<T, N, R, RW>, lds);
    if (a2 != hipSuccess) return a2;
    hipError_t e;
    BwdArgs gm = g;
    if (g.dlast_u_out != nullptr) {
        // the outgoing last_u's terms; its angle term seeds the angle passes
        hipLaunchKernelGGL((bwd_last_u_kernel<T, N, R>), dim3(bh), dim3(256), 0, s, a, g, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (a.theta != nullptr) gm.dangle_out = w.seed;
    }
    const BwdArgs &g2 = gm;
    hipLaunchKernelGGL((bwd_passes_kernel<T, N, R, RW>), dim3(2 * bh * (N / 32)), dim3(256), 0, s, a, g2, w,
                       nck);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_chunk_kernel<T, N, R, RW>), dim3(bhk), dim3(kBT), lds, s, a, g2, w, nck);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (a.theta != nullptr) {
        hipLaunchKernelGGL((bwd_angle_kernel<N>), dim3(bh), dim3(64), 0, s, a, g2, w, nck);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    hipLaunchKernelGGL((bwd_token_kernel<T, N, R, RW>), dim3(bhk), dim3(256), 0, s, a, g2, w, nck);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_head_kernel, dim3(a.heads), dim3(256), 0, s, a, g2, w, nck);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (g.dlast_u_out != nullptr) {
        hipLaunchKernelGGL((bwd_last_add_kernel<T, N, R>), dim3(bh), dim3(256), 0, s, a, g, w);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

template <typename T, int N64ROWS>
hipError_t launch_bwd_t(const ScanLaunch &a, const BwdArgs &g, char *ws, hipStream_t s) {
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_bwd<T, 128, 1, 32>(a, g, ws, s);
        if (r == 2) return launch_bwd<T, 128, 2, 32>(a, g, ws, s);
        if (r == 4) return launch_bwd<T, 128, 4, 32>(a, g, ws, s);
    } else if (n == 64) {
        if (r == 1) return launch_bwd<T, 64, 1, N64ROWS>(a, g, ws, s);
        if (r == 2) return launch_bwd<T, 64, 2, N64ROWS>(a, g, ws, s);
        if (r == 4) return launch_bwd<T, 64, 4, N64ROWS>(a, g, ws, s);
    }
    return hipErrorNotSupported;
}

}  // namespace

bool scan_backward_supported(const ScanLaunch &a) {
    return a.mode_raw && a.seq > 0 && scan_fast_supported(a);
}

size_t scan_backward_workspace(const ScanLaunch &a) {
    if (!scan_backward_supported(a)) return 0;
    const size_t qt = static_cast<size_t>(scan_backward_rows(a)) / a.rank;
    const size_t nck = (a.seq + qt - 1) / qt;
    return bwd_layout(a.batch * a.heads, nck, a.seq, a.d_state, a.rank).total;
}

hipError_t launch_scan_backward(const ScanLaunch &a, const ScanGrads &gr, void *workspace,
                                hipStream_t stream) {
    if (!scan_backward_supported(a)) return hipErrorNotSupported;
    BwdArgs g;
    g.dy = gr.dy;
    g.dh_out = gr.dh_out;
    g.dangle_out = gr.dangle_out;
    g.dlast_u_out = gr.dlast_u_out;
    g.dx = gr.dx;
    g.db = gr.db;
    g.dc = gr.dc;
    g.ddt = gr.ddt;
    g.dlambda = gr.dlambda;
    g.da_log = gr.da_log;
    g.dtheta = gr.dtheta;
    g.dd_skip = gr.dd_skip;
    g.dh0 = gr.dh0;
    g.dlast_u0 = gr.dlast_u0;
    g.dangle0 = gr.dangle0;
    char *ws = static_cast<char *>(workspace);
    if (a.bf16) return launch_bwd_t<bf16_t, 64>(a, g, ws, stream);
    return launch_bwd_t<float, 32>(a, g, ws, stream);
}

}  // namespace m3
