// Chunked SSD scan for gfx950, specialised for the common shapes:
// head_dim 64, d_state 64 or 128, MIMO rank 1, 2 or 4, f32 or bf16 storage,
// 16-byte aligned operands.  Other shapes take the generic kernel in
// ssd_scan.hip.  Both restate src/ssm/scan.rs:116-291 (ssd_chunked) and
// 458-638 (mamba3_scan) and are checked against the same oracle.
//
// One workgroup of four waves per (batch, head) walks the sequence chunk by
// chunk; the state S (f32) never leaves registers: wave w owns head_dim
// columns [16w, 16w+16).  What differs from the generic kernel is how a chunk
// reaches the chip:
//   * every input of chunk k+1 is requested with 16-byte loads into a second
//     register set while chunk k computes, so HBM latency is off the path;
//   * the thread that loads a (token, pair-slice) of B and C also loads the
//     matching theta slice and rotates them in registers (fused.rs:588-619);
//   * the in-chunk angle prefix (ops/scan.rs:18-51 over dt*theta) is a
//     two-level scan through LDS instead of a serial walk over global memory.
// The MFMA work per chunk (masked C B^T band, carry-in output, state advance,
// band times X) is the same as the generic kernel's.
#include "m3_device.hpp"
#include "m3_internal.hpp"

namespace m3 {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void lds_barrier() {
    // waits for LDS traffic only: prefetched global loads stay in flight
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt untouched
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T> struct Op;
template <> struct Op<bf16_t> {
    using t = __bf16;
    static constexpr int KB = 32;
};
template <> struct Op<float> {
    using t = float;
    static constexpr int KB = 16;
};

// Geometry of one instantiation.  A chunk holds ROWS rows; a row is a
// (token, rank) pair rho = t*R + r (the MIMO fold of scan.rs:537-589).
template <typename T, int N, int P, int R, int ROWS>
struct Geo {
    static constexpr int E = 16 / static_cast<int>(sizeof(T));   // elements per 16 B
    static constexpr int QT = ROWS / R;            // tokens per chunk
    static constexpr int NH = N / 2;               // rotation pairs
    static constexpr int TPT = kThreads / QT;      // threads per token
    static constexpr int PPT = NH / TPT;           // pairs per thread
    static constexpr int HE = PPT * R;             // elements of one half-row slice
    static constexpr int HV = HE / E;              // 16 B vectors per half-row slice
    static constexpr int THB = PPT * static_cast<int>(sizeof(T));   // theta bytes per thread
    static constexpr int TW = THB / 4;             // theta 32-bit words per thread
    static constexpr int XRV = P * R / E;          // x vectors per token row
    static constexpr int XV = ROWS * P / E / kThreads;
    static constexpr int NBLK = kThreads / NH;     // token blocks of the angle prefix
    static constexpr int TB = QT / NBLK;           // tokens per block
    static_assert(QT * TPT == kThreads, "tokens per chunk must divide the workgroup");
    static_assert(PPT * TPT == NH && HV * E == HE && HV >= 1, "pair slices");
    static_assert(TW * 4 == THB && TW >= 1, "theta slices");
    static_assert(XV * kThreads * E == ROWS * P && XV >= 1, "x slices");
    static_assert(NBLK * NH == kThreads && TB * NBLK == QT && TB >= 1, "angle blocks");
    static_assert(P == 64, "four waves own sixteen head_dim columns each");
};

template <typename T, int N, int P, int R, int ROWS>
struct Smem {
    using G = Geo<T, N, P, R, ROWS>;
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;    // pitch of [row][n] operands
    static constexpr int LDR = ROWS + PAD; // pitch of [*][row] operands
    op_t Bs[ROWS * LDN];        // B~[rho][n]
    op_t Cs[ROWS * LDN];        // C~[rho][n]
    op_t Bwt[N * LDR];          // (B~ * w * decay-to-end)^T [n][rho]
    op_t Xt[P * LDR];           // X^T [p][rho]
    op_t Ms[ROWS * LDR];        // masked band (C~ B~^T o L)[rho_t][rho_s]
    static constexpr int PSP = G::NH + 1;   // padded pitch: token rows hit distinct banks
    float psi[G::QT * PSP];     // dt*theta, then the wrapped frame angle [token][pair]
    float tot[G::NBLK * G::NH]; // block totals [block][pair]
    float phis[2][G::NH];       // running wrapped angle entering the chunk (ping-pong)
    float acum[G::QT], gw[G::QT], ww[G::QT], wdec[G::QT], eac[G::QT];
};

// Raw inputs of one chunk as this thread loads them.
template <typename T, int N, int P, int R, int ROWS>
struct Raw {
    using G = Geo<T, N, P, R, ROWS>;
    u32x4 b[2][G::HV];
    u32x4 c[2][G::HV];
    unsigned int th[G::TW];
    u32x4 x[G::XV];
    float dtt;              // dt of this thread's token (angle increments)
    float s0, s1, s2, s3;   // wave 0, lane = token: dt, lambda, dt_next, lambda_next
                            // (or a, g, w for ssd_chunked)
};

template <typename T> __device__ __forceinline__ float elem(const u32x4 *v, int i);
template <> __device__ __forceinline__ float elem<bf16_t>(const u32x4 *v, int i) {
    const unsigned int w = v[i >> 3][(i >> 1) & 3];
    return bf16_bits_to_f32(static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xFFFFu)));
}
template <> __device__ __forceinline__ float elem<float>(const u32x4 *v, int i) {
    return __uint_as_float(v[i >> 2][i & 3]);
}
template <typename T> __device__ __forceinline__ float welem(const unsigned int *w, int i);
template <> __device__ __forceinline__ float welem<bf16_t>(const unsigned int *w, int i) {
    const unsigned int u = w[i >> 1];
    return bf16_bits_to_f32(static_cast<uint16_t>((i & 1) ? (u >> 16) : (u & 0xFFFFu)));
}
template <> __device__ __forceinline__ float welem<float>(const unsigned int *w, int i) {
    return __uint_as_float(w[i]);
}

template <typename O> __device__ __forceinline__ O to_op(float v);
template <> __device__ __forceinline__ float to_op<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 to_op<__bf16>(float v) {
    return static_cast<__bf16>(v);
}
__device__ __forceinline__ float op_f32(float v) { return v; }
__device__ __forceinline__ float op_f32(__bf16 v) { return static_cast<float>(v); }

// Column order of a B~ / C~ row.  For bf16 the columns of each 32-block are
// stored as [g][h][r] instead of [h][g][r] (n = 32kb + 16h + 4g + r): one
// 16-byte read then yields the k-slots an MFMA lane needs both for the band
// (any k order works when both operands share it) and for the carry-in
// product, whose A operand comes straight from the state accumulators.
template <bool BF>
__device__ __forceinline__ int npos(int n) {
    if constexpr (!BF) return n;
    return (n & ~31) | ((n & 12) << 1) | ((n & 16) >> 2) | (n & 3);
}

// Row-position swizzle of the transposed operands (X^T, (B~ w)^T): 16-byte
// blocks of a row are XOR-ed with two bits of the row index, so the staging
// writes -- lanes that differ in row -- spread across LDS banks, while every
// MFMA read still finds its 16 bytes contiguous.
template <int EOP, int GRAN, int MASK>
__device__ __forceinline__ int rswz(int row, int rho) {
    return rho ^ (((row / GRAN) & MASK) * EOP);
}

// exp(clamp(d, -60, 0)), the scan's decay with its log floor (scan.rs:57,
// fused.rs:2064).  bf16 storage takes the hardware exp2; f32 keeps expf.
template <bool FAST>
__device__ __forceinline__ float dexp(float d) {
    d = fminf(fmaxf(d, -60.0f), 0.0f);
    if constexpr (FAST) return __builtin_amdgcn_exp2f(d * 1.44269504088896341f);
    return expf(d);
}

// Store `n` consecutive operand values (n * sizeof(op) a multiple of 4 bytes).
template <int NV>
__device__ __forceinline__ void st_row(__bf16 *dst, const float *v) {
    static_assert(NV % 2 == 0, "pairs of bf16");
#pragma unroll
    for (int i = 0; i < NV; i += 2) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        bf16x2 p;
        p[0] = static_cast<__bf16>(v[i]);
        p[1] = static_cast<__bf16>(v[i + 1]);
        *reinterpret_cast<bf16x2 *>(dst + i) = p;
    }
}
template <int NV>
__device__ __forceinline__ void st_row(float *dst, const float *v) {
#pragma unroll
    for (int i = 0; i < NV; ++i) dst[i] = v[i];
}

__device__ __forceinline__ f32x4 mma_kb(const __bf16 *ar, const __bf16 *br, f32x4 acc, int g) {
    bf16x8 av = *reinterpret_cast<const bf16x8 *>(ar + 8 * g);
    bf16x8 bv = *reinterpret_cast<const bf16x8 *>(br + 8 * g);
    return mfma_bf16(av, bv, acc);
}
__device__ __forceinline__ f32x4 mma_kb(const float *ar, const float *br, f32x4 acc, int g) {
    f32x4 av = *reinterpret_cast<const f32x4 *>(ar + 4 * g);
    f32x4 bv = *reinterpret_cast<const f32x4 *>(br + 4 * g);
    acc = mfma_f32(av[0], bv[0], acc);
    acc = mfma_f32(av[1], bv[1], acc);
    acc = mfma_f32(av[2], bv[2], acc);
    acc = mfma_f32(av[3], bv[3], acc);
    return acc;
}

// Buffer resources of one (batch, head) sequence; offsets are bytes from that
// sequence's token 0, so a token at or past the sequence end reads as zero.
struct SeqBufs {
    rsrc_t b, c, x, th, y, s0, s1, s2, s3;
    uint32_t tok_bc, tok_x, tok_th, tok_s;   // bytes between consecutive tokens
    uint32_t nxt_s;                          // token offset of s2/s3 (1 raw, 0 ssd)
};

// One K block of a 16x16 tile with both operands at this lane's own address
// (already offset to its k-slots).
__device__ __forceinline__ f32x4 mma_at(const __bf16 *a, const __bf16 *b, f32x4 acc) {
    return mfma_bf16(*reinterpret_cast<const bf16x8 *>(a), *reinterpret_cast<const bf16x8 *>(b),
                     acc);
}
__device__ __forceinline__ f32x4 mma_at(const float *a, const float *b, f32x4 acc) {
    const f32x4 av = *reinterpret_cast<const f32x4 *>(a);
    const f32x4 bv = *reinterpret_cast<const f32x4 *>(b);
    acc = mfma_f32(av[0], bv[0], acc);
    acc = mfma_f32(av[1], bv[1], acc);
    acc = mfma_f32(av[2], bv[2], acc);
    acc = mfma_f32(av[3], bv[3], acc);
    return acc;
}

template <typename T, int N, int P, int R, int ROWS>
__device__ __forceinline__ void load_chunk(const SeqBufs &rs, int ck,
                                           Raw<T, N, P, R, ROWS> &raw) {
    using G = Geo<T, N, P, R, ROWS>;
    constexpr uint32_t SZ = sizeof(T);
    const int tid = threadIdx.x;
    const uint32_t tau0 = static_cast<uint32_t>(ck) * G::QT;
    const uint32_t tok = tau0 + tid / G::TPT;
    const uint32_t i0 = (tid % G::TPT) * G::PPT;
    const uint32_t ob = tok * rs.tok_bc;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int v = 0; v < G::HV; ++v) {
            const uint32_t off = ob + ((i0 + h * G::NH) * R + v * G::E) * SZ;
            raw.b[h][v] = bld16(rs.b, off);
            raw.c[h][v] = bld16(rs.c, off);
        }
    const uint32_t ot = tok * rs.tok_th + i0 * SZ;
    if constexpr (G::THB >= 16) {
#pragma unroll
        for (int v = 0; v < G::THB / 16; ++v) {
            const u32x4 q = bld16(rs.th, ot + 16 * v);
#pragma unroll
            for (int j = 0; j < 4; ++j) raw.th[4 * v + j] = q[j];
        }
    } else if constexpr (G::THB == 8) {
        const u32x2 q = bld8(rs.th, ot);
        raw.th[0] = q[0];
        raw.th[1] = q[1];
    } else {
        raw.th[0] = bld4(rs.th, ot);
    }
    raw.dtt = bldf(rs.s0, tok * rs.tok_s);
#pragma unroll
    for (int j = 0; j < G::XV; ++j) {
        const uint32_t v = tid + kThreads * j;
        raw.x[j] = bld16(rs.x, (tau0 + v / G::XRV) * rs.tok_x + (v % G::XRV) * 16u);
    }
    const uint32_t tl = tau0 + (tid & 63);
    raw.s0 = bldf(rs.s0, tl * rs.tok_s);
    raw.s1 = bldf(rs.s1, tl * rs.tok_s);
    raw.s2 = bldf(rs.s2, (tl + rs.nxt_s) * rs.tok_s);
    raw.s3 = bldf(rs.s3, (tl + rs.nxt_s) * rs.tok_s);
}

template <typename T, int N, int P, int R, int ROWS>
__global__ void __launch_bounds__(kThreads, 1)
ssd_scan_fast_kernel(ScanLaunch a, int nchunks) {
    using G = Geo<T, N, P, R, ROWS>;
    using S = Smem<T, N, P, R, ROWS>;
    using RawT = Raw<T, N, P, R, ROWS>;
    using op_t = typename S::op_t;
    constexpr int KB = Op<T>::KB;
    constexpr int LDN = S::LDN, LDR = S::LDR;
    constexpr int QT = G::QT, NH = G::NH, PPT = G::PPT;
    constexpr int NT = ROWS / 16;    // row tiles per chunk
    constexpr int NTN = N / 16;      // state-column tiles
    constexpr bool kBf16 = sizeof(op_t) == 2;
    constexpr uint32_t SZ = sizeof(T);

    extern __shared__ __align__(16) unsigned char smem_raw[];
    S &sm = *reinterpret_cast<S *>(smem_raw);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const size_t H = a.heads, L = a.seq;
    const size_t bb = blockIdx.x / H, hh = blockIdx.x % H;
    const bool rot = a.theta != nullptr;

    // per-sequence buffer resources (token tau of this head at tau * tok bytes)
    SeqBufs rs;
    {
        const size_t row0 = bb * L * H + hh;
        const size_t rows = L * H - hh;
        auto mk = [&](const void *base, size_t row_bytes) {
            return make_rsrc(static_cast<const char *>(base) + row0 * row_bytes,
                             static_cast<uint32_t>(rows * row_bytes));
        };
        rs.b = mk(a.b, N * R * SZ);
        rs.c = mk(a.c, N * R * SZ);
        rs.x = mk(a.x, P * R * SZ);
        rs.y = mk(a.y, P * R * SZ);
        rs.th = rot ? mk(a.theta, NH * SZ) : make_rsrc(a.x, 0u);   // no records: zeros
        if (a.mode_raw) {
            rs.s0 = rs.s2 = mk(a.dt, 4);
            rs.s1 = rs.s3 = mk(a.lambda, 4);
            rs.nxt_s = 1;
        } else {
            rs.s0 = mk(a.a, 4);
            rs.s1 = mk(a.g, 4);
            rs.s2 = mk(a.w, 4);
            rs.s3 = make_rsrc(a.a, 0u);
            rs.nxt_s = 0;
        }
        rs.tok_bc = static_cast<uint32_t>(H * N * R * SZ);
        rs.tok_x = static_cast<uint32_t>(H * P * R * SZ);
        rs.tok_th = static_cast<uint32_t>(H * NH * SZ);
        rs.tok_s = static_cast<uint32_t>(H * 4);
    }

    // thread's (token, pair-slice) in the rotation mapping
    const int my_t = tid / G::TPT;
    const int i0 = (tid % G::TPT) * PPT;

    RawT bufA, bufB;
    load_chunk<T, N, P, R, ROWS>(rs, 0, bufA);

    // zero the operand buffers once: pads and the never-written upper band tiles
    {
        uint32_t *z = reinterpret_cast<uint32_t *>(smem_raw);
        const int words = static_cast<int>(sizeof(S) / 4);
        for (int i = tid; i < words; i += kThreads) z[i] = 0u;
    }

    // state registers: S^T[n][p] tiles, lane holds n = 16i + 4g + r, p = 16w + c
    f32x4 st[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) st[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int pcol = 16 * wave + c;
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
            for (int i = 0; i < NTN; ++i) {
                const size_t o = sbase + pcol * N + 16 * i + 4 * g;
                f32x4 v = *reinterpret_cast<const f32x4 *>(h0 + o);
                if (l0 != nullptr) v += *reinterpret_cast<const f32x4 *>(l0 + o) * first;
                st[i] = v;
            }
        }
    }
    // running wrapped frame angle entering the first chunk
    if (rot) {
        for (int i = tid; i < NH; i += kThreads)
            sm.phis[0][i] = a.angle0 ? a.angle0[(bb * H + hh) * NH + i] : 0.0f;
    }

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const bool skip = a.d_skip != nullptr;
    __syncthreads();

    // column position of a B~/C~ element, row position in X^T / (B~ w)^T
    constexpr int EOP = 16 / static_cast<int>(sizeof(op_t));
    constexpr int XGRAN = (G::E / R) > 0 ? (G::E / R) : 1;
    constexpr int SMASK = (ROWS / EOP) - 1 < 7 ? (ROWS / EOP) - 1 : 7;
    auto bwpos = [&](int n, int rho) { return n * LDR + rswz<EOP, PPT, SMASK>(n, rho); };
    auto xtpos = [&](int p, int rho) { return p * LDR + rswz<EOP, XGRAN, SMASK>(p, rho); };

    auto body = [&](int ck, RawT &cur, RawT &nxt) {
        const size_t tau0 = static_cast<size_t>(ck) * QT;
        // the next chunk's inputs; past the end they read as zeros
        load_chunk<T, N, P, R, ROWS>(rs, ck + 1, nxt);

        // ================= P1: X^T, per-token scalars, angle increments
#pragma unroll
        for (int j = 0; j < G::XV; ++j) {
            const int v = tid + kThreads * j;
            const int tx = v / G::XRV;
            const int o = (v % G::XRV) * G::E;
#pragma unroll
            for (int e = 0; e < G::E; ++e) {
                const int p = (o + e) / R, r = (o + e) % R;
                sm.Xt[xtpos(p, tx * R + r)] = to_op<op_t>(elem<T>(&cur.x[j], e));
            }
        }
        if (wave == 0) {
            const int t = lane;
            const bool live = t < QT && tau0 + t < L;
            float av = 0.f, gv = 0.f, wv = 0.f;
            if (live) {
                if (a.mode_raw) {
                    av = cur.s0 * A;
                    gv = cur.s1 * cur.s0;                        // fused.rs:2494
                    wv = gv + (1.0f - cur.s3) * cur.s2;          // fused.rs:2496-2498
                } else {
                    av = cur.s0;
                    gv = cur.s1;
                    wv = cur.s2;
                }
            }
            const float acum = wave_inclusive_scan(av, lane);
            const float last = __shfl(acum, QT - 1, 64);
            if (t < QT) {
                sm.acum[t] = acum;
                sm.gw[t] = gv;
                sm.ww[t] = wv;
                sm.wdec[t] = dexp<kBf16>(last - acum) * wv;   // exp_decay(last, acum, w)
                sm.eac[t] = dexp<kBf16>(acum);                // exp_decay(acum)
            }
        }
        if (rot) {
#pragma unroll
            for (int j = 0; j < PPT; ++j)
                sm.psi[my_t * S::PSP + i0 + j] = cur.dtt * welem<T>(cur.th, j);
        }
        lds_barrier();

        // ================= P2: frame angle of every (token, pair) of the chunk
        // (ops/scan.rs:18-51 on dt*theta, then elemwise.rs:349's wrap): an
        // in-block prefix, block offsets, and the running angle entering the chunk
        if (rot) {
            const int i = tid % NH, blk = tid / NH;
            float pv[G::TB];
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < G::TB; ++j) pv[j] = sm.psi[(blk * G::TB + j) * S::PSP + i];
#pragma unroll
            for (int j = 0; j < G::TB; ++j) {
                acc += pv[j];
                pv[j] = acc;
            }
            sm.tot[blk * NH + i] = acc;
            lds_barrier();
            float base = sm.phis[ck & 1][i];
#pragma unroll
            for (int k = 0; k < G::NBLK - 1; ++k)
                if (k < blk) base += sm.tot[k * NH + i];
#pragma unroll
            for (int j = 0; j < G::TB; ++j)
                sm.psi[(blk * G::TB + j) * S::PSP + i] = wrap_angle(base + pv[j]);
            if (blk == G::NBLK - 1) sm.phis[(ck + 1) & 1][i] = wrap_angle(base + acc);
            lds_barrier();
        }

        // ================= P3: rotate B and C in registers, stage operands
        {
            const size_t tau = tau0 + my_t;
            const float wd = sm.wdec[my_t];
            float cs[PPT], sn[PPT];
#pragma unroll
            for (int j = 0; j < PPT; ++j) {
                cs[j] = 1.0f;
                sn[j] = 0.0f;
            }
            if (rot) {
#pragma unroll
                for (int j = 0; j < PPT; ++j) {
                    const float phi = sm.psi[my_t * S::PSP + i0 + j];
                    if (a.angle_out && tau == L - 1)
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
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = my_t * R + r;
                float rb[2][PPT], rc[2][PPT];
#pragma unroll
                for (int j = 0; j < PPT; ++j) {
                    const float b1 = elem<T>(cur.b[0], j * R + r);
                    const float b2 = elem<T>(cur.b[1], j * R + r);
                    const float c1 = elem<T>(cur.c[0], j * R + r);
                    const float c2 = elem<T>(cur.c[1], j * R + r);
                    // rotation by -phi (fused.rs:610-617); identity without theta
                    rb[0][j] = b1 * cs[j] + b2 * sn[j];
                    rb[1][j] = -b1 * sn[j] + b2 * cs[j];
                    rc[0][j] = c1 * cs[j] + c2 * sn[j];
                    rc[1][j] = -c1 * sn[j] + c2 * cs[j];
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // groups of four consecutive columns stay contiguous under npos
#pragma unroll
                    for (int q = 0; q < PPT; q += 4) {
                        const int n = i0 + h * NH + q;
                        if constexpr (PPT >= 4) {
                            st_row<4>(&sm.Bs[rho * LDN + npos<kBf16>(n)], &rb[h][q]);
                            st_row<4>(&sm.Cs[rho * LDN + npos<kBf16>(n)], &rc[h][q]);
                        }
                    }
                    if constexpr (PPT < 4) {
#pragma unroll
                        for (int j = 0; j < PPT; ++j) {
                            const int n = i0 + h * NH + j;
                            sm.Bs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rb[h][j]);
                            sm.Cs[rho * LDN + npos<kBf16>(n)] = to_op<op_t>(rc[h][j]);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < PPT; ++j)
                        sm.Bwt[bwpos(i0 + h * NH + j, rho)] = to_op<op_t>(rb[h][j] * wd);
                }
            }
        }
        lds_barrier();

        // ================= P4: band -> Ms, carry-in output, state advance
        f32x4 yacc[NT];
        {
            int idx = 0;
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const int tlast = (16 * tj + 15) / R;
#pragma unroll
                for (int si = 0; si < NT; ++si) {
                    if ((16 * si) / R > tlast) continue;
                    if ((idx++) % 4 != wave) continue;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *ar = &sm.Bs[(16 * si + c) * LDN];
                    const op_t *br = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
                    for (int kb = 0; kb < N / KB; ++kb)
                        acc = mma_kb(ar + kb * KB, br + kb * KB, acc, g);
                    const int trow = 16 * tj + c;
                    const int tt = trow / R;
                    const float at = sm.acum[tt];
                    float vals[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int srow = 16 * si + 4 * g + r;
                        const int ts = srow / R;
                        float v = 0.0f;
                        if (ts <= tt) {
                            const float wgt = (ts == tt) ? sm.gw[ts] : sm.ww[ts];
                            v = acc[r] * wgt * dexp<kBf16>(at - sm.acum[ts]);
                        }
                        // the skip D x rides on the band's diagonal (scan.rs:593-597)
                        if (skip && srow == trow) v += dskip;
                        vals[r] = v;
                    }
                    op_t *dst = &sm.Ms[trow * LDR + 16 * si + 4 * g];
                    st_row<4>(dst, vals);
                }
            }

            // carry-in output: y^T[p][t] = exp(acum_t) * sum_n S[p][n] C~[t][n]
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
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const op_t *cr = &sm.Cs[(16 * tj + c) * LDN];
#pragma unroll
                    for (int kb = 0; kb < N / 32; ++kb)
                        acc = mfma_bf16(sa[kb], *reinterpret_cast<const bf16x8 *>(cr + 32 * kb + 8 * g),
                                        acc);
                    yacc[tj] = acc * sm.eac[(16 * tj + c) / R];
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
                    yacc[tj] = acc * sm.eac[(16 * tj + c) / R];
                }
            }

            // state advance: S^T = exp(dA) S^T + (B~ w decay)^T X
            const float edA = dexp<kBf16>(sm.acum[QT - 1]);
            const int prow = 16 * wave + c;
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                f32x4 acc = st[i] * edA;
                const int nrow = 16 * i + c;
#pragma unroll
                for (int kb = 0; kb < ROWS / KB; ++kb)
                    acc = mma_at(&sm.Bwt[bwpos(nrow, kb * KB + EOP * g)],
                                 &sm.Xt[xtpos(prow, kb * KB + EOP * g)], acc);
                st[i] = acc;
            }
        }
        lds_barrier();

        // ================= P5: y += (band o C B^T) X, store
        {
            const int prow = 16 * wave + c;
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const op_t *mr = &sm.Ms[(16 * tj + c) * LDR];
                const int tlast = (16 * tj + 15) / R;
                const int send = (tlast + 1) * R < ROWS ? (tlast + 1) * R : ROWS;
                const int nkb = (send + KB - 1) / KB;
#pragma unroll
                for (int kb = 0; kb < ROWS / KB; ++kb)
                    if (kb < nkb)
                        yacc[tj] = mma_at(&sm.Xt[xtpos(prow, kb * KB + EOP * g)],
                                          mr + kb * KB + EOP * g, yacc[tj]);
            }
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const int rho = 16 * tj + c;
                const int rr = rho % R;
                const uint32_t tau = static_cast<uint32_t>(tau0) + rho / R;
                const f32x4 v = yacc[tj];
                // rows past the sequence end fall outside the buffer: dropped
                const uint32_t oy = tau * rs.tok_x + ((16 * wave + 4 * g) * R + rr) * SZ;
                if constexpr (R == 1) {
                    if constexpr (kBf16) {
                        u32x2 pk;
                        pk[0] = static_cast<unsigned int>(from_f32<bf16_t>(v[0]).bits) |
                                (static_cast<unsigned int>(from_f32<bf16_t>(v[1]).bits) << 16);
                        pk[1] = static_cast<unsigned int>(from_f32<bf16_t>(v[2]).bits) |
                                (static_cast<unsigned int>(from_f32<bf16_t>(v[3]).bits) << 16);
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
        }
        lds_barrier();
    };

    for (int ck = 0; ck < nchunks; ck += 2) {
        body(ck, bufA, bufB);
        if (ck + 1 < nchunks) body(ck + 1, bufB, bufA);
    }

    // ---- boundary state (scan.rs:270-288, 599-638)
    if (a.h_out != nullptr) {
#pragma unroll
        for (int i = 0; i < NTN; ++i)
            *reinterpret_cast<f32x4 *>(a.h_out + sbase + pcol * N + 16 * i + 4 * g) = st[i];
    }
    if (a.last_u_out != nullptr) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T, from the final chunk's LDS tiles
        const int tl = static_cast<int>((L - 1) - static_cast<size_t>(nchunks - 1) * QT);
        for (int it = tid; it < P * N; it += kThreads) {
            const int p = it / N;
            const int n = it - p * N;
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int rho = tl * R + r;
                acc += op_f32(sm.Xt[xtpos(p, rho)]) * op_f32(sm.Bs[rho * LDN + npos<kBf16>(n)]);
            }
            a.last_u_out[sbase + it] = acc;
        }
    }
}

template <typename T, int N, int R, int ROWS>
hipError_t launch_one(const ScanLaunch &a, hipStream_t s) {
    constexpr int P = 64;
    using Sm = Smem<T, N, P, R, ROWS>;
    using G = Geo<T, N, P, R, ROWS>;
    const int nchunks = static_cast<int>((a.seq + G::QT - 1) / G::QT);
    const size_t smem = sizeof(Sm);
    auto kern = ssd_scan_fast_kernel<T, N, P, R, ROWS>;
    static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(smem));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(a.batch * a.heads), dim3(kThreads), smem, s, a, nchunks);
    return hipGetLastError();
}

template <typename T, int ROWS>
hipError_t launch_t(const ScanLaunch &a, hipStream_t s) {
    const size_t n = a.d_state, r = a.rank;
    if (n == 128) {
        if (r == 1) return launch_one<T, 128, 1, ROWS>(a, s);
        if (r == 2) return launch_one<T, 128, 2, ROWS>(a, s);
        if (r == 4) return launch_one<T, 128, 4, ROWS>(a, s);
    } else if (n == 64) {
        if (r == 1) return launch_one<T, 64, 1, ROWS>(a, s);
        if (r == 2) return launch_one<T, 64, 2, ROWS>(a, s);
        if (r == 4) return launch_one<T, 64, 4, ROWS>(a, s);
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
    return true;
}

hipError_t launch_scan_fast(const ScanLaunch &a, hipStream_t stream) {
    if (!scan_fast_supported(a)) return hipErrorNotSupported;
    if (a.bf16) return launch_t<bf16_t, 64>(a, stream);
    return launch_t<float, 32>(a, stream);
}

}  // namespace m3
