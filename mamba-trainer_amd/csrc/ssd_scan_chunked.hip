// Chunked SSD scan for gfx950 as three chunk-parallel launches over a caller
// workspace.  Same shapes as ssd_scan_fast.hip (head_dim 64, d_state 64/128,
// rank 1/2/4, aligned operands) and the same algorithm, src/ssm/scan.rs:116-291
// (ssd_chunked) and 458-638 (mamba3_scan), regrouped so that only an
// elementwise recurrence runs in sequence.  A sequence is cut into segments of
// kseg sub-chunks (64 rows of (token, rank) for bf16, 32 for f32):
//
//   chunk_state_kernel  one workgroup per (batch, head, segment).  In the
//       segment's own rotating frame (angles relative to the segment start, so
//       nothing from earlier segments is needed) it forms
//       U = sum_s (B_s w_s decay_s)^T x_s, the segment's contribution to the
//       state (scan.rs:207-251), sub-chunk by sub-chunk, with the segment's
//       decay exp(sum dt A) and, per rotation pair, its angle total Phi with
//       its cosine and sine.
//   state_pass_kernel   one thread per (batch, head, p, four state pairs):
//       S_0 = R(angle0) h0 and S_{j+1} = R(Phi_j) (decay_j S_j + U_j), the
//       state entering each segment expressed in that segment's frame, written
//       as MFMA operand fragments; at the end the boundary state in the global
//       frame (scan.rs:270-288, 599-638).
//   chunk_scan_kernel   one workgroup per (batch, head, segment), its
//       sub-chunks in turn from the segment's S:
//       y = (C~ B~^T o L) X + exp(acum) C~ S  (ssd_band fused.rs:2044-2070,
//       scan.rs:253-263), the skip D on the band's diagonal (scan.rs:593-597),
//       then S advanced in registers to the next sub-chunk.
//
// Frames.  With phi_t the running angle and phi^s its value entering a
// segment, B~_t = R(-phi_t) B_t = R(-phi^s) B^(s)_t where B^(s)_t is B_t rotated
// by its angle relative to the segment start.  The state in the segment's
// frame is S = R(phi^s) h, so C~_t . h = C^(s)_t . S; within the segment the
// state advances without rotation, and moving to the next segment's frame is a
// rotation of every (n, n + N/2) pair by the segment total Phi.
//
// Why three launches: a batch x head count of ~100 sequences fills under half
// of the chip's 256 CUs when each sequence is walked by one workgroup, and
// every sub-chunk's rotation (a sine and cosine per token and pair), decay
// weights and band are latency-bound there.  Here both heavy passes spread
// over every segment of every sequence; the sequential pass is a few FMAs per
// element and streams U from HBM.  Segments of several sub-chunks keep the U
// and S records (and the state pass) small while still filling the chip.
#include <type_traits>

#include "scan_common.hpp"
#include "mixer_math.hpp"

namespace m3 {

namespace {

using namespace scan;

constexpr int kP = 64;   // head_dim of these kernels
// State values (pairs) per thread of the state pass: all four of a lane's
// values in a record tile.  The pass is bound by its memory instructions, not
// by the threads in flight: splitting a lane's four over two or four threads
// measured 1.6x and 2.7x slower at config 1 (MI355X).
constexpr int kStatePairs = 4;

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
    void *u;        // [bhs][p-tile][n-tile][lane][4]: U^T tiles in MFMA D layout
    void *s;        // as u: S^T tiles of the state entering each segment
    float *eda;     // [bhs] exp(sum of the clamped dt A of each sub-chunk)
    float *phi;     // [bhs][N/2] angle total of the segment per pair (wrapped)
    float *cph;     // [bhs][N/2] cos Phi
    float *sph;     // [bhs][N/2] sin Phi
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
// Element offset, within one (segment, p-tile) record of NTN n-tiles, of a
// lane's four values of n-tile i (the MFMA D layout: n = 16 i + 4 g + r,
// p = 16 w + c).  The tiles of a rotation pair's two halves, i and
// i + NTN / 2, sit side by side per lane, so a 16-byte access (bf16) moves
// both halves: the state pass, which rotates each pair, reads and writes one
// vector per record and lane.
template <int NTN>
__device__ __forceinline__ size_t rec_off(int i, int lane) {
    constexpr int HT = NTN / 2;
    return static_cast<size_t>(i % HT) * 512 + static_cast<size_t>(lane) * 8 + (i / HT) * 4;
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
    // unpadded swizzled tiles (swz): 24.8 KB at N = 128, so six workgroups
    // share a CU
    op_t Bwt[N * ROWS];     // (B~ * w * decay-to-end)^T [n][rho], segment frame
    op_t Xt[kP * ROWS];     // X^T [p][rho]
    // wrapped angle per pair entering the sub-chunk, relative to the segment
    // start; each pair is read and rewritten by the one wave whose lanes own
    // it, so one copy serves every sub-chunk (a wave's LDS accesses execute
    // in order)
    float psi[N / 2];
};

// One workgroup per (batch, head, segment).  A segment is `kseg` sub-chunks
// of ROWS rows (ROWS / R tokens each), staged one after the other.  B is
// rotated by its angle relative to the segment start (a running wrapped
// angle per pair, as the single pass carries it), so every sub-chunk's
// contribution U_h is already in the segment's frame and the segment's U is
// U = e_h U + U_h over the sub-chunks: the state recurrence of
// scan.rs:207-251 composed over the segment.  The segment's decay and angle
// total (with its cosine and sine) go to the workspace beside U.  PF: the
// next sub-chunk's inputs are loaded into registers behind the current one's
// work.
template <typename T, int N, int R, int ROWS, bool PF>
__global__ void __launch_bounds__(kThreads, 2)
chunk_state_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    using G = Geo<T, N, P, R, ROWS, 4>;
    using S = StateSmem<T, N, R, ROWS>;
    using RawT = Raw<T, N, P, R, ROWS, 4, false>;
    using op_t = typename S::op_t;
    constexpr int KB = sizeof(typename S::op_t) == 2 ? 32 : 16;
    constexpr int E16 = 16 / static_cast<int>(sizeof(op_t));
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
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)

    // U^T[n][p] of this wave's p-tile, the segment's decay, and the wrapped
    // angle of my pairs relative to the segment start
    f32x4 uacc[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) uacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float eacc = 1.0f;
    if (tid < NH) sm.psi[tid] = 0.0f;
    constexpr bool kUni = G::SUBS == 1;   // pair angles wave-uniform (pair_angle)
    float run[kUni ? PPL : 1];
#pragma unroll
    for (int j = 0; j < (kUni ? PPL : 1); ++j) run[j] = 0.0f;
    __syncthreads();

    const int h_end = min(kseg, nsub - seg * kseg);
    RawT cur, nxt;
    if constexpr (PF) load_chunk<T, N, P, R, ROWS, 4, false>(rs, seg * kseg, wave, lane, nxt);
#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
        // lane-derived indices from an opaque copy of the lane number, so the
        // LDS addresses they feed are formed in the loop, not held across it
        int lane_v = lane;
        asm volatile("" : "+v"(lane_v));
        const int lane = lane_v;
        const int g = lane >> 4;
        const int c = lane & 15;
        const int sub = lane / G::SW;
        const int my_t = lane % G::SW;
        const bool tok_lane = my_t < QT;
        const int i0 = wave * G::PW + sub * PPL;
        const int sck = seg * kseg + h;
        if constexpr (PF) {
            cur = nxt;
            if (h + 1 < h_end) load_chunk<T, N, P, R, ROWS, 4, false>(rs, sck + 1, wave, lane, nxt);
        } else {
            load_chunk<T, N, P, R, ROWS, 4, false>(rs, sck, wave, lane, cur);
        }

        const size_t tau = static_cast<size_t>(sck) * QT + my_t;
        const bool live = tok_lane && tau < L;
        float av, gv, wv;
        token_scalars(a, cur, A, live, av, gv, wv);
        const float acum = seg_scan<G::SW>(av);
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        const float wd = dexp<kBf16>(last - acum) * wv;   // exp_decay(last, acum, w)
        const float eh = dexp<kBf16>(last);

        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / 4) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                sm.Xt[swz<op_t, ROWS>(p, my_t * R + r)] = op_elem<T>(cur.x, e);
            }
        }
        // per pair: the angle within the segment (the running angle plus the
        // in-sub-chunk inclusive cumsum of dt * theta), its sine and cosine,
        // and B rotated by its negative (fused.rs:610-617), weighted and
        // stored -- one pair's values live at a time.  Without theta its
        // loads read zeros: every angle is 0 (cosine 1, sine 0), with no
        // branch to keep the pairs from interleaving.
        const float dtt = live ? cur.s0 : 0.0f;
        // the prefixes four pairs at a time (interleaved DPP chains)
        constexpr int GP = PPL % 4 == 0 ? 4 : 1;
        float pre[GP];
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            float cs, sn;
            if (j % GP == 0) {
#pragma unroll
                for (int jj = 0; jj < GP; ++jj) pre[jj] = dtt * welem<T>(cur.th, j + jj);
                if constexpr (GP == 4)
                    seg_scan4<G::SW>(pre[0], pre[1], pre[2], pre[3]);
                else
                    pre[0] = seg_scan<G::SW>(pre[0]);
            }
            {
                const float phi = pair_angle<kUni, QT>(pre[j % GP], run[kUni ? j : 0],
                                                       &sm.psi[i0 + j], my_t == QT - 1);
                if constexpr (kBf16) {
                    // the hardware sine takes revolutions; |phi| <= pi
                    const float rev = phi * 0.15915494309189533577f;
                    sn = __builtin_amdgcn_sinf(rev);
                    cs = __builtin_amdgcn_cosf(rev);
                } else {
                    sincosf(phi, &sn, &cs);
                }
            }
            if (tok_lane) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int rho = my_t * R + r;
                    const float b1 = elem<T>(cur.b[0], j * R + r);
                    const float b2 = elem<T>(cur.b[1], j * R + r);
                    sm.Bwt[swz<op_t, ROWS>(i0 + j, rho)] = to_op<op_t>((b1 * cs + b2 * sn) * wd);
                    sm.Bwt[swz<op_t, ROWS>(i0 + NH + j, rho)] =
                        to_op<op_t>((-b1 * sn + b2 * cs) * wd);
                }
            }
        }
        __syncthreads();

        // U = e_h U + U_h, U_h^T[n][p] = sum_rho Bwt[n][rho] X^T[p][rho]; wave w
        // takes p-tile w
        // (rows 16 i + c share the swizzle of row c: one column offset per kb)
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            f32x4 acc = uacc[i] * eh;
#pragma unroll
            for (int kb = 0; kb < ROWS / KB; ++kb) {
                const int col = kb * KB + g * E16;
                acc = mma_kb(&sm.Bwt[swz<op_t, ROWS>(16 * i + c, col)],
                             &sm.Xt[swz<op_t, ROWS>(16 * wave + c, col)], acc, 0);
            }
            uacc[i] = acc;
        }
        eacc *= eh;
        __syncthreads();   // every read of this sub-chunk's LDS is done
    }

    const size_t uo = (bhs * 4 + wave) * NTN * 256;
#pragma unroll
    for (int i = 0; i < NTN; ++i) store_u<kBf16>(ws.u, uo + rec_off<NTN>(i, lane), uacc[i]);
    if (tid == 0) ws.eda[bhs] = eacc;
    if constexpr (kUni) {   // each wave's pair angles into LDS
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < PPL; ++j) sm.psi[i0 + j] = run[j];
        }
        __syncthreads();
    }
    // the segment's angle total per pair (wrapped), with its cosine and sine:
    // one thread per pair (the loop's last barrier ordered the angle writes)
    if (tid < NH) {
        const float tot = rot ? sm.psi[tid] : 0.0f;
        float ts = 0.0f, tc = 1.0f;
        if (rot) sincosf(tot, &ts, &tc);
        ws.phi[bhs * NH + tid] = tot;
        ws.cph[bhs * NH + tid] = tc;
        ws.sph[bhs * NH + tid] = ts;
    }
}

// The same for bf16 storage at rank 1, with the inputs staged by coalesced
// direct-to-LDS loads.  Lane = token loads put each lane of a load
// instruction on its own cache line (rows of one head are H * N * 2 bytes
// apart), and the L1's per-line work, not HBM, then bounds the kernel; here
// each instruction fetches whole rows (eight lines a kilobyte) into raw row
// tiles (rsw).  The stage reads its pair slices from the tiles, and writes B
// rotated and weighted back in place; the MFMA takes (B~w)^T and X^T from the
// row-major tiles by transposed reads.
//
// The loads are pipelined one sub-chunk ahead.  theta, X and the per-token
// scalars are double-buffered and fetched at the start of the previous
// sub-chunk; B, single-buffered, is fetched once the previous MFMA has read
// it, and arrives while the stage forms the angles, sines and cosines (which
// need theta only).  The waits count this wave's loads in issue order
// (vmcnt; the loop issues no stores).
template <int N>
struct StateDmaSmem {
    static constexpr int CB = N / 8, CT = N / 16, CX = kP / 8;   // chunks per row
    unsigned char b[64 * CB * 16];       // B, then B~ w decay-to-end, [t][n]
    unsigned char th[2][64 * CT * 16];   // theta [t][pair]; the pair angle totals at the end
    unsigned char x[2][64 * CX * 16];    // X [t][p]
    float sc[2][4][64];                  // dt, lambda, next dt, next lambda (or a, g, w)
};

template <int N>
__global__ void __launch_bounds__(kThreads, 2)
chunk_state_dma_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    using G = Geo<bf16_t, N, P, 1, 64, 4>;
    using S = StateDmaSmem<N>;
    constexpr int CB = S::CB, CT = S::CT, CX = S::CX;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL, PW = G::PW;
    constexpr int NTN = N / 16;
    constexpr int HV = PW / 8;        // 16-byte chunks of a lane's half-row slice
    static_assert(G::SUBS == 1 && QT == 64 && PPL == PW, "lane = token, one segment per wave");
    static_assert(CB % 4 == 0 && CT % 4 == 0 && CX % 4 == 0, "row loads spread over four waves");
    // load instructions a wave issues per sub-chunk: theta + X + one scalar, and B
    constexpr int kTX = CT / 4 + CX / 4 + 1, kB = CB / 4;

    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const size_t H = a.heads, L = a.seq;
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;
    const SeqBufs rs = seq_bufs<bf16_t, N, P, 1>(a, bb, hh);

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)

    // theta, X and the scalars of sub-chunk k into buffer k & 1; B of sub-chunk k
    auto load_tx = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
        const int buf = k & 1;
#pragma unroll
        for (int q = 0; q < CT / 4; ++q)
            lds_load_rows<CT>(rs.th, tok0 * rs.tok_th, rs.tok_th, sm.th[buf], wave + 4 * q, lane);
#pragma unroll
        for (int q = 0; q < CX / 4; ++q)
            lds_load_rows<CX>(rs.x, tok0 * rs.tok_x, rs.tok_x, sm.x[buf], wave + 4 * q, lane);
        // wave w fetches scalar w: s0, s1 at the token, s2, s3 at the next one
        // (a uniform branch per resource: a selected resource would go
        // through scratch)
        const uint32_t dst = lds_addr(&sm.sc[buf][wave][0]);
        const uint32_t o0 = (tok0 + lane) * rs.tok_s, o1 = (tok0 + rs.nxt_s + lane) * rs.tok_s;
        switch (wave) {
        case 0: lds_dma4(rs.s0, dst, o0); break;
        case 1: lds_dma4(rs.s1, dst, o0); break;
        case 2: lds_dma4(rs.s2, dst, o1); break;
        default: lds_dma4(rs.s3, dst, o1); break;
        }
    };
    auto load_b = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < CB / 4; ++q)
            lds_load_rows<CB>(rs.b, tok0 * rs.tok_bc, rs.tok_bc, sm.b, wave + 4 * q, lane);
    };

    f32x4 uacc[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) uacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float eacc = 1.0f;
    float run[PPL];   // wave-uniform running pair angles, in turns (pair_turns)
#pragma unroll
    for (int j = 0; j < PPL; ++j) run[j] = 0.0f;

    const int h_end = min(kseg, nsub - seg * kseg);
    load_tx(seg * kseg);
    load_b(seg * kseg);
#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
        int lane_v = lane;
        asm volatile("" : "+v"(lane_v));
        const int lane = lane_v;
        const int g = lane >> 4;
        const int c = lane & 15;
        const int sck = seg * kseg + h;
        const int buf = sck & 1;
        const bool more = h + 1 < h_end;

        // theta, X, scalars of this sub-chunk landed (only its B may be out)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kB>());
        __syncthreads();
        if (more) load_tx(sck + 1);

        TokScalars sc;
        sc.s0 = sm.sc[buf][0][lane];
        sc.s1 = sm.sc[buf][1][lane];
        sc.s2 = sm.sc[buf][2][lane];
        sc.s3 = sm.sc[buf][3][lane];
        const bool live = static_cast<size_t>(sck) * QT + lane < L;
        float av, gv, wv;
        token_scalars(a, sc, A, live, av, gv, wv);
        const float acum = seg_scan<64>(av);
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        const float wd = dexp<true>(last - acum) * wv;   // exp_decay(last, acum, w)
        const float eh = dexp<true>(last);
        // dt / 2 pi: the pair angles are carried in turns (pair_turns)
        const float dtt = live ? sc.s0 * 0.15915494309189533577f : 0.0f;

        // ---- stage, first half: every pair's angle within the segment and its
        //      sine and cosine (theta only; B is still arriving)
        const int i0 = wave * PW;
        float cs[PPL], sn[PPL];
        {
            u32x4 th[HV];
#pragma unroll
            for (int v = 0; v < HV; ++v)
                th[v] = *reinterpret_cast<const u32x4 *>(sm.th[buf] + rtile_off<CT>(lane, i0 + 8 * v));
#pragma unroll
            for (int q = 0; q < PPL; q += 4) {
                float pre[4];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) pre[jj] = dtt * elem<bf16_t>(th, q + jj);
                seg_scan4<64>(pre[0], pre[1], pre[2], pre[3]);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float w = pair_turns(pre[jj], run[q + jj]);
                    sn[q + jj] = __builtin_amdgcn_sinf(w);
                    cs[q + jj] = __builtin_amdgcn_cosf(w);
                }
            }
        }
        // B landed (the next sub-chunk's theta, X and scalars may be out)
        if (more)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<kTX>());
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
        __syncthreads();

        // ---- stage, second half: B rotated by the negative angle (fused.rs:610-617)
        //      and weighted, back in place, eight pairs (one chunk of each
        //      half-row) at a time
#pragma unroll
        for (int v = 0; v < HV; ++v) {
            u32x4 bv[2], out[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                bv[hf] = *reinterpret_cast<const u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v));
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float o[2][2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int j = 8 * v + e + u;
                    const float b1 = elem<bf16_t>(bv, e + u), b2 = elem<bf16_t>(bv + 1, e + u);
                    o[0][u] = (b1 * cs[j] + b2 * sn[j]) * wd;
                    o[1][u] = (-b1 * sn[j] + b2 * cs[j]) * wd;
                }
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) out[hf][e >> 1] = pk_bf16(o[hf][0], o[hf][1]);
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                *reinterpret_cast<u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v)) = out[hf];
        }
        __syncthreads();

        // ---- U = e_h U + U_h, U_h^T[n][p] = sum_rho (B~w)[rho][n] X[rho][p]:
        // A operand (n = 16 i + c, k = rho = 32 kb + 8 g + 0..7) and B operand
        // (p = 16 wave + c, same k) by two transposed reads each
        {
            const int r0 = 8 * g + (c >> 2);
            const int cq = 4 * (c & 3);
            bf16x8 xo[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(
                    sm.x[buf] + rtile_off<CX>(32 * kb + r0, 16 * wave + cq)));
                const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(
                    sm.x[buf] + rtile_off<CX>(32 * kb + r0 + 4, 16 * wave + cq)));
                xo[kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            // every fragment read first, so the LDS reads stream back to back
            // and the products follow without a wait between them
            bf16x8 av[NTN][2];
#pragma unroll
            for (int i = 0; i < NTN; ++i)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(
                        sm.b + rtile_off<CB>(32 * kb + r0, 16 * i + cq)));
                    const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(
                        sm.b + rtile_off<CB>(32 * kb + r0 + 4, 16 * i + cq)));
                    av[i][kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                f32x4 acc = uacc[i] * eh;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) acc = mfma_bf16(av[i][kb], xo[kb], acc);
                uacc[i] = acc;
            }
        }
        eacc *= eh;
        __syncthreads();   // every read of B is done
        if (more) load_b(sck + 1);
    }

    const size_t uo = (bhs * 4 + wave) * NTN * 256;
#pragma unroll
    for (int i = 0; i < NTN / 2; ++i) {   // both halves of a pair in one 16-byte store
        bf16x8 q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            q[r] = static_cast<__bf16>(uacc[i][r]);
            q[4 + r] = static_cast<__bf16>(uacc[i + NTN / 2][r]);
        }
        *reinterpret_cast<bf16x8 *>(static_cast<__bf16 *>(ws.u) + uo + rec_off<NTN>(i, lane)) = q;
    }
    if (tid == 0) ws.eda[bhs] = eacc;
    // the segment's angle total per pair (wrapped), with its cosine and sine,
    // one thread per pair: each wave's uniform angles through LDS
    float *psi = reinterpret_cast<float *>(sm.th[0]);
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < PPL; ++j) psi[wave * PW + j] = run[j];
    }
    __syncthreads();
    if (tid < NH) {
        const float tot = rot ? psi[tid] * 6.28318530717958647692f : 0.0f;   // turns -> radians
        float ts = 0.0f, tc = 1.0f;
        if (rot) sincosf(tot, &ts, &tc);
        ws.phi[bhs * NH + tid] = tot;
        ws.cph[bhs * NH + tid] = tc;
        ws.sph[bhs * NH + tid] = ts;
    }
}

// ================================================================ state pass
// RP consecutive state values (pairs) of one thread, as a vector.
template <int RP> using fvec = float __attribute__((ext_vector_type(RP)));

template <int RP>
__device__ __forceinline__ void sincosv(const fvec<RP> t, fvec<RP> &sn, fvec<RP> &cs) {
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        float s, c;
        sincosf(t[r], &s, &c);
        sn[r] = s;
        cs[r] = c;
    }
}

// v1 = element n, v2 = element n + N/2 of a pair; R(t) (v1, v2) =
// (v1 cos t - v2 sin t, v1 sin t + v2 cos t)
template <int RP>
__device__ __forceinline__ void rotate_pairs(fvec<RP> &lo, fvec<RP> &hi, const fvec<RP> cs,
                                             const fvec<RP> sn) {
    const fvec<RP> l = lo;
    lo = l * cs - hi * sn;
    hi = l * sn + hi * cs;
}

// RP consecutive values of a U / S record (element index e, a multiple of RP).
template <bool BF, int RP>
__device__ __forceinline__ fvec<RP> load_rec(const void *u, size_t e) {
    fvec<RP> v;
    if constexpr (BF) {
        typedef __bf16 bv_t __attribute__((ext_vector_type(RP)));
        const bv_t q = *reinterpret_cast<const bv_t *>(static_cast<const __bf16 *>(u) + e);
#pragma unroll
        for (int r = 0; r < RP; ++r) v[r] = static_cast<float>(q[r]);
    } else {
        v = *reinterpret_cast<const fvec<RP> *>(static_cast<const float *>(u) + e);
    }
    return v;
}
template <bool BF, int RP>
__device__ __forceinline__ void store_rec(void *u, size_t e, const fvec<RP> v) {
    if constexpr (BF) {
        typedef __bf16 bv_t __attribute__((ext_vector_type(RP)));
        bv_t q;
#pragma unroll
        for (int r = 0; r < RP; ++r) q[r] = static_cast<__bf16>(v[r]);
        *reinterpret_cast<bv_t *>(static_cast<__bf16 *>(u) + e) = q;
    } else {
        *reinterpret_cast<fvec<RP> *>(static_cast<float *>(u) + e) = v;
    }
}

// A pair's two halves, RP values each, of a record at element e (the low
// half at e, the high half four elements on: rec_off); all four pairs of a
// lane in one 16-byte access for bf16.
template <bool BF, int RP>
__device__ __forceinline__ void load_pair(const void *u, size_t e, fvec<RP> &lo, fvec<RP> &hi) {
    if constexpr (BF && RP == 4) {
        const bf16x8 q = *reinterpret_cast<const bf16x8 *>(static_cast<const __bf16 *>(u) + e);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            lo[r] = static_cast<float>(q[r]);
            hi[r] = static_cast<float>(q[4 + r]);
        }
    } else {
        lo = load_rec<BF, RP>(u, e);
        hi = load_rec<BF, RP>(u, e + 4);
    }
}
template <bool BF, int RP>
__device__ __forceinline__ void store_pair(void *u, size_t e, const fvec<RP> lo, const fvec<RP> hi) {
    if constexpr (BF && RP == 4) {
        bf16x8 q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            q[r] = static_cast<__bf16>(lo[r]);
            q[4 + r] = static_cast<__bf16>(hi[r]);
        }
        *reinterpret_cast<bf16x8 *>(static_cast<__bf16 *>(u) + e) = q;
    } else {
        store_rec<BF, RP>(u, e, lo);
        store_rec<BF, RP>(u, e + 4, hi);
    }
}

// One thread per (batch, head, p, RP state pairs): RP of the four values a
// lane holds in a record's MFMA D layout, so 4 / RP threads share a lane's
// four (more threads in flight for the same records).
template <typename T, int N, int RP>
__global__ void __launch_bounds__(kThreads)
state_pass_kernel(ScanLaunch a, ChunkWs ws, int nck) {   // nck: segments per sequence
    constexpr int P = kP;
    constexpr int NTN = N / 16;
    constexpr int HT = NTN / 2;   // n-tiles per half
    constexpr int NH = N / 2;
    constexpr int SPLIT = 4 / RP;
    constexpr bool kBf16 = sizeof(T) == 2;
    using V = fvec<RP>;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int pt = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;
    const size_t H = a.heads, L = a.seq;
    const int part = static_cast<int>(blockIdx.x % SPLIT);
    const int i1 = static_cast<int>((blockIdx.x / SPLIT) % HT);
    const size_t bh = blockIdx.x / (SPLIT * HT);
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int p = 16 * pt + c;
    const int nlo = 16 * i1 + 4 * g + RP * part;   // my pairs (nlo + r, nlo + r + N/2), r < RP
    const size_t sbase = bh * P * N + static_cast<size_t>(p) * N;

    V lo = V(0.0f), hi = V(0.0f);
    {
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        if (h0 != nullptr) {
            lo = *reinterpret_cast<const V *>(h0 + sbase + nlo);
            hi = *reinterpret_cast<const V *>(h0 + sbase + nlo + NH);
            if (l0 != nullptr) {
                // carry S = h + (1 - lambda_0) dt_0 last_u   (scan.rs:521-535)
                const size_t i0s = (bb * L) * H + hh;
                const float first = (1.0f - a.lambda[i0s]) * a.dt[i0s];
                lo += *reinterpret_cast<const V *>(l0 + sbase + nlo) * first;
                hi += *reinterpret_cast<const V *>(l0 + sbase + nlo + NH) * first;
            }
        }
    }
    // running wrapped angle of my pairs; the carried state into chunk 0's frame
    V phi = V(0.0f);
    if (rot && a.angle0 != nullptr) {
        phi = *reinterpret_cast<const V *>(a.angle0 + bh * NH + nlo);
        V cs, sn;
        sincosv<RP>(phi, sn, cs);
        rotate_pairs<RP>(lo, hi, cs, sn);
    }

    const size_t bhk0 = bh * nck;
    struct In {
        V ulo, uhi, cs, sn, ph;
        float e;
    };
    auto load = [&](int k, In &d) {
        const int kk = k < nck ? k : nck - 1;   // past the end: re-read the last chunk, unused
        const size_t bhk = bhk0 + kk;
        const size_t u = (bhk * 4 + pt) * NTN * 256 + rec_off<NTN>(i1, lane) + RP * part;
        load_pair<kBf16, RP>(ws.u, u, d.ulo, d.uhi);
        d.e = ws.eda[bhk];
        if (rot) {
            d.cs = *reinterpret_cast<const V *>(ws.cph + bhk * NH + nlo);
            d.sn = *reinterpret_cast<const V *>(ws.sph + bhk * NH + nlo);
            d.ph = *reinterpret_cast<const V *>(ws.phi + bhk * NH + nlo);
        }
    };
    auto step = [&](int k, const In &d) {
        const size_t so = ((bhk0 + k) * 4 + pt) * NTN * 256 + rec_off<NTN>(i1, lane) + RP * part;
        store_pair<kBf16, RP>(ws.s, so, lo, hi);
        lo = lo * d.e + d.ulo;
        hi = hi * d.e + d.uhi;
        if (rot) {
            rotate_pairs<RP>(lo, hi, d.cs, d.sn);
#pragma unroll
            for (int r = 0; r < RP; ++r) phi[r] = wrap_angle(phi[r] + d.ph[r]);
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
    V ce = V(1.0f), se = V(0.0f);
    if (rot) sincosv<RP>(phi, se, ce);
    if (a.h_out != nullptr) {
        V hl = lo, hh2 = hi;
        rotate_pairs<RP>(hl, hh2, ce, -se);   // R(-phi_end)
        *reinterpret_cast<V *>(a.h_out + sbase + nlo) = hl;
        *reinterpret_cast<V *>(a.h_out + sbase + nlo + NH) = hh2;
    }
    if (a.angle_out != nullptr && pt == 0 && c == 0)
        *reinterpret_cast<V *>(a.angle_out + bh * NH + nlo) = phi;
    if (a.last_u_out != nullptr) {
        // last_u = sum_r x_{L-1,r} B~_{L-1,r}^T with B~ = R(-phi_end) B  (scan.rs:599-618)
        const size_t tl = (bb * L + (L - 1)) * H + hh;
        const T *bp = static_cast<const T *>(a.b) + tl * N * a.rank;
        const T *xp = static_cast<const T *>(a.x) + (tl * P + static_cast<size_t>(p)) * a.rank;
        V ul = V(0.0f), uh = V(0.0f);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            if (m >= static_cast<int>(a.rank)) break;
            const float xv = to_f32(xp[m]);
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                const float b1 = to_f32(bp[(nlo + r) * a.rank + m]);
                const float b2 = to_f32(bp[(nlo + r + NH) * a.rank + m]);
                ul[r] += xv * (b1 * ce[r] + b2 * se[r]);
                uh[r] += xv * (-b1 * se[r] + b2 * ce[r]);
            }
        }
        *reinterpret_cast<V *>(a.last_u_out + sbase + nlo) = ul;
        *reinterpret_cast<V *>(a.last_u_out + sbase + nlo + NH) = uh;
    }
}

// ================================================================ chunk scan
template <typename T, int N, int R, int ROWS>
struct ScanSmem {
    using G = Geo<T, N, kP, R, ROWS, 4>;
    using op_t = typename Op<T>::t;
    static constexpr int PAD = 16 / static_cast<int>(sizeof(op_t));
    static constexpr int LDN = N + PAD;
    static constexpr int LDR = ROWS + PAD;
    op_t Bs[ROWS * LDN];    // B~[rho][npos(n)], segment frame
    op_t Cs[ROWS * LDN];    // C~[rho][npos(n)], segment frame
    op_t Xt[kP * LDR];      // X^T [p][rho]
    op_t Ms[ROWS * LDR];    // masked band (C B^T o L)[rho_t][rho_s]
    float acum[G::QT], gw[G::QT], ww[G::QT];
    float wdv[G::QT];       // w x decay to the sub-chunk's end, per token
    // wrapped angle per pair entering the sub-chunk, relative to the segment
    // start.  Each pair is read and rewritten by the one wave whose lanes own
    // it (the write depends on the read, and a wave's LDS accesses execute in
    // order), so one copy serves every sub-chunk.
    float psi[N / 2];
};

// One workgroup per (batch, head, segment): the segment's kseg sub-chunks of
// ROWS rows one after the other, starting from the state S the state pass
// left for the segment (in its frame).  Per sub-chunk:
//   y = (C~ B~^T o L) X + exp(acum) C~ S    (ssd_band fused.rs:2044-2070,
//       scan.rs:253-263; the skip D on the band's diagonal, scan.rs:593-597)
//   S <- e_h S + (B~ w decay-to-end)^T X    (scan.rs:207-251)
// with B~ and C~ rotated by their angle relative to the segment start, so the
// state needs no rotation between sub-chunks.  PF: the next sub-chunk's
// inputs are loaded into registers behind the current one's work.
template <typename T, int N, int R, int ROWS, bool PF>
__global__ void __launch_bounds__(kThreads, (R > 1 || PF) ? 2 : 3)
chunk_scan_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    using G = Geo<T, N, P, R, ROWS, 4>;
    using S = ScanSmem<T, N, R, ROWS>;
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
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;
    const int pcol = 16 * wave + c;

    const SeqBufs rs = seq_bufs<T, N, P, R>(a, bb, hh);
    const int h_end = min(kseg, nsub - seg * kseg);
    // The first sub-chunk's inputs go first: its stage waits for them while
    // the state fragments below are still in flight.
    RawT cur, nxt;
    load_chunk<T, N, P, R, ROWS, 4, true>(rs, seg * kseg, wave, lane, PF ? nxt : cur);

    // the state entering this segment, in its frame, as carry-in A operands
    // (bf16: n-tiles 2kb and 2kb + 1 form k-block kb, matching npos)
    using frag_t = typename std::conditional<kBf16, bf16x8, f32x4>::type;
    constexpr int NF = kBf16 ? N / 32 : NTN;
    frag_t sf[NF];
    if constexpr (kBf16) {
        const __bf16 *src = static_cast<const __bf16 *>(ws.s) + (bhs * 4 + wave) * NTN * 256;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(src + rec_off<NTN>(2 * f, lane));
            const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(src + rec_off<NTN>(2 * f + 1, lane));
            sf[f] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    } else {
        const float *src = static_cast<const float *>(ws.s) + (bhs * 4 + wave) * NTN * 256;
#pragma unroll
        for (int f = 0; f < NF; ++f) sf[f] = *reinterpret_cast<const f32x4 *>(src + rec_off<NTN>(f, lane));
    }

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    const bool skip = a.d_skip != nullptr;
    // the angle of every pair relative to the segment start is zero on entry
    if (tid < NH) sm.psi[tid] = 0.0f;
    constexpr bool kUni = G::SUBS == 1;   // pair angles wave-uniform (pair_angle)
    float run[kUni ? PPL : 1];
#pragma unroll
    for (int j = 0; j < (kUni ? PPL : 1); ++j) run[j] = 0.0f;
    // With the prefetch, the state fragments and the first sub-chunk's inputs
    // land before the loop: a wait for them inside it would also cover the
    // next sub-chunk's prefetch on every pass (vmcnt counts in issue order).
    // Without it, the first stage starts while the fragments are in flight.
    if constexpr (PF) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();

#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
    // The lane-derived indices are re-derived from an opaque copy of the lane
    // number in every sub-chunk: otherwise the compiler hoists every LDS
    // address they feed out of the loop and keeps them live across it, which
    // costs ~60 VGPRs and spills at three workgroups per CU.
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int lane = lane_v;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int sub = lane / G::SW;
    const int my_t = lane % G::SW;
    const bool tok_lane = my_t < QT;
    const int i0 = wave * G::PW + sub * PPL;
    const int pcol = 16 * wave + c;
    const int sck = seg * kseg + h;
    const bool advance = h + 1 < h_end;
    if constexpr (PF) {
        cur = nxt;
        if (advance) load_chunk<T, N, P, R, ROWS, 4, true>(rs, sck + 1, wave, lane, nxt);
    } else if (h > 0) {
        load_chunk<T, N, P, R, ROWS, 4, true>(rs, sck, wave, lane, cur);
    }
    // ---- stage: per-token scalars, angles, rotated B and C, X^T
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
            const float last = __int_as_float(
                __builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
            sm.wdv[my_t] = dexp<kBf16>(last - acum) * wv;   // w x decay to the end
        }
        if (tok_lane) {
#pragma unroll
            for (int e = 0; e < G::XE; ++e) {
                const int o = wave * (P / 4) * R + sub * G::XE + e;
                const int p = o / R, r = o % R;
                sm.Xt[p * LDR + my_t * R + r] = op_elem<T>(cur.x, e);
            }
        }
        // per group of (up to) four pairs: the angle within the segment (the
        // running angle plus the in-sub-chunk inclusive cumsum of dt * theta),
        // its sine and cosine, and B and C rotated by its negative
        // (fused.rs:610-617) and stored -- one group's values live at a time.
        // Without theta its loads read zeros: every angle is 0 (cosine 1,
        // sine 0), with no branch to keep the group's pairs from interleaving.
        const float dtt = live ? cur.s0 : 0.0f;
        constexpr int GP = PPL % 4 == 0 ? 4 : 1;
#pragma unroll
        for (int q = 0; q < PPL; q += GP) {
            float cs[GP], sn[GP], pre[GP];
#pragma unroll
            for (int jj = 0; jj < GP; ++jj) pre[jj] = dtt * welem<T>(cur.th, q + jj);
            if constexpr (GP == 4)
                seg_scan4<G::SW>(pre[0], pre[1], pre[2], pre[3]);
            else
                pre[0] = seg_scan<G::SW>(pre[0]);
#pragma unroll
            for (int jj = 0; jj < GP; ++jj) {
                const int j = q + jj;
                const float phi = pair_angle<kUni, QT>(pre[jj], run[kUni ? j : 0], &sm.psi[i0 + j],
                                                       my_t == QT - 1);
                if constexpr (kBf16) {
                    const float rev = phi * 0.15915494309189533577f;
                    sn[jj] = __builtin_amdgcn_sinf(rev);
                    cs[jj] = __builtin_amdgcn_cosf(rev);
                } else {
                    sincosf(phi, &sn[jj], &cs[jj]);
                }
            }
            if (tok_lane) {
#pragma unroll
                for (int which = 0; which < 2; ++which) {
                    const u32x4(&src)[2][G::HV] = which == 0 ? cur.b : cur.c;
                    op_t *dst = which == 0 ? sm.Bs : sm.Cs;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int rho = my_t * R + r;
                        float rv[2][GP];
#pragma unroll
                        for (int jj = 0; jj < GP; ++jj) {
                            const float v1 = elem<T>(src[0], (q + jj) * R + r);
                            const float v2 = elem<T>(src[1], (q + jj) * R + r);
                            rv[0][jj] = v1 * cs[jj] + v2 * sn[jj];
                            rv[1][jj] = -v1 * sn[jj] + v2 * cs[jj];
                        }
#pragma unroll
                        for (int hf = 0; hf < 2; ++hf) {
                            if constexpr (GP == 4)
                                st4(&dst[rho * LDN + npos<kBf16>(i0 + hf * NH + q)], rv[hf]);
                            else
                                dst[rho * LDN + npos<kBf16>(i0 + hf * NH + q)] = to_op<op_t>(rv[hf][0]);
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
        acc = acc * dexp<kBf16>(sm.acum[(16 * tj + c) / R]);   // exp_decay(acum)
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

    if (advance) {
        // ---- the state entering the next sub-chunk: S' = e_h S + U_h with
        // U_h^T[n][p] = sum_rho (B~ w decay-to-end)[rho][n] X^T[p][rho] over
        // this wave's p-tile.  This lane holds S at p = 16 wave + c,
        // n = 16 i + 4 g + r: the D layout of the U_h tiles.
        const float eh = dexp<kBf16>(sm.acum[QT - 1]);
        if constexpr (kBf16) {
            // A operand B~^T (rows n = 16 i + c, k-slot j <-> rho = 32 kb + 8 g + j)
            // by two transposed reads of the row-major B~; B operand the
            // weighted X^T slice (w decay per row, rounded to bf16 once).  One
            // fragment (two n-tiles) at a time, so few f32 tiles are live.
            constexpr int NKB = ROWS / 32;
            bf16x8 xw[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const bf16x8 xv = *reinterpret_cast<const bf16x8 *>(xr + 32 * kb + 8 * g);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    xw[kb][j] = static_cast<__bf16>(static_cast<float>(xv[j]) *
                                                    sm.wdv[(32 * kb + 8 * g + j) / R]);
            }
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                f32x4 st[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) st[q][r] = static_cast<float>(sf[f][q * 4 + r]) * eh;
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        const int row0 = 32 * kb + 8 * g + (c >> 2);
                        const __bf16 *p0 =
                            &sm.Bs[row0 * LDN + npos<true>(16 * (2 * f + q) + 4 * (c & 3))];
                        const bf16x4 lo = lds_read_tr16(p0);
                        const bf16x4 hi = lds_read_tr16(p0 + 4 * LDN);
                        const bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        st[q] = mfma_bf16(av, xw[kb], st[q]);
                    }
                }
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sf[f][q * 4 + r] = static_cast<__bf16>(st[q][r]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                f32x4 st = sf[i] * eh;
                const int n = 16 * i + c;
#pragma unroll
                for (int kb = 0; kb < ROWS / KB; ++kb) {
                    const f32x4 bv = *reinterpret_cast<const f32x4 *>(xr + 16 * kb + 4 * g);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int rho = 16 * kb + 4 * g + j;
                        st = mfma_f32(static_cast<float>(sm.Bs[rho * LDN + n]) * sm.wdv[rho / R],
                                      bv[j], st);
                    }
                }
                sf[i] = st;
            }
        }
        lds_barrier();   // the next sub-chunk's staging reuses the LDS
    }
    }   // sub-chunks
}

// The same for bf16 storage at rank 1, with B, C, theta and X staged by
// coalesced direct-to-LDS loads into raw row tiles (as chunk_state_dma_kernel
// does).  The stage rotates B and C in place; the band reads B~ and C~ rows in
// memory order (any k order serves when both operands share it); the carry-in
// takes C~ in the state fragments' k order by two 8-byte reads; X^T comes by
// transposed reads, once per sub-chunk, for the band product and the advance.
//
// The loads run one sub-chunk ahead, each into a region as soon as its last
// reader is done.  Per sub-chunk h (p = h & 1; theta(h) sits in region R[p],
// X(h) in R[1 - p]):
//   wait for B, C, theta (X may still be out); stage; band into R[p] and the
//   carry-in product C~ S (C~ is then dead): load C(h+1) and the scalars;
//   wait for X; X^T fragments and the advance (B~ and R[1 - p] are then
//   dead): load B(h+1) and theta(h+1) into R[1 - p]; y; load X(h+1) into R[p].
// Loads complete in issue order, so each wait counts the loads issued after
// the ones it needs (the y stores in between only add to the count).
template <int N>
struct ScanDmaSmem {
    static constexpr int CB = N / 8, CT = N / 16, CX = kP / 8;   // chunks per row
    static constexpr int LDM = 64 + 8;                           // band row stride
    static constexpr int RB = 64 * CX * 16 > 64 * LDM * 2 ? 64 * CX * 16 : 64 * LDM * 2;
    static_assert(64 * CT * 16 <= RB, "theta fits a region");
    unsigned char b[64 * CB * 16];    // B, then B~ [t][n]
    unsigned char c[64 * CB * 16];    // C, then C~ [t][n]
    unsigned char r[2][RB];           // theta, then the band (C B^T o L)[t][s]; X [t][p]
    float acum[64], gw[64], ww[64], wdv[64];
};

// GATE: y leaves through the mixer's gate, bf16(y) * silu(z) (the rounding
// of mixer_gate_vec_kernel).  A sub-chunk's gated y is stored during the next
// sub-chunk, once its z has landed: z's loads are ordinary (the compiler waits
// for them), so they are consumed where the only loads issued after them are
// that sub-chunk's X, which is waited for there anyway.
template <int N, bool GATE>
__global__ void __launch_bounds__(kThreads, 3)
chunk_scan_dma_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    using G = Geo<bf16_t, N, P, 1, 64, 4>;
    using S = ScanDmaSmem<N>;
    constexpr int CB = S::CB, CT = S::CT, CX = S::CX, LDM = S::LDM;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL, PW = G::PW;
    constexpr int NT = 4;             // 16-row tiles of a sub-chunk
    constexpr int NF = N / 32;        // state fragments (k-blocks of n)
    constexpr int HV = PW / 8;
    constexpr int RB = CB * 16;       // bytes per row of the B / C tiles
    static_assert(G::SUBS == 1 && QT == 64 && PPL == PW, "lane = token, one segment per wave");
    static_assert(CB % 4 == 0 && CT % 4 == 0 && CX % 4 == 0, "row loads spread over four waves");
    // loads a wave issues per sub-chunk: C with the four scalars, B with
    // theta, and X
    constexpr int kC = CB / 4 + 4, kX = CX / 4;

    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const size_t H = a.heads, L = a.seq;
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const SeqBufs rs = seq_bufs<bf16_t, N, P, 1>(a, bb, hh);
    const int h_end = min(kseg, nsub - seg * kseg);

    // the state entering this segment, in its frame, in the carry-in A
    // operand layout: n-tiles f and f + NF (a rotation pair's halves, side by
    // side in the record) form k-block f, n = 16 f + 16 NF h + 4 g + r for
    // k-slot 4 h + r.  Carried in f32 across the sub-chunks; its bf16 copy
    // is the carry-in operand.
    f32x4 sacc[NF][2];
    {
        const __bf16 *src = static_cast<const __bf16 *>(ws.s) + (bhs * 4 + wave) * (N / 16) * 256;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const bf16x8 v = *reinterpret_cast<const bf16x8 *>(src + rec_off<N / 16>(f, lane));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sacc[f][0][r] = static_cast<float>(v[r]);
                sacc[f][1][r] = static_cast<float>(v[4 + r]);
            }
        }
    }
    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    float run[PPL];   // wave-uniform running pair angles, in turns (pair_turns)
#pragma unroll
    for (int j = 0; j < PPL; ++j) run[j] = 0.0f;

    auto load_c = [&](int k, TokScalars &sc) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < CB / 4; ++q)
            lds_load_rows<CB>(rs.c, tok0 * rs.tok_bc, rs.tok_bc, sm.c, wave + 4 * q, lane);
        const uint32_t tok = tok0 + lane;
        sc.s0 = bldf(rs.s0, tok * rs.tok_s);
        sc.s1 = bldf(rs.s1, tok * rs.tok_s);
        sc.s2 = bldf(rs.s2, (tok + rs.nxt_s) * rs.tok_s);
        sc.s3 = bldf(rs.s3, (tok + rs.nxt_s) * rs.tok_s);
    };
    auto load_bt = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < CB / 4; ++q)
            lds_load_rows<CB>(rs.b, tok0 * rs.tok_bc, rs.tok_bc, sm.b, wave + 4 * q, lane);
#pragma unroll
        for (int q = 0; q < CT / 4; ++q)
            lds_load_rows<CT>(rs.th, tok0 * rs.tok_th, rs.tok_th, sm.r[k & 1], wave + 4 * q, lane);
    };
    auto load_x = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < CX / 4; ++q)
            lds_load_rows<CX>(rs.x, tok0 * rs.tok_x, rs.tok_x, sm.r[(k & 1) ^ 1], wave + 4 * q, lane);
    };

    // the gate: z of this sequence (tokens past its end read as zero), and
    // the previous sub-chunk's y (bf16) and z awaiting the gate
    const rsrc_t rz =
        GATE ? make_rsrc(static_cast<const char *>(a.gate_z) + (bb * L * a.gate_stride + hh * P) * 2,
                         static_cast<uint32_t>((L * a.gate_stride - hh * P) * 2))
             : make_rsrc(a.x, 0u);
    const uint32_t zs = GATE ? static_cast<uint32_t>(a.gate_stride * 2) : 0u;
    u32x2 ypend[NT], zpend[NT];
    uint32_t ytok0 = 0;
    bool pend = false;
    auto gate_store = [&]() {
        const int gg = lane >> 4, cc = lane & 15;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t yw = ypend[tj][r >> 1], zw = zpend[tj][r >> 1];
                const float yv = __uint_as_float((r & 1) ? (yw & 0xFFFF0000u) : (yw << 16));
                const float zv = __uint_as_float((r & 1) ? (zw & 0xFFFF0000u) : (zw << 16));
                v[r] = yv * mixm::silu_fast(zv);
            }
            u32x2 pk;
            pk[0] = pk_bf16(v[0], v[1]);
            pk[1] = pk_bf16(v[2], v[3]);
            bst8(pk, rs.y, (ytok0 + 16 * tj + cc) * rs.tok_x + (16 * wave + 4 * gg) * 2);
        }
    };

    TokScalars sc_next;
    load_c(seg * kseg, sc_next);
    load_bt(seg * kseg);
    load_x(seg * kseg);

#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int lane = lane_v;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int sck = seg * kseg + h;
    const int par = sck & 1;
    const uint32_t tok0 = static_cast<uint32_t>(sck) * QT;
    const bool more = h + 1 < h_end;
    // Tile addressing.  Rows 16 i + c of a B / C tile share the chunk
    // permutation rsw(c), and the k-chunk indices XORed with it below have
    // bits disjoint from the lane's own part, so every operand address is a
    // per-lane offset plus a constant (the LDS instruction's immediate).
    const int sw = rsw<CB>(c);
    const int crow = c * RB;

    // B, C, theta and the scalars of this sub-chunk landed (X may be out)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<kX>());
    __syncthreads();
    const TokScalars sc = sc_next;
    unsigned char *const rth = sm.r[par];         // theta, then the band
    unsigned char *const rx = sm.r[par ^ 1];      // X
    __bf16 *const ms = reinterpret_cast<__bf16 *>(rth);

    const bool live = tok0 + lane < L;
    float av, gv, wv;
    token_scalars(a, sc, A, live, av, gv, wv);
    const float acum = seg_scan<64>(av);
    if (wave == 0) {
        // the log decay prefix in log2 units, as the band and the carry-in
        // take it (dexp2)
        sm.acum[lane] = acum * kLog2e;
        sm.gw[lane] = gv;
        sm.ww[lane] = wv;
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        sm.wdv[lane] = dexp<true>(last - acum) * wv;   // w x decay to the end
    }
    // dt / 2 pi: the pair angles are carried in turns (pair_turns)
    const float dtt = live ? sc.s0 * 0.15915494309189533577f : 0.0f;

    // ---- stage: per group of four pairs the angle within the segment, its
    //      sine and cosine, and B and C rotated by its negative
    //      (fused.rs:610-617), written back in place
    {
        const int i0 = wave * PW;
        u32x4 th[HV];
#pragma unroll
        for (int v = 0; v < HV; ++v)
            th[v] = *reinterpret_cast<const u32x4 *>(rth + rtile_off<CT>(lane, i0 + 8 * v));
#pragma unroll
        for (int v = 0; v < HV; ++v) {
            u32x4 bv[2], cv[2], bo[2], co[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                bv[hf] = *reinterpret_cast<const u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v));
                cv[hf] = *reinterpret_cast<const u32x4 *>(sm.c + rtile_off<CB>(lane, hf * NH + i0 + 8 * v));
            }
#pragma unroll
            for (int q = 0; q < 8; q += 4) {
                float pre[4];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) pre[jj] = dtt * elem<bf16_t>(th, 8 * v + q + jj);
                seg_scan4<64>(pre[0], pre[1], pre[2], pre[3]);
#pragma unroll
                for (int jj = 0; jj < 4; jj += 2) {
                    float ob[2][2], oc[2][2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int e = q + jj + u;   // element within the chunk
                        const float w = pair_turns(pre[jj + u], run[8 * v + e]);
                        const float sn = __builtin_amdgcn_sinf(w);
                        const float cs = __builtin_amdgcn_cosf(w);
                        const float b1 = elem<bf16_t>(bv, e), b2 = elem<bf16_t>(bv + 1, e);
                        const float c1 = elem<bf16_t>(cv, e), c2 = elem<bf16_t>(cv + 1, e);
                        ob[0][u] = b1 * cs + b2 * sn;
                        ob[1][u] = -b1 * sn + b2 * cs;
                        oc[0][u] = c1 * cs + c2 * sn;
                        oc[1][u] = -c1 * sn + c2 * cs;
                    }
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        bo[hf][(q + jj) >> 1] = pk_bf16(ob[hf][0], ob[hf][1]);
                        co[hf][(q + jj) >> 1] = pk_bf16(oc[hf][0], oc[hf][1]);
                    }
                }
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                *reinterpret_cast<u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v)) = bo[hf];
                *reinterpret_cast<u32x4 *>(sm.c + rtile_off<CB>(lane, hf * NH + i0 + 8 * v)) = co[hf];
            }
        }
    }
    __syncthreads();   // B~, C~ complete; theta is dead, its region takes the band

    // ---- masked band into R[p]: tile (TJ, SI) of (C~ B~^T o L)[t][s],
    //      t = 16 TJ + c, s = 16 SI + 4 g + r, for SI <= TJ, and the zero
    //      tiles above the diagonal that the y product's 32-row k-blocks read
    {
        // the k-block kb of a row: chunk 4 kb + g, permuted
        const int zg = (g ^ sw) << 4;
        const int mrow = c * (LDM * 2) + 8 * g;   // this lane's band slot, bytes
        auto tile = [&](auto tj_c, auto si_c) {
            constexpr int TJ = decltype(tj_c)::value, SI = decltype(si_c)::value;
            __bf16 *const dst = reinterpret_cast<__bf16 *>(reinterpret_cast<unsigned char *>(ms) + mrow +
                                                           TJ * 16 * LDM * 2 + SI * 32);
            if constexpr (SI > TJ) {
                const float z[4] = {0.f, 0.f, 0.f, 0.f};
                st4(dst, z);
            } else {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < N / 32; ++kb) {
                    const int o = ((kb << 6) ^ zg) + crow;
                    const bf16x8 av = *reinterpret_cast<const bf16x8 *>(sm.b + SI * 16 * RB + o);
                    const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(sm.c + TJ * 16 * RB + o);
                    acc = mfma_bf16(av, bv, acc);
                }
                const float at = sm.acum[16 * TJ + c];
                const f32x4 as = *reinterpret_cast<const f32x4 *>(&sm.acum[16 * SI + 4 * g]);
                const f32x4 ws4 = *reinterpret_cast<const f32x4 *>(&sm.ww[16 * SI + 4 * g]);
                float vals[4];
                if constexpr (SI < TJ) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) vals[r] = acc[r] * ws4[r] * dexp2(at - as[r]);
                } else {
                    // the diagonal tile: s < t off-diagonal weight, s = t the
                    // diagonal weight and the skip D (scan.rs:593-597)
                    const f32x4 gs4 = *reinterpret_cast<const f32x4 *>(&sm.gw[16 * SI + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int d = 4 * g + r - c;
                        const float off = acc[r] * ws4[r] * dexp2(at - as[r]);
                        const float dia = acc[r] * gs4[r] + dskip;
                        vals[r] = d < 0 ? off : (d == 0 ? dia : 0.0f);
                    }
                }
                st4(dst, vals);
            }
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        // three or two product tiles per wave
        if (wave == 0) {
            tile(I0{}, I0{}); tile(I2{}, I0{}); tile(I3{}, I0{});
        } else if (wave == 1) {
            tile(I0{}, I1{}); tile(I2{}, I1{}); tile(I3{}, I1{});
        } else if (wave == 2) {
            tile(I1{}, I0{}); tile(I2{}, I2{}); tile(I3{}, I2{});
        } else {
            tile(I1{}, I1{}); tile(I2{}, I3{}); tile(I3{}, I3{});
        }
    }
    // ---- the carry-in product sum_n S[p][n] C~[t][n] per t-tile: k-slots
    //      4 h + 0..3 of block f are n = 16 (f + NF h) + 4 g + 0..3, i.e.
    //      chunk 2 (f + NF h) + (g >> 1) of the row, half g & 1
    bf16x8 sf[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sf[f][r] = static_cast<__bf16>(sacc[f][0][r]);
            sf[f][4 + r] = static_cast<__bf16>(sacc[f][1][r]);
        }
    f32x4 yc[NT];   // the carry-in part of y^T[p][t], scaled by exp_decay(acum_t)
    {
        const int zc = ((g >> 1) ^ sw) << 4;
        const int cbase = crow + (g & 1) * 8;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) yc[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int olo = (((2 * f) << 4) ^ zc) + cbase;
            const int ohi = (((2 * (f + NF)) << 4) ^ zc) + cbase;
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
                const bf16x4v lo = *reinterpret_cast<const bf16x4v *>(sm.c + tj * 16 * RB + olo);
                const bf16x4v hi = *reinterpret_cast<const bf16x4v *>(sm.c + tj * 16 * RB + ohi);
                const bf16x8 cv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                yc[tj] = mfma_bf16(sf[f], cv, yc[tj]);
            }
        }
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) yc[tj] = yc[tj] * dexp2(sm.acum[16 * tj + c]);
    }
    __syncthreads();   // the band is complete; C~ is dead
    if constexpr (GATE) {
        // the previous sub-chunk's gated y: its z was loaded before this
        // sub-chunk's X, which the wait below needs anyway
        if (pend) gate_store();
        pend = false;
    }
    if (more) load_c(sck + 1, sc_next);
    // X landed (the next sub-chunk's C and scalars may be out)
    if (more)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kC>());
    else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    __syncthreads();

    // ---- X^T operand fragments (p = 16 wave + c, s = 32 kb + 8 g + 0..7)
    bf16x8 xf[2];
    {
        const int r0 = 8 * g + (c >> 2);
        const int cq = 16 * wave + 4 * (c & 3);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(rx + rtile_off<CX>(32 * kb + r0, cq)));
            const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(rx + rtile_off<CX>(32 * kb + r0 + 4, cq)));
            xf[kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    }

    if (more) {
        // ---- S' = e_h S + U_h, U_h^T[n][p] = sum_s B~[s][n] (w decay X^T)[p][s]
        // over this wave's p-tile: A operand B~^T by transposed reads (row
        // 32 kb + r0 (+ 4), columns 16 (f + q NF) + 4 (c & 3) + 0..3: chunk
        // 2 (f + q NF) + ((c & 3) >> 1), half c & 1), B operand the weighted
        // X^T fragments (rounded to bf16 once)
        const float eh = dexp2(sm.acum[QT - 1]);
        bf16x8 xw[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                xw[kb][j] = static_cast<__bf16>(static_cast<float>(xf[kb][j]) * sm.wdv[32 * kb + 8 * g + j]);
        const int r0 = 8 * g + (c >> 2);
        const int zlo = (((c & 3) >> 1) ^ rsw<CB>(r0 & 15)) << 4;
        const int zhi = (((c & 3) >> 1) ^ rsw<CB>((r0 + 4) & 15)) << 4;
        const int blo = r0 * RB + (c & 1) * 8, bhi = (r0 + 4) * RB + (c & 1) * 8;
        // every fragment read first, so the LDS reads stream back to back
        bf16x8 av[NF][2][2];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int ch = (2 * (f + q * NF)) << 4;
                const int olo = (ch ^ zlo) + blo, ohi = (ch ^ zhi) + bhi;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(sm.b + 32 * kb * RB + olo));
                    const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(sm.b + 32 * kb * RB + ohi));
                    av[f][q][kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                f32x4 st = sacc[f][q] * eh;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) st = mfma_bf16(av[f][q][kb], xw[kb], st);
                sacc[f][q] = st;
            }
        __syncthreads();   // B~ and X are dead
        load_bt(sck + 1);
    }

    // ---- y^T[p][t] = exp(acum_t) sum_n S[p][n] C~[t][n] + sum_s X^T[p][s] M[t][s]
    {
        const unsigned char *const mb = reinterpret_cast<const unsigned char *>(ms) + c * (LDM * 2) + 16 * g;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            f32x4 acc = yc[tj];
            const int t = 16 * tj + c;
            const int nkb = tj < 2 ? 1 : 2;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                if (kb < nkb)
                    acc = mfma_bf16(xf[kb], *reinterpret_cast<const bf16x8 *>(mb + tj * 16 * LDM * 2 + kb * 64), acc);
            // rows past the sequence end fall outside the buffer: dropped
            const uint32_t oy = (tok0 + t) * rs.tok_x + (16 * wave + 4 * g) * 2;
            u32x2 pk;
            pk[0] = pk_bf16(acc[0], acc[1]);
            pk[1] = pk_bf16(acc[2], acc[3]);
            if constexpr (GATE) {
                ypend[tj] = pk;
                zpend[tj] = bld8(rz, (tok0 + t) * zs + (16 * wave + 4 * g) * 2);
            } else {
                bst8(pk, rs.y, oy);
            }
        }
        if constexpr (GATE) {
            ytok0 = tok0;
            pend = true;
            if (!more) {
                gate_store();
                pend = false;
            }
        }
    }
    if (more) {
        __syncthreads();   // every read of the band is done
        load_x(sck + 1);
    }
    }   // sub-chunks
}

// The single pass walks each (batch, head) sequence with one workgroup per CU,
// so its time goes in whole rounds of one sequence per CU; the three
// chunk-parallel launches cost about the same per sequence at any count.  The
// single pass is the faster form once its last round fills ~85 % of the chip
// (measured on MI355X at L = 2048, H = 12, N = 128, bf16, in us chunked vs
// single pass: 96 sequences 93.6 vs 219.8, 144: 165.4 vs 223.2, 192: 181.6
// vs 231.6, 240: 270.2 vs 235.6, 288: 302.9 vs 443.5, 384: 354.0 vs 452.3).
// The workspace is asked for only where the chunked form wins.
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

int rows_for(const ScanLaunch &a) { return a.bf16 ? 64 : 32; }

// How a sequence is cut: nsub sub-chunks of ROWS rows (ROWS / R tokens), kseg
// of them per segment, nseg segments.  The state passes between segments
// only, so U and S records and the state pass shrink with kseg, while the
// chunk_scan workgroups (one per segment) should still fill the chip once: a
// segment takes at least the caller's chunk_size tokens, and more where
// there are sub-chunks to spare beyond one resident workgroup per slot.
struct SegPlan {
    int nsub, kseg, nseg;
};

SegPlan seg_plan(const ScanLaunch &a) {
    const size_t qt = static_cast<size_t>(rows_for(a)) / a.rank;
    const size_t nsub = (a.seq + qt - 1) / qt;
    const size_t q = a.chunk_size ? a.chunk_size : 64;
    const size_t kmin = (q + qt - 1) / qt;
    // rounds of resident chunk_scan workgroups: one at rank 1, six for MIMO
    // (measured on MI355X, rotated inputs, us per call: config 1 with the
    // direct-to-LDS staging at 1 / 2 rounds 96.4-97.8 / 100.2-102.8, before it
    // at 1 / 2 / 4 rounds 123.1 / 120.0 / 132.0; config 2 at 4 / 5 / 6 / 7 /
    // 8 / 10 / 12 / 16 rounds, two passes on one box, 570-593 / 575-586 /
    // 556-574 / 573-596 / 581-590 / 596-603 / 596-615 / 594-609, against
    // 125.0 and 724.6 for one 64-token chunk per workgroup)
    const size_t slots = device_cus() * (a.rank > 1 ? 2 : 3);
    const size_t rounds = a.rank > 1 ? 6 : 1;
    // segments per sequence that fill the rounds without spilling into one
    // more, then the sub-chunks each needs
    const size_t bh = a.batch * a.heads;
    const size_t fill = bh < rounds * slots ? rounds * slots / bh : 1;
    size_t k = (nsub + fill - 1) / fill;
    if (k < kmin) k = kmin;
    if (k < 1) k = 1;
    if (k > nsub) k = nsub;
    SegPlan p;
    p.nsub = static_cast<int>(nsub);
    p.kseg = static_cast<int>(k);
    p.nseg = static_cast<int>((nsub + k - 1) / k);
    return p;
}

template <typename T, int N, int R, int ROWS>
hipError_t launch_three(const ScanLaunch &a, char *base, hipStream_t s) {
    // MIMO sub-chunks hold few tokens: their inputs are loaded behind the
    // previous one's work (bf16; f32 lacks the registers).  At rank 1 the
    // prefetch measured slower (its 52 VGPRs cost more than the loads it hides).
    constexpr bool kPf = R > 1 && sizeof(T) == 2;
    const SegPlan sp = seg_plan(a);
    const size_t bh = a.batch * a.heads;
    const size_t bhs = bh * sp.nseg;
    const ChunkWs ws = chunk_ws(base, chunked_layout(bhs, N, sizeof(T) == 2));
    if constexpr (sizeof(T) == 2 && R == 1)
        hipLaunchKernelGGL((chunk_state_dma_kernel<N>), dim3(bhs), dim3(kThreads), 0, s, a, ws,
                           sp.nsub, sp.kseg, sp.nseg);
    else
        hipLaunchKernelGGL((chunk_state_kernel<T, N, R, ROWS, kPf>), dim3(bhs),
                           dim3(kThreads), 0, s, a, ws, sp.nsub, sp.kseg, sp.nseg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((state_pass_kernel<T, N, kStatePairs>), dim3(bh * (N / 32) * (4 / kStatePairs)), dim3(kThreads), 0, s, a, ws,
                       sp.nseg);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if constexpr (sizeof(T) == 2 && R == 1) {
        if (a.gate_z != nullptr)
            hipLaunchKernelGGL((chunk_scan_dma_kernel<N, true>), dim3(bhs), dim3(kThreads), 0, s, a,
                               ws, sp.nsub, sp.kseg, sp.nseg);
        else
            hipLaunchKernelGGL((chunk_scan_dma_kernel<N, false>), dim3(bhs), dim3(kThreads), 0, s, a,
                               ws, sp.nsub, sp.kseg, sp.nseg);
    } else {
        if (a.gate_z != nullptr) return hipErrorNotSupported;   // the caller gates separately
        hipLaunchKernelGGL((chunk_scan_kernel<T, N, R, ROWS, kPf>), dim3(bhs), dim3(kThreads), 0,
                           s, a, ws, sp.nsub, sp.kseg, sp.nseg);
    }
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

}  // namespace

size_t scan_chunked_workspace(const ScanLaunch &a) {
    if (!scan_fast_supported(a) || a.seq == 0) return 0;
    const size_t seqs = a.batch * a.heads, cus = device_cus();
    const size_t rounds = (seqs + cus - 1) / cus;
    if (seqs * 100 >= rounds * cus * 85) return 0;
    return chunked_layout(seqs * seg_plan(a).nseg, a.d_state, a.bf16 != 0).total;
}

hipError_t launch_scan_chunked(const ScanLaunch &a, void *workspace, hipStream_t stream) {
    if (!scan_fast_supported(a) || a.seq == 0) return hipErrorNotSupported;
    char *ws = static_cast<char *>(workspace);
    if (a.bf16) return launch_t<bf16_t, 64>(a, ws, stream);
    return launch_t<float, 32>(a, ws, stream);
}

}  // namespace m3
