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
#include <atomic>
#include <chrono>
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

    const size_t H = a.heads, L = a.seq;
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const bool rot = a.theta != nullptr;

    const int sub = lane / G::SW;
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
                for (int hf = 0; hf < 2; ++hf) out[hf][e >> 1] = pack_bf16x2(o[hf][0], o[hf][1]);
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

    const size_t H = a.heads, L = a.seq;
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;


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
                pk[0] = pack_bf16x2(acc[0], acc[1]);
                pk[1] = pack_bf16x2(acc[2], acc[3]);
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
            pk[0] = pack_bf16x2(v[0], v[1]);
            pk[1] = pack_bf16x2(v[2], v[3]);
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
                        bo[hf][(q + jj) >> 1] = pack_bf16x2(ob[hf][0], ob[hf][1]);
                        co[hf][(q + jj) >> 1] = pack_bf16x2(oc[hf][0], oc[hf][1]);
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
            pk[0] = pack_bf16x2(acc[0], acc[1]);
            pk[1] = pack_bf16x2(acc[2], acc[3]);
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

// ================================================================ chunk scan, rank 4
// Raw token tiles of the rank-4 (MIMO) inputs.  A row is one token as it lies
// in memory: B and C rows hold [n][r], the four ranks of one state index in
// 8 bytes; X rows [p][r]; theta rows [pair].  Chunk m (16 bytes) of row t
// sits at chunk m ^ msw(t) of the row.  The operands of the products are
// read straight from this layout:
//   - band and carry-in: rows rho = (token, rank) with k = n.  In one
//     transposed read (ds_read_b64_tr_b16) lane 4 i + m of a 16-lane group
//     points at the ranks of n_i of token m; lane 4 m' + r then receives n_0
//     .. n_3 of row (token m', rank r): rows (token, rank) in rank-fastest
//     order with no rearranging of the tile;
//   - B~^T and X^T (rows n or p, k = rho): the four ranks of one n (p) of a
//     token are the four consecutive k of that token, one 8-byte read.
// msw rotates the token's four low bits, so that 16 consecutive tokens reading
// one chunk (the stage), and each 32-lane half of the transposed reads (four
// tokens, two k-groups, two chunks) and of the 8-byte reads (two tokens,
// sixteen columns), land in 16 distinct chunks of a 256-byte window.
__device__ __forceinline__ int msw(int t) { return ((t & 3) << 2) | ((t >> 2) & 3); }
template <int CH>
__device__ __forceinline__ int mt_off(int t, int chunk) {
    return t * CH * 16 + ((chunk ^ msw(t)) << 4);
}
// Rows of CH chunks (32 or 64), 1 KB per load instruction.
template <int CH>
__device__ __forceinline__ void lds_load_mrows(rsrc_t r, uint32_t first, uint32_t stride,
                                               unsigned char *tile, int I, int lane) {
    static_assert(CH == 32 || CH == 64, "rows of 512 or 1024 bytes");
    const int t = I * (64 / CH) + lane / CH;
    const int m = (lane % CH) ^ msw(t);
    lds_dma16(r, lds_addr(tile + I * 1024), first + static_cast<uint32_t>(t) * stride + m * 16);
}
// theta rows of CT chunks (8 or 4; 128 or 64 bytes), chunk m at m ^ tsw(t):
// the stage's 16 tokens reading one pair slice then fill a 256-byte window.
// Four bytes a lane, 256 bytes per load instruction.
template <int CT>
__device__ __forceinline__ int tsw(int t) {
    static_assert(CT == 8 || CT == 4, "theta rows of 128 or 64 bytes");
    return CT == 8 ? (t >> 1) & 7 : (t >> 2) & 3;
}
template <int CT>
__device__ __forceinline__ void lds_load_trows(rsrc_t r, uint32_t first, uint32_t stride,
                                               unsigned char *tile, int I, int lane) {
    constexpr int TB = CT * 16;
    const int t = I * (256 / TB) + (lane * 4) / TB;
    const int pos = ((lane * 4) % TB) >> 4;
    lds_dma4(r, lds_addr(tile + I * 256),
             first + static_cast<uint32_t>(t) * stride + ((pos ^ tsw<CT>(t)) << 4) + 4 * (lane & 3));
}
// Operand reads of the token tiles (rows of RB bytes).  Both kinds address a
// lane offset XORed with a few constants, plus an immediate:
//   - transposed: lane 4 i + m of each 16-lane group g points at n = 32 kb +
//     16 h + 4 g + i of token 4 T + m: chunk 16 kb + 8 h + 2 g + i / 2, which
//     msw(4 T + m) = 4 m + T sends to 16 kb + (tl ^ (8 h + T)) with tl =
//     (2 g + i / 2) ^ 4 m; tb = m RB + 8 (i % 2).  Eight k-slots of the
//     operand row (token 4 T + c / 4, rank c % 4): n = 32 kb + 16 (q / 4) +
//     4 g + q % 4 for slot q.
//   - 8-byte: column 16 (2 hi + f) + c of tokens 8 kb + 2 g + e (e = 0, 1;
//     kb < 2): chunk 16 hi + 8 f + c / 2, which msw(8 kb + 2 g + e) = 8 (g %
//     2) + 4 e + 2 kb + g / 2 sends to 16 hi + (pl ^ (8 f + 4 e + 2 kb)) with
//     pl = (c / 2) ^ 8 (g % 2) ^ (g / 2); pb = 2 g RB + 8 (c % 2).  Slot q of
//     the fragment is (token 8 kb + 2 g + q / 4, rank q % 4).
template <int RB>
__device__ __forceinline__ bf16x8 mimo_tr(const unsigned char *tile, int tl, int tb, int T, int kb) {
    const unsigned char *base = tile + tb + 4 * T * RB + 256 * kb;
    const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(base + ((tl ^ T) << 4)));
    const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(base + ((tl ^ (8 + T)) << 4)));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
template <int RB>
__device__ __forceinline__ bf16x8 mimo_pair(const unsigned char *tile, int pl, int pb, int kb, int hi,
                                            int f) {
    const int k0 = (8 * f) ^ (2 * kb);
    const unsigned char *base = tile + pb + 8 * kb * RB + 256 * hi;
    const bf16x4 a = *reinterpret_cast<const bf16x4 *>(base + ((pl ^ k0) << 4));
    const bf16x4 b = *reinterpret_cast<const bf16x4 *>(base + RB + ((pl ^ k0 ^ 4) << 4));
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// The per-token scalars of a 16-token sub-chunk into LDS, wave w < 4 taking
// s_w (dt, lambda, next dt, next lambda; or a, g, w): one 4-byte load by
// lanes 0..15 (a uniform branch per resource: a selected resource would go
// through scratch).  Loaded into registers instead, they would carry the
// compiler's own waits, which count only its own loads: a vmcnt(0) before
// their first use that also waits for every tile load issued after them.
__device__ __forceinline__ void lds_load_scalars16(const SeqBufs &rs, uint32_t tok0, float *dst,
                                                   int wave, int lane) {
    if (lane < 16) {
        const uint32_t d = lds_addr(dst);
        const uint32_t o0 = (tok0 + lane) * rs.tok_s, o1 = (tok0 + rs.nxt_s + lane) * rs.tok_s;
        switch (wave) {
        case 0: lds_dma4(rs.s0, d, o0); break;
        case 1: lds_dma4(rs.s1, d, o0); break;
        case 2: lds_dma4(rs.s2, d, o1); break;
        default: lds_dma4(rs.s3, d, o1); break;
        }
    }
}

template <int N>
struct ScanMimoSmem {
    static constexpr int CB = N / 2, CX = kP / 2, CT = N / 16;   // chunks per row
    static constexpr int LDM = 64 + 8;                           // band row stride
    static constexpr int RX = 16 * CX * 16;                      // an X tile
    static constexpr int RB = RX > 64 * LDM * 2 ? RX : 64 * LDM * 2;
    static_assert(16 * CT * 16 <= RB, "theta fits a region");
    unsigned char b[16 * CB * 16];    // B, then B~ [t][n][r]
    unsigned char c[16 * CB * 16];    // C, then C~ [t][n][r]
    unsigned char r[2][RB];           // theta, then the band (C~ B~^T o L)[rho][sigma]; X [t][p][r]
    float sc[4][16];                  // the next sub-chunk's per-token scalars
    float acum[16], gw[16], ww[16], wdv[16];
};

// chunk_scan_kernel for bf16 storage at rank 4: the sub-chunk's 16 tokens x
// 4 ranks are the 64 rows rho = 4 t + r of the same products, with B, C,
// theta and X staged by coalesced direct-to-LDS loads of whole token rows
// into the tiles above and pipelined one sub-chunk ahead as in
// chunk_scan_dma_kernel (the same regions, waits and barriers).  The stage
// rotates B and C in place; each lane owns a token and PPT pairs, its 16-lane
// row the row's pairs for all 16 tokens (the angle prefix runs along the row).
// The state entering the segment is carried in f32 across the sub-chunks.
template <int N>
__global__ void __launch_bounds__(kThreads, 3)
chunk_scan_mimo_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    constexpr int QT = 16;            // tokens of a sub-chunk (64 rows)
    using S = ScanMimoSmem<N>;
    constexpr int CB = S::CB, CX = S::CX, CT = S::CT, LDM = S::LDM;
    constexpr int RBB = CB * 16;      // bytes per B / C row
    constexpr int NH = N / 2;         // rotation pairs
    constexpr int PW = NH / 4;        // pairs per wave
    constexpr int PPT = PW / 4;       // pairs per lane (one per 16-lane row)
    constexpr int NT = 4;             // 16-row tiles of a sub-chunk
    constexpr int NTN = N / 16;       // n-tiles of the state
    constexpr int NKB = N / 32;       // k-blocks of n
    static_assert(PPT == 4 || PPT == 2, "two or four pairs a lane");
    // loads a wave issues per sub-chunk: B or C rows, theta, X
    constexpr int kLB = 16 * RBB / 1024 / 4, kLT = 16 * CT * 16 / 256 / 4, kLX = 16 * CX * 16 / 1024 / 4;
    static_assert(kLB >= 1 && kLT >= 1 && kLX >= 1, "loads spread over four waves");
    constexpr int kC = kLB + 1, kX = kLX;

    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const size_t H = a.heads, L = a.seq;
    const size_t bhs = blockIdx.x;
    const int seg = static_cast<int>(bhs % nseg);
    const size_t bh = bhs / nseg;
    const size_t bb = bh / H, hh = bh % H;
    const SeqBufs rs = seq_bufs<bf16_t, N, P, 4>(a, bb, hh);
    const int h_end = min(kseg, nsub - seg * kseg);

    // the state entering this segment, in its frame: S^T tiles in the D
    // layout (n = 16 i + 4 g + r, p = 16 wave + c), carried in f32
    f32x4 sacc[NTN];
    {
        const __bf16 *src = static_cast<const __bf16 *>(ws.s) + (bhs * 4 + wave) * NTN * 256;
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            const bf16x4 v = *reinterpret_cast<const bf16x4 *>(src + rec_off<NTN>(i, lane));
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[i][r] = static_cast<float>(v[r]);
        }
    }
    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    // running pair angles of this lane's row, in turns (every lane of a row
    // holds the same values)
    float run[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) run[j] = 0.0f;

    auto load_c = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kLB; ++q)
            lds_load_mrows<CB>(rs.c, tok0 * rs.tok_bc, rs.tok_bc, sm.c, wave + 4 * q, lane);
        lds_load_scalars16(rs, tok0, &sm.sc[wave][0], wave, lane);
    };
    auto load_bt = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kLB; ++q)
            lds_load_mrows<CB>(rs.b, tok0 * rs.tok_bc, rs.tok_bc, sm.b, wave + 4 * q, lane);
#pragma unroll
        for (int q = 0; q < kLT; ++q)
            lds_load_trows<CT>(rs.th, tok0 * rs.tok_th, rs.tok_th, sm.r[k & 1], wave + 4 * q, lane);
    };
    auto load_x = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kLX; ++q)
            lds_load_mrows<CX>(rs.x, tok0 * rs.tok_x, rs.tok_x, sm.r[(k & 1) ^ 1], wave + 4 * q, lane);
    };

    load_c(seg * kseg);
    load_bt(seg * kseg);
    load_x(seg * kseg);

#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int lane = lane_v;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int m = c & 3, i4 = c >> 2;   // transposed reads: lane 4 i4 + m
    // lane parts of the operand offsets (mimo_tr, mimo_pair)
    const int tl = (2 * g + (i4 >> 1)) ^ (m << 2), tb = m * RBB + ((i4 & 1) << 3);
    const int pl = (c >> 1) ^ ((g & 1) << 3) ^ (g >> 1);
    const int pbb = 2 * g * RBB + ((c & 1) << 3), pbx = 2 * g * (CX * 16) + ((c & 1) << 3);
    const int sck = seg * kseg + h;
    const int par = sck & 1;
    const uint32_t tok0 = static_cast<uint32_t>(sck) * QT;
    const bool more = h + 1 < h_end;

    // B, C, theta and the scalars of this sub-chunk landed (X may be out)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<kX>());
    __syncthreads();
    TokScalars sc;
    sc.s0 = sm.sc[0][c];
    sc.s1 = sm.sc[1][c];
    sc.s2 = sm.sc[2][c];
    sc.s3 = sm.sc[3][c];
    unsigned char *const rth = sm.r[par];         // theta, then the band
    unsigned char *const rx = sm.r[par ^ 1];      // X
    __bf16 *const ms = reinterpret_cast<__bf16 *>(rth);

    // lane c of every row holds token c
    const bool live = tok0 + c < L;
    float av, gv, wv;
    token_scalars(a, sc, A, live, av, gv, wv);
    const float acum = seg_scan<16>(av);
    if (wave == 0 && g == 0) {
        sm.acum[c] = acum * kLog2e;   // log2 units, as dexp2 takes them
        sm.gw[c] = gv;
        sm.ww[c] = wv;
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        sm.wdv[c] = dexp<true>(last - acum) * wv;   // w x decay to the end
    }
    const float dtt = live ? sc.s0 * 0.15915494309189533577f : 0.0f;

    // ---- stage: this lane's PPT pairs at its token: the angle within the
    //      segment, its sine and cosine, and B and C rotated by its negative
    //      (fused.rs:610-617), written back in place
    {
        const int i0 = wave * PW + g * PPT;
        const unsigned char *tp = rth + (c * CT * 16) + ((((2 * i0) >> 4) ^ tsw<CT>(c)) << 4) + ((2 * i0) & 15);
        float pre[PPT];
        if constexpr (PPT == 4) {
            const u32x2 tv = *reinterpret_cast<const u32x2 *>(tp);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const unsigned int w = tv[j >> 1];
                pre[j] = dtt * __uint_as_float((j & 1) ? (w & 0xFFFF0000u) : (w << 16));
            }
            seg_scan4<16>(pre[0], pre[1], pre[2], pre[3]);
        } else {
            const unsigned int w = *reinterpret_cast<const unsigned int *>(tp);
            pre[0] = seg_scan<16>(dtt * __uint_as_float(w << 16));
            pre[1] = seg_scan<16>(dtt * __uint_as_float(w & 0xFFFF0000u));
        }
        float cs[PPT], sn[PPT];
#pragma unroll
        for (int j = 0; j < PPT; ++j) {
            const float r = run[j] + pre[j];
            const float w = r - __builtin_rintf(r);
            run[j] = dpp_f<0x15F, 0xf, false>(w);   // row_newbcast:15, the row's last token
            sn[j] = __builtin_amdgcn_sinf(w);
            cs[j] = __builtin_amdgcn_cosf(w);
        }
#pragma unroll
        for (int v = 0; v < PPT / 2; ++v) {
            const int olo = mt_off<CB>(c, i0 / 2 + v), ohi = mt_off<CB>(c, i0 / 2 + v + NH / 2);
#pragma unroll
            for (int which = 0; which < 2; ++which) {
                unsigned char *tile = which == 0 ? sm.b : sm.c;
                u32x4 vv[2], out[2];
                vv[0] = *reinterpret_cast<const u32x4 *>(tile + olo);
                vv[1] = *reinterpret_cast<const u32x4 *>(tile + ohi);
                // element e: n = i0 + 2 v + (e >> 2) (pair 2 v + (e >> 2) of this lane), rank e & 3
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int j = 2 * v + (e >> 2);
                    float o[2][2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float v1 = elem<bf16_t>(vv, e + u), v2 = elem<bf16_t>(vv + 1, e + u);
                        o[0][u] = v1 * cs[j] + v2 * sn[j];
                        o[1][u] = -v1 * sn[j] + v2 * cs[j];
                    }
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) out[hf][e >> 1] = pack_bf16x2(o[hf][0], o[hf][1]);
                }
                *reinterpret_cast<u32x4 *>(tile + olo) = out[0];
                *reinterpret_cast<u32x4 *>(tile + ohi) = out[1];
            }
        }
    }
    __syncthreads();   // B~, C~ complete; theta is dead, its region takes the band

    // ---- masked band into R[p]: tile (TJ, SI) of (C~ B~^T o L)[rho][sigma],
    //      rho = 16 TJ + c (token 4 TJ + c / 4, rank c % 4), sigma = 16 SI +
    //      4 g + r (token 4 SI + g, rank r), k = n in the order n = 32 kb +
    //      16 (q / 4) + 4 g + q % 4 of k-slot q
    {
        auto tile = [&](auto tj_c, auto si_c) {
            constexpr int TJ = decltype(tj_c)::value, SI = decltype(si_c)::value;
            __bf16 *const dst = ms + (16 * TJ + c) * LDM + 16 * SI + 4 * g;
            if constexpr (SI > TJ) {
                const float z[4] = {0.f, 0.f, 0.f, 0.f};
                st4(dst, z);
            } else {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    const bf16x8 bv = mimo_tr<RBB>(sm.b, tl, tb, SI, kb);
                    const bf16x8 cv = mimo_tr<RBB>(sm.c, tl, tb, TJ, kb);
                    acc = mfma_bf16(bv, cv, acc);
                }
                const int s = 4 * SI + g, t = 4 * TJ + (c >> 2);
                const float wgt = sm.ww[s] * dexp2(sm.acum[t] - sm.acum[s]);
                float vals[4];
                if constexpr (SI < TJ) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) vals[r] = acc[r] * wgt;
                } else {
                    // the diagonal tile: s < t off-diagonal weight, s = t the
                    // diagonal weight, plus the skip D on rho = sigma
                    // (scan.rs:593-597)
                    const float gs = sm.gw[s];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float dia = acc[r] * gs + (r == (c & 3) ? dskip : 0.0f);
                        vals[r] = s < t ? acc[r] * wgt : (s == t ? dia : 0.0f);
                    }
                }
                st4(dst, vals);
            }
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
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
    // ---- the carry-in product y[rho][p] = sum_n C~[rho][n] S^T[n][p] per
    //      rho-tile: A operand C~ (rows rho), B operand the state (column p =
    //      16 wave + c), k-slot q of block kb at n = 32 kb + 16 (q / 4) + 4 g +
    //      q % 4: n-tiles 2 kb and 2 kb + 1 of the state, as the lane holds them.
    //      The D layout gives lane (c, g) rows rho = 16 tj + 4 g + r: the four
    //      ranks of token 4 tj + g at p = 16 wave + c.
    f32x4 yc[NT];
    {
        bf16x8 sf[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sf[kb][r] = static_cast<__bf16>(sacc[2 * kb][r]);
                sf[kb][4 + r] = static_cast<__bf16>(sacc[2 * kb + 1][r]);
            }
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) yc[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int tj = 0; tj < NT; ++tj)
                yc[tj] = mfma_bf16(mimo_tr<RBB>(sm.c, tl, tb, tj, kb), sf[kb], yc[tj]);
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) yc[tj] = yc[tj] * dexp2(sm.acum[4 * tj + g]);
    }
    __syncthreads();   // the band is complete; C~ is dead
    if (more) load_c(sck + 1);   // sm.sc was last read before the stage's barrier
    // X landed (the next sub-chunk's C and scalars may be out)
    if (more)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kC>());
    else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    __syncthreads();

    // ---- X^T operand fragments (p = 16 wave + c, k-slot q of block kb at
    //      rho = 32 kb + 8 g + q: token 8 kb + 2 g + q / 4, rank q % 4)
    bf16x8 xf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) xf[kb] = mimo_pair<CX * 16>(rx, pl, pbx, kb, wave >> 1, wave & 1);

    if (more) {
        // ---- S' = e_h S + U_h, U_h^T[n][p] = sum_rho B~[rho][n] (w decay X^T)[p][rho]:
        //      A operand B~^T (row n = 16 i + c, the k order of the X^T
        //      fragments), B operand the weighted X^T (rounded to bf16 once)
        const float eh = dexp2(sm.acum[QT - 1]);
        bf16x8 xw[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int q = 0; q < 8; ++q)
                xw[kb][q] = static_cast<__bf16>(static_cast<float>(xf[kb][q]) *
                                                sm.wdv[8 * kb + 2 * g + (q >> 2)]);
        // every fragment read first, so the LDS reads stream back to back
        bf16x8 bt[NTN][2];
#pragma unroll
        for (int i = 0; i < NTN; ++i)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) bt[i][kb] = mimo_pair<RBB>(sm.b, pl, pbb, kb, i >> 1, i & 1);
#pragma unroll
        for (int i = 0; i < NTN; ++i) {
            f32x4 st = sacc[i] * eh;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) st = mfma_bf16(bt[i][kb], xw[kb], st);
            sacc[i] = st;
        }
        __syncthreads();   // B~ and X are dead
        load_bt(sck + 1);
    }

    // ---- y[rho][p] = exp(acum_t) sum_n C~[rho][n] S^T[n][p] + sum_sigma M[rho][sigma] X[sigma][p]:
    //      A operand the band row rho = 16 tj + c, B operand the X^T fragment
    //      (column p).  Lane (c, g) holds the four ranks of token 4 tj + g at
    //      p = 16 wave + c, which lie together in memory: one 8-byte store a
    //      lane, 128 contiguous bytes per token.  Tokens past the sequence end
    //      fall outside the buffer: dropped.
    {
        const unsigned char *const mb = reinterpret_cast<const unsigned char *>(ms) + c * (LDM * 2) + 16 * g;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            f32x4 acc = yc[tj];
            const int nkb = tj < 2 ? 1 : 2;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                if (kb < nkb)
                    acc = mfma_bf16(*reinterpret_cast<const bf16x8 *>(mb + tj * 16 * LDM * 2 + kb * 64), xf[kb], acc);
            u32x2 pk;
            pk[0] = pack_bf16x2(acc[0], acc[1]);
            pk[1] = pack_bf16x2(acc[2], acc[3]);
            bst8(pk, rs.y, (tok0 + 4 * tj + g) * rs.tok_x + (16 * wave + c) * 8);
        }
    }
    if (more) {
        __syncthreads();   // every read of the band is done
        load_x(sck + 1);
    }
    }   // sub-chunks
}

// chunk_state_kernel for bf16 storage at rank 4, on the token tiles of
// chunk_scan_mimo_kernel: theta, X and the per-token scalars of the next
// sub-chunk are fetched at the start of the current one (theta and X
// double-buffered), B once the previous product has read it.  The stage
// forms the angles from theta while B arrives, then rotates B (fused.rs:
// 610-617) and weights it by w x decay-to-end in place; U's operands are
// 8-byte reads of the tiles, (B~ w)^T rows n and X^T rows p, k = rho.
template <int N>
struct StateMimoSmem {
    static constexpr int CB = N / 2, CX = kP / 2, CT = N / 16;   // chunks per row
    unsigned char b[16 * CB * 16];        // B, then B~ w decay-to-end [t][n][r]
    unsigned char th[2][16 * CT * 16];    // theta [t][pair]; the pair angle totals at the end
    unsigned char x[2][16 * CX * 16];     // X [t][p][r]
    float sc[2][4][16];                   // per-token scalars (lds_load_scalars16)
};

template <int N>
__global__ void __launch_bounds__(kThreads, 3)
chunk_state_mimo_kernel(ScanLaunch a, ChunkWs ws, int nsub, int kseg, int nseg) {
    constexpr int P = kP;
    constexpr int QT = 16;
    using S = StateMimoSmem<N>;
    constexpr int CB = S::CB, CX = S::CX, CT = S::CT;
    constexpr int RBB = CB * 16;
    constexpr int NH = N / 2, PW = NH / 4, PPT = PW / 4;
    constexpr int NTN = N / 16;
    static_assert(PPT == 4 || PPT == 2, "two or four pairs a lane");
    constexpr int kLB = 16 * RBB / 1024 / 4, kLT = 16 * CT * 16 / 256 / 4, kLX = 16 * CX * 16 / 1024 / 4;
    // loads a wave issues per sub-chunk: theta + X + one scalar, and B
    constexpr int kTX = kLT + kLX + 1, kB = kLB;

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
    const SeqBufs rs = seq_bufs<bf16_t, N, P, 4>(a, bb, hh);

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);   // a_log.exp().neg() (scan.rs:470-474)

    auto load_tx = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
        const int buf = k & 1;
#pragma unroll
        for (int q = 0; q < kLT; ++q)
            lds_load_trows<CT>(rs.th, tok0 * rs.tok_th, rs.tok_th, sm.th[buf], wave + 4 * q, lane);
#pragma unroll
        for (int q = 0; q < kLX; ++q)
            lds_load_mrows<CX>(rs.x, tok0 * rs.tok_x, rs.tok_x, sm.x[buf], wave + 4 * q, lane);
        lds_load_scalars16(rs, tok0, &sm.sc[buf][wave][0], wave, lane);
    };
    auto load_b = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kLB; ++q)
            lds_load_mrows<CB>(rs.b, tok0 * rs.tok_bc, rs.tok_bc, sm.b, wave + 4 * q, lane);
    };

    f32x4 uacc[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) uacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float eacc = 1.0f;
    float run[PPT];   // running pair angles of this lane's row, in turns
#pragma unroll
    for (int j = 0; j < PPT; ++j) run[j] = 0.0f;

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
        // lane parts of the 8-byte operand offsets (mimo_pair)
        const int pl = (c >> 1) ^ ((g & 1) << 3) ^ (g >> 1);
        const int pbb = 2 * g * RBB + ((c & 1) << 3), pbx = 2 * g * (CX * 16) + ((c & 1) << 3);

        // theta, X, scalars of this sub-chunk landed (only its B may be out)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kB>());
        __syncthreads();
        TokScalars sc;
        sc.s0 = sm.sc[buf][0][c];
        sc.s1 = sm.sc[buf][1][c];
        sc.s2 = sm.sc[buf][2][c];
        sc.s3 = sm.sc[buf][3][c];
        if (more) load_tx(sck + 1);

        const bool live = static_cast<size_t>(sck) * QT + c < L;
        float av, gv, wv;
        token_scalars(a, sc, A, live, av, gv, wv);
        const float acum = seg_scan<16>(av);
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        const float wd = dexp<true>(last - acum) * wv;   // exp_decay(last, acum, w)
        const float eh = dexp<true>(last);
        const float dtt = live ? sc.s0 * 0.15915494309189533577f : 0.0f;

        // ---- stage, first half: this lane's pair angles at its token and their
        //      sines and cosines (theta only; B is still arriving)
        const int i0 = wave * PW + g * PPT;
        float cs[PPT], sn[PPT];
        {
            const unsigned char *tp = sm.th[buf] + (c * CT * 16) +
                                      ((((2 * i0) >> 4) ^ tsw<CT>(c)) << 4) + ((2 * i0) & 15);
            float pre[PPT];
            if constexpr (PPT == 4) {
                const u32x2 tv = *reinterpret_cast<const u32x2 *>(tp);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const unsigned int w = tv[j >> 1];
                    pre[j] = dtt * __uint_as_float((j & 1) ? (w & 0xFFFF0000u) : (w << 16));
                }
                seg_scan4<16>(pre[0], pre[1], pre[2], pre[3]);
            } else {
                const unsigned int w = *reinterpret_cast<const unsigned int *>(tp);
                pre[0] = seg_scan<16>(dtt * __uint_as_float(w << 16));
                pre[1] = seg_scan<16>(dtt * __uint_as_float(w & 0xFFFF0000u));
            }
#pragma unroll
            for (int j = 0; j < PPT; ++j) {
                const float r = run[j] + pre[j];
                const float w = r - __builtin_rintf(r);
                run[j] = dpp_f<0x15F, 0xf, false>(w);   // row_newbcast:15, the row's last token
                sn[j] = __builtin_amdgcn_sinf(w);
                cs[j] = __builtin_amdgcn_cosf(w);
            }
        }
        // B landed (the next sub-chunk's theta, X and scalars may be out)
        if (more)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<kTX>());
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
        __syncthreads();

        // ---- stage, second half: B rotated by the negative angle and weighted,
        //      back in place (element e of a chunk: n = i0 + 2 v + e / 4, rank e % 4)
#pragma unroll
        for (int v = 0; v < PPT / 2; ++v) {
            const int olo = mt_off<CB>(c, i0 / 2 + v), ohi = mt_off<CB>(c, i0 / 2 + v + NH / 2);
            u32x4 vv[2], out[2];
            vv[0] = *reinterpret_cast<const u32x4 *>(sm.b + olo);
            vv[1] = *reinterpret_cast<const u32x4 *>(sm.b + ohi);
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int j = 2 * v + (e >> 2);
                float o[2][2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float b1 = elem<bf16_t>(vv, e + u), b2 = elem<bf16_t>(vv + 1, e + u);
                    o[0][u] = (b1 * cs[j] + b2 * sn[j]) * wd;
                    o[1][u] = (-b1 * sn[j] + b2 * cs[j]) * wd;
                }
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) out[hf][e >> 1] = pack_bf16x2(o[hf][0], o[hf][1]);
            }
            *reinterpret_cast<u32x4 *>(sm.b + olo) = out[0];
            *reinterpret_cast<u32x4 *>(sm.b + ohi) = out[1];
        }
        __syncthreads();

        // ---- U = e_h U + U_h, U_h^T[n][p] = sum_rho (B~w)[rho][n] X[rho][p]
        //      over p-tile = wave: A operand row n = 16 i + c, B operand column
        //      p = 16 wave + c, k-slot q of block kb at rho = 32 kb + 8 g + q
        {
            bf16x8 xo[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) xo[kb] = mimo_pair<CX * 16>(sm.x[buf], pl, pbx, kb, wave >> 1, wave & 1);
            bf16x8 bt[NTN][2];
#pragma unroll
            for (int i = 0; i < NTN; ++i)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) bt[i][kb] = mimo_pair<RBB>(sm.b, pl, pbb, kb, i >> 1, i & 1);
#pragma unroll
            for (int i = 0; i < NTN; ++i) {
                f32x4 acc = uacc[i] * eh;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) acc = mfma_bf16(bt[i][kb], xo[kb], acc);
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
    // one thread per pair: each row's angles through LDS (theta is dead: the
    // loop's last barrier followed every read, and no load is in flight)
    float *psi = reinterpret_cast<float *>(sm.th[0]);
    if ((lane & 15) == 0) {
        const int i0 = wave * PW + (lane >> 4) * PPT;
#pragma unroll
        for (int j = 0; j < PPT; ++j) psi[i0 + j] = run[j];
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

// ================================================================ fused single launch
// The whole scan in one launch that reads its inputs once.  One workgroup per
// segment of at most two sub-chunks (KS rows of 64 tokens), in three steps:
//   1. local pass: chunk_scan's stage, band, carry-in and advance over the
//      segment's sub-chunks starting from a zero state, in the segment's own
//      frame.  This yields y_local (kept in registers), C~ of every sub-chunk
//      (kept in LDS) and the segment's contribution U (the local state at its
//      end), decay e and angle total Phi (scan.rs:207-251 over the segment).
//   2. the state entering the segment, S_j, by a decoupled look-back: the
//      workgroup publishes (U, e, Phi) as its aggregate, then walks back
//      over the segments before it to the nearest one that has published
//      its inclusive state and applies S_{m+1} = R(Phi_m) (e_m S_m + U_m)
//      forward from there.  Every step is the same f32 arithmetic on the same
//      values whichever segment performs it, so S_j does not depend on the
//      order in which workgroups ran.  It publishes S_{j+1}.
//   3. y = y_local + decay(t) C~_t . S_j for every token (the carry-in of the
//      entering state, scan.rs:253-263), stored once; the last segment writes
//      the boundary state (scan.rs:270-288, 599-638).
// So B, C, x, theta, dt and lambda are read from HBM once and B and C are
// rotated once; the records of a segment are 16 KB of U (bf16), 32 KB of the
// inclusive state (f32) and a few hundred bytes of scalars.
//
// Records move through device-coherent (sc1) buffer loads and stores; a
// record is written, the writer waits for its stores (vmcnt(0)), the
// workgroup synchronises, and then one thread stores the segment's flag
// (epoch << 2 | state, a relaxed device-scope atomic).  A reader polls the
// flag and reads the record after it.  Every wait is bounded (lb_spin polls
// with a sleep between them); a workgroup that gives up takes S_j = NaN, so
// its outputs and every later segment of the sequence come out NaN, never
// stale.  Workgroups are numbered segment-major, so a segment's predecessor
// was dispatched before it on the same XCD; the bound covers any other order.
constexpr uint64_t kFlagAgg = 1, kFlagInc = 2;
constexpr int kCoh = 16;   // buffer cache policy sc1: coherent across the device

struct FusedWs {
    unsigned long long *flag;   // [segments] epoch << 2 | state
    __bf16 *u;                  // [segments][wave][n-tile][lane][4]: U in the rec_off layout
    float *eda;                 // [segments] decay of the segment
    float *phi, *cph, *sph;     // [segments][N/2] angle total (wrapped), cos, sin
    float *inc;                 // [segments][wave][f][half][lane][4]: S after the segment (f32)
    float *incphi;              // [segments][N/2] angle after the segment, from the sequence start
    size_t u_bytes, inc_bytes;
};

struct FusedLayout {
    size_t flag, u, eda, phi, cph, sph, inc, incphi, total;
};

FusedLayout fused_layout(size_t segs, size_t n) {
    FusedLayout l;
    size_t o = 0;
    l.flag = o;
    o = align256(o + segs * 8);
    l.u = o;
    o = align256(o + segs * kP * n * 2);
    l.eda = o;
    o = align256(o + segs * 4);
    l.phi = o;
    o = align256(o + segs * (n / 2) * 4);
    l.cph = o;
    o = align256(o + segs * (n / 2) * 4);
    l.sph = o;
    o = align256(o + segs * (n / 2) * 4);
    l.inc = o;
    o = align256(o + segs * kP * n * 4);
    l.incphi = o;
    o = align256(o + segs * (n / 2) * 4);
    l.total = o;
    return l;
}

FusedWs fused_ws(char *base, const FusedLayout &l, size_t segs, size_t n) {
    FusedWs w;
    w.flag = reinterpret_cast<unsigned long long *>(base + l.flag);
    w.u = reinterpret_cast<__bf16 *>(base + l.u);
    w.eda = reinterpret_cast<float *>(base + l.eda);
    w.phi = reinterpret_cast<float *>(base + l.phi);
    w.cph = reinterpret_cast<float *>(base + l.cph);
    w.sph = reinterpret_cast<float *>(base + l.sph);
    w.inc = reinterpret_cast<float *>(base + l.inc);
    w.incphi = reinterpret_cast<float *>(base + l.incphi);
    w.u_bytes = segs * kP * n * 2;
    w.inc_bytes = segs * kP * n * 4;
    return w;
}

// One step of the state chain for a lane's four pairs (lo: n, hi: n + N/2):
// S' = R(phi) (e S + U), R(phi) (v1, v2) = (v1 cos - v2 sin, v1 sin + v2 cos),
// with explicit fused multiply-adds so that every caller rounds alike.
__device__ __forceinline__ void chain_step(f32x4 &lo, f32x4 &hi, float e, const f32x4 &ulo,
                                           const f32x4 &uhi, const f32x4 &cs, const f32x4 &sn) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float l = __builtin_fmaf(lo[r], e, ulo[r]);
        const float h = __builtin_fmaf(hi[r], e, uhi[r]);
        lo[r] = __builtin_fmaf(l, cs[r], -(h * sn[r]));
        hi[r] = __builtin_fmaf(l, sn[r], h * cs[r]);
    }
}

__device__ __forceinline__ f32x4 cld16f(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoh));
}
__device__ __forceinline__ void cst16f(rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCoh);
}

template <int N>
struct FusedSmem {
    static constexpr int CB = N / 8, CT = N / 16, CX = kP / 8;   // chunks a row
    static constexpr int LDM = 64 + 8;                           // band row stride
    unsigned char b[64 * CB * 16];       // B, then B~ [t][n]
    unsigned char c[2][64 * CB * 16];    // C, then C~ [t][n], of each sub-chunk (kept)
    unsigned char th[64 * CT * 16];      // theta [t][pair]
    unsigned char x[64 * CX * 16];       // X [t][p]
    __bf16 band[64 * LDM];               // (C~ B~^T o L)[t][s]
    float sc[2][4][64];                  // dt, lambda, next dt, next lambda
    float acum[2][64];                   // decay prefix (log2 units) of each sub-chunk
    float gw[64], ww[64], wdv[64];
    float ang[N / 2];                    // the segment's angle total per pair (turns, then radians)
    float cph[N / 2], sph[N / 2];        // its cosine and sine
    float phc[N / 2];                    // the angle entering / leaving the segment from the sequence start
    int lb[2];                           // look-back: nearest inclusive segment, gave up
};

// The part of the fused launch after its local pass: the segment's
// aggregate, the look-back for the state entering it, its inclusive state,
// y with the entering state's part, and the boundary state: KS sub-chunks of
// QT tokens (NT 16-row tiles) per segment, C~ of each in sm.c[h] (rows of RB bytes, the rsw<RB/16>
// permutation), the decay prefix of each in sm.acum[h], y_local in ykeep;
// sm.ang holds the segment's angle total per pair in turns.
template <int N, int KS, int QT, bool GATE, typename Sm>
__device__ __forceinline__ void fused_tail(const ScanLaunch &a, const FusedWs &ws, Sm &sm,
                                           f32x4 (&sacc)[N / 32][2], f32x4 (&ykeep)[KS][QT / 16],
                                           const float (&eprod)[KS], float eacc, int k0, int h_end,
                                           int seg, int nseg, size_t bh, size_t bhs, const SeqBufs &rs,
                                           uint64_t epoch, int lb_mode, int lb_spin) {
    constexpr int P = kP;
    constexpr int NH = N / 2;
    constexpr int NT = QT / 16;
    constexpr int NF = N / 32;
    constexpr int NTN = N / 16;
    constexpr int CB = N / 8;
    constexpr int RB = CB * 16;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t H = a.heads, L = a.seq;
    const size_t bb = bh / H, hh = bh % H;
    // ---- the segment's aggregate: U (rounded to bf16, the record's values),
    //      its decay, and per pair its wrapped angle total with cos and sin
    const int lg = lane >> 4, lc = lane & 15;
    const size_t urec = (bhs * 4 + wave) * NTN * 256;
    const rsrc_t ru = make_rsrc(ws.u, static_cast<uint32_t>(ws.u_bytes));
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        bf16x8 q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            q[r] = static_cast<__bf16>(sacc[f][0][r]);
            q[4 + r] = static_cast<__bf16>(sacc[f][1][r]);
        }
        if (seg > 0)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, q), ru,
                                                   static_cast<uint32_t>((urec + rec_off<NTN>(f, lane)) * 2), 0, kCoh);
    }
    __syncthreads();   // sm.ang holds every pair's angle total in turns
    if (tid < NH) {
        const float tot = a.theta != nullptr ? sm.ang[tid] * 6.28318530717958647692f : 0.0f;
        float ts = 0.0f, tc = 1.0f;
        if (a.theta != nullptr) sincosf(tot, &ts, &tc);
        sm.ang[tid] = tot;
        sm.cph[tid] = tc;
        sm.sph[tid] = ts;
        if (seg > 0) {
            __hip_atomic_store(&ws.phi[bhs * NH + tid], tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws.cph[bhs * NH + tid], tc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws.sph[bhs * NH + tid], ts, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (seg > 0 && tid == 0)
        __hip_atomic_store(&ws.eda[bhs], eacc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());   // the record's stores are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (seg > 0 && tid == 0)
        __hip_atomic_store(&ws.flag[bhs], (epoch << 2) | kFlagAgg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- the state entering the segment, S_j (in its frame), and the angle
    //      entering it from the sequence start
    f32x4 slo[NF], shi[NF];
    const size_t seq0 = bh * nseg;   // record index of segment 0 of this sequence
    const rsrc_t rinc = make_rsrc(ws.inc, static_cast<uint32_t>(ws.inc_bytes));
    auto inc_off = [&](size_t rec, int f, int q) {
        return static_cast<uint32_t>(((((rec * 4 + wave) * NF + f) * 2 + q) * 64 + lane) * 16);
    };
    const int p = 16 * wave + lc;
    if (seg == 0) {
        // S_0 = R(angle0) (h0 + (1 - lambda_0) dt_0 last_u0)   (scan.rs:521-535)
        const float *h0 = a.mode_raw ? a.h0 : a.init_state;
        const float *l0 = a.mode_raw ? a.last_u0 : nullptr;
        float first = 0.0f;
        if (h0 != nullptr && l0 != nullptr) {
            const size_t i0s = (bb * L) * H + hh;
            first = (1.0f - a.lambda[i0s]) * a.dt[i0s];
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int nlo = 16 * f + 4 * lg;
            f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
            if (h0 != nullptr) {
                const size_t sb = (bh * P + p) * N;
                lo = *reinterpret_cast<const f32x4 *>(h0 + sb + nlo);
                hi = *reinterpret_cast<const f32x4 *>(h0 + sb + nlo + NH);
                if (l0 != nullptr) {
                    lo += *reinterpret_cast<const f32x4 *>(l0 + sb + nlo) * first;
                    hi += *reinterpret_cast<const f32x4 *>(l0 + sb + nlo + NH) * first;
                }
            }
            if (a.theta != nullptr && a.angle0 != nullptr) {
                const f32x4 ph = *reinterpret_cast<const f32x4 *>(a.angle0 + bh * NH + nlo);
                f32x4 cs, sn;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float s1, c1;
                    sincosf(ph[r], &s1, &c1);
                    sn[r] = s1;
                    cs[r] = c1;
                }
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                chain_step(lo, hi, 1.0f, z, z, cs, sn);
            }
            slo[f] = lo;
            shi[f] = hi;
        }
        if (tid < NH)
            sm.phc[tid] = (a.theta != nullptr && a.angle0 != nullptr) ? a.angle0[bh * NH + tid] : 0.0f;
        __syncthreads();
    } else {
        if (wave == 0) {
            // the look-back, all at once: lane l reads the flag of segment
            // seg - 1 - l; the walk ends at the nearest segment with an
            // inclusive state once every segment after it has published its
            // aggregate (the first segment of a sequence publishes an
            // inclusive state, and a segment's inclusive state never waits
            // for a later one, so the condition is eventually met)
            int kinc = -1;
            int gave = lb_mode != 0 ? 1 : 0;
            const int back = min(seg, 64);
            int n = 0;
            while (!gave) {
                unsigned long long v = 0;
                if (lane < back)
                    v = __hip_atomic_load(&ws.flag[seq0 + seg - 1 - lane], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                const bool cur = lane < back && (v >> 2) == epoch;
                const uint64_t inc = __ballot(cur && (v & 3) == kFlagInc);
                const uint64_t ready = __ballot(cur && (v & 3) != 0);
                if (inc != 0) {
                    const int l = __builtin_ctzll(inc);   // nearest inclusive state
                    const uint64_t need = (l == 63) ? ~0ull : ((2ull << l) - 1);
                    if ((ready & need) == need) {
                        kinc = seg - 1 - l;
                        break;
                    }
                }
                if (++n > lb_spin) {
                    gave = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (lane == 0) {
                sm.lb[0] = kinc;
                sm.lb[1] = gave;
            }
        }
        __syncthreads();
        const int kinc = sm.lb[0];
        const bool gave = sm.lb[1] != 0;
        if (gave) {
            const float qnan = __builtin_nanf("");
#pragma unroll
            for (int f = 0; f < NF; ++f) slo[f] = shi[f] = f32x4{qnan, qnan, qnan, qnan};
            if (tid < NH) sm.phc[tid] = qnan;
        } else {
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                slo[f] = cld16f(rinc, inc_off(seq0 + kinc, f, 0));
                shi[f] = cld16f(rinc, inc_off(seq0 + kinc, f, 1));
            }
            float phc = 0.0f;
            if (tid < NH)
                phc = __hip_atomic_load(&ws.incphi[(seq0 + kinc) * NH + tid], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
            // fold forward through the aggregates of segments kinc + 1 .. seg
            // - 1, two at a time: their scalars through LDS (the band region,
            // dead by now), every load of a pair of steps issued before its use
            float *fsc = reinterpret_cast<float *>(sm.band);   // [2][e | phi, cos, sin x NH]
            constexpr int FS = 1 + 3 * NH;
            for (int m0 = kinc + 1; m0 < seg; m0 += 2) {
                const int nm = min(2, seg - m0);
                __syncthreads();   // the previous pair's scalars are read
                for (int i = tid; i < nm * FS; i += kThreads) {
                    const int st = i / FS, w = i % FS;
                    const size_t rec = seq0 + m0 + st;
                    float v;
                    if (w == 0)
                        v = __hip_atomic_load(&ws.eda[rec], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else if (w <= NH)
                        v = __hip_atomic_load(&ws.phi[rec * NH + (w - 1)], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                    else if (w <= 2 * NH)
                        v = __hip_atomic_load(&ws.cph[rec * NH + (w - 1 - NH)], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                    else
                        v = __hip_atomic_load(&ws.sph[rec * NH + (w - 1 - 2 * NH)], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                    fsc[i] = v;
                }
                bf16x8 uq[2][NF];
#pragma unroll
                for (int st = 0; st < 2; ++st)
                    if (st < nm) {
                        const size_t rec = seq0 + m0 + st;
#pragma unroll
                        for (int f = 0; f < NF; ++f) {
                            const uint32_t uo =
                                static_cast<uint32_t>(((rec * 4 + wave) * NTN * 256 + rec_off<NTN>(f, lane)) * 2);
                            uq[st][f] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ru, uo, 0, kCoh));
                        }
                    }
                __syncthreads();   // the pair's scalars are in LDS
#pragma unroll
                for (int st = 0; st < 2; ++st)
                    if (st < nm) {
                        const float *sc = fsc + st * FS;
#pragma unroll
                        for (int f = 0; f < NF; ++f) {
                            f32x4 ul, uh, cs, sn;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                ul[r] = static_cast<float>(uq[st][f][r]);
                                uh[r] = static_cast<float>(uq[st][f][4 + r]);
                                cs[r] = sc[1 + NH + 16 * f + 4 * lg + r];
                                sn[r] = sc[1 + 2 * NH + 16 * f + 4 * lg + r];
                            }
                            chain_step(slo[f], shi[f], sc[0], ul, uh, cs, sn);
                        }
                        if (tid < NH) phc = wrap_angle(phc + sc[1 + tid]);
                    }
            }
            if (tid < NH) sm.phc[tid] = phc;
        }
        __syncthreads();
    }

    // ---- publish the state after the segment: S_{j+1} = R(Phi_j) (e_j S_j + U_j),
    //      U rounded to bf16 as its record holds it; after the last segment
    //      the boundary state (scan.rs:270-288, 599-638)
    float phe = 0.0f;   // the angle after the segment (pair tid)
    if (tid < NH) {
        phe = wrap_angle(sm.phc[tid] + sm.ang[tid]);
        __hip_atomic_store(&ws.incphi[bhs * NH + tid], phe, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool last_seg = seg == nseg - 1;
    if (last_seg) {
        __syncthreads();   // every pair's angle entering the segment is read
        if (tid < NH) sm.phc[tid] = phe;
        __syncthreads();
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        f32x4 olo = slo[f], ohi = shi[f], ul, uh, cs, sn;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ul[r] = static_cast<float>(static_cast<__bf16>(sacc[f][0][r]));
            uh[r] = static_cast<float>(static_cast<__bf16>(sacc[f][1][r]));
            cs[r] = sm.cph[16 * f + 4 * lg + r];
            sn[r] = sm.sph[16 * f + 4 * lg + r];
        }
        chain_step(olo, ohi, eacc, ul, uh, cs, sn);
        cst16f(rinc, inc_off(bhs, f, 0), olo);
        cst16f(rinc, inc_off(bhs, f, 1), ohi);
        if (last_seg) {
            const size_t sb = (bh * P + p) * N;
            const int nlo = 16 * f + 4 * lg;
            f32x4 ce, se;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (a.theta != nullptr) {
                    float s1, c1;
                    sincosf(sm.phc[nlo + r], &s1, &c1);
                    se[r] = s1;
                    ce[r] = c1;
                } else {
                    se[r] = 0.0f;
                    ce[r] = 1.0f;
                }
            }
            if (a.h_out != nullptr) {
                f32x4 hl, hh2;   // R(-phi_end) S
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    hl[r] = __builtin_fmaf(olo[r], ce[r], ohi[r] * se[r]);
                    hh2[r] = __builtin_fmaf(ohi[r], ce[r], -(olo[r] * se[r]));
                }
                *reinterpret_cast<f32x4 *>(a.h_out + sb + nlo) = hl;
                *reinterpret_cast<f32x4 *>(a.h_out + sb + nlo + NH) = hh2;
            }
            if (a.last_u_out != nullptr) {
                // last_u = x_{L-1} B~_{L-1}^T with B~ = R(-phi_end) B  (scan.rs:599-618)
                const size_t tl = (bb * L + (L - 1)) * H + hh;
                const bf16_t *bp = static_cast<const bf16_t *>(a.b) + tl * N;
                const float xv = to_f32(static_cast<const bf16_t *>(a.x)[tl * P + p]);
                f32x4 ulu, uhu;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float b1 = to_f32(bp[nlo + r]);
                    const float b2 = to_f32(bp[nlo + r + NH]);
                    ulu[r] = xv * (b1 * ce[r] + b2 * se[r]);
                    uhu[r] = xv * (-b1 * se[r] + b2 * ce[r]);
                }
                *reinterpret_cast<f32x4 *>(a.last_u_out + sb + nlo) = ulu;
                *reinterpret_cast<f32x4 *>(a.last_u_out + sb + nlo + NH) = uhu;
            }
        }
    }
    if (last_seg && a.angle_out != nullptr && tid < NH) a.angle_out[bh * NH + tid] = phe;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0)
        __hip_atomic_store(&ws.flag[bhs], (epoch << 2) | kFlagInc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- y = y_local + decay(t) C~_t . S_j, stored (or gated) once
    {
        const int g = lg, c = lc;
        const int sw = rsw<CB>(c);
        const int crow = c * RB;
        bf16x8 sf[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sf[f][r] = static_cast<__bf16>(slo[f][r]);
                sf[f][4 + r] = static_cast<__bf16>(shi[f][r]);
            }
        const int zc = ((g >> 1) ^ sw) << 4;
        const int cbase = crow + (g & 1) * 8;
        const rsrc_t rz =
            GATE ? make_rsrc(static_cast<const char *>(a.gate_z) + (bb * L * a.gate_stride + hh * P) * 2,
                             static_cast<uint32_t>((L * a.gate_stride - hh * P) * 2))
                 : make_rsrc(a.x, 0u);
        const uint32_t zs = GATE ? static_cast<uint32_t>(a.gate_stride * 2) : 0u;
#pragma unroll
        for (int h = 0; h < KS; ++h) {
            if (h >= h_end) break;
            const unsigned char *const cth = sm.c[h];
            const uint32_t tok0 = static_cast<uint32_t>(k0 + h) * QT;
            f32x4 yc[NT];
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) yc[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const int olo2 = (((2 * f) << 4) ^ zc) + cbase;
                const int ohi2 = (((2 * (f + NF)) << 4) ^ zc) + cbase;
#pragma unroll
                for (int tj = 0; tj < NT; ++tj) {
                    typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
                    const bf16x4v lo = *reinterpret_cast<const bf16x4v *>(cth + tj * 16 * RB + olo2);
                    const bf16x4v hi = *reinterpret_cast<const bf16x4v *>(cth + tj * 16 * RB + ohi2);
                    const bf16x8 cv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    yc[tj] = mfma_bf16(sf[f], cv, yc[tj]);
                }
            }
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                const int t = 16 * tj + c;
                const f32x4 yl = ykeep[h][tj];
                const float dec = dexp2(sm.acum[h][t]) * eprod[h];
                f32x4 yv;
#pragma unroll
                for (int r = 0; r < 4; ++r) yv[r] = __builtin_fmaf(yc[tj][r], dec, yl[r]);
                const uint32_t oy = (tok0 + t) * rs.tok_x + (16 * wave + 4 * g) * 2;
                u32x2 pk;
                pk[0] = pack_bf16x2(yv[0], yv[1]);
                pk[1] = pack_bf16x2(yv[2], yv[3]);
                if constexpr (GATE) {
                    // the gate: bf16(y) * silu(z)   (the rounding of mixer_gate_vec_kernel)
                    const u32x2 zw = bld8(rz, (tok0 + t) * zs + (16 * wave + 4 * g) * 2);
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t yw = pk[r >> 1], zz = zw[r >> 1];
                        const float y1 = __uint_as_float((r & 1) ? (yw & 0xFFFF0000u) : (yw << 16));
                        const float z1 = __uint_as_float((r & 1) ? (zz & 0xFFFF0000u) : (zz << 16));
                        v[r] = y1 * mixm::silu_fast(z1);
                    }
                    pk[0] = pack_bf16x2(v[0], v[1]);
                    pk[1] = pack_bf16x2(v[2], v[3]);
                }
                bst8(pk, rs.y, oy);
            }
        }
    }

}

template <int N, bool GATE>
__global__ void __launch_bounds__(kThreads, 2)
chunk_scan_fused_kernel(ScanLaunch a, FusedWs ws, int nsub, int kseg, int nseg, uint64_t epoch,
                        int lb_mode, int lb_spin) {
    constexpr int P = kP;
    using G = Geo<bf16_t, N, P, 1, 64, 4>;
    using S = FusedSmem<N>;
    constexpr int CB = S::CB, CT = S::CT, CX = S::CX, LDM = S::LDM;
    constexpr int QT = G::QT, NH = G::NH, PPL = G::PPL, PW = G::PW;
    constexpr int NT = 4;             // 16-row tiles of a sub-chunk
    constexpr int NF = N / 32;        // state k-blocks (a pair's halves side by side)
    constexpr int HV = PW / 8;
    constexpr int RB = CB * 16;       // bytes a row of the B / C tiles
    static_assert(G::SUBS == 1 && QT == 64 && PPL == PW, "lane = token, one segment a wave");
    static_assert(CB % 4 == 0 && CT % 4 == 0 && CX % 4 == 0, "row loads spread over four waves");
    // load instructions a wave issues: a B or C tile, theta, X, one scalar
    constexpr int kBC = CB / 4, kT = CT / 4, kX = CX / 4;

    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const size_t H = a.heads, L = a.seq;
    // segment-major numbering: workgroup seg * (B H) + bh
    const size_t nbh = a.batch * a.heads;
    const int seg = static_cast<int>(blockIdx.x / nbh);
    const size_t bh = blockIdx.x % nbh;
    const size_t bhs = bh * nseg + seg;             // record index
    const size_t bb = bh / H, hh = bh % H;
    const SeqBufs rs = seq_bufs<bf16_t, N, P, 1>(a, bb, hh);
    const int k0 = seg * kseg;
    const int h_end = min(kseg, nsub - k0);
    const bool two = h_end > 1;

    float A = 0.0f;
    if (a.mode_raw) A = 0.0f - expf(a.a_log[hh]);
    const float dskip = a.d_skip ? a.d_skip[hh] : 0.0f;
    float run[PPL];   // wave-uniform running pair angles, in turns (pair_turns)
#pragma unroll
    for (int j = 0; j < PPL; ++j) run[j] = 0.0f;

    auto load_c = [&](int k, int slot) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kBC; ++q)
            lds_load_rows<CB>(rs.c, tok0 * rs.tok_bc, rs.tok_bc, sm.c[slot], wave + 4 * q, lane);
    };
    auto load_b = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kBC; ++q)
            lds_load_rows<CB>(rs.b, tok0 * rs.tok_bc, rs.tok_bc, sm.b, wave + 4 * q, lane);
    };
    auto load_t = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kT; ++q)
            lds_load_rows<CT>(rs.th, tok0 * rs.tok_th, rs.tok_th, sm.th, wave + 4 * q, lane);
    };
    auto load_x = [&](int k) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
#pragma unroll
        for (int q = 0; q < kX; ++q)
            lds_load_rows<CX>(rs.x, tok0 * rs.tok_x, rs.tok_x, sm.x, wave + 4 * q, lane);
    };
    // scalar `wave` of every token of sub-chunk k: s0, s1 at the token, s2, s3 at the next
    auto load_s = [&](int k, int slot) {
        const uint32_t tok0 = static_cast<uint32_t>(k) * QT;
        const uint32_t dst = lds_addr(&sm.sc[slot][wave][0]);
        const uint32_t o0 = (tok0 + lane) * rs.tok_s, o1 = (tok0 + rs.nxt_s + lane) * rs.tok_s;
        switch (wave) {   // a uniform branch per resource
        case 0: lds_dma4(rs.s0, dst, o0); break;
        case 1: lds_dma4(rs.s1, dst, o0); break;
        case 2: lds_dma4(rs.s2, dst, o1); break;
        default: lds_dma4(rs.s3, dst, o1); break;
        }
    };

    // local state (from zero) in the carry-in operand layout: sacc[f][q] is
    // n-tile f + q NF, n = 16 (f + q NF) + 4 g + r, p = 16 wave + c
    f32x4 sacc[NF][2];
#pragma unroll
    for (int f = 0; f < NF; ++f) sacc[f][0] = sacc[f][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 ykeep[2][NT];               // y of each sub-chunk before the entering state's part
    float eprod[2] = {1.0f, 1.0f};    // decay from the segment start to each sub-chunk's start
    float eacc = 1.0f;

    // prologue: C, scalars, B, theta, X of the first sub-chunk; C and the scalars of the second
    load_c(k0, 0);
    load_s(k0, 0);
    load_b(k0);
    load_t(k0);
    load_x(k0);
    if (two) {
        load_c(k0 + 1, 1);
        load_s(k0 + 1, 1);
    }

    // ---- the local pass over the segment's sub-chunks
#pragma unroll 1
    for (int h = 0; h < h_end; ++h) {
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int lane = lane_v;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int sck = k0 + h;
    const uint32_t tok0 = static_cast<uint32_t>(sck) * QT;
    const bool more = h + 1 < h_end;
    const int sw = rsw<CB>(c);
    const int crow = c * RB;
    unsigned char *const cth = sm.c[h];

    // C, the scalars, B and theta of this sub-chunk landed (X and later ones may be out)
    if (h == 0) {
        if (two)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<kX + kBC + 1>());
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_imm<kX>());
    } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kX>());
    }
    __syncthreads();

    TokScalars sc;
    sc.s0 = sm.sc[h][0][lane];
    sc.s1 = sm.sc[h][1][lane];
    sc.s2 = sm.sc[h][2][lane];
    sc.s3 = sm.sc[h][3][lane];
    const bool live = tok0 + lane < L;
    float av, gv, wv;
    token_scalars(a, sc, A, live, av, gv, wv);
    const float acum = seg_scan<64>(av);
    if (wave == 0) {
        sm.acum[h][lane] = acum * kLog2e;
        sm.gw[lane] = gv;
        sm.ww[lane] = wv;
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), QT - 1));
        sm.wdv[lane] = dexp<true>(last - acum) * wv;
    }
    const float dtt = live ? sc.s0 * 0.15915494309189533577f : 0.0f;

    // ---- stage: the angle within the segment, B and C rotated by its negative
    {
        const int i0 = wave * PW;
        u32x4 th[HV];
#pragma unroll
        for (int v = 0; v < HV; ++v)
            th[v] = *reinterpret_cast<const u32x4 *>(sm.th + rtile_off<CT>(lane, i0 + 8 * v));
#pragma unroll
        for (int v = 0; v < HV; ++v) {
            u32x4 bv[2], cv[2], bo[2], co[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                bv[hf] = *reinterpret_cast<const u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v));
                cv[hf] = *reinterpret_cast<const u32x4 *>(cth + rtile_off<CB>(lane, hf * NH + i0 + 8 * v));
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
                        const int e = q + jj + u;
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
                        bo[hf][(q + jj) >> 1] = pack_bf16x2(ob[hf][0], ob[hf][1]);
                        co[hf][(q + jj) >> 1] = pack_bf16x2(oc[hf][0], oc[hf][1]);
                    }
                }
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                *reinterpret_cast<u32x4 *>(sm.b + rtile_off<CB>(lane, hf * NH + i0 + 8 * v)) = bo[hf];
                *reinterpret_cast<u32x4 *>(cth + rtile_off<CB>(lane, hf * NH + i0 + 8 * v)) = co[hf];
            }
        }
    }
    __syncthreads();   // B~, C~ complete; theta is dead
    if (more) load_t(sck + 1);

    // ---- masked band (C~ B~^T o L)[t][s], D on the diagonal (scan.rs:593-597)
    {
        const int zg = (g ^ sw) << 4;
        const int mrow = c * (LDM * 2) + 8 * g;
        const float *acs = sm.acum[h];
        auto tile = [&](auto tj_c, auto si_c) {
            constexpr int TJ = decltype(tj_c)::value, SI = decltype(si_c)::value;
            __bf16 *const dst = reinterpret_cast<__bf16 *>(reinterpret_cast<unsigned char *>(sm.band) +
                                                           mrow + TJ * 16 * LDM * 2 + SI * 32);
            if constexpr (SI > TJ) {
                const float z[4] = {0.f, 0.f, 0.f, 0.f};
                st4(dst, z);
            } else {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < N / 32; ++kb) {
                    const int o = ((kb << 6) ^ zg) + crow;
                    const bf16x8 av8 = *reinterpret_cast<const bf16x8 *>(sm.b + SI * 16 * RB + o);
                    const bf16x8 bv8 = *reinterpret_cast<const bf16x8 *>(cth + TJ * 16 * RB + o);
                    acc = mfma_bf16(av8, bv8, acc);
                }
                const float at = acs[16 * TJ + c];
                const f32x4 as = *reinterpret_cast<const f32x4 *>(&acs[16 * SI + 4 * g]);
                const f32x4 ws4 = *reinterpret_cast<const f32x4 *>(&sm.ww[16 * SI + 4 * g]);
                float vals[4];
                if constexpr (SI < TJ) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) vals[r] = acc[r] * ws4[r] * dexp2(at - as[r]);
                } else {
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
    // ---- carry-in of the local state (zero in the first sub-chunk)
    f32x4 yc[NT];
#pragma unroll
    for (int tj = 0; tj < NT; ++tj) yc[tj] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (h > 0) {
        bf16x8 sf[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sf[f][r] = static_cast<__bf16>(sacc[f][0][r]);
                sf[f][4 + r] = static_cast<__bf16>(sacc[f][1][r]);
            }
        const int zc = ((g >> 1) ^ sw) << 4;
        const int cbase = crow + (g & 1) * 8;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int olo = (((2 * f) << 4) ^ zc) + cbase;
            const int ohi = (((2 * (f + NF)) << 4) ^ zc) + cbase;
#pragma unroll
            for (int tj = 0; tj < NT; ++tj) {
                typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
                const bf16x4v lo = *reinterpret_cast<const bf16x4v *>(cth + tj * 16 * RB + olo);
                const bf16x4v hi = *reinterpret_cast<const bf16x4v *>(cth + tj * 16 * RB + ohi);
                const bf16x8 cv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                yc[tj] = mfma_bf16(sf[f], cv, yc[tj]);
            }
        }
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) yc[tj] = yc[tj] * dexp2(sm.acum[h][16 * tj + c]);
    }
    // X landed (theta of the next sub-chunk may be out)
    if (more)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<kT>());
    else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    __syncthreads();   // the band is complete

    // ---- X^T operand fragments (p = 16 wave + c, s = 32 kb + 8 g + 0..7)
    bf16x8 xf[2];
    {
        const int r0 = 8 * g + (c >> 2);
        const int cq = 16 * wave + 4 * (c & 3);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(sm.x + rtile_off<CX>(32 * kb + r0, cq)));
            const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(sm.x + rtile_off<CX>(32 * kb + r0 + 4, cq)));
            xf[kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    }
    // ---- advance: S <- e_h S + U_h (as chunk_scan_dma_kernel)
    {
        const float eh = dexp2(sm.acum[h][QT - 1]);
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
        bf16x8 afr[NF][2][2];
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
                    afr[f][q][kb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                f32x4 st = sacc[f][q] * eh;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) st = mfma_bf16(afr[f][q][kb], xw[kb], st);
                sacc[f][q] = st;
            }
        if (h == 0) eprod[1] = eh;
        eacc *= eh;
    }
    __syncthreads();   // B~ is dead
    if (more) load_b(sck + 1);

    // ---- y_local^T[p][t] = carry-in + sum_s X^T[p][s] M[t][s], kept
    {
        const unsigned char *const mb = reinterpret_cast<const unsigned char *>(sm.band) + c * (LDM * 2) + 16 * g;
#pragma unroll
        for (int tj = 0; tj < NT; ++tj) {
            f32x4 acc = yc[tj];
            const int nkb = tj < 2 ? 1 : 2;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                if (kb < nkb)
                    acc = mfma_bf16(xf[kb], *reinterpret_cast<const bf16x8 *>(mb + tj * 16 * LDM * 2 + kb * 64), acc);
            if (h == 0)
                ykeep[0][tj] = acc;
            else
                ykeep[1][tj] = acc;
        }
    }
    if (more) {
        __syncthreads();   // every read of the band and X is done
        load_x(sck + 1);
    }
    }   // sub-chunks

    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < PPL; ++j) sm.ang[wave * PW + j] = run[j];
    }
    fused_tail<N, 2, 64, GATE>(a, ws, sm, sacc, ykeep, eprod, eacc, k0, h_end, seg, nseg, bh, bhs, rs,
                               epoch, lb_mode, lb_spin);
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
    // The bf16 rank-4 kernels (direct-to-LDS token tiles, three chunk_scan
    // workgroups per CU) take one round too: at config 2, in us per call,
    // segments of 128 / 192 / 256 / 384 / 512 tokens (4 / 2.75 / 2 / 1.4 / 1
    // rounds) measured 445 / 472 / 431 / 485 / 415.
    const bool mimo4 = a.bf16 && a.rank == 4;
    const size_t slots = device_cus() * (a.rank > 1 && !mimo4 ? 2 : 3);
    const size_t rounds = a.rank > 1 && !mimo4 ? 6 : 1;
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
    else if constexpr (sizeof(T) == 2 && R == 4)
        hipLaunchKernelGGL((chunk_state_mimo_kernel<N>), dim3(bhs), dim3(kThreads), 0, s, a, ws,
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
    } else if constexpr (sizeof(T) == 2 && R == 4) {
        if (a.gate_z != nullptr) return hipErrorNotSupported;   // the caller gates separately
        hipLaunchKernelGGL((chunk_scan_mimo_kernel<N>), dim3(bhs), dim3(kThreads), 0, s, a, ws,
                           sp.nsub, sp.kseg, sp.nseg);
    } else {
        if (a.gate_z != nullptr) return hipErrorNotSupported;   // the caller gates separately
        hipLaunchKernelGGL((chunk_scan_kernel<T, N, R, ROWS, kPf>), dim3(bhs), dim3(kThreads), 0,
                           s, a, ws, sp.nsub, sp.kseg, sp.nseg);
    }
    return hipGetLastError();
}

// Segments of the fused launch: two sub-chunks each (the C~ of both stay in
// LDS for the entering state's part of y).
struct FusedPlan {
    int nsub, kseg, nseg;
};
FusedPlan fused_plan(const ScanLaunch &a) {
    FusedPlan p;
    p.nsub = static_cast<int>((a.seq + 63) / 64);
    p.kseg = p.nsub > 1 ? 2 : 1;
    p.nseg = (p.nsub + p.kseg - 1) / p.kseg;
    return p;
}

// The fused single launch covers bf16 storage at rank 1 (d_state 64 or 128)
// and is taken while its grid fits three rounds of two workgroups per CU.
// Each round ends in a look-back, while the three launches' cost grows with
// the sequences alone; measured on MI355X (us per call, fused vs three
// launches): config 1, 96 sequences of 2048 tokens (3 rounds), 81.5 vs 83.3
// summed over the kernels; the config-4 prefill's 192 sequences (6 rounds),
// 17.22 vs 16.94 ms per 24-layer prefill.
bool fused_covered(const ScanLaunch &a) {
    if (!(a.bf16 && a.rank == 1 && (a.d_state == 64 || a.d_state == 128) && a.path == 0)) return false;
    const size_t segs = a.batch * a.heads * static_cast<size_t>(fused_plan(a).nseg);
    return segs <= 3 * 2 * device_cus();
}

// Each call gets a fresh epoch, so flags left in a reused workspace by an
// earlier call never read as published (62 bits, seeded from the clock).
std::atomic<uint64_t> g_epoch{0};
uint64_t next_epoch() {
    uint64_t e = g_epoch.fetch_add(1, std::memory_order_relaxed);
    if (e == 0) {
        const uint64_t seed = static_cast<uint64_t>(
                                  std::chrono::steady_clock::now().time_since_epoch().count()) |
                              1u;
        uint64_t expected = 1;
        g_epoch.compare_exchange_strong(expected, (seed & ((uint64_t(1) << 61) - 1)) + 2);
        e = g_epoch.fetch_add(1, std::memory_order_relaxed);
    }
    return e & ((uint64_t(1) << 62) - 1);
}

template <int N>
hipError_t launch_fused(const ScanLaunch &a, char *base, hipStream_t s) {
    const FusedPlan fp = fused_plan(a);
    const size_t bh = a.batch * a.heads;
    const size_t segs = bh * fp.nseg;
    const FusedWs ws = fused_ws(base, fused_layout(segs, N), segs, N);
    const uint64_t epoch = next_epoch();
    // polls of one flag before a look-back gives up (each poll sleeps ~128
    // cycles and waits a memory round trip: about a second in all)
    const int spin = a.lb_spin > 0 ? a.lb_spin : (1 << 20);
    const dim3 grid(static_cast<unsigned int>(segs));
    if (a.gate_z != nullptr)
        hipLaunchKernelGGL((chunk_scan_fused_kernel<N, true>), grid, dim3(kThreads), 0, s, a, ws,
                           fp.nsub, fp.kseg, fp.nseg, epoch, a.lb_mode, spin);
    else
        hipLaunchKernelGGL((chunk_scan_fused_kernel<N, false>), grid, dim3(kThreads), 0, s, a, ws,
                           fp.nsub, fp.kseg, fp.nseg, epoch, a.lb_mode, spin);
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
    if (fused_covered(a)) return fused_layout(seqs * fused_plan(a).nseg, a.d_state).total;
    return chunked_layout(seqs * seg_plan(a).nseg, a.d_state, a.bf16 != 0).total;
}

int scan_chunked_launches(const ScanLaunch &a) { return fused_covered(a) ? 1 : 3; }

hipError_t launch_scan_chunked(const ScanLaunch &a, void *workspace, hipStream_t stream) {
    if (!scan_fast_supported(a) || a.seq == 0) return hipErrorNotSupported;
    char *ws = static_cast<char *>(workspace);
    if (fused_covered(a)) {
        if (a.d_state == 128) return launch_fused<128>(a, ws, stream);
        return launch_fused<64>(a, ws, stream);
    }
    if (a.bf16) return launch_t<bf16_t, 64>(a, ws, stream);
    return launch_t<float, 32>(a, ws, stream);
}

}  // namespace m3
