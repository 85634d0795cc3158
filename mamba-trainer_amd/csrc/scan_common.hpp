// Building blocks shared by the specialised scan kernels (ssd_scan_fast.hip,
// ssd_scan_split.hip): operand types, the lane = token geometry, element
// access into loaded vectors, the column order of B~/C~ rows, the decay
// exponential and the per-sequence buffer resources.
#pragma once

#include "m3_device.hpp"
#include "m3_internal.hpp"

namespace m3 {
namespace scan {

constexpr int kThreads = 256;

__device__ __forceinline__ void lds_barrier() {
    // waits for LDS traffic only: prefetched buffer loads stay in flight
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

// Geometry of one instantiation with NW waves.  A chunk holds ROWS rows; a
// row is a (token, rank) pair rho = t*R + r (the MIMO fold of
// scan.rs:537-589).  In the staging mapping lane = token: wave w owns the
// rotation pairs [w*PW, (w+1)*PW) and head_dim columns [w*P/NW, (w+1)*P/NW).
template <typename T, int N, int P, int R, int ROWS, int NW = 4>
struct Geo {
    static constexpr int SZ = static_cast<int>(sizeof(T));
    static constexpr int E = 16 / SZ;              // elements per 16 bytes
    static constexpr int QT = ROWS / R;            // tokens per chunk
    static constexpr int NH = N / 2;               // rotation pairs
    static constexpr int SW = QT > 16 ? QT : 16;   // lanes of one token segment
    static constexpr int SUBS = 64 / SW;           // segments per wave
    static constexpr int PW = NH / NW;             // pairs per wave
    static constexpr int PPL = PW / SUBS;          // pairs per lane
    static constexpr int HE = PPL * R;             // elements of a lane's half-row slice
    static constexpr int HV = HE / E;              // ... in 16-byte vectors
    static constexpr int THB = PPL * SZ;           // theta bytes per lane
    static constexpr int TW = THB / 4;
    static constexpr int XE = (P / NW) * R / SUBS; // x elements per lane
    static constexpr int XV = XE * SZ / 16;
    static_assert(SUBS * SW == 64 && PPL * SUBS == PW && PPL >= 1, "pair slices");
    static_assert(HV * E == HE && HV >= 1, "half-row slices are whole vectors");
    static_assert(TW * 4 == THB && TW >= 1, "theta slices are whole words");
    static_assert(XV * 16 == XE * SZ && XV >= 1, "x slices are whole vectors");
    static_assert(P == 64, "head_dim 64: sixteen-column MFMA tiles, one or two waves each");
};

template <typename T> __device__ __forceinline__ float elem(const u32x4 *v, int i);
template <> __device__ __forceinline__ float elem<bf16_t>(const u32x4 *v, int i) {
    const unsigned int w = v[i >> 3][(i >> 1) & 3];
    return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}
template <> __device__ __forceinline__ float elem<float>(const u32x4 *v, int i) {
    return __uint_as_float(v[i >> 2][i & 3]);
}
template <typename T> __device__ __forceinline__ float welem(const unsigned int *w, int i);
template <> __device__ __forceinline__ float welem<bf16_t>(const unsigned int *w, int i) {
    const unsigned int u = w[i >> 1];
    return __uint_as_float((i & 1) ? (u & 0xFFFF0000u) : (u << 16));
}
template <> __device__ __forceinline__ float welem<float>(const unsigned int *w, int i) {
    return __uint_as_float(w[i]);
}

// Element i of loaded vectors in the operand type, without arithmetic (a
// bf16 element is its 16 raw bits, not a round trip through f32).
template <typename T> __device__ __forceinline__ typename Op<T>::t op_elem(const u32x4 *v, int i);
template <> __device__ __forceinline__ __bf16 op_elem<bf16_t>(const u32x4 *v, int i) {
    const unsigned int w = v[i >> 3][(i >> 1) & 3];
    return __builtin_bit_cast(__bf16, static_cast<unsigned short>((i & 1) ? (w >> 16) : w));
}
template <> __device__ __forceinline__ float op_elem<float>(const u32x4 *v, int i) {
    return __uint_as_float(v[i >> 2][i & 3]);
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

// Element (row, col) of an unpadded row-major operand tile of COLS columns
// whose 16-byte groups are permuted per row by f(row) = (row & 7) ^
// ((row >> 3) & 1).  An MFMA operand read takes one 16-byte group from each
// of sixteen consecutive rows; f sends every eight of them to distinct groups
// of a 128-byte window and all sixteen to distinct groups of a 256-byte one,
// so the read is conflict-free with 32 or 64 banks, at no padding.  A row
// written by the 64 lanes of a wave stays one contiguous row.
template <typename O, int COLS>
__device__ __forceinline__ int swz(int row, int col) {
    constexpr int E = 16 / static_cast<int>(sizeof(O));
    static_assert(COLS % (8 * E) == 0, "rows of whole 128-byte windows");
    return row * COLS + (col ^ (((row & 7) ^ ((row >> 3) & 1)) * E));
}

// exp(clamp(d, -60, 0)), the scan's decay with its log floor (scan.rs:57,
// fused.rs:2064).  bf16 storage takes the hardware exp2; f32 keeps expf.
template <bool FAST>
__device__ __forceinline__ float dexp(float d) {
    d = fminf(fmaxf(d, -60.0f), 0.0f);
    if constexpr (FAST) return __builtin_amdgcn_exp2f(d * 1.44269504088896341f);
    return expf(d);
}

// dexp for a log decay given in log2 units (d * log2 e): the clamp is one
// median-of-three and the exponential the hardware exp2.
constexpr float kLog2e = 1.44269504088896341f;
__device__ __forceinline__ float dexp2(float d2) {
    return __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(d2, -60.0f * kLog2e, 0.0f));
}

// The wrapped angle of one rotation pair at this lane's token, relative to
// the segment start: the running angle entering the sub-chunk plus the
// in-sub-chunk inclusive prefix `pre`.  The sub-chunk's last token (lane
// QT - 1 of its token segment) carries it to the next sub-chunk.  With one
// token segment per wave (UNI) every lane of the wave owns the same pair, so
// the running angle is a wave-uniform value `run` (a scalar register, by a
// readlane); otherwise it lives in LDS at `slot`, read and rewritten by the
// one wave whose lanes own the pair (a wave's LDS accesses execute in order).
template <bool UNI, int QT>
__device__ __forceinline__ float pair_angle(float pre, float &run, float *slot, bool last_lane) {
    if constexpr (UNI) {
        const float phi = wrap_angle(run + pre);
        run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(phi), QT - 1));
        return phi;
    } else {
        const float phi = wrap_angle(*slot + pre);
        if (last_lane) *slot = phi;
        return phi;
    }
}

// pair_angle in turns (revolutions, what the hardware sine takes): `pre` is
// the in-sub-chunk prefix of dt theta / 2 pi, the result the wrapped angle
// in [-1/2, 1/2] (r - rint(r) is exact), and the wave-uniform running angle
// is carried by a readlane of the last token's lane.
__device__ __forceinline__ float pair_turns(float pre, float &run) {
    const float r = run + pre;
    const float w = r - __builtin_rintf(r);
    run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 63));
    return w;
}

// s_waitcnt immediate for vmcnt(V) alone (expcnt and lgkmcnt at their
// maxima), gfx9 encoding: vmcnt bits [3:0] and [15:14].
template <int V>
constexpr int vmcnt_imm() {
    static_assert(V >= 0 && V < 64, "vmcnt range");
    return (V & 15) | ((V >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// ---- raw row tiles staged by direct-to-LDS buffer loads (gfx950)
// A tile holds 64 rows (tokens) of CH 16-byte chunks as they lie in memory,
// except that chunk m of row t sits at chunk m ^ rsw<CH>(t) of the row.  The
// permutation keeps two kinds of reads free of bank conflicts: a wave's
// lane = token reads of one chunk from 64 consecutive rows (each 16
// consecutive rows land in 16 distinct 16-byte slots of a 256-byte window),
// and transposed operand reads, whose 16 lanes take two adjacent chunks from
// each of four consecutive rows (8 distinct slots).
template <int CH>
__device__ __forceinline__ int rsw(int t) {
    static_assert(CH == 4 || CH == 8 || CH == 16, "rows of 64, 128 or 256 bytes");
    const int u = t & 15;
    if constexpr (CH == 16) return ((u & 3) << 1) | ((u >> 2) & 1) | (u & 8);
    if constexpr (CH == 8) return (((u >> 1) & 3) << 1) | ((u >> 3) & 1);
    return (u >> 2) & 3;
}
// Byte offset of element `col` (16-bit elements) of row t in such a tile.
template <int CH>
__device__ __forceinline__ int rtile_off(int t, int col) {
    return t * CH * 16 + ((((col >> 3) ^ rsw<CH>(t))) << 4) + ((col & 7) << 1);
}
// Direct-to-LDS buffer loads, issued as inline asm.  Lane l of one
// instruction writes its 4 or 16 bytes to LDS at base + l * size (M0 holds
// the base; it is saved and restored around the load).  The compiler's wait
// insertion treats an outstanding LDS DMA it knows of as a write to all of
// LDS and waits for it (vmcnt(0)) before any later LDS read, which would
// serialise a pipelined stage; these loads are unknown to it, so every read
// of their destination must follow an explicit vmcnt wait (and a barrier
// for other waves' loads).  Its own waits stay correct: loads it does not
// see only make a counted wait stricter.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    typedef __attribute__((address_space(3))) const unsigned char lds_u8;
    return __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8 *)(p))));
}
__device__ __forceinline__ void lds_dma16(rsrc_t r, uint32_t base, uint32_t voff) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "buffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "s"(base), "v"(voff), "s"(r)
                 : "memory");
}
__device__ __forceinline__ void lds_dma4(rsrc_t r, uint32_t base, uint32_t voff) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "buffer_load_dword %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "s"(base), "v"(voff), "s"(r)
                 : "memory");
}

// One such load (16 bytes a lane) of rows [I * 64 / CH, (I + 1) * 64 / CH)
// of a tile at `tile`: lane l fills slot l of the instruction's kilobyte,
// i.e. chunk l % CH of row I * 64 / CH + l / CH, with the memory chunk that
// the permutation places there.  Row t is read from byte t * stride + first
// of the buffer; rows past its range read zeros.
template <int CH>
__device__ __forceinline__ void lds_load_rows(rsrc_t r, uint32_t first, uint32_t stride,
                                              unsigned char *tile, int I, int lane) {
    const int t = I * (64 / CH) + lane / CH;
    const int m = (lane % CH) ^ rsw<CH>(t);
    lds_dma16(r, lds_addr(tile + I * 1024), first + static_cast<uint32_t>(t) * stride + m * 16);
}

// Transposed LDS read (ds_read_b64_tr_b16, gfx950).  Within each group of 16
// lanes, lane l supplies the address of four consecutive 16-bit values W[l];
// lane j receives {W[j/4][j%4], W[4 + j/4][j%4], W[8 + j/4][j%4],
// W[12 + j/4][j%4]}: column j of the 4 x 16 block whose row r is
// W[4r] .. W[4r + 3].  So with lane 4r + q pointing at row r, columns
// 4q .. 4q + 3 of a row-major [k][col] array, lane j gets k = 0..3 of column j:
// an MFMA operand whose k runs down the rows.
__device__ __forceinline__ bf16x4 lds_read_tr16(const __bf16 *p) {
    typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p));
}

// Store four consecutive operand values.
__device__ __forceinline__ void st4(__bf16 *dst, const float *v) {
    typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
    bf16x4v p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = static_cast<__bf16>(v[i]);
    *reinterpret_cast<bf16x4v *>(dst) = p;
}
__device__ __forceinline__ void st4(float *dst, const float *v) {
    *reinterpret_cast<f32x4 *>(dst) = f32x4{v[0], v[1], v[2], v[3]};
}

__device__ __forceinline__ f32x4 mma_kb(const __bf16 *ar, const __bf16 *br, f32x4 acc, int g) {
    const bf16x8 av = *reinterpret_cast<const bf16x8 *>(ar + 8 * g);
    const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(br + 8 * g);
    return mfma_bf16(av, bv, acc);
}
__device__ __forceinline__ f32x4 mma_kb(const float *ar, const float *br, f32x4 acc, int g) {
    const f32x4 av = *reinterpret_cast<const f32x4 *>(ar + 4 * g);
    const f32x4 bv = *reinterpret_cast<const f32x4 *>(br + 4 * g);
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

// Buffer resources of sequence (bb, hh): token tau of this head at tau * tok
// bytes from the resource base; s0..s3 are dt, lambda and the next token's dt,
// lambda (mamba3_scan) or a, g, w (ssd_chunked).
// With `live` false every resource has no records: loads through it return
// zeros without touching memory (a prefetch past the last chunk).
template <typename T, int N, int P, int R>
__device__ __forceinline__ SeqBufs seq_bufs(const ScanLaunch &a, size_t bb, size_t hh,
                                            bool live = true) {
    constexpr uint32_t SZ = sizeof(T);
    constexpr int NH = N / 2;
    const size_t H = a.heads, L = a.seq;
    const bool rot = a.theta != nullptr;
    SeqBufs rs;
    const size_t row0 = bb * L * H + hh;
    const size_t rows = live ? L * H - hh : 0;
    auto mk = [&](const void *base, size_t row_bytes) {
        return make_rsrc(static_cast<const char *>(base) + row0 * row_bytes,
                         static_cast<uint32_t>(rows * row_bytes));
    };
    rs.b = mk(a.b, N * R * SZ);
    rs.c = mk(a.c, N * R * SZ);
    rs.x = mk(a.x, P * R * SZ);
    rs.y = mk(a.y, P * R * SZ);
    if (!rot) {
        rs.th = make_rsrc(a.x, 0u);   // no records: zeros
    } else if (a.theta_stride == 0) {
        rs.th = mk(a.theta, NH * SZ);
    } else {
        // token rows theta_stride elements apart: the range ends with this
        // head's row of the sequence's last token
        const size_t tok = a.theta_stride * SZ;
        rs.th = make_rsrc(static_cast<const char *>(a.theta) + bb * L * tok + hh * NH * SZ,
                          live ? static_cast<uint32_t>((L - 1) * tok + NH * SZ) : 0u);
    }
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
    rs.tok_th = static_cast<uint32_t>((a.theta_stride ? a.theta_stride : H * NH) * SZ);
    rs.tok_s = static_cast<uint32_t>(H * 4);
    return rs;
}

// Raw inputs of one chunk as this lane loads them (lane = token): its pair
// slices of B (and of C when WC), its theta slice, its head_dim slice of x,
// and dt / lambda of the token and of the next one.  Buffer loads: tokens at
// or past the sequence end read as zeros.
template <typename T, int N, int P, int R, int ROWS, int NW, bool WC = true>
struct Raw {
    using G = Geo<T, N, P, R, ROWS, NW>;
    u32x4 b[2][G::HV];
    u32x4 c[WC ? 2 : 1][WC ? G::HV : 1];
    unsigned int th[G::TW];
    u32x4 x[G::XV];
    float s0, s1, s2, s3;   // dt, lambda, dt_next, lambda_next (or a, g, w)
};

template <typename T, int N, int P, int R, int ROWS, int NW, bool WC>
__device__ __forceinline__ void load_chunk(const SeqBufs &rs, int ck, int wave, int lane,
                                           Raw<T, N, P, R, ROWS, NW, WC> &raw) {
    // issued in the order the stage consumes them (vmcnt counts in order):
    // the per-token scalars and theta feed the prefix scans and the sines
    // while B, C and x are still in flight
    using G = Geo<T, N, P, R, ROWS, NW>;
    constexpr uint32_t SZ = sizeof(T);
    const uint32_t sub = lane / G::SW;
    const uint32_t tok = static_cast<uint32_t>(ck) * G::QT + lane % G::SW;
    const uint32_t i0 = wave * G::PW + sub * G::PPL;
    raw.s0 = bldf(rs.s0, tok * rs.tok_s);
    raw.s1 = bldf(rs.s1, tok * rs.tok_s);
    raw.s2 = bldf(rs.s2, (tok + rs.nxt_s) * rs.tok_s);
    raw.s3 = bldf(rs.s3, (tok + rs.nxt_s) * rs.tok_s);
    // the scheduler keeps the groups in this order wherever the function is
    // inlined, so every call site leaves the same vmcnt pattern behind
    __builtin_amdgcn_sched_barrier(0);
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
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t ob = tok * rs.tok_bc;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int v = 0; v < G::HV; ++v) {
            const uint32_t off = ob + ((i0 + h * G::NH) * R + v * G::E) * SZ;
            raw.b[h][v] = bld16(rs.b, off);
            if constexpr (WC) raw.c[h][v] = bld16(rs.c, off);
        }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t ox = tok * rs.tok_x + (wave * (P / NW) * R + sub * G::XE) * SZ;
#pragma unroll
    for (int v = 0; v < G::XV; ++v) raw.x[v] = bld16(rs.x, ox + 16 * v);
    __builtin_amdgcn_sched_barrier(0);
}

// The per-token scalars of a lane's token as loaded (the fields of Raw that
// token_scalars reads).
struct TokScalars {
    float s0, s1, s2, s3;
};

// Per-token scalars of this lane's token: log decay a, diagonal weight g,
// off-diagonal weight w (fused.rs:2483-2503), zero for tokens past the end.
template <typename RawT>
__device__ __forceinline__ void token_scalars(const ScanLaunch &a, const RawT &cur, float A,
                                              bool live, float &av, float &gv, float &wv) {
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
}

}  // namespace scan
}  // namespace m3
