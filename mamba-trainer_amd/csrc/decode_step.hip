// Recurrent decode step of the Mamba-3 SSM for gfx950, in place on the f32
// state cache.  Restates src/ssm/scan.rs:649-712 (mamba3_step) and the fused
// kernels it calls:
//   ssm_coefficients  src/tensor/ops/fused.rs:1679-1697
//   ssm_angle         src/tensor/ops/fused.rs:1534-1555
//   rotate_halves     src/tensor/ops/fused.rs:588-619 (from_angle)
//   ssm_state_update  src/tensor/ops/fused.rs:1348-1364
// plus the u = x B^T and y = C^T h products (scan.rs:683-698) and the skip.
//
// One workgroup per (batch, head).  Its prologue advances the angle, rotates B
// and C into LDS and forms alpha, beta, gamma; the body then streams the
// [P, N] f32 state once: read h and last_u, write h' and last_u' = u, with
// y = C~^T h' reduced across the lanes that hold one row.  That is the
// minimum traffic of 16 bytes per state element -- the reference's step
// reads and writes the state about twice that (new u tensor, a separate
// update pass, and a materialised transpose of h for the readout).
//
// Factored form (FACT): last_u is the previous token's rank-R outer product
// x_prev B~_prev^T (scan.rs:683-691), so the state carries that token's x and
// unrotated b instead, with B~_prev = R(-angle) b_prev from the angle as it
// stood before this step's advance.  The body forms last_u in registers with
// the same f32 products the previous step stored, so the results equal the
// full form's bit for bit, and the state streams h only: 8 bytes per element.
#include "m3_device.hpp"
#include "m3_internal.hpp"
#include "mixer_math.hpp"

namespace m3 {

namespace {

constexpr int kStepThreads = 256;
constexpr int kStepConvTaps = static_cast<int>(kMixerStepConvTaps);

template <typename T>
__device__ __forceinline__ float ld(const void *p, size_t i) {
    return to_f32(static_cast<const T *>(p)[i]);
}

// A pair rotated by -phi, (x1 cos + x2 sin, -x1 sin + x2 cos), with explicit
// fused multiply-adds so that every instantiation rounds the same way (the
// factored form rotates the previous token's B again and must reproduce the
// B~ the step that took it used).
__device__ __forceinline__ float rot_lo(float x1, float x2, float cs, float sn) {
    return __builtin_fmaf(x1, cs, x2 * sn);
}
__device__ __forceinline__ float rot_hi(float x1, float x2, float cs, float sn) {
    return __builtin_fmaf(x2, cs, -(x1 * sn));
}

// Prologue shared by both bodies: angle advance, rotation of B and C into
// LDS (rank-last [N][R] layout kept), x into LDS, and the coefficients.  bh
// indexes the state, ib the inputs (bh except with in_bstride).
template <typename T, bool FACT = false>
__device__ __forceinline__ void step_prologue(const StepLaunch &a, size_t bh, size_t ib,
                                              float *bt, float *ct, float *xs, float &alpha,
                                              float &beta, float &gamma, float *bpt = nullptr,
                                              float *xps = nullptr) {
    const int tid = threadIdx.x;
    const size_t N = a.d_state, P = a.head_dim, R = a.rank;
    const size_t half = N / 2;
    const size_t hh = bh % a.heads;
    const float step = a.dt[ib];
    const float lam = a.lambda[ib];
    const size_t bc_base = ib * N * R;
    const size_t bp_base = bh * N * R;
    if (a.theta != nullptr) {
        for (size_t i = tid; i < half; i += kStepThreads) {
            // phi = wrap(prev + dt * theta)   (fused.rs:1549-1553)
            const float prev = a.angle[bh * half + i];
            float raw = ld<T>(a.theta, ib * half + i) * step + prev;
            float phi = wrap_angle(raw);
            a.angle[bh * half + i] = phi;
            float sn, cs;
            sincosf(phi, &sn, &cs);
            if constexpr (FACT) {
                // the previous token's B~, rotated by the angle it was taken at
                // with the roundings the previous step used (rot_lo / rot_hi)
                float ps, pc;
                sincosf(prev, &ps, &pc);
                for (size_t r = 0; r < R; ++r) {
                    const float b1 = ld<T>(a.b_prev, bp_base + i * R + r);
                    const float b2 = ld<T>(a.b_prev, bp_base + (i + half) * R + r);
                    bpt[i * R + r] = rot_lo(b1, b2, pc, ps);
                    bpt[(i + half) * R + r] = rot_hi(b1, b2, pc, ps);
                }
            }
            for (size_t r = 0; r < R; ++r) {
                float b1 = ld<T>(a.b, bc_base + i * R + r);
                float b2 = ld<T>(a.b, bc_base + (i + half) * R + r);
                float c1 = ld<T>(a.c, bc_base + i * R + r);
                float c2 = ld<T>(a.c, bc_base + (i + half) * R + r);
                // rotation by -phi: (x1 cos + x2 sin, -x1 sin + x2 cos)
                bt[i * R + r] = rot_lo(b1, b2, cs, sn);
                bt[(i + half) * R + r] = rot_hi(b1, b2, cs, sn);
                ct[i * R + r] = rot_lo(c1, c2, cs, sn);
                ct[(i + half) * R + r] = rot_hi(c1, c2, cs, sn);
            }
        }
        // odd N: the unpaired last component is not rotated (N is even whenever
        // theta is given; validation enforces it)
    } else {
        for (size_t i = tid; i < N * R; i += kStepThreads) {
            bt[i] = ld<T>(a.b, bc_base + i);
            ct[i] = ld<T>(a.c, bc_base + i);
            if constexpr (FACT) bpt[i] = ld<T>(a.b_prev, bp_base + i);
        }
    }
    for (size_t i = tid; i < P * R; i += kStepThreads) {
        xs[i] = ld<T>(a.x, ib * P * R + i);
        if constexpr (FACT) xps[i] = ld<T>(a.x_prev, bh * P * R + i);
    }
    // alpha = exp(dt * -exp(a_log)), beta = (1 - lambda) dt alpha, gamma = lambda dt
    const float A = 0.0f - expf(a.a_log[hh]);
    alpha = expf(step * A);
    beta = (1.0f - lam) * step * alpha;
    gamma = lam * step;
}

// Eight channels ch .. ch+7 of the causal convolution over [x | B | C] (px
// is this sequence's row from x on) at its one position: taps 0 .. k-2 read
// the history, tap k-1 the row, with the arithmetic of conv_taps8 (the same
// fused multiply-adds in the same order as m3_mixer_prologue_conv).  Every
// tap's inputs and weights are loaded before the first is used (k is at most
// kStepConvTaps; the host checks), so the lane waits for memory once.  With
// `write`, the lane then stores the new history of these channels from the
// values it holds, the window's last k-1 positions: row i takes the old row
// i+1, the last row this token.  The lane has read every old row of its
// channels before it writes any, so the history may be updated in place
// where no other lane or workgroup reads these channels (the host allows
// that only for groups == heads, where every channel belongs to one
// (sequence, head) workgroup).
__device__ __forceinline__ void step_conv8(const MixerStepLaunch &m, size_t bq, size_t C,
                                           const uint16_t *px, size_t ch, bool write, float *f) {
    const int k = static_cast<int>(m.conv_k);
    const uint16_t *hist =
        m.hist ? static_cast<const uint16_t *>(m.hist) + bq * (k - 1) * C : nullptr;
    uint4 raw[kStepConvTaps];
    float4 w0[kStepConvTaps], w1[kStepConvTaps];
#pragma unroll
    for (int j = 0; j < kStepConvTaps; ++j) {
        if (j < k) {
            const uint16_t *src = j + 1 == k ? px + ch : hist ? hist + j * C + ch : nullptr;
            raw[j] = src ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0u, 0u, 0u, 0u);
            w0[j] = *reinterpret_cast<const float4 *>(m.conv_w + j * C + ch);
            w1[j] = *reinterpret_cast<const float4 *>(m.conv_w + j * C + ch + 4);
        }
    }
    if (m.conv_b) {
        const float4 b0 = *reinterpret_cast<const float4 *>(m.conv_b + ch);
        const float4 b1 = *reinterpret_cast<const float4 *>(m.conv_b + ch + 4);
        f[0] = b0.x; f[1] = b0.y; f[2] = b0.z; f[3] = b0.w;
        f[4] = b1.x; f[5] = b1.y; f[6] = b1.z; f[7] = b1.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kStepConvTaps; ++j) {
        // a position before the sequence with no history is skipped, as conv_taps8 does
        if (j < k && (hist != nullptr || j + 1 == k)) {
            float v[8];
            mixm::unpack8(raw[j], v);
            const float wv[8] = {w0[j].x, w0[j].y, w0[j].z, w0[j].w,
                                 w1[j].x, w1[j].y, w1[j].z, w1[j].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = __builtin_fmaf(wv[e], v[e], f[e]);
        }
    }
    if (!write || m.new_hist == nullptr) return;
    uint16_t *nh = static_cast<uint16_t *>(m.new_hist) + bq * (k - 1) * C;
#pragma unroll
    for (int i = 0; i + 1 < kStepConvTaps; ++i)
        if (i + 1 < k) *reinterpret_cast<uint4 *>(nh + i * C + ch) = raw[i + 1];
}

// The fused step's prologue (MixerStepLaunch): the projection row of this
// sequence through the 16-byte prologue's arithmetic (mixer_math.hpp, the
// same roundings: every value is rounded to bf16 where m3_mixer_prologue
// stores it) into LDS -- B and C raw [N][R] (braw, craw), x, theta, dt and
// lambda -- then step_prologue's angle advance, rotation and coefficients on
// those values.  CONV: x, B and C through the causal convolution first
// (step_conv8), which also writes the new history of this head's channels.
template <int R, bool FACT, bool CONV>
__device__ __forceinline__ void mix_prologue(const MixerStepLaunch &m, size_t bh, float *bt,
                                             float *ct, float *xs, float &alpha, float &beta,
                                             float &gamma, float *bpt, float *braw, float *craw,
                                             float *thv, float *scal) {
    using namespace mixm;
    const StepLaunch &a = m.s;
    const int tid = threadIdx.x;
    const int H = static_cast<int>(a.heads), P = static_cast<int>(a.head_dim);
    const int N = static_cast<int>(a.d_state), half = N / 2;
    const size_t bq = bh / a.heads;
    const int h = static_cast<int>(bh % a.heads);
    const int din = H * P * R;
    const int bcw = static_cast<int>(m.groups) * R * N;
    const uint16_t *row = static_cast<const uint16_t *>(m.projected) + bq * m.width;
    const uint16_t *px = row + din;
    const uint16_t *pb = px + din;
    const uint16_t *pc = pb + bcw;
    const uint16_t *pdt = pc + bcw;
    const uint16_t *plam = pdt + H;
    const uint16_t *pth = plam + (m.learned_lambda ? H : 0);
    const int lq = N / 8;
    const int per_group = H / static_cast<int>(m.groups);
    const int grp = h / per_group;
    const int nx = P * R / 8;
    const size_t C = static_cast<size_t>(din) + 2 * static_cast<size_t>(bcw);
    if (tid < 2 * lq) {
        // B (lanes 0 .. lq-1) and C (lq .. 2 lq-1): eight states of every rank
        const int which = tid / lq, q = tid - which * lq;
        const uint16_t *src = (which ? pc : pb) + grp * R * N + q * 8;
        const float *bias = which ? m.c_bias : m.b_bias;
        float v[R][8], bb[8], w[8];
        if constexpr (CONV) {
            // the group's channels: their history is written by its first head
            const size_t ch0 = static_cast<size_t>(src - px);
#pragma unroll
            for (int r = 0; r < R; ++r)
                step_conv8(m, bq, C, px, ch0 + r * N, h % per_group == 0, v[r]);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) unpack8(*reinterpret_cast<const uint4 *>(src + r * N), v[r]);
        }
        if (bias) {
            const float4 b0 = *reinterpret_cast<const float4 *>(bias + h * N + q * 8);
            const float4 b1 = *reinterpret_cast<const float4 *>(bias + h * N + q * 8 + 4);
            bb[0] = b0.x; bb[1] = b0.y; bb[2] = b0.z; bb[3] = b0.w;
            bb[4] = b1.x; bb[5] = b1.y; bb[6] = b1.z; bb[7] = b1.w;
        }
        if (m.bc_norm) {
            const float4 w0 = *reinterpret_cast<const float4 *>(m.bc_norm + q * 8);
            const float4 w1 = *reinterpret_cast<const float4 *>(m.bc_norm + q * 8 + 4);
            w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
            w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
        }
        bc_row8<R>(v, bb, bias != nullptr, w, m.bc_norm != nullptr, lq, 1.0f / static_cast<float>(N),
                   m.norm_eps);
        float *dst = which ? craw : braw;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r) dst[(q * 8 + j) * R + r] = bf16_bits_to_f32(to_bits(v[r][j]));
    } else if (tid >= 64 && tid < 64 + nx) {
        const int k = tid - 64;
        float f[8];
        if constexpr (CONV)
            step_conv8(m, bq, C, px, static_cast<size_t>(h * P * R + k * 8), true, f);
        else
            unpack8(*reinterpret_cast<const uint4 *>(px + h * P * R + k * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[k * 8 + j] = bf16_bits_to_f32(to_bits(silu_fast(f[j])));
    } else if (tid >= 128 && tid < 128 + half && a.theta != nullptr) {
        thv[tid - 128] = bf(pth, static_cast<size_t>(h) * half + (tid - 128));
    } else if (tid == 255) {
        scal[0] = softplusf_(bf(pdt, h) + m.dt_bias[h]);
        scal[1] = m.learned_lambda ? sigmoidf_(bf(plam, h)) : m.fixed_lambda;
    }
    __syncthreads();

    const float step = scal[0];
    const float lam = scal[1];
    const size_t bc_base = bh * N * R;
    if (a.theta != nullptr) {
        for (int i = tid; i < half; i += kStepThreads) {
            // phi = wrap(prev + dt * theta)   (fused.rs:1549-1553)
            const float prev = a.angle[bh * half + i];
            float raw = thv[i] * step + prev;
            float phi = wrap_angle(raw);
            a.angle[bh * half + i] = phi;
            float sn, cs;
            sincosf(phi, &sn, &cs);
            if constexpr (FACT) {
                float ps, pc;
                sincosf(prev, &ps, &pc);
                for (int r = 0; r < R; ++r) {
                    const float b1 = ld<bf16_t>(a.b_prev, bc_base + i * R + r);
                    const float b2 = ld<bf16_t>(a.b_prev, bc_base + (i + half) * R + r);
                    bpt[i * R + r] = rot_lo(b1, b2, pc, ps);
                    bpt[(i + half) * R + r] = rot_hi(b1, b2, pc, ps);
                }
            }
            for (int r = 0; r < R; ++r) {
                const float b1 = braw[i * R + r], b2 = braw[(i + half) * R + r];
                const float c1 = craw[i * R + r], c2 = craw[(i + half) * R + r];
                bt[i * R + r] = rot_lo(b1, b2, cs, sn);
                bt[(i + half) * R + r] = rot_hi(b1, b2, cs, sn);
                ct[i * R + r] = rot_lo(c1, c2, cs, sn);
                ct[(i + half) * R + r] = rot_hi(c1, c2, cs, sn);
            }
        }
    } else {
        for (int i = tid; i < N * R; i += kStepThreads) {
            bt[i] = braw[i];
            ct[i] = craw[i];
            if constexpr (FACT) bpt[i] = ld<bf16_t>(a.b_prev, bc_base + i);
        }
    }
    const float A = 0.0f - expf(a.a_log[h]);
    alpha = expf(step * A);
    beta = (1.0f - lam) * step * alpha;
    gamma = lam * step;
}

// Vector body: N % 4 == 0 and G = N / 4 lanes per row with G a power of two
// that divides 64.  Each lane owns four consecutive state columns of a row.
// MIX: the fused mixer step (mix_prologue in, the gate out); CONV: its
// convolution.
template <typename T, int RK, bool FACT, bool MIX = false, bool CONV = false>
__device__ __forceinline__ void step_body_vec(const StepLaunch &a, size_t bh,
                                              const MixerStepLaunch *m = nullptr) {
    extern __shared__ float smem[];
    const size_t N = a.d_state, P = a.head_dim;
    constexpr int R = RK;
    float *bt = smem;
    float *ct = bt + N * R;
    float *xs = ct + N * R;
    float *bpt = xs + P * R;         // FACT: B~_prev [N][R], x_prev [P][R]
    float *xps = bpt + N * R;
    // MIX: raw B, C [N][R], theta, dt and lambda (over B~_prev's slot when
    // the state is not factored)
    float *braw = FACT ? xps + P * R : bpt;
    float *craw = braw + N * R;
    float *thv = craw + N * R;
    float *scal = thv + N / 2;
    float alpha, beta, gamma;
    if constexpr (MIX)
        mix_prologue<R, FACT, CONV>(*m, bh, bt, ct, xs, alpha, beta, gamma, bpt, braw, craw, thv,
                                    scal);
    else
        step_prologue<T, FACT>(a, bh, bh, bt, ct, xs, alpha, beta, gamma, bpt, xps);
    if constexpr (FACT && MIX) {
        for (size_t i = threadIdx.x; i < P * R; i += kStepThreads)
            xps[i] = ld<T>(a.x_prev, bh * P * R + i);
    }
    __syncthreads();
    if constexpr (FACT) {
        // this step's x and b become the state's previous token (every read of
        // the old ones happened before the barrier)
        T *xp = static_cast<T *>(a.x_prev) + bh * P * R;
        T *bp = static_cast<T *>(a.b_prev) + bh * N * R;
        if constexpr (MIX) {
            for (size_t i = threadIdx.x; i < P * R; i += kStepThreads) xp[i] = from_f32<T>(xs[i]);
            for (size_t i = threadIdx.x; i < N * R; i += kStepThreads) bp[i] = from_f32<T>(braw[i]);
        } else {
            const T *xb = static_cast<const T *>(a.x) + bh * P * R;
            const T *bb = static_cast<const T *>(a.b) + bh * N * R;
            for (size_t i = threadIdx.x; i < P * R; i += kStepThreads) xp[i] = xb[i];
            for (size_t i = threadIdx.x; i < N * R; i += kStepThreads) bp[i] = bb[i];
        }
    }

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = static_cast<int>(N / 4);          // lanes per row
    const int rows_per_wave = 64 / G;
    const int rows_per_pass = rows_per_wave * (kStepThreads / 64);
    const int col4 = (lane % G) * 4;
    const float dskip = a.d_skip ? a.d_skip[bh % a.heads] : 0.0f;
    f32x4 *h4 = reinterpret_cast<f32x4 *>(a.h + bh * P * N);
    f32x4 *u4 = reinterpret_cast<f32x4 *>(a.last_u + bh * P * N);

    // B~ columns this lane touches, hoisted out of the row loop.
    float bcol[4][R], ccol[4][R], pcol[4][FACT ? R : 1];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            bcol[j][r] = bt[(col4 + j) * R + r];
            ccol[j][r] = ct[(col4 + j) * R + r];
            if constexpr (FACT) pcol[j][r] = bpt[(col4 + j) * R + r];
        }

    constexpr int kBatch = 4;   // rows in flight per lane
    for (int base = wave * rows_per_wave + lane / G; base < static_cast<int>(P);
         base += rows_per_pass * kBatch) {
        f32x4 hv[kBatch], lv[kBatch];
        int rows[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            rows[k] = base + k * rows_per_pass;
            if (rows[k] < static_cast<int>(P)) {
                size_t idx = (static_cast<size_t>(rows[k]) * N + col4) / 4;
                hv[k] = __builtin_nontemporal_load(&h4[idx]);
                if constexpr (!FACT) lv[k] = __builtin_nontemporal_load(&u4[idx]);
            }
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int p = rows[k];
            // every lane of a row group shares `p`, so the guard is uniform per group
            const bool live = p < static_cast<int>(P);
            float ypart[R];
#pragma unroll
            for (int r = 0; r < R; ++r) ypart[r] = 0.0f;
            if (live) {
                float xr[R], xq[FACT ? R : 1];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    xr[r] = xs[p * R + r];
                    if constexpr (FACT) xq[r] = xps[p * R + r];
                }
                f32x4 hn, un;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // explicit fused multiply-adds: the rounding of u (stored as
                    // last_u, or formed again by the factored form from the same
                    // operands) and of h' must not depend on how the compiler
                    // contracts each instantiation
                    float u = xr[0] * bcol[j][0];
#pragma unroll
                    for (int r = 1; r < R; ++r) u = __builtin_fmaf(xr[r], bcol[j][r], u);
                    float lu;
                    if constexpr (FACT) {
                        // the previous step's u, the same products in the same order
                        lu = xq[0] * pcol[j][0];
#pragma unroll
                        for (int r = 1; r < R; ++r) lu = __builtin_fmaf(xq[r], pcol[j][r], lu);
                    } else {
                        lu = lv[k][j];
                    }
                    // h' = h*alpha + last_u*beta + u*gamma   (fused.rs:1360-1362)
                    const float ha = hv[k][j] * alpha;
                    float hnew = __builtin_fmaf(u, gamma, __builtin_fmaf(lu, beta, ha));
                    hn[j] = hnew;
                    un[j] = u;
#pragma unroll
                    for (int r = 0; r < R; ++r) ypart[r] = __builtin_fmaf(ccol[j][r], hnew, ypart[r]);
                }
                size_t idx = (static_cast<size_t>(p) * N + col4) / 4;
                __builtin_nontemporal_store(hn, &h4[idx]);
                if constexpr (!FACT) __builtin_nontemporal_store(un, &u4[idx]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) ypart[r] = group_sum(ypart[r], G);
            if (live && (lane % G) == 0) {
                if constexpr (MIX) {
                    // the gate: silu(z) * y with y rounded to bf16 first, as
                    // m3_mixer_gate reads it (models/mamba3.rs:468-477); y
                    // alone where a post-gate norm comes between
                    const uint16_t *z = static_cast<const uint16_t *>(m->projected) +
                                        (bh / a.heads) * m->width + (bh % a.heads) * P * R;
                    uint16_t *o = static_cast<uint16_t *>(m->out) + bh * P * R;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint16_t yb = mixm::to_bits(__builtin_fmaf(xs[p * R + r], dskip, ypart[r]));
                        o[p * R + r] = m->gate ? mixm::to_bits(bf16_bits_to_f32(yb) *
                                                               mixm::silu_fast(mixm::bf(z, p * R + r)))
                                               : yb;
                    }
                } else {
                    T *y = static_cast<T *>(a.y);
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        y[(bh * P + p) * R + r] = from_f32<T>(__builtin_fmaf(xs[p * R + r], dskip, ypart[r]));
                }
            }
        }
    }
}

template <typename T, int RK, bool FACT>
__global__ void __launch_bounds__(kStepThreads)
step_kernel_vec(StepLaunch a) {
    step_body_vec<T, RK, FACT>(a, blockIdx.x);
}

// Several layers' steps in one launch: workgroup w steps (batch, head)
// w % (B H) of layer w / (B H), whose buffers the table names (the shapes are
// the layers' common ones).
template <typename T, int RK, bool FACT>
__global__ void __launch_bounds__(kStepThreads)
step_kernel_vec_layers(StepLaunch base, StepLayerTable t) {
    const size_t per = base.batch * base.heads;
    const size_t l = blockIdx.x / per;
    StepLaunch a = base;
    const StepLayer &L = t.layer[l];
    a.x = L.x;
    a.b = L.b;
    a.c = L.c;
    a.dt = L.dt;
    a.lambda = L.lambda;
    a.a_log = L.a_log;
    a.theta = L.theta;
    a.d_skip = L.d_skip;
    a.h = L.h;
    a.last_u = L.last_u;
    a.angle = L.angle;
    a.y = L.y;
    a.x_prev = L.x_prev;
    a.b_prev = L.b_prev;
    step_body_vec<T, RK, FACT>(a, blockIdx.x - l * per);
}

template <int RK, bool FACT, bool CONV>
__global__ void __launch_bounds__(kStepThreads)
mixer_step_kernel(MixerStepLaunch m) {
    step_body_vec<bf16_t, RK, FACT, true, CONV>(m.s, blockIdx.x, &m);
}

// Generic body for shapes the vector body does not cover (odd N, N > 256,
// rank other than 1, 2, 3, 4 or 8, inputs at a batch stride): one thread per
// state row.
template <typename T>
__global__ void __launch_bounds__(kStepThreads)
step_kernel_generic(StepLaunch a) {
    extern __shared__ float smem[];
    const size_t N = a.d_state, P = a.head_dim, R = a.rank;
    float *bt = smem;
    float *ct = bt + N * R;
    float *xs = ct + N * R;
    const size_t bh = blockIdx.x;
    const size_t ib = a.in_bstride ? (bh / a.heads) * a.in_bstride * a.heads + bh % a.heads : bh;
    float alpha, beta, gamma;
    step_prologue<T>(a, bh, ib, bt, ct, xs, alpha, beta, gamma);
    __syncthreads();
    const float dskip = a.d_skip ? a.d_skip[bh % a.heads] : 0.0f;
    float *h = a.h + bh * P * N;
    float *lu = a.last_u + bh * P * N;
    T *y = static_cast<T *>(a.y);
    for (size_t p = threadIdx.x; p < P; p += kStepThreads) {
        for (size_t n = 0; n < N; ++n) {
            float u = 0.0f;
            for (size_t r = 0; r < R; ++r) u += xs[p * R + r] * bt[n * R + r];
            float hnew = h[p * N + n] * alpha + lu[p * N + n] * beta + u * gamma;
            h[p * N + n] = hnew;
            lu[p * N + n] = u;
        }
        for (size_t r = 0; r < R; ++r) {
            float acc = 0.0f;
            for (size_t n = 0; n < N; ++n) acc += ct[n * R + r] * h[p * N + n];
            y[(ib * P + p) * R + r] = from_f32<T>(acc + xs[p * R + r] * dskip);
        }
    }
}

template <typename T, int RK>
hipError_t launch_vec(const StepLaunch &a, size_t smem, hipStream_t s) {
    if (a.last_u == nullptr)
        hipLaunchKernelGGL((step_kernel_vec<T, RK, true>), dim3(a.batch * a.heads),
                           dim3(kStepThreads), smem, s, a);
    else
        hipLaunchKernelGGL((step_kernel_vec<T, RK, false>), dim3(a.batch * a.heads),
                           dim3(kStepThreads), smem, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t dispatch(const StepLaunch &a, hipStream_t s) {
    const size_t N = a.d_state, R = a.rank;
    const bool fact = a.last_u == nullptr;
    const size_t smem = ((fact ? 3 : 2) * N * R + (fact ? 2 : 1) * a.head_dim * R) * sizeof(float);
    if (fact && !step_factored_supported(N, R)) return hipErrorNotSupported;
    const size_t G = N / 4;
    const bool vec = (N % 4 == 0) && G >= 1 && G <= 64 && (G & (G - 1)) == 0 && a.in_bstride == 0;
    if (vec) {
        switch (R) {
            case 1: return launch_vec<T, 1>(a, smem, s);
            case 2: return launch_vec<T, 2>(a, smem, s);
            case 3: return launch_vec<T, 3>(a, smem, s);
            case 4: return launch_vec<T, 4>(a, smem, s);
            case 8: return launch_vec<T, 8>(a, smem, s);
            default: break;
        }
    }
    hipLaunchKernelGGL((step_kernel_generic<T>), dim3(a.batch * a.heads), dim3(kStepThreads),
                       smem, s, a);
    return hipGetLastError();
}

template <typename T, int RK>
hipError_t launch_vec_layers(const StepLaunch &a, const StepLayerTable &t, size_t n, size_t smem,
                             hipStream_t s) {
    const dim3 grid(static_cast<unsigned int>(n * a.batch * a.heads));
    if (a.last_u == nullptr)
        hipLaunchKernelGGL((step_kernel_vec_layers<T, RK, true>), grid, dim3(kStepThreads), smem, s,
                           a, t);
    else
        hipLaunchKernelGGL((step_kernel_vec_layers<T, RK, false>), grid, dim3(kStepThreads), smem,
                           s, a, t);
    return hipGetLastError();
}

template <typename T>
hipError_t dispatch_layers(const StepLaunch &a, const StepLayerTable &t, size_t n, hipStream_t s) {
    const size_t N = a.d_state, R = a.rank;
    const bool fact = a.last_u == nullptr;
    const size_t smem = ((fact ? 3 : 2) * N * R + (fact ? 2 : 1) * a.head_dim * R) * sizeof(float);
    switch (R) {
        case 1: return launch_vec_layers<T, 1>(a, t, n, smem, s);
        case 2: return launch_vec_layers<T, 2>(a, t, n, smem, s);
        case 3: return launch_vec_layers<T, 3>(a, t, n, smem, s);
        case 4: return launch_vec_layers<T, 4>(a, t, n, smem, s);
        case 8: return launch_vec_layers<T, 8>(a, t, n, smem, s);
        default: return hipErrorNotSupported;
    }
}

// last_u = x_prev (R(-angle) b_prev)^T for one (batch, head): the full state a
// factored one stands for.  One workgroup per (batch, head); the rotated b
// goes through LDS with the roundings the step used for it.
template <typename T>
__global__ void __launch_bounds__(kStepThreads)
unfactor_kernel(size_t heads, size_t P, size_t N, size_t R, const void *x_prev, const void *b_prev,
                const float *angle, float *last_u) {
    extern __shared__ float smem[];
    float *bt = smem;             // [N][R]
    float *xs = bt + N * R;       // [P][R]
    const size_t bh = blockIdx.x;
    const size_t half = N / 2;
    const size_t base = bh * N * R;
    for (size_t i = threadIdx.x; i < (angle ? half : N); i += kStepThreads) {
        if (angle != nullptr) {
            float sn, cs;
            sincosf(angle[bh * half + i], &sn, &cs);
            for (size_t r = 0; r < R; ++r) {
                const float b1 = ld<T>(b_prev, base + i * R + r);
                const float b2 = ld<T>(b_prev, base + (i + half) * R + r);
                bt[i * R + r] = rot_lo(b1, b2, cs, sn);
                bt[(i + half) * R + r] = rot_hi(b1, b2, cs, sn);
            }
        } else {
            for (size_t r = 0; r < R; ++r) bt[i * R + r] = ld<T>(b_prev, base + i * R + r);
        }
    }
    for (size_t i = threadIdx.x; i < P * R; i += kStepThreads) xs[i] = ld<T>(x_prev, bh * P * R + i);
    __syncthreads();
    float *lu = last_u + bh * P * N;
    for (size_t e = threadIdx.x; e < P * N; e += kStepThreads) {
        const size_t p = e / N, n = e % N;
        float u = xs[p * R] * bt[n * R];
        for (size_t r = 1; r < R; ++r) u = __builtin_fmaf(xs[p * R + r], bt[n * R + r], u);
        lu[e] = u;
    }
}

}  // namespace

hipError_t launch_unfactor(size_t batch, size_t heads, size_t P, size_t N, size_t R, bool bf16,
                           const void *x_prev, const void *b_prev, const float *angle,
                           float *last_u, hipStream_t s) {
    if (batch * heads == 0) return hipSuccess;
    const size_t smem = (N * R + P * R) * sizeof(float);
    if (bf16)
        hipLaunchKernelGGL(unfactor_kernel<bf16_t>, dim3(static_cast<unsigned int>(batch * heads)),
                           dim3(kStepThreads), smem, s, heads, P, N, R, x_prev, b_prev, angle, last_u);
    else
        hipLaunchKernelGGL(unfactor_kernel<float>, dim3(static_cast<unsigned int>(batch * heads)),
                           dim3(kStepThreads), smem, s, heads, P, N, R, x_prev, b_prev, angle, last_u);
    return hipGetLastError();
}

bool step_layers_supported(size_t d_state, size_t rank) { return step_factored_supported(d_state, rank); }

hipError_t launch_step_layers(const StepLaunch &a, const StepLayerTable &t, size_t n,
                              hipStream_t stream) {
    if (n == 0 || a.batch * a.heads == 0) return hipSuccess;
    if (n > kStepLayersPerLaunch || !step_layers_supported(a.d_state, a.rank))
        return hipErrorNotSupported;
    return a.bf16 ? dispatch_layers<bf16_t>(a, t, n, stream) : dispatch_layers<float>(a, t, n, stream);
}

bool step_factored_supported(size_t d_state, size_t rank) {
    const size_t G = d_state / 4;
    return d_state % 4 == 0 && G >= 1 && G <= 64 && (G & (G - 1)) == 0 &&
           (rank == 1 || rank == 2 || rank == 3 || rank == 4 || rank == 8);
}

bool mixer_step_supported(size_t head_dim, size_t d_state, size_t rank, size_t width) {
    const size_t lq = d_state / 8;
    // (d_state <= 128: the prologue's theta lanes are threads 128 .. 128 + N/2 - 1,
    // below the dt / lambda thread 255)
    return d_state % 8 == 0 && lq >= 1 && lq <= 16 && (lq & (lq - 1)) == 0 &&
           (head_dim * rank) % 8 == 0 && head_dim * rank / 8 <= 64 && width % 8 == 0 &&
           (rank == 1 || rank == 2 || rank == 4 || rank == 8) &&
           step_factored_supported(d_state, rank);
}

hipError_t launch_mixer_step(const MixerStepLaunch &m, hipStream_t stream) {
    const StepLaunch &a = m.s;
    if (a.batch * a.heads == 0) return hipSuccess;
    const size_t N = a.d_state, P = a.head_dim, R = a.rank;
    const bool fact = a.last_u == nullptr;
    const size_t smem =
        ((fact ? 5 : 4) * N * R + (fact ? 2 : 1) * P * R + N / 2 + 2) * sizeof(float);
    const dim3 grid(static_cast<unsigned int>(a.batch * a.heads));
#define M3_MIX2(RK, CV)                                                                            \
    if (fact)                                                                                      \
        hipLaunchKernelGGL((mixer_step_kernel<RK, true, CV>), grid, dim3(kStepThreads), smem,      \
                           stream, m);                                                             \
    else                                                                                           \
        hipLaunchKernelGGL((mixer_step_kernel<RK, false, CV>), grid, dim3(kStepThreads), smem,     \
                           stream, m);
#define M3_MIX(RK)                                                                                 \
    if (m.conv_k) {                                                                                \
        M3_MIX2(RK, true)                                                                          \
    } else {                                                                                       \
        M3_MIX2(RK, false)                                                                         \
    }
    switch (R) {
        case 1: M3_MIX(1) break;
        case 2: M3_MIX(2) break;
        case 4: M3_MIX(4) break;
        case 8: M3_MIX(8) break;
        default: return hipErrorNotSupported;
    }
#undef M3_MIX
#undef M3_MIX2
    return hipGetLastError();
}

hipError_t launch_step(const StepLaunch &a, hipStream_t stream) {
    if (a.batch * a.heads == 0) return hipSuccess;
    return a.bf16 ? dispatch<bf16_t>(a, stream) : dispatch<float>(a, stream);
}

}  // namespace m3
