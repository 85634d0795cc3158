// The token-parallel pieces of the Mamba-3 mixer around the scan, for bf16
// activations: RMSNorm rows (nn/norm.rs:95-105, fused.rs:140-185), the
// per-output-channel int8 weight grid (nn/quant.rs:231-245, 282-330), the
// projection prologue of Mamba3Mixer::project (models/mamba3.rs:376-466:
// split, silu, B/C bias and RMSNorm, softplus, sigmoid, the scan layouts), the
// gate of Mamba3Mixer::finish (models/mamba3.rs:468-477) and the embedding
// gather (nn/embedding.rs).  All are HBM-bound: each reads its inputs once and
// writes its outputs once, with f32 arithmetic in registers.
#include "m3_device.hpp"
#include "m3_internal.hpp"
#include "mixer_math.hpp"

namespace m3 {

namespace {

using namespace mixm;

// ---------------------------------------------------------------- RMSNorm
// One wave per row.  Rows whose width is a multiple of 8 and whose base is
// 16-byte aligned move as 16-byte vectors; others element by element.
__global__ void __launch_bounds__(256)
rms_norm_kernel(size_t rows, size_t dim, const uint16_t *x, size_t xs, const float *w, float eps,
                uint16_t *y, size_t ys) {
    const size_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const uint16_t *xr = x + row * xs;
    uint16_t *yr = y + row * ys;
    const bool vec = (dim % 8 == 0) && ((reinterpret_cast<uintptr_t>(xr) & 15) == 0) &&
                     ((reinterpret_cast<uintptr_t>(yr) & 15) == 0);
    if (vec && dim <= 2048 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
        // the whole row in registers (up to four 16-byte pieces a lane): the
        // row's and the gain's loads all in flight at once, no second read
        uint4 q[4];
        f32x4 wv[4][2];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const size_t i = lane * 8 + c * 512;
            q[c] = make_uint4(0u, 0u, 0u, 0u);
            wv[c][0] = wv[c][1] = f32x4{1.f, 1.f, 1.f, 1.f};
            if (i < dim) {
                q[c] = *reinterpret_cast<const uint4 *>(xr + i);
                if (w) {
                    wv[c][0] = *reinterpret_cast<const f32x4 *>(w + i);
                    wv[c][1] = *reinterpret_cast<const f32x4 *>(w + i + 4);
                }
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const unsigned int u[4] = {q[c].x, q[c].y, q[c].z, q[c].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = __uint_as_float(u[j] << 16), b = __uint_as_float(u[j] & 0xFFFF0000u);
                ss += a * a + b * b;
            }
        }
        ss = group_sum(ss, 64);
        const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const size_t i = lane * 8 + c * 512;
            if (i >= dim) continue;
            const unsigned int u[4] = {q[c].x, q[c].y, q[c].z, q[c].w};
            unsigned int o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float a = __uint_as_float(u[j] << 16) * scale, b = __uint_as_float(u[j] & 0xFFFF0000u) * scale;
                if (w) {
                    a *= wv[c][j >> 1][2 * (j & 1)];
                    b *= wv[c][j >> 1][2 * (j & 1) + 1];
                }
                o[j] = pack2(a, b);
            }
            *reinterpret_cast<uint4 *>(yr + i) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        return;
    }
    float ss = 0.0f;
    if (vec) {
        for (size_t i = lane * 8; i < dim; i += 512) {
            const uint4 q = *reinterpret_cast<const uint4 *>(xr + i);
            const unsigned int u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = __uint_as_float(u[j] << 16), b = __uint_as_float(u[j] & 0xFFFF0000u);
                ss += a * a + b * b;
            }
        }
    } else {
        for (size_t i = lane; i < dim; i += 64) {
            const float v = bf(xr, i);
            ss += v * v;
        }
    }
    ss = group_sum(ss, 64);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
    if (vec) {
        for (size_t i = lane * 8; i < dim; i += 512) {
            const uint4 q = *reinterpret_cast<const uint4 *>(xr + i);
            const unsigned int u[4] = {q.x, q.y, q.z, q.w};
            unsigned int o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float a = __uint_as_float(u[j] << 16) * scale, b = __uint_as_float(u[j] & 0xFFFF0000u) * scale;
                if (w) {
                    a *= w[i + 2 * j];
                    b *= w[i + 2 * j + 1];
                }
                o[j] = pack2(a, b);
            }
            *reinterpret_cast<uint4 *>(yr + i) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else {
        for (size_t i = lane; i < dim; i += 64) {
            float v = bf(xr, i) * scale;
            if (w) v *= w[i];
            yr[i] = to_bits(v);
        }
    }
}

// ---------------------------------------------------------------- int8 grid
// QuantConfig::int8_weights on a [k, n] weight: per output channel j,
// scale = max(max_i |w_ij|, 1e-12) / 127 (solve_scale, quant.rs:282-288) and
// code = clamp(round(w / scale), -127, 127) (quant.rs:240-244).  Codes are
// whole numbers of at most 7 bits, exact in bf16.  One thread per column.
__global__ void __launch_bounds__(256)
quantize_columns_kernel(size_t k, size_t n, const float *w, uint16_t *codes, float *scales) {
    const size_t j = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (j >= n) return;
    float m = 0.0f;
    for (size_t i = 0; i < k; ++i) m = fmaxf(m, fabsf(w[i * n + j]));
    const float scale = fmaxf(m, 1e-12f) / 127.0f;
    scales[j] = scale;
    for (size_t i = 0; i < k; ++i) {
        const float q = fminf(fmaxf(rintf(w[i * n + j] / scale), -127.0f), 127.0f);
        codes[i * n + j] = to_bits(q);
    }
}

// ---------------------------------------------------------------- convolution
// The causal convolution over [x | B | C] (nn/conv.rs:60-225, fused.rs:780-865)
// is computed where the prologue reads those channels: a token's workgroup
// reads the k rows ending at its own (its neighbours' rows, fetched by the
// neighbouring workgroups, come from L2), or the history for positions before
// the sequence start.  out[s, ch] = bias[ch] + sum_j w[j][ch] * in(s-(k-1)+j).
// The workgroup of a sequence's last position writes the new history, the
// last k-1 positions of history ++ input, after a barrier that ends every read
// of the old history in the workgroup: with one position per sequence that is
// every reader, so the history may be updated in place (the host allows
// aliasing only then).  Each channel's k-1 positions are copied by one thread
// in ascending order, which never reads a position it has already written.
__device__ __forceinline__ float xbc_at(const PrologueLaunch &a, const uint16_t *xbc_t, size_t s,
                                        size_t seqi, size_t C, size_t ch) {
    if (a.conv_k == 0) return bf(xbc_t, ch);
    const size_t k = a.conv_k;
    const uint16_t *hist = static_cast<const uint16_t *>(a.hist);
    float acc = a.conv_b ? a.conv_b[ch] : 0.0f;
    for (size_t j = 0; j < k; ++j) {
        const size_t back = k - 1 - j;                     // delay of tap j
        float v = 0.0f;
        if (back <= s) v = bf(xbc_t - back * a.width, ch);
        else if (hist) v = bf(hist, (seqi * (k - 1) + (k - 1 + s - back)) * C + ch);
        acc = __builtin_fmaf(a.conv_w[j * C + ch], v, acc);
    }
    return acc;
}

// The new history of sequence seqi, written by its last position's workgroup
// (xbc_t is that position's [x | B | C]); `vec` moves 16-byte vectors.
__device__ void write_history(const PrologueLaunch &a, const uint16_t *xbc_t, size_t seqi,
                              size_t C, bool vec) {
    __syncthreads();
    const size_t k = a.conv_k, T = a.seq_len;
    const uint16_t *hist = static_cast<const uint16_t *>(a.hist);
    uint16_t *nh = static_cast<uint16_t *>(a.new_hist) + seqi * (k - 1) * C;
    const uint16_t *oh = hist ? hist + seqi * (k - 1) * C : nullptr;
    const size_t step = vec ? 8 : 1;
    for (size_t ch = threadIdx.x * step; ch < C; ch += 256 * step) {
        for (size_t i = 0; i + 1 < k; ++i) {
            const size_t w = T + i;                        // window position
            const uint16_t *src = w < k - 1 ? (oh ? oh + w * C + ch : nullptr)
                                            : xbc_t - (T - 1 - (w - (k - 1))) * a.width + ch;
            if (vec) {
                const uint4 v = src ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
                *reinterpret_cast<uint4 *>(nh + i * C + ch) = v;
            } else {
                nh[i * C + ch] = src ? *src : uint16_t(0);
            }
        }
    }
}

// ---------------------------------------------------------------- prologue
// One workgroup per token.  The projection row is
//   [z | x | B | C | dt | lambda? | theta?]  (mamba3.rs:356-381)
// of widths d_inner, d_inner, G*R*N, G*R*N, H, H, H*N/2.  x, B and C pass
// through the convolution when there is one and then silu (mamba3.rs:386-396);
// B and C are broadcast from groups to heads (405-415), take the head's bias
// (418-423) and the RMSNorm over the state axis (424-427), and go out rank-last
// (429-431).  dt = softplus(dt + dt_bias) (435-438), lambda = sigmoid(lambda)
// or the fixed value (440-453).
__global__ void __launch_bounds__(256)
mixer_prologue_kernel(PrologueLaunch a) {
    const size_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const size_t H = a.heads, P = a.head_dim, N = a.d_state, R = a.rank, G = a.groups;
    const size_t din = H * P * R, bcw = G * R * N;
    const size_t C = din + 2 * bcw;
    const size_t pos = a.conv_k ? t % a.seq_len : 0, seqi = a.conv_k ? t / a.seq_len : 0;
    const uint16_t *row = static_cast<const uint16_t *>(a.projected) + t * a.width;
    const uint16_t *px = row + din;
    const uint16_t *pb = px + din;
    const uint16_t *pc = pb + bcw;
    const uint16_t *pdt = pc + bcw;
    const uint16_t *plam = pdt + H;
    const uint16_t *pth = plam + (a.learned_lambda ? H : 0);

    uint16_t *xo = static_cast<uint16_t *>(a.x) + t * din;
    for (size_t i = tid; i < din; i += 256) xo[i] = to_bits(siluf_(xbc_at(a, px, pos, seqi, C, i)));
    if (a.has_theta) {
        uint16_t *to = static_cast<uint16_t *>(a.theta) + t * H * (N / 2);
        for (size_t i = tid; i < H * (N / 2); i += 256) to[i] = pth[i];
    }
    for (size_t h = tid; h < H; h += 256) {
        a.dt[t * H + h] = softplusf_(bf(pdt, h) + a.dt_bias[h]);
        a.lambda[t * H + h] = a.learned_lambda ? sigmoidf_(bf(plam, h)) : a.fixed_lambda;
    }

    // B and C: one (head, rank) row of N per 16-lane group
    const size_t per_group = H / G;
    const int sub = tid & 15;
    const size_t nrows = H * R;
    for (int which = 0; which < 2; ++which) {
        const uint16_t *src = which ? pc : pb;
        const float *bias = which ? a.c_bias : a.b_bias;
        uint16_t *dst = static_cast<uint16_t *>(which ? a.c : a.b) + t * H * N * R;
        for (size_t rr = tid >> 4; rr < ((nrows + 15) / 16) * 16; rr += 16) {
            const bool live = rr < nrows;
            const size_t h = live ? rr / R : 0, r = live ? rr % R : 0;
            const size_t ch0 = static_cast<size_t>(src - px) + ((h / per_group) * R + r) * N;
            float ss = 0.0f;
            for (size_t n = sub; live && n < N; n += 16) {
                float v = siluf_(xbc_at(a, px, pos, seqi, C, ch0 + n));
                if (bias) v += bias[h * N + n];
                ss += v * v;
            }
            ss = group_sum(ss, 16);
            const float scale = a.bc_norm ? 1.0f / sqrtf(ss / static_cast<float>(N) + a.norm_eps) : 1.0f;
            for (size_t n = sub; live && n < N; n += 16) {
                float v = siluf_(xbc_at(a, px, pos, seqi, C, ch0 + n));
                if (bias) v += bias[h * N + n];
                if (a.bc_norm) v = v * scale * a.bc_norm[n];
                dst[(h * N + n) * R + r] = to_bits(v);
            }
        }
    }
    if (a.conv_k && a.new_hist && pos + 1 == a.seq_len) write_history(a, px, seqi, C, false);
}

// ---------------------------------------------------------------- prologue, 16-byte path
// The same prologue with every piece moved as 16-byte vectors of eight bf16.
// Needs d_state a multiple of 8 with d_state / 8 dividing 64, d_inner and the
// row width multiples of 8, a row width under 2^30 and H*N*R under 2^31 (the
// per-item offsets are 32-bit), and 16-byte aligned buffers (the host checks).
// Then theta's offset in the row, 2*d_inner + 2*G*R*N + H or 2H, is a multiple
// of 8 as well: the width is that offset plus H*N/2, which is 0 or 4 mod 8
// (4 only for odd H), and H or 2H is never 4 mod 8 for odd H.
// One workgroup per token walks a flat list of vector items:
//   [0, 2*H*lq)        B then C: head h, state lanes q = 0..lq-1 (lq = N/8),
//                      each lane holding eight states of every rank;
//   [.., + din/8)      x;
//   [.., + H*N/16)     theta, copied.
// A (B|C, head) row's lq lanes are consecutive and lq-aligned, so the RMSNorm
// sum over the state axis is a reduction over those lanes.  The rank-last
// output of a lane is the 8 x R block of states q*8.. of all ranks: R whole
// vectors.  silu is silu_fast (mixer_math.hpp).

// Eight channels ch..ch+7 of [x | B | C] at a token (xbc_t its row's [x | B |
// C]), through the convolution when CONV (see xbc_at).  The branch on the
// position is uniform over the workgroup.
template <bool CONV>
__device__ __forceinline__ void xbc8(const PrologueLaunch &a, const uint16_t *xbc_t, size_t s,
                                     size_t seqi, size_t C, size_t ch, float *f) {
    if (!CONV) {
        unpack8(*reinterpret_cast<const uint4 *>(xbc_t + ch), f);
        return;
    }
    const size_t k = a.conv_k;
    const uint16_t *hist = static_cast<const uint16_t *>(a.hist);
    conv_taps8(a.conv_w, a.conv_b, C, k, ch, [&](size_t j) -> const uint16_t * {
        const size_t back = k - 1 - j;
        return back <= s ? xbc_t - back * a.width + ch
               : hist ? hist + (seqi * (k - 1) + (k - 1 + s - back)) * C + ch : nullptr;
    }, f);
}

template <int R, bool CONV>
__global__ void __launch_bounds__(256)
mixer_prologue_vec_kernel(PrologueLaunch a, int lq, int per_group, float inv_n) {
    const size_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const int H = static_cast<int>(a.heads), N = static_cast<int>(a.d_state);
    const int din = static_cast<int>(a.heads * a.head_dim) * R;
    const int bcw = static_cast<int>(a.groups) * R * N;
    const size_t C = static_cast<size_t>(din) + 2 * static_cast<size_t>(bcw);
    const size_t pos = CONV ? t % a.seq_len : 0, seqi = CONV ? t / a.seq_len : 0;
    const uint16_t *__restrict__ row = static_cast<const uint16_t *>(a.projected) + t * a.width;
    const uint16_t *px = row + din;
    const uint16_t *pdt = px + C;
    const uint16_t *plam = pdt + H;
    const uint16_t *pth = plam + (a.learned_lambda ? H : 0);
    // This token's output rows; every per-item offset below is a 32-bit
    // element offset from these (the row width is under 2^30, checked on the
    // host), so the item loop does no 64-bit index arithmetic.
    const size_t bc_row = static_cast<size_t>(H) * N * R;
    uint16_t *ob = static_cast<uint16_t *>(a.b) + t * bc_row;
    uint16_t *oc = static_cast<uint16_t *>(a.c) + t * bc_row;
    uint16_t *ox = static_cast<uint16_t *>(a.x) + t * static_cast<size_t>(din);
    const int nbc = 2 * H * lq;
    const int lq_sh = __builtin_ctz(static_cast<unsigned>(lq));   // lq is a power of two
    const int nx = din / 8;
    const int thw = a.has_theta ? H * (N / 2) : 0;
    const int total = nbc + nx + thw / 8;

    for (int i = tid; i < total; i += 256) {
        if (i < nbc) {
            const int u = i >> lq_sh, q = i & (lq - 1);
            const int which = u >= H ? 1 : 0;
            const int h = u - which * H;
            const int hg = per_group == 1 ? h : h / per_group;
            // channel of state q*8, rank 0, within [x | B | C]
            const unsigned ch0 = static_cast<unsigned>(din + which * bcw + (hg * R * N + q * 8));
            const float *bias = which ? a.c_bias : a.b_bias;
            float v[R][8];
#pragma unroll
            for (int r = 0; r < R; ++r) xbc8<CONV>(a, px, pos, seqi, C, ch0 + r * N, v[r]);
            float bb[8], w[8];
            const unsigned el = static_cast<unsigned>(h * N + q * 8);   // [H, N] element
            if (bias) {
                const float4 b0 = *reinterpret_cast<const float4 *>(bias + el);
                const float4 b1 = *reinterpret_cast<const float4 *>(bias + el + 4);
                bb[0] = b0.x; bb[1] = b0.y; bb[2] = b0.z; bb[3] = b0.w;
                bb[4] = b1.x; bb[5] = b1.y; bb[6] = b1.z; bb[7] = b1.w;
            }
            if (a.bc_norm) {
                const float4 w0 = *reinterpret_cast<const float4 *>(a.bc_norm + q * 8);
                const float4 w1 = *reinterpret_cast<const float4 *>(a.bc_norm + q * 8 + 4);
                w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
                w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
            }
            bc_row8<R>(v, bb, bias != nullptr, w, a.bc_norm != nullptr, lq, inv_n, a.norm_eps);
            uint4 *dst = reinterpret_cast<uint4 *>((which ? oc : ob) + el * R);
#pragma unroll
            for (int k = 0; k < R; ++k) {
                unsigned int o[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int e0 = 8 * k + 2 * m, e1 = e0 + 1;     // element e = j * R + r
                    o[m] = pack2(v[e0 % R][e0 / R], v[e1 % R][e1 / R]);
                }
                dst[k] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else if (i < nbc + nx) {
            const unsigned k = static_cast<unsigned>(i - nbc);
            float f[8];
            xbc8<CONV>(a, px, pos, seqi, C, k * 8, f);
            *reinterpret_cast<uint4 *>(ox + k * 8) =
                make_uint4(pack2(silu_fast(f[0]), silu_fast(f[1])), pack2(silu_fast(f[2]), silu_fast(f[3])),
                           pack2(silu_fast(f[4]), silu_fast(f[5])), pack2(silu_fast(f[6]), silu_fast(f[7])));
        } else {
            const unsigned k = static_cast<unsigned>(i - nbc - nx) * 8;
            uint16_t *to = static_cast<uint16_t *>(a.theta) + t * thw;
            *reinterpret_cast<uint4 *>(to + k) = *reinterpret_cast<const uint4 *>(pth + k);
        }
    }
    for (int h = tid; h < H; h += 256) {
        a.dt[t * H + h] = softplusf_(bf(pdt, h) + a.dt_bias[h]);
        a.lambda[t * H + h] = a.learned_lambda ? sigmoidf_(bf(plam, h)) : a.fixed_lambda;
    }
    if (CONV && a.new_hist && pos + 1 == a.seq_len) write_history(a, px, seqi, C, true);
}

// ---------------------------------------------------------------- gate
// out = [RMSNorm(y)] * silu(z) over rows of d_inner (mamba3.rs:468-477); one
// wave per token.  silu is silu_fast here as in the vector kernel and the
// gate fused into the scan's output kernel, so every path rounds alike.
__global__ void __launch_bounds__(256)
mixer_gate_kernel(size_t tokens, size_t d, const uint16_t *y, const uint16_t *z, size_t zs,
                  const float *nw, float eps, uint16_t *out) {
    const size_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens) return;
    const uint16_t *yr = y + t * d;
    const uint16_t *zr = z + t * zs;
    uint16_t *orow = out + t * d;
    float scale = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (size_t i = lane; i < d; i += 64) {
            const float v = bf(yr, i);
            ss += v * v;
        }
        ss = group_sum(ss, 64);
        scale = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    }
    for (size_t i = lane; i < d; i += 64) {
        float v = bf(yr, i);
        if (nw) v = v * scale * nw[i];
        orow[i] = to_bits(v * silu_fast(bf(zr, i)));
    }
}

// The gate with 16-byte vectors: d_inner and the z stride multiples of 8,
// 16-byte aligned buffers (the host checks).  One wave per token.
__global__ void __launch_bounds__(256)
mixer_gate_vec_kernel(size_t tokens, size_t d, const uint16_t *y, const uint16_t *z, size_t zs,
                      const float *nw, float eps, uint16_t *out) {
    const size_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens) return;
    const uint16_t *yr = y + t * d;
    const uint16_t *zr = z + t * zs;
    uint16_t *orow = out + t * d;
    float scale = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (size_t i = lane * 8; i < d; i += 512) {
            float f[8];
            unpack8(*reinterpret_cast<const uint4 *>(yr + i), f);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
        }
        ss = group_sum(ss, 64);
        scale = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    }
    for (size_t i = lane * 8; i < d; i += 512) {
        float f[8], g[8];
        unpack8(*reinterpret_cast<const uint4 *>(yr + i), f);
        unpack8(*reinterpret_cast<const uint4 *>(zr + i), g);
        if (nw) {
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] * scale * nw[i + j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= silu_fast(g[j]);
        *reinterpret_cast<uint4 *>(orow + i) =
            make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
    }
}

// ---------------------------------------------------------------- embedding
// An id outside [0, vocab) reads nothing and yields a zero row.
__global__ void __launch_bounds__(256)
embedding_kernel(size_t n, size_t dim, const int32_t *ids, size_t vocab, const uint16_t *table,
                 uint16_t *out) {
    const size_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const int32_t id = ids[r];
    uint16_t *dst = out + r * dim;
    if (id < 0 || static_cast<size_t>(id) >= vocab) {
        for (size_t i = lane; i < dim; i += 64) dst[i] = 0;
        return;
    }
    const uint16_t *src = table + static_cast<size_t>(id) * dim;
    if (dim % 8 == 0) {
        for (size_t i = lane * 8; i < dim; i += 512)
            *reinterpret_cast<uint4 *>(dst + i) = *reinterpret_cast<const uint4 *>(src + i);
    } else {
        for (size_t i = lane; i < dim; i += 64) dst[i] = src[i];
    }
}

unsigned int blocks(size_t n, size_t per) { return static_cast<unsigned int>((n + per - 1) / per); }

}  // namespace

hipError_t launch_rms_norm(size_t rows, size_t dim, const void *x, size_t x_stride, const float *w,
                           float eps, void *y, size_t y_stride, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(blocks(rows, 4)), dim3(256), 0, s, rows, dim,
                       static_cast<const uint16_t *>(x), x_stride, w, eps, static_cast<uint16_t *>(y),
                       y_stride);
    return hipGetLastError();
}

hipError_t launch_quantize_columns(size_t k, size_t n, const float *w, void *codes, float *scales,
                                   hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_columns_kernel, dim3(blocks(n, 256)), dim3(256), 0, s, k, n, w,
                       static_cast<uint16_t *>(codes), scales);
    return hipGetLastError();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipError_t launch_mixer_prologue(const PrologueLaunch &a, hipStream_t s) {
    if (a.tokens == 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned int>(a.tokens));
    const size_t N = a.d_state, din = a.heads * a.head_dim * a.rank;
    const size_t lq = N / 8;
    const bool vec = N % 8 == 0 && lq >= 1 && lq <= 64 && (lq & (lq - 1)) == 0 && din % 8 == 0 &&
                     a.width % 8 == 0 && (a.rank == 1 || a.rank == 2 || a.rank == 4) &&
                     aligned16(a.projected) && aligned16(a.x) && aligned16(a.b) && aligned16(a.c) &&
                     aligned16(a.b_bias) && aligned16(a.c_bias) && aligned16(a.bc_norm) &&
                     aligned16(a.theta) && a.width < (1u << 30) && a.heads * N * a.rank < (1u << 31) &&
                     aligned16(a.conv_w) &&
                     aligned16(a.conv_b) && aligned16(a.hist) && aligned16(a.new_hist);
    if (!vec) {
        hipLaunchKernelGGL(mixer_prologue_kernel, grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const int l = static_cast<int>(lq), pg = static_cast<int>(a.heads / a.groups);
    const float inv_n = 1.0f / static_cast<float>(N);   // rounded as the kernels' 1.0f / N
    const bool conv = a.conv_k != 0;
    void (*kernel)(PrologueLaunch, int, int, float);
    switch (a.rank) {
    case 1: kernel = conv ? mixer_prologue_vec_kernel<1, true> : mixer_prologue_vec_kernel<1, false>; break;
    case 2: kernel = conv ? mixer_prologue_vec_kernel<2, true> : mixer_prologue_vec_kernel<2, false>; break;
    default: kernel = conv ? mixer_prologue_vec_kernel<4, true> : mixer_prologue_vec_kernel<4, false>; break;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, a, l, pg, inv_n);
    return hipGetLastError();
}

hipError_t launch_mixer_gate(size_t tokens, size_t d_inner, const void *y, const void *z,
                             size_t z_stride, const float *norm_w, float eps, void *out,
                             hipStream_t s) {
    if (tokens == 0) return hipSuccess;
    if (d_inner % 8 == 0 && z_stride % 8 == 0 && aligned16(y) && aligned16(z) && aligned16(out) &&
        aligned16(norm_w)) {
        hipLaunchKernelGGL(mixer_gate_vec_kernel, dim3(blocks(tokens, 4)), dim3(256), 0, s, tokens,
                           d_inner, static_cast<const uint16_t *>(y), static_cast<const uint16_t *>(z),
                           z_stride, norm_w, eps, static_cast<uint16_t *>(out));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(mixer_gate_kernel, dim3(blocks(tokens, 4)), dim3(256), 0, s, tokens, d_inner,
                       static_cast<const uint16_t *>(y), static_cast<const uint16_t *>(z), z_stride,
                       norm_w, eps, static_cast<uint16_t *>(out));
    return hipGetLastError();
}

hipError_t launch_embedding(size_t n, size_t dim, const int32_t *ids, size_t vocab, const void *table,
                            void *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(embedding_kernel, dim3(blocks(n, 4)), dim3(256), 0, s, n, dim, ids, vocab,
                       static_cast<const uint16_t *>(table), static_cast<uint16_t *>(out));
    return hipGetLastError();
}

}  // namespace m3
