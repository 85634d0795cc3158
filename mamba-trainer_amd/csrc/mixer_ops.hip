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

namespace m3 {

namespace {

__device__ __forceinline__ float bf(const uint16_t *p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ uint16_t to_bits(float v) { return from_f32<bf16_t>(v).bits; }
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
// max(x, 0) + ln(1 + exp(-|x|))  (fused.rs:1291-1293)
__device__ __forceinline__ float softplusf_(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

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
                o[j] = static_cast<unsigned int>(to_bits(a)) | (static_cast<unsigned int>(to_bits(b)) << 16);
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

// ---------------------------------------------------------------- prologue
// One workgroup per token.  The projection row is
//   [z | x | B | C | dt | lambda? | theta?]  (mamba3.rs:356-381)
// of widths d_inner, d_inner, G*R*N, G*R*N, H, H, H*N/2.  x, B and C pass
// through silu (mamba3.rs:396); B and C are broadcast from groups to heads
// (405-415), take the head's bias (418-423) and the RMSNorm over the state axis
// (424-427), and go out rank-last (429-431).  dt = softplus(dt + dt_bias)
// (435-438), lambda = sigmoid(lambda) or the fixed value (440-453).
__global__ void __launch_bounds__(256)
mixer_prologue_kernel(PrologueLaunch a) {
    const size_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const size_t H = a.heads, P = a.head_dim, N = a.d_state, R = a.rank, G = a.groups;
    const size_t din = H * P * R, bcw = G * R * N;
    const uint16_t *row = static_cast<const uint16_t *>(a.projected) + t * a.width;
    const uint16_t *px = row + din;
    const uint16_t *pb = px + din;
    const uint16_t *pc = pb + bcw;
    const uint16_t *pdt = pc + bcw;
    const uint16_t *plam = pdt + H;
    const uint16_t *pth = plam + (a.learned_lambda ? H : 0);

    uint16_t *xo = static_cast<uint16_t *>(a.x) + t * din;
    for (size_t i = tid; i < din; i += 256) xo[i] = to_bits(siluf_(bf(px, i)));
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
            const uint16_t *s = src + ((h / per_group) * R + r) * N;
            float ss = 0.0f;
            for (size_t n = sub; live && n < N; n += 16) {
                float v = siluf_(bf(s, n));
                if (bias) v += bias[h * N + n];
                ss += v * v;
            }
            ss = group_sum(ss, 16);
            const float scale = a.bc_norm ? 1.0f / sqrtf(ss / static_cast<float>(N) + a.norm_eps) : 1.0f;
            for (size_t n = sub; live && n < N; n += 16) {
                float v = siluf_(bf(s, n));
                if (bias) v += bias[h * N + n];
                if (a.bc_norm) v = v * scale * a.bc_norm[n];
                dst[(h * N + n) * R + r] = to_bits(v);
            }
        }
    }
}

// ---------------------------------------------------------------- gate
// out = [RMSNorm(y)] * silu(z) over rows of d_inner (mamba3.rs:468-477); one
// wave per token.
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
        orow[i] = to_bits(v * siluf_(bf(zr, i)));
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

hipError_t launch_mixer_prologue(const PrologueLaunch &a, hipStream_t s) {
    if (a.tokens == 0) return hipSuccess;
    hipLaunchKernelGGL(mixer_prologue_kernel, dim3(static_cast<unsigned int>(a.tokens)), dim3(256), 0, s,
                       a);
    return hipGetLastError();
}

hipError_t launch_mixer_gate(size_t tokens, size_t d_inner, const void *y, const void *z,
                             size_t z_stride, const float *norm_w, float eps, void *out,
                             hipStream_t s) {
    if (tokens == 0) return hipSuccess;
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
