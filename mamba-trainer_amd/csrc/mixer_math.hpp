// Element-wise pieces of the Mamba-3 mixer's projection prologue and gate
// (models/mamba3.rs:376-477), shared by the token-parallel kernels
// (mixer_ops.hip) and the fused decode step (decode_step.hip), so that both
// round every value the same way.
#pragma once

#include "m3_device.hpp"

namespace m3 {
namespace mixm {

__device__ __forceinline__ float bf(const uint16_t *p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ uint16_t to_bits(float v) { return from_f32<bf16_t>(v).bits; }
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
// max(x, 0) + ln(1 + exp(-|x|))  (fused.rs:1291-1293)
__device__ __forceinline__ float softplusf_(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

// silu with exp(-v) = 2^(-v log2 e) on v_exp_f32 and v_rcp_f32, within a few
// f32 ulps of the exact value, below bf16 rounding.
__device__ __forceinline__ float silu_fast(float v) {
    const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ void unpack8(const uint4 q, float *f) {
    const unsigned int u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(u[j] << 16);
        f[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ unsigned int pack2(float a, float b) { return pack_bf16x2(a, b); }

// Eight channels ch .. ch+7 of the depthwise causal convolution at one
// position (nn/conv.rs:60-225, fused.rs:780-832): f = bias + sum_j w[j] x_j
// over taps j = 0 .. k-1 in ascending order, one fused multiply-add each, so
// that every kernel computing it rounds alike.  `tap(j)` gives tap j's eight
// bf16 inputs (the position k-1-j before this one), or null for a position
// before the sequence with no history (the tap is skipped).  w is the
// [k, C] f32 weight, bias [C] or null.
template <typename Tap>
__device__ __forceinline__ void conv_taps8(const float *w, const float *bias, size_t C, size_t k,
                                           size_t ch, Tap tap, float *f) {
    if (bias) {
        const float4 b0 = *reinterpret_cast<const float4 *>(bias + ch);
        const float4 b1 = *reinterpret_cast<const float4 *>(bias + ch + 4);
        f[0] = b0.x; f[1] = b0.y; f[2] = b0.z; f[3] = b0.w;
        f[4] = b1.x; f[5] = b1.y; f[6] = b1.z; f[7] = b1.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = 0.0f;
    }
    for (size_t j = 0; j < k; ++j) {
        const uint16_t *src = tap(j);
        if (src == nullptr) continue;
        float v[8];
        unpack8(*reinterpret_cast<const uint4 *>(src), v);
        const float4 w0 = *reinterpret_cast<const float4 *>(w + j * C + ch);
        const float4 w1 = *reinterpret_cast<const float4 *>(w + j * C + ch + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = __builtin_fmaf(wv[e], v[e], f[e]);
    }
}

// Eight states q*8 .. q*8+7 of every rank of one (B | C, head) row after the
// silu (v holds the pre-silu values in, the final ones out): + bias8 (when
// has_bias), then the RMSNorm over the state axis with gain w8 (when
// has_norm), the sum over the row's lq lanes (lq consecutive lanes,
// lq-aligned, a power of two, all active; models/mamba3.rs:405-427); inv_n is
// 1 / d_state rounded to f32, the mean a multiply.  Rows of
// 8 or 16 lanes sum through DPP inside their 16-lane row (no LDS crossbar),
// and the scale is v_rsq_f32 of mean + eps (within an ulp of 1 / sqrt): the
// prologue kernel was bound by its instruction issue, not by its bytes.
template <int R>
__device__ __forceinline__ void bc_row8(float (&v)[R][8], const float (&bias8)[8], bool has_bias,
                                        const float (&w8)[8], bool has_norm, int lq, float inv_n,
                                        float eps) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) v[r][j] = silu_fast(v[r][j]) + (has_bias ? bias8[j] : 0.0f);
    if (has_norm) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += v[r][j] * v[r][j];
            if (lq == 16 || lq == 8) {
                // within a 16-lane DPP row: xor 1, xor 2 (quad_perm), then the
                // half-row mirror (8 lanes) and, for 16, the row mirror
                ss += dpp_f<0xB1, 0xf, false>(ss);
                ss += dpp_f<0x4E, 0xf, false>(ss);
                ss += dpp_f<0x141, 0xf, false>(ss);
                if (lq == 16) ss += dpp_f<0x140, 0xf, false>(ss);
            } else {
                ss = group_sum(ss, lq);
            }
            const float scale = __builtin_amdgcn_rsqf(ss * inv_n + eps);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[r][j] = v[r][j] * scale * w8[j];
        }
    }
}

}  // namespace mixm
}  // namespace m3
