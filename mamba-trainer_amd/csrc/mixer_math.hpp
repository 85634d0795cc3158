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

__device__ __forceinline__ unsigned int pack2(float a, float b) {
    return static_cast<unsigned int>(to_bits(a)) | (static_cast<unsigned int>(to_bits(b)) << 16);
}

// Eight states q*8 .. q*8+7 of every rank of one (B | C, head) row after the
// silu (v holds the pre-silu values in, the final ones out): + bias8 (when
// has_bias), then the RMSNorm over the state axis with gain w8 (when
// has_norm), the sum over the row's lq lanes (lq consecutive lanes,
// lq-aligned, a power of two; models/mamba3.rs:405-427).
template <int R>
__device__ __forceinline__ void bc_row8(float (&v)[R][8], const float (&bias8)[8], bool has_bias,
                                        const float (&w8)[8], bool has_norm, int lq, int n_state,
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
            ss = group_sum(ss, lq);
            const float scale = 1.0f / sqrtf(ss / static_cast<float>(n_state) + eps);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[r][j] = v[r][j] * scale * w8[j];
        }
    }
}

}  // namespace mixm
}  // namespace m3
