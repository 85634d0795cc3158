// Device-side helpers shared by the gfx950 kernels: storage conversions,
// MFMA wrappers with their lane layouts, and wave-level collectives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace m3 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// bf16 storage is raw 16-bit words; widening is a shift, narrowing rounds to
// nearest-even (v_cvt_pk_bf16_f32 on gfx950).
struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
    __bf16 h = static_cast<__bf16>(v);
    bf16_t r;
    r.bits = __builtin_bit_cast(uint16_t, h);
    return r;
}

__device__ __forceinline__ __bf16 to_bf16(float v) { return static_cast<__bf16>(v); }

// Two values rounded to bf16 (nearest-even) by one v_cvt_pk_bf16_f32, lo in
// bits 0-15: the same rounding as two from_f32<bf16_t> calls, in one
// instruction instead of two conversions, a shift and an or.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2 f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// ---------------------------------------------------------------------------
// MFMA.  Both variants compute a 16x16 f32 tile D += A(16xK) * B(Kx16).
// Lane l of the wave, g = l / 16, c = l % 16:
//   A operand: row c, k-slots owned by lane group g
//   B operand: column c, the same k-slots
//   D: column c, rows 4g + r for r = 0..3 (element r of the f32x4)
// bf16 16x16x32: lane group g owns k = 8g .. 8g+7 (eight bf16 per lane).
// f32  16x16x4 : lane group g owns k = g (one f32 per lane).
// Any permutation of k is valid as long as A and B use the same one; the
// kernels exploit this to feed accumulators straight back in as operands.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Wave-level (64-lane) collectives.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_inclusive_scan(float v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        float o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

// Inclusive scan over each aligned segment of SW lanes (SW = 16, 32 or 64):
// DPP row_shr steps within 16-lane rows, then row_bcast:15 / row_bcast:31
// carries across rows.  Lanes whose shifted source falls outside the row
// read zero (bound_ctrl).  Each carry is one in-place DPP add under a row
// mask (rows outside it keep their value), written out because the compiler
// otherwise moves the broadcast into a zeroed temporary and adds it: three
// instructions.  The s_nop 1 gives the two wait states a DPP read of a VGPR
// that the previous VALU instruction wrote needs.
template <int CTRL, int ROWM, bool BC>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWM, 0xf, BC));
}
template <int SW>
__device__ __forceinline__ float seg_scan(float v) {
    static_assert(SW == 16 || SW == 32 || SW == 64, "segments of 16, 32 or 64 lanes");
    v += dpp_f<0x111, 0xf, true>(v);   // row_shr:1
    v += dpp_f<0x112, 0xf, true>(v);   // row_shr:2
    v += dpp_f<0x114, 0xf, true>(v);   // row_shr:4
    v += dpp_f<0x118, 0xf, true>(v);   // row_shr:8
    if constexpr (SW == 32)   // row_bcast:15 -> rows 1, 3
        asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf"
            : "+v"(v));
    if constexpr (SW == 64)   // then row_bcast:31 -> rows 2, 3
        asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
            "s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf"
            : "+v"(v));
    return v;
}

// Four independent seg_scans, interleaved step by step in one block: each
// DPP add then reads a value written three instructions earlier, past the two
// wait states it needs, so a single s_nop serves the four chains (the
// compiler schedules DPP chains one after another, a nop between steps).
#define M3_DPP4(CTRL)                                                                 \
    "v_add_f32_dpp %0, %0, %0 " CTRL "\n\tv_add_f32_dpp %1, %1, %1 " CTRL "\n\t"     \
    "v_add_f32_dpp %2, %2, %2 " CTRL "\n\tv_add_f32_dpp %3, %3, %3 " CTRL "\n\t"
#define M3_SHR(n) "row_shr:" #n " row_mask:0xf bank_mask:0xf bound_ctrl:1"
#define M3_BC15 "row_bcast:15 row_mask:0xa bank_mask:0xf"
#define M3_BC31 "row_bcast:31 row_mask:0xc bank_mask:0xf"
template <int SW>
__device__ __forceinline__ void seg_scan4(float &a, float &b, float &c, float &d) {
    static_assert(SW == 16 || SW == 32 || SW == 64, "segments of 16, 32 or 64 lanes");
    if constexpr (SW == 16)
        asm("s_nop 1\n\t" M3_DPP4(M3_SHR(1)) M3_DPP4(M3_SHR(2)) M3_DPP4(M3_SHR(4))
                M3_DPP4(M3_SHR(8))
            : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
    if constexpr (SW == 32)
        asm("s_nop 1\n\t" M3_DPP4(M3_SHR(1)) M3_DPP4(M3_SHR(2)) M3_DPP4(M3_SHR(4))
                M3_DPP4(M3_SHR(8)) M3_DPP4(M3_BC15)
            : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
    if constexpr (SW == 64)
        asm("s_nop 1\n\t" M3_DPP4(M3_SHR(1)) M3_DPP4(M3_SHR(2)) M3_DPP4(M3_SHR(4))
                M3_DPP4(M3_SHR(8)) M3_DPP4(M3_BC15) M3_DPP4(M3_BC31)
            : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
#undef M3_DPP4
#undef M3_SHR
#undef M3_BC15
#undef M3_BC31

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Wrap an angle into [-pi, pi] by subtracting whole turns, as
// x - round(x / 2pi) * 2pi (the reference's wrap, elemwise.rs:349).
__device__ __forceinline__ float wrap_angle(float x) {
    const float two_pi = 6.28318530717958647692f;
    return x - rintf(x * 0.15915494309189533577f) * two_pi;
}

// exp(clamp(d, -60, 0)): the scan's decay factor with its log floor.
__device__ __forceinline__ float decay_exp(float d) {
    d = fminf(fmaxf(d, -60.0f), 0.0f);
    return expf(d);
}

// ---------------------------------------------------------------------------
// Buffer resources.  A raw buffer load at or past `bytes` returns zeros and a
// store there is dropped (the hardware range check), so padding tokens at the
// end of a sequence need no branches -- and a load sequence without branches
// lets the compiler wait for exactly the loads a value depends on.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    // dword3 0x00020000: 32-bit data format, the gfx9-family raw-buffer setting
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 bld16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 bld8(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bld4(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ float bldf(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void bst16(u32x4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
__device__ __forceinline__ void bst8(u32x2 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}
__device__ __forceinline__ void bst4(uint32_t v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ __forceinline__ void bst2(uint16_t v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}

}  // namespace m3
