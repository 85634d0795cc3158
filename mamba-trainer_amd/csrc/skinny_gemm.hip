// Linear::apply for few rows (the decode step's projections: one token per
// sequence, a few hundred rows) on gfx950:
//   y[m, n] = (x[m, :] . w[:, n]) * scale[n] + res[m, n]
// bf16 x [M, K] and w [K, N] (row-major, as nn/linear.rs:155-185 stores the
// weight) or its transpose w^T [N, K] (WT; the int8 projections hold their
// codes, whole numbers exact in bf16), f32 accumulation, the per-column scale
// and the residual in the epilogue, bf16 y.
//
// With M this small the product is a stream over the weights: every weight
// is read once, and x (M x K, under 1 MB) is re-read from L2 by each column
// block.  A workgroup owns a BN x BM block of y^T and walks K in steps of
// 128: each step's x and w tiles come in by direct-to-LDS buffer loads
// (16 bytes a lane, whole rows, the permuted-chunk tiles of scan_common.hpp)
// NS steps ahead, and y^T = W^T X^T is formed by bf16 MFMA 16x16x32 with the
// W^T operand read transposed (ds_read_b64_tr_b16) from the row-major w tile
// and the X^T operand read straight from x's rows (with WT both operands are
// row reads: w^T's tile is [n][k] like x's).  The y^T accumulator
// layout gives each lane four consecutive columns of one row: 8-byte stores.
#include "m3_internal.hpp"
#include "scan_common.hpp"

namespace m3 {

namespace {

using namespace scan;

constexpr int kKStep = 128;    // k per pipeline stage
constexpr int kStages = 3;     // stages in flight
// The block of y^T a workgroup owns: swept on MI355X at 256 rows (us per
// call, K = 1536; BM x BN / k-step / stages): N = 1536: 64x32/128/3 7.7,
// 32x32/64/4 7.8, 64x32/64/4 8.8, 64x64/128/2 9.6, 128x64/64/3 16.5, against
// hipBLASLt's 11-17 depending on its plan.  At N = 10800 the best block
// (128x64/64/3) took 24.1 against hipBLASLt's 22.5: x's re-reads from L2 grow
// with the column blocks, so wide products stay on hipBLASLt.
constexpr int kBM = 64, kBN = 32;

template <int BM, int BN, bool WT>
struct GemmSmem {
    static constexpr int CX = kKStep * 2 / 16;   // 16-byte chunks per x row
    static constexpr int CW = WT ? CX : BN * 2 / 16;   // ... per w row
    static constexpr int RW = WT ? BN : kKStep;        // w tile rows
    unsigned char x[kStages][BM * CX * 16];      // [m][k]
    unsigned char w[kStages][RW * CW * 16];      // [k][n], or [n][k] (WT)
};

template <int V>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<V>());
}

template <int BM, int BN, bool WT>
__global__ void __launch_bounds__(kThreads, 2)
skinny_gemm_kernel(uint32_t M, uint32_t K, uint32_t N, const void *x, const void *w,
                   const float *scale, const void *res, void *y) {
    using S = GemmSmem<BM, BN, WT>;
    constexpr int CX = S::CX, CW = S::CW;
    constexpr int NTW = BN / 32, MTW = BM / 32;          // 16-wide tiles per wave (2 x 2 waves)
    constexpr int LX = BM * CX / 64 / 4, LW = S::RW * CW / 64 / 4;   // loads per wave per stage
    constexpr int LPS = LX + LW;
    static_assert(LX >= 1 && LW >= 1 && BM * CX % 256 == 0 && S::RW * CW % 256 == 0,
                  "tiles in whole kilobytes per wave");

    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int g = lane >> 4, c = lane & 15;
    const uint32_t n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;

    const rsrc_t rx = make_rsrc(x, M * K * 2u);
    // w's columns from n0 on (rows past the end read as zeros); w^T whole
    const rsrc_t rw = WT ? make_rsrc(w, N * K * 2u)
                         : make_rsrc(static_cast<const char *>(w) + static_cast<size_t>(n0) * 2,
                                     (K * N - n0) * 2u);
    const int steps = static_cast<int>(K / kKStep);
    auto load = [&](int s) {
        const int b = s % kStages;
        const uint32_t k0 = static_cast<uint32_t>(s) * kKStep;
#pragma unroll
        for (int q = 0; q < LX; ++q)
            lds_load_rows<CX>(rx, (m0 * K + k0) * 2u, K * 2u, sm.x[b], wave + 4 * q, lane);
#pragma unroll
        for (int q = 0; q < LW; ++q) {
            if constexpr (WT)
                lds_load_rows<CW>(rw, (n0 * K + k0) * 2u, K * 2u, sm.w[b], wave + 4 * q, lane);
            else
                lds_load_rows<CW>(rw, k0 * N * 2u, N * 2u, sm.w[b], wave + 4 * q, lane);
        }
    };

    f32x4 acc[NTW][MTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int j = 0; j < MTW; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        if (s < steps) load(s);
#pragma unroll 1
    for (int s = 0; s < steps; ++s) {
        if (s + kStages - 1 < steps) load(s + kStages - 1);
        // stage s landed: the stages issued after it may still be out
        const int after = min(kStages - 1, steps - 1 - s);
        static_assert(kStages == 3, "the counted waits below cover three stages");
        if (after >= 2)
            wait_vm<2 * LPS>();
        else if (after == 1)
            wait_vm<LPS>();
        else
            wait_vm<0>();
        __syncthreads();
        const int b = s % kStages;
        const unsigned char *xt = sm.x[b];
        const unsigned char *wt = sm.w[b];
        const int r0 = 8 * g + (c >> 2);
#pragma unroll
        for (int kb = 0; kb < kKStep / 32; ++kb) {
            // W^T[n][k], k = 32 kb + 8 g + 0..7: row n of w^T's tile, or
            // column n of w's (transposed reads)
            bf16x8 af[NTW];
#pragma unroll
            for (int i = 0; i < NTW; ++i) {
                if constexpr (WT) {
                    af[i] = *reinterpret_cast<const bf16x8 *>(wt + rtile_off<CW>(16 * (NTW * wn + i) + c, 32 * kb + 8 * g));
                } else {
                    const int col = 16 * (NTW * wn + i) + 4 * (c & 3);
                    const bf16x4 lo = lds_read_tr16(reinterpret_cast<const __bf16 *>(wt + rtile_off<CW>(32 * kb + r0, col)));
                    const bf16x4 hi = lds_read_tr16(reinterpret_cast<const __bf16 *>(wt + rtile_off<CW>(32 * kb + r0 + 4, col)));
                    af[i] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
            // X^T[k][m]: row m of the x tile, the same k
            bf16x8 bfr[MTW];
#pragma unroll
            for (int j = 0; j < MTW; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(xt + rtile_off<CX>(16 * (MTW * wm + j) + c, 32 * kb + 8 * g));
#pragma unroll
            for (int i = 0; i < NTW; ++i)
#pragma unroll
                for (int j = 0; j < MTW; ++j) acc[i][j] = mfma_bf16(af[i], bfr[j], acc[i][j]);
        }
        __syncthreads();   // every read of this stage's tiles is done before they are reloaded
    }

    // ---- epilogue: lane (c, g) of tile (i, j) holds y[m][n .. n + 3],
    //      m = m0 + 16 (MTW wm + j) + c, n = n0 + 16 (NTW wn + i) + 4 g
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
        const uint32_t n = n0 + 16 * (NTW * wn + i) + 4 * g;
        if (n >= N) continue;
        f32x4 sc = f32x4{1.f, 1.f, 1.f, 1.f};
        if (scale) sc = *reinterpret_cast<const f32x4 *>(scale + n);
#pragma unroll
        for (int j = 0; j < MTW; ++j) {
            const uint32_t m = m0 + 16 * (MTW * wm + j) + c;
            if (m >= M) continue;
            const size_t o = static_cast<size_t>(m) * N + n;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] * sc[r];
            if (res) {
                const u32x2 rv = *reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(res) + o);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t wd = rv[r >> 1];
                    v[r] += __uint_as_float((r & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
                }
            }
            u32x2 pk;
            pk[0] = pack_bf16x2(v[0], v[1]);
            pk[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(y) + o) = pk;
        }
    }
}

}  // namespace

bool skinny_gemm_supported(size_t m, size_t k, size_t n, const void *x, const void *w,
                           const float *scale, const void *res, const void *y) {
    auto al16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return m >= 1 && m <= 512 && k >= kKStep && k % kKStep == 0 && n % 8 == 0 && n >= 32 &&
           n < 4096 &&
           k * n * 2 < (size_t(1) << 31) && m * k * 2 < (size_t(1) << 31) && al16(x) && al16(w) &&
           al16(y) && (scale == nullptr || al16(scale)) && (res == nullptr || al16(res));
}

hipError_t launch_skinny_gemm(size_t m, size_t k, size_t n, const void *x, const void *w,
                              bool w_transposed, const float *scale, const void *res, void *y,
                              hipStream_t s) {
    const uint32_t M = static_cast<uint32_t>(m), K = static_cast<uint32_t>(k),
                   N = static_cast<uint32_t>(n);
    const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
    if (w_transposed)
        hipLaunchKernelGGL((skinny_gemm_kernel<kBM, kBN, true>), grid, dim3(kThreads), 0, s, M, K, N,
                           x, w, scale, res, y);
    else
        hipLaunchKernelGGL((skinny_gemm_kernel<kBM, kBN, false>), grid, dim3(kThreads), 0, s, M, K, N,
                           x, w, scale, res, y);
    return hipGetLastError();
}

}  // namespace m3
