// On-device check of the MFMA lane layouts and the DPP segmented scans the
// scan kernels are written against (see m3_device.hpp): integer-valued
// operands, exact in bf16 and f32.
#include "m3_device.hpp"
#include "m3_internal.hpp"

namespace m3 {

namespace {

__device__ float a_val(int m, int k) { return static_cast<float>((m * 3 + k * 5) % 7 - 3); }
__device__ float b_val(int k, int n) { return static_cast<float>((k * 2 + n * 7) % 5 - 2); }

__global__ void mfma_layout_kernel(int *fail) {
    const int lane = threadIdx.x;
    const int g = lane >> 4, c = lane & 15;
    // bf16 16x16x32: A row c, k = 8g + j; B column c, k = 8g + j
    bf16x8 av, bv;
    for (int j = 0; j < 8; ++j) {
        av[j] = static_cast<__bf16>(a_val(c, 8 * g + j));
        bv[j] = static_cast<__bf16>(b_val(8 * g + j, c));
    }
    f32x4 d = mfma_bf16(av, bv, f32x4{0.f, 0.f, 0.f, 0.f});
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r, n = c;
        float want = 0.f;
        for (int k = 0; k < 32; ++k) want += a_val(m, k) * b_val(k, n);
        if (d[r] != want) atomicOr(fail, 1);
    }
    // f32 16x16x4: A row c, k = g; B column c, k = g
    f32x4 e = mfma_f32(a_val(c, g), b_val(g, c), f32x4{0.f, 0.f, 0.f, 0.f});
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r, n = c;
        float want = 0.f;
        for (int k = 0; k < 4; ++k) want += a_val(m, k) * b_val(k, n);
        if (e[r] != want) atomicOr(fail, 2);
    }
    // segmented inclusive scans (lane + 1 summed within 16/32/64-lane segments)
    const float v = static_cast<float>(lane + 1);
    const float s16 = seg_scan<16>(v), s32 = seg_scan<32>(v), s64 = seg_scan<64>(v);
    auto tri = [&](int seg) {
        const int first = lane - lane % seg;
        float want = 0.f;
        for (int j = first; j <= lane; ++j) want += static_cast<float>(j + 1);
        return want;
    };
    if (s16 != tri(16)) atomicOr(fail, 4);
    if (s32 != tri(32)) atomicOr(fail, 8);
    if (s64 != tri(64)) atomicOr(fail, 16);
}

}  // namespace

hipError_t launch_mfma_selftest(int *result_host) {
    int *dev = nullptr;
    hipError_t e = hipMalloc(&dev, sizeof(int));
    if (e != hipSuccess) return e;
    e = hipMemset(dev, 0, sizeof(int));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(mfma_layout_kernel, dim3(1), dim3(64), 0, 0, dev);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(result_host, dev, sizeof(int), hipMemcpyDeviceToHost);
    (void)hipFree(dev);
    return e;
}

}  // namespace m3
