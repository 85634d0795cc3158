// Host-side launcher declarations shared by the C ABI (m3_api.cpp) and the
// kernel translation units.  Shapes have been validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace m3 {

// Decode step: one token per sequence, state updated in place.
struct StepLaunch {
    size_t batch, heads, head_dim, d_state, rank;
    int bf16;                       // storage of x, b, c, theta, y
    const void *x, *b, *c;          // [B,H,P,R], [B,H,N,R], [B,H,N,R]
    const float *dt, *lambda;       // [B,H]
    const float *a_log;             // [H]
    const void *theta;              // [B,H,N/2] or null
    const float *d_skip;            // [H] or null
    float *h, *last_u, *angle;      // [B,H,P,N] x2, [B,H,N/2] (null without theta)
    void *y;                        // [B,H,P,R]
};
hipError_t launch_step(const StepLaunch &a, hipStream_t stream);

// Chunked scan.  `mode_raw` selects the mamba3_scan prologue (a, g, w built
// from dt, lambda, a_log) versus ssd_chunked's precomputed a, g, w.
struct ScanLaunch {
    size_t batch, seq, heads, head_dim, d_state, rank;
    int bf16;
    int mode_raw;
    const void *x, *b, *c;          // [B,T,H,P,R], [B,T,H,N,R] x2
    const float *dt, *lambda, *a_log;   // raw mode
    const float *a, *g, *w;             // ssd_chunked mode
    const void *theta;              // [B,T,H,N/2] or null (raw mode only)
    const float *d_skip;            // [H] or null
    const float *h0, *last_u0;      // incoming state or null (raw: both or neither)
    const float *angle0;            // [B,H,N/2] or null
    const float *init_state;        // ssd_chunked's initial_state or null
    void *y;                        // [B,T,H,P,R]
    float *h_out, *last_u_out, *angle_out;  // null when not wanted
};
hipError_t launch_scan(const ScanLaunch &a, hipStream_t stream);
// The specialised kernel (head_dim 64, d_state 64/128, rank 1/2/4, 16-byte
// aligned x/b/c/theta/y); hipErrorNotSupported for anything else.
bool scan_fast_supported(const ScanLaunch &a);
hipError_t launch_scan_fast(const ScanLaunch &a, hipStream_t stream);
// The chunk-parallel form of the same shapes (chunk states, an elementwise
// state pass, chunk outputs: three launches over a 256-byte aligned caller
// workspace): the workspace bytes it needs (0 when the shape is not covered),
// and the launch.
size_t scan_chunked_workspace(const ScanLaunch &a);
hipError_t launch_scan_chunked(const ScanLaunch &a, void *workspace, hipStream_t stream);

// Largest head_dim / d_state the scan kernels are instantiated for.
constexpr size_t kScanMaxHeadDim = 128;
constexpr size_t kScanMaxState = 256;
constexpr size_t kScanMaxRank = 64;

// MFMA lane-layout self test (writes 0 on success, else a failure code).
hipError_t launch_mfma_selftest(int *result_host);

}  // namespace m3
