// C ABI of the gfx950 Mamba-3 path: argument validation (mirroring the
// reference's rules and messages), dispatch to the HIP kernels, and the error
// channel.  See include/mamba3_ssm.h for the contract.
#include "mamba3_ssm.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "m3_internal.hpp"

namespace {

thread_local std::string g_last_error;
std::atomic<uint64_t> g_launches{0};

m3_status vfail(m3_status st, const char *fmt, va_list ap) {
    char buf[512];
    vsnprintf(buf, sizeof(buf), fmt, ap);
    const char *prefix = "";
    switch (st) {
        case M3_ERR_CONFIG: prefix = "invalid configuration: "; break;   // error.rs:12
        case M3_ERR_SHAPE: prefix = "shape error: "; break;              // error.rs:16
        case M3_ERR_UNSUPPORTED: prefix = "unsupported: "; break;        // error.rs:47
        case M3_ERR_STATE_DICT: prefix = "state dict error: "; break;    // error.rs:35
        case M3_ERR_IO: prefix = "io error: "; break;                    // error.rs:39
        case M3_ERR_JSON: prefix = "json error: "; break;                // error.rs:43
        default: break;
    }
    g_last_error = std::string(prefix) + buf;
    return st;
}

m3_status fail(m3_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const m3_status r = vfail(st, fmt, ap);
    va_end(ap);
    return r;
}

m3_status ok() {
    g_last_error.clear();
    return M3_OK;
}

m3_status hip_fail(hipError_t e, const char *what) {
    return fail(M3_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Largest rows-per-chunk the scan instantiations use for this dtype / d_state
// (a row is one (token, rank) pair, so rank may not exceed it).
size_t scan_rows(int dtype, size_t d_state) {
    if (dtype == M3_BF16) return d_state <= 128 ? 64 : 32;
    return d_state <= 128 ? 32 : 16;
}

bool dtype_ok(int32_t d) { return d == M3_F32 || d == M3_BF16 || d == M3_F16; }

// Zero `n` floats on `s` with a kernel rather than hipMemsetAsync, so that a
// caller who captures the call into a HIP graph records a kernel node only.
__global__ void zero_fill_kernel(float *p, size_t n) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        p[i] = 0.0f;
}

hipError_t zero_async(float *p, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(zero_fill_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)),
                       dim3(256), 0, s, p, n);
    g_launches.fetch_add(1, std::memory_order_relaxed);
    return hipGetLastError();
}

// ---- f16 storage (the reference's FloatElem for half::f16, backend.rs:86-98).
// The f32 kernels run on f32 copies of the caller's f16 tensors: inputs are
// widened before the call, outputs narrowed after it (round to nearest even),
// in temporaries allocated and freed in stream order on the call's stream.
// So an f16 call gives exactly the f32 call's results on the widened inputs,
// rounded to f16.
__global__ void f16_widen_kernel(const _Float16 *src, float *dst, size_t n) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        dst[i] = static_cast<float>(src[i]);
}
__global__ void f16_narrow_kernel(const float *src, _Float16 *dst, size_t n) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        dst[i] = static_cast<_Float16>(src[i]);
}

class F16Copies {
  public:
    explicit F16Copies(hipStream_t s) : s_(s) {}
    F16Copies(const F16Copies &) = delete;
    F16Copies &operator=(const F16Copies &) = delete;
    ~F16Copies() {
        for (const Item &it : items_) (void)hipFreeAsync(it.f32, s_);
    }
    // An f32 copy of the n f16 values at p (NULL for a NULL p): widened now
    // when `in`, narrowed back into p by narrow() when `out`.
    float *add(const void *p, size_t n, bool in, bool out) {
        if (p == nullptr || err_ != hipSuccess) return nullptr;
        void *f = nullptr;
        err_ = hipMallocAsync(&f, (n ? n : 1) * sizeof(float), s_);
        if (err_ != hipSuccess) return nullptr;
        items_.push_back({const_cast<void *>(p), static_cast<float *>(f), n, out});
        if (in && n > 0) {
            hipLaunchKernelGGL(f16_widen_kernel, dim3(grid(n)), dim3(256), 0, s_,
                               static_cast<const _Float16 *>(p), static_cast<float *>(f), n);
            g_launches.fetch_add(1, std::memory_order_relaxed);
            err_ = hipGetLastError();
        }
        return static_cast<float *>(f);
    }
    hipError_t error() const { return err_; }
    // every `out` copy back into its f16 tensor
    hipError_t narrow() {
        for (const Item &it : items_) {
            if (!it.out || it.n == 0 || err_ != hipSuccess) continue;
            hipLaunchKernelGGL(f16_narrow_kernel, dim3(grid(it.n)), dim3(256), 0, s_, it.f32,
                               static_cast<_Float16 *>(it.dst), it.n);
            g_launches.fetch_add(1, std::memory_order_relaxed);
            err_ = hipGetLastError();
        }
        return err_;
    }

  private:
    struct Item {
        void *dst;
        float *f32;
        size_t n;
        bool out;
    };
    static unsigned grid(size_t n) {
        const size_t b = (n + 255) / 256;
        return static_cast<unsigned>(b < 8192 ? b : 8192);
    }
    hipStream_t s_;
    std::vector<Item> items_;
    hipError_t err_ = hipSuccess;
};

}  // namespace

namespace m3 {
m3_status api_fail(m3_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const m3_status r = vfail(st, fmt, ap);
    va_end(ap);
    return r;
}
m3_status api_ok() { return ok(); }
m3_status api_hip_fail(hipError_t e, const char *what) { return hip_fail(e, what); }
void count_launches(uint64_t n) { g_launches.fetch_add(n, std::memory_order_relaxed); }
}  // namespace m3

extern "C" {

m3_status m3_config_default(m3_ssm_config *out) {
    if (out == nullptr) return fail(M3_ERR_ARGUMENT, "config pointer is NULL");
    // config.rs:130-156
    out->d_model = 768;
    out->n_heads = 24;
    out->head_dim = 64;
    out->d_state = 64;
    out->n_groups = 24;
    out->discretization = M3_LEARNED_TRAPEZOID;
    out->dynamics = M3_ROTATIONAL;
    out->rank = 1;
    out->chunk_size = 64;
    out->conv_kernel = 4;
    out->bc_norm = 1;
    out->bc_bias = 1;
    out->post_gate_norm = 0;
    out->skip_connection = 1;
    out->dt_min = 0.001f;
    out->dt_max = 0.1f;
    out->dt_init_floor = 1e-4f;
    out->a_init_min = 1.0f;
    out->a_init_max = 16.0f;
    out->bias = 0;
    return ok();
}

m3_status m3_config_validate(const m3_ssm_config *c) {
    if (c == nullptr) return fail(M3_ERR_ARGUMENT, "config pointer is NULL");
    // config.rs:203-245, rule for rule
    if (c->d_model == 0 || c->n_heads == 0 || c->head_dim == 0 || c->d_state == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    if (c->n_groups == 0 || c->n_heads % c->n_groups != 0)
        return fail(M3_ERR_CONFIG, "n_heads (%zu) must be a multiple of n_groups (%zu)",
                    c->n_heads, c->n_groups);
    if (c->dynamics == M3_ROTATIONAL && c->d_state % 2 != 0)
        return fail(M3_ERR_CONFIG,
                    "rotational dynamics pair up state dimensions, so d_state must be even, "
                    "got %zu",
                    c->d_state);
    if (c->chunk_size == 0) return fail(M3_ERR_CONFIG, "chunk_size must be positive");
    if (c->rank == 0) return fail(M3_ERR_CONFIG, "MIMO rank must be positive");
    if (!(c->dt_min > 0.0f) || !(c->dt_max > c->dt_min))
        return fail(M3_ERR_CONFIG, "expected 0 < dt_min < dt_max, got %g and %g",
                    static_cast<double>(c->dt_min), static_cast<double>(c->dt_max));
    if (!(c->a_init_min > 0.0f) || c->a_init_max < c->a_init_min)
        return fail(M3_ERR_CONFIG, "expected 0 < a_init_min <= a_init_max");
    if (c->conv_kernel != 0 && c->conv_kernel < 2)
        return fail(M3_ERR_CONFIG, "conv_kernel must be at least 2; use None to disable");
    if (c->discretization < M3_EULER || c->discretization > M3_LEARNED_TRAPEZOID)
        return fail(M3_ERR_CONFIG, "unknown discretization %d", c->discretization);
    if (c->dynamics != M3_REAL && c->dynamics != M3_ROTATIONAL)
        return fail(M3_ERR_CONFIG, "unknown dynamics %d", c->dynamics);
    return ok();
}

size_t m3_config_d_inner(const m3_ssm_config *c) { return c->n_heads * c->head_dim * c->rank; }
size_t m3_config_bc_width(const m3_ssm_config *c) { return c->n_groups * c->d_state * c->rank; }
size_t m3_config_theta_width(const m3_ssm_config *c) {
    return c->dynamics == M3_ROTATIONAL ? c->n_heads * c->d_state / 2 : 0;
}
size_t m3_config_lambda_width(const m3_ssm_config *c) {
    return c->discretization == M3_LEARNED_TRAPEZOID ? c->n_heads : 0;
}
size_t m3_config_in_proj_width(const m3_ssm_config *c) {
    // z gate, x, B, C, dt, lambda, theta  (config.rs:191-200)
    return 2 * m3_config_d_inner(c) + 2 * m3_config_bc_width(c) + c->n_heads +
           m3_config_lambda_width(c) + m3_config_theta_width(c);
}

float m3_discretization_fixed_lambda(int32_t d) {
    if (d == M3_EULER) return 1.0f;
    if (d == M3_TRAPEZOID) return 0.5f;
    return std::nanf("");
}

// Test and benchmark settings of the chunk-parallel scan (m3_debug_scan_options):
// the form (0 the fused single launch where it covers the shape, 1 the three
// launches) and the fused launch's look-back (give up at once; polls).
static std::atomic<int> g_scan_path{0}, g_lb_mode{0}, g_lb_spin{0};

// The scan, and with gate_z the mixer's gate on its y (in place): fused into
// the chunk-parallel kernel where that form runs (bf16, rank 1), else the
// gate kernel after the scan.  path: the chunk-parallel form (-1 the setting).
// theta_stride: elements between tokens' theta rows (0 contiguous), taken by
// the specialised kernels only.
static m3_status scan_entry(const m3_scan_inputs *in, const m3_scan_output *out,
                            const void *gate_z, size_t gate_stride, void *stream,
                            int path = -1, size_t theta_stride = 0);

// The step kernel's LDS holds B~, C~ (d_state x rank each) and x (head_dim x
// rank) as f32: 64 KB.
constexpr size_t kStepLdsFloats = 16384;

// Shapes the scan kernels do not cover (head_dim, d_state or rank beyond
// their tiles); the reference's mamba3_scan has no such limits
// (scan.rs:458-618).
static bool scan_by_steps_needed(const m3_scan_inputs *in) {
    return in->head_dim > m3::kScanMaxHeadDim || in->d_state > m3::kScanMaxState ||
           in->rank > scan_rows(in->dtype, in->d_state);
}
static bool step_covers(const m3_scan_inputs *in) {
    return (2 * in->d_state + in->head_dim) * in->rank <= kStepLdsFloats;
}

// The scan of such shapes as its definition as a recurrence: one launch of
// the step kernel's generic body per token over every (batch, head), in
// order, carrying (h, last_u, angle) from the incoming state (zeros without
// one).  mamba3_step on one token is the scan of that token from the state
// (the reference checks the one against the other, tests/ssm.rs:312-380).
// The carried state lives in the output state buffers when they are wanted,
// else in temporaries allocated and freed in stream order.  Arguments are
// validated by the caller; f32 or bf16 storage.
static m3_status scan_by_steps(const m3_scan_inputs *in, const m3_scan_output *out,
                               hipStream_t s) {
    const size_t B = in->batch, T = in->seq, H = in->heads, P = in->head_dim, N = in->d_state;
    const size_t R = in->rank, es = in->dtype == M3_BF16 ? 2 : 4;
    const bool rot = in->theta != nullptr;
    const size_t sn = B * H * P * N, an = B * H * (N / 2);
    std::vector<void *> temps;
    hipError_t e = hipSuccess;
    auto temp = [&](size_t n) -> float * {
        void *p = nullptr;
        if (e == hipSuccess) e = hipMallocAsync(&p, n * sizeof(float), s);
        if (e != hipSuccess) return nullptr;
        temps.push_back(p);
        return static_cast<float *>(p);
    };
    const bool want = in->want_state != 0;
    float *h = want ? out->state.h : temp(sn);
    float *lu = want ? out->state.last_u : temp(sn);
    float *ang = rot ? (want ? out->state.angle : temp(an)) : nullptr;
    const m3_ssm_state *st = in->state;
    if (e == hipSuccess) {
        if (st != nullptr) {
            e = hipMemcpyAsync(h, st->h, sn * sizeof(float), hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess)
                e = hipMemcpyAsync(lu, st->last_u, sn * sizeof(float), hipMemcpyDeviceToDevice, s);
        } else {
            e = zero_async(h, sn, s);
            if (e == hipSuccess) e = zero_async(lu, sn, s);
        }
        if (e == hipSuccess && rot)
            e = (st != nullptr && st->angle != nullptr)
                    ? hipMemcpyAsync(ang, st->angle, an * sizeof(float), hipMemcpyDeviceToDevice, s)
                    : zero_async(ang, an, s);
    }
    m3::StepLaunch a{};
    a.batch = B;
    a.heads = H;
    a.head_dim = P;
    a.d_state = N;
    a.rank = R;
    a.bf16 = in->dtype == M3_BF16;
    a.a_log = in->a_log;
    a.d_skip = in->d_skip;
    a.h = h;
    a.last_u = lu;
    a.angle = ang;
    a.in_bstride = T;
    for (size_t t = 0; t < T && e == hipSuccess; ++t) {
        a.x = static_cast<const char *>(in->x) + t * H * P * R * es;
        a.b = static_cast<const char *>(in->b) + t * H * N * R * es;
        a.c = static_cast<const char *>(in->c) + t * H * N * R * es;
        a.theta = rot ? static_cast<const char *>(in->theta) + t * H * (N / 2) * es : nullptr;
        a.dt = in->dt + t * H;
        a.lambda = in->lambda + t * H;
        a.y = static_cast<char *>(out->y) + t * H * P * R * es;
        e = m3::launch_step(a, s);
        if (e == hipSuccess) g_launches.fetch_add(1, std::memory_order_relaxed);
    }
    for (void *p : temps) (void)hipFreeAsync(p, s);
    if (e != hipSuccess) return hip_fail(e, "scan by steps");
    return ok();
}

// m3_scan with f16 storage: the f32 scan on widened copies of x, b, c and
// theta, y narrowed back (the arguments are validated by the caller).
static m3_status scan_f16(const m3_scan_inputs *in, const m3_scan_output *out, void *stream,
                          int path) {
    const size_t rows = in->batch * in->seq * in->heads;
    const size_t P = in->head_dim, N = in->d_state, R = in->rank;
    F16Copies cp(static_cast<hipStream_t>(stream));
    m3_scan_inputs local = *in;
    local.dtype = M3_F32;
    local.x = cp.add(in->x, rows * P * R, true, false);
    local.b = cp.add(in->b, rows * N * R, true, false);
    local.c = cp.add(in->c, rows * N * R, true, false);
    local.theta = cp.add(in->theta, rows * (N / 2), true, false);
    m3_scan_output o = *out;
    o.y = cp.add(out->y, rows * P * R, false, true);
    if (cp.error() != hipSuccess) return hip_fail(cp.error(), "f16 copies");
    const m3_status st = scan_entry(&local, &o, nullptr, 0, stream, path);
    if (st != M3_OK) return st;
    if (cp.narrow() != hipSuccess) return hip_fail(cp.error(), "f16 narrowing");
    return ok();
}

static m3_status scan_entry(const m3_scan_inputs *in, const m3_scan_output *out,
                            const void *gate_z, size_t gate_stride, void *stream,
                            int path, size_t theta_stride) {
    if (in == nullptr || out == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/outputs are NULL");
    if (!dtype_ok(in->dtype)) return fail(M3_ERR_ARGUMENT, "unknown dtype %d", in->dtype);
    if (in->rank == 0) return fail(M3_ERR_CONFIG, "MIMO rank must be positive");
    if (in->head_dim == 0 || in->d_state == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    if (in->theta != nullptr && in->d_state % 2 != 0)   // scan.rs:485-489
        return fail(M3_ERR_CONFIG, "rotational dynamics require an even d_state");
    // shapes beyond the scan kernels run token by token on the step kernel
    const bool by_steps = scan_by_steps_needed(in);
    if (by_steps && !step_covers(in))
        return fail(M3_ERR_UNSUPPORTED, "head_dim %zu, d_state %zu and rank %zu exceed both the "
                    "scan kernels (head_dim <= %zu, d_state <= %zu, rank <= %zu) and the step "
                    "kernel (2 d_state rank + head_dim rank <= %zu)", in->head_dim, in->d_state,
                    in->rank, m3::kScanMaxHeadDim, m3::kScanMaxState,
                    scan_rows(in->dtype, in->d_state), kStepLdsFloats);
    const m3_ssm_state *st = in->state;
    if (st != nullptr && (st->h == nullptr || st->last_u == nullptr))
        return fail(M3_ERR_ARGUMENT, "state needs both h and last_u");
    if (in->want_state) {
        if (out->state.h == nullptr || out->state.last_u == nullptr)
            return fail(M3_ERR_ARGUMENT, "want_state needs output h and last_u buffers");
        if (in->theta != nullptr && out->state.angle == nullptr)
            return fail(M3_ERR_ARGUMENT, "want_state with theta needs an output angle buffer");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t B = in->batch, H = in->heads, P = in->head_dim, N = in->d_state;
    const size_t sbytes = B * H * P * N * sizeof(float);
    if (B * H == 0) return ok();
    if (in->seq == 0) {
        // empty window: nothing to mix, the state passes through
        if (in->want_state) {
            hipError_t e;
            if (st != nullptr) {
                e = hipMemcpyAsync(out->state.h, st->h, sbytes, hipMemcpyDeviceToDevice, s);
                if (e == hipSuccess)
                    e = hipMemcpyAsync(out->state.last_u, st->last_u, sbytes,
                                       hipMemcpyDeviceToDevice, s);
            } else {
                e = zero_async(out->state.h, sbytes / sizeof(float), s);
                if (e == hipSuccess) e = zero_async(out->state.last_u, sbytes / sizeof(float), s);
            }
            // An empty theta tensor may arrive as a NULL pointer, so the angle
            // passes through whenever the caller gave an output angle buffer.
            if (e == hipSuccess && out->state.angle != nullptr) {
                const size_t abytes = B * H * (N / 2) * sizeof(float);
                if (st != nullptr && st->angle != nullptr)
                    e = hipMemcpyAsync(out->state.angle, st->angle, abytes,
                                       hipMemcpyDeviceToDevice, s);
                else
                    e = zero_async(out->state.angle, abytes / sizeof(float), s);
            }
            if (e != hipSuccess) return hip_fail(e, "state pass-through");
        }
        return ok();
    }
    if (in->x == nullptr || in->b == nullptr || in->c == nullptr || in->dt == nullptr ||
        in->a_log == nullptr || in->lambda == nullptr || out->y == nullptr)
        return fail(M3_ERR_ARGUMENT, "x, b, c, dt, a_log, lambda and y are required");
    if (in->dtype == M3_F16) {
        if (gate_z != nullptr || theta_stride != 0)
            return fail(M3_ERR_UNSUPPORTED, "the gate and theta in place cover bf16 storage");
        return scan_f16(in, out, stream, path);
    }
    if (by_steps) {
        if (theta_stride != 0)
            return fail(M3_ERR_UNSUPPORTED, "theta in place covers the scan kernels' shapes");
        const m3_status st2 = scan_by_steps(in, out, s);
        if (st2 != M3_OK || gate_z == nullptr) return st2;
        hipError_t e = m3::launch_mixer_gate(B * in->seq, H * P * in->rank, out->y, gate_z,
                                             gate_stride, nullptr, 0.0f, out->y, s);
        if (e != hipSuccess) return hip_fail(e, "gate launch");
        g_launches.fetch_add(1, std::memory_order_relaxed);
        return ok();
    }

    m3::ScanLaunch a{};
    a.batch = B;
    a.seq = in->seq;
    a.heads = H;
    a.head_dim = P;
    a.d_state = N;
    a.rank = in->rank;
    a.bf16 = in->dtype == M3_BF16;
    a.mode_raw = 1;
    a.chunk_size = in->chunk_size;
    a.x = in->x;
    a.b = in->b;
    a.c = in->c;
    a.dt = in->dt;
    a.lambda = in->lambda;
    a.a_log = in->a_log;
    a.theta = in->theta;
    a.theta_stride = in->theta ? theta_stride : 0;
    a.d_skip = in->d_skip;
    a.h0 = st ? st->h : nullptr;
    a.last_u0 = st ? st->last_u : nullptr;
    a.angle0 = (st && in->theta) ? st->angle : nullptr;
    a.y = out->y;
    a.path = path >= 0 ? path : g_scan_path.load(std::memory_order_relaxed);
    a.lb_mode = g_lb_mode.load(std::memory_order_relaxed);
    a.lb_spin = g_lb_spin.load(std::memory_order_relaxed);
    if (in->want_state) {
        a.h_out = out->state.h;
        a.last_u_out = out->state.last_u;
        a.angle_out = in->theta ? out->state.angle : nullptr;
    }
    if (a.theta_stride != 0 && !m3::scan_fast_supported(a))
        return fail(M3_ERR_UNSUPPORTED, "theta at a token stride of %zu elements needs head_dim 64, "
                    "d_state 64 or 128, rank 1, 2 or 4, 16-byte aligned buffers and rows of whole "
                    "16-byte pieces", a.theta_stride);
    hipError_t e;
    const size_t need = m3::scan_chunked_workspace(a);
    const bool ws_aligned = (reinterpret_cast<uintptr_t>(in->workspace) & 255u) == 0;
    const bool chunked =
        need > 0 && in->workspace != nullptr && in->workspace_bytes >= need && ws_aligned;
    // the fused gate reads z in 8-byte pieces through one 32-bit buffer range
    // per sequence
    const bool fuse_gate = gate_z != nullptr && chunked && a.bf16 && a.rank == 1 &&
                           (reinterpret_cast<uintptr_t>(gate_z) & 7u) == 0 && gate_stride % 4 == 0 &&
                           a.seq * gate_stride * 2 < (size_t(1) << 31);
    if (fuse_gate) {
        a.gate_z = gate_z;
        a.gate_stride = gate_stride;
    }
    if (chunked) {
        e = m3::launch_scan_chunked(a, in->workspace, s);
        if (e == hipSuccess)
            g_launches.fetch_add(m3::scan_chunked_launches(a), std::memory_order_relaxed);
    } else {
        e = m3::launch_scan(a, s);
        if (e == hipSuccess) g_launches.fetch_add(1, std::memory_order_relaxed);
    }
    if (e != hipSuccess) return hip_fail(e, "scan launch");
    if (gate_z != nullptr && !fuse_gate) {
        e = m3::launch_mixer_gate(B * in->seq, H * P * in->rank, out->y, gate_z, gate_stride,
                                  nullptr, 0.0f, out->y, s);
        if (e != hipSuccess) return hip_fail(e, "gate launch");
        g_launches.fetch_add(1, std::memory_order_relaxed);
    }
    return ok();
}

m3_status m3_scan(const m3_scan_inputs *in, const m3_scan_output *out, void *stream) {
    return scan_entry(in, out, nullptr, 0, stream);
}

m3_status m3_scan_gated(const m3_scan_inputs *in, const m3_scan_output *out, const void *z,
                        size_t z_stride, size_t theta_stride, void *stream) {
    if (in == nullptr || out == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/outputs are NULL");
    if (in->dtype != M3_BF16)
        return fail(M3_ERR_UNSUPPORTED, "the gated scan covers bf16 storage");
    if (z == nullptr) return fail(M3_ERR_ARGUMENT, "the gate's z is NULL");
    const size_t d_inner = in->heads * in->head_dim * in->rank;
    if (z_stride < d_inner)
        return fail(M3_ERR_SHAPE, "z stride %zu is shorter than d_inner %zu", z_stride, d_inner);
    const size_t theta_row = in->heads * (in->d_state / 2);
    if (in->theta != nullptr && theta_stride != 0 && theta_stride < theta_row)
        return fail(M3_ERR_SHAPE, "theta stride %zu is shorter than a token's %zu angles",
                    theta_stride, theta_row);
    return scan_entry(in, out, z, z_stride, stream, -1,
                      theta_stride == theta_row ? 0 : theta_stride);
}

}  // extern "C"

static size_t workspace_bytes_for(const m3_scan_inputs *in, int path) {
    if (in == nullptr || !dtype_ok(in->dtype) || in->seq == 0) return 0;
    m3::ScanLaunch a{};
    a.path = path;
    a.batch = in->batch;
    a.seq = in->seq;
    a.heads = in->heads;
    a.head_dim = in->head_dim;
    a.d_state = in->d_state;
    a.rank = in->rank;
    a.bf16 = in->dtype == M3_BF16;
    a.mode_raw = 1;   // m3_scan's prologue, as the launch sets it
    a.chunk_size = in->chunk_size;
    // alignment is checked at launch; size the shape as if aligned
    alignas(16) static float dummy[4] = {0, 0, 0, 0};
    a.x = a.b = a.c = dummy;
    a.y = dummy;
    return m3::scan_chunked_workspace(a);
}

extern "C" {

size_t m3_scan_workspace_bytes(const m3_scan_inputs *in) {
    return workspace_bytes_for(in, g_scan_path.load(std::memory_order_relaxed));
}

m3_status m3_debug_scan_options(int32_t path, int32_t lookback_mode, int32_t lookback_spin) {
    if (path < 0 || path > 1 || lookback_mode < 0 || lookback_mode > 1 || lookback_spin < 0)
        return fail(M3_ERR_ARGUMENT, "scan options: path 0 or 1, look-back mode 0 or 1, spin >= 0");
    g_scan_path.store(path, std::memory_order_relaxed);
    g_lb_mode.store(lookback_mode, std::memory_order_relaxed);
    g_lb_spin.store(lookback_spin, std::memory_order_relaxed);
    return ok();
}

}  // extern "C"

namespace {

// The chunk-parallel scan's workspace for m3_scan_no_alloc: one file-scope
// device array, so each GPU the library runs on holds its own copy until the
// process ends.  In host code `scratch` names a host-side stand-in, never the
// device memory: kernels get the address hipGetSymbolAddress returns for the
// current device, looked up once per device and kept in g_scratch.
constexpr size_t kNoAllocScratchBytes = size_t(M3_NO_ALLOC_SCRATCH_MIB) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

// The current device's copy of `scratch` (nullptr and a message on failure).
// The current device's scratch address (dev receives the device), or NULL
// with the error recorded in *st.
void *scratch_for_current_device(int &dev, m3_status *st) {
    dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *st = hip_fail(e, "hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *st = fail(M3_ERR_UNSUPPORTED, "device %d is beyond the %d devices the static scratch covers",
                   dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *st = hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        g_scratch[dev] = p;
    }
    return g_scratch[dev];
}

// Overlap guard of the eager (not graph-captured) calls: per device, the
// stream of the last call and an event recorded after it.  A call on another
// stream while that event is pending would race on the same scratch, so it is
// refused instead.  The lock is held from the check to the record, so host
// threads cannot slip a call in between.  Calls captured into a graph (and
// the graph's replays) are not tracked.
std::mutex g_guard_mu;
hipStream_t g_guard_stream[kMaxDevices];
hipEvent_t g_guard_event[kMaxDevices];
bool g_guard_set[kMaxDevices];

}  // namespace

extern "C" {

m3_status m3_scan_no_alloc(const m3_scan_inputs *in, const m3_scan_output *out, void *stream) {
    if (in == nullptr || out == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/outputs are NULL");
    if (in->dtype == M3_F16)
        return fail(M3_ERR_UNSUPPORTED, "f16 storage widens into temporaries it allocates: "
                    "call m3_scan instead");
    if (scan_by_steps_needed(in))
        return fail(M3_ERR_UNSUPPORTED, "head_dim %zu, d_state %zu and rank %zu are beyond the "
                    "scan kernels' tiles: call m3_scan instead", in->head_dim, in->d_state,
                    in->rank);
    m3_scan_inputs local = *in;
    local.workspace = nullptr;
    local.workspace_bytes = 0;
    int path = g_scan_path.load(std::memory_order_relaxed);
    size_t need = workspace_bytes_for(&local, path);
    if (need > kNoAllocScratchBytes && path == 0) {
        // the fused launch's records do not fit: the three launches' may
        const size_t three = workspace_bytes_for(&local, 1);
        if (three <= kNoAllocScratchBytes) {
            path = 1;
            need = three;
        }
    }
    if (need > kNoAllocScratchBytes)
        return fail(M3_ERR_UNSUPPORTED,
                    "this scan needs %zu bytes of scratch; m3_scan_no_alloc's static scratch holds "
                    "%zu (%d MiB): call m3_scan with a caller workspace instead",
                    need, kNoAllocScratchBytes, M3_NO_ALLOC_SCRATCH_MIB);
    if (need == 0) return scan_entry(&local, out, nullptr, 0, stream, path);
    int dev = -1;
    m3_status st = M3_ERR_HIP;
    void *p = scratch_for_current_device(dev, &st);
    if (p == nullptr) return st;
    local.workspace = p;
    local.workspace_bytes = kNoAllocScratchBytes;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone) return scan_entry(&local, out, nullptr, 0, stream, path);
    std::lock_guard<std::mutex> lock(g_guard_mu);
    if (g_guard_set[dev] && g_guard_stream[dev] != s) {
        e = hipEventQuery(g_guard_event[dev]);
        if (e == hipErrorNotReady) {
            (void)hipGetLastError();   // a pending event is not an error of the next launch
            return fail(M3_ERR_ARGUMENT, "an m3_scan_no_alloc call on another stream may still be "
                        "using this GPU's scratch: order the calls (one stream, or an event "
                        "between them), or give each stream m3_scan with its own workspace");
        }
        if (e != hipSuccess) return hip_fail(e, "hipEventQuery");
    }
    st = scan_entry(&local, out, nullptr, 0, stream, path);
    if (st != M3_OK) return st;
    if (g_guard_event[dev] == nullptr) {
        e = hipEventCreateWithFlags(&g_guard_event[dev], hipEventDisableTiming);
        if (e != hipSuccess) {
            g_guard_event[dev] = nullptr;
            return hip_fail(e, "hipEventCreateWithFlags");
        }
    }
    e = hipEventRecord(g_guard_event[dev], s);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    g_guard_stream[dev] = s;
    g_guard_set[dev] = true;
    return ok();
}

static m3::ScanLaunch scan_launch_of(const m3_scan_inputs *in) {
    m3::ScanLaunch a{};
    a.batch = in->batch;
    a.seq = in->seq;
    a.heads = in->heads;
    a.head_dim = in->head_dim;
    a.d_state = in->d_state;
    a.rank = in->rank;
    a.bf16 = in->dtype == M3_BF16;
    a.mode_raw = 1;
    a.x = in->x;
    a.b = in->b;
    a.c = in->c;
    a.dt = in->dt;
    a.lambda = in->lambda;
    a.a_log = in->a_log;
    a.theta = in->theta;
    a.d_skip = in->d_skip;
    const m3_ssm_state *st = in->state;
    a.h0 = st ? st->h : nullptr;
    a.last_u0 = st ? st->last_u : nullptr;
    a.angle0 = (st && in->theta) ? st->angle : nullptr;
    return a;
}

m3_status m3_scan_backward(const m3_scan_inputs *in, const m3_scan_grads *g, void *stream) {
    if (in == nullptr || g == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/grads are NULL");
    if (!dtype_ok(in->dtype)) return fail(M3_ERR_ARGUMENT, "unknown dtype %d", in->dtype);
    if (in->rank == 0) return fail(M3_ERR_CONFIG, "MIMO rank must be positive");
    if (in->head_dim == 0 || in->d_state == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    if (in->theta != nullptr && in->d_state % 2 != 0)   // scan.rs:485-489
        return fail(M3_ERR_CONFIG, "rotational dynamics require an even d_state");
    const m3_ssm_state *st = in->state;
    if (st != nullptr && (st->h == nullptr || st->last_u == nullptr))
        return fail(M3_ERR_ARGUMENT, "state needs both h and last_u");
    const size_t B = in->batch, H = in->heads, P = in->head_dim, N = in->d_state;
    if (B * H == 0) return ok();
    if (in->x == nullptr || in->b == nullptr || in->c == nullptr || in->dt == nullptr ||
        in->a_log == nullptr || in->lambda == nullptr)
        return fail(M3_ERR_ARGUMENT, "x, b, c, dt, a_log and lambda are required");
    if (g->dy == nullptr || g->dx == nullptr || g->db == nullptr || g->dc == nullptr ||
        g->ddt == nullptr || g->dlambda == nullptr || g->da_log == nullptr)
        return fail(M3_ERR_ARGUMENT, "dy, dx, db, dc, ddt, dlambda and da_log are required");
    if (in->theta != nullptr && g->dtheta == nullptr)
        return fail(M3_ERR_ARGUMENT, "theta is given: dtheta is required");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (in->dtype == M3_F16 && in->seq > 0) {
        // the f32 backward on widened copies; dx, db, dc and dtheta narrowed back
        m3_scan_inputs li = *in;
        li.dtype = M3_F32;
        m3::ScanLaunch chk = scan_launch_of(&li);
        alignas(16) static float dummy[4] = {0, 0, 0, 0};
        chk.x = chk.b = chk.c = dummy;   // the copies are aligned: the shape decides
        chk.theta = in->theta ? dummy : nullptr;
        if (!m3::scan_backward_supported(chk) && !m3::scan_backward_generic_supported(chk))
            return fail(M3_ERR_UNSUPPORTED, "the scan backward covers shapes whose per-token "
                        "vectors fit 64 KB (2 P R + 4 N R + 3 N/2 floats)");
        const size_t rows = B * in->seq * H, R = in->rank;
        F16Copies cp(s);
        li.x = cp.add(in->x, rows * P * R, true, false);
        li.b = cp.add(in->b, rows * N * R, true, false);
        li.c = cp.add(in->c, rows * N * R, true, false);
        li.theta = cp.add(in->theta, rows * (N / 2), true, false);
        m3_scan_grads lg = *g;
        lg.dy = cp.add(g->dy, rows * P * R, true, false);
        lg.dx = cp.add(g->dx, rows * P * R, false, true);
        lg.db = cp.add(g->db, rows * N * R, false, true);
        lg.dc = cp.add(g->dc, rows * N * R, false, true);
        lg.dtheta = in->theta ? cp.add(g->dtheta, rows * (N / 2), false, true) : g->dtheta;
        if (cp.error() != hipSuccess) return hip_fail(cp.error(), "f16 copies");
        const m3_status st2 = m3_scan_backward(&li, &lg, stream);
        if (st2 != M3_OK) return st2;
        if (cp.narrow() != hipSuccess) return hip_fail(cp.error(), "f16 narrowing");
        return ok();
    }
    if (in->seq == 0) {
        // empty window: the state passed through, nothing else was read
        const size_t sbytes = B * H * P * N * sizeof(float);
        e = hipMemsetAsync(g->da_log, 0, H * sizeof(float), s);
        if (e == hipSuccess && g->dd_skip) e = hipMemsetAsync(g->dd_skip, 0, H * sizeof(float), s);
        if (e == hipSuccess && g->dh0)
            e = g->dh ? hipMemcpyAsync(g->dh0, g->dh, sbytes, hipMemcpyDeviceToDevice, s)
                      : hipMemsetAsync(g->dh0, 0, sbytes, s);
        // the outgoing last_u is the incoming one
        if (e == hipSuccess && g->dlast_u0)
            e = g->dlast_u ? hipMemcpyAsync(g->dlast_u0, g->dlast_u, sbytes, hipMemcpyDeviceToDevice, s)
                           : hipMemsetAsync(g->dlast_u0, 0, sbytes, s);
        if (e == hipSuccess && g->dangle0) {
            const size_t abytes = B * H * (N / 2) * sizeof(float);
            e = g->dangle ? hipMemcpyAsync(g->dangle0, g->dangle, abytes, hipMemcpyDeviceToDevice, s)
                          : hipMemsetAsync(g->dangle0, 0, abytes, s);
        }
        if (e != hipSuccess) return hip_fail(e, "empty-window backward");
        return ok();
    }
    const m3::ScanLaunch a = scan_launch_of(in);
    // shapes (or alignments) the chunk kernels do not take run the reverse
    // mode of the recurrence token by token
    const bool generic = !m3::scan_backward_supported(a);
    if (generic && !m3::scan_backward_generic_supported(a))
        return fail(M3_ERR_UNSUPPORTED, "the scan backward covers shapes whose per-token vectors "
                    "fit 64 KB (2 P R + 4 N R + 3 N/2 floats): head_dim %zu, d_state %zu, rank %zu",
                    P, N, in->rank);
    if (!generic) {
        // gradient buffers are written (and dh read) in 8- and 16-byte pieces
        const void *ptrs[] = {g->dx, g->db, g->dc, g->dtheta, g->dh, g->dh0, g->dlast_u0, g->dlast_u};
        for (const void *q : ptrs)
            if ((reinterpret_cast<uintptr_t>(q) & 15u) != 0)
                return fail(M3_ERR_UNSUPPORTED,
                            "the scan backward needs 16-byte aligned gradient buffers");
    }
    const size_t need = generic ? m3::scan_backward_generic_workspace(a)
                                : m3::scan_backward_workspace(a);
    if (in->workspace == nullptr || in->workspace_bytes < need ||
        (reinterpret_cast<uintptr_t>(in->workspace) & 255u) != 0)
        return fail(M3_ERR_ARGUMENT, "the backward needs a 256-byte aligned workspace of %zu bytes",
                    need);
    m3::ScanGrads gr{};
    gr.dy = g->dy;
    gr.dh_out = g->dh;
    gr.dangle_out = in->theta ? g->dangle : nullptr;
    gr.dlast_u_out = g->dlast_u;
    gr.dx = g->dx;
    gr.db = g->db;
    gr.dc = g->dc;
    gr.ddt = g->ddt;
    gr.dlambda = g->dlambda;
    gr.da_log = g->da_log;
    gr.dtheta = in->theta ? g->dtheta : nullptr;
    gr.dd_skip = in->d_skip ? g->dd_skip : nullptr;
    gr.dh0 = st ? g->dh0 : nullptr;
    gr.dlast_u0 = st ? g->dlast_u0 : nullptr;
    gr.dangle0 = (st && st->angle && in->theta) ? g->dangle0 : nullptr;
    if (generic) {
        e = m3::launch_scan_backward_generic(a, gr, in->workspace, s);
        if (e != hipSuccess) return hip_fail(e, "scan backward launch");
        g_launches.fetch_add(2, std::memory_order_relaxed);
    } else {
        e = m3::launch_scan_backward(a, gr, in->workspace, s);
        if (e != hipSuccess) return hip_fail(e, "scan backward launch");
        g_launches.fetch_add((in->theta ? 5 : 4) + (g->dlast_u ? 2 : 0), std::memory_order_relaxed);
    }
    if (g->dd_skip != nullptr && in->d_skip == nullptr) {
        e = hipMemsetAsync(g->dd_skip, 0, H * sizeof(float), s);
        if (e != hipSuccess) return hip_fail(e, "dd_skip");
    }
    return ok();
}

size_t m3_scan_backward_workspace_bytes(const m3_scan_inputs *in) {
    if (in == nullptr || !dtype_ok(in->dtype) || in->seq == 0) return 0;
    m3::ScanLaunch a = scan_launch_of(in);
    alignas(16) static float dummy[4] = {0, 0, 0, 0};
    a.x = a.b = a.c = dummy;   // alignment is checked at launch
    a.theta = in->theta ? dummy : nullptr;
    a.h0 = a.last_u0 = nullptr;
    const size_t w = m3::scan_backward_workspace(a);
    return w ? w : m3::scan_backward_generic_workspace(a);
}

m3_status m3_ssd_chunked(const m3_ssd_args *in, void *y, float *final_state, void *stream) {
    if (in == nullptr) return fail(M3_ERR_ARGUMENT, "arguments are NULL");
    if (!dtype_ok(in->dtype)) return fail(M3_ERR_ARGUMENT, "unknown dtype %d", in->dtype);
    if (in->head_dim == 0 || in->d_state == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    if (in->head_dim > m3::kScanMaxHeadDim || in->d_state > m3::kScanMaxState)
        return fail(M3_ERR_UNSUPPORTED, "head_dim %zu / d_state %zu exceed the scan kernel's",
                    in->head_dim, in->d_state);
    if (in->want_state && final_state == nullptr)
        return fail(M3_ERR_ARGUMENT, "want_state needs a final_state buffer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t B = in->batch, H = in->heads, P = in->head_dim, N = in->d_state;
    if (B * H == 0) return ok();
    if (in->seq == 0) {   // scan.rs:134-144
        if (in->want_state) {
            const size_t sbytes = B * H * P * N * sizeof(float);
            hipError_t e = in->initial_state
                               ? hipMemcpyAsync(final_state, in->initial_state, sbytes,
                                                hipMemcpyDeviceToDevice, s)
                               : hipMemsetAsync(final_state, 0, sbytes, s);
            if (e != hipSuccess) return hip_fail(e, "state pass-through");
        }
        return ok();
    }
    if (in->x == nullptr || in->b == nullptr || in->c == nullptr || in->a == nullptr ||
        in->g == nullptr || in->w == nullptr || y == nullptr)
        return fail(M3_ERR_ARGUMENT, "x, b, c, a, g, w and y are required");
    if (in->dtype == M3_F16) {
        // the f32 form on widened copies of x, b and c; y narrowed back
        const size_t rows = B * in->seq * H;
        F16Copies cp(s);
        m3_ssd_args li = *in;
        li.dtype = M3_F32;
        li.x = cp.add(in->x, rows * P, true, false);
        li.b = cp.add(in->b, rows * N, true, false);
        li.c = cp.add(in->c, rows * N, true, false);
        float *y32 = cp.add(y, rows * P, false, true);
        if (cp.error() != hipSuccess) return hip_fail(cp.error(), "f16 copies");
        const m3_status st = m3_ssd_chunked(&li, y32, final_state, stream);
        if (st != M3_OK) return st;
        if (cp.narrow() != hipSuccess) return hip_fail(cp.error(), "f16 narrowing");
        return ok();
    }
    m3::ScanLaunch a{};
    a.batch = B;
    a.seq = in->seq;
    a.heads = H;
    a.head_dim = P;
    a.d_state = N;
    a.rank = 1;
    a.bf16 = in->dtype == M3_BF16;
    a.mode_raw = 0;
    a.x = in->x;
    a.b = in->b;
    a.c = in->c;
    a.a = in->a;
    a.g = in->g;
    a.w = in->w;
    a.init_state = in->initial_state;
    a.y = y;
    a.h_out = in->want_state ? final_state : nullptr;
    hipError_t e = m3::launch_scan(a, s);
    if (e != hipSuccess) return hip_fail(e, "ssd_chunked launch");
    g_launches.fetch_add(1, std::memory_order_relaxed);
    return ok();
}

}  // extern "C"

namespace {

// Validates one step's arguments (the full state or, with fst, the factored
// one) and fills `a`; *empty when there is nothing to launch (B H == 0).
m3_status build_step(const m3_step_inputs *in, const m3_ssm_state *state,
                     const m3_ssm_state_factored *fst, void *y, m3::StepLaunch &a, bool *empty) {
    *empty = false;
    if (in == nullptr || (state == nullptr && fst == nullptr))
        return fail(M3_ERR_ARGUMENT, "inputs/state are NULL");
    if (!dtype_ok(in->dtype)) return fail(M3_ERR_ARGUMENT, "unknown dtype %d", in->dtype);
    if (in->rank == 0) return fail(M3_ERR_CONFIG, "MIMO rank must be positive");
    if (in->head_dim == 0 || in->d_state == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    if (in->theta != nullptr && in->d_state % 2 != 0)
        return fail(M3_ERR_CONFIG, "rotational dynamics require an even d_state");
    if (fst != nullptr && !m3::step_factored_supported(in->d_state, in->rank))
        return fail(M3_ERR_UNSUPPORTED, "the factored step needs d_state a multiple of 4 with "
                    "d_state/4 a power of two up to 64 and rank 1, 2, 3, 4 or 8 (got %zu, %zu)",
                    in->d_state, in->rank);
    if (fst == nullptr && (state->h == nullptr || state->last_u == nullptr))
        return fail(M3_ERR_ARGUMENT, "state needs both h and last_u");
    if (fst != nullptr && (fst->h == nullptr || fst->x_prev == nullptr || fst->b_prev == nullptr))
        return fail(M3_ERR_ARGUMENT, "the factored state needs h, x_prev and b_prev");
    float *angle = fst ? fst->angle : state->angle;
    if (in->theta != nullptr && angle == nullptr)
        return fail(M3_ERR_ARGUMENT, "theta needs the state's angle buffer (updated in place)");
    if (in->batch * in->heads == 0) {
        *empty = true;
        return ok();
    }
    if (in->x == nullptr || in->b == nullptr || in->c == nullptr || in->dt == nullptr ||
        in->lambda == nullptr || in->a_log == nullptr || y == nullptr)
        return fail(M3_ERR_ARGUMENT, "x, b, c, dt, lambda, a_log and y are required");
    const size_t lds = fst ? in->d_state * in->rank * 3 + in->head_dim * in->rank * 2
                           : in->d_state * in->rank * 2 + in->head_dim * in->rank;
    if (lds > 16384)
        return fail(M3_ERR_UNSUPPORTED, "d_state/head_dim/rank too large for the step kernel");
    if (fst != nullptr) {
        const size_t es = in->dtype == M3_F32 ? 4 : 2;
        const size_t xb = in->batch * in->heads * in->head_dim * in->rank * es;
        const size_t bb = in->batch * in->heads * in->d_state * in->rank * es;
        auto overlap = [](const void *p, size_t pn, const void *q, size_t qn) {
            const uintptr_t u = reinterpret_cast<uintptr_t>(p), v = reinterpret_cast<uintptr_t>(q);
            return u < v + qn && v < u + pn;
        };
        if (overlap(fst->x_prev, xb, in->x, xb) || overlap(fst->b_prev, bb, in->b, bb) ||
            overlap(fst->x_prev, xb, in->b, bb) || overlap(fst->b_prev, bb, in->x, xb) ||
            overlap(fst->x_prev, xb, fst->b_prev, bb))
            return fail(M3_ERR_ARGUMENT, "x_prev and b_prev must not overlap each other or the inputs");
    }
    a = m3::StepLaunch{};
    a.batch = in->batch;
    a.heads = in->heads;
    a.head_dim = in->head_dim;
    a.d_state = in->d_state;
    a.rank = in->rank;
    a.bf16 = in->dtype == M3_BF16;
    a.x = in->x;
    a.b = in->b;
    a.c = in->c;
    a.dt = in->dt;
    a.lambda = in->lambda;
    a.a_log = in->a_log;
    a.theta = in->theta;
    a.d_skip = in->d_skip;
    a.h = fst ? fst->h : state->h;
    a.last_u = fst ? nullptr : state->last_u;
    a.x_prev = fst ? fst->x_prev : nullptr;
    a.b_prev = fst ? fst->b_prev : nullptr;
    a.angle = in->theta ? angle : nullptr;
    a.y = y;
    // the vector body issues 16-byte state accesses
    if (reinterpret_cast<uintptr_t>(a.h) % 16 != 0 ||
        (a.last_u != nullptr && reinterpret_cast<uintptr_t>(a.last_u) % 16 != 0))
        return fail(M3_ERR_ARGUMENT, "state buffers must be 16-byte aligned");
    return ok();
}

// A step with f16 storage (validated by build_step): the f32 step on widened
// copies of x, b, c and theta (and of the factored state's x_prev and b_prev,
// narrowed back as the step rewrites them); y narrowed back.
m3_status step_f16(const m3_step_inputs *in, m3_ssm_state *state,
                   m3_ssm_state_factored *fst, void *y, void *stream) {
    const size_t bh = in->batch * in->heads;
    const size_t P = in->head_dim, N = in->d_state, R = in->rank;
    F16Copies cp(static_cast<hipStream_t>(stream));
    m3_step_inputs li = *in;
    li.dtype = M3_F32;
    li.x = cp.add(in->x, bh * P * R, true, false);
    li.b = cp.add(in->b, bh * N * R, true, false);
    li.c = cp.add(in->c, bh * N * R, true, false);
    li.theta = cp.add(in->theta, bh * (N / 2), true, false);
    float *y32 = cp.add(y, bh * P * R, false, true);
    m3_ssm_state_factored lf{};
    if (fst != nullptr) {
        lf = *fst;
        lf.x_prev = cp.add(fst->x_prev, bh * P * R, true, true);
        lf.b_prev = cp.add(fst->b_prev, bh * N * R, true, true);
    }
    if (cp.error() != hipSuccess) return hip_fail(cp.error(), "f16 copies");
    m3::StepLaunch a;
    bool empty = false;
    const m3_status st = build_step(&li, state, fst ? &lf : nullptr, y32, a, &empty);
    if (st != M3_OK || empty) return st;
    hipError_t e = m3::launch_step(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "step launch");
    g_launches.fetch_add(1, std::memory_order_relaxed);
    if (cp.narrow() != hipSuccess) return hip_fail(cp.error(), "f16 narrowing");
    return ok();
}

}  // namespace

extern "C" {

m3_status m3_step(const m3_step_inputs *in, m3_ssm_state *state, void *y, void *stream) {
    m3::StepLaunch a;
    bool empty = false;
    if (state == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/state are NULL");
    const m3_status st = build_step(in, state, nullptr, y, a, &empty);
    if (st != M3_OK || empty) return st;
    if (in->dtype == M3_F16) return step_f16(in, state, nullptr, y, stream);
    hipError_t e = m3::launch_step(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "step launch");
    g_launches.fetch_add(1, std::memory_order_relaxed);
    return ok();
}

m3_status m3_step_factored(const m3_step_inputs *in, m3_ssm_state_factored *state, void *y,
                           void *stream) {
    m3::StepLaunch a;
    bool empty = false;
    if (state == nullptr) return fail(M3_ERR_ARGUMENT, "inputs/state are NULL");
    const m3_status st = build_step(in, nullptr, state, y, a, &empty);
    if (st != M3_OK || empty) return st;
    if (in->dtype == M3_F16) return step_f16(in, nullptr, state, y, stream);
    hipError_t e = m3::launch_step(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "step launch");
    g_launches.fetch_add(1, std::memory_order_relaxed);
    return ok();
}

m3_status m3_state_unfactor(size_t batch, size_t heads, size_t head_dim, size_t d_state,
                            size_t rank, int32_t dtype, const void *x_prev, const void *b_prev,
                            const float *angle, float *last_u, void *stream) {
    if (!dtype_ok(dtype)) return fail(M3_ERR_ARGUMENT, "unknown dtype %d", dtype);
    if (head_dim == 0 || d_state == 0 || rank == 0)
        return fail(M3_ERR_CONFIG, "SSM dimensions must all be positive");
    const bool f16 = dtype == M3_F16;
    if (angle != nullptr && d_state % 2 != 0)
        return fail(M3_ERR_CONFIG, "rotational dynamics require an even d_state");
    if ((d_state + head_dim) * rank > 16384)
        return fail(M3_ERR_UNSUPPORTED, "d_state/head_dim/rank too large for the step kernel");
    if (batch * heads == 0) return ok();
    if (x_prev == nullptr || b_prev == nullptr || last_u == nullptr)
        return fail(M3_ERR_ARGUMENT, "x_prev, b_prev and last_u are required");
    // f16: the f32 form on widened copies of x_prev and b_prev
    F16Copies cp(static_cast<hipStream_t>(stream));
    if (f16) {
        x_prev = cp.add(x_prev, batch * heads * head_dim * rank, true, false);
        b_prev = cp.add(b_prev, batch * heads * d_state * rank, true, false);
        if (cp.error() != hipSuccess) return hip_fail(cp.error(), "f16 copies");
    }
    hipError_t e = m3::launch_unfactor(batch, heads, head_dim, d_state, rank, dtype == M3_BF16,
                                       x_prev, b_prev, angle, last_u,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "unfactor launch");
    g_launches.fetch_add(1, std::memory_order_relaxed);
    return ok();
}

m3_status m3_step_layers(size_t n_layers, const m3_step_inputs *inputs, m3_ssm_state *states,
                         m3_ssm_state_factored *factored, void *const *ys, void *stream) {
    if (n_layers == 0) return ok();
    if (inputs == nullptr || ys == nullptr || (states == nullptr) == (factored == nullptr))
        return fail(M3_ERR_ARGUMENT, "m3_step_layers needs inputs, ys and exactly one of "
                    "states / factored");
    m3::StepLaunch base{};
    m3::StepLayerTable table{};
    size_t n = 0;
    for (size_t l = 0; l < n_layers; ++l) {
        const m3_step_inputs &in = inputs[l];
        const m3_step_inputs &in0 = inputs[0];
        if (in.batch != in0.batch || in.heads != in0.heads || in.head_dim != in0.head_dim ||
            in.d_state != in0.d_state || in.rank != in0.rank || in.dtype != in0.dtype ||
            (in.theta == nullptr) != (in0.theta == nullptr) ||
            (in.d_skip == nullptr) != (in0.d_skip == nullptr))
            return fail(M3_ERR_SHAPE, "layer %zu's shapes, dtype or theta / d_skip presence differ "
                        "from layer 0's", l);
        if (!m3::step_layers_supported(in.d_state, in.rank))
            return fail(M3_ERR_UNSUPPORTED, "m3_step_layers covers d_state a multiple of 4 with "
                        "d_state/4 a power of two up to 64 and rank 1, 2, 3, 4 or 8");
        if (in.dtype == M3_F16)
            return fail(M3_ERR_UNSUPPORTED, "m3_step_layers covers f32 and bf16 storage: step "
                        "f16 layers with m3_step");
    }
    // every layer's arguments are validated before the first launch, so an
    // error leaves no layer of the cache stepped
    for (size_t l = 0; l < n_layers; ++l) {
        m3::StepLaunch a;
        bool empty = false;
        const m3_status st = build_step(&inputs[l], states ? &states[l] : nullptr,
                                        factored ? &factored[l] : nullptr, ys[l], a, &empty);
        if (st != M3_OK) return st;
        if (empty) return ok();
    }
    for (size_t l = 0; l < n_layers; ++l) {
        m3::StepLaunch a;
        bool empty = false;
        const m3_status st = build_step(&inputs[l], states ? &states[l] : nullptr,
                                        factored ? &factored[l] : nullptr, ys[l], a, &empty);
        if (st != M3_OK) return st;
        if (n == 0) base = a;
        m3::StepLayer &L = table.layer[n++];
        L.x = a.x;
        L.b = a.b;
        L.c = a.c;
        L.dt = a.dt;
        L.lambda = a.lambda;
        L.a_log = a.a_log;
        L.theta = a.theta;
        L.d_skip = a.d_skip;
        L.h = a.h;
        L.last_u = a.last_u;
        L.angle = a.angle;
        L.y = a.y;
        L.x_prev = a.x_prev;
        L.b_prev = a.b_prev;
        if (n == m3::kStepLayersPerLaunch || l + 1 == n_layers) {
            hipError_t e = m3::launch_step_layers(base, table, n, static_cast<hipStream_t>(stream));
            if (e != hipSuccess) return hip_fail(e, "step launch");
            g_launches.fetch_add(1, std::memory_order_relaxed);
            n = 0;
        }
    }
    return ok();
}

const char *m3_status_string(m3_status s) {
    switch (s) {
        case M3_OK: return "M3_OK";
        case M3_ERR_CONFIG: return "M3_ERR_CONFIG";
        case M3_ERR_SHAPE: return "M3_ERR_SHAPE";
        case M3_ERR_RANK: return "M3_ERR_RANK";
        case M3_ERR_UNSUPPORTED: return "M3_ERR_UNSUPPORTED";
        case M3_ERR_HIP: return "M3_ERR_HIP";
        case M3_ERR_ARGUMENT: return "M3_ERR_ARGUMENT";
        case M3_ERR_STATE_DICT: return "M3_ERR_STATE_DICT";
        case M3_ERR_IO: return "M3_ERR_IO";
        case M3_ERR_JSON: return "M3_ERR_JSON";
    }
    return "M3_UNKNOWN";
}

const char *m3_last_error(void) { return g_last_error.c_str(); }

uint64_t m3_launch_count(void) { return g_launches.load(std::memory_order_relaxed); }

m3_status m3_selftest_mfma(int32_t *result) {
    if (result == nullptr) return fail(M3_ERR_ARGUMENT, "result pointer is NULL");
    int r = -1;
    hipError_t e = m3::launch_mfma_selftest(&r);
    if (e != hipSuccess) return hip_fail(e, "mfma self test");
    *result = r;
    return ok();
}

}  // extern "C"
