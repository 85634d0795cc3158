// C ABI of the mixer and language-model operations (include/mamba3_mixer.h):
// argument checks and dispatch.  Errors go through the library's error
// channel (m3_last_error).
#include "mamba3_mixer.h"

#include <hip/hip_runtime.h>

#include <cstdarg>

#include "m3_internal.hpp"

namespace m3 {
m3_status api_fail(m3_status st, const char *fmt, ...);
m3_status api_ok();
m3_status api_hip_fail(hipError_t e, const char *what);
void count_launches(uint64_t n);
}  // namespace m3

namespace {

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

bool lambda_learned(int32_t d) { return d == M3_LEARNED_TRAPEZOID; }

m3_status launched(hipError_t e, const char *what, uint64_t n = 1) {
    if (e != hipSuccess) return m3::api_hip_fail(e, what);
    m3::count_launches(n);
    return m3::api_ok();
}

}  // namespace

extern "C" {

m3_status m3_rms_norm(size_t rows, size_t dim, const void *x, size_t x_stride, const float *weight,
                      float eps, void *y, size_t y_stride, void *stream) {
    if (rows > 0 && (x == nullptr || y == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "rms_norm buffers are NULL");
    if (dim == 0) return m3::api_fail(M3_ERR_SHAPE, "RmsNorm over an empty axis");
    if (x_stride < dim || y_stride < dim)
        return m3::api_fail(M3_ERR_SHAPE, "row strides (%zu, %zu) are shorter than the row (%zu)",
                            x_stride, y_stride, dim);
    if (!(eps >= 0.0f)) return m3::api_fail(M3_ERR_CONFIG, "RmsNorm eps must be non-negative");
    return launched(m3::launch_rms_norm(rows, dim, x, x_stride, weight, eps, y, y_stride,
                                        as_stream(stream)),
                    "rms_norm launch");
}

m3_status m3_quantize_int8_columns(size_t in_features, size_t out_features, const float *w,
                                   void *codes, float *scales, void *stream) {
    if (in_features == 0 || out_features == 0)
        return m3::api_fail(M3_ERR_SHAPE, "quantizing an empty weight [%zu, %zu]", in_features,
                            out_features);
    if (w == nullptr || codes == nullptr || scales == nullptr)
        return m3::api_fail(M3_ERR_ARGUMENT, "quantization buffers are NULL");
    return launched(m3::launch_quantize_columns(in_features, out_features, w, codes, scales,
                                                as_stream(stream)),
                    "quantize launch");
}

size_t m3_linear_workspace_bytes(void) { return m3::kLinearWorkspace; }

namespace {
m3_status linear_call(size_t m, size_t k, size_t n, const void *x, const void *w, bool wt,
                      const float *col_scale, const void *residual, void *y, void *workspace,
                      size_t workspace_bytes, void *stream) {
    if (k == 0) return m3::api_fail(M3_ERR_SHAPE, "Linear with zero input features");
    if (m > 0 && n > 0 && (x == nullptr || w == nullptr || y == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "linear buffers are NULL");
    if (workspace != nullptr && (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return m3::api_fail(M3_ERR_ARGUMENT, "linear workspace must be 256-byte aligned");
    const size_t ws = workspace ? (workspace_bytes < m3::kLinearWorkspace ? workspace_bytes
                                                                           : m3::kLinearWorkspace)
                                : 0;
    const hipError_t e = m3::launch_linear(m, k, n, x, w, wt, col_scale, residual, y, workspace,
                                           ws, as_stream(stream));
    if (e == hipErrorNotSupported)
        return m3::api_fail(M3_ERR_UNSUPPORTED, "no hipBLASLt kernel for a [%zu x %zu] @ [%zu x %zu] "
                            "bf16 product", m, k, k, n);
    return launched(e, "linear launch");
}
}  // namespace

m3_status m3_linear(size_t m, size_t k, size_t n, const void *x, const void *w,
                    const float *col_scale, const void *residual, void *y, void *workspace,
                    size_t workspace_bytes, void *stream) {
    return linear_call(m, k, n, x, w, false, col_scale, residual, y, workspace, workspace_bytes,
                       stream);
}

m3_status m3_linear_nt(size_t m, size_t k, size_t n, const void *x, const void *w_t,
                       const float *col_scale, const void *residual, void *y, void *workspace,
                       size_t workspace_bytes, void *stream) {
    return linear_call(m, k, n, x, w_t, true, col_scale, residual, y, workspace, workspace_bytes,
                       stream);
}

size_t m3_mixer_in_proj_width(const m3_mixer_dims *d) {
    if (d == nullptr) return 0;
    const size_t din = d->heads * d->head_dim * d->rank;
    const size_t bc = d->groups * d->d_state * d->rank;
    return 2 * din + 2 * bc + d->heads + (lambda_learned(d->discretization) ? d->heads : 0) +
           (d->dynamics == M3_ROTATIONAL ? d->heads * d->d_state / 2 : 0);
}

namespace {

bool ranges_overlap(const void *p, const void *q, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
    return a < b + bytes && b < a + bytes;
}

}  // namespace

m3_status m3_mixer_prologue(const m3_mixer_dims *d, const void *projected, const float *dt_bias,
                            const float *b_bias, const float *c_bias, const float *bc_norm,
                            void *x, void *b, void *c, float *dt, float *lambda, void *theta,
                            void *stream) {
    return m3_mixer_prologue_conv(d, nullptr, projected, dt_bias, b_bias, c_bias, bc_norm, x, b, c,
                                  dt, lambda, theta, stream);
}

m3_status m3_mixer_prologue_conv(const m3_mixer_dims *d, const m3_conv1d *conv,
                                 const void *projected, const float *dt_bias,
                                 const float *b_bias, const float *c_bias, const float *bc_norm,
                                 void *x, void *b, void *c, float *dt, float *lambda, void *theta,
                                 void *stream) {
    if (d == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "mixer dims are NULL");
    if (d->heads == 0 || d->head_dim == 0 || d->d_state == 0 || d->rank == 0 || d->groups == 0)
        return m3::api_fail(M3_ERR_CONFIG, "heads, head_dim, d_state, rank and groups must be positive");
    if (d->heads % d->groups != 0)   // config.rs:207-212
        return m3::api_fail(M3_ERR_CONFIG, "n_heads (%zu) must be a multiple of n_groups (%zu)",
                            d->heads, d->groups);
    const bool rot = d->dynamics == M3_ROTATIONAL;
    if (rot && d->d_state % 2 != 0)
        return m3::api_fail(M3_ERR_CONFIG, "rotational dynamics need an even d_state, got %zu",
                            d->d_state);
    if (conv != nullptr) {
        if (conv->kernel_size < 2)   // config.rs:237-243
            return m3::api_fail(M3_ERR_CONFIG, "conv_kernel must be at least 2, got %zu",
                                conv->kernel_size);
        if (conv->seq_len == 0 || d->tokens % conv->seq_len != 0)
            return m3::api_fail(M3_ERR_SHAPE, "tokens (%zu) must be a whole number of sequences "
                                "of seq_len %zu", d->tokens, conv->seq_len);
        if (conv->weight == nullptr)
            return m3::api_fail(M3_ERR_ARGUMENT, "convolution weight is NULL");
        const size_t channels = d->heads * d->head_dim * d->rank + 2 * d->groups * d->d_state * d->rank;
        const size_t hist_bytes = (d->tokens / conv->seq_len) * (conv->kernel_size - 1) * channels * 2;
        if (conv->history != nullptr && conv->new_history != nullptr &&
            ranges_overlap(conv->history, conv->new_history, hist_bytes) &&
            !(conv->history == conv->new_history && conv->seq_len == 1))
            return m3::api_fail(M3_ERR_ARGUMENT, "the new convolution history may overlap the "
                                "history only as the same buffer with seq_len 1, got seq_len %zu",
                                conv->seq_len);
    }
    if (d->tokens == 0) return m3::api_ok();
    if (projected == nullptr || dt_bias == nullptr || x == nullptr || b == nullptr || c == nullptr ||
        dt == nullptr || lambda == nullptr)
        return m3::api_fail(M3_ERR_ARGUMENT, "prologue buffers are NULL");
    const bool learned = lambda_learned(d->discretization);
    const float fixed = m3_discretization_fixed_lambda(d->discretization);
    if (!learned && !(fixed == fixed))
        return m3::api_fail(M3_ERR_CONFIG, "unknown discretization %d", d->discretization);
    m3::PrologueLaunch a{};
    a.tokens = d->tokens;
    a.heads = d->heads;
    a.head_dim = d->head_dim;
    a.d_state = d->d_state;
    a.rank = d->rank;
    a.groups = d->groups;
    a.width = m3_mixer_in_proj_width(d);
    a.learned_lambda = learned ? 1 : 0;
    a.fixed_lambda = learned ? 0.0f : fixed;
    a.has_theta = rot && theta != nullptr ? 1 : 0;   // NULL: theta stays in the row
    a.norm_eps = d->norm_eps;
    a.projected = projected;
    a.dt_bias = dt_bias;
    a.b_bias = b_bias;
    a.c_bias = c_bias;
    a.bc_norm = bc_norm;
    a.x = x;
    a.b = b;
    a.c = c;
    a.dt = dt;
    a.lambda = lambda;
    a.theta = theta;
    if (conv != nullptr) {
        a.conv_k = conv->kernel_size;
        a.seq_len = conv->seq_len;
        a.conv_w = conv->weight;
        a.conv_b = conv->bias;
        a.hist = conv->history;
        a.new_hist = conv->new_history;
    }
    return launched(m3::launch_mixer_prologue(a, as_stream(stream)), "prologue launch");
}

m3_status m3_mixer_gate(size_t tokens, size_t d_inner, const void *y, const void *z,
                        size_t z_stride, const float *norm_weight, float eps, void *out,
                        void *stream) {
    if (d_inner == 0) return m3::api_fail(M3_ERR_SHAPE, "gate over an empty row");
    if (z_stride < d_inner)
        return m3::api_fail(M3_ERR_SHAPE, "z stride %zu is shorter than d_inner %zu", z_stride, d_inner);
    if (tokens > 0 && (y == nullptr || z == nullptr || out == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "gate buffers are NULL");
    return launched(m3::launch_mixer_gate(tokens, d_inner, y, z, z_stride, norm_weight, eps, out,
                                          as_stream(stream)),
                    "gate launch");
}

namespace {

// m3_mixer_step and m3_mixer_step_conv: the checks, then one launch (and the
// gate with the post-gate norm after it when there is one).
m3_status mixer_step_call(const m3_mixer_dims *d, const m3_conv1d *conv, const void *projected,
                          const float *dt_bias, const float *b_bias, const float *c_bias,
                          const float *bc_norm, const float *a_log, const float *d_skip,
                          const float *post_norm_weight, float post_norm_eps,
                          m3_ssm_state *state, m3_ssm_state_factored *factored, void *out,
                          void *stream) {
    const char *fn = conv || post_norm_weight ? "m3_mixer_step_conv" : "m3_mixer_step";
    if (d == nullptr) return m3::api_fail(M3_ERR_ARGUMENT, "mixer dims are NULL");
    if ((state == nullptr) == (factored == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "%s needs exactly one of state / factored", fn);
    if (d->heads == 0 || d->head_dim == 0 || d->d_state == 0 || d->rank == 0 || d->groups == 0)
        return m3::api_fail(M3_ERR_CONFIG, "heads, head_dim, d_state, rank and groups must be positive");
    if (d->heads % d->groups != 0)   // config.rs:207-212
        return m3::api_fail(M3_ERR_CONFIG, "n_heads (%zu) must be a multiple of n_groups (%zu)",
                            d->heads, d->groups);
    const bool rot = d->dynamics == M3_ROTATIONAL;
    if (rot && d->d_state % 2 != 0)
        return m3::api_fail(M3_ERR_CONFIG, "rotational dynamics need an even d_state, got %zu",
                            d->d_state);
    const bool learned = lambda_learned(d->discretization);
    const float fixed = m3_discretization_fixed_lambda(d->discretization);
    if (!learned && !(fixed == fixed))
        return m3::api_fail(M3_ERR_CONFIG, "unknown discretization %d", d->discretization);
    const size_t width = m3_mixer_in_proj_width(d);
    if (!m3::mixer_step_supported(d->head_dim, d->d_state, d->rank, width))
        return m3::api_fail(M3_ERR_UNSUPPORTED, "%s covers d_state a multiple of 8 up to "
                            "128 with d_state/8 a power of two, head_dim*rank a multiple of 8 up "
                            "to 512 and rank 1, 2, 4 or 8; compose m3_mixer_prologue(_conv), "
                            "m3_step and m3_mixer_gate", fn);
    auto al16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const size_t din = d->heads * d->head_dim * d->rank;
    if (conv != nullptr) {
        if (conv->kernel_size < 2)   // config.rs:237-243
            return m3::api_fail(M3_ERR_CONFIG, "conv_kernel must be at least 2, got %zu",
                                conv->kernel_size);
        if (conv->kernel_size > m3::kMixerStepConvTaps)
            return m3::api_fail(M3_ERR_UNSUPPORTED, "%s holds up to %zu convolution taps, got "
                                "conv_kernel %zu: compose m3_mixer_prologue_conv, m3_step and "
                                "m3_mixer_gate", fn, m3::kMixerStepConvTaps, conv->kernel_size);
        if (conv->seq_len != 1)
            return m3::api_fail(M3_ERR_SHAPE, "%s steps one position per sequence (seq_len 1), "
                                "got seq_len %zu", fn, conv->seq_len);
        if (conv->weight == nullptr)
            return m3::api_fail(M3_ERR_ARGUMENT, "convolution weight is NULL");
        if (!al16(conv->weight) || !al16(conv->bias) || !al16(conv->history) ||
            !al16(conv->new_history))
            return m3::api_fail(M3_ERR_ARGUMENT, "the convolution weight, bias and histories must "
                                "be 16-byte aligned");
        const size_t channels = din + 2 * d->groups * d->d_state * d->rank;
        const size_t hist_bytes = d->tokens * (conv->kernel_size - 1) * channels * 2;
        const bool in_place = conv->history != nullptr && conv->history == conv->new_history;
        if (in_place && d->groups != d->heads)
            return m3::api_fail(M3_ERR_UNSUPPORTED, "%s updates the history in place only "
                                "with n_groups == n_heads (got %zu groups of %zu heads): "
                                "pass a separate new_history or compose the calls", fn,
                                d->groups, d->heads);
        if (!in_place && conv->history != nullptr && conv->new_history != nullptr &&
            ranges_overlap(conv->history, conv->new_history, hist_bytes))
            return m3::api_fail(M3_ERR_ARGUMENT, "the new convolution history overlaps the "
                                "history without being the same buffer");
    }
    if (post_norm_weight != nullptr && !(post_norm_eps >= 0.0f))
        return m3::api_fail(M3_ERR_CONFIG, "RmsNorm eps must be non-negative");
    if (d->tokens == 0) return m3::api_ok();
    float *h = state ? state->h : factored->h;
    float *angle = state ? state->angle : factored->angle;
    if (projected == nullptr || dt_bias == nullptr || a_log == nullptr || out == nullptr ||
        h == nullptr || (state && state->last_u == nullptr) ||
        (factored && (factored->x_prev == nullptr || factored->b_prev == nullptr)))
        return m3::api_fail(M3_ERR_ARGUMENT, "mixer step buffers are NULL");
    if (rot && angle == nullptr)
        return m3::api_fail(M3_ERR_ARGUMENT, "rotational dynamics need the state's angle buffer "
                            "(updated in place)");
    if (!al16(projected) || !al16(out) || !al16(h) || (state && !al16(state->last_u)) ||
        (b_bias && !al16(b_bias)) || (c_bias && !al16(c_bias)) || (bc_norm && !al16(bc_norm)))
        return m3::api_fail(M3_ERR_ARGUMENT, "projected, out, the state and the bias / norm "
                            "vectors must be 16-byte aligned");
    m3::MixerStepLaunch m{};
    m3::StepLaunch &a = m.s;
    a.batch = d->tokens;
    a.heads = d->heads;
    a.head_dim = d->head_dim;
    a.d_state = d->d_state;
    a.rank = d->rank;
    a.bf16 = 1;
    a.a_log = a_log;
    a.d_skip = d_skip;
    a.theta = rot ? projected : nullptr;   // presence only: theta comes from the projection row
    a.h = h;
    a.last_u = state ? state->last_u : nullptr;
    a.angle = rot ? angle : nullptr;
    a.x_prev = factored ? factored->x_prev : nullptr;
    a.b_prev = factored ? factored->b_prev : nullptr;
    m.groups = d->groups;
    m.width = width;
    m.learned_lambda = learned ? 1 : 0;
    m.fixed_lambda = learned ? 0.0f : fixed;
    m.norm_eps = d->norm_eps;
    m.projected = projected;
    m.dt_bias = dt_bias;
    m.b_bias = b_bias;
    m.c_bias = c_bias;
    m.bc_norm = bc_norm;
    m.out = out;
    m.gate = post_norm_weight == nullptr ? 1 : 0;
    if (conv != nullptr) {
        m.conv_k = conv->kernel_size;
        m.conv_w = conv->weight;
        m.conv_b = conv->bias;
        m.hist = conv->history;
        m.new_hist = conv->new_history;
    }
    const m3_status st = launched(m3::launch_mixer_step(m, as_stream(stream)), "mixer step launch");
    if (st != M3_OK || post_norm_weight == nullptr) return st;
    // the post-gate norm spans every head of a row: the gate runs on y in place
    return launched(m3::launch_mixer_gate(d->tokens, din, out, projected, width, post_norm_weight,
                                          post_norm_eps, out, as_stream(stream)),
                    "gate launch");
}

}  // namespace

m3_status m3_mixer_step(const m3_mixer_dims *d, const void *projected, const float *dt_bias,
                        const float *b_bias, const float *c_bias, const float *bc_norm,
                        const float *a_log, const float *d_skip, m3_ssm_state *state,
                        m3_ssm_state_factored *factored, void *out, void *stream) {
    return mixer_step_call(d, nullptr, projected, dt_bias, b_bias, c_bias, bc_norm, a_log, d_skip,
                           nullptr, 0.0f, state, factored, out, stream);
}

m3_status m3_mixer_step_conv(const m3_mixer_dims *d, const m3_conv1d *conv, const void *projected,
                             const float *dt_bias, const float *b_bias, const float *c_bias,
                             const float *bc_norm, const float *a_log, const float *d_skip,
                             const float *post_norm_weight, float post_norm_eps,
                             m3_ssm_state *state, m3_ssm_state_factored *factored, void *out,
                             void *stream) {
    return mixer_step_call(d, conv, projected, dt_bias, b_bias, c_bias, bc_norm, a_log, d_skip,
                           post_norm_weight, post_norm_eps, state, factored, out, stream);
}

m3_status m3_embedding_lookup(size_t n, size_t dim, const int32_t *ids, size_t vocab,
                              const void *table, void *out, void *stream) {
    if (dim == 0 || vocab == 0) return m3::api_fail(M3_ERR_SHAPE, "empty embedding table");
    if (n > 0 && (ids == nullptr || table == nullptr || out == nullptr))
        return m3::api_fail(M3_ERR_ARGUMENT, "embedding buffers are NULL");
    return launched(m3::launch_embedding(n, dim, ids, vocab, table, out, as_stream(stream)),
                    "embedding launch");
}

}  // extern "C"
