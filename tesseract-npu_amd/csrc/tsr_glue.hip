// tsr_glue.hip -- host side of the decode-layer glue ops: argument checks and launches behind
// the C ABI of include/tsr_hip.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

#include "kernels.hpp"
#include "runtime.hpp"
#include "tsr_hip.h"

namespace {

constexpr uint32_t kRopeMaxDims = 1024u;    // the angle tables of k_rope hold n_dims / 2 <= 512

// Rows of n floats stride apart do not overlap (a single row needs no stride).
bool rows_ok(uint32_t n, uint32_t rows, uint64_t stride) { return rows <= 1u || stride >= n; }

hipStream_t enter(tsr_hip_ctx * ctx, void * stream) {
    (void)hipSetDevice(ctx->device);
    return ctx->pick(stream);
}

}  // namespace

int tsr_hip_rms_norm(tsr_hip_ctx * ctx, const float * x_dev, uint32_t n, uint32_t rows, uint64_t x_stride, float eps,
                     const float * w_dev, uint64_t w_stride, uint32_t w_period, float * y_dev, uint64_t y_stride,
                     void * stream) {
    if (ctx == nullptr || x_dev == nullptr || y_dev == nullptr || n == 0u || rows == 0u) return TSR_HIP_E_ARG;
    if (!rows_ok(n, rows, x_stride) || !rows_ok(n, rows, y_stride)) return TSR_HIP_E_ARG;
    if (w_dev != nullptr && (w_period == 0u || !rows_ok(n, w_period, w_stride))) return TSR_HIP_E_ARG;
    if (n > (1u << 24)) return TSR_HIP_E_SHAPE;                     // 1 / n from an exact float n
    const float inv_n = 1.0f / (float)n;                             // correctly rounded (IEEE division)
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_rms_norm(x_dev, x_stride, n, rows, eps, inv_n, w_dev, w_stride, w_period, y_dev, y_stride, s);
}

int tsr_hip_rope(tsr_hip_ctx * ctx, const float * x_dev, uint32_t T, uint64_t x_stride, uint32_t head_dim,
                 uint32_t n_heads, uint32_t n_dims, int mode, const int32_t * pos_dev, float freq_base, float freq_scale,
                 float attn_factor, const float * freq_factors_dev, float * y_dev, uint64_t y_stride, void * stream) {
    if (ctx == nullptr || x_dev == nullptr || y_dev == nullptr || pos_dev == nullptr || T == 0u || n_heads == 0u)
        return TSR_HIP_E_ARG;
    if (mode != TSR_HIP_ROPE_NORMAL && mode != TSR_HIP_ROPE_NEOX && mode != TSR_HIP_ROPE_IMROPE) return TSR_HIP_E_SHAPE;
    if (n_dims < 2u || n_dims % 2u != 0u || n_dims > head_dim || n_dims > kRopeMaxDims) return TSR_HIP_E_SHAPE;
    if (T > 0x7FFFFFFFu || n_heads > 65535u * 8u) return TSR_HIP_E_SHAPE;
    const uint64_t width = (uint64_t)head_dim * n_heads;
    if (T > 1u && (x_stride < width || y_stride < width)) return TSR_HIP_E_ARG;
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base)) return TSR_HIP_E_ARG;
    tsr::RopeArgs a{};
    a.x = x_dev;
    a.x_stride = x_stride;
    a.y = y_dev;
    a.y_stride = y_stride;
    a.pos = pos_dev;
    a.ff = freq_factors_dev;
    a.head_dim = head_dim;
    a.n_heads = n_heads;
    a.n_dims = n_dims;
    a.neox = mode != TSR_HIP_ROPE_NORMAL ? 1u : 0u;
    a.ts = powf(freq_base, -2.0f / (float)n_dims);                  // the host libm, as ggml-cpu's theta_scale
    a.m = attn_factor;
    a.freq_scale = freq_scale;
    a.fs = freq_scale != 1.0f ? 1u : 0u;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_rope(a, T, s);
}

int tsr_hip_rope_table(tsr_hip_ctx * ctx, const int32_t * pos_dev, uint32_t n_dims, float freq_base, float attn_factor,
                       float * tab_dev, void * stream) {
    if (ctx == nullptr || pos_dev == nullptr || tab_dev == nullptr || ((uintptr_t)tab_dev & 7u) != 0u) return TSR_HIP_E_ARG;
    if (n_dims < 2u || n_dims % 2u != 0u || n_dims > 128u) return TSR_HIP_E_SHAPE;
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base)) return TSR_HIP_E_ARG;
    const float ts = powf(freq_base, -2.0f / (float)n_dims);       // the host libm, as tsr_hip_rope
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_rope_table(pos_dev, n_dims / 2u, ts, attn_factor, tab_dev, s);
}

int tsr_hip_swiglu(tsr_hip_ctx * ctx, const float * g_dev, uint64_t g_stride, const float * u_dev, uint64_t u_stride,
                   uint32_t n, uint32_t rows, float * y_dev, uint64_t y_stride, void * stream) {
    if (ctx == nullptr || g_dev == nullptr || u_dev == nullptr || y_dev == nullptr || n == 0u || rows == 0u)
        return TSR_HIP_E_ARG;
    if (!rows_ok(n, rows, g_stride) || !rows_ok(n, rows, u_stride) || !rows_ok(n, rows, y_stride)) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_swiglu(g_dev, g_stride, u_dev, u_stride, y_dev, y_stride, n, rows, ctx->expk, s);
}

int tsr_hip_add(tsr_hip_ctx * ctx, const float * a_dev, uint64_t a_stride, const float * b_dev, uint64_t b_stride,
                uint32_t b_period, uint32_t n, uint32_t rows, float * y_dev, uint64_t y_stride, void * stream) {
    if (ctx == nullptr || a_dev == nullptr || b_dev == nullptr || y_dev == nullptr || n == 0u || rows == 0u ||
        b_period == 0u)
        return TSR_HIP_E_ARG;
    if (!rows_ok(n, rows, a_stride) || !rows_ok(n, b_period, b_stride) || !rows_ok(n, rows, y_stride))
        return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_add(a_dev, a_stride, b_dev, b_stride, b_period, y_dev, y_stride, n, rows, s);
}

int tsr_hip_get_rows(tsr_hip_ctx * ctx, const float * src_dev, uint64_t src_stride, uint32_t n, uint32_t n_src,
                     const int32_t * ids_dev, uint32_t count, float * y_dev, uint64_t y_stride, int32_t * bad_dev,
                     void * stream) {
    if (ctx == nullptr || src_dev == nullptr || ids_dev == nullptr || y_dev == nullptr || n == 0u || n_src == 0u ||
        count == 0u)
        return TSR_HIP_E_ARG;
    if (!rows_ok(n, n_src, src_stride) || !rows_ok(n, count, y_stride)) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_get_rows(src_dev, src_stride, n, n_src, ids_dev, count, y_dev, y_stride, ctx->flag(bad_dev), s);
}

int tsr_hip_argmax(tsr_hip_ctx * ctx, const float * x_dev, uint32_t n, uint32_t rows, uint64_t x_stride,
                   int32_t * out_dev, void * stream) {
    if (ctx == nullptr || x_dev == nullptr || out_dev == nullptr || n == 0u || rows == 0u) return TSR_HIP_E_ARG;
    if (!rows_ok(n, rows, x_stride) || n > 0x7FFFFFFFu || rows > 0x7FFFFFFFu) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = enter(ctx, stream);
    return tsr_launch_argmax(x_dev, x_stride, n, rows, out_dev, ctx->am_part(), s);
}
