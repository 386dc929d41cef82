// tsr_hip.hip -- host side of libtsr_hip: contexts, buffers, the weight layout, argument checks and
// kernel launches behind the C ABI of include/tsr_hip.h.
#include "tsr_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"
#include "wlayout.hpp"

// ---------------------------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------------------------
const char * tsr_hip_strerror(int code) {
    switch (code) {
        case TSR_HIP_OK: return "ok";
        case TSR_HIP_E_ARG: return "invalid argument";
        case TSR_HIP_E_SHAPE: return "unsupported shape";
        case TSR_HIP_E_NOMEM: return "out of memory";
        case TSR_HIP_E_HIP: return "HIP runtime error";
        case TSR_HIP_E_RANGE: return "range beyond the object";
        case TSR_HIP_E_NODEV: return "no such device";
        case TSR_HIP_E_FMT: return "unknown weight format or QA kind";
        case TSR_HIP_E_MASK: return "mask summary malformed or needs the f32 mask copy";
        default: return "unknown error";
    }
}

namespace tsr {

int hip_err(hipError_t e, const char * what) {
    if (e == hipSuccess) return TSR_HIP_OK;
    if (getenv("TSR_HIP_DEBUG")) fprintf(stderr, "tsr_hip: %s: %s\n", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? TSR_HIP_E_NOMEM : TSR_HIP_E_HIP;
}

}  // namespace tsr

using tsr::hip_err;

// EXPK constants from their definitions (long double: 64-bit significand, exact enough for every
// rounding here; VU 6.3 fixes LK = round(log2(e) 2^38), c_k = round(ln2^k / k! 2^32),
// t64[j] = round(2^(j/64) 2^30)).
void tsr_expk_table(tsr::ExpkTab * t) {
    const long double ln2 = 0.693147180559945309417232121458176568L;
    const long double log2e = 1.442695040888963407359924681001892137L;
    t->lk = (uint64_t)llroundl(ldexpl(log2e, 38));
    t->c1 = (uint64_t)llroundl(ldexpl(ln2, 32));
    t->c2 = (uint64_t)llroundl(ldexpl(ln2 * ln2 / 2.0L, 32));
    t->c3 = (uint64_t)llroundl(ldexpl(ln2 * ln2 * ln2 / 6.0L, 32));
    for (int j = 0; j < 64; ++j) t->t64[j] = (uint32_t)llroundl(ldexpl(exp2l((long double)j / 64.0L), 30));
}

// ---------------------------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------------------------
// The dispatcher places consecutive workgroups of a launch on consecutive XCDs (round-robin); the
// one-launch decode FLASH_ATTN_EXT relies on it to keep a KV head's workgroups on one XCD. At open, 64
// workgroups record their XCD: n_xcd is the period of that sequence (gfx950: 32 compute units per XCD,
// so n_cu / 32 XCDs when the whole device is visible). Any other pattern leaves n_xcd = 0 and the
// FLASH_ATTN_EXT on the agent-coherent exchange.
static int xcd_calibrate(tsr_hip_ctx * c) {
    c->n_xcd = 0;
    const uint32_t n = (c->n_cu % 32 == 0 && c->n_cu > 0 && c->n_cu <= 8 * 32) ? (uint32_t)(c->n_cu / 32) : 0u;
    if (n == 0u) return TSR_HIP_OK;
    uint32_t * d = nullptr;
    int rc = hip_err(hipMalloc(&d, 64 * sizeof(uint32_t)), "hipMalloc xcd probe");
    if (rc) return rc;
    uint32_t h[64] = {};
    rc = tsr_launch_xcd_probe(d, c->stream) ? TSR_HIP_E_HIP : 0;
    if (rc == 0) rc = hip_err(hipMemcpyAsync(h, d, sizeof h, hipMemcpyDeviceToHost, c->stream), "xcd probe copy");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(c->stream), "xcd probe sync");
    (void)hipFree(d);
    if (rc) return rc;
    bool ok = true;
    uint32_t seen = 0;
    for (uint32_t i = 0; i < 64; ++i) ok &= h[i] == h[i % n] && h[i] < 16u;
    for (uint32_t i = 0; ok && i < n; ++i) {
        ok &= ((seen >> h[i]) & 1u) == 0u;                        // n distinct XCDs
        seen |= 1u << h[i];
    }
    if (ok) c->n_xcd = n;
    return TSR_HIP_OK;
}
int tsr_hip_open(int device, tsr_hip_ctx ** out) {
    if (out == nullptr) return TSR_HIP_E_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return TSR_HIP_E_NODEV;
    int rc = hip_err(hipSetDevice(device), "hipSetDevice");
    if (rc) return rc;
    auto * c = new (std::nothrow) tsr_hip_ctx();
    if (c == nullptr) return TSR_HIP_E_NOMEM;
    c->device = device;
    hipDeviceProp_t p;
    if ((rc = hip_err(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties")) != 0) { delete c; return rc; }
    c->n_cu = p.multiProcessorCount;
    snprintf(c->name, sizeof c->name, "%s", p.gcnArchName);
    tsr_expk_table(&c->expk);
    if ((rc = hip_err(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate")) != 0) {
        delete c;
        return rc;
    }
    if ((rc = tsr_fa_fixed_init(c)) != 0 ||                       // the device address of the fixed FA array
        (rc = hip_err(hipMalloc((void **)&c->flags_dev, tsr_hip_ctx::kFlagsBytes), "hipMalloc flags")) != 0 ||
        (rc = hip_err(hipMemsetAsync(c->flags_dev, 0, 256, c->stream), "hipMemset flags")) != 0 ||
        (rc = hip_err(hipStreamSynchronize(c->stream), "hipStreamSynchronize")) != 0 ||
        (rc = xcd_calibrate(c)) != 0) {
        if (c->flags_dev) (void)hipFree(c->flags_dev);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return rc;
    }
    *out = c;
    return TSR_HIP_OK;
}

int tsr_hip_close(tsr_hip_ctx * ctx) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    {
        std::lock_guard<std::mutex> lk(ctx->mtx);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        ctx->scratch.release();
        ctx->staging.release();
        if (ctx->flags_dev) (void)hipFree(ctx->flags_dev);
        (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    return TSR_HIP_OK;
}

void * tsr_hip_stream(tsr_hip_ctx * ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int tsr_hip_sync(tsr_hip_ctx * ctx, void * stream) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    return hip_err(hipStreamSynchronize(ctx->pick(stream)), "hipStreamSynchronize");
}

int tsr_hip_get_flags(tsr_hip_ctx * ctx, int32_t * flags, int clear) {
    if (ctx == nullptr || flags == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    if (tsr_capturing(ctx->stream)) return TSR_HIP_E_ARG;
    int32_t v = 0;
    int rc = hip_err(hipMemcpyAsync(&v, ctx->flags_dev, 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy flags");
    if (rc == 0 && clear && (rc = hip_err(hipMemsetAsync(ctx->flags_dev, 0, 4, ctx->stream), "hipMemset flags")) != 0) return rc;
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc == 0) *flags = v;
    return rc;
}

int tsr_hip_device_info(tsr_hip_ctx * ctx, int * n_cu, char * name, size_t name_len, size_t * mem_free,
                        size_t * mem_total) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    if (n_cu) *n_cu = ctx->n_cu;
    if (name && name_len) snprintf(name, name_len, "%s", ctx->name);
    if (mem_free || mem_total) {
        size_t f = 0, t = 0;
        const int rc = hip_err(hipMemGetInfo(&f, &t), "hipMemGetInfo");
        if (rc) return rc;
        if (mem_free) *mem_free = f;
        if (mem_total) *mem_total = t;
    }
    return TSR_HIP_OK;
}

int tsr_hip_get_counters(tsr_hip_ctx * ctx, tsr_hip_counters * out) {
    if (ctx == nullptr || out == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    *out = ctx->ctr;
    return TSR_HIP_OK;
}

// ---------------------------------------------------------------------------------------------
// raw buffers
// ---------------------------------------------------------------------------------------------
int tsr_hip_alloc(tsr_hip_ctx * ctx, size_t bytes, void ** dev_out) {
    if (ctx == nullptr || dev_out == nullptr) return TSR_HIP_E_ARG;
    *dev_out = nullptr;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    return hip_err(hipMalloc(dev_out, bytes ? bytes : 1u), "hipMalloc");
}

int tsr_hip_free(tsr_hip_ctx * ctx, void * dev) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    if (dev == nullptr) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    return hip_err(hipFree(dev), "hipFree");
}

int tsr_hip_write(tsr_hip_ctx * ctx, void * dst_dev, const void * src, size_t bytes) {
    if (ctx == nullptr || (bytes && (dst_dev == nullptr || src == nullptr))) return TSR_HIP_E_ARG;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = hip_err(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy H2D");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return rc;
}

int tsr_hip_write_async(tsr_hip_ctx * ctx, void * dst_dev, const void * src, size_t bytes, void * stream) {
    if (ctx == nullptr || (bytes && (dst_dev == nullptr || src == nullptr))) return TSR_HIP_E_ARG;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    if (tsr_capturing(s)) return TSR_HIP_E_ARG;
    return ctx->staging.copy(dst_dev, src, bytes, s);
}

int tsr_hip_copy_async(tsr_hip_ctx * ctx, void * dst_dev, const void * src_dev, size_t bytes, void * stream) {
    if (ctx == nullptr || (bytes && (dst_dev == nullptr || src_dev == nullptr))) return TSR_HIP_E_ARG;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    return hip_err(hipMemcpyAsync(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, ctx->pick(stream)), "hipMemcpyAsync D2D");
}

int tsr_hip_read(tsr_hip_ctx * ctx, void * dst, const void * src_dev, size_t bytes) {
    if (ctx == nullptr || (bytes && (dst == nullptr || src_dev == nullptr))) return TSR_HIP_E_ARG;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = hip_err(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy D2H");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return rc;
}

int tsr_hip_memset(tsr_hip_ctx * ctx, void * dst_dev, int value, size_t bytes) {
    if (ctx == nullptr || (bytes && dst_dev == nullptr)) return TSR_HIP_E_ARG;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = hip_err(hipMemsetAsync(dst_dev, value, bytes, ctx->stream), "hipMemset");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return rc;
}

// ---------------------------------------------------------------------------------------------
// weights: ggml blocks <-> the device layout of wlayout.hpp (meta region | quant region)
// ---------------------------------------------------------------------------------------------
namespace {

constexpr uint32_t kKMax = 32768u;
constexpr uint32_t kMmMinTokens = 16u;   // MUL_MAT with at least this many tokens runs on the matrix cores
constexpr uint32_t kMmChunk = 4096u;     // tokens per prefill launch pair (bounds the scratch)

uint32_t blk_values(uint32_t fmt) { return fmt == TSR_HIP_FMT_Q8_0 ? 32u : 256u; }
uint32_t blk_bytes(uint32_t fmt) { return fmt == TSR_HIP_FMT_Q8_0 ? 34u : 144u; }

// Q4_K scales: ggml packs eight 6-bit scales sc_j and mins m_j into 12 bytes (get_scale_min_k4,
// sw/sim/tsr_ref.c:359-367). The device keeps the same 96 bits re-arranged so that one bit-field
// extract gives each value: byte j (j < 8) = sc_j | (m_j & 3) << 6, bytes 8-11 = the nibbles
// m_j >> 2 (nibble j at bit 4j). A bijection of the 12 bytes, so weight reads give back the exact
// ggml blocks.
void q4k_meta_encode(const uint8_t * q, uint8_t * e) {
    uint32_t hi = 0;
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        if (j < 4) { sc = q[j] & 63; m = q[j + 4] & 63; }
        else { sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4); m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
        e[j] = (uint8_t)(sc | ((m & 3) << 6));
        hi |= (uint32_t)(m >> 2) << (4 * j);
    }
    for (int k = 0; k < 4; ++k) e[8 + k] = (uint8_t)(hi >> (8 * k));
}

void q4k_meta_decode(const uint8_t * e, uint8_t * q) {
    const uint32_t hi = e[8] | (uint32_t)e[9] << 8 | (uint32_t)e[10] << 16 | (uint32_t)e[11] << 24;
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = e[j] & 63;
        m[j] = (e[j] >> 6) | (int)(((hi >> (4 * j)) & 15u) << 2);
    }
    for (int j = 0; j < 4; ++j) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
}

template <class F>
void parallel_rows(uint32_t N, F && f) {
    const uint32_t nt = std::max(1u, std::min<uint32_t>(16u, std::thread::hardware_concurrency()));
    if (N < 1024u || nt == 1u) { f(0u, N); return; }
    std::vector<std::thread> th;
    const uint32_t per = (N + nt - 1u) / nt;
    for (uint32_t lo = 0; lo < N; lo += per) th.emplace_back(f, lo, std::min(N, lo + per));
    for (auto & x : th) x.join();
}

}  // namespace

int tsr_hip_weight_upload(tsr_hip_ctx * ctx, uint32_t fmt, const void * ggml_blocks, uint32_t N, uint32_t K,
                          tsr_hip_weight ** out) {
    if (ctx == nullptr || ggml_blocks == nullptr || out == nullptr) return TSR_HIP_E_ARG;
    *out = nullptr;
    if (fmt != TSR_HIP_FMT_Q8_0 && fmt != TSR_HIP_FMT_Q4_K) return TSR_HIP_E_FMT;
    if (N == 0u || K == 0u || K % blk_values(fmt) != 0u || K > kKMax) return TSR_HIP_E_SHAPE;
    const uint32_t nb = K / blk_values(fmt);
    const uint32_t rb = tsr_wl_rows_per_block(fmt, N, K, (uint32_t)ctx->n_cu);
    const bool q4k = fmt == TSR_HIP_FMT_Q4_K;
    const tsr::WGeom g = tsr::wgeom(N, nb, rb, q4k);
    std::vector<uint8_t> host;
    try {
        host.assign(tsr::wl_bytes(g), 0u);                      // block padding stays zero
    } catch (...) {
        return TSR_HIP_E_NOMEM;
    }
    const uint8_t * src = (const uint8_t *)ggml_blocks;
    uint8_t * hd = host.data();
    const uint32_t bb = blk_bytes(fmt);
    parallel_rows(N, [&](uint32_t lo, uint32_t hi) {
        for (uint32_t n = lo; n < hi; ++n) {
            const uint32_t B = n / rb, r = n - B * rb, R = tsr::wl_rows(g, B);
            for (uint32_t s = 0; s < nb; ++s) {
                const uint8_t * b = src + ((size_t)n * nb + s) * bb;
                const uint32_t sl = tsr::wl_slot_of(g, s);
                uint8_t * m = hd + tsr::wl_meta_off(g, B, R, sl, r);
                if (q4k) {
                    memcpy(m, b, 4);
                    q4k_meta_encode(b + 4, m + 4);
                    for (uint32_t j = 0; j < 8u; ++j) memcpy(hd + tsr::wl_quant_off(g, B, R, j, sl, r), b + 16u + 16u * j, 16);
                } else {
                    memcpy(m, b, 2);
                    for (uint32_t h = 0; h < 2u; ++h) memcpy(hd + tsr::wl_quant_off(g, B, R, h, sl, r), b + 2u + 16u * h, 16);
                }
            }
        }
    });
    auto * w = new (std::nothrow) tsr_hip_weight();
    if (w == nullptr) return TSR_HIP_E_NOMEM;
    w->fmt = fmt;
    w->N = N;
    w->K = K;
    w->rb = rb;
    w->bytes = host.size();
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = hip_err(hipMalloc((void **)&w->dev, w->bytes), "hipMalloc weight");
    if (rc == 0) rc = hip_err(hipMemcpyAsync(w->dev, host.data(), w->bytes, hipMemcpyHostToDevice, ctx->stream), "weight H2D");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc != 0) {
        if (w->dev) (void)hipFree(w->dev);
        delete w;
        return rc;
    }
    *out = w;
    return TSR_HIP_OK;
}

int tsr_hip_weight_read(tsr_hip_ctx * ctx, const tsr_hip_weight * w, void * ggml_blocks) {
    if (ctx == nullptr || w == nullptr || ggml_blocks == nullptr) return TSR_HIP_E_ARG;
    std::vector<uint8_t> host(w->bytes);
    {
        std::lock_guard<std::mutex> lk(ctx->mtx);
        (void)hipSetDevice(ctx->device);
        int rc = hip_err(hipMemcpyAsync(host.data(), w->dev, w->bytes, hipMemcpyDeviceToHost, ctx->stream), "weight D2H");
        if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (rc) return rc;
    }
    const uint32_t nb = w->K / blk_values(w->fmt), bb = blk_bytes(w->fmt);
    const bool q4k = w->fmt == TSR_HIP_FMT_Q4_K;
    const tsr::WGeom g = tsr::wgeom(w->N, nb, w->rb, q4k);
    const uint8_t * hd = host.data();
    uint8_t * dst = (uint8_t *)ggml_blocks;
    parallel_rows(w->N, [&](uint32_t lo, uint32_t hi) {
        for (uint32_t n = lo; n < hi; ++n) {
            const uint32_t B = n / w->rb, r = n - B * w->rb, R = tsr::wl_rows(g, B);
            for (uint32_t s = 0; s < nb; ++s) {
                uint8_t * b = dst + ((size_t)n * nb + s) * bb;
                const uint32_t sl = tsr::wl_slot_of(g, s);
                const uint8_t * m = hd + tsr::wl_meta_off(g, B, R, sl, r);
                if (q4k) {
                    memcpy(b, m, 4);
                    q4k_meta_decode(m + 4, b + 4);
                    for (uint32_t j = 0; j < 8u; ++j) memcpy(b + 16u + 16u * j, hd + tsr::wl_quant_off(g, B, R, j, sl, r), 16);
                } else {
                    memcpy(b, m, 2);
                    for (uint32_t h = 0; h < 2u; ++h) memcpy(b + 2u + 16u * h, hd + tsr::wl_quant_off(g, B, R, h, sl, r), 16);
                }
            }
        }
    });
    return TSR_HIP_OK;
}

int tsr_hip_weight_free(tsr_hip_ctx * ctx, tsr_hip_weight * w) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    if (w == nullptr) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    const int rc = hip_err(hipFree(w->dev), "hipFree weight");
    delete w;
    return rc;
}

int tsr_hip_weight_info(const tsr_hip_weight * w, uint32_t * fmt, uint32_t * N, uint32_t * K, size_t * dev_bytes) {
    if (w == nullptr) return TSR_HIP_E_ARG;
    if (fmt) *fmt = w->fmt;
    if (N) *N = w->N;
    if (K) *K = w->K;
    if (dev_bytes) *dev_bytes = w->bytes;
    return TSR_HIP_OK;
}

// ---------------------------------------------------------------------------------------------
// QACT
// ---------------------------------------------------------------------------------------------
size_t tsr_hip_qa_bytes(uint32_t kind, uint32_t K) {
    if (kind > 1u) return 0;
    const uint32_t bs = kind == 0u ? 32u : 256u;
    size_t n = (K + 63u) / 64u * 64u + (4u * (K / bs) + 63u) / 64u * 64u;
    if (kind == 1u) n += (2u * (K / 16u) + 63u) / 64u * 64u;
    return n;
}

static bool aligned16(const void * p) { return ((uintptr_t)p & 15u) == 0u; }

int tsr_hip_qact(tsr_hip_ctx * ctx, uint32_t kind, const float * x_dev, uint32_t K, uint32_t T, uint64_t x_stride,
                 uint8_t * qa_dev, void * stream) {
    if (ctx == nullptr || x_dev == nullptr || qa_dev == nullptr || T == 0u) return TSR_HIP_E_ARG;
    if (kind > 1u) return TSR_HIP_E_FMT;
    const uint32_t bs = kind == 0u ? 32u : 256u;
    if (K == 0u || K % bs != 0u || K > kKMax) return TSR_HIP_E_SHAPE;
    if (!aligned16(x_dev) || (T > 1u && x_stride % 4u != 0u) || T > 65535u) return TSR_HIP_E_ARG;
    tsr::QactArgs a{};
    a.x = x_dev;
    a.x_stride = x_stride;
    a.qa = qa_dev;
    a.qa_bytes = (uint32_t)tsr_hip_qa_bytes(kind, K);
    a.K = K;
    a.kind = kind;
    a.d_off = (K + 63u) / 64u * 64u;
    a.bs_off = a.d_off + (4u * (K / bs) + 63u) / 64u * 64u;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    ctx->ctr.qact_calls++;
    return tsr_launch_qact(a, T, ctx->pick(stream));
}

// ---------------------------------------------------------------------------------------------
// MUL_MAT
// ---------------------------------------------------------------------------------------------
// What a fused MUL_MAT applies to x first (tsr_hip_mul_mat_norm).
struct MmPrep {
    uint32_t kind;           // tsr::MvPrep
    const float * pw;        // kPrepNorm: MUL weight (nullable)
    float eps, inv_n;
};

// The caller holds ctx->mtx.
static int mul_mat_locked(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T,
                          uint64_t x_stride, float * y_dev, uint64_t y_stride, const float * add_dev,
                          uint64_t add_stride, uint32_t flags, int32_t * isums, hipStream_t s,
                          const MmPrep * prep = nullptr) {
    if (w == nullptr || x_dev == nullptr || y_dev == nullptr || T == 0u) return TSR_HIP_E_ARG;
    const bool glu = (flags & TSR_HIP_MM_GLU) != 0u;
    if (prep != nullptr || glu) {
        // the fused forms run on the matvec kernels (not the matrix-core prefill shapes); the norm needs
        // the whole row in one round of loads: K <= 8192; GLU pairs whole rows in every row block
        if ((prep != nullptr && w->K > 8192u) || (T >= kMmMinTokens && w->fmt == TSR_HIP_FMT_Q8_0) ||
            (glu && ((w->N & 1u) || (w->rb & 1u))))
            return TSR_HIP_E_SHAPE;
        if (prep != nullptr && prep->pw != nullptr && !aligned16(prep->pw)) return TSR_HIP_E_ARG;
        if (glu && (add_dev != nullptr || (flags & TSR_HIP_MM_ACC_DST) || isums != nullptr)) return TSR_HIP_E_ARG;
    }
    if ((flags & ~(TSR_HIP_MM_ACC_DST | TSR_HIP_MM_GLU)) != 0u || (add_dev != nullptr && (flags & TSR_HIP_MM_ACC_DST)))
        return TSR_HIP_E_ARG;
    if (!aligned16(x_dev) || (T > 1u && x_stride % 4u != 0u)) return TSR_HIP_E_ARG;
    if (T > 1u && (x_stride < w->K || y_stride < (glu ? w->N / 2u : w->N))) return TSR_HIP_E_ARG;
    (void)hipSetDevice(ctx->device);
    tsr::MvArgs a{};
    const size_t nb = w->K / blk_values(w->fmt);
    a.w = w->dev;
    a.rb = w->rb;
    a.x = x_dev;
    a.x_stride = x_stride;
    a.y = y_dev;
    a.y_stride = y_stride;
    a.add = add_dev;
    a.add_stride = add_stride;
    a.isums = isums;
    a.N = w->N;
    a.K = w->K;
    a.acc = (flags & TSR_HIP_MM_ACC_DST) ? 1u : 0u;
    if (prep != nullptr) {
        a.prep = prep->kind;
        a.pw = prep->pw;
        a.eps = prep->eps;
        a.inv_n = prep->inv_n;
    }
    if (glu) {
        a.glu = 1u;
        a.ex = ctx->expk;
    }

    ctx->ctr.mul_mat_calls++;
    ctx->ctr.mul_mat_rows += (uint64_t)w->N * T;
    ctx->ctr.mul_mat_weight_bytes += (uint64_t)w->N * nb * blk_bytes(w->fmt);
    // prefill: T >= 16 tokens of Q8_0 on the matrix cores (QACT A32 of every token into scratch,
    // block-major), at most kMmChunk tokens per launch pair
    if (T >= kMmMinTokens && w->fmt == TSR_HIP_FMT_Q8_0 && isums == nullptr) {
        const uint32_t chunk = std::min(T, kMmChunk), nbx = w->K / 32u;
        const size_t q_bytes = (size_t)chunk * w->K, d_off = (q_bytes + 255u) & ~(size_t)255u;
        int rc = ctx->scratch.reserve(d_off + 4u * (size_t)chunk * nbx, s);
        if (rc) return rc;
        for (uint32_t t0 = 0; t0 < T; t0 += chunk) {
            const uint32_t tt = std::min(T - t0, chunk);
            uint8_t * xq = (uint8_t *)ctx->scratch.ptr;
            if (tsr_launch_qact_mm(x_dev + (size_t)t0 * x_stride, x_stride, w->K, tt, xq, (float *)(xq + d_off), s))
                return TSR_HIP_E_HIP;
            tsr::MmArgs m{};
            m.w = w->dev;
            m.rb = w->rb;
            m.qa = xq;
            m.qa_stride = 0u;
            m.d_off = (uint32_t)d_off;
            m.y = y_dev + (size_t)t0 * y_stride;
            m.y_stride = y_stride;
            m.add = add_dev ? add_dev + (size_t)t0 * add_stride : nullptr;
            m.add_stride = add_stride;
            m.N = w->N;
            m.K = w->K;
            m.T = tt;
            m.acc = a.acc;

            if (tsr_launch_mm_q8_0(m, s)) return TSR_HIP_E_HIP;
        }
        return TSR_HIP_OK;
    }
    // prefill: T >= 16 tokens of Q4_K on the matrix cores (QACT A256 of every token into scratch,
    // block-major), with the GLU epilogue when asked; the fused norm form stays on the matvec kernels
    if (T >= kMmMinTokens && w->fmt == TSR_HIP_FMT_Q4_K && isums == nullptr && prep == nullptr) {
        const uint32_t chunk = std::min(T, kMmChunk), tpc = (chunk + 31u) & ~31u;
        const size_t s_off = ((size_t)chunk * w->K + 255u) & ~(size_t)255u;
        const size_t d_off = (s_off + 4u * (size_t)chunk * (w->K / 32u) + 255u) & ~(size_t)255u;
        int rc = ctx->scratch.reserve(d_off + 4u * (size_t)tpc * (w->K / 256u), s);
        if (rc) return rc;
        for (uint32_t t0 = 0; t0 < T; t0 += chunk) {
            const uint32_t tt = std::min(T - t0, chunk), tp = (tt + 31u) & ~31u;
            uint8_t * xq = (uint8_t *)ctx->scratch.ptr;
            if (tsr_launch_qact_mm4(x_dev + (size_t)t0 * x_stride, x_stride, w->K, tt, tp, xq, (int32_t *)(xq + s_off),
                                    (float *)(xq + d_off), s))
                return TSR_HIP_E_HIP;
            tsr::MmArgs m{};
            m.w = w->dev;
            m.rb = w->rb;
            m.qa = xq;
            m.s_off = (uint32_t)s_off;
            m.d_off = (uint32_t)d_off;
            m.tp = tp;
            m.y = y_dev + (size_t)t0 * y_stride;
            m.y_stride = y_stride;
            m.add = add_dev ? add_dev + (size_t)t0 * add_stride : nullptr;
            m.add_stride = add_stride;
            m.N = w->N;
            m.K = w->K;
            m.T = tt;
            m.acc = a.acc;
            m.glu = a.glu;
            m.ex = a.ex;
            if (tsr_launch_mm_q4_k(m, s)) return TSR_HIP_E_HIP;
        }
        return TSR_HIP_OK;
    }
    for (uint32_t t0 = 0; t0 < T; t0 += 65535u) {
        const uint32_t tt = std::min(T - t0, 65535u);
        a.x = x_dev + (size_t)t0 * x_stride;
        a.y = y_dev + (size_t)t0 * y_stride;
        a.add = add_dev ? add_dev + (size_t)t0 * add_stride : nullptr;
        a.T = tt;
        const int rc = w->fmt == TSR_HIP_FMT_Q8_0 ? tsr_launch_mv_q8_0(a, s) : tsr_launch_mv_q4_k(a, s);
        if (rc) return rc == -2 ? TSR_HIP_E_SHAPE : TSR_HIP_E_HIP;
    }
    return TSR_HIP_OK;
}

int tsr_hip_mul_mat(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T, uint64_t x_stride,
                    float * y_dev, uint64_t y_stride, const float * add_dev, uint64_t add_stride, uint32_t flags,
                    void * stream) {
    if (ctx == nullptr || (flags & (TSR_HIP_MM_SCALE | TSR_HIP_MM_SOFTCAP))) return TSR_HIP_E_ARG;   // _epi has the scales
    std::lock_guard<std::mutex> lk(ctx->mtx);
    return mul_mat_locked(ctx, w, x_dev, T, x_stride, y_dev, y_stride, add_dev, add_stride, flags, nullptr,
                          ctx->pick(stream));
}

int tsr_hip_mul_mat_epi(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T, uint64_t x_stride,
                        float * y_dev, uint64_t y_stride, const float * add_dev, uint64_t add_stride, uint32_t flags,
                        float first_scale, float scale, void * stream) {
    // the MUL_MAT, then one elementwise launch over its T x N result: the MUL_MAT kernels carry no
    // epilogue code (their store tail is on the critical path of every decode launch)
    const uint32_t ef = flags & (TSR_HIP_MM_SCALE | TSR_HIP_MM_SOFTCAP);
    if (ctx == nullptr || w == nullptr || ef == 0u || ef == (TSR_HIP_MM_SCALE | TSR_HIP_MM_SOFTCAP) ||
        (flags & TSR_HIP_MM_GLU))
        return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    const hipStream_t s = ctx->pick(stream);
    int rc = mul_mat_locked(ctx, w, x_dev, T, x_stride, y_dev, y_stride, add_dev, add_stride, flags & ~ef, nullptr, s);
    if (rc) return rc;
    const uint32_t mode = ef == TSR_HIP_MM_SOFTCAP ? tsr::kEpiSoftcap : tsr::kEpiScale;
    for (uint32_t t0 = 0; t0 < T; t0 += 65535u) {
        rc = tsr_launch_mm_epilogue(y_dev + (size_t)t0 * y_stride, y_stride, w->N, std::min(T - t0, 65535u), mode,
                                    first_scale, scale, ctx->expk, s);
        if (rc) return TSR_HIP_E_HIP;
    }
    return TSR_HIP_OK;
}

int tsr_hip_mul_mat_norm(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T,
                         uint64_t x_stride, float eps, const float * norm_w_dev, float * y_dev, uint64_t y_stride,
                         const float * add_dev, uint64_t add_stride, uint32_t flags, void * stream) {
    if (ctx == nullptr || w == nullptr || (flags & (TSR_HIP_MM_SCALE | TSR_HIP_MM_SOFTCAP))) return TSR_HIP_E_ARG;
    MmPrep p{};
    p.kind = tsr::kPrepNorm;
    p.pw = norm_w_dev;
    p.eps = eps;
    p.inv_n = 1.0f / (float)w->K;                                   // correctly rounded (IEEE division)
    std::lock_guard<std::mutex> lk(ctx->mtx);
    return mul_mat_locked(ctx, w, x_dev, T, x_stride, y_dev, y_stride, add_dev, add_stride, flags, nullptr,
                          ctx->pick(stream), &p);
}

int tsr_hip_mul_mat_isums(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, int32_t * isums_dev,
                          void * stream) {
    if (ctx == nullptr || isums_dev == nullptr || w == nullptr) return TSR_HIP_E_ARG;
    // y goes to scratch: the integer sums are the product of this call
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    const int rc = ctx->scratch.reserve((size_t)w->N * sizeof(float), s);
    if (rc) return rc;
    return mul_mat_locked(ctx, w, x_dev, 1u, w->K, (float *)ctx->scratch.ptr, w->N, nullptr, 0u, 0u, isums_dev, s);
}

// ---------------------------------------------------------------------------------------------
// graphs: the launches one stream records between begin and end, replayed as one launch
// ---------------------------------------------------------------------------------------------
struct tsr_hip_graph {
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
    bool uses_scratch = false;                   // a captured launch holds the scratch's address
    uint64_t scratch_gen = 0;                    // the scratch's generation at capture
};

int tsr_hip_graph_begin(tsr_hip_ctx * ctx, void * stream) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    if (tsr_capturing(s)) return TSR_HIP_E_ARG;
    ctx->scratch.captured = false;
    return hip_err(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

int tsr_hip_graph_end(tsr_hip_ctx * ctx, void * stream, tsr_hip_graph ** out) {
    if (ctx == nullptr || out == nullptr) return TSR_HIP_E_ARG;
    *out = nullptr;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    hipGraph_t g = nullptr;
    int rc = hip_err(hipStreamEndCapture(s, &g), "hipStreamEndCapture");
    if (rc) return rc;
    auto * gr = new (std::nothrow) tsr_hip_graph();
    if (gr == nullptr) { (void)hipGraphDestroy(g); return TSR_HIP_E_NOMEM; }
    gr->g = g;
    gr->uses_scratch = ctx->scratch.captured;
    gr->scratch_gen = ctx->scratch.gen;
    ctx->scratch.captured = false;
    if ((rc = hip_err(hipGraphInstantiate(&gr->x, g, nullptr, nullptr, 0), "hipGraphInstantiate")) != 0) {
        (void)hipGraphDestroy(g);
        delete gr;
        return rc;
    }
    *out = gr;
    return TSR_HIP_OK;
}

int tsr_hip_graph_launch(tsr_hip_ctx * ctx, const tsr_hip_graph * graph, void * stream) {
    if (ctx == nullptr || graph == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    // the scratch block the capture used was freed by a later growth: capture again
    if (graph->uses_scratch && graph->scratch_gen != ctx->scratch.gen) return TSR_HIP_E_ARG;
    (void)hipSetDevice(ctx->device);
    return hip_err(hipGraphLaunch(graph->x, ctx->pick(stream)), "hipGraphLaunch");
}

int tsr_hip_graph_free(tsr_hip_ctx * ctx, tsr_hip_graph * graph) {
    if (ctx == nullptr || graph == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();                // no replay still runs
    (void)hipGraphExecDestroy(graph->x);
    (void)hipGraphDestroy(graph->g);
    delete graph;
    return TSR_HIP_OK;
}
