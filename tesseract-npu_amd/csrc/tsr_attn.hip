// tsr_attn.hip -- host side of the KV cache, the mask summary and FLASH_ATTN_EXT.
#include <hip/hip_runtime.h>

#include <cmath>

#include <algorithm>
#include <cstring>
#include <limits>
#include <mutex>
#include <new>
#include <type_traits>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"
#include "tsr_hip.h"

using tsr::hip_err;

static tsr::KvArgs kv_args(const tsr_hip_kv * kv) {
    tsr::KvArgs a{};
    a.base = kv->dev;
    a.quant_off = kv->quant_off;
    a.E = kv->E;
    a.kv_size = kv->kv_size;
    return a;
}

int tsr_hip_kv_create(tsr_hip_ctx * ctx, uint32_t E, uint32_t kv_size, tsr_hip_kv ** out) {
    if (ctx == nullptr || out == nullptr) return TSR_HIP_E_ARG;
    *out = nullptr;
    if (E == 0u || E % 64u != 0u || E > 32768u || kv_size == 0u) return TSR_HIP_E_SHAPE;
    auto * kv = new (std::nothrow) tsr_hip_kv();
    if (kv == nullptr) return TSR_HIP_E_NOMEM;
    const size_t ng = (kv_size + 15u) / 16u;
    kv->E = E;
    kv->kv_size = kv_size;
    kv->meta_row = (size_t)E / 32u * 2u;
    kv->quant_off = (ng * 16u * kv->meta_row + 255u) & ~(size_t)255u;
    kv->bytes = kv->quant_off + ng * 16u * E;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = hip_err(hipMalloc((void **)&kv->dev, kv->bytes), "hipMalloc kv");
    if (rc == 0) rc = hip_err(hipMemsetAsync(kv->dev, 0, kv->bytes, ctx->stream), "hipMemset kv");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) {
        if (kv->dev) (void)hipFree(kv->dev);
        delete kv;
        return rc;
    }
    *out = kv;
    return TSR_HIP_OK;
}

int tsr_hip_kv_free(tsr_hip_ctx * ctx, tsr_hip_kv * kv) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    if (kv == nullptr) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    const int rc = hip_err(hipFree(kv->dev), "hipFree kv");
    delete kv;
    return rc;
}

static int kv_bytes(tsr_hip_ctx * ctx, const tsr_hip_kv * kv, uint32_t which, size_t off, void * host, size_t bytes,
                    int to_dev) {
    if (ctx == nullptr || kv == nullptr || (bytes && host == nullptr)) return TSR_HIP_E_ARG;
    if (which > 1u) return TSR_HIP_E_ARG;
    const uint64_t total = (uint64_t)kv->kv_size * (kv->E / 32u) * 34u;
    if ((uint64_t)off > total || (uint64_t)bytes > total - off) return TSR_HIP_E_RANGE;
    if (bytes == 0) return TSR_HIP_OK;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    int rc = ctx->scratch.reserve(bytes, ctx->stream);
    if (rc) return rc;
    uint8_t * stage = (uint8_t *)ctx->scratch.ptr;
    if (to_dev) rc = hip_err(hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, ctx->stream), "kv H2D");
    if (rc == 0) rc = tsr_launch_kv_bytes(kv_args(kv), which, off, bytes, stage, to_dev, ctx->stream) ? TSR_HIP_E_HIP : 0;
    if (rc == 0 && !to_dev) rc = hip_err(hipMemcpyAsync(host, stage, bytes, hipMemcpyDeviceToHost, ctx->stream), "kv D2H");
    if (rc == 0) rc = hip_err(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return rc;
}

int tsr_hip_kv_set_bytes(tsr_hip_ctx * ctx, tsr_hip_kv * kv, uint32_t which, size_t off, const void * src, size_t bytes) {
    return kv_bytes(ctx, kv, which, off, const_cast<void *>(src), bytes, 1);
}

int tsr_hip_kv_get_bytes(tsr_hip_ctx * ctx, const tsr_hip_kv * kv, uint32_t which, size_t off, void * dst, size_t bytes) {
    return kv_bytes(ctx, kv, which, off, dst, bytes, 0);
}

int tsr_hip_kv_set_rows(tsr_hip_ctx * ctx, tsr_hip_kv * kv, uint32_t which, const float * src_dev, uint32_t n_rows,
                        uint64_t src_stride, const int64_t * idx_dev, int32_t * bad_dev, void * stream) {
    if (ctx == nullptr || kv == nullptr || src_dev == nullptr || idx_dev == nullptr || which > 1u) return TSR_HIP_E_ARG;
    if (n_rows == 0u) return TSR_HIP_OK;
    if (((uintptr_t)src_dev & 15u) != 0u || (n_rows > 1u && (src_stride % 4u != 0u || src_stride < kv->E)) ||
        n_rows > 65535u)
        return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    ctx->ctr.set_rows_calls++;
    return tsr_launch_kv_set_rows(kv_args(kv), which, src_dev, n_rows, src_stride, idx_dev, ctx->flag(bad_dev), ctx->pick(stream))
               ? TSR_HIP_E_HIP
               : TSR_HIP_OK;
}

int tsr_hip_rope_kv(tsr_hip_ctx * ctx, float * qkv_dev, uint32_t T, uint64_t stride, uint32_t head_dim, uint32_t n_head,
                    uint32_t n_head_kv, uint32_t n_dims, int mode, const int32_t * pos_dev, float freq_base,
                    float attn_factor, tsr_hip_kv * kc, tsr_hip_kv * vc, const int64_t * cell_dev, int32_t * bad_dev,
                    void * stream) {
    if (ctx == nullptr || qkv_dev == nullptr || pos_dev == nullptr || cell_dev == nullptr || kc == nullptr ||
        vc == nullptr || T == 0u)
        return TSR_HIP_E_ARG;
    if (mode != TSR_HIP_ROPE_NORMAL && mode != TSR_HIP_ROPE_NEOX && mode != TSR_HIP_ROPE_IMROPE) return TSR_HIP_E_SHAPE;
    const uint64_t E = (uint64_t)n_head_kv * head_dim, nrow = (uint64_t)n_head * head_dim + 2u * E;
    if (head_dim == 0u || head_dim % 32u != 0u || n_head == 0u || n_head_kv == 0u || n_dims < 2u || n_dims % 2u != 0u ||
        n_dims > head_dim || n_dims > 1024u || nrow > 16384u || T > 0x7FFFFFFFu)
        return TSR_HIP_E_SHAPE;
    if (kc->E != E || vc->E != E) return TSR_HIP_E_SHAPE;
    if (((uintptr_t)qkv_dev & 15u) != 0u || (T > 1u && (stride % 4u != 0u || stride < nrow))) return TSR_HIP_E_ARG;
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base)) return TSR_HIP_E_ARG;
    tsr::RopeKvArgs a{};
    a.qkv = qkv_dev;
    a.stride = stride;
    a.pos = pos_dev;
    a.cell = cell_dev;
    a.bad = ctx->flag(bad_dev);
    a.kc = kv_args(kc);
    a.vc = kv_args(vc);
    a.head_dim = head_dim;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.n_dims = n_dims;
    a.neox = mode != TSR_HIP_ROPE_NORMAL ? 1u : 0u;
    a.ts = powf(freq_base, -2.0f / (float)n_dims);                  // the host libm, as tsr_hip_rope
    a.m = attn_factor;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    ctx->ctr.set_rows_calls += 2u;
    const int rc = tsr_launch_rope_kv(a, T, ctx->pick(stream));
    return rc == -2 ? TSR_HIP_E_SHAPE : (rc ? TSR_HIP_E_HIP : TSR_HIP_OK);
}

// ---------------------------------------------------------------------------------------------
// MSUM: runs of +-0 per query row, GENERAL for any other finite / +inf / NaN value or > 2 runs
// (sw/sim/tsr_ref_at.c:646-693; AT section 7.3).
// ---------------------------------------------------------------------------------------------
int tsr_hip_msum_build_f16(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, uint32_t * words) {
    if (words == nullptr || (n_q && n_kv && mask == nullptr)) return TSR_HIP_E_ARG;
    bool general = false;
    for (uint32_t q = 0; q < n_q; ++q) {
        const uint16_t * m = mask + (size_t)q * row_stride;
        uint32_t * w = words + 8u + 4u * q;
        w[0] = w[1] = w[2] = w[3] = 0u;
        uint32_t nrun = 0;
        for (uint32_t j = 0; j < n_kv;) {
            if (m[j] == 0xFC00u) { ++j; continue; }
            if (m[j] & 0x7FFFu) { general = true; ++j; continue; }
            uint32_t e = j + 1u;
            while (e < n_kv && (m[e] & 0x7FFFu) == 0u) ++e;
            if (nrun < 2u) { w[2u * nrun] = j; w[2u * nrun + 1u] = e; }
            ++nrun;
            j = e;
        }
        if (nrun > 2u) general = true;
    }
    if (general) {
        for (uint32_t q = 0; q < n_q; ++q) {
            const uint16_t * m = mask + (size_t)q * row_stride;
            uint32_t lo = 0, hi = 0;
            bool seen = false;
            for (uint32_t j = 0; j < n_kv; ++j)
                if (m[j] != 0xFC00u) { if (!seen) lo = j; seen = true; hi = j + 1u; }
            uint32_t * w = words + 8u + 4u * q;
            w[0] = lo; w[1] = hi; w[2] = 0u; w[3] = 0u;
        }
    }
    words[0] = 0x4D55534Du;
    words[1] = n_q;
    words[2] = n_kv;
    words[3] = general ? 1u : 0u;
    words[4] = words[5] = words[6] = words[7] = 0u;
    return (int)words[3];
}

// The f32 mask copy of a GENERAL mask (tsr_msum_mask_f32, sw/sim/tsr_ref_at.c:704-715): cell j of row q
// is fdiv(f32(mask[q][j]), scale) under the f32 rule (DAZ operands, one IEEE division, FTZ result,
// canonical NaN), rows of 16 ceil(n_kv / 16) floats padded with -inf.
static float host_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    if (e == 31u) u = s | 0x7F800000u | (m ? (0x00400000u | (m << 13)) : 0u);
    else if (e != 0u) u = s | ((e + 112u) << 23) | (m << 13);
    else if (m == 0u) u = s;
    else {                                                         // subnormal fp16: a normal f32
        uint32_t k = 0, mm = m;
        while ((mm & 0x400u) == 0u) { mm <<= 1; ++k; }
        u = s | ((113u - k) << 23) | ((mm & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static float host_rule(float r) {
    uint32_t u;
    memcpy(&u, &r, 4);
    const uint32_t e = u & 0x7F800000u;
    if (e == 0u) u &= 0x80000000u;
    else if (e == 0x7F800000u && (u & 0x007FFFFFu)) u = 0x7FC00000u;
    memcpy(&r, &u, 4);
    return r;
}
static float host_daz(float x) { return host_rule(x) == 0.0f ? std::copysign(0.0f, x) : x; }

int tsr_hip_msum_mask_f32(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, float scale,
                          float * dst) {
    if (dst == nullptr || (n_q && n_kv && mask == nullptr)) return TSR_HIP_E_ARG;
    uint32_t sb;
    memcpy(&sb, &scale, 4);
    const uint32_t e = (sb >> 23) & 0xFFu;
    if ((sb & 0x80000000u) || e == 0u || e == 0xFFu) return TSR_HIP_E_ARG;   // finite, normal and > 0
    const size_t w = 16u * (((size_t)n_kv + 15u) / 16u);
    const float ninf = -std::numeric_limits<float>::infinity();
    for (uint32_t q = 0; q < n_q; ++q) {
        const uint16_t * m = mask + (size_t)q * row_stride;
        float * d = dst + (size_t)q * w;
        for (uint32_t j = 0; j < n_kv; ++j) {
            const float x = host_daz(host_h2f(m[j]));
            if (std::isnan(x)) { d[j] = host_rule(std::numeric_limits<float>::quiet_NaN()); continue; }
            volatile float num = x, den = scale;                   // one IEEE binary32 division
            d[j] = host_rule(num / den);
        }
        for (size_t j = n_kv; j < w; ++j) d[j] = ninf;
    }
    return TSR_HIP_OK;
}

// ---------------------------------------------------------------------------------------------
// FLASH_ATTN_EXT: plan on the host, four launches (QACT of q, scores, P.V, merge)
// ---------------------------------------------------------------------------------------------
namespace {

constexpr uint32_t kC = 4u, kPcap = 9344u;

struct Chunk {
    uint32_t u0, n, c_lo, c_hi, general;
};

// NCG = min(128, C floor(PCAP / (16 E / D)), max(4C, roundup_4C(ceil(n_total / 2))))
// (sw/sim/include/tsr_fa_plan.h:130-156).
uint32_t ncg_of(uint32_t E, uint32_t D, uint32_t n_total) {
    const uint64_t pc = (uint64_t)kC * (kPcap / (16u * (E / D)));
    const uint64_t half = ((uint64_t)n_total + 1u) / 2u, c4 = 4u * kC;
    const uint64_t m = half <= c4 ? c4 : (half + c4 - 1u) / c4 * c4;
    return (uint32_t)std::min<uint64_t>(std::min<uint64_t>(128u, pc), m);
}

// The chunks of one query row in execution order (one-row tiles: rules 1, 2, 4, 7, 8 of the planner,
// sw/sim/include/tsr_fa_plan.h:16-42). Returns false for a malformed MSUM row.
// A fixed-capacity stand-in for std::vector in the planner of the entry point that allocates nothing:
// push_back past the capacity records an overflow instead of growing.
template <class T, size_t N>
struct FixedVec {
    T v[N];
    size_t n = 0;
    bool overflow = false;
    void clear() { n = 0; overflow = false; }
    void push_back(const T & x) {
        if (n < N) v[n++] = x;
        else overflow = true;
    }
    void assign(size_t k, const T & x) {
        if (k > N) { overflow = true; k = N; }
        n = k;
        for (size_t i = 0; i < k; ++i) v[i] = x;
    }
    size_t size() const { return n; }
    T & operator[](size_t i) { return v[i]; }
    const T & operator[](size_t i) const { return v[i]; }
    T * data() { return v; }
    const T * begin() const { return v; }
    const T * end() const { return v + n; }
};
template <class V> bool overflowed(const V &) { return false; }
template <class T, size_t N> bool overflowed(const FixedVec<T, N> & v) { return v.overflow; }

template <class Out>
bool plan_row(uint32_t E, uint32_t D, const uint32_t * words, uint32_t q, const uint32_t (*new_runs)[2],
              uint32_t n_new, Out & out) {
    const uint32_t n_kv = words[2];
    const bool general = (words[3] & 1u) != 0u;
    struct Sub { uint32_t ulo, uhi; uint64_t lo, hi; } sub[2];
    uint32_t nsub = 0;
    if (general) {
        if (n_kv > 0u) sub[nsub++] = { 0u, (n_kv + 15u) / 16u, 0u, 0u };
    } else {
        const uint32_t * w = words + 8u + 4u * q;
        if (w[0] > w[1] || w[2] > w[3] || w[1] > n_kv || w[3] > n_kv) return false;
        if (w[1] > w[0] && w[3] > w[2] && !(w[1] <= w[2] || w[3] <= w[0])) return false;
        uint32_t r[2][2], nr = 0;
        if (w[1] > w[0]) { r[nr][0] = w[0]; r[nr][1] = w[1]; ++nr; }
        if (w[3] > w[2]) { r[nr][0] = w[2]; r[nr][1] = w[3]; ++nr; }
        if (nr == 2u && r[1][0] < r[0][0]) { std::swap(r[0][0], r[1][0]); std::swap(r[0][1], r[1][1]); }
        for (uint32_t k = 0; k < nr; ++k) sub[nsub++] = { r[k][0] / 16u, (r[k][1] + 15u) / 16u, r[k][0], r[k][1] };
    }
    if (nsub == 0u) {                                      // no visible cell: one empty chunk
        out.push_back({ 0u, 1u, 0u, 0u, 0u });
        return true;
    }
    uint32_t n_total = 0;
    for (uint32_t k = 0; k < nsub; ++k) n_total += sub[k].uhi - sub[k].ulo;
    const uint32_t ncg = ncg_of(E, D, n_total);
    if (ncg == 0u) return false;
    for (int pass = 0; pass < 2; ++pass)                   // chunks holding a new cell go last
        for (uint32_t k = 0; k < nsub; ++k)
            for (uint32_t a = sub[k].ulo; a < sub[k].uhi; a += ncg) {
                const uint32_t b = std::min(a + ncg, sub[k].uhi);
                bool has_new = false;
                for (uint32_t i = 0; i < n_new; ++i)
                    has_new |= new_runs[i][1] > new_runs[i][0] && (uint64_t)new_runs[i][0] < 16ull * b &&
                                (uint64_t)new_runs[i][1] > 16ull * a;
                if ((int)has_new != pass) continue;
                Chunk c{ a, b - a, 0u, 16u * (b - a), general ? 1u : 0u };
                if (!general) {
                    const int64_t A = 16 * (int64_t)a, n16 = 16 * (int64_t)(b - a);
                    c.c_lo = (uint32_t)std::max<int64_t>((int64_t)sub[k].lo - A, 0);
                    c.c_hi = (uint32_t)std::min<int64_t>((int64_t)sub[k].hi - A, n16);
                }
                out.push_back(c);
            }
    return true;
}

size_t up256(size_t x) { return (x + 255u) & ~(size_t)255u; }

// The shape checks FLASH_ATTN_EXT makes on its operands (the planned and the unplanned entry points).
int fa_check_shape(uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale) {
    if (!(D == 64u || D == 128u || D == 256u || D == 512u)) return TSR_HIP_E_SHAPE;
    if (n_head_kv == 0u || n_head % n_head_kv != 0u || n_head / n_head_kv > 64u) return TSR_HIP_E_SHAPE;
    const uint32_t E = n_head_kv * D, G = n_head / n_head_kv, K = n_head * D;
    if (E / 64u > 511u || (uint64_t)G * E > 32768u || K > 32768u) return TSR_HIP_E_SHAPE;
    uint32_t sb;
    memcpy(&sb, &scale, 4);
    if ((sb >> 31) || (sb & 0x7F800000u) == 0u || (sb & 0x7F800000u) == 0x7F800000u) return TSR_HIP_E_SHAPE;
    return TSR_HIP_OK;
}

// The work list of one call: every token row planned, flattened into items (chunks) with their
// 256-cell score tiles; tok = tok_first[T] | tok_count[T]. FaWorkFixed holds at most the inline list
// (kFaInlItems items of at most kFaInlTok tokens) in fixed arrays: planning it allocates nothing.
template <class Items, class Tok, class Chunks>
struct FaWorkT {
    Items items;
    Tok tok;
    Chunks ch;               // one row's chunks (planner temporary)
    uint64_t cells = 0;
    uint32_t n_tiles = 0, maxtiles = 1, max_groups = 0;
};
using FaWork = FaWorkT<std::vector<tsr::FaItem>, std::vector<uint32_t>, std::vector<Chunk>>;
using FaWorkFixed = FaWorkT<FixedVec<tsr::FaItem, tsr::kFaInlItems>, FixedVec<uint32_t, 2u * tsr::kFaInlTok>,
                            FixedVec<Chunk, tsr::kFaInlItems>>;

// Returns TSR_HIP_E_RANGE when a fixed-capacity work list overflows.
template <class W>
int fa_plan_rows(uint32_t E, uint32_t D, uint32_t T, const uint32_t * msum, const uint32_t (*new_runs)[2], uint32_t n_new,
                 bool have_mask, W & w) {
    w.items.clear();
    w.tok.assign(2u * (size_t)T, 0u);
    if (overflowed(w.tok)) return TSR_HIP_E_RANGE;
    w.cells = 0;
    w.n_tiles = 0;
    w.maxtiles = 1;
    w.max_groups = 0;
    auto & ch = w.ch;
    for (uint32_t t = 0; t < T; ++t) {
        ch.clear();
        if (!plan_row(E, D, msum, t, new_runs, n_new, ch)) return TSR_HIP_E_MASK;
        if (overflowed(ch)) return TSR_HIP_E_RANGE;
        w.tok[t] = (uint32_t)w.items.size();
        w.tok[T + t] = (uint32_t)ch.size();
        for (const Chunk & c : ch) {
            if (c.general && !have_mask) return TSR_HIP_E_MASK;
            tsr::FaItem it{};
            it.t = t;
            it.u0 = c.u0;
            it.n = c.n;
            it.c_lo = c.c_lo;
            it.c_hi = c.c_hi;
            it.general = c.general;
            it.s_off = (uint32_t)w.cells;
            it.tile0 = w.n_tiles;
            it.ntiles = (16u * c.n + 255u) / 256u;
            w.n_tiles += it.ntiles;
            w.maxtiles = std::max(w.maxtiles, it.ntiles);
            w.max_groups = std::max(w.max_groups, c.n);
            w.cells += 16u * c.n;
            w.items.push_back(it);
        }
        if (overflowed(w.items)) return TSR_HIP_E_RANGE;
    }
    return TSR_HIP_OK;
}

tsr::FaArgs fa_args(tsr_hip_ctx * ctx, const float * q_dev, uint64_t q_stride, const tsr_hip_kv * kc,
                    const tsr_hip_kv * vc, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                    const float * mask_f32_dev, uint32_t mstride, float * out_dev, uint64_t out_stride) {
    tsr::FaArgs a{};
    a.q = q_dev;
    a.q_stride = q_stride;
    a.kc = kv_args(kc);
    a.vc = kv_args(vc);
    a.D = D;
    a.G = n_head / n_head_kv;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.E = n_head_kv * D;
    a.scale = scale;
    a.mask = mask_f32_dev;
    a.mstride = mstride;
    a.out = out_dev;
    a.out_stride = out_stride;
    a.ex = ctx->expk;
    return a;
}

}  // namespace

// The unplanned FLASH_ATTN_EXT: the host plans the rows, the partials go to the context's scratch
// (NOALLOC false: grown by hipMalloc on demand, ordered across streams) or to the fixed device array of
// this file (NOALLOC true: the inline work list only, nothing allocated, nothing waited for).
template <bool NOALLOC>
static int fa_unplanned(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride, const tsr_hip_kv * kc,
                        const tsr_hip_kv * vc, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                        const uint32_t * msum, const float * mask_f32_dev, const uint32_t (*new_runs)[2], uint32_t n_new,
                        float * out_dev, uint64_t out_stride, void * stream) {
    if (ctx == nullptr || q_dev == nullptr || kc == nullptr || vc == nullptr || msum == nullptr || out_dev == nullptr ||
        T == 0u || (n_new && new_runs == nullptr))
        return TSR_HIP_E_ARG;
    int rc = fa_check_shape(D, n_head, n_head_kv, scale);
    if (rc) return rc;
    const uint32_t E = n_head_kv * D, K = n_head * D;
    if (kc->E != E || vc->E != E || kc->kv_size != vc->kv_size) return TSR_HIP_E_SHAPE;
    if (msum[0] != 0x4D55534Du || msum[1] != T || msum[2] > kc->kv_size) return TSR_HIP_E_MASK;
    if (((uintptr_t)q_dev & 15u) != 0u || (T > 1u && (q_stride % 4u != 0u || q_stride < K)) ||
        (T > 1u && out_stride < K) || T > 65535u)
        return TSR_HIP_E_ARG;
    if (NOALLOC && T > tsr::kFaInlTok) return TSR_HIP_E_RANGE;

    typename std::conditional<NOALLOC, FaWorkFixed, FaWork>::type w;
    if ((rc = fa_plan_rows(E, D, T, msum, new_runs, n_new, mask_f32_dev != nullptr, w)) != 0) return rc;
    const size_t n_items = w.items.size();
    if (w.cells * n_head > 0xFFFFFFFFull || n_items * 4u > 0x7FFFFFFFull || n_items * w.maxtiles > 0x7FFFFFFFull)
        return TSR_HIP_E_SHAPE;
    const bool inl = n_items <= tsr::kFaInlItems && T <= tsr::kFaInlTok;
    size_t off = 0;
    const size_t o_items = off; off = up256(off + (inl ? 0u : n_items * sizeof(tsr::FaItem) + 8u * (size_t)T));
    const size_t o_S = off; off = up256(off + 4u * (size_t)w.cells * n_head);
    const size_t o_Mp = off; off = up256(off + 4u * (size_t)w.n_tiles * n_head);
    const size_t o_OP = off; off = up256(off + 4u * n_items * kC * n_head * D);
    const size_t o_LP = off; off = up256(off + 4u * n_items * kC * n_head);
    if (NOALLOC && off > kFaNoAllocBytes) return TSR_HIP_E_RANGE;

    tsr::FaPlan p{};
    p.n_items = (uint32_t)n_items;
    p.maxtiles = w.maxtiles;
    std::vector<uint8_t> packed;
    if (inl) {
        std::copy(w.items.begin(), w.items.end(), p.items);
        for (uint32_t t = 0; t < T; ++t) { p.tok_first[t] = w.tok[t]; p.tok_count[t] = w.tok[T + t]; }
    } else if constexpr (!NOALLOC) {                              // items | tok_first | tok_count, one copy
        packed.resize(n_items * sizeof(tsr::FaItem) + 8u * (size_t)T);
        memcpy(packed.data(), w.items.data(), n_items * sizeof(tsr::FaItem));
        memcpy(packed.data() + n_items * sizeof(tsr::FaItem), w.tok.data(), 8u * (size_t)T);
    }

    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    uint8_t * base;
    if constexpr (NOALLOC) {
        if (ctx->fa_fixed == nullptr) return TSR_HIP_E_HIP;       // the array's address was not found at open
        base = ctx->fa_fixed;
    } else {
        rc = ctx->scratch.reserve(off, s);
        if (rc) return rc;
        base = (uint8_t *)ctx->scratch.ptr;
        if (!inl) {
            // a host-to-device copy of a host vector cannot be recorded into a graph (the vector is gone
            // when the graph replays): long work lists are for eager calls or a tsr_hip_fa_plan
            if (tsr_capturing(s)) return TSR_HIP_E_ARG;
            rc = hip_err(hipMemcpyAsync(base + o_items, packed.data(), packed.size(), hipMemcpyHostToDevice, s), "fa plan");
            if (rc) return rc;
        }
    }
    tsr::FaArgs a = fa_args(ctx, q_dev, q_stride, kc, vc, D, n_head, n_head_kv, scale, mask_f32_dev,
                            16u * ((msum[2] + 15u) / 16u), out_dev, out_stride);
    if (!inl) {
        a.items = (const tsr::FaItem *)(base + o_items);
        a.tok_first = (const uint32_t *)(base + o_items + n_items * sizeof(tsr::FaItem));
        a.tok_count = a.tok_first + T;
    }
    a.S = (float *)(base + o_S);
    a.Mpart = (float *)(base + o_Mp);
    a.OP = (float *)(base + o_OP);
    a.LP = (float *)(base + o_LP);
    a.max_groups = w.max_groups;
    ctx->ctr.flash_attn_calls++;
    ctx->ctr.flash_attn_kv_bytes += w.cells * (uint64_t)E / 32u * 34u * 2u;
    return tsr_launch_fa(a, p, T, (uint32_t)ctx->n_cu, s) ? TSR_HIP_E_HIP : TSR_HIP_OK;
}

int tsr_hip_flash_attn(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride, const tsr_hip_kv * kc,
                       const tsr_hip_kv * vc, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                       const uint32_t * msum, const float * mask_f32_dev, const uint32_t (*new_runs)[2], uint32_t n_new,
                       float * out_dev, uint64_t out_stride, void * stream) {
    return fa_unplanned<false>(ctx, q_dev, T, q_stride, kc, vc, D, n_head, n_head_kv, scale, msum, mask_f32_dev,
                               new_runs, n_new, out_dev, out_stride, stream);
}

// ---------------------------------------------------------------------------------------------
// The FLASH_ATTN_EXT entry point that allocates nothing (for callers that cannot call hipMalloc: code
// under graph capture, tight serving loops). Its partials live in fa_fixed_scratch, a file-scope device
// array of kFaNoAllocBytes that every GPU the library runs on holds until the process ends. On the host
// the array's name is a stand-in, not a device address: tsr_fa_fixed_init (run by tsr_hip_open with the
// context's device current) looks the device address up once, and launches use only that address. All
// calls on one GPU share its array (every context on that device): calls that overlap on one GPU race.
// Nothing in the array has to start at zero (every partial is written before it is read).
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) uint8_t fa_fixed_scratch[kFaNoAllocBytes];

int tsr_fa_fixed_init(tsr_hip_ctx * ctx) {
    void * p = nullptr;
    const int rc = hip_err(hipGetSymbolAddress(&p, HIP_SYMBOL(fa_fixed_scratch)), "hipGetSymbolAddress fa_fixed_scratch");
    if (rc) return rc;
    ctx->fa_fixed = (uint8_t *)p;
    return TSR_HIP_OK;
}

int tsr_hip_flash_attn_noalloc(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride,
                               const tsr_hip_kv * kc, const tsr_hip_kv * vc, uint32_t D, uint32_t n_head,
                               uint32_t n_head_kv, float scale, const uint32_t * msum, const float * mask_f32_dev,
                               const uint32_t (*new_runs)[2], uint32_t n_new, float * out_dev, uint64_t out_stride,
                               void * stream) {
    return fa_unplanned<true>(ctx, q_dev, T, q_stride, kc, vc, D, n_head, n_head_kv, scale, msum, mask_f32_dev,
                              new_runs, n_new, out_dev, out_stride, stream);
}

// ---------------------------------------------------------------------------------------------
// FA plans: the work list in device memory, refreshed per call by a stream-ordered copy, so that a
// captured graph of planned FLASH_ATTN_EXT launches replays over a mask that changes between
// replays (the per-graph plan cache of ggml-tesseract.cpp:3937-3952 and 3768-3779, as a graph)
// ---------------------------------------------------------------------------------------------
struct tsr_hip_fa_plan {
    uint32_t D = 0, n_head = 0, n_head_kv = 0, T = 0, kv_size = 0;
    uint32_t items_max = 0, tiles_max = 0;
    uint64_t cells_max = 0;
    uint8_t * dev = nullptr;
    size_t o_items = 0, o_S = 0, o_Mp = 0, o_OP = 0, o_LP = 0, o_SO = 0, o_SL = 0, o_MI = 0, o_TK = 0, o_EP = 0,
           o_QF = 0, bytes = 0;
    bool set = false, general = false;
    uint32_t n_items = 0, maxtiles = 0, max_groups = 0, mstride = 0;   // the shape a launch bakes in
    uint32_t seg_work = 0;   // the decode form's segments with work (64 cells of one channel) per KV head
    bool qkv_fits = false;   // tsr_hip_attn_qkv_plan_rope_tab's one launch fits the device at once
    uint64_t cells = 0;
};

int tsr_hip_fa_plan_create(tsr_hip_ctx * ctx, uint32_t D, uint32_t n_head, uint32_t n_head_kv, uint32_t T,
                           uint32_t kv_size, tsr_hip_fa_plan ** out) {
    if (ctx == nullptr || out == nullptr || T == 0u || kv_size == 0u) return TSR_HIP_E_ARG;
    *out = nullptr;
    int rc = fa_check_shape(D, n_head, n_head_kv, 1.0f);
    if (rc) return rc;
    if (T > 65535u) return TSR_HIP_E_SHAPE;
    const uint32_t E = n_head_kv * D;
    const uint64_t pc = (uint64_t)kC * (kPcap / (16u * (E / D)));
    const uint64_t ncg_min = std::max<uint64_t>(1u, std::min<uint64_t>(std::min<uint64_t>(128u, pc), 4u * kC));
    const uint64_t groups = ((uint64_t)kv_size + 15u) / 16u + 2u;             // two runs, each with a partial group
    const uint64_t items = (uint64_t)T * ((groups + ncg_min - 1u) / ncg_min + 2u);
    const uint64_t cells = (uint64_t)T * 16u * groups;
    const uint64_t tiles = cells / 256u + items;
    if (items > 0x7FFFFFFFull / 4u || cells * n_head > 0xFFFFFFFFull) return TSR_HIP_E_SHAPE;
    auto * p = new (std::nothrow) tsr_hip_fa_plan();
    if (p == nullptr) return TSR_HIP_E_NOMEM;
    p->D = D;
    p->n_head = n_head;
    p->n_head_kv = n_head_kv;
    p->T = T;
    p->kv_size = kv_size;
    p->items_max = (uint32_t)items;
    p->tiles_max = (uint32_t)tiles;
    p->cells_max = cells;
    size_t off = 0;
    p->o_items = off; off = up256(off + items * sizeof(tsr::FaItem) + 8u * (size_t)T);
    p->o_S = off; off = up256(off + 4u * (size_t)cells * n_head);
    p->o_Mp = off; off = up256(off + 4u * (size_t)tiles * n_head);
    p->o_OP = off; off = up256(off + 4u * (size_t)items * kC * n_head * D);
    p->o_LP = off; off = up256(off + 4u * (size_t)items * kC * n_head);
    // the fused decode form (T == 1): per-tile segment results and row sums, and its counters
    const uint64_t ftiles = T == 1u ? tiles : 0u;
    // (value, tag) pairs of the decode form: segment results, row sums, chunk maxima
    p->o_SO = off; off = up256(off + 8u * (size_t)ftiles * kC * n_head * D);
    p->o_SL = off; off = up256(off + 8u * (size_t)ftiles * kC * n_head);
    p->o_MI = off; off = up256(off + (T == 1u ? 8u * (size_t)items * n_head : 0u));
    // zero between launches: the 16-byte slots of segment maxima (an item has <= 8 tiles of 4 channels:
    // NCG <= 128 groups) and the counters
    // the decode form's segment slots (32 bytes) and per-reducer epochs (<= 4 heads x 2 value parts)
    p->o_TK = off; off = up256(off + (T == 1u ? 32u * 8u * 4u * (size_t)items * n_head_kv : 0u));
    p->o_EP = off; off = up256(off + (T == 1u ? 4u * 8u * (size_t)n_head_kv : 0u));
    // the flags of the Q|K|V row workgroups (tsr_hip_attn_qkv_plan_rope_tab): 64 words per KV head
    p->o_QF = off; off = up256(off + (T == 1u ? 4u * 64u * (size_t)n_head_kv : 0u));
    p->bytes = off;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    if ((rc = hip_err(hipMalloc(&p->dev, off), "hipMalloc fa plan")) != 0) {
        delete p;
        return rc;
    }
    // tags and epochs start at zero (the decode form's first launch tags with 1)
    if ((rc = hip_err(hipMemset(p->dev, 0, off), "hipMemset fa plan")) != 0 ||
        (rc = hip_err(hipDeviceSynchronize(), "fa plan counters")) != 0) {
        (void)hipFree(p->dev);
        delete p;
        return rc;
    }
    *out = p;
    return TSR_HIP_OK;
}

int tsr_hip_set_fa_wait_limit(tsr_hip_ctx * ctx, uint32_t polls) {
    if (ctx == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    ctx->fa_spin_max = polls ? polls : (1u << 20);
    return TSR_HIP_OK;
}

int tsr_hip_fa_plan_set_epoch(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan, uint32_t epoch) {
    if (ctx == nullptr || plan == nullptr) return TSR_HIP_E_ARG;
    if (plan->T != 1u) return TSR_HIP_E_SHAPE;
    std::vector<uint32_t> words(8u * (size_t)plan->n_head_kv, epoch);
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(nullptr);
    if (tsr_capturing(s)) return TSR_HIP_E_ARG;
    int rc = ctx->staging.copy(plan->dev + plan->o_EP, words.data(), 4u * words.size(), s);
    if (rc) return rc;
    return hip_err(hipStreamSynchronize(s), "fa plan epoch");
}

int tsr_hip_fa_plan_free(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan) {
    if (ctx == nullptr || plan == nullptr) return TSR_HIP_E_ARG;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();                // no queued launch still reads the list
    (void)hipFree(plan->dev);
    delete plan;
    return TSR_HIP_OK;
}

int tsr_hip_fa_plan_set(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan, const uint32_t * msum, int mask_f32,
                        const uint32_t (*new_runs)[2], uint32_t n_new, int * shape_changed, void * stream) {
    if (ctx == nullptr || plan == nullptr || msum == nullptr || (n_new && new_runs == nullptr)) return TSR_HIP_E_ARG;
    if (msum[0] != 0x4D55534Du || msum[1] != plan->T || msum[2] > plan->kv_size) return TSR_HIP_E_MASK;
    FaWork w;
    int rc = fa_plan_rows(plan->n_head_kv * plan->D, plan->D, plan->T, msum, new_runs, n_new, mask_f32 != 0, w);
    if (rc) return rc;
    if (w.items.size() > plan->items_max || w.cells > plan->cells_max || w.n_tiles > plan->tiles_max)
        return TSR_HIP_E_SHAPE;
    const uint32_t T = plan->T, n_items = (uint32_t)w.items.size();
    std::vector<uint8_t> packed(n_items * sizeof(tsr::FaItem) + 8u * (size_t)T);
    memcpy(packed.data(), w.items.data(), n_items * sizeof(tsr::FaItem));
    memcpy(packed.data() + n_items * sizeof(tsr::FaItem), w.tok.data(), 8u * (size_t)T);
    bool general = false;
    for (const tsr::FaItem & it : w.items) general |= it.general != 0u;
    const uint32_t mstride = 16u * ((msum[2] + 15u) / 16u);
    uint32_t seg_work = 0u;
    for (const tsr::FaItem & it : w.items)
        for (uint32_t c = 0; c < 4u; ++c) {                     // k_fa_dec.hip FaSeg: channel c's groups
            const uint32_t uf = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u), ue = it.u0 + it.n;
            const uint32_t nu = uf < ue ? (ue - 1u - uf) / 4u + 1u : 0u;
            seg_work += (nu + 3u) / 4u;
        }
    // the one launch of the Q|K|V rows + attention: the workgroups with work resident at once (4 per
    // CU); with more, the row workgroups hold slots that segments need (measured at the Llama-3-8B
    // shape: 8208 cells 24.8 -> 26.3 us in one launch, 4136 cells 20.1 -> 18.9 us)
    const uint32_t D = plan->D, nkv = plan->n_head_kv, G = plan->n_head / nkv;
    const bool qkv_fits = T == 1u && ctx->n_cu > 0 &&
                          ((uint64_t)seg_work + G * (D / 64u) + ((G + 2u) * D + 23u) / 24u) * nkv <=
                              4u * (uint64_t)ctx->n_cu;
    const bool changed = !plan->set || n_items != plan->n_items || w.maxtiles != plan->maxtiles ||
                         w.max_groups != plan->max_groups || (general && mstride != plan->mstride) ||
                         general != plan->general || qkv_fits != plan->qkv_fits;
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    if (tsr_capturing(s)) return TSR_HIP_E_ARG;      // the copy is made at each call, outside any graph
    // the tok arrays sit right after the items of this list: a launch baked with another n_items reads
    // them at another offset, which is why a changed shape asks for a new capture
    if ((rc = ctx->staging.copy(plan->dev + plan->o_items, packed.data(), packed.size(), s)) != 0) return rc;
    plan->set = true;
    plan->n_items = n_items;
    plan->maxtiles = w.maxtiles;
    plan->max_groups = w.max_groups;
    plan->mstride = mstride;
    plan->general = general;
    plan->cells = w.cells;
    plan->seg_work = seg_work;
    plan->qkv_fits = qkv_fits;
    if (shape_changed) *shape_changed = changed ? 1 : 0;
    return TSR_HIP_OK;
}

// The planned FLASH_ATTN_EXT launch (optionally with ROPE + SET_ROWS_KV in the score kernel).
static bool aligned16(const void * p) { return ((uintptr_t)p & 15u) == 0u; }

// The Q|K|V MUL_MAT computed inside the one-launch decode form (tsr_hip_attn_qkv_plan_rope_tab).
struct QkvIn {
    const tsr_hip_weight * w;
    const float * x;
    const float * pw;
    float eps;
};

static int fa_plan_launch(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * q_dev, uint64_t q_stride,
                          const tsr_hip_kv * kc, const tsr_hip_kv * vc, float scale, const float * mask_f32_dev,
                          float * out_dev, uint64_t out_stride, const tsr::FaArgs * rope, void * stream,
                          const QkvIn * qkv = nullptr) {
    if (ctx == nullptr || plan == nullptr || q_dev == nullptr || kc == nullptr || vc == nullptr || out_dev == nullptr)
        return TSR_HIP_E_ARG;
    if (!plan->set || (plan->general && mask_f32_dev == nullptr)) return TSR_HIP_E_MASK;
    int rc = fa_check_shape(plan->D, plan->n_head, plan->n_head_kv, scale);
    if (rc) return rc;
    const uint32_t E = plan->n_head_kv * plan->D, K = plan->n_head * plan->D, T = plan->T;
    if (kc->E != E || vc->E != E || kc->kv_size != vc->kv_size || kc->kv_size < plan->kv_size) return TSR_HIP_E_SHAPE;
    if (((uintptr_t)q_dev & 15u) != 0u || (T > 1u && (q_stride % 4u != 0u || q_stride < K)) || (T > 1u && out_stride < K))
        return TSR_HIP_E_ARG;
    const uint32_t G = plan->n_head / plan->n_head_kv;
    if (T == 1u && G <= 4u && (plan->D == 64u || plan->D == 128u) && plan->n_items <= 256u) {
        // one decode row: the one-launch form, one workgroup per ATTPV segment (k_fa_dec.hip)
        tsr::FaDecArgs d{};
        d.q = q_dev;
        d.kc = kv_args(kc);
        d.vc = kv_args(vc);
        d.D = plan->D;
        d.G = G;
        d.n_head = plan->n_head;
        d.n_head_kv = plan->n_head_kv;
        d.E = E;
        d.scale = scale;
        d.mask = mask_f32_dev;
        d.mstride = plan->mstride;
        d.items = (const tsr::FaItem *)(plan->dev + plan->o_items);
        d.n_items = plan->n_items;
        d.maxtiles = plan->maxtiles;
        d.seg_o = (uint64_t *)(plan->dev + plan->o_SO);
        d.seg_l = (uint64_t *)(plan->dev + plan->o_SL);
        d.m_item = (uint64_t *)(plan->dev + plan->o_MI);
        d.keys = (uint32_t *)(plan->dev + plan->o_TK);
        d.ep = (uint32_t *)(plan->dev + plan->o_EP);
        d.spin_max = ctx->fa_spin_max;
        d.n_xcd = ctx->n_xcd;
        if (qkv != nullptr) {                                // 24 rows per workgroup, first in dispatch order
            d.qkv_w = qkv->w->dev;
            d.qkv_x = qkv->x;
            d.qkv_pw = qkv->pw;
            d.qkv_y = const_cast<float *>(q_dev);
            d.qkv_flag = (uint32_t *)(plan->dev + plan->o_QF);
            d.qkv_N = qkv->w->N;
            d.qkv_K = qkv->w->K;
            d.qkv_rb = qkv->w->rb;
            d.nq = ((G + 2u) * plan->D + 23u) / 24u;
            d.qkv_eps = qkv->eps;
            d.qkv_inv_n = 1.0f / (float)qkv->w->K;          // correctly rounded (IEEE division), as the matvec's
        }
        {   // reducers first when the grid is resident at once (4 workgroups per CU: the kernel holds 4 or 5)
            const uint64_t wgs = ((uint64_t)plan->n_items * plan->maxtiles * 4u + G * (plan->D / 64u) + d.nq) *
                                 plan->n_head_kv;
            d.red_first = ctx->n_cu > 0 && wgs <= 4u * (uint64_t)ctx->n_cu ? 1u : 0u;
        }
        d.out = out_dev;
        d.ex = ctx->expk;
        d.bad = ctx->flags_dev;                              // the rope form below names its own
        if (rope != nullptr) {
            d.rtab = rope->rtab;
            d.pos = rope->pos;
            d.cell = rope->cell;
            d.bad = ctx->flag(rope->bad);
            d.n_dims = rope->n_dims;
            d.neox = rope->neox;
            d.ts = rope->ts;
            d.m = rope->m;
        }
        std::lock_guard<std::mutex> lk(ctx->mtx);
        (void)hipSetDevice(ctx->device);
        ctx->ctr.flash_attn_calls++;
        ctx->ctr.fa_dec_launches++;
        ctx->ctr.flash_attn_kv_bytes += plan->cells * (uint64_t)E / 32u * 34u * 2u;
        if (rope != nullptr) ctx->ctr.set_rows_calls += 2u;
        if (qkv != nullptr) {
            ctx->ctr.fa_dec_qkv_launches++;
            ctx->ctr.mul_mat_calls++;
            ctx->ctr.mul_mat_rows += qkv->w->N;
            ctx->ctr.mul_mat_weight_bytes += (uint64_t)qkv->w->N * (qkv->w->K / 256u) * 144u;
        }
        return tsr_launch_fa_dec(d, ctx->pick(stream)) ? TSR_HIP_E_HIP : TSR_HIP_OK;
    }
    if (qkv != nullptr) return TSR_HIP_E_SHAPE;              // (the caller checked the decode form)
    tsr::FaPlan p{};
    p.n_items = plan->n_items;
    p.maxtiles = plan->maxtiles;
    tsr::FaArgs a = fa_args(ctx, q_dev, q_stride, kc, vc, plan->D, plan->n_head, plan->n_head_kv, scale, mask_f32_dev,
                            plan->mstride, out_dev, out_stride);
    a.items = (const tsr::FaItem *)(plan->dev + plan->o_items);
    a.tok_first = (const uint32_t *)(plan->dev + plan->o_items + (size_t)plan->n_items * sizeof(tsr::FaItem));
    a.tok_count = a.tok_first + T;
    a.S = (float *)(plan->dev + plan->o_S);
    a.Mpart = (float *)(plan->dev + plan->o_Mp);
    a.OP = (float *)(plan->dev + plan->o_OP);
    a.LP = (float *)(plan->dev + plan->o_LP);
    a.max_groups = plan->max_groups;
    if (rope != nullptr) {
        a.rtab = rope->rtab;
        a.pos = rope->pos;
        a.cell = rope->cell;
        a.bad = ctx->flag(rope->bad);
        a.n_dims = rope->n_dims;
        a.neox = rope->neox;
        a.ts = rope->ts;
        a.m = rope->m;
    }
    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    ctx->ctr.flash_attn_calls++;
    ctx->ctr.flash_attn_kv_bytes += plan->cells * (uint64_t)E / 32u * 34u * 2u;
    if (rope != nullptr) ctx->ctr.set_rows_calls += 2u;
    return tsr_launch_fa(a, p, T, (uint32_t)ctx->n_cu, ctx->pick(stream)) ? TSR_HIP_E_HIP : TSR_HIP_OK;
}

int tsr_hip_flash_attn_plan(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * q_dev, uint64_t q_stride,
                            const tsr_hip_kv * kc, const tsr_hip_kv * vc, float scale, const float * mask_f32_dev,
                            float * out_dev, uint64_t out_stride, void * stream) {
    return fa_plan_launch(ctx, plan, q_dev, q_stride, kc, vc, scale, mask_f32_dev, out_dev, out_stride, nullptr, stream);
}

// The shape the score kernel's ROPE form takes: one token, K rows in registers (D <= 128), the query
// slots and the k and v rows of a KV head in one pass of its 256 threads, one angle per lane.
static int fa_rope_args(const tsr_hip_fa_plan * plan, uint32_t n_dims, int mode, const int64_t * cell_dev,
                        int32_t * bad_dev, tsr::FaArgs & r) {
    if (plan == nullptr || cell_dev == nullptr) return TSR_HIP_E_ARG;
    if (mode != TSR_HIP_ROPE_NORMAL && mode != TSR_HIP_ROPE_NEOX && mode != TSR_HIP_ROPE_IMROPE) return TSR_HIP_E_SHAPE;
    const uint32_t D = plan->D, G = plan->n_head_kv ? plan->n_head / plan->n_head_kv : 0u;
    if (plan->T != 1u || (D != 64u && D != 128u) || (G + 2u) * D > 1024u || n_dims < 8u || n_dims % 8u != 0u ||
        n_dims > D || n_dims / 2u > 64u)
        return TSR_HIP_E_SHAPE;
    r = tsr::FaArgs{};
    r.cell = cell_dev;
    r.bad = bad_dev;
    r.n_dims = n_dims;
    r.neox = mode != TSR_HIP_ROPE_NORMAL ? 1u : 0u;
    return TSR_HIP_OK;
}

int tsr_hip_flash_attn_plan_rope(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * qkv_dev,
                                 tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                 const int32_t * pos_dev, float freq_base, float attn_factor, const int64_t * cell_dev,
                                 int32_t * bad_dev, const float * mask_f32_dev, float * out_dev, uint64_t out_stride,
                                 void * stream) {
    if (ctx == nullptr || pos_dev == nullptr) return TSR_HIP_E_ARG;
    tsr::FaArgs r;
    const int rc = fa_rope_args(plan, n_dims, mode, cell_dev, bad_dev, r);
    if (rc) return rc;
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base)) return TSR_HIP_E_ARG;
    r.pos = pos_dev;
    r.ts = powf(freq_base, -2.0f / (float)n_dims);                  // the host libm, as tsr_hip_rope
    r.m = attn_factor;
    return fa_plan_launch(ctx, plan, qkv_dev, 0u, kc, vc, scale, mask_f32_dev, out_dev, out_stride, &r, stream);
}

int tsr_hip_flash_attn_plan_rope_tab(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * qkv_dev,
                                     tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                     const float * tab_dev, const int64_t * cell_dev, int32_t * bad_dev,
                                     const float * mask_f32_dev, float * out_dev, uint64_t out_stride, void * stream) {
    if (ctx == nullptr || tab_dev == nullptr || ((uintptr_t)tab_dev & 7u) != 0u) return TSR_HIP_E_ARG;
    tsr::FaArgs r;
    const int rc = fa_rope_args(plan, n_dims, mode, cell_dev, bad_dev, r);
    if (rc) return rc;
    r.rtab = tab_dev;
    return fa_plan_launch(ctx, plan, qkv_dev, 0u, kc, vc, scale, mask_f32_dev, out_dev, out_stride, &r, stream);
}

// MUL_MAT_NORM of the Q|K|V weight, then the planned FLASH_ATTN_EXT with ROPE + SET_ROWS_KV, in one launch
// when the decode form places every workgroup of a KV head on one XCD: the KV head's Q|K|V rows are
// computed by workgroups of the same launch on that XCD while its segments already load K.
int tsr_hip_attn_qkv_plan_rope_tab(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const tsr_hip_weight * w_qkv,
                                   const float * x_dev, float eps, const float * norm_w_dev, float * qkv_dev,
                                   tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                   const float * tab_dev, const int64_t * cell_dev, int32_t * bad_dev,
                                   const float * mask_f32_dev, float * out_dev, uint64_t out_stride, void * stream) {
    if (ctx == nullptr || plan == nullptr || w_qkv == nullptr || x_dev == nullptr || qkv_dev == nullptr ||
        tab_dev == nullptr || ((uintptr_t)tab_dev & 7u) != 0u)
        return TSR_HIP_E_ARG;
    const uint32_t D = plan->D, nkv = plan->n_head_kv, G = nkv ? plan->n_head / nkv : 0u;
    if (w_qkv->N != (plan->n_head + 2u * nkv) * D) return TSR_HIP_E_SHAPE;
    tsr::FaArgs r;
    int rc = fa_rope_args(plan, n_dims, mode, cell_dev, bad_dev, r);
    if (rc) return rc;
    r.rtab = tab_dev;
    const uint32_t K = w_qkv->K;
    // byte ranges that the one launch reads (x, the norm weights) while it writes others (the Q|K|V row,
    // the attention output of KV heads that finished): apart, or the two calls run
    auto apart = [](const void * a, size_t na, const void * b, size_t nb) {
        return a == nullptr || b == nullptr || (uintptr_t)a + na <= (uintptr_t)b || (uintptr_t)b + nb <= (uintptr_t)a;
    };
    const size_t out_span = 4u * (size_t)plan->n_head * D;
    const bool disjoint = apart(qkv_dev, 4u * (size_t)w_qkv->N, x_dev, 4u * (size_t)K) &&
                          apart(out_dev, out_span, x_dev, 4u * (size_t)K) &&
                          apart(out_dev, out_span, norm_w_dev, 4u * (size_t)K);
    const bool one = plan->set && !(plan->general && mask_f32_dev == nullptr) && G <= 4u && plan->n_items <= 256u &&
                     ctx->n_xcd != 0u && nkv % ctx->n_xcd == 0u && w_qkv->fmt == TSR_HIP_FMT_Q4_K && K % 256u == 0u &&
                     K <= 4096u && aligned16(x_dev) && (norm_w_dev == nullptr || aligned16(norm_w_dev)) &&
                     aligned16(qkv_dev) && disjoint && plan->qkv_fits;
    if (!one) {                                                   // the two records, two launches
        rc = tsr_hip_mul_mat_norm(ctx, w_qkv, x_dev, 1u, K, eps, norm_w_dev, qkv_dev, w_qkv->N, nullptr, 0u, 0u, stream);
        if (rc) return rc;
        return fa_plan_launch(ctx, plan, qkv_dev, 0u, kc, vc, scale, mask_f32_dev, out_dev, out_stride, &r, stream);
    }
    const QkvIn q{ w_qkv, x_dev, norm_w_dev, eps };
    return fa_plan_launch(ctx, plan, qkv_dev, 0u, kc, vc, scale, mask_f32_dev, out_dev, out_stride, &r, stream, &q);
}
