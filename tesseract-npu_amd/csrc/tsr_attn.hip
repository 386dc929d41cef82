// tsr_attn.hip -- host side of the KV cache, the mask summary and FLASH_ATTN_EXT.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
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
    return tsr_launch_kv_set_rows(kv_args(kv), which, src_dev, n_rows, src_stride, idx_dev, bad_dev, ctx->pick(stream))
               ? TSR_HIP_E_HIP
               : TSR_HIP_OK;
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
bool plan_row(uint32_t E, uint32_t D, const uint32_t * words, uint32_t q, const uint32_t (*new_runs)[2],
              uint32_t n_new, std::vector<Chunk> & out) {
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

}  // namespace

int tsr_hip_flash_attn(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride, const tsr_hip_kv * kc,
                       const tsr_hip_kv * vc, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                       const uint32_t * msum, const float * mask_f32_dev, const uint32_t (*new_runs)[2], uint32_t n_new,
                       float * out_dev, uint64_t out_stride, void * stream) {
    if (ctx == nullptr || q_dev == nullptr || kc == nullptr || vc == nullptr || msum == nullptr || out_dev == nullptr ||
        T == 0u || (n_new && new_runs == nullptr))
        return TSR_HIP_E_ARG;
    if (!(D == 64u || D == 128u || D == 256u || D == 512u)) return TSR_HIP_E_SHAPE;
    if (n_head_kv == 0u || n_head % n_head_kv != 0u || n_head / n_head_kv > 64u) return TSR_HIP_E_SHAPE;
    const uint32_t E = n_head_kv * D, G = n_head / n_head_kv, K = n_head * D;
    if (kc->E != E || vc->E != E || kc->kv_size != vc->kv_size || E / 64u > 511u || (uint64_t)G * E > 32768u || K > 32768u)
        return TSR_HIP_E_SHAPE;
    uint32_t sb;
    memcpy(&sb, &scale, 4);
    if ((sb >> 31) || (sb & 0x7F800000u) == 0u || (sb & 0x7F800000u) == 0x7F800000u) return TSR_HIP_E_SHAPE;
    if (msum[0] != 0x4D55534Du || msum[1] != T || msum[2] > kc->kv_size) return TSR_HIP_E_MASK;
    if (((uintptr_t)q_dev & 15u) != 0u || (T > 1u && (q_stride % 4u != 0u || q_stride < K)) ||
        (T > 1u && out_stride < K) || T > 65535u)
        return TSR_HIP_E_ARG;

    // plan every token row; flatten into items (chunks) with their 256-cell score tiles
    std::vector<tsr::FaItem> items;
    std::vector<uint32_t> tok(2u * (size_t)T);                    // tok_first [T] | tok_count [T]
    std::vector<Chunk> ch;
    uint64_t cells = 0;
    uint32_t n_tiles = 0, maxtiles = 1;
    for (uint32_t t = 0; t < T; ++t) {
        ch.clear();
        if (!plan_row(E, D, msum, t, new_runs, n_new, ch)) return TSR_HIP_E_MASK;
        tok[t] = (uint32_t)items.size();
        tok[T + t] = (uint32_t)ch.size();
        for (const Chunk & c : ch) {
            if (c.general && mask_f32_dev == nullptr) return TSR_HIP_E_MASK;
            tsr::FaItem it{};
            it.t = t;
            it.u0 = c.u0;
            it.n = c.n;
            it.c_lo = c.c_lo;
            it.c_hi = c.c_hi;
            it.general = c.general;
            it.s_off = (uint32_t)cells;
            it.tile0 = n_tiles;
            it.ntiles = (16u * c.n + 255u) / 256u;
            n_tiles += it.ntiles;
            maxtiles = std::max(maxtiles, it.ntiles);
            cells += 16u * c.n;
            items.push_back(it);
        }
    }
    const size_t n_items = items.size();
    if (cells * n_head > 0xFFFFFFFFull || n_items * 4u > 0x7FFFFFFFull || n_items * maxtiles > 0x7FFFFFFFull)
        return TSR_HIP_E_SHAPE;
    const bool inl = n_items <= tsr::kFaInlItems && T <= tsr::kFaInlTok;
    size_t off = 0;
    const size_t o_items = off; off = up256(off + (inl ? 0u : n_items * sizeof(tsr::FaItem) + 8u * (size_t)T));
    const size_t o_S = off; off = up256(off + 4u * (size_t)cells * n_head);
    const size_t o_Mp = off; off = up256(off + 4u * (size_t)n_tiles * n_head);
    const size_t o_OP = off; off = up256(off + 4u * n_items * kC * n_head * D);
    const size_t o_LP = off; off = up256(off + 4u * n_items * kC * n_head);

    tsr::FaPlan p{};
    p.n_items = (uint32_t)n_items;
    p.maxtiles = maxtiles;
    std::vector<uint8_t> packed;
    if (inl) {
        std::copy(items.begin(), items.end(), p.items);
        for (uint32_t t = 0; t < T; ++t) { p.tok_first[t] = tok[t]; p.tok_count[t] = tok[T + t]; }
    } else {                                                      // items | tok_first | tok_count, one copy
        packed.resize(n_items * sizeof(tsr::FaItem) + 8u * (size_t)T);
        memcpy(packed.data(), items.data(), n_items * sizeof(tsr::FaItem));
        memcpy(packed.data() + n_items * sizeof(tsr::FaItem), tok.data(), 8u * (size_t)T);
    }

    std::lock_guard<std::mutex> lk(ctx->mtx);
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->pick(stream);
    int rc = ctx->scratch.reserve(off, s);
    if (rc) return rc;
    uint8_t * base = (uint8_t *)ctx->scratch.ptr;
    if (!inl) {
        // a host-to-device copy of a host vector cannot be recorded into a graph (the vector is gone
        // when the graph replays): long work lists are for eager calls
        if (tsr_capturing(s)) return TSR_HIP_E_ARG;
        rc = hip_err(hipMemcpyAsync(base + o_items, packed.data(), packed.size(), hipMemcpyHostToDevice, s), "fa plan");
        if (rc) return rc;
    }

    tsr::FaArgs a{};
    a.q = q_dev;
    a.q_stride = q_stride;
    a.kc = kv_args(kc);
    a.vc = kv_args(vc);
    a.D = D;
    a.G = G;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.E = E;
    a.scale = scale;
    a.mask = mask_f32_dev;
    a.mstride = 16u * ((msum[2] + 15u) / 16u);
    if (!inl) {
        a.items = (const tsr::FaItem *)(base + o_items);
        a.tok_first = (const uint32_t *)(base + o_items + n_items * sizeof(tsr::FaItem));
        a.tok_count = a.tok_first + T;
    }
    a.S = (float *)(base + o_S);
    a.Mpart = (float *)(base + o_Mp);
    a.OP = (float *)(base + o_OP);
    a.LP = (float *)(base + o_LP);
    for (const tsr::FaItem & i : items) a.max_groups = std::max(a.max_groups, i.n);
    a.out = out_dev;
    a.out_stride = out_stride;
    a.ex = ctx->expk;
    ctx->ctr.flash_attn_calls++;
    ctx->ctr.flash_attn_kv_bytes += cells * (uint64_t)E / 32u * 34u * 2u;
    return tsr_launch_fa(a, p, T, (uint32_t)ctx->n_cu, s) ? TSR_HIP_E_HIP : TSR_HIP_OK;
}
