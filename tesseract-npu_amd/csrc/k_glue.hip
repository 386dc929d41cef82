// k_glue.hip -- the decode-layer glue ops on gfx950, bit-exact to the reference's vector unit
// (sw/sim/tsr_ref_vu.c, tsr_ref_math.c) on the f32 rules of tsr_dev.hpp: RMS_NORM with the weight
// MUL, ROPE (NORM / NEOX), SWIGLU, ADD, GET_ROWS and ARGMAX. Every output row holds n words.
#include "expk.hpp"
#include "glue.hpp"
#include "kernels.hpp"
#include "kvstore.hpp"
#include "mv_q4k.hpp"
#include "qact.hpp"
#include "tsr_dev.hpp"

namespace tsr {


// ---- RMS_NORM (sw/sim/tsr_ref_vu.c:171-263, 102-133; sw/ctrl/ref/rmsnorm_ref.hpp:11-14) ---------
// One workgroup of 128 threads per row: thread i holds the RED partial p_i (glue.hpp), the tree runs
// on DPP / swizzles and through LDS for its last level, s = RC(SQ(FA(FM(sum, inv_n), eps))), then
// y = FM(FM(x, s), w). The partials and their sums are rule results (never subnormal). The row is read
// in batches of kRmsBatch values per thread with all loads of a batch in flight at once; a row of at
// most 128 kRmsBatch values is read once and kept in registers, its norm weights loaded with it, and
// its products are the plain ones when the wave qualifies (prep_norm_apply_fast, 16 values at a time),
// the full rule otherwise. y may be x: every element is read by the thread that writes it, before it
// writes it.
constexpr uint32_t kRmsBatch = 32;

__global__ __launch_bounds__(128) void k_rms_norm(const float * x, uint64_t x_stride, uint32_t n, float eps, float inv_n,
                                                  const float * w, uint64_t w_stride, uint32_t w_period, float * y,
                                                  uint64_t y_stride) {
    __shared__ float s_hi, s_scale;
    const uint32_t r = blockIdx.x, i = threadIdx.x;
    const float * xr = x + (size_t)r * x_stride;
    const float * wr = w ? w + (size_t)(r % w_period) * w_stride : nullptr;
    float * yr = y + (size_t)r * y_stride;
    const bool kept = n <= 128u * kRmsBatch;                      // v holds the whole row
    float4 v[kRmsBatch / 4u], wv[kRmsBatch / 4u];                  // value k: component k % 4 of [k / 4]
    auto at = [](float4 (&a)[kRmsBatch / 4u], uint32_t k) -> float & {
        float4 & q = a[k >> 2];
        return (k & 3u) == 0u ? q.x : ((k & 3u) == 1u ? q.y : ((k & 3u) == 2u ? q.z : q.w));
    };
    float p = 0.0f;
    for (uint32_t j0 = 0; j0 < n; j0 += 128u * kRmsBatch) {
#pragma unroll
        for (uint32_t k = 0; k < kRmsBatch; ++k) {
            const uint32_t j = j0 + i + 128u * k;
            at(v, k) = j < n ? xr[j] : 0.0f;
        }
        if (kept) {                                               // the weights in flight with x
#pragma unroll
            for (uint32_t k = 0; k < kRmsBatch; ++k) {
                const uint32_t j = i + 128u * k;
                at(wv, k) = (wr && j < n) ? wr[j] : 0.0f;
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kRmsBatch; ++k)
            if (j0 + i + 128u * k < n) p = p + sq_rule(at(v, k));   // = FA(p, FM(v, v)): see rms_tree64
    }
    p = rms_tree64(p);
    if (i == 64u) s_hi = p;                                       // partials 64 .. 127
    __syncthreads();
    if (i == 0u) s_scale = rms_scale(p, s_hi, inv_n, eps);
    __syncthreads();
    const float s = s_scale;
    const bool has_w = wr != nullptr;
    if (kept) {
#pragma unroll
        for (uint32_t h = 0; h < kRmsBatch / 16u; ++h) {
            float4 (&vh)[4] = *reinterpret_cast<float4 (*)[4]>(&v[4u * h]);
            const float4 (&wh)[4] = *reinterpret_cast<const float4 (*)[4]>(&wv[4u * h]);
            if (!prep_norm_apply_fast(vh, s, wh, has_w)) {
#pragma unroll
                for (uint32_t c = 0; c < 4u; ++c) vh[c] = prep_norm_apply(vh[c], s, wh[c], has_w);
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kRmsBatch; ++k) {
            const uint32_t j = i + 128u * k;
            if (j < n) yr[j] = at(v, k);
        }
        return;
    }
    for (uint32_t j0 = 0; j0 < n; j0 += 128u * kRmsBatch) {
#pragma unroll
        for (uint32_t k = 0; k < kRmsBatch; ++k) {
            const uint32_t j = j0 + i + 128u * k;
            at(v, k) = j < n ? xr[j] : 0.0f;
            at(wv, k) = (wr && j < n) ? wr[j] : 0.0f;
        }
#pragma unroll
        for (uint32_t k = 0; k < kRmsBatch; ++k) {
            const uint32_t j = j0 + i + 128u * k;
            if (j < n) {
                const float t = smul(at(v, k), s);
                yr[j] = wr ? smul(t, at(wv, k)) : t;
            }
        }
    }
}

// ---- ROPE (sw/sim/tsr_ref_vu.c:308-376) -----------------------------------------------------------
// Workgroup (token, group of kRopeHeads heads). Every thread first loads the pairs it rotates; one
// lane runs the angle recurrence (rope_angles); the lanes then take sin / cos of the angles,
// c = FM(M, cos), s = FM(M, sin); every thread rotates its (head, pair)s: y0 = FS(FM(x0, c), FM(x1, s)),
// y1 = FA(FM(x0, s), FM(x1, c)), pairs (2i, 2i+1) or (i, i + n_dims/2); dims from n_dims on are
// copied raw. Every word is read before any is written (y may be x).
constexpr uint32_t kRopeHeads = 8, kRopeThreads = 256, kRopePairs = kRopeHeads * 512u / kRopeThreads;

__global__ __launch_bounds__(kRopeThreads) void k_rope(RopeArgs a) {
    __shared__ float s_phi[512], s_c[512], s_s[512];
    const uint32_t t = blockIdx.x, half = a.n_dims / 2u;
    const uint32_t h0 = blockIdx.y * kRopeHeads, hn = min(kRopeHeads, a.n_heads - h0);
    const float * xt = a.x + (size_t)t * a.x_stride;
    float * yt = a.y + (size_t)t * a.y_stride;
    const int32_t pos = a.pos[t];
    float x0[kRopePairs], x1[kRopePairs];
#pragma unroll
    for (uint32_t k = 0; k < kRopePairs; ++k) {
        const uint32_t idx = threadIdx.x + kRopeThreads * k;
        if (idx < hn * half) {
            const uint32_t h = h0 + idx / half, i = idx % half;
            const float * xr = xt + (size_t)h * a.head_dim;
            x0[k] = xr[a.neox ? i : 2u * i];
            x1[k] = xr[a.neox ? i + half : 2u * i + 1u];
        }
    }
    const uint32_t tail = a.head_dim - a.n_dims;
    for (uint32_t idx = threadIdx.x; idx < hn * tail; idx += blockDim.x) {
        const size_t o = (size_t)(h0 + idx / tail) * a.head_dim + a.n_dims + idx % tail;
        ((uint32_t *)yt)[o] = ((const uint32_t *)xt)[o];
    }
    if (threadIdx.x == 0u) rope_angles(pos, half, a.ts, a.ff, a.freq_scale, a.fs != 0u, s_phi);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
        float sn, cs;
        dsincos(s_phi[i], &sn, &cs);
        s_c[i] = smul(a.m, cs);
        s_s[i] = smul(a.m, sn);
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kRopePairs; ++k) {
        const uint32_t idx = threadIdx.x + kRopeThreads * k;
        if (idx < hn * half) {
            const uint32_t h = h0 + idx / half, i = idx % half;
            float * yr = yt + (size_t)h * a.head_dim;
            const float c = s_c[i], sn = s_s[i];
            yr[a.neox ? i : 2u * i] = ssub(smul(x0[k], c), smul(x1[k], sn));
            yr[a.neox ? i + half : 2u * i + 1u] = sadd(smul(x0[k], sn), smul(x1[k], c));
        }
    }
}

// ---- ROPE + SET_ROWS_KV (the decode layer's q / k rotation and KV store in one launch) --------------
// One workgroup per token. The token's Q|K|V row is staged in LDS (so the in-place rotation reads
// only staged words); one lane runs the angle recurrence while the row loads. Work unit = 4
// consecutive values: a q or k unit is rotated (k_rope's formulas; its partners come from LDS) and
// written back in place; a k unit is then QACT A32'd (8 lanes per 32-value block, k_kv_set_rows'
// rule) and stored at the token's cache cell, and so is every v unit. head_dim % 32 == 0, so every
// block's 8 units are one aligned group of 8 lanes. A cell outside the caches stores nothing and
// raises *bad (the rotation still happens, as ROPE then SET_ROWS would do).
constexpr uint32_t kRkThreads = 512, kRkMaxRow = 16384;

__device__ __forceinline__ float rk_value(const float * row, uint32_t j, uint32_t head_dim, uint32_t n_dims,
                                          uint32_t half, bool neox, const float * c, const float * sn) {
    const uint32_t jh = j % head_dim, hb = j - jh;
    if (jh >= n_dims) return row[j];
    uint32_t i, j0, j1;
    if (neox) { i = jh < half ? jh : jh - half; j0 = hb + i; j1 = hb + i + half; }
    else { i = jh >> 1; j0 = hb + 2u * i; j1 = j0 + 1u; }
    const float x0 = row[j0], x1 = row[j1];
    return j == j0 ? ssub(smul(x0, c[i]), smul(x1, sn[i])) : sadd(smul(x0, sn[i]), smul(x1, c[i]));
}

__global__ __launch_bounds__(kRkThreads) void k_rope_kv(RopeKvArgs a) {
    extern __shared__ __align__(16) float s_row[];
    __shared__ float s_phi[512], s_c[512], s_s[512];
    const uint32_t t = blockIdx.x, half = a.n_dims / 2u;
    const uint32_t nq = a.n_head * a.head_dim, E = a.n_head_kv * a.head_dim, nrow = nq + 2u * E;
    float * row = a.qkv + (size_t)t * a.stride;
    const int32_t pos = a.pos[t];
    const int64_t cell64 = a.cell[t];
    for (uint32_t u = threadIdx.x; u < nrow / 4u; u += blockDim.x)
        *(float4 *)(s_row + 4u * u) = *(const float4 *)(row + 4u * u);
    if (threadIdx.x == 0u) rope_angles(pos, half, a.ts, nullptr, 1.0f, false, s_phi);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
        float sn, cs;
        dsincos(s_phi[i], &sn, &cs);
        s_c[i] = smul(a.m, cs);
        s_s[i] = smul(a.m, sn);
    }
    __syncthreads();
    const bool cell_ok = cell64 >= 0 && cell64 < (int64_t)a.kc.kv_size && cell64 < (int64_t)a.vc.kv_size;
    if (!cell_ok && threadIdx.x == 0u && a.bad != nullptr) *a.bad = 1;
    const uint32_t cell = cell_ok ? (uint32_t)cell64 : 0u;
    for (uint32_t u = threadIdx.x; u < nrow / 4u; u += blockDim.x) {     // units of one 8-group: one trip count
        const uint32_t j = 4u * u;
        float4 v;
        if (j < nq + E) {
            v.x = rk_value(s_row, j, a.head_dim, a.n_dims, half, a.neox != 0u, s_c, s_s);
            v.y = rk_value(s_row, j + 1u, a.head_dim, a.n_dims, half, a.neox != 0u, s_c, s_s);
            v.z = rk_value(s_row, j + 2u, a.head_dim, a.n_dims, half, a.neox != 0u, s_c, s_s);
            v.w = rk_value(s_row, j + 3u, a.head_dim, a.n_dims, half, a.neox != 0u, s_c, s_s);
            *(float4 *)(row + j) = v;
        } else {
            v = *(const float4 *)(s_row + j);
        }
        if (j >= nq) {
            float D;
            const uint32_t q = qact_a32_lane(v, &D);
            const bool isk = j < nq + E;
            const uint32_t i = j - nq - (isk ? 0u : E);
            if (cell_ok) kv_store_unit(isk ? a.kc : a.vc, isk ? 0u : 1u, cell, i, q, D, (u & 7u) == 0u);
        }
    }
}

// ---- SWIGLU and ADD (sw/sim/tsr_ref_vu.c:102-133; sw/sim/tsr_ref_math.c:165-172) -------------------
// SILU(x) = FM(x, RC(FA(1, EXPK(x, N1)))), EXPK(x, N1) = EXPK(-x, P1); SWIGLU = FM(SILU(g), u).
// The angles of one position (rope_cs_lane of lane i < half): tab[2 i] = FM(M, cos theta_i),
// tab[2 i + 1] = FM(M, sin theta_i). One wave.
__global__ __launch_bounds__(64) void k_rope_table(const int32_t * pos, uint32_t half, float ts, float m, float * tab) {
    float c, s;
    rope_cs_lane(*pos, half, ts, m, threadIdx.x, &c, &s);
    if (threadIdx.x < half) *(float2 *)(tab + 2u * threadIdx.x) = make_float2(c, s);
}

// The MVM record's local scale (sw/sim/tsr_sim.c:1648-1667), applied to a stored MUL_MAT result:
// SOFTCAP y = FM(TANH(FM(y, fs)), sc), SCALE y = FM(y, sc). Thread = one value; the EXPK table in LDS.
__global__ __launch_bounds__(256) void k_mm_epilogue(float * y, uint64_t y_stride, uint32_t N, uint32_t mode, float fs,
                                                     float sc, ExpkTab ex) {
    __shared__ uint32_t s_t64[64];
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = ex.t64[threadIdx.x];
    __syncthreads();
    const uint32_t n = blockIdx.x * 256u + threadIdx.x;
    if (n >= N) return;
    float * p = y + (size_t)blockIdx.y * y_stride + n;
    const float v = *p;
    const uint32_t * t64 = s_t64;
    *p = mode == kEpiSoftcap ? smul(tanh_with(smul(v, fs), ex, [t64](uint32_t j) { return t64[j]; }), sc) : smul(v, sc);
}

__global__ __launch_bounds__(256) void k_swiglu(const float * g, uint64_t g_stride, const float * u, uint64_t u_stride,
                                                float * y, uint64_t y_stride, uint32_t n, uint32_t rows, ExpkTab ex) {
    __shared__ uint32_t s_t64[64];
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = ex.t64[threadIdx.x];
    __syncthreads();
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float gv = g[(size_t)r * g_stride + j], uv = u[(size_t)r * u_stride + j];
        const float sig = srcp(sadd(1.0f, expk(fneg(gv), ex, s_t64)));
        y[(size_t)r * y_stride + j] = smul(smul(gv, sig), uv);
    }
}

// ADD (the ew kind, sw/ggml-tesseract/tsr-build.cpp:289-332): y = FA(a, b), row r of b at
// b + (r % b_period) * b_stride (a row broadcast with period b_period).
__global__ __launch_bounds__(256) void k_add(const float * a, uint64_t a_stride, const float * b, uint64_t b_stride,
                                             uint32_t b_period, float * y, uint64_t y_stride, uint32_t n, uint32_t rows) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y)
        y[(size_t)r * y_stride + j] = sadd(a[(size_t)r * a_stride + j], b[(size_t)(r % b_period) * b_stride + j]);
}

// ---- GET_ROWS (sw/ctrl/ref/elem_ref.hpp:17-20): rows copied bit for bit; an id outside [0, n_src)
// copies nothing and raises the flag ------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_get_rows(const uint32_t * src, uint64_t src_stride, uint32_t n, uint32_t n_src,
                                                  const int32_t * ids, uint32_t count, uint32_t * dst, uint64_t dst_stride,
                                                  int32_t * bad) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    for (uint32_t i = blockIdx.y; i < count; i += gridDim.y) {
        const int32_t id = ids[i];
        if (id < 0 || (uint32_t)id >= n_src) {
            if (j == 0u && bad) *bad = 1;
            continue;
        }
        dst[(size_t)i * dst_stride + j] = src[(size_t)id * src_stride + j];
    }
}

// ---- ARGMAX (ggml's f32 ARGMAX): the first index of the largest value; NaN is never larger ---------
// Each thread scans its elements in increasing index order with a strict '>' (an equal later value
// never replaces); candidates then combine by value, ties to the smaller index, over the wave
// (bpermute) and the workgroup (LDS), so the assignment of elements to threads does not matter. A
// row 16-byte aligned with n % 4 == 0 is read as float4 (thread i: elements 4 (i + 1024 k) ..), in
// batches of kAmBatch loads in flight. A row without any value above -inf gives 0.
constexpr uint32_t kAmBatch = 8;
__device__ __forceinline__ void am_pick(float & v, uint32_t & i, float v2, uint32_t i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}
__global__ __launch_bounds__(1024) void k_argmax(const float * x, uint64_t x_stride, uint32_t n, int32_t * out) {
    __shared__ float s_v[16];
    __shared__ uint32_t s_i[16];
    const float * xr = x + (size_t)blockIdx.x * x_stride;
    float v = -__builtin_inff();
    uint32_t i = 0xFFFFFFFFu;
    if ((((uintptr_t)xr) & 15u) == 0u && (n & 3u) == 0u) {
        const uint32_t n4 = n / 4u;
        for (uint32_t q0 = 0; q0 < n4; q0 += 1024u * kAmBatch) {
            float4 e[kAmBatch];
#pragma unroll
            for (uint32_t k = 0; k < kAmBatch; ++k) {
                const uint32_t q = q0 + threadIdx.x + 1024u * k;
                e[k] = q < n4 ? *(const float4 *)(xr + 4u * q) : make_float4(-__builtin_inff(), -__builtin_inff(),
                                                                                -__builtin_inff(), -__builtin_inff());
            }
#pragma unroll
            for (uint32_t k = 0; k < kAmBatch; ++k) {
                const uint32_t j = 4u * (q0 + threadIdx.x + 1024u * k);
                if (e[k].x > v) { v = e[k].x; i = j; }
                if (e[k].y > v) { v = e[k].y; i = j + 1u; }
                if (e[k].z > v) { v = e[k].z; i = j + 2u; }
                if (e[k].w > v) { v = e[k].w; i = j + 3u; }
            }
        }
    } else {
        for (uint32_t j = threadIdx.x; j < n; j += blockDim.x) {
            const float e = xr[j];
            if (e > v) { v = e; i = j; }
        }
    }
    for (int d = 32; d >= 1; d >>= 1) {
        const int src = (int)(__lane_id() ^ (uint32_t)d);
        am_pick(v, i, shfl_f(v, src), (uint32_t)shfl_i((int)i, src));
    }
    const uint32_t wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (__lane_id() == 0u) { s_v[wave] = v; s_i[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t w = 1; w < nw; ++w) am_pick(v, i, s_v[w], s_i[w]);
        out[blockIdx.x] = i == 0xFFFFFFFFu ? 0 : (int32_t)i;
    }
}

// ARGMAX of long rows (the vocabulary) in two passes: workgroup (b, row) scans the slice
// [b span, min((b + 1) span, n)) as k_argmax scans a row and stores its (value, index) as one 8-byte
// word; then one wave per row picks among the slices. The pick -- the largest value, then the lowest
// index, only values above -inf -- does not depend on the order of the picks, so the result is
// k_argmax's. span is a multiple of 4.
__global__ __launch_bounds__(1024) void k_argmax_part(const float * x, uint64_t x_stride, uint32_t n, uint32_t span,
                                                      uint64_t * part) {
    __shared__ float s_v[16];
    __shared__ uint32_t s_i[16];
    const float * xr = x + (size_t)blockIdx.y * x_stride;
    const uint32_t lo = blockIdx.x * span, hi = min(n, lo + span);
    float v = -__builtin_inff();
    uint32_t i = 0xFFFFFFFFu;
    if ((((uintptr_t)xr) & 15u) == 0u && (n & 3u) == 0u) {
        const uint32_t q_hi = hi / 4u;
        for (uint32_t q0 = lo / 4u; q0 < q_hi; q0 += 1024u * kAmBatch) {
            float4 e[kAmBatch];
#pragma unroll
            for (uint32_t k = 0; k < kAmBatch; ++k) {
                const uint32_t q = q0 + threadIdx.x + 1024u * k;
                e[k] = q < q_hi ? *(const float4 *)(xr + 4u * q) : make_float4(-__builtin_inff(), -__builtin_inff(),
                                                                                 -__builtin_inff(), -__builtin_inff());
            }
#pragma unroll
            for (uint32_t k = 0; k < kAmBatch; ++k) {
                const uint32_t j = 4u * (q0 + threadIdx.x + 1024u * k);
                if (e[k].x > v) { v = e[k].x; i = j; }
                if (e[k].y > v) { v = e[k].y; i = j + 1u; }
                if (e[k].z > v) { v = e[k].z; i = j + 2u; }
                if (e[k].w > v) { v = e[k].w; i = j + 3u; }
            }
        }
    } else {
        for (uint32_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
            const float e = xr[j];
            if (e > v) { v = e; i = j; }
        }
    }
    for (int d = 32; d >= 1; d >>= 1) {
        const int src = (int)(__lane_id() ^ (uint32_t)d);
        am_pick(v, i, shfl_f(v, src), (uint32_t)shfl_i((int)i, src));
    }
    const uint32_t wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (__lane_id() == 0u) { s_v[wave] = v; s_i[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t w = 1; w < nw; ++w) am_pick(v, i, s_v[w], s_i[w]);
        part[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = ((uint64_t)i << 32) | __float_as_uint(v);
    }
}
__global__ __launch_bounds__(64) void k_argmax_pick(const uint64_t * part, uint32_t nb, int32_t * out) {
    const uint32_t lane = threadIdx.x;
    float v = -__builtin_inff();
    uint32_t i = 0xFFFFFFFFu;
    if (lane < nb) {
        const uint64_t w = part[(size_t)blockIdx.x * nb + lane];
        v = __uint_as_float((uint32_t)w);
        i = (uint32_t)(w >> 32);
    }
    for (int d = 32; d >= 1; d >>= 1) {
        const int src = (int)(lane ^ (uint32_t)d);
        am_pick(v, i, shfl_f(v, src), (uint32_t)shfl_i((int)i, src));
    }
    if (lane == 0u) out[blockIdx.x] = i == 0xFFFFFFFFu ? 0 : (int32_t)i;
}

}  // namespace tsr

// ---- launchers ------------------------------------------------------------------------------------
int tsr_launch_rms_norm(const float * x, uint64_t x_stride, uint32_t n, uint32_t rows, float eps, float inv_n,
                        const float * w, uint64_t w_stride, uint32_t w_period, float * y, uint64_t y_stride, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_rms_norm, dim3(rows), dim3(128), 0, s, x, x_stride, n, eps, inv_n, w, w_stride,
                       w_period ? w_period : 1u, y, y_stride);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_rope(const tsr::RopeArgs & a, uint32_t T, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_rope, dim3(T, (a.n_heads + tsr::kRopeHeads - 1u) / tsr::kRopeHeads), dim3(tsr::kRopeThreads),
                       0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_rope_table(const int32_t * pos, uint32_t half, float ts, float m, float * tab, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_rope_table, dim3(1), dim3(64), 0, s, pos, half, ts, m, tab);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mm_epilogue(float * y, uint64_t y_stride, uint32_t N, uint32_t T, uint32_t mode, float fs, float sc,
                           const tsr::ExpkTab & ex, hipStream_t s) {
    if (T > 65535u) return -2;
    hipLaunchKernelGGL(tsr::k_mm_epilogue, dim3((N + 255u) / 256u, T), dim3(256), 0, s, y, y_stride, N, mode, fs, sc, ex);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_rope_kv(const tsr::RopeKvArgs & a, uint32_t T, hipStream_t s) {
    const uint32_t nrow = (a.n_head + 2u * a.n_head_kv) * a.head_dim;
    if (nrow > tsr::kRkMaxRow || a.n_dims / 2u > 512u || a.head_dim % 32u != 0u) return -2;
    hipLaunchKernelGGL(tsr::k_rope_kv, dim3(T), dim3(tsr::kRkThreads), 4u * (size_t)nrow, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

static dim3 ew_grid(uint32_t n, uint32_t rows) { return dim3((n + 255u) / 256u, rows < 65535u ? rows : 65535u); }

int tsr_launch_swiglu(const float * g, uint64_t g_stride, const float * u, uint64_t u_stride, float * y, uint64_t y_stride,
                      uint32_t n, uint32_t rows, const tsr::ExpkTab & ex, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_swiglu, ew_grid(n, rows), dim3(256), 0, s, g, g_stride, u, u_stride, y, y_stride, n, rows, ex);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_add(const float * a, uint64_t a_stride, const float * b, uint64_t b_stride, uint32_t b_period, float * y,
                   uint64_t y_stride, uint32_t n, uint32_t rows, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_add, ew_grid(n, rows), dim3(256), 0, s, a, a_stride, b, b_stride, b_period, y, y_stride, n,
                       rows);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_get_rows(const float * src, uint64_t src_stride, uint32_t n, uint32_t n_src, const int32_t * ids,
                        uint32_t count, float * dst, uint64_t dst_stride, int32_t * bad, hipStream_t s) {
    hipLaunchKernelGGL(tsr::k_get_rows, ew_grid(n, count), dim3(256), 0, s, (const uint32_t *)src, src_stride, n, n_src,
                       ids, count, (uint32_t *)dst, dst_stride, bad);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_argmax(const float * x, uint64_t x_stride, uint32_t n, uint32_t rows, int32_t * out, uint64_t * part,
                      hipStream_t s) {
    // long rows, few of them: slices of ~4096 values over up to kAmParts workgroups a row (one
    // workgroup reading the 128256-value vocabulary alone spent ~8 us on its compute unit's loads)
    if (part != nullptr && rows <= tsr::kAmRows && n >= 32768u) {
        const uint32_t nb = min(tsr::kAmParts, (n + 4095u) / 4096u);
        const uint32_t span = ((n + nb - 1u) / nb + 3u) & ~3u;
        hipLaunchKernelGGL(tsr::k_argmax_part, dim3(nb, rows), dim3(1024), 0, s, x, x_stride, n, span, part);
        hipLaunchKernelGGL(tsr::k_argmax_pick, dim3(rows), dim3(64), 0, s, part, nb, out);
    } else {
        hipLaunchKernelGGL(tsr::k_argmax, dim3(rows), dim3(1024), 0, s, x, x_stride, n, out);
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
