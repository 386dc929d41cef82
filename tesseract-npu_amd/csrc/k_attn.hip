// k_attn.hip -- FLASH_ATTN_EXT over the q8_0 KV cache on gfx950, bit-exact to the reference's
// composite flash attention (tsr_ref_fa, sw/sim/tsr_ref_at.c:774-860; AT section 6.6) in its fixed
// configuration C = 4 channels, PCAP = 9344, T_MAX = 1 (one query row per tile).
//
// The host planner cuts every token's visible cells into chunks of NCG groups (16 cells each); the
// reference processes chunk after chunk: scores (ATTQK, MAXOUT), p = EXP((s - m) scale) with the
// chunk maximum m (ASMAX), per channel c (groups u = c mod 4) the block-float P.V over segments of
// 4 of its groups (ATTPV with LSUM), then CTREE over the 4 channel partials and the online merge
// (AMERGE), and finally O / l (ANORM). On the GPU the chunks of a token and the channels of a chunk
// are independent until the merge, so they run as parallel workgroups (split-K); only the f32 steps
// that the reference orders are kept in its order:
//   k_fa_qk     QACT of the query heads, scores of a 256-cell tile of one chunk for the query heads
//               of one KV head, and the tile's maxima (MAXT is an order-free total-order maximum)
//   k_fa_pv     one (chunk, channel, KV head, 64-value slice): EXP, block float per segment, the f32
//               segment sums in segment order, the segment row-sums (LSUM)
//   k_fa_merge  one (token, KV head, slice): CTREE of the channels, the online merge in chunk order,
//               ANORM
//
// Block float (AT 6.4; sw/sim/tsr_ref_at.c:380-488): in a segment every weight w = p dV is scaled
// to an integer W = RNE(w 2^(23 - E_S)) (|W| <= 2^24) and A = sum W q is exact. W is split into four
// balanced base-256 digits d_k in [-128, 127] (W = sum d_k 256^k), so A = sum_k 256^k (sum d_k q)
// runs on the int8 matrix core with exact int32 digit sums (|sum| <= 64 * 128 * 128).
//
// Subnormal operands. A score is a tree sum of terms (dK Dx) f32(isum) with fp16 dK and Dx: every
// term is 0 or a multiple of 2^-48 in magnitude, so is every sum, and a GENERAL mask is added with
// the full f32 rule: no score is subnormal. Maxima are scores or the floor; EXPK values,
// block-float values and the results of rule operations are never subnormal either. The f32 steps
// after the scores therefore use the rule without the input DAZ (sadd_n / smul_n).
#include "expk.hpp"
#include "glue.hpp"
#include "kernels.hpp"
#include "kvstore.hpp"
#include "qact.hpp"

#include <algorithm>

namespace tsr {

constexpr uint32_t kMFloor = 0xF1800000u;   // -2^100 (AT 6.3)
constexpr uint32_t kLFloor = 0x00800000u;   // 2^-126 (AT 5.7)


// MAXT (AT 5.4, sw/sim/tsr_ref_at.c:286-292): NaN wins as the canonical NaN; -0 < +0.
__device__ __forceinline__ uint32_t maxt_key(uint32_t u) { return (u >> 31) ? ~u : (u | 0x80000000u); }
__device__ __forceinline__ float maxt(float a, float b) {
    const uint32_t ua = fb(daz(a)), ub = fb(daz(b));
    if ((ua & 0x7FFFFFFFu) > 0x7F800000u || (ub & 0x7FFFFFFFu) > 0x7F800000u) return bf(kNaN);
    return maxt_key(ua) >= maxt_key(ub) ? bf(ua) : bf(ub);
}
// Order-preserving key of MAXT's total order (DAZ applied; NaN above everything; -0 < +0).
__device__ __forceinline__ uint32_t maxt_key_f(float v) {
    const uint32_t u = fb(daz(v));
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;
    return (u >> 31) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float maxt_unkey(uint32_t k) {
    if (k == 0xFFFFFFFFu) return bf(kNaN);
    return bf((k >> 31) ? (k & 0x7FFFFFFFu) : ~k);
}
// Wave-wide max / sum with DPP inside rows, a swizzle across the halves and two readlanes (every
// lane of the wave must be active).
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    v = umax_u(v, (uint32_t)dpp_i<kDppXor1>((int)v));
    v = umax_u(v, (uint32_t)dpp_i<kDppXor2>((int)v));
    v = umax_u(v, (uint32_t)dpp_i<kDppRowHalfMirror>((int)v));
    v = umax_u(v, (uint32_t)dpp_i<kDppRowMirror>((int)v));
    v = umax_u(v, (uint32_t)xor16_i((int)v));
    return umax_u((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
}
__device__ __forceinline__ int wave_max_i(int v) {   // via the order-preserving unsigned map
    return (int)(wave_max_u((uint32_t)v ^ 0x80000000u) ^ 0x80000000u);
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppRowHalfMirror>(v);
    v += dpp_i<kDppRowMirror>(v);
    v += xor16_i(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
}

// ---------------------------------------------------------------------------------------------
// P.V: block (item * 4 + channel c, KV head g, group hg of 4 query heads x value part vh of VS); one
// wave per segment of the channel (4 of its groups = 64 cells), looping if there are more segments
// than waves. Each segment's results go to LDS; the f32 segment chain then runs in segment order.
// A block covers D / VS values of its heads (VS > 1 when the grid would not fill the chip: the
// value-independent EXP and LSUM work is then repeated per part, the value work is split).
//
// Phase A (lane = head row hr = lane / 16, 4 consecutive cells of the segment: group kk = (lane /
// 4) % 4, cells 4 (lane % 4) .. + 3): EXP of the scores, the weights w = p dV of the value blocks,
// and, over the 16 lanes of a head row (DPP), the segment's block-float exponent E_S per 64-value
// slice, the non-finite flags per block and LSUM. The block-float integers W = RNE(w 2^(23 - E_S))
// (|W| <= 2^24) are split into four balanced base-256 digits d_k in [-128, 127]: the bytes of
// (W + 0x80808080) ^ 0x80808080 (the offset makes every byte d_k + 128, the xor subtracts 128).
// The digits go to LDS as [block][head][digit][group][16 cells].
// Phase B (matrix core): A[h][v] = sum_cells W[h][cell] q[cell][v] = sum_k 256^k sum_cells d_k q is
// v_mfma_i32_16x16x64_i8 with rows (head, digit), columns 16 values and K the 64 cells; lane l then
// holds the four digit sums of head l / 16 and value l % 16 and forms A exactly in f64.
// Every global load of the first batch is issued before the EXP work, so that a block waits for
// memory once.
// ---------------------------------------------------------------------------------------------
constexpr uint32_t kPvWaves = 8;                                  // NCG <= 128 -> <= 8 segments per channel
constexpr uint32_t kPvMaxSeg = 8;

// CTREE over 4 channel partials (never subnormal: results of the segment chains).
__device__ __forceinline__ float ctree4(float x0, float x1, float x2, float x3) { return sadd_n(sadd_n(x0, x1), sadd_n(x2, x3)); }
__device__ __forceinline__ int32_t row16_isum(int32_t v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppRowHalfMirror>(v);
    return v + dpp_i<kDppRowMirror>(v);
}
__device__ __forceinline__ uint32_t f_field(float f) { return (fb(f) >> 23) & 0xFFu; }   // biased exponent

// RNE_int(w 2^(23 - es)) of a zero or normal w with exponent(w) <= es (sw/sim/tsr_ref_at.c:386-410):
// the power-of-two scaling is exact while the scaled value is normal, v_rndne_f32 rounds half to even,
// and a scaled value below 2^-126 is below 1/2 and rounds to 0 either way. |result| <= 2^24.
__device__ __forceinline__ int32_t bf_int_n(float w, int32_t es) {
    return (int32_t)__builtin_rintf(__builtin_ldexpf(w, 23 - es));
}
// f = RNE24(A) (zero or normal) scaled by 2^k: below 2^-126 a signed zero, from 2^128 a signed Inf,
// A == 0 -> +0 (sw/sim/tsr_ref_at.c:412-436). The exponent field of f plus k is the result's.
__device__ __forceinline__ float bf_scale(float f, int32_t k) {
    const uint32_t u = fb(f), s = u & 0x80000000u;
    const int32_t ne = (int32_t)((u >> 23) & 0xFFu) + k;
    uint32_t out = u + ((uint32_t)k << 23);
    out = ne < 1 ? s : (ne > 254 ? (s | 0x7F800000u) : out);
    return bf((u & 0x7FFFFFFFu) == 0u ? 0u : out);
}

typedef int v4i_fa __attribute__((ext_vector_type(4)));

// A = d0 + 256 d1 + 65536 d2 + 2^24 d3 of four digit sums (|d_k| <= 2^20): every product and partial
// sum is exact in f64 (|A| < 2^45), and the one conversion to f32 is RNE24(A).
__device__ __forceinline__ float digits_rne24(const v4i_fa & acc) {
    const double A = ((double)acc[3] * 16777216.0 + (double)acc[2] * 65536.0) + ((double)acc[1] * 256.0 + (double)acc[0]);
    return (float)A;
}

// The P.V work of one block (chunk item, channel c, KV head g, head group hg, value part vh), shared by
// k_fa_pv (the item's scores in global memory) and the fused decode form of k_fa_qk (one tile's scores
// in LDS). Lane = (head row hr, group kk of the segment, cell quad); one wave per segment.
template <int D, int VS>
struct PvBlock {
    static constexpr uint32_t DV = D / VS;                        // values of the block (>= 64)
    static constexpr uint32_t NBV = DV / 32;                      // their value blocks
    static constexpr uint32_t BB = NBV < 4 ? NBV : 4;             // blocks per batch (2 or 4)
    static constexpr uint32_t NBT = NBV / BB;                     // batches
    static_assert(DV >= 64 && NBV % BB == 0, "value part");
    // the loads of one segment: scores, value scales and the value quants of a batch
    struct Loads {
        float4 sv;
        uint32_t mv[4][BB / 2];
        int4 bq[2 * BB];
    };
    const FaArgs & a;
    const float * S;                                              // the scores of head h, cell j at S[j - s_off]
    uint32_t g, c, vh, lane, hr, kk, quad, u0, u_first, nu, nseg, vb0, nbk, s_off;
    bool head_ok;
    const uint16_t * vmeta;
    const uint8_t * vq;

    __device__ __forceinline__ PvBlock(const FaArgs & a_, const FaItem & it, uint32_t c_, uint32_t g_, uint32_t hg,
                                       uint32_t vh_, const float * S_, uint32_t s_off_ = 0u)
        : a(a_), S(S_), g(g_), c(c_), vh(vh_), s_off(s_off_) {
        lane = __lane_id();
        hr = lane >> 4;
        kk = (lane >> 2) & 3u;
        quad = lane & 3u;
        head_ok = 4u * hg + hr < a.G;
        u0 = it.u0;
        u_first = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u);
        const uint32_t u_end = it.u0 + it.n;
        nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
        nseg = (nu + 3u) / 4u;
        vb0 = vh * NBV;                                           // first value block of the part (in the head)
        nbk = a.E / 32u;                                          // value blocks of a cell
        vmeta = (const uint16_t *)a.vc.base;
        vq = a.vc.base + a.vc.quant_off;
    }

    __device__ __forceinline__ void load_scores(uint32_t seg, Loads & L) const {
        const uint32_t u = u_first + 4u * min(4u * seg + kk, nu - 1u);
        L.sv = *(const float4 *)(S + 16u * (u - u0) + 4u * quad - s_off);
    }

    __device__ __forceinline__ void loads(uint32_t seg, uint32_t vb, Loads & L, bool scores) const {
        const uint32_t gi = 4u * seg + kk;
        const uint32_t u = u_first + 4u * min(gi, nu - 1u);        // clamped: loads stay in the item
        if (scores) load_scores(seg, L);
        const uint16_t * vm = vmeta + ((size_t)u * 16u + 4u * quad) * nbk + (size_t)g * (D / 32u) + vb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (BB == 4) {
                const uint2 m2 = *(const uint2 *)(vm + (size_t)i * nbk);
                L.mv[i][0] = m2.x; L.mv[i][1] = m2.y;
            } else {
                L.mv[i][0] = *(const uint32_t *)(vm + (size_t)i * nbk);
            }
        }
        const uint32_t uB = u_first + 4u * min(4u * seg + (lane >> 4), nu - 1u);
        const uint8_t * vqB = vq + ((size_t)uB * a.E + (size_t)g * D + 32u * vb + (lane & 15u)) * 16u;
#pragma unroll
        for (uint32_t t8 = 0; t8 < 2 * BB; ++t8) L.bq[t8] = *(const int4 *)(vqB + 256u * t8);
    }

    // One segment (L holds its loads): EXP, LSUM, the block-float weights, their digits and the
    // matrix-core digit sums; the segment's results go to s_c [slot][4 heads][DV] and s_l [slot][4 heads].
    __device__ __forceinline__ void segment(uint32_t seg, uint32_t slot, Loads & L, float m, const uint32_t * s_t64,
                                            float * s_c, float * s_l, uint8_t * dg) const {
        // ---- phase A: lane = (head row, 4 cells) ----------------------------------------------
        const bool cv = 4u * seg + kk < nu;
        const float ss[4] = { L.sv.x, L.sv.y, L.sv.z, L.sv.w };
        float pz[4];
        uint32_t pnf = 0u, pe = 0u;                                // non-finite flag; largest exponent field
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // EXPK results are zero, normal, Inf or NaN (never subnormal)
            pz[i] = (cv && head_ok) ? expk(smul_n(ssub_n(ss[i], m), a.scale), a.ex, s_t64) : 0.0f;
            const uint32_t f = f_field(pz[i]);
            pnf |= f == 255u ? 1u : 0u;
            pe = max(pe, f == 255u ? 0u : f);
        }
        // LSUM of the segment (AT 6.5): block float of its p values
        if (vh == 0u) {
            const bool badl = row16_or(pnf) != 0u;
            pe = row16_umax(pe);
            int32_t lsum = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) lsum += f_field(pz[i]) == 255u ? 0 : bf_int_n(pz[i], (int32_t)pe - 127);
            lsum = row16_isum(lsum);
            if ((lane & 15u) == 0u)
                s_l[slot * 4u + hr] = badl ? bf(kNaN) : (pe == 0u ? 0.0f : bf_scale((float)lsum, (int32_t)pe - 150));
        }

#pragma unroll
        for (uint32_t bt = 0; bt < NBT; ++bt) {                    // BB value blocks (32 BB values) at a time
            const uint32_t vb = vb0 + bt * BB;
            if (bt > 0u) loads(seg, vb, L, false);
            // weights of the 4 cells for the BB blocks: w = p dV, a subnormal product flushed to zero
            float w[4][BB];
            uint32_t ex[BB / 2], nfm = 0u;
#pragma unroll
            for (uint32_t sa = 0; sa < BB / 2; ++sa) ex[sa] = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool live = (fb(pz[i]) & 0x7FFFFFFFu) != 0u;
#pragma unroll
                for (uint32_t e = 0; e < BB; ++e) {
                    const uint32_t dv = (L.mv[i][e >> 1] >> (16u * (e & 1u))) & 0xFFFFu;
                    const float we = live ? pz[i] * h2f_fast(dv) : 0.0f;
                    const uint32_t f = f_field(we);
                    nfm |= (f == 255u ? 1u : 0u) << e;
                    w[i][e] = f == 0u ? 0.0f : we;
                    ex[e >> 1] = max(ex[e >> 1], f == 255u ? 0u : f);
                }
            }
            int32_t es[BB / 2];
            bool any[BB / 2];
#pragma unroll
            for (uint32_t sa = 0; sa < BB / 2; ++sa) {
                const uint32_t ef = row16_umax(ex[sa]);
                any[sa] = ef != 0u;
                es[sa] = (int32_t)ef - 127;
            }
            const uint32_t badm = row16_or(nfm);
            // digits: for block e and digit k, the 4 cells' digit bytes in one word
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) {
                const bool use = any[e >> 1] && ((badm >> e) & 1u) == 0u;
                uint32_t P[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int32_t W = use ? bf_int_n(w[i][e], es[e >> 1]) : 0;
                    P[i] = ((uint32_t)W + 0x80808080u) ^ 0x80808080u;     // byte k = digit k of W
                }
                // transpose the 4 x 4 bytes: word k = digit k of cells 0..3
                const uint32_t lo01 = __builtin_amdgcn_perm(P[1], P[0], 0x05010400u);   // d0c0 d0c1 d1c0 d1c1
                const uint32_t lo23 = __builtin_amdgcn_perm(P[3], P[2], 0x05010400u);
                const uint32_t hi01 = __builtin_amdgcn_perm(P[1], P[0], 0x07030602u);   // d2c0 d2c1 d3c0 d3c1
                const uint32_t hi23 = __builtin_amdgcn_perm(P[3], P[2], 0x07030602u);
                const uint32_t q[4] = { __builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                        __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u) };
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    *(uint32_t *)(dg + (((e * 4u + hr) * 4u + (uint32_t)k) * 4u + kk) * 16u + 4u * quad) = q[k];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // ---- phase B: 2 BB tiles of 16 values; lane = (head row l / 16 of the result, value l % 16)
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) {
                // A operand: row l % 16 = (head, digit), K = the 16 cells of group l / 16
                const v4i_fa Aop = *(const v4i_fa *)(dg + ((e * 16u + (lane & 15u)) * 4u + (lane >> 4)) * 16u);
                const bool bad = ((badm >> e) & 1u) != 0u;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int4 bq = L.bq[2 * e + half];
                    const v4i_fa Bop = { bq.x, bq.y, bq.z, bq.w };
                    v4i_fa acc = { 0, 0, 0, 0 };
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(Aop, Bop, acc, 0, 0, 0);
                    const float cval = bad ? bf(kNaN) : (any[e >> 1] ? bf_scale(digits_rne24(acc), es[e >> 1] - 23) : 0.0f);
                    s_c[(slot * 4u + hr) * DV + 32u * (bt * BB + e) + 16u * (uint32_t)half + (lane & 15u)] = cval;
                }
            }
        }
    }

    // After a block barrier: the segment chains in order (AT 6.4 O, 6.5 l) -> the channel partials.
    // Thread = (head row, value of the part).
    __device__ __forceinline__ void chains(uint32_t item, uint32_t hg, const float * s_c, const float * s_l) const {
        const uint32_t G = a.G, nh = a.n_head;
        for (uint32_t idx = threadIdx.x; idx < 4u * DV; idx += blockDim.x) {
            const uint32_t r4 = idx / DV, v = idx % DV, hi2 = 4u * hg + r4;
            if (hi2 >= G) continue;
            const uint32_t h2 = g * G + hi2;
            float O = 0.0f;
            for (uint32_t seg = 0; seg < nseg; ++seg) O = sadd_n(O, s_c[(seg * 4u + r4) * DV + v]);
            const size_t slot = ((size_t)item * 4u + c) * nh + h2;
            a.OP[slot * D + vh * DV + v] = O;
            if (vh == 0u && v == 0u) {
                float l = 0.0f;
                for (uint32_t seg = 0; seg < nseg; ++seg) l = sadd_n(l, s_l[seg * 4u + r4]);
                a.LP[slot] = l;
            }
        }
    }
};

// ---------------------------------------------------------------------------------------------
// scores: block (tile, KV head g), thread = one cell of the tile. The block quantizes the query
// values of the KV head's G heads (QACT A32: its 32-blocks never cross a head, so they are the
// blocks of the whole query row) while the K rows of its cells load.
// ---------------------------------------------------------------------------------------------
// The work list is inline in the kernel arguments (INL, decode) or in device memory: a compile-time
// choice, so that reading an item is never a branch around a load.
template <bool INL>
__device__ __forceinline__ FaItem fa_item(const FaArgs & a, const FaPlan & p, uint32_t i) {
    if constexpr (INL) return p.items[i];
    else return a.items[i];
}

// LDS of the score kernel: the query quants and scales, the per-wave maxima and (ROPE) the new k row.
__host__ __device__ inline uint32_t fa_qk_lds(uint32_t G, uint32_t D, bool rope) {
    const uint32_t b = G * D + 4u * G * (D / 32u) + 16u * G;
    return rope ? ((b + 15u) & ~15u) + D + D / 8u : b;
}
// The fused decode tail's LDS after it (16-aligned): EXPK table, the tile's scores [4 heads][256],
// segment results [4 waves][4 heads][D], row sums [4 waves][4 heads], digits [4 waves][BB][1024], two
// flags and 4 chunk maxima.
__host__ __device__ inline uint32_t fa_fuse_lds(uint32_t D) {
    const uint32_t bb = D / 32u < 4u ? D / 32u : 4u;
    return 256u + 4u * 4u * 256u + 4u * 4u * 4u * D + 4u * 16u + 4u * bb * 1024u + 32u;
}

// Data that blocks on other XCDs read after a counter moves only through accesses coherent at agent
// scope (relaxed atomics: sc1 stores write through to the coherence point, sc1 loads bypass stale
// L1 / L2 lines), so the counters need no L2-wide write-back or invalidation: a wave waits for its
// coherent stores to complete (vm_wait) before the block's barrier and the counter increment, and a
// reader issues its loads after it has seen the counter (program order behind the barrier).
__device__ __forceinline__ void st_co(float * p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_co4(float * p, float4 v) {     // 8-byte aligned p: two 8-byte stores
    uint64_t * q = (uint64_t *)p;
    __hip_atomic_store(q, ((uint64_t)fb(v.y) << 32) | fb(v.x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, ((uint64_t)fb(v.w) << 32) | fb(v.z), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_co(const float * p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 ld_co4(const float * p) {
    uint64_t * q = (uint64_t *)const_cast<float *>(p);
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(bf((uint32_t)lo), bf((uint32_t)(lo >> 32)), bf((uint32_t)hi), bf((uint32_t)(hi >> 32)));
}
__device__ __forceinline__ uint32_t ld_co_u(const uint32_t * p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co_u(uint32_t * p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void vm_wait() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);                           // vmcnt(0); expcnt and lgkmcnt untouched
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Counter increment by thread 0 after every wave's vm_wait and a barrier; the previous value.
__device__ __forceinline__ uint32_t count_up(uint32_t * ctr) {
    return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The fused decode form (T == 1, G <= 4, D <= 128, a plan's work list): after its scores and tile
// maxima, the block (item, tile tt, KV head g) goes on with P.V. Segment s of a channel is the 4 of
// its groups in tile s of the item (tiles are 16 groups), so the block's 4 waves take the segments
// in its tile of channels 0..3.
//   1. The block has published its maxima as MAXT keys (never 0: a NaN keys to ~0, every other value
//      to at least 0x007FFFFF) in slots that are 0 until then; its first wave reads the item's slots
//      until none is 0 (blocks of one item are consecutive in dispatch order, so they all run: the
//      wait is bounded all the same, and an expired wait raises *bad = 2). What it read gives the
//      chunk maxima.
//   2. Each wave: the chunk maximum of its heads, the segment (PvBlock, scores from LDS), its results
//      to seg_o / seg_l.
//   3. The last tile block of the item (a counter, no wait) chains the segments of each channel in
//      order into the item's channel partials (as k_fa_pv) and records the chunk maxima; the last
//      item of the KV head (a counter) merges the items in order and normalizes (as k_fa_merge), then
//      clears the counters for the next launch.
constexpr uint32_t kFuseSegMax = 8;                              // segments per channel (NCG <= 128)
constexpr uint32_t kFuseItems = 4;                               // items loaded per round of the merge

template <int D>
__device__ __forceinline__ void fa_fused_tail(const FaArgs & a, const FaPlan & p, const FaItem & it, uint32_t item,
                                              uint32_t tt, uint32_t g, uint8_t * ft, const PvBlock<D, 1> & pb,
                                              typename PvBlock<D, 1>::Loads & L) {
    using PB = PvBlock<D, 1>;
    constexpr uint32_t BB = PB::BB, D4 = D / 4u;
    const uint32_t G = a.G, nh = a.n_head, nkv = a.n_head_kv, ni = p.n_items;
    const uint32_t * s_t64 = (const uint32_t *)ft;
    const float * s_S = (const float *)(ft + 256);
    float * s_c = (float *)(ft + 256 + 4096);                     // [wave][4 heads][D]
    float * s_l = s_c + 16u * D;                                  // [wave][4 heads]
    uint8_t * s_dg = (uint8_t *)(s_l + 16);                       // [wave][BB][1024]
    uint32_t * s_flag = (uint32_t *)(s_dg + 4u * BB * 1024u);
    uint32_t * segdone = a.sync + (size_t)item * nkv + g;
    uint32_t * done = a.sync + (size_t)ni * nkv + g;
    uint32_t * s_mk = s_flag + 2;                                 // chunk maxima (keys) of the G heads
    const uint32_t lane = __lane_id(), c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave = channel
    const uint32_t hrow = min(lane >> 4, G - 1u), h = g * G + hrow;
    const bool has = tt < pb.nseg;                                // wave-uniform (the V rows are loading)
    (void)s_S;

    // 1. wait for the item's tile maxima; the chunk maxima: MAXOUT of the floor and the tile maxima
    const uint32_t floor_key = maxt_key_f(bf(kMFloor));
    if (c == 0u) {                                                // wave 0, every lane
        const uint32_t nk = it.ntiles * G;                        // lane l < nk: tile l / G, head l % G
        const uint32_t * kp = a.tkeys + ((size_t)g * p.n_items * p.maxtiles + it.tile0) * 4u + (lane / G) * 4u + lane % G;
        uint32_t v = 1u, spins = 0;
        for (;;) {
            v = lane < nk ? ld_co_u(kp) : 1u;
            if (__all(v != 0u)) break;
            if (++spins >= a.spin_max) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t k = wave_max_u(lane < nk && lane % G == i ? v : floor_key);
            if (lane == 0u && i < G) s_mk[i] = k;
        }
    }
    __syncthreads();
    const float m = maxt_unkey(s_mk[hrow]);

    // 2. the segment and its results
    const size_t tile = (size_t)it.tile0 + tt;
    if (has) {
        pb.load_scores(tt, L);
        pb.segment(tt, c, L, m, s_t64, s_c, s_l, s_dg + (size_t)c * (BB * 1024u));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (uint32_t idx = lane; idx < G * D4; idx += 64u) {
            const uint32_t r = idx / D4, v4 = idx % D4;
            st_co4(a.seg_o + ((tile * 4u + c) * nh + g * G + r) * D + 4u * v4, *(const float4 *)(s_c + (c * 4u + r) * D + 4u * v4));
        }
        if (lane < G) st_co(a.seg_l + (tile * 4u + c) * nh + g * G + lane, s_l[c * 4u + lane]);
    }
    vm_wait();
    __syncthreads();
    if (threadIdx.x == 0u) s_flag[0] = count_up(segdone) == it.ntiles - 1u;
    __syncthreads();
    if (s_flag[0] == 0u) return;                                  // block-uniform

    // 3a. the item's last tile: each channel's segment chain in segment order (AT 6.4 O, 6.5 l), all
    // of its loads first; and the chunk maxima of the KV head's heads
    if (c == 0u && (lane & 15u) == 0u && (lane >> 4) < G) st_co(a.m_item + (size_t)item * nh + h, m);
    constexpr uint32_t kPer = 2;                                  // 4 G D / 4 <= 512 entries: 2 per thread
    const uint32_t ne = 4u * G * D4;
    float4 x[kPer][kFuseSegMax];
    float xl[kPer][kFuseSegMax];
    uint32_t nsg[kPer], ent[kPer];
#pragma unroll
    for (uint32_t e = 0; e < kPer; ++e) {                         // every load first
        ent[e] = threadIdx.x + 256u * e;
        const uint32_t idx = min(ent[e], ne - 1u);
        const uint32_t cc = idx / (G * D4), r = (idx / D4) % G, v4 = idx % D4, hh = g * G + r;
        const uint32_t u_first = it.u0 + ((cc + 4u - (it.u0 & 3u)) & 3u), u_end = it.u0 + it.n;
        const uint32_t nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
        nsg[e] = (nu + 3u) / 4u;
#pragma unroll
        for (uint32_t sg = 0; sg < kFuseSegMax; ++sg) {
            const size_t row = ((size_t)(it.tile0 + min(sg, max(nsg[e], 1u) - 1u)) * 4u + cc) * nh + hh;
            x[e][sg] = ld_co4(a.seg_o + row * D + 4u * v4);
            xl[e][sg] = ld_co(a.seg_l + row);
        }
    }
#pragma unroll
    for (uint32_t e = 0; e < kPer; ++e) {
        if (ent[e] >= ne) continue;
        const uint32_t idx = ent[e];
        const uint32_t cc = idx / (G * D4), r = (idx / D4) % G, v4 = idx % D4, hh = g * G + r;
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float l = 0.0f;
#pragma unroll
        for (uint32_t sg = 0; sg < kFuseSegMax; ++sg) {
            if (sg < nsg[e]) {
                O.x = sadd_n(O.x, x[e][sg].x);
                O.y = sadd_n(O.y, x[e][sg].y);
                O.z = sadd_n(O.z, x[e][sg].z);
                O.w = sadd_n(O.w, x[e][sg].w);
                l = sadd_n(l, xl[e][sg]);
            }
        }
        const size_t slot = ((size_t)item * 4u + cc) * nh + hh;
        st_co4(a.OP + slot * D + 4u * v4, O);
        if (v4 == 0u) st_co(a.LP + slot, l);
    }
    vm_wait();
    __syncthreads();
    if (threadIdx.x == 0u) s_flag[1] = count_up(done) == ni - 1u;
    __syncthreads();
    if (s_flag[1] == 0u) return;

    // 3b. the KV head's last item: CTREE of the channels, the online merge in item (chunk) order and
    // ANORM (AT 5.6, 5.7), as k_fa_merge; the items' loads a round of kFuseItems at a time
    for (uint32_t idx = threadIdx.x; idx < G * D4; idx += blockDim.x) {
        const uint32_t r = idx / D4, v4 = idx % D4, hh = g * G + r;
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float l = 0.0f, mr = 0.0f;
        for (uint32_t k0 = 0; k0 < ni; k0 += kFuseItems) {
            float4 op[kFuseItems][4];
            float lp[kFuseItems][4], mk[kFuseItems];
#pragma unroll
            for (uint32_t k = 0; k < kFuseItems; ++k) {
                const uint32_t kk = min(k0 + k, ni - 1u);
                mk[k] = ld_co(a.m_item + (size_t)kk * nh + hh);
#pragma unroll
                for (uint32_t cc = 0; cc < 4u; ++cc) {
                    const size_t slot = ((size_t)kk * 4u + cc) * nh + hh;
                    op[k][cc] = ld_co4(a.OP + slot * D + 4u * v4);
                    lp[k][cc] = ld_co(a.LP + slot);
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < kFuseItems; ++k) {
                if (k0 + k >= ni) break;
                const float4 ok = make_float4(ctree4(op[k][0].x, op[k][1].x, op[k][2].x, op[k][3].x),
                                              ctree4(op[k][0].y, op[k][1].y, op[k][2].y, op[k][3].y),
                                              ctree4(op[k][0].z, op[k][1].z, op[k][2].z, op[k][3].z),
                                              ctree4(op[k][0].w, op[k][1].w, op[k][2].w, op[k][3].w));
                const float lk = ctree4(lp[k][0], lp[k][1], lp[k][2], lp[k][3]);
                if (k0 + k == 0u) {
                    O = ok;
                    l = lk;
                    mr = mk[k];
                } else {
                    const float mrun = maxt(mr, mk[k]);
                    const float fa = expk(smul_n(ssub_n(mr, mrun), a.scale), a.ex, s_t64);
                    const float fbv = expk(smul_n(ssub_n(mk[k], mrun), a.scale), a.ex, s_t64);
                    l = sadd_n(smul_n(l, fa), smul_n(lk, fbv));
                    O.x = sadd_n(smul_n(O.x, fa), smul_n(ok.x, fbv));
                    O.y = sadd_n(smul_n(O.y, fa), smul_n(ok.y, fbv));
                    O.z = sadd_n(smul_n(O.z, fa), smul_n(ok.z, fbv));
                    O.w = sadd_n(smul_n(O.w, fa), smul_n(ok.w, fbv));
                    mr = mrun;
                }
            }
        }
        const float rl = srcp(maxt(l, bf(kLFloor)));
        *(float4 *)(a.out + (size_t)hh * D + 4u * v4) = make_float4(smul_n(O.x, rl), smul_n(O.y, rl), smul_n(O.z, rl), smul_n(O.w, rl));
    }
    // every block of the KV head is past its waits: clear its counters for the next launch
    for (uint32_t k = threadIdx.x; k < ni; k += blockDim.x) a.sync[(size_t)k * nkv + g] = 0u;
    for (uint32_t t = threadIdx.x; t < 4u * ni * p.maxtiles; t += blockDim.x)
        a.tkeys[(size_t)g * 4u * ni * p.maxtiles + t] = 0u;
    if (threadIdx.x == 0u) *done = 0u;
}

// ROPE (T == 1, D <= 128, (G + 2) D <= 1024): the block also rotates the query heads (rope4, angles
// per lane by rope_cs_lane) before their QACT, rotates and QACTs the token's k row of head g and
// QACTs its v row (threads after the query slots, A32 as SET_ROWS_KV); the thread of the new cell
// scores with that fresh k row, and the first block of each KV head stores the k and v rows in the
// caches -- ROPE, SET_ROWS_KV and the scores in one launch.
// FUSE: the decode form that goes on with P.V and the merge (fa_fused_tail).
template <int D, bool INL, bool ROPE, bool FUSE = false>
__global__ __launch_bounds__(256) void k_fa_qk(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t NBD = D / 32u;                             // blocks per head
    constexpr bool KREG = D <= 128;                                // K row of the cell kept in registers
    static_assert(!ROPE || KREG, "the fused ROPE keeps the K rows in registers");
    static_assert(!FUSE || (KREG && !INL), "the fused decode form: D <= 128, a plan's work list");
    const uint32_t tt = blockIdx.x % p.maxtiles;
    const FaItem it = fa_item<INL>(a, p, blockIdx.x / p.maxtiles);
    if (tt >= it.ntiles) return;                                  // the item has fewer tiles (block-uniform)
    const uint32_t g = blockIdx.y, G = a.G;
    int8_t * s_q = (int8_t *)lds;                                 // G*D quants of the KV head's query heads
    float * s_dx = (float *)(lds + G * D);                        // G*D/32 scales
    uint32_t * s_red = (uint32_t *)(s_dx + G * NBD);              // 4 waves x G maxima (keys)
    int8_t * s_kq = (int8_t *)lds + ((G * D + 4u * G * NBD + 16u * G + 15u) & ~15u);   // ROPE: the new k row of
    float * s_kd = (float *)(s_kq + D);                           //       head g (D quants) and its D/32 scales
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6);
    int32_t pos = 0;
    int64_t cell64 = -1;
    if constexpr (ROPE) {                                         // scalar loads: not behind the vector loads
        if (a.rtab == nullptr) pos = *a.pos;
        cell64 = *a.cell;
    }
    uint8_t * ft = lds + ((fa_qk_lds(G, D, ROPE) + 15u) & ~15u);  // FUSE: the tail's LDS
    const uint32_t t64v = FUSE ? a.ex.t64[threadIdx.x & 63u] : 0u;

    const uint32_t n16 = 16u * it.n, j = 256u * tt + threadIdx.x;
    const bool in = j < n16;
    const uint32_t cell = 16u * it.u0 + j;
    const uint32_t ng = (a.kc.kv_size + 15u) / 16u;
    const uint32_t u = min(cell >> 4, ng - 1u), rr = cell & 15u;  // clamped: loads stay inside the plane
    const bool vis = in && (it.general || (j >= it.c_lo && j < it.c_hi));
    const uint32_t E = a.E, nbk = E / 32u;
    const uint16_t * kmeta = (const uint16_t *)a.kc.base + ((size_t)u * 16u + rr) * nbk + (size_t)g * NBD;
    const uint8_t * kq = a.kc.base + a.kc.quant_off + (size_t)u * 16u * E + (size_t)rr * 16u;
    const uint32_t ci0 = g * D / 16u;                             // first 16-byte chunk of the head

    // the query values of round 0 first (vector-memory counters retire in order: the QACT then waits
    // for them only, not for the K rows)
    const float * qrow = a.q + (size_t)it.t * a.q_stride + (size_t)g * G * D;
    const uint32_t nslot = G * D / 4u;                             // 8 lanes per 32-block
    const uint32_t half = a.n_dims / 2u;
    // ROPE: threads nslot .. nslot + D/4 - 1 hold the k row of head g, the next D/4 its v row
    const uint32_t kslot = threadIdx.x - nslot, vslot = kslot - D / 4u;
    const bool is_k = ROPE && threadIdx.x >= nslot && kslot < D / 4u, is_v = ROPE && !is_k && threadIdx.x >= nslot &&
                                                                             vslot < D / 4u;
    const float * src = a.q + (size_t)a.n_head * D + (size_t)g * D + (is_v ? E + 4u * vslot : 4u * (is_k ? kslot : 0u));
    const uint32_t jq = 4u * min(threadIdx.x, nslot - 1u);        // first query value of the thread
    const float4 qv0 = (ROPE && threadIdx.x >= nslot) ? *(const float4 *)src : *(const float4 *)(qrow + jq);
    float4 qpart = qv0;                                           // ROPE NEOX: the values half away
    // value index in the head of a rotated thread (q or k); D for the others (nothing to rotate)
    const uint32_t jh0 = threadIdx.x < nslot ? jq % D : (is_k ? 4u * kslot : D);
    if constexpr (ROPE) {
        if (a.neox && jh0 < a.n_dims) {                           // the partner lies in the same head row
            const int32_t dj = jh0 < half ? (int32_t)half : -(int32_t)half;
            qpart = *(const float4 *)((threadIdx.x < nslot ? qrow + jq : src) + dj);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    int4 kr[KREG ? 2 * NBD : 1];
    uint32_t km[NBD];
#pragma unroll
    for (uint32_t kb = 0; kb < NBD; ++kb) km[kb] = kmeta[kb];
    if constexpr (KREG) {
#pragma unroll
        for (uint32_t c = 0; c < 2 * NBD; ++c) kr[c] = *(const int4 *)(kq + (size_t)(ci0 + c) * 256u);
    }
    // FUSE: the P.V segments of the block (wave = channel); their V rows load after the QACT below
    const PvBlock<D, 1> pb(a, it, (uint32_t)__builtin_amdgcn_readfirstlane(wave), g, 0u, 0u,
                           (const float *)(ft + 256) + (size_t)min((uint32_t)lane >> 4, G - 1u) * 256u, 256u * tt);
    typename PvBlock<D, 1>::Loads pl;
    __builtin_amdgcn_sched_barrier(0);
    bool holds = false;                                           // FUSE + ROPE: the tile holds the new cell's group

    auto qact_slot = [&](uint32_t slot, const float4 v) {
        float Dq;
        const uint32_t qq = qact_a32_lane(v, &Dq);
        if (slot < nslot) {
            *(uint32_t *)(s_q + 4u * slot) = qq;
            if ((lane & 7) == 0) s_dx[slot >> 3] = Dq;
        }
    };
    if constexpr (ROPE) {
        float c_l, s_l;
        if (a.rtab != nullptr) {                                  // the token's table (block-uniform)
            const float2 cs = *(const float2 *)(a.rtab + 2u * min((uint32_t)lane, half - 1u));
            c_l = cs.x;
            s_l = cs.y;
        } else {
            rope_cs_lane(pos, half, a.ts, a.m, (uint32_t)lane, &c_l, &s_l);
        }
        // every lane runs rope4 (its table reads are cross-lane: a lane that skipped it would hide its
        // entries from the others); v lanes then keep their values (jh0 = D leaves them unrotated anyway)
        const float4 rot = rope4(qv0, qpart, jh0, a.n_dims, a.neox != 0u, c_l, s_l);
        const float4 r = is_v ? qv0 : rot;
        float Dq;
        const uint32_t qq = qact_a32_lane(r, &Dq);                // every lane (8-lane groups)
        if (threadIdx.x < nslot) {
            *(uint32_t *)(s_q + 4u * threadIdx.x) = qq;
            if ((lane & 7) == 0) s_dx[threadIdx.x >> 3] = Dq;
        } else if (is_k) {
            *(uint32_t *)(s_kq + 4u * kslot) = qq;
            if ((lane & 7) == 0) s_kd[kslot >> 3] = Dq;
        }
        const bool cell_ok = cell64 >= 0 && cell64 < (int64_t)a.kc.kv_size && cell64 < (int64_t)a.vc.kv_size;
        // FUSE: a tile holding the new cell's group reads its v row, so its block stores it too
        const uint32_t ug = (uint32_t)((uint64_t)cell64 >> 4), ut = it.u0 + 16u * tt;
        holds = FUSE && cell_ok && ug >= ut && ug < min(ut + 16u, it.u0 + it.n);
        if (blockIdx.x == 0u || holds) {                          // the caches' copy of the new rows
            if (cell_ok && (is_k || is_v))
                kv_store_unit(is_k ? a.kc : a.vc, is_k ? 0u : 1u, (uint32_t)cell64, g * D + 4u * (is_k ? kslot : vslot), qq,
                              Dq, (lane & 7) == 0);
            if (!cell_ok && blockIdx.x == 0u && threadIdx.x == 0u && g == 0u && a.bad != nullptr) *a.bad = 1;
        }
    } else {
        qact_slot(threadIdx.x, qv0);
        for (uint32_t s0 = blockDim.x; s0 < nslot; s0 += blockDim.x)   // G D > 1024 only
            qact_slot(s0 + threadIdx.x, *(const float4 *)(qrow + 4u * min(s0 + threadIdx.x, nslot - 1u)));
    }
    if constexpr (FUSE) {
        if (threadIdx.x < 64u) ((uint32_t *)ft)[threadIdx.x] = t64v;
    }
    lds_barrier();                                                // the K rows stay in flight
    if constexpr (FUSE) {                                         // the V rows (the new v row is stored now)
        if (tt < pb.nseg) pb.loads(tt, pb.vb0, pl, false);
    }
    if constexpr (ROPE) {                                         // the new cell scores with the fresh k row
        if ((int64_t)cell == cell64 && in) {
#pragma unroll
            for (uint32_t c = 0; c < 2 * NBD; ++c) kr[c] = *(const int4 *)(s_kq + 16u * c);
#pragma unroll
            for (uint32_t kb = 0; kb < NBD; ++kb) km[kb] = f2h_exact(s_kd[kb]);
        }
    }

    float * S = a.S + (size_t)it.s_off * a.n_head;
    for (uint32_t i = 0; i < G; ++i) {
        const uint32_t h = g * G + i;
        float s = bf(kNegInf);
        if (vis) {
            float p[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) p[k] = 0.0f;
#pragma unroll
            for (uint32_t kb = 0; kb < NBD; ++kb) {
                int4 w0, w1;
                if constexpr (KREG) { w0 = kr[2 * kb]; w1 = kr[2 * kb + 1]; }
                else {
                    w0 = *(const int4 *)(kq + (size_t)(ci0 + 2 * kb) * 256u);
                    w1 = *(const int4 *)(kq + (size_t)(ci0 + 2 * kb + 1) * 256u);
                }
                const int4 * xq = (const int4 *)(s_q + (size_t)i * D + 32u * kb);
                const int4 x0 = xq[0], x1 = xq[1];
                int is = dot4(w0.x, x0.x, 0);
                is = dot4(w0.y, x0.y, is);
                is = dot4(w0.z, x0.z, is);
                is = dot4(w0.w, x0.w, is);
                is = dot4(w1.x, x1.x, is);
                is = dot4(w1.y, x1.y, is);
                is = dot4(w1.z, x1.z, is);
                is = dot4(w1.w, x1.w, is);
                // SEG (AT 6.2): p_k = +0 + (dK Dx) f32(isum); |terms| >= 2^-48 or 0 (fp16 scales), so
                // the plain operations never meet a subnormal; NaN is canonicalized below
                const float t = (h2f_fast(km[kb]) * s_dx[i * NBD + kb]) * (float)is;
                p[kb] = 0.0f + t;
            }
#pragma unroll
            for (int w = 16; w > 1; w >>= 1)
#pragma unroll
                for (int k = 0; k < w / 2; ++k) p[k] = p[2 * k] + p[2 * k + 1];
            s = canon(p[0]);
            if (it.general) {
                const float m = a.mask[(size_t)it.t * a.mstride + cell];
                s = fb(m) == kNegInf ? bf(kNegInf) : sadd(s, m);
            }
        }
        if (in) {
            if constexpr (FUSE) ((float *)(ft + 256))[i * 256u + threadIdx.x] = s;
            else S[(size_t)h * n16 + j] = s;
        }
        const uint32_t mk = wave_max_u(in ? maxt_key_f(s) : maxt_key_f(bf(kMFloor)));
        if (lane == 0) s_red[wave * G + i] = mk;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < G; i += blockDim.x) {
        uint32_t m = s_red[i];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = umax_u(m, s_red[w * G + i]);
        if constexpr (FUSE) st_co_u(a.tkeys + ((size_t)g * p.n_items * p.maxtiles + it.tile0 + tt) * 4u + i, m);
        else a.Mpart[(size_t)(it.tile0 + tt) * a.n_head + g * G + i] = maxt_unkey(m);
    }
    if constexpr (FUSE) fa_fused_tail<D>(a, p, it, blockIdx.x / p.maxtiles, tt, g, ft, pb, pl);
}

template <int D, bool INL, int VS>
__global__ __launch_bounds__(64 * kPvWaves) void k_fa_pv(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    using PB = PvBlock<D, VS>;
    constexpr uint32_t DV = PB::DV, BB = PB::BB;
    const uint32_t G = a.G, nh = a.n_head;
    uint32_t * s_t64 = (uint32_t *)lds;                           // EXPK table
    float * s_c = (float *)(lds + 256);                           // [seg][4 heads][DV]
    float * s_l = s_c + kPvMaxSeg * 4u * DV;                      // [seg][4 heads]
    uint8_t * s_dg = (uint8_t *)(s_l + kPvMaxSeg * 4u);          // per wave: [BB blocks][4 heads][4 digits][4 groups][16]
    const uint32_t t64v = a.ex.t64[threadIdx.x & 63u];            // first: the table write waits for it only
    const uint32_t item = blockIdx.x >> 2, c = blockIdx.x & 3u, g = blockIdx.y;
    const uint32_t hg = blockIdx.z / VS, vh = blockIdx.z % VS;
    const FaItem it = fa_item<INL>(a, p, item);
    const uint32_t lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t h = g * G + min(4u * hg + (lane >> 4), G - 1u);
    const PB pb(a, it, c, g, hg, vh, a.S + (size_t)it.s_off * nh + (size_t)h * (16u * it.n));
    uint8_t * dg = s_dg + (size_t)wave * (BB * 1024u);
    const uint32_t mkey = maxt_key_f(a.Mpart[(size_t)(it.tile0 + min(lane & 15u, it.ntiles - 1u)) * nh + h]);

    typename PB::Loads L;
    if (wave < pb.nseg) pb.loads(wave, pb.vb0, L, true);
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = t64v;
    lds_barrier();

    // chunk maximum of head h: MAXOUT of the floor and the tile maxima (row lanes < ntiles read one each)
    const float m = maxt_unkey(row16_umax(max(mkey, maxt_key_f(bf(kMFloor)))));
    for (uint32_t seg = wave; seg < pb.nseg; seg += nw) {
        if (seg != wave) pb.loads(seg, pb.vb0, L, true);
        pb.segment(seg, seg, L, m, s_t64, s_c, s_l, dg);
    }
    __syncthreads();
    pb.chains(item, hg, s_c, s_l);
}

// ---------------------------------------------------------------------------------------------
// merge: block (token, KV head g x group of 4 heads, slice sl), lane = (head of the group, value).
// Each lane loads the channel partials, row sums and maxima of up to kMergeItems chunks at once (the
// first round's before the EXPK table is published), then runs CTREE over the 4 channels, the online
// merge in chunk order and finally ANORM (AT 5.6, 5.7). The running maxima of a round are
// wave-uniform, so its 2 kMergeItems merge factors are evaluated by as many lanes at once and read
// back with readlane.
// ---------------------------------------------------------------------------------------------
constexpr uint32_t kMergeItems = 4;                              // chunks loaded per round
constexpr uint32_t kMergeHeads = 4;                              // heads per block

template <bool INL>
__global__ __launch_bounds__(256) void k_fa_merge(FaArgs a, FaPlan p) {
    const uint32_t G = a.G, D = a.D, nh = a.n_head;
    const uint32_t ngrp = (G + kMergeHeads - 1u) / kMergeHeads;
    const uint32_t t = blockIdx.x, g = blockIdx.y / ngrp, h0 = g * G + (blockIdx.y % ngrp) * kMergeHeads;
    const uint32_t hn = min(kMergeHeads, g * G + G - h0), sl = blockIdx.z;
    const uint32_t i = threadIdx.x >> 6, L = threadIdx.x & 63u;
    __shared__ uint32_t s_t64[64];
    const uint32_t t64v = a.ex.t64[L];                            // first: the table write waits for it only
    const uint32_t first = INL ? p.tok_first[t] : a.tok_first[t];
    const uint32_t cnt = INL ? p.tok_count[t] : a.tok_count[t];  // >= 1 (a row without cells has one empty chunk)
    const uint32_t h = h0 + min(i, hn - 1u);                      // waves past the group load, then leave

    struct Round {
        float op[kMergeItems][4], lp[kMergeItems][4];
        uint32_t key;                                             // MAXT key of one tile maximum
    };
    auto load_round = [&](uint32_t k0, Round & R) {
        const uint32_t kn = min(kMergeItems, cnt - k0);
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {                // clamped: every load is issued up front
            const size_t kk = first + k0 + min(k, kn - 1u);
#pragma unroll
            for (uint32_t c = 0; c < 4u; ++c) {
                const size_t slot = (kk * 4u + c) * nh + h;
                R.op[k][c] = a.OP[slot * D + 64u * sl + L];
                R.lp[k][c] = a.LP[slot];
            }
        }
        // lane 8 k + j (k < kMergeItems) reads tile j (clamped) of chunk k: an item has at most 8
        // tiles (NCG <= 128 groups of 16 cells)
        uint32_t tile = 0;
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {                // uniform item reads, per-lane select
            const FaItem itk = fa_item<INL>(a, p, first + k0 + min(k, kn - 1u));
            if ((L >> 3) == k) tile = itk.tile0 + min(L & 7u, itk.ntiles - 1u);
        }
        R.key = maxt_key_f(a.Mpart[(size_t)tile * nh + h]);
    };

    Round R;
    load_round(0u, R);
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = t64v;
    lds_barrier();
    if (i >= hn) return;                                          // whole waves

    float O = 0.0f, l = 0.0f, mr = 0.0f;
    for (uint32_t k0 = 0; k0 < cnt; k0 += kMergeItems) {
        if (k0 != 0u) load_round(k0, R);
        const uint32_t kn = min(kMergeItems, cnt - k0);
        // chunk maxima: MAXOUT of the floor and the chunk's tile maxima over each 8-lane group
        uint32_t key = max(R.key, maxt_key_f(bf(kMFloor)));
        key = umax_u(key, (uint32_t)dpp_i<kDppXor1>((int)key));
        key = umax_u(key, (uint32_t)dpp_i<kDppXor2>((int)key));
        key = umax_u(key, (uint32_t)dpp_i<kDppRowHalfMirror>((int)key));
        float mk[kMergeItems], mrun[kMergeItems];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            mk[k] = maxt_unkey((uint32_t)__builtin_amdgcn_readlane((int)key, 8 * (int)k));
            const float prev = k == 0u ? mr : mrun[k - 1u];
            mrun[k] = k0 + k == 0u ? mk[k] : maxt(prev, mk[k]);
        }
        // lane 2 k + b: factor of chunk k, EXP((prev - mrun_k) scale) for b = 0 (the running sums),
        // EXP((m_k - mrun_k) scale) for b = 1 (the chunk's); the first chunk of a row uses none
        const uint32_t jk = (L >> 1) & (kMergeItems - 1u);
        float from = 0.0f, to = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k)
            if (jk == k) {
                from = (L & 1u) ? mk[k] : (k == 0u ? mr : mrun[k - 1u]);
                to = mrun[k];
            }
        const float fx = expk(smul_n(ssub_n(from, to), a.scale), a.ex, s_t64);
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            if (k >= kn) break;
            const float ok = ctree4(R.op[k][0], R.op[k][1], R.op[k][2], R.op[k][3]);
            const float lk = ctree4(R.lp[k][0], R.lp[k][1], R.lp[k][2], R.lp[k][3]);
            if (k0 + k == 0u) { O = ok; l = lk; }
            else {
                const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)k));
                const float fbv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)k + 1));
                l = sadd_n(smul_n(l, fa), smul_n(lk, fbv));
                O = sadd_n(smul_n(O, fa), smul_n(ok, fbv));
            }
            mr = mrun[k];
        }
    }
    a.out[(size_t)t * a.out_stride + (size_t)h * D + 64u * sl + L] = smul_n(O, srcp(maxt(l, bf(kLFloor))));
}

}  // namespace tsr

template <bool INL>
static int launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, uint32_t n_cu, hipStream_t s) {
    const bool rope = a.cell != nullptr;                          // ROPE + SET_ROWS_KV fused (host-checked shape)
    const size_t lds_qk = tsr::fa_qk_lds(a.G, a.D, rope);
    const dim3 gqk(p.n_items * p.maxtiles, a.n_head_kv);
    if (!INL && a.sync != nullptr && T == 1u && a.G <= 4u && (a.D == 64u || a.D == 128u)) {
        // decode over a plan's work list: scores, P.V and the merge in one launch
        const size_t lds = ((lds_qk + 15u) & ~(size_t)15u) + tsr::fa_fuse_lds(a.D);
        switch (a.D * 2u + (rope ? 1u : 0u)) {
            case 128: hipLaunchKernelGGL((tsr::k_fa_qk<64, false, false, true>), gqk, dim3(256), lds, s, a, p); break;
            case 129: hipLaunchKernelGGL((tsr::k_fa_qk<64, false, true, true>), gqk, dim3(256), lds, s, a, p); break;
            case 256: hipLaunchKernelGGL((tsr::k_fa_qk<128, false, false, true>), gqk, dim3(256), lds, s, a, p); break;
            case 257: hipLaunchKernelGGL((tsr::k_fa_qk<128, false, true, true>), gqk, dim3(256), lds, s, a, p); break;
            default: return -2;
        }
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    if (rope) {
        switch (a.D) {
            case 64: hipLaunchKernelGGL((tsr::k_fa_qk<64, INL, true>), gqk, dim3(256), lds_qk, s, a, p); break;
            case 128: hipLaunchKernelGGL((tsr::k_fa_qk<128, INL, true>), gqk, dim3(256), lds_qk, s, a, p); break;
            default: return -2;
        }
    } else {
        switch (a.D) {
            case 64: hipLaunchKernelGGL((tsr::k_fa_qk<64, INL, false>), gqk, dim3(256), lds_qk, s, a, p); break;
            case 128: hipLaunchKernelGGL((tsr::k_fa_qk<128, INL, false>), gqk, dim3(256), lds_qk, s, a, p); break;
            case 256: hipLaunchKernelGGL((tsr::k_fa_qk<256, INL, false>), gqk, dim3(256), lds_qk, s, a, p); break;
            case 512: hipLaunchKernelGGL((tsr::k_fa_qk<512, INL, false>), gqk, dim3(256), lds_qk, s, a, p); break;
            default: return -2;
        }
    }
    if (hipGetLastError() != hipSuccess) return -4;
    // P.V: waves = the most segments of any item (<= 8), LDS = table, segment results, digits; the
    // values of a head are split over VS blocks while the grid holds fewer than two blocks per CU
    uint32_t maxn = 0;
    if (INL) {
        for (uint32_t i = 0; i < p.n_items; ++i) maxn = std::max(maxn, p.items[i].n);
    } else {
        maxn = a.max_groups;
    }
    const uint32_t nwv = std::max(1u, std::min(tsr::kPvWaves, ((maxn + 3u) / 4u + 3u) / 4u));
    const uint64_t blocks = 4ull * p.n_items * a.n_head_kv * ((a.G + 3u) / 4u);
    uint32_t vs = 1;
    while (vs < 4u && a.D / (2u * vs) >= 64u && blocks * vs < 2ull * n_cu) vs *= 2u;
    const uint32_t dv = a.D / vs, bb = std::min(4u, dv / 32u);
    const size_t lds_pv = 256u + 4u * (size_t)tsr::kPvMaxSeg * 4u * dv + 4u * tsr::kPvMaxSeg * 4u + 1024u * bb * nwv;
    const dim3 gpv(4u * p.n_items, a.n_head_kv, (a.G + 3u) / 4u * vs);
    const dim3 bpv(64u * nwv);
#define TSR_PV(DD, VV) hipLaunchKernelGGL((tsr::k_fa_pv<DD, INL, VV>), gpv, bpv, lds_pv, s, a, p)
    switch (a.D * 8u + vs) {
        case 64 * 8 + 1: TSR_PV(64, 1); break;
        case 128 * 8 + 1: TSR_PV(128, 1); break;
        case 128 * 8 + 2: TSR_PV(128, 2); break;
        case 256 * 8 + 1: TSR_PV(256, 1); break;
        case 256 * 8 + 2: TSR_PV(256, 2); break;
        case 256 * 8 + 4: TSR_PV(256, 4); break;
        case 512 * 8 + 1: TSR_PV(512, 1); break;
        case 512 * 8 + 2: TSR_PV(512, 2); break;
        case 512 * 8 + 4: TSR_PV(512, 4); break;
        default: return -2;
    }
#undef TSR_PV
    if (hipGetLastError() != hipSuccess) return -4;
    const uint32_t ngrp = (a.G + tsr::kMergeHeads - 1u) / tsr::kMergeHeads;
    hipLaunchKernelGGL(tsr::k_fa_merge<INL>, dim3(T, a.n_head_kv * ngrp, a.D / 64u), dim3(256), 0, s, a, p);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, uint32_t n_cu, hipStream_t s) {
    return a.items ? launch_fa<false>(a, p, T, n_cu, s) : launch_fa<true>(a, p, T, n_cu, s);
}
