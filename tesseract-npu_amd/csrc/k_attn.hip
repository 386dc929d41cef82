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
#include "fa_common.hpp"

#include <algorithm>

namespace tsr {

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

// The P.V work of one block (chunk item, channel c, KV head g, head group hg, value part vh), shared by
// k_fa_pv (the item's scores in global memory). Lane = (head row hr, group kk of the segment, cell quad);
// one wave per segment.
template <int D, int VS>
struct PvBlock {
    static constexpr uint32_t DV = D / VS;                        // values of the block (>= 64)
    static constexpr uint32_t NBV = DV / 32;                      // their value blocks
    static constexpr uint32_t BB = 2;                             // blocks per batch: one 64-value slice (fewer registers: more waves per SIMD)
    static constexpr uint32_t NBT = NBV / BB;                     // batches
    static_assert(DV >= 64 && NBV % BB == 0, "value part");
    // the loads of one segment: scores, value scales and the value quants of a batch
    struct Loads {
        float4 sv;
        uint32_t mb[BB][2];                                       // block e: scales of cells 0, 1 | 2, 3
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
        const uint16_t * vm = vmeta + ((size_t)u * nbk + (size_t)g * (D / 32u) + vb) * 16u + 4u * quad;
#pragma unroll
        for (uint32_t e = 0; e < BB; ++e) {                       // the 4 cells' scales of block e: 8 bytes
            const uint2 m2 = *(const uint2 *)(vm + (size_t)e * 16u);
            L.mb[e][0] = m2.x;
            L.mb[e][1] = m2.y;
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
            const float ez = expk_diff(ss[i], m, a.scale, a.ex, s_t64);   // straight-line, then the select
            pz[i] = (cv && head_ok) ? ez : 0.0f;
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
                    const uint32_t dv = (L.mb[e][i >> 1] >> (16u * (i & 1u))) & 0xFFFFu;
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
            for (uint32_t seg = 0; seg < nseg; ++seg) O = sadd_z(O, s_c[(seg * 4u + r4) * DV + v]);
            const size_t slot = ((size_t)item * 4u + c) * nh + h2;
            a.OP[slot * D + vh * DV + v] = canon(O);
            if (vh == 0u && v == 0u) {
                float l = 0.0f;
                for (uint32_t seg = 0; seg < nseg; ++seg) l = l + s_l[seg * 4u + r4];   // see ctree4_l
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
// ROPE (T == 1, D <= 128, (G + 2) D <= 1024): the block also rotates the query heads (rope4, angles
// per lane by rope_cs_lane) before their QACT, rotates and QACTs the token's k row of head g and
// QACTs its v row (threads after the query slots, A32 as SET_ROWS_KV); the thread of the new cell
// scores with that fresh k row, and the first block of each KV head stores the k and v rows in the
// caches -- ROPE, SET_ROWS_KV and the scores in one launch.
template <int D, bool INL, bool ROPE>
__global__ __launch_bounds__(256) void k_fa_qk(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t NBD = D / 32u;                             // blocks per head
    constexpr bool KREG = D <= 128;                                // K row of the cell kept in registers
    static_assert(!ROPE || KREG, "the fused ROPE keeps the K rows in registers");
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

    const uint32_t n16 = 16u * it.n, j = 256u * tt + threadIdx.x;
    const bool in = j < n16;
    const uint32_t cell = 16u * it.u0 + j;
    const uint32_t ng = (a.kc.kv_size + 15u) / 16u;
    const uint32_t u = min(cell >> 4, ng - 1u), rr = cell & 15u;  // clamped: loads stay inside the plane
    const bool vis = in && (it.general || (j >= it.c_lo && j < it.c_hi));
    const uint32_t E = a.E, nbk = E / 32u;
    const uint16_t * kmeta = (const uint16_t *)a.kc.base + ((size_t)u * nbk + (size_t)g * NBD) * 16u + rr;
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
    for (uint32_t kb = 0; kb < NBD; ++kb) km[kb] = kmeta[(size_t)kb * 16u];
    if constexpr (KREG) {
#pragma unroll
        for (uint32_t c = 0; c < 2 * NBD; ++c) kr[c] = *(const int4 *)(kq + (size_t)(ci0 + c) * 256u);
    }
    __builtin_amdgcn_sched_barrier(0);

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
        if (blockIdx.x == 0u) {                                   // the caches' copy of the new rows
            if (cell_ok && (is_k || is_v)) {
                KvArgs kv;                                        // per-lane choice of the plane, field by field
                kv.base = is_k ? a.kc.base : a.vc.base;
                kv.quant_off = is_k ? a.kc.quant_off : a.vc.quant_off;
                kv.E = a.kc.E;
                kv.kv_size = is_k ? a.kc.kv_size : a.vc.kv_size;
                kv_store_unit(kv, is_k ? 0u : 1u, (uint32_t)cell64, g * D + 4u * (is_k ? kslot : vslot), qq, Dq,
                              (lane & 7) == 0);
            }
            if (!cell_ok && threadIdx.x == 0u && g == 0u && a.bad != nullptr) *a.bad = 1;
        }
    } else {
        qact_slot(threadIdx.x, qv0);
        for (uint32_t s0 = blockDim.x; s0 < nslot; s0 += blockDim.x)   // G D > 1024 only
            qact_slot(s0 + threadIdx.x, *(const float4 *)(qrow + 4u * min(s0 + threadIdx.x, nslot - 1u)));
    }
    lds_barrier();                                                // the K rows stay in flight
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
                // the plain operations never meet a subnormal; NaN is canonicalized below. The +0 is
                // added once to the tree's result instead: a -0 term changes a node only when every
                // term under it is -0, and then the node is -0 where the rule's is +0
                p[kb] = (h2f_fast(km[kb]) * s_dx[i * NBD + kb]) * (float)is;
            }
#pragma unroll
            for (int w = 16; w > 1; w >>= 1)
#pragma unroll
                for (int k = 0; k < w / 2; ++k) p[k] = p[2 * k] + p[2 * k + 1];
            s = canon(p[0] + 0.0f);
            if (it.general) {
                const float m = a.mask[(size_t)it.t * a.mstride + cell];
                s = fb(m) == kNegInf ? bf(kNegInf) : sadd(s, m);
            }
        }
        if (in) S[(size_t)h * n16 + j] = s;
        const uint32_t mk = wave_max_u(in ? maxt_key_f(s) : maxt_key_f(bf(kMFloor)));
        if (lane == 0) s_red[wave * G + i] = mk;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < G; i += blockDim.x) {
        uint32_t m = s_red[i];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = umax_u(m, s_red[w * G + i]);
        a.Mpart[(size_t)(it.tile0 + tt) * a.n_head + g * G + i] = maxt_unkey(m);
    }
}

template <int D, bool INL, int VS>
__global__ __launch_bounds__(64 * kPvWaves) void k_fa_pv(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    using PB = PvBlock<D, VS>;
    constexpr uint32_t DV = PB::DV, BB = PB::BB;
    const uint32_t G = a.G, nh = a.n_head;
    // the launch has one wave per segment of its longest channel (nw <= kPvWaves), so the segment
    // results need nw slots: the LDS is sized by the launch
    const uint32_t nw = blockDim.x >> 6;
    uint32_t * s_t64 = (uint32_t *)lds;                           // EXPK table
    float * s_c = (float *)(lds + 256);                           // [seg][4 heads][DV]
    float * s_l = s_c + nw * 4u * DV;                             // [seg][4 heads]
    uint8_t * s_dg = (uint8_t *)(s_l + nw * 4u);                  // per wave: [BB blocks][4 heads][4 digits][4 groups][16]
    const uint32_t t64v = a.ex.t64[threadIdx.x & 63u];            // first: the table write waits for it only
    const uint32_t item = blockIdx.x >> 2, c = blockIdx.x & 3u, g = blockIdx.y;
    const uint32_t hg = blockIdx.z / VS, vh = blockIdx.z % VS;
    const FaItem it = fa_item<INL>(a, p, item);
    const uint32_t lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
// back with readlane. A row of one chunk has nothing to merge: its lanes load the four channel
// partials and row sums only and go straight to CTREE and ANORM (the general path's bits for cnt 1).
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

    if (cnt == 1u) {                                              // one chunk (workgroup-uniform): no merge,
        float op[4], lp[4];                                       // so no maxima, items or factors to load
#pragma unroll
        for (uint32_t c = 0; c < 4u; ++c) {
            const size_t slot = ((size_t)first * 4u + c) * nh + h;
            op[c] = a.OP[slot * D + 64u * sl + L];
            lp[c] = a.LP[slot];
        }
        if (i >= hn) return;
        const float O = ctree4_o(op[0], op[1], op[2], op[3]);
        const float l = ctree4_l(lp[0], lp[1], lp[2], lp[3]);
        a.out[(size_t)t * a.out_stride + (size_t)h * D + 64u * sl + L] = smul_n(O, srcp(maxt(l, bf(kLFloor))));
        return;
    }

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
        const float fx = expk_diff(from, to, a.scale, a.ex, s_t64);
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            if (k >= kn) break;
            const float ok = ctree4_o(R.op[k][0], R.op[k][1], R.op[k][2], R.op[k][3]);
            const float lk = ctree4_l(R.lp[k][0], R.lp[k][1], R.lp[k][2], R.lp[k][3]);
            if (k0 + k == 0u) { O = ok; l = lk; }
            else {
                const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)k));
                const float fbv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)k + 1));
                l = sadd_c(smul_c(l, fa), smul_c(lk, fbv));
                O = sadd_z(smul_z(O, fa), smul_z(ok, fbv));
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
    const uint32_t dv = a.D / vs, bb = 2u;                        // PvBlock::BB
    const size_t lds_pv = 256u + 4u * (size_t)nwv * 4u * dv + 4u * nwv * 4u + 1024u * bb * nwv;
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
