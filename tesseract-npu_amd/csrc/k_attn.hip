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
// runs on v_dot4_i32_i8 with exact int32 partial sums (|sum| <= 64 * 128 * 128).
#include "kernels.hpp"
#include "qact.hpp"

#include <algorithm>

namespace tsr {

constexpr uint32_t kMFloor = 0xF1800000u;   // -2^100 (AT 6.3)
constexpr uint32_t kLFloor = 0x00800000u;   // 2^-126 (AT 5.7)

// EXPK(v, P1) (VU 6.3; sw/sim/tsr_ref_math.c:78-159), constants from the host (ExpkTab). The
// 2^(j/64) table is read from LDS (t64): an index into the kernel arguments that differs per lane
// would be a vector load from the argument segment on every call. Straight-line: the special cases
// are selected at the end, so a wave never splits into branches here.
__device__ __forceinline__ float expk(float v, const ExpkTab & e, const uint32_t * t64) {
    const uint32_t u = fb(daz(v));
    const uint32_t a = u & 0x7FFFFFFFu;
    const bool neg = (u >> 31) != 0u;
    const uint32_t ev = a >> 23;
    // T = floor(Mv LK / 2^(156 - ev)) for ev <= 156 (larger ev: overflow / underflow below)
    const uint64_t mv = 0x00800000u | (a & 0x007FFFFFu);
    const uint32_t sh = 156u - min(ev, 156u);
    const uint64_t prod = mv * e.lk;
    const uint64_t T = sh >= 64u ? 0ull : (prod >> sh);
    const uint32_t Thi = (uint32_t)(T >> 32), Tlo = (uint32_t)T;
    const int32_t n0 = neg ? -(int32_t)(Thi + (Tlo ? 1u : 0u)) : (int32_t)Thi;
    const uint32_t F = neg ? 0u - Tlo : Tlo;
    const uint64_t G = F & 0x03FFFFFFu;
    const uint64_t pf = (G * (e.c1 + ((G * (e.c2 + ((G * e.c3) >> 32))) >> 32))) >> 32;
    const uint64_t t = t64[F >> 26];
    const uint64_t M = t + ((t * pf) >> 32);
    const bool hiM = M >= (1ull << 31);
    const uint32_t drop = hiM ? 8u : 7u;
    uint32_t sig = (uint32_t)(M >> drop);
    const uint32_t rem = (uint32_t)M & ((1u << drop) - 1u), half = 1u << (drop - 1u);
    sig += (rem > half || (rem == half && (sig & 1u))) ? 1u : 0u;
    const bool carry = sig == (1u << 24);
    const int32_t be = n0 + (hiM ? 1 : 0) + (carry ? 1 : 0) + 127;
    const uint32_t mant = (carry ? sig >> 1 : sig) & 0x007FFFFFu;
    uint32_t r = be >= 255 ? 0x7F800000u : (be <= 0 ? 0u : (((uint32_t)be << 23) | mant));
    const uint32_t big = neg ? 0u : 0x7F800000u;                  // +Inf, or 0 for large negative v
    r = (ev > 156u || T >= (1ull << 40) || a == 0x7F800000u) ? big : r;
    r = a == 0u ? 0x3F800000u : r;
    r = a > 0x7F800000u ? kNaN : r;
    return bf(r);
}

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

// RNE_int(w 2^(23 - es)), exponent(w) <= es; zero / subnormal w -> 0 (sw/sim/tsr_ref_at.c:386-410).
// Straight-line: a shift of 26 or more leaves 0 after rounding (|m| < 2^24), so it is clamped to 31.
__device__ __forceinline__ int32_t bf_int(float w, int32_t es) {
    const uint32_t u = fb(w), e = (u >> 23) & 0xFFu;
    const uint32_t m = 0x00800000u | (u & 0x007FFFFFu);
    const int32_t sh0 = es - ((int32_t)e - 127);
    const uint32_t sh = (uint32_t)min(max(sh0, 0), 31);
    uint32_t v = m >> sh;
    const uint32_t r = m & ((1u << sh) - 1u), h = sh ? 1u << (sh - 1u) : 0u;
    v += (sh && (r > h || (r == h && (v & 1u)))) ? 1u : 0u;
    const int32_t sv = (u >> 31) ? -(int32_t)v : (int32_t)v;
    return e == 0u ? 0 : sv;
}
// RNE24(A) 2^k; below 2^-126 a signed zero, from 2^128 a signed Inf (sw/sim/tsr_ref_at.c:412-436).
// Straight-line.
__device__ __forceinline__ float bf_f(int64_t A, int32_t k) {
    const uint32_t s = A < 0 ? 0x80000000u : 0u;
    const uint64_t mag = A < 0 ? (uint64_t)0 - (uint64_t)A : (uint64_t)A;
    const int32_t msb = 63 - (int32_t)__builtin_clzll(mag | 1ull);
    const uint32_t shr = (uint32_t)max(msb - 23, 0), shl = (uint32_t)max(23 - msb, 0);
    uint64_t sig = mag >> shr;
    const uint64_t r = mag & ((1ull << shr) - 1ull), h = shr ? 1ull << (shr - 1u) : 0ull;
    sig += (shr && (r > h || (r == h && (sig & 1ull)))) ? 1ull : 0ull;
    const bool carry = (sig >> 24) != 0ull;
    sig = carry ? sig >> 1 : sig;
    sig = sig << shl;
    const int32_t e = msb + k + (carry ? 1 : 0);
    uint32_t out = s | ((uint32_t)(e + 127) << 23) | ((uint32_t)sig & 0x007FFFFFu);
    out = e < -126 ? s : (e > 127 ? (s | 0x7F800000u) : out);
    return bf(A == 0 ? 0u : out);
}

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

template <int D, bool INL>
__global__ __launch_bounds__(256) void k_fa_qk(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t NBD = D / 32u;                             // blocks per head
    constexpr bool KREG = D <= 128;                                // K row of the cell kept in registers
    const uint32_t tt = blockIdx.x % p.maxtiles;
    const FaItem it = fa_item<INL>(a, p, blockIdx.x / p.maxtiles);
    if (tt >= it.ntiles) return;                                  // the item has fewer tiles (block-uniform)
    const uint32_t g = blockIdx.y, G = a.G;
    int8_t * s_q = (int8_t *)lds;                                 // G*D quants of the KV head's query heads
    float * s_dx = (float *)(lds + G * D);                        // G*D/32 scales
    uint32_t * s_red = (uint32_t *)(s_dx + G * NBD);              // 4 waves x G maxima (keys)
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6);

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
    const float4 qv0 = *(const float4 *)(qrow + 4u * min(threadIdx.x, nslot - 1u));
    __builtin_amdgcn_sched_barrier(0);

    int4 kr[KREG ? 2 * NBD : 1];
    uint32_t km[NBD];
#pragma unroll
    for (uint32_t kb = 0; kb < NBD; ++kb) km[kb] = kmeta[kb];
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
    qact_slot(threadIdx.x, qv0);
    for (uint32_t s0 = blockDim.x; s0 < nslot; s0 += blockDim.x)   // G D > 1024 only
        qact_slot(s0 + threadIdx.x, *(const float4 *)(qrow + 4u * min(s0 + threadIdx.x, nslot - 1u)));
    lds_barrier();                                                // the K rows stay in flight

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

// ---------------------------------------------------------------------------------------------
// P.V: block (item * 4 + channel c, KV head g, group hg of 4 query heads); one wave per segment of
// the channel (4 of its groups = 64 cells), looping if there are more segments than waves. Each
// segment's results go to LDS; the f32 segment chain then runs in segment order.
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
// holds the four digit sums of head l / 16 and value l % 16 and forms A exactly in 64 bits.
// ---------------------------------------------------------------------------------------------
constexpr uint32_t kPvWaves = 8;                                  // NCG <= 128 -> <= 8 segments per channel
constexpr uint32_t kPvMaxSeg = 8;

__device__ __forceinline__ float ctree4(float x0, float x1, float x2, float x3) { return sadd(sadd(x0, x1), sadd(x2, x3)); }
__device__ __forceinline__ int32_t row16_imax(int32_t v) {          // signed max over a 16-lane row
    return (int32_t)(row16_umax((uint32_t)v ^ 0x80000000u) ^ 0x80000000u);
}
__device__ __forceinline__ int32_t row16_isum(int32_t v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppRowHalfMirror>(v);
    return v + dpp_i<kDppRowMirror>(v);
}
__device__ __forceinline__ int32_t f_exp(float f) { return (int32_t)((fb(f) >> 23) & 0xFFu) - 127; }
__device__ __forceinline__ bool f_nonfinite(float f) { return (fb(f) & 0x7F800000u) == 0x7F800000u; }

typedef int v4i_fa __attribute__((ext_vector_type(4)));

template <int D, bool INL>
__global__ __launch_bounds__(64 * kPvWaves) void k_fa_pv(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t NBD = D / 32;                              // value blocks of a head
    constexpr uint32_t BB = NBD < 4 ? NBD : 4;                    // blocks per batch (2 or 4)
    const uint32_t G = a.G, E = a.E, nh = a.n_head;
    const uint32_t nbk = E / 32u;                                 // value blocks of a cell
    uint32_t * s_t64 = (uint32_t *)lds;                           // EXPK table
    float * s_c = (float *)(lds + 256);                           // [seg][4 heads][D]
    float * s_l = s_c + kPvMaxSeg * 4u * D;                       // [seg][4 heads]
    uint8_t * s_dg = (uint8_t *)(s_l + kPvMaxSeg * 4u);          // per wave: [4 blocks][4 heads][4 digits][4 groups][16]
    const uint32_t t64v = a.ex.t64[threadIdx.x & 63u];            // first: the table write waits for it only
    const uint32_t item = blockIdx.x >> 2, c = blockIdx.x & 3u, g = blockIdx.y, hg = blockIdx.z;
    const FaItem it = fa_item<INL>(a, p, item);
    const uint32_t lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t hr = lane >> 4, kk = (lane >> 2) & 3u, quad = lane & 3u;
    const uint32_t hi = 4u * hg + hr;                             // query head within the KV head
    const bool head_ok = hi < G;
    const uint32_t h = g * G + min(hi, G - 1u);
    const uint32_t u_first = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u);
    const uint32_t u_end = it.u0 + it.n;
    const uint32_t nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
    const uint32_t nseg = (nu + 3u) / 4u;
    const uint32_t n16 = 16u * it.n;
    const float * S = a.S + (size_t)it.s_off * nh + (size_t)h * n16;
    const uint16_t * vmeta = (const uint16_t *)a.vc.base;
    const uint8_t * vq = a.vc.base + a.vc.quant_off;
    uint8_t * dg = s_dg + (size_t)wave * 4096u;
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = t64v;
    lds_barrier();

    // chunk maximum of head h: MAXOUT of the floor and the tile maxima (row lanes < ntiles read one each)
    const uint32_t mkey = maxt_key_f(a.Mpart[(size_t)(it.tile0 + min(lane & 15u, it.ntiles - 1u)) * nh + h]);
    const float m = maxt_unkey(row16_umax(max(mkey, maxt_key_f(bf(kMFloor)))));

    for (uint32_t seg = wave; seg < nseg; seg += nw) {
        // ---- phase A: lane = (head row, 4 cells) ----------------------------------------------
        const uint32_t gi = 4u * seg + kk;                         // the channel's group index
        const bool cv = gi < nu;
        const uint32_t u = u_first + 4u * min(gi, nu - 1u);        // clamped: loads stay in the item
        const uint32_t j0 = 16u * (u - it.u0) + 4u * quad;         // first cell of the lane in the chunk
        const float4 sv = *(const float4 *)(S + j0);
        const float ss[4] = { sv.x, sv.y, sv.z, sv.w };
        float pz[4];
        bool pnf_any = false;
        int32_t ep = -1000;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pe = (cv && head_ok) ? expk(smul(ssub(ss[i], m), a.scale), a.ex, s_t64) : 0.0f;
            pz[i] = daz(pe);
            const bool nf = f_nonfinite(pz[i]);
            pnf_any |= nf;
            if (!nf && (fb(pz[i]) & 0x7FFFFFFFu)) ep = max(ep, f_exp(pz[i]));
        }
        // LSUM of the segment (AT 6.5): block float of its p values
        const bool badl = row16_umax(pnf_any ? 1u : 0u) != 0u;
        ep = row16_imax(ep);
        int32_t lsum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lsum += f_nonfinite(pz[i]) ? 0 : bf_int(pz[i], ep);
        lsum = row16_isum(lsum);
        if ((lane & 15u) == 0u)
            s_l[seg * 4u + hr] = badl ? bf(kNaN) : (ep == -1000 ? 0.0f : bf_f((int64_t)lsum, ep - 23));

        const uint16_t * vm = vmeta + ((size_t)u * 16u + 4u * quad) * nbk + (size_t)g * NBD;
#pragma unroll 1
        for (uint32_t vb = 0; vb < NBD; vb += BB) {                // BB value blocks (32 BB values) at a time
            // weights of the 4 cells for the BB blocks
            float w[4][BB];
            int32_t ex[BB / 2];
            bool nfb[BB];
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) nfb[e] = false;
#pragma unroll
            for (uint32_t sa = 0; sa < BB / 2; ++sa) ex[sa] = -1000;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t dv[BB];
                if constexpr (BB == 4) {
                    const uint2 mv = *(const uint2 *)(vm + (size_t)i * nbk + vb);
                    dv[0] = mv.x & 0xFFFFu; dv[1] = mv.x >> 16; dv[2] = mv.y & 0xFFFFu; dv[3] = mv.y >> 16;
                } else {
                    const uint32_t mv = *(const uint32_t *)(vm + (size_t)i * nbk + vb);
                    dv[0] = mv & 0xFFFFu; dv[1] = mv >> 16;
                }
                const bool live = (fb(pz[i]) & 0x7FFFFFFFu) != 0u;
#pragma unroll
                for (uint32_t e = 0; e < BB; ++e) {
                    const float we = live ? smul(pz[i], h2f_exact(dv[e])) : 0.0f;
                    w[i][e] = we;
                    const bool nf = f_nonfinite(we);
                    nfb[e] |= nf;
                    if (!nf && (fb(we) & 0x7FFFFFFFu)) ex[e >> 1] = max(ex[e >> 1], f_exp(we));
                }
            }
            int32_t es[BB / 2];
            bool any[BB / 2], bad[BB];
#pragma unroll
            for (uint32_t sa = 0; sa < BB / 2; ++sa) { es[sa] = row16_imax(ex[sa]); any[sa] = es[sa] > -1000; }
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) bad[e] = row16_umax(nfb[e] ? 1u : 0u) != 0u;
            // digits: for block e and digit k, the 4 cells' digit bytes in one word
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) {
                uint32_t P[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int32_t W = (any[e >> 1] && !bad[e]) ? bf_int(w[i][e], es[e >> 1]) : 0;
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
            // ---- phase B: 8 tiles of 16 values; lane = (head row l / 16 of the result, value l % 16)
            const uint32_t kB = lane >> 4;                          // the operand's 16 cells: group kB
            const uint32_t uB = u_first + 4u * min(4u * seg + kB, nu - 1u);
            const uint8_t * vqB = vq + ((size_t)uB * E + (size_t)g * D + 32u * vb + (lane & 15u)) * 16u;
            int4 Bv[2 * BB];
#pragma unroll
            for (uint32_t t8 = 0; t8 < 2 * BB; ++t8) Bv[t8] = *(const int4 *)(vqB + 256u * t8);
#pragma unroll
            for (uint32_t e = 0; e < BB; ++e) {
                // A operand: row l % 16 = (head, digit), K = the 16 cells of group l / 16
                const v4i_fa Aop = *(const v4i_fa *)(dg + ((e * 16u + (lane & 15u)) * 4u + (lane >> 4)) * 16u);
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int4 bq = Bv[2 * e + half];
                    const v4i_fa Bop = { bq.x, bq.y, bq.z, bq.w };
                    v4i_fa acc = { 0, 0, 0, 0 };
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(Aop, Bop, acc, 0, 0, 0);
                    const int64_t A = (int64_t)acc[0] + ((int64_t)acc[1] << 8) + ((int64_t)acc[2] << 16) + ((int64_t)acc[3] << 24);
                    const float cval = bad[e] ? bf(kNaN) : (any[e >> 1] ? bf_f(A, es[e >> 1] - 23) : 0.0f);
                    s_c[(seg * 4u + hr) * D + 32u * (vb + e) + 16u * (uint32_t)half + (lane & 15u)] = cval;
                }
            }
        }
    }
    __syncthreads();
    // segment chains in order (AT 6.4 O, 6.5 l): thread = (head row, value)
    for (uint32_t idx = threadIdx.x; idx < 4u * D; idx += blockDim.x) {
        const uint32_t r4 = idx / D, v = idx % D, hi2 = 4u * hg + r4;
        if (hi2 >= G) continue;
        const uint32_t h2 = g * G + hi2;
        float O = 0.0f;
        for (uint32_t seg = 0; seg < nseg; ++seg) O = sadd(O, s_c[(seg * 4u + r4) * D + v]);
        const size_t slot = ((size_t)item * 4u + c) * nh + h2;
        a.OP[slot * D + v] = O;
        if (v == 0u) {
            float l = 0.0f;
            for (uint32_t seg = 0; seg < nseg; ++seg) l = sadd(l, s_l[seg * 4u + r4]);
            a.LP[slot] = l;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// merge: block (token, KV head g x group of 4 heads, slice sl), lane = (head of the group, value).
// Each lane loads the channel partials, row sums and maxima of up to kMergeItems chunks at once,
// then runs CTREE over the 4 channels, the online merge in chunk order and finally ANORM (AT 5.6,
// 5.7). No LDS and no barriers.
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
    if (threadIdx.x < 64u) s_t64[threadIdx.x] = a.ex.t64[threadIdx.x];
    __syncthreads();
    if (i >= hn) return;                                          // whole waves
    const uint32_t first = INL ? p.tok_first[t] : a.tok_first[t];
    const uint32_t cnt = INL ? p.tok_count[t] : a.tok_count[t];
    const uint32_t h = h0 + i;
    float O = 0.0f, l = 0.0f, mr = 0.0f;
    for (uint32_t k0 = 0; k0 < cnt; k0 += kMergeItems) {
        const uint32_t kn = min(kMergeItems, cnt - k0);
        float op[kMergeItems][4], lp[kMergeItems][4];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {                // clamped: every load is issued up front
            const size_t kk = first + k0 + min(k, kn - 1u);
#pragma unroll
            for (uint32_t c = 0; c < 4u; ++c) {
                const size_t slot = (kk * 4u + c) * nh + h;
                op[k][c] = a.OP[slot * D + 64u * sl + L];
                lp[k][c] = a.LP[slot];
            }
        }
        // chunk maxima: lane 8 k + j (k < 4) reads tile j (clamped) of chunk k; MAXOUT over the
        // 8-lane group (an item has at most 8 tiles: NCG <= 128 groups of 16 cells)
        uint32_t key;
        {
            uint32_t tile = 0;
#pragma unroll
            for (uint32_t k = 0; k < kMergeItems; ++k) {            // uniform item reads, per-lane select
                const FaItem itk = fa_item<INL>(a, p, first + k0 + min(k, kn - 1u));
                if ((L >> 3) == k) tile = itk.tile0 + min(L & 7u, itk.ntiles - 1u);
            }
            key = maxt_key_f(a.Mpart[(size_t)tile * nh + h]);
            key = max(key, maxt_key_f(bf(kMFloor)));
            key = umax_u(key, (uint32_t)dpp_i<kDppXor1>((int)key));
            key = umax_u(key, (uint32_t)dpp_i<kDppXor2>((int)key));
            key = umax_u(key, (uint32_t)dpp_i<kDppRowHalfMirror>((int)key));
        }
        float mk[kMergeItems];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) mk[k] = maxt_unkey((uint32_t)__builtin_amdgcn_readlane((int)key, 8 * (int)k));
        // the running maxima and the merge factors of every chunk are independent of O and l:
        // computed first, so the EXP evaluations of the chunks can overlap
        float mrun[kMergeItems], fa[kMergeItems], fbv[kMergeItems];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            const float prev = k == 0u ? mr : mrun[k - 1u];
            const bool first_chunk = k0 + k == 0u;
            mrun[k] = first_chunk ? mk[k] : maxt(prev, mk[k]);
            fa[k] = first_chunk ? 1.0f : expk(smul(ssub(prev, mrun[k]), a.scale), a.ex, s_t64);
            fbv[k] = first_chunk ? 1.0f : expk(smul(ssub(mk[k], mrun[k]), a.scale), a.ex, s_t64);
        }
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            if (k >= kn) break;
            const float ok = ctree4(op[k][0], op[k][1], op[k][2], op[k][3]);
            const float lk = ctree4(lp[k][0], lp[k][1], lp[k][2], lp[k][3]);
            if (k0 + k == 0u) { O = ok; l = lk; }
            else {
                l = sadd(smul(l, fa[k]), smul(lk, fbv[k]));
                O = sadd(smul(O, fa[k]), smul(ok, fbv[k]));
            }
            mr = mrun[k];
        }
    }
    a.out[(size_t)t * a.out_stride + (size_t)h * D + 64u * sl + L] = smul(O, srcp(maxt(l, bf(kLFloor))));
}

}  // namespace tsr

template <bool INL>
static int launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, hipStream_t s) {
    const size_t lds_qk = (size_t)a.G * a.D + 4u * (size_t)a.G * (a.D / 32u) + 4u * 4u * a.G;
    const dim3 gqk(p.n_items * p.maxtiles, a.n_head_kv);
    switch (a.D) {
        case 64: hipLaunchKernelGGL((tsr::k_fa_qk<64, INL>), gqk, dim3(256), lds_qk, s, a, p); break;
        case 128: hipLaunchKernelGGL((tsr::k_fa_qk<128, INL>), gqk, dim3(256), lds_qk, s, a, p); break;
        case 256: hipLaunchKernelGGL((tsr::k_fa_qk<256, INL>), gqk, dim3(256), lds_qk, s, a, p); break;
        case 512: hipLaunchKernelGGL((tsr::k_fa_qk<512, INL>), gqk, dim3(256), lds_qk, s, a, p); break;
        default: return -2;
    }
    if (hipGetLastError() != hipSuccess) return -4;
    // P.V: waves = the most segments of any item (<= 8), LDS = table, segment results, digits
    uint32_t maxn = 0;
    if (INL) {
        for (uint32_t i = 0; i < p.n_items; ++i) maxn = std::max(maxn, p.items[i].n);
    } else {
        maxn = a.max_groups;
    }
    const uint32_t nwv = std::max(1u, std::min(tsr::kPvWaves, ((maxn + 3u) / 4u + 3u) / 4u));
    const size_t lds_pv = 256u + 4u * (size_t)tsr::kPvMaxSeg * 4u * a.D + 4u * tsr::kPvMaxSeg * 4u + 4096u * nwv;
    const dim3 gpv(4u * p.n_items, a.n_head_kv, (a.G + 3u) / 4u);
    switch (a.D) {
        case 64: hipLaunchKernelGGL((tsr::k_fa_pv<64, INL>), gpv, dim3(64u * nwv), lds_pv, s, a, p); break;
        case 128: hipLaunchKernelGGL((tsr::k_fa_pv<128, INL>), gpv, dim3(64u * nwv), lds_pv, s, a, p); break;
        case 256: hipLaunchKernelGGL((tsr::k_fa_pv<256, INL>), gpv, dim3(64u * nwv), lds_pv, s, a, p); break;
        case 512: hipLaunchKernelGGL((tsr::k_fa_pv<512, INL>), gpv, dim3(64u * nwv), lds_pv, s, a, p); break;
        default: return -2;
    }
    if (hipGetLastError() != hipSuccess) return -4;
    const uint32_t ngrp = (a.G + tsr::kMergeHeads - 1u) / tsr::kMergeHeads;
    hipLaunchKernelGGL(tsr::k_fa_merge<INL>, dim3(T, a.n_head_kv * ngrp, a.D / 64u), dim3(256), 0, s, a, p);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, hipStream_t s) {
    return a.items ? launch_fa<false>(a, p, T, s) : launch_fa<true>(a, p, T, s);
}
