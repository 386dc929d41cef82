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

namespace tsr {

constexpr uint32_t kMFloor = 0xF1800000u;   // -2^100 (AT 6.3)
constexpr uint32_t kLFloor = 0x00800000u;   // 2^-126 (AT 5.7)

// EXPK(v, P1) (VU 6.3; sw/sim/tsr_ref_math.c:78-159), constants from the host (ExpkTab).
__device__ __forceinline__ float expk(float v, const ExpkTab & e) {
    const uint32_t u = fb(daz(v));
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return bf(kNaN);
    const bool neg = (u >> 31) != 0u;
    const uint32_t a = u & 0x7FFFFFFFu;
    const float big = neg ? 0.0f : bf(0x7F800000u);
    if (a == 0x7F800000u) return big;
    if (a == 0u) return 1.0f;
    const uint32_t ev = a >> 23;
    if (ev > 156u) return big;
    const uint64_t mv = 0x00800000u | (a & 0x007FFFFFu);
    const uint32_t sh = 156u - ev;
    const uint64_t T = sh >= 64u ? 0u : (mv * e.lk) >> sh;
    if (T >= (1ull << 40)) return big;
    int32_t n;
    uint32_t F;
    if (neg) { n = -(int32_t)((T + 0xFFFFFFFFull) >> 32); F = 0u - (uint32_t)T; }
    else     { n = (int32_t)(T >> 32);                     F = (uint32_t)T; }
    const uint64_t G = F & 0x03FFFFFFu;
    const uint64_t pf = (G * (e.c1 + ((G * (e.c2 + ((G * e.c3) >> 32))) >> 32))) >> 32;
    const uint64_t t = e.t64[F >> 26];
    const uint64_t M = t + ((t * pf) >> 32);
    uint32_t drop = 7u;
    if (M >= (1ull << 31)) { drop = 8u; n += 1; }
    uint64_t sig = M >> drop;
    const uint64_t rem = M & ((1ull << drop) - 1u), half = 1ull << (drop - 1u);
    if (rem > half || (rem == half && (sig & 1u))) sig += 1u;
    if (sig == (1ull << 24)) { sig >>= 1; n += 1; }
    const int32_t be = n + 127;
    if (be >= 255) return bf(0x7F800000u);
    if (be <= 0) return 0.0f;
    return bf(((uint32_t)be << 23) | (uint32_t)(sig & 0x007FFFFFu));
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
__device__ __forceinline__ int32_t bf_int(float w, int32_t es) {
    const uint32_t u = fb(w), e = (u >> 23) & 0xFFu;
    if (e == 0u) return 0;
    const uint32_t m = 0x00800000u | (u & 0x007FFFFFu);
    const int32_t sh = es - ((int32_t)e - 127);
    uint32_t v;
    if (sh <= 0) v = m;
    else if (sh >= 26) v = 0u;
    else {
        v = m >> sh;
        const uint32_t r = m & ((1u << sh) - 1u), h = 1u << (sh - 1);
        v += (r > h || (r == h && (v & 1u))) ? 1u : 0u;
    }
    return (u >> 31) ? -(int32_t)v : (int32_t)v;
}
// RNE24(A) 2^k; below 2^-126 a signed zero, from 2^128 a signed Inf (sw/sim/tsr_ref_at.c:412-436).
__device__ __forceinline__ float bf_f(int64_t A, int32_t k) {
    if (A == 0) return 0.0f;
    const uint32_t s = A < 0 ? 0x80000000u : 0u;
    uint64_t mag = A < 0 ? (uint64_t)0 - (uint64_t)A : (uint64_t)A;
    const int32_t msb = 63 - __builtin_clzll(mag);
    int64_t e = (int64_t)msb + k;
    if (msb > 23) {
        const int32_t sh = msb - 23;
        uint64_t sig = mag >> sh;
        const uint64_t r = mag & ((1ull << sh) - 1u), h = 1ull << (sh - 1);
        if (r > h || (r == h && (sig & 1u))) sig += 1u;
        if (sig >> 24) { sig >>= 1; e += 1; }
        mag = sig;
    } else {
        mag <<= (23 - msb);
    }
    if (e < -126) return bf(s);
    if (e > 127) return bf(s | 0x7F800000u);
    return bf(s | ((uint32_t)(e + 127) << 23) | ((uint32_t)mag & 0x007FFFFFu));
}

// ---------------------------------------------------------------------------------------------
// scores: block (tile, KV head g), thread = one cell of the tile. The block quantizes the query
// values of the KV head's G heads (QACT A32: its 32-blocks never cross a head, so they are the
// blocks of the whole query row) while the K rows of its cells load.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ FaItem fa_item(const FaArgs & a, const FaPlan & p, uint32_t i) {
    return a.items ? a.items[i] : p.items[i];
}

template <int D>
__global__ __launch_bounds__(256) void k_fa_qk(FaArgs a, FaPlan p) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t NBD = D / 32u;                             // blocks per head
    constexpr bool KREG = D <= 128;                                // K row of the cell kept in registers
    const uint32_t tt = blockIdx.x % p.maxtiles;
    const FaItem it = fa_item(a, p, blockIdx.x / p.maxtiles);
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

    int4 kr[KREG ? 2 * NBD : 1];
    uint32_t km[NBD];
#pragma unroll
    for (uint32_t kb = 0; kb < NBD; ++kb) km[kb] = kmeta[kb];
    if constexpr (KREG) {
#pragma unroll
        for (uint32_t c = 0; c < 2 * NBD; ++c) kr[c] = *(const int4 *)(kq + (size_t)(ci0 + c) * 256u);
    }
    __builtin_amdgcn_sched_barrier(0);

    const float * qrow = a.q + (size_t)it.t * a.q_stride + (size_t)g * G * D;
    for (uint32_t slot = threadIdx.x; slot < G * D / 4u; slot += blockDim.x) {   // 8 lanes per 32-block
        float Dq;
        const uint32_t qv = qact_a32_lane(*(const float4 *)(qrow + 4u * slot), &Dq);
        *(uint32_t *)(s_q + 4u * slot) = qv;
        if ((lane & 7) == 0) s_dx[slot >> 3] = Dq;
    }
    __syncthreads();

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
// P.V and the merge: block (item * 4 + channel c, KV head g, slice sl), 16 waves.
// A unit is (segment, head): lane = cell for EXP, the block-float weights and LSUM, then lane =
// value of the 64-value slice for the exact sum A = sum W q on v_dot4 over the base-256 digits.
// The per-segment results go to LDS; the f32 segment chain then runs in segment order.
// ---------------------------------------------------------------------------------------------
constexpr int kHB = 16;                                           // heads per LDS batch
constexpr int kMaxSeg = 8;                                        // NCG <= 128 -> <= 32 groups per channel

__device__ __forceinline__ float ctree4(float x0, float x1, float x2, float x3) { return sadd(sadd(x0, x1), sadd(x2, x3)); }

__global__ __launch_bounds__(1024) void k_fa_pv(FaArgs a, FaPlan p) {
    __shared__ __align__(16) int8_t s_dig[16][2][4][64];          // wave, block e, digit, cell
    __shared__ float s_c[kMaxSeg][kHB][64];
    __shared__ float s_l[kMaxSeg][kHB];
    __shared__ float s_m[64];
    __shared__ uint32_t s_mkey[64];
    const uint32_t item = blockIdx.x >> 2, c = blockIdx.x & 3u, g = blockIdx.y, sl = blockIdx.z;
    const FaItem it = fa_item(a, p, item);
    const uint32_t G = a.G, D = a.D, E = a.E, n16 = 16u * it.n, nbk = E / 32u, nh = a.n_head, nsl = D / 64u;
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t u_first = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u);
    const uint32_t u_end = it.u0 + it.n;
    const uint32_t nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
    const uint32_t nseg = (nu + 3u) / 4u;
    const uint32_t sa = g * nsl + sl;                             // slice of the cell row
    const uint32_t d = 64u * sa + (uint32_t)lane;                 // this lane's value in the cell row
    const int e_l = lane >> 5;
    const float * S = a.S + (size_t)it.s_off * nh;
    const uint16_t * vmeta = (const uint16_t *)a.vc.base;
    const uint8_t * vq = a.vc.base + a.vc.quant_off;

    // chunk maxima (MAXOUT over the tiles; MAXT is a total order, so the order of the folds is free)
    for (uint32_t i = threadIdx.x; i < G; i += blockDim.x) s_mkey[i] = maxt_key_f(bf(kMFloor));
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < G * it.ntiles; idx += blockDim.x)   // one load per thread
        atomicMax(&s_mkey[idx % G], maxt_key_f(a.Mpart[(size_t)(it.tile0 + idx / G) * nh + g * G + idx % G]));
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < G; i += blockDim.x) s_m[i] = maxt_unkey(s_mkey[i]);
    __syncthreads();

    for (uint32_t hb0 = 0; hb0 < G; hb0 += kHB) {
        const uint32_t hbn = min((uint32_t)kHB, G - hb0), units = nseg * hbn;
        for (uint32_t unit = (uint32_t)wave; unit < units; unit += (uint32_t)nw) {
            const uint32_t seg = unit / hbn, hi = unit % hbn, h = g * G + hb0 + hi;
            const float m = s_m[hb0 + hi];
            const uint32_t ngr = min(nu - 4u * seg, 4u);
            // loads first: V quants of the slice (lane = value) and, lane = cell, score and V scales
            int4 vqd[4];
#pragma unroll
            for (uint32_t gi = 0; gi < 4; ++gi) {
                const uint32_t ug = u_first + 4u * (4u * seg + min(gi, ngr - 1u));
                vqd[gi] = *(const int4 *)(vq + (size_t)ug * 16u * E + (size_t)d * 16u);
            }
            const uint32_t grp = 4u * seg + ((uint32_t)lane >> 4);
            const bool cv = grp < nu;
            const uint32_t u = u_first + 4u * min(grp, nu - 1u), rr = (uint32_t)lane & 15u;
            const float sv = S[(size_t)h * n16 + 16u * (u - it.u0) + rr];
            const uint32_t mv = *(const uint32_t *)(vmeta + ((size_t)u * 16u + rr) * nbk + 2u * sa);
            // --- lane = cell k of the segment ---------------------------------------------
            const float p = cv ? expk(smul(ssub(sv, m), a.scale), a.ex) : 0.0f;
            const float pz = daz(p);
            const bool live = cv && (fb(pz) & 0x7FFFFFFFu) != 0u;
            const float w0 = live ? smul(p, h2f_exact(mv & 0xFFFFu)) : 0.0f;
            const float w1 = live ? smul(p, h2f_exact(mv >> 16)) : 0.0f;
            const bool nf0 = (fb(w0) & 0x7F800000u) == 0x7F800000u;
            const bool nf1 = (fb(w1) & 0x7F800000u) == 0x7F800000u;
            const bool bad0 = __ballot(nf0) != 0ull, bad1 = __ballot(nf1) != 0ull;
            int ex = -1000;
            if (!nf0 && (fb(w0) & 0x7FFFFFFFu)) ex = (int)((fb(w0) >> 23) & 0xFFu) - 127;
            if (!nf1 && (fb(w1) & 0x7FFFFFFFu)) ex = max(ex, (int)((fb(w1) >> 23) & 0xFFu) - 127);
            const int es = wave_max_i(ex);
            const bool any = es > -1000;
            const int32_t W0 = (any && !bad0) ? bf_int(w0, es) : 0;
            const int32_t W1 = (any && !bad1) ? bf_int(w1, es) : 0;
            int32_t r0 = W0, r1 = W1;                               // balanced base-256 digits
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int32_t d0 = ((r0 + 128) & 255) - 128, d1 = ((r1 + 128) & 255) - 128;
                s_dig[wave][0][k][lane] = (int8_t)d0;
                s_dig[wave][1][k][lane] = (int8_t)d1;
                r0 = (r0 - d0) >> 8;
                r1 = (r1 - d1) >> 8;
            }
            // LSUM of the segment (AT 6.5): block float of its p values
            const bool pnf = cv && (fb(pz) & 0x7F800000u) == 0x7F800000u;
            const bool badl = __ballot(pnf) != 0ull;
            int ep = -1000;
            if (cv && !pnf && (fb(pz) & 0x7FFFFFFFu)) ep = (int)((fb(pz) >> 23) & 0xFFu) - 127;
            ep = wave_max_i(ep);
            float ls;
            if (badl) ls = bf(kNaN);
            else if (ep == -1000) ls = 0.0f;
            else ls = bf_f((int64_t)wave_sum_i((cv && !pnf) ? bf_int(pz, ep) : 0), ep - 23);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // --- lane = value of the slice ------------------------------------------------
            int32_t sk[4] = { 0, 0, 0, 0 };
#pragma unroll
            for (uint32_t gi = 0; gi < 4; ++gi) {
                if (gi < ngr) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int4 dg = *(const int4 *)&s_dig[wave][e_l][k][16u * gi];
                        int acc = sk[k];
                        acc = dot4(dg.x, vqd[gi].x, acc);
                        acc = dot4(dg.y, vqd[gi].y, acc);
                        acc = dot4(dg.z, vqd[gi].z, acc);
                        acc = dot4(dg.w, vqd[gi].w, acc);
                        sk[k] = acc;
                    }
                }
            }
            const int64_t A = (int64_t)sk[0] + ((int64_t)sk[1] << 8) + ((int64_t)sk[2] << 16) + ((int64_t)sk[3] << 24);
            const bool badv = e_l ? bad1 : bad0;
            s_c[seg][hi][lane] = badv ? bf(kNaN) : (any ? bf_f(A, es - 23) : 0.0f);
            if (lane == 0) s_l[seg][hi] = ls;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        __syncthreads();
        for (uint32_t idx = threadIdx.x; idx < hbn * 64u; idx += blockDim.x) {   // segment chains in order
            const uint32_t hi = idx >> 6, L = idx & 63u, h = g * G + hb0 + hi;
            float O = 0.0f;
            for (uint32_t seg = 0; seg < nseg; ++seg) O = sadd(O, s_c[seg][hi][L]);
            const size_t slot = ((size_t)item * 4u + c) * nh + h;
            a.OP[slot * D + 64u * sl + L] = O;
            if (L == 0u) {
                float l = 0.0f;
                for (uint32_t seg = 0; seg < nseg; ++seg) l = sadd(l, s_l[seg][hi]);
                a.LP[slot * nsl + sl] = l;
            }
        }
        __syncthreads();
    }

    if (c == 0u && sl == 0u)                                      // chunk maxima for the merge
        for (uint32_t i = threadIdx.x; i < G; i += blockDim.x) a.MK[(size_t)item * nh + g * G + i] = s_m[i];
}

// ---------------------------------------------------------------------------------------------
// merge: block (token, KV head g x group of 4 heads, slice sl), lane = (head of the group, value).
// Each lane loads the channel partials, row sums and maxima of up to kMergeItems chunks at once,
// then runs CTREE over the 4 channels, the online merge in chunk order and finally ANORM (AT 5.6,
// 5.7). No LDS and no barriers.
// ---------------------------------------------------------------------------------------------
constexpr uint32_t kMergeItems = 8;                              // chunks loaded per round
constexpr uint32_t kMergeHeads = 4;                              // heads per block

__global__ __launch_bounds__(256) void k_fa_merge(FaArgs a, FaPlan p) {
    const uint32_t G = a.G, D = a.D, nh = a.n_head, nsl = D / 64u;
    const uint32_t ngrp = (G + kMergeHeads - 1u) / kMergeHeads;
    const uint32_t t = blockIdx.x, g = blockIdx.y / ngrp, h0 = g * G + (blockIdx.y % ngrp) * kMergeHeads;
    const uint32_t hn = min(kMergeHeads, g * G + G - h0), sl = blockIdx.z;
    const uint32_t i = threadIdx.x >> 6, L = threadIdx.x & 63u;
    if (i >= hn) return;                                          // whole waves
    const uint32_t first = a.tok_first ? a.tok_first[t] : p.tok_first[t];
    const uint32_t cnt = a.tok_count ? a.tok_count[t] : p.tok_count[t];
    const uint32_t h = h0 + i;
    float O = 0.0f, l = 0.0f, mr = 0.0f;
    for (uint32_t k0 = 0; k0 < cnt; k0 += kMergeItems) {
        const uint32_t kn = min(kMergeItems, cnt - k0);
        float op[kMergeItems][4], lp[kMergeItems][4], mk[kMergeItems];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {                // clamped: every load is issued up front
            const size_t kk = first + k0 + min(k, kn - 1u);
#pragma unroll
            for (uint32_t c = 0; c < 4u; ++c) {
                const size_t slot = (kk * 4u + c) * nh + h;
                op[k][c] = a.OP[slot * D + 64u * sl + L];
                lp[k][c] = a.LP[slot * nsl + sl];
            }
            mk[k] = a.MK[kk * nh + h];
        }
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k) {
            if (k >= kn) break;
            const float ok = ctree4(op[k][0], op[k][1], op[k][2], op[k][3]);
            const float lk = ctree4(lp[k][0], lp[k][1], lp[k][2], lp[k][3]);
            if (k0 + k == 0u) { O = ok; l = lk; mr = mk[k]; }
            else {
                const float mn = maxt(mr, mk[k]);
                const float fa = expk(smul(ssub(mr, mn), a.scale), a.ex);
                const float fbv = expk(smul(ssub(mk[k], mn), a.scale), a.ex);
                l = sadd(smul(l, fa), smul(lk, fbv));
                O = sadd(smul(O, fa), smul(ok, fbv));
                mr = mn;
            }
        }
    }
    a.out[(size_t)t * a.out_stride + (size_t)h * D + 64u * sl + L] = smul(O, srcp(maxt(l, bf(kLFloor))));
}

}  // namespace tsr

int tsr_launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, hipStream_t s) {
    const size_t lds_qk = (size_t)a.G * a.D + 4u * (size_t)a.G * (a.D / 32u) + 4u * 4u * a.G;
    const dim3 gqk(p.n_items * p.maxtiles, a.n_head_kv);
    switch (a.D) {
        case 64: hipLaunchKernelGGL(tsr::k_fa_qk<64>, gqk, dim3(256), lds_qk, s, a, p); break;
        case 128: hipLaunchKernelGGL(tsr::k_fa_qk<128>, gqk, dim3(256), lds_qk, s, a, p); break;
        case 256: hipLaunchKernelGGL(tsr::k_fa_qk<256>, gqk, dim3(256), lds_qk, s, a, p); break;
        case 512: hipLaunchKernelGGL(tsr::k_fa_qk<512>, gqk, dim3(256), lds_qk, s, a, p); break;
        default: return -2;
    }
    if (hipGetLastError() != hipSuccess) return -4;
    hipLaunchKernelGGL(tsr::k_fa_pv, dim3(4u * p.n_items, a.n_head_kv, a.D / 64u), dim3(1024), 0, s, a, p);
    if (hipGetLastError() != hipSuccess) return -4;
    const uint32_t ngrp = (a.G + tsr::kMergeHeads - 1u) / tsr::kMergeHeads;
    hipLaunchKernelGGL(tsr::k_fa_merge, dim3(T, a.n_head_kv * ngrp, a.D / 64u), dim3(256), 0, s, a, p);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
