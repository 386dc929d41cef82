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
//   k_fa_qk     scores of a 256-cell tile of one chunk for the query heads of one KV head, and the
//               tile's maxima (MAXT is an order-free total-order maximum)
//   k_fa_pv     one (chunk, channel, KV head, 64-value slice): EXP, block float per segment, the
//               f32 segment sums in segment order, the segment row-sums (LSUM)
//   k_fa_merge  one (token, head): CTREE of the channels, the online merge in chunk order, ANORM
//
// Block float (AT 6.4; sw/sim/tsr_ref_at.c:380-488): in a segment every weight w = p dV is scaled
// to an integer W = RNE(w 2^(23 - E_S)) (|W| <= 2^24) and A = sum W q is exact. W is split into four
// balanced base-256 digits d_k in [-128, 127] (W = sum d_k 256^k), so A = sum_k 256^k (sum d_k q)
// runs on v_dot4_i32_i8 with exact int32 partial sums (|sum| <= 64 * 128 * 128).
#include "kernels.hpp"
#include "tsr_dev.hpp"

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
__device__ __forceinline__ float wave_maxt(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = maxt(v, shfl_f(v, (int)__lane_id() ^ off));
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) { const int o = shfl_i(v, (int)__lane_id() ^ off); v = o > v ? o : v; }
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += shfl_i(v, (int)__lane_id() ^ off);
    return v;
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
// scores: block (tile, KV head g); thread = one cell of the tile
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_fa_qk(FaArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const FaTile tl = a.tiles[blockIdx.x];
    const FaItem it = a.items[tl.item];
    const uint32_t g = blockIdx.y, G = a.G, D = a.D, nbd = D / 32u;
    int8_t * s_q = (int8_t *)lds;                                 // G*D quants of the KV head's query heads
    float * s_dx = (float *)(lds + G * D);                        // G*D/32 scales
    float * s_red = s_dx + G * nbd;                               // 4 waves x G maxima
    const uint8_t * qa = a.qa + (size_t)it.t * a.qa_bytes;
    for (uint32_t i = threadIdx.x; i < G * D / 16u; i += blockDim.x)
        ((uint4 *)s_q)[i] = ((const uint4 *)(qa + (size_t)g * G * D))[i];
    for (uint32_t i = threadIdx.x; i < G * nbd; i += blockDim.x)
        s_dx[i] = ((const float *)(qa + a.qa_d_off))[(size_t)g * G * nbd + i];
    __syncthreads();

    const uint32_t n16 = 16u * it.n, j = tl.c0 + threadIdx.x;
    const bool in = j < n16;
    const uint32_t cell = 16u * it.u0 + j, u = cell >> 4, rr = cell & 15u;
    const bool vis = in && (it.general || (j >= it.c_lo && j < it.c_hi));
    const uint32_t E = a.E, nbk = E / 32u;
    const uint16_t * kmeta = (const uint16_t *)a.kc.base + ((size_t)u * 16u + rr) * nbk + (size_t)g * nbd;
    const uint8_t * kq = a.kc.base + a.kc.quant_off + (size_t)u * 16u * E + (size_t)rr * 16u;
    float * S = a.S + (size_t)it.s_off * a.n_head;
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6);
    for (uint32_t i = 0; i < G; ++i) {
        const uint32_t h = g * G + i;
        float s = bf(kNegInf);
        if (vis) {
            float p[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) p[k] = 0.0f;
            for (uint32_t kb = 0; kb < nbd; ++kb) {
                const uint32_t ci = (g * D + 32u * kb) >> 4;      // first 16-byte chunk of the block
                const int4 w0 = *(const int4 *)(kq + (size_t)ci * 256u);
                const int4 w1 = *(const int4 *)(kq + (size_t)(ci + 1u) * 256u);
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
                const float t = (h2f_fast(kmeta[kb]) * s_dx[i * nbd + kb]) * (float)is;
                p[kb] = 0.0f + t;
            }
            // tree16 of the segment's partials (k >= D/32 stay +0)
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
        float mx = wave_maxt(in ? s : bf(kMFloor));
        if (lane == 0) s_red[wave * G + i] = mx;
    }
    __syncthreads();
    if (threadIdx.x < G) {
        float m = s_red[threadIdx.x];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = maxt(m, s_red[w * G + threadIdx.x]);
        a.Mpart[(size_t)blockIdx.x * a.n_head + g * G + threadIdx.x] = m;
    }
}

// ---------------------------------------------------------------------------------------------
// P.V: block (item * 4 + channel, KV head g, slice); wave = one query head at a time
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_fa_pv(FaArgs a) {
    __shared__ __align__(16) int8_t s_dig[4][2][4][64];           // wave, block e, digit, cell
    const uint32_t item = blockIdx.x >> 2, c = blockIdx.x & 3u, g = blockIdx.y, sl = blockIdx.z;
    const FaItem it = a.items[item];
    const uint32_t G = a.G, D = a.D, E = a.E, n16 = 16u * it.n, nbk = E / 32u;
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t u_first = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u);
    const uint32_t u_end = it.u0 + it.n;
    const uint32_t nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
    const uint32_t nseg = (nu + 3u) / 4u;
    const uint32_t sa = g * (D / 64u) + sl;                       // slice of the cell row
    const uint32_t d = 64u * sa + (uint32_t)lane;                 // this lane's value in the cell row
    const int e_l = lane >> 5;
    const float * S = a.S + (size_t)it.s_off * a.n_head;
    const uint16_t * vmeta = (const uint16_t *)a.vc.base;
    const uint8_t * vq = a.vc.base + a.vc.quant_off;

    for (uint32_t i = (uint32_t)wave; i < G; i += (uint32_t)nw) {
        const uint32_t h = g * G + i;
        float m = bf(kMFloor);
        for (uint32_t tt = 0; tt < it.ntiles; ++tt) m = maxt(m, a.Mpart[(size_t)(it.tile0 + tt) * a.n_head + h]);
        if (c == 0u && sl == 0u && lane == 0) a.MK[(size_t)item * a.n_head + h] = m;
        float O = 0.0f, l = 0.0f;
        for (uint32_t sg = 0; sg < nseg; ++sg) {
            // --- lane = cell k of the segment -----------------------------------------------
            const uint32_t grp = 4u * sg + ((uint32_t)lane >> 4);
            const bool cv = grp < nu;
            const uint32_t u = u_first + 4u * grp, rr = (uint32_t)lane & 15u;
            float p = 0.0f;
            if (cv) p = expk(smul(ssub(S[(size_t)h * n16 + 16u * (u - it.u0) + rr], m), a.scale), a.ex);
            const float pz = daz(p);
            const bool live = cv && (fb(pz) & 0x7FFFFFFFu) != 0u;
            float w0 = 0.0f, w1 = 0.0f;
            if (live) {
                const uint16_t * mv = vmeta + ((size_t)u * 16u + rr) * nbk + 2u * sa;
                w0 = smul(p, h2f_exact(mv[0]));
                w1 = smul(p, h2f_exact(mv[1]));
            }
            const bool nf0 = live && (fb(w0) & 0x7F800000u) == 0x7F800000u;
            const bool nf1 = live && (fb(w1) & 0x7F800000u) == 0x7F800000u;
            const bool bad0 = __any(nf0), bad1 = __any(nf1);
            int ex = -1000;
            if (live && !nf0 && (fb(w0) & 0x7FFFFFFFu)) ex = (int)((fb(w0) >> 23) & 0xFFu) - 127;
            if (live && !nf1 && (fb(w1) & 0x7FFFFFFFu)) { const int e1 = (int)((fb(w1) >> 23) & 0xFFu) - 127; ex = e1 > ex ? e1 : ex; }
            const int es = wave_max_i(ex);
            const bool any = es > -1000;
            int32_t W0 = 0, W1 = 0;
            if (any && live) {
                if (!bad0 && !nf0) W0 = bf_int(w0, es);
                if (!bad1 && !nf1) W1 = bf_int(w1, es);
            }
            // balanced base-256 digits of W0, W1 -> LDS
            int32_t r0 = W0, r1 = W1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int32_t d0 = ((r0 + 128) & 255) - 128, d1 = ((r1 + 128) & 255) - 128;
                s_dig[wave][0][k][lane] = (int8_t)d0;
                s_dig[wave][1][k][lane] = (int8_t)d1;
                r0 = (r0 - d0) >> 8;
                r1 = (r1 - d1) >> 8;
            }
            if (sl == 0u) {                                        // LSUM of the segment (AT 6.5)
                const bool pnf = cv && (fb(pz) & 0x7F800000u) == 0x7F800000u;
                const bool badl = __any(pnf);
                int ep = -1000;
                if (cv && !pnf && (fb(pz) & 0x7FFFFFFFu)) ep = (int)((fb(pz) >> 23) & 0xFFu) - 127;
                ep = wave_max_i(ep);
                float ls;
                if (badl) ls = bf(kNaN);
                else if (ep == -1000) ls = 0.0f;
                else ls = bf_f((int64_t)wave_sum_i(cv ? bf_int(pz, ep) : 0), ep - 23);
                l = sadd(l, ls);
            }
            __builtin_amdgcn_wave_barrier();
            // --- lane = value d of the slice ------------------------------------------------
            int32_t sk[4] = { 0, 0, 0, 0 };
            const uint32_t ng = nu - 4u * sg < 4u ? nu - 4u * sg : 4u;
            for (uint32_t gi = 0; gi < ng; ++gi) {
                const uint32_t ug = u_first + 4u * (4u * sg + gi);
                const int4 q = *(const int4 *)(vq + (size_t)ug * 16u * E + (size_t)d * 16u);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int4 dg = *(const int4 *)&s_dig[wave][e_l][k][16u * gi];
                    int acc = sk[k];
                    acc = dot4(dg.x, q.x, acc);
                    acc = dot4(dg.y, q.y, acc);
                    acc = dot4(dg.z, q.z, acc);
                    acc = dot4(dg.w, q.w, acc);
                    sk[k] = acc;
                }
            }
            const int64_t A = (int64_t)sk[0] + ((int64_t)sk[1] << 8) + ((int64_t)sk[2] << 16) + ((int64_t)sk[3] << 24);
            const bool badl2 = e_l ? bad1 : bad0;
            const float cval = badl2 ? bf(kNaN) : (any ? bf_f(A, es - 23) : 0.0f);
            O = sadd(O, cval);
            __builtin_amdgcn_wave_barrier();
        }
        const size_t slot = ((size_t)item * 4u + c) * a.n_head + h;
        a.OP[slot * D + 64u * sl + (uint32_t)lane] = O;
        if (sl == 0u && lane == 0) a.LP[slot] = l;
    }
}

// ---------------------------------------------------------------------------------------------
// merge: block (token, head); threads over D
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float ctree4(float x0, float x1, float x2, float x3) { return sadd(sadd(x0, x1), sadd(x2, x3)); }

__global__ __launch_bounds__(256) void k_fa_merge(FaArgs a) {
    const uint32_t t = blockIdx.x, h = blockIdx.y, D = a.D, nh = a.n_head;
    const uint32_t first = a.tok_first[t], cnt = a.tok_count[t];
    float O[2] = { 0.0f, 0.0f };
    float l = 0.0f, m = 0.0f;
    for (uint32_t k = 0; k < cnt; ++k) {
        const uint32_t item = first + k;
        const size_t s0 = (size_t)item * 4u * nh + h;
        const float lk = ctree4(a.LP[s0], a.LP[s0 + nh], a.LP[s0 + 2u * nh], a.LP[s0 + 3u * nh]);
        const float mk = a.MK[(size_t)item * nh + h];
        float fa = 0.0f, fb_ = 0.0f;
        if (k == 0u) { l = lk; m = mk; }
        else {
            const float mn = maxt(m, mk);
            fa = expk(smul(ssub(m, mn), a.scale), a.ex);
            fb_ = expk(smul(ssub(mk, mn), a.scale), a.ex);
            l = sadd(smul(l, fa), smul(lk, fb_));
            m = mn;
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t dd = threadIdx.x + 256u * (uint32_t)r;
            if (dd < D) {
                const float ok = ctree4(a.OP[s0 * D + dd], a.OP[(s0 + nh) * D + dd], a.OP[(s0 + 2u * nh) * D + dd],
                                        a.OP[(s0 + 3u * nh) * D + dd]);
                O[r] = k == 0u ? ok : sadd(smul(O[r], fa), smul(ok, fb_));
            }
        }
    }
    const float rinv = srcp(maxt(l, bf(kLFloor)));
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t dd = threadIdx.x + 256u * (uint32_t)r;
        if (dd < D) a.out[(size_t)t * a.out_stride + (size_t)h * D + dd] = smul(O[r], rinv);
    }
}

}  // namespace tsr

int tsr_launch_fa(const tsr::FaArgs & a, uint32_t n_tiles, uint32_t n_items, uint32_t T, hipStream_t s) {
    const size_t lds_qk = (size_t)a.G * a.D + 4u * (size_t)a.G * (a.D / 32u) + 4u * 4u * a.G;
    hipLaunchKernelGGL(tsr::k_fa_qk, dim3(n_tiles, a.n_head_kv), dim3(256), lds_qk, s, a);
    if (hipGetLastError() != hipSuccess) return -4;
    hipLaunchKernelGGL(tsr::k_fa_pv, dim3(4u * n_items, a.n_head_kv, a.D / 64u), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return -4;
    hipLaunchKernelGGL(tsr::k_fa_merge, dim3(T, a.n_head), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
