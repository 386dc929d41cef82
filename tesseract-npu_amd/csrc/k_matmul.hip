// k_matmul.hip -- prefill MUL_MAT (T >= 16 tokens) for Q8_0 weights on the int8 matrix cores.
//
// Numerics (sw/sim/tsr_ref.c:525-635): y[t][n] is the 16-partial tree of the terms
// (d[n][b] Dx[t][b]) f32(isum[t][n][b]), term b going to partial b mod 16 in order of b; the
// activation is quantized by QACT A32 first (k_qact_mm, into scratch, block-major: the quants
// [block][token][32 B] and the scales [block][token], so that a wave's operand load of 32 tokens
// is 1 KiB of consecutive bytes).
//
// Per 32-value block b and 32 x 32 tile (weight rows x tokens):
//   isum = v_mfma_i32_32x32x32_i8(W rows, X tokens): one block of K is exactly one instruction,
//          so the integer block sums come out of the matrix core exactly;
//   P    = v_mfma_f32_32x32x2_f32 with the second k column zero: the outer product d[n] Dx[t] in
//          the same lane layout, each element the IEEE product of the two (the matrix core rounds
//          a single product like v_mul_f32; the sign of an exact zero may differ, which cannot
//          change a sum that starts at +0);
//   p += P f32(isum)   (three VALU operations per output).
// Dx is an fp16 value and d an fp16 value, so no product or sum is ever subnormal and plain IEEE
// operations are the spec operations; NaN is canonicalized when y is stored.
//
// Work split. A workgroup of 16 waves computes one 32 x 32 tile; wave j computes partial p_j
// (blocks b = j, j + 16, ... in order: consecutive slots of the weight layout, wlayout.hpp). A wave
// requests block k + 1 once the matrix core has read block k's operands, and two workgroups share a
// compute unit (at most 64 VGPRs), so that one's loads overlap the other's VALU work: the three VALU
// operations per output are the bound. The loads are raw buffer loads (a 32-bit lane offset set up
// once, the block step in a scalar offset where it is uniform), so that the loop has no 64-bit
// address arithmetic. The 16 partials meet in LDS and one thread per output adds the tree
// ((p0 + p1) + (p2 + p3)) + ...
//
// Lane layouts (gfx950): an operand lane l supplies row l % 32 of its matrix and k = 16 (l / 32) ..
// 16 (l / 32) + 15; the result lane l holds column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4,
// r = 0..15.
#include "expk.hpp"
#include "kernels.hpp"
#include "qact.hpp"
#include "wlayout.hpp"

namespace tsr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Raw buffer loads over a window of bytes: 32-bit offsets (a vector part and a scalar part), and
// a load at or past the window's end returns 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t brsrc(const void * p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ float bloadf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}


// QACT A32 of T token rows into the block-major layout: 8 lanes per (token, block), 4 values each
// (qact_a32_lane: the spec rule, as for the QA image of k_qact). Pairs run token-fastest: a wave's 8
// pairs read one 128-byte line of x each and write 256 contiguous bytes of quants (block-fastest
// pairs wrote 32 bytes 16 KiB apart). The host keeps T (K / 32) below 2^32.
__global__ __launch_bounds__(256) void k_qact_mm(const float * x, uint64_t x_stride, uint32_t K, uint32_t T,
                                                 uint8_t * xq, float * xd) {
    const uint32_t nb = K >> 5;
    const uint32_t pair = (blockIdx.x * blockDim.x + threadIdx.x) >> 3;   // (block, token)
    const uint32_t l8 = threadIdx.x & 7u;
    const uint32_t npair = T * nb;
    const uint32_t pc = pair < npair ? pair : npair - 1u;         // clamped: whole 8-lane groups stay active
    const uint32_t b = pc / T, t = pc - b * T;
    float D;
    const uint32_t q = qact_a32_lane(*(const float4 *)(x + (size_t)t * x_stride + 32u * b + 4u * l8), &D);
    if (pair < npair) {
        *(uint32_t *)(xq + ((size_t)b * T + t) * 32u + 4u * l8) = q;
        if (l8 == 0u) xd[(size_t)b * T + t] = D;
    }
}

// The tile (row tile tx, token tile ty) of a workgroup. Workgroups are dispatched to the XCDs in
// turn (linear workgroup i on XCD i mod 8). The plain grid (gx, gy) runs the row tiles of one token
// tile together: an XCD's share of a weight of up to ~2 MB stays in its 4 MB L2 from one token tile
// to the next. The grouped grid (8 gy, gx / 8), for larger weights, gives row tile tx to XCD tx mod 8
// and its token tiles to that XCD one after another, so that the weight tile is read from memory once
// and then from the L2 by the token tiles running beside it.
__device__ __forceinline__ void mm_tile(bool grouped, uint32_t & tx, uint32_t & ty) {
    if (grouped) {
        tx = (blockIdx.x & 7u) + 8u * blockIdx.y;
        ty = blockIdx.x >> 3;
    } else {
        tx = blockIdx.x;
        ty = blockIdx.y;
    }
}

__global__ __launch_bounds__(1024, 8) void k_mm_q80(MmArgs a) {
    __shared__ float s_p[16][1024];                                // partial j of output (lane, r)
    const WGeom g = wgeom(a.N, a.K >> 5, a.rb, false);
    const uint32_t lane = __lane_id(), j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t tx, ty;
    mm_tile(a.grouped != 0u, tx, ty);
    const uint32_t n0 = tx * 32u, t0 = ty * 32u;
    const uint32_t h = lane >> 5, c = lane & 31u;
    // operand rows of this lane (clamped: rows / tokens beyond the matrix are not stored)
    const uint32_t n = min(n0 + c, a.N - 1u), t = min(t0 + c, a.T - 1u);
    const uint32_t B = n / g.rb, R = wl_rows(g, B), rr = n - B * g.rb;  // row block of the row
    // buffer windows: the row blocks of the workgroup's rows (the host checks that they span less
    // than 2^31 bytes), the activation scratch; a load at offset >= 2^31 reads 0 (the k = 1 column
    // of the scale product)
    const uint32_t B0 = n0 / g.rb, B1 = (min(n0 + 31u, a.N - 1u)) / g.rb;
    const uint64_t wbase = (uint64_t)B0 * g.bstride;
    const uint64_t wend = B1 + 1u < g.nblk ? (uint64_t)(B1 + 1u) * g.bstride : wl_bytes(g);
    const __amdgpu_buffer_rsrc_t rw = brsrc(a.w + wbase, (uint32_t)(wend - wbase));
    const __amdgpu_buffer_rsrc_t rx = brsrc(a.qa, a.d_off + 4u * a.T * g.nb);
    const uint32_t cnt = wl_count(g, j), sl0 = wl_slot(g, j, 0u);
    uint32_t ow = (uint32_t)(wl_quant_off(g, B, R, h, sl0, rr) - wbase);   // + 16 R per slot
    uint32_t om = h ? 0x80000000u : (uint32_t)(wl_meta_off(g, B, R, sl0, rr) - wbase);   // + 2 R
    const uint32_t sw = 16u * R, sm = 2u * R;
    const uint32_t ox = 32u * t + 16u * h, od = h ? 0x80000000u : a.d_off + 4u * t;
    const uint32_t sx = 512u * a.T, sd = 64u * a.T;                // per block of the wave (b += 16)
    uint32_t bx = 32u * a.T * j, bd = 4u * a.T * j;                // scalar: block b = j + 16 k

    v16f p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = 0.0f;
    // one block ahead: the next block's loads are issued once the matrix core has read this one's.
    // Every load is of a block the wave owns (k < cnt; the window's range check covers the vector
    // offset, which is how the k = 1 lanes read 0, and is not relied on for the scalar offset).
    v4i wa = {}, xb = {};
    uint32_t dwh = 0u;
    float dx = 0.0f;
    if (cnt > 0u) {
        wa = bload128(rw, ow, 0u);
        xb = bload128(rx, ox, bx);
        dwh = bload16(rw, om, 0u);
        dx = bloadf(rx, od, bd);
    }
    for (uint32_t k = 0; k < cnt; ++k) {
        v16i is = {};
        is = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, xb, is, 0, 0, 0);
        v16f P = {};
        P = __builtin_amdgcn_mfma_f32_32x32x2f32(h2f_fast(dwh), dx, P, 0, 0, 0);
        if (k + 1u < cnt) {                                        // wave-uniform
            ow += sw;
            om += sm;
            bx += sx;
            bd += sd;
            wa = bload128(rw, ow, 0u);
            xb = bload128(rx, ox, bx);
            dwh = bload16(rw, om, 0u);
            dx = bloadf(rx, od, bd);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = p[r] + P[r] * (float)is[r];
    }
    // the lane index again (not kept in a register through the loop)
    uint32_t ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
    for (int r = 0; r < 4; ++r)
        *(float4 *)&s_p[j][16u * ln + 4u * (uint32_t)r] = make_float4(p[4 * r], p[4 * r + 1], p[4 * r + 2], p[4 * r + 3]);
    lds_barrier();

    // one thread per output: o = 16 lane' + r of the wave layout above
    const uint32_t o = 64u * j + ln, ol = o >> 4, r = o & 15u;
    const uint32_t tt = t0 + (ol & 31u), nn = n0 + 8u * (r >> 2) + 4u * (ol >> 5) + (r & 3u);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = s_p[i][o];
#pragma unroll
    for (int w = 16; w > 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
    if (tt < a.T && nn < a.N) {
        float y = canon(v[0]);
        float * yp = a.y + (size_t)tt * a.y_stride + nn;
        if (a.add) y = sadd(a.add[(size_t)tt * a.add_stride + nn], y);
        else if (a.acc) y = sadd(*yp, y);
        *yp = y;
    }
}

// ---- Q4_K -----------------------------------------------------------------------------------
//
// Numerics (sw/sim/tsr_ref.c:543-567, 580-635): the term of super-block s is (d Dx) f32(isum) -
// (dmin Dx) f32(msum), isum = sum_j sc_j S_j, msum = sum_j m_j (BS[2j] + BS[2j+1]), S_j the int8
// dot of sub-block j; the activation is quantized by QACT A256 (k_qact_mm4). Terms go to partial
// s mod 16 in order of s, then the 16-partial tree, as for Q8_0.
//
// Per super-block s and 32 x 32 tile the tokens are the A operand and the weight rows the B operand,
// so that a result lane holds one weight row (whose scales the lane decoded itself) and 16 tokens:
//   S_j  = v_mfma_i32_32x32x32_i8(X sub-block j, W sub-block j), j = 0..7: the lane's 16-byte
//          piece 2g + h of the weight row holds values 16 h .. 16 h + 15 of sub-block 2g in its low
//          nibbles and of sub-block 2g + 1 in its high nibbles;
//   isum = sum_j sc_j S_j (one v_mad_i32_i24 per output and sub-block);
//   msum = four v_mfma_f32_32x32x2f32 over k = j of bs_j[token] m_j[row]: every product and every
//          partial sum is an integer below 2^24 in magnitude (|bs_j| <= 32 * 128, m_j < 64), so the
//          matrix core's f32 sum is the exact integer (an exact zero may come out as -0 where the
//          spec's f32(msum) is +0: that can only change the sign of a zero product or term, and a
//          zero term added to a partial that starts at +0 never changes it);
//   term and partial sum on the VALU. Dx is an A256 scale (any f32): while every Dx a wave has met
//   is 0 or >= 2^-60 in magnitude the plain IEEE operations are the spec operations (see
//   k_matvec.hip); from the first super-block with a smaller nonzero Dx on, the wave uses the spec
//   operations, and the tree of a workgroup with such a wave does too.

// QACT A256 of T token rows, block-major: one aligned 16-lane row per (token, super-block)
// (qact_a256_row: lane i holds values 16 i .. 16 i + 15, half i & 1 of sub-block i / 2). Writes
// the quants xq [K/32][T][32 B], the sub-block sums xs [K/32][T] and the scales xd [K/256][tp]
// (tp >= T, a multiple of 32; tokens T .. tp - 1 get d = 0). Every lane of a wave stays active
// (the row operations need them): lanes past the last pair quantize a copy and store nothing. Pairs
// run token-fastest (a wave's 4 rows write the quants of 4 consecutive tokens); the host keeps
// tp (K / 256) 16 below 2^32.
__global__ __launch_bounds__(256) void k_qact_mm4(const float * x, uint64_t x_stride, uint32_t K, uint32_t T,
                                                  uint32_t tp, uint8_t * xq, int32_t * xs, float * xd) {
    const uint32_t nsb = K >> 8;
    const uint32_t pair = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;   // (super-block, token < tp)
    const uint32_t l16 = threadIdx.x & 15u;
    const uint32_t npair = tp * nsb;
    const uint32_t pc = pair < npair ? pair : npair - 1u;
    const uint32_t sb = pc / tp, t = pc - sb * tp;
    const uint32_t tc = t < T ? t : T - 1u;
    const float * xp = x + (size_t)tc * x_stride + 256u * sb + 16u * l16;
    float4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *(const float4 *)(xp + 4 * i);
    float d;
    int s16;
    bool tiny;
    const uint4 q = qact_a256_row(v, &d, &s16, &tiny);
    const int bs = s16 + dpp_i<kDppXor1>(s16);                     // the two halves of sub-block l16 / 2
    if (pair < npair) {
        if (t < T) {
            const uint32_t j = 8u * sb + (l16 >> 1);
            *(uint4 *)(xq + ((size_t)j * T + t) * 32u + 16u * (l16 & 1u)) = q;
            if ((l16 & 1u) == 0u) xs[(size_t)j * T + t] = bs;
        }
        if (l16 == 0u) xd[(size_t)sb * tp + t] = t < T ? d : 0.0f;
    }
}

__device__ __forceinline__ uint32_t q4k_sc(const uint4 mt, uint32_t j) {
    // meta bytes 4 + j: sc_j | (m_j & 3) << 6; nibble j of bytes 12..15: m_j >> 2 (wlayout.hpp)
    return __builtin_amdgcn_ubfe(j < 4u ? mt.y : mt.z, 8u * (j & 3u), 6);
}
__device__ __forceinline__ uint32_t q4k_m(const uint4 mt, uint32_t j) {
    return __builtin_amdgcn_ubfe(j < 4u ? mt.y : mt.z, 8u * (j & 3u) + 6u, 2) | (__builtin_amdgcn_ubfe(mt.w, 4u * j, 4) << 2);
}

// GLU: weight rows 2j and 2j + 1 are the gate and up rows of output j; their results are in adjacent
// lanes of the output phase and y[j] = SWIGLU(gate, up) (as the matvec's GLU epilogue).
// Without GLU, at most 128 VGPRs: two workgroups share a compute unit (measured faster); the GLU form's
// epilogue would spill there, and it keeps one.
template <bool GLU>
__global__ __launch_bounds__(512, GLU ? 2 : 4) void k_mm_q4k(MmArgs a) {
    __shared__ float s_p[16][1024];                                // partial pj of output (r, lane)
    __shared__ int s_slow[8];
    const WGeom g = wgeom(a.N, a.K >> 8, a.rb, true);
    const uint32_t lane = __lane_id(), j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t tx, ty;
    mm_tile(a.grouped != 0u, tx, ty);
    const uint32_t n0 = tx * 32u, t0 = ty * 32u;
    const uint32_t h = lane >> 5, c = lane & 31u;
    // operand rows of this lane (clamped: rows / tokens beyond the matrix are not stored)
    const uint32_t n = min(n0 + c, a.N - 1u), t = min(t0 + c, a.T - 1u);
    const uint32_t B = n / g.rb, R = wl_rows(g, B), rr = n - B * g.rb;
    // buffer windows (as k_mm_q80): the row blocks of the tile's rows, the activation scratch; a load at
    // offset >= 2^31 reads 0 (the k = 1 column of the scale products)
    const uint32_t B0 = n0 / g.rb, B1 = (min(n0 + 31u, a.N - 1u)) / g.rb;
    const uint64_t wbase = (uint64_t)B0 * g.bstride;
    const uint64_t wend = B1 + 1u < g.nblk ? (uint64_t)(B1 + 1u) * g.bstride : wl_bytes(g);
    const __amdgpu_buffer_rsrc_t rw = brsrc(a.w + wbase, (uint32_t)(wend - wbase));
    const __amdgpu_buffer_rsrc_t rx = brsrc(a.qa, a.d_off + 4u * a.tp * g.nb);
    const uint32_t owq = (uint32_t)(wl_quant_off(g, B, R, h, 0u, rr) - wbase);   // piece 2 gg + h: + 16 R (2 gg nb + sl)
    const uint32_t owm = (uint32_t)(wl_meta_off(g, B, R, 0u, rr) - wbase);       // + 16 R sl
    const uint32_t sR = 16u * R, sG = 32u * R * g.nb;
    const uint32_t ox = 32u * t + 16u * h;                        // quants of sub-block jb: + 32 T jb
    const uint32_t obs = a.s_off + 4u * t + 4u * a.T * h;         // sums of sub-block 2 q + h: + 4 T 2 q
    const uint32_t odx = h ? 0x80000000u : a.d_off + 4u * (t0 + c);   // token t0 + c's scale: + 4 tp s
    const uint32_t m4 = 0x0F0F0F0Fu;
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    // byte-wise q * f of a dword of quants q <= 15 and f <= 7 (no byte carries into the next: q f <= 105)
    auto bmul = [](uint32_t q, uint32_t f) -> int {
        return (int)__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * (u16x2){(unsigned short)f, (unsigned short)f});
    };
    bool slow = false;
    // wave j computes partials j and j + 8 (8 waves of up to 256 VGPRs)
    for (uint32_t half = 0; half < 2u; ++half) {
    const uint32_t pj = j + 8u * half, cnt = wl_count(g, pj), sl0 = wl_slot(g, pj, 0u);
    v16f p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = 0.0f;
    for (uint32_t k = 0; k < cnt; ++k) {
        const uint32_t sl = sl0 + k, s = pj + 16u * k;
        v4i wv[4], xv[8];
#pragma unroll
        for (uint32_t gg = 0; gg < 4u; ++gg) wv[gg] = bload128(rw, owq + sR * sl + sG * gg, 0u);
        const uint4 mt = __builtin_bit_cast(uint4, bload128(rw, owm + sR * sl, 0u));
#pragma unroll
        for (uint32_t jb = 0; jb < 8u; ++jb) xv[jb] = bload128(rx, ox, 32u * a.T * (8u * s + jb));
        float bsf[4];
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) bsf[q] = (float)(int)__builtin_amdgcn_raw_buffer_load_b32(rx, (int)obs, (int)(4u * a.T * (8u * s + 2u * q)), 0);
        const float dxl = bloadf(rx, odx, 4u * a.tp * s);

        v16f ms = {};
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q)
            ms = __builtin_amdgcn_mfma_f32_32x32x2f32(bsf[q], (float)q4k_m(mt, 2u * q + h), ms, 0, 0, 0);
        // isum = sum_j sc_j S_j on the matrix core: sc_j = 8 a_j + b_j (a_j, b_j <= 7), the weight quants
        // scaled by a_j and by b_j (<= 105: int8) into two exact int32 accumulators, isum = 8 A + B
        v16i ia = {}, ib = {};
#pragma unroll
        for (uint32_t gg = 0; gg < 4u; ++gg) {
            const uint32_t sc0 = q4k_sc(mt, 2u * gg), sc1 = q4k_sc(mt, 2u * gg + 1u);
            v4i la, lb, ha, hb;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = (uint32_t)wv[gg][e] & m4, hi = ((uint32_t)wv[gg][e] >> 4) & m4;
                la[e] = bmul(lo, sc0 >> 3);
                lb[e] = bmul(lo, sc0 & 7u);
                ha[e] = bmul(hi, sc1 >> 3);
                hb[e] = bmul(hi, sc1 & 7u);
            }
            ia = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[2 * gg], la, ia, 0, 0, 0);
            ib = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[2 * gg], lb, ib, 0, 0, 0);
            ia = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[2 * gg + 1], ha, ia, 0, 0, 0);
            ib = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[2 * gg + 1], hb, ib, 0, 0, 0);
        }
        v16i isum;
#pragma unroll
        for (int r = 0; r < 16; ++r) isum[r] = (ia[r] << 3) + ib[r];
        const float d = h2f_fast(mt.x & 0xFFFFu), dm = h2f_fast(mt.x >> 16);
        {
            const uint32_t ad = fb(dxl) & 0x7FFFFFFFu;            // the 32 tokens' scales, one a lane
            slow = slow || __ballot(ad != 0u && ad < 0x21800000u) != 0ull;   // wave-uniform, sticky
        }
        if (!slow) {
            // d Dx and dmin Dx as outer products on the matrix core (one IEEE product each; k = 1 is zero)
            v16f P1 = {}, P2 = {};
            P1 = __builtin_amdgcn_mfma_f32_32x32x2f32(dxl, h ? 0.0f : d, P1, 0, 0, 0);
            P2 = __builtin_amdgcn_mfma_f32_32x32x2f32(dxl, h ? 0.0f : dm, P2, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float tt = P1[r] * (float)isum[r] - P2[r] * ms[r];
                p[r] = p[r] + tt;
            }
        } else {
            // tokens of result r = 4 q + i: t0 + 8 q + 4 h + i
            const float * xd = (const float *)(a.qa + a.d_off) + (size_t)a.tp * s + t0 + 4u * h;
            float4 dx4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) dx4[q] = *(const float4 *)(xd + 8u * q);
            const float dxs[16] = { dx4[0].x, dx4[0].y, dx4[0].z, dx4[0].w, dx4[1].x, dx4[1].y, dx4[1].z, dx4[1].w,
                                    dx4[2].x, dx4[2].y, dx4[2].z, dx4[2].w, dx4[3].x, dx4[3].y, dx4[3].z, dx4[3].w };
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float tt = ssub(smul(smul(d, dxs[r]), i2f(isum[r])), smul(smul(dm, dxs[r]), ms[r]));
                p[r] = sadd(p[r], tt);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s_p[pj][64u * (uint32_t)r + lane] = p[r];
    }
    if (lane == 0u) s_slow[j] = slow ? 1 : 0;
    lds_barrier();

    bool any_slow = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) any_slow |= s_slow[i] != 0;
    uint32_t t64 = 0;
    if constexpr (GLU) t64 = a.ex.t64[lane];
    // two outputs per thread, o = 64 r + lane of the wave layout above: weight row n0 + lane % 32,
    // token t0 + 8 (r / 4) + 4 (lane / 32) + r % 4 (a wave stores 32 consecutive rows of 2 tokens)
    for (uint32_t o = threadIdx.x; o < 1024u; o += 512u) {
    const uint32_t ol = o & 63u, r = o >> 6;
    const uint32_t nn = n0 + (ol & 31u), tt = t0 + 8u * (r >> 2) + 4u * (ol >> 5) + (r & 3u);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = s_p[i][o];
    if (!any_slow) {
#pragma unroll
        for (int w = 16; w > 1; w >>= 1)
#pragma unroll
            for (int i = 0; i < w / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
    } else {
#pragma unroll
        for (int w = 16; w > 1; w >>= 1)
#pragma unroll
            for (int i = 0; i < w / 2; ++i) v[i] = sadd(v[2 * i], v[2 * i + 1]);
    }
    if constexpr (GLU) {
        const float gt = canon(v[0]);
        const float h = swiglu_reg(gt, dpp_f<kDppXor1>(gt), a.ex, t64);   // every lane: the table is read by bpermute
        if ((ol & 1u) == 0u && tt < a.T && nn < a.N) a.y[(size_t)tt * a.y_stride + (nn >> 1)] = h;
    } else if (tt < a.T && nn < a.N) {
        float y = canon(v[0]);
        float * yp = a.y + (size_t)tt * a.y_stride + nn;
        if (a.add) y = sadd(a.add[(size_t)tt * a.add_stride + nn], y);
        else if (a.acc) y = sadd(*yp, y);
        *yp = y;
    }
    }
}

}  // namespace tsr

int tsr_launch_qact_mm4(const float * x, uint64_t x_stride, uint32_t K, uint32_t T, uint32_t tp, uint8_t * xq,
                        int32_t * xs, float * xd, hipStream_t s) {
    const uint64_t threads = (uint64_t)tp * (K / 256u) * 16u;
    if (threads + 255u >= 0x100000000ull) return -2;              // 32-bit pair indices
    hipLaunchKernelGGL(tsr::k_qact_mm4, dim3((uint32_t)((threads + 255u) / 256u)), dim3(256), 0, s, x, x_stride, K, T,
                       tp, xq, xs, xd);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mm_q4_k(const tsr::MmArgs & a, hipStream_t s) {
    const tsr::WGeom g = tsr::wgeom(a.N, a.K >> 8, a.rb, true);
    if ((uint64_t)(31u / a.rb + 2u) * g.bstride >= 0x80000000ull) return -2;   // a tile's buffer window
    const uint32_t gx = (a.N + 31u) / 32u, gy = (a.T + 31u) / 32u;
    tsr::MmArgs m = a;
    m.grouped = (gx & 7u) == 0u && (uint64_t)a.N * (a.K / 256u) * 144u > (48ull << 20) ? 1u : 0u;   // measured
    const dim3 grid = m.grouped ? dim3(8u * gy, gx / 8u) : dim3(gx, gy);
    if (a.glu) hipLaunchKernelGGL(tsr::k_mm_q4k<true>, grid, dim3(512), 0, s, m);
    else hipLaunchKernelGGL(tsr::k_mm_q4k<false>, grid, dim3(512), 0, s, m);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_qact_mm(const float * x, uint64_t x_stride, uint32_t K, uint32_t T, uint8_t * xq, float * xd,
                       hipStream_t s) {
    const uint64_t threads = (uint64_t)T * (K / 32u) * 8u;
    if (threads + 255u >= 0x100000000ull) return -2;              // 32-bit pair indices
    hipLaunchKernelGGL(tsr::k_qact_mm, dim3((uint32_t)((threads + 255u) / 256u)), dim3(256), 0, s, x, x_stride, K, T, xq, xd);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mm_q8_0(const tsr::MmArgs & a, hipStream_t s) {
    const tsr::WGeom g = tsr::wgeom(a.N, a.K >> 5, a.rb, false);
    if ((uint64_t)(31u / a.rb + 2u) * g.bstride >= 0x80000000ull) return -2;   // a tile's buffer window
    const uint32_t gx = (a.N + 31u) / 32u, gy = (a.T + 31u) / 32u;
    tsr::MmArgs m = a;
    m.grouped = (gx & 7u) == 0u && (uint64_t)a.N * (a.K / 32u) * 34u > (24ull << 20) ? 1u : 0u;
    const dim3 grid = m.grouped ? dim3(8u * gy, gx / 8u) : dim3(gx, gy);
    hipLaunchKernelGGL(tsr::k_mm_q80, grid, dim3(1024), 0, s, m);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
