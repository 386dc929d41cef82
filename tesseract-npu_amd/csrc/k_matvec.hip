// k_matvec.hip -- decode MUL_MAT (matrix-vector) kernels for Q8_0 and Q4_K weights on gfx950.
//
// Numerics (sw/sim/tsr_ref.c:525-635; docs/spec.md:438-477): per row, term i of block / super-block i
// is added into partial p[i mod 16] in order, then y = ((p0+p1)+(p2+p3))+... (the 16-partial tree);
// Q8_0 term = (d Dx) f32(isum), Q4_K term = (d Dx) f32(isum) - (dmin Dx) f32(msum). The integer sums
// are exact in any order, so they are split over lanes freely; the f32 adds keep the reference's
// pairing: each partial is owned by one lane group and the tree is a butterfly whose pairs are the
// tree's pairs (f32 addition is commutative).
//
// Each workgroup first quantizes the activation row (QACT) into LDS, then every wave streams its
// weight rows with 16-byte coalesced loads (one 1 KiB wave load per instruction), does int8 dot
// products with v_dot4_i32_i8 and reduces with DPP.
//
// Fast and exact f32 paths. With f32 denormals on and no FMA contraction, plain IEEE operations give
// the spec result whenever no operand or result is subnormal; NaN payloads are the only other
// difference and the stored y is canonicalized. Every term is (d Dx) f32(int) with d an fp16 value
// (|d| >= 2^-24 or 0) and |Dx| >= 2^-24 (A32: an fp16 value) or, for A256, checked per row of x:
// when every nonzero |Dx| >= 2^-60, every nonzero term and partial sum is a multiple of 2^-107 and
// so never subnormal. Otherwise (tiny A256 scales) the kernel takes the exact path with the spec
// operations on every step.
#include "kernels.hpp"
#include "qact.hpp"

namespace tsr {

// 6-bit scale / min of sub-block j from the packed scales (bytes 0-3 = s03, 4-7 = s47, 8-11 = s811);
// get_scale_min_k4 (sw/sim/tsr_ref.c:359-367).
__device__ __forceinline__ void q4k_sm(int j, uint32_t s03, uint32_t s47, uint32_t s811, int & sc, int & mn) {
    const int k = j & 3, sh = 8 * k;
    const int b03 = (int)((s03 >> sh) & 0xFFu), b47 = (int)((s47 >> sh) & 0xFFu), b811 = (int)((s811 >> sh) & 0xFFu);
    if (j < 4) {
        sc = b03 & 63;
        mn = b47 & 63;
    } else {
        sc = (b811 & 15) | ((b03 >> 6) << 4);
        mn = (b811 >> 4) | ((b47 >> 6) << 4);
    }
}

__device__ __forceinline__ void store_y(const MvArgs & a, uint32_t t, uint32_t row, float v) {
    float * yp = a.y + (size_t)t * a.y_stride + row;
    if (a.add) v = sadd(a.add[(size_t)t * a.add_stride + row], v);
    else if (a.acc) v = sadd(*yp, v);
    *yp = v;
}

// ---------------------------------------------------------------------------------------------
// Q4_K: block of 1024 threads (16 waves), one row per wave. Lane L, load i covers quant chunk
// c = 64 i + L (16 bytes) of the row: super-block s = c / 8, piece h = c % 8 of its 128 quant bytes,
// i.e. group g = h / 2 (sub-blocks 2g low nibbles, 2g+1 high nibbles), half h % 2. Eight lanes hold a
// super-block; term s goes to partial s mod 16 = 8 (i mod 2) + L / 8, kept in pa (i even) / pb (odd).
// ---------------------------------------------------------------------------------------------
template <int NL>
__global__ __launch_bounds__(1024) void k_mv_q4k(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t K = a.K, nsb = K / 256u;
    int8_t * s_qs = (int8_t *)lds;
    float * s_dx = (float *)(lds + K);
    int * s_bsp = (int *)(s_dx + nsb);                          // sum of the 32 q of each sub-block
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;

    int slow = 0;
    for (uint32_t s = (uint32_t)wave; s < nsb; s += (uint32_t)nw) {
        const float4 v = *(const float4 *)(x + 256u * s + 4u * (uint32_t)lane);
        float d;
        int s4;
        const uint32_t q = qact_a256_lane(v, lane, &d, &s4);
        *(uint32_t *)(s_qs + 256u * s + 4u * (uint32_t)lane) = q;
        const int s32 = sum8_i(s4);
        if (lane == 0) s_dx[s] = d;
        if ((lane & 7) == 0) s_bsp[8u * s + (uint32_t)(lane >> 3)] = s32;
        const uint32_t ad = fb(d) & 0x7FFFFFFFu;
        slow |= (ad != 0u && ad < 0x21800000u) ? 1 : 0;          // 0 < |d| < 2^-60
    }
    slow = __syncthreads_or(slow);

    const uint32_t row = blockIdx.x * (uint32_t)nw + (uint32_t)wave;
    if (row >= a.N) return;
    const uint8_t * rq = a.wq + (size_t)row * nsb * 128u;
    const uint8_t * rm = a.wm + (size_t)row * nsb * 16u;
    const uint32_t nchunk = nsb * 8u;

    uint4 qv[NL], mv[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t c = 64u * (uint32_t)i + (uint32_t)lane;
        if (c < nchunk) {
            qv[i] = *(const uint4 *)(rq + 16u * c);
            mv[i] = *(const uint4 *)(rm + 16u * (c >> 3));
        } else {
            qv[i] = make_uint4(0u, 0u, 0u, 0u);
            mv[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    }

    const int h = lane & 7, g = h >> 1, half = h & 1;
    float pa = 0.0f, pb = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t c = 64u * (uint32_t)i + (uint32_t)lane;
        const uint32_t s = c >> 3;
        const bool valid = c < nchunk;
        int4 xl = make_int4(0, 0, 0, 0), xh = make_int4(0, 0, 0, 0);
        int bsp = 0;
        float dx = 0.0f;
        if (valid) {
            xl = *(const int4 *)(s_qs + 256u * s + 64u * (uint32_t)g + 16u * (uint32_t)half);
            xh = *(const int4 *)(s_qs + 256u * s + 64u * (uint32_t)g + 32u + 16u * (uint32_t)half);
            bsp = s_bsp[8u * s + (uint32_t)h];
            dx = s_dx[s];
        }
        const uint32_t m4 = 0x0F0F0F0Fu;
        int slo = dot4((int)(qv[i].x & m4), xl.x, 0);
        slo = dot4((int)(qv[i].y & m4), xl.y, slo);
        slo = dot4((int)(qv[i].z & m4), xl.z, slo);
        slo = dot4((int)(qv[i].w & m4), xl.w, slo);
        int shi = dot4((int)((qv[i].x >> 4) & m4), xh.x, 0);
        shi = dot4((int)((qv[i].y >> 4) & m4), xh.y, shi);
        shi = dot4((int)((qv[i].z >> 4) & m4), xh.z, shi);
        shi = dot4((int)((qv[i].w >> 4) & m4), xh.w, shi);
        int sc_lo, sc_hi, mn, dummy;
        q4k_sm(2 * g, mv[i].y, mv[i].z, mv[i].w, sc_lo, dummy);
        q4k_sm(2 * g + 1, mv[i].y, mv[i].z, mv[i].w, sc_hi, dummy);
        q4k_sm(h, mv[i].y, mv[i].z, mv[i].w, dummy, mn);
        int ip = sc_lo * slo + sc_hi * shi;
        int mp = mn * bsp;
        ip = sum8_i(ip);
        mp = sum8_i(mp);
        if (a.isums != nullptr && t == 0u && h == 0 && valid) {
            a.isums[(size_t)row * 2u * nsb + 2u * s] = ip;
            a.isums[(size_t)row * 2u * nsb + 2u * s + 1u] = mp;
        }
        const float d = h2f_fast(mv[i].x & 0xFFFFu), dm = h2f_fast(mv[i].x >> 16);
        float tt;
        if (!slow) {
            const float t1 = (d * dx) * (float)ip;
            const float t2 = (dm * dx) * (float)mp;
            tt = t1 - t2;
        } else {
            tt = ssub(smul(smul(d, dx), i2f(ip)), smul(smul(dm, dx), i2f(mp)));
        }
        if (valid) {
            if (i & 1) pb = slow ? sadd(pb, tt) : pb + tt;
            else pa = slow ? sadd(pa, tt) : pa + tt;
        }
    }
    // tree: slots L/8 pair by xor 1, 2, 4 of the slot (lanes xor 8, 16, 32); pa = p0..p7, pb = p8..p15
    float y;
    if (!slow) {
        pa = pa + dpp_f<kDppRowMirror>(pa);
        pb = pb + dpp_f<kDppRowMirror>(pb);
        pa = pa + xor16_f(pa);
        pb = pb + xor16_f(pb);
        pa = pa + xor32_f(pa);
        pb = pb + xor32_f(pb);
        y = canon(pa + pb);
    } else {
        pa = sadd(pa, dpp_f<kDppRowMirror>(pa));
        pb = sadd(pb, dpp_f<kDppRowMirror>(pb));
        pa = sadd(pa, xor16_f(pa));
        pb = sadd(pb, xor16_f(pb));
        pa = sadd(pa, xor32_f(pa));
        pb = sadd(pb, xor32_f(pb));
        y = sadd(pa, pb);
    }
    if (lane == 0) store_y(a, t, row, y);
}

// ---------------------------------------------------------------------------------------------
// Q8_0: block of 256 threads (4 waves), RPW rows per wave. Lane L, load i covers quant chunk
// c = 64 i + L: block b = 32 i + L / 2, half L % 2. Blocks b (lane L < 32) and b + 16 (lane L + 32)
// both belong to partial b mod 16 = (L / 2) mod 16, in that order; the lower half owns the partials.
// ---------------------------------------------------------------------------------------------
template <int NL, int RPW>
__global__ __launch_bounds__(256) void k_mv_q80(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t K = a.K, nb = K / 32u;
    int8_t * s_qs = (int8_t *)lds;
    float * s_dx = (float *)(lds + K);
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;

    for (uint32_t slot = threadIdx.x; slot < K / 4u; slot += blockDim.x) {   // 8 lanes per 32-block
        const float4 v = *(const float4 *)(x + 4u * slot);
        float D;
        const uint32_t q = qact_a32_lane(v, &D);
        *(uint32_t *)(s_qs + 4u * slot) = q;
        if ((lane & 7) == 0) s_dx[slot >> 3] = D;
    }
    __syncthreads();

    const uint32_t row0 = (blockIdx.x * (uint32_t)nw + (uint32_t)wave) * RPW;
    if (row0 >= a.N) return;
    uint4 qv[RPW][NL];
    uint32_t dv[RPW][NL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint32_t row = row0 + (uint32_t)r;
        const uint8_t * rq = a.wq + (size_t)row * nb * 32u;
        const uint16_t * rm = (const uint16_t *)(a.wm + (size_t)row * nb * 2u);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const uint32_t c = 64u * (uint32_t)i + (uint32_t)lane, b = c >> 1;
            if (row < a.N && b < nb) {
                qv[r][i] = *(const uint4 *)(rq + 16u * c);
                dv[r][i] = rm[b];
            } else {
                qv[r][i] = make_uint4(0u, 0u, 0u, 0u);
                dv[r][i] = 0u;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint32_t row = row0 + (uint32_t)r;
        if (row >= a.N) break;
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const uint32_t c = 64u * (uint32_t)i + (uint32_t)lane, b = c >> 1;
            int4 xv = make_int4(0, 0, 0, 0);
            float dx = 0.0f;
            if (b < nb) {
                xv = *(const int4 *)(s_qs + 16u * c);
                dx = s_dx[b];
            }
            int is = dot4((int)qv[r][i].x, xv.x, 0);
            is = dot4((int)qv[r][i].y, xv.y, is);
            is = dot4((int)qv[r][i].z, xv.z, is);
            is = dot4((int)qv[r][i].w, xv.w, is);
            is += dpp_i<kDppXor1>(is);
            if (a.isums != nullptr && t == 0u && (lane & 1) == 0 && b < nb) a.isums[(size_t)row * nb + b] = is;
            const float tt = (h2f_fast(dv[r][i]) * dx) * (float)is;
            const float tu = xor32_f(tt);
            if (lane < 32) {
                if (b < nb) p = p + tt;
                if (b + 16u < nb) p = p + tu;
            }
        }
        p = p + dpp_f<kDppXor2>(p);
        p = p + dpp_f<kDppRowHalfMirror>(p);
        p = p + dpp_f<kDppRowMirror>(p);
        p = p + xor16_f(p);
        if (lane == 0) store_y(a, t, row, canon(p));
    }
}

}  // namespace tsr

// ---- launchers ------------------------------------------------------------------------------------
#define TSR_Q4K_CASE(n) case n: hipLaunchKernelGGL(tsr::k_mv_q4k<n>, grid, dim3(1024), lds, s, a); break;

int tsr_launch_mv_q4_k(const tsr::MvArgs & a, hipStream_t s) {
    const uint32_t nsb = a.K / 256u, NL = (nsb + 7u) / 8u;
    const size_t lds = (size_t)a.K + 4u * nsb + 32u * nsb;
    dim3 grid((a.N + 15u) / 16u, a.T);
    switch (NL) {
        TSR_Q4K_CASE(1) TSR_Q4K_CASE(2) TSR_Q4K_CASE(3) TSR_Q4K_CASE(4) TSR_Q4K_CASE(5) TSR_Q4K_CASE(6)
        TSR_Q4K_CASE(7) TSR_Q4K_CASE(8) TSR_Q4K_CASE(9) TSR_Q4K_CASE(10) TSR_Q4K_CASE(11) TSR_Q4K_CASE(12)
        TSR_Q4K_CASE(13) TSR_Q4K_CASE(14) TSR_Q4K_CASE(15) TSR_Q4K_CASE(16)
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

#define TSR_Q80_CASE(n, rpw) \
    case n: hipLaunchKernelGGL((tsr::k_mv_q80<n, rpw>), dim3((a.N + 4u * rpw - 1u) / (4u * rpw), a.T), dim3(256), lds, s, a); break;

int tsr_launch_mv_q8_0(const tsr::MvArgs & a, hipStream_t s) {
    const uint32_t nb = a.K / 32u, NL = (nb + 31u) / 32u;
    const size_t lds = (size_t)a.K + 4u * nb;
    switch (NL) {
        TSR_Q80_CASE(1, 4) TSR_Q80_CASE(2, 4) TSR_Q80_CASE(3, 2) TSR_Q80_CASE(4, 2) TSR_Q80_CASE(5, 1)
        TSR_Q80_CASE(6, 1) TSR_Q80_CASE(7, 1) TSR_Q80_CASE(8, 1) TSR_Q80_CASE(9, 1) TSR_Q80_CASE(10, 1)
        TSR_Q80_CASE(11, 1) TSR_Q80_CASE(12, 1) TSR_Q80_CASE(13, 1) TSR_Q80_CASE(14, 1) TSR_Q80_CASE(15, 1)
        TSR_Q80_CASE(16, 1) TSR_Q80_CASE(17, 1) TSR_Q80_CASE(18, 1) TSR_Q80_CASE(19, 1) TSR_Q80_CASE(20, 1)
        TSR_Q80_CASE(21, 1) TSR_Q80_CASE(22, 1) TSR_Q80_CASE(23, 1) TSR_Q80_CASE(24, 1) TSR_Q80_CASE(25, 1)
        TSR_Q80_CASE(26, 1) TSR_Q80_CASE(27, 1) TSR_Q80_CASE(28, 1) TSR_Q80_CASE(29, 1) TSR_Q80_CASE(30, 1)
        TSR_Q80_CASE(31, 1) TSR_Q80_CASE(32, 1)
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
