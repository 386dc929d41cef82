// mv_q4k.hpp -- device helpers of the Q4_K row dot shared by the matvec kernels (k_matvec.hip) and the
// Q|K|V rows of the one-launch decode attention (k_fa_dec.hip): the fused RMS_NORM + MUL applied to x
// ahead of its QACT, and the integer sums of one (row, super-block) unit.
//
// Numerics (sw/sim/tsr_ref.c:525-635): the Q4_K term of super-block s is (d Dx) f32(isum) -
// (dmin Dx) f32(msum) with isum = sum_j sc_j S_j and msum = sum_j m_j (bs[2j] + bs[2j + 1]) over its 8
// sub-blocks j (S_j: the sub-block's int8 dot product, bs: the 16-value sums of the quantized x).
#pragma once

#include "glue.hpp"
#include "tsr_dev.hpp"

namespace tsr {

constexpr uint32_t kXq4Stride = 272u;   // LDS bytes per quantized 256-value block (k slots on distinct banks)

// FM(FM(x, s), w) (w when has_w) of 4 values: RMS_NORM + MUL on the f32 rules.
__device__ __forceinline__ float4 prep_norm_apply(float4 v, float s, float4 w, bool has_w) {
    v.x = smul(v.x, s); v.y = smul(v.y, s); v.z = smul(v.z, s); v.w = smul(v.w, s);
    if (has_w) { v.x = smul(v.x, w.x); v.y = smul(v.y, w.y); v.z = smul(v.z, w.z); v.w = smul(v.w, w.w); }
    return v;
}
// prep_norm_apply over a lane's 16 values when the wave qualifies (wave-uniform result): the scale
// is a normal number, every x and w is a normal number or a zero, and no product x s or (x s) w of
// nonzero factors can be subnormal or overflow. Then DAZ and FTZ are the identity and no NaN arises,
// so the plain products equal FM(FM(x, s), w) of the general form. The test runs on bounds, not per
// product: with a value's magnitude bits t = bits << 1 (sign dropped), t >= 0xFF000000 is Inf or NaN
// and t - 1 < 0x00FFFFFF a subnormal (a zero wraps to 0xFFFFFFFF, above every other value), so one
// maximum of t and one minimum of t - 1 over the lane give the largest and the smallest nonzero
// magnitude; rounding is monotonic, so every product of nonzero factors lies between the products of
// the bounds (rounded the same way).
__device__ __forceinline__ bool prep_norm_apply_fast(float4 (&v)[4], float s, const float4 (&w)[4], bool has_w) {
    uint32_t xhi = 0u, xlo = 0xFFFFFFFFu, whi = 0u, wlo = 0xFFFFFFFFu;
    auto acc = [](uint32_t & hi, uint32_t & lo, float a, float b) {
        const uint32_t ta = fb(a) << 1, tb = fb(b) << 1;
        hi = max(hi, max(ta, tb));
        lo = min(lo, min(ta - 1u, tb - 1u));
    };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        acc(xhi, xlo, v[c].x, v[c].y);
        acc(xhi, xlo, v[c].z, v[c].w);
        if (has_w) {
            acc(whi, wlo, w[c].x, w[c].y);
            acc(whi, wlo, w[c].z, w[c].w);
        }
    }
    constexpr float kMin = 0x1p-126f, kMax = 0x1.fffffep127f;
    const float as = __builtin_fabsf(s);
    bool ok = __builtin_amdgcn_classf(s, 0x108) && xhi < 0xFF000000u && xlo >= 0x00FFFFFFu;   // s: +-normal
    const float tlo = bf((xlo + 1u) >> 1) * as, thi = bf(xhi >> 1) * as;
    const bool xz = xlo == 0xFFFFFFFFu;                           // every x a zero: every product a zero
    ok = ok && (xz || (tlo >= kMin && thi <= kMax));
    if (has_w) {
        ok = ok && whi < 0xFF000000u && wlo >= 0x00FFFFFFu;
        const float ylo = tlo * bf((wlo + 1u) >> 1), yhi = thi * bf(whi >> 1);
        ok = ok && (xz || wlo == 0xFFFFFFFFu || (ylo >= kMin && yhi <= kMax));
    }
    if (__ballot(!ok) != 0ull) return false;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        v[c].x = v[c].x * s; v[c].y = v[c].y * s; v[c].z = v[c].z * s; v[c].w = v[c].w * s;
        if (has_w) { v[c].x = v[c].x * w[c].x; v[c].y = v[c].y * w[c].y; v[c].z = v[c].z * w[c].z; v[c].w = v[c].w * w[c].w; }
    }
    return true;
}
__device__ __forceinline__ float4 sq4(float4 v) { return make_float4(sq_rule(v.x), sq_rule(v.y), sq_rule(v.z), sq_rule(v.w)); }

// The integer sums of one Q4_K unit over the lane's NP quant pieces. The F = 8 / NP lanes of a unit hold
// pieces NP q .. NP q + NP - 1 (piece p: group g = p / 2 of sub-blocks 2g (low nibbles) and 2g + 1 (high
// nibbles), values 64g + 16 (p mod 2) + 0..15 and the same + 32); the caller adds the F lanes' sums.
// qv: the pieces; mt: the meta piece (fp16 d, fp16 dmin; byte 4 + j = sc_j | (m_j & 3) << 6, nibble j
// of bytes 12..15 = m_j >> 2); xb: the x block's 256 quants (LDS); bsp: its 8 sub-block sums (LDS).
template <uint32_t NP>
__device__ __forceinline__ void q4k_unit_sums(const uint4 (&qv)[NP], const uint4 & mt, const int8_t * xb, const int * bsp,
                                              uint32_t q, int & isum, int & msum) {
    const uint32_t m4 = 0x0F0F0F0Fu;
    isum = 0;
    msum = 0;
#pragma unroll
    for (uint32_t gi = 0; gi < NP / 2u; ++gi) {
        const uint32_t gg = (NP / 2u) * q + gi;                   // group of sub-blocks 2gg (low), 2gg + 1 (high)
        int lo = 0, hi = 0;
#pragma unroll
        for (uint32_t hh = 0; hh < 2u; ++hh) {
            const uint4 qw = qv[2u * gi + hh];
            const int4 xl = *(const int4 *)(xb + 64u * gg + 16u * hh);
            const int4 xh = *(const int4 *)(xb + 64u * gg + 32u + 16u * hh);
            lo = dot4((int)(qw.x & m4), xl.x, lo);
            lo = dot4((int)(qw.y & m4), xl.y, lo);
            lo = dot4((int)(qw.z & m4), xl.z, lo);
            lo = dot4((int)(qw.w & m4), xl.w, lo);
            hi = dot4((int)((qw.x >> 4) & m4), xh.x, hi);
            hi = dot4((int)((qw.y >> 4) & m4), xh.y, hi);
            hi = dot4((int)((qw.z >> 4) & m4), xh.z, hi);
            hi = dot4((int)((qw.w >> 4) & m4), xh.w, hi);
        }
        const int2 bs = *(const int2 *)(bsp + 2u * gg);
        const uint32_t wd = gg < 2u ? mt.y : mt.z, sh = 16u * (gg & 1u);
        const int sc0 = (int)__builtin_amdgcn_ubfe(wd, sh, 6), sc1 = (int)__builtin_amdgcn_ubfe(wd, sh + 8u, 6);
        const int mn0 = (int)(__builtin_amdgcn_ubfe(wd, sh + 6u, 2) | (__builtin_amdgcn_ubfe(mt.w, 8u * gg, 4) << 2));
        const int mn1 = (int)(__builtin_amdgcn_ubfe(wd, sh + 14u, 2) | (__builtin_amdgcn_ubfe(mt.w, 8u * gg + 4u, 4) << 2));
        isum += __mul24(sc0, lo) + __mul24(sc1, hi);              // |S_j| < 2^16, sc < 64: v_mad_i32_i24
        msum += __mul24(mn0, bs.x) + __mul24(mn1, bs.y);
    }
}

}  // namespace tsr
