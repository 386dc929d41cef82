// qact.hpp -- QACT on the device (sw/sim/tsr_ref.c:456-520; docs/spec.md:411-425, 1419-1430).
//
// A32 (Q8_0 activations, also the FA query and the KV rows): blocks of 32, amax = max |DAZ(x)| with
// NaN excluded, d = FD(amax, 127), id = d != 0 ? RC(d) : 0, q = round_half_away(FM(x, id)),
// D = f32(fp16(d)). Eight lanes hold one block, four values each.
//
// A256 (Q4_K activations): blocks of 256, max = DAZ(x) of the first element with the largest |x|
// (NaN excluded); all zero: d = 0, q = 0; else iscale = FD(-127, max), q = round_half_even(FM(iscale,
// x)), d = RC(iscale); BS = sums of 16 q. One wave holds one block, four values per lane.
#pragma once

#include "tsr_dev.hpp"

namespace tsr {

__device__ __forceinline__ uint32_t mag_bits(float v) { return fb(daz(v)) & 0x7FFFFFFFu; }

__device__ __forceinline__ uint32_t umax_u(uint32_t a, uint32_t b) { return a > b ? a : b; }

// One A32 block held by the 8 lanes of an aligned group: returns this lane's 4 quants packed
// little-endian and the block's D in *D (every lane of the group).
__device__ __forceinline__ uint32_t qact_a32_lane(const float4 v, float * D) {
    const float xs[4] = { v.x, v.y, v.z, v.w };
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = mag_bits(xs[i]);
        if (a <= 0x7F800000u && a > m) m = a;
    }
    m = umax_u(m, (uint32_t)dpp_i<kDppXor1>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppXor2>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppRowHalfMirror>((int)m));
    const float d = sdiv(bf(m), 127.0f);
    const float id = (fb(d) & 0x7FFFFFFFu) ? srcp(d) : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed |= ((uint32_t)round_away8(smul(xs[i], id)) & 0xFFu) << (8 * i);
    *D = h2f_exact(f2h_exact(d));
    return packed;
}

// One A256 block held by a whole wave (lane l: values 4l .. 4l+3). Returns this lane's 4 quants
// packed; *d = the block's d (every lane); *sum4 = the sum of this lane's 4 quants.
__device__ __forceinline__ uint32_t qact_a256_lane(const float4 v, int lane, float * d, int * sum4) {
    const float xs[4] = { v.x, v.y, v.z, v.w };
    uint32_t m = 0;
    int at = 0;
    float best = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = mag_bits(xs[i]);
        if (a <= 0x7F800000u && a > m) { m = a; at = 4 * lane + i; best = daz(xs[i]); }
    }
    // wave-wide: the largest magnitude, the smallest index among equals
    uint32_t km = m, ki = 0xFFFFu - (uint32_t)at;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t om = (uint32_t)shfl_i((int)km, lane ^ off);
        const uint32_t oi = (uint32_t)shfl_i((int)ki, lane ^ off);
        if (om > km || (om == km && oi > ki)) { km = om; ki = oi; }
    }
    uint32_t packed = 0;
    int s = 0;
    float dd = 0.0f;
    if (km != 0u) {
        const int win = (int)(0xFFFFu - ki);
        const float mx = shfl_f(best, win >> 2);
        const float iscale = sdiv(-127.0f, mx);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = round_even8(smul(iscale, xs[i]));
            s += q;
            packed |= ((uint32_t)q & 0xFFu) << (8 * i);
        }
        dd = srcp(iscale);
    }
    *d = dd;
    *sum4 = s;
    return packed;
}

}  // namespace tsr
