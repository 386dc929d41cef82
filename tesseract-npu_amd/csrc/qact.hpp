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
// The common case of qact_a32_lane: a wave whose values are all finite and whose blocks have amax = 0
// or amax >= 2^-60. DAZ then acts on the maximum only (a subnormal maximum means a block of zeros after
// DAZ), d = amax / 127 and RC(d) are plain IEEE operations on normal numbers, the plain product
// rounds like FM (see below), and f32(fp16(d)) is the hardware's RNE conversion (fp16 denormals on),
// which is the rule's for every finite d. Returns false, wave-uniformly, when the wave does not
// qualify; the general form then runs.
__device__ __forceinline__ bool qact_a32_lane_fast(const float4 v, uint32_t * out, float * D) {
    const float xs[4] = { v.x, v.y, v.z, v.w };
    bool nonfin = false;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        nonfin |= __builtin_amdgcn_classf(xs[i], 0x207);           // NaN, +-Inf
        m = umax_u(m, fb(xs[i]) & 0x7FFFFFFFu);
    }
    if (__ballot(nonfin) != 0ull) return false;
    m = umax_u(m, (uint32_t)dpp_i<kDppXor1>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppXor2>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppRowHalfMirror>((int)m));
    m = m < 0x00800000u ? 0u : m;
    if (__ballot(m != 0u && m < 0x21800000u) != 0ull) return false;
    const float d = bf(m) / 127.0f;                               // = sdiv: normal operands and result
    const float id = m ? 1.0f / d : 0.0f;                         // = srcp
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed |= ((uint32_t)round_away8(xs[i] * id) & 0xFFu) << (8 * i);
    *out = packed;
    *D = (float)(_Float16)d;
    return true;
}

__device__ __forceinline__ uint32_t qact_a32_lane(const float4 v, float * D) {
    {
        uint32_t r;
        if (__builtin_expect(qact_a32_lane_fast(v, &r, D), 1)) return r;
    }
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
    // With amax >= 2^-60 (or Inf) the plain product rounds to the same integer as FM: a subnormal x
    // gives |x id| < 2^-59 (-> 0, as DAZ), a subnormal product also rounds to 0, NaN -> 0 either way.
    float pr[4];
    if (m >= 0x21800000u) {                                     // uniform within the 8-lane group
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = xs[i] * id;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = smul(xs[i], id);
    }
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed |= ((uint32_t)round_away8(pr[i]) & 0xFFu) << (8 * i);
    *D = h2f_exact(f2h_exact(d));
    return packed;
}

// Wave-wide maximum of an unsigned value (every lane gets it).
__device__ __forceinline__ uint32_t wave_umax(uint32_t m) {
    m = umax_u(m, (uint32_t)dpp_i<kDppXor1>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppXor2>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppRowHalfMirror>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppRowMirror>((int)m));
    m = umax_u(m, (uint32_t)xor16_i((int)m));
    return umax_u((uint32_t)__builtin_amdgcn_readlane((int)m, 0), (uint32_t)__builtin_amdgcn_readlane((int)m, 32));
}

// Shared steps of A256 (sw/sim/tsr_ref.c:485-520):
// - the NaN-excluded magnitude maximum as an integer maximum of |x| bits (a NaN counts as 0). A
//   subnormal maximum means every value is zero or subnormal, i.e. zero after DAZ, so the DAZ is
//   applied to the maximum only (normal magnitudes compare above subnormal ones as integers);
// - the first element of a lane whose magnitude equals the maximum (a reverse select pass);
// - q = round_half_even(iscale x) saturated to int8: v_rndne, v_cvt_i32 (NaN -> 0, saturating),
//   integer clamp; four quants packed with v_perm, their sum with v_dot4 against ones.
__device__ __forceinline__ uint32_t a256_mag_max(const float * xs, int n) {
    uint32_t m = 0;
    for (int i = 0; i < n; ++i) {
        const uint32_t a = fb(xs[i]) & 0x7FFFFFFFu;
        m = umax_u(m, a > 0x7F800000u ? 0u : a);
    }
    return m;
}
__device__ __forceinline__ float a256_first_of(const float * xs, int n, uint32_t amax) {
    float best = 0.0f;
    for (int i = n - 1; i >= 0; --i) best = (fb(xs[i]) & 0x7FFFFFFFu) == amax ? xs[i] : best;
    return best;
}
__device__ __forceinline__ uint32_t pack4_i8(int32_t q0, int32_t q1, int32_t q2, int32_t q3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0C0C0400u);   // q0.b0 q1.b0 0 0
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x0C0C0400u);   // q2.b0 q3.b0 0 0
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);                                    // lo.b0 lo.b1 hi.b0 hi.b1
}

// One A256 block held by a whole wave (lane l: values 4l .. 4l+3). Returns this lane's 4 quants
// packed; *d = the block's d (every lane); *sum4 = the sum of this lane's 4 quants; *tiny =
// 0 < |d| < 2^-60. First largest |x|: the lowest lane holding the maximum (its own first), read
// with one readlane. The plain product iscale x rounds like FM(iscale, x) when amax >= 2^-60 (see
// qact_a32_lane); below that the spec operation is used.
__device__ __forceinline__ uint32_t qact_a256_wave(const float4 v, float * d, int * sum4, bool * tiny) {
    const float xs[4] = { v.x, v.y, v.z, v.w };
    const uint32_t m = a256_mag_max(xs, 4);
    uint32_t amax = wave_umax(m);
    amax = amax < 0x00800000u ? 0u : amax;
    const float best = a256_first_of(xs, 4, amax);
    const uint64_t hold = __ballot(m == amax && amax != 0u);
    const float mx = hold ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best), __builtin_ctzll(hold))) : 0.0f;
    const bool zero = amax == 0u;
    const float iscale = zero ? 0.0f : sdiv(-127.0f, mx);
    int32_t q[4];
    if (zero || amax >= 0x21800000u) {                            // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = round_even8(iscale * xs[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = round_even8(smul(iscale, xs[i]));
    }
    const uint32_t packed = pack4_i8(q[0], q[1], q[2], q[3]);
    const float dd = zero ? 0.0f : srcp(iscale);
    const uint32_t ad = fb(dd) & 0x7FFFFFFFu;
    *d = dd;
    *sum4 = dot4((int)packed, 0x01010101, 0);
    *tiny = ad != 0u && ad < 0x21800000u;
    return packed;
}

// Max / min / or over an aligned 16-lane row (every lane of the row gets the result).
__device__ __forceinline__ uint32_t row16_umax(uint32_t m) {
    m = umax_u(m, (uint32_t)dpp_i<kDppXor1>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppXor2>((int)m));
    m = umax_u(m, (uint32_t)dpp_i<kDppRowHalfMirror>((int)m));
    return umax_u(m, (uint32_t)dpp_i<kDppRowMirror>((int)m));
}
__device__ __forceinline__ uint32_t row16_umin(uint32_t m) {
    m = min(m, (uint32_t)dpp_i<kDppXor1>((int)m));
    m = min(m, (uint32_t)dpp_i<kDppXor2>((int)m));
    m = min(m, (uint32_t)dpp_i<kDppRowHalfMirror>((int)m));
    return min(m, (uint32_t)dpp_i<kDppRowMirror>((int)m));
}
__device__ __forceinline__ uint32_t row16_or(uint32_t m) {
    m |= (uint32_t)dpp_i<kDppXor1>((int)m);
    m |= (uint32_t)dpp_i<kDppXor2>((int)m);
    m |= (uint32_t)dpp_i<kDppRowHalfMirror>((int)m);
    return m | (uint32_t)dpp_i<kDppRowMirror>((int)m);
}

// The common case of qact_a256_row in about a third of its instructions: a wave whose 64 lanes hold
// only finite values, in whose rows amax is 0 or >= 2^-60, and whose rows' values of magnitude amax
// all have one sign (the first largest is then any of them). A lane's largest positive and largest
// negative magnitudes are a signed and an unsigned maximum of the raw bits; the quant of y = iscale x
// (|y| <= 127 (1 + 2^-23)^2) is the low byte of the bits of y + 1.5 2^23, an f32 sum in [2^23, 2^24)
// rounded to the integer nearest y, ties to even (1.5 2^23 is even), which is round_even8(y).
// Returns false, wave-uniformly, when the wave does not qualify; the general form then runs.
__device__ __forceinline__ bool qact_a256_row_fast(const float4 (&v)[4], uint4 * out, float * d, int * s16,
                                                   bool * tiny) {
    float xs[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) { xs[4 * i] = v[i].x; xs[4 * i + 1] = v[i].y; xs[4 * i + 2] = v[i].z; xs[4 * i + 3] = v[i].w; }
    int32_t ps[8];
    uint32_t ns[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ps[i] = max((int32_t)fb(xs[2 * i]), (int32_t)fb(xs[2 * i + 1]));
        ns[i] = max(fb(xs[2 * i]), fb(xs[2 * i + 1]));
    }
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1) {
#pragma unroll
        for (int i = 0; i < w; ++i) { ps[i] = max(ps[i], ps[i + w]); ns[i] = max(ns[i], ns[i + w]); }
    }
    const uint32_t pm = ps[0] >= 0 ? (uint32_t)ps[0] : 0u;                 // largest positive magnitude
    const uint32_t nm = ns[0] >= 0x80000000u ? (ns[0] & 0x7FFFFFFFu) : 0u;  // largest negative magnitude
    const uint32_t m = umax_u(pm, nm);
    if (__ballot(m >= 0x7F800000u) != 0ull) return false;                 // Inf or NaN in the wave
    uint32_t amax = row16_umax(m);
    amax = amax < 0x00800000u ? 0u : amax;
    const bool zero = amax == 0u;
    if (__ballot(!zero && amax < 0x21800000u) != 0ull) return false;      // FM products
    const uint32_t sg = row16_or(zero ? 0u : ((pm == amax ? 1u : 0u) | (nm == amax ? 2u : 0u)));
    if (__ballot(sg == 3u) != 0ull) return false;                         // +amax and -amax in a row
    const float mx = bf(amax | (sg == 2u ? 0x80000000u : 0u));
    const float iscale = zero ? 0.0f : -127.0f / mx;                      // = sdiv: both normal
    uint32_t pk[4];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = fb(iscale * xs[4 * i + j] + 12582912.0f);
        pk[i] = pack4_i8((int32_t)t[0], (int32_t)t[1], (int32_t)t[2], (int32_t)t[3]);
        s = dot4((int)pk[i], 0x01010101, s);
    }
    const float dd = zero ? 0.0f : 1.0f / iscale;                         // = srcp: both normal
    const uint32_t ad = fb(dd) & 0x7FFFFFFFu;
    *d = dd;
    *s16 = s;
    *tiny = ad != 0u && ad < 0x21800000u;
    *out = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    return true;
}

// One A256 block held by an aligned 16-lane row: lane i of the row holds values 16 i .. 16 i + 15
// (v[0..3]); the four rows of a wave quantize four blocks at once. Every lane of the wave must be
// active. Returns the lane's 16 quants (bytes in value order); *d = the block's d (every lane of
// the row); *s16 = the sum of the lane's 16 quants; *tiny = 0 < |d| < 2^-60.
// First largest |x|: the row maximum of the lane maxima, then the lowest lane of the row holding it
// (its own first largest), fetched with an OR over the row (every other lane contributes 0).
// The plain product iscale x rounds like FM(iscale, x) when the block's amax >= 2^-60 (see
// qact_a32_lane); if any row of the wave has 0 < amax < 2^-60 the whole wave uses FM.
__device__ __forceinline__ uint4 qact_a256_row(const float4 (&v)[4], float * d, int * s16, bool * tiny) {
    {
        uint4 r;
        if (__builtin_expect(qact_a256_row_fast(v, &r, d, s16, tiny), 1)) return r;
    }
    float xs[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) { xs[4 * i] = v[i].x; xs[4 * i + 1] = v[i].y; xs[4 * i + 2] = v[i].z; xs[4 * i + 3] = v[i].w; }
    const uint32_t m = a256_mag_max(xs, 16);
    uint32_t amax = row16_umax(m);
    amax = amax < 0x00800000u ? 0u : amax;
    const float best = a256_first_of(xs, 16, amax);
    const uint32_t l16 = __lane_id() & 15u;
    const uint32_t win = row16_umin(m == amax && amax != 0u ? l16 : 16u);
    const float mx = bf(row16_or(l16 == win ? fb(best) : 0u));
    const bool zero = amax == 0u;
    const bool exact = __ballot(!zero && amax < 0x21800000u) != 0ull;   // wave-uniform
    const float iscale = zero ? 0.0f : sdiv(-127.0f, mx);
    int32_t q[16];
    if (!exact) {
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = round_even8(iscale * xs[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = round_even8(smul(iscale, xs[i]));
    }
    uint32_t pk[4];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pk[i] = pack4_i8(q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]);
        s = dot4((int)pk[i], 0x01010101, s);
    }
    const float dd = zero ? 0.0f : srcp(iscale);
    const uint32_t ad = fb(dd) & 0x7FFFFFFFu;
    *d = dd;
    *s16 = s;
    *tiny = ad != 0u && ad < 0x21800000u;
    return make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

}  // namespace tsr
