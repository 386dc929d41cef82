// fa_common.hpp -- device helpers shared by the FLASH_ATTN_EXT kernels (k_attn.hip, k_fa_dec.hip):
// MAXT and its order-preserving key, wave reductions, the block-float conversions of ATTPV and the
// agent-coherent accesses through which workgroups of one launch exchange data.
#pragma once

#include "qact.hpp"
#include "tsr_dev.hpp"

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

// CTREE over 4 channel partials. Row sums (ctree4_l): every segment row sum is +0, at least 2^-126
// (its largest p, a normal EXPK value, enters LSUM as an integer >= 2^23 times 2^(E - 23)), +Inf or the
// canonical NaN, and sums of such non-negative values never reach the subnormal range, never form
// Inf - Inf and keep the canonical NaN: the plain additions are the rule's (so are the row-sum chains
// over segments, plain additions as well).
// Output partials (ctree4_o) can be tiny: FTZ at every step, the NaN payload canonicalized where the
// merged output is stored.
__device__ __forceinline__ float ctree4_l(float x0, float x1, float x2, float x3) { return (x0 + x1) + (x2 + x3); }
__device__ __forceinline__ float ctree4_o(float x0, float x1, float x2, float x3) { return sadd_z(sadd_z(x0, x1), sadd_z(x2, x3)); }
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
__device__ __forceinline__ float2 ld_co2(const float * p) {      // 8-byte aligned p
    const uint64_t v = __hip_atomic_load((uint64_t *)const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(bf((uint32_t)v), bf((uint32_t)(v >> 32)));
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

}  // namespace tsr
