// tsr_dev.hpp -- device helpers shared by the gfx950 kernels: the spec's f32 rules, exact
// conversions, QACT rounding and wavefront (wave64) exchange primitives.
//
// f32 rules (sw/sim/tsr_ref.c:54-104; docs/spec.md:1405-1418): inputs with a zero exponent field
// are signed zeros (DAZ), the operation is one IEEE binary32 RNE operation with gradual underflow,
// a subnormal result becomes a signed zero (FTZ) and any NaN result 0x7FC00000. The kernels are
// compiled with -ffp-contract=off (no FMA fusion) and run with f32 denormals enabled, so the native
// operation is the gradual-underflow result the rule post-processes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsr {

constexpr uint32_t kNaN = 0x7FC00000u;
constexpr uint32_t kNegInf = 0xFF800000u;

__device__ __forceinline__ uint32_t fb(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bf(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ float daz(float x) {
    const uint32_t u = fb(x);
    return (u & 0x7F800000u) ? x : bf(u & 0x80000000u);
}
// Written as selects (no early returns) so that it compiles to straight-line code.
__device__ __forceinline__ float fin(float r) {
    const uint32_t u = fb(r), e = u & 0x7F800000u;
    const uint32_t nan = (e == 0x7F800000u && (u & 0x007FFFFFu)) ? kNaN : u;
    return bf(e == 0u ? (u & 0x80000000u) : nan);
}
// NaN -> canonical only (results that cannot be subnormal).
__device__ __forceinline__ float canon(float r) { return __builtin_amdgcn_classf(r, 0x3) ? bf(kNaN) : r; }
// FTZ only (a NaN keeps the payload the operation gave it): for chains whose values are canonicalized
// where they leave the chain, since every later IEEE operation keeps a NaN a NaN.
__device__ __forceinline__ float ftz(float r) { return __builtin_amdgcn_classf(r, 0x90) ? bf(fb(r) & 0x80000000u) : r; }

__device__ __forceinline__ float sadd(float a, float b) { return fin(daz(a) + daz(b)); }
__device__ __forceinline__ float ssub(float a, float b) { return fin(daz(a) - daz(b)); }
__device__ __forceinline__ float smul(float a, float b) { return fin(daz(a) * daz(b)); }
__device__ __forceinline__ float sdiv(float a, float b) { return fin(daz(a) / daz(b)); }
__device__ __forceinline__ float srcp(float a) { return fin(1.0f / daz(a)); }

// The same rule for operands that cannot be subnormal (results of earlier rule operations, EXPK
// values, block-float values, scores): DAZ is then the identity and only the result needs FTZ and
// NaN canonicalization, each tested with one v_cmp_class (mask 0x90: -/+ subnormal; 0x3: NaN).
__device__ __forceinline__ float fin_n(float r) {
    const uint32_t u = fb(r);
    const uint32_t o = __builtin_amdgcn_classf(r, 0x90) ? (u & 0x80000000u) : u;
    return bf(__builtin_amdgcn_classf(r, 0x3) ? kNaN : o);
}
__device__ __forceinline__ float sadd_n(float a, float b) { return fin_n(a + b); }
__device__ __forceinline__ float ssub_n(float a, float b) { return fin_n(a - b); }
__device__ __forceinline__ float smul_n(float a, float b) { return fin_n(a * b); }
// The two halves of that rule where the other half provably changes nothing: _c when the result can
// never be subnormal (canonical NaN kept), _z inside a chain that is canonicalized where it ends.
__device__ __forceinline__ float sadd_c(float a, float b) { return canon(a + b); }
__device__ __forceinline__ float smul_c(float a, float b) { return canon(a * b); }
__device__ __forceinline__ float sadd_z(float a, float b) { return ftz(a + b); }
__device__ __forceinline__ float smul_z(float a, float b) { return ftz(a * b); }

// int32 -> f32 RNE (v_cvt_f32_i32 rounds to nearest even).
__device__ __forceinline__ float i2f(int32_t v) { return (float)v; }

// fp16 bits -> f32, exact for every input; a NaN keeps sign and payload with the quiet bit set
// (sw/sim/tsr_ref.c:136-160).
__device__ __forceinline__ float h2f_exact(uint32_t h) {
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31u) return bf(s | 0x7F800000u | (m ? (0x00400000u | (m << 13)) : 0u));
    if (e == 0u) return bf(s | fb((float)m * 5.9604644775390625e-08f));
    return bf(s | ((e + 112u) << 23) | (m << 13));
}
// fp16 -> f32 by the hardware conversion: exact for every non-NaN input (f16 denormals enabled).
// Used for weight scales in the hot loops, where any NaN is canonicalized by a later f32 op.
__device__ __forceinline__ float h2f_fast(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// f32 -> fp16 bits, RNE, overflow -> Inf, NaN -> sign | 0x7E00 (sw/sim/tsr_ref.c:162-198).
__device__ __forceinline__ uint32_t f2h_exact(float f) {
    const uint32_t u = fb(f), s = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return s | 0x7E00u;
    if (a == 0x7F800000u) return s | 0x7C00u;
    const int be = (int)(a >> 23);
    if (be == 0) return s;
    const int e = be - 127;
    if (e > 15) return s | 0x7C00u;
    if (e < -25) return s;
    const uint32_t sig = 0x00800000u | (a & 0x007FFFFFu);
    const uint32_t rs = e >= -14 ? 13u : (uint32_t)(-e - 1);   // 13 .. 24
    uint32_t q = sig >> rs;
    const uint32_t rem = sig & ((1u << rs) - 1u), half = 1u << (rs - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    const uint32_t out = e >= -14 ? ((uint32_t)(e + 15) << 10) + (q - 1024u) : q;
    return s | out;
}

// QACT f32 -> int8: NaN -> 0; |x| >= 256 saturates; else round (half away: A32, half even: A256)
// and clamp to [-128, 127] (sw/sim/tsr_ref.c:200-232).
// v_cvt_i32_f32 converts NaN to 0 and saturates out-of-range values (Inf included) to INT_MIN /
// INT_MAX; the integer clamp then gives the int8 saturation. Written in asm because a C++
// float-to-int conversion of NaN or of an out-of-range value is undefined.
__device__ __forceinline__ int32_t cvt_i32_sat(float x) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
__device__ __forceinline__ int32_t clamp8(int32_t v) { return min(max(v, -128), 127); }
__device__ __forceinline__ int32_t round_away8(float x) {
    const float t = __builtin_truncf(x);
    const float fr = x - t;                                   // exact; NaN for NaN and Inf inputs
    const float up = __builtin_fabsf(fr) >= 0.5f ? __builtin_copysignf(1.0f, x) : 0.0f;
    return clamp8(cvt_i32_sat(t + up));                       // NaN -> 0, +-Inf -> 127 / -128
}
__device__ __forceinline__ int32_t round_even8(float x) {
    return clamp8(cvt_i32_sat(__builtin_rintf(x)));          // rintf: ties to even
}

// ---- wave64 exchange ----------------------------------------------------------------------------
// DPP controls (GCN/CDNA encoding).
constexpr int kDppXor1 = 0xB1;            // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;            // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- 7 - i within each 8
constexpr int kDppRowMirror = 0x140;      // lane i <- 15 - i within each 16

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Lane i <- lane i ^ 16 (within 32-lane halves) and lane i <- lane i ^ 32.
__device__ __forceinline__ int xor16_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }
__device__ __forceinline__ float xor16_f(float v) { return __int_as_float(xor16_i(__float_as_int(v))); }
__device__ __forceinline__ int xor32_i(int v) {
    return __builtin_amdgcn_ds_bpermute(((int)__lane_id() ^ 32) << 2, v);
}
__device__ __forceinline__ float xor32_f(float v) { return __int_as_float(xor32_i(__float_as_int(v))); }
__device__ __forceinline__ int shfl_i(int v, int src_lane) { return __builtin_amdgcn_ds_bpermute(src_lane << 2, v); }
__device__ __forceinline__ float shfl_f(float v, int src_lane) { return __int_as_float(shfl_i(__float_as_int(v), src_lane)); }

// Sum over the 8 lanes of an aligned group of 8 (every lane gets the total). Integer: exact in any order.
__device__ __forceinline__ int sum8_i(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppRowHalfMirror>(v);
    return v;
}

// Byte-wise signed dot product of 4 int8 pairs plus an accumulator (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Workgroup barrier that orders LDS only. It waits for this wave's LDS (and scalar) operations
// (s_waitcnt lgkmcnt(0); the vmcnt and expcnt fields are left at their maxima), then s_barrier.
// Global loads still in flight stay in flight: __syncthreads() is a release/acquire fence and
// waits for every outstanding vector-memory operation first, which would serialize a kernel's
// compute behind its whole weight stream. The signal fences keep the compiler from moving memory
// operations across the barrier. Use it only where the barrier publishes LDS data.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace tsr
