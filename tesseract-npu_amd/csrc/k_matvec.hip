// k_matvec.hip -- decode MUL_MAT (matrix-vector) kernels for Q8_0 and Q4_K weights on gfx950.
//
// Numerics (sw/sim/tsr_ref.c:525-635; docs/spec.md:438-477): per row, the term of block (Q8_0) or
// super-block (Q4_K) s is added into partial p[s mod 16] in order of s, then y = ((p0+p1)+(p2+p3))+...
// (the 16-partial tree). Q8_0 term = (d Dx) f32(isum); Q4_K term = (d Dx) f32(isum) -
// (dmin Dx) f32(msum) with isum = sum_j sc_j S_j and msum = sum_j m_j (bs[2j] + bs[2j+1]).
//
// Work split. A workgroup of 16 waves owns one row block of the weight layout (wlayout.hpp: rb
// consecutive rows); wave w computes the terms of the blocks s = w + 16 k (the blocks of partial
// p[w]) of every row in the block. The layout stores exactly these units (slot, row) of a wave
// contiguously, so a wave load reads one run of up to 1 KiB and a workgroup reads one contiguous
// region (measured: the same bytes in runs of 256 bytes 32 KiB apart take ~25 % longer to stream
// than in contiguous runs of 1 KiB). A lane computes a whole term: the integer
// sums stay in its registers and need no cross-lane reduction. Each wave quantizes the blocks of x
// it uses (QACT into its own LDS area), so no workgroup barrier separates the weight stream from
// the compute. The terms go to LDS; after the only barriers, the partials are summed in the order
// of s and the tree runs once per row.
//
// Fast and exact f32 paths. With f32 denormals on and no FMA contraction, plain IEEE operations give
// the spec result whenever no operand or result is subnormal; NaN payloads are the only other
// difference and the stored y is canonicalized. A term is (d Dx) f32(int) [- (dmin Dx) f32(int)]
// with d, dmin fp16 values (0 or >= 2^-24 in magnitude) and Dx an fp16 value (A32) or, for A256,
// any f32. When every nonzero |Dx| >= 2^-60, every product d Dx is 0 or a normal multiple of
// 2^-107, and so is every term and every sum of terms: nothing is ever subnormal. A wave that
// quantizes a block with 0 < |Dx| < 2^-60 computes its terms with the spec operations, and then the
// partial sums and the tree of the workgroup do too.
#include "expk.hpp"
#include "glue.hpp"
#include "kernels.hpp"
#include "mv_q4k.hpp"
#include "qact.hpp"
#include "tsr_hip.h"
#include "wlayout.hpp"

#include <algorithm>

namespace tsr {

constexpr int kMvWaves = 16;

// Partial p[w] of every row of the workgroup, by wave w from its own terms in LDS (s_t[row][s], nb
// terms per row): p = ((+0 + t_w) + t_w+16) + ... in order of s. The same wave wrote those terms,
// and the LDS executes one wave's operations in order, so no workgroup barrier is needed here.
__device__ __forceinline__ void mv_wave_partials(const WGeom & g, const float * s_t, float * s_p, uint32_t nrow,
                                                 uint32_t w, bool slow) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t cw = wl_count(g, w);
    for (uint32_t rl = __lane_id(); rl < nrow; rl += 64u) {
        const float * tr = s_t + (size_t)rl * g.nb + w;
        float p = 0.0f;
        if (__builtin_expect(!slow, 1)) {
            for (uint32_t k = 0; k < cw; ++k) p = p + tr[16u * k];
        } else {
            for (uint32_t k = 0; k < cw; ++k) p = sadd(p, tr[16u * k]);
        }
        s_p[16u * rl + w] = p;
    }
}

// After a workgroup barrier: the 16-partial tree of each row on an aligned 16-lane row of threads
// (lane i holds p[i]; the DPP pairs xor 1, xor 2, half mirror, mirror are the tree's pairs, and
// f32 addition is commutative), then y. Every thread of the workgroup calls it. add0: the addend of
// the thread's row in the first round (loaded early by the caller; used when a.add is set).
// GLU: weight rows 2j and 2j + 1 are the gate and up rows of output j (the workgroup's row block starts
// at an even row and holds whole pairs). The row results go to s_y (LDS, nrow floats, free after the
// partials), and after a barrier one thread per output forms y[j] = SWIGLU(gate, up) -- the
// GGML_GLU_OP_SWIGLU that follows the gate and up MUL_MATs -- on whole waves (64 outputs per wave, so
// that the EXPK table lookup, a cross-lane read, runs with every lane active). t64: lane j holds the
// EXPK table entry j.
template <bool GLU>
__device__ __forceinline__ void mv_tree_store(const MvArgs & a, const float * s_p, float * s_y, uint32_t nrow,
                                              uint32_t row_lo, uint32_t t, bool slow, uint32_t t64, float add0) {
    for (uint32_t base = 0; base < nrow * 16u; base += blockDim.x) {   // uniform trip count
        const uint32_t idx = base + threadIdx.x, rl = idx >> 4;
        float v = rl < nrow ? s_p[idx] : 0.0f;
        if (__builtin_expect(!slow, 1)) {
            v = v + dpp_f<kDppXor1>(v);
            v = v + dpp_f<kDppXor2>(v);
            v = v + dpp_f<kDppRowHalfMirror>(v);
            v = v + dpp_f<kDppRowMirror>(v);
            v = canon(v);
        } else {
            v = sadd(v, dpp_f<kDppXor1>(v));
            v = sadd(v, dpp_f<kDppXor2>(v));
            v = sadd(v, dpp_f<kDppRowHalfMirror>(v));
            v = sadd(v, dpp_f<kDppRowMirror>(v));
        }
        if ((idx & 15u) == 0u && rl < nrow) {
            if constexpr (GLU) {
                s_y[rl] = v;
            } else {
                float * yp = a.y + (size_t)t * a.y_stride + row_lo + rl;
                if (a.add) v = sadd(base == 0u ? add0 : a.add[(size_t)t * a.add_stride + row_lo + rl], v);
                else if (a.acc) v = sadd(*yp, v);
                *yp = v;
            }
        }
    }
    if constexpr (GLU) {
        lds_barrier();
        const uint32_t nout = nrow >> 1, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        for (uint32_t j0 = 64u * w; j0 < nout; j0 += blockDim.x) {   // whole waves
            const uint32_t j = j0 + __lane_id(), jc = min(j, nout - 1u);
            const float h = swiglu_reg(s_y[2u * jc], s_y[2u * jc + 1u], a.ex, t64);
            if (j < nout) a.y[(size_t)t * a.y_stride + (row_lo >> 1) + j] = h;
        }
    }
}

// Every wave's x requests enter the compute unit's memory queue before any weight request of the
// workgroup. The queue serves vector-memory requests in order, so an x load issued behind the
// weight loads of other waves would return only after them (measured: up to 5 us into a 9 us
// launch). A bare s_barrier orders the issue without waiting for any load.
__device__ __forceinline__ void x_first_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// The unit of lane `lane` in pass p: unit u = 64 p + lane of the wave's R cnt units (slot-major:
// slot k = u / R, row u % R of the block). Units beyond the last, and every unit of a wave without
// blocks (cnt == 0), load the last unit's address (a valid one) and are not used.
struct MvUnit {
    uint32_t k, r;
    bool valid;
};
__device__ __forceinline__ MvUnit mv_unit(uint32_t p, int lane, uint32_t R, uint32_t nunit) {
    const uint32_t u = 64u * p + (uint32_t)lane;
    const uint32_t uc = min(u, (nunit ? nunit : 1u) - 1u);
    MvUnit m;
    m.k = uc / R;
    m.r = uc - m.k * R;
    m.valid = u < nunit;
    return m;
}

// ---- fused x preparation (MvArgs::prep) and GLU epilogue -------------------------------------------
// kPrepNorm: every wave squares the x values it loaded (FM(x, x)) into s_sq at their index; after an
// LDS barrier threads 0 .. 127 run the 128 RED partials in order and the tree (glue.hpp), thread 0
// forms the scale s, and after another barrier every wave turns its values into FM(FM(x, s), pw) --
// exactly RMS_NORM + MUL, before QACT. Launched only when every value of x is loaded by some wave in
// the first round (K <= 8192, the host checks), so s_sq is complete. The loads of x and pw are
// straight-line with compile-time indices, issued before the weight stream, and the preparation
// waits only for them (prep_norm_apply and its fast form: mv_q4k.hpp).

// LDS flags between the waves of one workgroup (all resident together). A writer makes its earlier LDS
// writes complete (lgkmcnt(0)) before it writes the flag; a reader polls the flag with volatile LDS
// loads, then reads the data (the LDS executes one wave's operations in order). The polls are bounded
// (every wait ends): a flag that never comes lets the kernel finish with wrong values, never hang.
constexpr uint32_t kLdsSpinMax = 1u << 22;
__device__ __forceinline__ void lds_wait_writes() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);                           // lgkmcnt(0); vmcnt and expcnt untouched
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// (Relaxed workgroup-scope atomics on a static __shared__ array: plain ds_read / ds_write, which count
// on lgkmcnt only. A volatile access through a generic pointer would be a flat load that also waits
// for every outstanding vector-memory load.)
__device__ __forceinline__ uint32_t lds_ld(const uint32_t * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(uint32_t * p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_flag_set(uint32_t * f, uint32_t v) {
    lds_wait_writes();
    lds_st(f, v);
}
__device__ __forceinline__ void lds_flag_wait(const uint32_t * f, uint32_t want) {
    for (uint32_t n = 0; n < kLdsSpinMax; ++n) {
        if (lds_ld(f) >= want) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The RMS scale from s_sq[0 .. K): every thread of the workgroup calls it (three LDS barriers inside);
// returns s in every thread. s_sq[K] and s_sq[K + 1] are the exchange slots.
__device__ __forceinline__ float prep_norm_scale(float * s_sq, uint32_t K, float inv_n, float eps) {
    lds_barrier();
    float p = 0.0f;
    if (threadIdx.x < 128u) {                                     // plain additions: see rms_tree64
        // every partial has ceil((K - i) / 128) terms; reads at clamped indices, selects on the count
        for (uint32_t j0 = 0; j0 < K; j0 += 128u * 32u) {
            float v[32];
#pragma unroll
            for (uint32_t k = 0; k < 32u; ++k) v[k] = s_sq[min(j0 + threadIdx.x + 128u * k, K - 1u)];
#pragma unroll
            for (uint32_t k = 0; k < 32u; ++k) {
                const float q = p + v[k];
                p = j0 + threadIdx.x + 128u * k < K ? q : p;
            }
        }
        p = rms_tree64(p);
        if (threadIdx.x == 64u) s_sq[K + 1u] = p;
    }
    lds_barrier();
    if (threadIdx.x == 0u) s_sq[K] = rms_scale(p, s_sq[K + 1u], inv_n, eps);
    lds_barrier();
    return s_sq[K];
}

// ---------------------------------------------------------------------------------------------
// Q4_K. LDS: x quants [16 areas][kx][272 B] | sub-block sums [16][kx][8] int | d [16][kx] |
// terms [rb][nsb] | partials [rb][16] | 16 words | kPrepNorm: K squares + 2 slots.
// Block s of x lives in area s mod 16 at index s / 16 (area w holds the blocks of partial p[w]).
// Lane unit = (row, super-block): 8 quant pieces (piece j: group g = j / 2, low nibbles = values
// 64g + 16 (j % 2) + 0..15, high nibbles = the same + 32) and one meta piece. F adjacent lanes share
// a unit when a wave has few units (F = 4: at most 16, F = 2: at most 32): lane q of the F loads
// pieces (8/F) q .. (8/F)(q + 1) - 1 and the meta, computes the integer sums of its sub-blocks, and
// the F lanes add them by DPP (integer sums: exact in any order). A wave instruction then carries
// 64 lanes of work instead of 64/F.
//
// x: the leader waves (the first 4 or 8) load x before any weight load of the workgroup (round r:
// the 16-lane row h of a leader holds block 16r + 4 (v mod 4) + h, lane i of the row its values
// 16i .. 16i + 15), apply the fused RMS_NORM (kPrepNorm: squares into LDS, the two halves of the 128
// ordered partials on leaders 0 and 1, the scale through LDS flags), quantize every block (QACT
// A256, 16-lane-row form: four blocks per wave) into LDS; a workgroup barrier then publishes x to every wave.
// Every wave, leaders included, issues its weight loads before that barrier. Vector-memory counters retire in order, so a leader's wait for x must never cover a
// weight load: its x loads precede its weight loads, and their number is the same on every path
// (measured: when the count differed between paths the compiler's join waited for the weights too,
// and the quantization ended 1.8 us after x had arrived instead of 0.3 us). The x of the oldest
// waves also returns first when the compute unit's requests queue behind the weight stream.
// ---------------------------------------------------------------------------------------------
// Unit of lane slot ul in pass p when every pass covers upw units: u = upw p + ul (slot-major as in
// mv_unit).
__device__ __forceinline__ MvUnit mv_unit_f(uint32_t p, uint32_t ul, uint32_t upw, uint32_t R, uint32_t nunit) {
    const uint32_t u = upw * p + ul;
    const uint32_t uc = min(u, (nunit ? nunit : 1u) - 1u);
    MvUnit m;
    m.k = uc / R;
    m.r = uc - m.k * R;
    m.valid = u < nunit;
    return m;
}

template <int F, bool ISUMS, int PREP, bool GLU>
__global__ __launch_bounds__(1024) void k_mv_q4k(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t UPW = 64u / (uint32_t)F, NP = 8u / (uint32_t)F;   // units per pass, pieces per lane
    const WGeom g = wgeom(a.N, a.K >> 8, a.rb, true);
    const uint32_t nsb = g.nb, kx = g.q + (g.rem ? 1u : 0u);
    const int lane = (int)__lane_id();
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), cnt = wl_count(g, w);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;
    const uint32_t B = blockIdx.x, row_lo = B * g.rb, nrow = wl_rows(g, B);
    const uint32_t nunit = nrow * cnt, npass = (nunit + UPW - 1u) / UPW;
    int8_t * s_xq = (int8_t *)lds;
    int * s_xb = (int *)(lds + kMvWaves * kx * kXq4Stride);
    float * s_xd = (float *)(s_xb + kMvWaves * kx * 8u);
    float * s_t = s_xd + kMvWaves * kx;
    float * s_p = s_t + ((a.rb * nsb + 3u) & ~3u);                // 16-byte aligned
    float * s_sq = (float *)((int *)(s_p + a.rb * 16u) + 16);     // kPrepNorm: K squares + 2 slots
    // 0 leaders with squares stored, 1 halves of the RMS sum stored, 3 lo half, 4 hi half,
    // 5 leaders with quants stored (no norm), 6 some block has 0 < |d| < 2^-60
    __shared__ uint32_t s_ctl[8];

    // Leaders: NL = 4 nlg waves; leader v handles the rounds r = v / 4 + nlg i (i = 0, 1, ...), its row h
    // block 16 r + 4 (v mod 4) + h. The first RPL rounds of a leader are loaded before any weight load
    // (unconditionally, at clamped addresses, so that every path has the same count of loads in flight
    // and the waits for x never include a weight load); later rounds (K > 16384 only) after them.
    constexpr uint32_t RPL = PREP == kPrepNorm ? 1u : 2u;
    const uint32_t nrx = (nsb + 15u) >> 4;                        // rounds of 16 blocks
    const uint32_t nlg = PREP == kPrepNorm ? nrx : min((nrx + 1u) >> 1, 2u);   // kPrepNorm: K <= 8192
    const uint32_t nl = 4u * nlg, rg = w >> 2;
    const bool leader = w < nl;
    const uint32_t h4 = (uint32_t)lane >> 4, l16 = (uint32_t)lane & 15u;
    auto xblk = [&](uint32_t r) -> uint32_t { return 16u * r + 4u * (w & 3u) + h4; };
    auto xidx = [&](uint32_t r, uint32_t c) -> uint32_t { return 256u * min(xblk(r), nsb - 1u) + 16u * l16 + 4u * c; };
    auto load_xr = [&](uint32_t r, float4 (&xr)[4]) {
#pragma unroll
        for (uint32_t c = 0; c < 4u; ++c) xr[c] = *(const float4 *)(x + xidx(r, c));
    };
    float4 xv[RPL][4], pv[4];                                     // pv: the norm weights of the leader's round
    if (threadIdx.x < 8u) lds_st(s_ctl + threadIdx.x, 0u);
    if (leader) {
        // the norm weights first: in a decode layer they were last read a token ago and come from HBM,
        // while x was written by the launch before (layer in sequence 49.7 -> 49.0 us)
        if constexpr (PREP == kPrepNorm) {
            const float * pl = a.pw ? a.pw : x;                   // without MUL: a valid address, unused
#pragma unroll
            for (uint32_t c = 0; c < 4u; ++c) pv[c] = *(const float4 *)(pl + xidx(rg, c));
        }
#pragma unroll
        for (uint32_t i = 0; i < RPL; ++i) load_xr(rg + nlg * i, xv[i]);
    }
    uint32_t t64 = 0;
    if constexpr (GLU) t64 = a.ex.t64[lane];
    lds_wait_writes();                                            // the cleared flags before the barrier
    x_first_barrier();

    const uint32_t q = (uint32_t)lane % (uint32_t)F, ul = (uint32_t)lane / (uint32_t)F;
    // pass p's loads (the unit clamped to the last: a pass beyond the wave's units loads a valid address)
    auto loadp = [&](uint32_t p, uint4 (&qv)[NP], uint4 & mv) {
        const MvUnit m = mv_unit_f(p, ul, UPW, nrow, nunit);
        const uint32_t sl = min(wl_slot(g, w, m.k), nsb - 1u);
#pragma unroll
        for (uint32_t jj = 0; jj < NP; ++jj) qv[jj] = *(const uint4 *)(a.w + wl_quant_off(g, B, nrow, NP * q + jj, sl, m.r));
        mv = *(const uint4 *)(a.w + wl_meta_off(g, B, nrow, sl, m.r));   // last: the terms use it last
    };
    uint4 qa[NP], ma;
    loadp(0u, qa, ma);
    // the addend of this thread's first stored row (tree store, first round); loaded by every thread
    // at a clamped address, so that the count of loads in flight does not depend on the call
    float add0;
    {
        const float * ap = (!GLU && a.add != nullptr) ? a.add + (size_t)t * a.add_stride + row_lo : x;
        add0 = ap[min(threadIdx.x >> 4, nrow - 1u)];
    }
    __builtin_amdgcn_sched_barrier(0);

    if (leader) {
        bool tiny_any = false;
        auto qround = [&](uint32_t r, const float4 (&xr)[4]) {
            float d;
            int s16;
            bool tiny;
            const uint4 qq = qact_a256_row(xr, &d, &s16, &tiny);
            const int s32 = s16 + dpp_i<kDppXor1>(s16);           // sum of the 32 quants of a sub-block
            const uint32_t b = xblk(r);
            if (b < nsb) {
                const uint32_t xo = (b & 15u) * kx + (b >> 4);
                *(uint4 *)(s_xq + xo * kXq4Stride + 16u * l16) = qq;
                if ((l16 & 1u) == 0u) s_xb[xo * 8u + (l16 >> 1)] = s32;
                if (l16 == 0u) s_xd[xo] = d;
                tiny_any |= tiny;
            }
        };
        if constexpr (PREP == kPrepNorm) {
            const uint32_t nk = a.K >> 7;                         // terms per partial (K % 256 == 0)
            if (xblk(rg) < nsb) {
#pragma unroll
                for (uint32_t c = 0; c < 4u; ++c) *(float4 *)(s_sq + xidx(rg, c)) = sq4(xv[0][c]);
            }
            lds_wait_writes();
            if (lane == 0) __hip_atomic_fetch_add(s_ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (w < 2u) {
                lds_flag_wait(s_ctl, nl);
                const uint32_t i = 64u * w + (uint32_t)lane;
                float p = 0.0f;
                // batches of 32 reads in flight; a full batch adds without selects
                for (uint32_t k0 = 0; k0 < nk; k0 += 32u) {
                    float v[32];
#pragma unroll
                    for (uint32_t k = 0; k < 32u; ++k) v[k] = s_sq[i + 128u * min(k0 + k, nk - 1u)];
                    if (k0 + 32u <= nk) {
#pragma unroll
                        for (uint32_t k = 0; k < 32u; ++k) p = p + v[k];   // plain additions: see rms_tree64
                    } else {
#pragma unroll
                        for (uint32_t k = 0; k < 32u; ++k) {
                            const float t = p + v[k];
                            p = k0 + k < nk ? t : p;
                        }
                    }
                }
                p = rms_tree64(p);
                if (lane == 0) lds_st(s_ctl + 3 + w, __float_as_uint(p));
                lds_wait_writes();
                if (lane == 0) __hip_atomic_fetch_add(s_ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            lds_flag_wait(s_ctl + 1, 2u);                         // both halves: every leader forms the scale
            const float sc = rms_scale(__uint_as_float(lds_ld(s_ctl + 3)), __uint_as_float(lds_ld(s_ctl + 4)),
                                       a.inv_n, a.eps);
            if (__builtin_expect(!prep_norm_apply_fast(xv[0], sc, pv, a.pw != nullptr), 0)) {
#pragma unroll
                for (uint32_t c = 0; c < 4u; ++c) xv[0][c] = prep_norm_apply(xv[0][c], sc, pv[c], a.pw != nullptr);
            }
            if (rg < nrx) qround(rg, xv[0]);
        } else {
            if (rg < nrx) qround(rg, xv[0]);
            if (rg + nlg < nrx) qround(rg + nlg, xv[RPL - 1u]);
            for (uint32_t r = rg + 2u * nlg; r < nrx; r += nlg) {  // K > 16384 only: loaded behind the weights
                float4 xr[4];
                load_xr(r, xr);
                qround(r, xr);
            }
        }
        if (__ballot(tiny_any) != 0ull && lane == 0) lds_st(s_ctl + 6, 1u);
        if constexpr (PREP != kPrepNorm) {
            lds_wait_writes();
            if (lane == 0) __hip_atomic_fetch_add(s_ctl + 5, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    // every wave waits here for the leaders' quants: with the fused norm a bare barrier (loads in flight
    // stay in flight), otherwise the leaders' count on a flag (measured at the Llama-3-8B shapes:
    // gate|up 0.6 us faster with the barrier, down 0.6 us faster with the flag)
    if constexpr (PREP == kPrepNorm) lds_barrier();
    else lds_flag_wait(s_ctl + 5, nl);
    const bool slow = lds_ld(s_ctl + 6) != 0u;                    // workgroup-uniform

    auto term = [&](uint32_t p, const uint4 (&qv)[NP], const uint4 & mv) {
        const MvUnit m = mv_unit_f(p, ul, UPW, nrow, nunit);
        const uint32_t xo = w * kx + m.k;
        const int8_t * xb = s_xq + xo * kXq4Stride;
        const int * bsp = s_xb + xo * 8u;
        const uint4 mt = mv;
        int isum, msum;
        q4k_unit_sums<NP>(qv, mt, xb, bsp, q, isum, msum);
        if constexpr (F >= 2) {
            isum += dpp_i<kDppXor1>(isum);
            msum += dpp_i<kDppXor1>(msum);
        }
        if constexpr (F >= 4) {
            isum += dpp_i<kDppXor2>(isum);
            msum += dpp_i<kDppXor2>(msum);
        }
        const float dx = s_xd[xo];
        const float d = h2f_fast(mt.x & 0xFFFFu), dm = h2f_fast(mt.x >> 16);
        float tt;
        if (__builtin_expect(!slow, 1)) tt = (d * dx) * (float)isum - (dm * dx) * (float)msum;
        else tt = ssub(smul(smul(d, dx), i2f(isum)), smul(smul(dm, dx), i2f(msum)));
        const uint32_t s = w + 16u * m.k;
        if (m.valid && q == 0u) {
            s_t[m.r * nsb + s] = tt;
            if (ISUMS && t == 0u) {
                a.isums[(size_t)(row_lo + m.r) * 2u * nsb + 2u * s] = isum;
                a.isums[(size_t)(row_lo + m.r) * 2u * nsb + 2u * s + 1u] = msum;
            }
        }
    };
    for (uint32_t p = 0; p < npass; ++p) {
        if (p) loadp(p, qa, ma);
        term(p, qa, ma);
    }
    mv_wave_partials(g, s_t, s_p, nrow, w, slow);
    lds_barrier();
    mv_tree_store<GLU>(a, s_p, s_t, nrow, row_lo, t, slow, t64, add0);
}

// ---------------------------------------------------------------------------------------------
// Q8_0. LDS: x quants [16 waves][kx][32 B] | D [16][kx] | terms [rb][nb] | partials [rb][16].
// Lane unit = (row, block): two 16-byte quant loads and the fp16 scale. The A32 activation scale is
// an fp16 value, so every term is exact with plain IEEE operations.
// ---------------------------------------------------------------------------------------------
template <int P, bool ISUMS, int PREP, bool GLU>
__global__ __launch_bounds__(1024) void k_mv_q80(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const WGeom g = wgeom(a.N, a.K >> 5, a.rb, false);
    const uint32_t nb = g.nb, kx = g.q + (g.rem ? 1u : 0u);
    const int lane = (int)__lane_id();
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), cnt = wl_count(g, w);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;
    const uint32_t B = blockIdx.x, row_lo = B * g.rb, nrow = wl_rows(g, B);
    const uint32_t nunit = nrow * cnt, npass = (nunit + 63u) >> 6;
    int8_t * s_xq = (int8_t *)lds;
    float * s_xd = (float *)(lds + kMvWaves * kx * 32u);
    float * s_t = s_xd + kMvWaves * kx;
    float * s_p = s_t + ((a.rb * nb + 3u) & ~3u);                 // 16-byte aligned
    float * s_sq = s_p + a.rb * 16u;                              // kPrepNorm: K squares + 2 slots

    // x: 8 lanes per block; round i covers blocks k = 8 i + lane / 8 of this wave
    constexpr int XP = 2;
    float4 xv[XP], pv[XP];                                        // pv: norm weights
    auto xoff = [&](uint32_t i) -> uint32_t {
        const uint32_t k = 8u * i + ((uint32_t)lane >> 3);
        return 32u * min(w + 16u * k, nb - 1u) + 4u * ((uint32_t)lane & 7u);
    };
#pragma unroll
    for (int i = 0; i < XP; ++i) xv[i] = *(const float4 *)(x + xoff((uint32_t)i));
    if constexpr (PREP == kPrepNorm) {
        const float * pl = a.pw ? a.pw : x;                       // without MUL: a valid address, unused
#pragma unroll
        for (int i = 0; i < XP; ++i) pv[i] = *(const float4 *)(pl + xoff((uint32_t)i));
    }
    uint32_t t64 = 0;
    if constexpr (GLU) t64 = a.ex.t64[lane];
    x_first_barrier();

    uint4 q0[P], q1[P];
    uint32_t dv[P];
    auto load = [&](uint32_t p0) {
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            const MvUnit m = mv_unit(min(p0 + (uint32_t)pp, npass ? npass - 1u : 0u), lane, nrow, nunit);
            const uint32_t sl = min(wl_slot(g, w, m.k), nb - 1u);
            q0[pp] = *(const uint4 *)(a.w + wl_quant_off(g, B, nrow, 0u, sl, m.r));
            q1[pp] = *(const uint4 *)(a.w + wl_quant_off(g, B, nrow, 1u, sl, m.r));
            dv[pp] = *(const uint16_t *)(a.w + wl_meta_off(g, B, nrow, sl, m.r));
        }
    };
    load(0u);                                                     // unconditional: no join before QACT
    float add0 = 0.0f;                                            // the addend of this thread's first stored row
    if constexpr (!GLU) {
        if (a.add != nullptr && (threadIdx.x & 15u) == 0u && (threadIdx.x >> 4) < nrow)
            add0 = a.add[(size_t)t * a.add_stride + row_lo + (threadIdx.x >> 4)];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PREP == kPrepNorm) {
        float4 sq[XP];
#pragma unroll
        for (int i = 0; i < XP; ++i) sq[i] = sq4(xv[i]);
#pragma unroll
        for (int i = 0; i < XP; ++i)
            if (8u * (uint32_t)i + ((uint32_t)lane >> 3) < cnt) *(float4 *)(s_sq + xoff((uint32_t)i)) = sq[i];
        const float sc = prep_norm_scale(s_sq, a.K, a.inv_n, a.eps);
#pragma unroll
        for (int i = 0; i < XP; ++i) xv[i] = prep_norm_apply(xv[i], sc, pv[i], a.pw != nullptr);
    }

    auto qact_round = [&](uint32_t i, const float4 v) {
        const uint32_t k = 8u * i + ((uint32_t)lane >> 3);
        float D;
        const uint32_t qq = qact_a32_lane(v, &D);
        if (k < cnt) {
            *(uint32_t *)(s_xq + (w * kx + k) * 32u + 4u * ((uint32_t)lane & 7u)) = qq;
            if ((lane & 7) == 0) s_xd[w * kx + k] = D;
        }
    };
#pragma unroll
    for (int i = 0; i < XP; ++i)
        if (8u * (uint32_t)i < cnt) qact_round((uint32_t)i, xv[i]);
    for (uint32_t i = XP; 8u * i < cnt; ++i)                     // K > 8192 only (never with a prep)
        qact_round(i, *(const float4 *)(x + xoff(i)));

    for (uint32_t p0 = 0; p0 < npass; p0 += P) {
        if (p0) load(p0);
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            if (p0 + (uint32_t)pp >= npass) break;
            const MvUnit m = mv_unit(p0 + (uint32_t)pp, lane, nrow, nunit);
            const uint32_t xo = w * kx + m.k;
            const int4 xa = *(const int4 *)(s_xq + xo * 32u), xb = *(const int4 *)(s_xq + xo * 32u + 16u);
            int is = dot4((int)q0[pp].x, xa.x, 0);
            is = dot4((int)q0[pp].y, xa.y, is);
            is = dot4((int)q0[pp].z, xa.z, is);
            is = dot4((int)q0[pp].w, xa.w, is);
            is = dot4((int)q1[pp].x, xb.x, is);
            is = dot4((int)q1[pp].y, xb.y, is);
            is = dot4((int)q1[pp].z, xb.z, is);
            is = dot4((int)q1[pp].w, xb.w, is);
            const float tt = (h2f_fast(dv[pp]) * s_xd[xo]) * (float)is;
            const uint32_t b = w + 16u * m.k;
            if (m.valid) {
                s_t[m.r * nb + b] = tt;
                if (ISUMS && t == 0u) a.isums[(size_t)(row_lo + m.r) * nb + b] = is;
            }
        }
    }
    mv_wave_partials(g, s_t, s_p, nrow, w, false);
    lds_barrier();
    mv_tree_store<GLU>(a, s_p, s_t, nrow, row_lo, t, false, t64, add0);
}

}  // namespace tsr

// ---- launchers ------------------------------------------------------------------------------------
// One workgroup of 16 waves per row block of rb rows, rb = ceil(N / n_cu) (at least 16), so that every
// compute unit holds one workgroup with its whole share of the matrix; rb is lowered when the terms
// would not fit the LDS budget. The weight layout is built for this rb at upload.
static size_t mv_lds_rows(uint32_t rb, uint32_t nb) {   // terms (16-byte padded) and partials
    return 4u * ((((size_t)rb * nb + 3u) & ~(size_t)3u) + 16u * (size_t)rb);
}
static size_t mv_lds_fixed(uint32_t fmt, uint32_t nb) {  // x quants (+ sums) and scales of 16 waves, flags
    const uint32_t kx = (nb + 15u) / 16u;
    return fmt == TSR_HIP_FMT_Q4_K ? (size_t)tsr::kMvWaves * kx * (tsr::kXq4Stride + 32u + 4u) + 64u
                                   : (size_t)tsr::kMvWaves * kx * (32u + 4u);
}

uint32_t tsr_wl_rows_per_block(uint32_t fmt, uint32_t N, uint32_t K, uint32_t n_cu) {
    const uint32_t nb = K / (fmt == TSR_HIP_FMT_Q4_K ? 256u : 32u);
    const size_t fixed = mv_lds_fixed(fmt, nb);
    uint32_t rb = (N + n_cu - 1u) / n_cu;
    if (rb < 16u) rb = 16u;
    rb += rb & 1u;                       // even: whole gate / up pairs per workgroup (GLU)
    while (rb > 2u && fixed + mv_lds_rows(rb, nb) > 120u * 1024u) rb = (rb / 2u + 1u) & ~1u;
    return rb;
}

size_t tsr_mv_prep_lds(uint32_t prep, uint32_t K) {   // K squares (16-byte padded) + 8 control words
    return prep == tsr::kPrepNorm ? 4u * (((size_t)K + 3u) & ~(size_t)3u) + 32u : 0u;
}

template <int F, int PREP, bool GLU>
static void launch_q4k(const tsr::MvArgs & a, dim3 grid, size_t lds, hipStream_t s) {
    if constexpr (PREP == tsr::kPrepNone && !GLU) {
        if (a.isums) {
            hipLaunchKernelGGL((tsr::k_mv_q4k<F, true, PREP, GLU>), grid, dim3(1024), lds, s, a);
            return;
        }
    }
    hipLaunchKernelGGL((tsr::k_mv_q4k<F, false, PREP, GLU>), grid, dim3(1024), lds, s, a);
}
template <int F>
static void launch_q4k_v(const tsr::MvArgs & a, dim3 grid, size_t lds, hipStream_t s) {
    if (a.prep == tsr::kPrepNorm) {
        if (a.glu) launch_q4k<F, tsr::kPrepNorm, true>(a, grid, lds, s);
        else launch_q4k<F, tsr::kPrepNorm, false>(a, grid, lds, s);
    } else {
        if (a.glu) launch_q4k<F, tsr::kPrepNone, true>(a, grid, lds, s);
        else launch_q4k<F, tsr::kPrepNone, false>(a, grid, lds, s);
    }
}
template <int P, int PREP, bool GLU>
static void launch_q80(const tsr::MvArgs & a, dim3 grid, size_t lds, hipStream_t s) {
    if constexpr (PREP == tsr::kPrepNone && !GLU) {
        if (a.isums) {
            hipLaunchKernelGGL((tsr::k_mv_q80<P, true, PREP, GLU>), grid, dim3(1024), lds, s, a);
            return;
        }
    }
    hipLaunchKernelGGL((tsr::k_mv_q80<P, false, PREP, GLU>), grid, dim3(1024), lds, s, a);
}
template <int P>
static void launch_q80_v(const tsr::MvArgs & a, dim3 grid, size_t lds, hipStream_t s) {
    if (a.prep == tsr::kPrepNorm) {
        if (a.glu) launch_q80<P, tsr::kPrepNorm, true>(a, grid, lds, s);
        else launch_q80<P, tsr::kPrepNorm, false>(a, grid, lds, s);
    } else {
        if (a.glu) launch_q80<P, tsr::kPrepNone, true>(a, grid, lds, s);
        else launch_q80<P, tsr::kPrepNone, false>(a, grid, lds, s);
    }
}

// The fused norm needs every value of x loaded in the kernel's first round: K <= 8192 (Q4_K: at most 4
// super-blocks per wave, Q8_0 at most 16 blocks), which also bounds its LDS. GLU needs whole pairs of
// rows in every workgroup (even rb and N) and stores N / 2 outputs (no addend or accumulation).
static bool variant_ok(const tsr::MvArgs & a) {
    if (a.prep != tsr::kPrepNone && (a.isums != nullptr || a.K > 8192u)) return false;
    if (a.glu && (a.isums != nullptr || (a.rb & 1u) || (a.N & 1u) || a.add != nullptr || a.acc)) return false;
    return true;
}

int tsr_launch_mv_q4_k(const tsr::MvArgs & a, hipStream_t s) {
    if (!variant_ok(a)) return -2;
    const uint32_t nsb = a.K / 256u;
    const size_t lds = mv_lds_fixed(TSR_HIP_FMT_Q4_K, nsb) + mv_lds_rows(a.rb, nsb) + tsr_mv_prep_lds(a.prep, a.K);
    const dim3 grid((a.N + a.rb - 1u) / a.rb, a.T);
    // lanes per unit from the units of the wave with the most (rb rows x ceil(nsb / 16) slots): two up
    // to 64 units (two passes), one above. Four lanes would cut the o shape's instructions further
    // (0.2 us alone), but a decode layer then runs four matvec kernels instead of three, and their
    // code no longer fits the instruction cache together with the attention kernel's: the layer in
    // sequence was 0.5 us slower.
    const uint32_t upw = a.rb * ((nsb + 15u) / 16u);
    if (upw <= 64u) launch_q4k_v<2>(a, grid, lds, s);
    else launch_q4k_v<1>(a, grid, lds, s);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mv_q8_0(const tsr::MvArgs & a, hipStream_t s) {
    if (!variant_ok(a)) return -2;
    const uint32_t nb = a.K / 32u;
    const size_t lds = mv_lds_fixed(TSR_HIP_FMT_Q8_0, nb) + mv_lds_rows(a.rb, nb) + tsr_mv_prep_lds(a.prep, a.K);
    const dim3 grid((a.N + a.rb - 1u) / a.rb, a.T);
    // passes of the wave with the most units: rb rows x ceil(nb / 16) slots, 64 units a pass
    const uint32_t mp = (a.rb * ((nb + 15u) / 16u) + 63u) / 64u;
    if (mp <= 1u) launch_q80_v<1>(a, grid, lds, s);
    else if (mp <= 2u) launch_q80_v<2>(a, grid, lds, s);
    else if (mp <= 4u) launch_q80_v<4>(a, grid, lds, s);
    else launch_q80_v<8>(a, grid, lds, s);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
