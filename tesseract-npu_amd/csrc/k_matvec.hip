// k_matvec.hip -- decode MUL_MAT (matrix-vector) kernels for Q8_0 and Q4_K weights on gfx950.
//
// Numerics (sw/sim/tsr_ref.c:525-635; docs/spec.md:438-477): per row, term i of block / super-block i
// is added into partial p[i mod 16] in order, then y = ((p0+p1)+(p2+p3))+... (the 16-partial tree);
// Q8_0 term = (d Dx) f32(isum), Q4_K term = (d Dx) f32(isum) - (dmin Dx) f32(msum). The integer sums
// are exact in any order, so they are split over lanes freely; the f32 adds keep the reference's
// pairing: each partial is owned by one lane group and the tree is a butterfly whose pairs are the
// tree's pairs (f32 addition is commutative).
//
// Each wave first issues the loads of its slice of x and of all its weight rows (16-byte coalesced
// loads, one 1 KiB wave load per instruction), then the workgroup quantizes x into LDS (QACT) while
// the weights stream in; the rows are then reduced with v_dot4_i32_i8 and DPP.
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

// Scales of the device meta (see q4k_meta_encode in tsr_hip.hip): bytes 4-11 hold sc_j | (m_j & 3) << 6,
// bytes 12-15 the nibbles m_j >> 2. Lane piece h (group g = h / 2) needs sc_2g, sc_2g+1 and m_h.
struct Q4kLane {
    uint32_t sc_sh, m_sh, mh_sh;   // bit offsets inside the selected words
    bool sc_w2, m_w2;              // scales in bytes 8-11 (j >= 4)
};
__device__ __forceinline__ Q4kLane q4k_lane(int h) {
    const int g = h >> 1;
    Q4kLane l;
    l.sc_w2 = g >= 2;
    l.sc_sh = 16u * (uint32_t)(g & 1);
    l.m_w2 = h >= 4;
    l.m_sh = 8u * (uint32_t)(h & 3) + 6u;
    l.mh_sh = 4u * (uint32_t)h;
    return l;
}
__device__ __forceinline__ void q4k_scales(const Q4kLane & l, uint4 mt, int & sc_lo, int & sc_hi, int & mn) {
    const uint32_t ws = l.sc_w2 ? mt.z : mt.y, wm = l.m_w2 ? mt.z : mt.y;
    sc_lo = (int)__builtin_amdgcn_ubfe(ws, l.sc_sh, 6);
    sc_hi = (int)__builtin_amdgcn_ubfe(ws, l.sc_sh + 8u, 6);
    mn = (int)(__builtin_amdgcn_ubfe(wm, l.m_sh, 2) | (__builtin_amdgcn_ubfe(mt.w, l.mh_sh, 4) << 2));
}

__device__ __forceinline__ void store_y(const MvArgs & a, uint32_t t, uint32_t row, float v) {
    float * yp = a.y + (size_t)t * a.y_stride + row;
    if (a.add) v = sadd(a.add[(size_t)t * a.add_stride + row], v);
    else if (a.acc) v = sadd(*yp, v);
    *yp = v;
}

// ---------------------------------------------------------------------------------------------
// Q4_K. A block of W waves owns W * R consecutive rows, R per wave. Every wave first issues all
// weight loads of its R rows, then the block quantizes x into LDS (QACT A256) while those loads are
// in flight. Lane L, load i covers quant chunk c = 64 i + L (16 bytes) of a row: super-block
// s = c / 8, piece h = c % 8 of its 128 quant bytes, i.e. group g = h / 2 (sub-block 2g in the low
// nibbles, 2g+1 in the high nibbles), half h % 2. Eight lanes hold a super-block; its term goes to
// partial s mod 16 = 8 (i mod 2) + L / 8, kept in pa (i even) / pb (i odd) of the row.
// ---------------------------------------------------------------------------------------------
template <int NL, int R, int WMAX, bool ISUMS>
__global__ __launch_bounds__(64 * WMAX) void k_mv_q4k(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t K = a.K, nsb = K / 256u;
    int8_t * s_qs = (int8_t *)lds;
    float * s_dx = (float *)(lds + K);
    int * s_bsp = (int *)(s_dx + nsb);                          // sum of the 32 q of each sub-block
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;
    const uint32_t row0 = (blockIdx.x * (uint32_t)nw + (uint32_t)wave) * R;
    const uint32_t nchunk = nsb * 8u;

    // x slices of this wave's QACT blocks first: the vector-memory counter retires in order, so
    // loads issued before the weight loads can be waited for without waiting for the weights
    constexpr int XP = 4;
    float4 xv[XP];
#pragma unroll
    for (int k = 0; k < XP; ++k) {
        const uint32_t s = min((uint32_t)wave + (uint32_t)(k * nw), nsb - 1u);   // clamped: no branch
        xv[k] = *(const float4 *)(x + 256u * s + 4u * (uint32_t)lane);
    }
    __builtin_amdgcn_sched_barrier(0);

    // weight loads: rows and chunks beyond the matrix read a clamped (valid) address; their values
    // are never used (masked below), which keeps the load sequence free of branches
    uint4 qv[R][NL], mv[R][NL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, a.N - 1u);
        const uint8_t * rq = a.wq + (size_t)row * nsb * 128u;
        const uint8_t * rm = a.wm + (size_t)row * nsb * 16u;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const uint32_t c = min(64u * (uint32_t)i + (uint32_t)lane, nchunk - 1u);
            qv[r][i] = *(const uint4 *)(rq + 16u * c);
            mv[r][i] = *(const uint4 *)(rm + 16u * (c >> 3));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    int slow = 0;
    auto qact_sb = [&](uint32_t s, const float4 v) {
        float d;
        int s4;
        const uint32_t q = qact_a256_lane(v, lane, &d, &s4);
        *(uint32_t *)(s_qs + 256u * s + 4u * (uint32_t)lane) = q;
        const int s32 = sum8_i(s4);
        if (lane == 0) s_dx[s] = d;
        if ((lane & 7) == 0) s_bsp[8u * s + (uint32_t)(lane >> 3)] = s32;
        const uint32_t ad = fb(d) & 0x7FFFFFFFu;
        slow |= (ad != 0u && ad < 0x21800000u) ? 1 : 0;          // 0 < |d| < 2^-60
    };
#pragma unroll
    for (int k = 0; k < XP; ++k) {
        const uint32_t s = (uint32_t)wave + (uint32_t)(k * nw);
        if (s < nsb) qact_sb(s, xv[k]);
    }
    for (uint32_t s = (uint32_t)wave + (uint32_t)(XP * nw); s < nsb; s += (uint32_t)nw)
        qact_sb(s, *(const float4 *)(x + 256u * s + 4u * (uint32_t)lane));
    slow = __syncthreads_or(slow);
    if (row0 >= a.N) return;

    const int h = lane & 7, g = h >> 1, half = h & 1;
    const Q4kLane ql = q4k_lane(h);
    float pa[R], pb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) { pa[r] = 0.0f; pb[r] = 0.0f; }
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
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t m4 = 0x0F0F0F0Fu;
            const uint4 qw = qv[r][i], mt = mv[r][i];
            int slo = dot4((int)(qw.x & m4), xl.x, 0);
            slo = dot4((int)(qw.y & m4), xl.y, slo);
            slo = dot4((int)(qw.z & m4), xl.z, slo);
            slo = dot4((int)(qw.w & m4), xl.w, slo);
            int shi = dot4((int)((qw.x >> 4) & m4), xh.x, 0);
            shi = dot4((int)((qw.y >> 4) & m4), xh.y, shi);
            shi = dot4((int)((qw.z >> 4) & m4), xh.z, shi);
            shi = dot4((int)((qw.w >> 4) & m4), xh.w, shi);
            int sc_lo, sc_hi, mn;
            q4k_scales(ql, mt, sc_lo, sc_hi, mn);
            const int ip = sum8_i(__mul24(sc_lo, slo) + __mul24(sc_hi, shi));   // |operands| < 2^23: v_mul_i32_i24
            const int mp = sum8_i(__mul24(mn, bsp));
            const uint32_t row = row0 + (uint32_t)r;
            if (ISUMS && t == 0u && h == 0 && valid && row < a.N) {
                a.isums[(size_t)row * 2u * nsb + 2u * s] = ip;
                a.isums[(size_t)row * 2u * nsb + 2u * s + 1u] = mp;
            }
            const float d = h2f_fast(mt.x & 0xFFFFu), dm = h2f_fast(mt.x >> 16);
            float tt;
            if (!slow) {
                const float t1 = (d * dx) * (float)ip;
                const float t2 = (dm * dx) * (float)mp;
                tt = t1 - t2;
            } else {
                tt = ssub(smul(smul(d, dx), i2f(ip)), smul(smul(dm, dx), i2f(mp)));
            }
            if (valid) {
                if (i & 1) pb[r] = slow ? sadd(pb[r], tt) : pb[r] + tt;
                else pa[r] = slow ? sadd(pa[r], tt) : pa[r] + tt;
            }
        }
    }
    // tree: slots L/8 pair by xor 1, 2, 4 of the slot (lanes xor 8, 16, 32); pa = p0..p7, pb = p8..p15
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = row0 + (uint32_t)r;
        float qa_ = pa[r], qb_ = pb[r], y;
        if (!slow) {
            qa_ = qa_ + dpp_f<kDppRowMirror>(qa_);
            qb_ = qb_ + dpp_f<kDppRowMirror>(qb_);
            qa_ = qa_ + xor16_f(qa_);
            qb_ = qb_ + xor16_f(qb_);
            qa_ = qa_ + xor32_f(qa_);
            qb_ = qb_ + xor32_f(qb_);
            y = canon(qa_ + qb_);
        } else {
            qa_ = sadd(qa_, dpp_f<kDppRowMirror>(qa_));
            qb_ = sadd(qb_, dpp_f<kDppRowMirror>(qb_));
            qa_ = sadd(qa_, xor16_f(qa_));
            qb_ = sadd(qb_, xor16_f(qb_));
            qa_ = sadd(qa_, xor32_f(qa_));
            qb_ = sadd(qb_, xor32_f(qb_));
            y = sadd(qa_, qb_);
        }
        if (lane == 0 && row < a.N) store_y(a, t, row, y);
    }
}

// ---------------------------------------------------------------------------------------------
// Q8_0. A block of W waves owns W * R consecutive rows, R per wave; loads first, then QACT A32 into
// LDS. Lane L, load i covers quant chunk c = 64 i + L: block b = 32 i + L / 2, half L % 2. Blocks b
// (lane L < 32) and b + 16 (lane L + 32) both belong to partial b mod 16 = (L / 2) mod 16, in that
// order; the lower half of the wave owns the partials.
// ---------------------------------------------------------------------------------------------
template <int NL, int R, int WMAX, bool ISUMS>
__global__ __launch_bounds__(64 * WMAX) void k_mv_q80(MvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t K = a.K, nb = K / 32u;
    int8_t * s_qs = (int8_t *)lds;
    float * s_dx = (float *)(lds + K);
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;
    const uint32_t row0 = (blockIdx.x * (uint32_t)nw + (uint32_t)wave) * R;

    constexpr int XP = 4;                                        // x slots first (see k_mv_q4k)
    float4 xv[XP];
#pragma unroll
    for (int k = 0; k < XP; ++k) {
        const uint32_t slot = min(threadIdx.x + (uint32_t)k * blockDim.x, K / 4u - 1u);
        xv[k] = *(const float4 *)(x + 4u * slot);
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 qv[R][NL];
    uint32_t dv[R][NL];
#pragma unroll
    for (int r = 0; r < R; ++r) {                                // clamped addresses, as in k_mv_q4k
        const uint32_t row = min(row0 + (uint32_t)r, a.N - 1u);
        const uint8_t * rq = a.wq + (size_t)row * nb * 32u;
        const uint16_t * rm = (const uint16_t *)(a.wm + (size_t)row * nb * 2u);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const uint32_t c = min(64u * (uint32_t)i + (uint32_t)lane, 2u * nb - 1u);
            qv[r][i] = *(const uint4 *)(rq + 16u * c);
            dv[r][i] = rm[c >> 1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    auto qact_slot = [&](uint32_t slot, const float4 v) {       // 8 lanes per 32-block
        float D;
        const uint32_t q = qact_a32_lane(v, &D);
        *(uint32_t *)(s_qs + 4u * slot) = q;
        if ((lane & 7) == 0) s_dx[slot >> 3] = D;
    };
#pragma unroll
    for (int k = 0; k < XP; ++k) {
        const uint32_t slot = threadIdx.x + (uint32_t)k * blockDim.x;
        if (slot < K / 4u) qact_slot(slot, xv[k]);
    }
    for (uint32_t slot = threadIdx.x + (uint32_t)XP * blockDim.x; slot < K / 4u; slot += blockDim.x)
        qact_slot(slot, *(const float4 *)(x + 4u * slot));
    __syncthreads();
    if (row0 >= a.N) return;

    float p[R];
#pragma unroll
    for (int r = 0; r < R; ++r) p[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t c = 64u * (uint32_t)i + (uint32_t)lane, b = c >> 1;
        int4 xv = make_int4(0, 0, 0, 0);
        float dx = 0.0f;
        if (b < nb) {
            xv = *(const int4 *)(s_qs + 16u * c);
            dx = s_dx[b];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int is = dot4((int)qv[r][i].x, xv.x, 0);
            is = dot4((int)qv[r][i].y, xv.y, is);
            is = dot4((int)qv[r][i].z, xv.z, is);
            is = dot4((int)qv[r][i].w, xv.w, is);
            is += dpp_i<kDppXor1>(is);
            const uint32_t row = row0 + (uint32_t)r;
            if (ISUMS && t == 0u && (lane & 1) == 0 && b < nb && row < a.N) a.isums[(size_t)row * nb + b] = is;
            const float tt = (h2f_fast(dv[r][i]) * dx) * (float)is;
            const float tu = xor32_f(tt);
            if (lane < 32) {
                if (b < nb) p[r] = p[r] + tt;
                if (b + 16u < nb) p[r] = p[r] + tu;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = p[r];
        v = v + dpp_f<kDppXor2>(v);
        v = v + dpp_f<kDppRowHalfMirror>(v);
        v = v + dpp_f<kDppRowMirror>(v);
        v = v + xor16_f(v);
        const uint32_t row = row0 + (uint32_t)r;
        if (lane == 0 && row < a.N) store_y(a, t, row, canon(v));
    }
}

}  // namespace tsr

// ---- launchers ------------------------------------------------------------------------------------
// R rows per wave and W waves per block: about one block per compute unit with up to 16 waves, R
// as small as that allows (more waves hide more latency), capped so the weight registers of R rows
// (R * NL loads per lane) fit the register budget of WMAX waves per compute unit.
struct MvShape {
    uint32_t R, W;
};
static MvShape mv_shape(uint32_t N, uint32_t NL, uint32_t regs_per_load, uint32_t n_cu) {
    const uint32_t per_cu = (N + n_cu - 1u) / n_cu;
    uint32_t R = 1u;
    while (R < 8u && R * 16u < per_cu && 2u * R * NL * regs_per_load <= 64u) R *= 2u;
    uint32_t W = (per_cu + R - 1u) / R;
    W = W < 1u ? 1u : (W > 16u ? 16u : W);
    return { R, W };
}

template <int NL, int R>
static void launch_q4k(const tsr::MvArgs & a, uint32_t W, size_t lds, hipStream_t s) {
    constexpr int WMAX = (R * NL * 8 <= 64) ? 16 : 8;
    if (W > (uint32_t)WMAX) W = WMAX;
    const dim3 grid((a.N + W * R - 1u) / (W * R), a.T);
    if (a.isums) hipLaunchKernelGGL((tsr::k_mv_q4k<NL, R, WMAX, true>), grid, dim3(64u * W), lds, s, a);
    else hipLaunchKernelGGL((tsr::k_mv_q4k<NL, R, WMAX, false>), grid, dim3(64u * W), lds, s, a);
}
template <int NL, int R>
static void launch_q80(const tsr::MvArgs & a, uint32_t W, size_t lds, hipStream_t s) {
    constexpr int WMAX = (R * NL * 5 <= 80) ? 16 : 8;
    if (W > (uint32_t)WMAX) W = WMAX;
    const dim3 grid((a.N + W * R - 1u) / (W * R), a.T);
    if (a.isums) hipLaunchKernelGGL((tsr::k_mv_q80<NL, R, WMAX, true>), grid, dim3(64u * W), lds, s, a);
    else hipLaunchKernelGGL((tsr::k_mv_q80<NL, R, WMAX, false>), grid, dim3(64u * W), lds, s, a);
}

template <int NL>
static void dispatch_q4k(const tsr::MvArgs & a, MvShape sh, size_t lds, hipStream_t s) {
    if constexpr (NL <= 1) { if (sh.R >= 8u) return launch_q4k<NL, 8>(a, sh.W, lds, s); }
    if constexpr (NL <= 2) { if (sh.R >= 4u) return launch_q4k<NL, 4>(a, sh.W, lds, s); }
    if constexpr (NL <= 4) { if (sh.R >= 2u) return launch_q4k<NL, 2>(a, sh.W, lds, s); }
    launch_q4k<NL, 1>(a, sh.W, lds, s);
}
template <int NL>
static void dispatch_q80(const tsr::MvArgs & a, MvShape sh, size_t lds, hipStream_t s) {
    if constexpr (NL <= 1) { if (sh.R >= 8u) return launch_q80<NL, 8>(a, sh.W, lds, s); }
    if constexpr (NL <= 2) { if (sh.R >= 4u) return launch_q80<NL, 4>(a, sh.W, lds, s); }
    if constexpr (NL <= 4) { if (sh.R >= 2u) return launch_q80<NL, 2>(a, sh.W, lds, s); }
    launch_q80<NL, 1>(a, sh.W, lds, s);
}

#define TSR_CASE(f, n) case n: f<n>(a, sh, lds, s); break;

int tsr_launch_mv_q4_k(const tsr::MvArgs & a, uint32_t n_cu, hipStream_t s) {
    const uint32_t nsb = a.K / 256u, NL = (nsb + 7u) / 8u;
    const size_t lds = (size_t)a.K + 4u * nsb + 32u * nsb;
    const MvShape sh = mv_shape(a.N, NL, 8u, n_cu);
    switch (NL) {
        TSR_CASE(dispatch_q4k, 1) TSR_CASE(dispatch_q4k, 2) TSR_CASE(dispatch_q4k, 3) TSR_CASE(dispatch_q4k, 4)
        TSR_CASE(dispatch_q4k, 5) TSR_CASE(dispatch_q4k, 6) TSR_CASE(dispatch_q4k, 7) TSR_CASE(dispatch_q4k, 8)
        TSR_CASE(dispatch_q4k, 9) TSR_CASE(dispatch_q4k, 10) TSR_CASE(dispatch_q4k, 11) TSR_CASE(dispatch_q4k, 12)
        TSR_CASE(dispatch_q4k, 13) TSR_CASE(dispatch_q4k, 14) TSR_CASE(dispatch_q4k, 15) TSR_CASE(dispatch_q4k, 16)
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mv_q8_0(const tsr::MvArgs & a, uint32_t n_cu, hipStream_t s) {
    const uint32_t nb = a.K / 32u, NL = (nb + 31u) / 32u;
    const size_t lds = (size_t)a.K + 4u * nb;
    const MvShape sh = mv_shape(a.N, NL, 5u, n_cu);
    switch (NL) {
        TSR_CASE(dispatch_q80, 1) TSR_CASE(dispatch_q80, 2) TSR_CASE(dispatch_q80, 3) TSR_CASE(dispatch_q80, 4)
        TSR_CASE(dispatch_q80, 5) TSR_CASE(dispatch_q80, 6) TSR_CASE(dispatch_q80, 7) TSR_CASE(dispatch_q80, 8)
        TSR_CASE(dispatch_q80, 9) TSR_CASE(dispatch_q80, 10) TSR_CASE(dispatch_q80, 11) TSR_CASE(dispatch_q80, 12)
        TSR_CASE(dispatch_q80, 13) TSR_CASE(dispatch_q80, 14) TSR_CASE(dispatch_q80, 15) TSR_CASE(dispatch_q80, 16)
        TSR_CASE(dispatch_q80, 17) TSR_CASE(dispatch_q80, 18) TSR_CASE(dispatch_q80, 19) TSR_CASE(dispatch_q80, 20)
        TSR_CASE(dispatch_q80, 21) TSR_CASE(dispatch_q80, 22) TSR_CASE(dispatch_q80, 23) TSR_CASE(dispatch_q80, 24)
        TSR_CASE(dispatch_q80, 25) TSR_CASE(dispatch_q80, 26) TSR_CASE(dispatch_q80, 27) TSR_CASE(dispatch_q80, 28)
        TSR_CASE(dispatch_q80, 29) TSR_CASE(dispatch_q80, 30) TSR_CASE(dispatch_q80, 31) TSR_CASE(dispatch_q80, 32)
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
