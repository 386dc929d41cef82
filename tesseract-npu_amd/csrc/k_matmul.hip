// k_matmul.hip -- prefill MUL_MAT (T >= 16 tokens) for Q8_0 weights on the int8 matrix cores.
//
// Numerics (sw/sim/tsr_ref.c:525-635): y[t][n] is the 16-partial tree of the terms
// (d[n][b] Dx[t][b]) f32(isum[t][n][b]), term b going to partial b mod 16 in order of b; the
// activation is quantized by QACT A32 first (k_qact, into scratch).
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
// Order: the partials are computed one after the other (j = 0..15, blocks b = j, j + 16, ... in
// order), and each finished p_j enters the tree ((p0 + p1) + (p2 + p3)) + ... through a 4-level stack
// of pending sums, so an output holds 5 values instead of 16.
//
// Lane layouts (gfx950): an operand lane l supplies row l % 32 of its matrix and k = 16 (l / 32) ..
// 16 (l / 32) + 15; the result lane l holds column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4,
// r = 0..15.
#include "kernels.hpp"
#include "tsr_dev.hpp"
#include "wlayout.hpp"

namespace tsr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// A workgroup of 4 waves computes 64 weight rows x 64 tokens; wave (wr, wt) the 32 x 32 tile at
// rows n0 + 32 wr, tokens t0 + 32 wt. Rows and tokens beyond the matrix read clamped (valid)
// addresses and are not stored.
__global__ __launch_bounds__(256) void k_mm_q80(MmArgs a) {
    const WGeom g = wgeom(a.N, a.K >> 5);
    const uint32_t lane = __lane_id(), wave = threadIdx.x >> 6;
    const uint32_t nbase = blockIdx.x * 64u + 32u * (wave & 1u), tbase = blockIdx.y * 64u + 32u * (wave >> 1);
    const uint32_t h = lane >> 5, c = lane & 31u;
    // operand rows of this lane
    const uint32_t n = min(nbase + c, a.N - 1u), t = min(tbase + c, a.T - 1u);
    const uint8_t * xq = a.qa + (size_t)t * a.qa_stride;             // QS of token t
    const float * xd = (const float *)(a.qa + (size_t)t * a.qa_stride + a.d_off);

    v16f p, L0, L1, L2, L3;
    for (int r = 0; r < 16; ++r) { L0[r] = 0.0f; L1[r] = 0.0f; L2[r] = 0.0f; L3[r] = 0.0f; }
    for (uint32_t j = 0; j < 16u; ++j) {
        for (int r = 0; r < 16; ++r) p[r] = 0.0f;
        const uint32_t cnt = wl_count(g, j);
        for (uint32_t k = 0; k < cnt; ++k) {
            const uint32_t b = j + 16u * k, sl = wl_slot(g, j, k);
            const v4i wa = *(const v4i *)(a.wq + q80_quant_off(g, n >> 4, h, sl, n & 15u));
            const v4i xb = *(const v4i *)(xq + 32u * b + 16u * h);
            const float dw = h ? 0.0f : h2f_fast(*(const uint16_t *)(a.wm + q80_meta_off(g, n >> 4, sl, n & 15u)));
            const float dx = h ? 0.0f : xd[b];
            v16i is = {};
            is = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, xb, is, 0, 0, 0);
            v16f P = {};
            P = __builtin_amdgcn_mfma_f32_32x32x2f32(dw, dx, P, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = p[r] + P[r] * (float)is[r];
        }
        // p_j into the tree: level 0 holds an even partial, level 1 a pair, level 2 a quad, level 3 an octet
        if ((j & 1u) == 0u) {
            L0 = p;
        } else {
            v16f s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = L0[r] + p[r];
            if ((j & 2u) == 0u) L1 = s;
            else {
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = L1[r] + s[r];
                if ((j & 4u) == 0u) L2 = s;
                else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[r] = L2[r] + s[r];
                    if ((j & 8u) == 0u) L3 = s;
                    else {
#pragma unroll
                        for (int r = 0; r < 16; ++r) L0[r] = L3[r] + s[r];   // the full tree (j = 15)
                    }
                }
            }
        }
    }
    // result: lane holds token tbase + c, rows nbase + 8 (r / 4) + 4 h + r % 4; L0 = the tree
    const uint32_t tt = tbase + c;
    if (tt < a.T) {
        float * yr = a.y + (size_t)tt * a.y_stride;
        const float * ar = a.add ? a.add + (size_t)tt * a.add_stride : nullptr;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t nn = nbase + 8u * (uint32_t)(r >> 2) + 4u * h + (uint32_t)(r & 3);
            if (nn < a.N) {
                float v = canon(L0[r]);
                if (ar) v = sadd(ar[nn], v);
                else if (a.acc) v = sadd(yr[nn], v);
                yr[nn] = v;
            }
        }
    }
}

}  // namespace tsr

int tsr_launch_mm_q8_0(const tsr::MmArgs & a, hipStream_t s) {
    const dim3 grid((a.N + 63u) / 64u, (a.T + 63u) / 64u);
    hipLaunchKernelGGL(tsr::k_mm_q80, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
