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
// (blocks b = j, j + 16, ... in order: consecutive slots of the weight layout, wlayout.hpp). Each
// wave issues the loads of up to kMmPre of its blocks at once, then runs their matrix-core steps.
// The 16 partials meet in LDS and one thread per output adds the tree ((p0 + p1) + (p2 + p3)) + ...
//
// Lane layouts (gfx950): an operand lane l supplies row l % 32 of its matrix and k = 16 (l / 32) ..
// 16 (l / 32) + 15; the result lane l holds column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4,
// r = 0..15.
#include "kernels.hpp"
#include "qact.hpp"
#include "wlayout.hpp"

namespace tsr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr uint32_t kMmPre = 8;   // blocks whose loads one wave keeps in flight

// QACT A32 of T token rows into the block-major layout: 8 lanes per (token, block), 4 values each
// (qact_a32_lane: the spec rule, as for the QA image of k_qact).
__global__ __launch_bounds__(256) void k_qact_mm(const float * x, uint64_t x_stride, uint32_t K, uint32_t T,
                                                 uint8_t * xq, float * xd) {
    const uint32_t nb = K >> 5;
    const uint64_t pair = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;   // (token, block)
    const uint32_t l8 = threadIdx.x & 7u;
    const uint64_t npair = (uint64_t)T * nb;
    const uint64_t pc = pair < npair ? pair : npair - 1u;         // clamped: whole 8-lane groups stay active
    const uint32_t t = (uint32_t)(pc / nb), b = (uint32_t)(pc % nb);
    float D;
    const uint32_t q = qact_a32_lane(*(const float4 *)(x + (size_t)t * x_stride + 32u * b + 4u * l8), &D);
    if (pair < npair) {
        *(uint32_t *)(xq + ((size_t)b * T + t) * 32u + 4u * l8) = q;
        if (l8 == 0u) xd[(size_t)b * T + t] = D;
    }
}

__global__ __launch_bounds__(1024) void k_mm_q80(MmArgs a) {
    __shared__ float s_p[16][1024];                                // partial j of output (lane, r)
    const WGeom g = wgeom(a.N, a.K >> 5, a.rb, false);
    const uint32_t lane = __lane_id(), j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = blockIdx.x * 32u, t0 = blockIdx.y * 32u;
    const uint32_t h = lane >> 5, c = lane & 31u;
    // operand rows of this lane (clamped: rows / tokens beyond the matrix are not stored)
    const uint32_t n = min(n0 + c, a.N - 1u), t = min(t0 + c, a.T - 1u);
    const uint32_t B = n / g.rb, R = wl_rows(g, B), rr = n - B * g.rb;  // row block of the row
    const uint8_t * wq = a.w + wl_quant_off(g, B, R, h, 0u, rr);         // + 16 R slot
    const uint8_t * wm = a.w + wl_meta_off(g, B, R, 0u, rr);             // + 2 R slot
    const uint8_t * xq = a.qa + (size_t)t * 32u + 16u * h;                     // + 32 T b
    const float * xd = (const float *)(a.qa + a.d_off) + t;                      // + T b
    const uint32_t cnt = wl_count(g, j), sl0 = wl_slot(g, j, 0u);

    v16f p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = 0.0f;
    for (uint32_t k0 = 0; k0 < cnt; k0 += kMmPre) {
        v4i wa[kMmPre], xb[kMmPre];
        float dw[kMmPre], dx[kMmPre];
#pragma unroll
        for (uint32_t i = 0; i < kMmPre; ++i) {                    // clamped: every load is issued
            const uint32_t k = min(k0 + i, cnt - 1u), sl = sl0 + k, b = j + 16u * k;
            wa[i] = *(const v4i *)(wq + (size_t)16u * R * sl);
            xb[i] = *(const v4i *)(xq + (size_t)32u * a.T * b);
            dw[i] = h2f_fast(*(const uint16_t *)(wm + (size_t)2u * R * sl));
            dx[i] = xd[(size_t)a.T * b];
        }
#pragma unroll
        for (uint32_t i = 0; i < kMmPre; ++i) {
            if (k0 + i >= cnt) break;
            v16i is = {};
            is = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[i], xb[i], is, 0, 0, 0);
            v16f P = {};
            P = __builtin_amdgcn_mfma_f32_32x32x2f32(h ? 0.0f : dw[i], h ? 0.0f : dx[i], P, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = p[r] + P[r] * (float)is[r];
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
        *(float4 *)&s_p[j][16u * lane + 4u * (uint32_t)r] = make_float4(p[4 * r], p[4 * r + 1], p[4 * r + 2], p[4 * r + 3]);
    lds_barrier();

    // one thread per output: o = 16 lane' + r of the wave layout above
    const uint32_t o = threadIdx.x, ol = o >> 4, r = o & 15u;
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

}  // namespace tsr

int tsr_launch_qact_mm(const float * x, uint64_t x_stride, uint32_t K, uint32_t T, uint8_t * xq, float * xd,
                       hipStream_t s) {
    const uint64_t threads = (uint64_t)T * (K / 32u) * 8u;
    hipLaunchKernelGGL(tsr::k_qact_mm, dim3((uint32_t)((threads + 255u) / 256u)), dim3(256), 0, s, x, x_stride, K, T, xq, xd);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_mm_q8_0(const tsr::MmArgs & a, hipStream_t s) {
    const dim3 grid((a.N + 31u) / 32u, (a.T + 31u) / 32u);
    hipLaunchKernelGGL(tsr::k_mm_q80, grid, dim3(1024), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
