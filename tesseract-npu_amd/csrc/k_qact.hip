// k_qact.hip -- the standalone QACT kernel: T f32 rows -> T QA images in the spec layout
// (QS int8[K] | D f32[K/bs] | BS int16[K/16] for A256; each region padded to 64 bytes with zeros;
// docs/spec.md:402-425, sw/sim/tsr_ref.c:418-447).
#include "kernels.hpp"
#include "qact.hpp"

namespace tsr {

// grid: (ceil(units / 4), T); block 256 = 4 waves; one wave per unit (A32: 8 blocks, A256: 1 block).
__global__ __launch_bounds__(256) void k_qact(QactArgs a) {
    const int lane = (int)__lane_id(), wave = (int)(threadIdx.x >> 6);
    const uint32_t t = blockIdx.y;
    const float * x = a.x + (size_t)t * a.x_stride;
    uint8_t * qa = a.qa + (size_t)t * a.qa_bytes;
    const uint32_t K = a.K;
    const uint32_t unit = blockIdx.x * 4u + (uint32_t)wave;
    if (a.kind == 0u) {
        const uint32_t slot = unit * 64u + (uint32_t)lane;         // 4 values per slot
        if (slot < K / 4u) {
            const float4 v = *(const float4 *)(x + 4u * slot);
            float D;
            const uint32_t q = qact_a32_lane(v, &D);
            *(uint32_t *)(qa + 4u * slot) = q;
            if ((lane & 7) == 0) *(float *)(qa + a.d_off + 4u * (slot / 8u)) = D;
        }
    } else {
        if (unit < K / 256u) {
            const float4 v = *(const float4 *)(x + 256u * unit + 4u * (uint32_t)lane);
            float d;
            int s4;
            bool tiny;
            const uint32_t q = qact_a256_wave(v, &d, &s4, &tiny);
            *(uint32_t *)(qa + 256u * unit + 4u * (uint32_t)lane) = q;
            if (lane == 0) *(float *)(qa + a.d_off + 4u * unit) = d;
            int s16 = s4 + dpp_i<kDppXor1>(s4);
            s16 += dpp_i<kDppXor2>(s16);
            if ((lane & 3) == 0) *(int16_t *)(qa + a.bs_off + 2u * (16u * unit + (uint32_t)lane / 4u)) = (int16_t)s16;
        }
    }
    // zero padding of each region (the first wave of each token's first block)
    if (blockIdx.x == 0 && wave == 0) {
        const uint32_t nb = K / (a.kind == 0u ? 32u : 256u);
        for (uint32_t i = K + (uint32_t)lane; i < a.d_off; i += 64u) qa[i] = 0;
        for (uint32_t i = a.d_off + 4u * nb + (uint32_t)lane; i < a.bs_off; i += 64u) qa[i] = 0;
        for (uint32_t i = a.bs_off + (a.kind ? 2u * (K / 16u) : 0u) + (uint32_t)lane; i < a.qa_bytes; i += 64u) qa[i] = 0;
    }
}

}  // namespace tsr

int tsr_launch_qact(const tsr::QactArgs & a, uint32_t T, hipStream_t s) {
    const uint32_t units = a.kind == 0u ? (a.K / 4u + 63u) / 64u : a.K / 256u;
    dim3 grid((units + 3u) / 4u, T);
    hipLaunchKernelGGL(tsr::k_qact, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
