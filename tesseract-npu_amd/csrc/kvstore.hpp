// kvstore.hpp -- the store of one QACT'd unit of a KV row into the device KV layout (k_kv.hip),
// shared by SET_ROWS and by the fused ROPE + SET_ROWS_KV kernel.
#pragma once

#include "kernels.hpp"
#include "tsr_dev.hpp"

namespace tsr {

// Values i .. i + 3 of a row (i % 4 == 0), quantized to the 4 int8 in q (value i in the low byte), go
// to cell `cell` of plane `which` (0: K, chunk-major; 1: V, dim-major). `lead`: the lane holding the
// first 4 values of the 32-value block, which also stores its fp16 scale D.
__device__ __forceinline__ void kv_store_unit(const KvArgs & a, uint32_t which, uint32_t cell, uint32_t i, uint32_t q,
                                              float D, bool lead) {
    const uint32_t u = cell >> 4, rr = cell & 15u, nbk = a.E / 32u;
    uint8_t * qb = a.base + a.quant_off + (size_t)u * 16u * a.E;
    if (which == 0u) {
        *(uint32_t *)(qb + ((size_t)(i >> 4) * 16u + rr) * 16u + (i & 15u)) = q;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) qb[(size_t)(i + k) * 16u + rr] = (uint8_t)(q >> (8 * k));
    }
    if (lead) {
        ((uint16_t *)a.base)[((size_t)u * nbk + i / 32u) * 16u + rr] = (uint16_t)f2h_exact(D);
    }
}

}  // namespace tsr
