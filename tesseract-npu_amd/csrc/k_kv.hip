// k_kv.hip -- the q8_0 KV cache on the device: layout, byte conversion to / from llama.cpp's q8_0
// image, SET_ROWS, and the host mask summary.
//
// Device layout of one plane (K or V), E = n_head_kv * D values per cell, cells in groups of 16
// (AT's group, docs/design/03-attention-kv.md:141-205), ng = ceil(kv_size / 16) groups:
//   meta  [ng][E/32 blocks][16 cells]  fp16 block scales (block-major: the scales of one block of a
//                                      group's 16 cells are 32 contiguous bytes)
//   quant K: [ng][E/16 chunks][16 cells][16 bytes]  (chunk-major: a wave load of chunk i over 64
//                                                   cells is 4 runs of 256 contiguous bytes)
//         V: [ng][E dims][16 cells]                 (dim-major: 16 cells of one value contiguous,
//                                                   the operand order of the P.V products)
// The conversion to / from the ggml image (row j = cell j, E/32 blocks of {fp16 d, int8 qs[32]}) is
// a byte permutation, like the NPU's planes (tsr_kv_set_bytes / get_bytes, sw/sim/tsr_ref_at.c:178-212).
#include "kernels.hpp"
#include "kvstore.hpp"
#include "qact.hpp"

namespace tsr {

// Device byte offset of byte k (0..33) of ggml block b of cell `cell`.
__device__ __forceinline__ size_t kv_dev_off(const KvArgs & a, uint32_t which, uint32_t cell, uint32_t b, uint32_t k) {
    const uint32_t u = cell >> 4, rr = cell & 15u, nbk = a.E / 32u;
    if (k < 2u) return (((size_t)u * nbk + b) * 16u + rr) * 2u + k;
    const uint32_t i = 32u * b + (k - 2u);                  // value index in the row
    size_t q = a.quant_off + (size_t)u * 16u * a.E;
    if (which == 0u) q += ((size_t)(i >> 4) * 16u + rr) * 16u + (i & 15u);
    else q += (size_t)i * 16u + rr;
    return q;
}

// one thread per ggml byte of [off, off + n)
__global__ void k_kv_bytes(KvArgs a, uint32_t which, uint64_t off, uint64_t n, uint8_t * stage, int to_dev) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t pos = off + i, rowb = (uint64_t)(a.E / 32u) * 34u;
    const uint32_t cell = (uint32_t)(pos / rowb);
    const uint32_t inrow = (uint32_t)(pos % rowb);
    const size_t d = kv_dev_off(a, which, cell, inrow / 34u, inrow % 34u);
    if (to_dev) a.base[d] = stage[i];
    else stage[i] = a.base[d];
}

// SET_ROWS: one wave per 256 values of a row (8 A32 blocks), grid (ceil(E/256), n_rows).
__global__ __launch_bounds__(64) void k_kv_set_rows(KvArgs a, uint32_t which, const float * src, uint64_t src_stride,
                                                    const int64_t * idx, int32_t * bad) {
    const uint32_t r = blockIdx.y, lane = __lane_id();
    const int64_t cell64 = idx[r];
    if (cell64 < 0 || cell64 >= (int64_t)a.kv_size) {
        if (bad != nullptr && lane == 0) *bad = 1;
        return;
    }
    const uint32_t cell = (uint32_t)cell64;
    const uint32_t slot = blockIdx.x * 64u + lane;            // values 4 slot .. 4 slot + 3
    if (slot >= a.E / 4u) return;
    const float4 v = *(const float4 *)(src + (size_t)r * src_stride + 4u * slot);
    float D;
    const uint32_t q = qact_a32_lane(v, &D);
    kv_store_unit(a, which, cell, 4u * slot, q, D, (lane & 7u) == 0u);
}

}  // namespace tsr

int tsr_launch_kv_bytes(const tsr::KvArgs & a, uint32_t which, uint64_t off, uint64_t n, uint8_t * stage, int to_dev,
                        hipStream_t s) {
    if (n == 0) return 0;
    const uint64_t blocks = (n + 255u) / 256u;
    hipLaunchKernelGGL(tsr::k_kv_bytes, dim3((uint32_t)blocks), dim3(256), 0, s, a, which, off, n, stage, to_dev);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int tsr_launch_kv_set_rows(const tsr::KvArgs & a, uint32_t which, const float * src, uint32_t n_rows,
                           uint64_t src_stride, const int64_t * idx, int32_t * bad, hipStream_t s) {
    dim3 grid((a.E / 4u + 63u) / 64u, n_rows);
    hipLaunchKernelGGL(tsr::k_kv_set_rows, grid, dim3(64), 0, s, a, which, src, src_stride, idx, bad);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
