// wlayout.hpp -- the device layout of Q8_0 / Q4_K weights (host and device).
//
// Rows are stored in groups of 16 (ng = ceil(N / 16); the rows of the last group beyond N are zero).
// Inside a row, the blocks (Q8_0: 32 values) or super-blocks (Q4_K: 256 values) are ordered by the
// tree partial they feed: block s = w + 16 k (w = s mod 16, the partial p[w] of the row rule) sits at
// slot w q + min(w, rem) + k, with q = nb / 16 and rem = nb % 16. The blocks of one partial are then
// consecutive slots, and the matvec kernel gives each partial to one wave.
//   Q4_K quant [ng][8 pieces][nb slots][16 rows][16 B]   piece j = bytes 16j .. 16j+15 of qs[128]
//        meta  [ng][nb slots][16 rows][16 B]             fp16 d, fp16 dmin, 12 re-encoded scale bytes
//   Q8_0 quant [ng][2 halves][nb slots][16 rows][16 B]   half h = bytes 16h .. 16h+15 of qs[32]
//        meta  [ng][nb slots][16 rows]                   fp16 d
// A wave load of one piece over (4 slots x 16 rows) reads 256-byte runs. The meta region comes
// first; the quant region starts 256-byte aligned. The layout is a byte permutation of the ggml
// blocks plus the Q4_K scale re-encoding (both inverted by tsr_hip_weight_read).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsr {

struct WGeom {
    uint32_t nb, q, rem, ng;   // blocks per row, nb / 16, nb % 16, row groups
};

__host__ __device__ inline WGeom wgeom(uint32_t N, uint32_t nb) { return { nb, nb >> 4, nb & 15u, (N + 15u) >> 4 }; }
// Blocks of partial w in a row, and the slot of block s = w + 16 k.
__host__ __device__ inline uint32_t wl_count(const WGeom & g, uint32_t w) { return g.q + (w < g.rem ? 1u : 0u); }
__host__ __device__ inline uint32_t wl_slot(const WGeom & g, uint32_t w, uint32_t k) {
    return w * g.q + (w < g.rem ? w : g.rem) + k;
}
__host__ __device__ inline uint32_t wl_slot_of(const WGeom & g, uint32_t s) { return wl_slot(g, s & 15u, s >> 4); }

// Q4_K byte offsets (quant offsets relative to the quant region).
__host__ __device__ inline size_t q4k_quant_off(const WGeom & g, uint32_t G, uint32_t j, uint32_t slot, uint32_t r) {
    return ((((size_t)G * 8u + j) * g.nb + slot) * 16u + r) * 16u;
}
__host__ __device__ inline size_t q4k_meta_off(const WGeom & g, uint32_t G, uint32_t slot, uint32_t r) {
    return (((size_t)G * g.nb + slot) * 16u + r) * 16u;
}
// Q8_0 byte offsets.
__host__ __device__ inline size_t q80_quant_off(const WGeom & g, uint32_t G, uint32_t h, uint32_t slot, uint32_t r) {
    return ((((size_t)G * 2u + h) * g.nb + slot) * 16u + r) * 16u;
}
__host__ __device__ inline size_t q80_meta_off(const WGeom & g, uint32_t G, uint32_t slot, uint32_t r) {
    return (((size_t)G * g.nb + slot) * 16u + r) * 2u;
}

}  // namespace tsr
