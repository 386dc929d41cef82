// wlayout.hpp -- the device layout of Q8_0 / Q4_K weights (host and device).
//
// Rows are stored in row blocks of rb consecutive rows: the rows one matvec workgroup owns (rb is
// chosen at upload from the device's compute units, k_matvec.hip: tsr_wl_rows_per_block). The last
// block holds the remaining R = N - (nblk - 1) rb rows. Inside a row, the blocks (Q8_0: 32 values)
// or super-blocks (Q4_K: 256 values) are ordered by the tree partial they feed: block s = w + 16 k
// (w = s mod 16, the partial p[w] of the row rule) sits at slot w q + min(w, rem) + k, with
// q = nb / 16 and rem = nb % 16. The blocks of one partial are then consecutive slots, and the
// matvec gives each partial to one wave.
//
// Row block B starts at B * bstride (bstride: a full block's bytes, 256-aligned) and holds, with R
// its rows:
//   Q4_K quant [8 pieces][nb slots][R rows][16 B]   piece j = bytes 16j .. 16j+15 of qs[128]
//        meta  [nb slots][R rows][16 B]             fp16 d, fp16 dmin, 12 re-encoded scale bytes
//   Q8_0 quant [2 halves][nb slots][R rows][16 B]   half h = bytes 16h .. 16h+15 of qs[32]
//        meta  [nb slots][R rows]                   fp16 d
// A wave's unit u (0 .. cnt R - 1) is (slot k = u / R, row u % R): for a fixed piece, consecutive
// units are consecutive 16-byte runs, so a wave load reads one contiguous run of up to 1 KiB and
// a workgroup reads one contiguous region. The layout is a byte permutation of the ggml blocks
// plus the Q4_K scale re-encoding (both inverted by tsr_hip_weight_read).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsr {

struct WGeom {
    uint32_t nb, q, rem;       // blocks per row, nb / 16, nb % 16
    uint32_t N, rb, nblk;      // rows, rows per row block, row blocks
    uint32_t qb, mb;           // quant and meta bytes per (block, row): Q4_K 128, 16; Q8_0 32, 2
    uint64_t bstride;          // bytes of a full row block (256-aligned)
};

__host__ __device__ inline WGeom wgeom(uint32_t N, uint32_t nb, uint32_t rb, bool q4k) {
    WGeom g;
    g.nb = nb;
    g.q = nb >> 4;
    g.rem = nb & 15u;
    g.N = N;
    g.rb = rb;
    g.nblk = (N + rb - 1u) / rb;
    g.qb = q4k ? 128u : 32u;
    g.mb = q4k ? 16u : 2u;
    g.bstride = ((uint64_t)nb * rb * (g.qb + g.mb) + 255u) & ~(uint64_t)255u;
    return g;
}
// Total device bytes: the full blocks and the last block.
__host__ __device__ inline uint64_t wl_bytes(const WGeom & g) {
    const uint32_t R = g.N - (g.nblk - 1u) * g.rb;
    return (uint64_t)(g.nblk - 1u) * g.bstride + (((uint64_t)g.nb * R * (g.qb + g.mb) + 255u) & ~(uint64_t)255u);
}
// Rows of row block B.
__host__ __device__ inline uint32_t wl_rows(const WGeom & g, uint32_t B) {
    const uint32_t lo = B * g.rb;
    return g.N - lo < g.rb ? g.N - lo : g.rb;
}
// Blocks of partial w in a row, and the slot of block s = w + 16 k.
__host__ __device__ inline uint32_t wl_count(const WGeom & g, uint32_t w) { return g.q + (w < g.rem ? 1u : 0u); }
__host__ __device__ inline uint32_t wl_slot(const WGeom & g, uint32_t w, uint32_t k) {
    return w * g.q + (w < g.rem ? w : g.rem) + k;
}
__host__ __device__ inline uint32_t wl_slot_of(const WGeom & g, uint32_t s) { return wl_slot(g, s & 15u, s >> 4); }

// Byte offsets inside the weight: row block B with R rows, piece (Q4_K) or half (Q8_0) j, slot, row r
// of the block.
__host__ __device__ inline uint64_t wl_quant_off(const WGeom & g, uint32_t B, uint32_t R, uint32_t j, uint32_t slot,
                                                 uint32_t r) {
    return (uint64_t)B * g.bstride + (((uint64_t)j * g.nb + slot) * R + r) * 16u;
}
__host__ __device__ inline uint64_t wl_meta_off(const WGeom & g, uint32_t B, uint32_t R, uint32_t slot, uint32_t r) {
    return (uint64_t)B * g.bstride + (uint64_t)g.qb * g.nb * R + ((uint64_t)slot * R + r) * g.mb;
}

}  // namespace tsr
