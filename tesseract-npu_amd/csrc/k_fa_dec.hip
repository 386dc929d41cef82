// k_fa_dec.hip -- the one-launch decode FLASH_ATTN_EXT (one query row, a plan's device work list),
// bit-exact to the reference's composite flash attention (tsr_ref_fa, sw/sim/tsr_ref_at.c:774-860) in
// its fixed configuration C = 4 channels, PCAP = 9344, T_MAX = 1.
//
// Work unit: one segment of ATTPV (AT 6.4) = 4 groups of one channel (groups u = c mod 4) of one chunk
// item, i.e. 64 cells, for the G <= 4 query heads of one KV head g. Segment s of channel c is the 4 of
// its groups in tile s (16 groups) of the item. One workgroup of 4 waves per segment:
//   scores     wave b = K block b (32 values) of the 64 cells: the block's term for every query head;
//              then wave h = head h: the tree16 of the 64 scores (SEG, AT 6.2) and their MAXT
//   publish    the segment's 4 maxima as MAXT keys in a slot tagged with the launch's epoch
//   wait       wave 0 reads the item's slots until every segment has published (bounded: an expired
//              wait raises *bad = 2): the chunk maxima, MAXOUT with the floor (AT 6.3)
//   EXP        wave h = head h: p = EXPK((s - m) scale) of its 64 cells and the segment's LSUM (AT 6.5)
//   P.V        wave b = value block b: the block-float weights of its 32 values (E_S over the 64-value
//              slice: both blocks of the slice), their base-256 digits and two int8 matrix-core
//              products for the 4 heads (16 values each)
//   results    the segment's O (G x D) and l (G) to the plan, each value with the launch's tag in one
//              8-byte agent-coherent store
//   reduce     G x D/64 reducer workgroups per KV head (ahead of the segments in dispatch order when
//              the grid is resident at once, after them otherwise): each
//              polls the results until all carry the tag, then chains, in order, the segments of every
//              channel of every item
//              for its 64 values of one head, CTREE over the channels, merges the items in chunk order
//              (AMERGE) and normalizes (ANORM); no atomic operation, nothing to clear (tags)
// The chunk maximum needs every score of the chunk before any P.V of it (p depends on it bit for bit),
// and the segment chains need every segment: two exchanges between workgroups, the least the reference's
// order allows. Segments of one item are consecutive in dispatch order, so every segment an item's
// wait needs has been dispatched before or is dispatched next (no wait can starve); reducers wait on
// segments only, and no segment waits on a reducer.
//
// ROPE (the layer's ROPE + SET_ROWS_KV folded in): q is then the token's unrotated Q|K|V row. Every
// workgroup rotates and quantizes its KV head's query heads, the new k row (and quantizes the new v
// row) into LDS; the workgroup of the new cell's segment scores and weighs the new cell from those LDS
// rows (the caches may not hold them yet), and the workgroup of the item's first segment stores them
// into the caches (SET_ROWS_KV, sw/ctrl/ref/kv_ref.cpp:20-45).
#include "expk.hpp"
#include "fa_common.hpp"
#include "glue.hpp"
#include "kernels.hpp"
#include "kvstore.hpp"
#include "mv_q4k.hpp"
#include "qact.hpp"
#include "wlayout.hpp"

namespace tsr {

// A buffer resource over [p, p + bytes) (gfx9 descriptor word 3): loads beyond it return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fa_rsrc(const void * p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr int kSc1 = 16;                                           // cache policy: agent-coherent (sc1)
typedef unsigned v4u_fa __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_co16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}
// Stores of the exchanged slots and results: agent-coherent (write-through, sc1) when the workgroups of
// a KV head may sit on different XCDs; plain (into the XCD's L2, where the readers' agent-coherent
// loads find them) when they all sit on one (LOCAL).
template <bool LOCAL>
__device__ __forceinline__ void st_co16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_fa, v), r, off, 0, LOCAL ? 0 : kSc1);
}

// Tags: the low 28 bits are the launch's tag, the high 4 bits the writer's XCD, so a reader checks in the
// same word that a value is this launch's and, in the LOCAL form, that its writer shared its XCD (and so
// its L2). A launch's tag follows its KV head's epoch: epoch + 1, wrapping from 2^28 - 1 to 1, never 0,
// the tag field of plan memory no launch has written yet (the plan is zeroed at creation).
constexpr uint32_t kTagMask = 0x0FFFFFFFu;
__device__ __forceinline__ bool tag_is(uint32_t t, uint32_t tag) { return (t & kTagMask) == tag; }
__device__ __forceinline__ uint32_t tag_after(uint32_t epoch) {
    const uint32_t t = (epoch & kTagMask) + 1u;
    return t > kTagMask ? 1u : t;
}

// A result with the launch's tag in one 8-byte agent-coherent store (a reader sees both or neither) and
// its load.
template <bool LOCAL>
__device__ __forceinline__ void st_tag(uint64_t * p, float v, uint32_t tag) {
    if constexpr (LOCAL) __hip_atomic_store(p, ((uint64_t)tag << 32) | fb(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(p, ((uint64_t)tag << 32) | fb(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t * p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Byte r (0..15) of a 16-byte value replaced by b (selects only: the value stays in registers).
__device__ __forceinline__ int4 put_byte(int4 v, uint32_t r, uint32_t b) {
    const uint32_t sh = 8u * (r & 3u), m = ~(0xFFu << sh), x = (b & 0xFFu) << sh, w = r >> 2;
    v.x = w == 0u ? (int)(((uint32_t)v.x & m) | x) : v.x;
    v.y = w == 1u ? (int)(((uint32_t)v.y & m) | x) : v.y;
    v.z = w == 2u ? (int)(((uint32_t)v.z & m) | x) : v.z;
    v.w = w == 3u ? (int)(((uint32_t)v.w & m) | x) : v.w;
    return v;
}

// Segments of channel c in an item: its groups u = c (mod 4) in [u0, u0 + n), 4 per segment.
struct FaSeg {
    uint32_t u_first, nu, nseg;
    __device__ __forceinline__ FaSeg(const FaItem & it, uint32_t c) {
        u_first = it.u0 + ((c + 4u - (it.u0 & 3u)) & 3u);
        const uint32_t u_end = it.u0 + it.n;
        nu = u_first < u_end ? (u_end - 1u - u_first) / 4u + 1u : 0u;
        nseg = (nu + 3u) / 4u;
    }
};

// The workgroup's work: index x among its KV head's workgroups (segments, then reducers) and the head g.
// LOCAL: a 1-D grid with g = blockIdx.x mod n_head_kv, so that under the dispatcher's round-robin of
// workgroups over the XCDs (consecutive workgroups on consecutive XCDs, n_head_kv a multiple of n_xcd)
// every workgroup of a head runs on one XCD: their exchanges stay in that XCD's L2. Every exchanged
// word carries its writer's XCD; a reader that finds another XCD than its own raises *bad |= 4 (the
// exchange is then not guaranteed: a wait that misses it expires and raises 2 as well), never silently.
struct FaDecBlock {
    uint32_t x, g;
};
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xFu;
}
template <bool LOCAL>
__device__ __forceinline__ FaDecBlock fa_dec_block(const FaDecArgs & a) {
    if constexpr (LOCAL) {
        return { blockIdx.x / a.n_head_kv, blockIdx.x % a.n_head_kv };
    } else {
        return { blockIdx.x, blockIdx.y };
    }
}

// LDS of one workgroup (bytes): table 256 | q quants 512 | q scales 64 | new k quants 128, scales 16 |
// new v quants 128, scales 16 | terms [4 heads][4 blocks][64] f32 4096 | scores [4][64] 1024 |
// p [4][64] 1024 | digits [4 waves][1024] | keys 16 | maxima 16 | flag 16.
constexpr uint32_t kDecLds = 256 + 512 + 64 + 128 + 16 + 128 + 16 + 4096 + 1024 + 1024 + 4096 + 48;

// ---- the Q|K|V rows of the launch (FaDecArgs::qkv_w) ----------------------------------------------
// Workgroup j of KV head g computes rows 24 j .. 24 j + 23 of the KV head's rows (its q heads', then its
// k head's, then its v head's) of the Q|K|V MUL_MAT with the fused RMS_NORM + MUL, bit-identical to
// k_mv_q4k with kPrepNorm (the same x preparation, A256 quantization, Q4_K terms and 16-partial tree).
// 24 rows: (G + 2) D / 24 workgroups, one per compute unit of the XCD at the Llama-3-8B shape (with 16
// rows, half the units held two and their quantization came ~1.5 us later). K <= 4096: one
// super-block per (row, partial), so thread (wave v, lane 16 i + r) computes the term of super-block
// 4 v + i of row r, which is the row's partial p[4 v + i] (+0 + term), and the thread holding x block
// b = 4 v + i (16 values per lane) quantizes it; rows 16 .. 23 are a second unit shared by thread
// pairs: threads 2 u and 2 u + 1 hold unit u (super-block u / 8, row 16 + u % 8), four pieces each,
// their integer sums met by DPP. Every load is issued at once and every wave issues the same ones (the
// memory counters retire in order, so a wave's waits never cover loads another path lacks): the norm
// weights and x, then (after a bare barrier, so that every wave's x is ahead in the queue) the first
// unit's 9 weight pieces (from any row block of the weight's layout), the epoch (read into a register
// only at the end: a wait for it would cover the weights), the second unit's pieces straight into LDS
// and its meta. The rows go to qkv_y with plain stores (the XCD's L2); after they are complete (vmcnt)
// the workgroup raises its flag.
// LDS (bytes): x quants [16][272] | sub-block sums [16][8] | scales [16] | partials [24][16] |
// control 16 | squares [K] | second unit [4 waves][4 pieces][64 lanes][16].
constexpr uint32_t kQkvMaxK = 4096, kQkvRows = 24;
constexpr uint32_t kQkvStage = 16 * kXq4Stride + 16 * 8 * 4 + 16 * 4 + kQkvRows * 16 * 4 + 16 + 4 * kQkvMaxK;
constexpr uint32_t kQkvLds = kQkvStage + 4 * 4 * 64 * 16;
static_assert(kQkvStage % 16 == 0, "the second unit's pieces land on 16-byte lanes");

template <int D>
__device__ __forceinline__ void fa_qkv_rows(const FaDecArgs & a, uint8_t * lds, uint32_t j, uint32_t g) {
    int8_t * s_xq = (int8_t *)lds;
    int * s_xb = (int *)(lds + 16u * kXq4Stride);
    float * s_xd = (float *)(s_xb + 16u * 8u);
    float * s_p = s_xd + 16u;                                     // [row][partial]
    uint32_t * s_ctl = (uint32_t *)(s_p + 16u * kQkvRows);        // halves of the RMS sum, tiny flag
    float * s_sq = (float *)(s_ctl + 4u);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, v = tid >> 6;
    const uint32_t G = a.G, K = a.qkv_K, nsb = K >> 8;
    const WGeom wg = wgeom(a.qkv_N, nsb, a.qkv_rb, true);
    // the KV head's rows in order: its q heads', its k head's, its v head's; the weight row of each
    const uint32_t nset = (G + 2u) * D;
    auto wrow = [&](uint32_t r) -> uint32_t {
        r = min(r, nset - 1u);
        return r < G * D ? g * G * D + r : a.n_head * D + (r < (G + 1u) * D ? g * D + (r - G * D) : a.E + g * D + (r - (G + 1u) * D));
    };
    // x block b = 4 v + i (lane 16 i + l16: values 16 l16 .. + 15) and the first unit (super-block b,
    // row l16 of the workgroup's 24)
    const uint32_t i4 = lane >> 4, l16 = lane & 15u, b = 4u * v + i4, bc = min(b, nsb - 1u);
    const bool has_w = a.qkv_pw != nullptr;
    const float * pl = has_w ? a.qkv_pw : a.qkv_x;                // without MUL: a valid address, unused
    const uint32_t r_0 = kQkvRows * j;
    const uint32_t n = wrow(r_0 + l16), B = n / wg.rb, rin = n - B * wg.rb, R = wl_rows(wg, B), sl = wl_slot_of(wg, bc);
    float4 pv[4], xv[4];
#pragma unroll
    for (uint32_t c = 0; c < 4u; ++c) pv[c] = *(const float4 *)(pl + 256u * bc + 16u * l16 + 4u * c);
#pragma unroll
    for (uint32_t c = 0; c < 4u; ++c) xv[c] = *(const float4 *)(a.qkv_x + 256u * bc + 16u * l16 + 4u * c);
    // every wave's x requests enter the compute unit's memory queue before any weight request (a bare
    // barrier orders the issue and waits for no load): the queue serves them in order
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    uint4 qv[8];
#pragma unroll
    for (uint32_t jj = 0; jj < 8u; ++jj) qv[jj] = *(const uint4 *)(a.qkv_w + wl_quant_off(wg, B, R, jj, sl, rin));
    const uint4 mv = *(const uint4 *)(a.qkv_w + wl_meta_off(wg, B, R, sl, rin));
    uint32_t epv = a.ep[(size_t)g * G * (D / 64u)];               // the epoch the launch's tag follows
    const uint32_t u2 = tid >> 1, hq = tid & 1u, b2 = u2 >> 3, r2 = 16u + (u2 & 7u);
    const uint32_t n2 = wrow(r_0 + r2), B2 = n2 / wg.rb, rin2 = n2 - B2 * wg.rb, R2 = wl_rows(wg, B2);
    const uint32_t sl2 = wl_slot_of(wg, min(b2, nsb - 1u));
    uint4 q4[4];
#pragma unroll
    for (uint32_t jj = 0; jj < 4u; ++jj) q4[jj] = *(const uint4 *)(a.qkv_w + wl_quant_off(wg, B2, R2, 4u * hq + jj, sl2, rin2));
    const uint4 mv2 = *(const uint4 *)(a.qkv_w + wl_meta_off(wg, B2, R2, sl2, rin2));
    __builtin_amdgcn_sched_barrier(0);

    // RMS_NORM: the squares, the two halves of the 128 ordered partials on waves 0 and 1, the scale
    if (b < nsb) {
#pragma unroll
        for (uint32_t c = 0; c < 4u; ++c) *(float4 *)(s_sq + 256u * b + 16u * l16 + 4u * c) = sq4(xv[c]);
    }
    if (tid == 0u) s_ctl[2] = 0u;
    lds_barrier();
    if (v < 2u) {
        const uint32_t i = 64u * v + lane, nk = K >> 7;           // terms per partial
        float p = 0.0f;
        for (uint32_t k0 = 0; k0 < nk; k0 += 16u) {             // 16-read batches: the second unit holds registers
            float t[16];
#pragma unroll
            for (uint32_t k = 0; k < 16u; ++k) t[k] = s_sq[i + 128u * min(k0 + k, nk - 1u)];
#pragma unroll
            for (uint32_t k = 0; k < 16u; ++k) {
                const float q = p + t[k];                         // plain additions: see rms_tree64
                p = k0 + k < nk ? q : p;
            }
        }
        p = rms_tree64(p);
        if (lane == 0u) s_ctl[v] = __float_as_uint(p);
    }
    lds_barrier();
    const float sc = rms_scale(__uint_as_float(s_ctl[0]), __uint_as_float(s_ctl[1]), a.qkv_inv_n, a.qkv_eps);
    if (__builtin_expect(!prep_norm_apply_fast(xv, sc, pv, has_w), 0)) {
#pragma unroll
        for (uint32_t c = 0; c < 4u; ++c) xv[c] = prep_norm_apply(xv[c], sc, pv[c], has_w);
    }
    // QACT A256 of block b (a 16-lane row per block)
    float d;
    int s16;
    bool tiny;
    const uint4 qq = qact_a256_row(xv, &d, &s16, &tiny);
    const int s32 = s16 + dpp_i<kDppXor1>(s16);                   // sum of the 32 quants of a sub-block
    if (b < nsb) {
        *(uint4 *)(s_xq + b * kXq4Stride + 16u * l16) = qq;
        if ((l16 & 1u) == 0u) s_xb[b * 8u + (l16 >> 1)] = s32;
        if (l16 == 0u) s_xd[b] = d;
    }
    if (__ballot(tiny && b < nsb) != 0ull && lane == 0u) s_ctl[2] = 1u;
    lds_barrier();
    const bool slow = s_ctl[2] != 0u;                             // some block has 0 < |Dx| < 2^-60

    // a unit's term = partial p[s] of its row (+0 + term); partials of missing super-blocks are +0
    auto term = [&](int isum, int msum, const uint4 & m, uint32_t s) -> float {
        const float dx = s_xd[min(s, nsb - 1u)];
        const float dq = h2f_fast(m.x & 0xFFFFu), dm = h2f_fast(m.x >> 16);
        float tt;
        if (__builtin_expect(!slow, 1)) tt = 0.0f + ((dq * dx) * (float)isum - (dm * dx) * (float)msum);
        else tt = sadd(0.0f, ssub(smul(smul(dq, dx), i2f(isum)), smul(smul(dm, dx), i2f(msum))));
        return s < nsb ? tt : 0.0f;
    };
    {
        const uint32_t sc = min(b, nsb - 1u);
        int isum, msum;
        q4k_unit_sums<8>(qv, mv, s_xq + sc * kXq4Stride, s_xb + sc * 8u, 0u, isum, msum);
        s_p[16u * l16 + b] = term(isum, msum, mv, b);
    }
    {
        const uint32_t sc = min(b2, nsb - 1u);
        int isum, msum;
        q4k_unit_sums<4>(q4, mv2, s_xq + sc * kXq4Stride, s_xb + sc * 8u, hq, isum, msum);
        isum += dpp_i<kDppXor1>(isum);                            // exact: the pair's two halves
        msum += dpp_i<kDppXor1>(msum);
        const float tt = term(isum, msum, mv2, b2);
        if (hq == 0u) s_p[16u * r2 + b2] = tt;
    }
    lds_barrier();
    // the 16-partial tree of each row (lane i of a 16-lane row holds p[i]): rows 0..15, then 16..23
    auto tree = [&](float y) -> float {
        if (__builtin_expect(!slow, 1)) {
            y = y + dpp_f<kDppXor1>(y);
            y = y + dpp_f<kDppXor2>(y);
            y = y + dpp_f<kDppRowHalfMirror>(y);
            y = y + dpp_f<kDppRowMirror>(y);
            return canon(y);
        }
        y = sadd(y, dpp_f<kDppXor1>(y));
        y = sadd(y, dpp_f<kDppXor2>(y));
        y = sadd(y, dpp_f<kDppRowHalfMirror>(y));
        return sadd(y, dpp_f<kDppRowMirror>(y));
    };
    const float y1 = tree(s_p[tid]);
    if ((tid & 15u) == 0u && r_0 + (tid >> 4) < nset) a.qkv_y[wrow(r_0 + (tid >> 4))] = y1;
    if (v < 2u) {
        const float y2 = tree(s_p[256u + tid]);
        if ((tid & 15u) == 0u && r_0 + 16u + (tid >> 4) < nset) a.qkv_y[wrow(r_0 + 16u + (tid >> 4))] = y2;
    }
    vm_wait();                                                    // the rows are in the L2
    lds_barrier();
    asm volatile("" : "+v"(epv));                                 // a register value: no earlier wait for it
    if (tid == 0u) {
        const uint32_t tagw = tag_after(epv) | (xcc_id() << 28);
        __hip_atomic_store(a.qkv_flag + (size_t)g * 64u + j, tagw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

template <int D, bool ROPE, bool LOCAL, bool QKV>
__global__ __launch_bounds__(256, 4) void k_fa_dec(FaDecArgs a) {
    constexpr uint32_t NBD = D / 32u;                             // K / V blocks of a head
    __shared__ __align__(16) uint8_t lds[QKV && kQkvLds > kDecLds ? kQkvLds : kDecLds];
    uint32_t * s_t64 = (uint32_t *)lds;
    int8_t * s_q = (int8_t *)(lds + 256);                         // [G][D]
    float * s_dx = (float *)(lds + 768);                          // [G][NBD]
    int8_t * s_kq = (int8_t *)(lds + 832);                        // new k row of head g [D], scales [NBD]
    float * s_kd = (float *)(lds + 960);
    int8_t * s_vq = (int8_t *)(lds + 976);                        // new v row [D], scales [NBD]
    float * s_vd = (float *)(lds + 1104);
    float * s_t = (float *)(lds + 1120);                          // [h][b][64] block terms
    float * s_S = (float *)(lds + 5216);                          // [h][64] scores
    float * s_P = (float *)(lds + 6240);                          // [h][64] p
    uint8_t * s_dg = lds + 7264;                                  // [wave][1024] digits
    uint32_t * s_key = (uint32_t *)(lds + 11360);                 // [4] segment maxima (keys)
    float * s_m = (float *)(lds + 11376);                         // [4] chunk maxima

    const uint32_t per_item = 4u * a.maxtiles, nred = a.G * (D / 64u), nseg_slots = a.n_items * per_item;
    FaDecBlock blk = fa_dec_block<LOCAL>(a);
    if constexpr (QKV) {                                          // the Q|K|V rows first in dispatch order
        if (blk.x < a.nq) {
            fa_qkv_rows<D>(a, lds, blk.x, blk.g);
            return;
        }
        blk.x -= a.nq;
    }
    // The KV head's reducers: first in dispatch order when the whole grid is resident at once (they
    // then poll from the start, and finish sooner), after the segments otherwise (then the reducers
    // would hold slots that segments need; segments never wait on reducers)
    const uint32_t xr = a.red_first ? blk.x : blk.x - nseg_slots;
    if (a.red_first ? blk.x < nred : blk.x >= nseg_slots) {
        fa_dec_reduce<D, LOCAL>(a, lds, xr, blk.g);
        return;
    }
    const uint32_t xs = a.red_first ? blk.x - nred : blk.x;       // the segment slot
    const uint32_t item = xs / per_item, tt = (xs / 4u) % a.maxtiles, c = xs & 3u;
    const uint32_t g = blk.g, G = a.G, nh = a.n_head, E = a.E, nbk = E / 32u;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // Everything that does not depend on the work item is requested before the item itself: the item
    // read is a dependent round trip ahead of the K and V addresses, and the query values (whose
    // quantization is the first step) then arrive at the same time as the item.
    // (scalars in device memory are read with vector loads: a scalar load shares its counter with the
    // LDS operations, so every LDS wait of the quantization below would wait for it too)
    // First every address, from the kernel arguments only and branch-free (a branch splits the code, and
    // each argument was then read where first used: one dependent scalar round trip apiece, four to six
    // in a row); then, after a scheduling barrier, every load at once.
    const uint32_t nslot = G * D / 4u;                            // 8 lanes per 32-value block
    const float * qrow = a.q + (size_t)g * G * D;
    const uint32_t kslot = tid - nslot, vslot = kslot - D / 4u;
    const bool is_k = ROPE && tid >= nslot && kslot < D / 4u;
    const bool is_v = ROPE && !is_k && tid >= nslot && vslot < D / 4u;
    const float * src = a.q + (size_t)nh * D + (size_t)g * D + (is_v ? E + 4u * vslot : 4u * (is_k ? kslot : 0u));
    const uint32_t jq = 4u * min(tid, nslot - 1u);
    const float * qsrc = (ROPE && tid >= nslot) ? src : qrow + jq;
    const uint32_t half = a.n_dims / 2u;
    const uint32_t jh0 = tid < nslot ? jq % D : (is_k ? 4u * kslot : D);
    // ROPE NEOX: the 4 values half a rotation away (their own address otherwise: no load waits on a branch)
    const int32_t dj = (ROPE && a.neox && jh0 < a.n_dims) ? (jh0 < half ? (int32_t)half : -(int32_t)half) : 0;
    // ROPE angles of the token (table): lane l's pair for the general form (read across lanes), and
    // the pairs of the lane's own 4 values for the fast form (n_dims >= 8: NORM angles jh0 / 2 .. + 1,
    // NEOX angles jh0 mod half .. + 3; clamped, even, so each float4 is aligned); buffer loads over the
    // table, an empty range without one (such loads return 0 and touch nothing)
    const bool tab_fast = ROPE && a.rtab != nullptr && a.n_dims >= 8u;
    const uint32_t nx = 0u - (a.neox != 0u ? 1u : 0u);            // all ones for NEOX (a select, not a branch)
    const uint32_t ib = (nx & (jh0 < half ? jh0 : (jh0 < a.n_dims ? jh0 - half : 0u))) | (~nx & (min(jh0, a.n_dims) >> 1));
    const uint32_t ia = tab_fast ? min(ib, half - 2u) & ~1u : 0u, ic = tab_fast ? min(ib + 2u, half - 2u) & ~1u : 0u;
    const __amdgpu_buffer_rsrc_t rt = fa_rsrc(a.rtab, ROPE && a.rtab != nullptr ? 4u * a.n_dims : 0u);
    // without a table: the position; with one, an empty range
    const __amdgpu_buffer_rsrc_t rpos = fa_rsrc(a.pos, ROPE && a.rtab == nullptr ? 4u : 0u);
    const __amdgpu_buffer_rsrc_t rcell = fa_rsrc(a.cell, ROPE ? 8u : 0u);
    const __amdgpu_buffer_rsrc_t rep = fa_rsrc(a.ep + (size_t)g * G * (D / 64u), 4u);
    const uint32_t * itp = (const uint32_t *)(a.items + item) + min(lane, 8u);
    __builtin_amdgcn_sched_barrier(0);

    // the work item first, one word per lane: the oldest load returns first (loads retire in order), so
    // the K and V addresses, which depend on it, wait for it alone; the ROPE and quantization of the
    // query then run while K and V fly (a vector load: waiting for it does not wait for LDS traffic)
    static_assert(sizeof(FaItem) == 36, "FaItem: 9 words");
    const uint32_t itw = *itp;
    const int64_t cell_new = ROPE ? (int64_t)__builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rcell, 0, 0, 0))
                                  : (int64_t)-1;
    const int32_t pos = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rpos, 0, 0, 0);
    float2 cs_tab = make_float2(0.0f, 0.0f);
    float4 cs_a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), cs_b = cs_a;
    if constexpr (ROPE) {
        cs_tab = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rt, 8u * min(lane, half - 1u), 0, 0));
        cs_a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rt, 8u * ia, 0, 0));
        cs_b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rt, 8u * ic, 0, 0));
    }
    float4 qv0, qpart;
    if constexpr (!QKV) {                                         // (in the launch: after its rows' flags)
        qv0 = *(const float4 *)qsrc;
        qpart = ROPE ? *(const float4 *)(qsrc + dj) : qv0;
    }
    // the EXPK table (kernel-argument memory) and the epochs last: nothing before the quantization's LDS
    // stores waits for them (loads retire in order; the epochs were written by the previous launch, in
    // a decode layer's sequence too long ago to be in a cache)
    const uint32_t t64v = a.ex.t64[lane];
    // the launch's tag: reducer 0's epoch of the KV head + 1 (the epochs advance at the end of a launch)
    const uint32_t epv = __builtin_amdgcn_raw_buffer_load_b32(rep, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    // what this workgroup writes carries its XCD in the tag's high bits (read here, after the loads
    // above: the register read is a volatile asm, which no load is scheduled across)
    const uint32_t xcc = xcc_id();
    const uint32_t tag = tag_after(epv), tagw = tag | (xcc << 28);

    // ---- the work item; the segment's K requested (ROPE and QACT below run while it flies) ----
    FaItem it;
    it.t = __builtin_amdgcn_readlane(itw, 0);
    it.u0 = __builtin_amdgcn_readlane(itw, 1);
    it.n = __builtin_amdgcn_readlane(itw, 2);
    it.c_lo = __builtin_amdgcn_readlane(itw, 3);
    it.c_hi = __builtin_amdgcn_readlane(itw, 4);
    it.general = __builtin_amdgcn_readlane(itw, 5);
    it.s_off = __builtin_amdgcn_readlane(itw, 6);
    it.tile0 = __builtin_amdgcn_readlane(itw, 7);
    it.ntiles = __builtin_amdgcn_readlane(itw, 8);
    const FaSeg sg(it, c);
    if (tt >= sg.nseg) return;                                    // no such segment (block-uniform)
    // A short lone segment (a tail chunk's: fewer than 4 groups) shares its compute unit with two full
    // segments and, the youngest, was served last: it ended ~1-1.5 us after them and held up the
    // reducers. Its waves issue first.
    if (a.n_items > 1u && sg.nseg == 1u && sg.nu < 4u) __builtin_amdgcn_s_setprio(2);
    const uint32_t ng = (a.kc.kv_size + 15u) / 16u;
    // the segment's groups (clamped: loads of a missing group stay inside the item)
    uint32_t ug[4];
    bool gv[4];
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        const uint32_t gi = 4u * tt + k;
        gv[k] = gi < sg.nu;
        ug[k] = min(sg.u_first + 4u * min(gi, sg.nu - 1u), ng - 1u);
    }
    // K: thread = (cell j, block b = wave)
    const uint32_t j = lane, kkj = j >> 4, rrj = j & 15u;
    const uint32_t bk = wave < NBD ? wave : 0u;
    const uint8_t * kbase = a.kc.base + a.kc.quant_off + ((size_t)ug[kkj] * (E / 16u) + (size_t)g * (D / 16u) + 2u * bk) * 256u +
                            (size_t)rrj * 16u;
    int4 kr0 = *(const int4 *)kbase, kr1 = *(const int4 *)(kbase + 256u);
    uint32_t km = ((const uint16_t *)a.kc.base)[((size_t)ug[kkj] * nbk + (size_t)g * NBD + bk) * 16u + rrj];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (QKV) {
        // every wave polls the flags of its KV head's row workgroups (lane j: workgroup j), then loads its
        // Q|K|V values (agent-coherent loads: the rows were stored in this launch)
        const uint32_t * fl = a.qkv_flag + (size_t)g * 64u + min(lane, a.nq - 1u);
        uint32_t fv = 0u, spins = 0;
        for (;;) {
            fv = ld_co_u(fl);
            if (__all(tag_is(fv, tag))) break;
            if (__builtin_expect(++spins >= a.spin_max, 0)) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);                  // the value loads stay behind the poll
        if (__builtin_expect(__any(tag_is(fv, tag) && (fv >> 28) != xcc), 0) && lane == 0u && a.bad != nullptr)
            __hip_atomic_fetch_or(a.bad, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const __amdgpu_buffer_rsrc_t rq = fa_rsrc(a.q, 4u * (nh * D + 2u * E));
        const uint32_t qo = 4u * (uint32_t)(qsrc - a.q);
        qv0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo, 0, kSc1));
        qpart = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 4u * (uint32_t)dj, 0, kSc1));
    }

    // ---- ROPE of the query heads and the new k row ----
    float4 r = qv0;
    if constexpr (ROPE) {
        float c_l, s_l;
        if (__builtin_expect(a.rtab != nullptr, 1)) {
            c_l = cs_tab.x;
            s_l = cs_tab.y;
        } else {
            rope_cs_lane(pos, half, a.ts, a.m, lane, &c_l, &s_l);
        }
        float4 rot;
        if (__builtin_expect(!(tab_fast && rope4_tab_fast(rot, qv0, qpart, jh0, a.n_dims, a.neox != 0u, cs_a, cs_b)), 0))
            rot = rope4(qv0, qpart, jh0, a.n_dims, a.neox != 0u, c_l, s_l);   // every lane (bpermute)
        r = is_v ? qv0 : rot;
    }

    // ---- QACT of the query heads, the new k and v rows ----
    float Dq;
    const uint32_t qq = qact_a32_lane(r, &Dq);                    // every lane (8-lane groups)
    if (tid < nslot) {
        *(uint32_t *)(s_q + 4u * tid) = qq;
        if ((lane & 7u) == 0u) s_dx[tid >> 3] = Dq;
    } else if (is_k) {
        *(uint32_t *)(s_kq + 4u * kslot) = qq;
        if ((lane & 7u) == 0u) s_kd[kslot >> 3] = Dq;
    } else if (is_v) {
        *(uint32_t *)(s_vq + 4u * vslot) = qq;
        if ((lane & 7u) == 0u) s_vd[vslot >> 3] = Dq;
    }
    if (tid < 64u) s_t64[tid] = t64v;
    if constexpr (ROPE) {
        const bool cell_ok = cell_new >= 0 && cell_new < (int64_t)a.kc.kv_size && cell_new < (int64_t)a.vc.kv_size;
        if (__builtin_expect(item == 0u && tt == 0u && c == (it.u0 & 3u), 0)) {       // the caches' copy of the new rows
            if (cell_ok && (is_k || is_v))
            {
                KvArgs kv;                                        // per-lane choice of the plane, field by field
                kv.base = is_k ? a.kc.base : a.vc.base;
                kv.quant_off = is_k ? a.kc.quant_off : a.vc.quant_off;
                kv.E = a.kc.E;
                kv.kv_size = is_k ? a.kc.kv_size : a.vc.kv_size;
                kv_store_unit(kv, is_k ? 0u : 1u, (uint32_t)cell_new, g * D + 4u * (is_k ? kslot : vslot), qq, Dq,
                              (lane & 7u) == 0u);
            }
            if (!cell_ok && tid == 0u && g == 0u && a.bad != nullptr) *a.bad = 1;
        }
    }
    lds_barrier();                                                // K stays in flight
    // V is requested only now: K streams alone first (the scores wait for it; V is needed at P.V)
    // V: wave b = value block b; lane (head row hr, group kk, cell quad) for the weights, lane
    // (value l % 16, group l / 16) for the matrix-core operand
    const uint32_t hr = lane >> 4, kk = (lane >> 2) & 3u, quad = lane & 3u;
    const uint32_t bv = wave < NBD ? wave : 0u, b0 = bv & ~1u;    // the 64-value slice: blocks b0, b0 + 1
    // V: the scales of the lane's 4 cells in the slice's two blocks (8 contiguous bytes each), and the
    // matrix-core operand
    uint2 mvb[2];
#pragma unroll
    for (uint32_t e = 0; e < 2u; ++e)
        mvb[e] = *(const uint2 *)((const uint16_t *)a.vc.base + ((size_t)ug[kk] * nbk + (size_t)g * NBD + b0 + e) * 16u +
                                  4u * quad);
    const uint8_t * vq = a.vc.base + a.vc.quant_off + ((size_t)ug[lane >> 4] * E + (size_t)g * D + 32u * bv + (lane & 15u)) * 16u;
    int4 bq0 = *(const int4 *)vq, bq1 = *(const int4 *)(vq + 256u);
    __builtin_amdgcn_sched_barrier(0);

    // ---- scores: the block terms of (cell j, block b) for every head ----
    const uint32_t u_j = ug[kkj];
    const int64_t cell_j = 16 * (int64_t)u_j + rrj;
    if (wave < NBD) {
        if (__builtin_expect(ROPE && cell_j == cell_new, 0)) {                         // the new cell: the fresh k row
            kr0 = *(const int4 *)(s_kq + 32u * wave);
            kr1 = *(const int4 *)(s_kq + 32u * wave + 16u);
            km = f2h_exact(s_kd[wave]);
        }
        const float dk = h2f_fast(km);
        for (uint32_t h = 0; h < G; ++h) {
            const int4 * xq = (const int4 *)(s_q + (size_t)h * D + 32u * wave);
            const int4 x0 = xq[0], x1 = xq[1];
            int is = dot4(kr0.x, x0.x, 0);
            is = dot4(kr0.y, x0.y, is);
            is = dot4(kr0.z, x0.z, is);
            is = dot4(kr0.w, x0.w, is);
            is = dot4(kr1.x, x1.x, is);
            is = dot4(kr1.y, x1.y, is);
            is = dot4(kr1.z, x1.z, is);
            is = dot4(kr1.w, x1.w, is);
            // SEG (AT 6.2): p_k = +0 + (dK Dx) f32(isum); |terms| >= 2^-48 or 0 (fp16 scales); the +0
            // goes to the tree's result (see k_fa_qk)
            s_t[(h * 4u + wave) * 64u + j] = (dk * s_dx[h * NBD + wave]) * (float)is;
        }
    }
    __syncthreads();
    // wave h = head h: tree16 over the block terms, the mask, the segment maximum
    const uint32_t floor_key = maxt_key_f(bf(kMFloor));
    const uint32_t jc = 16u * (u_j - it.u0) + rrj;                // cell index in the chunk
    const bool in = gv[kkj];
    const bool vis = in && (it.general || (jc >= it.c_lo && jc < it.c_hi));
    if (wave < G) {
        const uint32_t h = wave;
        float s = bf(kNegInf);
        if (vis) {
            float p[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) p[k] = (uint32_t)k < NBD ? s_t[(h * 4u + (uint32_t)k) * 64u + j] : 0.0f;
#pragma unroll
            for (int w = 16; w > 1; w >>= 1)
#pragma unroll
                for (int k = 0; k < w / 2; ++k) p[k] = p[2 * k] + p[2 * k + 1];
            s = canon(p[0] + 0.0f);
            if (it.general) {
                const float mval = a.mask[(size_t)it.t * a.mstride + (uint32_t)cell_j];
                s = fb(mval) == kNegInf ? bf(kNegInf) : sadd(s, mval);
            }
        }
        s_S[h * 64u + j] = s;
        const uint32_t key = wave_max_u(in ? maxt_key_f(s) : floor_key);
        if (lane == 0u) s_key[h] = key;
    } else if (wave < 4u && lane == 0u) {
        s_key[wave] = floor_key;
    }
    __syncthreads();

    // ---- publish the segment maxima; wait for the item's segments ----
    // A slot holds (key, tag) for each of 4 heads (32 bytes, written as two 16-byte stores: a reader
    // sees whole 8-byte pairs); tag = the launch's epoch + 1, so slots of earlier launches never match.
    const uint32_t nslots = a.n_items * a.maxtiles * 4u;          // segment slots per KV head
    const __amdgpu_buffer_rsrc_t rk = fa_rsrc(a.keys + (size_t)g * nslots * 8u, nslots * 32u);
    const uint32_t my_slot = (item * a.maxtiles + tt) * 4u + c;
    if (tid == 0u) {
        st_co16<LOCAL>(rk, my_slot * 32u, make_uint4(s_key[0], tagw, s_key[1], tagw));
        st_co16<LOCAL>(rk, my_slot * 32u + 16u, make_uint4(s_key[2], tagw, s_key[3], tagw));
    }
    if (wave == 0u) {
        // lane: half (lane & 1: heads 2 hf, 2 hf + 1) of segment sl = lane / 2 (tile sl / 4, channel sl % 4)
        const uint32_t sl = lane >> 1, hf = lane & 1u, tl = sl >> 2, cl = sl & 3u;
        const FaSeg fs(it, cl);
        const bool want = tl < a.maxtiles && tl < fs.nseg;
        const uint32_t off = ((item * a.maxtiles + min(tl, a.maxtiles - 1u)) * 4u + cl) * 32u + 16u * hf;
        uint4 v = make_uint4(floor_key, tagw, floor_key, tagw);
        uint32_t spins = 0;
        for (;;) {
            if (want) v = ld_co16(rk, off);
            if (__all(tag_is(v.y, tag) && tag_is(v.w, tag))) break;
            if (__builtin_expect(++spins >= a.spin_max, 0)) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // (a word the wait gave up on may be another launch's: only this launch's words count here)
        if (LOCAL && __any((tag_is(v.y, tag) && (v.y >> 28) != xcc) || (tag_is(v.w, tag) && (v.w >> 28) != xcc)) &&
            lane == 0u && a.bad != nullptr)
            __hip_atomic_fetch_or(a.bad, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // chunk maxima: MAXOUT of the floor and the segment maxima (AT 6.3)
        const uint32_t a0 = want && hf == 0u ? v.x : floor_key, a1 = want && hf == 0u ? v.z : floor_key;
        const uint32_t a2 = want && hf == 1u ? v.x : floor_key, a3 = want && hf == 1u ? v.z : floor_key;
        const uint32_t k0 = wave_max_u(umax_u(a0, floor_key)), k1 = wave_max_u(umax_u(a1, floor_key));
        const uint32_t k2 = wave_max_u(umax_u(a2, floor_key)), k3 = wave_max_u(umax_u(a3, floor_key));
        if (lane < 4u) s_m[lane] = maxt_unkey(lane == 0u ? k0 : lane == 1u ? k1 : lane == 2u ? k2 : k3);
    }
    __syncthreads();
    if (item < a.n_items && tt == 0u && c == (it.u0 & 3u) && tid < G)   // the item's first segment records them
        st_tag<LOCAL>(a.m_item + (size_t)item * nh + g * G + tid, s_m[tid], tagw);

    // ---- EXP (wave h = head h) and the segment's LSUM ----
    const size_t segrow = ((size_t)(it.tile0 + tt) * 4u + c) * nh + (size_t)g * G;   // + head
    if (wave < G) {
        const uint32_t h = wave;
        // EXPK results are zero, normal, Inf or NaN (never subnormal)
        const float ez = expk_diff(s_S[h * 64u + j], s_m[h], a.scale, a.ex, s_t64);
        const float p = in ? ez : 0.0f;
        s_P[h * 64u + j] = p;
        const uint32_t f = f_field(p);
        const bool badl = __any(f == 255u);
        const uint32_t pe = wave_max_u(f == 255u ? 0u : f);
        const int32_t w = f == 255u ? 0 : bf_int_n(p, (int32_t)pe - 127);
        const int32_t lsum = wave_sum_i(w);
        if (lane == 0u)
            st_tag<LOCAL>(a.seg_l + segrow + h, badl ? bf(kNaN) : (pe == 0u ? 0.0f : bf_scale((float)lsum, (int32_t)pe - 150)), tagw);
    }
    __syncthreads();

    // ---- P.V: wave b = value block b ----
    if (wave < NBD) {
        const bool head_ok = hr < G;
        const float4 pv = *(const float4 *)(s_P + min(hr, G - 1u) * 64u + 16u * kk + 4u * quad);
        const float pz[4] = { head_ok ? pv.x : 0.0f, head_ok ? pv.y : 0.0f, head_ok ? pv.z : 0.0f, head_ok ? pv.w : 0.0f };
        const uint32_t own = bv - b0;                             // the wave's block in the slice
        if constexpr (ROPE) {                                     // the new cell: the fresh v scales
            const int64_t base = 16 * (int64_t)ug[kk] + 4u * quad;
            if (cell_new >= base && cell_new < base + 4) {
                const uint32_t i = (uint32_t)(cell_new - base), sh = 16u * (i & 1u), keep = ~(0xFFFFu << sh);
#pragma unroll
                for (uint32_t e = 0; e < 2u; ++e) {
                    const uint32_t h16 = f2h_exact(s_vd[b0 + e]) << sh;
                    if (i < 2u) mvb[e].x = (mvb[e].x & keep) | h16;
                    else mvb[e].y = (mvb[e].y & keep) | h16;
                }
            }
        }
        // weights w = p dV of the slice's two blocks, a subnormal product flushed to zero
        float w[4][2];
        uint32_t ex = 0u, nfm = 0u;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const bool live = (fb(pz[i]) & 0x7FFFFFFFu) != 0u;
#pragma unroll
            for (uint32_t e = 0; e < 2u; ++e) {
                const float we = live ? pz[i] * h2f_fast(((i < 2u ? mvb[e].x : mvb[e].y) >> (16u * (i & 1u))) & 0xFFFFu) : 0.0f;
                const uint32_t f = f_field(we);
                nfm |= (f == 255u ? 1u : 0u) << e;
                w[i][e] = f == 0u ? 0.0f : we;
                ex = max(ex, f == 255u ? 0u : f);
            }
        }
        const uint32_t ef = row16_umax(ex);                        // E_S over the head's 64 cells and the slice
        const bool any = ef != 0u;
        const int32_t es = (int32_t)ef - 127;
        const bool bad = ((row16_or(nfm) >> own) & 1u) != 0u;
        const bool use = any && !bad;
        uint32_t P[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const int32_t W = use ? bf_int_n(w[i][own], es) : 0;
            P[i] = ((uint32_t)W + 0x80808080u) ^ 0x80808080u;      // byte k = digit k of W
        }
        uint8_t * dg = s_dg + wave * 1024u;
        const uint32_t lo01 = __builtin_amdgcn_perm(P[1], P[0], 0x05010400u);
        const uint32_t lo23 = __builtin_amdgcn_perm(P[3], P[2], 0x05010400u);
        const uint32_t hi01 = __builtin_amdgcn_perm(P[1], P[0], 0x07030602u);
        const uint32_t hi23 = __builtin_amdgcn_perm(P[3], P[2], 0x07030602u);
        const uint32_t q4[4] = { __builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                 __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u) };
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) *(uint32_t *)(dg + ((hr * 4u + k) * 4u + kk) * 16u + 4u * quad) = q4[k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // matrix core: rows (head, digit), K = the 16 cells of group l / 16, columns 16 values
        const v4i_fa Aop = *(const v4i_fa *)(dg + ((lane & 15u) * 4u + (lane >> 4)) * 16u);
        if constexpr (ROPE) {                                     // the new cell's v quants
            const int64_t base = 16 * (int64_t)ug[lane >> 4];
            if (cell_new >= base && cell_new < base + 16) {
                const uint32_t r = (uint32_t)(cell_new - base);
                bq0 = put_byte(bq0, r, (uint8_t)s_vq[32u * bv + (lane & 15u)]);
                bq1 = put_byte(bq1, r, (uint8_t)s_vq[32u * bv + 16u + (lane & 15u)]);
            }
        }
        const uint32_t hres = lane >> 4;
        const bool store = hres < G;
        uint64_t * orow = a.seg_o + (segrow + min(hres, G - 1u)) * D + 32u * bv + (lane & 15u);
#pragma unroll
        for (uint32_t hf = 0; hf < 2u; ++hf) {
            const int4 bq = hf ? bq1 : bq0;
            const v4i_fa Bop = { bq.x, bq.y, bq.z, bq.w };
            v4i_fa acc = { 0, 0, 0, 0 };
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(Aop, Bop, acc, 0, 0, 0);
            const float cval = bad ? bf(kNaN) : (any ? bf_scale(digits_rne24(acc), es - 23) : 0.0f);
            if (store) st_tag<LOCAL>(orow + 16u * hf, cval, tagw);
        }
    }
}

// The reducers of a KV head: workgroup (head r, 64-value part vp), thread = (value, channel c): channel c's
// chains of segment results in order (AT 6.4 O, 6.5 l), CTREE over the channels (AT 5.6), the merge of
// the items in chunk order (AMERGE) and ANORM (AT 5.7). With one round of items (<= kRedItems or exactly
// 4: the decode at up to ~8 K cells) the row-sum side comes first: the chunk maxima and the segments' row sums
// are stored at the segments' EXP step, so the merge factors and the l merge are done while the
// segments' P.V still runs, and only the O side waits for the last segment. Several rounds poll each
// round's outputs, row sums and maxima together (their reducers start late: the grid is larger than the
// resident workgroups). Every result carries
// the launch's tag (an epoch + 1, one epoch word per reducer, each advanced by its reducer at its end):
// nothing is cleared, and a store that lands after an expired wait carries a tag no later launch
// expects. A reducer only waits for segments, which come before it in dispatch order.
constexpr uint32_t kRedItems = 3;                                 // items loaded per round (several rounds)

template <int D, bool LOCAL>
__device__ __forceinline__ void fa_dec_reduce(const FaDecArgs & a, uint8_t * lds, uint32_t ri, uint32_t g) {
    uint32_t * s_t64 = (uint32_t *)lds;
    uint32_t * s_it = (uint32_t *)(lds + 256);                    // [item] u0, n, tile0 (<= 256 items)
    float * s_x = (float *)(lds + 256 + 3072);                    // [item][channel][64] O, then [item][channel] l
    const uint32_t G = a.G, nh = a.n_head, ni = a.n_items;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    constexpr uint32_t NVP = D / 64u;                             // 64-value parts of a head
    const uint32_t r = ri / NVP, vp = ri % NVP, hh = g * G + r;
    const uint32_t c = tid >> 6, v = 64u * vp + lane;             // channel c, value v
    uint32_t * ep = a.ep + (size_t)g * G * NVP + ri;              // this reducer's epoch of the KV head
    const uint32_t tag = tag_after(*ep), xcc = xcc_id();
    s_t64[lane] = a.ex.t64[lane];
    for (uint32_t k = tid; k < ni; k += blockDim.x) {
        const FaItem ik = a.items[k];
        s_it[3u * k] = ik.u0;
        s_it[3u * k + 1u] = ik.n;
        s_it[3u * k + 2u] = ik.tile0;
    }
    __syncthreads();
    // the segments of channel c of the round's items
    auto round_items = [&](uint32_t k0, auto & ns, auto & tl0) {
        constexpr uint32_t R = sizeof(ns) / sizeof(ns[0]);
#pragma unroll
        for (uint32_t kq = 0; kq < R; ++kq) {
            const uint32_t k = min(k0 + kq, ni - 1u);
            FaItem ik{};
            ik.u0 = s_it[3u * k];
            ik.n = s_it[3u * k + 1u];
            tl0[kq] = s_it[3u * k + 2u];
            ns[kq] = FaSeg(ik, c).nseg;
        }
    };
    float O = 0.0f, l = 0.0f, mr = 0.0f;
    // One round of R items (R = 3, or 4 for exactly 4 items: one round instead of 3 + 1)
    auto one_round = [&]<uint32_t R>() {
        // One round: the chunk maxima first (the merge factors on wave 0), then the row sums (published at
        // the segments' EXP step) and the l merge on wave 0 while the other waves already poll the outputs.
        const uint32_t k0 = 0;
        float fx = 0.0f;
        uint32_t ns[R], tl0[R];
        round_items(k0, ns, tl0);
        uint64_t pl[R], pm;
        uint32_t spins = 0;
        // the chunk maxima first (an item's first segment stores them once its chunk's segments have
        // met, well before the row sums of the last segments): wave 0 forms the merge factors while the
        // row sums are still coming
        for (;;) {
            pm = ld_tag(a.m_item + (size_t)min(k0 + min(lane, R - 1u), ni - 1u) * nh + hh);
            if (__all(tag_is((uint32_t)(pm >> 32), tag))) break;
            if (__builtin_expect(++spins >= a.spin_max, 0)) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        float mkr[R], mrun[R];
        {
            // the running maxima are a MAXT scan of the chunk maxima, so every merge factor of the round is
            // known now: lane 2 kq + b evaluates EXP((prev - mrun_kq) scale) for b = 0 (the running sums) or
            // EXP((m_kq - mrun_kq) scale) for b = 1 (the chunk's), all at once; kept for both merges
            float prev[R];
            float m = mr;
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {
                mkr[kq] = bf((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)pm, (int)kq));
                prev[kq] = m;
                mrun[kq] = k0 + kq == 0u ? mkr[kq] : maxt(m, mkr[kq]);
                m = mrun[kq];
            }
            if (c == 0u) {
                const uint32_t jk = min(lane >> 1, R - 1u);  // lanes 2 kq, 2 kq + 1 hold item kq's factors
                float from = 0.0f, to = 0.0f;
#pragma unroll
                for (uint32_t kq = 0; kq < R; ++kq)
                    if (jk == kq) {
                        from = (lane & 1u) ? mkr[kq] : prev[kq];
                        to = mrun[kq];
                    }
                fx = expk_diff(from, to, a.scale, a.ex, s_t64);
            }
        }
        // the row sums of channel c's segments
        spins = 0;
        for (;;) {
            bool ok = true;
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {
                const size_t lrow = ((size_t)(tl0[kq] + min(lane, max(ns[kq], 1u) - 1u)) * 4u + c) * nh + hh;
                pl[kq] = ld_tag(a.seg_l + lrow);
                ok &= lane >= ns[kq] || tag_is((uint32_t)(pl[kq] >> 32), tag);
            }
            if (__all(ok)) break;
            if (__builtin_expect(++spins >= a.spin_max, 0)) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
#pragma unroll
        for (uint32_t kq = 0; kq < R; ++kq) {             // channel c's segment sums in order
            float Lc = 0.0f;
#pragma unroll
            for (uint32_t sgi = 0; sgi < 8u; ++sgi)
                if (sgi < ns[kq]) Lc = Lc + bf((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)pl[kq], (int)sgi));   // see ctree4_l
            if (lane == 0u) s_x[1024u + kq * 4u + c] = Lc;
        }
        __syncthreads();
        if (c == 0u) {
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {        // CTREE, then AMERGE, in chunk order: l
                if (k0 + kq >= ni) break;
                const float * xl4 = s_x + 1024u + kq * 4u;
                const float lk = ctree4_l(xl4[0], xl4[1], xl4[2], xl4[3]);
                if (k0 + kq == 0u) {
                    l = lk;
                } else {
                    const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq));
                    const float fbv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq + 1));
                    l = sadd_c(smul_c(l, fa), smul_c(lk, fbv));
                }
                mr = mrun[kq];
            }
        }
        // ---- the segments' outputs: lane v's value of channel c in each segment ----
        uint64_t po[R][8];
        spins = 0;
        for (;;) {
            bool ok = true, near = true;                          // near: every writer shared this XCD
            round_items(k0, ns, tl0);                             // (re-read: fewer registers held)
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {
#pragma unroll
                for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                    const size_t row = ((size_t)(tl0[kq] + min(sgi, max(ns[kq], 1u) - 1u)) * 4u + c) * nh + hh;
                    po[kq][sgi] = ld_tag(a.seg_o + row * D + v);
                }
            }
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {
#pragma unroll
                for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                    ok &= sgi >= ns[kq] || tag_is((uint32_t)(po[kq][sgi] >> 32), tag);
                    near &= sgi >= ns[kq] || (uint32_t)(po[kq][sgi] >> 60) == xcc;
                }
            }
            if (__all(ok)) {
                if (__builtin_expect(LOCAL && __any(!near) && lane == 0u && a.bad != nullptr, 0))
                    __hip_atomic_fetch_or(a.bad, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if (__builtin_expect(++spins >= a.spin_max, 0)) {
                if (lane == 0u && a.bad != nullptr)
                    __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
#pragma unroll
        for (uint32_t kq = 0; kq < R; ++kq) {             // channel c's segments in order
            float Oc = 0.0f;
#pragma unroll
            for (uint32_t sgi = 0; sgi < 8u; ++sgi)
                if (sgi < ns[kq]) Oc = sadd_z(Oc, bf((uint32_t)po[kq][sgi]));
            s_x[(kq * 4u + c) * 64u + lane] = Oc;
        }
        __syncthreads();
        if (c == 0u) {                                            // CTREE, then AMERGE, in chunk order: O
#pragma unroll
            for (uint32_t kq = 0; kq < R; ++kq) {
                if (k0 + kq >= ni) break;
                const float * x = s_x + kq * 256u + lane;
                const float ok = ctree4_o(x[0], x[64], x[128], x[192]);
                if (k0 + kq == 0u) {
                    O = ok;
                } else {
                    const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq));
                    const float fbv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq + 1));
                    O = sadd_z(smul_z(O, fa), smul_z(ok, fbv));
                }
            }
        }
    };
    if (__builtin_expect(ni <= kRedItems, 1)) {
        one_round.template operator()<kRedItems>();
    } else if (ni == 4u) {
        one_round.template operator()<4u>();
    } else {
        // Several rounds: each round polls its items' outputs, row sums and maxima together
        for (uint32_t k0 = 0; k0 < ni; k0 += kRedItems) {
            // wave c polls its round's results until every one carries the launch's tag: lane v's value of
            // channel c in each segment, lane s's row sum of segment s, lane kq's chunk maximum of item kq
            uint64_t po[kRedItems][8], pl[kRedItems], pm;
            uint32_t ns[kRedItems];
            uint32_t spins = 0;
            for (;;) {
                bool ok = true;
#pragma unroll
                for (uint32_t kq = 0; kq < kRedItems; ++kq) {
                    const uint32_t k = min(k0 + kq, ni - 1u);
                    FaItem ik{};
                    ik.u0 = s_it[3u * k];
                    ik.n = s_it[3u * k + 1u];
                    const uint32_t tile0 = s_it[3u * k + 2u];
                    const FaSeg sc(ik, c);
                    ns[kq] = sc.nseg;
#pragma unroll
                    for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                        const size_t row = ((size_t)(tile0 + min(sgi, max(sc.nseg, 1u) - 1u)) * 4u + c) * nh + hh;
                        po[kq][sgi] = ld_tag(a.seg_o + row * D + v);
                    }
                    const size_t lrow = ((size_t)(tile0 + min(lane, max(sc.nseg, 1u) - 1u)) * 4u + c) * nh + hh;
                    pl[kq] = ld_tag(a.seg_l + lrow);
                }
                pm = ld_tag(a.m_item + (size_t)min(k0 + min(lane, kRedItems - 1u), ni - 1u) * nh + hh);
                bool near = true;                                     // every writer shared this XCD
#pragma unroll
                for (uint32_t kq = 0; kq < kRedItems; ++kq) {
#pragma unroll
                    for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                        ok &= sgi >= ns[kq] || tag_is((uint32_t)(po[kq][sgi] >> 32), tag);
                        near &= sgi >= ns[kq] || (uint32_t)(po[kq][sgi] >> 60) == xcc;
                    }
                    ok &= lane >= ns[kq] || tag_is((uint32_t)(pl[kq] >> 32), tag);
                }
                ok &= tag_is((uint32_t)(pm >> 32), tag);
                if (__all(ok)) {
                    if (__builtin_expect(LOCAL && __any(!near) && lane == 0u && a.bad != nullptr, 0))
                        __hip_atomic_fetch_or(a.bad, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                if (__builtin_expect(++spins >= a.spin_max, 0)) {
                    if (lane == 0u && a.bad != nullptr)
                        __hip_atomic_fetch_or(a.bad, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            float xo[kRedItems][8], xl[kRedItems][8], mkr[kRedItems];
#pragma unroll
            for (uint32_t kq = 0; kq < kRedItems; ++kq) {
#pragma unroll
                for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                    xo[kq][sgi] = bf((uint32_t)po[kq][sgi]);
                    xl[kq][sgi] = bf((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)pl[kq], (int)sgi));
                }
                mkr[kq] = bf((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)pm, (int)kq));
            }
#pragma unroll
            for (uint32_t kq = 0; kq < kRedItems; ++kq) {             // channel c's segments in order
                float Oc = 0.0f, Lc = 0.0f;
#pragma unroll
                for (uint32_t sgi = 0; sgi < 8u; ++sgi) {
                    if (sgi < ns[kq]) {
                        Oc = sadd_z(Oc, xo[kq][sgi]);
                        Lc = Lc + xl[kq][sgi];                    // see ctree4_l
                    }
                }
                s_x[(kq * 4u + c) * 64u + lane] = Oc;
                if (lane == 0u) s_x[1024u + kq * 4u + c] = Lc;
            }
            __syncthreads();
            if (c == 0u) {                                            // CTREE, then AMERGE, in chunk order
                // the running maxima are a MAXT scan of the chunk maxima, so every merge factor of the round is
                // known before the merge: lane 2 kq + b evaluates EXP((prev - mrun_kq) scale) for b = 0 (the
                // running sums) or EXP((m_kq - mrun_kq) scale) for b = 1 (the chunk's), all at once
                float mrun[kRedItems], prev[kRedItems];
                float m = mr;
#pragma unroll
                for (uint32_t kq = 0; kq < kRedItems; ++kq) {
                    prev[kq] = m;
                    mrun[kq] = k0 + kq == 0u ? mkr[kq] : maxt(m, mkr[kq]);
                    m = mrun[kq];
                }
                const uint32_t jk = min(lane >> 1, kRedItems - 1u);  // lanes 2 kq, 2 kq + 1 hold item kq's factors
                float from = 0.0f, to = 0.0f;
#pragma unroll
                for (uint32_t kq = 0; kq < kRedItems; ++kq)
                    if (jk == kq) {
                        from = (lane & 1u) ? mkr[kq] : prev[kq];
                        to = mrun[kq];
                    }
                const float fx = expk_diff(from, to, a.scale, a.ex, s_t64);
#pragma unroll
                for (uint32_t kq = 0; kq < kRedItems; ++kq) {
                    if (k0 + kq >= ni) break;
                    const float * x = s_x + kq * 256u + lane;
                    const float ok = ctree4_o(x[0], x[64], x[128], x[192]);
                    const float * xl4 = s_x + 1024u + kq * 4u;
                    const float lk = ctree4_l(xl4[0], xl4[1], xl4[2], xl4[3]);
                    if (k0 + kq == 0u) {
                        O = ok;
                        l = lk;
                    } else {
                        const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq));
                        const float fbv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fx), 2 * (int)kq + 1));
                        l = sadd_c(smul_c(l, fa), smul_c(lk, fbv));
                        O = sadd_z(smul_z(O, fa), smul_z(ok, fbv));
                    }
                    mr = mrun[kq];
                }
            }
            __syncthreads();
        }
    }
    if (c == 0u) a.out[(size_t)hh * D + v] = smul_n(O, srcp(maxt(l, bf(kLFloor))));   // ANORM
    // every segment of the KV head has read the epochs (its flag is in): the next launch's tags
    if (tid == 0u) st_co_u(ep, tag);
}

}  // namespace tsr

int tsr_launch_fa_dec(const tsr::FaDecArgs & a, hipStream_t s) {
    // (Q|K|V rows,) segments and reducers of each KV head
    const uint32_t per_head = a.n_items * a.maxtiles * 4u + a.G * (a.D / 64u) + (a.qkv_w != nullptr ? a.nq : 0u);
    const bool local = a.n_xcd != 0u && a.n_head_kv % a.n_xcd == 0u;
    const dim3 grid = local ? dim3(per_head * a.n_head_kv, 1) : dim3(per_head, a.n_head_kv);
    const bool rope = a.cell != nullptr;
    if (a.qkv_w != nullptr) {                                     // the host checked the shape
        if (!local || !rope || a.qkv_K > tsr::kQkvMaxK || a.nq > 64u) return -2;
        if (a.D == 128u) hipLaunchKernelGGL((tsr::k_fa_dec<128, true, true, true>), grid, dim3(256), 0, s, a);
        else if (a.D == 64u) hipLaunchKernelGGL((tsr::k_fa_dec<64, true, true, true>), grid, dim3(256), 0, s, a);
        else return -2;
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
#define TSR_DEC(DD, RR, LL) hipLaunchKernelGGL((tsr::k_fa_dec<DD, RR, LL, false>), grid, dim3(256), 0, s, a)
    switch (a.D * 4u + (rope ? 2u : 0u) + (local ? 1u : 0u)) {
        case 256: TSR_DEC(64, false, false); break;
        case 257: TSR_DEC(64, false, true); break;
        case 258: TSR_DEC(64, true, false); break;
        case 259: TSR_DEC(64, true, true); break;
        case 512: TSR_DEC(128, false, false); break;
        case 513: TSR_DEC(128, false, true); break;
        case 514: TSR_DEC(128, true, false); break;
        case 515: TSR_DEC(128, true, true); break;
        default: return -2;
    }
#undef TSR_DEC
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// The XCD of each of the first 64 workgroups of a launch (the context's check of the dispatcher's
// round-robin over the XCDs).
__global__ void k_xcd_probe(uint32_t * out) {
    if (threadIdx.x == 0u) out[blockIdx.x] = tsr::xcc_id();
}
int tsr_launch_xcd_probe(uint32_t * out64, hipStream_t s) {
    hipLaunchKernelGGL(k_xcd_probe, dim3(64), dim3(64), 0, s, out64);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
