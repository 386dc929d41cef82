// kernels.hpp -- argument blocks and launchers of the gfx950 kernels (host and device side).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsr {

struct QactArgs {
    const float * x;
    uint64_t x_stride;       // floats between token rows
    uint8_t * qa;
    uint32_t qa_bytes;       // bytes between QA images
    uint32_t K, kind;
    uint32_t d_off, bs_off;  // byte offsets of the D and BS regions
};

// EXPK constants (VU 6.3): LK = round(log2(e) 2^38), c_k = round(ln(2)^k / k! 2^32),
// t64[j] = round(2^(j/64) 2^30); computed on the host from their definitions.
constexpr uint32_t kAmRows = 8, kAmParts = 32;   // ARGMAX two-pass form: rows, slices per row
struct ExpkTab {
    uint32_t t64[64];
    uint64_t lk, c1, c2, c3;
};

// What the matvec applies to x in front of its activation quantization (MvArgs::prep).
enum MvPrep : uint32_t {
    kPrepNone = 0,           // x as given
    kPrepNorm = 1,           // RMS_NORM of the token row, times pw when pw != 0 (k_rms_norm's rule)
};

// What tsr_hip_mul_mat_epi applies to y after the addend / ACC (the MVM record's local scale).
enum MmEpi : uint32_t {
    kEpiNone = 0,
    kEpiScale = 1,           // y = FM(y, sc)
    kEpiSoftcap = 2,         // y = FM(TANH(FM(y, fs)), sc)
};

// MUL_MAT over the device weight layout of wlayout.hpp (row blocks of rb rows at w).
struct MvArgs {
    const uint8_t * w;
    const float * x;
    uint64_t x_stride;
    float * y;
    uint64_t y_stride;
    const float * add;       // nullable
    uint64_t add_stride;
    int32_t * isums;         // nullable: per-block integer sums of token 0 (checking)
    uint32_t N, K, T;
    uint32_t acc;            // y = FA(y_old, v)
    uint32_t rb;             // rows per row block = per workgroup (the weight's)
    uint32_t prep;           // MvPrep
    const float * pw;        // kPrepNorm: the MUL weight [K] (nullable)
    float eps, inv_n;        // kPrepNorm
    uint32_t glu;            // rows 2j, 2j + 1 are gate / up of output j: y[j] = SWIGLU(gate, up), N / 2 outputs
    ExpkTab ex;              // glu
};

// Prefill MUL_MAT (T >= 16) on the matrix cores: the activations are first quantized (k_qact_mm)
// into block-major quants at qa ([K/32][T][32 B]) and f32 scales at qa + d_off ([K/32][T]).
struct MmArgs {
    const uint8_t * w;       // weight layout of wlayout.hpp, row blocks of rb rows
    const uint8_t * qa;
    uint32_t qa_stride, d_off;
    float * y;
    uint64_t y_stride;
    const float * add;       // nullable
    uint64_t add_stride;
    uint32_t N, K, T;
    uint32_t acc;
    uint32_t rb;
    // Q4_K (k_qact_mm4's A256 form): sub-block sums int32 [K/32][T] at qa + s_off, the super-block
    // scales f32 [K/256][tp] at qa + d_off (tp: T rounded up to 32, padding tokens d = 0)
    uint32_t s_off, tp;
    uint32_t glu;            // Q4_K: rows 2j, 2j + 1 are gate / up of output j: y[j] = SWIGLU(gate, up)
    ExpkTab ex;              // glu
    uint32_t grouped;        // set by the launch: the grid's tile order (k_matmul.hip: mm_tile)
};

// A KV plane (see k_kv.hip for the layout).
struct KvArgs {
    uint8_t * base;          // meta region at 0
    size_t quant_off;        // byte offset of the quant region
    uint32_t E, kv_size;
};

// One chunk of one query token (the planner's output), in execution order per token.
struct FaItem {
    uint32_t t;              // token
    uint32_t u0, n;          // groups [u0, u0 + n)
    uint32_t c_lo, c_hi;     // visible chunk-relative cells (FAST)
    uint32_t general;        // GENERAL chunk: all cells, f32 mask added
    uint32_t s_off;          // first score cell of the item in S (scores at S + s_off * n_head)
    uint32_t tile0, ntiles;  // its 256-cell score tiles (rows tile0 .. tile0 + ntiles - 1 of Mpart)
};
// The work list of one call. Small lists (decode) travel inline in the kernel arguments; larger ones
// are copied to device memory once per call and the kernels read them there (FaArgs::items != 0).
constexpr uint32_t kFaInlItems = 48, kFaInlTok = 8;
struct FaPlan {
    uint32_t n_items, maxtiles;                        // items; tiles of the largest item
    uint32_t tok_first[kFaInlTok], tok_count[kFaInlTok];
    FaItem items[kFaInlItems];
};
struct FaArgs {
    const float * q;         // query rows [T][n_head][D] f32, token t at q + t * q_stride
    uint64_t q_stride;
    KvArgs kc, vc;
    uint32_t D, G, n_head, n_head_kv, E;
    float scale;
    const float * mask;      // GENERAL: f32 mask rows of mstride floats
    uint32_t mstride;
    const FaItem * items;    // device copy of a large work list, else 0 (inline FaPlan)
    const uint32_t * tok_first;
    const uint32_t * tok_count;
    float * S;               // scores
    float * Mpart;           // [tile][n_head] tile maxima
    float * OP;              // [item][4][n_head][D] channel partials
    float * LP;              // [item][4][n_head] channel row sums
    uint32_t max_groups;     // the largest item (groups), for a work list in device memory
    float * out;
    uint64_t out_stride;
    ExpkTab ex;
    // ROPE + SET_ROWS_KV fused into the score kernel (T == 1): q is then the token's unrotated Q|K|V
    // row (k at q + n_head D, v at q + n_head D + E), rotated by position *pos; the new k and v rows
    // go to cell *cell (a cell outside the caches stores nothing and sets *bad)
    const int32_t * pos;
    const int64_t * cell;
    int32_t * bad;
    uint32_t n_dims, neox;
    float ts, m;
    const float * rtab;      // or the angles of *pos from tsr_hip_rope_table: [n_dims / 2] (M cos, M sin)
};

// The one-launch decode FLASH_ATTN_EXT (k_fa_dec.hip): one query row over a plan's device work list,
// one workgroup per ATTPV segment (64 cells of one channel of one chunk, one KV head).
struct FaDecArgs {
    // The fields that the first loads of every workgroup need, contiguous at the start: they are
    // fetched as one block of kernel arguments instead of one scalar round trip per scattered field.
    const float * q;         // the query row [n_head][D]; with ROPE the token's unrotated Q|K|V row
    const FaItem * items;    // the plan's work list (n_items items, chunk order)
    uint32_t * ep;           // [n_head_kv][reducer] epochs (zero at creation); a launch's tag is epoch + 1
    // ROPE + SET_ROWS_KV folded in (cell != 0): position *pos or the angle table rtab, new cell *cell
    const int32_t * pos;
    const int64_t * cell;
    const float * rtab;
    uint32_t G, n_head, E, n_dims, neox, n_items, maxtiles, n_head_kv;
    KvArgs kc, vc;
    uint32_t D;
    float scale;
    const float * mask;      // GENERAL: the f32 mask row (mstride floats)
    uint32_t mstride;
    // results as (f32 bits | tag << 32): segment results [tile][4][n_head][D], segment row sums
    // [tile][4][n_head], chunk maxima [item][n_head]
    uint64_t * seg_o;
    uint64_t * seg_l;
    uint64_t * m_item;
    uint32_t * keys;         // [n_head_kv][n_items][maxtiles][4] 32-byte slots: (MAXT key, tag) of 4 heads
    uint32_t spin_max;       // polls of a wait before it gives up (*bad |= 2)
    uint32_t n_xcd;          // XCDs of the device (workgroups go to them round-robin); 0: unknown
    uint32_t red_first;      // reducers dispatched ahead of the segments (the grid is resident at once)
    float * out;             // [n_head][D]
    int32_t * bad;
    float ts, m;
    ExpkTab ex;
    // The token's Q|K|V row computed in the same launch (qkv_w != 0; ROPE, one XCD per KV head): nq
    // workgroups per KV head, first in dispatch order, each compute 24 of the KV head's rows (its q
    // heads, then its k and v heads) of MUL_MAT(W, RMS_NORM(x) * pw) into qkv_y (== q) and raise a
    // flag with the launch's tag; the segments read q after every flag of their KV head is up
    const uint8_t * qkv_w;   // Q4_K weight layout (wlayout.hpp): qkv_N = (n_head + 2 n_head_kv) D rows of qkv_K
    const float * qkv_x;     // the token's row [qkv_K]
    const float * qkv_pw;    // the norm's MUL weight [qkv_K] (nullable)
    float * qkv_y;
    uint32_t * qkv_flag;     // [n_head_kv][64] (tag | XCD << 28) words
    uint32_t qkv_N, qkv_K, qkv_rb, nq;
    float qkv_eps, qkv_inv_n;
};

// ROPE over T tokens of n_heads heads (head h of token t at x + t * x_stride + h * head_dim).
struct RopeArgs {
    const float * x;
    uint64_t x_stride;
    float * y;
    uint64_t y_stride;
    const int32_t * pos;     // [T] positions
    const float * ff;        // nullable: [n_dims / 2] freq factors
    uint32_t head_dim, n_heads, n_dims, neox;
    float ts, m, freq_scale; // TS = powf(freq_base, -2 / n_dims); M = attn_factor
    uint32_t fs;             // freq_scale != 1
};

// ROPE of the q and k heads of a fused Q|K|V row, then SET_ROWS_KV of the rotated k and of v
// (one workgroup per token). Token t's row is at qkv + t * stride: n_head q heads, n_head_kv k
// heads, n_head_kv v heads of head_dim values; q and k are rotated in place.
struct RopeKvArgs {
    float * qkv;
    uint64_t stride;
    const int32_t * pos;     // [T] positions
    const int64_t * cell;    // [T] cache cells
    int32_t * bad;           // nullable: set when a cell is outside the caches
    KvArgs kc, vc;
    uint32_t head_dim, n_head, n_head_kv, n_dims, neox;
    float ts, m;             // TS = powf(freq_base, -2 / n_dims); M = attn_factor
};

}  // namespace tsr

int tsr_launch_qact(const tsr::QactArgs & a, uint32_t T, hipStream_t s);
// Rows per row block of a weight uploaded for a device with n_cu compute units (fmt: TSR_HIP_FMT_*).
uint32_t tsr_wl_rows_per_block(uint32_t fmt, uint32_t N, uint32_t K, uint32_t n_cu);
int tsr_launch_mv_q8_0(const tsr::MvArgs & a, hipStream_t s);
int tsr_launch_mv_q4_k(const tsr::MvArgs & a, hipStream_t s);
int tsr_launch_qact_mm(const float * x, uint64_t x_stride, uint32_t K, uint32_t T, uint8_t * xq, float * xd,
                       hipStream_t s);
int tsr_launch_mm_q8_0(const tsr::MmArgs & a, hipStream_t s);
int tsr_launch_qact_mm4(const float * x, uint64_t x_stride, uint32_t K, uint32_t T, uint32_t tp, uint8_t * xq,
                        int32_t * xs, float * xd, hipStream_t s);
int tsr_launch_mm_q4_k(const tsr::MmArgs & a, hipStream_t s);
int tsr_launch_kv_bytes(const tsr::KvArgs & a, uint32_t which, uint64_t off, uint64_t n, uint8_t * stage, int to_dev,
                        hipStream_t s);
int tsr_launch_kv_set_rows(const tsr::KvArgs & a, uint32_t which, const float * src, uint32_t n_rows,
                           uint64_t src_stride, const int64_t * idx, int32_t * bad, hipStream_t s);
int tsr_launch_fa(const tsr::FaArgs & a, const tsr::FaPlan & p, uint32_t T, uint32_t n_cu, hipStream_t s);
int tsr_launch_fa_dec(const tsr::FaDecArgs & a, hipStream_t s);
int tsr_launch_xcd_probe(uint32_t * out64, hipStream_t s);
int tsr_launch_rms_norm(const float * x, uint64_t x_stride, uint32_t n, uint32_t rows, float eps, float inv_n,
                        const float * w, uint64_t w_stride, uint32_t w_period, float * y, uint64_t y_stride, hipStream_t s);
int tsr_launch_rope(const tsr::RopeArgs & a, uint32_t T, hipStream_t s);
int tsr_launch_rope_table(const int32_t * pos, uint32_t half, float ts, float m, float * tab, hipStream_t s);
int tsr_launch_mm_epilogue(float * y, uint64_t y_stride, uint32_t N, uint32_t T, uint32_t mode, float fs, float sc,
                           const tsr::ExpkTab & ex, hipStream_t s);
int tsr_launch_swiglu(const float * g, uint64_t g_stride, const float * u, uint64_t u_stride, float * y, uint64_t y_stride,
                      uint32_t n, uint32_t rows, const tsr::ExpkTab & ex, hipStream_t s);
int tsr_launch_add(const float * a, uint64_t a_stride, const float * b, uint64_t b_stride, uint32_t b_period, float * y,
                   uint64_t y_stride, uint32_t n, uint32_t rows, hipStream_t s);
int tsr_launch_get_rows(const float * src, uint64_t src_stride, uint32_t n, uint32_t n_src, const int32_t * ids,
                        uint32_t count, float * dst, uint64_t dst_stride, int32_t * bad, hipStream_t s);
// part: the two-pass form's slice results (kAmRows x kAmParts words; null: one pass)
int tsr_launch_argmax(const float * x, uint64_t x_stride, uint32_t n, uint32_t rows, int32_t * out, uint64_t * part,
                      hipStream_t s);
int tsr_launch_rope_kv(const tsr::RopeKvArgs & a, uint32_t T, hipStream_t s);
// LDS bytes the fused x preparation adds to a matvec launch (0 when none)
size_t tsr_mv_prep_lds(uint32_t prep, uint32_t K);
