/* oc.h -- CPU restatement ("oracle") of the Tesseract quantized-inference numerics.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libtsr_hip, its host adapter, bench.py's GPU
 * path) may link, load or call this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the CPU baseline.
 *
 * What it restates (reference file:line it follows):
 *   spec f32 rules (DAZ inputs, RNE, FTZ of a subnormal rounded result,
 *   canonical NaN 0x7FC00000)                        sw/sim/tsr_ref.c:54-104, docs/spec.md:1405-1418
 *   int32 -> f32, fp16 <-> f32                         sw/sim/tsr_ref.c:107-198
 *   QACT A32 / A256 and the QA image layout           sw/sim/tsr_ref.c:418-520, docs/spec.md:402-425
 *   Q8_0 / Q4_K block terms, 16-partial row tree      sw/sim/tsr_ref.c:525-635, docs/spec.md:438-477
 *   MUL_MAT per token (QACT -> MVM -> optional ACC)   sw/ctrl/ref/mulmat_ref.cpp:43-63
 *   EXPK (the device EXP)                             sw/sim/tsr_ref_math.c:53-159
 *   ATTQK / ASMAX / ATTPV block float / AMERGE /
 *   ANORM / MAXT / CTREE                              sw/sim/tsr_ref_at.c:286-641
 *   MSUM mask summary and the f32 mask copy           sw/sim/tsr_ref_at.c:646-715
 *   chunk planner for one-row tiles (T_MAX = 1)       sw/sim/include/tsr_fa_plan.h:16-42, :130-156, :259-482
 *   composite flash attention                         sw/sim/tsr_ref_at.c:774-860
 *   SET_ROWS into a q8_0 KV row                       sw/ctrl/ref/kv_ref.cpp:20-45, sw/sim/tsr_ref_at.c:244-264
 *
 * The attention restatement works on llama.cpp's q8_0 cache image (row j = cell j, E/32 blocks of
 * {fp16 d, int8 qs[32]}) rather than on the NPU's channel planes: the planes are a byte permutation
 * of that image (sw/sim/tsr_ref_at.c:105-212), and the numerics depend only on which cells and
 * channels a term belongs to, which this file derives from the cell index (group u = cell / 16,
 * channel = u mod C).
 *
 * Fixed oracle configuration for the attention numerics: C = 4 channels, PCAP = 9344, T_MAX = 1
 * (sw/sim/include/tsr_isa.h:64-67, tsr_tables.h:98). Every query token is its own tile.
 *
 * Build: gcc -std=c11 -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile). */
#ifndef OC_H
#define OC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OC_FMT_Q8_0 = 0, OC_FMT_Q4_K = 1 };
enum { OC_QA_A32 = 0, OC_QA_A256 = 1 };

#define OC_NAN_BITS 0x7FC00000u

/* ---- spec f32 arithmetic ---------------------------------------------------------------- */
float    oc_fadd(float a, float b);
float    oc_fsub(float a, float b);
float    oc_fmul(float a, float b);
float    oc_fdiv(float a, float b);
float    oc_frecip(float a);
float    oc_fsqrt(float a);
float    oc_i2f(int32_t v);
float    oc_h2f(uint16_t h);
uint16_t oc_f2h(float f);
int32_t  oc_round_away8(float x);
int32_t  oc_round_even8(float x);
float    oc_tree16(const float p[16]);

/* ---- QA image --------------------------------------------------------------------------- */
uint32_t oc_qa_bytes(uint32_t kind, uint32_t K);           /* QA_LINES(kind, K) * 64 */
uint32_t oc_qa_d_off(uint32_t kind, uint32_t K);           /* byte offset of the D region */
uint32_t oc_qa_bs_off(uint32_t kind, uint32_t K);          /* byte offset of the BS region (A256) */
void     oc_qact(uint32_t kind, const float * x, uint32_t K, uint8_t * qa);

/* ---- MVM on ggml-layout blocks ---------------------------------------------------------- */
/* row: K/32 block_q8_0 (34 B) or K/256 block_q4_K (144 B); qa: image of oc_qact. */
float oc_dot_row(uint32_t fmt, const uint8_t * row, uint32_t K, const uint8_t * qa);
/* Integer block sums of one row (the MVM's exact part). Q8_0: isum per 32-block (K/32 values);
 * Q4_K: isum and msum per super-block interleaved (2 * K/256 values). */
void  oc_row_isums(uint32_t fmt, const uint8_t * row, uint32_t K, const uint8_t * qa, int32_t * out);
/* MUL_MAT: y[t][n] = (add ? FA(add[t][n], dot) : dot) for T tokens, x rows at x_stride floats,
 * y / add rows at y_stride / add_stride floats (add_stride 0: row 0 for every token). */
void  oc_mul_mat(uint32_t fmt, const uint8_t * w, uint32_t N, uint32_t K, const float * x, uint32_t T,
                 uint64_t x_stride, const float * add, uint64_t add_stride, float * y, uint64_t y_stride,
                 uint32_t threads);

/* ---- attention --------------------------------------------------------------------------- */
#define OC_C          4u
#define OC_PCAP       9344u
#define OC_M_FLOOR    0xF1800000u
#define OC_L_FLOOR    0x00800000u
#define OC_MSUM_MAGIC 0x4D55534Du

float   oc_expk(float v);                      /* EXPK(v, P1) */
float   oc_maxt(float a, float b);
float   oc_ctree(const float * x, uint32_t n);
int32_t oc_bf_int(float w, int32_t es);
float   oc_bf_f(int64_t A, int32_t k);

/* MSUM words (8-word header + 4 words per query row) of an f16 mask [n_q][row_stride]. */
uint32_t oc_msum_build(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, uint32_t * words);
/* The f32 copy a GENERAL chunk adds: rows of 16*ceil(n_kv/16) words, fdiv(mask, scale), -inf pad. */
void oc_mask_f32(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, float scale, float * dst);

typedef struct oc_chunk {
    uint32_t u0, n_groups, c_lo, c_hi, general;
} oc_chunk;
/* Chunk list of one query row (T_MAX = 1). words: an MSUM image; q: the row. Returns the count
 * (written up to cap), or < 0 for a malformed row / a shape without chunks. */
long oc_fa_plan_row(uint32_t E, uint32_t D, const uint32_t * words, uint32_t q,
                    const uint32_t (*new_runs)[2], uint32_t n_new, oc_chunk * out, size_t cap);

/* SET_ROWS of one f32 row x[E] into a q8_0 cache row (E/32 blocks of 34 bytes). */
void oc_kv_store_row(const float * x, uint32_t E, uint8_t * row);

/* Composite flash attention over q8_0 K / V caches [kv_size][E/32 blocks], E = n_head_kv * D.
 * q: [T][n_head][D] f32 at q_stride floats per token; out: [T][n_head][D] at out_stride.
 * mask_f32: the GENERAL copy (NULL if the MSUM is FAST). Returns 0, or a negative code. */
int oc_flash_attn(const float * q, uint32_t T, uint64_t q_stride, const uint8_t * kc, const uint8_t * vc,
                  uint32_t kv_size, uint32_t D, uint32_t n_head, uint32_t n_head_kv, float scale,
                  const uint32_t * msum, const float * mask_f32, const uint32_t (*new_runs)[2], uint32_t n_new,
                  float * out, uint64_t out_stride);

#ifdef __cplusplus
}
#endif
/* ---- decode-layer glue ops (oc_glue.c) ------------------------------------------------------ */
float oc_rms_scale(const float * x, uint32_t n, float eps, float inv_n);
void  oc_rms_norm_rows(uint32_t n, uint32_t rows, const float * x, uint64_t x_stride, float eps, float inv_n,
                       const float * w, uint64_t w_stride, uint32_t w_period, float * y, uint64_t y_stride);
void  oc_sincos(float t, float * s_out, float * c_out);
void  oc_rope(uint32_t neox, uint32_t head_dim, uint32_t n_dims, uint32_t n_heads, uint32_t T,
              const float * x, uint64_t x_stride, float * y, uint64_t y_stride, const int32_t * pos,
              float ts, float m, float freq_scale, const float * ff);
float oc_silu(float x);
float oc_tanh(float x);
void  oc_mm_epilogue(float * y, uint64_t n, uint32_t mode, float fs, float sc);
void  oc_swiglu_rows(uint32_t n, uint32_t rows, const float * g, uint64_t g_stride, const float * u, uint64_t u_stride,
                     float * y, uint64_t y_stride);
void  oc_add_rows(uint32_t n, uint32_t rows, const float * a, uint64_t a_stride, const float * b, uint64_t b_stride,
                  float * y, uint64_t y_stride);
void  oc_get_rows(uint32_t n, const float * src, uint64_t src_stride, const int32_t * ids, uint32_t count, float * dst,
                  uint64_t dst_stride);
void  oc_argmax_rows(uint32_t n, uint32_t rows, const float * x, uint64_t x_stride, int32_t * out);

#endif
