/* tsr_hip.h -- C ABI of libtsr_hip, the MI355X (gfx950) implementation of Tesseract's quantized
 * inference hot path: on-the-fly activation quantization (QACT A32 / A256), Q8_0 and Q4_K
 * MUL_MAT, the q8_0 KV cache (SET_ROWS, byte get / set) and flash attention over it.
 *
 * The library sits where the reference's ggml backend hands work to its device: the backend's
 * buffer, tensor and graph-compute callbacks (sw/ggml-tesseract/ggml-tesseract.cpp) and the
 * transport below them (sw/transport/tsr_transport.h:61-134). Each entry point below names the
 * reference interface it replaces. Results are the reference simulator's bits (sw/sim/tsr_ref*.c):
 * integer block sums and quantized activations bit-exact, f32 outputs bit-exact (the contract
 * allows 1e-5 relative), attention bit-exact (the contract allows 2e-3 absolute).
 *
 * Conventions
 *   - Every function returns 0 or a negative TSR_HIP_E_* code; tsr_hip_strerror names it.
 *   - Pointers named *_dev are device addresses (from tsr_hip_alloc or any HIP allocation on the
 *     context's device); every other pointer is host memory.
 *   - `stream` is a hipStream_t of the context's device, or NULL for the context's own stream.
 *     Kernel entry points are asynchronous on that stream; tsr_hip_sync waits.
 *   - A context is thread-safe: calls on one context are serialized by its mutex (the reference
 *     backend's device mutex, ggml-tesseract.cpp:3932).
 *   - Strides are in elements (floats) unless named *_bytes.
 */
#ifndef TSR_HIP_H
#define TSR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes (the transport's TSR_TE_* role, sw/transport/tsr_transport.h:266-276) ---- */
#define TSR_HIP_OK          0
#define TSR_HIP_E_ARG      -1   /* a NULL or malformed argument */
#define TSR_HIP_E_SHAPE    -2   /* a shape the op does not support (K % block, D, GQA ratio, ...) */
#define TSR_HIP_E_NOMEM    -3   /* device or host allocation failed */
#define TSR_HIP_E_HIP      -4   /* a HIP runtime call failed */
#define TSR_HIP_E_RANGE    -5   /* a byte range or cell index beyond the object */
#define TSR_HIP_E_NODEV    -6   /* no such device */
#define TSR_HIP_E_FMT      -7   /* unknown weight format / QA kind */
#define TSR_HIP_E_MASK     -8   /* the mask summary needs the f32 mask copy, or is malformed */

/* weight formats (ISA MVM sub field, sw/sim/include/tsr_tables.h:103-104) */
#define TSR_HIP_FMT_Q8_0    0u
#define TSR_HIP_FMT_Q4_K    1u
/* QA kinds (QACT sub field, sw/sim/include/tsr_tables.h:105-106) */
#define TSR_HIP_QA_A32      0u
#define TSR_HIP_QA_A256     1u
/* KV planes (KVST sub field, sw/sim/include/tsr_ref_at.h:56-57) */
#define TSR_HIP_KV_K        0u
#define TSR_HIP_KV_V        1u
/* tsr_hip_mul_mat flags (the MUL_MAT record's FLAGS word, sw/ctrl/ref/mulmat_ref.hpp:14-16) */
#define TSR_HIP_MM_ACC_DST  0x1u  /* y = FA(y_old, W.x) */
/* The weight's rows 2j and 2j + 1 are the gate and up rows of output j, and y[j] = SWIGLU(gate . x,
 * up . x) for j < N / 2 -- the MUL_MATs of the FFN gate and up weights followed by GGML_GLU_OP_SWIGLU
 * (tsr_hip_swiglu), bit-identical, in one launch. No addend, no ACC_DST; Q4_K at any T (matvec, or the
 * matrix-core path at T >= 16), Q8_0 at T < 16 (not its matrix-core prefill shapes); N even. */
#define TSR_HIP_MM_GLU      0x2u
/* tsr_hip_mul_mat_epi: the MVM record's local scale applied to y after the addend / ACC
 * (TSR_MVM_LOCAL_SCALE / _SOFTCAP, sw/sim/tsr_sim.c:1648-1667; GGML MUL_MAT followed by SCALE, or the
 * logit softcap tanh(y fs) sc): SCALE y = FM(y, scale); SOFTCAP y = FM(TANH(FM(y, first_scale)), scale)
 * with the VU's TANH (sw/sim/tsr_ref_math.c:182-199). Not with TSR_HIP_MM_GLU; not both. */
#define TSR_HIP_MM_SCALE    0x4u
#define TSR_HIP_MM_SOFTCAP  0x8u

typedef struct tsr_hip_ctx tsr_hip_ctx;
typedef struct tsr_hip_weight tsr_hip_weight;
typedef struct tsr_hip_kv tsr_hip_kv;

/* ---- device and context ---------------------------------------------------------------------
 * Replaces the backend's device open (tsr_dev_open_locked, ggml-tesseract.cpp:463) and
 * tsr_transport_open / _close (tsr_transport.h:61-72). One context per (process, device); it owns a
 * default-priority hipStream and its scratch memory. */
int         tsr_hip_open(int device, tsr_hip_ctx ** out);
int         tsr_hip_close(tsr_hip_ctx * ctx);
const char * tsr_hip_strerror(int code);
/* The context's stream (a hipStream_t) for callers that order their own work against it. */
void *      tsr_hip_stream(tsr_hip_ctx * ctx);
/* Wait for all work on `stream` (NULL: the context's stream). Replaces tsr_transport_wait
 * (tsr_transport.h:112-116). */
int         tsr_hip_sync(tsr_hip_ctx * ctx, void * stream);
/* Number of compute units and the device name (get_props / get_memory, ggml-tesseract.cpp:4312-4328). */
int         tsr_hip_device_info(tsr_hip_ctx * ctx, int * n_cu, char * name, size_t name_len,
                                size_t * mem_free, size_t * mem_total);

/* ---- raw device buffers (ggml buffer alloc / set_tensor / get_tensor / memset_tensor / free for
 * non-weight tensors, ggml-tesseract.cpp:1905-2042; tsr_transport_write / _read, tsr_transport.h:80-98) */
int tsr_hip_alloc(tsr_hip_ctx * ctx, size_t bytes, void ** dev_out);
int tsr_hip_free(tsr_hip_ctx * ctx, void * dev);
int tsr_hip_write(tsr_hip_ctx * ctx, void * dst_dev, const void * src, size_t bytes);
int tsr_hip_read(tsr_hip_ctx * ctx, void * dst, const void * src_dev, size_t bytes);
/* A host-to-device copy ordered on `stream` that does not wait: the bytes are taken at the call (src
 * may be reused at once) into pinned staging, from which the device copy reads. bytes <= 16384. Not
 * under graph capture. (The backend's set_tensor for small per-token inputs, positions and ids,
 * ggml-tesseract.cpp:1905-1945, without a device wait.) */
int tsr_hip_write_async(tsr_hip_ctx * ctx, void * dst_dev, const void * src, size_t bytes, void * stream);
/* A device-to-device copy ordered on `stream` (the backend's cpy_tensor between its own buffers,
 * ggml-tesseract.cpp:2026-2042). */
int tsr_hip_copy_async(tsr_hip_ctx * ctx, void * dst_dev, const void * src_dev, size_t bytes, void * stream);
int tsr_hip_memset(tsr_hip_ctx * ctx, void * dst_dev, int value, size_t bytes);

/* ---- weights ---------------------------------------------------------------------------------
 * Upload an N x K weight given as ggml blocks (row n = K/32 block_q8_0 or K/256 block_q4_K,
 * consecutive) and convert it to the device layout: per-row scale ("meta") bytes split from the
 * quant bytes, both row-contiguous. Replaces the weight path of set_tensor: tsr_buffer_set_tensor
 * -> tsr_store_weight_rows -> tsr_repack_row (ggml-tesseract.cpp:852-878, 1905-1945;
 * sw/sim/tsr_ref.c:296-316). K must be a positive multiple of the block size and <= 32768
 * (K_MAX, sw/sim/include/tsr_isa.h:64-67); N >= 1. */
int tsr_hip_weight_upload(tsr_hip_ctx * ctx, uint32_t fmt, const void * ggml_blocks, uint32_t N, uint32_t K,
                          tsr_hip_weight ** out);
/* The exact ggml blocks back (get_tensor of a weight; tsr_unrepack_row, sw/sim/tsr_ref.c:318-333). */
int tsr_hip_weight_read(tsr_hip_ctx * ctx, const tsr_hip_weight * w, void * ggml_blocks);
int tsr_hip_weight_free(tsr_hip_ctx * ctx, tsr_hip_weight * w);
/* Format, N, K and the device bytes a weight occupies. */
int tsr_hip_weight_info(const tsr_hip_weight * w, uint32_t * fmt, uint32_t * N, uint32_t * K, size_t * dev_bytes);

/* ---- QACT --------------------------------------------------------------------------------------
 * T token rows x_dev[t * x_stride + k] (f32, k < K) -> T QA images in the spec layout
 * (QS int8[K] | D f32[K/bs] | BS int16[K/16] for A256, each region padded to 64 bytes, tails zero;
 * docs/spec.md:402-425) at qa_dev + t * tsr_hip_qa_bytes(kind, K). The QACT tile op
 * (sw/sim/tsr_sim.c:1507-1522, tsr_qact sw/sim/tsr_ref.c:456). MUL_MAT and FLASH_ATTN quantize
 * their activations themselves; this entry point exposes the quantizer for checking and for
 * callers that keep QA images. */
size_t tsr_hip_qa_bytes(uint32_t kind, uint32_t K);
int tsr_hip_qact(tsr_hip_ctx * ctx, uint32_t kind, const float * x_dev, uint32_t K, uint32_t T, uint64_t x_stride,
                 uint8_t * qa_dev, void * stream);

/* ---- MUL_MAT -------------------------------------------------------------------------------------
 * GGML_OP_MUL_MAT with a Q8_0 / Q4_K weight and f32 activations (the MUL_MAT kind record,
 * sw/ctrl/include/tsr/opl.hpp:214-218; lowered by tsr_lower_mul_mat, ggml-tesseract.cpp:2790-2928;
 * executed as QACT -> MVM per token, sw/ctrl/ref/mulmat_ref.cpp:43-105):
 *   y_dev[t * y_stride + n] = v                      v = tree16 row dot of W row n and QACT(x_t)
 *                           = FA(add_dev[t * add_stride + n], v)   with an addend (add_stride 0: row 0)
 *                           = FA(y_old, v)                          with TSR_HIP_MM_ACC_DST
 * for t < T, n < N. An addend together with ACC_DST is refused (TSR_HIP_E_ARG), as the kernel's record
 * check does. x, y and add must not overlap. T >= 1. T < 16 runs the matvec kernels; T >= 16 the int8
 * matrix cores (both formats; the activations are quantized into the context's scratch first), with
 * the same bits. */
int tsr_hip_mul_mat(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T, uint64_t x_stride,
                    float * y_dev, uint64_t y_stride, const float * add_dev, uint64_t add_stride, uint32_t flags,
                    void * stream);
/* MUL_MAT of RMS_NORM(x) * norm_w in one launch, bit-identical to tsr_hip_rms_norm over n = K with
 * norm_w_dev (nullable: no MUL) and w_period 1 followed by tsr_hip_mul_mat on its output (the fused
 * RMS_NORM + MUL record, sw/ggml-tesseract/ggml-tesseract.cpp:33, 426, feeding the Q|K|V and FFN
 * MUL_MATs of the decoder layer, sw/ctrl/tests/test_fw_m7_layer.cpp:646-686). The reference runs the
 * norm as its own record before the MUL_MAT; here it runs inside the matvec's activation
 * quantization. Flags, addend as tsr_hip_mul_mat (TSR_HIP_MM_GLU included). K <= 8192 and not the
 * Q8_0 T >= 16 prefill shapes, else TSR_HIP_E_SHAPE: run the two ops separately. */
int tsr_hip_mul_mat_norm(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T,
                         uint64_t x_stride, float eps, const float * norm_w_dev, float * y_dev, uint64_t y_stride,
                         const float * add_dev, uint64_t add_stride, uint32_t flags, void * stream);
/* tsr_hip_mul_mat with the SCALE / SOFTCAP epilogue of its flags (TSR_HIP_MM_SCALE, TSR_HIP_MM_SOFTCAP,
 * the words 6 and 7 of the MVM record: first_scale, scale). Every MUL_MAT shape, the prefill path too. */
int tsr_hip_mul_mat_epi(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, uint32_t T, uint64_t x_stride,
                        float * y_dev, uint64_t y_stride, const float * add_dev, uint64_t add_stride, uint32_t flags,
                        float first_scale, float scale, void * stream);
/* The exact integer part of MUL_MAT for checking: for token 0, the per-block sums of every row
 * (Q8_0: isum per 32-block, N x K/32; Q4_K: isum and msum per super-block interleaved,
 * N x 2K/256) as the MVM computes them (term_q8_0 / term_q4_K, sw/sim/tsr_ref.c:525-567). */
int tsr_hip_mul_mat_isums(tsr_hip_ctx * ctx, const tsr_hip_weight * w, const float * x_dev, int32_t * isums_dev,
                          void * stream);

/* ---- KV cache ----------------------------------------------------------------------------------
 * A q8_0 K or V cache of kv_size cells of E = n_head_kv * D values (llama.cpp's cache_k_l<n> /
 * cache_v_l<n> tensors, q8_0; recognized by the backend in tsr-kvbuf.h:61-63). The device layout is
 * the library's own; get / set bytes convert to and from the ggml q8_0 image exactly
 * (tsr_kv_set_bytes / tsr_kv_get_bytes, sw/sim/tsr_ref_at.c:178-212). E % 64 == 0. */
int tsr_hip_kv_create(tsr_hip_ctx * ctx, uint32_t E, uint32_t kv_size, tsr_hip_kv ** out);
int tsr_hip_kv_free(tsr_hip_ctx * ctx, tsr_hip_kv * kv);
/* Bytes [off, off + bytes) of the ggml image of plane `which` (row j = cell j, E/32 * 34 bytes). */
int tsr_hip_kv_set_bytes(tsr_hip_ctx * ctx, tsr_hip_kv * kv, uint32_t which, size_t off, const void * src, size_t bytes);
int tsr_hip_kv_get_bytes(tsr_hip_ctx * ctx, const tsr_hip_kv * kv, uint32_t which, size_t off, void * dst, size_t bytes);
/* GGML_OP_SET_ROWS into the cache (the SET_ROWS_KV kind, sw/ctrl/ref/kv_ref.cpp:20-45): rows
 * src_dev[i * src_stride + e] (f32, e < E) are quantized (QACT A32, fp16 scales) into cells
 * idx_dev[i] (int64, device), i < n_rows. Every index must be < kv_size (checked on the device: an
 * out-of-range index stores nothing and sets *bad_dev if bad_dev is not NULL). */
int tsr_hip_kv_set_rows(tsr_hip_ctx * ctx, tsr_hip_kv * kv, uint32_t which, const float * src_dev, uint32_t n_rows,
                        uint64_t src_stride, const int64_t * idx_dev, int32_t * bad_dev, void * stream);

/* The decoder layer's ROPE of q and k followed by SET_ROWS_KV of k and v (the ROPE, SET_ROWS_KV records
 * of sw/ctrl/tests/test_fw_m7_layer.cpp:646-686) in one launch, bit-identical to tsr_hip_rope over the
 * n_head + n_head_kv q and k heads (freq_scale 1, no freq factors) in place, then tsr_hip_kv_set_rows of
 * the rotated k into kc and of v into vc. Token t's row at qkv_dev + t * stride holds n_head q heads,
 * n_head_kv k heads and n_head_kv v heads of head_dim floats (head_dim % 32 == 0; the row at most 16384
 * floats); its position is pos_dev[t] (int32) and its cell cell_dev[t] (int64), both on the device. A
 * cell outside either cache stores nothing and sets *bad_dev (nullable). */
int tsr_hip_rope_kv(tsr_hip_ctx * ctx, float * qkv_dev, uint32_t T, uint64_t stride, uint32_t head_dim, uint32_t n_head,
                    uint32_t n_head_kv, uint32_t n_dims, int mode, const int32_t * pos_dev, float freq_base,
                    float attn_factor, tsr_hip_kv * kc, tsr_hip_kv * vc, const int64_t * cell_dev, int32_t * bad_dev,
                    void * stream);

/* ---- FA plans ------------------------------------------------------------------------------------
 * The work list of FLASH_ATTN_EXT kept in device memory, so that graphs of planned launches replay
 * over masks that change between replays (a decode token per replay): the backend's per-graph plan
 * cache (ggml-tesseract.cpp:3937-3952, 3768-3779) with the FA record's chunk plan refreshed per call.
 *   create   for T query rows of D / n_head / n_head_kv over caches of at most kv_size cells
 *   set      plans the MSUM (and new_runs, as tsr_hip_flash_attn) on the host and copies the list to
 *            the device in stream order (not under capture). *shape_changed = 1 when the list's shape
 *            (items, tiles per item, groups per item, GENERAL, and for one query row whether the
 *            workgroups of tsr_hip_attn_qkv_plan_rope_tab's one launch fit the device at once) differs
 *            from the previous set: launches captured before then must be captured again.
 *            mask_f32 != 0: an f32 mask copy will be given.
 *   flash_attn_plan  FLASH_ATTN_EXT with the plan's current list (capturable; numerics as
 *            tsr_hip_flash_attn). The plan's partials live in the plan: launches that use one plan run
 *            in stream order, one at a time. */
typedef struct tsr_hip_fa_plan tsr_hip_fa_plan;
int tsr_hip_fa_plan_create(tsr_hip_ctx * ctx, uint32_t D, uint32_t n_head, uint32_t n_head_kv, uint32_t T,
                           uint32_t kv_size, tsr_hip_fa_plan ** out);
int tsr_hip_fa_plan_set(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan, const uint32_t * msum, int mask_f32,
                        const uint32_t (*new_runs)[2], uint32_t n_new, int * shape_changed, void * stream);
int tsr_hip_flash_attn_plan(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * q_dev, uint64_t q_stride,
                            const tsr_hip_kv * kc, const tsr_hip_kv * vc, float scale, const float * mask_f32_dev,
                            float * out_dev, uint64_t out_stride, void * stream);
/* The planned FLASH_ATTN_EXT of one decode token with the layer's ROPE and SET_ROWS_KV folded into its
 * score kernel: bit-identical to tsr_hip_rope_kv(qkv_dev, T = 1, head_dim = D, n_head, n_head_kv,
 * n_dims, mode, pos_dev, freq_base, attn_factor, kc, vc, cell_dev, bad_dev) followed by
 * tsr_hip_flash_attn_plan on the rotated q -- the ROPE / SET_ROWS_KV / FLASH_ATTN_EXT records of
 * sw/ctrl/tests/test_fw_m7_layer.cpp:646-686 in one call, one launch fewer. qkv_dev holds the token's
 * unrotated Q|K|V row (n_head q heads, n_head_kv k heads, n_head_kv v heads of D floats); it is read,
 * not rotated in place. The plan's T is 1; D is 64 or 128 with (n_head / n_head_kv + 2) D <= 1024,
 * n_dims % 8 == 0 and n_dims <= min(D, 128); otherwise TSR_HIP_E_SHAPE. */
int tsr_hip_flash_attn_plan_rope(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * qkv_dev,
                                 tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                 const int32_t * pos_dev, float freq_base, float attn_factor, const int64_t * cell_dev,
                                 int32_t * bad_dev, const float * mask_f32_dev, float * out_dev, uint64_t out_stride,
                                 void * stream);
/* The same with the ROPE angles of the token's position read from a table made by tsr_hip_rope_table
 * (pos_dev, n_dims, freq_base, attn_factor of that call) instead of computed per launch: the layers of
 * one token share the table, so the per-layer launch spends no time on the angle recurrence. tab_dev:
 * n_dims floats, 8-byte aligned. Same shapes and results as tsr_hip_flash_attn_plan_rope. */
int tsr_hip_flash_attn_plan_rope_tab(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const float * qkv_dev,
                                     tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                     const float * tab_dev, const int64_t * cell_dev, int32_t * bad_dev,
                                     const float * mask_f32_dev, float * out_dev, uint64_t out_stride, void * stream);
/* The attention half of a decode layer in one call: bit-identical to
 *   tsr_hip_mul_mat_norm(w_qkv, x_dev, T = 1, eps, norm_w_dev -> qkv_dev)
 * followed by tsr_hip_flash_attn_plan_rope_tab(plan, qkv_dev, ...) -- the RMS_NORM + MUL, Q|K|V
 * MUL_MAT, ROPE, SET_ROWS_KV and FLASH_ATTN_EXT records of sw/ctrl/tests/test_fw_m7_layer.cpp:646-686.
 * qkv_dev receives the unrotated Q|K|V row as the MUL_MAT writes it. When the one-launch decode form
 * places each KV head's workgroups on one XCD (n_head_kv a multiple of the device's XCD count), its
 * workgroups with work fit the device at once (4 per compute unit: at the Llama-3-8B shape up to ~5.4 K
 * cells), w_qkv is Q4_K with K <= 4096 and the buffers are 16-byte aligned, it is one launch: workgroups of the launch
 * compute each KV head's Q|K|V rows on that head's XCD while its segments load K. Otherwise the two
 * calls run; so do they when out_dev overlaps x_dev or norm_w_dev (in one launch a KV head's reducers
 * write out_dev while other heads' row workgroups still read x and the norm weights). Whether the form
 * fits is decided per tsr_hip_fa_plan_set: its *shape_changed is 1 when the decision flips, so that a
 * captured launch is captured again. tsr_hip_counters.fa_dec_qkv_launches counts the one-launch calls.
 * w_qkv: N = (n_head + 2 n_head_kv) D rows of K = the x row's length; x_dev and qkv_dev must
 * not overlap. Shapes and errors otherwise as the two calls. (No counterpart in the reference: its
 * records run one after another.) */
int tsr_hip_attn_qkv_plan_rope_tab(tsr_hip_ctx * ctx, const tsr_hip_fa_plan * plan, const tsr_hip_weight * w_qkv,
                                   const float * x_dev, float eps, const float * norm_w_dev, float * qkv_dev,
                                   tsr_hip_kv * kc, tsr_hip_kv * vc, float scale, uint32_t n_dims, int mode,
                                   const float * tab_dev, const int64_t * cell_dev, int32_t * bad_dev,
                                   const float * mask_f32_dev, float * out_dev, uint64_t out_stride, void * stream);
int tsr_hip_fa_plan_free(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan);
/* The one-launch decode form of the planned FLASH_ATTN_EXT (one query row) runs a workgroup per ATTPV
 * segment and exchanges the chunk maxima and the segment results between its workgroups (no
 * counterpart in the reference, whose chunks run in order on one engine). Its waits are bounded: polls
 * of a wait before it gives up and raises *bad_dev |= 2 (the results are then not valid). 0 restores the
 * default (2^20 polls, tens of milliseconds); a small limit forces the expired path (tests of it).
 * When n_head_kv is a multiple of the device's XCD count, all workgroups of a KV head are placed on one
 * XCD (the dispatcher's round-robin) and exchange through its L2; a workgroup found on another XCD
 * raises *bad_dev |= 4 (results not valid). bad_dev is the argument of the _rope entry points. */
int tsr_hip_set_fa_wait_limit(tsr_hip_ctx * ctx, uint32_t polls);
/* Test hook (no counterpart in the reference): sets every KV head's epoch word of the plan's one-launch
 * decode form to `epoch` (stream-ordered on the context's stream, not under capture), so that a test
 * reaches the tag wrap (epoch 2^28 - 1 -> tag 1; a launch's tag is never 0, the value of plan memory no
 * launch has written) without 2^28 launches. */
int tsr_hip_fa_plan_set_epoch(tsr_hip_ctx * ctx, tsr_hip_fa_plan * plan, uint32_t epoch);

/* ---- graphs -------------------------------------------------------------------------------------
 * Every launch the library makes on `stream` between begin and end is recorded (stream capture) and
 * replayed by one launch: one decode token per replay (the backend's one op list per token,
 * sw/ctrl/ref/opl_ref.hpp:1-9). The stream must not be the null stream. Entry points that copy from
 * the host or allocate (tsr_hip_write, _write_async, _fa_plan_set, a first FA or prefill call that
 * grows the scratch) refuse to run under capture. A graph whose captured launches use the context's
 * scratch (tsr_hip_flash_attn, MUL_MAT at T >= 16, tsr_hip_mul_mat_isums) holds its address: once a
 * later call has grown the scratch (and freed the old block), tsr_hip_graph_launch refuses that graph
 * with TSR_HIP_E_ARG; capture it again. Graphs of planned FA launches and matvecs use no scratch. */
typedef struct tsr_hip_graph tsr_hip_graph;
int tsr_hip_graph_begin(tsr_hip_ctx * ctx, void * stream);
int tsr_hip_graph_end(tsr_hip_ctx * ctx, void * stream, tsr_hip_graph ** out);
int tsr_hip_graph_launch(tsr_hip_ctx * ctx, const tsr_hip_graph * graph, void * stream);
int tsr_hip_graph_free(tsr_hip_ctx * ctx, tsr_hip_graph * graph);

/* ---- mask summary (the backend's MSUM producer, tsr_msum_build_f16 sw/sim/tsr_ref_at.c:646-693) --
 * words: 8 + 4 * n_q uint32 (host). Returns the flags word (bit 0 GENERAL) or a negative code. */
int tsr_hip_msum_build_f16(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, uint32_t * words);
/* The f32 mask copy a GENERAL summary needs (tsr_msum_mask_f32, sw/sim/tsr_ref_at.c:704-715): row q of
 * dst (16 ceil(n_kv / 16) floats) holds fdiv(f32(mask[q][j]), scale) under the f32 rule for j < n_kv and
 * -inf after. Host only. scale must be finite, normal and > 0 (else TSR_HIP_E_ARG). */
int tsr_hip_msum_mask_f32(const uint16_t * mask, size_t row_stride, uint32_t n_kv, uint32_t n_q, float scale,
                          float * dst);

/* ---- FLASH_ATTN_EXT ----------------------------------------------------------------------------
 * GGML_OP_FLASH_ATTN_EXT with f32 q and a q8_0 K / V cache (the FLASH_ATTN kind, lowered by
 * tsr_lower_fa sw/ggml-tesseract/tsr-build.cpp:673-773; numerics tsr_ref_fa sw/sim/tsr_ref_at.c:774-860):
 *   q_dev  [T][n_head][D] f32, token t at q_dev + t * q_stride
 *   out_dev[T][n_head][D] f32, token t at out_dev + t * out_stride
 *   msum   the host MSUM words of the op's mask (n_q = T, n_kv cells visible at most)
 *   mask_f32_dev  the f32 mask copy (rows of 16*ceil(n_kv/16) floats, fdiv(mask, scale), -inf pad;
 *          tsr_msum_mask_f32) -- required only when the MSUM is GENERAL, else NULL
 *   new_runs / n_new  cell runs [lo, hi) written in this launch (their chunks are merged last)
 * D in {64, 128, 256, 512}; n_head % n_head_kv == 0; n_head / n_head_kv <= 64; n_head_kv * D == E of
 * both caches; scale finite, normal and > 0. */
int tsr_hip_flash_attn(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride,
                       const tsr_hip_kv * kc, const tsr_hip_kv * vc, uint32_t D, uint32_t n_head, uint32_t n_head_kv,
                       float scale, const uint32_t * msum, const float * mask_f32_dev,
                       const uint32_t (*new_runs)[2], uint32_t n_new, float * out_dev, uint64_t out_stride,
                       void * stream);

/* FLASH_ATTN_EXT exactly as tsr_hip_flash_attn (same arguments, same bits), allocating nothing: no
 * hipMalloc / hipFree / pinned staging / host-to-device copy, no wait on another stream. No counterpart
 * in the reference; it is for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Its partials live in a fixed device array of 16 MiB that each
 * GPU holds from the library's load until the process ends; the work list travels in the kernel
 * arguments. Limits: T <= 8 query rows, at most 48 planned chunks (about 98 K visible cells per row), and
 * partials (scores 4 n_head B per visible cell and row, 2 KiB-per-head chunk partials) within the 16 MiB;
 * beyond them TSR_HIP_E_RANGE, before anything runs. Every call on one GPU shares that GPU's array
 * (from every context): calls that overlap on one GPU (two streams, two threads, two contexts) race. */
int tsr_hip_flash_attn_noalloc(tsr_hip_ctx * ctx, const float * q_dev, uint32_t T, uint64_t q_stride,
                               const tsr_hip_kv * kc, const tsr_hip_kv * vc, uint32_t D, uint32_t n_head,
                               uint32_t n_head_kv, float scale, const uint32_t * msum, const float * mask_f32_dev,
                               const uint32_t (*new_runs)[2], uint32_t n_new, float * out_dev, uint64_t out_stride,
                               void * stream);

/* ---- decode-layer glue ops ----------------------------------------------------------------------
 * The f32 ops around MUL_MAT and FLASH_ATTN in a decoder layer, on the vector unit's f32 rules
 * (every input denormal-as-zero, one IEEE round-to-nearest-even operation, result flushed to zero,
 * NaN canonical 0x7FC00000; sw/sim/tsr_ref_vu.c). Rows of n f32 values; the *_stride arguments are
 * floats between rows. Outputs may alias their first input exactly (in place) but must not overlap
 * any other input. */

/* GGML_OP_RMS_NORM, fused with the GGML_OP_MUL by a weight when w_dev is not NULL (tsr_lower_rms,
 * sw/ggml-tesseract/tsr-build.cpp:357-421; RED.SUMSQ post RMS then VOP.MULCB, sw/sim/tsr_ref_vu.c:
 * 171-263): s = 1 / sqrt(sum(x^2) / n + eps) over 128 partial sums added in a fixed tree,
 * y = (x s) w with weight row r % w_period (w_stride floats apart). n >= 1, rows >= 1. */
int tsr_hip_rms_norm(tsr_hip_ctx * ctx, const float * x_dev, uint32_t n, uint32_t rows, uint64_t x_stride, float eps,
                     const float * w_dev, uint64_t w_stride, uint32_t w_period, float * y_dev, uint64_t y_stride,
                     void * stream);

/* GGML_OP_ROPE modes NORMAL (0), NEOX (2) and IMROPE (40, text positions: rotated as NEOX) without
 * YaRN (tsr_lower_rope, sw/ggml-tesseract/tsr-build.cpp:492-554; tsr_ref_rope sw/sim/tsr_ref_vu.c:
 * 308-376). Token t, head h at x_dev + t * x_stride + h * head_dim; positions pos_dev[t] (int32,
 * device); TS = powf(freq_base, -2 / n_dims) on the host; freq_factors_dev (nullable) holds n_dims/2
 * floats. 2 <= n_dims <= head_dim, n_dims even and <= 1024; dims from n_dims on are copied. */
#define TSR_HIP_ROPE_NORMAL 0
#define TSR_HIP_ROPE_NEOX   2
#define TSR_HIP_ROPE_IMROPE 40
int tsr_hip_rope(tsr_hip_ctx * ctx, const float * x_dev, uint32_t T, uint64_t x_stride, uint32_t head_dim,
                 uint32_t n_heads, uint32_t n_dims, int mode, const int32_t * pos_dev, float freq_base, float freq_scale,
                 float attn_factor, const float * freq_factors_dev, float * y_dev, uint64_t y_stride, void * stream);
/* The ROPE angles of one position (*pos_dev) as tsr_hip_rope computes them without freq factors and
 * with freq_scale 1 (theta_0 = pos, theta_i = theta_(i-1) TS, tsr_ref_rope sw/sim/tsr_ref_vu.c:
 * 308-376): tab_dev[2 i] = FM(attn_factor, cos theta_i), tab_dev[2 i + 1] = FM(attn_factor,
 * sin theta_i) for i < n_dims / 2; n_dims even, 2 <= n_dims <= 128; tab_dev 8-byte aligned. The table
 * of tsr_hip_flash_attn_plan_rope_tab (no counterpart in the reference, which derives the angles in
 * every ROPE record: a decode token's layers share one position). */
int tsr_hip_rope_table(tsr_hip_ctx * ctx, const int32_t * pos_dev, uint32_t n_dims, float freq_base, float attn_factor,
                       float * tab_dev, void * stream);

/* GGML_GLU_OP_SWIGLU, split form (tsr_lower_glu, sw/ggml-tesseract/tsr-build.cpp:423-490; VOP.SWIGLU
 * sw/sim/tsr_ref_vu.c:102-133): y = SILU(g) u, SILU(g) = g / (1 + EXPK(-g)). */
int tsr_hip_swiglu(tsr_hip_ctx * ctx, const float * g_dev, uint64_t g_stride, const float * u_dev, uint64_t u_stride,
                   uint32_t n, uint32_t rows, float * y_dev, uint64_t y_stride, void * stream);

/* GGML_OP_ADD (the ew kind, sw/ggml-tesseract/tsr-build.cpp:289-332): y = a + b, row r of b at
 * b_dev + (r % b_period) * b_stride (b_period >= 1: a row broadcast). */
int tsr_hip_add(tsr_hip_ctx * ctx, const float * a_dev, uint64_t a_stride, const float * b_dev, uint64_t b_stride,
                uint32_t b_period, uint32_t n, uint32_t rows, float * y_dev, uint64_t y_stride, void * stream);

/* GGML_OP_GET_ROWS on f32 rows (tsr_lower_get_rows, sw/ggml-tesseract/tsr-build.cpp:557-581):
 * y row i = src row ids_dev[i] bit for bit, i < count. An id outside [0, n_src) writes nothing and
 * sets *bad_dev (nullable) to 1 (checked on the device). */
int tsr_hip_get_rows(tsr_hip_ctx * ctx, const float * src_dev, uint64_t src_stride, uint32_t n, uint32_t n_src,
                     const int32_t * ids_dev, uint32_t count, float * y_dev, uint64_t y_stride, int32_t * bad_dev,
                     void * stream);

/* The greedy token pick over logits rows (argmax_row, sw/tools/klcheck.cpp:777-785; std::max_element,
 * sw/ggml-tesseract/tests/test-tsr-mtp.cpp:77-79): out_dev[r] = the first index of the largest value
 * of row r; NaN is never the largest; a row with no value above -inf gives 0. Up to 8 rows of at
 * least 32768 values are picked in two passes whose slice results live in a small per-context array:
 * such calls on different streams of one context must not overlap in time. */
int tsr_hip_argmax(tsr_hip_ctx * ctx, const float * x_dev, uint32_t n, uint32_t rows, uint64_t x_stride,
                   int32_t * out_dev, void * stream);

/* ---- device flags --------------------------------------------------------------------------------
 * Kernels that find a bad input or give up a bounded wait raise a flag word: the bad_dev argument of
 * their entry point, or the context's own word when bad_dev is NULL (and for the entry points that
 * take none, such as tsr_hip_flash_attn_plan): bit 0 an index outside its range (SET_ROWS_KV cell,
 * GET_ROWS id), bit 1 an expired FLASH_ATTN_EXT wait, bit 2 a workgroup on another XCD than its KV
 * head's (results of the launch not valid in every case). Reads the context's word, waiting for the
 * context's stream, and clears it when clear != 0 (the backend's device-failure check after a
 * graph_compute, ggml-tesseract.cpp:2260-2271). Not under capture. */
int tsr_hip_get_flags(tsr_hip_ctx * ctx, int32_t * flags, int clear);

/* ---- counters (the backend's TSR_STATS report, ggml-tesseract.cpp:3799-3866) --------------------- */
/* fa_dec_launches: planned FLASH_ATTN_EXT calls that ran as the one-launch decode form (k_fa_dec);
 * fa_dec_qkv_launches: those of them that also computed the layer's Q|K|V rows
 * (tsr_hip_attn_qkv_plan_rope_tab in one launch rather than its two-call fallback). */
typedef struct tsr_hip_counters {
    uint64_t mul_mat_calls, mul_mat_rows, mul_mat_weight_bytes;
    uint64_t flash_attn_calls, flash_attn_kv_bytes;
    uint64_t set_rows_calls, qact_calls;
    uint64_t fa_dec_launches, fa_dec_qkv_launches;
} tsr_hip_counters;
int tsr_hip_get_counters(tsr_hip_ctx * ctx, tsr_hip_counters * out);

#ifdef __cplusplus
}
#endif
#endif
