/* tsr_ggml.h -- the ggml-backend adapter over libtsr_hip: the backend half of the reference's
 * ggml-tesseract (sw/ggml-tesseract/ggml-tesseract.cpp) that decides what runs on the device, holds
 * the device's buffers and lowers a ggml graph onto the C ABI of include/tsr_hip.h.
 *
 * ggml itself is not linked. The ggml side (a small shim in the backend's registration code) fills
 * one tsr_gg_tensor per ggml_tensor it asks about -- type and op mapped to the
 * values below, ne / nb / op_params / flags / name / view_offs copied, sources, view source, data
 * address and buffer linked -- and forwards the backend callbacks:
 *   ggml_backend_buffer_type_i   get_alignment, get_alloc_size      tsr_gg_alignment, tsr_gg_alloc_size
 *   ggml_backend_buffer_type_i   alloc_buffer                       tsr_gg_buffer_alloc
 *   ggml_backend_buffer_i        get_base, init_tensor, set / get / memset_tensor, clear, free
 *                                                                   tsr_gg_buffer_*
 *   ggml_backend_device_i        supports_op                        tsr_gg_supports_op
 *   ggml_backend_i               graph_compute, synchronize         tsr_gg_graph_compute, tsr_gg_synchronize
 * (reference interfaces: ggml-tesseract.cpp:2026-2042 buffer_i, :2068-2130 buffer type, :4011-4028
 * backend, :4126-4300 supports_op, :3929-3966 graph_compute).
 *
 * Every function returns TSR_GG_OK (0) or a negative TSR_GG_E_* code; tsr_gg_last_error names the node
 * and the reason of the last failure of a device. A device serializes its calls with one mutex (the
 * backend's device mutex, ggml-tesseract.cpp:3932). */
#ifndef TSR_GGML_H
#define TSR_GGML_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSR_GG_OK              0
#define TSR_GG_E_ARG          -1   /* a NULL or malformed argument */
#define TSR_GG_E_UNSUPPORTED  -2   /* a node the device does not run (supports_op says no) */
#define TSR_GG_E_DEVICE       -3   /* a libtsr_hip call failed */
#define TSR_GG_E_NOMEM        -4   /* device or host memory exhausted */
#define TSR_GG_E_FLAG         -5   /* a kernel raised a device flag (an index out of range, an expired wait) */
#define TSR_GG_E_NODEV        -6   /* a probe device (no GPU) was asked for device work */

/* Tensor types (ggml_type: the shim maps GGML_TYPE_F32 -> TSR_GG_TYPE_F32 and so on). A weight of any
 * other ggml type that ggml can dequantize is a "foreign" type: the shim registers it with
 * tsr_gg_register_type (its block size, its block bytes and ggml's to_float) and passes its id. */
#define TSR_GG_TYPE_F32        0
#define TSR_GG_TYPE_F16        1
#define TSR_GG_TYPE_BF16       2
#define TSR_GG_TYPE_Q8_0       3
#define TSR_GG_TYPE_Q4_K       4
#define TSR_GG_TYPE_I32        5
#define TSR_GG_TYPE_I64        6
#define TSR_GG_TYPE_FOREIGN   64   /* 64 + k: the k-th registered type (k < 64) */

/* Ops (ggml_op). Sub-ops are passed in op_params[0] as the shim maps them: GLU -> TSR_GG_GLU_*,
 * UNARY -> TSR_GG_UNARY_*. Every other op_params word is ggml's, unchanged (ROPE's modes are ggml's
 * GGML_ROPE_TYPE_* values). */
#define TSR_GG_OP_NONE            0
#define TSR_GG_OP_RESHAPE         1
#define TSR_GG_OP_VIEW            2
#define TSR_GG_OP_PERMUTE         3
#define TSR_GG_OP_TRANSPOSE       4
#define TSR_GG_OP_MUL_MAT         5
#define TSR_GG_OP_FLASH_ATTN_EXT  6
#define TSR_GG_OP_SET_ROWS        7
#define TSR_GG_OP_RMS_NORM        8
#define TSR_GG_OP_MUL             9
#define TSR_GG_OP_ADD            10
#define TSR_GG_OP_ROPE           11
#define TSR_GG_OP_GLU            12
#define TSR_GG_OP_GET_ROWS       13
#define TSR_GG_OP_ARGMAX         14
#define TSR_GG_OP_SCALE          15
#define TSR_GG_OP_UNARY          16
#define TSR_GG_OP_OTHER         255   /* any other ggml op: refused */

#define TSR_GG_GLU_SWIGLU         2   /* GGML_GLU_OP_SWIGLU */
#define TSR_GG_UNARY_TANH         1   /* GGML_UNARY_OP_TANH */

/* ggml_tensor_flag */
#define TSR_GG_FLAG_INPUT         1
#define TSR_GG_FLAG_OUTPUT        2
#define TSR_GG_FLAG_PARAM         4
#define TSR_GG_FLAG_COMPUTE      16

/* Buffer usage (ggml_backend_buffer_usage) */
#define TSR_GG_USAGE_ANY          0
#define TSR_GG_USAGE_WEIGHTS      1
#define TSR_GG_USAGE_COMPUTE      2

typedef struct tsr_gg_dev tsr_gg_dev;
typedef struct tsr_gg_buffer tsr_gg_buffer;

/* The fields of a ggml_tensor the adapter reads. data is the address ggml holds (base of the tensor's
 * buffer + its offset; a view's data is its view source's data + view_offs); buffer is the adapter
 * buffer that holds the tensor (or its view source), NULL for an unallocated tensor or one in another
 * backend's memory. */
typedef struct tsr_gg_tensor {
    int32_t type;
    int32_t op;
    int64_t ne[4];
    uint64_t nb[4];
    int32_t op_params[16];
    int32_t flags;
    const struct tsr_gg_tensor * src[10];
    const struct tsr_gg_tensor * view_src;
    uint64_t view_offs;
    uint64_t data;
    tsr_gg_buffer * buffer;
    char name[64];
} tsr_gg_tensor;

/* ---- device ------------------------------------------------------------------------------------
 * device >= 0: the GPU with that index (tsr_hip_open). device == -1: a probe device with no GPU:
 * buffers get addresses but no memory, supports_op and tsr_gg_lower work, data access and
 * graph_compute return TSR_GG_E_NODEV (the placement questions llama.cpp asks before any data moves). */
int tsr_gg_open(int device, tsr_gg_dev ** out);
int tsr_gg_close(tsr_gg_dev * dev);
const char * tsr_gg_last_error(const tsr_gg_dev * dev);
/* The libtsr_hip context of a GPU device (NULL for a probe device). */
void * tsr_gg_hip_ctx(tsr_gg_dev * dev);
/* device_i.get_memory (ggml-tesseract.cpp:4046-4057): free and total bytes of the device's memory
 * (hipMemGetInfo of the GPU; the reference reports its weight heap), from which llama.cpp sizes -ngl.
 * A probe device reports 0 and 0. */
int tsr_gg_get_memory(tsr_gg_dev * dev, size_t * free_bytes, size_t * total_bytes);

/* A weight type ggml can dequantize (its type_traits: blck_size values in type_size bytes per block,
 * to_float(blocks, floats, n_values)). MUL_MAT weights of the type are converted to Q8_0 when first
 * used (ggml's to_float, then ggml's quantize_row_q8_0_ref: the reference's load-time conversion,
 * sw/ggml-tesseract/tsr-weights.cpp:33-49). Returns the type id (TSR_GG_TYPE_FOREIGN + k) in *id. */
typedef void (*tsr_gg_to_float_fn)(const void * blocks, float * dst, int64_t n);
int tsr_gg_register_type(tsr_gg_dev * dev, const char * name, uint32_t blck_size, uint32_t type_size,
                         tsr_gg_to_float_fn to_float, int32_t * id);

/* ---- buffer type --------------------------------------------------------------------------------
 * 64-byte alignment and allocation sizes padded to 64 bytes, not host memory (ggml-tesseract.cpp:
 * 2068-2130). */
size_t tsr_gg_alignment(void);
size_t tsr_gg_alloc_size(const tsr_gg_dev * dev, const tsr_gg_tensor * t);

/* ---- buffers ------------------------------------------------------------------------------------
 * A buffer is a range of addresses; its storage is decided at its first data access (or first use by
 * graph_compute) from its usage and its tensors (init_tensor): a buffer whose tensors are all q8_0
 * KV-cache tensors "cache_<tag>k_l<n>" / "cache_<tag>v_l<n>" [E, kv_size, 1] becomes KV planes in the
 * library's layout (tsr-kvbuf.h:61-63; set / get / memset convert the exact ggml q8_0 image); every
 * other buffer is device memory holding ggml's bytes. A weights buffer's 2-D matrices are in addition
 * repacked into the library's weight layout when a MUL_MAT first uses them (and again after a write
 * to them). Writes of a tensor named "*kq_mask*" (F16 [n_kv, n_q]) also build its mask summary (the
 * MSUM producer, tsr-msum.h). */
int tsr_gg_buffer_alloc(tsr_gg_dev * dev, size_t size, int usage, tsr_gg_buffer ** out);
int tsr_gg_buffer_set_usage(tsr_gg_buffer * buf, int usage);
uint64_t tsr_gg_buffer_base(const tsr_gg_buffer * buf);
size_t tsr_gg_buffer_size(const tsr_gg_buffer * buf);
int tsr_gg_buffer_init_tensor(tsr_gg_buffer * buf, const tsr_gg_tensor * t);
int tsr_gg_buffer_set_tensor(tsr_gg_buffer * buf, const tsr_gg_tensor * t, const void * data, size_t offset, size_t size);
int tsr_gg_buffer_get_tensor(tsr_gg_buffer * buf, const tsr_gg_tensor * t, void * data, size_t offset, size_t size);
int tsr_gg_buffer_memset_tensor(tsr_gg_buffer * buf, const tsr_gg_tensor * t, uint8_t value, size_t offset, size_t size);
int tsr_gg_buffer_clear(tsr_gg_buffer * buf, uint8_t value);
/* buffer_i.cpy_tensor (ggml-tesseract.cpp:2026-2042): dst = src in the device's stream order, both in
 * device memory of this device and of the same byte size. Returns 1 when copied, 0 when it cannot copy
 * (ggml then copies through the host), or a negative code. */
int tsr_gg_buffer_cpy_tensor(tsr_gg_buffer * buf, const tsr_gg_tensor * src, const tsr_gg_tensor * dst);
int tsr_gg_buffer_free(tsr_gg_buffer * buf);
/* buffer_i.reset (ggml-tesseract.cpp:2015-2024): ggml-alloc is about to lay the buffer's tensors out
 * anew. A buffer whose storage is not decided yet forgets the tensors init_tensor announced (it is
 * decided from the ones announced after); a buffer that is not KV planes forgets the mask summaries
 * and the host copies of index inputs kept for addresses inside it, so that no FLASH_ATTN_EXT is
 * planned from what an earlier layout wrote there (a mask not written again since fails the
 * graph_compute that needs it). Decided storage, weights and KV planes stay. */
int tsr_gg_buffer_reset(tsr_gg_buffer * buf);
/* The storage the buffer got: 0 undecided, 1 device memory, 2 weights, 3 KV planes. */
int tsr_gg_buffer_mode(const tsr_gg_buffer * buf);

/* ---- supports_op --------------------------------------------------------------------------------
 * 1 when the node runs on the device, 0 when it does not (with the reason in why), negative on a bad
 * argument. The rules of tsr_dev_supports_op (ggml-tesseract.cpp:4126-4300) and tsr_build_supports
 * (tsr-build.cpp) for the ops of this path: MUL_MAT (f32 src1 / dst, 2-D contiguous weight of a
 * loadable type in a weights buffer, K % 32 == 0 and K <= 32768), FLASH_ATTN_EXT (q F32 [D, T, H]
 * heads contiguous, K / V views of one layer's KV planes, D in {64, 128, 256, 512}, H % H_kv == 0, no
 * ALiBi / softcap / sinks / n_kv_max, mask F16 [n_kv, T], T <= 680), SET_ROWS into a KV cache, RMS_NORM,
 * MUL by an f32 weight row behind RMS_NORM, ADD, ROPE (NORMAL / NEOX / IMROPE, no YaRN), GLU SWIGLU,
 * GET_ROWS of f32 rows, ARGMAX, SCALE and TANH behind a MUL_MAT (its epilogue); the no-ops (NONE,
 * RESHAPE, VIEW, PERMUTE, TRANSPOSE). */
int tsr_gg_supports_op(tsr_gg_dev * dev, const tsr_gg_tensor * op, char * why, size_t why_len);

/* ---- graph_compute ------------------------------------------------------------------------------
 * Runs the nodes in order on the device's stream (the caller's inputs written by set_tensor before,
 * its outputs read by get_tensor after, both in stream order). The lowered calls of a graph are kept
 * per graph identity (every node's op, type, shape, strides, data address and op_params and those of
 * its sources; the values are not part of it: ggml-tesseract.cpp:3937-3952, at most 16 graphs, least
 * recently used out). A graph met again re-plans only its FLASH_ATTN_EXT chunk lists from the current
 * mask summaries and new cells; a graph whose calls can all be captured (decode: every MUL_MAT of
 * fewer than 16 tokens) is captured into a HIP graph on its second run and replayed from then on
 * (captured again when a chunk list changes shape). Returns when the work is queued: device flags
 * raised by its kernels are reported by the next get_tensor or synchronize (TSR_GG_E_FLAG). */
int tsr_gg_graph_compute(tsr_gg_dev * dev, const tsr_gg_tensor * const * nodes, int n_nodes);
int tsr_gg_synchronize(tsr_gg_dev * dev);

/* Options of a device: TSR_GG_OPT_NO_FUSION lowers every node on its own (no fold, group or epilogue
 * fusion; the results are the same bits). Plans made under other options are not reused. */
#define TSR_GG_OPT_NO_FUSION  1u
int tsr_gg_set_options(tsr_gg_dev * dev, uint32_t options);

typedef struct tsr_gg_stats {
    uint64_t graphs, plan_hits, plan_misses, captures, replays, eager_runs;
    uint64_t calls, fused, weights_converted, masks_summarized;
} tsr_gg_stats;
int tsr_gg_get_stats(tsr_gg_dev * dev, tsr_gg_stats * out);

/* ---- lowering, for inspection ---------------------------------------------------------------------
 * The calls graph_compute would make for the nodes, without running them (also on a probe device).
 * kind: one of TSR_GG_CALL_*; node / node2 / node3: the graph indices of the node and of the nodes fused
 * into it (-1 for none; for a MUL_MAT node3 is the RMS_NORM folded into it); the other fields as each
 * call reads them (addresses are ggml data addresses; 0 for a plan's own buffer).
 * graph_compute fuses llama.cpp's layer pattern into the decoder's launch list:
 *   - RMS_NORM * w read only by MUL_MATs of fewer than 16 tokens: the norm inside each matvec;
 *   - the Q, K, V MUL_MATs of one input, whose results only reach the ROPEs, the K / V SET_ROWS and
 *     the FLASH_ATTN_EXT: one MUL_MAT over their rows into a plan buffer, then for one token one
 *     ROPE + SET_ROWS_KV + FLASH_ATTN_EXT launch (TSR_GG_CALL_ROPE_TABLE once per graph), for more
 *     tokens TSR_GG_CALL_ROPE_KV and the planned FLASH_ATTN_EXT; the K and V SET_ROWS must then write
 *     the same cells (else graph_compute fails: TSR_GG_E_UNSUPPORTED); for one token with the norm
 *     folded into that MUL_MAT, the MUL_MAT runs inside the FLASH_ATTN_EXT call
 *     (tsr_hip_attn_qkv_plan_rope_tab) and its own call carries TSR_GG_CALL_IN_NEXT in flags;
 *   - the gate and up MUL_MATs read only by a SWIGLU: one MUL_MAT with the GLU epilogue.
 * Each fusion leaves the results bit-identical to the unfused calls. */
#define TSR_GG_CALL_MUL_MAT     1
#define TSR_GG_CALL_FLASH_ATTN  2
#define TSR_GG_CALL_SET_ROWS    3
#define TSR_GG_CALL_RMS_NORM    4
#define TSR_GG_CALL_ADD         5
#define TSR_GG_CALL_ROPE        6
#define TSR_GG_CALL_SWIGLU      7
#define TSR_GG_CALL_GET_ROWS    8
#define TSR_GG_CALL_ARGMAX      9
#define TSR_GG_CALL_ROPE_TABLE 10   /* the ROPE angles of a decode token, once per graph */
#define TSR_GG_CALL_ROPE_KV    11   /* ROPE of q and k + SET_ROWS of k and v over a ubatch's Q|K|V rows */
#define TSR_GG_CALL_IN_NEXT    0x80000000u   /* flags: the call's work runs inside its group's FLASH_ATTN_EXT call */
typedef struct tsr_gg_call {
    int32_t kind, node, node2, node3;
    uint32_t N, K, T, flags;            /* MUL_MAT: rows, K, tokens, TSR_HIP_MM_* ; elementwise: n, rows */
    uint64_t x, y, add, w;              /* operands: input, output, addend / second input, weight / table */
    uint64_t x_stride, y_stride, add_stride;   /* in floats */
    float scale, scale2;                /* FA scale, RMS eps, MUL_MAT epilogue scales, ROPE freq_base */
    uint32_t D, n_head, n_head_kv, n_kv, kv_size, which, mode, n_dims;
} tsr_gg_call;
int tsr_gg_lower(tsr_gg_dev * dev, const tsr_gg_tensor * const * nodes, int n_nodes, tsr_gg_call * out, int cap,
                 int * n_out);

/* ---- helpers the backend shares with its tests ----------------------------------------------------
 * tsr_gg_kv_parse_name: "cache_<tag>k_l<n>" -> which 0, "cache_<tag>v_l<n>" -> 1 (tsr-kvbuf.h:
 * tsr_kv_parse_name); 1 on a match, 0 otherwise.
 * tsr_gg_graph_key: the identity graph_compute caches by, mixed with salt.
 * tsr_gg_quantize_q8_0: K f32 values (K % 32 == 0) -> K/32 ggml block_q8_0 (ggml's
 * quantize_row_q8_0_ref: d = max|x| / 127, id = 1 / d (0 when d is 0), q = round-half-away(x id),
 * the block's scale stored as fp16(d)). */
int tsr_gg_kv_parse_name(const char * name, uint32_t * which, int * layer);
uint64_t tsr_gg_graph_key(const tsr_gg_tensor * const * nodes, int n_nodes, uint64_t salt);
int tsr_gg_quantize_q8_0(const float * x, int64_t K, void * blocks);

#ifdef __cplusplus
}
#endif

#endif /* TSR_GGML_H */
