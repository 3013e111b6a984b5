/*
 * vkml_hip.h -- the C ABI over HIP that replaces vkml's Vulkan HAL.
 *
 * The reference's ops reach the GPU through src/hal (Device, Buffer,
 * ComputePipeline, Stream) and src/core/runtime.hpp. This library replaces
 * that seam with plain C entry points on one HIP device and one in-order HIP
 * stream: lifecycle and device info, device and pinned host memory, stream
 * copies, a submit/wait fence timeline, per-kernel profiling, HIP graphs for
 * the decode step, and one launch entry per kernel family whose parameter
 * struct mirrors the reference's push constants. The C++ API (vkml::Context,
 * vkml::Tensor, the ops, vkml::Llama) is built on these calls only.
 *
 * Conventions: every function returns VKML_OK (0) or an error code; the
 * message of the last error on the calling thread is vkml_last_error().
 * Pointers named d_* are device memory from vkml_malloc (or any HIP device
 * allocation); all launches are asynchronous on the library's stream, in
 * order. One vkml_init per process (the reference allows one live Context,
 * src/hal/device.cpp:104-108). Sizes are counts of elements unless they say
 * bytes. Not thread-safe: one thread drives the library, as one drives a
 * vkml::Context (src/core/runtime.hpp:24).
 */
#ifndef VKML_HIP_H
#define VKML_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VKML_ABI_VERSION 1

enum vkml_status {
    VKML_OK = 0,
    VKML_ERROR_INVALID_ARGUMENT = 1,
    VKML_ERROR_NO_DEVICE = 2,
    VKML_ERROR_DEVICE = 3,
    VKML_ERROR_STATE = 4,
    VKML_ERROR_UNSUPPORTED = 5,
    VKML_ERROR_OUT_OF_MEMORY = 6
};

/* Element and weight formats. 0-5 are the TYPE_ constants of the reference's
 * shaders/include/halves.glsl:5-24; VKML_Q4_K is llama.cpp's q4_K kept in its
 * own 256-value super-blocks (values: the 128 code bytes of each super-block;
 * scales: its 16-byte header, f16 d, f16 dmin and 12 bytes of 6-bit scales
 * and mins), decoded in-kernel to the Q4_1 values the reference repacks it
 * into (src/io/gguf.cpp:596-627). */
enum vkml_type {
    VKML_F32 = 0, VKML_F16 = 1, VKML_BF16 = 2,
    VKML_Q8_0 = 3, VKML_Q4_0 = 4, VKML_Q4_1 = 5, VKML_Q4_K = 6,
    VKML_I32 = 7
};

/* ---------------------------------------------------------------------- */
/* Device lifecycle: replaces hal::Device (src/hal/device.cpp:103-118,    */
/* 234-286) and DeviceInfo (include/vkml/context.hpp:28-70).              */
/* ---------------------------------------------------------------------- */

typedef struct vkml_device_info {
    char name[256];          /* marketing name, e.g. "AMD Instinct MI355X" */
    char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    char driver[64];         /* HIP runtime version */
    uint64_t global_memory_bytes;
    uint32_t compute_units;
    uint32_t wave_size;
    uint32_t max_threads_per_block;
    uint32_t max_block_dims[3];
    uint32_t max_grid_dims[3];
    uint32_t lds_bytes_per_block;
    uint32_t l2_bytes;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_bits;
    int32_t integer_dot_product; /* v_dot4_i32_i8 on gfx950: always 1 */
    int32_t timestamps;          /* hipEvent timing available: always 1 */
    double timestamp_period_ns;
} vkml_device_info;

const char* vkml_last_error(void);
int vkml_abi_version(void);
/* device_name: case-insensitive substring of the name or arch; NULL or "" means
 * the VKML_DEVICE environment variable, then device 0 (context.cpp:24-26). */
int vkml_init(const char* device_name);
int vkml_shutdown(void);
int vkml_is_initialized(void);
int vkml_get_device_info(vkml_device_info* out);

/* ---------------------------------------------------------------------- */
/* Memory and copies: replaces hal::Buffer (src/hal/buffer.cpp:26-54) and */
/* Stream::copy; copies are ordered on the stream.                        */
/* ---------------------------------------------------------------------- */

int vkml_malloc(uint64_t bytes, void** d_out);
int vkml_free(void* d_ptr);
int vkml_host_malloc(uint64_t bytes, void** h_out); /* pinned */
int vkml_host_free(void* h_ptr);
int vkml_memcpy_h2d(void* d_dst, const void* h_src, uint64_t bytes);
int vkml_memcpy_d2h(void* h_dst, const void* d_src, uint64_t bytes);
int vkml_memcpy_d2d(void* d_dst, const void* d_src, uint64_t bytes);
/* words 32-bit words of value at d_dst, by a kernel (runtime.cpp:97-103). */
int vkml_fill_u32(void* d_dst, uint32_t value, uint64_t words);

/* ---------------------------------------------------------------------- */
/* Timeline: Stream::submit/wait (src/hal/stream.cpp:156-206). A fence is */
/* a monotonically increasing value; work submitted before it is done     */
/* once vkml_completed reports it.                                        */
/* ---------------------------------------------------------------------- */

int vkml_submit(uint64_t* fence_out);
int vkml_wait(uint64_t fence);
int vkml_completed(uint64_t* fence_out);
int vkml_synchronize(void);
/* The library's one in-order stream, as a hipStream_t, so a caller can
 * order its own HIP work (events, copies) with the library's launches. No
 * reference counterpart: the reference's Stream is internal to its HAL. */
void* vkml_stream(void);

/* ---------------------------------------------------------------------- */
/* Profiling: Context::set_profiling/profile/reset_profile               */
/* (include/vkml/context.hpp:115-126, src/hal/stream.cpp:258-306). With   */
/* profiling on, each launch is bracketed by HIP events and totalled per  */
/* kernel label when waited on; graphs are not replayed while profiling.  */
/* ---------------------------------------------------------------------- */

typedef struct vkml_kernel_time {
    char name[48];
    uint64_t calls;
    double milliseconds;
} vkml_kernel_time;

int vkml_set_profiling(int enabled);
int vkml_get_profiling(void);

/* Polls a workgroup that waits for another workgroup of its launch (the o
 * GEMV of vkml_attend_step_o / _fused / _fast waiting for the merges)
 * makes before it gives up and sets the launch's error flag (0: the default,
 * 1 << 20). Launches made afterwards take the new limit, captured graphs
 * the one they were captured with. No reference counterpart: the
 * reference's dispatches never wait on one another. For tests that force
 * a timeout from the host, and callers sharing the GPU's compute units. */
int vkml_set_wait_limit(uint32_t polls);
/* While tag is non-empty, profiled launches are labelled "kernel:tag" (the
 * model tags its projections: "gemv_dot:qkv", "gemv_dot_add:down", ...). */
int vkml_set_profile_tag(const char* tag);
/* Writes up to capacity entries, slowest first; *count gets the total. */
int vkml_profile(vkml_kernel_time* out, uint32_t capacity, uint32_t* count);
int vkml_reset_profile(void);

/* ---------------------------------------------------------------------- */
/* HIP graphs: capture launches on the stream into a replayable graph     */
/* (the decode step). No reference counterpart: vkml records command     */
/* buffers per step (src/hal/stream.cpp:86-141).                          */
/* ---------------------------------------------------------------------- */

int vkml_graph_begin(void);
int vkml_graph_end(uint64_t* graph_out);
int vkml_graph_launch(uint64_t graph);
int vkml_graph_destroy(uint64_t graph);

/* ---------------------------------------------------------------------- */
/* Kernels. Each struct mirrors the push constants (and specialization     */
/* constants) of the reference shader it replaces.                        */
/* ---------------------------------------------------------------------- */

/* shaders/quantize.comp, src/ops/quantize.cpp:21-63. x: [blocks * 32] of
 * src_type (F32/F16/BF16); quant Q8_0/Q4_0/Q4_1; scale_type F32 or F16.
 * values: 8 (Q8_0) or 4 words per block; scales: one per block, or
 * (scale, offset) pairs for Q4_1. */
typedef struct vkml_quantize_params {
    uint32_t blocks;
    uint32_t src_type;
    uint32_t quant;
    uint32_t scale_type;
} vkml_quantize_params;
int vkml_quantize(const vkml_quantize_params* p, const void* d_x, void* d_values, void* d_scales);
/* The SwiGLU product of a prompt's MLP and its Q8_0 form in one pass, as
 * llama.cpp:381-384 dispatches silu (shaders/unary.comp:21-24), mul
 * (binary.comp) and, for the int8 down projection, quantize.comp
 * (matmul.cpp:225-229): h[i] = silu(gate[i]) * up[i] in those f32
 * operations, then h's Q8_0 codes (count bytes) and f32 scales (one per 32
 * values) as vkml_quantize's Q8_0/F32 form. count a multiple of 32; gate
 * and up 16-byte aligned. */
int vkml_swiglu_quantize(uint32_t count, const float* d_gate, const float* d_up, void* d_values,
                         float* d_scales);

/* shaders/dequantize.comp, src/ops/quantize.cpp:79-94: count values of a
 * [rows, cols] matrix (cols given for Q4_K's super-block rows). */
typedef struct vkml_dequantize_params {
    uint32_t count;
    uint32_t quant;
    uint32_t scale_type;
    uint32_t cols;
} vkml_dequantize_params;
int vkml_dequantize(const vkml_dequantize_params* p, const void* d_values, const void* d_scales,
                    float* d_out);

/* The largest k the one-row int8 GEMVs stage in LDS. Above it (any
 * multiple of 32 for q8_0 / q4_0 / q4_1, of 256 for q4_K), vkml_gemv_dot
 * and vkml_gemv_dot_add take the rows kernel, which reads the activation
 * from memory, in the same order; the fused forms (SwiGLU, RMSNorm
 * prologue) take k up to this bound. */
#define VKML_GEMV_STAGED_MAX_K 32768u

/* shaders/gemv_dot.comp, src/ops/matmul.cpp:225-245: c[m, n] = a_q[m] . b[n]
 * for m <= 8 rows of Q8_0 activations (f32 scales) and weights b [n, k] of
 * b_type Q8_0/Q4_0/Q4_1/Q4_K (scales F16, or F32 for Q8_0/Q4_0/Q4_1).
 * Argument order is the reference's buffer order (matmul.cpp:234-237). */
typedef struct vkml_gemv_dot_params {
    uint32_t m, n, k;
    uint32_t b_type;
    uint32_t scale_type;
} vkml_gemv_dot_params;
int vkml_gemv_dot(const vkml_gemv_dot_params* p, const void* d_a_values, const void* d_b_values,
                  float* d_out, const void* d_b_scales, const float* d_a_scales);
/* shaders/matmul_dot.comp (src/ops/matmul.cpp:246-259): c = a_q . b^T for
 * any m (the reference's path for m > 8: prompts), in its order: each
 * output sums K's 32-value blocks in order, the block's exact integer dot
 * product scaled in f32 (q8_0 / q4_0: float(sum) * (sa * sb); q4_1 / q4_K:
 * sa * (float(sum) * sb + float(asum) * offset)). Arguments as
 * vkml_gemv_dot's; k a multiple of 32 (q4_K: 256). On the matrix cores
 * (v_mfma_i32_16x16x32_i8: one block of a 16 x 16 tile). */
int vkml_matmul_dot(const vkml_gemv_dot_params* p, const void* d_a_values, const void* d_b_values,
                    float* d_out, const void* d_b_scales, const float* d_a_scales);
/* vkml_matmul_dot with the residual add that follows a prompt's o and down
 * projections (llama.cpp:374,386; binary.comp's add, src/ops/
 * elementwise.cpp:23-60) done as each output is stored: d_out[m, n] =
 * d_residual[m, n] + (a_q . b^T)[m, n], the same f32 sum (d_out may equal
 * d_residual). */
int vkml_matmul_dot_add(const vkml_gemv_dot_params* p, const void* d_a_values, const void* d_b_values,
                        float* d_out, const void* d_b_scales, const float* d_a_scales,
                        const float* d_residual);
/* As vkml_gemv_dot for m = 1, with the residual add that follows the o and
 * down projections (llama.cpp:374,386) done in the epilogue:
 * d_out[n] = d_residual[n] + a_q . b[n] (d_out may equal d_residual). */
int vkml_gemv_dot_add(const vkml_gemv_dot_params* p, const void* d_a_values,
                      const void* d_b_values, float* d_out, const void* d_b_scales,
                      const float* d_a_scales, const float* d_residual);
/* The SwiGLU MLP's first half for m = 1 (llama.cpp:380-382): with g = a_q .
 * gate[n] and u = a_q . up[n], d_h[n] = silu(g) * u, silu(v) = v / (1 +
 * exp(-v)) (shaders/unary.comp:21-24). gate and up share b_type/scale_type. */
int vkml_gemv_dot_swiglu(const vkml_gemv_dot_params* p, const void* d_a_values,
                         const float* d_a_scales, const void* d_gate_values,
                         const void* d_gate_scales, const void* d_up_values,
                         const void* d_up_scales, float* d_h);

/* vkml_gemv_dot with the steps around it folded in (no single reference
 * counterpart: rms_norm.comp + quantize.comp before gemv_dot.comp, and
 * binary/unary + quantize.comp after, as llama.cpp:313-386 dispatches them).
 * norm = 1: d_a is the f32 row x [k], RMS-normalized with d_norm_weight and
 * eps and quantized to Q8_0 inside the kernel (k <= 4096), bit for bit as
 * vkml_rms_norm_quantize; norm = 2 (store epilogue only): d_a is the f32
 * row, quantized to Q8_0 inside the kernel without a norm (k <= 4096), bit
 * for bit as vkml_quantize
 * (quantize.comp; matmul.cpp:225-229's activation quantize folded into the
 * product); norm = 0: d_a / d_a_scales are its Q8_0 codes and
 * f32 scales. epilogue 0 stores y, 1 adds d_residual (not with norm), 2 is
 * SwiGLU with the up matrix d_b2_*; quantize_out (SwiGLU, n % 32 == 0) also
 * writes h's Q8_0 codes and f32 scales. m = 1. */
typedef struct vkml_gemv_fused_params {
    uint32_t n;
    uint32_t k;
    uint32_t b_type;
    uint32_t scale_type;
    uint32_t epilogue;
    uint32_t norm;
    float eps;
    uint32_t quantize_out;
} vkml_gemv_fused_params;
int vkml_gemv_fused(const vkml_gemv_fused_params* p, const void* d_a, const float* d_a_scales,
                    const float* d_norm_weight, const void* d_b_values, const void* d_b_scales,
                    const void* d_b2_values, const void* d_b2_scales, const float* d_residual,
                    float* d_out, void* d_out_values, float* d_out_scales);

/* A decode step's q|k|v projection with the work that follows it in the
 * reference folded into the epilogue: llama.cpp:313-355's rms_norm +
 * quantize (as vkml_gemv_fused norm 1), the projection, RoPE of q and k at
 * d_state->position (interleaved pairs, rope.comp:94-118, as
 * vkml_rope_kv_append rotates them) and the new key and value rounded to
 * the cache type and written at row position % capacity of each KV head
 * (cast.comp + write_rows.comp, llama.cpp:344-355). The b rows are rows
 * row0 .. row0 + n of [q | k | v] (heads * head_dim, then kv_heads *
 * head_dim each); d_qkv receives rows row0 .. row0 + n of the rotated q and
 * k and of v. With rotate = 0 nothing is rotated. A step whose attention
 * then reads q and the caches as left here sets prepared in
 * vkml_attend_step_params. No reference counterpart as one call. */
typedef struct vkml_gemv_rope_params {
    uint32_t n;
    uint32_t k;
    uint32_t b_type;
    uint32_t scale_type;
    float eps;
    uint32_t row0;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t capacity;
    uint32_t kv_type;
    uint32_t rotate;
} vkml_gemv_rope_params;
struct vkml_decode_state;
int vkml_gemv_rope(const vkml_gemv_rope_params* p, const float* d_x, const float* d_norm_weight,
                   const void* d_b_values, const void* d_b_scales, float* d_qkv,
                   const float* d_rope_table, const struct vkml_decode_state* d_state,
                   void* d_k_cache, void* d_v_cache);

/* shaders/gemv.comp, src/ops/matmul.cpp:88-120: the float path, c[m, n] =
 * a[m] . b[n] with f32 a (m <= 8) and b [n, k] of b_type F32/F16/BF16 or
 * Q8_0/Q4_0/Q4_1/Q4_K decoded in registers (ContextOptions::
 * integer_dot_product off, and f32 models). With batches > 1 (float b
 * only) as gemv.comp's z: a [batches, m, k], c [batches, m, n], batch z
 * against b's batch z / b_group, b_stride elements apart (attention's
 * scores for up to 8 queries, matmul.cpp:96). batches and b_group 0 mean 1. */
typedef struct vkml_gemv_params {
    uint32_t m, n, k;
    uint32_t b_type;
    uint32_t scale_type;
    uint32_t b_stride;
    uint32_t b_group;
    uint32_t batches;
} vkml_gemv_params;
int vkml_gemv(const vkml_gemv_params* p, const float* d_a, const void* d_b, float* d_out,
              const void* d_b_scales);

/* shaders/matmul.comp (src/ops/matmul.cpp:44-120): c = a . b or a . b^T for
 * f32 a [batches * b_group, m, k] and b [batches, k, n] (or [n, k]) of b_type
 * F32/F16/BF16; b_stride elements between b's batches (0: shared b). Each
 * output sums its k products in k order. b may also be one transposed
 * quantized matrix (Q8_0/Q4_0/Q4_1/Q4_K, scales of scale_type in d_b_scales,
 * values widened as vkml_gemv's): the float path's projections of more than
 * 8 rows (matmul.cpp:96-97). Argument order is the reference's buffers
 * (a, b, c, scales; matmul.cpp:107). causal = 1 skips the work a causal
 * mask makes moot, row r of each batch seeing keys 0 .. r + causal_offset:
 * with b_transposed (scores) the outputs past that are not written; else
 * (probs . v) a's entries past it must be 0, and the sums stop where every
 * row of a tile has passed its last key (adding the zeros would change
 * nothing). No counterpart in the reference, which computes both. */
typedef struct vkml_matmul_params {
    uint32_t m, n, k;
    uint32_t b_stride;
    uint32_t b_group;
    uint32_t batches;
    uint32_t b_transposed;
    uint32_t b_type;
    uint32_t scale_type;
    uint32_t causal;
    uint32_t causal_offset;
} vkml_matmul_params;
int vkml_matmul(const vkml_matmul_params* p, const float* d_a, const void* d_b, float* d_out,
                const void* d_b_scales);

/* shaders/rms_norm.comp, src/ops/norms.cpp:230-253. */
typedef struct vkml_rms_norm_params {
    uint32_t rows, cols;
    float eps;
} vkml_rms_norm_params;
int vkml_rms_norm(const vkml_rms_norm_params* p, const float* d_x, const float* d_w, float* d_out);
/* rms_norm then quantize_q8 with f32 scales (the SharedInput of the next
 * projections, matmul.cpp:229): d_out (optional, may be NULL) gets the f32
 * normalized rows, d_values/d_a_scales their Q8_0 form. cols % 32 == 0. */
int vkml_rms_norm_quantize(const vkml_rms_norm_params* p, const float* d_x, const float* d_w,
                           float* d_out, void* d_values, float* d_scales);

/* shaders/softmax.comp, src/ops/norms.cpp:176-211: rows of scale * x, with
 * an optional causal mask (query row % q_len at key position offset + that)
 * and window; -inf entries become 0. With ring (and causal), the columns
 * are a ring of that many keys holding key position p in column p % ring
 * (CausalMask::ring, ops/internal.hpp:67-74): row r sees positions up to
 * r % q_len + offset, the last `window` of them with a window. */
typedef struct vkml_softmax_params {
    uint32_t rows, cols;
    float scale;
    uint32_t causal;
    uint32_t q_len;
    uint32_t offset;
    uint32_t window;
    float softcap;
    uint32_t ring;
} vkml_softmax_params;
int vkml_softmax(const vkml_softmax_params* p, const float* d_x, float* d_out);

/* shaders/argmax.comp, src/ops/norms.cpp:213-228: first index of each row's
 * largest non-NaN entry; 0 if all are NaN. */
int vkml_argmax(uint32_t rows, uint32_t cols, const float* d_x, int32_t* d_out);

/* shaders/rope.comp, src/ops/rope.cpp:20-28,88-129. style 0 interleaved
 * pairs (2i, 2i+1), 1 rotate-half (i, i + dim/2). */
typedef struct vkml_rope_params {
    uint32_t pairs;
    uint32_t half_dim;
    uint32_t dim;
    uint32_t heads;
    uint32_t seq;
    uint32_t start_pos;
    uint32_t copies;
    uint32_t style;
} vkml_rope_params;
int vkml_rope(const vkml_rope_params* p, const float* d_x, const float* d_table, float* d_out);

/* shaders/cast.comp, src/ops/cast.cpp:24-46: f32 -> f16/bf16 rounding to
 * nearest even on the bits (no flush), f16/bf16 -> f32 exact, f32 copy. */
int vkml_cast(uint32_t count, uint32_t src_type, uint32_t dst_type, const void* d_x, void* d_out);

/* shaders/write_rows.comp, src/ops/attention.cpp:86-122 (CopyRowsParams):
 * 32-bit words. */
typedef struct vkml_copy_rows_params {
    uint32_t count;
    uint32_t block;
    uint32_t src_stride;
    uint32_t src_start;
    uint32_t dst_stride;
    uint32_t dst_start;
} vkml_copy_rows_params;
int vkml_copy_rows(const vkml_copy_rows_params* p, const void* d_src, void* d_dst);

/* shaders/permute.comp, src/ops/permute.cpp:34-81: out dimension i is input
 * dimension dims[i], up to 6 dimensions of 32-bit elements. */
typedef struct vkml_permute_params {
    uint32_t rank;
    uint32_t count;
    uint32_t in_shape[6];
    uint32_t dims[6];
} vkml_permute_params;
int vkml_permute(const vkml_permute_params* p, const void* d_x, void* d_out);

/* shaders/binary.comp and unary.comp (src/ops/elementwise.cpp:23-87).
 * binary op: 0 add, 1 sub, 2 mul, 3 div, b repeating every b_count;
 * unary op: 0 silu, 1 gelu (tanh), 2 softcap(param). */
int vkml_binary(uint32_t op, uint32_t count, uint32_t b_count, const float* d_a, const float* d_b,
                float* d_out);
int vkml_unary(uint32_t op, uint32_t count, float param, const float* d_x, float* d_out);

/* shaders/embedding.comp and embedding_quantized.comp (src/ops/
 * embedding.cpp:19-91): rows ids of a [vocab, dim] table of table_type
 * (F32/F16/BF16/Q8_0/Q4_0/Q4_1/Q4_K); out-of-range ids give zero rows. */
typedef struct vkml_embedding_params {
    uint32_t count; /* ids * dim */
    uint32_t dim;
    uint32_t vocab;
    uint32_t table_type;
    uint32_t scale_type;
} vkml_embedding_params;
int vkml_embedding(const vkml_embedding_params* p, const void* d_values, const void* d_scales,
                   const int32_t* d_ids, float* d_out);

/* ---------------------------------------------------------------------- */
/* Decode attention (shaders/attend.comp + attend_merge.comp,             */
/* src/ops/attention.cpp:22-84). Keys kv_start..kv_len (at most capacity  */
/* of them) of caches [kv_heads, capacity, head_dim] (F32 or F16), key    */
/* position p at row p % capacity (a sliding window's ring), in the       */
/* reference's chunks of 128 keys from kv_start, a                        */
/* workgroup per (chunk, query head). With d_state non-NULL, kv_len is    */
/* d_state->position + 1 (the replayed decode step) and the launch covers */
/* the whole cache. chunks: the partial buffers' stride, at least         */
/* ceil((kv_len - kv_start) / 128), or ceil((capacity - kv_start) / 128)  */
/* with d_state. partial: [heads, chunks, head_dim] f32; stats: [heads,   */
/* chunks, 2] (max score, sum of exp); chunks past kv_len get max -inf.   */
/* ---------------------------------------------------------------------- */

typedef struct vkml_decode_state {
    int32_t token;    /* input token of the next step */
    int32_t position; /* its position; the KV rows written by the step */
    int32_t steps;    /* tokens appended to the log so far */
    int32_t reserved;
} vkml_decode_state;

typedef struct vkml_attend_params {
    uint32_t kv_start;
    uint32_t kv_len;
    uint32_t capacity;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t kv_type;
    uint32_t chunks;
    float scale;
    float softcap;
} vkml_attend_params;
int vkml_attend(const vkml_attend_params* p, const float* d_q, const void* d_k_cache,
                const void* d_v_cache, float* d_partial, float* d_stats,
                const vkml_decode_state* d_state);
/* Merges the chunks into out [heads, head_dim] f32 and, when d_values is
 * non-NULL, its Q8_0 form with f32 scales (the o projection's input). */
int vkml_attend_merge(const vkml_attend_params* p, const float* d_partial, const float* d_stats,
                      float* d_out, void* d_values, float* d_scales);

/* One layer's attention for a decode step: rope of q and of the new key,
 * the new key and value appended at the position as vkml_rope_kv_append
 * does, vkml_attend over keys kv_start..position, and vkml_attend_merge into
 * d_out [heads, head_dim] f32 with its Q8_0 form in d_values / d_scales
 * (when non-NULL): two launches, arithmetic that of those kernels
 * (llama.cpp:320-369 in order). d_qkv = [q | k | v] f32 of this token.
 * partial / stats as vkml_attend, chunks >= ceil((capacity - kv_start) /
 * 128). Position from d_state if non-NULL. */
typedef struct vkml_attend_step_params {
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t capacity;
    uint32_t kv_start;
    uint32_t position;
    uint32_t kv_type;
    uint32_t chunks;
    uint32_t rope_style; /* 0 interleaved pairs, 1 rotate-half */
    uint32_t rotate;     /* 0: no rope in this layer */
    float scale;
    float softcap;
    /* Sliding window: the step's query sees keys max(kv_start, position + 1
     * - window) .. position (attention.cpp:40-47 with a window), in chunks of
     * 128 from the first (0: no window). With a window the caches can be a
     * ring (capacity rows, position p at row p % capacity), and chunks must
     * cover min(window, capacity) keys. */
    uint32_t window;
    /* 1: q in d_qkv is already rotated and the new key and value are already
     * in the caches (vkml_gemv_rope ran before, with d_state); the step then
     * neither rotates nor appends. */
    uint32_t prepared;
    /* vkml_attend_step_fused: chunks that hold keys at every position the
     * call may see (a hint; 0: none); their items load q, K and V before
     * reading the position. Prepared steps without a window only. */
    uint32_t ready_chunks;
} vkml_attend_step_params;
int vkml_attend_step(const vkml_attend_step_params* p, const float* d_qkv, const float* d_rope_table,
                     void* d_k_cache, void* d_v_cache, float* d_partial, float* d_stats,
                     float* d_out, void* d_values, float* d_scales, const vkml_decode_state* d_state);

/* vkml_attend_step, then the o projection with its residual add,
 * d_x[n] += o[n] . (the attention output's Q8_0 form) as vkml_gemv_dot_add
 * (llama.cpp:320-374): bit for bit those calls. The merge and the GEMV
 * share a launch where the o weights are q4_K or q8_0 with f16 scales, the
 * GEMV reads every attention output (o->k = heads * head_dim) and the grid
 * fits the GPU at once: the merge's workgroups publish the Q8_0 output and
 * the GEMV's, their first weight loads issued, wait for it on d_sync (a
 * bounded wait; vkml_attend_o_check reports one that gave up). Otherwise
 * the three launches. d_values / d_scales are required (the o input).
 * d_sync: vkml_attend_o_sync_bytes() bytes, zeroed once before first use;
 * one per stream of calls (the chunk pass clears it for the launch after). */
uint64_t vkml_attend_o_sync_bytes(void);
int vkml_attend_step_o(const vkml_attend_step_params* p, const float* d_qkv, const float* d_rope_table,
                       void* d_k_cache, void* d_v_cache, float* d_partial, float* d_stats, float* d_out,
                       void* d_values, float* d_scales, const vkml_decode_state* d_state,
                       const vkml_gemv_dot_params* o, const void* d_o_values, const void* d_o_scales,
                       float* d_x, uint32_t* d_sync);
/* Synchronizes, then reports (VKML_ERROR_DEVICE) and clears a wait of an
 * earlier vkml_attend_step_o on this sync buffer that timed out. */
int vkml_attend_o_check(uint32_t* d_sync);
/* The same check without the error: *flag gets 0, or 1 for a wait that
 * gave up (then cleared). */
int vkml_attend_o_status(uint32_t* d_sync, uint32_t* flag);

/* vkml_attend_step_o (llama.cpp:313-374, attention.cpp:54-84) in one
 * launch where the shapes allow it (q4_K, or q8_0 with f16 scales, o
 * weights; a decode state): the chunk pass, then per KV head and head
 * group the last chunk item to finish merges its heads (attend_merge.comp's
 * order), and the o GEMV + residual, whose workgroups load their weights
 * at once and wait (bounded) for every merge. Same results bit for bit.
 * d_sync holds `blocks` (>= 2) blocks of vkml_attend_fused_sync_bytes(1)
 * bytes, zeroed before the first call; a call uses block `block` and
 * zeroes the counters of block (block + 1) % blocks, so consecutive calls
 * on the stream take consecutive blocks, cyclically (in a model, layer L
 * takes block L of one block per layer). Other shapes, and steps of more
 * than 64 chunks (whose one-workgroup merges would outlast separate
 * launches): the chunk pass, the merge (spread over (head, 32-element
 * slice) workgroups) and vkml_gemv_dot_add as separate launches, with the
 * same block bookkeeping. p->chunks may cover fewer keys than the cache (a
 * launch sized for the position rather than the capacity): keys past
 * kv_start + 128 * chunks are then not attended, and a step whose position
 * reaches them raises the error vkml_attend_fused_check reports (the one
 * launch, and steps of more than 64 chunks; the separate launches of other
 * shapes need chunks covering the cache). */
uint64_t vkml_attend_fused_sync_bytes(uint32_t blocks);
int vkml_attend_step_fused(const vkml_attend_step_params* p, const float* d_qkv, const float* d_rope_table,
                           void* d_k_cache, void* d_v_cache, float* d_partial, float* d_stats, float* d_out,
                           void* d_values, float* d_scales, const vkml_decode_state* d_state,
                           const vkml_gemv_dot_params* o, const void* d_o_values, const void* d_o_scales,
                           float* d_x, uint32_t* d_sync, uint32_t block, uint32_t blocks);
/* Synchronizes, then reports (VKML_ERROR_DEVICE) and clears (every block) a
 * wait of an earlier vkml_attend_step_fused on these blocks that timed out. */
int vkml_attend_fused_check(uint32_t* d_sync, uint32_t blocks);
/* The same check without the error: *flag gets 0, 1 for a wait that gave
 * up, or 2 for a position past the launched chunks (then every block is
 * cleared). */
int vkml_attend_fused_status(uint32_t* d_sync, uint32_t blocks, uint32_t* flag);
/* 1 when vkml_attend_step_fused takes these shapes in its one launch on
 * this device (the o format, the item's LDS, the merge's chunk count and a
 * grid whose waiting o workgroups leave the chunk items a slot) at every
 * chunk count up to min(p->chunks, 64); 0 when it would take the separate
 * launches, which then need p->chunks covering the cache. Steps of more
 * than 64 chunks always take the separate launches (the merge spread over
 * many workgroups); those may be sized below the cache, and a position
 * past their chunks sets the error flag as the one launch does. No
 * reference counterpart (a host-side plan query). */
int vkml_attend_step_fused_supported(const vkml_attend_step_params* p, const vkml_gemv_dot_params* o);

/* Decode attention on the matrix cores, the tolerance form of
 * vkml_attend + vkml_attend_merge (attend.comp + attend_merge.comp,
 * attention.cpp:54-84 there): not the reference's order of f32 operations
 * but f32 attention to within f32 rounding (the products exact, f16 x f16
 * with q and the softmax weights split in two f16 terms; the sums in f32 in
 * the matrix unit's order). An option beside the bit-exact kernels, which
 * stay the default. f16 caches, head_dim 64 or 128, at most 8 query heads
 * a KV head, at most 1024 chunks of 128 keys. One launch: the chunk items,
 * then per KV head a merge by its last item into d_out [heads, head_dim]
 * f32 (may be NULL) and, when d_values is non-NULL, its Q8_0 form with f32
 * scales. d_partial [heads, chunks, head_dim] and d_stats [heads, chunks, 2]
 * f32 are its workspace; d_sync: vkml_attend_fused_sync_bytes(1) bytes,
 * zeroed before the first call (each call leaves it zeroed). Position
 * from d_state (kv_len = position + 1) if non-NULL; chunks cover kv_len -
 * kv_start (with d_state, capacity - kv_start). */
int vkml_attend_fast(const vkml_attend_params* p, const float* d_q, const void* d_k_cache, const void* d_v_cache,
                     float* d_partial, float* d_stats, float* d_out, void* d_values, float* d_scales, uint32_t* d_sync,
                     const vkml_decode_state* d_state);
/* vkml_attend_step_fused's one launch (chunks, merges, o GEMV + residual)
 * with vkml_attend_fast's items and merges: a prepared step (vkml_gemv_rope
 * rotated q and appended the new key and value) without a window, at the
 * decode state's position; the same sync blocks, check
 * (vkml_attend_fused_check) and chunk tiers (p->chunks may cover fewer keys
 * than the cache; p->ready_chunks as there). The o GEMV and residual are
 * vkml_gemv_dot_add's bit for bit on the attention output it is given. */
int vkml_attend_step_fast(const vkml_attend_step_params* p, const float* d_qkv, void* d_k_cache, void* d_v_cache,
                          float* d_partial, float* d_stats, float* d_out, void* d_values, float* d_scales,
                          const vkml_decode_state* d_state, const vkml_gemv_dot_params* o, const void* d_o_values,
                          const void* d_o_scales, float* d_x, uint32_t* d_sync, uint32_t block, uint32_t blocks);
/* 1 when vkml_attend_step_fast takes these shapes on this device (cache
 * type, head_dim, group, window, prepared, o format, and a grid whose o
 * workgroups leave the chunk items a slot); 0 otherwise. */
int vkml_attend_step_fast_supported(const vkml_attend_step_params* p, const vkml_gemv_dot_params* o);

/* A prompt's causal attention on the matrix cores: the tolerance form of
 * the reference's chunked q.k^T, causal softmax and probs.v
 * (attention.cpp:127-138,205-226; softmax.comp's soft cap), f32 attention
 * within f32 rounding, online over blocks of keys (not the reference's
 * order of f32 operations). d_q [heads, t, head_dim] f32 (rotated, heads
 * first, as vkml_rope_kv_prompt leaves it); the caches [kv_heads,
 * capacity, head_dim] f16 hold keys 0 .. first + t - 1 at rows of the same
 * number; query i sees keys 0 .. first + i. d_out [t, heads, head_dim] f32:
 * the o projection's input rows (no permute after it). head_dim 64 or 128,
 * a multiple of 4 query heads a KV head. No reference counterpart as one
 * call. */
typedef struct vkml_attend_prompt_params {
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t capacity;
    uint32_t t;      /* queries */
    uint32_t first;  /* key position of query 0 */
    uint32_t kv_type;
    float scale;
    float softcap;   /* 0: none */
} vkml_attend_prompt_params;
int vkml_attend_prompt_fast(const vkml_attend_prompt_params* p, const float* d_q, const void* d_k_cache, const void* d_v_cache,
                            float* d_out);
/* 1 when vkml_attend_prompt_fast takes these shapes. */
int vkml_attend_prompt_fast_supported(const vkml_attend_prompt_params* p);

/* vkml_attend_step without the d_partial / d_stats workspace, allocating
 * nothing: no counterpart in the reference. For callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation). The partials and statistics live in the
 * library's own device scratch of VKML_ATTEND_SCRATCH_BYTES per GPU (held
 * until the process ends): heads * chunks * head_dim * 4 bytes rounded up to
 * 256, plus heads * chunks * 8, must fit (VKML_ERROR_INVALID_ARGUMENT
 * otherwise; 32 heads of 128 at 32768 positions need 4.3 MB). Results are
 * bit for bit vkml_attend_step's. Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (graphs replayed on other streams)
 * race; calls on the library's stream are ordered and do not. */
#define VKML_ATTEND_SCRATCH_BYTES (8u << 20)
int vkml_attend_step_noalloc(const vkml_attend_step_params* p, const float* d_qkv, const float* d_rope_table,
                             void* d_k_cache, void* d_v_cache, float* d_out, void* d_values, float* d_scales,
                             const vkml_decode_state* d_state);


/* ---------------------------------------------------------------------- */
/* Fused decode-step kernels (no single reference counterpart: each       */
/* replaces a sequence of the reference's dispatches, cited).             */
/* ---------------------------------------------------------------------- */

/* heads_first + rope + cast + write_rows for one token (llama.cpp:320-355):
 * qkv = [q (heads*hd) | k (kv_heads*hd) | v (kv_heads*hd)] f32; q is rotated
 * into d_q; k rotated and v are rounded to the cache type and written at row
 * position of every KV head. Position from d_state if non-NULL. */
typedef struct vkml_rope_kv_params {
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t capacity;
    uint32_t position;
    uint32_t style;
    uint32_t kv_type;
    uint32_t rotate; /* 0: no rope in this layer */
} vkml_rope_kv_params;
int vkml_rope_kv_append(const vkml_rope_kv_params* p, const float* d_qkv, const float* d_table,
                        float* d_q, void* d_k_cache, void* d_v_cache,
                        const vkml_decode_state* d_state);
/* The same for a prompt of `tokens` tokens at positions p->position..: row
 * t of d_qkv (row_stride floats apart) holds token t's q | k | v; q is
 * rotated into d_q [heads, tokens, head_dim] (heads first, llama.cpp:
 * 320-327), k rotated and v rounded to the cache type and written at rows
 * (position + t) % capacity (llama.cpp:344-355; a ring wraps around,
 * attention.cpp:260-266). tokens <= capacity; the RoPE table holds
 * position + tokens rows. */
int vkml_rope_kv_prompt(const vkml_rope_kv_params* p, uint32_t tokens, uint32_t row_stride,
                        const float* d_qkv, const float* d_table, float* d_q, void* d_k_cache,
                        void* d_v_cache);

/* Decode-state helpers for the replayable step: set the state, embed its
 * token, and finish the step (argmax into the state and a token log, then
 * position += 1; with d_logits NULL only the position advances). */
int vkml_state_set(vkml_decode_state* d_state, int32_t token, int32_t position, int32_t steps);
int vkml_embedding_state(const vkml_embedding_params* p, const void* d_values,
                         const void* d_scales, const vkml_decode_state* d_state, float* d_out);
int vkml_step_finish(uint32_t vocab, const float* d_logits, vkml_decode_state* d_state,
                     int32_t* d_token_log, uint32_t log_capacity);


#ifdef __cplusplus
}
#endif
#endif
