/*
 * runit_hip.h — C ABI of the MI355X (gfx950) quantized-GEMV decode path.
 *
 * This library replaces the Metal kernel runtime of RunIT's `crates/kernels`
 * crate for the decode hot path.  Every `rt_<name>` kernel entry point takes
 * the same arguments, in the same order and with the same meaning, as the
 * reference's `dispatch::<name>(ctx, ...)` Rust function; Metal `&Buffer`
 * arguments become device pointers and `u32` dimensions stay `uint32_t`.
 *
 * Execution model (mirrors crates/kernels/src/context.rs:248-296):
 *   - every kernel call only ENQUEUES work on the context's HIP stream
 *     (the reference encodes onto one open command buffer);
 *   - rt_flush() waits for all enqueued work (the reference's `flush()`).
 *   - A context is not thread-safe (the reference's MetalContext is !Sync,
 *     context.rs:158); use one context per host thread.
 *
 * Weights are raw GGUF block streams, row-major, each row = K/blk blocks:
 *   Q8_0 34 B / 32 el, Q4_0 18 B / 32 el, Q4_K 144 B / 256 el,
 *   Q6_K 210 B / 256 el  (crates/gguf/src/types.rs:158-191),
 * decoded with the reference's own layouts (crates/engine/src/forward.rs).
 *
 * Pointer rules: every pointer must be a device pointer (rt_malloc or any
 * hipMalloc'd memory).  f32 activation vectors must be 16-byte aligned and
 * f16 ones 8-byte aligned (the reference reads x as float4 / half4).
 * `output` may alias `residual` (forward.rs:1619,1702 pass the same buffer).
 *
 * Status codes map one-to-one onto crates/kernels/src/error.rs:4-21.
 */
#ifndef RUNIT_HIP_H
#define RUNIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KernelError variants (crates/kernels/src/error.rs:4-21). */
typedef enum rt_status {
    RT_OK = 0,
    RT_ERR_NO_DEVICE = 1,          /* KernelError::NoDevice */
    RT_ERR_LIBRARY_LOAD = 2,       /* KernelError::LibraryLoad { path, reason } */
    RT_ERR_PIPELINE_NOT_FOUND = 3, /* KernelError::PipelineNotFound(name) */
    RT_ERR_PIPELINE_CREATE = 4,    /* KernelError::PipelineCreate { name, reason } */
    RT_ERR_DISPATCH = 5,           /* KernelError::Dispatch(msg) */
    RT_ERR_BUFFER_SIZE = 6,        /* KernelError::BufferSize { expected, actual } */
    /* GgufError variants (crates/gguf/src/error.rs:4-31), rt_gguf_* only */
    RT_ERR_GGUF_IO = 16,             /* GgufError::Io */
    RT_ERR_GGUF_MAGIC = 17,          /* GgufError::InvalidMagic */
    RT_ERR_GGUF_VERSION = 18,        /* GgufError::UnsupportedVersion */
    RT_ERR_GGUF_DTYPE = 19,          /* GgufError::UnknownDtype */
    RT_ERR_GGUF_METADATA_TYPE = 20,  /* GgufError::UnknownMetadataType */
    RT_ERR_GGUF_EOF = 21,            /* GgufError::UnexpectedEof */
    RT_ERR_GGUF_UTF8 = 22,           /* GgufError::InvalidUtf8 */
    RT_ERR_GGUF_DATA_OVERFLOW = 23   /* GgufError::DataRegionOverflow */
} rt_status;

typedef struct rt_ctx rt_ctx;

/* ───────────────────────── context / runtime ───────────────────────── */

/* MetalContext::new() (context.rs:163-205): selects device 0, loads the
 * gfx950 code objects at `code_object_path` (one .hsaco file or a directory of
 * them; NULL → the lib/kernels/ directory next to this library), resolves
 * every kernel, creates one stream. */
int rt_ctx_create(rt_ctx** out, const char* code_object_path);
/* Drop for MetalContext (context.rs:299-304): flushes, then releases. */
void rt_ctx_destroy(rt_ctx* ctx);
/* MetalContext::flush() (context.rs:289-296): waits for all enqueued work. */
int rt_flush(rt_ctx* ctx);
/* Human-readable text of the last error on this context (KernelError's
 * Display string); never NULL. */
const char* rt_last_error(const rt_ctx* ctx);
/* Text for an error raised before a context exists (rt_ctx_create). */
const char* rt_global_last_error(void);
/* Number of compute units of the context's device. */
int rt_device_cu_count(const rt_ctx* ctx);
/* Resolves a kernel by name, like the reference's PSO lookup
 * (context.rs:207-212): RT_ERR_PIPELINE_NOT_FOUND if absent. */
int rt_has_kernel(rt_ctx* ctx, const char* name);

/* MetalContext::new_buffer (context.rs:215-220) — device memory.  MI355X
 * memory is not CPU-visible here, so contents move with upload/download. */
int rt_malloc(rt_ctx* ctx, size_t bytes, void** out);
int rt_free(rt_ctx* ctx, void* ptr);
/* Synchronous on the context stream (orders after enqueued kernels). */
int rt_upload(rt_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
int rt_download(rt_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
int rt_memset(rt_ctx* ctx, void* dst_dev, int value, size_t bytes);
int rt_copy_d2d(rt_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);

/* Stream timing (HIP events recorded on the context stream). */
typedef struct rt_event rt_event;
int rt_event_create(rt_ctx* ctx, rt_event** out);
int rt_event_record(rt_ctx* ctx, rt_event* ev);
int rt_event_elapsed_ms(rt_ctx* ctx, rt_event* start, rt_event* stop, float* ms);
void rt_event_destroy(rt_event* ev);

/* HIP-graph capture of a sequence of enqueued kernels (replaces the
 * reference's single reusable command buffer for a whole decode step). */
typedef struct rt_graph rt_graph;
int rt_capture_begin(rt_ctx* ctx);
int rt_capture_end(rt_ctx* ctx, rt_graph** out);
int rt_graph_launch(rt_ctx* ctx, rt_graph* g);
void rt_graph_destroy(rt_graph* g);

/* ───────────────────────── Q8_0 GEMV family ─────────────────────────
 * y[r] = Σ_k d_b·q[r,k]·x[k]; m = rows, k = reduction length (k % 32 == 0). */

/* dispatch.rs:1280-1295  → gemv_q8_0.metal:56-82 */
int rt_gemv_q8_0_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                              float* output, uint32_t m, uint32_t k);
/* dispatch.rs:1298-1314  → gemv_q8_0.metal:88-114 (output may alias residual) */
int rt_gemv_q8_0_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
/* dispatch.rs:1317-1332  → gemv_q8_0.metal:120-145 (f16 output, RNE) */
int rt_gemv_q8_0_f32in(rt_ctx* ctx, const void* weight, const float* input,
                       uint16_t* output, uint32_t m, uint32_t k);
/* dispatch.rs:1335-1351  → gemv_q8_0.metal:151-176 (f16 in, f16 out) */
int rt_gemv_q8_0_f16(rt_ctx* ctx, const void* weight, const uint16_t* input,
                     uint16_t* output, uint32_t m, uint32_t k);
/* dispatch.rs:1353-1370  → gemv_q8_0.metal:182-208 (f16 in/out/residual) */
int rt_gemv_q8_0_add_f16(rt_ctx* ctx, const void* weight, const uint16_t* input,
                         uint16_t* output, const uint16_t* residual, uint32_t m, uint32_t k);
/* dispatch.rs:1372-1388  → gemv_q8_0.metal:214-240 (f16 in, f32 out/residual) */
int rt_gemv_q8_0_add_f32res_f16(rt_ctx* ctx, const void* weight, const uint16_t* input,
                                float* output, const float* residual, uint32_t m, uint32_t k);
/* dispatch.rs:1083-1098 → gemv_multirow.metal:163-200 (same result as the
 * non-_mr kernel; kept as its own entry point for drop-in call sites). */
int rt_gemv_q8_0_f32in_f32out_mr(rt_ctx* ctx, const void* weight, const float* input,
                                 float* output, uint32_t m, uint32_t k);
/* dispatch.rs:1101-1117 → gemv_multirow.metal:205-243 */
int rt_gemv_q8_0_add_f32_f32in_mr(rt_ctx* ctx, const void* weight, const float* input,
                                  float* output, const float* residual, uint32_t m, uint32_t k);

/* ───────────────────────── Q4_0 GEMV family ───────────────────────── */

/* dispatch.rs:1456-1469 → gemv_q4_0.metal:75-104 */
int rt_gemv_q4_0_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                              float* output, uint32_t m, uint32_t k);
/* dispatch.rs:1471-1484 → gemv_q4_0.metal:110-140 */
int rt_gemv_q4_0_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
/* dispatch.rs:1486-1499 → gemv_q4_0.metal:146-175 (f16 output) */
int rt_gemv_q4_0_f32in(rt_ctx* ctx, const void* weight, const float* input,
                       uint16_t* output, uint32_t m, uint32_t k);
/* dispatch.rs:1501-1514 → gemv_q4_0.metal:181-210 */
int rt_gemv_q4_0_f16(rt_ctx* ctx, const void* weight, const uint16_t* input,
                     uint16_t* output, uint32_t m, uint32_t k);
/* dispatch.rs:1516-1529 → gemv_q4_0.metal:216-246 */
int rt_gemv_q4_0_add_f16(rt_ctx* ctx, const void* weight, const uint16_t* input,
                         uint16_t* output, const uint16_t* residual, uint32_t m, uint32_t k);

/* ───────────────────────── Q4_K GEMV family ───────────────────────── */

/* dispatch.rs:1229-1249 → gemv_q4k.metal:186-211 (k % 256 == 0) */
int rt_gemv_q4k_f32in_f32out(rt_ctx* ctx, const void* weight_q4k, const float* input,
                             float* output, uint32_t m, uint32_t k);
/* dispatch.rs:1251-1272 → gemv_q4k.metal:215-241 */
int rt_gemv_q4k_add_f32_f32in(rt_ctx* ctx, const void* weight_q4k, const float* input,
                              float* output, const float* residual, uint32_t m, uint32_t k);
/* dispatch.rs:621 (gemv_q4k_f16) → gemv_q4k.metal:126-150 */
int rt_gemv_q4k_f16(rt_ctx* ctx, const void* weight_q4k, const uint16_t* input,
                    uint16_t* output, uint32_t m, uint32_t k);
/* dispatch.rs:585 (gemv_q4k_add_f16) → gemv_q4k.metal:156-181 */
int rt_gemv_q4k_add_f16(rt_ctx* ctx, const void* weight_q4k, const uint16_t* input,
                        uint16_t* output, const uint16_t* residual, uint32_t m, uint32_t k);
/* dispatch.rs:358 (gemv_q4k_add_f32res_f16) → gemv_q4k.metal:245-271 */
int rt_gemv_q4k_add_f32res_f16(rt_ctx* ctx, const void* weight_q4k, const uint16_t* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);

/* ───────────────────────── Q6_K GEMV (new) ─────────────────────────
 * The reference has no Q6_K GEMV: it dequantises Q6_K to f16 on the CPU
 * (forward.rs:513-557) and runs gemv_f16w_f32in_f32out(_mr) /
 * gemv_add_f32_f16w(_mr).  These read the packed 210-byte blocks directly,
 * with the reference's decode (forward.rs:921-950, one scale per 32). */
int rt_gemv_q6k_f32in_f32out(rt_ctx* ctx, const void* weight_q6k, const float* input,
                             float* output, uint32_t m, uint32_t k);
int rt_gemv_q6k_add_f32_f32in(rt_ctx* ctx, const void* weight_q6k, const float* input,
                              float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q6k_f32in(rt_ctx* ctx, const void* weight_q6k, const float* input,
                      uint16_t* output, uint32_t m, uint32_t k);
/* No counterpart in the reference.  rt_gemv_q6k_add_f32_f32in for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops that forbid hipMalloc): it calls no hipMalloc / hipFree and takes its
 * K-split partial sums, activation records and arrival counters from a fixed
 * 4 MiB array in the code object (one per device, held until the process
 * ends) instead of the context's on-demand workspace.  Same kernels and
 * results as rt_gemv_q6k_add_f32_f32in.  Shapes needing more than the
 * array's regions (K-split partials: ~2.9 MiB, i.e. chunks × m floats;
 * activation records: 1 MiB) return RT_ERR_DISPATCH.  All calls on one
 * device share the array, which keeps the last call's contents: calls that
 * overlap on one device (two contexts or streams) race. */
int rt_gemv_q6k_add_f32_f32in_noalloc(rt_ctx* ctx, const void* weight_q6k, const float* input,
                                      float* output, const float* residual, uint32_t m,
                                      uint32_t k);

/* ───────────────────────── Q5_0 / Q5_K GEMV (new) ─────────────────────────
 * The reference has no Q5 GEMVs: the loader dequantises Q5_0 (forward.rs:
 * 900-920) and Q5_K (forward.rs:979-1012) on the CPU and runs the f16-weight
 * GEMVs.  These read the packed 22-byte / 176-byte blocks directly, with the
 * reference's decode (its Q5_K high-bit order: bit e%8 of qh[e/8] for
 * element e).  Arguments as the Q4_K family. */
int rt_gemv_q5_0_f32in_f32out(rt_ctx* ctx, const void* weight_q5_0, const float* input,
                              float* output, uint32_t m, uint32_t k);
int rt_gemv_q5_0_add_f32_f32in(rt_ctx* ctx, const void* weight_q5_0, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q5_0_f32in(rt_ctx* ctx, const void* weight_q5_0, const float* input,
                       uint16_t* output, uint32_t m, uint32_t k);
int rt_gemv_q5k_f32in_f32out(rt_ctx* ctx, const void* weight_q5k, const float* input,
                             float* output, uint32_t m, uint32_t k);
int rt_gemv_q5k_add_f32_f32in(rt_ctx* ctx, const void* weight_q5k, const float* input,
                              float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q5k_f32in(rt_ctx* ctx, const void* weight_q5k, const float* input,
                      uint16_t* output, uint32_t m, uint32_t k);

/* ───────────────────── ggml layouts (new) ─────────────────────
 * The reference decodes Q4_0, Q4_K and Q6_K (and Q5_K) in layouts that
 * differ from upstream ggml (forward.rs:964-978 interleaved Q4_0 nibbles,
 * :1026-1057 Q4_K sub-block pairs (j, j+4), :921-950 one Q6_K scale per 32,
 * :979-1012 Q5_K high bit e%8 of qh[e/8]).  Real GGUF files use ggml's:
 *   q4_0g: element j < 16 = low nibble of qs[j], 16 + j = its high nibble;
 *   q4kg : 64-element chunk j uses sub-blocks 2j (low) and 2j+1 (high);
 *   q5kg : as q4kg, fifth bit = bit 2j (low) / 2j+1 (high) of qh[l];
 *   q6kg : element h + 32t + l uses sc[h/16 + l/16 + 2t] (16 scales).
 * Same block sizes and arguments as the reference-layout entry points. */
int rt_gemv_q4_0g_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, uint32_t m, uint32_t k);
int rt_gemv_q4_0g_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                                float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q4_0g_f32in(rt_ctx* ctx, const void* weight, const float* input, uint16_t* output,
                        uint32_t m, uint32_t k);
int rt_gemv_q4kg_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                              float* output, uint32_t m, uint32_t k);
int rt_gemv_q4kg_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q4kg_f32in(rt_ctx* ctx, const void* weight, const float* input, uint16_t* output,
                       uint32_t m, uint32_t k);
int rt_gemv_q5kg_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                              float* output, uint32_t m, uint32_t k);
int rt_gemv_q5kg_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q5kg_f32in(rt_ctx* ctx, const void* weight, const float* input, uint16_t* output,
                       uint32_t m, uint32_t k);
int rt_gemv_q6kg_f32in_f32out(rt_ctx* ctx, const void* weight, const float* input,
                              float* output, uint32_t m, uint32_t k);
int rt_gemv_q6kg_add_f32_f32in(rt_ctx* ctx, const void* weight, const float* input,
                               float* output, const float* residual, uint32_t m, uint32_t k);
int rt_gemv_q6kg_f32in(rt_ctx* ctx, const void* weight, const float* input, uint16_t* output,
                       uint32_t m, uint32_t k);
int rt_fused_ffn_q4_0g_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                           const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
int rt_fused_ffn_q4kg_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                          const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
int rt_fused_ffn_q5kg_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                          const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
int rt_dequant_q4_0g_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q4kg_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q5kg_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q6kg_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);

/* ───────────────────────── fused kernels ───────────────────────── */

/* dispatch.rs:813-838 → fused_qkv.metal:72-119 */
int rt_fused_qkv_q8_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                          const float* x_vec, float* out_q, float* out_k, float* out_v,
                          uint32_t q_dim, uint32_t kv_dim, uint32_t k);
/* dispatch.rs:842-871 → fused_qkv.metal:13-69; out = W·x + f32(bias_f16) */
int rt_fused_qkv_bias_q8_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                               const float* x_vec, float* out_q, float* out_k, float* out_v,
                               const uint16_t* bias_q, const uint16_t* bias_k,
                               const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                               uint32_t k);
/* New: the Q4_0 twin of fused_qkv_bias_q8_0_f32 (same arguments). */
int rt_fused_qkv_bias_q4_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                               const float* x_vec, float* out_q, float* out_k, float* out_v,
                               const uint16_t* bias_q, const uint16_t* bias_k,
                               const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                               uint32_t k);
/* New: Q/K/V projections of Q4_K / Q4_K_M files in one launch.  They replace
 * the reference's fallback sequence for non-Q8_0 projections: three
 * WeightBuf GEMVs, each followed by add_f16_into_f32 of its bias
 * (forward.rs:1561-1568).  Arguments follow fused_qkv_bias_q8_0_f32.  The
 * three bias pointers may all be NULL (no bias); giving only some of them is
 * an error.
 *   _q4k      : Q, K and V in Q4_K;
 *   _q4k_q6k  : Q and K in Q4_K, V in Q6_K (the Q4_K_M mix);
 *   _q4kg / _q4kg_q6kg : the same in the ggml layouts. */
int rt_fused_qkv_bias_q4k_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                              const float* x_vec, float* out_q, float* out_k, float* out_v,
                              const uint16_t* bias_q, const uint16_t* bias_k,
                              const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                              uint32_t k);
int rt_fused_qkv_bias_q4k_q6k_f32(rt_ctx* ctx, const void* w_q, const void* w_k,
                                  const void* w_v, const float* x_vec, float* out_q,
                                  float* out_k, float* out_v, const uint16_t* bias_q,
                                  const uint16_t* bias_k, const uint16_t* bias_v, uint32_t q_dim,
                                  uint32_t kv_dim, uint32_t k);
int rt_fused_qkv_bias_q4kg_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                               const float* x_vec, float* out_q, float* out_k, float* out_v,
                               const uint16_t* bias_q, const uint16_t* bias_k,
                               const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                               uint32_t k);
int rt_fused_qkv_bias_q4kg_q6kg_f32(rt_ctx* ctx, const void* w_q, const void* w_k,
                                    const void* w_v, const float* x_vec, float* out_q,
                                    float* out_k, float* out_v, const uint16_t* bias_q,
                                    const uint16_t* bias_k, const uint16_t* bias_v,
                                    uint32_t q_dim, uint32_t kv_dim, uint32_t k);
/* dispatch.rs:903-921 → fused_ffn.metal:36-93; act = silu(Wg·x)·(Wu·x) */
int rt_fused_ffn_q8_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                          const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
/* dispatch.rs:1531-1544 → gemv_q4_0.metal:254-311 */
int rt_fused_ffn_q4_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                          const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
/* New: Q4_K gate+up+SiLU (same arguments). */
int rt_fused_ffn_q4k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                         const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);

/* New: Q5_0 / Q5_K twins of fused_qkv_bias_q8_0_f32 and fused_ffn_q8_0_f32
 * (same arguments). */
int rt_fused_qkv_bias_q5_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                               const float* x_vec, float* out_q, float* out_k, float* out_v,
                               const uint16_t* bias_q, const uint16_t* bias_k,
                               const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                               uint32_t k);
int rt_fused_qkv_bias_q5k_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                              const float* x_vec, float* out_q, float* out_k, float* out_v,
                              const uint16_t* bias_q, const uint16_t* bias_k,
                              const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                              uint32_t k);
int rt_fused_ffn_q5_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                          const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);
int rt_fused_ffn_q5k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                         const float* x_vec, float* act_out, uint32_t ff_dim, uint32_t k);

/* ───────────────────────── dequantisation ─────────────────────────
 * Bit-exact restatements of the reference decoders, to f32:
 *   Q8_0 forward.rs:951-963, Q4_0 :964-978, Q4_K :1026-1057 (+:359-369),
 *   Q6_K :921-950.  n_blocks = number of GGUF blocks. */
int rt_dequant_q8_0_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q4_0_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q4k_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q6k_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
/* New: Q5_0 forward.rs:900-920, Q5_K forward.rs:979-1012 (+:359-369). */
int rt_dequant_q5_0_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
int rt_dequant_q5k_f32(rt_ctx* ctx, const void* input, float* output, uint32_t n_blocks);
/* dispatch.rs:756-772 → dequant.metal:53-98 (Q4_K → f16, RNE). */
int rt_dequant_q4k_f16(rt_ctx* ctx, const void* input, uint16_t* output, uint32_t n_blocks);

/* ───────────────────────── batched Q8_0 GEMM (new) ─────────────────────────
 * Y[M,N] = X[M,K] · W[N,K]ᵀ with W in Q8_0; X, Y f32 row-major.
 * Replaces the reference's only M>1 path, gemm_f16 on f16-dequantised
 * weights in verify_draft (forward.rs:2193-2271, gemm.metal:39-190). */
int rt_gemm_q8_0_f32(rt_ctx* ctx, const void* weight, const float* x, float* y,
                     uint32_t m_rows, uint32_t n, uint32_t k);
/* New: the same batched GEMM on Q4_0 and Q4_K weights in the reference's
 * layouts (7B verify / prefill of Q4_0 and Q4_K_M files; the reference
 * dequantises to f16 for gemm_f16, forward.rs:2193-2271).  Q4_K needs k a
 * multiple of 256.  Shapes whose row segments are not 8/16-byte aligned run
 * as one GEMV per activation row. */
int rt_gemm_q4_0_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k);
int rt_gemm_q4k_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k);
/* New: the same batched GEMM on the remaining block formats of Q4_K_M /
 * Q5_K_M files and on the ggml layouts: Q5_0 (reference: CPU dequant,
 * forward.rs:900-920), Q5_K (forward.rs:979-1012), Q6_K (forward.rs:921-950;
 * k a multiple of 512 for the staged kernel), and the ggml-layout families
 * (rt_gemv_*g).  K-quants need k a multiple of 256. */
int rt_gemm_q5_0_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k);
int rt_gemm_q5k_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k);
int rt_gemm_q6k_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k);
int rt_gemm_q4_0g_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                      uint32_t n, uint32_t k);
int rt_gemm_q4kg_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k);
int rt_gemm_q5kg_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k);
int rt_gemm_q6kg_f32(rt_ctx* ctx, const void* weight, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k);
/* New: the batched GEMMs of verify_draft that share one activation matrix,
 * with the kernels between them folded in (forward.rs:2186-2271: the Q/K/V
 * projections of the normalised rows + their f16 biases; gate and up + SiLU;
 * O and down + the residual).  count (1..4) weight matrices, fmts[i] the
 * block format of weight[i] ("q8_0", "q4_0", "q4k", "q5_0", "q5k", "q6k",
 * "q4_0g", "q4kg", "q5kg", "q6kg"), y[i] [m_rows][n[i]]:
 *   X = x, or RMSNorm(x)·gamma (eps) when gamma is given, written to xn
 *       ([m_rows][k], required with gamma);
 *   y[i] = X·weight[i]ᵀ (+ f32(bias[i]) on every row, bias and bias[i] may
 *       be NULL);
 *   res (count 1, not y[0]): y[0] = res + X·weight[0]ᵀ;
 *   silu_pair (count 2, one shape, no bias / res): y[0] = silu(X·weight[0]ᵀ)
 *       · (X·weight[1]ᵀ), y[1] left unspecified.
 * Where every matrix takes the f16 matrix-core form with one row grouping,
 * x is prepared once (the norm in the preparation) and the bias / residual /
 * SiLU run in the K-split sums; otherwise as the separate launches. */
int rt_gemm_set_f32(rt_ctx* ctx, uint32_t count, const char* const* fmts, const void* const* weight,
                    float* const* y, const uint32_t* n, const uint16_t* const* bias,
                    const float* res, const float* x, uint32_t m_rows, uint32_t k,
                    const float* gamma, float eps, float* xn, uint32_t silu_pair);
/* New: the Q/K/V projections of verify_draft (forward.rs:2186-2231) as one
 * call: rt_gemm_set_f32 of the three matrices with their f16 biases over
 * RMSNorm(x)·gamma (written to xn), then RoPE of q and k at positions
 * start_pos + r (rt_rope_kv_write_batch_f32) and k / v written to the caches
 * ([kv_dim / head_dim][max_seq][head_dim]).  q receives the rotated rows;
 * k and v ([m_rows][kv_dim]) are left unspecified.  On the shared f16 form
 * the rotation and the cache writes run in the K-split sum launch. */
int rt_gemm_qkv_rope_f32(rt_ctx* ctx, const char* fmt_q, const void* w_q, const char* fmt_k,
                         const void* w_k, const char* fmt_v, const void* w_v, const uint16_t* b_q,
                         const uint16_t* b_k, const uint16_t* b_v, const float* x,
                         const float* gamma, float eps, float* xn, float* q, float* k, float* v,
                         float* k_cache, float* v_cache, uint32_t m_rows, uint32_t hidden,
                         uint32_t q_dim, uint32_t kv_dim, uint32_t head_dim, uint32_t start_pos,
                         float theta, uint32_t max_seq);
/* New: the part of a verify_draft layer after the attention
 * (forward.rs:2227-2271) over M rows as one call: O + residual, RMSNorm,
 * gate / up + SiLU, down + residual, each projection in its own block format:
 *   x_mid = x + att·w_oᵀ;  X2 = RMSNorm(x_mid)·gamma;
 *   g = silu(X2·w_gateᵀ) · (X2·w_upᵀ);  x = x_mid + g·w_downᵀ
 * (att [m_rows][qd], x and x_mid [m_rows][h], x_mid apart from x).  Where all
 * four take the f16 matrix-core form with one row grouping, each sum of K
 * splits is folded into the next projection's activation preparation
 * (8 launches); otherwise it runs as three rt_gemm_set_f32 calls, which also
 * write g, u ([m_rows][ff]) and xn ([m_rows][h], X2); the shared form leaves
 * them unspecified. */
int rt_gemm_ffn_block_f32(rt_ctx* ctx, const char* fmt_o, const void* w_o, const char* fmt_gate,
                          const void* w_gate, const char* fmt_up, const void* w_up,
                          const char* fmt_down, const void* w_down, const float* att, float* x,
                          float* x_mid, const float* gamma, float eps, float* g, float* u,
                          float* xn, uint32_t m_rows, uint32_t h, uint32_t qd, uint32_t ff);
/* New: the attention of a verify_draft layer (forward.rs:2225-2226,
 * rt_flash_attention_f32 with batch 1, q_len = m_rows) followed by
 * rt_gemm_ffn_block_f32 over its output, as one call (qd = num_heads ·
 * head_dim).  Where the block takes its shared form and the attention its
 * multi-range matrix-core form, the attention leaves per-range partials and
 * the O projection's operand preparation merges them, as the attention's own
 * last workgroup would; att is then left unspecified.  Otherwise att receives
 * the attention output and the two calls run in turn. */
int rt_gemm_attn_ffn_block_f32(rt_ctx* ctx, const float* q, const float* k_cache,
                               const float* v_cache, uint32_t kv_len, uint32_t num_heads,
                               uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride,
                               uint32_t q_start, float* att, const char* fmt_o, const void* w_o,
                               const char* fmt_gate, const void* w_gate, const char* fmt_up,
                               const void* w_up, const char* fmt_down, const void* w_down, float* x,
                               float* x_mid, const float* gamma, float eps, float* g, float* u,
                               float* xn, uint32_t m_rows, uint32_t h, uint32_t ff);

/* ──────────────── multi-row GEMVs (batched verify / prefill) ────────────────
 * New: the M-row projections of verify_draft (forward.rs:2186-2271, which
 * dequantises to f16 and runs gemm_f16) on the quantized weights: rows
 * activation rows x [rows][k] f32 (16-byte aligned), outputs [rows][n].  A
 * pre-pass builds each row's activation records (RMS-normalised with gamma,
 * x·rsqrt(mean(x²)+eps)·γ, when gamma is not NULL); the weights are read once
 * per 8 rows.  k must be a multiple of 64 (K-quants: 256).
 *   rt_gemv_rows_<f>_f32     y = (norm)x · Wᵀ
 *   rt_gemv_rows_<f>_add_f32 y = res + x · Wᵀ   (y may alias res)
 *   rt_qkv_bias_rows_<f>_f32 q/k/v = (norm)x · W_{q,k,v}ᵀ + f32(bias); a NULL
 *                            weight skips that matrix (mixed-format Q/K/V:
 *                            one call per format)
 *   rt_fused_ffn_rows_<f>_f32 act = silu((norm)x·W_gᵀ) · ((norm)x·W_uᵀ) */
int rt_gemv_rows_q8_0_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q8_0_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q8_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q8_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q4_0_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q4_0_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q4_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q4_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q4k_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q4k_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q4k_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q4k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q6k_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q6k_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q6k_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q6k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q5_0_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q5_0_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q5_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q5_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q5k_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q5k_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q5k_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q5k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q4_0g_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q4_0g_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q4_0g_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q4_0g_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q4kg_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q4kg_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q4kg_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q4kg_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q5kg_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q5kg_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q5kg_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q5kg_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);
int rt_gemv_rows_q6kg_f32(rt_ctx* ctx, const void* weight, const float* x, const float* gamma,
                       float eps, float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_gemv_rows_q6kg_add_f32(rt_ctx* ctx, const void* weight, const float* x, const float* res,
                           float* y, uint32_t rows, uint32_t n, uint32_t k);
int rt_qkv_bias_rows_q6kg_f32(rt_ctx* ctx, const void* w_q, const void* w_k, const void* w_v,
                           const float* x, const float* gamma, float eps, float* q, float* k_out,
                           float* v, const uint16_t* bias_q, const uint16_t* bias_k,
                           const uint16_t* bias_v, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                           uint32_t k);
int rt_fused_ffn_rows_q6kg_f32(rt_ctx* ctx, const void* w_gate, const void* w_up, const float* x,
                            const float* gamma, float eps, float* act, uint32_t rows, uint32_t ff,
                            uint32_t k);

/* ───────────────────────── argmax ───────────────────────── */

/* greedy_argmax_f32 (crates/engine/src/sampler.rs:111-116) on the GPU:
 * Rust max_by semantics — the LAST index of the maximum wins ties; a NaN
 * compares Equal.  Writes one uint32 to result; n == 0 → 0. */
int rt_argmax_f32(rt_ctx* ctx, const float* input, uint32_t* result, uint32_t n);
/* dispatch.rs:1615-1631 → activation.metal:56-109 (f16 logits). */
int rt_argmax_f16(rt_ctx* ctx, const uint16_t* input, uint32_t* result, uint32_t n);

/* ───────────────────────── synthetic data (bench/tests) ─────────────────
 * Seeded, counter-based generators: w ~ N(0, std) quantised per block with
 * the documented quantisers; x ~ N(mean, std) in f32.  No reference
 * counterpart (the reference reads GGUF files). */
int rt_synth_normal_f32(rt_ctx* ctx, float* out, uint64_t n, uint64_t seed, float mean,
                        float std);
int rt_synth_normal_f16(rt_ctx* ctx, uint16_t* out, uint64_t n, uint64_t seed, float mean,
                        float std);
int rt_synth_q8_0(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);
int rt_synth_q4_0(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);
int rt_synth_q4k(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);
int rt_synth_q6k(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);
int rt_synth_q5_0(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);
int rt_synth_q5k(rt_ctx* ctx, void* out, uint64_t n_blocks, uint64_t seed, float std);

/* ───────────────────────── decode-step glue ─────────────────────────
 * The non-GEMV kernels of one decode step (forward.rs:1523-1771). */

/* dispatch.rs:177-200 → norm.metal:126-154: y = x·rsqrt(mean(x²)+eps)·γ per
 * row; y may alias x. */
int rt_rms_norm_f32_f32_f32g(rt_ctx* ctx, const float* x, float* y, const float* gamma, float eps,
                             uint32_t hidden, uint32_t num_rows);
/* dispatch.rs:945-971 → fused_rope.metal:17-56 (pairs (d, d+head_dim/2)). */
int rt_fused_rope_qk_f32(rt_ctx* ctx, float* q, float* k, uint32_t head_dim, uint32_t q_heads,
                         uint32_t kv_heads, uint32_t pos, float theta);
/* dispatch.rs:1183-1205 → activation.metal:30-45: cache[h][pos][d] = src[h][d]. */
int rt_kv_copy_to_cache_f32(rt_ctx* ctx, const float* src, float* dst, uint32_t pos,
                            uint32_t max_seq, uint32_t head_dim, uint32_t num_kv_heads);
/* dispatch.rs:1575-1612 → attention.metal:248-308 (GQA, scale 1/sqrt(hd)).
 * head_dim must be 64, 128 or 256. */
int rt_decode_attention_f32(rt_ctx* ctx, const float* q, const float* k, const float* v,
                            float* out, uint32_t batch, uint32_t kv_len, uint32_t num_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride);
/* New: fused_rope_qk_f32 + kv_copy_to_cache_f32 (k and v, at pos) +
 * decode_attention_f32 (kv_len = pos+1) in one launch; q/k/v are the raw
 * projections, the caches are [num_kv_heads][max_seq][head_dim]. */
int rt_decode_attention_rope_f32(rt_ctx* ctx, const float* q_raw, const float* k_raw,
                                 const float* v_raw, float* k_cache, float* v_cache, float* out,
                                 uint32_t pos, uint32_t max_seq, uint32_t num_heads,
                                 uint32_t num_kv_heads, uint32_t head_dim, float theta);
/* New: decode_attention_rope_f32 followed by gemv_q8_0_add_f32_f32in of the
 * output projection (forward.rs:1588-1619), x_io += W_o · attention(...).
 * When q_dim = num_heads·head_dim ≤ 1024 and the attention splits the KV
 * range in 2..8 parts, each split writes its unnormalised output and
 * (max, sum) and the projection merges them while staging its input (the
 * attention's own merge, without its extra memory round trips); otherwise
 * the two kernels run as in the unfused sequence.  w_o: [hidden, q_dim] Q8_0. */
int rt_decode_attention_rope_oproj_q8_0_f32(rt_ctx* ctx, const float* q_raw, const float* k_raw,
                                            const float* v_raw, float* k_cache, float* v_cache,
                                            const void* w_o, float* x_io, uint32_t pos,
                                            uint32_t max_seq, uint32_t num_heads,
                                            uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                            uint32_t hidden);
/* The same for Q4_K output projections (reference layout; the 7B Q4_K_M
 * models' attn_output), whose merging form stages q_dim ≤ 4096 in one round
 * of up to 1024 threads; w_o: [hidden, q_dim] Q4_K.  New: the reference runs
 * decode_attention_f32 then the Q4_K GEMV (forward.rs:1588-1619). */
int rt_decode_attention_rope_oproj_q4k_f32(rt_ctx* ctx, const float* q_raw, const float* k_raw,
                                           const float* v_raw, float* k_cache, float* v_cache,
                                           const void* w_o, float* x_io, uint32_t pos,
                                           uint32_t max_seq, uint32_t num_heads,
                                           uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                           uint32_t hidden);
/* The same for ggml-layout Q4_K output projections (upstream GGUF files). New. */
int rt_decode_attention_rope_oproj_q4kg_f32(rt_ctx* ctx, const float* q_raw, const float* k_raw,
                                            const float* v_raw, float* k_cache, float* v_cache,
                                            const void* w_o, float* x_io, uint32_t pos,
                                            uint32_t max_seq, uint32_t num_heads,
                                            uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                            uint32_t hidden);
/* Kernel launches enqueued on the context so far (graph capture included). New. */
uint64_t rt_launch_count(const rt_ctx* ctx);
/* Name of the kernel the context launched last ("" before the first launch;
 * valid until the next call on the context).  New: for profiles and
 * benchmarks that label a launch by the kernel the library chose. */
const char* rt_last_launch_name(const rt_ctx* ctx);
/* add_f16_into_f32 (dispatch.rs:316-330): acc[i] += f32(src[i]) for i < n
 * (the bias add of the separate-dispatch Q/K/V fallback, forward.rs:1561-1568). */
int rt_add_f16_into_f32(rt_ctx* ctx, const uint16_t* src, float* acc, uint32_t n);
/* ─────────────── batched verify / prefill (verify_draft's M-row path) ───────────────
 * The kernels between the GEMMs of verify_draft (forward.rs:2118-2309) on f32
 * activations [seq][dim]; the GEMMs are rt_gemm_<fmt>_f32. */
/* dispatch.rs:1660-1680 → activation.metal:211-227: x[s][i] += f32(bias[i]). */
int rt_add_bias_broadcast_f32(rt_ctx* ctx, float* x, const uint16_t* bias, uint32_t seq,
                              uint32_t dim);
/* dispatch.rs:1125-1150 → rope.metal:92-121: x [seq][num_heads][head_dim],
 * row s rotated at position start_pos + s. */
int rt_rope_batch_inplace_f32(rt_ctx* ctx, float* x, uint32_t head_dim, uint32_t num_heads,
                              uint32_t start_pos, float theta, uint32_t seq);
/* New: rt_rope_batch_inplace_f32 of q (num_heads) and k (num_kv_heads) and
 * rt_kv_write_batch_f32 of the rotated k and of v in one launch; q is rotated
 * in place, k and v are read only. */
int rt_rope_kv_write_batch_f32(rt_ctx* ctx, float* q, const float* k, const float* v,
                               float* k_cache, float* v_cache, uint32_t head_dim,
                               uint32_t num_heads, uint32_t num_kv_heads, uint32_t start_pos,
                               float theta, uint32_t seq, uint32_t max_seq);
/* KvCache::write_at (kv_cache.rs:132-150) for positions start_pos ..
 * start_pos+seq-1 (forward.rs:2216-2231): k, v [seq][num_kv_heads][head_dim]
 * → caches [num_kv_heads][max_seq][head_dim]. */
int rt_kv_write_batch_f32(rt_ctx* ctx, const float* k, const float* v, float* k_cache,
                          float* v_cache, uint32_t start_pos, uint32_t seq, uint32_t max_seq,
                          uint32_t head_dim, uint32_t num_kv_heads);
/* dispatch.rs:645-687 → attention.metal:36-160 (flash_attention_f16) on f32:
 * q, out [batch][q_len][num_heads][head_dim], caches [batch][num_kv_heads]
 * [kv_head_stride][head_dim], scale 1/sqrt(head_dim).  Query row r attends to
 * cache positions j < kv_len with j <= q_start + r.  q_start = 0 is the
 * reference kernel's mask (j <= r); verify_draft with history needs
 * q_start = kv_len - q_len (row r sits at absolute position q_start + r).
 * head_dim 64, 128 or 256; batch·q_len ≤ 65535. */
int rt_flash_attention_f32(rt_ctx* ctx, const float* q, const float* k, const float* v, float* out,
                           uint32_t batch, uint32_t q_len, uint32_t kv_len, uint32_t num_heads,
                           uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride,
                           uint32_t q_start);
/* dispatch.rs:57-75 → activation.metal:175-185 on f32: out = a + b (out may
 * alias a or b). */
int rt_add_f32(rt_ctx* ctx, const float* a, const float* b, float* out, uint32_t n);
/* dispatch.rs:35-55 → activation.metal:156-173: out = silu(gate)·up. */
int rt_silu_mul_f32(rt_ctx* ctx, const float* gate, const float* up, float* out, uint32_t n);
/* The per-row argmax of verify_draft (forward.rs:2283-2293), on the GPU:
 * result[r] = the first index of row r's maximum (strictly-greater scan from
 * −inf; NaN never wins; a row of −inf/NaN gives 0).  in [rows][n]. */
int rt_argmax_rows_first_f32(rt_ctx* ctx, const float* in, uint32_t* result, uint32_t rows,
                             uint32_t n);

/* New: out = dequant(table row *token) for a [vocab, k] table in the named
 * block format (reference or ggml layout, or plain f16 / f32 rows, as
 * token_embd.weight is stored); the token id is read from device memory
 * (forward.rs:1494-1505 dequantises the row on the CPU). */
int rt_embed_q8_0_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q4_0_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q4k_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q6k_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q5_0_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q5k_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q4_0g_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q4kg_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q5kg_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_q6kg_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_f16_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);
int rt_embed_f32_f32(rt_ctx* ctx, const void* table, const uint32_t* token, float* out,
                      uint32_t k);

/* New: rt_embed_<fmt>_f32 for `rows` tokens at once: out[r·k ..] = row of
 * tokens[r] (verify_draft embeds its sequence on the CPU, forward.rs:2142-2162). */
int rt_embed_rows_q8_0_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q4_0_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q4k_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q6k_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q5_0_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q5k_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q4_0g_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q4kg_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q5kg_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_q6kg_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_f16_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);
int rt_embed_rows_f32_f32(rt_ctx* ctx, const void* table, const uint32_t* tokens, float* out,
                         uint32_t k, uint32_t rows);

/* New: rms_norm_f32_f32_f32g(x → x̂) fused into the following GEMV's
 * activation staging (same arguments as the pair of calls, minus x̂). */
int rt_rms_norm_fused_qkv_bias_q8_0_f32(rt_ctx* ctx, const void* w_q, const void* w_k,
                                        const void* w_v, const float* x, const float* gamma,
                                        float eps, float* out_q, float* out_k, float* out_v,
                                        const uint16_t* bias_q, const uint16_t* bias_k,
                                        const uint16_t* bias_v, uint32_t q_dim, uint32_t kv_dim,
                                        uint32_t k);
int rt_rms_norm_fused_ffn_q8_0_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                                   const float* x, const float* gamma, float eps, float* act_out,
                                   uint32_t ff_dim, uint32_t k);
int rt_rms_norm_gemv_q8_0_f32in_f32out(rt_ctx* ctx, const void* weight, const float* x,
                                       const float* gamma, float eps, float* output, uint32_t m,
                                       uint32_t k);
/* New: a decode step's RMSNorm factor handed from the launch that produces
 * x to the norm-fused launch that consumes it.  The producing forms (down
 * projection + residual, attention + output projection + residual) also
 * write ssq[i] = Σ y² over output rows 4i..4i+3 (⌈m/4⌉ floats); the
 * consuming forms take Σx² as those nparts partial sums instead of reducing
 * x inside every workgroup (nparts ≤ 256; more: x is reduced as in the forms
 * above).  The partial sums must be those of the x passed.  Results equal the
 * forms without _ssq to f32 rounding of Σx². */
int rt_gemv_q8_0_add_f32_f32in_ssq(rt_ctx* ctx, const void* weight, const float* input,
                                   float* output, const float* residual, uint32_t m, uint32_t k,
                                   float* ssq);
int rt_decode_attention_rope_oproj_q8_0_f32_ssq(rt_ctx* ctx, const float* q_raw,
                                                const float* k_raw, const float* v_raw,
                                                float* k_cache, float* v_cache, const void* w_o,
                                                float* x_io, uint32_t pos, uint32_t max_seq,
                                                uint32_t num_heads, uint32_t num_kv_heads,
                                                uint32_t head_dim, float theta, uint32_t hidden,
                                                float* ssq);
int rt_rms_norm_fused_qkv_bias_q8_0_f32_ssq(rt_ctx* ctx, const void* w_q, const void* w_k,
                                            const void* w_v, const float* x, const float* gamma,
                                            float eps, float* out_q, float* out_k, float* out_v,
                                            const uint16_t* bias_q, const uint16_t* bias_k,
                                            const uint16_t* bias_v, uint32_t q_dim,
                                            uint32_t kv_dim, uint32_t k, const float* ssq,
                                            uint32_t nparts);
int rt_rms_norm_fused_ffn_q8_0_f32_ssq(rt_ctx* ctx, const void* w_gate, const void* w_up,
                                       const float* x, const float* gamma, float eps,
                                       float* act_out, uint32_t ff_dim, uint32_t k,
                                       const float* ssq, uint32_t nparts);
/* The same for the Q4_K_M projections: Q/K (Q4_K) + V (Q6_K) with biases
 * (k ≤ 8192), the Q4_K gate+up+SiLU, and a Q6_K GEMV (the LM head). */
int rt_rms_norm_fused_qkv_bias_q4k_q6k_f32(rt_ctx* ctx, const void* w_q, const void* w_k,
                                           const void* w_v, const float* x, const float* gamma,
                                           float eps, float* out_q, float* out_k, float* out_v,
                                           const uint16_t* bias_q, const uint16_t* bias_k,
                                           const uint16_t* bias_v, uint32_t q_dim,
                                           uint32_t kv_dim, uint32_t k);
int rt_rms_norm_fused_ffn_q4k_f32(rt_ctx* ctx, const void* w_gate, const void* w_up,
                                  const float* x, const float* gamma, float eps, float* act_out,
                                  uint32_t ff_dim, uint32_t k);
int rt_rms_norm_gemv_q6k_f32in_f32out(rt_ctx* ctx, const void* weight, const float* x,
                                      const float* gamma, float eps, float* output, uint32_t m,
                                      uint32_t k);

/* ───────────────────────── calibration (bench only) ─────────────────────────
 * Plain HBM streams of known size; no reference counterpart.  stream_read
 * reads `bytes` (multiple of 16) and writes one dword per wave to `sink`
 * (sink needs grid·4 dwords; pass sink_dwords); stream_copy copies `bytes`. */
int rt_stream_read(rt_ctx* ctx, const void* src, size_t bytes, uint32_t* sink,
                   size_t sink_dwords);
int rt_stream_copy(rt_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ───────────────────────── GGUF files ───────────────────────── */
/* The wire format in front of the path: crates/gguf (parser.rs:22-57,
 * types.rs:142-198) plus the engine's mmap loader (crates/engine/src/
 * loader.rs:124-218).  rt_gguf_open parses header, metadata and tensor
 * table of a GGUF v2/v3 file and maps it read-only; errors are the GgufError
 * variants above, with the message in rt_gguf_last_error().  Metadata value
 * types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
 * 9 array, 10 u64, 11 i64, 12 f64.  Tensor dtypes are GgufDtype ids. */
typedef struct rt_gguf rt_gguf;
int rt_gguf_open(const char* path, rt_gguf** out);
void rt_gguf_close(rt_gguf* g);
const char* rt_gguf_last_error(void);
uint32_t rt_gguf_version(const rt_gguf* g);
uint64_t rt_gguf_alignment(const rt_gguf* g);
/* absolute file offset of the (aligned) tensor data region */
uint64_t rt_gguf_data_offset(const rt_gguf* g);
uint64_t rt_gguf_tensor_count(const rt_gguf* g);
/* index of a tensor by name, -1 if absent */
int64_t rt_gguf_find_tensor(const rt_gguf* g, const char* name);
/* name, shape (up to 8 dims), dtype, offset within the data region, bytes */
int rt_gguf_tensor_info(const rt_gguf* g, uint64_t i, const char** name, uint32_t* n_dims,
                        uint64_t dims[8], uint32_t* dtype, uint64_t* offset, uint64_t* bytes);
/* host pointer to the tensor's bytes inside the mapping */
const void* rt_gguf_tensor_data(const rt_gguf* g, uint64_t i);
/* copies the tensor's bytes to device memory (dst_dev holds ≥ bytes) */
int rt_gguf_upload(rt_ctx* ctx, const rt_gguf* g, uint64_t i, void* dst_dev);
uint64_t rt_gguf_meta_count(const rt_gguf* g);
int64_t rt_gguf_find_meta(const rt_gguf* g, const char* key);
int rt_gguf_meta_info(const rt_gguf* g, uint64_t i, const char** key, uint32_t* type,
                      uint32_t* elem_type, uint64_t* count);
int rt_gguf_meta_int(const rt_gguf* g, uint64_t i, int64_t* out);
int rt_gguf_meta_float(const rt_gguf* g, uint64_t i, double* out);
const char* rt_gguf_meta_string(const rt_gguf* g, uint64_t i);
int rt_gguf_meta_array_numbers(const rt_gguf* g, uint64_t i, double* out, uint64_t max);
int rt_gguf_meta_array_string(const rt_gguf* g, uint64_t i, uint64_t k, const char** s,
                              uint64_t* len);

/* ───────────────────────── persistent decode step (new) ─────────────────────────
 * No counterpart in the reference, whose engine encodes one command buffer of
 * ~10 dispatches per layer (forward.rs:1470-1787).  One greedy decode step of
 * a Q8_0 Qwen2-shape model (head size 64) with the arithmetic of that
 * sequence, as ONE persistent launch (token embedding and every layer: RMSNorm
 * + Q/K/V + bias, RoPE + KV write + attention, O + residual, RMSNorm +
 * gate/up + SiLU, down + residual), then the norm-fused LM head and the
 * argmax (two more launches).  create() plans the step for one position `pos`
 * (kv_len = pos + 1) and allocates its activation buffers; run() enqueues it
 * (no allocation; capturable); status() flushes and reports a grid barrier
 * that timed out (the kernel bounds every wait) since the last status() call,
 * then clears the report: a run that timed out left an invalid token and
 * invalid activations, so check status() before using a token.  The token id is read from
 * *token and the greedy next token written back there. */
typedef struct rt_step rt_step;
typedef struct {
    const void *wq, *wk, *wv, *wo, *wg, *wu, *wd; /* Q8_0 [rows][k] */
    const uint16_t *bq, *bk, *bv;                  /* f16 biases */
    const float *attn_norm, *ffn_norm;
    float *k_cache, *v_cache;                      /* f32 [kv_heads][max_seq][head_dim] */
} rt_step_layer;
typedef struct {
    uint32_t layers, hidden, heads, kv_heads, head_dim, ff, vocab, max_seq;
    float eps, theta;
    const rt_step_layer* layer;
    const void* token_embd;  /* Q8_0 [vocab][hidden] */
    const void* lm_head;     /* Q8_0 [vocab][hidden] (may equal token_embd) */
    const float* output_norm;
    uint32_t* token;         /* device: the input token id; receives the next one */
    float* logits;           /* device: [vocab] */
} rt_step_model;
int rt_decode_step_q8_0_create(rt_ctx* ctx, const rt_step_model* model, uint32_t pos,
                               rt_step** out);
int rt_decode_step_run(rt_ctx* ctx, rt_step* step);
int rt_decode_step_status(rt_ctx* ctx, rt_step* step);
void rt_decode_step_destroy(rt_step* step);

#ifdef __cplusplus
}
#endif

#endif /* RUNIT_HIP_H */
