// runtime.cpp — host side of the C ABI declared in include/runit_hip.h.
//
// The context loads the prebuilt gfx950 code objects (lib/kernels/*.hsaco)
// with hipModuleLoad, resolves every kernel up front (the reference builds
// every pipeline state at MetalContext::new, context.rs:163-205), owns one
// HIP stream, and launches with hipModuleLaunchKernel.  Kernel entry points
// validate their arguments, pick a launch shape for the problem and enqueue;
// nothing synchronises until rt_flush (context.rs:289-296).
#include <hip/hip_runtime.h>
#include "rt_shared.h"
#include <dirent.h>
#include <dlfcn.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <array>
#include <vector>

#include "../../include/runit_hip.h"

namespace {

// Mirrors the kernel-side GemvArgs (rt_gemv.h); passed by value.
struct GemvArgs {
    const uint8_t* w[3];
    void* out[3];
    const void* aux[3];
    const void* x;
    uint32_t n[3];
    uint32_t nvrows;
    uint32_t K;
    uint32_t lpr;
    uint32_t ksw;
    uint32_t x_rec;
    const float* gamma;
    float eps;
    uint32_t xb_chunk;
    uint64_t row_bytes;
    uint32_t ksplit;
    uint32_t kc_units;
    float* part;
    uint32_t* counters;
    uint32_t cstride;
    const float* xml;
    uint32_t xnsp, xhd;
    uint32_t ls_rs;
    uint32_t ls_res;
    uint32_t ls_xcd;
    uint32_t blk0, nblk;
    uint32_t nx;
    float* ssq_out;        // Σy² per output row quad (for the next RMSNorm), or null
    const float* ssq_in;   // Σx² of x as ssq_n partial sums, or null
    uint32_t ssq_n;
};

constexpr uint32_t XREC_BYTES = 112;
constexpr uint32_t kAttnXMaxSplits = 8;  // splits the merging projection stages  // one activation record per 32 elements
// argmax: 256 workgroup states of 12 bytes, then the arrival counter
constexpr uint32_t kArgmaxWgs = 256;
constexpr uint32_t kOnePassMaxK = 8192;  // 512 threads × 4 slices × 4 elements
constexpr uint32_t kKSplitElems = 4096;  // K chunk of a split matrix-core launch
constexpr uint32_t kMaxSplitTiles = 256;  // tiles per workgroup of a split launch (kernel LDS)
constexpr size_t kAuxCounterOff = 4096;
constexpr size_t kAuxAttnOff = 8192;  // attention arrival counters
constexpr size_t kAuxBytes = 65536;
constexpr uint32_t kAttnCounters = (kAuxBytes - kAuxAttnOff) / 4;

const char* const kKernelNames[] = {
    "k_fill_u32", "k_decode_step_q8_0",
    "k_gemv_q8_0_f32_f32_r1", "k_gemv_q8_0_f32_f32_r2", "k_gemv_q8_0_attn_f32add_r1",
    "k_gemv_q4k_attn_f32add_r1", "k_gemv_q4kg_attn_f32add_r1",
    "k_gemv_q8_0_f32_f32add_r1", "k_gemv_q8_0_f32_f32add_r2",
    "k_gemv_q8_0_f32_f16_r1", "k_gemv_q8_0_f32_f16_r2",
    "k_gemv_q8_0_f16_f16_r1", "k_gemv_q8_0_f16_f16_r2",
    "k_gemv_q8_0_f16_f16add_r1", "k_gemv_q8_0_f16_f16add_r2",
    "k_gemv_q8_0_f16_f32add_r1", "k_gemv_q8_0_f16_f32add_r2",
    "k_qkv_q8_0_r1", "k_qkv_q8_0_r2",
    "k_qkv_bias_q8_0_r1", "k_qkv_bias_q8_0_r2",
    "k_ffn_q8_0_r1", "k_ffn_q8_0_r2",
    "k_gemv_q4_0_f32_f32_r1", "k_gemv_q4_0_f32_f32_r2",
    "k_gemv_q4_0_f32_f32add_r1", "k_gemv_q4_0_f32_f32add_r2",
    "k_gemv_q4_0_f32_f16_r1", "k_gemv_q4_0_f32_f16_r2",
    "k_gemv_q4_0_f16_f16_r1", "k_gemv_q4_0_f16_f16_r2",
    "k_gemv_q4_0_f16_f16add_r1", "k_gemv_q4_0_f16_f16add_r2",
    "k_qkv_bias_q4_0_r1", "k_qkv_bias_q4_0_r2",
    "k_ffn_q4_0_r1", "k_ffn_q4_0_r2",
    "k_gemv_q4k_f32_f32_r1", "k_gemv_q4k_f32_f32_r2",
    "k_gemv_q4k_f32_f32add_r1", "k_gemv_q4k_f32_f32add_r2",
    "k_gemv_q4k_f16_f16_r1", "k_gemv_q4k_f16_f16_r2",
    "k_gemv_q4k_f16_f16add_r1", "k_gemv_q4k_f16_f16add_r2",
    "k_gemv_q4k_f16_f32add_r1", "k_gemv_q4k_f16_f32add_r2",
    "k_ffn_q4k_r1", "k_ffn_q4k_r2",
    "k_gemv_q6k_f32_f32_r1", "k_gemv_q6k_f32_f32_r2",
    "k_gemv_q6k_f32_f32add_r1", "k_gemv_q6k_f32_f32add_r2",
    "k_gemv_q6k_f32_f16_r1", "k_gemv_q6k_f32_f16_r2",
    "k_gemv_q8_0_f32_f32_s1", "k_gemv_q8_0_f32_f32add_s1", "k_gemv_q8_0_f32_f16_s1",
    "k_gemv_q8_0_f16_f16_s1", "k_gemv_q8_0_f16_f16add_s1", "k_gemv_q8_0_f16_f32add_s1",
    "k_qkv_q8_0_s1", "k_qkv_bias_q8_0_s1", "k_ffn_q8_0_s1",
    "k_gemv_q4_0_f32_f32_s1", "k_gemv_q4_0_f32_f32add_s1", "k_gemv_q4_0_f32_f16_s1",
    "k_gemv_q4_0_f16_f16_s1", "k_gemv_q4_0_f16_f16add_s1", "k_qkv_bias_q4_0_s1", "k_ffn_q4_0_s1",
    "k_dequant_q8_0_f32", "k_dequant_q4_0_f32", "k_dequant_q4k_f32", "k_dequant_q4k_f16",
    "k_dequant_q6k_f32", "k_dequant_q5_0_f32", "k_dequant_q5k_f32",
    "k_dequant_q4_0g_f32", "k_dequant_q4kg_f32", "k_dequant_q5kg_f32", "k_dequant_q6kg_f32",
    "k_gemv_q4_0g_f32_f32_r1", "k_gemv_q4_0g_f32_f32_r2", "k_gemv_q4_0g_f32_f32add_r1",
    "k_gemv_q4_0g_f32_f32add_r2", "k_gemv_q4_0g_f32_f16_r1", "k_gemv_q4_0g_f32_f16_r2",
    "k_ffn_q4_0g_r1", "k_ffn_q4_0g_r2", "k_gemv_q4_0g_f32_f32_s1", "k_gemv_q4_0g_f32_f32add_s1",
    "k_gemv_q4_0g_f32_f16_s1", "k_ffn_q4_0g_s1",
    "k_gemv_q4kg_f32_f32_r1", "k_gemv_q4kg_f32_f32_r2", "k_gemv_q4kg_f32_f32add_r1",
    "k_gemv_q4kg_f32_f32add_r2", "k_gemv_q4kg_f32_f16_r1", "k_gemv_q4kg_f32_f16_r2",
    "k_ffn_q4kg_r1", "k_ffn_q4kg_r2",
    "k_gemv_q5kg_f32_f32_r1", "k_gemv_q5kg_f32_f32_r2", "k_gemv_q5kg_f32_f32add_r1",
    "k_gemv_q5kg_f32_f32add_r2", "k_gemv_q5kg_f32_f16_r1", "k_gemv_q5kg_f32_f16_r2",
    "k_ffn_q5kg_r1", "k_ffn_q5kg_r2",
    "k_gemv_q6kg_f32_f32_r1", "k_gemv_q6kg_f32_f32_r2", "k_gemv_q6kg_f32_f32add_r1",
    "k_gemv_q6kg_f32_f32add_r2", "k_gemv_q6kg_f32_f16_r1", "k_gemv_q6kg_f32_f16_r2",
    "k_gemv_q5_0_f32_f32_r1", "k_gemv_q5_0_f32_f32_r2",
    "k_gemv_q5_0_f32_f32add_r1", "k_gemv_q5_0_f32_f32add_r2",
    "k_gemv_q5_0_f32_f16_r1", "k_gemv_q5_0_f32_f16_r2",
    "k_qkv_bias_q5_0_r1", "k_qkv_bias_q5_0_r2", "k_ffn_q5_0_r1", "k_ffn_q5_0_r2",
    "k_gemv_q5_0_f32_f32_s1", "k_gemv_q5_0_f32_f32add_s1", "k_gemv_q5_0_f32_f16_s1",
    "k_qkv_bias_q5_0_s1", "k_ffn_q5_0_s1",
    "k_gemv_q5k_f32_f32_r1", "k_gemv_q5k_f32_f32_r2",
    "k_gemv_q5k_f32_f32add_r1", "k_gemv_q5k_f32_f32add_r2",
    "k_gemv_q5k_f32_f16_r1", "k_gemv_q5k_f32_f16_r2",
    "k_qkv_bias_q5k_r1", "k_qkv_bias_q5k_r2", "k_ffn_q5k_r1", "k_ffn_q5k_r2",
    "k_qkv_bias_q4k_r1", "k_qkv_bias_q4k_r2", "k_qkv_q4k_r1", "k_qkv_q4k_r2",
    "k_qkv_bias_q4kg_r1", "k_qkv_bias_q4kg_r2", "k_qkv_q4kg_r1", "k_qkv_q4kg_r2",
    "k_qkv2_bias_q4k_q6k_r1", "k_qkv2_q4k_q6k_r1", "k_qkv2_bias_q4kg_q6kg_r1", "k_qkv2_q4kg_q6kg_r1",
    "k_argmax_f32", "k_argmax_f16",
    "k_synth_normal_f32", "k_synth_normal_f16", "k_synth_q8_0", "k_synth_q4_0",
    "k_synth_q4k", "k_synth_q6k", "k_synth_q5_0", "k_synth_q5k",
    "k_stream_read", "k_stream_copy",
    "k_act_limbs_f32", "k_act_limbs_f32_q40", "k_act_limbs_f16", "k_act_limbs_f16_q40",
    "k_rms_norm_f32g", "k_rope_qk_f32", "k_kv_copy_f32",
    "k_decode_attention_f32_hd64", "k_decode_attention_f32_hd128", "k_decode_attention_f32_hd256",
    "k_attn_mq_f32_hd64", "k_attn_mq_f32_hd128", "k_attn_mq_f32_hd256",
    "k_attn_rope_f32_hd64", "k_attn_rope_f32_hd128", "k_attn_rope_f32_hd256",
    "k_attn_rope_w_f32_hd64", "k_attn_rope_w_f32_hd128",
    "k_add_f16_into_f32", "k_ssq_quads", "k_add_bias_broadcast_f32", "k_rope_batch_f32", "k_kv_write_batch_f32",
    "k_add_f32", "k_silu_mul_f32", "k_argmax_rows_first_f32", "k_rope_kv_write_batch_f32",
    "k_embed_q8_0_f32", "k_embed_q4_0_f32", "k_embed_q4k_f32", "k_embed_q6k_f32", "k_embed_q5_0_f32", "k_embed_q5k_f32", "k_embed_q4_0g_f32", "k_embed_q4kg_f32", "k_embed_q5kg_f32", "k_embed_q6kg_f32", "k_embed_f16_f32", "k_embed_f32_f32",
    "k_gemm_split_sum", "k_gemm_split_sum_ep", "k_gemm_split_sum_ep3", "k_gemm_split_sum_qkv_rope", "k_gemm_xh_prep1s_mg1",
    "k_gemm_xh_prep1s_mg2", "k_gemm_xh_prep1s_mg4", "k_gemm_xh_prep1sn_mg1", "k_gemm_xh_prep1sn_mg2",
    "k_gemm_xh_prep1sn_mg4", "k_gemm_xh_prep1a_mg1", "k_gemm_xh_prep1a_mg2", "k_gemm_xh_prep1a_mg4", "k_gemm_xh_prep1n_mg1", "k_gemm_xh_prep1n_mg2",
    "k_gemm_xh_prep1n_mg4", "k_gemm_xh_prep1_mg1", "k_gemm_xh_prep1_mg2", "k_gemm_xh_prep1_mg4", "k_gemm_x_prep_mg1", "k_gemm_x_prep_mg2", "k_gemm_x_prep_mg4", "k_gemm_x_prep_mg8",
    "k_gemm_q8_0_mg1_ct1", "k_gemm_q8_0_mg2_ct1", "k_gemm_q8_0_mg4_ct1", "k_gemm_q8_0_mg8_ct1",
    "k_gemm_q8_0_mg1_ct2", "k_gemm_q8_0_mg2_ct2", "k_gemm_q8_0_mg4_ct2", "k_gemm_q8_0_mg8_ct2",
    "k_gemm2_q8_0_mg1", "k_gemm2_q8_0_mg2", "k_gemm2_q8_0_mg4", "k_gemm2_q8_0_mg8",
    "k_gemm2_q4_0_mg1", "k_gemm2_q4_0_mg2", "k_gemm2_q4_0_mg4", "k_gemm2_q4_0_mg8",
    "k_gemm2_q4k_mg1", "k_gemm2_q4k_mg2", "k_gemm2_q4k_mg4", "k_gemm2_q4k_mg8",
    "k_gemm2_q8_0_mg1_w8", "k_gemm2_q8_0_mg2_w8", "k_gemm2_q8_0_mg4_w8", "k_gemm2_q8_0_mg8_w8",
    "k_gemm2_q4_0_mg1_w8", "k_gemm2_q4_0_mg2_w8", "k_gemm2_q4_0_mg4_w8", "k_gemm2_q4_0_mg8_w8",
    "k_gemm2_q4k_mg1_w8", "k_gemm2_q4k_mg2_w8", "k_gemm2_q4k_mg4_w8", "k_gemm2_q4k_mg8_w8",
    "k_gemm2_q4kg_mg1", "k_gemm2_q4kg_mg2", "k_gemm2_q4kg_mg4", "k_gemm2_q4kg_mg8", "k_gemm2_q4kg_mg1_w8", "k_gemm2_q4kg_mg2_w8", "k_gemm2_q4kg_mg4_w8", "k_gemm2_q4kg_mg8_w8",
    "k_gemm2_q4_0g_mg1", "k_gemm2_q4_0g_mg2", "k_gemm2_q4_0g_mg4", "k_gemm2_q4_0g_mg8", "k_gemm2_q4_0g_mg1_w8", "k_gemm2_q4_0g_mg2_w8", "k_gemm2_q4_0g_mg4_w8", "k_gemm2_q4_0g_mg8_w8",
    "k_gemm2_q5_0_mg1", "k_gemm2_q5_0_mg2", "k_gemm2_q5_0_mg4", "k_gemm2_q5_0_mg8", "k_gemm2_q5_0_mg1_w8", "k_gemm2_q5_0_mg2_w8", "k_gemm2_q5_0_mg4_w8", "k_gemm2_q5_0_mg8_w8",
    "k_gemm2_q5k_mg1", "k_gemm2_q5k_mg2", "k_gemm2_q5k_mg4", "k_gemm2_q5k_mg8", "k_gemm2_q5k_mg1_w8", "k_gemm2_q5k_mg2_w8", "k_gemm2_q5k_mg4_w8", "k_gemm2_q5k_mg8_w8",
    "k_gemm2_q5kg_mg1", "k_gemm2_q5kg_mg2", "k_gemm2_q5kg_mg4", "k_gemm2_q5kg_mg8", "k_gemm2_q5kg_mg1_w8", "k_gemm2_q5kg_mg2_w8", "k_gemm2_q5kg_mg4_w8", "k_gemm2_q5kg_mg8_w8",
    "k_gemm2_q6k_mg1", "k_gemm2_q6k_mg2", "k_gemm2_q6k_mg4",
    "k_gemm2_q6kg_mg1", "k_gemm2_q6kg_mg2", "k_gemm2_q6kg_mg4",
    "k_gemm3_q8_0_mg1", "k_gemm3_q8_0_mg1_w8", "k_gemm3_q8_0_mg2", "k_gemm3_q8_0_mg2_w8",
    "k_gemm3_q8_0_mg4", "k_gemm3_q8_0_mg4_w8", "k_gemm3_q8_0_mg4_w16", "k_gemm3_q4k_mg4_w16", "k_gemm3_q4kg_mg4_w16",
    "k_gemm3_q5k_mg4_w16", "k_gemm3_q5kg_mg4_w16", "k_gemm3_q4_0_mg1", "k_gemm3_q4_0_mg1_w8",
    "k_gemm3_q4_0_mg2", "k_gemm3_q4_0_mg2_w8", "k_gemm3_q4_0_mg4", "k_gemm3_q4_0_mg4_w8",
    "k_gemm3_q4k_mg1", "k_gemm3_q4k_mg1_w8", "k_gemm3_q4k_mg2", "k_gemm3_q4k_mg2_w8",
    "k_gemm3_q4k_mg4", "k_gemm3_q4k_mg4_w8", "k_gemm3_q4kg_mg1", "k_gemm3_q4kg_mg1_w8",
    "k_gemm3_q4kg_mg2", "k_gemm3_q4kg_mg2_w8", "k_gemm3_q4kg_mg4", "k_gemm3_q4kg_mg4_w8",
    "k_gemm3_q4_0g_mg1", "k_gemm3_q4_0g_mg1_w8", "k_gemm3_q4_0g_mg2", "k_gemm3_q4_0g_mg2_w8",
    "k_gemm3_q4_0g_mg4", "k_gemm3_q4_0g_mg4_w8", "k_gemm3_q5_0_mg1", "k_gemm3_q5_0_mg1_w8",
    "k_gemm3_q5_0_mg2", "k_gemm3_q5_0_mg2_w8", "k_gemm3_q5_0_mg4", "k_gemm3_q5_0_mg4_w8",
    "k_gemm3_q5k_mg1", "k_gemm3_q5k_mg1_w8", "k_gemm3_q5k_mg2", "k_gemm3_q5k_mg2_w8",
    "k_gemm3_q5k_mg4", "k_gemm3_q5k_mg4_w8", "k_gemm3_q5kg_mg1", "k_gemm3_q5kg_mg1_w8",
    "k_gemm3_q5kg_mg2", "k_gemm3_q5kg_mg2_w8", "k_gemm3_q5kg_mg4", "k_gemm3_q5kg_mg4_w8",
    "k_gemm3_q6k_mg1", "k_gemm3_q6k_mg2", "k_gemm3_q6k_mg4", "k_gemm3_q6kg_mg1", "k_gemm3_q6kg_mg2",
    "k_gemm3_q6kg_mg4", "k_gemm3_q6k_mg1_w8", "k_gemm3_q6kg_mg1_w8", "k_gemm3_q6k_mg2_w8", "k_gemm3_q6k_mg4_w8", "k_gemm3_q6kg_mg2_w8",
    "k_gemm3_q6kg_mg4_w8",
    "k_gemm_xh_prep_mg1", "k_gemm_xh_prep_mg2", "k_gemm_xh_prep_mg4",
};

// Kernels of the LDS-streamed GEMV body: <base>_ls<NI>, NI = 1..3 global→LDS
// loads of 1 KB per row chunk.
const char* const kLsBases[] = {
    "k_gemv_q8_0_f32_f32", "k_gemv_q8_0_f32_f32add", "k_gemv_q8_0_f32_f16", "k_qkv_bias_q8_0",
    "k_ffn_q8_0", "k_gemv_q4_0_f32_f32", "k_gemv_q4_0_f32_f32add", "k_qkv_bias_q4_0",
    "k_ffn_q4_0", "k_gemv_q4k_f32_f32", "k_gemv_q4k_f32_f32add", "k_ffn_q4k",
    "k_gemv_q6k_f32_f32", "k_gemv_q6k_f32_f32add", "k_gemv_q6kg_f32_f32", "k_gemv_q6kg_f32_f32add",
    "k_gemv_q5_0_f32_f32", "k_gemv_q5_0_f32_f32add", "k_ffn_q5_0",
    "k_gemv_q5k_f32_f32", "k_gemv_q5k_f32_f32add", "k_ffn_q5k",
    "k_gemv_q4_0g_f32_f32", "k_gemv_q4_0g_f32_f32add", "k_ffn_q4_0g",
    "k_gemv_q4kg_f32_f32", "k_gemv_q4kg_f32_f32add", "k_ffn_q4kg",
    "k_gemv_q5kg_f32_f32", "k_gemv_q5kg_f32_f32add", "k_ffn_q5kg",
};
// Kernels of the workgroup-local K split: <base>_lsk1.
const char* const kLskBases[] = {
    "k_ffn_q4_0", "k_ffn_q4_0g", "k_ffn_q4k", "k_ffn_q4kg", "k_ffn_q5_0", "k_ffn_q5k", "k_ffn_q5kg",
    "k_ffn_q8_0", "k_gemv_q4_0_f32_f32", "k_gemv_q4_0_f32_f32add", "k_gemv_q4_0g_f32_f32",
    "k_gemv_q4_0g_f32_f32add", "k_gemv_q4k_f32_f32", "k_gemv_q4k_f32_f32add", "k_gemv_q4kg_f32_f32",
    "k_gemv_q4kg_f32_f32add", "k_gemv_q5_0_f32_f32", "k_gemv_q5_0_f32_f32add", "k_gemv_q5k_f32_f32",
    "k_gemv_q5k_f32_f32add", "k_gemv_q5kg_f32_f32", "k_gemv_q5kg_f32_f32add",
    "k_gemv_q6k_f32_f32add", "k_gemv_q6kg_f32_f32add", "k_gemv_q8_0_f32_f32",
    "k_gemv_q8_0_f32_f32add",
};
// VALU small-launch kernels: <base>_vs, and with the norm in the body <base>_vsn.
const char* const kVsBases[] = {"k_gemv_q8_0_f32_f32", "k_gemv_q8_0_f32_f32add", "k_qkv_bias_q8_0",
                                "k_ffn_q8_0"};
const char* const kVsnBases[] = {"k_gemv_q8_0_f32_f32", "k_qkv_bias_q8_0", "k_ffn_q8_0"};
// Small-launch kernels: <base>_sm1, <base>_sm2.
const char* const kSmBases[] = {
    "k_gemv_q8_0_f32_f32", "k_gemv_q8_0_f32_f32add", "k_qkv_bias_q8_0", "k_ffn_q8_0",
    "k_gemv_q8_0_attn_f32add", "k_gemv_q4k_f32_f32", "k_gemv_q4k_f32_f32add",
};
// Multi-row kernels: <base>_x8 for each format's four epilogues.
const char* const kRowsFmts[] = {"q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k",
                                 "q4_0g", "q4kg", "q5kg", "q6kg"};
// Kernels with a VALU-dot twin <base>_ls<NI>v (the dot-form A/B).
const char* const kLsValuBases[] = {"k_ffn_q4k", "k_gemv_q6k_f32_f32"};
constexpr uint32_t kLsMaxNI = 3;
constexpr uint32_t kVsMaxQuadsPerCu = 2;  // VALU small-launch body: row quads per CU (at most)
constexpr uint32_t kMaxSsqParts = 256;    // Σx² partial sums a norm-fused staging reads (at most)
constexpr int kLsDecline = -1;
constexpr uint32_t kLsThreads = 256;
constexpr uint32_t kLsRowPad = 48;      // LDS row stride = NI KB + pad (bank spread)
constexpr uint32_t kPrepassK = 8192;    // K from which x is converted once by a pre-pass

struct Fmt {
    uint32_t blk_el, blk_bytes, unit_el;  // unit_el: elements per lane unit (v_dot4 path)
    uint32_t unroll;  // UNR template constant of the format's kernels
    const char* name;
    const Fmt* single;  // single-block-unit fallback for odd block counts
    uint32_t mq_unit_el = 0;  // matrix-core path unit, if it differs from unit_el
    bool q40perm = false;     // activation records in the reference Q4_0 order
    uint32_t ls_chunk = 3072;  // LDS-streamed K split: chunk bytes per row (at most)
    bool xpair = false;        // units of two whole records (the K-split body can hold their limbs)
    uint32_t mq_units() const { return mq_unit_el ? mq_unit_el : unit_el; }
};
// Q8_0 / Q4_0 kernels take two blocks per unit (4-byte-aligned loads); rows
// with an odd number of blocks use the one-block "_s1" kernels.
constexpr Fmt kQ8_0S{32, 34, 32, 2, "Q8_0", nullptr};
constexpr Fmt kQ4_0S{32, 18, 32, 4, "Q4_0", nullptr, 0, true};
constexpr Fmt kQ8_0{32, 34, 64, 1, "Q8_0", &kQ8_0S, 0, false, 3072, true};
constexpr Fmt kQ4_0{32, 18, 64, 2, "Q4_0", &kQ4_0S, 0, true, 3072, true};
constexpr Fmt kQ4K{256, 144, 64, 1, "Q4_K", nullptr, 0, false, 3072, true};
constexpr Fmt kQ6K{256, 210, 64, 1, "Q6_K", nullptr, 256};  // matrix-core: one block per lane
constexpr Fmt kQ5_0S{32, 22, 32, 4, "Q5_0", nullptr};
constexpr Fmt kQ5_0{32, 22, 64, 2, "Q5_0", &kQ5_0S, 0, false, 3072, true};
constexpr Fmt kQ5K{256, 176, 64, 1, "Q5_K", nullptr, 0, false, 2048, true};  // (2 KB chunks: 18.0 against 19.4 µs for 3 KB)
// ggml layouts (upstream GGUF files)
constexpr Fmt kQ4_0GS{32, 18, 32, 4, "Q4_0 (ggml)", nullptr};
constexpr Fmt kQ4_0G{32, 18, 64, 2, "Q4_0 (ggml)", &kQ4_0GS, 0, false, 3072, true};
constexpr Fmt kQ4KG{256, 144, 64, 1, "Q4_K (ggml)", nullptr, 0, false, 3072, true};
constexpr Fmt kQ5KG{256, 176, 64, 1, "Q5_K (ggml)", nullptr, 0, false, 2048, true};
constexpr Fmt kQ6KG{256, 210, 64, 1, "Q6_K (ggml)", nullptr, 256};
// Q6_K on the matrix-core path with 64-element lane units (small launches:
// four times the lanes of the one-super-block-per-lane form)
constexpr Fmt kQ6KU{256, 210, 64, 1, "Q6_K", nullptr};
constexpr Fmt kQ6KGU{256, 210, 64, 1, "Q6_K (ggml)", nullptr};

thread_local std::string g_global_error = "no error";

}  // namespace

struct Plan {
    uint32_t T, TL, rpl;
};

struct rt_ctx {
    int device = 0;
    std::vector<hipModule_t> modules;  // the loaded code objects
    hipStream_t stream = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns;
    int cu_count = 0;
    size_t max_lds = 65536;
    std::string err = "no error";
    bool capturing = false;
    bool gemm_direct = false;   // RUNIT_GEMM_DIRECT: force the unstaged GEMM kernel (tests)
    bool ksplit_enabled = true; // RUNIT_GEMV_KSPLIT=0: long K via the pre-pass instead (tests)
    // Workspace for activation records built by the long-K pre-pass; grows on
    // demand (stream-ordered, so one buffer serves every launch).
    void* ws = nullptr;
    size_t ws_bytes = 0;
    std::unordered_map<std::string, uint32_t> occ;  // occupancy cache
    void* part = nullptr;  // K-split GEMV partial sums
    size_t part_bytes = 0;
    void* attn_out = nullptr;  // attention output between the two launches of
    size_t attn_out_bytes = 0;  // the unmerged attention + o_proj sequence
    bool ls_enabled = true;      // RUNIT_GEMV_LS=0: the per-lane-load matrix-core body instead
    bool sm_enabled = true;      // RUNIT_GEMV_SM=0: no small-launch body (A/B)
    uint64_t launches = 0;       // kernel launches enqueued so far (rt_launch_count)
    const char* last_name = "";  // the last launched kernel (rt_last_launch_name)
    bool gemv_valu = false;      // RUNIT_GEMV_VALU=1: VALU-dot twins of the LDS body (A/B)
    uint32_t ls_min_items = 16;  // RUNIT_GEMV_LS_MIN: items per CU from which the LDS body runs
    bool gemm_set = true;  // RUNIT_GEMM_SET=0: rt_gemm_set_f32 as separate launches (A/B)
    uint32_t gemm_set_min = 1;  // RUNIT_GEMM_SET_MIN: rows above which a set takes the shared f16 form
    bool gemm_multi = true;     // RUNIT_GEMM_MULTI=0: a set's GEMMs one launch each (A/B)
    bool gemm_nb4 = true;       // RUNIT_GEMM_NB4=0: no 4-block-stage 8-row variant (A/B)
    bool gemm_bigm_split = true;  // RUNIT_GEMM_BIGM_SPLIT=0: 256+ rows split as short launches (A/B)
    uint32_t gemm_bigm_chunks = 2;  // RUNIT_GEMM_BIGM_CHUNKS: activation chunks from which that holds
    bool gemm_set_sum1 = true;  // RUNIT_GEMM_SET_SUM1=0: a set's split sums one launch per matrix (A/B)
    bool gemm_block = true;     // RUNIT_GEMM_BLOCK=0: rt_gemm_ffn_block_f32 as three sets (A/B)
    bool attn_fold = true;      // RUNIT_ATTN_FOLD=0: rt_gemm_attn_ffn_block_f32 merges in the attention (A/B)
    bool gemm_rope = true;      // RUNIT_GEMM_ROPE=0: rt_gemm_qkv_rope_f32 with a separate RoPE launch (A/B)
    uint32_t gemm_block_silu_min = 64;  // RUNIT_GEMM_BLOCK_SILU_MIN: rows from which the block
                                        // sums the SiLU pair in the down preparation
    bool gemm_sum_kernel = true;  // RUNIT_GEMM_SUM_KERNEL=0: K splits meet in the GEMM (arrival counters)
    uint32_t gemm_splits = 0;    // RUNIT_GEMM_SPLITS=n: the f16 GEMM's K splits forced (A/B)
    bool attn_w = true;          // RUNIT_ATTN_W=0: the token's RoPE attention on attn_split (A/B)
    bool attn_mq = true;         // RUNIT_ATTN_MQ=0: multi-query attention on attn_split per row (A/B)
    uint32_t attn_mq_nsp = 0, attn_mq_w = 0;  // probe: forced ranges / waves (0: planned)
    // RUNIT_ATTN_MQ_MIN / _FOLD_MIN: column-group pairs up to which the
    // per-row kernel runs (rt_flash_attention_f32 / rt_gemm_attn_ffn_block_f32)
    uint32_t attn_mq_min = 8, attn_mq_fold_min = 0;
    uint32_t gemm_f16_min = 4;   // RUNIT_GEMM_F16_MIN: batches above this many rows run the f16 form
    uint32_t gemm_f16_min_q6 = 1;  // RUNIT_GEMM_F16_MIN_Q6: the same for Q6_K
    bool lsk_whole = true;       // RUNIT_GEMV_LSK_WHOLE=0: whole-K launches off the K-split body (A/B)
    bool vs_enabled = true;      // RUNIT_GEMV_VS=0: no VALU small-launch body (A/B)
    uint32_t vs_max_q = kVsMaxQuadsPerCu;  // RUNIT_GEMV_VS_MAXQ: row quads per CU up to which it runs
    bool gemm_w16 = true;        // RUNIT_GEMM_W16=0: no 256-row tiles (A/B)
    int gemm_q6w8 = 7;           // RUNIT_GEMM_Q6W8: Q6_K f16 form on 128-row tiles at MG = 4 / 2 / 1 (bits 0 / 1 / 2)
    bool gemm_f16 = true;        // RUNIT_GEMM_F16=0: the int8 limb form of the staged GEMM at every M
    // Small per-context device buffer: argmax range states + arrival counter
    // (the counter is reset by the kernel that consumes it).
    void* aux = nullptr;
    // Arrival counters of split launches: the aux buffer's counter area, or
    // the scratch array's inside a no-allocation call.
    uint32_t* counters = nullptr;
    // This device's copy of the code object's `scratch` array (address taken
    // from the loaded module at context creation), and whether a
    // no-allocation call is running: then the workspace buffers point into
    // the scratch array and never grow.
    uint8_t* scratch = nullptr;
    bool noalloc = false;
    // workspace buffers replaced by larger ones (freed with the context)
    std::vector<void*> retired;
};
struct rt_event { hipEvent_t ev; };
struct rt_graph { hipGraph_t graph; hipGraphExec_t exec; };
struct rt_step {
    void* phases = nullptr;  // StepPhase[nph] (device)
    uint32_t nph = 0;
    void* sync = nullptr;    // StepSync (device)
    void* acts = nullptr;    // the step's activation buffers (device)
    uint32_t grid = 0;
    size_t lds = 0;
    // after the persistent launch: RMSNorm + LM head, argmax
    const void* lm_head = nullptr;
    const float* final_norm = nullptr;
    const float* x_final = nullptr;
    float* logits = nullptr;
    uint32_t* token = nullptr;
    uint32_t vocab = 0, hidden = 0;
    float eps = 0.0f;
};

namespace {

int fail(rt_ctx* c, int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf; else g_global_error = buf;
    return code;
}

int hip_fail(rt_ctx* c, hipError_t e, const char* what) {
    return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: %s", what, hipGetErrorString(e));
}

// lib/kernels/ next to the host library: one code object per kernel unit
std::string default_code_object_path() {
    Dl_info info;
    if (dladdr((void*)&rt_ctx_create, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t s = p.find_last_of('/');
        return (s == std::string::npos ? std::string(".") : p.substr(0, s)) + "/kernels";
    }
    return "kernels";
}

// The code objects of a path: every *.hsaco of a directory (sorted), or the
// one file named.
std::vector<std::string> code_object_files(const std::string& path) {
    std::vector<std::string> files;
    if (DIR* d = opendir(path.c_str())) {
        while (dirent* e = readdir(d)) {
            const std::string n = e->d_name;
            if (n.size() > 6 && n.compare(n.size() - 6, 6, ".hsaco") == 0) files.push_back(path + "/" + n);
        }
        closedir(d);
        std::sort(files.begin(), files.end());
    } else {
        files.push_back(path);
    }
    return files;
}

int launch(rt_ctx* c, const char* name, dim3 grid, dim3 block, size_t lds, void** params) {
    auto it = c->fns.find(name);
    if (it == c->fns.end())
        return fail(c, RT_ERR_PIPELINE_NOT_FOUND, "pipeline function '%s' not found in code object",
                    name);
    hipError_t e = hipModuleLaunchKernel(it->second, grid.x, grid.y, grid.z, block.x, block.y,
                                         block.z, (unsigned)lds, c->stream, params, nullptr);
    if (e != hipSuccess) return hip_fail(c, e, name);
    ++c->launches;
    c->last_name = it->first.c_str();
    return RT_OK;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Resident workgroups per CU of a kernel at a block size and dynamic LDS
// size (cached per context).
uint32_t occupancy(rt_ctx* c, const char* name, uint32_t threads, size_t lds) {
    const std::string key = std::string(name) + "/" + std::to_string(threads) + "/" +
                            std::to_string(lds);
    auto hit = c->occ.find(key);
    if (hit != c->occ.end()) return hit->second;
    auto it = c->fns.find(name);
    int n = 0;
    if (it == c->fns.end() ||
        hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, it->second, (int)threads, lds) !=
            hipSuccess || n < 1)
        n = 1;
    c->occ[key] = (uint32_t)n;
    return (uint32_t)n;
}

// Launch plan for one GEMV-family call.
//   T   threads per workgroup (256, or 512 when K is long so the activation
//       staging is shared by more lanes);
//   TL  threads per row group: the smallest power of two ≥ 16 that covers a
//       row in ≤ 2 unrolled steps with ≥ 85% busy lanes (row groups wider
//       than a wave reduce across waves through LDS);
//   rows per lane group: 2 (kernel suffix _r2) when that still leaves ≥ 2
//       workgroups per CU, else 1 (_r1) to spread small-N problems wider.
Plan plan_gemv(const rt_ctx* c, const Fmt& f, uint32_t nvrows, uint32_t K, bool paired) {
    const uint32_t units = K / f.unit_el;
    Plan p{};
    p.T = (K / 32 >= 256) ? 512 : 256;
    p.TL = 0;
    for (uint32_t tl = 16; tl <= p.T; tl *= 2) {
        const uint32_t steps = (units + tl - 1) / tl;
        const double eff = (double)units / (double)(steps * tl);
        if (steps <= 2 * f.unroll && eff >= 0.85) {
            p.TL = tl;
            break;
        }
    }
    if (!p.TL) {
        double best = -1.0;
        for (uint32_t tl = 16; tl <= p.T; tl *= 2) {
            const uint32_t steps = (units + tl - 1) / tl;
            const double eff = (double)units / (double)(steps * tl);
            if (eff > best + 1e-9) {
                best = eff;
                p.TL = tl;
            }
        }
    }
    const uint32_t groups = p.T / p.TL;
    const uint32_t r2 = paired ? 4 : 2;
    const uint32_t wgs_r2 = (nvrows + groups * r2 - 1) / (groups * r2);
    p.rpl = (wgs_r2 >= (uint32_t)(2 * c->cu_count)) ? 2 : 1;
    return p;
}

// Grows a context buffer to `need` bytes (not during graph capture).
int ensure_buf(rt_ctx* c, void*& buf, size_t& bytes, size_t need, const char* who) {
    if (need <= bytes) return RT_OK;
    if (c->noalloc)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: needs %zu bytes of scratch, the no-allocation "
                    "entry point has %zu",
                    who, need, bytes);
    if (c->capturing)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: workspace must be sized before graph capture", who);
    if (buf) {
        // the old buffer stays allocated until the context is destroyed: a
        // graph captured before this growth holds its address in its kernel
        // arguments and may still be replayed
        c->retired.push_back(buf);
        buf = nullptr;
        bytes = 0;
    }
    hipError_t e = hipMalloc(&buf, need);
    if (e != hipSuccess) return hip_fail(c, e, "workspace hipMalloc");
    bytes = need;
    return RT_OK;
}
// The activation workspace (pre-pass records, normalised x, GEMM operands,
// attention partials) ...
int ensure_ws(rt_ctx* c, size_t need, const char* who) {
    return ensure_buf(c, c->ws, c->ws_bytes, need, who);
}
// ... and, separately, the partial sums of K-split GEMVs, whose activations
// may live in the workspace.
int ensure_part(rt_ctx* c, size_t need, const char* who) {
    return ensure_buf(c, c->part, c->part_bytes, need, who);
}

bool has_ls_kernel(const rt_ctx* c, const char* kname) {
    return c->fns.count(std::string(kname) + "_ls1") != 0;
}

// LDS-streamed matrix-core launch (rt_gemv_ls.h).  Items are row quads of
// one K chunk; a chunk's rows are read with NI ≤ 3 coalesced 1 KB loads
// each, so rows longer than 3 KB (or K beyond one staging pass) are split
// into S chunks whose partial sums meet in the workspace.  Returns 1 when the
// shape does not suit the body (kLsDecline: the caller takes the other bodies).
// Workgroup-local K split (rt_gemv_ls.h, *_lsk1): every K chunk of a row
// quad in one workgroup, 1 KB row chunks, the whole K's activation records in
// LDS; the chunks' partial sums meet in LDS.
int gemv_launch_lsk(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a, bool whole = false) {
    char name[96];
    snprintf(name, sizeof name, "%s_lsk1", kname);
    if (!c->fns.count(name)) return kLsDecline;
    // lane units of this body: the format's 64-element units (Q6_K too,
    // whose matrix-core unit is a whole super-block)
    const uint32_t ue = f.unit_el;
    const uint32_t units = a.K / ue;
    const uint32_t gu = f.blk_el > ue ? f.blk_el / ue : 1;
    const uint64_t unum = (uint64_t)ue * f.blk_bytes;  // unit bytes × blk_el
    uint32_t cap = (uint32_t)((1024 - 15) * (uint64_t)f.blk_el / unum);
    cap -= cap % gu;
    if (cap == 0) return kLsDecline;
    uint32_t S = (units + cap - 1) / cap;
    uint32_t kc = (units + S - 1) / S;
    kc = (kc + gu - 1) / gu * gu;
    S = (units + kc - 1) / kc;
    const uint32_t nq = (a.nvrows + 3) / 4;
    // A whole-K launch takes this body only where each wave keeps one chunk
    // (16 waves a multiple of S) of ≤ 2 steps of 16 units, whose activation
    // limbs it then holds in registers (formats with two-record units)
    if (whole && !(f.xpair && 16 % S == 0 && kc <= 32)) return kLsDecline;
    // Taken where the whole K's activation records stay small (≤ 32 KB, K ≤
    // 9,362: the 0.5B model's down projection, 896×4864, runs 1.3 µs faster
    // than with the K split through memory) and the units suit 1024-thread
    // workgroups; longer K (the 7B down projections) keeps the split through
    // memory, whose workgroups stage only their own chunk.
    // Q6_K: the 7B down projection (K = 18944, 66 KB of records) too — the
    // K split through memory costs it ~3 µs of hand-off at the end
    const size_t rec_cap = f.mq_unit_el == 256 ? 80 * 1024 : 32 * 1024;
    if ((size_t)(a.K / 32) * XREC_BYTES > rec_cap) return kLsDecline;
    const uint32_t t = 1024;
    const uint32_t nwv = t / 64;
    a.ksplit = S;
    a.kc_units = kc;
    a.ls_rs = 1024 + kLsRowPad;
    const size_t xbytes = (size_t)(a.K / 32) * XREC_BYTES;
    uint32_t nwg = 0, occ = 1;
    size_t lds = 0;
    for (int it = 0; it < 3; ++it) {  // workgroups ↔ result buffer size
        const uint32_t g = nwg ? nwg : std::min<uint32_t>(nq, (uint32_t)c->cu_count);
        const uint32_t nql = (nq + g - 1) / g;
        lds = xbytes + (size_t)nql * S * 16 + (size_t)nwv * 4 * a.ls_rs;
        if (lds > c->max_lds) return kLsDecline;
        occ = occupancy(c, name, t, lds);
        const uint32_t want = std::min<uint32_t>(nq, (uint32_t)c->cu_count * occ);
        if (want == g && nwg) break;
        nwg = want;
    }
    const uint32_t nql = (nq + nwg - 1) / nwg;
    a.ls_res = nql * S;
    lds = xbytes + (size_t)a.ls_res * 16 + (size_t)nwv * 4 * a.ls_rs;
    if (lds > c->max_lds) return kLsDecline;
    void* params[] = {&a};
    return launch(c, name, dim3(nwg), dim3(t), lds, params);
}

int gemv_launch_ls(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a) {
    const uint32_t ue = f.mq_units();
    const uint32_t units_total = a.K / ue;
    const uint32_t gu = f.blk_el > ue ? f.blk_el / ue : 1;  // units per whole block
    const uint32_t ubytes_num = ue * f.blk_bytes;           // unit bytes × blk_el
    auto chunk_bytes = [&](uint32_t u) { return (uint64_t)u * ubytes_num / f.blk_el; };
    const uint32_t max_recs = 4 * kLsThreads / 8;  // one staging pass
    uint32_t kc = units_total, S = 1, NI = 0;
    const uint64_t rb = chunk_bytes(units_total);
    if (rb + 15 <= kLsMaxNI * 1024 && (a.x_rec || a.gamma || a.K / 32 <= max_recs)) {
        NI = (uint32_t)((rb + 15 + 1023) / 1024);
    } else {
        if (a.x_rec || a.gamma || !c->ksplit_enabled) return kLsDecline;
        // chunks of ≤ f.ls_chunk bytes (3 KB, NI ≤ 3; Q5_K 2 KB), a whole
        // number of blocks, ≤ one staging pass (the 7B down projections:
        // Q6_K 21.5 → 19.9 µs, Q4_0 15.2 → 14.5 µs with 3 KB against 2 KB
        // chunks; 1 KB chunks are slower still)
        const uint32_t chunk = f.ls_chunk;
        uint32_t cap = (uint32_t)((chunk - 15) * (uint64_t)f.blk_el / ubytes_num);
        cap = std::min<uint32_t>(cap, max_recs * 32 / ue);
        cap -= cap % gu;
        if (cap == 0) return kLsDecline;
        S = (units_total + cap - 1) / cap;
        kc = (units_total + S - 1) / S;
        kc = (kc + gu - 1) / gu * gu;
        S = (units_total + kc - 1) / kc;
        NI = (uint32_t)((chunk_bytes(kc) + 15 + 1023) / 1024);
        if (NI > kLsMaxNI) return kLsDecline;
    }
    const uint32_t nq = (a.nvrows + 3) / 4;
    // Whole-K launches of ≥ 16 row quads per CU (the 7B FFNs) on the
    // K-split body: every workgroup owns nq / nwg whole quads, its waves
    // take (quad, 1 KB chunk) items, so waves differ by at most one 4 KB
    // item (dealt whole quads of 8 KB left 30% of the 7B FFN's waves a third
    // item), and the activation limbs stay in registers.  Q4_K FFN 2×18944
    // ×3584: 21.0 → 18.3 µs, Q4_0: 19.5 → 17.3 µs.
    if (S == 1 && c->lsk_whole && (uint64_t)nq >= (uint64_t)c->cu_count * c->ls_min_items) {
        const int st = gemv_launch_lsk(c, kname, f, a, true);
        if (st != kLsDecline) return st;
    }
    if (S > 1 && !a.gamma) {
        const int st = gemv_launch_lsk(c, kname, f, a);
        if (st != kLsDecline) return st;
    }
    a.ksplit = S;
    a.kc_units = kc;
    a.ls_rs = NI * 1024 + kLsRowPad;
    // The body pays off from ~16 items (row quads × K chunks) per CU: the
    // 7B FFN / down / LM-head launches; launches with fewer items (the QKV
    // and attention projections, the 0.5B model's GEMVs) run faster on the
    // matrix-core body, whose per-lane loads start streaming sooner.
    if ((uint64_t)nq * S < (uint64_t)c->cu_count * c->ls_min_items) return kLsDecline;
    // buffer sizes address each matrix with 32-bit offsets
    if ((uint64_t)a.nvrows * a.row_bytes + 16 >= (1ull << 31)) return kLsDecline;
    char name[96];
    snprintf(name, sizeof name, "%s_ls%u", kname, NI);
    if (c->gemv_valu && c->fns.count(std::string(name) + "v")) strcat(name, "v");
    // Block size: the one with the most resident waves per CU (larger
    // blocks share one copy of the activation records), one round of
    // resident workgroups, result buffers sized to the items per wave.
    const uint32_t tmax = f.mq_unit_el == 256 ? 256 : 1024;  // Q6_K: register-heavy units
    const size_t xbytes = (size_t)kc * ue / 32 * XREC_BYTES;
    uint32_t bt = 0, bg = 0, bres = 0, bwaves = 0;
    size_t blds = 0;
    for (uint32_t t = 256; t <= tmax; t *= 2) {
        const uint32_t nwv = t / 64;
        uint32_t res = 16, g = 0, occ = 0;
        size_t lds = 0;
        for (int it = 0; it < 4; ++it) {  // result capacity ↔ grid size
            lds = xbytes + (size_t)nwv * res * 16 + (size_t)nwv * 4 * a.ls_rs;
            if (lds > c->max_lds) break;
            occ = occupancy(c, name, t, lds);
            g = std::max<uint32_t>(1, (uint32_t)c->cu_count * occ / S);
            g = std::min<uint32_t>(g, (nq + nwv - 1) / nwv);
            const uint32_t per = (nq + g * nwv - 1) / (g * nwv);
            const uint32_t need = std::min<uint32_t>(64, (per + 15) / 16 * 16);
            if (need == res) break;
            res = need;
        }
        if (lds > c->max_lds || g == 0) continue;
        g = std::max<uint32_t>(g, (nq + nwv * res - 1) / (nwv * res));  // ≤ res items per wave
        const uint32_t waves = std::min<uint32_t>(occ * nwv, g * nwv * S / std::max(1, c->cu_count));
        if (waves > bwaves || (waves == bwaves && t > bt)) {
            bt = t; bg = g; bres = res; bwaves = waves; blds = lds;
        }
    }
    if (!bt) return kLsDecline;
    a.ls_res = bres;
    a.ls_xcd = 1;
    if (S > 1) {
        if (nq > kAttnCounters)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: %u row quads exceed %u",
                        kname, nq, kAttnCounters);
        const int st = ensure_part(c, (size_t)S * a.nvrows * sizeof(float), kname);
        if (st != RT_OK) return st;
        a.part = (float*)c->part;
        a.counters = c->counters;
        a.cstride = 32;
        while (a.cstride > 1 && (size_t)nq * a.cstride > kAttnCounters) a.cstride >>= 1;
    }
    void* params[] = {&a};
    return launch(c, name, dim3(bg * S), dim3(bt), blds, params);
}

// Small-launch body (rt_gemv_ls.h, *_sm<NI>): whole K in one staging pass,
// rows of ≤ 2 KB read with coalesced 1 KB loads, about one row quad per wave
// (256-thread workgroups).  Taken for launches of at most kSmMaxQuadsPerCu
// row quads per CU (the 0.5B model's Q/K/V, O and gate+up launches: 72, 56
// and 608 workgroups), where the chain before the first dot, not the weight
// stream, bounds the launch.
constexpr uint32_t kSmThreads = 256;
constexpr uint32_t kSmMaxQuadsPerCu = 12;
int gemv_launch_sm(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a) {
    const uint64_t rb = a.row_bytes;
    const uint32_t NI = (uint32_t)((rb + 15 + 1023) / 1024);
    if (NI > 2) return kLsDecline;
    const uint32_t nxb = a.K / 32;
    // one staging pass of ≤ 4 slices per thread (a merged attention input: one)
    if (nxb * 8 > (a.xnsp ? 1u : 4u) * kSmThreads) return kLsDecline;
    if (a.K % f.mq_units() != 0 || a.x_rec) return kLsDecline;
    const uint32_t nq = (a.nvrows + 3) / 4;
    if (nq > (uint64_t)c->cu_count * kSmMaxQuadsPerCu) return kLsDecline;
    char name[96];
    snprintf(name, sizeof name, "%s_sm%u", kname, NI);
    if (!c->fns.count(name)) return kLsDecline;
    a.ksplit = 1;
    a.kc_units = a.K / f.mq_units();
    a.ls_rs = NI * 1024 + kLsRowPad;
    const uint32_t nwv = kSmThreads / 64;
    const size_t lds = (size_t)nxb * XREC_BYTES + (size_t)nwv * 4 * a.ls_rs;
    if (lds > c->max_lds) return kLsDecline;
    const uint32_t occ = std::max<uint32_t>(1, occupancy(c, name, kSmThreads, lds));
    const uint32_t grid = std::min<uint32_t>((nq + nwv - 1) / nwv, (uint32_t)c->cu_count * occ);
    void* params[] = {&a};
    return launch(c, name, dim3(grid), dim3(kSmThreads), lds, params);
}

// VALU small-launch body (rt_gemv_vs.h, *_vs / *_vsn): Q8_0, whole K, f32
// activations (no merged attention input), a lane per (row, 32-element
// block), ⌈K/32/16⌉ waves per row quad, the norm in the body for K ≤ 1024.
// Taken for launches of at most kVsMaxQuadsPerCu row quads per CU: the 0.5B
// model's norm-fused Q/K/V (1152×896: 4.07 → 3.65 µs) and down + residual
// (896×4864: 5.64 → 4.02 µs).  Its per-lane 34-byte block loads and
// per-lane activation reads cost more than they save on larger launches
// (0.5B norm-fused gate+up 2×4864×896: 5.57 → 11.1 µs).
int gemv_launch_vs(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a) {
    // (a merged attention input stays on the small-launch body: merging 8
    // splits per lane made the 0.5B attention + O pair 8.9 → 9.1 µs)
    if (f.blk_bytes != 34 || f.blk_el != 32 || a.x_rec || a.xnsp || a.nx > 1) return kLsDecline;
    if (a.gamma && a.K > 1024) return kLsDecline;
    const uint32_t nb = a.K / 32;
    const uint32_t wpq = (nb + 15) / 16;
    if (wpq > 16) return kLsDecline;  // (K ≤ 8192: the quad's waves in one workgroup)
    const uint32_t nq = (a.nvrows + 3) / 4;
    if (nq > (uint64_t)c->cu_count * c->vs_max_q) return kLsDecline;
    char name[96];
    snprintf(name, sizeof name, "%s_%s", kname, a.gamma ? "vsn" : "vs");
    if (!c->fns.count(name)) return kLsDecline;
    // quads per workgroup: enough workgroups for every CU, ≤ 1024 threads
    const uint32_t qmax = 16 / wpq;
    const uint32_t qpw = std::max<uint32_t>(
        1, std::min<uint32_t>(qmax, (nq + (uint32_t)c->cu_count - 1) / (uint32_t)c->cu_count));
    const uint32_t grid = (nq + qpw - 1) / qpw;
    void* params[] = {&a};
    return launch(c, name, dim3(grid), dim3(qpw * wpq * 64), 0, params);
}

int gemv_launch(rt_ctx* c, const char* kname, const Fmt& fmt, GemvArgs a, bool x_f16,
                bool paired = false) {
    const bool single = fmt.single && (a.K % fmt.unit_el) != 0;
    const Fmt& f = single ? *fmt.single : fmt;
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (a.K == 0 || a.K % f.blk_el != 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: k=%u must be a positive multiple of %u (%s)",
                    kname, a.K, f.blk_el, f.name);
    if (a.nvrows == 0) return RT_OK;
    if (!a.x || !a.out[0] || !a.w[0])
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    if (!aligned(a.x, x_f16 ? 8 : 16))
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: input must be %d-byte aligned", kname,
                    x_f16 ? 8 : 16);
    a.row_bytes = (uint64_t)(a.K / f.blk_el) * f.blk_bytes;
    if (c->vs_enabled && !x_f16 && a.nblk == 0) {
        const int st = gemv_launch_vs(c, kname, f, a);
        if (st != kLsDecline) return st;
    }
    if (c->sm_enabled && !single && !x_f16 && a.nx <= 1 && a.nblk == 0) {
        const int st = gemv_launch_sm(c, kname, f, a);
        if (st != kLsDecline) return st;
    }
    if (c->ls_enabled && !single && !x_f16 && !a.xnsp && has_ls_kernel(c, kname)) {
        const int st = gemv_launch_ls(c, kname, f, a);
        if (st != kLsDecline) return st;
    }
    const uint32_t nxb = a.K / 32;
    const bool mq_shape = !single;
    const uint32_t mq_el = f.mq_units();
    const uint32_t units = a.K / mq_el;
    // Matrix-core launches stage x in one pass of ≤ 4 slices of 4 elements
    // per thread (K ≤ 8192 at 512 threads).  Longer K is split over
    // workgroups in chunks of kKSplitElems, each staged in one pass; the
    // partial sums meet in the workspace.
    uint32_t S = 1, kcu = units;
    if (mq_shape && c->ksplit_enabled && !a.x_rec && !a.gamma && !a.xnsp && a.K > kOnePassMaxK) {
        kcu = kKSplitElems / mq_el;
        S = (units + kcu - 1) / kcu;
    }
    a.ksplit = S;
    a.kc_units = kcu;
    if (S == 1 && !a.x_rec && !a.gamma && !a.xnsp &&
        (a.K >= kPrepassK || (mq_shape && a.K > kOnePassMaxK))) {
        // convert the activations once into the context workspace
        const size_t need = (size_t)nxb * XREC_BYTES;
        const int st0 = ensure_ws(c, need, kname);
        if (st0 != RT_OK) return st0;
        const bool q40 = f.q40perm;
        const char* pk = x_f16 ? (q40 ? "k_act_limbs_f16_q40" : "k_act_limbs_f16")
                               : (q40 ? "k_act_limbs_f32_q40" : "k_act_limbs_f32");
        const void* xin = a.x;
        void* xout = c->ws;
        uint32_t nx = nxb;
        void* pp[] = {&xin, &xout, &nx};
        const uint32_t pgrid = (nxb * 8 + 255) / 256;
        int st = launch(c, pk, dim3(pgrid), dim3(256), 0, pp);
        if (st != RT_OK) return st;
        a.x = c->ws;
        a.x_rec = 1;
    }
    const size_t red_bytes = 16 * 2 * 4 * sizeof(float);  // [waves ≤ 16][rows ≤ 2][4]
    const size_t lds_cap = std::min<size_t>(c->max_lds, 80 * 1024) - red_bytes;
    // records staged per workgroup: the K chunk (split), else all of K if it
    // fits, else LDS-sized chunks (v_dot4 path)
    const uint32_t recs = S > 1 ? kcu * mq_el / 32 : nxb;
    uint32_t chunk = (uint32_t)(lds_cap / XREC_BYTES) & ~7u;
    if (chunk >= recs) chunk = recs;
    const bool mq = mq_shape && chunk == recs;
    a.xb_chunk = mq ? nxb : chunk;  // the kernel takes the matrix-core body when ≥ K/32
    const size_t lds = (size_t)chunk * XREC_BYTES + red_bytes;
    Plan p;
    uint32_t rows_per_wg;
    uint32_t resident;
    if (mq) {
        // Matrix-core path: a wave covers RQ quads of 4 rows, 16 lanes per
        // row; persistent grid of `gpc` workgroups per CU.
        p = Plan{256, 16, 1};
        if (!a.x_rec && recs * 8 > 4 * p.T) p.T = 512;  // one staging pass
        // large whole-K launches of the two-items-in-flight formats (4- and
        // 5-bit): one 1024-thread workgroup per CU, whose 16 waves issue
        // their activation loads before any weight load of the CU.  (Q8_0
        // and Q6_K keep one item in flight per wave and run slower so; Q6_K's
        // ~240-register kernels are built for 512 threads.)
        const bool one_item = f.blk_bytes == 34 || mq_el == 256;
        if (S == 1 && a.K >= 2048 && !one_item && !a.xnsp) p.T = 1024;
        // a merging projection stages its whole input in one slice round
        if (a.xnsp)
            while (p.T < nxb * 8 && p.T < 1024) p.T *= 2;
        // split K over the waves of a workgroup while the split waves still
        // fit in the resident waves (latency-bound small problems; a split
        // past that leaves a second round of workgroups as a tail)
        const uint32_t nwaves = p.T / 64;
        const uint32_t quads = (a.nvrows + 4 * p.rpl - 1) / (4 * p.rpl);
        const uint32_t nsteps = (kcu + 15) / 16;
        const uint32_t resident_waves = (uint32_t)c->cu_count * 16;
        uint32_t ksw = 1;
        while (ksw < nwaves && quads * S * ksw * 2 <= resident_waves && ksw * 2 <= nsteps) ksw *= 2;
        a.ksw = ksw;
        rows_per_wg = (nwaves / ksw) * 4 * p.rpl;
        resident = 4;
        // never more than the kernel's occupancy allows (registers / LDS)
        char rn[96];
        snprintf(rn, sizeof rn, "%s_r%u", kname, p.rpl);
        resident = std::max<uint32_t>(1, std::min(resident, occupancy(c, rn, p.T, lds)));
        if (S > 1) {
            const uint32_t ntiles = (a.nvrows + rows_per_wg - 1) / rows_per_wg;
            if (ntiles > kAttnCounters)
                return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: %u row tiles exceed %u",
                            kname, ntiles, kAttnCounters);
            const int st = ensure_part(c, (size_t)S * a.nvrows * sizeof(float), kname);
            if (st != RT_OK) return st;
            a.part = (float*)c->part;
            a.counters = c->counters;
            // one 128-byte line per tile's counter while they fit: arrivals on
            // one line serialise (≈11 ns each) at the end of the kernel
            a.cstride = 32;
            while (a.cstride > 1 && (size_t)ntiles * a.cstride > kAttnCounters) a.cstride >>= 1;
        }
    } else {
        // chunked (long-K) and single-block kernels: one row (FFN: one gate/up
        // pair) per row group
        p = plan_gemv(c, f, a.nvrows, a.K, paired);
        p.rpl = 1;
        rows_per_wg = (p.T / p.TL) * (paired ? 2 * p.rpl : p.rpl);
        resident = std::min<uint32_t>(2048 / p.T, (uint32_t)(160 * 1024 / lds));
        resident = std::max<uint32_t>(resident, 1);
    }
    a.lpr = p.TL;
    const uint32_t ntiles = (a.nvrows + rows_per_wg - 1) / rows_per_wg;
    // persistent grid with the same number of tiles per workgroup: the
    // fewest rounds the resident capacity allows, spread evenly (a grid of
    // `cap` with ntiles slightly above it would leave most workgroups idle
    // while a few run a second tile)
    // (with a K split, each of the S chunks gets the same number of
    // workgroups, and the grid is a multiple of S)
    const uint32_t cap = (uint32_t)c->cu_count * resident;
    const uint32_t rounds = (ntiles * S + cap - 1) / cap;
    const uint32_t grid = (ntiles + rounds - 1) / rounds * S;
    if (S > 1 && rounds > kMaxSplitTiles)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: %u tiles per workgroup exceed %u",
                    kname, rounds, kMaxSplitTiles);
    char name[96];
    if (single)
        snprintf(name, sizeof name, "%s_s1", kname);
    else
        snprintf(name, sizeof name, "%s_r%u", kname, p.rpl);
    void* params[] = {&a};
    return launch(c, name, dim3(grid), dim3(p.T), lds, params);
}

// ─────────────── multi-row launches (batched verify / prefill) ───────────────
//
// rows activation rows [rows][K] through one weight pass per 8 rows: a
// pre-pass builds every row's limb records (RMS-normalised first when gamma
// is given) into the workspace, then the <kname>_x8 kernel runs the
// matrix-core body with up to 8 rows per launch, whole K per workgroup when
// 8 rows' records fit in LDS, else split over workgroups (partials in `part`).
constexpr uint32_t kRowsNX = 8;  // activation rows per launch (the kernels' NX)

int gemv_rows_launch(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a, uint32_t rows,
                     const float* gamma, float eps) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    const uint32_t mq_el = f.mq_units();
    if (a.K == 0 || a.K % f.blk_el != 0 || a.K % mq_el != 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s rows: k=%u must be a positive multiple of %u (%s)",
                    kname, a.K, std::max(f.blk_el, mq_el), f.name);
    if (rows == 0 || a.nvrows == 0) return RT_OK;
    if (!a.x || !a.out[0])
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s rows: null buffer", kname);
    if (!aligned(a.x, 16) || (gamma && !aligned(gamma, 16)))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s rows: input must be 16-byte aligned",
                    kname);
    char name[96];
    snprintf(name, sizeof name, "%s_x%u", kname, kRowsNX);
    if (!c->fns.count(name))
        return fail(c, RT_ERR_PIPELINE_NOT_FOUND, "pipeline function '%s' not found", name);
    a.row_bytes = (uint64_t)(a.K / f.blk_el) * f.blk_bytes;
    const uint32_t nxb = a.K / 32;
    // rows of at most 1024 elements are staged (and normalised) by the
    // kernel itself, one wave per row; longer ones by the pre-pass
    const bool in_kernel = nxb * 8 <= 4 * 64 && !f.q40perm;
    int st = RT_OK;
    if (!in_kernel) st = ensure_ws(c, (size_t)rows * nxb * XREC_BYTES, kname);
    if (st != RT_OK) return st;
    if (in_kernel) {
        a.gamma = gamma;
        a.eps = eps;
    } else {
        const char* pk = f.q40perm ? "k_act_limbs_rows_f32_q40" : "k_act_limbs_rows_f32";
        const void* xin = a.x;
        void* xout = c->ws;
        uint32_t K = a.K;
        void* pp[] = {&xin, (void*)&gamma, &eps, &K, &xout};
        st = launch(c, pk, dim3(rows), dim3(256), 0, pp);
        if (st != RT_OK) return st;
        a.x_rec = 1;
        a.gamma = nullptr;
    }
    // K chunk per workgroup: whole K when 8 rows' records fit in LDS
    const uint32_t T = 512, nwaves = T / 64;
    const size_t red_bytes = (size_t)16 * kRowsNX * 4 * sizeof(float);
    const size_t lds_cap = std::min<size_t>(c->max_lds, 160 * 1024) - red_bytes;
    const uint32_t units = a.K / mq_el, rec_per_unit = mq_el / 32;
    uint32_t kcu = units;
    if ((size_t)kRowsNX * nxb * XREC_BYTES > lds_cap) {
        if (!c->ksplit_enabled)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s rows: k=%u needs a K split",
                        kname, a.K);
        kcu = (uint32_t)(lds_cap / ((size_t)kRowsNX * XREC_BYTES * rec_per_unit));
    }
    const uint32_t S = (units + kcu - 1) / kcu;
    kcu = (units + S - 1) / S;
    a.ksplit = S;
    a.kc_units = kcu;
    a.xb_chunk = nxb;  // whole-K form of the kernel (matrix-core body)
    const size_t lds = (size_t)kRowsNX * kcu * rec_per_unit * XREC_BYTES + red_bytes;
    const uint32_t quads = (a.nvrows + 3) / 4;
    const uint32_t nsteps = (kcu + 15) / 16;
    const uint32_t resident_waves = (uint32_t)c->cu_count * 16;
    uint32_t ksw = 1;
    while (ksw < nwaves && quads * S * ksw * 2 <= resident_waves && ksw * 2 <= nsteps) ksw *= 2;
    a.ksw = ksw;
    a.lpr = 16;
    const uint32_t rows_per_wg = (nwaves / ksw) * 4;
    const uint32_t resident = std::max<uint32_t>(1, std::min<uint32_t>(4, occupancy(c, name, T, lds)));
    const uint32_t ntiles = (a.nvrows + rows_per_wg - 1) / rows_per_wg;
    const uint32_t cap = (uint32_t)c->cu_count * resident;
    const uint32_t rounds = (ntiles * S + cap - 1) / cap;
    const uint32_t grid = (ntiles + rounds - 1) / rounds * S;
    if (S > 1) {
        if (ntiles > kAttnCounters)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s rows: %u row tiles exceed %u",
                        kname, ntiles, kAttnCounters);
        if (rounds > kMaxSplitTiles)
            return fail(c, RT_ERR_DISPATCH,
                        "kernel dispatch error: %s rows: %u tiles per workgroup exceed %u", kname,
                        rounds, kMaxSplitTiles);
        st = ensure_part(c, (size_t)S * kRowsNX * a.nvrows * sizeof(float), kname);
        if (st != RT_OK) return st;
        a.part = (float*)c->part;
        a.counters = c->counters;
        a.cstride = 32;
        while (a.cstride > 1 && (size_t)ntiles * a.cstride > kAttnCounters) a.cstride >>= 1;
    }
    // outputs (and residual) of row r0 of a matrix lie r0 of its lengths on
    const bool ffn = strstr(kname, "k_ffn_") == kname;
    const bool qkv = strstr(kname, "k_qkv") == kname;
    auto len = [&](uint32_t mat) -> size_t {
        return ffn ? a.nvrows / 2 : qkv ? a.n[mat] : a.nvrows;
    };
    for (uint32_t r0 = 0; r0 < rows; r0 += kRowsNX) {
        GemvArgs b = a;
        b.nx = std::min(kRowsNX, rows - r0);
        b.x = in_kernel ? (const void*)((const float*)a.x + (size_t)r0 * a.K)
                        : (const void*)((const uint8_t*)c->ws + (size_t)r0 * nxb * XREC_BYTES);
        for (uint32_t mat = 0; mat < 3; ++mat)
            if (b.out[mat]) b.out[mat] = (float*)b.out[mat] + r0 * len(mat);
        if (!qkv && b.aux[0]) b.aux[0] = (const float*)b.aux[0] + r0 * len(0);  // residual
        void* params[] = {&b};
        st = launch(c, name, dim3(grid), dim3(T), lds, params);
        if (st != RT_OK) return st;
    }
    return RT_OK;
}

// Multi-row entry points per format: plain (optionally RMS-normalised input:
// the LM head after the final norm), + residual (y may alias res), Q/K/V
// (+ bias; a null weight skips that matrix, so a mixed-format Q/K/V takes
// two calls) and gate+up+SiLU (optionally normalised input).
static int rows_qkv(rt_ctx* c, const char* kname, const Fmt& f, const void* wq, const void* wk,
                    const void* wv, const float* x, const float* gamma, float eps, float* oq,
                    float* ok, float* ov, const uint16_t* bq, const uint16_t* bk,
                    const uint16_t* bv, uint32_t rows, uint32_t q_dim, uint32_t kv_dim,
                    uint32_t k) {
    GemvArgs a{};
    uint32_t nm = 0;
    const void* w3[3] = {wq, wk, wv};
    float* o3[3] = {oq, ok, ov};
    const uint16_t* b3[3] = {bq, bk, bv};
    const uint32_t n3[3] = {q_dim, kv_dim, kv_dim};
    for (int i = 0; i < 3; ++i) {
        if (!w3[i]) continue;
        if (!o3[i] || !b3[i])
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s rows: null buffer", kname);
        a.w[nm] = (const uint8_t*)w3[i];
        a.out[nm] = o3[i];
        a.aux[nm] = b3[i];
        a.n[nm] = n3[i];
        ++nm;
    }
    if (nm == 0) return RT_OK;
    a.x = x;
    a.nvrows = a.n[0] + a.n[1] + a.n[2];
    a.K = k;
    return gemv_rows_launch(c, kname, f, a, rows, gamma, eps);
}
#define RT_ROWS_ENTRIES(FN, FMT)                                                                 \
    int rt_gemv_rows_##FN##_f32(rt_ctx* c, const void* w, const float* x, const float* gamma,      \
                                float eps, float* y, uint32_t rows, uint32_t n, uint32_t k) {      \
        if (!w) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemv_rows: null weight");  \
        return gemv_rows_launch(c, "k_gemv_" #FN "_f32_f32", FMT, plain_args(w, x, y, nullptr, n, k), \
                                rows, gamma, eps);                                                 \
    }                                                                                              \
    int rt_gemv_rows_##FN##_add_f32(rt_ctx* c, const void* w, const float* x, const float* res,    \
                                    float* y, uint32_t rows, uint32_t n, uint32_t k) {             \
        if (!w || !res)                                                                            \
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemv_rows_add: null buffer");  \
        return gemv_rows_launch(c, "k_gemv_" #FN "_f32_f32add", FMT, plain_args(w, x, y, res, n, k), \
                                rows, nullptr, 0.0f);                                              \
    }                                                                                              \
    int rt_qkv_bias_rows_##FN##_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,     \
                                    const float* x, const float* gamma, float eps, float* q,       \
                                    float* k_out, float* v, const uint16_t* bq,                    \
                                    const uint16_t* bk, const uint16_t* bv, uint32_t rows,         \
                                    uint32_t q_dim, uint32_t kv_dim, uint32_t k) {                 \
        return rows_qkv(c, "k_qkv_bias_" #FN, FMT, wq, wk, wv, x, gamma, eps, q, k_out, v, bq, bk,   \
                        bv, rows, q_dim, kv_dim, k);                                               \
    }                                                                                              \
    int rt_fused_ffn_rows_##FN##_f32(rt_ctx* c, const void* wg, const void* wu, const float* x,    \
                                     const float* gamma, float eps, float* act, uint32_t rows,     \
                                     uint32_t ff, uint32_t k) {                                    \
        if (!wg || !wu)                                                                            \
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: ffn_rows: null weight");       \
        GemvArgs a{};                                                                              \
        a.w[0] = (const uint8_t*)wg; a.w[1] = (const uint8_t*)wu;                                  \
        a.out[0] = act;                                                                            \
        a.x = x;                                                                                   \
        a.n[0] = ff; a.n[1] = ff;                                                                  \
        a.nvrows = 2 * ff;                                                                         \
        a.K = k;                                                                                   \
        return gemv_rows_launch(c, "k_ffn_" #FN, FMT, a, rows, gamma, eps);                        \
    }

GemvArgs plain_args(const void* w, const void* x, void* y, const void* aux, uint32_t m,
                    uint32_t k) {
    GemvArgs a{};
    a.w[0] = (const uint8_t*)w;
    a.out[0] = y;
    a.aux[0] = aux;
    a.x = x;
    a.n[0] = m;
    a.nvrows = m;
    a.K = k;
    return a;
}

int gemv_plain(rt_ctx* c, const char* kname, const Fmt& f, const void* w, const void* x,
               void* y, const void* res, bool need_res, uint32_t m, uint32_t k, bool x_f16) {
    if (need_res && !res)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null residual", kname);
    return gemv_launch(c, kname, f, plain_args(w, x, y, res, m, k), x_f16);
}

int qkv_launch(rt_ctx* c, const char* kname, const Fmt& f, const void* wq, const void* wk,
               const void* wv, const float* x, float* oq, float* ok, float* ov,
               const uint16_t* bq, const uint16_t* bk, const uint16_t* bv, bool bias,
               uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    if (!wq || !wk || !wv || !oq || !ok || !ov || (bias && (!bq || !bk || !bv)))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wq; a.w[1] = (const uint8_t*)wk; a.w[2] = (const uint8_t*)wv;
    a.out[0] = oq; a.out[1] = ok; a.out[2] = ov;
    a.aux[0] = bq; a.aux[1] = bk; a.aux[2] = bv;
    a.x = x;
    a.n[0] = q_dim; a.n[1] = kv_dim; a.n[2] = kv_dim;
    a.nvrows = q_dim + 2 * kv_dim;
    a.K = k;
    return gemv_launch(c, kname, f, a, false);
}

// One part of a two-part matrix-core launch: whole K, `ksw` waves per row
// quad group; returns the part's workgroups (every tile in one round: the
// caller keeps the two parts' waves within the resident capacity).
uint32_t pair_part_grid(const Fmt& f, GemvArgs& a, uint32_t threads, uint32_t ksw) {
    if (a.nvrows == 0) return 0;
    a.ksw = ksw;
    a.ksplit = 1;
    a.kc_units = a.K / f.mq_units();
    a.xb_chunk = a.K / 32;
    a.lpr = 16;
    a.row_bytes = (uint64_t)(a.K / f.blk_el) * f.blk_bytes;
    const uint32_t rows_per_wg = (threads / 64 / ksw) * 4;
    return (a.nvrows + rows_per_wg - 1) / rows_per_wg;
}

// K-split waves of the two parts: the part whose waves stream the most bytes
// (steps per wave × bytes per 64-element lane unit) doubles its split while
// the two parts' waves stay within the resident waves of the device.
void pair_ksw(const Fmt& fa, uint32_t nva, const Fmt& fb, uint32_t nvb, uint32_t K,
              uint32_t nwaves, uint32_t budget, uint32_t& ka, uint32_t& kb) {
    const uint32_t qa = (nva + 3) / 4, qb = (nvb + 3) / 4;
    const uint32_t sa = (K / fa.mq_units() + 15) / 16, sb = (K / fb.mq_units() + 15) / 16;
    const double ua = (double)fa.blk_bytes * fa.mq_units() / fa.blk_el;
    const double ub = (double)fb.blk_bytes * fb.mq_units() / fb.blk_el;
    ka = kb = 1;
    for (;;) {
        const double ta = qa ? ua * ((sa + ka - 1) / ka) : 0.0;
        const double tb = qb ? ub * ((sb + kb - 1) / kb) : 0.0;
        const bool pick_a = ta >= tb;
        uint32_t& kk = pick_a ? ka : kb;
        const uint32_t steps = pick_a ? sa : sb;
        const uint32_t quads = pick_a ? qa : qb;
        const uint64_t total = (uint64_t)qa * ka + (uint64_t)qb * kb + (uint64_t)quads * kk;
        if (kk * 2 > nwaves || kk * 2 > steps || total > budget) break;
        kk *= 2;
    }
}

// Q and K in format fa, V in format fb, in one launch (kernel <kname>_r1 of
// gemv_mq_pair).  Biases: all three or none.
int qkv_pair_launch(rt_ctx* c, const char* kname_bias, const char* kname_nobias, const Fmt& fa,
                    const Fmt& fb, const void* wq, const void* wk, const void* wv, const float* x,
                    float* oq, float* ok, float* ov, const uint16_t* bq, const uint16_t* bk,
                    const uint16_t* bv, uint32_t q_dim, uint32_t kv_dim, uint32_t k,
                    const float* gamma = nullptr, float eps = 0.0f) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    const char* kname = bq ? kname_bias : kname_nobias;
    if (!wq || !wk || !wv || !x || !oq || !ok || !ov)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    if ((bq == nullptr) != (bk == nullptr) || (bq == nullptr) != (bv == nullptr))
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: give all three biases or none", kname);
    if (k == 0 || k % fa.blk_el != 0 || k % fb.blk_el != 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: k=%u must be a positive multiple of %u", kname, k,
                    std::max(fa.blk_el, fb.blk_el));
    if (!aligned(x, 16))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: input must be 16-byte aligned",
                    kname);
    if (q_dim + kv_dim == 0) return RT_OK;
    // (RMSNorm folds into the staging of one pass over x: 4 slices of 4
    // elements per thread at 512 threads)
    if (gamma && k > 8192)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: %s: k=%u exceeds 8192 for the norm-fused form", kname, k);
    const uint32_t nxb = k / 32;
    const size_t red_bytes = 16 * 2 * 4 * sizeof(float);
    const size_t lds = (size_t)nxb * XREC_BYTES + red_bytes;
    if (lds > std::min<size_t>(c->max_lds, 80 * 1024))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: k=%u exceeds the staged %u",
                    kname, k, (uint32_t)((std::min<size_t>(c->max_lds, 80 * 1024) - red_bytes) /
                                         XREC_BYTES * 32));
    uint32_t threads = 512;
    GemvArgs a{};  // Q and K
    a.w[0] = (const uint8_t*)wq; a.w[1] = (const uint8_t*)wk; a.w[2] = (const uint8_t*)wk;
    a.out[0] = oq; a.out[1] = ok; a.out[2] = ok;
    a.aux[0] = bq; a.aux[1] = bk; a.aux[2] = bk;
    a.n[0] = q_dim; a.n[1] = kv_dim; a.n[2] = 0;
    a.nvrows = q_dim + kv_dim;
    a.K = k;
    a.x = x;
    GemvArgs b{};  // V (matrix slot 2: virtual row = row)
    b.w[0] = b.w[1] = b.w[2] = (const uint8_t*)wv;
    b.out[0] = b.out[1] = b.out[2] = ov;
    b.aux[0] = b.aux[1] = b.aux[2] = bv;
    b.n[0] = 0; b.n[1] = 0; b.n[2] = kv_dim;
    b.nvrows = kv_dim;
    b.K = k;
    b.x = x;
    a.gamma = b.gamma = gamma;
    a.eps = b.eps = eps;
    // Q and K (rows of 1–2 KB) on the small-launch body, V on the matrix-core
    // body with 4 K-split waves (≤ its dot steps), in one 512-thread launch
    // (kernel <kname>_smr; the 7B Q4_K / Q6_K projections: 8.9 → 8.1 µs, V
    // with 1 / 2 / 8 split waves 12.0 / 8.4 / 8.2 µs)
    if (c->sm_enabled) {
        char sn[96];
        snprintf(sn, sizeof sn, "%s_smr", kname);
        a.row_bytes = (uint64_t)(k / fa.blk_el) * fa.blk_bytes;
        const uint32_t nia = (uint32_t)((a.row_bytes + 15 + 1023) / 1024);
        const uint32_t T = 512, nwv = T / 64;
        if (c->fns.count(sn) && nia == 2 && nxb * 8 <= 4 * T && k % fa.mq_units() == 0) {
            a.ksplit = 1;
            a.kc_units = k / fa.mq_units();
            a.ls_rs = 2 * 1024 + kLsRowPad;
            const uint32_t ga = ((a.nvrows + 3) / 4 + nwv - 1) / nwv;
            const uint32_t steps_b = (k / fb.mq_units() + 15) / 16;
            const uint32_t gb = pair_part_grid(fb, b, T, std::max<uint32_t>(1, std::min<uint32_t>(4, steps_b)));
            const size_t lds2 = std::max((size_t)nxb * XREC_BYTES + (size_t)nwv * 4 * a.ls_rs,
                                         (size_t)nxb * XREC_BYTES + red_bytes);
            if (lds2 <= c->max_lds) {
                a.blk0 = 0; a.nblk = ga;
                b.blk0 = ga; b.nblk = gb;
                void* params[] = {&a, &b};
                return launch(c, sn, dim3(ga + gb), dim3(T), lds2, params);
            }
        }
    }
    // x in one staging pass (4 slices of 4 elements per thread), else
    // converted once into the workspace
    if (gamma && (size_t)nxb * 8 > 4 * (size_t)threads) threads = 512;
    if (!gamma && (size_t)nxb * 8 > 4 * (size_t)threads) {
        const int st0 = ensure_ws(c, (size_t)nxb * XREC_BYTES, kname);
        if (st0 != RT_OK) return st0;
        const void* xin = x;
        void* xout = c->ws;
        uint32_t nx = nxb;
        void* pp[] = {&xin, &xout, &nx};
        const int st = launch(c, "k_act_limbs_f32", dim3((nxb * 8 + 255) / 256), dim3(256), 0, pp);
        if (st != RT_OK) return st;
        a.x = b.x = c->ws;
        a.x_rec = b.x_rec = 1;
    }
    char name[96];
    snprintf(name, sizeof name, "%s_r1", kname);
    const uint32_t nwaves = threads / 64;
    const uint32_t budget = (uint32_t)c->cu_count * nwaves *
                            std::max<uint32_t>(1, occupancy(c, name, threads, lds));
    uint32_t ka, kb;
    pair_ksw(fa, a.nvrows, fb, b.nvrows, k, nwaves, budget, ka, kb);
    const uint32_t ga = pair_part_grid(fa, a, threads, ka);
    const uint32_t gb = pair_part_grid(fb, b, threads, kb);
    a.blk0 = 0; a.nblk = ga;
    b.blk0 = ga; b.nblk = gb;
    void* params[] = {&a, &b};
    return launch(c, name, dim3(ga + gb), dim3(threads), lds, params);
}

int ffn_launch(rt_ctx* c, const char* kname, const Fmt& f, const void* wg, const void* wu,
               const float* x, float* act, uint32_t ff, uint32_t k) {
    if (!wg || !wu || !act)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wg; a.w[1] = (const uint8_t*)wu;
    a.out[0] = act;
    a.x = x;
    a.n[0] = ff; a.n[1] = ff;
    a.nvrows = 2 * ff;
    a.K = k;
    return gemv_launch(c, kname, f, a, false, true);
}

int elementwise_launch(rt_ctx* c, const char* kname, const void* in, void* out, uint64_t n_el) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n_el == 0) return RT_OK;
    if (!in || !out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    const uint64_t blocks = (n_el + 255) / 256;
    if (blocks > 0x7FFFFFFFull)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: too many elements", kname);
    void* params[] = {&in, &out, &n_el};
    return launch(c, kname, dim3((uint32_t)blocks), dim3(256), 0, params);
}

int synth_launch(rt_ctx* c, const char* kname, void* out, uint64_t n, uint64_t seed, float std,
                 bool has_mean, float mean) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    if (!out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    const uint64_t want = (n + 255) / 256;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(want, (uint64_t)c->cu_count * 16);
    if (has_mean) {
        void* params[] = {&out, &n, &seed, &mean, &std};
        return launch(c, kname, dim3(grid), dim3(256), 0, params);
    }
    void* params[] = {&out, &n, &seed, &std};
    return launch(c, kname, dim3(grid), dim3(256), 0, params);
}

}  // namespace

extern "C" {

// ───────────────────────────── context ─────────────────────────────

int rt_ctx_create(rt_ctx** out, const char* code_object_path) {
    if (!out) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null out pointer");
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return fail(nullptr, RT_ERR_NO_DEVICE, "HIP device not found — is an MI355X visible?");
    rt_ctx* c = new rt_ctx();
    c->device = 0;
    hipError_t e = hipSetDevice(0);
    if (e != hipSuccess) {
        delete c;
        return fail(nullptr, RT_ERR_NO_DEVICE, "HIP device not found: %s", hipGetErrorString(e));
    }
    hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, 0);
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, 0) == hipSuccess &&
        lds > 0)
        c->max_lds = (size_t)lds;
    // A/B switches between the kernel bodies (tests and measurements)
    if (const char* g = getenv("RUNIT_GEMM_DIRECT")) c->gemm_direct = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_F16")) c->gemm_f16 = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_W16")) c->gemm_w16 = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_Q6W8")) c->gemm_q6w8 = atoi(g);
    if (const char* g = getenv("RUNIT_GEMM_SPLITS")) c->gemm_splits = (uint32_t)atoi(g);
    if (const char* g = getenv("RUNIT_GEMM_SUM_KERNEL")) c->gemm_sum_kernel = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_SET")) c->gemm_set = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_SET_MIN")) c->gemm_set_min = atoi(g);
    if (const char* g = getenv("RUNIT_GEMM_MULTI")) c->gemm_multi = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_NB4")) c->gemm_nb4 = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_BIGM_SPLIT")) c->gemm_bigm_split = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_BIGM_CHUNKS")) c->gemm_bigm_chunks = std::max(1, atoi(g));
    if (const char* g = getenv("RUNIT_GEMM_SET_SUM1")) c->gemm_set_sum1 = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_BLOCK")) c->gemm_block = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_ATTN_FOLD")) c->attn_fold = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_ROPE")) c->gemm_rope = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_BLOCK_SILU_MIN")) c->gemm_block_silu_min = atoi(g);
    if (const char* g = getenv("RUNIT_GEMV_KSPLIT")) c->ksplit_enabled = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMV_LS")) c->ls_enabled = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMV_SM")) c->sm_enabled = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMV_LS_MIN")) c->ls_min_items = (uint32_t)atoi(g);
    if (const char* g = getenv("RUNIT_GEMV_VALU")) c->gemv_valu = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMV_LSK_WHOLE")) c->lsk_whole = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMM_F16_MIN")) c->gemm_f16_min = (uint32_t)atoi(g);
    if (const char* g = getenv("RUNIT_GEMM_F16_MIN_Q6")) c->gemm_f16_min_q6 = (uint32_t)atoi(g);
    if (const char* g = getenv("RUNIT_ATTN_W")) c->attn_w = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_ATTN_MQ")) c->attn_mq = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_ATTN_MQ_NSP")) c->attn_mq_nsp = atoi(g);
    if (const char* g = getenv("RUNIT_ATTN_MQ_MIN")) c->attn_mq_min = atoi(g);
    if (const char* g = getenv("RUNIT_ATTN_MQ_FOLD_MIN")) c->attn_mq_fold_min = atoi(g);
    if (const char* g = getenv("RUNIT_ATTN_MQ_W")) c->attn_mq_w = atoi(g);
    if (const char* g = getenv("RUNIT_GEMV_VS")) c->vs_enabled = atoi(g) != 0;
    if (const char* g = getenv("RUNIT_GEMV_VS_MAXQ")) c->vs_max_q = (uint32_t)atoi(g);
    std::string path = code_object_path ? std::string(code_object_path) : default_code_object_path();
    auto unload = [](rt_ctx* cc) {
        for (hipModule_t m : cc->modules) hipModuleUnload(m);
        delete cc;
    };
    const std::vector<std::string> files = code_object_files(path);
    if (files.empty()) {
        delete c;
        return fail(nullptr, RT_ERR_LIBRARY_LOAD, "no code object in '%s'", path.c_str());
    }
    for (const std::string& f : files) {
        hipModule_t m = nullptr;
        e = hipModuleLoad(&m, f.c_str());
        if (e != hipSuccess) {
            unload(c);
            return fail(nullptr, RT_ERR_LIBRARY_LOAD, "failed to load code object from '%s': %s",
                        f.c_str(), hipGetErrorString(e));
        }
        c->modules.push_back(m);
    }
    std::vector<std::string> names(std::begin(kKernelNames), std::end(kKernelNames));
    for (const char* b : kLsBases)
        for (uint32_t ni = 1; ni <= kLsMaxNI; ++ni) names.push_back(std::string(b) + "_ls" + std::to_string(ni));
    for (const char* b : kLskBases) names.push_back(std::string(b) + "_lsk1");
    for (const char* b : kVsBases) names.push_back(std::string(b) + "_vs");
    for (const char* b : kVsnBases) names.push_back(std::string(b) + "_vsn");
    for (const char* b : kSmBases)
        for (uint32_t ni = 1; ni <= 2; ++ni) names.push_back(std::string(b) + "_sm" + std::to_string(ni));
    for (const char* b : {"k_qkv2_bias_q4k_q6k", "k_qkv2_q4k_q6k", "k_qkv2_bias_q4kg_q6kg", "k_qkv2_q4kg_q6kg"})
        names.push_back(std::string(b) + "_smr");
    for (const char* fm : kRowsFmts)
        for (const char* pat : {"k_gemv_%s_f32_f32_x8", "k_gemv_%s_f32_f32add_x8", "k_qkv_bias_%s_x8",
                                "k_ffn_%s_x8"}) {
            char nb[64];
            snprintf(nb, sizeof nb, pat, fm);
            names.push_back(nb);
        }
    names.push_back("k_act_limbs_rows_f32");
    names.push_back("k_act_limbs_rows_f32_q40");
    names.push_back("k_gemm3_q8_0_nb4_mg1");
    names.push_back("k_gemm3_q4_0_nb4_mg1");
    for (const char* b : kLsValuBases)
        for (uint32_t ni = 1; ni <= kLsMaxNI; ++ni)
            names.push_back(std::string(b) + "_ls" + std::to_string(ni) + "v");
    for (const std::string& ns : names) {
        const char* n = ns.c_str();
        hipFunction_t f = nullptr;
        for (hipModule_t m : c->modules)
            if (hipModuleGetFunction(&f, m, n) == hipSuccess && f) break;
        if (!f) {
            unload(c);
            return fail(nullptr, RT_ERR_PIPELINE_NOT_FOUND,
                        "pipeline function '%s' not found in code object", n);
        }
        c->fns[n] = f;
    }
    // the multi-matrix twins of the f16 GEMM kernels (where built)
    for (const std::string& ns : names) {
        if (ns.compare(0, 8, "k_gemm3_") != 0) continue;
        const std::string x3 = ns + "_x3";
        hipFunction_t f = nullptr;
        for (hipModule_t m : c->modules)
            if (hipModuleGetFunction(&f, m, x3.c_str()) == hipSuccess && f) break;
        if (f) c->fns[x3] = f;
    }
    (void)hipGetLastError();  // the lookups of absent twins
    e = hipMalloc(&c->aux, kAuxBytes);
    if (e == hipSuccess) e = hipMemset(c->aux, 0, kAuxBytes);
    if (e != hipSuccess) {
        unload(c);
        return fail(nullptr, RT_ERR_PIPELINE_CREATE, "failed to allocate context buffer: %s",
                    hipGetErrorString(e));
    }
    c->counters = (uint32_t*)((char*)c->aux + kAuxAttnOff);
    {
        // this device's copy of the code object's scratch array
        hipDeviceptr_t p = nullptr;
        size_t bytes = 0;
        for (hipModule_t m : c->modules) {
            e = hipModuleGetGlobal(&p, &bytes, m, "scratch");
            if (e == hipSuccess && p) break;
        }
        if (e != hipSuccess || !p || bytes != RT_SCRATCH_BYTES) {
            hipFree(c->aux);
            unload(c);
            return fail(nullptr, RT_ERR_PIPELINE_NOT_FOUND,
                        "code object has no %llu-byte 'scratch' array (%s)",
                        (unsigned long long)RT_SCRATCH_BYTES, hipGetErrorString(e));
        }
        c->scratch = (uint8_t*)p;
    }
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hipFree(c->aux);
        unload(c);
        return fail(nullptr, RT_ERR_PIPELINE_CREATE, "failed to create stream: %s",
                    hipGetErrorString(e));
    }
    *out = c;
    return RT_OK;
}

void rt_ctx_destroy(rt_ctx* c) {
    if (!c) return;
    if (c->stream) {
        hipStreamSynchronize(c->stream);
        hipStreamDestroy(c->stream);
    }
    if (c->ws) hipFree(c->ws);
    if (c->part) hipFree(c->part);
    if (c->attn_out) hipFree(c->attn_out);
    if (c->aux) hipFree(c->aux);
    for (void* p : c->retired) hipFree(p);
    for (hipModule_t m : c->modules) hipModuleUnload(m);
    delete c;
}

int rt_flush(rt_ctx* c) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "flush");
    return RT_OK;
}

const char* rt_last_error(const rt_ctx* c) { return c ? c->err.c_str() : g_global_error.c_str(); }
const char* rt_global_last_error(void) { return g_global_error.c_str(); }
int rt_device_cu_count(const rt_ctx* c) { return c ? c->cu_count : 0; }

int rt_has_kernel(rt_ctx* c, const char* name) {
    if (!c || !name) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    if (c->fns.count(name)) return RT_OK;
    return fail(c, RT_ERR_PIPELINE_NOT_FOUND, "pipeline function '%s' not found in code object",
                name);
}

int rt_malloc(rt_ctx* c, size_t bytes, void** out) {
    if (!c || !out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    *out = nullptr;
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc");
    return RT_OK;
}
int rt_free(rt_ctx* c, void* p) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!p) return RT_OK;
    hipError_t e = hipFree(p);
    if (e != hipSuccess) return hip_fail(c, e, "hipFree");
    return RT_OK;
}
static int copy_sync(rt_ctx* c, void* dst, const void* src, size_t n, hipMemcpyKind k,
                     const char* what) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    if (!dst || !src) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", what);
    hipError_t e = hipMemcpyAsync(dst, src, n, k, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, what);
    if (!c->capturing) {
        e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return hip_fail(c, e, what);
    }
    return RT_OK;
}
int rt_upload(rt_ctx* c, void* d, const void* h, size_t n) {
    return copy_sync(c, d, h, n, hipMemcpyHostToDevice, "upload");
}
int rt_download(rt_ctx* c, void* h, const void* d, size_t n) {
    return copy_sync(c, h, d, n, hipMemcpyDeviceToHost, "download");
}
int rt_copy_d2d(rt_ctx* c, void* d, const void* s, size_t n) {
    return copy_sync(c, d, s, n, hipMemcpyDeviceToDevice, "copy");
}
int rt_memset(rt_ctx* c, void* d, int v, size_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    hipError_t e = hipMemsetAsync(d, v, n, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "memset");
    e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "memset");
    return RT_OK;
}

int rt_event_create(rt_ctx* c, rt_event** out) {
    if (!c || !out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    rt_event* ev = new rt_event();
    hipError_t e = hipEventCreate(&ev->ev);
    if (e != hipSuccess) {
        delete ev;
        return hip_fail(c, e, "hipEventCreate");
    }
    *out = ev;
    return RT_OK;
}
int rt_event_record(rt_ctx* c, rt_event* ev) {
    if (!c || !ev) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    hipError_t e = hipEventRecord(ev->ev, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventRecord");
    return RT_OK;
}
int rt_event_elapsed_ms(rt_ctx* c, rt_event* a, rt_event* b, float* ms) {
    if (!c || !a || !b || !ms) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    hipError_t e = hipEventSynchronize(b->ev);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventSynchronize");
    e = hipEventElapsedTime(ms, a->ev, b->ev);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventElapsedTime");
    return RT_OK;
}
void rt_event_destroy(rt_event* ev) {
    if (!ev) return;
    hipEventDestroy(ev->ev);
    delete ev;
}

int rt_capture_begin(rt_ctx* c) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(c, e, "hipStreamBeginCapture");
    c->capturing = true;
    return RT_OK;
}
int rt_capture_end(rt_ctx* c, rt_graph** out) {
    if (!c || !out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    *out = nullptr;
    c->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (e != hipSuccess) return hip_fail(c, e, "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g);
        return hip_fail(c, e, "hipGraphInstantiate");
    }
    *out = new rt_graph{g, x};
    return RT_OK;
}
int rt_graph_launch(rt_ctx* c, rt_graph* g) {
    if (!c || !g) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: null argument");
    hipError_t e = hipGraphLaunch(g->exec, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "hipGraphLaunch");
    return RT_OK;
}
void rt_graph_destroy(rt_graph* g) {
    if (!g) return;
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    delete g;
}

// ───────────────────────────── Q8_0 ─────────────────────────────

int rt_gemv_q8_0_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                              uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f32_f32", kQ8_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q8_0_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                               const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f32_f32add", kQ8_0, w, x, y, r, true, m, k, false);
}
int rt_gemv_q8_0_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y, uint32_t m,
                       uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f32_f16", kQ8_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q8_0_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y, uint32_t m,
                     uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f16_f16", kQ8_0, w, x, y, nullptr, false, m, k, true);
}
int rt_gemv_q8_0_add_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y,
                         const uint16_t* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f16_f16add", kQ8_0, w, x, y, r, true, m, k, true);
}
int rt_gemv_q8_0_add_f32res_f16(rt_ctx* c, const void* w, const uint16_t* x, float* y,
                                const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q8_0_f16_f32add", kQ8_0, w, x, y, r, true, m, k, true);
}
int rt_gemv_q8_0_f32in_f32out_mr(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                                 uint32_t k) {
    return rt_gemv_q8_0_f32in_f32out(c, w, x, y, m, k);
}
int rt_gemv_q8_0_add_f32_f32in_mr(rt_ctx* c, const void* w, const float* x, float* y,
                                  const float* r, uint32_t m, uint32_t k) {
    return rt_gemv_q8_0_add_f32_f32in(c, w, x, y, r, m, k);
}

// ───────────────────────────── Q4_0 ─────────────────────────────

int rt_gemv_q4_0_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                              uint32_t k) {
    return gemv_plain(c, "k_gemv_q4_0_f32_f32", kQ4_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q4_0_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                               const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q4_0_f32_f32add", kQ4_0, w, x, y, r, true, m, k, false);
}
int rt_gemv_q4_0_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y, uint32_t m,
                       uint32_t k) {
    return gemv_plain(c, "k_gemv_q4_0_f32_f16", kQ4_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q4_0_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y, uint32_t m,
                     uint32_t k) {
    return gemv_plain(c, "k_gemv_q4_0_f16_f16", kQ4_0, w, x, y, nullptr, false, m, k, true);
}
int rt_gemv_q4_0_add_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y,
                         const uint16_t* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q4_0_f16_f16add", kQ4_0, w, x, y, r, true, m, k, true);
}

// ───────────────────────────── Q4_K ─────────────────────────────

int rt_gemv_q4k_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                             uint32_t k) {
    return gemv_plain(c, "k_gemv_q4k_f32_f32", kQ4K, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q4k_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                              const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q4k_f32_f32add", kQ4K, w, x, y, r, true, m, k, false);
}
int rt_gemv_q4k_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y, uint32_t m,
                    uint32_t k) {
    return gemv_plain(c, "k_gemv_q4k_f16_f16", kQ4K, w, x, y, nullptr, false, m, k, true);
}
int rt_gemv_q4k_add_f16(rt_ctx* c, const void* w, const uint16_t* x, uint16_t* y,
                        const uint16_t* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q4k_f16_f16add", kQ4K, w, x, y, r, true, m, k, true);
}
int rt_gemv_q4k_add_f32res_f16(rt_ctx* c, const void* w, const uint16_t* x, float* y,
                               const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q4k_f16_f32add", kQ4K, w, x, y, r, true, m, k, true);
}

// ───────────────────────────── Q6_K ─────────────────────────────

int rt_gemv_q6k_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                             uint32_t k) {
    return gemv_plain(c, "k_gemv_q6k_f32_f32", kQ6K, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q6k_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                              const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q6k_f32_f32add", kQ6K, w, x, y, r, true, m, k, false);
}
int rt_gemv_q6k_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y, uint32_t m,
                      uint32_t k) {
    return gemv_plain(c, "k_gemv_q6k_f32_f16", kQ6K, w, x, y, nullptr, false, m, k, false);
}

// rt_gemv_q6k_add_f32_f32in without any device allocation: the K-split
// partial sums, activation records and arrival counters come from the code
// object's scratch array instead of the context's workspace (see
// k_scratch.hip).  The counters are cleared by a fill kernel first.  Shapes
// whose launch needs more scratch than the array's regions fail with
// RT_ERR_DISPATCH before their first use of it.
int rt_gemv_q6k_add_f32_f32in_noalloc(rt_ctx* c, const void* w, const float* x, float* y,
                                      const float* r, uint32_t m, uint32_t k) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!c->scratch) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: no scratch array");
    uint32_t* cnt = (uint32_t*)c->scratch;
    uint32_t zero = 0, ncnt = (uint32_t)(RT_SCRATCH_COUNTER_BYTES / 4);
    void* fp[] = {&cnt, &zero, &ncnt};
    int st = launch(c, "k_fill_u32", dim3((ncnt + 255) / 256), dim3(256), 0, fp);
    if (st != RT_OK) return st;
    void* const ws = c->ws;
    void* const part = c->part;
    uint32_t* const counters = c->counters;
    const size_t ws_bytes = c->ws_bytes, part_bytes = c->part_bytes;
    c->noalloc = true;
    c->counters = cnt;
    c->ws = c->scratch + RT_SCRATCH_WS_OFF;
    c->ws_bytes = RT_SCRATCH_WS_BYTES;
    c->part = c->scratch + RT_SCRATCH_PART_OFF;
    c->part_bytes = RT_SCRATCH_PART_BYTES;
    st = gemv_plain(c, "k_gemv_q6k_f32_f32add", kQ6K, w, x, y, r, true, m, k, false);
    c->noalloc = false;
    c->counters = counters;
    c->ws = ws;
    c->ws_bytes = ws_bytes;
    c->part = part;
    c->part_bytes = part_bytes;
    return st;
}

// ───────────────────────────── Q5_0 / Q5_K ─────────────────────────────

int rt_gemv_q5_0_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                              uint32_t k) {
    return gemv_plain(c, "k_gemv_q5_0_f32_f32", kQ5_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q5_0_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                               const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q5_0_f32_f32add", kQ5_0, w, x, y, r, true, m, k, false);
}
int rt_gemv_q5_0_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y, uint32_t m,
                       uint32_t k) {
    return gemv_plain(c, "k_gemv_q5_0_f32_f16", kQ5_0, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q5k_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m,
                             uint32_t k) {
    return gemv_plain(c, "k_gemv_q5k_f32_f32", kQ5K, w, x, y, nullptr, false, m, k, false);
}
int rt_gemv_q5k_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,
                              const float* r, uint32_t m, uint32_t k) {
    return gemv_plain(c, "k_gemv_q5k_f32_f32add", kQ5K, w, x, y, r, true, m, k, false);
}
int rt_gemv_q5k_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y, uint32_t m,
                      uint32_t k) {
    return gemv_plain(c, "k_gemv_q5k_f32_f16", kQ5K, w, x, y, nullptr, false, m, k, false);
}
int rt_fused_qkv_bias_q5_0_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                               const float* x, float* oq, float* ok, float* ov,
                               const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                               uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_launch(c, "k_qkv_bias_q5_0", kQ5_0, wq, wk, wv, x, oq, ok, ov, bq, bk, bv, true,
                      q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q5k_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                              const float* x, float* oq, float* ok, float* ov,
                              const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                              uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_launch(c, "k_qkv_bias_q5k", kQ5K, wq, wk, wv, x, oq, ok, ov, bq, bk, bv, true,
                      q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q4k_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                              const float* x, float* oq, float* ok, float* ov,
                              const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                              uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    const bool bias = bq || bk || bv;
    return qkv_launch(c, bias ? "k_qkv_bias_q4k" : "k_qkv_q4k", kQ4K, wq, wk, wv, x, oq, ok, ov,
                      bq, bk, bv, bias, q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q4kg_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                               const float* x, float* oq, float* ok, float* ov,
                               const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                               uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    const bool bias = bq || bk || bv;
    return qkv_launch(c, bias ? "k_qkv_bias_q4kg" : "k_qkv_q4kg", kQ4KG, wq, wk, wv, x, oq, ok,
                      ov, bq, bk, bv, bias, q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q4k_q6k_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                                  const float* x, float* oq, float* ok, float* ov,
                                  const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                                  uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_pair_launch(c, "k_qkv2_bias_q4k_q6k", "k_qkv2_q4k_q6k", kQ4K, kQ6KU, wq, wk, wv,
                           x, oq, ok, ov, bq, bk, bv, q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q4kg_q6kg_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                                    const float* x, float* oq, float* ok, float* ov,
                                    const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                                    uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_pair_launch(c, "k_qkv2_bias_q4kg_q6kg", "k_qkv2_q4kg_q6kg", kQ4KG, kQ6KGU, wq, wk,
                           wv, x, oq, ok, ov, bq, bk, bv, q_dim, kv_dim, k);
}
int rt_fused_ffn_q5_0_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                          uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q5_0", kQ5_0, wg, wu, x, act, ff, k);
}
int rt_fused_ffn_q5k_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                         uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q5k", kQ5K, wg, wu, x, act, ff, k);
}

// ───────────────────────────── ggml layouts ─────────────────────────────

#define RT_GGML_GEMVS(NAME, FMT)                                                                 \
    int rt_gemv_##NAME##_f32in_f32out(rt_ctx* c, const void* w, const float* x, float* y,       \
                                      uint32_t m, uint32_t k) {                                  \
        return gemv_plain(c, "k_gemv_" #NAME "_f32_f32", FMT, w, x, y, nullptr, false, m, k,     \
                          false);                                                                \
    }                                                                                            \
    int rt_gemv_##NAME##_add_f32_f32in(rt_ctx* c, const void* w, const float* x, float* y,      \
                                       const float* r, uint32_t m, uint32_t k) {                 \
        return gemv_plain(c, "k_gemv_" #NAME "_f32_f32add", FMT, w, x, y, r, true, m, k, false); \
    }                                                                                            \
    int rt_gemv_##NAME##_f32in(rt_ctx* c, const void* w, const float* x, uint16_t* y,           \
                               uint32_t m, uint32_t k) {                                         \
        return gemv_plain(c, "k_gemv_" #NAME "_f32_f16", FMT, w, x, y, nullptr, false, m, k,     \
                          false);                                                                \
    }
RT_GGML_GEMVS(q4_0g, kQ4_0G)
RT_GGML_GEMVS(q4kg, kQ4KG)
RT_GGML_GEMVS(q5kg, kQ5KG)
RT_GGML_GEMVS(q6kg, kQ6KG)
#undef RT_GGML_GEMVS
int rt_fused_ffn_q4_0g_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                           uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q4_0g", kQ4_0G, wg, wu, x, act, ff, k);
}
int rt_fused_ffn_q4kg_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                          uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q4kg", kQ4KG, wg, wu, x, act, ff, k);
}
int rt_fused_ffn_q5kg_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                          uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q5kg", kQ5KG, wg, wu, x, act, ff, k);
}

// ───────────────────────────── fused ─────────────────────────────

int rt_fused_qkv_q8_0_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                          const float* x, float* oq, float* ok, float* ov, uint32_t q_dim,
                          uint32_t kv_dim, uint32_t k) {
    return qkv_launch(c, "k_qkv_q8_0", kQ8_0, wq, wk, wv, x, oq, ok, ov, nullptr, nullptr,
                      nullptr, false, q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q8_0_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                               const float* x, float* oq, float* ok, float* ov,
                               const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                               uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_launch(c, "k_qkv_bias_q8_0", kQ8_0, wq, wk, wv, x, oq, ok, ov, bq, bk, bv, true,
                      q_dim, kv_dim, k);
}
int rt_fused_qkv_bias_q4_0_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                               const float* x, float* oq, float* ok, float* ov,
                               const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                               uint32_t q_dim, uint32_t kv_dim, uint32_t k) {
    return qkv_launch(c, "k_qkv_bias_q4_0", kQ4_0, wq, wk, wv, x, oq, ok, ov, bq, bk, bv, true,
                      q_dim, kv_dim, k);
}
int rt_fused_ffn_q8_0_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                          uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q8_0", kQ8_0, wg, wu, x, act, ff, k);
}
int rt_fused_ffn_q4_0_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                          uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q4_0", kQ4_0, wg, wu, x, act, ff, k);
}
int rt_fused_ffn_q4k_f32(rt_ctx* c, const void* wg, const void* wu, const float* x, float* act,
                         uint32_t ff, uint32_t k) {
    return ffn_launch(c, "k_ffn_q4k", kQ4K, wg, wu, x, act, ff, k);
}

// ───────────────────────────── batched Q8_0 ─────────────────────────────

// Mirror the device-side GemmArgs / Gemm2Args (k_gemm.hip).
struct Gemm2Args {
    const void* w;
    const void* aops;
    const int* etab;
    const float* stab;
    float* y;
    float* part;
    uint32_t* counters;
    uint32_t M, N, nxb, tiles, splits, kbs, nchunks;
    uint64_t row_bytes;
    uint32_t cstride;
    const uint16_t* bias;
    const float* res;
};
struct GemmArgs {
    const void* w;
    const void* aops;
    const int* etab;
    float* y;
    uint32_t M, N, K, nxb, ksw;
    uint64_t row_bytes;
};

// Block formats of the batched GEMM (the k_gemm2_<name>_mg* kernels)
struct GemmFmt {
    const char* name;
    uint32_t blk_el, blk_bytes, recs;  // recs: 32-element records per block
    uint32_t nb_small, nb_large;       // blocks per stage for MG ≤ 2 / MG ≥ 4
    bool has_min;                      // needs per-record activation sums
    int (*gemv)(rt_ctx*, const void*, const float*, float*, uint32_t, uint32_t);
    uint32_t max_mg = 8;               // activation-row groups per chunk (LDS budget)
    uint32_t max_mg_f16 = 4;           // the f16 form's 8-row groups per chunk
};

// Y = the sum of the K splits' partial sums ([chunk][split][crow][N]),
// in split order (k_gemm_split_sum).
static int gemm_split_sum(rt_ctx* c, float* part, float* y, uint32_t m, uint32_t n, uint32_t splits,
                          uint32_t crow) {
    void* pp[] = {&part, &y, &m, &n, &splits, &crow};
    return launch(c, "k_gemm_split_sum", dim3((n + 1023) / 1024, m), dim3(256), 0, pp);
}

// Launch plan of the f16 matrix-core form (k_gemm3_*) for one weight matrix.
struct Gemm3Plan {
    char kn[48];
    uint32_t waves, MG, nchunks, nrec, nblk, tiles, base, cap, splits, kbs;
    uint64_t row_bytes;
    size_t a_bytes, e_bytes, s_bytes;  // prepared operands, row exponents, record sums
    size_t p_bytes;                    // K-split partial sums (splits > 1)
};

// Plans the f16 form: 8 activation rows per group (MG ∈ {1, 2, 4}), hi/lo
// f16 operands prepared by k_gemm_xh_prep*_mg*.  Returns kLsDecline where
// the staged layout does not apply (the caller then takes the other forms).
static int gemm3_plan(rt_ctx* c, const GemmFmt& f, const void* w, uint32_t m_rows, uint32_t n,
                      uint32_t k, Gemm3Plan& p) {
    const uint32_t cu = (uint32_t)c->cu_count;
    const uint32_t groups = (m_rows + 7) / 8;
    const uint32_t MG = std::min<uint32_t>(f.max_mg_f16, groups <= 1 ? 1 : groups <= 2 ? 2 : 4);
    const uint32_t nchunks = (m_rows + 8 * MG - 1) / (8 * MG);
    const uint32_t nrec = k / 32;
    const uint32_t nblk = k / f.blk_el;
    const uint64_t row_bytes = (uint64_t)nblk * f.blk_bytes;
    uint32_t NB = MG <= 1 ? f.nb_small : f.nb_large;
    // 8 rows whose blocks do not fill the 8-row stages: the 4-block stage
    // variant (k_gemm3_<fmt>_nb4_mg1) where there is one
    bool nb4 = false;
    if (MG == 1 && nblk % NB != 0 && NB == 8 && nblk % 4 == 0 && c->gemm_nb4) {
        char kb[48];
        snprintf(kb, sizeof kb, "k_gemm3_%s_nb4_mg1", f.name);
        if (c->fns.count(kb)) {
            NB = 4;
            nb4 = true;
        }
    }
    const uint32_t seg = NB * f.blk_bytes, vb = seg % 16 == 0 ? 16 : (seg % 8 == 0 ? 8 : 4);
    if (nblk % NB != 0 || !aligned(w, 16) || row_bytes % vb != 0 || c->gemm_direct)
        return kLsDecline;
    // Q6_K: 128-row tiles with one operand and one weight buffer
    const bool q6 = f.blk_bytes == 210;
    const bool w8ok = !q6 || (c->gemm_q6w8 >> (MG == 4 ? 0 : MG == 2 ? 1 : 2) & 1);
    uint32_t waves = ((MG >= 2 || q6) && f.blk_bytes != 34 && w8ok ? 8 : 4);
    char kn[48];
    snprintf(kn, sizeof kn, waves == 8 ? "k_gemm3_%s_mg%u_w8" : "k_gemm3_%s_mg%u", f.name, MG);
    if (nb4) {
        snprintf(kn, sizeof kn, "k_gemm3_%s_nb4_mg1", f.name);
        waves = 4;
    }
    // 256-row tiles (16 waves share each stage of activation operands: a
    // quarter of the operand reads from L2) where they leave ≥ 1/4 of the CUs
    // a tile without a K split: Q8_0 18944×3584 at M = 32 51.0 → 44.6 µs
    // (3584×18944, 14 such tiles, 64.3 → 85.4 µs)
    if (c->gemm_w16 && MG == 4 && (n + 255) / 256 >= cu / 4) {
        char k16[48];
        snprintf(k16, sizeof k16, "k_gemm3_%s_mg%u_w16", f.name, MG);
        if (c->fns.count(k16)) {
            strcpy(kn, k16);
            waves = 16;
        }
    }
    if (!c->fns.count(kn)) return kLsDecline;
    const uint32_t tiles = (n + 16 * waves - 1) / (16 * waves);
    const uint32_t per_cu = std::max<uint32_t>(1, occupancy(c, kn, 64 * waves, 0));
    const uint32_t cap = cu * per_cu;
    const uint32_t base = tiles * nchunks;
    uint32_t splits = 1;
    double best = 1e30;
    for (uint32_t sp = 1; sp <= std::min<uint32_t>(16, nblk / NB); ++sp) {
        const double rounds = (double)((base * sp + cap - 1) / cap);
        const double t = rounds / sp + 0.02 * sp;
        if (t < best - 1e-9) { best = t; splits = sp; }
    }
    // splits as launched: K ranges of whole stages
    auto eff = [&](uint32_t sp) {
        const uint32_t kb = ((nblk + sp - 1) / sp + NB - 1) / NB * NB;
        return (nblk + kb - 1) / kb;
    };
    // One workgroup per CU: where the chosen split leaves more than a tenth of
    // the CUs idle, the next larger split whose items still fit 1.15 rounds
    // (Q6_K 3584×18944 at M = 8 / 16 / 32: 8 splits of 5 stages for 7 of 6,
    // 37.1 / 41.9 / 50.0 → 33.9 / 38.4 / 45.2 µs, where 10 of 4 took 35.6 /
    // 40.2 / 47.7; Q4_K 18944×3584 keeps 3, where 4 took 34.0 → 41.8 µs, and
    // Q6_K 18944×3584 keeps 1, 45.1 against 53.1 µs)
    if (per_cu == 1 && (uint64_t)base * eff(splits) * 10 < (uint64_t)cap * 9) {
        for (uint32_t sp = splits + 1; sp <= std::min<uint32_t>(16, nblk / NB); ++sp) {
            if (eff(sp) <= eff(splits)) continue;
            if ((uint64_t)base * eff(sp) * 100 <= (uint64_t)cap * 115) splits = sp;
            break;
        }
    }
    // 2+ activation chunks (64+ rows at 32 per chunk): the chunks fill the
    // grid, and each split adds its partial sums; split only as far as half
    // the resident grid (against the rounds model above, whose splits are for
    // short launches: 0.5B prefill 4.49 → 3.81 ms, 128-row pass 2.56 → 2.35
    // ms; 7B 128 rows 13.80 → 13.00 ms, 256 rows 23.43 → 23.63 ms)
    if (nchunks >= c->gemm_bigm_chunks && c->gemm_bigm_split) {
        splits = 1;
        while ((uint64_t)base * splits * 2 <= cap && splits < nblk / NB) ++splits;
    }
    if (c->gemm_splits) splits = std::min<uint32_t>(c->gemm_splits, nblk / NB);
    const uint32_t kbs = ((nblk + splits - 1) / splits + NB - 1) / NB * NB;
    splits = (nblk + kbs - 1) / kbs;
    if (splits > 1 && base > kAttnCounters)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_%s_f32: %u tiles exceed %u counters",
                    f.name, base, kAttnCounters);
    memcpy(p.kn, kn, sizeof kn);
    p.waves = waves;
    p.MG = MG;
    p.nchunks = nchunks;
    p.nrec = nrec;
    p.nblk = nblk;
    p.tiles = tiles;
    p.base = base;
    p.cap = cap;
    p.splits = splits;
    p.kbs = kbs;
    p.row_bytes = row_bytes;
    p.a_bytes = (size_t)nchunks * nrec * MG * 64 * 16;
    p.e_bytes = (size_t)nchunks * 8 * MG * sizeof(int);  // per padded row
    p.s_bytes = f.has_min ? (size_t)nchunks * nrec * 8 * MG * sizeof(float) : 0;
    p.p_bytes = splits > 1 ? (size_t)splits * nchunks * 8 * MG * n * sizeof(float) : 0;
    return RT_OK;
}

// The activation preparation of a plan: x (or RMSNorm(x)·γ with gamma, the
// normalised rows also into xn when given) into aops / erow / stab.
static int gemm3_prep(rt_ctx* c, const Gemm3Plan& p, const float* x, uint32_t m_rows, uint32_t k,
                      void* aops, int* erow, float* stab, const float* gamma = nullptr,
                      float eps = 0.0f, float* xn = nullptr) {
    const uint32_t MG = p.MG, nchunks = p.nchunks, cu = (uint32_t)c->cu_count;
    uint32_t M = m_rows, K = k;
    char pk[48];
    if (gamma) {
        if (k > 20480)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm: norm-fused preparation "
                        "of k=%u > 20480", k);
        snprintf(pk, sizeof pk, "k_gemm_xh_prep1n_mg%u", MG);
        void* pp[] = {(void*)&x, &M, &K, &aops, &erow, &stab, (void*)&gamma, &eps, &xn};
        return launch(c, pk, dim3(nchunks * 8 * MG), dim3(1024), 0, pp);
    }
    if (k <= 20480) {
        // one workgroup per padded row, the row held in registers
        snprintf(pk, sizeof pk, "k_gemm_xh_prep1_mg%u", MG);
        void* pp[] = {(void*)&x, &M, &K, &aops, &erow, &stab};
        return launch(c, pk, dim3(nchunks * 8 * MG), dim3(1024), 0, pp);
    }
    snprintf(pk, sizeof pk, "k_gemm_xh_prep_mg%u", MG);
    uint32_t nc = nchunks;
    // workgroups (padded row, record range): ~2 per CU, ranges of ≥ 16
    // records; each workgroup also reads its whole row for the row's
    // exponent (Q8_0 3584-wide rows at M = 32: 5.0 µs with one
    // workgroup per row)
    const uint32_t rows = nchunks * 8 * MG;
    const uint32_t parts = std::max<uint32_t>(1, std::min<uint32_t>((2 * cu + rows - 1) / rows, p.nrec / 16));
    const uint32_t threads = k <= 8192 ? 256 : 512;
    void* pp[] = {(void*)&x, &M, &K, &nc, &aops, &erow, &stab};
    return launch(c, pk, dim3(rows, parts), dim3(threads), 0, pp);
}

// The GEMM of a plan over prepared operands.  part: the partial sums
// (splits > 1), left for the caller's sum when `leave_parts`; otherwise
// summed here (k_gemm_split_sum, or in the GEMM with arrival counters).
// Unsplit launches apply bias / res in their stores (y = acc + bias, then
// res + y).
static int gemm3_run(rt_ctx* c, const Gemm3Plan& p, const void* w, void* aops, int* erow,
                     float* stab, float* y, float* part, uint32_t m_rows, uint32_t n,
                     bool leave_parts = false, const uint16_t* bias = nullptr,
                     const float* res = nullptr) {
    uint32_t cstride = 32;
    while (cstride > 1 && (size_t)p.base * cstride > kAttnCounters) cstride >>= 1;
    const bool sum_kernel = p.splits > 1 && (c->gemm_sum_kernel || leave_parts);
    Gemm2Args a2{w, aops, erow, stab, y, part, sum_kernel ? nullptr : c->counters,
                 m_rows, n, p.nblk, p.tiles, p.splits, p.kbs, p.nchunks, p.row_bytes, cstride,
                 p.splits == 1 ? bias : nullptr, p.splits == 1 ? res : nullptr};
    void* p2[] = {&a2};
    int st = launch(c, p.kn, dim3(std::min(p.base * p.splits, p.cap)), dim3(64 * p.waves), 0, p2);
    if (st != RT_OK || !sum_kernel || leave_parts) return st;
    return gemm_split_sum(c, part, y, m_rows, n, p.splits, 8 * p.MG);
}

// Mirrors the device-side Gemm3Multi (k_gemm.hip).
struct Gemm3Multi {
    Gemm2Args a[3];
    uint32_t g0[4];
    uint32_t count;
};

// One GEMM of a multi-matrix launch (gemm3_many): its plan, weights, output,
// partial sums and the store epilogue of an unsplit launch.
struct Gemm3Job {
    const Gemm3Plan* p;
    const void* w;
    float* stab;
    float* y;
    float* part;
    uint32_t n;
    bool leave_parts;
    const uint16_t* bias;
    const float* res;
};

// The GEMMs of `jobs` over the same prepared operands: those that share a
// kernel run in one launch of its _x3 twin (up to three), each on its own
// range of workgroups; then the K-split sums the jobs do not leave.
static int gemm3_many(rt_ctx* c, const Gemm3Job* jobs, uint32_t count, void* aops, int* erow,
                      uint32_t m_rows) {
    bool done[4] = {false, false, false, false};
    int st = RT_OK;
    for (uint32_t i = 0; i < count && st == RT_OK; ++i) {
        if (done[i]) continue;
        // group the jobs of one kernel that each take at most two rounds of
        // resident workgroups (at the 7B prefill's 512 rows gate and up take
        // five each, and one launch of both took 36.8 against 36.4 ms; a
        // grouping that fits one round in all left out gate + up at 8 rows:
        // 7B verify 3.55 against 3.75 ms)
        auto short_job = [&](const Gemm3Job& b) {
            return (uint64_t)b.p->base * b.p->splits <= 2ull * b.p->cap;
        };
        uint32_t grp[3] = {i, 0, 0}, ng = 1;
        for (uint32_t j = i + 1; j < count && ng < 3 && c->gemm_multi && short_job(jobs[i]); ++j)
            if (!done[j] && strcmp(jobs[j].p->kn, jobs[i].p->kn) == 0 && short_job(jobs[j]))
                grp[ng++] = j;
        char x3[56];
        snprintf(x3, sizeof x3, "%s_x3", jobs[i].p->kn);
        if (ng == 1 || !c->fns.count(x3)) {
            const Gemm3Job& b = jobs[i];
            st = gemm3_run(c, *b.p, b.w, aops, erow, b.stab, b.y, b.part, m_rows, b.n, b.leave_parts,
                           b.bias, b.res);
            done[i] = true;
            continue;
        }
        Gemm3Multi mm{};
        uint32_t g = 0;
        for (uint32_t q = 0; q < ng; ++q) {
            const Gemm3Job& b = jobs[grp[q]];
            const Gemm3Plan& p = *b.p;
            uint32_t cstride = 32;
            while (cstride > 1 && (size_t)p.base * cstride > kAttnCounters) cstride >>= 1;
            mm.a[q] = Gemm2Args{b.w, aops, erow, b.stab, b.y, b.part, nullptr, m_rows, b.n, p.nblk,
                                p.tiles, p.splits, p.kbs, p.nchunks, p.row_bytes, cstride,
                                p.splits == 1 ? b.bias : nullptr, p.splits == 1 ? b.res : nullptr};
            mm.g0[q] = g;
            g += std::min(p.base * p.splits, p.cap);
            done[grp[q]] = true;
        }
        mm.g0[ng] = g;
        mm.count = ng;
        void* pp[] = {&mm};
        st = launch(c, x3, dim3(g), dim3(64 * jobs[i].p->waves), 0, pp);
        for (uint32_t q = 0; q < ng && st == RT_OK; ++q) {
            const Gemm3Job& b = jobs[grp[q]];
            if (b.p->splits > 1 && !b.leave_parts)
                st = gemm_split_sum(c, b.part, b.y, m_rows, b.n, b.p->splits, 8 * b.p->MG);
        }
    }
    return st;
}

// f16 matrix-core form of the staged GEMM for one weight matrix: plan,
// workspace, preparation, GEMM.
int gemm3_launch(rt_ctx* c, const GemmFmt& f, const void* w, const float* x, float* y,
                 uint32_t m_rows, uint32_t n, uint32_t k) {
    Gemm3Plan p;
    int st = gemm3_plan(c, f, w, m_rows, n, k, p);
    if (st != RT_OK) return st;
    st = ensure_ws(c, p.a_bytes + p.e_bytes + p.s_bytes + p.p_bytes, "gemm");
    if (st != RT_OK) return st;
    void* aops = c->ws;
    int* erow = (int*)((char*)c->ws + p.a_bytes);
    float* stab = p.s_bytes ? (float*)((char*)c->ws + p.a_bytes + p.e_bytes) : nullptr;
    float* part = p.p_bytes ? (float*)((char*)c->ws + p.a_bytes + p.e_bytes + p.s_bytes) : nullptr;
    st = gemm3_prep(c, p, x, m_rows, k, aops, erow, stab);
    if (st != RT_OK) return st;
    return gemm3_run(c, p, w, aops, erow, stab, y, part, m_rows, n);
}

int gemm_launch(rt_ctx* c, const GemmFmt& f, const void* w, const float* x, float* y,
                uint32_t m_rows, uint32_t n, uint32_t k) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (m_rows == 0 || n == 0) return RT_OK;
    if (!w || !x || !y)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_%s_f32: null buffer", f.name);
    if (k == 0 || k % f.blk_el != 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: gemm_%s_f32: k=%u must be a positive multiple of %u",
                    f.name, k, f.blk_el);
    if (!aligned(x, 16))
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: gemm_%s_f32: input must be 16-byte aligned", f.name);
    if (m_rows == 1) return f.gemv(c, w, x, y, n, k);
    // f16 form from 5 rows on (with one exponent per activation row it runs
    // M = 8 faster than the int8 limb form: Q8_0 18944×3584 27.7 → 25.9 µs,
    // Q6_K 3584×18944 51.0 → 42.6 µs; at M = 4 the int8 form stays ahead:
    // 24.1 against 25.8 µs); Q6_K from 2 rows on (its 128-row f16 tiles:
    // M = 2 / 4 on 3584×18944 42.8 / 43.0 → 36.5 / 36.7 µs)
    if (c->gemm_f16 && m_rows > (f.blk_bytes == 210 ? c->gemm_f16_min_q6 : c->gemm_f16_min)) {
        const int st = gemm3_launch(c, f, w, x, y, m_rows, n, k);
        if (st != kLsDecline) return st;
    }
    const uint32_t cu = (uint32_t)c->cu_count;
    // 4·MG activation rows per chunk (MG ∈ {1, 2, 4, 8}); longer batches
    // take several chunks, each streaming W once
    const uint32_t groups = (m_rows + 3) / 4;
    const uint32_t MG = std::min<uint32_t>(f.max_mg, groups <= 1 ? 1 : groups <= 2 ? 2 : groups <= 4 ? 4 : 8);
    const uint32_t nchunks = (m_rows + 4 * MG - 1) / (4 * MG);
    const uint32_t nrec = k / 32;        // activation records
    const uint32_t nblk = k / f.blk_el;  // weight blocks per row
    const uint64_t row_bytes = (uint64_t)nblk * f.blk_bytes;
    const uint32_t NB = MG <= 2 ? f.nb_small : f.nb_large;
    const uint32_t seg = NB * f.blk_bytes, vb = seg % 16 == 0 ? 16 : (seg % 8 == 0 ? 8 : 4);

    // Plan.  LDS-staged kernel when every row's stage segments stay
    // vb-aligned: 64-row tiles, K in stages of NB blocks, items (tile, K
    // split, chunk) on a persistent grid of `cap` workgroups.  Otherwise Q8_0
    // takes the direct kernel (16·CT weight rows per workgroup whose ksw
    // waves split the blocks) and the other formats one GEMV per row.
    const bool staged = nblk % NB == 0 && aligned(w, 16) && row_bytes % vb == 0 && !c->gemm_direct;
    const bool direct = !staged && f.blk_bytes == 34;
    if (!staged && !direct) {
        for (uint32_t m = 0; m < m_rows; ++m) {
            const int st = f.gemv(c, w, x + (size_t)m * k, y + (size_t)m * n, n, k);
            if (st != RT_OK) return st;
        }
        return RT_OK;
    }
    // Workgroups of 4 waves (64-row tiles), or of 8 waves (128-row tiles)
    // for the 4-bit formats at 16+ rows, whose activation operands per stage
    // are larger than the weights': the 8 waves share each staged operand
    // stage (Q4_K at M = 32: 90 → 61 µs; Q8_0 runs slower so: 55 → 66 µs).
    // (Q6_K: 4-wave workgroups only, its two-super-block stages fill LDS)
    const bool w8ok = f.blk_bytes != 210;
    const uint32_t waves = (MG >= 4 && f.blk_bytes != 34 && w8ok ? 8 : 4);
    char kn2[48];
    if (waves == 8)
        snprintf(kn2, sizeof kn2, "k_gemm2_%s_mg%u_w8", f.name, MG);
    else
        snprintf(kn2, sizeof kn2, "k_gemm2_%s_mg%u", f.name, MG);
    const uint32_t tiles = (n + 16 * waves - 1) / (16 * waves);
    const uint32_t per_cu = std::max<uint32_t>(1, occupancy(c, kn2, 64 * waves, 0));
    const uint32_t cap = cu * per_cu;
    const uint32_t base = tiles * nchunks;
    uint32_t splits = 1, kbs = nblk;
    if (staged) {
        double best = 1e30;
        for (uint32_t sp = 1; sp <= std::min<uint32_t>(16, nblk / NB); ++sp) {
            // rounds of items, each 1/sp of the K range, plus a small cost per split
            const double rounds = (double)((base * sp + cap - 1) / cap);
            const double t = rounds / sp + 0.02 * sp;
            if (t < best - 1e-9) { best = t; splits = sp; }
        }
        kbs = ((nblk + splits - 1) / splits + NB - 1) / NB * NB;
        splits = (nblk + kbs - 1) / kbs;
        if (splits > 1 && base > kAttnCounters)
            return fail(c, RT_ERR_DISPATCH,
                        "kernel dispatch error: gemm_%s_f32: %u tiles exceed %u counters", f.name,
                        base, kAttnCounters);
    }
    const size_t a_bytes = (size_t)nchunks * nrec * MG * 64 * 8;
    const size_t e_bytes = (size_t)nchunks * nrec * 4 * MG * sizeof(int);
    const size_t s_bytes = f.has_min ? e_bytes : 0;
    const size_t p_bytes = splits > 1 ? (size_t)splits * nchunks * 4 * MG * n * sizeof(float) : 0;
    int st = ensure_ws(c, a_bytes + e_bytes + s_bytes + p_bytes, "gemm");
    if (st != RT_OK) return st;
    void* aops = c->ws;
    int* etab = (int*)((char*)c->ws + a_bytes);
    float* stab = s_bytes ? (float*)((char*)c->ws + a_bytes + e_bytes) : nullptr;
    float* part = p_bytes ? (float*)((char*)c->ws + a_bytes + e_bytes + s_bytes) : nullptr;
    {
        char pk[48];
        snprintf(pk, sizeof pk, "k_gemm_x_prep_mg%u", MG);
        const uint64_t threads = (uint64_t)nchunks * 4 * MG * nrec * 8;
        const uint32_t grid = (uint32_t)std::min<uint64_t>((threads + 255) / 256, (uint64_t)cu * 16);
        uint32_t M = m_rows, K = k, nc = nchunks;
        void* pp[] = {(void*)&x, &M, &K, &nc, &aops, &etab, &stab};
        st = launch(c, pk, dim3(grid), dim3(256), 0, pp);
        if (st != RT_OK) return st;
    }
    if (staged) {
        uint32_t cstride = 32;  // counters on their own cache lines while they fit
        while (cstride > 1 && (size_t)base * cstride > kAttnCounters) cstride >>= 1;
        const bool sum_kernel = splits > 1 && c->gemm_sum_kernel;
        Gemm2Args a2{w, aops, etab, stab, y, part, sum_kernel ? nullptr : c->counters,
                     m_rows, n, nblk, tiles, splits, kbs, nchunks, row_bytes, cstride};
        void* p2[] = {&a2};
        st = launch(c, kn2, dim3(std::min(base * splits, cap)), dim3(64 * waves), 0, p2);
        if (st != RT_OK || !sum_kernel) return st;
        return gemm_split_sum(c, part, y, m_rows, n, splits, 4 * MG);
    }
    const uint32_t CT = ((n + 31) / 32 >= 2 * cu) ? 2 : 1;
    const uint32_t gx = (n + 16 * CT - 1) / (16 * CT);
    uint32_t ksw = 1;
    while (ksw < 8 && (uint64_t)gx * nchunks * ksw < 8ull * cu && ksw * 2 <= nrec) ksw *= 2;
    GemmArgs a{w, aops, etab, y, m_rows, n, k, nrec, ksw, row_bytes};
    char kn[48];
    snprintf(kn, sizeof kn, "k_gemm_q8_0_mg%u_ct%u", MG, CT);
    void* params[] = {&a};
    return launch(c, kn, dim3(gx, nchunks), dim3(64 * ksw), 0, params);
}

constexpr GemmFmt kGemmQ8_0{"q8_0", 32, 34, 1, 8, 4, false, rt_gemv_q8_0_f32in_f32out};
constexpr GemmFmt kGemmQ4_0{"q4_0", 32, 18, 1, 8, 4, false, rt_gemv_q4_0_f32in_f32out};
constexpr GemmFmt kGemmQ4K{"q4k", 256, 144, 8, 1, 1, true, rt_gemv_q4k_f32in_f32out};
constexpr GemmFmt kGemmQ5_0{"q5_0", 32, 22, 1, 8, 4, false, rt_gemv_q5_0_f32in_f32out};
constexpr GemmFmt kGemmQ5K{"q5k", 256, 176, 8, 1, 1, true, rt_gemv_q5k_f32in_f32out};
constexpr GemmFmt kGemmQ6K{"q6k", 256, 210, 8, 2, 2, false, rt_gemv_q6k_f32in_f32out, 4, 4};
constexpr GemmFmt kGemmQ4_0G{"q4_0g", 32, 18, 1, 8, 4, false, rt_gemv_q4_0g_f32in_f32out};
constexpr GemmFmt kGemmQ4KG{"q4kg", 256, 144, 8, 1, 1, true, rt_gemv_q4kg_f32in_f32out};
constexpr GemmFmt kGemmQ5KG{"q5kg", 256, 176, 8, 1, 1, true, rt_gemv_q5kg_f32in_f32out};
constexpr GemmFmt kGemmQ6KG{"q6kg", 256, 210, 8, 2, 2, false, rt_gemv_q6kg_f32in_f32out, 4, 4};

RT_ROWS_ENTRIES(q8_0, kQ8_0)
RT_ROWS_ENTRIES(q4_0, kQ4_0)
RT_ROWS_ENTRIES(q4k, kQ4K)
RT_ROWS_ENTRIES(q6k, kQ6KU)
RT_ROWS_ENTRIES(q5_0, kQ5_0)
RT_ROWS_ENTRIES(q5k, kQ5K)
RT_ROWS_ENTRIES(q4_0g, kQ4_0G)
RT_ROWS_ENTRIES(q4kg, kQ4KG)
RT_ROWS_ENTRIES(q5kg, kQ5KG)
RT_ROWS_ENTRIES(q6kg, kQ6KGU)

int rt_gemm_q8_0_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ8_0, w, x, y, m_rows, n, k);
}
int rt_gemm_q4_0_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ4_0, w, x, y, m_rows, n, k);
}
int rt_gemm_q4k_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ4K, w, x, y, m_rows, n, k);
}
int rt_gemm_q5_0_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ5_0, w, x, y, m_rows, n, k);
}
int rt_gemm_q5k_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ5K, w, x, y, m_rows, n, k);
}
int rt_gemm_q6k_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                    uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ6K, w, x, y, m_rows, n, k);
}
int rt_gemm_q4_0g_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                      uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ4_0G, w, x, y, m_rows, n, k);
}
int rt_gemm_q4kg_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ4KG, w, x, y, m_rows, n, k);
}
int rt_gemm_q5kg_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ5KG, w, x, y, m_rows, n, k);
}
int rt_gemm_q6kg_f32(rt_ctx* c, const void* w, const float* x, float* y, uint32_t m_rows,
                     uint32_t n, uint32_t k) {
    return gemm_launch(c, kGemmQ6KG, w, x, y, m_rows, n, k);
}

static const GemmFmt* gemm_fmt_named(const char* name) {
    static const GemmFmt* const all[] = {&kGemmQ8_0, &kGemmQ4_0, &kGemmQ4K, &kGemmQ5_0, &kGemmQ5K,
                                         &kGemmQ6K, &kGemmQ4_0G, &kGemmQ4KG, &kGemmQ5KG, &kGemmQ6KG};
    for (const GemmFmt* f : all)
        if (name && strcmp(name, f->name) == 0) return f;
    return nullptr;
}

// Mirrors the device-side EpSeg / EpSegs (k_gemm.hip).
struct EpSeg {
    const float* part;
    float* y;
    const uint16_t* bias;
    uint32_t n, splits, blk0;
};
struct EpSegs {
    EpSeg s[3];
    uint32_t count, crow;
};

static int gemm_split_sum_ep(rt_ctx* c, const float* part, const float* part2, float* y, uint32_t m,
                             uint32_t n, uint32_t splits, uint32_t crow, const uint16_t* bias,
                             const float* res) {
    void* pp[] = {(void*)&part, (void*)&part2, &y, &m, &n, &splits, &crow, (void*)&bias, (void*)&res};
    return launch(c, "k_gemm_split_sum_ep", dim3((n + 1023) / 1024, m), dim3(256), 0, pp);
}

// Mirrors the device-side RopeKv (k_gemm.hip).
struct RopeKv {
    float* kc;
    float* vc;
    uint32_t head_dim, start_pos, max_seq;
    float theta;
};

// rt_gemm_set_f32; with `rope` (count 3: q, k, v) the sums also rotate q and
// k and write k and v to the caches (k_gemm_split_sum_qkv_rope), or, on the
// separate launches, rope_kv_write_batch runs after them.
static int gemm_set_impl(rt_ctx* c, uint32_t count, const char* const* fmts, const void* const* w,
                         float* const* y, const uint32_t* n, const uint16_t* const* bias,
                         const float* res, const float* x, uint32_t m_rows, uint32_t k,
                         const float* gamma, float eps, float* xn, uint32_t silu_pair,
                         const RopeKv* rope) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (count == 0 || count > 4 || !fmts || !w || !y || !n)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: count=%u (1..4) or null "
                    "array", count);
    if (m_rows == 0) return RT_OK;
    if (!x || (gamma && !xn))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: null x, or gamma without xn");
    if (silu_pair && (count != 2 || bias || res || n[0] != n[1]))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: the SiLU pair takes two "
                    "matrices of one shape, no bias or residual");
    if (res && (count != 1 || res == y[0]))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: the residual takes one "
                    "matrix and an output apart from it");
    const GemmFmt* f[4];
    for (uint32_t i = 0; i < count; ++i) {
        f[i] = gemm_fmt_named(fmts[i]);
        if (!f[i] || !w[i] || !y[i] || n[i] == 0)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: matrix %u: format "
                        "'%s', null buffer or n = 0", i, fmts[i] ? fmts[i] : "(null)");
        if (k == 0 || k % f[i]->blk_el != 0)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_set: k=%u must be a "
                        "positive multiple of %u", k, f[i]->blk_el);
    }
    if (rope && (count != 3 || silu_pair || res || n[1] != n[2] || rope->head_dim == 0 ||
                 n[0] % rope->head_dim || n[1] % rope->head_dim))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_qkv_rope: q_dim / kv_dim "
                    "not multiples of head_dim");
    // The shared form: every matrix on the f16 form with one row grouping,
    // one preparation (norm-fused when gamma), epilogues in the split sums.
    Gemm3Plan pl[4];
    // (the shared form's kernels move x, γ, the normalised rows, the
    // residual and the rotated / cached rows in 16-byte, biases in 8-byte units)
    bool shared = c->gemm_set && c->gemm_f16 && m_rows >= 2 && m_rows > c->gemm_set_min &&
                  k <= 20480 && aligned(x, 16) && (!gamma || (aligned(gamma, 16) && aligned(xn, 16))) &&
                  (!res || aligned(res, 16)) &&
                  (!rope || (aligned(y[0], 16) && aligned(rope->kc, 16) && aligned(rope->vc, 16))) &&
                  (!rope || (1024 % rope->head_dim == 0 && rope->head_dim % 4 == 0 && rope->head_dim <= 512 && n[0] % 4 == 0 && n[1] % 4 == 0 &&
                             c->gemm_rope));
    for (uint32_t i = 0; shared && i < count; ++i) {
        if (bias && bias[i] && !aligned(bias[i], 8)) {
            shared = false;
            break;
        }
        const int st = gemm3_plan(c, *f[i], w[i], m_rows, n[i], k, pl[i]);
        if (st != RT_OK && st != kLsDecline) return st;
        shared = st == RT_OK && pl[i].MG == pl[0].MG;
    }
    if (!shared) {
        // the separate launches: norm, one GEMM per matrix, then the
        // bias / residual / SiLU kernels
        const float* X = x;
        if (gamma) {
            int st = rt_rms_norm_f32_f32_f32g(c, x, xn, gamma, eps, k, m_rows);
            if (st != RT_OK) return st;
            X = xn;
        }
        for (uint32_t i = 0; i < count; ++i) {
            int st = gemm_launch(c, *f[i], w[i], X, y[i], m_rows, n[i], k);
            if (st == RT_OK && bias && bias[i]) st = rt_add_bias_broadcast_f32(c, y[i], bias[i], m_rows, n[i]);
            if (st != RT_OK) return st;
        }
        if (res) return rt_add_f32(c, res, y[0], y[0], m_rows * n[0]);
        if (silu_pair) return rt_silu_mul_f32(c, y[0], y[1], y[0], m_rows * n[0]);
        if (rope)
            return rt_rope_kv_write_batch_f32(c, y[0], y[1], y[2], rope->kc, rope->vc,
                                              rope->head_dim, n[0] / rope->head_dim,
                                              n[1] / rope->head_dim, rope->start_pos, rope->theta,
                                              m_rows, rope->max_seq);
        return RT_OK;
    }
    // workspace: [operands | row exponents | record sums | partials of each matrix]
    bool any_min = false;
    for (uint32_t i = 0; i < count; ++i) any_min |= f[i]->has_min;
    const Gemm3Plan& p0 = pl[0];
    const size_t s_bytes = any_min ? (size_t)p0.nchunks * p0.nrec * 8 * p0.MG * sizeof(float) : 0;
    const uint32_t crow = 8 * p0.MG;
    size_t poff[4], total = p0.a_bytes + p0.e_bytes + s_bytes;
    bool ep[4];
    for (uint32_t i = 0; i < count; ++i) {
        // epilogue in the split sum: split launches, and the SiLU pair (an
        // unsplit launch adds its bias / residual in its own stores)
        ep[i] = rope || ((silu_pair || res || (bias && bias[i])) && (silu_pair || pl[i].splits > 1));
        poff[i] = total;
        // a matrix with an epilogue leaves its partial sums (one "split"
        // when unsplit) for k_gemm_split_sum_ep
        total += ep[i] ? (size_t)std::max<uint32_t>(1, pl[i].splits) * p0.nchunks * crow * n[i] * sizeof(float)
                       : pl[i].p_bytes;
        total = (total + 255) & ~(size_t)255;
    }
    int st = ensure_ws(c, total, "gemm_set");
    if (st != RT_OK) return st;
    char* ws = (char*)c->ws;
    void* aops = ws;
    int* erow = (int*)(ws + p0.a_bytes);
    float* stab = s_bytes ? (float*)(ws + p0.a_bytes + p0.e_bytes) : nullptr;
    st = gemm3_prep(c, p0, x, m_rows, k, aops, erow, stab, gamma, eps, gamma ? xn : nullptr);
    if (st != RT_OK) return st;
    // the sums (+ bias) of the matrices of a set without residual or SiLU
    // pair: one launch for all of them (k_gemm_split_sum_ep3)
    EpSegs es{};
    es.crow = crow;
    const bool one_sum = !silu_pair && !res && (c->gemm_set_sum1 || rope) && count <= 3;
    Gemm3Job jobs[4];
    for (uint32_t i = 0; i < count; ++i) {
        float* part = (float*)(ws + poff[i]);
        // unsplit with an epilogue: the GEMM writes its rows into the partials
        jobs[i] = Gemm3Job{&pl[i], w[i], f[i]->has_min ? stab : nullptr,
                           ep[i] && pl[i].splits == 1 ? part : y[i], part, n[i], ep[i],
                           ep[i] || !bias ? nullptr : bias[i], ep[i] ? nullptr : res};
    }
    st = gemm3_many(c, jobs, count, aops, erow, m_rows);
    if (st != RT_OK) return st;
    for (uint32_t i = 0; i < count; ++i) {
        float* part = (float*)(ws + poff[i]);
        if (ep[i] && one_sum) {
            EpSeg& g = es.s[es.count];
            g.blk0 = es.count ? es.s[es.count - 1].blk0 + (es.s[es.count - 1].n + 1023) / 1024 : 0;
            g.part = part;
            g.y = y[i];
            g.bias = bias ? bias[i] : nullptr;
            g.n = n[i];
            g.splits = pl[i].splits;
            ++es.count;
        } else if (ep[i] && !silu_pair) {
            st = gemm_split_sum_ep(c, part, nullptr, y[i], m_rows, n[i], pl[i].splits, crow,
                                   bias ? bias[i] : nullptr, res);
        }
        if (st != RT_OK) return st;
    }
    if (es.count == 1) {
        const EpSeg& g = es.s[0];
        st = gemm_split_sum_ep(c, g.part, nullptr, g.y, m_rows, g.n, g.splits, crow, g.bias, nullptr);
    } else if (es.count > 1) {
        const EpSeg& g = es.s[es.count - 1];
        RopeKv rk = rope ? *rope : RopeKv{};
        void* pp[] = {&es, &rk};
        st = launch(c, rope ? "k_gemm_split_sum_qkv_rope" : "k_gemm_split_sum_ep3",
                    dim3(g.blk0 + (g.n + 1023) / 1024, m_rows), dim3(256), 0, pp);
    }
    if (st != RT_OK) return st;
    if (!silu_pair) return RT_OK;
    float* pg = (float*)(ws + poff[0]);
    float* pu = (float*)(ws + poff[1]);
    if (pl[0].splits == pl[1].splits)
        return gemm_split_sum_ep(c, pg, pu, y[0], m_rows, n[0], pl[0].splits, crow, nullptr, nullptr);
    st = gemm_split_sum_ep(c, pu, nullptr, y[1], m_rows, n[1], pl[1].splits, crow, nullptr, nullptr);
    if (st == RT_OK)
        st = gemm_split_sum_ep(c, pg, nullptr, y[0], m_rows, n[0], pl[0].splits, crow, nullptr, nullptr);
    if (st != RT_OK) return st;
    return rt_silu_mul_f32(c, y[0], y[1], y[0], m_rows * n[0]);
}

int rt_gemm_set_f32(rt_ctx* c, uint32_t count, const char* const* fmts, const void* const* w,
                    float* const* y, const uint32_t* n, const uint16_t* const* bias,
                    const float* res, const float* x, uint32_t m_rows, uint32_t k,
                    const float* gamma, float eps, float* xn, uint32_t silu_pair) {
    return gemm_set_impl(c, count, fmts, w, y, n, bias, res, x, m_rows, k, gamma, eps, xn,
                         silu_pair, nullptr);
}

int rt_gemm_qkv_rope_f32(rt_ctx* c, const char* fmt_q, const void* w_q, const char* fmt_k,
                         const void* w_k, const char* fmt_v, const void* w_v, const uint16_t* b_q,
                         const uint16_t* b_k, const uint16_t* b_v, const float* x,
                         const float* gamma, float eps, float* xn, float* q, float* k, float* v,
                         float* k_cache, float* v_cache, uint32_t m_rows, uint32_t hidden,
                         uint32_t q_dim, uint32_t kv_dim, uint32_t head_dim, uint32_t start_pos,
                         float theta, uint32_t max_seq) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (m_rows == 0) return RT_OK;
    if (!k_cache || !v_cache || (uint64_t)start_pos + m_rows > max_seq)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_qkv_rope: null cache, or "
                    "start_pos=%u + %u rows > max_seq=%u", start_pos, m_rows, max_seq);
    const char* fm[] = {fmt_q, fmt_k, fmt_v};
    const void* wv[] = {w_q, w_k, w_v};
    float* yv[] = {q, k, v};
    const uint32_t nv[] = {q_dim, kv_dim, kv_dim};
    const uint16_t* bv[] = {b_q, b_k, b_v};
    const RopeKv rk{k_cache, v_cache, head_dim, start_pos, max_seq, theta};
    return gemm_set_impl(c, 3, fm, wv, yv, nv, bv, nullptr, x, m_rows, hidden, gamma, eps, xn, 0,
                         &rk);
}

// Mirrors the device-side PrepSum (k_gemm.hip).
struct PrepSum {
    const float* part;
    const float* part2;
    const float* res;
    float* y;
    uint32_t splits, crow;
};

// Mirrors the device-side PrepAttn (k_gemm.hip).
struct PrepAttnHost {
    const float* part;
    const float* ml;
    uint32_t nsp, G, hd, cgs;
};

// rt_gemm_ffn_block_f32.  plan_only: report in *shared whether the shared
// form applies, launching nothing; pa: the O projection's input given as
// multi-query attention partials (merged in its operand preparation) instead
// of att (shared form only).
static int ffn_block_impl(rt_ctx* c, const char* fmt_o, const void* w_o, const char* fmt_gate,
                          const void* w_gate, const char* fmt_up, const void* w_up,
                          const char* fmt_down, const void* w_down, const float* att, float* x,
                          float* x_mid, const float* gamma, float eps, float* g, float* u,
                          float* xn, uint32_t m_rows, uint32_t h, uint32_t qd, uint32_t ff,
                          bool plan_only, bool* shared, const PrepAttnHost* pa) {
    if (shared) *shared = false;
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (m_rows == 0) return RT_OK;
    if (!att || !x || !x_mid || !gamma || !g || !u || !xn || x_mid == x)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: gemm_ffn_block: null buffer, or "
                    "x_mid the same as x");
    const GemmFmt* fo = gemm_fmt_named(fmt_o);
    const GemmFmt* fg = gemm_fmt_named(fmt_gate);
    const GemmFmt* fu = gemm_fmt_named(fmt_up);
    const GemmFmt* fd = gemm_fmt_named(fmt_down);
    // the separate sets: O + residual, gate/up + SiLU of the normalised
    // rows, down + residual (every argument check is theirs)
    auto sets = [&]() {
        const char* f1[] = {fmt_o};
        const void* w1[] = {w_o};
        float* y1[] = {x_mid};
        const uint32_t n1[] = {h};
        int st = rt_gemm_set_f32(c, 1, f1, w1, y1, n1, nullptr, x, att, m_rows, qd, nullptr, 0.0f,
                                 nullptr, 0);
        if (st != RT_OK) return st;
        const char* f2[] = {fmt_gate, fmt_up};
        const void* w2[] = {w_gate, w_up};
        float* y2[] = {g, u};
        const uint32_t n2[] = {ff, ff};
        st = rt_gemm_set_f32(c, 2, f2, w2, y2, n2, nullptr, nullptr, x_mid, m_rows, h, gamma, eps,
                             xn, 1);
        if (st != RT_OK) return st;
        const char* f3[] = {fmt_down};
        const void* w3[] = {w_down};
        float* y3[] = {x};
        const uint32_t n3[] = {h};
        return rt_gemm_set_f32(c, 1, f3, w3, y3, n3, nullptr, x_mid, g, m_rows, ff, nullptr, 0.0f,
                               nullptr, 0);
    };
    if (!fo || !fg || !fu || !fd || !c->gemm_set || !c->gemm_block || !c->gemm_f16 || m_rows < 2 ||
        m_rows <= c->gemm_set_min || qd > 20480 || h > 20480 || ff > 20480 || !aligned(att, 16) ||
        !aligned(x, 16) || !aligned(x_mid, 16) || !aligned(gamma, 16) ||
        qd % fo->blk_el || h % fg->blk_el || h % fu->blk_el || ff % fd->blk_el)
        return plan_only ? RT_OK : sets();
    Gemm3Plan po, pg, pu, pd;
    int st = gemm3_plan(c, *fo, w_o, m_rows, h, qd, po);
    if (st == RT_OK) st = gemm3_plan(c, *fg, w_gate, m_rows, ff, h, pg);
    if (st == RT_OK) st = gemm3_plan(c, *fu, w_up, m_rows, ff, h, pu);
    if (st == RT_OK) st = gemm3_plan(c, *fd, w_down, m_rows, h, ff, pd);
    if (st == kLsDecline || (st == RT_OK && (pg.MG != po.MG || pu.MG != po.MG || pd.MG != po.MG ||
                                             pg.splits != pu.splits)))
        return plan_only ? RT_OK : sets();
    if (st != RT_OK) return st;
    if (plan_only) {
        if (shared) *shared = true;
        return RT_OK;
    }
    // workspace: operands of att (K = qd), of the normalised x_mid (K = h),
    // of the SiLU product (K = ff), then the partial sums of O, gate, up, down
    const uint32_t MG = po.MG, nch = po.nchunks, crow = 8 * MG;
    auto ops = [&](uint32_t k, bool mins) {
        const size_t a = (size_t)nch * (k / 32) * MG * 64 * 16, e = (size_t)nch * 8 * MG * sizeof(int);
        const size_t sb = mins ? (size_t)nch * (k / 32) * 8 * MG * sizeof(float) : 0;
        return std::array<size_t, 3>{a, e, sb};
    };
    auto parts = [&](const Gemm3Plan& p, uint32_t n) {
        return (size_t)std::max<uint32_t>(1, p.splits) * nch * crow * n * sizeof(float);
    };
    const auto oa = ops(qd, fo->has_min), oh = ops(h, fg->has_min || fu->has_min), of = ops(ff, fd->has_min);
    size_t off[12], total = 0;
    const size_t sizes[12] = {oa[0], oa[1], oa[2], oh[0], oh[1], oh[2], of[0], of[1], of[2],
                              parts(po, h), parts(pg, ff), parts(pu, ff)};
    for (int i = 0; i < 12; ++i) {
        off[i] = total;
        total = (total + sizes[i] + 255) & ~(size_t)255;
    }
    const size_t off_pd = total;
    total += parts(pd, h);
    st = ensure_ws(c, total, "gemm_ffn_block");
    if (st != RT_OK) return st;
    char* ws = (char*)c->ws;
    auto at = [&](int i) { return sizes[i] ? (void*)(ws + off[i]) : nullptr; };
    float* part_o = (float*)at(9);
    float* part_g = (float*)at(10);
    float* part_u = (float*)at(11);
    float* part_d = (float*)(ws + off_pd);
    // O over att (or over the attention partials, merged per row in the
    // preparation), its partials left; x_mid = x + Σ, normalised and prepared
    if (pa) {
        PrepAttnHost pah = *pa;
        uint32_t Mr = m_rows, Kq = qd;
        void* aops = at(0);
        int* erow = (int*)at(1);
        float* stab = (float*)at(2);
        char pk0[48];
        snprintf(pk0, sizeof pk0, "k_gemm_xh_prep1a_mg%u", po.MG);
        void* pp0[] = {&pah, &Mr, &Kq, &aops, &erow, &stab};
        st = launch(c, pk0, dim3(po.nchunks * 8 * po.MG), dim3(1024), 0, pp0);
    } else {
        st = gemm3_prep(c, po, att, m_rows, qd, at(0), (int*)at(1), (float*)at(2));
    }
    if (st == RT_OK)
        st = gemm3_run(c, po, w_o, at(0), (int*)at(1), fo->has_min ? (float*)at(2) : nullptr,
                       po.splits == 1 ? part_o : x_mid, part_o, m_rows, h, true);
    if (st != RT_OK) return st;
    char pk[48];
    uint32_t M = m_rows, K = h;
    {
        PrepSum ps{part_o, nullptr, x, x_mid, po.splits, crow};
        void* aops = at(3);
        int* erow = (int*)at(4);
        float* stab = (float*)at(5);
        snprintf(pk, sizeof pk, "k_gemm_xh_prep1sn_mg%u", MG);
        void* pp[] = {&ps, &M, &K, &aops, &erow, &stab, (void*)&gamma, &eps};
        st = launch(c, pk, dim3(nch * 8 * MG), dim3(1024), 0, pp);
    }
    // gate and up (one launch where they share a kernel), their partials
    // left; silu(Σ gate)·Σ up prepared for down
    if (st == RT_OK) {
        const Gemm3Job gu[2] = {
            {&pg, w_gate, fg->has_min ? (float*)at(5) : nullptr, part_g, part_g, ff, true, nullptr, nullptr},
            {&pu, w_up, fu->has_min ? (float*)at(5) : nullptr, part_u, part_u, ff, true, nullptr, nullptr}};
        st = gemm3_many(c, gu, 2, at(3), (int*)at(4), m_rows);
    }
    if (st != RT_OK) return st;
    if (m_rows >= c->gemm_block_silu_min) {
        // the SiLU sum in the preparation (one workgroup per row reads the
        // row's partials of gate and up)
        PrepSum ps{part_g, part_u, nullptr, nullptr, pg.splits, crow};
        void* aops = at(6);
        int* erow = (int*)at(7);
        float* stab = (float*)at(8);
        K = ff;
        snprintf(pk, sizeof pk, "k_gemm_xh_prep1s_mg%u", MG);
        void* pp[] = {&ps, &M, &K, &aops, &erow, &stab};
        st = launch(c, pk, dim3(nch * 8 * MG), dim3(1024), 0, pp);
    } else {
        // few rows: the sum over the whole grid into g, then g prepared (8
        // rows of 18944 summed in their 8 preparation workgroups made the 7B
        // verify pass 50-60 µs slower)
        st = gemm_split_sum_ep(c, part_g, part_u, g, m_rows, ff, pg.splits, crow, nullptr, nullptr);
        if (st == RT_OK) st = gemm3_prep(c, pd, g, m_rows, ff, at(6), (int*)at(7), (float*)at(8));
    }
    // down, then x = x_mid + Σ
    if (st == RT_OK)
        st = gemm3_run(c, pd, w_down, at(6), (int*)at(7), fd->has_min ? (float*)at(8) : nullptr,
                       part_d, part_d, m_rows, h, true);
    if (st != RT_OK) return st;
    return gemm_split_sum_ep(c, part_d, nullptr, x, m_rows, h, pd.splits, crow, nullptr, x_mid);
}

int rt_gemm_ffn_block_f32(rt_ctx* c, const char* fmt_o, const void* w_o, const char* fmt_gate,
                          const void* w_gate, const char* fmt_up, const void* w_up,
                          const char* fmt_down, const void* w_down, const float* att, float* x,
                          float* x_mid, const float* gamma, float eps, float* g, float* u,
                          float* xn, uint32_t m_rows, uint32_t h, uint32_t qd, uint32_t ff) {
    return ffn_block_impl(c, fmt_o, w_o, fmt_gate, w_gate, fmt_up, w_up, fmt_down, w_down, att, x,
                          x_mid, gamma, eps, g, u, xn, m_rows, h, qd, ff, false, nullptr, nullptr);
}


// ───────────────────────────── dequant ─────────────────────────────

int rt_dequant_q8_0_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q8_0_f32", in, out, (uint64_t)nb * 32);
}
int rt_dequant_q4_0_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q4_0_f32", in, out, (uint64_t)nb * 32);
}
int rt_dequant_q4k_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q4k_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q6k_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q6k_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q5_0_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q5_0_f32", in, out, (uint64_t)nb * 32);
}
int rt_dequant_q5k_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q5k_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q4_0g_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q4_0g_f32", in, out, (uint64_t)nb * 32);
}
int rt_dequant_q4kg_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q4kg_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q5kg_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q5kg_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q6kg_f32(rt_ctx* c, const void* in, float* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q6kg_f32", in, out, (uint64_t)nb * 256);
}
int rt_dequant_q4k_f16(rt_ctx* c, const void* in, uint16_t* out, uint32_t nb) {
    return elementwise_launch(c, "k_dequant_q4k_f16", in, out, (uint64_t)nb * 256);
}

// ───────────────────────────── argmax ─────────────────────────────

static int argmax_launch(rt_ctx* c, const char* kname, const void* in, uint32_t* res, uint32_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!res || (n && !in))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null buffer", kname);
    void* states = c->aux;
    void* counter = (char*)c->aux + kAuxCounterOff;
    // 1024 elements per workgroup up to 256 workgroups; longer inputs give
    // each workgroup a longer range
    const uint32_t grid = std::max<uint32_t>(1, std::min<uint32_t>(kArgmaxWgs, (n + 1023) / 1024));
    void* params[] = {&in, &res, &n, &states, &counter};
    return launch(c, kname, dim3(grid), dim3(256), 0, params);
}
int rt_argmax_f32(rt_ctx* c, const float* in, uint32_t* res, uint32_t n) {
    return argmax_launch(c, "k_argmax_f32", in, res, n);
}
int rt_argmax_f16(rt_ctx* c, const uint16_t* in, uint32_t* res, uint32_t n) {
    return argmax_launch(c, "k_argmax_f16", in, res, n);
}

// ───────────────────────────── synth ─────────────────────────────

int rt_synth_normal_f32(rt_ctx* c, float* out, uint64_t n, uint64_t seed, float mean, float std) {
    return synth_launch(c, "k_synth_normal_f32", out, n, seed, std, true, mean);
}
int rt_synth_normal_f16(rt_ctx* c, uint16_t* out, uint64_t n, uint64_t seed, float mean,
                        float std) {
    return synth_launch(c, "k_synth_normal_f16", out, n, seed, std, true, mean);
}
int rt_synth_q8_0(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q8_0", out, nb, seed, std, false, 0.0f);
}
int rt_synth_q4_0(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q4_0", out, nb, seed, std, false, 0.0f);
}
int rt_synth_q4k(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q4k", out, nb, seed, std, false, 0.0f);
}
int rt_synth_q6k(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q6k", out, nb, seed, std, false, 0.0f);
}
int rt_synth_q5_0(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q5_0", out, nb, seed, std, false, 0.0f);
}
int rt_synth_q5k(rt_ctx* c, void* out, uint64_t nb, uint64_t seed, float std) {
    return synth_launch(c, "k_synth_q5k", out, nb, seed, std, false, 0.0f);
}

// ───────────────────────────── calibration ─────────────────────────────

int rt_stream_read(rt_ctx* c, const void* src, size_t bytes, uint32_t* sink, size_t sink_dwords) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!src || !sink || bytes % 16)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: stream_read: bad arguments");
    uint32_t grid = (uint32_t)std::min<size_t>(sink_dwords / 4, (size_t)c->cu_count * 8);
    if (grid == 0) return fail(c, RT_ERR_BUFFER_SIZE, "buffer size mismatch: expected 16 bytes, got %zu", sink_dwords * 4);
    uint64_t n16 = bytes / 16;
    void* params[] = {&src, &n16, &sink};
    return launch(c, "k_stream_read", dim3(grid), dim3(256), 0, params);
}

int rt_stream_copy(rt_ctx* c, void* dst, const void* src, size_t bytes) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!src || !dst || bytes % 16)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: stream_copy: bad arguments");
    uint64_t n16 = bytes / 16;
    uint32_t grid = (uint32_t)std::min<uint64_t>((n16 + 255) / 256, (uint64_t)c->cu_count * 8);
    void* params[] = {&src, &dst, &n16};
    return launch(c, "k_stream_copy", dim3(grid), dim3(256), 0, params);
}

}  // extern "C"

// ───────────────────────────── decode-step glue ─────────────────────────────

namespace {

constexpr uint32_t kMaxNormK = 8192;  // whole-K staging limit of the norm-fused GEMVs

// Norm-fused GEMV: whole-K launches fold the norm into the staging; longer K
// runs rms_norm into the workspace, then the plain kernel.
int norm_then(rt_ctx* c, const char* kname, const Fmt& f, GemvArgs a, bool paired,
              const float* gamma, float eps) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!gamma) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: %s: null gamma", kname);
    if (a.K <= kMaxNormK) {
        a.gamma = gamma;
        a.eps = eps;
        return gemv_launch(c, kname, f, a, false, paired);
    }
    // The normalised x sits past the activation-record area at the start of
    // the workspace: a pre-pass of the GEMV writes its records there, and
    // must never overwrite input that other workgroups have not read yet.
    const size_t rec_off = ((size_t)(a.K / 32) * XREC_BYTES + 255) & ~(size_t)255;
    int st = ensure_ws(c, rec_off + (size_t)a.K * sizeof(float), kname);
    if (st != RT_OK) return st;
    float* xn = (float*)((char*)c->ws + rec_off);
    st = rt_rms_norm_f32_f32_f32g(c, (const float*)a.x, xn, gamma, eps, a.K, 1);
    if (st != RT_OK) return st;
    a.x = xn;
    return gemv_launch(c, kname, f, a, false, paired);
}

// Σy² partial sums for the next norm-fused launch (rt_*_ssq): one float per
// row quad of y, by a kernel of their own ...
int ssq_quads(rt_ctx* c, const float* y, uint32_t m, float* ssq) {
    if (!ssq) return RT_OK;
    const uint32_t nq = (m + 3) / 4;
    void* params[] = {&y, &m, &ssq};
    return launch(c, "k_ssq_quads", dim3((nq + 255) / 256), dim3(256), 0, params);
}
// ... unless the launch just made was one whose epilogue writes them (the
// small-launch and VALU small-launch bodies, with a + residual epilogue)
int ssq_after(rt_ctx* c, const float* y, uint32_t m, float* ssq) {
    const std::string n = c->last_name;
    const bool written = (n.size() > 3 && n.compare(n.size() - 3, 3, "_vs") == 0) ||
                         n.find("_sm1") != std::string::npos || n.find("_sm2") != std::string::npos;
    return written ? RT_OK : ssq_quads(c, y, m, ssq);
}

}  // namespace

extern "C" {

int rt_rms_norm_f32_f32_f32g(rt_ctx* c, const float* x, float* y, const float* gamma, float eps,
                             uint32_t hidden, uint32_t num_rows) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (num_rows == 0 || hidden == 0) return RT_OK;
    if (!x || !y || !gamma)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rms_norm: null buffer");
    void* params[] = {&x, &y, &gamma, &eps, &hidden};
    return launch(c, "k_rms_norm_f32g", dim3(num_rows), dim3(256), 0, params);
}

int rt_fused_rope_qk_f32(rt_ctx* c, float* q, float* k, uint32_t head_dim, uint32_t q_heads,
                         uint32_t kv_heads, uint32_t pos, float theta) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (head_dim < 2 || head_dim % 2)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope: head_dim=%u must be even",
                    head_dim);
    const uint32_t heads = q_heads > kv_heads ? q_heads : kv_heads;
    if (heads == 0) return RT_OK;
    if ((q_heads && !q) || (kv_heads && !k))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope: null buffer");
    const uint32_t half = head_dim / 2;
    void* params[] = {&q, &k, &head_dim, &q_heads, &kv_heads, &pos, &theta};
    return launch(c, "k_rope_qk_f32", dim3((half + 63) / 64, heads), dim3(64), 0, params);
}

int rt_kv_copy_to_cache_f32(rt_ctx* c, const float* src, float* dst, uint32_t pos,
                            uint32_t max_seq, uint32_t head_dim, uint32_t num_kv_heads) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    const uint32_t n = head_dim * num_kv_heads;
    if (n == 0) return RT_OK;
    if (!src || !dst) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: kv_copy: null buffer");
    if (pos >= max_seq)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: kv_copy: pos=%u ≥ max_seq=%u", pos,
                    max_seq);
    void* params[] = {&src, &dst, &pos, &max_seq, &head_dim, (void*)&n};
    return launch(c, "k_kv_copy_f32", dim3((n + 255) / 256), dim3(256), 0, params);
}

static int attn_check(rt_ctx* c, uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_dim) {
    if (num_kv_heads == 0 || num_heads % num_kv_heads)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: attention: num_heads=%u not a multiple of "
                    "num_kv_heads=%u", num_heads, num_kv_heads);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: attention: head_dim=%u (supported: 64, 128, 256)",
                    head_dim);
    return RT_OK;
}

// Mirrors the device-side AttnArgs (k_decode.hip).
struct AttnArgs {
    const float* q;
    float* kc;
    float* vc;
    float* out;
    const float* k_new;
    const float* v_new;
    float* part;
    float* ml;
    uint32_t* counters;
    uint32_t kv_len, stride, H, KVH, chunk, pos;
    float scale, theta;
    uint32_t parts_only;
    uint32_t q_len, q_start;
};

// Splits kv_len into ranges of a multiple of 64 positions so that the grid
// holds about two workgroups per CU; sizes the partial-output workspace.
// KV positions per split (a multiple of 64): as many splits as give the
// head groups about two workgroups per CU
static uint32_t attn_chunk(rt_ctx* c, uint32_t kv_len, uint32_t groups, uint32_t max_split_cap = 0) {
    uint32_t max_split = std::max<uint32_t>(1, 2 * c->cu_count / groups);
    if (max_split_cap) max_split = std::min(max_split, max_split_cap);
    const uint32_t n64 = std::max<uint32_t>(1, (kv_len + 63) / 64);
    return (n64 + max_split - 1) / max_split * 64;
}
static uint32_t attn_nsplit(rt_ctx* c, uint32_t kv_len, uint32_t groups) {
    const uint32_t chunk = attn_chunk(c, kv_len, groups);
    return kv_len ? (kv_len + chunk - 1) / chunk : 1;
}

static int attn_launch(rt_ctx* c, const char* kname, AttnArgs a, uint32_t batch,
                       uint32_t max_split_cap = 0, AttnArgs* used = nullptr) {
    const uint32_t hd = strstr(kname, "hd256") ? 256 : strstr(kname, "hd128") ? 128 : 64;
    const uint32_t gm = rt_attn_gm(hd);  // query heads per workgroup, as the kernel's
    const uint32_t G = a.H / a.KVH, HB = (G + gm - 1) / gm;
    const uint32_t groups = batch * a.KVH * HB;
    a.chunk = attn_chunk(c, a.kv_len, groups, max_split_cap);
    const uint32_t nsplit = a.kv_len ? (a.kv_len + a.chunk - 1) / a.chunk : 1;
    if (nsplit > 1 || a.parts_only) {
        if (groups > kAttnCounters)
            return fail(c, RT_ERR_DISPATCH,
                        "kernel dispatch error: attention: %u head groups exceed %u", groups,
                        kAttnCounters);
        const size_t rows = (size_t)batch * a.H * nsplit;
        int st = ensure_ws(c, rows * (hd + 2) * sizeof(float), kname);
        if (st != RT_OK) return st;
        a.part = (float*)c->ws;
        a.ml = a.part + rows * hd;
        a.counters = c->counters;
    }
    if (used) *used = a;
    void* params[] = {&a};
    const uint32_t nt = 256 * rt_attn_hg(hd);  // 256 threads per head group
    // the wave form for the token's RoPE attention at head sizes 64 / 128
    // when no split merge is needed in the launch
    if (c->attn_w && gm == 1 && a.q_len == 0 && (a.parts_only || nsplit == 1) &&
        strncmp(kname, "k_attn_rope_f32_hd", 18) == 0 && (hd == 64 || hd == 128)) {
        char wn[48];
        snprintf(wn, sizeof wn, "k_attn_rope_w_f32_hd%u", hd);
        if (c->fns.count(wn)) return launch(c, wn, dim3(nsplit, a.KVH * HB, batch), dim3(256), 0, params);
    }
    return launch(c, kname, dim3(nsplit, a.KVH * HB, batch), dim3(nt), 0, params);
}

int rt_decode_attention_f32(rt_ctx* c, const float* q, const float* k, const float* v, float* out,
                            uint32_t batch, uint32_t kv_len, uint32_t num_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (batch == 0 || num_heads == 0) return RT_OK;
    int st = attn_check(c, num_heads, num_kv_heads, head_dim);
    if (st != RT_OK) return st;
    if (!q || !k || !v || !out)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: attention: null buffer");
    if (kv_len > kv_head_stride)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: attention: kv_len=%u > kv_head_stride=%u", kv_len,
                    kv_head_stride);
    AttnArgs a{};
    a.q = q;
    a.kc = const_cast<float*>(k);  // read only without rope
    a.vc = const_cast<float*>(v);
    a.out = out;
    a.kv_len = kv_len;
    a.stride = kv_head_stride;
    a.H = num_heads;
    a.KVH = num_kv_heads;
    a.scale = 1.0f / sqrtf((float)head_dim);  // dispatch.rs:1588
    char kn[64];
    snprintf(kn, sizeof kn, "k_decode_attention_f32_hd%u", head_dim);
    return attn_launch(c, kn, a, batch);
}

int rt_decode_attention_rope_f32(rt_ctx* c, const float* q_raw, const float* k_raw,
                                 const float* v_raw, float* k_cache, float* v_cache, float* out,
                                 uint32_t pos, uint32_t max_seq, uint32_t num_heads,
                                 uint32_t num_kv_heads, uint32_t head_dim, float theta) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (num_heads == 0) return RT_OK;
    int st = attn_check(c, num_heads, num_kv_heads, head_dim);
    if (st != RT_OK) return st;
    if (!q_raw || !k_raw || !v_raw || !k_cache || !v_cache || !out)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: attention: null buffer");
    if (pos >= max_seq)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: attention: pos=%u ≥ max_seq=%u",
                    pos, max_seq);
    AttnArgs a{};
    a.q = q_raw;
    a.kc = k_cache;
    a.vc = v_cache;
    a.out = out;
    a.k_new = k_raw;
    a.v_new = v_raw;
    a.kv_len = pos + 1;
    a.stride = max_seq;
    a.H = num_heads;
    a.KVH = num_kv_heads;
    a.pos = pos;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.theta = theta;
    char kn[64];
    snprintf(kn, sizeof kn, "k_attn_rope_f32_hd%u", head_dim);
    return attn_launch(c, kn, a, 1);
}

// Attention (RoPE, KV write) and x_io += W_o·attention as two launches: the
// attention writes every split's (o, m, l) and the projection's staging
// merges them (the attention's own merge without its memory round trips).
// `gkern` is the projection's merging kernel, `max_t` its largest workgroup
// (the staging takes one 4-element slice per thread, so q_dim ≤ 4·max_t);
// `plain` is the unfused projection for the shapes the merged form does not
// take (no KV split, more than 8 splits, or q_dim too long).
typedef int (*GemvAddFn)(rt_ctx*, const void*, const float*, float*, const float*, uint32_t,
                         uint32_t);
static int attention_oproj(rt_ctx* c, const float* q_raw, const float* k_raw, const float* v_raw,
                           float* k_cache, float* v_cache, const void* w_o, float* x_io,
                           uint32_t pos, uint32_t max_seq, uint32_t num_heads,
                           uint32_t num_kv_heads, uint32_t head_dim, float theta, uint32_t hidden,
                           const char* gkern, const Fmt& fmt, uint32_t max_t, GemvAddFn plain,
                           float* ssq = nullptr) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (num_heads == 0 || hidden == 0) return RT_OK;
    int st = attn_check(c, num_heads, num_kv_heads, head_dim);
    if (st != RT_OK) return st;
    if (!q_raw || !k_raw || !v_raw || !k_cache || !v_cache || !w_o || !x_io)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: attention_oproj: null buffer");
    if (pos >= max_seq)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: attention: pos=%u ≥ max_seq=%u",
                    pos, max_seq);
    const uint32_t q_dim = num_heads * head_dim;
    if (!aligned(x_io, 16))
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: attention_oproj: x must be 16-byte aligned");
    if (q_dim % fmt.blk_el != 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: attention_oproj: q_dim=%u must be a multiple of %u (%s)",
                    q_dim, fmt.blk_el, fmt.name);
    // The merged form needs the projection to stage in one slice round and
    // pays off while the attention splits the KV range in 2..8 (one split has
    // no merge to save; more splits than the projection stages would slow the
    // attention down); otherwise: attention, then the GEMV.
    const uint32_t gm = rt_attn_gm(head_dim);  // query heads per attention workgroup
    const uint32_t nsplit0 =
        attn_nsplit(c, pos + 1, num_kv_heads * ((num_heads / num_kv_heads + gm - 1) / gm));
    const bool merged = q_dim % 64 == 0 && q_dim / 32 * 8 <= max_t && nsplit0 >= 2 &&
                        nsplit0 <= kAttnXMaxSplits && c->fns.count(std::string(gkern) + "_r1");
    AttnArgs a{};
    a.q = q_raw;
    a.kc = k_cache;
    a.vc = v_cache;
    a.k_new = k_raw;
    a.v_new = v_raw;
    a.kv_len = pos + 1;
    a.stride = max_seq;
    a.H = num_heads;
    a.KVH = num_kv_heads;
    a.pos = pos;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.theta = theta;
    char kn[64];
    snprintf(kn, sizeof kn, "k_attn_rope_f32_hd%u", head_dim);
    if (!merged) {
        // attention (with its own merge) into a context buffer, then the
        // plain projection
        st = ensure_buf(c, c->attn_out, c->attn_out_bytes, (size_t)q_dim * sizeof(float),
                        "attention_oproj");
        if (st != RT_OK) return st;
        a.out = (float*)c->attn_out;
        st = attn_launch(c, kn, a, 1);
        if (st != RT_OK) return st;
        // (ssq is given by the Q8_0 form only, whose plain projection also
        // writes the partial sums)
        if (ssq)
            return rt_gemv_q8_0_add_f32_f32in_ssq(c, w_o, (const float*)c->attn_out, x_io, x_io,
                                                  hidden, q_dim, ssq);
        return plain(c, w_o, (const float*)c->attn_out, x_io, x_io, hidden, q_dim);
    }
    a.parts_only = 1;
    AttnArgs used{};
    st = attn_launch(c, kn, a, 1, kAttnXMaxSplits, &used);
    if (st != RT_OK) return st;
    const uint32_t nsplit = (a.kv_len + used.chunk - 1) / used.chunk;
    GemvArgs g = plain_args(w_o, used.part, x_io, x_io, hidden, q_dim);
    g.xml = used.ml;
    g.xnsp = nsplit;
    g.xhd = head_dim;
    g.ssq_out = ssq;
    st = gemv_launch(c, gkern, fmt, g, false);
    if (st != RT_OK || !ssq) return st;
    return ssq_after(c, x_io, hidden, ssq);
}

int rt_decode_attention_rope_oproj_q8_0_f32(rt_ctx* c, const float* q_raw, const float* k_raw,
                                            const float* v_raw, float* k_cache, float* v_cache,
                                            const void* w_o, float* x_io, uint32_t pos,
                                            uint32_t max_seq, uint32_t num_heads,
                                            uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                            uint32_t hidden) {
    // (512-thread body: the 0.5B shapes' q_dim = 896 stage in 224 slices)
    return attention_oproj(c, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io, pos, max_seq,
                           num_heads, num_kv_heads, head_dim, theta, hidden,
                           "k_gemv_q8_0_attn_f32add", kQ8_0, 256, rt_gemv_q8_0_add_f32_f32in);
}
int rt_decode_attention_rope_oproj_q4k_f32(rt_ctx* c, const float* q_raw, const float* k_raw,
                                           const float* v_raw, float* k_cache, float* v_cache,
                                           const void* w_o, float* x_io, uint32_t pos,
                                           uint32_t max_seq, uint32_t num_heads,
                                           uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                           uint32_t hidden) {
    return attention_oproj(c, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io, pos, max_seq,
                           num_heads, num_kv_heads, head_dim, theta, hidden,
                           "k_gemv_q4k_attn_f32add", kQ4K, 1024, rt_gemv_q4k_add_f32_f32in);
}
int rt_decode_attention_rope_oproj_q4kg_f32(rt_ctx* c, const float* q_raw, const float* k_raw,
                                            const float* v_raw, float* k_cache, float* v_cache,
                                            const void* w_o, float* x_io, uint32_t pos,
                                            uint32_t max_seq, uint32_t num_heads,
                                            uint32_t num_kv_heads, uint32_t head_dim, float theta,
                                            uint32_t hidden) {
    return attention_oproj(c, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io, pos, max_seq,
                           num_heads, num_kv_heads, head_dim, theta, hidden,
                           "k_gemv_q4kg_attn_f32add", kQ4KG, 1024, rt_gemv_q4kg_add_f32_f32in);
}

// The decode step's RMSNorm factor handed from producer to consumer: the
// producing launches also write Σy² per output row quad, the consuming
// norm-fused launches read those partial sums instead of reducing x.
int rt_gemv_q8_0_add_f32_f32in_ssq(rt_ctx* c, const void* w, const float* x, float* y,
                                   const float* r, uint32_t m, uint32_t k, float* ssq) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!r) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_gemv_q8_0_f32_f32add: null residual");
    GemvArgs a = plain_args(w, x, y, r, m, k);
    a.ssq_out = ssq;
    int st = gemv_launch(c, "k_gemv_q8_0_f32_f32add", kQ8_0, a, false);
    if (st != RT_OK || !ssq || m == 0) return st;
    return ssq_after(c, y, m, ssq);
}
int rt_decode_attention_rope_oproj_q8_0_f32_ssq(rt_ctx* c, const float* q_raw, const float* k_raw,
                                                const float* v_raw, float* k_cache, float* v_cache,
                                                const void* w_o, float* x_io, uint32_t pos,
                                                uint32_t max_seq, uint32_t num_heads,
                                                uint32_t num_kv_heads, uint32_t head_dim,
                                                float theta, uint32_t hidden, float* ssq) {
    return attention_oproj(c, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io, pos, max_seq,
                           num_heads, num_kv_heads, head_dim, theta, hidden,
                           "k_gemv_q8_0_attn_f32add", kQ8_0, 256, rt_gemv_q8_0_add_f32_f32in, ssq);
}
int rt_rms_norm_fused_qkv_bias_q8_0_f32_ssq(rt_ctx* c, const void* wq, const void* wk,
                                            const void* wv, const float* x, const float* gamma,
                                            float eps, float* oq, float* ok, float* ov,
                                            const uint16_t* bq, const uint16_t* bk,
                                            const uint16_t* bv, uint32_t q_dim, uint32_t kv_dim,
                                            uint32_t k, const float* ssq, uint32_t nparts) {
    if (!wq || !wk || !wv || !oq || !ok || !ov || !bq || !bk || !bv)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_qkv_bias_q8_0: null buffer");
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wq; a.w[1] = (const uint8_t*)wk; a.w[2] = (const uint8_t*)wv;
    a.out[0] = oq; a.out[1] = ok; a.out[2] = ov;
    a.aux[0] = bq; a.aux[1] = bk; a.aux[2] = bv;
    a.x = x;
    a.n[0] = q_dim; a.n[1] = kv_dim; a.n[2] = kv_dim;
    a.nvrows = q_dim + 2 * kv_dim;
    a.K = k;
    if (ssq && nparts && nparts <= kMaxSsqParts) {
        a.ssq_in = ssq;
        a.ssq_n = nparts;
    }
    return norm_then(c, "k_qkv_bias_q8_0", kQ8_0, a, false, gamma, eps);
}
int rt_rms_norm_fused_ffn_q8_0_f32_ssq(rt_ctx* c, const void* wg, const void* wu, const float* x,
                                       const float* gamma, float eps, float* act, uint32_t ff,
                                       uint32_t k, const float* ssq, uint32_t nparts) {
    if (!wg || !wu || !act)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_ffn_q8_0: null buffer");
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wg; a.w[1] = (const uint8_t*)wu;
    a.out[0] = act;
    a.x = x;
    a.n[0] = ff; a.n[1] = ff;
    a.nvrows = 2 * ff;
    a.K = k;
    if (ssq && nparts && nparts <= kMaxSsqParts) {
        a.ssq_in = ssq;
        a.ssq_n = nparts;
    }
    return norm_then(c, "k_ffn_q8_0", kQ8_0, a, true, gamma, eps);
}

uint64_t rt_launch_count(const rt_ctx* c) { return c ? c->launches : 0; }
const char* rt_last_launch_name(const rt_ctx* c) { return c ? c->last_name : ""; }

int rt_add_f16_into_f32(rt_ctx* c, const uint16_t* src, float* acc, uint32_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    if (!src || !acc)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: add_f16_into_f32: null buffer");
    void* params[] = {&src, &acc, &n};
    return launch(c, "k_add_f16_into_f32", dim3(std::min<uint32_t>((n + 255) / 256, 1024)),
                  dim3(256), 0, params);
}

// ───────────────────── batched verify / prefill glue ─────────────────────

static uint32_t grid_1d(uint64_t n) {
    return (uint32_t)std::min<uint64_t>((n + 255) / 256, 4096);
}

int rt_add_bias_broadcast_f32(rt_ctx* c, float* x, const uint16_t* bias, uint32_t seq,
                              uint32_t dim) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (seq == 0 || dim == 0) return RT_OK;
    if (!x || !bias)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: add_bias_broadcast: null buffer");
    void* params[] = {&x, &bias, &seq, &dim};
    return launch(c, "k_add_bias_broadcast_f32", dim3(grid_1d((uint64_t)seq * dim)), dim3(256), 0,
                  params);
}

int rt_rope_batch_inplace_f32(rt_ctx* c, float* x, uint32_t head_dim, uint32_t num_heads,
                              uint32_t start_pos, float theta, uint32_t seq) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (head_dim < 2 || head_dim % 2)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_batch: head_dim=%u must be even",
                    head_dim);
    if (seq == 0 || num_heads == 0) return RT_OK;
    if (!x) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_batch: null buffer");
    if (seq > 65535 || num_heads > 65535)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_batch: seq=%u heads=%u > 65535",
                    seq, num_heads);
    void* params[] = {&x, &head_dim, &num_heads, &start_pos, &theta};
    return launch(c, "k_rope_batch_f32", dim3((head_dim / 2 + 63) / 64, num_heads, seq), dim3(64),
                  0, params);
}

int rt_rope_kv_write_batch_f32(rt_ctx* c, float* q, const float* k, const float* v,
                               float* k_cache, float* v_cache, uint32_t head_dim,
                               uint32_t num_heads, uint32_t num_kv_heads, uint32_t start_pos,
                               float theta, uint32_t seq, uint32_t max_seq) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (head_dim < 2 || head_dim % 2)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_kv: head_dim=%u must be even",
                    head_dim);
    const uint32_t heads = std::max(num_heads, num_kv_heads);
    if (seq == 0 || heads == 0) return RT_OK;
    if ((num_heads && !q) || (num_kv_heads && (!k || !v || !k_cache || !v_cache)))
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_kv: null buffer");
    if ((uint64_t)start_pos + seq > max_seq)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: rope_kv: start_pos=%u + seq=%u > max_seq=%u", start_pos,
                    seq, max_seq);
    if (seq > 65535 || heads > 65535)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: rope_kv: seq=%u heads=%u > 65535",
                    seq, heads);
    void* params[] = {&q, (void*)&k, (void*)&v, &k_cache, &v_cache, &head_dim, &num_heads,
                      &num_kv_heads, &start_pos, &theta, &max_seq};
    return launch(c, "k_rope_kv_write_batch_f32", dim3((head_dim / 2 + 63) / 64, heads, seq),
                  dim3(64), 0, params);
}

int rt_kv_write_batch_f32(rt_ctx* c, const float* k, const float* v, float* k_cache,
                          float* v_cache, uint32_t start_pos, uint32_t seq, uint32_t max_seq,
                          uint32_t head_dim, uint32_t num_kv_heads) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    const uint64_t n64 = (uint64_t)seq * num_kv_heads * head_dim;
    if (n64 == 0) return RT_OK;
    if (!k || !v || !k_cache || !v_cache)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: kv_write_batch: null buffer");
    if ((uint64_t)start_pos + seq > max_seq)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: kv_write_batch: start_pos=%u + seq=%u > max_seq=%u",
                    start_pos, seq, max_seq);
    if (n64 > 0xFFFFFFFFull)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: kv_write_batch: too many elements");
    const uint32_t n = (uint32_t)n64;
    void* params[] = {&k, &v, &k_cache, &v_cache, &start_pos, &max_seq, &head_dim, &num_kv_heads,
                      (void*)&n};
    return launch(c, "k_kv_write_batch_f32", dim3((n + 255) / 256), dim3(256), 0, params);
}

int rt_add_f32(rt_ctx* c, const float* a, const float* b, float* out, uint32_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    if (!a || !b || !out) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: add: null buffer");
    void* params[] = {&a, &b, &out, &n};
    return launch(c, "k_add_f32", dim3(grid_1d(n)), dim3(256), 0, params);
}

int rt_silu_mul_f32(rt_ctx* c, const float* gate, const float* up, float* out, uint32_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (n == 0) return RT_OK;
    if (!gate || !up || !out)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: silu_mul: null buffer");
    void* params[] = {&gate, &up, &out, &n};
    return launch(c, "k_silu_mul_f32", dim3(grid_1d(n)), dim3(256), 0, params);
}

int rt_argmax_rows_first_f32(rt_ctx* c, const float* in, uint32_t* result, uint32_t rows,
                             uint32_t n) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (rows == 0) return RT_OK;
    if (!in || !result)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: argmax_rows: null buffer");
    if (rows > kAttnCounters || rows > 65535)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: argmax_rows: rows=%u > %u", rows,
                    std::min<uint32_t>(kAttnCounters, 65535));
    // ranges of ≥ 4096 elements, at most 64 per row
    const uint32_t G = std::max<uint32_t>(1, std::min<uint32_t>(64, (n + 4095) / 4096));
    int st = ensure_ws(c, (size_t)rows * G * 8, "argmax_rows");
    if (st != RT_OK) return st;
    void* states = c->ws;
    uint32_t* counters = c->counters;
    void* params[] = {(void*)&in, &result, &n, &states, &counters};
    return launch(c, "k_argmax_rows_first_f32", dim3(G, rows), dim3(256), 0, params);
}


// The multi-query attention on the matrix cores (k_attn_mq_f32_hd*): plan and
// launch; kLsDecline where the per-row kernel is the better one.  in_part:
// the split partials in the context's second scratch buffer (c->part) instead
// of the workspace; parts_only: no merge in the launch (declined when the
// plan has a single key range), the partials' layout returned in *pa.
static int attn_mq_launch(rt_ctx* c, AttnArgs a, uint32_t batch, uint32_t q_len, uint32_t kv_len,
                          uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_dim,
                          uint32_t q_start, uint32_t min_pairs, bool in_part, bool parts_only,
                          PrepAttnHost* pa) {
    char kn[64];
    snprintf(kn, sizeof kn, "k_attn_mq_f32_hd%u", head_dim);
    // up to min_pairs column groups the per-row kernel below.  Alone
    // (rt_flash_attention_f32) up to 8 (7B at 2 rows: 14.3 against 10.2 µs,
    // 0.5B at 4 rows 9.5 against 8.9; at 8 groups even); with the range
    // merge in the O preparation none (0.5B at 8 rows 1583 -> 1521 µs per
    // verify pass, 7B at 4 rows 3510 -> 3418 µs)
    const uint64_t mq_pairs = ((uint64_t)q_len * (num_heads / num_kv_heads) + 15) / 16 * num_kv_heads * batch;
    if (c->attn_mq && c->fns.count(kn) && mq_pairs > min_pairs) {
        // workgroups of 16 (row, head) columns per KV head and range of key
        // tiles.  Fewer than 256 column groups (verify): the key range split
        // so that the grid holds about 1024 waves of 4 per range, ranges of
        // at least 4 tiles, at most RT_ATTN_MQ_NSP_MAX of them (the last
        // workgroup of a group merges them).  Otherwise (prefill) one range,
        // W waves doubled while the grid stays under 4096 waves and each
        // wave keeps 2 tiles of the longest range.
        const uint32_t G = num_heads / num_kv_heads;
        const uint64_t cols = ((uint64_t)q_len * G + 15) / 16;
        const uint64_t pairs = cols * num_kv_heads * batch;
        const uint32_t tiles = (std::min<uint32_t>(kv_len, q_start + q_len) + 15) / 16;
        const uint32_t wmax = rt_attn_mq_wmax(head_dim);
        uint32_t nsp = 1;
        if (pairs < 256)
            nsp = std::max<uint32_t>(1, std::min<uint32_t>({(uint32_t)(256 / pairs), tiles / 4,
                                                            RT_ATTN_MQ_NSP_MAX}));
        if (c->attn_mq_nsp) nsp = std::min({c->attn_mq_nsp, tiles, RT_ATTN_MQ_NSP_MAX});
        const uint32_t chunk = (tiles + nsp - 1) / nsp;
        nsp = (tiles + chunk - 1) / chunk;
        uint32_t w = 1;
        if (nsp > 1)
            while (w < 4 && w * 2 <= chunk) w *= 2;
        else
            while (w < wmax && w * 2 * pairs <= 4096 && w * 4 <= chunk) w *= 2;
        if (c->attn_mq_w) w = std::min(c->attn_mq_w, wmax);
        if (cols * nsp > 0x7FFFFFFFull || batch > 65535)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: flash_attention: %llu column "
                        "groups, batch %u", (unsigned long long)cols, batch);
        if (parts_only && nsp == 1) return kLsDecline;
        if (nsp > 1) {
            if (pairs > kAttnCounters)
                return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: flash_attention: %llu "
                            "column groups exceed %u", (unsigned long long)pairs, kAttnCounters);
            const size_t parts = (size_t)pairs * nsp * 16;
            const size_t bytes = parts * (head_dim + 2) * sizeof(float);
            int st = in_part ? ensure_part(c, bytes, kn) : ensure_ws(c, bytes, kn);
            if (st != RT_OK) return st;
            a.part = (float*)(in_part ? c->part : c->ws);
            a.ml = a.part + parts * head_dim;
            a.counters = c->counters;
            a.parts_only = parts_only ? 1u : 0u;
            if (pa) *pa = PrepAttnHost{a.part, a.ml, nsp, num_heads / num_kv_heads, head_dim,
                                       (uint32_t)cols};
        }
        a.chunk = chunk;
        void* params[] = {&a};
        return launch(c, kn, dim3((uint32_t)(cols * nsp), num_kv_heads, batch), dim3(64 * w),
                      rt_attn_mq_lds(head_dim, w), params);
    }
    return kLsDecline;
}

int rt_gemm_attn_ffn_block_f32(rt_ctx* c, const float* q, const float* k_cache,
                               const float* v_cache, uint32_t kv_len, uint32_t num_heads,
                               uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride,
                               uint32_t q_start, float* att, const char* fmt_o, const void* w_o,
                               const char* fmt_gate, const void* w_gate, const char* fmt_up,
                               const void* w_up, const char* fmt_down, const void* w_down, float* x,
                               float* x_mid, const float* gamma, float eps, float* g, float* u,
                               float* xn, uint32_t m_rows, uint32_t h, uint32_t ff) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (m_rows == 0) return RT_OK;
    const uint32_t qd = num_heads * head_dim;
    // the attention's split partials merged in the O projection's operand
    // preparation, where the FFN block takes its shared form and the
    // attention its multi-range matrix-core form
    bool shared = false;
    int st = RT_OK;
    if (c->attn_fold && q && k_cache && v_cache && num_kv_heads && num_heads % num_kv_heads == 0 &&
        kv_len >= 1 && kv_len <= kv_head_stride && aligned(q, 16) &&
        attn_check(c, num_heads, num_kv_heads, head_dim) == RT_OK) {
        st = ffn_block_impl(c, fmt_o, w_o, fmt_gate, w_gate, fmt_up, w_up, fmt_down, w_down, att, x,
                            x_mid, gamma, eps, g, u, xn, m_rows, h, qd, ff, true, &shared, nullptr);
        if (st != RT_OK) return st;
    }
    if (shared) {
        AttnArgs a{};
        a.q = q;
        a.kc = const_cast<float*>(k_cache);
        a.vc = const_cast<float*>(v_cache);
        a.out = att;
        a.kv_len = kv_len;
        a.stride = kv_head_stride;
        a.H = num_heads;
        a.KVH = num_kv_heads;
        a.scale = 1.0f / sqrtf((float)head_dim);  // dispatch.rs:659
        a.q_len = m_rows;
        a.q_start = q_start;
        PrepAttnHost pa{};
        st = attn_mq_launch(c, a, 1, m_rows, kv_len, num_heads, num_kv_heads, head_dim, q_start,
                            c->attn_mq_fold_min, true, true, &pa);
        if (st == RT_OK)
            return ffn_block_impl(c, fmt_o, w_o, fmt_gate, w_gate, fmt_up, w_up, fmt_down, w_down,
                                  att, x, x_mid, gamma, eps, g, u, xn, m_rows, h, qd, ff, false,
                                  nullptr, &pa);
        if (st != kLsDecline) return st;
    }
    st = rt_flash_attention_f32(c, q, k_cache, v_cache, att, 1, m_rows, kv_len, num_heads,
                                num_kv_heads, head_dim, kv_head_stride, q_start);
    if (st != RT_OK) return st;
    return rt_gemm_ffn_block_f32(c, fmt_o, w_o, fmt_gate, w_gate, fmt_up, w_up, fmt_down, w_down,
                                 att, x, x_mid, gamma, eps, g, u, xn, m_rows, h, qd, ff);
}

int rt_flash_attention_f32(rt_ctx* c, const float* q, const float* k, const float* v, float* out,
                           uint32_t batch, uint32_t q_len, uint32_t kv_len, uint32_t num_heads,
                           uint32_t num_kv_heads, uint32_t head_dim, uint32_t kv_head_stride,
                           uint32_t q_start) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (batch == 0 || q_len == 0 || num_heads == 0) return RT_OK;
    int st = attn_check(c, num_heads, num_kv_heads, head_dim);
    if (st != RT_OK) return st;
    if (!q || !k || !v || !out)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: flash_attention: null buffer");
    if (kv_len == 0 || kv_len > kv_head_stride)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: flash_attention: kv_len=%u (need 1..kv_head_stride=%u)",
                    kv_len, kv_head_stride);
    const uint64_t rows = (uint64_t)batch * q_len;
    if (rows > 65535)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: flash_attention: batch·q_len=%llu > 65535",
                    (unsigned long long)rows);
    AttnArgs a{};
    a.q = q;
    a.kc = const_cast<float*>(k);  // read only without rope
    a.vc = const_cast<float*>(v);
    a.out = out;
    a.kv_len = kv_len;
    a.stride = kv_head_stride;
    a.H = num_heads;
    a.KVH = num_kv_heads;
    a.scale = 1.0f / sqrtf((float)head_dim);  // dispatch.rs:659
    a.q_len = q_len;
    a.q_start = q_start;
    char kn[64];
    const int mq = attn_mq_launch(c, a, batch, q_len, kv_len, num_heads, num_kv_heads, head_dim,
                                  q_start, c->attn_mq_min, false, false, nullptr);
    if (mq != kLsDecline) return mq;
    snprintf(kn, sizeof kn, "k_decode_attention_f32_hd%u", head_dim);
    return attn_launch(c, kn, a, (uint32_t)rows);
}

static int embed_launch(rt_ctx* c, const char* kname, uint32_t blk_el, const void* table,
                        const uint32_t* token, float* out, uint32_t k, uint32_t rows = 1) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (k == 0 || rows == 0) return RT_OK;
    if (k % blk_el)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: embed: k=%u not a multiple of %u",
                    k, blk_el);
    if (!table || !token || !out)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: embed: null buffer");
    if (rows > 65535)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: embed: rows=%u > 65535", rows);
    void* params[] = {&table, &token, &out, &k};
    return launch(c, kname, dim3((k + 255) / 256, rows), dim3(256), 0, params);
}
#define RT_EMBED_ENTRY(NAME, EL)                                                               \
    int rt_embed_##NAME##_f32(rt_ctx* c, const void* table, const uint32_t* token, float* out,  \
                              uint32_t k) {                                                    \
        return embed_launch(c, "k_embed_" #NAME "_f32", EL, table, token, out, k);             \
    }                                                                                          \
    int rt_embed_rows_##NAME##_f32(rt_ctx* c, const void* table, const uint32_t* tokens,        \
                                   float* out, uint32_t k, uint32_t rows) {                    \
        return embed_launch(c, "k_embed_" #NAME "_f32", EL, table, tokens, out, k, rows);      \
    }
RT_EMBED_ENTRY(q8_0, 32)
RT_EMBED_ENTRY(q4_0, 32)
RT_EMBED_ENTRY(q4k, 256)
RT_EMBED_ENTRY(q6k, 256)
RT_EMBED_ENTRY(q5_0, 32)
RT_EMBED_ENTRY(q5k, 256)
RT_EMBED_ENTRY(q4_0g, 32)
RT_EMBED_ENTRY(q4kg, 256)
RT_EMBED_ENTRY(q5kg, 256)
RT_EMBED_ENTRY(q6kg, 256)
RT_EMBED_ENTRY(f16, 1)
RT_EMBED_ENTRY(f32, 1)

int rt_rms_norm_fused_qkv_bias_q8_0_f32(rt_ctx* c, const void* wq, const void* wk, const void* wv,
                                        const float* x, const float* gamma, float eps, float* oq,
                                        float* ok, float* ov, const uint16_t* bq,
                                        const uint16_t* bk, const uint16_t* bv, uint32_t q_dim,
                                        uint32_t kv_dim, uint32_t k) {
    if (!wq || !wk || !wv || !oq || !ok || !ov || !bq || !bk || !bv)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_qkv_bias_q8_0: null buffer");
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wq; a.w[1] = (const uint8_t*)wk; a.w[2] = (const uint8_t*)wv;
    a.out[0] = oq; a.out[1] = ok; a.out[2] = ov;
    a.aux[0] = bq; a.aux[1] = bk; a.aux[2] = bv;
    a.x = x;
    a.n[0] = q_dim; a.n[1] = kv_dim; a.n[2] = kv_dim;
    a.nvrows = q_dim + 2 * kv_dim;
    a.K = k;
    return norm_then(c, "k_qkv_bias_q8_0", kQ8_0, a, false, gamma, eps);
}

int rt_rms_norm_fused_ffn_q8_0_f32(rt_ctx* c, const void* wg, const void* wu, const float* x,
                                   const float* gamma, float eps, float* act, uint32_t ff,
                                   uint32_t k) {
    if (!wg || !wu || !act)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_ffn_q8_0: null buffer");
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wg; a.w[1] = (const uint8_t*)wu;
    a.out[0] = act;
    a.x = x;
    a.n[0] = ff; a.n[1] = ff;
    a.nvrows = 2 * ff;
    a.K = k;
    return norm_then(c, "k_ffn_q8_0", kQ8_0, a, true, gamma, eps);
}

int rt_rms_norm_fused_qkv_bias_q4k_q6k_f32(rt_ctx* c, const void* wq, const void* wk,
                                           const void* wv, const float* x, const float* gamma,
                                           float eps, float* oq, float* ok, float* ov,
                                           const uint16_t* bq, const uint16_t* bk,
                                           const uint16_t* bv, uint32_t q_dim, uint32_t kv_dim,
                                           uint32_t k) {
    if (!gamma)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_qkv2_bias_q4k_q6k: null gamma");
    return qkv_pair_launch(c, "k_qkv2_bias_q4k_q6k", "k_qkv2_q4k_q6k", kQ4K, kQ6KU, wq, wk, wv,
                           x, oq, ok, ov, bq, bk, bv, q_dim, kv_dim, k, gamma, eps);
}
int rt_rms_norm_fused_ffn_q4k_f32(rt_ctx* c, const void* wg, const void* wu, const float* x,
                                  const float* gamma, float eps, float* act, uint32_t ff,
                                  uint32_t k) {
    if (!wg || !wu || !act)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: k_ffn_q4k: null buffer");
    GemvArgs a{};
    a.w[0] = (const uint8_t*)wg; a.w[1] = (const uint8_t*)wu;
    a.out[0] = act;
    a.x = x;
    a.n[0] = ff; a.n[1] = ff;
    a.nvrows = 2 * ff;
    a.K = k;
    return norm_then(c, "k_ffn_q4k", kQ4K, a, true, gamma, eps);
}
int rt_rms_norm_gemv_q6k_f32in_f32out(rt_ctx* c, const void* w, const float* x,
                                      const float* gamma, float eps, float* y, uint32_t m,
                                      uint32_t k) {
    return norm_then(c, "k_gemv_q6k_f32_f32", kQ6K, plain_args(w, x, y, nullptr, m, k), false,
                     gamma, eps);
}
int rt_rms_norm_gemv_q8_0_f32in_f32out(rt_ctx* c, const void* w, const float* x,
                                       const float* gamma, float eps, float* y, uint32_t m,
                                       uint32_t k) {
    return norm_then(c, "k_gemv_q8_0_f32_f32", kQ8_0, plain_args(w, x, y, nullptr, m, k), false,
                     gamma, eps);
}

}  // extern "C"

// ───────────────────────────── persistent decode step ─────────────────────────────

namespace {

// Mirrors the device-side StepPhase / StepSync (k_step.hip).
struct StepPhaseH {
    uint32_t kind, n0, n1, n2;
    const void* p0;
    const void* p1;
    void* p2;
    uint64_t pad;
    GemvArgs g;
    AttnArgs at;
};
static_assert(sizeof(StepPhaseH) == RT_STEP_PHASE_BYTES, "StepPhase layout");
constexpr size_t kStepSyncBytes = RT_STEP_SYNC_BYTES;
constexpr uint32_t kStepThreads = RT_STEP_THREADS;
enum : uint32_t { SK_EMBED_Q8_0 = 0, SK_QKV_Q8_0 = 1, SK_ATTN_HD64 = 2, SK_OPROJ_Q8_0 = 3,
                  SK_FFN_Q8_0 = 4, SK_DOWN_Q8_0 = 5 };

// Matrix-core GEMV phase on a persistent grid of G workgroups × T threads:
// whole K staged per workgroup, no K split through memory.  The waves that
// share a row-quad group (ksw) split its K steps; ksw is chosen for the
// fewest items per wave (all of which are then in flight before the grid
// barrier), then for the most workgroups with work.
GemvArgs step_gemv_args(const Fmt& f, uint32_t nvrows, uint32_t K, uint32_t G, uint32_t T) {
    GemvArgs a{};
    a.nvrows = nvrows;
    a.K = K;
    a.lpr = 16;
    a.row_bytes = (uint64_t)(K / f.blk_el) * f.blk_bytes;
    const uint32_t units = K / f.mq_units();
    a.ksplit = 1;
    a.kc_units = units;
    a.xb_chunk = K / 32;
    const uint32_t nwaves = T / 64, nsteps = (units + 15) / 16;
    uint32_t best = 0, best_cost = ~0u, best_tiles = 0;
    for (uint32_t ksw = 1; ksw <= nwaves; ksw *= 2) {
        const uint32_t rows_per_wg = (nwaves / ksw) * 4;
        const uint32_t ntiles = (nvrows + rows_per_wg - 1) / rows_per_wg;
        const uint32_t rounds = (ntiles + G - 1) / G;
        const uint32_t spw = (nsteps + ksw - 1) / ksw;
        const uint32_t cost = rounds * spw;
        const uint32_t used = std::min(ntiles, G);
        if (cost < best_cost || (cost == best_cost && used > best_tiles)) {
            best = ksw; best_cost = cost; best_tiles = used;
        }
    }
    a.ksw = best;
    return a;
}
size_t step_gemv_lds(uint32_t K) { return (size_t)(K / 32) * XREC_BYTES + 16 * 2 * 4 * sizeof(float); }

}  // namespace

extern "C" {

int rt_decode_step_q8_0_create(rt_ctx* c, const rt_step_model* m, uint32_t pos, rt_step** out) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!m || !out || !m->layer || !m->token_embd || !m->lm_head || !m->output_norm || !m->token ||
        !m->logits)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: decode_step: null argument");
    const uint32_t L = m->layers, h = m->hidden, H = m->heads, KVH = m->kv_heads, hd = m->head_dim;
    const uint32_t ff = m->ff, qd = H * hd, kvd = KVH * hd;
    if (hd != 64 || H == 0 || KVH == 0 || H % KVH || L == 0)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: decode_step: head_dim %u, heads %u / %u (built for "
                    "head size 64, heads a multiple of the KV heads)", hd, H, KVH);
    if (h % 64 || ff % 64 || qd % 64 || qd / 32 * 8 > kStepThreads || ff / 32 * 8 > 4 * kStepThreads)
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: decode_step: hidden %u / ff %u / q_dim %u must be "
                    "multiples of 64 within one staging pass", h, ff, qd);
    if (pos >= m->max_seq)
        return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: decode_step: pos=%u ≥ max_seq=%u",
                    pos, m->max_seq);
    for (uint32_t l = 0; l < L; ++l) {
        const rt_step_layer& y = m->layer[l];
        if (!y.wq || !y.wk || !y.wv || !y.wo || !y.wg || !y.wu || !y.wd || !y.bq || !y.bk || !y.bv ||
            !y.attn_norm || !y.ffn_norm || !y.k_cache || !y.v_cache)
            return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: decode_step: layer %u: null buffer", l);
    }
    // one workgroup per CU, all resident (the grid barrier needs every
    // workgroup running at once)
    const uint32_t G = std::min<uint32_t>((uint32_t)c->cu_count, RT_STEP_MAX_WGS);
    // attention splits: ≤ 8 (the O projection's staging merges ≤ 8), ≥ 64
    // positions each
    const uint32_t kv_len = pos + 1;
    const uint32_t nsp = std::min<uint32_t>(kAttnXMaxSplits, (kv_len + 63) / 64);
    const uint32_t chunk = ((kv_len + nsp - 1) / nsp + 63) / 64 * 64;
    const uint32_t nsp_used = (kv_len + chunk - 1) / chunk;
    const uint32_t gm = rt_step_attn_gm(hd), HB = (H / KVH + gm - 1) / gm;
    // activation buffers, each on its own 256-byte lines, fresh for every
    // phase of the step
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t b_h = al(4 * h), b_q = al(4 * qd), b_kv = al(4 * kvd), b_ff = al(4 * ff);
    const size_t b_part = al(4 * (size_t)H * nsp_used * hd), b_ml = al(8 * (size_t)H * nsp_used);
    const size_t per_layer = b_q + 2 * b_kv + b_part + b_ml + b_h + b_ff + b_h;
    const size_t acts_bytes = b_h + (size_t)L * per_layer;
    rt_step* st = new rt_step();
    auto cleanup = [&](int code) {
        if (st->phases) hipFree(st->phases);
        if (st->sync) hipFree(st->sync);
        if (st->acts) hipFree(st->acts);
        delete st;
        return code;
    };
    hipError_t e = hipMalloc(&st->acts, acts_bytes);
    if (e == hipSuccess) e = hipMalloc(&st->sync, kStepSyncBytes);
    if (e == hipSuccess) e = hipMemset(st->sync, 0, kStepSyncBytes);
    if (e != hipSuccess) return cleanup(hip_fail(c, e, "decode_step buffers"));
    char* ap = (char*)st->acts;
    auto take = [&](size_t b) { char* p = ap; ap += b; return (float*)p; };
    std::vector<StepPhaseH> ph;
    size_t lds = 0;
    float* x = take(b_h);
    {
        StepPhaseH p{};
        p.kind = SK_EMBED_Q8_0;
        p.n0 = h;
        p.p0 = m->token_embd;
        p.p1 = m->token;
        p.p2 = x;
        ph.push_back(p);
    }
    for (uint32_t l = 0; l < L; ++l) {
        const rt_step_layer& y = m->layer[l];
        float* q = take(b_q);
        float* k = take(b_kv);
        float* v = take(b_kv);
        float* part = take(b_part);
        float* ml = take(b_ml);
        float* x1 = take(b_h);
        float* act = take(b_ff);
        float* x2 = take(b_h);
        StepPhaseH p{};
        // RMSNorm + Q/K/V + bias
        p.kind = SK_QKV_Q8_0;
        p.g = step_gemv_args(kQ8_0, qd + 2 * kvd, h, G, kStepThreads);
        p.g.w[0] = (const uint8_t*)y.wq; p.g.w[1] = (const uint8_t*)y.wk; p.g.w[2] = (const uint8_t*)y.wv;
        p.g.out[0] = q; p.g.out[1] = k; p.g.out[2] = v;
        p.g.aux[0] = y.bq; p.g.aux[1] = y.bk; p.g.aux[2] = y.bv;
        p.g.n[0] = qd; p.g.n[1] = kvd; p.g.n[2] = kvd;
        p.g.x = x;
        p.g.gamma = y.attn_norm;
        p.g.eps = m->eps;
        lds = std::max(lds, step_gemv_lds(h));
        ph.push_back(p);
        // RoPE + KV write + split attention (partials only)
        p = StepPhaseH{};
        p.kind = SK_ATTN_HD64;
        p.n0 = nsp_used;
        p.n1 = KVH * HB;
        p.at.q = q; p.at.kc = y.k_cache; p.at.vc = y.v_cache; p.at.out = nullptr;
        p.at.k_new = k; p.at.v_new = v; p.at.part = part; p.at.ml = ml;
        p.at.kv_len = kv_len; p.at.stride = m->max_seq; p.at.H = H; p.at.KVH = KVH;
        p.at.chunk = chunk; p.at.pos = pos;
        p.at.scale = 1.0f / sqrtf((float)hd);
        p.at.theta = m->theta;
        p.at.parts_only = 1;
        ph.push_back(p);
        // O (staging merges the partials) + residual
        p = StepPhaseH{};
        p.kind = SK_OPROJ_Q8_0;
        p.g = step_gemv_args(kQ8_0, h, qd, G, kStepThreads);
        p.g.w[0] = (const uint8_t*)y.wo;
        p.g.out[0] = x1;
        p.g.aux[0] = x;
        p.g.n[0] = h;
        p.g.x = part;
        p.g.xml = ml;
        p.g.xnsp = nsp_used;
        p.g.xhd = hd;
        lds = std::max(lds, step_gemv_lds(qd));
        ph.push_back(p);
        // RMSNorm + gate/up + SiLU
        p = StepPhaseH{};
        p.kind = SK_FFN_Q8_0;
        p.g = step_gemv_args(kQ8_0, 2 * ff, h, G, kStepThreads);
        p.g.w[0] = (const uint8_t*)y.wg; p.g.w[1] = (const uint8_t*)y.wu;
        p.g.out[0] = act;
        p.g.n[0] = ff; p.g.n[1] = ff;
        p.g.x = x1;
        p.g.gamma = y.ffn_norm;
        p.g.eps = m->eps;
        ph.push_back(p);
        // down + residual
        p = StepPhaseH{};
        p.kind = SK_DOWN_Q8_0;
        p.g = step_gemv_args(kQ8_0, h, ff, G, kStepThreads);
        p.g.w[0] = (const uint8_t*)y.wd;
        p.g.out[0] = x2;
        p.g.aux[0] = x1;
        p.g.n[0] = h;
        p.g.x = act;
        lds = std::max(lds, step_gemv_lds(ff));
        ph.push_back(p);
        x = x2;
    }
    // occupancy: one workgroup of kStepThreads per CU must fit
    if (occupancy(c, "k_decode_step_q8_0", kStepThreads, lds) < 1)
        return cleanup(fail(c, RT_ERR_DISPATCH,
                            "kernel dispatch error: decode_step: %zu bytes of LDS leave no "
                            "resident workgroup", lds));
    e = hipMalloc(&st->phases, ph.size() * sizeof(StepPhaseH));
    if (e == hipSuccess)
        e = hipMemcpy(st->phases, ph.data(), ph.size() * sizeof(StepPhaseH), hipMemcpyHostToDevice);
    if (e != hipSuccess) return cleanup(hip_fail(c, e, "decode_step phases"));
    st->nph = (uint32_t)ph.size();
    st->grid = G;
    st->lds = lds;
    st->lm_head = m->lm_head;
    st->final_norm = m->output_norm;
    st->x_final = x;
    st->logits = m->logits;
    st->token = m->token;
    st->vocab = m->vocab;
    st->hidden = h;
    st->eps = m->eps;
    *out = st;
    return RT_OK;
}

int rt_decode_step_run(rt_ctx* c, rt_step* st) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!st) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: decode_step: null step");
    void* params[] = {&st->phases, &st->nph, &st->sync};
    int rc = launch(c, "k_decode_step_q8_0", dim3(st->grid), dim3(kStepThreads), st->lds, params);
    if (rc != RT_OK) return rc;
    rc = rt_rms_norm_gemv_q8_0_f32in_f32out(c, st->lm_head, st->x_final, st->final_norm, st->eps,
                                            st->logits, st->vocab, st->hidden);
    if (rc != RT_OK) return rc;
    return rt_argmax_f32(c, st->logits, st->token, st->vocab);
}

int rt_decode_step_status(rt_ctx* c, rt_step* st) {
    if (!c) return fail(nullptr, RT_ERR_DISPATCH, "kernel dispatch error: null context");
    if (!st) return fail(c, RT_ERR_DISPATCH, "kernel dispatch error: decode_step: null step");
    int rc = rt_flush(c);
    if (rc != RT_OK) return rc;
    uint32_t status = 0;
    hipError_t e = hipMemcpy(&status, (char*)st->sync + RT_STEP_STATUS_OFF, 4,
                             hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "decode_step status");
    if (status) {
        // reported once: cleared so that the next runs report their own
        // outcome (the token of the run that timed out is not valid)
        const uint32_t zero = 0;
        e = hipMemcpy((char*)st->sync + RT_STEP_STATUS_OFF, &zero, 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(c, e, "decode_step status reset");
        return fail(c, RT_ERR_DISPATCH,
                    "kernel dispatch error: decode_step: a grid barrier timed out (workgroups "
                    "not all resident?)");
    }
    return RT_OK;
}

void rt_decode_step_destroy(rt_step* st) {
    if (!st) return;
    if (st->phases) hipFree(st->phases);
    if (st->sync) hipFree(st->sync);
    if (st->acts) hipFree(st->acts);
    delete st;
}

}  // extern "C"
