/*
 * oracle.h — CPU restatement of RunIT's quantized-GEMV decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (runit_mac_amd/) links,
 * imports or calls this code; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py do, and only as the checker / CPU baseline.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the RunIT_Mac repository).  Compiled with -ffp-contract=off so every f32
 * product/difference rounds exactly as the reference's Rust code does.
 */
#ifndef RUNIT_ORACLE_H
#define RUNIT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORA_Q8_0 = 0, ORA_Q4_0 = 1, ORA_Q4K = 2, ORA_Q6K = 3, ORA_Q5_0 = 4, ORA_Q5K = 5,
    /* ggml layouts of the same blocks (upstream GGUF files) */
    ORA_Q4_0G = 6, ORA_Q4KG = 7, ORA_Q5KG = 8, ORA_Q6KG = 9
};

/* half 2.7.1 crate (Cargo.lock): f16::to_f32 (exact) and f16::from_f32
 * (IEEE binary16, round to nearest even) — used at forward.rs:958,577. */
float ora_h2f(uint16_t h);
uint16_t ora_f2h(float f);

/* Block geometry (crates/gguf/src/types.rs:158-191). */
size_t ora_block_elems(int fmt);
size_t ora_block_bytes(int fmt);

/* Dequantisers to f32. */
void ora_dequant_q8_0(const uint8_t* in, size_t nblk, float* out); /* forward.rs:951-963 */
void ora_dequant_q4_0(const uint8_t* in, size_t nblk, float* out); /* forward.rs:964-978 */
void ora_dequant_q4k(const uint8_t* in, size_t nblk, float* out);  /* forward.rs:1026-1057, 359-369 */
void ora_dequant_q6k(const uint8_t* in, size_t nblk, float* out);  /* forward.rs:921-950 */
void ora_dequant_q5_0(const uint8_t* in, size_t nblk, float* out); /* forward.rs:900-920 */
void ora_dequant_q5k(const uint8_t* in, size_t nblk, float* out);  /* forward.rs:979-1012, 359-369 */
/* ggml layouts, restated from ggml's published decoders (ggml-quants.c
 * dequantize_row_q4_0 / _q4_K / _q5_K / _q6_K; no copy of ggml is vendored
 * in the reference, which documents the divergence at docs/STATUS_REPORT.md:184):
 *   Q4_0: element j < 16 = low nibble of qs[j], 16 + j = high nibble;
 *   Q4_K: chunk j of 64 uses sub-blocks 2j, 2j+1 (get_scale_min_k4 packing);
 *   Q5_K: as Q4_K, fifth bit = bit 2j (low) / 2j+1 (high) of qh[l];
 *   Q6_K: element h + 32t + l uses sc[h/16 + l/16 + 2t]. */
void ora_dequant_q4_0g(const uint8_t* in, size_t nblk, float* out);
void ora_dequant_q4kg(const uint8_t* in, size_t nblk, float* out);
void ora_dequant_q5kg(const uint8_t* in, size_t nblk, float* out);
void ora_dequant_q6kg(const uint8_t* in, size_t nblk, float* out);
void ora_dequant(int fmt, const uint8_t* in, size_t nblk, float* out);
/* dequant.metal:53-98 — Q4_K → f16 (f32 value, then RNE to half). */
void ora_dequant_q4k_f16(const uint8_t* in, size_t nblk, uint16_t* out);

/* cpu_gemv (crates/kernels/src/dispatch.rs:1705-1709) on packed weights,
 * rows dequantised one at a time, accumulated in f64 (precedent:
 * crates/engine/src/bin/test_gemv.rs:110-115).  Also returns the per-row
 * tolerance base sabs[r] = Σ_k |w[r,k]·x[k]|.  x is m_vec × k (row-major),
 * y and sabs are m_vec × n. */
void ora_gemv_packed(int fmt, const uint8_t* w, const float* x, size_t m_vec, size_t n,
                     size_t k, double* y, double* sabs);

/* The reference's CPU path as it runs (f32): dequantise a row
 * (forward.rs decoders) then cpu_gemv's sequential f32 sum
 * (dispatch.rs:1705-1709).  Used as the timed CPU baseline; threads > 1 splits
 * rows over OpenMP threads (the reference itself is single-threaded). */
void ora_gemv_ref_f32(int fmt, const uint8_t* w, const float* x, size_t n, size_t k, float* y,
                      int threads);

/* cpu_silu (dispatch.rs:1684-1686) in f64. */
double ora_silu(double x);

/* greedy_argmax_f32 (crates/engine/src/sampler.rs:111-116): Rust max_by
 * with partial_cmp().unwrap_or(Equal) — last maximal index, NaN = Equal,
 * n == 0 → 0. */
uint32_t ora_argmax_f32(const float* v, size_t n);

/* cpu_rms_norm (dispatch.rs:1699-1702) / rms_norm_f32_f32_f32g in f64:
 * y = x / sqrt(mean(x²) + eps) · γ, per row of `hidden`. */
void ora_rms_norm(const float* x, const float* gamma, double eps, size_t hidden, size_t rows,
                  double* y);

/* fused_rope_qk_f32 (fused_rope.metal:28-55) on one vector of `heads` heads,
 * in place (f64 data).  The angle is formed exactly as the kernel forms it in
 * f32 — freq = 1/powf(θ, (2d)/hd), angle = f32(pos)·freq — and the rotation is
 * evaluated in f64. */
void ora_rope(double* v, size_t heads, size_t head_dim, uint32_t pos, float theta);

/* rope_batch_inplace_f16 (rope.metal:92-121) on f64 data [seq][heads][hd]:
 * row s at position start_pos + s, angle = f32(pos) / powf(θ, (2d)/hd) formed
 * in f32 as the kernel forms it (a division, unlike ora_rope), the rotation
 * in f64. */
void ora_rope_batch(double* v, size_t seq, size_t heads, size_t head_dim, uint32_t start_pos,
                    float theta);

/* The per-row argmax of verify_draft (forward.rs:2283-2293): best = 0,
 * best_val = −inf; for j in row: if v[j] > best_val {best = j; best_val = v[j]}
 * — the first maximal index; NaN never compares greater. */
void ora_argmax_rows_first_f32(const float* v, size_t rows, size_t n, uint32_t* out);

/* Decode attention (attention.metal:248-308; cpu_attention dispatch.rs:
 * 1712-1742 generalised to GQA): per query head h, kv head h/(H/KVH),
 * softmax(q·k_j · scale) · v over j < kv_len, in f64.  K/V: [kvh][stride][hd]. */
void ora_attention(const double* q, const float* k, const float* v, size_t num_heads,
                   size_t num_kv_heads, size_t head_dim, size_t kv_len, size_t kv_stride,
                   double scale, double* out);

/* One greedy decode step of a Qwen2-shape model as the reference's CPU
 * helpers compute it, in f32 (the timed CPU baseline): embedding row
 * dequantised (forward.rs:1494-1505); per layer cpu_rms_norm
 * (dispatch.rs:1699-1702), Q/K/V by dequantise-row + cpu_gemv's sequential
 * f32 sum (dispatch.rs:1705-1709) plus the f16 bias (fused_qkv.metal:68),
 * RoPE on (d, d + hd/2) pairs (fused_rope.metal:28-55), the new K/V row
 * written to the cache at pos (kv_copy_to_cache), softmax attention over
 * pos + 1 positions with GQA head h → kv head h/(H/KVH) (cpu_attention
 * dispatch.rs:1712-1742), o_proj + residual, cpu_rms_norm, gate/up GEMVs,
 * cpu_silu_mul (dispatch.rs:1684-1690), down + residual; final norm, LM head,
 * greedy_argmax_f32.  `threads` splits GEMV rows over OpenMP threads (the
 * reference's CPU code is single-threaded: threads = 1).  Updates the KV
 * caches; writes the logits; returns the greedy token. */
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd; /* packed blocks, formats below */
    const uint16_t *bq, *bk, *bv;                     /* f16 biases */
    const float *attn_norm, *ffn_norm;
    float *kc, *vc;                                   /* [kv_heads][max_seq][head_dim] */
    int32_t fq, fk, fv, fo, fg, fu, fd;               /* ORA_* formats */
} ora_layer_t;
typedef struct {
    uint32_t layers, hidden, heads, kv_heads, head_dim, ff, vocab, max_seq;
    float eps, theta;
    const ora_layer_t* layer;
    const float* final_norm;
    const uint8_t* embd; /* [vocab][hidden] in format f_embd */
    const uint8_t* lm_head;
    int32_t f_lm, f_embd;
} ora_model_t;
uint32_t ora_decode_step_ref_f32(const ora_model_t* m, uint32_t token, uint32_t pos,
                                 float* logits, int threads);

/* Seeded synthetic data with the same definitions as the device generators
 * (splitmix64 → Box–Muller), used to build golden fixtures on the CPU. */
float ora_synth_normal(uint64_t seed, uint64_t idx);
/* out[i] = mean + stdv·N(seed, i), i < n (f32 arithmetic). */
void ora_synth_normal_f32(uint64_t seed, uint64_t n, float mean, float stdv, float* out);
/* nblk blocks of fmt (reference layouts: Q8_0, Q4_0, Q4_K, Q6_K, Q5_0, Q5_K)
 * from w_i = stdv·N(seed, i), exactly as the device generators build them. */
void ora_synth_weights(int fmt, uint64_t seed, float stdv, size_t nblk, uint8_t* out);
void ora_quantize_q8_0(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q4_0(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q4k(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q6k(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q5_0(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q5k(const float* w, size_t nblk, uint8_t* out);
/* Test data in the ggml layouts: the reference-layout quantiser's blocks
 * re-laid out value for value (Q6_K: the odd scale slots, unused by the
 * reference layout, get a value near their even neighbour). */
void ora_quantize_q4_0g(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q4kg(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q5kg(const float* w, size_t nblk, uint8_t* out);
void ora_quantize_q6kg(const float* w, size_t nblk, uint8_t* out);
/* Re-layout one block stream from the reference layout to ggml's (fmt =
 * ORA_Q4_0 / ORA_Q4K / ORA_Q5K), values preserved. */
void ora_relayout_to_ggml(int fmt, const uint8_t* in, size_t nblk, uint8_t* out);

#ifdef __cplusplus
}
#endif
#endif
