/*
 * oracle.h - CPU restatement of Sulimo's Q4_0 prefill path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (sulimo_amd/) links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker and as the timed CPU baseline.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the Sulimo source tree). The arithmetic order of the reference is kept:
 * fp32 sequential sums where the reference sums sequentially, the AVX2 lane
 * order where the reference uses AVX2, IEEE binary16 round-to-nearest-even for
 * every f32->f16 conversion (the `half` 2.7.1 crate's from_f32), and glibc libm
 * for exp/pow/sin/cos/sqrt/round (Rust's f32 methods call the same functions).
 * Compiled with -ffp-contract=off so that no a*b+c is fused unless the
 * reference itself fuses it (_mm256_fmadd_ps).
 *
 * Parity pins (what checks each function; see tests/test_oracle_*.py):
 *   q4_0 repack/dequant      - brute force over all 256 byte values x scales,
 *                              and the repack.rs:137-179 known-answer pattern
 *   q8_0 quantize            - closed-form special cases (zero block, .5 ties,
 *                              +-amax -> +-127, f16-subnormal scale), numpy's
 *                              independent float16 conversion, kv_cache.rs:216-234
 *   gemm scalar reference    - float64 textbook X @ dequant(W)^T, test_gemm.rs patterns
 *   q4_0 x q8_0 dot (scalar, avx2) - exact integer identity, avx2.rs:352-396 pattern
 *   rmsnorm / rope / softmax / swiglu - closed forms and invariants (unit RMS,
 *                              rotation norm, complex-multiply form, silu(0)=0)
 *   attention                - float64 brute-force softmax(QK^T/sqrt(d))V
 *   forward_token, prefill   - float64 textbook transformer on tiny models
 */
#ifndef SULIMO_ORACLE_H
#define SULIMO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 helpers (IEEE binary16, RNE) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- Q4_0 format (crates/sulimo-core/src/repack.rs) ---- */
int64_t orc_repack_q4_0_aos_to_soa(const uint8_t *aos, size_t aos_len, uint8_t *scales,
                                   size_t scales_len, uint8_t *quants, size_t quants_len);
void orc_dequant_q4_0_aos(const uint8_t *aos, size_t nblocks, float *out);
void orc_dequant_q4_0_soa(const uint8_t *scales, const uint8_t *quants, size_t nblocks,
                          float *out);

/* ---- Q8_0 format (crates/sulimo-core/src/kv_cache.rs) ---- */
void orc_quantize_f32_to_q8_0(const float *src, size_t n, uint8_t *dst);
void orc_dequant_q8_0(const uint8_t *src, size_t nblocks, float *dst);

/* ---- GEMM scalar reference (crates/sulimo-ocl/src/gemm.rs:106-147) ----
 * Reference naming: m = output features, k = inputs, n = tokens. */
void orc_gemm_q4_0_f16_scalar_reference(const uint16_t *scales, const uint8_t *quants,
                                        const uint16_t *x, size_t m, size_t k, size_t n,
                                        uint16_t *out);

/* ---- CPU kernels (crates/sulimo-cpu/src/scalar.rs, avx2.rs) ---- */
float orc_vec_dot_q4_0_q8_0_scalar(const uint8_t *w_scales, const uint8_t *w_quants,
                                   const uint8_t *x_q8, size_t nblocks);
float orc_vec_dot_q4_0_q8_0_avx2(const uint8_t *w_scales, const uint8_t *w_quants,
                                 const uint8_t *x_q8, size_t nblocks);
void orc_matvec_q4_0_q8_0_avx2(const uint8_t *w_scales, const uint8_t *w_quants,
                               const uint8_t *x_q8, size_t rows, size_t cols, float *out);
void orc_rmsnorm_scalar(const float *x, const float *w, float eps, size_t n, float *out);
void orc_rmsnorm_avx2(const float *x, const float *w, float eps, size_t n, float *out);
void orc_rope_head_scalar(float *vec, size_t pos, size_t rope_dim, float freq_base, int mode);
void orc_softmax_scalar(float *x, size_t n);
void orc_swiglu_scalar(const float *gate, const float *up, size_t n, float *out);
/* causal_gqa_decode_scalar_ext (scalar.rs:287-359) over a Q8_0 ring: key j of the
 * context is absolute position first_pos + j, stored at slot (first_pos+j) % capacity.
 * first_pos = 0 reproduces the reference's get_k(p) closure exactly. */
void orc_causal_gqa_decode_scalar(const float *q, const uint8_t *k_ring, const uint8_t *v_ring,
                                  size_t bytes_per_pos, size_t capacity, size_t first_pos,
                                  size_t context_len, size_t head_count, size_t head_count_kv,
                                  size_t head_dim, float *scores_buf, float *dequant_buf,
                                  float *out);

/* ---- Reference GPU kernels restated on the CPU (kernels/prefill.cl) ---- */
void orc_cl_rmsnorm_f16_f32w(const uint16_t *x, const float *w, uint16_t *out, int d, float eps,
                             int n);
void orc_cl_rope_f16(uint16_t *vec, int head_count, int head_dim, int rope_dim, float freq_base,
                     int mode, int start_pos, int n);
void orc_cl_kv_store_q8_0(const uint16_t *act, uint8_t *kv, int start_pos, int capacity,
                          int blocks_per_pos, int n);
void orc_cl_silu_mul_f16(const uint16_t *gate, const uint16_t *up, uint16_t *out, int total);
void orc_cl_add_f16(uint16_t *a, const uint16_t *b, int total);
void orc_cl_logits_f16_output(const uint16_t *x_all, const uint16_t *scales,
                              const uint8_t *quants, float *logits, int m, int k, int token_idx);
/* Attention of prefill.cl:120-237 with the CPU twin's fp32 accumulation
 * (scalar.rs:287-359): query n (absolute position start_pos+n) attends to the last
 * min(start_pos+n+1, capacity) positions, each read once at slot p % capacity. */
void orc_attention_prefill_f32(const float *q, const uint8_t *k_ring, const uint8_t *v_ring,
                               float *out, int start_pos, int capacity, int head_count,
                               int head_count_kv, int head_dim, int n);

/* ---- Host embedding gather (crates/sulimo-engine/src/scheduler.rs:329-374) ---- */
void orc_lookup_token_embedding_f16(const uint8_t *scales, const uint8_t *quants, size_t embd,
                                    uint32_t token, uint16_t *out);

/* ---- Whole-model paths ---- */
typedef struct {
  int32_t n_layers, embd, ffn, n_head, n_head_kv, head_dim, rope_dim, vocab;
  float rope_base, eps;
  int32_t rope_mode; /* 0 = Norm (Llama), 1 = NeoX (Qwen2) */
} orc_config;

typedef struct {
  const uint8_t *scales; /* f16 [rows * cols/32] */
  const uint8_t *quants; /* u8 [rows * cols/32 * 16] */
} orc_q4;

typedef struct {
  const float *attn_norm;
  orc_q4 q, k, v, o;
  const float *ffn_norm;
  orc_q4 gate, up, down;
  /* optional (NULL when absent), forward_pass.rs:250-272: f32 q/k/v biases added to
   * the projections, f32 [head_dim] RMSNorm weights applied per head of q and k
   * before RoPE (apply_head_norms, forward_pass.rs:466-491) */
  const float *q_bias, *k_bias, *v_bias;
  const float *q_norm, *k_norm;
} orc_layer;

typedef struct {
  orc_config cfg;
  orc_q4 token_embd;
  const float *output_norm;
  orc_q4 output;
  const orc_layer *layers;
} orc_model;

/* Q8_0 ring KV cache, layout of kv_cache.rs:27-90: per layer [capacity][kv_dim/32][34 B]. */
typedef struct {
  uint8_t **k; /* n_layers pointers */
  uint8_t **v;
  size_t capacity;
} orc_kv;

/* forward_token (crates/sulimo-engine/src/forward_pass.rs:190-417), Llama/Qwen2
 * graph with the optional q/k/v biases and QK-norm (no post-norm tensors). Writes
 * vocab logits.
 * Returns 0, or -1 when a scratch allocation fails. */
int orc_forward_token(const orc_model *m, orc_kv *kv, uint32_t token, size_t pos, float *logits);
int orc_forward_token_mt(const orc_model *m, orc_kv *kv, uint32_t token, size_t pos, float *logits,
                         int threads);

/* fp32 reference prefill in the device op order of execute_prefill_ubatch
 * (crates/sulimo-ocl/src/prefill.rs:362-560) with the rounding points of the
 * reference's own CPU oracle (crates/sulimo-ocl/tests/test_prefill.rs:582-885):
 * f32 residual, f16 at every GEMM input and output, RoPE in f32, K quantized to
 * Q8_0 from the rotated f32 values, V from the f16 GEMM output, f32 attention.
 * Optional biases are added to the f32 GEMM result before its f16 rounding; the
 * optional QK-norm runs in f32 on the rounded q/k heads before RoPE.
 * x_in: f16 [n][embd] token embeddings. Attention is a sliding window of the
 * last `capacity` positions; new K/V are committed to the ring after attention.
 * logits: f32 [vocab] of token n-1, or [n][vocab] when all_logits != 0.
 * h_final (optional): f32 [n][embd] output-normed hidden states.
 * x_final (optional): f32 [n][embd] residual stream after the last layer (the input of
 * the output norm). */
int orc_prefill_reference(const orc_model *m, orc_kv *kv, const uint16_t *x_in, size_t start_pos,
                          size_t n, int all_logits, float *logits, float *h_final, float *x_final);

#ifdef __cplusplus
}
#endif
#endif
