/*
 * sulimo_hip.h - C ABI of libsulimo_hip.so, the MI355X (gfx950) prefill backend
 * for the Sulimo engine. It takes the place of the `sulimo-ocl` crate behind
 * `sulimo-engine`'s prefill interface.
 *
 * Every entry point names the reference item it replaces (paths relative to the
 * Sulimo source tree). Conventions:
 *   - Status: int32_t, 0 = ok, negative = one of SULIMO_HIP_ERR_* (the OclError
 *     variants, crates/sulimo-ocl/src/program.rs:27-40, plus INVALID_ARGUMENT for
 *     the reference's assert! preconditions, which panic there). The message of
 *     the last failure on the calling thread is in sulimo_hip_last_error().
 *   - Host pointers are borrowed, never freed, and never retained past the call
 *     except the host mirror given to sulimo_hip_buffer_create.
 *   - GEMM naming follows the reference: m = output features, k = input
 *     features, n = tokens. Activations are row-major [n][k] f16; outputs [n][m].
 *   - Q4_0 weights are the loader's SoA split (crates/sulimo-core/src/loader.rs:141-160):
 *     scales f16[m * k/32], quants u8[m * k/32 * 16]; element i of a block is the low
 *     nibble of byte i, element i+16 its high nibble, weight = (q - 8) * d.
 *     The first GEMM that reads a (scales, quants) pair builds a device copy in the
 *     GEMM's own layout (the same 18 bytes per 32 weights), kept until the quants
 *     buffer is released; a write through this library to either buffer (upload or
 *     a kernel output) makes the next GEMM rebuild it.
 *   - Q8_0 KV ring per layer (crates/sulimo-core/src/kv_cache.rs:27-90):
 *     [capacity][kv_dim/32] blocks of 34 bytes (f16 scale + 32 int8 codes).
 *   - enqueue_* calls are asynchronous on the context's single in-order stream;
 *     sulimo_hip_wait() blocks the caller without spinning.
 *   - One context is driven by one engine thread at a time (not re-entrant).
 */
#ifndef SULIMO_HIP_H
#define SULIMO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (OclError, crates/sulimo-ocl/src/program.rs:27-40) ---- */
#define SULIMO_HIP_OK 0
#define SULIMO_HIP_ERR_DEVICE_NOT_FOUND (-1) /* OclError::DeviceNotFound */
#define SULIMO_HIP_ERR_DRIVER (-2)           /* OclError::Driver */
#define SULIMO_HIP_ERR_BUILD_FAILED (-3)     /* OclError::BuildFailed: no gfx950 code object */
#define SULIMO_HIP_ERR_ZERO_COPY (-4)        /* OclError::ZeroCopyViolation: host mirror mismatch */
#define SULIMO_HIP_ERR_EXECUTION_FAILED (-5) /* OclError::ExecutionFailed */
#define SULIMO_HIP_ERR_IO (-6)               /* OclError::Io */
#define SULIMO_HIP_ERR_INVALID_ARGUMENT (-7) /* a reference assert! precondition failed */

typedef struct sulimo_hip_ctx sulimo_hip_ctx;
typedef struct sulimo_hip_buffer sulimo_hip_buffer;

/* OclDeviceInfo (crates/sulimo-ocl/src/probe.rs:9-34), HIP fields. */
typedef struct {
  char device_name[256];
  char arch_name[64]; /* e.g. "gfx950:sramecc+:xnack-" */
  char driver_version[64];
  int32_t device_index;
  int32_t compute_units;
  int32_t clock_khz;
  int32_t wavefront_size;
  size_t global_mem_bytes;
  size_t lds_bytes_per_block;
  int32_t host_unified_memory; /* 0 on MI355X: every transfer is explicit */
  int32_t has_fp16;            /* always 1 on gfx950 */
} sulimo_hip_device_info;

/* OclProbeResult (probe.rs:47-60): available != 0 and info filled, or reason set. */
typedef struct {
  int32_t available;
  sulimo_hip_device_info info;
  char reason[256];
} sulimo_hip_probe_result;

/* GemmProfile (crates/sulimo-ocl/src/gemm.rs:14-19). */
typedef struct {
  double duration_seconds; /* GPU time of the launch (hipEvent) */
  double gflops;           /* 2*m*n*k / duration */
  const char *kernel_variant;
} sulimo_hip_gemm_profile;

/* ---- context (crates/sulimo-ocl/src/program.rs) ---- */

/* OclContext::get_or_init (program.rs:79-87): one process-wide context per device. */
int32_t sulimo_hip_get_or_init(int32_t device, sulimo_hip_ctx **out);
/* OclContext::new (program.rs:94-216): a private context with its own stream. */
int32_t sulimo_hip_context_new(int32_t device, sulimo_hip_ctx **out);
/* Drop of a context from sulimo_hip_context_new (the shared one is never freed). */
int32_t sulimo_hip_context_release(sulimo_hip_ctx *ctx);
/* OclContext::finish (program.rs:89-92). */
int32_t sulimo_hip_finish(sulimo_hip_ctx *ctx);
/* ctx.device_info (program.rs:52-70). */
int32_t sulimo_hip_get_device_info(const sulimo_hip_ctx *ctx, sulimo_hip_device_info *out);
/* probe() (probe.rs:62-208): never fails; reports why no device is usable. */
int32_t sulimo_hip_probe(sulimo_hip_probe_result *out);
/* Message of the last failure on this thread ("" if none). */
const char *sulimo_hip_last_error(void);

/* ---- buffers (crates/sulimo-ocl/src/buffer.rs) ---- */

/* OclBuffer::from_host_ptr (buffer.rs:42-115). MI355X memory is discrete, so the
 * buffer is an HBM allocation of `bytes` that mirrors `host_ptr` (may be NULL for a
 * device-only buffer): the host contents are uploaded at creation, and map_read /
 * the *_sync_* calls copy between the two. The zero-copy alignment asserts of the
 * reference (4096-aligned pointer, size % 64) have no purpose here and are not
 * required. bytes == 0 is SULIMO_HIP_ERR_INVALID_ARGUMENT. */
int32_t sulimo_hip_buffer_create(sulimo_hip_ctx *ctx, void *host_ptr, size_t bytes,
                                 int32_t read_only, sulimo_hip_buffer **out);
/* Drop (buffer.rs:163-172). NULL is a no-op. */
int32_t sulimo_hip_buffer_release(sulimo_hip_buffer *buf);
/* active_cl_mem_count (buffer.rs:21-23). */
size_t sulimo_hip_active_buffer_count(void);
size_t sulimo_hip_buffer_size(const sulimo_hip_buffer *buf);
void *sulimo_hip_buffer_device_ptr(const sulimo_hip_buffer *buf);
void *sulimo_hip_buffer_host_ptr(const sulimo_hip_buffer *buf);
/* Host writes that the zero-copy buffer made visible implicitly (engine.rs:241-257
 * writes scratch.x): copy host -> device, ordered on the context stream. */
int32_t sulimo_hip_buffer_upload(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf, size_t offset,
                                 size_t bytes, const void *src);
/* Blocking device -> host copy after all queued work (a CL_TRUE map). */
int32_t sulimo_hip_buffer_download(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *buf,
                                   size_t offset, size_t bytes, void *dst);
/* OclBuffer::map_read (buffer.rs:128-145): waits for queued work, copies the whole
 * buffer into its host mirror and returns the mirror. ZERO_COPY error if the buffer
 * has no host mirror. */
int32_t sulimo_hip_buffer_map_read(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf,
                                   const void **mapped);
/* OclBuffer::unmap (buffer.rs:148-160). */
int32_t sulimo_hip_buffer_unmap(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf, const void *mapped);

/* ---- per-op enqueue (crates/sulimo-ocl/src/prefill.rs:67-330) ---- */

/* enqueue_gemm_q4_0_f16 (prefill.rs:69-105), kernels/gemm_q4_0.cl:13-58:
 * out[n][m] = f16( sum_b d[m][b] * sum_i x[n][32b+i] * (q[m][32b+i]-8) ), f32 accumulate.
 * Requires k % 32 == 0 and m % 8 == 0 (gemm.rs:39-40). */
int32_t sulimo_hip_enqueue_gemm_q4_0_f16(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                         const sulimo_hip_buffer *quants,
                                         const sulimo_hip_buffer *x, sulimo_hip_buffer *out,
                                         size_t m, size_t k, size_t n);
/* No counterpart in the reference: sulimo_hip_enqueue_gemm_q4_0_f16 for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, preconditions and result; it
 * calls no hipMalloc/hipFree and does not build or use the cached GEMM-layout copy of
 * the weights. Instead it rebuilds that layout, and keeps its K-split partial sums,
 * in a static device array of 64 MiB that every GPU the library runs on holds until
 * the process ends. Matrices whose layout exceeds it (m * k * 18/32 bytes, rounded up
 * to 32 rows and 64 columns) are rejected with SULIMO_HIP_ERR_INVALID_ARGUMENT. All
 * calls on one GPU share that array, so the library orders them: each call's stream
 * first waits for an event the previous no-alloc call on that GPU recorded, from
 * whichever context or thread it came. Calls from two streams therefore run one after
 * the other, never at once. */
int32_t sulimo_hip_enqueue_gemm_q4_0_f16_noalloc(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                                 const sulimo_hip_buffer *quants,
                                                 const sulimo_hip_buffer *x, sulimo_hip_buffer *out,
                                                 size_t m, size_t k, size_t n);
/* enqueue_rmsnorm (prefill.rs:108-135), prefill.cl:4-29: x f16 [n][d], w f32 [d]. */
int32_t sulimo_hip_enqueue_rmsnorm(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *x,
                                   const sulimo_hip_buffer *w, sulimo_hip_buffer *out, size_t d,
                                   float eps, size_t n);
/* enqueue_rope (prefill.rs:139-173), prefill.cl:32-68: in place on f16
 * [n][head_count][head_dim]; mode 0 = Norm (Llama), 1 = NeoX (Qwen2). */
int32_t sulimo_hip_enqueue_rope(sulimo_hip_ctx *ctx, sulimo_hip_buffer *vec, size_t head_count,
                                size_t head_dim, size_t rope_dim, float freq_base, int32_t mode,
                                size_t start_pos, size_t n);
/* enqueue_kv_store (prefill.rs:176-205), prefill.cl:72-116: quantizes f16
 * [n][blocks_per_pos*32] to Q8_0 at ring slots (start_pos+t) % capacity. Codes and
 * scales are bit-identical to quantize_f32_to_q8_0 (kv_cache.rs:162-193). */
int32_t sulimo_hip_enqueue_kv_store(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *act,
                                    sulimo_hip_buffer *kv_cache, size_t start_pos,
                                    size_t capacity, size_t blocks_per_pos, size_t n);
/* enqueue_attention_prefill (prefill.rs:209-248), prefill.cl:120-237: q f16
 * [n][head_count][head_dim]; query t (position start_pos+t) attends to the last
 * min(start_pos+t+1, capacity) positions read from the rings at slot p % capacity;
 * softmax and the output sum are f32 (the CPU twin, scalar.rs:287-359); out f16.
 * Requires head_dim % 32 == 0 and head_count % head_count_kv == 0. */
int32_t sulimo_hip_enqueue_attention_prefill(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *q,
                                             const sulimo_hip_buffer *k_cache,
                                             const sulimo_hip_buffer *v_cache,
                                             sulimo_hip_buffer *out, size_t start_pos,
                                             size_t capacity, size_t head_count,
                                             size_t head_count_kv, size_t head_dim, size_t n);
/* enqueue_silu_mul (prefill.rs:251-273), prefill.cl:240-253. */
int32_t sulimo_hip_enqueue_silu_mul(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *gate,
                                    const sulimo_hip_buffer *up, sulimo_hip_buffer *out,
                                    size_t total_elements);
/* enqueue_add (prefill.rs:276-296), prefill.cl:256-266: a = f16(a + b). */
int32_t sulimo_hip_enqueue_add(sulimo_hip_ctx *ctx, sulimo_hip_buffer *a,
                               const sulimo_hip_buffer *b, size_t total_elements);
/* enqueue_logits_final (prefill.rs:300-330), prefill.cl:269-308: f32 logits of
 * row token_idx of x_all f16 [*][embd_dim]. */
int32_t sulimo_hip_enqueue_logits_final(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *x_all,
                                        const sulimo_hip_buffer *scales,
                                        const sulimo_hip_buffer *quants, sulimo_hip_buffer *logits,
                                        size_t vocab_size, size_t embd_dim, size_t token_idx);
/* wait_event_zero_spin (crates/sulimo-ocl/src/waiter.rs:39-82): blocks until the
 * stream drains. The calling thread sleeps on a condition variable that a HIP host
 * function queued behind the work signals (the reference's event callback + park);
 * it does not spin while the GPU runs. Reports an
 * asynchronous kernel failure as SULIMO_HIP_ERR_EXECUTION_FAILED. */
int32_t sulimo_hip_wait(sulimo_hip_ctx *ctx);
/* gemm_q4_0_f16 (crates/sulimo-ocl/src/gemm.rs:28-102): one GEMM, waited, timed. */
int32_t sulimo_hip_gemm_q4_0_f16(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                 const sulimo_hip_buffer *quants, const sulimo_hip_buffer *x,
                                 sulimo_hip_buffer *out, size_t m, size_t k, size_t n,
                                 sulimo_hip_gemm_profile *profile);

/* ---- whole-ubatch prefill (crates/sulimo-ocl/src/prefill.rs:14-65, 337-566) ---- */

/* The ModelConfig fields execute_prefill_ubatch reads (prefill.rs:346-359). */
typedef struct {
  int32_t n_layers;    /* block_count */
  int32_t embd;        /* embedding_length */
  int32_t ffn;         /* feed_forward_length */
  int32_t n_head;      /* head_count */
  int32_t n_head_kv;   /* head_count_kv */
  int32_t head_dim;    /* head_dim */
  int32_t rope_dim;    /* rope_dimension_count */
  int32_t vocab;       /* vocab_size */
  float rope_base;     /* rope_freq_base */
  float eps;           /* rms_epsilon */
  int32_t rope_mode;   /* 0 = Norm (ModelArch::Llama), 1 = NeoX (Qwen2 and others) */
} sulimo_hip_model_config;

/* OclLayerTensors (prefill.rs:15-32). */
typedef struct {
  sulimo_hip_buffer *attn_norm; /* f32 [embd] */
  sulimo_hip_buffer *attn_q_scales, *attn_q_quants;
  sulimo_hip_buffer *attn_k_scales, *attn_k_quants;
  sulimo_hip_buffer *attn_v_scales, *attn_v_quants;
  sulimo_hip_buffer *attn_out_scales, *attn_out_quants;
  sulimo_hip_buffer *ffn_norm; /* f32 [embd] */
  sulimo_hip_buffer *ffn_gate_scales, *ffn_gate_quants;
  sulimo_hip_buffer *ffn_up_scales, *ffn_up_quants;
  sulimo_hip_buffer *ffn_down_scales, *ffn_down_quants;
  /* Optional tensors of the CPU path (forward_pass.rs:250-272), NULL when absent;
   * the reference's GPU path has none (prefill.rs:15-32): */
  sulimo_hip_buffer *attn_q_bias, *attn_k_bias, *attn_v_bias; /* f32 [q_dim], [kv_dim], [kv_dim] */
  sulimo_hip_buffer *attn_q_norm, *attn_k_norm;               /* f32 [head_dim] QK-norm weights */
} sulimo_hip_layer_tensors;

/* OclModelTensors (prefill.rs:35-40). */
typedef struct {
  sulimo_hip_buffer *output_norm; /* f32 [embd] */
  sulimo_hip_buffer *output_scales, *output_quants;
  const sulimo_hip_layer_tensors *layers;
  int32_t n_layers;
} sulimo_hip_model_tensors;

/* OclKvCache (prefill.rs:43-49): one K and one V buffer per layer. */
typedef struct {
  sulimo_hip_buffer *const *k_buffers;
  sulimo_hip_buffer *const *v_buffers;
  int32_t n_layers;
  size_t capacity;
  size_t head_count_kv;
  size_t head_dim;
} sulimo_hip_kv_cache;

/* OclPrefillScratch (prefill.rs:52-65). Sizes as scheduler.rs:190-206 (f16 unless
 * stated). On return x holds the final residual stream (f16), h the output-normed
 * hidden states of all n tokens, logits the f32 logits of token n-1.
 * q/k/v/attn_out/ffn_* are used as intermediates. */
typedef struct {
  sulimo_hip_buffer *x, *h, *q, *k, *v, *attn_out;
  sulimo_hip_buffer *ffn_gate, *ffn_up, *ffn_swiglu, *ffn_down;
  sulimo_hip_buffer *logits; /* f32 [vocab] */
  size_t max_n;
} sulimo_hip_prefill_scratch;

/* execute_prefill_ubatch (prefill.rs:337-566): all layers of one micro-batch of n
 * tokens at positions start_pos.. on the context stream, then one blocking wait.
 * scratch.x must hold the n f16 token embeddings (sulimo_hip_embed_tokens or an
 * upload). Optional biases are added to the q/k/v GEMM results before their f16
 * rounding, and the optional QK-norm (per-head RMSNorm, eps = cfg.eps) runs on q and
 * k before RoPE, as forward_token does. Differences from the reference, all
 * documented in the design notes:
 * the residual stream is kept in f32 between the kernels; when the ubatch wraps
 * the ring (start_pos+n > capacity), each query sees exactly the last `capacity`
 * positions (new K/V are staged and committed to the ring after attention). */
int32_t sulimo_hip_execute_prefill_ubatch(sulimo_hip_ctx *ctx, const sulimo_hip_model_config *cfg,
                                          const sulimo_hip_model_tensors *tensors,
                                          sulimo_hip_kv_cache *kv_cache,
                                          sulimo_hip_prefill_scratch *scratch, size_t start_pos,
                                          size_t n);

/* Optional outputs and switches of a prefill for validation (no reference
 * counterpart; the engine's CPU prefill computes logits for every token,
 * engine.rs:287-319). */
typedef struct {
  sulimo_hip_buffer *logits_all; /* f32 [n][vocab], or NULL */
  sulimo_hip_buffer *argmax_all; /* int32 [n] per-position top-1 token, or NULL */
  /* Nonzero: every op of prefill.rs:362-536 runs as its own kernel, as the reference
   * enqueues them: the q/k/v, o, gate, up and down GEMMs store f16, followed by the
   * separate RoPE + Q8_0 store, SwiGLU, residual add and RMSNorm kernels, instead of
   * those steps running in GEMM epilogues and the K-split reduction. The arithmetic
   * of each step is the same; scratch.ffn_gate, ffn_up and ffn_down (f16 [n][ffn],
   * [n][ffn], [n][embd]) must then be given. */
  int32_t unfused;
} sulimo_hip_prefill_outputs;

/* execute_prefill_ubatch plus the per-position outputs above. */
int32_t sulimo_hip_execute_prefill_ubatch_ex(
    sulimo_hip_ctx *ctx, const sulimo_hip_model_config *cfg,
    const sulimo_hip_model_tensors *tensors, sulimo_hip_kv_cache *kv_cache,
    sulimo_hip_prefill_scratch *scratch, size_t start_pos, size_t n,
    const sulimo_hip_prefill_outputs *outputs);

/* Device embedding gather replacing the host loop lookup_token_embedding_f16
 * (crates/sulimo-engine/src/scheduler.rs:329-374, called at engine.rs:242-257):
 * x[t] = f16(d * (q - 8)) of row tokens[t] of the Q4_0 token_embd table. Bit-exact.
 * tokens is a host array of n ids (< vocab, else INVALID_ARGUMENT). */
int32_t sulimo_hip_embed_tokens(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *embd_scales,
                                const sulimo_hip_buffer *embd_quants, const uint32_t *tokens,
                                size_t n, size_t embd, size_t vocab, sulimo_hip_buffer *x);

/* KV hand-over between the device ring and the host KvCache that CPU decode reads
 * (forward_pass.rs:307-319 reads kv_cache.key_ptr/value_ptr): copy ring slots of
 * positions [start_pos, start_pos+n) of every layer device -> host mirror (blocking),
 * or host mirror -> device (ordered on the stream). */
int32_t sulimo_hip_kv_sync_to_host(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv,
                                   size_t start_pos, size_t n);
int32_t sulimo_hip_kv_sync_from_host(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv,
                                     size_t start_pos, size_t n);

/* Validation accessors (no counterpart in the reference, whose attention reads the
 * Q8_0 ring directly, kernels/prefill.cl:120-237).
 *
 * kv_window_download: the f16 attention window the prefill keeps for `layer` when a
 * prompt fits the ring (start_pos + n <= capacity; window index = position). Layout
 * (f16): K [n_head_kv][pad][head_dim], then V transposed, n_head_kv * head_dim rows of
 * v_row_stride elements; position j of a V^T row sits at column j with slots 4-7 and
 * 8-11 of each group of 16 swapped. Entries [0, valid_len) equal f16(code * f16(d)) of
 * the ring; valid_len is 0 once either ring buffer was written outside the prefill.
 * host == NULL only reports bytes, valid_len, pad and v_row_stride. Blocking.
 *
 * rope_table: the cos/sin pairs every RoPE rotation of a ubatch uses, f32
 * [n][rope_dim/2][2] = (cos, sin) of (start_pos + t) / freq_base^(2i/rope_dim)
 * (the angle of prefill.cl:32-68). */
int32_t sulimo_hip_kv_window_download(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv, int32_t layer,
                                      void *host, size_t host_bytes, size_t *bytes, int64_t *valid_len,
                                      int32_t *pad, int32_t *v_row_stride);
int32_t sulimo_hip_rope_table(sulimo_hip_ctx *ctx, size_t rope_dim, float freq_base, size_t start_pos,
                              size_t n, sulimo_hip_buffer *table);

/* ---- timing (the queue's CL_QUEUE_PROFILING_ENABLE, program.rs:145-153) ---- */
/* Per kernel class GPU time of execute_prefill_ubatch launches while profiling is on,
 * plus the algorithmic work the launches performed. The GEMM kernels stamp a hipEvent
 * pair with their own start and end (a K-split GEMM: the partial-sum kernel's start
 * and the reduction's end); the other launches sit between hipEvents recorded on the
 * context stream. */
typedef struct {
  uint64_t launches;
  double total_ms;
  double flop;  /* algorithmic FLOPs (GEMM 2*m*n*k; attention 4*head_dim*sum of keys per head) */
  double bytes; /* algorithmic HBM bytes (inputs read once + outputs written once) */
} sulimo_hip_kernel_stat;

typedef struct {
  sulimo_hip_kernel_stat gemm;      /* Q4_0 x f16 GEMMs (QKV, O, gate/up, down, LM head) */
  sulimo_hip_kernel_stat attention; /* causal GQA attention */
  sulimo_hip_kernel_stat norm;      /* RMSNorm and residual conversion */
  sulimo_hip_kernel_stat rope_kv;   /* RoPE + Q8_0 KV quantize/write + ring commit */
  sulimo_hip_kernel_stat other;     /* embedding gather, argmax */
  uint64_t prefill_calls;
  /* The gemm class by projection (each launch counted there and in gemm): */
  sulimo_hip_kernel_stat gemm_qkv;     /* q/k/v with the RoPE + Q8_0 K/V store epilogue */
  sulimo_hip_kernel_stat gemm_o;       /* output projection (+ residual, + its K-split reduction) */
  sulimo_hip_kernel_stat gemm_gate_up; /* gate and up with the SwiGLU epilogue */
  sulimo_hip_kernel_stat gemm_down;    /* down projection (+ residual, + its K-split reduction) */
  sulimo_hip_kernel_stat gemm_lm_head; /* last-token logits */
} sulimo_hip_prefill_stats;

/* Turns per-launch event timing on or off and clears the statistics. */
int32_t sulimo_hip_set_profiling(sulimo_hip_ctx *ctx, int32_t enable);

/* Graph replay of execute_prefill_ubatch (no counterpart in the reference; on by
 * default). The first call with a given set of shapes, buffers and kept-window state
 * captures its launches into two HIP graphs, split where the wake-up of the final wait
 * is gated; later identical calls replay them, which costs the engine thread a few
 * microseconds of CPU instead of one launch each (the reference's engine thread must
 * stay under 5 % of a core while the GPU runs a prefill). Calls with profiling on or
 * with per-position outputs run eagerly. Results are bit-identical either way.
 * Disabling it also frees the cached graphs. */
int32_t sulimo_hip_set_graph_replay(sulimo_hip_ctx *ctx, int32_t enable);
/* Backend tuning switch (no counterpart in the reference). When the attention splits a
 * query block's keys over several workgroups, the last workgroup to finish a block
 * merges its pieces (default), or with enable != 0 a separate kernel launch merges them.
 * Results are bit-identical either way. */
int32_t sulimo_hip_set_attention_merge_kernel(sulimo_hip_ctx *ctx, int32_t enable);
int32_t sulimo_hip_get_prefill_stats(const sulimo_hip_ctx *ctx, sulimo_hip_prefill_stats *out);

/* Record a start event on the context stream; stop records the end event, waits for
 * it and returns the elapsed GPU milliseconds between them. */
int32_t sulimo_hip_timer_start(sulimo_hip_ctx *ctx);
int32_t sulimo_hip_timer_stop(sulimo_hip_ctx *ctx, float *elapsed_ms);

#ifdef __cplusplus
}
#endif
#endif
