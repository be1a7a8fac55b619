// prefill.hip - C ABI of the per-op enqueue calls and of the whole-ubatch prefill.
//
// Mirrors crates/sulimo-ocl/src/prefill.rs (enqueue_* :67-330,
// execute_prefill_ubatch :337-566) and crates/sulimo-ocl/src/gemm.rs:28-102.
// Every call checks buffer sizes against the shapes on the host before it
// enqueues anything, so a bad argument becomes SULIMO_HIP_ERR_INVALID_ARGUMENT
// instead of an out-of-bounds device access.
#include <limits.h>

#include <algorithm>
#include <stdio.h>
#include <string.h>

#include <string>

#include "common.h"

using namespace sulimo;

namespace {

constexpr int32_t kInval = SULIMO_HIP_ERR_INVALID_ARGUMENT;

bool too_small(const sulimo_hip_buffer *b, size_t need, const char *name, int32_t *rc) {
  if (!b) {
    *rc = fail(kInval, std::string(name) + " buffer is null");
    return true;
  }
  if (b->bytes < need) {
    *rc = fail(kInval, std::string(name) + " buffer holds " + std::to_string(b->bytes) +
                           " bytes, needs " + std::to_string(need));
    return true;
  }
  return false;
}

#define NEED(buf, bytes, name)                      \
  do {                                              \
    int32_t rc_;                                    \
    if (too_small((buf), (bytes), (name), &rc_)) return rc_; \
  } while (0)

template <typename T>
T *dp(const sulimo_hip_buffer *b) {
  return reinterpret_cast<T *>(b->dev);
}

bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

int32_t begin(sulimo_hip_ctx *ctx) {
  if (!ctx) return fail(kInval, "ctx is null");
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  return SULIMO_HIP_OK;
}

// Y[n][m] = X[n][k] W[m][k]^T for the Q4_0 matrix W = (scales, quants), through its
// panel copy (built on first use).
// With own_workspace, a K split may use the context workspace for its partials (only
// where no other data lives in it).
int32_t gemm_plain(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                   const sulimo_hip_buffer *quants, const void *x, void *out, size_t m, size_t k,
                   size_t n, int epi, bool own_workspace = false, const LaunchStamp *stamp = nullptr) {
  const uint8_t *pan = nullptr;
  int32_t rc = get_q4_panels(ctx, scales, quants, nullptr, nullptr, (int)m, (int)k, &pan);
  if (rc) return rc;
  GemmArgs a{};
  a.x = reinterpret_cast<const uint16_t *>(x);
  a.m = (int)n;
  a.k = (int)k;
  a.ldx = (int)k;
  a.epi = epi;
  a.seg[0] = GemmSegment{pan, out, (int)m, (int)m, 0};
  a.nseg = 1;
  if (own_workspace) {
    const size_t need = gemm_q4_0_workspace_bytes(a);
    if (need) {
      if ((rc = ensure_workspace(ctx, need))) return rc;
      a.part = reinterpret_cast<float *>(ctx->ws);
      a.part_bytes = need;
    }
  }
  return launch_gemm_q4_0(a, ctx->stream, nullptr, stamp);
}

// Device pointer of an optional f32 tensor (null when absent).
const float *opt_f32(const sulimo_hip_buffer *b) { return b ? reinterpret_cast<const float *>(b->dev) : nullptr; }

// Runs one launch between profiling events (no events when profiling is off).
template <typename F>
int32_t timed(sulimo_hip_ctx *ctx, int cls, double flop, double bytes, F &&launch) {
  const int ev = prof_begin(ctx);
  const int32_t rc = launch();
  prof_end(ctx, ev, cls, flop, bytes);
  return rc;
}

// Runs one GEMM (m > 0) whose kernels stamp the profiling events with their own start
// and end times: launch(stamp), stamp null when profiling is off.
template <typename F>
int32_t timed_gemm(sulimo_hip_ctx *ctx, int cls, double flop, double bytes, F &&launch) {
  LaunchStamp st;
  const int ev = prof_begin_stamp(ctx, &st);
  const int32_t rc = launch(ev >= 0 ? &st : nullptr);
  if (rc == SULIMO_HIP_OK) prof_end_stamp(ctx, ev, cls, flop, bytes);
  return rc;
}

// Algorithmic work of a GEMM launch: 2*m*n*k FLOPs; Q4_0 weights (18 bytes per 32),
// activations and outputs moved once.
double gemm_flop(const GemmArgs &g) {
  double n = 0;
  for (int i = 0; i < g.nseg; i++) n += g.seg[i].n;
  if (g.epi == EPI_SWIGLU) n *= 2;
  return 2.0 * g.m * n * g.k;
}
double gemm_bytes(const GemmArgs &g) {
  double n = 0;
  for (int i = 0; i < g.nseg; i++) n += g.seg[i].n;
  const double wn = g.epi == EPI_SWIGLU ? 2 * n : n;
  const double out = g.epi == EPI_F32 ? 4.0 * g.m * n
                     : g.epi == EPI_RESID ? 8.0 * g.m * n  // f32 residual read + write
                                          : 2.0 * g.m * n;
  return wn * g.k * 18.0 / 32.0 + 2.0 * g.m * g.k + out;
}

}  // namespace

extern "C" {

int32_t sulimo_hip_enqueue_gemm_q4_0_f16(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                         const sulimo_hip_buffer *quants,
                                         const sulimo_hip_buffer *x, sulimo_hip_buffer *out,
                                         size_t m, size_t k, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (k == 0 || k % 32 != 0) return fail(kInval, "K must be a multiple of 32 (Q4_0 block size)");
  if (m == 0 || m % 8 != 0) return fail(kInval, "M must be a multiple of 8");
  if (!fits_int(m) || !fits_int(k) || !fits_int(n)) return fail(kInval, "GEMM dimension too large");
  NEED(scales, m * (k / 32) * 2, "scales");
  NEED(quants, m * (k / 32) * 16, "quants");
  NEED(x, n * k * 2, "x");
  NEED(out, n * m * 2, "out");
  if (n == 0) return SULIMO_HIP_OK;
  wrote(out);
  return gemm_plain(ctx, scales, quants, x->dev, out->dev, m, k, n, EPI_F16, true);
}

int32_t sulimo_hip_enqueue_gemm_q4_0_f16_noalloc(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                                 const sulimo_hip_buffer *quants,
                                                 const sulimo_hip_buffer *x, sulimo_hip_buffer *out,
                                                 size_t m, size_t k, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (k == 0 || k % 32 != 0) return fail(kInval, "K must be a multiple of 32 (Q4_0 block size)");
  if (m == 0 || m % 8 != 0) return fail(kInval, "M must be a multiple of 8");
  if (!fits_int(m) || !fits_int(k) || !fits_int(n)) return fail(kInval, "GEMM dimension too large");
  NEED(scales, m * (k / 32) * 2, "scales");
  NEED(quants, m * (k / 32) * 16, "quants");
  NEED(x, n * k * 2, "x");
  NEED(out, n * m * 2, "out");
  if (!ctx->scratch) return fail(SULIMO_HIP_ERR_DRIVER, "the device scratch array was not resolved");
  // The weights' GEMM layout goes to the start of the scratch array (rebuilt on every
  // call: nothing in the array is assumed to survive from an earlier call), the K-split
  // partial sums after it. Every byte either region is read from is written first in
  // the same call, so nothing needs clearing.
  const size_t pan = q4_panel_bytes((int)m, (int)k, false);
  const size_t pan_al = (pan + 255) & ~(size_t)255;
  if (pan_al > kNoAllocScratchBytes)
    return fail(kInval, "the no-alloc GEMM holds at most " + std::to_string(kNoAllocScratchBytes) +
                            " bytes of weights in its GEMM layout; this matrix needs " + std::to_string(pan));
  if (n == 0) return SULIMO_HIP_OK;
  NoAllocOrder *order = noalloc_order(ctx->device);
  if (!order) return fail(SULIMO_HIP_ERR_DRIVER, "the no-alloc ordering event was not created");
  // After the previous no-alloc call on this device, from whatever stream it came.
  std::lock_guard<std::mutex> serial(order->m);
  SULIMO_HIP_TRY(hipStreamWaitEvent(ctx->stream, order->ev, 0));
  wrote(out);
  uint8_t *scr = reinterpret_cast<uint8_t *>(ctx->scratch);
  if ((rc = launch_pack_q4_panels(dp<const uint16_t>(scales), dp<const uint8_t>(quants), nullptr, nullptr, (int)m,
                                  (int)k, scr, ctx->stream)))
    return rc;
  GemmArgs a{};
  a.x = dp<const uint16_t>(x);
  a.m = (int)n;
  a.k = (int)k;
  a.ldx = (int)k;
  a.epi = EPI_F16;
  a.seg[0] = GemmSegment{scr, out->dev, (int)m, (int)m, 0};
  a.nseg = 1;
  a.part = reinterpret_cast<float *>(scr + pan_al);
  a.part_bytes = kNoAllocScratchBytes - pan_al;
  if ((rc = launch_gemm_q4_0(a, ctx->stream))) return rc;
  SULIMO_HIP_TRY(hipEventRecord(order->ev, ctx->stream));
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_gemm_q4_0_f16(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales,
                                 const sulimo_hip_buffer *quants, const sulimo_hip_buffer *x,
                                 sulimo_hip_buffer *out, size_t m, size_t k, size_t n,
                                 sulimo_hip_gemm_profile *profile) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if ((rc = sulimo_hip_timer_start(ctx))) return rc;
  if ((rc = sulimo_hip_enqueue_gemm_q4_0_f16(ctx, scales, quants, x, out, m, k, n))) return rc;
  float ms = 0.0f;
  if ((rc = sulimo_hip_timer_stop(ctx, &ms))) return rc;
  if (profile) {
    profile->duration_seconds = ms * 1e-3;
    profile->gflops = ms > 0 ? 2.0 * m * n * k / (ms * 1e-3) / 1e9 : 0.0;
    profile->kernel_variant = "gfx950-mfma-f16-q4_0";
  }
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_enqueue_rmsnorm(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *x,
                                   const sulimo_hip_buffer *w, sulimo_hip_buffer *out, size_t d,
                                   float eps, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (d == 0 || !fits_int(d) || !fits_int(n)) return fail(kInval, "bad rmsnorm shape");
  NEED(x, n * d * 2, "x");
  NEED(w, d * 4, "w");
  NEED(out, n * d * 2, "out");
  wrote(out);
  return launch_rmsnorm_f16(dp<const uint16_t>(x), dp<const float>(w), dp<uint16_t>(out), (int)d,
                            eps, (int)n, ctx->stream);
}

int32_t sulimo_hip_enqueue_rope(sulimo_hip_ctx *ctx, sulimo_hip_buffer *vec, size_t head_count,
                                size_t head_dim, size_t rope_dim, float freq_base, int32_t mode,
                                size_t start_pos, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (rope_dim > head_dim || rope_dim % 2 != 0) return fail(kInval, "rope_dim must be even and <= head_dim");
  if (mode != 0 && mode != 1) return fail(kInval, "rope mode must be 0 (Norm) or 1 (NeoX)");
  if (!fits_int(head_count * head_dim) || !fits_int(start_pos + n)) return fail(kInval, "rope shape too large");
  NEED(vec, n * head_count * head_dim * 2, "vec");
  wrote(vec);
  return launch_rope_f16(dp<uint16_t>(vec), (int)head_count, (int)head_dim, (int)rope_dim,
                         freq_base, mode, (int)start_pos, (int)n, ctx->stream);
}

int32_t sulimo_hip_enqueue_kv_store(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *act,
                                    sulimo_hip_buffer *kv_cache, size_t start_pos,
                                    size_t capacity, size_t blocks_per_pos, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (capacity == 0 || blocks_per_pos == 0) return fail(kInval, "capacity and blocks_per_pos must be positive");
  if (!fits_int(start_pos + n) || !fits_int(capacity)) return fail(kInval, "kv_store shape too large");
  NEED(act, n * blocks_per_pos * 32 * 2, "act");
  NEED(kv_cache, capacity * blocks_per_pos * 34, "kv_cache");
  wrote(kv_cache);
  return launch_kv_store_q8_0(dp<const uint16_t>(act), dp<uint8_t>(kv_cache), (int)start_pos,
                              (int)capacity, (int)blocks_per_pos, (int)n, ctx->stream);
}

int32_t sulimo_hip_enqueue_attention_prefill(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *q,
                                             const sulimo_hip_buffer *k_cache,
                                             const sulimo_hip_buffer *v_cache,
                                             sulimo_hip_buffer *out, size_t start_pos,
                                             size_t capacity, size_t head_count,
                                             size_t head_count_kv, size_t head_dim, size_t n) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (head_dim % 32 != 0 || head_count_kv == 0 || head_count % head_count_kv != 0 || capacity == 0)
    return fail(kInval, "attention needs head_dim % 32 == 0, head_count % head_count_kv == 0, capacity > 0");
  if (!fits_int(start_pos + n) || !fits_int(capacity)) return fail(kInval, "attention shape too large");
  const size_t bpp = head_count_kv * (head_dim / 32) * 34;
  NEED(q, n * head_count * head_dim * 2, "q");
  NEED(out, n * head_count * head_dim * 2, "out");
  NEED(k_cache, capacity * bpp, "k_cache");
  NEED(v_cache, capacity * bpp, "v_cache");
  AttnArgs a{};
  a.q = dp<const uint16_t>(q);
  a.out = dp<uint16_t>(out);
  a.k_ring = dp<const uint8_t>(k_cache);
  a.v_ring = dp<const uint8_t>(v_cache);
  a.new_k = a.new_v = nullptr;
  a.new_pos0 = LONG_MAX;
  a.start_pos = (int)start_pos;
  a.n = (int)n;
  a.capacity = (int)capacity;
  a.n_head = (int)head_count;
  a.n_head_kv = (int)head_count_kv;
  a.head_dim = (int)head_dim;
  if ((rc = ensure_workspace(ctx, attention_workspace_bytes(a)))) return rc;
  a.window = ctx->ws;
  a.ctr_ints = attention_counter_ints(a);
  if ((rc = ensure_attn_counters(ctx, a.ctr_ints, &a.ctr))) return rc;
  wrote(out);
  return launch_attention(a, ctx->stream);
}

int32_t sulimo_hip_enqueue_silu_mul(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *gate,
                                    const sulimo_hip_buffer *up, sulimo_hip_buffer *out,
                                    size_t total_elements) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  NEED(gate, total_elements * 2, "gate");
  NEED(up, total_elements * 2, "up");
  NEED(out, total_elements * 2, "out");
  wrote(out);
  return launch_silu_mul(dp<const uint16_t>(gate), dp<const uint16_t>(up), dp<uint16_t>(out),
                         total_elements, ctx->stream);
}

int32_t sulimo_hip_enqueue_add(sulimo_hip_ctx *ctx, sulimo_hip_buffer *a,
                               const sulimo_hip_buffer *b, size_t total_elements) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  NEED(a, total_elements * 2, "a");
  NEED(b, total_elements * 2, "b");
  wrote(a);
  return launch_add_f16(dp<uint16_t>(a), dp<const uint16_t>(b), total_elements, ctx->stream);
}

int32_t sulimo_hip_enqueue_logits_final(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *x_all,
                                        const sulimo_hip_buffer *scales,
                                        const sulimo_hip_buffer *quants, sulimo_hip_buffer *logits,
                                        size_t vocab_size, size_t embd_dim, size_t token_idx) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (embd_dim == 0 || embd_dim % 32 != 0) return fail(kInval, "embd_dim must be a multiple of 32");
  if (vocab_size == 0 || !fits_int(vocab_size) || !fits_int(embd_dim)) return fail(kInval, "bad vocab size");
  NEED(x_all, (token_idx + 1) * embd_dim * 2, "x_all");
  NEED(scales, vocab_size * (embd_dim / 32) * 2, "scales");
  NEED(quants, vocab_size * (embd_dim / 32) * 16, "quants");
  NEED(logits, vocab_size * 4, "logits");
  wrote(logits);
  const char *xrow = reinterpret_cast<const char *>(x_all->dev) + token_idx * embd_dim * 2;
  return gemm_plain(ctx, scales, quants, xrow, logits->dev, vocab_size, embd_dim, 1, EPI_F32);
}

int32_t sulimo_hip_embed_tokens(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *embd_scales,
                                const sulimo_hip_buffer *embd_quants, const uint32_t *tokens,
                                size_t n, size_t embd, size_t vocab, sulimo_hip_buffer *x) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (embd == 0 || embd % 32 != 0 || !fits_int(embd) || !fits_int(n)) return fail(kInval, "embd must be a multiple of 32");
  if (n == 0) return SULIMO_HIP_OK;
  if (!tokens) return fail(kInval, "tokens is null");
  for (size_t t = 0; t < n; t++)
    if (tokens[t] >= vocab) return fail(kInval, "token id " + std::to_string(tokens[t]) + " >= vocab");
  NEED(embd_scales, vocab * (embd / 32) * 2, "embd_scales");
  NEED(embd_quants, vocab * (embd / 32) * 16, "embd_quants");
  NEED(x, n * embd * 2, "x");
  wrote(x);
  // The ids are staged in a buffer of this context, so that the copy and the gather
  // are ordered on this context's stream (another context cannot overwrite them).
  if (ctx->tok_bytes < n * 4) {
    if (ctx->tok) {
      SULIMO_HIP_TRY(hipStreamSynchronize(ctx->stream));
      hipFree(ctx->tok);
      ctx->tok = nullptr;
      ctx->tok_bytes = 0;
    }
    size_t sz = ((n * 4) + 4095) & ~(size_t)4095;
    SULIMO_HIP_TRY(hipMalloc(&ctx->tok, sz));
    ctx->tok_bytes = sz;
  }
  SULIMO_HIP_TRY(hipMemcpyAsync(ctx->tok, tokens, n * 4, hipMemcpyHostToDevice, ctx->stream));
  return launch_embed_q4_0(dp<const uint16_t>(embd_scales), dp<const uint8_t>(embd_quants),
                           reinterpret_cast<const uint32_t *>(ctx->tok), (int)n, (int)embd,
                           dp<uint16_t>(x), ctx->stream);
}

// ---- KV hand-over ----

static int32_t kv_sync(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv, size_t start_pos,
                       size_t n, bool to_host) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (!kv || !kv->k_buffers || !kv->v_buffers || kv->capacity == 0 || kv->head_dim % 32 != 0)
    return fail(kInval, "bad kv cache descriptor");
  const size_t bpp = kv->head_count_kv * (kv->head_dim / 32) * 34;
  const size_t cap = kv->capacity;
  if (n == 0) return SULIMO_HIP_OK;
  size_t segs[2][2];  // (first slot, count)
  int ns = 0;
  if (n >= cap) {
    segs[0][0] = 0;
    segs[0][1] = cap;
    ns = 1;
  } else {
    size_t a = start_pos % cap;
    size_t first = std::min(n, cap - a);
    segs[ns][0] = a;
    segs[ns++][1] = first;
    if (first < n) {
      segs[ns][0] = 0;
      segs[ns++][1] = n - first;
    }
  }
  for (int l = 0; l < kv->n_layers; l++) {
    for (int which = 0; which < 2; which++) {
      sulimo_hip_buffer *b = which ? kv->v_buffers[l] : kv->k_buffers[l];
      NEED(b, cap * bpp, "kv layer");
      if (!b->host) return fail(SULIMO_HIP_ERR_ZERO_COPY, "kv buffer has no host mirror");
      if (!to_host) wrote(b);
      for (int s = 0; s < ns; s++) {
        char *dev = (char *)b->dev + segs[s][0] * bpp;
        char *host = (char *)b->host + segs[s][0] * bpp;
        size_t bytes = segs[s][1] * bpp;
        if (to_host)
          SULIMO_HIP_TRY(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
        else
          SULIMO_HIP_TRY(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream));
      }
    }
  }
  if (to_host) return sulimo_hip_wait(ctx);
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_kv_sync_to_host(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv,
                                   size_t start_pos, size_t n) {
  return kv_sync(ctx, kv, start_pos, n, true);
}

int32_t sulimo_hip_kv_sync_from_host(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv,
                                     size_t start_pos, size_t n) {
  return kv_sync(ctx, kv, start_pos, n, false);
}

int32_t sulimo_hip_kv_window_download(sulimo_hip_ctx *ctx, const sulimo_hip_kv_cache *kv, int32_t layer,
                                      void *host, size_t host_bytes, size_t *bytes, int64_t *valid_len,
                                      int32_t *pad, int32_t *v_row_stride) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (!kv || !kv->k_buffers || !kv->v_buffers || layer < 0 || layer >= kv->n_layers)
    return fail(kInval, "bad kv cache or layer");
  const sulimo_hip_buffer *kb = kv->k_buffers[layer], *vb = kv->v_buffers[layer];
  if (!kb || !vb) return fail(kInval, "null kv buffer");
  const KvWindowCache &wc = kb->kvwin;
  if (!wc.dev) return fail(kInval, "no kept attention window for this layer");
  AttnArgs a{};
  a.n = 1;
  a.capacity = (int)kv->capacity;
  a.n_head = wc.n_head_kv;
  a.n_head_kv = wc.n_head_kv;
  a.head_dim = wc.head_dim;
  a.win_pad = wc.pad;
  const AttnWindowLayout wl = attention_window_layout(a);
  const bool valid = wc.v_id == vb->id && wc.k_ver == kb->version && wc.v_ver == vb->version;
  if (bytes) *bytes = wc.bytes;
  if (valid_len) *valid_len = valid ? (int64_t)wc.len : 0;
  if (pad) *pad = wl.pad;
  if (v_row_stride) *v_row_stride = wl.vst;
  if (!host) return SULIMO_HIP_OK;
  if (host_bytes < wc.bytes) return fail(kInval, "host buffer smaller than the window");
  SULIMO_HIP_TRY(hipMemcpyAsync(host, wc.dev, wc.bytes, hipMemcpyDeviceToHost, ctx->stream));
  return sulimo_hip_wait(ctx);
}

int32_t sulimo_hip_rope_table(sulimo_hip_ctx *ctx, size_t rope_dim, float freq_base, size_t start_pos,
                              size_t n, sulimo_hip_buffer *table) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (rope_dim == 0 || rope_dim % 2 != 0 || rope_dim > 512) return fail(kInval, "rope_dim must be even, 2..512");
  if (!fits_int(start_pos + n) || !fits_int(n * rope_dim)) return fail(kInval, "rope table too large");
  NEED(table, n * (rope_dim / 2) * 8, "table");
  wrote(table);
  return launch_rope_table(dp<float>(table), (int)rope_dim, freq_base, (int)start_pos, (int)n, ctx->stream);
}

// ---- whole-ubatch prefill ----

int32_t sulimo_hip_execute_prefill_ubatch_ex(
    sulimo_hip_ctx *ctx, const sulimo_hip_model_config *cfg,
    const sulimo_hip_model_tensors *tensors, sulimo_hip_kv_cache *kv,
    sulimo_hip_prefill_scratch *scratch, size_t start_pos, size_t n,
    const sulimo_hip_prefill_outputs *outputs) {
  int32_t rc = begin(ctx);
  if (rc) return rc;
  if (!cfg || !tensors || !kv || !scratch) return fail(kInval, "null argument");
  if (n == 0) return SULIMO_HIP_OK;
  const size_t D = cfg->embd, F = cfg->ffn, Hq = cfg->n_head, Hkv = cfg->n_head_kv,
               hd = cfg->head_dim, V = cfg->vocab, L = cfg->n_layers;
  const size_t qd = Hq * hd, kvd = Hkv * hd;
  const size_t cap = kv->capacity;
  if (D == 0 || D % 32 || F == 0 || F % 32 || qd % 32 || kvd % 32 || Hkv == 0 || Hq % Hkv ||
      (hd != 64 && hd != 128) || V == 0 || L == 0)
    return fail(kInval, "unsupported model shape (needs dims % 32 == 0, head_dim 64 or 128, head_count % head_count_kv == 0)");
  if (cfg->rope_dim < 0 || (size_t)cfg->rope_dim > hd || cfg->rope_dim % 2 || (cfg->rope_mode != 0 && cfg->rope_mode != 1))
    return fail(kInval, "bad rope configuration");
  if (tensors->n_layers != (int)L || kv->n_layers != (int)L || !tensors->layers || !kv->k_buffers || !kv->v_buffers)
    return fail(kInval, "layer count mismatch");
  if (kv->head_count_kv != Hkv || kv->head_dim != hd || cap == 0) return fail(kInval, "kv cache shape mismatch");
  if (n > scratch->max_n) return fail(kInval, "n exceeds scratch.max_n");
  if (!fits_int(start_pos + n) || !fits_int(cap) || !fits_int(V * D)) return fail(kInval, "shape too large");
  const size_t bpp = Hkv * (hd / 32) * 34;
  const size_t nbD = D / 32, nbF = F / 32, nbQ = qd / 32;
  NEED(scratch->x, n * D * 2, "scratch.x");
  NEED(scratch->h, n * D * 2, "scratch.h");
  NEED(scratch->q, n * qd * 2, "scratch.q");
  NEED(scratch->k, n * kvd * 2, "scratch.k");
  NEED(scratch->v, n * kvd * 2, "scratch.v");
  NEED(scratch->attn_out, n * qd * 2, "scratch.attn_out");
  NEED(scratch->ffn_swiglu, n * F * 2, "scratch.ffn_swiglu");
  NEED(scratch->logits, V * 4, "scratch.logits");
  NEED(tensors->output_norm, D * 4, "output_norm");
  NEED(tensors->output_scales, V * nbD * 2, "output_scales");
  NEED(tensors->output_quants, V * nbD * 16, "output_quants");
  for (size_t l = 0; l < L; l++) {
    const sulimo_hip_layer_tensors &T = tensors->layers[l];
    NEED(T.attn_norm, D * 4, "attn_norm");
    NEED(T.ffn_norm, D * 4, "ffn_norm");
    NEED(T.attn_q_scales, qd * nbD * 2, "attn_q_scales");
    NEED(T.attn_q_quants, qd * nbD * 16, "attn_q_quants");
    NEED(T.attn_k_scales, kvd * nbD * 2, "attn_k_scales");
    NEED(T.attn_k_quants, kvd * nbD * 16, "attn_k_quants");
    NEED(T.attn_v_scales, kvd * nbD * 2, "attn_v_scales");
    NEED(T.attn_v_quants, kvd * nbD * 16, "attn_v_quants");
    NEED(T.attn_out_scales, D * nbQ * 2, "attn_out_scales");
    NEED(T.attn_out_quants, D * nbQ * 16, "attn_out_quants");
    NEED(T.ffn_gate_scales, F * nbD * 2, "ffn_gate_scales");
    NEED(T.ffn_gate_quants, F * nbD * 16, "ffn_gate_quants");
    NEED(T.ffn_up_scales, F * nbD * 2, "ffn_up_scales");
    NEED(T.ffn_up_quants, F * nbD * 16, "ffn_up_quants");
    NEED(T.ffn_down_scales, D * nbF * 2, "ffn_down_scales");
    NEED(T.ffn_down_quants, D * nbF * 16, "ffn_down_quants");
    if (T.attn_q_bias) NEED(T.attn_q_bias, qd * 4, "attn_q_bias");
    if (T.attn_k_bias) NEED(T.attn_k_bias, kvd * 4, "attn_k_bias");
    if (T.attn_v_bias) NEED(T.attn_v_bias, kvd * 4, "attn_v_bias");
    if (T.attn_q_norm) NEED(T.attn_q_norm, hd * 4, "attn_q_norm");
    if (T.attn_k_norm) NEED(T.attn_k_norm, hd * 4, "attn_k_norm");
    NEED(kv->k_buffers[l], cap * bpp, "kv k");
    NEED(kv->v_buffers[l], cap * bpp, "kv v");
  }
  if (outputs && outputs->logits_all) NEED(outputs->logits_all, n * V * 4, "logits_all");
  if (outputs && outputs->argmax_all) NEED(outputs->argmax_all, n * 4, "argmax_all");
  // Validation mode: every op as its own kernel (no GEMM epilogue fusion).
  const bool unfused = outputs && outputs->unfused;
  if (unfused) {
    NEED(scratch->ffn_gate, n * F * 2, "scratch.ffn_gate");
    NEED(scratch->ffn_up, n * F * 2, "scratch.ffn_up");
    NEED(scratch->ffn_down, n * D * 2, "scratch.ffn_down");
  }

  // Workspace: f32 residual [n][D] | staged K codes [n][bpp] | staged V codes | argmax logits chunk.
  const bool staged = start_pos + n > cap;
  const size_t off_k = (n * D * 4 + 255) & ~(size_t)255;
  const size_t off_v = off_k + ((staged ? n * bpp : 0) + 255 & ~(size_t)255);
  const size_t off_l = off_v + ((staged ? n * bpp : 0) + 255 & ~(size_t)255);
  const bool want_argmax = outputs && outputs->argmax_all;
  const bool own_logits = want_argmax && !outputs->logits_all;
  const size_t chunk_rows = 256;
  // attention workspace: f16 key window (the same for every layer of the ubatch) and
  // split-key partial results
  AttnArgs probe_at{};
  probe_at.start_pos = (int)start_pos;
  probe_at.n = (int)n;
  probe_at.capacity = (int)cap;
  probe_at.n_head = (int)Hq;
  probe_at.n_head_kv = (int)Hkv;
  probe_at.head_dim = (int)hd;
  const size_t off_w = off_l + ((own_logits ? chunk_rows * V * 4 : 0) + 255 & ~(size_t)255);
  // RoPE cos/sin table of the ubatch (shared by all layers)
  const size_t off_r = off_w + (attention_workspace_bytes(probe_at) + 255 & ~(size_t)255);
  // K-split partials of the q/k/v, o and down GEMMs (sized by the GEMM planner)
  const size_t off_g = off_r + (n * (size_t)(cfg->rope_dim / 2) * 8 + 255 & ~(size_t)255);
  size_t gemm_ws = 0;
  {
    GemmArgs p{};
    p.m = (int)n;
    p.k = (int)D;
    p.ldx = (int)D;
    p.epi = EPI_F16;
    p.seg[0] = GemmSegment{nullptr, nullptr, (int)qd, (int)qd, 0};
    p.seg[1] = GemmSegment{nullptr, nullptr, (int)kvd, (int)kvd, 0};
    p.seg[2] = GemmSegment{nullptr, nullptr, (int)kvd, (int)kvd, 0};
    p.nseg = 3;
    gemm_ws = std::max(gemm_ws, gemm_q4_0_workspace_bytes(p));
    p.k = (int)qd;
    p.epi = EPI_RESID;
    p.seg[0] = GemmSegment{nullptr, nullptr, (int)D, (int)D, 0};
    p.nseg = 1;
    gemm_ws = std::max(gemm_ws, gemm_q4_0_workspace_bytes(p));
    p.k = (int)F;
    gemm_ws = std::max(gemm_ws, gemm_q4_0_workspace_bytes(p));
  }
  const size_t ws_need = off_g + gemm_ws;
  if ((rc = ensure_workspace(ctx, ws_need))) return rc;
  int *attn_ctr = nullptr;
  const size_t attn_ctr_ints = attention_counter_ints(probe_at);
  if ((rc = ensure_attn_counters(ctx, attn_ctr_ints, &attn_ctr))) return rc;
  char *ws = reinterpret_cast<char *>(ctx->ws);
  float *xres = reinterpret_cast<float *>(ws);
  float *gemm_part = reinterpret_cast<float *>(ws + off_g);
  uint8_t *stg_k = reinterpret_cast<uint8_t *>(ws + off_k);
  uint8_t *stg_v = reinterpret_cast<uint8_t *>(ws + off_v);
  hipStream_t s = ctx->stream;
  const int in = (int)n;

  // Kept attention windows (a prompt that fits the ring): one per layer on its K ring
  // buffer, valid for the positions the last prefill left in it if nothing else wrote
  // either ring since. Checked before this call marks the rings written.
  const bool keep_win = start_pos + n <= cap;
  std::vector<int> win_valid(L, 0);
  if (keep_win) {
    AttnArgs wa = probe_at;
    wa.win_pad = (int)((cap + 63) / 64 * 64);
    const size_t wbytes = attention_window_bytes(wa);
    for (size_t l = 0; l < L; l++) {
      sulimo_hip_buffer *kb = kv->k_buffers[l], *vb = kv->v_buffers[l];
      KvWindowCache &wc = kb->kvwin;
      if (!wc.dev || wc.bytes != wbytes || wc.pad != wa.win_pad || wc.n_head_kv != (int)Hkv ||
          wc.head_dim != (int)hd || wc.v_id != vb->id) {
        if (wc.dev) {
          SULIMO_HIP_TRY(hipStreamSynchronize(ctx->stream));
          hipFree(wc.dev);
          wc = KvWindowCache{};
        }
        SULIMO_HIP_TRY(hipMalloc(&wc.dev, wbytes));
        // the padding past the last position must hold finite values
        SULIMO_HIP_TRY(hipMemsetAsync(wc.dev, 0, wbytes, ctx->stream));
        wc.bytes = wbytes;
        wc.pad = wa.win_pad;
        wc.n_head_kv = (int)Hkv;
        wc.head_dim = (int)hd;
        wc.v_id = vb->id;
      } else if (wc.k_ver == kb->version && wc.v_ver == vb->version) {
        win_valid[l] = (int)std::min<long>(wc.len, (long)start_pos);
      }
      wc.len = 0;  // until this call completes
    }
  }
  for (sulimo_hip_buffer *b : {scratch->x, scratch->h, scratch->q, scratch->k, scratch->v, scratch->attn_out,
                               scratch->ffn_swiglu, scratch->logits})
    wrote(b);
  if (unfused)
    for (sulimo_hip_buffer *b : {scratch->ffn_gate, scratch->ffn_up, scratch->ffn_down}) wrote(b);
  for (size_t l = 0; l < L; l++) {
    wrote(kv->k_buffers[l]);
    wrote(kv->v_buffers[l]);
  }
  if (outputs) {
    wrote(outputs->logits_all);
    wrote(outputs->argmax_all);
  }
  // Panel copies of every layer's weights and of the LM head (built by the first
  // ubatch), resolved before the first launch so that no allocation or panel build
  // falls inside a graph capture.
  std::vector<const uint8_t *> panels(6 * L);
  const uint8_t *lm_panel = nullptr;
  for (size_t l = 0; l < L; l++) {
    const sulimo_hip_layer_tensors &T = tensors->layers[l];
    const uint8_t **pp = &panels[6 * l];
    if ((rc = get_q4_panels(ctx, T.attn_q_scales, T.attn_q_quants, nullptr, nullptr, (int)qd, (int)D, &pp[0])) ||
        (rc = get_q4_panels(ctx, T.attn_k_scales, T.attn_k_quants, nullptr, nullptr, (int)kvd, (int)D, &pp[1])) ||
        (rc = get_q4_panels(ctx, T.attn_v_scales, T.attn_v_quants, nullptr, nullptr, (int)kvd, (int)D, &pp[2])) ||
        (rc = get_q4_panels(ctx, T.attn_out_scales, T.attn_out_quants, nullptr, nullptr, (int)D, (int)qd, &pp[3])) ||
        (rc = get_q4_panels(ctx, T.ffn_gate_scales, T.ffn_gate_quants, T.ffn_up_scales, T.ffn_up_quants, (int)F,
                            (int)D, &pp[4])) ||
        (rc = get_q4_panels(ctx, T.ffn_down_scales, T.ffn_down_quants, nullptr, nullptr, (int)D, (int)F, &pp[5])))
      return rc;
  }
  if ((rc = get_q4_panels(ctx, tensors->output_scales, tensors->output_quants, nullptr, nullptr, (int)V, (int)D,
                          &lm_panel)))
    return rc;
  const bool want_outputs = outputs && (outputs->logits_all || outputs->argmax_all || outputs->unfused);

  // Every launch of the ubatch, in order. gate() runs where the wake-up of the final
  // wait is gated (before the last down projection): it records near_event, or, under
  // graph capture, closes the first graph and opens the second.
  auto body = [&](auto &&gate) -> int32_t {
  int32_t rc = SULIMO_HIP_OK;
  if ((rc = timed(ctx, PROF_NORM, 0, 6.0 * n * D, [&] { return launch_f16_to_f32(dp<const uint16_t>(scratch->x), xres, n * D, s); }))) return rc;
  float *rope_tab = reinterpret_cast<float *>(ws + off_r);
  if ((rc = timed(ctx, PROF_ROPE_KV, 0, 8.0 * n * (cfg->rope_dim / 2), [&] {
         return launch_rope_table(rope_tab, cfg->rope_dim, cfg->rope_base, (int)start_pos, in, s);
       })))
    return rc;
  // An EPI_RESID GEMM whose K split runs the RMSNorm of the rows it updates (o-proj:
  // the FFN norm, down-proj: the next layer's attention norm or the output norm) leaves
  // h ready, and the separate norm launch is skipped.
  bool h_ready = false;
  for (size_t l = 0; l < L; l++) {
    const sulimo_hip_layer_tensors &T = tensors->layers[l];
    uint8_t *ring_k = dp<uint8_t>(kv->k_buffers[l]);
    uint8_t *ring_v = dp<uint8_t>(kv->v_buffers[l]);
    // 1. attention RMSNorm
    if (!h_ready && (rc = timed(ctx, PROF_NORM, 0, 6.0 * n * D + 4.0 * D, [&] {
                       return launch_rmsnorm_f32(xres, dp<const float>(T.attn_norm), dp<uint16_t>(scratch->h),
                                                 nullptr, (int)D, cfg->eps, in, s);
                     })))
      return rc;
    const uint8_t *pq = panels[6 * l], *pk = panels[6 * l + 1], *pv = panels[6 * l + 2],
                  *po = panels[6 * l + 3], *pgu = panels[6 * l + 4], *pd = panels[6 * l + 5];
    // attention arguments first: the RoPE + Q8_0 store also writes the f16 window
    // entries of the new positions
    AttnArgs at{};
    at.q = dp<const uint16_t>(scratch->q);
    at.out = dp<uint16_t>(scratch->attn_out);
    at.k_ring = ring_k;
    at.v_ring = ring_v;
    at.new_k = staged ? stg_k : nullptr;
    at.new_v = staged ? stg_v : nullptr;
    at.new_pos0 = staged ? (long)start_pos : LONG_MAX;
    at.start_pos = (int)start_pos;
    at.n = in;
    at.capacity = (int)cap;
    at.n_head = (int)Hq;
    at.n_head_kv = (int)Hkv;
    at.head_dim = (int)hd;
    at.window = ws + off_w;
    at.ctr = attn_ctr;
    at.ctr_ints = attn_ctr_ints;
    if (keep_win) {
      at.win_pad = kv->k_buffers[l]->kvwin.pad;
      at.win_valid = win_valid[l];
      at.window = kv->k_buffers[l]->kvwin.dev;
      at.part = reinterpret_cast<float *>(ws + off_w + attention_window_bytes(probe_at));
    }
    const AttnWindowLayout wl = attention_window_layout(at);
    RopeWindowTarget wt{};
    wt.k = reinterpret_cast<uint16_t *>(at.window);
    wt.vt = wt.k + Hkv * (size_t)wl.pad * hd;
    wt.j0 = (int)(start_pos - wl.lo);
    wt.pad = wl.pad;
    wt.vst = wl.vst;
    uint8_t *k_dst = staged ? stg_k : ring_k, *v_dst = staged ? stg_v : ring_v;
    const int slot0 = staged ? 0 : (int)(start_pos % cap), wrap = staged ? in : (int)cap;
    // 2. q, k, v projections as one segmented GEMM. Without QK-norm and with a full-width
    // rotation its epilogue also runs 3-4 (RoPE, Q8_0 of k and v, window entries); a
    // ubatch of at most 4 tokens takes the GEMV and the separate kernel.
    const bool fuse_rope = !unfused && !opt_f32(T.attn_q_norm) && !opt_f32(T.attn_k_norm) &&
                           cfg->rope_dim == (int)hd && (hd == 64 || hd == 128) && n > 4;
    GemmArgs g{};
    g.x = dp<const uint16_t>(scratch->h);
    g.m = in;
    g.k = (int)D;
    g.ldx = (int)D;
    g.epi = fuse_rope ? EPI_ROPE : EPI_F16;
    g.seg[0] = GemmSegment{pq, scratch->q->dev, (int)qd, (int)qd, 0, opt_f32(T.attn_q_bias)};
    g.seg[1] = GemmSegment{pk, scratch->k->dev, (int)kvd, (int)kvd, 0, opt_f32(T.attn_k_bias)};
    g.seg[2] = GemmSegment{pv, scratch->v->dev, (int)kvd, (int)kvd, 0, opt_f32(T.attn_v_bias)};
    g.nseg = 3;
    g.part = gemm_part;
    g.part_bytes = gemm_ws;
    if (fuse_rope) g.rope = GemmRope{rope_tab, cfg->rope_mode, (int)hd, k_dst, v_dst, slot0, wrap, (int)bpp, wt};
    if ((rc = timed_gemm(ctx, PROF_GEMM_QKV, gemm_flop(g), gemm_bytes(g),
                         [&](const LaunchStamp *st) { return launch_gemm_q4_0(g, s, nullptr, st); })))
      return rc;
    bool wrote_window = fuse_rope;
    // 3-4. RoPE on q and k, Q8_0 of k and v into the ring (or staging when wrapping)
    if (!fuse_rope && (rc = timed(ctx, PROF_ROPE_KV, 0, 2.0 * n * (qd + 2 * kvd) + 2.0 * n * qd + 2.0 * n * bpp, [&] {
           return launch_rope_qkv_store(dp<uint16_t>(scratch->q), dp<const uint16_t>(scratch->k),
                                        dp<const uint16_t>(scratch->v), (int)Hq, (int)Hkv, (int)hd,
                                        cfg->rope_dim, rope_tab, cfg->rope_mode, in, k_dst, v_dst, slot0,
                                        wrap, opt_f32(T.attn_q_norm), opt_f32(T.attn_k_norm), cfg->eps, s, &wt,
                                        &wrote_window);
         })))
      return rc;
    at.win_new_done = wrote_window ? 1 : 0;
    // 5. causal GQA attention
    double keys = 0;  // sum over queries of visible keys
    for (size_t t = 0; t < n; t++) keys += (double)std::min(start_pos + t + 1, cap);
    const double kv_read = 2.0 * (double)std::min(start_pos + n, cap) * bpp;
    if ((rc = timed(ctx, PROF_ATTN, 4.0 * hd * Hq * keys, 4.0 * n * qd + kv_read, [&] { return launch_attention(at, s); }))) return rc;
    if (staged) {
      const size_t keep = std::min(n, cap);
      const size_t first = n - keep;
      if ((rc = timed(ctx, PROF_ROPE_KV, 0, 4.0 * keep * bpp, [&] {
             int32_t r = launch_ring_commit(stg_k + first * bpp, ring_k, bpp, (int)((start_pos + first) % cap), (int)cap, (int)keep, s);
             return r ? r : launch_ring_commit(stg_v + first * bpp, ring_v, bpp, (int)((start_pos + first) % cap), (int)cap, (int)keep, s);
           })))
        return rc;
    }
    // 6-7. output projection, residual add fused: x += f16(Wo a)
    GemmArgs go{};
    go.x = dp<const uint16_t>(scratch->attn_out);
    go.m = in;
    go.k = (int)qd;
    go.ldx = (int)qd;
    go.epi = EPI_RESID;
    go.seg[0] = GemmSegment{po, xres, (int)D, (int)D, 0};
    go.nseg = 1;
    go.part = gemm_part;
    go.part_bytes = gemm_ws;
    go.norm_w = dp<const float>(T.ffn_norm);
    go.norm_out = dp<uint16_t>(scratch->h);
    go.norm_eps = cfg->eps;
    if (unfused) {
      go.epi = EPI_F16;
      go.seg[0].out = scratch->ffn_down->dev;
      go.norm_w = nullptr;
      go.norm_out = nullptr;
      h_ready = false;
      if ((rc = launch_gemm_q4_0(go, s)) ||
          (rc = launch_add_f16_to_f32(xres, dp<const uint16_t>(scratch->ffn_down), n * D, s)))
        return rc;
    } else if ((rc = timed_gemm(ctx, PROF_GEMM_O, gemm_flop(go), gemm_bytes(go),
                                [&](const LaunchStamp *st) { return launch_gemm_q4_0(go, s, &h_ready, st); })))
      return rc;
    // 8. FFN RMSNorm
    if (!h_ready && (rc = timed(ctx, PROF_NORM, 0, 6.0 * n * D + 4.0 * D, [&] {
                       return launch_rmsnorm_f32(xres, dp<const float>(T.ffn_norm), dp<uint16_t>(scratch->h),
                                                 nullptr, (int)D, cfg->eps, in, s);
                     })))
      return rc;
    // 9-10. gate and up projections with SwiGLU fused into the epilogue
    GemmArgs gu{};
    gu.x = dp<const uint16_t>(scratch->h);
    gu.m = in;
    gu.k = (int)D;
    gu.ldx = (int)D;
    gu.epi = EPI_SWIGLU;
    gu.seg[0] = GemmSegment{pgu, scratch->ffn_swiglu->dev, (int)F, (int)F, 0};
    gu.nseg = 1;
    if (unfused) {
      // gate and up as separate f16 GEMMs, then silu(gate) * up
      const uint8_t *pg, *pu;
      if ((rc = get_q4_panels(ctx, T.ffn_gate_scales, T.ffn_gate_quants, nullptr, nullptr, (int)F, (int)D, &pg)) ||
          (rc = get_q4_panels(ctx, T.ffn_up_scales, T.ffn_up_quants, nullptr, nullptr, (int)F, (int)D, &pu)))
        return rc;
      gu.epi = EPI_F16;
      gu.part = gemm_part;
      gu.part_bytes = gemm_ws;
      gu.seg[0] = GemmSegment{pg, scratch->ffn_gate->dev, (int)F, (int)F, 0};
      if ((rc = launch_gemm_q4_0(gu, s))) return rc;
      gu.seg[0] = GemmSegment{pu, scratch->ffn_up->dev, (int)F, (int)F, 0};
      if ((rc = launch_gemm_q4_0(gu, s)) ||
          (rc = launch_silu_mul(dp<const uint16_t>(scratch->ffn_gate), dp<const uint16_t>(scratch->ffn_up),
                                dp<uint16_t>(scratch->ffn_swiglu), n * F, s)))
        return rc;
    } else if ((rc = timed_gemm(ctx, PROF_GEMM_GATE_UP, gemm_flop(gu), gemm_bytes(gu),
                                [&](const LaunchStamp *st) { return launch_gemm_q4_0(gu, s, nullptr, st); })))
      return rc;
    // 11-12. down projection, residual add fused
    GemmArgs gd{};
    gd.x = dp<const uint16_t>(scratch->ffn_swiglu);
    gd.m = in;
    gd.k = (int)F;
    gd.ldx = (int)F;
    gd.epi = EPI_RESID;
    gd.seg[0] = GemmSegment{pd, xres, (int)D, (int)D, 0};
    gd.nseg = 1;
    gd.part = gemm_part;
    gd.part_bytes = gemm_ws;
    const bool last = l + 1 == L;
    // the wake-up of the final wait is gated here, some 50-100 us before the end
    if (last && (rc = gate())) return rc;
    gd.norm_w = dp<const float>(last ? tensors->output_norm : tensors->layers[l + 1].attn_norm);
    gd.norm_out = dp<uint16_t>(scratch->h);
    gd.norm_x16 = last ? dp<uint16_t>(scratch->x) : nullptr;
    gd.norm_eps = cfg->eps;
    if (unfused) {
      gd.epi = EPI_F16;
      gd.seg[0].out = scratch->ffn_down->dev;
      gd.norm_w = nullptr;
      gd.norm_out = gd.norm_x16 = nullptr;
      h_ready = false;
      if ((rc = launch_gemm_q4_0(gd, s)) ||
          (rc = launch_add_f16_to_f32(xres, dp<const uint16_t>(scratch->ffn_down), n * D, s)))
        return rc;
    } else if ((rc = timed_gemm(ctx, PROF_GEMM_DOWN, gemm_flop(gd), gemm_bytes(gd),
                                [&](const LaunchStamp *st) { return launch_gemm_q4_0(gd, s, &h_ready, st); })))
      return rc;
  }
  // 13. output RMSNorm of all n rows (h), final residual back to scratch.x as f16
  if (!h_ready && (rc = timed(ctx, PROF_NORM, 0, 8.0 * n * D + 4.0 * D, [&] {
                     return launch_rmsnorm_f32(xres, dp<const float>(tensors->output_norm), dp<uint16_t>(scratch->h),
                                               dp<uint16_t>(scratch->x), (int)D, cfg->eps, in, s);
                   })))
    return rc;
  // 14. logits of the last token
  const char *hlast = reinterpret_cast<const char *>(scratch->h->dev) + (n - 1) * D * 2;
  if ((rc = timed_gemm(ctx, PROF_GEMM_LM_HEAD, 2.0 * V * D, V * D * 18.0 / 32.0 + 2.0 * D + 4.0 * V,
                       [&](const LaunchStamp *st) {
                         return gemm_plain(ctx, tensors->output_scales, tensors->output_quants, hlast,
                                           scratch->logits->dev, V, D, 1, EPI_F32, false, st);
                       })))
    return rc;
  // Optional per-position logits / top-1.
  if (outputs && (outputs->logits_all || outputs->argmax_all)) {
    for (size_t r0 = 0; r0 < n; r0 += (outputs->logits_all ? n : chunk_rows)) {
      const size_t rows = outputs->logits_all ? n : std::min(chunk_rows, n - r0);
      float *lg = outputs->logits_all ? dp<float>(outputs->logits_all) + r0 * V
                                      : reinterpret_cast<float *>(ws + off_l);
      const char *hx = reinterpret_cast<const char *>(scratch->h->dev) + r0 * D * 2;
      if ((rc = gemm_plain(ctx, tensors->output_scales, tensors->output_quants, hx, lg, V, D, rows, EPI_F32))) return rc;
      if (want_argmax &&
          (rc = launch_argmax_rows(lg, (int)rows, (int)V, dp<int32_t>(outputs->argmax_all) + r0, s)))
        return rc;
    }
  }
  return SULIMO_HIP_OK;
  };

  if (!ctx->graph_replay || ctx->prof || want_outputs) {
    // Eager launches. With per-position outputs the LM head over all rows follows the
    // gate point, so the wake-up is not gated (the host function ends the queue).
    rc = body([&]() -> int32_t {
      if (!want_outputs) SULIMO_HIP_TRY(hipEventRecord(ctx->near_event, s));
      return SULIMO_HIP_OK;
    });
    if (rc) return rc;
  } else {
    // Graph replay: the key holds every value the launches are built from.
    std::vector<uint64_t> key;
    auto put = [&](uint64_t v) { key.push_back(v); };
    auto putp = [&](const void *p) { key.push_back((uint64_t)(uintptr_t)p); };
    auto putf = [&](float f) {
      uint32_t u;
      memcpy(&u, &f, 4);
      key.push_back(u);
    };
    put(L); put(D); put(F); put(Hq); put(Hkv); put(hd); put((uint64_t)cfg->rope_dim); put(V);
    put((uint64_t)cfg->rope_mode); putf(cfg->rope_base); putf(cfg->eps);
    put(start_pos); put(n); put(cap);
    putp(ws); put(gemm_ws); putp(lm_panel); putp(tensors->output_norm->dev); putp(attn_ctr);
    for (sulimo_hip_buffer *b : {scratch->x, scratch->h, scratch->q, scratch->k, scratch->v, scratch->attn_out,
                                 scratch->ffn_swiglu, scratch->logits})
      putp(b->dev);
    for (size_t l = 0; l < L; l++) {
      const sulimo_hip_layer_tensors &T = tensors->layers[l];
      for (int i = 0; i < 6; i++) putp(panels[6 * l + i]);
      putp(T.attn_norm->dev); putp(T.ffn_norm->dev);
      putp(opt_f32(T.attn_q_bias)); putp(opt_f32(T.attn_k_bias)); putp(opt_f32(T.attn_v_bias));
      putp(opt_f32(T.attn_q_norm)); putp(opt_f32(T.attn_k_norm));
      putp(kv->k_buffers[l]->dev); putp(kv->v_buffers[l]->dev);
      if (keep_win) {
        putp(kv->k_buffers[l]->kvwin.dev);
        put((uint64_t)kv->k_buffers[l]->kvwin.pad);
        put((uint64_t)win_valid[l]);
      }
    }
    PrefillGraph *hit = nullptr;
    for (PrefillGraph &g : ctx->graphs)
      if (g.key == key) hit = &g;
    if (!hit) {
      hipGraph_t g1 = nullptr, g2 = nullptr;
      SULIMO_HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      bool split = false;
      int32_t brc = body([&]() -> int32_t {
        hipError_t e = hipStreamEndCapture(s, &g1);
        if (e != hipSuccess) return hip_fail(e, "graph capture");
        e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return hip_fail(e, "graph capture");
        split = true;
        return SULIMO_HIP_OK;
      });
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      hipError_t ce = hipStreamIsCapturing(s, &cs);
      if (ce == hipSuccess && cs != hipStreamCaptureStatusNone) ce = hipStreamEndCapture(s, &g2);
      PrefillGraph pg;
      pg.key = std::move(key);
      if (brc == SULIMO_HIP_OK && ce == hipSuccess && split && g1 && g2) {
        ce = hipGraphInstantiate(&pg.pre, g1, nullptr, nullptr, 0);
        if (ce == hipSuccess) ce = hipGraphInstantiate(&pg.post, g2, nullptr, nullptr, 0);
      } else if (brc == SULIMO_HIP_OK && ce == hipSuccess) {
        ce = hipErrorInvalidValue;
      }
      if (g1) hipGraphDestroy(g1);
      if (g2) hipGraphDestroy(g2);
      if (brc || ce != hipSuccess) {
        if (pg.pre) hipGraphExecDestroy(pg.pre);
        if (pg.post) hipGraphExecDestroy(pg.post);
        return brc ? brc : hip_fail(ce, "prefill graph capture");
      }
      if (ctx->graphs.size() >= 8) {  // evict the least recently used
        auto lru = std::min_element(ctx->graphs.begin(), ctx->graphs.end(),
                                    [](const PrefillGraph &a, const PrefillGraph &b) { return a.last_use < b.last_use; });
        hipGraphExecDestroy(lru->pre);
        hipGraphExecDestroy(lru->post);
        ctx->graphs.erase(lru);
      }
      ctx->graphs.push_back(std::move(pg));
      hit = &ctx->graphs.back();
    }
    hit->last_use = ++ctx->graph_tick;
    SULIMO_HIP_TRY(hipGraphLaunch(hit->pre, s));
    SULIMO_HIP_TRY(hipEventRecord(ctx->near_event, s));
    SULIMO_HIP_TRY(hipGraphLaunch(hit->post, s));
  }
  // 15. one wait for the whole ubatch (the thread sleeps while the GPU works)
  rc = wait_parked(ctx, want_outputs ? nullptr : ctx->near_event);
  if (rc == SULIMO_HIP_OK && keep_win) {
    for (size_t l = 0; l < L; l++) {  // the kept windows now hold positions [0, start_pos + n)
      KvWindowCache &wc = kv->k_buffers[l]->kvwin;
      wc.len = (long)(start_pos + n);
      wc.k_ver = kv->k_buffers[l]->version;
      wc.v_ver = kv->v_buffers[l]->version;
    }
  }
  if (ctx->prof) {
    prof_collect(ctx);
    ctx->stats.prefill_calls++;
  }
  return rc;
}

int32_t sulimo_hip_execute_prefill_ubatch(sulimo_hip_ctx *ctx, const sulimo_hip_model_config *cfg,
                                          const sulimo_hip_model_tensors *tensors,
                                          sulimo_hip_kv_cache *kv_cache,
                                          sulimo_hip_prefill_scratch *scratch, size_t start_pos,
                                          size_t n) {
  return sulimo_hip_execute_prefill_ubatch_ex(ctx, cfg, tensors, kv_cache, scratch, start_pos, n,
                                              nullptr);
}

}  // extern "C"
