/*
 * oracle.c - CPU restatement of Sulimo's Q4_0 prefill path (test infrastructure only;
 * see oracle.h for the contract and the parity pins).
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -mf16c -ffp-contract=off -fopenmp).
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* f16 helpers: the `half` crate's to_f32 (exact) and from_f32 (RNE).        */
/* ------------------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
uint16_t orc_f32_to_f16(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_u16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}

/* ------------------------------------------------------------------------- */
/* Q4_0 (crates/sulimo-core/src/repack.rs)                                   */
/* ------------------------------------------------------------------------- */

/* repack_q4_0_aos_to_soa, repack.rs:45-80. Returns blocks, or -1/-2/-3 for the
 * InvalidAosLength / ScalesBufferTooSmall / QuantsBufferTooSmall errors. */
int64_t orc_repack_q4_0_aos_to_soa(const uint8_t *aos, size_t aos_len, uint8_t *scales,
                                   size_t scales_len, uint8_t *quants, size_t quants_len) {
  if (aos_len % 18 != 0) return -1;
  size_t nb = aos_len / 18;
  if (scales_len < nb * 2) return -2;
  if (quants_len < nb * 16) return -3;
  for (size_t b = 0; b < nb; b++) {
    memcpy(scales + b * 2, aos + b * 18, 2);
    memcpy(quants + b * 16, aos + b * 18 + 2, 16);
  }
  return (int64_t)nb;
}

/* dequantize_q4_0_aos, repack.rs:84-104: element i = (lo(qs[i])-8)*d,
 * element i+16 = (hi(qs[i])-8)*d. */
void orc_dequant_q4_0_aos(const uint8_t *aos, size_t nblocks, float *out) {
  for (size_t b = 0; b < nblocks; b++) {
    const uint8_t *blk = aos + b * 18;
    float d = orc_f16_to_f32(rd_u16(blk));
    for (int i = 0; i < 16; i++) {
      uint8_t q = blk[2 + i];
      out[b * 32 + i] = (float)((int)(q & 0x0F) - 8) * d;
      out[b * 32 + i + 16] = (float)((int)(q >> 4) - 8) * d;
    }
  }
}

/* dequantize_q4_0_soa, repack.rs:107-131. */
void orc_dequant_q4_0_soa(const uint8_t *scales, const uint8_t *quants, size_t nblocks,
                          float *out) {
  for (size_t b = 0; b < nblocks; b++) {
    float d = orc_f16_to_f32(rd_u16(scales + b * 2));
    const uint8_t *qs = quants + b * 16;
    for (int i = 0; i < 16; i++) {
      out[b * 32 + i] = (float)((int)(qs[i] & 0x0F) - 8) * d;
      out[b * 32 + i + 16] = (float)((int)(qs[i] >> 4) - 8) * d;
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Q8_0 (crates/sulimo-core/src/kv_cache.rs)                                 */
/* ------------------------------------------------------------------------- */

/* quantize_f32_to_q8_0, kv_cache.rs:162-193: d = amax/127 (f32), stored as
 * f16(d); id = d != 0 ? 1/d : 0 with the f32 d; code = clamp(round(x*id)). */
void orc_quantize_f32_to_q8_0(const float *src, size_t n, uint8_t *dst) {
  size_t nb = n / 32;
  for (size_t b = 0; b < nb; b++) {
    const float *s = src + b * 32;
    uint8_t *o = dst + b * 34;
    float max_abs = 0.0f;
    for (int i = 0; i < 32; i++) {
      float a = fabsf(s[i]);
      if (a > max_abs) max_abs = a;
    }
    float d = max_abs / 127.0f;
    wr_u16(o, orc_f32_to_f16(d));
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) {
      float q = roundf(s[i] * id);
      if (q < -128.0f) q = -128.0f;
      if (q > 127.0f) q = 127.0f;
      o[2 + i] = (uint8_t)(int8_t)q;
    }
  }
}

/* dequantize_q8_0_to_f32, kv_cache.rs:195-209. */
void orc_dequant_q8_0(const uint8_t *src, size_t nblocks, float *dst) {
  for (size_t b = 0; b < nblocks; b++) {
    const uint8_t *blk = src + b * 34;
    float d = orc_f16_to_f32(rd_u16(blk));
    for (int i = 0; i < 32; i++) dst[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
  }
}

/* ------------------------------------------------------------------------- */
/* GEMM scalar reference (crates/sulimo-ocl/src/gemm.rs:106-147)             */
/* ------------------------------------------------------------------------- */

/* Core of gemm_q4_0_f16_scalar_reference for tokens given as f32 in a
 * token-interleaved layout xt[k][8] (8 tokens per group). Each SIMD lane is one
 * token and performs, in the same order, the scalar reference's operations:
 *   block_sum += x_lo*q_lo + x_hi*q_hi  (two products, one add, one accumulate)
 *   acc += block_sum * d
 * Products of an f16 value and an integer in [-8,7] are exact in f32, so only
 * the adds round, exactly as in the scalar loop. Rows are independent, so the
 * OpenMP split over rows does not change any result. */
static void gemm_q4_rows_x8(const uint8_t *scales, const uint8_t *quants, const float *xt,
                            size_t m, size_t k, float *acc_out /* [m][8] */) {
  size_t nb = k / 32;
#pragma omp parallel for schedule(static)
  for (size_t r = 0; r < m; r++) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
      float d = orc_f16_to_f32(rd_u16(scales + (r * nb + b) * 2));
      const uint8_t *qs = quants + (r * nb + b) * 16;
      const float *xb = xt + b * 32 * 8;
      __m256 bs = _mm256_setzero_ps();
      for (int i = 0; i < 16; i++) {
        __m256 ql = _mm256_set1_ps((float)((int)(qs[i] & 0x0F) - 8));
        __m256 qh = _mm256_set1_ps((float)((int)((qs[i] >> 4) & 0x0F) - 8));
        __m256 xl = _mm256_loadu_ps(xb + i * 8);
        __m256 xh = _mm256_loadu_ps(xb + (16 + i) * 8);
        __m256 t = _mm256_add_ps(_mm256_mul_ps(xl, ql), _mm256_mul_ps(xh, qh));
        bs = _mm256_add_ps(bs, t);
      }
      acc = _mm256_add_ps(acc, _mm256_mul_ps(bs, _mm256_set1_ps(d)));
    }
    _mm256_storeu_ps(acc_out + r * 8, acc);
  }
}

/* out_f32[t][r] for tokens given as f32 rows x[n][k]. */
static int gemm_q4_f32x(const uint8_t *scales, const uint8_t *quants, const float *x, size_t m,
                        size_t k, size_t n, float *out, size_t ldo) {
  float *xt = (float *)malloc(k * 8 * sizeof(float));
  float *acc = (float *)malloc(m * 8 * sizeof(float));
  if (!xt || !acc) {
    free(xt);
    free(acc);
    return -1;
  }
  for (size_t t0 = 0; t0 < n; t0 += 8) {
    size_t cnt = n - t0 < 8 ? n - t0 : 8;
    for (size_t kk = 0; kk < k; kk++)
      for (size_t j = 0; j < 8; j++) xt[kk * 8 + j] = j < cnt ? x[(t0 + j) * k + kk] : 0.0f;
    gemm_q4_rows_x8(scales, quants, xt, m, k, acc);
    for (size_t j = 0; j < cnt; j++)
      for (size_t r = 0; r < m; r++) out[(t0 + j) * ldo + r] = acc[r * 8 + j];
  }
  free(xt);
  free(acc);
  return 0;
}

void orc_gemm_q4_0_f16_scalar_reference(const uint16_t *scales, const uint8_t *quants,
                                        const uint16_t *x, size_t m, size_t k, size_t n,
                                        uint16_t *out) {
  float *xf = (float *)malloc(n * k * sizeof(float));
  float *of = (float *)malloc(n * m * sizeof(float));
  if (!xf || !of) {
    free(xf);
    free(of);
    return;
  }
  for (size_t i = 0; i < n * k; i++) xf[i] = orc_f16_to_f32(x[i]);
  gemm_q4_f32x((const uint8_t *)scales, quants, xf, m, k, n, of, m);
  for (size_t i = 0; i < n * m; i++) out[i] = orc_f32_to_f16(of[i]);
  free(xf);
  free(of);
}

/* ------------------------------------------------------------------------- */
/* CPU kernels (crates/sulimo-cpu/src/scalar.rs, avx2.rs)                    */
/* ------------------------------------------------------------------------- */

/* vec_dot_q4_0_q8_0_scalar, scalar.rs:173-205. */
float orc_vec_dot_q4_0_q8_0_scalar(const uint8_t *w_scales, const uint8_t *w_quants,
                                   const uint8_t *x_q8, size_t nblocks) {
  float total = 0.0f;
  for (size_t b = 0; b < nblocks; b++) {
    float ws = orc_f16_to_f32(rd_u16(w_scales + b * 2));
    float xs = orc_f16_to_f32(rd_u16(x_q8 + b * 34));
    float d = ws * xs;
    const uint8_t *wq = w_quants + b * 16;
    const int8_t *xq = (const int8_t *)(x_q8 + b * 34 + 2);
    int32_t bsum = 0;
    for (int i = 0; i < 16; i++) {
      int w0 = (int)(wq[i] & 0x0F) - 8, w1 = (int)(wq[i] >> 4) - 8;
      bsum += w0 * xq[i] + w1 * xq[i + 16];
    }
    total += (float)bsum * d;
  }
  return total;
}

/* hsum_256, avx2.rs:331-342. */
static inline float hsum_256(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 s = _mm_add_ps(lo, hi);
  __m128 sh = _mm_movehdup_ps(s);
  __m128 sums = _mm_add_ps(s, sh);
  __m128 sh2 = _mm_movehl_ps(sums, sums);
  return _mm_cvtss_f32(_mm_add_ss(sums, sh2));
}

/* vec_dot_q4_0_q8_0_avx2, avx2.rs:113-164 (same instruction sequence). */
float orc_vec_dot_q4_0_q8_0_avx2(const uint8_t *w_scales, const uint8_t *w_quants,
                                 const uint8_t *x_q8, size_t nblocks) {
  __m256 acc = _mm256_setzero_ps();
  const __m128i mask_low = _mm_set1_epi8(0x0F);
  const __m128i eight = _mm_set1_epi8(8);
  for (size_t b = 0; b < nblocks; b++) {
    float ws = orc_f16_to_f32(rd_u16(w_scales + b * 2));
    float xs = orc_f16_to_f32(rd_u16(x_q8 + b * 34));
    float d = ws * xs;
    __m128i w128 = _mm_loadu_si128((const __m128i *)(w_quants + b * 16));
    __m128i w_low = _mm_sub_epi8(_mm_and_si128(w128, mask_low), eight);
    __m128i w_high = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(w128, 4), mask_low), eight);
    __m256i w256 = _mm256_set_m128i(w_high, w_low);
    __m256i x256 = _mm256_loadu_si256((const __m256i *)(x_q8 + b * 34 + 2));
    __m256i w_lo_16 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(w256, 0));
    __m256i w_hi_16 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(w256, 1));
    __m256i x_lo_16 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(x256, 0));
    __m256i x_hi_16 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(x256, 1));
    __m256i prod_lo = _mm256_madd_epi16(w_lo_16, x_lo_16);
    __m256i prod_hi = _mm256_madd_epi16(w_hi_16, x_hi_16);
    __m256 sum_ps = _mm256_cvtepi32_ps(_mm256_add_epi32(prod_lo, prod_hi));
    acc = _mm256_fmadd_ps(sum_ps, _mm256_set1_ps(d), acc);
  }
  return hsum_256(acc);
}

/* matvec_q4_0_q8_0_avx2, avx2.rs:172-190 (single thread, as forward_token). */
void orc_matvec_q4_0_q8_0_avx2(const uint8_t *w_scales, const uint8_t *w_quants,
                               const uint8_t *x_q8, size_t rows, size_t cols, float *out) {
  size_t bpr = cols / 32;
  for (size_t r = 0; r < rows; r++)
    out[r] = orc_vec_dot_q4_0_q8_0_avx2(w_scales + r * bpr * 2, w_quants + r * bpr * 16, x_q8,
                                        bpr);
}

/* The same rows split over `threads` OpenMP threads, as ThreadPool::execute_parallel
 * splits matvec rows (crates/sulimo-cpu/src/thread_pool.rs:98-126). Each row is one
 * independent dot, so the result equals the single-thread matvec bit for bit. */
static void matvec_threads(const uint8_t *w_scales, const uint8_t *w_quants, const uint8_t *x_q8,
                           size_t rows, size_t cols, float *out, int threads) {
  if (threads <= 1) {
    orc_matvec_q4_0_q8_0_avx2(w_scales, w_quants, x_q8, rows, cols, out);
    return;
  }
  size_t bpr = cols / 32;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (size_t r = 0; r < rows; r++)
    out[r] = orc_vec_dot_q4_0_q8_0_avx2(w_scales + r * bpr * 2, w_quants + r * bpr * 16, x_q8,
                                        bpr);
}

/* rmsnorm_scalar, scalar.rs:23-38. */
void orc_rmsnorm_scalar(const float *x, const float *w, float eps, size_t n, float *out) {
  float sum_sq = 0.0f;
  for (size_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
  float mean = sum_sq / (float)n;
  float scale = 1.0f / sqrtf(mean + eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* rmsnorm_avx2, avx2.rs:197-226. */
void orc_rmsnorm_avx2(const float *x, const float *w, float eps, size_t n, float *out) {
  size_t chunks = n / 8;
  __m256 ssv = _mm256_setzero_ps();
  for (size_t i = 0; i < chunks; i++) {
    __m256 xv = _mm256_loadu_ps(x + i * 8);
    ssv = _mm256_fmadd_ps(xv, xv, ssv);
  }
  float sum_sq = hsum_256(ssv);
  for (size_t i = chunks * 8; i < n; i++) sum_sq += x[i] * x[i];
  float mean = sum_sq / (float)n;
  float scale = 1.0f / sqrtf(mean + eps);
  __m256 sv = _mm256_set1_ps(scale);
  for (size_t i = 0; i < chunks; i++) {
    __m256 xv = _mm256_loadu_ps(x + i * 8);
    __m256 wv = _mm256_loadu_ps(w + i * 8);
    _mm256_storeu_ps(out + i * 8, _mm256_mul_ps(_mm256_mul_ps(xv, sv), wv));
  }
  for (size_t i = chunks * 8; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* rope_head_scalar, scalar.rs:92-130 (no frequency factors). mode 0 = Norm, 1 = NeoX. */
void orc_rope_head_scalar(float *vec, size_t pos, size_t rope_dim, float freq_base, int mode) {
  size_t half = rope_dim / 2;
  for (size_t i = 0; i < half; i++) {
    float freq = 1.0f / powf(freq_base, (float)(2 * i) / (float)rope_dim);
    float theta = (float)pos * freq;
    float c = cosf(theta), s = sinf(theta);
    size_t i0 = mode == 0 ? 2 * i : i;
    size_t i1 = mode == 0 ? 2 * i + 1 : i + half;
    float v0 = vec[i0], v1 = vec[i1];
    vec[i0] = v0 * c - v1 * s;
    vec[i1] = v0 * s + v1 * c;
  }
}

/* softmax_scalar, scalar.rs:133-158. */
void orc_softmax_scalar(float *x, size_t n) {
  if (n == 0) return;
  float mx = x[0];
  for (size_t i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    float e = expf(x[i] - mx);
    x[i] = e;
    sum += e;
  }
  if (sum > 0.0f) {
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
  }
}

/* swiglu_scalar, scalar.rs:161-170. */
void orc_swiglu_scalar(const float *gate, const float *up, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) {
    float g = gate[i];
    float silu = g / (1.0f + expf(-g));
    out[i] = silu * up[i];
  }
}

/* causal_gqa_decode_scalar_ext, scalar.rs:287-359 (no soft-cap). */
void orc_causal_gqa_decode_scalar(const float *q, const uint8_t *k_ring, const uint8_t *v_ring,
                                  size_t bytes_per_pos, size_t capacity, size_t first_pos,
                                  size_t context_len, size_t head_count, size_t head_count_kv,
                                  size_t head_dim, float *scores, float *deq, float *out) {
  size_t heads_per_kv = head_count / head_count_kv;
  float scale = 1.0f / sqrtf((float)head_dim);
  size_t head_bytes = (head_dim / 32) * 34;
  for (size_t h = 0; h < head_count; h++) {
    size_t kvh = h / heads_per_kv;
    const float *qh = q + h * head_dim;
    for (size_t j = 0; j < context_len; j++) {
      size_t slot = (first_pos + j) % capacity;
      orc_dequant_q8_0(k_ring + slot * bytes_per_pos + kvh * head_bytes, head_dim / 32, deq);
      float dot = 0.0f;
      for (size_t d = 0; d < head_dim; d++) dot += qh[d] * deq[d];
      scores[j] = dot * scale;
    }
    orc_softmax_scalar(scores, context_len);
    float *oh = out + h * head_dim;
    for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
    for (size_t j = 0; j < context_len; j++) {
      size_t slot = (first_pos + j) % capacity;
      orc_dequant_q8_0(v_ring + slot * bytes_per_pos + kvh * head_bytes, head_dim / 32, deq);
      for (size_t d = 0; d < head_dim; d++) oh[d] += scores[j] * deq[d];
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Reference GPU kernels restated (kernels/prefill.cl)                       */
/* ------------------------------------------------------------------------- */

/* rmsnorm_f16_f32w, prefill.cl:4-29. */
void orc_cl_rmsnorm_f16_f32w(const uint16_t *x, const float *w, uint16_t *out, int d, float eps,
                             int n) {
  for (int t = 0; t < n; t++) {
    const uint16_t *xr = x + (size_t)t * d;
    float ss = 0.0f;
    for (int i = 0; i < d; i++) {
      float v = orc_f16_to_f32(xr[i]);
      ss += v * v;
    }
    float mean = ss / (float)d;
    float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < d; i++)
      out[(size_t)t * d + i] = orc_f32_to_f16(orc_f16_to_f32(xr[i]) * scale * w[i]);
  }
}

/* rope_f16, prefill.cl:32-68: pos = start_pos + n, fp32 rotation, f16 result. */
void orc_cl_rope_f16(uint16_t *vec, int head_count, int head_dim, int rope_dim, float freq_base,
                     int mode, int start_pos, int n) {
  int half = rope_dim / 2;
  for (int t = 0; t < n; t++)
    for (int h = 0; h < head_count; h++) {
      uint16_t *hp = vec + ((size_t)t * head_count + h) * head_dim;
      int pos = start_pos + t;
      for (int i = 0; i < half; i++) {
        float freq = 1.0f / powf(freq_base, (float)(2 * i) / (float)rope_dim);
        float theta = (float)pos * freq;
        float c = cosf(theta), s = sinf(theta);
        int i0 = mode == 0 ? 2 * i : i;
        int i1 = mode == 0 ? 2 * i + 1 : i + half;
        float v0 = orc_f16_to_f32(hp[i0]), v1 = orc_f16_to_f32(hp[i1]);
        hp[i0] = orc_f32_to_f16(v0 * c - v1 * s);
        hp[i1] = orc_f32_to_f16(v0 * s + v1 * c);
      }
    }
}

/* kv_store_q8_0, prefill.cl:72-116: same codes as quantize_f32_to_q8_0 applied to
 * the f16 activations (|x*id| <= 127 so the +-127 and [-128,127] clamps agree). */
void orc_cl_kv_store_q8_0(const uint16_t *act, uint8_t *kv, int start_pos, int capacity,
                          int blocks_per_pos, int n) {
  float blk[32];
  for (int t = 0; t < n; t++) {
    int ring = (start_pos + t) % capacity;
    for (int b = 0; b < blocks_per_pos; b++) {
      const uint16_t *in = act + ((size_t)t * blocks_per_pos + b) * 32;
      for (int i = 0; i < 32; i++) blk[i] = orc_f16_to_f32(in[i]);
      orc_quantize_f32_to_q8_0(blk, 32, kv + ((size_t)ring * blocks_per_pos + b) * 34);
    }
  }
}

/* silu_mul_f16, prefill.cl:240-253. */
void orc_cl_silu_mul_f16(const uint16_t *gate, const uint16_t *up, uint16_t *out, int total) {
  for (int i = 0; i < total; i++) {
    float g = orc_f16_to_f32(gate[i]), u = orc_f16_to_f32(up[i]);
    float silu = g / (1.0f + expf(-g));
    out[i] = orc_f32_to_f16(silu * u);
  }
}

/* add_f16, prefill.cl:256-266. */
void orc_cl_add_f16(uint16_t *a, const uint16_t *b, int total) {
  for (int i = 0; i < total; i++)
    a[i] = orc_f32_to_f16(orc_f16_to_f32(a[i]) + orc_f16_to_f32(b[i]));
}

/* logits_f16_output, prefill.cl:269-308: fp32 logits of row token_idx. */
void orc_cl_logits_f16_output(const uint16_t *x_all, const uint16_t *scales,
                              const uint8_t *quants, float *logits, int m, int k, int token_idx) {
  float *xf = (float *)malloc((size_t)k * sizeof(float));
  if (!xf) return;
  for (int i = 0; i < k; i++) xf[i] = orc_f16_to_f32(x_all[(size_t)token_idx * k + i]);
  gemm_q4_f32x((const uint8_t *)scales, quants, xf, (size_t)m, (size_t)k, 1, logits, (size_t)m);
  free(xf);
}

void orc_attention_prefill_f32(const float *q, const uint8_t *k_ring, const uint8_t *v_ring,
                               float *out, int start_pos, int capacity, int head_count,
                               int head_count_kv, int head_dim, int n) {
  size_t bpp = (size_t)head_count_kv * (head_dim / 32) * 34;
  size_t qd = (size_t)head_count * head_dim;
#pragma omp parallel
  {
    float *scores = (float *)malloc((size_t)capacity * sizeof(float));
    float *deq = (float *)malloc((size_t)head_dim * sizeof(float));
#pragma omp for schedule(dynamic, 4)
    for (int t = 0; t < n; t++) {
      if (!scores || !deq) continue;
      size_t P = (size_t)start_pos + t;
      size_t ctx = P + 1 < (size_t)capacity ? P + 1 : (size_t)capacity;
      size_t first = P + 1 - ctx;
      orc_causal_gqa_decode_scalar(q + t * qd, k_ring, v_ring, bpp, capacity, first, ctx,
                                   head_count, head_count_kv, head_dim, scores, deq,
                                   out + t * qd);
    }
    free(scores);
    free(deq);
  }
}

/* lookup_token_embedding_f16, scheduler.rs:329-374 (Q4_0 table):
 * out = d * f16(q-8) in f16 arithmetic, i.e. f16(f32(d) * (q-8)). */
void orc_lookup_token_embedding_f16(const uint8_t *scales, const uint8_t *quants, size_t embd,
                                    uint32_t token, uint16_t *out) {
  size_t bpr = embd / 32;
  const uint8_t *rs = scales + (size_t)token * bpr * 2;
  const uint8_t *rq = quants + (size_t)token * bpr * 16;
  for (size_t b = 0; b < bpr; b++) {
    float d = orc_f16_to_f32(rd_u16(rs + b * 2));
    for (int i = 0; i < 16; i++) {
      uint8_t byte = rq[b * 16 + i];
      float lo = orc_f16_to_f32(orc_f32_to_f16((float)((int)(byte & 0x0F) - 8)));
      float hi = orc_f16_to_f32(orc_f32_to_f16((float)((int)((byte >> 4) & 0x0F) - 8)));
      out[b * 32 + i] = orc_f32_to_f16(d * lo);
      out[b * 32 + 16 + i] = orc_f32_to_f16(d * hi);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* forward_token (crates/sulimo-engine/src/forward_pass.rs:190-417)          */
/* ------------------------------------------------------------------------- */

static size_t kv_bpp(const orc_config *c) { return (size_t)c->n_head_kv * (c->head_dim / 32) * 34; }

/* add_bias (forward_pass.rs:452-464) */
static void add_bias(const float *b, float *v, size_t n) {
  if (!b) return;
  for (size_t i = 0; i < n; i++) v[i] += b[i];
}

/* apply_head_norms (forward_pass.rs:466-491): RMSNorm of every head with the shared
 * [head_dim] weights (the non-Gemma form). */
static void head_norms(const float *w, float *v, size_t heads, size_t hd, float eps, float *buf) {
  if (!w) return;
  for (size_t h = 0; h < heads; h++) {
    memcpy(buf, v + h * hd, hd * 4);
    orc_rmsnorm_scalar(buf, w, eps, hd, v + h * hd);
  }
}

int orc_forward_token(const orc_model *m, orc_kv *kv, uint32_t token, size_t pos, float *logits) {
  return orc_forward_token_mt(m, kv, token, pos, logits, 1);
}

/* forward_token with its matvecs' rows split over `threads` threads (1 = the
 * reference's single-core path, forward_pass.rs:197 leaves its pool unused). */
int orc_forward_token_mt(const orc_model *m, orc_kv *kv, uint32_t token, size_t pos, float *logits,
                         int threads) {
  const orc_config *c = &m->cfg;
  size_t D = c->embd, F = c->ffn, hd = c->head_dim;
  size_t qd = (size_t)c->n_head * hd, kvd = (size_t)c->n_head_kv * hd;
  size_t bpp = kv_bpp(c);
  size_t cap = kv->capacity;
  size_t maxd = F > D ? F : D;
  if (qd > maxd) maxd = qd;
  float *x = malloc(D * 4), *h = malloc(D * 4), *q = malloc(qd * 4), *k = malloc(kvd * 4),
        *v = malloc(kvd * 4), *ao = malloc(qd * 4), *g = malloc(F * 4), *u = malloc(F * 4),
        *sw = malloc(F * 4), *dn = malloc(D * 4), *scores = malloc(cap * 4), *deq = malloc(hd * 4);
  uint8_t *q8 = malloc((maxd / 32 + 1) * 34), *q8f = malloc((F / 32 + 1) * 34);
  int rc = 0;
  if (!x || !h || !q || !k || !v || !ao || !g || !u || !sw || !dn || !scores || !deq || !q8 ||
      !q8f) {
    rc = -1;
    goto done;
  }
  /* 1. embedding (forward_pass.rs:419-450, Q4_0 row dequantized to f32) */
  orc_dequant_q4_0_soa(m->token_embd.scales + (size_t)token * (D / 32) * 2,
                       m->token_embd.quants + (size_t)token * (D / 32) * 16, D / 32, x);
  for (int l = 0; l < c->n_layers; l++) {
    const orc_layer *L = &m->layers[l];
    orc_rmsnorm_avx2(x, L->attn_norm, c->eps, D, h);
    orc_quantize_f32_to_q8_0(h, D, q8);
    matvec_threads(L->q.scales, L->q.quants, q8, qd, D, q, threads);
    matvec_threads(L->k.scales, L->k.quants, q8, kvd, D, k, threads);
    matvec_threads(L->v.scales, L->v.quants, q8, kvd, D, v, threads);
    add_bias(L->q_bias, q, qd);
    add_bias(L->k_bias, k, kvd);
    add_bias(L->v_bias, v, kvd);
    head_norms(L->q_norm, q, c->n_head, hd, c->eps, deq);
    head_norms(L->k_norm, k, c->n_head_kv, hd, c->eps, deq);
    for (int hh = 0; hh < c->n_head; hh++)
      orc_rope_head_scalar(q + hh * hd, pos, c->rope_dim, c->rope_base, c->rope_mode);
    for (int hh = 0; hh < c->n_head_kv; hh++)
      orc_rope_head_scalar(k + hh * hd, pos, c->rope_dim, c->rope_base, c->rope_mode);
    /* store_key / store_value (kv_cache.rs:93-111) */
    orc_quantize_f32_to_q8_0(k, kvd, kv->k[l] + (pos % cap) * bpp);
    orc_quantize_f32_to_q8_0(v, kvd, kv->v[l] + (pos % cap) * bpp);
    /* the reference attends over pos+1 keys; past capacity it keeps the last cap */
    size_t ctx = pos + 1 < cap ? pos + 1 : cap;
    orc_causal_gqa_decode_scalar(q, kv->k[l], kv->v[l], bpp, cap, pos + 1 - ctx, ctx,
                                 c->n_head, c->n_head_kv, hd, scores, deq, ao);
    orc_quantize_f32_to_q8_0(ao, qd, q8);
    matvec_threads(L->o.scales, L->o.quants, q8, D, qd, h, threads);
    for (size_t i = 0; i < D; i++) x[i] += h[i];
    orc_rmsnorm_avx2(x, L->ffn_norm, c->eps, D, h);
    orc_quantize_f32_to_q8_0(h, D, q8);
    matvec_threads(L->gate.scales, L->gate.quants, q8, F, D, g, threads);
    matvec_threads(L->up.scales, L->up.quants, q8, F, D, u, threads);
    orc_swiglu_scalar(g, u, F, sw);
    orc_quantize_f32_to_q8_0(sw, F, q8f);
    matvec_threads(L->down.scales, L->down.quants, q8f, D, F, dn, threads);
    for (size_t i = 0; i < D; i++) x[i] += dn[i];
  }
  orc_rmsnorm_avx2(x, m->output_norm, c->eps, D, h);
  orc_quantize_f32_to_q8_0(h, D, q8);
  matvec_threads(m->output.scales, m->output.quants, q8, c->vocab, D, logits, threads);
done:
  free(x); free(h); free(q); free(k); free(v); free(ao); free(g); free(u); free(sw); free(dn);
  free(scores); free(deq); free(q8); free(q8f);
  return rc;
}

/* ------------------------------------------------------------------------- */
/* fp32 reference prefill (op order of prefill.rs:362-560, rounding points of */
/* test_prefill.rs:582-885)                                                   */
/* ------------------------------------------------------------------------- */

static void round_f16_inplace(float *a, size_t n) {
  for (size_t i = 0; i < n; i++) a[i] = orc_f16_to_f32(orc_f32_to_f16(a[i]));
}

/* GEMM with f16 input rounding and f16 output rounding, as gemm_q4_0_f16_scalar_reference
 * on f16 buffers (values kept as f32 holding exact f16 numbers); an optional bias
 * [m] is added before the output rounding. */
static int gemm_f16io(orc_q4 w, const float *x16, size_t m, size_t k, size_t n, float *out,
                      const float *bias) {
  if (gemm_q4_f32x(w.scales, w.quants, x16, m, k, n, out, m)) return -1;
  if (bias)
    for (size_t t = 0; t < n; t++) add_bias(bias, out + t * m, m);
  round_f16_inplace(out, n * m);
  return 0;
}

int orc_prefill_reference(const orc_model *m, orc_kv *kv, const uint16_t *x_in, size_t start_pos,
                          size_t n, int all_logits, float *logits, float *h_final, float *x_final) {
  const orc_config *c = &m->cfg;
  size_t D = c->embd, F = c->ffn, hd = c->head_dim;
  size_t qd = (size_t)c->n_head * hd, kvd = (size_t)c->n_head_kv * hd;
  size_t bpp = kv_bpp(c), cap = kv->capacity;
  int rc = 0;
  float *x = malloc(n * D * 4), *h = malloc(n * D * 4), *q = malloc(n * qd * 4),
        *k = malloc(n * kvd * 4), *v = malloc(n * kvd * 4), *ao = malloc(n * qd * 4),
        *g = malloc(n * F * 4), *u = malloc(n * F * 4), *t2 = malloc(n * (qd > D ? qd : D) * 4);
  uint8_t *nk = malloc(n * bpp), *nv = malloc(n * bpp);
  if (!x || !h || !q || !k || !v || !ao || !g || !u || !t2 || !nk || !nv) {
    rc = -1;
    goto done;
  }
  for (size_t i = 0; i < n * D; i++) x[i] = orc_f16_to_f32(x_in[i]);
  for (int l = 0; l < c->n_layers && rc == 0; l++) {
    const orc_layer *L = &m->layers[l];
    for (size_t t = 0; t < n; t++) orc_rmsnorm_scalar(x + t * D, L->attn_norm, c->eps, D, h + t * D);
    round_f16_inplace(h, n * D);
    rc |= gemm_f16io(L->q, h, qd, D, n, q, L->q_bias);
    rc |= gemm_f16io(L->k, h, kvd, D, n, k, L->k_bias);
    rc |= gemm_f16io(L->v, h, kvd, D, n, v, L->v_bias);
    for (size_t t = 0; t < n; t++) {
      size_t pos = start_pos + t;
      head_norms(L->q_norm, q + t * qd, c->n_head, hd, c->eps, t2);
      head_norms(L->k_norm, k + t * kvd, c->n_head_kv, hd, c->eps, t2);
      for (int hh = 0; hh < c->n_head; hh++)
        orc_rope_head_scalar(q + t * qd + hh * hd, pos, c->rope_dim, c->rope_base, c->rope_mode);
      for (int hh = 0; hh < c->n_head_kv; hh++)
        orc_rope_head_scalar(k + t * kvd + hh * hd, pos, c->rope_dim, c->rope_base, c->rope_mode);
      orc_quantize_f32_to_q8_0(k + t * kvd, kvd, nk + t * bpp);
      orc_quantize_f32_to_q8_0(v + t * kvd, kvd, nv + t * bpp);
    }
    /* attention: sliding window of the last `cap` positions; positions before
     * start_pos come from the ring, new ones from this ubatch's staged codes. The
     * window's K/V rows are dequantized once per layer (Q8_0 dequantization is exact,
     * code * f32(d)), so every score and output sum sees the values and the order
     * of causal_gqa_decode_scalar. */
    {
      size_t lo = start_pos + 1 > cap ? start_pos + 1 - cap : 0;
      size_t span = start_pos + n - lo;
      float *kf = malloc(span * kvd * 4), *vf = malloc(span * kvd * 4);
      if (!kf || !vf) {
        free(kf);
        free(vf);
        rc = -1;
        break;
      }
#pragma omp parallel for schedule(static)
      for (size_t p = lo; p < start_pos + n; p++) {
        const uint8_t *kp = p < start_pos ? kv->k[l] + (p % cap) * bpp : nk + (p - start_pos) * bpp;
        const uint8_t *vp = p < start_pos ? kv->v[l] + (p % cap) * bpp : nv + (p - start_pos) * bpp;
        orc_dequant_q8_0(kp, kvd / 32, kf + (p - lo) * kvd);
        orc_dequant_q8_0(vp, kvd / 32, vf + (p - lo) * kvd);
      }
#pragma omp parallel
      {
        float *scores = malloc(cap * 4);
        size_t hpk = (size_t)c->n_head / c->n_head_kv;
        float scale = 1.0f / sqrtf((float)hd);
#pragma omp for schedule(dynamic, 4)
        for (size_t t = 0; t < n; t++) {
          if (!scores) continue;
          size_t P = start_pos + t;
          size_t ctx = P + 1 < cap ? P + 1 : cap;
          size_t first = P + 1 - ctx;
          for (int hh = 0; hh < c->n_head; hh++) {
            size_t kvh = hh / hpk;
            const float *qh = q + t * qd + hh * hd;
            for (size_t j = 0; j < ctx; j++) {
              const float *kr = kf + (first + j - lo) * kvd + kvh * hd;
              float dot = 0.0f;
              for (size_t d = 0; d < hd; d++) dot += qh[d] * kr[d];
              scores[j] = dot * scale;
            }
            orc_softmax_scalar(scores, ctx);
            float *oh = ao + t * qd + hh * hd;
            for (size_t d = 0; d < hd; d++) oh[d] = 0.0f;
            for (size_t j = 0; j < ctx; j++) {
              const float *vr = vf + (first + j - lo) * kvd + kvh * hd;
              for (size_t d = 0; d < hd; d++) oh[d] += scores[j] * vr[d];
            }
          }
        }
        free(scores);
      }
      free(kf);
      free(vf);
    }
    for (size_t t = 0; t < n; t++) {
      memcpy(kv->k[l] + ((start_pos + t) % cap) * bpp, nk + t * bpp, bpp);
      memcpy(kv->v[l] + ((start_pos + t) % cap) * bpp, nv + t * bpp, bpp);
    }
    round_f16_inplace(ao, n * qd);
    rc |= gemm_f16io(L->o, ao, D, qd, n, t2, NULL);
    for (size_t i = 0; i < n * D; i++) x[i] += t2[i];
    for (size_t t = 0; t < n; t++) orc_rmsnorm_scalar(x + t * D, L->ffn_norm, c->eps, D, h + t * D);
    round_f16_inplace(h, n * D);
    rc |= gemm_f16io(L->gate, h, F, D, n, g, NULL);
    rc |= gemm_f16io(L->up, h, F, D, n, u, NULL);
    orc_swiglu_scalar(g, u, n * F, g);
    round_f16_inplace(g, n * F);
    rc |= gemm_f16io(L->down, g, D, F, n, t2, NULL);
    for (size_t i = 0; i < n * D; i++) x[i] += t2[i];
  }
  if (rc) goto done;
  for (size_t t = 0; t < n; t++) orc_rmsnorm_scalar(x + t * D, m->output_norm, c->eps, D, h + t * D);
  if (h_final) memcpy(h_final, h, n * D * 4);
  if (x_final) memcpy(x_final, x, n * D * 4);
  if (all_logits)
    rc = gemm_q4_f32x(m->output.scales, m->output.quants, h, c->vocab, D, n, logits, c->vocab);
  else
    rc = gemm_q4_f32x(m->output.scales, m->output.quants, h + (n - 1) * D, c->vocab, D, 1, logits,
                      c->vocab);
done:
  free(x); free(h); free(q); free(k); free(v); free(ao); free(g); free(u); free(t2);
  free(nk); free(nv);
  return rc;
}
