// prefill_ops.hip - HBM-bound prefill kernels for gfx950 (wave64 reductions).
//
// Reference formulas: kernels/prefill.cl (rmsnorm_f16_f32w :4-29, rope_f16 :32-68,
// kv_store_q8_0 :72-116, silu_mul_f16 :240-253, add_f16 :256-266) and the host
// embedding gather of crates/sulimo-engine/src/scheduler.rs:329-374.
#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Max over the 32 lanes of a half-wave (one Q8_0 block).
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float load_f(const _Float16 *p, size_t i) { return (float)p[i]; }
__device__ __forceinline__ float load_f(const float *p, size_t i) { return p[i]; }

// Four consecutive elements of x as f32 (16-byte f32 or 8-byte f16 load).
__device__ __forceinline__ float4 load4(const float *p, size_t i) { return *reinterpret_cast<const float4 *>(p + i); }
__device__ __forceinline__ float4 load4(const _Float16 *p, size_t i) {
  typedef _Float16 half4v __attribute__((ext_vector_type(4)));
  const half4v h = *reinterpret_cast<const half4v *>(p + i);
  return float4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

// Row width d = 256 * V: one wave per row, the row held in registers between the sum of
// squares and the scaling (one HBM read of x), 16-byte loads, 8-byte f16 stores.
template <typename T, int V>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const T *__restrict__ x, const float *__restrict__ w,
                                                          _Float16 *__restrict__ out,
                                                          _Float16 *__restrict__ x16_out, float eps, int n) {
  typedef _Float16 half4v __attribute__((ext_vector_type(4)));
  constexpr int D = 256 * V;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const T *xr = x + (size_t)row * D;
  // the weights are loaded with the row: loaded between the stores, each load would
  // wait for the stores before it (loads and stores retire in issue order)
  float4 v[V], wl[V];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < V; j++) {
    v[j] = load4(xr, 256 * j + 4 * lane);
    wl[j] = *reinterpret_cast<const float4 *>(w + 256 * j + 4 * lane);
  }
#pragma unroll
  for (int j = 0; j < V; j++) ss = rms_sumsq4(v[j], ss);
  const float scale = rms_scale(rms_wave_sum(ss), D, eps);
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int i = 256 * j + 4 * lane;
    *reinterpret_cast<rms_half4 *>(out + (size_t)row * D + i) = rms_out4(v[j], scale, wl[j]);
    if (x16_out) {
      const half4v h = {(_Float16)v[j].x, (_Float16)v[j].y, (_Float16)v[j].z, (_Float16)v[j].w};
      *reinterpret_cast<half4v *>(x16_out + (size_t)row * D + i) = h;
    }
  }
}

// Any width: one wave per row: out = f16(x * (1/sqrt(mean(x^2)+eps)) * w).
// With x16_out, also writes f16(x) (final residual hand-back).
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      _Float16 *__restrict__ out,
                                                      _Float16 *__restrict__ x16_out, int d,
                                                      float eps, int n) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const T *xr = x + (size_t)row * d;
  float ss = 0.0f;
  for (int i = lane; i < d; i += 64) {
    float v = load_f(xr, i);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / (float)d + eps);
  _Float16 *o = out + (size_t)row * d;
  for (int i = lane; i < d; i += 64) {
    float v = load_f(xr, i);
    o[i] = (_Float16)(v * scale * w[i]);
    if (x16_out) x16_out[(size_t)row * d + i] = (_Float16)v;
  }
}

// Rotation angle of pair i at position pos: pos / base^(2i/rope_dim).
__device__ __forceinline__ void rope_cs(int pos, int i, int rope_dim, float base, float &c,
                                        float &s) {
  float freq = 1.0f / powf(base, (float)(2 * i) / (float)rope_dim);
  float theta = (float)pos * freq;
  sincosf(theta, &s, &c);
}

// cos/sin of every (position, pair) of a ubatch, [n][rope_dim/2]: the same values
// rope_cs gives, computed once and shared by all heads and layers.
__global__ void rope_table_kernel(float2 *tab, int rope_dim, float base, int start_pos, int n) {
  const int half = rope_dim / 2;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)n * half) return;
  const int t = (int)(gid / half), i = (int)(gid % half);
  float c, sn;
  rope_cs(start_pos + t, i, rope_dim, base, c, sn);
  tab[gid] = float2{c, sn};
}

// One thread per (token, head, pair): in-place f16 rotation.
__global__ void rope_f16_kernel(_Float16 *vec, int head_count, int head_dim, int rope_dim,
                                float base, int mode, int start_pos, int n) {
  const int half = rope_dim / 2;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)n * head_count * half;
  if (gid >= total) return;
  const int i = (int)(gid % half);
  const long th = gid / half;
  const int h = (int)(th % head_count);
  const int t = (int)(th / head_count);
  _Float16 *hp = vec + ((size_t)t * head_count + h) * head_dim;
  float c, s;
  rope_cs(start_pos + t, i, rope_dim, base, c, s);
  const int i0 = mode == 0 ? 2 * i : i;
  const int i1 = mode == 0 ? 2 * i + 1 : i + half;
  const float v0 = (float)hp[i0], v1 = (float)hp[i1];
  hp[i0] = (_Float16)rot_sub(v0, c, v1, s);
  hp[i1] = (_Float16)rot_add(v0, s, v1, c);
}

// Q8_0 quantization of the 32 values held by the 32 lanes of a half-wave
// (quantize_f32_to_q8_0, crates/sulimo-core/src/kv_cache.rs:162-193): d = amax/127,
// f16 scale with RNE, id = 1/d (correctly rounded division), code = round-half-away.
__device__ __forceinline__ void q8_block_store(float v, int e, uint8_t *blk) {
  const float amax = half_wave_max(fabsf(v));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  float q = roundf(v * id);
  q = fminf(fmaxf(q, -128.0f), 127.0f);
  if (e == 0) *reinterpret_cast<_Float16 *>(blk) = (_Float16)d;
  blk[2 + e] = (uint8_t)(int8_t)(int)q;
}

// Half-wave per (token, block).
__global__ __launch_bounds__(256) void kv_store_kernel(const _Float16 *act, uint8_t *kv,
                                                       int start_pos, int capacity,
                                                       int blocks_per_pos, int n) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long bid = gid >> 5;
  const int e = (int)(gid & 31);
  const long nblk = (long)n * blocks_per_pos;
  if (bid >= nblk) return;  // whole half-waves exit together (nblk*32 boundary)
  const int t = (int)(bid / blocks_per_pos), b = (int)(bid % blocks_per_pos);
  const int ring = (start_pos + t) % capacity;
  const float v = (float)act[(size_t)bid * 32 + e];
  q8_block_store(v, e, kv + ((size_t)ring * blocks_per_pos + b) * 34);
}

__global__ void silu_mul_kernel(const _Float16 *g, const _Float16 *u, _Float16 *out,
                                size_t total) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  out[i] = (_Float16)silu_mul((float)g[i], (float)u[i]);
}

__global__ void add_f16_kernel(_Float16 *a, const _Float16 *b, size_t total) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  a[i] = (_Float16)((float)a[i] + (float)b[i]);
}

// The f32 residual update x += f16 value (the residual epilogue's x += f16(acc) on a
// GEMM output already stored in f16).
__global__ void add_f16_to_f32_kernel(float *x, const _Float16 *b, size_t total) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  x[i] += (float)b[i];
}

__global__ void f16_to_f32_kernel(const _Float16 *in, float *out, size_t total) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  out[i] = (float)in[i];
}

// One thread per (token, byte): x = f16(d * (q-8)) for the low and high nibble.
__global__ void embed_q4_kernel(const uint16_t *scales, const uint8_t *quants,
                                const uint32_t *tokens, int n, int embd, _Float16 *x) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int bytes_per_row = embd / 2;
  if (gid >= (long)n * bytes_per_row) return;
  const int t = (int)(gid / bytes_per_row);
  const int byte = (int)(gid % bytes_per_row);
  const int b = byte >> 4, i = byte & 15;
  const size_t row = tokens[t];
  const size_t bpr = embd / 32;
  const float d = (float)__builtin_bit_cast(_Float16, scales[row * bpr + b]);
  const uint8_t q = quants[(row * bpr + b) * 16 + i];
  _Float16 *o = x + (size_t)t * embd + b * 32;
  o[i] = (_Float16)(d * (float)((int)(q & 15) - 8));
  o[16 + i] = (_Float16)(d * (float)((int)(q >> 4) - 8));
}

// One wave per (token, head slot). Slots [0, n_head) are q heads (rotated in
// place, f16), [n_head, n_head+n_head_kv) k heads (rotated in f32, then Q8_0),
// the rest v heads (Q8_0 of the f16 values). head_dim <= 256, multiple of 32.
__global__ __launch_bounds__(256) void rope_qkv_store_kernel(
    _Float16 *q, const _Float16 *k, const _Float16 *v, int n_head, int n_head_kv, int head_dim,
    int rope_dim, const float2 *cs_tab, int mode, int n, uint8_t *k_dst, uint8_t *v_dst,
    int slot0, int wrap, const float *q_norm, const float *k_norm, float eps) {
  __shared__ float sh[4][256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int slots = n_head + 2 * n_head_kv;
  const long job = (long)blockIdx.x * 4 + wave;
  if (job >= (long)n * slots) return;  // whole waves exit; no block barrier below
  const int t = (int)(job / slots), hs = (int)(job % slots);
  float *buf = sh[wave];
  const int half = rope_dim / 2;
  const int kvd = n_head_kv * head_dim;
  const size_t row_bytes = (size_t)n_head_kv * (head_dim / 32) * 34;
  if (hs < n_head + n_head_kv) {
    _Float16 *hp;
    if (hs < n_head)
      hp = q + ((size_t)t * n_head + hs) * head_dim;
    else
      hp = const_cast<_Float16 *>(k) + (size_t)t * kvd + (size_t)(hs - n_head) * head_dim;
    for (int i = lane; i < head_dim; i += 64) buf[i] = (float)hp[i];
    __builtin_amdgcn_wave_barrier();
    // optional QK-norm: RMSNorm of the head with the shared [head_dim] weights
    const float *nw = hs < n_head ? q_norm : k_norm;
    if (nw) {
      float ss = 0.0f;
      for (int i = lane; i < head_dim; i += 64) ss += buf[i] * buf[i];
      ss = wave_sum(ss);
      const float scale = 1.0f / sqrtf(ss / (float)head_dim + eps);
      for (int i = lane; i < head_dim; i += 64) buf[i] = buf[i] * scale * nw[i];
      __builtin_amdgcn_wave_barrier();
    }
    for (int i = lane; i < half; i += 64) {
      const float2 cs = cs_tab[(size_t)t * half + i];
      const float c = cs.x, s = cs.y;
      const int i0 = mode == 0 ? 2 * i : i;
      const int i1 = mode == 0 ? 2 * i + 1 : i + half;
      const float v0 = buf[i0], v1 = buf[i1];
      buf[i0] = rot_sub(v0, c, v1, s);
      buf[i1] = rot_add(v0, s, v1, c);
    }
    __builtin_amdgcn_wave_barrier();
    if (hs < n_head) {
      for (int i = lane; i < head_dim; i += 64) hp[i] = (_Float16)buf[i];
      return;
    }
  } else {
    const _Float16 *hp = v + (size_t)t * kvd + (size_t)(hs - n_head - n_head_kv) * head_dim;
    for (int i = lane; i < head_dim; i += 64) buf[i] = (float)hp[i];
    __builtin_amdgcn_wave_barrier();
  }
  const bool is_k = hs < n_head + n_head_kv;
  const int kvh = is_k ? hs - n_head : hs - n_head - n_head_kv;
  const int row = (int)(((long)slot0 + t) % wrap);
  uint8_t *dst = (is_k ? k_dst : v_dst) + (size_t)row * row_bytes + (size_t)kvh * (head_dim / 32) * 34;
  for (int i = lane; i < head_dim; i += 64) q8_block_store(buf[i], i & 31, dst + (i >> 5) * 34);
}

// Vector form of rope_qkv_store_kernel for rope_dim % 16 == 0: one thread per 8
// consecutive elements ("unit") of one head slot of one token, 16-byte loads and
// stores. A NeoX unit loads its 8 partner elements (rope_dim/2 away) as well; a Norm
// unit holds its pairs. Same arithmetic as rope_qkv_store_kernel; a Q8_0 block is 4
// neighbouring units (max over 4 lanes).
__global__ __launch_bounds__(256) void rope_qkv_store_vec_kernel(
    _Float16 *q, const _Float16 *k, const _Float16 *v, int n_head, int n_head_kv, int head_dim,
    int rope_dim, const float2 *cs_tab, int mode, int n, uint8_t *k_dst, uint8_t *v_dst,
    int slot0, int wrap, const float *q_norm, const float *k_norm, float eps, RopeWindowTarget win) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  // grid: x = token, y = blocks of 256 units (8 elements) of the token's q, k, v heads
  const int upw = head_dim / 8;  // units per head (a power of two)
  const int ush = __builtin_ctz(upw);
  const int slots = n_head + 2 * n_head_kv;
  const int t = blockIdx.x;
  const int w0 = blockIdx.y * blockDim.x + threadIdx.x;
  const bool valid = w0 < slots * upw;
  const int w = valid ? w0 : 0;
  const int u = w & (upw - 1), hs = w >> ush;
  const int half = rope_dim / 2;
  const int kvd = n_head_kv * head_dim;
  const int e0 = 8 * u;  // first element of the unit
  const _Float16 *src;
  if (hs < n_head) src = q + ((size_t)t * n_head + hs) * head_dim;
  else if (hs < n_head + n_head_kv) src = k + (size_t)t * kvd + (size_t)(hs - n_head) * head_dim;
  else src = v + (size_t)t * kvd + (size_t)(hs - n_head - n_head_kv) * head_dim;
  const bool rot = hs < n_head + n_head_kv && e0 < rope_dim;
  const bool lo = e0 < half;
  const half8 xv = *reinterpret_cast<const half8 *>(src + e0);
  half8 pv = xv;
  if (rot && mode != 0) pv = *reinterpret_cast<const half8 *>(src + (lo ? e0 + half : e0 - half));
  // q rotates in place and a NeoX partner unit belongs to another thread of the same
  // workgroup (a head's units never straddle workgroups: 256 % (head_dim/8) == 0 and
  // every workgroup starts at a head of one token)
  __syncthreads();
  if (!valid) return;  // whole heads exit together (slots * head_dim/8 units a token)
  // optional QK-norm: RMSNorm of the head (its head_dim/8 consecutive lanes) with the
  // shared [head_dim] weights, before the rotation; partner values use the same scale
  float xf[8], pf[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    xf[j] = (float)xv[j];
    pf[j] = (float)pv[j];
  }
  const float *nw = hs < n_head ? q_norm : hs < n_head + n_head_kv ? k_norm : nullptr;
  if (nw) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) ss += xf[j] * xf[j];
    for (int sh = upw / 2; sh >= 1; sh >>= 1) ss += __shfl_xor(ss, sh, 64);
    const float scale = 1.0f / sqrtf(ss / (float)head_dim + eps);
    const int pe0 = rot && mode != 0 ? (lo ? e0 + half : e0 - half) : e0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      xf[j] = xf[j] * scale * nw[e0 + j];
      pf[j] = pf[j] * scale * nw[pe0 + j];
    }
  }
  float o[8];
  if (rot) {
    const float2 *cs = cs_tab + (size_t)t * half;
    if (mode == 0) {  // pairs (2i, 2i+1) inside the unit
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float2 r = cs[(e0 + j) / 2];
        const float c = r.x, s = r.y;
        const float v0 = xf[j], v1 = xf[j + 1];
        o[j] = rot_sub(v0, c, v1, s);
        o[j + 1] = rot_add(v0, s, v1, c);
      }
    } else {  // pairs (i, i + half): the partner unit is half away
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float2 r = cs[(lo ? e0 : e0 - half) + j];
        const float c = r.x, s = r.y;
        if (lo) {
          const float v0 = xf[j], v1 = pf[j];
          o[j] = rot_sub(v0, c, v1, s);
        } else {
          const float v0 = pf[j], v1 = xf[j];
          o[j] = rot_add(v0, s, v1, c);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = xf[j];
  }
  if (hs < n_head) {
    half8 r;
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = (_Float16)o[j];
    *reinterpret_cast<half8 *>(q + ((size_t)t * n_head + hs) * head_dim + e0) = r;
    return;
  }
  // Q8_0 of block e0/32, held by the 4 lanes of units 4(u/4) .. +3
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(o[j]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const bool is_k = hs < n_head + n_head_kv;
  const int kvh = is_k ? hs - n_head : hs - n_head - n_head_kv;
  const size_t row_bytes = (size_t)n_head_kv * (head_dim / 32) * 34;
  const int row = (slot0 + t) % wrap;  // slot0 + t fits int (positions are checked by the callers)
  uint8_t *blk = (is_k ? k_dst : v_dst) + (size_t)row * row_bytes + (size_t)kvh * (head_dim / 32) * 34 + (size_t)(u / 4) * 34;
  if ((u & 3) == 0) *reinterpret_cast<_Float16 *>(blk) = (_Float16)d;
  uint16_t *codes = reinterpret_cast<uint16_t *>(blk + 2 + 8 * (u & 3));  // 2-byte aligned
  float qc[8];
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    qc[j] = fminf(fmaxf(roundf(o[j] * id), -128.0f), 127.0f);
    qc[j + 1] = fminf(fmaxf(roundf(o[j + 1] * id), -128.0f), 127.0f);
    codes[j / 2] = (uint16_t)((uint8_t)(int8_t)(int)qc[j] | ((uint16_t)(uint8_t)(int8_t)(int)qc[j + 1] << 8));
  }
  if (win.k) {  // the attention window entries of this position: f16(code * f16(d))
    const float dq = (float)(_Float16)d;
    const int j = win.j0 + t;
    if (is_k) {
      half8 r;
#pragma unroll
      for (int e = 0; e < 8; e++) r[e] = (_Float16)(qc[e] * dq);
      *reinterpret_cast<half8 *>(reinterpret_cast<_Float16 *>(win.k) + ((size_t)kvh * win.pad + j) * head_dim + e0) = r;
    } else {
      _Float16 *vt = reinterpret_cast<_Float16 *>(win.vt) + ((size_t)kvh * head_dim + e0) * win.vst + window_vt_col(j);
#pragma unroll
      for (int e = 0; e < 8; e++) vt[(size_t)e * win.vst] = (_Float16)(qc[e] * dq);
    }
  }
}

__global__ void ring_commit_kernel(const uint16_t *src, uint16_t *ring, size_t row_u16, int slot0,
                                   int capacity, int n) {
  const int t = blockIdx.x;
  if (t >= n) return;
  const size_t slot = ((size_t)slot0 + t) % capacity;
  for (size_t i = threadIdx.x; i < row_u16; i += blockDim.x)
    ring[slot * row_u16 + i] = src[(size_t)t * row_u16 + i];
}

// One workgroup per row; ties resolve to the highest index (Rust Iterator::max_by).
__global__ __launch_bounds__(256) void argmax_kernel(const float *logits, int cols, int32_t *out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const float *r = logits + (size_t)blockIdx.x * cols;
  float bv = -INFINITY;
  int bi = -1;
  for (int i = threadIdx.x; i < cols; i += 256) {
    float v = r[i];
    if (v >= bv) {
      bv = v;
      bi = i;
    }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) {
      float v2 = sv[threadIdx.x + o];
      int i2 = si[threadIdx.x + o];
      if (v2 > sv[threadIdx.x] || (v2 == sv[threadIdx.x] && i2 > si[threadIdx.x])) {
        sv[threadIdx.x] = v2;
        si[threadIdx.x] = i2;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = si[0];
}

inline int32_t check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, what);
}
inline unsigned blocks_for(size_t total, unsigned bs) { return (unsigned)((total + bs - 1) / bs); }

}  // namespace

namespace {
// RMSNorm launch: the register-resident kernel for d = 256 * {1..16} (the hidden sizes
// of the supported models), the generic one otherwise.
template <typename T>
int32_t launch_rmsnorm_t(const T *x, const float *w, _Float16 *out, _Float16 *x16_out, int d, float eps, int n,
                         hipStream_t s) {
  if (n <= 0) return SULIMO_HIP_OK;
  const dim3 grid((n + 3) / 4), block(256);
  switch (d % 256 == 0 ? d / 256 : 0) {
#define SULIMO_RMS_CASE(V) \
  case V: hipLaunchKernelGGL((rmsnorm_vec_kernel<T, V>), grid, block, 0, s, x, w, out, x16_out, eps, n); break;
    SULIMO_RMS_CASE(1) SULIMO_RMS_CASE(2) SULIMO_RMS_CASE(3) SULIMO_RMS_CASE(4) SULIMO_RMS_CASE(5)
    SULIMO_RMS_CASE(6) SULIMO_RMS_CASE(8) SULIMO_RMS_CASE(10) SULIMO_RMS_CASE(12) SULIMO_RMS_CASE(14)
    SULIMO_RMS_CASE(16)
#undef SULIMO_RMS_CASE
    default: hipLaunchKernelGGL(rmsnorm_kernel<T>, grid, block, 0, s, x, w, out, x16_out, d, eps, n); break;
  }
  return check_launch("rmsnorm_kernel");
}
}  // namespace

int32_t launch_rmsnorm_f16(const uint16_t *x, const float *w, uint16_t *out, int d, float eps,
                           int n, hipStream_t s) {
  return launch_rmsnorm_t(reinterpret_cast<const _Float16 *>(x), w, reinterpret_cast<_Float16 *>(out),
                          (_Float16 *)nullptr, d, eps, n, s);
}

int32_t launch_rmsnorm_f32(const float *x, const float *w, uint16_t *out, uint16_t *x16_out, int d,
                           float eps, int n, hipStream_t s) {
  return launch_rmsnorm_t(x, w, reinterpret_cast<_Float16 *>(out), reinterpret_cast<_Float16 *>(x16_out), d, eps,
                          n, s);
}

int32_t launch_rope_f16(uint16_t *vec, int head_count, int head_dim, int rope_dim,
                        float freq_base, int mode, int start_pos, int n, hipStream_t s) {
  const size_t total = (size_t)n * head_count * (rope_dim / 2);
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(rope_f16_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<_Float16 *>(vec), head_count, head_dim, rope_dim, freq_base,
                     mode, start_pos, n);
  return check_launch("rope_f16_kernel");
}

int32_t launch_kv_store_q8_0(const uint16_t *act, uint8_t *kv, int start_pos, int capacity,
                             int blocks_per_pos, int n, hipStream_t s) {
  // With n > capacity, tokens t and t+capacity share a slot and the later one wins
  // (the sequential semantics of the host KvCache); write only the last `capacity`.
  if (n > capacity) {
    const int skip = n - capacity;
    act += (size_t)skip * blocks_per_pos * 32;
    start_pos += skip;
    n = capacity;
  }
  const size_t total = (size_t)n * blocks_per_pos * 32;
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(kv_store_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<const _Float16 *>(act), kv, start_pos, capacity,
                     blocks_per_pos, n);
  return check_launch("kv_store_kernel");
}

int32_t launch_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t total,
                        hipStream_t s) {
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<const _Float16 *>(g), reinterpret_cast<const _Float16 *>(u),
                     reinterpret_cast<_Float16 *>(out), total);
  return check_launch("silu_mul_kernel");
}

int32_t launch_add_f16(uint16_t *a, const uint16_t *b, size_t total, hipStream_t s) {
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(add_f16_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<_Float16 *>(a), reinterpret_cast<const _Float16 *>(b),
                     total);
  return check_launch("add_f16_kernel");
}

int32_t launch_add_f16_to_f32(float *x, const uint16_t *b, size_t total, hipStream_t s) {
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(add_f16_to_f32_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, x,
                     reinterpret_cast<const _Float16 *>(b), total);
  return check_launch("add_f16_to_f32_kernel");
}

int32_t launch_f16_to_f32(const uint16_t *in, float *out, size_t total, hipStream_t s) {
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<const _Float16 *>(in), out, total);
  return check_launch("f16_to_f32_kernel");
}

int32_t launch_embed_q4_0(const uint16_t *scales, const uint8_t *quants, const uint32_t *tokens,
                          int n, int embd, uint16_t *x, hipStream_t s) {
  const size_t total = (size_t)n * (embd / 2);
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(embed_q4_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, scales,
                     quants, tokens, n, embd, reinterpret_cast<_Float16 *>(x));
  return check_launch("embed_q4_kernel");
}

int32_t launch_rope_table(float *tab, int rope_dim, float freq_base, int start_pos, int n, hipStream_t s) {
  const size_t total = (size_t)n * (rope_dim / 2);
  if (total == 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(rope_table_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s,
                     reinterpret_cast<float2 *>(tab), rope_dim, freq_base, start_pos, n);
  return check_launch("rope_table_kernel");
}

int32_t launch_rope_qkv_store(uint16_t *q, const uint16_t *k, const uint16_t *v, int n_head,
                              int n_head_kv, int head_dim, int rope_dim, const float *cs_tab,
                              int mode, int n, uint8_t *k_dst, uint8_t *v_dst,
                              int slot0, int wrap, const float *q_norm, const float *k_norm,
                              float eps, hipStream_t s, const RopeWindowTarget *win, bool *wrote_window) {
  if (wrote_window) *wrote_window = false;
  if (head_dim > 256 || head_dim % 32 != 0)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "head_dim must be a multiple of 32 and <= 256");
  const size_t jobs = (size_t)n * (n_head + 2 * n_head_kv);
  if (jobs == 0) return SULIMO_HIP_OK;
  if (rope_dim % 16 == 0 && 256 % (head_dim / 8) == 0) {
    const int units = (n_head + 2 * n_head_kv) * (head_dim / 8);  // per token
    hipLaunchKernelGGL(rope_qkv_store_vec_kernel, dim3((unsigned)n, (unsigned)((units + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<_Float16 *>(q), reinterpret_cast<const _Float16 *>(k),
                       reinterpret_cast<const _Float16 *>(v), n_head, n_head_kv, head_dim, rope_dim,
                       reinterpret_cast<const float2 *>(cs_tab), mode, n, k_dst, v_dst, slot0, wrap, q_norm,
                       k_norm, eps, win ? *win : RopeWindowTarget{});
    const int32_t rc = check_launch("rope_qkv_store_vec_kernel");
    if (rc == SULIMO_HIP_OK && win && wrote_window) *wrote_window = true;
    return rc;
  }
  hipLaunchKernelGGL(rope_qkv_store_kernel, dim3(blocks_for(jobs, 4)), dim3(256), 0, s,
                     reinterpret_cast<_Float16 *>(q), reinterpret_cast<const _Float16 *>(k),
                     reinterpret_cast<const _Float16 *>(v), n_head, n_head_kv, head_dim, rope_dim,
                     reinterpret_cast<const float2 *>(cs_tab), mode, n, k_dst, v_dst, slot0, wrap, q_norm, k_norm,
                     eps);
  return check_launch("rope_qkv_store_kernel");
}

int32_t launch_ring_commit(const uint8_t *src, uint8_t *ring, size_t row_bytes, int slot0,
                           int capacity, int n, hipStream_t s) {
  if (n <= 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(ring_commit_kernel, dim3(n), dim3(128), 0, s,
                     reinterpret_cast<const uint16_t *>(src), reinterpret_cast<uint16_t *>(ring),
                     row_bytes / 2, slot0, capacity, n);
  return check_launch("ring_commit_kernel");
}

int32_t launch_argmax_rows(const float *logits, int rows, int cols, int32_t *out, hipStream_t s) {
  if (rows <= 0) return SULIMO_HIP_OK;
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, s, logits, cols, out);
  return check_launch("argmax_kernel");
}

}  // namespace sulimo
