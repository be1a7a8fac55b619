// attention.hip - causal GQA attention over the Q8_0 KV ring on gfx950 MFMA.
//
// Replaces kernels/prefill.cl:120-237 (one work-item per (token, head), three
// passes over the keys, f16 accumulation). Semantics follow the CPU twin
// causal_gqa_decode_scalar_ext (crates/sulimo-cpu/src/scalar.rs:287-359):
// score = (q . deq(K_p)) / sqrt(head_dim), softmax over the window, out = sum
// softmax * deq(V_p) in f32. Query at absolute position P sees keys
// max(0, P-capacity+1) .. P (each once, at ring slot p % capacity), which is the
// reference's range whenever P < capacity.
//
// Flash formulation, one workgroup = 4 wave64s = (BQ query positions) x (HG query
// heads of one KV head):
//  * K/V tiles of 64 keys are dequantized once per workgroup into LDS as f16
//    (K row-major, V transposed), shared by all HG heads of the GQA group.
//  * Each wave owns RF fragments of 16 query rows (one head, 16 positions) and
//    computes S^T = K Q^T with v_mfma_f32_16x16x32_f16 (K as the A operand, Q^T as
//    B, held in registers), so each lane holds 4 consecutive keys of one query:
//    the running max/sum of the online softmax are per-lane scalars.
//  * P^T (f16) feeds O^T = V^T P^T directly as the B operand: lane group g holds
//    keys {4g..4g+3, 16+4g..16+4g+3} of each 32-key step, and the V^T A operand
//    is read from LDS with the same key order.
#include <algorithm>

#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kKT = 64;  // keys per tile

template <int HD, int RF>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a, int BQ, int HG, int n_qblk,
                                                   int n_hgrp) {
  constexpr int KLD = HD + 8;   // Ks pitch (halves)
  constexpr int VLD = kKT + 8;  // Vt pitch (halves)
  constexpr int KS = HD / 32;   // MFMA k-steps over head_dim
  constexpr int DF = HD / 16;   // output fragments over head_dim
  __shared__ __attribute__((aligned(16))) _Float16 Ks[kKT * KLD];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[HD * VLD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;

  // Heaviest query blocks first (causal work grows with the position).
  int bid = blockIdx.x;
  const int hgrp = bid % n_hgrp;
  bid /= n_hgrp;
  const int kvh = bid % a.n_head_kv;
  const int qblk = n_qblk - 1 - bid / a.n_head_kv;
  const int G = a.n_head / a.n_head_kv;
  const int q0 = qblk * BQ;                      // first token of the block
  const int h0 = kvh * G + hgrp * HG;            // first query head
  const int cap = a.capacity;
  const size_t bpp = (size_t)a.n_head_kv * (HD / 32) * 34;
  const size_t hoff = (size_t)kvh * (HD / 32) * 34;
  const int qd = a.n_head * HD;
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);

  // --- load Q fragments (B operand of S^T = K Q^T) ---
  half8 qf[RF][KS];
  int tq[RF], hq[RF];
  long pq[RF];
#pragma unroll
  for (int i = 0; i < RF; i++) {
    const int f = wave + 4 * i;
    const int pb = f / HG, hj = f % HG;
    tq[i] = q0 + 16 * pb + l16;
    hq[i] = h0 + hj;
    pq[i] = (long)a.start_pos + tq[i];
    const bool ok = tq[i] < a.n && 16 * pb < BQ;
    const _Float16 *src = reinterpret_cast<const _Float16 *>(a.q) + (size_t)(ok ? tq[i] : 0) * qd +
                          (size_t)hq[i] * HD + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS; s++)
      qf[i][s] = ok ? *reinterpret_cast<const half8 *>(src + 32 * s) : half8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  floatx4 o[RF][DF];
  float mrun[RF], lrun[RF];
#pragma unroll
  for (int i = 0; i < RF; i++) {
    mrun[i] = -INFINITY;
    lrun[i] = 0.0f;
#pragma unroll
    for (int d = 0; d < DF; d++) o[i][d] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Key window of the whole block.
  const int t_last = min(q0 + BQ, a.n) - 1;
  const long p_min = (long)a.start_pos + q0, p_max = (long)a.start_pos + t_last;
  const long k_lo = max(0L, p_min - cap + 1), k_hi = p_max + 1;  // [k_lo, k_hi)
  const long kt_begin = (k_lo / kKT) * kKT;

  for (long kb = kt_begin; kb < k_hi; kb += kKT) {
    // --- dequantize K and V tiles into LDS: jobs = 64 keys x KS blocks x {K,V} ---
    for (int job = tid; job < kKT * KS * 2; job += 256) {
      const int isv = job / (kKT * KS);
      const int rem = job % (kKT * KS);
      const int key = rem / KS, b = rem % KS;
      const long p = kb + key;
      float d = 0.0f;
      int8_t codes[32];
      if (p >= k_lo && p < k_hi) {
        const uint8_t *base = (p < a.new_pos0) ? (isv ? a.v_ring : a.k_ring) + (size_t)(p % cap) * bpp
                                               : (isv ? a.new_v : a.new_k) + (size_t)(p - a.new_pos0) * bpp;
        const uint16_t *blk = reinterpret_cast<const uint16_t *>(base + hoff + (size_t)b * 34);
        d = (float)__builtin_bit_cast(_Float16, blk[0]);
#pragma unroll
        for (int j = 0; j < 16; j++) {
          uint16_t w = blk[1 + j];
          codes[2 * j] = (int8_t)(w & 0xff);
          codes[2 * j + 1] = (int8_t)(w >> 8);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 32; j++) codes[j] = 0;
      }
      if (!isv) {
        _Float16 *dst = &Ks[key * KLD + 32 * b];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          half8 v;
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = (_Float16)((float)codes[8 * c + e] * d);
          *reinterpret_cast<half8 *>(dst + 8 * c) = v;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 32; e++) Vt[(32 * b + e) * VLD + key] = (_Float16)((float)codes[e] * d);
      }
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < RF; i++) {
      // --- S^T[key][query] for 4 key fragments ---
      floatx4 s[4];
#pragma unroll
      for (int kf = 0; kf < 4; kf++) {
        s[kf] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
          half8 ka = *reinterpret_cast<const half8 *>(&Ks[(16 * kf + l16) * KLD + 32 * ks + 8 * lg]);
          s[kf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[i][ks], s[kf], 0, 0, 0);
        }
      }
      // --- mask + online softmax (lane = one query, 16 keys) ---
      const long P = pq[i];
      const bool qok = tq[i] < a.n;
      float mt = -INFINITY;
#pragma unroll
      for (int kf = 0; kf < 4; kf++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const long p = kb + 16 * kf + 4 * lg + r;
          const bool ok = qok && p <= P && p > P - cap && p >= k_lo;
          const float v = ok ? s[kf][r] * scale_log2 : -INFINITY;
          s[kf][r] = v;
          mt = fmaxf(mt, v);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      // A query that sees no key yet keeps m = -inf; msafe keeps exp2 finite so that
      // every lane runs the same MFMA sequence (no divergence around MFMA).
      const float mnew = fmaxf(mrun[i], mt);
      const float msafe = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = exp2f(mrun[i] - msafe);
      mrun[i] = mnew;
      float lsum = 0.0f;
      half8 pb[2];
#pragma unroll
      for (int kf = 0; kf < 4; kf++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float e = exp2f(s[kf][r] - msafe);
          lsum += e;
          pb[kf >> 1][(kf & 1) * 4 + r] = (_Float16)e;
        }
      lrun[i] = lrun[i] * alpha + lsum;
#pragma unroll
      for (int d = 0; d < DF; d++) o[i][d] *= alpha;
      // --- O^T[d][query] += V^T P^T over two 32-key steps ---
#pragma unroll
      for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int d = 0; d < DF; d++) {
          const _Float16 *vr = &Vt[(16 * d + l16) * VLD + 32 * j + 4 * lg];
          half4 v0 = *reinterpret_cast<const half4 *>(vr);
          half4 v1 = *reinterpret_cast<const half4 *>(vr + 16);
          half8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          o[i][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[j], o[i][d], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // --- normalize and store: lane holds O[query][16d + 4*lg + r] ---
#pragma unroll
  for (int i = 0; i < RF; i++) {
    float l = lrun[i];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int f = wave + 4 * i;
    if (tq[i] >= a.n || 16 * (f / HG) >= BQ) continue;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    _Float16 *dst = reinterpret_cast<_Float16 *>(a.out) + (size_t)tq[i] * qd + (size_t)hq[i] * HD;
#pragma unroll
    for (int d = 0; d < DF; d++) {
      half4 v = {(_Float16)(o[i][d][0] * inv), (_Float16)(o[i][d][1] * inv),
                 (_Float16)(o[i][d][2] * inv), (_Float16)(o[i][d][3] * inv)};
      *reinterpret_cast<half4 *>(dst + 16 * d + 4 * lg) = v;
    }
  }
}

struct AttnShape {
  int bq, hg, rf;
};

// Picks (positions, heads, fragments per wave) with 4 * rf == (bq/16) * hg:
// prefer the most K/V reuse that still gives about two workgroups per CU.
AttnShape pick_shape(int n, int G, int n_head_kv) {
  static const AttnShape cands[] = {{32, 6, 3}, {64, 3, 3}, {48, 4, 3}, {192, 1, 3}, {16, 12, 3},
                                    {32, 4, 2}, {64, 2, 2}, {128, 1, 2}, {16, 8, 2},
                                    {32, 2, 1}, {64, 1, 1}, {16, 4, 1}};
  AttnShape best{0, 0, 0};
  long best_score = -1;
  for (const AttnShape &c : cands) {
    if (G % c.hg != 0) continue;
    long wgs = (long)((n + c.bq - 1) / c.bq) * n_head_kv * (G / c.hg);
    // score: enough workgroups first (up to 512), then reuse (rf * hg).
    long score = std::min(wgs, 512L) * 64 + c.rf * c.hg;
    if (score > best_score) {
      best_score = score;
      best = c;
    }
  }
  return best;
}

template <int HD>
int32_t launch_hd(const AttnArgs &a, hipStream_t s) {
  const int G = a.n_head / a.n_head_kv;
  AttnShape sh = pick_shape(a.n, G, a.n_head_kv);
  if (sh.rf == 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "no attention tiling for this head grouping");
  const int n_qblk = (a.n + sh.bq - 1) / sh.bq;
  const int n_hgrp = G / sh.hg;
  dim3 grid(n_qblk * a.n_head_kv * n_hgrp), block(256);
  switch (sh.rf) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, block, 0, s, a, sh.bq, sh.hg, n_qblk, n_hgrp); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, block, 0, s, a, sh.bq, sh.hg, n_qblk, n_hgrp); break;
    default: hipLaunchKernelGGL((attn_kernel<HD, 3>), grid, block, 0, s, a, sh.bq, sh.hg, n_qblk, n_hgrp); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "attn_kernel launch");
}

}  // namespace

int32_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (a.n <= 0) return SULIMO_HIP_OK;
  if (a.n_head_kv <= 0 || a.n_head % a.n_head_kv != 0)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "head_count must be a multiple of head_count_kv");
  if (a.capacity <= 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "capacity must be positive");
  switch (a.head_dim) {
    case 64: return launch_hd<64>(a, s);
    case 128: return launch_hd<128>(a, s);
    default: return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "attention supports head_dim 64 or 128");
  }
}

}  // namespace sulimo
