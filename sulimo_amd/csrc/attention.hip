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
// Two kernels per call:
//  1. kv_window_kernel dequantizes every key position the ubatch can see, once,
//     from the ring (or the staging of a wrapping ubatch) into f16: K row-major
//     [kv head][position][head_dim], V transposed [kv head][head_dim][position] with
//     the positions of each 16-key group stored in the order the P V^T MFMA reads
//     them (kperm). Values are f16(code * d), as the ring holds them.
//  2. flash_attn_kernel: one workgroup = 8 wave64s. Four of them cover HG query
//     heads of one KV head x PB blocks of 32 positions over the first half of the
//     visible key tiles, the other four the same queries over the second half (two
//     waves per SIMD, half the serial chain); the halves merge (m, l, O) through LDS
//     at the end. K and V^T tiles of 64 keys stream into each half's two LDS slots by
//     buffer DMA and are shared by its four waves. Per wave:
//       S^T = K Q^T   v_mfma_f32_32x32x16_f16, K (LDS) as A, Q^T (registers) as B:
//                     lane l holds 16 keys of query l%32, so the online-softmax
//                     max and sum are per-lane scalars (plus one swap with l^32);
//       P = exp2(S c - m), c = log2(e)/sqrt(head_dim) folded into one fma;
//       O^T += V^T P^T  V^T (LDS) as A, P^T straight from the S^T registers as B.
//     The running max m only moves when a tile's max exceeds it by more than 2^8, so
//     the accumulator is rescaled on few tiles (P <= 256, exact to f16 precision).
//     Tiles that a wave cannot see are skipped; masks are applied only on the
//     tiles that cross the causal diagonal or the window start.
//     Causal work grows with the position, so a query block's key steps may be cut
//     into pieces of at most C steps (C from a cost model of the workgroups, which
//     also favours splitting few long blocks over many CUs): every workgroup runs
//     one piece, heaviest blocks first. A block in one piece writes
//     its f16 output; the pieces of a split block write (O, m, l) partials with
//     device-scope stores and count in on a per-(block, query wave) counter; the wave
//     that completes the count combines the pieces in piece order (the same
//     rescale-and-add as the halves). Device-scope (sc1) stores and loads stay
//     coherent across the XCDs' L2 caches, so no cache writeback fence is needed.
//  3. attn_merge_kernel does that combination instead, as a separate launch, when
//     the caller passes no counters.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kKT = 64;  // keys per tile
constexpr float kLazy = 8.0f;  // log2 growth of the running max before O is rescaled
// V^T rows are wpad + kVPad positions apart: a 4 KB power-of-two row stride would send
// all 128 rows of a tile to the same few L2 channels.
constexpr int kVPad = 64;
constexpr uint32_t kRsrcWord3 = 0x00020000u;

// Stored slot s of a 16-key group holds key kperm(s): slots 0-7 = keys {0-3, 8-11}
// and slots 8-15 = keys {4-7, 12-15}, the keys that lane halves 0 and 1 of the
// S^T accumulator hold (an involution).
__device__ __forceinline__ int kperm(int s) { return (s & 4) ? ((s & 8) ? s : s + 4) : ((s & 8) ? s - 4 : s); }

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)kRsrcWord3);
}
__device__ __forceinline__ void dma16(rsrc_t r, void *dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, (int)voff, soff, 0, 0);
}
// s_waitcnt vmcnt(n) with expcnt and lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_vmcnt0() { wait_vmcnt<0>(); }

// Device-scope (sc1) stores and loads: coherent across the XCDs' L2 caches by
// themselves, for the partials one workgroup hands to another within a launch.
__device__ __forceinline__ void st_dev(half4 *p, half4 v) {
  __hip_atomic_store(reinterpret_cast<uint64_t *>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ half4 ld_dev(const half4 *p) {
  return __builtin_bit_cast(half4, __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<half4 *>(p)),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ float ld_dev(const float *p) {
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(p)),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// f16(v * s) for four values: the f32 product, then its f16 rounding. Kept from fusing
// into one rounding (v_fma_mix), so that every path storing an output row or a piece's
// record rounds the same way.
__device__ __forceinline__ half4 scale_h4(float a, float b, float c, float d, float s) {
  float x = a * s, y = b * s, z = c * s, w = d * s;
  asm("" : "+v"(x), "+v"(y), "+v"(z), "+v"(w));
  return half4{(_Float16)x, (_Float16)y, (_Float16)z, (_Float16)w};
}

// Combination of a split block's pieces in piece order: piece p's normalized f16 output
// counts with weight l_p * 2^(m_p - max m) (m in log2 units, l its row sum); the result
// is the weighted sum over the summed weights.
template <int NV>
struct PieceMerge {
  float ms, l, o[NV];
  __device__ __forceinline__ explicit PieceMerge(float mmax) : ms(mmax == -INFINITY ? 0.0f : mmax), l(0.0f) {
#pragma unroll
    for (int r = 0; r < NV; r++) o[r] = 0.0f;
  }
  __device__ __forceinline__ void add(float mp, float lp, const half4 *v) {
    // no contraction: l += w must not become fma(lp, 2^.., l) at one call site and not
    // at another (the in-kernel merge takes its own piece from registers, the others
    // from memory, and must give the same bits whichever piece finishes last)
#pragma clang fp contract(off)
    const float w = lp * __builtin_amdgcn_exp2f(mp - ms);
    l += w;
#pragma unroll
    for (int r = 0; r < NV; r++) o[r] = __builtin_fmaf((float)v[r >> 2][r & 3], w, o[r]);
  }
  __device__ __forceinline__ float inv() const { return l > 0.0f ? 1.0f / l : 0.0f; }
};

// 4 query waves = HG query heads of one KV group x PB blocks of 32 positions.
__host__ __device__ inline void query_wave_layout(int G, int *HG, int *PB) {
  *HG = (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
  *PB = 4 / *HG;
}

// Key steps of query block qblk (64-key tiles, one per half and step).
__host__ __device__ inline int attn_block_steps(int qblk, int PB, int n, int start_pos, int cap, int wlo,
                                                int halves) {
  const int tg0 = qblk * PB * 32;
  const int tg_last = (tg0 + PB * 32 < n ? tg0 + PB * 32 : n) - 1;
  const int jlo0 = start_pos + tg0 - cap + 1 - wlo;
  const int jlo = jlo0 > 0 ? jlo0 : 0, jhi = start_pos + tg_last - wlo;
  return (jhi / kKT - jlo / kKT + halves) / halves;
}
__host__ __device__ inline int attn_pieces(int steps, int C) { return (steps + C - 1) / C; }

struct Window {
  long lo;    // absolute position of window index 0
  int len;    // visible positions
  int pad;    // len rounded up to the tile
};

Window window_of(const AttnArgs &a) {
  Window w;
  w.lo = a.win_pad > 0 ? 0L : std::max(0L, (long)a.start_pos - a.capacity + 1);
  w.len = (int)((long)a.start_pos + a.n - w.lo);
  w.pad = a.win_pad > 0 ? a.win_pad : (w.len + kKT - 1) / kKT * kKT;
  return w;
}

// ---------------------------------------------------------------------------
// 1. Q8_0 window -> f16 K [kvh][pos][HD] and V^T [kvh][HD][pos]
// ---------------------------------------------------------------------------
// One wave per 16 window positions of one KV head (a 16-key group of the V^T chunk order).
constexpr int kWinKeys = 16;
template <int HD>
__global__ __launch_bounds__(64) void kv_window_kernel(AttnArgs a, long wlo, int wlen, int wpad, int jb0) {
  constexpr int NB = HD / 32;
  __shared__ _Float16 vt[kWinKeys][HD + 2];
  const int kvh = blockIdx.y, j0 = (jb0 + (int)blockIdx.x) * kWinKeys;
  const int cap = a.capacity;
  const size_t bpp = (size_t)a.n_head_kv * NB * 34;
  const size_t hoff = (size_t)kvh * NB * 34;
  _Float16 *kwin = reinterpret_cast<_Float16 *>(a.window);
  _Float16 *vwin = kwin + (size_t)a.n_head_kv * wpad * HD;

  for (int job = threadIdx.x; job < kWinKeys * NB; job += blockDim.x) {
    const int jj = job / NB, b = job % NB;
    const int j = j0 + jj;
    const long p = wlo + j;
    float dk = 0.0f, dv = 0.0f;
    const uint16_t *bk = nullptr, *bv = nullptr;
    if (j < wlen) {
      const bool staged = p >= a.new_pos0;
      const size_t off = staged ? (size_t)(p - a.new_pos0) * bpp : (size_t)(p % cap) * bpp;
      bk = reinterpret_cast<const uint16_t *>((staged ? a.new_k : a.k_ring) + off + hoff + (size_t)b * 34);
      bv = reinterpret_cast<const uint16_t *>((staged ? a.new_v : a.v_ring) + off + hoff + (size_t)b * 34);
      dk = (float)__builtin_bit_cast(_Float16, bk[0]);
      dv = (float)__builtin_bit_cast(_Float16, bv[0]);
    }
    _Float16 *kdst = kwin + ((size_t)kvh * wpad + j) * HD + 32 * b;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      half8 kv8, vv8;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint16_t wk = bk ? bk[1 + 4 * c + e] : 0, wv = bv ? bv[1 + 4 * c + e] : 0;
        kv8[2 * e] = (_Float16)((float)(int8_t)(wk & 0xff) * dk);
        kv8[2 * e + 1] = (_Float16)((float)(int8_t)(wk >> 8) * dk);
        vv8[2 * e] = (_Float16)((float)(int8_t)(wv & 0xff) * dv);
        vv8[2 * e + 1] = (_Float16)((float)(int8_t)(wv >> 8) * dv);
      }
      *reinterpret_cast<half8 *>(kdst + 8 * c) = kv8;
#pragma unroll
      for (int e = 0; e < 8; e++) vt[jj][32 * b + 8 * c + e] = vv8[e];
    }
  }
  __syncthreads();
  // V^T rows: chunk c (8 keys) of row h holds keys 16*(c/2) + kperm(8*(c%2) + e)
  for (int job = threadIdx.x; job < HD * (kWinKeys / 8); job += blockDim.x) {
    const int h = job / (kWinKeys / 8), c = job % (kWinKeys / 8);
    half8 v;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = vt[16 * (c >> 1) + kperm(8 * (c & 1) + e)][h];
    *reinterpret_cast<half8 *>(vwin + ((size_t)kvh * HD + h) * (wpad + kVPad) + j0 + 8 * c) = v;
  }
}

// ---------------------------------------------------------------------------
// 2. flash attention over the f16 window
// ---------------------------------------------------------------------------
// Split-key partial of one piece, per (query wave x lane) = 256 entries: the normalized
// O^T registers O/l as f16, in 4*OT groups of 256 x 4 f16 (group 4i + g holds registers
// 4g .. 4g+3 of O^T tile i, one 8-byte chunk per entry), then m and the query's l as f32.
template <int HD>
constexpr int part_rec_floats() { return 16 * (HD / 32) * 128 + 2 * 256; }

template <int HD, int H2>
__global__ __launch_bounds__(256 * H2, 2 / H2) void flash_attn_kernel(AttnArgs a, long wlo, int wpad, int HG,
                                                                      int PB, int n_qblk, int n_hgrp, int C,
                                                                      float *part, int pmax, int *ctr) {
  constexpr int KS = HD / 16;          // S^T k-steps over head_dim
  constexpr int OT = HD / 32;          // O^T tiles over head_dim
  constexpr int KCH = HD / 8;          // 16-byte chunks per K row
  constexpr int KROW = HD * 2;         // bytes per K row
  constexpr int K_BYTES = kKT * KROW;
  constexpr int V_BYTES = HD * kKT * 2;
  constexpr int RPI = 64 / KCH;        // K rows per DMA instruction
  constexpr int NKI = kKT / RPI / 4;   // K DMA instructions per wave per tile
  constexpr int NVI = HD / 8 / 4;      // V^T DMA instructions per wave per tile (8 rows each)
  // H2 halves of 4 waves (the key range split in two inside the workgroup, or not),
  // each with a two-slot ring; every slot is its own variable
  constexpr int K2 = H2 == 2 ? K_BYTES : 16, V2 = H2 == 2 ? V_BYTES : 16;
  __shared__ __attribute__((aligned(16))) char ka0[K_BYTES], va0[V_BYTES], ka1[K_BYTES], va1[V_BYTES];
  __shared__ __attribute__((aligned(16))) char kb0[K2], vb0[V2], kb1[K2], vb1[V2];
  // one O^T tile of the second half, register group g of lane ci at float4 g * 256 + ci
  // (consecutive lanes, consecutive 16 bytes: no bank conflicts), and its running max and sum
  __shared__ __attribute__((aligned(16))) float4 comb[H2 == 2 ? 4 * 256 : 1];
  __shared__ __attribute__((aligned(8))) float2 cml[H2 == 2 ? 256 : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = H2 == 2 ? wave >> 2 : 0, qw = wave & 3;
  const int l32 = lane & 31, lg = lane >> 5;

  // workgroup -> (head group, query block, piece): heaviest blocks first, the pieces of
  // a block consecutive, the head groups innermost
  const int n_groups = a.n_head_kv * n_hgrp;
  const int grp = blockIdx.x % n_groups;
  const int hgrp = grp % n_hgrp, kvh = grp / n_hgrp;
  int wi = blockIdx.x / n_groups;
  int qblk = n_qblk - 1, npiece;
  for (;;) {
    npiece = attn_pieces(attn_block_steps(qblk, PB, a.n, a.start_pos, a.capacity, (int)wlo, H2), C);
    if (wi < npiece || qblk == 0) break;
    wi -= npiece;
    qblk--;
  }
  const int piece = wi;
  const int G = a.n_head / a.n_head_kv;
  const int hj = qw % HG, pb = qw / HG;
  const int h = kvh * G + hgrp * HG + hj;
  const int tw0 = (qblk * PB + pb) * 32;    // first token of this wave
  const int t = tw0 + l32;                  // this lane's query token
  const int qd = a.n_head * HD;
  const int cap = a.capacity;
  const float c = 1.4426950408889634f / sqrtf((float)HD);

  // Q^T fragments (B operand): lane holds Q[t][h][16s + 8lg .. +7]
  half8 qf[KS];
  {
    const bool ok = t < a.n;
    const _Float16 *src = reinterpret_cast<const _Float16 *>(a.q) + (size_t)(ok ? t : 0) * qd + (size_t)h * HD + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS; s++) {  // rows past n read row 0 and are zeroed (no branch)
      const half8 v = *reinterpret_cast<const half8 *>(src + 16 * s);
      qf[s] = ok ? v : half8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  // Absolute positions: this wave's queries, and the whole workgroup's.
  const int P = a.start_pos + t;  // positions fit in int (checked by the callers)
  const int tw_last = min(tw0 + 31, a.n - 1);
  const bool wave_live = tw0 < a.n;
  const int Pw_min = a.start_pos + tw0, Pw_max = a.start_pos + tw_last;
  const int tg0 = qblk * PB * 32, tg_last = min(tg0 + PB * 32, a.n) - 1;
  const int Pg_min = a.start_pos + tg0, Pg_max = a.start_pos + tg_last;
  // window indices j = p - wlo of the keys any query of the workgroup sees
  const int jlo = max(0, Pg_min - cap + 1 - (int)wlo), jhi = Pg_max - (int)wlo;  // inclusive
  const int tile0 = jlo / kKT, tile1 = jhi / kKT;                                 // inclusive
  // the first half takes the first ceil(n/2) tiles, the second half the rest; this
  // piece runs steps [sa, sb) of both
  const int nsteps = (tile1 - tile0 + H2) / H2;
  const int sa = piece * nsteps / npiece, sb = (piece + 1) * nsteps / npiece;
  const int tb = (half ? tile0 + nsteps : tile0) + sa;
  const int te = min(half ? tile1 : tile0 + nsteps - 1, tb + (sb - sa) - 1);  // te < tb: nothing for this half
  const int psteps = sb - sa;

  // DMA sources (bytes): K rows and V^T rows of this kv head; the tile start goes in soffset.
  const _Float16 *kwin = reinterpret_cast<const _Float16 *>(a.window);
  const _Float16 *vwin = kwin + (size_t)a.n_head_kv * wpad * HD;
  const rsrc_t rk = make_rsrc(kwin + (size_t)kvh * wpad * HD, (uint32_t)wpad * HD * 2);
  const int vst = wpad + kVPad;  // V^T row stride (positions)
  const rsrc_t rv = make_rsrc(vwin + (size_t)kvh * HD * vst, (uint32_t)HD * vst * 2);
  uint32_t koff[NKI], voff[NVI];
#pragma unroll
  for (int i = 0; i < NKI; i++) {
    const int row = RPI * (NKI * qw + i) + lane / KCH;
    const int ch = (lane % KCH) ^ (row % KCH);
    koff[i] = (uint32_t)(row * HD + 8 * ch) * 2u;
  }
#pragma unroll
  for (int i = 0; i < NVI; i++) {
    const int hr = 8 * (NVI * qw + i) + lane / 8;
    const int ch = (lane % 8) ^ ((hr >> 1) & 7);
    voff[i] = (uint32_t)(hr * vst + 8 * ch) * 2u;
  }
  // always issued (an idle half reloads a valid tile), so every wave waits the same way
  auto issue = [&](char *sk, char *sv, int tile) __attribute__((always_inline)) {
    const int kb = min(tile, tile1) * kKT;
#pragma unroll
    for (int i = 0; i < NKI; i++) dma16(rk, sk + RPI * (NKI * qw + i) * KROW, koff[i], kb * HD * 2);
#pragma unroll
    for (int i = 0; i < NVI; i++) dma16(rv, sv + 8 * (NVI * qw + i) * kKT * 2, voff[i], kb * 2);
  };

  floatx16 o[OT];
#pragma unroll
  for (int i = 0; i < OT; i++) o[i] = floatx16{};
  float mrun = -INFINITY, lrun = 0.0f;

  // --- one tile of 64 keys, as two 32-key online-softmax steps, software-pipelined so
  // that the MFMAs of one step run under the VALU softmax of the other:
  //   S0 | S1 + softmax0 | PV0 + softmax1 | PV1
  auto s_step = [&](const char *sk, int kt, floatx16 &st) __attribute__((always_inline)) {
    st = floatx16{};
    const int row = 32 * kt + l32;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const int pos = (2 * s + lg) ^ (row % KCH);
      const half8 kf = *reinterpret_cast<const half8 *>(sk + row * KROW + 16 * pos);
      st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], st, 0, 0, 0);
    }
  };
  auto pv_step = [&](const char *sv, int kt, const half8 (&pbk)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int jh = 0; jh < 2; jh++) {
      const int j = 2 * kt + jh;  // 16-key step of the tile
#pragma unroll
      for (int i = 0; i < OT; i++) {
        const int hr = 32 * i + l32;
        const int pos = (2 * j + lg) ^ ((hr >> 1) & 7);
        const half8 vf = *reinterpret_cast<const half8 *>(sv + hr * (kKT * 2) + 16 * pos);
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pbk[jh], o[i], 0, 0, 0);
      }
    }
  };
  // mask (diagonal / window-start tiles only), running max, exp2, sum, P^T as f16
  auto softmax = [&](floatx16 &st, int p_reg0, bool masked, half8 (&pbk)[2]) __attribute__((always_inline)) -> float {
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int p = p_reg0 + 8 * (r >> 2) + (r & 3);
        st[r] = (p > P || p <= P - cap) ? -INFINITY : st[r];
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) mt = fmaxf(mt, st[r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // The running max only moves when the tile's max exceeds it by more than 2^8 (log2
    // units): P = exp2(s c - m) then stays <= 256, exact to f16 precision, and O and l
    // are rescaled on few tiles. Softmax is shift-invariant, so the result is the same.
    // A query that sees no key yet keeps m = -inf (and O = l = 0).
    const float mcand = mt * c;
    const bool grow = mcand > mrun + kLazy;
    const float alpha = (grow && mrun != -INFINITY) ? __builtin_amdgcn_exp2f(mrun - mcand) : 1.0f;
    if (grow) mrun = mcand;
    // msafe keeps exp2 finite so that every lane runs the same MFMA sequence
    const float msafe = mrun == -INFINITY ? 0.0f : mrun;
#pragma unroll
    for (int r = 0; r < 16; r++) pbk[r >> 3][r & 7] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(st[r], c, -msafe));
    // l sums the f16 P the MFMA consumes, two per dot2 with f32 accumulation
    const half2v one2 = {(_Float16)1.0f, (_Float16)1.0f};
    float lsum = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        lsum = __builtin_amdgcn_fdot2(half2v{pbk[j][e], pbk[j][e + 1]}, one2, lsum, false);
    lrun = lrun * alpha + lsum;
    return alpha;
  };
  auto rescale = [&](float alpha) __attribute__((always_inline)) {
    if (__ballot(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < OT; i++) o[i] *= alpha;
    }
  };
  // MFMA / VALU / LDS-read interleave of one pipelined phase (8 MFMAs)
  auto interleave = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // 6 VALU
    }
  };
  auto compute = [&](const char *sk, const char *sv, int tile, auto kMasked) __attribute__((always_inline)) {
    constexpr bool M = decltype(kMasked)::value;
    const int p0 = (int)wlo + tile * kKT;  // absolute position of the tile's first key
    floatx16 st0, st1;
    half8 pa[2], pbv[2];
    s_step(sk, 0, st0);
    __builtin_amdgcn_sched_barrier(0);
    s_step(sk, 1, st1);
    const float al0 = softmax(st0, p0 + 4 * lg, M, pa);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    rescale(al0);
    __builtin_amdgcn_sched_barrier(0);
    pv_step(sv, 0, pa);
    const float al1 = softmax(st1, p0 + 32 + 4 * lg, M, pbv);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    rescale(al1);
    __builtin_amdgcn_sched_barrier(0);
    pv_step(sv, 1, pbv);
  };
  auto tile_work = [&](const char *sk, const char *sv, int tile) __attribute__((always_inline)) {
    const int p0 = (int)wlo + tile * kKT;
    if (tile > te || !wave_live || p0 > Pw_max || p0 + kKT - 1 <= Pw_min - cap) return;  // nothing visible
    if (p0 + kKT - 1 <= Pw_min && p0 > Pw_max - cap) compute(sk, sv, tile, std::false_type{});
    else compute(sk, sv, tile, std::true_type{});
  };

  // Per step: wait for this half's tile, barrier (it landed for all waves, and every
  // wave finished the previous step), prefetch the next tile into the other slot,
  // compute. Both halves run the same number of steps and barriers.
  auto run = [&](char *k0, char *v0, char *k1, char *v1) __attribute__((always_inline)) {
    issue(k0, v0, tb);
    int s = 0;
    for (; s + 1 < psteps; s += 2) {
      wait_vmcnt0();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(k1, v1, tb + s + 1);
      tile_work(k0, v0, tb + s);
      wait_vmcnt0();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(k0, v0, tb + s + 2);
      tile_work(k1, v1, tb + s + 1);
    }
    if (s < psteps) {
      wait_vmcnt0();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      tile_work(k0, v0, tb + s);
    }
  };
  if constexpr (H2 == 1) run(ka0, va0, ka1, va1);
  else if (half == 0) run(ka0, va0, ka1, va1);
  else run(kb0, vb0, kb1, vb1);
  wait_vmcnt0();  // no DMA may still be writing this workgroup's LDS
  __syncthreads();

  // --- the second half hands its (m, l, O^T) to the first, one O^T tile at a time ---
  const int ci = (qw * 64 + lane);
  if constexpr (H2 == 2) {
  if (half) cml[ci] = float2{mrun, lrun};
  float a0 = 1.0f, a1 = 0.0f;
#pragma unroll
  for (int i = 0; i < OT; i++) {
    if (half) {
#pragma unroll
      for (int g = 0; g < 4; g++) comb[g * 256 + ci] = float4{o[i][4 * g], o[i][4 * g + 1], o[i][4 * g + 2], o[i][4 * g + 3]};
    }
    __syncthreads();
    if (!half) {
      if (i == 0) {
        const float2 ml = cml[ci];
        const float m1 = ml.x, l1 = ml.y;
        const float mm = fmaxf(mrun, m1);
        const float ms = mm == -INFINITY ? 0.0f : mm;
        a0 = __builtin_amdgcn_exp2f(mrun - ms);
        a1 = __builtin_amdgcn_exp2f(m1 - ms);
        lrun = lrun * a0 + l1 * a1;
        mrun = mm;  // O and l are now relative to the joint max (a split block's partial keeps it)
      }
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 v = comb[g * 256 + ci];
        o[i][4 * g] = o[i][4 * g] * a0 + v.x * a1;
        o[i][4 * g + 1] = o[i][4 * g + 1] * a0 + v.y * a1;
        o[i][4 * g + 2] = o[i][4 * g + 2] * a0 + v.z * a1;
        o[i][4 * g + 3] = o[i][4 * g + 3] * a0 + v.w * a1;
      }
    }
    __syncthreads();
  }
  if (half) return;
  }

  if (npiece > 1) {  // a piece of a split block: its partial (O^T, m, l) for the merge
    constexpr int RF = part_rec_floats<HD>();
    constexpr int MOFF = 16 * OT * 128;  // m, then l, after the O^T groups
    float *rec0 = part + ((size_t)grp * n_qblk + qblk) * pmax * (size_t)RF;
    float *rec = rec0 + (size_t)piece * RF;
    const float lt = lrun + __shfl_xor(lrun, 32, 64);  // the query's l (lane halves hold parts)
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    half4 mine[4 * OT];
#pragma unroll
    for (int i = 0; i < OT; i++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        mine[4 * i + g] = scale_h4(o[i][4 * g], o[i][4 * g + 1], o[i][4 * g + 2], o[i][4 * g + 3], inv);
    half4 *ro = reinterpret_cast<half4 *>(rec) + ci;
#pragma unroll
    for (int k = 0; k < 4 * OT; k++) {
      // one materialization: the merge below uses exactly the stored f16 values
      uint64_t u = __builtin_bit_cast(uint64_t, mine[k]);
      asm volatile("" : "+v"(u));
      mine[k] = __builtin_bit_cast(half4, u);
      st_dev(ro + k * 256, mine[k]);
    }
    st_dev(rec + MOFF + ci, mrun);
    st_dev(rec + MOFF + 256 + ci, lt);
    if (!ctr || !wave_live) return;  // a wave past the last token is past it in every piece
    // Count in once this wave's record is complete (device-scope stores, acknowledged);
    // the wave that completes the count merges the pieces for its 32 queries and
    // leaves the counter at zero for the next launch.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int *cw = ctr + (((size_t)grp * n_qblk + qblk) << 2) + qw;
    int prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(cw, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != npiece - 1) return;
    if (lane == 0) __hip_atomic_store(cw, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // piece p's (O, m, l): this piece's from registers, the others' loaded (issued
    // one piece ahead of their use, so two pieces' loads are in flight at a time)
    auto fetch = [&](int p, half4 (&v)[4 * OT], float &mp, float &lp) __attribute__((always_inline)) {
      if (p == piece) {
#pragma unroll
        for (int k = 0; k < 4 * OT; k++) v[k] = mine[k];
        mp = mrun;
        lp = lt;
        return;
      }
      const float *r = rec0 + (size_t)p * RF;
      const half4 *rv = reinterpret_cast<const half4 *>(r) + ci;
#pragma unroll
      for (int k = 0; k < 4 * OT; k++) v[k] = ld_dev(rv + k * 256);
      mp = ld_dev(r + MOFF + ci);
      lp = ld_dev(r + MOFF + 256 + ci);
    };
    half4 va[4 * OT], vb[4 * OT];
    float ma, la, mb = 0.0f, lb = 0.0f;
    fetch(0, va, ma, la);
    if (npiece > 1) fetch(1, vb, mb, lb);
    float mmax = -INFINITY;
    for (int p0 = 0; p0 < npiece; p0 += 8) {  // loads of 8 pieces issued before any is used
      float mp[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int p = p0 + j;
        mp[j] = p >= npiece ? -INFINITY : p == piece ? mrun : ld_dev(rec0 + (size_t)p * RF + MOFF + ci);
      }
#pragma unroll
      for (int j = 0; j < 8; j++) mmax = fmaxf(mmax, mp[j]);
    }
    PieceMerge<16 * OT> mg(mmax);
    int p = 0;
    for (; p + 1 < npiece; p += 2) {
      mg.add(ma, la, va);
      if (p + 2 < npiece) fetch(p + 2, va, ma, la);
      mg.add(mb, lb, vb);
      if (p + 3 < npiece) fetch(p + 3, vb, mb, lb);
    }
    if (p < npiece) mg.add(ma, la, va);
    if (t >= a.n) return;
    const float minv = mg.inv();
    _Float16 *dst = reinterpret_cast<_Float16 *>(a.out) + (size_t)t * qd + (size_t)h * HD;
#pragma unroll
    for (int i = 0; i < OT; i++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float *w = mg.o + 16 * i + 4 * g;
        *reinterpret_cast<half4 *>(dst + 32 * i + 8 * g + 4 * lg) = scale_h4(w[0], w[1], w[2], w[3], minv);
      }
    return;
  }

  // --- normalize and store: lane holds O[t][32i + 8(r/4) + 4lg + r%4] ---
  float l = lrun + __shfl_xor(lrun, 32, 64);
  if (t >= a.n) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  _Float16 *dst = reinterpret_cast<_Float16 *>(a.out) + (size_t)t * qd + (size_t)h * HD;
#pragma unroll
  for (int i = 0; i < OT; i++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      *reinterpret_cast<half4 *>(dst + 32 * i + 8 * g + 4 * lg) =
          scale_h4(o[i][4 * g], o[i][4 * g + 1], o[i][4 * g + 2], o[i][4 * g + 3], inv);
    }
}

// ---------------------------------------------------------------------------
// 3. merge the pieces of split query blocks
// ---------------------------------------------------------------------------
// One workgroup = 4 waves per (head group, query block); wave qw and lane hold the
// same queries and O^T registers as in flash_attn_kernel.
template <int HD>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a, long wlo, int HG, int PB, int n_qblk,
                                                         int n_hgrp, int C, const float *part, int pmax,
                                                         int halves) {
  constexpr int OT = HD / 32;
  constexpr int RF = part_rec_floats<HD>();
  constexpr int PMAX = 16;  // pieces combined per pass
  const int qblk = blockIdx.x, grp = blockIdx.y, i = blockIdx.z;  // i: the O^T tile (32 head-dim rows)
  const int npiece = attn_pieces(attn_block_steps(qblk, PB, a.n, a.start_pos, a.capacity, (int)wlo, halves), C);
  if (npiece < 2) return;  // written by flash_attn_kernel
  const int lane = threadIdx.x & 63, qw = threadIdx.x >> 6, ci = threadIdx.x;
  const int hgrp = grp % n_hgrp, kvh = grp / n_hgrp;
  const int G = a.n_head / a.n_head_kv;
  const int hj = qw % HG, pb = qw / HG;
  const int h = kvh * G + hgrp * HG + hj;
  const int t = (qblk * PB + pb) * 32 + (lane & 31);
  const int lg = lane >> 5;
  constexpr int MOFF = 16 * OT * 128;
  const float *rec0 = part + ((size_t)grp * n_qblk + qblk) * pmax * (size_t)RF;
  // the block's max first (the loads of PMAX pieces issued before any is used)
  float mmax = -INFINITY;
  for (int p0 = 0; p0 < npiece; p0 += PMAX) {
    float mp[PMAX];
#pragma unroll
    for (int p = 0; p < PMAX; p++) mp[p] = p0 + p < npiece ? rec0[(size_t)(p0 + p) * RF + MOFF + ci] : -INFINITY;
#pragma unroll
    for (int p = 0; p < PMAX; p++) mmax = fmaxf(mmax, mp[p]);
  }
  PieceMerge<16> mg(mmax);
  for (int p = 0; p < npiece; p++) {
    const float *rec = rec0 + (size_t)p * RF;
    const half4 *ro = reinterpret_cast<const half4 *>(rec) + ci;
    half4 v[4];
#pragma unroll
    for (int g = 0; g < 4; g++) v[g] = ro[(4 * i + g) * 256];
    mg.add(rec[MOFF + ci], rec[MOFF + 256 + ci], v);
  }
  if (t >= a.n) return;
  const float inv = mg.inv();
  _Float16 *dst = reinterpret_cast<_Float16 *>(a.out) + (size_t)t * a.n_head * HD + (size_t)h * HD;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const float *w = mg.o + 4 * g;
    *reinterpret_cast<half4 *>(dst + 32 * i + 8 * g + 4 * lg) = scale_h4(w[0], w[1], w[2], w[3], inv);
  }
}

// Work split of one attention call.
struct AttnPlan {
  int HG, PB, n_qblk, n_hgrp, C, pmax, pieces;  // pieces = workgroups per head group
  int halves;                                   // key halves inside a workgroup (1 or 2)
};

// Predicted time (us) of one layout, fitted to the measured time of every layout and
// piece size on MI355X over 17 shapes (Qwen2.5-1.5B, Llama-3.2-3B and a head_dim-64
// model; prompts of 7 to 4096 tokens at several start positions; its picks checked
// against a second sweep that timed each plan on a warm clock, in shuffled order): the
// workgroups run in rounds of one per slot (two per CU with one key half, one with two),
// each round as long as a piece of C steps, fixed + per-step cost; a split block adds
// ~1 us per piece of the longest split (its last wave merges the pieces).
AttnPlan plan_layout(const AttnArgs &a, const Window &w, int halves, int force_c, double *t_out) {
  AttnPlan p;
  p.halves = halves;
  const int G = a.n_head / a.n_head_kv;
  query_wave_layout(G, &p.HG, &p.PB);
  p.n_qblk = (a.n + 32 * p.PB - 1) / (32 * p.PB);
  p.n_hgrp = G / p.HG;
  const int n_groups = a.n_head_kv * p.n_hgrp;
  int maxs = 1;
  for (int b = 0; b < p.n_qblk; b++)
    maxs = std::max(maxs, attn_block_steps(b, p.PB, a.n, a.start_pos, a.capacity, (int)w.lo, halves));
  const double slots = (double)device_cu_count() * (halves == 2 ? 1 : 2);
  const bool hd64 = a.head_dim <= 64;
  const double f = (halves == 2 ? 11.515 : 7.482) * (hd64 ? 1.181 : 1.0);
  const double g = (halves == 2 ? 1.101 : 1.55) * (hd64 ? 0.473 : 1.0);
  auto cost = [&](int C, int *pieces, int *pmax) {
    int np = 0, pm = 1;
    for (int b = 0; b < p.n_qblk; b++) {
      const int k = attn_pieces(attn_block_steps(b, p.PB, a.n, a.start_pos, a.capacity, (int)w.lo, halves), C);
      np += k;
      pm = std::max(pm, k);
    }
    *pieces = np;
    *pmax = pm;
    const double rounds = std::ceil((double)np * n_groups / slots);
    double t = rounds * (f + g * std::min(C, maxs));
    if (pm > 1) t += 1.017 * pm;
    return t;
  };
  if (force_c > 0) {
    p.C = std::min(force_c, maxs);
    *t_out = cost(p.C, &p.pieces, &p.pmax);
    return p;
  }
  p.C = maxs;
  double best = cost(maxs, &p.pieces, &p.pmax);
  for (int C = 2; C < maxs; C++) {
    int np, pm;
    const double t = cost(C, &np, &pm);
    if (t < best) {
      best = t;
      p.C = C;
      p.pieces = np;
      p.pmax = pm;
    }
  }
  *t_out = best;
  return p;
}

// The cheaper of the two layouts (halves = 0), or the given one.
AttnPlan plan_attention_uncached(const AttnArgs &a, const Window &w, int halves, int force_c) {
  double t2, t1;
  if (halves) return plan_layout(a, w, halves, force_c, &t2);
  const AttnPlan p1 = plan_layout(a, w, 1, 0, &t1);
  // Unsplit blocks of one key half that already fill every slot (two per CU) run best
  // as they are: splits only add workgroups (Llama-3.2-3B, 4096 tokens: 139.6 us
  // unsplit against 155-160 us for the best splits and for two key halves).
  if (p1.n_qblk * a.n_head_kv * p1.n_hgrp >= 2 * device_cu_count()) return plan_layout(a, w, 1, 1 << 30, &t1);
  const AttnPlan p2 = plan_layout(a, w, 2, 0, &t2);
  return t1 < t2 ? p1 : p2;
}

// The plan depends only on the shape, the window (a function of the shape) and the CU
// count; recent plans are kept per host thread (scoring every piece size over every
// query block costs ~10 us, and every layer of a ubatch asks for the same plan).
AttnPlan plan_attention(const AttnArgs &a, const Window &w, int halves = 0, int force_c = 0) {
  struct Entry {
    int key[9];
    AttnPlan plan;
  };
  constexpr int kEntries = 8;
  thread_local Entry cache[kEntries];
  thread_local int used = 0, next = 0;
  const int key[9] = {a.start_pos, a.n, a.capacity, a.n_head, a.n_head_kv, a.head_dim, halves, force_c,
                      device_cu_count()};
  for (int i = 0; i < used; i++)
    if (std::equal(key, key + 9, cache[i].key)) return cache[i].plan;
  const AttnPlan p = plan_attention_uncached(a, w, halves, force_c);
  std::copy(key, key + 9, cache[next].key);
  cache[next].plan = p;
  next = (next + 1) % kEntries;
  used = std::min(used + 1, kEntries);
  return p;
}

size_t window_bytes(const AttnArgs &a, const Window &w) {
  return ((size_t)a.n_head_kv * a.head_dim * (2 * (size_t)w.pad + kVPad) * 2 + 255) & ~(size_t)255;
}

size_t partial_bytes(const AttnArgs &a, const AttnPlan &p) {
  if (p.pmax < 2) return 0;
  const size_t rf = 16 * (size_t)(a.head_dim / 32) * 128 + 2 * 256;
  return (size_t)a.n_head_kv * p.n_hgrp * p.n_qblk * p.pmax * rf * 4;
}

template <int HD>
int32_t launch_hd(const AttnArgs &a, hipStream_t s) {
  const Window w = window_of(a);
  // window blocks of 16 positions: all of them, or (when the ubatch's own positions are
  // already there) those holding earlier positions or padding; a block that also holds
  // new positions rewrites them with the same values
  auto window_blocks = [&](int b0, int b1) -> int32_t {
    if (b1 <= b0) return SULIMO_HIP_OK;
    hipLaunchKernelGGL((kv_window_kernel<HD>), dim3(b1 - b0, a.n_head_kv), dim3(64), 0, s, a, w.lo, w.len, w.pad, b0);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "kv_window_kernel launch");
  };
  const int nblk = w.pad / kWinKeys;
  int32_t rc;
  if (a.win_pad > 0) {
    // kept window: the earlier positions not yet valid (and, unless the caller wrote
    // them, the ubatch's own), nothing past the last position
    const int jn0 = a.start_pos;
    const int end = a.win_new_done ? (jn0 + kWinKeys - 1) / kWinKeys : (w.len + kWinKeys - 1) / kWinKeys;
    if ((rc = window_blocks(std::min(a.win_valid, jn0) / kWinKeys, end))) return rc;
  } else if (a.win_new_done) {
    const int jn0 = (int)(a.start_pos - w.lo);  // window index of the first new position
    const int pre = (jn0 + kWinKeys - 1) / kWinKeys, tail = w.len / kWinKeys;
    if ((rc = window_blocks(0, pre)) || (rc = window_blocks(std::max(pre, tail), nblk))) return rc;
  } else if ((rc = window_blocks(0, nblk))) {
    return rc;
  }
  hipError_t e;
  const AttnPlan p = plan_attention(a, w);
  float *part = a.part ? a.part : reinterpret_cast<float *>(reinterpret_cast<char *>(a.window) + window_bytes(a, w));
  const int n_groups = a.n_head_kv * p.n_hgrp;
  // the pieces of split blocks merge themselves when the caller passes counters
  int *ctr = p.pmax >= 2 ? a.ctr : nullptr;
  if (ctr && a.ctr_ints < (size_t)n_groups * p.n_qblk * 4)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "attention counters too small for the call");
  if (p.halves == 2)
    hipLaunchKernelGGL((flash_attn_kernel<HD, 2>), dim3(p.pieces * n_groups), dim3(512), 0, s, a, w.lo, w.pad, p.HG,
                       p.PB, p.n_qblk, p.n_hgrp, p.C, part, p.pmax, ctr);
  else
    hipLaunchKernelGGL((flash_attn_kernel<HD, 1>), dim3(p.pieces * n_groups), dim3(256), 0, s, a, w.lo, w.pad, p.HG,
                       p.PB, p.n_qblk, p.n_hgrp, p.C, part, p.pmax, ctr);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "flash_attn_kernel launch");
  if (p.pmax < 2 || ctr) return SULIMO_HIP_OK;
  hipLaunchKernelGGL((attn_merge_kernel<HD>), dim3(p.n_qblk, n_groups, HD / 32), dim3(256), 0, s, a, w.lo, p.HG, p.PB,
                     p.n_qblk, p.n_hgrp, p.C, part, p.pmax, p.halves);
  e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "attn_merge_kernel launch");
}

}  // namespace

AttnWindowLayout attention_window_layout(const AttnArgs &a) {
  const Window w = window_of(a);
  return AttnWindowLayout{w.lo, w.len, w.pad, w.pad + kVPad};
}

size_t attention_window_bytes(const AttnArgs &a) { return window_bytes(a, window_of(a)); }

size_t attention_counter_ints(const AttnArgs &a) {
  if (a.n <= 0 || a.n_head_kv <= 0 || a.n_head % a.n_head_kv != 0) return 0;
  const int G = a.n_head / a.n_head_kv;
  int HG, PB;
  query_wave_layout(G, &HG, &PB);
  return (size_t)a.n_head_kv * (G / HG) * ((a.n + 32 * PB - 1) / (32 * PB)) * 4;
}

size_t attention_workspace_bytes(const AttnArgs &a) {
  if (a.n <= 0 || a.n_head_kv <= 0 || a.n_head % a.n_head_kv != 0 || a.capacity <= 0) return 0;
  const Window w = window_of(a);
  return window_bytes(a, w) + partial_bytes(a, plan_attention(a, w));
}

int32_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (a.n <= 0) return SULIMO_HIP_OK;
  if (a.n_head_kv <= 0 || a.n_head % a.n_head_kv != 0)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "head_count must be a multiple of head_count_kv");
  if (a.capacity <= 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "capacity must be positive");
  if (!a.window) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "attention needs its key-window workspace");
  if (window_bytes(a, window_of(a)) / 2 >= (1ull << 31))
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "attention key window exceeds 2 GiB");
  switch (a.head_dim) {
    case 64: return launch_hd<64>(a, s);
    case 128: return launch_hd<128>(a, s);
    default: return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "attention supports head_dim 64 or 128");
  }
}

}  // namespace sulimo
