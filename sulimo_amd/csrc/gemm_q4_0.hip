// gemm_q4_0.hip - Q4_0 weight x f16 activation GEMM on gfx950 MFMA.
//
// Replaces kernels/gemm_q4_0.cl:13-130 (one work-item per output, no reuse).
// Y[t][j] = sum_k X[t][k] * W[j][k], W[j][32b+i] = (q-8) * d[j][b] (Q4_0 SoA,
// crates/sulimo-core/src/repack.rs:107-131), f32 accumulation, epilogue per use.
//
// One workgroup = 4 wave64s; tile BM tokens x BN weight rows (BN = 4 waves x 32*FN).
// k advances in stages of 64 (two Q4_0 blocks).
//  * Every operand streams global -> LDS with buffer_load ... lds (no VGPR staging)
//    into a ring of NS stage slots, NS-1 stages ahead of use. Each lane's buffer
//    offset is fixed for the whole kernel and the stage advances through the scalar
//    offset, so a stage's DMA costs no vector instructions. Rows past the matrix
//    get an offset past the buffer's end, which the buffer unit turns into zeros.
//  * Weights come from the panel copy (q4_panels.hip): one stage of 32 rows is one
//    1 KB run of quants plus 128 bytes of scales, fetched with full 16-byte lanes.
//  * A slot holds the X tile (BM rows x 128 bytes, 16-byte chunk c of row r at slot
//    position c ^ ((r >> 1) & 7): the MFMA A-fragment reads are bank-conflict free),
//    the quants (per 32-row fragment: lane l's 16 bytes at 16*l, one linear read) and
//    the scales [BN rows][2 x f16].
//  * Every ring slot is its own LDS variable and the stage loop is unrolled by NS, so
//    the compiler can tell the refill of one slot from the reads of another and keeps
//    the ring in flight instead of draining it before each read.
//  * Each wave dequantizes its own 32*FN weight rows straight into MFMA B operands and
//    reuses them for all BM rows: (1024+q) - 1032 exactly (low nibbles) or
//    (1024+16q)/16 - 72 exactly (high nibbles), then * d with one rounding to f16.
//  * v_mfma_f32_32x32x16_f16, lane layout: lane l supplies A[row l%32][k 8*(l/32)..+7]
//    and B[k 8*(l/32)..+7][col l%32], and receives C[8*(r/4) + 4*(l/32) + r%4][l%32]
//    in accumulator register r. MFMA step s of a stage covers stage k 16s..16s+15:
//    block s/2, elements 16*(s%2) + 8*(l/32)..+7, i.e. the low (s even) or high
//    (s odd) nibbles of bytes 8*(l/32)..+7 of the block.
//  * One barrier per stage: wait for this stage's slot (explicit vmcnt), barrier,
//    then refill the slot every wave finished reading in the previous stage.
//  * An odd block count ends in a half stage: its second block has scale 0 in the
//    panels and its X chunks past K are zero-filled.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kBK = 64;                   // k per stage
constexpr uint32_t kOob = 0x80000000u;    // buffer offset past every buffer: reads as zero
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9)
constexpr int kXcds = 8;                      // XCDs of an MI355X

template <int J>
using ic = std::integral_constant<int, J>;

template <typename F, int... J>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, J...>) {
  (f(ic<J>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)kRsrcWord3);
}

// One buffer -> LDS DMA: active lane i writes 16 bytes at dst + 16*i.
__device__ __forceinline__ void dma16(rsrc_t r, void *dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, (int)voff, soff, 0, 0);
}

// Four nibbles, one per byte in bits [3:0] (HI = false) or [7:4] (HI = true) with the
// other bits clear -> two half2 of (q-8)*d.
template <bool HI>
__device__ __forceinline__ void dq4(uint32_t nib, half2v d2, half2v &a, half2v &b) {
  // bytes [n0, 0x64, n1, 0x64] -> half2(1024 + n0, 1024 + n1), exact
  const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
  const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
  if constexpr (HI) {  // 1024 + 16q: /16 - 72 = q - 8, one exact fma
    const half2v s = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2v o = {(_Float16)-72.0f, (_Float16)-72.0f};
    a = __builtin_elementwise_fma(as_h2(p0), s, o) * d2;
    b = __builtin_elementwise_fma(as_h2(p1), s, o) * d2;
  } else {
    const half2v o = {(_Float16)1032.0f, (_Float16)1032.0f};
    a = (as_h2(p0) - o) * d2;
    b = (as_h2(p1) - o) * d2;
  }
}

// The same four nibbles -> two half2 of q-8 (exact, unscaled).
template <bool HI>
__device__ __forceinline__ void dq4_raw(uint32_t nib, half2v &a, half2v &b) {
  const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
  const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
  if constexpr (HI) {
    const half2v s = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2v o = {(_Float16)-72.0f, (_Float16)-72.0f};
    a = __builtin_elementwise_fma(as_h2(p0), s, o);
    b = __builtin_elementwise_fma(as_h2(p1), s, o);
  } else {
    const half2v o = {(_Float16)1032.0f, (_Float16)1032.0f};
    a = as_h2(p0) - o;
    b = as_h2(p1) - o;
  }
}

// s_waitcnt vmcnt(n) with expcnt and lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier that orders LDS accesses only: global loads and stores in flight
// stay in flight (__syncthreads also waits for those).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Lane exchanges within a quad of lanes (DPP quad_perm): partner lane j^1, j^2.
__device__ __forceinline__ uint32_t dpp_xor1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t dpp_xor2(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t fu(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float uf(uint32_t v) { return __builtin_bit_cast(float, v); }

// 4 x 4 transposes across a lane quad. Lane j of the quad holds rows 0..3 of column j;
// afterwards it holds row j, columns 0..3. Every lane of the quad must be active.
// f16: p = rows 0,1 and q = rows 2,3 (packed); returns columns 0,1 and 2,3 (packed).
__device__ __forceinline__ uint2 quad_t16(uint32_t p, uint32_t q, int j) {
  const uint32_t sel = (j & 1) ? 0x03020706u : 0x05040100u;
  const uint32_t x = __builtin_amdgcn_perm(dpp_xor1(p), p, sel);  // row j&1 (odd) or 0, columns pair of j
  const uint32_t y = __builtin_amdgcn_perm(dpp_xor1(q), q, sel);  // row 2 + (j&1)
  const uint32_t r = dpp_xor2((j & 2) ? x : y);
  return (j & 2) ? uint2{r, y} : uint2{x, r};
}
__device__ __forceinline__ float4 quad_t32(float a0, float a1, float a2, float a3, int j) {
  const bool odd = j & 1, h = j & 2;
  const float r1 = uf(dpp_xor1(fu(odd ? a0 : a1)));
  const float r2 = uf(dpp_xor1(fu(odd ? a2 : a3)));
  const float x0 = odd ? r1 : a0, x1 = odd ? a1 : r1;  // row j&1, the pair of columns holding j
  const float y0 = odd ? r2 : a2, y1 = odd ? a3 : r2;  // row 2 + (j&1)
  const float t0 = uf(dpp_xor2(fu(h ? x0 : y0))), t1 = uf(dpp_xor2(fu(h ? x1 : y1)));
  return h ? float4{t0, t1, y0, y1} : float4{x0, x1, t0, t1};
}
// Four consecutive K-split partials as f32, stored as f16 or f32.
template <bool F16>
__device__ __forceinline__ float4 load_part4(const float *part, size_t idx) {
  if constexpr (F16) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 v = *reinterpret_cast<const h4 *>(reinterpret_cast<const _Float16 *>(part) + idx);
    return float4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  } else {
    return *reinterpret_cast<const float4 *>(part + idx);
  }
}
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

template <int FM, int FN, int kNS, int EPI, int KSPLIT, int WM>
__global__ __launch_bounds__(256 * KSPLIT, (WM == 2 || KSPLIT > 1) ? 1 : 2) void gemm_q4_kernel(GemmArgs a) {
  constexpr int WN = 4 / WM;                      // waves along the weight rows
  constexpr int BM = 32 * FM * WM;
  constexpr int BN = 32 * FN * WN;                // weight rows per tile
  constexpr bool kSwiglu = (EPI == EPI_SWIGLU);
  constexpr int OUT_BN = kSwiglu ? BN / 2 : BN;   // output columns per tile
  constexpr int NX = FM * WM;                     // X DMA instructions per wave per stage
  constexpr int NQ = FN * WN / 4;                 // quant DMA instructions per wave per stage
  constexpr int NDMA = NX + NQ + 1;               // + one scale DMA per wave per stage
  // Order of a stage's DMA group. Tiles with at least twice as many X as quant
  // instructions issue the weights (quants, scales) first: measured 1-2.6 % faster on
  // those kernels and 0.4-2.2 % slower on the others (same-box kernel traces).
  constexpr bool kWeightsFirst = NX >= 2 * NQ;
  constexpr int X_BYTES = BM * kBK * 2;
  constexpr int Q_BYTES = BN * 32;
  constexpr int S_BYTES = BN * 4;
  constexpr int SLOT = X_BYTES + Q_BYTES + S_BYTES;
  static_assert(!kSwiglu || FN % 2 == 0, "SwiGLU pairs gate and up fragments in one wave");
  static_assert(kNS >= 2 && kNS <= 6, "ring depth");
  static_assert(KSPLIT == 1 || KSPLIT == 2 || (KSPLIT == 4 && FM == 1), "k split (four parts: 32-row tiles, 128 VGPRs a wave)");
  static_assert(WM == 1 || (WM == 2 && KSPLIT == 1 && FN % 2 == 0), "wave grid");

  // Ring slots of each part of the K range the workgroup splits (one part: no split).
  constexpr int SLOT2 = KSPLIT > 1 ? SLOT : 16;
  constexpr int SLOT4 = KSPLIT > 2 ? SLOT : 16;
  __shared__ __attribute__((aligned(16))) char smem0[SLOT];
  __shared__ __attribute__((aligned(16))) char smem1[SLOT];
  __shared__ __attribute__((aligned(16))) char smem2[kNS > 2 ? SLOT : 16];
  __shared__ __attribute__((aligned(16))) char smem3[kNS > 3 ? SLOT : 16];
  __shared__ __attribute__((aligned(16))) char smem4[kNS > 4 ? SLOT : 16];
  __shared__ __attribute__((aligned(16))) char smem5[kNS > 5 ? SLOT : 16];
  __shared__ __attribute__((aligned(16))) char smemb0[SLOT2];
  __shared__ __attribute__((aligned(16))) char smemb1[SLOT2];
  __shared__ __attribute__((aligned(16))) char smemb2[kNS > 2 ? SLOT2 : 16];
  __shared__ __attribute__((aligned(16))) char smemb3[kNS > 3 ? SLOT2 : 16];
  __shared__ __attribute__((aligned(16))) char smemb4[kNS > 4 ? SLOT2 : 16];
  __shared__ __attribute__((aligned(16))) char smemb5[kNS > 5 ? SLOT2 : 16];
  __shared__ __attribute__((aligned(16))) char smemc0[SLOT4];
  __shared__ __attribute__((aligned(16))) char smemc1[SLOT4];
  __shared__ __attribute__((aligned(16))) char smemc2[kNS > 2 ? SLOT4 : 16];
  __shared__ __attribute__((aligned(16))) char smemd0[SLOT4];
  __shared__ __attribute__((aligned(16))) char smemd1[SLOT4];
  __shared__ __attribute__((aligned(16))) char smemd2[kNS > 2 ? SLOT4 : 16];
  static_assert(KSPLIT < 4 || kNS == 3, "four K parts keep three ring slots each");
  auto slot_ptr = [&](auto H, auto J) -> char * {
    constexpr int j = decltype(J)::value % kNS;
    constexpr int h = decltype(H)::value;
    if constexpr (h == 0) {
      if constexpr (j == 0) return smem0;
      else if constexpr (j == 1) return smem1;
      else if constexpr (j == 2) return smem2;
      else if constexpr (j == 3) return smem3;
      else if constexpr (j == 4) return smem4;
      else return smem5;
    } else if constexpr (h == 1) {
      if constexpr (j == 0) return smemb0;
      else if constexpr (j == 1) return smemb1;
      else if constexpr (j == 2) return smemb2;
      else if constexpr (j == 3) return smemb3;
      else if constexpr (j == 4) return smemb4;
      else return smemb5;
    } else if constexpr (h == 2) {
      if constexpr (j == 0) return smemc0;
      else if constexpr (j == 1) return smemc1;
      else return smemc2;
    } else {
      if constexpr (j == 0) return smemd0;
      else if constexpr (j == 1) return smemd1;
      else return smemd2;
    }
  };

  // wave = wave within its part of the K range (4 per part); kh = the part it runs
  // wave and kh are wave-uniform: read into scalars, so that the LDS destinations of the
  // DMA (M0) are computed once in scalar registers instead of per stage
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3), kh = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int l32 = lane & 31, lg = lane >> 5;
  const int wave_m = wave % WM, wave_n = wave / WM;  // the wave's 32*FM rows and 32*FN weight rows

  // --- workgroup -> (K split, tile). Workgroups are dispatched round-robin over the
  // XCDs, each with its own L2: XCD e runs a contiguous range of the work order (split
  // major, then tiles), and the tile order walks group_m tile rows at a time, so the
  // workgroups resident on one XCD share their X rows and weight rows in its L2. Any
  // XCD count gives the same work items.
  // Persistent mode (a.persist set by the launcher: a grid of resident workgroups,
  // one-part tiles of one segment, no split, an even block count, stages a multiple of
  // NS, the f16 or SwiGLU epilogue): a workgroup runs every (workgroups per XCD)-th item
  // of its XCD's range, and the last NS-1 refills of a tile load the next tile's first
  // NS-1 stages into the same ring slots, so they land under the epilogue. Otherwise a
  // workgroup runs one item. The loop over items below spans the rest of the kernel
  // body (not indented).
  const int ntiles = a.tiles_m * a.tiles_n;
  const int nwork = ntiles * a.splits;
  const int xcd = blockIdx.x % kXcds, jx = blockIdx.x / kXcds;
  const int xlo = xcd * (nwork / kXcds) + min(xcd, nwork % kXcds);
  const int xend = xlo + nwork / kXcds + (xcd < nwork % kXcds ? 1 : 0);
  constexpr bool kCanPersist = KSPLIT == 1 && WM == 1 && (EPI == EPI_SWIGLU || EPI == EPI_F16);
  const int xstep = (kCanPersist && a.persist) ? (int)(gridDim.x / kXcds) : 0;
  if (xlo + jx >= xend) return;  // persistent grid wider than the XCD's range
  auto tile_of = [&](int w, int &tm, int &tn) {
    const int tt = w % ntiles;
    const int gr = tt / (a.group_m * a.tiles_n), tgg = tt - gr * a.group_m * a.tiles_n;
    const int gmm = min(a.group_m, a.tiles_m - gr * a.group_m);
    tm = gr * a.group_m + tgg % gmm;
    tn = tgg / gmm;
  };
  bool primed = false;  // this tile's first NS-1 stages were issued by the previous tile
  for (int w_item = xlo + jx;; w_item += xstep) {  // work items of this workgroup
  const bool has_next = xstep > 0 && w_item + xstep < xend;
  const int ks = w_item / ntiles;
  int tile_m, tile_n;
  tile_of(w_item, tile_m, tile_n);
  // --- tile -> (segment, first output column, first row) ---
  int si = 0, colbase = 0;  // colbase: columns of the segments before (partial sums)
  for (; si < a.nseg - 1; si++) {
    const int tn = (a.seg[si].n + OUT_BN - 1) / OUT_BN;
    if (tile_n < tn) break;
    tile_n -= tn;
    colbase += a.seg[si].n;
  }
  const GemmSegment seg = a.seg[si];
  const int c0 = tile_n * OUT_BN;
  const int m0 = tile_m * BM;
  const int nb = a.k >> 5;           // Q4_0 blocks per weight row
  const int nst = (nb + 1) >> 1;     // stages (the last is a half stage when nb is odd)

  const int npanels = (seg.n + 31) / 32 * (kSwiglu ? 2 : 1);
  const rsrc_t rx = make_rsrc(a.x, (uint32_t)a.m * (uint32_t)a.ldx * 2u);
  const rsrc_t rp = make_rsrc(seg.panels, (uint32_t)npanels * (uint32_t)nst * (uint32_t)kQ4PanelRecord);

  // Tile fragment g = FN*wn + f (fragment f of the waves at wave_n = wn) -> panel (or -1
  // past the matrix). Fragment g covers output columns c0 + 32*g ..; with SwiGLU the
  // waves at wn cover 16*FN columns, their first FN/2 fragments are the gate panels and
  // the rest the up panels.
  auto panel_of = [&](int g) -> int {
    int p;
    if constexpr (kSwiglu) {
      const int wn = g / FN, f = g % FN;
      const int j = c0 / 32 + wn * (FN / 2) + (f % (FN / 2));
      p = 2 * j + (f >= FN / 2 ? 1 : 0);
    } else {
      p = c0 / 32 + g;
    }
    return p < npanels ? p : -1;
  };

  // --- per-lane DMA offsets (bytes), fixed for the whole kernel ---
  // X: wave instruction i covers tile rows 8*(NX*wave+i) .. +7; chunk c of row r lands at
  // slot position c ^ ((r >> 1) & 7).
  uint32_t xoff[NX];
  bool xhi[NX];  // chunk in the stage's second block
#pragma unroll
  for (int i = 0; i < NX; i++) {
    const int row = 8 * (NX * wave + i) + (lane >> 3);
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    const int r = m0 + row;
    xoff[i] = r < a.m ? ((uint32_t)r * (uint32_t)a.ldx + 8u * chunk) * 2u : kOob;
    xhi[i] = chunk >= 4;
  }
  // Quants: wave instruction f copies tile fragment NQ*wave + f's 1 KB record run (lane =
  // 16 bytes). Scales: lanes 8f .. 8f+7 of the wave's scale instruction copy tile
  // fragment NQ*wave + f's 128 bytes.
  uint32_t qoff[NQ], soff;
#pragma unroll
  for (int f = 0; f < NQ; f++) {
    const int p = panel_of(NQ * wave + f);
    qoff[f] = p >= 0 ? (uint32_t)p * (uint32_t)nst * kQ4PanelRecord + 16u * lane : kOob;
  }
  {
    const int f = lane >> 3;  // lanes past 8*NQ never issue
    const int p = f < NQ ? panel_of(NQ * wave + f) : -1;
    soff = p >= 0 ? (uint32_t)p * (uint32_t)nst * kQ4PanelRecord + 1024u + 16u * (lane & 7) : kOob;
  }
  auto issue = [&](auto H, auto J, int st, auto kCheck) __attribute__((always_inline)) {
    char *slot = slot_ptr(H, J);
    const int sst = st < nst ? st : 0;
    bool half = false;
    if constexpr (decltype(kCheck)::value) half = (2 * sst + 1 == nb);
    auto x_part = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NX; i++) {
        const uint32_t off = (half && xhi[i]) ? kOob : xoff[i];
        dma16(rx, slot + 8 * (NX * wave + i) * kBK * 2, off, sst * kBK * 2);
      }
    };
    auto w_part = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int f = 0; f < NQ; f++) dma16(rp, slot + X_BYTES + (NQ * wave + f) * 1024, qoff[f], sst * kQ4PanelRecord);
      if (lane < 8 * NQ) dma16(rp, slot + X_BYTES + Q_BYTES + NQ * wave * 128, soff, sst * kQ4PanelRecord);
    };
    if constexpr (kWeightsFirst) {
      w_part();
      x_part();
    } else {
      x_part();
      w_part();
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int f = 0; f < FN; f++) acc[i][f] = floatx16{};

  auto read_a = [&](const _Float16 *xb, int s, half8 (&ao)[FM]) {
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int row = 32 * (FM * wave_m + i) + l32;
      const int pos = (2 * s + lg) ^ ((row >> 1) & 7);
      ao[i] = *reinterpret_cast<const half8 *>(xb + row * kBK + 8 * pos);
    }
  };
  auto mfmas = [&](const half8 (&ao)[FM], const half8 (&bo)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int f = 0; f < FN; f++)
        acc[i][f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ao[i], bo[f], acc[i][f], 0, 0, 0);
  };

  // One stage in slot J of half H. kCheck: the stage or the one it prefetches may be
  // the half stage. An inactive stage (past the half's range) only keeps the ring and the
  // barrier count in step.
  // The next tile's stage nsst into slot J (persistent mode, one segment, no split, even
  // block count): the same offsets as issue's, for the next tile's rows and panels.
  uint32_t nxoff[NX], nqoff[NQ], nsoff;
  auto issue_next = [&](auto J, int nsst) __attribute__((always_inline)) {
    char *slot = slot_ptr(ic<0>{}, J);
    auto x_part = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NX; i++) dma16(rx, slot + 8 * (NX * wave + i) * kBK * 2, nxoff[i], nsst * kBK * 2);
    };
    auto w_part = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int f = 0; f < NQ; f++)
        dma16(rp, slot + X_BYTES + (NQ * wave + f) * 1024, nqoff[f], nsst * kQ4PanelRecord);
      if (lane < 8 * NQ) dma16(rp, slot + X_BYTES + Q_BYTES + NQ * wave * 128, nsoff, nsst * kQ4PanelRecord);
    };
    if constexpr (kWeightsFirst) {
      w_part();
      x_part();
    } else {
      x_part();
      w_part();
    }
  };
  auto next_offsets = [&]() __attribute__((always_inline)) {
    int ntm, ntn;
    tile_of(w_item + xstep, ntm, ntn);
    const int nm0 = ntm * BM, nc0 = ntn * OUT_BN;
#pragma unroll
    for (int i = 0; i < NX; i++) {
      const int row = 8 * (NX * wave + i) + (lane >> 3);
      const int chunk = (lane & 7) ^ ((row >> 1) & 7);
      const int r = nm0 + row;
      nxoff[i] = r < a.m ? ((uint32_t)r * (uint32_t)a.ldx + 8u * chunk) * 2u : kOob;
    }
    auto npanel_of = [&](int g) -> int {
      int p;
      if constexpr (kSwiglu) {
        const int wn = g / FN, f = g % FN;
        const int j = nc0 / 32 + wn * (FN / 2) + (f % (FN / 2));
        p = 2 * j + (f >= FN / 2 ? 1 : 0);
      } else {
        p = nc0 / 32 + g;
      }
      return p < npanels ? p : -1;
    };
#pragma unroll
    for (int f = 0; f < NQ; f++) {
      const int p = npanel_of(NQ * wave + f);
      nqoff[f] = p >= 0 ? (uint32_t)p * (uint32_t)nst * kQ4PanelRecord + 16u * lane : kOob;
    }
    const int f = lane >> 3;
    const int p = f < NQ ? npanel_of(NQ * wave + f) : -1;
    nsoff = p >= 0 ? (uint32_t)p * (uint32_t)nst * kQ4PanelRecord + 1024u + 16u * (lane & 7) : kOob;
  };

  // need_wait false: the stage's slot was waited for before the previous tile's epilogue
  // (stage 0 of a tile whose first stages the previous tile loaded).
  auto stage = [&](auto H, auto J, int st, auto kCheck, bool active, auto kNext, bool need_wait) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    // stage st was issued NS-1 stages ago, (NS-2)*NDMA DMA instructions after it
    if (need_wait) wait_vmcnt<(kNS - 2) * NDMA>();
    // plain s_barrier: the slot is filled (vmcnt above) and the previous stage's LDS
    // reads were consumed by its MFMAs; a fenced barrier would drain every prefetch
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // refills the slot of stage st-1; in a tile's last ring cycle with kNext, with the
    // next tile's stage J-1 (stage st-1 is its tile's last when J is 0)
    if constexpr (decltype(kNext)::value && decltype(J)::value > 0)
      issue_next(ic<decltype(J)::value - 1>{}, decltype(J)::value - 1);
    else
      issue(H, ic<decltype(J)::value + kNS - 1>{}, st + kNS - 1, kCheck);
    if (!active) return;
    const char *slot = slot_ptr(H, J);
    const _Float16 *xb = reinterpret_cast<const _Float16 *>(slot);
    // raw weights of this wave's fragments: 8 bytes per block, and the stage's 2 scales
    uint2 q[FN][2];
    half2v d2[FN][2];
#pragma unroll
    for (int f = 0; f < FN; f++) {
      const int L = wave_n * 32 * FN + 32 * f + l32;
      const uint4 qv = *reinterpret_cast<const uint4 *>(slot + X_BYTES + (FN * wave_n + f) * 1024 + 16 * lane);
      q[f][0] = uint2{qv.x, qv.y};
      q[f][1] = uint2{qv.z, qv.w};
      const uint32_t w = *reinterpret_cast<const uint32_t *>(slot + X_BYTES + Q_BYTES + L * 4);
      d2[f][0] = as_h2(__builtin_amdgcn_perm(w, w, 0x01000100u));
      d2[f][1] = as_h2(__builtin_amdgcn_perm(w, w, 0x03020302u));
    }
    auto dequant_step = [&](int s, half8 (&bo)[FN]) {
      const int b = s >> 1;
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const uint2 qq = q[f][b];
        half2v p0, p1, p2, p3;
        if (s & 1) {
          dq4<true>(qq.x & 0xF0F0F0F0u, d2[f][b], p0, p1);
          dq4<true>(qq.y & 0xF0F0F0F0u, d2[f][b], p2, p3);
        } else {
          dq4<false>(qq.x & 0x0F0F0F0Fu, d2[f][b], p0, p1);
          dq4<false>(qq.y & 0x0F0F0F0Fu, d2[f][b], p2, p3);
        }
        bo[f] = half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      }
    };
    // k-step pipeline: operands of step s+1 are prepared before the MFMAs of step s
    half8 a0[FM], a1[FM], b0[FN], b1[FN];
    read_a(xb, 0, a0);
    dequant_step(0, b0);
    read_a(xb, 1, a1);
    dequant_step(1, b1);
    mfmas(a0, b0);
    read_a(xb, 2, a0);
    dequant_step(2, b0);
    mfmas(a1, b1);
    read_a(xb, 3, a1);
    dequant_step(3, b1);
    mfmas(a0, b0);
    mfmas(a1, b1);
  };

  // The workgroup's K split covers stages [kb, ke); each k half runs nst_h stages
  // [sb, sb + nst_h) of it (the last half fewer real ones). Main loop: straight-line bodies of NS stages (no branches between
  // stages keeps the wait analysis per slot) over the stages that are active, full, and
  // prefetch no half stage; the rest go through the checked tail. Every half runs the
  // same number of stages, hence of barriers.
  using yes = std::true_type;
  using no = std::false_type;
  const int kb = ks * a.split_stages;
  const int ke = min(nst, kb + a.split_stages);
  const int nst_h = (ke - kb + KSPLIT - 1) / KSPLIT;
  auto run = [&](auto H) __attribute__((always_inline)) {
    const int sb = kb + decltype(H)::value * nst_h;
    const int se = min(ke, sb + nst_h);
    if (!primed) static_for<kNS - 1>([&](auto J) { issue(H, J, sb + decltype(J)::value, yes{}); });
    int lim = se - sb;
    if (nb & 1) lim = min(lim, nst - kNS - sb);  // stage nst-NS prefetches the half stage
    lim = max(lim, 0);
    int s0 = 0;
    // with a next tile (stages a multiple of NS), the last ring cycle is peeled
    const int lim_main = (kCanPersist && has_next) ? lim - kNS : lim;
    for (; s0 + kNS <= lim_main; s0 += kNS)
      static_for<kNS>([&](auto J) {
        stage(H, J, sb + s0 + decltype(J)::value, no{}, true, no{}, decltype(J)::value != 0 || s0 != 0 || !primed);
      });
    if constexpr (kCanPersist) {
      if (has_next) {
        next_offsets();
        static_for<kNS>([&](auto J) {
          stage(H, J, sb + s0 + decltype(J)::value, no{}, true, yes{}, decltype(J)::value != 0 || s0 != 0 || !primed);
        });
        s0 += kNS;
        // the next tile's stage 0 (NS-2 DMA groups issued after it) lands before the
        // epilogue, so that tile's first stage waits for none of the epilogue's stores
        wait_vmcnt<(kNS - 2) * NDMA>();
      }
    }
    static_for<2 * kNS>([&](auto J) {
      const int st = sb + s0 + decltype(J)::value;
      if (s0 + decltype(J)::value < nst_h) stage(H, J, st, yes{}, st < se, no{}, true);
    });
  };
  if constexpr (KSPLIT == 1) {
    run(ic<0>{});
  } else if constexpr (KSPLIT == 2) {
    if (kh == 0) run(ic<0>{});
    else run(ic<1>{});
  } else {
    if (kh == 0) run(ic<0>{});
    else if (kh == 1) run(ic<1>{});
    else if (kh == 2) run(ic<2>{});
    else run(ic<3>{});
  }
  // no DMA may still be writing this workgroup's LDS when it exits (a next tile's first
  // stages stay in flight: the epilogues that allow persistence use no LDS)
  if (!has_next) wait_vmcnt<0>();
  // Accumulator register group q (registers 4q .. 4q+3: rows 8q + 4lg .. +3 of every
  // fragment) belongs to K part q / NQO. After the combine each part holds the full sums
  // of its NQO groups in registers 0 .. 4*NQO-1 and runs the epilogue for those rows:
  // every wave of the workgroup shares the epilogue.
  constexpr int NQO = 4 / KSPLIT;
  const int qbase = kh * NQO;
  // RoPE epilogue: cos/sin of the lane's 4 elements in fragment i (NeoX: 4 pairs from
  // index e mod half; Norm: 2 pairs from e/2), rows past the ubatch clamped to its last
  // row. Fragment 0's loads are issued here, under the K-part combine.
  float4 rca[FN][NQO], rcb[FN][NQO];
  auto rope_cs_load = [&](int i) __attribute__((always_inline)) {
    if constexpr (EPI == EPI_ROPE) {
      const int hd = a.rope.head_dim, hhalf = hd >> 1;
      const bool neox = a.rope.mode != 0;
      const int qj = lane & 3, cq = 4 * (l32 >> 2);
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const int e = (c0 + wave_n * 32 * FN + 32 * f + cq) & (hd - 1);
        const int idx = neox ? (e < hhalf ? e : e - hhalf) : e / 2;
#pragma unroll
        for (int lq = 0; lq < NQO; lq++) {
          const int row = min(m0 + 32 * i + 4 * lg + qj + 8 * (qbase + lq), a.m - 1);
          const float4 *cs = reinterpret_cast<const float4 *>(a.rope.cs + 2 * ((size_t)row * hhalf + idx));
          rca[f][lq] = cs[0];
          rcb[f][lq] = cs[neox ? 1 : 0];  // unconditional load: no branch between the loads
        }
      }
    }
  };
  // (loaded by every wave and tile, so that no branch joins the loads to their uses: the
  // rows are clamped and the indices valid in every case)
  if constexpr (EPI == EPI_ROPE) rope_cs_load(0);
  if constexpr (KSPLIT > 1) {
    // Reduce-scatter through the parts' first ring slots (every DMA has landed and every
    // ring read is done): in round o of a fragment the parts other than o write their
    // registers 4*NQO*o .. +4*NQO-1, and part o adds all parts' values in part order,
    // the sums the parts would give added into part 0 one after another.
    constexpr int RG = 4 * NQO;  // registers per round
    static_assert(SLOT >= 256 * RG * 4, "combine buffer fits a ring slot");
    auto slot0 = [&](int part) -> float * {
      return reinterpret_cast<float *>(part == 0 ? smem0 : part == 1 ? smemb0 : part == 2 ? smemc0 : smemd0);
    };
    // registers r .. r+3 of lane cidx at float4 (r / 4) * 256 + cidx: consecutive lanes
    // write and read consecutive 16 bytes (no bank conflicts)
    const int cidx = wave * 64 + lane;
    float4 *mine = reinterpret_cast<float4 *>(slot0(kh)) + cidx;
    lds_barrier();
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int f = 0; f < FN; f++)
#pragma unroll
        for (int o = 0; o < KSPLIT; o++) {
          if (kh != o) {
#pragma unroll
            for (int r = 0; r < RG; r += 4)
              mine[r / 4 * 256] =
                  float4{acc[i][f][RG * o + r], acc[i][f][RG * o + r + 1], acc[i][f][RG * o + r + 2], acc[i][f][RG * o + r + 3]};
          }
          lds_barrier();
          if (kh == o) {
#pragma unroll
            for (int r = 0; r < RG; r += 4) {
              float w[KSPLIT][4];
#pragma unroll
              for (int p = 0; p < KSPLIT; p++) {
                if (p == o) continue;
                const float4 t = reinterpret_cast<const float4 *>(slot0(p))[r / 4 * 256 + cidx];
                w[p][0] = t.x;
                w[p][1] = t.y;
                w[p][2] = t.z;
                w[p][3] = t.w;
              }
#pragma unroll
              for (int e = 0; e < 4; e++) {
                float v = o == 0 ? acc[i][f][RG * o + r + e] : w[0][e];
#pragma unroll
                for (int p = 1; p < KSPLIT; p++) v += p == o ? acc[i][f][RG * o + r + e] : w[p][e];
                acc[i][f][RG * o + r + e] = v;
              }
            }
          }
          lds_barrier();
        }
    // the part's own groups to registers 0 .. RG-1 (static register indices)
#pragma unroll
    for (int o = 1; o < KSPLIT; o++) {
      if (kh == o) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int f = 0; f < FN; f++)
#pragma unroll
            for (int r = 0; r < RG; r++) acc[i][f][r] = acc[i][f][RG * o + r];
      }
    }
  }

  if constexpr (EPI == EPI_ROPE) {
    // --- RoPE + Q8_0 K/V store (segment 0: q, 1: k, 2: v; the tile holds whole heads).
    // Per 32-row fragment i: the f16-rounded outputs (+ bias) are quad-transposed so that
    // lane (qj, g = l32/4, lg) holds row 8q + 4lg + qj, columns 4g .. 4g+3 of fragment f.
    // NeoX partners (column ^ head_dim/2) come through a [32][BN + 8] f16 exchange tile
    // in ring slot 0. A Q8_0 block is one fragment's 32 columns of a row: 8 lanes (lane
    // bits 2-4). The f16 window entries of v go to V^T rows after transposing back (lane
    // = one column, 4 consecutive tokens). Every load of a fragment is issued before its
    // first store (the stores could alias the table as far as the compiler knows), and
    // the block maxima of all its rows reduce together. With K parts, each part does its
    // own row groups.
    const GemmRope &rp = a.rope;
    const int hd = rp.head_dim, hsh = __builtin_ctz((unsigned)hd), hhalf = hd >> 1;
    const bool neox = rp.mode != 0, rotate = si < 2;
    constexpr int RS = BN + 8;  // exchange tile row stride (f16)
    static_assert(32 * RS * 2 <= SLOT, "the exchange tile fits a ring slot");
    _Float16 *xt = reinterpret_cast<_Float16 *>(smem0);
    const int qj = lane & 3, cq = 4 * (l32 >> 2);
    float bias[FN];  // of the lane's column before the transpose
#pragma unroll
    for (int f = 0; f < FN; f++) {
      const int lcol = c0 + wave_n * 32 * FN + 32 * f;
      bias[f] = (seg.bias && lcol + l32 < seg.n) ? seg.bias[lcol + l32] : 0.0f;
    }
    if constexpr (KSPLIT == 1) lds_barrier();  // every wave has finished reading the ring
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int rbase = m0 + 32 * i + 4 * lg + qj;  // the lane's row for q = 0 (+ 8q)
      uint2 xv[FN][NQO], pv[FN][NQO];
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const float b = bias[f];
#pragma unroll
        for (int lq = 0; lq < NQO; lq++) {
          xv[f][lq] = quad_t16(pack_h2(acc[i][f][4 * lq] + b, acc[i][f][4 * lq + 1] + b),
                               pack_h2(acc[i][f][4 * lq + 2] + b, acc[i][f][4 * lq + 3] + b), qj);
          pv[f][lq] = xv[f][lq];
        }
      }
      const auto &ca = rca, &cb = rcb;
      if (rotate && neox) {
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
          for (int lq = 0; lq < NQO; lq++)
            *reinterpret_cast<uint2 *>(xt + (8 * (qbase + lq) + 4 * lg + qj) * RS + wave_n * 32 * FN + 32 * f + cq) =
                xv[f][lq];
        lds_barrier();
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
          for (int lq = 0; lq < NQO; lq++)
            pv[f][lq] = *reinterpret_cast<const uint2 *>(xt + (8 * (qbase + lq) + 4 * lg + qj) * RS +
                                                         ((wave_n * 32 * FN + 32 * f + cq) ^ hhalf));
        lds_barrier();
      }
      float o[FN][NQO][4];
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const int e = (c0 + wave_n * 32 * FN + 32 * f + cq) & (hd - 1);
#pragma unroll
        for (int q = 0; q < NQO; q++) {  // q: the part's row group qbase + q
          const half2v x01 = as_h2(xv[f][q].x), x23 = as_h2(xv[f][q].y);
          const float x[4] = {(float)x01[0], (float)x01[1], (float)x23[0], (float)x23[1]};
#pragma unroll
          for (int j = 0; j < 4; j++) o[f][q][j] = x[j];
          if (!rotate) continue;
          if (neox) {
            const half2v p01 = as_h2(pv[f][q].x), p23 = as_h2(pv[f][q].y);
            const float p[4] = {(float)p01[0], (float)p01[1], (float)p23[0], (float)p23[1]};
            const float cc[4] = {ca[f][q].x, ca[f][q].z, cb[f][q].x, cb[f][q].z};
            const float ss[4] = {ca[f][q].y, ca[f][q].w, cb[f][q].y, cb[f][q].w};
            const bool lo = e < hhalf;
#pragma unroll
            for (int j = 0; j < 4; j++) {
              if (lo) {
                const float v0 = x[j], v1 = p[j];
                o[f][q][j] = rot_sub(v0, cc[j], v1, ss[j]);
              } else {
                const float v0 = p[j], v1 = x[j];
                o[f][q][j] = rot_add(v0, ss[j], v1, cc[j]);
              }
            }
          } else {
            const float cc[2] = {ca[f][q].x, ca[f][q].z}, ss[2] = {ca[f][q].y, ca[f][q].w};
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
              const float v0 = x[j], v1 = x[j + 1];
              o[f][q][j] = rot_sub(v0, cc[j / 2], v1, ss[j / 2]);
              o[f][q][j + 1] = rot_add(v0, ss[j / 2], v1, cc[j / 2]);
            }
          }
        }
      }
      // the next fragment's cos/sin, issued before this fragment's stores (loads and
      // stores retire in issue order, so its wait then covers no store)
      if (i + 1 < FM) rope_cs_load(i + 1);
      if (si == 0) {
#pragma unroll
        for (int f = 0; f < FN; f++) {
          const int col = c0 + wave_n * 32 * FN + 32 * f + cq;  // the lane's first column in the segment
#pragma unroll
          for (int q = 0; q < NQO; q++) {
            const int row = rbase + 8 * (qbase + q);
            if (row < a.m && col < seg.n)
              *reinterpret_cast<uint2 *>(reinterpret_cast<_Float16 *>(seg.out) + (size_t)row * seg.ldo + seg.col0 + col) =
                  uint2{pack_h2(o[f][q][0], o[f][q][1]), pack_h2(o[f][q][2], o[f][q][3])};
          }
        }
        continue;
      }
      // Q8_0 of each block (8 lanes, same row): amax, d = amax / 127, codes
      float amax[FN][NQO];
#pragma unroll
      for (int f = 0; f < FN; f++)
#pragma unroll
        for (int q = 0; q < NQO; q++)
          amax[f][q] = fmaxf(fmaxf(fabsf(o[f][q][0]), fabsf(o[f][q][1])), fmaxf(fabsf(o[f][q][2]), fabsf(o[f][q][3])));
#pragma unroll
      for (int sh = 4; sh <= 16; sh *= 2)
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
          for (int q = 0; q < NQO; q++) amax[f][q] = fmaxf(amax[f][q], __shfl_xor(amax[f][q], sh, 64));
      uint8_t *dst = si == 1 ? rp.k_dst : rp.v_dst;
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const int col = c0 + wave_n * 32 * FN + 32 * f + cq;
        const int kvh = col >> hsh, e = col & (hd - 1);
#pragma unroll
        for (int q = 0; q < NQO; q++) {
          const int row = rbase + 8 * (qbase + q);
          const bool ok = row < a.m && col < seg.n;
          const float d = amax[f][q] / 127.0f;
          const float id = d != 0.0f ? 1.0f / d : 0.0f;
          float qc[4];
#pragma unroll
          for (int j = 0; j < 4; j++) qc[j] = fminf(fmaxf(roundf(o[f][q][j] * id), -128.0f), 127.0f);
          if (ok) {
            int slot = rp.slot0 + row;
            if (slot >= rp.wrap) slot %= rp.wrap;
            uint8_t *blk = dst + (size_t)slot * rp.row_bytes + (size_t)(kvh * (hd >> 5) + (e >> 5)) * 34;
            if ((e & 31) == 0) *reinterpret_cast<_Float16 *>(blk) = (_Float16)d;
            uint16_t *codes = reinterpret_cast<uint16_t *>(blk + 2 + (e & 31));  // 2-byte aligned
#pragma unroll
            for (int j = 0; j < 4; j += 2)
              codes[j / 2] = (uint16_t)((uint8_t)(int8_t)(int)qc[j] | ((uint16_t)(uint8_t)(int8_t)(int)qc[j + 1] << 8));
          }
          if (!rp.win.k) continue;
          // window entries f16(code * f16(d))
          const float dq = (float)(_Float16)d;
          const uint2 w = uint2{pack_h2(qc[0] * dq, qc[1] * dq), pack_h2(qc[2] * dq, qc[3] * dq)};
          if (si == 1) {
            if (ok)
              *reinterpret_cast<uint2 *>(reinterpret_cast<_Float16 *>(rp.win.k) +
                                         ((size_t)kvh * rp.win.pad + rp.win.j0 + row) * hd + e) = w;
          } else {
            // back to one column per lane: column l32 of fragment f, tokens t0 .. t0+3
            const uint2 wt = quad_t16(w.x, w.y, qj);
            const int t0 = m0 + 32 * i + 8 * (qbase + q) + 4 * lg;
            const int cv = c0 + wave_n * 32 * FN + 32 * f + l32;
            if (t0 >= a.m || cv >= seg.n) continue;
            _Float16 *vrow = reinterpret_cast<_Float16 *>(rp.win.vt) +
                             ((size_t)(cv >> hsh) * hd + (cv & (hd - 1))) * rp.win.vst;
            const int j = rp.win.j0 + t0;
            if ((j & 3) == 0 && t0 + 3 < a.m) {
              *reinterpret_cast<uint2 *>(vrow + window_vt_col(j)) = wt;  // 4 consecutive columns
            } else {
              const uint32_t ww[2] = {wt.x, wt.y};
              for (int jj = 0; jj < 4 && t0 + jj < a.m; jj++)
                reinterpret_cast<uint16_t *>(vrow)[window_vt_col(j + jj)] = (uint16_t)(ww[jj >> 1] >> (16 * (jj & 1)));
            }
          }
        }
      }
    }
    return;
  }

  // --- epilogue: acc register r of fragment (i, f) is C[8*(r/4) + 4*lg + r%4][l32], and
  // after a K-part combine register 4*lq + e is row group q = qbase + lq. Each
  // group q of 4 registers (4 rows of one column) is transposed across the lane quad, so
  // lane j of the quad stores row 8q + 4*lg + j, 4 consecutive columns, in one 8-byte
  // (f16) or 16-byte (f32) store. Vector stores need 4-element aligned rows; the last
  // group of a segment whose width is not a multiple of 4 stores element by element.
  const int qj = lane & 3;
  const int cq = 4 * (l32 >> 2);  // first column of the lane's 4 after the transpose
  const bool vec_ok = ((seg.ldo | seg.col0) & 3) == 0 && ((uintptr_t)seg.out & 15) == 0;
  // Residual epilogue of a small tile: every residual value of the vector path is loaded
  // before the first store (a load issued after a store waits for it: loads and stores
  // retire in issue order). Lanes outside the vector path read the row's first element
  // and load again in the element-wise path.
  constexpr bool kOldFirst = EPI == EPI_RESID && FM * NQO * FN <= 8;
  float4 rold[kOldFirst ? FM : 1][kOldFirst ? NQO : 1][kOldFirst ? FN : 1];
  if constexpr (kOldFirst) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int lq = 0; lq < NQO; lq++)
#pragma unroll
        for (int f = 0; f < FN; f++) {
          const int row = m0 + 32 * (FM * wave_m + i) + 8 * (qbase + lq) + 4 * lg + qj;
          const int col = c0 + wave_n * 32 * FN + 32 * f + cq;
          const bool ok = vec_ok && row < a.m && col + 4 <= seg.n;
          const float *src = reinterpret_cast<const float *>(seg.out) + (ok ? (size_t)row * seg.ldo + seg.col0 + col : 0);
          rold[i][lq][f] = *reinterpret_cast<const float4 *>(src);
        }
  }
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int lq = 0; lq < NQO; lq++) {  // the part's row groups q = qbase + lq (registers 4*lq ..)
      const int q = qbase + lq;
      const int row = m0 + 32 * (FM * wave_m + i) + 8 * q + 4 * lg + qj;
      if constexpr (kSwiglu) {
#pragma unroll
        for (int f = 0; f < FN / 2; f++) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            // gate and up rounded to f16 first, as their separate GEMM outputs would be
            const float g = (float)(_Float16)acc[i][f][4 * lq + e], u = (float)(_Float16)acc[i][f + FN / 2][4 * lq + e];
            v[e] = silu_mul(g, u);
          }
          const uint2 o = quad_t16(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), qj);
          const int col = c0 + wave_n * 16 * FN + 32 * f + cq;
          if (row < a.m && col < seg.n) {
            _Float16 *dst = reinterpret_cast<_Float16 *>(seg.out) + (size_t)row * seg.ldo + seg.col0 + col;
            if (vec_ok && col + 4 <= seg.n) {
              *reinterpret_cast<uint2 *>(dst) = o;
            } else {
              const uint32_t w[2] = {o.x, o.y};
              for (int e = 0; e < 4 && col + e < seg.n; e++)
                reinterpret_cast<uint16_t *>(dst)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
      } else {
#pragma unroll
        for (int f = 0; f < FN; f++) {
          const int lcol = c0 + wave_n * 32 * FN + 32 * f;  // first column of the fragment
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] = acc[i][f][4 * lq + e];
          if constexpr (EPI == EPI_F16 || EPI == EPI_F32) {
            if (seg.bias) {
              const float b = lcol + l32 < seg.n ? seg.bias[lcol + l32] : 0.0f;
#pragma unroll
              for (int e = 0; e < 4; e++) v[e] += b;
            }
          }
          const int col = lcol + cq;
          if constexpr (EPI == EPI_F16) {
            const uint2 o = quad_t16(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), qj);
            if (row < a.m && col < seg.n) {
              _Float16 *dst = reinterpret_cast<_Float16 *>(seg.out) + (size_t)row * seg.ldo + seg.col0 + col;
              if (vec_ok && col + 4 <= seg.n) {
                *reinterpret_cast<uint2 *>(dst) = o;
              } else {
                const uint32_t w[2] = {o.x, o.y};
                for (int e = 0; e < 4 && col + e < seg.n; e++)
                  reinterpret_cast<uint16_t *>(dst)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
              }
            }
          } else {
            if constexpr (EPI == EPI_RESID) {
#pragma unroll
              for (int e = 0; e < 4; e++) v[e] = (float)(_Float16)v[e];  // x += f16(acc)
            }
            const float4 o = quad_t32(v[0], v[1], v[2], v[3], qj);
            if (row < a.m && col < seg.n) {
              float *dst;
              bool vec;
              if constexpr (EPI == EPI_PART) {
                const size_t pi = (size_t)ks * a.m * a.ldp + colbase + (size_t)row * a.ldp + col;
                if (a.part_f16) {  // partials of an f16 output: one f16 rounding each
                  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                  _Float16 *pd = reinterpret_cast<_Float16 *>(a.part) + pi;
                  if (col + 4 <= seg.n) {  // partial planes are 4-column aligned
                    *reinterpret_cast<h4 *>(pd) = h4{(_Float16)o.x, (_Float16)o.y, (_Float16)o.z, (_Float16)o.w};
                  } else {
                    const float w[4] = {o.x, o.y, o.z, o.w};
                    for (int e = 0; e < 4 && col + e < seg.n; e++) pd[e] = (_Float16)w[e];
                  }
                  continue;
                }
                dst = a.part + pi;
                vec = col + 4 <= seg.n;
              } else {
                dst = reinterpret_cast<float *>(seg.out) + (size_t)row * seg.ldo + seg.col0 + col;
                vec = vec_ok && col + 4 <= seg.n;
              }
              if (vec) {
                float4 w = o;
                if constexpr (EPI == EPI_RESID) {
                  float4 old;
                  if constexpr (kOldFirst) old = rold[i][lq][f];
                  else old = *reinterpret_cast<const float4 *>(dst);
                  w = float4{old.x + o.x, old.y + o.y, old.z + o.z, old.w + o.w};
                }
                *reinterpret_cast<float4 *>(dst) = w;
              } else {
                const float w[4] = {o.x, o.y, o.z, o.w};
                for (int e = 0; e < 4 && col + e < seg.n; e++) dst[e] = EPI == EPI_RESID ? dst[e] + w[e] : w[e];
              }
            }
          }
        }
      }
    }
  }
  if (!has_next) break;
  primed = true;
  }  // work items
}

// Sum of the K splits' partials in split order (deterministic), then the real epilogue:
// one thread per 4 consecutive columns of the concatenated segment columns of a row.
template <int EPI>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs a) {
  constexpr bool kF16 = EPI != EPI_F32;  // partials at the output's precision
  const int c4 = a.ldp / 4;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)a.m * c4) return;
  const int row = (int)(gid / c4);
  int col = (int)(gid - (long)row * c4) * 4;
  const size_t plane = (size_t)a.m * a.ldp;
  const size_t p = (size_t)row * a.ldp + col;
  float4 v = load_part4<kF16>(a.part, p);
  for (int s = 1; s < a.splits; s++) {
    const float4 w = load_part4<kF16>(a.part, p + s * plane);
    v.x += w.x;
    v.y += w.y;
    v.z += w.z;
    v.w += w.w;
  }
  int si = 0;
  while (si < a.nseg - 1 && col >= a.seg[si].n) col -= a.seg[si++].n;  // segment widths are multiples of 4
  const GemmSegment seg = a.seg[si];
  if (seg.bias) {
    const float4 b = *reinterpret_cast<const float4 *>(seg.bias + col);
    v.x += b.x;
    v.y += b.y;
    v.z += b.z;
    v.w += b.w;
  }
  const size_t o = (size_t)row * seg.ldo + seg.col0 + col;
  if constexpr (EPI == EPI_F16) {
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    *reinterpret_cast<half4v *>(reinterpret_cast<_Float16 *>(seg.out) + o) =
        half4v{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  } else if constexpr (EPI == EPI_F32) {
    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(seg.out) + o) = v;
  } else {  // EPI_RESID: x += f16(acc)
    float4 *x = reinterpret_cast<float4 *>(reinterpret_cast<float *>(seg.out) + o);
    const float4 old = *x;
    *x = float4{old.x + (float)(_Float16)v.x, old.y + (float)(_Float16)v.y, old.z + (float)(_Float16)v.z,
                old.w + (float)(_Float16)v.w};
  }
}

// The same for rows of 256*V columns, one wave per row: lane l holds columns 256j + 4l ..
// +3 (j < V), the layout and summation order of the RMSNorm kernels (rmsnorm_vec_kernel),
// so the normed rows equal theirs on the updated residual bit for bit, and the row's sum
// of squares needs no workgroup barrier.
template <int V>
__global__ __launch_bounds__(256) void split_reduce_norm_vec_kernel(GemmArgs a) {
  typedef _Float16 half4v __attribute__((ext_vector_type(4)));
  constexpr int D = 256 * V;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.m) return;
  const GemmSegment seg = a.seg[0];
  const size_t plane = (size_t)a.m * a.ldp;
  const size_t p = (size_t)row * a.ldp;  // f16 partials (a residual GEMM's output is f16)
  float *x = reinterpret_cast<float *>(seg.out) + (size_t)row * seg.ldo;
  // every load before the first store (loads and stores retire in issue order)
  float4 v[V], nw[V], old[V];
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int c = 256 * j + 4 * lane;
    nw[j] = *reinterpret_cast<const float4 *>(a.norm_w + c);
    v[j] = load_part4<true>(a.part, p + c);
    old[j] = *reinterpret_cast<const float4 *>(x + c);
  }
  for (int sp = 1; sp < a.splits; sp++) {
    float4 w[V];
#pragma unroll
    for (int j = 0; j < V; j++) w[j] = load_part4<true>(a.part, p + sp * plane + 256 * j + 4 * lane);
#pragma unroll
    for (int j = 0; j < V; j++) {
      v[j].x += w[j].x;
      v[j].y += w[j].y;
      v[j].z += w[j].z;
      v[j].w += w[j].w;
    }
  }
  if (seg.bias) {
#pragma unroll
    for (int j = 0; j < V; j++) {
      const float4 b = *reinterpret_cast<const float4 *>(seg.bias + 256 * j + 4 * lane);
      v[j].x += b.x;
      v[j].y += b.y;
      v[j].z += b.z;
      v[j].w += b.w;
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const float4 nx = float4{old[j].x + (float)(_Float16)v[j].x, old[j].y + (float)(_Float16)v[j].y,
                             old[j].z + (float)(_Float16)v[j].z, old[j].w + (float)(_Float16)v[j].w};
    *reinterpret_cast<float4 *>(x + 256 * j + 4 * lane) = nx;
    v[j] = nx;
  }
#pragma unroll
  for (int j = 0; j < V; j++) ss = rms_sumsq4(v[j], ss);
  const float scale = rms_scale(rms_wave_sum(ss), D, a.norm_eps);
  _Float16 *out = reinterpret_cast<_Float16 *>(a.norm_out) + (size_t)row * D;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int c = 256 * j + 4 * lane;
    *reinterpret_cast<rms_half4 *>(out + c) = rms_out4(v[j], scale, nw[j]);
    if (a.norm_x16)
      *reinterpret_cast<half4v *>(reinterpret_cast<_Float16 *>(a.norm_x16) + (size_t)row * D + c) =
          half4v{(_Float16)v[j].x, (_Float16)v[j].y, (_Float16)v[j].z, (_Float16)v[j].w};
  }
}

// K-split reduction of an EPI_RESID GEMM fused with the RMSNorm of the rows it updates:
// one workgroup per row holding its V*1024 columns in registers. x += f16(partials summed
// in split order (+ bias)), as split_reduce_kernel does, then norm_out = f16(x * scale *
// norm_w) with scale = 1 / sqrt(mean(x^2) + eps), and norm_x16 = f16(x) when set.
template <int V>
__global__ __launch_bounds__(256) void split_reduce_norm_kernel(GemmArgs a) {
  typedef _Float16 half4v __attribute__((ext_vector_type(4)));
  const int row = blockIdx.x, tid = threadIdx.x;
  const GemmSegment seg = a.seg[0];
  const int n4 = seg.n / 4;
  const size_t plane = (size_t)a.m * a.ldp;
  const size_t p = (size_t)row * a.ldp;  // f16 partials (a residual GEMM's output is f16)
  float *x = reinterpret_cast<float *>(seg.out) + (size_t)row * seg.ldo;
  // the norm weights are loaded first: loaded between the stores at the end, each load
  // would wait for the stores before it (loads and stores retire in issue order)
  float4 xv[V], nw[V];
#pragma unroll
  for (int j = 0; j < V; j++) nw[j] = *reinterpret_cast<const float4 *>(a.norm_w + 4 * min(tid + 256 * j, n4 - 1));
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int c4 = tid + 256 * j;
    xv[j] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if (c4 >= n4) continue;
    float4 v = load_part4<true>(a.part, p + 4 * c4);
    for (int sp = 1; sp < a.splits; sp++) {
      const float4 w = load_part4<true>(a.part, p + sp * plane + 4 * c4);
      v.x += w.x;
      v.y += w.y;
      v.z += w.z;
      v.w += w.w;
    }
    if (seg.bias) {
      const float4 b = *reinterpret_cast<const float4 *>(seg.bias + 4 * c4);
      v.x += b.x;
      v.y += b.y;
      v.z += b.z;
      v.w += b.w;
    }
    const float4 old = *reinterpret_cast<const float4 *>(x + 4 * c4);
    const float4 nx = float4{old.x + (float)(_Float16)v.x, old.y + (float)(_Float16)v.y,
                             old.z + (float)(_Float16)v.z, old.w + (float)(_Float16)v.w};
    *reinterpret_cast<float4 *>(x + 4 * c4) = nx;
    xv[j] = nx;
    ss += nx.x * nx.x + nx.y * nx.y + nx.z * nx.z + nx.w * nx.w;
  }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) ss += __shfl_xor(ss, sh, 64);
  __shared__ float red[4];
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
  const float scale = 1.0f / sqrtf(ss / (float)seg.n + a.norm_eps);
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int c4 = tid + 256 * j;
    if (c4 >= n4) continue;
    const float4 w = nw[j];
    const float4 nx = xv[j];
    *reinterpret_cast<half4v *>(reinterpret_cast<_Float16 *>(a.norm_out) + (size_t)row * seg.n + 4 * c4) =
        half4v{(_Float16)(nx.x * scale * w.x), (_Float16)(nx.y * scale * w.y), (_Float16)(nx.z * scale * w.z),
               (_Float16)(nx.w * scale * w.w)};
    if (a.norm_x16)
      *reinterpret_cast<half4v *>(reinterpret_cast<_Float16 *>(a.norm_x16) + (size_t)row * seg.n + 4 * c4) =
          half4v{(_Float16)nx.x, (_Float16)nx.y, (_Float16)nx.z, (_Float16)nx.w};
  }
}

// GEMV for MT <= 4 tokens (decode, the last-token LM head): HBM-bound, so no MFMA and
// no LDS staging of the weights. One wave per 32-row panel reads the panel's records
// (lane l: quant bytes at 16*l, its row's two scales) U stages at a time and, in the
// order of logits_f16_output (kernels/prefill.cl:269-308), sums each block's x*(q-8)
// in f32 (exact f16 q-8 products, v_dot2_f32_f16, against x held in LDS) before one
// multiply by the block's d; the two half-waves of a row combine at the end. x beyond
// K is zero in LDS, so the odd-block half stage adds nothing.
constexpr int kGemvMaxXBytes = 64 * 1024;

template <int MT, int EPI>
__global__ __launch_bounds__(256) void gemv_q4_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // [MT][kpad]
  constexpr int U = 8;  // stages in flight per wave
  const int nb = a.k >> 5, nst = (nb + 1) >> 1, kpad = nst * 64;
  for (int i = threadIdx.x; i < MT * kpad / 8; i += blockDim.x) {
    const int t = i / (kpad / 8), c = (i % (kpad / 8)) * 8;
    half8 v = half8{0, 0, 0, 0, 0, 0, 0, 0};
    if (t < a.m && c < a.k) v = *reinterpret_cast<const half8 *>(a.x + (size_t)t * a.ldx + c);  // k % 32 == 0
    *reinterpret_cast<half8 *>(xs + t * kpad + c) = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  int p = blockIdx.x * 4 + (threadIdx.x >> 6);  // panel across the segments
  int si = 0;
  for (; si < a.nseg; si++) {
    const int np = (a.seg[si].n + 31) / 32;
    if (p < np) break;
    p -= np;
  }
  if (si >= a.nseg) return;  // whole waves past the last panel (no barrier below)
  const GemmSegment seg = a.seg[si];
  const uint8_t *rec0 = seg.panels + (size_t)p * nst * kQ4PanelRecord;
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = 0.0f;
  for (int s0 = 0; s0 < nst; s0 += U) {
    uint4 qv[U];
    uint32_t sw[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int st = min(s0 + u, nst - 1);  // repeats the last stage, not used below
      qv[u] = *reinterpret_cast<const uint4 *>(rec0 + (size_t)st * kQ4PanelRecord + 16 * lane);
      sw[u] = *reinterpret_cast<const uint32_t *>(rec0 + (size_t)st * kQ4PanelRecord + 1024 + 4 * r);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (s0 + u >= nst) break;
      const int kb = (s0 + u) * 64;
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const uint32_t lo = b ? qv[u].z : qv[u].x, hi = b ? qv[u].w : qv[u].y;
        const float d = (float)as_h2(sw[u])[b];
        half2v w[8];  // q-8 of elements 8h .. 8h+7, then 16+8h .. 16+8h+7 of block b
        dq4_raw<false>(lo & 0x0F0F0F0Fu, w[0], w[1]);
        dq4_raw<false>(hi & 0x0F0F0F0Fu, w[2], w[3]);
        dq4_raw<true>(lo & 0xF0F0F0F0u, w[4], w[5]);
        dq4_raw<true>(hi & 0xF0F0F0F0u, w[6], w[7]);
        // the reference's order: the block's sum of x*(q-8), then one multiply by d
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const _Float16 *xr = xs + t * kpad + kb + 32 * b + 8 * h;
          const half8 xl = *reinterpret_cast<const half8 *>(xr);
          const half8 xh = *reinterpret_cast<const half8 *>(xr + 16);
          float bs = 0.0f;
#pragma unroll
          for (int j = 0; j < 4; j++) {
            bs = __builtin_amdgcn_fdot2(w[j], half2v{xl[2 * j], xl[2 * j + 1]}, bs, false);
            bs = __builtin_amdgcn_fdot2(w[4 + j], half2v{xh[2 * j], xh[2 * j + 1]}, bs, false);
          }
          acc[t] += bs * d;
        }
      }
    }
  }
  const int row = p * 32 + r;
#pragma unroll
  for (int t = 0; t < MT; t++) {
    float v = acc[t] + __shfl_xor(acc[t], 32, 64);
    if (h || t >= a.m || row >= seg.n) continue;
    if (seg.bias) v += seg.bias[row];
    const size_t o = (size_t)t * seg.ldo + seg.col0 + row;
    if constexpr (EPI == EPI_F16) reinterpret_cast<_Float16 *>(seg.out)[o] = (_Float16)v;
    else if constexpr (EPI == EPI_F32) reinterpret_cast<float *>(seg.out)[o] = v;
    else {  // EPI_RESID
      float *x = reinterpret_cast<float *>(seg.out) + o;
      *x = *x + (float)(_Float16)v;
    }
  }
}

template <int MT>
int32_t launch_gemv_mt(const GemmArgs &a, hipStream_t s, LaunchStamp st) {
  int panels = 0;
  for (int i = 0; i < a.nseg; i++) panels += (a.seg[i].n + 31) / 32;
  const int kpad = ((a.k / 32 + 1) / 2) * 64;
  const size_t lds = (size_t)MT * kpad * 2;
  const dim3 grid((unsigned)((panels + 3) / 4)), block(256);
  switch (a.epi) {
    case EPI_F16: launch_stamped(gemv_q4_kernel<MT, EPI_F16>, grid, block, lds, s, st.start, st.stop, a); break;
    case EPI_F32: launch_stamped(gemv_q4_kernel<MT, EPI_F32>, grid, block, lds, s, st.start, st.stop, a); break;
    default: launch_stamped(gemv_q4_kernel<MT, EPI_RESID>, grid, block, lds, s, st.start, st.stop, a); break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "gemv_q4_kernel launch");
}

// The GEMV handles up to 4 tokens with f16/f32/residual epilogues and x in 64 KB of LDS.
int gemv_tokens(int m) { return m == 1 ? 1 : m == 2 ? 2 : 4; }
bool gemv_fits(const GemmArgs &a) {
  const int kpad = ((a.k / 32 + 1) / 2) * 64;
  return a.m <= 4 && (a.epi == EPI_F16 || a.epi == EPI_F32 || a.epi == EPI_RESID) &&
         (size_t)gemv_tokens(a.m) * kpad * 2 <= (size_t)kGemvMaxXBytes && a.ldx % 8 == 0;
}

int32_t launch_gemv(const GemmArgs &a, hipStream_t s, LaunchStamp st) {
  if (a.m == 1) return launch_gemv_mt<1>(a, s, st);
  if (a.m == 2) return launch_gemv_mt<2>(a, s, st);
  return launch_gemv_mt<4>(a, s, st);
}

// Splits of nst stages into equal runs with none empty: returns the split count and
// the stages per split.
int normalize_splits(int k, int splits, int *split_stages) {
  const int nst = (k / 32 + 1) / 2;
  splits = std::max(1, std::min(splits, nst));
  const int per = (nst + splits - 1) / splits;
  *split_stages = per;
  return (nst + per - 1) / per;
}

// Workgroups of kernel K the GPU holds at once (a multiple of the XCD count), measured
// once per kernel.
template <auto K>
int resident_wgs(int threads) {
  static const int r = [threads] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K, threads, 0) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    return n * (device_cu_count() / kXcds) * kXcds;
  }();
  return r;
}

template <int FM, int FN, int NS = 3, int KSPLIT = 1, int WM = 1>
int32_t launch_cfg(const GemmArgs &args, hipStream_t s, LaunchStamp st) {
  constexpr int BM = 32 * FM * WM;
  constexpr int BN = 32 * FN * (4 / WM);
  GemmArgs a = args;
  const int out_bn = (a.epi == EPI_SWIGLU) ? BN / 2 : BN;
  a.tiles_n = 0;
  for (int i = 0; i < a.nseg; i++) a.tiles_n += (a.seg[i].n + out_bn - 1) / out_bn;
  a.tiles_m = (a.m + BM - 1) / BM;
  a.group_m = 4;
  if (a.epi != EPI_PART || a.splits < 1) a.splits = 1;
  a.splits = normalize_splits(a.k, a.splits, &a.split_stages);
  // Persistent launch when the tiles outnumber the workgroups the GPU holds at once and
  // the kernel can chain tiles: one grid of resident workgroups, a multiple of the XCD
  // count, each running every (grid / XCDs)-th tile of its XCD's range.
  const int nwork = a.tiles_m * a.tiles_n * a.splits;
  const int nb = a.k / 32, nst = (nb + 1) / 2;
  const bool chain = KSPLIT == 1 && WM == 1 && a.splits == 1 && a.nseg == 1 && nb % 2 == 0 && nst % NS == 0 &&
                     (a.epi == EPI_SWIGLU || a.epi == EPI_F16);
  const dim3 block(256 * KSPLIT);
  auto go = [&](auto kern, int resident) {
    a.persist = chain && resident >= kXcds && nwork > resident;
    launch_stamped(kern, dim3(a.persist ? resident : nwork), block, 0, s, st.start, st.stop, a);
  };
  switch (a.epi) {
    case EPI_F16: {
      constexpr auto k = gemm_q4_kernel<FM, FN, NS, EPI_F16, KSPLIT, WM>;
      go(k, resident_wgs<k>(256 * KSPLIT));
      break;
    }
    case EPI_F32: {
      constexpr auto k = gemm_q4_kernel<FM, FN, NS, EPI_F32, KSPLIT, WM>;
      go(k, resident_wgs<k>(256 * KSPLIT));
      break;
    }
    case EPI_RESID: {
      constexpr auto k = gemm_q4_kernel<FM, FN, NS, EPI_RESID, KSPLIT, WM>;
      go(k, resident_wgs<k>(256 * KSPLIT));
      break;
    }
    case EPI_SWIGLU:
      if constexpr (FN % 2 == 0) {
        constexpr auto k = gemm_q4_kernel<FM, FN, NS, EPI_SWIGLU, KSPLIT, WM>;
        go(k, resident_wgs<k>(256 * KSPLIT));
        break;
      } else {
        return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "SwiGLU tiles pair gate and up fragments (even FN)");
      }
    case EPI_PART: go(gemm_q4_kernel<FM, FN, NS, EPI_PART, KSPLIT, WM>, 0); break;
    case EPI_ROPE:
      if constexpr (WM == 1 && FN == 1) {
        go(gemm_q4_kernel<FM, FN, NS, EPI_ROPE, KSPLIT, WM>, 0);
        break;
      } else {
        return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "the RoPE epilogue runs on 128-column tiles");
      }
    default: return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "unknown GEMM epilogue");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "gemm_q4_kernel launch");
}

}  // namespace

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

namespace {

// Tile configurations the planner chooses from (all with 3 ring slots): token rows,
// weight rows (128 * FN), K parts inside the workgroup, and the workgroups one CU holds
// at once (registers and LDS of the compiled kernels).
enum GemmCfg : int { kT32, kT32K2, kT64, kT64K2, kT128, kT128K2, kN32, kN32K2, kN32K4, kN64, kN64K2, kNumCfg };
constexpr int kCfgRows[kNumCfg] = {32, 32, 64, 64, 128, 128, 32, 32, 32, 64, 64};
constexpr int kCfgCols[kNumCfg] = {256, 256, 256, 256, 256, 256, 128, 128, 128, 128, 128};
constexpr int kCfgKsplit[kNumCfg] = {1, 2, 1, 2, 1, 2, 1, 2, 4, 1, 2};
constexpr int kCfgOcc[kNumCfg] = {4, 2, 3, 1, 2, 1, 6, 3, 1, 4, 2};

// Cost model fitted to 1980 measurements on MI355X (clock ramped) of six layer shapes
// (N x K = 2048 x 1536, 1536 x 1536, 8960 x 1536, 1536 x 8960, 256 x 1536, 3072 x 3072)
// at M = 128 .. 3071 and S = 1 .. 8, weighted to M = 512 and 2048 (median error 6 %;
// its picks sum to within 1.6 % of the measured best): per workgroup, fixed +
// stages x per-stage (us). The busiest CU runs ceil(workgroups / CUs) of them in
// rounds of up to kCfgOcc at once, the per-stage cost rising with each workgroup that
// shares the CU. The time is floored by the operand bytes every workgroup pulls into
// LDS over the chip's fetch rate; a K split adds the reduction kernel.
constexpr double kCostFixed[kNumCfg] = {3.955, 4.070, 5.297, 5.459, 7.302, 9.483, 3.286, 3.221, 3.773, 4.174, 4.080};
constexpr double kCostStage[kNumCfg] = {0.446, 0.754, 0.518, 0.952, 0.829, 1.507, 0.287, 0.454, 0.790, 0.321, 0.566};
constexpr double kCostShared[kNumCfg] = {0.264, 0.474, 0.418, 0.0, 0.614, 0.0, 0.144, 0.289, 0.0, 0.212, 0.432};
constexpr double kFetchMBperUs = 10.968;
constexpr double kReduceFixed = 4.982, kReducePerMB = 0.1744;

struct GemmPlan {
  int cfg;
  int splits;  // K splits across workgroups (1: the epilogue runs in the GEMM)
};

int seg_cols(const GemmArgs &a) {
  int n = 0;
  for (int i = 0; i < a.nseg; i++) n += a.seg[i].n;
  return n;
}

// Bytes per stored K-split partial: f16 for f16-rounded outputs, f32 for an f32 output.
int part_elem_bytes(const GemmArgs &a) { return a.epi == EPI_F32 ? 4 : 2; }

double predict_us(const GemmArgs &a, int cfg, int splits, int cus) {
  int per;
  splits = normalize_splits(a.k, splits, &per);
  const int out_bn = a.epi == EPI_SWIGLU ? kCfgCols[cfg] / 2 : kCfgCols[cfg];
  long tn = 0;
  for (int i = 0; i < a.nseg; i++) tn += (a.seg[i].n + out_bn - 1) / out_bn;
  const long wgs = (long)(a.m + kCfgRows[cfg] - 1) / kCfgRows[cfg] * tn * splits;
  const int stages = (per + kCfgKsplit[cfg] - 1) / kCfgKsplit[cfg];
  const long load = (wgs + cus - 1) / cus;  // workgroups on the busiest CU
  const int occ = kCfgOcc[cfg];
  auto round_us = [&](long c) { return kCostFixed[cfg] + stages * (kCostStage[cfg] + (c - 1) * kCostShared[cfg]); };
  double t = (load / occ) * round_us(occ) + (load % occ ? round_us(load % occ) : 0.0);
  t = std::max(t, (double)wgs * per * (kCfgRows[cfg] * 128.0 + kCfgCols[cfg] * 36.0) / 1e6 / kFetchMBperUs);
  if (splits > 1) {
    const double mn = (double)a.m * seg_cols(a);
    const double out_bytes = a.epi == EPI_RESID ? 8 : a.epi == EPI_F32 ? 4 : 2;
    t += kReduceFixed + kReducePerMB * (splits * mn * part_elem_bytes(a) + mn * out_bytes) / 1e6;
  }
  return t;
}

// A K split needs a splittable epilogue, 4-column aligned segments and room for the
// partials (unless `unbounded`, used to size the workspace).
bool can_split(const GemmArgs &a, int splits, bool unbounded) {
  if (a.epi != EPI_F16 && a.epi != EPI_F32 && a.epi != EPI_RESID) return false;
  for (int i = 0; i < a.nseg; i++)
    if (a.seg[i].n % 4 || a.seg[i].ldo % 4 || a.seg[i].col0 % 4) return false;
  if (unbounded) return true;
  return a.part && (size_t)splits * a.m * seg_cols(a) * part_elem_bytes(a) <= a.part_bytes;
}

// The RoPE epilogue runs on 128-column tiles (one wave per 32 columns: its cos/sin,
// partner and output registers fit beside the accumulators without spills).
bool rope_tile_fits(int cfg) { return kCfgCols[cfg] == 128; }

GemmPlan plan_gemm_uncached(const GemmArgs &a, bool unbounded) {
  const int cus = device_cu_count();
  if (a.epi == EPI_SWIGLU) {
    // measured rule: 128 x 256 tiles once they fill the GPU four times over
    int ntn = 0;
    for (int i = 0; i < a.nseg; i++) ntn += (a.seg[i].n + 127) / 128;
    const bool ks = a.k >= 512;
    if (a.m <= 32) return {ks && ntn < 2 * cus ? kT32K2 : kT32, 1};
    if (a.m > 64 && ntn * ((a.m + 127) / 128) >= 4 * cus) return {kT128, 1};
    return {ks && ntn * ((a.m + 63) / 64) < 2 * cus ? kT64K2 : kT64, 1};
  }
  GemmPlan best1{kT64, 1}, bestn{kT64, 1};
  double t1 = 1e30, tn = 1e30;
  static const int kSplits[] = {1, 2, 3, 4, 5, 6, 7, 8};
  for (int cfg = 0; cfg < kNumCfg; cfg++) {
    if (kCfgKsplit[cfg] > 1 && a.k < 256 * kCfgKsplit[cfg]) continue;  // at least four stages per part
    if (kCfgRows[cfg] > 32 && a.m <= 32) continue;
    if (a.epi == EPI_ROPE && !rope_tile_fits(cfg)) continue;
    for (int sp : kSplits) {
      int per;
      if (normalize_splits(a.k, sp, &per) != sp) continue;
      if (sp > 1 && !can_split(a, sp, unbounded)) continue;
      const double t = predict_us(a, cfg, sp, cus);
      if (sp == 1 && t < t1) { t1 = t; best1 = {cfg, 1}; }
      if (sp > 1 && t < tn) { tn = t; bestn = {cfg, sp}; }
    }
  }
  return tn < t1 ? bestn : best1;
}

// Recent plans per host thread, keyed by everything the planner reads: the shape, the
// epilogue, segment alignment (K splits need 4-column alignment), the partial workspace
// and the CU count.
GemmPlan plan_gemm(const GemmArgs &a, bool unbounded) {
  constexpr int kKey = 16;
  struct Entry {
    long long key[kKey];
    GemmPlan plan;
  };
  constexpr int kEntries = 16;
  thread_local Entry cache[kEntries];
  thread_local int used = 0, next = 0;
  long long key[kKey] = {a.m, a.k, a.epi, a.nseg, unbounded, a.part != nullptr, (long long)a.part_bytes,
                         device_cu_count()};
  for (int i = 0; i < a.nseg; i++) {
    key[8 + 2 * i] = a.seg[i].n;
    key[9 + 2 * i] = (a.seg[i].ldo | a.seg[i].col0) & 3;
  }
  for (int i = 0; i < used; i++)
    if (std::equal(key, key + kKey, cache[i].key)) return cache[i].plan;
  const GemmPlan p = plan_gemm_uncached(a, unbounded);
  std::copy(key, key + kKey, cache[next].key);
  cache[next].plan = p;
  next = (next + 1) % kEntries;
  used = std::min(used + 1, kEntries);
  return p;
}

int32_t launch_plan(const GemmArgs &a, int cfg, hipStream_t s, LaunchStamp st) {
  switch (cfg) {
    case kT32: return launch_cfg<1, 2, 3, 1>(a, s, st);
    case kT32K2: return launch_cfg<1, 2, 3, 2>(a, s, st);
    case kT64: return launch_cfg<2, 2, 3, 1>(a, s, st);
    case kT64K2: return launch_cfg<2, 2, 3, 2>(a, s, st);
    case kT128: return launch_cfg<4, 2, 3, 1>(a, s, st);
    case kT128K2: return launch_cfg<4, 2, 3, 2>(a, s, st);
    case kN32: return launch_cfg<1, 1, 3, 1>(a, s, st);
    case kN32K2: return launch_cfg<1, 1, 3, 2>(a, s, st);
    case kN32K4: return launch_cfg<1, 1, 3, 4>(a, s, st);
    case kN64: return launch_cfg<2, 1, 3, 1>(a, s, st);
    default: return launch_cfg<2, 1, 3, 2>(a, s, st);
  }
}

}  // namespace

size_t gemm_q4_0_workspace_bytes(const GemmArgs &a) {
  if (a.m <= 0 || a.k <= 0 || a.k % 32 != 0 || a.nseg < 1 || a.nseg > 3) return 0;
  if (gemv_fits(a)) return 0;
  const GemmPlan p = plan_gemm(a, true);
  return p.splits > 1 ? (size_t)p.splits * a.m * seg_cols(a) * part_elem_bytes(a) : 0;
}

int32_t launch_gemm_q4_0(const GemmArgs &a, hipStream_t s, bool *norm_done, const LaunchStamp *stamp) {
  if (norm_done) *norm_done = false;
  if (a.m <= 0) return SULIMO_HIP_OK;
  if (a.k <= 0 || a.k % 32 != 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM k must be a positive multiple of 32");
  if (a.ldx < a.k) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM activation row stride below k");
  if (a.nseg < 1 || a.nseg > 3) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM needs 1..3 segments");
  if (a.epi == EPI_PART) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM epilogue must be a final one");
  // Buffer offsets are 32-bit and stay below 2^31 (larger offsets mark rows past the end).
  const uint64_t lim = 1ull << 31;
  if ((uint64_t)a.m * (uint64_t)a.ldx * 2u >= lim)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM activations exceed 2 GiB");
  for (int i = 0; i < a.nseg; i++) {
    if (a.seg[i].n <= 0 || !a.seg[i].panels)
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM segments need rows and a panel array");
    if (q4_panel_bytes(a.seg[i].n, a.k, a.epi == EPI_SWIGLU) >= lim)
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM weight matrix exceeds 2 GiB");
  }
  if (a.epi == EPI_SWIGLU && a.nseg != 1)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "SwiGLU GEMM takes one segment");
  if (a.epi == EPI_ROPE) {
    const GemmRope &r = a.rope;
    const int hd = r.head_dim;
    if (a.nseg != 3 || (hd != 64 && hd != 128))
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM takes q, k, v segments of head_dim 64 or 128");
    if (!r.cs || !r.k_dst || !r.v_dst || r.wrap <= 0 || r.slot0 < 0 || (r.mode != 0 && r.mode != 1))
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM needs a cos/sin table, K/V targets and a ring size");
    for (int i = 0; i < 3; i++)
      if (a.seg[i].n % hd) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM segments must hold whole heads");
    if (!a.seg[0].out || a.seg[0].ldo % 4 || a.seg[0].col0 % 4 || ((uintptr_t)a.seg[0].out & 7))
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM q output must be 4-element aligned");
    if (a.seg[1].n != a.seg[2].n || r.row_bytes != a.seg[1].n / 32 * 34)
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM K/V rows must be the k and v widths in Q8_0");
    if (r.win.k && (!r.win.vt || r.win.j0 < 0 || r.win.vst % 4 || ((uintptr_t)r.win.vt & 7) || ((uintptr_t)r.win.k & 7)))
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "RoPE GEMM window target misaligned");
  }
  const LaunchStamp st = stamp ? *stamp : LaunchStamp{};
  if (gemv_fits(a)) return launch_gemv(a, s, st);
  const GemmPlan p = plan_gemm(a, false);
  if (p.splits == 1) return launch_plan(a, p.cfg, s, st);
  // K split: partials per split, then their sum in split order with the epilogue
  GemmArgs g = a;
  g.epi = EPI_PART;
  g.splits = p.splits;
  g.ldp = seg_cols(a);
  g.part_f16 = part_elem_bytes(a) == 2;
  int32_t rc = launch_plan(g, p.cfg, s, LaunchStamp{st.start, nullptr});
  if (rc) return rc;
  GemmArgs r = g;
  r.epi = a.epi;
  r.splits = normalize_splits(a.k, p.splits, &r.split_stages);
  // the residual update and the RMSNorm of its rows in one pass, rows up to 8192 wide
  const int v4 = (a.seg[0].n / 4 + 255) / 256;
  if (norm_done && a.epi == EPI_RESID && a.norm_w && a.norm_out && a.nseg == 1 && a.seg[0].col0 == 0 && v4 <= 8) {
    const int n = a.seg[0].n;
    if (n % 256 == 0 && n <= 256 * 16) {  // one wave per row
      const dim3 grid((unsigned)((a.m + 3) / 4)), block(256);
      switch (n / 256) {
#define SULIMO_SRN_CASE(V) \
  case V: launch_stamped(split_reduce_norm_vec_kernel<V>, grid, block, 0, s, nullptr, st.stop, r); break;
        SULIMO_SRN_CASE(1) SULIMO_SRN_CASE(2) SULIMO_SRN_CASE(3) SULIMO_SRN_CASE(4) SULIMO_SRN_CASE(5)
        SULIMO_SRN_CASE(6) SULIMO_SRN_CASE(7) SULIMO_SRN_CASE(8) SULIMO_SRN_CASE(9) SULIMO_SRN_CASE(10)
        SULIMO_SRN_CASE(11) SULIMO_SRN_CASE(12) SULIMO_SRN_CASE(13) SULIMO_SRN_CASE(14) SULIMO_SRN_CASE(15)
        SULIMO_SRN_CASE(16)
#undef SULIMO_SRN_CASE
      }
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return hip_fail(e, "split_reduce_norm_vec_kernel launch");
      *norm_done = true;
      return SULIMO_HIP_OK;
    }
    const dim3 grid((unsigned)a.m), block(256);
    switch (v4) {
      case 1: launch_stamped(split_reduce_norm_kernel<1>, grid, block, 0, s, nullptr, st.stop, r); break;
      case 2: launch_stamped(split_reduce_norm_kernel<2>, grid, block, 0, s, nullptr, st.stop, r); break;
      case 3: launch_stamped(split_reduce_norm_kernel<3>, grid, block, 0, s, nullptr, st.stop, r); break;
      case 4: launch_stamped(split_reduce_norm_kernel<4>, grid, block, 0, s, nullptr, st.stop, r); break;
      default: launch_stamped(split_reduce_norm_kernel<8>, grid, block, 0, s, nullptr, st.stop, r); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "split_reduce_norm_kernel launch");
    *norm_done = true;
    return SULIMO_HIP_OK;
  }
  const long threads = (long)a.m * (r.ldp / 4);
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  switch (a.epi) {
    case EPI_F16: launch_stamped(split_reduce_kernel<EPI_F16>, grid, block, 0, s, nullptr, st.stop, r); break;
    case EPI_F32: launch_stamped(split_reduce_kernel<EPI_F32>, grid, block, 0, s, nullptr, st.stop, r); break;
    default: launch_stamped(split_reduce_kernel<EPI_RESID>, grid, block, 0, s, nullptr, st.stop, r); break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "split_reduce_kernel launch");
}

}  // namespace sulimo
