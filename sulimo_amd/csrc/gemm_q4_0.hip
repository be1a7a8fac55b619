// gemm_q4_0.hip - Q4_0 weight x f16 activation GEMM on gfx950 MFMA.
//
// Replaces kernels/gemm_q4_0.cl:13-130 (one work-item per output, no reuse).
// Y[t][j] = sum_k X[t][k] * W[j][k], W[j][32b+i] = (q-8) * d[j][b] (Q4_0 SoA,
// crates/sulimo-core/src/repack.rs:107-131), f32 accumulation, epilogue per use.
//
// One workgroup = 4 wave64s; tile BM tokens x BN weight rows (BN = 4 waves x 32*FN).
// k advances in stages of 64 (two Q4_0 blocks). The path is latency-bound unless
// several stages are in flight, so:
//  * X (activations) streams global -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging) into a ring of NS stage slots, NS-1 stages ahead of use. A slot is
//    BM rows x 128 bytes with the 16-byte chunk c of row r stored at slot position
//    c ^ ((r >> 1) & 7), which makes the MFMA A-fragment reads bank-conflict free.
//  * Each wave streams the raw Q4_0 bytes of its own 32*FN weight rows (8 bytes per
//    lane per block, plus the f16 scale) into registers PD stages ahead, and
//    dequantizes them straight into MFMA B operands: (1024+q) - 1032 exactly, then
//    * d (one rounding to f16). Every weight is dequantized once per workgroup and
//    reused for all BM rows.
//  * v_mfma_f32_32x32x16_f16, lane layout: lane l supplies A[row l%32][k 8*(l/32)..+7]
//    and B[k 8*(l/32)..+7][col l%32], and receives C[8*(r/4) + 4*(l/32) + r%4][l%32]
//    in accumulator register r. MFMA step s of a stage covers stage k 16s..16s+15:
//    block s/2, elements 16*(s%2) + 8*(l/32)..+7, i.e. the low (s even) or high
//    (s odd) nibbles of bytes 8*(l/32)..+7 of the block.
//  * One barrier per stage: wait for this stage's X slot (explicit vmcnt), barrier,
//    then refill the slot every wave finished reading in the previous stage.
#include <type_traits>

#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int kBK = 64;  // k per stage

template <int J>
using ic = std::integral_constant<int, J>;

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// Four nibbles packed one per byte (values 0..15) -> two half2 of (q-8)*d.
__device__ __forceinline__ void dq4(uint32_t nib, half2v d2, half2v &a, half2v &b) {
  const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
  // bytes [n0, 0x64, n1, 0x64] -> half2(1024+n0, 1024+n1), exact
  const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
  const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
  a = (as_h2(p0) - off) * d2;
  b = (as_h2(p1) - off) * d2;
}

// 8 bytes of one block row -> B operands of its low-nibble and high-nibble k-steps.
__device__ __forceinline__ void dq8(uint2 q, uint32_t d, half8 &lo, half8 &hi) {
  const half2v d2 = as_h2(d | (d << 16));
  half2v l0, l1, l2, l3, h0, h1, h2, h3;
  dq4(q.x & 0x0F0F0F0Fu, d2, l0, l1);
  dq4(q.y & 0x0F0F0F0Fu, d2, l2, l3);
  dq4((q.x >> 4) & 0x0F0F0F0Fu, d2, h0, h1);
  dq4((q.y >> 4) & 0x0F0F0F0Fu, d2, h2, h3);
  lo = half8{l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
  hi = half8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// s_waitcnt vmcnt(n) with expcnt and lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int FM, int FN, int kNS, int EPI>
__global__ __launch_bounds__(256) void gemm_q4_kernel(GemmArgs a) {
  constexpr int BM = 32 * FM;
  constexpr int BN = 128 * FN;                    // weight rows per tile (4 waves)
  constexpr bool kSwiglu = (EPI == EPI_SWIGLU);
  constexpr int OUT_BN = kSwiglu ? BN / 2 : BN;   // output columns per tile
  constexpr int NX = FM;                          // X DMA instructions per wave per stage
  constexpr int NQ = BN / 128;                    // quant DMA instructions per wave per stage
  constexpr int NSC = BN / 128;                   // scale DMA instructions per wave per stage
  constexpr int NDMA = NX + NQ + NSC;
  // LDS slot layout: X tile | quants [BN rows][2 blocks][16 B] | scales [BN rows][2 dwords]
  constexpr int X_BYTES = BM * kBK * 2;
  constexpr int Q_BYTES = BN * 32;
  constexpr int S_BYTES = BN * 8;
  constexpr int SLOT = X_BYTES + Q_BYTES + S_BYTES;
  static_assert(!kSwiglu || FN % 2 == 0, "SwiGLU pairs gate and up fragments in one wave");
  static_assert(BN % 128 == 0, "DMA split");

  __shared__ __attribute__((aligned(16))) char smem[kNS * SLOT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lg = lane >> 5;

  // --- tile -> (segment, first output column, first row) ---
  int tile_n = blockIdx.x;
  int si = 0;
  for (; si < a.nseg - 1; si++) {
    const int tn = (a.seg[si].n + OUT_BN - 1) / OUT_BN;
    if (tile_n < tn) break;
    tile_n -= tn;
  }
  const GemmSegment seg = a.seg[si];
  const int c0 = tile_n * OUT_BN;
  const int m0 = blockIdx.y * BM;
  const int nb = a.k >> 5;           // Q4_0 blocks per weight row
  const int nst = (nb + 1) >> 1;     // stages
  const size_t nscale = (size_t)seg.n * nb;  // scales of one weight matrix

  // Logical tile row L -> (weight matrix, row). Wave w's fragment f covers rows
  // w*32*FN + 32f .. +31; with SwiGLU its first FN/2 fragments are gate rows and the
  // rest up rows of the same output columns.
  auto map_row = [&](int L, const uint16_t *&sc, const uint8_t *&qu, bool &ok) -> int {
    sc = seg.scales;
    qu = seg.quants;
    int col;
    if constexpr (kSwiglu) {
      const int w = L / (32 * FN), f = (L % (32 * FN)) / 32, r = L & 31;
      const bool up = f >= FN / 2;
      col = c0 + w * 16 * FN + 32 * (up ? f - FN / 2 : f) + r;
      if (up) {
        sc = a.scales_up;
        qu = a.quants_up;
      }
    } else {
      col = c0 + L;
    }
    ok = col < seg.n;
    return ok ? col : 0;
  };

  // --- per-lane DMA sources ---
  // X: wave instruction i covers tile rows 8*(FM*wave+i) .. +7, chunk c of row r lands at
  // slot position c ^ ((r >> 1) & 7).
  const _Float16 *xsrc[NX];
  int xhalf[NX];
#pragma unroll
  for (int i = 0; i < NX; i++) {
    const int row = 8 * (FM * wave + i) + (lane >> 3);
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    int r = m0 + row;
    if (r >= a.m) r = a.m - 1;
    xsrc[i] = reinterpret_cast<const _Float16 *>(a.x) + (size_t)r * a.ldx + 8 * chunk;
    xhalf[i] = chunk >> 2;
  }
  // Quants: wave instruction i covers logical rows 32*(NQ*wave+i) + lane/2, block lane%2.
  const uint8_t *qsrc[NQ];
#pragma unroll
  for (int i = 0; i < NQ; i++) {
    const int L = 32 * (NQ * wave + i) + (lane >> 1);
    const uint16_t *sc;
    const uint8_t *qu;
    bool ok;
    const int row = map_row(L, sc, qu, ok);
    qsrc[i] = qu + ((size_t)row * nb + (lane & 1)) * 16;
  }
  // Scales: the two scales of a stage start at e = row*nb + 2*st, which is odd when nb is
  // odd; each row loads the two aligned dwords covering e .. e+1 (clamped to the array).
  const uint16_t *ssrc[NSC];
  int srow[NSC];
#pragma unroll
  for (int i = 0; i < NSC; i++) {
    const int L = 32 * (NSC * wave + i) + (lane >> 1);
    const uint16_t *sc;
    const uint8_t *qu;
    bool ok;
    srow[i] = map_row(L, sc, qu, ok);
    ssrc[i] = sc;
  }

  auto issue = [&](int st) {  // always NDMA instructions (stages past the end reload stage 0)
    const int sst = st < nst ? st : 0;
    char *slot = smem + (st % kNS) * SLOT;
#pragma unroll
    for (int i = 0; i < NX; i++) {
      // a chunk past K (odd block count) re-reads the stage's first block: its weights are 0
      const int kc = sst * kBK - ((sst * 2 + xhalf[i] < nb) ? 0 : 32);
      __builtin_amdgcn_global_load_lds((glb_void *)(xsrc[i] + kc),
                                       (lds_void *)(slot + 8 * (FM * wave + i) * kBK * 2), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NQ; i++) {
      const int blk = min(sst * 2 + (lane & 1), nb - 1) - (lane & 1);  // clamp the odd tail block
      __builtin_amdgcn_global_load_lds((glb_void *)(qsrc[i] + (size_t)blk * 16),
                                       (lds_void *)(slot + X_BYTES + 32 * (NQ * wave + i) * 32), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NSC; i++) {
      const size_t e = (size_t)srow[i] * nb + 2 * sst;
      size_t d = (e & ~(size_t)1) + 2 * (lane & 1);
      if (d + 2 > nscale) d = nscale - 2;  // never past the array (the value is then unused)
      __builtin_amdgcn_global_load_lds((glb_void *)(ssrc[i] + d),
                                       (lds_void *)(slot + X_BYTES + Q_BYTES + 32 * (NSC * wave + i) * 8), 4, 0, 0);
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int f = 0; f < FN; f++) acc[i][f] = floatx16{};

  // Per-lane weight rows of this wave's fragments (validity and scale parity).
  bool wok[FN];
  int epar[FN];
#pragma unroll
  for (int f = 0; f < FN; f++) {
    const uint16_t *sc;
    const uint8_t *qu;
    bool ok;
    const int row = map_row(wave * 32 * FN + 32 * f + l32, sc, qu, ok);
    wok[f] = ok;
    epar[f] = (row * nb) & 1;
  }

  auto read_a = [&](const _Float16 *xb, int s, half8 (&ao)[FM]) {
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int row = 32 * i + l32;
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

  // prologue: stages 0..NS-2 in flight
#pragma unroll
  for (int s = 0; s < kNS - 1; s++) issue(s);

  for (int st = 0; st < nst; st++) {
    __builtin_amdgcn_sched_barrier(0);
    // stage st was issued NS-1 stages ago, (NS-2)*NDMA DMA instructions after it
    wait_vmcnt<(kNS - 2) * NDMA>();
    // plain s_barrier: the slot is filled (vmcnt above) and the previous stage's LDS
    // reads were consumed by its MFMAs; a fenced barrier would drain every prefetch
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(st + kNS - 1);  // refills the slot read in stage st-1
    const char *slot = smem + (st % kNS) * SLOT;
    const _Float16 *xb = reinterpret_cast<const _Float16 *>(slot);
    // raw weights of this wave's fragments: 8 bytes per block, and the 4 scales around e
    uint2 q[FN][2];
    uint32_t dsc[FN][2];
#pragma unroll
    for (int f = 0; f < FN; f++) {
      const int L = wave * 32 * FN + 32 * f + l32;
#pragma unroll
      for (int b = 0; b < 2; b++)
        q[f][b] = *reinterpret_cast<const uint2 *>(slot + X_BYTES + L * 32 + b * 16 + 8 * lg);
      const uint2 w = *reinterpret_cast<const uint2 *>(slot + X_BYTES + Q_BYTES + L * 8);
      const uint32_t d0 = epar[f] ? (w.x >> 16) : (w.x & 0xffff);
      const uint32_t d1 = epar[f] ? (w.y & 0xffff) : (w.x >> 16);
      dsc[f][0] = (wok[f] && st * 2 < nb) ? d0 : 0u;
      dsc[f][1] = (wok[f] && st * 2 + 1 < nb) ? d1 : 0u;
    }
    auto dequant_step = [&](int s, half8 (&bo)[FN]) {
      const int b = s >> 1;
#pragma unroll
      for (int f = 0; f < FN; f++) {
        const half2v d2 = as_h2(dsc[f][b] | (dsc[f][b] << 16));
        const uint2 qq = q[f][b];
        const uint32_t x0 = (s & 1) ? (qq.x >> 4) & 0x0F0F0F0Fu : qq.x & 0x0F0F0F0Fu;
        const uint32_t x1 = (s & 1) ? (qq.y >> 4) & 0x0F0F0F0Fu : qq.y & 0x0F0F0F0Fu;
        half2v p0, p1, p2, p3;
        dq4(x0, d2, p0, p1);
        dq4(x1, d2, p2, p3);
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
  }
  // no DMA may still be writing this workgroup's LDS when it exits
  wait_vmcnt<0>();

  // --- epilogue: acc register r of fragment (i, f) is C[8*(r/4) + 4*lg + r%4][l32] ---
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + 32 * i + 8 * (r >> 2) + 4 * lg + (r & 3);
      if (row >= a.m) continue;
      if constexpr (kSwiglu) {
#pragma unroll
        for (int f = 0; f < FN / 2; f++) {
          const int col = c0 + wave * 16 * FN + 32 * f + l32;
          if (col >= seg.n) continue;
          const float g = acc[i][f][r], u = acc[i][f + FN / 2][r];
          const float silu = g / (1.0f + __expf(-g));
          reinterpret_cast<_Float16 *>(seg.out)[(size_t)row * seg.ldo + seg.col0 + col] = (_Float16)(silu * u);
        }
      } else {
#pragma unroll
        for (int f = 0; f < FN; f++) {
          const int col = c0 + wave * 32 * FN + 32 * f + l32;
          if (col >= seg.n) continue;
          const size_t o = (size_t)row * seg.ldo + seg.col0 + col;
          const float v = acc[i][f][r];
          if constexpr (EPI == EPI_F16) {
            reinterpret_cast<_Float16 *>(seg.out)[o] = (_Float16)v;
          } else if constexpr (EPI == EPI_F32) {
            reinterpret_cast<float *>(seg.out)[o] = v;
          } else {  // EPI_RESID: x += f16(acc)
            float *xo = reinterpret_cast<float *>(seg.out) + o;
            *xo = *xo + (float)(_Float16)v;
          }
        }
      }
    }
  }
}

template <int FM, int FN, int NS = 3>
int32_t launch_cfg(const GemmArgs &a, hipStream_t s) {
  constexpr int BM = 32 * FM;
  constexpr int BN = 128 * FN;
  const int out_bn = (a.epi == EPI_SWIGLU) ? BN / 2 : BN;
  int tiles_n = 0;
  for (int i = 0; i < a.nseg; i++) tiles_n += (a.seg[i].n + out_bn - 1) / out_bn;
  const int tiles_m = (a.m + BM - 1) / BM;
  const dim3 grid(tiles_n, tiles_m), block(256);
  switch (a.epi) {
    case EPI_F16: hipLaunchKernelGGL((gemm_q4_kernel<FM, FN, NS, EPI_F16>), grid, block, 0, s, a); break;
    case EPI_F32: hipLaunchKernelGGL((gemm_q4_kernel<FM, FN, NS, EPI_F32>), grid, block, 0, s, a); break;
    case EPI_RESID: hipLaunchKernelGGL((gemm_q4_kernel<FM, FN, NS, EPI_RESID>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: hipLaunchKernelGGL((gemm_q4_kernel<FM, FN, NS, EPI_SWIGLU>), grid, block, 0, s, a); break;
    default: return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "unknown GEMM epilogue");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "gemm_q4_kernel launch");
}

}  // namespace

int32_t launch_gemm_q4_0(const GemmArgs &a, hipStream_t s) {
  if (a.m <= 0) return SULIMO_HIP_OK;
  if (a.k <= 0 || a.k % 32 != 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM k must be a positive multiple of 32");
  if (a.nseg < 1 || a.nseg > 3) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM needs 1..3 segments");
  for (int i = 0; i < a.nseg; i++)  // even row counts keep the scale DMA dword-aligned and in bounds
    if (a.seg[i].n <= 0 || a.seg[i].n % 2 != 0)
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM segments need a positive, even number of rows");
  if (a.epi == EPI_SWIGLU && a.nseg != 1)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "SwiGLU GEMM takes one segment");
  // Tile choice: each weight is dequantized once per workgroup and used for BM rows.
  if (a.m <= 32) return launch_cfg<1, 2>(a, s);   // 32 x 256
  if (a.m <= 64) return launch_cfg<2, 2>(a, s);   // 64 x 256
  return launch_cfg<4, 2>(a, s);                  // 128 x 256
}

}  // namespace sulimo
