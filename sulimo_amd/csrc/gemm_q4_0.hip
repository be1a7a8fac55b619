// gemm_q4_0.hip - Q4_0 weight x f16 activation GEMM on gfx950 MFMA.
//
// Replaces kernels/gemm_q4_0.cl:13-130 (one work-item per output, no reuse).
// Y[t][j] = sum_k X[t][k] * W[j][k], W[j][32b+i] = (q-8) * d[j][b] (Q4_0 SoA,
// crates/sulimo-core/src/repack.rs:107-131), f32 accumulation, epilogue per use.
//
// Structure (one workgroup = 4 wave64s, tile BM tokens x BN weight rows):
//  * k advances in stages of 128 (four Q4_0 blocks).
//  * The workgroup streams the stage's BN x 72 bytes of Q4_0 (16-byte quant
//    loads, four lanes per 64-byte row segment) from HBM, dequantizes each
//    weight once to f16 ((1024+q) - 1032 exactly, then * d, one rounding) and
//    writes the tile to LDS (double-buffered, one barrier per stage).
//  * Each wave owns a (16*MF) x (16*NF) sub-tile; its A fragments come straight
//    from global memory (16 bytes per lane), its B fragments from LDS (16 bytes
//    per lane, conflict-free 272-byte row pitch), and it issues MF*NF*4
//    v_mfma_f32_16x16x32_f16 per stage.
//  * MFMA lane layout (16x16x32): lane l supplies A[row l%16][8 k's of group l/16]
//    and B[8 k's of group l/16][col l%16]; it receives C[4*(l/16)+r][l%16], r<4.
//    Inside a stage the 32 k's of MFMA step s are, for lane group g, elements
//    8s..8s+7 of Q4_0 block g: the same permutation is applied to A and B, so
//    the contraction is unchanged.
#include "common.h"

namespace sulimo {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 128;           // k per stage (4 Q4_0 blocks)
constexpr int kWLD = kBK + 8;      // LDS row pitch (halves) of the dequantized W tile

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// Dequantize four nibbles packed one per byte (values 0..15) to two half2 of (q-8)*d.
__device__ __forceinline__ void dq4(uint32_t nib, half2v d2, half2v &a, half2v &b) {
  const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
  // bytes [n0, 0x64, n1, 0x64] -> half2(1024+n0, 1024+n1); exact.
  uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
  uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
  a = (as_h2(p0) - off) * d2;
  b = (as_h2(p1) - off) * d2;
}

template <int EPI>
struct EpiTraits {
  static constexpr bool kSwiglu = (EPI == EPI_SWIGLU);
};

// MF x NF fragments per wave, WM x WN waves per workgroup.
template <int MF, int NF, int WM, int WN, int EPI>
__global__ __launch_bounds__(256) void gemm_q4_kernel(GemmArgs a, int tiles_m) {
  static_assert(WM * WN == 4, "4 waves per workgroup");
  constexpr int BM = 16 * MF * WM;
  constexpr int BN = 16 * NF * WN;             // weight rows per workgroup tile
  constexpr int OUT_BN = EpiTraits<EPI>::kSwiglu ? BN / 2 : BN;  // output columns
  constexpr int CHUNKS = BN * 4 / 256;         // 16-byte quant chunks per thread per stage
  static_assert(CHUNKS >= 1, "BN too small");

  __shared__ __attribute__((aligned(16))) _Float16 ws[2][BN * kWLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l16 = lane & 15, lg = lane >> 4;

  // --- tile -> (segment, column block, row block) ---
  int tile_n = blockIdx.x;
  const int tile_m = blockIdx.y;
  int si = 0;
  for (; si < a.nseg - 1; si++) {
    int tn = (a.seg[si].n + OUT_BN - 1) / OUT_BN;
    if (tile_n < tn) break;
    tile_n -= tn;
  }
  const GemmSegment seg = a.seg[si];
  const int c0 = tile_n * OUT_BN;  // first output column of the tile (within the segment)
  const int m0 = tile_m * BM;
  const int K = a.k;
  const int nb = K >> 5;           // Q4_0 blocks per weight row
  const int nst = (K + kBK - 1) / kBK;

  // --- per-thread W chunk assignment: logical tile row L, block-in-stage j ---
  const uint8_t *qsrc[CHUNKS];
  const uint16_t *ssrc[CHUNKS];
  bool rvalid[CHUNKS];
  int lrow[CHUNKS], lblk[CHUNKS];
#pragma unroll
  for (int c = 0; c < CHUNKS; c++) {
    int ch = tid + 256 * c;
    int L = ch >> 2, j = ch & 3;
    lrow[c] = L;
    lblk[c] = j;
    int col;  // output column of this weight row
    const uint16_t *sc = seg.scales;
    const uint8_t *qu = seg.quants;
    if constexpr (EpiTraits<EPI>::kSwiglu) {
      int w = L / (16 * NF), f = (L % (16 * NF)) / 16, r = L & 15;
      bool up = f >= NF / 2;
      col = c0 + w * 8 * NF + 16 * (up ? f - NF / 2 : f) + r;
      if (up) {
        sc = a.scales_up;
        qu = a.quants_up;
      }
    } else {
      col = c0 + L;
    }
    rvalid[c] = col < seg.n;
    int row = rvalid[c] ? col : 0;
    qsrc[c] = qu + ((size_t)row * nb + j) * 16;
    ssrc[c] = sc + (size_t)row * nb + j;
  }

  uint4 wq[CHUNKS];
  uint16_t wsc[CHUNKS];
  auto load_w = [&](int st) {
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
      int blk = st * 4 + lblk[c];
      if (rvalid[c] && blk < nb) {
        wq[c] = *reinterpret_cast<const uint4 *>(qsrc[c] + (size_t)st * 64);
        wsc[c] = ssrc[c][st * 4];
      } else {
        wq[c] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
        wsc[c] = 0;
      }
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
      half2v d2 = as_h2((uint32_t)wsc[c] | ((uint32_t)wsc[c] << 16));
      uint32_t q[4] = {wq[c].x, wq[c].y, wq[c].z, wq[c].w};
      half2v lo[8], hi[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dq4(q[i] & 0x0F0F0F0Fu, d2, lo[2 * i], lo[2 * i + 1]);
        dq4((q[i] >> 4) & 0x0F0F0F0Fu, d2, hi[2 * i], hi[2 * i + 1]);
      }
      _Float16 *dst = &ws[buf][lrow[c] * kWLD + lblk[c] * 32];
      half8 v0 = {lo[0][0], lo[0][1], lo[1][0], lo[1][1], lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
      half8 v1 = {lo[4][0], lo[4][1], lo[5][0], lo[5][1], lo[6][0], lo[6][1], lo[7][0], lo[7][1]};
      half8 v2 = {hi[0][0], hi[0][1], hi[1][0], hi[1][1], hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
      half8 v3 = {hi[4][0], hi[4][1], hi[5][0], hi[5][1], hi[6][0], hi[6][1], hi[7][0], hi[7][1]};
      *reinterpret_cast<half8 *>(dst + 0) = v0;
      *reinterpret_cast<half8 *>(dst + 8) = v1;
      *reinterpret_cast<half8 *>(dst + 16) = v2;
      *reinterpret_cast<half8 *>(dst + 24) = v3;
    }
  };

  // --- A fragments: rows m0 + wm*16*MF + 16*i + l16, k = st*128 + 32*lg + 8*s ---
  const _Float16 *xrow[MF];
#pragma unroll
  for (int i = 0; i < MF; i++) {
    int r = m0 + wm * 16 * MF + 16 * i + l16;
    if (r >= a.m) r = a.m - 1;
    xrow[i] = reinterpret_cast<const _Float16 *>(a.x) + (size_t)r * a.ldx + 32 * lg;
  }
  half8 afr[MF][4];
  auto load_a = [&](int st, half8 (&dst)[MF][4]) {
    bool ok = (st * 4 + lg) < nb;
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
      for (int s = 0; s < 4; s++) {
        if (ok)
          dst[i][s] = *reinterpret_cast<const half8 *>(xrow[i] + (size_t)st * kBK + 8 * s);
        else
          dst[i][s] = half8{0, 0, 0, 0, 0, 0, 0, 0};
      }
  };

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; i++)
#pragma unroll
    for (int f = 0; f < NF; f++) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  load_w(0);
  load_a(0, afr);
  store_w(0);
  __syncthreads();

  for (int st = 0; st < nst; st++) {
    const int buf = st & 1;
    half8 anext[MF][4];
    const bool more = st + 1 < nst;
    if (more) {
      load_w(st + 1);
      load_a(st + 1, anext);
    }
    const _Float16 *wb = &ws[buf][(wn * 16 * NF + l16) * kWLD + 32 * lg];
#pragma unroll
    for (int s = 0; s < 4; s++) {
#pragma unroll
      for (int f = 0; f < NF; f++) {
        half8 b = *reinterpret_cast<const half8 *>(wb + f * 16 * kWLD + 8 * s);
#pragma unroll
        for (int i = 0; i < MF; i++)
          acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[i][s], b, acc[i][f], 0, 0, 0);
      }
    }
    if (more) {
      store_w(buf ^ 1);
#pragma unroll
      for (int i = 0; i < MF; i++)
#pragma unroll
        for (int s = 0; s < 4; s++) afr[i][s] = anext[i][s];
    }
    __syncthreads();
  }

  // --- epilogue: lane holds C[4*lg + r][l16] of each fragment ---
#pragma unroll
  for (int i = 0; i < MF; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = m0 + wm * 16 * MF + 16 * i + 4 * lg + r;
      if (row >= a.m) continue;
      if constexpr (EpiTraits<EPI>::kSwiglu) {
#pragma unroll
        for (int f = 0; f < NF / 2; f++) {
          const int col = c0 + wn * 8 * NF + 16 * f + l16;
          if (col >= seg.n) continue;
          float g = acc[i][f][r], u = acc[i][f + NF / 2][r];
          float silu = g / (1.0f + __expf(-g));
          reinterpret_cast<_Float16 *>(seg.out)[(size_t)row * seg.ldo + seg.col0 + col] =
              (_Float16)(silu * u);
        }
      } else {
#pragma unroll
        for (int f = 0; f < NF; f++) {
          const int col = c0 + wn * 16 * NF + 16 * f + l16;
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

template <int MF, int NF, int WM, int WN>
int32_t launch_cfg(const GemmArgs &a, hipStream_t s) {
  constexpr int BM = 16 * MF * WM;
  constexpr int BN = 16 * NF * WN;
  const int out_bn = (a.epi == EPI_SWIGLU) ? BN / 2 : BN;
  int tiles_n = 0;
  for (int i = 0; i < a.nseg; i++) tiles_n += (a.seg[i].n + out_bn - 1) / out_bn;
  const int tiles_m = (a.m + BM - 1) / BM;
  dim3 grid(tiles_n, tiles_m), block(256);
  switch (a.epi) {
    case EPI_F16:
      hipLaunchKernelGGL((gemm_q4_kernel<MF, NF, WM, WN, EPI_F16>), grid, block, 0, s, a, tiles_m);
      break;
    case EPI_F32:
      hipLaunchKernelGGL((gemm_q4_kernel<MF, NF, WM, WN, EPI_F32>), grid, block, 0, s, a, tiles_m);
      break;
    case EPI_RESID:
      hipLaunchKernelGGL((gemm_q4_kernel<MF, NF, WM, WN, EPI_RESID>), grid, block, 0, s, a,
                         tiles_m);
      break;
    case EPI_SWIGLU:
      hipLaunchKernelGGL((gemm_q4_kernel<MF, NF, WM, WN, EPI_SWIGLU>), grid, block, 0, s, a,
                         tiles_m);
      break;
    default:
      return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "unknown GEMM epilogue");
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "gemm_q4_kernel launch");
  return SULIMO_HIP_OK;
}

}  // namespace

int32_t launch_gemm_q4_0(const GemmArgs &a, hipStream_t s) {
  if (a.m <= 0) return SULIMO_HIP_OK;
  if (a.k <= 0 || a.k % 32 != 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM k must be a positive multiple of 32");
  if (a.nseg < 1 || a.nseg > 3) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM needs 1..3 segments");
  for (int i = 0; i < a.nseg; i++)
    if (a.seg[i].n <= 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "GEMM segment with no rows");
  if (a.epi == EPI_SWIGLU && a.nseg != 1)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "SwiGLU GEMM takes one segment");
  // Tile choice: wide M tiles amortize the dequantization (each weight is
  // dequantized once per workgroup and used for BM rows).
  if (a.m <= 16) return launch_cfg<1, 2, 1, 4>(a, s);   // 16 x 128
  if (a.m <= 64) return launch_cfg<1, 8, 4, 1>(a, s);   // 64 x 128
  if (a.m <= 128) return launch_cfg<2, 8, 4, 1>(a, s);  // 128 x 128
  return launch_cfg<4, 8, 4, 1>(a, s);                  // 256 x 128
}

}  // namespace sulimo
