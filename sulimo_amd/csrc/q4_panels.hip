// q4_panels.hip - the GEMM's device layout of Q4_0 weights ("panels") and its cache.
//
// The reference hands its backend each Q4_0 matrix as two SoA arrays, scales f16
// [rows][k/32] and quants [rows][k/32][16] (crates/sulimo-core/src/repack.rs:107-131),
// and its OpenCL backend builds that SoA copy from the GGUF blocks at load time.
// This backend keeps the same input buffers and, once per matrix, builds a second
// copy laid out for the GEMM's fetches:
//
//   panel p = weight rows 32p .. 32p+31, stage st = blocks 2st, 2st+1 (64 k);
//   record (p, st) = 1152 bytes at (p * nst + st) * 1152, nst = ceil(nb / 2):
//     bytes [0, 1024): 16-byte chunk 32h + r = quant bytes 8h .. 8h+7 of block 2st and
//       then of block 2st+1, both of row 32p + r (h = 0, 1: the two half-waves of the
//       MFMA B operand), so lane l of a wave reads its 16 bytes at 16*l
//     bytes [1024, 1152): row r's scales of blocks 2st, 2st+1 at 1024 + 4r
//   Rows past the matrix and the missing block of an odd block count hold scale 0
//   and quants 0 (weight exactly zero). Same 18 bytes per 32 weights as Q4_0.
//
// A GEMM workgroup then fetches one stage of 32 rows as a single contiguous 1 KB
// chunk run and 128 bytes of scales, instead of 32 scattered 32-byte row pieces and
// 4-byte scale pairs (those fetches cost several times more per byte).
//
// SwiGLU packs gate and up into one panel array, alternating: panel 2j = gate rows
// 32j.., panel 2j+1 = up rows 32j.., so one fetch stream serves both matrices.
//
// The copy is cached on the quants buffer of the (first) matrix, keyed on the ids and
// write versions of its source buffers, and rebuilt when any of them changed.
#include <mutex>

#include "common.h"

namespace sulimo {
namespace {

constexpr int kChunks = kQ4PanelRecord / 16;  // 64 quant chunks + 8 scale chunks

struct PackArgs {
  const uint16_t *scales[2];
  const uint8_t *quants[2];
  uint8_t *out;
  int n, nb, nst, npanels;
  int interleave;  // panels alternate matrix 0 and matrix 1
};

__global__ __launch_bounds__(256) void pack_q4_panels_kernel(PackArgs a) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)a.npanels * a.nst * kChunks;
  if (t >= total) return;
  const long rec = t / kChunks;
  const int c = (int)(t - rec * kChunks);
  const int p = (int)(rec / a.nst), st = (int)(rec - (long)p * a.nst);
  const int m = a.interleave ? (p & 1) : 0;
  const int sp = a.interleave ? (p >> 1) : p;
  uint4 v = {0u, 0u, 0u, 0u};
  if (c < 64) {
    const int row = 32 * sp + (c & 31), h = c >> 5;
    if (row < a.n) {
      const uint8_t *q = a.quants[m] + ((size_t)row * a.nb + 2 * st) * 16 + 8 * h;
      const uint2 lo = *reinterpret_cast<const uint2 *>(q);
      const uint2 hi = 2 * st + 1 < a.nb ? *reinterpret_cast<const uint2 *>(q + 16) : uint2{0u, 0u};
      v = uint4{lo.x, lo.y, hi.x, hi.y};
    }
  } else {
    uint32_t w[4];
    for (int i = 0; i < 4; i++) {  // rows 4j .. 4j+3 of the panel, two scales each
      const int row = 32 * sp + 4 * (c - 64) + i;
      uint32_t lo = 0, hi = 0;
      if (row < a.n) {
        const uint16_t *s = a.scales[m] + (size_t)row * a.nb;
        if (2 * st < a.nb) lo = s[2 * st];
        if (2 * st + 1 < a.nb) hi = s[2 * st + 1];
      }
      w[i] = lo | (hi << 16);
    }
    v = uint4{w[0], w[1], w[2], w[3]};
  }
  *reinterpret_cast<uint4 *>(a.out + rec * kQ4PanelRecord + (size_t)c * 16) = v;
}

std::mutex g_panel_mu;

}  // namespace

int32_t launch_pack_q4_panels(const uint16_t *scales, const uint8_t *quants, const uint16_t *up_scales,
                              const uint8_t *up_quants, int n, int k, uint8_t *dst, hipStream_t s) {
  const bool inter = up_scales != nullptr;
  PackArgs pa{};
  pa.scales[0] = scales;
  pa.quants[0] = quants;
  pa.scales[1] = inter ? up_scales : scales;
  pa.quants[1] = inter ? up_quants : quants;
  pa.out = dst;
  pa.n = n;
  pa.nb = k / 32;
  pa.nst = (pa.nb + 1) / 2;
  pa.npanels = (n + 31) / 32 * (inter ? 2 : 1);
  pa.interleave = inter ? 1 : 0;
  const long total = (long)pa.npanels * pa.nst * kChunks;
  hipLaunchKernelGGL(pack_q4_panels_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, pa);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "pack_q4_panels_kernel launch");
  return SULIMO_HIP_OK;
}

size_t q4_panel_bytes(int n, int k, bool interleave) {
  const size_t np = (size_t)(n + 31) / 32 * (interleave ? 2 : 1);
  const size_t nst = ((size_t)k / 32 + 1) / 2;
  return np * nst * kQ4PanelRecord;
}

int32_t get_q4_panels(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales, const sulimo_hip_buffer *quants,
                      const sulimo_hip_buffer *up_scales, const sulimo_hip_buffer *up_quants, int n, int k,
                      const uint8_t **out) {
  const bool inter = up_scales != nullptr;
  std::lock_guard<std::mutex> lock(g_panel_mu);
  sulimo_hip_buffer *owner = const_cast<sulimo_hip_buffer *>(quants);
  const uint64_t ids[4] = {scales->id, quants->id, inter ? up_scales->id : 0, inter ? up_quants->id : 0};
  const uint64_t vers[4] = {scales->version, quants->version, inter ? up_scales->version : 0,
                            inter ? up_quants->version : 0};
  for (auto it = owner->panels.begin(); it != owner->panels.end(); ++it) {
    bool same_role = it->n == n && it->k == k && it->interleave == inter;
    for (int i = 0; i < 4 && same_role; i++) same_role = it->ids[i] == ids[i];
    if (!same_role) continue;
    bool fresh = true;
    for (int i = 0; i < 4; i++) fresh = fresh && it->vers[i] == vers[i];
    if (fresh) {
      *out = reinterpret_cast<const uint8_t *>(it->dev);
      return SULIMO_HIP_OK;
    }
    // sources changed since the copy was built: drop it (hipFree waits for its readers)
    hipFree(it->dev);
    owner->panels.erase(it);
    break;
  }
  const size_t bytes = q4_panel_bytes(n, k, inter);
  if (bytes >= (1ull << 31)) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "Q4_0 matrix exceeds the 2 GiB GEMM limit");
  Q4Panels e;
  SULIMO_HIP_TRY(hipMalloc(&e.dev, bytes));
  e.bytes = bytes;
  e.n = n;
  e.k = k;
  e.interleave = inter;
  for (int i = 0; i < 4; i++) {
    e.ids[i] = ids[i];
    e.vers[i] = vers[i];
  }
  const int32_t rc = launch_pack_q4_panels(
      reinterpret_cast<const uint16_t *>(scales->dev), reinterpret_cast<const uint8_t *>(quants->dev),
      inter ? reinterpret_cast<const uint16_t *>(up_scales->dev) : nullptr,
      inter ? reinterpret_cast<const uint8_t *>(up_quants->dev) : nullptr, n, k,
      reinterpret_cast<uint8_t *>(e.dev), ctx->stream);
  if (rc) {
    hipFree(e.dev);
    return rc;
  }
  owner->panels.push_back(e);
  *out = reinterpret_cast<const uint8_t *>(e.dev);
  return SULIMO_HIP_OK;
}

void release_q4_panels(sulimo_hip_buffer *b) {
  std::lock_guard<std::mutex> lock(g_panel_mu);
  for (auto &e : b->panels) hipFree(e.dev);
  b->panels.clear();
}

}  // namespace sulimo
