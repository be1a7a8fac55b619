// common.h - shared declarations of libsulimo_hip.so (host runtime + gfx950 kernels).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <condition_variable>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/sulimo_hip.h"

// Kernel classes of the prefill statistics (sulimo_hip_prefill_stats fields).
// The GEMM roles are counted in their own statistic and in the gemm class.
enum ProfClass : int {
  PROF_GEMM = 0, PROF_ATTN = 1, PROF_NORM = 2, PROF_ROPE_KV = 3, PROF_OTHER = 4,
  PROF_GEMM_QKV = 5, PROF_GEMM_O = 6, PROF_GEMM_GATE_UP = 7, PROF_GEMM_DOWN = 8, PROF_GEMM_LM_HEAD = 9
};

struct ProfRecord {
  int cls;
  int ev;  // index into sulimo_hip_ctx::ev_pool
  double flop, bytes;
};

// ---------------------------------------------------------------------------
// Host-side objects behind the opaque C handles
// ---------------------------------------------------------------------------
// Where a waiting engine thread sleeps until a host function on the context's waiter
// stream wakes it (posted counts the wake-ups).
struct ParkSlot {
  std::mutex m;
  std::condition_variable cv;
  uint64_t posted = 0;
};

// A ubatch's launches captured once and replayed: two executable graphs split at the
// wake-up gate (the host records near_event between them), keyed by every value the
// launches were built from.
struct PrefillGraph {
  std::vector<uint64_t> key;
  hipGraphExec_t pre = nullptr, post = nullptr;
  uint64_t last_use = 0;
};

struct sulimo_hip_ctx {
  int device = 0;
  bool shared = false;  // the get_or_init singleton (never freed)
  hipStream_t stream = nullptr;
  hipEvent_t done_event = nullptr;  // end of the queued work, recorded by every wait
  // Zero-spin waiting: a host function on `side` (gated on an event of `stream`)
  // wakes the thread parked in `park`; near_event marks a point shortly before the
  // end of a prefill, so that the wake-up latency of the host function overlaps the
  // last kernels.
  hipStream_t side = nullptr;
  hipEvent_t near_event = nullptr;
  ParkSlot park;
  uint64_t park_want = 0;
  // This device's copy of the library's static scratch array (no-alloc entry point),
  // resolved with hipGetSymbolAddress when the context is created.
  void *scratch = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  sulimo_hip_device_info info{};
  // Prefill workspace (grown on demand): f32 residual stream, Q8_0 K/V staging
  // for ring-wrapping ubatches, per-row argmax partials.
  void *ws = nullptr;
  size_t ws_bytes = 0;
  // Token ids staged for sulimo_hip_embed_tokens (grown on demand).
  void *tok = nullptr;
  size_t tok_bytes = 0;
  // Per-launch event timing (sulimo_hip_set_profiling).
  bool prof = false;
  std::vector<hipEvent_t> ev_pool;  // pairs: [2i] start, [2i+1] end
  std::vector<ProfRecord> pending;
  sulimo_hip_prefill_stats stats{};
  // Graph replay of execute_prefill_ubatch (sulimo_hip_set_graph_replay).
  bool graph_replay = true;
  // Arrival counters of split attention blocks (AttnArgs::ctr; zero between calls),
  // and whether a separate kernel merges the pieces instead
  // (sulimo_hip_set_attention_merge_kernel).
  int *attn_ctr = nullptr;
  size_t attn_ctr_n = 0;
  bool attn_merge_kernel = false;
  std::vector<PrefillGraph> graphs;
  uint64_t graph_tick = 0;
};

// GEMM-layout copy of one Q4_0 matrix (or an interleaved gate/up pair), built from
// the SoA buffers it is keyed on (q4_panels.hip).
struct Q4Panels {
  void *dev = nullptr;
  size_t bytes = 0;
  int n = 0, k = 0;
  bool interleave = false;
  uint64_t ids[4] = {0, 0, 0, 0};   // scales, quants, up scales, up quants
  uint64_t vers[4] = {0, 0, 0, 0};  // their write versions when the copy was built
};

// The f16 copy of a layer's K/V ring that the attention reads (its key window), kept
// on the K ring buffer between prefills of prompts that fit the ring: window index j =
// position j, K [n_head_kv][pad][head_dim] then V^T [n_head_kv][head_dim][pad + 64].
// Positions [0, len) hold f16(code * d) of the ring as it was when the K and V ring
// buffers had write versions k_ver and v_ver (any other write invalidates it).
struct KvWindowCache {
  void *dev = nullptr;
  size_t bytes = 0;
  int pad = 0, n_head_kv = 0, head_dim = 0;
  uint64_t v_id = 0, k_ver = 0, v_ver = 0;
  long len = 0;
};

struct sulimo_hip_buffer {
  void *dev = nullptr;
  void *host = nullptr;  // host mirror (the reference's arena slice), may be null
  size_t bytes = 0;
  bool read_only = false;
  int device = 0;
  uint64_t id = 0;       // unique per created buffer
  uint64_t version = 0;  // bumped by every write through this library
  std::vector<Q4Panels> panels;  // owned GEMM-layout copies (this buffer = their quants)
  KvWindowCache kvwin;           // attention window of the ring (this buffer = its K ring)
};

namespace sulimo {

// Thread-local last error; returns `code` for convenient `return fail(...)`.
int32_t fail(int32_t code, const std::string &msg);
int32_t hip_fail(hipError_t e, const char *what);
// Grows ctx->ws to at least `bytes` (synchronizes the stream before freeing the old one).
int32_t ensure_workspace(sulimo_hip_ctx *ctx, size_t bytes);
// Grows ctx->attn_ctr to at least n zeroed ints (on the context stream; not while a
// graph is being captured). *out: the counters, or null when the separate merge kernel
// is selected.
int32_t ensure_attn_counters(sulimo_hip_ctx *ctx, size_t n, int **out);
// Events a launch stamps with its kernels' own start and end times (hipExtLaunchKernel):
// the interval between them leaves out the dispatch gap that an event recorded on the
// stream ahead of the launch adds. Both null: an ordinary launch.
struct LaunchStamp {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Launches kern on s; a non-null start / stop event takes the kernel's start / end time.
template <typename K, typename... A>
inline void launch_stamped(K kern, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, hipEvent_t start,
                           hipEvent_t stop, A... args) {
  if (start || stop) hipExtLaunchKernelGGL(kern, grid, block, lds, s, start, stop, 0u, args...);
  else hipLaunchKernelGGL(kern, grid, block, lds, s, args...);
}

// Event pair around one launch when profiling is on: prof_begin returns the pair
// index (or -1), prof_end records the end event and queues the record;
// prof_collect (after the stream drained) adds the elapsed times to ctx->stats.
// prof_begin_stamp / prof_end_stamp hand the pair to the launch instead (LaunchStamp).
int prof_begin(sulimo_hip_ctx *ctx);
void prof_end(sulimo_hip_ctx *ctx, int ev, int cls, double flop, double bytes);
int prof_begin_stamp(sulimo_hip_ctx *ctx, LaunchStamp *stamp);
void prof_end_stamp(sulimo_hip_ctx *ctx, int ev, int cls, double flop, double bytes);
void prof_collect(sulimo_hip_ctx *ctx);

#define SULIMO_HIP_TRY(call)                                   \
  do {                                                         \
    hipError_t e_ = (call);                                    \
    if (e_ != hipSuccess) return ::sulimo::hip_fail(e_, #call); \
  } while (0)

// ---------------------------------------------------------------------------
// Kernel launchers (implemented in the .hip files; all enqueue on `s`)
// ---------------------------------------------------------------------------

// Epilogues of the Q4_0 x f16 GEMM.
enum GemmEpilogue : int {
  EPI_F16 = 0,     // out f16 [rows][ldo]
  EPI_F32 = 1,     // out f32 [rows][ldo]
  EPI_RESID = 2,   // out f32 residual [rows][ldo] += f16(acc)
  EPI_SWIGLU = 3,  // out f16 [rows][ldo] = silu(acc_w0) * acc_w1 (w0 = gate, w1 = up)
  EPI_PART = 4,    // f32 partial sums of one K split: part[split][rows][ldp], reduced by a later kernel
  EPI_ROPE = 5,    // q/k/v projection with RoPE and the Q8_0 K/V store (GemmArgs::rope)
};

// One weight matrix of a (possibly segmented) GEMM: `n` output rows, its
// scales/quants, and where its outputs go (column offset `col0` in out, row stride ldo).
// One output segment of a GEMM: n output columns from a Q4_0 panel array (for
// EPI_SWIGLU the interleaved gate/up panels of n output columns).
struct GemmSegment {
  const uint8_t *panels;
  void *out;
  int n;
  int ldo;
  int col0;
  const float *bias;  // optional f32 [n] added before the output rounding (F16/F32 epilogues)
};

// Optional window target of the RoPE + Q8_0 store: the K rows and V^T columns of token
// t go to window index j0 + t (the values f16(code * d) of the codes it stores).
struct RopeWindowTarget {
  uint16_t *k;  // f16 [n_head_kv][pad][head_dim]
  uint16_t *vt; // f16 [n_head_kv][head_dim][vst]
  int j0, pad, vst;
};
// RoPE + Q8_0 K/V store of a q/k/v projection (EPI_ROPE). Segments 0, 1, 2 are q, k and
// v of whole heads (rope_dim = head_dim, 64 or 128). q leaves rotated in f16 through
// segment 0's output; k (rotated) and v are quantized to Q8_0 rows of row_bytes at
// row (slot0 + t) % wrap of k_dst / v_dst, and with win.k set their window entries
// f16(code * f16(d)) go to window index win.j0 + t. The values are those of
// launch_rope_qkv_store applied to the f16 outputs of the plain projection.
struct GemmRope {
  const float *cs;  // float2 [m][head_dim / 2] cos/sin table of the ubatch
  int mode;         // 0: pairs (2i, 2i+1), 1: NeoX pairs (i, i + head_dim/2)
  int head_dim;
  uint8_t *k_dst, *v_dst;
  int slot0, wrap, row_bytes;
  RopeWindowTarget win;
};
struct GemmArgs {
  const uint16_t *x;  // f16 [m][ldx]
  int m, k, ldx;
  int epi;
  GemmSegment seg[3];
  int nseg;
  // K split across workgroups (EPI_PART only): `splits` workgroups per tile, split s
  // covering k stages [s * split_stages, (s + 1) * split_stages) of 64, each writing its
  // partial sums to element s * m * ldp + row * ldp + column of part (column = columns
  // of the segments before + col). part_f16: the partials are stored as f16 (for a
  // GEMM whose output is rounded to f16 anyway), else f32.
  int splits, split_stages;
  float *part;
  int ldp;
  int part_f16;
  // Workspace launch_gemm_q4_0 may use for K-split partials (none when part is null).
  size_t part_bytes;
  // Tile grid, filled by the launcher: tiles_m x tiles_n tiles, visited in groups of
  // group_m tile rows.
  int tiles_m, tiles_n, group_m;
  // Optional RMSNorm of the rows an EPI_RESID GEMM updates (one segment of whole rows:
  // col0 0, n the row width), run by the K-split reduction when the GEMM splits:
  // norm_out[row] = f16(x * (1 / sqrt(mean(x^2) + norm_eps)) * norm_w) ([m][n]) and, if
  // set, norm_x16[row] = f16(x). launch_gemm_q4_0 reports whether it ran it.
  const float *norm_w;
  uint16_t *norm_out, *norm_x16;
  float norm_eps;
  GemmRope rope;  // EPI_ROPE only
  // Persistent launch (filled by the launcher): fewer workgroups than tiles, each running
  // a strided run of its XCD's tiles and loading the next tile's first stages under the
  // current tile's epilogue. One segment, no split, an even block count, stages a
  // multiple of the ring depth, and the f16 or SwiGLU epilogue (no LDS use).
  int persist;
};

// Runs X W^T with the tile configuration and K split a cost model picks for the shape;
// a K split writes partials to a.part (a.part_bytes), f16 when the output is f16 (the
// f16 and residual epilogues) and f32 for an f32 output, and reduces them in f32 in a
// second kernel. With a.norm_w set and norm_done given, *norm_done tells whether that
// reduction also produced the RMSNorm of the updated rows.
// A non-null stamp takes the start of the first kernel and the end of the last.
int32_t launch_gemm_q4_0(const GemmArgs &a, hipStream_t s, bool *norm_done = nullptr,
                         const LaunchStamp *stamp = nullptr);
// Partial-sum workspace launch_gemm_q4_0 would use for this GEMM given unlimited room.
size_t gemm_q4_0_workspace_bytes(const GemmArgs &a);

// Size of the static device scratch array of the no-alloc GEMM entry point (one per
// device, held until the process ends).
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
// Orders the no-alloc GEMM calls of every context on one device: each call's stream
// waits for the event the previous call recorded (under the mutex), so that one call's
// panel pack cannot overwrite weights that another call's GEMM still reads.
struct NoAllocOrder {
  std::mutex m;
  hipEvent_t ev = nullptr;
};
// The device's NoAllocOrder (its event created with the scratch address), or null.
NoAllocOrder *noalloc_order(int device);

// Blocks the calling thread until all work queued on ctx->stream is done, without
// spinning while the GPU runs: the thread sleeps until a host function enqueued after
// `gate` (an event already recorded on ctx->stream; null = the end of the queue)
// wakes it, then waits for the rest of the queue. Reports asynchronous failures.
int32_t wait_parked(sulimo_hip_ctx *ctx, hipEvent_t gate);
// Destroys the context's cached prefill graphs.
void drop_prefill_graphs(sulimo_hip_ctx *ctx);

// The RoPE rotation terms a*b - c*d and a*b + c*d with both products rounded to f32
// before the add (no fused multiply-add), as the reference's rope_f16 and
// rope_head_scalar compute them; every kernel that rotates uses these, so the fused
// and the separate RoPE give identical bits.
__device__ __forceinline__ float rot_sub(float a, float b, float c, float d) {
#pragma clang fp contract(off)
  return a * b - c * d;
}
__device__ __forceinline__ float rot_add(float a, float b, float c, float d) {
#pragma clang fp contract(off)
  return a * b + c * d;
}

// silu(g) * u as the reference's silu_mul_f16 computes it in its OpenCL build, which
// uses -cl-fast-relaxed-math (kernels/prefill.cl:240-253, crates/sulimo-ocl/src/
// program.rs:23): the hardware exp2 and reciprocal, within a few f32 ulps of
// g / (1 + e^-g) * u, far below the f16 rounding that follows. Every kernel that
// applies SwiGLU uses this, so the fused and the separate SwiGLU give identical bits.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// One RMSNorm row held by one wave, lane l holding columns 256 j + 4 l .. +3. Every
// kernel that normalizes rows this way uses these helpers, so the separate RMSNorm and
// the one fused into the K-split reduction give identical bits: the sum of squares runs
// over j in order as one fma chain per lane, then across the wave; the output is the
// f32 product x * scale * w rounded to f16 once.
typedef _Float16 rms_half4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float rms_sumsq4(float4 v, float ss) {
  return __builtin_fmaf(v.w, v.w, __builtin_fmaf(v.z, v.z, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.x, v.x, ss))));
}
__device__ __forceinline__ float rms_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float rms_scale(float ss, int d, float eps) { return 1.0f / sqrtf(ss / (float)d + eps); }
__device__ __forceinline__ rms_half4 rms_out4(float4 v, float scale, float4 w) {
#pragma clang fp contract(off)
  float a = v.x * scale * w.x, b = v.y * scale * w.y, c = v.z * scale * w.z, d = v.w * scale * w.w;
  asm("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));  // no fused product-and-round (v_fma_mix)
  return rms_half4{(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
}

// Compute units of the current device (cached per device).
int device_cu_count();

// Bytes of one panel record: 32 weight rows x one 64-wide k stage (1 KB quants + 128 B scales).
constexpr int kQ4PanelRecord = 1152;

// Panel copy (q4_panels.hip) of the n x k Q4_0 matrix (scales, quants), or of the
// interleaved gate/up pair when up_scales is given; built on ctx's stream when
// missing or stale. Buffer sizes are the caller's to check.
int32_t get_q4_panels(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *scales, const sulimo_hip_buffer *quants,
                      const sulimo_hip_buffer *up_scales, const sulimo_hip_buffer *up_quants, int n, int k,
                      const uint8_t **out);
size_t q4_panel_bytes(int n, int k, bool interleave);
// Writes the panel copy of (scales, quants) (interleaved with (up_scales, up_quants)
// when given) to dst, q4_panel_bytes(n, k, up_scales != nullptr) bytes, on stream s.
int32_t launch_pack_q4_panels(const uint16_t *scales, const uint8_t *quants, const uint16_t *up_scales,
                              const uint8_t *up_quants, int n, int k, uint8_t *dst, hipStream_t s);
void release_q4_panels(sulimo_hip_buffer *b);
// Marks a buffer as written (invalidates panel copies built from it).
inline void wrote(const sulimo_hip_buffer *b) {
  if (b) const_cast<sulimo_hip_buffer *>(b)->version++;
}

// Bandwidth kernels (prefill_ops.hip).
int32_t launch_rmsnorm_f16(const uint16_t *x, const float *w, uint16_t *out, int d, float eps,
                           int n, hipStream_t s);
int32_t launch_rmsnorm_f32(const float *x, const float *w, uint16_t *out, uint16_t *x16_out,
                           int d, float eps, int n, hipStream_t s);
int32_t launch_rope_f16(uint16_t *vec, int head_count, int head_dim, int rope_dim,
                        float freq_base, int mode, int start_pos, int n, hipStream_t s);
int32_t launch_kv_store_q8_0(const uint16_t *act, uint8_t *kv, int start_pos, int capacity,
                             int blocks_per_pos, int n, hipStream_t s);
int32_t launch_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t total,
                        hipStream_t s);
int32_t launch_add_f16(uint16_t *a, const uint16_t *b, size_t total, hipStream_t s);
int32_t launch_f16_to_f32(const uint16_t *in, float *out, size_t total, hipStream_t s);
int32_t launch_add_f16_to_f32(float *x, const uint16_t *b, size_t total, hipStream_t s);
int32_t launch_embed_q4_0(const uint16_t *scales, const uint8_t *quants, const uint32_t *tokens,
                          int n, int embd, uint16_t *x, hipStream_t s);
// RoPE on q (in place, f16) and k (f32 rotation), then Q8_0 of k and v into
// k_dst/v_dst rows of `dst_stride` bytes; row t goes to slot (slot0 + t) % wrap.
// cos/sin table of a ubatch for the fused RoPE: float2 [n][rope_dim/2] at positions
// start_pos .. start_pos+n-1.
int32_t launch_rope_table(float *tab, int rope_dim, float freq_base, int start_pos, int n, hipStream_t s);
// q_norm / k_norm: optional f32 [head_dim] QK-norm weights (per-head RMSNorm with eps
// before the rotation), or null.
int32_t launch_rope_qkv_store(uint16_t *q, const uint16_t *k, const uint16_t *v, int n_head,
                              int n_head_kv, int head_dim, int rope_dim, const float *cs_tab,
                              int mode, int n, uint8_t *k_dst, uint8_t *v_dst,
                              int slot0, int wrap, const float *q_norm, const float *k_norm,
                              float eps, hipStream_t s, const RopeWindowTarget *win = nullptr,
                              bool *wrote_window = nullptr);
// Copies n rows of `row_bytes` from src to ring slots (slot0 + t) % capacity.
int32_t launch_ring_commit(const uint8_t *src, uint8_t *ring, size_t row_bytes, int slot0,
                           int capacity, int n, hipStream_t s);
int32_t launch_argmax_rows(const float *logits, int rows, int cols, int32_t *out, hipStream_t s);

// Causal GQA attention over the Q8_0 ring (attention.hip). Keys at positions
// p < new_pos0 are read from the ring at slot p % capacity; p >= new_pos0 from
// `new_k/new_v` row (p - new_pos0) (row stride bytes_per_pos).
struct AttnArgs {
  const uint16_t *q;  // f16 [n][n_head][head_dim]
  uint16_t *out;      // f16 [n][n_head][head_dim]
  const uint8_t *k_ring, *v_ring;
  const uint8_t *new_k, *new_v;
  long new_pos0;
  int start_pos, n, capacity, n_head, n_head_kv, head_dim;
  // Attention workspace (attention_workspace_bytes of device memory): the f16 copy of
  // the visible key window, then the partial results of query blocks whose keys are
  // split over several workgroups.
  void *window;
  // Nonzero when the caller already wrote the window entries of the ubatch's own
  // positions [start_pos, start_pos + n) (the RoPE + Q8_0 store does, from the codes it
  // stores); the window pass then covers only the earlier positions and the padding.
  int win_new_done;
  // Kept window (start_pos + n <= capacity): win_pad > 0 is its fixed padded length,
  // window index = position, and positions [0, win_valid) already hold their values;
  // only the rest of the positions before the ubatch are dequantized. The padding past
  // the last position holds finite values (zeros or older positions), which the causal
  // mask removes. part is then where the split-key partials go (else after the window).
  int win_pad, win_valid;
  float *part;
  // ctr_ints (at least attention_counter_ints) zero-initialized ints, or null. When
  // set, the last wave to finish a split block's queries merges the block's pieces
  // itself (and resets its counter to zero); when null, a separate kernel merges them.
  int *ctr;
  size_t ctr_ints;
};
// Device bytes of AttnArgs::window for this attention call (depends on the shapes and
// on the device's compute-unit count).
size_t attention_workspace_bytes(const AttnArgs &a);
// Arrival counters AttnArgs::ctr must hold for this call's shape.
size_t attention_counter_ints(const AttnArgs &a);
int32_t launch_attention(const AttnArgs &a, hipStream_t s);

// The f16 key window of an attention call: window index j holds position lo + j for
// j < len (zeros up to pad); K is [n_head_kv][pad][head_dim] at AttnArgs::window, V^T
// is [n_head_kv][head_dim][vst] after it.
struct AttnWindowLayout {
  long lo;
  int len, pad, vst;
};
AttnWindowLayout attention_window_layout(const AttnArgs &a);
// Bytes of the f16 key window of attention call a (with win_pad set: of the kept window).
size_t attention_window_bytes(const AttnArgs &a);
// Column of window index j in a V^T row: inside each group of 16 keys, slots 4-7 and
// 8-11 are swapped (the order in which the attention reads P^T operands).
__host__ __device__ inline int window_vt_col(int j) {
  const int s = j & 15;
  return (j & ~15) + ((s & 4) ? ((s & 8) ? s : s + 4) : ((s & 8) ? s - 4 : s));
}

}  // namespace sulimo
