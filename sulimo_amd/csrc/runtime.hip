// runtime.hip - host runtime of libsulimo_hip.so: contexts, buffers, errors,
// waiting, probing and timing. Replaces crates/sulimo-ocl/src/{program,buffer,
// waiter,probe}.rs with HIP equivalents for one discrete MI355X device.
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>

#include <chrono>

#include "common.h"

namespace sulimo {

static thread_local std::string g_last_error;
static std::atomic<size_t> g_active_buffers{0};
static std::atomic<uint64_t> g_next_buffer_id{1};

int32_t fail(int32_t code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int32_t hip_fail(hipError_t e, const char *what) {
  std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  int32_t code = SULIMO_HIP_ERR_DRIVER;
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) code = SULIMO_HIP_ERR_DEVICE_NOT_FOUND;
  if (e == hipErrorNoBinaryForGpu || e == hipErrorInvalidImage || e == hipErrorInvalidKernelFile)
    code = SULIMO_HIP_ERR_BUILD_FAILED;
  if (e == hipErrorLaunchFailure || e == hipErrorIllegalAddress || e == hipErrorAssert ||
      e == hipErrorLaunchTimeOut)
    code = SULIMO_HIP_ERR_EXECUTION_FAILED;
  return fail(code, m);
}

int32_t ensure_workspace(sulimo_hip_ctx *ctx, size_t bytes) {
  if (ctx->ws_bytes >= bytes) return SULIMO_HIP_OK;
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  if (ctx->ws) {
    SULIMO_HIP_TRY(hipStreamSynchronize(ctx->stream));
    SULIMO_HIP_TRY(hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
  }
  size_t sz = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
  SULIMO_HIP_TRY(hipMalloc(&ctx->ws, sz));
  ctx->ws_bytes = sz;
  return SULIMO_HIP_OK;
}

int32_t ensure_attn_counters(sulimo_hip_ctx *ctx, size_t n, int **out) {
  *out = nullptr;
  if (ctx->attn_merge_kernel || n == 0) return SULIMO_HIP_OK;
  if (ctx->attn_ctr_n < n) {
    SULIMO_HIP_TRY(hipSetDevice(ctx->device));
    if (ctx->attn_ctr) {
      SULIMO_HIP_TRY(hipStreamSynchronize(ctx->stream));
      SULIMO_HIP_TRY(hipFree(ctx->attn_ctr));
      ctx->attn_ctr = nullptr;
      ctx->attn_ctr_n = 0;
    }
    const size_t sz = (n + 1023) & ~(size_t)1023;
    SULIMO_HIP_TRY(hipMalloc(&ctx->attn_ctr, sz * sizeof(int)));
    SULIMO_HIP_TRY(hipMemsetAsync(ctx->attn_ctr, 0, sz * sizeof(int), ctx->stream));
    ctx->attn_ctr_n = sz;
  }
  *out = ctx->attn_ctr;
  return SULIMO_HIP_OK;
}

int prof_begin(sulimo_hip_ctx *ctx) {
  if (!ctx->prof) return -1;
  const int i = (int)ctx->pending.size();
  while ((int)ctx->ev_pool.size() < 2 * (i + 1)) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -1;
    ctx->ev_pool.push_back(e);
  }
  if (hipEventRecord(ctx->ev_pool[2 * i], ctx->stream) != hipSuccess) return -1;
  return i;
}

void prof_end(sulimo_hip_ctx *ctx, int ev, int cls, double flop, double bytes) {
  if (ev < 0) return;
  if (hipEventRecord(ctx->ev_pool[2 * ev + 1], ctx->stream) != hipSuccess) return;
  ctx->pending.push_back(ProfRecord{cls, ev, flop, bytes});
}

int prof_begin_stamp(sulimo_hip_ctx *ctx, LaunchStamp *stamp) {
  if (!ctx->prof) return -1;
  const int i = (int)ctx->pending.size();
  while ((int)ctx->ev_pool.size() < 2 * (i + 1)) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -1;
    ctx->ev_pool.push_back(e);
  }
  stamp->start = ctx->ev_pool[2 * i];
  stamp->stop = ctx->ev_pool[2 * i + 1];
  return i;
}

void prof_end_stamp(sulimo_hip_ctx *ctx, int ev, int cls, double flop, double bytes) {
  if (ev >= 0) ctx->pending.push_back(ProfRecord{cls, ev, flop, bytes});
}

void prof_collect(sulimo_hip_ctx *ctx) {
  sulimo_hip_kernel_stat *st[10] = {&ctx->stats.gemm,     &ctx->stats.attention,    &ctx->stats.norm,
                                    &ctx->stats.rope_kv,  &ctx->stats.other,        &ctx->stats.gemm_qkv,
                                    &ctx->stats.gemm_o,   &ctx->stats.gemm_gate_up, &ctx->stats.gemm_down,
                                    &ctx->stats.gemm_lm_head};
  for (const ProfRecord &r : ctx->pending) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ctx->ev_pool[2 * r.ev], ctx->ev_pool[2 * r.ev + 1]) != hipSuccess) {
      (void)hipGetLastError();  // not an error of a later launch
      continue;
    }
    for (int c : {r.cls, r.cls >= PROF_GEMM_QKV ? (int)PROF_GEMM : -1}) {
      if (c < 0) continue;
      sulimo_hip_kernel_stat *k = st[c];
      k->launches++;
      k->total_ms += ms;
      k->flop += r.flop;
      k->bytes += r.bytes;
    }
  }
  ctx->pending.clear();
}

static int32_t fill_info(int device, sulimo_hip_device_info *info) {
  hipDeviceProp_t p;
  SULIMO_HIP_TRY(hipGetDeviceProperties(&p, device));
  memset(info, 0, sizeof(*info));
  snprintf(info->device_name, sizeof(info->device_name), "%s", p.name);
  snprintf(info->arch_name, sizeof(info->arch_name), "%s", p.gcnArchName);
  int drv = 0;
  hipDriverGetVersion(&drv);
  snprintf(info->driver_version, sizeof(info->driver_version), "%d", drv);
  info->device_index = device;
  info->compute_units = p.multiProcessorCount;
  info->clock_khz = p.clockRate;
  info->wavefront_size = p.warpSize;
  info->global_mem_bytes = p.totalGlobalMem;
  info->lds_bytes_per_block = p.sharedMemPerBlock;
  info->host_unified_memory = p.integrated ? 1 : 0;
  info->has_fp16 = 1;
  return SULIMO_HIP_OK;
}

// Scratch of sulimo_hip_enqueue_gemm_q4_0_f16_noalloc: the packed weight panels and
// the K-split partial sums of one GEMM. Each device holds its own copy of this array;
// host code must use the address hipGetSymbolAddress returns for the device (the
// array's name on the host is not a device address).
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static NoAllocOrder g_noalloc_order[64];

NoAllocOrder *noalloc_order(int device) {
  return device >= 0 && device < 64 && g_noalloc_order[device].ev ? &g_noalloc_order[device] : nullptr;
}

// Per-device address of `scratch`, resolved once per device with that device current,
// and the event that orders the no-alloc calls on it.
static int32_t resolve_scratch(int device, void **out) {
  static std::mutex mu;
  static void *ptrs[64] = {nullptr};
  std::lock_guard<std::mutex> g(mu);
  if (!ptrs[device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "scratch symbol address");
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "no-alloc ordering event");
    g_noalloc_order[device].ev = ev;
    ptrs[device] = p;
  }
  *out = ptrs[device];
  return SULIMO_HIP_OK;
}

static int32_t create_ctx(int device, bool shared, sulimo_hip_ctx **out) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(SULIMO_HIP_ERR_DEVICE_NOT_FOUND, "no HIP device visible");
  if (device < 0 || device >= count)
    return fail(SULIMO_HIP_ERR_DEVICE_NOT_FOUND, "device index out of range");
  sulimo_hip_ctx *c = new sulimo_hip_ctx();
  c->device = device;
  c->shared = shared;
  int32_t rc = fill_info(device, &c->info);
  if (rc) {
    delete c;
    return rc;
  }
  if (strncmp(c->info.arch_name, "gfx950", 6) != 0) {
    std::string m = std::string("kernels are built for gfx950, device is ") + c->info.arch_name;
    delete c;
    return fail(SULIMO_HIP_ERR_BUILD_FAILED, m);
  }
  if ((e = hipSetDevice(device)) != hipSuccess || (e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&c->done_event, hipEventDisableTiming)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&c->near_event, hipEventDisableTiming)) != hipSuccess ||
      (e = hipEventCreate(&c->t0)) != hipSuccess || (e = hipEventCreate(&c->t1)) != hipSuccess) {
    int32_t r = hip_fail(e, "context creation");
    delete c;
    return r;
  }
  if ((rc = resolve_scratch(device, &c->scratch))) {  // device `device` is current here
    hipEventDestroy(c->done_event);
    hipEventDestroy(c->near_event);
    hipEventDestroy(c->t0);
    hipEventDestroy(c->t1);
    hipStreamDestroy(c->stream);
    hipStreamDestroy(c->side);
    delete c;
    return rc;
  }
  *out = c;
  return SULIMO_HIP_OK;
}

void drop_prefill_graphs(sulimo_hip_ctx *ctx) {
  for (PrefillGraph &g : ctx->graphs) {
    if (g.pre) hipGraphExecDestroy(g.pre);
    if (g.post) hipGraphExecDestroy(g.post);
  }
  ctx->graphs.clear();
}

// Host function run by the HIP runtime on the waiter stream.
static void park_post(void *p) {
  ParkSlot *k = static_cast<ParkSlot *>(p);
  std::lock_guard<std::mutex> g(k->m);
  k->posted++;
  k->cv.notify_all();
}

// The reference parks the engine thread until an OpenCL event callback unparks it
// (crates/sulimo-ocl/src/waiter.rs:25-82). HIP's own synchronization calls spin on
// the completion signal for their whole duration (a core at 100 % while the GPU
// runs), so the park is built the same way here: a host function (hipLaunchHostFunc)
// notifies a condition variable. It runs some 70 us after the work before it, so a
// gate placed a little before the end of the work (near_event) hides that latency;
// that host function goes on the second stream, behind the gate, so that the work
// stream does not stall on it. Without a gate it goes on the work stream itself (a
// cross-stream wait costs some 20 us of CPU), where nothing follows it. The final
// hipEventSynchronize spins only over what is left after the wake-up.
int32_t wait_parked(sulimo_hip_ctx *ctx, hipEvent_t gate) {
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  SULIMO_HIP_TRY(hipEventRecord(ctx->done_event, ctx->stream));
  if (hipEventQuery(ctx->done_event) == hipErrorNotReady) {
    const uint64_t want = ++ctx->park_want;
    hipError_t e = hipSuccess;
    hipStream_t hs = ctx->stream;
    if (gate) {
      hs = ctx->side;
      e = hipStreamWaitEvent(ctx->side, gate, 0);
    }
    if (e == hipSuccess) e = hipLaunchHostFunc(hs, park_post, &ctx->park);
    if (e == hipSuccess) {
      // Sleep until the host function runs. Every 10 ms the thread also asks the
      // runtime about the end event: a stream that failed never runs the host
      // function, and the error is reported instead of waiting for ever.
      std::unique_lock<std::mutex> l(ctx->park.m);
      while (!ctx->park.cv.wait_for(l, std::chrono::milliseconds(10),
                                    [&] { return ctx->park.posted >= want; })) {
        const hipError_t q = hipEventQuery(ctx->done_event);
        if (q != hipSuccess && q != hipErrorNotReady) return hip_fail(q, "stream execution");
        if (q == hipSuccess) break;  // finished; the host function may still be on its way
      }
    } else {
      ctx->park_want--;  // no host function queued: fall back to the runtime's wait
    }
  }
  hipError_t e = hipEventSynchronize(ctx->done_event);
  if (e != hipSuccess) return hip_fail(e, "stream execution");
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "stream execution");
  return SULIMO_HIP_OK;
}

}  // namespace sulimo

using namespace sulimo;

extern "C" {

const char *sulimo_hip_last_error(void) { return g_last_error.c_str(); }

int32_t sulimo_hip_get_or_init(int32_t device, sulimo_hip_ctx **out) {
  static std::mutex mu;
  static sulimo_hip_ctx *shared[64] = {nullptr};
  if (!out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "out is null");
  if (device < 0 || device >= 64) return fail(SULIMO_HIP_ERR_DEVICE_NOT_FOUND, "device index out of range");
  std::lock_guard<std::mutex> g(mu);
  if (!shared[device]) {
    int32_t rc = create_ctx(device, true, &shared[device]);
    if (rc) return rc;
  }
  *out = shared[device];
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_context_new(int32_t device, sulimo_hip_ctx **out) {
  if (!out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "out is null");
  return create_ctx(device, false, out);
}

int32_t sulimo_hip_context_release(sulimo_hip_ctx *ctx) {
  if (!ctx || ctx->shared) return SULIMO_HIP_OK;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  if (ctx->ws) hipFree(ctx->ws);
  if (ctx->tok) hipFree(ctx->tok);
  if (ctx->attn_ctr) hipFree(ctx->attn_ctr);
  hipStreamSynchronize(ctx->side);
  hipEventDestroy(ctx->done_event);
  hipEventDestroy(ctx->near_event);
  hipEventDestroy(ctx->t0);
  hipEventDestroy(ctx->t1);
  for (hipEvent_t e : ctx->ev_pool) hipEventDestroy(e);
  drop_prefill_graphs(ctx);
  hipStreamDestroy(ctx->stream);
  hipStreamDestroy(ctx->side);
  delete ctx;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_finish(sulimo_hip_ctx *ctx) { return sulimo_hip_wait(ctx); }

int32_t sulimo_hip_get_device_info(const sulimo_hip_ctx *ctx, sulimo_hip_device_info *out) {
  if (!ctx || !out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  *out = ctx->info;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_probe(sulimo_hip_probe_result *out) {
  if (!out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "out is null");
  memset(out, 0, sizeof(*out));
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    snprintf(out->reason, sizeof(out->reason), "no HIP device: %s",
             e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
    return SULIMO_HIP_OK;
  }
  for (int d = 0; d < count; d++) {
    sulimo_hip_device_info info;
    if (fill_info(d, &info) == SULIMO_HIP_OK && strncmp(info.arch_name, "gfx950", 6) == 0) {
      out->available = 1;
      out->info = info;
      return SULIMO_HIP_OK;
    }
  }
  snprintf(out->reason, sizeof(out->reason), "no gfx950 device among %d HIP devices", count);
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_wait(sulimo_hip_ctx *ctx) {
  if (!ctx) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "ctx is null");
  return wait_parked(ctx, nullptr);
}

int32_t sulimo_hip_set_graph_replay(sulimo_hip_ctx *ctx, int32_t enable) {
  if (!ctx) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "ctx is null");
  int32_t rc = sulimo_hip_wait(ctx);
  if (rc) return rc;
  ctx->graph_replay = enable != 0;
  if (!ctx->graph_replay) drop_prefill_graphs(ctx);
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_set_attention_merge_kernel(sulimo_hip_ctx *ctx, int32_t enable) {
  if (!ctx) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "ctx is null");
  int32_t rc = sulimo_hip_wait(ctx);
  if (rc) return rc;
  ctx->attn_merge_kernel = enable != 0;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_set_profiling(sulimo_hip_ctx *ctx, int32_t enable) {
  if (!ctx) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "ctx is null");
  int32_t rc = sulimo_hip_wait(ctx);
  if (rc) return rc;
  ctx->pending.clear();
  ctx->stats = sulimo_hip_prefill_stats{};
  ctx->prof = enable != 0;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_get_prefill_stats(const sulimo_hip_ctx *ctx, sulimo_hip_prefill_stats *out) {
  if (!ctx || !out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  *out = ctx->stats;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_timer_start(sulimo_hip_ctx *ctx) {
  if (!ctx) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "ctx is null");
  SULIMO_HIP_TRY(hipEventRecord(ctx->t0, ctx->stream));
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_timer_stop(sulimo_hip_ctx *ctx, float *elapsed_ms) {
  if (!ctx || !elapsed_ms) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  SULIMO_HIP_TRY(hipEventRecord(ctx->t1, ctx->stream));
  int32_t rc = wait_parked(ctx, nullptr);
  if (rc) return rc;
  SULIMO_HIP_TRY(hipEventElapsedTime(elapsed_ms, ctx->t0, ctx->t1));
  return SULIMO_HIP_OK;
}

// ---- buffers ----

int32_t sulimo_hip_buffer_create(sulimo_hip_ctx *ctx, void *host_ptr, size_t bytes,
                                 int32_t read_only, sulimo_hip_buffer **out) {
  if (!ctx || !out) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (bytes == 0) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "buffer size must be positive");
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  void *dev = nullptr;
  SULIMO_HIP_TRY(hipMalloc(&dev, bytes));
  if (host_ptr) {
    hipError_t e = hipMemcpyAsync(dev, host_ptr, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      hipFree(dev);
      return hip_fail(e, "buffer upload");
    }
  }
  sulimo_hip_buffer *b = new sulimo_hip_buffer();
  b->dev = dev;
  b->host = host_ptr;
  b->bytes = bytes;
  b->read_only = read_only != 0;
  b->device = ctx->device;
  b->id = g_next_buffer_id.fetch_add(1);
  g_active_buffers.fetch_add(1);
  *out = b;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_buffer_release(sulimo_hip_buffer *buf) {
  if (!buf) return SULIMO_HIP_OK;
  hipSetDevice(buf->device);
  release_q4_panels(buf);
  if (buf->kvwin.dev) hipFree(buf->kvwin.dev);
  // hipFree waits for work that may still use the allocation.
  hipError_t e = hipFree(buf->dev);
  delete buf;
  g_active_buffers.fetch_sub(1);
  return e == hipSuccess ? SULIMO_HIP_OK : hip_fail(e, "buffer release");
}

size_t sulimo_hip_active_buffer_count(void) { return g_active_buffers.load(); }
size_t sulimo_hip_buffer_size(const sulimo_hip_buffer *b) { return b ? b->bytes : 0; }
void *sulimo_hip_buffer_device_ptr(const sulimo_hip_buffer *b) { return b ? b->dev : nullptr; }
void *sulimo_hip_buffer_host_ptr(const sulimo_hip_buffer *b) { return b ? b->host : nullptr; }

int32_t sulimo_hip_buffer_upload(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf, size_t offset,
                                 size_t bytes, const void *src) {
  if (!ctx || !buf || (!src && bytes)) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (offset > buf->bytes || bytes > buf->bytes - offset)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "upload range exceeds the buffer");
  if (!bytes) return SULIMO_HIP_OK;
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  // Pageable source: the copy is staged before the call returns, so `src` may be reused.
  SULIMO_HIP_TRY(hipMemcpyAsync((char *)buf->dev + offset, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  wrote(buf);
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_buffer_download(sulimo_hip_ctx *ctx, const sulimo_hip_buffer *buf,
                                   size_t offset, size_t bytes, void *dst) {
  if (!ctx || !buf || (!dst && bytes)) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (offset > buf->bytes || bytes > buf->bytes - offset)
    return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "download range exceeds the buffer");
  if (!bytes) return SULIMO_HIP_OK;
  SULIMO_HIP_TRY(hipSetDevice(ctx->device));
  SULIMO_HIP_TRY(hipMemcpyAsync(dst, (const char *)buf->dev + offset, bytes, hipMemcpyDeviceToHost, ctx->stream));
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "download");
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_buffer_map_read(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf,
                                   const void **mapped) {
  if (!ctx || !buf || !mapped) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (!buf->host) return fail(SULIMO_HIP_ERR_ZERO_COPY, "buffer has no host mirror to map");
  int32_t rc = sulimo_hip_buffer_download(ctx, buf, 0, buf->bytes, buf->host);
  if (rc) return rc;
  *mapped = buf->host;
  return SULIMO_HIP_OK;
}

int32_t sulimo_hip_buffer_unmap(sulimo_hip_ctx *ctx, sulimo_hip_buffer *buf, const void *mapped) {
  if (!ctx || !buf) return fail(SULIMO_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (mapped && mapped != buf->host) return fail(SULIMO_HIP_ERR_ZERO_COPY, "pointer was not mapped from this buffer");
  return SULIMO_HIP_OK;
}

}  // extern "C"
