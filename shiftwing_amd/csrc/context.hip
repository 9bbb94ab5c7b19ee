// The ColiCuda context: device probe, the context stream, the stream-ordered
// block cache behind coli_cuda_malloc/free, host staging, stream timers and
// the 8-stage MoE profiler.  Entry points and their 0 / -1 convention follow
// the reference ABI (c/backend_cuda.h:13-40); the design below is this
// library's own:
//
//  * One context = one device and one default-priority stream.  Nothing here
//    blocks the host except coli_cuda_sync, coli_cuda_timer_stop, the
//    profile calls and the allocator's out-of-memory path.
//  * Device allocations go through a block cache.  A freed block is parked
//    on an idle list and handed to a later malloc of about the same size;
//    since every use of every block is ordered on the context stream, a block
//    can be reused before the stream has drained.  The cache is trimmed
//    (stream drained, idle blocks released) only when hipMalloc reports that
//    the device is full.  CUDA_ASYNC_ALLOC=0 (the reference backend's switch
//    between its stream-ordered and synchronous allocators) turns the cache
//    off: every malloc is a hipMalloc and every free a hipFree.
//  * Stage profiling (CUDA_PROFILE_STAGES=1, the reference's switch) keeps a
//    list of (event, stage) marks per MoE transaction.  The time between two
//    consecutive marks is charged to the stage of the later mark, so any
//    sequence of entry points (the reference's grouped + shared calls, or
//    this library's fused step) lands in the same 8 stages.  The persistent
//    decode kernel is one launch; its stages come from its own device-clock
//    stamps.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <vector>

#include "sw_backend.h"
#include "sw_stack.h"

namespace {

// The calling thread's error text (the ABI reports errors per thread).
thread_local char t_error[512];

void set_error(const char *fmt, va_list ap) { vsnprintf(t_error, sizeof(t_error), fmt, ap); }

int env_flag(const char *name, int dflt) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) != 0 : dflt;
}

// Sizes are rounded so that near-equal requests share blocks: 256 B steps
// below 64 KiB, 64 KiB steps below 64 MiB, 2 MiB steps above.
size_t block_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  const size_t step = bytes < (64u << 10) ? 256 : bytes < (64u << 20) ? (64u << 10) : (2u << 20);
  return (bytes + step - 1) / step * step;
}

}  // namespace

namespace sw {

int fail_arg(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  set_error(fmt, ap);
  va_end(ap);
  return -1;
}

int fail_hip(const char *where, hipError_t e) {
  return fail_arg("%s failed: %s (%s)", where, hipGetErrorName(e), hipGetErrorString(e));
}

int launch_status(const char *where) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  return fail_hip(where, e);
}

int ensure_scratch(ColiCuda *ctx, Scratch which, size_t bytes, const char *where) {
  if (ctx->scratch_cap[which] >= bytes) return 0;
  // the old slot may still be read by queued kernels
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return fail_hip(where, e);
  if (ctx->scratch[which]) (void)hipFree(ctx->scratch[which]);
  ctx->scratch[which] = nullptr;
  ctx->scratch_cap[which] = 0;
  const size_t cap = block_size(bytes);
  e = hipMalloc(&ctx->scratch[which], cap);
  if (e != hipSuccess) return fail_hip(where, e);
  ctx->scratch_cap[which] = cap;
  return 0;
}

// ---- block cache ------------------------------------------------------------

static void cache_trim(ColiCuda *ctx) {
  BlockCache &c = ctx->cache;
  if (c.idle.empty()) return;
  (void)hipStreamSynchronize(ctx->stream);
  for (auto &kv : c.idle) (void)hipFree(kv.second);
  c.idle.clear();
  c.idle_bytes = 0;
}

static int cache_alloc(ColiCuda *ctx, void **out, size_t bytes) {
  BlockCache &c = ctx->cache;
  const size_t n = block_size(bytes);
  if (c.enabled) {
    // smallest idle block that fits, unless it would waste more than a quarter
    auto it = c.idle.lower_bound(n);
    if (it != c.idle.end() && it->first - n <= n / 4) {
      void *p = it->second;
      const size_t sz = it->first;
      c.idle.erase(it);
      c.idle_bytes -= sz;
      c.live.emplace(p, sz);
      c.live_bytes += sz;
      *out = p;
      return 0;
    }
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, n);
  if (e == hipErrorOutOfMemory && !c.idle.empty()) {
    (void)hipGetLastError();
    cache_trim(ctx);
    e = hipMalloc(&p, n);
  }
  if (e != hipSuccess) return fail_hip("coli_cuda_malloc: hipMalloc", e);
  c.live.emplace(p, n);
  c.live_bytes += n;
  *out = p;
  return 0;
}

static void cache_free(ColiCuda *ctx, void *p) {
  BlockCache &c = ctx->cache;
  auto it = c.live.find(p);
  if (it == c.live.end()) {
    // not a block of this context: release it directly
    (void)hipFree(p);
    return;
  }
  const size_t sz = it->second;
  c.live.erase(it);
  c.live_bytes -= sz;
  if (!c.enabled) {
    (void)hipFree(p);
    return;
  }
  c.idle.emplace(sz, p);
  c.idle_bytes += sz;
}

// ---- stage profiler ---------------------------------------------------------

static hipEvent_t prof_event(StageProfiler &p, size_t i) {
  while (p.events.size() <= i) {
    hipEvent_t ev = nullptr;
    if (hipEventCreate(&ev) != hipSuccess) return nullptr;
    p.events.push_back(ev);
  }
  return p.events[i];
}

static void prof_record(ColiCuda *ctx, int stage) {
  StageProfiler &p = ctx->prof;
  hipEvent_t ev = prof_event(p, p.marks.size());
  if (!ev || hipEventRecord(ev, ctx->stream) != hipSuccess) {
    p.open = false;  // an incomplete transaction is dropped, not misreported
    p.marks.clear();
    return;
  }
  p.marks.push_back({ev, stage});
}

void prof_open(ColiCuda *ctx) {
  StageProfiler &p = ctx->prof;
  if (!p.on) return;
  p.marks.clear();
  p.open = true;
  p.downloaded = false;
  p.stamp_layers = 0;
  prof_record(ctx, -1);
}

void prof_mark(ColiCuda *ctx, ProfStage s) {
  StageProfiler &p = ctx->prof;
  if (p.on && p.open) prof_record(ctx, (int)s);
}

bool prof_active(const ColiCuda *ctx) { return ctx->prof.on && ctx->prof.open; }

unsigned long long *prof_stamp_buffer(ColiCuda *ctx, int layers, size_t *words) {
  StageProfiler &p = ctx->prof;
  *words = 0;
  if (!p.on || !p.open) return nullptr;
  const size_t need = (size_t)layers * (size_t)ctx->sm_count * 8;
  if (p.stamp_words < need) {
    if (p.stamps) (void)hipFree(p.stamps);
    p.stamps = nullptr;
    p.stamp_words = 0;
    if (hipMalloc(&p.stamps, need * sizeof(unsigned long long)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    p.stamp_words = need;
  }
  p.stamp_layers = layers;
  *words = need;
  return p.stamps;
}

// Stamps of one persistent launch, per layer and workgroup: layer start,
// router/shared done, router records in, selection done, routed gate/up done,
// hidden barrier passed, down done, layer barrier passed.  Per layer the
// latest workgroup to reach each point fixes it; the spans between points go
// to: setup (router + record exchange), shared hidden (selection with the
// shared hidden vector), routed hidden (gate/up), routed down (hidden barrier
// and down with the shared down), reduce (the layer barrier).
void prof_flush_stamps(ColiCuda *ctx) {
  StageProfiler &p = ctx->prof;
  const int L = p.stamp_layers, NB = ctx->sm_count;
  p.stamp_layers = 0;
  if (L <= 0 || !p.stamps) return;
  std::vector<unsigned long long> h((size_t)L * NB * 8);
  if (hipMemcpy(h.data(), p.stamps, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
    return;
  static const int to_stage[7] = {kStageSetup, kStageSetup, kStageSharedHidden, kStageRoutedHidden,
                                  kStageRoutedDown, kStageRoutedDown, kStageReduce};
  for (int l = 0; l < L; l++) {
    unsigned long long pt[8];
    for (int k = 0; k < 8; k++) {
      unsigned long long m = 0;
      for (int b = 0; b < NB; b++) m = std::max(m, h[((size_t)l * NB + b) * 8 + k]);
      pt[k] = m;
    }
    for (int k = 0; k < 7; k++) {
      const double ms = pt[k + 1] > pt[k] ? (double)(pt[k + 1] - pt[k]) * 1e-5 : 0.0;  // 100 MHz
      p.ms[to_stage[k]] += ms;
    }
  }
}

static void prof_close(ColiCuda *ctx) {
  StageProfiler &p = ctx->prof;
  if (!p.open || !p.downloaded) return;
  // a persistent launch's own span is not charged: its stamps split it
  for (size_t i = 1; i < p.marks.size(); i++) {
    if (p.marks[i].stage == kStageStamped) continue;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, p.marks[i - 1].ev, p.marks[i].ev) == hipSuccess) p.ms[p.marks[i].stage] += ms;
  }
  prof_flush_stamps(ctx);
  p.transactions++;
  p.open = false;
  p.downloaded = false;
  p.marks.clear();
}

}  // namespace sw

using namespace sw;

// ---------------------------------------------------------------------------
// context (backend_cuda.h:13-22)
// ---------------------------------------------------------------------------
extern "C" const char *coli_cuda_last_error(void) { return t_error[0] ? t_error : "no error"; }

extern "C" int coli_cuda_create(ColiCuda **out, int device) {
  if (!out) return fail_arg("coli_cuda_create: null output pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return fail_hip("hipGetDeviceCount", e);
  if (device < 0 || device >= n) return fail_arg("coli_cuda_create: device %d, %d device(s) visible", device, n);
  if ((e = hipSetDevice(device)) != hipSuccess) return fail_hip("hipSetDevice", e);
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return fail_hip("hipGetDeviceProperties", e);
  ColiCuda *ctx = new (std::nothrow) ColiCuda();
  if (!ctx) return fail_arg("coli_cuda_create: out of host memory");
  ctx->device = device;
  ctx->major = prop.major;
  ctx->minor = prop.minor;
  ctx->sm_count = prop.multiProcessorCount;
  ctx->shared_per_block = (int)prop.sharedMemPerBlock;
  // The marketing name can be empty on these hosts: always report the ISA,
  // the compute units and the HBM size.
  char arch[64];
  snprintf(arch, sizeof(arch), "%s", prop.gcnArchName);
  if (char *colon = strchr(arch, ':')) *colon = 0;
  snprintf(ctx->name, sizeof(ctx->name), "%s%s%s (%d CUs, %.0f GiB HBM)", prop.name[0] ? prop.name : "AMD GPU",
           " ", arch, prop.multiProcessorCount, (double)prop.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
  if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
    delete ctx;
    return fail_hip("hipStreamCreateWithFlags", e);
  }
  if (noalloc_bind(ctx)) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return -1;
  }
  ctx->cache.enabled = env_flag("CUDA_ASYNC_ALLOC", 1) != 0;
  ctx->prof.on = env_flag("CUDA_PROFILE_STAGES", 0) != 0;
  t_error[0] = 0;
  *out = ctx;
  return 0;
}

extern "C" void coli_cuda_destroy(ColiCuda *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  cache_trim(ctx);  // blocks the caller still holds are the caller's
  for (void *p : ctx->scratch)
    if (p) (void)hipFree(p);
  stack_release(ctx);
  for (hipEvent_t ev : ctx->prof.events) (void)hipEventDestroy(ev);
  if (ctx->prof.stamps) (void)hipFree(ctx->prof.stamps);
  for (hipEvent_t ev : ctx->timer_event)
    if (ev) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : ctx->moe_event)
    if (ev) (void)hipEventDestroy(ev);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" const char *coli_cuda_device_name(const ColiCuda *ctx) { return ctx ? ctx->name : ""; }

extern "C" int coli_cuda_compute_capability(const ColiCuda *ctx, int *major, int *minor) {
  if (!ctx || !major || !minor) return fail_arg("coli_cuda_compute_capability: null argument");
  *major = ctx->major;
  *minor = ctx->minor;
  return 0;
}

extern "C" int coli_cuda_device_limits(const ColiCuda *ctx, int *sm_count, int *shared_per_block) {
  if (!ctx) return fail_arg("coli_cuda_device_limits: null context");
  if (sm_count) *sm_count = ctx->sm_count;
  if (shared_per_block) *shared_per_block = ctx->shared_per_block;
  return 0;
}

extern "C" int coli_cuda_async_alloc_enabled(const ColiCuda *ctx) { return ctx && ctx->cache.enabled ? 1 : 0; }

// Free memory as this context sees it: the device's free bytes plus the idle
// blocks of its own cache, which its next allocations take first.
extern "C" int coli_cuda_memory_info(ColiCuda *ctx, size_t *free_bytes, size_t *total_bytes) {
  if (!ctx || !free_bytes || !total_bytes) return fail_arg("coli_cuda_memory_info: null argument");
  (void)hipSetDevice(ctx->device);
  const hipError_t e = hipMemGetInfo(free_bytes, total_bytes);
  if (e != hipSuccess) return fail_hip("hipMemGetInfo", e);
  *free_bytes += ctx->cache.idle_bytes;
  return 0;
}

// ---------------------------------------------------------------------------
// memory (backend_cuda.h:24-33)
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_malloc(ColiCuda *ctx, void **ptr, size_t bytes) {
  if (!ctx || !ptr) return fail_arg("coli_cuda_malloc: null argument");
  *ptr = nullptr;
  (void)hipSetDevice(ctx->device);
  return cache_alloc(ctx, ptr, bytes);
}

extern "C" void coli_cuda_free(ColiCuda *ctx, void *ptr) {
  if (!ctx || !ptr) return;
  (void)hipSetDevice(ctx->device);
  cache_free(ctx, ptr);
}

extern "C" int coli_cuda_malloc_host(ColiCuda *ctx, void **ptr, size_t bytes) {
  if (!ctx || !ptr) return fail_arg("coli_cuda_malloc_host: null argument");
  *ptr = nullptr;
  const hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault);
  return e == hipSuccess ? 0 : fail_hip("hipHostMalloc", e);
}

extern "C" void coli_cuda_free_host(ColiCuda *ctx, void *ptr) {
  if (ctx && ptr) (void)hipHostFree(ptr);
}

// Registering memory the caller already allocated is not offered on these
// hosts: the call fails, and the reference host code then keeps its pageable
// path (c/qwen.c treats the failure as "not registered").  Host buffers that
// must be page-locked come from coli_cuda_malloc_host.
extern "C" int coli_cuda_host_register(ColiCuda *ctx, void *ptr, size_t bytes) {
  if (!ctx || !ptr || !bytes) return fail_arg("coli_cuda_host_register: null argument");
  return fail_arg("coli_cuda_host_register: page-locking existing host memory is not available here; "
                  "use coli_cuda_malloc_host");
}

extern "C" void coli_cuda_host_unregister(ColiCuda *ctx, void *ptr) {
  (void)ctx;
  (void)ptr;
}

static int stream_copy(ColiCuda *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                       const char *what) {
  if (!ctx || !dst || !src) return fail_arg("%s: null argument", what);
  if (!bytes) return 0;
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
  return e == hipSuccess ? 0 : fail_hip(what, e);
}

extern "C" int coli_cuda_upload(ColiCuda *ctx, void *dst, const void *src, size_t bytes) {
  return stream_copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, "coli_cuda_upload");
}

extern "C" int coli_cuda_download(ColiCuda *ctx, void *dst, const void *src, size_t bytes) {
  const int rc = stream_copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, "coli_cuda_download");
  if (rc == 0 && prof_active(ctx)) {
    prof_mark(ctx, kStageDownload);
    ctx->prof.downloaded = true;
  }
  return rc;
}

extern "C" int coli_cuda_copy(ColiCuda *ctx, void *dst, const void *src, size_t bytes) {
  return stream_copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, "coli_cuda_copy");
}

extern "C" int coli_cuda_memset(ColiCuda *ctx, void *dst, int value, size_t bytes) {
  if (!ctx || !dst) return fail_arg("coli_cuda_memset: null argument");
  const hipError_t e = hipMemsetAsync(dst, value, bytes, ctx->stream);
  return e == hipSuccess ? 0 : fail_hip("coli_cuda_memset", e);
}

extern "C" int coli_cuda_sync(ColiCuda *ctx) {
  if (!ctx) return fail_arg("coli_cuda_sync: null context");
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return fail_hip("coli_cuda_sync", e);
  if (stack_check_abort(ctx)) return -1;
  prof_close(ctx);
  return 0;
}

// ---------------------------------------------------------------------------
// stage profile (backend_cuda.h:35-40)
// ---------------------------------------------------------------------------
extern "C" void coli_cuda_profile_reset(ColiCuda *ctx) {
  if (!ctx || !ctx->prof.on) return;
  (void)hipStreamSynchronize(ctx->stream);
  StageProfiler &p = ctx->prof;
  std::fill(p.ms, p.ms + 8, 0.0);
  p.transactions = 0;
  p.open = p.downloaded = false;
  p.marks.clear();
  p.stamp_layers = 0;
}

extern "C" int coli_cuda_profile_snapshot(ColiCuda *ctx, unsigned long long *transactions,
                                          double stage_ms[8]) {
  if (!ctx || !transactions || !stage_ms) return fail_arg("coli_cuda_profile_snapshot: null argument");
  if (!ctx->prof.on) {
    *transactions = 0;
    std::fill(stage_ms, stage_ms + 8, 0.0);
    return 1;  // profiling is off
  }
  if (coli_cuda_sync(ctx)) return -1;
  *transactions = ctx->prof.transactions;
  std::copy(ctx->prof.ms, ctx->prof.ms + 8, stage_ms);
  return 0;
}

// ---------------------------------------------------------------------------
// stream timer (HIP events on the context stream)
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_timer_start(ColiCuda *ctx) {
  if (!ctx) return fail_arg("coli_cuda_timer_start: null context");
  for (hipEvent_t &ev : ctx->timer_event)
    if (!ev) {
      const hipError_t e = hipEventCreate(&ev);
      if (e != hipSuccess) return fail_hip("hipEventCreate", e);
    }
  const hipError_t e = hipEventRecord(ctx->timer_event[0], ctx->stream);
  return e == hipSuccess ? 0 : fail_hip("coli_cuda_timer_start", e);
}

extern "C" int coli_cuda_timer_stop(ColiCuda *ctx, float *ms) {
  if (!ctx || !ms || !ctx->timer_event[0]) return fail_arg("coli_cuda_timer_stop: timer not started");
  hipError_t e = hipEventRecord(ctx->timer_event[1], ctx->stream);
  if (e == hipSuccess) e = hipEventSynchronize(ctx->timer_event[1]);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->timer_event[0], ctx->timer_event[1]);
  return e == hipSuccess ? 0 : fail_hip("coli_cuda_timer_stop", e);
}
