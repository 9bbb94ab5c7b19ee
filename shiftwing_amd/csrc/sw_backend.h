// Internal: the context object behind the C ABI and its error / scratch
// helpers.  Semantics follow c/backend_cuda.cu:47-177 (thread-local error
// text, 0/-1 returns, one non-blocking stream per context, backend-owned
// scratch grown on demand and freed by coli_cuda_destroy).
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include "shiftwing_moe.h"

namespace sw {

enum Scratch {
  kScrSetup = 0,   // per-call pointer tables / route maps (legacy grouped calls)
  kScrHidden,      // routed hidden activations
  kScrRouteOut,    // per-route down outputs (legacy batch)
  kScrGate,        // shared / misc fp32 vectors
  kScrUp,
  kScrWeight,
  kScrXPrep,       // activation digits (fast path)
  kScrRouter,      // router logit bounds (fast path)
  kScrRoutes,      // idx / weights / buckets (fast path)
  kScrShared,      // shared expert int32 partials + h (fast path)
  kScrStack,       // persistent decode: router records, exact logits, h records
  kScrCount
};

}  // namespace sw

struct ColiCuda {
  int device;
  int major, minor;
  int sm_count;
  int shared_per_block;
  int async_alloc;
  char name[256];
  hipStream_t stream;
  void *scratch[sw::kScrCount];
  size_t scratch_cap[sw::kScrCount];
  // stage profiling (CUDA_PROFILE_STAGES=1), c/backend_cuda.cu:118-131
  int profile_stages, profile_pending, profile_shared_marked, profile_download_marked;
  hipEvent_t profile_event[9];
  double profile_ms[8];
  unsigned long long profile_transactions;
  // stream timer and MoE stage timing
  hipEvent_t timer_event[2];
  int moe_timing;
  hipEvent_t moe_event[8];
  double moe_ms[8];
  unsigned long long moe_calls;
  double moe_dec_ms[3];
  unsigned long long moe_dec_calls;
  int moe_generic_only;  // single-token steps take the many-token kernels
  int moe_decode_mode;   // 0 persistent stack kernel (default), 1 three-kernel decode
  // persistent stack kernel (moe_stack.hip): counters / integer sums in two
  // parity sets (the call state that selects them is device-side), the
  // device layer table, the abort status
  void *stack_sync;
  int stack_cap_layers;
  void *stack_table_dev;
  size_t stack_table_cap;
  void *stack_table_host;
  int stack_table_n;
  void *stack_abort;
  unsigned *stack_abort_host, *stack_abort_host_dev;
  unsigned long long *stack_trace;  // optional stage stamps (coli_cuda_moe_stack_trace)
  size_t stack_trace_words;
};

namespace sw {

int fail_hip(const char *where, hipError_t e);
int fail_arg(const char *fmt, ...);
int launch_status(const char *where);
// Grow-only scratch owned by the context (released by coli_cuda_destroy).
int ensure_scratch(ColiCuda *ctx, Scratch which, size_t bytes, const char *where);

}  // namespace sw
