// Internal: the context object behind the C ABI.
//
// A context is one device and one stream; every entry point is ordered on
// that stream and only coli_cuda_sync blocks the host (the reference ABI's
// contract, c/backend_cuda.h:10-41).  What the context owns:
//   * BlockCache: the device allocator behind coli_cuda_malloc/free.  Blocks
//     freed by the caller go to an idle list and are handed out again in
//     stream order (every later use is queued behind every earlier one on the
//     same stream), so the steady state of a serving loop makes no hipMalloc
//     or hipFree calls at all.
//   * StageProfiler: the 8-stage MoE attribution of coli_cuda_profile_*.
//     Entry points drop stage marks on the stream; the time between two
//     consecutive marks belongs to the stage of the later one.
//   * grow-only scratch slots for the kernels' own workspaces.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <unordered_map>
#include <vector>

#include "shiftwing_moe.h"

namespace sw {

enum Scratch {
  kScrSetup = 0,   // reference grouped calls: route weights on the device
  kScrHidden,      // reference grouped calls: routed hidden activations
  kScrRouteOut,    // reference grouped calls: per-route down outputs
  kScrGate,        // reference shared-expert calls: hidden vectors, gate logits
  kScrUp,
  kScrWeight,
  kScrXPrep,       // many-token step: activation digits, routes, buckets
  kScrRouter,      // many-token step: router logit bounds
  kScrRoutes,      // many-token step: idx / weights / buckets
  kScrShared,      // three-kernel decode: shared expert int32 sums + h
  kScrStack,       // persistent decode: router records, exact logits, h records
  kScrBlock,       // MoE block: normalised activations and the MoE output
  kScrHead,        // output head: quantised normalised rows and their scales
  kScrMixer,       // Gated DeltaNet / GQA layers: staged inputs, projections, partials
  kScrCount
};

// The reference backend's eight MoE stages (profile_snapshot's stage_ms[]).
enum ProfStage {
  kStageSetup = 0,
  kStageRoutedHidden = 1,
  kStageRoutedDown = 2,
  kStageReduce = 3,
  kStageSharedHidden = 4,
  kStageSharedScale = 5,
  kStageSharedDown = 6,
  kStageDownload = 7,
  kStageStamped = 8,  // internal: a persistent launch, split by its own stamps
};

struct BlockCache {
  bool enabled = true;                        // false: plain hipMalloc / hipFree
  std::unordered_map<void *, size_t> live;    // caller-held block -> size
  std::multimap<size_t, void *> idle;         // reusable in stream order
  size_t live_bytes = 0, idle_bytes = 0;
};

struct StageProfiler {
  bool on = false;
  struct Mark {
    hipEvent_t ev;
    int stage;  // -1: the transaction's opening mark
  };
  std::vector<hipEvent_t> events;  // created once, reused by every transaction
  std::vector<Mark> marks;         // the open transaction, in stream order
  bool open = false, downloaded = false;
  double ms[8] = {};
  unsigned long long transactions = 0;
  // persistent decode kernel: its stages come from device clock stamps
  unsigned long long *stamps = nullptr;  // device [layers][CUs][8]
  size_t stamp_words = 0;
  int stamp_layers = 0;                  // layers of the launch awaiting attribution
};

}  // namespace sw

struct ColiCuda {
  int device = 0;
  int major = 0, minor = 0;
  int sm_count = 0;
  int shared_per_block = 0;
  char name[192] = {};
  hipStream_t stream = nullptr;
  sw::BlockCache cache;
  sw::StageProfiler prof;
  void *scratch[sw::kScrCount] = {};
  size_t scratch_cap[sw::kScrCount] = {};
  // stream timer and MoE stage timing
  hipEvent_t timer_event[2] = {};
  int moe_timing = 0;
  hipEvent_t moe_event[8] = {};
  double moe_ms[8] = {};
  unsigned long long moe_calls = 0;
  double moe_dec_ms[3] = {};
  unsigned long long moe_dec_calls = 0;
  int moe_generic_only = 0;  // single-token steps take the many-token kernels
  int moe_decode_mode = 0;   // 0 persistent stack kernel (default), 1 three-kernel decode
  int moe_item_tokens = 0;   // many-token steps: tokens per expert item (0 automatic, 8, 16)
  // persistent stack kernel (moe_stack.hip): counters / integer sums in two
  // parity sets (the call state that selects them is device-side), the
  // device layer table, the abort status
  void *stack_sync = nullptr;
  int stack_cap_layers = 0;
  void *stack_table_dev = nullptr;
  size_t stack_table_cap = 0;
  void *stack_table_host = nullptr;
  int stack_table_n = 0;
  void *stack_abort = nullptr;
  unsigned *stack_abort_host = nullptr, *stack_abort_host_dev = nullptr;
  unsigned long long *stack_trace = nullptr;  // optional stage stamps (coli_cuda_moe_stack_trace)
  size_t stack_trace_words = 0;
  // dynamic LDS bytes per format (index 0: int3, 1: int4) at which a compute
  // unit was last found to hold one workgroup of the kernel (0: not checked)
  size_t stack_fit_lds[2] = {0, 0};
  // fault drill (coli_cuda_moe_stack_drill), armed until the next launch:
  // workgroups kept out, wait limit in 100 MHz ticks
  int stack_drill_absent = 0;
  long long stack_drill_ticks = 0;
  // device address of the fixed scratch of coli_cuda_idot_q8_gemm_noalloc
  void *noalloc_scratch = nullptr;
};

namespace sw {

// Error reporting: set the calling thread's error text, return -1.
int fail_hip(const char *where, hipError_t e);
int fail_arg(const char *fmt, ...);
// -1 with the error text when the last launch on this thread failed.
int launch_status(const char *where);
// Grow-only scratch owned by the context (released by coli_cuda_destroy).
int ensure_scratch(ColiCuda *ctx, Scratch which, size_t bytes, const char *where);

// Stage profiler (no-ops unless CUDA_PROFILE_STAGES is set at create).
void prof_open(ColiCuda *ctx);                 // a MoE transaction starts here
void prof_mark(ColiCuda *ctx, ProfStage s);    // time since the last mark is stage s
bool prof_active(const ColiCuda *ctx);         // a transaction is open
// The persistent kernel's stamp buffer for a launch of `layers` layers (or
// nullptr when profiling is off or the buffer cannot be had).
unsigned long long *prof_stamp_buffer(ColiCuda *ctx, int layers, size_t *words);
// Charge a finished persistent launch's stamps to the stages (stream drained).
void prof_flush_stamps(ColiCuda *ctx);

// Fetch (once per device) the device address of the no-alloc entry point's
// fixed scratch; called by coli_cuda_create with the device current.
int noalloc_bind(ColiCuda *ctx);

}  // namespace sw
