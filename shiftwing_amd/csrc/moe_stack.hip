// Batch-1 decode through a stack of HBM-resident MoE layers in ONE persistent
// kernel (moe_forward, c/qwen.c:3717-3739, applied layer after layer).
//
// One workgroup of 512 threads per CU, all resident for the whole call.  Per
// layer l, every workgroup runs four stages separated by grid exchanges:
//
//   R  router rows (fp64 logit + rigorous bound of the reference's serial fp32
//      dot, c/qwen.c:1674) for the rows this workgroup owns (row r belongs to
//      workgroup r % NB), one shared-expert gate/up IDOT task (exact int32
//      dots, c/qwen.c:1696-1705, summed over k-slices with integer atomics),
//      the activation digits of x for the routed GEMV, and the thread's part
//      of the shared gate's logit.  Each workgroup's shared sums go out first;
//      its router records follow, tagged with the layer (no barrier: readers
//      read the records until all carry the tag).
//   S  every workgroup selects the top-k itself from the published records
//      (router_topk, c/qwen.c:3421-3426): certified by the bounds, else by
//      the exact fp32 chains of the ambiguous experts (computed by the rows'
//      owners and exchanged through one more barrier), else by the reference's
//      full computation on every expert's exact chain.  Meanwhile wave 1
//      computes this workgroup's Ish/NB values of the shared hidden vector
//      (SwiGLU of the counted sums) and publishes them tagged, and waves 2..7
//      copy the shared down rows of the workgroup's output tile into LDS.
//   G  routed gate/up: units (route, 16 rows) over the grid; each unit's
//      h = silu(g) * u (c/qwen.c:3419) is quantised into two int8 digits per
//      16-value chunk and published as a 48-byte record.  At the end, the
//      whole shared hidden vector (copied in a few items earlier), its qrow_i8
//      and the shared down dots of the workgroup's output rows.
//   -- barrier "h".
//   D  routed down + combine for 16 output rows per task, in moe_forward's
//      order (fma over k in route order, then shared * gate).
//   -- barrier "y" (strict decode order: layer l+1 starts after layer l).
//
// Weights that do not depend on the token (the next layer's router rows and
// shared gate/up tile) are loaded into registers while stage D computes; the
// down tiles of the selected experts are loaded into LDS before the "h"
// barrier.
//
// Cross-workgroup data is published with device-scope stores and atomics and
// read with device-scope loads; barriers are two-level counters (8 groups,
// then one top counter) and a release word.  Counters and integer sums come in two parity sets:
// a call uses set p and clears set 1-p for the next call.  The call state
// (parity, dirty extents, the running layer count behind the tags) lives in
// device memory and is advanced by the kernel itself, so no call needs a
// memset and a captured graph replays correctly.  Every wait is bounded in
// wall-clock time: on expiry the kernel raises an abort flag, every workgroup
// leaves, and the host reports the error at the next sync.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "sw_backend.h"
#include "sw_device.h"
#include "sw_moe_kernels.h"
#include "sw_moe_layer.h"
#include "sw_stack.h"
#include "sw_lds_dma.h"

using namespace sw;

namespace {

constexpr int kT = 512;          // threads per workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kMaxK = kStackMaxK;
constexpr int kRSlots = 3;       // router rows per workgroup held in registers
constexpr int kNch = 2;          // 2048-float chunks per router row (H <= 4096)
constexpr int kMaxAmbig = 64;    // experts the targeted exact selection can take
constexpr int kLine = 32;        // words between counters (one 128-byte line)
constexpr int kBars = 5;         // barriers per layer: lb, exact-1, exact-2, h, y
constexpr int kBarWords = 10 * kLine;  // release word, 8 group counters, top counter
constexpr int kRecWords = 12;    // h chunk record: d1[16] d2[16] (8 words) | A B Q1 Q2
constexpr int kGMax = 4;         // stage G: groups per wave and unit
#ifndef SW_STACK_GRING
#define SW_STACK_GRING 2
#endif
constexpr int kGRing = SW_STACK_GRING;  // stage G: ring slots per wave
constexpr int kGHead = 2560;     // stage G: partial sums and digit staging before the rings
enum { kBarLb = 0, kBarEx1, kBarEx2, kBarH, kBarY };

// Layer pointers as the kernel receives them: typed as device-global memory,
// so that every access through them compiles to global (not flat) memory
// instructions (a flat access also counts as an LDS access, so every later
// wait for LDS would wait for it too).  LayerPtrs is the same set as the
// kernel uses it.
#define SW_G __attribute__((address_space(1)))
struct LayerRef {
  const SW_G float *router, *sgate;
  const SW_G signed char *gq, *uq, *dq;
  const SW_G float *gs, *us, *ds;
  const SW_G unsigned char *experts;  // routed experts' records (sw_expert_layout.h)
  SW_G unsigned long long *stats;
  int mode, pad;
};
struct LayerPtrs {
  const SW_G float *router, *sgate;
  const SW_G signed char *gq, *uq, *dq;
  const SW_G float *gs, *us, *ds;
  const SW_G unsigned char *experts;
  SW_G unsigned long long *stats;
  int mode;
};

// Device-side call state: [0..1] layers run by every call so far (64-bit),
// [2] the parity set this call uses, [3..4] layers and [5..6] integer-sum
// words the last call of each parity dirtied.
enum { kStLayersLo = 0, kStLayersHi, kStParity, kStDirtyN0, kStDirtyN1, kStDirtyAcc0, kStDirtyAcc1, kStWords };
struct CallState {
  int parity;
  unsigned tag0;  // layer 0's tag (1..255) in the exchanged words
};

struct StackArgs {
  LayerRef one;                 // n == 1
  const SW_G LayerRef *table;   // n > 1
  int n;
  int H, E, K, I, Ish, fmt, ngh, ngi, Hp, nrt_i, nch;
  size_t expert_bytes, gu_bytes;  // one expert's records, its gate/up records (sw_expert_layout.h)
  int NB, rslots, KQ, n_sh_tasks, shkc;
  const float *x;
  size_t xs;
  float *y;
  size_t ys;
  int *route_idx;
  float *route_w;
  double *rec;          // [E+1][2] logit, bound
  float *ex;            // [E] exact logits
  unsigned *hd;         // [K][ngi*8][kRecWords]
  unsigned long long *hs;  // [Ish] the shared hidden vector: (layer tag << 32) | f32 bits
  float *shv;           // [H] shared down values computed by a paired workgroup (see g_pairing)
  unsigned long long *acc;  // [layer][parity][2*Ish] counted shared gate/up sums
  unsigned *bars;       // [layer][parity][kBars][kBarWords]
  size_t acc_stride;    // words per (layer, parity) acc block
  unsigned *state;      // call state, advanced by every call (StackState)
  unsigned *abort_word; // device
  unsigned *abort_host; // host-mapped status
  long long spin_ticks; // wall-clock budget of one wait (100 MHz ticks)
  int absent;           // fault drill: the last `absent` workgroups stay out (0 otherwise)
  unsigned long long *trace;  // optional stage stamps [layer][NB][kStamps]
  size_t trace_words;
};


// The kernel arguments, read again from the kernel-argument segment (scalar
// loads through the constant cache): laundered so that no stage keeps every
// field live in scalar registers across the whole layer loop.
__device__ __forceinline__ StackArgs kargs() {
  typedef const __attribute__((address_space(4))) StackArgs KA;
  KA *p = (KA *)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *(const StackArgs *)(const void *)p;
}

// Optional per-stage wall-clock stamps (100 MHz device clock), thread 0 of
// every workgroup: layer start, R done, lb passed, S done, G done, h passed,
// D done, y passed.
constexpr int kStamps = 8;
__device__ __forceinline__ void stamp(const StackArgs &a, int l, int k) {
  if (__builtin_expect(a.trace != nullptr, 0) && threadIdx.x == 0) {
    const size_t i = ((size_t)l * a.NB + blockIdx.x) * kStamps + k;
    if (i < a.trace_words) a.trace[i] = wall_clock64();
  }
}

// ---------------------------------------------------------------------------
// device-scope access
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned ld_agent(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_agent(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_agent(const unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_agent(const double *p) {
  return __longlong_as_double((long long)ld_agent((const unsigned long long *)p));
}
// A device-scope load that waits for itself inside the same statement: the
// compiler sees no load in flight afterwards, so it places no wait for it
// elsewhere (such a wait would also wait for every copy issued before it).
__device__ __forceinline__ unsigned long long ld_agent_sync(const unsigned long long *p) {
  unsigned long long v;
  asm volatile("global_load_dwordx2 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}
// A returning exchange: once its value is back, the word is visible to every
// device-scope load on the device.  The xor of the returns feeds published().
__device__ __forceinline__ unsigned pub(unsigned *p, unsigned v) { return atomicExch(p, v); }
__device__ __forceinline__ unsigned pub(double *p, double v) {
  unsigned long long o = atomicExch((unsigned long long *)p, (unsigned long long)__double_as_longlong(v));
  return (unsigned)o ^ (unsigned)(o >> 32);
}
__device__ __forceinline__ void published(unsigned dep) {
  asm volatile("" ::"v"(dep));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Workgroup barrier for LDS traffic only.  __syncthreads() also waits for
// every outstanding global load of the wave (vmcnt(0)), which would drain the
// weight tiles kept in flight across the barrier; global ordering is made
// explicit where it is needed (published(), the DMA waits).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


// Field by field, so that the kernel-argument copy and the table copy are
// never merged into one flat pointer.
__device__ __forceinline__ LayerPtrs layer_ref(const StackArgs &a, int l) {
  LayerPtrs p;
  const bool one = a.n == 1;
#define SW_FIELD(f) p.f = one ? a.one.f : a.table[l].f
  SW_FIELD(router);
  SW_FIELD(sgate);
  SW_FIELD(gq);
  SW_FIELD(uq);
  SW_FIELD(dq);
  SW_FIELD(gs);
  SW_FIELD(us);
  SW_FIELD(ds);
  SW_FIELD(experts);
  SW_FIELD(stats);
#undef SW_FIELD
  p.mode = one ? a.one.mode : a.table[l].mode;
  return p;
}
// A layer's pointers as words in LDS (kept for this layer and the next one,
// so that no stage waits on a load of the layer table): every lane reads the
// same words, made scalar again.
constexpr int kRefWords = (int)(sizeof(LayerRef) / 4);
static_assert(sizeof(LayerRef) % 4 == 0 && kRefWords <= 64, "layer pointers: one word per lane of a wave");
__device__ __forceinline__ LayerPtrs layer_ref_lds(const unsigned *w) {
  auto u32 = [&](size_t off) { return (unsigned)__builtin_amdgcn_readfirstlane((int)w[off / 4]); };
  auto p64 = [&](size_t off) { return ((unsigned long long)u32(off + 4) << 32) | u32(off); };
  LayerPtrs p;
  p.router = (const SW_G float *)p64(offsetof(LayerRef, router));
  p.sgate = (const SW_G float *)p64(offsetof(LayerRef, sgate));
  p.gq = (const SW_G signed char *)p64(offsetof(LayerRef, gq));
  p.uq = (const SW_G signed char *)p64(offsetof(LayerRef, uq));
  p.dq = (const SW_G signed char *)p64(offsetof(LayerRef, dq));
  p.gs = (const SW_G float *)p64(offsetof(LayerRef, gs));
  p.us = (const SW_G float *)p64(offsetof(LayerRef, us));
  p.ds = (const SW_G float *)p64(offsetof(LayerRef, ds));
  p.experts = (const SW_G unsigned char *)p64(offsetof(LayerRef, experts));
  p.stats = (SW_G unsigned long long *)p64(offsetof(LayerRef, stats));
  p.mode = (int)u32(offsetof(LayerRef, mode));
  return p;
}
// word i of layer l's pointers from the kernel arguments or the layer table
__device__ __forceinline__ unsigned layer_ref_word(const StackArgs &a, int l, int i) {
  const __attribute__((address_space(4))) unsigned *one =
      (const __attribute__((address_space(4))) unsigned *)__builtin_amdgcn_kernarg_segment_ptr() +
      offsetof(StackArgs, one) / 4;
  return a.n == 1 ? one[i] : ((const SW_G unsigned *)(a.table + l))[i];
}
__device__ __forceinline__ unsigned *bar_of(const StackArgs &a, const CallState &cs, int l, int which) {
  return a.bars + ((size_t)(l * 2 + cs.parity) * kBars + which) * kBarWords;
}

// ---------------------------------------------------------------------------
// Bounded waits and the two-level grid barrier (thread 0 acts; the caller
// brackets with __syncthreads and distributes the result through LDS).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool wait_ge(const unsigned *p, unsigned target, const StackArgs &a) {
  const long long t0 = (long long)wall_clock64();
  for (unsigned it = 0;; it++) {
    if (ld_agent(p) >= target) return true;
    if ((it & 31) == 31) {
      if (__builtin_expect(ld_agent(a.abort_word) != 0, 0)) return false;
      if (__builtin_expect((long long)wall_clock64() - t0 > a.spin_ticks, 0)) {
        atomicMax(a.abort_word, 1u);
        __hip_atomic_store(a.abort_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Counted integer sums.  A shared gate/up row's sum has KQ parts (one per
// k-range task); each part is added as (v + 2^32) + 2^48, so the word holds
// the number of parts in bits 48.. and the biased sum below: the sum is exact
// (|sum| < 2^31, at most 255 parts) and a reader knows when it is complete.
__device__ __forceinline__ unsigned long long acc_term(int v) {
  return (unsigned long long)((long long)v + (1ll << 32)) + (1ull << 48);
}
__device__ __forceinline__ int acc_parts(unsigned long long w) { return (int)(w >> 48); }
__device__ __forceinline__ int acc_sum(unsigned long long w) {
  return (int)((long long)(w & ((1ull << 48) - 1)) - ((long long)(w >> 48) << 32));
}

// Tagged words.  A word exchanged between workgroups within a layer carries
// the layer's tag (1..255; consecutive layers, also across calls, differ) in
// its low byte, so a reader needs no barrier: it reads the words themselves
// until every one shows the tag.  64-bit words are read and written whole.
// Between calls every tagged word is zero (never a tag): each call clears
// what it wrote once no one reads it any more, fresh scratch is cleared, and
// so is the scratch of an aborted call.
__device__ __forceinline__ unsigned layer_tag(const CallState &cs, int l) {
  return 1u + (cs.tag0 - 1u + (unsigned)l) % 255u;
}
__device__ __forceinline__ unsigned long long with_tag(unsigned long long bits, unsigned tag) {
  return (bits & ~0xFFull) | tag;
}
__device__ __forceinline__ bool has_tag(unsigned long long v, unsigned tag) { return (unsigned)(v & 0xFFull) == tag; }
// A reader re-reads all of its words not yet tagged at once (one memory
// round trip per round) until every one is.  Rounds are bounded: true when
// the wait started at t0 must end (the abort word is set, or the time is up;
// then every workgroup leaves through the abort word).
__device__ __forceinline__ bool wait_expired(long long t0, const StackArgs &a) {
  if (__builtin_expect(ld_agent(a.abort_word) != 0, 0)) return true;
  if (__builtin_expect((long long)wall_clock64() - t0 > a.spin_ticks, 0)) {
    atomicMax(a.abort_word, 1u);
    __hip_atomic_store(a.abort_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return true;
  }
  return false;
}

// arrive: the workgroup's published words must have returned already.  The
// last arriver of each group of workgroups (b % 8) counts its group on the top
// counter; the last group's arriver then stores the release word, which the
// waiters poll (a word written once, not a counter taking 8 additions).
__device__ __forceinline__ void bar_arrive(unsigned *bar, int NB) {
  const int g = blockIdx.x & 7;
  const unsigned cnt = (unsigned)((NB - 1 - g) / 8 + 1);
  const unsigned ng = (unsigned)(NB < 8 ? NB : 8);
  const unsigned old = atomicAdd(&bar[kLine * (1 + g)], 1u);
  if (old == cnt - 1) {
    const unsigned o2 = atomicAdd(&bar[kLine * 9], 1u);
    if (o2 == ng - 1) __hip_atomic_store(&bar[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
__device__ __forceinline__ bool bar_wait(unsigned *bar, const StackArgs &a) { return wait_ge(&bar[0], 1u, a); }

// ---------------------------------------------------------------------------
// wave helpers
// ---------------------------------------------------------------------------
// Inclusive prefix sums in lane order: within each 16-lane row (row_shr 1,
// 2, 4, 8), then over the rows (row_bcast15 into rows 1 and 3, row_bcast31
// into rows 2 and 3).
__device__ __forceinline__ float row16_inclusive_scan_f(float v) {
  v += SW_DPP_F(0.0f, v, 0x111, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x112, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x114, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x118, 0xF, true);
  return v;
}
__device__ __forceinline__ float wave_inclusive_scan_f(float v) {
  v = row16_inclusive_scan_f(v);
  v += SW_DPP_F(0.0f, v, 0x142, 0xA, false);
  v += SW_DPP_F(0.0f, v, 0x143, 0xC, false);
  return v;
}
// lane l receives lane l-1 (wave_shr 1; lane 0 receives 0)
__device__ __forceinline__ float dpp_wave_shr1_f(float v) { return SW_DPP_F(0.0f, v, 0x138, 0xF, true); }
// lane l receives lane l-1 within its 16-lane row (the row's lane 0 receives 0)
__device__ __forceinline__ float dpp_row_shr1_f(float v) { return SW_DPP_F(0.0f, v, 0x111, 0xF, true); }
// total of each 16-lane row, in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v += SW_DPP_F(0.0f, v, 0xB1, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x4E, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x141, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x140, 0xF, true);
  return v;
}
// Row shift left within each 16-lane row: lane l receives lane l+1 (the
// row's last lane receives 0).
__device__ __forceinline__ double dpp_row_shl1_d(double v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), 0x101, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), 0x101, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}
__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long v, int q) {
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, q);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), q);
  return ((unsigned long long)hi << 32) | lo;
}
// How many of lanes 0..n-1 hold a key above this lane's (n <= 64; lanes n..63
// hold 0, below every key).  Four independent compares per step: a chain of
// single broadcasts waits on each one's latency.
__device__ __forceinline__ int count_greater(unsigned long long v, int n) {
  int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
  for (int q = 0; q < n; q += 4) {
    r0 += readlane_u64(v, q) > v;
    r1 += readlane_u64(v, q + 1) > v;
    r2 += readlane_u64(v, q + 2) > v;
    r3 += readlane_u64(v, q + 3) > v;
  }
  return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ double readlane_d(double v, int q) {
  return __longlong_as_double((long long)readlane_u64((unsigned long long)__double_as_longlong(v), q));
}
// forward permute of a double: the lane whose byte address is pa receives v
__device__ __forceinline__ double permute_d(int pa, double v) {
  const int lo = __builtin_amdgcn_ds_permute(pa, __double2loint(v));
  const int hi = __builtin_amdgcn_ds_permute(pa, __double2hiint(v));
  return __hiloint2double(hi, lo);
}
// minimum / maximum over each 16-lane row, read from lane 0
#define SW_DPP_D_OP(v, ctrl, op)                                                     \
  {                                                                                  \
    const int lo_ = __builtin_amdgcn_update_dpp(0, __double2loint(v), ctrl, 0xF, 0xF, false); \
    const int hi_ = __builtin_amdgcn_update_dpp(0, __double2hiint(v), ctrl, 0xF, 0xF, false); \
    v = op(v, __hiloint2double(hi_, lo_));                                           \
  }
__device__ __forceinline__ double row16_min_d(double v) {
  SW_DPP_D_OP(v, 0xB1, fmin);
  SW_DPP_D_OP(v, 0x4E, fmin);
  SW_DPP_D_OP(v, 0x141, fmin);
  SW_DPP_D_OP(v, 0x140, fmin);
  return readlane_d(v, 0);
}
__device__ __forceinline__ double row16_max_d(double v) {
  SW_DPP_D_OP(v, 0xB1, fmax);
  SW_DPP_D_OP(v, 0x4E, fmax);
  SW_DPP_D_OP(v, 0x141, fmax);
  SW_DPP_D_OP(v, 0x140, fmax);
  return readlane_d(v, 0);
}
#undef SW_DPP_D_OP
__device__ __forceinline__ double order_margin(double a, double b, double mx) {
  return 0x1p-20 * (1.0 + fabs(a) + fabs(b) + 2.0 * fabs(mx));
}

// ---------------------------------------------------------------------------
// LDS layout (bytes): persistent per layer, then one stage-local union.
// ---------------------------------------------------------------------------
struct Lds {
  signed char *xd;   // [2][Hp] routed activation digits
  float4 *xgp;       // [ngh]
  signed char *xq;   // [Hp] IDOT quantisation of x
  unsigned char *u;  // stage-local union
};
__host__ __device__ inline size_t lds_fixed(int Hp, int ngh, int Ish) {
  return (((size_t)2 * Hp + 15) & ~(size_t)15) + (size_t)ngh * 16 + (((size_t)Hp + 15) & ~(size_t)15) + 16;
}
__device__ __forceinline__ Lds lds_carve(unsigned char *smem, int Hp, int ngh, int Ish) {
  Lds s;
  s.xd = (signed char *)smem;
  s.xgp = (float4 *)(smem + (((size_t)2 * Hp + 15) & ~(size_t)15));
  s.xq = (signed char *)(s.xgp + ngh);
  s.u = smem + lds_fixed(Hp, ngh, Ish);
  return s;
}

// The stage-local union (bytes from its start), by the stages that use it:
//   R      RStageLds at 0.
//   S      SelLds, the records (logit, bound) [E], the keys [E] and the exact
//          chains' products [kRSlots][H] from 0 (sel_end).  The shared down
//          rows of this workgroup's output tile (gdsh) are copied in during
//          stage S, past sel_end.
//   G      partials and digit staging (kGHead), the rings of gate/up records;
//          the shared hidden vector as tagged words (hsw, copied in near the
//          end); a paired workgroup's shared down rows (gdsh2, copied in
//          stage S).
//   D      (after the hidden barrier) the routed down records of the output
//          tile (dtile, copied while the barrier completes), h records and
//          partial sums over gdsh and what follows it.
struct ULayout {
  size_t ring, dtile, gdsh, hsw, gdsh2, hrec, part, end;
};
__host__ __device__ inline size_t sel_end(int E, int H);
__host__ __device__ inline ULayout u_layout(int E, int H, int K, int ngi, int Ish, int fmt) {
  auto al = [](size_t v) { return (v + 15) & ~(size_t)15; };
  const size_t rec = 2 * (size_t)tile_codes_bytes(fmt) + 128;
  const size_t bpl = fmt == 4 ? 16 : 12;
  ULayout u;
  u.ring = kGHead;
  u.dtile = al(u.ring + (size_t)kW * kGRing * rec);
  const size_t dend = u.dtile + (size_t)K * ngi * (64 * bpl + 64);
  const size_t s_end = sel_end(E, H);
  u.gdsh = al(dend > s_end ? dend : s_end);
  u.hsw = al(u.gdsh + (size_t)kTileRows * (Ish + 16));
  u.gdsh2 = al(u.hsw + (size_t)((Ish + 127) / 128) * 1024);
  const size_t g_end = u.gdsh2 + (size_t)kTileRows * (Ish + 16);
  u.hrec = u.gdsh;
  u.part = al(u.hrec + (size_t)K * ngi * 8 * kRecWords * 4);
  const size_t d_end = u.part + (size_t)kW * 16 * 4;
  u.end = g_end > d_end ? g_end : d_end;
  return u;
}

// ---------------------------------------------------------------------------
// Stage R
// ---------------------------------------------------------------------------
// The shared gate/up task of this workgroup: matrix m, row tile rt, k-chunks [kc0, kc1)
struct ShTask {
  int valid, m, rt, kc0, kc1;
};
__device__ __forceinline__ ShTask sh_task(const StackArgs &a) {
  ShTask t;
  const int b = blockIdx.x;
  t.valid = b < a.n_sh_tasks;
  const int per_m = (a.Ish / kTileRows) * a.KQ;
  const int tt = t.valid ? b : 0;
  t.m = tt / per_m;
  const int rem = tt % per_m;
  t.rt = rem / a.KQ;
  const int q = rem % a.KQ, nk = a.H / 64;
  t.kc0 = q * nk / a.KQ;
  t.kc1 = (q + 1) * nk / a.KQ;
  return t;
}
// this wave's k-chunks of the task
// the task as five words in LDS (computed once per call: the divisions by
// runtime values cost tens of scalar instructions each)
__device__ __forceinline__ ShTask sh_task_lds(const int *w) {
  ShTask t;
  t.valid = __builtin_amdgcn_readfirstlane(w[0]);
  t.m = __builtin_amdgcn_readfirstlane(w[1]);
  t.rt = __builtin_amdgcn_readfirstlane(w[2]);
  t.kc0 = __builtin_amdgcn_readfirstlane(w[3]);
  t.kc1 = __builtin_amdgcn_readfirstlane(w[4]);
  return t;
}
__device__ __forceinline__ void sh_wave_range(const ShTask &t, int wave, int &k0, int &k1) {
  const int n = t.kc1 - t.kc0;
  k0 = t.kc0 + wave * n / kW;
  k1 = t.kc0 + (wave + 1) * n / kW;
}

struct RStageLds {
  float segT[kRSlots][16];        // prefix-scan segment totals, segment c*8 + wave
  double Lp[kRSlots][kW];         // per-wave partial logits
  float Ap[kRSlots][kW], Pp[kRSlots][kW];
  float red[kW];
  int acc_i[kW][16];
};
__host__ __device__ inline size_t r_lds_bytes() { return (sizeof(RStageLds) + 255) & ~(size_t)255; }

// Stage R's inputs do not depend on the token: every thread loads its own
// part of them into registers while the previous layer's stage D computes
// (HBM is otherwise idle then), in the layout it uses them in.
//   w[s][c]: router row b + s*NB, elements 2048c + 4t .. +3, the thread's
//            elements of x;
//   g[c]:    the same elements of the shared expert's gate row (every
//            workgroup computes the gate logit itself, off the path of the
//            router records);
//   sa[i]:   k-chunk k0 + i of the workgroup's shared gate/up task, in the
//            int8 MFMA A layout (lane l: row l % 16, bytes (l / 16) * 16).
constexpr int kShMaxKc = 4;  // shared task k-chunks per wave
struct StaticRegs {
  v4f w[kRSlots][kNch];
  v4f g[kNch];
  v4i sa[kShMaxKc];
};
__device__ __forceinline__ void static_load(const StackArgs &a, const LayerPtrs &L, const ShTask &st, StaticRegs &sr,
                                            int t) {
  const int b = blockIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
  for (int s2 = 0; s2 < kRSlots; s2++) {
    const int r = b + s2 * a.NB;
    const bool valid = s2 < a.rslots && r < a.E;  // uniform
    const SW_G float *row = L.router + (size_t)(valid ? r : 0) * a.H;
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      const int e0 = 2048 * c + 4 * t;
      sr.w[s2][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (valid && c < a.nch && e0 < a.H) sr.w[s2][c] = __builtin_nontemporal_load((const SW_G v4f *)(row + e0));
    }
  }
#pragma unroll
  for (int c = 0; c < kNch; c++) {
    const int e0 = 2048 * c + 4 * t;
    sr.g[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (c < a.nch && e0 < a.H) sr.g[c] = *(const SW_G v4f *)(L.sgate + e0);
  }
  int k0, k1;
  sh_wave_range(st, wave, k0, k1);
  const SW_G signed char *sbase = (st.m == 0 ? L.gq : L.uq) + (size_t)(st.rt * kTileRows + (lane & 15)) * a.H +
                                  (lane >> 4) * 16;
#pragma unroll
  for (int i = 0; i < kShMaxKc; i++) {
    sr.sa[i] = v4i{0, 0, 0, 0};
    if (st.valid && k0 + i < k1) sr.sa[i] = __builtin_nontemporal_load((const SW_G v4i *)(sbase + (k0 + i) * 64));
  }
}

// The exact fp32 chain of the reference's dot() for the listed slots (rows
// b + s*NB): products rn(x*w) written to LDS by every thread, then one wave per
// slot adds them in index order (H % 8 == 0: no fused tail).  Rows and x are
// read again from memory: this path is rare, and keeping them in registers
// through the selection would cost every stage after it.
__device__ __forceinline__ void exact_chains(const StackArgs &a, const LayerPtrs &L, const float *x, unsigned want,
                                             float *prod, float *out) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int s = 0; s < kRSlots; s++)
    if (want & (1u << s)) {
      const int r = blockIdx.x + s * a.NB;
      const SW_G float *row = L.router + (size_t)r * a.H;
      for (int e0 = 4 * t; e0 < a.H; e0 += 4 * kT) {
        const v4f w = *(const v4f *)(row + e0);
        const v4f xv = *(const v4f *)(x + e0);
        v4f p;
        p.x = xv.x * w.x;
        p.y = xv.y * w.y;
        p.z = xv.z * w.z;
        p.w = xv.w * w.w;
        *(v4f *)(prod + (size_t)s * a.H + e0) = p;
      }
    }
  lds_barrier();
  if (wave < kRSlots && (want & (1u << wave))) {
    // The chain is serial and its products wait in LDS: a whole wave reads
    // 256 of them at a time (one v4f per lane, the next 256 in flight) and
    // readlane feeds them to the adds in index order.  Few registers are
    // held, so the long-lived state of the stages around this rare path is
    // not pushed out of registers.
    const v4f *p = (const v4f *)(prod + (size_t)wave * a.H);
    const int nv = a.H / 4, nfull = nv & ~63;
    float acc = 0.0f;
    v4f cur = nfull ? p[lane] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < nfull; i += 64) {
      v4f nxt = cur;
      if (i + 64 < nfull) nxt = p[i + 64 + lane];
#pragma unroll
      for (int k = 0; k < 64; k++) {
        acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.x), k));
        acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.y), k));
        acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.z), k));
        acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.w), k));
      }
      cur = nxt;
    }
    for (int i = nfull; i < nv; i++) {  // H % 256 != 0: the rest one by one
      const v4f v = p[i];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
    if (lane == 0) out[wave] = acc;
  }
  lds_barrier();
}

// The x operands of one wave's groups, kept in registers for the whole G
// stage (the wave always takes the same groups): the MFMA B operands of both
// steps (column c = lane%16: digit c of token 0 for c < 2, zero otherwise)
// and the group's digit scale and offset correction.
struct XOps {
  v4i b0[kGMax], b1[kGMax];
  float dsc[kGMax], zq[kGMax];
};
template <int FMT>
__device__ __forceinline__ void xops_load(XOps &xo, const DigitSrc &ds, int g0, int n, int lane) {
  constexpr int OFF = FMT == 4 ? 8 : 4;
  const int kb = lane >> 4;
#pragma unroll
  for (int gi = 0; gi < kGMax; gi++) {
    xo.b0[gi] = xo.b1[gi] = v4i{0, 0, 0, 0};
    xo.dsc[gi] = xo.zq[gi] = 0.0f;
    if (gi < n) {
      const int g = g0 + gi;
      const int off = (g * kGroup + kb * 16) & ds.mask;
      xo.b0[gi] = *(const v4i *)(ds.d + off);
      xo.b1[gi] = *(const v4i *)(ds.d + ((off + 64) & ds.mask));
      if (ds.gp) {
        const float4 p = ds.gp[g];
        const float d = ds.second ? p.y : p.x;
        const int Q = __float_as_int(ds.second ? p.w : p.z);
        xo.dsc[gi] = d;
        xo.zq[gi] = (float)(OFF * Q) * d;  // exact integer, one rounding
      }
    }
  }
}

// One tile-group from LDS: its codes at cbase, its 16 row scales at sbase.
template <int FMT>
__device__ __forceinline__ void g_item(const unsigned char *cbase, const unsigned char *sbase, const v4i &b0,
                                       const v4i &b1, float dsc, float zq, float acc[4], int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
  TileWord<FMT> tw;
  const unsigned char *cp = cbase + lane * BPL;
  if constexpr (FMT == 4) {
    const v4u v = *(const v4u *)cp;
    tw.w[0] = v.x;
    tw.w[1] = v.y;
    tw.w[2] = v.z;
    tw.w[3] = v.w;
  } else {
    tw.w[0] = ((const unsigned *)cp)[0];
    tw.w[1] = ((const unsigned *)cp)[1];
    tw.w[2] = ((const unsigned *)cp)[2];
  }
  const v4f s4 = *(const v4f *)(sbase + 16 * (lane >> 4));
  v4i a0, a1;
  unpack_tile<FMT>(tw, a0, a1);
  v4i c = {0, 0, 0, 0};
  c = mfma_i8(a0, b0, c);
  c = mfma_i8(a1, b1, c);
  const float scv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(__builtin_fmaf((float)c[r], dsc, -zq), scv[r], acc[r]);
}

// 16-lane row reductions by DPP (quad xor 1, quad xor 2, half-row mirror,
// row mirror): every lane of the row ends with the row's result
__device__ __forceinline__ float row16_max(float v) {
  const float ninf = -__builtin_huge_valf();
  v = fmaxf(v, SW_DPP_F(ninf, v, 0xB1, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x4E, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x141, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x140, 0xF, true));
  return v;
}
__device__ __forceinline__ int row16_sum_i(int v) {
  v += SW_DPP_I(0, v, 0xB1, 0xF, true);
  v += SW_DPP_I(0, v, 0x4E, 0xF, true);
  v += SW_DPP_I(0, v, 0x141, 0xF, true);
  v += SW_DPP_I(0, v, 0x140, 0xF, true);
  return v;
}


// Stage G's pairing: the first rr = nU % NB workgroups take one unit more than
// the others (nU units round-robin).  When rr <= NB/2, light workgroup b + rr
// also computes heavy workgroup b's shared down values (it finishes its units
// about one unit earlier) and publishes them for b's stage D, so the heavy
// ones, which the hidden barrier waits for, skip that work.
struct GPair {
  bool heavy;    // this workgroup's shared down values come from b + rr
  int partner;   // the heavy workgroup whose values this one also computes, or -1
};
__device__ __forceinline__ GPair g_pairing(const StackArgs &a, int b) {
  const int nU = a.K * a.nrt_i, rr = nU % a.NB, ntiles = a.H / kTileRows;
  const bool pairs = rr > 0 && 2 * rr <= a.NB;
  GPair p;
  p.heavy = pairs && b < rr && b < ntiles;
  p.partner = (pairs && b >= rr && b < 2 * rr && b - rr < ntiles) ? b - rr : -1;
  return p;
}

// ---------------------------------------------------------------------------
// Stage S: selection from the published records (all workgroups identically).
// ---------------------------------------------------------------------------
constexpr int kSelRec = 3;  // records per thread (E <= 3 * 512)
static_assert(kStackMaxE <= kSelRec * kT, "every record has a thread in stage S");
constexpr int kHrecPT = 8;  // h-record words (64-bit) per thread loaded in one batch
struct SelLds {
  unsigned long long samp[64];  // each 64-expert list's c largest keys
  unsigned long long mc[64];    // keys at or above the sample threshold
  unsigned long long wup[kW];   // each wave's largest upper bound below it
  int nmc;
  double theta, mxd;
  int nm;
  int m[kMaxAmbig];
  float exv[kMaxAmbig];
  float sl[kMaxAmbig];
  int se[kMaxAmbig];
  float mx, den;
  int chosen[kMaxK];
  float wsel[kMaxK];
};

// stage S's own part of the union: selection state, records [E], keys [E],
// exact-chain products [kRSlots][H]
__host__ __device__ inline size_t sel_end(int E, int H) {
  return ((sizeof(SelLds) + 15) & ~(size_t)15) + (size_t)E * 16 + (((size_t)E * 8 + 15) & ~(size_t)15) +
         (size_t)kRSlots * H * 4;
}

struct Routes {  // result of stage S, in static LDS
  int idx[kMaxK];
  float w[kMaxK];
  float sg;        // sigmoid of the shared gate logit
  int flag;        // barrier result broadcast
  int state;       // selection path: 0 certified, 1 targeted exact, 2 full exact
  float shm[kW];   // each wave's largest |shared hidden value|
  double gp[kW];   // each wave's part of the shared gate logit (fp64)
};

__device__ __forceinline__ bool sync_barrier(const StackArgs &a, const CallState &cs, int l, int which, Routes &rt) {
  lds_barrier();
  if (threadIdx.x == 0) {
    unsigned *bar = bar_of(a, cs, l, which);
    bar_arrive(bar, a.NB);
    rt.flag = bar_wait(bar, a) ? 1 : 0;
  }
  lds_barrier();
  return rt.flag != 0;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(kT, 1) void k_stack(StackArgs a0) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ Routes rt;
  __shared__ __align__(16) signed char zero16[16];
  __shared__ float s_misc[4];  // [0] sx of x, [1] sx of the shared hidden vector
  __shared__ int s_abort;      // a wait of this workgroup timed out or saw the abort word
  // the shared down projection's per-wave int32 sums of this workgroup's
  // output rows: written at the end of stage G while other waves may still
  // read the shared down rows, so kept out of the stage-local union
  __shared__ int s_shp[kW * 16];
  __shared__ int s_shp2[kW * 16];  // the same for the paired heavy workgroup's rows
  __shared__ unsigned s_lref[2][kRefWords];  // layer l's pointers in s_lref[l & 1]
  __shared__ int s_sht[5];                   // this workgroup's shared gate/up task
  __shared__ uint64_t s_exp2[32];            // expf's table: LDS reads wait behind no global load
  const int b = blockIdx.x;
  const Lds S = lds_carve(smem, a0.Hp, a0.ngh, a0.Ish);
  if (threadIdx.x < 4) ((int *)zero16)[threadIdx.x] = 0;
  if (threadIdx.x == 0) s_abort = 0;
  if (threadIdx.x < 32) s_exp2[threadIdx.x] = kExp2Tab[threadIdx.x];
  // Fault drill: these workgroups leave before taking any part, as if they
  // never became resident.  Every other one then meets a wait that cannot be
  // met (their router records, at the latest) and leaves through the abort word.
  if (b >= a0.NB - a0.absent) return;

  // The call state, read by every workgroup before any of them can pass the
  // first grid barrier (workgroup 0 advances it after the last one).
  CallState cs;
  unsigned long long layers_run;
  int zero_layers, zero_acc_words;
  {
    unsigned v[kStWords];
#pragma unroll
    for (int i = 0; i < kStWords; i++) v[i] = __builtin_amdgcn_readfirstlane(ld_agent(a0.state + i));
    layers_run = ((unsigned long long)v[kStLayersHi] << 32) | v[kStLayersLo];
    cs.parity = (int)(v[kStParity] & 1u);
    cs.tag0 = 1u + (unsigned)(layers_run % 255u);
    zero_layers = (int)v[cs.parity ? kStDirtyN0 : kStDirtyN1];
    zero_acc_words = (int)v[cs.parity ? kStDirtyAcc0 : kStDirtyAcc1];
  }
  // clear the other parity set's counters and integer sums for the next call
  {
    const StackArgs &a = a0;
    const int t = threadIdx.x;
    const int op = cs.parity ^ 1;
    const size_t bw = (size_t)kBars * kBarWords;
    for (int l = 0; l < zero_layers; l++) {
      unsigned *bz = a.bars + (size_t)(l * 2 + op) * bw;
      for (size_t i = (size_t)b * kT + t; i < bw; i += (size_t)a.NB * kT) bz[i] = 0u;
      unsigned long long *az = a.acc + (size_t)(l * 2 + op) * a.acc_stride;
      for (size_t i = (size_t)b * kT + t; i < (size_t)zero_acc_words; i += (size_t)a.NB * kT) az[i] = 0ull;
    }
  }

  if (threadIdx.x == 0) {
    const ShTask st = sh_task(a0);
    s_sht[0] = st.valid;
    s_sht[1] = st.m;
    s_sht[2] = st.rt;
    s_sht[3] = st.kc0;
    s_sht[4] = st.kc1;
  }
  __syncthreads();
  StaticRegs sreg;
  static_load(a0, layer_ref(a0, 0), sh_task_lds(s_sht), sreg, threadIdx.x);
  if (threadIdx.x < kRefWords) s_lref[0][threadIdx.x] = layer_ref_word(a0, 0, threadIdx.x);
  lds_barrier();

  for (int l = 0; l < a0.n; l++) {
    // Lane indices are re-derived every layer: values hoisted out of the loop
    // would stay live through every stage and spill.
    const StackArgs a = kargs();
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const LayerPtrs L = layer_ref_lds(s_lref[l & 1]);
    // the next layer's pointers: loaded now by wave 7 (which waits on no
    // memory before stage S), written to LDS once stage S is done
    unsigned nref = 0;
    if (l + 1 < a.n && t >= kT - 64 && t - (kT - 64) < kRefWords) nref = layer_ref_word(a, l + 1, t - (kT - 64));
    const float *x = a.x + (size_t)l * a.xs;
    unsigned long long *acc = a.acc + (size_t)(l * 2 + cs.parity) * a.acc_stride;

    // ======================= stage R =======================
    stamp(a, l, 0);
    RStageLds &R = *(RStageLds *)S.u;
    v4f xv[kNch];
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      const int e0 = 2048 * c + 4 * t;
      xv[c] = (c < a.nch && e0 < a.H) ? *(const v4f *)(x + e0) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // routed activation digits from the registers: a 128-group is 32 lanes x
    // 4 values (quantize_group's arithmetic: A = amax/127, B = A/254, two
    // rounded digits per element, digit sums)
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      const int e0 = 2048 * c + 4 * t;
      if (c < a.nch) {
        const float v[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
        float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        m = row16_max(m);
        m = fmaxf(m, __shfl_xor(m, 16, 32));
        const float A = m / 127.0f, B = A / 254.0f;
        int q1[4] = {0, 0, 0, 0}, q2[4] = {0, 0, 0, 0};
        if (m > 0.0f) {
          const float invA = 127.0f / m, invB = 254.0f / A;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            q1[i] = (int)fminf(fmaxf(__builtin_rintf(v[i] * invA), -127.0f), 127.0f);
            const float r = __builtin_fmaf(-(float)q1[i], A, v[i]);
            q2[i] = (int)fminf(fmaxf(__builtin_rintf(r * invB), -127.0f), 127.0f);
          }
        }
        int s1 = q1[0] + q1[1] + q1[2] + q1[3], s2 = q2[0] + q2[1] + q2[2] + q2[3];
        s1 = row16_sum_i(s1);
        s2 = row16_sum_i(s2);
        s1 += __shfl_xor(s1, 16, 32);
        s2 += __shfl_xor(s2, 16, 32);
        if (e0 < a.Hp) {
          *(int *)(S.xd + e0) = (q1[0] & 255) | (q1[1] & 255) << 8 | (q1[2] & 255) << 16 | (q1[3] & 255) << 24;
          *(int *)(S.xd + a.Hp + e0) =
              (q2[0] & 255) | (q2[1] & 255) << 8 | (q2[2] & 255) << 16 | (q2[3] & 255) << 24;
          if ((t & 31) == 0) S.xgp[e0 >> 7] = make_float4(A, B, __int_as_float(s1), __int_as_float(s2));
        }
      }
    }
    // qrow_i8 of x (c/qwen.c:1696): amax, sx = amax/127 (floor 1e-12), q = rint(x/sx)
    {
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < kNch; c++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[c].x), fabsf(xv[c].y)), fmaxf(fabsf(xv[c].z), fabsf(xv[c].w))));
      m = wave_max_dpp(m);
      if (lane == 0) R.red[wave] = m;
    }
    // Router pass 1, on the rows in registers.  The logit is the fp64 sum of
    // the exact products.  The bound needs A = sum |p| and P = sum_k |S_k|
    // over the prefix sums S_k of the serial order; both are taken in fp32
    // with their own rounding accounted for at the end: the prefixes go
    // thread (4 elements), wave (a 256-element segment, inclusive scan), then
    // over the row's segments (c * 8 + wave), whose carries need every wave's
    // segment total.
    double Lt[kRSlots];
    float At[kRSlots], sv[kRSlots][kNch][4];
    // the shared gate logit's part of this thread: the fp64 sum of exact products
    double Lgt = 0.0;
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      if (c >= a.nch) continue;
      const v4f w = c * 2048 + 4 * t < a.H ? sreg.g[c] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      Lgt = __builtin_fma((double)xv[c].x, (double)w.x, Lgt);
      Lgt = __builtin_fma((double)xv[c].y, (double)w.y, Lgt);
      Lgt = __builtin_fma((double)xv[c].z, (double)w.z, Lgt);
      Lgt = __builtin_fma((double)xv[c].w, (double)w.w, Lgt);
    }
#pragma unroll
    for (int s = 0; s < kRSlots; s++) {
      Lt[s] = 0.0;
      At[s] = 0.0f;
      const int r = b + s * a.NB;
      if (s < a.rslots && r < a.E) {
#pragma unroll
        for (int c = 0; c < kNch; c++) {
          if (c < a.nch) {
            const v4f w = sreg.w[s][c];
            const float p0 = xv[c].x * w.x, p1 = xv[c].y * w.y, p2 = xv[c].z * w.z, p3 = xv[c].w * w.w;
            Lt[s] = __builtin_fma((double)xv[c].x, (double)w.x, Lt[s]);
            Lt[s] = __builtin_fma((double)xv[c].y, (double)w.y, Lt[s]);
            Lt[s] = __builtin_fma((double)xv[c].z, (double)w.z, Lt[s]);
            Lt[s] = __builtin_fma((double)xv[c].w, (double)w.w, Lt[s]);
            At[s] += (fabsf(p0) + fabsf(p1)) + (fabsf(p2) + fabsf(p3));
            const float q1 = p0 + p1, q2 = q1 + p2, q3 = q2 + p3;
            const float inc = wave_inclusive_scan_f(q3);
            const float ex = dpp_wave_shr1_f(inc);
            sv[s][c][0] = ex + p0;
            sv[s][c][1] = ex + q1;
            sv[s][c][2] = ex + q2;
            sv[s][c][3] = ex + q3;
            if (lane == 63) R.segT[s][c * 8 + wave] = inc;
          }
        }
      }
    }
    lds_barrier();  // red, segT complete
    // qrow_i8 of x (c/qwen.c:1696): sx = amax/127 (floor 1e-12), q = rint(x/sx)
    float sx;
    {
      float amax = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; w++) amax = fmaxf(amax, R.red[w]);
      sx = amax / 127.0f;
      if (sx < 1e-12f) sx = 1e-12f;
      const float inv = 1.0f / sx;
#pragma unroll
      for (int c = 0; c < kNch; c++) {
        const int e0 = 2048 * c + 4 * t;
        if (c < a.nch && e0 < a.H) {
          int q0 = (int)__builtin_rintf(xv[c].x * inv), q1 = (int)__builtin_rintf(xv[c].y * inv);
          int q2 = (int)__builtin_rintf(xv[c].z * inv), q3 = (int)__builtin_rintf(xv[c].w * inv);
          *(int *)(S.xq + e0) = (q0 & 255) | (q1 & 255) << 8 | (q2 & 255) << 16 | (q3 & 255) << 24;
        }
      }
      if (t == 0) s_misc[0] = sx;
    }
    // Router pass 2: the carries of the segments (an exclusive scan of the
    // segment totals, 16 lanes), sum |S_k| and the wave sums of L, A, P.
#pragma unroll
    for (int s = 0; s < kRSlots; s++) {
      const int r = b + s * a.NB;
      if (s < a.rslots && r < a.E) {
        const float g = lane < a.nch * 8 ? R.segT[s][lane] : 0.0f;
        const float ge = dpp_row_shr1_f(row16_inclusive_scan_f(g));
        float P = 0.0f;
#pragma unroll
        for (int c = 0; c < kNch; c++) {
          const int e0 = 2048 * c + 4 * t;
          if (c < a.nch) {
            const float carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ge), c * 8 + wave));
            if (e0 < a.H)
              P += (fabsf(carry + sv[s][c][0]) + fabsf(carry + sv[s][c][1])) +
                   (fabsf(carry + sv[s][c][2]) + fabsf(carry + sv[s][c][3]));
          }
        }
        const double Lw = wave_sum_dpp(Lt[s]);
        const float Aw = wave_sum_dpp(At[s]), Pw = wave_sum_dpp(P);
        if (lane == 63) {
          R.Lp[s][wave] = Lw;
          R.Ap[s][wave] = Aw;
          R.Pp[s][wave] = Pw;
        }
      }
    }
    lds_barrier();  // xq, Lp/Ap/Pp complete
    if (wave == 0) {
      // Router records of this workgroup's rows, published before the shared
      // task below (every workgroup's selection waits for the last record),
      // lanes 2s (logit) and 2s+1
      // (bound).  The bound of the reference's serial fp32 dot:
      //   |fl(x.w) - x.w| <= u (A + sum_k |s^_k|) (u = 2^-24, s^_k its own
      //   partial sums), sum_k |s^_k| <= (P* + n u A)(1 + 2 n u) with P* the
      //   exact prefixes' sum; and P* <= P (1 + 2^-19) + 2^-7 A for the fp32
      //   P above (every prefix within 22 u A, n <= 4096), A* <= A (1 + 2^-18).
      // The fp64 logit is within 1e-12 A; flushed denormals within 1e-30.
      if (lane < 2 * kRSlots) {
        const int s = lane >> 1;
        const int r = b + s * a.NB;
        if (s < a.rslots && r < a.E) {
          double Lg = 0.0, A = 0.0, P = 0.0;
#pragma unroll
          for (int w = 0; w < kW; w++) {
            Lg += R.Lp[s][w];
            A += (double)R.Ap[s][w];
            P += (double)R.Pp[s][w];
          }
          double B = 0x1p-24 * (A * (1.0 + 0x1p-6) + P) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-30;
          B = (B + fabs(Lg) * 0x1p-43) * (1.0 + 0x1p-40);
          const double v = (lane & 1) ? B : Lg;
          // the tag replaces the low 8 bits of each double; the bound grows
          // by more than the logit can move (2^-44 relative)
          __hip_atomic_store((unsigned long long *)a.rec + 2 * r + (lane & 1),
                             with_tag((unsigned long long)__double_as_longlong(v), layer_tag(cs, l)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    // shared gate/up task: exact int32 dots of 16 rows with xq (A operands in
    // registers), added to the layer's counted sums (stage S reads each sum
    // once all of its KQ parts are in)
    const ShTask st = sh_task_lds(s_sht);
    {
      v4i cs = {0, 0, 0, 0};
      if (st.valid) {
        int k0, k1;
        sh_wave_range(st, wave, k0, k1);
#pragma unroll
        for (int i = 0; i < kShMaxKc; i++)
          if (k0 + i < k1) {
            const int kc = k0 + i;
            const v4i bv = (lane & 15) == 0 ? *(const v4i *)(S.xq + kc * 64 + (lane >> 4) * 16) : v4i{0, 0, 0, 0};
            cs = mfma_i8(sreg.sa[i], bv, cs);
          }
        if ((lane & 15) == 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) R.acc_i[wave][4 * (lane >> 4) + i] = cs[i];
        }
      }
    }
    lds_barrier();  // acc_i complete
    if (wave == 0) {
      if (st.valid && lane >= 16 && lane < 32) {
        const int r = lane - 16;
        int v = 0;
#pragma unroll
        for (int w = 0; w < kW; w++) v += R.acc_i[w][r];
        atomicAdd(&acc[st.m * a.Ish + st.rt * kTileRows + r], acc_term(v));
      }
    }
    stamp(a, l, 1);
    lds_barrier();  // stage R's LDS is reused below
    stamp(a, l, 2);

    // stage G's waves: groups [g0, g0+n) of every unit, gate and up (n may be <= 0)
    const int per = (a.ngh + kW - 1) / kW, g0 = wave * per;
    const int n = (a.ngh < g0 + per ? a.ngh : g0 + per) - g0;
    XOps xo;

    // ======================= stage S =======================
    {
      const StackArgs a = kargs();
      SelLds &sel = *(SelLds *)S.u;
      double2 *lb = (double2 *)(S.u + ((sizeof(SelLds) + 15) & ~(size_t)15));
      unsigned long long *lk = (unsigned long long *)(lb + a.E);
      float *prod = (float *)((unsigned char *)lk + (((size_t)a.E * 8 + 15) & ~(size_t)15));  // [kRSlots][H]
      const int E = a.E, K = a.K;
      // records -> LDS, and this thread's keys (experts t + i*kT) in registers;
      // every load is issued before the first is used
      const unsigned tag = layer_tag(cs, l);
      const unsigned long long *rec = (const unsigned long long *)a.rec;
      unsigned long long rx[kSelRec], ry[kSelRec];
#pragma unroll
      for (int i = 0; i < kSelRec; i++) {
        const int e = t + i * kT;
        rx[i] = ry[i] = 0ull;
        if (e < E) {
          rx[i] = ld_agent(rec + 2 * e);
          ry[i] = ld_agent(rec + 2 * e + 1);
        }
      }
      // stage G's activation operands from LDS while the records travel
      xops_load<FMT>(xo, lane_digits(lane, 1, S.xd, a.Hp, S.xgp, a.ngh, zero16), g0, n, lane);
      // records not yet tagged with this layer: read again until they are
      {
        const long long t0 = (long long)wall_clock64();
        for (unsigned it = 0;; it++) {
          bool all = true;
#pragma unroll
          for (int i = 0; i < kSelRec; i++)
            if (t + i * kT < E) all = all && has_tag(rx[i], tag) && has_tag(ry[i], tag);
          if (all) break;
          if ((it & 15) == 15 && __builtin_expect(wait_expired(t0, a), 0)) {
            s_abort = 1;
            break;
          }
#pragma unroll
          for (int i = 0; i < kSelRec; i++) {
            const int e = t + i * kT;
            if (e < E) {
              if (!has_tag(rx[i], tag)) rx[i] = ld_agent(rec + 2 * e);
              if (!has_tag(ry[i], tag)) ry[i] = ld_agent(rec + 2 * e + 1);
            }
          }
        }
      }
      double lx[kSelRec], ly[kSelRec];
#pragma unroll
      for (int i = 0; i < kSelRec; i++) {
        lx[i] = __longlong_as_double((long long)rx[i]);
        ly[i] = __longlong_as_double((long long)ry[i]);
      }
      unsigned long long key[kSelRec];
#pragma unroll
      for (int i = 0; i < kSelRec; i++) {
        const int e = t + i * kT;
        if (e < E) lb[e] = make_double2(lx[i], ly[i]);
        key[i] = e < E ? ((unsigned long long)float_key((float)lx[i]) << 32) | (unsigned)(~e) : 0ull;
      }
      // the shared gate logit's part of this wave (waves 1..7 now, wave 0
      // once it has selected)
      if (wave != 0) {
        const double g = wave_sum_dpp(Lgt);
        if (lane == 63) rt.gp[wave] = g;
      }
      if (t == 0) {
        sel.nm = 0;
        sel.nmc = 0;
      }
      // Candidates by a sampled threshold.  List L holds experts [64L, 64L+64)
      // (one wave, one record round); the c largest keys of each of the nl
      // non-empty lists form the sample, with c chosen so that it holds at
      // least K keys.  T0 = the sample's K-th largest key is at most the K-th
      // largest key overall, so the top K lie among the keys >= T0: usually a
      // few more than K, at most 64 on this path (else the full exact path).
      const int nl = (E + 63) >> 6;
      const int c = nl == 1 ? K : max(2, (K - 1 + nl - 2) / (nl - 1));  // nl * c <= 64
#pragma unroll
      for (int i = 0; i < kSelRec; i++) {
        const int li = i * kW + wave;
        if (li >= nl) continue;  // wave-uniform
        unsigned long long kk = key[i];
        for (int j = 0; j < c; j++) {
          const unsigned long long m = wave_max_u64(kk);
          if (lane == 0) sel.samp[li * c + j] = m;
          if (kk == m) kk = 0ull;
        }
      }
      lds_barrier();
      if (__builtin_expect(s_abort != 0, 0)) return;
      // T0, found by every wave: the sample with exactly K-1 larger ones
      unsigned long long T0;
      {
        const int ns = nl * c;
        const unsigned long long sv = lane < ns ? sel.samp[lane] : 0ull;
        const int rk = count_greater(sv, ns);
        const unsigned long long bal = __ballot(sv != 0ull && rk == K - 1);
        T0 = 1ull;  // (unreachable: the sample holds K keys) every key
        if (bal) {
          const int src = __ffsll((long long)bal) - 1;
          const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)sv, src);
          const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(sv >> 32), src);
          T0 = ((unsigned long long)hi << 32) | lo;
        }
      }
      // keys >= T0 to the candidate list; the largest upper bound of the rest
      {
        unsigned long long up = 0;
#pragma unroll
        for (int i = 0; i < kSelRec; i++) {
          if (i * kT + wave * 64 >= E) continue;  // wave-uniform: no key in this round
          const bool in = key[i] >= T0;           // key 0 (no expert) is below every T0
          const unsigned long long bal = __ballot(in);
          if (bal) {
            int base = 0;
            if (lane == 0) base = atomicAdd(&sel.nmc, __popcll(bal));
            base = __builtin_amdgcn_readfirstlane(base);
            const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
            if (in && pos < 64) sel.mc[pos] = key[i];
          }
          if (key[i] && !in) {
            const unsigned long long k2 = double_key(lx[i] + ly[i]);
            up = k2 > up ? k2 : up;
          }
        }
        up = wave_max_u64(up);
        if (lane == 0) sel.wup[wave] = up;
      }
      lds_barrier();
      if (wave >= 2) {
        // The shared expert's down rows of this workgroup's output tile, for
        // stage D, copied while HBM is otherwise idle.  Issued after this
        // wave's last use of its records: the compiler's wait for those loads
        // would otherwise wait for the copies too.
        const ULayout ul = u_layout(a.E, a.H, a.K, a.ngi, a.Ish, FMT);
        const GPair gp = g_pairing(a, b);
        auto copy_tile = [&](int tile, size_t dst) {
          for (int r = wave - 2; r < kTileRows; r += kW - 2)
            for (int c0 = 0; c0 < a.Ish; c0 += 1024)
              if (c0 + 16 * lane < a.Ish)
                dma_b128((const void *)(L.dq + (size_t)(tile * kTileRows + r) * a.Ish + c0 + 16 * lane),
                         lds_addr(S.u + dst + (size_t)r * (a.Ish + 16) + c0));
        };
        if (b < a.H / kTileRows && !gp.heavy) copy_tile(b, ul.gdsh);
        if (gp.partner >= 0) copy_tile(gp.partner, ul.gdsh2);
      } else if (wave == 1) {
        // This workgroup's values of the shared hidden vector, i = b + j*NB
        // (lane j), while wave 0 selects: the counted gate/up sums (complete
        // once all KQ parts are in: the call started with the set cleared, so
        // a count of KQ is this call's), the IDOT epilogue
        // ((float)dot * s_row) * sx (c/qwen.c:1766) and SwiGLU (c/qwen.c:3419),
        // published (tagged with the layer) for every workgroup's stage G.
        const int i = b + lane * a.NB;
        if (i < a.Ish) {
          unsigned long long wg = ld_agent(&acc[i]), wu = ld_agent(&acc[a.Ish + i]);
          const float gsr = L.gs[i], usr = L.us[i];
          const long long t0 = (long long)wall_clock64();
          for (unsigned it = 0; acc_parts(wg) != a.KQ || acc_parts(wu) != a.KQ; it++) {
            if ((it & 15) == 15 && __builtin_expect(wait_expired(t0, a), 0)) {
              s_abort = 1;
              break;
            }
            wg = ld_agent(&acc[i]);
            wu = ld_agent(&acc[a.Ish + i]);
          }
          const float sx = s_misc[0];
          const float h = silu_ref_t((float)acc_sum(wg) * gsr * sx, s_exp2) * ((float)acc_sum(wu) * usr * sx);
          __hip_atomic_store(a.hs + i, ((unsigned long long)layer_tag(cs, l) << 32) | __float_as_uint(h),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else if (wave == 0) {
        const int M = sel.nmc;
        if (__builtin_expect(M > 64 || M < K, 0)) {
          if (lane == 0) rt.state = 2;
        } else {
          // every candidate in a lane: key, record (logit, bound), rank among
          // the candidates (ranks by register broadcasts, no LDS round trips)
          const unsigned long long ck = lane < M ? sel.mc[lane] : 0ull;
          const int ce = lane < M ? (int)(~(unsigned)ck) : 0;
          const double2 v = lb[ce];
          const int rk = count_greater(ck, M);
          // the largest upper bound outside the top K: candidates ranked K
          // and below, and every wave's bound of the keys below T0
          unsigned long long upk = lane < kW ? sel.wup[lane] : 0ull;
          if (lane < M && rk >= K) {
            const unsigned long long k2 = double_key(v.x + v.y);
            upk = k2 > upk ? k2 : upk;
          }
          upk = wave_max_u64(upk);
          // the candidates in rank order (a forward permute: lane r receives
          // the candidate of rank r; lanes past M keep their own)
          const int pa = 4 * (lane < M ? rk : lane);
          const double sL = permute_d(pa, v.x), sB = permute_d(pa, v.y);
          const int se = __builtin_amdgcn_ds_permute(pa, ce);
          const double vlo = sL - sB;
          const double mx = readlane_d(sL, 0), mxy = readlane_d(sB, 0);
          // The lowest lower bound among the K candidates and their largest
          // magnitude.  When every consecutive pair is certified the lower
          // bounds fall with the rank and theta is the K-th one; otherwise a
          // candidate ranked above K-1 may have the lowest lower bound, and
          // the set test must use that one.
          const double theta = row16_min_d(lane < K ? vlo : 1e300);
          const double kax = row16_max_d(lane < K ? fabs(sL) : 0.0);
          // the next candidate's bounds (row shift left within lanes 0..15)
          const double nx = dpp_row_shl1_d(sL), ny = dpp_row_shl1_d(sB);
          bool pair_ok = true;
          if (lane + 1 < K) pair_ok = vlo - (nx + ny) > order_margin(sL, nx, mx);
          // The set of K is certified by the lowest lower bound among the K
          // against every other expert's upper bound; their order by the
          // pairs.  Without a route output (a stack call) the order only
          // changes the rounding of the combine, so an uncertain order among
          // a certified set is taken as is (the set is exact either way; the
          // weights come from the fp64 logits in either order, within the
          // weights' tolerance).
          bool ok = L.mode == 0 && (__all(pair_ok) || (a.route_idx == nullptr && a.route_w == nullptr));
          if (ok && K < E) {
            const double up = key_double(upk);
            ok = theta - up > order_margin(kax, up, mx);
          }
          if (ok) ok = theta - (mx + mxy) > -75.0;
          if (ok) {
            // softmax over the K (lanes 0..15 hold them): fp32 suffices for
            // the weights' 1e-5 tolerance
            const float ev = lane < K ? __expf((float)(sL - mx)) : 0.0f;
            const float den = row16_sum(ev);
            if (lane < K) {
              rt.idx[lane] = se;
              rt.w[lane] = ev / den;
            }
          } else {
            if (lane == 0) {
              sel.theta = theta;
              sel.mxd = mx;
            }
          }
          if (lane == 0) rt.state = ok ? 0 : (L.mode != 0 ? 2 : 1);
        }
        const double g = wave_sum_dpp(Lgt);
        if (lane == 63) rt.gp[0] = g;
      }
      lds_barrier();
      if (__builtin_expect(rt.state == 1, 0)) {
        // Every expert whose upper bound reaches the lowest lower bound among
        // the K candidates (less a margin): the exact top K lies in this set,
        // since anything outside it is strictly below all K candidates.
        const double theta = sel.theta, mx = sel.mxd;
#pragma unroll
        for (int i = 0; i < kSelRec; i++) {
          const int e = t + i * kT;
          if (e < E && lx[i] + ly[i] >= theta - order_margin(lx[i], theta, mx)) {
            const int slot = atomicAdd(&sel.nm, 1);
            if (slot < kMaxAmbig) sel.m[slot] = e;
          }
        }
        lds_barrier();
        if (t == 0 && !(sel.nm <= kMaxAmbig && sel.nm >= K)) rt.state = 2;
        lds_barrier();
      }
      if (b == 0 && t == 0) {
        __hip_atomic_fetch_add(&L.stats[0], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (rt.state != 0) __hip_atomic_fetch_add(&L.stats[1], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (__builtin_expect(rt.state == 1, 0)) {
        // exact chains of the ambiguous experts this workgroup owns
        unsigned want = 0;
        for (int i = 0; i < sel.nm; i++) {
          const int e = sel.m[i];
          if (e % a.NB == b) want |= 1u << (e / a.NB);
        }
        if (want) {
          __shared__ float s_out[kRSlots];
          exact_chains(a, L, x, want, prod, s_out);
          if (wave == 0) {
            unsigned dep = 0;
            if (lane < kRSlots && (want & (1u << lane))) dep = pub((unsigned *)&a.ex[b + lane * a.NB], __float_as_uint(s_out[lane]));
            published(dep);
          }
        }
        if (!sync_barrier(a, cs, l, kBarEx1, rt)) return;
        if (wave == 0) {
          const int nm = sel.nm;
          const float lv = lane < nm ? ld_agent(&a.ex[sel.m[lane]]) : -__builtin_huge_valf();
          const int e = lane < nm ? sel.m[lane] : 0x7fffffff;
          if (lane < nm) sel.exv[lane] = lv;
          __builtin_amdgcn_wave_barrier();
          int rank = 0;
          for (int q = 0; q < nm; q++) {
            const float lq = sel.exv[q];
            const int eq = sel.m[q];
            rank += (lq > lv) || (lq == lv && eq < e);
          }
          if (lane < nm) {
            sel.sl[rank] = lv;
            sel.se[rank] = e;
          }
          __builtin_amdgcn_wave_barrier();
          const double mx = sel.sl[0];
          bool pair_ok = true;
          if (lane < K && lane + 1 < nm) {
            const double p = sel.sl[lane], q = sel.sl[lane + 1];
            pair_ok = p == q || p - q > order_margin(p, q, mx);
          }
          const bool ok = __all(pair_ok) && ((double)sel.sl[K - 1] - mx > -75.0);
          if (ok) {
            const float ev = lane < K ? __expf((float)((double)sel.sl[lane < K ? lane : 0] - mx)) : 0.0f;
            const float den = row16_sum(ev);
            if (lane < K) {
              rt.idx[lane] = sel.se[lane];
              rt.w[lane] = ev / den;
            }
          }
          if (lane == 0 && !ok) rt.state = 2;
        }
        lds_barrier();
      }
      if (__builtin_expect(rt.state == 2, 0)) {
        // every expert's exact chain (owners compute theirs), then router_topk
        // (c/qwen.c:3421-3426) bit for bit: max, expf(l - max), the serial
        // denominator in expert order, division, K argmax rounds (lowest index
        // on ties), serial renormalisation
        unsigned want = 0;
        for (int s = 0; s < a.rslots && s < kRSlots; s++)
          if (b + s * a.NB < E) want |= 1u << s;
        if (want) {
          __shared__ float s_out2[kRSlots];
          exact_chains(a, L, x, want, prod, s_out2);
          if (wave == 0) {
            unsigned dep = 0;
            if (lane < kRSlots && (want & (1u << lane))) dep = pub((unsigned *)&a.ex[b + lane * a.NB], __float_as_uint(s_out2[lane]));
            published(dep);
          }
        }
        if (!sync_barrier(a, cs, l, kBarEx2, rt)) return;
        float *lgs = prod;  // [E]
        for (int e = t; e < E; e += kT) lgs[e] = ld_agent(&a.ex[e]);
        lds_barrier();
        if (wave == 0) {
          float m = -__builtin_huge_valf();
          for (int e = lane; e < E; e += 64) m = fmaxf(m, lgs[e]);
          m = wave_max_dpp(m);
          if (lane == 0) sel.mx = m;
        }
        lds_barrier();
        for (int e = t; e < E; e += kT) lgs[e] = expf_glibc_t(lgs[e] - sel.mx, s_exp2);
        lds_barrier();
        if (t == 0) {
          float den = 0.0f;
          for (int e = 0; e < E; e++) den += lgs[e];
          sel.den = den;
        }
        lds_barrier();
        for (int e = t; e < E; e += kT) lgs[e] = lgs[e] / sel.den;
        lds_barrier();
        if (wave == 0) {
          for (int j = 0; j < K; j++) {
            unsigned long long best = 0;
            for (int e = lane; e < E; e += 64) {
              bool used = false;
              for (int q = 0; q < j; q++) used |= sel.chosen[q] == e;
              const float pv = lgs[e];
              const unsigned long long k2 = (((unsigned long long)float_key(pv)) << 32) | (unsigned)(~e);
              if (!used && pv > -1.0f && k2 > best) best = k2;
            }
            best = wave_max_u64(best);
            const int c = best ? (int)(~(unsigned)best) : -1;
            if (lane == 0) {
              sel.chosen[j] = c;
              sel.wsel[j] = best ? lgs[c] : -1.0f;
            }
            __builtin_amdgcn_wave_barrier();
          }
          if (lane == 0) {
            float topden = 0.0f;
            for (int j = 0; j < K; j++) topden += sel.wsel[j];
            for (int j = 0; j < K; j++) {
              rt.idx[j] = sel.chosen[j];
              rt.w[j] = sel.wsel[j] / topden;
            }
            if (b == 0) __hip_atomic_fetch_add(&L.stats[2], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        lds_barrier();
      }
      if (b == 0 && t < K) {
        if (a.route_idx) a.route_idx[t] = rt.idx[t];
        if (a.route_w) a.route_w[t] = rt.w[t];
      }
      // No barrier: the routes are in static LDS, the exact paths end with
      // one, and after the last one nothing reads this stage's LDS but the
      // shared hidden vector, which lies past stage G's regions.
    }
    stamp(a, l, 3);
    if (l + 1 < a.n && t >= kT - 64 && t - (kT - 64) < kRefWords) s_lref[(l + 1) & 1][t - (kT - 64)] = nref;

    // ======================= stage G =======================
    {
      const StackArgs a = kargs();
      const ULayout ul = u_layout(a.E, a.H, a.K, a.ngi, a.Ish, FMT);
      float(*red)[2][16] = (float(*)[2][16])S.u;                 // [2][kW][gate, up][16] partials
      unsigned *stage = (unsigned *)(S.u + 2 * kW * 2 * 16 * 4);  // [kW][8] packed digits
      const int nU = a.K * a.nrt_i;
      constexpr int BPL = FMT == 4 ? 16 : 12;
      constexpr int TGC = 64 * BPL;  // codes of one tile-group
      // Each wave streams its own gate/up records (its groups, unit after
      // unit) through a ring of kGRing slots in LDS: one record (both
      // matrices' codes and row scales of one group) per slot, copied in
      // 1 KB pieces, kGRing-1 records in flight while one is computed.
      constexpr int kSlotG = 2 * TGC + 128;
      constexpr int kGChunks = (kSlotG + 1023) / 1024;
      static_assert(kGHead >= 2 * kW * 2 * 16 * 4 + kW * 8 * 4, "stage G head");
      unsigned char *ring = S.u + ul.ring + (size_t)wave * kGRing * kSlotG;
      // Units (route, 16 rows) go round-robin over the workgroups.
      const int nent = b < nU ? (nU - 1 - b) / a.NB + 1 : 0;
      const int nitems = n > 0 ? nent * n : 0;
      // This wave's unit table, one entry per lane: byte offset of the
      // entry's first record of this wave's groups (an invalid route reads the
      // layer's first bytes instead; its results are discarded).
      unsigned long long tc = 0ull;
      if (lane < nent) {
        const int u = b + lane * a.NB, j = u / a.nrt_i, r16 = u - j * a.nrt_i;
        const int e = rt.idx[j];
        if ((unsigned)e < (unsigned)a.E) tc = (size_t)e * a.expert_bytes + ((size_t)r16 * a.ngh + g0) * kSlotG;
      }
      // Issue cursor (entry iu, group gu, ring slot su).  Every step issues
      // the kGChunks copies of one record, up to kGRing-1 items ahead of the
      // one consumed, and none past the last item.
      int iu = 0, gu = 0, su = 0, issued = 0;
      const unsigned char *cb = (const unsigned char *)L.experts;
      auto unit_base = [&](int i) {
        const int ii = i < nent ? i : nent - 1;
        const unsigned lo_c = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)tc, ii);
        const unsigned hi_c = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(tc >> 32), ii);
        cb = (const unsigned char *)L.experts + (((unsigned long long)hi_c << 32) | lo_c);
      };
      auto issue_next = [&]() {
        if (issued == nitems) return;
        const unsigned slot = lds_addr(ring + su * kSlotG);
#pragma unroll
        for (int k = 0; k < kGChunks; k++)
          if (16 * lane < kSlotG - 1024 * k) dma_b128_s(cb + gu * kSlotG + 1024 * k, 16 * lane, slot + 1024 * k);
        issued++;
        if (++su == kGRing) su = 0;
        if (++gu == n) {
          gu = 0;
          unit_base(++iu);
        }
      };
      // h of 16 rows from their gate and up sums (lanes 0..15 of the calling
      // wave): SwiGLU (c/qwen.c:3419), then two int8 digits per 16-value chunk
      // (A = amax/127, B = A/254) and the record.  The hidden vector is
      // quantised next, so the hardware exponential is within the tolerance.
      auto finish_h = [&](float gsum, float usum, int u) {
        const int j = u / a.nrt_i, r16 = u % a.nrt_i;
        const int e = rt.idx[j];
        const int r = lane;
        float h = gsum / (1.0f + __expf(-gsum)) * usum;
        if ((unsigned)e >= (unsigned)a.E || r16 * kTileRows + r >= a.I) h = 0.0f;
        const float mm = row16_max(fabsf(h));
        const float A = mm / 127.0f, B = A / 254.0f;
        int q1 = 0, q2 = 0;
        if (mm > 0.0f) {
          const float invA = 127.0f / mm, invB = 254.0f / A;
          q1 = (int)fminf(fmaxf(__builtin_rintf(h * invA), -127.0f), 127.0f);
          const float rr2 = __builtin_fmaf(-(float)q1, A, h);
          q2 = (int)fminf(fmaxf(__builtin_rintf(rr2 * invB), -127.0f), 127.0f);
        }
        const int s1 = row16_sum_i(q1), s2 = row16_sum_i(q2);
        // stage D's digit scales with the route weight folded in, and the code
        // offset's correction (OFF x digit sum x scale) ready to subtract
        constexpr int OFFD = FMT == 4 ? 8 : 4;
        const float wj = (unsigned)e < (unsigned)a.E ? rt.w[j] : 0.0f;
        const float Aw = A * wj, Bw = B * wj;
        const float z1 = (float)(OFFD * s1) * Aw, z2 = (float)(OFFD * s2) * Bw;
        signed char *stg = (signed char *)(stage + 8 * wave);
        stg[r] = (signed char)q1;
        stg[16 + r] = (signed char)q2;
        __builtin_amdgcn_wave_barrier();
        unsigned v = 0;
        if (r < 8) v = ((const unsigned *)stg)[r];
        else if (r == 8) v = __float_as_uint(Aw);
        else if (r == 9) v = __float_as_uint(Bw);
        else if (r == 10) v = __float_as_uint(z1);
        else if (r == 11) v = __float_as_uint(z2);
        // a device-scope store: complete (and visible to every device-scope
        // load) once vmcnt drains, which every wave waits for before the
        // workgroup arrives at the barrier
        if (r < kRecWords)
          __hip_atomic_store(&a.hd[((size_t)j * a.ngi * 8 + r16) * kRecWords + r], v, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      };
      // Partials of entry i go to red[i & 1]; after one barrier, wave i % 8
      // finishes the entry while the others go on to the next one (the next
      // entry's barrier keeps red[i & 1] until the finisher is done).
      auto finish_entry = [&](float accg[4], float accu[4], int i) {
        float(*rb)[2][16] = red + (i & 1) * kW;
        digit_fold(accg);
        digit_fold(accu);
        if ((lane & 15) == 1) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            rb[wave][0][4 * (lane >> 4) + q] = accg[q];
            rb[wave][1][4 * (lane >> 4) + q] = accu[q];
          }
        }
        lds_barrier();
        if (wave == (i & (kW - 1)) && lane < 16) {
          const int r = lane;
          float gsum = 0.0f, usum = 0.0f;
#pragma unroll
          for (int w = 0; w < kW; w++) {
            gsum += rb[w][0][r];
            usum += rb[w][1][r];
          }
          finish_h(gsum, usum, b + i * a.NB);
        }
      };
      if (nitems > 0) {
        unit_base(0);
#pragma unroll
        for (int k = 0; k < kGRing - 1; k++) issue_next();
      }
      // The shared hidden vector (every workgroup's values, published in stage
      // S) as tagged words, copied into LDS in 1 KB pieces (piece p by wave
      // p % kW) a few items before this wave's last, so that they have landed
      // by the end of the stage: at consume step kh, after that step's
      // record, so the waits for the records issued before them allow nhp
      // more copies outstanding.
      const int nhpc = g_pairing(a, b).heavy ? 0 : (a.Ish + 127) / 128;  // a heavy workgroup needs none
      const int nhp = nhpc > wave ? (nhpc - 1 - wave) / kW + 1 : 0;
      const int kh = nitems > 3 ? nitems - 3 : 0;
      auto issue_hs = [&]() {
        for (int q = 0; q < nhp; q++) {
          const int pc = wave + kW * q, rem = a.Ish - 128 * pc;
          if (2 * lane < rem) dma_b128_dev(a.hs + (size_t)pc * 128 + 2 * lane, lds_addr(S.u + ul.hsw) + 1024 * pc);
        }
      };
      if (nitems == 0) issue_hs();
      if (t == 64) {
        // the shared expert's gate (c/qwen.c:3737) for stage D: its fp64
        // logit, the waves' parts added in order, rounded, through
        // sigmoidf_stable
        double g = 0.0;
#pragma unroll
        for (int w = 0; w < kW; w++) g += rt.gp[w];
        rt.sg = sigmoid_ref_t((float)g, s_exp2);
      }
      int csl = 0, consumed = 0;  // consume slot, items consumed
      for (int i = 0; i < nent; i++) {
        float accg[4] = {0, 0, 0, 0}, accu[4] = {0, 0, 0, 0};
        if (n > 0) {
#pragma unroll
          for (int gi = 0; gi < kGMax; gi++)
            if (gi < n) {
              issue_next();
              if (consumed == kh) issue_hs();
              // this item's copies are done once at most the copies issued
              // after it are outstanding (a wave's memory operations complete
              // in order; a store of finish_h only makes the wait longer)
              wait_vm(kGChunks * (issued - consumed - 1) + (consumed >= kh && consumed < kh + kGRing ? nhp : 0));
              consumed++;
              const unsigned char *rec = ring + csl * kSlotG;
              g_item<FMT>(rec, rec + 2 * TGC, xo.b0[gi], xo.b1[gi], xo.dsc[gi], xo.zq[gi], accg, lane);
              g_item<FMT>(rec + TGC, rec + 2 * TGC + 64, xo.b0[gi], xo.b1[gi], xo.dsc[gi], xo.zq[gi], accu, lane);
              if (++csl == kGRing) csl = 0;
            }
        }
        finish_entry(accg, accu, i);
      }
      // Every copy has landed.  The last entry's finisher may still have its
      // h-record store in flight (its last memory operation): it is waited
      // for before the workgroup arrives at the hidden barrier.
      if (nent > 0 && wave == ((nent - 1) & (kW - 1)))
        wait_vm(1);
      else
        wait_dma();
      lds_barrier();  // the last finisher is done with its partials; the tagged words are in
      const GPair gp = g_pairing(a, b);
      if (!gp.heavy) {
        // The shared hidden vector's values (a word not yet carrying this
        // layer's tag when copied is read again: rare), its qrow_i8
        // (c/qwen.c:1696: s = amax/127, floor 1e-12, q = rint(h/s)) applied
        // as the operands are read, and the shared down: exact int32 dots of
        // the tile's 16 rows with it, into s_shp (the ring is no longer read);
        // with a partner, its tile's too, published as the combine's shared
        // values ((float)dot * s_row) * sx.
        const unsigned tag = layer_tag(cs, l);
        unsigned long long *hw = (unsigned long long *)(S.u + ul.hsw);
        const int ntiles = a.H / kTileRows;
        const float pds = gp.partner >= 0 && t < kTileRows ? L.ds[gp.partner * kTileRows + t] : 0.0f;
        float hm = 0.0f;
        for (int i = t; i < a.Ish; i += kT) {
          unsigned long long w = hw[i];
          if (__builtin_expect((unsigned)(w >> 32) != tag, 0)) {
            const long long t0 = (long long)wall_clock64();
            for (unsigned it = 0; (unsigned)(w >> 32) != tag; it++) {
              if ((it & 15) == 15 && __builtin_expect(wait_expired(t0, a), 0)) {
                s_abort = 1;
                break;
              }
              w = ld_agent_sync(a.hs + i);
            }
            hw[i] = w;
          }
          hm = fmaxf(hm, fabsf(__uint_as_float((unsigned)w)));
        }
        hm = wave_max_dpp(hm);
        if (lane == 0) rt.shm[wave] = hm;
        lds_barrier();
        float shx = 0.0f;
#pragma unroll
        for (int w = 0; w < kW; w++) shx = fmaxf(shx, rt.shm[w]);
        shx = shx / 127.0f;
        if (shx < 1e-12f) shx = 1e-12f;
        const float hinv = 1.0f / shx;
        if (t == 0) s_misc[1] = shx;
        const int nkd = a.Ish / 64, kb = lane >> 4;
        const int dk0 = wave * nkd / kW, dk1 = (wave + 1) * nkd / kW;
        auto shared_down = [&](const signed char *rows, int *out) {
          v4i cd = {0, 0, 0, 0};
          const signed char *arow = rows + (size_t)(lane & 15) * (a.Ish + 16) + kb * 16;
          for (int kc = dk0; kc < dk1; kc++) {
            const v4i av = *(const v4i *)(arow + kc * 64);
            v4i bv = {0, 0, 0, 0};
            if ((lane & 15) == 0) {
              const v4u *hp = (const v4u *)(hw + kc * 64 + kb * 16);  // 16 words: (tag, bits) pairs
#pragma unroll
              for (int q = 0; q < 4; q++) {
                const v4u u0 = hp[2 * q], u1 = hp[2 * q + 1];
                const int q0 = (int)__builtin_rintf(__uint_as_float(u0.x) * hinv);
                const int q1 = (int)__builtin_rintf(__uint_as_float(u0.z) * hinv);
                const int q2 = (int)__builtin_rintf(__uint_as_float(u1.x) * hinv);
                const int q3 = (int)__builtin_rintf(__uint_as_float(u1.z) * hinv);
                bv[q] = (q0 & 255) | (q1 & 255) << 8 | (q2 & 255) << 16 | (q3 & 255) << 24;
              }
            }
            cd = mfma_i8(av, bv, cd);
          }
          if ((lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) out[wave * 16 + 4 * kb + i] = cd[i];
          }
        };
        if (b < ntiles) shared_down((const signed char *)(S.u + ul.gdsh), s_shp);
        if (gp.partner >= 0) {
          shared_down((const signed char *)(S.u + ul.gdsh2), s_shp2);
          lds_barrier();
          if (t < kTileRows) {
            int dot = 0;
#pragma unroll
            for (int w = 0; w < kW; w++) dot += s_shp2[w * 16 + t];
            // stored before this workgroup arrives at the hidden barrier
            __hip_atomic_store(a.shv + gp.partner * kTileRows + t, (float)dot * pds * shx, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      if (__builtin_expect(s_abort != 0, 0)) return;
      // zero records of chunks past I inside the last group (only when I % 128 != 0)
      if (b == 0 && wave == 0) {
        const int pad = a.ngi * 8 - a.nrt_i;
        for (int i = lane; i < a.K * pad * kRecWords; i += 64) {
          const int j = i / (pad * kRecWords), rem = i % (pad * kRecWords);
          __hip_atomic_store(&a.hd[((size_t)j * a.ngi * 8 + a.nrt_i) * kRecWords + rem], 0u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (wave == 0) published(0);
    }

    // ======================= stage D (loads, then barrier h) =======================
    {
      const StackArgs a = kargs();
      const ULayout dl = u_layout(a.E, a.H, a.K, a.ngi, a.Ish, FMT);
      constexpr int BPL = FMT == 4 ? 16 : 12;
      constexpr int kSlot = 64 * BPL + 64;  // one tile-group: codes, then 16 row scales
      const int nq = a.K * a.ngi;
      const int tile = b, ntiles = a.H / kTileRows;
      unsigned char *dtile = S.u + dl.dtile;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every h record store is complete
      lds_barrier();
      stamp(a, l, 4);
      if (t == 0) bar_arrive(bar_of(a, cs, l, kBarH), a.NB);
      // the tile's routed down records, straight into LDS in 1 KB copies by
      // waves 1..7 while the barrier completes (wave 0 polls it: a wave's
      // loads return in order, so its poll waits behind no copy).  A route's
      // ngi records of this tile are contiguous in HBM and in LDS.
      if (tile < ntiles && wave != 0) {
        const int rbytes = a.ngi * kSlot, nck = (rbytes + 1023) >> 10;
        for (int c = wave - 1; c < a.K * nck; c += kW - 1) {
          const int j = c / nck, k = c - j * nck;
          int e = rt.idx[j];
          if ((unsigned)e >= (unsigned)a.E) e = 0;  // in bounds; such a route's weight is zero
          const void *src =
              (const void *)(L.experts + (size_t)e * a.expert_bytes + a.gu_bytes + (size_t)tile * rbytes + 1024 * k);
          if (16 * lane < rbytes - 1024 * k)
            dma_b128((const unsigned char *)src + 16 * lane, lds_addr(dtile + (size_t)j * rbytes + 1024 * k));
        }
      }
      if (t == 0) rt.flag = bar_wait(bar_of(a, cs, l, kBarH), a) ? 1 : 0;
      lds_barrier();
      if (__builtin_expect(!rt.flag, 0)) return;
      stamp(a, l, 5);
      if (__builtin_expect(l == a.n - 1, 0) && wave == 0 && lane < kRSlots) {
        // Every workgroup has passed this call's last selection, so no one
        // reads the records any more: clear this workgroup's, so that a later
        // call never meets a word left by an older one (records are read
        // only where a call writes them, and tags repeat)
        const int r = b + lane * a.NB;
        if (lane < a.rslots && r < a.E) {
          __hip_atomic_store((unsigned long long *)a.rec + 2 * r, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store((unsigned long long *)a.rec + 2 * r + 1, 0ull, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (__builtin_expect(l == a.n - 1, 0) && wave == 1 && b + lane * a.NB < a.Ish) {
        // the shared hidden words this workgroup published: every workgroup
        // has read them (before the hidden barrier), so cleared as the
        // records are
        __hip_atomic_store(a.hs + b + lane * a.NB, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (__builtin_expect(l == a.n - 1, 0) && b == 0 && t == 0) {
        // every workgroup has read the call state: advance it for the next call
        const unsigned long long nl = layers_run + (unsigned long long)a.n;
        const int p = cs.parity;
        __hip_atomic_store(a.state + kStLayersLo, (unsigned)nl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.state + kStLayersHi, (unsigned)(nl >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.state + (p ? kStDirtyN1 : kStDirtyN0), (unsigned)a.n, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.state + (p ? kStDirtyAcc1 : kStDirtyAcc0), (unsigned)(2 * a.Ish), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.state + kStParity, (unsigned)(p ^ 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }

      // a heavy workgroup's shared down values, computed by its partner
      const bool heavy = g_pairing(a, b).heavy;
      const float hshv = heavy ? ld_agent(a.shv + (tile < ntiles ? tile : 0) * kTileRows + (t & (kTileRows - 1))) : 0.0f;
      // h records of every route -> LDS (every load issued before the first is used)
      unsigned *hrec = (unsigned *)(S.u + dl.hrec);  // [K][ngi*8][12]
      float *part = (float *)(S.u + dl.part);        // [K][kW][16]
      const int *shp = s_shp;                        // [kW][16]
      const float shx = s_misc[1];
      const int n64 = a.K * a.ngi * 8 * kRecWords / 2;
      // Every load unconditional, from a clamped index (values past the end
      // are loaded twice and not used): a register first zeroed and then
      // loaded under a lane mask makes the compiler wait for the earlier
      // loads before zeroing the next one.
      // the shared down row scales of this workgroup's tile, for the combine
      const float dsr = L.ds[(tile < ntiles ? tile : 0) * kTileRows + (t & (kTileRows - 1))];
      {
        unsigned long long hv[kHrecPT];
#pragma unroll
        for (int i = 0; i < kHrecPT; i++) {
          const int j = t + i * kT;
          hv[i] = ld_agent((const unsigned long long *)a.hd + (j < n64 ? j : 0));
        }
#pragma unroll
        for (int i = 0; i < kHrecPT; i++) {
          const int j = t + i * kT;
          if (j < n64) ((unsigned long long *)hrec)[j] = hv[i];
        }
        for (int j = t + kHrecPT * kT; j < n64; j += kT)
          ((unsigned long long *)hrec)[j] = ld_agent((const unsigned long long *)a.hd + j);
      }

      wait_dma();     // this wave's LDS copies have landed
      lds_barrier();  // ... and every other wave's; every h record is in
      if (tile < ntiles) {
        const int c = lane & 15, kb = lane >> 4;
        const bool lo = c < 8 && (c >> 1) == kb;
        const bool hi = c >= 8 && ((c - 8) >> 1) == kb;
        const int chb = lo ? kb : 4 + kb;
        // routed: per tile-group two MFMAs; B column c = (chunk c>>1, digit c&1).
        // Wave w takes the tile-groups q = j*ngi + g with q % kW == w; the
        // route weight is folded into the h records' digit scales (the
        // combine's sum over routes, per wave).  Items go in pairs, both
        // pairs' LDS operands read before either is computed.
        struct DOps {
          TileWord<FMT> cw;
          v4f s4;
          v4i d0, d1;  // MFMA B operands of both steps (zero where the lane's column is the other step's)
          float dscl, zq;
        };
        auto load_ops = [&](DOps &o, int jq, int gq) {
          const unsigned char *tq = dtile + (size_t)(jq * a.ngi + gq) * kSlot;
          if constexpr (FMT == 4) {
            const v4u v = *(const v4u *)(tq + 16 * lane);
            o.cw.w[0] = v.x;
            o.cw.w[1] = v.y;
            o.cw.w[2] = v.z;
            o.cw.w[3] = v.w;
          } else {
            const unsigned *wp = (const unsigned *)(tq + 12 * lane);
            o.cw.w[0] = wp[0];
            o.cw.w[1] = wp[1];
            o.cw.w[2] = wp[2];
          }
          o.s4 = *(const v4f *)(tq + 64 * BPL + 16 * kb);
          const unsigned *rbase = hrec + (size_t)(jq * a.ngi * 8 + gq * 8) * kRecWords;
          const v4i *dp = (const v4i *)(rbase + chb * kRecWords + (c & 1) * 4);
          o.d0 = *(lo ? dp : (const v4i *)zero16);
          o.d1 = *(hi ? dp : (const v4i *)zero16);
          // digit scale and offset correction (route weight folded in; an
          // invalid route's are zero)
          const unsigned *prm = rbase + (c >> 1) * kRecWords + 8;
          o.dscl = __uint_as_float(prm[c & 1]);
          o.zq = __uint_as_float(prm[2 + (c & 1)]);
        };
        float tot[4] = {0, 0, 0, 0};
        auto compute = [&](const DOps &o) {
          v4i a0, a1;
          unpack_tile<FMT>(o.cw, a0, a1);
          v4i cc = {0, 0, 0, 0};
          cc = mfma_i8(a0, o.d0, cc);
          cc = mfma_i8(a1, o.d1, cc);
          const float sv[4] = {o.s4.x, o.s4.y, o.s4.z, o.s4.w};
#pragma unroll
          for (int r = 0; r < 4; r++) tot[r] = __builtin_fmaf(__builtin_fmaf((float)cc[r], o.dscl, -o.zq), sv[r], tot[r]);
        };
        // this wave's items, one per lane: item i is tile-group q = wave + kW*i
        // (route q / ngi, group q % ngi)
        const int nitw = nq > wave ? (nq - 1 - wave) / kW + 1 : 0;  // <= 64 (K*ngi <= 512)
        int jl = 0, gl = 0;
        {
          const int q = wave + kW * lane;
          jl = q / a.ngi;
          gl = q - jl * a.ngi;
        }
        for (int i = 0; i < nitw; i += 2) {
          DOps o0, o1;
          const bool two = i + 1 < nitw;
          load_ops(o0, __builtin_amdgcn_readlane(jl, i), __builtin_amdgcn_readlane(gl, i));
          if (two) load_ops(o1, __builtin_amdgcn_readlane(jl, i + 1), __builtin_amdgcn_readlane(gl, i + 1));
          compute(o0);
          if (two) compute(o1);
        }
        // the next layer's stage R inputs, loaded while this stage finishes
        // (HBM is otherwise idle then)
        if (l + 1 < a.n) static_load(a, layer_ref_lds(s_lref[(l + 1) & 1]), sh_task_lds(s_sht), sreg, t);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float v = row16_sum(tot[r]);
          if (c == 0) part[wave * 16 + 4 * kb + r] = v;
        }
        lds_barrier();
        if (t < kTileRows) {
          // moe_forward's combine (routed sum, then fma(shared, gate)); the
          // routed sum is taken per wave, then over the waves in order
          float out = 0.0f;
#pragma unroll
          for (int w = 0; w < kW; w++) out += part[w * 16 + t];
          int dot = 0;
#pragma unroll
          for (int w = 0; w < kW; w++) dot += shp[w * 16 + t];
          const float shv = heavy ? hshv : (float)dot * dsr * shx;
          out = __builtin_fmaf(shv, rt.sg, out);
          a.y[(size_t)l * a.ys + tile * kTileRows + t] = out;
        }
        // the layer barrier's arrival follows the workgroup's output rows
        // directly (their stores issued by this wave)
        if (t == 0 && l + 1 < a.n) bar_arrive(bar_of(a, cs, l, kBarY), a.NB);
      } else if (l + 1 < a.n) {
        if (t == 0) bar_arrive(bar_of(a, cs, l, kBarY), a.NB);
        static_load(a, layer_ref_lds(s_lref[(l + 1) & 1]), sh_task_lds(s_sht), sreg, t);
      }
      // The next layer's stage R inputs are in flight (every wave's share,
      // issued before the combine).  Wave 0's returning barrier arrival
      // waits behind its share (a wave's loads complete in order); deferring
      // that share past the barrier measured slower (it then delays the next
      // layer's router pass).
      lds_barrier();
    }

    // ======================= barrier y (next layer) =======================
    stamp(a, l, 6);
    if (l + 1 < a.n) {
      if (t == 0) rt.flag = bar_wait(bar_of(a, cs, l, kBarY), a) ? 1 : 0;
      lds_barrier();
      if (__builtin_expect(!rt.flag, 0)) return;
      stamp(a, l, 7);
    }
  }
}

}  // namespace

// ===========================================================================
// host side
// ===========================================================================
namespace sw {

static LayerRef make_ref(const ColiMoeLayer *L) {
  LayerRef r;
  memset(&r, 0, sizeof(r));
  r.router = (const SW_G float *)L->router;
  r.sgate = (const SW_G float *)L->sgate_row;
  r.gq = (const SW_G signed char *)L->sh_gq;
  r.uq = (const SW_G signed char *)L->sh_uq;
  r.dq = (const SW_G signed char *)L->sh_dq;
  r.gs = (const SW_G float *)L->sh_gs;
  r.us = (const SW_G float *)L->sh_us;
  r.ds = (const SW_G float *)L->sh_ds;
  r.experts = (const SW_G unsigned char *)L->experts;
  r.stats = (SW_G unsigned long long *)L->stats;
  r.mode = L->router_mode;
  return r;
}

// Bytes of the stage-local LDS union: the largest of stage R's inputs,
// the selection's arrays, stage G's ring and stage D's layout.
static size_t stack_union_bytes(int E, int H, int K, int ngh, int ngi, int Ish, int fmt, int rslots, int shkc) {
  const size_t rlay = r_lds_bytes();
  const size_t u = u_layout(E, H, K, ngi, Ish, fmt).end;
  return u > rlay ? u : rlay;
}

// shared gate/up tasks: 16-row tiles of both matrices, each split into KQ
// k-ranges (KQ at most NB / tiles, E / tiles and H / 64)
static int stack_kq(int NB, int H, int E, int Ish) {
  const int nsh_rt = 2 * (Ish / kTileRows);
  if (nsh_rt == 0) return 1;
  int KQ = NB / nsh_rt;
  if (KQ > E / nsh_rt) KQ = E / nsh_rt;
  if (KQ > H / 64) KQ = H / 64;
  return KQ < 1 ? 1 : KQ;
}

bool stack_shape_ok(const ColiCuda *ctx, const ColiMoeShape &s) {
  const int NB = ctx->sm_count;
  const int H = s.hidden, E = s.experts, K = s.topk, I = s.intermediate, Ish = s.shared_intermediate;
  if (H > 2048 * kNch || H % 64 || K > kMaxK || K > E || I % 16 || Ish % 64 || Ish > kStackMaxIsh) return false;
  if ((E + NB - 1) / NB > kRSlots) return false;                     // router rows in registers
  if (E > kStackMaxE) return false;                                   // selection keys in registers
  if (2 * (Ish / kTileRows) > NB) return false;                       // one shared task per workgroup
  if (Ish > 64 * NB) return false;                                    // shared hidden: a lane per value
  const int ngh = (H + kGroup - 1) / kGroup, ngi = (I + kGroup - 1) / kGroup;
  if ((ngh + kW - 1) / kW > kGMax) return false;                     // G: groups per wave
  if (K * ngi > 64 * kW) return false;                                // D: one item per lane of a wave
  if (H / kTileRows > NB) return false;                               // D: one output tile per workgroup
  if ((K * (I / kTileRows) + NB - 1) / NB > 64) return false;         // G: one entry per lane
  const int Hp = ngh * kGroup;
  const int rslots = (E + NB - 1) / NB;
  const int KQ = stack_kq(NB, H, E, Ish);
  if (2 * (Ish / kTileRows) * KQ > E) return false;                  // tasks' workgroups own records
  const int shkc = (H / 64 + KQ - 1) / KQ;
  if ((shkc + kW - 1) / kW > kShMaxKc) return false;                 // shared task A operands in registers
  const size_t u = stack_union_bytes(E, H, K, ngh, ngi, Ish, s.expert_format, rslots, shkc);
  return lds_fixed(Hp, ngh, Ish) + u + 1024 <= (size_t)ctx->shared_per_block;
}

// Scratch regions at offsets that no shape changes: a tagged word must never
// land where another shape's untagged data (exact logits) was written.
constexpr size_t kRecRegion = ((size_t)(kStackMaxE + 1) * 16 + 255) & ~(size_t)255;  // router records
constexpr size_t kExRegion = ((size_t)kStackMaxE * 4 + 255) & ~(size_t)255;          // exact logits
constexpr size_t kStateRegion = 256;                                                  // call state
constexpr size_t kHsRegion = (size_t)kStackMaxIsh * 8;                                 // shared hidden vector
constexpr size_t kShvRegion = (size_t)2048 * kNch * 4;                                 // paired shared down values

static int stack_prepare(ColiCuda *ctx, int n, const ColiMoeShape &s) {
  // device scratch: records, exact logits, h records; per layer and parity:
  // counters and the shared expert's integer sums
  const size_t acc_words = 2 * (size_t)kStackMaxIsh;
  const size_t per_layer = ((size_t)kBars * kBarWords * 4 + acc_words * 8) * 2;
  if (n > ctx->stack_cap_layers) {
    hipError_t e = hipSuccess;
    if (ctx->stack_sync) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess && ctx->stack_sync) e = hipFree(ctx->stack_sync);
    ctx->stack_sync = nullptr;
    int cap = n < 64 ? 64 : n;
    if (e == hipSuccess) e = hipMalloc(&ctx->stack_sync, per_layer * cap);
    if (e == hipSuccess) e = hipMemsetAsync(ctx->stack_sync, 0, per_layer * cap, ctx->stream);
    if (e != hipSuccess) return fail_hip("MoE stack counter allocation", e);
    ctx->stack_cap_layers = cap;
  }
  const int ngi = (s.intermediate + kGroup - 1) / kGroup;
  const size_t scratch =
      kRecRegion + kExRegion + kStateRegion + kHsRegion + kShvRegion + (size_t)s.topk * ngi * 8 * kRecWords * 4;
  const void *before = ctx->scratch[kScrStack];
  if (ensure_scratch(ctx, kScrStack, scratch, "MoE stack scratch allocation")) return -1;
  if (ctx->scratch[kScrStack] != before) {
    // tagged words are trusted by their low byte: fresh memory starts at zero
    // (a tag is never 0); a fresh call state says nothing is dirty, so the
    // counters and integer sums are cleared with it
    hipError_t e = hipMemsetAsync(ctx->scratch[kScrStack], 0, ctx->scratch_cap[kScrStack], ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(ctx->stack_sync, 0, per_layer * ctx->stack_cap_layers, ctx->stream);
    if (e != hipSuccess) return fail_hip("MoE stack scratch clear", e);
  }
  if (!ctx->stack_abort) {
    hipError_t e = hipMalloc(&ctx->stack_abort, 256);
    if (e == hipSuccess) e = hipMemsetAsync(ctx->stack_abort, 0, 256, ctx->stream);
    if (e == hipSuccess) e = hipHostMalloc((void **)&ctx->stack_abort_host, 64, hipHostMallocMapped | hipHostMallocCoherent);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void **)&ctx->stack_abort_host_dev, ctx->stack_abort_host, 0);
    if (e != hipSuccess) return fail_hip("MoE stack status allocation", e);
    *ctx->stack_abort_host = 0;
  }
  return 0;
}

static int stack_table(ColiCuda *ctx, ColiMoeLayer *const *layers, int n, const SW_G LayerRef **out) {
  // the device copy of the layer table; re-uploaded only when the list changes
  bool same = ctx->stack_table_n == n && ctx->stack_table_dev;
  LayerRef *host = (LayerRef *)malloc(sizeof(LayerRef) * n);
  if (!host) return fail_arg("out of memory building the MoE layer table");
  for (int l = 0; l < n; l++) host[l] = make_ref(layers[l]);
  if (same) same = ctx->stack_table_host && memcmp(ctx->stack_table_host, host, sizeof(LayerRef) * n) == 0;
  if (!same) {
    hipError_t e = hipSuccess;
    if ((size_t)n > ctx->stack_table_cap) {
      if (ctx->stack_table_dev) {
        e = hipStreamSynchronize(ctx->stream);
        if (e == hipSuccess) e = hipFree(ctx->stack_table_dev);
      }
      ctx->stack_table_dev = nullptr;
      if (e == hipSuccess) e = hipMalloc(&ctx->stack_table_dev, sizeof(LayerRef) * n);
      if (e != hipSuccess) {
        free(host);
        return fail_hip("MoE layer table allocation", e);
      }
      ctx->stack_table_cap = n;
    }
    // pageable source: the runtime has consumed it when the call returns
    e = hipMemcpyAsync(ctx->stack_table_dev, host, sizeof(LayerRef) * n, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
      free(host);
      return fail_hip("MoE layer table upload", e);
    }
    free(ctx->stack_table_host);
    ctx->stack_table_host = host;
    ctx->stack_table_n = n;
  } else {
    free(host);
  }
  *out = (const SW_G LayerRef *)ctx->stack_table_dev;
  return 0;
}

int stack_check_abort(ColiCuda *ctx) {
  if (!ctx->stack_abort_host || !*ctx->stack_abort_host) return 0;
  // clear the device state the aborted call left behind
  *ctx->stack_abort_host = 0;
  const size_t per_layer = ((size_t)kBars * kBarWords * 4 + 2 * (size_t)kStackMaxIsh * 8) * 2;
  (void)hipMemsetAsync(ctx->stack_sync, 0, per_layer * ctx->stack_cap_layers, ctx->stream);
  (void)hipMemsetAsync(ctx->stack_abort, 0, 256, ctx->stream);
  if (ctx->scratch[kScrStack])  // tagged words an aborted call left behind
    (void)hipMemsetAsync(ctx->scratch[kScrStack], 0, ctx->scratch_cap[kScrStack], ctx->stream);
  (void)hipStreamSynchronize(ctx->stream);
  return fail_arg("MoE stack step aborted: a grid barrier timed out (the kernel needs every workgroup "
                  "resident; another kernel may have held compute units)");
}

int stack_step(ColiCuda *ctx, ColiMoeLayer *const *layers, int n, float *y, size_t ys, const float *x, size_t xs,
               int *route_idx, float *route_weight) {
  const ColiMoeShape s = layers[0]->sh;
  for (int l = 1; l < n; l++)
    if (memcmp(&layers[l]->sh, &s, sizeof(s))) return 1;
  if (!stack_shape_ok(ctx, s)) return 1;
  if (stack_check_abort(ctx)) return -1;
  if (stack_prepare(ctx, n, s)) return -1;
  const ColiMoeLayer *L0 = layers[0];
  StackArgs a;
  memset(&a, 0, sizeof(a));
  if (n == 1) {
    a.one = make_ref(L0);
  } else if (stack_table(ctx, layers, n, &a.table)) {
    return -1;
  }
  a.n = n;
  a.H = s.hidden;
  a.E = s.experts;
  a.K = s.topk;
  a.I = s.intermediate;
  a.Ish = s.shared_intermediate;
  a.fmt = s.expert_format;
  a.ngh = L0->ngh;
  a.ngi = L0->ngi;
  a.Hp = a.ngh * kGroup;
  a.nrt_i = a.I / kTileRows;
  a.nch = (a.H + 2047) / 2048;
  a.expert_bytes = L0->xl.expert_bytes;
  a.gu_bytes = L0->xl.gu_bytes;
  a.NB = ctx->sm_count;
  a.rslots = (a.E + a.NB - 1) / a.NB;
  const int nsh_rt = 2 * (a.Ish / kTileRows);
  const int KQ = stack_kq(a.NB, a.H, a.E, a.Ish);
  a.KQ = KQ;
  a.n_sh_tasks = nsh_rt * KQ;
  a.shkc = (a.H / 64 + KQ - 1) / KQ;
  a.x = x;
  a.xs = xs;
  a.y = y;
  a.ys = ys;
  a.route_idx = route_idx;
  a.route_w = route_weight;
  char *scr = (char *)ctx->scratch[kScrStack];
  a.rec = (double *)scr;
  a.ex = (float *)(scr + kRecRegion);
  a.hs = (unsigned long long *)(scr + kRecRegion + kExRegion + kStateRegion);
  a.shv = (float *)(scr + kRecRegion + kExRegion + kStateRegion + kHsRegion);
  a.hd = (unsigned *)(scr + kRecRegion + kExRegion + kStateRegion + kHsRegion + kShvRegion);
  const size_t acc_words = 2 * (size_t)kStackMaxIsh;
  a.bars = (unsigned *)ctx->stack_sync;
  a.acc = (unsigned long long *)((unsigned *)ctx->stack_sync + (size_t)ctx->stack_cap_layers * 2 * kBars * kBarWords);
  a.acc_stride = acc_words;
  a.state = (unsigned *)(scr + kRecRegion + kExRegion);
  a.abort_word = (unsigned *)ctx->stack_abort;
  a.abort_host = ctx->stack_abort_host_dev;
  a.spin_ticks = 200000000LL;  // 2 s of the 100 MHz wall clock
  a.absent = 0;
  if (ctx->stack_drill_absent) {  // coli_cuda_moe_stack_drill: disarmed at the launch
    a.absent = ctx->stack_drill_absent;
    a.spin_ticks = ctx->stack_drill_ticks;
  }
  a.trace = (unsigned long long *)ctx->stack_trace;
  a.trace_words = ctx->stack_trace_words;
  if (!a.trace) {
    // stage profiling: the launch's stages come from its own clock stamps
    if (ctx->prof.stamp_layers > 0) {
      // an earlier launch of this transaction still holds the buffer
      (void)hipStreamSynchronize(ctx->stream);
      prof_flush_stamps(ctx);
    }
    a.trace = prof_stamp_buffer(ctx, n, &a.trace_words);
  }
  const size_t Hp = (size_t)a.Hp;
  const size_t u = stack_union_bytes(a.E, a.H, a.K, a.ngh, a.ngi, a.Ish, a.fmt, a.rslots, a.shkc);
  size_t lds = lds_fixed((int)Hp, a.ngh, a.Ish) + u;
  // more than half of a CU's LDS: exactly one workgroup per CU
  const size_t one_per_cu = (size_t)ctx->shared_per_block / 2 + 1024;
  if (lds < one_per_cu) lds = one_per_cu;
  if (lds + 1024 > (size_t)ctx->shared_per_block) return 1;
  hipError_t e;
  {
    // every workgroup must be resident at once, one per compute unit: a
    // compute unit must hold one with this LDS (registers and waves
    // included), else the shape takes the three-kernel path
    size_t &fit = ctx->stack_fit_lds[a.fmt == 4];
    if (fit != lds) {
      int per_cu = 0;
      const void *fn = a.fmt == 4 ? (const void *)k_stack<4> : (const void *)k_stack<3>;
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kT, lds);
      if (e != hipSuccess) return fail_hip("MoE stack occupancy query", e);
      if (per_cu < 1) return 1;
      fit = lds;
    }
  }
  ctx->stack_drill_absent = 0;
  if (a.fmt == 4) {
    e = hipFuncSetAttribute((const void *)k_stack<4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) k_stack<4><<<a.NB, kT, lds, ctx->stream>>>(a);
  } else {
    e = hipFuncSetAttribute((const void *)k_stack<3>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) k_stack<3><<<a.NB, kT, lds, ctx->stream>>>(a);
  }
  if (e != hipSuccess) return fail_hip("MoE stack kernel attributes", e);
  int rc = launch_status("MoE stack step");
  if (rc) return rc;
  prof_mark(ctx, kStageStamped);  // the launch's span; its stamps split it
  return 0;
}

void stack_release(ColiCuda *ctx) {
  if (ctx->stack_sync) (void)hipFree(ctx->stack_sync);
  if (ctx->stack_table_dev) (void)hipFree(ctx->stack_table_dev);
  free(ctx->stack_table_host);
  if (ctx->stack_abort) (void)hipFree(ctx->stack_abort);
  if (ctx->stack_abort_host) (void)hipHostFree(ctx->stack_abort_host);
  ctx->stack_sync = nullptr;
  ctx->stack_table_dev = nullptr;
  ctx->stack_table_host = nullptr;
  ctx->stack_abort = nullptr;
  ctx->stack_abort_host = nullptr;
}

}  // namespace sw

extern "C" int coli_cuda_moe_stack_trace(ColiCuda *ctx, unsigned long long *trace, size_t words) {
  if (!ctx || (words && !trace)) return sw::fail_arg("coli_cuda_moe_stack_trace: invalid argument");
  ctx->stack_trace = trace;
  ctx->stack_trace_words = trace ? words : 0;
  return 0;
}

extern "C" int coli_cuda_moe_stack_drill(ColiCuda *ctx, int absent_workgroups, int wait_limit_us) {
  if (!ctx) return sw::fail_arg("coli_cuda_moe_stack_drill: null context");
  if (absent_workgroups < 0 || absent_workgroups >= ctx->sm_count)
    return sw::fail_arg("coli_cuda_moe_stack_drill: %d absent workgroups (0 disarms, at most %d)", absent_workgroups,
                        ctx->sm_count - 1);
  if (absent_workgroups && (wait_limit_us < 1 || wait_limit_us > 2000000))
    return sw::fail_arg("coli_cuda_moe_stack_drill: wait limit %d us outside [1, 2000000]", wait_limit_us);
  ctx->stack_drill_absent = absent_workgroups;
  ctx->stack_drill_ticks = 100LL * wait_limit_us;  // 100 MHz wall clock
  return 0;
}
