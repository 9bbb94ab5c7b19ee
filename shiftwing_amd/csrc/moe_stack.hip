// Batch-1 decode through a stack of HBM-resident MoE layers in ONE persistent
// kernel (moe_forward, c/qwen.c:3717-3739, applied layer after layer).
//
// One workgroup of 512 threads per CU, all resident for the whole call.  Per
// layer l, every workgroup runs four stages separated by grid barriers:
//
//   R  router rows (fp64 logit + rigorous bound of the reference's serial fp32
//      dot, c/qwen.c:1674) for the rows this workgroup owns (row r belongs to
//      workgroup r % NB), one shared-expert gate/up IDOT task (exact int32
//      dots, c/qwen.c:1696-1705, summed over k-slices with integer atomics),
//      and the activation digits of x for the routed GEMV.
//   -- barrier "lb": every router record and shared sum is published.
//   S  every workgroup selects the top-k itself from the published records
//      (router_topk, c/qwen.c:3421-3426): certified by the bounds, else by
//      the exact fp32 chains of the ambiguous experts (computed by the rows'
//      owners and exchanged through one more barrier), else by the reference's
//      full computation on every expert's exact chain.
//   G  routed gate/up: units (route, 16 rows) over the grid; each unit's
//      h = silu(g) * u (c/qwen.c:3419) is quantised into two int8 digits per
//      16-value chunk and published as a 48-byte record.
//   -- barrier "h".
//   D  routed down + shared down + combine for 16 output rows per task, in
//      moe_forward's order (fma over k in route order, then shared * gate).
//   -- barrier "y" (strict decode order: layer l+1 starts after layer l).
//
// Weights that do not depend on the token (the next layer's router rows and
// shared gate/up tile) are loaded into registers before the "y" barrier; the
// down tiles of the selected experts are loaded before the "h" barrier.
//
// Cross-workgroup data is published with returning device-scope atomics and
// read with device-scope loads; barriers are two-level counters (8 groups,
// then one top counter).  Counters and integer sums come in two parity sets:
// a call uses set p and clears set 1-p for the next call, so no call needs a
// memset and the host keeps no device state beyond the parity.  Every wait is
// bounded in wall-clock time: on expiry the kernel raises an abort flag, every
// workgroup leaves, and the host reports the error at the next sync.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sw_backend.h"
#include "sw_device.h"
#include "sw_moe_kernels.h"
#include "sw_moe_layer.h"
#include "sw_stack.h"

using namespace sw;

namespace {

constexpr int kT = 512;          // threads per workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kMaxK = kStackMaxK;
constexpr int kRSlots = 3;       // router rows per workgroup held in registers
constexpr int kNch = 2;          // 2048-float chunks per router row (H <= 4096)
constexpr int kSPF = 4;          // shared gate/up k-chunks per lane held in registers
constexpr int kMaxAmbig = 64;    // experts the targeted exact selection can take
constexpr int kLine = 32;        // words between counters (one 128-byte line)
constexpr int kBars = 5;         // barriers per layer: lb, exact-1, exact-2, h, y
constexpr int kBarWords = 9 * kLine;
constexpr int kRecWords = 12;    // h chunk record: d1[16] d2[16] (8 words) | A B Q1 Q2
enum { kBarLb = 0, kBarEx1, kBarEx2, kBarH, kBarY };

// Layer pointers as the kernel receives them: typed as device-global memory,
// so that every access through them compiles to global (not flat) memory
// instructions.  LayerPtrs is the same set as plain pointers.
#define SW_G __attribute__((address_space(1)))
struct LayerRef {
  const SW_G float *router, *sgate;
  const SW_G signed char *gq, *uq, *dq;
  const SW_G float *gs, *us, *ds;
  const SW_G unsigned char *codes;
  const SW_G float *scales;
  SW_G unsigned long long *stats;
  int mode, pad;
};
struct LayerPtrs {
  const float *router, *sgate;
  const signed char *gq, *uq, *dq;
  const float *gs, *us, *ds;
  const unsigned char *codes;
  const float *scales;
  unsigned long long *stats;
  int mode;
};

struct StackArgs {
  LayerRef one;                 // n == 1
  const SW_G LayerRef *table;   // n > 1
  int n;
  int H, E, K, I, Ish, fmt, ngh, ngi, Hp, nrt_i, nch;
  size_t expert_codes, expert_scales, gate_codes, gate_scales;
  int NB, rslots, KQ, n_sh_tasks;
  const float *x;
  size_t xs;
  float *y;
  size_t ys;
  int *route_idx;
  float *route_w;
  double *rec;          // [E+1][2] logit, bound
  float *ex;            // [E] exact logits
  unsigned *hd;         // [K][ngi*8][kRecWords]
  int *acc;             // [layer][parity][2*Ish]
  unsigned *bars;       // [layer][parity][kBars][kBarWords]
  size_t acc_stride;    // words per (layer, parity) acc block
  int parity;
  int zero_layers;      // layers of the other parity to clear
  int zero_acc_words;
  unsigned *abort_word; // device
  unsigned *abort_host; // host-mapped status
  long long spin_ticks; // wall-clock budget of one wait (100 MHz ticks)
  unsigned long long *trace;  // optional stage stamps [layer][NB][kStamps]
  size_t trace_words;
};

// Optional per-stage wall-clock stamps (100 MHz device clock), thread 0 of
// every workgroup: layer start, R done, lb passed, S done, G done, h passed,
// D done, y passed.
constexpr int kStamps = 8;
__device__ __forceinline__ void stamp(const StackArgs &a, int l, int k) {
  if (a.trace && threadIdx.x == 0) {
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

// Field by field, so that the kernel-argument copy and the table copy are
// never merged into one flat pointer.
__device__ __forceinline__ LayerPtrs layer_ref(const StackArgs &a, int l) {
  LayerPtrs p;
  const bool one = a.n == 1;
#define SW_FIELD(f, T) p.f = (T)(one ? a.one.f : a.table[l].f)
  SW_FIELD(router, const float *);
  SW_FIELD(sgate, const float *);
  SW_FIELD(gq, const signed char *);
  SW_FIELD(uq, const signed char *);
  SW_FIELD(dq, const signed char *);
  SW_FIELD(gs, const float *);
  SW_FIELD(us, const float *);
  SW_FIELD(ds, const float *);
  SW_FIELD(codes, const unsigned char *);
  SW_FIELD(scales, const float *);
  SW_FIELD(stats, unsigned long long *);
#undef SW_FIELD
  p.mode = one ? a.one.mode : a.table[l].mode;
  return p;
}
__device__ __forceinline__ unsigned *bar_of(const StackArgs &a, int l, int which) {
  return a.bars + ((size_t)(l * 2 + a.parity) * kBars + which) * kBarWords;
}

// ---------------------------------------------------------------------------
// Bounded waits and the two-level grid barrier (thread 0 acts; the caller
// brackets with __syncthreads and distributes the result through LDS).
// ---------------------------------------------------------------------------
__device__ bool wait_ge(const unsigned *p, unsigned target, const StackArgs &a) {
  const long long t0 = (long long)wall_clock64();
  for (unsigned it = 0;; it++) {
    if (ld_agent(p) >= target) return true;
    if ((it & 31) == 31) {
      if (ld_agent(a.abort_word)) return false;
      if ((long long)wall_clock64() - t0 > a.spin_ticks) {
        atomicMax(a.abort_word, 1u);
        __hip_atomic_store(a.abort_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// arrive: the workgroup's published words must have returned already
__device__ __forceinline__ void bar_arrive(unsigned *bar, int NB) {
  const int g = blockIdx.x & 7;
  const unsigned cnt = (unsigned)((NB - 1 - g) / 8 + 1);
  unsigned old = atomicAdd(&bar[kLine * (1 + g)], 1u);
  if (old == cnt - 1) atomicAdd(&bar[0], 1u);
}
__device__ __forceinline__ bool bar_wait(unsigned *bar, const StackArgs &a) {
  return wait_ge(&bar[0], (unsigned)(a.NB < 8 ? a.NB : 8), a);
}

// ---------------------------------------------------------------------------
// wave helpers
// ---------------------------------------------------------------------------
#define SW_DPP_D_ADD(v, ctrl, rm, bc)                             \
  {                                                               \
    int lo_ = SW_DPP_I(0, (int)__double2loint(v), ctrl, rm, bc); \
    int hi_ = SW_DPP_I(0, (int)__double2hiint(v), ctrl, rm, bc); \
    v += __hiloint2double(hi_, lo_);                              \
  }
__device__ __forceinline__ double wave_inclusive_scan_d(double v) {
  SW_DPP_D_ADD(v, 0x111, 0xF, true);
  SW_DPP_D_ADD(v, 0x112, 0xF, true);
  SW_DPP_D_ADD(v, 0x114, 0xF, true);
  SW_DPP_D_ADD(v, 0x118, 0xF, true);
  SW_DPP_D_ADD(v, 0x142, 0xA, false);
  SW_DPP_D_ADD(v, 0x143, 0xC, false);
  return v;
}
// total of each 16-lane row, in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v += SW_DPP_F(0.0f, v, 0xB1, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x4E, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x141, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x140, 0xF, true);
  return v;
}
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
__host__ __device__ inline size_t lds_fixed(int Hp, int ngh) {
  return (((size_t)2 * Hp + 15) & ~(size_t)15) + (size_t)ngh * 16 + (((size_t)Hp + 15) & ~(size_t)15) + 16;
}
__device__ __forceinline__ Lds lds_carve(unsigned char *smem, int Hp, int ngh) {
  Lds s;
  s.xd = (signed char *)smem;
  s.xgp = (float4 *)(smem + (((size_t)2 * Hp + 15) & ~(size_t)15));
  s.xq = (signed char *)(s.xgp + ngh);
  s.u = smem + lds_fixed(Hp, ngh);
  return s;
}

// Stage D's part of the stage-local union: h records, the shared hidden
// vector, partial sums, then the LDS-loaded down tiles and shared down rows
// (placed past everything stage G uses, since they are loaded before the "h"
// barrier while stage G's buffers may still be read).
struct DLayout {
  size_t hrec, hsh, hq, part, shp, redm, dtile, dsh, end;
};
__host__ __device__ inline DLayout d_layout(int K, int ngi, int Ish, int fmt) {
  DLayout d;
  size_t o = 0;
  auto take = [&o](size_t n) {
    const size_t p = o;
    o = (o + n + 15) & ~(size_t)15;
    return p;
  };
  const size_t bpl = fmt == 4 ? 16 : 12;
  d.hrec = take((size_t)K * ngi * 8 * kRecWords * 4);
  d.hsh = take((size_t)Ish * 4);
  d.hq = take((size_t)Ish);
  d.part = take((size_t)kMaxK * kW * 16 * 4);
  d.shp = take((size_t)kW * 16 * 4);
  d.redm = take((size_t)kW * 4);
  d.dtile = take((size_t)K * ngi * (64 * bpl + 64));
  d.dsh = take((size_t)kTileRows * (Ish + 16));
  d.end = o;
  return d;
}

// Per-workgroup registers carried between stages.
struct RouterRegs {
  v4f w[kRSlots * kNch];  // router rows: slot s, chunk c -> floats 2048c + 4t
};
typedef RowPrefetch<kSPF> SharedRegs;

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
__device__ __forceinline__ void sh_wave_range(const ShTask &t, int wave, int &k0, int &k1) {
  const int n = t.kc1 - t.kc0;
  k0 = t.kc0 + wave * n / kW;
  k1 = t.kc0 + (wave + 1) * n / kW;
}

// Loads that do not depend on the token: router rows and the shared task.
// Every register is written (zero where there is nothing to load), so no
// stale value stays live across the stages in between.
__device__ __forceinline__ void prefetch_static(const StackArgs &a, const LayerPtrs &L, RouterRegs &rr,
                                                SharedRegs &sr) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
  for (int s = 0; s < kRSlots; s++) {
    const int r = blockIdx.x + s * a.NB;
    const bool rv = s < a.rslots && r <= a.E;
    const float *row = r < a.E ? L.router + (size_t)r * a.H : L.sgate;
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      const int e0 = 2048 * c + 4 * t;
      v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (rv && c < a.nch && e0 < a.H) v = __builtin_nontemporal_load((const v4f *)(row + e0));
      rr.w[s * kNch + c] = v;
    }
  }
  const ShTask st = sh_task(a);
  int k0 = 0, k1 = 0;
  if (st.valid) sh_wave_range(st, wave, k0, k1);
  const signed char *arow = (st.m == 0 ? L.gq : L.uq) + (size_t)(st.rt * kTileRows + (lane & 15)) * a.H + (lane >> 4) * 16;
#pragma unroll
  for (int i = 0; i < kSPF; i++) {
    v4i v = {0, 0, 0, 0};
    if (st.valid && k0 + i < k1) v = __builtin_nontemporal_load((const v4i *)(arow + (size_t)(k0 + i) * 64));
    sr.a[i] = v;
  }
}

// ---------------------------------------------------------------------------
// Stage R
// ---------------------------------------------------------------------------
struct RStageLds {
  double segT[kRSlots][kNch * 8];
  double Ap[kRSlots][kW], Pp[kRSlots][kW];
  float red[kW];
  int acc_i[kW][16];
};

// The exact fp32 chain of the reference's dot() for the listed slots (rows
// b + s*NB): products rn(x*w) written to LDS by every thread, then one lane per
// slot adds them in index order (H % 8 == 0: no fused tail).  Rows and x are
// read again from memory: this path is rare, and keeping them in registers
// through the selection would cost every stage after it.
__device__ __forceinline__ void exact_chains(const StackArgs &a, const LayerPtrs &L, const float *x, unsigned want,
                                             float *prod, float *out) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int s = 0; s < kRSlots; s++)
    if (want & (1u << s)) {
      const int r = blockIdx.x + s * a.NB;
      const float *row = L.router + (size_t)r * a.H;
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
  __syncthreads();
  if (lane == 0 && wave < kRSlots && (want & (1u << wave))) {
    const float *p = prod + (size_t)wave * a.H;
    float acc = 0.0f;
    v4f nx = *(const v4f *)p;
    for (int i = 0; i < a.H; i += 4) {
      const v4f cur = nx;
      if (i + 4 < a.H) nx = *(const v4f *)(p + i + 4);
      acc = acc + cur.x;
      acc = acc + cur.y;
      acc = acc + cur.z;
      acc = acc + cur.w;
    }
    out[wave] = acc;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Stage S: selection from the published records (all workgroups identically).
// ---------------------------------------------------------------------------
struct SelLds {
  int cand[kMaxK + 1];
  int state;      // 0 certified, 1 targeted exact, 2 full exact
  int nm;
  int m[kMaxAmbig];
  float exv[kMaxAmbig];
  float sl[kMaxAmbig];
  int se[kMaxAmbig];
  float mx, den;
  int chosen[kMaxK];
  float wsel[kMaxK];
};

struct Routes {  // result of stage S, in static LDS
  int idx[kMaxK];
  float w[kMaxK];
  float sg;      // sigmoid of the shared gate logit
  int flag;      // barrier result broadcast
};

__device__ bool sync_barrier(const StackArgs &a, int l, int which, Routes &rt) {
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned *bar = bar_of(a, l, which);
    bar_arrive(bar, a.NB);
    rt.flag = bar_wait(bar, a) ? 1 : 0;
  }
  __syncthreads();
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
  __shared__ float s_misc[4];  // [0] sx of x
  const int b = blockIdx.x;
  const Lds S = lds_carve(smem, a0.Hp, a0.ngh);
  if (threadIdx.x < 4) ((int *)zero16)[threadIdx.x] = 0;

  // clear the other parity set's counters and integer sums for the next call
  {
    const StackArgs &a = a0;
    const int t = threadIdx.x;
    const int op = a.parity ^ 1;
    const size_t bw = (size_t)kBars * kBarWords;
    for (int l = 0; l < a.zero_layers; l++) {
      unsigned *bz = a.bars + (size_t)(l * 2 + op) * bw;
      for (size_t i = (size_t)b * kT + t; i < bw; i += (size_t)a.NB * kT) bz[i] = 0u;
      int *az = a.acc + (size_t)(l * 2 + op) * a.acc_stride;
      for (size_t i = (size_t)b * kT + t; i < (size_t)a.zero_acc_words; i += (size_t)a.NB * kT) az[i] = 0;
    }
  }

  RouterRegs rr;
  SharedRegs sr;
  prefetch_static(a0, layer_ref(a0, 0), rr, sr);

  for (int l = 0; l < a0.n; l++) {
    // Lane indices are re-derived every layer: values hoisted out of the loop
    // would stay live through every stage and spill.
    const StackArgs &a = a0;
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    const int lane = t & 63, wave = t >> 6;
    const LayerPtrs L = layer_ref(a, l);
    const float *x = a.x + (size_t)l * a.xs;
    int *acc = a.acc + (size_t)(l * 2 + a.parity) * a.acc_stride;

    // ======================= stage R =======================
    stamp(a, l, 0);
    RStageLds &R = *(RStageLds *)S.u;
    v4f xv[kNch];
#pragma unroll
    for (int c = 0; c < kNch; c++) {
      const int e0 = 2048 * c + 4 * t;
      xv[c] = (c < a.nch && e0 < a.H) ? *(const v4f *)(x + e0) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // routed activation digits, one 128-group per wave
    for (int g = wave; g < a.ngh; g += kW) quantize_group(x, a.H, g, S.xd, S.xd + a.Hp, S.xgp, lane);
    // qrow_i8 of x (c/qwen.c:1696): amax, sx = amax/127 (floor 1e-12), q = rint(x/sx)
    {
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < kNch; c++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[c].x), fabsf(xv[c].y)), fmaxf(fabsf(xv[c].z), fabsf(xv[c].w))));
      m = wave_max_dpp(m);
      if (lane == 0) R.red[wave] = m;
    }
    // router pass 1: segment totals and |products|
    double Aacc[kRSlots];
#pragma unroll
    for (int s = 0; s < kRSlots; s++) {
      Aacc[s] = 0.0;
      const int r = b + s * a.NB;
      if (s < a.rslots && r <= a.E) {
#pragma unroll
        for (int c = 0; c < kNch; c++) {
          if (c < a.nch) {
            const int e0 = 2048 * c + 4 * t;
            double p0 = 0, p1 = 0, p2 = 0, p3 = 0;
            if (e0 < a.H) {
              const v4f w = rr.w[s * kNch + c];
              p0 = (double)xv[c].x * (double)w.x;
              p1 = (double)xv[c].y * (double)w.y;
              p2 = (double)xv[c].z * (double)w.z;
              p3 = (double)xv[c].w * (double)w.w;
            }
            Aacc[s] += fabs(p0) + fabs(p1) + fabs(p2) + fabs(p3);
            const double q = wave_sum_dpp(((p0 + p1) + p2) + p3);
            if (lane == 0) R.segT[s][c * 8 + wave] = q;
          }
        }
      }
    }
    __syncthreads();
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
    // router pass 2: exact prefix sums -> sum |S_k|
#pragma unroll
    for (int s = 0; s < kRSlots; s++) {
      const int r = b + s * a.NB;
      double P = 0.0;
      if (s < a.rslots && r <= a.E) {
#pragma unroll
        for (int c = 0; c < kNch; c++) {
          if (c < a.nch) {
            const int e0 = 2048 * c + 4 * t;
            double carry = 0.0;
            for (int k = 0; k < c * 8 + wave; k++) carry += R.segT[s][k];
            double p0 = 0, p1 = 0, p2 = 0, p3 = 0;
            if (e0 < a.H) {
              const v4f w = rr.w[s * kNch + c];
              p0 = (double)xv[c].x * (double)w.x;
              p1 = (double)xv[c].y * (double)w.y;
              p2 = (double)xv[c].z * (double)w.z;
              p3 = (double)xv[c].w * (double)w.w;
            }
            const double q0 = p0, q1 = q0 + p1, q2 = q1 + p2, q3 = q2 + p3;
            const double inc = wave_inclusive_scan_d(q3);
            const double pre = carry + (inc - q3);
            if (e0 < a.H) P += fabs(pre + q0) + fabs(pre + q1) + fabs(pre + q2) + fabs(pre + q3);
          }
        }
        const double As = wave_sum_dpp(Aacc[s]);
        P = wave_sum_dpp(P);
        if (lane == 0) {
          R.Ap[s][wave] = As;
          R.Pp[s][wave] = P;
        }
      }
    }
    // shared gate/up task: exact int32 dots of 16 rows with xq
    const ShTask st = sh_task(a);
    __syncthreads();  // xq, segT, Ap/Pp complete
    v4i cs = {0, 0, 0, 0};
    if (st.valid) {
      int k0, k1;
      sh_wave_range(st, wave, k0, k1);
      const bool bvalid = (lane & 15) == 0;
      const int ke = k0 + kSPF < k1 ? k0 + kSPF : k1;
      rows_compute<kSPF>(sr, k0, ke, S.xq, 0, bvalid, cs, lane);
      for (int kc = ke; kc < k1; kc += kSPF) {
        const int e1 = kc + kSPF < k1 ? kc + kSPF : k1;
        idot_tile<kSPF>(st.m == 0 ? L.gq : L.uq, a.H, st.rt * kTileRows, kc, e1, S.xq, 0, bvalid, cs, lane);
      }
      if ((lane & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) R.acc_i[wave][4 * (lane >> 4) + i] = cs[i];
      }
    }
    __syncthreads();
    if (wave == 0) {
      unsigned dep = 0;
      // router records of this workgroup's rows: lanes 2s (logit), 2s+1 (bound)
      if (lane < 2 * kRSlots) {
        const int s = lane >> 1;
        const int r = b + s * a.NB;
        if (s < a.rslots && r <= a.E) {
          double Lg = 0.0, A = 0.0, P = 0.0;
          for (int k = 0; k < a.nch * 8; k++) Lg += R.segT[s][k];
#pragma unroll
          for (int w = 0; w < kW; w++) {
            A += R.Ap[s][w];
            P += R.Pp[s][w];
          }
          const double B = 0x1p-24 * (A + P) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-36;
          dep ^= pub(&a.rec[2 * r + (lane & 1)], (lane & 1) ? B : Lg);
        }
      }
      if (st.valid && lane >= 16 && lane < 32) {
        const int r = lane - 16;
        int v = 0;
#pragma unroll
        for (int w = 0; w < kW; w++) v += R.acc_i[w][r];
        dep ^= (unsigned)atomicAdd(&acc[st.m * a.Ish + st.rt * kTileRows + r], v);
      }
      published(dep);
    }
    stamp(a, l, 1);
    if (!sync_barrier(a, l, kBarLb, rt)) return;
    stamp(a, l, 2);

    // ======================= stage S =======================
    {
      SelLds &sel = *(SelLds *)S.u;
      double2 *lb = (double2 *)(S.u + ((sizeof(SelLds) + 15) & ~(size_t)15));
      unsigned long long *lk = (unsigned long long *)(lb + a.E + 1);
      float *prod = (float *)((unsigned char *)lk + (((size_t)a.E * 8 + 15) & ~(size_t)15));  // [kRSlots][H]
      const int E = a.E, K = a.K;
      for (int e = t; e <= E; e += kT) {
        const double2 v = make_double2(ld_agent(&a.rec[2 * e]), ld_agent(&a.rec[2 * e + 1]));
        lb[e] = v;
        if (e < E) lk[e] = ((unsigned long long)float_key((float)v.x) << 32) | (unsigned)(~e);
      }
      if (t == 0) sel.nm = 0;
      __syncthreads();
      if (wave == 0) {
        const int nc = K + 1 < E ? K + 1 : E;
        for (int r = 0; r < nc; r++) {
          unsigned long long best = 0;
          for (int e = lane; e < E; e += 64) best = lk[e] > best ? lk[e] : best;
          best = wave_max_u64(best);
          const int e = (int)(~(unsigned)best);
          if ((e & 63) == lane) lk[e] = 0;
          if (lane == 0) sel.cand[r] = e;
        }
        __builtin_amdgcn_wave_barrier();
        const int candK = K < E ? sel.cand[K] : -1;
        unsigned long long upk = 0;
        for (int e = lane; e < E; e += 64)
          if (lk[e] != 0 || e == candK) {
            const unsigned long long k2 = double_key(lb[e].x + lb[e].y);
            upk = k2 > upk ? k2 : upk;
          }
        upk = wave_max_u64(upk);
        const double mx = lb[sel.cand[0]].x;
        const double2 kth = lb[sel.cand[K - 1]];
        bool pair_ok = true;
        if (lane + 1 < K) {
          const double2 p = lb[sel.cand[lane]], q = lb[sel.cand[lane + 1]];
          pair_ok = (p.x - p.y) - (q.x + q.y) > order_margin(p.x, q.x, mx);
        }
        bool ok = L.mode == 0 && __all(pair_ok);
        if (ok && K < E) {
          const double up = key_double(upk);
          ok = (kth.x - kth.y) - up > order_margin(kth.x, up, mx);
        }
        if (ok) ok = (kth.x - kth.y) - (mx + lb[sel.cand[0]].y) > -75.0;
        int state = 0;
        if (ok) {
          const double ev = lane < K ? exp(lb[sel.cand[lane < K ? lane : 0]].x - mx) : 0.0;
          const double den = wave_sum_dpp(ev);
          if (lane < K) {
            rt.idx[lane] = sel.cand[lane];
            rt.w[lane] = (float)(ev / den);
          }
        } else if (L.mode != 0) {
          state = 2;
        } else {
          double theta = 1e300;
          for (int r = 0; r < K; r++) theta = fmin(theta, lb[sel.cand[r]].x - lb[sel.cand[r]].y);
          for (int e = lane; e < E; e += 64) {
            const double2 v = lb[e];
            if (v.x + v.y >= theta - order_margin(v.x, theta, mx)) {
              const int slot = atomicAdd(&sel.nm, 1);
              if (slot < kMaxAmbig) sel.m[slot] = e;
            }
          }
          __builtin_amdgcn_wave_barrier();
          state = sel.nm <= kMaxAmbig && sel.nm >= K ? 1 : 2;
        }
        if (lane == 0) {
          sel.state = state;
          rt.sg = sigmoid_ref((float)lb[E].x);
          if (b == 0) {
            atomicAdd(&L.stats[0], 1ull);
            if (state != 0) atomicAdd(&L.stats[1], 1ull);
          }
        }
      }
      __syncthreads();
      if (sel.state == 1) {
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
        if (!sync_barrier(a, l, kBarEx1, rt)) return;
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
            const double ev = lane < K ? exp((double)sel.sl[lane < K ? lane : 0] - mx) : 0.0;
            const double den = wave_sum_dpp(ev);
            if (lane < K) {
              rt.idx[lane] = sel.se[lane];
              rt.w[lane] = (float)(ev / den);
            }
          }
          if (lane == 0 && !ok) sel.state = 2;
        }
        __syncthreads();
      }
      if (sel.state == 2) {
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
        if (!sync_barrier(a, l, kBarEx2, rt)) return;
        float *lgs = prod;  // [E]
        for (int e = t; e < E; e += kT) lgs[e] = ld_agent(&a.ex[e]);
        __syncthreads();
        if (wave == 0) {
          float m = -__builtin_huge_valf();
          for (int e = lane; e < E; e += 64) m = fmaxf(m, lgs[e]);
          m = wave_max_dpp(m);
          if (lane == 0) sel.mx = m;
        }
        __syncthreads();
        for (int e = t; e < E; e += kT) lgs[e] = expf_glibc(lgs[e] - sel.mx);
        __syncthreads();
        if (t == 0) {
          float den = 0.0f;
          for (int e = 0; e < E; e++) den += lgs[e];
          sel.den = den;
        }
        __syncthreads();
        for (int e = t; e < E; e += kT) lgs[e] = lgs[e] / sel.den;
        __syncthreads();
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
            if (b == 0) atomicAdd(&L.stats[2], 1ull);
          }
        }
        __syncthreads();
      }
      if (b == 0 && t < K) {
        if (a.route_idx) a.route_idx[t] = rt.idx[t];
        if (a.route_w) a.route_w[t] = rt.w[t];
      }
      __syncthreads();  // the selection's LDS is reused below
    }
    stamp(a, l, 3);

    // ======================= stage G =======================
    {
      float(*red)[16] = (float(*)[16])S.u;              // [kW][16]
      unsigned *stage = (unsigned *)(S.u + kW * 16 * 4);  // [8] packed digits
      const int nU = a.K * a.nrt_i;
      const int m = wave >> 2, qd = wave & 3;
      const int per = (a.ngh + 3) / 4, g0 = qd * per;
      const int n = (a.ngh < g0 + per ? a.ngh : g0 + per) - g0;
      const DigitSrc src = lane_digits(lane, 1, S.xd, a.Hp, S.xgp, a.ngh, zero16);
      // pieces of 4 groups: piece k = (unit b + (k/2)*NB, half k%2), loaded one ahead
      auto load_piece = [&](TilePrefetch<FMT, 4> &tp, int k) {
        const int u = b + (k >> 1) * a.NB;
        const int j = u / a.nrt_i, r16 = u % a.nrt_i;
        const int e = rt.idx[j];
        const int ga = g0 + (k & 1) * 4;
        const int nn = n - (k & 1) * 4;
        if ((unsigned)e < (unsigned)a.E && nn > 0)
          tile_prefetch<FMT, 4>(tp, L.codes + (size_t)e * a.expert_codes + (size_t)m * a.gate_codes,
                                L.scales + (size_t)e * a.expert_scales + (size_t)m * a.gate_scales, r16, a.ngh,
                                ga, nn < 4 ? nn : 4, lane);
      };
      auto compute_piece = [&](const TilePrefetch<FMT, 4> &tp, int k, float acc4[4]) {
        const int u = b + (k >> 1) * a.NB;
        const int e = rt.idx[u / a.nrt_i];
        const int ga = g0 + (k & 1) * 4;
        const int nn = n - (k & 1) * 4;
        if ((unsigned)e < (unsigned)a.E && nn > 0) tile_compute<FMT, 4>(tp, ga, nn < 4 ? nn : 4, src, acc4, lane);
      };
      unsigned dep = 0;
      auto finish_unit = [&](float acc4[4], int u) {
        const int j = u / a.nrt_i, r16 = u % a.nrt_i;
        const int e = rt.idx[j];
        digit_fold(acc4);
        if ((lane & 15) == 1) {
#pragma unroll
          for (int i = 0; i < 4; i++) red[wave][4 * (lane >> 4) + i] = acc4[i];
        }
        __syncthreads();
        if (wave == 0 && lane < 16) {
          const int r = lane;
          const float gsum = red[0][r] + red[1][r] + red[2][r] + red[3][r];
          const float usum = red[4][r] + red[5][r] + red[6][r] + red[7][r];
          float h = silu_ref(gsum) * usum;  // c/qwen.c:3419
          if ((unsigned)e >= (unsigned)a.E || r16 * kTileRows + r >= a.I) h = 0.0f;
          // two int8 digits of this 16-value chunk: A = amax/127, B = A/254
          float mm = fabsf(h);
          mm = fmaxf(mm, __shfl_xor(mm, 1, 16));
          mm = fmaxf(mm, __shfl_xor(mm, 2, 16));
          mm = fmaxf(mm, __shfl_xor(mm, 4, 16));
          mm = fmaxf(mm, __shfl_xor(mm, 8, 16));
          const float A = mm / 127.0f, B = A / 254.0f;
          int q1 = 0, q2 = 0;
          if (mm > 0.0f) {
            const float invA = 127.0f / mm, invB = 254.0f / A;
            q1 = (int)fminf(fmaxf(__builtin_rintf(h * invA), -127.0f), 127.0f);
            const float rr2 = __builtin_fmaf(-(float)q1, A, h);
            q2 = (int)fminf(fmaxf(__builtin_rintf(rr2 * invB), -127.0f), 127.0f);
          }
          int s1 = q1, s2 = q2;
          s1 += __shfl_xor(s1, 1, 16);
          s1 += __shfl_xor(s1, 2, 16);
          s1 += __shfl_xor(s1, 4, 16);
          s1 += __shfl_xor(s1, 8, 16);
          s2 += __shfl_xor(s2, 1, 16);
          s2 += __shfl_xor(s2, 2, 16);
          s2 += __shfl_xor(s2, 4, 16);
          s2 += __shfl_xor(s2, 8, 16);
          ((signed char *)stage)[r] = (signed char)q1;
          ((signed char *)stage)[16 + r] = (signed char)q2;
          __builtin_amdgcn_wave_barrier();
          unsigned v = 0;
          if (r < 8) v = stage[r];
          else if (r == 8) v = __float_as_uint(A);
          else if (r == 9) v = __float_as_uint(B);
          else if (r == 10) v = (unsigned)s1;
          else if (r == 11) v = (unsigned)s2;
          if (r < kRecWords) dep ^= pub(&a.hd[((size_t)j * a.ngi * 8 + r16) * kRecWords + r], v);
        }
        __syncthreads();
      };
      const int nunits = b < nU ? (nU - 1 - b) / a.NB + 1 : 0;
      const int npieces = 2 * nunits;
      TilePrefetch<FMT, 4> ta, tb;
      float acc4[4] = {0, 0, 0, 0};
      if (npieces > 0) load_piece(ta, 0);
      for (int k = 0; k < npieces; k += 2) {
        load_piece(tb, k + 1);
        compute_piece(ta, k, acc4);
        if (k + 2 < npieces) load_piece(ta, k + 2);
        compute_piece(tb, k + 1, acc4);
        finish_unit(acc4, b + (k >> 1) * a.NB);
#pragma unroll
        for (int i = 0; i < 4; i++) acc4[i] = 0.0f;
      }
      // zero records of chunks past I inside the last group (only when I % 128 != 0)
      if (b == 0 && wave == 0) {
        const int pad = a.ngi * 8 - a.nrt_i;
        for (int i = lane; i < a.K * pad * kRecWords; i += 64) {
          const int j = i / (pad * kRecWords), rem = i % (pad * kRecWords);
          dep ^= pub(&a.hd[((size_t)j * a.ngi * 8 + a.nrt_i) * kRecWords + rem], 0u);
        }
      }
      if (wave == 0) published(dep);
    }

    // ======================= stage D (loads, then barrier h) =======================
    {
      const DLayout dl = d_layout(a.K, a.ngi, a.Ish, FMT);
      constexpr int BPL = FMT == 4 ? 16 : 12;
      constexpr int kSlot = 64 * BPL + 64;  // one tile-group: codes, then 16 row scales
      const int nq = a.K * a.ngi;
      const int qa = wave * nq / kW, qb = (wave + 1) * nq / kW;
      const int nkd = a.Ish / 64;
      const int dk0 = wave * nkd / kW, dk1 = (wave + 1) * nkd / kW;
      const int tile0 = b, ntiles = a.H / kTileRows;
      unsigned char *dtile = S.u + dl.dtile;
      signed char *dsh = (signed char *)(S.u + dl.dsh);
      // the tile's routed down tile-groups and shared down rows, straight into LDS
      auto issue_down = [&](int tile) {
        for (int q = qa; q < qb; q++) {
          const int j = q / a.ngi, g = q % a.ngi;
          const int e = rt.idx[j];
          if ((unsigned)e >= (unsigned)a.E) continue;
          const size_t tg = (size_t)tile * a.ngi + g;
          const unsigned char *src = L.codes + (size_t)e * a.expert_codes + 2 * a.gate_codes + (tg * 64 + lane) * BPL;
          if constexpr (FMT == 4) {
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (__attribute__((address_space(3))) void *)(dtile + (size_t)q * kSlot), 16, 0, 0);
          } else {
            // three dword planes [3][64]: plane i holds word i of every lane's 12 bytes
#pragma unroll
            for (int i = 0; i < 3; i++)
              __builtin_amdgcn_global_load_lds((const void *)(src + 4 * i),
                                               (__attribute__((address_space(3))) void *)(dtile + (size_t)q * kSlot + 256 * i),
                                               4, 0, 0);
          }
          if (lane < kTileRows)
            __builtin_amdgcn_global_load_lds(
                (const void *)(L.scales + (size_t)e * a.expert_scales + 2 * a.gate_scales + tg * kTileRows + lane),
                (__attribute__((address_space(3))) void *)(dtile + (size_t)q * kSlot + 64 * BPL), 4, 0, 0);
        }
        for (int r = wave; r < kTileRows; r += kW)
          for (int c0 = 0; c0 < a.Ish; c0 += 1024)
            if (c0 + 16 * lane < a.Ish)
              __builtin_amdgcn_global_load_lds(
                  (const void *)(L.dq + (size_t)(tile * kTileRows + r) * a.Ish + c0 + 16 * lane),
                  (__attribute__((address_space(3))) void *)(dsh + (size_t)r * (a.Ish + 16) + c0), 16, 0, 0);
      };
      if (tile0 < ntiles && wave != 0) issue_down(tile0);
      __syncthreads();
      stamp(a, l, 4);
      if (t == 0) bar_arrive(bar_of(a, l, kBarH), a.NB);
      if (tile0 < ntiles && wave == 0) issue_down(tile0);
      if (t == 0) rt.flag = bar_wait(bar_of(a, l, kBarH), a) ? 1 : 0;
      __syncthreads();
      if (!rt.flag) return;
      stamp(a, l, 5);

      // h records of every route -> LDS; shared hidden vector -> int8
      unsigned *hrec = (unsigned *)(S.u + dl.hrec);  // [K][ngi*8][12]
      float *hsh = (float *)(S.u + dl.hsh);          // [Ish]
      signed char *hq = (signed char *)(S.u + dl.hq);
      float *part = (float *)(S.u + dl.part);        // [K][kW][16]
      int *shp = (int *)(S.u + dl.shp);              // [kW][16]
      float *redm = (float *)(S.u + dl.redm);        // [kW]
      const int nrec_words = a.K * a.ngi * 8 * kRecWords;
      for (int i = t; i < nrec_words / 2; i += kT)
        ((unsigned long long *)hrec)[i] = ld_agent((const unsigned long long *)a.hd + i);
      for (int i = t; i < kMaxK * kW * 16; i += kT) part[i] = 0.0f;
      float hm = 0.0f;
      for (int i = t; i < a.Ish; i += kT) {
        const int ag = ld_agent(&acc[i]), au = ld_agent(&acc[a.Ish + i]);
        // IDOT epilogue ((float)dot * s_row) * sx (c/qwen.c:1766), then SwiGLU
        const float h = silu_ref((float)ag * L.gs[i] * sx) * ((float)au * L.us[i] * sx);
        hsh[i] = h;
        hm = fmaxf(hm, fabsf(h));
      }
      hm = wave_max_dpp(hm);
      if (lane == 0) redm[wave] = hm;
      __syncthreads();
      float shx = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; w++) shx = fmaxf(shx, redm[w]);
      shx = shx / 127.0f;
      if (shx < 1e-12f) shx = 1e-12f;
      {
        const float hinv = 1.0f / shx;
        for (int i = t; i < a.Ish; i += kT) hq[i] = (signed char)__builtin_rintf(hsh[i] * hinv);
      }

      for (int tile = tile0; tile < ntiles; tile += a.NB) {
        if (tile != tile0) issue_down(tile);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS loads have landed
        __syncthreads();                                    // ... and every other wave's
        constexpr int OFF = FMT == 4 ? 8 : 4;
        const int c = lane & 15, kb = lane >> 4;
        const bool lo = c < 8 && (c >> 1) == kb;
        const bool hi = c >= 8 && ((c - 8) >> 1) == kb;
        const int chb = lo ? kb : 4 + kb;
        // routed: per tile-group two MFMAs; B column c = (chunk c>>1, digit c&1)
        float accr[4] = {0, 0, 0, 0};
        int jcur = -1;
        for (int q = qa; q < qb; q++) {
          const int j = q / a.ngi, g = q % a.ngi;
          if (j != jcur) {
            if (jcur >= 0) {
#pragma unroll
              for (int r = 0; r < 4; r++) {
                const float v = row16_sum(accr[r]);
                if (c == 0) part[(jcur * kW + wave) * 16 + 4 * kb + r] = v;
                accr[r] = 0.0f;
              }
            }
            jcur = j;
          }
          const int e = rt.idx[j];
          if ((unsigned)e >= (unsigned)a.E) continue;
          const unsigned char *tq = dtile + (size_t)q * kSlot;
          TileWord<FMT> cw;
          if constexpr (FMT == 4) {
            const v4u v = *(const v4u *)(tq + 16 * lane);
            cw.w[0] = v.x;
            cw.w[1] = v.y;
            cw.w[2] = v.z;
            cw.w[3] = v.w;
          } else {
            const unsigned *wp = (const unsigned *)tq + lane;
            cw.w[0] = wp[0];
            cw.w[1] = wp[64];
            cw.w[2] = wp[128];
          }
          const v4f s4 = *(const v4f *)(tq + 64 * BPL + 16 * kb);
          v4i a0, a1;
          unpack_tile<FMT>(cw, a0, a1);
          const unsigned *rbase = hrec + (size_t)(j * a.ngi * 8 + g * 8) * kRecWords;
          const v4i dv = *(const v4i *)(rbase + chb * kRecWords + (c & 1) * 4);
          const v4i z = {0, 0, 0, 0};
          v4i cc = {0, 0, 0, 0};
          cc = mfma_i8(a0, lo ? dv : z, cc);
          cc = mfma_i8(a1, hi ? dv : z, cc);
          const unsigned *prm = rbase + (c >> 1) * kRecWords + 8;
          const float dscl = __uint_as_float(prm[c & 1]);
          const int Q = (int)prm[2 + (c & 1)];
          const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
          for (int r = 0; r < 4; r++) accr[r] = __builtin_fmaf((float)(cc[r] - OFF * Q) * dscl, sv[r], accr[r]);
        }
        if (jcur >= 0) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float v = row16_sum(accr[r]);
            if (c == 0) part[(jcur * kW + wave) * 16 + 4 * kb + r] = v;
          }
        }
        // shared down: exact int32 dots of 16 rows (LDS) with hq
        {
          v4i cd = {0, 0, 0, 0};
          const signed char *arow = dsh + (size_t)(lane & 15) * (a.Ish + 16) + kb * 16;
          for (int kc = dk0; kc < dk1; kc++) {
            const v4i av = *(const v4i *)(arow + kc * 64);
            const v4i bv = c == 0 ? *(const v4i *)(hq + kc * 64 + kb * 16) : v4i{0, 0, 0, 0};
            cd = mfma_i8(av, bv, cd);
          }
          if (c == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) shp[wave * 16 + 4 * kb + i] = cd[i];
          }
        }
        __syncthreads();
        if (t < kTileRows) {
          // moe_forward's combine: fma over k in route order, then shared * gate
          float out = 0.0f;
          for (int k = 0; k < a.K; k++) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < kW; w++) v += part[(k * kW + w) * 16 + t];
            out = __builtin_fmaf(v, rt.w[k], out);
          }
          int dot = 0;
#pragma unroll
          for (int w = 0; w < kW; w++) dot += shp[w * 16 + t];
          const float shv = (float)dot * L.ds[tile * kTileRows + t] * shx;
          out = __builtin_fmaf(shv, rt.sg, out);
          a.y[(size_t)l * a.ys + tile * kTileRows + t] = out;
        }
        __syncthreads();
        for (int i = t; i < kMaxK * kW * 16; i += kT) part[i] = 0.0f;
      }
      __syncthreads();
    }

    // ======================= barrier y (next layer) =======================
    stamp(a, l, 6);
    if (l + 1 < a.n) {
      __syncthreads();
      if (t == 0) bar_arrive(bar_of(a, l, kBarY), a.NB);
      prefetch_static(a, layer_ref(a, l + 1), rr, sr);
      if (t == 0) rt.flag = bar_wait(bar_of(a, l, kBarY), a) ? 1 : 0;
      __syncthreads();
      if (!rt.flag) return;
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
  r.codes = (const SW_G unsigned char *)L->codes;
  r.scales = (const SW_G float *)L->scales;
  r.stats = (SW_G unsigned long long *)L->stats;
  r.mode = L->router_mode;
  return r;
}

bool stack_shape_ok(const ColiCuda *ctx, const ColiMoeShape &s) {
  const int NB = ctx->sm_count;
  const int H = s.hidden, E = s.experts, K = s.topk, I = s.intermediate, Ish = s.shared_intermediate;
  if (H > 2048 * kNch || H % 64 || K > kMaxK || K > E || I % 16 || Ish % 64 || Ish > kStackMaxIsh) return false;
  if ((E + 1 + NB - 1) / NB > kRSlots) return false;                 // router rows in registers
  if (2 * (Ish / kTileRows) > NB) return false;                       // one shared task per workgroup
  const int ngh = (H + kGroup - 1) / kGroup, ngi = (I + kGroup - 1) / kGroup;
  if (ngh > 32) return false;                                         // G: 8 groups per wave
  const int Hp = ngh * kGroup;
  const size_t sel = ((sizeof(SelLds) + 15) & ~(size_t)15) + (size_t)(E + 1) * 16 + (size_t)E * 8 + 16 +
                     (size_t)kRSlots * H * 4;
  const size_t dst = d_layout(K, ngi, Ish, s.expert_format).end;
  size_t u = sizeof(RStageLds);
  if (sel > u) u = sel;
  if (dst > u) u = dst;
  return lds_fixed(Hp, ngh) + u <= (size_t)ctx->shared_per_block;
}

static int stack_prepare(ColiCuda *ctx, int n, const ColiMoeShape &s) {
  // device scratch: records, exact logits, h records; per layer and parity:
  // counters and the shared expert's integer sums
  const size_t acc_words = 2 * (size_t)kStackMaxIsh;
  const size_t per_layer = ((size_t)kBars * kBarWords + acc_words) * 2 * 4;
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
    ctx->stack_dirty[0] = ctx->stack_dirty[1] = 0;
    ctx->stack_dirty_acc[0] = ctx->stack_dirty_acc[1] = 0;
  }
  const int ngi = (s.intermediate + kGroup - 1) / kGroup;
  const size_t scratch = (size_t)(s.experts + 1) * 16 + 256 + (size_t)s.experts * 4 + 256 +
                         (size_t)s.topk * ngi * 8 * kRecWords * 4;
  if (ensure_scratch(ctx, kScrStack, scratch, "MoE stack scratch allocation")) return -1;
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
  const size_t per_layer = ((size_t)kBars * kBarWords + 2 * (size_t)kStackMaxIsh) * 2 * 4;
  hipMemsetAsync(ctx->stack_sync, 0, per_layer * ctx->stack_cap_layers, ctx->stream);
  hipMemsetAsync(ctx->stack_abort, 0, 256, ctx->stream);
  hipStreamSynchronize(ctx->stream);
  ctx->stack_dirty[0] = ctx->stack_dirty[1] = 0;
  ctx->stack_dirty_acc[0] = ctx->stack_dirty_acc[1] = 0;
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
  a.expert_codes = L0->expert_codes;
  a.expert_scales = L0->expert_scales;
  a.gate_codes = L0->gate_codes;
  a.gate_scales = L0->gate_scales;
  a.NB = ctx->sm_count;
  a.rslots = (a.E + 1 + a.NB - 1) / a.NB;
  const int nsh_rt = 2 * (a.Ish / kTileRows);
  int KQ = a.NB / nsh_rt;
  if (KQ < 1) KQ = 1;
  if (KQ > a.H / 64) KQ = a.H / 64;
  a.KQ = KQ;
  a.n_sh_tasks = nsh_rt * KQ;
  a.x = x;
  a.xs = xs;
  a.y = y;
  a.ys = ys;
  a.route_idx = route_idx;
  a.route_w = route_weight;
  char *scr = (char *)ctx->scratch[kScrStack];
  a.rec = (double *)scr;
  a.ex = (float *)(scr + (((size_t)(a.E + 1) * 16 + 255) & ~(size_t)255));
  a.hd = (unsigned *)((char *)a.ex + (((size_t)a.E * 4 + 255) & ~(size_t)255));
  const size_t acc_words = 2 * (size_t)kStackMaxIsh;
  a.bars = (unsigned *)ctx->stack_sync;
  a.acc = (int *)((unsigned *)ctx->stack_sync + (size_t)ctx->stack_cap_layers * 2 * kBars * kBarWords);
  a.acc_stride = acc_words;
  a.parity = (int)(ctx->stack_epoch & 1);
  const int op = a.parity ^ 1;
  a.zero_layers = ctx->stack_dirty[op];
  a.zero_acc_words = ctx->stack_dirty_acc[op];
  a.abort_word = (unsigned *)ctx->stack_abort;
  a.abort_host = ctx->stack_abort_host_dev;
  a.spin_ticks = 200000000LL;  // 2 s of the 100 MHz wall clock
  a.trace = (unsigned long long *)ctx->stack_trace;
  a.trace_words = ctx->stack_trace_words;
  const size_t Hp = (size_t)a.Hp;
  const size_t sel = ((sizeof(SelLds) + 15) & ~(size_t)15) + (size_t)(a.E + 1) * 16 + (size_t)a.E * 8 + 16 +
                     (size_t)kRSlots * a.H * 4;
  const size_t dst = d_layout(a.K, a.ngi, a.Ish, a.fmt).end;
  size_t u = sizeof(RStageLds);
  if (sel > u) u = sel;
  if (dst > u) u = dst;
  size_t lds = lds_fixed((int)Hp, a.ngh) + u;
  // more than half of a CU's LDS: exactly one workgroup per CU
  const size_t one_per_cu = (size_t)ctx->shared_per_block / 2 + 1024;
  if (lds < one_per_cu) lds = one_per_cu;
  if (lds > (size_t)ctx->shared_per_block) return 1;
  hipError_t e;
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
  ctx->stack_dirty[a.parity] = n;
  ctx->stack_dirty_acc[a.parity] = 2 * a.Ish;
  ctx->stack_epoch++;
  return 0;
}

void stack_release(ColiCuda *ctx) {
  if (ctx->stack_sync) hipFree(ctx->stack_sync);
  if (ctx->stack_table_dev) hipFree(ctx->stack_table_dev);
  free(ctx->stack_table_host);
  if (ctx->stack_abort) hipFree(ctx->stack_abort);
  if (ctx->stack_abort_host) hipHostFree(ctx->stack_abort_host);
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
