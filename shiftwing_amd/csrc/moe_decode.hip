// One decoded token through one HBM-resident MoE layer in three kernels
// (moe_forward, c/qwen.c:3717-3739):
//
//   K1 route   router workgroups (four router rows each: an fp64 logit and a
//              rigorous bound on the reference's serial fp32 dot), shared
//              expert workgroups (gate/up int8 dots, exact int32, split over k
//              and summed with integer atomics) and activation-digit
//              workgroups.  The last router workgroup to finish selects the
//              top-k: certified from the bounds, else from exact fp32 logits of
//              the experts the bounds leave ambiguous, else (near ties) by the
//              reference's full serial computation.  Router workgroups come
//              first in the grid, so the selection overlaps the shared-expert
//              streaming.
//   K2 experts one workgroup per (route, 16 rows): each wave takes a quarter
//              of the groups of both the gate and the up tile; the workgroup
//              writes h = silu(g) * u for its 16 rows.
//   K3 down    one workgroup per 16 output rows: one wave per route (it
//              quantises its route's h, 8 lanes per 128-group, while its down
//              tiles are in flight) and two waves for the shared down
//              projection, whose hidden vector every workgroup rebuilds from
//              the integer sums; then the reference's combine order.
//
// Fan-in (router rows in K1) publishes with device-scope atomics; every other
// hand-off is a kernel boundary.  Counters are reset by their last arriver.  The shared
// expert's integer sums alternate between two buffers (a parity word kept on
// the device), so the buffer one call reads is cleared by the next one.  No
// memset, no host state: consecutive calls and graph replays need nothing.
// Each kernel issues its weight loads before it waits for anything else.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sw_backend.h"
#include "sw_device.h"
#include "sw_moe_kernels.h"
#include "sw_moe_layer.h"

using namespace sw;

namespace {

constexpr int kMaxK = 32;
constexpr int kThreads = 256;       // K1 / K2 workgroup
constexpr int kMaxAmbig = 64;       // experts the targeted exact selection can take
constexpr int kMaxDownWaves = 10;   // K3 routed waves per workgroup (+1 shared)
constexpr int kSegPrefetch = 16;    // router row segments (of 256) loaded ahead

struct Dec {
  int H, E, K, I, Ish, ngh, ngi, Hp, Ip, KQ;
  int n_router_wg, n_shared_wg;
  signed char *xd;  // [2][Hp] routed activation digits
  float4 *xgp;      // [ngh]
  double2 *lb;      // [E+1] fp64 logit, bound (row E: shared gate)
  float *misc;      // [0] sx (IDOT scale of x)  [1] shared gate
  int *imisc;       // [0] parity of this call's integer sums
  int *idx;         // [K]
  float *w;         // [K]
  float *h;         // [K][I] routed hidden vectors silu(g) * u
  unsigned *cnt;    // per layer: [0] router fan-in  [1] parity
  int *acc;         // per layer: [2][2][Ish] shared gate/up int32 dots
};

size_t dec_carve(Dec &d, char *base) {
  size_t off = 0;
  auto take = [&](size_t n) -> char * {
    off = (off + 255) & ~(size_t)255;
    char *p = base ? base + off : nullptr;
    off += n;
    return p;
  };
  d.xd = (signed char *)take((size_t)2 * d.Hp);
  d.xgp = (float4 *)take((size_t)d.ngh * 16);
  d.lb = (double2 *)take((size_t)(d.E + 1) * 16);
  d.misc = (float *)take(32);
  d.imisc = (int *)take(32);
  d.idx = (int *)take((size_t)kMaxK * 4);
  d.w = (float *)take((size_t)kMaxK * 4);
  d.h = (float *)take((size_t)d.K * d.I * 4);
  return off + 256;
}

// inclusive DPP prefix sum of a double over the wave (lane order)
#define SW_DPP_D_ADD(v, ctrl, rm, bc)                             \
  {                                                               \
    int lo_ = SW_DPP_I(0, (int)__double2loint(v), ctrl, rm, bc); \
    int hi_ = SW_DPP_I(0, (int)__double2hiint(v), ctrl, rm, bc); \
    v += __hiloint2double(hi_, lo_);                              \
  }
__device__ __forceinline__ double wave_inclusive_scan_dpp(double v) {
  SW_DPP_D_ADD(v, 0x111, 0xF, true);
  SW_DPP_D_ADD(v, 0x112, 0xF, true);
  SW_DPP_D_ADD(v, 0x114, 0xF, true);
  SW_DPP_D_ADD(v, 0x118, 0xF, true);
  SW_DPP_D_ADD(v, 0x142, 0xA, false);
  SW_DPP_D_ADD(v, 0x143, 0xC, false);
  return v;
}
__device__ __forceinline__ double readlane63_d(double v) {
  int lo = __builtin_amdgcn_readlane((int)__double2loint(v), 63);
  int hi = __builtin_amdgcn_readlane((int)__double2hiint(v), 63);
  return __hiloint2double(hi, lo);
}

// ---------------------------------------------------------------------------
// Fan-in without release fences.  On this chip an agent-scope release fence
// writes back the issuing XCD's whole L2; issued by hundreds of workgroups
// they serialise into tens of microseconds.  Instead, a workgroup publishes
// its words with returning device-scope atomics (performed at the coherence
// point every XCD's device-scope atomics go through), waits for them to
// return, and only then bumps the counter with another device-scope atomic.
// The last arriver reads the published words with device-scope atomic loads,
// served from the same coherence point.
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned publish(float *p, float v) { return __float_as_uint(atomicExch(p, v)); }
__device__ __forceinline__ unsigned publish(unsigned long long *p, unsigned long long v) {
  unsigned long long o = atomicExch(p, v);
  return (unsigned)o ^ (unsigned)(o >> 32);
}
// Every publish of this wave has returned.  dep: the xor of the lane's
// publish results (0 for lanes that published nothing), consumed only here so
// that all of a wave's atomics are in flight together.
__device__ __forceinline__ void published(unsigned dep) {
  asm volatile("" ::"v"(dep));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ float read_published(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double read_published(const double *p) {
  unsigned long long v = __hip_atomic_load((const unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __longlong_as_double((long long)v);
}

// ---------------------------------------------------------------------------
// Router row bound.  The reference logit is dot() (c/qwen.c:1674), evaluated
// with gcc -O3 as s_k = rn(s_{k-1} + rn(x_k w_k)) (a tail of H%8 terms fused).
// With exact prefix sums S_k and u = 2^-24:
//   |s_H - L| <= u * (sum_k |x_k w_k| + sum_k |s_k|),  |s_k| <= |S_k| + err,
// so B = u (A + P) (1 + 2^-10) bounds the error for H <= 16384.  A wave
// walks the row in 256-element segments (float4 per lane, coalesced); S_k
// comes from an fp64 lane scan plus the running carry, exact to 1e-16.
// ---------------------------------------------------------------------------
struct RowSegs {
  v4f w[kSegPrefetch];
};

__device__ __forceinline__ void row_prefetch(RowSegs &s, const float *row, int H, int base, int lane) {
#pragma unroll
  for (int q = 0; q < kSegPrefetch; q++) {
    int i0 = base + 256 * q + 4 * lane;
    s.w[q] = i0 < H ? __builtin_nontemporal_load((const v4f *)(row + i0)) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
}

__device__ __forceinline__ void row_accumulate(const RowSegs &s, const float *xs, int H, int base, int lane,
                                               double &carry, double &A, double &P) {
#pragma unroll
  for (int q = 0; q < kSegPrefetch; q++) {
    if (base + 256 * q >= H) break;
    int i0 = base + 256 * q + 4 * lane;
    double p[4] = {0.0, 0.0, 0.0, 0.0};
    if (i0 < H) {
      float4 xv = *(const float4 *)(xs + i0);
      p[0] = (double)xv.x * (double)s.w[q].x;
      p[1] = (double)xv.y * (double)s.w[q].y;
      p[2] = (double)xv.z * (double)s.w[q].z;
      p[3] = (double)xv.w * (double)s.w[q].w;
    }
    double q0 = p[0], q1 = q0 + p[1], q2 = q1 + p[2], q3 = q2 + p[3];
    A += fabs(p[0]) + fabs(p[1]) + fabs(p[2]) + fabs(p[3]);
    double inc = wave_inclusive_scan_dpp(q3);
    double pre = carry + (inc - q3);
    if (i0 < H) P += fabs(pre + q0) + fabs(pre + q1) + fabs(pre + q2) + fabs(pre + q3);
    carry += readlane63_d(inc);
  }
}

__device__ __forceinline__ double2 row_finish(double carry, double A, double P) {
  A = wave_sum_dpp(A);
  P = wave_sum_dpp(P);
  const double u = 0x1p-24;
  double B = u * (A + P) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-36;
  return make_double2(carry, B);
}

// The reference's router logit bit for bit: dot() at c/qwen.c:1674 as gcc
// compiles it (products rounded, then added in index order; a fused tail of
// H%8 terms).  One chain per thread; rows streamed 32 floats ahead.
__device__ float exact_logit(const float *row, const float *xs, int H) {
  const int m8 = (H / 8) * 8;
  float s = 0.0f;
  int i = 0;
  for (; i + 32 <= m8; i += 32) {
    v4f a[8];
#pragma unroll
    for (int q = 0; q < 8; q++) a[q] = *(const v4f *)(row + i + 4 * q);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      float4 xv = *(const float4 *)(xs + i + 4 * q);
      s = s + xv.x * a[q].x;
      s = s + xv.y * a[q].y;
      s = s + xv.z * a[q].z;
      s = s + xv.w * a[q].w;
    }
  }
  for (; i < m8; i++) s = s + xs[i] * row[i];
  for (; i < H; i++) s = __builtin_fmaf(xs[i], row[i], s);
  return s;
}

// Separation that makes two logits' softmax probabilities strictly ordered
// after the reference's fp32 rounding (l - max, expf, division).
__device__ __forceinline__ double order_margin(double a, double b, double mx) {
  return 0x1p-20 * (1.0 + fabs(a) + fabs(b) + 2.0 * fabs(mx));
}


// ---------------------------------------------------------------------------
// Top-k selection by the last router workgroup (all 256 threads).
//   lds: at least 24*E + 16 bytes (bounds, then keys; reused for the exact
//   logits).  xs: x in LDS.
// Writes d.idx / d.w (router_topk's indices exactly; weights from the fp64
// logits, or the reference's fp32 values on the full serial path) and the
// shared gate.
// ---------------------------------------------------------------------------
__device__ void select_routes(const Dec &d, const float *xs, const float *router, int mode,
                              unsigned long long *stats, unsigned char *lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = d.E, K = d.K;
  double2 *lb = (double2 *)lds;                                 // [E+1]
  unsigned long long *lk = (unsigned long long *)(lb + E + 1);  // [E]
  __shared__ int s_cand[kMaxK + 1];
  __shared__ int s_state;  // 0 certified, 1 targeted exact, 2 full exact
  __shared__ int s_nm;
  __shared__ int s_m[kMaxAmbig];
  __shared__ float s_ex[kMaxAmbig];
  __shared__ float s_sl[kMaxAmbig];
  __shared__ int s_se[kMaxAmbig];
  // bounds -> LDS with device-scope loads, all issued before the first use
  constexpr int kLbRegs = 3;
  double bx[kLbRegs], by[kLbRegs];
#pragma unroll
  for (int q = 0; q < kLbRegs; q++) {
    int e = threadIdx.x + q * kThreads;
    e = e < E ? e : E;
    bx[q] = read_published(&d.lb[e].x);
    by[q] = read_published(&d.lb[e].y);
  }
#pragma unroll
  for (int q = 0; q < kLbRegs; q++) {
    int e = threadIdx.x + q * kThreads;
    if (e <= E) {
      lb[e] = make_double2(bx[q], by[q]);
      if (e < E) lk[e] = ((unsigned long long)float_key((float)bx[q]) << 32) | (unsigned)(~e);
    }
  }
  for (int e = threadIdx.x + kLbRegs * kThreads; e <= E; e += kThreads) {
    double2 b = make_double2(read_published(&d.lb[e].x), read_published(&d.lb[e].y));
    lb[e] = b;
    if (e < E) lk[e] = ((unsigned long long)float_key((float)b.x) << 32) | (unsigned)(~e);
  }
  if (threadIdx.x == 0) s_nm = 0;
  __syncthreads();
  if (wave == 0) {
    // top K+1 by fp64 logit (float keys, lowest index first on equal keys;
    // near-ties fail the separation tests below).  Lane l alone clears the
    // keys l+64i it scans, so the rounds need no LDS sync.
    const int nc = K + 1 < E ? K + 1 : E;
    for (int r = 0; r < nc; r++) {
      unsigned long long best = 0;
      for (int e = lane; e < E; e += 64) best = lk[e] > best ? lk[e] : best;
      best = wave_max_u64(best);
      int e = (int)(~(unsigned)best);
      if ((e & 63) == lane) lk[e] = 0;
      if (lane == 0) s_cand[r] = e;
    }
    __builtin_amdgcn_wave_barrier();
    // the largest upper bound outside the top K (selected keys are zero)
    const int candK = K < E ? s_cand[K] : -1;
    unsigned long long upk = 0;
    for (int e = lane; e < E; e += 64)
      if (lk[e] != 0 || e == candK) {
        unsigned long long k2 = double_key(lb[e].x + lb[e].y);
        upk = k2 > upk ? k2 : upk;
      }
    upk = wave_max_u64(upk);
    const double mx = lb[s_cand[0]].x;
    const double2 kth = lb[s_cand[K - 1]];
    // adjacent candidates separated (lane r tests the pair r, r+1)
    bool pair_ok = true;
    if (lane + 1 < K) {
      double2 a = lb[s_cand[lane]], b = lb[s_cand[lane + 1]];
      pair_ok = (a.x - a.y) - (b.x + b.y) > order_margin(a.x, b.x, mx);
    }
    bool ok = mode == 0 && __all(pair_ok);
    if (ok && K < E) {
      double up = key_double(upk);
      ok = (kth.x - kth.y) - up > order_margin(kth.x, up, mx);
    }
    // keep every selected probability a normal float (den <= E <= 4096)
    if (ok) ok = (kth.x - kth.y) - (mx + lb[s_cand[0]].y) > -75.0;
    int state = 0;
    if (ok) {
      double ev = lane < K ? exp(lb[s_cand[lane < K ? lane : 0]].x - mx) : 0.0;
      double den = wave_sum_dpp(ev);
      if (lane < K) {
        d.idx[lane] = s_cand[lane];
        d.w[lane] = (float)(ev / den);
      }
    } else if (mode != 0) {
      state = 2;
    } else {
      // Every expert whose upper bound reaches the lowest lower bound among
      // the K candidates (less a margin): the exact top K lies in this set,
      // since anything outside it is strictly below all K candidates.
      double theta = 1e300;
      for (int r = 0; r < K; r++) theta = fmin(theta, lb[s_cand[r]].x - lb[s_cand[r]].y);
      for (int e = lane; e < E; e += 64) {
        double2 b = lb[e];
        if (b.x + b.y >= theta - order_margin(b.x, theta, mx)) {
          int slot = atomicAdd(&s_nm, 1);
          if (slot < kMaxAmbig) s_m[slot] = e;
        }
      }
      __builtin_amdgcn_wave_barrier();
      state = s_nm <= kMaxAmbig && s_nm >= K ? 1 : 2;
    }
    if (lane == 0) {
      s_state = state;
      d.misc[1] = sigmoid_ref((float)lb[E].x);
      atomicAdd(&stats[0], 1ull);
      if (state != 0) atomicAdd(&stats[1], 1ull);
    }
  }
  __syncthreads();
  if (s_state == 1) {
    const int nm = s_nm;
    if ((int)threadIdx.x < nm) s_ex[threadIdx.x] = exact_logit(router + (size_t)s_m[threadIdx.x] * d.H, xs, d.H);
    __syncthreads();
    if (wave == 0) {
      // order by (exact logit desc, index asc) = router_topk's order whenever
      // consecutive logits are equal or separated by the margin
      float l = lane < nm ? s_ex[lane] : -__builtin_huge_valf();
      int e = lane < nm ? s_m[lane] : 0x7fffffff;
      int rank = 0;
      for (int q = 0; q < nm; q++) {
        float lq = s_ex[q];
        int eq = s_m[q];
        rank += (lq > l) || (lq == l && eq < e);
      }
      if (lane < nm) {
        s_sl[rank] = l;
        s_se[rank] = e;
      }
      __builtin_amdgcn_wave_barrier();
      const double mx = s_sl[0];
      bool pair_ok = true;
      if (lane < K && lane + 1 < nm) {
        double a = s_sl[lane], b = s_sl[lane + 1];
        pair_ok = a == b || a - b > order_margin(a, b, mx);
      }
      bool ok = __all(pair_ok) && ((double)s_sl[K - 1] - mx > -75.0);
      if (ok) {
        double ev = lane < K ? exp((double)s_sl[lane < K ? lane : 0] - mx) : 0.0;
        double den = wave_sum_dpp(ev);
        if (lane < K) {
          d.idx[lane] = s_se[lane];
          d.w[lane] = (float)(ev / den);
        }
      }
      if (lane == 0 && !ok) s_state = 2;
    }
    __syncthreads();
  }
  if (s_state != 2) return;
  if (threadIdx.x == 0) atomicAdd(&stats[2], 1ull);
  // router_topk (c/qwen.c:3421-3426) on the exact logits of every expert,
  // bit-exact: max, expf(l - max), serial denominator in expert order,
  // division, K argmax rounds (lowest index on ties), serial renormalisation.
  float *lgs = (float *)lk;  // [E]
  __shared__ float s_mx, s_den;
  for (int e = threadIdx.x; e < E; e += kThreads) lgs[e] = exact_logit(router + (size_t)e * d.H, xs, d.H);
  __syncthreads();
  if (wave == 0) {
    float m = -__builtin_huge_valf();
    for (int e = lane; e < E; e += 64) m = fmaxf(m, lgs[e]);
    m = wave_max_dpp(m);
    if (lane == 0) s_mx = m;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kThreads) lgs[e] = expf_glibc(lgs[e] - s_mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float den = 0.0f;
    for (int e = 0; e < E; e++) den += lgs[e];
    s_den = den;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kThreads) lgs[e] = lgs[e] / s_den;
  __syncthreads();
  if (wave == 0) {
    __shared__ int chosen[kMaxK];
    __shared__ float wsel[kMaxK];
    for (int j = 0; j < K; j++) {
      unsigned long long best = 0;
      for (int e = lane; e < E; e += 64) {
        bool used = false;
        for (int q = 0; q < j; q++) used |= chosen[q] == e;
        float pv = lgs[e];
        unsigned long long k2 = (((unsigned long long)float_key(pv)) << 32) | (unsigned)(~e);
        if (!used && pv > -1.0f && k2 > best) best = k2;
      }
      best = wave_max_u64(best);
      int c = best ? (int)(~(unsigned)best) : -1;
      if (lane == 0) {
        chosen[j] = c;
        wsel[j] = best ? lgs[c] : -1.0f;
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) {
      float topden = 0.0f;
      for (int j = 0; j < K; j++) topden += wsel[j];
      for (int j = 0; j < K; j++) {
        d.idx[j] = chosen[j];
        d.w[j] = wsel[j] / topden;
      }
    }
  }
}

// x [H] into LDS in two steps, so that the (cached) x loads are issued before
// a workgroup's weight loads: loads return in issue order.
constexpr int kXRegs = 4;
struct XRegs {
  v4f v[kXRegs];
};
// (unconditional loads at clamped indices: no branch ahead of the weights)
__device__ __forceinline__ void x_load(XRegs &xr, const float *x, int H) {
#pragma unroll
  for (int q = 0; q < kXRegs; q++) {
    int i = (q * kThreads + (int)threadIdx.x) * 4;
    xr.v[q] = *(const v4f *)(x + (i < H ? i : H - 4));
  }
}
__device__ __forceinline__ void x_store(const XRegs &xr, const float *x, float *xs, int H) {
#pragma unroll
  for (int q = 0; q < kXRegs; q++) {
    int i = (q * kThreads + (int)threadIdx.x) * 4;
    if (i < H) *(v4f *)(xs + i) = xr.v[q];
  }
  for (int i = (kXRegs * kThreads + (int)threadIdx.x) * 4; i < H; i += kThreads * 4)
    *(float4 *)(xs + i) = *(const float4 *)(x + i);
}

// ---------------------------------------------------------------------------
// K1.  grid: n_router_wg | n_shared_wg | digit workgroups; 256 threads.
// LDS: x [H] f32 | xq [H] i8 (shared rows) or bounds + keys (selection).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_dec_route(Dec d, const float *__restrict__ x,
                                                        const float *__restrict__ router,
                                                        const float *__restrict__ sgrow,
                                                        const signed char *__restrict__ gq,
                                                        const signed char *__restrict__ uq, int mode,
                                                        unsigned long long *stats) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x;
  if (b >= d.n_router_wg + d.n_shared_wg) {
    // activation digits for the routed experts, one 128-group per wave
    int g = (b - d.n_router_wg - d.n_shared_wg) * 4 + wave;
    if (g < d.ngh) quantize_group(x, d.H, g, d.xd, d.xd + d.Hp, d.xgp, lane);
    return;
  }
  float *xs = (float *)smem;
  unsigned char *tail = smem + (((size_t)d.H * 4 + 15) & ~(size_t)15);
  __shared__ float red[4];

  if (b < d.n_router_wg) {
    // ---- router rows: weights first, then x ----
    const int r = b * 4 + wave;
    const float *row = r < d.E ? router + (size_t)r * d.H : sgrow;
    XRegs xr;
    x_load(xr, x, d.H);
    RowSegs rs;
    if (r <= d.E) row_prefetch(rs, row, d.H, 0, lane);
    x_store(xr, x, xs, d.H);
    __syncthreads();
    __shared__ double2 s_lb[4];
    if (r <= d.E) {
      double carry = 0.0, A = 0.0, P = 0.0;
      row_accumulate(rs, xs, d.H, 0, lane, carry, A, P);
      for (int base = 256 * kSegPrefetch; base < d.H; base += 256 * kSegPrefetch) {
        row_prefetch(rs, row, d.H, base, lane);
        row_accumulate(rs, xs, d.H, base, lane, carry, A, P);
      }
      double2 bb = row_finish(carry, A, P);
      if (lane == 0) s_lb[wave] = bb;
    }
    __syncthreads();
    // fan-in: thread 0 publishes the workgroup's rows, releases, counts
    __shared__ unsigned s_last;
    if (wave == 0) {
      // lanes 0..7: one word each of the four (logit, bound) pairs
      unsigned dep = 0;
      const int q = lane >> 1;
      if (lane < 8 && b * 4 + q <= d.E) {
        double v = (lane & 1) ? s_lb[q].y : s_lb[q].x;
        dep = publish((unsigned long long *)&d.lb[b * 4 + q] + (lane & 1), (unsigned long long)__double_as_longlong(v));
      }
      published(dep);
      if (lane == 0) s_last = atomicAdd(&d.cnt[0], 1u) == (unsigned)d.n_router_wg - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x == 0) atomicExch(&d.cnt[0], 0u);
    select_routes(d, xs, router, mode, stats, tail);
    return;
  }

  // ---- shared expert gate/up: 16 rows x one k-slice per wave ----
  const int t = (b - d.n_router_wg) * 4 + wave;
  const int n_tasks = (d.Ish / kTileRows) * d.KQ;
  const int nk = d.H / 64;
  int rt = 0, kc0 = 0, kc1 = 0;
  if (t < n_tasks) {
    rt = t / d.KQ;
    int kq = t % d.KQ;
    kc0 = kq * nk / d.KQ;
    kc1 = (kq + 1) * nk / d.KQ;
  }
  XRegs xr;
  x_load(xr, x, d.H);
  const int p = (int)(d.cnt[1] & 1u);
  RowPrefetch<8> pg, pu;
  const int e0 = kc0 + 8 < kc1 ? kc0 + 8 : kc1;
  rows_prefetch<8>(pg, gq, d.H, rt * kTileRows, kc0, e0, lane);
  rows_prefetch<8>(pu, uq, d.H, rt * kTileRows, kc0, e0, lane);
  // x and its IDOT quantisation (qrow_i8, c/qwen.c:1696)
  x_store(xr, x, xs, d.H);
  float m = 0.0f;
  for (int i = threadIdx.x * 4; i < d.H; i += kThreads * 4) {
    float4 v = *(const float4 *)(xs + i);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  m = wave_max_dpp(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sx = amax / 127.0f;
  if (sx < 1e-12f) sx = 1e-12f;
  const float inv = 1.0f / sx;
  signed char *xq = (signed char *)tail;
  for (int i = threadIdx.x; i < d.H; i += kThreads) xq[i] = (signed char)__builtin_rintf(xs[i] * inv);
  __syncthreads();
  if (b == d.n_router_wg && threadIdx.x == 0) {
    d.misc[0] = sx;
    d.imisc[0] = p;
  }
  if (t >= n_tasks) return;
  v4i cg = {0, 0, 0, 0}, cu = {0, 0, 0, 0};
  const bool bvalid = (lane & 15) == 0;
  rows_compute<8>(pg, kc0, e0, xq, 0, bvalid, cg, lane);
  rows_compute<8>(pu, kc0, e0, xq, 0, bvalid, cu, lane);
  for (int kc = e0; kc < kc1; kc += 8) {
    int e1 = kc + 8 < kc1 ? kc + 8 : kc1;
    idot_tile<8>(gq, d.H, rt * kTileRows, kc, e1, xq, 0, bvalid, cg, lane);
    idot_tile<8>(uq, d.H, rt * kTileRows, kc, e1, xq, 0, bvalid, cu, lane);
  }
  if ((lane & 15) == 0) {
    int *acc = d.acc + (size_t)p * 2 * d.Ish;
    int r0 = rt * kTileRows + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      atomicAdd(&acc[r0 + i], cg[i]);
      atomicAdd(&acc[d.Ish + r0 + i], cu[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// K2: routed gate/up.  grid K * I/16 (route, row tile), 256 threads.  Wave w
// takes groups [w*per, w*per + per) of both matrices; the tile's scales for
// both matrices are staged in LDS, so a wave holds only codes in flight.
// LDS: digits [2][Hp] | group parameters [ngh] | scales [2][ngh][16].
// ---------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(kThreads) void k_dec_experts(Dec d, ExpertLayout xl) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float part[2][4][64][4];
  __shared__ __align__(16) signed char zero16[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
  const int n_rt = d.I / kTileRows;
  const int j = blockIdx.x / n_rt, rt = blockIdx.x % n_rt;
  signed char *dig = (signed char *)smem;                         // [2][Hp]
  float4 *gp = (float4 *)(smem + 2 * (size_t)d.Hp);               // [ngh]
  float *scl = (float *)(gp + d.ngh);                             // [2][ngh][16]
  // activation digits and group parameters (cached): unconditional loads at
  // clamped indices, issued before anything that depends on the route
  const int n16 = (2 * d.Hp) / 16;
  const v4i *xdv = (const v4i *)d.xd;
  const v4i dr0 = xdv[tid < n16 ? tid : n16 - 1];
  const v4i dr1 = xdv[tid + kThreads < n16 ? tid + kThreads : n16 - 1];
  const float4 gr = d.xgp[tid < d.ngh ? tid : d.ngh - 1];
  const int e = d.idx[j];
  if ((unsigned)e >= (unsigned)d.E) return;  // router_topk's -1: the route contributes nothing
  const TileMat mg = xl.mat(e, 0), mu = xl.mat(e, 1);
  // this row tile's scales (2 x ngh x 16 floats): quad i is matrix i / ns4,
  // group (i % ns4) / 4, rows 4 (i % 4) ..
  const int ns4 = d.ngh * 4;  // float4 per matrix
  auto scale_quad = [&](int i) {
    const int q = i % ns4;
    return *(const v4f *)(tm_scales(i < ns4 ? mg : mu, (size_t)rt * d.ngh + (q >> 2)) + 4 * (q & 3));
  };
  const int sq = tid < 2 * ns4 ? tid : 2 * ns4 - 1;
  const v4f sr = scale_quad(sq);
  const int per = (d.ngh + 3) / 4, g0 = wave * per;
  const int n = (d.ngh < g0 + per ? d.ngh : g0 + per) - g0;
  const DigitSrc src = lane_digits(lane, 1, dig, d.Hp, gp, d.ngh, zero16);
  float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0};
  // every wave runs the first iteration (it holds the workgroup barrier)
  for (int c0 = 0; c0 == 0 || c0 < n; c0 += 8) {
    const int nn = n - c0 < 8 ? n - c0 : 8;
    TileCodes<FMT, 8> tg, tu;
    tile_codes_prefetch<FMT, 8>(tg, mg, rt, d.ngh, g0 + c0, nn, lane);
    tile_codes_prefetch<FMT, 8>(tu, mu, rt, d.ngh, g0 + c0, nn, lane);
    if (c0 == 0) {
      if (tid < n16) ((v4i *)dig)[tid] = dr0;
      if (tid + kThreads < n16) ((v4i *)dig)[tid + kThreads] = dr1;
      for (int i = 2 * kThreads + tid; i < n16; i += kThreads) ((v4i *)dig)[i] = xdv[i];
      if (tid < d.ngh) gp[tid] = gr;
      for (int i = kThreads + tid; i < d.ngh; i += kThreads) gp[i] = d.xgp[i];
      if (tid < 2 * ns4) ((v4f *)scl)[tid] = sr;
      for (int i = kThreads + tid; i < 2 * ns4; i += kThreads)
        ((v4f *)scl)[i] = scale_quad(i);
      if (tid < 4) ((int *)zero16)[tid] = 0;
      __syncthreads();
    }
    tile_compute_lds<FMT, 8>(tg, g0 + c0, nn, src, scl, ag, lane);
    tile_compute_lds<FMT, 8>(tu, g0 + c0, nn, src, scl + d.ngh * kTileRows, au, lane);
  }
  digit_fold(ag);
  digit_fold(au);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    part[0][wave][lane][i] = ag[i];
    part[1][wave][lane][i] = au[i];
  }
  __syncthreads();
  if (wave == 0 && (lane & 15) == 1) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float g = part[0][0][lane][i] + part[0][1][lane][i] + part[0][2][lane][i] + part[0][3][lane][i];
      float u = part[1][0][lane][i] + part[1][1][lane][i] + part[1][2][lane][i] + part[1][3][lane][i];
      int row = rt * kTileRows + 4 * (lane >> 4) + i;
      d.h[(size_t)j * d.I + row] = silu_ref(g) * u;  // c/qwen.c:3419
    }
  }
}

// ---------------------------------------------------------------------------
// K3: routed down + shared down + combine.  grid H/16; waves 0..nwr-1 take
// routes j = wave, wave + nwr, ...; waves nwr and nwr+1 each take half of the
// shared expert's k range: they rebuild that half of the shared hidden vector
// from the integer sums and run its rows of the int8 down projection.
// LDS: per routed wave digits [2][Ip] | group parameters [ngi]; then the
// shared hidden vector h [Ish] f32 and its int8 quantisation [Ish].
// ---------------------------------------------------------------------------
constexpr int kShRegs = 8;  // shared hidden rows per lane loaded ahead

// A route's hidden vector -> digits in this wave's LDS, 1024 values per pass
// (the lane's 16 values of the first pass come loaded ahead in hv).
__device__ __forceinline__ void route_digits(const float *hj, int I, int Ip, const v4f hv[4], signed char *dig,
                                             float4 *gp, int lane) {
  quantize_slice8(hv, 0, Ip, dig, dig + Ip, gp, lane);
  for (int base = 1024; base < Ip; base += 1024) {
    v4f w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      int i = base + 16 * lane + 4 * q;
      w[q] = i < I ? *(const v4f *)(hj + i) : v4f{0, 0, 0, 0};
    }
    quantize_slice8(w, base, Ip, dig, dig + Ip, gp, lane);
  }
}

__device__ __forceinline__ void route_h_load(const float *hj, int I, v4f hv[4], int lane) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    int i = 16 * lane + 4 * q;
    hv[q] = *(const v4f *)(hj + (i < I ? i : 0));
    if (i >= I) hv[q] = v4f{0, 0, 0, 0};
  }
}

template <int FMT>
__global__ __launch_bounds__(64 * (kMaxDownWaves + 2)) void k_dec_down(
    Dec d, ExpertLayout xl, const signed char *__restrict__ dq,
    const float *__restrict__ ds, const float *__restrict__ gs, const float *__restrict__ us,
    float *__restrict__ y, int *route_idx, float *route_weight) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float vals[kMaxK][kTileRows];
  __shared__ int ish[2][kTileRows];
  __shared__ float red[2];
  __shared__ float cw[kMaxK + 1];     // route weights, shared gate
  __shared__ float cds[kTileRows];    // shared down row scales
  __shared__ __align__(16) signed char zero16[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6, nwr = nw - 2;
  const int rt = blockIdx.x;
  const size_t wbytes = 2 * (size_t)d.Ip + 16 * (size_t)d.ngi;
  float *hf = (float *)(smem + nwr * wbytes);    // [Ish]
  signed char *hq = (signed char *)(hf + d.Ish);  // [Ish]
  const bool routed = wave < nwr;
  for (int i = threadIdx.x; i < kMaxK * kTileRows; i += blockDim.x) (&vals[0][0])[i] = 0.0f;
  if (threadIdx.x < 4) ((int *)zero16)[threadIdx.x] = 0;
  const int p = d.imisc[0];
  const float sx = d.misc[0];
  const int nk = d.Ish / 64, sw = wave - nwr;
  const int kc0 = routed ? 0 : sw * nk / 2, kc1 = routed ? 0 : (sw + 1) * nk / 2;

  TilePrefetch<FMT, 8> t;
  RowPrefetch<8> pd;
  float hm = 0.0f;
  int e = -1;
  if (routed) {
    // ---- route `wave`: its hidden vector (cached) and expert id, then tiles
    signed char *dig = (signed char *)(smem + wave * wbytes);
    float4 *gp = (float4 *)(dig + 2 * (size_t)d.Ip);
    if (wave < d.K) {
      const float *hj = d.h + (size_t)wave * d.I;
      v4f hv[4];
      route_h_load(hj, d.I, hv, lane);
      e = d.idx[wave];
      if ((unsigned)e < (unsigned)d.E) {
        tile_prefetch<FMT, 8>(t, xl.mat(e, 2), rt, d.ngi, 0,
                              d.ngi < 8 ? d.ngi : 8, lane);
        route_digits(hj, d.I, d.Ip, hv, dig, gp, lane);
      }
    }
  } else {
    // ---- shared half: integer sums (cached) first, then the int8 rows ----
    if (sw == 1) {
      // the combine's operands, early
      if (lane < d.K) cw[lane] = d.w[lane];
      if (lane == 32) cw[kMaxK] = d.misc[1];
      if (lane >= 48) cds[lane - 48] = ds[rt * kTileRows + lane - 48];
    }
    const int *accp = d.acc + (size_t)p * 2 * d.Ish;
    const int r0 = kc0 * 64, r1 = kc1 * 64;
    int ag[kShRegs], au[kShRegs];
    float sg[kShRegs], su[kShRegs];
#pragma unroll
    for (int q = 0; q < kShRegs; q++) {
      int i = r0 + q * 64 + lane;
      i = i < r1 ? i : (r1 > 0 ? r1 - 1 : 0);  // clamped: no branch ahead of the rows
      ag[q] = accp[i];
      au[q] = accp[d.Ish + i];
      sg[q] = gs[i];
      su[q] = us[i];
    }
    const int ke0 = kc0 + 8 < kc1 ? kc0 + 8 : kc1;
    rows_prefetch<8>(pd, dq, d.Ish, rt * kTileRows, kc0, ke0, lane);
    // h = silu(g) * u from the exact integer dots (IDOT epilogue
    // ((float)dot * s_row) * sx, c/qwen.c:1766)
#pragma unroll
    for (int q = 0; q < kShRegs; q++) {
      int i = r0 + q * 64 + lane;
      if (i < r1) {
        float h = silu_ref((float)ag[q] * sg[q] * sx) * ((float)au[q] * su[q] * sx);
        hf[i] = h;
        hm = fmaxf(hm, fabsf(h));
      }
    }
    for (int i = r0 + kShRegs * 64 + lane; i < r1; i += 64) {
      float h = silu_ref((float)accp[i] * gs[i] * sx) * ((float)accp[d.Ish + i] * us[i] * sx);
      hf[i] = h;
      hm = fmaxf(hm, fabsf(h));
    }
    hm = wave_max_dpp(hm);
    if (lane == 0) red[sw] = hm;
  }
  __syncthreads();
  // qrow_i8 scale of the whole shared hidden vector
  float shx = fmaxf(red[0], red[1]) / 127.0f;
  if (shx < 1e-12f) shx = 1e-12f;

  if (routed) {
    signed char *dig = (signed char *)(smem + wave * wbytes);
    float4 *gp = (float4 *)(dig + 2 * (size_t)d.Ip);
    const DigitSrc src = lane_digits(lane, 1, dig, d.Ip, gp, d.ngi, zero16);
    for (int j = wave; j < d.K; j += nwr) {
      if (j != wave) e = d.idx[j];
      if ((unsigned)e >= (unsigned)d.E) continue;
      const TileMat md = xl.mat(e, 2);
      float acc[4] = {0, 0, 0, 0};
      for (int c0 = 0; c0 < d.ngi; c0 += 8) {
        const int nn = d.ngi - c0 < 8 ? d.ngi - c0 : 8;
        if (j != wave || c0 != 0) {
          tile_prefetch<FMT, 8>(t, md, rt, d.ngi, c0, nn, lane);
          if (c0 == 0) {
            // a later route: its digits -> this wave's LDS (wave-local)
            const float *hj = d.h + (size_t)j * d.I;
            v4f hv[4];
            route_h_load(hj, d.I, hv, lane);
            route_digits(hj, d.I, d.Ip, hv, dig, gp, lane);
          }
        }
        __builtin_amdgcn_wave_barrier();
        tile_compute<FMT, 8>(t, c0, nn, src, acc, lane);
      }
      digit_fold(acc);
      if ((lane & 15) == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) vals[j][4 * (lane >> 4) + i] = acc[i];
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else {
    // this half's int8 hidden values (wave-local rows), then the dots
    const float hinv = 1.0f / shx;
    for (int i = kc0 * 64 + lane; i < kc1 * 64; i += 64) hq[i] = (signed char)__builtin_rintf(hf[i] * hinv);
    __builtin_amdgcn_wave_barrier();
    v4i c = {0, 0, 0, 0};
    const bool bvalid = (lane & 15) == 0;
    const int ke0 = kc0 + 8 < kc1 ? kc0 + 8 : kc1;
    rows_compute<8>(pd, kc0, ke0, hq, 0, bvalid, c, lane);
    for (int kc = ke0; kc < kc1; kc += 8) {
      int e1 = kc + 8 < kc1 ? kc + 8 : kc1;
      idot_tile<8>(dq, d.Ish, rt * kTileRows, kc, e1, hq, 0, bvalid, c, lane);
    }
    if ((lane & 15) == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) ish[sw][4 * (lane >> 4) + i] = c[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < kTileRows) {
    // moe_forward's combine: fma over k in route order, then shared * gate
    float out = 0.0f;
    for (int k = 0; k < d.K; k++) out = __builtin_fmaf(vals[k][threadIdx.x], cw[k], out);
    const float shv = (float)(ish[0][threadIdx.x] + ish[1][threadIdx.x]) * cds[threadIdx.x] * shx;
    out = __builtin_fmaf(shv, cw[kMaxK], out);
    y[rt * kTileRows + threadIdx.x] = out;
  }
  // clear the other parity's integer sums for the next call; flip the parity
  int *accz = d.acc + (size_t)(1 - p) * 2 * d.Ish;
  const int n_acc = 2 * d.Ish, chunk = (n_acc + gridDim.x - 1) / gridDim.x;
  const int z0 = blockIdx.x * chunk, z1 = z0 + chunk < n_acc ? z0 + chunk : n_acc;
  for (int i = z0 + threadIdx.x; i < z1; i += blockDim.x) accz[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) d.cnt[1] = (unsigned)(1 - p);
  if (blockIdx.x == 0 && (int)threadIdx.x < d.K) {
    if (route_idx) route_idx[threadIdx.x] = d.idx[threadIdx.x];
    if (route_weight) route_weight[threadIdx.x] = cw[threadIdx.x];
  }
}

struct DecLaunch {
  Dec d;
  int g1, g2, g3, t3;
  size_t lds1, lds2, lds3;
};

// Shapes the decode kernels take; others run the many-token path.
bool decode_plan(const ColiMoeLayer *L, DecLaunch &p) {
  Dec &d = p.d;
  memset(&d, 0, sizeof(d));
  d.H = L->sh.hidden;
  d.E = L->sh.experts;
  d.K = L->sh.topk;
  d.I = L->sh.intermediate;
  d.Ish = L->sh.shared_intermediate;
  d.ngh = L->ngh;
  d.ngi = L->ngi;
  d.Hp = d.ngh * kGroup;
  d.Ip = d.ngi * kGroup;
  d.KQ = d.H >= 512 ? d.H / 512 : 1;
  if (d.H > 16384 || d.K > kMaxK) return false;
  d.n_router_wg = (d.E + 1 + 3) / 4;
  d.n_shared_wg = ((d.Ish / kTileRows) * d.KQ + 3) / 4;
  p.g1 = d.n_router_wg + d.n_shared_wg + (d.ngh + 3) / 4;
  size_t xs_bytes = ((size_t)d.H * 4 + 15) & ~(size_t)15;
  size_t sel = (size_t)(d.E + 1) * 16 + (size_t)d.E * 8;
  p.lds1 = xs_bytes + (sel > (size_t)d.H ? sel : (size_t)d.H);
  p.g2 = d.K * (d.I / kTileRows);
  p.lds2 = 2 * (size_t)d.Hp + (size_t)d.ngh * 16 + 2 * (size_t)d.ngh * kTileRows * 4;
  size_t wbytes = 2 * (size_t)d.Ip + 16 * (size_t)d.ngi;
  int nwr = d.K < kMaxDownWaves ? d.K : kMaxDownWaves;
  p.g3 = d.H / kTileRows;
  p.t3 = 64 * (nwr + 2);
  p.lds3 = nwr * wbytes + 5 * (size_t)d.Ish;
  const size_t lim = 64 * 1024;
  return p.lds1 <= lim && p.lds2 <= lim && p.lds3 <= lim;
}

}  // namespace

namespace sw {

// layout of ColiMoeLayer::sync: cnt[16] | acc[2][2*Ish]
size_t decode_sync_words(const ColiMoeShape &s) { return 16 + 4 * (size_t)s.shared_intermediate; }

int decode_step(ColiCuda *ctx, ColiMoeLayer *L, float *y, const float *x, int *route_idx, float *route_weight) {
  DecLaunch p;
  if (!decode_plan(L, p)) return 1;
  Dec &d = p.d;
  size_t bytes = dec_carve(d, nullptr);
  if (ensure_scratch(ctx, kScrShared, bytes, "decode workspace allocation")) return -1;
  dec_carve(d, (char *)ctx->scratch[kScrShared]);
  d.cnt = L->sync;
  d.acc = (int *)(L->sync + 16);
  hipStream_t st = ctx->stream;
  const bool timing = ctx->moe_timing != 0;
  if (timing) (void)hipEventRecord(ctx->moe_event[0], st);
  k_dec_route<<<p.g1, kThreads, p.lds1, st>>>(d, x, L->router, L->sgate_row, L->sh_gq, L->sh_uq, L->router_mode,
                                              L->stats);
  if (timing) (void)hipEventRecord(ctx->moe_event[1], st);
  prof_mark(ctx, kStageSetup);  // router, top-k and the shared gate/up
  if (L->sh.expert_format == 4)
    k_dec_experts<4><<<p.g2, kThreads, p.lds2, st>>>(d, L->xl);
  else
    k_dec_experts<3><<<p.g2, kThreads, p.lds2, st>>>(d, L->xl);
  if (timing) (void)hipEventRecord(ctx->moe_event[2], st);
  prof_mark(ctx, kStageRoutedHidden);
  if (L->sh.expert_format == 4)
    k_dec_down<4><<<p.g3, p.t3, p.lds3, st>>>(d, L->xl, L->sh_dq, L->sh_ds, L->sh_gs, L->sh_us, y, route_idx,
                                              route_weight);
  else
    k_dec_down<3><<<p.g3, p.t3, p.lds3, st>>>(d, L->xl, L->sh_dq, L->sh_ds, L->sh_gs, L->sh_us, y, route_idx,
                                              route_weight);
  if (timing) (void)hipEventRecord(ctx->moe_event[3], st);
  prof_mark(ctx, kStageRoutedDown);  // routed and shared down, combine
  int rc = launch_status("MoE decode step");
  if (timing && rc == 0) {
    (void)hipEventSynchronize(ctx->moe_event[3]);
    for (int i = 0; i < 3; i++) {
      float ms = 0.0f;
      if (hipEventElapsedTime(&ms, ctx->moe_event[i], ctx->moe_event[i + 1]) == hipSuccess) ctx->moe_dec_ms[i] += ms;
    }
    ctx->moe_dec_calls++;
  }
  return rc;
}

}  // namespace sw
