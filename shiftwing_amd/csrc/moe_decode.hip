// One decoded token through one HBM-resident MoE layer in three kernels
// (moe_forward, c/qwen.c:3717-3739):
//
//   K1 route   wave tasks over all CUs: the router rows (fp64 logit + a
//              rigorous bound on the reference's serial fp32 dot), the shared
//              expert's gate/up int8 dots (exact int32, split over k and
//              summed with integer atomics), and the activation digits for the
//              routed experts.  The last workgroup to finish certifies the
//              top-k (or runs the exact serial chain), and quantises the
//              shared hidden vector (qrow_i8).
//   K2 experts routed gate/up tiles for the K chosen experts (the last
//              workgroup of each expert quantises its hidden vector) and the
//              shared down projection.
//   K3 down    one workgroup per 16 output rows: the K routed down tiles, then
//              the reference's combine order (fma over k, then shared * gate).
//
// The hand-offs inside a kernel use a fan-in counter (the last arriver does
// the dependent tail; nobody spins), so the only device-wide waits are the
// two kernel boundaries.  Counters and integer accumulators are returned to
// zero by their last user, so consecutive calls (and graph replays) need no
// memset.
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
constexpr int kDecThreads = 256;  // K1 / K2 workgroup

struct Dec {
  int H, E, K, I, Ish, ngh, ngi, Hp, Ip, KQ;
  signed char *xd;    // [2][Hp] routed activation digits
  float4 *xgp;        // [ngh]
  double2 *lb;        // [E+1] fp64 logit, bound (row E: shared gate)
  int *acc;           // [2][Ish] shared gate/up int32 partial dots
  unsigned *rtcnt;    // [Ish/16]
  unsigned *cnt;      // [8] fan-in counters
  float *hsh;         // [Ish]
  signed char *hq;    // [Ish]
  float *misc;        // [0] shx  [1] sgate  [2] sx
  int *idx;           // [K]
  float *w;           // [K]
  float *logits;      // [E] exact fallback logits
  float *hroute;      // [K][I]
  signed char *hd;    // [K][2][Ip]
  float4 *hgp;        // [K][ngi]
  unsigned *ecnt;     // [K]
  float *shout;       // [H]
  size_t bytes;
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
  d.hsh = (float *)take((size_t)d.Ish * 4);
  d.hq = (signed char *)take((size_t)d.Ish);
  d.misc = (float *)take(64);
  d.idx = (int *)take((size_t)kMaxK * 4);
  d.w = (float *)take((size_t)kMaxK * 4);
  d.logits = (float *)take((size_t)d.E * 4);
  d.hroute = (float *)take((size_t)d.K * d.I * 4);
  d.hd = (signed char *)take((size_t)d.K * 2 * d.Ip);
  d.hgp = (float4 *)take((size_t)d.K * d.ngi * 16);
  d.shout = (float *)take((size_t)d.H * 4);
  d.bytes = off + 256;
  return d.bytes;
}

// ---------------------------------------------------------------------------
// fan-in: every thread releases its writes; returns true in all threads of the
// last workgroup to arrive (which then acquires).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool block_last_arrival(unsigned *counter, unsigned total, unsigned *s_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) *s_flag = (atomicAdd(counter, 1u) == total - 1) ? 1u : 0u;
  __syncthreads();
  bool last = *s_flag != 0;
  if (last) __threadfence();
  return last;
}

// same for a single wave
__device__ __forceinline__ bool wave_last_arrival(unsigned *counter, unsigned total, int lane) {
  __threadfence();
  unsigned prev = 0;
  if (lane == 0) prev = atomicAdd(counter, 1u);
  prev = (unsigned)__builtin_amdgcn_readfirstlane((int)prev);
  bool last = prev == total - 1;
  if (last) __threadfence();
  return last;
}

// inclusive DPP prefix sum of a double over the wave (lane order)
#define SW_DPP_D_ADD(v, ctrl, rm, bc)                                   \
  {                                                                     \
    int lo_ = SW_DPP_I(0, (int)__double2loint(v), ctrl, rm, bc);       \
    int hi_ = SW_DPP_I(0, (int)__double2hiint(v), ctrl, rm, bc);       \
    v += __hiloint2double(hi_, lo_);                                    \
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
// Router row bound.  The reference logit is dot() (c/qwen.c:1674), evaluated
// with gcc -O3 as s_k = rn(s_{k-1} + rn(x_k w_k)) (a tail of H%8 terms fused).
// With exact prefix sums S_k and u = 2^-24:
//   |s_H - L| <= u * (sum_k |x_k w_k| + sum_k |s_k|),  |s_k| <= |S_k| + err,
// so B = u (A + P) (1 + 2^-10) bounds the error for H <= 16384.  A wave
// walks the row in 256-element segments (float4 per lane, coalesced); S_k
// comes from an fp64 lane scan plus the running carry, exact to 1e-16.
// ---------------------------------------------------------------------------
__device__ double2 row_bound(const float *row, const float *xs, int H, int lane) {
  double carry = 0.0, A = 0.0, P = 0.0;
  for (int base = 0; base < H; base += 256) {
    int i0 = base + 4 * lane;
    double p[4] = {0.0, 0.0, 0.0, 0.0};
    if (i0 < H) {
      v4f wv = __builtin_nontemporal_load((const v4f *)(row + i0));
      float4 xv = *(const float4 *)(xs + i0);
      p[0] = (double)xv.x * (double)wv.x;
      p[1] = (double)xv.y * (double)wv.y;
      p[2] = (double)xv.z * (double)wv.z;
      p[3] = (double)xv.w * (double)wv.w;
    }
    double q0 = p[0], q1 = q0 + p[1], q2 = q1 + p[2], q3 = q2 + p[3];
    A += fabs(p[0]) + fabs(p[1]) + fabs(p[2]) + fabs(p[3]);
    double inc = wave_inclusive_scan_dpp(q3);
    double pre = carry + (inc - q3);
    if (i0 < H) P += fabs(pre + q0) + fabs(pre + q1) + fabs(pre + q2) + fabs(pre + q3);
    carry += readlane63_d(inc);
  }
  A = wave_sum_dpp(A);
  P = wave_sum_dpp(P);
  const double u = 0x1p-24;
  double B = u * (A + P) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-36;
  return make_double2(carry, B);
}

// ---------------------------------------------------------------------------
// K1
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kDecThreads) void k_dec_route(Dec d, const float *__restrict__ x,
                                                           const float *__restrict__ router,
                                                           const float *__restrict__ sgrow,
                                                           const signed char *__restrict__ gq,
                                                           const float *__restrict__ gs,
                                                           const signed char *__restrict__ uq,
                                                           const float *__restrict__ us, int mode,
                                                           unsigned long long *stats) {
  extern __shared__ __align__(16) unsigned char smem[];
  float *xs = (float *)smem;                           // [H]
  signed char *xq = (signed char *)(xs + d.H);         // [H]
  __shared__ float red[8];
  __shared__ unsigned s_flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // stage x and its IDOT quantisation (qrow_i8, c/qwen.c:1696)
  float m = 0.0f;
  for (int i = threadIdx.x; i < d.H; i += blockDim.x) {
    float v = x[i];
    xs[i] = v;
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max_dpp(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sx = amax / 127.0f;
  if (sx < 1e-12f) sx = 1e-12f;
  const float inv = 1.0f / sx;
  for (int i = threadIdx.x; i < d.H; i += blockDim.x) xq[i] = (signed char)__builtin_rintf(xs[i] * inv);
  __syncthreads();

  // one task per wave: router rows, shared gate/up slices, digit groups
  const int task = blockIdx.x * 4 + wave;
  const int n_router = d.E + 1;
  const int n_shared = (d.Ish / kTileRows) * d.KQ;
  if (task < n_router) {
    const float *row = task < d.E ? router + (size_t)task * d.H : sgrow;
    double2 b = row_bound(row, xs, d.H, lane);
    if (lane == 0) d.lb[task] = b;
  } else if (task < n_router + n_shared) {
    int t = task - n_router, rt = t / d.KQ, kq = t % d.KQ;
    int nk = d.H / 64, per = nk / d.KQ, kc0 = kq * per, kc1 = kc0 + per;
    v4i cg = {0, 0, 0, 0}, cu = {0, 0, 0, 0};
    bool bvalid = (lane & 15) == 0;
    for (int kc = kc0; kc < kc1; kc += 8) {
      int e1 = kc + 8 < kc1 ? kc + 8 : kc1;
      idot_tile<8>(gq, d.H, rt * kTileRows, kc, e1, xq, 0, bvalid, cg, lane);
      idot_tile<8>(uq, d.H, rt * kTileRows, kc, e1, xq, 0, bvalid, cu, lane);
    }
    if ((lane & 15) == 0) {
      int r0 = rt * kTileRows + 4 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        atomicAdd(&d.acc[r0 + i], cg[i]);
        atomicAdd(&d.acc[d.Ish + r0 + i], cu[i]);
      }
    }
    if (wave_last_arrival(&d.rtcnt[rt], (unsigned)d.KQ, lane)) {
      // h = silu(g) * u for the tile's 16 rows (c/qwen.c:3419, 1767)
      if (lane < kTileRows) {
        int row = rt * kTileRows + lane;
        int dg = __hip_atomic_load(&d.acc[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int du = __hip_atomic_load(&d.acc[d.Ish + row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float g = (float)dg * gs[row] * sx;
        float u = (float)du * us[row] * sx;
        d.hsh[row] = silu_ref(g) * u;
        atomicExch(&d.acc[row], 0);
        atomicExch(&d.acc[d.Ish + row], 0);
      }
      if (lane == 0) atomicExch(&d.rtcnt[rt], 0u);
    }
  } else if (task < n_router + n_shared + d.ngh) {
    int g = task - n_router - n_shared;
    quantize_group(xs, d.H, g, d.xd, d.xd + d.Hp, d.xgp, lane);
  }

  if (!block_last_arrival(&d.cnt[0], gridDim.x, &s_flag)) return;

  // ---- last workgroup: routes, shared hidden quantisation ----
  __shared__ int s_ok;
  if (wave == 0) {
    const int E = d.E, K = d.K;
    // top K+1 by fp64 logit (float keys; ties / near-ties fail certification)
    unsigned long long key[64];
    int per = (E + 63) / 64;
    for (int i = 0; i < per && i < 64; i++) {
      int e = lane + 64 * i;
      key[i] = e < E ? (((unsigned long long)float_key((float)d.lb[e].x) << 32) | (unsigned)(~e)) : 0ull;
    }
    int cand[kMaxK + 1];
    int nc = K + 1 < E ? K + 1 : E;
    for (int r = 0; r < nc; r++) {
      unsigned long long best = 0;
      for (int i = 0; i < per && i < 64; i++) best = key[i] > best ? key[i] : best;
      best = wave_max_u64(best);
      int e = (int)(~(unsigned)best);
      for (int i = 0; i < per && i < 64; i++)
        if (key[i] == best) key[i] = 0;
      cand[r] = e;
    }
    // the largest upper bound outside the top K
    unsigned long long upk = 0;
    for (int i = 0; i < per && i < 64; i++) {
      int e = lane + 64 * i;
      if (e >= E) continue;
      bool top = false;
      for (int r = 0; r < K; r++) top |= cand[r] == e;
      if (!top) {
        unsigned long long k2 = double_key(d.lb[e].x + d.lb[e].y);
        upk = k2 > upk ? k2 : upk;
      }
    }
    upk = wave_max_u64(upk);
    {
      double mx = d.lb[cand[0]].x;
      bool ok = mode == 0;
      for (int r = 0; ok && r + 1 < K; r++) {
        double2 a = d.lb[cand[r]], b = d.lb[cand[r + 1]];
        double margin = 0x1p-20 * (1.0 + fabs(a.x) + fabs(b.x) + 2.0 * fabs(mx));
        ok = (a.x - a.y) - (b.x + b.y) > margin;
      }
      if (ok && K < E) {
        double2 a = d.lb[cand[K - 1]];
        double up = key_double(upk);
        double margin = 0x1p-20 * (1.0 + fabs(a.x) + fabs(up) + 2.0 * fabs(mx));
        ok = (a.x - a.y) - up > margin;
      }
      if (ok) ok = (d.lb[cand[K - 1]].x - d.lb[cand[K - 1]].y) - (mx + d.lb[cand[0]].y) > -80.0;
      if (ok) {
        double p[kMaxK], den = 0.0;
        for (int r = 0; r < K; r++) {
          p[r] = exp(d.lb[cand[r]].x - mx);
          den += p[r];
        }
        if (lane == 0)
          for (int r = 0; r < K; r++) {
            d.idx[r] = cand[r];
            d.w[r] = (float)(p[r] / den);
          }
      }
      if (lane == 0) {
        s_ok = ok;
        d.misc[1] = sigmoid_ref((float)d.lb[E].x);
        atomicAdd(&stats[0], 1ull);
        if (!ok) atomicAdd(&stats[1], 1ull);
      }
    }
  }
  __syncthreads();
  if (!s_ok) {
    // exact serial fp32 router dot for every expert (two chains per lane),
    // kept in LDS for the exact top-k below
    float *lgs = (float *)(smem + ((size_t)d.H * 5 + 15) / 16 * 16);  // [E]
    __shared__ float s_mx, s_den;
    const int m8 = (d.H / 8) * 8;
    for (int e0 = threadIdx.x; e0 < d.E; e0 += 2 * blockDim.x) {
      int e1 = e0 + blockDim.x;
      const float *r0 = router + (size_t)e0 * d.H;
      const float *r1 = router + (size_t)(e1 < d.E ? e1 : e0) * d.H;
      float s0 = 0.0f, s1 = 0.0f;
      int i = 0;
      for (; i + 4 <= m8; i += 4) {
        float4 a = *(const float4 *)(r0 + i), b = *(const float4 *)(r1 + i);
        float4 xv = *(const float4 *)(xs + i);
        s0 = s0 + xv.x * a.x;
        s1 = s1 + xv.x * b.x;
        s0 = s0 + xv.y * a.y;
        s1 = s1 + xv.y * b.y;
        s0 = s0 + xv.z * a.z;
        s1 = s1 + xv.z * b.z;
        s0 = s0 + xv.w * a.w;
        s1 = s1 + xv.w * b.w;
      }
      for (; i < m8; i++) {
        s0 = s0 + xs[i] * r0[i];
        s1 = s1 + xs[i] * r1[i];
      }
      for (; i < d.H; i++) {
        s0 = __builtin_fmaf(xs[i], r0[i], s0);
        s1 = __builtin_fmaf(xs[i], r1[i], s1);
      }
      lgs[e0] = s0;
      if (e1 < d.E) lgs[e1] = s1;
    }
    __syncthreads();
    // router_topk (c/qwen.c:3421-3426) on the exact logits, bit-exact:
    // max, expf(l - max), serial denominator in expert order, division,
    // K argmax rounds (lowest index on ties), serial renormalisation
    if (wave == 0) {
      float mx = -__builtin_huge_valf();
      for (int e = lane; e < d.E; e += 64) mx = fmaxf(mx, lgs[e]);
      mx = wave_max_dpp(mx);
      if (lane == 0) s_mx = mx;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < d.E; e += blockDim.x) lgs[e] = expf_glibc(lgs[e] - s_mx);
    __syncthreads();
    if (threadIdx.x == 0) {
      float den = 0.0f;
      for (int e = 0; e < d.E; e++) den += lgs[e];
      s_den = den;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < d.E; e += blockDim.x) lgs[e] = lgs[e] / s_den;
    __syncthreads();
    if (wave == 0) {
      int chosen[kMaxK];
      float wsel[kMaxK];
      for (int j = 0; j < d.K; j++) {
        unsigned long long best = 0;
        for (int e = lane; e < d.E; e += 64) {
          bool used = false;
          for (int q = 0; q < j; q++) used |= chosen[q] == e;
          float pv = lgs[e];
          unsigned long long k2 = (((unsigned long long)float_key(pv)) << 32) | (unsigned)(~e);
          if (!used && pv > -1.0f && k2 > best) best = k2;
        }
        best = wave_max_u64(best);
        chosen[j] = best ? (int)(~(unsigned)best) : -1;
        wsel[j] = best ? lgs[chosen[j]] : -1.0f;
      }
      if (lane == 0) {
        float topden = 0.0f;
        for (int j = 0; j < d.K; j++) topden += wsel[j];
        for (int j = 0; j < d.K; j++) {
          d.idx[j] = chosen[j];
          d.w[j] = wsel[j] / topden;
        }
      }
    }
  }
  // shared hidden -> int8 (qrow_i8) for the IDOT down projection
  __syncthreads();
  {
    float hm = 0.0f;
    for (int i = threadIdx.x; i < d.Ish; i += blockDim.x) hm = fmaxf(hm, fabsf(d.hsh[i]));
    hm = wave_max_dpp(hm);
    __syncthreads();
    if (lane == 0) red[wave] = hm;
    __syncthreads();
    float ha = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float shx = ha / 127.0f;
    if (shx < 1e-12f) shx = 1e-12f;
    float hinv = 1.0f / shx;
    for (int i = threadIdx.x; i < d.Ish; i += blockDim.x)
      d.hq[i] = (signed char)__builtin_rintf(d.hsh[i] * hinv);
    if (threadIdx.x == 0) {
      d.misc[0] = shx;
      atomicExch(&d.cnt[0], 0u);
    }
  }
}

// ---------------------------------------------------------------------------
// K2: routed gate/up tiles + shared down.  grid K*I/16 + H/16, 256 threads
// ---------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(kDecThreads) void k_dec_experts(Dec d, const unsigned char *__restrict__ codes,
                                                             const float *__restrict__ scales, size_t expert_codes,
                                                             size_t expert_scales, size_t gate_codes,
                                                             size_t gate_scales,
                                                             const signed char *__restrict__ dq,
                                                             const float *__restrict__ ds) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float part[4][2][64][4];
  __shared__ int ipart[4][64][4];
  __shared__ __align__(16) signed char zero16[16];
  __shared__ unsigned s_flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_route_tiles = d.I / kTileRows;
  const int routed = d.K * n_route_tiles;
  if ((int)blockIdx.x >= routed) {
    // shared down: 16 rows of the int8 [H x Ish] matrix, exact int32 dots
    int rt = blockIdx.x - routed;
    int nk = d.Ish / 64, per = (nk + 3) / 4, kc0 = wave * per, kc1 = min(nk, kc0 + per);
    v4i c = {0, 0, 0, 0};
    bool bvalid = (lane & 15) == 0;
    for (int kc = kc0; kc < kc1; kc += 8) {
      int e1 = kc + 8 < kc1 ? kc + 8 : kc1;
      idot_tile<8>(dq, d.Ish, rt * kTileRows, kc, e1, d.hq, 0, bvalid, c, lane);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) ipart[wave][lane][i] = c[i];
    __syncthreads();
    if (wave == 0 && (lane & 15) == 0) {
      float shx = d.misc[0];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int dot = ipart[0][lane][i] + ipart[1][lane][i] + ipart[2][lane][i] + ipart[3][lane][i];
        int row = rt * kTileRows + 4 * (lane >> 4) + i;
        d.shout[row] = (float)dot * ds[row] * shx;
      }
    }
    return;
  }
  const int j = blockIdx.x / n_route_tiles, rt = blockIdx.x % n_route_tiles;
  const int e = d.idx[j];
  if ((unsigned)e >= (unsigned)d.E) return;  // no expert (router_topk's -1): contributes nothing
  // activation digits -> LDS
  signed char *dig = (signed char *)smem;                 // [2][Hp]
  float4 *gp = (float4 *)(smem + 2 * (size_t)d.Hp);       // [ngh]
  for (int i = threadIdx.x; i < (2 * d.Hp) / 16; i += blockDim.x)
    ((int4 *)dig)[i] = ((const int4 *)d.xd)[i];
  for (int i = threadIdx.x; i < d.ngh; i += blockDim.x) gp[i] = d.xgp[i];
  if (threadIdx.x < 4) ((int *)zero16)[threadIdx.x] = 0;
  __syncthreads();
  DigitSrc src = lane_digits(lane, 1, dig, d.Hp, gp, d.ngh, zero16);
  const unsigned char *ce = codes + (size_t)e * expert_codes;
  const float *se = scales + (size_t)e * expert_scales;
  int per = (d.ngh + 3) / 4, g0 = wave * per, n = min(d.ngh, g0 + per) - g0;
  float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0};
  for (int c0 = 0; c0 < n; c0 += 8) {
    int nn = n - c0 < 8 ? n - c0 : 8;
    tile_gemv<FMT, 8>(ce, se, rt, d.ngh, g0 + c0, nn, src, ag, lane);
    tile_gemv<FMT, 8>(ce + gate_codes, se + gate_scales, rt, d.ngh, g0 + c0, nn, src, au, lane);
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    part[wave][0][lane][i] = ag[i];
    part[wave][1][lane][i] = au[i];
  }
  __syncthreads();
  if (wave == 0 && (lane & 15) == 1) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float g = part[0][0][lane][i] + part[1][0][lane][i] + part[2][0][lane][i] + part[3][0][lane][i];
      float u = part[0][1][lane][i] + part[1][1][lane][i] + part[2][1][lane][i] + part[3][1][lane][i];
      int row = rt * kTileRows + 4 * (lane >> 4) + i;
      d.hroute[(size_t)j * d.I + row] = silu_ref(g) * u;
    }
  }
  if (!block_last_arrival(&d.ecnt[j], (unsigned)n_route_tiles, &s_flag)) return;
  // last tile of expert j: its hidden vector -> digits for the down projection
  signed char *hd = d.hd + (size_t)j * 2 * d.Ip;
  for (int g = wave; g < d.ngi; g += 4)
    quantize_group(d.hroute + (size_t)j * d.I, d.I, g, hd, hd + d.Ip, d.hgp + (size_t)j * d.ngi, lane);
  if (threadIdx.x == 0) atomicExch(&d.ecnt[j], 0u);
}

// ---------------------------------------------------------------------------
// K3: down + combine.  grid H/16, one wave per route (64*K threads)
// ---------------------------------------------------------------------------
template <int FMT>
__global__ void k_dec_down(Dec d, const unsigned char *__restrict__ codes, const float *__restrict__ scales,
                           size_t expert_codes, size_t expert_scales, size_t down_codes_off, size_t down_scales_off,
                           float *__restrict__ y, int *route_idx, float *route_weight) {
  __shared__ float vals[kMaxK][kTileRows];
  for (int i = threadIdx.x; i < kMaxK * kTileRows; i += blockDim.x) (&vals[0][0])[i] = 0.0f;
  __shared__ __align__(16) signed char zero16[16];
  const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;
  const int rt = blockIdx.x;
  if (threadIdx.x < 4) ((int *)zero16)[threadIdx.x] = 0;
  __syncthreads();
  if (j < d.K && (unsigned)d.idx[j] < (unsigned)d.E) {
    const int e = d.idx[j];
    const signed char *hd = d.hd + (size_t)j * 2 * d.Ip;
    DigitSrc src = lane_digits(lane, 1, hd, d.Ip, d.hgp + (size_t)j * d.ngi, d.ngi, zero16);
    float acc[4] = {0, 0, 0, 0};
    const unsigned char *ce = codes + (size_t)e * expert_codes + down_codes_off;
    const float *se = scales + (size_t)e * expert_scales + down_scales_off;
    for (int c0 = 0; c0 < d.ngi; c0 += 8) {
      int nn = d.ngi - c0 < 8 ? d.ngi - c0 : 8;
      tile_gemv<FMT, 8>(ce, se, rt, d.ngi, c0, nn, src, acc, lane);
    }
    if ((lane & 15) == 1) {
#pragma unroll
      for (int i = 0; i < 4; i++) vals[j][4 * (lane >> 4) + i] = acc[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < kTileRows) {
    int row = rt * kTileRows + threadIdx.x;
    float out = 0.0f;
    for (int k = 0; k < d.K; k++) out = __builtin_fmaf(vals[k][threadIdx.x], d.w[k], out);
    out = __builtin_fmaf(d.shout[row], d.misc[1], out);
    y[row] = out;
  }
  if (blockIdx.x == 0 && threadIdx.x < d.K) {
    if (route_idx) route_idx[threadIdx.x] = d.idx[threadIdx.x];
    if (route_weight) route_weight[threadIdx.x] = d.w[threadIdx.x];
  }
}

}  // namespace

namespace sw {

// layout of ColiMoeLayer::sync: cnt[16] | ecnt[32] | rtcnt[Ish/16] | acc[2*Ish]
size_t decode_sync_words(const ColiMoeShape &s) {
  return 16 + kMaxK + (size_t)(s.shared_intermediate / kTileRows) + 2 * (size_t)s.shared_intermediate;
}

int decode_step(ColiCuda *ctx, ColiMoeLayer *L, float *y, const float *x, int *route_idx, float *route_weight) {
  Dec d;
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
  size_t bytes = dec_carve(d, nullptr);
  if (ensure_scratch(ctx, kScrShared, bytes, "decode workspace allocation")) return -1;
  dec_carve(d, (char *)ctx->scratch[kScrShared]);
  d.cnt = L->sync;
  d.ecnt = L->sync + 16;
  d.rtcnt = L->sync + 16 + kMaxK;
  d.acc = (int *)(L->sync + 16 + kMaxK + d.Ish / kTileRows);
  hipStream_t st = ctx->stream;
  int n_tasks = (d.E + 1) + (d.Ish / kTileRows) * d.KQ + d.ngh;
  int g1 = (n_tasks + 3) / 4;
  size_t lds1 = ((size_t)d.H * 5 + 15) / 16 * 16 + (size_t)d.E * 4;
  k_dec_route<<<g1, kDecThreads, lds1, st>>>(d, x, L->router, L->sgate_row, L->sh_gq, L->sh_gs, L->sh_uq, L->sh_us,
                                           L->router_mode, L->stats);
  int g2 = d.K * (d.I / kTileRows) + d.H / kTileRows;
  size_t lds2 = 2 * (size_t)d.Hp + (size_t)d.ngh * 16;
  if (L->sh.expert_format == 4)
    k_dec_experts<4><<<g2, kDecThreads, lds2, st>>>(d, L->codes, L->scales, L->expert_codes, L->expert_scales,
                                                     L->gate_codes, L->gate_scales, L->sh_dq, L->sh_ds);
  else
    k_dec_experts<3><<<g2, kDecThreads, lds2, st>>>(d, L->codes, L->scales, L->expert_codes, L->expert_scales,
                                                     L->gate_codes, L->gate_scales, L->sh_dq, L->sh_ds);
  int t3 = 64 * d.K;
  if (L->sh.expert_format == 4)
    k_dec_down<4><<<d.H / kTileRows, t3, 0, st>>>(d, L->codes, L->scales, L->expert_codes, L->expert_scales,
                                                   2 * L->gate_codes, 2 * L->gate_scales, y, route_idx, route_weight);
  else
    k_dec_down<3><<<d.H / kTileRows, t3, 0, st>>>(d, L->codes, L->scales, L->expert_codes, L->expert_scales,
                                                   2 * L->gate_codes, 2 * L->gate_scales, y, route_idx, route_weight);
  return launch_status("MoE decode step");
}

}  // namespace sw
