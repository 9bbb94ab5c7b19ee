// HBM-resident MoE layer step for gfx950 (the coli_cuda_moe_* entry points).
//
// What it computes is the reference's CPU MoE step (c/qwen.c): moe_forward
// 3717-3739 for one token and moe_prefill_grouped 4141-4206 for many, with
// router_topk 3421-3426, the int8 IDOT shared expert 1696-1705/1765-1768 and
// grouped int4 / int3 routed experts 1706-1754.
//
// Device layout (set at registration, see tile_* below).  Routed expert
// matrices are repacked into MFMA tiles: a tile is 16 rows x one 128-wide
// quant group; lane l of a wave owns row (l%16) and the 32 codes at group
// positions kb*16+[0,16) and 64+kb*16+[0,16), kb = l/16.  Those 32 codes are
// stored as 16 bytes (int4: byte m of word i holds codes 8i+m (low nibble)
// and 8i+4+m (high nibble)) or 12 bytes (int3: two 2-bit planes L0, L1 and a
// high-bit plane H).  One coalesced 1 KB / 768 B wave load fetches a tile.
// Per-(row, group) f32 scales are stored in the same tile order.
//
// Arithmetic.  Routed experts run on v_mfma_i32_16x16x64_i8: the activation
// is split per 128-group into two int8 digits, x ~= A*q1 + B*q2 (A =
// amax/127, B = A/254), the codes are unpacked to int8 bytes, and exact int32
// group dots are scaled once per group in fp32.  The shared expert's int8
// dots are exact int32 on the same MFMA (IDOT, bit-identical to the CPU).
// Routing is bit-exact: a certified fp64 pass proves the top-k order of the
// reference's serial fp32 router dot, and tokens it cannot certify run the
// serial chain itself.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sw_backend.h"
#include "sw_device.h"
#include "sw_synth.h"
#include "sw_moe_layer.h"
#include "sw_stack.h"
#include "sw_lds_dma.h"

using namespace sw;

namespace {

constexpr int kTileRows = 16;
constexpr int kGroup = 128;
constexpr int kMaxTopK = 32;
constexpr int kMaxTokensPerItem = 8;   // routed MFMA B columns: 8 tokens x 2 digits
constexpr int kSharedTokens = 16;      // shared IDOT B columns: 16 tokens
constexpr int kMaxTokens = 2048;       // per call (bucketing LDS bitmap)

}  // namespace



namespace {

// ---------------------------------------------------------------------------
// tile addressing
// ---------------------------------------------------------------------------
// group-relative k of lane slot s (0..31) for k-slice kb
__host__ __device__ inline int slot_k(int s, int kb) { return s < 16 ? kb * 16 + s : 64 + kb * 16 + (s - 16); }

__device__ inline int container_code(const unsigned char *row, int k, int cols, int fmt) {
  if (k >= cols) return fmt == 4 ? 8 : 4;  // zero value
  if (fmt == 4) {
    unsigned char b = row[k >> 1];
    return (k & 1) ? (b >> 4) : (b & 15);
  }
  int bit = 3 * k, byte = bit >> 3, shift = bit & 7;
  unsigned w = row[byte];
  if (shift > 5) w |= (unsigned)row[byte + 1] << 8;
  return (int)((w >> shift) & 7u);
}

// one thread per (row tile, group, lane): container codes -> tile bytes of
// the tile-group's record (record stride rs)
// (rows past rows_src, the tile padding of a ragged I, get zero values)
__global__ void k_repack_codes(unsigned char *dst, unsigned rs, const unsigned char *src, int rows, int rows_src,
                               int cols, int rb, int ng, int fmt) {
  long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long total = (long long)(rows / kTileRows) * ng * 64;
  if (tid >= total) return;
  int lane = (int)(tid & 63);
  long long tg = tid >> 6;  // rt * ng + g
  int g = (int)(tg % ng);
  int rt = (int)(tg / ng);
  int r = rt * kTileRows + (lane & 15), kb = lane >> 4;
  const bool live = r < rows_src;
  const unsigned char *row = src + (size_t)(live ? r : 0) * rb;
  int code[32];
#pragma unroll
  for (int s = 0; s < 32; s++) code[s] = container_code(row, g * kGroup + slot_k(s, kb), live ? cols : 0, fmt);
  if (fmt == 4) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t v = 0;
#pragma unroll
      for (int m = 0; m < 4; m++) v |= (uint32_t)(code[8 * i + m] | (code[8 * i + 4 + m] << 4)) << (8 * m);
      w[i] = v;
    }
    uint32_t *d = (uint32_t *)(dst + (size_t)tg * rs + lane * 16);
    d[0] = w[0];
    d[1] = w[1];
    d[2] = w[2];
    d[3] = w[3];
  } else {
    uint32_t L[2] = {0, 0}, H = 0;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int m = 0; m < 4; m++) {
        int c = code[4 * j + m];
        L[j >> 2] |= (uint32_t)(c & 3) << (8 * m + 2 * (j & 3));
        H |= (uint32_t)((c >> 2) & 1) << (8 * m + j);
      }
    uint32_t *d = (uint32_t *)(dst + (size_t)tg * rs + lane * 12);
    d[0] = L[0];
    d[1] = L[1];
    d[2] = H;
  }
}

// scales [rows][ng] -> 16 per tile-group record, at byte so of the record
__global__ void k_repack_scales(unsigned char *dst, unsigned rs, unsigned so, const float *src, int rows,
                                int rows_src, int ng) {
  long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long total = (long long)rows * ng;
  if (tid >= total) return;
  int r = (int)(tid & 15);
  long long tg = tid >> 4;
  int g = (int)(tg % ng);
  int rt = (int)(tg / ng);
  const int row = rt * kTileRows + r;
  ((float *)(dst + (size_t)tg * rs + so))[r] = row < rows_src ? src[(size_t)row * ng + g] : 0.0f;
}

// ---------------------------------------------------------------------------
// synthetic weights (sw_synth.h), generated in place
// ---------------------------------------------------------------------------
__global__ void k_synth_bytes(unsigned char *dst, size_t n, uint64_t key) {
  size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t i = w * 8;
  if (i >= n) return;
  uint64_t h = sw_word(key, w);
  if (i + 8 <= n && ((((uintptr_t)dst) & 7) == 0)) {
    *(uint64_t *)(dst + i) = h;
  } else {
    for (int b = 0; b < 8 && i + b < n; b++) dst[i + b] = (unsigned char)(h >> (8 * b));
  }
}
__global__ void k_synth_i8(signed char *dst, size_t n, uint64_t key) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = sw_i8(key, i);
}
// a [rows x cols] matrix generated as if contiguous, stored with row pitch `pitch`
__global__ void k_synth_i8_rows(signed char *dst, int rows, int cols, int pitch, uint64_t key) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * cols) return;
  const size_t r = i / (size_t)cols, c = i - r * (size_t)cols;
  dst[r * (size_t)pitch + c] = sw_i8(key, i);
}
__global__ void k_synth_normal(float *dst, size_t n, uint64_t key, float sigma, int absolute) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = absolute ? sw_abs_normal_sigma(key, i, sigma) : sw_normal_sigma(key, i, sigma);
}
// tile-group scales straight from the hash at their container index
__global__ void k_synth_scales_tiled(unsigned char *dst, unsigned rs, unsigned so, int rows, int rows_src, int ng,
                                     uint64_t key) {
  long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (long long)rows * ng) return;
  int r = (int)(tid & 15);
  long long tg = tid >> 4;
  int g = (int)(tg % ng);
  int rt = (int)(tg / ng);
  const int row = rt * kTileRows + r;
  ((float *)(dst + (size_t)tg * rs + so))[r] =
      row < rows_src ? sw_abs_normal_sigma(key, (uint64_t)row * ng + g, 0.01f) : 0.0f;
}

inline unsigned blocks_for(size_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

// capture-safe clear (a kernel, not a memset node)
__global__ void k_zero_u32(unsigned *p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ---------------------------------------------------------------------------
// activation digits: v (len n, zero-padded to ng*128) ->
//   d1, d2 int8 [ng*128], gp[g] = {A, B, Q1, Q2} with v ~= A*d1 + B*d2 and
//   Q = sum of the digits of the group.  One block; waves loop over groups.
// ---------------------------------------------------------------------------
__device__ void quantize_digits(const float *v, int n, int ng, signed char *d1, signed char *d2, float4 *gp) {
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int g = wave; g < ng; g += nw) {
    int i0 = g * kGroup + 2 * lane;
    float a = i0 < n ? v[i0] : 0.0f;
    float b = i0 + 1 < n ? v[i0 + 1] : 0.0f;
    float amax = wave_max(fmaxf(fabsf(a), fabsf(b)));
    float A = amax / 127.0f;
    float B = A / 254.0f;
    int qa1 = 0, qa2 = 0, qb1 = 0, qb2 = 0;
    if (amax > 0.0f) {
      float invA = 127.0f / amax, invB = 254.0f / A;
      qa1 = (int)fminf(fmaxf(__builtin_rintf(a * invA), -127.0f), 127.0f);
      qb1 = (int)fminf(fmaxf(__builtin_rintf(b * invA), -127.0f), 127.0f);
      float ra = __builtin_fmaf(-(float)qa1, A, a);
      float rb = __builtin_fmaf(-(float)qb1, A, b);
      qa2 = (int)fminf(fmaxf(__builtin_rintf(ra * invB), -127.0f), 127.0f);
      qb2 = (int)fminf(fmaxf(__builtin_rintf(rb * invB), -127.0f), 127.0f);
    }
    d1[i0] = (signed char)qa1;
    d1[i0 + 1] = (signed char)qb1;
    d2[i0] = (signed char)qa2;
    d2[i0 + 1] = (signed char)qb2;
    int Q1 = wave_sum_i(qa1 + qb1), Q2 = wave_sum_i(qa2 + qb2);
    if (lane == 0) gp[g] = make_float4(A, B, __int_as_float(Q1), __int_as_float(Q2));
  }
}

// qrow_i8 (c/qwen.c:1696) by one block: returns s, writes q
__device__ float qrow_i8_block(const float *x, int n, signed char *q, float *red) {
  float m = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, fabsf(x[i]));
  m = wave_max(m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float a = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) a = fmaxf(a, red[i]);
  float s = a / 127.0f;
  if (s < 1e-12f) s = 1e-12f;
  float inv = 1.0f / s;
  for (int i = threadIdx.x; i < n; i += blockDim.x) q[i] = (signed char)__builtin_rintf(x[i] * inv);
  return s;
}

// Shared expert of many tokens: token chunks per block (kSharedBlockTokens
// a block for the shared down), and steps of at most kShSplitTokens tokens
// split the shared gate/up's k range over kShSplit blocks per row tile.
constexpr int kSharedSub = 4;
constexpr int kSharedBlockTokens = 16 * kSharedSub;
#ifndef SW_SH_SPLIT_TOKENS
#define SW_SH_SPLIT_TOKENS 64
#endif
constexpr int kShSplit = 4, kShSplitTokens = SW_SH_SPLIT_TOKENS;

// ---------------------------------------------------------------------------
// per-call workspace carved from one scratch buffer
// ---------------------------------------------------------------------------
struct Work {
  int T, H, E, K, I, Ish, ngh, ngi, Hp, Ip;
  int itok;  // tokens per bucketing item: 8 (one MFMA column set) or kWideTokens
  // 1 when the step returns no routes: a certified set of K experts is taken
  // in the order of its bounds when they cannot settle it (the set is exact
  // either way, the weights come from the fp64 logits within tolerance; only
  // the combine's rounding order depends on the order)
  int order_free;
  // prep
  signed char *xq; float *sx;
  signed char *xd1, *xd2; float4 *xgp;
  // router
  double2 *lb; float *sgate; int *certified; float *logits;
  int *ulist, *ucount;  // tokens on the targeted exact path, and their count
  int *udone, *fdone;   // per token: exact chains finished (targeted, full path)
  int *flist, *fcount;  // tokens needing every expert's chain and the router_topk replica
  int *mset, *mcount;  // per token: experts of the targeted exact path (<= 64)
  int *idx; float *w;
  // bucket
  int *offsets, *btok, *bslot, *pos; int4 *items; int *nitems;
  // shared
  float *hsh; signed char *hq; float *shx; float *shout;
  int *shpart; int shks;  // k-split shared gate/up: int32 partial dots [kShSplit][T][2][Ish] (shks 0: none)
  // routed
  float *hroute; signed char *hd1, *hd2; float4 *hgp; float *rout;
  size_t bytes;
};

size_t carve(Work &w, char *base) {
  size_t off = 0;
  auto take = [&](size_t n) -> char * {
    off = (off + 255) & ~(size_t)255;
    char *p = base ? base + off : nullptr;
    off += n;
    return p;
  };
  int T = w.T, R = w.T * w.K;
  w.xq = (signed char *)take((size_t)T * w.H);
  w.sx = (float *)take((size_t)T * 4);
  w.xd1 = (signed char *)take((size_t)T * w.Hp);
  w.xd2 = (signed char *)take((size_t)T * w.Hp);
  w.xgp = (float4 *)take((size_t)T * w.ngh * 16);
  w.lb = (double2 *)take((size_t)T * (w.E + 1) * 16);
  w.sgate = (float *)take((size_t)T * 4);
  w.certified = (int *)take((size_t)T * 4);
  w.ulist = (int *)take((size_t)T * 4);
  w.udone = (int *)take((size_t)T * 4);
  w.fdone = (int *)take((size_t)T * 4);
  w.ucount = (int *)take(16);
  w.flist = (int *)take((size_t)T * 4);
  w.fcount = (int *)take(16);
  w.mset = (int *)take((size_t)T * 64 * 4);
  w.mcount = (int *)take((size_t)T * 4);
  w.logits = (float *)take((size_t)T * w.E * 4);
  w.idx = (int *)take((size_t)R * 4);
  w.w = (float *)take((size_t)R * 4);
  w.offsets = (int *)take((size_t)(w.E + 1) * 4);
  w.btok = (int *)take((size_t)R * 4);
  w.bslot = (int *)take((size_t)R * 4);
  w.pos = (int *)take((size_t)R * 4);
  w.items = (int4 *)take((size_t)(R + w.E) * 16);
  w.nitems = (int *)take(16);
  w.hsh = (float *)take((size_t)T * w.Ish * 4);
  w.shpart = (int *)take((size_t)(T <= kShSplitTokens ? kShSplit : 0) * T * 2 * w.Ish * 4);
  w.hq = (signed char *)take((size_t)T * w.Ish);
  w.shx = (float *)take((size_t)T * 4);
  w.shout = (float *)take((size_t)T * w.H * 4);
  w.hroute = (float *)take((size_t)R * w.I * 4);
  w.hd1 = (signed char *)take((size_t)R * w.Ip);
  w.hd2 = (signed char *)take((size_t)R * w.Ip);
  w.hgp = (float4 *)take((size_t)R * w.ngi * 16);
  w.rout = (float *)take((size_t)R * w.H * 4);
  w.bytes = off + 256;
  return w.bytes;
}

// ---------------------------------------------------------------------------
// 1. activation prep: IDOT quantisation + routed digits.  The row is read once
// into registers: C float4 chunks per thread (1024 threads, padded row of up
// to C*4096 values); a group of 128 values is one half-wave's 32 chunks.
// grid T, 1024 threads.  Rows longer than 32768 take k_prep_x_any.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int half_wave_sum_i(int v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ unsigned pack_i8x4(int a, int b, int c, int d) {
  return (unsigned)(a & 255) | ((unsigned)(b & 255) << 8) | ((unsigned)(c & 255) << 16) | ((unsigned)d << 24);
}

// The shared-expert gate sigmoid(x . g) of token t from the block's fp64
// partial dots (every product exact, one fp64 rounding per sum): wave sums,
// then thread 0 adds the 16 waves' in wave order.  The gate scales the shared
// expert's output, which is compared within the output tolerance.
__device__ __forceinline__ void block_gate(Work &w, int t, double d, double *redd) {
  d = wave_sum_dpp(d);
  if ((threadIdx.x & 63) == 0) redd[threadIdx.x >> 6] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double L = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) L += redd[i];
    w.sgate[t] = sigmoid_ref((float)L);
  }
}

// The certification's lists and per-token chain counters start the step at
// zero (the certification appends to the lists).
__device__ __forceinline__ void reset_counters(Work &w, int t) {
  if (threadIdx.x == 0) {
    if (t == 0) *w.ucount = *w.fcount = 0;
    w.udone[t] = w.fdone[t] = 0;
  }
}

// Token t's activation forms, by a block of NT threads (C float4s each,
// C * NT >= the padded row's float4s): the row quantisation, the two-digit
// groups, the shared gate; RESET: the step's certification counters too.
template <int C, int NT, bool RESET>
__device__ __forceinline__ void prep_token(Work &w, const float *x, const float *sgate_row, int t, float *red,
                                           double *redd) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const float *xt = x + (size_t)t * w.H;
  if (RESET) reset_counters(w, t);
  const int nq = w.H / 4, nqp = w.ngh * 32;  // float4 chunks of the row, of the padded row
  const bool al = ((uintptr_t)xt & 15) == 0;
  float4 v[C];
  float m = 0.0f;
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int i = tid + NT * c;
    v[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (i < nq) v[c] = al ? *(const float4 *)(xt + 4 * i) : make_float4(xt[4 * i], xt[4 * i + 1], xt[4 * i + 2], xt[4 * i + 3]);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[c].x), fabsf(v[c].y)), fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
  }
  double gd = 0.0;
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int i = tid + NT * c;
    if (i < nq) {
      const float4 g = *(const float4 *)(sgate_row + 4 * i);
      gd = __builtin_fma((double)v[c].x, (double)g.x, gd);
      gd = __builtin_fma((double)v[c].y, (double)g.y, gd);
      gd = __builtin_fma((double)v[c].z, (double)g.z, gd);
      gd = __builtin_fma((double)v[c].w, (double)g.w, gd);
    }
  }
  block_gate(w, t, gd, redd);
  // qrow_i8 (c/qwen.c:1696): s = max|x|/127 (at least 1e-12), q = rint(x/s)
  m = wave_max(m);
  if (lane == 0) red[tid >> 6] = m;
  __syncthreads();
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; i++) a = fmaxf(a, red[i]);
  float sx = a / 127.0f;
  if (sx < 1e-12f) sx = 1e-12f;
  const float inv = 1.0f / sx;
  if (tid == 0) w.sx[t] = sx;
  unsigned *xq = (unsigned *)(w.xq + (size_t)t * w.H);
  unsigned *d1 = (unsigned *)(w.xd1 + (size_t)t * w.Hp), *d2 = (unsigned *)(w.xd2 + (size_t)t * w.Hp);
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int i = tid + NT * c;
    if (i < nq)
      xq[i] = pack_i8x4((int)__builtin_rintf(v[c].x * inv), (int)__builtin_rintf(v[c].y * inv),
                        (int)__builtin_rintf(v[c].z * inv), (int)__builtin_rintf(v[c].w * inv));
    // two digits per value of the group (half-wave), as quantize_digits
    if (i < nqp) {  // uniform over the half-wave: nqp and NT are multiples of 32
      const float amax = half_wave_max(fmaxf(fmaxf(fabsf(v[c].x), fabsf(v[c].y)), fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
      const float A = amax / 127.0f, B = A / 254.0f;
      int q1[4] = {0, 0, 0, 0}, q2[4] = {0, 0, 0, 0};
      if (amax > 0.0f) {
        const float invA = 127.0f / amax, invB = 254.0f / A;
        const float e[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          q1[k] = (int)fminf(fmaxf(__builtin_rintf(e[k] * invA), -127.0f), 127.0f);
          const float r = __builtin_fmaf(-(float)q1[k], A, e[k]);
          q2[k] = (int)fminf(fmaxf(__builtin_rintf(r * invB), -127.0f), 127.0f);
        }
      }
      d1[i] = pack_i8x4(q1[0], q1[1], q1[2], q1[3]);
      d2[i] = pack_i8x4(q2[0], q2[1], q2[2], q2[3]);
      const int Q1 = half_wave_sum_i(q1[0] + q1[1] + q1[2] + q1[3]);
      const int Q2 = half_wave_sum_i(q2[0] + q2[1] + q2[2] + q2[3]);
      if ((lane & 31) == 0) w.xgp[(size_t)t * w.ngh + i / 32] = make_float4(A, B, __int_as_float(Q1), __int_as_float(Q2));
    }
  }
}

template <int C>
__global__ __launch_bounds__(1024) void k_prep_x(Work w, const float *x, const float *sgate_row) {
  __shared__ float red[16];
  __shared__ double redd[16];
  prep_token<C, 1024, true>(w, x, sgate_row, blockIdx.x, red, redd);
}

// Any row length: quantize_digits and qrow_i8_block read the row from memory.
// grid T, 1024 threads.
__global__ void k_prep_x_any(Work w, const float *x, const float *sgate_row) {
  __shared__ float red[16];
  __shared__ double redd[16];
  int t = blockIdx.x;
  const float *xt = x + (size_t)t * w.H;
  double gd = 0.0;
  for (int i = threadIdx.x; i < w.H; i += blockDim.x) gd = __builtin_fma((double)xt[i], (double)sgate_row[i], gd);
  block_gate(w, t, gd, redd);
  if (t == 0 && threadIdx.x == 0) *w.ucount = *w.fcount = 0;  // the certification appends to them
  if (threadIdx.x == 0) w.udone[t] = w.fdone[t] = 0;
  float s = qrow_i8_block(xt, w.H, w.xq + (size_t)t * w.H, red);
  if (threadIdx.x == 0) w.sx[t] = s;
  quantize_digits(xt, w.H, w.ngh, w.xd1 + (size_t)t * w.Hp, w.xd2 + (size_t)t * w.Hp, w.xgp + (size_t)t * w.ngh);
}

// ---------------------------------------------------------------------------
// 2. router: per (token, expert) the fp64 logit L and a rigorous bound B on
// |fl32 serial dot - L| (c/qwen.c:1674 evaluated as s = rn(s + rn(x*w)),
// tail FMA).  Each step's rounding is at most u*|partial| (u = 2^-24), each
// product's at most u*|x*w|, so |err| <= u*(sum|x w| + sum_k |S_k|)*(1+uH).
// Lane j owns the contiguous chunk j of the row; the prefix sums S_k are the
// chunk offset O_j plus the local prefix, bounded by |O_j| + |local|.  L and
// the prefix sums are fp64 (every product exact); sum|x w| is an fp32 sum of
// non-negative terms per lane, at most gamma_n (n = chunk length) below the
// exact one, so it is scaled by 1 + 2^-23 n.  grid (ceil(E/4), T), 256 threads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double router_bound(double A, double Pb) {
  const double u = 0x1p-24;
  return u * (A + Pb) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-36;
}

__global__ void k_router_bounds(Work w, const float *x, const float *router) {
  int lane = threadIdx.x & 63;
  int e = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
  if (e >= w.E) return;
  const float *row = router + (size_t)e * w.H;
  const float *xt = x + (size_t)t * w.H;
  int chunk = (w.H + 63) / 64;
  int i0 = lane * chunk, i1 = min(i0 + chunk, w.H);
  double lp = 0.0, pa = 0.0;
  float aa = 0.0f;
  for (int i = i0; i < i1; i++) {
    const float xf = xt[i], wf = row[i];
    lp = __builtin_fma((double)xf, (double)wf, lp);
    aa = __builtin_fmaf(fabsf(xf), fabsf(wf), aa);
    pa += fabs(lp);
  }
  double off = wave_exclusive_scan(lp, lane);
  double L = wave_sum(lp);
  double Pb = wave_sum((double)(i1 > i0 ? i1 - i0 : 0) * fabs(off) + pa);
  double A = wave_sum((double)aa) * (1.0 + 0x1p-23 * chunk);
  if (lane == 0) w.lb[(size_t)t * (w.E + 1) + e] = make_double2(L, router_bound(A, Pb));
}

// The bound of k_router_bounds (lane j owns the contiguous chunk j of CH =
// H/64 elements, same per-lane fma order), arranged for many tokens: wave w of
// a block holds router row e = RB*blockIdx.x + w in registers, read once, and
// walks the block's tokens kRbRound at a time.  A round's tokens share each
// element's conversion of the row value and run as kRbRound independent fma
// chains, element-major, so the chains hide each other's latency.
//
// A round's activations reach LDS by global->LDS copies, all in flight at
// once.  Lane j reads its chunk as float4s; the chunk's 16-byte units are
// stored XOR-swizzled (unit q of chunk j at position q ^ (j & m), m = min(7,
// CH/4 - 1)), so the eight lanes of a 128-bit LDS pass hit distinct banks.
// The first column of blocks also resets the certification counters of its
// tokens.  grid (ceil(E/RB), ceil(T/tokens_per_block)), 64*RB threads, dynamic
// LDS kRbRound*H floats.  Requires x 16-byte aligned, CH % 4 == 0.
constexpr int kRbRound = 4;
template <int CH, int RB>
__global__ __launch_bounds__(64 * RB) __attribute__((amdgpu_waves_per_eu(4))) void k_router_bounds_tiled(
    Work w, const float *x, const float *router, int tokens_per_block) {
  extern __shared__ float4 rb_xs4[];  // [kRbRound][H / 4], swizzled within chunks
  static_assert(CH % 4 == 0 && (CH & (CH - 1)) == 0, "chunks of a power of two of float4s");
  constexpr unsigned H = 64 * CH, U = CH / 4, M = U < 8 ? U - 1 : 7, HU = H / 4;
  if (blockIdx.x == 0)
    for (int t = blockIdx.y * tokens_per_block; t < min((int)(blockIdx.y + 1) * tokens_per_block, w.T); t++)
      reset_counters(w, t);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = blockIdx.x * RB + wave;
  const bool live = e < w.E;
  float wr[CH];
  if (live) {
    const float4 *r4 = (const float4 *)(router + (size_t)e * H + lane * CH);
#pragma unroll
    for (int c = 0; c < CH / 4; c++) {
      float4 v = r4[c];
      wr[4 * c] = v.x;
      wr[4 * c + 1] = v.y;
      wr[4 * c + 2] = v.z;
      wr[4 * c + 3] = v.w;
    }
  }
  const unsigned sw16 = (unsigned)(lane & M) << 4;  // this lane's read swizzle, bytes
  const int t0 = blockIdx.y * tokens_per_block, t1 = min(t0 + tokens_per_block, w.T);
  for (int tb = t0; tb < t1; tb += kRbRound) {
    const unsigned ng = min(kRbRound, t1 - tb);
    __syncthreads();  // the previous round's reads are done
    // LDS unit u (a wave's 64 consecutive units per copy) of token g = u / HU
    // holds element 4 q of chunk j: uu = u mod HU, j = uu / U, q = uu mod U ^ (j & M)
    for (unsigned u0 = wave * 64; u0 < ng * HU; u0 += 64 * RB) {  // wave-uniform
      const unsigned u = u0 + lane, g = u / HU, uu = u % HU, j = uu / U, q = (uu % U) ^ (j & M);
      dma_b128(x + (size_t)(tb + g) * H + j * CH + 4 * q, lds_addr(rb_xs4 + u0));
    }
    wait_dma();
    __syncthreads();
    if (!live) continue;
    // the row is converted per round, not hoisted out of the round loop (a
    // double copy would take 2*CH registers): opaque to the compiler from here
#pragma unroll
    for (int c = 0; c < CH; c++) asm volatile("" : "+v"(wr[c]));
    // rounds of fewer tokens compute on stale activations and store nothing
    double lp[kRbRound], pa[kRbRound];
    float aa[kRbRound];
#pragma unroll
    for (int g = 0; g < kRbRound; g++) {
      lp[g] = pa[g] = 0.0;
      aa[g] = 0.0f;
    }
    const char *xs = (const char *)rb_xs4 + lane * CH * 4;  // the lane's chunk of token 0
    float4 xv[kRbRound], xn[kRbRound];
#pragma unroll
    for (int g = 0; g < kRbRound; g++) xn[g] = *(const float4 *)(xs + sw16 + g * H * 4);
#pragma unroll
    for (int c0 = 0; c0 < CH; c0 += 4) {
      // one step of prefetch: the next reads' address depends (opaquely) on
      // every chain's step before, so the compiler neither hoists every read
      // of the unrolled loop to the top (which spills) nor sinks a chain's
      // arithmetic to the end
      static_assert(kRbRound == 4, "the dependency names four chains");
      unsigned dep = 0;
      if (c0 >= 4)
        asm("v_mov_b32 %0, 0"
            : "=v"(dep)
            : "v"(lp[0]), "v"(lp[1]), "v"(lp[2]), "v"(lp[3]), "v"(pa[0]), "v"(pa[1]), "v"(pa[2]), "v"(pa[3]),
              "v"(aa[0]), "v"(aa[1]), "v"(aa[2]), "v"(aa[3]));
      const unsigned nx = ((unsigned)(c0 + 4) << 2 ^ sw16) + dep;  // next step's unit, bytes
#pragma unroll
      for (int g = 0; g < kRbRound; g++) {
        xv[g] = xn[g];
        if (c0 + 4 < CH) xn[g] = *(const float4 *)(xs + nx + g * H * 4);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float wf = wr[c0 + q];
        const double wd = (double)wf;
#pragma unroll
        for (int g = 0; g < kRbRound; g++) {
          const float xf = q == 0 ? xv[g].x : q == 1 ? xv[g].y : q == 2 ? xv[g].z : xv[g].w;
          lp[g] = __builtin_fma((double)xf, wd, lp[g]);
          aa[g] = __builtin_fmaf(fabsf(xf), fabsf(wf), aa[g]);
          pa[g] += fabs(lp[g]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < kRbRound; g++) {
      // DPP reductions: the inclusive scan's last lane is the logit
      const double inc = wave_incl_scan_dpp(lp[g]);
      const double off = inc - lp[g];
      const double L = readlane_d63(inc);
      const double Pb = wave_sum_dpp((double)CH * fabs(off) + pa[g]);
      const double A = wave_sum_dpp((double)aa[g]) * (1.0 + 0x1p-23 * CH);
      if (lane == 0 && g < (int)ng) w.lb[(size_t)(tb + g) * (w.E + 1) + e] = make_double2(L, router_bound(A, Pb));
    }
  }
}

// ---------------------------------------------------------------------------
// 2g. Router for many tokens as an fp64 GEMM on MFMA, with an a-priori bound
// tightened where it matters.
//
// L[t][e] = sum_i x_t[i] w_e[i] in fp64 (fp32 inputs: every product is exact
// in fp64) on v_mfma_f64_16x16x4.  Any evaluation order of the reference's
// fp32 dot (c/qwen.c:1674) is within gamma_H * sum|x_i w_i| of the exact sum
// (gamma_n = n u / (1 - n u), u = 2^-24, products and sums rounded once
// each), and so is L within the fp64 analogue; sum|x_i w_i| <= ||x_t|| ||w_e||
// (Cauchy-Schwarz).  So B0 = (gamma_H + gamma'_H) ||x_t|| ||w_e|| (with
// slack) bounds |fp32 logit - L| for every (t, e).  B0 is about a hundred
// times looser than the prefix-sum bound of k_router_bounds, so
// k_router_refine replaces it by that tight bound for the experts that could
// be among a token's top K; the rest are far below the K-th logit and keep
// B0.  Every (L, B) pair stays a valid enclosure, so the certification that
// follows is rigorous whichever experts were refined.
// ---------------------------------------------------------------------------
typedef double v4d __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
  return v;
}

// a-priori bound factor: (gamma_H(2^-24) + gamma_H(2^-53)) with slack for the
// rounding of the norms and of the product that applies it
__device__ __forceinline__ double gemm_bound_factor(int H) {
  const double n = (double)H, u = 0x1p-24, v = 0x1p-53;
  return (n * u / (1.0 - n * u) + n * v / (1.0 - n * v)) * (1.0 + 0x1p-20);
}

// One 16-token x 16-row tile of L per block; its 4 waves take a quarter of
// the k range each and their sums meet in LDS in wave order.  MFMA step c of
// k block kb pairs x_t[16 kb + 4 (l >> 4) + c] with w_e[16 kb + 4 (l >> 4) +
// c] at lane l (A: token t0 + l % 16, B: row e0 + l % 16), so every lane
// loads float4s; the result holds token t0 + (l >> 4) + 4 v, row e0 + l % 16
// at lane l, item v (the f64 16x16x4 output layout: D[(l >> 4) + 4 v][l % 16]).
// The same loads give ||x_t|| and ||w_e|| (fp64 sums of squares).
// grid (ceil(E/16), ceil(T/16)), 256 threads.  H % 64 == 0, x 16-byte aligned.
__global__ __launch_bounds__(256) void k_router_gemm(Work w, const float *x, const float *router) {
  __shared__ double s_acc[4][4][64];
  __shared__ double s_nx[4][64], s_nw[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
  const int H = w.H, kq = H / 4;
  const int ta = min(t0 + (lane & 15), w.T - 1), eb = min(e0 + (lane & 15), w.E - 1);
  const float *xa = x + (size_t)ta * H + wave * kq + 4 * (lane >> 4);
  const float *wb = router + (size_t)eb * H + wave * kq + 4 * (lane >> 4);
  v4d acc = {0.0, 0.0, 0.0, 0.0};
  double qa = 0.0, qb = 0.0;
#pragma unroll 4
  for (int k = 0; k < kq; k += 16) {
    const float4 a = *(const float4 *)(xa + k), b = *(const float4 *)(wb + k);
    const double a0 = a.x, a1 = a.y, a2 = a.z, a3 = a.w, b0 = b.x, b1 = b.y, b2 = b.z, b3 = b.w;
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a2, b2, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a3, b3, acc, 0, 0, 0);
    qa = __builtin_fma(a0, a0, __builtin_fma(a1, a1, __builtin_fma(a2, a2, __builtin_fma(a3, a3, qa))));
    qb = __builtin_fma(b0, b0, __builtin_fma(b1, b1, __builtin_fma(b2, b2, __builtin_fma(b3, b3, qb))));
  }
  // sums of squares: lanes l, l^16, l^32, l^48 share a token / a row
  qa += __shfl_xor(qa, 16, 64);
  qa += __shfl_xor(qa, 32, 64);
  qb += __shfl_xor(qb, 16, 64);
  qb += __shfl_xor(qb, 32, 64);
#pragma unroll
  for (int v = 0; v < 4; v++) s_acc[wave][v][lane] = acc[v];
  s_nx[wave][lane] = qa;
  s_nw[wave][lane] = qb;
  __syncthreads();
  if (wave != 0) return;
  const int e = e0 + (lane & 15);
  if (e >= w.E) return;
  const double nw = sqrt(((s_nw[0][lane] + s_nw[1][lane]) + s_nw[2][lane]) + s_nw[3][lane]);
  const double f = gemm_bound_factor(H) * nw;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int i = (lane >> 4) + 4 * v, t = t0 + i;
    if (t >= w.T) continue;
    const double L = ((s_acc[0][v][lane] + s_acc[1][v][lane]) + s_acc[2][v][lane]) + s_acc[3][v][lane];
    const double nx = sqrt(((s_nx[0][i] + s_nx[1][i]) + s_nx[2][i]) + s_nx[3][i]);
    w.lb[(size_t)t * (w.E + 1) + e] = make_double2(L, f * nx + 1e-36);
  }
}

// Per token: the experts whose interval reaches below-threshold get the tight
// bound of k_router_bounds (lane j's contiguous chunk, exact local prefixes,
// chunk offsets by a wave scan).  The threshold is the K-th largest of the
// lanes' largest logits (at most the K-th largest logit) less the largest
// a-priori bound; experts under it cannot reach any of the top K.  Wave 0
// selects; the waves refine the candidates in turn, the token's x staged in
// LDS lane-major with one pad word per lane.  More than kRefineMax candidates:
// the token keeps the a-priori bounds (the certification then takes its exact
// paths).  grid T, 256 threads, dynamic LDS 64 (H/64 + 1) floats.
constexpr int kRefineMax = 64;
__global__ __launch_bounds__(256) void k_router_refine(Work w, const float *x, const float *router) {
  extern __shared__ float rf_x[];
  __shared__ int cand[kRefineMax];
  __shared__ int s_n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = blockIdx.x;
  const int E = w.E, K = w.K, H = w.H, CH = H / 64, P = CH + 1;
  const double2 *lb = w.lb + (size_t)t * (E + 1);
  const float *xt = x + (size_t)t * H;
  for (int i = threadIdx.x; i < H; i += blockDim.x) rf_x[(i / CH) * P + i % CH] = xt[i];
  if (wave == 0) {
    double m = -1e300, bmax = 0.0;
    for (int e = lane; e < E; e += 64) {
      const double2 v = lb[e];
      m = fmax(m, v.x);
      bmax = fmax(bmax, v.y);
    }
    bmax = wave_max_dpp(bmax);
    // K-th largest lane maximum: K rounds that retire the largest
    double thr = m;
    bool out = false;
    for (int k = 0; k < K && k < 64; k++) {
      const double v = out ? -1e300 : m;
      const double g = wave_max_dpp(v);
      const unsigned long long hit = __ballot(!out && m == g);
      if (hit && lane == __ffsll((long long)hit) - 1) out = true;
      thr = g;
    }
    thr -= bmax;
    int n = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      bool c = false;
      if (e < E) {
        const double2 v = lb[e];
        c = v.x + v.y >= thr;
      }
      const unsigned long long bal = __ballot(c);
      const int before = __popcll(bal & ((1ull << lane) - 1ull));
      if (c && n + before < kRefineMax) cand[n + before] = e;
      n += __popcll(bal);
    }
    if (lane == 0) s_n = n <= kRefineMax ? n : 0;
  }
  __syncthreads();
  const int n = s_n;
  const float *xl = rf_x + lane * P;
  for (int c = wave; c < n; c += 4) {
    const int e = cand[c];
    const float *row = router + (size_t)e * H + lane * CH;
    double lp = 0.0, pa = 0.0, aa = 0.0;
    if ((CH & 3) == 0) {
      for (int i = 0; i < CH; i += 4) {
        const float4 r = *(const float4 *)(row + i);
        const float rv[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const double xd = (double)xl[i + q], wd = (double)rv[q];
          lp = __builtin_fma(xd, wd, lp);
          aa = __builtin_fma(fabs(xd), fabs(wd), aa);
          pa += fabs(lp);
        }
      }
    } else {
      for (int i = 0; i < CH; i++) {
        const double xd = (double)xl[i], wd = (double)row[i];
        lp = __builtin_fma(xd, wd, lp);
        aa = __builtin_fma(fabs(xd), fabs(wd), aa);
        pa += fabs(lp);
      }
    }
    const double inc = wave_incl_scan_dpp(lp);
    const double off = inc - lp;
    const double L = readlane_d63(inc);
    const double Pb = wave_sum_dpp((double)CH * fabs(off) + pa);
    const double A = wave_sum_dpp(aa);
    if (lane == 0) {
      const double u = 0x1p-24;
      const double B = u * (A + Pb) * (1.0 + 0x1p-10) + 1e-12 * A + 1e-36;
      w.lb[(size_t)t * (E + 1) + e] = make_double2(L, B);
    }
  }
}

// block argmax over (value, index): largest value, lowest index on ties
struct VI {
  double v;
  int i;
};
__device__ inline VI vi_better(VI a, VI b) {
  if (b.i < 0) return a;
  if (a.i < 0) return b;
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}
__device__ VI block_argmax(VI x, VI *red) {
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    VI y;
    y.v = __shfl_xor(x.v, o, 64);
    y.i = __shfl_xor(x.i, o, 64);
    x = vi_better(x, y);
  }
  __syncthreads();
  if (lane == 0) red[wave] = x;
  __syncthreads();
  VI r = red[0];
  for (int i = 1; i < nw; i++) r = vi_better(r, red[i]);
  return r;
}

// ---------------------------------------------------------------------------
// 3. certify: the top-k order (and the k|k+1 boundary) of the fp32 logits is
// fixed if the bound intervals of adjacent candidates are disjoint with a
// margin that also covers the rounding of (l - max), expf and the division,
// so router_topk on the true fp32 logits picks exactly these indices.
// grid T, 512 threads.
// ---------------------------------------------------------------------------
__global__ void k_certify(Work w, int mode, unsigned long long *stats) {
  __shared__ VI red[16];
  __shared__ int cand[kMaxTopK + 1];
  __shared__ unsigned char chosen[4096];
  int t = blockIdx.x;
  const double2 *lb = w.lb + (size_t)t * (w.E + 1);
  for (int e = threadIdx.x; e < w.E; e += blockDim.x) chosen[e] = 0;
  __syncthreads();
  int nc = min(w.K + 1, w.E);
  for (int r = 0; r < nc; r++) {
    VI best = {0.0, -1};
    for (int e = threadIdx.x; e < w.E; e += blockDim.x)
      if (!chosen[e]) best = vi_better(best, VI{lb[e].x, e});
    best = block_argmax(best, red);
    if (threadIdx.x == 0) {
      cand[r] = best.i;
      chosen[best.i] = 1;
    }
    __syncthreads();
  }
  // largest upper bound among experts outside the top-k
  VI up = {0.0, -1};
  for (int e = threadIdx.x; e < w.E; e += blockDim.x) {
    bool in_top = false;
    for (int r = 0; r < w.K && r < nc; r++) in_top |= cand[r] == e;
    if (!in_top) up = vi_better(up, VI{lb[e].x + lb[e].y, e});
  }
  up = block_argmax(up, red);
  if (threadIdx.x == 0) {
    double mx = lb[cand[0]].x;
    bool ok = mode == 0 && w.K <= w.E;
    for (int r = 0; ok && r + 1 < w.K; r++) {
      double2 a = lb[cand[r]], b = lb[cand[r + 1]];
      double margin = 0x1p-20 * (1.0 + fabs(a.x) + fabs(b.x) + 2.0 * fabs(mx));
      ok = (a.x - a.y) - (b.x + b.y) > margin;
    }
    if (ok && up.i >= 0) {
      double2 a = lb[cand[w.K - 1]];
      double margin = 0x1p-20 * (1.0 + fabs(a.x) + fabs(up.v) + 2.0 * fabs(mx));
      ok = (a.x - a.y) - up.v > margin;
    }
    if (ok) ok = (lb[cand[w.K - 1]].x - lb[cand[w.K - 1]].y) - (mx + lb[cand[0]].y) > -80.0;
    w.certified[t] = ok ? 1 : 0;
    if (!ok) w.flist[atomicAdd(w.fcount, 1)] = t;
    if (ok) {
      double p[kMaxTopK], den = 0.0;
      for (int r = 0; r < w.K; r++) {
        p[r] = exp(lb[cand[r]].x - mx);
        den += p[r];
      }
      for (int r = 0; r < w.K; r++) {
        w.idx[(size_t)t * w.K + r] = cand[r];
        w.w[(size_t)t * w.K + r] = (float)(p[r] / den);
      }
    }
    if (!ok) {  // (tokens routed: counted once per step by k_exact_logits)
      atomicAdd(&stats[1], 1ull);
      atomicAdd(&stats[2], 1ull);  // this path always re-runs every expert's chain
    }
  }
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

// Certification with one wave per token (E <= 64*NV): the same tests as
// k_certify.  A token the bounds do not certify gets the targeted exact set
// M = {e : L_e + B_e >= lo - m}, lo the lowest lower bound among the K
// candidates and m = 2^-20 (1 + 4 max_e(|L_e| + B_e)), which is at least the
// separation margin of any pair: every expert outside M has an exact logit
// below each candidate's by more than the margin, so the exact top-k lies in
// M.  certified[t]: 1 certified, 2 targeted (M in mset, |M| <= 64), 0 every
// chain.  grid ceil(T/4), 256 threads.
// order-preserving unsigned key of a float (larger float, larger key)
__device__ __forceinline__ unsigned order_key(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// PC > 0: the blocks after the certification's form the activations of one
// token each (prep_token with C = PC), independent of the certification; the
// counters were reset by the bounds kernel.  grid ceil(T/4) (+ T), 256 threads.
template <int NV, int PC>
__global__ __launch_bounds__(256) void k_certify_wave(Work w, int mode, unsigned long long *stats, const float *x,
                                                      const float *sgate_row) {
  __shared__ int cand_s[4][kMaxTopK + 1];
  __shared__ double2 cv_s[4][kMaxTopK + 1];  // the candidates' (L, B)
  if (PC > 0 && (int)blockIdx.x >= (w.T + 3) / 4) {
    __shared__ float red[4];
    __shared__ double redd[4];
    prep_token<(PC > 0 ? PC : 1), 256, false>(w, x, sgate_row, blockIdx.x - (w.T + 3) / 4, red, redd);
    return;
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wv;
  if (t >= w.T) return;
  int *cand = cand_s[wv];
  double2 *cv = cv_s[wv];
  const double2 *lb = w.lb + (size_t)t * (w.E + 1);
  double2 v[NV];
  double amax = 0.0;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    int e = lane + 64 * j;
    v[j] = e < w.E ? lb[e] : make_double2(0.0, 0.0);
    if (e < w.E) amax = fmax(amax, fabs(v[j].x) + v[j].y);
  }
  amax = wave_max_d(amax);
  // The K+1 candidates by rounds of a wave maximum over 64-bit keys (the
  // logit rounded to fp32, order-preserving, then the complemented index:
  // the lowest index first among equal keys).  Candidates that the fp32
  // rounding ranks wrongly differ by less than the pair margin, so the
  // checks below send their token to the exact path.
  const int nc = min(w.K + 1, w.E);
  unsigned long long key[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int e = lane + 64 * j;
    key[j] = e < w.E ? ((unsigned long long)order_key((float)v[j].x) << 32) | (unsigned)(~e) : 0ull;
  }
  unsigned chosen = 0;
  for (int r = 0; r < nc; r++) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < NV; j++)
      if (!((chosen >> j) & 1) && key[j] > best) best = key[j];
    best = wave_max_u64(best);
    const int eb = best ? (int)(~(unsigned)best) : -1;
    if (eb >= 0 && (eb & 63) == lane) {
      const int jb = eb >> 6;
      chosen |= 1u << jb;
#pragma unroll
      for (int j = 0; j < NV; j++)
        if (j == jb) cv[r] = v[j];
    }
    if (lane == 0) cand[r] = eb;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // largest upper bound outside the top K
  const int candK = nc > w.K ? cand[w.K] : -1;
  double up = -__builtin_huge_val();
  int upi = -1;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    int e = lane + 64 * j;
    bool in_top = ((chosen >> j) & 1) && e != candK;
    if (e < w.E && !in_top && v[j].x + v[j].y > up) {
      up = v[j].x + v[j].y;
      upi = e;
    }
  }
  up = wave_max_d(up);
  upi = wave_max_i(upi);
  // the consecutive pairs (lane r: ranks r and r+1), the set against the
  // largest outside upper bound and the softmax range, all lane-parallel;
  // then the weights from the fp64 logits, one exp per lane
  const double mx = cv[0].x;
  bool pair = true;
  if (lane + 1 < w.K) {
    const double2 a = cv[lane], b = cv[lane + 1];
    const double margin = 0x1p-20 * (1.0 + fabs(a.x) + fabs(b.x) + 2.0 * fabs(mx));
    pair = (a.x - a.y) - (b.x + b.y) > margin;
  }
  bool ok = mode == 0 && w.K <= w.E && (w.order_free || __all(pair));
  // the lowest lower bound among the K and its candidate's logit (the K-th
  // candidate's when every pair is certified; any of them when the order is
  // taken as it is)
  double klo = lane < w.K ? cv[lane].x - cv[lane].y : __builtin_huge_val();
  double kax = lane < w.K ? fabs(cv[lane].x) : 0.0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    klo = fmin(klo, __shfl_xor(klo, o, 64));
    kax = fmax(kax, __shfl_xor(kax, o, 64));
  }
  if (ok && upi >= 0) {
    const double margin = 0x1p-20 * (1.0 + kax + fabs(up) + 2.0 * fabs(mx));
    ok = klo - up > margin;
  }
  if (ok) ok = klo - (mx + cv[0].y) > -80.0;
  int verdict = ok ? 1 : 0;
  double lo = 0.0;
  if (ok) {
    const double ev = lane < w.K ? exp(cv[lane].x - mx) : 0.0;
    const double den = wave_sum(ev);
    if (lane < w.K) {
      w.idx[(size_t)t * w.K + lane] = cand[lane];
      w.w[(size_t)t * w.K + lane] = (float)(ev / den);
    }
  } else if (mode == 0 && w.K <= w.E) {
    lo = lane < w.K ? cv[lane].x - cv[lane].y : __builtin_huge_val();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lo = fmin(lo, __shfl_xor(lo, o, 64));
    verdict = 2;
  }
  if (verdict == 2) {
    lo = lo - 0x1p-20 * (1.0 + 4.0 * amax);
    int base = 0;
#pragma unroll
    for (int j = 0; j < NV; j++) {
      int e = lane + 64 * j;
      bool in_m = e < w.E && v[j].x + v[j].y >= lo;
      unsigned long long bal = __ballot(in_m);
      int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
      if (in_m && pos < 64) w.mset[(size_t)t * 64 + pos] = e;
      base += __popcll(bal);
    }
    if (base > 64) verdict = 0;
    if (lane == 0) w.mcount[t] = base;
  }
  if (lane == 0) {
    w.certified[t] = verdict;
    if (verdict == 2) w.ulist[atomicAdd(w.ucount, 1)] = t;
    if (verdict == 0) w.flist[atomicAdd(w.fcount, 1)] = t;
    // (tokens routed are counted once per step by k_exact_logits: one atomic
    // per token on one word would serialise hundreds of them)
    if (verdict != 1) atomicAdd(&stats[1], 1ull);
    if (verdict == 0) atomicAdd(&stats[2], 1ull);
  }
}

// The reference's fp32 serial dot (c/qwen.c:1674 at -O3): s = rn(s + rn(x*w))
// over the first H - H%8 terms in order, then fused multiply-adds.
__device__ float exact_chain(const float *xt, const float *row, int H) {
  int m = (H / 8) * 8;
  float s = 0.0f;
  int i = 0;
  for (; i + 4 <= m; i += 4) {
    float4 wv = *(const float4 *)(row + i);
    float4 xv = *(const float4 *)(xt + i);
    s = __fadd_rn(s, __fmul_rn(xv.x, wv.x));
    s = __fadd_rn(s, __fmul_rn(xv.y, wv.y));
    s = __fadd_rn(s, __fmul_rn(xv.z, wv.z));
    s = __fadd_rn(s, __fmul_rn(xv.w, wv.w));
  }
  for (; i < m; i++) s = __fadd_rn(s, __fmul_rn(xt[i], row[i]));
  for (; i < H; i++) s = __fmaf_rn(xt[i], row[i], s);
  return s;
}

// prod[i] = rn(x[i]*row[i]) for i < m (m % 4 == 0) by the block's 64 lanes:
// kProdBatch float4 pairs of loads in flight per lane before the first store
constexpr int kProdBatch = 8;
__device__ __forceinline__ void form_products(const float *xt, const float *row, int m, float *prod) {
  for (int i0 = threadIdx.x * 4; i0 < m; i0 += 256 * kProdBatch) {
    float4 a[kProdBatch], b[kProdBatch];
#pragma unroll
    for (int u = 0; u < kProdBatch; u++) {
      const int i = i0 + 256 * u;
      if (i < m) {
        a[u] = *(const float4 *)(xt + i);
        b[u] = *(const float4 *)(row + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kProdBatch; u++) {
      const int i = i0 + 256 * u;
      if (i < m)
        *(float4 *)(prod + i) = make_float4(__fmul_rn(a[u].x, b[u].x), __fmul_rn(a[u].y, b[u].y),
                                            __fmul_rn(a[u].z, b[u].z), __fmul_rn(a[u].w, b[u].w));
    }
  }
}

// Token t on the targeted path: M ordered by (exact logit desc, index asc);
// the order and the k|k+1 boundary hold if consecutive exact logits are
// separated by the margin and the K-th lies within 80 of the max (experts
// outside M are below every candidate by more than the margin).  Weights then
// come from the fp64 logits as for certified tokens.  Otherwise the token
// joins the full path (every chain and the router_topk replica).  Run by one
// 64-thread block once every chain of the token's M is written.
__device__ void topk_check_token(Work &w, int t, unsigned long long *stats) {
  __shared__ int um[64], sm[64];
  __shared__ float ul[64], sl[64];
  const int i = threadIdx.x;
  const int n = w.mcount[t];
  if (i < n) {
    um[i] = w.mset[(size_t)t * 64 + i];
    ul[i] = __hip_atomic_load(&w.logits[(size_t)t * w.E + um[i]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (i < n) {  // rank by (exact logit desc, index asc)
    const int e = um[i];
    const float l = ul[i];
    int rank = 0;
    for (int j = 0; j < n; j++) rank += ul[j] > l || (ul[j] == l && um[j] < e);
    sm[rank] = e;
    sl[rank] = l;
  }
  __syncthreads();
  {
    // lane r checks ranks r and r+1; the weights one exp per lane
    const double mx = sl[0];
    bool pair = true;
    if (i < w.K && i + 1 < n) {
      const double a = sl[i], b = sl[i + 1];
      pair = a - b > 0x1p-20 * (1.0 + fabs(a) + fabs(b) + 2.0 * fabs(mx));
    }
    bool ok = n >= w.K && __all(pair);
    if (ok) ok = (double)sl[w.K - 1] - mx > -80.0;
    if (ok) {
      const double2 *lb = w.lb + (size_t)t * (w.E + 1);
      const double lmx = lb[sm[0]].x;
      const double ev = i < w.K ? exp(lb[sm[i]].x - lmx) : 0.0;
      const double den = wave_sum(ev);
      if (i < w.K) {
        w.idx[(size_t)t * w.K + i] = sm[i];
        w.w[(size_t)t * w.K + i] = (float)(ev / den);
      }
    } else if (i == 0) {
      atomicAdd(&stats[2], 1ull);
      w.certified[t] = 0;
      w.flist[atomicAdd(w.fcount, 1)] = t;
    }
  }
  __syncthreads();  // the token's LDS is read no more
}

// ---------------------------------------------------------------------------
// 4. exact logits for the tokens the bounds did not certify: the experts of
// the targeted set (certified 2) or every expert (certified 0).  The products
// rn(x*w) are independent of the chain order: the block's lanes form them
// with coalesced loads into LDS, then one lane runs the serial sum over LDS,
// s = rn(s + p_i), and the fused tail.  Same result as exact_chain.
// Blocks walk the list of uncertain tokens (few: most launches find none).
// grid (64, kUncertainSlots), 64 threads, dynamic LDS 4*H bytes.
// ---------------------------------------------------------------------------
constexpr int kUncertainSlots = 128;
__global__ __launch_bounds__(64) void k_exact_logits(Work w, const float *x, const float *router,
                                                     unsigned long long *stats) {
  extern __shared__ float prod[];
  __shared__ int s_last;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    atomicAdd(&stats[0], (unsigned long long)w.T);  // tokens routed, once per step
  const int nu = *w.ucount;
  const int m = (w.H / 8) * 8;
  for (int ui = blockIdx.y; ui < nu; ui += gridDim.y) {
    const int t = w.ulist[ui];
    const int n = w.mcount[t];
    const float *xt = x + (size_t)t * w.H;
    for (int k = blockIdx.x; k < n; k += gridDim.x) {
      const int e = w.mset[(size_t)t * 64 + k];
      const float *row = router + (size_t)e * w.H;
      form_products(xt, row, m, prod);
      __syncthreads();
      if (threadIdx.x == 0) {
        const int m64 = m / 64 * 64;
        float s = serial_sum_lds(prod, m64);
        for (int i = m64; i < m; i++) s = __fadd_rn(s, prod[i]);
        for (int i = m; i < w.H; i++) s = __fmaf_rn(xt[i], row[i], s);
        __hip_atomic_store(&w.logits[(size_t)t * w.E + e], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the block that writes the token's last chain checks it
        s_last = __hip_atomic_fetch_add(&w.udone[t], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
      }
      __syncthreads();
      if (s_last) topk_check_token(w, t, stats);
      __syncthreads();
    }
  }
}

// router_topk (c/qwen.c:3421-3426) on fp32 logits, bit-exact: serial max and
// denominator in expert order, glibc expf, K argmax rounds with strict '>'
// (lowest index on ties, -1 if nothing beats -1), serial renormalisation.
// One block per token; `skip` (may be null) marks certified tokens.
__device__ void topk_exact_block(const float *logit, int E, int K, int *idx, float *weight, float *prob) {
  __shared__ float s_mx, s_den;
  if (threadIdx.x < 64) {
    // the largest logit (its value does not depend on the scan order: +0 and
    // -0 give the same logit - max)
    float mx = -__builtin_huge_valf();
    for (int e = threadIdx.x; e < E; e += 64)
      if (logit[e] > mx) mx = logit[e];
    mx = wave_max_dpp(mx);
    if (threadIdx.x == 0) s_mx = mx;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) prob[e] = expf_glibc(logit[e] - s_mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    // the serial denominator in expert order, its LDS reads run ahead
    const int e64 = E / 64 * 64;
    float den = serial_sum_lds(prob, e64);
    for (int e = e64; e < E; e++) den = __fadd_rn(den, prob[e]);
    s_den = den;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) prob[e] = prob[e] / s_den;
  __syncthreads();
  __shared__ int s_idx[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  if (threadIdx.x < 64) {
    // K argmax rounds by wave 0 over 64-bit keys (probability, order-
    // preserving, then the complemented index: the lowest index among
    // equal values, as the reference's strict '>' in expert order); values
    // not above -1 never qualify
    const int lane = threadIdx.x;
    for (int j = 0; j < K; j++) {
      unsigned long long best = 0ull;
      for (int e = lane; e < E; e += 64) {
        bool used = false;
        for (int p = 0; p < j; p++) used |= s_idx[p] == e;
        const float pv = prob[e];
        const unsigned long long k2 = ((unsigned long long)order_key(pv) << 32) | (unsigned)(~e);
        if (!used && pv > -1.0f && k2 > best) best = k2;
      }
      best = wave_max_u64(best);
      if (lane == 0) {
        const int c = best ? (int)(~(unsigned)best) : -1;
        s_idx[j] = c;
        s_w[j] = c >= 0 ? prob[c] : -1.0f;
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float topden = 0.0f;
    for (int j = 0; j < K; j++) topden += s_w[j];
    for (int j = 0; j < K; j++) {
      idx[j] = s_idx[j];
      weight[j] = s_w[j] / topden;
    }
  }
  __syncthreads();
}

// Every expert's exact logit for the tokens on the full path: one block an
// (expert, token) pair, the products formed with coalesced loads into LDS and
// summed serially by one lane as in k_exact_logits.  The block that writes a
// token's last chain runs router_topk's replica for it.
// grid (min(E, 1024), kFullSlots), 64 threads, dynamic LDS 4*max(H, 2*round4(E)) bytes.
constexpr int kFullSlots = 8;
__global__ __launch_bounds__(64) void k_exact_full(Work w, const float *x, const float *router) {
  extern __shared__ float prod[];  // the products; for the replica, the token's logits and probabilities
  __shared__ int s_last;
  const int nf = *w.fcount;
  const int m = (w.H / 8) * 8;
  for (int fi = blockIdx.y; fi < nf; fi += gridDim.y) {
    const int t = w.flist[fi];
    const float *xt = x + (size_t)t * w.H;
    for (int e = blockIdx.x; e < w.E; e += gridDim.x) {
      const float *row = router + (size_t)e * w.H;
      form_products(xt, row, m, prod);
      __syncthreads();
      if (threadIdx.x == 0) {
        const int m64 = m / 64 * 64;
        float s = serial_sum_lds(prod, m64);
        for (int i = m64; i < m; i++) s = __fadd_rn(s, prod[i]);
        for (int i = m; i < w.H; i++) s = __fmaf_rn(xt[i], row[i], s);
        __hip_atomic_store(&w.logits[(size_t)t * w.E + e], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = __hip_atomic_fetch_add(&w.fdone[t], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == w.E - 1;
      }
      __syncthreads();
      if (s_last) {
        float *lg = prod, *pb = prod + ((w.E + 3) & ~3);  // 16-byte aligned: read as float4
        for (int e2 = threadIdx.x; e2 < w.E; e2 += blockDim.x)
          lg[e2] = __hip_atomic_load(&w.logits[(size_t)t * w.E + e2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        topk_exact_block(lg, w.E, w.K, w.idx + (size_t)t * w.K, w.w + (size_t)t * w.K, pb);
      }
      __syncthreads();
    }
  }
}

__global__ void k_router_topk_logits(const float *logits, int E, int K, int *idx, float *weight) {
  __shared__ __align__(16) float prob[4096];
  int t = blockIdx.x;
  topk_exact_block(logits + (size_t)t * E, E, K, idx + (size_t)t * K, weight + (size_t)t * K, prob);
}

// ---------------------------------------------------------------------------
// 5. bucketing (c/qwen.c:4168 expert order, 3956-3968 token order): a stable
// counting sort through per-expert token bitmaps.  Also emits the routed work
// items {expert, first CSR entry, count <= 8} and pos[t*K+k] (CSR entry of
// route (t,k)).  One block of 1024 threads; tokens_per_step(E) tokens at most (the E x T bit map fits 160 KiB).
// ---------------------------------------------------------------------------
__device__ void bucket_block(const int *idx, int T, int K, int E, int *offsets, int *btok, int *bslot,
                             int *pos, int4 *items, int *nitems, unsigned *bits, int *cnt, int *iofs, int itok) {
  __shared__ int s_dup;  // some token lists an expert twice
  int words = (T + 31) / 32;
  for (int i = threadIdx.x; i < E * words; i += blockDim.x) bits[i] = 0;
  if (threadIdx.x == 0) s_dup = 0;
  __syncthreads();
  for (int r = threadIdx.x; r < T * K; r += blockDim.x) {
    int e = idx[r];
    if (e >= 0 && e < E) {
      const unsigned bit = 1u << ((r / K) & 31);
      if (atomicOr(&bits[e * words + r / K / 32], bit) & bit) s_dup = 1;
    }
  }
  __syncthreads();
  const bool dup = s_dup != 0;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
    for (int q = 0; q < words; q++) c += __popc(bits[e * words + q]);
    cnt[e] = c;
  }
  __syncthreads();
  {  // exclusive scans of the counts and item counts: thread i owns experts [per*i, per*i+per)
    __shared__ int wsum[2][16];
    const int nthr = blockDim.x, per = (E + nthr - 1) / nthr;
    const int e0 = threadIdx.x * per, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int c = 0, ni = 0;
    for (int e = e0; e < e0 + per && e < E; e++) {
      c += cnt[e];
      ni += (cnt[e] + itok - 1) / itok;
    }
    int ic = c, ii = ni;  // inclusive wave scans
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int a = __shfl_up(ic, o, 64), b = __shfl_up(ii, o, 64);
      if (lane >= o) {
        ic += a;
        ii += b;
      }
    }
    if (lane == 63) {
      wsum[0][wave] = ic;
      wsum[1][wave] = ii;
    }
    __syncthreads();
    int bc = 0, bi = 0;
    for (int v = 0; v < wave; v++) {
      bc += wsum[0][v];
      bi += wsum[1][v];
    }
    int acc = bc + ic - c, ia = bi + ii - ni;
    for (int e = e0; e < e0 + per && e < E; e++) {
      offsets[e] = acc;
      iofs[e] = ia;
      acc += cnt[e];
      ia += (cnt[e] + itok - 1) / itok;
    }
    if (e0 < E && e0 + per >= E) {  // the thread owning the last expert
      offsets[E] = acc;
      iofs[E] = ia;
      *nitems = ia;
    }
  }
  __syncthreads();
  for (int r = threadIdx.x; r < T * K; r += blockDim.x) {
    int e = idx[r], t = r / K, k = r % K;
    if (e < 0 || e >= E) {
      pos[r] = -1;
      continue;
    }
    // the reference's gather takes the first matching k of a token (only a
    // step with a repeated expert in some token's list needs the check)
    bool first = true;
    if (dup)
      for (int k2 = 0; k2 < k; k2++) first &= idx[t * K + k2] != e;
    if (!first) {
      pos[r] = -1;
      continue;
    }
    const unsigned *b = bits + e * words;
    int rank = 0;
    for (int q = 0; q < t / 32; q++) rank += __popc(b[q]);
    rank += __popc(b[t / 32] & ((1u << (t & 31)) - 1u));
    int p = offsets[e] + rank;
    btok[p] = t;
    bslot[p] = k;
    pos[r] = p;
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int n = cnt[e];
    for (int i = 0, it = iofs[e]; i < n; i += itok, it++) items[it] = make_int4(e, offsets[e] + i, min(itok, n - i), 0);
  }
}

__device__ __forceinline__ void bucket_step(Work &w, unsigned *smem) {
  int words = (w.T + 31) / 32;
  unsigned *bits = smem;
  int *cnt = (int *)(smem + w.E * words);
  int *iofs = cnt + w.E;
  bucket_block(w.idx, w.T, w.K, w.E, w.offsets, w.btok, w.bslot, w.pos, w.items, w.nitems, bits, cnt, iofs,
               w.itok);
}

__global__ void k_bucket(Work w) {
  extern __shared__ unsigned smem[];
  bucket_step(w, smem);
}

__global__ void k_bucket_only(const int *idx, int T, int K, int E, int *offsets, int *btok, int *bslot,
                              int *pos, int4 *items, int *nitems) {
  extern __shared__ unsigned smem[];
  int words = (T + 31) / 32;
  unsigned *bits = smem;
  int *cnt = (int *)(smem + E * words);
  int *iofs = cnt + E;
  bucket_block(idx, T, K, E, offsets, btok, bslot, pos, items, nitems, bits, cnt, iofs, kMaxTokensPerItem);
}

// ---------------------------------------------------------------------------
// Tile unpacking: a lane's codes of one tile-group (16 bytes int4, 12 bytes
// int3) become the two int8 MFMA A operands (group positions kb*16+[0,16) and
// 64+kb*16+[0,16) of row lane%16), codes unsigned.
// ---------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ void unpack_words(const uint32_t *q, v4i &a0, v4i &a1) {
  uint32_t d[8];
  if (FMT == 4) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      d[2 * i] = q[i] & 0x0F0F0F0Fu;
      d[2 * i + 1] = (q[i] >> 4) & 0x0F0F0F0Fu;
    }
  } else {
    uint32_t L0 = q[0], L1 = q[1], H = q[2];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t L = j < 4 ? L0 : L1;
      uint32_t lo = (L >> (2 * (j & 3))) & 0x03030303u;
      uint32_t hi = j <= 2 ? (H << (2 - j)) : (H >> (j - 2));
      d[j] = lo | (hi & 0x04040404u);
    }
  }
  a0 = v4i{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
  a1 = v4i{(int)d[4], (int)d[5], (int)d[6], (int)d[7]};
}

template <int FMT>
__device__ __forceinline__ void load_words(const unsigned char *tp, uint32_t *q) {
  if (FMT == 4) {
    uint4 v = *(const uint4 *)tp;
    q[0] = v.x;
    q[1] = v.y;
    q[2] = v.z;
    q[3] = v.w;
  } else {
    const uint32_t *p = (const uint32_t *)tp;
    q[0] = p[0];
    q[1] = p[1];
    q[2] = p[2];
  }
}

template <int FMT>
__device__ __forceinline__ void unpack_tile(const unsigned char *tp, v4i &a0, v4i &a1) {
  uint32_t q[4];
  load_words<FMT>(tp, q);
  unpack_words<FMT>(q, a0, a1);
}

// Routed tile GEMV on int8 MFMA for up to 8 tokens: the loads of kMtBatch
// consecutive groups (codes, row scales, token digits and digit parameters)
// are issued together ahead of their MFMAs, so a wave has a batch of HBM
// reads in flight.  Per group: two MFMAs give the exact int32 dots of the
// codes with both digits of each token (B column c = lane%16: token c/2,
// digit c%2); f = (dot - OFF*digit sum) * digit scale, the two digit columns
// are added across lanes, and acc += f * row scale.  Results sit in the odd
// lanes of each 16-lane row group.
constexpr int kMtBatch = 4;
template <int FMT>
struct MtTiles {
  uint32_t q[kMtBatch][FMT == 4 ? 4 : 3];
  float4 sc[kMtBatch];
};
struct MtDigits {
  v4i b0[kMtBatch], b1[kMtBatch];
  float dsc[kMtBatch];
  int Q[kMtBatch];
};

template <int FMT>
__device__ __forceinline__ void mt_load(MtTiles<FMT> &t, const TileMat &mat, size_t tg0, int n, int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < kMtBatch; i++)
    if (i < n) {
      load_words<FMT>(tm_codes(mat, tg0 + i) + lane * BPL, t.q[i]);
      t.sc[i] = *(const float4 *)(tm_scales(mat, tg0 + i) + 4 * kb);
    }
}

__device__ __forceinline__ void mt_digits(MtDigits &d, const signed char *dsrc, const float4 *gpsrc, int g0, int n,
                                          int lane) {
  const int kb = lane >> 4;
  const bool second = lane & 1;
#pragma unroll
  for (int i = 0; i < kMtBatch; i++)
    if (i < n) {
      const int g = g0 + i;
      d.b0[i] = v4i{0, 0, 0, 0};
      d.b1[i] = v4i{0, 0, 0, 0};
      d.dsc[i] = 0.0f;
      d.Q[i] = 0;
      if (dsrc) {
        d.b0[i] = *(const v4i *)(dsrc + g * kGroup + kb * 16);
        d.b1[i] = *(const v4i *)(dsrc + g * kGroup + 64 + kb * 16);
      }
      if (gpsrc) {
        float4 p = gpsrc[g];
        d.dsc[i] = second ? p.y : p.x;
        d.Q[i] = __float_as_int(second ? p.w : p.z);
      }
    }
}

// kMtBatch tile-groups of one group column g in consecutive row tiles
// (tile-group stride ng), for the down projection, whose waves split groups.
template <int FMT>
__device__ __forceinline__ void mt_load_rows(MtTiles<FMT> &t, const TileMat &mat, size_t tg0, int ng, int n,
                                             int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < kMtBatch; i++)
    if (i < n) {
      load_words<FMT>(tm_codes(mat, tg0 + (size_t)i * ng) + lane * BPL, t.q[i]);
      t.sc[i] = *(const float4 *)(tm_scales(mat, tg0 + (size_t)i * ng) + 4 * kb);
    }
}

// mt_compute for tiles of one group (digits d slot 0) in kMtBatch row tiles:
// acc[i] of row tile i.
template <int FMT>
__device__ __forceinline__ void mt_compute_rows(const MtTiles<FMT> &t, const MtDigits &d, int n,
                                                float acc[kMtBatch][4]) {
  constexpr int OFF = FMT == 4 ? 8 : 4;
#pragma unroll
  for (int i = 0; i < kMtBatch; i++)
    if (i < n) {
      v4i a0, a1;
      unpack_words<FMT>(t.q[i], a0, a1);
      v4i c = {0, 0, 0, 0};
      c = mfma_i8(a0, d.b0[0], c);
      c = mfma_i8(a1, d.b1[0], c);
      const float scv[4] = {t.sc[i].x, t.sc[i].y, t.sc[i].z, t.sc[i].w};
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float f = (float)(c[r] - OFF * d.Q[0]) * d.dsc[0];
        float tsum = f + dpp_row_shr1(f);
        acc[i][r] = __builtin_fmaf(tsum, scv[r], acc[i][r]);
      }
    }
}

template <int FMT>
__device__ __forceinline__ void mt_compute(const MtTiles<FMT> &t, const MtDigits &d, int n, float acc[4]) {
  constexpr int OFF = FMT == 4 ? 8 : 4;
#pragma unroll
  for (int i = 0; i < kMtBatch; i++)
    if (i < n) {
      v4i a0, a1;
      unpack_words<FMT>(t.q[i], a0, a1);
      v4i c = {0, 0, 0, 0};
      c = mfma_i8(a0, d.b0[i], c);
      c = mfma_i8(a1, d.b1[i], c);
      const float scv[4] = {t.sc[i].x, t.sc[i].y, t.sc[i].z, t.sc[i].w};
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float f = (float)(c[r] - OFF * d.Q[i]) * d.dsc[i];
        float tsum = f + dpp_row_shr1(f);
        acc[r] = __builtin_fmaf(tsum, scv[r], acc[r]);
      }
    }
}

// ---------------------------------------------------------------------------
// 6. shared expert gate/up, IDOT on MFMA: exact int32 dots for 16 rows x
// 16*NS tokens, k split over the block's waves, then h = silu(g)*u with the
// reference's rounding.  grid (Ish/16, ceil(T/(16 NS))), 256 threads; steps
// of at most kShSplitTokens tokens take k_shared_gu_split instead.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void idot_tile(const signed char *W, int ld, int row0, int kc0, int kc1,
                                          const signed char *xq, int xld, int t0, int T, v4i &c, int lane) {
  const int r = lane & 15, kb = lane >> 4;
  const signed char *arow = W + (size_t)(row0 + r) * ld + kb * 16;
  int tok = t0 + r;  // B column = lane%16 = token
  const signed char *brow = tok < T ? xq + (size_t)tok * xld + kb * 16 : nullptr;
  for (int kc = kc0; kc < kc1; kc++) {
    v4i a = *(const v4i *)(arow + kc * 64);
    v4i b = {0, 0, 0, 0};
    if (brow) b = *(const v4i *)(brow + kc * 64);
    c = mfma_i8(a, b, c);
  }
}

// idot_tile for NS consecutive 16-token chunks sharing each A load: c[s]
// holds tokens t0 + 16 s + lane % 16 (exact int32 sums, like idot_tile)
template <int NS>
__device__ __forceinline__ void idot_tiles(const signed char *W, int ld, int row0, int kc0, int kc1,
                                           const signed char *xq, int xld, int t0, int T, v4i c[NS], int lane) {
  const int r = lane & 15, kb = lane >> 4;
  const signed char *arow = W + (size_t)(row0 + r) * ld + kb * 16;
  const signed char *brow[NS];
#pragma unroll
  for (int q = 0; q < NS; q++) {
    const int tok = t0 + 16 * q + r;
    brow[q] = tok < T ? xq + (size_t)tok * xld + kb * 16 : nullptr;
  }
  for (int kc = kc0; kc < kc1; kc++) {
    const v4i a = *(const v4i *)(arow + kc * 64);
#pragma unroll
    for (int q = 0; q < NS; q++) {
      v4i b = {0, 0, 0, 0};
      if (brow[q]) b = *(const v4i *)(brow[q] + kc * 64);
      c[q] = mfma_i8(a, b, c[q]);
    }
  }
}

// Shared expert steps of many tokens: blocks take NS 16-token chunks (1, 2
// or 4 by the step's size), so each shared weight tile is read once per
// 16*NS tokens.  The shared-down part of the down kernels takes
// kSharedBlockTokens tokens a block.
// k chunks per batch: a wave issues the gate, up and activation loads of
// kShBatch chunks before the first MFMA, so a wave's k range costs
// per/kShBatch memory latencies instead of 2*per
constexpr int kShBatch = 4;

__device__ __forceinline__ v4i ld_v4i_if(const signed char *p, bool ok) {
  v4i v = {0, 0, 0, 0};
  if (ok) v = *(const v4i *)p;
  return v;
}

template <int NS>
__global__ __launch_bounds__(256) void k_shared_swiglu(Work w, const signed char *gq, const float *gs,
                                                       const signed char *uq, const float *us) {
  __shared__ int part[4][2][NS][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rt = blockIdx.x, t0 = blockIdx.y * 16 * NS;
  const int nk = w.H / 64;
  const int per = (nk + 3) / 4, kc0 = wave * per, kc1 = min(nk, kc0 + per);
  v4i cg[NS] = {}, cu[NS] = {};
  {
    const int r = lane & 15, kb = lane >> 4;
    const signed char *ga = gq + (size_t)(rt * kTileRows + r) * w.H + kb * 16;
    const signed char *ua = uq + (size_t)(rt * kTileRows + r) * w.H + kb * 16;
    const signed char *brow[NS];
    bool bok[NS];
#pragma unroll
    for (int q = 0; q < NS; q++) {
      const int tok = t0 + 16 * q + r;
      bok[q] = tok < w.T;
      brow[q] = w.xq + (size_t)(bok[q] ? tok : 0) * w.H + kb * 16;
    }
    for (int kc = kc0; kc < kc1; kc += kShBatch) {
      v4i ag[kShBatch], au[kShBatch], bb[kShBatch][NS];
#pragma unroll
      for (int u = 0; u < kShBatch; u++) {
        const bool ok = kc + u < kc1;
        const int k = ok ? kc + u : kc0;  // in bounds; the operand is zeroed
        ag[u] = ld_v4i_if(ga + k * 64, ok);
        au[u] = ld_v4i_if(ua + k * 64, ok);
#pragma unroll
        for (int q = 0; q < NS; q++) bb[u][q] = ld_v4i_if(brow[q] + k * 64, ok && bok[q]);
      }
#pragma unroll
      for (int u = 0; u < kShBatch; u++)
#pragma unroll
        for (int q = 0; q < NS; q++) {
          cg[q] = mfma_i8(ag[u], bb[u][q], cg[q]);
          cu[q] = mfma_i8(au[u], bb[u][q], cu[q]);
        }
    }
  }
#pragma unroll
  for (int q = 0; q < NS; q++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      part[wave][0][q][lane * 4 + i] = cg[q][i];
      part[wave][1][q][lane * 4 + i] = cu[q][i];
    }
  __syncthreads();
  // wave q finishes chunk q: the waves' k-range sums (exact), then the
  // reference's rounding of g, u and h
  const int q = wave;
  if (q >= NS) return;
  const int kb = lane >> 4, tok = t0 + 16 * q + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int dg = 0, du = 0;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      dg += part[v][0][q][lane * 4 + i];
      du += part[v][1][q][lane * 4 + i];
    }
    const int row = rt * kTileRows + 4 * kb + i;
    if (tok < w.T) {
      const float sx = w.sx[tok];
      const float g = (float)dg * gs[row] * sx;
      const float u = (float)du * us[row] * sx;
      w.hsh[(size_t)tok * w.Ish + row] = silu_ref(g) * u;
    }
  }
}

// Shared gate/up of small steps (T <= kShSplitTokens, 64: at S397 the split
// halves the stage at 64 tokens and costs 4 us at 512): block (row tile, k
// part ks, token block z) forms the exact int32 dots of its 16 rows over k
// chunks [ks*nk/kShSplit, (ks+1)*nk/kShSplit) for NS 16-token chunks from
// token 16*NS*z, 4 waves splitting the part, and stores them to shpart[ks];
// k_prep_hidden adds the parts (exact) and applies the reference's rounding.
// grid (Ish/16, kShSplit, ceil(T/(16 NS))), 256 threads.
template <int NS>
__device__ __forceinline__ void shared_gu_tile(Work &w, const signed char *gq, const signed char *uq, int rt, int ks,
                                               int bz, int (*part)[2][NS][256]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = bz * 16 * NS;
  const int nk = w.H / 64;
  const int p0 = ks * nk / kShSplit, p1 = (ks + 1) * nk / kShSplit;
  const int kc0 = p0 + wave * (p1 - p0) / 4, kc1 = p0 + (wave + 1) * (p1 - p0) / 4;
  v4i cg[NS] = {}, cu[NS] = {};
  {
    const int r = lane & 15, kb = lane >> 4;
    const signed char *ga = gq + (size_t)(rt * kTileRows + r) * w.H + kb * 16;
    const signed char *ua = uq + (size_t)(rt * kTileRows + r) * w.H + kb * 16;
    const signed char *brow[NS];
    bool bok[NS];
#pragma unroll
    for (int q = 0; q < NS; q++) {
      const int tok = t0 + 16 * q + r;
      bok[q] = tok < w.T;
      brow[q] = w.xq + (size_t)(bok[q] ? tok : 0) * w.H + kb * 16;
    }
    for (int kc = kc0; kc < kc1; kc += kShBatch) {
      v4i ag[kShBatch], au[kShBatch], bb[kShBatch][NS];
#pragma unroll
      for (int u = 0; u < kShBatch; u++) {
        const bool ok = kc + u < kc1;
        const int k = ok ? kc + u : kc0;  // in bounds; the operand is zeroed
        ag[u] = ld_v4i_if(ga + k * 64, ok);
        au[u] = ld_v4i_if(ua + k * 64, ok);
#pragma unroll
        for (int q = 0; q < NS; q++) bb[u][q] = ld_v4i_if(brow[q] + k * 64, ok && bok[q]);
      }
#pragma unroll
      for (int u = 0; u < kShBatch; u++)
#pragma unroll
        for (int q = 0; q < NS; q++) {
          cg[q] = mfma_i8(ag[u], bb[u][q], cg[q]);
          cu[q] = mfma_i8(au[u], bb[u][q], cu[q]);
        }
    }
  }
#pragma unroll
  for (int q = 0; q < NS; q++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      part[wave][0][q][lane * 4 + i] = cg[q][i];
      part[wave][1][q][lane * 4 + i] = cu[q][i];
    }
  __syncthreads();
  const int q = wave;
  if (q >= NS) return;
  const int kb = lane >> 4, tok = t0 + 16 * q + (lane & 15);
  if (tok >= w.T) return;
  int *dst = w.shpart + ((size_t)ks * w.T + tok) * 2 * w.Ish;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int dg = 0, du = 0;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      dg += part[v][0][q][lane * 4 + i];
      du += part[v][1][q][lane * 4 + i];
    }
    const int row = rt * kTileRows + 4 * kb + i;
    dst[row] = dg;
    dst[w.Ish + row] = du;
  }
}

template <int NS>
__global__ __launch_bounds__(256) void k_shared_gu_split(Work w, const signed char *gq, const signed char *uq) {
  __shared__ int part[4][2][NS][256];
  shared_gu_tile<NS>(w, gq, uq, blockIdx.x, blockIdx.y, blockIdx.z, part);
}

// The bucketing (block 0, dispatched first: the routed kernels wait for it)
// and the shared gate/up tiles of k_shared_gu_split (the other blocks, linear
// over (row tile, k part, token block)) in one launch: neither reads the
// other's results, and a launch boundary costs more than the bucketing's
// block.  256 threads, dynamic LDS max(bucket_lds_bytes, 32 * 256 * NS).
template <int NS>
__global__ __launch_bounds__(256) void k_bucket_shared(Work w, const signed char *gq, const signed char *uq) {
  extern __shared__ unsigned bs_dyn[];
  if (blockIdx.x == 0) {
    bucket_step(w, bs_dyn);
    return;
  }
  const int b = blockIdx.x - 1, nrt = w.Ish / kTileRows;
  shared_gu_tile<NS>(w, gq, uq, b % nrt, (b / nrt) % kShSplit, b / (nrt * kShSplit), (int(*)[2][NS][256])bs_dyn);
}

// qrow_i8 of the shared hidden rows + digits of the routed hidden rows
// Token b's shared hidden row: the k parts of the split shared gate/up dots
// (exact int32 sums) and h = silu(g)*u with the reference's rounding (as
// k_shared_swiglu) when the step split them, then qrow_i8 of the row (hq,
// shx).  By one block of any size.
__device__ void prep_shared_hidden(Work &w, const float *gs, const float *us, int b, float *red) {
    if (w.shks > 0) {
      // the k parts of the shared gate/up dots (exact int32 sums), then
      // h = silu(g)*u with the reference's rounding (as k_shared_swiglu)
      // (every part's loads issued before the first add)
      constexpr int kRows = 4;  // rows per thread per batch
      const float sx = w.sx[b];
      for (int i0 = threadIdx.x; i0 < w.Ish; i0 += kRows * blockDim.x) {
        int pg[kRows][kShSplit], pu[kRows][kShSplit];
        float gsi[kRows], usi[kRows];
#pragma unroll
        for (int j = 0; j < kRows; j++) {
          const int i = min(i0 + j * (int)blockDim.x, w.Ish - 1);  // in bounds; stored only below Ish
#pragma unroll
          for (int ks = 0; ks < kShSplit; ks++) {
            const int *src = w.shpart + ((size_t)ks * w.T + b) * 2 * w.Ish;
            pg[j][ks] = src[i];
            pu[j][ks] = src[w.Ish + i];
          }
          gsi[j] = gs[i];
          usi[j] = us[i];
        }
#pragma unroll
        for (int j = 0; j < kRows; j++) {
          const int i = i0 + j * (int)blockDim.x;
          int dg = 0, du = 0;
#pragma unroll
          for (int ks = 0; ks < kShSplit; ks++) {
            dg += pg[j][ks];
            du += pu[j][ks];
          }
          const float g = (float)dg * gsi[j] * sx;
          const float u = (float)du * usi[j] * sx;
          if (i < w.Ish) w.hsh[(size_t)b * w.Ish + i] = silu_ref(g) * u;
        }
      }
      __syncthreads();
    }
    float s = qrow_i8_block(w.hsh + (size_t)b * w.Ish, w.Ish, w.hq + (size_t)b * w.Ish, red);
    if (threadIdx.x == 0) w.shx[b] = s;
}

__global__ void k_prep_hidden(Work w, const float *gs, const float *us) {
  __shared__ float red[16];
  int b = blockIdx.x;
  if (b < w.T) {
    prep_shared_hidden(w, gs, us, b, red);
    return;
  }
  int p = b - w.T;
  if (p >= w.offsets[w.E]) return;
  quantize_digits(w.hroute + (size_t)p * w.I, w.I, w.ngi, w.hd1 + (size_t)p * w.Ip, w.hd2 + (size_t)p * w.Ip,
                  w.hgp + (size_t)p * w.ngi);
}

// Workgroup barrier for LDS traffic only: __syncthreads() would also wait for
// the next row tile's loads, which are meant to stay in flight across it.
__device__ __forceinline__ void lds_only_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// h = silu(g)*u for one row tile of an item from the 8 waves' partial sums.
__device__ __forceinline__ void gu_store(float (*part)[2][64][4], const float ag[4], const float au[4], int rt,
                                         int p0, int cnt, const Work &w, int lane, int wave) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    part[wave][0][lane][i] = ag[i];
    part[wave][1][lane][i] = au[i];
  }
  lds_only_barrier();
  if (wave == 0 && (lane & 1) && ((lane & 15) >> 1) < cnt) {
    int tt = (lane & 15) >> 1, kb = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float g = part[0][0][lane][i], u = part[0][1][lane][i];
      for (int v = 1; v < 8; v++) {
        g += part[v][0][lane][i];
        u += part[v][1][lane][i];
      }
      int row = rt * kTileRows + 4 * kb + i;
      w.hroute[(size_t)(p0 + tt) * w.I + row] = silu_ref(g) * u;
    }
  }
  lds_only_barrier();
}

// ---------------------------------------------------------------------------
// 7. routed gate/up: item = (expert, <=8 tokens) x kGuRowTiles row tiles; 8
// waves split the H groups.  A wave loads its groups' token digits once per
// item and keeps the next row tile's gate and up tiles in flight while it
// computes the current one; then h = silu(g)*u per token.
// grid (ceil(I/16/kGuRowTiles), min(items bound, 1024)), 512 threads.
// ---------------------------------------------------------------------------
// Row tiles per block: 8, or 4 for small steps (T*K <= 64), where few items
// leave the device short of blocks (measured at S397: 4 is faster at B = 4,
// 8 at B = 32 and T = 512).
constexpr int kGuRowTiles = 8, kGuRowTilesSmall = 4;
template <int FMT, bool WIDE>
__global__ __launch_bounds__(512) void k_expert_gateup(Work w, ExpertLayout xl, int row_tiles) {
  __shared__ float part[8][2][64][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nrt = w.I / kTileRows;
  const int rt0 = blockIdx.x * row_tiles, rt1 = min(nrt, rt0 + row_tiles);
  const int per = (w.ngh + 7) / 8, g0 = min(w.ngh, wave * per), g1 = min(w.ngh, g0 + per);
  const int n = g1 - g0;
  int n_items = *w.nitems;
  for (int it = blockIdx.y; it < n_items; it += gridDim.y) {
    int4 item = w.items[it];
    int e = item.x, p0 = item.y, cnt = item.z;
    // B column c = lane%16: token c/2 of the item, digit c%2
    const int tt = (lane & 15) >> 1;
    const signed char *dsrc = nullptr;
    const float4 *gp = nullptr;
    if (tt < cnt) {
      const int tok = w.btok[p0 + tt];
      dsrc = ((lane & 1) ? w.xd2 : w.xd1) + (size_t)tok * w.Hp;
      gp = w.xgp + (size_t)tok * w.ngh;
    }
    const TileMat mg = xl.mat(e, 0), mu = xl.mat(e, 1);
    if constexpr (!WIDE) {  // n <= kMtBatch
      // pipeline over (row tile, matrix): the up tiles of rt load while its
      // gate tiles are multiplied, the gate tiles of rt+1 while its up tiles are
      MtDigits dg;
      MtTiles<FMT> tg, tu;
      if (n > 0) {
        mt_digits(dg, dsrc, gp, g0, n, lane);
        mt_load<FMT>(tg, mg, (size_t)rt0 * w.ngh + g0, n, lane);
      }
      for (int rt = rt0; rt < rt1; rt++) {
        float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0};
        if (n > 0) {
          mt_load<FMT>(tu, mu, (size_t)rt * w.ngh + g0, n, lane);
          mt_compute<FMT>(tg, dg, n, ag);
          if (rt + 1 < rt1) mt_load<FMT>(tg, mg, (size_t)(rt + 1) * w.ngh + g0, n, lane);
          mt_compute<FMT>(tu, dg, n, au);
        }
        gu_store(part, ag, au, rt, p0, cnt, w, lane, wave);
      }
    } else {  // more than kMtBatch groups per wave (H > 4096): batches in turn, no prefetch
      for (int rt = rt0; rt < rt1; rt++) {
        float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0};
        for (int g = g0; g < g1; g += kMtBatch) {
          const int m = min(kMtBatch, g1 - g);
          MtTiles<FMT> tg, tu;
          MtDigits dg;
          mt_load<FMT>(tg, mg, (size_t)rt * w.ngh + g, m, lane);
          mt_load<FMT>(tu, mu, (size_t)rt * w.ngh + g, m, lane);
          mt_digits(dg, dsrc, gp, g, m, lane);
          mt_compute<FMT>(tg, dg, m, ag);
          mt_compute<FMT>(tu, dg, m, au);
        }
        gu_store(part, ag, au, rt, p0, cnt, w, lane, wave);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 7b. routed gate/up of items of <= 8 tokens with the weights streamed through
// LDS: each wave copies its groups' records (gate and up codes and row scales
// of one (row tile, group), contiguous in HBM) for the block's row tiles into
// a ring of kGuRing slots with global_load_lds in 1 KB pieces, kGuRing-1
// records in flight while one is multiplied.  Same arithmetic and order as
// k_expert_gateup (H <= 4096: a wave's groups fit one batch).
// grid (ceil(I/16/row_tiles), item slots), 512 threads, dynamic LDS
// 8*kGuRing*record bytes.
// ---------------------------------------------------------------------------
#ifndef SW_GU_RING
#define SW_GU_RING 4
#endif
#ifndef SW_GU_USE_RING
#define SW_GU_USE_RING 1
#endif
constexpr int kGuRing = SW_GU_RING;
static_assert(3 * (kGuRing - 1) <= 30, "gate/up ring: waits within wait_vm's range");

template <int FMT>
__global__ __launch_bounds__(512) void k_gateup_ring(Work w, ExpertLayout xl, int row_tiles) {
  extern __shared__ __align__(16) unsigned char glds[];
  __shared__ float part[8][2][64][4];
  constexpr int BPL = FMT == 4 ? 16 : 12;
  constexpr int OFF = FMT == 4 ? 8 : 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kb = lane >> 4;
  const int nrt = w.I / kTileRows;
  const int rt0 = blockIdx.x * row_tiles, rt1 = min(nrt, rt0 + row_tiles);
  const int per = (w.ngh + 7) / 8, g0 = min(w.ngh, wave * per), g1 = min(w.ngh, g0 + per);
  const int n = g1 - g0;  // <= kMtBatch
  const unsigned tgc = xl.tgc, rec = xl.rec_gu();
  const int nck = (int)((rec + 1023) >> 10);
  unsigned char *ring = glds + (size_t)wave * kGuRing * rec;
  const int nit = n > 0 ? (rt1 - rt0) * n : 0;
  const int n_items = *w.nitems;
  for (int it = blockIdx.y; it < n_items; it += gridDim.y) {
    const int4 item = w.items[it];
    const int e = item.x, p0 = item.y, cnt = item.z;
    // this wave's records in order: row tile rt0 + j / n, group g0 + j % n
    const unsigned char *xb = xl.base + (size_t)e * xl.expert_bytes + ((size_t)rt0 * w.ngh + g0) * rec;
    int issued = 0, consumed = 0, su = 0, csl = 0, ir = 0, ig = 0;
    auto issue = [&]() {
      if (issued == nit) return;
      const unsigned char *src = xb + ((size_t)ir * w.ngh + ig) * rec;
      const unsigned slot = lds_addr(ring + (size_t)su * rec);
      for (int k = 0; k < nck; k++)
        if (16 * lane < (int)rec - 1024 * k) dma_b128_s(src + 1024 * k, 16 * lane, slot + 1024 * k);
      issued++;
      if (++su == kGuRing) su = 0;
      if (++ig == n) {
        ig = 0;
        ir++;
      }
    };
    for (int k = 0; k < kGuRing - 1; k++) issue();
    // B column c = lane%16: token c/2 of the item, digit c%2 (loaded behind
    // the first copies; the first record's wait covers them)
    const int tt = (lane & 15) >> 1;
    const signed char *dsrc = nullptr;
    const float4 *gp = nullptr;
    if (tt < cnt) {
      const int tok = w.btok[p0 + tt];
      dsrc = ((lane & 1) ? w.xd2 : w.xd1) + (size_t)tok * w.Hp;
      gp = w.xgp + (size_t)tok * w.ngh;
    }
    MtDigits dg;
    if (n > 0) mt_digits(dg, dsrc, gp, g0, n, lane);
    for (int rt = rt0; rt < rt1; rt++) {
      float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0};
#pragma unroll
      for (int gi = 0; gi < kMtBatch; gi++)
        if (gi < n) {
          issue();
          // this record's copies are done once at most the copies of the
          // records issued after it are outstanding (in order)
          wait_vm(nck * (issued - consumed - 1));
          consumed++;
          const unsigned char *r = ring + (size_t)csl * rec;
          if (++csl == kGuRing) csl = 0;
#pragma unroll
          for (int m = 0; m < 2; m++) {
            uint32_t q[BPL / 4];
            const unsigned *cp = (const unsigned *)(r + m * tgc + lane * BPL);
#pragma unroll
            for (int k = 0; k < BPL / 4; k++) q[k] = cp[k];
            const float4 sc = *(const float4 *)(r + 2 * tgc + 64 * m + 16 * kb);
            v4i a0, a1;
            unpack_words<FMT>(q, a0, a1);
            v4i c = {0, 0, 0, 0};
            c = mfma_i8(a0, dg.b0[gi], c);
            c = mfma_i8(a1, dg.b1[gi], c);
            const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
            float *acc = m == 0 ? ag : au;
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
              const float f = (float)(c[rr] - OFF * dg.Q[gi]) * dg.dsc[gi];
              const float tsum = f + dpp_row_shr1(f);
              acc[rr] = __builtin_fmaf(tsum, scv[rr], acc[rr]);
            }
          }
        }
      gu_store(part, ag, au, rt, p0, cnt, w, lane, wave);
    }
  }
}

// ---------------------------------------------------------------------------
// 8. down: routed items -> rout[p][row]; shared token chunks (IDOT) ->
// shout[t][row].  Each wave takes kDnRowTiles consecutive row tiles.
// grid (ceil(H/16/(4*kDnRowTiles)), n_item_slots + ceil(T/16)), 256 threads.
// ---------------------------------------------------------------------------
#ifndef SW_DN_ROW_TILES
#define SW_DN_ROW_TILES 1
#endif
constexpr int kDnRowTiles = SW_DN_ROW_TILES;  // row tiles per wave
template <int FMT>
__global__ __launch_bounds__(256) void k_down(Work w, ExpertLayout xl, int item_slots, const signed char *dq,
                                              const float *ds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kb = lane >> 4;
  const int nrt = w.H / kTileRows;
  const int rt0 = min(nrt, (blockIdx.x * 4 + wave) * kDnRowTiles), rt1 = min(nrt, rt0 + kDnRowTiles);
  if ((int)blockIdx.y >= item_slots) {
    int t0 = ((int)blockIdx.y - item_slots) * kSharedTokens;
    int tok = t0 + (lane & 15);
    for (int rt = rt0; rt < rt1; rt++) {
      v4i c = {0, 0, 0, 0};
      idot_tile(dq, w.Ish, rt * kTileRows, 0, w.Ish / 64, w.hq, w.Ish, t0, w.T, c, lane);
      if (tok < w.T) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          int row = rt * kTileRows + 4 * kb + i;
          w.shout[(size_t)tok * w.H + row] = (float)c[i] * ds[row] * w.shx[tok];
        }
      }
    }
    return;
  }
  // the wave's units (row tile, batch of groups) in order; unit u+1's tiles
  // and digits load while unit u is multiplied
  const int nb = (w.ngi + kMtBatch - 1) / kMtBatch;
  const int units = (rt1 - rt0) * nb;
  int n_items = *w.nitems;
  for (int it = blockIdx.y; it < n_items; it += item_slots) {
    int4 item = w.items[it];
    int e = item.x, p0 = item.y, cnt = item.z;
    const int tt = (lane & 15) >> 1;
    const signed char *dsrc = nullptr;
    const float4 *gp = nullptr;
    if (tt < cnt) {
      dsrc = ((lane & 1) ? w.hd2 : w.hd1) + (size_t)(p0 + tt) * w.Ip;
      gp = w.hgp + (size_t)(p0 + tt) * w.ngi;
    }
    const TileMat md = xl.mat(e, 2);
    auto unit_load = [&](MtTiles<FMT> &t, MtDigits &d, int u) {
      const int rt = rt0 + u / nb, g = (u % nb) * kMtBatch, n = min(kMtBatch, w.ngi - g);
      mt_load<FMT>(t, md, (size_t)rt * w.ngi + g, n, lane);
      mt_digits(d, dsrc, gp, g, n, lane);
    };
    float acc[4] = {0, 0, 0, 0};
    auto unit_compute = [&](const MtTiles<FMT> &t, const MtDigits &d, int u) {
      const int rt = rt0 + u / nb, b = u % nb, g = b * kMtBatch, n = min(kMtBatch, w.ngi - g);
      if (b == 0) acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
      mt_compute<FMT>(t, d, n, acc);
      if (b == nb - 1 && (lane & 1) && tt < cnt) {
#pragma unroll
        for (int i = 0; i < 4; i++) w.rout[(size_t)(p0 + tt) * w.H + rt * kTileRows + 4 * kb + i] = acc[i];
      }
    };
    MtTiles<FMT> ta, tb;
    MtDigits da, db;
    if (units > 0) unit_load(ta, da, 0);
    for (int u = 0; u < units; u += 2) {
      if (u + 1 < units) unit_load(tb, db, u + 1);
      unit_compute(ta, da, u);
      if (u + 1 >= units) break;
      if (u + 2 < units) unit_load(ta, da, u + 2);
      unit_compute(tb, db, u + 1);
    }
  }
}

// ---------------------------------------------------------------------------
// 8b. down for I <= 1024 (at most 8 groups): 8 waves split the groups (wave w
// takes group w) over kDnBlockRows row tiles of an item, kMtBatch row tiles
// per batch, the next batch's tiles in flight while the current one
// multiplies; the waves' partial sums meet in LDS.  Shared token chunks
// (IDOT) in extra blocks, waves taking row tiles.
// grid (ceil(H/16/kDnBlockRows), n_item_slots + ceil(T/16)), 512 threads.
// ---------------------------------------------------------------------------
constexpr int kDnBlockRows = 16;
template <int FMT>
__global__ __launch_bounds__(512) void k_down_split(Work w, ExpertLayout xl, int item_slots, const signed char *dq,
                                                    const float *ds) {
  __shared__ float part[8][kMtBatch][64][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kb = lane >> 4;
  const int nrt = w.H / kTileRows;
  const int rt0 = blockIdx.x * kDnBlockRows, rt1 = min(nrt, rt0 + kDnBlockRows);
  if ((int)blockIdx.y >= item_slots) {
    int t0 = ((int)blockIdx.y - item_slots) * kSharedTokens;
    int tok = t0 + (lane & 15);
    for (int rt = rt0 + wave; rt < rt1; rt += 8) {
      v4i c = {0, 0, 0, 0};
      idot_tile(dq, w.Ish, rt * kTileRows, 0, w.Ish / 64, w.hq, w.Ish, t0, w.T, c, lane);
      if (tok < w.T) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          int row = rt * kTileRows + 4 * kb + i;
          w.shout[(size_t)tok * w.H + row] = (float)c[i] * ds[row] * w.shx[tok];
        }
      }
    }
    return;
  }
  const bool has = wave < w.ngi;
  const int g = wave;
  const int nw = min(8, w.ngi);
  int n_items = *w.nitems;
  for (int it = blockIdx.y; it < n_items; it += item_slots) {
    int4 item = w.items[it];
    int e = item.x, p0 = item.y, cnt = item.z;
    const int tt = (lane & 15) >> 1;
    const signed char *dsrc = nullptr;
    const float4 *gp = nullptr;
    if (tt < cnt) {
      dsrc = ((lane & 1) ? w.hd2 : w.hd1) + (size_t)(p0 + tt) * w.Ip;
      gp = w.hgp + (size_t)(p0 + tt) * w.ngi;
    }
    const TileMat md = xl.mat(e, 2);
    MtDigits dd;
    MtTiles<FMT> ta, tb;
    if (has) {
      mt_digits(dd, dsrc, gp, g, 1, lane);
      mt_load_rows<FMT>(ta, md, (size_t)rt0 * w.ngi + g, w.ngi, min(kMtBatch, rt1 - rt0), lane);
    }
    for (int rb = rt0; rb < rt1; rb += 2 * kMtBatch) {
      for (int h = 0; h < 2; h++) {
        const int r0 = rb + h * kMtBatch;
        if (r0 >= rt1) break;
        const int n = min(kMtBatch, rt1 - r0), r1 = r0 + kMtBatch;
        float acc[kMtBatch][4] = {};
        if (has) {
          MtTiles<FMT> &cur = h == 0 ? ta : tb;
          MtTiles<FMT> &nxt = h == 0 ? tb : ta;
          if (r1 < rt1) mt_load_rows<FMT>(nxt, md, (size_t)r1 * w.ngi + g, w.ngi, min(kMtBatch, rt1 - r1), lane);
          mt_compute_rows<FMT>(cur, dd, n, acc);
        }
#pragma unroll
        for (int i = 0; i < kMtBatch; i++)
#pragma unroll
          for (int r = 0; r < 4; r++) part[wave][i][lane][r] = acc[i][r];
        lds_only_barrier();
        for (int q = threadIdx.x; q < kMtBatch * 64 * 4; q += 512) {
          const int i = q >> 8, l = (q >> 2) & 63, r = q & 3;
          const int tq = (l & 15) >> 1;
          if (i < n && (l & 1) && tq < cnt) {
            float v = part[0][i][l][r];
            for (int u = 1; u < nw; u++) v += part[u][i][l][r];
            w.rout[(size_t)(p0 + tq) * w.H + (r0 + i) * kTileRows + 4 * (l >> 4) + r] = v;
          }
        }
        lds_only_barrier();
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 7w / 8w.  Wide items, for many-token steps with several tokens per expert:
// an item holds up to kWideTokens = 16 tokens of one expert, so every weight
// tile of the expert is read once per 16 tokens instead of once per 8.  The
// MFMA's 16 B columns are the item's 16 tokens, one digit plane per MFMA
// pair: c_d = sum code * digit_d (codes unsigned, exact int32), and a row's
// group value is A c_1 + B c_2 - K with K = OFF (A Q_1 + B Q_2) staged per
// (group, token) (Q_d: the token's digit sums, A and B its digit scales), so
// no lane is spent on the digit combination.  The item's digits and (A, B,
// K) are staged in LDS in the B-operand order; waves own row tiles and walk
// every group, a ring of groups' tiles in flight while one multiplies.  A
// wave's dot over the groups is one accumulation in group order.
// grid (row-tile blocks, item slots), 512 threads, dynamic LDS wide_lds_bytes.
// ---------------------------------------------------------------------------
constexpr int kWideTokens = 16;  // tokens per item (the MFMA's B columns)
// Row tiles per wave and groups in flight (the tile ring's slots): gate/up
// 1 row tile of both matrices x 2 groups, down 2 row tiles x 1 group; with
// the digits staged at most SW_WIDE_LDS_KB at a time, two 8-wave blocks share
// a compute unit.  Measured at S397 and S35 (512-token prefill): more waves a
// compute unit beat deeper rings.
#ifndef SW_WIDE_GU_RING
#define SW_WIDE_GU_RING 2
#endif
#ifndef SW_WIDE_DN_RING
#define SW_WIDE_DN_RING 1
#endif
#ifndef SW_WIDE_WAVES
#define SW_WIDE_WAVES 8
#endif
constexpr int kWideWaves = SW_WIDE_WAVES;  // waves per block
#ifndef SW_WIDE_GU_RT
#define SW_WIDE_GU_RT 1
#endif
#ifndef SW_WIDE_DN_RT
#define SW_WIDE_DN_RT 2
#endif
constexpr int kWideRt = SW_WIDE_GU_RT, kWideGuBatch = SW_WIDE_GU_RING;
constexpr int kWideDnRt = SW_WIDE_DN_RT, kWideDnBatch = SW_WIDE_DN_RING;

// LDS of one item over ng groups: digits [group][plane][half][lane] 16 B,
// then (A, B, K, 0) per [group][token]
__host__ __device__ inline size_t wide_lds_bytes(int ng) { return (size_t)ng * (4 * 1024 + 16 * 16); }

// Stage an item's digits.  Token tt of the item is row rows_of[p0+tt] of the
// digit planes (rows_of null: row p0+tt); tokens past cnt stage zeros.  Lane
// l of unit (g, plane d, half h) holds token l % 16's digits d at k = 128 g
// + 64 h + 16 (l >> 4): a thread's token is the same for every unit it
// stages (blockDim.x % 64 == 0), so its row is looked up once, and four
// units' loads are issued before their stores.
__device__ void wide_stage(unsigned char *lds, int hg, int g0, int gn, int ng, int ld, const signed char *d1,
                           const signed char *d2, const float4 *gp, const int *rows_of, int p0, int cnt, float off) {
  const int l = threadIdx.x & 63, tok = l & 15;
  const bool live = tok < cnt;
  const int row = live ? (rows_of ? rows_of[p0 + tok] : p0 + tok) : 0;
  const int nunits = gn * 256;
  for (int u0 = threadIdx.x; u0 < nunits; u0 += 4 * blockDim.x) {
    v4i v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int u = u0 + q * blockDim.x;
      const int h = (u >> 6) & 1, d = (u >> 7) & 1, g = g0 + (u >> 8);
      v[q] = v4i{0, 0, 0, 0};
      if (u < nunits && live)
        v[q] = *(const v4i *)((d ? d2 : d1) + (size_t)row * ld + g * kGroup + h * 64 + (l >> 4) * 16);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int u = u0 + q * blockDim.x;
      if (u < nunits) *(v4i *)(lds + (size_t)u * 16) = v[q];
    }
  }
  float4 *P = (float4 *)(lds + (size_t)hg * 4096);
  for (int v = threadIdx.x; v < gn * 16; v += blockDim.x) {
    const int t = v & 15, g = g0 + (v >> 4);
    float4 pv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < cnt) {
      const int r = rows_of ? rows_of[p0 + t] : p0 + t;
      const float4 q = gp[(size_t)r * ng + g];  // A, B, Q1, Q2
      const float k = off * (q.x * (float)__float_as_int(q.z) + q.y * (float)__float_as_int(q.w));
      pv = make_float4(q.x, q.y, k, 0.0f);
    }
    P[v] = pv;
  }
}

struct WideDigits {
  v4i b[2][2];  // [plane][half]
  float A, B, K;
};
__device__ __forceinline__ void wide_digits(WideDigits &d, const unsigned char *lds, int hg, int g, int lane) {
  const v4i *D = (const v4i *)lds;
#pragma unroll
  for (int q = 0; q < 4; q++) d.b[q >> 1][q & 1] = D[(g * 4 + q) * 64 + lane];
  const float4 p = ((const float4 *)(lds + (size_t)hg * 4096))[g * 16 + (lane & 15)];
  d.A = p.x;
  d.B = p.y;
  d.K = p.z;
}

// one tile (codes, row scales sc) into acc: rows 4 (lane >> 4) + r, token lane % 16
template <int FMT>
__device__ __forceinline__ void wide_mac(const uint32_t *q, const float4 sc, const WideDigits &d, float acc[4]) {
  v4i a0, a1;
  unpack_words<FMT>(q, a0, a1);
  v4i c1 = {0, 0, 0, 0}, c2 = {0, 0, 0, 0};
  c1 = mfma_i8(a0, d.b[0][0], c1);
  c2 = mfma_i8(a0, d.b[1][0], c2);
  c1 = mfma_i8(a1, d.b[0][1], c1);
  c2 = mfma_i8(a1, d.b[1][1], c2);
  const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float f = __builtin_fmaf(d.A, (float)c1[r], __builtin_fmaf(d.B, (float)c2[r], -d.K));
    acc[r] = __builtin_fmaf(f, scv[r], acc[r]);
  }
}

template <int FMT, int NB, int NR, int NM>
struct WideTiles {
  uint32_t q[NB][NR][NM][FMT == 4 ? 4 : 3];
  float4 sc[NB][NR][NM];
};

// Slot i of the tile ring holds one group's tiles for row tiles [rt0, rt0 +
// NR) of the NM matrices (mats[m]); row tiles past nrt are skipped.
template <int FMT, int NB, int NR, int NM>
__device__ __forceinline__ void wide_load_slot(WideTiles<FMT, NB, NR, NM> &t, int i, const TileMat *mats, int rt0,
                                               int nrt, int ng, int g, int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
  const int kb = lane >> 4;
#pragma unroll
  for (int rr = 0; rr < NR; rr++)
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const int rt = rt0 + rr;
      if (rt < nrt) {
        const size_t tg = (size_t)rt * ng + g;
        load_words<FMT>(tm_codes(mats[m], tg) + lane * BPL, t.q[i][rr][m]);
        t.sc[i][rr][m] = *(const float4 *)(tm_scales(mats[m], tg) + 4 * kb);
      }
    }
}

// Every group of row tiles [rt0, rt0 + NR) through a ring of NB slots: group
// g's tiles are loaded NB groups ahead, into the slot group g - NB has just
// left, so NB groups' tiles are in flight while one multiplies.  The item's
// digits are staged hg groups at a time (hg % NB == 0) between block
// barriers; the ring's loads run on across them.  Waves without row tiles
// (active false) take part in the staging and the barriers only.
template <int FMT, int NB, int NR, int NM, class Stage>
__device__ __forceinline__ void wide_rows(const TileMat *mats, const unsigned char *lds, int hg, int rt0, int nrt,
                                          int ng, bool active, int lane, float acc[NR][NM][4], Stage stage) {
  WideTiles<FMT, NB, NR, NM> t;
  if (active) {
#pragma unroll
    for (int i = 0; i < NB; i++)
      if (i < ng) wide_load_slot<FMT, NB, NR, NM>(t, i, mats, rt0, nrt, ng, i, lane);
  }
  for (int g0 = 0; g0 < ng; g0 += hg) {
    const int g1 = min(ng, g0 + hg);
    __syncthreads();  // every wave is done with the previous digits
    stage(g0, g1 - g0);
    __syncthreads();
    if (!active) continue;
    for (int gb = g0; gb < g1; gb += NB) {
#pragma unroll
      for (int i = 0; i < NB; i++) {
        const int g = gb + i;
        if (g >= g1) break;
        WideDigits d;
        wide_digits(d, lds, hg, g - g0, lane);
#pragma unroll
        for (int rr = 0; rr < NR; rr++)
          if (rt0 + rr < nrt)
#pragma unroll
            for (int m = 0; m < NM; m++) wide_mac<FMT>(t.q[i][rr][m], t.sc[i][rr][m], d, acc[rr][m]);
        if (g + NB < ng) wide_load_slot<FMT, NB, NR, NM>(t, i, mats, rt0, nrt, ng, g + NB, lane);
      }
    }
  }
}

// Groups per staging round for ng groups: the fewest rounds whose LDS fits a
// compute unit, rounded up to the ring's slot count.
#ifndef SW_WIDE_LDS_KB
#define SW_WIDE_LDS_KB 76
#endif
__host__ __device__ inline int wide_stage_groups(int ng, int nb) {
  const size_t cap = SW_WIDE_LDS_KB * 1024;
  int parts = (int)(((size_t)ng * 4352 + cap - 1) / cap);
  if (parts < 1) parts = 1;
  const int hg = (ng + parts - 1) / parts;
  return (hg + nb - 1) / nb * nb;
}

// (chunk, slot) of block `lin` of a 1-D grid of nx chunks x ny item slots,
// placed so that the nx chunks of one slot run on one XCD.  Blocks go to the
// device's 8 XCDs round-robin by linear id and each XCD has its own L2, so an
// item's activation digits, which every chunk stages, come from HBM once per
// item instead of once per chunk.  Within each group of 8 slots, block
// g*8*nx + 8*c + j is chunk c of slot g*8 + j; the slots past the last full
// group follow in plain order.
__device__ __forceinline__ void xcd_block(int lin, int nx, int ny, int &chunk, int &slot) {
  const int full = ny / 8 * 8;
  if (lin < full * nx) {
    const int g = lin / (8 * nx), r = lin - g * 8 * nx;
    chunk = r >> 3;
    slot = g * 8 + (r & 7);
  } else {
    const int r = lin - full * nx;
    chunk = r % nx;
    slot = full + r / nx;
  }
}

// routed gate/up of wide items: h = silu(g)*u.  Block: kWideWaves waves x
// kWideRt row tiles of I; a 1-D grid of nx = ceil(I/16 / (kWideWaves kWideRt))
// chunks x ny item slots placed by xcd_block, dynamic LDS wide_lds_bytes(hg).
//
// A block's kWideWaves row tiles are one 128-value group of I, so the block
// also forms the down kernel's activation digits of its group (as
// quantize_digits: the group's maximum, two int8 digits per value, the digit
// sums), the waves meeting in LDS for the group's maximum and sums; rows past
// I are zero values.  The first nsb blocks (a multiple of 8, so that the
// item blocks keep their XCD placement) form the shared expert's hidden rows
// (prep_shared_hidden) of tokens 0..T-1 instead: k_prep_hidden's work, with
// no launch of its own.
static_assert(kWideWaves * kWideRt * kTileRows == kGroup, "a wide gate/up block is one digit group of I");
template <int FMT>
__global__ __launch_bounds__(64 * kWideWaves) void k_gateup_wide(Work w, ExpertLayout xl, int hg, int nx, int ny,
                                                                 int nsb, const float *sh_gs, const float *sh_us) {
  extern __shared__ __align__(16) unsigned char wlds[];
  __shared__ float s_red[16];
  __shared__ float s_amax[kWideWaves][16];
  __shared__ int s_q[kWideWaves][2][16];
  if ((int)blockIdx.x < nsb) {
    if ((int)blockIdx.x < w.T) prep_shared_hidden(w, sh_gs, sh_us, blockIdx.x, s_red);
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kb = lane >> 4;
  const int nrt = w.I / kTileRows;
  int chunk, slot;
  xcd_block((int)blockIdx.x - nsb, nx, ny, chunk, slot);
  const int rt0 = (chunk * kWideWaves + wave) * kWideRt;
  const int n_items = *w.nitems;
  for (int it = slot; it < n_items; it += ny) {
    const int4 item = w.items[it];
    const int e = item.x, p0 = item.y, cnt = item.z;
    const TileMat mats[2] = {xl.mat(e, 0), xl.mat(e, 1)};
    float acc[kWideRt][2][4] = {};
    wide_rows<FMT, kWideGuBatch, kWideRt, 2>(
        mats, wlds, hg, rt0, nrt, w.ngh, rt0 < nrt, lane, acc, [&](int g0, int gn) {
          wide_stage(wlds, hg, g0, gn, w.ngh, w.Hp, w.xd1, w.xd2, w.xgp, w.btok, p0, cnt, FMT == 4 ? 8.0f : 4.0f);
        });
    // h = silu(g)*u of the wave's 16 rows (4 a lane) for token lane % 16
    // (zero past I: a wave without rows holds zero sums), then the group's
    // digits for the down kernel
    const int tt = lane & 15;
    float h[4];
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      h[r] = silu_ref(acc[0][0][r]) * acc[0][1][r];
      m = fmaxf(m, fabsf(h[r]));
    }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (kb == 0) s_amax[wave][tt] = m;
    __syncthreads();
    float amax = 0.0f;
#pragma unroll
    for (int v = 0; v < kWideWaves; v++) amax = fmaxf(amax, s_amax[v][tt]);
    const float A = amax / 127.0f, B = A / 254.0f;
    int q1[4] = {0, 0, 0, 0}, q2[4] = {0, 0, 0, 0};
    if (amax > 0.0f) {
      const float invA = 127.0f / amax, invB = 254.0f / A;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        q1[r] = (int)fminf(fmaxf(__builtin_rintf(h[r] * invA), -127.0f), 127.0f);
        const float rr = __builtin_fmaf(-(float)q1[r], A, h[r]);
        q2[r] = (int)fminf(fmaxf(__builtin_rintf(rr * invB), -127.0f), 127.0f);
      }
    }
    const int g = chunk;  // this block's group of I
    const size_t at = (size_t)(p0 + tt) * w.Ip + (size_t)g * kGroup + (size_t)wave * kTileRows + 4 * kb;
    if (tt < cnt) {
      *(unsigned *)(w.hd1 + at) = pack_i8x4(q1[0], q1[1], q1[2], q1[3]);
      *(unsigned *)(w.hd2 + at) = pack_i8x4(q2[0], q2[1], q2[2], q2[3]);
    }
    int Q1 = q1[0] + q1[1] + q1[2] + q1[3], Q2 = q2[0] + q2[1] + q2[2] + q2[3];
    Q1 += __shfl_xor(Q1, 16, 64);
    Q1 += __shfl_xor(Q1, 32, 64);
    Q2 += __shfl_xor(Q2, 16, 64);
    Q2 += __shfl_xor(Q2, 32, 64);
    if (kb == 0) {
      s_q[wave][0][tt] = Q1;
      s_q[wave][1][tt] = Q2;
    }
    __syncthreads();
    if (wave == 0 && kb == 0 && tt < cnt) {
      int S1 = 0, S2 = 0;
#pragma unroll
      for (int v = 0; v < kWideWaves; v++) {
        S1 += s_q[v][0][tt];
        S2 += s_q[v][1][tt];
      }
      w.hgp[(size_t)(p0 + tt) * w.ngi + g] = make_float4(A, B, __int_as_float(S1), __int_as_float(S2));
    }
  }
}

// routed down of wide items, plus the shared expert's token chunks (IDOT) in
// the first blocks y < shc (scheduled first, they overlap the routed work).
// Block: kWideWaves waves x kWideDnRt row tiles of H; a 1-D grid of shc*nx
// shared blocks, then nx = ceil(H/16 / (kWideWaves kWideDnRt)) chunks x ny
// item slots placed by xcd_block.
template <int FMT>
__global__ __launch_bounds__(64 * kWideWaves) void k_down_wide(Work w, ExpertLayout xl, int shc,
                                                               const signed char *dq, const float *ds, int hg,
                                                               int nx, int ny) {
  extern __shared__ __align__(16) unsigned char wlds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kb = lane >> 4;
  const int nrt = w.H / kTileRows;
  const int lin = (int)blockIdx.x;
  if (lin < shc * nx) {  // shared down, kSharedBlockTokens tokens a block
    const int rtb = lin % nx * kWideWaves * kWideDnRt;
    const int rt1 = min(nrt, rtb + kWideWaves * kWideDnRt);
    const int t0 = lin / nx * kSharedBlockTokens;
    for (int rt = rtb + wave; rt < rt1; rt += kWideWaves) {
      v4i c[kSharedSub] = {};
      idot_tiles<kSharedSub>(dq, w.Ish, rt * kTileRows, 0, w.Ish / 64, w.hq, w.Ish, t0, w.T, c, lane);
#pragma unroll
      for (int q = 0; q < kSharedSub; q++) {
        const int tok = t0 + 16 * q + (lane & 15);
        if (tok < w.T) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int row = rt * kTileRows + 4 * kb + i;
            w.shout[(size_t)tok * w.H + row] = (float)c[q][i] * ds[row] * w.shx[tok];
          }
        }
      }
    }
    return;
  }
  int chunk, slot;
  xcd_block(lin - shc * nx, nx, ny, chunk, slot);
  const int rt0 = chunk * kWideWaves * kWideDnRt + wave * kWideDnRt;
  const int n_items = *w.nitems;
  for (int it = slot; it < n_items; it += ny) {
    const int4 item = w.items[it];
    const int e = item.x, p0 = item.y, cnt = item.z;
    const TileMat mats[1] = {xl.mat(e, 2)};
    float acc[kWideDnRt][1][4] = {};
    wide_rows<FMT, kWideDnBatch, kWideDnRt, 1>(
        mats, wlds, hg, rt0, nrt, w.ngi, rt0 < nrt, lane, acc, [&](int g0, int gn) {
          wide_stage(wlds, hg, g0, gn, w.ngi, w.Ip, w.hd1, w.hd2, w.hgp, nullptr, p0, cnt, FMT == 4 ? 8.0f : 4.0f);
        });
    const int tt = lane & 15;
    if (tt < cnt && rt0 < nrt) {
#pragma unroll
      for (int rr = 0; rr < kWideDnRt; rr++) {
        const int rt = rt0 + rr;
        if (rt >= nrt) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) w.rout[(size_t)(p0 + tt) * w.H + rt * kTileRows + 4 * kb + r] = acc[rr][0][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 9. combine.  One token (moe_forward 3734-3737): out = fma chain over k of
// tmp_k * w_k, then fma(shared, sg).  Many tokens (moe_prefill_grouped
// 4151-4152, 3977, 4203): shared *= sg, routed = tmp*w, out = sum_k routed +
// shared.  grid (ceil(H/256), T), 256 threads.
// ---------------------------------------------------------------------------
__global__ void k_combine(Work w, float *y, int *route_idx, float *route_weight) {
  // the token's positions and weights in LDS, then every route's value of
  // this column loaded before the sums (which keep the reference's order)
  __shared__ int s_pos[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  const int h = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
  if (threadIdx.x < w.K) {
    s_pos[threadIdx.x] = w.pos[(size_t)t * w.K + threadIdx.x];
    s_w[threadIdx.x] = w.w[(size_t)t * w.K + threadIdx.x];
  }
  __syncthreads();
  if (h < w.H) {
    const float sg = w.sgate[t];
    const float sh = w.shout[(size_t)t * w.H + h];
    float v[kMaxTopK];
#pragma unroll
    for (int k = 0; k < kMaxTopK; k++)
      if (k < w.K) {
        const int p = s_pos[k];
        v[k] = p >= 0 ? w.rout[(size_t)p * w.H + h] : 0.0f;
      }
    float out = 0.0f;
    if (w.T == 1) {
#pragma unroll
      for (int k = 0; k < kMaxTopK; k++)
        if (k < w.K) out = __builtin_fmaf(v[k], s_w[k], out);
      out = __builtin_fmaf(sh, sg, out);
    } else {
      const float shs = sh * sg;
#pragma unroll
      for (int k = 0; k < kMaxTopK; k++)
        if (k < w.K) {
          const float r = v[k] * s_w[k];
          out = out + r;
        }
      out = out + shs;
    }
    y[(size_t)t * w.H + h] = out;
  }
  if (blockIdx.x == 0 && threadIdx.x < w.K) {
    size_t r = (size_t)t * w.K + threadIdx.x;
    if (route_idx) route_idx[r] = w.idx[r];
    if (route_weight) route_weight[r] = w.w[r];
  }
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
static int layer_alloc(ColiMoeLayer *L, void **p, size_t bytes, const char *what) {
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return fail_hip(what, e);
  L->alloc[L->nalloc++] = *p;
  L->bytes += bytes;
  return 0;
}

extern "C" int coli_cuda_moe_layer_create(ColiCuda *ctx, ColiMoeLayer **out, const ColiMoeShape *s) {
  if (!ctx || !out || !s) return fail_arg("coli_cuda_moe_layer_create: null argument");
  *out = nullptr;
  if (s->hidden <= 0 || s->experts <= 0 || s->topk <= 0 || s->intermediate <= 0 ||
      s->shared_intermediate <= 0 || s->hidden % 64 || s->topk > kMaxTopK || s->topk > s->experts ||
      s->experts > 4096 || s->group_size != kGroup || s->expert_format < 2 || s->expert_format > 4)
    return fail_arg("coli_cuda_moe_layer_create: unsupported shape (H%%64, group_size 128, format 2|3|4, "
                    "topk<=32, experts<=4096)");
  ColiMoeLayer *L = (ColiMoeLayer *)calloc(1, sizeof(ColiMoeLayer));
  if (!L) return fail_arg("out of memory creating MoE layer");
  // A ragged I or shared I is held as the next multiple of the row tiles:
  // the extra rows have zero codes and scales, so they add exact zeros (the
  // hidden values there are silu(0)*0 = 0, and the down columns they meet
  // hold zero values).
  L->sh = *s;
  // int2 experts are held as int4 records: code c is the nibble 5 + 2c, the
  // same value 2c - 3 (the reference widens them the same way for its device
  // path, q2_expand_q4 at c/qwen.c:567-575)
  L->src_fmt = s->expert_format;
  if (L->src_fmt == 2) L->sh.expert_format = 4;
  L->I_src = s->intermediate;
  L->Ish_src = s->shared_intermediate;
  L->sh.intermediate = (s->intermediate + kTileRows - 1) / kTileRows * kTileRows;
  L->sh.shared_intermediate = (s->shared_intermediate + 63) / 64 * 64;
  const bool ragged = L->sh.intermediate != L->I_src || L->sh.shared_intermediate != L->Ish_src;
  int H = s->hidden, I = L->sh.intermediate, E = s->experts, Ish = L->sh.shared_intermediate;
  L->ngh = (H + kGroup - 1) / kGroup;
  L->ngi = (I + kGroup - 1) / kGroup;
  L->xl = expert_layout(nullptr, H, I, L->sh.expert_format);
  int rc = layer_alloc(L, (void **)&L->router, (size_t)E * H * 4, "router allocation") ||
           layer_alloc(L, (void **)&L->sgate_row, (size_t)H * 4, "shared gate allocation") ||
           layer_alloc(L, (void **)&L->sh_gq, (size_t)Ish * H, "shared gate allocation") ||
           layer_alloc(L, (void **)&L->sh_uq, (size_t)Ish * H, "shared up allocation") ||
           layer_alloc(L, (void **)&L->sh_dq, (size_t)H * Ish, "shared down allocation") ||
           layer_alloc(L, (void **)&L->sh_gs, (size_t)Ish * 4, "shared scale allocation") ||
           layer_alloc(L, (void **)&L->sh_us, (size_t)Ish * 4, "shared scale allocation") ||
           layer_alloc(L, (void **)&L->sh_ds, (size_t)H * 4, "shared scale allocation") ||
           layer_alloc(L, (void **)&L->experts, (size_t)E * L->xl.expert_bytes, "expert allocation") ||
           layer_alloc(L, (void **)&L->stats, 64, "router stats allocation");
  L->sync_words = decode_sync_words(L->sh);
  rc = rc || layer_alloc(L, (void **)&L->sync, L->sync_words * 4, "decode counter allocation");
  if (rc) {
    coli_cuda_moe_layer_destroy(ctx, L);
    return -1;
  }
  L->xl.base = L->experts;
  k_zero_u32<<<blocks_for(16, 256), 256, 0, ctx->stream>>>((unsigned *)L->stats, 16);
  k_zero_u32<<<blocks_for(L->sync_words, 256), 256, 0, ctx->stream>>>(L->sync, L->sync_words);
  if (ragged) {  // the padding rows and columns start (and stay) zero
    const struct { void *p; size_t n; } z[] = {
        {L->sh_gq, (size_t)Ish * H}, {L->sh_uq, (size_t)Ish * H}, {L->sh_dq, (size_t)H * Ish},
        {L->sh_gs, (size_t)Ish * 4}, {L->sh_us, (size_t)Ish * 4}, {L->experts, (size_t)E * L->xl.expert_bytes}};
    for (const auto &r : z)
      k_zero_u32<<<blocks_for(r.n / 4, 256), 256, 0, ctx->stream>>>((unsigned *)r.p, r.n / 4);
  }
  *out = L;
  return launch_status("coli_cuda_moe_layer_create");
}

extern "C" void coli_cuda_moe_layer_destroy(ColiCuda *ctx, ColiMoeLayer *L) {
  if (!L) return;
  if (ctx) hipStreamSynchronize(ctx->stream);
  for (int i = 0; i < L->nalloc; i++) hipFree(L->alloc[i]);
  free(L);
}

extern "C" size_t coli_cuda_moe_layer_bytes(const ColiMoeLayer *L) { return L ? L->bytes : 0; }

extern "C" float *coli_cuda_moe_layer_router(ColiMoeLayer *L) { return L ? L->router : nullptr; }

extern "C" int coli_cuda_moe_set_router_mode(ColiMoeLayer *L, int mode) {
  if (!L || (mode != 0 && mode != 1)) return fail_arg("coli_cuda_moe_set_router_mode: invalid argument");
  L->router_mode = mode;
  return 0;
}

extern "C" int coli_cuda_moe_layer_set_router(ColiCuda *ctx, ColiMoeLayer *L, const float *router,
                                              const float *shared_gate) {
  if (!ctx || !L || !router || !shared_gate) return fail_arg("coli_cuda_moe_layer_set_router: null argument");
  hipMemcpyAsync(L->router, router, (size_t)L->sh.experts * L->sh.hidden * 4, hipMemcpyDeviceToDevice,
                 ctx->stream);
  hipMemcpyAsync(L->sgate_row, shared_gate, (size_t)L->sh.hidden * 4, hipMemcpyDeviceToDevice, ctx->stream);
  return launch_status("coli_cuda_moe_layer_set_router");
}

extern "C" int coli_cuda_moe_layer_set_shared_q8(ColiCuda *ctx, ColiMoeLayer *L, const signed char *gq,
                                                 const float *gs, const signed char *uq, const float *us,
                                                 const signed char *dq, const float *ds) {
  if (!ctx || !L || !gq || !gs || !uq || !us || !dq || !ds)
    return fail_arg("coli_cuda_moe_layer_set_shared_q8: null argument");
  // the caller's I rows; the down rows land at the device pitch (I rounded up)
  size_t H = L->sh.hidden, I = L->Ish_src, Ip = L->sh.shared_intermediate;
  hipStream_t st = ctx->stream;
  hipError_t e = hipMemcpyAsync(L->sh_gq, gq, I * H, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(L->sh_uq, uq, I * H, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpy2DAsync(L->sh_dq, Ip, dq, I, I, H, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(L->sh_gs, gs, I * 4, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(L->sh_us, us, I * 4, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(L->sh_ds, ds, H * 4, hipMemcpyDeviceToDevice, st);
  if (e != hipSuccess) return fail_hip("coli_cuda_moe_layer_set_shared_q8", e);
  return launch_status("coli_cuda_moe_layer_set_shared_q8");
}

// int2 container bytes (four codes a byte, lowest bits first, value 2c - 3)
// into int4 bytes (two nibbles a byte, low first, value n - 8): n = 5 + 2c
__global__ void k_widen_q2(unsigned short *out, const unsigned char *in, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned b = in[i];
  const unsigned c0 = 5 + 2 * (b & 3), c1 = 5 + 2 * ((b >> 2) & 3), c2 = 5 + 2 * ((b >> 4) & 3), c3 = 5 + 2 * (b >> 6);
  out[i] = (unsigned short)((c0 | c1 << 4) | (c2 | c3 << 4) << 8);
}

// container rows [rows_src x cols] into tile records of `rows` (a multiple of
// the tile rows) rows
static int repack_matrix(ColiCuda *ctx, const TileMat &dst, const unsigned char *q, const float *s, int rows,
                         int rows_src, int cols, int fmt) {
  int ng = (cols + kGroup - 1) / kGroup;
  int rb = fmt == 4 ? ng * kGroup / 2 : ng * kGroup * 3 / 8;
  unsigned char *base = const_cast<unsigned char *>(dst.base);
  size_t lanes = (size_t)(rows / kTileRows) * ng * 64;
  k_repack_codes<<<blocks_for(lanes, 256), 256, 0, ctx->stream>>>(base, dst.rs, q, rows, rows_src, cols, rb, ng,
                                                                   fmt);
  size_t ns = (size_t)rows * ng;
  k_repack_scales<<<blocks_for(ns, 256), 256, 0, ctx->stream>>>(base, dst.rs, dst.so, s, rows, rows_src, ng);
  return launch_status("expert repack");
}

namespace sw {
// One expert in container format `fmt`: the layer's own, or, for a layer held
// as int4 records (int4 or int2 experts), 2 or 4 per expert (EXPERT_Q2=1 takes
// an expert's .q2 sidecar where it has one, else its int4 payload,
// c/qwen.c:2207-2214).
int set_expert_as(ColiCuda *ctx, ColiMoeLayer *L, int expert, int src_fmt, const unsigned char *gq, const float *gs,
                  const unsigned char *uq, const float *us, const unsigned char *dq, const float *ds) {
  if (!ctx || !L || !gq || !gs || !uq || !us || !dq || !ds)
    return fail_arg("coli_cuda_moe_layer_set_expert: null argument");
  if (expert < 0 || expert >= L->sh.experts)
    return fail_arg("coli_cuda_moe_layer_set_expert: expert %d outside [0,%d)", expert, L->sh.experts);
  int H = L->sh.hidden, I = L->sh.intermediate, Is = L->I_src, fmt = L->sh.expert_format;
  if (src_fmt != L->src_fmt && !(fmt == 4 && (src_fmt == 2 || src_fmt == 4)))
    return fail_arg("coli_cuda_moe_layer_set_expert: format %d in a layer of format %d", src_fmt, L->src_fmt);
  if (src_fmt == 2) {
    // each matrix widened into scratch, then repacked as int4 (stream
    // order keeps one matrix's repack ahead of the next one's widening)
    const size_t bh = (size_t)Is * (L->ngh * kGroup / 4), bi = (size_t)H * (L->ngi * kGroup / 4);
    if (ensure_scratch(ctx, kScrSetup, 2 * (bh > bi ? bh : bi), "int2 expert widening")) return -1;
    unsigned char *w4 = (unsigned char *)ctx->scratch[kScrSetup];
    const unsigned char *src[3] = {gq, uq, dq};
    const float *sc[3] = {gs, us, ds};
    for (int m = 0; m < 3; m++) {
      const size_t nb = m < 2 ? bh : bi;
      k_widen_q2<<<blocks_for(nb, 256), 256, 0, ctx->stream>>>((unsigned short *)w4, src[m], nb);
      if (repack_matrix(ctx, L->xl.mat(expert, m), w4, sc[m], m < 2 ? I : H, m < 2 ? Is : H, m < 2 ? H : Is, 4))
        return -1;
    }
    return 0;
  }
  if (repack_matrix(ctx, L->xl.mat(expert, 0), gq, gs, I, Is, H, fmt) ||
      repack_matrix(ctx, L->xl.mat(expert, 1), uq, us, I, Is, H, fmt) ||
      repack_matrix(ctx, L->xl.mat(expert, 2), dq, ds, H, H, Is, fmt))
    return -1;
  return 0;
}
}  // namespace sw

extern "C" int coli_cuda_moe_layer_set_expert(ColiCuda *ctx, ColiMoeLayer *L, int expert,
                                              const unsigned char *gq, const float *gs, const unsigned char *uq,
                                              const float *us, const unsigned char *dq, const float *ds) {
  if (!L) return fail_arg("coli_cuda_moe_layer_set_expert: null argument");
  return sw::set_expert_as(ctx, L, expert, L->src_fmt, gq, gs, uq, us, dq, ds);
}

extern "C" int coli_cuda_moe_layer_set_expert_format(ColiCuda *ctx, ColiMoeLayer *L, int expert, int expert_format,
                                                     const unsigned char *gq, const float *gs,
                                                     const unsigned char *uq, const float *us,
                                                     const unsigned char *dq, const float *ds) {
  if (!L) return fail_arg("coli_cuda_moe_layer_set_expert_format: null argument");
  return sw::set_expert_as(ctx, L, expert, expert_format, gq, gs, uq, us, dq, ds);
}

extern "C" int coli_cuda_moe_layer_synthesize(ColiCuda *ctx, ColiMoeLayer *L, unsigned long long seed,
                                              int layer_index) {
  if (!ctx || !L) return fail_arg("coli_cuda_moe_layer_synthesize: null argument");
  // generated at the caller's shape (I_src, Ish_src), stored at the device's
  int H = L->sh.hidden, I = L->I_src, E = L->sh.experts, Ish = L->Ish_src;
  const int Ip = L->sh.intermediate, Ishp = L->sh.shared_intermediate;
  int fmt = L->sh.expert_format;
  uint32_t li = (uint32_t)layer_index;
  hipStream_t st = ctx->stream;
  size_t n;
  n = (size_t)E * H;
  k_synth_normal<<<blocks_for(n, 256), 256, 0, st>>>(L->router, n, sw_key(seed, li, 0, SW_T_ROUTER), 0.02f, 0);
  k_synth_normal<<<blocks_for(H, 256), 256, 0, st>>>(L->sgate_row, H, sw_key(seed, li, 0, SW_T_SHARED_GATE),
                                                     0.02f, 0);
  n = (size_t)Ish * H;
  k_synth_i8<<<blocks_for(n, 256), 256, 0, st>>>(L->sh_gq, n, sw_key(seed, li, 0, SW_T_SH_GATE_Q));
  k_synth_i8<<<blocks_for(n, 256), 256, 0, st>>>(L->sh_uq, n, sw_key(seed, li, 0, SW_T_SH_UP_Q));
  k_synth_i8_rows<<<blocks_for(n, 256), 256, 0, st>>>(L->sh_dq, H, Ish, Ishp, sw_key(seed, li, 0, SW_T_SH_DOWN_Q));
  k_synth_normal<<<blocks_for(Ish, 256), 256, 0, st>>>(L->sh_gs, Ish, sw_key(seed, li, 0, SW_T_SH_GATE_S), 0.01f, 1);
  k_synth_normal<<<blocks_for(Ish, 256), 256, 0, st>>>(L->sh_us, Ish, sw_key(seed, li, 0, SW_T_SH_UP_S), 0.01f, 1);
  k_synth_normal<<<blocks_for(H, 256), 256, 0, st>>>(L->sh_ds, H, sw_key(seed, li, 0, SW_T_SH_DOWN_S), 0.01f, 1);
  // routed experts: container bytes into scratch, repacked per matrix (int2
  // bytes widened to int4 first, behind them in the same scratch)
  const bool q2 = L->src_fmt == 2;
  auto row_b = [&](int ng) { return q2 ? ng * kGroup / 4 : fmt == 4 ? ng * kGroup / 2 : ng * kGroup * 3 / 8; };
  int rbh = row_b(L->ngh), rbi = row_b(L->ngi);
  size_t need = (size_t)I * rbh > (size_t)H * rbi ? (size_t)I * rbh : (size_t)H * rbi;
  const size_t wide_off = (need + 255) & ~(size_t)255;
  if (ensure_scratch(ctx, kScrSetup, q2 ? wide_off + 2 * need : need, "synthesis scratch")) return -1;
  unsigned char *tmp = (unsigned char *)ctx->scratch[kScrSetup];
  for (int e = 0; e < E; e++) {
    const int tq[3] = {SW_T_GATE_Q, SW_T_UP_Q, SW_T_DOWN_Q}, ts[3] = {SW_T_GATE_S, SW_T_UP_S, SW_T_DOWN_S};
    for (int m = 0; m < 3; m++) {
      int rows = m < 2 ? I : H, cols = m < 2 ? H : I, rb = m < 2 ? rbh : rbi, ng = m < 2 ? L->ngh : L->ngi;
      const int rows_dev = m < 2 ? Ip : H;
      size_t nb = (size_t)rows * rb;
      k_synth_bytes<<<blocks_for((nb + 7) / 8, 256), 256, 0, st>>>(tmp, nb, sw_key(seed, li, (uint32_t)e, tq[m]));
      const unsigned char *codes = tmp;
      int rbd = rb;
      if (q2) {
        k_widen_q2<<<blocks_for(nb, 256), 256, 0, st>>>((unsigned short *)(tmp + wide_off), tmp, nb);
        codes = tmp + wide_off;
        rbd = 2 * rb;
      }
      const TileMat dst = L->xl.mat(e, m);
      unsigned char *base = const_cast<unsigned char *>(dst.base);
      size_t lanes = (size_t)(rows_dev / kTileRows) * ng * 64;
      k_repack_codes<<<blocks_for(lanes, 256), 256, 0, st>>>(base, dst.rs, codes, rows_dev, rows, cols, rbd, ng, fmt);
      k_synth_scales_tiled<<<blocks_for((size_t)rows_dev * ng, 256), 256, 0, st>>>(
          base, dst.rs, dst.so, rows_dev, rows, ng, sw_key(seed, li, (uint32_t)e, ts[m]));
    }
  }
  return launch_status("coli_cuda_moe_layer_synthesize");
}

static Work make_work(const ColiMoeLayer *L, int T) {
  Work w;
  memset(&w, 0, sizeof(w));
  w.itok = kMaxTokensPerItem;
  w.T = T;
  w.H = L->sh.hidden;
  w.E = L->sh.experts;
  w.K = L->sh.topk;
  w.I = L->sh.intermediate;
  w.Ish = L->sh.shared_intermediate;
  w.ngh = L->ngh;
  w.ngi = L->ngi;
  w.Hp = w.ngh * kGroup;
  w.Ip = w.ngi * kGroup;
  w.shks = T <= kShSplitTokens ? kShSplit : 0;
  return w;
}

// dynamic LDS above 64 KiB must be enabled per kernel (gfx950: 160 KiB/CU)
// Bytes of LDS the bucketing kernels need: an E x T bit map (one 32-token
// word per expert and 32 tokens) plus 2E+1 counters.
static size_t bucket_lds_bytes(int E, int T) {
  return (size_t)E * ((T + 31) / 32) * 4 + (size_t)(2 * E + 1) * 4;
}

// Tokens one many-token step takes for E experts: the bucketing map must fit
// a workgroup's 160 KiB of LDS, and at most kMaxTokens.  Longer blocks run as
// several steps of balanced size (tokens are independent of each other).
static int tokens_per_step(int E) {
  const size_t cap = 160 * 1024, fixed = (size_t)(2 * E + 1) * 4;
  if (E <= 0 || fixed >= cap) return 0;
  const size_t t = (cap - fixed) / ((size_t)E * 4) * 32;
  return t < (size_t)kMaxTokens ? (int)t : kMaxTokens;
}

static int set_lds(const void *fn, size_t bytes) {
  if (bytes > 160 * 1024) return fail_arg("MoE step kernel needs %zu bytes of LDS (> 160 KiB)", bytes);
  if (bytes <= 64 * 1024) return 0;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return e == hipSuccess ? 0 : fail_hip("hipFuncSetAttribute", e);
}

// Block shape of the tiled bounds kernel: RB rows (waves) by tpb tokens.
// Every wave-round (one row, kRbRound tokens) costs about the same, so the
// shape that gives the busiest SIMD the fewest wave-rounds wins, then the one
// whose blocks all stay resident (two per compute unit: LDS), then the one
// with the most blocks (latency hiding).  S397 (512 rows): 8 tokens take 4-row
// blocks, one per compute unit; 32 tokens 8-row blocks of 4 tokens, two per
// compute unit.
struct RbShape {
  int rb, tpb, nb;
};
static RbShape rb_shape(int E, int T, int cus) {
  RbShape best = {0, 0, 0};
  long long best_w = 0;
  bool best_over = true;
  for (int rb = 8; rb >= 4; rb -= 4)
    for (int tpb = kRbRound; tpb < T + kRbRound; tpb += kRbRound) {
      const int nb = (E + rb - 1) / rb * ((T + tpb - 1) / tpb);
      const long long wr = (long long)((nb + cus - 1) / cus) * (rb / 4) * (tpb / kRbRound);
      const bool over = nb > 2 * cus;
      const bool better = best.rb == 0 || wr < best_w || (wr == best_w && best_over && !over) ||
                          (wr == best_w && over == best_over && !over && nb > best.nb);
      if (better) {
        best = {rb, tpb, nb};
        best_w = wr;
        best_over = over;
      }
    }
  return best;
}

template <int CH>
static int router_bounds_tiled(ColiCuda *ctx, ColiMoeLayer *L, Work &w, const float *x) {
  const size_t lds = (size_t)kRbRound * 64 * CH * 4;
  const RbShape sh = rb_shape(w.E, w.T, ctx->sm_count > 0 ? ctx->sm_count : 256);
  const dim3 grid((w.E + sh.rb - 1) / sh.rb, (w.T + sh.tpb - 1) / sh.tpb);
  if (sh.rb == 8) {
    if (set_lds((const void *)k_router_bounds_tiled<CH, 8>, lds)) return -1;
    k_router_bounds_tiled<CH, 8><<<grid, 512, lds, ctx->stream>>>(w, x, L->router, sh.tpb);
  } else {
    if (set_lds((const void *)k_router_bounds_tiled<CH, 4>, lds)) return -1;
    k_router_bounds_tiled<CH, 4><<<grid, 256, lds, ctx->stream>>>(w, x, L->router, sh.tpb);
  }
  return 0;
}

// Steps of at least this many tokens route through the fp64 MFMA GEMM (at
// S397 the tiled bounds kernel is faster up to 32 tokens: 110 against 124 us)
#ifndef SW_ROUTER_GEMM_TOKENS
#define SW_ROUTER_GEMM_TOKENS 64
#endif
constexpr int kRouterGemmTokens = SW_ROUTER_GEMM_TOKENS;

template <int NV, int PC>
static void certify_launch(ColiCuda *ctx, ColiMoeLayer *L, Work &w, const float *x) {
  k_certify_wave<NV, PC><<<(w.T + 3) / 4 + (PC > 0 ? w.T : 0), 256, 0, ctx->stream>>>(w, L->router_mode, L->stats, x,
                                                                                       L->sgate_row);
}

static int route_launch(ColiCuda *ctx, ColiMoeLayer *L, Work &w, const float *x) {
  hipStream_t st = ctx->stream;
  // the tiled bounds kernel resets the certification counters and the
  // certification kernel forms the activations in blocks of its own; the
  // other router paths take k_prep_x first
  int rc = 1;  // 1: shape or alignment outside the tiled router kernel
  if (w.T < kRouterGemmTokens && ((uintptr_t)x & 15) == 0 && w.E <= 1024) switch (w.H) {
      case 256: rc = router_bounds_tiled<4>(ctx, L, w, x); break;
      case 512: rc = router_bounds_tiled<8>(ctx, L, w, x); break;
      case 1024: rc = router_bounds_tiled<16>(ctx, L, w, x); break;
      case 2048: rc = router_bounds_tiled<32>(ctx, L, w, x); break;
      case 4096: rc = router_bounds_tiled<64>(ctx, L, w, x); break;
      default: break;
    }
  if (rc < 0) return -1;
  if (rc == 0) {
    // prep_token with 256 threads: C = padded row float4s / 256 = H / 1024
    const bool e8 = w.E <= 512;
    switch (w.H) {
      case 256:
      case 512:
      case 1024: e8 ? certify_launch<8, 1>(ctx, L, w, x) : certify_launch<16, 1>(ctx, L, w, x); break;
      case 2048: e8 ? certify_launch<8, 2>(ctx, L, w, x) : certify_launch<16, 2>(ctx, L, w, x); break;
      default: e8 ? certify_launch<8, 4>(ctx, L, w, x) : certify_launch<16, 4>(ctx, L, w, x); break;
    }
  } else {
    const int hp4 = w.ngh * 128 / 4;  // float4 chunks of the padded row
    if (hp4 <= 1024)
      k_prep_x<1><<<w.T, 1024, 0, st>>>(w, x, L->sgate_row);
    else if (hp4 <= 2048)
      k_prep_x<2><<<w.T, 1024, 0, st>>>(w, x, L->sgate_row);
    else if (hp4 <= 4096)
      k_prep_x<4><<<w.T, 1024, 0, st>>>(w, x, L->sgate_row);
    else if (hp4 <= 8192)
      k_prep_x<8><<<w.T, 1024, 0, st>>>(w, x, L->sgate_row);
    else
      k_prep_x_any<<<w.T, 1024, 0, st>>>(w, x, L->sgate_row);
    if (w.T >= kRouterGemmTokens && w.H % 64 == 0 && ((uintptr_t)x & 15) == 0) {
      k_router_gemm<<<dim3((w.E + 15) / 16, (w.T + 15) / 16), 256, 0, st>>>(w, x, L->router);
      k_router_refine<<<w.T, 256, (size_t)64 * (w.H / 64 + 1) * 4, st>>>(w, x, L->router);
    } else {
      k_router_bounds<<<dim3((w.E + 3) / 4, w.T), 256, 0, st>>>(w, x, L->router);
    }
    if (w.E <= 512)
      certify_launch<8, 0>(ctx, L, w, x);
    else if (w.E <= 1024)
      certify_launch<16, 0>(ctx, L, w, x);
    else
      k_certify<<<w.T, 512, 0, st>>>(w, L->router_mode, L->stats);
  }
  if (set_lds((const void *)k_exact_logits, (size_t)w.H * 4)) return -1;
  k_exact_logits<<<dim3(64, w.T < kUncertainSlots ? w.T : kUncertainSlots), 64, (size_t)w.H * 4, st>>>(
      w, x, L->router, L->stats);
  const int e4 = (w.E + 3) & ~3;
  const size_t full_lds = (size_t)4 * (w.H > 2 * e4 ? w.H : 2 * e4);
  if (set_lds((const void *)k_exact_full, full_lds)) return -1;
  k_exact_full<<<dim3(w.E < 1024 ? w.E : 1024, w.T < kFullSlots ? w.T : kFullSlots), 64, full_lds, st>>>(w, x,
                                                                                                       L->router);
  return launch_status("MoE routing kernels");
}

// Tokens per bucketing item: the wide items (each expert's tiles read once
// per kWideTokens tokens) whenever an item's digits fit the LDS.  Their
// kernels give each wave whole row tiles, streamed through every group with
// no block barrier, and are faster at every step size measured, however few
// tokens an expert holds (S397: 834 against 686 tok/s at 8 tokens a step,
// 1763 against 1388 at 32).  The context's setting
// (coli_cuda_moe_set_item_tokens) can force either.
static int item_tokens(const ColiCuda *ctx, const ColiMoeLayer *L) {
  const int mode = ctx->moe_item_tokens;
  const bool fits = wide_lds_bytes(wide_stage_groups(L->ngh, kWideGuBatch)) <= 160 * 1024 &&
                    wide_lds_bytes(wide_stage_groups(L->ngi, kWideDnBatch)) <= 160 * 1024;
  return fits && mode != kMaxTokensPerItem ? kWideTokens : kMaxTokensPerItem;
}

static int prepare(ColiCuda *ctx, ColiMoeLayer *L, int T, Work &w) {
  if (T <= 0 || T > kMaxTokens) return fail_arg("MoE step: tokens %d outside [1,%d]", T, kMaxTokens);
  w = make_work(L, T);
  w.itok = item_tokens(ctx, L);
  size_t bytes = carve(w, nullptr);
  if (ensure_scratch(ctx, kScrXPrep, bytes, "MoE workspace allocation")) return -1;
  carve(w, (char *)ctx->scratch[kScrXPrep]);
  return 0;
}

extern "C" int coli_cuda_moe_route(ColiCuda *ctx, ColiMoeLayer *L, const float *x, int tokens, int *idx,
                                   float *weight) {
  if (!ctx || !L || !x || !idx || !weight) return fail_arg("coli_cuda_moe_route: null argument");
  const int tmax = tokens_per_step(L->sh.experts);
  if (tokens > tmax && tmax > 0) {
    const int nc = (tokens + tmax - 1) / tmax;
    const size_t H = (size_t)L->sh.hidden, K = (size_t)L->sh.topk;
    for (int c = 0, t0 = 0; c < nc; c++) {
      const int n = tokens / nc + (c < tokens % nc ? 1 : 0);
      if (coli_cuda_moe_route(ctx, L, x + (size_t)t0 * H, n, idx + (size_t)t0 * K, weight + (size_t)t0 * K))
        return -1;
      t0 += n;
    }
    return 0;
  }
  Work w;
  if (prepare(ctx, L, tokens, w)) return -1;
  if (route_launch(ctx, L, w, x)) return -1;
  hipMemcpyAsync(idx, w.idx, (size_t)tokens * w.K * 4, hipMemcpyDeviceToDevice, ctx->stream);
  hipMemcpyAsync(weight, w.w, (size_t)tokens * w.K * 4, hipMemcpyDeviceToDevice, ctx->stream);
  return launch_status("coli_cuda_moe_route");
}

// stage marks (coli_cuda_moe_stage_timing): event i closes stage i-1
static inline void mark(ColiCuda *ctx, int i) {
  if (ctx->moe_timing) hipEventRecord(ctx->moe_event[i], ctx->stream);
}

static void stage_accumulate(ColiCuda *ctx) {
  if (!ctx->moe_timing) return;
  hipEventSynchronize(ctx->moe_event[7]);
  for (int i = 0; i < 7; i++) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ctx->moe_event[i], ctx->moe_event[i + 1]) == hipSuccess) ctx->moe_ms[i] += ms;
  }
  ctx->moe_calls++;
}

extern "C" int coli_cuda_moe_forward(ColiCuda *ctx, ColiMoeLayer *L, float *y, const float *x, int tokens,
                                     int *route_idx, float *route_weight) {
  if (!ctx || !L || !y || !x) return fail_arg("coli_cuda_moe_forward: null argument");
  if (!prof_active(ctx)) prof_open(ctx);
  const int tmax = tokens_per_step(L->sh.experts);
  if (tokens > tmax && tmax > 0) {
    // a long block (a whole prompt): balanced steps of at most tmax tokens,
    // never a lone token (which would take the decode kernels)
    const int nc = (tokens + tmax - 1) / tmax;
    const size_t H = (size_t)L->sh.hidden, K = (size_t)L->sh.topk;
    for (int c = 0, t0 = 0; c < nc; c++) {
      const int n = tokens / nc + (c < tokens % nc ? 1 : 0);
      if (coli_cuda_moe_forward(ctx, L, y + (size_t)t0 * H, x + (size_t)t0 * H, n,
                                route_idx ? route_idx + (size_t)t0 * K : nullptr,
                                route_weight ? route_weight + (size_t)t0 * K : nullptr))
        return -1;
      t0 += n;
    }
    return 0;
  }
  if (tokens == 1 && !ctx->moe_generic_only) {
    if (ctx->moe_decode_mode == 0) {
      ColiMoeLayer *one[1] = {L};
      int rc = stack_step(ctx, one, 1, y, 0, x, 0, route_idx, route_weight);
      if (rc <= 0) return rc;  // 1: shape outside the persistent kernel's limits
    }
    int rc = decode_step(ctx, L, y, x, route_idx, route_weight);
    if (rc <= 0) return rc;  // 1: shape outside the decode kernels' limits
  }
  Work w;
  if (prepare(ctx, L, tokens, w)) return -1;
  w.order_free = route_idx == nullptr && route_weight == nullptr;
  hipStream_t st = ctx->stream;
  int T = tokens;
  mark(ctx, 0);
  if (route_launch(ctx, L, w, x)) return -1;
  mark(ctx, 1);
  const size_t bucket_lds = bucket_lds_bytes(w.E, T);
  if (T <= kShSplitTokens) {
    // the bucketing and the split shared gate/up in one launch
    const int ns = T <= 16 ? 1 : T <= 32 ? 2 : 4;
    const int nsh = w.Ish / kTileRows * kShSplit * (ns == 4 ? (T + 63) / 64 : 1);
    const size_t lds = std::max(bucket_lds, (size_t)32 * 256 * ns);
    const void *fn = ns == 1 ? (const void *)k_bucket_shared<1> : ns == 2 ? (const void *)k_bucket_shared<2>
                                                                          : (const void *)k_bucket_shared<4>;
    if (set_lds(fn, lds)) return -1;
    if (ns == 1)
      k_bucket_shared<1><<<1 + nsh, 256, lds, st>>>(w, L->sh_gq, L->sh_uq);
    else if (ns == 2)
      k_bucket_shared<2><<<1 + nsh, 256, lds, st>>>(w, L->sh_gq, L->sh_uq);
    else
      k_bucket_shared<4><<<1 + nsh, 256, lds, st>>>(w, L->sh_gq, L->sh_uq);
    mark(ctx, 2);
    prof_mark(ctx, kStageSetup);
  } else {
    if (set_lds((const void *)k_bucket, bucket_lds)) return -1;
    k_bucket<<<1, 1024, bucket_lds, st>>>(w);
    mark(ctx, 2);
    prof_mark(ctx, kStageSetup);
    k_shared_swiglu<4><<<dim3(w.Ish / kTileRows, (T + 63) / 64), 256, 0, st>>>(w, L->sh_gq, L->sh_gs, L->sh_uq,
                                                                              L->sh_us);
  }
  mark(ctx, 3);
  prof_mark(ctx, kStageSharedHidden);
  int item_bound = w.E + (T * w.K + w.itok - 1) / w.itok;
  int slots = item_bound < T * w.K ? item_bound : T * w.K;
  if (slots > 1024) slots = 1024;
  const bool fmt4 = L->sh.expert_format == 4;
  const bool wide_items = w.itok > kMaxTokensPerItem;
  if (wide_items) {
    const int hg = wide_stage_groups(w.ngh, kWideGuBatch);
    const size_t lg = wide_lds_bytes(hg);
    const void *fn = fmt4 ? (const void *)k_gateup_wide<4> : (const void *)k_gateup_wide<3>;
    if (set_lds(fn, lg)) return -1;
    const int nx = (w.I / kTileRows + kWideWaves * kWideRt - 1) / (kWideWaves * kWideRt);
    const int nsb = (T + 7) / 8 * 8;  // the shared hidden rows' blocks (k_prep_hidden's work)
    if (fmt4)
      k_gateup_wide<4><<<nsb + nx * slots, 64 * kWideWaves, lg, st>>>(w, L->xl, hg, nx, slots, nsb, L->sh_gs,
                                                                      L->sh_us);
    else
      k_gateup_wide<3><<<nsb + nx * slots, 64 * kWideWaves, lg, st>>>(w, L->xl, hg, nx, slots, nsb, L->sh_gs,
                                                                      L->sh_us);
  } else {
    const int gu_rt = T * w.K <= 64 ? kGuRowTilesSmall : kGuRowTiles;
    const int gu_blocks_x = (w.I / kTileRows + gu_rt - 1) / gu_rt;
    const bool wide = (w.ngh + 7) / 8 > kMtBatch;  // a wave's groups exceed one batch
    if (!wide && SW_GU_USE_RING) {
      const size_t lg = (size_t)8 * kGuRing * L->xl.rec_gu();
      const void *fn = fmt4 ? (const void *)k_gateup_ring<4> : (const void *)k_gateup_ring<3>;
      if (set_lds(fn, lg + sizeof(float) * 8 * 2 * 64 * 4)) return -1;
      if (fmt4)
        k_gateup_ring<4><<<dim3(gu_blocks_x, slots), 512, lg, st>>>(w, L->xl, gu_rt);
      else
        k_gateup_ring<3><<<dim3(gu_blocks_x, slots), 512, lg, st>>>(w, L->xl, gu_rt);
    } else if (fmt4)
      wide ? k_expert_gateup<4, true><<<dim3(gu_blocks_x, slots), 512, 0, st>>>(w, L->xl, gu_rt)
           : k_expert_gateup<4, false><<<dim3(gu_blocks_x, slots), 512, 0, st>>>(w, L->xl, gu_rt);
    else
      wide ? k_expert_gateup<3, true><<<dim3(gu_blocks_x, slots), 512, 0, st>>>(w, L->xl, gu_rt)
           : k_expert_gateup<3, false><<<dim3(gu_blocks_x, slots), 512, 0, st>>>(w, L->xl, gu_rt);
  }
  mark(ctx, 4);
  prof_mark(ctx, kStageRoutedHidden);
  if (!wide_items) k_prep_hidden<<<T + T * w.K, 256, 0, st>>>(w, L->sh_gs, L->sh_us);  // else in k_gateup_wide
  mark(ctx, 5);
  int sh_chunks = (T + kSharedTokens - 1) / kSharedTokens;
  const int dn_blocks_x = (w.H / kTileRows + 4 * kDnRowTiles - 1) / (4 * kDnRowTiles);
  const bool dn_split = w.ngi <= 8;
  const int ds_blocks_x = (w.H / kTileRows + kDnBlockRows - 1) / kDnBlockRows;
  if (wide_items) {
    const int hg = wide_stage_groups(w.ngi, kWideDnBatch);
    const size_t ld = wide_lds_bytes(hg);
    const void *fn = fmt4 ? (const void *)k_down_wide<4> : (const void *)k_down_wide<3>;
    if (set_lds(fn, ld)) return -1;
    const int shc = (T + kSharedBlockTokens - 1) / kSharedBlockTokens;
    const int nx = (w.H / kTileRows + kWideWaves * kWideDnRt - 1) / (kWideWaves * kWideDnRt);
    if (fmt4)
      k_down_wide<4><<<nx * (shc + slots), 64 * kWideWaves, ld, st>>>(w, L->xl, shc, L->sh_dq, L->sh_ds, hg, nx, slots);
    else
      k_down_wide<3><<<nx * (shc + slots), 64 * kWideWaves, ld, st>>>(w, L->xl, shc, L->sh_dq, L->sh_ds, hg, nx, slots);
  } else if (fmt4) {
    dn_split ? k_down_split<4><<<dim3(ds_blocks_x, slots + sh_chunks), 512, 0, st>>>(w, L->xl, slots, L->sh_dq, L->sh_ds)
             : k_down<4><<<dim3(dn_blocks_x, slots + sh_chunks), 256, 0, st>>>(w, L->xl, slots, L->sh_dq, L->sh_ds);
  } else {
    dn_split ? k_down_split<3><<<dim3(ds_blocks_x, slots + sh_chunks), 512, 0, st>>>(w, L->xl, slots, L->sh_dq, L->sh_ds)
             : k_down<3><<<dim3(dn_blocks_x, slots + sh_chunks), 256, 0, st>>>(w, L->xl, slots, L->sh_dq, L->sh_ds);
  }
  mark(ctx, 6);
  prof_mark(ctx, kStageRoutedDown);
  k_combine<<<dim3((w.H + 255) / 256, T), 256, 0, st>>>(w, y, route_idx, route_weight);
  mark(ctx, 7);
  prof_mark(ctx, kStageReduce);
  int rc = launch_status("coli_cuda_moe_forward");
  stage_accumulate(ctx);
  return rc;
}

// Token counts a stack call runs through the persistent kernel token by token
// (S397, 60 layers: 1.96 ms per token, against 5.18 ms for a 2-token, 5.41 ms
// for a 3-token and 5.97 ms for a 4-token many-token step; S35, 40 layers:
// 0.81 ms per token, against 2.20, 2.24 and 2.33 ms).
#ifndef SW_STACK_SEQ_TOKENS
#define SW_STACK_SEQ_TOKENS 2
#endif
constexpr int kStackSeqTokens = SW_STACK_SEQ_TOKENS;

extern "C" int coli_cuda_moe_forward_layers(ColiCuda *ctx, ColiMoeLayer *const *layers, int n_layers, float *y,
                                            const float *x, int tokens, size_t xs, size_t ys) {
  if (!ctx || !layers || !y || !x || n_layers <= 0)
    return fail_arg("coli_cuda_moe_forward_layers: invalid argument");
  for (int l = 0; l < n_layers; l++)
    if (!layers[l]) return fail_arg("coli_cuda_moe_forward_layers: null layer %d", l);
  if (!prof_active(ctx)) prof_open(ctx);
  // One to kStackSeqTokens tokens: the persistent decode kernel once per token
  // (each launch runs every layer); below that count its fixed per-layer cost
  // is less than the many-token step's.  Token t's rows are x + t*H, y + t*H.
  if (tokens >= 1 && tokens <= kStackSeqTokens && !ctx->moe_generic_only && ctx->moe_decode_mode == 0) {
    const size_t H = (size_t)layers[0]->sh.hidden;
    int rc = 0;
    for (int t = 0; t < tokens && rc == 0; t++) rc = stack_step(ctx, layers, n_layers, y + t * H, ys, x + t * H, xs, nullptr, nullptr);
    if (rc <= 0) return rc;
  }
  for (int l = 0; l < n_layers; l++)
    if (coli_cuda_moe_forward(ctx, layers[l], y + (size_t)l * ys, x + (size_t)l * xs, tokens, nullptr, nullptr))
      return -1;
  return 0;
}

// x[i] += y[i] (the residual add after the MoE, c/qwen.c:4596)
__global__ static void k_residual_add(float *x, const float *y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] += y[i];
}

extern "C" int coli_cuda_moe_block_ex(ColiCuda *ctx, ColiMoeLayer *L, float *x, const float *norm_weight,
                                      float eps, int tokens, float *hidden, int *route_idx, float *route_weight) {
  if (!ctx || !L || !x || !norm_weight || tokens <= 0) return fail_arg("coli_cuda_moe_block: invalid argument");
  const size_t H = (size_t)L->sh.hidden, n = (size_t)tokens * H;
  if (ensure_scratch(ctx, kScrBlock, 2 * n * sizeof(float), "MoE block scratch")) return -1;
  float *xn = hidden ? hidden : (float *)ctx->scratch[kScrBlock], *y = (float *)ctx->scratch[kScrBlock] + n;
  // the serial sum of squares of the CPU path, so the router sees its n bit for bit
  if (coli_cuda_rmsnorm_zero_batch(ctx, xn, x, norm_weight, tokens, (int)H, eps) ||
      coli_cuda_moe_forward(ctx, L, y, xn, tokens, route_idx, route_weight))
    return -1;
  k_residual_add<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(x, y, n);
  return launch_status("coli_cuda_moe_block");
}

extern "C" int coli_cuda_moe_block(ColiCuda *ctx, ColiMoeLayer *L, float *x, const float *norm_weight, float eps,
                                   int tokens) {
  return coli_cuda_moe_block_ex(ctx, L, x, norm_weight, eps, tokens, nullptr, nullptr, nullptr);
}

__global__ static void k_synth_x(float *x, int rows, int cols, uint64_t seed, uint32_t layer, int step0) {
  int r = blockIdx.y;
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= cols || r >= rows) return;
  x[(size_t)r * cols + i] = sw_normal(sw_key(seed, layer, (uint32_t)(step0 + r), SW_T_X), (uint64_t)i);
}

extern "C" int coli_cuda_synth_activations(ColiCuda *ctx, float *x, int rows, int cols, unsigned long long seed,
                                           int layer, int step0) {
  if (!ctx || !x || rows <= 0 || cols <= 0 || rows > 65535)
    return fail_arg("coli_cuda_synth_activations: invalid argument");
  k_synth_x<<<dim3((cols + 255) / 256, rows), 256, 0, ctx->stream>>>(x, rows, cols, seed, (uint32_t)layer, step0);
  return launch_status("coli_cuda_synth_activations");
}

extern "C" int coli_cuda_moe_stage_timing(ColiCuda *ctx, int enable) {
  if (!ctx) return fail_arg("coli_cuda_moe_stage_timing: null context");
  if (enable) {
    for (int i = 0; i < 8; i++)
      if (!ctx->moe_event[i]) {
        hipError_t e = hipEventCreate(&ctx->moe_event[i]);
        if (e != hipSuccess) return fail_hip("hipEventCreate", e);
      }
    memset(ctx->moe_ms, 0, sizeof(ctx->moe_ms));
    ctx->moe_calls = 0;
    memset(ctx->moe_dec_ms, 0, sizeof(ctx->moe_dec_ms));
    ctx->moe_dec_calls = 0;
  }
  ctx->moe_timing = enable ? 1 : 0;
  return 0;
}

extern "C" int coli_cuda_moe_stage_times(ColiCuda *ctx, double ms[8], unsigned long long *calls) {
  if (!ctx || !ms || !calls) return fail_arg("coli_cuda_moe_stage_times: null argument");
  memcpy(ms, ctx->moe_ms, sizeof(ctx->moe_ms));
  *calls = ctx->moe_calls;
  return 0;
}

extern "C" int coli_cuda_moe_decode_times(ColiCuda *ctx, double ms[3], unsigned long long *calls) {
  if (!ctx || !ms || !calls) return fail_arg("coli_cuda_moe_decode_times: null argument");
  memcpy(ms, ctx->moe_dec_ms, sizeof(ctx->moe_dec_ms));
  *calls = ctx->moe_dec_calls;
  return 0;
}

extern "C" int coli_cuda_moe_set_item_tokens(ColiCuda *ctx, int tokens) {
  if (!ctx || (tokens != 0 && tokens != kMaxTokensPerItem && tokens != kWideTokens))
    return fail_arg("coli_cuda_moe_set_item_tokens: %d (0 automatic, %d or %d)", tokens, kMaxTokensPerItem,
                    kWideTokens);
  ctx->moe_item_tokens = tokens;
  return 0;
}

extern "C" int coli_cuda_moe_set_decode_kernels(ColiCuda *ctx, int mode) {
  if (!ctx || mode < 0 || mode > 2) return fail_arg("coli_cuda_moe_set_decode_kernels: invalid argument");
  ctx->moe_generic_only = mode == 0 ? 1 : 0;
  ctx->moe_decode_mode = mode == 2 ? 1 : 0;
  return 0;
}

extern "C" int coli_cuda_moe_route_stats(ColiCuda *ctx, ColiMoeLayer *L, unsigned long long *tokens,
                                         unsigned long long *fallbacks) {
  if (!ctx || !L || !tokens || !fallbacks) return fail_arg("coli_cuda_moe_route_stats: null argument");
  unsigned long long s[3];
  if (coli_cuda_moe_route_stats_full(ctx, L, s)) return -1;
  *tokens = s[0];
  *fallbacks = s[1];
  return 0;
}

extern "C" int coli_cuda_moe_route_stats_full(ColiCuda *ctx, ColiMoeLayer *L, unsigned long long out[3]) {
  if (!ctx || !L || !out) return fail_arg("coli_cuda_moe_route_stats_full: null argument");
  hipError_t e = hipMemcpyAsync(out, L->stats, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return fail_hip("coli_cuda_moe_route_stats_full", e);
  return 0;
}

extern "C" int coli_cuda_router_topk(ColiCuda *ctx, const float *logits, int tokens, int experts, int topk,
                                     int *idx, float *weight) {
  if (!ctx || !logits || !idx || !weight || tokens <= 0 || experts <= 0 || experts > 4096 || topk <= 0 ||
      topk > kMaxTopK)
    return fail_arg("coli_cuda_router_topk: invalid argument");
  k_router_topk_logits<<<tokens, 512, 0, ctx->stream>>>(logits, experts, topk, idx, weight);
  return launch_status("coli_cuda_router_topk");
}

extern "C" int coli_cuda_moe_bucket(ColiCuda *ctx, const int *idx, int tokens, int topk, int experts, int *offsets,
                                    int *token, int *slot) {
  if (!ctx || !idx || !offsets || !token || !slot || tokens <= 0 || topk <= 0 || experts <= 0 || experts > 4096)
    return fail_arg("coli_cuda_moe_bucket: invalid argument");
  if (tokens > tokens_per_step(experts))
    return fail_arg("coli_cuda_moe_bucket: %d tokens x %d experts exceed one workgroup's bucketing map "
                    "(at most %d tokens for %d experts)",
                    tokens, experts, tokens_per_step(experts), experts);
  size_t R = (size_t)tokens * topk;
  size_t need = R * 4 + (R + experts) * 16 + 256;
  if (ensure_scratch(ctx, kScrRoutes, need, "bucket scratch")) return -1;
  char *b = (char *)ctx->scratch[kScrRoutes];
  int *pos = (int *)b;
  int4 *items = (int4 *)(b + ((R * 4 + 15) & ~(size_t)15));
  int *nitems = (int *)(b + need - 64);
  const size_t lds = bucket_lds_bytes(experts, tokens);
  if (set_lds((const void *)k_bucket_only, lds)) return -1;
  k_bucket_only<<<1, 1024, lds, ctx->stream>>>(idx, tokens, topk, experts, offsets, token, slot, pos, items,
                                                nitems);
  return launch_status("coli_cuda_moe_bucket");
}
