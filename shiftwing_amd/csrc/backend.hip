// The reference backend's MoE-path compute entry points on gfx950
// (c/backend_cuda.h:42-148): elementwise ops, row GEMVs over the container
// layouts, the grouped routed-expert calls over caller pointer tables and the
// shared-expert calls.  Arguments, limits and y-overwrite vs y-accumulate
// semantics are the reference's; the kernels are written for wave64 and read
// the container layouts directly (no repack):
//   int4: row stride row_bytes, value i in byte i>>1 (low nibble first),
//         w = (nibble-8)*scale[row*groups + i/group_size];
//   int3: 8 codes per 24-bit little-endian triplet, w = (code-4)*scale;
//   int8: one scale per row.
// The context (memory, streams, profiling) is context.hip; the HBM-resident
// fused MoE step is moe.hip / moe_decode.hip / moe_stack.hip.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "sw_backend.h"
#include "sw_stack.h"
#include "sw_device.h"

using namespace sw;

// ---------------------------------------------------------------------------
// elementwise and small kernels (backend_cuda.h:46-59)
// ---------------------------------------------------------------------------
// rmsnorm_zero (c/qwen.c:1780-1784) with the CPU path's arithmetic bit for
// bit: ms = rn(ms + rn(x_i*x_i)) in element order (the serial chain the
// reference's flags compile), r = 1/sqrtf(ms/n + eps) (correctly rounded
// division and square root), y_i = rn(rn(x_i*r)*rn(1+w_i)).  One block per
// row: the block writes a chunk of squares to LDS, one lane adds them in
// order, the next chunk follows.
constexpr int kNormChunk = 4096;
__global__ __launch_bounds__(256) static void k_rmsnorm_zero(float *y, const float *x, const float *w, int n,
                                                             float eps) {
  __shared__ float sq[kNormChunk];
  __shared__ float s_r;
  const float *xs = x + (size_t)blockIdx.x * n;
  float *ys = y + (size_t)blockIdx.x * n;
  float ms = 0.0f;
  for (int c0 = 0; c0 < n; c0 += kNormChunk) {
    const int m = n - c0 < kNormChunk ? n - c0 : kNormChunk;
    for (int i = threadIdx.x; i < m; i += blockDim.x) sq[i] = __fmul_rn(xs[c0 + i], xs[c0 + i]);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int m64 = m / 64 * 64;
      ms = serial_sum_lds(sq, m64, ms);
      for (int i = m64; i < m; i++) ms = __fadd_rn(ms, sq[i]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) s_r = 1.0f / sqrtf(ms / (float)n + eps);
  __syncthreads();
  const float r = s_r;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ys[i] = __fmul_rn(__fmul_rn(xs[i], r), 1.0f + w[i]);
}

extern "C" int coli_cuda_rmsnorm_zero(ColiCuda *ctx, float *y, const float *x, const float *w, int n,
                                      float eps) {
  if (!ctx || !y || !x || !w || n <= 0) return fail_arg("coli_cuda_rmsnorm_zero: invalid argument");
  k_rmsnorm_zero<<<1, 256, 0, ctx->stream>>>(y, x, w, n, eps);
  return launch_status("k_rmsnorm_zero");
}

extern "C" int coli_cuda_rmsnorm_zero_batch(ColiCuda *ctx, float *y, const float *x, const float *w,
                                            int batch, int n, float eps) {
  if (!ctx || !y || !x || !w || batch <= 0 || n <= 0)
    return fail_arg("coli_cuda_rmsnorm_zero_batch: invalid argument");
  k_rmsnorm_zero<<<batch, 256, 0, ctx->stream>>>(y, x, w, n, eps);
  return launch_status("k_rmsnorm_zero_batch");
}

// one wave per (row, sample); fp32 GEMV y[b,r] = x[b,:] . w[r,:]
__global__ static void k_f32_gemm(float *y, const float *x, const float *w, int rows, int cols) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= rows) return;
  const float *xs = x + (size_t)b * cols, *ws = w + (size_t)row * cols;
  float s = 0.0f;
  for (int i = lane; i < cols; i += 64) s += xs[i] * ws[i];
  s = wave_sum(s);
  if (lane == 0) y[(size_t)b * rows + row] = s;
}

extern "C" int coli_cuda_f32_gemm(ColiCuda *ctx, float *y, const float *x, const float *w, int batch,
                                  int rows, int cols) {
  if (!ctx || !y || !x || !w || batch <= 0 || rows <= 0 || cols <= 0)
    return fail_arg("coli_cuda_f32_gemm: invalid argument");
  k_f32_gemm<<<dim3((rows + 3) / 4, batch), 256, 0, ctx->stream>>>(y, x, w, rows, cols);
  return launch_status("k_f32_gemm");
}

__global__ static void k_sigmoid(float *y, const float *x, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = sigmoid_ref(x[i]);
}
__global__ static void k_silu_mul(float *y, const float *g, const float *u, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = silu_ref(g[i]) * u[i];
}
__global__ static void k_axpy(float *y, const float *x, float a, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += a * x[i];
}
__global__ static void k_sigmoid_axpy(float *y, const float *x, const float *logit, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  float gate = sigmoid_ref(logit[0]);
  if (i < n) y[i] += gate * x[i];
}
__global__ static void k_f32_to_f16(__half *y, const float *x, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = __float2half_rn(x[i]);
}

#define SW_ELEMENTWISE_CHECK(cond, name) \
  if (!(cond)) return fail_arg(name ": invalid argument")

extern "C" int coli_cuda_sigmoid(ColiCuda *ctx, float *y, const float *x, int n) {
  SW_ELEMENTWISE_CHECK(ctx && y && x && n > 0, "coli_cuda_sigmoid");
  k_sigmoid<<<(n + 255) / 256, 256, 0, ctx->stream>>>(y, x, n);
  return launch_status("k_sigmoid");
}
extern "C" int coli_cuda_silu_mul(ColiCuda *ctx, float *y, const float *gate, const float *up, int n) {
  SW_ELEMENTWISE_CHECK(ctx && y && gate && up && n > 0, "coli_cuda_silu_mul");
  k_silu_mul<<<(n + 255) / 256, 256, 0, ctx->stream>>>(y, gate, up, n);
  return launch_status("k_silu_mul");
}
extern "C" int coli_cuda_axpy(ColiCuda *ctx, float *y, const float *x, float scale, int n) {
  SW_ELEMENTWISE_CHECK(ctx && y && x && n > 0, "coli_cuda_axpy");
  k_axpy<<<(n + 255) / 256, 256, 0, ctx->stream>>>(y, x, scale, n);
  return launch_status("k_axpy");
}
extern "C" int coli_cuda_sigmoid_axpy(ColiCuda *ctx, float *y, const float *x, const float *logit, int n) {
  SW_ELEMENTWISE_CHECK(ctx && y && x && logit && n > 0, "coli_cuda_sigmoid_axpy");
  k_sigmoid_axpy<<<(n + 255) / 256, 256, 0, ctx->stream>>>(y, x, logit, n);
  return launch_status("k_sigmoid_axpy");
}
extern "C" int coli_cuda_f32_to_f16(ColiCuda *ctx, unsigned short *y, const float *x, int n) {
  SW_ELEMENTWISE_CHECK(ctx && y && x && n > 0, "coli_cuda_f32_to_f16");
  k_f32_to_f16<<<(n + 255) / 256, 256, 0, ctx->stream>>>((__half *)y, x, n);
  return launch_status("k_f32_to_f16");
}

// ---------------------------------------------------------------------------
// row dots over the container layouts (one wave per output row)
// ---------------------------------------------------------------------------
template <typename XT>
__device__ __forceinline__ float ld(const XT *p, int i);
template <>
__device__ __forceinline__ float ld<float>(const float *p, int i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<__half>(const __half *p, int i) { return __half2float(p[i]); }

// lane partial of sum_i x_i * (nib_i - 8) * s[i/gs] over cols
template <typename XT>
__device__ float lane_dot_q4(const unsigned char *q, const float *s, const XT *x, int cols, int gs,
                             int lane) {
  float acc = 0.0f;
  bool fast = (gs % 8 == 0) && (cols % 8 == 0) && ((((uintptr_t)q) & 3) == 0);
  if (fast) {
    const uint32_t *q32 = (const uint32_t *)q;
    for (int u = lane; u < cols / 8; u += 64) {
      uint32_t w = q32[u];
      int i0 = u * 8;
      float part = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j++) part = __builtin_fmaf(ld(x, i0 + j), (float)((int)((w >> (4 * j)) & 15u) - 8), part);
      acc = __builtin_fmaf(part, s[i0 / gs], acc);
    }
  } else {
    for (int p = lane; p < (cols + 1) / 2; p += 64) {
      int i = 2 * p;
      unsigned char b = q[p];
      acc += ld(x, i) * (float)((int)(b & 15) - 8) * s[i / gs];
      if (i + 1 < cols) acc += ld(x, i + 1) * (float)((int)(b >> 4) - 8) * s[(i + 1) / gs];
    }
  }
  return acc;
}

// lane partial for packed int3 (gs is a multiple of 8, so one scale per triplet)
template <typename XT>
__device__ float lane_dot_q3(const unsigned char *q, const float *s, const XT *x, int cols, int gs,
                             int lane) {
  float acc = 0.0f;
  int triplets = (cols + 7) / 8;
  for (int t = lane; t < triplets; t += 64) {
    const unsigned char *p = q + 3 * t;
    uint32_t w = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16);
    int i0 = 8 * t;
    float part = 0.0f;
    if (i0 + 8 <= cols) {
#pragma unroll
      for (int j = 0; j < 8; j++) part = __builtin_fmaf(ld(x, i0 + j), (float)((int)((w >> (3 * j)) & 7u) - 4), part);
      acc = __builtin_fmaf(part, s[i0 / gs], acc);
    } else {
      for (int j = 0; i0 + j < cols; j++)
        acc += ld(x, i0 + j) * (float)((int)((w >> (3 * j)) & 7u) - 4) * s[(i0 + j) / gs];
    }
  }
  return acc;
}

template <typename XT>
__device__ float lane_dot_q8(const signed char *q, const XT *x, int cols, int lane) {
  float acc = 0.0f;
  for (int i = lane; i < cols; i += 64) acc = __builtin_fmaf(ld(x, i), (float)q[i], acc);
  return acc;
}

template <int BITS, typename XT>
__device__ __forceinline__ float lane_dot_qx(const unsigned char *q, const float *s, const XT *x, int cols,
                                             int gs, int lane) {
  if (BITS == 4) return lane_dot_q4(q, s, x, cols, gs, lane);
  return lane_dot_q3(q, s, x, cols, gs, lane);
}

// y[b,row] = dot (BITS 8: * scale[row]); grid (ceil(rows/4), batch), 256 threads
template <int BITS, typename XT>
__global__ static void k_q_gemm(float *y, const XT *x, const unsigned char *q, const float *scales,
                                int rows, int cols, int gs, int row_bytes, int groups) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= rows) return;
  const XT *xs = x + (size_t)b * cols;
  const unsigned char *qr = q + (size_t)row * row_bytes;
  float v;
  if (BITS == 8)
    v = lane_dot_q8((const signed char *)qr, xs, cols, lane);
  else
    v = lane_dot_qx<BITS>(qr, scales + (size_t)row * groups, xs, cols, gs, lane);
  v = wave_sum(v);
  if (lane == 0) y[(size_t)b * rows + row] = BITS == 8 ? v * scales[row] : v;
}

static int q_args_ok(int bits, const void *y, const void *x, const void *q, const float *s, int batch,
                     int rows, int cols, int gs, int row_bytes, int groups) {
  if (!y || !x || !q || !s || batch <= 0 || rows <= 0 || cols <= 0) return 0;
  if (bits == 8) return row_bytes >= cols;
  int need_groups = (cols + gs - 1) / (gs > 0 ? gs : 1);
  int need_bytes = bits == 4 ? (cols + 1) / 2 : ((cols + 7) / 8) * 3;
  if (gs <= 0 || groups < need_groups || row_bytes < need_bytes) return 0;
  if (bits == 3 && gs % 8) return 0;
  return 1;
}

template <int BITS, typename XT>
static int launch_q_gemm(ColiCuda *ctx, const char *name, float *y, const XT *x, int batch,
                         const unsigned char *q, const float *s, int rows, int cols, int gs,
                         int row_bytes, int groups) {
  if (!ctx || !q_args_ok(BITS, y, x, q, s, batch, rows, cols, gs, row_bytes, groups))
    return fail_arg("%s: invalid argument", name);
  k_q_gemm<BITS, XT><<<dim3((rows + 3) / 4, batch), 256, 0, ctx->stream>>>(y, x, q, s, rows, cols, gs,
                                                                           row_bytes, groups);
  return launch_status(name);
}

extern "C" int coli_cuda_q8_gemv(ColiCuda *ctx, float *y, const float *x, const signed char *q,
                                 const float *scales, int rows, int cols, int row_bytes) {
  return launch_q_gemm<8, float>(ctx, "coli_cuda_q8_gemv", y, x, 1, (const unsigned char *)q, scales, rows,
                                 cols, 0, row_bytes, 0);
}
extern "C" int coli_cuda_q8_gemm(ColiCuda *ctx, float *y, const float *x, int batch, const signed char *q,
                                 const float *scales, int rows, int cols, int row_bytes) {
  return launch_q_gemm<8, float>(ctx, "coli_cuda_q8_gemm", y, x, batch, (const unsigned char *)q, scales,
                                 rows, cols, 0, row_bytes, 0);
}
extern "C" int coli_cuda_q4_gemv(ColiCuda *ctx, float *y, const float *x, const unsigned char *q,
                                 const float *scales, int rows, int cols, int group_size, int row_bytes,
                                 int groups_per_row) {
  return launch_q_gemm<4, float>(ctx, "coli_cuda_q4_gemv", y, x, 1, q, scales, rows, cols, group_size,
                                 row_bytes, groups_per_row);
}
extern "C" int coli_cuda_q4_gemm(ColiCuda *ctx, float *y, const float *x, int batch, const unsigned char *q,
                                 const float *scales, int rows, int cols, int group_size, int row_bytes,
                                 int groups_per_row) {
  return launch_q_gemm<4, float>(ctx, "coli_cuda_q4_gemm", y, x, batch, q, scales, rows, cols, group_size,
                                 row_bytes, groups_per_row);
}
extern "C" int coli_cuda_q4_gemv_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                                     const unsigned char *q, const float *scales, int rows, int cols,
                                     int group_size, int row_bytes, int groups_per_row) {
  return launch_q_gemm<4, __half>(ctx, "coli_cuda_q4_gemv_f16", y, (const __half *)x, 1, q, scales, rows,
                                  cols, group_size, row_bytes, groups_per_row);
}
extern "C" int coli_cuda_q3_gemv(ColiCuda *ctx, float *y, const float *x, const unsigned char *q,
                                 const float *scales, int rows, int cols, int group_size, int row_bytes,
                                 int groups_per_row) {
  return launch_q_gemm<3, float>(ctx, "coli_cuda_q3_gemv", y, x, 1, q, scales, rows, cols, group_size,
                                 row_bytes, groups_per_row);
}
extern "C" int coli_cuda_q3_gemv_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                                     const unsigned char *q, const float *scales, int rows, int cols,
                                     int group_size, int row_bytes, int groups_per_row) {
  return launch_q_gemm<3, __half>(ctx, "coli_cuda_q3_gemv_f16", y, (const __half *)x, 1, q, scales, rows,
                                  cols, group_size, row_bytes, groups_per_row);
}

// ---------------------------------------------------------------------------
// grouped routed experts over caller pointer tables (backend_cuda.h:87-118).
// Tables travel as kernel arguments (<=16 routes per launch), so no per-call
// host->device copy is issued.  Hidden activations stay fp32.
// ---------------------------------------------------------------------------
constexpr int kRoutesPerLaunch = 16;

struct RouteTable {
  const unsigned char *gq[kRoutesPerLaunch];
  const float *gs[kRoutesPerLaunch];
  const unsigned char *uq[kRoutesPerLaunch];
  const float *us[kRoutesPerLaunch];
  const unsigned char *dq[kRoutesPerLaunch];
  const float *ds[kRoutesPerLaunch];
  int xrow[kRoutesPerLaunch];  // activation row used by the route
};

// h[route0 + r, row] = silu(gate . x) * (up . x); grid (ceil(I/4), routes)
template <int BITS, typename XT>
__global__ static void k_grouped_hidden(float *h, int route0, const XT *x, RouteTable t, int I, int H,
                                        int gs, int rb, int groups) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y;
  if (row >= I) return;
  const XT *xs = x + (size_t)t.xrow[r] * H;
  float g = lane_dot_qx<BITS>(t.gq[r] + (size_t)row * rb, t.gs[r] + (size_t)row * groups, xs, H, gs, lane);
  float u = lane_dot_qx<BITS>(t.uq[r] + (size_t)row * rb, t.us[r] + (size_t)row * groups, xs, H, gs, lane);
  g = wave_sum(g);
  u = wave_sum(u);
  if (lane == 0) h[(size_t)(route0 + r) * I + row] = silu_ref(g) * u;
}

// out[route0 + r, row] = down_r . h[route0 + r]; grid (ceil(H/4), routes)
template <int BITS>
__global__ static void k_grouped_down(float *out, int route0, const float *h, RouteTable t, int H, int I,
                                      int gs, int rb, int groups) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y;
  if (row >= H) return;
  const float *hs = h + (size_t)(route0 + r) * I;
  float v = lane_dot_qx<BITS, float>(t.dq[r] + (size_t)row * rb, t.ds[r] + (size_t)row * groups, hs, I, gs,
                                     lane);
  v = wave_sum(v);
  if (lane == 0) out[(size_t)(route0 + r) * H + row] = v;
}

// y[s, row] = sum_j w[s*K+j] * out[s*K+j, row] (j ascending)
__global__ static void k_route_reduce(float *y, const float *out, const float *w, int batch, int K, int H) {
  int row = blockIdx.x * blockDim.x + threadIdx.x, s = blockIdx.y;
  if (row >= H || s >= batch) return;
  float total = 0.0f;
  for (int j = 0; j < K; j++) total += w[s * K + j] * out[(size_t)(s * K + j) * H + row];
  y[(size_t)s * H + row] = total;
}

template <int BITS, typename XT>
static int grouped_mlp(ColiCuda *ctx, const char *name, float *y, const XT *x,
                       const unsigned char *const *gate_q, const float *const *gate_s,
                       const unsigned char *const *up_q, const float *const *up_s,
                       const unsigned char *const *down_q, const float *const *down_s,
                       const float *route_weight, int batch, int K, int H, int I, int gs, int hrb,
                       int hgroups, int drb, int dgroups) {
  int routes = batch * K;
  // route weights are host values (c/backend_cuda.cu:1568); copy them once
  size_t hbytes = (size_t)routes * I * sizeof(float), obytes = (size_t)routes * H * sizeof(float);
  if (ensure_scratch(ctx, kScrHidden, hbytes, "grouped hidden allocation") ||
      ensure_scratch(ctx, kScrRouteOut, obytes, "grouped route output allocation") ||
      ensure_scratch(ctx, kScrWeight, (size_t)routes * sizeof(float), "grouped weight allocation"))
    return -1;
  float *h = (float *)ctx->scratch[kScrHidden];
  float *out = (float *)ctx->scratch[kScrRouteOut];
  float *dw = (float *)ctx->scratch[kScrWeight];
  prof_open(ctx);
  hipError_t e = hipMemcpyAsync(dw, route_weight, (size_t)routes * sizeof(float), hipMemcpyHostToDevice,
                                ctx->stream);
  if (e != hipSuccess) return fail_hip("grouped route weight upload", e);
  prof_mark(ctx, kStageSetup);
  for (int r0 = 0; r0 < routes; r0 += kRoutesPerLaunch) {
    int n = routes - r0 < kRoutesPerLaunch ? routes - r0 : kRoutesPerLaunch;
    RouteTable t;
    memset(&t, 0, sizeof(t));
    for (int i = 0; i < n; i++) {
      t.gq[i] = gate_q[r0 + i];
      t.gs[i] = gate_s[r0 + i];
      t.uq[i] = up_q[r0 + i];
      t.us[i] = up_s[r0 + i];
      t.dq[i] = down_q[r0 + i];
      t.ds[i] = down_s[r0 + i];
      t.xrow[i] = (r0 + i) / K;
      if (!t.gq[i] || !t.gs[i] || !t.uq[i] || !t.us[i] || !t.dq[i] || !t.ds[i])
        return fail_arg("%s: null expert pointer", name);
    }
    k_grouped_hidden<BITS, XT><<<dim3((I + 3) / 4, n), 256, 0, ctx->stream>>>(h, r0, x, t, I, H, gs, hrb,
                                                                             hgroups);
  }
  prof_mark(ctx, kStageRoutedHidden);
  for (int r0 = 0; r0 < routes; r0 += kRoutesPerLaunch) {
    int n = routes - r0 < kRoutesPerLaunch ? routes - r0 : kRoutesPerLaunch;
    RouteTable t;
    memset(&t, 0, sizeof(t));
    for (int i = 0; i < n; i++) {
      t.dq[i] = down_q[r0 + i];
      t.ds[i] = down_s[r0 + i];
    }
    k_grouped_down<BITS><<<dim3((H + 3) / 4, n), 256, 0, ctx->stream>>>(out, r0, h, t, H, I, gs, drb,
                                                                       dgroups);
  }
  prof_mark(ctx, kStageRoutedDown);
  k_route_reduce<<<dim3((H + 255) / 256, batch), 256, 0, ctx->stream>>>(y, out, dw, batch, K, H);
  int st = launch_status(name);
  if (!st) prof_mark(ctx, kStageReduce);
  return st;
}

static int grouped_args_ok(const void *y, const void *x, const void *gq, const void *gs, const void *uq,
                           const void *us, const void *dq, const void *ds, const void *w, int H, int I,
                           int group_size) {
  return y && x && gq && gs && uq && us && dq && ds && w && H > 0 && I > 0 && group_size > 0;
}

#define SW_GROUPED_SINGLE(NAME, BITS, XT)                                                                   \
  extern "C" int NAME(ColiCuda *ctx, float *y, const XT *x, const unsigned char *const *gate_q,            \
                      const float *const *gate_s, const unsigned char *const *up_q,                        \
                      const float *const *up_s, const unsigned char *const *down_q,                        \
                      const float *const *down_s, const float *route_weight, int experts, int hidden,      \
                      int intermediate, int group_size, int hidden_row_bytes, int hidden_groups,           \
                      int down_row_bytes, int down_groups) {                                               \
    if (!ctx || experts <= 0 ||                                                                            \
        !grouped_args_ok(y, x, gate_q, gate_s, up_q, up_s, down_q, down_s, route_weight, hidden,           \
                         intermediate, group_size))                                                        \
      return fail_arg("grouped qx MLP: invalid argument");                                                 \
    if (experts > 32) return fail_arg("grouped expert count exceeds 32");                                  \
    return grouped_mlp<BITS>(ctx, #NAME, y, (const XTYPE_##XT *)x, gate_q, gate_s, up_q, up_s, down_q,     \
                             down_s, route_weight, 1, experts, hidden, intermediate, group_size,          \
                             hidden_row_bytes, hidden_groups, down_row_bytes, down_groups);               \
  }
#define XTYPE_float float
#define XTYPE_unsigned_short __half
typedef unsigned short unsigned_short;

SW_GROUPED_SINGLE(coli_cuda_grouped_q4_mlp_f16, 4, unsigned_short)
SW_GROUPED_SINGLE(coli_cuda_grouped_q3_mlp_f16, 3, unsigned_short)
SW_GROUPED_SINGLE(coli_cuda_grouped_q4_mlp, 4, float)
SW_GROUPED_SINGLE(coli_cuda_grouped_q3_mlp, 3, float)

#define SW_GROUPED_BATCH(NAME, BITS)                                                                        \
  extern "C" int NAME(ColiCuda *ctx, float *y, const unsigned short *x, const unsigned char *const *gate_q, \
                      const float *const *gate_s, const unsigned char *const *up_q,                        \
                      const float *const *up_s, const unsigned char *const *down_q,                        \
                      const float *const *down_s, const float *route_weight, int batch,                    \
                      int experts_per_token, int hidden, int intermediate, int group_size,                 \
                      int hidden_row_bytes, int hidden_groups, int down_row_bytes, int down_groups) {      \
    int routes = batch * experts_per_token;                                                                \
    if (!ctx || batch <= 0 || batch > 8 || experts_per_token <= 0 || routes > 64 ||                        \
        !grouped_args_ok(y, x, gate_q, gate_s, up_q, up_s, down_q, down_s, route_weight, hidden,           \
                         intermediate, group_size))                                                        \
      return fail_arg("grouped qx batch MLP: invalid argument");                                           \
    return grouped_mlp<BITS>(ctx, #NAME, y, (const __half *)x, gate_q, gate_s, up_q, up_s, down_q, down_s, \
                             route_weight, batch, experts_per_token, hidden, intermediate, group_size,    \
                             hidden_row_bytes, hidden_groups, down_row_bytes, down_groups);               \
  }

SW_GROUPED_BATCH(coli_cuda_grouped_q4_mlp_batch_f16, 4)
SW_GROUPED_BATCH(coli_cuda_grouped_q3_mlp_batch_f16, 3)

// ---------------------------------------------------------------------------
// shared expert, int4 (backend_cuda.h:119-127, 140-148)
// ---------------------------------------------------------------------------
// h[b,row] = silu(gate.x_b)*(up.x_b); grid (ceil(I/4), batch)
__global__ static void k_shared_q4_hidden(float *h, const __half *x, const unsigned char *gq,
                                          const float *gs, const unsigned char *uq, const float *us, int I,
                                          int H, int group, int rb, int groups) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= I) return;
  const __half *xs = x + (size_t)b * H;
  float g = lane_dot_q4(gq + (size_t)row * rb, gs + (size_t)row * groups, xs, H, group, lane);
  float u = lane_dot_q4(uq + (size_t)row * rb, us + (size_t)row * groups, xs, H, group, lane);
  g = wave_sum(g);
  u = wave_sum(u);
  if (lane == 0) h[(size_t)b * I + row] = silu_ref(g) * u;
}

// y[b,row] += sigmoid(logit[b]) * (down[row] . h_b); grid (ceil(H/4), batch)
__global__ static void k_shared_q4_down(float *y, const float *h, const unsigned char *dq, const float *ds,
                                        const float *logit, int H, int I, int group, int rb, int groups) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= H) return;
  float v = lane_dot_q4(dq + (size_t)row * rb, ds + (size_t)row * groups, h + (size_t)b * I, I, group, lane);
  v = wave_sum(v);
  if (lane == 0) y[(size_t)b * H + row] += sigmoid_ref(logit[b]) * v;
}

static int shared_q4(ColiCuda *ctx, const char *name, float *y, const unsigned short *x,
                     const unsigned char *gate_q, const float *gate_s, const unsigned char *up_q,
                     const float *up_s, const unsigned char *down_q, const float *down_s,
                     const unsigned char *scale_q, const float *scale_s, int batch, int H, int I, int gs,
                     int hrb, int hgroups, int drb, int dgroups, int srb, int sgroups) {
  if (ensure_scratch(ctx, kScrGate, (size_t)batch * I * sizeof(float), "shared hidden allocation") ||
      ensure_scratch(ctx, kScrUp, (size_t)batch * sizeof(float), "shared gate allocation"))
    return -1;
  float *h = (float *)ctx->scratch[kScrGate];
  float *logit = (float *)ctx->scratch[kScrUp];
  const __half *xh = (const __half *)x;
  k_shared_q4_hidden<<<dim3((I + 3) / 4, batch), 256, 0, ctx->stream>>>(h, xh, gate_q, gate_s, up_q, up_s,
                                                                       I, H, gs, hrb, hgroups);
  prof_mark(ctx, kStageSharedHidden);
  k_q_gemm<4, __half><<<dim3(1, batch), 256, 0, ctx->stream>>>(logit, xh, scale_q, scale_s, 1, H, gs, srb,
                                                               sgroups);
  prof_mark(ctx, kStageSharedScale);
  k_shared_q4_down<<<dim3((H + 3) / 4, batch), 256, 0, ctx->stream>>>(y, h, down_q, down_s, logit, H, I, gs,
                                                                     drb, dgroups);
  int st = launch_status(name);
  if (!st) prof_mark(ctx, kStageSharedDown);
  return st;
}

extern "C" int coli_cuda_shared_q4_mlp_batch_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                                                 const unsigned char *gate_q, const float *gate_s,
                                                 const unsigned char *up_q, const float *up_s,
                                                 const unsigned char *down_q, const float *down_s,
                                                 const unsigned char *scale_q, const float *scale_s,
                                                 int batch, int hidden, int intermediate, int group_size,
                                                 int hidden_row_bytes, int hidden_groups,
                                                 int down_row_bytes, int down_groups, int scale_row_bytes,
                                                 int scale_groups) {
  if (!ctx || !y || !x || !gate_q || !gate_s || !up_q || !up_s || !down_q || !down_s || !scale_q ||
      !scale_s || batch <= 0 || batch > 8 || hidden <= 0 || intermediate <= 0 || group_size <= 0)
    return fail_arg("coli_cuda_shared_q4_mlp_batch_f16: invalid argument");
  return shared_q4(ctx, "coli_cuda_shared_q4_mlp_batch_f16", y, x, gate_q, gate_s, up_q, up_s, down_q,
                   down_s, scale_q, scale_s, batch, hidden, intermediate, group_size, hidden_row_bytes,
                   hidden_groups, down_row_bytes, down_groups, scale_row_bytes, scale_groups);
}

extern "C" int coli_cuda_shared_q4_mlp_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                                           const unsigned char *gate_q, const float *gate_s,
                                           const unsigned char *up_q, const float *up_s,
                                           const unsigned char *down_q, const float *down_s,
                                           const unsigned char *scale_q, const float *scale_s, int hidden,
                                           int intermediate, int group_size, int hidden_row_bytes,
                                           int hidden_groups, int down_row_bytes, int down_groups,
                                           int scale_row_bytes, int scale_groups) {
  if (!ctx || !y || !x || !gate_q || !gate_s || !up_q || !up_s || !down_q || !down_s || !scale_q ||
      !scale_s || hidden <= 0 || intermediate <= 0 || group_size <= 0)
    return fail_arg("coli_cuda_shared_q4_mlp_f16: invalid argument");
  return shared_q4(ctx, "coli_cuda_shared_q4_mlp_f16", y, x, gate_q, gate_s, up_q, up_s, down_q, down_s,
                   scale_q, scale_s, 1, hidden, intermediate, group_size, hidden_row_bytes, hidden_groups,
                   down_row_bytes, down_groups, scale_row_bytes, scale_groups);
}

// ---------------------------------------------------------------------------
// IDOT int8 (c/qwen.c:1696-1705, 1765-1768, 3313-3319), bit-exact
// ---------------------------------------------------------------------------
// qrow_i8 per row of x: xq[b,:] = (int8)rint(x*(1/s)), s = max(amax/127, 1e-12)
__global__ static void k_qrow_i8(signed char *xq, float *sx, const float *x, int n) {
  const float *xs = x + (size_t)blockIdx.x * n;
  signed char *qs = xq + (size_t)blockIdx.x * n;
  __shared__ float red[16];
  float m = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, fabsf(xs[i]));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) a = fmaxf(a, red[i]);
    float s = a / 127.0f;
    if (s < 1e-12f) s = 1e-12f;
    red[0] = s;
    sx[blockIdx.x] = s;
  }
  __syncthreads();
  float inv = 1.0f / red[0];
  for (int i = threadIdx.x; i < n; i += blockDim.x) qs[i] = (signed char)__builtin_rintf(xs[i] * inv);
}

// exact int32 dot of one int8 row with xq; lanes stride 16-byte chunks
__device__ __forceinline__ int lane_idot(const signed char *w, const signed char *xq, int n, int lane) {
  int acc = 0;
  bool fast = ((((uintptr_t)w) | ((uintptr_t)xq)) & 3) == 0;
  int i = 0;
  if (fast) {
    int chunks = n / 4;
    const int *w4 = (const int *)w, *x4 = (const int *)xq;
    for (int c = lane; c < chunks; c += 64) acc = __builtin_amdgcn_sdot4(w4[c], x4[c], acc, false);
    i = chunks * 4;
  }
  for (int j = i + lane; j < n; j += 64) acc += (int)w[j] * (int)xq[j];
  return acc;
}

// y[b,row] = ((float)dot * scale[row]) * sx[b]
__global__ static void k_idot_gemm(float *y, const signed char *xq, const float *sx, const signed char *q,
                                   const float *scales, int rows, int cols, int row_bytes) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= rows) return;
  int d = wave_sum_i(lane_idot(q + (size_t)row * row_bytes, xq + (size_t)b * cols, cols, lane));
  if (lane == 0) y[(size_t)b * rows + row] = (float)d * scales[row] * sx[b];
}

extern "C" int coli_cuda_idot_q8_gemm(ColiCuda *ctx, float *y, const float *x, int batch,
                                      const signed char *q, const float *scales, int rows, int cols,
                                      int row_bytes) {
  if (!ctx || !y || !x || !q || !scales || batch <= 0 || rows <= 0 || cols <= 0 || row_bytes < cols)
    return fail_arg("coli_cuda_idot_q8_gemm: invalid argument");
  size_t qbytes = ((size_t)batch * cols + 255) & ~(size_t)255;
  if (ensure_scratch(ctx, kScrGate, qbytes + (size_t)batch * sizeof(float), "idot activation allocation"))
    return -1;
  signed char *xq = (signed char *)ctx->scratch[kScrGate];
  float *sx = (float *)((char *)ctx->scratch[kScrGate] + qbytes);
  k_qrow_i8<<<batch, 256, 0, ctx->stream>>>(xq, sx, x, cols);
  k_idot_gemm<<<dim3((rows + 3) / 4, batch), 256, 0, ctx->stream>>>(y, xq, sx, q, scales, rows, cols,
                                                                    row_bytes);
  return launch_status("coli_cuda_idot_q8_gemm");
}

// ---------------------------------------------------------------------------
// IDOT GEMM without allocation (coli_cuda_idot_q8_gemm_noalloc).  The
// quantised activations and their scales live in a fixed device array instead
// of context scratch.  In host code `g_noalloc_scratch` names a host-side
// stand-in, not the device array: its device address is fetched once per
// device with hipGetSymbolAddress (at coli_cuda_create, with the device
// current) and only that address is ever handed to kernels.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;  // 1 MiB per device
static __device__ __align__(256) unsigned char g_noalloc_scratch[kNoAllocScratchBytes];

namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kNoAllocMaxDevices];  // device address per device ordinal
}  // namespace

namespace sw {
// Called by coli_cuda_create with ctx->device current.
int noalloc_bind(ColiCuda *ctx) {
  if (ctx->device < 0 || ctx->device >= kNoAllocMaxDevices) return 0;  // entry point reports it
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[ctx->device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_noalloc_scratch));
    if (e != hipSuccess || !p) return fail_hip("hipGetSymbolAddress(no-alloc scratch)", e);
    g_noalloc_ptr[ctx->device] = p;
  }
  ctx->noalloc_scratch = g_noalloc_ptr[ctx->device];
  return 0;
}
}  // namespace sw

extern "C" int coli_cuda_idot_q8_gemm_noalloc(ColiCuda *ctx, float *y, const float *x, int batch,
                                              const signed char *q, const float *scales, int rows, int cols,
                                              int row_bytes) {
  if (!ctx || !y || !x || !q || !scales || batch <= 0 || rows <= 0 || cols <= 0 || row_bytes < cols ||
      batch > 65535)
    return fail_arg("coli_cuda_idot_q8_gemm_noalloc: invalid argument");
  const size_t qbytes = ((size_t)batch * (size_t)cols + 255) & ~(size_t)255;
  const size_t need = qbytes + (size_t)batch * sizeof(float);
  if (need > kNoAllocScratchBytes)
    return fail_arg("coli_cuda_idot_q8_gemm_noalloc: batch x cols = %d x %d needs %zu scratch bytes, "
                    "the fixed scratch holds %zu",
                    batch, cols, need, kNoAllocScratchBytes);
  if (!ctx->noalloc_scratch)
    return fail_arg("coli_cuda_idot_q8_gemm_noalloc: no scratch address for device %d", ctx->device);
  // Every byte read below is written first by k_qrow_i8 of this call, so
  // nothing is cleared; calls overlapping on one device share the array.
  signed char *xq = (signed char *)ctx->noalloc_scratch;
  float *sx = (float *)((unsigned char *)ctx->noalloc_scratch + qbytes);
  k_qrow_i8<<<batch, 256, 0, ctx->stream>>>(xq, sx, x, cols);
  k_idot_gemm<<<dim3((rows + 3) / 4, batch), 256, 0, ctx->stream>>>(y, xq, sx, q, scales, rows, cols,
                                                                    row_bytes);
  return launch_status("coli_cuda_idot_q8_gemm_noalloc");
}

// shared int8 expert for the reference's batched call (backend_cuda.h:128-139):
// fp32 activations x int8 rows, the same row dot as coli_cuda_q8_gemv, so a
// batch equals per-token q8_gemv + silu_mul + q8_gemv calls bit for bit (the
// reference's batch-vs-single contract, c/tests/test_backend_cuda.c:487-531).
// The CPU path's IDOT arithmetic is coli_cuda_idot_q8_gemm and the fused MoE
// step, which match c/qwen.c:1765-1768 bit for bit.
//
// y[b,row] += ((down[row] . h_b) * ds[row]) * sample_scale[b]
__global__ static void k_q8_down_scaled_add(float *y, const float *h, const signed char *dq, const float *ds,
                                            int drb, const float *sample_scale, int H, int I) {
  int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= H) return;
  float v = wave_sum(lane_dot_q8(dq + (size_t)row * drb, h + (size_t)b * I, I, lane));
  if (lane == 0) y[(size_t)b * H + row] += v * ds[row] * sample_scale[b];
}

static int shared_q8(ColiCuda *ctx, float *y, const float *x, const float *scale, int device_scale,
                     const signed char *gate_q, const float *gate_s, int grb, const signed char *up_q,
                     const float *up_s, int urb, const signed char *down_q, const float *down_s, int drb,
                     int batch, int H, int I) {
  if (!ctx || !y || !x || !scale || !gate_q || !gate_s || !up_q || !up_s || !down_q || !down_s ||
      batch <= 0 || batch > 8 || H <= 0 || I <= 0 || grb < H || urb < H || drb < I)
    return fail_arg("coli_cuda_shared_q8_mlp_batch: invalid argument");
  const size_t gb = (size_t)batch * I * sizeof(float);
  const size_t total = 2 * gb + (size_t)batch * sizeof(float);
  if (ensure_scratch(ctx, kScrGate, total, "shared q8 allocation")) return -1;
  float *g = (float *)ctx->scratch[kScrGate];
  float *u = g + (size_t)batch * I;
  float *dscale = u + (size_t)batch * I;
  const dim3 hid((I + 3) / 4, batch);
  k_q_gemm<8, float><<<hid, 256, 0, ctx->stream>>>(g, x, (const unsigned char *)gate_q, gate_s, I, H, 0, grb, 0);
  k_q_gemm<8, float><<<hid, 256, 0, ctx->stream>>>(u, x, (const unsigned char *)up_q, up_s, I, H, 0, urb, 0);
  k_silu_mul<<<(batch * I + 255) / 256, 256, 0, ctx->stream>>>(g, g, u, batch * I);
  prof_mark(ctx, kStageSharedHidden);
  const float *sc = scale;
  if (!device_scale) {
    hipError_t e = hipMemcpyAsync(dscale, scale, (size_t)batch * sizeof(float), hipMemcpyHostToDevice,
                                  ctx->stream);
    if (e != hipSuccess) return fail_hip("shared q8 scale upload", e);
    sc = dscale;
  }
  prof_mark(ctx, kStageSharedScale);
  k_q8_down_scaled_add<<<dim3((H + 3) / 4, batch), 256, 0, ctx->stream>>>(y, g, down_q, down_s, drb, sc, H, I);
  int st = launch_status("shared batch q8 MLP kernels");
  if (!st) prof_mark(ctx, kStageSharedDown);
  return st;
}

extern "C" int coli_cuda_shared_q8_mlp_batch(ColiCuda *ctx, float *y, const float *x, const float *scale,
                                             const signed char *gate_q, const float *gate_s,
                                             int gate_row_bytes, const signed char *up_q,
                                             const float *up_s, int up_row_bytes,
                                             const signed char *down_q, const float *down_s,
                                             int down_row_bytes, int batch, int hidden, int intermediate) {
  return shared_q8(ctx, y, x, scale, 0, gate_q, gate_s, gate_row_bytes, up_q, up_s, up_row_bytes, down_q,
                   down_s, down_row_bytes, batch, hidden, intermediate);
}

extern "C" int coli_cuda_shared_q8_mlp_batch_device_scale(
    ColiCuda *ctx, float *y, const float *x, const float *device_scale, const signed char *gate_q,
    const float *gate_s, int gate_row_bytes, const signed char *up_q, const float *up_s, int up_row_bytes,
    const signed char *down_q, const float *down_s, int down_row_bytes, int batch, int hidden,
    int intermediate) {
  return shared_q8(ctx, y, x, device_scale, 1, gate_q, gate_s, gate_row_bytes, up_q, up_s, up_row_bytes,
                   down_q, down_s, down_row_bytes, batch, hidden, intermediate);
}
