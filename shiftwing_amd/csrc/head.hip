// The output head on gfx950: the final norm and the int8 lm_head projection
// of the reference's decode and prefill output (c/qwen.c:4505-4516,
// 4613-4616; the device glue cuda_resident_output_try, 1097-1124), with the
// CPU path's arithmetic bit for bit:
//   n = rmsnorm_zero(x, norm_w): ms = serial fp32 sum of rn(x_i*x_i) in
//       element order, r = 1/sqrtf(ms/n + eps), n_i = (x_i*r)*(1+w_i)
//       (c/qwen.c:1780-1784);
//   logits[v] = ((float)dot(q_v, xq) * scale[v]) * sx, xq = qrow_i8(n): the
//       IDOT of qmat_mul_ex / qmat_mul_batch for an int8 matrix
//       (c/qwen.c:1696-1705, 1765-1768, 3313-3319; allow_idot = 1 at 4512-4513
//       and 4616).
// The projection streams the vocab x hidden int8 matrix once per group of up
// to four tokens (HBM-bound: 1.02 GB for 248,320 x 4096).  Each lane keeps
// its 16-byte column chunks of the quantised activations in registers; a
// wave takes kHeadRows rows (one: 1, 2, 4 and 8 measured 5,750, 5,680, 5,520
// and 5,420 calls/s at S397), loads every chunk of them before the first
// dot, and reduces the exact int32 sums across the wave by DPP.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sw_backend.h"
#include "sw_device.h"

using namespace sw;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// rmsnorm_zero then qrow_i8, one token per block.  The sum of squares is the
// reference's serial chain, run by one thread over products computed in
// parallel (each product rounds once, as x[i]*x[i] does before the add).
__global__ __launch_bounds__(256) void k_head_norm(signed char *xq, float *sx, float *hidden, const float *x,
                                                   const float *w, int n, float eps, int pitch) {
  extern __shared__ float hp[];  // [n]: squares, then the normalised row
  __shared__ float s_r, red[4];
  const float *xs = x + (size_t)blockIdx.x * n;
  for (int i = threadIdx.x; i < n; i += blockDim.x) hp[i] = xs[i] * xs[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    // LDS reads of the next 32 squares issued before the current 32 adds
    const int n64 = n / 64 * 64;
    float ms = serial_sum_lds(hp, n64);
    for (int i = n64; i < n; i++) ms = __fadd_rn(ms, hp[i]);
    s_r = 1.0f / sqrtf(ms / (float)n + eps);
  }
  __syncthreads();
  const float r = s_r;
  float m = 0.0f;
  float *hs = hidden ? hidden + (size_t)blockIdx.x * n : nullptr;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = (xs[i] * r) * (1.0f + w[i]);
    hp[i] = v;
    if (hs) hs[i] = v;
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = a / 127.0f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.0f / s;
  if (threadIdx.x == 0) sx[blockIdx.x] = s;
  signed char *qs = xq + (size_t)blockIdx.x * pitch;
  for (int i = threadIdx.x; i < pitch; i += blockDim.x) qs[i] = i < n ? (signed char)__builtin_rintf(hp[i] * inv) : 0;
}

#ifndef SW_HEAD_DPP
#define SW_HEAD_DPP 1
#endif
#ifndef SW_HEAD_ROWS
#define SW_HEAD_ROWS 1
#endif
constexpr int kHeadRows = SW_HEAD_ROWS;  // rows per wave

__device__ __forceinline__ int dot16(const v4i w, const v4i x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  return __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
}

// NB tokens, NCH chunks of 1024 columns (64 lanes x 16 bytes) per row.
// grid ceil(rows / (4 * kHeadRows)), 256 threads.  Requires cols % 16 == 0,
// row_bytes % 16 == 0, q 16-byte aligned and cols <= 1024 * NCH.
template <int NB, int NCH>
__global__ __launch_bounds__(256) void k_head_q8(float *logits, const signed char *xq, const float *sx, int pitch,
                                                 const signed char *q, const float *scales, int rows, int cols,
                                                 int row_bytes) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kHeadRows;
  if (r0 >= rows) return;
  v4i wv[kHeadRows][NCH];
#pragma unroll
  for (int i = 0; i < kHeadRows; i++) {
    const int row = r0 + i < rows ? r0 + i : rows - 1;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      const int col = 1024 * c + 16 * lane;
      wv[i][c] = col < cols ? __builtin_nontemporal_load((const v4i *)(q + (size_t)row * row_bytes + col))
                            : v4i{0, 0, 0, 0};
    }
  }
  v4i xr[NB][NCH];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      const int col = 1024 * c + 16 * lane;
      xr[b][c] = col < cols ? *(const v4i *)(xq + (size_t)b * pitch + col) : v4i{0, 0, 0, 0};
    }
#pragma unroll
  for (int i = 0; i < kHeadRows; i++) {
    const int row = r0 + i;
#pragma unroll
    for (int b = 0; b < NB; b++) {
      int acc = 0;
#pragma unroll
      for (int c = 0; c < NCH; c++) acc = dot16(wv[i][c], xr[b][c], acc);
#if SW_HEAD_DPP
      acc = wave_sum_dpp(acc);
#else
      acc = wave_sum_i(acc);
#endif
      if (lane == 0 && row < rows) logits[(size_t)b * rows + row] = ((float)acc * scales[row]) * sx[b];
    }
  }
}

// any shape: one wave per (row, token), dword dots where aligned
__global__ __launch_bounds__(256) void k_head_q8_any(float *logits, const signed char *xq, const float *sx,
                                                     int pitch, const signed char *q, const float *scales,
                                                     int rows, int cols, int row_bytes) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y;
  if (row >= rows) return;
  const signed char *w = q + (size_t)row * row_bytes, *xb = xq + (size_t)b * pitch;
  int acc = 0;
  for (int j = lane; j < cols; j += 64) acc += (int)w[j] * (int)xb[j];
  acc = wave_sum_i(acc);
  if (lane == 0) logits[(size_t)b * rows + row] = ((float)acc * scales[row]) * sx[b];
}

template <int NB>
int launch_head(int nch, float *logits, const signed char *xq, const float *sx, int pitch, const signed char *q,
                const float *scales, int rows, int cols, int row_bytes, hipStream_t st) {
  const unsigned blocks = (unsigned)((rows + 4 * kHeadRows - 1) / (4 * kHeadRows));
  switch (nch) {
    case 1: k_head_q8<NB, 1><<<blocks, 256, 0, st>>>(logits, xq, sx, pitch, q, scales, rows, cols, row_bytes); break;
    case 2: k_head_q8<NB, 2><<<blocks, 256, 0, st>>>(logits, xq, sx, pitch, q, scales, rows, cols, row_bytes); break;
    case 4: k_head_q8<NB, 4><<<blocks, 256, 0, st>>>(logits, xq, sx, pitch, q, scales, rows, cols, row_bytes); break;
    default: k_head_q8<NB, 8><<<blocks, 256, 0, st>>>(logits, xq, sx, pitch, q, scales, rows, cols, row_bytes); break;
  }
  return 0;
}

}  // namespace

extern "C" int coli_cuda_output_head_q8(ColiCuda *ctx, float *logits, float *hidden, const float *x,
                                        const float *norm_w, float eps, int batch, const signed char *q,
                                        const float *scales, int vocab, int cols, int row_bytes) {
  if (!ctx || !logits || !x || !norm_w || !q || !scales || batch <= 0 || vocab <= 0 || cols <= 0 ||
      row_bytes < cols)
    return fail_arg("coli_cuda_output_head_q8: invalid argument");
  if (cols > 16384) return fail_arg("coli_cuda_output_head_q8: hidden %d exceeds 16384", cols);
  const int pitch = (cols + 15) & ~15;
  const size_t qbytes = ((size_t)batch * pitch + 255) & ~(size_t)255;
  if (ensure_scratch(ctx, kScrHead, qbytes + (size_t)batch * sizeof(float), "output head activation allocation"))
    return -1;
  signed char *xq = (signed char *)ctx->scratch[kScrHead];
  float *sx = (float *)((char *)ctx->scratch[kScrHead] + qbytes);
  hipStream_t st = ctx->stream;
  const size_t lds = (size_t)cols * sizeof(float);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)k_head_norm, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail_hip("output head norm attributes", e);
  }
  k_head_norm<<<batch, 256, lds, st>>>(xq, sx, hidden, x, norm_w, cols, eps, pitch);
  const bool fast = cols % 16 == 0 && row_bytes % 16 == 0 && ((uintptr_t)q & 15) == 0 && cols <= 8192;
  const int nch = (cols + 1023) / 1024;
  const int nchp = nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : 8;
  for (int b0 = 0; b0 < batch; b0 += 4) {
    const int nb = batch - b0 < 4 ? batch - b0 : 4;
    float *lg = logits + (size_t)b0 * vocab;
    const signed char *xb = xq + (size_t)b0 * pitch;
    const float *sb = sx + b0;
    if (!fast) {
      k_head_q8_any<<<dim3((vocab + 3) / 4, nb), 256, 0, st>>>(lg, xb, sb, pitch, q, scales, vocab, cols, row_bytes);
      continue;
    }
    switch (nb) {
      case 1: launch_head<1>(nchp, lg, xb, sb, pitch, q, scales, vocab, cols, row_bytes, st); break;
      case 2: launch_head<2>(nchp, lg, xb, sb, pitch, q, scales, vocab, cols, row_bytes, st); break;
      case 3: launch_head<3>(nchp, lg, xb, sb, pitch, q, scales, vocab, cols, row_bytes, st); break;
      default: launch_head<4>(nchp, lg, xb, sb, pitch, q, scales, vocab, cols, row_bytes, st); break;
    }
  }
  return launch_status("coli_cuda_output_head_q8");
}
