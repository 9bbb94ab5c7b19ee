// Device helpers shared by the gfx950 kernels: bit-exact replicas of the host
// arithmetic the reference relies on, wave64 reductions and the int8 MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sw {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// expf, bit-identical to glibc 2.35's expf (the libm the reference links) on
// every non-positive float -- the whole domain of router_topk's softmax
// (logit - max <= 0) and of sigmoidf_stable (expf(-|x|)), c/qwen.c:307, 3423.
//
// Method: the published table-driven scheme of ARM optimized-routines that
// glibc uses for expf (sysdeps/ieee754/flt-32/e_expf.c): x*N/ln2 = k + r with
// N = 32, 2^(k/N) from a 32-entry table of correctly rounded 2^(i/32), and a
// cubic in r evaluated in double, rounded to float once.  The table is
// bits(2^(i/32)) - (i << 47); the coefficients are the published minimax
// values.  glibc's x86-64 build with FMA (the ifunc chosen on every FMA host)
// fuses the reduction r = x*N/ln2 - k; that variant is restated here with
// explicit fma and was checked equal to host expf on all 2^31 non-positive
// floats.
// ---------------------------------------------------------------------------
__device__ __constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,
    0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,
    0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,
    0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,
    0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,
    0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,
    0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,
    0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,
    0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

// The table may be passed in: a kernel that keeps a copy in LDS reads it
// without waiting behind its own outstanding global loads.
__device__ __forceinline__ float expf_glibc_t(float x, const uint64_t *tab) {
  // Special cases first (glibc: NaN propagates, overflow -> inf,
  // x < -0x1.9fe368p6 underflows to +0).
  if (!(x == x)) return x + x;
  if (x > 0x1.62e42ep6f) return __builtin_huge_valf();
  if (x < -0x1.9fe368p6f) return 0.0f;
  constexpr double kN = 32.0;
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
  double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  double r = __builtin_fma(kInvLn2N, xd, -kd);
  uint64_t t = tab[ki & 31];
  t += ki << (52 - 5);
  double s = __builtin_bit_cast(double, t);
  double z = __builtin_fma(kC0, r, kC1);
  double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_t(x, kExp2Tab); }

// sigmoidf_stable / siluf, c/qwen.c:307-308, bit-exact with glibc expf.
__device__ __forceinline__ float sigmoid_ref_t(float x, const uint64_t *tab) {
  if (x >= 0.0f) {
    float z = expf_glibc_t(-x, tab);
    return 1.0f / (1.0f + z);
  }
  float z = expf_glibc_t(x, tab);
  return z / (1.0f + z);
}
__device__ __forceinline__ float sigmoid_ref(float x) { return sigmoid_ref_t(x, kExp2Tab); }
__device__ __forceinline__ float silu_ref_t(float x, const uint64_t *tab) { return x * sigmoid_ref_t(x, tab); }
__device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// exclusive prefix sum over the wave (lane order)
__device__ __forceinline__ double wave_exclusive_scan(double v, int lane) {
  double inc = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    double n = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += n;
  }
  return inc - v;
}

// ---------------------------------------------------------------------------
// int8 MFMA: C[16x16] += A[16x64] * B[64x16], exact int32.
// Lane l supplies A row (l%16), B column (l%16), both for the k-slice (l/16)
// (16 bytes each); C lane l holds rows 4*(l/16)+i, column l%16.
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// DPP wave64 all-reductions: four intra-row steps (quad_perm 1032, 2301,
// row_half_mirror, row_mirror) leave each 16-lane row's total in every lane
// of the row; row_bcast15 / row_bcast31 fold the rows into lane 63, which is
// read back as a wave-uniform value.  No LDS traffic, ~6 VALU ops.
// ---------------------------------------------------------------------------
#define SW_DPP_I(old, v, ctrl, rm, bc) __builtin_amdgcn_update_dpp((old), (v), (ctrl), (rm), 0xF, (bc))
#define SW_DPP_F(old, v, ctrl, rm, bc) \
  __builtin_bit_cast(float, SW_DPP_I(__builtin_bit_cast(int, (float)(old)), __builtin_bit_cast(int, (v)), ctrl, rm, bc))

__device__ __forceinline__ float readlane63(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += SW_DPP_F(0.0f, v, 0xB1, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x4E, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x141, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x140, 0xF, true);
  v += SW_DPP_F(0.0f, v, 0x142, 0xA, false);
  v += SW_DPP_F(0.0f, v, 0x143, 0xC, false);
  return readlane63(v);
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  const float ninf = -__builtin_huge_valf();
  v = fmaxf(v, SW_DPP_F(ninf, v, 0xB1, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x4E, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x141, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x140, 0xF, true));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x142, 0xA, false));
  v = fmaxf(v, SW_DPP_F(ninf, v, 0x143, 0xC, false));
  return readlane63(v);
}

__device__ __forceinline__ int wave_sum_dpp(int v) {
  v += SW_DPP_I(0, v, 0xB1, 0xF, true);
  v += SW_DPP_I(0, v, 0x4E, 0xF, true);
  v += SW_DPP_I(0, v, 0x141, 0xF, true);
  v += SW_DPP_I(0, v, 0x140, 0xF, true);
  v += SW_DPP_I(0, v, 0x142, 0xA, false);
  v += SW_DPP_I(0, v, 0x143, 0xC, false);
  return __builtin_amdgcn_readlane(v, 63);
}

#define SW_DPP_D_STEP(v, ctrl, rm, bc)                                              \
  {                                                                                 \
    int lo_ = SW_DPP_I(0, (int)__double2loint(v), ctrl, rm, bc);                   \
    int hi_ = SW_DPP_I(0, (int)__double2hiint(v), ctrl, rm, bc);                   \
    v += __hiloint2double(hi_, lo_);                                                \
  }

__device__ __forceinline__ double wave_sum_dpp(double v) {
  SW_DPP_D_STEP(v, 0xB1, 0xF, true);
  SW_DPP_D_STEP(v, 0x4E, 0xF, true);
  SW_DPP_D_STEP(v, 0x141, 0xF, true);
  SW_DPP_D_STEP(v, 0x140, 0xF, true);
  SW_DPP_D_STEP(v, 0x142, 0xA, false);
  SW_DPP_D_STEP(v, 0x143, 0xC, false);
  int lo = __builtin_amdgcn_readlane((int)__double2loint(v), 63);
  int hi = __builtin_amdgcn_readlane((int)__double2hiint(v), 63);
  return __hiloint2double(hi, lo);
}

// inclusive scan of a double over the wave in lane order: row_shr 1, 2, 4, 8
// within each 16-lane row, then row_bcast 15 and 31 carry the row totals
__device__ __forceinline__ double wave_incl_scan_dpp(double v) {
  SW_DPP_D_STEP(v, 0x111, 0xF, true);
  SW_DPP_D_STEP(v, 0x112, 0xF, true);
  SW_DPP_D_STEP(v, 0x114, 0xF, true);
  SW_DPP_D_STEP(v, 0x118, 0xF, true);
  SW_DPP_D_STEP(v, 0x142, 0xA, false);
  SW_DPP_D_STEP(v, 0x143, 0xC, false);
  return v;
}
// largest double over the wave (every lane), by DPP
__device__ __forceinline__ double wave_max_dpp(double v) {
#define SW_DPP_D_MAX(ctrl, rm, bc)                                                      \
  {                                                                                     \
    const int lo_ = SW_DPP_I((int)__double2loint(v), (int)__double2loint(v), ctrl, rm, bc); \
    const int hi_ = SW_DPP_I((int)__double2hiint(v), (int)__double2hiint(v), ctrl, rm, bc); \
    v = fmax(v, __hiloint2double(hi_, lo_));                                            \
  }
  SW_DPP_D_MAX(0xB1, 0xF, false);
  SW_DPP_D_MAX(0x4E, 0xF, false);
  SW_DPP_D_MAX(0x141, 0xF, false);
  SW_DPP_D_MAX(0x140, 0xF, false);
  SW_DPP_D_MAX(0x142, 0xA, false);
  SW_DPP_D_MAX(0x143, 0xC, false);
#undef SW_DPP_D_MAX
  const int lo = __builtin_amdgcn_readlane((int)__double2loint(v), 63);
  const int hi = __builtin_amdgcn_readlane((int)__double2hiint(v), 63);
  return __hiloint2double(hi, lo);
}
__device__ __forceinline__ double readlane_d63(double v) {
  const int lo = __builtin_amdgcn_readlane((int)__double2loint(v), 63);
  const int hi = __builtin_amdgcn_readlane((int)__double2hiint(v), 63);
  return __hiloint2double(hi, lo);
}

// s = rn(s + p[i]) for i < m in order, from s (the reference's serial chain
// over precomputed products), by one lane, m % 64 == 0: the LDS reads of the next
// 32 terms are issued before the adds of the current 32, so the chain runs at
// the rate of its dependent adds.
__device__ __forceinline__ void add32(float &s, const float4 (&v)[8]) {
#pragma unroll
  for (int k = 0; k < 8; k++) {
    s = __fadd_rn(s, v[k].x);
    s = __fadd_rn(s, v[k].y);
    s = __fadd_rn(s, v[k].z);
    s = __fadd_rn(s, v[k].w);
  }
}
__device__ __forceinline__ float serial_sum_lds(const float *p, int m, float s = 0.0f) {
  if (m <= 0) return s;
  float4 a[8], b[8];
#pragma unroll
  for (int k = 0; k < 8; k++) a[k] = ((const float4 *)p)[k];
  for (int i = 0; i < m; i += 64) {
#pragma unroll
    for (int k = 0; k < 8; k++) b[k] = ((const float4 *)(p + i + 32))[k];
    add32(s, a);
    if (i + 64 < m) {
#pragma unroll
      for (int k = 0; k < 8; k++) a[k] = ((const float4 *)(p + i + 64))[k];
    }
    add32(s, b);
  }
  return s;
}

// largest unsigned value over the wave; rows a step leaves out keep 0, the
// identity of the maximum, and lane 63 ends with the whole wave's maximum
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
#define SW_U32_STEP(ctrl, rm, bc)                                         \
  {                                                                       \
    const unsigned o_ = (unsigned)SW_DPP_I(0, (int)v, ctrl, rm, bc);      \
    v = o_ > v ? o_ : v;                                                  \
  }
  SW_U32_STEP(0xB1, 0xF, true);
  SW_U32_STEP(0x4E, 0xF, true);
  SW_U32_STEP(0x141, 0xF, true);
  SW_U32_STEP(0x140, 0xF, true);
  SW_U32_STEP(0x142, 0xA, false);
  SW_U32_STEP(0x143, 0xC, false);
#undef SW_U32_STEP
  return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

// largest 64-bit key over the wave (keys encode value and index): the
// largest high word, then the largest low word among the lanes holding it
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
  const unsigned hi = wave_max_u32((unsigned)(k >> 32));
  const unsigned lo = wave_max_u32((unsigned)(k >> 32) == hi ? (unsigned)k : 0u);
  return ((unsigned long long)hi << 32) | lo;
}

// Row shift within each 16-lane row: lane l receives lane l-1 (lane 0 of the
// row receives 0).
__device__ __forceinline__ float dpp_row_shr1(float v) {
  int r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xF, 0xF, false);
  return __builtin_bit_cast(float, r);
}

}  // namespace sw
