// Device building blocks of the MoE step shared by the decode path
// (moe_decode.hip) and the many-token path (moe.hip).
//
// Routed-expert tile layout (written by the registration repack): a tile is
// 16 rows x one 128-wide quant group.  Lane l (row l%16, k-slice kb = l/16)
// owns group positions kb*16+[0,16) (MFMA step 0) and 64+kb*16+[0,16)
// (step 1), stored as
//   int4: 16 bytes, word i byte m = code(8i+m) | code(8i+4+m) << 4;
//   int3: 12 bytes, two 2-bit planes L0, L1 (byte m bits 2j'..2j'+1 = low
//         bits of code 4(4a+j')+m) and a high-bit plane H (byte m bit j =
//         bit 2 of code 4j+m).
// Unpacking yields 8 dwords D_j whose byte m is the code of lane slot 4j+m.
// A tile-group's codes and its 16 per-row scales lie in one record
// (sw_expert_layout.h).
#pragma once

#include "sw_device.h"
#include "sw_expert_layout.h"

namespace sw {

constexpr int kTileRows = 16;
constexpr int kGroup = 128;

template <int FMT>
struct TileWord;
template <>
struct TileWord<4> {
  uint32_t w[4];
};
template <>
struct TileWord<3> {
  uint32_t w[3];
};

template <int FMT>
__device__ __forceinline__ TileWord<FMT> load_tile(const unsigned char *p) {
  TileWord<FMT> t;
  if constexpr (FMT == 4) {
    v4u v = __builtin_nontemporal_load((const v4u *)p);
    t.w[0] = v.x;
    t.w[1] = v.y;
    t.w[2] = v.z;
    t.w[3] = v.w;
  } else {
    const uint32_t *q = (const uint32_t *)p;
    t.w[0] = __builtin_nontemporal_load(q);
    t.w[1] = __builtin_nontemporal_load(q + 1);
    t.w[2] = __builtin_nontemporal_load(q + 2);
  }
  return t;
}

template <int FMT>
__device__ __forceinline__ void unpack_tile(const TileWord<FMT> &t, v4i &a0, v4i &a1) {
  uint32_t d[8];
  if constexpr (FMT == 4) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      d[2 * i] = t.w[i] & 0x0F0F0F0Fu;
      d[2 * i + 1] = (t.w[i] >> 4) & 0x0F0F0F0Fu;
    }
  } else {
    const uint32_t L0 = t.w[0], L1 = t.w[1], H = t.w[2];
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

// Per-group activation digits: x ~= A*d1 + B*d2 over each 128-group, with
// gp[g] = {A, B, sum d1, sum d2 (int bits)}.
struct DigitSrc {
  const signed char *d;  // this lane's digit array (group-major), or a 16-byte zero row
  const float4 *gp;      // this lane's token group parameters, or null
  int second;            // 1: lane carries digit 2 (B), 0: digit 1 (A)
  int mask;              // offset mask: ~0 for a digit array, 0 for the zero row
};

// Column c = lane%16 of the MFMA B operand is token c/2, digit c%2.
__device__ __forceinline__ DigitSrc lane_digits(int lane, int tokens, const signed char *dig, int dstride,
                                                const float4 *gp, int gstride, const signed char *zero) {
  int c = lane & 15, tt = c >> 1;
  DigitSrc s;
  s.second = c & 1;
  if (tt < tokens) {
    s.d = dig + (size_t)(2 * tt + (c & 1)) * dstride;
    s.gp = gp + (size_t)tt * gstride;
    s.mask = ~0;
  } else {
    s.d = zero;
    s.gp = nullptr;
    s.mask = 0;
  }
  return s;
}

// Tile data of one row tile for up to NMAX consecutive groups, loaded ahead
// of the MFMAs so that all of a wave's HBM reads are in flight at once.
template <int FMT, int NMAX>
struct TilePrefetch {
  TileWord<FMT> q[NMAX];
  v4f sc[NMAX];
};

template <int FMT, int NMAX>
__device__ __forceinline__ void tile_prefetch(TilePrefetch<FMT, NMAX> &t, const TileMat &mat, int rt, int ng, int g0,
                                              int n, int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (i < n) {
      size_t tg = (size_t)rt * ng + g0 + i;
      t.q[i] = load_tile<FMT>(tm_codes(mat, tg) + lane * BPL);
      t.sc[i] = __builtin_nontemporal_load((const v4f *)(tm_scales(mat, tg) + 4 * kb));
    }
}

// Group-scaled dots over the prefetched groups: per group, the two int8
// MFMAs give exact int32 dots of the codes with both activation digits; the
// epilogue applies the lane's digit scale, removes the code offset (8 for
// int4, 4 for int3) through the digit sum, and accumulates
// scale[row, group] * dot into the lane's own accumulator.  The two digit
// columns of a token are folded once, after the last group (digit_fold).
template <int FMT, int NMAX>
__device__ __forceinline__ void tile_compute(const TilePrefetch<FMT, NMAX> &t, int g0, int n, const DigitSrc &ds,
                                             float acc[4], int lane) {
  constexpr int OFF = FMT == 4 ? 8 : 4;
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (i < n) {
      int g = g0 + i;
      v4i a0, a1;
      unpack_tile<FMT>(t.q[i], a0, a1);
      int off = (g * kGroup + kb * 16) & ds.mask;
      v4i b0 = *(const v4i *)(ds.d + off);
      v4i b1 = *(const v4i *)(ds.d + ((off + 64) & ds.mask));
      float dsc = 0.0f;
      int Q = 0;
      if (ds.gp) {
        float4 p = ds.gp[g];
        dsc = ds.second ? p.y : p.x;
        Q = __float_as_int(ds.second ? p.w : p.z);
      }
      v4i c = {0, 0, 0, 0};
      c = mfma_i8(a0, b0, c);
      c = mfma_i8(a1, b1, c);
      const float scv[4] = {t.sc[i].x, t.sc[i].y, t.sc[i].z, t.sc[i].w};
#pragma unroll
      for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf((float)(c[r] - OFF * Q) * dsc, scv[r], acc[r]);
    }
}

// Codes only (the group scales come from LDS): 3 or 4 registers per group.
template <int FMT, int NMAX>
struct TileCodes {
  TileWord<FMT> q[NMAX];
};

template <int FMT, int NMAX>
__device__ __forceinline__ void tile_codes_prefetch(TileCodes<FMT, NMAX> &t, const TileMat &mat, int rt, int ng,
                                                    int g0, int n, int lane) {
  constexpr int BPL = FMT == 4 ? 16 : 12;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (i < n) t.q[i] = load_tile<FMT>(tm_codes(mat, (size_t)rt * ng + g0 + i) + lane * BPL);
}

// tile_compute with the row tile's scales in LDS: sc[g][16 rows].
template <int FMT, int NMAX>
__device__ __forceinline__ void tile_compute_lds(const TileCodes<FMT, NMAX> &t, int g0, int n, const DigitSrc &ds,
                                                 const float *sc, float acc[4], int lane) {
  constexpr int OFF = FMT == 4 ? 8 : 4;
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (i < n) {
      int g = g0 + i;
      v4i a0, a1;
      unpack_tile<FMT>(t.q[i], a0, a1);
      int off = (g * kGroup + kb * 16) & ds.mask;
      v4i b0 = *(const v4i *)(ds.d + off);
      v4i b1 = *(const v4i *)(ds.d + ((off + 64) & ds.mask));
      float dsc = 0.0f;
      int Q = 0;
      if (ds.gp) {
        float4 p = ds.gp[g];
        dsc = ds.second ? p.y : p.x;
        Q = __float_as_int(ds.second ? p.w : p.z);
      }
      v4i c = {0, 0, 0, 0};
      c = mfma_i8(a0, b0, c);
      c = mfma_i8(a1, b1, c);
      const v4f s4 = *(const v4f *)(sc + g * kTileRows + 4 * kb);
      const float scv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
      for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf((float)(c[r] - OFF * Q) * dsc, scv[r], acc[r]);
    }
}

// Digits of one 1024-wide slice of v (v[base .. base+1024), zero padded)
// with 8 lanes per 128-group: lane l owns elements base+16l .. base+16l+15.
// Same arithmetic as quantize_group (amax of the group, A = amax/127,
// B = A/254, two rounded digits per element, digit sums); d1 / d2 / gp are
// indexed like quantize_group's and written below `limit` (the padded
// length, a multiple of 128) only.  vv: the lane's 16 values, loaded ahead.
__device__ __forceinline__ void quantize_slice8(const v4f vv[4], int base, int limit, signed char *d1,
                                                signed char *d2, float4 *gp, int lane) {
  float v[16];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    v[4 * q] = vv[q].x;
    v[4 * q + 1] = vv[q].y;
    v[4 * q + 2] = vv[q].z;
    v[4 * q + 3] = vv[q].w;
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
  m = fmaxf(m, __shfl_xor(m, 1, 8));
  m = fmaxf(m, __shfl_xor(m, 2, 8));
  m = fmaxf(m, __shfl_xor(m, 4, 8));
  const float A = m / 127.0f;
  const float B = A / 254.0f;
  int q1[16], q2[16];
  int s1 = 0, s2 = 0;
  if (m > 0.0f) {
    const float invA = 127.0f / m, invB = 254.0f / A;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      q1[i] = (int)fminf(fmaxf(__builtin_rintf(v[i] * invA), -127.0f), 127.0f);
      float r = __builtin_fmaf(-(float)q1[i], A, v[i]);
      q2[i] = (int)fminf(fmaxf(__builtin_rintf(r * invB), -127.0f), 127.0f);
      s1 += q1[i];
      s2 += q2[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) q1[i] = q2[i] = 0;
  }
  v4i p1, p2;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    p1[w] = (q1[4 * w] & 255) | (q1[4 * w + 1] & 255) << 8 | (q1[4 * w + 2] & 255) << 16 | (q1[4 * w + 3] & 255) << 24;
    p2[w] = (q2[4 * w] & 255) | (q2[4 * w + 1] & 255) << 8 | (q2[4 * w + 2] & 255) << 16 | (q2[4 * w + 3] & 255) << 24;
  }
  const bool mine = base + 16 * lane < limit;
  if (mine) {
    *(v4i *)(d1 + base + 16 * lane) = p1;
    *(v4i *)(d2 + base + 16 * lane) = p2;
  }
  s1 += __shfl_xor(s1, 1, 8);
  s1 += __shfl_xor(s1, 2, 8);
  s1 += __shfl_xor(s1, 4, 8);
  s2 += __shfl_xor(s2, 1, 8);
  s2 += __shfl_xor(s2, 2, 8);
  s2 += __shfl_xor(s2, 4, 8);
  if (mine && (lane & 7) == 0) gp[(base >> 7) + (lane >> 3)] = make_float4(A, B, __int_as_float(s1), __int_as_float(s2));
}

// Digit 1 (even column) + digit 2 (odd column): valid in lanes with odd
// column c (token c/2), rows 4*kb+i.
__device__ __forceinline__ void digit_fold(float acc[4]) {
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = acc[r] + dpp_row_shr1(acc[r]);
}

template <int FMT, int NMAX>
__device__ __forceinline__ void tile_gemv(const TileMat &mat, int rt, int ng, int g0, int n, const DigitSrc &ds,
                                          float acc[4], int lane) {
  TilePrefetch<FMT, NMAX> t;
  tile_prefetch<FMT, NMAX>(t, mat, rt, ng, g0, n, lane);
  tile_compute<FMT, NMAX>(t, g0, n, ds, acc, lane);
}

// Per-group digits of v[0..n) (zero padded to ng*128) by one wave per group.
// d1 / d2 are group-major int8 arrays, gp[g] = {A, B, Q1, Q2}.
__device__ __forceinline__ void quantize_group(const float *v, int n, int g, signed char *d1, signed char *d2,
                                               float4 *gp, int lane) {
  int i0 = g * kGroup + 2 * lane;
  float a = i0 < n ? v[i0] : 0.0f;
  float b = i0 + 1 < n ? v[i0 + 1] : 0.0f;
  float amax = wave_max_dpp(fmaxf(fabsf(a), fabsf(b)));
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
  int Q1 = wave_sum_dpp(qa1 + qb1), Q2 = wave_sum_dpp(qa2 + qb2);
  if (lane == 0) gp[g] = make_float4(A, B, __int_as_float(Q1), __int_as_float(Q2));
}

// Exact int32 dots of 16 int8 rows (row-major, leading dim ld) with up to 16
// int8 activation rows (B column = lane%16 = activation row), over 64-wide
// k chunks [kc0, kc1), at most NMAX chunks per call.  The weight loads are a
// separate step so that a caller can issue them before it has produced the
// activations.
template <int NMAX>
struct RowPrefetch {
  v4i a[NMAX];
};

template <int NMAX>
__device__ __forceinline__ void rows_prefetch(RowPrefetch<NMAX> &p, const signed char *W, int ld, int row0, int kc0,
                                              int kc1, int lane) {
  const signed char *arow = W + (size_t)(row0 + (lane & 15)) * ld + (lane >> 4) * 16;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (kc0 + i < kc1) p.a[i] = __builtin_nontemporal_load((const v4i *)(arow + (size_t)(kc0 + i) * 64));
}

template <int NMAX>
__device__ __forceinline__ void rows_compute(const RowPrefetch<NMAX> &p, int kc0, int kc1, const signed char *bsrc,
                                             int bld, bool bvalid, v4i &c, int lane) {
  const signed char *brow = bsrc + (size_t)(lane & 15) * bld + (lane >> 4) * 16;
#pragma unroll
  for (int i = 0; i < NMAX; i++)
    if (kc0 + i < kc1) {
      v4i b = bvalid ? *(const v4i *)(brow + (size_t)(kc0 + i) * 64) : v4i{0, 0, 0, 0};
      c = mfma_i8(p.a[i], b, c);
    }
}

template <int NMAX>
__device__ __forceinline__ void idot_tile(const signed char *W, int ld, int row0, int kc0, int kc1,
                                          const signed char *bsrc, int bld, bool bvalid, v4i &c, int lane) {
  RowPrefetch<NMAX> p;
  rows_prefetch<NMAX>(p, W, ld, row0, kc0, kc1, lane);
  rows_compute<NMAX>(p, kc0, kc1, bsrc, bld, bvalid, c, lane);
}

// Order-preserving 32-bit key of a float (larger float -> larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Order-preserving 64-bit key of a double.
__device__ __forceinline__ unsigned long long double_key(double d) {
  unsigned long long b = (unsigned long long)__double_as_longlong(d);
  return (b & 0x8000000000000000ull) ? ~b : (b | 0x8000000000000000ull);
}
__device__ __forceinline__ double key_double(unsigned long long k) {
  unsigned long long b = (k & 0x8000000000000000ull) ? (k & ~0x8000000000000000ull) : ~k;
  return __longlong_as_double((long long)b);
}

}  // namespace sw
