// The mixer layers either side of the MoE block in the reference's hybrid
// decoder, on the device: the Gated DeltaNet layer (coli_cuda_gdn_*) and the
// gated GQA attention layer (coli_cuda_gqa_*), c/backend_cuda.h:149-236.
//
// What the reference computes (its CPU path, the contract): gdn_forward
// c/qwen.c:3005-3030 with gdn_rule_step 2907-2927, gdn_decode_block 4642, and
// attn_forward 3094-3137 with rope_head 3031.  Activations stay fp32 here
// (the reference's GPU path rounds them to fp16 first); outputs agree with
// the CPU path within 1e-3 x RMS.
//
// Gated DeltaNet step, three launches:
//   k_mix_proj<4,..,CONV>  qkv and z projections of every token in one grid;
//                          a wave that owns a qkv channel also runs that
//                          channel's causal convolution ring for the tokens in
//                          order (write the new raw value, SiLU of the tap sum),
//                          so the ring never crosses workgroups;
//   k_gdn_recur            one workgroup per (value head, slot group): the
//                          head's dk x dv state lives in registers (lane halves
//                          split the key index, 64 values a lane) for all of the
//                          group's tokens, read and written once per call;
//   k_mix_proj<4>          the out projection.
// GQA attention step, five launches:
//   k_mix_proj<4>          q (query | gate per head), k and v projections;
//   k_gqa_prep             per-head RMS norm (1 + w) and partial rotary
//                          embedding of q and k, the K/V append;
//   k_gqa_attn<HD>         flash decoding on the fp32 matrix cores: one wave per
//                          (row, kv head, key split) streams 16-key blocks,
//                          S^T = K Q^T and O^T += V^T P^T with
//                          v_mfma_f32_16x16x4f32 (the kv head's query heads are
//                          the 16 MFMA columns), online softmax in between;
//   k_gqa_combine          merges the splits, divides, applies the sigmoid gate;
//   k_mix_proj<4|8>        the o projection (int4 groups or int8 rows).
//
// The projection kernel is one design for all of them: a workgroup owns 8
// rows, each wave 2; every lane loads 16 bytes of each row per 64-lane chunk
// (32 int4 or 16 int8 columns) with one scale, decodes them to fp32 once and
// applies them to every token of the call (up to 16) staged in LDS
// conflict-free ([token][float4 k][lane]).  HBM traffic is the weights once
// per call; activations come from LDS.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sw_backend.h"
#include "sw_device.h"
#include "sw_lds_dma.h"

namespace sw {
namespace {

constexpr int kMixMaxTok = 16;  // tokens of one projection / slot-table launch

typedef float v4f __attribute__((ext_vector_type(4)));

// Per-token slot and position: a table (slot calls, blocks) or base + t.
struct MixTok {
  int tab;
  int distinct;  // tab: every token has a slot of its own
  int base;
  int slot[kMixMaxTok];
  int pos[kMixMaxTok];
};
__device__ __forceinline__ int tok_slot(const MixTok &k, int t) { return k.tab ? k.slot[t] : 0; }
__device__ __forceinline__ int tok_pos(const MixTok &k, int t) { return k.tab ? k.pos[t] : k.base + t; }

struct ProjMat {
  const unsigned char *q;
  const float *s;
  float *y;  // y[t * ldy + row]
  int rows, rb, ng, ldy;
};

struct ProjArgs {
  ProjMat m[3];
  int nm, rows_total;
  const float *x;  // token t at x + t * ldx
  int ldx, cols, gs, B;
  // causal convolution on matrix 0 (Gated DeltaNet qkv channels)
  float *conv_state;  // [slot][K][channels]
  const float *conv_w;  // [channels][K]
  float *mix;         // [B][channels]
  int K;
  long long conv_slot_stride;
  MixTok tok;
  // optional per-(token, head) activation scale r = 1/sqrt(sum(msp) / hw + eps),
  // msp [B][cols / hw][nsp] partial sums of squares (the Gated DeltaNet
  // output's RMS norm, applied as the out projection reads its input)
  const float *msp;
  int nsp, hw;
  float eps;
};

__device__ __forceinline__ float proj_xscale(const ProjArgs &a, int t, int c) {
  if (!a.msp) return 1.0f;
  const int nh = a.cols / a.hw, h = c / a.hw;
  const float *m = a.msp + ((size_t)t * nh + h) * a.nsp;
  float ms = 0.0f;
  for (int k = 0; k < a.nsp; k++) ms += m[k];
  return 1.f / sqrtf(ms / (float)a.hw + a.eps);
}

// The Gated DeltaNet causal convolution of qkv channel ch for the call's
// tokens in order (c/qwen.c:3018-3023), red[t] its raw values; lane-0 code.
// Tokens in slots of their own with K <= 4: every ring word and tap weight
// loads before any store; otherwise each token writes its ring slot and reads
// its taps in turn (a slot's later token sees the earlier one's word).
template <int NT>
__device__ __forceinline__ void conv_channel(const ProjArgs &a, int ch, const float (&red)[NT]) {
  const int C = a.m[0].rows, K = a.K;
  if (a.tok.tab && a.tok.distinct && K <= 4) {
    float tw[4], tv[NT][4];
#pragma unroll
    for (int k = 0; k < 4; k++) tw[k] = a.conv_w[(size_t)ch * K + (k < K ? k : 0)];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float *cs = a.conv_state + (size_t)tok_slot(a.tok, t < a.B ? t : 0) * a.conv_slot_stride;
#pragma unroll
      for (int k = 0; k < 4; k++) tv[t][k] = cs[(size_t)(k < K ? k : 0) * C + ch];
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t >= a.B) continue;
      const int pos = tok_pos(a.tok, t);
      float sconv = 0.0f;
#pragma unroll
      for (int tap = 0; tap < 4; tap++) {
        const int src = pos - (K - 1 - tap);
        if (tap >= K || src < 0) continue;
        const int ks = src % K;
        float v = red[t];
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (src != pos && k == ks) v = tv[t][k];
        sconv = __builtin_fmaf(tw[tap], v, sconv);
      }
      a.mix[(size_t)t * C + ch] = silu_ref(sconv);
      a.conv_state[(size_t)tok_slot(a.tok, t) * a.conv_slot_stride + (size_t)(pos % K) * C + ch] = red[t];
    }
    return;
  }
  const float *cw = a.conv_w + (size_t)ch * K;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    if (t >= a.B) continue;
    const int pos = tok_pos(a.tok, t);
    float *cs = a.conv_state + (size_t)tok_slot(a.tok, t) * a.conv_slot_stride;
    cs[(size_t)(pos % K) * C + ch] = red[t];
    float sconv = 0.0f;
    for (int tap = 0; tap < K; tap++) {
      const int src = pos - (K - 1 - tap);
      if (src >= 0) sconv = __builtin_fmaf(cw[tap], src == pos ? red[t] : cs[(size_t)(src % K) * C + ch], sconv);
    }
    a.mix[(size_t)t * C + ch] = silu_ref(sconv);
  }
}

// y[t][row] = sum_g s[row][g] * sum_{i in g} code(row, i) * x[t][i]
// FMT 4: int4 low nibble first, code = nibble - 8, one scale per group;
// FMT 8: int8 rows, one scale per row.
// Persistent workgroups of 4 waves walk groups of 4 * RW rows.  A lane loads
// 16 bytes of each of its wave's RW rows per 64-lane chunk (32 int4 or 16 int8
// columns, one scale), every chunk of a round at once.  The activations of a
// call are staged in LDS ([token][chunk][float4 k][lane], conflict-free reads)
// once per workgroup when they fit in 64 KB, else per round.
// The CONV form runs the Gated DeltaNet causal convolution of a qkv channel
// in the epilogue (c/qwen.c:3018-3023): lane 0 owns the channel's ring for the
// call's tokens in order; for single-sequence calls with K <= 4 the ring and
// the tap weights are read into registers before the projection.
// grid <= 2 x CUs, 256 threads, 64 KB dynamic LDS.
constexpr int kProjLdsFloats = 16384;

template <int FMT, int NT, bool CONV>
__global__ __launch_bounds__(256) void k_mix_proj(ProjArgs a) {
  constexpr int CPL = FMT == 4 ? 32 : 16;  // columns per lane per 16-byte load
  constexpr int CH = 64 * CPL;             // columns per chunk
  constexpr int F4 = CPL / 4;              // float4 of activations per lane per chunk
  constexpr int RW = NT <= 4 ? 4 : 2;      // rows per wave
  constexpr int NP = NT < 8 ? NT : 8;      // tokens staged per pass
  constexpr int NPASS = (NT + NP - 1) / NP;
  constexpr int MAXC0 = kProjLdsFloats / (NP * CH);
  constexpr int MAXC1 = NT <= 2 ? 4 : 2;   // chunks per round (registers)
  constexpr int MAXC = MAXC0 > MAXC1 ? MAXC1 : (MAXC0 < 1 ? 1 : MAXC0);
  extern __shared__ float4 xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = (a.cols + CH - 1) / CH;
  const bool once = NPASS == 1 && NP * nch * CH <= kProjLdsFloats;
  bool staged = false;  // once: staged after the first round's weight loads are issued
  // activations -> LDS in batches of 8 float4 per thread: all loads of a batch
  // are issued before its first LDS write.  Layout [token][chunk][k][lane] over
  // `nc` chunks from column c0; out-of-range entries are zero.
  auto stage_get = [&](float4(&v)[8], int b0, int total, int nc, int c0, int t0) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int u = b0 + j * 256 + threadIdx.x;
      // branch-free: out-of-range entries load x[0] and are zeroed after, so
      // the compiler counts these loads exactly and waits for them alone
      const int tt = u / (nc * F4 * 64), ci = (u / (F4 * 64)) % nc, k = (u / 64) % F4, l = u % 64;
      const int t = t0 + tt, c = c0 + ci * CH + l * CPL + 4 * k;
      const bool ok = u < total && t < a.B && c < a.cols;
      const float4 ld = *(const float4 *)(a.x + (ok ? (size_t)t * a.ldx + c : 0));
      const float sc = ok ? proj_xscale(a, t, c) : 0.0f;
      v[j] = ok ? make_float4(ld.x * sc, ld.y * sc, ld.z * sc, ld.w * sc) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stage_put = [&](const float4(&v)[8], int b0, int total) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int u = b0 + j * 256 + threadIdx.x;
      if (u < total) xs[u] = v[j];
    }
  };
  // the single-sequence calls (decode, blocks of <= 8 tokens) keep the ring in registers
  const bool ring_regs = CONV && NT <= 8 && !a.tok.tab && a.K <= 4;
  const int ngroups = (a.rows_total + 4 * RW - 1) / (4 * RW);
  for (int g = blockIdx.x; g < ngroups; g += gridDim.x) {
    const int r0 = (g * 4 + wave) * RW;
    const unsigned char *qrow[RW];
    const float *srow[RW];
    int mi[RW], rr[RW];
    bool live[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
      int row = r0 + r;
      live[r] = row < a.rows_total;
      int m = 0;
      if (row >= a.m[0].rows) {
        row -= a.m[0].rows;
        m = 1;
        if (a.nm > 2 && row >= a.m[1].rows) {
          row -= a.m[1].rows;
          m = 2;
        }
      }
      mi[r] = m;
      rr[r] = row;
      const ProjMat &pm = a.m[m];
      qrow[r] = pm.q + (size_t)row * pm.rb;
      srow[r] = FMT == 4 ? pm.s + (size_t)row * pm.ng : pm.s + row;
    }
    // the conv ring and tap weights of the wave's channels (lane 0)
    constexpr int RR = CONV && NT <= 8 ? RW : 1;
    float ring[RR][4], cwv[RR][4];
    if (CONV && NT <= 8 && ring_regs && lane == 0) {
#pragma unroll
      for (int r = 0; r < RR; r++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
          ring[r][k] = 0.0f;
          cwv[r][k] = 0.0f;
          if (live[r] && mi[r] == 0 && k < a.K) {
            ring[r][k] = a.conv_state[(size_t)k * a.m[0].rows + rr[r]];
            cwv[r][k] = a.conv_w[(size_t)rr[r] * a.K + k];
          }
        }
    }

    float acc[RW][NT];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
      for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;

    for (int cr = 0; cr < a.cols; cr += MAXC * CH) {
      float4 xb[8];
      if (once && !staged) stage_get(xb, 0, NP * nch * F4 * 64, nch, 0, 0);
      uint4 w[MAXC][RW];
      float sc[MAXC][RW];
#pragma unroll
      for (int ci = 0; ci < MAXC; ci++) {
        const int col = cr + ci * CH + lane * CPL;
#pragma unroll
        for (int r = 0; r < RW; r++) {
          // branch-free as above: a dead lane or row reads its row's first bytes
          const bool ok = live[r] && col < a.cols;
          const unsigned char *qa = live[r] ? qrow[r] : a.m[0].q;
          const uint4 wl = *(const uint4 *)(qa + (ok ? (FMT == 4 ? col / 2 : col) : 0));
          const float sl = FMT == 4 ? (live[r] ? srow[r] : a.m[0].s)[ok ? col / a.gs : 0] : 1.0f;
          w[ci][r] = ok ? wl : make_uint4(0, 0, 0, 0);
          sc[ci][r] = ok ? sl : 0.0f;
        }
      }
      if (once && !staged) {
        // the first batch's loads were issued before the weights'
        stage_put(xb, 0, NP * nch * F4 * 64);
        for (int b0 = 8 * 256; b0 < NP * nch * F4 * 64; b0 += 8 * 256) {
          stage_get(xb, b0, NP * nch * F4 * 64, nch, 0, 0);
          stage_put(xb, b0, NP * nch * F4 * 64);
        }
        __syncthreads();
        staged = true;
      }
#pragma unroll
      for (int p = 0; p < NPASS; p++) {
        if (!once) {
          __syncthreads();
          for (int b0 = 0; b0 < NP * MAXC * F4 * 64; b0 += 8 * 256) {
            stage_get(xb, b0, NP * MAXC * F4 * 64, MAXC, cr, p * NP);
            stage_put(xb, b0, NP * MAXC * F4 * 64);
          }
          __syncthreads();
        }
#pragma unroll
        for (int ci = 0; ci < MAXC; ci++) {
          if (cr + ci * CH >= a.cols) continue;
#pragma unroll
          for (int r2 = 0; r2 < RW; r2 += 2) {
            float wf[2][CPL];
#pragma unroll
            for (int q = 0; q < 2; q++) {
              const uint4 wq = w[ci][r2 + q];
              const unsigned wd[4] = {wq.x, wq.y, wq.z, wq.w};
              if (FMT == 4) {
                // nibble bytes through opaque masks, so that each value is
                // one v_cvt_f32_ubyte0..3 (column 8d + 2b: low nibble of
                // byte b, 8d + 2b + 1: its high nibble)
#pragma unroll
                for (int d = 0; d < 4; d++) {
                  unsigned lo, hi;
                  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(wd[d]));
                  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(wd[d] >> 4));
#pragma unroll
                  for (int b = 0; b < 4; b++) {
                    wf[q][8 * d + 2 * b] = (float)((lo >> (8 * b)) & 255u) - 8.0f;
                    wf[q][8 * d + 2 * b + 1] = (float)((hi >> (8 * b)) & 255u) - 8.0f;
                  }
                }
              } else {
#pragma unroll
                for (int e = 0; e < CPL; e++) wf[q][e] = (float)(signed char)((wd[e / 4] >> (8 * (e % 4))) & 255u);
              }
            }
#pragma unroll
            for (int tt = 0; tt < NP; tt++) {
              const int t = p * NP + tt;
              if (t < NT && t < a.B) {
                const int base = once ? ((tt * nch + cr / CH + ci) * F4) * 64 : ((tt * MAXC + ci) * F4) * 64;
                float xv[CPL];
#pragma unroll
                for (int k = 0; k < F4; k++) {
                  const float4 v = xs[base + k * 64 + lane];
                  xv[4 * k] = v.x;
                  xv[4 * k + 1] = v.y;
                  xv[4 * k + 2] = v.z;
                  xv[4 * k + 3] = v.w;
                }
#pragma unroll
                for (int q = 0; q < 2; q++) {
                  float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
                  for (int e = 0; e < CPL; e += 2) {
                    p0 = __builtin_fmaf(wf[q][e], xv[e], p0);
                    p1 = __builtin_fmaf(wf[q][e + 1], xv[e + 1], p1);
                  }
                  acc[r2 + q][t] = __builtin_fmaf(p0 + p1, sc[ci][r2 + q], acc[r2 + q][t]);
                }
              }
            }
          }
        }
      }
    }

#pragma unroll
    for (int r = 0; r < RW; r++) {
      float red[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) red[t] = wave_sum_dpp(acc[r][t]);
      if (!live[r] || lane != 0) continue;
      const ProjMat &pm = a.m[mi[r]];
      if (CONV && mi[r] == 0) {
        const int ch = rr[r], C = a.m[0].rows, K = a.K;
        if (CONV && NT <= 8 && ring_regs) {
          // one sequence (slot 0): the ring lives in registers for the call
          const int rq = r < RR ? r : 0;
#pragma unroll
          for (int t = 0; t < NT; t++) {
            if (t >= a.B) continue;
            const int pos = tok_pos(a.tok, t), slot_w = pos % K;
#pragma unroll
            for (int k = 0; k < 4; k++)
              if (k == slot_w) ring[rq][k] = red[t];
            float s = 0.0f;
#pragma unroll
            for (int tap = 0; tap < 4; tap++) {
              if (tap >= K) continue;
              const int src = pos - (K - 1 - tap);
              if (src < 0) continue;
              const int ks = src % K;
              float v = 0.0f;
#pragma unroll
              for (int k = 0; k < 4; k++)
                if (k == ks) v = ring[rq][k];
              s = __builtin_fmaf(cwv[rq][tap], v, s);
            }
            a.mix[(size_t)t * C + ch] = silu_ref(s);
            a.conv_state[(size_t)slot_w * C + ch] = red[t];
          }
        } else {
          conv_channel<NT>(a, ch, red);
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; t++)
          if (t < a.B) pm.y[(size_t)t * pm.ldy + rr[r]] = FMT == 8 ? red[t] * srow[r][0] : red[t];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Gated DeltaNet recurrence (gdn_rule_step, c/qwen.c:2907-2927) for one value
// head, one run of 32 value columns and one group of tokens that share a
// slot, in order: one wave, lanes j = lane & 31 hold the columns, lane half
// (lane >> 5) holds key rows [64 half, 64 half + 64) of them in registers
// (dk <= 128), read and written once per call.  The head's RMS norm couples
// its columns, so the wave writes u = o * norm * silu(z) and its partial sum
// of o^2; the out projection applies 1/sqrt(sum / dv + eps) as it reads u.
// grid (value_heads * ceil(dv / 32), groups), 64 threads.
struct GdnGroups {
  int n;
  int start[kMixMaxTok + 1];
  int tok[kMixMaxTok];
};
struct GdnArgs {
  const float *mix, *z, *a, *b;  // [B][channels], [B][vd], [B][vh], [B][vh]
  const float *A_log, *dt_bias, *norm;
  float *state;  // [slot][vh][dk][dv]
  long long state_slot_stride;
  float *core;  // [B][vd]: o * norm * silu(z)
  float *msp;   // [B][vh][ceil(dv / 32)]: partial sums of o^2
  int kh, vh, dk, dv;
  MixTok tok;
  GdnGroups grp;
};

__device__ __forceinline__ float softplus_ref(float x) {
  return x > 20.f ? x : (x < -20.f ? expf(x) : log1pf(expf(x)));
}

__global__ __launch_bounds__(64) void k_gdn_recur(GdnArgs g) {
  const int nsp = (g.dv + 31) / 32;
  const int h = blockIdx.x / nsp, js = blockIdx.x % nsp, gi = blockIdx.y;
  if (gi >= g.grp.n) return;
  __shared__ float sq[128], sk[128];
  const int lane = threadIdx.x, half = lane >> 5, j = js * 32 + (lane & 31), i0 = half * 64;
  const int dk = g.dk, dv = g.dv, kd = g.kh * dk, vd = g.vh * dv, C = 2 * kd + vd;
  const int hk = h / (g.vh / g.kh);
  const int t_first = g.grp.tok[g.grp.start[gi]];
  float *st = g.state + (size_t)tok_slot(g.tok, t_first) * g.state_slot_stride + (size_t)h * dk * dv;
  // dv is a multiple of 32, so every lane's column exists; a half holds 64
  // key rows when dk = 128 (the loads and stores then take no branches)
  const bool rows64 = i0 + 64 <= dk;
  float S[64];
  if (rows64) {
#pragma unroll
    for (int m = 0; m < 64; m++) S[m] = st[(size_t)(i0 + m) * dv + j];
  } else {
#pragma unroll
    for (int m = 0; m < 64; m++) S[m] = (i0 + m < dk) ? st[(size_t)(i0 + m) * dv + j] : 0.0f;
  }
  const float invsqrt = 1.f / sqrtf((float)dk);
  const float Ah = expf(g.A_log[h]);
  const float nj = g.norm[j];
  const float dtb = g.dt_bias[h];
  for (int gt = g.grp.start[gi]; gt < g.grp.start[gi + 1]; gt++) {
    const int t = g.grp.tok[gt];
    const float *mt = g.mix + (size_t)t * C;
    // every load of the token issues before the barrier (which waits for
    // all of them, the state's included), so they share one round trip
    float qa[2], ka[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int i = lane + 64 * u;
      qa[u] = i < dk ? mt[hk * dk + i] : 0.0f;
      ka[u] = i < dk ? mt[kd + hk * dk + i] : 0.0f;
    }
    const float v = mt[2 * kd + h * dv + j];
    const float zt = g.z[(size_t)t * vd + (size_t)h * dv + j];
    const float bt = g.b[(size_t)t * g.vh + h], at = g.a[(size_t)t * g.vh + h];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; u++) {
      sq[lane + 64 * u] = qa[u];
      sk[lane + 64 * u] = ka[u];
    }
    __syncthreads();
    float pq = 0.0f, pk = 0.0f;
    for (int i = lane; i < 128; i += 64) {
      pq = __builtin_fmaf(sq[i], sq[i], pq);
      pk = __builtin_fmaf(sk[i], sk[i], pk);
    }
    const float qn = 1.f / sqrtf(wave_sum_dpp(pq) + 1e-6f);
    const float kn = 1.f / sqrtf(wave_sum_dpp(pk) + 1e-6f);
    const float beta = sigmoid_ref(bt);
    const float decay = expf(-Ah * softplus_ref(at + dtb));
    float mem0 = 0.0f, mem1 = 0.0f;
#pragma unroll
    for (int m = 0; m < 64; m += 2) {
      S[m] *= decay;
      S[m + 1] *= decay;
      mem0 = __builtin_fmaf(S[m], sk[i0 + m] * kn, mem0);
      mem1 = __builtin_fmaf(S[m + 1], sk[i0 + m + 1] * kn, mem1);
    }
    float mem = mem0 + mem1;
    mem += __shfl_xor(mem, 32);
    const float delta = (v - mem) * beta;
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int m = 0; m < 64; m += 2) {
      S[m] = __builtin_fmaf(sk[i0 + m] * kn, delta, S[m]);
      S[m + 1] = __builtin_fmaf(sk[i0 + m + 1] * kn, delta, S[m + 1]);
      o0 = __builtin_fmaf(S[m], sq[i0 + m] * qn * invsqrt, o0);
      o1 = __builtin_fmaf(S[m + 1], sq[i0 + m + 1] * qn * invsqrt, o1);
    }
    float o = o0 + o1;
    o += __shfl_xor(o, 32);
    const float p2 = wave_sum_dpp(half == 0 ? o * o : 0.0f);
    if (half == 0) g.core[(size_t)t * vd + (size_t)h * dv + j] = o * nj * silu_ref(zt);
    if (lane == 0) g.msp[((size_t)t * g.vh + h) * nsp + js] = p2;
  }
  if (rows64) {
#pragma unroll
    for (int m = 0; m < 64; m++) st[(size_t)(i0 + m) * dv + j] = S[m];
  } else {
#pragma unroll
    for (int m = 0; m < 64; m++)
      if (i0 + m < dk) st[(size_t)(i0 + m) * dv + j] = S[m];
  }
}

// ---------------------------------------------------------------------------
// GQA: q/k RMS norm (1 + w) and partial rotary embedding (c/qwen.c:3110-3113,
// rmsnorm_zero 1780, rope_head 3031), the gate split and the K/V append.
// grid (query_heads + kv_heads, rows), head_dim threads (a multiple of 64).
struct PrepArgs {
  const float *qp, *kr, *vr;  // [B][2*nh*hd], [B][kvrows], [B][kvrows]
  const float *q_norm, *k_norm;
  float *q, *gate;  // [B][nh*hd]
  float *k_cache, *v_cache;
  long long slot_stride;  // floats per slot
  int nh, nkv, hd, rd;
  float theta, eps;
  MixTok tok;
};

__global__ __launch_bounds__(256) void k_gqa_prep(PrepArgs p) {
  __shared__ float row[256], sred[4];
  const int hh = blockIdx.x, t = blockIdx.y, j = threadIdx.x, hd = p.hd;
  const int lane = j & 63, wave = j >> 6, nw = hd >> 6;
  const int kvrows = p.nkv * hd, ctxn = p.nh * hd;
  const bool isq = hh < p.nh;
  const int kvh = hh - p.nh;
  float v, vv = 0.0f;
  if (isq) {
    const float *src = p.qp + (size_t)t * 2 * ctxn + (size_t)hh * 2 * hd;
    v = src[j];
    p.gate[(size_t)t * ctxn + (size_t)hh * hd + j] = src[hd + j];
  } else {
    v = p.kr[(size_t)t * kvrows + (size_t)kvh * hd + j];
    vv = p.vr[(size_t)t * kvrows + (size_t)kvh * hd + j];
  }
  const float nw1 = 1.f + (isq ? p.q_norm : p.k_norm)[j];
  // the rotation's angle depends on the position only: formed while the
  // row's loads are in flight
  const int half = p.rd / 2, pos = tok_pos(p.tok, t);
  float co = 1.0f, si = 0.0f;
  if (j < p.rd) {
    const int i = j < half ? j : j - half;
    const float e = -2.f * (float)i / (float)p.rd;
    const float fr = (float)pow((double)p.theta, (double)e);
    const float ang = (float)pos * fr;
    co = (float)cos((double)ang);
    si = (float)sin((double)ang);
  }
  const float s2 = wave_sum_dpp(v * v);
  if (lane == 0) sred[wave] = s2;
  __syncthreads();
  float ms = 0.0f;
  for (int w = 0; w < nw; w++) ms += sred[w];
  const float r = 1.f / sqrtf(ms / (float)hd + p.eps);
  row[j] = v * r * nw1;
  __syncthreads();
  float y = row[j];
  if (j < p.rd) {
    const int i = j < half ? j : j - half;
    const float a = row[i], b = row[i + half];
    y = j < half ? __builtin_fmaf(a, co, -(b * si)) : __builtin_fmaf(b, co, a * si);
  }
  if (isq) {
    p.q[(size_t)t * ctxn + (size_t)hh * hd + j] = y;
  } else {
    const size_t at = (size_t)tok_slot(p.tok, t) * p.slot_stride + (size_t)pos * kvrows + (size_t)kvh * hd + j;
    p.k_cache[at] = y;
    p.v_cache[at] = vv;
  }
}

// ---------------------------------------------------------------------------
// Flash decoding over fp32 caches on v_mfma_f32_16x16x4f32.  One workgroup
// of kAttnWaves (4) waves per (row, kv head, split); the split owns a run of
// 16-key blocks of the row's T = pos + 1 keys and wave w takes every fourth.
// Operand layouts of the 16x16x4 instruction: lane l gives A[l % 16][l / 16]
// and B[l / 16][l % 16]; D lane l, register i holds D[4 (l / 16) + i][l % 16].
//   scores S^T (keys x heads): A = K block rows, B = Q^T; lane group
//     g = l / 16 at step i, float4 component c, contracts dim 16 i + 4 g + c,
//     so the four lane groups of a key read 64 contiguous bytes per load; four
//     accumulators (one per float4 component) keep the MFMA chain short;
//   O^T (dims x heads) += V^T P^T: step s takes keys 4g + s of the block, the
//     probabilities lane l already holds for its head, and V[key][dim], the
//     A row r of dim tile d being dim 64 (d / 4) + 4 r + d % 4, so a lane's
//     values of four tiles are one float4.  The block's V values are loaded
//     before the score MFMAs, so their latency overlaps them.
// The waves' (m, l, O) merge in LDS in wave order; the workgroup writes
// one partial record: O [16][HD] unnormalised, the max m [16], the sum l [16].
struct AttnArgs {
  const float *q;  // [B][nh*hd]
  const float *k_cache, *v_cache;
  long long slot_stride;
  float *part;
  int nh, nkv, S;
  MixTok tok;
};

__device__ __forceinline__ v4f mfma_f32_16x16x4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kAttnWaves = 4;  // waves of a k_gqa_attn workgroup
template <int HD>
__global__ __launch_bounds__(64 * kAttnWaves) void k_gqa_attn(AttnArgs a) {
  constexpr int KQ = HD / 4, NT16 = HD / 16, PSZ = 16 * HD + 32;
  __shared__ float s_m[kAttnWaves][16], s_l[kAttnWaves][16];
  __shared__ float s_o[16 * (HD + 1)];  // [head][dim], rows padded
  __shared__ float s_q[16 * 4 * (HD / 4 + 4)];
  const int t = blockIdx.y, kvh = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
  const int G = a.nh / a.nkv;
  const int T = tok_pos(a.tok, t) + 1;
  const int nb = (T + 15) / 16, per = (nb + a.S - 1) / a.S;
  const int b0 = s * per, b1 = min(nb, b0 + per);
  const int kvrows = a.nkv * HD;
  const size_t sbase = (size_t)tok_slot(a.tok, t) * a.slot_stride + (size_t)kvh * HD;
  const float *kc = a.k_cache + sbase, *vc = a.v_cache + sbase;

  // a block's K rows (A operand) and V values (A operand of O^T); rows past
  // T read the block's first row and are masked below
  float4 kv[KQ / 4];
  float vv[4][NT16];
  auto load_block = [&](int blk) {
    const int key0 = blk * 16, km = key0 + n;
    const float *kr = kc + (size_t)(km < T ? km : key0) * kvrows + 4 * kg;
#pragma unroll
    for (int i = 0; i < KQ / 4; i++) kv[i] = *(const float4 *)(kr + 16 * i);
#pragma unroll
    for (int s2 = 0; s2 < 4; s2++) {
      const int key = key0 + 4 * kg + s2;
      const float *vr = vc + (size_t)(key < T ? key : key0) * kvrows + 4 * n;
#pragma unroll
      for (int q4 = 0; q4 < NT16 / 4; q4++) {
        const float4 v4 = *(const float4 *)(vr + 64 * q4);
        vv[s2][4 * q4] = v4.x;
        vv[s2][4 * q4 + 1] = v4.y;
        vv[s2][4 * q4 + 2] = v4.z;
        vv[s2][4 * q4 + 3] = v4.w;
      }
    }
  };
  // the wave's first block issues before the queries' staging barrier (which
  // waits for every load in flight), so both share one round trip
  const int bfirst = b0 + wave;
  if (bfirst < b1) load_block(bfirst);

  // the kv head's queries in LDS, [head n][lane group g][KQ + 4] (heads past
  // G are zero); a lane reads its B operands from there, keeping registers
  // for the K and V values of a whole block in flight
  for (int u = threadIdx.x; u < 16 * HD / 4; u += 64 * kAttnWaves) {
    const int hn = u / (HD / 4), e4 = u % (HD / 4), g4 = e4 % 4, i4 = e4 / 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (hn < G) v = *(const float4 *)(a.q + (size_t)t * a.nh * HD + (size_t)(kvh * G + hn) * HD + 4 * e4);
    *(float4 *)(s_q + (hn * 4 + g4) * (KQ + 4) + 4 * i4) = v;
  }
  __syncthreads();
  const float *qs = s_q + (n * 4 + kg) * (KQ + 4);
  v4f o[NT16];
#pragma unroll
  for (int d = 0; d < NT16; d++) o[d] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float scale = 1.f / sqrtf((float)HD);

  for (int b = bfirst; b < b1; b += kAttnWaves) {
    const int key0 = b * 16;
    if (b != bfirst) load_block(b);
    // all of the block's K and V loads are in flight before the first MFMA
    asm volatile("" ::: "memory");
    v4f c0 = v4f{0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
    for (int i = 0; i < KQ / 4; i++) {
      const float4 qv = *(const float4 *)(qs + 4 * i);
      c0 = mfma_f32_16x16x4(kv[i].x, qv.x, c0);
      c1 = mfma_f32_16x16x4(kv[i].y, qv.y, c1);
      c2 = mfma_f32_16x16x4(kv[i].z, qv.z, c2);
      c3 = mfma_f32_16x16x4(kv[i].w, qv.w, c3);
    }
    const v4f sc = (c0 + c1) + (c2 + c3);
    float sv[4];
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key = key0 + 4 * kg + i;
      sv[i] = key < T ? sc[i] * scale : -INFINITY;
      bm = fmaxf(bm, sv[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float m_new = fmaxf(m_run, bm);
    const float alpha = expf(m_run - m_new);
    float pr[4], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pr[i] = expf(sv[i] - m_new);
      ps += pr[i];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < NT16; d++) o[d] *= alpha;
#pragma unroll
    for (int s2 = 0; s2 < 4; s2++)
#pragma unroll
      for (int d = 0; d < NT16; d++) o[d] = mfma_f32_16x16x4(vv[s2][d], pr[s2], o[d]);
  }

  // merge the waves in wave order
  if (kg == 0) {
    s_m[wave][n] = m_run;
    s_l[wave][n] = l_run;
  }
  __syncthreads();
  float M = s_m[0][n];
#pragma unroll
  for (int w = 1; w < kAttnWaves; w++) M = fmaxf(M, s_m[w][n]);
  const float f = m_run == -INFINITY ? 0.0f : expf(m_run - M);
  for (int w = 0; w < kAttnWaves; w++) {
    if (wave == w) {
#pragma unroll
      for (int d = 0; d < NT16; d++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float *p = s_o + (size_t)n * (HD + 1) + 64 * (d / 4) + 16 * kg + 4 * i + (d % 4);
          *p = w == 0 ? o[d][i] * f : __builtin_fmaf(o[d][i], f, *p);
        }
    }
    __syncthreads();
  }
  float *rec = a.part + ((size_t)(t * a.nkv + kvh) * a.S + s) * PSZ;
  for (int u = threadIdx.x; u < 16 * HD; u += 64 * kAttnWaves) rec[u] = s_o[(u / HD) * (HD + 1) + u % HD];
  if (threadIdx.x < 16) {
    const int h = threadIdx.x;
    float Mh = s_m[0][h], L = 0.0f;
    for (int w = 1; w < kAttnWaves; w++) Mh = fmaxf(Mh, s_m[w][h]);
    for (int w = 0; w < kAttnWaves; w++)
      if (s_m[w][h] != -INFINITY) L = __builtin_fmaf(s_l[w][h], expf(s_m[w][h] - Mh), L);
    rec[16 * HD + h] = Mh;
    rec[16 * HD + 16 + h] = L;
  }
}

// Merge the splits of one (row, query head), divide by the softmax sum and
// apply the sigmoid gate (c/qwen.c:3129-3134).  A workgroup takes 64 dims of
// one head (one per lane), its 4 waves the splits w, w + 4, ...: lane i of
// wave w loads split w + 4i's maximum and sum (one load each for the wave),
// the wave's maximum and weights follow by lane reductions, and its lanes'
// partial outputs of up to 32 splits a round issue before the first is used
// (each split's weight read from the lane that holds it).  The waves meet in
// LDS in wave order.  grid (nh * hd / 64, B), 256 threads; S <= kMaxSplits.
constexpr int kMaxSplits = 256;
constexpr int kCombWaves = 4, kCombBatch = 32;
struct CombArgs {
  const float *part, *gate;
  float *ctx;  // [B][nh*hd]
  int nh, nkv, hd, S;
};

__global__ __launch_bounds__(256) void k_gqa_combine(CombArgs c) {
  __shared__ float s_o[kCombWaves][64], s_m[kCombWaves], s_l[kCombWaves];
  const int hd = c.hd, dq = hd >> 6, h = blockIdx.x / dq, t = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, j = 64 * (blockIdx.x % dq) + lane;
  const int G = c.nh / c.nkv, kvh = h / G, n = h % G, S = c.S;
  const size_t psz = (size_t)16 * hd + 32;
  const float *base = c.part + (size_t)(t * c.nkv + kvh) * S * psz;
  const size_t at = (size_t)t * c.nh * hd + (size_t)h * hd + j;
  const float g = w == 0 ? c.gate[at] : 0.0f;
  const int sl = w + kCombWaves * lane;  // this lane's split for the maximum and sum
  float m = -INFINITY, lv = 0.0f;
  if (sl < S) {
    m = base[(size_t)sl * psz + 16 * hd + n];
    lv = base[(size_t)sl * psz + 16 * hd + 16 + n];
  }
  const int ns = S > w ? (S - w + kCombWaves - 1) / kCombWaves : 0;  // the wave's splits
  float o = 0.0f, mb = -INFINITY, lsum = 0.0f;
  if (ns > 0) {
    float vo[kCombBatch];
    const float *op = base + (size_t)n * hd + j;
#pragma unroll
    for (int k = 0; k < kCombBatch; k++)
      vo[k] = op[(size_t)(k < ns ? w + kCombWaves * k : w) * psz];
    mb = wave_max_dpp(m);
    const float wl = m == -INFINITY ? 0.0f : expf(m - mb);
    lsum = wave_sum_dpp(lv * wl);
#pragma unroll
    for (int k = 0; k < kCombBatch; k++)
      o = __builtin_fmaf(vo[k], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k)), o);
    for (int k0 = kCombBatch; k0 < ns; k0 += kCombBatch) {
#pragma unroll
      for (int k = 0; k < kCombBatch; k++)
        vo[k] = op[(size_t)(k0 + k < ns ? w + kCombWaves * (k0 + k) : w) * psz];
#pragma unroll
      for (int k = 0; k < kCombBatch; k++)
        o = __builtin_fmaf(vo[k], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k0 + k)), o);
    }
  }
  s_o[w][lane] = o;
  if (lane == 0) {
    s_m[w] = mb;
    s_l[w] = lsum;
  }
  __syncthreads();
  if (w != 0) return;
  float Mx = -INFINITY;
  for (int q = 0; q < kCombWaves; q++) Mx = fmaxf(Mx, s_m[q]);
  float O = 0.0f, L = 0.0f;
  for (int q = 0; q < kCombWaves; q++) {
    const float f = s_m[q] == -INFINITY ? 0.0f : expf(s_m[q] - Mx);
    O = __builtin_fmaf(s_o[q][lane], f, O);
    L = __builtin_fmaf(s_l[q], f, L);
  }
  c.ctx[at] = (O / L) * sigmoid_ref(g);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int tok_bucket(int B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : B <= 8 ? 8 : 16; }

// A projection layout the kernel takes: 16-byte rows, 32-column groups.
bool q4_ok(const void *q, const float *s, int rows, int cols, int gs, int rb, int ng) {
  return q && s && rows > 0 && cols > 0 && gs > 0 && gs % 32 == 0 && cols % 32 == 0 && rb >= cols / 2 &&
         rb % 16 == 0 && ng >= (cols + gs - 1) / gs && ((uintptr_t)q & 15) == 0;
}
bool q8_ok(const void *q, const float *s, int rows, int cols, int rb) {
  return q && s && rows > 0 && cols > 0 && cols % 16 == 0 && rb >= cols && rb % 16 == 0 && ((uintptr_t)q & 15) == 0;
}

// The one- to four-token form of k_mix_proj: no activation staging, the
// columns split over waves.  A workgroup owns RW rows for every wk of its 4
// waves (wk = 1, 2 or 4 waves along the columns, by the row's chunk count).
// Per 64-lane chunk of its column share a wave copies 16 bytes a lane of
// each of its RW rows into its own LDS slice (global_load_lds: the bytes in
// flight hold no registers) and loads the lanes' own 32 (int4) or 16 (int8)
// activations straight from global memory (L2-resident), so a wave's loads
// issue at once and many short waves keep HBM busy.  The waves' partial sums
// meet in LDS in a fixed order; lane r of the row group's first wave
// finishes row r (k_mix_proj's epilogue, the rows in parallel, its loads
// issued at the start).  grid ceil(rows_total / (4 RW / wk)), 256 threads,
// 4 RW KB of dynamic LDS.
constexpr int kDirectRows = 8;  // rows a wave of k_mix_proj_direct takes
template <int FMT, int NT, bool CONV, int RW>
__global__ __launch_bounds__(256) void k_mix_proj_direct(ProjArgs a) {
  constexpr int CPL = FMT == 4 ? 32 : 16, CH = 64 * CPL, F4 = CPL / 4;
  __shared__ float s_part[4][RW][NT];
  extern __shared__ __align__(16) unsigned char wlds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = (a.cols + CH - 1) / CH;
  const int wk = nch >= 4 ? 4 : (nch >= 2 ? 2 : 1);
  const int rg = wave / wk, kw = wave % wk;
  const int r0 = (blockIdx.x * (4 / wk) + rg) * RW;
  unsigned char *const wbuf = wlds + wave * (RW * 1024);
  // Lane r < RW of the row group's first wave finishes row r0 + r; what its
  // epilogue reads (the int8 row scale; one token's conv ring slots and tap
  // weights, K <= 4) is loaded now, with the projection's own loads.
  const bool ring1 = CONV && NT == 1 && a.K <= 4;
  int err = r0 + lane, em = 0;
  const bool elive = kw == 0 && lane < RW && err < a.rows_total;
  if (err >= a.m[0].rows) {
    err -= a.m[0].rows;
    em = 1;
    if (a.nm > 2 && err >= a.m[1].rows) {
      err -= a.m[1].rows;
      em = 2;
    }
  }
  if (!elive) err = em = 0;
  float tv[4] = {}, tw[4] = {}, escale = 1.0f;
  if (ring1) {
    const int C = a.m[0].rows, K = a.K, ch = em == 0 ? err : 0;
    const float *cs = a.conv_state + (size_t)tok_slot(a.tok, 0) * a.conv_slot_stride;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      tv[k] = cs[(size_t)(k < K ? k : 0) * C + ch];
      tw[k] = a.conv_w[(size_t)ch * K + (k < K ? k : 0)];
    }
  }
  if (FMT == 8) escale = (em == 0 ? a.m[0].s : (em == 1 ? a.m[1].s : a.m[2].s))[err];
  const unsigned char *qrow[RW];
  const float *srow[RW];
  int mi[RW], rr[RW];
  bool live[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) {
    int row = r0 + r;
    live[r] = row < a.rows_total;
    int m = 0;
    if (row >= a.m[0].rows) {
      row -= a.m[0].rows;
      m = 1;
      if (a.nm > 2 && row >= a.m[1].rows) {
        row -= a.m[1].rows;
        m = 2;
      }
    }
    mi[r] = m;
    rr[r] = live[r] ? row : 0;
    const ProjMat &pm = a.m[live[r] ? m : 0];
    qrow[r] = pm.q + (size_t)rr[r] * pm.rb;
    srow[r] = FMT == 4 ? pm.s + (size_t)rr[r] * pm.ng : pm.s + rr[r];
  }
  float acc[RW][NT];
#pragma unroll
  for (int r = 0; r < RW; r++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
  for (int ci = kw; ci < nch; ci += wk) {
    const int col = ci * CH + lane * CPL;
    const bool ok = col < a.cols;
    const int cc = ok ? col : 0;
    // every load of the chunk is issued before the first use (the empty
    // asm with a memory clobber keeps the compiler from sinking loads to
    // their uses, which would serialise their latencies)
    // the rows' 16 bytes a lane go global -> LDS (the wave's own slice,
    // 1 KB a row), so a wave has RW KB in flight without holding it in
    // registers; the previous chunk's LDS reads are done before the copies
    // overwrite them
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int r = 0; r < RW; r++) dma_b128(qrow[r] + (FMT == 4 ? cc / 2 : cc), lds_addr(wbuf + r * 1024));
    float4 xl[NT][F4];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int tc = t < a.B ? t : 0;
#pragma unroll
      for (int k = 0; k < F4; k++) xl[t][k] = *(const float4 *)(a.x + (size_t)tc * a.ldx + cc + 4 * k);
    }
    float sl[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) sl[r] = FMT == 4 ? srow[r][cc / a.gs] : 1.0f;
    wait_dma();
    float sc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) sc[r] = (ok && live[r]) ? sl[r] : 0.0f;
    float xv[NT][CPL];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float xs = proj_xscale(a, t < a.B ? t : 0, cc);
#pragma unroll
      for (int k = 0; k < F4; k++) {
        xv[t][4 * k] = xl[t][k].x * xs;
        xv[t][4 * k + 1] = xl[t][k].y * xs;
        xv[t][4 * k + 2] = xl[t][k].z * xs;
        xv[t][4 * k + 3] = xl[t][k].w * xs;
      }
    }
    // int4: sum (n - 8) x = sum n x - 8 sum x, the nibbles n converted from
    // the bytes of (w & 0x0F0F0F0F) and ((w >> 4) & 0x0F0F0F0F); the lane's
    // sum of x serves every row
    float sx[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float s0 = 0.0f, s1 = 0.0f;
      if (FMT == 4) {
#pragma unroll
        for (int e = 0; e < CPL; e += 2) {
          s0 += xv[t][e];
          s1 += xv[t][e + 1];
        }
      }
      sx[t] = s0 + s1;
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const uint4 wr = *(const uint4 *)(wbuf + r * 1024 + 16 * lane);
      const unsigned wd[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float p0 = 0.0f, p1 = 0.0f;
        if (FMT == 4) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            // the masks as opaque instructions: seen through, they become a
            // bit-field extract per nibble instead of v_cvt_f32_ubyte1..3
            unsigned lo, hi;
            asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(wd[q]));
            asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(wd[q] >> 4));
#pragma unroll
            for (int b = 0; b < 4; b++) {
              p0 = __builtin_fmaf((float)((lo >> (8 * b)) & 255u), xv[t][8 * q + 2 * b], p0);
              p1 = __builtin_fmaf((float)((hi >> (8 * b)) & 255u), xv[t][8 * q + 2 * b + 1], p1);
            }
          }
          p0 = __builtin_fmaf(-8.0f, sx[t], p0);
        } else {
#pragma unroll
          for (int e = 0; e < CPL; e += 2) {
            p0 = __builtin_fmaf((float)(signed char)((wd[e / 4] >> (8 * (e % 4))) & 255u), xv[t][e], p0);
            p1 = __builtin_fmaf((float)(signed char)((wd[(e + 1) / 4] >> (8 * ((e + 1) % 4))) & 255u), xv[t][e + 1],
                                p1);
          }
        }
        acc[r][t] = __builtin_fmaf(p0 + p1, sc[r], acc[r][t]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; r++)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float v = wave_sum_dpp(acc[r][t]);
      if (lane == 0) s_part[wave][r][t] = v;
    }
  __syncthreads();
  if (!elive) return;
  float red[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    float v = s_part[wave][lane][t];
    for (int k = 1; k < wk; k++) v += s_part[wave + k][lane][t];
    red[t] = v;
  }
  if (CONV && em == 0 && ring1) {
    const int C = a.m[0].rows, K = a.K;
    const int pos = tok_pos(a.tok, 0);
    float sconv = 0.0f;
#pragma unroll
    for (int tap = 0; tap < 4; tap++) {
      const int src = pos - (K - 1 - tap);
      if (tap >= K || src < 0) continue;
      const int ks = src % K;
      float v = red[0];
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (src != pos && k == ks) v = tv[k];
      sconv = __builtin_fmaf(tw[tap], v, sconv);
    }
    a.conv_state[(size_t)tok_slot(a.tok, 0) * a.conv_slot_stride + (size_t)(pos % K) * C + err] = red[0];
    a.mix[err] = silu_ref(sconv);
  } else if (CONV && em == 0) {
    conv_channel<NT>(a, err, red);
  } else {
    float *const y = em == 0 ? a.m[0].y : (em == 1 ? a.m[1].y : a.m[2].y);
    const int ldy = em == 0 ? a.m[0].ldy : (em == 1 ? a.m[1].ldy : a.m[2].ldy);
#pragma unroll
    for (int t = 0; t < NT; t++)
      if (t < a.B) y[(size_t)t * ldy + err] = FMT == 8 ? red[t] * escale : red[t];
  }
}

template <int FMT, int NT, bool CONV>
void launch_proj_nt(ColiCuda *ctx, const ProjArgs &a) {
  constexpr int RW = NT <= 4 ? 4 : 2;
  const int groups = (a.rows_total + 4 * RW - 1) / (4 * RW);
  const int cap = 2 * (ctx->sm_count > 0 ? ctx->sm_count : 256);
  k_mix_proj<FMT, NT, CONV><<<groups < cap ? groups : cap, 256, kProjLdsFloats * 4, ctx->stream>>>(a);
}

template <int FMT, int NT, bool CONV>
void launch_proj_direct(ColiCuda *ctx, const ProjArgs &a) {
  constexpr int CH = 64 * (FMT == 4 ? 32 : 16), RW = kDirectRows;
  const int nch = (a.cols + CH - 1) / CH;
  const int rows_per_block = 4 * RW / (nch >= 4 ? 4 : (nch >= 2 ? 2 : 1));
  k_mix_proj_direct<FMT, NT, CONV, RW>
      <<<(a.rows_total + rows_per_block - 1) / rows_per_block, 256, 4 * RW * 1024, ctx->stream>>>(a);
}

template <int FMT, bool CONV>
void launch_proj(ColiCuda *ctx, const ProjArgs &a) {
  switch (tok_bucket(a.B)) {
    case 1: launch_proj_direct<FMT, 1, CONV>(ctx, a); break;
    case 2: launch_proj_direct<FMT, 2, CONV>(ctx, a); break;
    case 4: launch_proj_direct<FMT, 4, CONV>(ctx, a); break;
    case 8: launch_proj_nt<FMT, 8, CONV>(ctx, a); break;
    default: launch_proj_nt<FMT, 16, CONV>(ctx, a); break;
  }
}

ProjMat pmat(const unsigned char *q, const float *s, float *y, int rows, int rb, int ng, int ldy) {
  ProjMat m;
  m.q = q;
  m.s = s;
  m.y = y;
  m.rows = rows;
  m.rb = rb;
  m.ng = ng;
  m.ldy = ldy;
  return m;
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct GdnCall {
  const char *name;
  float *out;
  const float *x, *a, *b;
  int batch;
  bool device_io;
  MixTok tok;
  const unsigned char *qkv_q, *z_q, *out_q;
  const float *qkv_s, *z_s, *out_s;
  int qkv_rb, qkv_ng, z_rb, z_ng, out_rb, out_ng;
  const float *conv_w, *a_log, *dt_bias, *norm;
  float *conv_state, *state;
  int slots, hidden, kh, vh, dk, dv, K, gs;
  float eps;
};

int gdn_run(ColiCuda *ctx, const GdnCall &c) {
  const int kd = c.kh * c.dk, vd = c.vh * c.dv, C = 2 * kd + vd, B = c.batch, H = c.hidden;
  if (!q4_ok(c.qkv_q, c.qkv_s, C, H, c.gs, c.qkv_rb, c.qkv_ng) || !q4_ok(c.z_q, c.z_s, vd, H, c.gs, c.z_rb, c.z_ng) ||
      !q4_ok(c.out_q, c.out_s, H, vd, c.gs, c.out_rb, c.out_ng))
    return fail_arg("%s: int4 projections need group sizes and widths that are multiples of 32 and 16-byte rows",
                    c.name);
  if (c.dk > 128 || c.dv > 256 || c.dv % 32)
    return fail_arg("%s: key_dim above 128, or value_dim above 256 or not a multiple of 32, is not supported",
                    c.name);
  if (((uintptr_t)c.x & 15) || (H % 4)) return fail_arg("%s: activations must be 16-byte aligned", c.name);
  // scratch: [x][a][b] (host I/O), mix, z, core, y
  const size_t ox = 0, oa = ox + align_up((size_t)B * H * 4), ob = oa + align_up((size_t)B * c.vh * 4),
               om = ob + align_up((size_t)B * c.vh * 4), oz = om + align_up((size_t)B * C * 4),
               oc = oz + align_up((size_t)B * vd * 4), oy = oc + align_up((size_t)B * vd * 4),
               oms = oy + align_up((size_t)B * H * 4),
               total = oms + align_up((size_t)B * c.vh * ((c.dv + 31) / 32) * 4);
  if (ensure_scratch(ctx, kScrMixer, total, c.name)) return -1;
  char *w = (char *)ctx->scratch[kScrMixer];
  const float *x = c.x, *av = c.a, *bv = c.b;
  if (!c.device_io) {
    hipError_t e = hipMemcpyAsync(w + ox, c.x, (size_t)B * H * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(w + oa, c.a, (size_t)B * c.vh * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(w + ob, c.b, (size_t)B * c.vh * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip(c.name, e);
    x = (const float *)(w + ox);
    av = (const float *)(w + oa);
    bv = (const float *)(w + ob);
  }
  float *mix = (float *)(w + om), *z = (float *)(w + oz), *core = (float *)(w + oc), *msp = (float *)(w + oms);
  float *y = c.device_io ? c.out : (float *)(w + oy);

  ProjArgs p;
  memset(&p, 0, sizeof(p));
  p.m[0] = pmat(c.qkv_q, c.qkv_s, nullptr, C, c.qkv_rb, c.qkv_ng, C);
  p.m[1] = pmat(c.z_q, c.z_s, z, vd, c.z_rb, c.z_ng, vd);
  p.nm = 2;
  p.rows_total = C + vd;
  p.x = x;
  p.ldx = H;
  p.cols = H;
  p.gs = c.gs;
  p.B = B;
  p.conv_state = c.conv_state;
  p.conv_w = c.conv_w;
  p.mix = mix;
  p.K = c.K;
  p.conv_slot_stride = (long long)c.K * C;
  p.tok = c.tok;
  launch_proj<4, true>(ctx, p);

  GdnArgs g;
  memset(&g, 0, sizeof(g));
  g.mix = mix;
  g.z = z;
  g.a = av;
  g.b = bv;
  g.A_log = c.a_log;
  g.dt_bias = c.dt_bias;
  g.norm = c.norm;
  g.state = c.state;
  g.state_slot_stride = (long long)c.vh * c.dk * c.dv;
  g.core = core;
  g.msp = msp;
  g.kh = c.kh;
  g.vh = c.vh;
  g.dk = c.dk;
  g.dv = c.dv;
  g.tok = c.tok;
  // groups of tokens sharing a slot, each in token order
  int gslot[kMixMaxTok];
  int members[kMixMaxTok][kMixMaxTok], count[kMixMaxTok];
  int ng = 0;
  for (int t = 0; t < B; t++) {
    const int sl = c.tok.tab ? c.tok.slot[t] : 0;
    int k = 0;
    while (k < ng && gslot[k] != sl) k++;
    if (k == ng) {
      gslot[ng] = sl;
      count[ng++] = 0;
    }
    members[k][count[k]++] = t;
  }
  g.grp.n = ng;
  int at = 0;
  for (int k = 0; k < ng; k++) {
    g.grp.start[k] = at;
    for (int i = 0; i < count[k]; i++) g.grp.tok[at++] = members[k][i];
  }
  g.grp.start[ng] = at;
  const int nsp = (c.dv + 31) / 32;
  k_gdn_recur<<<dim3(c.vh * nsp, ng), 64, 0, ctx->stream>>>(g);

  ProjArgs o;
  memset(&o, 0, sizeof(o));
  o.m[0] = pmat(c.out_q, c.out_s, y, H, c.out_rb, c.out_ng, H);
  o.nm = 1;
  o.rows_total = H;
  o.x = core;
  o.ldx = vd;
  o.cols = vd;
  o.gs = c.gs;
  o.B = B;
  o.msp = msp;
  o.nsp = nsp;
  o.hw = c.dv;
  o.eps = c.eps;
  launch_proj<4, false>(ctx, o);
  if (launch_status(c.name)) return -1;
  if (c.device_io) return 0;
  hipError_t e = hipMemcpyAsync(c.out, y, (size_t)B * H * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return fail_hip(c.name, e);
  e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? 0 : fail_hip(c.name, e);
}

struct GqaCall {
  const char *name;
  float *out;
  const float *x;
  int rows;
  bool device_io;
  MixTok tok;  // tab: per-row slot/pos (<= 16 rows); else pos = base + row, slot 0
  int max_pos;  // largest position of the call
  const unsigned char *q_q, *k_q, *v_q;
  const float *q_s, *k_s, *v_s;
  int q_rb, q_ng, k_rb, k_ng, v_rb, v_ng;
  const void *o_q;
  const float *o_s;
  int o_fmt, o_rb, o_ng;
  const float *q_norm, *k_norm;
  float *k_cache, *v_cache;
  long long slot_stride;
  int hidden, nh, nkv, hd, rd, gs;
  float theta, eps;
};

template <int HD>
void launch_attn(ColiCuda *ctx, const AttnArgs &a, int rows) {
  k_gqa_attn<HD><<<dim3(a.nkv * a.S, rows), 64 * kAttnWaves, 0, ctx->stream>>>(a);
}

int gqa_run(ColiCuda *ctx, const GqaCall &c) {
  const int H = c.hidden, hd = c.hd, R = c.rows;
  const int qrows = 2 * c.nh * hd, kvrows = c.nkv * hd, ctxn = c.nh * hd;
  if (!q4_ok(c.q_q, c.q_s, qrows, H, c.gs, c.q_rb, c.q_ng) || !q4_ok(c.k_q, c.k_s, kvrows, H, c.gs, c.k_rb, c.k_ng) ||
      !q4_ok(c.v_q, c.v_s, kvrows, H, c.gs, c.v_rb, c.v_ng))
    return fail_arg("%s: int4 projections need group sizes and widths that are multiples of 32 and 16-byte rows",
                    c.name);
  if (c.o_fmt == 4 ? !q4_ok(c.o_q, c.o_s, H, ctxn, c.gs, c.o_rb, c.o_ng) : !q8_ok(c.o_q, c.o_s, H, ctxn, c.o_rb))
    return fail_arg("%s: o projection layout not supported (int4 groups of 32k columns or int8 rows of 16k bytes)",
                    c.name);
  if ((hd != 64 && hd != 128 && hd != 256) || c.nh / c.nkv > 16 || c.rd > hd || (c.rd & 1))
    return fail_arg("%s: head_dim must be 64, 128 or 256 with at most 16 query heads per kv head", c.name);
  if (((uintptr_t)c.x & 15) || (H % 4)) return fail_arg("%s: activations must be 16-byte aligned", c.name);
  // key splits: about 256 workgroups in all, each split at least one 16-key
  // block per wave
  const int T = c.max_pos + 1;
  const int nb = (T + 15) / 16;
  int S = (256 + c.nkv * R - 1) / (c.nkv * R);
  const int smax = (nb + kAttnWaves - 1) / kAttnWaves;
  S = S > smax ? smax : S;
  S = S > kMaxSplits ? kMaxSplits : S;
  S = S < 1 ? 1 : S;
  const size_t psz = (size_t)16 * hd + 32;
  const size_t ox = 0, oqp = ox + align_up((size_t)R * H * 4), ok = oqp + align_up((size_t)R * qrows * 4),
               ov = ok + align_up((size_t)R * kvrows * 4), oq = ov + align_up((size_t)R * kvrows * 4),
               og = oq + align_up((size_t)R * ctxn * 4), oc = og + align_up((size_t)R * ctxn * 4),
               oy = oc + align_up((size_t)R * ctxn * 4), op = oy + align_up((size_t)R * H * 4),
               total = op + align_up((size_t)R * c.nkv * S * psz * 4);
  if (ensure_scratch(ctx, kScrMixer, total, c.name)) return -1;
  char *w = (char *)ctx->scratch[kScrMixer];
  const float *x = c.x;
  if (!c.device_io) {
    hipError_t e = hipMemcpyAsync(w + ox, c.x, (size_t)R * H * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip(c.name, e);
    x = (const float *)(w + ox);
  }
  float *qp = (float *)(w + oqp), *kr = (float *)(w + ok), *vr = (float *)(w + ov);
  float *q = (float *)(w + oq), *gate = (float *)(w + og), *cx = (float *)(w + oc);
  float *y = c.device_io ? c.out : (float *)(w + oy), *part = (float *)(w + op);

  for (int r0 = 0; r0 < R; r0 += kMixMaxTok) {
    const int n = R - r0 < kMixMaxTok ? R - r0 : kMixMaxTok;
    ProjArgs p;
    memset(&p, 0, sizeof(p));
    p.m[0] = pmat(c.q_q, c.q_s, qp + (size_t)r0 * qrows, qrows, c.q_rb, c.q_ng, qrows);
    p.m[1] = pmat(c.k_q, c.k_s, kr + (size_t)r0 * kvrows, kvrows, c.k_rb, c.k_ng, kvrows);
    p.m[2] = pmat(c.v_q, c.v_s, vr + (size_t)r0 * kvrows, kvrows, c.v_rb, c.v_ng, kvrows);
    p.nm = 3;
    p.rows_total = qrows + 2 * kvrows;
    p.x = x + (size_t)r0 * H;
    p.ldx = H;
    p.cols = H;
    p.gs = c.gs;
    p.B = n;
    launch_proj<4, false>(ctx, p);
  }
  PrepArgs pr;
  memset(&pr, 0, sizeof(pr));
  pr.qp = qp;
  pr.kr = kr;
  pr.vr = vr;
  pr.q_norm = c.q_norm;
  pr.k_norm = c.k_norm;
  pr.q = q;
  pr.gate = gate;
  pr.k_cache = c.k_cache;
  pr.v_cache = c.v_cache;
  pr.slot_stride = c.slot_stride;
  pr.nh = c.nh;
  pr.nkv = c.nkv;
  pr.hd = hd;
  pr.rd = c.rd;
  pr.theta = c.theta;
  pr.eps = c.eps;
  pr.tok = c.tok;
  k_gqa_prep<<<dim3(c.nh + c.nkv, R), hd, 0, ctx->stream>>>(pr);

  AttnArgs at;
  memset(&at, 0, sizeof(at));
  at.q = q;
  at.k_cache = c.k_cache;
  at.v_cache = c.v_cache;
  at.slot_stride = c.slot_stride;
  at.part = part;
  at.nh = c.nh;
  at.nkv = c.nkv;
  at.S = S;
  at.tok = c.tok;
  if (hd == 256)
    launch_attn<256>(ctx, at, R);
  else if (hd == 128)
    launch_attn<128>(ctx, at, R);
  else
    launch_attn<64>(ctx, at, R);

  CombArgs cb;
  cb.part = part;
  cb.gate = gate;
  cb.ctx = cx;
  cb.nh = c.nh;
  cb.nkv = c.nkv;
  cb.hd = hd;
  cb.S = S;
  k_gqa_combine<<<dim3(c.nh * (hd / 64), R), 256, 0, ctx->stream>>>(cb);

  for (int r0 = 0; r0 < R; r0 += kMixMaxTok) {
    const int n = R - r0 < kMixMaxTok ? R - r0 : kMixMaxTok;
    ProjArgs o;
    memset(&o, 0, sizeof(o));
    o.m[0] = pmat((const unsigned char *)c.o_q, c.o_s, y + (size_t)r0 * H, H, c.o_rb, c.o_ng, H);
    o.nm = 1;
    o.rows_total = H;
    o.x = cx + (size_t)r0 * ctxn;
    o.ldx = ctxn;
    o.cols = ctxn;
    o.gs = c.gs;
    o.B = n;
    if (c.o_fmt == 4)
      launch_proj<4, false>(ctx, o);
    else
      launch_proj<8, false>(ctx, o);
  }
  if (launch_status(c.name)) return -1;
  if (c.device_io) return 0;
  hipError_t e = hipMemcpyAsync(c.out, y, (size_t)R * H * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return fail_hip(c.name, e);
  e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? 0 : fail_hip(c.name, e);
}

bool gdn_common_ok(ColiCuda *ctx, float *out, const float *x, const float *a, const float *b,
                   const unsigned char *qkv_q, const float *qkv_s, const unsigned char *z_q, const float *z_s,
                   const unsigned char *out_q, const float *out_s, const float *conv_weight, const float *a_log,
                   const float *dt_bias, const float *norm_weight, float *conv_state, float *recurrent_state,
                   int hidden, int key_heads, int value_heads, int key_dim, int value_dim, int conv_kernel,
                   int group_size) {
  return ctx && out && x && a && b && qkv_q && qkv_s && z_q && z_s && out_q && out_s && conv_weight && a_log &&
         dt_bias && norm_weight && conv_state && recurrent_state && hidden > 0 && key_heads > 0 && value_heads > 0 &&
         key_dim > 0 && value_dim > 0 && value_heads % key_heads == 0 && conv_kernel > 0 && group_size > 0;
}

}  // namespace
}  // namespace sw

using namespace sw;

extern "C" int coli_cuda_gdn_decode_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b, const unsigned char *qkv_q,
    const float *qkv_s, int qkv_row_bytes, int qkv_groups, const unsigned char *z_q, const float *z_s,
    int z_row_bytes, int z_groups, const unsigned char *out_q, const float *out_s, int out_row_bytes, int out_groups,
    const float *conv_weight, const float *a_log, const float *dt_bias, const float *norm_weight, float *conv_state,
    float *recurrent_state, int position, int hidden, int key_heads, int value_heads, int key_dim, int value_dim,
    int conv_kernel, int group_size, float eps) {
  if (!gdn_common_ok(ctx, out, x, a, b, qkv_q, qkv_s, z_q, z_s, out_q, out_s, conv_weight, a_log, dt_bias,
                     norm_weight, conv_state, recurrent_state, hidden, key_heads, value_heads, key_dim, value_dim,
                     conv_kernel, group_size) ||
      position < 0 || value_dim > 256)
    return fail_arg("coli_cuda_gdn_decode_q4_f16: invalid argument");
  GdnCall c;
  memset(&c, 0, sizeof(c));
  c.name = "coli_cuda_gdn_decode_q4_f16";
  c.out = out;
  c.x = x;
  c.a = a;
  c.b = b;
  c.batch = 1;
  c.tok.tab = 0;
  c.tok.base = position;
  c.qkv_q = qkv_q, c.qkv_s = qkv_s, c.qkv_rb = qkv_row_bytes, c.qkv_ng = qkv_groups;
  c.z_q = z_q, c.z_s = z_s, c.z_rb = z_row_bytes, c.z_ng = z_groups;
  c.out_q = out_q, c.out_s = out_s, c.out_rb = out_row_bytes, c.out_ng = out_groups;
  c.conv_w = conv_weight, c.a_log = a_log, c.dt_bias = dt_bias, c.norm = norm_weight;
  c.conv_state = conv_state, c.state = recurrent_state;
  c.slots = 1, c.hidden = hidden, c.kh = key_heads, c.vh = value_heads, c.dk = key_dim, c.dv = value_dim;
  c.K = conv_kernel, c.gs = group_size, c.eps = eps;
  return gdn_run(ctx, c);
}

extern "C" int coli_cuda_gdn_block_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b, int batch, const unsigned char *qkv_q,
    const float *qkv_s, int qkv_row_bytes, int qkv_groups, const unsigned char *z_q, const float *z_s,
    int z_row_bytes, int z_groups, const unsigned char *out_q, const float *out_s, int out_row_bytes, int out_groups,
    const float *conv_weight, const float *a_log, const float *dt_bias, const float *norm_weight, float *conv_state,
    float *recurrent_state, int position, int hidden, int key_heads, int value_heads, int key_dim, int value_dim,
    int conv_kernel, int group_size, float eps) {
  if (!gdn_common_ok(ctx, out, x, a, b, qkv_q, qkv_s, z_q, z_s, out_q, out_s, conv_weight, a_log, dt_bias,
                     norm_weight, conv_state, recurrent_state, hidden, key_heads, value_heads, key_dim, value_dim,
                     conv_kernel, group_size) ||
      batch < 1 || batch > 8 || position < 0)
    return fail_arg("coli_cuda_gdn_block_q4_f16: invalid argument");
  GdnCall c;
  memset(&c, 0, sizeof(c));
  c.name = "coli_cuda_gdn_block_q4_f16";
  c.out = out;
  c.x = x;
  c.a = a;
  c.b = b;
  c.batch = batch;
  c.tok.tab = 0;
  c.tok.base = position;
  c.qkv_q = qkv_q, c.qkv_s = qkv_s, c.qkv_rb = qkv_row_bytes, c.qkv_ng = qkv_groups;
  c.z_q = z_q, c.z_s = z_s, c.z_rb = z_row_bytes, c.z_ng = z_groups;
  c.out_q = out_q, c.out_s = out_s, c.out_rb = out_row_bytes, c.out_ng = out_groups;
  c.conv_w = conv_weight, c.a_log = a_log, c.dt_bias = dt_bias, c.norm = norm_weight;
  c.conv_state = conv_state, c.state = recurrent_state;
  c.slots = 1, c.hidden = hidden, c.kh = key_heads, c.vh = value_heads, c.dk = key_dim, c.dv = value_dim;
  c.K = conv_kernel, c.gs = group_size, c.eps = eps;
  return gdn_run(ctx, c);
}

static int gdn_slots(const char *name, int device_io, ColiCuda *ctx, float *out, const float *x, const float *a,
                     const float *b, int batch, const int *slot, const int *position, const unsigned char *qkv_q,
                     const float *qkv_s, int qkv_row_bytes, int qkv_groups, const unsigned char *z_q,
                     const float *z_s, int z_row_bytes, int z_groups, const unsigned char *out_q, const float *out_s,
                     int out_row_bytes, int out_groups, const float *conv_weight, const float *a_log,
                     const float *dt_bias, const float *norm_weight, float *conv_state, float *recurrent_state,
                     int slots, int hidden, int key_heads, int value_heads, int key_dim, int value_dim,
                     int conv_kernel, int group_size, float eps) {
  if (!gdn_common_ok(ctx, out, x, a, b, qkv_q, qkv_s, z_q, z_s, out_q, out_s, conv_weight, a_log, dt_bias,
                     norm_weight, conv_state, recurrent_state, hidden, key_heads, value_heads, key_dim, value_dim,
                     conv_kernel, group_size) ||
      batch < 1 || batch > 16 || !slot || !position || slots < 1)
    return fail_arg("%s: invalid argument", name);
  GdnCall c;
  memset(&c, 0, sizeof(c));
  c.tok.tab = 1;
  c.tok.distinct = 1;
  for (int r = 0; r < batch; r++) {
    if (slot[r] < 0 || slot[r] >= slots || position[r] < 0) return fail_arg("%s: invalid slot", name);
    c.tok.slot[r] = slot[r];
    c.tok.pos[r] = position[r];
    for (int q = 0; q < r; q++)
      if (slot[q] == slot[r]) c.tok.distinct = 0;
  }
  c.name = name;
  c.out = out;
  c.x = x;
  c.a = a;
  c.b = b;
  c.batch = batch;
  c.device_io = device_io != 0;
  c.qkv_q = qkv_q, c.qkv_s = qkv_s, c.qkv_rb = qkv_row_bytes, c.qkv_ng = qkv_groups;
  c.z_q = z_q, c.z_s = z_s, c.z_rb = z_row_bytes, c.z_ng = z_groups;
  c.out_q = out_q, c.out_s = out_s, c.out_rb = out_row_bytes, c.out_ng = out_groups;
  c.conv_w = conv_weight, c.a_log = a_log, c.dt_bias = dt_bias, c.norm = norm_weight;
  c.conv_state = conv_state, c.state = recurrent_state;
  c.slots = slots, c.hidden = hidden, c.kh = key_heads, c.vh = value_heads, c.dk = key_dim, c.dv = value_dim;
  c.K = conv_kernel, c.gs = group_size, c.eps = eps;
  return gdn_run(ctx, c);
}

extern "C" int coli_cuda_gdn_slots_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b, int batch, const int *slot,
    const int *position, const unsigned char *qkv_q, const float *qkv_s, int qkv_row_bytes, int qkv_groups,
    const unsigned char *z_q, const float *z_s, int z_row_bytes, int z_groups, const unsigned char *out_q,
    const float *out_s, int out_row_bytes, int out_groups, const float *conv_weight, const float *a_log,
    const float *dt_bias, const float *norm_weight, float *conv_state, float *recurrent_state, int slots, int hidden,
    int key_heads, int value_heads, int key_dim, int value_dim, int conv_kernel, int group_size, float eps) {
  return gdn_slots("coli_cuda_gdn_slots_q4_f16", 0, ctx, out, x, a, b, batch, slot, position, qkv_q, qkv_s,
                   qkv_row_bytes, qkv_groups, z_q, z_s, z_row_bytes, z_groups, out_q, out_s, out_row_bytes,
                   out_groups, conv_weight, a_log, dt_bias, norm_weight, conv_state, recurrent_state, slots, hidden,
                   key_heads, value_heads, key_dim, value_dim, conv_kernel, group_size, eps);
}

extern "C" int coli_cuda_gdn_slots_q4_f16_device(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b, int batch, const int *slot,
    const int *position, const unsigned char *qkv_q, const float *qkv_s, int qkv_row_bytes, int qkv_groups,
    const unsigned char *z_q, const float *z_s, int z_row_bytes, int z_groups, const unsigned char *out_q,
    const float *out_s, int out_row_bytes, int out_groups, const float *conv_weight, const float *a_log,
    const float *dt_bias, const float *norm_weight, float *conv_state, float *recurrent_state, int slots, int hidden,
    int key_heads, int value_heads, int key_dim, int value_dim, int conv_kernel, int group_size, float eps) {
  return gdn_slots("coli_cuda_gdn_slots_q4_f16_device", 1, ctx, out, x, a, b, batch, slot, position, qkv_q, qkv_s,
                   qkv_row_bytes, qkv_groups, z_q, z_s, z_row_bytes, z_groups, out_q, out_s, out_row_bytes,
                   out_groups, conv_weight, a_log, dt_bias, norm_weight, conv_state, recurrent_state, slots, hidden,
                   key_heads, value_heads, key_dim, value_dim, conv_kernel, group_size, eps);
}

static bool gqa_common_ok(ColiCuda *ctx, float *out, const float *x, const unsigned char *q_q, const float *q_s,
                          const unsigned char *k_q, const float *k_s, const unsigned char *v_q, const float *v_s,
                          const void *o_q, const float *o_s, int o_fmt, const float *q_norm, const float *k_norm,
                          float *k_cache, float *v_cache, int hidden, int query_heads, int kv_heads, int head_dim) {
  return ctx && out && x && q_q && q_s && k_q && k_s && v_q && v_s && o_q && o_s && q_norm && k_norm && k_cache &&
         v_cache && hidden > 0 && query_heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim <= 256 &&
         query_heads % kv_heads == 0 && (o_fmt == 1 || o_fmt == 4);
}

static void gqa_fill(GqaCall &c, float *out, const float *x, const unsigned char *q_q, const float *q_s, int q_rb,
                     int q_ng, const unsigned char *k_q, const float *k_s, int k_rb, int k_ng,
                     const unsigned char *v_q, const float *v_s, int v_rb, int v_ng, const void *o_q,
                     const float *o_s, int o_fmt, int o_rb, int o_ng, const float *q_norm, const float *k_norm,
                     float *k_cache, float *v_cache, int hidden, int query_heads, int kv_heads, int head_dim,
                     int rotary_dim, int group_size, float theta, float eps) {
  c.out = out, c.x = x;
  c.q_q = q_q, c.q_s = q_s, c.q_rb = q_rb, c.q_ng = q_ng;
  c.k_q = k_q, c.k_s = k_s, c.k_rb = k_rb, c.k_ng = k_ng;
  c.v_q = v_q, c.v_s = v_s, c.v_rb = v_rb, c.v_ng = v_ng;
  c.o_q = o_q, c.o_s = o_s, c.o_fmt = o_fmt, c.o_rb = o_rb, c.o_ng = o_ng;
  c.q_norm = q_norm, c.k_norm = k_norm, c.k_cache = k_cache, c.v_cache = v_cache;
  c.hidden = hidden, c.nh = query_heads, c.nkv = kv_heads, c.hd = head_dim, c.rd = rotary_dim;
  c.gs = group_size, c.theta = theta, c.eps = eps;
}

extern "C" int coli_cuda_gqa_decode_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const unsigned char *q_q, const float *q_s, int q_rb, int q_ng,
    const unsigned char *k_q, const float *k_s, int k_rb, int k_ng, const unsigned char *v_q, const float *v_s,
    int v_rb, int v_ng, const void *o_q, const float *o_s, int o_fmt, int o_rb, int o_ng, const float *q_norm,
    const float *k_norm, float *k_cache, float *v_cache, int position, int hidden, int query_heads, int kv_heads,
    int head_dim, int rotary_dim, int group_size, float theta, float eps) {
  if (!gqa_common_ok(ctx, out, x, q_q, q_s, k_q, k_s, v_q, v_s, o_q, o_s, o_fmt, q_norm, k_norm, k_cache, v_cache,
                     hidden, query_heads, kv_heads, head_dim) ||
      position < 0)
    return fail_arg("coli_cuda_gqa_decode_q4_f16: invalid argument");
  GqaCall c;
  memset(&c, 0, sizeof(c));
  c.name = "coli_cuda_gqa_decode_q4_f16";
  gqa_fill(c, out, x, q_q, q_s, q_rb, q_ng, k_q, k_s, k_rb, k_ng, v_q, v_s, v_rb, v_ng, o_q, o_s, o_fmt, o_rb, o_ng,
           q_norm, k_norm, k_cache, v_cache, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta,
           eps);
  c.rows = 1;
  c.tok.tab = 0;
  c.tok.base = position;
  c.max_pos = position;
  c.slot_stride = 0;
  return gqa_run(ctx, c);
}

extern "C" int coli_cuda_gqa_prefill_q4_f16(
    ColiCuda *ctx, float *out, const float *x, int rows, int base, const unsigned char *q_q, const float *q_s,
    int q_rb, int q_ng, const unsigned char *k_q, const float *k_s, int k_rb, int k_ng, const unsigned char *v_q,
    const float *v_s, int v_rb, int v_ng, const void *o_q, const float *o_s, int o_fmt, int o_rb, int o_ng,
    const float *q_norm, const float *k_norm, float *k_cache, float *v_cache, int max_seq, int hidden,
    int query_heads, int kv_heads, int head_dim, int rotary_dim, int group_size, float theta, float eps) {
  if (!gqa_common_ok(ctx, out, x, q_q, q_s, k_q, k_s, v_q, v_s, o_q, o_s, o_fmt, q_norm, k_norm, k_cache, v_cache,
                     hidden, query_heads, kv_heads, head_dim) ||
      rows <= 0 || base < 0 || max_seq <= 0 || base + rows > max_seq)
    return fail_arg("coli_cuda_gqa_prefill_q4_f16: invalid argument");
  GqaCall c;
  memset(&c, 0, sizeof(c));
  c.name = "coli_cuda_gqa_prefill_q4_f16";
  gqa_fill(c, out, x, q_q, q_s, q_rb, q_ng, k_q, k_s, k_rb, k_ng, v_q, v_s, v_rb, v_ng, o_q, o_s, o_fmt, o_rb, o_ng,
           q_norm, k_norm, k_cache, v_cache, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta,
           eps);
  c.rows = rows;
  c.tok.tab = 0;
  c.tok.base = base;
  c.max_pos = base + rows - 1;
  c.slot_stride = 0;
  return gqa_run(ctx, c);
}

static int gqa_slots(const char *name, int device_io, ColiCuda *ctx, float *out, const float *x, int batch,
                     const int *slot, const int *position, const unsigned char *q_q, const float *q_s, int q_rb,
                     int q_ng, const unsigned char *k_q, const float *k_s, int k_rb, int k_ng,
                     const unsigned char *v_q, const float *v_s, int v_rb, int v_ng, const void *o_q,
                     const float *o_s, int o_fmt, int o_rb, int o_ng, const float *q_norm, const float *k_norm,
                     float *k_cache, float *v_cache, int slots, int max_seq, int hidden, int query_heads,
                     int kv_heads, int head_dim, int rotary_dim, int group_size, float theta, float eps) {
  if (!gqa_common_ok(ctx, out, x, q_q, q_s, k_q, k_s, v_q, v_s, o_q, o_s, o_fmt, q_norm, k_norm, k_cache, v_cache,
                     hidden, query_heads, kv_heads, head_dim) ||
      batch < 1 || batch > 16 || !slot || !position || slots < 1 || max_seq < 1)
    return fail_arg("%s: invalid argument", name);
  GqaCall c;
  memset(&c, 0, sizeof(c));
  c.tok.tab = 1;
  c.max_pos = 0;
  for (int r = 0; r < batch; r++) {
    if (slot[r] < 0 || slot[r] >= slots || position[r] < 0 || position[r] >= max_seq)
      return fail_arg("%s: invalid slot", name);
    c.tok.slot[r] = slot[r];
    c.tok.pos[r] = position[r];
    if (position[r] > c.max_pos) c.max_pos = position[r];
  }
  c.name = name;
  gqa_fill(c, out, x, q_q, q_s, q_rb, q_ng, k_q, k_s, k_rb, k_ng, v_q, v_s, v_rb, v_ng, o_q, o_s, o_fmt, o_rb, o_ng,
           q_norm, k_norm, k_cache, v_cache, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta,
           eps);
  c.rows = batch;
  c.device_io = device_io != 0;
  c.slot_stride = (long long)max_seq * kv_heads * head_dim;
  return gqa_run(ctx, c);
}

extern "C" int coli_cuda_gqa_slots_q4_f16(
    ColiCuda *ctx, float *out, const float *x, int batch, const int *slot, const int *position,
    const unsigned char *q_q, const float *q_s, int q_rb, int q_ng, const unsigned char *k_q, const float *k_s,
    int k_rb, int k_ng, const unsigned char *v_q, const float *v_s, int v_rb, int v_ng, const void *o_q,
    const float *o_s, int o_fmt, int o_rb, int o_ng, const float *q_norm, const float *k_norm, float *k_cache,
    float *v_cache, int slots, int max_seq, int hidden, int query_heads, int kv_heads, int head_dim, int rotary_dim,
    int group_size, float theta, float eps) {
  return gqa_slots("coli_cuda_gqa_slots_q4_f16", 0, ctx, out, x, batch, slot, position, q_q, q_s, q_rb, q_ng, k_q,
                   k_s, k_rb, k_ng, v_q, v_s, v_rb, v_ng, o_q, o_s, o_fmt, o_rb, o_ng, q_norm, k_norm, k_cache,
                   v_cache, slots, max_seq, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta,
                   eps);
}

extern "C" int coli_cuda_gqa_slots_q4_f16_device(
    ColiCuda *ctx, float *out, const float *x, int batch, const int *slot, const int *position,
    const unsigned char *q_q, const float *q_s, int q_rb, int q_ng, const unsigned char *k_q, const float *k_s,
    int k_rb, int k_ng, const unsigned char *v_q, const float *v_s, int v_rb, int v_ng, const void *o_q,
    const float *o_s, int o_fmt, int o_rb, int o_ng, const float *q_norm, const float *k_norm, float *k_cache,
    float *v_cache, int slots, int max_seq, int hidden, int query_heads, int kv_heads, int head_dim, int rotary_dim,
    int group_size, float theta, float eps) {
  return gqa_slots("coli_cuda_gqa_slots_q4_f16_device", 1, ctx, out, x, batch, slot, position, q_q, q_s, q_rb, q_ng,
                   k_q, k_s, k_rb, k_ng, v_q, v_s, v_rb, v_ng, o_q, o_s, o_fmt, o_rb, o_ng, q_norm, k_norm, k_cache,
                   v_cache, slots, max_seq, hidden, query_heads, kv_heads, head_dim, rotary_dim, group_size, theta,
                   eps);
}
