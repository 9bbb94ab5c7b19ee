/* CPU restatement of the reference's quantized MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the "port" CPU
 * baseline.  Nothing under shiftwing_amd/ links, loads or calls this file.
 *
 * What it restates (all in /root/reference/c/qwen.c):
 *   dot 1674, parallel_work 1675-1682, dot_q8f 1687-1695, qrow_i8 1696,
 *   dot_i8i8 1697-1705, dot_q4_group 1706-1716, dot_q2_group 1717-1724,
 *   q3_value 1725-1729,
 *   dot_q3_group 1730-1754 (+ q3_lut_init 416-429 / q3_word24 430-433),
 *   qmat_dot_row 1755-1760, qmat_mul_ex 1761-1773, qmat_mul_batch 3305-3329,
 *   sigmoidf_stable / siluf 307-308, mlp_batch 3407-3413, mlp_one 3415-3420,
 *   router_topk 3421-3426, moe_forward 3717-3739, moe_prefill_grouped
 *   4141-4206 with moe_prefill_route_gather 3956-3968 and
 *   moe_prefill_route_scatter 3969-3979.
 *
 * Arithmetic order.  The reference is built with gcc -O3 -march=native
 * (c/Makefile:42) on AVX-512 machines.  Its rounding is restated explicitly:
 *   - dot(): gcc vectorises the products in blocks of 8 and keeps an
 *     in-order scalar sum, s = rn(s + rn(a*b)); a remainder of n % 8 terms
 *     is an FMA chain (or_tail);
 *   - the scalar remainder loops of the grouped dots are FMA chains;
 *   - grouped dots: the AVX-512 lane structure (16- or 2x16-lane FMA
 *     accumulators, then _mm512_reduce_add_ps's halving tree), see
 *     or_reduce16;
 *   - loops that gcc contracts (group accumulation in qmat_dot_row, the
 *     weighted combine in moe_forward) use fmaf.
 * This file is compiled with -ffp-contract=off so that only the written
 * fmaf calls fuse.  The restatement is pinned bit for bit against the
 * compiled reference (oracle/_ref) and the reference's golden vectors by
 * tests/test_oracle_*.py.
 *
 * expf is glibc's, the same library the reference calls. */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../shiftwing_amd/csrc/sw_synth.h"

static int or_threads = 0;
void or_set_threads(int n) {
    or_threads = n;
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#endif
}
int or_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* parallel_work, qwen.c:1675-1682 (OMP_MIN_WORK default 262144). */
static int or_parallel_work(int64_t work) {
    static int64_t threshold = -1;
    if (threshold < 0) {
        const char *e = getenv("OMP_MIN_WORK");
        threshold = e ? atoll(e) : 262144;
    }
#ifdef _OPENMP
    return work >= threshold && !omp_in_parallel();
#else
    (void)work;
    return 0;
#endif
}

/* _mm512_reduce_add_ps: upper 256 + lower 256, upper 128 + lower 128, then
 * lanes {2,3} onto {0,1}, then lane 1 onto lane 0. */
static float or_reduce16(const float *t) {
    float a[8], b[4], c0, c1;
    for (int j = 0; j < 8; j++) a[j] = t[8 + j] + t[j];
    for (int j = 0; j < 4; j++) b[j] = a[4 + j] + a[j];
    c0 = b[0] + b[2];
    c1 = b[1] + b[3];
    return c0 + c1;
}

/* In-order float sum over products p_i = a_i * b_i as gcc -O3 emits dot():
 * whole blocks of 8 are vectorised (products rounded, then added in order)
 * and the remainder is a contracted FMA chain. */
static float or_tail(float sum, const float *a, const float *b, int n) {
    int m = (n / 8) * 8, i = 0;
    for (; i < m; i++) {
        float p = a[i] * b[i];
        sum = sum + p;
    }
    for (; i < n; i++) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* The scalar remainder loops after the AVX-512 bodies of the grouped dots
 * are not vectorised; gcc contracts them to one FMA chain. */
static float or_tail_fma(float sum, const float *a, const float *b, int n) {
    for (int i = 0; i < n; i++) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* dot, qwen.c:1674 */
float or_dot_f32(const float *a, const float *b, int n) {
    return or_tail(0.f, a, b, n);
}

/* dot_q8f, qwen.c:1687-1695 (AVX-512 branch) */
float or_dot_q8f(const int8_t *w, const float *x, int n) {
    float acc[16] = {0}, sum;
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++)
            acc[j] = fmaf(x[i + j], (float)w[i + j], acc[j]);
    sum = or_reduce16(acc);
    float wf[16];
    int r = n - i;
    for (int j = 0; j < r; j++) wf[j] = (float)w[i + j];
    return or_tail_fma(sum, x + i, wf, r);
}

/* qrow_i8, qwen.c:1696 */
float or_qrow_i8(const float *x, int8_t *q, int n) {
    float amax = 0.f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float s = amax / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    float inv = 1.f / s;
    for (int i = 0; i < n; i++) q[i] = (int8_t)lrintf(x[i] * inv);
    return s;
}

/* dot_i8i8, qwen.c:1697-1705: an exact integer dot in any order. */
int32_t or_dot_i8i8(const int8_t *w, const int8_t *x, int n) {
    int32_t sum = 0;
    for (int i = 0; i < n; i++) sum += (int32_t)w[i] * x[i];
    return sum;
}

/* dot_q4_group, qwen.c:1706-1716 (AVX-512 branch: a0 covers i..i+15 and a1
 * covers i+16..i+31 of each 32-wide step). */
float or_dot_q4_group(const uint8_t *w, const float *x, int n) {
    float a0[16] = {0}, a1[16] = {0}, t[16], sum;
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 16; j++) {
            int k0 = i + j, k1 = i + 16 + j;
            uint8_t b0 = w[k0 >> 1], b1 = w[k1 >> 1];
            int q0 = ((k0 & 1) ? (b0 >> 4) : (b0 & 15)) - 8;
            int q1 = ((k1 & 1) ? (b1 >> 4) : (b1 & 15)) - 8;
            a0[j] = fmaf(x[k0], (float)q0, a0[j]);
            a1[j] = fmaf(x[k1], (float)q1, a1[j]);
        }
    for (int j = 0; j < 16; j++) t[j] = a0[j] + a1[j];
    sum = or_reduce16(t);
    float wf[32];
    int r = n - i;
    for (int j = 0; j < r; j++) {
        uint8_t b = w[(i + j) >> 1];
        wf[j] = (float)((((i + j) & 1) ? (b >> 4) : (b & 15)) - 8);
    }
    return or_tail_fma(sum, x + i, wf, r);
}

/* dot_q2_group, qwen.c:1717-1724: four 2-bit codes a byte, lowest bits
 * first, value 2 code - 3; a scalar loop, which gcc keeps in order and
 * contracts into an FMA chain. */
float or_dot_q2_group(const uint8_t *w, const float *x, int n) {
    float sum = 0.f;
    for (int i = 0; i < n; i++) {
        const int code = (w[i >> 2] >> (2 * (i & 3))) & 3;
        sum = fmaf(x[i], (float)(2 * code - 3), sum);
    }
    return sum;
}

/* q3_value, qwen.c:1725-1729 */
int or_q3_value(const uint8_t *w, int i) {
    int bit = 3 * i, byte = bit >> 3, shift = bit & 7;
    uint16_t word = w[byte];
    if (shift > 5) word |= (uint16_t)w[byte + 1] << 8;
    return (int)((word >> shift) & 7) - 4;
}

/* dot_q3_group, qwen.c:1730-1754 (AVX-512 branch: one 16-lane accumulator,
 * two 24-bit triplet words per step). */
float or_dot_q3_group(const uint8_t *w, const float *x, int n) {
    float acc[16] = {0}, sum;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        const uint8_t *p = w + (i * 3 / 8);
        uint32_t wa = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16);
        uint32_t wb = (uint32_t)p[3] | ((uint32_t)p[4] << 8) | ((uint32_t)p[5] << 16);
        for (int j = 0; j < 16; j++) {
            uint32_t word = j < 8 ? wa : wb;
            int v = (int)((word >> (3 * (j & 7))) & 7u) - 4;
            acc[j] = fmaf(x[i + j], (float)v, acc[j]);
        }
    }
    sum = or_reduce16(acc);
    float wf[16];
    int r = n - i;
    for (int j = 0; j < r; j++) wf[j] = (float)or_q3_value(w, i + j);
    return or_tail_fma(sum, x + i, wf, r);
}

/* qmat_dot_row, qwen.c:1755-1760 (fmt 0, 1, 2, 3, 4). */
float or_qmat_dot_row(const or_qmat *w, int row, const float *x) {
    if (w->fmt == 0) return or_dot_f32(x, w->f + (int64_t)row * w->I, w->I);
    if (w->fmt == 1)
        return or_dot_q8f((const int8_t *)w->q + (int64_t)row * w->rb, x, w->I) *
               w->s[row];
    const uint8_t *q = (const uint8_t *)w->q + (int64_t)row * w->rb;
    const float *s = w->s + (int64_t)row * w->ng;
    float out = 0.f;
    for (int g = 0; g < w->ng; g++) {
        int base = g * w->gs, n = w->gs;
        if (base + n > w->I) n = w->I - base;
        if (n > 0) {
            float v = w->fmt == 2   ? or_dot_q2_group(q + (base >> 2), x + base, n)
                      : w->fmt == 3 ? or_dot_q3_group(q + (base * 3 / 8), x + base, n)
                                    : or_dot_q4_group(q + (base >> 1), x + base, n);
            out = fmaf(v, s[g], out);
        }
    }
    return out;
}

static int or_idot_enabled(void) {
    static int idot = -1;
    if (idot < 0) {
        const char *e = getenv("IDOT");
        idot = e ? atoi(e) != 0 : 1;
    }
    return idot;
}

/* qmat_mul_ex, qwen.c:1761-1773 (IDOT branch for fmt 1). */
void or_qmat_mul(float *y, const float *x, const or_qmat *w, int allow_idot) {
    if (w->fmt == 1 && or_idot_enabled() && allow_idot) {
        int8_t *qb = (int8_t *)malloc((size_t)w->I);
        float sx = or_qrow_i8(x, qb, w->I);
        int par = or_parallel_work((int64_t)w->O * w->I);
        const int8_t *q8 = (const int8_t *)w->q;
#pragma omp parallel for schedule(static) if (par)
        for (int o = 0; o < w->O; o++)
            y[o] = (float)or_dot_i8i8(q8 + (int64_t)o * w->rb, qb, w->I) * w->s[o] * sx;
        free(qb);
        return;
    }
    int par = or_parallel_work((int64_t)w->O * w->I);
#pragma omp parallel for schedule(static) if (par)
    for (int o = 0; o < w->O; o++) y[o] = or_qmat_dot_row(w, o, x);
}

/* qmat_mul_batch, qwen.c:3305-3329.  The AVX-512 panel path (3251-3298) is
 * bit-identical to per-row qmat_dot_row (c/tests/test_quant_matmul.c:72-86),
 * so the per-row form is restated. */
void or_qmat_mul_batch(float *y, const float *x, int B, int ldx,
                       const or_qmat *w, int allow_idot) {
    if (B <= 0) return;
    if (B == 1) {
        or_qmat_mul(y, x, w, allow_idot);
        return;
    }
    int par = or_parallel_work((int64_t)w->O * w->I * B);
    if (w->fmt == 1 && or_idot_enabled() && allow_idot) {
        int8_t *q = (int8_t *)calloc((size_t)B * w->I, 1);
        float *sx = (float *)calloc((size_t)B, sizeof(float));
        const int8_t *q8 = (const int8_t *)w->q;
        for (int b = 0; b < B; b++)
            sx[b] = or_qrow_i8(x + (int64_t)b * ldx, q + (int64_t)b * w->I, w->I);
#pragma omp parallel for schedule(static) if (par)
        for (int o = 0; o < w->O; o++) {
            const int8_t *row = q8 + (int64_t)o * w->rb;
            float s = w->s[o];
            for (int b = 0; b < B; b++)
                y[(int64_t)b * w->O + o] =
                    (float)or_dot_i8i8(row, q + (int64_t)b * w->I, w->I) * s * sx[b];
        }
        free(q);
        free(sx);
        return;
    }
#pragma omp parallel for schedule(static) if (par)
    for (int o = 0; o < w->O; o++)
        for (int b = 0; b < B; b++)
            y[(int64_t)b * w->O + o] = or_qmat_dot_row(w, o, x + (int64_t)b * ldx);
}

/* sigmoidf_stable / siluf, qwen.c:307-308 (glibc expf). */
/* rmsnorm_zero (c/qwen.c:1780-1784), the step before the MoE
 * (c/qwen.c:4593): the sum of squares is a serial chain, multiply then add,
 * as the reference's flags compile it (the same finding as for dot()). */
void or_rmsnorm_zero(float *out, const float *x, const float *w, int n, float eps) {
    float ms = 0.f;
    for (int i = 0; i < n; i++) {
        const float p = x[i] * x[i];
        ms = ms + p;
    }
    const float r = 1.f / sqrtf(ms / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * r * (1.f + w[i]);
}

float or_expf(float x) { return expf(x); }
float or_sigmoidf(float x) {
    if (x >= 0) {
        float z = expf(-x);
        return 1.f / (1.f + z);
    }
    float z = expf(x);
    return z / (1.f + z);
}
float or_siluf(float x) { return x * or_sigmoidf(x); }

/* Batch forms of the above for exhaustive device comparisons. */
void or_sigmoid_batch(const float *x, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = or_sigmoidf(x[i]);
}
void or_expf_batch(const float *x, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* router_topk, qwen.c:3421-3426: softmax over all E (serial denominator in
 * expert order), K rounds of argmax with strict '>' (lowest index wins a
 * tie), then renormalisation of the K picked probabilities. */
void or_router_topk(const float *logit, int E, int K, int *idx, float *weight) {
    float mx = -INFINITY;
    for (int e = 0; e < E; e++)
        if (logit[e] > mx) mx = logit[e];
    float *prob = (float *)calloc((size_t)E, sizeof(float)), den = 0.f;
    for (int e = 0; e < E; e++) {
        prob[e] = expf(logit[e] - mx);
        den += prob[e];
    }
    for (int e = 0; e < E; e++) prob[e] /= den;
    for (int j = 0; j < K; j++) {
        int best = -1;
        float bv = -1.f;
        for (int e = 0; e < E; e++) {
            int used = 0;
            for (int p = 0; p < j; p++)
                if (idx[p] == e) used = 1;
            if (!used && prob[e] > bv) {
                bv = prob[e];
                best = e;
            }
        }
        idx[j] = best;
        weight[j] = bv;
    }
    float topden = 0.f;
    for (int j = 0; j < K; j++) topden += weight[j];
    for (int j = 0; j < K; j++) weight[j] /= topden;
    free(prob);
}

/* mlp_one, qwen.c:3415-3420 */
void or_mlp_one(float *out, const float *x, const or_qmat *gate,
                const or_qmat *up, const or_qmat *down, int I) {
    float *g = (float *)calloc((size_t)I, sizeof(float));
    float *u = (float *)calloc((size_t)I, sizeof(float));
    or_qmat_mul(g, x, gate, 1);
    or_qmat_mul(u, x, up, 1);
    for (int i = 0; i < I; i++) g[i] = or_siluf(g[i]) * u[i];
    or_qmat_mul(out, g, down, 1);
    free(g);
    free(u);
}

/* mlp_batch, qwen.c:3407-3413 */
void or_mlp_batch(float *out, const float *x, int B, int ldx,
                  const or_qmat *gate, const or_qmat *up, const or_qmat *down,
                  int I) {
    float *g = (float *)calloc((size_t)B * I, sizeof(float));
    float *u = (float *)calloc((size_t)B * I, sizeof(float));
    or_qmat_mul_batch(g, x, B, ldx, gate, 1);
    or_qmat_mul_batch(u, x, B, ldx, up, 1);
    for (int64_t i = 0; i < (int64_t)B * I; i++) g[i] = or_siluf(g[i]) * u[i];
    or_qmat_mul_batch(out, g, B, I, down, 1);
    free(g);
    free(u);
}

/* moe_forward, qwen.c:3717-3739 (expert cache and CUDA branches removed:
 * every expert is resident). */
void or_moe_forward(const or_layer *L, const float *x, float *out, or_trace *tr) {
    int E = L->E, K = L->K, H = L->H;
    float *logit = (float *)calloc((size_t)E, sizeof(float));
    float *tmp = (float *)calloc((size_t)K * H, sizeof(float));
    float *shared = (float *)calloc((size_t)H, sizeof(float));
    int *idx = (int *)calloc((size_t)K, sizeof(int));
    float *weight = (float *)calloc((size_t)K, sizeof(float));
    or_qmat_mul(logit, x, &L->router, 0);
    or_router_topk(logit, E, K, idx, weight);
    memset(out, 0, (size_t)H * sizeof(float));
    int par = or_parallel_work((int64_t)K * (2 * L->I * H + L->I * H));
#pragma omp parallel for schedule(static) if (par)
    for (int j = 0; j < K; j++)
        or_mlp_one(tmp + (int64_t)j * H, x, &L->gate[idx[j]], &L->up[idx[j]],
                   &L->down[idx[j]], L->I);
    for (int j = 0; j < K; j++)
        for (int h = 0; h < H; h++) out[h] = fmaf(tmp[(int64_t)j * H + h], weight[j], out[h]);
    or_mlp_one(shared, x, &L->shared_gate, &L->shared_up, &L->shared_down, L->I_sh);
    float sglog;
    or_qmat_mul(&sglog, x, &L->shared_scale, 0);
    float sg = or_sigmoidf(sglog);
    for (int h = 0; h < H; h++) out[h] = fmaf(shared[h], sg, out[h]);
    if (tr) {
        if (tr->logits) memcpy(tr->logits, logit, (size_t)E * sizeof(float));
        if (tr->idx) memcpy(tr->idx, idx, (size_t)K * sizeof(int));
        if (tr->weight) memcpy(tr->weight, weight, (size_t)K * sizeof(float));
        if (tr->shared) memcpy(tr->shared, shared, (size_t)H * sizeof(float));
        if (tr->sgate) tr->sgate[0] = sg;
    }
    free(logit);
    free(tmp);
    free(shared);
    free(idx);
    free(weight);
}

/* moe_prefill_route_gather, qwen.c:3956-3968 (indices only). */
static int or_route_gather(int eid, const int *idx, const float *weight, int T,
                           int K, int *tok, float *wt) {
    int B = 0;
    for (int t = 0; t < T; t++)
        for (int j = 0; j < K; j++)
            if (idx[(int64_t)t * K + j] == eid) {
                tok[B] = t;
                wt[B] = weight[(int64_t)t * K + j];
                B++;
                break;
            }
    return B;
}

int or_bucket(const int *idx, int T, int K, int E, int *offsets, int *token,
              int *slot) {
    int n = 0;
    for (int e = 0; e < E; e++) {
        offsets[e] = n;
        for (int t = 0; t < T; t++)
            for (int j = 0; j < K; j++)
                if (idx[(int64_t)t * K + j] == e) {
                    token[n] = t;
                    slot[n] = j;
                    n++;
                    break;
                }
    }
    offsets[E] = n;
    return n;
}

/* moe_prefill_grouped, qwen.c:4141-4206 (host path; every expert resident,
 * PREFILL_EXPERT_BATCH=1 so experts run one at a time in ascending id). */
void or_moe_prefill_grouped(const or_layer *L, const float *x, int T, float *out,
                            or_trace *tr) {
    int E = L->E, K = L->K, H = L->H;
    int *idx = (int *)calloc((size_t)T * K, sizeof(int));
    float *weight = (float *)calloc((size_t)T * K, sizeof(float));
    float *tmp = (float *)calloc((size_t)T * H, sizeof(float));
    float *routed = (float *)calloc((size_t)T * K * H, sizeof(float));
    float *shared = (float *)calloc((size_t)T * H, sizeof(float));
    float *sgs = (float *)calloc((size_t)T, sizeof(float));
    unsigned char *used = (unsigned char *)calloc((size_t)E, 1);
    float *logits = (float *)calloc((size_t)T * E, sizeof(float));
#pragma omp parallel for schedule(static) if (T > 1)
    for (int t = 0; t < T; t++) {
        float *logit = logits + (int64_t)t * E;
        or_qmat_mul(logit, x + (int64_t)t * H, &L->router, 0);
        or_router_topk(logit, E, K, idx + (int64_t)t * K, weight + (int64_t)t * K);
    }
    for (int t = 0; t < T; t++)
        for (int j = 0; j < K; j++) used[idx[(int64_t)t * K + j]] = 1;
    or_mlp_batch(shared, x, T, H, &L->shared_gate, &L->shared_up, &L->shared_down,
                 L->I_sh);
    if (tr && tr->shared) memcpy(tr->shared, shared, (size_t)T * H * sizeof(float));
#pragma omp parallel for schedule(static) if (T > 1)
    for (int t = 0; t < T; t++) {
        float *ot = shared + (int64_t)t * H, sg;
        or_qmat_mul(&sg, x + (int64_t)t * H, &L->shared_scale, 0);
        sg = or_sigmoidf(sg);
        sgs[t] = sg;
        for (int h = 0; h < H; h++) ot[h] *= sg;
    }
    int *tok = (int *)calloc((size_t)T, sizeof(int));
    float *wt = (float *)calloc((size_t)T, sizeof(float));
    float *xb = (float *)calloc((size_t)T * H, sizeof(float));
    for (int eid = 0; eid < E; eid++) {
        if (!used[eid]) continue;
        int B = or_route_gather(eid, idx, weight, T, K, tok, wt);
        for (int b = 0; b < B; b++)
            memcpy(xb + (int64_t)b * H, x + (int64_t)tok[b] * H, (size_t)H * sizeof(float));
        or_mlp_batch(tmp, xb, B, H, &L->gate[eid], &L->up[eid], &L->down[eid], L->I);
        for (int b = 0; b < B; b++) {
            int t = tok[b], route = 0;
            while (route < K && idx[(int64_t)t * K + route] != eid) route++;
            float *ot = routed + ((int64_t)t * K + route) * H;
            const float *tt = tmp + (int64_t)b * H;
            float g = wt[b];
            for (int h = 0; h < H; h++) ot[h] = tt[h] * g;
        }
    }
    for (int t = 0; t < T; t++) {
        float *ot = out + (int64_t)t * H;
        memset(ot, 0, (size_t)H * sizeof(float));
        for (int j = 0; j < K; j++) {
            const float *rt = routed + ((int64_t)t * K + j) * H;
            for (int h = 0; h < H; h++) ot[h] += rt[h];
        }
        for (int h = 0; h < H; h++) ot[h] += shared[(int64_t)t * H + h];
    }
    if (tr) {
        if (tr->logits) memcpy(tr->logits, logits, (size_t)T * E * sizeof(float));
        if (tr->idx) memcpy(tr->idx, idx, (size_t)T * K * sizeof(int));
        if (tr->weight) memcpy(tr->weight, weight, (size_t)T * K * sizeof(float));
        if (tr->sgate) memcpy(tr->sgate, sgs, (size_t)T * sizeof(float));
    }
    free(tok);
    free(wt);
    free(xb);
    free(idx);
    free(weight);
    free(tmp);
    free(routed);
    free(shared);
    free(sgs);
    free(used);
    free(logits);
}

/* ---- host materialisation of the synthetic inputs (sw_synth.h) ---- */

void or_synth_bytes(uint64_t seed, int layer, int eid, int tensor, uint8_t *out,
                    uint64_t n) {
    uint64_t key = sw_key(seed, (uint32_t)layer, (uint32_t)eid, (uint32_t)tensor);
    int64_t words = (int64_t)((n + 7) / 8);
#pragma omp parallel for schedule(static) if (n >= (1u << 22))
    for (int64_t w = 0; w < words; w++) {
        uint64_t h = sw_word(key, (uint64_t)w);
        for (int b = 0; b < 8; b++) {
            uint64_t i = (uint64_t)w * 8 + (uint64_t)b;
            if (i < n) out[i] = (uint8_t)(h >> (8 * b));
        }
    }
}

static void or_synth_normals(uint64_t key, float *out, int64_t n, float sigma,
                             int absolute) {
#pragma omp parallel for schedule(static) if (n >= (1 << 18))
    for (int64_t i = 0; i < n; i++)
        out[i] = absolute ? sw_abs_normal_sigma(key, (uint64_t)i, sigma)
                          : sw_normal_sigma(key, (uint64_t)i, sigma);
}

void or_synth_router(uint64_t seed, int layer, int E, int H, float *router,
                     float *shared_gate) {
    if (router)
        or_synth_normals(sw_key(seed, (uint32_t)layer, 0, SW_T_ROUTER), router,
                         (int64_t)E * H, 0.02f, 0);
    if (shared_gate)
        or_synth_normals(sw_key(seed, (uint32_t)layer, 0, SW_T_SHARED_GATE),
                         shared_gate, H, 0.02f, 0);
}

static void or_synth_i8(uint64_t key, int8_t *out, int64_t n) {
#pragma omp parallel for schedule(static) if (n >= (1 << 20))
    for (int64_t i = 0; i < n; i++) out[i] = sw_i8(key, (uint64_t)i);
}

void or_synth_shared_q8(uint64_t seed, int layer, int H, int I_sh, int8_t *gq,
                        float *gs, int8_t *uq, float *us, int8_t *dq, float *ds) {
    uint32_t l = (uint32_t)layer;
    or_synth_i8(sw_key(seed, l, 0, SW_T_SH_GATE_Q), gq, (int64_t)I_sh * H);
    or_synth_normals(sw_key(seed, l, 0, SW_T_SH_GATE_S), gs, I_sh, 0.01f, 1);
    or_synth_i8(sw_key(seed, l, 0, SW_T_SH_UP_Q), uq, (int64_t)I_sh * H);
    or_synth_normals(sw_key(seed, l, 0, SW_T_SH_UP_S), us, I_sh, 0.01f, 1);
    or_synth_i8(sw_key(seed, l, 0, SW_T_SH_DOWN_Q), dq, (int64_t)H * I_sh);
    or_synth_normals(sw_key(seed, l, 0, SW_T_SH_DOWN_S), ds, H, 0.01f, 1);
}

static int or_row_bytes(int fmt, int cols, int gs) {
    int ng = (cols + gs - 1) / gs;
    return fmt == 4 ? ng * gs / 2 : fmt == 2 ? ng * gs / 4 : ng * gs * 3 / 8;
}

void or_synth_expert(uint64_t seed, int layer, int eid, int fmt, int H, int I,
                     int gs, uint8_t *gq, float *gsc, uint8_t *uq, float *usc,
                     uint8_t *dq, float *dsc) {
    int rbh = or_row_bytes(fmt, H, gs), rbi = or_row_bytes(fmt, I, gs);
    int ngh = (H + gs - 1) / gs, ngi = (I + gs - 1) / gs;
    uint32_t l = (uint32_t)layer, e = (uint32_t)eid;
    or_synth_bytes(seed, layer, eid, SW_T_GATE_Q, gq, (uint64_t)I * rbh);
    or_synth_normals(sw_key(seed, l, e, SW_T_GATE_S), gsc, (int64_t)I * ngh, 0.01f, 1);
    or_synth_bytes(seed, layer, eid, SW_T_UP_Q, uq, (uint64_t)I * rbh);
    or_synth_normals(sw_key(seed, l, e, SW_T_UP_S), usc, (int64_t)I * ngh, 0.01f, 1);
    or_synth_bytes(seed, layer, eid, SW_T_DOWN_Q, dq, (uint64_t)H * rbi);
    or_synth_normals(sw_key(seed, l, e, SW_T_DOWN_S), dsc, (int64_t)H * ngi, 0.01f, 1);
}

void or_synth_x(uint64_t seed, int layer, int step, int H, float *x) {
    or_synth_normals(sw_key(seed, (uint32_t)layer, (uint32_t)step, SW_T_X), x, H,
                     1.0f, 0);
}

/* ---- the mixer layers either side of the MoE block ----------------------
 * Gated DeltaNet decode (gdn_forward, c/qwen.c:3005-3030, with
 * gdn_rule_step 2907-2927) and gated GQA attention decode (attn_forward,
 * c/qwen.c:3094-3137, with rope_head 3031-3033).  The projections are
 * qmat_mul_ex (restated above); the transcendental functions are glibc's, as
 * the reference calls them.  Which products gcc fuses into an FMA in these
 * loops is pinned against the compiled reference (tests/test_oracle_cpu.py). */

/* softplusf_stable, c/qwen.c:309 */
static float or_softplusf(float x) {
    return x > 20.f ? x : (x < -20.f ? expf(x) : log1pf(expf(x)));
}

void or_gdn_gates(const or_gdn *G, const float *x, float *a, float *b) {
    or_qmat_mul(b, x, &G->b, 0);
    or_qmat_mul(a, x, &G->a, 0);
}

/* gdn_rule_step, c/qwen.c:2907-2927, for one token */
static void or_gdn_rule_step(float *core, float *state, const float *q, const float *k,
                             const float *v, const float *z, const float *a, const float *b,
                             const or_gdn *G) {
    const int kh = G->kh, vh = G->vh, dk = G->dk, dv = G->dv, ratio = vh / kh;
    const float invsqrt = 1.f / sqrtf((float)dk);
    for (int h = 0; h < vh; h++) {
        const int hk = h / ratio;
        float *S = state + (int64_t)h * dk * dv;
        const float *qh = q + (int64_t)hk * dk, *kv = k + (int64_t)hk * dk, *vv = v + (int64_t)h * dv;
        float qn = 0.f, kn = 0.f;
        for (int i = 0; i < dk; i++) {
            const float pq = qh[i] * qh[i], pk = kv[i] * kv[i];
            qn = qn + pq;
            kn = kn + pk;
        }
        qn = 1.f / sqrtf(qn + 1e-6f);
        kn = 1.f / sqrtf(kn + 1e-6f);
        const float beta = or_sigmoidf(b[h]);
        const float decay = expf(-expf(G->A_log[h]) * or_softplusf(a[h] + G->dt_bias[h]));
        for (int64_t i = 0; i < (int64_t)dk * dv; i++) S[i] *= decay;
        for (int j = 0; j < dv; j++) {
            float mem = 0.f;
            for (int i = 0; i < dk; i++) {
                const float p = S[(int64_t)i * dv + j] * (kv[i] * kn);
                mem = mem + p;
            }
            const float delta = (vv[j] - mem) * beta;
            for (int i = 0; i < dk; i++)
                S[(int64_t)i * dv + j] = fmaf(kv[i] * kn, delta, S[(int64_t)i * dv + j]);
        }
        for (int j = 0; j < dv; j++) {
            float sum = 0.f;
            for (int i = 0; i < dk; i++) {
                const float p = S[(int64_t)i * dv + j] * (qh[i] * qn * invsqrt);
                sum = sum + p;
            }
            core[(int64_t)h * dv + j] = sum;
        }
        float ms = 0.f;
        for (int j = 0; j < dv; j++) {
            const float c0 = core[(int64_t)h * dv + j];
            const float p = c0 * c0;
            ms = ms + p;
        }
        const float r = 1.f / sqrtf(ms / (float)dv + G->eps);
        for (int j = 0; j < dv; j++)
            core[(int64_t)h * dv + j] =
                core[(int64_t)h * dv + j] * r * G->norm[j] * or_siluf(z[(int64_t)h * dv + j]);
    }
}

/* gdn_forward, c/qwen.c:3005-3030, after the a/b projections */
void or_gdn_forward(const or_gdn *G, const float *x, const float *a, const float *b, int pos,
                    float *conv_state, float *state, float *out) {
    const int kd = G->kh * G->dk, vd = G->vh * G->dv, cd = 2 * kd + vd, K = G->K;
    float *raw = (float *)calloc((size_t)cd, sizeof(float));
    float *mix = (float *)calloc((size_t)cd, sizeof(float));
    float *z = (float *)calloc((size_t)vd, sizeof(float));
    float *core = (float *)calloc((size_t)vd, sizeof(float));
    or_qmat_mul(raw, x, &G->qkv, 0);
    or_qmat_mul(z, x, &G->z, 0);
    memcpy(conv_state + (int64_t)(pos % K) * cd, raw, (size_t)cd * sizeof(float));
    for (int ch = 0; ch < cd; ch++) {
        float acc = 0.f;
        for (int tap = 0; tap < K; tap++) {
            const int src = pos - (K - 1 - tap);
            if (src >= 0)
                acc = fmaf(G->conv[(int64_t)ch * K + tap], conv_state[(int64_t)(src % K) * cd + ch], acc);
        }
        mix[ch] = or_siluf(acc);
    }
    or_gdn_rule_step(core, state, mix, mix + kd, mix + 2 * kd, z, a, b, G);
    or_qmat_mul(out, core, &G->out, 0);
    free(raw);
    free(mix);
    free(z);
    free(core);
}

/* rope_head, c/qwen.c:3031-3033 */
static void or_rope_head(float *x, int rd, int pos, float theta) {
    const int half = rd / 2;
    for (int i = 0; i < half; i++) {
        const float angle = (float)pos * powf(theta, -2.f * (float)i / (float)rd);
        const float co = cosf(angle), si = sinf(angle);
        const float a = x[i], b = x[i + half];
        x[i] = fmaf(a, co, -(b * si));
        x[i + half] = fmaf(b, co, a * si);
    }
}

/* attn_forward, c/qwen.c:3094-3137: fp32 caches, no indexer mask */
void or_attn_forward(const or_attn *A, const float *x, int pos, float *k_cache, float *v_cache,
                     float *out) {
    const int nh = A->nh, nkv = A->nkv, hd = A->hd;
    const int qrows = nh * hd * 2, kvrows = nkv * hd;
    float *qp = (float *)calloc((size_t)qrows, sizeof(float));
    float *q = (float *)calloc((size_t)nh * hd, sizeof(float));
    float *gate = (float *)calloc((size_t)nh * hd, sizeof(float));
    float *k = (float *)calloc((size_t)kvrows, sizeof(float));
    float *v = (float *)calloc((size_t)kvrows, sizeof(float));
    float *ctx = (float *)calloc((size_t)nh * hd, sizeof(float));
    float *scores = (float *)calloc((size_t)nh * (pos + 1), sizeof(float));
    or_qmat_mul(qp, x, &A->q, 0);
    or_qmat_mul(k, x, &A->k, 0);
    or_qmat_mul(v, x, &A->v, 0);
    for (int h = 0; h < nh; h++) {
        memcpy(q + (int64_t)h * hd, qp + (int64_t)h * 2 * hd, (size_t)hd * sizeof(float));
        memcpy(gate + (int64_t)h * hd, qp + (int64_t)h * 2 * hd + hd, (size_t)hd * sizeof(float));
        or_rmsnorm_zero(q + (int64_t)h * hd, q + (int64_t)h * hd, A->q_norm, hd, A->eps);
        or_rope_head(q + (int64_t)h * hd, A->rd, pos, A->theta);
    }
    for (int h = 0; h < nkv; h++) {
        or_rmsnorm_zero(k + (int64_t)h * hd, k + (int64_t)h * hd, A->k_norm, hd, A->eps);
        or_rope_head(k + (int64_t)h * hd, A->rd, pos, A->theta);
    }
    memcpy(k_cache + (int64_t)pos * kvrows, k, (size_t)kvrows * sizeof(float));
    memcpy(v_cache + (int64_t)pos * kvrows, v, (size_t)kvrows * sizeof(float));
    const int rep = nh / nkv;
    const float scale = 1.f / sqrtf((float)hd);
    for (int h = 0; h < nh; h++) {
        const int hk = h / rep;
        float *sh = scores + (int64_t)h * (pos + 1);
        float mx = -INFINITY;
        for (int t = 0; t <= pos; t++) {
            float z0 = 0.f;
            const int64_t off = (int64_t)t * kvrows + (int64_t)hk * hd;
            for (int j = 0; j < hd; j++) z0 = fmaf(q[(int64_t)h * hd + j], k_cache[off + j], z0);
            sh[t] = z0 * scale;
            if (sh[t] > mx) mx = sh[t];
        }
        float den = 0.f;
        for (int t = 0; t <= pos; t++) {
            sh[t] = sh[t] == -INFINITY ? 0.f : expf(sh[t] - mx);
            den += sh[t];
        }
        for (int j = 0; j < hd; j++) {
            float sum = 0.f;
            for (int t = 0; t <= pos; t++) {
                const int64_t off = (int64_t)t * kvrows + (int64_t)hk * hd + j;
                sum = fmaf(sh[t] / den, v_cache[off], sum);
            }
            ctx[(int64_t)h * hd + j] = sum * or_sigmoidf(gate[(int64_t)h * hd + j]);
        }
    }
    or_qmat_mul(out, ctx, &A->o, 0);
    free(qp);
    free(q);
    free(gate);
    free(k);
    free(v);
    free(ctx);
    free(scores);
}
