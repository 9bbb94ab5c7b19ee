/* CPU restatement of the reference's quantized MoE layer (qwen.c CPU path).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against, and the "port" CPU baseline timed by bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product (shiftwing_amd/) never links, loads or calls it.
 *
 * Citations are /root/reference paths.  Each function restates one reference
 * function; the header comment of moe_oracle.c lists how each one is pinned
 * (reference golden vectors, the compiled reference, closed forms). */
#ifndef SW_MOE_ORACLE_H
#define SW_MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QMat, c/qwen.c:68-81 (host fields only).
 * fmt 0 = f32 (f), 1 = int8 (q, one scale per row), 2 = int2 (four codes a
 * byte, value 2 code - 3), 3 = packed int3 triplets, 4 = int4
 * low-nibble-first; fmt 2/3/4 carry one f32 scale per (row, group). */
typedef struct {
    int fmt, O, I, gs, rb, ng;
    const float *f;
    const float *s;
    const void *q;
} or_qmat;

/* MoeW + Expert + the Cfg fields the MoE step reads, c/qwen.c:82-94, 53. */
typedef struct {
    int H, E, K, I, I_sh;
    or_qmat router;        /* fmt 0, E x H */
    or_qmat shared_gate;   /* fmt 1, I_sh x H */
    or_qmat shared_up;     /* fmt 1, I_sh x H */
    or_qmat shared_down;   /* fmt 1, H x I_sh */
    or_qmat shared_scale;  /* fmt 0, 1 x H: the shared-expert sigmoid gate row */
    const or_qmat *gate;   /* E entries */
    const or_qmat *up;     /* E entries */
    const or_qmat *down;   /* E entries */
} or_layer;

/* Optional intermediate outputs of one layer call (any pointer may be NULL).
 * logits [T*E], idx [T*K], weight [T*K], shared [T*H] (shared expert output
 * before the sigmoid gate), sgate [T] (sigmoid of the gate logit). */
typedef struct {
    float *logits;
    int *idx;
    float *weight;
    float *shared;
    float *sgate;
} or_trace;

/* Arithmetic building blocks. */
float or_dot_f32(const float *a, const float *b, int n);
float or_dot_q8f(const int8_t *w, const float *x, int n);
float or_qrow_i8(const float *x, int8_t *q, int n);
int32_t or_dot_i8i8(const int8_t *w, const int8_t *x, int n);
float or_dot_q4_group(const uint8_t *w, const float *x, int n);
int or_q3_value(const uint8_t *w, int i);
float or_dot_q3_group(const uint8_t *w, const float *x, int n);
float or_dot_q2_group(const uint8_t *w, const float *x, int n);
float or_qmat_dot_row(const or_qmat *w, int row, const float *x);
void or_qmat_mul(float *y, const float *x, const or_qmat *w, int allow_idot);
void or_qmat_mul_batch(float *y, const float *x, int B, int ldx,
                       const or_qmat *w, int allow_idot);
float or_expf(float x);
void or_rmsnorm_zero(float *out, const float *x, const float *w, int n, float eps);
float or_sigmoidf(float x);
float or_siluf(float x);
void or_sigmoid_batch(const float *x, float *y, int64_t n);
void or_expf_batch(const float *x, float *y, int64_t n);
void or_router_topk(const float *logit, int E, int K, int *idx, float *weight);
void or_mlp_one(float *out, const float *x, const or_qmat *gate,
                const or_qmat *up, const or_qmat *down, int I);
void or_mlp_batch(float *out, const float *x, int B, int ldx,
                  const or_qmat *gate, const or_qmat *up, const or_qmat *down,
                  int I);

/* Layer steps. */
void or_moe_forward(const or_layer *L, const float *x, float *out,
                    or_trace *tr);
void or_moe_prefill_grouped(const or_layer *L, const float *x, int T,
                            float *out, or_trace *tr);

/* The two mixer layers either side of the MoE block in the reference's
 * hybrid decoder: the Gated DeltaNet layer (GdnW, c/qwen.c:95-104, with the
 * Cfg fields lin_* and conv_kernel) and the gated GQA attention layer (AttnW,
 * c/qwen.c:105-114, Cfg n_heads, n_kv_heads, head_dim, partial_rotary,
 * theta).  Channels of qkv: [q: kh*dk | k: kh*dk | v: vh*dv]. */
typedef struct {
    int H, kh, vh, dk, dv, K;
    float eps;
    or_qmat qkv, z, a, b, out;   /* qkv, z, out int4; a, b any format (vh x H) */
    const float *conv;           /* channels x K */
    const float *A_log, *dt_bias; /* vh */
    const float *norm;           /* dv */
} or_gdn;

typedef struct {
    int H, nh, nkv, hd, rd;
    float theta, eps;
    or_qmat q, k, v, o;          /* q: 2*nh*hd rows (query | gate per head) */
    const float *q_norm, *k_norm; /* hd */
} or_attn;

/* a = W_a x, b = W_b x as gdn_forward forms them (c/qwen.c:3008). */
void or_gdn_gates(const or_gdn *G, const float *x, float *a, float *b);
/* One decode step at position pos; conv_state [K][channels] and state
 * [vh][dk][dv] are updated in place (c/qwen.c:3004-3025, 2907-2927). */
void or_gdn_forward(const or_gdn *G, const float *x, const float *a,
                    const float *b, int pos, float *conv_state, float *state,
                    float *out);
/* One decode step at position pos over fp32 caches [positions][nkv*hd]
 * (attn_forward without the Qwen4-Exp indexer, c/qwen.c:3116-3153). */
void or_attn_forward(const or_attn *A, const float *x, int pos,
                     float *k_cache, float *v_cache, float *out);

/* token->expert bucketing in the order of moe_prefill_grouped as a CSR:
 * offsets[E+1]; entry n of expert e holds token[n] (ascending) and slot[n]
 * (the route index k with idx[token*K+k]==e).  Returns the route count. */
int or_bucket(const int *idx, int T, int K, int E, int *offsets, int *token,
              int *slot);

/* Host materialisation of the synthetic layer (same bytes as the device). */
void or_synth_router(uint64_t seed, int layer, int E, int H, float *router,
                     float *shared_gate);
void or_synth_shared_q8(uint64_t seed, int layer, int H, int I_sh,
                        int8_t *gq, float *gs, int8_t *uq, float *us,
                        int8_t *dq, float *ds);
void or_synth_expert(uint64_t seed, int layer, int eid, int fmt, int H, int I,
                     int gs, uint8_t *gq, float *gsc, uint8_t *uq, float *usc,
                     uint8_t *dq, float *dsc);
void or_synth_x(uint64_t seed, int layer, int step, int H, float *x);
void or_synth_bytes(uint64_t seed, int layer, int eid, int tensor, uint8_t *out,
                    uint64_t n);

/* OpenMP thread count used by the layer steps (0 = runtime default). */
void or_set_threads(int n);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
