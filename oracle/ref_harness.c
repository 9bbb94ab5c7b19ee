/* In-memory harness over the reference's own CPU MoE code.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile from the reference
 * sources where they lie (-I <reference>/c, the same QWEN_NO_MAIN inclusion
 * the reference's own white-box tests use, c/tests/test_router.c:1-2) into
 * oracle/_ref/.  Nothing is copied from the reference; this file only wires
 * caller-owned buffers into the reference's QMat / MoeW / Model structs
 * (c/qwen.c:68-94, 225-243) and calls its static functions:
 *   dot 1674, qrow_i8 1696, dot_i8i8 1697, dot_q4_group 1706,
 *   dot_q3_group 1730, qmat_mul_ex 1761, qmat_mul_batch 3305,
 *   router_topk 3421, mlp_one 3415, moe_forward 3717,
 *   moe_prefill_grouped 4141.
 * Every expert is resident (cap = E), so the expert cache never loads. */
#define QWEN_NO_MAIN
#include "qwen.c"

#include "moe_oracle.h"

static QMat ref_qmat(const or_qmat *w) {
    QMat q;
    memset(&q, 0, sizeof(q));
    q.fmt = w->fmt;
    q.O = w->O;
    q.I = w->I;
    q.gs = w->gs;
    q.rb = w->rb;
    q.ng = w->ng;
    q.drb = w->fmt == 3 ? (w->rb / 3) * 4 : w->rb;
    q.f = (float *)w->f;
    q.s = (float *)w->s;
    if (w->fmt == 1)
        q.q8 = (int8_t *)w->q;
    else
        q.q4 = (uint8_t *)w->q;
    return q;
}

float ref_dot(const float *a, const float *b, int n) { return dot(a, b, n); }
float ref_dot_q8f(const int8_t *w, const float *x, int n) { return dot_q8f(w, x, n); }
float ref_qrow_i8(const float *x, int8_t *q, int n) { return qrow_i8(x, q, n); }
int32_t ref_dot_i8i8(const int8_t *w, const int8_t *x, int n) { return dot_i8i8(w, x, n); }
float ref_dot_q4_group(const uint8_t *w, const float *x, int n) { return dot_q4_group(w, x, n); }
float ref_dot_q3_group(const uint8_t *w, const float *x, int n) { return dot_q3_group(w, x, n); }
float ref_expf(float x) { return expf(x); }
float ref_siluf(float x) { return siluf(x); }

void ref_qmat_mul(float *y, const float *x, const or_qmat *w, int allow_idot) {
    QMat q = ref_qmat(w);
    qmat_mul_ex(y, x, &q, allow_idot);
}

void ref_qmat_mul_batch(float *y, const float *x, int B, int ldx, const or_qmat *w,
                        int allow_idot) {
    QMat q = ref_qmat(w);
    qmat_mul_batch(y, x, B, ldx, &q, allow_idot);
}

void ref_router_topk(const float *logit, int E, int K, int *idx, float *weight) {
    router_topk(logit, E, K, idx, weight);
}

void ref_mlp_one(float *out, const float *x, const or_qmat *g, const or_qmat *u,
                 const or_qmat *d, int I) {
    QMat qg = ref_qmat(g), qu = ref_qmat(u), qd = ref_qmat(d);
    mlp_one(out, x, &qg, &qu, &qd, I);
}

typedef struct {
    Model m;
    Layer l;
} RefLayer;

void *ref_layer_create(const or_layer *L) {
    RefLayer *r = (RefLayer *)calloc(1, sizeof(RefLayer));
    if (!r) return NULL;
    Cfg *c = &r->m.c;
    c->n_layers = 1;
    c->hidden = L->H;
    c->n_experts = L->E;
    c->topk = L->K;
    c->moe_inter = L->I;
    c->shared_inter = L->I_sh;
    c->norm_topk = 1;
    r->m.layer = &r->l;
    r->m.expert_cap = L->E;
    MoeW *w = &r->l.moe;
    w->router = ref_qmat(&L->router);
    w->shared_gate = ref_qmat(&L->shared_gate);
    w->shared_up = ref_qmat(&L->shared_up);
    w->shared_down = ref_qmat(&L->shared_down);
    w->shared_scale = ref_qmat(&L->shared_scale);
    w->cap = L->E;
    w->layer = 0;
    w->expert = (Expert *)calloc((size_t)L->E, sizeof(Expert));
    w->heat = (uint32_t *)calloc((size_t)L->E, sizeof(uint32_t));
    w->last = (uint32_t *)calloc((size_t)L->E, sizeof(uint32_t));
    w->prefetched = (unsigned char *)calloc((size_t)L->E, 1);
    pthread_mutex_init(&w->lock, NULL);
    pthread_cond_init(&w->pf_done, NULL);
    for (int e = 0; e < L->E; e++) {
        w->expert[e].eid = e;
        w->expert[e].gate = ref_qmat(&L->gate[e]);
        w->expert[e].up = ref_qmat(&L->up[e]);
        w->expert[e].down = ref_qmat(&L->down[e]);
    }
    return r;
}

void ref_layer_destroy(void *h) {
    RefLayer *r = (RefLayer *)h;
    if (!r) return;
    free(r->l.moe.expert);
    free(r->l.moe.heat);
    free(r->l.moe.last);
    free(r->l.moe.prefetched);
    free(r->m.turn_hits);
    free(r);
}

void ref_moe_forward(void *h, const float *x, float *out) {
    RefLayer *r = (RefLayer *)h;
    moe_forward(&r->m, &r->l, x, out);
}

void ref_moe_prefill_grouped(void *h, const float *x, int T, float *out) {
    RefLayer *r = (RefLayer *)h;
    moe_prefill_grouped(&r->m, &r->l, x, T, out, 0);
}

int ref_omp_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ref_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
