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
 *   router_topk 3421, mlp_one 3415, moe_forward 3717, rmsnorm_zero 1780,
 *   moe_prefill_grouped 4141.
 * Every expert is resident (cap = E), so the expert cache never loads. */
#define QWEN_NO_MAIN
#include "qwen.c"
#ifdef COLI_CUDA
/* the device-resident MoE step as the reference engine would include it */
#include "sw_qwen_bridge.inc"
#endif

#include "moe_oracle.h"

static QMat ref_qmat_named(const or_qmat *w, const char *name) {
    QMat q;
    memset(&q, 0, sizeof(q));
#ifdef COLI_CUDA
    /* the reference's device weight cache keys tensors by name (c/qwen.c:576) */
    if (name) {
        snprintf(q.cuda_key, sizeof(q.cuda_key), "%s", name);
        q.cuda_eligible = w->fmt == 1 || w->fmt == 2 || w->fmt == 3 || w->fmt == 4;
    }
#else
    (void)name;
#endif
    q.fmt = w->fmt;
    q.O = w->O;
    q.I = w->I;
    q.gs = w->gs;
    q.rb = w->rb;
    q.ng = w->ng;
    q.drb = w->fmt == 3 ? (w->rb / 3) * 4 : w->fmt == 2 ? w->rb * 2 : w->rb;
    q.f = (float *)w->f;
    q.s = (float *)w->s;
    if (w->fmt == 1)
        q.q8 = (int8_t *)w->q;
    else
        q.q4 = (uint8_t *)w->q;
    return q;
}

static QMat ref_qmat(const or_qmat *w) { return ref_qmat_named(w, NULL); }

float ref_dot(const float *a, const float *b, int n) { return dot(a, b, n); }
float ref_dot_q8f(const int8_t *w, const float *x, int n) { return dot_q8f(w, x, n); }
float ref_qrow_i8(const float *x, int8_t *q, int n) { return qrow_i8(x, q, n); }
int32_t ref_dot_i8i8(const int8_t *w, const int8_t *x, int n) { return dot_i8i8(w, x, n); }
float ref_dot_q4_group(const uint8_t *w, const float *x, int n) { return dot_q4_group(w, x, n); }
float ref_dot_q3_group(const uint8_t *w, const float *x, int n) { return dot_q3_group(w, x, n); }
float ref_dot_q2_group(const uint8_t *w, const float *x, int n) { return dot_q2_group(w, x, n); }
float ref_expf(float x) { return expf(x); }
void ref_rmsnorm_zero(float *out, const float *x, const float *w, int n, float eps) {
    rmsnorm_zero(out, x, w, n, eps);
}
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
    /* Tensor names as the reference container spells them (c/qwen.c:2198-2206).
     * The reference's device weight cache is keyed by these names
     * (c/qwen.c:576-578), so every harness layer gets a layer number of its
     * own: layers of different shapes must never share a cached buffer. */
    static int serial;
    const int ln = __atomic_fetch_add(&serial, 1, __ATOMIC_RELAXED);
    char nm[160];
    snprintf(nm, sizeof(nm), "layers.%d.mlp.gate.weight", ln);
    w->router = ref_qmat_named(&L->router, nm);
    snprintf(nm, sizeof(nm), "layers.%d.mlp.shared_expert.gate_proj.weight", ln);
    w->shared_gate = ref_qmat_named(&L->shared_gate, nm);
    snprintf(nm, sizeof(nm), "layers.%d.mlp.shared_expert.up_proj.weight", ln);
    w->shared_up = ref_qmat_named(&L->shared_up, nm);
    snprintf(nm, sizeof(nm), "layers.%d.mlp.shared_expert.down_proj.weight", ln);
    w->shared_down = ref_qmat_named(&L->shared_down, nm);
    snprintf(nm, sizeof(nm), "layers.%d.mlp.shared_expert_gate.weight", ln);
    w->shared_scale = ref_qmat_named(&L->shared_scale, nm);
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
        snprintf(nm, sizeof(nm), "layers.%d.mlp.experts.%d.gate_proj.weight", ln, e);
        w->expert[e].gate = ref_qmat_named(&L->gate[e], nm);
        snprintf(nm, sizeof(nm), "layers.%d.mlp.experts.%d.up_proj.weight", ln, e);
        w->expert[e].up = ref_qmat_named(&L->up[e], nm);
        snprintf(nm, sizeof(nm), "layers.%d.mlp.experts.%d.down_proj.weight", ln, e);
        w->expert[e].down = ref_qmat_named(&L->down[e], nm);
    }
    return r;
}

void ref_layer_destroy(void *h) {
    RefLayer *r = (RefLayer *)h;
    if (!r) return;
#ifdef COLI_CUDA
    sw_moe_unregister(&r->l);
    /* device cache entries must not point back at the freed matrices */
    MoeW *w = &r->l.moe;
    cuda_qmat_detach(&w->shared_gate);
    cuda_qmat_detach(&w->shared_up);
    cuda_qmat_detach(&w->shared_down);
    cuda_qmat_detach(&w->shared_scale);
    for (int e = 0; e < r->m.c.n_experts; e++) {
        cuda_qmat_detach(&w->expert[e].gate);
        cuda_qmat_detach(&w->expert[e].up);
        cuda_qmat_detach(&w->expert[e].down);
    }
#endif
    free(r->l.moe.expert);
    free(r->l.moe.heat);
    free(r->l.moe.last);
    free(r->l.moe.prefetched);
    free(r->m.turn_hits);
    free(r);
}

/* The mixer layers of the hybrid decoder: a Gated DeltaNet layer (GdnW,
 * c/qwen.c:95-104) and a gated GQA attention layer (AttnW, 105-114) in a
 * one-layer Model, driven through gdn_forward 3005, gdn_decode_block 4642,
 * attn_forward 3094 and attn_prefill_layer 3138.  The caller owns every
 * buffer, including the CPU-side conv/recurrent state and KV caches; in the
 * -DCOLI_CUDA build those functions take the reference's device paths
 * (cuda_gdn_try 881, cuda_gdn_block_try 888, cuda_attn_try 935,
 * cuda_attn_prefill_try 957) whenever its switches allow. */
void *ref_gdn_create(const or_gdn *G, float *conv_state, float *state) {
    RefLayer *r = (RefLayer *)calloc(1, sizeof(RefLayer));
    if (!r) return NULL;
    Cfg *c = &r->m.c;
    c->n_layers = 1;
    c->hidden = G->H;
    c->lin_k_heads = G->kh;
    c->lin_v_heads = G->vh;
    c->lin_k_dim = G->dk;
    c->lin_v_dim = G->dv;
    c->conv_kernel = G->K;
    c->eps = G->eps;
    r->m.layer = &r->l;
    r->l.type = LT_LINEAR;
    static int serial;
    const int ln = __atomic_fetch_add(&serial, 1, __ATOMIC_RELAXED);
    char nm[160];
    GdnW *w = &r->l.gdn;
    snprintf(nm, sizeof(nm), "mixer.%d.linear_attn.in_proj_qkv.weight", ln);
    w->qkv = ref_qmat_named(&G->qkv, nm);
    snprintf(nm, sizeof(nm), "mixer.%d.linear_attn.in_proj_z.weight", ln);
    w->z = ref_qmat_named(&G->z, nm);
    snprintf(nm, sizeof(nm), "mixer.%d.linear_attn.out_proj.weight", ln);
    w->out = ref_qmat_named(&G->out, nm);
    w->a = ref_qmat(&G->a);
    w->b = ref_qmat(&G->b);
    w->conv = (float *)G->conv;
    w->A_log = (float *)G->A_log;
    w->dt_bias = (float *)G->dt_bias;
    w->norm = (float *)G->norm;
    w->conv_state = conv_state;
    w->state = state;
    return r;
}

/* one decode token at position pos (gdn_forward); a and b receive the gate
 * projections gdn_forward forms from x */
void ref_gdn_forward(void *h, const float *x, int pos, float *out, float *a, float *b) {
    RefLayer *r = (RefLayer *)h;
    if (a) qmat_mul_ex(a, x, &r->l.gdn.a, 0);
    if (b) qmat_mul_ex(b, x, &r->l.gdn.b, 0);
    r->m.pos = pos;
    gdn_forward(&r->m, &r->l, x, out);
}

/* T consecutive tokens from position base (gdn_decode_block) */
void ref_gdn_block(void *h, const float *x, int T, int base, float *out) {
    RefLayer *r = (RefLayer *)h;
    gdn_decode_block(&r->m, &r->l, x, T, base, out);
}

void *ref_attn_create(const or_attn *A, float *k_cache, float *v_cache, int max_seq) {
    RefLayer *r = (RefLayer *)calloc(1, sizeof(RefLayer));
    if (!r) return NULL;
    Cfg *c = &r->m.c;
    c->n_layers = 1;
    c->hidden = A->H;
    c->n_heads = A->nh;
    c->n_kv_heads = A->nkv;
    c->head_dim = A->hd;
    c->partial_rotary = (float)A->rd / (float)A->hd;
    c->theta = A->theta;
    c->eps = A->eps;
    r->m.layer = &r->l;
    r->m.max_seq = max_seq;
    r->l.type = LT_FULL;
    static int serial;
    const int ln = __atomic_fetch_add(&serial, 1, __ATOMIC_RELAXED);
    char nm[160];
    AttnW *w = &r->l.attn;
    snprintf(nm, sizeof(nm), "mixer.%d.self_attn.q_proj.weight", ln);
    w->q = ref_qmat_named(&A->q, nm);
    snprintf(nm, sizeof(nm), "mixer.%d.self_attn.k_proj.weight", ln);
    w->k = ref_qmat_named(&A->k, nm);
    snprintf(nm, sizeof(nm), "mixer.%d.self_attn.v_proj.weight", ln);
    w->v = ref_qmat_named(&A->v, nm);
    snprintf(nm, sizeof(nm), "mixer.%d.self_attn.o_proj.weight", ln);
    w->o = ref_qmat_named(&A->o, nm);
    w->q_norm = (float *)A->q_norm;
    w->k_norm = (float *)A->k_norm;
    w->k_cache = k_cache;
    w->v_cache = v_cache;
    return r;
}

void ref_attn_forward(void *h, const float *x, int pos, float *out) {
    RefLayer *r = (RefLayer *)h;
    r->m.pos = pos;
    attn_forward(&r->m, &r->l, x, out);
}

/* T consecutive rows from position base (attn_prefill_layer) */
void ref_attn_prefill(void *h, const float *x, int T, int base, float *out) {
    RefLayer *r = (RefLayer *)h;
    attn_prefill_layer(&r->m, &r->l, x, T, base, out);
}

void ref_mixer_destroy(void *h) {
    RefLayer *r = (RefLayer *)h;
    if (!r) return;
#ifdef COLI_CUDA
    if (r->l.type == LT_LINEAR) {
        GdnW *w = &r->l.gdn;
        cuda_qmat_detach(&w->qkv);
        cuda_qmat_detach(&w->z);
        cuda_qmat_detach(&w->out);
        float *d[] = {w->d_conv, w->d_A_log, w->d_dt_bias, w->d_norm, w->d_conv_state, w->d_state};
        for (size_t i = 0; i < sizeof(d) / sizeof(d[0]); i++)
            if (d[i]) coli_cuda_free(cuda_rt.ctx, d[i]);
    } else {
        AttnW *w = &r->l.attn;
        cuda_qmat_detach(&w->q);
        cuda_qmat_detach(&w->k);
        cuda_qmat_detach(&w->v);
        cuda_qmat_detach(&w->o);
        float *d[] = {w->d_q_norm, w->d_k_norm, w->d_k_cache, w->d_v_cache};
        for (size_t i = 0; i < sizeof(d) / sizeof(d[0]); i++)
            if (d[i]) coli_cuda_free(cuda_rt.ctx, d[i]);
    }
#endif
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

/* moe_prefill_route_gather (c/qwen.c:3956-3968) for every expert in
 * ascending id, the order moe_prefill_grouped serves them in: per expert its
 * tokens and weights in gather order.  The gathered rows come from x[t] = t
 * (H = 1), so xb also shows which token each row copied.  Returns the total. */
int ref_route_gather_all(const int *idx, const float *weight, int T, int K, int E, int *offsets, int *token,
                         float *wt, float *xb) {
    float *x = (float *)malloc((size_t)(T > 0 ? T : 1) * sizeof(float));
    if (!x) return -1;
    for (int t = 0; t < T; t++) x[t] = (float)t;
    int n = 0;
    for (int e = 0; e < E; e++) {
        offsets[e] = n;
        n += moe_prefill_route_gather(e, idx, weight, x, T, K, 1, token + n, wt + n, xb + n);
    }
    offsets[E] = n;
    free(x);
    return n;
}

/* The reference's own reading of one matrix from a snapshot directory:
 * st_init (c/st.h:211-297) indexes the shard files, load_qmat_mode
 * (c/qwen.c:2224-2257) finds the tensor (find_qmat_named 2198-2214: the
 * EXPERT_Q3 / EXPERT_Q2 sidecars of routed experts, set here from use_q3 /
 * use_q2) and detects its format.  info = {fmt, gs, rb, ng, drb}.  payload
 * receives rows*rb code bytes (fmt 1-4) or rows*cols floats (fmt 0), scales
 * rows*ng floats, when the capacities (bytes, floats) allow; returns -1 when
 * they do not.  The reference exits the process on a malformed file: this is
 * for well-formed snapshots only. */
int ref_load_qmat(const char *dir, const char *base, int rows, int cols, int use_q3, int use_q2, int info[5],
                  void *payload, size_t payload_cap, float *scales, size_t scales_cap) {
    Model *m = (Model *)calloc(1, sizeof(Model));
    if (!m) return -1;
    if (use_q3) setenv("EXPERT_Q3", "1", 1); else unsetenv("EXPERT_Q3");
    if (use_q2) setenv("EXPERT_Q2", "1", 1); else unsetenv("EXPERT_Q2");
    st_init(&m->S, dir);
    QMat q = load_qmat_mode(m, base, rows, cols, 0);
    info[0] = q.fmt;
    info[1] = q.gs;
    info[2] = q.rb;
    info[3] = q.ng;
    info[4] = q.drb;
    int rc = 0;
    if (q.fmt == 0) {
        if ((size_t)rows * cols * 4 > payload_cap) rc = -1;
        else memcpy(payload, q.f, (size_t)rows * cols * 4);
    } else {
        const size_t nb = (size_t)rows * q.rb, ns = (size_t)rows * (q.fmt == 1 ? 1 : q.ng);
        if (nb > payload_cap || ns > scales_cap) rc = -1;
        else {
            memcpy(payload, q.fmt == 1 ? (const void *)q.q8 : (const void *)q.q4, nb);
            memcpy(scales, q.s, ns * 4);
        }
    }
    free(q.f);
    free(q.q8);
    free(q.q4);
    free(q.s);
    for (int i = 0; i < m->S.nfd; i++) close(m->S.fds[i]);
    for (int i = 0; i < m->S.n; i++) free(m->S.t[i].name);
    free(m->S.t);
    free(m->S.hidx);
    free(m);
    unsetenv("EXPERT_Q3");
    unsetenv("EXPERT_Q2");
    return rc;
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

#ifdef COLI_CUDA
/* The device-resident MoE step of the bridge included above, on a harness
 * layer. */
int ref_sw_register(void *h) {
    RefLayer *r = (RefLayer *)h;
    return sw_moe_register(&r->m, &r->l);
}

int ref_sw_forward(void *h, const float *x, int T, float *out, int *idx) {
    RefLayer *r = (RefLayer *)h;
    return sw_moe_try(&r->m, &r->l, x, T, out, idx);
}

/* sw_moe_try_device on activations the engine holds in device memory (the
 * resident decode loop, c/qwen.c:4404-4522, in place of
 * cuda_resident_moe_try 3825-3954): x goes to a device buffer of the
 * reference's context, the step runs device to device, out comes back.
 * Returns 1 when the device step ran, 0 when the caller would run its CPU
 * path, -1 on a harness allocation or copy failure. */
int ref_sw_forward_device(void *h, const float *x, int T, float *out) {
    RefLayer *r = (RefLayer *)h;
    const size_t bytes = (size_t)T * r->m.c.hidden * sizeof(float);
    void *dx = NULL, *dy = NULL;
    int used = -1;
    pthread_mutex_lock(&cuda_rt.lock);
    int ok = !coli_cuda_malloc(cuda_rt.ctx, &dx, bytes) && !coli_cuda_malloc(cuda_rt.ctx, &dy, bytes) &&
             !coli_cuda_upload(cuda_rt.ctx, dx, x, bytes) && !coli_cuda_sync(cuda_rt.ctx);
    pthread_mutex_unlock(&cuda_rt.lock);
    if (ok) {
        used = sw_moe_try_device(&r->m, &r->l, (float *)dy, (const float *)dx, T);
        pthread_mutex_lock(&cuda_rt.lock);
        if (used == 1 && (coli_cuda_download(cuda_rt.ctx, out, dy, bytes) || coli_cuda_sync(cuda_rt.ctx))) used = -1;
        pthread_mutex_unlock(&cuda_rt.lock);
    }
    pthread_mutex_lock(&cuda_rt.lock);
    if (dx) coli_cuda_free(cuda_rt.ctx, dx);
    if (dy) coli_cuda_free(cuda_rt.ctx, dy);
    pthread_mutex_unlock(&cuda_rt.lock);
    return used;
}

/* moe_forward (c/qwen.c:3717) and moe_prefill_grouped (4141) with the hook
 * the integration patch puts first in each: the bridge's device step, and the
 * reference's own body when the bridge declines (layer not registered, or the
 * bridge switched off after a device error).  Returns whether the device step
 * produced out. */
int ref_hooked_moe_forward(void *h, const float *x, float *out) {
    RefLayer *r = (RefLayer *)h;
    if (sw_moe_try(&r->m, &r->l, x, 1, out, NULL)) return 1;
    moe_forward(&r->m, &r->l, x, out);
    return 0;
}

int ref_hooked_moe_prefill(void *h, const float *x, int T, float *out) {
    RefLayer *r = (RefLayer *)h;
    if (sw_moe_try(&r->m, &r->l, x, T, out, NULL)) return 1;
    moe_prefill_grouped(&r->m, &r->l, x, T, out, 0);
    return 0;
}

/* whether the bridge has switched itself off after a device error */
int ref_sw_disabled(void) { return sw_moe.disabled; }

/* The reference's own GPU glue (c/qwen.c:462-1474, 3741-3809) driving
 * whatever library provides the coli_cuda_* symbols it was linked against.
 * The caller sets the reference's switches (COLI_CUDA=1, CUDA_DENSE=1,
 * optionally CUDA_F16=1) before ref_cuda_start. */
int ref_cuda_start(void) { return cuda_backend_start() && cuda_rt.active; }

void ref_cuda_set_f16(int on) { cuda_rt.use_f16 = on != 0; }

/* out: active, failed, grouped expert calls, grouped kernel calls, batched
 * transactions, fused MLP calls, q3 native grouped calls */
void ref_cuda_counters(unsigned long long out[7]) {
    out[0] = (unsigned long long)cuda_rt.active;
    out[1] = (unsigned long long)cuda_rt.failed;
    out[2] = cuda_rt.grouped_calls;
    out[3] = cuda_rt.grouped_kernel_calls;
    out[4] = cuda_rt.batch_transactions;
    out[5] = cuda_rt.mlp_calls;
    out[6] = cuda_rt.q3_grouped_calls;
}

/* out: GDN device calls, attention device calls, attention prefill calls
 * (cuda_rt counters bumped by cuda_gdn_try 889, cuda_gdn_block_try 890,
 * cuda_attn_try 940 and cuda_attn_prefill_try 968) */
void ref_cuda_mixer_counters(unsigned long long out[3]) {
    out[0] = (unsigned long long)cuda_rt.gdn_calls;
    out[1] = (unsigned long long)cuda_rt.attn_calls;
    out[2] = (unsigned long long)cuda_rt.attn_prefill_calls;
}

/* A speculative block of T = 2..8 tokens (moe_cuda_block, c/qwen.c:3741):
 * returns 1 when the device path produced out. */
int ref_moe_cuda_block(void *h, const float *x, int T, float *out) {
    RefLayer *r = (RefLayer *)h;
    memset(out, 0, (size_t)T * r->m.c.hidden * sizeof(float));
    return moe_cuda_block(&r->m, &r->l, x, T, out);
}

void ref_cuda_stop(void) { cuda_backend_stop(); }
#endif
