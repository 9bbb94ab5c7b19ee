/* shiftwing MoE path for MI355X (gfx950): the C ABI.
 *
 * Part 1 keeps the reference backend's MoE-path entry points with identical
 * prototypes, so c/qwen.c links against this library instead of
 * backend_cuda.o unchanged (reference: /root/reference/c/backend_cuda.h; line
 * numbers cited per entry point).  Conventions are the reference's
 * (c/backend_cuda.cu:47-70): every call returns 0 on success and -1 on
 * failure with a message in a thread-local buffer read by
 * coli_cuda_last_error(); tensors are device pointers owned by the caller;
 * every call is stream-ordered on the context's one stream and only
 * coli_cuda_sync() (and profile_snapshot) blocks the host; the caller
 * serialises calls on one context.
 *
 * Part 2 adds the device-resident MoE step that has no counterpart in the
 * reference backend: a registered HBM-resident layer (router, int8 shared
 * expert, all routed experts), device routing with the reference's exact
 * top-k, device token->expert bucketing, and the fused layer step with no
 * per-call host pointer tables and no batch/route limits.
 */
#ifndef SHIFTWING_MOE_H
#define SHIFTWING_MOE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ColiCuda ColiCuda; /* backend_cuda.h:10 */

/* ---- Part 1: reference backend entry points (c/backend_cuda.h) ---------- */

const char *coli_cuda_last_error(void);                 /* backend_cuda.h:13 */
int coli_cuda_create(ColiCuda **out, int device);         /* :14 */
void coli_cuda_destroy(ColiCuda *ctx);                    /* :15 */
const char *coli_cuda_device_name(const ColiCuda *ctx);   /* :16 */
int coli_cuda_compute_capability(const ColiCuda *ctx, int *major,
                                 int *minor);             /* :17 */
int coli_cuda_device_limits(const ColiCuda *ctx, int *sm_count,
                            int *shared_per_block);       /* :18-19 */
int coli_cuda_async_alloc_enabled(const ColiCuda *ctx);   /* :20 */
int coli_cuda_memory_info(ColiCuda *ctx, size_t *free_bytes,
                          size_t *total_bytes);           /* :21-22 */
int coli_cuda_malloc(ColiCuda *ctx, void **ptr, size_t bytes);        /* :24 */
void coli_cuda_free(ColiCuda *ctx, void *ptr);                        /* :25 */
int coli_cuda_malloc_host(ColiCuda *ctx, void **ptr, size_t bytes);   /* :26 */
void coli_cuda_free_host(ColiCuda *ctx, void *ptr);                   /* :27 */
int coli_cuda_host_register(ColiCuda *ctx, void *ptr, size_t bytes);  /* :28 */
void coli_cuda_host_unregister(ColiCuda *ctx, void *ptr);             /* :29 */
int coli_cuda_upload(ColiCuda *ctx, void *dst, const void *src,
                     size_t bytes);                                   /* :30 */
int coli_cuda_download(ColiCuda *ctx, void *dst, const void *src,
                       size_t bytes);                                 /* :31 */
int coli_cuda_copy(ColiCuda *ctx, void *dst, const void *src,
                   size_t bytes);                                     /* :32 */
int coli_cuda_memset(ColiCuda *ctx, void *dst, int value, size_t bytes); /* :33 */
int coli_cuda_sync(ColiCuda *ctx);                                    /* :34 */
void coli_cuda_profile_reset(ColiCuda *ctx);                          /* :35 */
int coli_cuda_profile_snapshot(ColiCuda *ctx, unsigned long long *transactions,
                               double stage_ms[8]);                   /* :38-40 */

int coli_cuda_rmsnorm_zero(ColiCuda *ctx, float *y, const float *x,
                           const float *w, int n, float eps);         /* :46-47 */
int coli_cuda_rmsnorm_zero_batch(ColiCuda *ctx, float *y, const float *x,
                                 const float *w, int batch, int n,
                                 float eps);                          /* :48-49 */
int coli_cuda_f32_gemm(ColiCuda *ctx, float *y, const float *x,
                       const float *w, int batch, int rows, int cols); /* :50-51 */
int coli_cuda_sigmoid(ColiCuda *ctx, float *y, const float *x, int n); /* :52 */
int coli_cuda_silu_mul(ColiCuda *ctx, float *y, const float *gate,
                       const float *up, int n);                       /* :53-54 */
int coli_cuda_axpy(ColiCuda *ctx, float *y, const float *x, float scale,
                   int n);                                            /* :55 */
int coli_cuda_sigmoid_axpy(ColiCuda *ctx, float *y, const float *x,
                           const float *logit, int n);                /* :56-57 */
int coli_cuda_f32_to_f16(ColiCuda *ctx, unsigned short *y, const float *x,
                         int n);                                      /* :58-59 */
int coli_cuda_q8_gemv(ColiCuda *ctx, float *y, const float *x,
                      const signed char *q, const float *scales, int rows,
                      int cols, int row_bytes);                       /* :60-62 */
int coli_cuda_q8_gemm(ColiCuda *ctx, float *y, const float *x, int batch,
                      const signed char *q, const float *scales, int rows,
                      int cols, int row_bytes);                       /* :63-65 */
int coli_cuda_q4_gemv(ColiCuda *ctx, float *y, const float *x,
                      const unsigned char *q, const float *scales, int rows,
                      int cols, int group_size, int row_bytes,
                      int groups_per_row);                            /* :66-69 */
int coli_cuda_q4_gemm(ColiCuda *ctx, float *y, const float *x, int batch,
                      const unsigned char *q, const float *scales, int rows,
                      int cols, int group_size, int row_bytes,
                      int groups_per_row);                            /* :70-73 */
int coli_cuda_q4_gemv_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                          const unsigned char *q, const float *scales,
                          int rows, int cols, int group_size, int row_bytes,
                          int groups_per_row);                        /* :74-77 */
int coli_cuda_q3_gemv(ColiCuda *ctx, float *y, const float *x,
                      const unsigned char *q, const float *scales, int rows,
                      int cols, int group_size, int row_bytes,
                      int groups_per_row);                            /* :78-81 */
int coli_cuda_q3_gemv_f16(ColiCuda *ctx, float *y, const unsigned short *x,
                          const unsigned char *q, const float *scales,
                          int rows, int cols, int group_size, int row_bytes,
                          int groups_per_row);                        /* :82-86 */
int coli_cuda_grouped_q4_mlp_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int experts, int hidden, int intermediate,
    int group_size, int hidden_row_bytes, int hidden_groups,
    int down_row_bytes, int down_groups);                            /* :87-94 */
int coli_cuda_grouped_q3_mlp_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int experts, int hidden, int intermediate,
    int group_size, int hidden_row_bytes, int hidden_groups,
    int down_row_bytes, int down_groups);                            /* :95-102 */
int coli_cuda_grouped_q4_mlp_batch_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int batch, int experts_per_token, int hidden,
    int intermediate, int group_size, int hidden_row_bytes,
    int hidden_groups, int down_row_bytes, int down_groups);         /* :103-110 */
int coli_cuda_grouped_q3_mlp_batch_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int batch, int experts_per_token, int hidden,
    int intermediate, int group_size, int hidden_row_bytes,
    int hidden_groups, int down_row_bytes, int down_groups);         /* :111-118 */
int coli_cuda_shared_q4_mlp_batch_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *gate_q, const float *gate_s,
    const unsigned char *up_q, const float *up_s,
    const unsigned char *down_q, const float *down_s,
    const unsigned char *scale_q, const float *scale_s,
    int batch, int hidden, int intermediate, int group_size,
    int hidden_row_bytes, int hidden_groups, int down_row_bytes,
    int down_groups, int scale_row_bytes, int scale_groups);         /* :119-127 */
int coli_cuda_shared_q8_mlp_batch(
    ColiCuda *ctx, float *y, const float *x, const float *scale,
    const signed char *gate_q, const float *gate_s, int gate_row_bytes,
    const signed char *up_q, const float *up_s, int up_row_bytes,
    const signed char *down_q, const float *down_s, int down_row_bytes,
    int batch, int hidden, int intermediate);                        /* :128-133 */
int coli_cuda_shared_q8_mlp_batch_device_scale(
    ColiCuda *ctx, float *y, const float *x, const float *device_scale,
    const signed char *gate_q, const float *gate_s, int gate_row_bytes,
    const signed char *up_q, const float *up_s, int up_row_bytes,
    const signed char *down_q, const float *down_s, int down_row_bytes,
    int batch, int hidden, int intermediate);                        /* :134-139 */
int coli_cuda_shared_q4_mlp_f16(
    ColiCuda *ctx, float *y, const unsigned short *x,
    const unsigned char *gate_q, const float *gate_s,
    const unsigned char *up_q, const float *up_s,
    const unsigned char *down_q, const float *down_s,
    const unsigned char *scale_q, const float *scale_s,
    int hidden, int intermediate, int group_size, int hidden_row_bytes,
    int hidden_groups, int down_row_bytes, int down_groups,
    int scale_row_bytes, int scale_groups);                          /* :140-148 */

/* ---- Part 1b: the mixer layers either side of the MoE block ------------- */
/* The hybrid decoder's Gated DeltaNet and gated GQA attention layers
 * (c/backend_cuda.h:149-236), called by the reference engine through
 * cuda_gdn_try, cuda_gdn_block_try, cuda_gdn_slots_try (c/qwen.c:881-911),
 * cuda_attn_try, cuda_attn_prefill_try, cuda_attn_slots_try (935-991) and
 * cuda_resident_core_try (994-1075).  Same arguments, ownership and 0/-1
 * convention as the reference: weights, norms, conv/recurrent state and KV
 * caches are device pointers; x, a, b and out are host pointers except in the
 * *_device forms (which do not synchronize); slot and position tables are
 * host arrays.  Arithmetic is fp32 on fp32 activations (the reference rounds
 * them to fp16 first) and matches the reference CPU path (gdn_forward
 * c/qwen.c:3005, attn_forward 3094) within 1e-3 x RMS.  Layouts taken: int4
 * projections with group sizes and widths that are multiples of 32 and row
 * strides that are multiples of 16 bytes (the converter's g128 rows), int8 or
 * int4 o projection, key_dim <= 128, value_dim <= 256, head_dim 64, 128 or
 * 256 with at most 16 query heads per kv head; other layouts return -1 with a
 * message. */
int coli_cuda_gdn_decode_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b,
    const unsigned char *qkv_q, const float *qkv_s, int qkv_row_bytes,
    int qkv_groups, const unsigned char *z_q, const float *z_s,
    int z_row_bytes, int z_groups, const unsigned char *out_q,
    const float *out_s, int out_row_bytes, int out_groups,
    const float *conv_weight, const float *a_log, const float *dt_bias,
    const float *norm_weight, float *conv_state, float *recurrent_state,
    int position, int hidden, int key_heads, int value_heads, int key_dim,
    int value_dim, int conv_kernel, int group_size, float eps); /* :149-158 */
int coli_cuda_gdn_block_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b,
    int batch, const unsigned char *qkv_q, const float *qkv_s,
    int qkv_row_bytes, int qkv_groups, const unsigned char *z_q,
    const float *z_s, int z_row_bytes, int z_groups,
    const unsigned char *out_q, const float *out_s, int out_row_bytes,
    int out_groups, const float *conv_weight, const float *a_log,
    const float *dt_bias, const float *norm_weight, float *conv_state,
    float *recurrent_state, int position, int hidden, int key_heads,
    int value_heads, int key_dim, int value_dim, int conv_kernel,
    int group_size, float eps);                                  /* :159-169 */
int coli_cuda_gdn_slots_q4_f16(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b,
    int batch, const int *slot, const int *position,
    const unsigned char *qkv_q, const float *qkv_s, int qkv_row_bytes,
    int qkv_groups, const unsigned char *z_q, const float *z_s,
    int z_row_bytes, int z_groups, const unsigned char *out_q,
    const float *out_s, int out_row_bytes, int out_groups,
    const float *conv_weight, const float *a_log, const float *dt_bias,
    const float *norm_weight, float *conv_state, float *recurrent_state,
    int slots, int hidden, int key_heads, int value_heads, int key_dim,
    int value_dim, int conv_kernel, int group_size, float eps);  /* :170-180 */
int coli_cuda_gdn_slots_q4_f16_device(
    ColiCuda *ctx, float *out, const float *x, const float *a, const float *b,
    int batch, const int *slot, const int *position,
    const unsigned char *qkv_q, const float *qkv_s, int qkv_row_bytes,
    int qkv_groups, const unsigned char *z_q, const float *z_s,
    int z_row_bytes, int z_groups, const unsigned char *out_q,
    const float *out_s, int out_row_bytes, int out_groups,
    const float *conv_weight, const float *a_log, const float *dt_bias,
    const float *norm_weight, float *conv_state, float *recurrent_state,
    int slots, int hidden, int key_heads, int value_heads, int key_dim,
    int value_dim, int conv_kernel, int group_size, float eps);  /* :183-193 */
int coli_cuda_gqa_decode_q4_f16(
    ColiCuda *ctx, float *out, const float *x,
    const unsigned char *q_q, const float *q_s, int q_rb, int q_ng,
    const unsigned char *k_q, const float *k_s, int k_rb, int k_ng,
    const unsigned char *v_q, const float *v_s, int v_rb, int v_ng,
    const void *o_q, const float *o_s, int o_fmt, int o_rb, int o_ng,
    const float *q_norm, const float *k_norm, float *k_cache,
    float *v_cache, int position, int hidden, int query_heads,
    int kv_heads, int head_dim, int rotary_dim, int group_size,
    float theta, float eps);                                     /* :194-203 */
int coli_cuda_gqa_prefill_q4_f16(
    ColiCuda *ctx, float *out, const float *x, int rows, int base,
    const unsigned char *q_q, const float *q_s, int q_rb, int q_ng,
    const unsigned char *k_q, const float *k_s, int k_rb, int k_ng,
    const unsigned char *v_q, const float *v_s, int v_rb, int v_ng,
    const void *o_q, const float *o_s, int o_fmt, int o_rb, int o_ng,
    const float *q_norm, const float *k_norm, float *k_cache,
    float *v_cache, int max_seq, int hidden, int query_heads,
    int kv_heads, int head_dim, int rotary_dim, int group_size,
    float theta, float eps);                                     /* :206-215 */
int coli_cuda_gqa_slots_q4_f16(
    ColiCuda *ctx, float *out, const float *x, int batch, const int *slot,
    const int *position, const unsigned char *q_q, const float *q_s,
    int q_rb, int q_ng, const unsigned char *k_q, const float *k_s,
    int k_rb, int k_ng, const unsigned char *v_q, const float *v_s,
    int v_rb, int v_ng, const void *o_q, const float *o_s, int o_fmt,
    int o_rb, int o_ng, const float *q_norm, const float *k_norm,
    float *k_cache, float *v_cache, int slots, int max_seq, int hidden,
    int query_heads, int kv_heads, int head_dim, int rotary_dim,
    int group_size, float theta, float eps);                     /* :216-225 */
int coli_cuda_gqa_slots_q4_f16_device(
    ColiCuda *ctx, float *out, const float *x, int batch, const int *slot,
    const int *position, const unsigned char *q_q, const float *q_s,
    int q_rb, int q_ng, const unsigned char *k_q, const float *k_s,
    int k_rb, int k_ng, const unsigned char *v_q, const float *v_s,
    int v_rb, int v_ng, const void *o_q, const float *o_s, int o_fmt,
    int o_rb, int o_ng, const float *q_norm, const float *k_norm,
    float *k_cache, float *v_cache, int slots, int max_seq, int hidden,
    int query_heads, int kv_heads, int head_dim, int rotary_dim,
    int group_size, float theta, float eps);                     /* :227-236 */

/* ---- Part 2: device-resident MoE step (no reference counterpart) -------- */

/* fp32-activation variants of the grouped calls above (same arguments with
 * x as float*).  The reference only has fp16-activation grouped kernels; its
 * CPU path is fp32, which these match within tolerance. */
int coli_cuda_grouped_q4_mlp(
    ColiCuda *ctx, float *y, const float *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int experts, int hidden, int intermediate,
    int group_size, int hidden_row_bytes, int hidden_groups,
    int down_row_bytes, int down_groups);
int coli_cuda_grouped_q3_mlp(
    ColiCuda *ctx, float *y, const float *x,
    const unsigned char *const *gate_q, const float *const *gate_s,
    const unsigned char *const *up_q, const float *const *up_s,
    const unsigned char *const *down_q, const float *const *down_s,
    const float *route_weight, int experts, int hidden, int intermediate,
    int group_size, int hidden_row_bytes, int hidden_groups,
    int down_row_bytes, int down_groups);

/* Bit-exact IDOT int8 GEMM (c/qwen.c:1696-1705, 1765-1768, 3313-3319):
 * per token xq = qrow_i8(x) (amax/127, 1/s, lrintf), then
 * y[b,o] = ((float)sum_i q[o,i]*xq[b,i] * scales[o]) * sx[b]. */
int coli_cuda_idot_q8_gemm(ColiCuda *ctx, float *y, const float *x, int batch,
                           const signed char *q, const float *scales,
                           int rows, int cols, int row_bytes);

/* coli_cuda_idot_q8_gemm without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc).  The
 * quantised activations live in a fixed 1 MiB device array per device instead
 * of context scratch, so round_up(batch * cols, 256) + 4 * batch must not
 * exceed 1 MiB (else -1 with a message).  Same results as
 * coli_cuda_idot_q8_gemm bit for bit.  Calls that overlap on one device
 * (several contexts or streams) race on that array. */
int coli_cuda_idot_q8_gemm_noalloc(ColiCuda *ctx, float *y, const float *x,
                                   int batch, const signed char *q,
                                   const float *scales, int rows, int cols,
                                   int row_bytes);

/* router_topk (c/qwen.c:3421-3426) on device logits, bit-exact:
 * logits [tokens x experts] -> idx / weight [tokens x topk]. */
int coli_cuda_router_topk(ColiCuda *ctx, const float *logits, int tokens,
                          int experts, int topk, int *idx, float *weight);

/* Token->expert bucketing in the reference's grouped-prefill order
 * (c/qwen.c:4168, 3956-3968): experts ascending, tokens ascending.
 * idx [tokens x topk] -> offsets [experts+1], token [tokens*topk],
 * slot [tokens*topk] (the route index k).  Entries past offsets[experts]
 * are left untouched.  One call takes experts <= 4096 and as many tokens as
 * one workgroup's 160 KiB map holds: experts * ceil(tokens/32) * 4 +
 * (2 * experts + 1) * 4 bytes (2048 tokens up to 512 experts, 1184 at 1024,
 * 224 at 4096); else -1 with a message. */
int coli_cuda_moe_bucket(ColiCuda *ctx, const int *idx, int tokens, int topk,
                         int experts, int *offsets, int *token, int *slot);

typedef struct ColiMoeLayer ColiMoeLayer;

typedef struct {
    int hidden;              /* H */
    int experts;             /* E */
    int topk;                /* K */
    int intermediate;        /* routed expert I */
    int shared_intermediate; /* shared expert I */
    int expert_format;       /* 4 = grouped int4, 3 = packed int3 triplets,
                                2 = int2 (four codes a byte, value 2c - 3) */
    int group_size;          /* routed-expert quant group (128) */
} ColiMoeShape;

/* Allocate an HBM-resident layer (all experts).  Requires hidden % 64 == 0,
 * group_size 128, expert_format 2, 3 or 4, topk <= 32 and experts <= 4096.
 * int2 experts are held as int4 records (code c as the nibble 5 + 2c, the
 * same value; c/qwen.c:567-575 widens them so for the reference's device
 * path), so they stream as many bytes as int4.
 * Any intermediate and shared_intermediate: a ragged one is held rounded up
 * to the row tiles (16 and 64 rows) with zero rows, which add exact zeros
 * (the reference's tail groups, c/qwen.c:1706-1754, as in
 * c/tests/test_quant_matmul.c:12-93); the set_* calls take the caller's
 * shape. */
int coli_cuda_moe_layer_create(ColiCuda *ctx, ColiMoeLayer **out,
                               const ColiMoeShape *shape);
void coli_cuda_moe_layer_destroy(ColiCuda *ctx, ColiMoeLayer *layer);
/* Device bytes held by the layer. */
size_t coli_cuda_moe_layer_bytes(const ColiMoeLayer *layer);

/* Load weights from device buffers in the container layouts of c/qwen.c
 * (QMat, c/qwen.c:68-81): router f32 [E x H] and shared gate row f32 [H];
 * shared expert int8 rows (row_bytes = cols) with one f32 scale per row;
 * routed expert codes [rows x row_bytes] with f32 scales [rows x groups].
 * Routed experts are repacked on the device into the MFMA tile layout. */
int coli_cuda_moe_layer_set_router(ColiCuda *ctx, ColiMoeLayer *layer,
                                   const float *router,
                                   const float *shared_gate);
int coli_cuda_moe_layer_set_shared_q8(ColiCuda *ctx, ColiMoeLayer *layer,
                                      const signed char *gate_q,
                                      const float *gate_s,
                                      const signed char *up_q,
                                      const float *up_s,
                                      const signed char *down_q,
                                      const float *down_s);
int coli_cuda_moe_layer_set_expert(ColiCuda *ctx, ColiMoeLayer *layer,
                                   int expert, const unsigned char *gate_q,
                                   const float *gate_s,
                                   const unsigned char *up_q,
                                   const float *up_s,
                                   const unsigned char *down_q,
                                   const float *down_s);
/* The same for one expert in container format expert_format: the layer's
 * own, or 2 or 4 in a layer created with format 2 or 4 (both held as int4
 * records).  No counterpart in the reference backend: for loaders whose
 * layers mix int2 and int4 experts, as EXPERT_Q2=1 reads a snapshot whose
 * .q2 sidecars cover only some experts (c/qwen.c:2207-2214). */
int coli_cuda_moe_layer_set_expert_format(ColiCuda *ctx, ColiMoeLayer *layer,
                                          int expert, int expert_format,
                                          const unsigned char *gate_q,
                                          const float *gate_s,
                                          const unsigned char *up_q,
                                          const float *up_s,
                                          const unsigned char *down_q,
                                          const float *down_s);
/* Generate the whole layer on the device from the counter hash of
 * shiftwing_amd/csrc/sw_synth.h (identical bytes to the host generator). */
int coli_cuda_moe_layer_synthesize(ColiCuda *ctx, ColiMoeLayer *layer,
                                   unsigned long long seed, int layer_index);
/* Device pointer to the layer's router [E x H] (for in-place edits). */
float *coli_cuda_moe_layer_router(ColiMoeLayer *layer);

/* A converted snapshot (the reference's container: every *.safetensors
 * file of a directory, c/st.h; tensor names and formats of c/qwen.c:2165-2295,
 * 2443-2457; the .q3 sidecar of c/tools/requantize_expert_q2.py).  Names are
 * looked up with the reference's prefixes "", "model.", "model.language_model."
 * and quantised matrices are classified as load_qmat_mode does (the .qtype
 * tag, else the payload and scale sizes).  Errors return -1 with a message
 * (the reference exits instead). */
typedef struct ColiContainer ColiContainer;
int coli_cuda_container_open(ColiContainer **out, const char *snapshot_dir);
void coli_cuda_container_close(ColiContainer *c);
/* tensors indexed over all files */
int coli_cuda_container_tensors(const ColiContainer *c);
/* MoE layer `layer` as stored: hidden, experts, intermediate,
 * shared_intermediate, expert_format (3 or 4; 2 for int2) and group_size.
 * topk is not stored: shape->topk is left as the caller set it.  sidecar
 * selects the routed experts' payload as the reference's switches do
 * (find_qmat_named, c/qwen.c:2198-2214): 0 the main payload, 1 the .q3
 * sidecar of every expert (EXPERT_Q3=1; required), 2 the .q2 sidecar where an
 * expert has one, else its main payload (EXPERT_Q2=1). */
int coli_cuda_container_moe_shape(const ColiContainer *c, int layer, int sidecar,
                                  ColiMoeShape *shape);
/* Create an HBM-resident layer and fill it from the container: router and
 * gate row (F32, BF16 or F16), the int8 shared expert (one scale per row),
 * every routed expert (int4, int3 from the .q3 sidecar, or int2 from .q2
 * sidecars / .qtype 2, in groups of 128; with sidecar 2 an expert without a
 * .q2 sidecar keeps its int4 payload, both held as int4 records), repacked
 * on the device.  Other
 * group sizes, which the reference's CPU path reads, return -1 with a
 * message: the device layer does not take them. */
int coli_cuda_moe_layer_load(ColiCuda *ctx, const ColiContainer *c, int layer,
                             int topk, int sidecar, ColiMoeLayer **out);

/* The MoE step for `tokens` activation rows (any number: a long block runs
 * as balanced steps of at most 2048 tokens, fewer for more than 512
 * experts; tokens are independent): y[t] = sum_k w[t,k] *
 * expert_{idx[t,k]}(x[t]) + sigmoid(gate . x[t]) * shared(x[t]).
 * x, y: device [tokens x H] f32.  route_idx / route_weight: optional device
 * outputs [tokens x K].  Routing is bit-exact with router_topk over the
 * reference's fp32 router logits; the shared expert uses IDOT. */
int coli_cuda_moe_forward(ColiCuda *ctx, ColiMoeLayer *layer, float *y,
                          const float *x, int tokens, int *route_idx,
                          float *route_weight);

/* The MoE half of a decoder layer on the residual stream, in place:
 * n = rmsnorm_zero(x, norm_weight) (c/qwen.c:1780-1784, 4593), then
 * x += MoE(n) (c/qwen.c:4594-4596).  x: device [tokens x H] f32, norm_weight:
 * device [H] (the layer's post_norm).  n is the CPU path's bit for bit (its
 * serial fp32 sum of squares), so the router sees the reference's input. */
int coli_cuda_moe_block(ColiCuda *ctx, ColiMoeLayer *layer, float *x,
                        const float *norm_weight, float eps, int tokens);
/* coli_cuda_moe_block with its intermediates (each optional, device):
 * hidden [tokens x H] receives n; route_idx / route_weight [tokens x K] the
 * routes chosen on n, as coli_cuda_moe_forward returns them. */
int coli_cuda_moe_block_ex(ColiCuda *ctx, ColiMoeLayer *layer, float *x,
                           const float *norm_weight, float eps, int tokens,
                           float *hidden, int *route_idx, float *route_weight);

/* Router only: idx / weight [tokens x K] (device). */
int coli_cuda_moe_route(ColiCuda *ctx, ColiMoeLayer *layer, const float *x,
                        int tokens, int *idx, float *weight);

/* Routing statistics since the layer was created: tokens routed, tokens that
 * needed the exact serial-chain fallback. */
int coli_cuda_moe_route_stats(ColiCuda *ctx, ColiMoeLayer *layer,
                              unsigned long long *tokens,
                              unsigned long long *exact_fallbacks);
/* out[0] tokens routed, out[1] tokens the bounds did not certify, out[2]
 * tokens that needed every expert's serial chain (the rest of out[1] were
 * settled by exact chains of the ambiguous experts only). */
int coli_cuda_moe_route_stats_full(ColiCuda *ctx, ColiMoeLayer *layer,
                                   unsigned long long out[3]);

/* Router policy: 0 = certified fast path with exact fallback (default),
 * 1 = always run the exact serial chain. */
int coli_cuda_moe_set_router_mode(ColiMoeLayer *layer, int mode);

/* n_layers MoE steps in order on the context stream: layer l reads
 * x + l*x_layer_stride and writes y + l*y_layer_stride (floats).  Strict
 * decode order: layer l+1 starts after layer l's output is written.  With
 * tokens == 1 and layers of one shape this is one persistent kernel that
 * needs every compute unit of the device for the duration of the call; a
 * call that cannot get them reports an error at the next coli_cuda_sync.
 * With 2 tokens the persistent kernel runs once per token (the tokens are
 * independent), which is faster than one many-token step per layer; from 3
 * tokens the many-token step is the faster. */
int coli_cuda_moe_forward_layers(ColiCuda *ctx, ColiMoeLayer *const *layers,
                                 int n_layers, float *y, const float *x,
                                 int tokens, size_t x_layer_stride,
                                 size_t y_layer_stride);

/* rows x cols synthetic activations ~N(0,1) (sw_synth.h), row r keyed by
 * (seed, layer, step0 + r): identical to the host generator. */
int coli_cuda_synth_activations(ColiCuda *ctx, float *x, int rows, int cols,
                                unsigned long long seed, int layer, int step0);

/* Stream timer on the context stream (HIP events). */
int coli_cuda_timer_start(ColiCuda *ctx);
int coli_cuda_timer_stop(ColiCuda *ctx, float *ms);

/* Per-stage device timing of the MoE step (HIP events between the step's
 * kernels).  Stages: 0 activation prep + router + top-k, 1 bucketing,
 * 2 shared gate/up, 3 routed gate/up, 4 hidden prep, 5 down (routed +
 * shared), 6 combine.  Accumulated over calls until reset. */
int coli_cuda_moe_stage_timing(ColiCuda *ctx, int enable);
int coli_cuda_moe_stage_times(ColiCuda *ctx, double ms[8],
                              unsigned long long *calls);

/* Single-token steps run the three-kernel decode path (route / experts /
 * down); with stage timing enabled its kernels are timed separately:
 * ms[0] route (router bounds + top-k, shared gate/up, digits), ms[1] experts
 * (routed gate/up, shared down), ms[2] routed down + combine. */
int coli_cuda_moe_decode_times(ColiCuda *ctx, double ms[3],
                               unsigned long long *calls);
/* Kernels for single-token steps: 1 (default) the persistent decode kernel
 * (one launch for a whole coli_cuda_moe_forward_layers stack; shapes it does
 * not take fall back to 2); 2 the three per-layer decode kernels; 0 the
 * many-token kernels.  Same results to the stated tolerance (for tests). */
int coli_cuda_moe_set_decode_kernels(ColiCuda *ctx, int mode);
/* Many-token steps: tokens per expert work item.  0 (default) picks 16 (each
 * expert's tiles read once per 16 tokens) when an item's activation digits
 * fit the LDS, else 8; 8 or 16 force one.  Same indices; outputs to the
 * stated tolerance (for tests and measurement). */
int coli_cuda_moe_set_item_tokens(ColiCuda *ctx, int tokens);
/* Stage stamps of the persistent decode kernel (measurement): while set,
 * every call writes the device wall clock (100 MHz) into the caller's device
 * buffer at [layer][workgroup][8]: layer start, router/shared done, router
 * barrier passed, selection done, routed gate/up done, hidden barrier passed,
 * down done, layer barrier passed.  Workgroups = the device's CU count.
 * trace = NULL, words = 0 switches it off. */
int coli_cuda_moe_stack_trace(ColiCuda *ctx, unsigned long long *trace,
                              size_t words);
/* The output head (c/qwen.c:4505-4516 for B rows, 4613-4616 for decode; the
 * device glue cuda_resident_output_try, 1097-1124): for each of `batch` rows
 * of x [batch x cols], n = rmsnorm_zero(x, norm_w, eps) (c/qwen.c:1780-1784,
 * the serial fp32 sum of squares) and logits [batch x vocab] = the int8
 * lm_head [vocab x row_bytes] (one f32 scale per row) applied with the CPU
 * path's IDOT (qrow_i8(n), exact int32 dots, ((float)dot * scale) * sx;
 * c/qwen.c:1696-1705, 1765-1768).  Bit-exact with the CPU path.  `hidden`
 * (optional, [batch x cols]) receives n, which the reference also returns.
 * cols <= 16384; the matrix is streamed once per group of four rows. */
int coli_cuda_output_head_q8(ColiCuda *ctx, float *logits, float *hidden,
                             const float *x, const float *norm_w, float eps,
                             int batch, const signed char *q,
                             const float *scales, int vocab, int cols,
                             int row_bytes);
/* Fault drill of the persistent decode kernel (no counterpart in the
 * reference; for tests of its timeout path).  The next launch keeps its last
 * `absent_workgroups` workgroups out, as if they never became resident, and
 * gives each wait `wait_limit_us` (1..2,000,000) instead of 2 s: every other
 * workgroup times out, raises the abort word and leaves, and the next
 * coli_cuda_sync returns -1 with the abort message after clearing the
 * kernel's device state.  0 absent workgroups disarms; a launch disarms. */
int coli_cuda_moe_stack_drill(ColiCuda *ctx, int absent_workgroups,
                              int wait_limit_us);

#ifdef __cplusplus
}
#endif

#endif
