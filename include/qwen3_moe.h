/* qwen3_moe.h — the reference's Qwen3-30B-A3B block / port interface, served by the MI355X
 * engine (C11 host code over the HIP kernels of cpg.h).
 *
 * Every type and function here has the reference's name, signature and meaning
 * (engine/blocks/qwen3_moe.h:15-115), so a caller written against the reference links
 * against libcachepotato_amd.so unchanged. What differs is where the work happens:
 *   - qwen3_map / qwen3_map_ex memory-map the CPW1 v4 file as the reference does, then upload
 *     its payload to HBM once and keep it there (the whole Q4 model is ~17.5 GB of 288 GB).
 *     The pager budget argument is accepted and ignored: nothing is ever evicted.
 *   - the QW3Layer's tensor pointers still point into the host mapping (the reference's
 *     contract: borrowed from the map, valid for the model's lifetime); each call translates
 *     them to the device copies.
 *   - qwen3_layer / qwen3_layer_kv / qwen3_mm take and return host buffers like the
 *     reference; the computation runs on the GPU (see cpg.h for the numerics).
 *   - QW3KV's k and v are DEVICE pointers (the cache lives in HBM); qwen3_kv_alloc and
 *     qwen3_kv_free manage them. Callers that only pass the cache around are unaffected.
 * Error codes are the reference's (engine/blocks/qwen3_moe.c:318-459): -1 generic, -2 out of
 * memory, -3 table mismatch, -4 incomplete layer, -5 d_exp, plus -7 for a device error.
 */
#ifndef QWEN3_MOE_H
#define QWEN3_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tensor encodings (engine/blocks/qwen3_moe.h:15-17) */
#define QW3_ENC_F32 0
#define QW3_ENC_Q8  8
#define QW3_ENC_Q4  4

/* a tensor and its encoding (qwen3_moe.h:19) */
typedef struct { const void *p; int enc; } QW3T;

/* One decoder layer plus the model-wide tensors, field for field as qwen3_moe.h:21-59 (the
   pager fields are kept for layout compatibility and hold -1 / 0). */
typedef struct {
    int d_model, n_heads, n_kv, head_dim, d_exp, n_experts, topk, vocab;
    int n_layers;
    float rope_theta, rms_eps;
    const float *ln1, *ln2, *q_norm, *k_norm;
    QW3T Wq, Wk, Wv, Wo;
    QW3T Wgate;
    QW3T *exp;              /* [e * 3 + kind], kind 0 gate, 1 up, 2 down */
    int exp_owned;
    const void *map;        /* the whole-file mapping */
    size_t map_len;
    QW3T embed, lm_head;
    const float *final_norm;
    uint64_t off_tens, off_data;
    uint32_t n_tens, n_enc;
    int enc_code[64];
    int cur_layer;
    int pager;
    int n_regions;
    int *tensor_reg;
    int *reg_exp;
    int reg_ln1, reg_ln2, reg_qnorm, reg_knorm;
    int reg_Wq, reg_Wk, reg_Wv, reg_Wo, reg_Wgate;
    int reg_embed, reg_lm_head, reg_final_norm;
    int embed_chunks, embed_rows;
    int *reg_embed_chunk;
    const void **embed_chunk_ptr;
} QW3Layer;

/* per-call outputs (qwen3_moe.h:61-66) */
typedef struct {
    float *attn;        /* (T, d_model)  pre-residual attention output */
    float *mlp;         /* (T, d_model)  pre-residual MoE output */
    float *router;      /* (T, n_experts) router logits */
    int *topk_idx;      /* (T, topk) selected experts, descending probability */
} QW3Out;

/* key/value cache (qwen3_moe.h:68-71); k and v are device pointers here, cap positions */
typedef struct { float *k, *v; int cap; } QW3KV;

/* qwen3_moe.h:73-75: host buffers of QW3Out (calloc'ed, so mlp starts at zero) */
int qwen3_layer_alloc(QW3Out *o, const QW3Layer *m, int T);
void qwen3_layer_free(QW3Out *o);
/* qwen3_moe.h:75: releases what qwen3_map / qwen3_load_blob allocated (host and device) */
void qwen3_layer_free_weights(QW3Layer *m);

/* qwen3_moe.h:77-78: T tokens at positions 0..T-1, no cache kept */
int qwen3_layer(const QW3Layer *m, const float *x, int T, QW3Out *o);
/* qwen3_moe.h:80-83: T tokens at positions pos0..pos0+T-1 against `cache` */
int qwen3_layer_kv(const QW3Layer *m, const float *x, int T, int pos0, QW3KV *cache, QW3Out *o);
int qwen3_kv_alloc(QW3KV *kv, const QW3Layer *m, int cap);
void qwen3_kv_free(QW3KV *kv);

/* qwen3_moe.h:85-88: out = W . x for one tensor of any encoding (host x and out) */
void qwen3_mm(const QW3T *t, float *out, const float *x, int n_in, int n_out);

/* qwen3_moe.h:90-91: flat host-endian blob (the reference's arithmetic-gate format) */
int qwen3_load_blob(QW3Layer *m, const char *path, float **owned);

/* qwen3_moe.h:93-103: CPW1 v4 loading */
int qwen3_map(QW3Layer *m, const char *path);
#define QW3_BUDGET_ENV  (-2L)
#define QW3_BUDGET_NONE (-1L)
int qwen3_map_ex(QW3Layer *m, const char *path, long budget_bytes);
int qwen3_bind_layer(QW3Layer *m, int layer);
int qwen3_load_v4(QW3Layer *m, const char *path, int layer);

#ifdef __cplusplus
}
#endif
#endif
