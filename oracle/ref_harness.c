/* ref_harness.c — drives the reference engine's own qwen3_layer on a hand-filled layer.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile together with the reference's
 * sources (read in place under the reference tree, never copied) into oracle/_ref/libref.so.
 * It is the pattern of the reference's block gate runner (tools/verify_qwen3_blocks.py:16-39):
 * fill QW3Layer, call qwen3_layer, read QW3Out.
 *
 * The attention half is made to produce exactly zero so that the MoE half
 * (engine/blocks/qwen3_moe.c:169-223) sees hh = x: one head of dimension 2 with all-zero
 * f32 Wq/Wk/Wv/Wo, so o->attn = Wo . ao = +0.0f exactly and x + attn == x (bit-for-bit,
 * +0.0 added to any non-NaN x leaves it unchanged except -0.0, which becomes +0.0 in the
 * reference as well).
 */
#include "blocks/qwen3_moe.h"
#include "kernels/parallel.h"

#include <stdlib.h>
#include <string.h>

/* Start the reference's process-global pool (engine/kernels/parallel.c:126-132). Only the
   first call counts; the thread count selects the Q4 numerics (kernels.c:514-540). */
int ref_threads_init(int n) { return cp_threads_init(n, 0); }

/* Runs qwen3_layer(m, x, T, o) with the MoE weights given and zero attention.
   exp_ptr[e*3 + kind] (kind 0 Wg, 1 Wu, 2 Wd); enc is 0 (f32), 4 (Q4_0) or 8 (Q8_0).
   Outputs: mlp (T,D), router (T,E), topk (T,K). Returns 0, or a negative code. */
int ref_moe_layer(int D, int E, int K, int F, float eps, const float *ln2,
                  const float *wgate, const void *const *exp_ptr, int enc,
                  const float *x, int T, float *mlp, float *router, int *topk) {
    const int H = 1, KVH = 1, HD = 2;
    QW3Layer m;
    memset(&m, 0, sizeof m);
    m.d_model = D; m.n_heads = H; m.n_kv = KVH; m.head_dim = HD; m.d_exp = F;
    m.n_experts = E; m.topk = K; m.vocab = 0; m.n_layers = 1;
    m.rope_theta = 1000000.0f; m.rms_eps = eps;
    float *ones = malloc(sizeof(float) * (size_t)D);
    float *zq = calloc((size_t)H * HD * D, sizeof(float));
    float *zk = calloc((size_t)KVH * HD * D, sizeof(float));
    float *zv = calloc((size_t)KVH * HD * D, sizeof(float));
    float *zo = calloc((size_t)D * H * HD, sizeof(float));
    float qk_ones[2] = {1.0f, 1.0f};
    if (!ones || !zq || !zk || !zv || !zo) return -2;
    for (int i = 0; i < D; i++) ones[i] = 1.0f;
    m.ln1 = ones; m.ln2 = ln2; m.q_norm = qk_ones; m.k_norm = qk_ones;
    m.Wq.p = zq; m.Wk.p = zk; m.Wv.p = zv; m.Wo.p = zo;
    m.Wq.enc = m.Wk.enc = m.Wv.enc = m.Wo.enc = QW3_ENC_F32;
    m.Wgate.p = wgate; m.Wgate.enc = QW3_ENC_F32;
    m.exp = calloc((size_t)E * 3, sizeof(QW3T));
    if (!m.exp) return -2;
    for (int i = 0; i < E * 3; i++) { m.exp[i].p = exp_ptr[i]; m.exp[i].enc = enc; }
    QW3Out o;
    int rc = qwen3_layer_alloc(&o, &m, T) ? -2 : qwen3_layer(&m, x, T, &o);
    if (rc == 0) {
        for (size_t i = 0; i < (size_t)T * D; i++)
            if (o.attn[i] != 0.0f) { rc = -9; break; }
        memcpy(mlp, o.mlp, sizeof(float) * (size_t)T * D);
        if (router) memcpy(router, o.router, sizeof(float) * (size_t)T * E);
        if (topk) memcpy(topk, o.topk_idx, sizeof(int) * (size_t)T * K);
    }
    qwen3_layer_free(&o);
    free(m.exp); free(ones); free(zq); free(zk); free(zv); free(zo);
    return rc;
}

/* Runs the reference's qwen3_layer_kv(m, x, T, pos0, cache, o) on a hand-filled layer with
   the given attention weights (encoding enc for Wq/Wk/Wv/Wo) and a MoE half of one f32
   expert with zero weights (so o->mlp stays zero). kc/vc: a cache of `cap` rows the caller
   owns (rows < pos0 filled by earlier calls). attn (T, D) receives o->attn. Returns 0 or a
   negative code. */
int ref_attn_layer(int D, int H, int KVH, int HD, float theta, float eps, const float *ln1,
                   const float *qn, const float *kn, const void *wq, const void *wk,
                   const void *wv, const void *wo, int enc, const float *x, int T, int pos0,
                   float *kc, float *vc, int cap, float *attn) {
    QW3Layer m;
    memset(&m, 0, sizeof m);
    m.d_model = D; m.n_heads = H; m.n_kv = KVH; m.head_dim = HD; m.d_exp = 32;
    m.n_experts = 1; m.topk = 1; m.n_layers = 1;
    m.rope_theta = theta; m.rms_eps = eps;
    float *ones = malloc(sizeof(float) * (size_t)D);
    float *wg = calloc((size_t)D, sizeof(float));
    float *ex = calloc((size_t)32 * D, sizeof(float));
    if (!ones || !wg || !ex) return -2;
    for (int i = 0; i < D; i++) ones[i] = 1.0f;
    m.ln1 = ln1; m.ln2 = ones; m.q_norm = qn; m.k_norm = kn;
    m.Wq.p = wq; m.Wk.p = wk; m.Wv.p = wv; m.Wo.p = wo;
    m.Wq.enc = m.Wk.enc = m.Wv.enc = m.Wo.enc = enc;
    m.Wgate.p = wg; m.Wgate.enc = QW3_ENC_F32;
    QW3T exp3[3] = {{ex, QW3_ENC_F32}, {ex, QW3_ENC_F32}, {ex, QW3_ENC_F32}};
    m.exp = exp3;
    QW3KV cache = {kc, vc, cap};
    QW3Out o;
    int rc = qwen3_layer_alloc(&o, &m, T) ? -2 : qwen3_layer_kv(&m, x, T, pos0, &cache, &o);
    if (rc == 0) memcpy(attn, o.attn, sizeof(float) * (size_t)T * D);
    qwen3_layer_free(&o);
    free(ones); free(wg); free(ex);
    return rc;
}
