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
#define _POSIX_C_SOURCE 199309L   /* clock_gettime under -std=c11 */
#include "blocks/qwen3_moe.h"
#include "kernels/parallel.h"

#include <stdlib.h>
#include <string.h>

/* Start the reference's process-global pool (engine/kernels/parallel.c:126-132). Only the
   first call counts; the thread count selects the Q4 numerics (kernels.c:514-540). */
int ref_threads_init(int n) { return cp_threads_init(n, 0); }
/* The same with the reference's core pinning on or off (engine/kernels/parallel.c:45-56,
   :94: the caller on core 0, worker i on core i + 1), as CP_PIN_CORES=1 selects. */
int ref_threads_init_pinned(int n, int pin) { return cp_threads_init(n, pin); }

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

/* ---------------------------------------------------------------- whole-model greedy decode
 * The reference eval driver's --decode mode (tools/qwen3_eval.c:280-400) over the reference's
 * own qwen3_map / qwen3_bind_layer / qwen3_layer_kv / rmsnorm / qwen3_mm / q8_dequant_row, as
 * a library call: the driver's main() parses argv and writes files, so its three static
 * helpers (embed_rows :200-225, run_layers :155-179, apply_head :183-195) are restated here
 * in its order of operations, with its token loop.
 *   tokens[gen], route[L][gen][K] (optional), step_ms[gen] (optional), *prefill_ms (optional).
 * vocab > 0 replaces the 151936 that qwen3_map_ex assumes for every file (qwen3_moe.c:394-403),
 * so that small test files with another vocabulary can be run; the converter's files have
 * exactly that many rows, where it changes nothing.
 * Stops after max_seconds of decode (0 = no limit) and returns the number of tokens produced,
 * or a negative code. */
#include "kernels/kernels.h"
#include <math.h>
#include <time.h>

static double h_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static void h_embed_rows(QW3Layer *m, const int *ids, int T, float *x, int D) {
    const size_t q8_row = (size_t)((D / 32) * 34), q4_row = (size_t)((D / 32) * 18);
    for (int t = 0; t < T; t++) {
        int row = ids[t];
        const void *base;
        if (m->embed_chunks > 0 && m->embed_rows > 0) {
            int c = row / m->embed_rows, r = row - c * m->embed_rows;
            if (c >= m->embed_chunks) { c = m->embed_chunks - 1; r = row - c * m->embed_rows; }
            base = m->embed_chunk_ptr[c];
            row = r;
        } else {
            base = m->embed.p;
        }
        if (m->embed.enc == QW3_ENC_Q8)
            q8_dequant_row((const unsigned char *)base + (size_t)row * q8_row, x + (size_t)t * D, D);
        else if (m->embed.enc == QW3_ENC_Q4)
            q4_dequant_row((const unsigned char *)base + (size_t)row * q4_row, x + (size_t)t * D, D);
        else
            memcpy(x + (size_t)t * D, (const float *)base + (size_t)row * D, sizeof(float) * D);
    }
}

static int h_run_layers(QW3Layer *layers, float *x, int T, int pos0, QW3KV *kv, int L,
                        int *route, size_t route_stride) {
    QW3Out o;
    for (int l = 0; l < L; l++) {
        QW3Layer *m = &layers[l];
        const int D = m->d_model, K = m->topk;
        if (qwen3_layer_alloc(&o, m, T)) return -1;
        if (qwen3_layer_kv(m, x, T, pos0, &kv[l], &o)) { qwen3_layer_free(&o); return -1; }
        for (int t = 0; t < T; t++)
            for (int j = 0; j < D; j++)
                x[(size_t)t * D + j] += o.attn[(size_t)t * D + j] + o.mlp[(size_t)t * D + j];
        if (route) memcpy(route + (size_t)l * route_stride, o.topk_idx, sizeof(int) * (size_t)T * K);
        qwen3_layer_free(&o);
    }
    return 0;
}

static void h_apply_head(QW3Layer *m, float *x, float *logits, int V) {
    const int D = m->d_model;
    rmsnorm(x, x, m->final_norm, D, m->rms_eps);
    qwen3_mm(&m->lm_head, logits, x, D, V);
}

static int h_argmax(const float *v, int n) {
    int best = 0;
    for (int j = 1; j < n; j++) if (v[j] > v[best]) best = j;
    return best;
}

/* Optional: gap[s] = the step's largest logit minus the second largest (how close the greedy
   choice was to a tie), for ref_eval_decode calls made while set. */
static float *g_gap;
void ref_set_gap_out(float *gap) { g_gap = gap; }

/* Optional: the logits of the first step (the head on the prompt's last position, after the
   prefill; what tools/qwen3_eval.c:417-423 writes as the step's .logits), copied to `out`
   (vocab floats) by ref_eval_decode calls made while set. */
static float *g_logits0;
void ref_set_logits0_out(float *out) { g_logits0 = out; }

static float h_gap(const float *v, int n, int best) {
    float second = -INFINITY;
    for (int j = 0; j < n; j++)
        if (j != best && v[j] > second) second = v[j];
    return v[best] - second;
}

int ref_eval_decode(const char *path, int L, int vocab, const int *ids, int T, int gen,
                    double max_seconds, int *tokens, int *route, float *step_ms,
                    float *prefill_ms) {
    QW3Layer m;
    memset(&m, 0, sizeof m);
    if (qwen3_map(&m, path) || qwen3_bind_layer(&m, 0)) return -1;
    if (vocab > 0) m.vocab = vocab;
    const int D = m.d_model, V = m.vocab, K = m.topk, E = m.n_experts;
    if (L <= 0 || L > m.n_layers) L = m.n_layers;
    QW3Layer *layers = calloc((size_t)L, sizeof(QW3Layer));
    QW3KV *kv = calloc((size_t)L, sizeof(QW3KV));
    float *x = malloc(sizeof(float) * (size_t)T * D), *row = malloc(sizeof(float) * D);
    float *logits = malloc(sizeof(float) * (size_t)V);
    int rc = 0, s = 0;
    if (!layers || !kv || !x || !row || !logits) { rc = -2; goto out; }
    /* qwen3_bind_layer clears 128 region ids whatever the expert count (qwen3_moe.c:476) */
    const int EA = E > 128 ? E : 128;
    for (int l = 0; l < L; l++) {
        layers[l] = m;
        layers[l].exp = calloc((size_t)EA * 3, sizeof(QW3T));
        layers[l].reg_exp = calloc((size_t)EA, sizeof(int));
        if (!layers[l].exp || !layers[l].reg_exp || qwen3_bind_layer(&layers[l], l) ||
            qwen3_kv_alloc(&kv[l], &m, T + gen)) { rc = -1; goto out; }
    }
    h_embed_rows(&layers[0], ids, T, x, D);
    double t0 = h_now();
    if (h_run_layers(layers, x, T, 0, kv, L, NULL, 0)) { rc = -3; goto out; }
    if (prefill_ms) *prefill_ms = (float)((h_now() - t0) * 1e3);
    const float *last = x + (size_t)(T - 1) * D;
    const double d0 = h_now();
    for (s = 0; s < gen; s++) {
        const double ts = h_now();
        memcpy(row, last, sizeof(float) * D);
        h_apply_head(&layers[0], row, logits, V);
        tokens[s] = h_argmax(logits, V);
        if (g_gap) g_gap[s] = h_gap(logits, V, tokens[s]);
        if (g_logits0 && s == 0) memcpy(g_logits0, logits, sizeof(float) * (size_t)V);
        h_embed_rows(&layers[0], &tokens[s], 1, row, D);
        if (h_run_layers(layers, row, 1, T + s, kv, L, route ? route + (size_t)s * K : NULL,
                         (size_t)gen * K)) { rc = -3; goto out; }
        if (step_ms) step_ms[s] = (float)((h_now() - ts) * 1e3);
        last = row;
        if (max_seconds > 0 && h_now() - d0 > max_seconds) { s++; break; }
    }
out:
    if (layers)
        for (int l = 0; l < L; l++) {
            free(layers[l].exp);
            free(layers[l].reg_exp);
            if (kv) qwen3_kv_free(&kv[l]);
        }
    free(layers); free(kv); free(x); free(row); free(logits);
    qwen3_layer_free_weights(&m);
    return rc ? rc : s;
}

/* ---- the tokenizer's special tokens, made well defined ----------------------------------
 * tokenizer_qwen_encode advances past a matched special token by strlen() of its vocabulary
 * entry (engine/tokenizers/tokenizer_qwen.c:110), but tokenizer_load stores entries without
 * a terminating NUL (engine/tokenizers/tokenizer.c:30-33): the advance then depends on
 * whatever byte follows the entry on the heap. It is the token's length when that byte is
 * zero, which is what the reference's own runs see on a fresh heap. These give every entry
 * from the first special id on that terminating NUL (a copy one byte longer), so the
 * reference's encoding is that length-based one whatever the heap holds. Returns the number
 * of entries terminated, or -1 if tk does not look like a loaded tokenizer. */
#include "tokenizers/tokenizer.h"
#define REF_SPECIAL_FIRST 151643u

int ref_tok_terminate_specials(Tokenizer *tk) {
    if (!tk || !tk->vocab || !tk->vocab_len || tk->n_vocab > (1u << 24)) return -1;
    int n = 0;
    for (uint32_t id = REF_SPECIAL_FIRST; id < tk->n_vocab; id++) {
        const size_t len = tk->vocab_len[id];
        char *s = malloc(len + 1);
        if (!s) return -1;
        memcpy(s, tk->vocab[id], len);
        s[len] = 0;
        free(tk->vocab[id]);
        tk->vocab[id] = s;
        n++;
    }
    return n;
}

/* The Tokenizer inside a model from the reference's cp_open: struct cp_model
   (engine/api/cachepotato.c:33-43) is a QW3Layer, two pointers, then the Tokenizer. The
   caller checks the result against the files it wrote (vocabulary size). */
Tokenizer *ref_model_tokenizer(void *model) {
    return model ? (Tokenizer *)((char *)model + sizeof(QW3Layer) + 2 * sizeof(void *)) : NULL;
}
