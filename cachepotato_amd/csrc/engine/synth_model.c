/* synth_model.c — random-init Qwen3-MoE models as CPW1 v4 files (see cpw4.h). */
#define _GNU_SOURCE
#include "cpg.h"
#include "cpw4.h"
#include "qwen3_moe.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    uint64_t stream;
    double sigma;
    int enc, norm;          /* norm: 1 + N(0, sigma^2) f32 */
    size_t n;
} synth_src;

typedef struct {
    const qw3_synth_cfg *c;
    synth_src *src;
    void *stage;            /* device staging buffer of the GPU generator, or NULL */
    size_t stage_bytes;
} synth_ctx;

/* Quantised tensors of at least this many elements are generated on the GPU when a device
   context is open (the generator is bit-identical there), the rest on the host. */
#define SYNTH_DEV_MIN ((size_t)1 << 16)

static int synth_fill(void *user, int t, uint8_t *dst, size_t nbytes) {
    synth_ctx *x = (synth_ctx *)user;
    const synth_src *s = &x->src[t];
    if (s->enc == QW3_ENC_F32) {
        if (nbytes != s->n * 4) return -1;
        float *o = (float *)dst;
        cpg_gen_host(x->c->seed, s->stream, 0, s->n, s->sigma, o);
        if (s->norm)
            for (size_t i = 0; i < s->n; i++) o[i] = s->sigma > 0.0 ? 1.0f + o[i] : 1.0f;
        return 0;
    }
    if (nbytes != s->n / 32 * (s->enc == QW3_ENC_Q8 ? 34 : 18)) return -1;
    if (s->n >= SYNTH_DEV_MIN && cpg_current_device() >= 0) {
        if (nbytes > x->stage_bytes) {
            cpg_free(x->stage);
            x->stage = cpg_malloc(nbytes);
            x->stage_bytes = x->stage ? nbytes : 0;
        }
        /* element i of the stream is element i of a (n/32) x 32 matrix: the same blocks */
        if (x->stage && cpg_gen_blocks(s->enc, x->c->seed, s->stream, (int)(s->n / 32), 32,
                                       s->sigma, x->stage) == 0 &&
            cpg_d2h(dst, x->stage, nbytes) == 0)
            return 0;
        fprintf(stderr, "synthetic model: device generator failed (%s); using the host\n",
                cpg_last_error());
    }
    cpg_gen_blocks_host(s->enc, x->c->seed, s->stream, s->n, s->sigma, dst);
    return 0;
}

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

int qwen3_write_synthetic(const char *path, const qw3_synth_cfg *c, char *err, size_t errlen) {
    const int L = c->n_layers, D = c->d_model, H = c->n_heads, KV = c->n_kv, HD = c->head_dim;
    const int E = c->n_experts, K = c->topk, F = c->d_exp, V = c->vocab;
    if (L <= 0 || D <= 0 || H <= 0 || KV <= 0 || HD <= 0 || E <= 0 || K <= 0 || F <= 0 || V <= 0) {
        snprintf(err, errlen, "synthetic model: bad geometry");
        return -1;
    }
    const int nt = 1 + L * (9 + 3 * E) + 2;
    synth_src *src = calloc((size_t)nt, sizeof(synth_src));
    int *ids = calloc((size_t)nt, sizeof(int));
    cpw4_writer *w = cpw4_writer_create();
    int rc = 0;
    if (!src || !ids || !w) { rc = -2; goto out; }
    char name[96];
    int n = 0;
#define ADD(nm, enc_, role_, r, d0, d1, stream_, sigma_, norm_)                                 \
    do {                                                                                     \
        const uint32_t dims_[2] = {(uint32_t)(d0), (uint32_t)(d1)};                          \
        const int id_ = cpw4_add_tensor(w, nm, enc_, r, dims_, role_);                       \
        if (id_ < 0) { rc = id_; snprintf(err, errlen, "synthetic model: tensor %s", nm); goto out; } \
        src[id_] = (synth_src){stream_, sigma_, enc_, norm_, (size_t)(d0) * ((r) == 2 ? (size_t)(d1) : 1)}; \
        ids[n++] = id_;                                                                      \
    } while (0)
    const int embed_id = 0;
    const double embed_sigma = c->embed_sigma > 0.0 ? c->embed_sigma : 0.02;
    const double out_sigma = c->out_sigma > 0.0 ? c->out_sigma : 0.02;
    ADD("embed", c->enc_embed, CPW4_ROLE_EMBED, 2, V, D, CPG_STREAM(0, CPG_K_EMBED, 0), embed_sigma, 0);
    for (int l = 0; l < L; l++) {
        snprintf(name, sizeof name, "ln1.%d", l);
        ADD(name, QW3_ENC_F32, CPW4_ROLE_NORM, 1, D, 1, CPG_STREAM(l, CPG_K_NORM, 1), c->norm_sigma, 1);
        snprintf(name, sizeof name, "ln2.%d", l);
        ADD(name, QW3_ENC_F32, CPW4_ROLE_NORM, 1, D, 1, CPG_STREAM(l, CPG_K_NORM, 2), c->norm_sigma, 1);
        snprintf(name, sizeof name, "q_norm.%d", l);
        ADD(name, QW3_ENC_F32, CPW4_ROLE_NORM, 1, HD, 1, CPG_STREAM(l, CPG_K_NORM, 3), c->norm_sigma, 1);
        snprintf(name, sizeof name, "k_norm.%d", l);
        ADD(name, QW3_ENC_F32, CPW4_ROLE_NORM, 1, HD, 1, CPG_STREAM(l, CPG_K_NORM, 4), c->norm_sigma, 1);
        snprintf(name, sizeof name, "Wq.%d", l);
        ADD(name, c->enc_attn, CPW4_ROLE_ATTN, 2, H * HD, D, CPG_STREAM(l, CPG_K_ATTN, 0), 0.02, 0);
        snprintf(name, sizeof name, "Wk.%d", l);
        ADD(name, c->enc_attn, CPW4_ROLE_ATTN, 2, KV * HD, D, CPG_STREAM(l, CPG_K_ATTN, 1), 0.02, 0);
        snprintf(name, sizeof name, "Wv.%d", l);
        ADD(name, c->enc_attn, CPW4_ROLE_ATTN, 2, KV * HD, D, CPG_STREAM(l, CPG_K_ATTN, 2), 0.02, 0);
        snprintf(name, sizeof name, "Wo.%d", l);
        ADD(name, c->enc_attn, CPW4_ROLE_ATTN, 2, D, H * HD, CPG_STREAM(l, CPG_K_ATTN, 3), out_sigma, 0);
        snprintf(name, sizeof name, "Wgate.%d", l);
        ADD(name, QW3_ENC_F32, CPW4_ROLE_ROUTER, 2, E, D, CPG_STREAM(l, CPG_K_WGATE, 0), 0.02, 0);
        for (int e = 0; e < E; e++) {
            snprintf(name, sizeof name, "expert.%d.%d.Wg", l, e);
            ADD(name, c->enc_exp, CPW4_ROLE_EXPERT, 2, F, D, CPG_STREAM(l, CPG_K_WG, e), 0.02, 0);
            snprintf(name, sizeof name, "expert.%d.%d.Wu", l, e);
            ADD(name, c->enc_exp, CPW4_ROLE_EXPERT, 2, F, D, CPG_STREAM(l, CPG_K_WU, e), 0.02, 0);
            snprintf(name, sizeof name, "expert.%d.%d.Wd", l, e);
            ADD(name, c->enc_exp, CPW4_ROLE_EXPERT, 2, D, F, CPG_STREAM(l, CPG_K_WD, e), out_sigma, 0);
        }
    }
    ADD("final_norm", QW3_ENC_F32, CPW4_ROLE_NORM, 1, D, 1, CPG_STREAM(L, CPG_K_NORM, 5), c->norm_sigma, 1);
    const int head_id = n;
    ADD("lm_head", c->enc_head, CPW4_ROLE_HEAD, 2, V, D, CPG_STREAM(0, CPG_K_HEAD, 0), 0.02, 0);
#undef ADD
    {   /* blocks (convert.py:204-215) */
        const uint32_t eref = (uint32_t)embed_id, ep[3] = {(uint32_t)V, (uint32_t)D, 0};
        if ((rc = cpw4_add_block(w, CPW4_BLK_EMBED, 0xFFFFFFFFu, &eref, 1, ep, 3)) < 0) goto out;
        for (int l = 0; l < L; l++) {
            const int b = 1 + l * (9 + 3 * E);   /* ids: ln1 ln2 qn kn Wq Wk Wv Wo Wgate experts */
            const uint32_t ar[6] = {(uint32_t)(b + 4), (uint32_t)(b + 5), (uint32_t)(b + 6),
                                    (uint32_t)(b + 7), (uint32_t)(b + 2), (uint32_t)(b + 3)};
            const uint32_t ap[6] = {(uint32_t)H, (uint32_t)KV, (uint32_t)HD, f32_bits(c->rope_theta), 1, 0};
            if ((rc = cpw4_add_block(w, CPW4_BLK_ATTN, (uint32_t)l, ar, 6, ap, 6)) < 0) goto out;
            const uint32_t mr = (uint32_t)(b + 8);
            const uint32_t mp[10] = {(uint32_t)E, (uint32_t)K, 0, 1, 0, f32_bits(1.0f), 0, 0, 0, 1};
            if ((rc = cpw4_add_block(w, CPW4_BLK_MOE, (uint32_t)l, &mr, 1, mp, 10)) < 0) goto out;
        }
    }
    for (int l = 0; l < L; l++)                   /* one region per expert (convert.py:217-222) */
        for (int e = 0; e < E; e++) {
            const int lo = 1 + l * (9 + 3 * E) + 9 + 3 * e;
            if ((rc = cpw4_add_region(w, lo, lo + 3, CPW4_REG_EXPERT, l, (uint32_t)e, (uint32_t)e + 1)) < 0) goto out;
        }
    for (int t = 0; t < n; t++) {                 /* and one per other tensor */
        if (src[t].enc != QW3_ENC_F32 && t != embed_id && t != head_id) {
            const int rel = (t - 1) % (9 + 3 * E);
            if (t >= 1 && t < 1 + L * (9 + 3 * E) && rel >= 9) continue;      /* an expert */
        }
        if ((rc = cpw4_add_region(w, t, t + 1, CPW4_REG_TENSOR, 0xFFFF, 0, 1)) < 0) goto out;
    }
    {   /* f32 tensors first, then the quantised ones (convert.py:239-242) */
        int *order = malloc(sizeof(int) * (size_t)n), k = 0;
        if (!order) { rc = -2; goto out; }
        for (int t = 0; t < n; t++) if (src[t].enc == QW3_ENC_F32) order[k++] = t;
        for (int t = 0; t < n; t++) if (src[t].enc != QW3_ENC_F32) order[k++] = t;
        synth_ctx ctx = {c, src, NULL, 0};
        rc = cpw4_write(w, path, order, synth_fill, &ctx, err, errlen);
        if (ctx.stage) cpg_free(ctx.stage);
        free(order);
    }
out:
    cpw4_writer_destroy(w);
    free(src);
    free(ids);
    return rc;
}
