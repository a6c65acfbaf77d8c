/* qwen3_moe.c — the reference's Qwen3-MoE block / port interface (engine/blocks/qwen3_moe.h:
 * 73-115) served from HBM by the kernels of cpg.h.
 *
 * Loading follows the reference (engine/blocks/qwen3_moe.c:296-459): the CPW1 v4 file is
 * memory-mapped, its tables validated (cpw4.c), and a layer is bound by tensor name into
 * host pointers into the mapping. On top of that, the payload is copied to HBM once, and the
 * first call on a layer builds its device form: q|k|v and Wo repacked row-tiled, the layer's
 * experts repacked into one row-tiled pool, norms and router used in place. The
 * host-buffer entry points (qwen3_layer_kv, qwen3_mm) upload their inputs, run the kernels
 * and copy the outputs back, with the reference's semantics (QW3Out.mlp accumulated into,
 * router logits and top-k indices filled).
 */
#define _GNU_SOURCE
#include "qw3_engine.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define QW3_MAX_MAPS 16
#define QW3_CHUNK_T 256         /* tokens per device pass of the host-buffer entry points */

static qw3_state g_maps[QW3_MAX_MAPS];

int qw3_ensure_device(void) {
    if (cpg_current_device() >= 0) return 0;
    if (cpg_init(0)) {
        fprintf(stderr, "qwen3: no device: %s\n", cpg_last_error());
        return -7;
    }
    return 0;
}

qw3_state *qw3_state_of(const void *map) {
    if (!map) return NULL;
    for (int i = 0; i < QW3_MAX_MAPS; i++)
        if (g_maps[i].used && g_maps[i].map == (const uint8_t *)map) return &g_maps[i];
    return NULL;
}

const void *qw3_dev_ptr(const qw3_state *st, const void *host) {
    const uint8_t *p = (const uint8_t *)host, *d0 = st->map + st->f.off_data;
    if (!p || p < d0 || p >= st->map + st->map_len) return NULL;
    return st->dev + (p - d0);
}

static int dev_err(const char *what) {
    fprintf(stderr, "qwen3: %s: %s\n", what, cpg_last_error());
    return -7;
}

/* ------------------------------------------------------------------ outputs and caches */

int qwen3_layer_alloc(QW3Out *o, const QW3Layer *m, int T) {
    o->attn = calloc((size_t)T * m->d_model, sizeof(float));
    o->mlp = calloc((size_t)T * m->d_model, sizeof(float));
    o->router = calloc((size_t)T * m->n_experts, sizeof(float));
    o->topk_idx = calloc((size_t)T * m->topk, sizeof(int));
    return (o->attn && o->mlp && o->router && o->topk_idx) ? 0 : -1;
}

void qwen3_layer_free(QW3Out *o) {
    free(o->attn);
    free(o->mlp);
    free(o->router);
    free(o->topk_idx);
    memset(o, 0, sizeof *o);
}

int qwen3_kv_alloc(QW3KV *kv, const QW3Layer *m, int cap) {
    memset(kv, 0, sizeof *kv);
    if (cap <= 0 || qw3_ensure_device()) return -1;
    const size_t n = sizeof(float) * (size_t)cap * m->n_kv * m->head_dim;
    kv->k = cpg_malloc(n);
    kv->v = cpg_malloc(n);
    if (!kv->k || !kv->v || cpg_memset(kv->k, 0, n) || cpg_memset(kv->v, 0, n) || cpg_sync()) {
        cpg_free(kv->k);
        cpg_free(kv->v);
        memset(kv, 0, sizeof *kv);
        return -1;
    }
    kv->cap = cap;
    return 0;
}

void qwen3_kv_free(QW3KV *kv) {
    if (cpg_current_device() >= 0) {
        cpg_free(kv->k);
        cpg_free(kv->v);
    }
    memset(kv, 0, sizeof *kv);
}

/* ------------------------------------------------------------------ mapping */

static void state_release(qw3_state *st) {
    if (cpg_current_device() >= 0) {
        cpg_sync();
        if (st->lay)
            for (int l = 0; l < st->n_layers; l++) {
                cpg_free(st->lay[l].wqkv);
                cpg_free(st->lay[l].wo);
                cpg_free(st->lay[l].experts);
            }
        cpg_free(st->dev);
        cpg_free(st->rope);
        cpg_free(st->dx);
        cpg_free(st->dattn);
        cpg_free(st->dmlp);
        cpg_free(st->drouter);
        cpg_free(st->dtopk);
        cpg_moe_ws_destroy(st->mws);
        cpg_attn_ws_destroy(st->aws);
    }
    free(st->lay);
    if (st->owns_map && st->map) munmap((void *)st->map, st->map_len);
    cpw4_release(&st->f);
    memset(st, 0, sizeof *st);
}

static int tensor_index(const cpw4_file *f, const char *fmt, int a, int b) {
    char name[96];
    snprintf(name, sizeof name, fmt, a, b);
    return cpw4_find(f, name);
}

static float f32_of(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t param(const cpw4_block *b, uint32_t i) {
    const uint8_t *p = b->params + 4 * i;
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

int qwen3_map(QW3Layer *m, const char *path) { return qwen3_map_ex(m, path, QW3_BUDGET_ENV); }

int qwen3_map_ex(QW3Layer *m, const char *path, long budget_bytes) {
    (void)budget_bytes;         /* the whole model is resident in HBM: there is no pager */
    memset(m, 0, sizeof *m);
    int fd = open(path, O_RDONLY);
    if (fd < 0) { perror(path); return -1; }
    struct stat sb;
    if (fstat(fd, &sb) != 0) { close(fd); return -1; }
    const size_t len = (size_t)sb.st_size;
    const uint8_t *base = mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) { perror("mmap"); return -1; }
    qw3_state *st = NULL;
    for (int i = 0; i < QW3_MAX_MAPS && !st; i++)
        if (!g_maps[i].used) st = &g_maps[i];
    if (!st) { munmap((void *)base, len); fprintf(stderr, "qwen3: too many mapped models\n"); return -2; }
    memset(st, 0, sizeof *st);
    st->map = base;
    st->map_len = len;
    st->owns_map = 1;
    char err[256] = {0};
    int rc = cpw4_parse(&st->f, base, len, err, sizeof err);
    if (rc) {
        fprintf(stderr, "%s\n", err[0] ? err : "v4: parse failed");
        munmap((void *)base, len);
        memset(st, 0, sizeof *st);
        return rc;
    }
    /* every tensor the engine binds against the file's own geometry, before anything is
       sized from one tensor and used on another */
    cpw4_qwen3_geom geo;
    if ((rc = cpw4_qwen3_geometry(&st->f, &geo, err, sizeof err))) {
        fprintf(stderr, "%s\n", err);
        cpw4_release(&st->f);
        munmap((void *)base, len);
        memset(st, 0, sizeof *st);
        return rc;
    }
    const cpw4_file *f = &st->f;
    m->map = base;
    m->map_len = len;
    m->n_tens = f->n_tensors;
    m->n_enc = f->n_enc;
    m->n_regions = (int)f->n_regions;
    m->off_tens = f->off_tensors;
    m->off_data = f->off_data;
    m->n_layers = f->n_layers;
    for (uint32_t i = 0; i < f->n_enc && i < 64; i++) m->enc_code[i] = f->enc[i].code;
    /* the reference's constants (qwen3_moe.c:394-403), replaced by what the file's blocks
       declare where they declare it */
    m->rope_theta = 1000000.0f;
    m->rms_eps = 1e-6f;
    m->topk = 8;
    m->vocab = 151936;
    int n_exp = 128;
    for (uint32_t i = 0; i < f->n_blocks; i++) {
        const cpw4_block *b = &f->blocks[i];
        if (b->kind == CPW4_BLK_ATTN && b->n_params > 3) m->rope_theta = f32_of(param(b, 3));
        if (b->kind == CPW4_BLK_MOE && b->n_params > 1) {
            m->topk = (int)param(b, 1);
            if ((int)param(b, 0) > n_exp) n_exp = (int)param(b, 0);
        }
    }
    const int head = cpw4_find(f, "lm_head");
    if (head >= 0) m->vocab = (int)f->tensors[head].dims[0];
    if (geo.n_experts > n_exp) n_exp = geo.n_experts;   /* every layer's E is geo.n_experts */
    m->exp = calloc((size_t)n_exp * 3, sizeof(QW3T));
    m->reg_exp = calloc((size_t)n_exp, sizeof(int));
    m->tensor_reg = calloc(f->n_tensors ? f->n_tensors : 1, sizeof(int));
    if (!m->exp || !m->reg_exp || !m->tensor_reg) { rc = -2; goto fail; }
    m->exp_owned = 1;
    for (uint32_t i = 0; i < f->n_tensors; i++) m->tensor_reg[i] = -1;
    for (uint32_t g = 0; g < f->n_regions; g++)
        for (uint32_t t = f->regions[g].tensor_lo; t < f->regions[g].tensor_hi; t++) m->tensor_reg[t] = (int)g;
    m->cur_layer = -1;
    m->reg_ln1 = m->reg_ln2 = m->reg_qnorm = m->reg_knorm = -1;
    m->reg_Wq = m->reg_Wk = m->reg_Wv = m->reg_Wo = m->reg_Wgate = -1;
    m->reg_embed = m->reg_lm_head = m->reg_final_norm = -1;

    /* the payload to HBM, once */
    if ((rc = qw3_ensure_device())) goto fail;
    const size_t plen = len - f->off_data;
    st->dev = cpg_malloc(plen);
    if (!st->dev) { rc = -2; fprintf(stderr, "qwen3: %s\n", cpg_last_error()); goto fail; }
    if (cpg_h2d(st->dev, base + f->off_data, plen)) { rc = dev_err("upload"); goto fail; }
    st->theta = m->rope_theta;
    st->eps = m->rms_eps;
    st->topk = m->topk;
    st->n_layers = f->n_layers;
    st->lay = calloc((size_t)(f->n_layers > 0 ? f->n_layers : 1), sizeof(qw3_dev_layer));
    if (!st->lay) { rc = -2; goto fail; }
    const int qn0 = cpw4_find(f, "q_norm.0");
    st->head_dim = qn0 >= 0 ? (int)f->tensors[qn0].dims[0] : 0;
    if (st->head_dim > 0) {
        const size_t n = (size_t)QW3_MAX_POS * st->head_dim;
        float *tab = malloc(sizeof(float) * n);
        st->rope = cpg_malloc(sizeof(float) * n);
        if (!tab || !st->rope) { free(tab); rc = -2; goto fail; }
        rc = cpg_rope_table(st->theta, st->head_dim, QW3_MAX_POS, tab) ||
             cpg_h2d(st->rope, tab, sizeof(float) * n);
        free(tab);
        if (rc) { rc = dev_err("rope table"); goto fail; }
    }
    st->used = 1;
    return 0;
fail:
    free(m->exp);
    free(m->reg_exp);
    free(m->tensor_reg);
    state_release(st);
    memset(m, 0, sizeof *m);
    return rc;
}

int qwen3_bind_layer(QW3Layer *m, int layer) {
    qw3_state *st = qw3_state_of(m->map);
    if (!st) { fprintf(stderr, "qwen3: bind on a layer that qwen3_map did not map\n"); return -1; }
    const cpw4_file *f = &st->f;
    m->cur_layer = layer;
    m->ln1 = m->ln2 = m->q_norm = m->k_norm = m->final_norm = NULL;
    m->Wq.p = m->Wk.p = m->Wv.p = m->Wo.p = m->Wgate.p = NULL;
    m->embed.p = m->lm_head.p = NULL;
    m->reg_ln1 = m->reg_ln2 = m->reg_qnorm = m->reg_knorm = -1;
    m->reg_Wq = m->reg_Wk = m->reg_Wv = m->reg_Wo = m->reg_Wgate = -1;
    m->reg_embed = m->reg_lm_head = m->reg_final_norm = -1;
#define T_(i) (&f->tensors[i])
#define ENC_(i) (f->enc[f->tensors[i].enc].code)
#define REG_(i) (m->tensor_reg ? m->tensor_reg[i] : -1)
    int i;
    if ((i = cpw4_find(f, "embed")) >= 0) {
        m->embed.p = cpw4_data(f, i); m->embed.enc = ENC_(i); m->reg_embed = REG_(i);
    } else {
        int c = 0;
        while (tensor_index(f, "embed.%d", c, 0) >= 0) c++;
        if (c > 0) {
            int *rg = realloc(m->reg_embed_chunk, sizeof(int) * (size_t)c);
            const void **pp = realloc(m->embed_chunk_ptr, sizeof(void *) * (size_t)c);
            if (!rg || !pp) return -2;
            m->reg_embed_chunk = rg;
            m->embed_chunk_ptr = pp;
            for (int k = 0; k < c; k++) {
                const int t = tensor_index(f, "embed.%d", k, 0);
                m->embed_chunk_ptr[k] = cpw4_data(f, t);
                m->reg_embed_chunk[k] = REG_(t);
                if (k == 0) { m->embed_rows = (int)T_(t)->dims[0]; m->embed.enc = ENC_(t); }
            }
            m->embed_chunks = c;
        }
    }
    if ((i = cpw4_find(f, "lm_head")) >= 0) { m->lm_head.p = cpw4_data(f, i); m->lm_head.enc = ENC_(i); m->reg_lm_head = REG_(i); }
    if ((i = cpw4_find(f, "final_norm")) >= 0) {
        m->final_norm = (const float *)cpw4_data(f, i); m->d_model = (int)T_(i)->dims[0]; m->reg_final_norm = REG_(i);
    }
    if ((i = tensor_index(f, "ln1.%d", layer, 0)) >= 0) {
        m->ln1 = (const float *)cpw4_data(f, i); m->d_model = (int)T_(i)->dims[0]; m->reg_ln1 = REG_(i);
    }
    if ((i = tensor_index(f, "ln2.%d", layer, 0)) >= 0) { m->ln2 = (const float *)cpw4_data(f, i); m->reg_ln2 = REG_(i); }
    if ((i = tensor_index(f, "q_norm.%d", layer, 0)) >= 0) {
        m->q_norm = (const float *)cpw4_data(f, i); m->head_dim = (int)T_(i)->dims[0]; m->reg_qnorm = REG_(i);
    }
    if ((i = tensor_index(f, "k_norm.%d", layer, 0)) >= 0) { m->k_norm = (const float *)cpw4_data(f, i); m->reg_knorm = REG_(i); }
    if ((i = tensor_index(f, "Wgate.%d", layer, 0)) >= 0) {
        m->Wgate.p = cpw4_data(f, i); m->Wgate.enc = ENC_(i); m->n_experts = (int)T_(i)->dims[0]; m->reg_Wgate = REG_(i);
    }
    if ((i = tensor_index(f, "Wq.%d", layer, 0)) >= 0) {
        m->Wq.p = cpw4_data(f, i); m->Wq.enc = ENC_(i); m->reg_Wq = REG_(i);
        if (m->head_dim) m->n_heads = (int)(T_(i)->dims[0] / (uint32_t)m->head_dim);
    }
    if ((i = tensor_index(f, "Wk.%d", layer, 0)) >= 0) {
        m->Wk.p = cpw4_data(f, i); m->Wk.enc = ENC_(i); m->reg_Wk = REG_(i);
        if (m->head_dim) m->n_kv = (int)(T_(i)->dims[0] / (uint32_t)m->head_dim);
    }
    if ((i = tensor_index(f, "Wv.%d", layer, 0)) >= 0) { m->Wv.p = cpw4_data(f, i); m->Wv.enc = ENC_(i); m->reg_Wv = REG_(i); }
    if ((i = tensor_index(f, "Wo.%d", layer, 0)) >= 0) { m->Wo.p = cpw4_data(f, i); m->Wo.enc = ENC_(i); m->reg_Wo = REG_(i); }
    if (m->exp) {
        static const char *kinds[3] = {"Wg", "Wu", "Wd"};
        for (int e = 0; e < m->n_experts; e++) {
            if (m->reg_exp) m->reg_exp[e] = -1;
            for (int k = 0; k < 3; k++) {
                char name[96];
                snprintf(name, sizeof name, "expert.%d.%d.%s", layer, e, kinds[k]);
                const int t = cpw4_find(f, name);
                m->exp[(size_t)e * 3 + k].p = t >= 0 ? cpw4_data(f, t) : NULL;
                m->exp[(size_t)e * 3 + k].enc = t >= 0 ? ENC_(t) : 0;
                if (t >= 0 && m->reg_exp) m->reg_exp[e] = REG_(t);
            }
        }
    }
    if (!m->ln1 || !m->Wq.p || !m->Wgate.p || !m->exp || !m->exp[0].p) {
        fprintf(stderr, "v4: layer %d is incomplete\n", layer);
        return -4;
    }
    i = tensor_index(f, "expert.%d.0.Wg", layer, 0);
    m->d_exp = i >= 0 ? (int)T_(i)->dims[0] : 0;
    if (!m->d_exp) { fprintf(stderr, "v4: cannot determine d_exp for layer %d\n", layer); return -5; }
#undef T_
#undef ENC_
#undef REG_
    return 0;
}

int qwen3_load_v4(QW3Layer *m, const char *path, int layer) {
    const int rc = qwen3_map(m, path);
    return rc ? rc : qwen3_bind_layer(m, layer);
}

void qwen3_layer_free_weights(QW3Layer *m) {
    qw3_state *st = m->exp_owned ? qw3_state_of(m->map) : NULL;
    if (m->exp_owned) {
        free(m->exp);
        free(m->reg_exp);
        free(m->tensor_reg);
        free(m->reg_embed_chunk);
        free((void *)m->embed_chunk_ptr);
        m->reg_exp = NULL;
        m->tensor_reg = NULL;
        m->reg_embed_chunk = NULL;
        m->embed_chunk_ptr = NULL;
    }
    m->exp = NULL;
    m->exp_owned = 0;
    if (st) {                   /* the struct qwen3_map filled owns the mapping */
        state_release(st);
        m->map = NULL;
        m->map_len = 0;
    }
}

/* ------------------------------------------------------------------ the device form of a layer */

int qw3_dev_layer_get(qw3_state *st, int layer, qw3_dev_layer **out) {
    if (layer < 0 || layer >= st->n_layers) { fprintf(stderr, "qwen3: layer %d is not bound\n", layer); return -1; }
    qw3_dev_layer *L = &st->lay[layer];
    *out = L;
    if (L->ready) return 0;
    const cpw4_file *f = &st->f;
    const int iln1 = tensor_index(f, "ln1.%d", layer, 0), iln2 = tensor_index(f, "ln2.%d", layer, 0);
    const int iqn = tensor_index(f, "q_norm.%d", layer, 0), ikn = tensor_index(f, "k_norm.%d", layer, 0);
    const int iq = tensor_index(f, "Wq.%d", layer, 0), ik = tensor_index(f, "Wk.%d", layer, 0);
    const int iv = tensor_index(f, "Wv.%d", layer, 0), io = tensor_index(f, "Wo.%d", layer, 0);
    const int ig = tensor_index(f, "Wgate.%d", layer, 0), ie0 = tensor_index(f, "expert.%d.%d.Wg", layer, 0);
    if (iln1 < 0 || iln2 < 0 || iqn < 0 || ikn < 0 || iq < 0 || ik < 0 || iv < 0 || io < 0 ||
        ig < 0 || ie0 < 0) {
        fprintf(stderr, "v4: layer %d is incomplete\n", layer);
        return -4;
    }
#define ENC_(i) (f->enc[f->tensors[i].enc].code)
    const int D = (int)f->tensors[iln1].dims[0], HD = (int)f->tensors[iqn].dims[0];
    const int H = (int)f->tensors[iq].dims[0] / HD, KV = (int)f->tensors[ik].dims[0] / HD;
    const int E = (int)f->tensors[ig].dims[0], F = (int)f->tensors[ie0].dims[0];
    const int ea = ENC_(iq), ee = ENC_(ie0);
    if ((ea != QW3_ENC_Q4 && ea != QW3_ENC_Q8) || ENC_(ik) != ea || ENC_(iv) != ea || ENC_(io) != ea ||
        (ee != QW3_ENC_Q4 && ee != QW3_ENC_Q8) || ENC_(ig) != QW3_ENC_F32 || ENC_(iln1) != QW3_ENC_F32 ||
        ENC_(iln2) != QW3_ENC_F32 || ENC_(iqn) != QW3_ENC_F32 || ENC_(ikn) != QW3_ENC_F32) {
        fprintf(stderr, "qwen3: layer %d: the device path takes Q4_0/Q8_0 projections and experts "
                        "with f32 norms and router\n", layer);
        return -1;
    }
    const int nqkv = (H + 2 * KV) * HD;
    const size_t qb = (size_t)H * HD * D / 32 * (ea == QW3_ENC_Q8 ? 34 : 18);
    const size_t kb = (size_t)KV * HD * D / 32 * (ea == QW3_ENC_Q8 ? 34 : 18);
    uint8_t *stage = cpg_malloc(qb + 2 * kb);
    L->wqkv = cpg_malloc(cpg_matrix_bytes(ea, nqkv, D));
    L->wo = cpg_malloc(cpg_matrix_bytes(ea, D, H * HD));
    const size_t eb = cpg_expert_bytes(ee, D, F), mg = cpg_matrix_bytes(ee, F, D);
    L->experts = cpg_malloc(eb * (size_t)E);
    int rc = 0;
    if (!stage || !L->wqkv || !L->wo || !L->experts) { rc = -2; fprintf(stderr, "qwen3: %s\n", cpg_last_error()); goto done; }
    if (cpg_d2d(stage, qw3_dev_ptr(st, cpw4_data(f, iq)), qb) ||
        cpg_d2d(stage + qb, qw3_dev_ptr(st, cpw4_data(f, ik)), kb) ||
        cpg_d2d(stage + qb + kb, qw3_dev_ptr(st, cpw4_data(f, iv)), kb) ||
        cpg_repack(ea, L->wqkv, stage, nqkv, D) ||
        cpg_repack(ea, L->wo, qw3_dev_ptr(st, cpw4_data(f, io)), D, H * HD)) {
        rc = dev_err("attention weights");
        goto done;
    }
    for (int e = 0; e < E && !rc; e++) {
        static const char *kinds[3] = {"expert.%d.%d.Wg", "expert.%d.%d.Wu", "expert.%d.%d.Wd"};
        for (int k = 0; k < 3 && !rc; k++) {
            const int t = tensor_index(f, kinds[k], layer, e);
            if (t < 0 || ENC_(t) != ee) { fprintf(stderr, "v4: layer %d expert %d is incomplete\n", layer, e); rc = -4; break; }
            const int rows = k == 2 ? D : F, cols = k == 2 ? F : D;
            if (cpg_repack(ee, (uint8_t *)L->experts + (size_t)e * eb + (size_t)k * mg,
                           qw3_dev_ptr(st, cpw4_data(f, t)), rows, cols))
                rc = dev_err("expert weights");
        }
    }
    if (!rc && cpg_sync()) rc = dev_err("layer upload");
    if (!rc) {
        L->a = (cpg_attn_layer){D, H, KV, HD, st->theta, st->eps, ea,
                                (const float *)qw3_dev_ptr(st, cpw4_data(f, iln1)),
                                (const float *)qw3_dev_ptr(st, cpw4_data(f, iqn)),
                                (const float *)qw3_dev_ptr(st, cpw4_data(f, ikn)), L->wqkv, L->wo,
                                st->rope, QW3_MAX_POS};
        L->m = (cpg_moe_layer){D, E, st->topk, F, ee, st->eps,
                               (const float *)qw3_dev_ptr(st, cpw4_data(f, iln2)),
                               (const float *)qw3_dev_ptr(st, cpw4_data(f, ig)), L->experts};
        L->ready = 1;
    }
#undef ENC_
done:
    cpg_free(stage);
    if (rc) {
        cpg_free(L->wqkv);
        cpg_free(L->wo);
        cpg_free(L->experts);
        memset(L, 0, sizeof *L);
    }
    return rc;
}

int qw3_scratch(qw3_state *st, int T) {
    if (T <= st->cap_T) return 0;
    const qw3_dev_layer *L = NULL;
    for (int l = 0; l < st->n_layers && !L; l++)
        if (st->lay[l].ready) L = &st->lay[l];
    if (!L) return -1;
    const int D = L->a.D, E = L->m.E, K = L->m.K;
    cpg_free(st->dx); cpg_free(st->dattn); cpg_free(st->dmlp); cpg_free(st->drouter); cpg_free(st->dtopk);
    cpg_moe_ws_destroy(st->mws);
    cpg_attn_ws_destroy(st->aws);
    st->dx = cpg_malloc(sizeof(float) * (size_t)T * D);
    st->dattn = cpg_malloc(sizeof(float) * (size_t)T * D);
    st->dmlp = cpg_malloc(sizeof(float) * (size_t)T * D);
    st->drouter = cpg_malloc(sizeof(float) * (size_t)T * E);
    st->dtopk = cpg_malloc(sizeof(int) * (size_t)T * K);
    st->mws = cpg_moe_ws_create(D, E, K, L->m.F, T);
    st->aws = cpg_attn_ws_create(D, L->a.H, L->a.KV, L->a.HD, T);
    if (!st->dx || !st->dattn || !st->dmlp || !st->drouter || !st->dtopk || !st->mws || !st->aws) {
        fprintf(stderr, "qwen3: scratch for %d tokens: %s\n", T, cpg_last_error());
        st->cap_T = 0;
        return -2;
    }
    st->cap_T = T;
    return 0;
}

/* ------------------------------------------------------------------ forward */

int qwen3_layer(const QW3Layer *m, const float *x, int T, QW3Out *o) {
    QW3KV tmp;
    if (qwen3_kv_alloc(&tmp, m, T)) return -1;
    const int rc = qwen3_layer_kv(m, x, T, 0, &tmp, o);
    qwen3_kv_free(&tmp);
    return rc;
}

int qwen3_layer_kv(const QW3Layer *m, const float *x, int T, int pos0, QW3KV *cache, QW3Out *o) {
    if (!cache || pos0 < 0 || T <= 0 || pos0 + T > cache->cap) {
        fprintf(stderr, "qwen3: kv range %d+%d outside cache cap %d\n", pos0, T, cache ? cache->cap : 0);
        return -1;
    }
    qw3_state *st = qw3_state_of(m->map);
    if (!st) { fprintf(stderr, "qwen3: layer was not mapped by qwen3_map\n"); return -1; }
    qw3_dev_layer *L;
    int rc = qw3_dev_layer_get(st, m->cur_layer, &L);
    if (rc) return rc;
    if (pos0 + T > QW3_MAX_POS) { fprintf(stderr, "qwen3: position %d beyond %d\n", pos0 + T, QW3_MAX_POS); return -1; }
    const int D = L->a.D, E = L->m.E, K = L->m.K;
    const int ch = T < QW3_CHUNK_T ? T : QW3_CHUNK_T;
    if ((rc = qw3_scratch(st, ch))) return rc;
    for (int t0 = 0; t0 < T; t0 += ch) {
        const int n = T - t0 < ch ? T - t0 : ch;
        const size_t dn = sizeof(float) * (size_t)n * D;
        if (cpg_h2d(st->dx, x + (size_t)t0 * D, dn) ||
            cpg_attn_forward(&L->a, st->dx, n, pos0 + t0, cache->k, cache->v, cache->cap,
                             st->dattn, st->aws) ||
            cpg_h2d(st->dmlp, o->mlp + (size_t)t0 * D, dn) ||
            cpg_moe_forward(&L->m, st->dx, st->dattn, n, NULL, st->drouter, st->dtopk, NULL,
                            st->dmlp, st->mws) ||
            cpg_d2h(o->attn + (size_t)t0 * D, st->dattn, dn) ||
            cpg_d2h(o->mlp + (size_t)t0 * D, st->dmlp, dn) ||
            cpg_d2h(o->router + (size_t)t0 * E, st->drouter, sizeof(float) * (size_t)n * E) ||
            cpg_d2h(o->topk_idx + (size_t)t0 * K, st->dtopk, sizeof(int) * (size_t)n * K))
            return dev_err("layer forward");
    }
    return 0;
}

void qwen3_mm(const QW3T *t, float *out, const float *x, int n_in, int n_out) {
    const size_t row = t->enc == QW3_ENC_F32 ? sizeof(float) * (size_t)n_in
                     : (size_t)n_in / 32 * (t->enc == QW3_ENC_Q8 ? 34 : 18);
    const void *w = NULL;
    void *tmp = NULL;
    float *xd = NULL, *od = NULL;
    int ok = qw3_ensure_device() == 0;
    for (int i = 0; ok && i < QW3_MAX_MAPS && !w; i++)
        if (g_maps[i].used) w = qw3_dev_ptr(&g_maps[i], t->p);
    if (ok && !w) {             /* a tensor outside every mapped file: bring it over */
        tmp = cpg_malloc(row * (size_t)n_out);
        ok = tmp && cpg_h2d(tmp, t->p, row * (size_t)n_out) == 0;
        w = tmp;
    }
    if (ok) {
        xd = cpg_malloc(sizeof(float) * (size_t)n_in);
        od = cpg_malloc(sizeof(float) * (size_t)n_out);
        ok = xd && od && cpg_h2d(xd, x, sizeof(float) * (size_t)n_in) == 0 &&
             cpg_mm(t->enc, w, xd, n_in, n_out, od) == 0 &&
             cpg_d2h(out, od, sizeof(float) * (size_t)n_out) == 0;
    }
    if (!ok) {                  /* the reference's signature has no error channel */
        fprintf(stderr, "qwen3_mm: %s\n", cpg_last_error());
        for (int i = 0; i < n_out; i++) out[i] = NAN;
    }
    cpg_free(tmp);
    cpg_free(xd);
    cpg_free(od);
}

/* qwen3_moe.c:234-286: the flat blob (eight ints D, H, KV, HD, F, E, K, V; theta and eps; then
   every tensor f32 in a fixed order). Loaded into host memory as the reference does; its f32
   weights are served by qwen3_mm, while qwen3_layer's device path takes Q4_0/Q8_0 v4 files. */
int qwen3_load_blob(QW3Layer *m, const char *path, float **owned) {
    memset(m, 0, sizeof *m);
    FILE *fp = fopen(path, "rb");
    if (!fp) { perror(path); return -1; }
    int h[8];
    float fl[2];
    if (fread(h, sizeof(int), 8, fp) != 8 || fread(fl, sizeof(float), 2, fp) != 2) { fclose(fp); return -1; }
    m->d_model = h[0]; m->n_heads = h[1]; m->n_kv = h[2]; m->head_dim = h[3];
    m->d_exp = h[4]; m->n_experts = h[5]; m->topk = h[6]; m->vocab = h[7];
    m->rope_theta = fl[0];
    m->rms_eps = fl[1];
    const long D = m->d_model, H = m->n_heads, KV = m->n_kv, HD = m->head_dim, E = m->n_experts, F = m->d_exp;
    const long total = 2 * D + 2 * HD + H * HD * D + 2 * KV * HD * D + D * H * HD + E * D + 3 * E * F * D;
    if (D <= 0 || HD <= 0 || E <= 0 || F <= 0 || total <= 0) { fclose(fp); return -1; }
    float *buf = malloc(sizeof(float) * (size_t)total);
    if (!buf) { fclose(fp); return -2; }
    if (fread(buf, sizeof(float), (size_t)total, fp) != (size_t)total) { free(buf); fclose(fp); return -1; }
    fclose(fp);
    *owned = buf;
    float *p = buf;
    m->ln1 = p; p += D;
    m->ln2 = p; p += D;
    m->q_norm = p; p += HD;
    m->k_norm = p; p += HD;
    m->Wq.p = p; p += H * HD * D;
    m->Wk.p = p; p += KV * HD * D;
    m->Wv.p = p; p += KV * HD * D;
    m->Wo.p = p; p += D * H * HD;
    m->Wgate.p = p; p += E * D;
    m->Wq.enc = m->Wk.enc = m->Wv.enc = m->Wo.enc = m->Wgate.enc = QW3_ENC_F32;
    m->exp = calloc((size_t)E * 3, sizeof(QW3T));
    if (!m->exp) { free(buf); *owned = NULL; return -2; }
    m->exp_owned = 1;
    const float *wg = p, *wu = p + E * F * D, *wd = p + 2 * E * F * D;
    for (long e = 0; e < E; e++) {
        m->exp[e * 3 + 0] = (QW3T){wg + e * F * D, QW3_ENC_F32};
        m->exp[e * 3 + 1] = (QW3T){wu + e * F * D, QW3_ENC_F32};
        m->exp[e * 3 + 2] = (QW3T){wd + e * D * F, QW3_ENC_F32};
    }
    return 0;
}
