/* cachepotato.c — the public API (cachepotato.h) over the device-resident Qwen3 engine.
 *
 * The reference's API (engine/api/cachepotato.c:205-378) runs its forward on the CPU with the
 * weights paged from disk. Here cp_open uploads the CPW1 v4 payload to HBM once (qwen3_map_ex)
 * and builds every layer's device form (qw3_dev_layer_get), and a token is computed without
 * a host round trip: the embedding row is gathered by the device from the token id the
 * previous step's argmax left in device memory, every layer's attention half, MoE half and
 * residual run on the context's stream, and the head's argmax writes the next id. The host
 * only enqueues. The flow per token is the reference eval driver's
 * (tools/qwen3_eval.c:155-195, :338-400):
 *   embed_rows -> for each layer: x += attn + mlp -> rmsnorm(final_norm) -> lm_head -> argmax
 * A decode step (about 440 kernels) is captured once as a HIP graph and replayed: the position
 * and the step index live in device memory and advance at the end of each replay.
 */
#define _GNU_SOURCE
#include "cachepotato.h"
#include "cptok.h"
#include "qw3_engine.h"

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#define CP_DEFAULT_CTX 2048      /* cachepotato.c:29 */
#define CP_PREFILL_CHUNK 512     /* prompt tokens per device pass */
#define CP_EV_BASE 2048          /* event slots of the per-step timing */
#define CP_EV_MAX 2000
#define CP_IM_END 151645         /* <|im_end|>, the end of an assistant turn (cachepotato.c:27) */
#define CP_TOK_FILE "qwen2.5-tokenizer.bin"      /* cachepotato.c:29-30 */
#define CP_UNI_FILE "qwen2.5-unicode.bin"

struct cp_model {
    QW3Layer base;
    qw3_state *st;
    int L, D, V, E, K, max_ctx, hist, has_ids;
    long long file_bytes;
    /* device */
    const void *embed;          /* v4-layout table, V rows (contiguous) */
    void *embed_owned;          /* a contiguous copy when the file's chunks are not adjacent */
    int embed_enc;
    void *head;                 /* lm_head: row-tiled (head_tiled) or the file's v4 rows */
    int head_enc, head_tiled;
    const float *final_norm;
    QW3KV *kv;
    float *x, *attn, *mlp, *xf, *logits;
    int *tok_cur;               /* the token the last argmax chose */
    int *tok_hist;              /* [CP_EV_MAX] the decoded tokens */
    int *state;                 /* {position of the next token, step index} */
    int *topk_l;                /* [L][K] the experts of the current token, per layer */
    int *ids;                   /* [max_ctx] prompt ids */
    int *route;                 /* [L][route_cap] x K, or NULL */
    void *head_scratch;         /* cpg_head_next's per-tile candidates and counter (zeroed) */
    size_t route_cap;
    int use_graph;
    cpt_tokenizer *tk;          /* NULL when no tokenizer files were found: cp_chat -> -2 */
    int *turn_ids;              /* host: the current chat fragment's ids */
    cpg_graph *layers_graph;    /* cp_chat: every layer at state[0], then the step end */
    int head_fused;             /* cpg_head_next for the head (CP_HEAD_SEPARATE=1: three kernels) */
    cpg_moe_ws *mws;
    cpg_attn_ws *aws;
};

static int g_open;               /* one model at a time (cachepotato.c:45) */

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static void set_err(char *err, size_t n, const char *fmt, ...) {
    if (!err || !n) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, n, fmt, ap);
    va_end(ap);
}

/* ---------------------------------------------------------------- machine probes
 * The public API's three probes (engine/api/cachepotato.h:88-90, behaviour of
 * engine/api/cachepotato.c:59-106) keep their meaning: cores are distinct (package, core)
 * pairs, memory is the kernel's MemAvailable, and the automatic pager budget is that memory
 * less 2 GiB of headroom, capped at the file's size and refused below 2 GiB. The device path
 * depends on none of them (the weights live in HBM and no CPU thread runs the forward); they
 * are here so that callers of the public API keep working. */

/* a non-negative integer held in a small text file (sysfs), or -1 */
static long read_small_long(const char *path) {
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    char buf[32] = {0};
    const size_t n = fread(buf, 1, sizeof buf - 1, f);
    fclose(f);
    if (n == 0) return -1;
    char *end;
    const long v = strtol(buf, &end, 10);
    return end == buf || v < 0 ? -1 : v;
}

static int cmp_u64(const void *a, const void *b) {
    const uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : x > y;
}

int cp_physical_cores(void) {
    /* The kernel's topology directory names, for every logical CPU present, its package and
       core; the hyperthreads of one core share both. Each pair becomes one 64-bit key, and
       the distinct keys are counted after a sort. */
    const long ncpu = sysconf(_SC_NPROCESSORS_CONF);
    int cores = 0;
    uint64_t *key = ncpu > 0 ? malloc(sizeof(uint64_t) * (size_t)ncpu) : NULL;
    if (key) {
        int nk = 0;
        for (long c = 0; c < ncpu; c++) {
            char path[96];
            snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%ld/topology/physical_package_id", c);
            const long pkg = read_small_long(path);
            snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%ld/topology/core_id", c);
            const long core = read_small_long(path);
            if (pkg >= 0 && core >= 0)        /* an offline CPU has no topology */
                key[nk++] = (uint64_t)pkg << 32 | (uint64_t)(uint32_t)core;
        }
        qsort(key, (size_t)nk, sizeof *key, cmp_u64);
        for (int i = 0; i < nk; i++) cores += i == 0 || key[i] != key[i - 1];
        free(key);
    }
    if (cores > 0) return cores;
    const long online = sysconf(_SC_NPROCESSORS_ONLN);
    return online > 0 ? (int)online : 1;
}

long cp_mem_available_mb(void) {
    FILE *f = fopen("/proc/meminfo", "r");
    if (!f) return -1;
    static const char key[] = "MemAvailable:";
    char line[160];
    long mb = -1;
    while (mb < 0 && fgets(line, sizeof line, f)) {
        if (strncmp(line, key, sizeof key - 1) != 0) continue;
        char *end;
        const long kib = strtol(line + sizeof key - 1, &end, 10);
        if (end != line + sizeof key - 1 && kib >= 0) mb = kib / 1024;
    }
    fclose(f);
    return mb;
}

long cp_auto_budget_mb(long long model_file_bytes) {
    enum { HEADROOM_MB = 2048, FLOOR_MB = 2048 };   /* KV cache, activations, the desktop */
    const long avail = cp_mem_available_mb();
    if (avail < 0) return -1;
    long budget = avail - HEADROOM_MB;
    if (model_file_bytes > 0) {                       /* never more than the whole file */
        const long whole = (long)(model_file_bytes >> 20) + 1;
        if (whole < budget) budget = whole;
    }
    return budget >= FLOOR_MB ? budget : -1;
}

void cp_options_default(cp_options *opt) {
    memset(opt, 0, sizeof *opt);
    opt->budget_mb = CP_BUDGET_AUTO;
    opt->pin_cores = -1;
}

/* ---------------------------------------------------------------- open / close */

static size_t v4_row_bytes(int enc, int D) {
    return enc == QW3_ENC_F32 ? sizeof(float) * (size_t)D
                              : (size_t)D / 32 * (enc == QW3_ENC_Q8 ? 34 : 18);
}

/* the embedding table as one contiguous device array of V rows */
static int setup_embed(cp_model *m) {
    const QW3Layer *b = &m->base;
    const size_t row = v4_row_bytes(b->embed.enc, m->D);
    m->embed_enc = b->embed.enc;
    if (b->embed.p) {
        m->embed = qw3_dev_ptr(m->st, b->embed.p);
        return m->embed ? 0 : -1;
    }
    if (b->embed_chunks <= 0 || b->embed_rows <= 0) return -1;
    /* chunks of embed_rows rows (convert.py:166-181); adjacent in the payload in the
       converter's files, copied together otherwise */
    const uint8_t *p0 = qw3_dev_ptr(m->st, b->embed_chunk_ptr[0]);
    int adjacent = p0 != NULL;
    for (int c = 1; c < b->embed_chunks && adjacent; c++)
        adjacent = qw3_dev_ptr(m->st, b->embed_chunk_ptr[c]) ==
                   p0 + (size_t)c * b->embed_rows * row;
    if (adjacent) { m->embed = p0; return 0; }
    uint8_t *dst = cpg_malloc(row * (size_t)m->V);
    if (!dst) return -2;
    m->embed_owned = dst;
    for (int c = 0; c < b->embed_chunks; c++) {
        const int r0 = c * b->embed_rows;
        const int n = r0 + b->embed_rows <= m->V ? b->embed_rows : m->V - r0;
        if (n <= 0) break;
        if (cpg_d2d(dst + (size_t)r0 * row, qw3_dev_ptr(m->st, b->embed_chunk_ptr[c]),
                    (size_t)n * row))
            return -7;
    }
    m->embed = dst;
    return 0;
}

/* the head: row-tiled for the tiled GEMV when its shape allows, else the file's rows */
static int setup_head(cp_model *m) {
    const QW3Layer *b = &m->base;
    const void *src = qw3_dev_ptr(m->st, b->lm_head.p);
    if (!src) return -1;
    m->head_enc = b->lm_head.enc;
    if ((m->head_enc == QW3_ENC_Q4 || m->head_enc == QW3_ENC_Q8) && m->V % 64 == 0 &&
        m->D % 32 == 0 && m->D <= 4096) {
        m->head = cpg_malloc(cpg_matrix_bytes(m->head_enc, m->V, m->D));
        if (!m->head) return -2;
        if (cpg_repack(m->head_enc, m->head, src, m->V, m->D)) return -7;
        m->head_tiled = 1;
        return 0;
    }
    m->head = (void *)src;
    m->head_tiled = 0;
    return 0;
}

/* ---------------------------------------------------------------- the tokenizer
 * Found as the reference finds it (cachepotato.c:180-200): in opt.tokenizer_dir when given,
 * else in the model's directory's tokenizer/ folder, the model's directory, or ./weights. A
 * model opened without them still serves the id-level entry points; cp_chat then returns -2
 * (the reference's cp_open refuses such a model instead). */

static int file_exists(const char *p) {
    struct stat sb;
    return stat(p, &sb) == 0 && S_ISREG(sb.st_mode);
}

static int tokenizer_dir_ok(const char *dir, char *vocab, char *uni, size_t n) {
    return snprintf(vocab, n, "%s/" CP_TOK_FILE, dir) < (int)n &&
           snprintf(uni, n, "%s/" CP_UNI_FILE, dir) < (int)n && file_exists(vocab) &&
           file_exists(uni);
}

/* 0 with the tokenizer loaded, 1 when none was found (and none was asked for), -1 on error */
static int open_tokenizer(cp_model *m, const char *model_path, const char *dir, char *err,
                          size_t errlen) {
    char vocab[4352], uni[4352], mdir[4096];
    if (dir) {
        if (!tokenizer_dir_ok(dir, vocab, uni, sizeof vocab)) {
            set_err(err, errlen, "tokenizer files (" CP_TOK_FILE ", " CP_UNI_FILE ") not found in %s", dir);
            return -1;
        }
    } else {
        snprintf(mdir, sizeof mdir, "%s", model_path);
        char *slash = strrchr(mdir, '/');
        if (slash) *slash = 0; else snprintf(mdir, sizeof mdir, ".");
        char cand[3][4224];
        snprintf(cand[0], sizeof cand[0], "%s/tokenizer", mdir);
        snprintf(cand[1], sizeof cand[1], "%s", mdir);
        snprintf(cand[2], sizeof cand[2], "weights");
        int found = 0;
        for (int i = 0; i < 3 && !found; i++) found = tokenizer_dir_ok(cand[i], vocab, uni, sizeof vocab);
        if (!found) return 1;
    }
    char why[256] = {0};
    m->tk = cpt_load(vocab, uni, why, sizeof why);
    if (!m->tk) { set_err(err, errlen, "cannot load tokenizer: %s", why); return -1; }
    return 0;
}

cp_model *cp_open(const char *model_path, const cp_options *opt_in, char *err, size_t errlen) {
    cp_options opt;
    if (opt_in) opt = *opt_in; else cp_options_default(&opt);
    if (g_open) { set_err(err, errlen, "one model per process: a model is already open"); return NULL; }
    struct stat sb;
    if (!model_path || stat(model_path, &sb) != 0) {
        set_err(err, errlen, "cannot open model file %s", model_path ? model_path : "(null)");
        return NULL;
    }
    if (qw3_ensure_device()) { set_err(err, errlen, "no usable GPU: %s", cpg_last_error()); return NULL; }
    cp_model *m = calloc(1, sizeof *m);
    if (!m) { set_err(err, errlen, "out of memory"); return NULL; }
    g_open = 1;
    m->file_bytes = (long long)sb.st_size;
    m->max_ctx = opt.max_ctx > 0 ? opt.max_ctx : CP_DEFAULT_CTX;
    QW3Layer *b = &m->base;
    int rc;
    if (m->max_ctx > QW3_MAX_POS) {
        set_err(err, errlen, "max_ctx %d beyond the %d positions of the RoPE table", m->max_ctx, QW3_MAX_POS);
        goto fail;
    }
    if ((rc = qwen3_map_ex(b, model_path, CP_BUDGET_NONE))) {
        set_err(err, errlen, "cannot map %s (not a CPW1 v4 Qwen3 file?): code %d", model_path, rc);
        goto fail;
    }
    if (qwen3_bind_layer(b, 0)) { set_err(err, errlen, "cannot bind layer 0"); goto fail; }
    m->st = qw3_state_of(b->map);
    m->L = b->n_layers;
    m->D = b->d_model;
    m->V = b->vocab;
    m->E = b->n_experts;
    m->K = b->topk;
    if (m->L <= 0 || !m->st) { set_err(err, errlen, "the file declares no attention blocks"); goto fail; }
    if (open_tokenizer(m, model_path, opt.tokenizer_dir, err, errlen) < 0) goto fail;
    m->turn_ids = malloc(sizeof(int) * (size_t)m->max_ctx);
    if (!m->turn_ids) { set_err(err, errlen, "out of memory"); goto fail; }
    if ((!b->embed.p && b->embed_chunks == 0) || !b->lm_head.p || !b->final_norm) {
        set_err(err, errlen, "missing embed / lm_head / final_norm");
        goto fail;
    }
    for (int l = 0; l < m->L; l++) {
        qw3_dev_layer *dl;
        if ((rc = qw3_dev_layer_get(m->st, l, &dl))) {
            set_err(err, errlen, "layer %d: device form failed (code %d)", l, rc);
            goto fail;
        }
    }
    if ((rc = setup_embed(m)) || (rc = setup_head(m))) {
        set_err(err, errlen, "embedding / head setup failed (code %d): %s", rc, cpg_last_error());
        goto fail;
    }
    m->final_norm = qw3_dev_ptr(m->st, b->final_norm);
    m->kv = calloc((size_t)m->L, sizeof(QW3KV));
    if (!m->kv || !m->final_norm) { set_err(err, errlen, "out of memory"); goto fail; }
    for (int l = 0; l < m->L; l++)
        if (qwen3_kv_alloc(&m->kv[l], b, m->max_ctx)) {
            set_err(err, errlen, "KV cache allocation failed");
            goto fail;
        }
    const qw3_dev_layer *l0 = &m->st->lay[0];
    const int chunk = m->max_ctx < CP_PREFILL_CHUNK ? m->max_ctx : CP_PREFILL_CHUNK;
    const size_t xd = sizeof(float) * (size_t)chunk * m->D;
    m->x = cpg_malloc(xd);
    m->attn = cpg_malloc(xd);
    m->mlp = cpg_malloc(xd);
    m->xf = cpg_malloc(sizeof(float) * (size_t)m->D);
    m->logits = cpg_malloc(sizeof(float) * (size_t)m->V);
    m->tok_cur = cpg_malloc(sizeof(int));
    m->tok_hist = cpg_malloc(sizeof(int) * CP_EV_MAX);
    m->state = cpg_malloc(sizeof(int) * 2);
    m->topk_l = cpg_malloc(sizeof(int) * (size_t)m->L * m->K);
    m->ids = cpg_malloc(sizeof(int) * (size_t)m->max_ctx);
    m->head_scratch = cpg_malloc(cpg_head_scratch_bytes(m->V));
    m->use_graph = getenv("CP_NO_GRAPH") ? 0 : 1;
    m->head_fused = m->head_tiled && m->D % 256 == 0 && m->D <= 2048 && m->V % 64 == 0 &&
                    !getenv("CP_HEAD_SEPARATE");
    m->mws = cpg_moe_ws_create(m->D, l0->m.E, l0->m.K, l0->m.F, chunk);
    m->aws = cpg_attn_ws_create(m->D, l0->a.H, l0->a.KV, l0->a.HD, chunk);
    if (!m->x || !m->attn || !m->mlp || !m->xf || !m->logits || !m->tok_cur || !m->tok_hist ||
        !m->state || !m->topk_l || !m->ids || !m->mws || !m->head_scratch ||
        !m->aws || cpg_memset(m->mlp, 0, xd) ||
        cpg_memset(m->head_scratch, 0, cpg_head_scratch_bytes(m->V)) || cpg_sync()) {
        set_err(err, errlen, "device scratch: %s", cpg_last_error());
        goto fail;
    }
    return m;
fail:
    cp_close(m);
    return NULL;
}

void cp_close(cp_model *m) {
    if (!m) return;
    if (cpg_current_device() >= 0) {
        cpg_sync();
        if (m->kv)
            for (int l = 0; l < m->L; l++) qwen3_kv_free(&m->kv[l]);
        if (m->head_tiled) cpg_free(m->head);
        cpg_free(m->embed_owned);
        cpg_free(m->x);
        cpg_free(m->attn);
        cpg_free(m->mlp);
        cpg_free(m->xf);
        cpg_free(m->logits);
        cpg_free(m->tok_cur);
        cpg_free(m->tok_hist);
        cpg_free(m->state);
        cpg_free(m->topk_l);
        cpg_free(m->ids);
        cpg_free(m->route);
        cpg_free(m->head_scratch);
        cpg_moe_ws_destroy(m->mws);
        cpg_attn_ws_destroy(m->aws);
    }
    cpg_graph_destroy(m->layers_graph);
    free(m->kv);
    cpt_free(m->tk);
    free(m->turn_ids);
    qwen3_layer_free_weights(&m->base);
    free(m);
    g_open = 0;
}

void cp_reset(cp_model *m) { m->hist = 0; }

void cp_get_stats(const cp_model *m, cp_stats *s) {
    memset(s, 0, sizeof *s);
    s->n_layers = m->L;
    s->d_model = m->D;
    s->n_experts = m->E;
    s->topk = m->K;
    s->vocab = m->V;
    s->max_ctx = m->max_ctx;
    s->threads = 0;
    s->budget_mb = -1;          /* no pager: the model is resident */
    s->file_bytes = m->file_bytes;
    s->resident_bytes = m->file_bytes;
}

/* ---------------------------------------------------------------- the forward */

/* T tokens x (device) at positions pos0.. through every layer (cachepotato.c:149-166:
   x += attn + mlp, attn + mlp summed first). route: n_layers blocks of `stride` ints, this
   call's topk written at the start of each, or NULL. */
static int run_layers(cp_model *m, int T, int pos0, int *route, size_t stride) {
    for (int l = 0; l < m->L; l++) {
        const qw3_dev_layer *dl = &m->st->lay[l];
        QW3KV *kv = &m->kv[l];
        if (cpg_attn_forward(&dl->a, m->x, T, pos0, kv->k, kv->v, kv->cap, m->attn, m->aws) ||
            cpg_moe_forward_res(&dl->m, m->x, m->attn, T,
                                route ? route + (size_t)l * stride : NULL, m->mlp, m->mws))
            return -7;
    }
    return 0;
}

/* the head on hidden row x_row (device): final RMSNorm, lm_head, argmax into *tok_out
   (qwen3_eval.c:183-195, cachepotato.c:355-356) */
static int head_argmax(cp_model *m, const float *x_row, int *tok_out) {
    int rc;
    if (m->head_tiled) {        /* the final RMSNorm folded into the head GEMV */
        rc = cpg_gemv_norm(m->head_enc, m->head, m->D, m->V, x_row, 1, m->final_norm,
                           m->base.rms_eps, m->logits);
    } else {
        rc = cpg_rmsnorm(x_row, m->final_norm, 1, m->D, m->base.rms_eps, m->xf) ||
             cpg_mm(m->head_enc, m->head, m->xf, m->D, m->V, m->logits);
    }
    if (rc) return -7;
    return cpg_argmax(m->logits, m->V, tok_out) ? -7 : 0;
}

/* One decode step, all on the device (qwen3_eval.c:378-390): the head on x (row 0) chooses
   tok_cur, its embedding replaces x, every layer runs at the position held in state[0], and
   the step's token and experts are recorded at state[1]. Nothing here reads a host value
   that changes between steps, so the sequence can be captured once and replayed. */
/* the head on x (row 0), the argmax into tok_cur and that token's embedding row into x: one
   launch where the head is row-tiled and its shape allows, else three */
static int enqueue_head(cp_model *m) {
    if (m->head_fused ? cpg_head_next(m->head_enc, m->head, m->D, m->V, m->x, m->final_norm,
                              m->base.rms_eps, m->logits, m->tok_cur, m->embed_enc, m->embed,
                              m->V, m->head_scratch) != 0
              : (head_argmax(m, m->x, m->tok_cur) ||
                 cpg_embed_rows(m->embed_enc, m->embed, m->V, m->D, m->tok_cur, 1, m->x)))
        return -7;
    return 0;
}

/* every layer on x at the position state[0], then the step's end (record, advance). lim:
   the positions this sequence of steps can reach (below it), at most the cache's rows; the
   attention kernels size their grids to it (split attention: a workgroup per 32 positions) */
static int enqueue_layers(cp_model *m, int *route, int gen, int lim) {
    for (int l = 0; l < m->L; l++) {
        const qw3_dev_layer *dl = &m->st->lay[l];
        QW3KV *kv = &m->kv[l];
        const int cap = lim < kv->cap ? lim : kv->cap;
        if (cpg_attn_forward_at(&dl->a, m->x, 1, m->state, kv->k, kv->v, cap, m->attn,
                                m->aws) ||
            cpg_moe_forward_res(&dl->m, m->x, m->attn, 1, m->topk_l + (size_t)l * m->K, m->mlp,
                                m->mws))
            return -7;
    }
    return cpg_decode_step_end(m->tok_cur, m->tok_hist, m->topk_l, route, m->L, m->K, gen,
                               m->state) ? -7 : 0;
}

static int enqueue_step(cp_model *m, int *route, int gen, int lim) {
    return enqueue_head(m) || enqueue_layers(m, route, gen, lim) ? -7 : 0;
}

int cp_eval_decode(cp_model *m, const int *ids, int T, int gen, int *tokens, int *route,
                   float *step_ms, cp_turn *turn) {
    if (!m || !ids || !tokens || T <= 0 || gen <= 0 || gen > CP_EV_MAX || T + gen > m->max_ctx) {
        fprintf(stderr, "cp_eval_decode: bad arguments (T=%d gen=%d, T+gen <= %d, gen <= %d)\n",
                T, gen, m ? m->max_ctx : 0, CP_EV_MAX);
        return -1;
    }
    cp_turn t;
    memset(&t, 0, sizeof t);
    const int K = m->K, L = m->L, D = m->D;
    if (route && (size_t)gen > m->route_cap) {
        cpg_free(m->route);
        m->route = cpg_malloc(sizeof(int) * (size_t)L * gen * K);
        m->route_cap = m->route ? (size_t)gen : 0;
        if (!m->route) return -7;
    }
    m->hist = 0;
    if (cpg_h2d(m->ids, ids, sizeof(int) * (size_t)T)) return -7;
    /* ---- prefill, in chunks of the workspace size */
    const double t0 = now_s();
    const int chunk = m->max_ctx < CP_PREFILL_CHUNK ? m->max_ctx : CP_PREFILL_CHUNK;
    int last_n = 0;
    for (int p0 = 0; p0 < T; p0 += chunk) {
        const int n = T - p0 < chunk ? T - p0 : chunk;
        if (cpg_embed_rows(m->embed_enc, m->embed, m->V, m->D, m->ids + p0, n, m->x) ||
            run_layers(m, n, p0, NULL, 0))
            return -3;
        last_n = n;
    }
    /* the last prompt position's hidden state becomes row 0, where every step reads it */
    if (last_n > 1 && cpg_d2d(m->x, m->x + (size_t)(last_n - 1) * D, sizeof(float) * D)) return -7;
    const int st0[2] = {T, 0};
    if (cpg_h2d(m->state, st0, sizeof st0) || cpg_sync()) return -7;
    const double t1 = now_s();
    m->hist = T;
    /* ---- decode: one captured step replayed gen times (or enqueued gen times) */
    int *rt = route ? m->route : NULL;
    cpg_graph *g = NULL;
    if (m->use_graph) {
        if (cpg_capture_begin()) return -7;
        const int rc = enqueue_step(m, rt, gen, T + gen);   /* positions T .. T+gen-1 */
        g = cpg_capture_end();
        if (rc || !g) {
            fprintf(stderr, "cp_eval_decode: graph capture failed (%s); enqueueing steps\n",
                    cpg_last_error());
            cpg_graph_destroy(g);
            g = NULL;
            m->use_graph = 0;
        }
    }
    const double t2 = now_s();
    if (cpg_event_record(CP_EV_BASE)) { cpg_graph_destroy(g); return -7; }
    for (int s = 0; s < gen; s++) {
        const int rc = g ? cpg_graph_launch(g) : enqueue_step(m, rt, gen, T + gen);
        if (rc || cpg_event_record(CP_EV_BASE + 1 + s)) { cpg_graph_destroy(g); return -3; }
    }
    const int rs = cpg_sync();
    cpg_graph_destroy(g);
    if (rs) return -7;
    /* a step's position outside the cache leaves NaN in its attention and flags the
       workspace (positions live on the device while the graph replays) */
    const int as = cpg_attn_ws_status(m->aws);
    if (as) {
        fprintf(stderr, "cp_eval_decode: a decode step's position fell outside the KV cache\n");
        return as < 0 ? -7 : -3;
    }
    const double t3 = now_s();
    if (cpg_d2h(tokens, m->tok_hist, sizeof(int) * (size_t)gen)) return -7;
    if (route && cpg_d2h(route, m->route, sizeof(int) * (size_t)L * gen * K)) return -7;
    if (step_ms)
        for (int s = 0; s < gen; s++)
            step_ms[s] = cpg_event_elapsed_ms(CP_EV_BASE + s, CP_EV_BASE + 1 + s);
    m->hist = T + gen;
    m->has_ids = 1;
    t.prompt_tokens = T;
    t.context_tokens = m->hist;
    t.generated_tokens = gen;
    t.prefill_s = t1 - t0;
    t.decode_s = t3 - t2;
    t.stop = CP_STOP_MAX_TOKENS;
    if (turn) *turn = t;
    return 0;
}

int cp_last_logits(const cp_model *m, float *out) {
    if (!m || !out || !m->has_ids) return -1;
    return cpg_d2h(out, m->logits, sizeof(float) * (size_t)m->V) ? -1 : 0;
}

/* ---------------------------------------------------------------- a chat turn
 * engine/api/cachepotato.c:315-378: the user's message wrapped in ChatML (with /no_think, so
 * that the visible budget is not spent in a think block) is APPENDED to the conversation: its
 * tokens are prefilled at the positions after the earlier turns, whose keys and values stay
 * in the cache. The last prefill position gives the first token; then greedily, per token and
 * in the reference's order: stop at <|im_end|> (not fed back), at max_new tokens, or at the
 * end of the context; otherwise hand the token's bytes to the callback, record it, run it
 * through every layer (always, so the cache holds every token hist counts), and stop after
 * that if the callback asked to. The context restarts (context_reset) when fewer than
 * max_new + 64 positions remain.
 *
 * On the device: the fused head (logits, argmax, the next token's embedding row) runs per
 * token, its token is read back (the stop rules and the callback need it on the host), and
 * the layers run as one captured graph that reads the position from device memory. */
static int chat_prefill(cp_model *m, int Tn, int pos0) {
    if (cpg_h2d(m->ids, m->turn_ids, sizeof(int) * (size_t)Tn)) return -7;
    const int chunk = m->max_ctx < CP_PREFILL_CHUNK ? m->max_ctx : CP_PREFILL_CHUNK;
    int last_n = 0;
    for (int p0 = 0; p0 < Tn; p0 += chunk) {
        const int n = Tn - p0 < chunk ? Tn - p0 : chunk;
        if (cpg_embed_rows(m->embed_enc, m->embed, m->V, m->D, m->ids + p0, n, m->x) ||
            run_layers(m, n, pos0 + p0, NULL, 0))
            return -3;
        last_n = n;
    }
    if (last_n > 1 && cpg_d2d(m->x, m->x + (size_t)(last_n - 1) * m->D, sizeof(float) * m->D))
        return -7;
    return 0;
}

int cp_chat(cp_model *m, const char *user_msg, int max_new, cp_token_fn on_token, void *user,
            cp_turn *out) {
    cp_turn t;
    memset(&t, 0, sizeof t);
    if (out) *out = t;
    if (!m || !user_msg) return -1;
    if (!m->tk) {
        fprintf(stderr, "cp_chat: no tokenizer files (" CP_TOK_FILE ", " CP_UNI_FILE ") were "
                        "found for this model; cp_eval_decode takes token ids\n");
        return -2;              /* the reference's tokenizer-failure code (cachepotato.c:338) */
    }
    const int MAX_CTX = m->max_ctx;
    if (m->hist > MAX_CTX - max_new - 64) { m->hist = 0; t.context_reset = 1; }
    const size_t plen = strlen(user_msg) + 128;
    char *prompt = malloc(plen);
    if (!prompt) return -1;
    snprintf(prompt, plen, "<|im_start|>user\n%s /no_think<|im_end|>\n<|im_start|>assistant\n",
             user_msg);
    const int Tn = cpt_encode(m->tk, prompt, m->turn_ids, MAX_CTX - m->hist - 8);
    free(prompt);
    if (Tn <= 0) return -2;
    const int pos0 = m->hist;
    m->hist += Tn;
    t.prompt_tokens = Tn;

    const double t0 = now_s();
    int rc = chat_prefill(m, Tn, pos0);
    if (rc) { if (out) *out = t; return rc == -7 ? -3 : rc; }
    /* the layers' position and a step index beyond any recording (the chat records nothing) */
    const int st0[2] = {m->hist, CP_EV_MAX};
    if (cpg_h2d(m->state, st0, sizeof st0)) return -3;
    const double t1 = now_s();
    if (!m->layers_graph && m->use_graph) {
        if (cpg_capture_begin()) return -3;
        const int crc = enqueue_layers(m, NULL, 1, m->max_ctx);
        m->layers_graph = cpg_capture_end();
        if (crc || !m->layers_graph) {
            cpg_graph_destroy(m->layers_graph);
            m->layers_graph = NULL;
            m->use_graph = 0;
        }
    }
    int pos = m->hist, produced = 0, stop_req = 0;
    t.stop = CP_STOP_EOS;
    const double t2 = now_s();
    for (;;) {
        int best = 0;
        if (enqueue_head(m) || cpg_d2h(&best, m->tok_cur, sizeof best)) { rc = -3; break; }
        if (best == CP_IM_END) { t.stop = CP_STOP_EOS; break; }
        if (produced >= max_new) { t.stop = CP_STOP_MAX_TOKENS; break; }
        if (pos >= MAX_CTX - 1) { t.stop = CP_STOP_CONTEXT; break; }
        const char *bytes;
        size_t len;
        if (on_token && cpt_token_bytes(m->tk, best, &bytes, &len) == 0)
            stop_req = on_token(bytes, len, user);
        if (pos < MAX_CTX - 2) m->hist = pos + 1;
        if (m->layers_graph ? cpg_graph_launch(m->layers_graph)
                            : enqueue_layers(m, NULL, 1, m->max_ctx)) {
            rc = -3;
            break;
        }
        pos++;
        produced++;
        if (stop_req) { t.stop = CP_STOP_CALLER; break; }
    }
    if (cpg_sync() && !rc) rc = -3;
    if (cpg_attn_ws_status(m->aws) && !rc) {
        fprintf(stderr, "cp_chat: a step's position fell outside the KV cache\n");
        rc = -3;
    }
    const double t3 = now_s();
    t.generated_tokens = produced;
    t.context_tokens = m->hist;
    t.prefill_s = t1 - t0;
    t.decode_s = t3 - t2;
    m->has_ids = 1;
    if (out) *out = t;
    return rc;
}
