/* cpw4.c — CPW1 v4 parser and streaming writer (format/SPEC.md §3-§8; byte layout of
 * format/v4_writer.py:183-299). */
#define _GNU_SOURCE
#include "cpw4.h"
#include "qwen3_moe.h"

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ CRC-32 */

/* Table-driven, eight bytes per step ("slicing-by-8"): tab[k][b] is the CRC register after
   byte b followed by k zero bytes, so eight table lookups advance the register by eight
   input bytes. tab[0] is the classic bytewise table. */
static uint32_t crc_tab[8][256];
static int crc_ready;

static void crc_init(void) {
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
        crc_tab[0][i] = c;
    }
    for (uint32_t i = 0; i < 256; i++)
        for (int k = 1; k < 8; k++)
            crc_tab[k][i] = crc_tab[0][crc_tab[k - 1][i] & 0xFFu] ^ (crc_tab[k - 1][i] >> 8);
    crc_ready = 1;
}

uint32_t cpw4_crc32(uint32_t crc, const void *p, size_t n) {
    if (!crc_ready) crc_init();
    const uint8_t *b = (const uint8_t *)p;
    uint32_t c = crc ^ 0xFFFFFFFFu;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        const uint32_t lo = c ^ ((uint32_t)b[i] | (uint32_t)b[i + 1] << 8 |
                                 (uint32_t)b[i + 2] << 16 | (uint32_t)b[i + 3] << 24);
        c = crc_tab[7][lo & 0xFFu] ^ crc_tab[6][(lo >> 8) & 0xFFu] ^
            crc_tab[5][(lo >> 16) & 0xFFu] ^ crc_tab[4][lo >> 24] ^
            crc_tab[3][b[i + 4]] ^ crc_tab[2][b[i + 5]] ^ crc_tab[1][b[i + 6]] ^
            crc_tab[0][b[i + 7]];
    }
    for (; i < n; i++) c = crc_tab[0][(c ^ b[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

/* ------------------------------------------------------------------ reader */

typedef struct {
    const uint8_t *p, *end;
    int bad;
} rd;

static uint64_t rd_n(rd *r, int n) {
    if (r->bad || (size_t)(r->end - r->p) < (size_t)n) { r->bad = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)r->p[i] << (8 * i);
    r->p += n;
    return v;
}
static const uint8_t *rd_skip(rd *r, size_t n) {
    if (r->bad || (size_t)(r->end - r->p) < n) { r->bad = 1; return NULL; }
    const uint8_t *q = r->p;
    r->p += n;
    return q;
}

static int fail(char *err, size_t errlen, const char *fmt, ...) {
    if (err && errlen) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, errlen, fmt, ap);
        va_end(ap);
    }
    return -3;
}

static int cmp_off(const void *a, const void *b) {
    const cpw4_tensor *x = *(const cpw4_tensor *const *)a, *y = *(const cpw4_tensor *const *)b;
    return x->offset < y->offset ? -1 : x->offset > y->offset;
}

void cpw4_release(cpw4_file *f) {
    free(f->tensors);
    free(f->blocks);
    free(f->regions);
    memset(f, 0, sizeof *f);
}

/* format the message first: it may name a tensor whose record the release frees */
#define BAD(...)                          \
    do {                                  \
        fail(err, errlen, __VA_ARGS__);   \
        cpw4_release(f);                  \
        return -3;                        \
    } while (0)

int cpw4_parse(cpw4_file *f, const uint8_t *base, size_t len, char *err, size_t errlen) {
    memset(f, 0, sizeof *f);
    f->base = base;
    f->len = len;
    rd h = {base, base + len, 0};
    const uint32_t magic = (uint32_t)rd_n(&h, 4), version = (uint32_t)rd_n(&h, 4);
    const uint32_t hdr = (uint32_t)rd_n(&h, 4);
    rd_n(&h, 4);                                                      /* flags */
    f->n_tensors = (uint32_t)rd_n(&h, 4);
    f->n_blocks = (uint32_t)rd_n(&h, 4);
    f->n_regions = (uint32_t)rd_n(&h, 4);
    f->n_enc = (uint32_t)rd_n(&h, 4);
    f->off_enc = rd_n(&h, 8);
    f->off_tensors = rd_n(&h, 8);
    f->off_blocks = rd_n(&h, 8);
    f->off_regions = rd_n(&h, 8);
    f->off_data = rd_n(&h, 8);
    uint32_t reserved = 0;
    for (int i = 0; i < 4; i++) reserved |= (uint32_t)rd_n(&h, 4);
    if (h.bad) return fail(err, errlen, "v4: file shorter than its header");
    if (magic != CPW4_MAGIC || version != 4 || hdr != CPW4_HDR_BYTES)
        return fail(err, errlen, "v4: not a CPW4 version-4 file (magic %08x version %u header %u)",
                    magic, version, hdr);
    if (reserved) return fail(err, errlen, "v4: reserved header words are not zero");
    const uint64_t offs[5] = {f->off_enc, f->off_tensors, f->off_blocks, f->off_regions, f->off_data};
    for (int i = 0; i < 5; i++)
        if (offs[i] < CPW4_HDR_BYTES || offs[i] > len)
            return fail(err, errlen, "v4: table offset %llu outside the file", (unsigned long long)offs[i]);
    if (f->n_enc > CPW4_MAX_ENC) return fail(err, errlen, "v4: %u encodings (at most %d)", f->n_enc, CPW4_MAX_ENC);

    /* encodings */
    rd r = {base + f->off_enc, base + len, 0};
    for (uint32_t i = 0; i < f->n_enc; i++) {
        cpw4_enc *e = &f->enc[i];
        rd_n(&r, 4);
        e->kind = (uint8_t)rd_n(&r, 1);
        e->scalar = (uint8_t)rd_n(&r, 1);
        e->group = (uint16_t)rd_n(&r, 2);
        e->block_bytes = (uint16_t)rd_n(&r, 2);
        e->sub = (uint8_t)rd_n(&r, 1);
        e->flags = (uint8_t)rd_n(&r, 1);
        e->align = (uint8_t)rd_n(&r, 1);
        rd_skip(&r, (size_t)rd_n(&r, 2));
        e->code = e->kind == 0 && e->scalar == 0 ? QW3_ENC_F32
                : e->kind == 1 && e->scalar == 3 && e->group == 32 && e->block_bytes == 34 ? QW3_ENC_Q8
                : e->kind == 1 && e->scalar == 4 && e->group == 32 && e->block_bytes == 18 ? QW3_ENC_Q4
                : -1;
    }
    if (r.bad) return fail(err, errlen, "v4: encoding table runs past the file");

    /* tensors */
    f->tensors = calloc(f->n_tensors ? f->n_tensors : 1, sizeof(cpw4_tensor));
    f->blocks = calloc(f->n_blocks ? f->n_blocks : 1, sizeof(cpw4_block));
    f->regions = calloc(f->n_regions ? f->n_regions : 1, sizeof(cpw4_region));
    if (!f->tensors || !f->blocks || !f->regions) { cpw4_release(f); return -2; }
    r = (rd){base + f->off_tensors, base + len, 0};
    if (rd_n(&r, 4) != f->n_tensors) { BAD("v4: tensor count differs from the header"); }
    const uint64_t payload = len - f->off_data;
    for (uint32_t i = 0; i < f->n_tensors && !r.bad; i++) {
        cpw4_tensor *t = &f->tensors[i];
        t->name_len = (uint16_t)rd_n(&r, 2);
        t->name = (const char *)rd_skip(&r, t->name_len);
        t->enc = (uint32_t)rd_n(&r, 4);
        t->rank = (uint32_t)rd_n(&r, 1);
        if (t->rank < 1 || t->rank > 4) { BAD("v4: tensor %u has rank %u", i, t->rank); }
        /* the element count, and below the byte count, must not wrap: a shape whose product
           overflows could otherwise "need" as few bytes as the record claims */
        uint64_t n = 1;
        int wraps = 0;
        for (uint32_t d = 0; d < t->rank; d++) {
            t->dims[d] = (uint32_t)rd_n(&r, 4);
            if (t->dims[d] && n > UINT64_MAX / t->dims[d]) wraps = 1;
            n *= t->dims[d];
        }
        t->offset = rd_n(&r, 8);
        t->length = rd_n(&r, 8);
        t->block = (uint32_t)rd_n(&r, 4);
        t->role = (uint16_t)rd_n(&r, 2);
        if (r.bad) break;
        if (t->enc >= f->n_enc) { BAD("v4: tensor %.*s: encoding index %u", t->name_len, t->name, t->enc); }
        const cpw4_enc *e = &f->enc[t->enc];
        if (t->offset > payload || t->length > payload - t->offset) { BAD("v4: tensor %.*s lies outside the file", t->name_len, t->name); }
        if (t->length && (t->offset % 64 || (e->align > 1 && t->offset % e->align))) { BAD("v4: tensor %.*s is not aligned", t->name_len, t->name); }
        uint64_t want = 0;
        if (e->kind == 0) {
            if (n > UINT64_MAX / 4) wraps = 1;
            want = n * 4;
        } else if (e->group) {
            const uint64_t nb = n / e->group + (n % e->group != 0);
            if (e->block_bytes && nb > UINT64_MAX / e->block_bytes) wraps = 1;
            want = nb * e->block_bytes;
        }
        if (wraps) { BAD("v4: tensor %.*s: its shape's size overflows", t->name_len, t->name); }
        if (e->code >= 0 && t->length != want) { BAD("v4: tensor %.*s holds %llu bytes, its shape needs %llu",
                        t->name_len, t->name, (unsigned long long)t->length, (unsigned long long)want); }
    }
    if (r.bad) { BAD("v4: tensor table runs past the file"); }
    if (f->n_tensors > 1) {                         /* no two tensors share a byte */
        const cpw4_tensor **by = malloc(sizeof(*by) * f->n_tensors);
        if (!by) { cpw4_release(f); return -2; }
        for (uint32_t i = 0; i < f->n_tensors; i++) by[i] = &f->tensors[i];
        qsort(by, f->n_tensors, sizeof(*by), cmp_off);
        for (uint32_t i = 1; i < f->n_tensors; i++)
            if (by[i - 1]->length && by[i]->length && by[i - 1]->offset + by[i - 1]->length > by[i]->offset) {
                free(by);
                BAD("v4: tensors overlap");
            }
        free(by);
    }

    /* blocks; the layer count is the highest attention block's layer + 1 */
    r = (rd){base + f->off_blocks, base + len, 0};
    if (rd_n(&r, 4) != f->n_blocks) { BAD("v4: block count differs from the header"); }
    for (uint32_t i = 0; i < f->n_blocks && !r.bad; i++) {
        cpw4_block *b = &f->blocks[i];
        b->kind = (uint8_t)rd_n(&r, 1);
        b->layer = (uint32_t)rd_n(&r, 4);
        b->n_refs = (uint32_t)rd_n(&r, 1);
        b->refs = rd_skip(&r, 4u * b->n_refs);
        b->n_params = (uint32_t)rd_n(&r, 1);
        b->params = rd_skip(&r, 4u * b->n_params);
        if (r.bad) break;
        for (uint32_t k = 0; k < b->n_refs; k++) {
            const uint32_t ref = (uint32_t)b->refs[4 * k] | (uint32_t)b->refs[4 * k + 1] << 8 |
                                 (uint32_t)b->refs[4 * k + 2] << 16 | (uint32_t)b->refs[4 * k + 3] << 24;
            if (ref >= f->n_tensors) { BAD("v4: block %u refers to tensor %u", i, ref); }
        }
        if (b->kind == CPW4_BLK_ATTN && (int)b->layer + 1 > f->n_layers) f->n_layers = (int)b->layer + 1;
    }
    if (r.bad) { BAD("v4: block table runs past the file"); }

    /* regions */
    r = (rd){base + f->off_regions, base + len, 0};
    if (rd_n(&r, 4) != f->n_regions) { BAD("v4: region count differs from the header"); }
    for (uint32_t i = 0; i < f->n_regions && !r.bad; i++) {
        cpw4_region *g = &f->regions[i];
        g->offset = rd_n(&r, 8);
        g->length = rd_n(&r, 8);
        g->tensor_lo = (uint32_t)rd_n(&r, 4);
        g->tensor_hi = (uint32_t)rd_n(&r, 4);
        g->kind = (uint8_t)rd_n(&r, 1);
        g->slot = (uint16_t)rd_n(&r, 2);
        g->member_lo = (uint32_t)rd_n(&r, 4);
        g->member_hi = (uint32_t)rd_n(&r, 4);
        g->digest = rd_n(&r, 8);
        if (r.bad) break;
        if (g->tensor_lo >= g->tensor_hi || g->tensor_hi > f->n_tensors || g->offset > payload ||
            g->length > payload - g->offset) { BAD("v4: region %u is outside the file or covers no tensor", i); }
    }
    if (r.bad) { BAD("v4: region table runs past the file"); }
    return 0;
}

int cpw4_find(const cpw4_file *f, const char *name) {
    const size_t n = strlen(name);
    for (uint32_t i = 0; i < f->n_tensors; i++)
        if (f->tensors[i].name_len == n && memcmp(f->tensors[i].name, name, n) == 0) return (int)i;
    return -1;
}

/* ------------------------------------------------------------------ Qwen3 geometry */

static int find_fmt(const cpw4_file *f, const char *fmt, int a, int b) {
    char name[96];
    snprintf(name, sizeof name, fmt, a, b);
    return cpw4_find(f, name);
}

/* Tensor i (when present) must have exactly `rank` dims {d0, d1} and an encoding the engine
   decodes; a quantised tensor's rows must be whole 32-element blocks, and f32_only tensors
   (norms, router) must be f32. Returns 0, or -3 with the reason in err. */
static int expect_shape(const cpw4_file *f, int i, int f32_only, uint32_t rank, uint32_t d0,
                        uint32_t d1, char *err, size_t errlen) {
    if (i < 0) return 0;
    const cpw4_tensor *t = &f->tensors[i];
    const int code = f->enc[t->enc].code;
    if (t->rank != rank || t->dims[0] != d0 || (rank == 2 && t->dims[1] != d1))
        return fail(err, errlen, "v4: tensor %.*s has shape [%u%s%u], the model's geometry needs "
                    "[%u%s%u]", t->name_len, t->name, t->dims[0], t->rank > 1 ? ", " : "",
                    t->rank > 1 ? t->dims[1] : 0u, d0, rank > 1 ? ", " : "", rank > 1 ? d1 : 0u);
    if (code < 0 || (f32_only && code != QW3_ENC_F32))
        return fail(err, errlen, "v4: tensor %.*s has an encoding the engine cannot use here",
                    t->name_len, t->name);
    if (code != QW3_ENC_F32 && (t->rank != 2 || t->dims[1] % 32))
        return fail(err, errlen, "v4: quantised tensor %.*s: rows are not whole 32-element blocks",
                    t->name_len, t->name);
    return 0;
}

int cpw4_qwen3_geometry(const cpw4_file *f, cpw4_qwen3_geom *g, char *err, size_t errlen) {
    memset(g, 0, sizeof *g);
    g->n_layers = f->n_layers;
    g->topk = 8;
    if (f->n_layers <= 0) return 0;
    const int iln = find_fmt(f, "ln1.%d", 0, 0), iqn = find_fmt(f, "q_norm.%d", 0, 0);
    const int iq = find_fmt(f, "Wq.%d", 0, 0), ik = find_fmt(f, "Wk.%d", 0, 0);
    const int ig = find_fmt(f, "Wgate.%d", 0, 0), ie = find_fmt(f, "expert.%d.%d.Wg", 0, 0);
    if (iln < 0 || iqn < 0 || iq < 0 || ik < 0 || ig < 0 || ie < 0) {
        fail(err, errlen, "v4: layer 0 lacks ln1, q_norm, Wq, Wk, Wgate or expert 0");
        return -4;
    }
    const cpw4_tensor *T = f->tensors;
    /* the geometry, from layer 0 */
    const uint32_t D = T[iln].dims[0], HD = T[iqn].dims[0];
    if (T[iln].rank != 1 || T[iqn].rank != 1 || T[iq].rank != 2 || T[ik].rank != 2 ||
        T[ig].rank != 2 || T[ie].rank != 2)
        return fail(err, errlen, "v4: layer 0's norms must be vectors and its projections matrices");
    if (D == 0 || D % 32 || D > (1u << 16) || HD == 0 || HD % 2 || HD > D)
        return fail(err, errlen, "v4: hidden size %u / head_dim %u unusable (hidden a positive "
                    "multiple of 32, head_dim even and at most the hidden size)", D, HD);
    if (T[iq].dims[0] % HD || T[ik].dims[0] % HD)
        return fail(err, errlen, "v4: Wq / Wk rows are not whole heads of %u", HD);
    const uint32_t H = T[iq].dims[0] / HD, KV = T[ik].dims[0] / HD;
    const uint32_t E = T[ig].dims[0], F = T[ie].dims[0];
    if (H == 0 || KV == 0 || H % KV || H > 1024)
        return fail(err, errlen, "v4: %u query heads over %u key/value heads", H, KV);
    if (E == 0 || E > 4096 || F == 0 || F % 32 || F > (1u << 16))
        return fail(err, errlen, "v4: %u experts of intermediate size %u", E, F);
    int K = 8;
    for (uint32_t i = 0; i < f->n_blocks; i++) {
        const cpw4_block *b = &f->blocks[i];
        if (b->kind == CPW4_BLK_MOE && b->n_params > 1) {
            const uint8_t *p = b->params + 4;
            K = (int)((uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 |
                      (uint32_t)p[3] << 24);
            if (K < 1 || (uint32_t)K > E)
                return fail(err, errlen, "v4: MoE block of layer %u selects %d of %u experts",
                            b->layer, K, E);
        }
    }
    /* every layer's tensors against it */
    int rc = 0;
    for (int l = 0; l < f->n_layers && !rc; l++) {
        rc = expect_shape(f, find_fmt(f, "ln1.%d", l, 0), 1, 1, D, 0, err, errlen) ||
             expect_shape(f, find_fmt(f, "ln2.%d", l, 0), 1, 1, D, 0, err, errlen) ||
             expect_shape(f, find_fmt(f, "q_norm.%d", l, 0), 1, 1, HD, 0, err, errlen) ||
             expect_shape(f, find_fmt(f, "k_norm.%d", l, 0), 1, 1, HD, 0, err, errlen) ||
             expect_shape(f, find_fmt(f, "Wq.%d", l, 0), 0, 2, H * HD, D, err, errlen) ||
             expect_shape(f, find_fmt(f, "Wk.%d", l, 0), 0, 2, KV * HD, D, err, errlen) ||
             expect_shape(f, find_fmt(f, "Wv.%d", l, 0), 0, 2, KV * HD, D, err, errlen) ||
             expect_shape(f, find_fmt(f, "Wo.%d", l, 0), 0, 2, D, H * HD, err, errlen) ||
             expect_shape(f, find_fmt(f, "Wgate.%d", l, 0), 0, 2, E, D, err, errlen);
        for (uint32_t e = 0; e < E && !rc; e++)
            rc = expect_shape(f, find_fmt(f, "expert.%d.%d.Wg", l, (int)e), 0, 2, F, D, err, errlen) ||
                 expect_shape(f, find_fmt(f, "expert.%d.%d.Wu", l, (int)e), 0, 2, F, D, err, errlen) ||
                 expect_shape(f, find_fmt(f, "expert.%d.%d.Wd", l, (int)e), 0, 2, D, F, err, errlen);
    }
    if (rc) return -3;
    /* model-wide tensors: the head fixes the vocabulary, the embedding must cover it */
    const int ih = cpw4_find(f, "lm_head"), ifn = cpw4_find(f, "final_norm");
    if (ih >= 0 && (T[ih].rank != 2 || T[ih].dims[0] == 0))
        return fail(err, errlen, "v4: lm_head must be a matrix with rows");
    const uint32_t V = ih >= 0 ? T[ih].dims[0] : 0;
    if (expect_shape(f, ih, 0, 2, V, D, err, errlen) ||
        expect_shape(f, ifn, 1, 1, D, 0, err, errlen))
        return -3;
    const int iem = cpw4_find(f, "embed");
    if (iem >= 0) {
        if (T[iem].rank != 2 || T[iem].dims[0] < V ||
            expect_shape(f, iem, 0, 2, T[iem].dims[0], D, err, errlen))
            return fail(err, errlen, "v4: embed must be [>= %u, %u]", V, D);
    } else {
        uint64_t rows = 0;
        uint32_t rows0 = 0;
        for (int c = 0; find_fmt(f, "embed.%d", c, 0) >= 0; c++) {
            const int it = find_fmt(f, "embed.%d", c, 0);
            if (T[it].rank != 2 || (c > 0 && T[it].dims[0] > rows0) ||
                expect_shape(f, it, 0, 2, T[it].dims[0], D, err, errlen))
                return fail(err, errlen, "v4: embedding chunk %d must be [<= %u, %u]", c, rows0, D);
            if (c == 0) rows0 = T[it].dims[0];
            rows += T[it].dims[0];
        }
        if (rows && rows < V)
            return fail(err, errlen, "v4: the embedding chunks hold %llu rows, the head %u",
                        (unsigned long long)rows, V);
    }
    g->d_model = (int)D; g->head_dim = (int)HD; g->n_heads = (int)H; g->n_kv = (int)KV;
    g->n_experts = (int)E; g->d_exp = (int)F; g->topk = K; g->vocab = (int)V;
    return 0;
}

/* ------------------------------------------------------------------ writer */

typedef struct {
    char *name;
    int enc_index, code, rank, role;
    uint32_t dims[4];
    uint64_t nbytes, offset, pad;
} wt_tensor;

typedef struct {
    int kind;
    uint32_t layer;
    int n_refs, n_params;
    uint32_t refs[255], params[255];
} wt_block;

typedef struct {
    int lo, hi, kind, slot;
    uint32_t mlo, mhi;
} wt_region;

struct cpw4_writer {
    wt_tensor *t;
    wt_block *b;
    wt_region *r;
    int nt, nb, nr, ct, cb, cr;
    int enc_code[8];
    int n_enc;
};

cpw4_writer *cpw4_writer_create(void) { return calloc(1, sizeof(cpw4_writer)); }

void cpw4_writer_destroy(cpw4_writer *w) {
    if (!w) return;
    for (int i = 0; i < w->nt; i++) free(w->t[i].name);
    free(w->t);
    free(w->b);
    free(w->r);
    free(w);
}

static int grow(void **p, int *cap, int need, size_t sz) {
    if (need <= *cap) return 0;
    int nc = *cap ? *cap * 2 : 64;
    while (nc < need) nc *= 2;
    void *q = realloc(*p, (size_t)nc * sz);
    if (!q) return -2;
    *p = q;
    *cap = nc;
    return 0;
}

int cpw4_add_tensor(cpw4_writer *w, const char *name, int enc, int rank, const uint32_t *dims,
                    int role) {
    if (enc != QW3_ENC_F32 && enc != QW3_ENC_Q8 && enc != QW3_ENC_Q4) return -1;
    if (rank < 1 || rank > 4 || strlen(name) >= 65535) return -1;
    if (grow((void **)&w->t, &w->ct, w->nt + 1, sizeof(wt_tensor))) return -2;
    wt_tensor *t = &w->t[w->nt];
    memset(t, 0, sizeof *t);
    t->name = strdup(name);
    if (!t->name) return -2;
    int ei = -1;                                    /* encodings in order of first use */
    for (int i = 0; i < w->n_enc; i++)
        if (w->enc_code[i] == enc) ei = i;
    if (ei < 0) { ei = w->n_enc; w->enc_code[w->n_enc++] = enc; }
    t->enc_index = ei;
    t->code = enc;
    t->rank = rank;
    t->role = role;
    uint64_t n = 1;
    for (int d = 0; d < rank; d++) { t->dims[d] = dims[d]; n *= dims[d]; }
    if (enc != QW3_ENC_F32 && n % 32) { free(t->name); return -1; }
    t->nbytes = enc == QW3_ENC_F32 ? n * 4 : n / 32 * (enc == QW3_ENC_Q8 ? 34 : 18);
    return w->nt++;
}

int cpw4_add_block(cpw4_writer *w, int kind, uint32_t layer, const uint32_t *refs, int n_refs,
                   const uint32_t *params, int n_params) {
    if (n_refs < 0 || n_refs > 255 || n_params < 0 || n_params > 255) return -1;
    for (int i = 0; i < n_refs; i++)
        if ((int)refs[i] >= w->nt) return -1;
    if (grow((void **)&w->b, &w->cb, w->nb + 1, sizeof(wt_block))) return -2;
    wt_block *b = &w->b[w->nb];
    b->kind = kind;
    b->layer = layer;
    b->n_refs = n_refs;
    b->n_params = n_params;
    if (n_refs) memcpy(b->refs, refs, sizeof(uint32_t) * (size_t)n_refs);
    if (n_params) memcpy(b->params, params, sizeof(uint32_t) * (size_t)n_params);
    return w->nb++;
}

int cpw4_add_region(cpw4_writer *w, int lo, int hi, int kind, int slot, uint32_t mlo,
                    uint32_t mhi) {
    if (lo < 0 || hi <= lo || hi > w->nt) return -1;
    if (grow((void **)&w->r, &w->cr, w->nr + 1, sizeof(wt_region))) return -2;
    w->r[w->nr] = (wt_region){lo, hi, kind, slot, mlo, mhi};
    return w->nr++;
}

typedef struct {
    uint8_t *b;
    size_t n, cap;
    int oom;
} buf;

static void put(buf *o, uint64_t v, int n) {
    if (o->oom) return;
    if (o->n + (size_t)n > o->cap) {
        size_t nc = o->cap ? o->cap * 2 : 4096;
        while (nc < o->n + (size_t)n) nc *= 2;
        uint8_t *q = realloc(o->b, nc);
        if (!q) { o->oom = 1; return; }
        o->b = q;
        o->cap = nc;
    }
    for (int i = 0; i < n; i++) o->b[o->n++] = (uint8_t)(v >> (8 * i));
}
static void put_str(buf *o, const char *s) {
    const size_t n = strlen(s);
    put(o, n, 2);
    for (size_t i = 0; i < n; i++) put(o, (uint8_t)s[i], 1);
}

int cpw4_write(cpw4_writer *w, const char *path, const int *order, cpw4_fill_fn fill,
               void *user, char *err, size_t errlen) {
    /* physical placement: each tensor padded to 64 bytes, in `order` */
    int *ord = malloc(sizeof(int) * (size_t)(w->nt ? w->nt : 1));
    char *seen = calloc((size_t)(w->nt ? w->nt : 1), 1);
    if (!ord || !seen) { free(ord); free(seen); return -2; }
    for (int i = 0; i < w->nt; i++) {
        ord[i] = order ? order[i] : i;
        if (ord[i] < 0 || ord[i] >= w->nt || seen[ord[i]]) {
            free(ord); free(seen);
            return fail(err, errlen, "v4 writer: the layout is not a permutation of the tensors");
        }
        seen[ord[i]] = 1;
    }
    free(seen);
    uint64_t off = 0;
    for (int k = 0; k < w->nt; k++) {
        wt_tensor *t = &w->t[ord[k]];
        t->offset = off;
        t->pad = (64 - t->nbytes % 64) % 64;
        off += t->nbytes + t->pad;
    }
    static const uint8_t desc[3][7] = {{0, 0, 0, 4, 1, 0, 4}, {1, 3, 32, 34, 1, 3, 64},
                                       {1, 4, 32, 18, 1, 3, 64}};
    static const char *names[3] = {"f32", "Q8_0", "Q4_0"};
    buf enc = {0}, ten = {0}, blk = {0}, reg = {0};
    for (int i = 0; i < w->n_enc; i++) {
        const int d = w->enc_code[i] == QW3_ENC_F32 ? 0 : w->enc_code[i] == QW3_ENC_Q8 ? 1 : 2;
        put(&enc, (uint64_t)i, 4);
        put(&enc, desc[d][0], 1);
        put(&enc, desc[d][1], 1);
        put(&enc, desc[d][2], 2);
        put(&enc, desc[d][3], 2);
        put(&enc, desc[d][4], 1);
        put(&enc, desc[d][5], 1);
        put(&enc, desc[d][6], 1);
        put_str(&enc, names[d]);
    }
    put(&ten, (uint64_t)w->nt, 4);
    for (int i = 0; i < w->nt; i++) {
        const wt_tensor *t = &w->t[i];
        put_str(&ten, t->name);
        put(&ten, (uint64_t)t->enc_index, 4);
        put(&ten, (uint64_t)t->rank, 1);
        for (int d = 0; d < t->rank; d++) put(&ten, t->dims[d], 4);
        put(&ten, t->offset, 8);
        put(&ten, t->nbytes, 8);
        put(&ten, 0xFFFFFFFFu, 4);
        put(&ten, (uint64_t)t->role, 2);
    }
    put(&blk, (uint64_t)w->nb, 4);
    for (int i = 0; i < w->nb; i++) {
        const wt_block *b = &w->b[i];
        put(&blk, (uint64_t)b->kind, 1);
        put(&blk, b->layer, 4);
        put(&blk, (uint64_t)b->n_refs, 1);
        for (int k = 0; k < b->n_refs; k++) put(&blk, b->refs[k], 4);
        put(&blk, (uint64_t)b->n_params, 1);
        for (int k = 0; k < b->n_params; k++) put(&blk, b->params[k], 4);
    }
    put(&reg, (uint64_t)w->nr, 4);
    for (int i = 0; i < w->nr; i++) {            /* digests patched once the payload is known */
        const wt_region *g = &w->r[i];
        const wt_tensor *a = &w->t[g->lo], *z = &w->t[g->hi - 1];
        put(&reg, a->offset, 8);
        put(&reg, z->offset + z->nbytes - a->offset, 8);
        put(&reg, (uint64_t)g->lo, 4);
        put(&reg, (uint64_t)g->hi, 4);
        put(&reg, (uint64_t)g->kind, 1);
        put(&reg, (uint64_t)(uint16_t)g->slot, 2);
        put(&reg, g->mlo, 4);
        put(&reg, g->mhi, 4);
        put(&reg, 0, 8);
    }
    if (enc.oom || ten.oom || blk.oom || reg.oom) {
        free(ord); free(enc.b); free(ten.b); free(blk.b); free(reg.b);
        return -2;
    }
    const uint64_t off_enc = CPW4_HDR_BYTES, off_ten = off_enc + enc.n, off_blk = off_ten + ten.n;
    const uint64_t off_reg = off_blk + blk.n, off_data = (off_reg + reg.n + 63) / 64 * 64;
    buf hb = {0};
    const uint64_t hv[] = {CPW4_MAGIC, 4, CPW4_HDR_BYTES, 0, (uint64_t)w->nt, (uint64_t)w->nb,
                           (uint64_t)w->nr, (uint64_t)w->n_enc};
    for (int i = 0; i < 8; i++) put(&hb, hv[i], 4);
    const uint64_t ho[] = {off_enc, off_ten, off_blk, off_reg, off_data};
    for (int i = 0; i < 5; i++) put(&hb, ho[i], 8);
    for (int i = 0; i < 4; i++) put(&hb, 0, 4);

    int rc = 0;
    FILE *fp = fopen(path, "wb");
    uint64_t maxb = 0;
    for (int i = 0; i < w->nt; i++) maxb = w->t[i].nbytes > maxb ? w->t[i].nbytes : maxb;
    uint8_t *tb = malloc(maxb + 64);
    uint32_t *crc = calloc((size_t)(w->nr ? w->nr : 1), sizeof(uint32_t));
    if (!fp || !tb || !crc || hb.oom) {
        rc = fp ? -2 : fail(err, errlen, "v4 writer: cannot create %s", path);
        goto done;
    }
    static const uint8_t zeros[64];
    if (fwrite(hb.b, 1, hb.n, fp) != hb.n || fwrite(enc.b, 1, enc.n, fp) != enc.n ||
        fwrite(ten.b, 1, ten.n, fp) != ten.n || fwrite(blk.b, 1, blk.n, fp) != blk.n ||
        fwrite(reg.b, 1, reg.n, fp) != reg.n ||
        fwrite(zeros, 1, off_data - (off_reg + reg.n), fp) != off_data - (off_reg + reg.n)) {
        rc = fail(err, errlen, "v4 writer: write failed");
        goto done;
    }
    for (int k = 0; k < w->nt; k++) {
        const int ti = ord[k];
        const wt_tensor *t = &w->t[ti];
        if (fill(user, ti, tb, t->nbytes)) { rc = fail(err, errlen, "v4 writer: no payload for %s", t->name); goto done; }
        memset(tb + t->nbytes, 0, t->pad);
        if (fwrite(tb, 1, t->nbytes + t->pad, fp) != t->nbytes + t->pad) { rc = fail(err, errlen, "v4 writer: write failed"); goto done; }
        /* the digest runs over each covered tensor's payload and padding, in tensor order
           (v4_writer.py:250-252); the tensors of a region are consecutive in the layouts
           this writer is given, so write order is tensor order */
        for (int g = 0; g < w->nr; g++)
            if (ti >= w->r[g].lo && ti < w->r[g].hi)
                crc[g] = cpw4_crc32(crc[g], tb, t->nbytes + t->pad);
    }
    for (int g = 0; g < w->nr; g++) {                /* patch the digests */
        uint8_t d[8];
        for (int i = 0; i < 8; i++) d[i] = (uint8_t)((uint64_t)crc[g] >> (8 * i));
        const long at = (long)(off_reg + 4 + (uint64_t)g * 43 + 35);    /* 43-byte records */
        if (fseek(fp, at, SEEK_SET) || fwrite(d, 1, 8, fp) != 8) { rc = fail(err, errlen, "v4 writer: write failed"); goto done; }
    }
done:
    if (fp && fclose(fp) && !rc) rc = fail(err, errlen, "v4 writer: close failed");
    free(tb); free(crc); free(ord); free(hb.b); free(enc.b); free(ten.b); free(blk.b); free(reg.b);
    return rc;
}

/* map `path`, validate its tables, release: 0, or the parser's code with the reason in err */
int cpw4_check_file(const char *path, char *err, size_t errlen) {
    FILE *fp = fopen(path, "rb");
    if (!fp) return fail(err, errlen, "cannot open %s", path) == -3 ? -1 : -1;
    if (fseek(fp, 0, SEEK_END)) { fclose(fp); return -1; }
    const long n = ftell(fp);
    if (n < 0 || fseek(fp, 0, SEEK_SET)) { fclose(fp); return -1; }
    uint8_t *img = malloc((size_t)n ? (size_t)n : 1);
    if (!img) { fclose(fp); return -2; }
    const size_t got = fread(img, 1, (size_t)n, fp);
    fclose(fp);
    if (got != (size_t)n) { free(img); return -1; }
    cpw4_file f;
    cpw4_qwen3_geom g;
    int rc = cpw4_parse(&f, img, (size_t)n, err, errlen);
    if (rc == 0 && (rc = cpw4_qwen3_geometry(&f, &g, err, errlen)) != 0) cpw4_release(&f);
    if (rc == 0) {
        if (err && errlen) snprintf(err, errlen, "%u tensors, %u blocks, %u regions, %d layers",
                                    f.n_tensors, f.n_blocks, f.n_regions, f.n_layers);
        cpw4_release(&f);
    }
    free(img);
    return rc;
}
