/* tokenizer.c — the Qwen2 byte-level BPE tokenizer behind cp_chat (cptok.h).
 *
 * The files and the rules are the reference's (engine/tokenizers/tokenizer.c,
 * tokenizer_qwen.c); the ids must be identical, so every rule below keeps the reference's
 * behaviour, including its edges: a chunk is cut to its first 512 bytes, bytes that have no
 * single-byte token are dropped, UTF-8 is decoded leniently (a lead byte without enough
 * bytes after it is one code point of its own value, continuation bytes are not checked),
 * and special tokens are tried in id order at the start of each chunk only.
 *
 * Data layout here: the vocabulary in one byte arena with offsets, the merges in an
 * open-addressing hash table keyed by the pair, and BPE on a doubly linked list of symbols
 * with a binary heap of candidate pairs keyed by (rank, position): each step takes the
 * lowest-rank pair and, among equal ranks, the leftmost, which is the reference's order.
 */
#define _GNU_SOURCE
#include "cptok.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CPT_MAGIC 0x31545043u        /* "CPT1" */
#define UNI_MAGIC 0x31494E55u        /* "UNI1" */
#define SPECIAL_FIRST 151643         /* <|endoftext|>: every id from here is a special token */
#define CHUNK_MAX 512                /* bytes of one pre-token chunk that are encoded */

struct cpt_tokenizer {
    int n_vocab;
    uint8_t *arena;                  /* all token bytes */
    uint64_t *off;                   /* [n_vocab + 1] offsets into arena */
    int byte_tok[256];               /* the single-byte token of each byte value, or -1 */
    uint64_t *mkey;                  /* merge table: key (a << 32 | b) + 1, 0 = empty */
    uint32_t *mrank, *mout;
    size_t mmask;
    int *special;                    /* ids >= SPECIAL_FIRST with bytes, ascending */
    int n_special;
    uint32_t *ulo, *uhi;             /* code point ranges and their classes */
    uint8_t *ucls;
    uint32_t n_ranges;
};

/* ---------------------------------------------------------------- file reading */

static uint8_t *slurp(const char *path, size_t *len, char *err, size_t errlen) {
    FILE *f = fopen(path, "rb");
    if (!f) { snprintf(err, errlen, "cannot open %s", path); return NULL; }
    uint8_t *buf = NULL;
    size_t cap = 0, n = 0;
    for (;;) {
        if (n == cap) {
            cap = cap ? cap * 2 : (1 << 20);
            uint8_t *nb = realloc(buf, cap);
            if (!nb) { free(buf); fclose(f); snprintf(err, errlen, "out of memory"); return NULL; }
            buf = nb;
        }
        const size_t got = fread(buf + n, 1, cap - n, f);
        n += got;
        if (got == 0) break;
    }
    fclose(f);
    *len = n;
    return buf;
}

static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

static uint64_t mix(uint64_t k) {              /* splitmix64 finaliser: a hash of the pair */
    k ^= k >> 30; k *= 0xbf58476d1ce4e5b9ull;
    k ^= k >> 27; k *= 0x94d049bb133111ebull;
    return k ^ (k >> 31);
}

/* rank and product of merging (a, b), or -1 */
static long merge_find(const cpt_tokenizer *t, uint32_t a, uint32_t b, uint32_t *out) {
    const uint64_t key = ((uint64_t)a << 32 | b) + 1;
    for (size_t i = mix(key) & t->mmask;; i = (i + 1) & t->mmask) {
        if (t->mkey[i] == 0) return -1;
        if (t->mkey[i] == key) { *out = t->mout[i]; return (long)t->mrank[i]; }
    }
}

static int load_vocab(cpt_tokenizer *t, const uint8_t *p, size_t len, char *err, size_t errlen) {
    if (len < 16 || rd32(p) != CPT_MAGIC || rd32(p + 4) != 1) {
        snprintf(err, errlen, "bad tokenizer file (magic/version)");
        return -1;
    }
    const uint32_t nv = rd32(p + 8), nm = rd32(p + 12);
    if (nv == 0 || nv > (1u << 24)) { snprintf(err, errlen, "bad tokenizer file (%u tokens)", nv); return -1; }
    size_t o = 16, bytes = 0;
    for (uint32_t i = 0; i < nv; i++) {          /* first pass: sizes */
        if (o + 2 > len) goto truncated;
        const size_t l = (size_t)p[o] | (size_t)p[o + 1] << 8;
        if (o + 2 + l > len) goto truncated;
        bytes += l;
        o += 2 + l;
    }
    if (len - o < (size_t)nm * 12) goto truncated;
    t->n_vocab = (int)nv;
    t->arena = malloc(bytes ? bytes : 1);
    t->off = malloc(sizeof(uint64_t) * ((size_t)nv + 1));
    if (!t->arena || !t->off) { snprintf(err, errlen, "out of memory"); return -1; }
    o = 16;
    uint64_t at = 0;
    for (uint32_t i = 0; i < nv; i++) {
        const size_t l = (size_t)p[o] | (size_t)p[o + 1] << 8;
        memcpy(t->arena + at, p + o + 2, l);
        t->off[i] = at;
        at += l;
        o += 2 + l;
    }
    t->off[nv] = at;
    /* a byte's token is the last single-byte token holding it (tokenizer.c:39-42) */
    for (int b = 0; b < 256; b++) t->byte_tok[b] = -1;
    for (uint32_t i = 0; i < nv; i++)
        if (t->off[i + 1] - t->off[i] == 1) t->byte_tok[t->arena[t->off[i]]] = (int)i;
    /* merges: rank = position in the file; a pair listed twice keeps its first rank */
    size_t cap = 16;
    while (cap < (size_t)nm * 2) cap <<= 1;
    t->mmask = cap - 1;
    t->mkey = calloc(cap, sizeof(uint64_t));
    t->mrank = malloc(sizeof(uint32_t) * cap);
    t->mout = malloc(sizeof(uint32_t) * cap);
    if (!t->mkey || !t->mrank || !t->mout) { snprintf(err, errlen, "out of memory"); return -1; }
    for (uint32_t r = 0; r < nm; r++, o += 12) {
        const uint64_t key = ((uint64_t)rd32(p + o) << 32 | rd32(p + o + 4)) + 1;
        size_t i = mix(key) & t->mmask;
        while (t->mkey[i] != 0 && t->mkey[i] != key) i = (i + 1) & t->mmask;
        if (t->mkey[i] == key) continue;
        t->mkey[i] = key;
        t->mrank[i] = r;
        t->mout[i] = rd32(p + o + 8);
    }
    /* the special tokens, in id order */
    t->special = malloc(sizeof(int) * (nv > SPECIAL_FIRST ? nv - SPECIAL_FIRST : 1));
    if (!t->special) { snprintf(err, errlen, "out of memory"); return -1; }
    for (uint32_t i = SPECIAL_FIRST; i < nv; i++)
        if (t->off[i + 1] > t->off[i]) t->special[t->n_special++] = (int)i;
    return 0;
truncated:
    snprintf(err, errlen, "truncated tokenizer file");
    return -1;
}

static int load_unicode(cpt_tokenizer *t, const uint8_t *p, size_t len, char *err, size_t errlen) {
    if (len < 8 || rd32(p) != UNI_MAGIC) { snprintf(err, errlen, "bad unicode table (magic)"); return -1; }
    const uint32_t n = rd32(p + 4);
    if ((len - 8) / 12 < n) { snprintf(err, errlen, "truncated unicode table"); return -1; }
    t->ulo = malloc(sizeof(uint32_t) * (n ? n : 1));
    t->uhi = malloc(sizeof(uint32_t) * (n ? n : 1));
    t->ucls = malloc(n ? n : 1);
    if (!t->ulo || !t->uhi || !t->ucls) { snprintf(err, errlen, "out of memory"); return -1; }
    for (uint32_t i = 0; i < n; i++) {
        t->ulo[i] = rd32(p + 8 + 12 * (size_t)i);
        t->uhi[i] = rd32(p + 12 + 12 * (size_t)i);
        t->ucls[i] = (uint8_t)rd32(p + 16 + 12 * (size_t)i);
    }
    t->n_ranges = n;
    return 0;
}

cpt_tokenizer *cpt_load(const char *vocab_path, const char *unicode_path, char *err,
                        size_t errlen) {
    char dummy[8];
    if (!err || !errlen) { err = dummy; errlen = sizeof dummy; }
    cpt_tokenizer *t = calloc(1, sizeof *t);
    if (!t) { snprintf(err, errlen, "out of memory"); return NULL; }
    size_t lv = 0, lu = 0;
    uint8_t *v = slurp(vocab_path, &lv, err, errlen);
    uint8_t *u = v ? slurp(unicode_path, &lu, err, errlen) : NULL;
    const int ok = v && u && load_vocab(t, v, lv, err, errlen) == 0 &&
                   load_unicode(t, u, lu, err, errlen) == 0;
    free(v);
    free(u);
    if (!ok) { cpt_free(t); return NULL; }
    return t;
}

void cpt_free(cpt_tokenizer *t) {
    if (!t) return;
    free(t->arena); free(t->off); free(t->mkey); free(t->mrank); free(t->mout);
    free(t->special); free(t->ulo); free(t->uhi); free(t->ucls);
    free(t);
}

int cpt_vocab_size(const cpt_tokenizer *t) { return t ? t->n_vocab : 0; }

int cpt_token_bytes(const cpt_tokenizer *t, int id, const char **bytes, size_t *len) {
    if (!t || id < 0 || id >= t->n_vocab) return -1;
    *bytes = (const char *)t->arena + t->off[id];
    *len = (size_t)(t->off[id + 1] - t->off[id]);
    return 0;
}

/* ---------------------------------------------------------------- BPE of one chunk */

typedef struct { uint64_t key; uint32_t a, b; } cand;    /* key = rank << 32 | left index */

static void heap_push(cand *h, int *n, cand c) {
    int i = (*n)++;
    while (i > 0 && h[(i - 1) / 2].key > c.key) { h[i] = h[(i - 1) / 2]; i = (i - 1) / 2; }
    h[i] = c;
}

static cand heap_pop(cand *h, int *n) {
    const cand top = h[0], last = h[--(*n)];
    int i = 0;
    for (;;) {
        int c = 2 * i + 1;
        if (c >= *n) break;
        if (c + 1 < *n && h[c + 1].key < h[c].key) c++;
        if (h[c].key >= last.key) break;
        h[i] = h[c];
        i = c;
    }
    if (*n > 0) h[i] = last;
    return top;
}

/* the ids of bytes s[0..n) (the first CHUNK_MAX only), appended to ids up to max_ids;
   returns how many were written (tokenizer.c:73-106) */
static int bpe(const cpt_tokenizer *t, const uint8_t *s, int n, int *ids, int max_ids) {
    if (n > CHUNK_MAX) n = CHUNK_MAX;
    int tok[CHUNK_MAX], prv[CHUNK_MAX], nxt[CHUNK_MAX], m = 0;
    cand heap[3 * CHUNK_MAX];
    int nh = 0;
    for (int i = 0; i < n; i++) {
        const int id = t->byte_tok[s[i]];
        if (id >= 0) tok[m++] = id;
    }
    for (int i = 0; i < m; i++) { prv[i] = i - 1; nxt[i] = i + 1 < m ? i + 1 : -1; }
    for (int i = 0; i + 1 < m; i++) {
        uint32_t out;
        const long r = merge_find(t, (uint32_t)tok[i], (uint32_t)tok[i + 1], &out);
        if (r >= 0) heap_push(heap, &nh, (cand){(uint64_t)r << 32 | (uint32_t)i, (uint32_t)tok[i], (uint32_t)tok[i + 1]});
    }
    while (nh > 0) {
        const cand c = heap_pop(heap, &nh);
        const int i = (int)(uint32_t)c.key, j = tok[i] >= 0 ? nxt[i] : -1;
        /* stale: the left symbol merged away, or either side changed since the pair formed */
        if (tok[i] < 0 || j < 0 || (uint32_t)tok[i] != c.a || (uint32_t)tok[j] != c.b) continue;
        uint32_t out;
        merge_find(t, c.a, c.b, &out);
        tok[i] = (int)out;
        tok[j] = -1;                               /* the right symbol is gone */
        nxt[i] = nxt[j];
        if (nxt[j] >= 0) prv[nxt[j]] = i;
        if (prv[i] >= 0) {
            const long r = merge_find(t, (uint32_t)tok[prv[i]], (uint32_t)tok[i], &out);
            if (r >= 0) heap_push(heap, &nh, (cand){(uint64_t)r << 32 | (uint32_t)prv[i], (uint32_t)tok[prv[i]], (uint32_t)tok[i]});
        }
        if (nxt[i] >= 0) {
            const long r = merge_find(t, (uint32_t)tok[i], (uint32_t)tok[nxt[i]], &out);
            if (r >= 0) heap_push(heap, &nh, (cand){(uint64_t)r << 32 | (uint32_t)i, (uint32_t)tok[i], (uint32_t)tok[nxt[i]]});
        }
    }
    int w = 0;
    for (int i = m > 0 ? 0 : -1; i >= 0 && w < max_ids; i = nxt[i]) ids[w++] = tok[i];
    return w;
}

/* ---------------------------------------------------------------- the Qwen2 pre-tokenizer */

typedef struct { uint32_t cp; int off; } uchar_t;

/* UTF-8 to code points, leniently (tokenizer_qwen.c:67-82): a lead byte needs all its
   continuation bytes inside the text, else it is a code point of its own byte value; the
   continuation bytes are not checked */
static int decode(const uint8_t *s, int n, uchar_t *u) {
    int k = 0;
    for (int i = 0; i < n;) {
        const uint8_t c = s[i];
        int len = 1;
        uint32_t cp = c;
        if (c >= 0xF0 && i + 3 < n) { len = 4; cp = c & 0x07u; }
        else if (c >= 0xE0 && i + 2 < n) { len = 3; cp = c & 0x0Fu; }
        else if (c >= 0xC0 && i + 1 < n) { len = 2; cp = c & 0x1Fu; }
        for (int j = 1; j < len; j++) cp = cp << 6 | (s[i + j] & 0x3Fu);
        u[k].cp = cp;
        u[k].off = i;
        k++;
        i += len;
    }
    return k;
}

/* 1 letter, 2 number, 0 other */
static int cls(const cpt_tokenizer *t, uint32_t cp) {
    uint32_t lo = 0, hi = t->n_ranges;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (cp < t->ulo[mid]) hi = mid;
        else if (cp > t->uhi[mid]) lo = mid + 1;
        else return t->ucls[mid];
    }
    return 0;
}

static int is_space(uint32_t c) {
    return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\v' || c == '\f';
}
static int is_newline(uint32_t c) { return c == '\n' || c == '\r'; }

/* the special token whose bytes start at byte i, the lowest such id, or -1 */
static int special_at(const cpt_tokenizer *t, const uint8_t *s, int i, int n) {
    for (int q = 0; q < t->n_special; q++) {
        const int id = t->special[q];
        const size_t l = (size_t)(t->off[id + 1] - t->off[id]);
        if ((size_t)(n - i) >= l && memcmp(s + i, t->arena + t->off[id], l) == 0) return id;
    }
    return -1;
}

/* the end (exclusive code point index) of the chunk starting at k: the first of the
   reference's alternatives that matches (tokenizer_qwen.c:116-170) */
static int chunk_end(const cpt_tokenizer *t, const uchar_t *u, int nu, int k) {
    static const char *const contr[] = {"'s", "'t", "'re", "'ve", "'m", "'ll", "'d"};
    const uint32_t c = u[k].cp;
    /* (?i:'s|'t|'re|'ve|'m|'ll|'d): ASCII letters matched without case */
    if (c == '\'')
        for (int q = 0; q < 7; q++) {
            const int L = (int)strlen(contr[q]);
            int j = 1;
            while (j < L && k + j < nu && (u[k + j].cp | 0x20u) == (uint32_t)(uint8_t)contr[q][j]) j++;
            if (j == L) return k + L;
        }
    /* [^\r\n\p{L}\p{N}]?\p{L}+ */
    {
        int j = k;
        const int cc = cls(t, c);
        if (!is_newline(c) && cc != 1 && cc != 2 && j + 1 < nu && cls(t, u[j + 1].cp) == 1) j++;
        if (j < nu && cls(t, u[j].cp) == 1) {
            while (j < nu && cls(t, u[j].cp) == 1) j++;
            return j;
        }
    }
    /* \p{N}: one number character */
    if (cls(t, c) == 2) return k + 1;
    /* ' '?[^\s\p{L}\p{N}]+[\r\n]* */
    {
        int j = k;
        if (c == ' ' && j + 1 < nu && !is_space(u[j + 1].cp) && cls(t, u[j + 1].cp) == 0) j++;
        int q = j;
        while (q < nu && !is_space(u[q].cp) && cls(t, u[q].cp) == 0) q++;
        if (q > j) {
            while (q < nu && is_newline(u[q].cp)) q++;
            return q;
        }
    }
    /* \s*[\r\n]+ (then the rest of the whitespace run, as the reference takes it) */
    {
        int j = k;
        while (j < nu && is_space(u[j].cp) && !is_newline(u[j].cp)) j++;
        if (j < nu && is_newline(u[j].cp)) {
            while (j < nu && is_space(u[j].cp)) j++;
            return j;
        }
    }
    /* \s+(?!\S), else \s+: a run followed by more text leaves its last space to that text */
    if (is_space(c)) {
        int j = k;
        while (j < nu && is_space(u[j].cp)) j++;
        const int m = j < nu ? j - 1 : j;
        return m > k ? m : j;
    }
    return k + 1;                                  /* never stall */
}

int cpt_encode(const cpt_tokenizer *t, const char *text, int *ids, int max_ids) {
    if (!t || !text || !ids || max_ids <= 0) return 0;
    const uint8_t *s = (const uint8_t *)text;
    const int n = (int)strlen(text);
    uchar_t *u = malloc(sizeof(uchar_t) * (size_t)(n > 0 ? n : 1));
    if (!u) return 0;
    const int nu = decode(s, n, u);
    int out = 0;
    for (int k = 0; k < nu && out < max_ids;) {
        const int sp = special_at(t, s, u[k].off, n);
        if (sp >= 0) {
            ids[out++] = sp;
            k += (int)(t->off[sp + 1] - t->off[sp]);    /* specials are ASCII: one per byte */
            continue;
        }
        const int end = chunk_end(t, u, nu, k);
        const int b0 = u[k].off, b1 = end < nu ? u[end].off : n;
        out += bpe(t, s + b0, b1 - b0, ids + out, max_ids - out);
        k = end;
    }
    free(u);
    return out;
}
