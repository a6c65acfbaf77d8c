/* tokenizer.c — the Qwen2 byte-level BPE tokenizer behind cp_chat (cptok.h).
 *
 * The files and the rules are the reference's (engine/tokenizers/tokenizer.c,
 * tokenizer_qwen.c); the ids must be identical, so every rule below keeps the reference's
 * behaviour, including its edges: a chunk is cut to its first 512 bytes, bytes that have no
 * single-byte token are dropped, UTF-8 is decoded leniently (a lead byte opens the longest
 * sequence its leading ones allow that still fits in the text, continuation bytes are not
 * checked), and special tokens are tried in id order at the start of each chunk only.
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
    uint64_t sp_first[4];            /* bit b: some special token starts with byte b */
    uint32_t *ulo, *uhi;             /* code point ranges and their classes */
    uint8_t *ucls;
    uint32_t n_ranges;
    uint8_t aflags[128];             /* the pre-tokenizer's flags of each ASCII code point */
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
        if (t->off[i + 1] > t->off[i]) {
            const uint8_t b = t->arena[t->off[i]];
            t->special[t->n_special++] = (int)i;
            t->sp_first[b >> 6] |= 1ull << (b & 63);
        }
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
        /* the class lookup bisects: the ranges must be ordered and disjoint */
        if (t->ulo[i] > t->uhi[i] || (i > 0 && t->ulo[i] <= t->uhi[i - 1])) {
            snprintf(err, errlen, "unicode table ranges not ordered at entry %u", i);
            return -1;
        }
    }
    t->n_ranges = n;
    return 0;
}

static uint8_t flags_of(const cpt_tokenizer *t, uint32_t cp);

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
    for (uint32_t c = 0; c < 128; c++) t->aflags[c] = flags_of(t, c);
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

/* ---------------------------------------------------------------- the Qwen2 pre-tokenizer
 *
 * The split (tokenizer_qwen.c:116-170) is, highest priority first,
 *   '(?i:s|t|re|ve|m|ll|d) | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} | ' '?[^\s\p{L}\p{N}]+[\r\n]*
 *   | [ \t\v\f]*[\r\n]\s* | \s+(?!\S) | \s+
 * with \s the six ASCII whitespace characters and the newline rule taking the rest of the
 * whitespace run, as the reference's code applies it. Special tokens are recognised where a
 * piece would start, the lowest id first.
 *
 * Here the text is lexed once into glyphs: one per code point, holding its byte offset, its
 * ASCII value (0 beyond ASCII) and flag bits carrying everything the rules ask of a character
 * (its class from the range table, whitespace, newline). A piece is then found without more
 * table lookups, by dispatching on the flags of its first glyph and the one after it and
 * measuring runs of glyphs whose flags satisfy a mask (piece_end). */

#define G_LET 0x01u                  /* class 1, \p{L} */
#define G_NUM 0x02u                  /* class 2, \p{N} */
#define G_CL0 0x04u                  /* class 0 */
#define G_WS 0x08u                   /* space, \t, \n, \v, \f, \r */
#define G_NL 0x10u                   /* \n, \r */

typedef struct { int off; uint8_t flags, ascii; } glyph;

/* the class of a code point in the range table (0 where no range holds it) */
static unsigned range_class(const cpt_tokenizer *t, uint32_t cp) {
    size_t a = 0, b = t->n_ranges;   /* the range holding cp, if any, is in [a, b) */
    while (b > a) {
        const size_t m = a + (b - a) / 2;
        if (cp > t->uhi[m]) a = m + 1;
        else if (cp >= t->ulo[m]) return t->ucls[m];
        else b = m;
    }
    return 0;
}

static uint8_t flags_of(const cpt_tokenizer *t, uint32_t cp) {
    const unsigned c = range_class(t, cp);
    unsigned f = c == 1 ? G_LET : c == 2 ? G_NUM : c == 0 ? G_CL0 : 0u;
    if (cp == ' ' || (cp >= '\t' && cp <= '\r')) f |= G_WS;    /* \t \n \v \f \r: 9..13 */
    if (cp == '\n' || cp == '\r') f |= G_NL;
    return (uint8_t)f;
}

/* Lenient UTF-8: a byte with L >= 2 leading one bits opens a sequence of m = min(L, 4, bytes
   left) bytes when m >= 2, its own payload being its low 7 - m bits and the m - 1 bytes after
   it taken unchecked as 6-bit continuations; any other byte (ASCII, a stray continuation, a
   lead byte at the very end) is a code point of its own value. */
static int lex(const cpt_tokenizer *t, const uint8_t *s, int n, glyph *g) {
    int k = 0;
    for (int i = 0; i < n; k++) {
        const uint32_t b = s[i];
        const int ones = __builtin_clz(~(b << 24));
        int m = ones > 4 ? 4 : ones;
        if (m > n - i) m = n - i;
        uint32_t cp = b;
        if (m >= 2) {
            cp = b & (0x7Fu >> m);
            for (int q = 1; q < m; q++) cp = cp << 6 | (s[i + q] & 0x3Fu);
        } else {
            m = 1;
        }
        g[k].off = i;
        g[k].ascii = cp < 0x80 ? (uint8_t)cp : 0;
        g[k].flags = cp < 0x80 ? t->aflags[cp] : flags_of(t, cp);
        i += m;
    }
    return k;
}

/* the end of the run of glyphs from i whose flags hold every bit of `all` and none of `none` */
static int run_end(const glyph *g, int n, int i, unsigned all, unsigned none) {
    while (i < n && (g[i].flags & all) == all && !(g[i].flags & none)) i++;
    return i;
}

/* the length of the contraction ('s 't 'm 'd 're 've 'll, letters of either case) opened by
   the apostrophe at glyph k, or 0 */
static int contraction_len(const glyph *g, int n, int k) {
    const unsigned a = k + 1 < n ? g[k + 1].ascii | 0x20u : 0u;
    const unsigned b = k + 2 < n ? g[k + 2].ascii | 0x20u : 0u;
    switch (a) {
    case 's': case 't': case 'm': case 'd': return 2;
    case 'r': case 'v': return b == 'e' ? 3 : 0;
    case 'l': return b == 'l' ? 3 : 0;
    default: return 0;
    }
}

/* the end (exclusive glyph index) of the piece starting at glyph k < n */
static int piece_end(const glyph *g, int n, int k) {
    const unsigned f = g[k].flags, f1 = k + 1 < n ? g[k + 1].flags : 0u;
    if (g[k].ascii == '\'') {
        const int c = contraction_len(g, n, k);
        if (c) return k + c;
    }
    /* a word: letters, after at most one glyph that is no newline, letter or number */
    if (f & G_LET) return run_end(g, n, k, G_LET, 0);
    if (!(f & (G_NL | G_NUM)) && (f1 & G_LET)) return run_end(g, n, k + 1, G_LET, 0);
    if (f & G_NUM) return k + 1;                        /* one number glyph */
    /* symbols (class 0, not whitespace), after at most one space, then any newlines */
    const int h = k + (g[k].ascii == ' ' && (f1 & (G_CL0 | G_WS)) == G_CL0);
    const int e = run_end(g, n, h, G_CL0, G_WS);
    if (e > h) return run_end(g, n, e, G_NL, 0);
    if (!(f & G_WS)) return k + 1;                      /* no rule matches: one glyph */
    /* whitespace: the whole run when a newline comes before any other glyph than horizontal
       whitespace; else the run, less its last glyph when text follows a run of two or more */
    const int ws = run_end(g, n, k, G_WS, 0), hz = run_end(g, n, k, G_WS, G_NL);
    if (hz < n && (g[hz].flags & G_NL)) return ws;
    return ws < n && ws - 1 > k ? ws - 1 : ws;
}

/* the special token whose bytes start at byte i, the lowest such id, or -1 */
static int special_at(const cpt_tokenizer *t, const uint8_t *s, int i, int n) {
    if (!(t->sp_first[s[i] >> 6] >> (s[i] & 63) & 1)) return -1;
    for (int q = 0; q < t->n_special; q++) {
        const int id = t->special[q];
        const size_t l = (size_t)(t->off[id + 1] - t->off[id]);
        if ((size_t)(n - i) >= l && memcmp(s + i, t->arena + t->off[id], l) == 0) return id;
    }
    return -1;
}

int cpt_encode(const cpt_tokenizer *t, const char *text, int *ids, int max_ids) {
    if (!t || !text || !ids || max_ids <= 0) return 0;
    const uint8_t *s = (const uint8_t *)text;
    const int n = (int)strlen(text);
    glyph small[256];
    glyph *g = n <= 256 ? small : malloc(sizeof(glyph) * (size_t)n);
    if (!g) return 0;
    const int ng = lex(t, s, n, g);
    int out = 0;
    for (int k = 0; k < ng && out < max_ids;) {
        /* a special token is one id; the scan then moves on by as many glyphs as the token
           has bytes (all of Qwen2's special tokens are ASCII) */
        const int sp = special_at(t, s, g[k].off, n);
        if (sp >= 0) {
            ids[out++] = sp;
            k += (int)(t->off[sp + 1] - t->off[sp]);
            continue;
        }
        const int end = piece_end(g, ng, k);
        const int b1 = end < ng ? g[end].off : n;
        out += bpe(t, s + g[k].off, b1 - g[k].off, ids + out, max_ids - out);
        k = end;
    }
    if (g != small) free(g);
    return out;
}
