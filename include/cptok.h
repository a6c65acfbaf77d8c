/* cptok.h — the Qwen2 byte-level BPE tokenizer behind cp_chat, in C11, no device code.
 *
 * Reads the two files the reference's converter writes (tools/convert_tokenizer_qwen.py) and
 * its loaders read (engine/tokenizers/tokenizer.c:13-58, tokenizer_qwen.c:32-48):
 *   CPT1 vocabulary: u32 magic "CPT1", u32 version 1, u32 n_vocab, u32 n_merges; then n_vocab
 *     times (u16 length, the token's raw bytes); then n_merges times (u32 a, u32 b, u32 out),
 *     merge rank = position in the file.
 *   UNI1 classes: u32 magic "UNI1", u32 n; then n sorted ranges (u32 lo, u32 hi, u32 class)
 *     of code points, class 1 letter (\p{L}), 2 number (\p{N}), 0 other.
 * Encoding follows engine/tokenizers/tokenizer_qwen.c:100-181 (the Qwen2 pre-tokenizer: special
 * tokens at a chunk start, contractions, [^\r\n\p{L}\p{N}]?\p{L}+, single \p{N}, punctuation
 * runs with trailing newlines, whitespace rules) and the BPE of tokenizer.c:73-106 (lowest
 * merge rank first, the leftmost of equal ranks; at most the first 512 bytes of a chunk; bytes
 * without a single-byte token are dropped), so the ids are the reference's ids.
 * Returns follow the reference: 0 / negative, NULL plus a reason for a failed load. */
#ifndef CPTOK_H
#define CPTOK_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cpt_tokenizer cpt_tokenizer;

/* Load both files (tokenizer.c:13-58 and tokenizer_qwen.c:32-48). NULL on failure, the
   reason in err. */
cpt_tokenizer *cpt_load(const char *vocab_path, const char *unicode_path, char *err,
                        size_t errlen);
void cpt_free(cpt_tokenizer *t);
/* text (NUL-terminated UTF-8) to at most max_ids ids (tokenizer_qwen.c:100); returns the
   count. */
int cpt_encode(const cpt_tokenizer *t, const char *text, int *ids, int max_ids);
int cpt_vocab_size(const cpt_tokenizer *t);
/* the raw bytes of token id (not NUL-terminated): 0, or -1 for an id outside the vocabulary */
int cpt_token_bytes(const cpt_tokenizer *t, int id, const char **bytes, size_t *len);

#ifdef __cplusplus
}
#endif
#endif
