/* cachepotato.h — the engine's public API (open a model, run it, read its counters) served by
 * the MI355X engine: the whole model resident in HBM, every token computed by the HIP
 * kernels of cpg.h, nothing copied back to the host but the token ids.
 *
 * Types, functions and their meaning are the reference's (engine/api/cachepotato.h:24-90), and
 * the structs keep its layout, so the Rust front-end's mirror (cli/src/ffi.rs:13-87) links
 * against libcachepotato_amd.so unchanged. Differences:
 *   - budget_mb, threads and pin_cores are accepted and ignored: nothing is paged (the Q4 model
 *     is ~17.5 GB of the GPU's 288 GB) and the CPU does not compute. cp_stats.budget_mb is -1.
 *   - cp_open finds the tokenizer files where the reference looks (tokenizer_dir, else
 *     <model dir>/tokenizer, <model dir>, weights) and loads them with cptok.h; it refuses a
 *     tokenizer_dir without them, as the reference does, but opens a model with none found by
 *     the search: cp_chat then returns -2 (the reference's "tokenizer failure" code) with a
 *     message on stderr, and token ids go in and out through cp_eval_decode, the flow of the
 *     reference's eval driver (tools/qwen3_eval.c:338-400).
 *   - ONE MODEL PER PROCESS is kept (cachepotato.c:45, :208), as the reference's callers rely
 *     on it.
 */
#ifndef CACHEPOTATO_H
#define CACHEPOTATO_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cp_model cp_model;

/* engine/api/cachepotato.h:26-29 */
#define CP_BUDGET_AUTO 0L
#define CP_BUDGET_ENV  (-2L)
#define CP_BUDGET_NONE (-1L)

/* engine/api/cachepotato.h:31-37 */
typedef struct {
    long budget_mb;             /* accepted, ignored: the model is resident */
    int threads;                /* accepted, ignored */
    int pin_cores;              /* accepted, ignored */
    int max_ctx;                /* 0 = 2048 tokens: the KV cache capacity per layer */
    const char *tokenizer_dir;  /* NULL = search: <model dir>/tokenizer, <model dir>, weights */
} cp_options;

/* engine/api/cachepotato.h:39-40 */
void cp_options_default(cp_options *opt);

/* engine/api/cachepotato.h:42-44: maps the CPW1 v4 file, uploads it to GPU 0 and builds every
   layer's device form. NULL and a one-line reason in err on failure. */
cp_model *cp_open(const char *model_path, const cp_options *opt, char *err, size_t errlen);
void cp_close(cp_model *m);

/* engine/api/cachepotato.h:46-50 */
typedef int (*cp_token_fn)(const char *bytes, size_t len, void *user);

typedef enum { CP_STOP_EOS = 0, CP_STOP_MAX_TOKENS, CP_STOP_CONTEXT, CP_STOP_CALLER } cp_stop;

/* engine/api/cachepotato.h:54-62 */
typedef struct {
    int prompt_tokens;
    int context_tokens;
    int generated_tokens;
    int context_reset;
    double prefill_s, decode_s;
    cp_stop stop;
} cp_turn;

/* engine/api/cachepotato.h:64-69 (engine/api/cachepotato.c:315-378): the message wrapped in
   ChatML with /no_think is appended to the conversation (earlier turns stay in the KV cache),
   then greedy decoding until <|im_end|>, max_new tokens, the context limit, or the callback
   stops it; the conversation restarts first when fewer than max_new + 64 positions remain.
   Returns 0; -2 when the model was opened without tokenizer files (the reference refuses
   such an open instead; here cp_eval_decode still works on it) or the message encodes to
   nothing; -3 on a forward failure; -1 on bad arguments. */
int cp_chat(cp_model *m, const char *user_msg, int max_new,
            cp_token_fn on_token, void *user, cp_turn *turn);

/* engine/api/cachepotato.h:71-72 */
void cp_reset(cp_model *m);

/* engine/api/cachepotato.h:74-85 */
typedef struct {
    int n_layers, d_model, n_experts, topk, vocab, max_ctx;
    int threads;
    long budget_mb;
    long long file_bytes;
    long hits, misses, evictions;
    long long bytes_fetched, resident_bytes;
} cp_stats;

void cp_get_stats(const cp_model *m, cp_stats *out);

/* engine/api/cachepotato.h:87-90 */
int  cp_physical_cores(void);
long cp_mem_available_mb(void);
long cp_auto_budget_mb(long long model_file_bytes);

/* Greedy decode from token ids: the reference's eval driver in --decode mode
 * (tools/qwen3_eval.c:338-400). The conversation restarts: ids[0..T) are prefilled at
 * positions 0..T-1, then for s = 0..gen-1 the head of the last position gives
 * tokens[s] = argmax (the lowest id on ties, cachepotato.c:355-356) and tokens[s] is forwarded
 * at position T + s. There is no end-of-sequence stop: exactly gen tokens.
 *   route   (optional) n_layers x gen x topk: the experts each layer chose for each forwarded
 *           token, in selection order (qwen3_eval.c's .route file)
 *   step_ms (optional) gen: GPU time of each step (head, argmax, embedding, all layers)
 *   turn    (optional) prompt/context/generated counts and the prefill and decode times
 * Requires T + gen <= max_ctx. Returns 0, -1 on bad arguments, -3 on a forward failure (the
 * reference's cp_chat code, cachepotato.c:346), -7 on a device error. */
int cp_eval_decode(cp_model *m, const int *ids, int T, int gen, int *tokens, int *route,
                   float *step_ms, cp_turn *turn);

/* The final-position logits of the last cp_eval_decode step (vocab floats, host). 0 or -1. */
int cp_last_logits(const cp_model *m, float *out);

#ifdef __cplusplus
}
#endif
#endif
