/* cpg.h — C ABI of the MI355X (gfx950) Qwen3-MoE path: device-resident weights and
 * activations, hand-written HIP kernels, no torch types.
 *
 * One process drives one GPU through one context (cpg_init), mirroring the reference's
 * one-model-per-process rule (engine/api/cachepotato.h:12-13). Calls are made from one
 * host thread. Every entry point returns 0 on success or a negative code with the reason
 * in cpg_last_error(): -1 bad argument, -2 out of memory, -7 HIP/device error — the
 * reference's negative-code contract (engine/blocks/qwen3_moe.c:318-459, :565-584)
 * extended with -7 for the device.
 *
 * Work is enqueued on the context's stream and is asynchronous unless the function says
 * otherwise; cpg_sync() waits for it.
 */
#ifndef CPG_H
#define CPG_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight encodings, numbered as the reference does (engine/blocks/qwen3_moe.h:15-17). */
#define CPG_ENC_F32 0
#define CPG_ENC_Q4  4
#define CPG_ENC_Q8  8

/* ---------------------------------------------------------------- context and memory */

/* Select `device`, create the context's stream. Returns 0, or -7 when no usable GPU. */
int cpg_init(int device);
void cpg_shutdown(void);
/* the device of the initialised context, or -1 */
int cpg_current_device(void);
const char *cpg_last_error(void);
int cpg_device_count(void);
/* Device name (e.g. "AMD Instinct MI355X") and gfx arch into buf. */
int cpg_device_name(char *buf, size_t n);

void *cpg_malloc(size_t bytes);              /* NULL on failure (cpg_last_error says why) */
int cpg_free(void *dev);
int cpg_h2d(void *dst_dev, const void *src_host, size_t bytes);   /* synchronous */
int cpg_d2h(void *dst_host, const void *src_dev, size_t bytes);   /* synchronous */
int cpg_memset(void *dev, int value, size_t bytes);               /* asynchronous */
int cpg_d2d(void *dst_dev, const void *src_dev, size_t bytes);    /* asynchronous */
/* Measurement only, no counterpart in the reference: one plain streaming read of `bytes`
   (a multiple of 64 KiB * grid) by `grid` workgroups, asynchronous, to time the read floor
   that a bandwidth-bound kernel of that size can reach. out: one device float (untouched). */
int cpg_read_stream(const void *src_dev, size_t bytes, int grid, float *out_dev);
int cpg_sync(void);

/* Events on the context's stream, for timing: cpg_event_record(i) marks slot i
   (0 <= i < 4096); cpg_event_elapsed_ms(a, b) waits for b and returns the ms between. */
int cpg_event_record(int slot);
float cpg_event_elapsed_ms(int a, int b);

/* ---------------------------------------------------------------- weight layout
 *
 * In HBM a Q4_0 / Q8_0 matrix W (rows x cols, rows a multiple of 64, cols a multiple of
 * 32) is stored "row-tiled": rows in tiles of 64, and within a tile block b of all 64 rows
 * consecutively, so one wavefront (lane = row) reads one block column as one contiguous
 * 1 KiB (Q4) or 2 KiB (Q8) span.
 *   payload plane: [rows/64][cols/32][64] x 16 B (Q4) or 32 B (Q8)
 *   scale plane  : [rows/64][cols/32][64] x fp16 (the block's d, unchanged)
 * Q4 payload byte k holds (q[k]+8) | (q[k+16]+8) << 4 (the v4 byte XOR 0x88); Q8 payload
 * byte i holds q[i]+128 (the v4 byte XOR 0x80). Dequantised values are unchanged:
 * q*d is exact in fp32 either way. Planes start on 256-byte boundaries.
 */
size_t cpg_matrix_bytes(int enc, int rows, int cols);    /* payload + scale planes */
/* Bytes of one expert: Wg (F,D) | Wu (F,D) | Wd (D,F), each cpg_matrix_bytes. */
size_t cpg_expert_bytes(int enc, int D, int F);

/* Convert a matrix from the CPW1 v4 row-major block layout (format/SPEC.md:157-197;
   rows*cols/32 blocks of 18 or 34 bytes) on the device into the row-tiled layout. */
int cpg_repack(int enc, void *dst_dev, const void *src_v4_dev, int rows, int cols);
/* Host-side helper: upload v4-layout bytes of one matrix and repack (synchronous). */
int cpg_upload_matrix(int enc, void *dst_dev, const void *src_v4_host, int rows, int cols);

/* ---------------------------------------------------------------- synthetic weights
 * The counter-based generator of cpg_math.h: element i of stream s under seed S is a
 * N(0, sigma^2) draw, bit-identical on the host and the GPU. Streams are named
 * CPG_STREAM(layer, kind, index). */
#define CPG_STREAM(layer, kind, index) \
    (((uint64_t)(layer) << 40) | ((uint64_t)(kind) << 32) | (uint64_t)(index))
enum { CPG_K_WGATE = 1, CPG_K_WG = 2, CPG_K_WU = 3, CPG_K_WD = 4, CPG_K_INPUT = 5,
       CPG_K_ATTN = 6, CPG_K_EMBED = 7, CPG_K_HEAD = 8, CPG_K_NORM = 9 };

/* Host: n values of stream `stream` (elements first..first+n-1) into out. */
void cpg_gen_host(uint64_t seed, uint64_t stream, uint64_t first, size_t n, double sigma,
                  float *out);
/* Host: the same values encoded as Q4_0/Q8_0 v4 blocks (n a multiple of 32). */
void cpg_gen_blocks_host(int enc, uint64_t seed, uint64_t stream, size_t n, double sigma,
                         uint8_t *out);
/* Device: generate all E experts of synthetic layer `layer` directly into the row-tiled
   layout at dst_dev (E * cpg_expert_bytes). Expert e's matrices use streams
   CPG_STREAM(layer, kind, e) with kind 2 (Wg), 3 (Wu), 4 (Wd), sigma 0.02. Matches
   cpg_gen_blocks_host followed by cpg_repack, byte for byte. */
int cpg_gen_experts(int enc, uint64_t seed, int layer, int D, int E, int F, void *dst_dev);
/* Device: the v4-layout blocks of one generated matrix (rows*cols/32 blocks). */
int cpg_gen_blocks(int enc, uint64_t seed, uint64_t stream, int rows, int cols, double sigma,
                   void *dst_v4_dev);

/* ---------------------------------------------------------------- the MoE half
 *
 * The MoE half of one Qwen3 decoder layer, engine/blocks/qwen3_moe.c:169-223, for T tokens:
 *   hh = x + attn; xn = rmsnorm(hh, ln2, eps); logits = Wgate . xn; p = softmax(logits);
 *   top-K by (p desc, expert id asc); wt = p[idx] / sum(p[idx]) (norm_topk_prob);
 *   mlp += sum_j wt_j * Wd_e (silu(Wg_e . xn) * (Wu_e . xn))  for e = idx_j, j in order.
 * Top-K indices are bit-identical to the reference; xn, the router logits and the weights
 * too whenever they are asked for (same operation order, no contraction, glibc-identical
 * expf; see cpg_moe_route_mode). The expert GEMVs accumulate in fp32 in a different order
 * than the CPU (relative error ~1e-6).
 */
typedef struct {
    int D, E, K, F;       /* d_model, n_experts, top_k, expert intermediate size */
    int enc;              /* CPG_ENC_Q4 or CPG_ENC_Q8 */
    float eps;            /* RMSNorm epsilon (1e-6, qwen3_moe.c:401) */
    const float *ln2;     /* device (D) */
    const float *wgate;   /* device (E, D) f32 row-major */
    const void *experts;  /* device: E experts, each cpg_expert_bytes(enc, D, F) */
} cpg_moe_layer;

typedef struct cpg_moe_ws cpg_moe_ws;   /* per-call scratch, sized for up to max_T tokens */
cpg_moe_ws *cpg_moe_ws_create(int D, int E, int K, int F, int max_T);
void cpg_moe_ws_destroy(cpg_moe_ws *ws);

/* x, attn (attn may be NULL = zeros): device (T, D). Outputs on the device, any but
   mlp may be NULL: xn (T,D), router (T,E) logits, topk (T,K) int32 in selection order,
   wt (T,K). mlp (T,D) is accumulated into, as QW3Out.mlp is (qwen3_moe.c:221).
   Asynchronous. */
int cpg_moe_forward(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                    float *xn, float *router, int *topk, float *wt, float *mlp,
                    cpg_moe_ws *ws);

/* The MoE half plus the layer's residual (cachepotato.c:157-159): x += attn + mlp with
   mlp = MoE(x + attn), in the reference's order (attn + mlp first). attn is required; mlp is
   device scratch (T, D) that must be zero on entry and is zero on return (one token: the
   residual is taken in the down projection and mlp is not touched). */
int cpg_moe_forward_res(const cpg_moe_layer *L, float *x, const float *attn, int T, int *topk,
                        float *mlp, cpg_moe_ws *ws);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
   HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same
   computation, kernels and results as cpg_moe_forward, for T <= CPG_NOALLOC_MAX_T tokens, with
   the workspace taken from a static device array of 4 MiB that the library holds on each GPU
   it runs on until the process ends, instead of a cpg_moe_ws: it calls no hipMalloc, hipFree
   or allocating routine. The caller still passes the inputs and outputs. Returns -1 (with the
   reason) when T is out of range or the layer's geometry needs more than the array holds
   (Qwen3-30B-A3B needs about 3 MB). Every call on one GPU uses that GPU's one array: calls
   that overlap on a GPU (another host thread, or streams other than the context's) race, and
   must not be made. The array keeps the last call's contents; the counters in it start at
   zero and every call leaves them zero. Asynchronous, on the context's stream. */
#define CPG_NOALLOC_MAX_T 16
int cpg_moe_forward_noalloc(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                            float *xn, float *router, int *topk, float *wt, float *mlp);

/* cpg_moe_fused(1): one token (T = 1, the certified routing path) runs as one kernel:
   routing, the experts and the combine in one launch of workgroups that are all resident at
   once, the phases handing over through tagged data instead of kernel boundaries (same
   arithmetic, same bits as the separate kernels). Off by default: on MI355X it takes ~25 us
   per Qwen3-30B-A3B layer against ~21 us for the three separate kernels and their two
   boundaries, its waits polling lines that all 256 workgroups read. The fused kernel is used
   only where the device can hold all its workgroups at once. */
int cpg_moe_fused(int enable);
/* Waits of the fused kernel that gave up (after ~100 ms) since `ws` was created:
   0 unless the device could not run every workgroup at once (synchronous). */
int cpg_moe_ws_status(cpg_moe_ws *ws);

/* Number of distinct experts in the last cpg_moe_forward through `ws` (synchronous). */
int cpg_moe_ws_distinct(cpg_moe_ws *ws);

/* Tokens whose routing took a fallback of the certified path since `ws` was created
   (synchronous): the refined order, or the exact chains where that did not certify. */
int cpg_moe_ws_fallbacks(cpg_moe_ws *ws);

/* Of those, the tokens that needed the exact chains of every router row (synchronous). */
int cpg_moe_ws_exact_routings(cpg_moe_ws *ws);

/* Routing of cpg_moe_forward.
 *   CPG_ROUTE_AUTO (default): when T <= 16 and neither xn nor router is asked for, the router
 *     rows are summed in parallel and the top-K order is certified against a rigorous bound on
 *     the reference's serial-chain rounding. A token whose order cannot be certified is
 *     refined: the reference's xn and the exact chains of the few experts whose bounds reach
 *     the top K, then the order certified again; where even that cannot be certified, the
 *     exact chains of every router row. topk is bit-identical to the reference either way;
 *     wt is within a few ulps (bit-identical after the exact chains); xn (internal) within a
 *     common scale factor of a few ulps.
 *     Otherwise the exact chains: xn, router logits, topk and wt bit-identical.
 *   CPG_ROUTE_EXACT: always the exact chains.
 *   CPG_ROUTE_FORCE_FALLBACK: the certified path with every certification failed and the
 *     refined step skipped, so the exact chains run for every token (for testing them).
 *   CPG_ROUTE_FORCE_REFINE: every certification failed, so the refined step runs for every
 *     token (for testing it). */
#define CPG_ROUTE_AUTO 0
#define CPG_ROUTE_EXACT 1
#define CPG_ROUTE_FORCE_FALLBACK 2
#define CPG_ROUTE_FORCE_REFINE 3
int cpg_moe_route_mode(int mode);

/* Expert computation of cpg_moe_forward for T tokens.
 *   CPG_EXPERTS_AUTO (default): from 8 tokens the MFMA grouped GEMMs (f16 MFMA on the exact
 *     quantised weights with the block scale folded in as exact hi + lo halves, activations
 *     split into f16 hi + lo, fp32 accumulation), below that the grouped dequant-fused GEMVs
 *     (whose results do not depend on the batch a token is in); one token always the
 *     one-token GEMVs.
 *   CPG_EXPERTS_GEMV / CPG_EXPERTS_MFMA: always the one path for T > 1 (for testing). */
#define CPG_EXPERTS_AUTO 0
#define CPG_EXPERTS_GEMV 1
#define CPG_EXPERTS_MFMA 2
int cpg_moe_expert_mode(int mode);

/* Kernel timing for measurement: while enabled, cpg_moe_forward launches each kernel with a
   HIP event pair bound to the dispatch itself (hipExtLaunchKernel), so the elapsed time is
   the kernel's own execution, up to 8192 launches per kernel slot. cpg_moe_timing_read waits
   for them and returns, per slot, the summed milliseconds and the number of launches (arrays
   of at least min(n, CPG_KT_COUNT)), then clears the record. */
#define CPG_KT_ROUTE 0      /* k_route_fast, k_route_small, k_rmsnorm_tok, k_router_tok */
#define CPG_KT_SELECT 1     /* k_select_bucket, k_select, k_bucket (exact routing), k_chunks,
                               k_split_hilo */
#define CPG_KT_GATEUP 2     /* k_gateup1, k_gateup_mm, k_mfma_gateup */
#define CPG_KT_DOWN 3       /* k_down1, k_down_mm (with the weighted combine), k_mfma_down */
#define CPG_KT_COMBINE 4    /* k_pair_combine (the prefill path's weighted combine) */
#define CPG_KT_FUSED 5      /* k_moe1 (one token: routing, experts and combine in one launch) */
#define CPG_KT_COUNT 6
int cpg_moe_timing(int enable);
int cpg_moe_timing_read(double *ms, int *launches, int n);

/* ---------------------------------------------------------------- one matrix
 * out = W . x for a matrix in the v4 layout on the device (W: n_out rows of n_in), the device
 * side of qwen3_mm (engine/blocks/qwen3_moe.c:36-40). enc F32: bit-identical to matmul_wx
 * (engine/kernels/kernels.c:84-95, one serial chain per row). Q4/Q8: fp32 accumulation,
 * within rounding of matmul_wx_q4 / matmul_wx_q8. Asynchronous. */
int cpg_mm(int enc, const void *w_dev, const float *x_dev, int n_in, int n_out, float *out_dev);

/* ---------------------------------------------------------------- attention half
 * The attention half of qwen3_layer_kv (engine/blocks/qwen3_moe.c:110-167): RMSNorm (ln1),
 * q/k/v projections, per-head RMSNorm of q and k (q_norm, k_norm: (HD)), RoPE, causal GQA
 * attention over a key/value cache, output projection. The attention core (scores,
 * softmax, weighted sum) and the head norms follow the reference's operation order; the
 * projections accumulate in fp32 in another order (~1e-6 relative).
 */
typedef struct {
    int D, H, KV, HD;       /* d_model, query heads, key/value heads, head_dim (<= 128) */
    float theta, eps;       /* RoPE base, RMSNorm epsilon */
    int enc;                /* CPG_ENC_Q4 or CPG_ENC_Q8: encoding of wqkv and wo */
    const float *ln1, *q_norm, *k_norm;     /* device (D), (HD), (HD) */
    const void *wqkv;       /* device, row-tiled [(H + 2 KV) * HD, D]: Wq rows, Wk, Wv */
    const void *wo;         /* device, row-tiled [D, H * HD] */
    const float *rope;      /* device [max_pos][HD/2] (cos, sin) pairs, from cpg_rope_table */
    int max_pos;
} cpg_attn_layer;

/* Host: the RoPE table of kernels.c:430-433 for positions 0..max_pos-1 with the C library's
   powf/cosf/sinf: out[(p*HD/2 + i)*2 + {0,1}] = {cosf, sinf}((float)p * powf(theta, -2i/HD)). */
int cpg_rope_table(float theta, int HD, int max_pos, float *out_host);

typedef struct cpg_attn_ws cpg_attn_ws;
cpg_attn_ws *cpg_attn_ws_create(int D, int H, int KV, int HD, int max_T);
void cpg_attn_ws_destroy(cpg_attn_ws *ws);
/* T new tokens x (T, D) at positions pos0..pos0+T-1 (all device). kc, vc: the cache, cap
   rows of KV*HD floats; rows < pos0 are read, rows pos0..pos0+T-1 written. attn (T, D)
   receives the pre-residual attention output. -1 when pos0 + T exceeds cap, the RoPE table
   or the workspace (qwen3_moe.c:94-97 refuses such a range). Asynchronous. */
int cpg_attn_forward(const cpg_attn_layer *A, const float *x, int T, int pos0, float *kc,
                     float *vc, int cap, float *attn, cpg_attn_ws *ws);

/* As cpg_attn_forward, with the position of the first new token read on the device from
   *pos_dev when the kernels run (so a captured graph can be replayed at every position).
   Rows at or beyond min(cap, the RoPE table) are neither written nor attended: for a position
   out of range the kernels read nothing outside the cache, write NaN where they would have
   written the attention (for one token: attn's input to the output projection, so attn
   becomes NaN), and record the event in the workspace's status word (cpg_attn_ws_status). */
int cpg_attn_forward_at(const cpg_attn_layer *A, const float *x, int T, const int *pos_dev,
                        float *kc, float *vc, int cap, float *attn, cpg_attn_ws *ws);

/* Synchronises, then returns 1 when a call on ws since the last cpg_attn_ws_status met a
   position outside the cache (and clears that), 0 when none did, negative on a device
   error. No counterpart in the reference, whose positions are host values checked before
   each call (qwen3_moe.c:94-97). */
int cpg_attn_ws_status(cpg_attn_ws *ws);

/* The one-token attention kernel. CPG_ATTN_SPLIT (default): the positions split over
   workgroups of one kv head's 8 query heads, 32 positions each (k_attn_split), the last
   split of each kv head to arrive merging the splits in the same launch; only for HD = 128
   with 8 query heads per kv head (else the per-head kernel runs). CPG_ATTN_PER_HEAD: one
   workgroup per query head over all positions (k_attn_decode). On MI355X the per-head form
   is ahead by ~0.4 us per layer below ~150 positions and the split form ahead beyond (the
   whole-model decode over positions 144-400: 458-460 against 454 tokens/s). Both follow
   qwen3_moe.c:144-160 in fp32 and differ in rounding. */
#define CPG_ATTN_PER_HEAD 0
#define CPG_ATTN_SPLIT 1
int cpg_attn_decode_mode(int mode);

/* out[t] = W . x[t] for t < T, W row-tiled (CPG_ENC_Q4 / Q8; n_out a multiple of 64, n_in of
   32, at most 4096); all device. Asynchronous. */
int cpg_gemv(int enc, const void *w_tiled, int n_in, int n_out, const float *x, int T,
             float *out);
/* cpg_gemv of rmsnorm(x[t], g, eps) (the bits of cpg_rmsnorm), the norm applied while x is
   staged: one kernel instead of two. */
int cpg_gemv_norm(int enc, const void *w_tiled, int n_in, int n_out, const float *x, int T,
                  const float *g, float eps, float *out);
/* out[t] = rmsnorm(x[t], g) (kernels.c:408-413; the sum of squares accumulated in double). */
int cpg_rmsnorm(const float *x, const float *g, int T, int D, float eps, float *out);

/* ---------------------------------------------------------------- model glue
 * engine/api/cachepotato.c:108-166, :355-356 */
/* out[t] = row ids[t] of a v4-layout table (rows x D; f32, Q8_0 or Q4_0), dequantised exactly;
   ids outside [0, rows) read the last row. ids is a device array. */
int cpg_embed_rows(int enc, const void *table_v4_dev, int rows, int D, const int *ids_dev,
                   int T, float *out_dev);
/* x[i] += attn[i] + mlp[i] (attn + mlp summed first, cachepotato.c:157-159), then mlp[i] = 0. */
int cpg_residual(float *x, const float *attn, float *mlp, size_t n);
/* *out = the index of the largest of v[0..n) (the first on ties, cachepotato.c:355-356). */
int cpg_argmax(const float *v_dev, int n, int *out_dev);
/* The head and the next token in one launch, all device memory (cachepotato.c:135-147,
   :355-356, :108-133): logits = W . rmsnorm(x, g, eps) for the row-tiled Q4_0 / Q8_0 head W
   (V rows, V a multiple of 64; D = 256, 512, 1024 or 2048), *tok = the greedy argmax of logits
   (the largest value, the lowest index among equal maxima, NaN never chosen), then x is
   replaced by row *tok of the v4-layout embedding table (emb_rows rows of D, f32 / Q8_0 /
   Q4_0; a token at or beyond emb_rows reads the last row), dequantised exactly. The logits are
   within fp32 rounding of cpg_gemv_norm's (another summation order); the token is the argmax
   of the logits written. scratch: cpg_head_scratch_bytes(V) bytes of device memory, zero
   before the first call (every call leaves its counter zero); one call at a time per
   scratch. Asynchronous. */
size_t cpg_head_scratch_bytes(int V);
int cpg_head_next(int enc, const void *w_tiled, int D, int V, float *x, const float *g,
                  float eps, float *logits, int *tok, int emb_enc, const void *embed_v4,
                  int emb_rows, void *scratch);
/* End of a device-driven decode step, all device memory: hist[step] = *tok, and when route
   is not null route[(l * gen + step) * K + k] = topk[l * K + k] for l < L; then state[0] (the
   position) and state[1] (the step) advance by one. Steps outside [0, gen) record nothing. */
int cpg_decode_step_end(const int *tok, int *hist, const int *topk, int *route, int L, int K,
                        int gen, int *state);

/* ---------------------------------------------------------------- graphs
 * Work enqueued on the context's stream between cpg_capture_begin and cpg_capture_end is
 * recorded instead of run, and becomes one graph that cpg_graph_launch replays on the stream
 * (one submission for the whole sequence of kernels). No synchronous call may be made while
 * capturing. */
typedef struct cpg_graph cpg_graph;
int cpg_capture_begin(void);
cpg_graph *cpg_capture_end(void);        /* NULL on failure, the reason in cpg_last_error */
int cpg_graph_launch(cpg_graph *g);
void cpg_graph_destroy(cpg_graph *g);

/* ---------------------------------------------------------------- dequant
 * engine/kernels/kernels.c:143-151 (Q8_0) and :463-477 (Q4_0): rows of v4-layout blocks
 * on the device to f32, bit-exact. n_rows rows of `cols` elements; row r starts at
 * src + r * cols/32 * block_bytes. */
int cpg_dequant_rows(int enc, const void *src_v4_dev, int n_rows, int cols, float *dst_dev);
/* The same from the row-tiled layout (rows [row0, row0+n_rows) of a rows x cols matrix). */
int cpg_dequant_tiled(int enc, const void *tiled_dev, int rows, int cols, int row0,
                      int n_rows, float *dst_dev);

/* The device's scalar math of the exact routing path, over n values, for parity tests:
   CPG_MATH_EXPF out = expf(x) (the softmax's exponential, glibc-identical),
   CPG_MATH_SQRT out = sqrtf(x) correctly rounded (the RMSNorm), CPG_MATH_DIV out = x / y
   correctly rounded, CPG_MATH_SILU out = x / (1 + expf(-x)) (engine/kernels/kernels.c:416),
   CPG_MATH_F16 out = the fp16 number whose bits are the low 16 bits of x's bits, converted to
   fp32 by the hardware instruction the one-token GEMVs use for block scales
   (engine/kernels/kernels.c:109-130 is the reference's conversion). */
#define CPG_MATH_EXPF 0
#define CPG_MATH_SQRT 1
#define CPG_MATH_DIV  2
#define CPG_MATH_SILU 3
#define CPG_MATH_F16  4
int cpg_math_dev(int op, const float *x_dev, const float *y_dev, float *out_dev, size_t n);

#ifdef __cplusplus
}
#endif
#endif
