/* oracle.h — CPU restatement of the reference's Qwen3-MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is compared
 * against; it is never linked into, loaded by, or called from the product library
 * (cachepotato_amd/). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Every function restates one reference routine in plain C11 (built with
 * -ffp-contract=off, so a*b+c is two roundings unless fmaf() is written out, exactly as
 * GCC -std=c11 compiles the reference). The reference file:line each one follows is
 * given beside it. How each function is pinned (golden vectors from the reference engine
 * compiled by oracle/Makefile, exhaustive sweeps, closed forms) is listed in the header
 * of oracle.c.
 */
#ifndef CP_ORACLE_H
#define CP_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* encodings, numbered as engine/blocks/qwen3_moe.h:15-17 */
#define OR_ENC_F32 0
#define OR_ENC_Q8  8
#define OR_ENC_Q4  4

/* engine/kernels/kernels.c:109-130 */
float or_f16_to_f32(uint16_t h);
/* engine/kernels/kernels.c:143-151 */
void or_q8_dequant_row(const uint8_t *blocks, float *out, int n);
/* engine/kernels/kernels.c:463-477 */
void or_q4_dequant_row(const uint8_t *blocks, float *out, int n);

/* engine/kernels/kernels.c:84-95 (serial per-row dot, thread-invariant) */
void or_matmul_wx(float *out, const float *x, const float *w, int n_in, int n_out);
/* engine/kernels/kernels.c:368-396 with the AVX2 lane order of :299-366 (the reference
   build has AVX2, so this order is used at every thread count) */
void or_matmul_wx_q8(float *out, const float *x, const uint8_t *w, int n_in, int n_out);
/* engine/kernels/kernels.c:514-540. `threads` selects the numerics the reference uses:
   the AVX2 two-accumulator slice (:487-511) when threads > 1, n_in*n_out >= 60000 and
   n_out > 1; the scalar loop (:524-539) otherwise. */
void or_matmul_wx_q4(float *out, const float *x, const uint8_t *w, int n_in, int n_out,
                     int threads);

/* engine/kernels/kernels.c:408-413 */
void or_rmsnorm(float *out, const float *x, const float *g, int n, float eps);
/* glibc 2.35 expf (sysdeps/ieee754/flt-32/e_expf.c, ARM optimized-routines method), as
   the x86_64 FMA ifunc variant evaluates it. Called by engine/kernels/kernels.c:24,416. */
float or_expf(float x);
/* engine/kernels/kernels.c:20-26 */
void or_softmax(float *x, int n);
/* engine/kernels/kernels.c:416 */
float or_silu(float x);

/* The MoE half of engine/blocks/qwen3_moe.c:169-223 for T tokens.
 *   x, attn : (T, D) residual stream and attention output (attn may be NULL = zeros)
 *   ln2     : (D) RMSNorm gain;  wgate : (E, D) f32 router
 *   exp_ptr : [e*3 + kind] kind 0=Wg (F,D) 1=Wu (F,D) 2=Wd (D,F), all of encoding `enc`
 * Outputs (any may be NULL): xn (T,D), router logits (T,E), topk (T,K) in selection order,
 * wt (T,K) renormalised weights, and mlp (T,D) which is ACCUMULATED into, as
 * qwen3_moe.c:221 does (pass zeros for the reference's calloc'd QW3Out.mlp). */
void or_moe(int D, int E, int K, int F, float eps, const float *ln2, const float *wgate,
            const void *const *exp_ptr, int enc, int threads,
            const float *x, const float *attn, int T,
            float *xn, float *router, int *topk, float *wt, float *mlp);

/* engine/kernels/kernels.c:425-447: RoPE in place on q (T, nq, hd) and k (T, nk, hd) for
   positions pos0..pos0+T-1 (glibc powf/cosf/sinf, as the reference calls them). */
void or_rope(float *q, float *k, int T, int pos0, int nq, int nk, int hd, float theta);
/* The attention half of engine/blocks/qwen3_moe.c:110-167 (qwen3_layer_kv) for T tokens
   at positions pos0..pos0+T-1: RMSNorm (ln1), q/k/v projections of encoding `enc`, per-head
   q/k RMSNorm (qn, kn: (HD)), RoPE, causal GQA attention over the cache, Wo.
   kc, vc: (pos0+T, KV*HD) cache; rows < pos0 are inputs, rows pos0.. are written.
   attn: (T, D) output. */
void or_attn(int D, int H, int KV, int HD, float theta, float eps, const float *ln1,
             const float *qn, const float *kn, const void *wq, const void *wk, const void *wv,
             const void *wo, int enc, int threads, const float *x, int T, int pos0, float *kc,
             float *vc, float *attn);

/* format/q4.py:30-57 and format/q8.py:35-58: encode n floats (n a multiple of 32) into
   Q4_0 (18 B/32) or Q8_0 (34 B/32) blocks, bit-identical to the numpy encoders. */
void or_encode_q4_0(const float *x, size_t n, uint8_t *out);
void or_encode_q8_0(const float *x, size_t n, uint8_t *out);
/* IEEE binary64 / binary32 -> binary16 bits, round to nearest even (numpy astype). */
uint16_t or_f64_to_f16(double v);
uint16_t or_f32_to_f16(float v);

/* bulk helpers for the tests */
uint64_t or_exp2f_tab(int i);
void or_expf_array(const float *x, float *y, size_t n);
/* Count of bit patterns start..start+n-1 where or_expf differs from y[] (or from the host
   libm expf when y is NULL), using `threads` threads; *first_bad gets the first one. */
long or_expf_check(uint64_t start, uint64_t n, const float *y, int threads, uint64_t *first_bad);

#ifdef __cplusplus
}
#endif
#endif
