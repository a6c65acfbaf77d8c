/* model.hip — the model-level glue of a Qwen3 decode step on gfx950: the embedding gather
 * (engine/api/cachepotato.c:108-133), the residual update between layers (:157-159) and the
 * greedy argmax over the head's logits (:355-356). */
#include "cpg_internal.h"
#include "cpg_gemv.h"

/* grid T, 256 threads: row ids[t] of a v4-layout Q8_0 / Q4_0 / f32 table (rows of D) to
   out[t] (kernels.c:143-151 / :463-477: q * d, exact). Ids outside [0, rows) read row
   rows - 1, as the reference's chunked lookup clamps (cachepotato.c:115-116). */
__global__ __launch_bounds__(256) void k_embed_rows(int enc, const uint8_t *__restrict__ table,
                                                    int rows, int D,
                                                    const int *__restrict__ ids,
                                                    float *__restrict__ out) {
    const int t = blockIdx.x;
    int r = ids[t];
    r = r < 0 ? 0 : r >= rows ? rows - 1 : r;
    float *o = out + (size_t)t * D;
    if (enc == CPG_ENC_F32) {
        const float *src = (const float *)table + (size_t)r * D;
        for (int i = threadIdx.x; i < D; i += 256) o[i] = src[i];
        return;
    }
    const int bb = enc == CPG_ENC_Q8 ? 34 : 18, nb = D / 32;
    const uint8_t *row = table + (size_t)r * nb * bb;
    for (int i = threadIdx.x; i < D; i += 256) {
        const uint8_t *blk = row + (size_t)(i / 32) * bb;
        const float d = cpg_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        const int k = i % 32;
        int q;
        if (enc == CPG_ENC_Q8) {
            q = (int8_t)blk[2 + k];
        } else {
            const int byte = blk[2 + (k & 15)];
            q = (k < 16 ? byte & 15 : byte >> 4);
            q = q > 7 ? q - 16 : q;
        }
        o[i] = __fmul_rn((float)q, d);
    }
}

/* x[i] += attn[i] + mlp[i] (the sum of the two first, cachepotato.c:157-159), then mlp[i] = 0
   so the next layer's MoE half accumulates into zeros. */
__global__ __launch_bounds__(256) void k_residual(float *__restrict__ x,
                                                  const float *__restrict__ attn,
                                                  float *__restrict__ mlp, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    x[i] = __fadd_rn(x[i], __fadd_rn(attn[i], mlp[i]));
    mlp[i] = 0.0f;
}

/* Greedy argmax (cachepotato.c:355-356: the largest value, the lowest index among equal
   maxima; NaN never wins) in two passes: AM_PARTS workgroups each reduce a contiguous range to
   one candidate, then one workgroup reduces the candidates. The candidates live in this file's
   device arrays: calls are ordered on the context's stream, so they never overlap. */
#define AM_PARTS 256
__device__ float g_am_val[AM_PARTS];
__device__ int g_am_idx[AM_PARTS];

__device__ static inline void am_pick(float &best, int &idx, float ob, int oi) {
    if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
}

/* reduce (best, idx) over the 256 threads of a workgroup; the result in thread 0 */
__device__ static inline void am_block(float &best, int &idx) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    for (int o = 32; o >= 1; o >>= 1) am_pick(best, idx, __shfl_xor(best, o), __shfl_xor(idx, o));
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; w++) am_pick(best, idx, bv[w], bi[w]);
}

__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ v, int n, int per) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    const int lo = blockIdx.x * per, hi = min(n, lo + per);
    for (int i = lo + threadIdx.x; i < hi; i += 256) am_pick(best, idx, v[i], i);
    am_block(best, idx);
    if (threadIdx.x == 0) { g_am_val[blockIdx.x] = best; g_am_idx[blockIdx.x] = idx; }
}

__global__ __launch_bounds__(256) void k_argmax_final(int parts, int *__restrict__ out) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    if ((int)threadIdx.x < parts) { best = g_am_val[threadIdx.x]; idx = g_am_idx[threadIdx.x]; }
    am_block(best, idx);
    if (threadIdx.x == 0) *out = idx == 0x7fffffff ? 0 : idx;
}

/* One workgroup, after a decode step: hist[step] = *tok; route[(l * gen + step) * K + k] =
   topk[l * K + k] for the L layers (when route is not null); then the step's position and
   index advance by one (state = {pos, step}). A step beyond gen writes nothing. */
__global__ __launch_bounds__(256) void k_step_end(const int *__restrict__ tok, int *__restrict__ hist,
                                                  const int *__restrict__ topk, int *__restrict__ route,
                                                  int L, int K, int gen, int *state) {
    const int step = state[1];
    if (step >= 0 && step < gen) {
        if (threadIdx.x == 0) hist[step] = *tok;
        if (route)
            for (int i = threadIdx.x; i < L * K; i += 256)
                route[((size_t)(i / K) * gen + step) * K + i % K] = topk[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) { state[0] += 1; state[1] = step + 1; }
}

extern "C" int cpg_embed_rows(int enc, const void *table_v4, int rows, int D, const int *ids,
                              int T, float *out) {
    CPG_REQUIRE_INIT();
    if (!table_v4 || !ids || !out || T <= 0 || rows <= 0 || D <= 0 ||
        (enc != CPG_ENC_F32 && D % 32) ||
        (enc != CPG_ENC_F32 && enc != CPG_ENC_Q4 && enc != CPG_ENC_Q8)) {
        cpg_set_error("cpg_embed_rows: bad arguments");
        return -1;
    }
    hipLaunchKernelGGL(k_embed_rows, dim3(T), dim3(256), 0, g_cpg.stream, enc,
                       (const uint8_t *)table_v4, rows, D, ids, out);
    CPG_LAUNCH_CHECK("k_embed_rows");
    return 0;
}

extern "C" int cpg_residual(float *x, const float *attn, float *mlp, size_t n) {
    CPG_REQUIRE_INIT();
    if (!x || !attn || !mlp || !n) { cpg_set_error("cpg_residual: bad arguments"); return -1; }
    hipLaunchKernelGGL(k_residual, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       g_cpg.stream, x, attn, mlp, n);
    CPG_LAUNCH_CHECK("k_residual");
    return 0;
}

extern "C" int cpg_argmax(const float *v, int n, int *out) {
    CPG_REQUIRE_INIT();
    if (!v || !out || n <= 0) { cpg_set_error("cpg_argmax: bad arguments"); return -1; }
    const int per = ((n + AM_PARTS - 1) / AM_PARTS + 255) / 256 * 256;
    const int parts = (n + per - 1) / per;
    hipLaunchKernelGGL(k_argmax_part, dim3(parts), dim3(256), 0, g_cpg.stream, v, n, per);
    CPG_LAUNCH_CHECK("k_argmax_part");
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, g_cpg.stream, parts, out);
    CPG_LAUNCH_CHECK("k_argmax_final");
    return 0;
}

extern "C" int cpg_decode_step_end(const int *tok, int *hist, const int *topk, int *route,
                                   int L, int K, int gen, int *state) {
    CPG_REQUIRE_INIT();
    if (!tok || !hist || !state || gen <= 0 || (route && (!topk || L <= 0 || K <= 0))) {
        cpg_set_error("cpg_decode_step_end: bad arguments");
        return -1;
    }
    hipLaunchKernelGGL(k_step_end, dim3(1), dim3(256), 0, g_cpg.stream, tok, hist, topk, route,
                       L, K, gen, state);
    CPG_LAUNCH_CHECK("k_step_end");
    return 0;
}
