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

/* one workgroup of 1024 threads: the index of the largest value, the lowest index among
   equal maxima (cachepotato.c:355-356 keeps the first best on ties). NaN never wins. */
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ v, int n,
                                                 int *__restrict__ out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float x = v[i];
        if (x > best || (x == best && i < idx)) { best = x; idx = i; }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float ob = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) { best = bv[w]; idx = bi[w]; }
        *out = idx == 0x7fffffff ? 0 : idx;
    }
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
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, g_cpg.stream, v, n, out);
    CPG_LAUNCH_CHECK("k_argmax");
    return 0;
}
