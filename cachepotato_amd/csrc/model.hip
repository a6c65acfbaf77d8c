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

/* ---- the head and the next token in one launch
 *
 * grid V/64 (one 64-row tile of the row-tiled head per workgroup), HEAD_GW*64 threads,
 * D = HEAD_GW * BPW * 32. Lane = row of the tile, wavefront w = blocks [w*BPW, (w+1)*BPW) of
 * it, loaded first (so the final RMSNorm overlaps them). The workgroup forms
 * xn = rmsnorm(x, g, eps) with the bits of k_rmsnorm_rows (rms_inv_row, then (x*inv)*g), takes
 * its 64 rows' dot products (the wavefronts' partials summed in a fixed order), writes the
 * logits, and posts its tile's best (value, index) as one key: the order-preserving bits of
 * the value above the complement of the index, so the largest key is the largest value with
 * the lowest index (the greedy rule of cachepotato.c:355-356); NaN keys are 0 and never win.
 * The last workgroup to arrive takes the largest key of all tiles, writes the token, and
 * replaces x by that token's embedding row (cachepotato.c:108-133, exact dequantisation): every
 * other workgroup has finished reading x by then. */
#define HEAD_GW 8

__device__ static inline float embed_elem(int enc, const uint8_t *row, int i) {
    const int bb = enc == CPG_ENC_Q8 ? 34 : 18;
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
    return __fmul_rn((float)q, d);
}

template <int ENC, int BPW>
__global__ __launch_bounds__(HEAD_GW * 64) void k_head_next(
    const uint8_t *__restrict__ W, size_t payload_plane, int D, float *x,
    const float *__restrict__ g, float eps, float *__restrict__ logits,
    unsigned long long *cand, int *ctr, int *tok, int emb_enc,
    const uint8_t *__restrict__ embed, int emb_rows) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    __shared__ double npart[4];
    __shared__ int flag_s;
    __shared__ unsigned long long wbest[HEAD_GW];
    const int nb = D / 32;
    float *xs = smem;                            /* D */
    float *bsum = xs + D;                        /* nb */
    float *red = bsum + nb;                      /* HEAD_GW * 64 */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tile = blockIdx.x, row = tile * 64 + lane, b0 = w * BPW;
    WBlk<ENC> wv[BPW];
    uint16_t sv[BPW];            /* fp16 scales, converted where used: no load waited for here */
    load_row_blocks_raw<ENC, BPW>(W, payload_plane, row, b0, nb - 1, nb, wv, sv);
    const float inv = rms_inv_row(x, D, eps, npart);
    stage_tokens<ENC, HEAD_GW * 64>(xs, bsum, D, 1, [&](int, int k4) {
        const float4 v = *(const float4 *)(x + 4 * k4);
        const float4 gv = *(const float4 *)(g + 4 * k4);
        return make_float4(__fmul_rn(__fmul_rn(v.x, inv), gv.x), __fmul_rn(__fmul_rn(v.y, inv), gv.y),
                           __fmul_rn(__fmul_rn(v.z, inv), gv.z), __fmul_rn(__fmul_rn(v.w, inv), gv.w));
    });
    float dv[BPW];
#pragma unroll
    for (int j = 0; j < BPW; j++) dv[j] = f16_to_f32_hw(sv[j]);
    float acc = 0.0f;
    row_dots_mc<ENC, 1, BPW>(wv, dv, b0, BPW, xs, bsum, D, nb, &acc);
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w == 0) {
        float v = 0.0f;
        for (int ww = 0; ww < HEAD_GW; ww++) v += red[ww * 64 + lane];
        logits[row] = v;
        const unsigned long long key =
            v == v ? ((unsigned long long)ord_f(v) << 32) | (0xFFFFFFFFu - (uint32_t)row) : 0ull;
        const unsigned long long m = wave_max_u64(key);
        if (lane == 0) st_agent(&cand[tile], m);
    }
    if (!last_arriver(ctr, gridDim.x - 1, &flag_s)) return;
    /* ---- the last workgroup: the greedy token and its embedding row */
    unsigned long long best = 0;
    for (int i = tid; i < (int)gridDim.x; i += blockDim.x) {
        const unsigned long long c = ld_agent(&cand[i]);
        best = c > best ? c : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) wbest[w] = best;
    __syncthreads();
    best = wbest[0];
    for (int ww = 1; ww < HEAD_GW; ww++) best = wbest[ww] > best ? wbest[ww] : best;
    const int t = best == 0 ? 0 : (int)(0xFFFFFFFFu - (uint32_t)best);
    if (tid == 0) *tok = t;
    const int r = t >= emb_rows ? emb_rows - 1 : t;
    if (emb_enc == CPG_ENC_F32) {
        const float *src = (const float *)embed + (size_t)r * D;
        for (int i = tid; i < D; i += blockDim.x) x[i] = src[i];
    } else {
        const uint8_t *erow = embed + (size_t)r * (D / 32) * (emb_enc == CPG_ENC_Q8 ? 34 : 18);
        for (int i = tid; i < D; i += blockDim.x) x[i] = embed_elem(emb_enc, erow, i);
    }
}

extern "C" size_t cpg_head_scratch_bytes(int V) {
    return V > 0 ? cpg_round256((size_t)(V / 64) * 8) + 256 : 0;
}

template <int ENC, int BPW>
static int launch_head_next(const void *w, int D, int V, float *x, const float *g, float eps,
                            float *logits, int *tok, int emb_enc, const void *embed,
                            int emb_rows, void *scratch) {
    unsigned long long *cand = (unsigned long long *)scratch;
    int *ctr = (int *)((uint8_t *)scratch + cpg_round256((size_t)(V / 64) * 8));
    const size_t smem = sizeof(float) * ((size_t)D + D / 32 + HEAD_GW * 64);
    hipLaunchKernelGGL((k_head_next<ENC, BPW>), dim3(V / 64), dim3(HEAD_GW * 64), smem,
                       g_cpg.stream, (const uint8_t *)w, cpg_payload_plane(ENC, V, D), D, x, g,
                       eps, logits, cand, ctr, tok, emb_enc, (const uint8_t *)embed, emb_rows);
    CPG_LAUNCH_CHECK("k_head_next");
    return 0;
}

extern "C" int cpg_head_next(int enc, const void *w_tiled, int D, int V, float *x,
                             const float *g, float eps, float *logits, int *tok, int emb_enc,
                             const void *embed_v4, int emb_rows, void *scratch) {
    CPG_REQUIRE_INIT();
    const int bpw = D / 32 / HEAD_GW;
    if (!w_tiled || !x || !g || !logits || !tok || !embed_v4 || !scratch || V <= 0 ||
        V % 64 || emb_rows <= 0 || D % (32 * HEAD_GW) ||
        !(bpw == 1 || bpw == 2 || bpw == 4 || bpw == 8) ||
        (enc != CPG_ENC_Q4 && enc != CPG_ENC_Q8) ||
        (emb_enc != CPG_ENC_F32 && emb_enc != CPG_ENC_Q4 && emb_enc != CPG_ENC_Q8)) {
        cpg_set_error("cpg_head_next: bad arguments (V a multiple of 64, D = 256, 512, 1024 or "
                      "2048, Q4_0 / Q8_0 head)");
        return -1;
    }
#define HEAD_CASE(E, B)     return launch_head_next<E, B>(w_tiled, D, V, x, g, eps, logits, tok, emb_enc, embed_v4, emb_rows, scratch)
    if (enc == CPG_ENC_Q8) {
        switch (bpw) {
        case 1: HEAD_CASE(CPG_ENC_Q8, 1);
        case 2: HEAD_CASE(CPG_ENC_Q8, 2);
        case 4: HEAD_CASE(CPG_ENC_Q8, 4);
        default: HEAD_CASE(CPG_ENC_Q8, 8);
        }
    }
    switch (bpw) {
    case 1: HEAD_CASE(CPG_ENC_Q4, 1);
    case 2: HEAD_CASE(CPG_ENC_Q4, 2);
    case 4: HEAD_CASE(CPG_ENC_Q4, 4);
    default: HEAD_CASE(CPG_ENC_Q4, 8);
    }
#undef HEAD_CASE
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
