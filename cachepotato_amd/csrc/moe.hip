/* moe.hip — the MoE half of a Qwen3-30B-A3B decoder layer on gfx950.
 *
 * Reference: engine/blocks/qwen3_moe.c:169-223 (the MoE half of qwen3_layer_kv), with the
 * kernels it calls in engine/kernels/kernels.c (rmsnorm :408-413, matmul_wx :84-95,
 * softmax :20-26, silu :416, matmul_wx_q4 :514-540, matmul_wx_q8 :368-396).
 *
 * Pipeline for T tokens (all on one stream, no host round trip):
 *   1. routing: hh = x + attn, xn = rmsnorm(hh), logits = Wgate . xn — every sum is the
 *      reference's serial add chain with separate rounding of products, so xn and the
 *      logits are bit-identical to the CPU engine.
 *   2. k_select: softmax with glibc-identical expf and the serial sum, top-K with the
 *      reference's tie rule (lower expert id wins), renormalised weights. Bit-identical.
 *   3. k_bucket: groups the T*K (token, slot) pairs by expert (stable, deterministic), so
 *      an expert chosen by several tokens streams its weights once.
 *   4. k_gateup: per (expert group, 64-row tile) gate and up dot products for every token of
 *      the group, dequantising Q4_0/Q8_0 in registers; SwiGLU fused; h to scratch.
 *   5. k_down: per (expert group, 64-row tile) the down projection of h.
 *   6. k_combine: mlp += wt_j * y_j in slot order j = 0..K-1, the reference's order.
 *
 * The expert GEMVs read the row-tiled layout of cpg.h: lane = row, so a wavefront's load of
 * one block column is one contiguous 1 KiB (Q4) / 2 KiB (Q8) span, and the activations come
 * from LDS as wave-uniform (broadcast) reads.
 */
#include "cpg_internal.h"

#include <stdlib.h>

#define WAVE 64

/* ================================================================ 1. routing (strict) */

/* Chains per workgroup in the small-T router and the k-chunk of staged products. */
#define RCPW 8
#define RKC 512

/* The RMSNorm prologue shared by the router kernels: hh = x + attn in xs[], squares in sq[],
   one lane runs the serial sum (kernels.c:410), then xs[] = (hh * inv) * g (kernels.c:412).
   Returns after a barrier with xs[] holding xn. */
__device__ static void rmsnorm_strict_wg(const float *__restrict__ xt, const float *__restrict__ at,
                                         const float *__restrict__ ln2, int D, float eps,
                                         float *xs, float *sq, float *inv_s) {
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int i = tid; i < D; i += nt) {
        const float h = __fadd_rn(xt[i], at ? at[i] : 0.0f);
        xs[i] = h;
        sq[i] = __fmul_rn(h, h);
    }
    __syncthreads();
    if (tid == 0) {
        float ss = 0.0f;
        for (int i = 0; i < D; i += 4) {
            const float4 v = *(const float4 *)(sq + i);
            ss = __fadd_rn(ss, v.x);
            ss = __fadd_rn(ss, v.y);
            ss = __fadd_rn(ss, v.z);
            ss = __fadd_rn(ss, v.w);
        }
        *inv_s = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
    }
    __syncthreads();
    const float inv = *inv_s;
    for (int i = tid; i < D; i += nt) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), ln2[i]);
    __syncthreads();
}

/* Small T: grid (ceil(E/RCPW), T), one wavefront. Every workgroup recomputes the token's
   RMSNorm (identical bits), workgroup 0 stores xn. Then RCPW router rows: all 64 lanes form
   the products fl(w*x) of a k-chunk into LDS, and lane c runs row c's serial add chain. */
__global__ __launch_bounds__(64) void k_router_small(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, int D, int E, float eps, float *__restrict__ xn_out,
    float *__restrict__ logits) {
    extern __shared__ float smem[];
    float *xs = smem;                         /* D */
    float *ps = smem + D;                     /* max(D, RCPW * (RKC + 4)) */
    __shared__ float inv_s;
    const int t = blockIdx.y, lane = threadIdx.x;
    rmsnorm_strict_wg(x + (size_t)t * D, attn ? attn + (size_t)t * D : nullptr, ln2, D, eps,
                      xs, ps, &inv_s);
    if (blockIdx.x == 0 && xn_out)
        for (int i = lane; i < D; i += WAVE) xn_out[(size_t)t * D + i] = xs[i];
    const int e0 = blockIdx.x * RCPW;
    const int nc = min(RCPW, E - e0);
    float acc = 0.0f;
    for (int k0 = 0; k0 < D; k0 += RKC) {
        const int kc = min(RKC, D - k0);
        const int q = kc / 4;
        for (int idx = lane; idx < nc * q; idx += WAVE) {
            const int c = idx / q, kk = (idx % q) * 4;
            const float4 w = *(const float4 *)(wgate + (size_t)(e0 + c) * D + k0 + kk);
            const float4 xv = *(const float4 *)(xs + k0 + kk);
            float4 p;
            p.x = __fmul_rn(w.x, xv.x);
            p.y = __fmul_rn(w.y, xv.y);
            p.z = __fmul_rn(w.z, xv.z);
            p.w = __fmul_rn(w.w, xv.w);
            *(float4 *)(ps + c * (RKC + 4) + kk) = p;
        }
        __syncthreads();
        if (lane < nc) {
            const float *pr = ps + lane * (RKC + 4);
            for (int kk = 0; kk < kc; kk += 4) {
                const float4 p = *(const float4 *)(pr + kk);
                acc = __fadd_rn(acc, p.x);
                acc = __fadd_rn(acc, p.y);
                acc = __fadd_rn(acc, p.z);
                acc = __fadd_rn(acc, p.w);
            }
        }
        __syncthreads();
    }
    if (lane < nc) logits[(size_t)t * E + e0 + lane] = acc;
}

/* Large T, step a: one lane per token runs its own RMSNorm chain. grid ceil(T/64). */
__global__ __launch_bounds__(64) void k_rmsnorm_lanes(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    int T, int D, float eps, float *__restrict__ xn) {
    const int t = blockIdx.x * WAVE + threadIdx.x;
    if (t >= T) return;
    const float *xt = x + (size_t)t * D;
    const float *at = attn ? attn + (size_t)t * D : nullptr;
    float ss = 0.0f;
    for (int k = 0; k < D; k += 4) {
        float4 v = *(const float4 *)(xt + k);
        if (at) {
            const float4 a = *(const float4 *)(at + k);
            v.x = __fadd_rn(v.x, a.x); v.y = __fadd_rn(v.y, a.y);
            v.z = __fadd_rn(v.z, a.z); v.w = __fadd_rn(v.w, a.w);
        } else {
            v.x = __fadd_rn(v.x, 0.0f); v.y = __fadd_rn(v.y, 0.0f);
            v.z = __fadd_rn(v.z, 0.0f); v.w = __fadd_rn(v.w, 0.0f);
        }
        ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
        ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
        ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
        ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
    }
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
    float *o = xn + (size_t)t * D;
    for (int k = 0; k < D; k++) {
        const float h = __fadd_rn(xt[k], at ? at[k] : 0.0f);
        o[k] = __fmul_rn(__fmul_rn(h, inv), ln2[k]);
    }
}

/* Large T, step b: grid (ceil(T/64), E); lane = token, the router row is wave-uniform. */
__global__ __launch_bounds__(64) void k_router_lanes(
    const float *__restrict__ xn, const float *__restrict__ wgate, int T, int D, int E,
    float *__restrict__ logits) {
    const int t = blockIdx.x * WAVE + threadIdx.x, e = blockIdx.y;
    if (t >= T) return;
    const float *w = wgate + (size_t)e * D;
    const float *xr = xn + (size_t)t * D;
    float acc = 0.0f;
    for (int k = 0; k < D; k += 4) {
        const float4 xv = *(const float4 *)(xr + k);
        const float4 wv = *(const float4 *)(w + k);
        acc = __fadd_rn(acc, __fmul_rn(wv.x, xv.x));
        acc = __fadd_rn(acc, __fmul_rn(wv.y, xv.y));
        acc = __fadd_rn(acc, __fmul_rn(wv.z, xv.z));
        acc = __fadd_rn(acc, __fmul_rn(wv.w, xv.w));
    }
    logits[(size_t)t * E + e] = acc;
}

/* ================================================================ 2. softmax / top-K */

#define MAX_E 256
#define MAX_K 16

/* grid T, one wavefront per token. kernels.c:20-26 then qwen3_moe.c:184-197. */
__global__ __launch_bounds__(64) void k_select(const float *__restrict__ logits, int E, int K,
                                               int *__restrict__ topk, float *__restrict__ wt) {
    __shared__ float es[MAX_E];
    __shared__ int taken[MAX_E];
    __shared__ float sum_s;
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *lg = logits + (size_t)t * E;
    /* max: the serial scan of kernels.c:22 returns the largest value; max is exact in any
       order for non-NaN input */
    float mx = lg[0];
    for (int i = lane; i < E; i += WAVE) mx = lg[i] > mx ? lg[i] : mx;
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off);
        mx = o > mx ? o : mx;
    }
    for (int i = lane; i < E; i += WAVE) {
        es[i] = cpg_expf(__fsub_rn(lg[i], mx));
        taken[i] = 0;
    }
    __syncthreads();
    if (lane == 0) {
        float s = 0.0f;
        for (int i = 0; i < E; i++) s = __fadd_rn(s, es[i]);
        sum_s = s;
    }
    __syncthreads();
    const float sum = sum_s;
    for (int i = lane; i < E; i += WAVE) es[i] = __fdiv_rn(es[i], sum);
    __syncthreads();
    int sel[MAX_K];
    for (int j = 0; j < K; j++) {
        float bp = 0.0f;
        int bi = 0x7fffffff;
        for (int i = lane; i < E; i += WAVE)
            if (!taken[i]) {
                const float p = es[i];
                if (bi == 0x7fffffff || p > bp || (p == bp && i < bi)) { bp = p; bi = i; }
            }
        for (int off = 32; off >= 1; off >>= 1) {
            const float op = __shfl_xor(bp, off);
            const int oi = __shfl_xor(bi, off);
            if (oi != 0x7fffffff &&
                (bi == 0x7fffffff || op > bp || (op == bp && oi < bi))) { bp = op; bi = oi; }
        }
        sel[j] = bi;
        if (lane == 0) taken[bi] = 1;
        __syncthreads();
    }
    if (lane == 0) {
        float s = 0.0f;
        for (int j = 0; j < K; j++) s = __fadd_rn(s, es[sel[j]]);
        for (int j = 0; j < K; j++) {
            topk[(size_t)t * K + j] = sel[j];
            wt[(size_t)t * K + j] = __fdiv_rn(es[sel[j]], s);
        }
    }
}

/* ================================================================ 3. bucketing */

#define BUCKET_MAX_T 1024   /* 16 chunks of 64 tokens */

/* One workgroup. The T*K (token, slot) pairs are grouped by expert, tokens ascending within
   a group. mask[c][e] has bit (t mod 64) set when token t of chunk c chose e (each token's
   K experts are distinct), so a pair's rank in its group is popcounts, with no ordering
   dependence on thread scheduling. Groups are numbered by ascending expert id. */
__global__ __launch_bounds__(256) void k_bucket(
    const int *__restrict__ topk, int T, int K, int E, int *__restrict__ pair_pos,
    int *__restrict__ list_tok, int *__restrict__ grp_expert, int *__restrict__ grp_off,
    int *__restrict__ grp_cnt, int *__restrict__ n_groups) {
    __shared__ unsigned long long mask[BUCKET_MAX_T / 64][MAX_E];
    __shared__ int base[MAX_E], gid[MAX_E], cnt[MAX_E];
    const int tid = threadIdx.x, C = (T + 63) / 64;
    for (int i = tid; i < C * MAX_E; i += 256) mask[i / MAX_E][i % MAX_E] = 0ull;
    __syncthreads();
    for (int p = tid; p < T * K; p += 256) {
        const int t = p / K, e = topk[p];
        atomicOr(&mask[t >> 6][e], 1ull << (t & 63));
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256) {
        int c = 0;
        for (int ch = 0; ch < C; ch++) c += __popcll(mask[ch][e]);
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int off = 0, g = 0;
        for (int e = 0; e < E; e++) {
            base[e] = off;
            gid[e] = g;
            if (cnt[e]) {
                grp_expert[g] = e;
                grp_off[g] = off;
                grp_cnt[g] = cnt[e];
                g++;
            }
            off += cnt[e];
        }
        *n_groups = g;
    }
    __syncthreads();
    for (int p = tid; p < T * K; p += 256) {
        const int t = p / K, e = topk[p], ch = t >> 6;
        int pos = base[e];
        for (int c = 0; c < ch; c++) pos += __popcll(mask[c][e]);
        pos += __popcll(mask[ch][e] & ((1ull << (t & 63)) - 1ull));
        pair_pos[p] = pos;
        list_tok[pos] = t;
    }
}

/* ================================================================ 4-5. expert GEMVs */

#define MT 4          /* tokens of a group processed per pass over the weight tile */
#define NWAVE 4       /* wavefronts per workgroup; they split the k range */

/* Dequantise one block (32 elements) of the row-tiled payload into q[0..31] (exact small
   integers: Q4 nibble - 8, Q8 byte - 128). Element k of the block is q[k]. */
template <int ENC>
__device__ static inline void load_block(const uint8_t *__restrict__ pay, size_t t, float *q) {
    if (ENC == CPG_ENC_Q4) {
        const uint4 w = *(const uint4 *)(pay + t * 16);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t byte = (wd[d] >> (8 * b)) & 0xFFu;
                q[4 * d + b] = (float)(int)(byte & 15u) - 8.0f;
                q[16 + 4 * d + b] = (float)(int)(byte >> 4) - 8.0f;
            }
    } else {
        const uint4 *p = (const uint4 *)(pay + t * 32);
        const uint4 w0 = p[0], w1 = p[1];
        const uint32_t wd[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int d = 0; d < 8; d++)
#pragma unroll
            for (int b = 0; b < 4; b++)
                q[4 * d + b] = (float)(int)((wd[d] >> (8 * b)) & 0xFFu) - 128.0f;
    }
}

/* Sum over the block of q[k] * x[k] (fp32 FMA chain), x from LDS (wave-uniform address). */
__device__ static inline float block_dot(const float *q, const float *__restrict__ xb) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k += 4) {
        const float4 xv = *(const float4 *)(xb + k);
        s = fmaf(q[k], xv.x, s);
        s = fmaf(q[k + 1], xv.y, s);
        s = fmaf(q[k + 2], xv.z, s);
        s = fmaf(q[k + 3], xv.w, s);
    }
    return s;
}

/* grid (F/64, groups), NWAVE wavefronts. Lane = row of the tile, wave w covers blocks
   [w*nb/NWAVE, (w+1)*nb/NWAVE). Computes g and u for every token of the group, reduces the
   wave partials in a fixed order, h = silu(g) * u (kernels.c:416, qwen3_moe.c:219). */
template <int ENC>
__global__ __launch_bounds__(256) void k_gateup(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes,
    size_t payload_plane, int D, int F, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ n_groups, const int *__restrict__ list_tok,
    const float *__restrict__ xn, float *__restrict__ h_list) {
    extern __shared__ float smem[];
    float *xs = smem;                                   /* MT * D */
    float *red = smem + MT * D;                         /* NWAVE * MT * 2 * 64 */
    const int g = blockIdx.y;
    if (g >= *n_groups) return;
    const int e = grp_expert[g], off = grp_off[g], m = grp_cnt[g];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nb = D / 32, bq = nb / NWAVE, b0 = w * bq;
    const int row = blockIdx.x * 64 + lane;
    const uint8_t *mg = experts + (size_t)e * exp_stride;
    const uint8_t *mu = mg + mat_bytes;
    const uint16_t *sg = (const uint16_t *)(mg + payload_plane);
    const uint16_t *su = (const uint16_t *)(mu + payload_plane);
    for (int i0 = 0; i0 < m; i0 += MT) {
        const int mc = min(MT, m - i0);
        for (int idx = tid; idx < mc * D; idx += 256) {
            const int i = idx / D, k = idx % D;
            xs[idx] = xn[(size_t)list_tok[off + i0 + i] * D + k];
        }
        __syncthreads();
        float ag[MT], au[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) { ag[i] = 0.0f; au[i] = 0.0f; }
        for (int b = b0; b < b0 + bq; b++) {
            const size_t t = cpg_tile_index(row, b, nb);
            float qg[32], qu[32];
            load_block<ENC>(mg, t, qg);
            load_block<ENC>(mu, t, qu);
            const float dg = cpg_f16_to_f32(sg[t]), du = cpg_f16_to_f32(su[t]);
#pragma unroll
            for (int i = 0; i < MT; i++)
                if (i < mc) {
                    const float *xb = xs + i * D + b * 32;
                    ag[i] = fmaf(dg, block_dot(qg, xb), ag[i]);
                    au[i] = fmaf(du, block_dot(qu, xb), au[i]);
                }
        }
#pragma unroll
        for (int i = 0; i < MT; i++) {
            red[((w * MT + i) * 2 + 0) * 64 + lane] = ag[i];
            red[((w * MT + i) * 2 + 1) * 64 + lane] = au[i];
        }
        __syncthreads();
        if (w == 0) {
            for (int i = 0; i < mc; i++) {
                float gs = 0.0f, us = 0.0f;
                for (int ww = 0; ww < NWAVE; ww++) {
                    gs += red[((ww * MT + i) * 2 + 0) * 64 + lane];
                    us += red[((ww * MT + i) * 2 + 1) * 64 + lane];
                }
                const float silu = __fdiv_rn(gs, __fadd_rn(1.0f, cpg_expf(-gs)));
                h_list[(size_t)(off + i0 + i) * F + row] = __fmul_rn(silu, us);
            }
        }
        __syncthreads();
    }
}

/* grid (D/64, groups): y = Wd . h for every token of the group. */
template <int ENC>
__global__ __launch_bounds__(256) void k_down(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t wd_off,
    size_t payload_plane, int D, int F, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ n_groups, const float *__restrict__ h_list,
    float *__restrict__ y_list) {
    extern __shared__ float smem[];
    float *hs = smem;                                   /* MT * F */
    float *red = smem + MT * F;                         /* NWAVE * MT * 64 */
    const int g = blockIdx.y;
    if (g >= *n_groups) return;
    const int e = grp_expert[g], off = grp_off[g], m = grp_cnt[g];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nb = F / 32, bq = nb / NWAVE, b0 = w * bq;
    const int row = blockIdx.x * 64 + lane;
    const uint8_t *md = experts + (size_t)e * exp_stride + wd_off;
    const uint16_t *sd = (const uint16_t *)(md + payload_plane);
    for (int i0 = 0; i0 < m; i0 += MT) {
        const int mc = min(MT, m - i0);
        for (int idx = tid; idx < mc * F; idx += 256) hs[idx] = h_list[(size_t)(off + i0) * F + idx];
        __syncthreads();
        float ay[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) ay[i] = 0.0f;
        for (int b = b0; b < b0 + bq; b++) {
            const size_t t = cpg_tile_index(row, b, nb);
            float q[32];
            load_block<ENC>(md, t, q);
            const float d = cpg_f16_to_f32(sd[t]);
#pragma unroll
            for (int i = 0; i < MT; i++)
                if (i < mc) ay[i] = fmaf(d, block_dot(q, hs + i * F + b * 32), ay[i]);
        }
#pragma unroll
        for (int i = 0; i < MT; i++) red[(w * MT + i) * 64 + lane] = ay[i];
        __syncthreads();
        if (w == 0)
            for (int i = 0; i < mc; i++) {
                float s = 0.0f;
                for (int ww = 0; ww < NWAVE; ww++) s += red[(ww * MT + i) * 64 + lane];
                y_list[(size_t)(off + i0 + i) * D + row] = s;
            }
        __syncthreads();
    }
}

/* ================================================================ 6. combine */

/* grid (ceil(D/256), T): mlp[t,i] += wt_j * y_j[i] for j = 0..K-1 (qwen3_moe.c:221). */
__global__ __launch_bounds__(256) void k_combine(
    const float *__restrict__ y_list, const int *__restrict__ pair_pos,
    const float *__restrict__ wt, int D, int K, float *__restrict__ mlp) {
    const int i = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (i >= D) return;
    float o = mlp[(size_t)t * D + i];
    for (int j = 0; j < K; j++) {
        const int pos = pair_pos[(size_t)t * K + j];
        o = __fadd_rn(o, __fmul_rn(wt[(size_t)t * K + j], y_list[(size_t)pos * D + i]));
    }
    mlp[(size_t)t * D + i] = o;
}

/* ================================================================ host side */

/* event pairs around the expert GEMVs, for the benchmark's per-kernel roofline */
#define TIMING_MAX 8192
static struct {
    int on, n;
    hipEvent_t ev[TIMING_MAX][4];
} g_timing;

extern "C" int cpg_moe_timing(int enable) {
    CPG_REQUIRE_INIT();
    g_timing.on = enable != 0;
    g_timing.n = 0;
    return 0;
}

extern "C" int cpg_moe_timing_read(double *gateup_ms, double *down_ms, int *calls) {
    CPG_REQUIRE_INIT();
    double g = 0.0, d = 0.0;
    for (int i = 0; i < g_timing.n; i++) {
        float a = 0.0f, b = 0.0f;
        CPG_HIP(hipEventSynchronize(g_timing.ev[i][3]));
        CPG_HIP(hipEventElapsedTime(&a, g_timing.ev[i][0], g_timing.ev[i][1]));
        CPG_HIP(hipEventElapsedTime(&b, g_timing.ev[i][2], g_timing.ev[i][3]));
        g += a;
        d += b;
    }
    if (gateup_ms) *gateup_ms = g;
    if (down_ms) *down_ms = d;
    if (calls) *calls = g_timing.n;
    g_timing.n = 0;
    return 0;
}

static int timing_mark(int which) {
    if (!g_timing.on || g_timing.n >= TIMING_MAX) return 0;
    hipEvent_t *e = &g_timing.ev[g_timing.n][which];
    if (!*e) CPG_HIP(hipEventCreate(e));
    CPG_HIP(hipEventRecord(*e, g_cpg.stream));
    if (which == 3) g_timing.n++;
    return 0;
}

struct cpg_moe_ws {
    int D, E, K, F, max_T;
    float *xn, *logits, *wt, *h_list, *y_list;
    int *topk, *pair_pos, *list_tok, *grp_expert, *grp_off, *grp_cnt, *n_groups;
    void *block;
};

extern "C" cpg_moe_ws *cpg_moe_ws_create(int D, int E, int K, int F, int max_T) {
    if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return nullptr; }
    if (D <= 0 || E <= 0 || E > MAX_E || K <= 0 || K > MAX_K || K > E || F <= 0 ||
        max_T <= 0) {
        cpg_set_error("cpg_moe_ws_create: bad geometry D=%d E=%d K=%d F=%d max_T=%d", D, E, K, F, max_T);
        return nullptr;
    }
    cpg_moe_ws *ws = (cpg_moe_ws *)calloc(1, sizeof *ws);
    if (!ws) { cpg_set_error("out of host memory"); return nullptr; }
    ws->D = D; ws->E = E; ws->K = K; ws->F = F; ws->max_T = max_T;
    const size_t TK = (size_t)max_T * K;
    size_t sz[12] = {
        (size_t)max_T * D * 4, (size_t)max_T * E * 4, TK * 4, TK * F * 4, TK * D * 4,
        TK * 4, TK * 4, TK * 4, (size_t)E * 4, (size_t)E * 4, (size_t)E * 4, 256};
    size_t total = 0;
    for (int i = 0; i < 12; i++) total += cpg_round256(sz[i]);
    uint8_t *p = (uint8_t *)cpg_malloc(total);
    if (!p) { free(ws); return nullptr; }
    ws->block = p;
    void **dst[12] = {(void **)&ws->xn, (void **)&ws->logits, (void **)&ws->wt,
                      (void **)&ws->h_list, (void **)&ws->y_list, (void **)&ws->topk,
                      (void **)&ws->pair_pos, (void **)&ws->list_tok, (void **)&ws->grp_expert,
                      (void **)&ws->grp_off, (void **)&ws->grp_cnt, (void **)&ws->n_groups};
    for (int i = 0; i < 12; i++) { *dst[i] = p; p += cpg_round256(sz[i]); }
    return ws;
}

extern "C" void cpg_moe_ws_destroy(cpg_moe_ws *ws) {
    if (!ws) return;
    cpg_free(ws->block);
    free(ws);
}

extern "C" int cpg_moe_ws_distinct(cpg_moe_ws *ws) {
    CPG_REQUIRE_INIT();
    int n = 0;
    if (cpg_d2h(&n, ws->n_groups, sizeof n)) return -7;
    return n;
}

static int check_layer(const cpg_moe_layer *L, int T, const cpg_moe_ws *ws) {
    if (!L || !ws || !L->wgate || !L->ln2 || !L->experts) { cpg_set_error("null layer/workspace"); return -1; }
    if (L->enc != CPG_ENC_Q4 && L->enc != CPG_ENC_Q8) { cpg_set_error("expert encoding %d unsupported", L->enc); return -1; }
    if (L->D != ws->D || L->E != ws->E || L->K != ws->K || L->F != ws->F) {
        cpg_set_error("workspace geometry does not match the layer"); return -1;
    }
    if (T <= 0 || T > ws->max_T || T > BUCKET_MAX_T) {
        cpg_set_error("T=%d outside [1, %d]", T, ws->max_T < BUCKET_MAX_T ? ws->max_T : BUCKET_MAX_T);
        return -1;
    }
    /* shapes the kernels assume: 64-row tiles, NWAVE-way k split over whole blocks,
       float4 router loads */
    if (L->D % (32 * NWAVE) || L->F % (32 * NWAVE) || L->D % 64 || L->F % 64) {
        cpg_set_error("D=%d and F=%d must be multiples of %d", L->D, L->F, 32 * NWAVE); return -1;
    }
    return 0;
}

extern "C" int cpg_moe_forward(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                               float *xn, float *router, int *topk, float *wt, float *mlp,
                               cpg_moe_ws *ws) {
    CPG_REQUIRE_INIT();
    if (check_layer(L, T, ws)) return -1;
    if (!x || !mlp) { cpg_set_error("x and mlp are required"); return -1; }
    const int D = L->D, E = L->E, K = L->K, F = L->F, enc = L->enc;
    hipStream_t s = g_cpg.stream;
    float *xn_d = xn ? xn : ws->xn;
    float *lg_d = router ? router : ws->logits;
    int *tk_d = topk ? topk : ws->topk;
    float *wt_d = wt ? wt : ws->wt;

    /* 1. routing */
    if (T <= 16) {
        const size_t smem = sizeof(float) * (size_t)(D + (D > RCPW * (RKC + 4) ? D : RCPW * (RKC + 4)));
        hipLaunchKernelGGL(k_router_small, dim3((E + RCPW - 1) / RCPW, T), dim3(64), smem, s,
                           x, attn, L->ln2, L->wgate, D, E, L->eps, xn_d, lg_d);
        CPG_LAUNCH_CHECK("k_router_small");
    } else {
        hipLaunchKernelGGL(k_rmsnorm_lanes, dim3((T + 63) / 64), dim3(64), 0, s, x, attn, L->ln2,
                           T, D, L->eps, xn_d);
        CPG_LAUNCH_CHECK("k_rmsnorm_lanes");
        hipLaunchKernelGGL(k_router_lanes, dim3((T + 63) / 64, E), dim3(64), 0, s, xn_d,
                           L->wgate, T, D, E, lg_d);
        CPG_LAUNCH_CHECK("k_router_lanes");
    }
    /* 2. softmax, top-K, renormalise */
    hipLaunchKernelGGL(k_select, dim3(T), dim3(64), 0, s, lg_d, E, K, tk_d, wt_d);
    CPG_LAUNCH_CHECK("k_select");
    /* 3. group pairs by expert */
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(256), 0, s, tk_d, T, K, E, ws->pair_pos,
                       ws->list_tok, ws->grp_expert, ws->grp_off, ws->grp_cnt, ws->n_groups);
    CPG_LAUNCH_CHECK("k_bucket");
    /* 4-5. expert GEMVs over at most min(E, T*K) groups */
    const int gmax = T * K < E ? T * K : E;
    const size_t mg = cpg_matrix_bytes(enc, F, D), md = cpg_matrix_bytes(enc, D, F);
    const size_t es = cpg_expert_bytes(enc, D, F);
    const size_t ppg = cpg_payload_plane(enc, F, D), ppd = cpg_payload_plane(enc, D, F);
    const size_t smem_gu = sizeof(float) * ((size_t)MT * D + NWAVE * MT * 2 * 64);
    const size_t smem_dn = sizeof(float) * ((size_t)MT * F + NWAVE * MT * 64);
    const uint8_t *ex = (const uint8_t *)L->experts;
    if (timing_mark(0)) return -7;
    if (enc == CPG_ENC_Q4) {
        hipLaunchKernelGGL(k_gateup<CPG_ENC_Q4>, dim3(F / 64, gmax), dim3(256), smem_gu, s, ex,
                           es, mg, ppg, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->list_tok, xn_d, ws->h_list);
        CPG_LAUNCH_CHECK("k_gateup");
        if (timing_mark(1) || timing_mark(2)) return -7;
        hipLaunchKernelGGL(k_down<CPG_ENC_Q4>, dim3(D / 64, gmax), dim3(256), smem_dn, s, ex,
                           es, 2 * mg, ppd, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->h_list, ws->y_list);
        CPG_LAUNCH_CHECK("k_down");
    } else {
        hipLaunchKernelGGL(k_gateup<CPG_ENC_Q8>, dim3(F / 64, gmax), dim3(256), smem_gu, s, ex,
                           es, mg, ppg, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->list_tok, xn_d, ws->h_list);
        CPG_LAUNCH_CHECK("k_gateup");
        if (timing_mark(1) || timing_mark(2)) return -7;
        hipLaunchKernelGGL(k_down<CPG_ENC_Q8>, dim3(D / 64, gmax), dim3(256), smem_dn, s, ex,
                           es, 2 * mg, ppd, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->h_list, ws->y_list);
        CPG_LAUNCH_CHECK("k_down");
    }
    (void)md;
    if (timing_mark(3)) return -7;
    /* 6. weighted combine in slot order */
    hipLaunchKernelGGL(k_combine, dim3((D + 255) / 256, T), dim3(256), 0, s, ws->y_list,
                       ws->pair_pos, wt_d, D, K, mlp);
    CPG_LAUNCH_CHECK("k_combine");
    return 0;
}
