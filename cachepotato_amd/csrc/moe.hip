/* moe.hip — the MoE half of a Qwen3-30B-A3B decoder layer on gfx950.
 *
 * Reference: engine/blocks/qwen3_moe.c:169-223 (the MoE half of qwen3_layer_kv), with the
 * kernels it calls in engine/kernels/kernels.c (rmsnorm :408-413, matmul_wx :84-95,
 * softmax :20-26, silu :416, matmul_wx_q4 :514-540, matmul_wx_q8 :368-396).
 *
 * One forward of T tokens is five kernels on one stream, no host round trip:
 *   routing        hh = x + attn, xn = rmsnorm(hh), logits = Wgate . xn with the reference's
 *                  serial add chains and separately rounded products: bit-identical.
 *                  T <= 16: k_route_small (the token's RMSNorm chain, then one router row
 *                  per lane); larger T: k_rmsnorm_lanes + k_router_lanes (one token per lane).
 *   selection      softmax (glibc-identical expf, serial sum), top-K with the reference's
 *                  tie rule, renormalised weights; then the T*K (token, slot) pairs are
 *                  grouped by expert so an expert chosen by several tokens streams its
 *                  weights once. T <= 16: k_select_bucket, one workgroup; else k_select +
 *                  k_bucket.
 *   k_gateup       per (64-row tile, gate|up, half of k, expert group): partial dot products
 *                  for every token of the group, Q4_0/Q8_0 dequantised in registers.
 *   k_down         h = silu(g) * u from the partials (kernels.c:416, qwen3_moe.c:219), then
 *                  y = Wd . h per 64-row tile.
 *   k_combine      mlp += wt_j * y_j in slot order j = 0..K-1 (qwen3_moe.c:221).
 * Dependent steps are separate kernels: on gfx950 a device-scope fence inside a kernel
 * writes back / invalidates a whole XCD's L2, which costs more than a kernel boundary.
 *
 * The expert GEMVs read the row-tiled layout of cpg.h: lane = row, so a wavefront's load of
 * one block column is one contiguous 1 KiB (Q4) / 2 KiB (Q8) span; the activations come
 * from LDS as wave-uniform (broadcast) reads. A block's dot product is computed on the
 * stored offset values u (Q4: q+8, Q8: q+128) and corrected once: d*(sum u*x - c*sum x).
 */
#include "cpg_internal.h"

#include <stdlib.h>

#define WAVE 64
#define MAX_E 256
#define MAX_K 16
#define SMALL_T 16          /* routing and selection in one workgroup per call up to here */
#define BUCKET_MAX_T 1024   /* k_bucket: 16 chunks of 64 tokens */
#define RPW 4               /* router rows per k_route_small workgroup */
#define MT 4                /* tokens of an expert group per pass over the weight tile */
#define GW 8                /* wavefronts per expert-GEMV workgroup (they split k) */
#define MAX_BPW 4           /* blocks per lane held in registers */
#define KS 2                /* k_gateup: workgroups splitting k of one row tile */

/* ================================================================ serial sums */

__device__ static inline float add4(float acc, float4 v) {
    acc = __fadd_rn(acc, v.x);
    acc = __fadd_rn(acc, v.y);
    acc = __fadd_rn(acc, v.z);
    return __fadd_rn(acc, v.w);
}

/* acc + p[0] + p[1] + ... + p[n-1], left to right, every add rounded: the reference's loop
   order (kernels.c:79, :410). p is in LDS, 16-byte aligned, n % 64 == 0. Two register
   buffers of 32 values alternate, each refilled as soon as it has been added, so a value
   is loaded 32 adds (256 cycles of dependent adds) before it is needed and the chain runs
   at the add latency instead of waiting on LDS. */
__device__ static inline float chain_lds(float acc, const float *p, int n) {
    const float4 *p4 = (const float4 *)p;
    const int n4 = n >> 2;
    float4 a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = p4[j];
#pragma unroll
    for (int j = 0; j < 8; j++) b[j] = p4[8 + j];
    for (int i = 16; i < n4; i += 16) {
#pragma unroll
        for (int j = 0; j < 8; j++) acc = add4(acc, a[j]);
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = p4[i + j];
#pragma unroll
        for (int j = 0; j < 8; j++) acc = add4(acc, b[j]);
#pragma unroll
        for (int j = 0; j < 8; j++) b[j] = p4[i + 8 + j];
    }
#pragma unroll
    for (int j = 0; j < 8; j++) acc = add4(acc, a[j]);
#pragma unroll
    for (int j = 0; j < 8; j++) acc = add4(acc, b[j]);
    return acc;
}

__device__ static inline float chain_any(const float *p, int n) {
    if ((n & 63) == 0) return chain_lds(0.0f, p, n);
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = __fadd_rn(s, p[i]);
    return s;
}

__device__ static inline float rms_inv(float ss, int D, float eps) {
    /* kernels.c:411: 1 / sqrtf(ss / n + eps), each operation rounded */
    return __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
}

/* LDS written by some lanes of a wavefront, then read by others of the same wavefront:
   its LDS operations execute in order, the compiler must only not reorder them. */
__device__ static inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

/* ================================================================ softmax / top-K */

/* One token, one wavefront (all 64 lanes call it). kernels.c:20-26 (max, expf(x - max),
   serial sum, divide) then qwen3_moe.c:184-197 (K passes of a strict-greater scan, the lower
   id wins ties; renormalise by the serial sum of the selected probabilities).
   es: this wavefront's LDS scratch of E entries. */
__device__ static void select_token(const float *__restrict__ lg, int E, int K,
                                    int *__restrict__ topk_row, float *__restrict__ wt_row,
                                    float *es) {
    const int lane = threadIdx.x & 63;
    float mx = lg[0];
    for (int i = lane; i < E; i += WAVE) mx = lg[i] > mx ? lg[i] : mx;
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off);
        mx = o > mx ? o : mx;
    }
    for (int i = lane; i < E; i += WAVE) es[i] = cpg_expf(__fsub_rn(lg[i], mx));
    wave_lds_sync();
    float sum = 0.0f;
    if (lane == 0) sum = chain_any(es, E);
    sum = __shfl(sum, 0);
    wave_lds_sync();
    for (int i = lane; i < E; i += WAVE) es[i] = __fdiv_rn(es[i], sum);
    wave_lds_sync();
    /* The K passes of the reference's scan pick the experts in the order of the key
       (p descending, id ascending), which is a total order: expert e is picked in pass
       rank(e) = #{e' : p[e'] > p[e] or (p[e'] == p[e] and e' < e)}. Every lane ranks its
       (at most MAX_E/64) experts against all E at once instead of K dependent passes, then
       the expert of rank j is found with a ballot. */
    int rk[MAX_E / WAVE];
#pragma unroll
    for (int k = 0; k < MAX_E / WAVE; k++) {
        const int i = lane + WAVE * k;
        rk[k] = 0x7fffffff;
        if (i < E) {
            const float p = es[i];
            int r = 0;
            for (int q = 0; q < E; q++) {
                const float o = es[q];
                r += (o > p) || (o == p && q < i);
            }
            rk[k] = r;
        }
    }
    int sel[MAX_K];
    for (int j = 0; j < K; j++) {
        int cand = -1;
#pragma unroll
        for (int k = 0; k < MAX_E / WAVE; k++)
            if (rk[k] == j) cand = lane + WAVE * k;
        const unsigned long long b = __ballot(cand >= 0);
        sel[j] = b ? __shfl(cand, __ffsll((long long)b) - 1) : 0;     /* b == 0 only with NaN */
    }
    float s = 0.0f;
    if (lane == 0)
        for (int j = 0; j < K; j++) s = __fadd_rn(s, es[sel[j]]);
    s = __shfl(s, 0);
    for (int j = lane; j < K; j += WAVE) {
        int sj = sel[0];
#pragma unroll
        for (int q = 1; q < MAX_K; q++)
            if (q == j) sj = sel[q];
        topk_row[j] = sj;
        wt_row[j] = __fdiv_rn(es[sj], s);
    }
}

/* ================================================================ bucketing */

/* Whole workgroup. Groups the T*K (token, slot) pairs by expert, tokens ascending within a
   group, groups by ascending expert id. mask[c*E + e] has bit (t mod 64) set when token t of
   chunk c chose e (a token's K experts are distinct), so a pair's rank in its group is a sum
   of popcounts: the result does not depend on thread scheduling. Group slots from the
   number of groups up to E get a count of 0, so a consumer can read a slot's (expert,
   offset, count) in one round trip and skip empty ones. list_tok[pos] / list_pair[pos]:
   token and pair index (t*K + j) of the pos-th entry. mask: C*E u64 of LDS, base/cnt: E
   ints of LDS. */
__device__ static void bucket_pairs(const int *__restrict__ topk, int T, int K, int E,
                                    unsigned long long *mask, int *base, int *cnt,
                                    int *__restrict__ pair_pos, int *__restrict__ list_tok,
                                    int *__restrict__ list_pair, int *__restrict__ grp_expert,
                                    int *__restrict__ grp_off, int *__restrict__ grp_cnt,
                                    int *__restrict__ n_groups) {
    const int tid = threadIdx.x, nt = blockDim.x, C = (T + 63) / 64;
    for (int i = tid; i < C * E; i += nt) mask[i] = 0ull;
    /* every list entry holds a valid index even if routing was degenerate (NaN logits can
       repeat an expert within a token; such pairs are dropped, never written out of range) */
    for (int i = tid; i < T * K; i += nt) { list_tok[i] = 0; list_pair[i] = 0; }
    __syncthreads();
    for (int p = tid; p < T * K; p += nt) {
        const int t = p / K, e = topk[p];
        if ((unsigned)e < (unsigned)E) atomicOr(&mask[(t >> 6) * E + e], 1ull << (t & 63));
    }
    __syncthreads();
    for (int e = tid; e < E; e += nt) {
        int c = 0;
        for (int ch = 0; ch < C; ch++) c += __popcll(mask[ch * E + e]);
        cnt[e] = c;
    }
    __syncthreads();
    if (tid < WAVE) {
        /* exclusive prefix sums over experts (4 per lane) of the pair counts and of the
           number of non-empty experts */
        int c[MAX_E / WAVE], ls = 0, lg = 0;
#pragma unroll
        for (int k = 0; k < MAX_E / WAVE; k++) {
            const int e = tid * (MAX_E / WAVE) + k;
            c[k] = e < E ? cnt[e] : 0;
            ls += c[k];
            lg += c[k] > 0;
        }
        int ps = ls, pg = lg;
        for (int o = 1; o < WAVE; o <<= 1) {
            const int a = __shfl_up(ps, o), b = __shfl_up(pg, o);
            if (tid >= o) { ps += a; pg += b; }
        }
        int off = ps - ls, g = pg - lg;
#pragma unroll
        for (int k = 0; k < MAX_E / WAVE; k++) {
            const int e = tid * (MAX_E / WAVE) + k;
            if (e < E) {
                base[e] = off;
                if (c[k]) {
                    grp_expert[g] = e;
                    grp_off[g] = off;
                    grp_cnt[g] = c[k];
                    g++;
                }
                off += c[k];
            }
        }
        const int ng = __shfl(pg, WAVE - 1);
        if (tid == 0) *n_groups = ng;
        for (int q = ng + tid; q < E; q += WAVE) grp_cnt[q] = 0;
    }
    __syncthreads();
    for (int p = tid; p < T * K; p += nt) {
        const int t = p / K, e = topk[p], ch = t >> 6;
        int pos = 0;
        if ((unsigned)e < (unsigned)E) {
            pos = base[e];
            for (int c = 0; c < ch; c++) pos += __popcll(mask[c * E + e]);
            pos += __popcll(mask[ch * E + e] & ((1ull << (t & 63)) - 1ull));
        }
        pair_pos[p] = pos;
        if (pos < T * K) {
            list_tok[pos] = t;
            list_pair[pos] = p;
        }
    }
}

/* ================================================================ routing, T <= 16 */

/* grid (ceil(E/RPW), T), 256 threads. Every workgroup of a token computes the token's RMSNorm
   (identical bits; workgroup 0 stores xn): wave 0 lane 0 runs the serial sum of squares
   while waves 1-3 copy the workgroup's RPW router rows into LDS. The rows are multiplied by
   xn in place (the reference's separately rounded products) and lane c of wave 0 runs row
   c's serial add chain. */
__global__ __launch_bounds__(256) void k_route_small(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, int D, int E, float eps, float *__restrict__ xn_out,
    float *__restrict__ logits) {
    extern __shared__ float smem[];
    float *xs = smem;                      /* D */
    float *sq = xs + D;                    /* D */
    float *wp = sq + D;                    /* RPW rows of D + 4 */
    __shared__ float inv_s;
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int e0 = blockIdx.x * RPW, nc = min(RPW, E - e0), ld = D + 4, d4 = D / 4;
    const float *xt = x + (size_t)t * D;
    const float *at = attn ? attn + (size_t)t * D : nullptr;

    for (int i = tid; i < D; i += 256) {
        const float h = __fadd_rn(xt[i], at ? at[i] : 0.0f);          /* qwen3_moe.c:178 */
        xs[i] = h;
        sq[i] = __fmul_rn(h, h);
    }
    __syncthreads();
    if (w == 0) {
        if (lane == 0) inv_s = rms_inv(chain_lds(0.0f, sq, D), D, eps);
    } else {
        /* all of this thread's router-row loads are in flight before the first store */
        const int per = (nc * d4 + 191) / 192;
        for (int base = 0; base < per; base += 16) {
            float4 v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int idx = (tid - WAVE) + 192 * (base + j);
                if (base + j < per && idx < nc * d4) {
                    const int c = idx / d4, k4 = idx - c * d4;
                    v[j] = *(const float4 *)(wgate + (size_t)(e0 + c) * D + 4 * k4);
                }
            }
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int idx = (tid - WAVE) + 192 * (base + j);
                if (base + j < per && idx < nc * d4) {
                    const int c = idx / d4, k4 = idx - c * d4;
                    *(float4 *)(wp + c * ld + 4 * k4) = v[j];
                }
            }
        }
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = tid; i < D; i += 256) {
        const float v = __fmul_rn(__fmul_rn(xs[i], inv), ln2[i]);     /* kernels.c:412 */
        xs[i] = v;
        if (blockIdx.x == 0) xn_out[(size_t)t * D + i] = v;
    }
    __syncthreads();
    for (int idx = tid; idx < nc * d4; idx += 256) {
        const int c = idx / d4, k4 = idx - c * d4;
        float4 *pw = (float4 *)(wp + c * ld + 4 * k4);
        const float4 wv = *pw, xv = *(const float4 *)(xs + 4 * k4);
        *pw = make_float4(__fmul_rn(wv.x, xv.x), __fmul_rn(wv.y, xv.y), __fmul_rn(wv.z, xv.z),
                          __fmul_rn(wv.w, xv.w));
    }
    __syncthreads();
    if (w == 0 && lane < nc)
        logits[(size_t)t * E + e0 + lane] = chain_lds(0.0f, wp + lane * ld, D);
}

/* One workgroup of 64*T threads (T <= SMALL_T): wavefront t selects token t's experts, then
   the workgroup groups the pairs by expert. */
__global__ __launch_bounds__(64 * SMALL_T) void k_select_bucket(
    const float *__restrict__ logits, int T, int E, int K, int *__restrict__ topk,
    float *__restrict__ wt, int *__restrict__ pair_pos, int *__restrict__ list_tok,
    int *__restrict__ list_pair, int *__restrict__ grp_expert, int *__restrict__ grp_off,
    int *__restrict__ grp_cnt, int *__restrict__ n_groups) {
    __shared__ float es[SMALL_T][MAX_E];
    __shared__ unsigned long long mask[MAX_E];
    __shared__ int base[MAX_E], cnt[MAX_E];
    const int t = threadIdx.x >> 6;
    select_token(logits + (size_t)t * E, E, K, topk + (size_t)t * K, wt + (size_t)t * K, es[t]);
    __syncthreads();
    bucket_pairs(topk, T, K, E, mask, base, cnt, pair_pos, list_tok, list_pair, grp_expert,
                 grp_off, grp_cnt, n_groups);
}

/* ================================================================ routing, T > 16 */

/* step a: one lane per token runs its own RMSNorm chain. grid ceil(T/64). */
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
        const float4 a = at ? *(const float4 *)(at + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v = make_float4(__fadd_rn(v.x, a.x), __fadd_rn(v.y, a.y), __fadd_rn(v.z, a.z),
                        __fadd_rn(v.w, a.w));
        ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
        ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
        ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
        ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
    }
    const float inv = rms_inv(ss, D, eps);
    float *o = xn + (size_t)t * D;
    for (int k = 0; k < D; k++) {
        const float h = __fadd_rn(xt[k], at ? at[k] : 0.0f);
        o[k] = __fmul_rn(__fmul_rn(h, inv), ln2[k]);
    }
}

/* step b: grid (ceil(T/64), E); lane = token, the router row is wave-uniform. */
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

/* grid T, 64 threads: softmax and top-K of one token */
__global__ __launch_bounds__(64) void k_select(const float *__restrict__ logits, int E, int K,
                                               int *__restrict__ topk, float *__restrict__ wt) {
    __shared__ float es[MAX_E];
    const int t = blockIdx.x;
    select_token(logits + (size_t)t * E, E, K, topk + (size_t)t * K, wt + (size_t)t * K, es);
}

/* one workgroup of 256 threads */
__global__ __launch_bounds__(256) void k_bucket(
    const int *__restrict__ topk, int T, int K, int E, int *__restrict__ pair_pos,
    int *__restrict__ list_tok, int *__restrict__ list_pair, int *__restrict__ grp_expert,
    int *__restrict__ grp_off, int *__restrict__ grp_cnt, int *__restrict__ n_groups) {
    __shared__ unsigned long long mask[(BUCKET_MAX_T / 64) * MAX_E];
    __shared__ int base[MAX_E], cnt[MAX_E];
    bucket_pairs(topk, T, K, E, mask, base, cnt, pair_pos, list_tok, list_pair, grp_expert,
                 grp_off, grp_cnt, n_groups);
}

/* ================================================================ expert GEMVs */

/* v & m, opaque to the optimiser: with the mask visible the compiler folds the byte
   extraction that follows into a bit-field extract plus a convert; hidden, every byte of the
   masked word converts with one v_cvt_f32_ubyteN. */
__device__ static inline uint32_t and_opaque(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(m));
    return r;
}

/* s += the four bytes of w times xv (one dependent FMA chain) */
__device__ static inline float fma_bytes(uint32_t w, float4 xv, float s) {
    s = fmaf((float)(w & 0xFFu), xv.x, s);
    s = fmaf((float)((w >> 8) & 0xFFu), xv.y, s);
    s = fmaf((float)((w >> 16) & 0xFFu), xv.z, s);
    return fmaf((float)(w >> 24), xv.w, s);
}

/* One block of the row-tiled payload held in registers. Stored values u (Q4: q+8 in 0..15,
   Q8: q+128 in 0..255) are exact small integers; the block's dot product is taken on u and
   corrected once by offset * (sum of x over the block). Staged activations hold, per
   32-element block, x[0..15] then x[16..31]/16 for Q4 (the high nibbles are used in place,
   worth 16u, so the power-of-two scale moves to x exactly), plain x for Q8. */
template <int ENC> struct WBlk;
template <> struct WBlk<CPG_ENC_Q4> {
    uint4 v;
    __device__ void load(const uint8_t *pay, size_t t) { v = *(const uint4 *)(pay + t * 16); }
    /* the conversions must happen where they are used: without this the compiler hoists
       every block's byte-to-float conversions out of the token loop and spills them */
    __device__ void pin() { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
    static constexpr float offset = 8.0f;
    /* s[i] = sum over the block of u * x for tokens i < MC. Word d holds elements 4d..4d+3
       in its low nibbles and 16+4d..16+4d+3 in its high nibbles; low and high products go
       to separate chains. */
    template <int MC>
    __device__ void dots(const float *xb, int ncol, float *s) const {
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        float a[MC], b[MC];
#pragma unroll
        for (int i = 0; i < MC; i++) { a[i] = 0.0f; b[i] = 0.0f; }
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t lo = and_opaque(wd[d], 0x0F0F0F0Fu), hi = and_opaque(wd[d], 0xF0F0F0F0u);
#pragma unroll
            for (int i = 0; i < MC; i++) {
                a[i] = fma_bytes(lo, *(const float4 *)(xb + i * ncol + 4 * d), a[i]);
                b[i] = fma_bytes(hi, *(const float4 *)(xb + i * ncol + 16 + 4 * d), b[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < MC; i++) s[i] = a[i] + b[i];
    }
};
template <> struct WBlk<CPG_ENC_Q8> {
    uint4 v0, v1;
    __device__ void load(const uint8_t *pay, size_t t) {
        const uint4 *p = (const uint4 *)(pay + t * 32);
        v0 = p[0];
        v1 = p[1];
    }
    __device__ void pin() {
        asm volatile("" : "+v"(v0.x), "+v"(v0.y), "+v"(v0.z), "+v"(v0.w));
        asm volatile("" : "+v"(v1.x), "+v"(v1.y), "+v"(v1.z), "+v"(v1.w));
    }
    static constexpr float offset = 128.0f;
    template <int MC>
    __device__ void dots(const float *xb, int ncol, float *s) const {
        const uint32_t wd[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float a[MC], b[MC];
#pragma unroll
        for (int i = 0; i < MC; i++) { a[i] = 0.0f; b[i] = 0.0f; }
#pragma unroll
        for (int d = 0; d < 8; d += 2) {
#pragma unroll
            for (int i = 0; i < MC; i++) {
                a[i] = fma_bytes(wd[d], *(const float4 *)(xb + i * ncol + 4 * d), a[i]);
                b[i] = fma_bytes(wd[d + 1], *(const float4 *)(xb + i * ncol + 4 * d + 4), b[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < MC; i++) s[i] = a[i] + b[i];
    }
};

/* acc[i] = dot product of this lane's row (blocks b0 .. b0+nbw-1 of the staged range, in
   registers) with staged token i < MC. Blocks are added in order, each corrected and
   scaled. */
template <int ENC, int MC>
__device__ static inline void row_dots_mc(const WBlk<ENC> *wv, const float *dv, int b0, int nbw,
                                          const float *xs, const float *bsum, int ncol, int nb,
                                          float *acc) {
#pragma unroll
    for (int j = 0; j < MAX_BPW; j++)
        if (j < nbw) {
            const int b = b0 + j;
            float s[MC];
            wv[j].template dots<MC>(xs + b * 32, ncol, s);
#pragma unroll
            for (int i = 0; i < MC; i++)
                acc[i] = fmaf(dv[j], fmaf(-WBlk<ENC>::offset, bsum[i * nb + b], s[i]), acc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
}

template <int ENC>
__device__ static inline void row_dots(const WBlk<ENC> *wv, const float *dv, int b0, int nbw,
                                       const float *xs, const float *bsum, int ncol, int nb,
                                       int mc, float *acc) {
    switch (mc) {
    case 1: row_dots_mc<ENC, 1>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    case 2: row_dots_mc<ENC, 2>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    case 3: row_dots_mc<ENC, 3>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    default: row_dots_mc<ENC, 4>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    }
}

/* h = silu(g) * u, kernels.c:416 and qwen3_moe.c:219 */
__device__ static inline float swiglu(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, cpg_expf(-g))), u);
}

/* Stage mc token vectors of ncol floats into LDS: xs[i*ncol + k] = get(i, k/4) (a float4),
   the second half of every 32-element block pre-scaled by 1/16 for Q4; bs[i*nb + b] = the
   block's sum (unscaled). One float4 per thread per pass; the eight float4 of a block are in
   eight consecutive lanes, summed by xor shuffles. Ends with a barrier. ncol % 32 == 0. */
template <int ENC, int NT, typename Get>
__device__ static inline void stage_tokens(float *xs, float *bs, int ncol, int mc, Get get) {
    const int q = ncol / 4, nb = ncol / 32;
    for (int idx = threadIdx.x; idx < ((mc * q + 63) & ~63); idx += NT) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const int i = idx / q, k4 = idx - i * q;
        if (idx < mc * q) v = get(i, k4);
        float s = ((v.x + v.y) + v.z) + v.w;
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        if (idx < mc * q) {
            if ((k4 & 7) == 0) bs[i * nb + (k4 >> 3)] = s;
            if (ENC == CPG_ENC_Q4 && (k4 & 7) >= 4)
                v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
            *(float4 *)(xs + i * ncol + 4 * k4) = v;
        }
    }
    __syncthreads();
}

/* grid (F/64, 2*KS, groups): blockIdx.y = matrix (0 gate, 1 up) * KS + k part. One 64-row
   tile of the matrix over one KS-th of its columns, for every token of one expert group.
   Lane = row; wave w holds its share of the part's blocks in registers for the whole call;
   tokens are staged MT at a time. Writes the partial dot products
   gu[((pair * 2 + matrix) * KS + part) * F + row]. */
template <int ENC>
__global__ __launch_bounds__(GW * 64) void k_gateup(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes,
    size_t payload_plane, int D, int F, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ n_groups, const int *__restrict__ list_tok,
    const float *__restrict__ xn, float *__restrict__ gu) {
    extern __shared__ float smem[];
    const int g = blockIdx.z;
    const int e = grp_expert[g], off = grp_off[g], m = grp_cnt[g];
    if (m == 0) return;
    const int nbt = D / 32, nb = nbt / KS, ncol = nb * 32;      /* this part's blocks */
    const int mat = blockIdx.y / KS, part = blockIdx.y % KS, c0 = part * ncol;
    float *xs = smem;                            /* MT * ncol */
    float *bsum = xs + MT * ncol;                /* MT * nb */
    float *red = bsum + MT * nb;                 /* GW * MT * 64 */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bpw = (nb + GW - 1) / GW, b0 = w * bpw, nbw = max(0, min(bpw, nb - b0));
    const int row = blockIdx.x * 64 + lane;
    const uint8_t *M = experts + (size_t)e * exp_stride + (size_t)mat * mat_bytes;
    const uint16_t *S = (const uint16_t *)(M + payload_plane);
    WBlk<ENC> wv[MAX_BPW];
    float dv[MAX_BPW];
#pragma unroll
    for (int j = 0; j < MAX_BPW; j++)
        if (j < nbw) {
            const size_t t = cpg_tile_index(row, part * nb + b0 + j, nbt);
            wv[j].load(M, t);
            dv[j] = cpg_f16_to_f32(S[t]);
        }
    for (int i0 = 0; i0 < m; i0 += MT) {
        const int mc = min(MT, m - i0);
#pragma unroll
        for (int j = 0; j < MAX_BPW; j++) wv[j].pin();
        stage_tokens<ENC, GW * 64>(xs, bsum, ncol, mc, [&](int i, int k4) {
            return *(const float4 *)(xn + (size_t)list_tok[off + i0 + i] * D + c0 + 4 * k4);
        });
        float acc[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i] = 0.0f;
        row_dots<ENC>(wv, dv, b0, nbw, xs, bsum, ncol, nb, mc, acc);
#pragma unroll
        for (int i = 0; i < MT; i++) red[(w * MT + i) * 64 + lane] = acc[i];
        __syncthreads();
        if (w == 0)
            for (int i = 0; i < mc; i++) {
                float s = 0.0f;
                for (int ww = 0; ww < GW; ww++) s += red[(ww * MT + i) * 64 + lane];
                gu[(((size_t)(off + i0 + i) * 2 + mat) * KS + part) * F + row] = s;
            }
        __syncthreads();
    }
}

/* grid (D/64, groups): h = silu(g) * u for the group's tokens from the k partials (summed
   in part order), staged MT at a time, then y = Wd . h for one 64-row tile, stored at the
   pair's index t*K + j. */
template <int ENC>
__global__ __launch_bounds__(GW * 64) void k_down(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t wd_off,
    size_t payload_plane, int D, int F, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ list_pair, const float *__restrict__ gu, float *__restrict__ y) {
    extern __shared__ float smem[];
    const int nb = F / 32;
    float *hs = smem;                            /* MT * F */
    float *bsum = hs + MT * F;                   /* MT * nb */
    float *red = bsum + MT * nb;                 /* GW * MT * 64 */
    const int g = blockIdx.y;
    const int e = grp_expert[g], off = grp_off[g], m = grp_cnt[g];
    if (m == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bpw = (nb + GW - 1) / GW, b0 = w * bpw, nbw = max(0, min(bpw, nb - b0));
    const int row = blockIdx.x * 64 + lane;
    const uint8_t *M = experts + (size_t)e * exp_stride + wd_off;
    const uint16_t *S = (const uint16_t *)(M + payload_plane);
    WBlk<ENC> wv[MAX_BPW];
    float dv[MAX_BPW];
#pragma unroll
    for (int j = 0; j < MAX_BPW; j++)
        if (j < nbw) {
            const size_t t = cpg_tile_index(row, b0 + j, nb);
            wv[j].load(M, t);
            dv[j] = cpg_f16_to_f32(S[t]);
        }
    for (int i0 = 0; i0 < m; i0 += MT) {
        const int mc = min(MT, m - i0);
#pragma unroll
        for (int j = 0; j < MAX_BPW; j++) wv[j].pin();
        stage_tokens<ENC, GW * 64>(hs, bsum, F, mc, [&](int i, int k4) {
            const float *p = gu + (size_t)(off + i0 + i) * 2 * KS * F + 4 * k4;
            float4 gv = *(const float4 *)p, uv = *(const float4 *)(p + KS * F);
#pragma unroll
            for (int q = 1; q < KS; q++) {
                const float4 g2 = *(const float4 *)(p + q * F), u2 = *(const float4 *)(p + (KS + q) * F);
                gv = make_float4(gv.x + g2.x, gv.y + g2.y, gv.z + g2.z, gv.w + g2.w);
                uv = make_float4(uv.x + u2.x, uv.y + u2.y, uv.z + u2.z, uv.w + u2.w);
            }
            return make_float4(swiglu(gv.x, uv.x), swiglu(gv.y, uv.y), swiglu(gv.z, uv.z),
                               swiglu(gv.w, uv.w));
        });
        float acc[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i] = 0.0f;
        row_dots<ENC>(wv, dv, b0, nbw, hs, bsum, F, nb, mc, acc);
#pragma unroll
        for (int i = 0; i < MT; i++) red[(w * MT + i) * 64 + lane] = acc[i];
        __syncthreads();
        if (w == 0)
            for (int i = 0; i < mc; i++) {
                float s = 0.0f;
                for (int ww = 0; ww < GW; ww++) s += red[(ww * MT + i) * 64 + lane];
                y[(size_t)list_pair[off + i0 + i] * D + row] = s;
            }
        __syncthreads();
    }
}

/* grid (ceil(D/256), T): mlp[t,i] += wt_j * y_j[i] for j = 0..K-1 (qwen3_moe.c:221), with
   y_j of token t at row t*K + j. */
__global__ __launch_bounds__(256) void k_combine(
    const float *__restrict__ y, const float *__restrict__ wt, int D, int K,
    float *__restrict__ mlp) {
    const int i = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (i >= D) return;
    float yv[MAX_K], wv[MAX_K];
#pragma unroll
    for (int j = 0; j < MAX_K; j++)
        if (j < K) {
            yv[j] = y[((size_t)t * K + j) * D + i];
            wv[j] = wt[(size_t)t * K + j];
        }
    float o = mlp[(size_t)t * D + i];
#pragma unroll
    for (int j = 0; j < MAX_K; j++)
        if (j < K) o = __fadd_rn(o, __fmul_rn(wv[j], yv[j]));
    mlp[(size_t)t * D + i] = o;
}

/* ================================================================ host side */

struct cpg_moe_ws {
    int D, E, K, F, max_T;
    float *xn, *logits, *wt, *gu, *y;
    int *topk, *pair_pos, *list_tok, *list_pair, *grp_expert, *grp_off, *grp_cnt, *n_groups;
    void *block;
};

extern "C" cpg_moe_ws *cpg_moe_ws_create(int D, int E, int K, int F, int max_T) {
    if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return nullptr; }
    if (D <= 0 || E <= 0 || E > MAX_E || K <= 0 || K > MAX_K || K > E || F <= 0 ||
        max_T <= 0 || max_T > BUCKET_MAX_T) {
        cpg_set_error("cpg_moe_ws_create: bad geometry D=%d E=%d K=%d F=%d max_T=%d "
                      "(E <= %d, K <= %d, max_T <= %d)", D, E, K, F, max_T, MAX_E, MAX_K,
                      BUCKET_MAX_T);
        return nullptr;
    }
    cpg_moe_ws *ws = (cpg_moe_ws *)calloc(1, sizeof *ws);
    if (!ws) { cpg_set_error("out of host memory"); return nullptr; }
    ws->D = D; ws->E = E; ws->K = K; ws->F = F; ws->max_T = max_T;
    const size_t TK = (size_t)max_T * K;
    const size_t sz[13] = {(size_t)max_T * D * 4, (size_t)max_T * E * 4, TK * 4,
                           TK * 2 * KS * F * 4, TK * D * 4, TK * 4, TK * 4, TK * 4, TK * 4,
                           (size_t)E * 4, (size_t)E * 4, (size_t)E * 4, 256};
    size_t total = 0;
    for (int i = 0; i < 13; i++) total += cpg_round256(sz[i]);
    uint8_t *p = (uint8_t *)cpg_malloc(total);
    if (!p) { free(ws); return nullptr; }
    ws->block = p;
    void **dst[13] = {(void **)&ws->xn, (void **)&ws->logits, (void **)&ws->wt, (void **)&ws->gu,
                      (void **)&ws->y, (void **)&ws->topk, (void **)&ws->pair_pos,
                      (void **)&ws->list_tok, (void **)&ws->list_pair, (void **)&ws->grp_expert,
                      (void **)&ws->grp_off, (void **)&ws->grp_cnt, (void **)&ws->n_groups};
    for (int i = 0; i < 13; i++) { *dst[i] = p; p += cpg_round256(sz[i]); }
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

static int check_layer(const cpg_moe_layer *L, int T, const cpg_moe_ws *ws) {
    if (!L || !ws || !L->wgate || !L->ln2 || !L->experts) { cpg_set_error("null layer/workspace"); return -1; }
    if (L->enc != CPG_ENC_Q4 && L->enc != CPG_ENC_Q8) { cpg_set_error("expert encoding %d unsupported", L->enc); return -1; }
    if (L->D != ws->D || L->E != ws->E || L->K != ws->K || L->F != ws->F) {
        cpg_set_error("workspace geometry does not match the layer"); return -1;
    }
    if (T <= 0 || T > ws->max_T) { cpg_set_error("T=%d outside [1, %d]", T, ws->max_T); return -1; }
    /* shapes the kernels assume: 64-row tiles; whole 32-element blocks in each of the KS
       k parts; at most MAX_BPW blocks per lane; serial chains over multiples of 64 */
    const int nbd = L->D / KS / 32, nbf = L->F / 32;
    if (L->D % (64 * KS) || L->F % 64 || (nbd + GW - 1) / GW > MAX_BPW ||
        (nbf + GW - 1) / GW > MAX_BPW) {
        cpg_set_error("unsupported shape D=%d F=%d: D a multiple of %d, F of 64, each at most %d",
                      L->D, L->F, 64 * KS, GW * MAX_BPW * 32);
        return -1;
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

    /* routing, selection, bucketing */
    if (T <= SMALL_T) {
        const size_t smem = sizeof(float) * ((size_t)2 * D + (size_t)RPW * (D + 4));
        hipLaunchKernelGGL(k_route_small, dim3((E + RPW - 1) / RPW, T), dim3(256), smem, s, x,
                           attn, L->ln2, L->wgate, D, E, L->eps, xn_d, lg_d);
        CPG_LAUNCH_CHECK("k_route_small");
        hipLaunchKernelGGL(k_select_bucket, dim3(1), dim3(64 * T), 0, s, lg_d, T, E, K, tk_d,
                           wt_d, ws->pair_pos, ws->list_tok, ws->list_pair, ws->grp_expert,
                           ws->grp_off, ws->grp_cnt, ws->n_groups);
        CPG_LAUNCH_CHECK("k_select_bucket");
    } else {
        hipLaunchKernelGGL(k_rmsnorm_lanes, dim3((T + 63) / 64), dim3(64), 0, s, x, attn, L->ln2,
                           T, D, L->eps, xn_d);
        CPG_LAUNCH_CHECK("k_rmsnorm_lanes");
        hipLaunchKernelGGL(k_router_lanes, dim3((T + 63) / 64, E), dim3(64), 0, s, xn_d,
                           L->wgate, T, D, E, lg_d);
        CPG_LAUNCH_CHECK("k_router_lanes");
        hipLaunchKernelGGL(k_select, dim3(T), dim3(64), 0, s, lg_d, E, K, tk_d, wt_d);
        CPG_LAUNCH_CHECK("k_select");
        hipLaunchKernelGGL(k_bucket, dim3(1), dim3(256), 0, s, tk_d, T, K, E, ws->pair_pos,
                           ws->list_tok, ws->list_pair, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups);
        CPG_LAUNCH_CHECK("k_bucket");
    }
    /* expert GEMVs over at most min(E, T*K) groups, then the combine */
    const int gmax = T * K < E ? T * K : E;
    const size_t mg = cpg_matrix_bytes(enc, F, D), es = cpg_expert_bytes(enc, D, F);
    const size_t ppg = cpg_payload_plane(enc, F, D), ppd = cpg_payload_plane(enc, D, F);
    const int ncol = D / KS;
    const size_t smem_gu = sizeof(float) * ((size_t)MT * ncol + MT * (ncol / 32) + GW * MT * 64);
    const size_t smem_dn = sizeof(float) * ((size_t)MT * F + MT * (F / 32) + GW * MT * 64);
    const uint8_t *ex = (const uint8_t *)L->experts;
    if (timing_mark(0)) return -7;
    if (enc == CPG_ENC_Q4)
        hipLaunchKernelGGL(k_gateup<CPG_ENC_Q4>, dim3(F / 64, 2 * KS, gmax), dim3(GW * 64), smem_gu,
                           s, ex, es, mg, ppg, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->list_tok, xn_d, ws->gu);
    else
        hipLaunchKernelGGL(k_gateup<CPG_ENC_Q8>, dim3(F / 64, 2 * KS, gmax), dim3(GW * 64), smem_gu,
                           s, ex, es, mg, ppg, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->n_groups, ws->list_tok, xn_d, ws->gu);
    CPG_LAUNCH_CHECK("k_gateup");
    if (timing_mark(1) || timing_mark(2)) return -7;
    if (enc == CPG_ENC_Q4)
        hipLaunchKernelGGL(k_down<CPG_ENC_Q4>, dim3(D / 64, gmax), dim3(GW * 64), smem_dn, s, ex,
                           es, 2 * mg, ppd, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->list_pair, ws->gu, ws->y);
    else
        hipLaunchKernelGGL(k_down<CPG_ENC_Q8>, dim3(D / 64, gmax), dim3(GW * 64), smem_dn, s, ex,
                           es, 2 * mg, ppd, D, F, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                           ws->list_pair, ws->gu, ws->y);
    CPG_LAUNCH_CHECK("k_down");
    if (timing_mark(3)) return -7;
    hipLaunchKernelGGL(k_combine, dim3((D + 255) / 256, T), dim3(256), 0, s, ws->y, wt_d, D, K,
                       mlp);
    CPG_LAUNCH_CHECK("k_combine");
    return 0;
}
