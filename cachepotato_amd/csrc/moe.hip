/* moe.hip — the MoE half of a Qwen3-30B-A3B decoder layer on gfx950.
 *
 * Reference: engine/blocks/qwen3_moe.c:169-223 (the MoE half of qwen3_layer_kv), with the
 * kernels it calls in engine/kernels/kernels.c (rmsnorm :408-413, matmul_wx :84-95,
 * softmax :20-26, silu :416, matmul_wx_q4 :514-540, matmul_wx_q8 :368-396).
 *
 * One forward of T tokens is three kernels on one stream, no host round trip:
 *   routing        hh = x + attn, xn = rmsnorm(hh), logits = Wgate . xn, softmax, top-K with
 *                  the reference's tie rule, renormalised weights, then the T*K (token, slot)
 *                  pairs grouped by expert so that an expert chosen by several tokens streams
 *                  its weights once.
 *                  Certified (T <= 16, no logits or xn asked for): k_route_fast sums every
 *                  router row in parallel in double and bounds, a posteriori, how far the
 *                  reference's serial float chain can be from that sum. When every gap the
 *                  top-K order depends on is wider than the bounds, the order is provably the
 *                  reference's; otherwise that token is recomputed with the exact chains.
 *                  Exact (logits or xn asked for, or T > 16): the reference's serial add
 *                  chains with separately rounded products, bit-identical logits and xn
 *                  (k_route_small + k_select_bucket, or the per-lane kernels for large T).
 *   experts        one token: k_gateup1 (each workgroup ranks and certifies the router
 *                  records itself, then 32 rows of Wg and Wu of its expert, SwiGLU) and
 *                  k_down1 (all K experts' rows of a 64-row tile of Wd, the weighted combine
 *                  and the residual). 2-63 tokens: k_gateup_mm / k_down_mm, one workgroup per
 *                  (row tile, expert group) with the weights in registers and the group's
 *                  tokens 16 at a time on MFMA; the last of a token's K pairs to finish a
 *                  tile adds mlp += wt_j * y_j for that tile in slot order j = 0..K-1
 *                  (qwen3_moe.c:221). From 64 tokens: the MFMA grouped GEMMs of prefill.hip.
 * Workgroups of one launch hand results to each other only through agent-scope stores and
 * loads plus an arrival counter (see "cross-workgroup handoff"): a device-scope fence on
 * gfx950 writes back or invalidates a whole XCD's L2, which costs more than the work here.
 *
 * The one-token expert GEMVs read the row-tiled layout of cpg.h: lane = row, so a
 * wavefront's load of one block column is one contiguous 1 KiB (Q4) / 2 KiB (Q8) span; the
 * activations come from LDS as wave-uniform (broadcast) reads. A block's dot product is
 * computed on the stored offset values u (Q4: q+8, Q8: q+128) and corrected once:
 * d*(sum u*x - c*sum x). The batch kernels take the MFMA operands of cpg_mfma.h.
 */
#include "cpg_internal.h"
#include "cpg_gemv.h"
#include "cpg_mfma.h"

#include <stdlib.h>
#include <string.h>

#define MAX_K 16
#define SMALL_T 16          /* routing and selection in one workgroup per call up to here */
#define BUCKET_MAX_T 1024   /* k_bucket: 16 chunks of 64 tokens */
#define RPW 4               /* router rows per k_route_small workgroup */
#define KS 2                /* the expert scratch holds TK * 2 * KS * F floats (h; MFMA planes) */
/* k_route_fast: router rows per workgroup, one per wavefront (NQ = D / 256): eight, or four
   where a row's registers would not fit two wavefronts per SIMD */
__host__ __device__ constexpr int route_rows(int nq) { return nq >= 16 ? 4 : 8; }
#define XWAIT_SPINS 4096    /* k_gateup1: polls (of ~512 cycles) for workgroup 0's exact routing */
#define PREFILL_MIN_T 8     /* from this many tokens the experts run as MFMA grouped GEMMs */

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


/* ================================================================ softmax / top-K */

/* One token, one wavefront (all 64 lanes call it). kernels.c:20-26 (max, expf(x - max),
   serial sum, divide) then qwen3_moe.c:184-197 (K passes of a strict-greater scan, the lower
   id wins ties; renormalise by the serial sum of the selected probabilities).
   es: this wavefront's LDS scratch of E entries. */
__device__ __forceinline__ static void select_token(const float *__restrict__ lg, int E, int K,
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
       (p descending, id ascending), a total order. With key = (order-preserving bits of p,
       then ~id) pass j's pick is the largest key not yet taken: K wavefront maxima. p >= 0
       (an expf over a positive sum; + 0.0f folds -0). NaN probabilities, which compare
       false both ways in the scan, take the rank form below. */
    float pk[MAX_E / WAVE];
    bool nan = false;
#pragma unroll
    for (int k = 0; k < MAX_E / WAVE; k++) {
        pk[k] = es[min(lane + WAVE * k, E - 1)] + 0.0f;
        nan |= lane + WAVE * k < E && pk[k] != pk[k];
    }
    int sel[MAX_K];
    if (!__ballot(nan)) {
        unsigned long long key[MAX_E / WAVE];
#pragma unroll
        for (int k = 0; k < MAX_E / WAVE; k++)
            key[k] = lane + WAVE * k < E
                ? ((unsigned long long)ord_f(pk[k]) << 32) | (0xFFFFFFFFu - (unsigned)(lane + WAVE * k))
                : 0ull;
#pragma unroll
        for (int j = 0; j < MAX_K; j++) {
            if (j >= K) continue;
            unsigned long long m = key[0];
#pragma unroll
            for (int k = 1; k < MAX_E / WAVE; k++) m = key[k] > m ? key[k] : m;
            m = wave_max_u64(m);
            sel[j] = (int)(0xFFFFFFFFu - (uint32_t)m);
#pragma unroll
            for (int k = 0; k < MAX_E / WAVE; k++)
                if (key[k] == m) key[k] = 0ull;
        }
    } else {
        /* expert e is picked in pass rank(e) = #{e' : p[e'] > p[e] or (p[e'] == p[e] and
           e' < e)}; the expert of rank j is found with a ballot */
        int rk[MAX_E / WAVE];
#pragma unroll
        for (int k = 0; k < MAX_E / WAVE; k++) {
            const int i = lane + WAVE * k;
            rk[k] = 0x7fffffff;
            if (i < E) {
                int r = 0;
                for (int q = 0; q < E; q++) {
                    const float o = es[q];
                    r += (o > pk[k]) || (o == pk[k] && q < i);
                }
                rk[k] = r;
            }
        }
        unsigned taken = 0;                    /* bit k: expert lane + 64k already selected */
#pragma unroll
        for (int j = 0; j < MAX_K; j++) {
            if (j >= K) continue;
            int cand = -1;
#pragma unroll
            for (int k = 0; k < MAX_E / WAVE; k++)
                if (rk[k] == j && !((taken >> k) & 1u)) cand = lane + WAVE * k;
            const unsigned long long b = __ballot(cand >= 0);
            if (b) {
                sel[j] = __shfl(cand, __ffsll((long long)b) - 1);
            } else {
                /* no expert of rank j: NaN probabilities, which compare false both ways. Take the
                   lowest id not yet selected (the reference's scan keeps its first untaken
                   candidate when every comparison is false), so a token's K experts stay
                   distinct whatever the input. */
                sel[j] = 0;
#pragma unroll
                for (int k = MAX_E / WAVE - 1; k >= 0; k--) {
                    const unsigned long long f =
                        __ballot(lane + WAVE * k < E && !((taken >> k) & 1u));
                    if (f) sel[j] = WAVE * k + __ffsll((long long)f) - 1;
                }
            }
            if (lane == (sel[j] & (WAVE - 1))) taken |= 1u << (sel[j] / WAVE);
        }
    }
    float s = 0.0f;
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < MAX_K; j++)
            if (j < K) s = __fadd_rn(s, es[sel[j]]);
    }
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

/* One wavefront, after bucket_pairs (cnt final): the chunk list of the groups (pf_chunk_list;
   group g is the g-th expert with pairs, in expert order, as bucket_pairs numbers them);
   experts 4t..4t+3 of lane t. */
__device__ static void chunks_of_counts(const int *cnt, int E, int max_chunks, int *chunk_grp,
                                        int *chunk_m0) {
    static_assert(MAX_E / WAVE == 4, "four experts per lane");
    const int t = threadIdx.x;
    int c[4], g[4], lg = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = 4 * t + k;
        c[k] = e < E ? cnt[e] : 0;
        lg += c[k] > 0;
    }
    int pg = lg;
    for (int o = 1; o < WAVE; o <<= 1) {
        const int v = __shfl_up(pg, o);
        if (t >= o) pg += v;
    }
    int gi = pg - lg;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        g[k] = gi;
        gi += c[k] > 0;
    }
    pf_chunk_list(c, g, max_chunks, chunk_grp, chunk_m0);
}

/* grid (ceil(E/RPW), T), 256 threads. Every workgroup of a token computes the token's RMSNorm
   (identical bits; workgroup 0 stores xn): wave 0 lane 0 runs the serial sum of squares
   while waves 1-3 copy the workgroup's RPW router rows into LDS. The rows are multiplied by
   xn in place (the reference's separately rounded products) and lane c of wave 0 runs row
   c's serial add chain. */
__global__ __launch_bounds__(256) void k_route_small(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, int D, int E, float eps, float *__restrict__ xn_out,
    float *__restrict__ logits) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
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
    __shared__ __align__(16) float es[SMALL_T][MAX_E];
    __shared__ unsigned long long mask[MAX_E];
    __shared__ int base[MAX_E], cnt[MAX_E];
    const int t = threadIdx.x >> 6;
    select_token(logits + (size_t)t * E, E, K, topk + (size_t)t * K, wt + (size_t)t * K, es[t]);
    __syncthreads();
    bucket_pairs(topk, T, K, E, mask, base, cnt, pair_pos, list_tok, list_pair, grp_expert,
                 grp_off, grp_cnt, n_groups);
}

/* ================================================================ certified routing */

/* Per (token, expert): the router row's dot product summed in double, and a bound on how far
   the reference's serial float chain can be from it. */
struct route_rec {
    double s;
    float bound;
    int pad;            /* k_route_fast: the bits of the RMSNorm inverse S was formed with */
};

/* One router row in the reference's order, exactly: products of the row (global memory) and
   xn (LDS) rounded separately, added left to right (kernels.c:79). Eight float4 of the row
   are in flight ahead of the chain. D % 32 == 0. */
__device__ static float exact_row_chain(const float *__restrict__ w, const float *xs, int D) {
    const float4 *w4 = (const float4 *)w, *x4 = (const float4 *)xs;
    const int n4 = D / 4;
    float4 buf[8];
#pragma unroll
    for (int j = 0; j < 8; j++) buf[j] = w4[j];
    float acc = 0.0f;
    for (int i = 0; i < n4; i += 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 v = buf[j], xv = x4[i + j];
            if (i + 8 + j < n4) buf[j] = w4[i + 8 + j];
            acc = __fadd_rn(acc, __fmul_rn(v.x, xv.x));
            acc = __fadd_rn(acc, __fmul_rn(v.y, xv.y));
            acc = __fadd_rn(acc, __fmul_rn(v.z, xv.z));
            acc = __fadd_rn(acc, __fmul_rn(v.w, xv.w));
        }
    }
    return acc;
}

#define XCK 32              /* exact router chains: columns per LDS tile */
#define XREG 4              /* exact router chains: float4 of a tile per thread (E*XCK/4 <= XREG*threads) */

/* LDS floats route_exact_token needs: xn, the squares, logits, scratch of E (16-byte aligned),
   two tiles */
static inline size_t exact_route_lds_floats(int D, int E) {
    return (size_t)2 * D + 2 * E + 4 + (size_t)2 * E * (XCK + 1);
}

/* Whole workgroup: all E router rows in the reference's order (exact_row_chain's arithmetic),
   thread r < E running row r's chain over tiles of XCK columns staged in LDS. The tile loads
   are coalesced (the wgate rows lie 4*D bytes apart, so a thread reading its own row would
   pull a separate cache line for every lane) and issued XLA tiles ahead by threads < 256,
   XREG float4 each, into a ring of registers (slot = tile % XLA). tile: 2 * E * (XCK + 1)
   floats. Requires D % (XCK * XLA) == 0, E <= blockDim.x and E * XCK / 4 <= XREG *
   min(256, blockDim.x). */
#define XLA 4
__device__ static void exact_rows_tiled(const float *__restrict__ wgate, const float *xs, int D,
                                        int E, float *tile, float *lg) {
    const int tid = threadIdx.x, nl = min(256, (int)blockDim.x), ld = XCK + 1, q4 = XCK / 4;
    const int nc = D / XCK, nv = E * q4;
    float4 rg[XLA][XREG];
    /* unconditional loads at clamped (always valid) addresses: loads under a branch would
       make the compiler wait for every load in flight where the branches join */
    auto fetch = [&](int c, float4 *r) {
        const int cc = min(c, nc - 1);
#pragma unroll
        for (int q = 0; q < XREG; q++) {
            const int idx = min(tid % nl + q * nl, nv - 1), row = idx / q4, c4 = idx - row * q4;
            r[q] = *(const float4 *)(wgate + (size_t)row * D + (size_t)cc * XCK + 4 * c4);
        }
    };
    auto put = [&](int c, const float4 *r) {
        float *bf = tile + (size_t)(c & 1) * E * ld;
#pragma unroll
        for (int q = 0; q < XREG; q++) {
            const int idx = tid + q * nl;
            if (tid < nl && idx < nv) {
                const int row = idx / q4, c4 = idx - row * q4;
                float *d = bf + row * ld + 4 * c4;
                d[0] = r[q].x; d[1] = r[q].y; d[2] = r[q].z; d[3] = r[q].w;
            }
        }
    };
#pragma unroll
    for (int u = 0; u < XLA; u++) fetch(u, rg[u]);
    put(0, rg[0]);
    fetch(XLA, rg[0]);
    __syncthreads();
    float acc = 0.0f;
    for (int c = 0; c < nc; c += XLA) {
#pragma unroll
        for (int u = 0; u < XLA; u++) {
            const int t = c + u;
            if (tid < E) {
                const float *w = tile + (size_t)((t & 1) * E + tid) * ld;
                float4 xv[XCK / 4];
#pragma unroll
                for (int k = 0; k < XCK / 4; k++) xv[k] = ((const float4 *)(xs + (size_t)t * XCK))[k];
                float wv[XCK];
#pragma unroll
                for (int k = 0; k < XCK; k++) wv[k] = w[k];
#pragma unroll
                for (int k = 0; k < XCK / 4; k++) {
                    acc = __fadd_rn(acc, __fmul_rn(wv[4 * k], xv[k].x));
                    acc = __fadd_rn(acc, __fmul_rn(wv[4 * k + 1], xv[k].y));
                    acc = __fadd_rn(acc, __fmul_rn(wv[4 * k + 2], xv[k].z));
                    acc = __fadd_rn(acc, __fmul_rn(wv[4 * k + 3], xv[k].w));
                }
            }
            if (t + 1 < nc) put(t + 1, rg[(u + 1) % XLA]);
            fetch(t + 1 + XLA, rg[(u + 1) % XLA]);
            __syncthreads();
        }
    }
    if (tid < E) lg[tid] = acc;
}

/* Whole workgroup: token t's routing with the reference's exact arithmetic (the RMSNorm and
   all E router chains serial, then select_token). Used when the certified order could not be
   proved. smem: exact_route_lds_floats(D, E) floats. */
__device__ __forceinline__ static void route_exact_token(const float *__restrict__ xt, const float *__restrict__ at,
                                         const float *__restrict__ ln2,
                                         const float *__restrict__ wgate, int D, int E, int K,
                                         float eps, float *smem, int *topk_row, float *wt_row) {
    __shared__ float inv_s;
    __shared__ int tk_s[MAX_K];
    __shared__ float wt_s[MAX_K];
    float *xs = smem, *sq = xs + D, *lg = sq + D, *es = lg + ((E + 3) & ~3);   /* es 16-byte aligned */
    const int tid = threadIdx.x;
    for (int i = tid; i < D; i += blockDim.x) {
        const float h = __fadd_rn(xt[i], at ? at[i] : 0.0f);
        xs[i] = h;
        sq[i] = __fmul_rn(h, h);
    }
    __syncthreads();
    if (tid == 0) inv_s = rms_inv(chain_lds(0.0f, sq, D), D, eps);
    __syncthreads();
    const float inv = inv_s;
    for (int i = tid; i < D; i += blockDim.x) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), ln2[i]);
    __syncthreads();
    if (D % (XCK * XLA) == 0 && E <= (int)blockDim.x && E * XCK / 4 <= XREG * min(256, (int)blockDim.x))
        exact_rows_tiled(wgate, xs, D, E, es + E, lg);
    else
        for (int r = tid; r < E; r += blockDim.x) lg[r] = exact_row_chain(wgate + (size_t)r * D, xs, D);
    __syncthreads();
    if (tid < WAVE) select_token(lg, E, K, tk_s, wt_s, es);
    __syncthreads();
    if (tid < K) {
        st_agent(&topk_row[tid], tk_s[tid]);
        st_agent(&wt_row[tid], wt_s[tid]);
    }
}

/* grid (ceil(E/R), T), 64 * R threads with R = route_rows(NQ), T <= SMALL_T, D = 256 * NQ.
 *
 * Wavefront w of workgroup b handles router row e = b*R + w of token t. Every lane
 * holds D/64 consecutive elements of hh = x + attn and of the row. The RMSNorm sum of squares
 * is taken in double (the products rounded as the reference rounds them), xn is formed as the
 * reference forms it from that inv, and the row's products p_k = fl(w_k * xn_k) are summed in
 * double together with every prefix S_k.
 *
 * Why the order is the reference's. Let inv' be the reference's 1/sqrt (from its float chain)
 * and 1 + r = inv'/inv. Its xn differs from ours by the common factor (1 + r) and at most
 * 4 roundings per element, so its products are (1 + r) p_k (1 + psi_k), |psi_k| < 2^-21. Its
 * serial chain adds a rounding error of at most 2^-24 |acc_k| at step k. Hence
 *   |l_ref - (1 + r) S| <= (1 + r) (2^-21 sum|p_k| + 1.0003 * 2^-24 sum|S_k|) + tiny = B,
 * a bound computed here from the same sums. A common factor 1 + r > 0 does not change an
 * order, so only the gaps matter. The reference ranks by p = fl(expf(fl(l - max)) / sum):
 * two logits more than 2^-20 + 2^-23 (|l_a - max| + |l_b - max|) apart give distinct p in the
 * same order (subtraction error 2^-24 relative, expf error under one ulp, quotients 2^-21
 * apart stay ordered after rounding). The last workgroup of the token takes the top K by
 * (S desc, id asc) and checks that each one's lower bound S - B beats the largest upper bound
 * S + B of every expert after it (the later selected ones and all unselected) by that margin,
 * 1% wider; if any gap is too narrow (or anything is not finite, or the sum of squares is near the
 * float range limits), the token's routing is recomputed exactly. The renormalised weights
 * are formed from the certified logits (within a few ulps of the reference's).
 *
 * The last token's last workgroup then groups the pairs by expert. */
/* One router row of one token, one wavefront (the first phase of k_route_fast): every lane
   holds D/64 consecutive elements of hh = x + attn and of the row w (D = 256 * NQ). The
   RMSNorm sum of squares is taken in double, xn is formed from that inverse as the reference
   forms it, and the row's products are summed in double with every prefix; *S_out and *B_out
   (lane 0) receive the sum and the certified bound on the reference's serial chain (see
   k_route_fast), *inv_out (when not null) the RMSNorm inverse the products were formed
   with. xo not null: each lane writes its xn elements there. */
template <int NQ>
__device__ static inline void route_row_core(const float4 (&h)[NQ], const float4 (&wr)[NQ],
                                             const float4 (&gq)[NQ], int D, float eps,
                                             float4 *xo, double *S_out, float *B_out,
                                             float *inv_out, _Float16 *xh = nullptr,
                                             _Float16 *xl = nullptr);

template <int NQ>
__device__ static inline void route_row(const float *__restrict__ xt, const float *__restrict__ at,
                                        const float *__restrict__ ln2,
                                        const float *__restrict__ wrow, int D, float eps,
                                        float4 *xo, double *S_out, float *B_out,
                                        float *inv_out = nullptr) {
    const int lane = threadIdx.x & 63, nq = NQ;
    const float4 *x4 = (const float4 *)xt + lane * nq;
    const float4 *a4 = at ? (const float4 *)at + lane * nq : nullptr;
    const float4 *w4 = (const float4 *)wrow + lane * nq;
    const float4 *g4 = (const float4 *)ln2 + lane * nq;
    /* every load at once, unconditionally (attn's slot reads x again when there is no attn):
       a load under a branch, or one after the xo stores below, would be a round trip of its
       own */
    const float4 *a4s = a4 ? a4 : x4;
    float4 h[NQ], wr[NQ], gq[NQ], av[NQ];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        h[q] = x4[q];
        wr[q] = w4[q];
        gq[q] = g4[q];
        av[q] = a4s[q];
    }
    if (a4) {
#pragma unroll
        for (int q = 0; q < NQ; q++)
            h[q] = make_float4(__fadd_rn(h[q].x, av[q].x), __fadd_rn(h[q].y, av[q].y),
                               __fadd_rn(h[q].z, av[q].z), __fadd_rn(h[q].w, av[q].w));
    }
    route_row_core<NQ>(h, wr, gq, D, eps, xo, S_out, B_out, inv_out);
}

/* route_row's arithmetic once the lane's elements of hh (h), of the row (wr) and of ln2 (gq)
   are in registers. xo and xh not null: xn is also written as hi/lo f16 planes xh / xl (hi =
   f16(v), lo = f16(v - hi)), from the registers. */
template <int NQ>
__device__ static inline void route_row_core(const float4 (&h)[NQ], const float4 (&wr)[NQ],
                                             const float4 (&gq)[NQ], int D, float eps,
                                             float4 *xo, double *S_out, float *B_out,
                                             float *inv_out, _Float16 *xh, _Float16 *xl) {
    const int lane = threadIdx.x & 63, nq = NQ;
    double ss = 0.0;
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        ss += (double)__fmul_rn(h[q].x, h[q].x);
        ss += (double)__fmul_rn(h[q].y, h[q].y);
        ss += (double)__fmul_rn(h[q].z, h[q].z);
        ss += (double)__fmul_rn(h[q].w, h[q].w);
    }
    ss = wave_sum_d(ss);
    const float inv = rms_inv((float)ss, D, eps);
    float p[4 * NQ];
    double tl = 0.0, P = 0.0;
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const float4 g = gq[q];
        const float4 v = make_float4(__fmul_rn(__fmul_rn(h[q].x, inv), g.x),
                                     __fmul_rn(__fmul_rn(h[q].y, inv), g.y),
                                     __fmul_rn(__fmul_rn(h[q].z, inv), g.z),
                                     __fmul_rn(__fmul_rn(h[q].w, inv), g.w));
        if (xo) {
            xo[lane * nq + q] = v;
            if (xh) {
                typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
                const float vv[4] = {v.x, v.y, v.z, v.w};
                half4_t hi, lo;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const f16pair sp = split_f16(vv[c]);
                    hi[c] = sp.hi;
                    lo[c] = sp.lo;
                }
                *(half4_t *)(xh + 4 * (lane * nq + q)) = hi;
                *(half4_t *)(xl + 4 * (lane * nq + q)) = lo;
            }
        }
        p[4 * q + 0] = __fmul_rn(wr[q].x, v.x);
        p[4 * q + 1] = __fmul_rn(wr[q].y, v.y);
        p[4 * q + 2] = __fmul_rn(wr[q].z, v.z);
        p[4 * q + 3] = __fmul_rn(wr[q].w, v.w);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            tl += (double)p[4 * q + c];
            P += fabs((double)p[4 * q + c]);
        }
    }
    double S = wave_incl_scan_d(tl) - tl, A = 0.0;
#pragma unroll
    for (int q = 0; q < NQ; q++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            S += (double)p[4 * q + c];
            A += fabs(S);
        }
    }
    S = readlane_d(S, WAVE - 1);           /* the last lane's last prefix is the sum */
    A = wave_sum_d(A);
    P = wave_sum_d(P);
    double bound = 1.01 * (0x1p-21 * P + 1.0003 * 0x1p-24 * A) + D * 0x1p-148 +
                   0x1p-40 * (P + fabs(S));
    /* near the float range limits the reference's chain may overflow or lose precision */
    if (!(ss < 1e37) || !(ss > 1e-30)) bound = INFINITY;
    *S_out = S;
    *B_out = (float)(bound * (1.0 + 0x1p-20));
    if (inv_out) *inv_out = inv;
}

/* The RMSNorm inverse of route_row for hh = x + attn, the same bits: one wavefront. */
template <int NQ>
__device__ static inline float route_inv(const float *__restrict__ xt, const float *__restrict__ at,
                                         int D, float eps) {
    const int lane = threadIdx.x & 63;
    const float4 *x4 = (const float4 *)xt + lane * NQ;
    const float4 *a4 = (const float4 *)(at ? at : xt) + lane * NQ;   /* unconditional loads */
    float4 xv[NQ], av[NQ];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        xv[q] = x4[q];
        av[q] = a4[q];
    }
    double ss = 0.0;
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        float4 h = xv[q];
        if (at)
            h = make_float4(__fadd_rn(h.x, av[q].x), __fadd_rn(h.y, av[q].y),
                            __fadd_rn(h.z, av[q].z), __fadd_rn(h.w, av[q].w));
        ss += (double)__fmul_rn(h.x, h.x);
        ss += (double)__fmul_rn(h.y, h.y);
        ss += (double)__fmul_rn(h.z, h.z);
        ss += (double)__fmul_rn(h.w, h.w);
    }
    ss = wave_sum_d(ss);
    return rms_inv((float)ss, D, eps);
}

/* LDS of the top-K certification (cert_rank, cert_check). */
struct cert_lds {
    double cS[MAX_E];
    float cB[MAX_E];
    __align__(16) uint32_t ckey[MAX_E];
    int crank[MAX_E];
    int cslot[MAX_K];
    double slS[MAX_K], slH[MAX_K];
    float slB[MAX_K];
    unsigned long long chr;
    int bad;                /* cert_check: some gap too narrow */
};

/* The whole workgroup (any multiple of 64 threads), first half of the certified top-K of one
   token from its E records (see k_route_fast): ranks the experts and leaves, in c, the
   selection in slot order (cslot[0..K)) with its S, B and S + B, and the largest upper bound
   S + B among the experts not selected (chr). Returns whether any record was not finite
   (the same value in every thread); ends with the workgroup synchronised. nt: the
   workgroup's thread count (a constant of the caller: blockDim would be a memory load).

   Experts are ranked by a 32-bit key (S desc, id asc): the top 24 bits of S as a float
   (relative resolution 2^-15), 255 - id below. Experts closer than that may come out in id
   order; the certificate compares the true S and bounds of every expert, so such an order
   can only fail certification, never pass wrongly. Each expert's rank is the number of keys
   above its own (the keys are distinct), counted by all threads in parallel; rank j < K is
   slot j. */
/* expert e's record (S, B) into c for cert_rank_tail; returns whether both are finite */
__device__ static inline bool cert_put(cert_lds &c, int e, double s, float bd) {
    c.cS[e] = s;
    c.cB[e] = bd;
    c.ckey[e] = (ord_f((float)s) & ~0xFFu) | (uint32_t)(255 - e);
    c.crank[e] = 0;
    return isfinite(s) && isfinite(bd);
}

__device__ static bool cert_rank_tail(cert_lds &c, int E, int K, int nt, bool finite);

/* k_gateup1's form of cert_rank and cert_check, arranged so that the weight loads issue as
   soon as the slot's expert is known and nothing after them waits at a barrier: a barrier
   there would wait until every wavefront of the workgroup had issued all its loads, which,
   with the memory pipeline full, is about when the last of them land.
   cert_rank_open: thread tid < E puts its record r (expert tid, E <= nt); then each expert's
   rank is counted by CR_P consecutive threads over CR_P parts of the keys and summed by DPP,
   and the thread holding the sum writes the expert's slot entry (rank < K: cslot, slS, slB,
   slH) or takes part in chr (the largest S + B not selected), each expert from its own rank
   alone. The caller stages what else it needs into LDS and calls cert_rank_close (the
   second barrier); cslot[] then holds the selection in slot order. *nonfinite: some record
   not finite (the same in every thread). Requires nt >= CR_P * E. */
#define CR_P 4
__device__ static void cert_rank_open(cert_lds &c, v4i_t r, int E, int K, int nt,
                                      bool *nonfinite) {
    __shared__ int nfw[16];
    const int tid = threadIdx.x, lane = tid & 63, len = (E + 16 * CR_P - 1) / (16 * CR_P) * 16;
    if (tid == 0) c.chr = 0ull;
    bool finite = true;
    if (tid < E) {
        const double s = __longlong_as_double(((long long)(uint32_t)r.y << 32) | (uint32_t)r.x);
        finite = cert_put(c, tid, s, __int_as_float(r.z));
    }
    for (int e = E + tid; e < CR_P * len; e += nt) c.ckey[e] = 0u;
    if (lane == 0) nfw[tid >> 6] = __ballot(!finite) != 0ull;
    lds_barrier();
    const int e = tid / CR_P, part = tid % CR_P;
    int n = 0;
    if (e < E) {
        const uint32_t k = c.ckey[e];
        const uint4 *kp = (const uint4 *)(c.ckey + part * len);
        for (int q0 = 0; q0 < len / 4; q0 += 4) {
            uint4 a[4];
#pragma unroll
            for (int q = 0; q < 4; q++) a[q] = kp[q0 + q];
#pragma unroll
            for (int q = 0; q < 4; q++)
                n += (int)(a[q].x > k) + (int)(a[q].y > k) + (int)(a[q].z > k) + (int)(a[q].w > k);
        }
    }
    n += __builtin_amdgcn_update_dpp(0, n, DPP_QUAD_1032, 0xf, 0xf, false);
    n += __builtin_amdgcn_update_dpp(0, n, DPP_QUAD_2301, 0xf, 0xf, false);
    unsigned long long u = 0ull;
    if (e < E && part == 0) {
        const double se = c.cS[e];
        const float bf = c.cB[e];
        const double hs = se + (double)bf;
        if (n < K) {
            c.cslot[n] = e;
            c.slS[n] = se;
            c.slB[n] = bf;
            c.slH[n] = hs;
        } else {
            u = ord_d(hs);
        }
    }
    u = wave_max_u64(u);
    if (lane == 0 && u) atomicMax(&c.chr, u);
    bool nf = false;
    for (int v = 0; v < (nt + 63) / 64; v++) nf = nf || nfw[v];
    *nonfinite = nf;
}

__device__ static inline void cert_rank_close() { lds_barrier(); }

/* cert_check's test and weights, one wavefront on its own (no barrier): whether the order
   in c is certified (the same in every lane); if so and tk is not null, lanes j < K write
   tk[j] / wt[j] (global memory). */
__device__ static bool cert_check_wave(const cert_lds &c, int K, bool nonfinite,
                                       int force_exact, int *tk, float *wt,
                                       int *tk2 = nullptr, float *wt2 = nullptr) {
    const int lane = threadIdx.x & 63;
    bool good = true;
    double sj = 0.0, s0 = 0.0;
    if (lane < K) {
        s0 = c.slS[0];
        sj = c.slS[lane];
        const double b0 = (double)c.slB[0], bj = (double)c.slB[lane];
        double hi_after = c.chr ? unord_d(c.chr) : -INFINITY;
#pragma unroll
        for (int i = 1; i < MAX_K; i++)
            if (i > lane && i < K) {
                const double hi = c.slH[i];
                hi_after = hi > hi_after ? hi : hi_after;
            }
        const double lo = sj - bj;
        if (hi_after != -INFINITY) {
            const double need = 1.01 * (0x1p-20 + 0x1p-23 * (fabs(sj - s0) +
                                        fabs(hi_after - s0) + 2.0 * (bj + b0)));
            good = lo - hi_after > need;
        }
        good = good && (s0 + b0) - lo < 80.0;
    }
    const bool ok = __ballot(!good) == 0ull && !nonfinite && !force_exact;
    if (ok && (tk || tk2)) {
        const float ev = lane < K ? cpg_expf(__fsub_rn((float)sj, (float)s0)) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < K; j++)
            sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j)));
        if (lane < K) {
            const float wj = __fdiv_rn(ev, sum);
            if (tk) {
                tk[lane] = c.cslot[lane];
                wt[lane] = wj;
            }
            if (tk2) {
                tk2[lane] = c.cslot[lane];
                wt2[lane] = wj;
            }
        }
    }
    return ok;
}

__device__ static bool cert_rank(cert_lds &c, const route_rec *rec, int E, int K, int nt) {
    const int tid = threadIdx.x;
    if (tid == 0) c.chr = 0ull;
    bool finite = true;
    for (int e = tid; e < E; e += nt) {
        const v4i_t r = ld_agent16(rec, (uint32_t)(e * sizeof(route_rec)));
        const double s = __longlong_as_double(((long long)(uint32_t)r.y << 32) | (uint32_t)r.x);
        finite = cert_put(c, e, s, __int_as_float(r.z)) && finite;
    }
    return cert_rank_tail(c, E, K, nt, finite);
}

/* The rest of cert_rank, once every expert's record is in c (cert_put) and c.chr is zero:
   finite says whether this thread's records were finite. */
__device__ static bool cert_rank_tail(cert_lds &c, int E, int K, int nt, bool finite) {
    const int tid = threadIdx.x, lane = tid & 63;
    /* P threads per expert, each counting over len keys (a multiple of 16, the keys past E
       zero, which is below every key): P <= 4 keeps P * len <= MAX_E */
    const int P = min(4, max(1, nt / E)), len = (E + 16 * P - 1) / (16 * P) * 16;
    for (int e = E + tid; e < P * len; e += nt) c.ckey[e] = 0u;
    if (tid == 0) c.bad = 0;
    const bool nonfinite = __syncthreads_or(!finite) != 0;
    /* rank = the number of keys above the expert's own; 16 keys per round of independent
       128-bit LDS reads (the same address across a wavefront when E % 64 == 0) */
    for (int idx = tid; idx < E * P; idx += nt) {
        const int e = idx % E, part = idx / E;
        const uint32_t k = c.ckey[e];
        const uint4 *kp = (const uint4 *)(c.ckey + part * len);
        int n = 0;
        for (int q0 = 0; q0 < len / 4; q0 += 4) {
            uint4 a[4];
#pragma unroll
            for (int q = 0; q < 4; q++) a[q] = kp[q0 + q];
#pragma unroll
            for (int q = 0; q < 4; q++)
                n += (int)(a[q].x > k) + (int)(a[q].y > k) + (int)(a[q].z > k) + (int)(a[q].w > k);
        }
        atomicAdd(&c.crank[e], n);
    }
    __syncthreads();
    /* the selected in slot order with their S, B and S + B; the largest upper bound S + B
       among the experts not selected */
    unsigned long long u = 0ull;
    for (int e = tid; e < E; e += nt) {
        const int r = c.crank[e];
        const double se = c.cS[e], be = (double)c.cB[e];
        if (r < K) {
            c.cslot[r] = e;
            c.slS[r] = se;
            c.slB[r] = c.cB[e];
            c.slH[r] = se + be;
        } else {
            const unsigned long long o = ord_d(se + be);
            u = o > u ? o : u;
        }
    }
    u = wave_max_u64(u);
    if (lane == 0 && u) atomicMax(&c.chr, u);
    __syncthreads();
    return nonfinite;
}

/* The whole workgroup, second half: whether the ranking in c is certified (the same value in
   every thread); if so tk[0..K) and wt[0..K) (LDS, written by threads < K) receive the
   selection and its renormalised weights. tab: the expf table in LDS. */
__device__ static bool cert_check(cert_lds &c, int K, bool nonfinite, int force_exact,
                                  const uint64_t *tab, int *tk, float *wt) {
    const int tid = threadIdx.x, lane = tid & 63;
    /* Thread j < K: expert j is certainly ranked above every expert after it (the later
       selected ones and all unselected) when its lower bound beats their largest upper
       bound by the margin. */
    bool good = true;
    double sj = 0.0, s0 = 0.0;
    if (tid < K) {
        s0 = c.slS[0];
        sj = c.slS[tid];
        const double b0 = (double)c.slB[0], bj = (double)c.slB[tid];
        double hi_after = c.chr ? unord_d(c.chr) : -INFINITY;
#pragma unroll
        for (int i = 1; i < MAX_K; i++)
            if (i > tid && i < K) {
                const double hi = c.slH[i];
                hi_after = hi > hi_after ? hi : hi_after;
            }
        const double lo = sj - bj;
        if (hi_after != -INFINITY) {
            const double need = 1.01 * (0x1p-20 + 0x1p-23 * (fabs(sj - s0) +
                                        fabs(hi_after - s0) + 2.0 * (bj + b0)));
            good = lo - hi_after > need;
        }
        good = good && (s0 + b0) - lo < 80.0;
    }
    /* the workgroup's verdict through LDS, without waiting for global loads in flight (the
       expert kernel's weights): see lds_barrier */
    if (!good) c.bad = 1;
    lds_barrier();
    const bool ok = !c.bad && !nonfinite && !force_exact;
    if (ok && tid < 64) {
        /* wt_j = p_j / sum_i p_i over the selection, with p_j proportional to
           expf(l_j - l_0); the full softmax denominator cancels */
        const float ev = lane < K ? cpg_expf_tab(__fsub_rn((float)sj, (float)s0), tab) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < K; j++)
            sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j)));
        if (lane < K) {
            tk[lane] = c.cslot[lane];
            wt[lane] = __fdiv_rn(ev, sum);
        }
    }
    return ok;
}

/* ---- the refined fallback: exact chains for the candidates only
 * When the bounds cannot certify a token's order, most experts are still certainly out of
 * the top K; only those whose upper bound reaches the K-th largest lower bound (within
 * RF_SLACK) can be in it. The reference's xn is formed exactly (its serial sum of squares),
 * then the exact logits of those candidates only (their serial chains, products formed by the
 * loading threads), and the order is certified again: consecutive candidates by the softmax
 * margin, the K-th against the largest upper bound of the rest, moved to the reference's
 * scale by inv'/inv (the two RMSNorm inverses; see k_route_fast). Certified: topk and the
 * renormalised weights from the exact logits (a few ulps from the reference's, as the
 * certified path's). Otherwise the exact chains for every row (route_exact_token). */
#define RF_CMAX 16          /* candidates at most */
#define RF_XC 256           /* columns per product tile */
#define RF_LA 3             /* tiles of row loads in flight ahead of the one being put */
#define RF_NH 192           /* loading threads: 64 .. 255 (wavefronts 1-3) */
#define RF_RG 6             /* float4 of a tile per loading thread: RF_CMAX * RF_XC / 4 / RF_NH */
#define RF_V4 2             /* float4 of the token held per thread */
#define RF_SLACK(t) (1e-4 + 1e-5 * fabs(t))

/* LDS floats route_refine needs: hh / xn, the squares, the candidate list and logits, two
   product tiles */
static inline size_t refine_lds_floats(int D) {
    return (size_t)2 * D + 2 * RF_CMAX + 8 + (size_t)2 * RF_CMAX * (RF_XC + 4);
}
/* what the fallback of the certified path needs (refined, then possibly exact) */
static inline size_t fallback_lds_floats(int D, int E) {
    const size_t a = exact_route_lds_floats(D, E), b = refine_lds_floats(D);
    return a > b ? a : b;
}

/* Whole workgroup (blockDim.x >= 256, D % RF_XC == 0): token xt's refined routing (see
   above) from c's records and slots (cS, cB of every expert, all finite; slS, slB of the K
   experts the certification ranked first) and inv, the RMSNorm inverse the records were
   formed with. Returns whether the order was certified (the same in every thread); if so,
   topk_row / wt_row are written (agent-scope stores). smem: refine_lds_floats(D) floats.
   The latency is the two serial sums of 2048-odd adds, so everything else runs beside them:
     A  every thread: its part of hh = x + attn and of the squares into LDS, of ln2 into
        registers; wavefront 1: the candidates, from thr = the smallest lower bound among
        the K ranked first (no larger than the K-th largest lower bound, so the candidates
        are a superset of those whose bounds reach it);
     B  wavefront 0, lane 0: the serial sum of squares and the reference's inverse inv';
        wavefronts 1-3: the first RF_LA tiles of the candidates' rows into registers;
     C  every thread: the reference's xn = (hh * inv') * ln2 into LDS;
     D  per tile of RF_XC columns: wavefronts 1-3 put the products fl(w * xn) into LDS and
        fetch RF_LA tiles ahead; lane i < nc of wavefront 0 adds its row's products in order;
     E  wavefront 0: the candidates ordered by (exact logit desc, id asc) and certified. */
__device__ static bool route_refine(const float *__restrict__ xt, const float *__restrict__ at,
                                    const float *__restrict__ ln2, const float *__restrict__ wgate,
                                    int D, int E, int K, float eps, float *smem, const cert_lds &c,
                                    float inv, int *topk_row, float *wt_row) {
    __shared__ float invr_s;
    __shared__ unsigned long long hrest_s;
    __shared__ int nc_s, ok_s;
    __shared__ uint64_t etab[32];
    float *xs = smem, *sq = xs + D;
    int *cidx = (int *)(sq + D);
    float *lg = (float *)(cidx + RF_CMAX), *tile = lg + RF_CMAX + 8;
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, w = tid >> 6, n4 = D / 4;
    const int q4 = RF_XC / 4, ntile = D / RF_XC, ld = RF_XC + 4, th = tid - WAVE;
    const bool helper = w >= 1 && w <= 3;
    /* ---- A */
    if (tid < 32) etab[tid] = cpg_exp2f_tab[tid];
    float4 g4[RF_V4];
#pragma unroll
    for (int r = 0; r < RF_V4; r++) {
        const int i = tid + r * nt;
        g4[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < n4) {
            float4 h = ((const float4 *)xt)[i];
            g4[r] = ((const float4 *)ln2)[i];
            if (at) {
                const float4 a = ((const float4 *)at)[i];
                h = make_float4(__fadd_rn(h.x, a.x), __fadd_rn(h.y, a.y), __fadd_rn(h.z, a.z),
                                __fadd_rn(h.w, a.w));
            }
            ((float4 *)xs)[i] = h;
            ((float4 *)sq)[i] = make_float4(__fmul_rn(h.x, h.x), __fmul_rn(h.y, h.y),
                                            __fmul_rn(h.z, h.z), __fmul_rn(h.w, h.w));
        }
    }
    for (int i = tid + RF_V4 * nt; i < n4; i += nt) {
        float4 h = ((const float4 *)xt)[i];
        if (at) {
            const float4 a = ((const float4 *)at)[i];
            h = make_float4(__fadd_rn(h.x, a.x), __fadd_rn(h.y, a.y), __fadd_rn(h.z, a.z),
                            __fadd_rn(h.w, a.w));
        }
        ((float4 *)xs)[i] = h;
        ((float4 *)sq)[i] = make_float4(__fmul_rn(h.x, h.x), __fmul_rn(h.y, h.y),
                                        __fmul_rn(h.z, h.z), __fmul_rn(h.w, h.w));
    }
    if (w == 1) {
        /* the candidates in id order; the largest upper bound among the rest */
        double thr = INFINITY;
        for (int j = 0; j < K; j++) {
            const double lo = c.slS[j] - (double)c.slB[j];
            thr = lo < thr ? lo : thr;
        }
        const double cut = thr - RF_SLACK(thr);
        int n = 0;
        unsigned long long hr = 0ull;
        for (int e0 = 0; e0 < E; e0 += WAVE) {
            const int e = e0 + lane;
            bool cand = false;
            if (e < E) {
                const double hi = c.cS[e] + (double)c.cB[e];
                cand = hi >= cut;
                if (!cand) {
                    const unsigned long long o = ord_d(hi);
                    hr = o > hr ? o : hr;
                }
            }
            const unsigned long long bal = __ballot(cand);
            const int pos = n + __popcll(bal & ((1ull << lane) - 1ull));
            if (cand && pos < RF_CMAX) cidx[pos] = e;
            n += __popcll(bal);
        }
        hr = wave_max_u64(hr);
        if (lane == 0) {
            nc_s = n;
            hrest_s = hr;
        }
    }
    __syncthreads();
    const int nc = nc_s;
    if (nc > RF_CMAX || nc < K) return false;      /* the same in every thread */
    /* ---- B */
    const int nv = nc * q4;
    float4 rg[RF_LA][RF_RG];
    /* unconditional loads at clamped (always valid) addresses */
    auto fetch = [&](int t, float4 *r) {
        const int tt = min(t, ntile - 1);
#pragma unroll
        for (int q = 0; q < RF_RG; q++) {
            const int idx = min(th + q * RF_NH, nv - 1), row = idx / q4, c4 = idx - row * q4;
            r[q] = *(const float4 *)(wgate + (size_t)cidx[row] * D + (size_t)tt * RF_XC + 4 * c4);
        }
    };
    auto put = [&](int t, const float4 *r) {
        float *bf = tile + (size_t)(t & 1) * RF_CMAX * ld;
#pragma unroll
        for (int q = 0; q < RF_RG; q++) {
            const int idx = th + q * RF_NH;
            if (idx < nv) {
                const int row = idx / q4, c4 = idx - row * q4;
                const float4 x4 = *(const float4 *)(xs + (size_t)t * RF_XC + 4 * c4);
                *(float4 *)(bf + row * ld + 4 * c4) =
                    make_float4(__fmul_rn(r[q].x, x4.x), __fmul_rn(r[q].y, x4.y),
                                __fmul_rn(r[q].z, x4.z), __fmul_rn(r[q].w, x4.w));
            }
        }
    };
    if (w == 0) {
        if (lane == 0) invr_s = rms_inv(chain_lds(0.0f, sq, D), D, eps);
    } else if (helper) {
#pragma unroll
        for (int u = 0; u < RF_LA; u++) fetch(u, rg[u]);
    }
    __syncthreads();
    /* ---- C */
    const float invr = invr_s;
#pragma unroll
    for (int r = 0; r < RF_V4; r++) {
        const int i = tid + r * nt;
        if (i < n4) {
            const float4 h = ((const float4 *)xs)[i];
            ((float4 *)xs)[i] = make_float4(__fmul_rn(__fmul_rn(h.x, invr), g4[r].x),
                                            __fmul_rn(__fmul_rn(h.y, invr), g4[r].y),
                                            __fmul_rn(__fmul_rn(h.z, invr), g4[r].z),
                                            __fmul_rn(__fmul_rn(h.w, invr), g4[r].w));
        }
    }
    for (int i = tid + RF_V4 * nt; i < n4; i += nt) {
        const float4 h = ((const float4 *)xs)[i], g = ((const float4 *)ln2)[i];
        ((float4 *)xs)[i] = make_float4(__fmul_rn(__fmul_rn(h.x, invr), g.x),
                                        __fmul_rn(__fmul_rn(h.y, invr), g.y),
                                        __fmul_rn(__fmul_rn(h.z, invr), g.z),
                                        __fmul_rn(__fmul_rn(h.w, invr), g.w));
    }
    __syncthreads();
    /* ---- D */
    if (helper) {
        put(0, rg[0]);
        fetch(RF_LA, rg[0]);
    }
    __syncthreads();
    float acc = 0.0f;
    for (int t0 = 0; t0 < ntile; t0 += RF_LA) {
#pragma unroll
        for (int u = 0; u < RF_LA; u++) {
            const int t = t0 + u;
            if (t < ntile) {
                if (w == 0 && lane < nc) {
                    acc = chain_lds(acc, tile + (size_t)((t & 1) * RF_CMAX + lane) * ld, RF_XC);
                } else if (helper) {
                    if (t + 1 < ntile) put(t + 1, rg[(u + 1) % RF_LA]);
                    fetch(t + 1 + RF_LA, rg[(u + 1) % RF_LA]);
                }
                __syncthreads();
            }
        }
    }
    if (w == 0 && lane < nc) lg[lane] = acc;
    /* ---- E: wavefront 0 alone from here (its own LDS writes are ordered before its reads) */
    if (w == 0) {
        wave_lds_sync();
        /* candidate order by (logit desc, id asc): lane i's rank, then position r's lane */
        float lv[RF_CMAX];
        int iv[RF_CMAX];
#pragma unroll
        for (int q = 0; q < RF_CMAX / 4; q++) {
            const float4 a = ((const float4 *)lg)[q];
            const int4 b = ((const int4 *)cidx)[q];
            lv[4 * q] = a.x; lv[4 * q + 1] = a.y; lv[4 * q + 2] = a.z; lv[4 * q + 3] = a.w;
            iv[4 * q] = b.x; iv[4 * q + 1] = b.y; iv[4 * q + 2] = b.z; iv[4 * q + 3] = b.w;
        }
        const float li = lane < nc ? lg[lane] : 0.0f;
        const int ei = lane < nc ? cidx[lane] : 0;
        int rk = 0;
#pragma unroll
        for (int j = 0; j < RF_CMAX; j++)
            rk += (int)(j < nc && (lv[j] > li || (lv[j] == li && iv[j] < ei)));
        bool good = lane >= nc || isfinite(li);
        const int nr = min(nc, K + 1);
        float lr[MAX_K + 1];
        int er[MAX_K + 1];
#pragma unroll
        for (int r = 0; r <= MAX_K; r++) {
            lr[r] = 0.0f;
            er[r] = 0;
            if (r < nr) {
                const unsigned long long b = __ballot(lane < nc && rk == r);
                const int src = b ? __ffsll((long long)b) - 1 : 0;
                lr[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(li), src));
                er[r] = __builtin_amdgcn_readlane(ei, src);
            }
        }
        /* the certificate: consecutive positions 0..K apart by the softmax margin, position
           K - 1 above the rest's largest upper bound (in the reference's scale) */
        const double mx = (double)lr[0];
        const double ratio = (double)invr / (double)inv;
        const unsigned long long hr = hrest_s;
        double hrest = -INFINITY;
        if (hr) {
            const double h0 = unord_d(hr) * ratio;
            hrest = h0 + 0x1p-40 * fabs(h0);
        }
        auto apart = [&](double a, double b) {
            return a - b > 1.01 * (0x1p-20 + 0x1p-23 * (fabs(a - mx) + fabs(b - mx)));
        };
        if (lane < K) {
            double cur = (double)lr[0];
#pragma unroll
            for (int r = 1; r < MAX_K; r++)
                if (r == lane) cur = (double)lr[r];
            double nxt = -INFINITY;
#pragma unroll
            for (int r = 1; r <= MAX_K; r++)
                if (r == lane + 1 && r < nr) nxt = (double)lr[r];
            if (lane + 1 < nr) good = good && apart(cur, nxt);
            if (lane == K - 1 && hrest != -INFINITY) good = good && apart(cur, hrest);
            good = good && mx - cur < 80.0 && isfinite(ratio);
        }
        const bool ok = __ballot(!good) == 0ull;
        if (ok) {
            float lj = 0.0f;
            int ej = 0;
#pragma unroll
            for (int r = 0; r < MAX_K; r++)
                if (r == lane) { lj = lr[r]; ej = er[r]; }
            const float ev = lane < K ? cpg_expf_tab(__fsub_rn(lj, lr[0]), etab) : 0.0f;
            float sum = 0.0f;
            for (int j = 0; j < K; j++)
                sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j)));
            if (lane < K) {
                st_agent(&topk_row[lane], ej);
                st_agent(&wt_row[lane], __fdiv_rn(ev, sum));
            }
        }
        if (lane == 0) ok_s = ok;
    }
    __syncthreads();
    return ok_s != 0;
}

/* The fallback of the certified path for one token (whole workgroup): the refined routing
   when it certifies the order, else the exact chains for every row. force == 1 skips the
   refined step (CPG_ROUTE_FORCE_FALLBACK); a NaN inv (no inverse recorded) too. Returns
   whether the exact chains ran. smem: fallback_lds_floats(D, E) floats. */
#define FORCE_EXACT_CHAINS 1
__device__ __forceinline__ static bool route_fallback(const float *__restrict__ xt,
                                                      const float *__restrict__ at,
                                                      const float *__restrict__ ln2,
                                                      const float *__restrict__ wgate, int D,
                                                      int E, int K, float eps, float *smem,
                                                      const cert_lds &c, bool nonfinite,
                                                      float inv, int force, int *topk_row,
                                                      float *wt_row) {
    if (force != FORCE_EXACT_CHAINS && !nonfinite && isfinite(inv) && inv > 0.0f &&
        blockDim.x >= 256 && D % RF_XC == 0 && D % 64 == 0 &&
        route_refine(xt, at, ln2, wgate, D, E, K, eps, smem, c, inv, topk_row, wt_row))
        return false;
    route_exact_token(xt, at, ln2, wgate, D, E, K, eps, smem, topk_row, wt_row);
    return true;
}

/* grid (ceil(E/R), T), 64 * R threads with R = route_rows(NQ), T <= SMALL_T, D = 256 * NQ; for one token
 * without selection (select == 0) grid (E, 1), 64 threads, one row per workgroup.
 *
 * Wavefront w of workgroup b handles router row e = b*R + w of token t (route_row):
 * every lane holds D/64 consecutive elements of hh = x + attn and of the row. The RMSNorm sum
 * of squares is taken in double (the products rounded as the reference rounds them), xn is
 * formed as the reference forms it from that inv, and the row's products p_k = fl(w_k * xn_k)
 * are summed in double together with every prefix S_k.
 *
 * Why the order is the reference's. Let inv' be the reference's 1/sqrt (from its float chain)
 * and 1 + r = inv'/inv. Its xn differs from ours by the common factor (1 + r) and at most
 * 4 roundings per element, so its products are (1 + r) p_k (1 + psi_k), |psi_k| < 2^-21. Its
 * serial chain adds a rounding error of at most 2^-24 |acc_k| at step k. Hence
 *   |l_ref - (1 + r) S| <= (1 + r) (2^-21 sum|p_k| + 1.0003 * 2^-24 sum|S_k|) + tiny = B,
 * a bound computed here from the same sums. A common factor 1 + r > 0 does not change an
 * order, so only the gaps matter. The reference ranks by p = fl(expf(fl(l - max)) / sum):
 * two logits more than 2^-20 + 2^-23 (|l_a - max| + |l_b - max|) apart give distinct p in the
 * same order (subtraction error 2^-24 relative, expf error under one ulp, quotients 2^-21
 * apart stay ordered after rounding). The last workgroup of the token takes the top K by
 * (S desc, id asc) and checks that each one's lower bound S - B beats the largest upper bound
 * S + B of every expert after it (the later selected ones and all unselected) by that margin,
 * 1% wider (cert_rank, cert_check); if any gap is too narrow (or anything is not finite, or the sum of
 * squares is near the float range limits), the token's routing is recomputed exactly. The
 * renormalised weights are formed from the certified logits (within a few ulps of the
 * reference's).
 *
 * The last token's last workgroup then groups the pairs by expert. */
template <int NQ>
__global__ __launch_bounds__(64 * route_rows(NQ)) void k_route_fast(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, int T, int D, int E, int K, float eps, int force_exact,
    float *__restrict__ xn_out, route_rec *rec, int *ctr, int *topk, float *__restrict__ wt,
    int *stat, int select, int bucket,
    int *__restrict__ pair_pos, int *__restrict__ list_tok, int *__restrict__ list_pair,
    int *__restrict__ grp_expert, int *__restrict__ grp_off, int *__restrict__ grp_cnt,
    int *__restrict__ n_groups, _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
    int max_chunks, int *__restrict__ chunk_grp, int *__restrict__ chunk_m0) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    __shared__ int flag_s;
    __shared__ uint64_t tab[32];
    __shared__ int tk_all[SMALL_T * MAX_K];
    __shared__ int tk_s[MAX_K];
    __shared__ float wt_s[MAX_K];
    __shared__ unsigned long long mask[MAX_E];
    __shared__ int base[MAX_E], cnt[MAX_E];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    /* one token (select == 0): one wavefront per workgroup, E workgroups, so that the router
       rows stream through E CUs; else route_rows(NQ) rows per workgroup */
    const int row = blockIdx.x * (select ? route_rows(NQ) : 1) + w;
    const float *xt = x + (size_t)t * D;
    const float *at = attn ? attn + (size_t)t * D : nullptr;
    {
        double S;
        float B;
        float4 *xo = blockIdx.x == 0 && w == 0 ? (float4 *)(xn_out + (size_t)t * D) : nullptr;
        float inv;
        if (select) {
            /* route_rows(NQ) rows of one token: the token's hh = x + attn and ln2 are staged in
               LDS once for the workgroup (each wavefront would otherwise load them itself);
               the row's loads go first */
            const float4 *w4 = (const float4 *)(wgate + (size_t)(row < E ? row : 0) * D) +
                               lane * NQ;
            float4 wr[NQ];
#pragma unroll
            for (int q = 0; q < NQ; q++) wr[q] = w4[q];
            float4 *hs = (float4 *)smem, *gs = hs + D / 4;
            const float4 *x4 = (const float4 *)xt, *a4 = (const float4 *)(at ? at : xt),
                         *g4 = (const float4 *)ln2;
            constexpr int NTH = 64 * route_rows(NQ);
            constexpr int PER = (64 * NQ + NTH - 1) / NTH;   /* float4 of each per thread */
            float4 xv[PER], av[PER], gv[PER];
#pragma unroll
            for (int r = 0; r < PER; r++) {          /* clamped: the loads stay unconditional */
                const int i = min(tid + NTH * r, D / 4 - 1);
                xv[r] = x4[i];
                av[r] = a4[i];
                gv[r] = g4[i];
            }
#pragma unroll
            for (int r = 0; r < PER; r++) {
                const int i = tid + NTH * r;
                if (i < D / 4) {
                    hs[i] = at ? make_float4(__fadd_rn(xv[r].x, av[r].x), __fadd_rn(xv[r].y, av[r].y),
                                             __fadd_rn(xv[r].z, av[r].z), __fadd_rn(xv[r].w, av[r].w))
                               : xv[r];
                    gs[i] = gv[r];
                }
            }
            lds_barrier();
            float4 h[NQ], gq[NQ];
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                h[q] = hs[lane * NQ + q];
                gq[q] = gs[lane * NQ + q];
            }
            route_row_core<NQ>(h, wr, gq, D, eps, xo, &S, &B, &inv,
                               xh ? xh + (size_t)t * D : nullptr,
                               xh ? xl + (size_t)t * D : nullptr);
        } else {
            route_row<NQ>(xt, at, ln2, wgate + (size_t)(row < E ? row : 0) * D, D, eps, xo, &S,
                          &B, &inv);
        }
        if (lane == 0 && row < E) {
            route_rec *r = rec + (size_t)t * E + row;
            st_agent(&r->s, S);
            st_agent(&r->bound, B);
            st_agent(&r->pad, __float_as_int(inv));
        }
    }
    /* select == 0 (one token): the records are all; the expert kernel ranks them. It also
       needs the epoch of exact one-token routings as it stands before this call (stat[2]):
       its waiting workgroups look for stat[1] to move past that value, and a snapshot taken
       here, before any of them starts, is the same for all of them. */
    if (!select) {
        if (blockIdx.x == 0 && tid == 0) st_agent(&stat[2], ld_agent(&stat[1]));
        return;
    }
    /* the expf table, for the workgroup that finishes the token (the arrival below waits
       for this load with everything else) */
    if (w == 0 && lane < 32) tab[lane] = cpg_exp2f_tab[lane];
    if (!last_arriver(&ctr[t], gridDim.x - 1, &flag_s)) return;

    /* ---- the token's last workgroup: certified top-K, or the exact fallback. With CR_P
       threads per expert the ranking takes two LDS-only barriers (cert_rank_open / close)
       and wavefront 0 checks the certificate alone; otherwise the general cert_rank. */
    __shared__ cert_lds cl;
    __shared__ int ok_s;
    bool nonfinite, ok;
    if (E * CR_P <= (int)blockDim.x) {
        const v4i_t rr = ld_agent16(rec + (size_t)t * E,
                                    (uint32_t)(min(tid, E - 1) * sizeof(route_rec)));
        cert_rank_open(cl, rr, E, K, blockDim.x, &nonfinite);
        cert_rank_close();
        if (w == 0) {
            const bool okw = cert_check_wave(cl, K, nonfinite, force_exact, tk_s, wt_s);
            if (lane == 0) ok_s = okw;
        }
        lds_barrier();
        ok = ok_s != 0;
    } else {
        nonfinite = cert_rank(cl, rec + (size_t)t * E, E, K, blockDim.x);
        ok = cert_check(cl, K, nonfinite, force_exact, tab, tk_s, wt_s);
    }
    if (ok && tid < K) {
        st_agent(&topk[(size_t)t * K + tid], tk_s[tid]);
        wt[(size_t)t * K + tid] = wt_s[tid];
    }
    if (!ok) {
        const float inv = __int_as_float(ld_agent(&rec[(size_t)t * E].pad));
        const bool full = route_fallback(xt, at, ln2, wgate, D, E, K, eps, smem, cl, nonfinite,
                                         inv, force_exact, topk + (size_t)t * K,
                                         wt + (size_t)t * K);
        if (tid == 0) {
            atomicAdd(stat, 1);
            if (full) atomicAdd(&stat[3], 1);
        }
    }

    /* ---- the last token: group all T*K pairs by expert (not needed by the one-token path,
       which reads topk directly) */
    if (!bucket || !last_arriver(&ctr[SMALL_T], T - 1, &flag_s)) return;
    for (int i = tid; i < T * K; i += blockDim.x) tk_all[i] = ld_agent(&topk[i]);
    __syncthreads();
    bucket_pairs(tk_all, T, K, E, mask, base, cnt, pair_pos, list_tok, list_pair, grp_expert,
                 grp_off, grp_cnt, n_groups);
    if (chunk_grp && tid < WAVE) chunks_of_counts(cnt, E, max_chunks, chunk_grp, chunk_m0);
}

/* ================================================================ routing, T > 16 */

#define RN_V4 4             /* k_rmsnorm_tok: float4 of a row per thread held in registers */

/* step a: grid T, 256 threads: hh = x + attn (qwen3_moe.c:178) and xn = rmsnorm(hh, ln2)
   with the reference's serial sum of squares (kernels.c:408-413), lane 0 running the chain
   from LDS. Every thread loads its float4s of x, attn and ln2 at once (D <= 4096: one round
   trip before the chain, none after it). xh / xl not null: xn is also written as the hi/lo
   f16 planes of the prefill GEMMs (hi = f16(v), lo = f16(v - hi)). D % 4 == 0. */
__global__ __launch_bounds__(256) void k_rmsnorm_tok(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    int D, float eps, float *__restrict__ xn, _Float16 *__restrict__ xh,
    _Float16 *__restrict__ xl) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    float *sq = smem;
    __shared__ float inv_s;
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    const int t = blockIdx.x, tid = threadIdx.x, n4 = D / 4;
    const float4 *x4 = (const float4 *)(x + (size_t)t * D);
    const float4 *a4 = attn ? (const float4 *)(attn + (size_t)t * D) : nullptr;
    const float4 *g4 = (const float4 *)ln2;
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 hv[RN_V4], gv[RN_V4];
#pragma unroll
    for (int r = 0; r < RN_V4; r++) {
        const int i = min(tid + 256 * r, n4 - 1);   /* clamped: loads stay unconditional */
        const float4 xv = x4[i], av = a4 ? a4[i] : z;
        gv[r] = g4[i];
        hv[r] = make_float4(__fadd_rn(xv.x, av.x), __fadd_rn(xv.y, av.y), __fadd_rn(xv.z, av.z),
                            __fadd_rn(xv.w, av.w));
    }
#pragma unroll
    for (int r = 0; r < RN_V4; r++)
        if (tid + 256 * r < n4)
            ((float4 *)sq)[tid + 256 * r] =
                make_float4(__fmul_rn(hv[r].x, hv[r].x), __fmul_rn(hv[r].y, hv[r].y),
                            __fmul_rn(hv[r].z, hv[r].z), __fmul_rn(hv[r].w, hv[r].w));
    __syncthreads();
    if (tid == 0) inv_s = rms_inv(chain_any(sq, D), D, eps);
    __syncthreads();
    const float inv = inv_s;
#pragma unroll
    for (int r = 0; r < RN_V4; r++) {
        const int i = tid + 256 * r;
        if (i < n4) {
            const float o[4] = {__fmul_rn(__fmul_rn(hv[r].x, inv), gv[r].x),
                                __fmul_rn(__fmul_rn(hv[r].y, inv), gv[r].y),
                                __fmul_rn(__fmul_rn(hv[r].z, inv), gv[r].z),
                                __fmul_rn(__fmul_rn(hv[r].w, inv), gv[r].w)};
            ((float4 *)(xn + (size_t)t * D))[i] = make_float4(o[0], o[1], o[2], o[3]);
            if (xh) {
                half4_t h, l;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f16pair p = split_f16(o[j]);
                    h[j] = p.hi;
                    l[j] = p.lo;
                }
                *(half4_t *)(xh + (size_t)t * D + 4 * i) = h;
                *(half4_t *)(xl + (size_t)t * D + 4 * i) = l;
            }
        }
    }
}

#define RL_TOK 16           /* k_router_tok: tokens per workgroup */
#define RL_ROWS 16          /* router rows per workgroup */

/* step b: grid (ceil(T/16), ceil(E/16)), 256 threads. Thread (i, r) = (tid % 16, tid / 16)
   runs the chain of token t0+i and router row e0+r: logits[t][e] = the reference's serial
   chain of separately rounded products (kernels.c:75-95), one chain per lane, so the GPU's
   lanes together hold all T * E chains. A stage puts KC columns (128, or 64 where D is not a
   multiple of 128) of the 16 tokens' xn and of the 16 rows in LDS (row stride KC + 4 floats,
   so the 16 rows a wavefront reads as float4 fall in distinct banks; the 4 lanes of a token
   and the 16 lanes of a row read the same address). Each thread loads KC/64 float4 of each
   per stage, two stages ahead into two register sets in a loop unrolled by two with no exit
   between the halves (a branch there would make the compiler copy registers whose loads are
   in flight): a stage of 128 columns is long enough to cover the loads' latency, one of 64
   was not (each stage waited for its loads). A chain's stage is unrolled whole, so its LDS
   reads issue together and wait once. Tokens and rows past the ends read clamped (valid)
   addresses and are not stored. */
template <int KC>
__global__ __launch_bounds__(256) void k_router_tok(
    const float *__restrict__ xn, const float *__restrict__ wgate, int T, int D, int E,
    float *__restrict__ logits) {
    constexpr int LX = KC + 4, NI = KC / 64;     /* float4 items per thread and array */
    static_assert(NI == 1 || NI == 2, "stage width");
    __shared__ __align__(16) float xs[2][RL_TOK * LX];
    __shared__ __align__(16) float ws[2][RL_ROWS * LX];
    const int tid = threadIdx.x, i = tid & 15, r = tid >> 4;
    const int t0 = blockIdx.x * RL_TOK, e0 = blockIdx.y * RL_ROWS;
    const int nt = min(RL_TOK, T - t0), ne = min(RL_ROWS, E - e0), S = D / KC;
    /* this thread's stage items q < NI: item tid + 256 q = (row, float4 column) of the
       16 x KC/4 tile, for xn and for the router rows, named (an array of them would be kept
       in scratch) */
#define RK_ITEM(q)                                                                          \
    const int lr##q = (tid + 256 * (q)) / (KC / 4), lc##q = (tid + 256 * (q)) % (KC / 4);    \
    const float *xp##q = xn + (size_t)(t0 + min(lr##q, nt - 1)) * D + 4 * lc##q;            \
    const float *wp##q = wgate + (size_t)(e0 + min(lr##q, ne - 1)) * D + 4 * lc##q;          \
    const int so##q = lr##q * LX + 4 * lc##q;                                               \
    float4 ax##q, aw##q, bx##q, bw##q;
#define RK_EACH(M) { M(0) } if constexpr (NI > 1) { M(1) }
    RK_ITEM(0)
    RK_ITEM(1)
    float acc = 0.0f;
    auto chain = [&](int b) {
        const float4 *xr = (const float4 *)(xs[b] + i * LX), *wr = (const float4 *)(ws[b] + r * LX);
#pragma unroll
        for (int k = 0; k < KC / 4; k++) {
            const float4 xv = xr[k], wv = wr[k];
            acc = __fadd_rn(acc, __fmul_rn(wv.x, xv.x));
            acc = __fadd_rn(acc, __fmul_rn(wv.y, xv.y));
            acc = __fadd_rn(acc, __fmul_rn(wv.z, xv.z));
            acc = __fadd_rn(acc, __fmul_rn(wv.w, xv.w));
        }
    };
#define RK_LOAD(set, q, st)                                                                 \
    set##x##q = *(const float4 *)(xp##q + min((st), S - 1) * KC);                           \
    set##w##q = *(const float4 *)(wp##q + min((st), S - 1) * KC);
#define RK_PUT(set, q, buf)                                                                 \
    *(float4 *)(xs[buf] + so##q) = set##x##q;                                               \
    *(float4 *)(ws[buf] + so##q) = set##w##q;
#define RK_LA0(q) RK_LOAD(a, q, 0)
#define RK_LB1(q) RK_LOAD(b, q, 1)
#define RK_LA2(q) RK_LOAD(a, q, 2)
#define RK_LB3(q) RK_LOAD(b, q, st + 3)
#define RK_LA4(q) RK_LOAD(a, q, st + 4)
#define RK_PA0(q) RK_PUT(a, q, 0)
#define RK_PB1(q) RK_PUT(b, q, 1)
    RK_EACH(RK_LA0)
    RK_EACH(RK_LB1)
    RK_EACH(RK_PA0)
    RK_EACH(RK_LA2)
    __syncthreads();
    for (int st = 0; st < S; st += 2) {
        chain(0);                                /* stage st in buffer 0 */
        RK_EACH(RK_PB1)                          /* stage st + 1 */
        RK_EACH(RK_LB3)
        __syncthreads();
        if (st + 1 < S) chain(1);                /* stage st + 1 in buffer 1 */
        RK_EACH(RK_PA0)                          /* stage st + 2 */
        RK_EACH(RK_LA4)
        __syncthreads();
    }
#undef RK_ITEM
#undef RK_EACH
#undef RK_LOAD
#undef RK_PUT
#undef RK_LA0
#undef RK_LB1
#undef RK_LA2
#undef RK_LB3
#undef RK_LA4
#undef RK_PA0
#undef RK_PB1
    if (i < nt && r < ne) logits[(size_t)(t0 + i) * E + e0 + r] = acc;
}

/* grid T, 64 threads: softmax and top-K of one token */
__global__ __launch_bounds__(64) void k_select(const float *__restrict__ logits, int E, int K,
                                               int *__restrict__ topk, float *__restrict__ wt) {
    __shared__ __align__(16) float es[MAX_E];
    const int t = blockIdx.x;
    select_token(logits + (size_t)t * E, E, K, topk + (size_t)t * K, wt + (size_t)t * K, es);
}

/* one workgroup of 1024 threads. chunk_grp not null: wavefront 0 then forms the prefill
   chunk list of the groups (pf_chunk_list; group g is the g-th expert with pairs, in expert
   order, as bucket_pairs numbers them) */
__global__ __launch_bounds__(1024) void k_bucket(
    const int *__restrict__ topk, int T, int K, int E, int *__restrict__ pair_pos,
    int *__restrict__ list_tok, int *__restrict__ list_pair, int *__restrict__ grp_expert,
    int *__restrict__ grp_off, int *__restrict__ grp_cnt, int *__restrict__ n_groups,
    int max_chunks, int *__restrict__ chunk_grp, int *__restrict__ chunk_m0) {
    __shared__ unsigned long long mask[(BUCKET_MAX_T / 64) * MAX_E];
    __shared__ int base[MAX_E], cnt[MAX_E];
    bucket_pairs(topk, T, K, E, mask, base, cnt, pair_pos, list_tok, list_pair, grp_expert,
                 grp_off, grp_cnt, n_groups);
    /* cnt is final since bucket_pairs' last barrier */
    if (chunk_grp && threadIdx.x < WAVE) chunks_of_counts(cnt, E, max_chunks, chunk_grp, chunk_m0);
}

/* ================================================================ expert GEMVs */

/* ---------------------------------------------------------------- batches on MFMA */

/* The batch expert GEMVs with the products on MFMA (v_mfma_f32_16x16x32_f16; operand layout,
   exact weights and hi/lo activations as the helpers of cpg_mfma.h describe). A workgroup keeps
   its weight tiles in registers, all loads issued at once (the GEMV schedule, not the prefill
   GEMMs' k loop), and takes the group's tokens 16 at a time as the A operand, read straight
   from the activation rows and split into hi/lo halves in registers. Every output (token, row)
   is summed in the same order whatever the other tokens of its tile are: over each wavefront's
   blocks in order (each block's product scaled by its fp16 scale in fp32), then over the
   wavefronts in order. */
#define MM_BPW 4            /* k_gateup_mm: blocks of 32 per wavefront (waves = D / 128) */
#define MM_BPWD 3           /* k_down_mm: blocks of 32 per wavefront (waves = ceil(F/96)) */

/* grid (F/32 * groups), 64 * nw threads with nw = D / 128 <= 16. Workgroup (b, g) (the xcd_pair
   of its index) computes rows 32b..32b+31 of Wg and of Wu of expert group g's expert as four
   16-row B tiles (gate 32b, 32b+16; up 32b, 32b+16), wavefront w over blocks 4w..4w+3, for all
   the group's tokens; then h = silu(g) * u (kernels.c:416, qwen3_moe.c:219) for those rows,
   written at the pair's list position: h[(off + i) * F + row]. The payloads stay in registers;
   the workgroup's fp16 scales (32 rows x D/32 blocks of each matrix) go to LDS, one 32-bit
   pair per thread and matrix. Dynamic LDS: nw * 1024 floats + 4 * D bytes. */
template <int ENC>
__global__ __launch_bounds__(1024) void k_gateup_mm(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes,
    size_t payload_plane, int D, int F, int nw, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ list_tok, const float *__restrict__ xn, float *__restrict__ h) {
    extern __shared__ __align__(16) float red[];    /* [wave][tile][token 16][row 16], scales */
    __shared__ uint64_t tab[32];
    const int nt = F / 32, lid = xcd_pair(blockIdx.x, gridDim.x), grp = lid / nt;
    const int bt = lid - grp * nt, m = grp_cnt[grp];
    if (m <= 0) return;
    const int e = grp_expert[grp], off = grp_off[grp];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4, c = l & 15;
    const int nb = D / 32, b0 = w * MM_BPW, nthr = nw * 64;
    uint16_t *scl = (uint16_t *)(red + nw * 1024);   /* [matrix][block][row 32] */
    /* the first tile's token ids and the scales ahead of the payloads (completion is counted
       in issue order: issued after the payloads, waiting for them would wait for every one) */
    int tk = list_tok[off + min(c, m - 1)];
    if (tid < 32) tab[tid] = cpg_exp2f_tab[tid];
    const uint8_t *Mg = experts + (size_t)e * exp_stride;
    uint32_t sp[2];                               /* rows 2p, 2p+1 of block tid / 16 */
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
        sp[mt] = *(const uint32_t *)(Mg + mt * mat_bytes + payload_plane +
                                     2 * (cpg_tile_index(32 * bt, tid >> 4, nb) + 2 * (tid & 15)));
    uint2 wp[4][MM_BPW];                          /* tiles: gate, gate + 16, up, up + 16 */
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
        for (int q = 0; q < MM_BPW; q++)
            wp[n][q] = weight_payload<ENC>(Mg + (n >> 1) * mat_bytes, 32 * bt + 16 * (n & 1) + c,
                                           b0 + q, nb, g);
#pragma unroll
    for (int mt = 0; mt < 2; mt++) *(uint32_t *)(scl + (mt * nb + (tid >> 4)) * 32 + 2 * (tid & 15)) = sp[mt];
    __syncthreads();
    /* one tile of 16 tokens from t0 (lane c: token t0 + c, id tk); the first straight-line,
       any further ones in a loop (a loop around the first would keep its invariants live) */
    auto tile = [&](int t0, int tk) __attribute__((always_inline)) {
        float4 xr[MM_BPW][2];                     /* all loads first, split at use */
#pragma unroll
        for (int q = 0; q < MM_BPW; q++) {
            const float4 *xp = (const float4 *)(xn + (size_t)tk * D + (b0 + q) * 32 + 8 * g);
            xr[q][0] = xp[0];
            xr[q][1] = xp[1];
        }
        f32x4_t acc[4];
#pragma unroll
        for (int n = 0; n < 4; n++) acc[n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < MM_BPW; q++) {
            half8_t ah, al;
            split_hilo8(xr[q][0], xr[q][1], ah, al);
#pragma unroll
            for (int n = 0; n < 4; n++) {
                const half8_t b = weight_half8<ENC>(WRaw{wp[n][q], 0}, g);
                const float d = scale_f32(scl[((n >> 1) * nb + b0 + q) * 32 + 16 * (n & 1) + c]);
                f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b,
                                                                  f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, t, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[n][i] = fmaf(d, t[i], acc[n][i]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int n = 0; n < 4; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[((w * 4 + n) * 16 + 4 * g + i) * 16 + c] = acc[n][i];
        __syncthreads();
        for (int o = tid; o < 16 * 32; o += nthr) {  /* token o / 32, row o % 32 of the 32 */
            const int i = o >> 5, r = o & 31, n = r >> 4, rr = r & 15;
            float gs = 0.0f, us = 0.0f;
            for (int ww = 0; ww < nw; ww++) {
                gs += red[((ww * 4 + n) * 16 + i) * 16 + rr];
                us += red[((ww * 4 + n + 2) * 16 + i) * 16 + rr];
            }
            if (t0 + i < m) h[(size_t)(off + t0 + i) * F + 32 * bt + r] = swiglu_t(gs, us, tab);
        }
    };
    tile(0, tk);
    for (int t0 = 16; t0 < m; t0 += 16) {
#pragma unroll
        for (int n = 0; n < 4; n++)              /* converted at use, not hoisted out */
#pragma unroll
            for (int q = 0; q < MM_BPW; q++) asm volatile("" : "+v"(wp[n][q].x), "+v"(wp[n][q].y));
        __syncthreads();                         /* the previous tile's sums are read */
        tile(t0, list_tok[off + min(t0 + c, m - 1)]);
    }
}

/* grid (D/64, groups), 64 * nw threads with nw = ceil(F / 96) <= 16. Workgroup (tile, g) computes
   y = Wd . h for rows 64 tile .. 64 tile + 63 (four 16-row B tiles; wavefront w over blocks
   3w..3w+2 of the F/32) for all of group g's pairs (their h rows, from k_gateup_mm), stored at
   the pair's index t*K + j; then the combine: each of the group's tokens counts this
   tile in at ctr2[t][tile], and the workgroup that brings the count to K adds
   mlp[t, tile] += wt_j * y_j for j = 0..K-1 in order (qwen3_moe.c:221) and resets the counter
   (the tokens it completes spread over its wavefronts). Dynamic LDS: nw * 1024 floats. */
template <int ENC>
__global__ __launch_bounds__(1024) void k_down_mm(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t wd_off, size_t payload_plane,
    int D, int F, int K, int nw, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ list_tok, const int *__restrict__ list_pair,
    const float *__restrict__ h, float *y, const float *__restrict__ wt, int *ctr2,
    float *__restrict__ mlp) {
    extern __shared__ __align__(16) float red[];    /* [wave][tile][token 16][row 16] */
    const int grp = blockIdx.y, m = grp_cnt[grp];
    if (m <= 0) return;
    const int e = grp_expert[grp], off = grp_off[grp], tile = blockIdx.x;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4, c = l & 15;
    const int nb = F / 32, b0 = w * MM_BPWD, nbw = max(0, min(MM_BPWD, nb - b0)), nthr = nw * 64;
    const uint8_t *M = experts + (size_t)e * exp_stride + wd_off;
    WRaw wr[4][MM_BPWD];
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
        for (int q = 0; q < MM_BPWD; q++)
            wr[n][q] = weight_raw<ENC>(M, payload_plane, 64 * tile + 16 * n + c,
                                       min(b0 + q, nb - 1), nb, g);
    for (int t0 = 0; t0 < m; t0 += 16) {
#pragma unroll
        for (int n = 0; n < 4; n++)
#pragma unroll
            for (int q = 0; q < MM_BPWD; q++) wr[n][q].pin();
        const float *hr = h + (size_t)(off + min(t0 + c, m - 1)) * F;
        half8_t ah[MM_BPWD], al[MM_BPWD];
#pragma unroll
        for (int q = 0; q < MM_BPWD; q++) {
            const float4 *hp = (const float4 *)(hr + min(b0 + q, nb - 1) * 32 + 8 * g);
            split_hilo8(hp[0], hp[1], ah[q], al[q]);
        }
        f32x4_t acc[4];
#pragma unroll
        for (int n = 0; n < 4; n++) acc[n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < MM_BPWD; q++)
            if (q < nbw)
#pragma unroll
                for (int n = 0; n < 4; n++) {
                    const half8_t b = weight_half8<ENC>(wr[n][q], g);
                    const float d = scale_f32(wr[n][q].d);
                    f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        ah[q], b, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[q], b, t, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[n][i] = fmaf(d, t[i], acc[n][i]);
                }
        if (t0 > 0) __syncthreads();
#pragma unroll
        for (int n = 0; n < 4; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[((w * 4 + n) * 16 + 4 * g + i) * 16 + c] = acc[n][i];
        __syncthreads();
        for (int o = tid; o < 16 * 64; o += nthr) {  /* token o / 64, row o % 64 of the tile */
            const int i = o >> 6, r = o & 63, n = r >> 4, rr = r & 15;
            float s = 0.0f;
            for (int ww = 0; ww < nw; ww++) s += red[((ww * 4 + n) * 16 + i) * 16 + rr];
            if (t0 + i < m) st_agent(&y[(size_t)list_pair[off + t0 + i] * D + 64 * tile + r], s);
        }
    }
    mem_done();
    __syncthreads();
    /* wavefront 0 counts the group's tokens in and lists those whose count this workgroup
       completes; all wavefronts then combine them, one token per wavefront at a time */
    int *clist = (int *)red;
    __shared__ int ncl;
    const int ntile = D / 64, row = tile * 64 + l;
    if (w == 0) {
        int n = 0;
        for (int i0 = 0; i0 < m; i0 += WAVE) {
            int tok = 0, last = 0;
            if (i0 + l < m) {
                tok = list_tok[off + i0 + l];
                last = arrive(&ctr2[(size_t)tok * ntile + tile]) == K - 1;
            }
            const unsigned long long bal = __ballot(last);
            if (last) {
                clist[n + __popcll(bal & ((1ull << l) - 1))] = tok;
                st_agent(&ctr2[(size_t)tok * ntile + tile], 0);
            }
            n += __popcll(bal);
        }
        if (l == 0) ncl = n;
    }
    __syncthreads();
    for (int idx = w; idx < ncl; idx += nw) {
        const int tt = clist[idx];
        float o = mlp[(size_t)tt * D + row];
        for (int j = 0; j < K; j++)
            o = __fadd_rn(o, __fmul_rn(wt[(size_t)tt * K + j],
                                       ld_agent(&y[((size_t)tt * K + j) * D + row])));
        mlp[(size_t)tt * D + row] = o;
    }
}

/* ================================================================ one token (decode) */

/* grid (F/NR * K), GW*64 threads, T == 1, NR = 32 or 24 rows per matrix (gu_load).
   Workgroup (b, j) (the xcd_tile of its index, so that one XCD streams one expert and the
   workgroups of a 64-row tile share an L2) computes rows NR*b..NR*b+NR-1 of both Wg and Wu of
   the token's j-th expert: lanes 0..NR-1 end with the gate rows, lanes NR..2NR-1 with the up
   rows, the GW wavefronts splitting k (BPW blocks each); then
   h = silu(g) * u for those rows (kernels.c:416, qwen3_moe.c:219), written to h[j*F + row].

   The selection happens here, in every workgroup, from the E router records k_route_fast
   left (its select == 0 form): the workgroup ranks them and forms the slot order with two
   LDS-only barriers (cert_rank_open, cert_rank_close), xn staged in between, issues the loads
   of slot j's expert's weights at once, and every wavefront certifies the order on its own
   while they are in flight (cert_check_wave): no barrier stands between the loads and the
   dot products.
   Certified: workgroup 0 publishes topk / wt (the down kernel reads them). Not certified
   (about 2 % of tokens): workgroup 0 computes the exact routing (route_exact_token, written
   to topk / wt), counts it in stat[0] and then advances stat[1]; the other workgroups wait
   for stat[1] to move past stat[2], the value k_route_fast recorded before this launch, at
   most XWAIT_SPINS polls, and compute the same routing themselves if it does not (the same
   bits either way); each then loads the weights of its exact expert. xn (the router's input, formed by
   k_route_fast) is staged while the weights are in flight. Requires E * CR_P <= GW * 64, D == GW * BPW * 32,
   D <= 4 * GW * 64, dynamic LDS of max(D + D/32 + GW*64, exact_route_lds_floats(D, E)) floats. */
template <int ENC, int BPW, int NR>
__global__ __launch_bounds__(GW * 64) void k_gateup1(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes,
    size_t payload_plane, int D, int F, const route_rec *rec, int E, int K, int force_exact,
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, float eps, int *topk, float *wt, int *stat,
    const float *__restrict__ xn, float *__restrict__ h, int *xsel) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    __shared__ uint64_t tab[32];
    __shared__ cert_lds cl;
    const int nb = D / 32;
    float *xs = smem;                            /* xn, GU_XB * nb (gu_stage) */
    float *bsum = xs + GU_XB * nb;               /* nb */
    float *red = bsum + nb;                      /* GW * 64 */
    const int nt = F / NR, l = xcd_tile(blockIdx.x, gridDim.x), j = l / nt, bt = l - j * nt;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    __shared__ int got_s;
    /* the expf table, this thread's router record and xn in flight together, xn last */
    const uint64_t tv = cpg_exp2f_tab[tid & 31];
    const v4i_t rr = ld_agent16(rec, (uint32_t)(min(tid, E - 1) * sizeof(route_rec)));
    const bool hasx = tid < D / 4;
    /* at a clamped index, unconditionally: a load under a branch is waited for where the
       branch joins, and that would be the records' first use (gu_stage ignores the lanes
       past D, whose blocks are whole) */
    const float4 xv = *((const float4 *)xn + min(tid, D / 4 - 1));
    bool nonfinite;
    cert_rank_open(cl, rr, E, K, GW * 64, &nonfinite);
    gu_stage<ENC>(xs, bsum, tid, xv, hasx);
    if (tid < 32) tab[tid] = tv;
    cert_rank_close();
    const int e = cl.cslot[j], row = bt * NR + lane;
    WBlk<ENC> wv[BPW];
    uint16_t sv[BPW];
    gu_load<ENC, BPW, NR>(experts + (size_t)e * exp_stride, mat_bytes, payload_plane, bt * NR,
                          nb, wv, sv);
    /* certified while they are in flight, every wavefront on its own; wavefront 0 of
       workgroup 0 publishes topk / wt */
    const bool pub = blockIdx.x == 0 && w == 0;
    /* workgroup x < 8 runs on XCD x: it leaves the selection in that XCD's copy too, where
       the down kernel's workgroups on the XCD read it from their own L2 */
    int *xs_x = xsel && blockIdx.x < NXCD && w == 0 ? xsel + blockIdx.x * 2 * K : nullptr;
    const bool ok = cert_check_wave(cl, K, nonfinite, force_exact, pub ? topk : nullptr,
                                    pub ? wt : nullptr, xs_x,
                                    xs_x ? (float *)(xs_x + K) : nullptr);
    /* the wavefronts' partial sums reduced in order, SwiGLU, h out */
    auto finish = [&](float p) {
        red[w * 64 + lane] = p;
        __syncthreads();
        if (w == 0) {
            float v = 0.0f;
            for (int ww = 0; ww < GW; ww++) v += red[ww * 64 + lane];
            const float u = __shfl(v, lane + NR);
            if (lane < NR) h[(size_t)j * F + row] = swiglu_t(v, u, tab);
        }
    };
    if (ok) {
        /* the dot products, each waiting only for its own loads */
        finish(gu_dots<ENC, BPW, NR>(wv, sv, xs, bsum));
        return;
    }
    /* not certified: the same in every workgroup */
    if (blockIdx.x != 0 && tid == 0) {
        /* workgroup 0 advances stat[1] once its exact routing is stored; measured against the
           epoch before this launch, a workgroup that arrives after that sees it at once. If
           workgroup 0 has not run yet when the polls run out, the routing is computed here
           (the same bits). */
        const int ep = ld_agent(&stat[2]);
        int got = ld_agent(&stat[1]) != ep;
        for (int i = 0; i < XWAIT_SPINS && !got; i++) {
            __builtin_amdgcn_s_sleep(8);
            got = ld_agent(&stat[1]) != ep;
        }
        got_s = got;
    }
    __syncthreads();
    __shared__ int full_s;
    if (blockIdx.x == 0 || !got_s) {             /* one call site: the code is inlined */
        const float inv = __int_as_float(ld_agent(&rec[0].pad));
        const bool full = route_fallback(x, attn, ln2, wgate, D, E, K, eps, smem, cl, nonfinite,
                                         inv, force_exact, topk, wt);
        if (tid == 0) full_s = full;
        mem_done();                              /* topk / wt written before stat[1] moves */
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid == 0) {
        atomicAdd(&stat[0], 1);
        if (full_s) atomicAdd(&stat[3], 1);
        arrive(&stat[1]);
    }
    if (xs_x && lane < K) {         /* the XCD's copy of the exact routing */
        xs_x[lane] = ld_agent(&topk[lane]);
        xs_x[K + lane] = ld_agent((const int *)wt + lane);
    }
    const int ex = ld_agent(&topk[j]);
    WBlk<ENC> wx[BPW];
    uint16_t sx[BPW];
    gu_load<ENC, BPW, NR>(experts + (size_t)ex * exp_stride, mat_bytes,
                          payload_plane, bt * NR, nb, wx, sx);
    /* the exact routing used the LDS; xn is loaded again rather than held in registers
       across it */
    const float4 xv2 = hasx ? *((const float4 *)xn + tid) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    gu_stage<ENC>(xs, bsum, tid, xv2, hasx);
    lds_barrier();
    finish(gu_dots<ENC, BPW, NR>(wx, sx, xs, bsum));
}

#define HMAX 4              /* k_down1: float4 of the K vectors h staged per thread */

/* grid (D/R), GW*64 threads, T == 1, R = 64/K rows per workgroup. With b the xcd_tile of the
   workgroup's index (one XCD takes D/8 consecutive rows, whole 64-row tiles), lane (j, r) =
   (lane / R, lane % R) computes row R*b + r of Wd of expert topk[j] against h_j, the GW wavefronts
   splitting k (BPW blocks each); then lanes r < R add mlp[row] += wt_j * y_j[row] for
   j = 0..K-1 in order (qwen3_moe.c:221), all within the workgroup. The K vectors h_j are
   staged with a row stride of F+4 floats, so the K groups of lanes read K different LDS
   banks. Requires 64 % K == 0, D % R == 0, ceil(F/32/GW) == BPW, K*F <= 16 * GW * 64.
   xres not null: the layer's residual is taken here instead (cachepotato.c:157-159):
   xres[row] = xres[row] + (attn[row] + o), o = 0 + sum_j wt_j y_j in slot order, and mlp is
   not touched. */
template <int ENC, int BPW>
__global__ __launch_bounds__(GW * 64) void k_down1(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t wd_off,
    size_t payload_plane, int D, int F, int K, const int *__restrict__ topk,
    const float *__restrict__ h, const float *__restrict__ wt, float *__restrict__ mlp,
    float *__restrict__ xres, const float *__restrict__ attn, const int *__restrict__ xsel) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    const int nb = F / 32, ld = F + 4, R = WAVE / K, q = F / 4;
    /* the selection from this XCD's copy (the gate/up kernel's workgroup on the XCD wrote it,
       so it is in the XCD's L2), else the published one */
    if (xsel) {
        topk = xsel + (blockIdx.x % NXCD) * 2 * K;
        wt = (const float *)(topk + K);
    }
    float *hs = smem;                            /* K * (F + 4) */
    float *bsum = hs + K * ld;                   /* K * nb */
    float *red = bsum + K * nb;                  /* GW * 64 */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j = lane / R, row = xcd_tile(blockIdx.x, gridDim.x) * R + lane % R, b0 = w * BPW;
    /* every load before the weights' is unconditional, at valid addresses (the lanes past
       the staged vectors read the last float4 and are not staged): a load under a branch is
       waited for where the branch joins, and that would hold the weights' requests back
       until h had arrived */
    const int e = topk[j];
    float4 hv[HMAX];
#pragma unroll
    for (int r = 0; r < HMAX; r++)
        hv[r] = *((const float4 *)h + min(tid + r * GW * 64, K * q - 1));
    const float *rs = xres ? xres : mlp;         /* the residual, or mlp to add to */
    const float rv = rs[row], av = (attn ? attn : rs)[row], wj = wt[j];
    const float m0 = xres ? 0.0f : rv, xr = xres ? rv : 0.0f, ar = xres ? av : 0.0f;
    const uint8_t *M = experts + (size_t)e * exp_stride + wd_off;
    WBlk<ENC> wv[BPW];
    uint16_t sv[BPW];
    load_row_blocks_raw<ENC, BPW>(M, payload_plane, row, b0, nb - 1, nb, wv, sv);
#pragma unroll
    for (int r = 0; r < HMAX; r++) {
        const int idx = tid + r * GW * 64, i = idx / q;
        stage_put<ENC>(hs, bsum, ld, nb, i, idx - i * q, hv[r], idx < K * q);
    }
    lds_barrier();                               /* the dot products wait for their own loads */
    float dv[BPW];
#pragma unroll
    for (int r = 0; r < BPW; r++) dv[r] = f16_to_f32_hw(sv[r]);
    const int nbw = max(0, min(BPW, nb - b0));
    float acc = 0.0f;
    row_dots_mc<ENC, 1, BPW>(wv, dv, b0, nbw, hs + j * ld, bsum + j * nb, ld, nb, &acc);
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w == 0) {
        float y = 0.0f;
        for (int ww = 0; ww < GW; ww++) y += red[ww * 64 + lane];
        float o = m0;
        for (int jj = 0; jj < K; jj++) {
            const float yj = __shfl(y, jj * R + lane % R);
            const float wtj = __shfl(wj, jj * R);
            o = __fadd_rn(o, __fmul_rn(wtj, yj));
        }
        if (lane < R) {
            if (xres) xres[row] = __fadd_rn(xr, __fadd_rn(ar, o));
            else mlp[row] = o;
        }
    }
}

/* ================================================================ one token, one kernel */

/* The state the one-launch MoE (k_moe1) keeps between its launches, at a fixed place in the
   workspace: zero when the workspace is first used. */
#define MOE1_MAX_TILES 512  /* k_moe1: gate/up tiles (K * F/32) and workgroups at most */
#define MOE1_SPINS (1 << 20) /* k_moe1: polls of a wait (about 100 ms) before it gives up */
#define CNT_STRIDE 64       /* k_moe1: ints between arrival counters (256 bytes) */
struct moe1_state {
    int epoch;          /* the tag of the last launch */
    int selflag;        /* the tag of the fallback routing in sel / selw */
    int pad[62];
    int cnt_a[NXCD * CNT_STRIDE];   /* router rows stored, counted by row % 8 (counter x at
                                       x * CNT_STRIDE, a line of its own), over every launch */
    int cnt_g[NXCD * CNT_STRIDE];   /* gate/up tiles stored, counted by tile % 8, likewise */
    int checkin[MOE1_MAX_TILES];    /* workgroup b has read epoch: its tag */
    route_rec rec[MAX_E];           /* router row e: S and B */
};

/* Whole workgroup: wait until every counter c[x * CNT_STRIDE] has counted the n arrivals of
   launch `tag` (arrival i counted at counter i % 8: tag * ceil((n - x) / 8) in all, compared
   modulo 2^32);
   thread 0 polls the eight counters, bounded. Ends with the workgroup synchronised;
   returns false (in every thread) when the wait gave up. flag: an LDS int. */
__device__ static bool wait_counts(const int *c, int tag, int n, int *flag) {
    if (threadIdx.x == 0) {
        bool ok = false;
        for (int i = 0; i < MOE1_SPINS && !ok; i++) {
            int v[NXCD];
#pragma unroll
            for (int x = 0; x < NXCD; x++) v[x] = ld_agent(&c[x * CNT_STRIDE]);
            ok = true;
#pragma unroll
            for (int x = 0; x < NXCD; x++) {
                const unsigned need = (unsigned)tag * (unsigned)((n - x + NXCD - 1) / NXCD);
                ok = ok && (int)((unsigned)v[x] - need) >= 0;
            }
            if (!ok) __builtin_amdgcn_s_sleep(4);
        }
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

/* The MoE half of one token (T = 1) in one launch of NWG = max(E, (F/32)*K, D/R) workgroups
   (R = 64/K down rows per workgroup), all resident at once (the host checks the occupancy).
   The phases hand their results over through counted arrivals, with no grid barrier and no
   kernel boundary between them. Every launch has its own tag ep + 1: each workgroup reads
   ep = st->epoch at its start and checks in (st->checkin[b] = ep + 1); the last workgroup,
   idle until the down phase, waits for every check-in (every workgroup has read ep by then)
   and stores ep + 1 for the next launch. A producer completes its stores, then counts itself
   in at one of eight counters (by its index mod 8, so no address takes more than a few
   arrivals); a consumer's thread 0 polls the eight counters until they hold this launch's
   arrivals (wait_counts). Waits are bounded: after about 100 ms one gives up and counts a
   timeout in *timeouts (that call's results are then undefined; cpg_moe_ws_status reports
   it).
     A  workgroup b < E, wavefront 0: router row b (route_row) -> st->rec[b], counted in
        cnt_a. Wavefront GW-1: the RMSNorm inverse of hh = x + attn (route_inv, the same bits).
        Every thread: its float4 of x, attn and ln2 for xn, loaded at the start.
     B  every workgroup: all E rows counted in, then the ranking and slot order with xn
        staged in between (cert_rank_open, cert_rank_close, as k_gateup1).
     C  workgroup b: the weights of its gate/up tile (k_gateup1's rows 32b' of Wg and Wu of
        slot j', b = j' * F/32 + b') are requested, every wavefront certifies the order while
        they fly (cert_check_wave), and the weights of its down rows (k_down1's rows R*b of
        the K slots) are requested behind them. Not certified: workgroup 0 runs the fallback (route_fallback) into
        sel / selw and tags it (st->selflag); the others wait for the tag and read it, or
        compute the same routing themselves if the wait gives up; the weights are requested
        again for that selection. Then gate/up dots, SwiGLU -> h (agent-scope stores),
        counted in cnt_g.
     D  every workgroup with down rows: all F/32*K gate/up tiles counted in; h of the K
        experts staged from memory, down dots, then mlp[row] += sum_j wt_j y_j in slot order
        (qwen3_moe.c:221), or with xres the layer's residual xres[row] += attn[row] + that sum
        (cachepotato.c:157-159).
   Every sum is taken in the order of the three-kernel path (route_row, k_gateup1, k_down1),
   so the results are bit-identical to it. */
/* thread-level bounded wait for *p == tag (agent scope); false if it gave up */
__device__ static inline bool wait_tag(const int *p, int tag) {
    for (int i = 0; i < MOE1_SPINS; i++) {
        if (ld_agent(p) == tag) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

template <int ENC, int NQ, int BG, int BD>
__global__ __launch_bounds__(GW * 64) void k_moe1(
    const float *__restrict__ x, const float *__restrict__ attn, const float *__restrict__ ln2,
    const float *__restrict__ wgate, int D, int E, int K, int F, float eps, int force_exact,
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes, size_t pp_g,
    size_t wd_off, size_t pp_d, moe1_state *st, float *hbuf, int *sel, float *selw, int *stat,
    int *timeouts, int *topk_out, float *wt_out, float *mlp, float *xres) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    __shared__ uint64_t tab[32];
    __shared__ cert_lds cl;
    __shared__ int tk_s[MAX_K];
    __shared__ float wt_s[MAX_K];
    __shared__ float inv_s;
    __shared__ int ep_s, got_s;
    const int b = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int R = WAVE / K, nbd = D / 32, nbf = F / 32;
    /* ---- every load of the start first: the expf table, and x, attn, ln2 for xn */
    const uint64_t tv = cpg_exp2f_tab[tid & 31];
    const bool hasx = tid < D / 4;
    const int xi = min(tid, D / 4 - 1);
    const float4 xa = ((const float4 *)x)[xi], aa = ((const float4 *)(attn ? attn : x))[xi],
                 ga = ((const float4 *)ln2)[xi];
    tab[tid & 31] = tv;
    const int G = nbf * K;                       /* gate/up tiles */
    /* ---- A: router row b; this launch's epoch; the RMSNorm inverse */
    if (w == 0 && b < E) {
        double S;
        float B;
        route_row<NQ>(x, attn, ln2, wgate + (size_t)b * D, D, eps, nullptr, &S, &B);
        if (lane == 0) {
            st_agent(&st->rec[b].s, S);
            st_agent(&st->rec[b].bound, B);
            mem_done();                          /* S and B complete before the count */
            arrive(&st->cnt_a[(b % NXCD) * CNT_STRIDE]);
        }
    }
    if (w == GW - 2 && lane == 0) {
        const int ep = ld_agent(&st->epoch);
        ep_s = ep;
        st_agent(&st->checkin[b], ep + 1);
    }
    if (w == GW - 1) {
        const float inv = route_inv<NQ>(x, attn, D, eps);
        if (lane == 0) inv_s = inv;
    }
    __syncthreads();
    const int tag = ep_s + 1;
    /* the next launch's epoch, once every workgroup of this one has read it */
    if (b == nwg - 1) {
        bool ok = true;
        for (int i = tid; i < nwg; i += GW * 64) ok = wait_tag(&st->checkin[i], tag) && ok;
        if (!__syncthreads_and(ok) && tid == 0)
            __hip_atomic_fetch_add(timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (tid == 0) st_agent(&st->epoch, tag);
    }
    /* ---- B: every router row in, then the ranking, xn staged in between */
    if (!wait_counts(st->cnt_a, tag, E, &got_s) && tid == 0)
        __hip_atomic_fetch_add(timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const v4i_t rr = ld_agent16(st->rec, (uint32_t)(min(tid, E - 1) * sizeof(route_rec)));
    float *red = smem;                           /* GW * 64 */
    float *xs = red + GW * 64;                   /* xn (D), later the staged h (K * (F + 4)) */
    float *bsum = xs + max(max(D, K * (F + 4)), gu_lds_floats(nbd));   /* max(D/32, K * F/32) */
    float *gbs = xs + GU_XB * nbd;               /* within xs's region (gu_lds_floats) */
    auto stage_xn = [&]() {
        const float inv = inv_s;
        const float4 hh = attn ? make_float4(__fadd_rn(xa.x, aa.x), __fadd_rn(xa.y, aa.y),
                                             __fadd_rn(xa.z, aa.z), __fadd_rn(xa.w, aa.w))
                               : xa;
        const float4 xv = make_float4(__fmul_rn(__fmul_rn(hh.x, inv), ga.x),
                                      __fmul_rn(__fmul_rn(hh.y, inv), ga.y),
                                      __fmul_rn(__fmul_rn(hh.z, inv), ga.z),
                                      __fmul_rn(__fmul_rn(hh.w, inv), ga.w));
        gu_stage<ENC>(xs, gbs, tid, xv, hasx);
    };
    bool nonfinite;
    cert_rank_open(cl, rr, E, K, GW * 64, &nonfinite);
    stage_xn();
    cert_rank_close();
    /* ---- C: the gate/up and down weights of the ranked experts requested together, their
       fp16 scales kept raw until the dot products; the order certified while they fly */
    const bool has_gu = b < G;
    const int jg = has_gu ? b / nbf : 0, bg = has_gu ? b % nbf : 0;
    const int grow = bg * 32 + (lane & 31);
    const bool has_dn = b * R < D;
    const int jd = lane / R, drow = min(b * R, D - R) + lane % R;
    WBlk<ENC> wgv[BG];
    uint16_t sgv[BG];
    WBlk<ENC> wdv[BD];
    uint16_t sdv[BD];
    auto load_gu = [&](int eg) {
        if (has_gu)                              /* uniform in the workgroup */
            gu_load<ENC, BG>(experts + (size_t)eg * exp_stride, mat_bytes, pp_g, bg * 32, nbd,
                             wgv, sgv);
    };
    auto load_dn = [&](int ed) {
        if (has_dn)
            load_row_blocks_raw<ENC, BD>(experts + (size_t)ed * exp_stride + wd_off, pp_d, drow,
                                         w * BD, nbf - 1, nbf, wdv, sdv);
    };
    load_gu(cl.cslot[jg]);
    const bool cert = cert_check_wave(cl, K, nonfinite, force_exact, w == 0 ? tk_s : nullptr,
                                      w == 0 ? wt_s : nullptr);
    if (cert) load_dn(cl.cslot[jd]);
    if (!cert) {                                 /* the same in every workgroup */
        if (b == 0) {
            const bool full = route_fallback(x, attn, ln2, wgate, D, E, K, eps, smem, cl,
                                             nonfinite, inv_s, force_exact, sel, selw);
            mem_done();
            __syncthreads();
            if (tid == 0) {
                atomicAdd(stat, 1);
                if (full) atomicAdd(&stat[3], 1);
                st_agent(&st->selflag, tag);
            }
        } else {
            if (tid == 0) got_s = wait_tag(&st->selflag, tag);
            __syncthreads();
            if (!got_s) {
                if (tid == 0)
                    __hip_atomic_fetch_add(timeouts, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                route_fallback(x, attn, ln2, wgate, D, E, K, eps, smem, cl, nonfinite, inv_s,
                               force_exact, sel, selw);
                mem_done();
            }
            __syncthreads();
        }
        if (tid < K) {
            tk_s[tid] = ld_agent(&sel[tid]);
            wt_s[tid] = ld_agent(&selw[tid]);
        }
        __syncthreads();
        load_gu(tk_s[jg]);
        load_dn(tk_s[jd]);
        stage_xn();                              /* the fallback used the LDS */
    }
    lds_barrier();                               /* tk_s / wt_s; xn staged */
    if (b == 0 && tid < K) {
        if (topk_out) topk_out[tid] = tk_s[tid];
        if (wt_out) wt_out[tid] = wt_s[tid];
    }
    if (has_gu) {
        red[w * 64 + lane] = gu_dots<ENC, BG>(wgv, sgv, xs, gbs);
        lds_barrier();                           /* the down weights may still be in flight */
        if (w == 0) {
            float v = 0.0f;
            for (int ww = 0; ww < GW; ww++) v += red[ww * 64 + lane];
            const float u = __shfl(v, lane + 32);
            if (lane < 32) st_agent(&hbuf[(size_t)jg * F + grow], swiglu_t(v, u, tab));
            mem_done();                          /* the tile's h complete before its count */
            if (lane == 0) arrive(&st->cnt_g[(b % NXCD) * CNT_STRIDE]);
        }
    }
    if (!has_dn) return;
    /* ---- D: every gate/up tile in, then h staged and the down rows */
    if (!wait_counts(st->cnt_g, tag, G, &got_s) && tid == 0)
        __hip_atomic_fetch_add(timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int ld = F + 4, q = F / 4;
    for (int idx0 = 0; idx0 < K * q; idx0 += GW * 64) {
        const int idx = idx0 + tid, i = idx / q;
        const bool valid = idx < K * q;
        const v4i_t r = ld_agent16(hbuf, (uint32_t)(min(idx, K * q - 1) * 16));
        const float4 hv = make_float4(__int_as_float(r.x), __int_as_float(r.y),
                                      __int_as_float(r.z), __int_as_float(r.w));
        stage_put<ENC>(xs, bsum, ld, nbf, i, idx - i * q, hv, valid);
    }
    __syncthreads();
    const int nbw = max(0, min(BD, nbf - w * BD));
    float ddv[BD];
#pragma unroll
    for (int q = 0; q < BD; q++) ddv[q] = cpg_f16_to_f32(sdv[q]);
    float acc = 0.0f;
    row_dots_mc<ENC, 1, BD>(wdv, ddv, w * BD, nbw, xs + jd * ld, bsum + jd * nbf, ld, nbf, &acc);
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w == 0) {
        float y = 0.0f;
        for (int ww = 0; ww < GW; ww++) y += red[ww * 64 + lane];
        float o = 0.0f;
        if (!xres && lane < R) o = mlp[drow];
        for (int jj = 0; jj < K; jj++) {
            const float yj = __shfl(y, jj * R + lane % R);
            o = __fadd_rn(o, __fmul_rn(wt_s[jj], yj));
        }
        if (lane < R) {
            if (xres) xres[drow] = __fadd_rn(xres[drow], __fadd_rn(attn[drow], o));
            else mlp[drow] = o;
        }
    }
}

/* ================================================================ host side */


struct cpg_moe_ws {
    int D, E, K, F, max_T;
    float *xn, *logits, *wt, *gu, *y;
    int *topk, *pair_pos, *list_tok, *list_pair, *grp_expert, *grp_off, *grp_cnt, *n_groups;
    route_rec *rec;     /* SMALL_T * E: certified router sums and bounds */
    int *ctr;           /* SMALL_T + 1 arrival counters of k_route_fast (zero between calls) */
    int *ctr2;          /* max_T * D/64 arrival counters of k_down_mm (zero between calls) */
    int *stat;          /* [0] tokens whose certificate failed (the refined or the exact
                           fallback) since creation; [1] the one-token fallback routings
                           k_gateup1's workgroup 0 has published; [2] [1] as it stood when
                           the current call's routing ran; [3] tokens that needed the exact
                           chains for every row */
    int *chunk_grp, *chunk_m0;  /* prefill: chunks of up to 64 tokens of one expert group */
    moe1_state *st1;            /* k_moe1: its epoch, tags and tagged router records */
    int *timeouts;              /* k_moe1: waits that gave up */
    int *sel;                   /* k_moe1: exact fallback routing, K ids then K weights */
    int *xsel;                  /* one token: the selection (K ids, then the K weights' bits)
                                   once per XCD, written by a k_gateup1 workgroup on it */
    void *block;
};

/* The workspace laid out from `base` (nothing is written when base is null); returns its
   size. The arrival counters and epochs, which must be zero when a workspace is first used
   and which the kernels leave zero (or monotone) after every call, come first and are sized
   for (cnt_D, cnt_T) >= (D, max_T): with fixed sizes they stay at the same offsets whatever
   geometry a shared scratch region is later carved for. */
static size_t moe_ws_carve(cpg_moe_ws *ws, uint8_t *base, int D, int E, int K, int F,
                           int max_T, int cnt_D, int cnt_T) {
    const size_t TK = (size_t)max_T * K;
    enum { N = 23 };
    const size_t mc = (size_t)cpg_prefill_max_chunks(max_T, K, E);
    const size_t sz[N] = {(SMALL_T + 1) * 4, (size_t)cnt_T * (cnt_D / 64) * 4, 16,
                          sizeof(moe1_state), 4,
                          (size_t)max_T * D * 4, (size_t)max_T * E * 4, TK * 4,
                          TK * 2 * KS * F * 4, TK * D * 4, TK * 4, TK * 4, TK * 4, TK * 4,
                          (size_t)E * 4, (size_t)E * 4, (size_t)E * 4, 256,
                          (size_t)SMALL_T * E * sizeof(route_rec), mc * 4, mc * 4,
                          (size_t)2 * K * 4, (size_t)NXCD * 2 * K * 4};
    void **dst[N] = {(void **)&ws->ctr, (void **)&ws->ctr2, (void **)&ws->stat,
                     (void **)&ws->st1, (void **)&ws->timeouts,
                     (void **)&ws->xn, (void **)&ws->logits, (void **)&ws->wt, (void **)&ws->gu,
                     (void **)&ws->y, (void **)&ws->topk, (void **)&ws->pair_pos,
                     (void **)&ws->list_tok, (void **)&ws->list_pair, (void **)&ws->grp_expert,
                     (void **)&ws->grp_off, (void **)&ws->grp_cnt, (void **)&ws->n_groups,
                     (void **)&ws->rec, (void **)&ws->chunk_grp, (void **)&ws->chunk_m0,
                     (void **)&ws->sel, (void **)&ws->xsel};
    size_t off = 0;
    for (int i = 0; i < N; i++) {
        if (base) *dst[i] = base + off;
        off += cpg_round256(sz[i]);
    }
    if (base) {
        ws->D = D; ws->E = E; ws->K = K; ws->F = F; ws->max_T = max_T;
        ws->block = base;
    }
    return off;
}

static bool moe_ws_geometry_ok(int D, int E, int K, int F, int max_T) {
    return D > 0 && D % 64 == 0 && E > 0 && E <= MAX_E && K > 0 && K <= MAX_K && K <= E &&
           F > 0 && max_T > 0 && max_T <= BUCKET_MAX_T;
}

extern "C" cpg_moe_ws *cpg_moe_ws_create(int D, int E, int K, int F, int max_T) {
    if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return nullptr; }
    if (!moe_ws_geometry_ok(D, E, K, F, max_T)) {
        cpg_set_error("cpg_moe_ws_create: bad geometry D=%d E=%d K=%d F=%d max_T=%d "
                      "(D a multiple of 64, E <= %d, K <= %d, max_T <= %d)", D, E, K, F, max_T,
                      MAX_E, MAX_K, BUCKET_MAX_T);
        return nullptr;
    }
    cpg_moe_ws *ws = (cpg_moe_ws *)calloc(1, sizeof *ws);
    if (!ws) { cpg_set_error("out of host memory"); return nullptr; }
    const size_t total = moe_ws_carve(ws, nullptr, D, E, K, F, max_T, D, max_T);
    uint8_t *p = (uint8_t *)cpg_malloc(total);
    if (!p) { free(ws); return nullptr; }
    moe_ws_carve(ws, p, D, E, K, F, max_T, D, max_T);
    /* everything zero: the counters must start at zero, the rest is defined */
    if (cpg_memset(ws->block, 0, total) || cpg_sync()) {
        cpg_free(ws->block);
        free(ws);
        return nullptr;
    }
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

extern "C" int cpg_moe_ws_fallbacks(cpg_moe_ws *ws) {
    CPG_REQUIRE_INIT();
    int n = 0;
    if (cpg_sync() || cpg_d2h(&n, ws->stat, sizeof n)) return -7;
    return n;
}

extern "C" int cpg_moe_ws_exact_routings(cpg_moe_ws *ws) {
    CPG_REQUIRE_INIT();
    int n = 0;
    if (cpg_sync() || cpg_d2h(&n, ws->stat + 3, sizeof n)) return -7;
    return n;
}

extern "C" int cpg_moe_ws_status(cpg_moe_ws *ws) {
    CPG_REQUIRE_INIT();
    int n = 0;
    if (cpg_sync() || cpg_d2h(&n, ws->timeouts, sizeof n)) return -7;
    return n;
}

static int g_fused = 0;   /* measured slower than the separate kernels: opt-in */

extern "C" int cpg_moe_fused(int enable) {
    g_fused = enable != 0;
    return 0;
}

static int g_route_mode = CPG_ROUTE_AUTO;
static int g_expert_mode = CPG_EXPERTS_AUTO;

extern "C" int cpg_moe_expert_mode(int mode) {
    if (mode < CPG_EXPERTS_AUTO || mode > CPG_EXPERTS_MFMA) {
        cpg_set_error("unknown expert mode %d", mode);
        return -1;
    }
    g_expert_mode = mode;
    return 0;
}

/* the kernels' force argument: 1 fails every certificate and skips the refined step (the
   exact chains for every token), 2 fails every certificate (the refined step for every
   token, then the exact chains where it does not certify) */
static int route_force() {
    return g_route_mode == CPG_ROUTE_FORCE_FALLBACK ? FORCE_EXACT_CHAINS
           : g_route_mode == CPG_ROUTE_FORCE_REFINE ? FORCE_EXACT_CHAINS + 1
                                                     : 0;
}

extern "C" int cpg_moe_route_mode(int mode) {
    if (mode < CPG_ROUTE_AUTO || mode > CPG_ROUTE_FORCE_REFINE) {
        cpg_set_error("unknown routing mode %d", mode);
        return -1;
    }
    g_route_mode = mode;
    return 0;
}

/* ---- per-kernel timing: while enabled, launches go through hipExtLaunchKernel with an event
   pair, whose elapsed time is the kernel's own execution (no extra packets in the stream) */
#define TIMING_MAX 8192
static struct {
    int on;
    int n[CPG_KT_COUNT];
    hipEvent_t ev[CPG_KT_COUNT][TIMING_MAX][2];
} g_timing;

extern "C" int cpg_moe_timing(int enable) {
    CPG_REQUIRE_INIT();
    g_timing.on = enable != 0;
    for (int k = 0; k < CPG_KT_COUNT; k++) g_timing.n[k] = 0;
    return 0;
}

extern "C" int cpg_moe_timing_read(double *ms, int *launches, int n) {
    CPG_REQUIRE_INIT();
    for (int k = 0; k < CPG_KT_COUNT && k < n; k++) {
        double tot = 0.0;
        for (int i = 0; i < g_timing.n[k]; i++) {
            float a = 0.0f;
            CPG_HIP(hipEventSynchronize(g_timing.ev[k][i][1]));
            CPG_HIP(hipEventElapsedTime(&a, g_timing.ev[k][i][0], g_timing.ev[k][i][1]));
            tot += a;
        }
        if (ms) ms[k] = tot;
        if (launches) launches[k] = g_timing.n[k];
        g_timing.n[k] = 0;
    }
    return 0;
}

static int g_noalloc_call;   /* inside cpg_moe_forward_noalloc: no event is created */

/* the event pair for the next timed launch of kernel slot k, or null when not timing */
hipEvent_t *cpg_timing_pair(int k) {
    if (!g_timing.on || g_noalloc_call || g_timing.n[k] >= TIMING_MAX) return nullptr;
    hipEvent_t *e = g_timing.ev[k][g_timing.n[k]];
    for (int i = 0; i < 2; i++)
        if (!e[i] && hipEventCreate(&e[i]) != hipSuccess) return nullptr;
    g_timing.n[k]++;
    return e;
}

/* LAUNCH(slot, kern, grid, block, smem, args...): cpg_internal.h */

static int check_layer(const cpg_moe_layer *L, int T, const cpg_moe_ws *ws) {
    if (!L || !ws || !L->wgate || !L->ln2 || !L->experts) { cpg_set_error("null layer/workspace"); return -1; }
    if (L->enc != CPG_ENC_Q4 && L->enc != CPG_ENC_Q8) { cpg_set_error("expert encoding %d unsupported", L->enc); return -1; }
    if (L->D != ws->D || L->E != ws->E || L->K != ws->K || L->F != ws->F) {
        cpg_set_error("workspace geometry does not match the layer"); return -1;
    }
    if (T <= 0 || T > ws->max_T) { cpg_set_error("T=%d outside [1, %d]", T, ws->max_T); return -1; }
    /* shapes the kernels assume: 64-row tiles; the gate/up kernels' GW wavefronts share D's
       blocks evenly (1, 2, 3, 4 or 8 each); at most MAX_BPW blocks of F per lane; serial
       chains over multiples of 64 */
    const int nbd = L->D / 32, nbf = L->F / 32, bg = nbd / GW;
    if (L->D % (32 * GW) || L->D % 64 || L->F % 64 || bg < 1 || (bg > 4 && bg != 8) ||
        (nbf + GW - 1) / GW > MAX_BPW) {
        cpg_set_error("unsupported shape D=%d F=%d: D a multiple of %d up to %d (or %d), F of "
                      "64 up to %d", L->D, L->F, 32 * GW, 4 * 32 * GW, 8 * 32 * GW,
                      GW * MAX_BPW * 32);
        return -1;
    }
    return 0;
}

static int route_fast(const cpg_moe_layer *L, const float *x, const float *attn, int T, int *tk,
                      float *wt, int select, int bucket, cpg_moe_ws *ws, bool planes = false) {
    const int D = L->D, E = L->E;
    /* select == 0: one router row per one-wavefront workgroup; the exact fallback then runs
       in the expert kernel, so no LDS for it here */
    const int rr = route_rows(D / 256);
    const dim3 grid(select ? (E + rr - 1) / rr : E, T), block(select ? 64 * rr : 64);
    const size_t smem = select ? sizeof(float) * fallback_lds_floats(D, E) : 0;
    const int force = route_force();
    /* planes (many tokens on the MFMA GEMMs): the routing step also writes xn's hi/lo planes
       (in the expert scratch) and the chunk list */
    _Float16 *xh = planes ? (_Float16 *)ws->gu : nullptr;
    const int mc = planes ? cpg_prefill_max_chunks(T, L->K, E) : 0;
#define ROUTE_FAST_ARGS x, attn, L->ln2, L->wgate, T, D, E, L->K, L->eps, force, ws->xn, ws->rec, ws->ctr, \
        tk, wt, ws->stat, select, bucket, ws->pair_pos, ws->list_tok, ws->list_pair, ws->grp_expert, ws->grp_off,  \
        ws->grp_cnt, ws->n_groups, xh, xh ? xh + (size_t)T * D : nullptr, mc, \
        planes ? ws->chunk_grp : nullptr, ws->chunk_m0
    switch (D / 256) {
    case 1: LAUNCH(CPG_KT_ROUTE, k_route_fast<1>, grid, block, smem, ROUTE_FAST_ARGS); break;
    case 2: LAUNCH(CPG_KT_ROUTE, k_route_fast<2>, grid, block, smem, ROUTE_FAST_ARGS); break;
    case 4: LAUNCH(CPG_KT_ROUTE, k_route_fast<4>, grid, block, smem, ROUTE_FAST_ARGS); break;
    case 8: LAUNCH(CPG_KT_ROUTE, k_route_fast<8>, grid, block, smem, ROUTE_FAST_ARGS); break;
    default: LAUNCH(CPG_KT_ROUTE, k_route_fast<16>, grid, block, smem, ROUTE_FAST_ARGS); break;
    }
#undef ROUTE_FAST_ARGS
    return 0;
}

/* ---- expert GEMV launches, one instantiation per encoding and blocks per lane */
struct gemv_args {
    const cpg_moe_layer *L;
    const float *x;         /* k_gateup1: the token (its exact routing, when not certified) */
    const float *xn;
    const int *tk;
    const float *wt;
    float *mlp;
    cpg_moe_ws *ws;
    int gmax;
    int T;
    float *xres;            /* k_down1: take the residual into xres (with attn) instead of mlp */
    const float *attn;
};

/* the per-XCD copies of the one-token selection: used when k_gateup1 has a workgroup on
   every XCD (grid F/32 * K >= 8; a grid of F/24 * K is larger) */
static int *xsel_of(const gemv_args &a) {
    return a.L->F / 32 * a.L->K >= NXCD ? a.ws->xsel : nullptr;
}

/* k_gateup1's rows per matrix and workgroup: 24 where they divide F and the lane groups are
   of 8 (B == 8), so that F = 768 and K = 8 give 256 workgroups, one per CU */
template <int B>
static int gateup1_rows(int F) {
    return B == 8 && F % 24 == 0 ? 24 : 32;
}

template <int ENC, int B>
static int launch_gateup1(const gemv_args &a) {
    const cpg_moe_layer *L = a.L;
    const int D = L->D, F = L->F, E = L->E, nr = gateup1_rows<B>(F);
    auto kfn = nr == 24 ? k_gateup1<ENC, B, B == 8 ? 24 : 32> : k_gateup1<ENC, B, 32>;
    const size_t smem = sizeof(float) * max((size_t)gu_lds_floats(D / 32) + GW * 64,
                                            fallback_lds_floats(D, E));
    LAUNCH(CPG_KT_GATEUP, kfn, dim3(F / nr * L->K), dim3(GW * 64), smem,
           (const uint8_t *)L->experts, cpg_expert_bytes(ENC, D, F), cpg_matrix_bytes(ENC, F, D),
           cpg_payload_plane(ENC, F, D), D, F, a.ws->rec, E, L->K,
           route_force(), a.x, a.attn, L->ln2, L->wgate, L->eps,
           (int *)a.tk, (float *)a.wt, a.ws->stat, a.xn, a.ws->gu, xsel_of(a));
    return 0;
}

template <int ENC, int B>
static int launch_down1(const gemv_args &a) {
    auto kfn = k_down1<ENC, B>;
    const cpg_moe_layer *L = a.L;
    const int D = L->D, F = L->F, K = L->K;
    const size_t smem = sizeof(float) * ((size_t)K * (F + 4) + K * (F / 32) + GW * 64);
    LAUNCH(CPG_KT_DOWN, kfn, dim3(D / (WAVE / K)), dim3(GW * 64), smem,
           (const uint8_t *)L->experts, cpg_expert_bytes(ENC, D, F),
           2 * cpg_matrix_bytes(ENC, F, D), cpg_payload_plane(ENC, D, F), D, F, K, a.tk,
           a.ws->gu, a.wt, a.mlp, a.xres, a.attn, (const int *)xsel_of(a));
    return 0;
}

/* blocks per lane B in 1..4 (and 8 where allowed) */
#define BPW_CASES(FN, ENC, bpw, a)                                                        \
    switch (bpw) {                                                                        \
    case 1: return FN<ENC, 1>(a);                                                         \
    case 2: return FN<ENC, 2>(a);                                                         \
    case 3: return FN<ENC, 3>(a);                                                         \
    case 4: return FN<ENC, 4>(a);                                                         \
    default: break;                                                                       \
    }

template <int ENC>
static int launch_gateup_mm(const gemv_args &a) {
    const cpg_moe_layer *L = a.L;
    const int D = L->D, F = L->F, nw = D / (32 * MM_BPW);
    const size_t smem = sizeof(float) * 1024 * nw + 4 * (size_t)D;   /* sums, scales */
    cpg_moe_ws *ws = a.ws;
    LAUNCH(CPG_KT_GATEUP, k_gateup_mm<ENC>, dim3(F / 32 * a.gmax), dim3(64 * nw), smem,
           (const uint8_t *)L->experts, cpg_expert_bytes(ENC, D, F), cpg_matrix_bytes(ENC, F, D),
           cpg_payload_plane(ENC, F, D), D, F, nw, ws->grp_expert, ws->grp_off, ws->grp_cnt,
           ws->list_tok, a.xn, ws->gu);
    return 0;
}

template <int ENC>
static int launch_down_mm(const gemv_args &a) {
    const cpg_moe_layer *L = a.L;
    const int D = L->D, F = L->F, nw = (F / 32 + MM_BPWD - 1) / MM_BPWD;
    const size_t smem = sizeof(float) * 1024 * nw;
    cpg_moe_ws *ws = a.ws;
    if (smem > 64 * 1024)
        CPG_HIP(hipFuncSetAttribute((const void *)k_down_mm<ENC>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    LAUNCH(CPG_KT_DOWN, k_down_mm<ENC>, dim3(D / 64, a.gmax), dim3(64 * nw), smem,
           (const uint8_t *)L->experts, cpg_expert_bytes(ENC, D, F),
           2 * cpg_matrix_bytes(ENC, F, D), cpg_payload_plane(ENC, D, F), D, F, L->K, nw,
           ws->grp_expert, ws->grp_off, ws->grp_cnt, ws->list_tok, ws->list_pair, ws->gu, ws->y,
           a.wt, ws->ctr2, a.mlp);
    return 0;
}

template <int ENC>
static int gemvs_grouped(const gemv_args &a) {
    /* the shapes check_layer admits: D / 128 <= 16 wavefronts of 4 blocks, F / 96 <= 16 of 3 */
    const int rc = launch_gateup_mm<ENC>(a);
    return rc ? rc : launch_down_mm<ENC>(a);
}

template <int ENC>
static int gemvs_one(const gemv_args &a) {
    const int bg = a.L->D / 32 / GW, bd = (a.L->F / 32 + GW - 1) / GW;
    int rc = -1;
    switch (bg) {
    case 1: rc = launch_gateup1<ENC, 1>(a); break;
    case 2: rc = launch_gateup1<ENC, 2>(a); break;
    case 4: rc = launch_gateup1<ENC, 4>(a); break;
    case 8: rc = launch_gateup1<ENC, 8>(a); break;
    default: cpg_set_error("k_gateup1: %d blocks per lane unsupported", bg); return -1;
    }
    if (rc) return rc;
    BPW_CASES(launch_down1, ENC, bd, a);
    cpg_set_error("k_down1: %d blocks per lane unsupported", bd);
    return -1;
}

/* ---- the fused one-token kernel */
struct moe1_geom {
    int nwg;
    size_t smem;
};

static moe1_geom moe1_shape(int D, int E, int K, int F) {
    const int R = WAVE / K;
    int nwg = E;
    nwg = max(nwg, F / 32 * K);
    nwg = max(nwg, (D + R - 1) / R);
    const size_t xs = (size_t)max(max(D, K * (F + 4)), gu_lds_floats(D / 32)),
                 bs = (size_t)max(D / 32, K * F / 32);
    size_t smem = sizeof(float) * ((size_t)GW * 64 + xs + bs);
    smem = max(smem, sizeof(float) * fallback_lds_floats(D, E));   /* the fallback */
    return {nwg, smem};
}

template <int ENC, int NQ, int BG, int BD>
static int launch_moe1(const cpg_moe_layer *L, const float *x, const float *attn, int *tk,
                       float *wt, float *mlp, float *xres, cpg_moe_ws *ws) {
    auto kfn = k_moe1<ENC, NQ, BG, BD>;
    const int D = L->D, E = L->E, K = L->K, F = L->F;
    const moe1_geom gm = moe1_shape(D, E, K, F);
    /* every workgroup must be resident at once for the waits between phases: checked once */
    static int resident = -1;
    if (resident < 0) {
        int per_cu = 0, dev = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)kfn, GW * 64,
                                                         gm.smem) != hipSuccess ||
            hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            per_cu = 0;
        resident = (long)per_cu * cus >= gm.nwg;
    }
    if (!resident || gm.nwg > MOE1_MAX_TILES) return 1;   /* the caller takes the three kernels */
    const size_t es = cpg_expert_bytes(ENC, D, F), mg = cpg_matrix_bytes(ENC, F, D);
    LAUNCH(CPG_KT_FUSED, kfn, dim3(gm.nwg), dim3(GW * 64), gm.smem, x, attn, L->ln2, L->wgate, D,
           E, K, F, L->eps, route_force(), (const uint8_t *)L->experts,
           es, mg, cpg_payload_plane(ENC, F, D), 2 * mg, cpg_payload_plane(ENC, D, F), ws->st1,
           ws->gu, ws->sel, (float *)(ws->sel + K), ws->stat, ws->timeouts, tk, wt, mlp, xres);
    return 0;
}

/* 0 launched, 1 not applicable (shape or residency), < 0 error */
static int moe1(const cpg_moe_layer *L, const float *x, const float *attn, int *tk, float *wt,
                float *mlp, float *xres, cpg_moe_ws *ws) {
    const int D = L->D, K = L->K, F = L->F;
    if (D != 2048 || F % 32 || (F / 32 + GW - 1) / GW != 3 || WAVE % K || K > MAX_K ||
        F / 32 * K > MOE1_MAX_TILES || L->E > MAX_E)
        return 1;                                /* the instantiated shape: Qwen3-30B-A3B */
    return L->enc == CPG_ENC_Q4 ? launch_moe1<CPG_ENC_Q4, 8, 8, 3>(L, x, attn, tk, wt, mlp, xres, ws)
                                : launch_moe1<CPG_ENC_Q8, 8, 8, 3>(L, x, attn, tk, wt, mlp, xres, ws);
}

/* shapes k_gateup1 / k_down1 assume */
static bool one_token_shape(int D, int K, int F) {
    const int nb = D / 32, R = WAVE / K, bg = nb / GW, bd = (F / 32 + GW - 1) / GW;
    return D % 32 == 0 && nb % GW == 0 && (bg == 1 || bg == 2 || bg == 4 || bg == 8) &&
           D <= 4 * GW * 64 && F % 32 == 0 && bd >= 1 && bd <= MAX_BPW && WAVE % K == 0 &&
           D % R == 0 && K * F <= HMAX * 4 * GW * 64;
}

static bool fast_shape(int D) {
    const int q = D / 256;
    return D % 256 == 0 && (q == 1 || q == 2 || q == 4 || q == 8 || q == 16);
}

static int moe_forward(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                       float *xn, float *router, int *topk, float *wt, float *mlp,
                       cpg_moe_ws *ws, float *xres);

extern "C" int cpg_moe_forward(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                               float *xn, float *router, int *topk, float *wt, float *mlp,
                               cpg_moe_ws *ws) {
    return moe_forward(L, x, attn, T, xn, router, topk, wt, mlp, ws, nullptr);
}

/* cpg_moe_forward with its workspace carved from the static scratch instead of a
   cpg_moe_ws: T <= CPG_NOALLOC_MAX_T tokens, a geometry whose workspace fits the scratch. The
   counters come first in the carve at fixed offsets (sized for D up to NOALLOC_CNT_D), so
   they are the same words whatever geometry a call carves: zero when the context was
   created and left zero by every call. Nothing is allocated: the host-side workspace
   descriptor lives on the stack and no timing event is created. */
#define NOALLOC_CNT_D 8192

extern "C" int cpg_moe_forward_noalloc(const cpg_moe_layer *L, const float *x,
                                       const float *attn, int T, float *xn, float *router,
                                       int *topk, float *wt, float *mlp) {
    CPG_REQUIRE_INIT();
    if (!L) { cpg_set_error("cpg_moe_forward_noalloc: null layer"); return -1; }
    if (T <= 0 || T > CPG_NOALLOC_MAX_T) {
        cpg_set_error("cpg_moe_forward_noalloc: T=%d outside [1, %d]", T, CPG_NOALLOC_MAX_T);
        return -1;
    }
    if (!moe_ws_geometry_ok(L->D, L->E, L->K, L->F, CPG_NOALLOC_MAX_T) || L->D > NOALLOC_CNT_D) {
        cpg_set_error("cpg_moe_forward_noalloc: bad geometry D=%d E=%d K=%d F=%d", L->D, L->E,
                      L->K, L->F);
        return -1;
    }
    size_t have = 0;
    uint8_t *base = (uint8_t *)cpg_static_scratch(&have);
    cpg_moe_ws w;
    memset(&w, 0, sizeof w);
    const size_t need = moe_ws_carve(&w, nullptr, L->D, L->E, L->K, L->F, CPG_NOALLOC_MAX_T,
                                     NOALLOC_CNT_D, CPG_NOALLOC_MAX_T);
    if (!base || need > have) {
        cpg_set_error("cpg_moe_forward_noalloc: this geometry needs %zu bytes of scratch, the "
                      "static scratch holds %zu", need, have);
        return -1;
    }
    moe_ws_carve(&w, base, L->D, L->E, L->K, L->F, CPG_NOALLOC_MAX_T, NOALLOC_CNT_D,
                 CPG_NOALLOC_MAX_T);
    g_noalloc_call = 1;
    const int rc = moe_forward(L, x, attn, T, xn, router, topk, wt, mlp, &w, nullptr);
    g_noalloc_call = 0;
    return rc;
}

/* x += attn + MoE(x + attn), the layer's residual (cachepotato.c:157-159). One token: folded
   into the down projection's combine. More: mlp (zero on entry) accumulates, then
   cpg_residual adds and clears it. */
extern "C" int cpg_moe_forward_res(const cpg_moe_layer *L, float *x, const float *attn, int T,
                                   int *topk, float *mlp, cpg_moe_ws *ws) {
    if (!attn) { cpg_set_error("cpg_moe_forward_res: attn is required"); return -1; }
    return moe_forward(L, x, attn, T, nullptr, nullptr, topk, nullptr, mlp, ws, x);
}

static int moe_forward(const cpg_moe_layer *L, const float *x, const float *attn, int T,
                       float *xn, float *router, int *topk, float *wt, float *mlp,
                       cpg_moe_ws *ws, float *xres) {
    CPG_REQUIRE_INIT();
    if (check_layer(L, T, ws)) return -1;
    if (!x || !mlp) { cpg_set_error("x and mlp are required"); return -1; }
    const int D = L->D, E = L->E, K = L->K, F = L->F, enc = L->enc;
    float *xn_d = xn ? xn : ws->xn;
    float *lg_d = router ? router : ws->logits;
    int *tk_d = topk ? topk : ws->topk;
    float *wt_d = wt ? wt : ws->wt;

    /* many tokens: the expert products as MFMA grouped GEMMs (prefill.hip) */
    const bool mfma = cpg_prefill_shape_ok(D, F) &&
                      cpg_prefill_scratch_bytes(T, D, K, F) <= (size_t)T * K * 2 * KS * F * 4 &&
                      (g_expert_mode == CPG_EXPERTS_MFMA ||
                       (g_expert_mode == CPG_EXPERTS_AUTO && T >= PREFILL_MIN_T));
    bool prepared = false;      /* chunk list and xn planes formed by the routing step */

    /* routing, selection, bucketing */
    const bool fast = T <= SMALL_T && !xn && !router && g_route_mode != CPG_ROUTE_EXACT &&
                      fast_shape(D);
    const bool one = fast && T == 1 && one_token_shape(D, K, F) && E * CR_P <= GW * 64;
    if (one && g_fused) {
        const int rc = moe1(L, x, attn, topk, wt, mlp, xres, ws);
        if (rc <= 0) return rc ? -7 : 0;
    }
    /* up to 16 tokens on the MFMA GEMMs: they find their experts' pairs in the selections
       themselves, so the routing launch does not group them */
    const bool sel = fast && !one && mfma && cpg_prefill_sel_ok(T, K, E);
    if (fast) {
        if (route_fast(L, x, attn, T, tk_d, wt_d, !one, !one && !sel, ws, mfma && !one))
            return -7;
        prepared = mfma && !one;
    } else if (T <= SMALL_T) {
        const size_t smem = sizeof(float) * ((size_t)2 * D + (size_t)RPW * (D + 4));
        LAUNCH(CPG_KT_ROUTE, k_route_small, dim3((E + RPW - 1) / RPW, T), dim3(256), smem, x,
               attn, L->ln2, L->wgate, D, E, L->eps, xn_d, lg_d);
        LAUNCH(CPG_KT_SELECT, k_select_bucket, dim3(1), dim3(64 * T), 0, lg_d, T, E, K, tk_d,
               wt_d, ws->pair_pos, ws->list_tok, ws->list_pair, ws->grp_expert, ws->grp_off,
               ws->grp_cnt, ws->n_groups);
    } else {
        if (D % 64) { cpg_set_error("routing of %d tokens needs D %% 64 == 0", T); return -1; }
        if (D % 4 || D > 4 * 256 * RN_V4) {
            cpg_set_error("routing of %d tokens needs D %% 4 == 0 and D <= %d", T, 4 * 256 * RN_V4);
            return -1;
        }
        /* for the MFMA GEMMs the norm also writes the hi/lo planes of xn and the bucketing
           the chunk list */
        _Float16 *xh = mfma ? (_Float16 *)ws->gu : nullptr;
        LAUNCH(CPG_KT_ROUTE, k_rmsnorm_tok, dim3(T), dim3(256), sizeof(float) * (size_t)D, x,
               attn, L->ln2, D, L->eps, xn_d, xh, xh ? xh + (size_t)T * D : nullptr);
        const dim3 rgrid((T + RL_TOK - 1) / RL_TOK, (E + RL_ROWS - 1) / RL_ROWS);
        if (D % 128 == 0)
            LAUNCH(CPG_KT_ROUTE, k_router_tok<128>, rgrid, dim3(256), 0, xn_d, L->wgate, T, D, E,
                   lg_d);
        else
            LAUNCH(CPG_KT_ROUTE, k_router_tok<64>, rgrid, dim3(256), 0, xn_d, L->wgate, T, D, E,
                   lg_d);
        LAUNCH(CPG_KT_SELECT, k_select, dim3(T), dim3(64), 0, lg_d, E, K, tk_d, wt_d);
        LAUNCH(CPG_KT_SELECT, k_bucket, dim3(1), dim3(1024), 0, tk_d, T, K, E, ws->pair_pos,
               ws->list_tok, ws->list_pair, ws->grp_expert, ws->grp_off, ws->grp_cnt,
               ws->n_groups, cpg_prefill_max_chunks(T, K, E), mfma ? ws->chunk_grp : nullptr,
               ws->chunk_m0);
        prepared = mfma;
    }
    gemv_args a{L, x, xn_d, tk_d, wt_d, mlp, ws, T * K < E ? T * K : E, T, nullptr, nullptr};
    if (one) {
        a.xres = xres;
        a.attn = attn;
        return enc == CPG_ENC_Q4 ? gemvs_one<CPG_ENC_Q4>(a) : gemvs_one<CPG_ENC_Q8>(a);
    }
    /* many tokens: the MFMA grouped GEMMs over chunks of each expert's tokens */
    if (mfma)       /* the hi/lo planes live in the GEMV partials' space (TK*2*KS*F floats) */
        return cpg_prefill_experts(L, T, xn_d, wt_d, ws->grp_expert, ws->grp_off, ws->grp_cnt,
                                   ws->list_tok, ws->list_pair, ws->chunk_grp, ws->chunk_m0,
                                   ws->gu, ws->y, mlp, xres, attn, prepared,
                                   sel ? tk_d : nullptr, ws->n_groups);

    /* expert GEMVs over at most min(E, T*K) groups; the combine is fused into k_down_mm */
    const int rc = enc == CPG_ENC_Q4 ? gemvs_grouped<CPG_ENC_Q4>(a) : gemvs_grouped<CPG_ENC_Q8>(a);
    if (rc || !xres) return rc;
    return cpg_residual(xres, attn, mlp, (size_t)T * D);
}
