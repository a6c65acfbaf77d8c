/* attn.hip — the attention half of a Qwen3 decoder layer on gfx950, plus the row-tiled GEMV
 * it (and the output head) uses.
 *
 * Reference: engine/blocks/qwen3_moe.c:110-167 (attention half of qwen3_layer_kv), with
 * engine/kernels/kernels.c rmsnorm :408-413, rope_apply_from :425-447, softmax :20-26, and the
 * per-head RMSNorm of qwen3_moe.c:44-49.
 *
 * One call for T new tokens at positions pos0..pos0+T-1, on one stream:
 *   k_gemv           q|k|v = [Wq; Wk; Wv] . rmsnorm(x, ln1), one row-tiled matrix of
 *                    (H + 2 KV) * HD rows, the norm folded into the staging of x (its sum of
 *                    squares in double, then the reference's float formula for 1/sqrt).
 *   k_qk_norm_rope   per head: the reference's RMSNorm of the head (serial sum of squares, so
 *                    bit-identical given the same q/k), then RoPE with a cos/sin table the
 *                    host computes with the same libm calls as the reference; k and v rows go
 *                    to the cache at pos0 + t.
 *   attention        T = 1: k_attn_split (or k_attn_decode); T > 1: k_attn_mma on MFMA for
 *                    head dim 128 and G = H/KV dividing 16, else k_attn_blk or k_attn_core.
 *                    Scores q.k_j / sqrtf(HD), softmax with the glibc-identical expf, the
 *                    weighted sum over positions; the sums run in another order than the
 *                    reference's serial loops (fp32, ~1e-7 to 1e-6 relative).
 *   k_gemv           attn = Wo . ao.
 * From DENSE_MIN_T tokens on, both projections run as MFMA GEMMs instead (k_mfma_dense and
 * k_sum_parts of prefill.hip): k_rmsnorm_rows_hilo writes ln1's output as the hi + lo f16
 * planes of the q|k|v product, k_qk_norm_rope adds that product's k parts as it reads them,
 * and the attention core writes the planes of the Wo product; exact f16 weight integers, fp32
 * accumulation with the block scale applied in fp32, the k range split into parts summed in a
 * fixed order. The projections accumulate in fp32 in a different order than the CPU GEMVs
 * (within ~1e-6 relative), which is what separates this path from the reference's bits.
 *
 * The position of the first new token is either an argument or read from device memory
 * (cpg_attn_forward_at), so that a decode step can be captured once as a HIP graph and
 * replayed at every position; kernels that read it check the cache bound themselves.
 */
#include "cpg_internal.h"
#include "cpg_gemv.h"
#include "cpg_mfma.h"

#include <math.h>
#include <stdlib.h>

#define GROWS 16            /* k_gemv: rows per workgroup (8 where that fills more CUs) */
#define GSLICES (4 * GW)    /* k_gemv: k slices per row (4 per wavefront) */
#define AV_DEPTH 8          /* k_attn_decode: value rows per thread per batch */
#define ADT 512             /* k_attn_decode: threads (ADT / 8 key rows per pass) */
#define AP 32               /* k_attn_split: positions per workgroup */
#define AG 8                /* k_attn_split: query heads per kv head */
#define AHD 128             /* k_attn_split: head dimension */
#define ASPLIT_MAX_POS 32768 /* k_attn_split: positions its workspace holds */
#define AMG 16              /* k_attn_split: splits merged per group of loads */

/* grid T, 256 threads: out[t] = (x[t] * inv) * g with inv = rms_inv_row(x[t]) */
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ x,
                                                      const float *__restrict__ g, int D,
                                                      float eps, float *__restrict__ out) {
    __shared__ double part[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float inv = rms_inv_row(x + (size_t)t * D, D, eps, part);
    const float4 *x4 = (const float4 *)(x + (size_t)t * D);
    const float4 *g4 = (const float4 *)g;
    float4 *o4 = (float4 *)(out + (size_t)t * D);
    for (int i = tid; i < D / 4; i += 256) {
        const float4 v = x4[i], gv = g4[i];
        o4[i] = make_float4(__fmul_rn(__fmul_rn(v.x, inv), gv.x), __fmul_rn(__fmul_rn(v.y, inv), gv.y),
                            __fmul_rn(__fmul_rn(v.z, inv), gv.z), __fmul_rn(__fmul_rn(v.w, inv), gv.w));
    }
}

/* the same rows as k_rmsnorm_rows, written as the hi/lo f16 planes of the dense MFMA
   product (hi = f16(v), lo = f16(v - hi), the arithmetic of k_split_hilo) instead of fp32 */
__global__ __launch_bounds__(256) void k_rmsnorm_rows_hilo(const float *__restrict__ x,
                                                           const float *__restrict__ g, int D,
                                                           float eps, _Float16 *__restrict__ hi,
                                                           _Float16 *__restrict__ lo) {
    __shared__ double part[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float inv = rms_inv_row(x + (size_t)t * D, D, eps, part);
    const float4 *x4 = (const float4 *)(x + (size_t)t * D);
    const float4 *g4 = (const float4 *)g;
    for (int i = tid; i < D / 4; i += 256) {
        const float4 v = x4[i], gv = g4[i];
        const float o[4] = {__fmul_rn(__fmul_rn(v.x, inv), gv.x), __fmul_rn(__fmul_rn(v.y, inv), gv.y),
                            __fmul_rn(__fmul_rn(v.z, inv), gv.z), __fmul_rn(__fmul_rn(v.w, inv), gv.w)};
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        half4_t h, l;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f16pair p = split_f16(o[j]);
            h[j] = p.hi;
            l[j] = p.lo;
        }
        *(half4_t *)(hi + (size_t)t * D + 4 * i) = h;
        *(half4_t *)(lo + (size_t)t * D + 4 * i) = l;
    }
}

/* grid (n_out/GR), GW*64 threads: out[t*n_out + row] = W[row] . x[t] for t < T, W row-tiled
   (n_out a multiple of 64). Lane = (row r = lane % GR, slice lane / GR); slice s of
   wavefront w holds blocks [(w * 64/GR + s) * BPW, +BPW) of the row in registers for the
   whole call, tokens are staged MT at a time, and the GW * 64/GR slices are summed in a
   fixed order (shuffles in the wavefront, then the GW wavefronts through LDS).
   BPW = ceil(n_in / 32 / (GW * 64/GR)). GR = 8 doubles the workgroups of a small matrix
   (Wo: 2048 rows, 256 workgroups instead of 128, one per CU).
   norm_g not null: x[t] is replaced by rmsnorm(x[t], norm_g, eps) as it is staged, with the
   bits of k_rmsnorm_rows (the same rms_inv_row and scaling). */
template <int ENC, int BPW, int GR>
__global__ __launch_bounds__(GW * 64)
__attribute__((amdgpu_waves_per_eu(BPW <= 2 ? 4 : 1)))   /* BPW <= 2: two workgroups per CU */
void k_gemv(const uint8_t *__restrict__ W,
                                                  size_t payload_plane, int n_in, int n_out,
                                                  const float *__restrict__ x, int T,
                                                  const float *__restrict__ norm_g, float eps,
                                                  float *__restrict__ out) {
    extern __shared__ __align__(16) float smem[];   /* float4 accesses: 16-byte aligned */
    __shared__ double npart[4];
    __shared__ float ninv[MT];
    const int nb = n_in / 32;
    float *xs = smem;                            /* MT * n_in */
    float *bsum = xs + MT * n_in;                /* MT * nb */
    float *red = bsum + MT * nb;                 /* GW * MT * GR */
    /* T >= 1 (the host checks): the loop below then runs at least once, so the loads ahead of
       the weights are not sunk into it past the weight loads */
    if (T <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % GR, sl = w * (64 / GR) + lane / GR, b0 = sl * BPW;
    /* the four workgroups of a 64-row tile on one XCD (they share its scale lines) */
    const int row = xcd_tile(blockIdx.x, gridDim.x) * GR + r, nbw = max(0, min(BPW, nb - b0));
    /* one token, n_in <= 4 * GW * 64 with the norm, 8 * GW * 64 without (the decode
       projections): x loaded once, ahead of the weights (thread t: float4 t, and without the
       norm float4 t + GW * 64, staged from the registers; with the norm, t < 256 also float4
       t + 256 for the sum of squares, and the gain), instead of passes over x after them,
       each waiting for every weight load issued before it */
    const int q4 = n_in / 4;
    const bool one = T == 1 && (norm_g ? q4 <= GW * 64 && q4 <= 2 * 256 : q4 <= 2 * GW * 64);
    /* unconditional loads at clamped indices (a load under a branch is waited for where the
       branch joins); used only when `one` */
    const float4 *x4 = (const float4 *)x, *g4 = (const float4 *)(norm_g ? norm_g : x);
    const int off1 = norm_g ? 256 : GW * 64;
    float4 xr0 = x4[min(tid, q4 - 1)], xr1 = x4[min(tid + off1, q4 - 1)], gr = g4[min(tid, q4 - 1)];
    WBlk<ENC> wv[BPW];
    uint16_t sv[BPW];               /* fp16 scales, converted where used: every load issues first */
    load_row_blocks_raw<ENC, BPW>(W, payload_plane, row, b0, nb - 1, nb, wv, sv);
    /* nothing computed from x may be scheduled above the weight loads (it would wait for x
       there, before they issue); a scheduling fence, not a barrier (__syncthreads() would
       wait for every weight load) */
    __builtin_amdgcn_sched_barrier(0);
    for (int t0 = 0; t0 < T; t0 += MT) {
        const int mc = min(MT, T - t0);
#pragma unroll
        for (int j = 0; j < BPW; j++) wv[j].pin();
        if (one) {
            float4 v = xr0;
            if (norm_g) {
                double ss = 0.0;
                if (tid < 256 && tid < q4) {     /* rms_inv_row's terms: float4 tid, tid + 256 */
                    ss = rms_sq4(ss, xr0);
                    if (tid + 256 < q4) ss = rms_sq4(ss, xr1);
                }
                const float inv = rms_inv_from(ss, n_in, eps, npart);
                v = make_float4(__fmul_rn(__fmul_rn(xr0.x, inv), gr.x),
                                __fmul_rn(__fmul_rn(xr0.y, inv), gr.y),
                                __fmul_rn(__fmul_rn(xr0.z, inv), gr.z),
                                __fmul_rn(__fmul_rn(xr0.w, inv), gr.w));
            }
            if (tid < ((q4 + 63) & ~63)) stage_put<ENC>(xs, bsum, n_in, nb, 0, tid, v, tid < q4);
            const int k1 = tid + GW * 64;        /* the same in every lane of a wavefront */
            if (!norm_g && k1 < ((q4 + 63) & ~63)) stage_put<ENC>(xs, bsum, n_in, nb, 0, k1, xr1, k1 < q4);
            lds_barrier();                       /* the dot products wait for their own loads */
        } else if (norm_g) {
            for (int i = 0; i < mc; i++) {
                const float inv = rms_inv_row(x + (size_t)(t0 + i) * n_in, n_in, eps, npart);
                if (tid == 0) ninv[i] = inv;
            }
            __syncthreads();
            stage_tokens<ENC, GW * 64>(xs, bsum, n_in, mc, [&](int i, int k4) {
                const float4 v = *(const float4 *)(x + (size_t)(t0 + i) * n_in + 4 * k4);
                const float4 g = *(const float4 *)(norm_g + 4 * k4);
                const float inv = ninv[i];
                return make_float4(__fmul_rn(__fmul_rn(v.x, inv), g.x),
                                   __fmul_rn(__fmul_rn(v.y, inv), g.y),
                                   __fmul_rn(__fmul_rn(v.z, inv), g.z),
                                   __fmul_rn(__fmul_rn(v.w, inv), g.w));
            });
        } else {
            stage_tokens<ENC, GW * 64>(xs, bsum, n_in, mc, [&](int i, int k4) {
                return *(const float4 *)(x + (size_t)(t0 + i) * n_in + 4 * k4);
            });
        }
        float acc[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i] = 0.0f;
        float dv[BPW];
#pragma unroll
        for (int j = 0; j < BPW; j++) dv[j] = f16_to_f32_hw(sv[j]);
        row_dots<ENC, BPW>(wv, dv, b0, nbw, xs, bsum, n_in, nb, mc, acc);
#pragma unroll
        for (int i = 0; i < MT; i++) {
#pragma unroll
            for (int o = GR; o < 64; o <<= 1) acc[i] += __shfl_xor(acc[i], o);
            if (lane < GR) red[(w * MT + i) * GR + r] = acc[i];
        }
        __syncthreads();
        if (w == 0 && lane < GR)
            for (int i = 0; i < mc; i++) {
                float s = 0.0f;
                for (int ww = 0; ww < GW; ww++) s += red[(ww * MT + i) * GR + r];
                out[(size_t)(t0 + i) * n_out + row] = s;
            }
        __syncthreads();
    }
}

/* One head row of HD floats in LDS normalised in place (qwen3_moe.c:44-49, kernels.c:408-413):
   the sum of squares accumulated in double across the wavefront (each lane its elements in
   order, then a fixed reduction tree), then the reference's float formula for 1/sqrt and the
   scaling. Whole wavefront. */
__device__ static inline void head_rmsnorm_lds(float *v, const float *__restrict__ g, int HD,
                                               float eps) {
    const int lane = threadIdx.x & 63;
    double ss = 0.0;
    for (int i = lane; i < HD; i += 64) ss += (double)__fmul_rn(v[i], v[i]);
    ss = wave_sum_d(ss);
    const float inv = __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn((float)ss, (float)HD), eps)));
    for (int i = lane; i < HD; i += 64) v[i] = __fmul_rn(__fmul_rn(v[i], inv), g[i]);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

/* grid (T, H + 2*KV), 64 threads. Head hh of token t in qkv (T, (H + 2 KV) * HD): q heads are
   RMS-normed with qn and rotated into q (T, H*HD); k heads normed with kn, rotated, and written
   to the cache row pos0 + t; v heads copied to the value cache. rope: [pos][HD/2] (cos, sin)
   pairs (kernels.c:430-433, computed on the host). HD <= 256, even. */
__global__ __launch_bounds__(64) void k_qk_norm_rope(const float *__restrict__ qkv, int ks,
                                                     size_t pstride,
                                                     const float *__restrict__ qn,
                                                     const float *__restrict__ kn,
                                                     const float2 *__restrict__ rope, int H,
                                                     int KV, int HD, float eps, int pos0_arg,
                                                     const int *__restrict__ pos_dev, int lim,
                                                     float *__restrict__ q, float *__restrict__ kc,
                                                     float *__restrict__ vc, int *stat) {
    __shared__ float v[256];
    const int t = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x, half = HD / 2;
    const int pos0 = pos_dev ? *pos_dev : pos0_arg;
    if (pos0 < 0 || pos0 + t >= lim) {           /* lim = min(cache rows, RoPE rows) */
        /* a position outside the cache (possible only when it is read on the device): the
           query row becomes NaN, nothing enters the cache, and the status word records it */
        if (hh < H)
            for (int i = lane; i < HD; i += 64) q[((size_t)t * H + hh) * HD + i] = __int_as_float(0x7fc00000);
        if (lane == 0) stat[0] = 1;
        return;
    }
    const float *src = qkv + (size_t)t * (H + 2 * KV) * HD + (size_t)hh * HD;
    const size_t crow = (size_t)(pos0 + t) * KV * HD;
    /* the projection's ks k-parts (pstride floats apart) added in part order, as k_sum_parts */
    auto val = [&](int i) {
        float a = src[i];
        for (int z = 1; z < ks; z++) a = __fadd_rn(a, src[(size_t)z * pstride + i]);
        return a;
    };
    if (hh >= H + KV) {                          /* value head: to the cache unchanged */
        for (int i = lane; i < HD; i += 64) vc[crow + (size_t)(hh - H - KV) * HD + i] = val(i);
        return;
    }
    for (int i = lane; i < HD; i += 64) v[i] = val(i);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    head_rmsnorm_lds(v, hh < H ? qn : kn, HD, eps);
    float *dst = hh < H ? q + (size_t)t * H * HD + (size_t)hh * HD
                        : kc + crow + (size_t)(hh - H) * HD;
    const float2 *cs = rope + (size_t)(pos0 + t) * half;
    for (int i = lane; i < half; i += 64) {
        const float a = v[i], b = v[i + half], c = cs[i].x, s = cs[i].y;
        dst[i] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
        dst[i + half] = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
    }
}

/* Scores, softmax and weighted sum of one (head, token) over positions 0..n-1
   (qwen3_moe.c:144-160): s_j = (q . k_j) / sqrtf(HD); p = softmax(s) (kernels.c:20-26, the
   glibc-identical expf); out = sum_j p_j v_j. 256 threads. Rows j < n_cache come from the
   cache (kc/vc at kv head kh, row stride kvw floats), row n_cache (when n > n_cache) from
   knew/vnew. Eight lanes per key row for the scores; block reductions for the maximum and
   the sum; the weighted sum with a float4 of the head dimension per thread and
   G = 256 / (HD/4) groups over interleaved positions, AVD rows in flight per thread (8 here:
   many workgroups of this kind run at once, so registers count more than depth; the rows
   are added in the same order for any AVD), the groups added in order and the total divided
   by the sum once. sc: LDS for n scores; qs, knew, vnew: LDS; red: 4 floats; part: 1024. */
template <int NT, int AVD>
__device__ __forceinline__ static void attn_load_v(const float *__restrict__ vc, int kvw, int kh,
                                                   int HD, int n_cache, float4 (&v0)[AVD],
                                                   float4 (&v1)[AVD]);
template <int NT, int AVD>
__device__ __forceinline__ static void attn_softmax_av(const float *__restrict__ vc, int kvw,
                                                       int kh, int HD, int n, int n_cache,
                                                       const float *vnew, float4 (&v0)[AVD],
                                                       float4 (&v1)[AVD], float *sc, float mx,
                                                       float *red, float *part,
                                                       const uint64_t *etab,
                                                       float *__restrict__ out);

__device__ static void attn_one(const float *qs, const float *__restrict__ kc,
                                const float *__restrict__ vc, int kvw, int kh, int HD, int n,
                                int n_cache, const float *knew, const float *vnew, float *sc,
                                float *red, float *part, float *__restrict__ out) {
    const int tid = threadIdx.x, hd4 = HD / 4;
    const float rs = cpg_sqrt_rn((float)HD);
    /* eight lanes per key row (lane r = tid & 7 holds float4s r, r + 8, r + 16 and r + 24 of
       the row, so that a wavefront reads eight whole rows per load), each lane's 16 products
       in order, then the row's eight lanes added by a butterfly: the arithmetic of
       k_attn_decode's scores. Loads are unconditional at clamped rows and columns; columns
       past HD multiply a zero q. */
    const int sub = tid >> 3, r = tid & 7;
    int col[4];
    float4 qr[4], knr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        col[i] = min(r + 8 * i, hd4 - 1);
        qr[i] = r + 8 * i < hd4 ? ((const float4 *)qs)[col[i]] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        knr[i] = knew ? ((const float4 *)knew)[col[i]] : qr[i];
    }
    const float4 *k4 = (const float4 *)(kc + (size_t)kh * HD);
    const int kvw4 = kvw / 4, lastc = max(n_cache - 1, 0);
    float4 v0[8], v1[8];
    attn_load_v<256, 8>(vc, kvw, kh, HD, n_cache, v0, v1);
    float mx = -INFINITY;
    for (int j0 = 0; j0 < n; j0 += 4 * 32) {
        float4 kp[4][4];
#pragma unroll
        for (int p = 0; p < 4; p++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                kp[p][i] = k4[(size_t)min(j0 + 32 * p + sub, lastc) * kvw4 + col[i]];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int j = j0 + 32 * p + sub;
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k = j >= n_cache ? knr[i] : kp[p][i];
                a = fmaf(qr[i].x, k.x, a);
                a = fmaf(qr[i].y, k.y, a);
                a = fmaf(qr[i].z, k.z, a);
                a = fmaf(qr[i].w, k.w, a);
            }
            a += __shfl_xor(a, 1);
            a += __shfl_xor(a, 2);
            a += __shfl_xor(a, 4);
            const float sj = __fdiv_rn(a, rs);
            if (j < n) {
                if (r == 0) sc[j] = sj;
                mx = sj > mx ? sj : mx;
            }
        }
    }
    attn_softmax_av<256, 8>(vc, kvw, kh, HD, n, n_cache, vnew, v0, v1, sc, mx, red, part,
                            cpg_exp2f_tab, out);
}

/* the sum of v[0..NW) as a balanced tree in a fixed order */
template <int NW> __device__ static inline float tree_sum(const float *v) {
    if constexpr (NW == 1) return v[0];
    else return tree_sum<NW / 2>(v) + tree_sum<NW / 2>(v + NW / 2);
}

/* The first two batches of AVD value rows of thread tid (NT threads), rows
   g, g + G, ... with g = tid / (HD/4), G = NT / (HD/4), float4 tid % (HD/4) of each: every
   load unconditional at a clamped row (loads under a branch would each wait for all earlier
   ones); rows past the cache (the new one) and past n are replaced by selects where they are
   used (attn_softmax_av). */
template <int NT, int AVD>
__device__ __forceinline__ static void attn_load_v(const float *__restrict__ vc, int kvw, int kh,
                                                   int HD, int n_cache, float4 (&v0)[AVD],
                                                   float4 (&v1)[AVD]) {
    const int tid = threadIdx.x, hd4 = HD / 4;
    const int G = NT / hd4, c4 = tid % hd4, gc = min(tid / hd4, G - 1);
    const int last = max(n_cache - 1, 0), step = AVD * G;
    const float *vh = vc + (size_t)kh * HD;
#pragma unroll
    for (int u = 0; u < AVD; u++)
        v0[u] = ((const float4 *)(vh + (size_t)min(gc + u * G, last) * kvw))[c4];
#pragma unroll
    for (int u = 0; u < AVD; u++)
        v1[u] = ((const float4 *)(vh + (size_t)min(gc + step + u * G, last) * kvw))[c4];
}

/* The second half of attn_one: given the scores sc[0..n) and each thread's running maximum,
   the softmax and the weighted sum over the value rows (NT threads). v0, v1: the first two
   batches of value rows (attn_load_v), loaded by the caller ahead of the scores so that they
   arrive with the key rows. */
template <int NT, int AVD>
__device__ __forceinline__ static void attn_softmax_av(const float *__restrict__ vc, int kvw,
                                                       int kh, int HD, int n, int n_cache,
                                                       const float *vnew, float4 (&v0)[AVD],
                                                       float4 (&v1)[AVD], float *sc, float mx,
                                                       float *red, float *part,
                                                       const uint64_t *etab,
                                                       float *__restrict__ out) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hd4 = HD / 4;
    const int G = NT / hd4, c4 = tid % hd4, g = tid / hd4, gc = min(g, G - 1);
    const int last = max(n_cache - 1, 0), step = AVD * G;
    const float *vh = vc + (size_t)kh * HD;
    for (int o = 32; o >= 1; o >>= 1) {
        const float other = __shfl_xor(mx, o);
        mx = other > mx ? other : mx;
    }
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int i = 1; i < NW; i++) mx = fmaxf(mx, red[i]);
    float sum = 0.0f;
    for (int j = tid; j < n; j += NT) {
        const float e = cpg_expf_tab(__fsub_rn(sc[j], mx), etab);
        sc[j] = e;
        sum += e;
    }
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    __syncthreads();                             /* every thread has read red[] */
    if (lane == 0) red[w] = sum;
    __syncthreads();
    sum = tree_sum<NW>(red);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 vn = n > n_cache ? ((const float4 *)vnew)[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    /* rows j0, j0 + G, ... of register set VB, in order */
#define CPG_AV_BATCH(VB, J0)                                                                    \
    do {                                                                                        \
        float pj[AVD];                                                                     \
        _Pragma("unroll") for (int u = 0; u < AVD; u++) {                                  \
            const int j = (J0) + u * G;                                                         \
            pj[u] = j < n ? sc[min(j, n - 1)] : 0.0f;                                           \
        }                                                                                       \
        _Pragma("unroll") for (int u = 0; u < AVD; u++) {                                  \
            const float4 x = (J0) + u * G >= n_cache ? vn : VB[u];                              \
            acc.x = fmaf(pj[u], x.x, acc.x);                                                    \
            acc.y = fmaf(pj[u], x.y, acc.y);                                                    \
            acc.z = fmaf(pj[u], x.z, acc.z);                                                    \
            acc.w = fmaf(pj[u], x.w, acc.w);                                                    \
        }                                                                                       \
    } while (0)
    CPG_AV_BATCH(v0, gc);                        /* rows past n count with weight 0 */
    CPG_AV_BATCH(v1, gc + step);
    for (int j0 = gc + 2 * step; j0 < n; j0 += step) {       /* n > 2 step: further batches */
#pragma unroll
        for (int u = 0; u < AVD; u++)
            v0[u] = ((const float4 *)(vh + (size_t)min(j0 + u * G, last) * kvw))[c4];
        CPG_AV_BATCH(v0, j0);
    }
#undef CPG_AV_BATCH
    if (g < G) *(float4 *)(part + g * HD + 4 * c4) = acc;
    __syncthreads();
    if (tid < HD) {
        float o = part[tid];
        for (int gg = 1; gg < G; gg++) o += part[gg * HD + tid];
        out[tid] = __fdiv_rn(o, sum);
    }
}

__device__ static inline int head_on_xcd(int b, int H, int KV);

/* grid (H, T), 256 threads, HD <= 128, HD % 4 == 0: head h of token i (position pos0 + i)
   against cache rows 0..pos0+i of kv head h / (H/KV), all rows already in the cache
   (k_qk_norm_rope wrote the new ones). lim bounds the positions (the LDS holds lim scores).
   Head h = head_on_xcd(blockIdx.x): with H a multiple of 8 every row of the grid starts on
   XCD 0, so the heads of one kv head land on as few XCDs as they do in k_attn_decode. */
__global__ __launch_bounds__(256) void k_attn_core(const float *__restrict__ q,
                                                   const float *__restrict__ kc,
                                                   const float *__restrict__ vc, int H, int KV,
                                                   int HD, int pos0_arg,
                                                   const int *__restrict__ pos_dev, int lim,
                                                   float *__restrict__ ao) {
    extern __shared__ __align__(16) float sc[];
    __shared__ __align__(16) float qs[128];
    __shared__ float red[4];
    __shared__ __align__(16) float part[1024];
    const int h = head_on_xcd(blockIdx.x, H, KV), i = blockIdx.y, tid = threadIdx.x;
    const int pos0 = pos_dev ? *pos_dev : pos0_arg;
    const int n = pos0 + i + 1;
    if (pos0 < 0 || n > lim) return;
    if (tid < HD) qs[tid] = q[((size_t)i * H + h) * HD + tid];
    __syncthreads();
    attn_one(qs, kc, vc, KV * HD, h / (H / KV), HD, n, n, nullptr, nullptr, sc, red, part,
             ao + ((size_t)i * H + h) * HD);
}

/* The query head of workgroup b (of H): workgroup b runs on XCD b % 8, and the heads that
   share a kv head (and so read the same cache rows) are placed on as few XCDs as possible,
   H / KV / (H / 8) heads of one kv head per XCD, so that their cache reads hit one L2. The
   identity unless 8 divides H and H / 8 divides H / KV. */
__device__ static inline int head_on_xcd(int b, int H, int KV) {
    const int per_xcd = H / NXCD, group = H / KV;
    if (H % NXCD || group % per_xcd) return b;
    const int x = b % NXCD, i = b / NXCD;      /* XCD x, its i-th workgroup */
    return x * per_xcd + i;                    /* XCD x takes heads x*per_xcd .. +per_xcd-1 */
}

/* Many tokens on MFMA: grid (KV, ceil(T / (64/G))), 256 threads, HD == 128, G = H/KV
   dividing 16. Workgroup (kh, b) takes 64 query rows, wavefront w rows 16w..16w+15, row r =
   (token b*TB + r / G, head kh*G + r % G) with TB = 64/G tokens; all of them share each tile
   of AMT key positions of kv head kh staged in LDS as hi/lo f16 halves (x = hi + lo, hi =
   f16(x), lo = f16(x - hi): 22 significant bits). Per tile:
     S^T = K . Q^T on v_mfma_f32_16x16x32_f16 (A = key rows, B = the wavefront's query rows,
       held in registers for the whole call), each product as hi.hi + lo.hi + hi.lo (the lo.lo
       term, below 2^-22 of the sum, is not formed); lane l then holds the scores of query
       l%16 against keys 16kt + 4(l/16) + i (kt, i < 4), divided by sqrt(HD) and masked
       (key j > the query's position, or past the cache: -inf);
     online softmax per query (the 4 lanes of a query reduce by shuffles): running maximum m,
       sum l of expf(s - m) with the reference's expf, the accumulators rescaled by
       expf(m_old - m_new) when the maximum grows;
     O += P . V, A = the lane's own probabilities (hi/lo, in the lane order above: slot 8g + j
       of a 32-key step u is key 32u + 4g + j for j < 4 and 32u + 16 + 4g + j - 4 after), B =
       value rows read in that key order from LDS, where a value tile is laid out as
       [key / 4][dim][key % 4] so that a lane's four consecutive keys of one dimension are one
       8-byte read.
   out = O / l, written as ao (fp32) or, aoh not null, as the hi/lo planes of the output
   projection. The sums run in another order than the reference's two-pass softmax
   (qwen3_moe.c:127-157) and the products carry 22-bit operands, so the output agrees to
   rounding. Dynamic LDS: amma_lds_bytes(). */
#define AMT 64              /* k_attn_mma: key positions per tile */
#define AMQ 64              /* k_attn_mma: query rows per workgroup (4 wavefronts of 16) */
#define AMLK (128 + 8)      /* k_attn_mma: K row stride in halves (16 B of padding) */
#define AMMA_MIN_T 2        /* k_attn_mma from this many tokens on (HD 128, G | 16) */

#define AMMA_BUF (2 * AMT * AMLK + 2 * AMT * 128)   /* halves of one K/V tile buffer */

static inline size_t amma_lds_bytes() { return sizeof(_Float16) * 2 * (size_t)AMMA_BUF; }

/* k_attn_mma's staging of one key tile, in two halves so that the next tile's loads fly
   while the current one is computed: thread tid takes items tid and tid + 256, item = (key
   group kg of 4 keys, float4 column c4) of kv head kh, keys from j0 (clamped to n - 1) */
__device__ __forceinline__ static void amma_load(float4 (&kv)[2][4], float4 (&vv)[2][4],
                                                 const float *__restrict__ kc,
                                                 const float *__restrict__ vc, int kvw, int kh,
                                                 int j0, int n) {
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int item = threadIdx.x + 256 * it, kg = item >> 5, c4 = item & 31;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int jj = min(j0 + 4 * kg + e, n - 1);
            const size_t off = (size_t)jj * kvw + (size_t)kh * 128 + 4 * c4;
            kv[it][e] = *(const float4 *)(kc + off);
            vv[it][e] = *(const float4 *)(vc + off);
        }
    }
}

/* the loaded items as hi/lo halves into buffer buf: K rows [key][AMLK], V as
   [key / 4][dim][key % 4] */
__device__ __forceinline__ static void amma_store(const float4 (&kv)[2][4],
                                                  const float4 (&vv)[2][4], _Float16 *buf) {
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    _Float16 *kh_s = buf, *kl_s = kh_s + AMT * AMLK;
    _Float16 *vh_s = kl_s + AMT * AMLK, *vl_s = vh_s + AMT * 128;
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int item = threadIdx.x + 256 * it, kg = item >> 5, c4 = item & 31;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x[4] = {kv[it][e].x, kv[it][e].y, kv[it][e].z, kv[it][e].w};
            half4_t h, lo;
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const f16pair p = split_f16(x[d]);
                h[d] = p.hi;
                lo[d] = p.lo;
            }
            *(half4_t *)(kh_s + (4 * kg + e) * AMLK + 4 * c4) = h;
            *(half4_t *)(kl_s + (4 * kg + e) * AMLK + 4 * c4) = lo;
        }
#pragma unroll
        for (int d = 0; d < 4; d++) {
            half4_t h, lo;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float4 v = vv[it][e];
                const f16pair p = split_f16(d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w);
                h[e] = p.hi;
                lo[e] = p.lo;
            }
            *(half4_t *)(vh_s + ((size_t)kg * 128 + 4 * c4 + d) * 4) = h;
            *(half4_t *)(vl_s + ((size_t)kg * 128 + 4 * c4 + d) * 4) = lo;
        }
    }
}

__global__ __launch_bounds__(256) void k_attn_mma(const float *__restrict__ q,
                                                  const float *__restrict__ kc,
                                                  const float *__restrict__ vc, int H, int KV,
                                                  int T, int pos0_arg,
                                                  const int *__restrict__ pos_dev, int lim,
                                                  float *__restrict__ ao,
                                                  _Float16 *__restrict__ aoh,
                                                  _Float16 *__restrict__ aol) {
    constexpr int HD = 128;
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) _Float16 smh[];   /* two tile buffers (amma_store) */
    __shared__ uint64_t tab[32];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4, c = l & 15;
    const int G = H / KV, TB = AMQ / G, kh = blockIdx.x, t0 = blockIdx.y * TB;
    const int kvw = KV * HD;
    const int pos0 = pos_dev ? *pos_dev : pos0_arg;
    if (pos0 < 0 || pos0 + t0 >= lim) return;
    const int tl = min(T, t0 + TB) - 1;          /* the last token of the block */
    const int n = min(pos0 + tl + 1, lim);       /* keys 0 .. n-1 */
    if (tid < 32) tab[tid] = cpg_exp2f_tab[tid];
    /* this lane's query (scores, softmax state): row 16w + c; rows past the block's last
       token compute with its query and are not stored */
    const int rq = 16 * w + c, tq = min(t0 + rq / G, tl), hq = kh * G + rq % G;
    const int pq = pos0 + tq;                    /* its last key */
    half8_t qh[4], ql[4];                        /* B operand: dims 32s + 8g .. + 7 */
    {
        const float *qr = q + ((size_t)tq * H + hq) * HD + 8 * g;
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const float4 a = *(const float4 *)(qr + 32 * s4), b = *(const float4 *)(qr + 32 * s4 + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const f16pair p = split_f16(v[j]);
                qh[s4][j] = p.hi;
                ql[s4][j] = p.lo;
            }
        }
    }
    const float rs = cpg_sqrt_rn((float)HD);
    float m = -INFINITY, lsum = 0.0f;
    f32x4_t o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) o[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float4 kv[2][4], vv[2][4];
    amma_load(kv, vv, kc, vc, kvw, kh, 0, n);
    amma_store(kv, vv, smh);
    __syncthreads();
    for (int j0 = 0; j0 < n; j0 += AMT) {
        /* the next tile's loads fly while this one is computed */
        const bool more = j0 + AMT < n;
        if (more) amma_load(kv, vv, kc, vc, kvw, kh, j0 + AMT, n);
        const _Float16 *buf = smh + ((j0 / AMT) & 1) * AMMA_BUF;
        const _Float16 *kh_s = buf, *kl_s = kh_s + AMT * AMLK;
        const _Float16 *vh_s = kl_s + AMT * AMLK, *vl_s = vh_s + AMT * HD;
        /* scores: st[kt][i] = S[query c][key j0 + 16kt + 4g + i] */
        float st[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f32x4_t a = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const _Float16 *kr = kh_s + (16 * kt + c) * AMLK + 8 * g;
            const _Float16 *kl = kl_s + (16 * kt + c) * AMLK + 8 * g;
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                const half8_t ah = *(const half8_t *)(kr + 32 * s4);
                const half8_t al = *(const half8_t *)(kl + 32 * s4);
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qh[s4], a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, qh[s4], a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ql[s4], a, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {   /* computed unconditionally, then masked: no branch */
                const int j = j0 + 16 * kt + 4 * g + i;
                const float sv = __fdiv_rn(a[i], rs);
                st[kt][i] = j <= pq && j < n ? sv : -INFINITY;
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) mt = fmaxf(mt, st[kt][i]);
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                /* a masked score is -inf, whose expf is 0 (mn is finite: key 0 is every
                   query's and comes first) */
                const float e = cpg_expf_tab(__fsub_rn(st[kt][i], mn), tab);
                st[kt][i] = e;
                psum += e;
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        const float f = m == -INFINITY ? 0.0f : cpg_expf_tab(__fsub_rn(m, mn), tab);
        lsum = fmaf(lsum, f, psum);
        m = mn;
        /* the accumulators hold queries 4g + i: their factors from lanes 4g + i */
        float fi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fi[i] = __shfl(f, 4 * g + i);
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[dt][i] *= fi[i];
        /* O += P . V over the tile, two steps of 32 keys */
#pragma unroll
        for (int u = 0; u < 2; u++) {
            half8_t ph, pl;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float pv = j < 4 ? st[2 * u][j] : st[2 * u + 1][j - 4];
                const f16pair p = split_f16(pv);
                ph[j] = p.hi;
                pl[j] = p.lo;
            }
            const int kg0 = 8 * u + g, kg1 = 8 * u + 4 + g;
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) {
                const int d = 16 * dt + c;
                const half4_t h0 = *(const half4_t *)(vh_s + ((size_t)kg0 * HD + d) * 4);
                const half4_t h1 = *(const half4_t *)(vh_s + ((size_t)kg1 * HD + d) * 4);
                const half4_t l0 = *(const half4_t *)(vl_s + ((size_t)kg0 * HD + d) * 4);
                const half4_t l1 = *(const half4_t *)(vl_s + ((size_t)kg1 * HD + d) * 4);
                const half8_t bh = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                const half8_t bl = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, bh, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, bh, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, bl, o[dt], 0, 0, 0);
            }
        }
        /* the other buffer was last read before the previous barrier */
        if (more) amma_store(kv, vv, smh + ((j0 / AMT + 1) & 1) * AMMA_BUF);
        __syncthreads();
    }
    /* out: o[dt][i] is query row 16w + 4g + i, dimension 16dt + c */
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float li = __shfl(lsum, 4 * g + i);
        const int r = 16 * w + 4 * g + i, t = t0 + r / G, h = kh * G + r % G;
        if (t > tl) continue;
        const size_t e0 = ((size_t)t * H + h) * HD + c;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) {
            const float v = __fdiv_rn(o[dt][i], li);
            if (aoh) {
                const f16pair p = split_f16(v);
                aoh[e0 + 16 * dt] = p.hi;
                aol[e0 + 16 * dt] = p.lo;
            } else {
                ao[e0 + 16 * dt] = v;
            }
        }
    }
}

/* Many tokens: grid (KV, ceil(T / (R/G))), 256 threads, G = H/KV query heads per kv head
   dividing R, HD <= 128, HD % 4 == 0. Workgroup (kh, b) takes the R query rows of tokens
   b*TB .. b*TB+TB-1 (TB = R/G) and the G heads of kv head kh, row r = (token r / G, head
   kh*G + r % G), and reads each cache row of kv head kh once for all of them (k_attn_core
   reads it once per head and token). The keys run in tiles of AKT positions staged in LDS
   (row stride HD + 4 floats, so the 16 key rows a wavefront reads as float4 fall in
   distinct banks), with the softmax online: per row the running maximum m, the sum l of
   expf(s - m) and the weighted sum of value rows, rescaled by expf(m_old - m_new) when the
   maximum grows; out = acc / l. A score is q . k in 4-element steps (fmaf, in order) divided
   by sqrt(HD); expf is the reference's (cpg_expf_tab). The sums run in another order than
   the reference's two-pass softmax (qwen3_moe.c:127-157), so the output agrees to rounding.
   Thread roles: scores, row (tid / 16) * (R/16) + i for i < R/16 against keys tid % 16 + 16 j
   (j < 4); values, row tid / (256/R) and HD*R/256 consecutive dimensions. */
#define AKT 64              /* k_attn_blk: key positions per tile */

template <int R>
__global__ __launch_bounds__(256) void k_attn_blk(const float *__restrict__ q,
                                                  const float *__restrict__ kc,
                                                  const float *__restrict__ vc, int H, int KV,
                                                  int HD, int T, int pos0_arg,
                                                  const int *__restrict__ pos_dev, int lim,
                                                  float *__restrict__ ao,
                                                  _Float16 *__restrict__ aoh,
                                                  _Float16 *__restrict__ aol) {
    constexpr int RS = R / 16, DPT = 128 * R / 256 / 4;   /* float4 of values per thread (HD 128) */
    extern __shared__ __align__(16) float sm[];
    const int LQ = HD + 4;
    float *qs = sm;                              /* R x LQ */
    float *ks = qs + R * LQ;                     /* AKT x LQ */
    float *vs = ks + AKT * LQ;                   /* AKT x HD */
    float *ps = vs + AKT * HD;                   /* R x AKT */
    __shared__ float m_s[R], l_s[R], sc_s[R];
    __shared__ uint64_t tab[32];
    const int tid = threadIdx.x, G = H / KV, TB = R / G, kh = blockIdx.x;
    const int t0 = blockIdx.y * TB, hd4 = HD / 4, kvw = KV * HD;
    const int pos0 = pos_dev ? *pos_dev : pos0_arg;
    if (pos0 < 0 || pos0 + t0 >= lim) return;
    const int tl = min(T, t0 + TB) - 1;          /* the last token of the block */
    const int n = min(pos0 + tl + 1, lim);       /* keys 0 .. n-1 */
    if (tid < 32) tab[tid] = cpg_exp2f_tab[tid];
    if (tid < R) { m_s[tid] = -INFINITY; l_s[tid] = 0.0f; }
    for (int i = tid; i < R * hd4; i += 256) {   /* the R query rows (tokens past T: the last) */
        const int r = i / hd4, c = i % hd4, t = min(t0 + r / G, tl), h = kh * G + r % G;
        *(float4 *)(qs + r * LQ + 4 * c) = ((const float4 *)(q + ((size_t)t * H + h) * HD))[c];
    }
    const float rs = cpg_sqrt_rn((float)HD);
    const int sr0 = (tid >> 4) * RS, sk = tid & 15;              /* score roles */
    const int vr = tid / (256 / R), vd = (tid % (256 / R)) * DPT; /* value roles (float4) */
    float4 acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; i++) acc[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j0 = 0; j0 < n; j0 += AKT) {
        __syncthreads();                         /* the previous tile's reads are done */
        for (int i = tid; i < AKT * hd4; i += 256) {
            const int j = i / hd4, c = i % hd4, jj = min(j0 + j, n - 1);
            const size_t off = (size_t)jj * kvw + (size_t)kh * HD + 4 * c;
            *(float4 *)(ks + j * LQ + 4 * c) = *(const float4 *)(kc + off);
            *(float4 *)(vs + j * HD + 4 * c) = *(const float4 *)(vc + off);
        }
        __syncthreads();
        /* scores of rows sr0 .. sr0+RS-1 against keys sk + 16 jj */
        float a[RS][4];
#pragma unroll
        for (int i = 0; i < RS; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) a[i][jj] = 0.0f;
        for (int c = 0; c < hd4; c++) {
            float4 qv[RS], kv[4];
#pragma unroll
            for (int i = 0; i < RS; i++) qv[i] = *(const float4 *)(qs + (sr0 + i) * LQ + 4 * c);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) kv[jj] = *(const float4 *)(ks + (sk + 16 * jj) * LQ + 4 * c);
#pragma unroll
            for (int i = 0; i < RS; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    a[i][jj] = fmaf(qv[i].x, kv[jj].x, a[i][jj]);
                    a[i][jj] = fmaf(qv[i].y, kv[jj].y, a[i][jj]);
                    a[i][jj] = fmaf(qv[i].z, kv[jj].z, a[i][jj]);
                    a[i][jj] = fmaf(qv[i].w, kv[jj].w, a[i][jj]);
                }
        }
#pragma unroll
        for (int i = 0; i < RS; i++) {
            const int r = sr0 + i, pr = pos0 + t0 + r / G;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = j0 + sk + 16 * jj;
                ps[r * AKT + sk + 16 * jj] = j <= pr && j < n ? __fdiv_rn(a[i][jj], rs) : -INFINITY;
            }
        }
        __syncthreads();
        /* per row (the 256/R consecutive threads of row vr, entries part, part + 256/R, ...):
           the new maximum, the tile's exponentials in place, the running sum and the rescale
           factor */
        {
            constexpr int P = 256 / R;
            const int part = tid % P;
            float mt = -INFINITY;
            for (int j = part; j < AKT; j += P) mt = fmaxf(mt, ps[vr * AKT + j]);
#pragma unroll
            for (int o = 1; o < P; o <<= 1) mt = fmaxf(mt, __shfl_xor(mt, o));
            const float mo = m_s[vr], mn = fmaxf(mo, mt);
            float sum = 0.0f;
            for (int j = part; j < AKT; j += P) {
                const float sj = ps[vr * AKT + j];
                const float e = sj == -INFINITY ? 0.0f : cpg_expf_tab(__fsub_rn(sj, mn), tab);
                ps[vr * AKT + j] = e;
                sum += e;
            }
#pragma unroll
            for (int o = 1; o < P; o <<= 1) sum += __shfl_xor(sum, o);
            __syncthreads();                     /* every thread of the row has read m_s */
            if (part == 0) {
                const float f = mo == -INFINITY ? 0.0f : cpg_expf_tab(__fsub_rn(mo, mn), tab);
                sc_s[vr] = f;
                l_s[vr] = fmaf(l_s[vr], f, sum);
                m_s[vr] = mn;
            }
        }
        __syncthreads();
        /* values: row vr, float4 vd .. vd+DPT-1 */
        const float f = sc_s[vr];
#pragma unroll
        for (int i = 0; i < DPT; i++)
            acc[i] = make_float4(acc[i].x * f, acc[i].y * f, acc[i].z * f, acc[i].w * f);
        const int jmax = min(AKT, n - j0);
        for (int j = 0; j < jmax; j++) {
            const float pj = ps[vr * AKT + j];
#pragma unroll
            for (int i = 0; i < DPT; i++) {
                if (4 * (vd + i) < HD) {
                    const float4 v = *(const float4 *)(vs + j * HD + 4 * (vd + i));
                    acc[i].x = fmaf(pj, v.x, acc[i].x);
                    acc[i].y = fmaf(pj, v.y, acc[i].y);
                    acc[i].z = fmaf(pj, v.z, acc[i].z);
                    acc[i].w = fmaf(pj, v.w, acc[i].w);
                }
            }
        }
    }
    const int t = t0 + vr / G, h = kh * G + vr % G;
    if (t < T) {
        const float l = l_s[vr];
        float *o = ao + ((size_t)t * H + h) * HD;
#pragma unroll
        for (int i = 0; i < DPT; i++)
            if (4 * (vd + i) < HD) {
                const float r4[4] = {__fdiv_rn(acc[i].x, l), __fdiv_rn(acc[i].y, l),
                                     __fdiv_rn(acc[i].z, l), __fdiv_rn(acc[i].w, l)};
                if (aoh) {                       /* the output projection's hi/lo planes */
                    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
                    const size_t e = ((size_t)t * H + h) * HD + 4 * (vd + i);
                    half4_t hv, lv;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const f16pair p = split_f16(r4[j]);
                        hv[j] = p.hi;
                        lv[j] = p.lo;
                    }
                    *(half4_t *)(aoh + e) = hv;
                    *(half4_t *)(aol + e) = lv;
                } else {
                    *(float4 *)(o + 4 * (vd + i)) = make_float4(r4[0], r4[1], r4[2], r4[3]);
                }
            }
    }
}

/* One new token (T = 1) at position pos: k_qk_norm_rope and k_attn_core in one kernel.
   grid H, ADT threads. Workgroup h normalises and rotates q head h and the new key of its kv
   head kh (the reference's per-head RMSNorm and RoPE, the same arithmetic as k_qk_norm_rope),
   attends over cache rows 0..pos-1 plus the new row from LDS, and the first workgroup of each
   kv head writes the new key and value rows to the cache (row pos is read by no other
   workgroup of this launch). */
__global__ __launch_bounds__(ADT) void k_attn_decode(const float *__restrict__ qkv,
                                                     const float *__restrict__ qn,
                                                     const float *__restrict__ kn,
                                                     const float2 *__restrict__ rope, int H,
                                                     int KV, int HD, float eps, int pos_arg,
                                                     const int *__restrict__ pos_dev, int lim,
                                                     float *__restrict__ kc,
                                                     float *__restrict__ vc,
                                                     float *__restrict__ ao, int *stat) {
    extern __shared__ __align__(16) float sc[];
    __shared__ __align__(16) float raw[2][128], vq[128], rot[2][128], gnorm[2][128];
    __shared__ float2 csp[64];
    __shared__ float red[ADT / 64];
    __shared__ __align__(16) float part[ADT / 32 * 128];
    __shared__ uint64_t etab[32];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = HD / 2;
    const int h = head_on_xcd(blockIdx.x, H, KV);
    const int pos = pos_dev ? *pos_dev : pos_arg;
    if (pos < 0 || pos + 1 > lim) {
        /* outside the cache (a position read on the device): NaN out, the status recorded */
        if (tid < HD) ao[(size_t)h * HD + tid] = __int_as_float(0x7fc00000);
        if (tid == 0) stat[0] = 1;
        return;
    }
    const int kh = h / (H / KV), kvw = KV * HD, hd4 = HD / 4, n = pos + 1;
    /* this head's q, k and v first (completion is counted in order: loaded after the key
       row, they would wait for all of it) */
    const uint64_t et = cpg_exp2f_tab[tid & 31];  /* expf's table, copied to LDS with q, k, v */
    /* unconditional at a clamped index: a load under a branch is waited for where the
       branch joins, before anything after it could be issued */
    const int tc = min(tid, HD - 1);
    const float rq = qkv[(size_t)h * HD + tc];               /* one token: [q | k | v] heads */
    const float rk = qkv[(size_t)(H + kh) * HD + tc];
    const float rv = qkv[(size_t)(H + KV + kh) * HD + tc];
    /* the norm weights and this position's rotation pairs, also ahead of the key rows, and
       through LDS: loaded where waves 0 and 1 use them they would be waited for with the key
       rows */
    const float gqv = qn[tc], gkv = kn[tc];
    const float2 csv = rope[(size_t)pos * half + min(tid, half - 1)];
    /* scores: eight lanes per key row, lane r = tid & 7 holding float4s r, r + 8, r + 16 and
       r + 24 of the row, so that a wave reads eight whole rows per load; ADT / 8 rows per pass
       and SP passes in registers. The first SP passes (rows 0..SP*ADT/8-1) are in flight
       during the norms: unconditional loads at clamped rows and columns (a load under a branch
       makes the compiler wait for every load in flight where the branches join). */
    constexpr int RPP = ADT / 8, SP = 4;
    const int sub = tid >> 3, r = tid & 7;
    const float4 *k4 = (const float4 *)(kc + (size_t)kh * HD);
    const int kvw4 = kvw / 4, lastc = max(pos - 1, 0);
    int col[4];
#pragma unroll
    for (int i = 0; i < 4; i++) col[i] = min(r + 8 * i, hd4 - 1);
    float4 kp[SP][4];
#pragma unroll
    for (int p = 0; p < SP; p++)
#pragma unroll
        for (int i = 0; i < 4; i++) kp[p][i] = k4[(size_t)min(p * RPP + sub, lastc) * kvw4 + col[i]];
    /* and the first two batches of value rows behind them, in flight during the scores */
    float4 v0[AV_DEPTH], v1[AV_DEPTH];
    attn_load_v<ADT, AV_DEPTH>(vc, kvw, kh, HD, pos, v0, v1);
    raw[0][tc] = rq;             /* threads past HD store element HD - 1 again, the same value */
    raw[1][tc] = rk;
    vq[tc] = rv;
    gnorm[0][tc] = gqv;
    gnorm[1][tc] = gkv;
    csp[min(tid, half - 1)] = csv;
    etab[tid & 31] = et;         /* every thread: a store under a branch draws its load in */
    __syncthreads();
    if (w < 2) {                 /* wave 0: q, wave 1: the new key (head_rmsnorm_lds, then RoPE) */
        float *v = raw[w];
        const float g0 = gnorm[w][min(lane, HD - 1)], g1 = gnorm[w][min(lane + 64, HD - 1)];
        const float2 csl = csp[min(lane, half - 1)];
        double ss = 0.0;
        for (int i = lane; i < HD; i += 64) ss += (double)__fmul_rn(v[i], v[i]);
        ss = wave_sum_d(ss);
        const float inv = __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn((float)ss, (float)HD), eps)));
        if (lane < HD) v[lane] = __fmul_rn(__fmul_rn(v[lane], inv), g0);
        if (lane + 64 < HD) v[lane + 64] = __fmul_rn(__fmul_rn(v[lane + 64], inv), g1);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane < half) {
            const float a = v[lane], b = v[lane + half];
            rot[w][lane] = __fsub_rn(__fmul_rn(a, csl.x), __fmul_rn(b, csl.y));
            rot[w][lane + half] = __fadd_rn(__fmul_rn(b, csl.x), __fmul_rn(a, csl.y));
        }
    }
    __syncthreads();
    if (h % (H / KV) == 0 && tid < HD) {
        kc[(size_t)pos * kvw + (size_t)kh * HD + tid] = rot[1][tid];
        vc[(size_t)pos * kvw + (size_t)kh * HD + tid] = vq[tid];
    }
    /* the dot products: each lane's 16 products in order, then the eight lanes of a row added
       by a butterfly (every lane ends with the same bits); row pos, the new key, from LDS */
    const float rs = cpg_sqrt_rn((float)HD);
    float4 qr[4], knr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bool ok = r + 8 * i < hd4;
        qr[i] = ok ? ((const float4 *)rot[0])[col[i]] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        knr[i] = ((const float4 *)rot[1])[col[i]];
    }
    float mx = -INFINITY;
    for (int p0 = 0; p0 * RPP < n; p0 += SP) {
        if (p0 > 0) {
#pragma unroll
            for (int p = 0; p < SP; p++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    kp[p][i] = k4[(size_t)min((p0 + p) * RPP + sub, lastc) * kvw4 + col[i]];
        }
#pragma unroll
        for (int p = 0; p < SP; p++) {
            const int j = (p0 + p) * RPP + sub;
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k = j >= pos ? knr[i] : kp[p][i];
                a = fmaf(qr[i].x, k.x, a);
                a = fmaf(qr[i].y, k.y, a);
                a = fmaf(qr[i].z, k.z, a);
                a = fmaf(qr[i].w, k.w, a);
            }
            a += __shfl_xor(a, 1);
            a += __shfl_xor(a, 2);
            a += __shfl_xor(a, 4);
            const float sj = __fdiv_rn(a, rs);
            if (j < n) {
                if (r == 0) sc[j] = sj;
                mx = sj > mx ? sj : mx;
            }
        }
    }
    attn_softmax_av<ADT, AV_DEPTH>(vc, kvw, kh, HD, n, pos, vq, v0, v1, sc, mx, red, part, etab,
                         ao + (size_t)h * HD);
}

/* The maximum and the sum over each half of the wavefront (lanes 0-31, 32-63), the same
   bits in every lane of the half: DPP steps within rows of 16 lanes, then one exchange
   between the two rows of the half. */
__device__ static inline float half_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_1032, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_2301, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_HALF_MIRROR, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_MIRROR, 0xf, 0xf, false)));
    return fmaxf(v, __shfl_xor(v, 16));
}
__device__ static inline float half_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_1032, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_2301, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_HALF_MIRROR, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_MIRROR, 0xf, 0xf, false));
    return v + __shfl_xor(v, 16);
}

/* The reference's per-head RMSNorm and RoPE (qwen3_moe.c:137-143, kernels.c:408-413, 430-447)
   of one head of 128 floats in LDS, the bits of head_rmsnorm_lds followed by the rotation:
   lane l holds elements l and l + 64 (one rotation pair). g0, g1: the norm weights of those
   elements; cs: the pair's (cos, sin) at this position. Whole wavefront. */
__device__ static inline void norm_rope_128(float *v, float g0, float g1, float2 cs, float eps) {
    const int lane = threadIdx.x & 63;
    const float a0 = v[lane], b0 = v[lane + 64];
    double ss = (double)__fmul_rn(a0, a0);
    ss += (double)__fmul_rn(b0, b0);
    ss = wave_sum_d(ss);
    const float inv = __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn((float)ss, 128.0f), eps)));
    const float a = __fmul_rn(__fmul_rn(a0, inv), g0), b = __fmul_rn(__fmul_rn(b0, inv), g1);
    v[lane] = __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(b, cs.y));
    v[lane + 64] = __fadd_rn(__fmul_rn(b, cs.x), __fmul_rn(a, cs.y));
}

/* One new token (T = 1) at position pos, the AG = 8 query heads of one kv head over one split
   of AP = 32 positions per workgroup: grid (KV, smax), 256 threads, HD == AHD, H == AG * KV.
   Workgroup (kh, s) takes positions s*AP .. min(s*AP + AP, pos + 1) - 1; splits past pos + 1
   leave at once. Every load is issued first: the split's cached key and value rows (one
   float4 of each per thread and row group, clamped rows, coalesced), the 8 query heads, the
   new key and value, the norm weights and this position's rotation pairs. Then the query
   heads (and, in the split holding row pos, the new key) are normalised and rotated
   (norm_rope_128), the split holding row pos writes the new key and value to the cache, the
   rows are staged in LDS (row pos from the new key and value), thread (h, j) takes the score
   s_hj = (q_h . k_j) / sqrtf(HD) (four partial sums over the float4 columns mod 4), and for
   each head the split's maximum m, e_j = expf(s_hj - m), their sum l and acc = sum_j e_j v_j
   are left in pml / pacc (agent-scope stores) for head h, split s at (h * smax + s).
   The last of the ns = ceil((pos + 1) / AP) splits of kv head kh to count itself in at
   ctr[kh] (which it resets for the next launch) merges them, thread (h, c) float4 c of head h:
   M the largest m_s, w_s = expf(m_s - M) formed once per split, L = sum_s w_s l_s (a fixed
   shuffle tree per group of AMG splits, the groups in order), o = sum_s w_s acc_s in split
   order; ao = o / L. Up to AMG splits (positions <= AMG * AP) every load is issued at once.
   qwen3_moe.c:144-160 in fp32, in another order (within rounding of k_attn_decode). */
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ qkv,
                                                    const float *__restrict__ qn,
                                                    const float *__restrict__ kn,
                                                    const float2 *__restrict__ rope, int H,
                                                    int KV, float eps, int pos_arg,
                                                    const int *__restrict__ pos_dev, int lim,
                                                    float *__restrict__ kc, float *__restrict__ vc,
                                                    float *pacc, float2 *pml, int smax, int *ctr,
                                                    float *__restrict__ ao, int *stat, int nsp,
                                                    l2_warm_t warm) {
    __shared__ __align__(16) float qs[AG][AHD];
    __shared__ __align__(16) float kr[AHD], vr[AHD];
    __shared__ __align__(16) float ks[AP][AHD + 4];   /* rows 16-byte aligned, lanes of a read on distinct banks */
    __shared__ float4 vs[AP][AHD / 4];
    __shared__ float wsp[AG][AMG];
    __shared__ float ps[AG][AP];
    __shared__ uint64_t etab[32];
    __shared__ int flag_s;
    if ((int)blockIdx.x >= KV * nsp) {          /* the L2 warming workgroups */
        l2_warm(warm, blockIdx.x - KV * nsp);
        return;
    }
    const int kh = blockIdx.x % KV, sp = blockIdx.x / KV, tid = threadIdx.x, lane = tid & 63,
              w = tid >> 6;
    const int pos = pos_dev ? *pos_dev : pos_arg;
    if (pos < 0 || pos + 1 > lim) {
        /* outside the cache (a position read on the device): the kv head's first split
           writes NaN for its AG query heads and records the status */
        if (sp == 0) {
            ((float4 *)(ao + (size_t)kh * AG * AHD))[tid] = make_float4(
                __int_as_float(0x7fc00000), __int_as_float(0x7fc00000),
                __int_as_float(0x7fc00000), __int_as_float(0x7fc00000));
            if (tid == 0) stat[0] = 1;
        }
        return;
    }
    const int n = pos + 1, j0 = sp * AP;
    if (j0 >= n) return;
    const int cnt = min(AP, n - j0), kvw = KV * AHD, half = AHD / 2, ns = (n + AP - 1) / AP;
    const bool has_new = pos < j0 + cnt;             /* this split holds the new row */
    /* ---- every load first */
    const int lastc = max(pos - 1, 0);
    float4 kreg[4], vreg[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int idx = tid + 256 * r, jj = idx / (AHD / 4), c = idx % (AHD / 4);
        const size_t o = (size_t)min(j0 + jj, lastc) * kvw + (size_t)kh * AHD + 4 * c;
        kreg[r] = *(const float4 *)(kc + o);
        vreg[r] = *(const float4 *)(vc + o);
    }
    const float4 q4 = ((const float4 *)(qkv + (size_t)kh * AG * AHD))[tid];  /* [q | k | v] */
    const int tc = min(tid, AHD - 1);
    const float knew = qkv[(size_t)(H + kh) * AHD + tc], vnew = qkv[(size_t)(H + KV + kh) * AHD + tc];
    const float gq0 = qn[lane], gq1 = qn[lane + 64], gk0 = kn[lane], gk1 = kn[lane + 64];
    const float2 csl = rope[(size_t)pos * half + lane];
    const uint64_t et = cpg_exp2f_tab[tid & 31];
    ((float4 *)qs)[tid] = q4;
    if (tid < 32) etab[tid] = et;
    if (tid < AHD) {
        kr[tid] = knew;
        vr[tid] = vnew;
    }
    __syncthreads();
    /* ---- wavefront w: query heads w and w + 4; wavefront 0 of the last split the new key */
    norm_rope_128(qs[w], gq0, gq1, csl, eps);
    norm_rope_128(qs[w + 4], gq0, gq1, csl, eps);
    if (w == 0 && has_new) norm_rope_128(kr, gk0, gk1, csl, eps);
    __syncthreads();
    if (has_new && tid < AHD) {
        kc[(size_t)pos * kvw + (size_t)kh * AHD + tid] = kr[tid];
        vc[(size_t)pos * kvw + (size_t)kh * AHD + tid] = vr[tid];
    }
    auto stage = [&](int r, float4 kv4, float4 vv4) {
        const int idx = tid + 256 * r, jj = idx / (AHD / 4), c = idx % (AHD / 4), j = j0 + jj;
        if (jj < cnt) {
            if (j >= pos) {
                kv4 = ((const float4 *)kr)[c];
                vv4 = ((const float4 *)vr)[c];
            }
            *(float4 *)&ks[jj][4 * c] = kv4;
            vs[jj][c] = vv4;
        }
    };
    stage(0, kreg[0], vreg[0]);       /* constant indices keep kreg / vreg in registers */
    stage(1, kreg[1], vreg[1]);
    stage(2, kreg[2], vreg[2]);
    stage(3, kreg[3], vreg[3]);
    __syncthreads();
    /* ---- thread (h, jj): the score; the 32 threads of a head are one half of a wavefront */
    const int h = tid / AP, jj = tid % AP;
    float sc = -INFINITY;
    if (jj < cnt) {
        const float4 *qh = (const float4 *)qs[h], *kh4 = (const float4 *)ks[jj];
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < AHD / 4; e++) {
            const float4 qv = qh[e], kv = kh4[e];
            a[e & 3] = fmaf(qv.x, kv.x, a[e & 3]);
            a[e & 3] = fmaf(qv.y, kv.y, a[e & 3]);
            a[e & 3] = fmaf(qv.z, kv.z, a[e & 3]);
            a[e & 3] = fmaf(qv.w, kv.w, a[e & 3]);
        }
        sc = __fdiv_rn((a[0] + a[1]) + (a[2] + a[3]), cpg_sqrt_rn((float)AHD));
    }
    const float m = half_max(sc);
    const float e = jj < cnt ? cpg_expf_tab(__fsub_rn(sc, m), etab) : 0.0f;
    const float l = half_sum(e);
    ps[h][jj] = e;
    __syncthreads();
    /* ---- thread (h, c): float4 c of the head's weighted sum of value rows */
    const int c = tid % AP;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j = 0; j < cnt; j++) {
        const float p = ps[h][j];
        const float4 v = vs[j][c];
        acc = make_float4(fmaf(p, v.x, acc.x), fmaf(p, v.y, acc.y), fmaf(p, v.z, acc.z),
                          fmaf(p, v.w, acc.w));
    }
    const size_t hb = (size_t)(kh * AG + h) * smax;
    float *pa = pacc + (hb + sp) * AHD + 4 * c;
    st_agent(pa + 0, acc.x);
    st_agent(pa + 1, acc.y);
    st_agent(pa + 2, acc.z);
    st_agent(pa + 3, acc.w);
    if (c == 0) {
        st_agent((float *)(pml + hb + sp), m);
        st_agent((float *)(pml + hb + sp) + 1, l);
    }
    /* ---- the last split of this kv head merges */
    if (!last_arriver(&ctr[kh], ns - 1, &flag_s)) return;
    /* Thread (h, c): float4 c of head h. The weights w_s = expf(m_s - M) (M the largest m_s)
       and L = sum_s w_s l_s are formed once per split by the head's 32 threads (split
       s0 + lane32 each) and shared through LDS within the wavefront; each thread then adds
       w_s acc_s over its splits in order, the loads of a group of AMG splits issued at once
       with the (m, l) of the group. */
    const int l32 = tid & 31;
    if (ns <= AMG) {
        /* one round of loads: split l32's (m, l), then every split's acc */
        const unsigned long long mlb = __hip_atomic_load(
            (unsigned long long *)(pml + hb + min(l32, ns - 1)), __ATOMIC_RELAXED,
            __HIP_MEMORY_SCOPE_AGENT);
        float4 aa[AMG];
#pragma unroll
        for (int u = 0; u < AMG; u++) {
            const size_t hs = hb + min(u, ns - 1);
            const v4i_t r = ld_agent16(pacc, (uint32_t)((hs * AHD + 4 * c) * sizeof(float)));
            aa[u] = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                                __int_as_float(r.w));
        }
        const float ms = __uint_as_float((uint32_t)mlb), ls = __uint_as_float((uint32_t)(mlb >> 32));
        const bool mine = l32 < ns;
        const float M1 = half_max(mine ? ms : -INFINITY);
        const float wgt = mine ? cpg_expf_tab(__fsub_rn(ms, M1), etab) : 0.0f;
        const float L1 = half_sum(mine ? __fmul_rn(wgt, ls) : 0.0f);
        if (l32 < AMG) wsp[h][l32] = wgt;
        wave_lds_sync();
        float4 o1 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int u = 0; u < AMG; u++) {          /* w = 0 past ns (its acc a valid split's) */
            const float wg = wsp[h][u];
            o1 = make_float4(fmaf(wg, aa[u].x, o1.x), fmaf(wg, aa[u].y, o1.y),
                             fmaf(wg, aa[u].z, o1.z), fmaf(wg, aa[u].w, o1.w));
        }
        *(float4 *)(ao + (size_t)(kh * AG + h) * AHD + 4 * c) =
            make_float4(__fdiv_rn(o1.x, L1), __fdiv_rn(o1.y, L1), __fdiv_rn(o1.z, L1),
                        __fdiv_rn(o1.w, L1));
        return;
    }
    float M = -INFINITY;
    for (int s0 = 0; s0 < ns; s0 += 32) {
        const int sidx = min(s0 + l32, ns - 1);
        M = fmaxf(M, ld_agent((const float *)(pml + hb + sidx)));
    }
    for (int o = 16; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    float L = 0.0f;
    float4 o4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 < ns; s0 += AMG) {
        float4 aa[AMG];
#pragma unroll
        for (int u = 0; u < AMG; u++) {          /* clamped, unconditional: in flight together */
            const size_t hs = hb + min(s0 + u, ns - 1);
            const v4i_t r = ld_agent16(pacc, (uint32_t)((hs * AHD + 4 * c) * sizeof(float)));
            aa[u] = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                                __int_as_float(r.w));
        }
        /* the group's weights: lane l32 < AMG of head h takes split s0 + l32 */
        {
            const bool mine = l32 < AMG && s0 + l32 < ns;
            const size_t hs = hb + min(s0 + (l32 < AMG ? l32 : 0), ns - 1);
            const float ms = ld_agent((const float *)(pml + hs));
            const float ls = ld_agent((const float *)(pml + hs) + 1);
            const float wgt = mine ? cpg_expf_tab(__fsub_rn(ms, M), etab) : 0.0f;
            float lw = mine ? __fmul_rn(wgt, ls) : 0.0f;
            for (int o = 1; o < 32; o <<= 1) lw += __shfl_xor(lw, o);
            L = __fadd_rn(L, lw);
            if (l32 < AMG) wsp[h][l32] = wgt;
            wave_lds_sync();
        }
#pragma unroll
        for (int u = 0; u < AMG; u++) {          /* w = 0 past ns (its acc a valid split's) */
            const float wg = wsp[h][u];
            o4 = make_float4(fmaf(wg, aa[u].x, o4.x), fmaf(wg, aa[u].y, o4.y),
                             fmaf(wg, aa[u].z, o4.z), fmaf(wg, aa[u].w, o4.w));
        }
        wave_lds_sync();                         /* wsp is rewritten by the next group */
    }
    *(float4 *)(ao + (size_t)(kh * AG + h) * AHD + 4 * c) =
        make_float4(__fdiv_rn(o4.x, L), __fdiv_rn(o4.y, L), __fdiv_rn(o4.z, L), __fdiv_rn(o4.w, L));
}

/* ================================================================ host side */

extern "C" int cpg_rope_table(float theta, int HD, int max_pos, float *out) {
    /* kernels.c:430-433: inv = powf(theta, -2i/hd); ang = (float)pos * inv; cosf, sinf */
    if (!out || HD <= 0 || HD % 2 || max_pos <= 0) { cpg_set_error("cpg_rope_table: bad arguments"); return -1; }
    const int half = HD / 2;
    for (int i = 0; i < half; i++) {
        const float inv = powf(theta, -2.0f * (float)i / (float)HD);
        for (int p = 0; p < max_pos; p++) {
            const float ang = (float)p * inv;
            out[((size_t)p * half + i) * 2 + 0] = cosf(ang);
            out[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    }
    return 0;
}

extern "C" int cpg_rmsnorm(const float *x, const float *g, int T, int D, float eps, float *out) {
    CPG_REQUIRE_INIT();
    if (!x || !g || !out || T <= 0 || D <= 0 || D % 4) { cpg_set_error("cpg_rmsnorm: bad arguments"); return -1; }
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, g_cpg.stream, x, g, D, eps, out);
    CPG_LAUNCH_CHECK("k_rmsnorm_rows");
    return 0;
}

template <int ENC, int B, int GR>
static int launch_gemv(const void *w, int n_in, int n_out, const float *x, int T,
                       const float *norm_g, float eps, float *out) {
    auto kfn = k_gemv<ENC, B, GR>;
    const size_t smem = sizeof(float) * ((size_t)MT * n_in + MT * (n_in / 32) + GW * MT * GR);
    if (smem > 160 * 1024) { cpg_set_error("cpg_gemv: n_in %d too large", n_in); return -1; }
    if (smem > 64 * 1024)
        CPG_HIP(hipFuncSetAttribute((const void *)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)smem));
    hipLaunchKernelGGL(kfn, dim3(n_out / GR), dim3(GW * 64), smem, g_cpg.stream,
                       (const uint8_t *)w, cpg_payload_plane(ENC, n_out, n_in), n_in, n_out, x, T,
                       norm_g, eps, out);
    CPG_LAUNCH_CHECK("k_gemv");
    return 0;
}

template <int ENC>
static int gemv_enc(const void *w, int n_in, int n_out, const float *x, int T,
                    const float *norm_g, float eps, float *out) {
    /* 8 rows per workgroup where 16 would leave CUs without a workgroup (one token) */
    if (T == 1 && n_out / GROWS < 256) {
        switch ((n_in / 32 + 2 * GSLICES - 1) / (2 * GSLICES)) {
        case 1: return launch_gemv<ENC, 1, 8>(w, n_in, n_out, x, T, norm_g, eps, out);
        case 2: return launch_gemv<ENC, 2, 8>(w, n_in, n_out, x, T, norm_g, eps, out);
        case 3: return launch_gemv<ENC, 3, 8>(w, n_in, n_out, x, T, norm_g, eps, out);
        case 4: return launch_gemv<ENC, 4, 8>(w, n_in, n_out, x, T, norm_g, eps, out);
        default: break;
        }
    }
    switch ((n_in / 32 + GSLICES - 1) / GSLICES) {
    case 1: return launch_gemv<ENC, 1, GROWS>(w, n_in, n_out, x, T, norm_g, eps, out);
    case 2: return launch_gemv<ENC, 2, GROWS>(w, n_in, n_out, x, T, norm_g, eps, out);
    case 3: return launch_gemv<ENC, 3, GROWS>(w, n_in, n_out, x, T, norm_g, eps, out);
    case 4: return launch_gemv<ENC, 4, GROWS>(w, n_in, n_out, x, T, norm_g, eps, out);
    default: cpg_set_error("cpg_gemv: n_in %d unsupported (at most %d)", n_in, 4 * 32 * GSLICES);
             return -1;
    }
}

static int gemv_any(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                    const float *norm_g, float eps, float *out) {
    CPG_REQUIRE_INIT();
    if (!w || !x || !out || T <= 0 || n_in <= 0 || n_in % 32 || n_out <= 0 || n_out % 64) {
        cpg_set_error("cpg_gemv: bad arguments (n_in %% 32, n_out %% 64 must be 0)");
        return -1;
    }
    if (enc == CPG_ENC_Q4) return gemv_enc<CPG_ENC_Q4>(w, n_in, n_out, x, T, norm_g, eps, out);
    if (enc == CPG_ENC_Q8) return gemv_enc<CPG_ENC_Q8>(w, n_in, n_out, x, T, norm_g, eps, out);
    cpg_set_error("cpg_gemv: encoding %d is not row-tiled (Q4_0 or Q8_0 only)", enc);
    return -1;
}

extern "C" int cpg_gemv(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                        float *out) {
    return gemv_any(enc, w, n_in, n_out, x, T, nullptr, 0.0f, out);
}

extern "C" int cpg_gemv_norm(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                             const float *g, float eps, float *out) {
    if (!g) { cpg_set_error("cpg_gemv_norm: null gain"); return -1; }
    return gemv_any(enc, w, n_in, n_out, x, T, g, eps, out);
}

struct cpg_attn_ws {
    int D, H, KV, HD, max_T;
    float *qkv, *q, *ao;
    float *pacc;            /* k_attn_split: (H, ASPLIT_MAX_POS / AP, HD), or null */
    float2 *pml;            /* k_attn_split: (H, ASPLIT_MAX_POS / AP) */
    int *ctr;               /* k_attn_split: KV arrival counters, zero between launches */
    int *stat;              /* 1 once a kernel saw a position outside the cache */
    void *dense;            /* cpg_dense_mfma for T >= DENSE_MIN_T, or null */
    void *block;
};

/* from this many tokens on the q|k|v and output projections run on MFMA (cpg_dense_mfma)
   instead of k_gemv, whose passes of MT tokens each re-stream the matrix */
#define DENSE_MIN_T 32

static int g_attn_mode = CPG_ATTN_SPLIT;     /* the per-head kernel where split does not apply */

extern "C" int cpg_attn_decode_mode(int mode) {
    if (mode != CPG_ATTN_PER_HEAD && mode != CPG_ATTN_SPLIT) {
        cpg_set_error("cpg_attn_decode_mode: unknown mode %d", mode);
        return -1;
    }
    g_attn_mode = mode;
    return 0;
}

/* the shapes k_attn_split is written for (Qwen3-30B-A3B: 32 query heads of 128, 4 kv heads) */
static bool attn_split_shape(int H, int KV, int HD) {
    return HD == AHD && KV > 0 && H == AG * KV;
}

extern "C" cpg_attn_ws *cpg_attn_ws_create(int D, int H, int KV, int HD, int max_T) {
    if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return nullptr; }
    if (D <= 0 || H <= 0 || KV <= 0 || H % KV || HD <= 0 || HD > 128 || HD % 4 || max_T <= 0) {
        cpg_set_error("cpg_attn_ws_create: bad geometry D=%d H=%d KV=%d HD=%d", D, H, KV, HD);
        return nullptr;
    }
    cpg_attn_ws *ws = (cpg_attn_ws *)calloc(1, sizeof *ws);
    if (!ws) { cpg_set_error("out of host memory"); return nullptr; }
    ws->D = D; ws->H = H; ws->KV = KV; ws->HD = HD; ws->max_T = max_T;
    const size_t T = (size_t)max_T, smax = ASPLIT_MAX_POS / AP;
    const bool split = attn_split_shape(H, KV, HD);
    const int nqkv = (H + 2 * KV) * HD;
    size_t dense = 0;
    if (cpg_dense_shape_ok(D, nqkv) && cpg_dense_shape_ok(H * HD, D))
        for (int t = DENSE_MIN_T; t <= max_T; t++) {
            const size_t a = cpg_dense_scratch_bytes(t, D, nqkv),
                         b = cpg_dense_scratch_bytes(t, H * HD, D);
            dense = a > dense ? a : dense;
            dense = b > dense ? b : dense;
        }
    const size_t sz[8] = {T * nqkv * 4, T * H * HD * 4, T * H * HD * 4,
                          split ? H * smax * HD * 4 : 0, split ? H * smax * 8 : 0, dense,
                          split ? (size_t)KV * 4 : 0, 4};
    size_t total = 0;
    for (int i = 0; i < 8; i++) total += cpg_round256(sz[i]);
    uint8_t *p = (uint8_t *)cpg_malloc(total);
    if (!p) { free(ws); return nullptr; }
    ws->block = p;
    void **dst[8] = {(void **)&ws->qkv, (void **)&ws->q, (void **)&ws->ao, (void **)&ws->pacc,
                     (void **)&ws->pml, &ws->dense, (void **)&ws->ctr, (void **)&ws->stat};
    for (int i = 0; i < 8; i++) {
        *dst[i] = sz[i] ? (void *)p : nullptr;
        p += cpg_round256(sz[i]);
    }
    if ((ws->ctr && cpg_memset(ws->ctr, 0, sz[6])) || cpg_memset(ws->stat, 0, sz[7])) {
        cpg_attn_ws_destroy(ws);
        return nullptr;
    }
    return ws;
}

extern "C" int cpg_attn_ws_status(cpg_attn_ws *ws) {
    CPG_REQUIRE_INIT();
    if (!ws) { cpg_set_error("cpg_attn_ws_status: null workspace"); return -1; }
    int v = 0;
    if (cpg_sync() || cpg_d2h(&v, ws->stat, sizeof v)) return -7;
    if (v && cpg_memset(ws->stat, 0, sizeof v)) return -7;
    return v;
}

extern "C" void cpg_attn_ws_destroy(cpg_attn_ws *ws) {
    if (!ws) return;
    cpg_free(ws->block);
    free(ws);
}

/* pos0 >= 0: the position as a value; pos_dev: read on the device (pos0 is then the largest
   value it may hold, which sizes the attention's LDS). */
static int attn_forward(const cpg_attn_layer *A, const float *x, int T, int pos0,
                        const int *pos_dev, float *kc, float *vc, int cap, float *attn,
                        cpg_attn_ws *ws) {
    CPG_REQUIRE_INIT();
    if (!A || !ws || !x || !kc || !vc || !attn || !A->ln1 || !A->q_norm || !A->k_norm ||
        !A->wqkv || !A->wo || !A->rope) {
        cpg_set_error("cpg_attn_forward: null argument");
        return -1;
    }
    if (A->D != ws->D || A->H != ws->H || A->KV != ws->KV || A->HD != ws->HD) {
        cpg_set_error("cpg_attn_forward: workspace geometry does not match the layer");
        return -1;
    }
    if (T <= 0 || T > ws->max_T || pos0 < 0 || pos0 + T > cap || pos0 + T > A->max_pos) {
        /* qwen3_moe.c:94-97 refuses a range outside the cache the same way */
        cpg_set_error("cpg_attn_forward: kv range %d+%d outside cache cap %d (rope table %d, "
                      "max T %d)", pos0, T, cap, A->max_pos, ws->max_T);
        return -1;
    }
    const int D = A->D, H = A->H, KV = A->KV, HD = A->HD, nqkv = (H + 2 * KV) * HD;
    const int lim = cap < A->max_pos ? cap : A->max_pos;
    hipStream_t s = g_cpg.stream;
    const bool dense = T >= DENSE_MIN_T && ws->dense;
    int rc;
    /* dense: ln1 writes the hi/lo planes of the product directly, the q|k|v product's k parts
       are summed by k_qk_norm_rope as it reads them, and the attention core writes the planes
       of the output projection's input (the scratch's planes are free again by then) */
    const float *qparts = ws->qkv;
    int qks = 1;
    _Float16 *ph = (_Float16 *)ws->dense;
    if (dense) {
        hipLaunchKernelGGL(k_rmsnorm_rows_hilo, dim3(T), dim3(256), 0, s, x, A->ln1, D, A->eps,
                           ph, ph + (size_t)T * D);
        CPG_LAUNCH_CHECK("k_rmsnorm_rows_hilo");
        rc = cpg_dense_from_planes(A->enc, A->wqkv, D, nqkv, T, ws->dense, ws->qkv, 0, &qparts,
                                   &qks);
    } else {
        /* RMSNorm(ln1) folded into the q|k|v GEMV's staging of x */
        rc = gemv_any(A->enc, A->wqkv, D, nqkv, x, T, A->ln1, A->eps, ws->qkv);
    }
    if (rc) return rc;
    const int nmax = pos_dev ? lim : pos0 + T;
    const size_t smem = sizeof(float) * (size_t)nmax;
    bool planes = false;                         /* the output projection's planes written */
    if (T == 1 && g_attn_mode == CPG_ATTN_SPLIT && ws->pacc && lim <= ASPLIT_MAX_POS) {
        const int smax = (lim + AP - 1) / AP;
        /* while the few attention workgroups run, the output projection's rows are read into
           the L2 of the XCD whose workgroups will read them */
        const l2_warm_t warm = l2_warm_rows(A->enc, A->wo, D, H * HD);
        hipLaunchKernelGGL(k_attn_split, dim3(KV * smax + NXCD * warm.parts), dim3(256), 0, s,
                           ws->qkv, A->q_norm, A->k_norm, (const float2 *)A->rope, H, KV, A->eps,
                           pos0, pos_dev, lim, kc, vc, ws->pacc, ws->pml, ASPLIT_MAX_POS / AP,
                           ws->ctr, ws->ao, ws->stat, smax, warm);
        CPG_LAUNCH_CHECK("k_attn_split");
    } else if (T == 1) {
        if (smem > 32 * 1024)
            CPG_HIP(hipFuncSetAttribute((const void *)k_attn_decode,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
        hipLaunchKernelGGL(k_attn_decode, dim3(H), dim3(ADT), smem, s, ws->qkv, A->q_norm,
                           A->k_norm, (const float2 *)A->rope, H, KV, HD, A->eps, pos0, pos_dev,
                           nmax, kc, vc, ws->ao, ws->stat);
        CPG_LAUNCH_CHECK("k_attn_decode");
    } else {
        hipLaunchKernelGGL(k_qk_norm_rope, dim3(T, H + 2 * KV), dim3(64), 0, s, qparts, qks,
                           (size_t)T * nqkv, A->q_norm, A->k_norm, (const float2 *)A->rope, H,
                           KV, HD, A->eps, pos0, pos_dev, lim, ws->q, kc, vc, ws->stat);
        CPG_LAUNCH_CHECK("k_qk_norm_rope");
        const int G = H / KV;
        _Float16 *aoh = dense ? ph : nullptr, *aol = dense ? ph + (size_t)T * H * HD : nullptr;
        if (HD == 128 && G <= 16 && 16 % G == 0 && T >= AMMA_MIN_T) {
            /* on MFMA: 64 query rows per workgroup share every key tile */
            const size_t sm = amma_lds_bytes();
            if (sm > 64 * 1024)
                CPG_HIP(hipFuncSetAttribute((const void *)k_attn_mma,
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm));
            const int TB = AMQ / G;
            hipLaunchKernelGGL(k_attn_mma, dim3(KV, (T + TB - 1) / TB), dim3(256), sm, s, ws->q,
                               kc, vc, H, KV, T, pos0, pos_dev, lim, ws->ao, aoh, aol);
            CPG_LAUNCH_CHECK("k_attn_mma");
            planes = dense;
        } else if (G <= 32 && 32 % G == 0 && HD <= 128) {
            /* the kv head's rows read once per block of tokens (k_attn_blk): 16 query rows
               per workgroup while 32 would leave CUs without one */
            const bool r16 = G <= 16 && (size_t)KV * ((T + 32 / G - 1) / (32 / G)) < 256;
            const int Rr = r16 ? 16 : 32, TB = Rr / G;
            const size_t sm = sizeof(float) * ((size_t)(Rr + AKT) * (HD + 4) + AKT * HD + Rr * AKT);
            const void *kf = r16 ? (const void *)k_attn_blk<16> : (const void *)k_attn_blk<32>;
            if (sm > 64 * 1024)
                CPG_HIP(hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm));
            if (r16)
                hipLaunchKernelGGL(k_attn_blk<16>, dim3(KV, (T + TB - 1) / TB), dim3(256), sm, s,
                                   ws->q, kc, vc, H, KV, HD, T, pos0, pos_dev, lim, ws->ao, aoh,
                                   aol);
            else
                hipLaunchKernelGGL(k_attn_blk<32>, dim3(KV, (T + TB - 1) / TB), dim3(256), sm, s,
                                   ws->q, kc, vc, H, KV, HD, T, pos0, pos_dev, lim, ws->ao, aoh,
                                   aol);
            CPG_LAUNCH_CHECK("k_attn_blk");
            planes = dense;
        } else {
            if (smem > 48 * 1024)
                CPG_HIP(hipFuncSetAttribute((const void *)k_attn_core,
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            hipLaunchKernelGGL(k_attn_core, dim3(H, T), dim3(256), smem, s, ws->q, kc, vc, H, KV,
                               HD, pos0, pos_dev, nmax, ws->ao);
            CPG_LAUNCH_CHECK("k_attn_core");
        }
    }
    if (dense && planes)
        return cpg_dense_from_planes(A->enc, A->wo, H * HD, D, T, ws->dense, attn, 1, nullptr,
                                     nullptr);
    if (dense) return cpg_dense_mfma(A->enc, A->wo, H * HD, D, ws->ao, T, ws->dense, attn);
    return cpg_gemv(A->enc, A->wo, H * HD, D, ws->ao, T, attn);
}

extern "C" int cpg_attn_forward(const cpg_attn_layer *A, const float *x, int T, int pos0,
                                float *kc, float *vc, int cap, float *attn, cpg_attn_ws *ws) {
    return attn_forward(A, x, T, pos0, nullptr, kc, vc, cap, attn, ws);
}

extern "C" int cpg_attn_forward_at(const cpg_attn_layer *A, const float *x, int T,
                                   const int *pos_dev, float *kc, float *vc, int cap,
                                   float *attn, cpg_attn_ws *ws) {
    if (!pos_dev) { cpg_set_error("cpg_attn_forward_at: null position"); return -1; }
    const int lim = A && cap > A->max_pos ? A->max_pos : cap;
    return attn_forward(A, x, T, lim - T, pos_dev, kc, vc, cap, attn, ws);
}
