/* attn.hip — the attention half of a Qwen3 decoder layer on gfx950, plus the row-tiled GEMV
 * it (and the output head) uses.
 *
 * Reference: engine/blocks/qwen3_moe.c:110-167 (attention half of qwen3_layer_kv), with
 * engine/kernels/kernels.c rmsnorm :408-413, rope_apply_from :425-447, softmax :20-26, and the
 * per-head RMSNorm of qwen3_moe.c:44-49.
 *
 * One call for T new tokens at positions pos0..pos0+T-1, five kernels on one stream:
 *   k_rmsnorm_rows   xn = rmsnorm(x, ln1): the sum of squares accumulated in double, then
 *                    the reference's float formula for 1/sqrt and the scaling.
 *   k_gemv           q|k|v = [Wq; Wk; Wv] . xn, one row-tiled matrix of (H + 2 KV) * HD rows.
 *   k_qk_norm_rope   per head: the reference's RMSNorm of the head (serial sum of squares, so
 *                    bit-identical given the same q/k), then RoPE with a cos/sin table the
 *                    host computes with the same libm calls as the reference; k and v rows go
 *                    to the cache at pos0 + t.
 *   k_attn_core      per (head, token): scores with the reference's serial dot products and
 *                    division by sqrtf(HD), softmax with serial max/sum and the
 *                    glibc-identical expf, and the serial weighted sum over positions: given
 *                    the same q/k/v this is bit-identical to the reference.
 *   k_gemv           attn = Wo . ao.
 * The projections accumulate in fp32 in a different order than the CPU GEMVs (within ~1e-6
 * relative), which is what separates this path from the reference's bits.
 */
#include "cpg_internal.h"
#include "cpg_gemv.h"

#include <math.h>
#include <stdlib.h>

#define GROWS 16            /* k_gemv: rows per workgroup */
#define GSLICES (4 * GW)    /* k_gemv: k slices per row (4 per wavefront) */

/* grid T, 256 threads: out[t] = (x[t] * inv) * g with inv = 1/sqrtf(ss/D + eps), ss = sum x^2
   accumulated in double (kernels.c:408-413 up to the order of that sum). D % 4 == 0. */
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ x,
                                                      const float *__restrict__ g, int D,
                                                      float eps, float *__restrict__ out) {
    __shared__ double part[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float4 *x4 = (const float4 *)(x + (size_t)t * D);
    double ss = 0.0;
    for (int i = tid; i < D / 4; i += 256) {
        const float4 v = x4[i];
        ss += (double)__fmul_rn(v.x, v.x) + (double)__fmul_rn(v.y, v.y) +
              (double)__fmul_rn(v.z, v.z) + (double)__fmul_rn(v.w, v.w);
    }
    ss = wave_sum_d(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn((float)ss, (float)D), eps)));
    const float4 *g4 = (const float4 *)g;
    float4 *o4 = (float4 *)(out + (size_t)t * D);
    for (int i = tid; i < D / 4; i += 256) {
        const float4 v = x4[i], gv = g4[i];
        o4[i] = make_float4(__fmul_rn(__fmul_rn(v.x, inv), gv.x), __fmul_rn(__fmul_rn(v.y, inv), gv.y),
                            __fmul_rn(__fmul_rn(v.z, inv), gv.z), __fmul_rn(__fmul_rn(v.w, inv), gv.w));
    }
}

/* grid (n_out/16), GW*64 threads: out[t*n_out + row] = W[row] . x[t] for t < T, W row-tiled
   (n_out a multiple of 64). Lane = (row r = lane % 16, slice lane / 16); slice s of wavefront
   w holds blocks [(4w + s) * BPW, +BPW) of the row in registers for the whole call, tokens
   are staged MT at a time, and the 32 slices are summed in a fixed order (two shuffles in
   the wavefront, then the GW wavefronts through LDS). BPW = ceil(n_in / 32 / 32). */
template <int ENC, int BPW>
__global__ __launch_bounds__(GW * 64) void k_gemv(const uint8_t *__restrict__ W,
                                                  size_t payload_plane, int n_in, int n_out,
                                                  const float *__restrict__ x, int T,
                                                  float *__restrict__ out) {
    extern __shared__ float smem[];
    const int nb = n_in / 32;
    float *xs = smem;                            /* MT * n_in */
    float *bsum = xs + MT * n_in;                /* MT * nb */
    float *red = bsum + MT * nb;                 /* GW * MT * GROWS */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % GROWS, sl = w * 4 + lane / GROWS, b0 = sl * BPW;
    const int row = blockIdx.x * GROWS + r, nbw = max(0, min(BPW, nb - b0));
    WBlk<ENC> wv[BPW];
    float dv[BPW];
    load_row_blocks<ENC, BPW>(W, payload_plane, row, b0, nb - 1, nb, wv, dv);
    for (int t0 = 0; t0 < T; t0 += MT) {
        const int mc = min(MT, T - t0);
#pragma unroll
        for (int j = 0; j < BPW; j++) wv[j].pin();
        stage_tokens<ENC, GW * 64>(xs, bsum, n_in, mc, [&](int i, int k4) {
            return *(const float4 *)(x + (size_t)(t0 + i) * n_in + 4 * k4);
        });
        float acc[MT];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i] = 0.0f;
        row_dots<ENC, BPW>(wv, dv, b0, nbw, xs, bsum, n_in, nb, mc, acc);
#pragma unroll
        for (int i = 0; i < MT; i++) {
            acc[i] += __shfl_xor(acc[i], 16);
            acc[i] += __shfl_xor(acc[i], 32);
            if (lane < GROWS) red[(w * MT + i) * GROWS + r] = acc[i];
        }
        __syncthreads();
        if (w == 0 && lane < GROWS)
            for (int i = 0; i < mc; i++) {
                float s = 0.0f;
                for (int ww = 0; ww < GW; ww++) s += red[(ww * MT + i) * GROWS + r];
                out[(size_t)(t0 + i) * n_out + row] = s;
            }
        __syncthreads();
    }
}

/* One head row of HD floats in LDS: the reference's rmsnorm (serial sum of squares by one
   lane, kernels.c:410) with gain g, in place. Whole wavefront. */
__device__ static inline void head_rmsnorm_lds(float *v, const float *__restrict__ g, int HD,
                                               float eps, float *inv_lds) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) {
        float ss = 0.0f;
        for (int i = 0; i < HD; i++) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
        *inv_lds = __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)HD), eps)));
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const float inv = *inv_lds;
    for (int i = lane; i < HD; i += 64) v[i] = __fmul_rn(__fmul_rn(v[i], inv), g[i]);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

/* grid (T, H + 2*KV), 64 threads. Head hh of token t in qkv (T, (H + 2 KV) * HD): q heads are
   RMS-normed with qn and rotated into q (T, H*HD); k heads normed with kn, rotated, and written
   to the cache row pos0 + t; v heads copied to the value cache. rope: [pos][HD/2] (cos, sin)
   pairs (kernels.c:430-433, computed on the host). HD <= 256, even. */
__global__ __launch_bounds__(64) void k_qk_norm_rope(const float *__restrict__ qkv,
                                                     const float *__restrict__ qn,
                                                     const float *__restrict__ kn,
                                                     const float2 *__restrict__ rope, int H,
                                                     int KV, int HD, float eps, int pos0,
                                                     float *__restrict__ q, float *__restrict__ kc,
                                                     float *__restrict__ vc) {
    __shared__ float v[256];
    __shared__ float inv_s;
    const int t = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x, half = HD / 2;
    const float *src = qkv + (size_t)t * (H + 2 * KV) * HD + (size_t)hh * HD;
    const size_t crow = (size_t)(pos0 + t) * KV * HD;
    if (hh >= H + KV) {                          /* value head: to the cache unchanged */
        for (int i = lane; i < HD; i += 64) vc[crow + (size_t)(hh - H - KV) * HD + i] = src[i];
        return;
    }
    for (int i = lane; i < HD; i += 64) v[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    head_rmsnorm_lds(v, hh < H ? qn : kn, HD, eps, &inv_s);
    float *dst = hh < H ? q + (size_t)t * H * HD + (size_t)hh * HD
                        : kc + crow + (size_t)(hh - H) * HD;
    const float2 *cs = rope + (size_t)(pos0 + t) * half;
    for (int i = lane; i < half; i += 64) {
        const float a = v[i], b = v[i + half], c = cs[i].x, s = cs[i].y;
        dst[i] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
        dst[i + half] = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
    }
}

/* grid (H, T), 128 threads, HD <= 128. Head h of token i (position last = pos0 + i) against
   cache rows 0..last of kv head h / (H/KV): qwen3_moe.c:144-160 in the reference's order. */
__global__ __launch_bounds__(128) void k_attn_core(const float *__restrict__ q,
                                                   const float *__restrict__ kc,
                                                   const float *__restrict__ vc, int H, int KV,
                                                   int HD, int pos0, float *__restrict__ ao) {
    extern __shared__ float sc[];                /* last + 1 scores, then probabilities */
    __shared__ float qs[128];
    __shared__ float red[2];
    __shared__ float sum_s;
    const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const int kh = h / (H / KV), n = pos0 + i + 1, kvw = KV * HD;
    const float *qi = q + ((size_t)i * H + h) * HD;
    for (int e = tid; e < HD; e += 128) qs[e] = qi[e];
    __syncthreads();
    const float rs = cpg_sqrt_rn((float)HD);
    float mx = -INFINITY;
    for (int j = tid; j < n; j += 128) {
        const float *kj = kc + (size_t)j * kvw + (size_t)kh * HD;
        float s = 0.0f;
        for (int e = 0; e < HD; e += 4) {
            const float4 kv4 = *(const float4 *)(kj + e);
            s = __fadd_rn(s, __fmul_rn(qs[e], kv4.x));
            s = __fadd_rn(s, __fmul_rn(qs[e + 1], kv4.y));
            s = __fadd_rn(s, __fmul_rn(qs[e + 2], kv4.z));
            s = __fadd_rn(s, __fmul_rn(qs[e + 3], kv4.w));
        }
        s = __fdiv_rn(s, rs);
        sc[j] = s;
        mx = s > mx ? s : mx;
    }
    /* softmax (kernels.c:20-26): the maximum does not depend on the order it is taken in */
    for (int o = 32; o >= 1; o >>= 1) {
        const float other = __shfl_xor(mx, o);
        mx = other > mx ? other : mx;
    }
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0] > red[1] ? red[0] : red[1];
    for (int j = tid; j < n; j += 128) sc[j] = cpg_expf(__fsub_rn(sc[j], mx));
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int j = 0; j < n; j++) s = __fadd_rn(s, sc[j]);
        sum_s = s;
    }
    __syncthreads();
    const float sum = sum_s;
    for (int j = tid; j < n; j += 128) sc[j] = __fdiv_rn(sc[j], sum);
    __syncthreads();
    if (tid < HD) {
        const float *vcol = vc + (size_t)kh * HD + tid;
        float acc = 0.0f;
        for (int j = 0; j < n; j++) acc = __fadd_rn(acc, __fmul_rn(sc[j], vcol[(size_t)j * kvw]));
        ao[(size_t)i * H * HD + (size_t)h * HD + tid] = acc;
    }
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

template <int ENC, int B>
static int launch_gemv(const void *w, int n_in, int n_out, const float *x, int T, float *out) {
    auto kfn = k_gemv<ENC, B>;
    const size_t smem = sizeof(float) * ((size_t)MT * n_in + MT * (n_in / 32) + GW * MT * GROWS);
    if (smem > 160 * 1024) { cpg_set_error("cpg_gemv: n_in %d too large", n_in); return -1; }
    if (smem > 64 * 1024)
        CPG_HIP(hipFuncSetAttribute((const void *)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)smem));
    hipLaunchKernelGGL(kfn, dim3(n_out / GROWS), dim3(GW * 64), smem, g_cpg.stream,
                       (const uint8_t *)w, cpg_payload_plane(ENC, n_out, n_in), n_in, n_out, x, T,
                       out);
    CPG_LAUNCH_CHECK("k_gemv");
    return 0;
}

template <int ENC>
static int gemv_enc(const void *w, int n_in, int n_out, const float *x, int T, float *out) {
    switch ((n_in / 32 + GSLICES - 1) / GSLICES) {
    case 1: return launch_gemv<ENC, 1>(w, n_in, n_out, x, T, out);
    case 2: return launch_gemv<ENC, 2>(w, n_in, n_out, x, T, out);
    case 3: return launch_gemv<ENC, 3>(w, n_in, n_out, x, T, out);
    case 4: return launch_gemv<ENC, 4>(w, n_in, n_out, x, T, out);
    default: cpg_set_error("cpg_gemv: n_in %d unsupported (at most %d)", n_in, 4 * 32 * GSLICES);
             return -1;
    }
}

extern "C" int cpg_gemv(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                        float *out) {
    CPG_REQUIRE_INIT();
    if (!w || !x || !out || T <= 0 || n_in <= 0 || n_in % 32 || n_out <= 0 || n_out % 64) {
        cpg_set_error("cpg_gemv: bad arguments (n_in %% 32, n_out %% 64 must be 0)");
        return -1;
    }
    if (enc == CPG_ENC_Q4) return gemv_enc<CPG_ENC_Q4>(w, n_in, n_out, x, T, out);
    if (enc == CPG_ENC_Q8) return gemv_enc<CPG_ENC_Q8>(w, n_in, n_out, x, T, out);
    cpg_set_error("cpg_gemv: encoding %d is not row-tiled (Q4_0 or Q8_0 only)", enc);
    return -1;
}

struct cpg_attn_ws {
    int D, H, KV, HD, max_T;
    float *xn, *qkv, *q, *ao;
    void *block;
};

extern "C" cpg_attn_ws *cpg_attn_ws_create(int D, int H, int KV, int HD, int max_T) {
    if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return nullptr; }
    if (D <= 0 || H <= 0 || KV <= 0 || H % KV || HD <= 0 || HD > 128 || HD % 4 || max_T <= 0) {
        cpg_set_error("cpg_attn_ws_create: bad geometry D=%d H=%d KV=%d HD=%d", D, H, KV, HD);
        return nullptr;
    }
    cpg_attn_ws *ws = (cpg_attn_ws *)calloc(1, sizeof *ws);
    if (!ws) { cpg_set_error("out of host memory"); return nullptr; }
    ws->D = D; ws->H = H; ws->KV = KV; ws->HD = HD; ws->max_T = max_T;
    const size_t T = (size_t)max_T;
    const size_t sz[4] = {T * D * 4, T * (H + 2 * KV) * HD * 4, T * H * HD * 4, T * H * HD * 4};
    size_t total = 0;
    for (int i = 0; i < 4; i++) total += cpg_round256(sz[i]);
    uint8_t *p = (uint8_t *)cpg_malloc(total);
    if (!p) { free(ws); return nullptr; }
    ws->block = p;
    float **dst[4] = {&ws->xn, &ws->qkv, &ws->q, &ws->ao};
    for (int i = 0; i < 4; i++) { *dst[i] = (float *)p; p += cpg_round256(sz[i]); }
    return ws;
}

extern "C" void cpg_attn_ws_destroy(cpg_attn_ws *ws) {
    if (!ws) return;
    cpg_free(ws->block);
    free(ws);
}

extern "C" int cpg_attn_forward(const cpg_attn_layer *A, const float *x, int T, int pos0,
                                float *kc, float *vc, int cap, float *attn, cpg_attn_ws *ws) {
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
    hipStream_t s = g_cpg.stream;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, x, A->ln1, D, A->eps, ws->xn);
    CPG_LAUNCH_CHECK("k_rmsnorm_rows");
    int rc = cpg_gemv(A->enc, A->wqkv, D, nqkv, ws->xn, T, ws->qkv);
    if (rc) return rc;
    hipLaunchKernelGGL(k_qk_norm_rope, dim3(T, H + 2 * KV), dim3(64), 0, s, ws->qkv, A->q_norm,
                       A->k_norm, (const float2 *)A->rope, H, KV, HD, A->eps, pos0, ws->q, kc, vc);
    CPG_LAUNCH_CHECK("k_qk_norm_rope");
    const size_t smem = sizeof(float) * (size_t)(pos0 + T);
    if (smem > 64 * 1024)
        CPG_HIP(hipFuncSetAttribute((const void *)k_attn_core,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    hipLaunchKernelGGL(k_attn_core, dim3(H, T), dim3(128), smem, s, ws->q, kc, vc, H, KV, HD,
                       pos0, ws->ao);
    CPG_LAUNCH_CHECK("k_attn_core");
    return cpg_gemv(A->enc, A->wo, H * HD, D, ws->ao, T, attn);
}
