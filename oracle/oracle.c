/* oracle.c — CPU restatement of the reference's Qwen3-MoE arithmetic (the checker).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg; never by the product library.
 *
 * Built with gcc -std=c11 -ffp-contract=off -mfma: every `a * b + c` below rounds twice,
 * as GCC -std=c11 compiles the reference, and every fused multiply-add the reference gets
 * from an AVX2 intrinsic is written out as fmaf().
 *
 * How each function is pinned (tests/test_oracle.py):
 *   or_f16_to_f32, or_q4/q8_dequant_row : exhaustive over all 65,536 fp16 scales x every
 *       nibble / int8 value against the reference decoders compiled from source
 *       (oracle/_ref) and against the closed form y = q * d (exact in fp32).
 *   or_expf          : exhaustive over all 2^32 float inputs against the host glibc expf.
 *   or_softmax, or_silu, or_rmsnorm, or_matmul_wx : reference engine on seeded vectors,
 *       bit-exact; closed forms (constant vectors, ties) for softmax/rmsnorm.
 *   or_matmul_wx_q4/_q8 : reference engine bit-exact at both thread-count numerics, and
 *       float64 dequant+matmul to 1e-5 (the reference's own gate tolerance).
 *   or_moe           : golden fixtures written by the reference engine's qwen3_layer
 *       (tests/golden/), bit-exact, at CP_THREADS=1 and CP_THREADS=8.
 *   or_attn, or_rope : the reference engine's qwen3_layer_kv (oracle/_ref, through
 *       ref_attn_layer) on seeded layers, bit-exact, prefill and incremental positions,
 *       f32 / Q8_0 / Q4_0 projections; RoPE at position 0 is the identity and rotations
 *       preserve each pair's norm (closed forms).
 *   or_encode_q4_0/_q8_0, or_f64_to_f16 : vectors written by the reference's own numpy
 *       encoders (tests/golden/make_encoder_vectors.py) and numpy's float16 cast.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 and dequant */

/* engine/kernels/kernels.c:109-130: sign, exponent and mantissa moved into place;
   subnormals renormalised; inf/NaN keep their mantissa. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            uint32_t ee = 113;                 /* 127 - 15 + 1 */
            while (!(m & 0x400u)) { m <<= 1; ee--; }
            bits = sign | (ee << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

static float blk_scale(const uint8_t *blk) {           /* kernels.c:132-135 */
    return or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
}

/* engine/kernels/kernels.c:143-151: y = (float)int8 * d */
void or_q8_dequant_row(const uint8_t *blocks, float *out, int n) {
    for (int g = 0; g < n / 32; g++) {
        const uint8_t *b = blocks + (size_t)g * 34;
        const float d = blk_scale(b);
        for (int i = 0; i < 32; i++) out[g * 32 + i] = (float)(int8_t)b[2 + i] * d;
    }
}

static int nib_signed(int v) { return v > 7 ? v - 16 : v; }

/* engine/kernels/kernels.c:463-477: byte k -> element k (low nibble), k+16 (high) */
void or_q4_dequant_row(const uint8_t *blocks, float *out, int n) {
    for (int g = 0; g < n / 32; g++) {
        const uint8_t *b = blocks + (size_t)g * 18;
        const float d = blk_scale(b);
        for (int k = 0; k < 16; k++) {
            out[g * 32 + k] = (float)nib_signed(b[2 + k] & 15) * d;
            out[g * 32 + k + 16] = (float)nib_signed(b[2 + k] >> 4) * d;
        }
    }
}

/* ------------------------------------------------------------------ GEMVs */

/* engine/kernels/kernels.c:84-95 (and wx_slice :75-82): out[i] = serial sum of
   fl(w[i,k] * x[k]) over k = 0..n_in-1. Splitting rows over threads keeps the order. */
void or_matmul_wx(float *out, const float *x, const float *w, int n_in, int n_out) {
    for (int i = 0; i < n_out; i++) {
        float acc = 0.0f;
        const float *row = w + (size_t)i * n_in;
        for (int k = 0; k < n_in; k++) acc += row[k] * x[k];
        out[i] = acc;
    }
}

/* kernels.c:208-213: fixed pairwise order over the 8 AVX2 lanes */
static float hsum8(const float l[8]) {
    return ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
}

/* engine/kernels/kernels.c:368-396 through wx_q8_slice :316-366. With AVX2 every row is
   one 8-lane accumulator; block g, quarter h: lane j += fl(q[8h+j]*d) * x[32g+8h+j] as an
   FMA (q8_dot_acc_avx2_x4 :299-313 and q8_dot_acc_avx2 :196-206 are the same per row). */
void or_matmul_wx_q8(float *out, const float *x, const uint8_t *w, int n_in, int n_out) {
    const int ng = n_in / 32;
    const size_t rowbytes = (size_t)ng * 34;
    for (int i = 0; i < n_out; i++) {
        const uint8_t *row = w + (size_t)i * rowbytes;
        float s[8] = {0};
        for (int g = 0; g < ng; g++) {
            const uint8_t *b = row + (size_t)g * 34;
            const float d = blk_scale(b);
            for (int h = 0; h < 4; h++)
                for (int j = 0; j < 8; j++) {
                    const float v = (float)(int8_t)b[2 + 8 * h + j] * d;
                    s[j] = fmaf(v, x[g * 32 + 8 * h + j], s[j]);
                }
        }
        out[i] = hsum8(s);
    }
}

/* engine/kernels/kernels.c:514-540. */
void or_matmul_wx_q4(float *out, const float *x, const uint8_t *w, int n_in, int n_out,
                     int threads) {
    const int ng = n_in / 32;
    const size_t rowbytes = (size_t)ng * 18;
    const int avx2 = threads > 1 && (long)n_in * n_out >= 60000L && n_out > 1;
    for (int i = 0; i < n_out; i++) {
        const uint8_t *row = w + (size_t)i * rowbytes;
        if (avx2) {
            /* wx_q4_slice :487-511. s0 takes elements 0-7 then 16-23 of each block,
               s1 takes 8-15 then 24-31; lane j of each run is element (run start + j). */
            float s0[8] = {0}, s1[8] = {0};
            for (int g = 0; g < ng; g++) {
                const uint8_t *b = row + (size_t)g * 18;
                const float d = blk_scale(b);
                const float *xg = x + g * 32;
                for (int j = 0; j < 8; j++) {
                    const float lo0 = (float)nib_signed(b[2 + j] & 15) * d;
                    const float lo1 = (float)nib_signed(b[2 + 8 + j] & 15) * d;
                    const float hi0 = (float)nib_signed(b[2 + j] >> 4) * d;
                    const float hi1 = (float)nib_signed(b[2 + 8 + j] >> 4) * d;
                    s0[j] = fmaf(lo0, xg[j], s0[j]);
                    s1[j] = fmaf(lo1, xg[8 + j], s1[j]);
                    s0[j] = fmaf(hi0, xg[16 + j], s0[j]);
                    s1[j] = fmaf(hi1, xg[24 + j], s1[j]);
                }
            }
            float l[8];
            for (int j = 0; j < 8; j++) l[j] = s0[j] + s1[j];
            out[i] = hsum8(l);
        } else {
            /* scalar loop :524-539: element k then element k+16, no FMA */
            float acc = 0.0f;
            for (int g = 0; g < ng; g++) {
                const uint8_t *b = row + (size_t)g * 18;
                const float d = blk_scale(b);
                for (int k = 0; k < 16; k++) {
                    const float lo = (float)nib_signed(b[2 + k] & 15) * d;
                    const float hi = (float)nib_signed(b[2 + k] >> 4) * d;
                    acc += lo * x[g * 32 + k];
                    acc += hi * x[g * 32 + k + 16];
                }
            }
            out[i] = acc;
        }
    }
}

/* ------------------------------------------------------------------ norms, softmax */

/* engine/kernels/kernels.c:408-413 */
void or_rmsnorm(float *out, const float *x, const float *g, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * g[i];
}

/* glibc 2.35 expf: x*32/ln2 = k + r, exp(x) = 2^(k/32) * p(r/32) with a 32-entry table
   of 2^(i/32) and a cubic evaluated in double (ARM optimized-routines exp2f_data). The
   table entries are the binary64 values of 2^(i/32) with i<<47 subtracted from their bit
   patterns (oracle/derive_exp2_table.py recomputes them from first principles). glibc's
   x86_64 build selects an FMA variant, so every multiply-add that GCC contracts there is
   an fma() here; this is the variant that matches the host libm on all 2^32 inputs. */
static const uint64_t EXP2F_T[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static double u64_f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static uint64_t f64_u64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

float or_expf(float x) {
    const uint32_t abstop = (f32_bits(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       /* |x| >= 88 (top12(88.0f)), or NaN */
        if (f32_bits(x) == 0xff800000u) return 0.0f;              /* -inf */
        if (abstop >= 0x7f8) return x + x;                         /* inf or NaN */
        if (x > 0x1.62e42ep6f) return HUGE_VALF;                   /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                       /* underflow */
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);        /* round(x*32/ln2) via the shift trick */
    const uint64_t ki = f64_u64(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const double s = u64_f64(EXP2F_T[ki % 32] + (ki << 47));
    const double z = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

/* engine/kernels/kernels.c:20-26: serial max, expf(x - max), serial sum, divide. */
void or_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = or_expf(x[i] - mx); sum += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

/* engine/kernels/kernels.c:416 */
float or_silu(float x) { return x / (1.0f + or_expf(-x)); }

/* engine/blocks/qwen3_moe.c:36-40 */
static void mm(const void *p, int enc, float *out, const float *x, int n_in, int n_out,
               int threads) {
    if (enc == OR_ENC_Q4) or_matmul_wx_q4(out, x, (const uint8_t *)p, n_in, n_out, threads);
    else if (enc == OR_ENC_Q8) or_matmul_wx_q8(out, x, (const uint8_t *)p, n_in, n_out);
    else or_matmul_wx(out, x, (const float *)p, n_in, n_out);
}

/* ------------------------------------------------------------------ the MoE half */

/* engine/blocks/qwen3_moe.c:169-223, one token at a time as the reference does. */
void or_moe(int D, int E, int K, int F, float eps, const float *ln2, const float *wgate,
            const void *const *exp_ptr, int enc, int threads,
            const float *x, const float *attn, int T,
            float *xn_out, float *router_out, int *topk_out, float *wt_out, float *mlp) {
    const int HF = F > D ? F : D;
    float *hh = malloc(sizeof(float) * (size_t)HF), *gu = malloc(sizeof(float) * (size_t)HF);
    float *xn = malloc(sizeof(float) * (size_t)D), *lg = malloc(sizeof(float) * (size_t)E);
    float *probs = malloc(sizeof(float) * (size_t)E), *wt = malloc(sizeof(float) * (size_t)K);
    int *idx = malloc(sizeof(int) * (size_t)K);
    for (int t = 0; t < T; t++) {
        /* :178 hh = x + attn (the reference always adds; attn NULL means +0.0f) */
        for (int j = 0; j < D; j++)
            hh[j] = x[(size_t)t * D + j] + (attn ? attn[(size_t)t * D + j] : 0.0f);
        or_rmsnorm(xn, hh, ln2, D, eps);                                    /* :179 */
        or_matmul_wx(lg, xn, wgate, D, E);                                  /* :180 */
        memcpy(probs, lg, sizeof(float) * (size_t)E);                       /* :181 */
        or_softmax(probs, E);                                               /* :182 */
        for (int j = 0; j < K; j++) {                                       /* :185-194 */
            int best = -1;
            for (int e = 0; e < E; e++) {
                int taken = 0;
                for (int p = 0; p < j; p++) if (idx[p] == e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || probs[e] > probs[best]) best = e;
            }
            idx[j] = best;
        }
        float sum = 0.0f;                                                   /* :195-197 */
        for (int j = 0; j < K; j++) sum += probs[idx[j]];
        for (int j = 0; j < K; j++) wt[j] = probs[idx[j]] / sum;
        for (int j = 0; j < K; j++) {                                       /* :199-222 */
            const int e = idx[j];
            mm(exp_ptr[(size_t)e * 3 + 0], enc, gu, xn, D, F, threads);     /* gate */
            mm(exp_ptr[(size_t)e * 3 + 1], enc, hh, xn, D, F, threads);     /* up   */
            for (int i = 0; i < F; i++) gu[i] = or_silu(gu[i]) * hh[i];
            mm(exp_ptr[(size_t)e * 3 + 2], enc, hh, gu, F, D, threads);     /* down */
            if (mlp)
                for (int i = 0; i < D; i++) mlp[(size_t)t * D + i] += wt[j] * hh[i];
        }
        if (xn_out) memcpy(xn_out + (size_t)t * D, xn, sizeof(float) * (size_t)D);
        if (router_out) memcpy(router_out + (size_t)t * E, lg, sizeof(float) * (size_t)E);
        if (topk_out) memcpy(topk_out + (size_t)t * K, idx, sizeof(int) * (size_t)K);
        if (wt_out) memcpy(wt_out + (size_t)t * K, wt, sizeof(float) * (size_t)K);
    }
    free(hh); free(gu); free(xn); free(lg); free(probs); free(wt); free(idx);
}

/* ------------------------------------------------------------------ the attention half */

/* engine/kernels/kernels.c:425-447 (rope_apply_from): pairs (i, i + hd/2) of every q and k
   head of token t rotate by (float)(pos0 + t) * powf(theta, -2i/hd). */
void or_rope(float *q, float *k, int T, int pos0, int nq, int nk, int hd, float theta) {
    const int half = hd / 2;
    for (int t = 0; t < T; t++) {
        for (int i = 0; i < half; i++) {
            const float inv = powf(theta, -2.0f * (float)i / (float)hd);
            const float ang = (float)(pos0 + t) * inv;
            const float c = cosf(ang), s = sinf(ang);
            float *rows[2] = {q + (size_t)t * nq * hd, k + (size_t)t * nk * hd};
            const int nh[2] = {nq, nk};
            for (int r = 0; r < 2; r++)
                for (int h = 0; h < nh[r]; h++) {
                    float *v = rows[r] + (size_t)h * hd;
                    const float a = v[i], b = v[i + half];
                    v[i] = a * c - b * s;
                    v[i + half] = b * c + a * s;
                }
        }
    }
}

/* engine/blocks/qwen3_moe.c:44-49: RMSNorm of every head_dim row with the shared gain */
static void head_rmsnorm(float *v, int rows, int hd, const float *g, float eps) {
    for (int r = 0; r < rows; r++) or_rmsnorm(v + (size_t)r * hd, v + (size_t)r * hd, g, hd, eps);
}

/* engine/blocks/qwen3_moe.c:110-167: the attention half of qwen3_layer_kv for T new tokens
   at positions pos0..pos0+T-1. kc/vc: the cache, (pos0+T) rows of KV*HD floats; rows below
   pos0 are read, rows pos0.. are written. attn (T, D) receives the pre-residual output. */
void or_attn(int D, int H, int KV, int HD, float theta, float eps, const float *ln1,
             const float *qn, const float *kn, const void *wq, const void *wk, const void *wv,
             const void *wo, int enc, int threads, const float *x, int T, int pos0, float *kc,
             float *vc, float *attn) {
    const int rep = H / KV;
    float *xn = malloc(sizeof(float) * (size_t)T * D);
    float *q = malloc(sizeof(float) * (size_t)T * H * HD);
    float *ao = malloc(sizeof(float) * (size_t)T * H * HD);
    float *sc = malloc(sizeof(float) * (size_t)(pos0 + T));
    for (int t = 0; t < T; t++) {                                            /* :134-139 */
        or_rmsnorm(xn + (size_t)t * D, x + (size_t)t * D, ln1, D, eps);
        mm(wq, enc, q + (size_t)t * H * HD, xn + (size_t)t * D, D, H * HD, threads);
        mm(wk, enc, kc + (size_t)(pos0 + t) * KV * HD, xn + (size_t)t * D, D, KV * HD, threads);
        mm(wv, enc, vc + (size_t)(pos0 + t) * KV * HD, xn + (size_t)t * D, D, KV * HD, threads);
        head_rmsnorm(q + (size_t)t * H * HD, H, HD, qn, eps);
        head_rmsnorm(kc + (size_t)(pos0 + t) * KV * HD, KV, HD, kn, eps);
    }
    or_rope(q, kc + (size_t)pos0 * KV * HD, T, pos0, H, KV, HD, theta);      /* :142 */
    for (int h = 0; h < H; h++) {                                            /* :144-161 */
        const int kh = h / rep;
        for (int i = 0; i < T; i++) {
            const float *qi = q + ((size_t)i * H + h) * HD;
            const int last = pos0 + i;
            for (int j = 0; j <= last; j++) {
                const float *kj = kc + ((size_t)j * KV + kh) * HD;
                float s = 0.0f;
                for (int e = 0; e < HD; e++) s += qi[e] * kj[e];
                sc[j] = s / sqrtf((float)HD);
            }
            or_softmax(sc, last + 1);
            for (int e = 0; e < HD; e++) {
                float acc = 0.0f;
                for (int j = 0; j <= last; j++) acc += sc[j] * vc[((size_t)j * KV + kh) * HD + e];
                ao[(size_t)i * H * HD + (size_t)h * HD + e] = acc;
            }
        }
    }
    for (int t = 0; t < T; t++)                                              /* :162-166 */
        mm(wo, enc, attn + (size_t)t * D, ao + (size_t)t * H * HD, H * HD, D, threads);
    free(xn); free(q); free(ao); free(sc);
}

/* ------------------------------------------------------------------ encoders */

/* binary64 -> binary16, round to nearest even, with subnormal results and overflow to
   infinity (numpy's astype(np.float16) on float64 and float32 input). */
uint16_t or_f64_to_f16(double v) {
    const uint64_t b = f64_u64(v);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const int ex = (int)((b >> 52) & 0x7FF);
    const uint64_t man = b & 0xFFFFFFFFFFFFFull;
    if (ex == 0x7FF) return (uint16_t)(sign | (man ? 0x7E00u : 0x7C00u));
    if (ex == 0) return sign;                         /* below half's range entirely */
    const int e = ex - 1023;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    const uint64_t m = (1ull << 52) | man;
    const int s = 42 + (e < -14 ? -14 - e : 0);
    if (s >= 64) return sign;
    uint64_t q = m >> s;
    const uint64_t rem = m & ((1ull << s) - 1), half = 1ull << (s - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    if (e < -14) return (uint16_t)(sign | q);          /* q <= 0x400: subnormal or min normal */
    return (uint16_t)(sign | ((((uint64_t)(e + 15)) << 10) + (q - 1024)));
}

uint16_t or_f32_to_f16(float v) { return or_f64_to_f16((double)v); }

/* format/q4.py:30-57: d = max|x|/8 in float64 rounded to fp16, q = clip(rint(x / d32),
   -8, 7) with the division in float32, nibbles packed k | (k+16) << 4. */
void or_encode_q4_0(const float *x, size_t n, uint8_t *out) {
    for (size_t g = 0; g < n / 32; g++) {
        const float *v = x + g * 32;
        uint8_t *o = out + g * 18;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) { const float a = fabsf(v[i]); if (a > amax) amax = a; }
        const double d = amax > 0.0f ? (double)amax / 8.0 : 0.0;
        const uint16_t dh = or_f64_to_f16(d);
        const float dq = or_f16_to_f32(dh);
        int q[32];
        for (int i = 0; i < 32; i++) {
            int qi = 0;
            if (dq > 0.0f) {
                float r = rintf(v[i] / dq);
                if (r < -8.0f) r = -8.0f;
                if (r > 7.0f) r = 7.0f;
                qi = (int)r;
            }
            q[i] = qi & 0xF;
        }
        o[0] = (uint8_t)(dh & 0xFF);
        o[1] = (uint8_t)(dh >> 8);
        for (int k = 0; k < 16; k++) o[2 + k] = (uint8_t)((q[k] | (q[k + 16] << 4)) & 0xFF);
    }
}

/* format/q8.py:35-58: d = fl32(max|x| / 127) rounded to fp16, q = clip(rint(x / d32),
   -127, 127), all zero when the stored scale is zero. */
void or_encode_q8_0(const float *x, size_t n, uint8_t *out) {
    for (size_t g = 0; g < n / 32; g++) {
        const float *v = x + g * 32;
        uint8_t *o = out + g * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) { const float a = fabsf(v[i]); if (a > amax) amax = a; }
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const uint16_t dh = or_f32_to_f16(d);
        const float dq = or_f16_to_f32(dh);
        o[0] = (uint8_t)(dh & 0xFF);
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; i++) {
            int qi = 0;
            if (dq > 0.0f) {
                float r = rintf(v[i] / dq);
                if (r < -127.0f) r = -127.0f;
                if (r > 127.0f) r = 127.0f;
                qi = (int)r;
            }
            o[2 + i] = (uint8_t)(int8_t)qi;
        }
    }
}

/* ------------------------------------------------------------------ bulk checks */
#include <pthread.h>

uint64_t or_exp2f_tab(int i) { return EXP2F_T[i & 31]; }

void or_expf_array(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = or_expf(x[i]);
}

typedef struct { uint64_t lo, hi; const float *y; int vs_libm; long bad; uint64_t first_bad; } ExpJob;

static int same_float(float a, float b) {
    return f32_bits(a) == f32_bits(b) || (isnan(a) && isnan(b));
}

static void *exp_job(void *arg) {
    ExpJob *j = arg;
    j->first_bad = UINT64_MAX;
    for (uint64_t u = j->lo; u < j->hi; u++) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float mine = or_expf(x);
        const float other = j->vs_libm ? expf(x) : j->y[u - j->lo];
        if (!same_float(mine, other)) { if (!j->bad) j->first_bad = u; j->bad++; }
    }
    return NULL;
}

/* Mismatches between or_expf and either the host libm expf (y == NULL) or the array y
   holding results for the bit patterns start .. start+n-1. */
long or_expf_check(uint64_t start, uint64_t n, const float *y, int threads, uint64_t *first_bad) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    ExpJob jobs[64];
    for (int i = 0; i < threads; i++) {
        jobs[i].lo = start + n * (uint64_t)i / (uint64_t)threads;
        jobs[i].hi = start + n * (uint64_t)(i + 1) / (uint64_t)threads;
        jobs[i].y = y ? y + (jobs[i].lo - start) : NULL;
        jobs[i].vs_libm = y == NULL;
        jobs[i].bad = 0;
        pthread_create(&th[i], NULL, exp_job, &jobs[i]);
    }
    long bad = 0;
    uint64_t fb = UINT64_MAX;
    for (int i = 0; i < threads; i++) {
        pthread_join(th[i], NULL);
        bad += jobs[i].bad;
        if (jobs[i].bad && jobs[i].first_bad < fb) fb = jobs[i].first_bad;
    }
    if (first_bad) *first_bad = fb;
    return bad;
}
