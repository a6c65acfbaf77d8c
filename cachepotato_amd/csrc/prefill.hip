/* prefill.hip — the expert half of the MoE layer for many tokens (a prefill chunk) as MFMA
 * grouped GEMMs on gfx950.
 *
 * Reference: engine/blocks/qwen3_moe.c:199-222 runs, for each token in turn, its 8 experts'
 * gate/up GEMVs (matmul_wx_q4 / _q8, engine/kernels/kernels.c:368-396, :514-540), SwiGLU
 * (kernels.c:416) and the down GEMV, and adds wt_j * y_j into the token's output. With
 * hundreds of tokens the same expert serves tens of them, so here each expert's tokens (the
 * groups the routing step formed) are one dense product:
 *   G = X_e Wg_e^T, U = X_e Wu_e^T, H = silu(G) * U          k_mfma_gateup
 *   Y = H Wd_e^T                                              k_mfma_down
 *   out[t] (+)= sum_j wt_j Y[t, j]  (slot order j = 0..K-1)   k_pair_combine
 *
 * Numerics. A Q4_0 / Q8_0 weight is q * d with q a small integer (Q4: -8..7, Q8: -127..127),
 * exact in f16, and d the block's fp16 scale. Each 32-wide step of k is one block: the MFMA
 * takes the exact q values as its B operand and the activations as its A operand, and the
 * step's product is scaled by d in fp32 and added to the fp32 accumulator, so no weight is
 * ever rounded. Activations are split x = hi + lo with hi = f16(x) and lo = f16(x - hi) and
 * both halves go through the MFMA (22 significant bits), so the products differ from the fp32
 * CPU GEMVs by roughly fp32 rounding, not by f16's.
 *
 * MFMA v_mfma_f32_16x16x32_f16 operand layout (checked on the device): lane l holds
 * A[l%16][8(l/16) + j] and B[8(l/16) + j][l%16] for j = 0..7, and D[4(l/16) + i][l%16] for
 * i = 0..3. A block's 32 elements map to k-slot s = element s: a Q4 lane group g takes the low
 * (g < 2) or high (g >= 2) nibbles of payload bytes 8(g%2)..8(g%2)+7, which hold elements
 * 8g..8g+7 (byte i holds elements i and i+16).
 *
 * Work decomposition. A chunk is up to 64 tokens of one expert group (an expert with 150
 * tokens is three chunks); a workgroup computes a tile of the weights for one chunk: each of
 * its wavefronts takes 16 rows and every non-empty token tile of 16 (a chunk of 20 tokens
 * costs 2 tiles, not 4); gate/up uses 8 wavefronts (128 rows) and stages of 2 blocks (64 of
 * k), down 4 wavefronts (64 rows) and stages of 1 block (PfGeo). The activations are split
 * into hi/lo f16 planes once per call (k_split_hilo for xn; the gate/up epilogue writes h
 * split), so a stage is a plain copy of the chunk's rows into LDS, shared by the
 * wavefronts. The k loop is software-pipelined: LDS is double-buffered, and both the
 * activations and each wavefront's weight blocks (read straight from the row-tiled layout,
 * 8 bytes per lane per block) are loaded two stages ahead.
 */
#include "cpg_internal.h"
#include "cpg_gemv.h"
#include "cpg_mfma.h"

#define PF_CHUNK 64         /* tokens per chunk (4 MFMA tiles of 16) */

/* A workgroup's tiling: NW wavefronts of 16 weight rows each, stages of KB blocks of 32 in
   LDS with a row stride of KS + 8 halves (16 B of padding against bank conflicts), and
   PIECES 16-byte pieces of a stage's activations per thread. Measured: the gate/up GEMM is
   fastest with 8 wavefronts and stages of 64, the down GEMM with 4 and stages of 32. */
template <int NW_, int KB_> struct PfGeo {
    static constexpr int NW = NW_, NT = NW_ * 64, ROWS = NW_ * 16, KB = KB_, KS = KB_ * 32,
                         LDA = KB_ * 32 + 8, PIECES = PF_CHUNK * (KB_ * 32 / 8) / (NW_ * 64);
    static_assert(PIECES >= 1 && PF_CHUNK * (KB_ * 32 / 8) % (NW_ * 64) == 0, "stage pieces");
};
typedef PfGeo<8, 2> PfGateup;
typedef PfGeo<4, 1> PfDown;

/* ---------------------------------------------------------------- chunk list */

/* One workgroup: chunks (group g, first token m0) of at most PF_CHUNK tokens over the groups
   the routing step formed (grp_cnt[g] > 0), in group order; slots up to max_chunks without a
   chunk get group -1. */
__global__ __launch_bounds__(256) void k_chunks(const int *__restrict__ grp_cnt, int E,
                                                int max_chunks, int *__restrict__ chunk_grp,
                                                int *__restrict__ chunk_m0) {
    __shared__ int base[1024];
    const int tid = threadIdx.x;
    if (tid == 0) {
        int c = 0;
        for (int g = 0; g < E; g++) {
            base[g] = c;
            c += (grp_cnt[g] + PF_CHUNK - 1) / PF_CHUNK;
        }
        base[E] = c;
    }
    __syncthreads();
    const int total = min(base[E], max_chunks);
    for (int i = tid; i < max_chunks; i += 256) chunk_grp[i] = -1;
    __syncthreads();
    for (int g = tid; g < E; g += 256) {
        const int n = (grp_cnt[g] + PF_CHUNK - 1) / PF_CHUNK;
        for (int c = 0; c < n; c++) {
            const int idx = base[g] + c;
            if (idx < total) {
                chunk_grp[idx] = g;
                chunk_m0[idx] = c * PF_CHUNK;
            }
        }
    }
}

/* grid rows, 256 threads: hi[r] = f16(x[r]), lo[r] = f16(x[r] - hi[r]) for rows of n floats
   (n % 8 == 0) */
__global__ __launch_bounds__(256) void k_split_hilo(const float *__restrict__ x, int n,
                                                    _Float16 *__restrict__ hi,
                                                    _Float16 *__restrict__ lo) {
    const size_t r = blockIdx.x;
    for (int c = threadIdx.x; c < n / 8; c += 256) {
        const float4 v0 = *(const float4 *)(x + r * n + 8 * c);
        const float4 v1 = *(const float4 *)(x + r * n + 8 * c + 4);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        half8_t h, l;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            h[j] = (_Float16)v[j];
            l[j] = (_Float16)(v[j] - (float)h[j]);
        }
        *(half8_t *)(hi + r * n + 8 * c) = h;
        *(half8_t *)(lo + r * n + 8 * c) = l;
    }
}

/* One stage of activations: G::KS halves of each of the chunk's 64 rows, hi and lo, as
   16-byte pieces; thread tid moves pieces tid, tid + G::NT, ... (G::PIECES each of hi and
   lo). */
template <class G> struct AStage {
    half8_t h[G::PIECES], l[G::PIECES];
};

template <class G, typename Row>
__device__ static inline void stage_load(AStage<G> &a, int m, int k0, Row row_of,
                                         const _Float16 *__restrict__ hi,
                                         const _Float16 *__restrict__ lo, size_t ld) {
    /* unconditional loads (a load under a branch makes the compiler wait for every load in
       flight where the branches join): rows past m repeat row m-1, whose MFMA output rows
       are never stored (an MFMA output row depends on its own A row only) */
#pragma unroll
    for (int p = 0; p < G::PIECES; p++) {
        const int idx = threadIdx.x + G::NT * p, i = idx / (G::KS / 8), c = idx % (G::KS / 8);
        const size_t off = (size_t)row_of(min(i, m - 1)) * ld + k0 + 8 * c;
        a.h[p] = *(const half8_t *)(hi + off);
        a.l[p] = *(const half8_t *)(lo + off);
    }
}

template <class G>
__device__ static inline void stage_store(const AStage<G> &a, _Float16 *ah, _Float16 *al) {
#pragma unroll
    for (int p = 0; p < G::PIECES; p++) {
        const int idx = threadIdx.x + G::NT * p, i = idx / (G::KS / 8), c = idx % (G::KS / 8);
        *(half8_t *)(ah + i * G::LDA + 8 * c) = a.h[p];
        *(half8_t *)(al + i * G::LDA + 8 * c) = a.l[p];
    }
}

/* One block (index kb of the LDS stage) for NMT token tiles and NB weight operands b[n]
   with scales d[n]: acc[n][mt] += d[n] * (A_hi + A_lo)[mt] . b[n]. All A fragments are read
   first and the 2 * NMT * NB MFMAs are independent chains, so they issue back to back. */
template <class G, int NMT, int NB>
__device__ static inline void mma_block(const _Float16 *ah, const _Float16 *al, int kb,
                                        const half8_t *b, const float *d,
                                        f32x4_t (*acc)[PF_CHUNK / 16]) {
    const int l = threadIdx.x & 63;
    half8_t a_hi[NMT], a_lo[NMT];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++) {
        const int off = (mt * 16 + (l & 15)) * G::LDA + kb * 32 + 8 * (l >> 4);
        a_hi[mt] = *(const half8_t *)(ah + off);
        a_lo[mt] = *(const half8_t *)(al + off);
    }
    f32x4_t t[NB][NMT];
#pragma unroll
    for (int n = 0; n < NB; n++)
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
            t[n][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi[mt], b[n], z, 0, 0, 0);
        }
#pragma unroll
    for (int n = 0; n < NB; n++)
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
            t[n][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo[mt], b[n], t[n][mt], 0, 0, 0);
#pragma unroll
    for (int n = 0; n < NB; n++)
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[n][mt][i] = fmaf(d[n], t[n][mt][i], acc[n][mt][i]);
}

/* The k loop shared by both GEMMs: NB weight matrices (2: gate and up, 1: down) with rows
   `row` of M[n] (nb blocks per row), S stages of G::KB blocks from block b0; the A operand rows come from planes hi/lo (row
   stride ld) through row_of(i). Software pipeline: LDS double-buffered, next stage's
   activations loaded during the current stage's MFMAs, weights two stages ahead in three
   register sets named per stage of a 3-way unrolled loop (no register copies of loads in
   flight, which would make the compiler wait for them). */
template <int ENC, class G, int NMT, int NB, typename Row>
__device__ static inline void gemm_k_loop(const uint8_t *const *M, size_t payload_plane, int row,
                                          int nb, int g, int S, int m, Row row_of,
                                          const _Float16 *__restrict__ hi,
                                          const _Float16 *__restrict__ lo, size_t ld,
                                          _Float16 (*ah)[PF_CHUNK * G::LDA],
                                          _Float16 (*al)[PF_CHUNK * G::LDA],
                                          f32x4_t (*acc)[PF_CHUNK / 16], int b0 = 0) {
    WRaw w0[NB][G::KB], w1[NB][G::KB], w2[NB][G::KB];
    auto wload = [&](WRaw (&wr)[NB][G::KB], int st) {
        st = min(st, S - 1);                     /* past the end: a valid block, unused */
#pragma unroll
        for (int n = 0; n < NB; n++)
#pragma unroll
            for (int kb = 0; kb < G::KB; kb++)
                wr[n][kb] = weight_raw<ENC>(M[n], payload_plane, row, b0 + st * G::KB + kb, nb,
                                            g);
    };
    wload(w0, 0);
    wload(w1, 1);
    /* activations two stages ahead as well, in three register sets named per stage of the
       same unrolled loop: stage s loads stage s+2 and stores stage s+1 (loaded one stage
       earlier) into the other LDS buffer */
    AStage<G> a0, a1, a2;
    stage_load(a0, m, 0, row_of, hi, lo, ld);
    stage_load(a1, m, min(1, S - 1) * G::KS, row_of, hi, lo, ld);
    stage_store(a0, ah[0], al[0]);
    __syncthreads();
    auto stage = [&](int s, WRaw (&wc)[NB][G::KB], WRaw (&wn)[NB][G::KB], AStage<G> &anext,
                     AStage<G> &astore) {
        stage_load(anext, m, min(s + 2, S - 1) * G::KS, row_of, hi, lo, ld);
        wload(wn, s + 2);
#pragma unroll
        for (int kb = 0; kb < G::KB; kb++) {
            half8_t b[NB];
            float d[NB];
#pragma unroll
            for (int n = 0; n < NB; n++) {
                b[n] = weight_half8<ENC>(wc[n][kb], g);
                d[n] = scale_f32(wc[n][kb].d);
            }
            mma_block<G, NMT, NB>(ah[s & 1], al[s & 1], kb, b, d, acc);
        }
        if (s + 1 < S) stage_store(astore, ah[(s + 1) & 1], al[(s + 1) & 1]);
        __syncthreads();
    };
    for (int s = 0; s < S; s += 3) {
        stage(s, w0, w2, a2, a1);
        if (s + 1 < S) stage(s + 1, w1, w0, a0, a2);
        if (s + 2 < S) stage(s + 2, w2, w1, a1, a0);
    }
}

/* ---------------------------------------------------------------- gate / up */

/* grid (F/PfGateup::ROWS, max_chunks), PfGateup::NT threads. Chunk c = (group g, tokens m0..m0+m-1) of
   expert e; rows n0..n0+PfGateup::ROWS-1 of Wg and Wu over xh/xl (the hi/lo planes of xn, one row per token).
   h = silu(g) * u (kernels.c:416) for the chunk's tokens, written as hi/lo f16 rows hh/hl at
   the token's position in the group list (off + m0 + i), the A operand of k_mfma_down. */
template <int ENC>
__global__ __launch_bounds__(PfGateup::NT) void k_mfma_gateup(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat_bytes, size_t payload_plane,
    int D, int F, const int *__restrict__ chunk_grp, const int *__restrict__ chunk_m0,
    const int *__restrict__ grp_expert, const int *__restrict__ grp_off,
    const int *__restrict__ grp_cnt, const int *__restrict__ list_tok,
    const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl,
    _Float16 *__restrict__ hh, _Float16 *__restrict__ hl) {
    __shared__ __align__(16) _Float16 ah[2][PF_CHUNK * PfGateup::LDA], al[2][PF_CHUNK * PfGateup::LDA];
    __shared__ int tok[PF_CHUNK];
    __shared__ uint64_t tab[32];
    const int c = blockIdx.y, grp = chunk_grp[c];
    if (grp < 0) return;
    const int e = grp_expert[grp], off = grp_off[grp], m0 = chunk_m0[c];
    const int m = min(PF_CHUNK, grp_cnt[grp] - m0), nmt = (m + 15) / 16;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4;
    const int row = blockIdx.x * PfGateup::ROWS + w * 16 + (l & 15);
    const int nb = D / 32, S = D / PfGateup::KS;
    const uint8_t *Mg = experts + (size_t)e * exp_stride, *Mu = Mg + mat_bytes;
    if (tid < PF_CHUNK) tok[tid] = tid < m ? list_tok[off + m0 + tid] : 0;
    if (tid < 32) tab[tid] = cpg_exp2f_tab[tid];
    f32x4_t acc[2][PF_CHUNK / 16];
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int mt = 0; mt < PF_CHUNK / 16; mt++)
            for (int i = 0; i < 4; i++) acc[n][mt][i] = 0.0f;
    __syncthreads();
    auto row_of = [&](int i) { return tok[i]; };
    const uint8_t *M[2] = {Mg, Mu};
    switch (nmt) {
    case 1: gemm_k_loop<ENC, PfGateup, 1, 2>(M, payload_plane, row, nb, g, S, m, row_of, xh, xl, (size_t)D, ah, al, acc); break;
    case 2: gemm_k_loop<ENC, PfGateup, 2, 2>(M, payload_plane, row, nb, g, S, m, row_of, xh, xl, (size_t)D, ah, al, acc); break;
    case 3: gemm_k_loop<ENC, PfGateup, 3, 2>(M, payload_plane, row, nb, g, S, m, row_of, xh, xl, (size_t)D, ah, al, acc); break;
    default: gemm_k_loop<ENC, PfGateup, 4, 2>(M, payload_plane, row, nb, g, S, m, row_of, xh, xl, (size_t)D, ah, al, acc); break;
    }
    f32x4_t *accg = acc[0], *accu = acc[1];
#pragma unroll
    for (int mt = 0; mt < PF_CHUNK / 16; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = mt * 16 + 4 * g + i;
            if (r < m) {
                const float hv = swiglu_t(accg[mt][i], accu[mt][i], tab);
                const _Float16 h16 = (_Float16)hv;
                const size_t o = (size_t)(off + m0 + r) * F + row;
                hh[o] = h16;
                hl[o] = (_Float16)(hv - (float)h16);
            }
        }
}

/* ---------------------------------------------------------------- down */

/* grid (D/PfDown::ROWS, max_chunks), PfDown::NT threads: y[pair] (rows n0..n0+PfDown::ROWS-1) = Wd_e . h for the chunk's
   tokens, h from the hi/lo planes hh/hl at the group-list positions; pair = list_pair of the
   position. */
template <int ENC>
__global__ __launch_bounds__(PfDown::NT) void k_mfma_down(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t wd_off, size_t payload_plane,
    int D, int F, const int *__restrict__ chunk_grp, const int *__restrict__ chunk_m0,
    const int *__restrict__ grp_expert, const int *__restrict__ grp_off,
    const int *__restrict__ grp_cnt, const int *__restrict__ list_pair,
    const _Float16 *__restrict__ hh, const _Float16 *__restrict__ hl, float *__restrict__ y) {
    __shared__ __align__(16) _Float16 ah[2][PF_CHUNK * PfDown::LDA], al[2][PF_CHUNK * PfDown::LDA];
    __shared__ int pair[PF_CHUNK];
    const int c = blockIdx.y, grp = chunk_grp[c];
    if (grp < 0) return;
    const int e = grp_expert[grp], off = grp_off[grp], m0 = chunk_m0[c];
    const int m = min(PF_CHUNK, grp_cnt[grp] - m0), nmt = (m + 15) / 16;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4;
    const int row = blockIdx.x * PfDown::ROWS + w * 16 + (l & 15);
    const int nb = F / 32, S = F / PfDown::KS;
    const uint8_t *Md = experts + (size_t)e * exp_stride + wd_off;
    if (tid < PF_CHUNK) pair[tid] = tid < m ? list_pair[off + m0 + tid] : 0;
    f32x4_t accd[1][PF_CHUNK / 16];
#pragma unroll
    for (int mt = 0; mt < PF_CHUNK / 16; mt++)
        for (int i = 0; i < 4; i++) accd[0][mt][i] = 0.0f;
    auto row_of = [&](int i) { return off + m0 + i; };
    const uint8_t *M[1] = {Md};
    switch (nmt) {
    case 1: gemm_k_loop<ENC, PfDown, 1, 1>(M, payload_plane, row, nb, g, S, m, row_of, hh, hl, (size_t)F, ah, al, accd); break;
    case 2: gemm_k_loop<ENC, PfDown, 2, 1>(M, payload_plane, row, nb, g, S, m, row_of, hh, hl, (size_t)F, ah, al, accd); break;
    case 3: gemm_k_loop<ENC, PfDown, 3, 1>(M, payload_plane, row, nb, g, S, m, row_of, hh, hl, (size_t)F, ah, al, accd); break;
    default: gemm_k_loop<ENC, PfDown, 4, 1>(M, payload_plane, row, nb, g, S, m, row_of, hh, hl, (size_t)F, ah, al, accd); break;
    }
    f32x4_t *acc = accd[0];
#pragma unroll
    for (int mt = 0; mt < PF_CHUNK / 16; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = mt * 16 + 4 * g + i;
            if (r < m) y[(size_t)pair[r] * D + row] = acc[mt][i];
        }
}

/* ---------------------------------------------------------------- dense */

/* grid (n_out/PfDown::ROWS, ceil(T/PF_CHUNK), ks), PfDown::NT threads: one row-tiled matrix W
   (n_out rows of n_in) times the tokens m0..m0+m-1 (m0 = blockIdx.y * PF_CHUNK) of the hi/lo
   planes xh/xl (T rows of n_in), over the nbs blocks of 32 from b0 = blockIdx.z * nbs; written
   to out[(blockIdx.z * T + t) * n_out + row], one part per blockIdx.z. */
template <int ENC>
__global__ __launch_bounds__(PfDown::NT) void k_mfma_dense(
    const uint8_t *__restrict__ W, size_t payload_plane, int n_in, int n_out, int T, int nbs,
    const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl, float *__restrict__ out) {
    __shared__ __align__(16) _Float16 ah[2][PF_CHUNK * PfDown::LDA], al[2][PF_CHUNK * PfDown::LDA];
    const int m0 = blockIdx.y * PF_CHUNK, m = min(PF_CHUNK, T - m0), nmt = (m + 15) / 16;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4;
    const int row = blockIdx.x * PfDown::ROWS + w * 16 + (l & 15);
    const int b0 = blockIdx.z * nbs, S = nbs / PfDown::KB, nb = n_in / 32;
    f32x4_t acc[1][PF_CHUNK / 16];
#pragma unroll
    for (int mt = 0; mt < PF_CHUNK / 16; mt++)
        for (int i = 0; i < 4; i++) acc[0][mt][i] = 0.0f;
    auto row_of = [&](int i) { return m0 + i; };
    const uint8_t *M[1] = {W};
    /* the activation planes from block b0 on: stage k0 offsets then count from there */
    const _Float16 *hi = xh + (size_t)b0 * 32, *lo = xl + (size_t)b0 * 32;
    switch (nmt) {
    case 1: gemm_k_loop<ENC, PfDown, 1, 1>(M, payload_plane, row, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    case 2: gemm_k_loop<ENC, PfDown, 2, 1>(M, payload_plane, row, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    case 3: gemm_k_loop<ENC, PfDown, 3, 1>(M, payload_plane, row, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    default: gemm_k_loop<ENC, PfDown, 4, 1>(M, payload_plane, row, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    }
    float *o = out + ((size_t)blockIdx.z * T + m0) * n_out + row;
#pragma unroll
    for (int mt = 0; mt < PF_CHUNK / 16; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = mt * 16 + 4 * g + i;
            if (r < m) o[(size_t)r * n_out] = acc[0][mt][i];
        }
}

/* grid ceil(n/256), 256 threads: out[i] = ((part[0][i] + part[1][i]) + part[2][i]) + ...,
   ks parts of n floats, in part order */
__global__ __launch_bounds__(256) void k_sum_parts(const float *__restrict__ part, int ks,
                                                   size_t n, float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float a = part[i];
    for (int z = 1; z < ks; z++) a = __fadd_rn(a, part[(size_t)z * n + i]);
    out[i] = a;
}

/* ---------------------------------------------------------------- combine */

/* grid (D/256, T), 256 threads: o = mlp[t][d] + sum_j wt[t][j] * y[t*K + j][d] in slot order
   (qwen3_moe.c:221); written to mlp, or with xres: xres[t][d] += attn[t][d] + o and mlp
   untouched (mlp must then be zero, the reference's calloc'ed start, cachepotato.c:157-159). */
__global__ __launch_bounds__(256) void k_pair_combine(const float *__restrict__ y,
                                                      const float *__restrict__ wt, int D, int K,
                                                      float *__restrict__ mlp,
                                                      float *__restrict__ xres,
                                                      const float *__restrict__ attn) {
    const int t = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D) return;
    const size_t o = (size_t)t * D + d;
    float acc = xres ? 0.0f : mlp[o];
    for (int j = 0; j < K; j++)
        acc = __fadd_rn(acc, __fmul_rn(wt[(size_t)t * K + j], y[((size_t)t * K + j) * D + d]));
    if (xres) xres[o] = __fadd_rn(xres[o], __fadd_rn(attn[o], acc));
    else mlp[o] = acc;
}

/* ---------------------------------------------------------------- host */

/* the most chunks T tokens with K experts each over E experts can form */
int cpg_prefill_max_chunks(int T, int K, int E) {
    const int pairs = T * K;
    const int groups = pairs < E ? pairs : E;
    return (pairs + PF_CHUNK - 1) / PF_CHUNK + groups;
}

bool cpg_prefill_shape_ok(int D, int F) {
    return D % PfGateup::KS == 0 && F % PfDown::KS == 0 && F % PfGateup::ROWS == 0 &&
           D % PfDown::ROWS == 0;
}

template <int ENC>
static int prefill_experts(const cpg_moe_layer *L, int T, const float *xn, const float *wt,
                           const int *grp_expert, const int *grp_off, const int *grp_cnt,
                           const int *list_tok, const int *list_pair, int *chunk_grp,
                           int *chunk_m0, void *scratch, float *y, float *mlp, float *xres,
                           const float *attn) {
    const int D = L->D, F = L->F, E = L->E, K = L->K;
    const int mc = cpg_prefill_max_chunks(T, K, E);
    _Float16 *xh = (_Float16 *)scratch, *xl = xh + (size_t)T * D;
    _Float16 *hh = xl + (size_t)T * D, *hl = hh + (size_t)T * K * F;
    LAUNCH(CPG_KT_SELECT, k_chunks, dim3(1), dim3(256), 0, grp_cnt, E, mc, chunk_grp, chunk_m0);
    LAUNCH(CPG_KT_SELECT, k_split_hilo, dim3(T), dim3(256), 0, xn, D, xh, xl);
    const uint8_t *ex = (const uint8_t *)L->experts;
    const size_t es = cpg_expert_bytes(ENC, D, F), mg = cpg_matrix_bytes(ENC, F, D);
    LAUNCH(CPG_KT_GATEUP, k_mfma_gateup<ENC>, dim3(F / PfGateup::ROWS, mc), dim3(PfGateup::NT), 0,
           ex, es, mg,
           cpg_payload_plane(ENC, F, D), D, F, chunk_grp, chunk_m0, grp_expert, grp_off, grp_cnt,
           list_tok, xh, xl, hh, hl);
    LAUNCH(CPG_KT_DOWN, k_mfma_down<ENC>, dim3(D / PfDown::ROWS, mc), dim3(PfDown::NT), 0, ex, es,
           2 * mg,
           cpg_payload_plane(ENC, D, F), D, F, chunk_grp, chunk_m0, grp_expert, grp_off, grp_cnt,
           list_pair, hh, hl, y);
    LAUNCH(CPG_KT_COMBINE, k_pair_combine, dim3((D + 255) / 256, T), dim3(256), 0, y, wt, D, K,
           mlp, xres, attn);
    return 0;
}

/* split of the k range of a dense product over T tokens: halved while every part keeps at
   least 8 blocks of 32 and the grid stays within 1024 workgroups (four per CU) */
static int dense_ksplit(int T, int n_in, int n_out) {
    const int nb = n_in / 32, base = n_out / PfDown::ROWS * ((T + PF_CHUNK - 1) / PF_CHUNK);
    int ks = 1;
    while (ks < 16 && nb % (2 * ks) == 0 && nb / (2 * ks) >= 8 && base * 2 * ks <= 1024) ks *= 2;
    return ks;
}

bool cpg_dense_shape_ok(int n_in, int n_out) {
    return n_in > 0 && n_out > 0 && n_in % PfDown::KS == 0 && n_out % PfDown::ROWS == 0;
}

size_t cpg_dense_scratch_bytes(int T, int n_in, int n_out) {
    const int ks = dense_ksplit(T, n_in, n_out);
    return cpg_round256((size_t)4 * T * n_in) + (ks > 1 ? (size_t)4 * ks * T * n_out : 0);
}

template <int ENC>
static int dense_mfma(const void *w, int n_in, int n_out, const float *x, int T, void *scratch,
                      float *out) {
    const int ks = dense_ksplit(T, n_in, n_out);
    _Float16 *xh = (_Float16 *)scratch, *xl = xh + (size_t)T * n_in;
    float *part = ks > 1 ? (float *)((uint8_t *)scratch + cpg_round256((size_t)4 * T * n_in))
                         : out;
    hipStream_t s = g_cpg.stream;
    hipLaunchKernelGGL(k_split_hilo, dim3(T), dim3(256), 0, s, x, n_in, xh, xl);
    CPG_LAUNCH_CHECK("k_split_hilo");
    hipLaunchKernelGGL(k_mfma_dense<ENC>, dim3(n_out / PfDown::ROWS, (T + PF_CHUNK - 1) / PF_CHUNK, ks),
                       dim3(PfDown::NT), 0, s, (const uint8_t *)w,
                       cpg_payload_plane(ENC, n_out, n_in), n_in, n_out, T, n_in / 32 / ks, xh,
                       xl, part);
    CPG_LAUNCH_CHECK("k_mfma_dense");
    if (ks > 1) {
        const size_t n = (size_t)T * n_out;
        hipLaunchKernelGGL(k_sum_parts, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part,
                           ks, n, out);
        CPG_LAUNCH_CHECK("k_sum_parts");
    }
    return 0;
}

int cpg_dense_mfma(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                   void *scratch, float *out) {
    if (!w || !x || !scratch || !out || T <= 0 || !cpg_dense_shape_ok(n_in, n_out)) {
        cpg_set_error("cpg_dense_mfma: bad arguments (n_in %d, n_out %d, T %d)", n_in, n_out, T);
        return -1;
    }
    if (enc == CPG_ENC_Q4) return dense_mfma<CPG_ENC_Q4>(w, n_in, n_out, x, T, scratch, out);
    if (enc == CPG_ENC_Q8) return dense_mfma<CPG_ENC_Q8>(w, n_in, n_out, x, T, scratch, out);
    cpg_set_error("cpg_dense_mfma: encoding %d is not row-tiled (Q4_0 or Q8_0 only)", enc);
    return -1;
}

size_t cpg_prefill_scratch_bytes(int T, int D, int K, int F) {
    return (size_t)2 * 2 * ((size_t)T * D + (size_t)T * K * F);
}

int cpg_prefill_experts(const cpg_moe_layer *L, int T, const float *xn, const float *wt,
                        const int *grp_expert, const int *grp_off, const int *grp_cnt,
                        const int *list_tok, const int *list_pair, int *chunk_grp,
                        int *chunk_m0, void *scratch, float *y, float *mlp, float *xres,
                        const float *attn) {
    if (L->enc == CPG_ENC_Q4)
        return prefill_experts<CPG_ENC_Q4>(L, T, xn, wt, grp_expert, grp_off, grp_cnt, list_tok,
                                           list_pair, chunk_grp, chunk_m0, scratch, y, mlp, xres,
                                           attn);
    return prefill_experts<CPG_ENC_Q8>(L, T, xn, wt, grp_expert, grp_off, grp_cnt, list_tok,
                                       list_pair, chunk_grp, chunk_m0, scratch, y, mlp, xres, attn);
}
