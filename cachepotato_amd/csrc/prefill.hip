/* prefill.hip — the expert half of the MoE layer for many tokens (a prefill chunk) as MFMA
 * grouped GEMMs on gfx950.
 *
 * Reference: engine/blocks/qwen3_moe.c:199-222 runs, for each token in turn, its 8 experts'
 * gate/up GEMVs (matmul_wx_q4 / _q8, engine/kernels/kernels.c:368-396, :514-540), SwiGLU
 * (kernels.c:416) and the down GEMV, and adds wt_j * y_j into the token's output. With
 * hundreds of tokens the same expert serves tens of them, so here each expert's tokens (the
 * groups the routing step formed) are one dense product:
 *   G = X_e Wg_e^T, U = X_e Wu_e^T, H = silu(G) * U          k_pf_gemm<ENC, true>
 *   Y = H Wd_e^T                                              k_pf_gemm<ENC, false>
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
 * tokens is three chunks); a workgroup of 4 wavefronts computes 128 rows of each of its
 * matrices for one chunk (gate/up: 128 rows of Wg and the same rows of Wu, so SwiGLU pairs
 * are in one lane; down: 128 rows of Wd), each wavefront 32 rows for every non-empty token
 * tile of 16 (a chunk of 20 tokens costs 2 tiles, not 4). Batches of at most 16 tokens (one
 * token tile per chunk) use a variant with 64 gate/up rows per workgroup and a ring of four
 * stages: there the VALU weight conversion, not the MFMAs, sets each wavefront's pace, and
 * twice the workgroups spread it over the CUs. The activations are split into
 * hi/lo f16 planes once per call (k_split_hilo for xn; the gate/up epilogue writes h split).
 * Both operands reach the MFMAs through a ring of stages in LDS filled by direct
 * global-to-LDS loads (k_pf_gemm); the dense projections keep a register-staged k loop
 * (gemm_k_loop).
 */
#include "cpg_internal.h"
#include "cpg_gemv.h"
#include "cpg_mfma.h"

/* The dense GEMM's tiling (gemm_k_loop): NW wavefronts of RW weight rows each, stages of KB
   blocks of 32 in LDS with a row stride of KS + 8 halves (16 B of padding against bank
   conflicts), and PIECES 16-byte pieces of a stage's activations per thread. */
template <int NW_, int KB_, int RW_ = 16> struct PfGeo {
    static constexpr int NW = NW_, NT = NW_ * 64, RW = RW_, ROWS = NW_ * RW_, KB = KB_,
                         KS = KB_ * 32, LDA = KB_ * 32 + 8,
                         PIECES = PF_CHUNK * (KB_ * 32 / 8) / (NW_ * 64);
    static_assert(PIECES >= 1 && PF_CHUNK * (KB_ * 32 / 8) % (NW_ * 64) == 0, "stage pieces");
    static_assert(RW_ % 16 == 0, "whole B tiles");
};
typedef PfGeo<4, 1> PfDown;

/* ---------------------------------------------------------------- chunk list */

/* One wavefront: the chunk list over the groups the routing step formed (pf_chunk_list), for
   routing steps that do not form it themselves; lane t takes groups 4t..4t+3 (E <= 256). */
__global__ __launch_bounds__(64) void k_chunks(const int *__restrict__ grp_cnt, int E,
                                               int max_chunks, int *__restrict__ chunk_grp,
                                               int *__restrict__ chunk_m0) {
    int cnt[4], grp[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        grp[j] = 4 * threadIdx.x + j;
        cnt[j] = grp[j] < E ? grp_cnt[grp[j]] : 0;
    }
    pf_chunk_list(cnt, grp, max_chunks, chunk_grp, chunk_m0);
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
            const f16pair p = split_f16(v[j]);
            h[j] = p.hi;
            l[j] = p.lo;
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
   with scales d[n]: acc[n][mt] += d[n] * (A_hi + A_lo)[mt] . b[n]. The A fragments are read
   once and feed every B operand; for each n the NMT hi products are independent chains that
   issue back to back, then the lo products accumulate onto them. */
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
#pragma unroll
    for (int n = 0; n < NB; n++) {
        f32x4_t t[NMT];
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
            t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi[mt], b[n], z, 0, 0, 0);
        }
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
            t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo[mt], b[n], t[mt], 0, 0, 0);
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[n][mt][i] = fmaf(d[n], t[mt][i], acc[n][mt][i]);
    }
}

/* The k loop shared by the GEMMs: NB B operands, operand n being 16 rows of matrix M[n]
   (this lane's row rows[n], nb blocks per row), S stages of G::KB blocks from block b0; the
   A operand rows come from planes hi/lo (row stride ld) through row_of(i). Software
   pipeline: LDS double-buffered, next stage's activations loaded during the current stage's
   MFMAs, weights two stages ahead in three register sets named per stage of a 3-way unrolled
   loop (no register copies of loads in flight, which would make the compiler wait for
   them). */
template <int ENC, class G, int NMT, int NB, typename Row>
__device__ static inline void gemm_k_loop(const uint8_t *const *M, size_t payload_plane,
                                          const int (&rows)[NB], int nb, int g, int S, int m,
                                          Row row_of, const _Float16 *__restrict__ hi,
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
                wr[n][kb] = weight_raw<ENC>(M[n], payload_plane, rows[n], b0 + st * G::KB + kb,
                                            nb, g);
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

/* ---------------------------------------------------------------- expert GEMMs */

/* The expert GEMMs stream both operands through a ring of P stages in LDS, filled by direct
   global-to-LDS loads (global_load_lds_dwordx4: 16 bytes per lane, a wavefront's 64 lanes
   into 1 KiB of consecutive LDS), so loads in flight hold no registers and a stage is never
   copied through them. A stage is one block of 32 of the k range:
     A hi, A lo   the chunk's 64 activation rows, 32 halves each (a 64-byte row per token;
                  a wavefront's 1 KiB is 16 rows), rows past the chunk repeating its last;
                  16-byte piece c of row r sits at piece c ^ ((r >> 2) & 3) of its row, so
                  the 16 rows one MFMA operand read touches fall in distinct LDS banks (rows
                  64 bytes apart would put rows r and r + 4 in the same banks);
     W            NSEG 64-row segments of weight payload (the row-tiled layout keeps a
                  segment's block contiguous: 64 * PB bytes);
     Sc           their fp16 scales, 128 bytes per segment.
   Every wavefront issues the same number Q of loads per stage, so "stage s has landed" is
   vmcnt <= Q * (P - 2) for each wavefront, followed by a barrier for the others' loads. The
   barrier is s_barrier alone: __syncthreads() would wait for every load in flight. The
   workgroup (4 wavefronts) computes 128 rows of each of its matrices for the chunk; a
   wavefront 32 rows of each (GU: gate rows, up rows: four 16-row B tiles; down: two). */
#define PF_NT 256
/* batches of at most 16 tokens: ring depth, rows of each matrix per workgroup (gate/up,
   down), blocks per stage; measured at 16 tokens (gate/up, down us): 128 rows in rings of 4
   38.4, 16.6; 64 rows 29.3, 20.1; 64 rows in rings of 6 30.9, 22.4; stages of 4 blocks in
   rings of 3 28.3 (gate/up, against 28.0 with stages of 2), in rings of 4 32.7 */
#define PF_SMALL_RING 4
#define PF_SMALL_RW_GU 64
#define PF_SMALL_RW_DN 128
#define PF_SMALL_KB 2
#define R_Q_FITS(q, p) ((q) * ((p) - 2) < 64)   /* the stage wait's vmcnt fits its field */

template <int ENC, bool GU, int TT_ = PF_CHUNK / 16, int P_ = 2, int RW_ = 128, int KB_ = 2>
struct PfRing {
    static constexpr int ENCODING = ENC;
    static constexpr bool GATE_UP = GU;
    static constexpr int TT = TT_;                            /* token tiles of 16 at most */
    static constexpr int KB = KB_;                            /* blocks of 32 per stage */
    static constexpr int PB = ENC == CPG_ENC_Q4 ? 16 : 32;   /* payload bytes per row-block */
    static constexpr int RW = RW_;                            /* rows of each matrix */
    static constexpr int TPM = RW / 64;                       /* B tiles per matrix per wave */
    static constexpr int NSEG = GU ? 2 * TPM : TPM;           /* 64-row weight segments */
    static constexpr int NBT = NSEG;                          /* B tiles per wavefront */
    static constexpr int PP = 4 * KB;                         /* 16-byte pieces per A row */
    static constexpr int A_BYTES = TT * 16 * 32 * KB * 2;     /* one activation plane */
    static constexpr int W_BYTES = NSEG * KB * 64 * PB;
    static constexpr int S_BYTES = NSEG * KB * 128;
    static constexpr int STAGE = 2 * A_BYTES + W_BYTES + S_BYTES;
    static constexpr int WB = W_BYTES / 4;                    /* weight bytes per wavefront */
    static constexpr int WI = (WB + 1023) / 1024;             /* their loads */
    static constexpr int SB = S_BYTES / 4;                    /* scale bytes per wavefront */
    static constexpr int Q = 2 * KB + WI + 1;                 /* loads per stage per wavefront */
    /* ring depth: chunks of up to 64 tokens (TT = 4) use 2, the next stage loading while
       this one is computed. Stages of two blocks with two slots (37-52 KiB) let three
       workgroups share a CU (the register limit) and halve the barriers of one-block stages;
       measured: gate/up 134 us with one-block stages in three slots, 144 with two-block
       stages in three slots (two workgroups per CU), 125 with two in two; deeper rings were
       slower still, as fewer workgroups then hide each other's barriers and LDS latency.
       Chunks of one token tile (batches of up to 16 tokens) compute little per stage and
       wait for its loads: their ring is deeper (pf_small_ring). */
    static constexpr int P = P_;
    static_assert((RW == 64 || RW == 128) && P >= 2 && WB % 16 == 0 && SB % 16 == 0 && SB <= 1024 && PP <= 16 &&
                      TT >= 1 && TT <= PF_CHUNK / 16 && R_Q_FITS(2 * KB + WI + 1, P),
                  "ring geometry");
    /* the position of logical piece c of A row r: rows 16 * 4 / PP apart share banks, so the
       16 rows of an MFMA operand read land in distinct banks */
    __device__ static int apos(int r, int c) { return c ^ ((r / (16 / PP)) % PP); }
};

/* One global_load_lds_dwordx4: 16 bytes from src per lane into LDS at lds_dst + 16 * lane
   (lds_dst the same for the whole wavefront). Written as inline asm: the compiler, which
   cannot tell the ring's slots apart, would otherwise wait for every such load in flight
   before each LDS read. The waits are the caller's (wait_vm_lgkm), and the memory clobber
   keeps the compiler's own LDS accesses on their side of it. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"     /* m0 is written on purpose */
__device__ static inline void lds_dma16(const void *src, const void *lds_dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const void __attribute__((address_space(3))) *)lds_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

/* s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding; expcnt left at its maximum) */
template <int N> __device__ static inline void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

/* One lane's B operand of one block as exact f16 integers q, in natural k order: the nibble
   mask (Q4, after a shift to the lane group's nibbles) or nothing (Q8) leaves each byte u, a
   byte permute puts bytes 2i, 2i+1 under 0x64 (the f16 1024 + u), and the bias 1024 + 8 (Q4)
   or 1024 + 128 (Q8) is subtracted exactly: 12 instructions for Q4's 8 weights. */
template <int ENC>
__device__ static inline half8_t weight_q(uint2 pw, int g) {
    uint32_t src[2] = {pw.x, pw.y};
    if (ENC == CPG_ENC_Q4) {
        const int sh = (g >> 1) * 4;
        src[0] = (src[0] >> sh) & 0x0F0F0F0Fu;
        src[1] = (src[1] >> sh) & 0x0F0F0F0Fu;
    }
    const _Float16 bias = ENC == CPG_ENC_Q4 ? (_Float16)1032.0f : (_Float16)1152.0f;
    const half2_t bb = {bias, bias};
    half8_t q;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t p = __builtin_amdgcn_perm(0x64646464u, src[i >> 1],
                                                 (i & 1) ? 0x07030702u : 0x07010700u);
        const half2_t v = __builtin_bit_cast(half2_t, p) - bb;
        q[2 * i] = v.x;
        q[2 * i + 1] = v.y;
    }
    return q;
}

/* the k loop of one chunk for NMT token tiles: per block, t = A_hi[mt] . q[n] + A_lo[mt] . q[n]
   (two MFMAs, the second accumulating onto the first) and acc[n][mt] += d[n] * t in fp32,
   blocks in order. Measured against the B operand w = q * d as an exact f16 pair hi + lo
   (three MFMAs accumulating across blocks, 22 instructions per lane to form hi and lo from
   a block's 8 weights, against 12 for q here plus 4 fused multiply-adds per token tile):
   gate/up 112.7 -> 103.5 us, down 60.2 -> 57.6 us at 512 tokens. */
template <class R, int NMT>
__device__ static void pf_loop(uint8_t *ring, int S, const _Float16 *const (&asrc_h)[R::KB],
                               const _Float16 *const (&asrc_l)[R::KB],
                               const uint8_t *wsrc, size_t wstep, const uint8_t *ssrc,
                               f32x4_t (*acc)[R::TT]) {
    static_assert(NMT <= R::TT, "token tiles");
    constexpr int ENC = R::ENCODING;
    constexpr int KB = R::KB;
    const int l = threadIdx.x & 63, g = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   /* wavefront-uniform */
    auto issue = [&](int st) {
        uint8_t *slot = ring + (st % R::P) * R::STAGE;
        st = min(st, S - 1);            /* past the end: a valid stage into a free slot */
        if (w < NMT) {                  /* empty token tiles are not loaded */
#pragma unroll
            for (int i = 0; i < KB; i++) {
                lds_dma16(asrc_h[i] + st * 32 * KB, slot + 1024 * (KB * w + i));
                lds_dma16(asrc_l[i] + st * 32 * KB, slot + R::A_BYTES + 1024 * (KB * w + i));
            }
        }
#pragma unroll
        for (int i = 0; i < R::WI; i++)
            if (R::WB >= 1024 * (i + 1) || l * 16 < R::WB - 1024 * i)
                lds_dma16(wsrc + (size_t)st * wstep + 1024 * i + 16 * l,
                          slot + 2 * R::A_BYTES + w * R::WB + 1024 * i);
        if (l * 16 < R::SB)
            lds_dma16(ssrc + (size_t)st * 128 * KB + 16 * l,
                      slot + 2 * R::A_BYTES + R::W_BYTES + w * R::SB);
    };
    /* this lane's B rows: segment and row within it, per tile */
    int boff[R::NBT], soff[R::NBT];
#pragma unroll
    for (int n = 0; n < R::NBT; n++) {
        /* tile n: matrix n / TPM (GU: gate, then up), rows RW/4 * w + 16 * (n % TPM) of it;
           the workgroup's RW rows of a matrix are its segments TPM * matrix .. */
        const int r = R::RW * (n / R::TPM) + R::RW / 4 * w + 16 * (n % R::TPM) + (l & 15);
        const int seg = r >> 6, rs = r & 63;
        boff[n] = (seg * KB * 64 + rs) * R::PB + (ENC == CPG_ENC_Q4 ? 8 * (g & 1) : 8 * g);
        soff[n] = (seg * KB * 64 + rs) * 2;
    }
    for (int st = 0; st < R::P - 1; st++) issue(st);
    for (int s = 0; s < S; s++) {
        asm volatile("" ::: "memory");
        /* stage s has landed when at most the later stages' loads are in flight: Q per stage
           for a wavefront that loads A tiles, Q - 2 * KB for one that does not */
        if (w < NMT) wait_vm_lgkm<R::Q * (R::P - 2)>();
        else wait_vm_lgkm<(R::Q - 2 * KB) * (R::P - 2)>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(s + R::P - 1);
        const uint8_t *slot = ring + (s % R::P) * R::STAGE;
        const _Float16 *ah = (const _Float16 *)slot, *al = (const _Float16 *)(slot + R::A_BYTES);
        const uint8_t *wl = slot + 2 * R::A_BYTES;
        const uint16_t *sl = (const uint16_t *)(wl + R::W_BYTES);
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            half8_t a_hi[NMT], a_lo[NMT];
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const int r = mt * 16 + (l & 15);
                const int o = r * 32 * KB + 8 * R::apos(r, 4 * kb + g);
                a_hi[mt] = *(const half8_t *)(ah + o);
                a_lo[mt] = *(const half8_t *)(al + o);
            }
#pragma unroll
            for (int n = 0; n < R::NBT; n++) {
                WRaw r;
                r.w = *(const uint2 *)(wl + boff[n] + kb * 64 * R::PB);
                r.d = *(const uint16_t *)((const uint8_t *)sl + soff[n] + kb * 128);
                const half8_t q = weight_q<ENC>(r.w, g);
                const float d = scale_f32(r.d);
                f32x4_t t[NMT];
#pragma unroll
                for (int mt = 0; mt < NMT; mt++) {
                    const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
                    t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi[mt], q, z, 0, 0, 0);
                }
#pragma unroll
                for (int mt = 0; mt < NMT; mt++)
                    t[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo[mt], q, t[mt], 0, 0, 0);
#pragma unroll
                for (int mt = 0; mt < NMT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[n][mt][i] = fmaf(d, t[mt][i], acc[n][mt][i]);
            }
        }
    }
    /* no load may still write this workgroup's LDS when it ends */
    asm volatile("" ::: "memory");
    wait_vm_lgkm<0>();
}

/* grid (rows / RW, max_chunks), PF_NT threads, dynamic LDS PfRing::P * PfRing::STAGE,
   max_chunks a multiple of 8. Chunk c = (group g, tokens m0..m0+m-1) of expert e.
   GU (gate/up): rows r0..r0+RW-1 of Wg and of Wu (n_in = D) over the hi/lo planes of xn (one
     row per token id), then h = silu(g) * u (kernels.c:416) written as hi/lo f16 rows hh/hl
     at the token's position in the group list (off + m0 + i), the A operand of the down GEMM.
   down: rows r0..r0+RW-1 of Wd (n_in = F) over hh/hl at the group-list positions; y[pair]
     (row stride n_out) for the pair of each position.
   TT < 4 (a ring for TT token tiles): every chunk holds at most 16 * TT tokens (the host
   guarantees it: batches of at most 16 * TT tokens, as a token's K experts are distinct). */
template <int ENC, bool GU, int TT = PF_CHUNK / 16, int P = 2, int RW = 128, int KB = 2>
__global__ __launch_bounds__(PF_NT) __attribute__((amdgpu_waves_per_eu(TT == 4 ? 3 : 1))) void k_pf_gemm(
    const uint8_t *__restrict__ experts, size_t exp_stride, size_t mat0, size_t mat_bytes,
    size_t payload_plane, int n_in, int n_out, const int *__restrict__ chunk_grp,
    const int *__restrict__ chunk_m0, const int *__restrict__ grp_expert,
    const int *__restrict__ grp_off, const int *__restrict__ grp_cnt,
    const int *__restrict__ list, const _Float16 *__restrict__ xh,
    const _Float16 *__restrict__ xl, _Float16 *__restrict__ hh, _Float16 *__restrict__ hl,
    float *__restrict__ y, const int *__restrict__ sel, int npairs, int K, int E,
    int *__restrict__ ngroups) {
    using R = PfRing<ENC, GU, TT, P, RW, KB>;
    extern __shared__ __align__(16) uint8_t ring[];
    __shared__ int arow[PF_CHUNK], orow[PF_CHUNK];
    __shared__ uint64_t tab[32];
    /* workgroup i runs on XCD i % 8: the row tiles of chunk c are placed on XCD c % 8, next
       to each other in its dispatch order, so the chunk's activations are fetched into one L2
       (gridDim.y is a multiple of 8) */
    const int nx = gridDim.x, id = blockIdx.x + nx * blockIdx.y, sidx = id >> 3;
    const int c = 8 * (sidx / nx) + (id & 7);
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = l >> 4;
    const int r0 = (sidx % nx) * RW, nb = n_in / 32;
    int e, m;
    if (TT == 1 && sel) {
        /* chunk c is the c-th expert with pairs (ascending id) of the npairs <= 256 selections
           sel[t * K + j] (ids below E <= 256 count): found by wavefront 0 from sel itself, with the expert's
           pairs in ascending pair order (at most 16: one token tile); no grouping step
           before this launch. Gate/up: A rows the pairs' tokens, outputs at the pair
           indices; down: A rows and outputs at the pair indices. */
        __shared__ int used[MAX_E], pick[2];
        if (w == 0) {
            int v[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                v[q] = l + 64 * q < npairs ? sel[l + 64 * q] : -1;
                if ((unsigned)v[q] >= (unsigned)E) v[q] = -1;
            }
#pragma unroll
            for (int q = 0; q < 4; q++) used[l + 64 * q] = 0;
            wave_lds_sync();
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (v[q] >= 0) used[v[q]] = 1;
            wave_lds_sync();
            const unsigned long long lt = (1ull << l) - 1ull;
            int ex = -1, before = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const unsigned long long u = __ballot(used[l + 64 * q] != 0);
                const int cc = c - before;
                const bool hit = cc >= 0 && ((u >> l) & 1ull) && __popcll(u & lt) == cc;
                const unsigned long long hb = __ballot(hit);
                if (hb) ex = 64 * q + __ffsll((long long)hb) - 1;
                before += __popcll(u);
            }
            /* the number of experts with pairs, for the caller (one workgroup writes it) */
            if (ngroups && id == 0 && l == 0) *ngroups = before;
            int n = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const bool mine = ex >= 0 && v[q] == ex;
                const unsigned long long pb = __ballot(mine);
                const int i = n + __popcll(pb & lt), pr = l + 64 * q;
                if (mine && i < 16) {
                    arow[i] = GU ? pr / K : pr;
                    orow[i] = pr;
                }
                n += __popcll(pb);
            }
            n = min(n, 16);
            wave_lds_sync();
            /* rows past the expert's pairs repeat its last one (valid addresses) */
            if (ex >= 0 && l >= n) {
                arow[l] = arow[n - 1];
                orow[l] = orow[n - 1];
            }
            if (l == 0) {
                pick[0] = ex;
                pick[1] = n;
            }
        }
        if (GU && tid < 32) tab[tid] = cpg_exp2f_tab[tid];
        __syncthreads();
        e = pick[0];
        m = pick[1];
        if (e < 0) return;
    } else {
        const int grp = chunk_grp[c];
        if (grp < 0) return;
        e = grp_expert[grp];
        const int off = grp_off[grp], m0 = chunk_m0[c];
        m = min(PF_CHUNK, grp_cnt[grp] - m0);
        if (tid < PF_CHUNK) {
            const int i = min(tid, m - 1);
            arow[tid] = GU ? list[off + m0 + i] : off + m0 + i;
            orow[tid] = GU ? off + m0 + i : list[off + m0 + i];
        }
        if (GU && tid < 32) tab[tid] = cpg_exp2f_tab[tid];
        __syncthreads();
    }
    const int nmt = (m + 15) / 16;
    /* the sources of this lane's loads for block 0 (block st adds st * 32 halves, or one
       block's bytes): A row 16w + l/4, piece l%4; the wavefront's WB weight bytes and SB
       scale bytes of the stage */
    /* A load i of the wavefront fills rows 16w + i * 64/PP .. (PP lanes per row): this lane's
       row and the logical piece that belongs at its position */
    const _Float16 *ash[R::KB], *asl[R::KB];
#pragma unroll
    for (int i = 0; i < R::KB; i++) {
        const int ar = 16 * w + i * (64 / R::PP) + l / R::PP;
        const size_t ao = (size_t)arow[ar] * n_in + 8 * R::apos(ar, l % R::PP);
        ash[i] = xh + ao;
        asl[i] = xl + ao;
    }
    const uint8_t *M0 = experts + (size_t)e * exp_stride + mat0;
    const int wseg = w * R::WB / (R::KB * 64 * R::PB), wofs = w * R::WB % (R::KB * 64 * R::PB);
    const int sseg = w * R::SB / (R::KB * 128), sofs = w * R::SB % (R::KB * 128);
    /* a segment's matrix (GU: gate, then up) and 64-row tile */
    auto seg_mat = [&](int seg) { return GU ? M0 + (size_t)(seg / R::TPM) * mat_bytes : M0; };
    auto seg_tile = [&](int seg) { return (size_t)((r0 >> 6) + seg % R::TPM); };
    const uint8_t *wsrc = seg_mat(wseg) + seg_tile(wseg) * nb * 64 * R::PB + wofs;
    const uint8_t *ssrc = seg_mat(sseg) + payload_plane + seg_tile(sseg) * nb * 128 + sofs;
    f32x4_t acc[R::NBT][TT];
#pragma unroll
    for (int n = 0; n < R::NBT; n++)
#pragma unroll
        for (int mt = 0; mt < TT; mt++)
            for (int i = 0; i < 4; i++) acc[n][mt][i] = 0.0f;
    const size_t wstep = (size_t)R::KB * 64 * R::PB;
    const int S = nb / R::KB;
    if constexpr (TT == 1) {
        pf_loop<R, 1>(ring, S, ash, asl, wsrc, wstep, ssrc, acc);
    } else {
        switch (nmt) {
        case 1: pf_loop<R, 1>(ring, S, ash, asl, wsrc, wstep, ssrc, acc); break;
        case 2: pf_loop<R, 2>(ring, S, ash, asl, wsrc, wstep, ssrc, acc); break;
        case 3: pf_loop<R, 3>(ring, S, ash, asl, wsrc, wstep, ssrc, acc); break;
        default: pf_loop<R, 4>(ring, S, ash, asl, wsrc, wstep, ssrc, acc); break;
        }
    }
    if constexpr (GU) {
#pragma unroll
        for (int half = 0; half < R::TPM; half++)
#pragma unroll
            for (int mt = 0; mt < TT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = mt * 16 + 4 * g + i;
                    if (r < m) {
                        const float hv =
                            swiglu_t(acc[half][mt][i], acc[R::TPM + half][mt][i], tab);
                        const f16pair p = split_f16(hv);
                        const size_t o = (size_t)orow[r] * n_out + r0 + RW / 4 * w +
                                         16 * half + (l & 15);
                        hh[o] = p.hi;
                        hl[o] = p.lo;
                    }
                }
    } else {
#pragma unroll
        for (int n = 0; n < R::NBT; n++)
#pragma unroll
            for (int mt = 0; mt < TT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = mt * 16 + 4 * g + i;
                    if (r < m)
                        y[(size_t)orow[r] * n_out + r0 + RW / 4 * w + 16 * n + (l & 15)] =
                            acc[n][mt][i];
                }
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
    const int rows[1] = {row};
    /* the activation planes from block b0 on: stage k0 offsets then count from there */
    const _Float16 *hi = xh + (size_t)b0 * 32, *lo = xl + (size_t)b0 * 32;
    switch (nmt) {
    case 1: gemm_k_loop<ENC, PfDown, 1, 1>(M, payload_plane, rows, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    case 2: gemm_k_loop<ENC, PfDown, 2, 1>(M, payload_plane, rows, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    case 3: gemm_k_loop<ENC, PfDown, 3, 1>(M, payload_plane, rows, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
    default: gemm_k_loop<ENC, PfDown, 4, 1>(M, payload_plane, rows, nb, g, S, m, row_of, hi, lo, (size_t)n_in, ah, al, acc, b0); break;
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

/* grid (ceil(D/1024), T), 256 threads, D % 4 == 0: o = mlp[t][d] + sum_j wt[t][j] *
   y[t*K + j][d] in slot order (qwen3_moe.c:221), four consecutive d per thread (float4);
   written to mlp, or with xres: xres[t][d] += attn[t][d] + o and mlp untouched (mlp must then
   be zero, the reference's calloc'ed start, cachepotato.c:157-159). KT > 0: K == KT, every
   pair's load issued before the sums. */
template <int KT>
__global__ __launch_bounds__(256) void k_pair_combine(const float *__restrict__ y,
                                                      const float *__restrict__ wt, int D, int K,
                                                      float *__restrict__ mlp,
                                                      float *__restrict__ xres,
                                                      const float *__restrict__ attn) {
    const int t = blockIdx.y, d = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (d >= D) return;
    if (KT) K = KT;
    const size_t o = (size_t)t * D + d;
    float4 acc = xres ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : *(const float4 *)(mlp + o);
    auto add = [&](float w, float4 v) {
        acc = make_float4(__fadd_rn(acc.x, __fmul_rn(w, v.x)), __fadd_rn(acc.y, __fmul_rn(w, v.y)),
                          __fadd_rn(acc.z, __fmul_rn(w, v.z)), __fadd_rn(acc.w, __fmul_rn(w, v.w)));
    };
    if constexpr (KT > 0) {
        float4 v[KT];
#pragma unroll
        for (int j = 0; j < KT; j++) v[j] = *(const float4 *)(y + ((size_t)t * KT + j) * D + d);
#pragma unroll
        for (int j = 0; j < KT; j++) add(wt[(size_t)t * KT + j], v[j]);
    } else {
        for (int j = 0; j < K; j++)
            add(wt[(size_t)t * K + j], *(const float4 *)(y + ((size_t)t * K + j) * D + d));
    }
    if (xres) {
        const float4 xr = *(const float4 *)(xres + o), ar = *(const float4 *)(attn + o);
        *(float4 *)(xres + o) = make_float4(__fadd_rn(xr.x, __fadd_rn(ar.x, acc.x)),
                                            __fadd_rn(xr.y, __fadd_rn(ar.y, acc.y)),
                                            __fadd_rn(xr.z, __fadd_rn(ar.z, acc.z)),
                                            __fadd_rn(xr.w, __fadd_rn(ar.w, acc.w)));
    } else {
        *(float4 *)(mlp + o) = acc;
    }
}

/* ---------------------------------------------------------------- host */

/* the most chunks T tokens with K experts each over E experts can form */
int cpg_prefill_max_chunks(int T, int K, int E) {
    const int pairs = T * K;
    const int groups = pairs < E ? pairs : E;
    const int n = (pairs + PF_CHUNK - 1) / PF_CHUNK + groups;
    return (n + 7) / 8 * 8;                      /* k_pf_gemm places chunk c on XCD c % 8 */
}

bool cpg_prefill_shape_ok(int D, int F) {
    return D % 128 == 0 && F % 128 == 0;
}

template <int ENC>
static int prefill_experts(const cpg_moe_layer *L, int T, const float *xn, const float *wt,
                           const int *grp_expert, const int *grp_off, const int *grp_cnt,
                           const int *list_tok, const int *list_pair, int *chunk_grp,
                           int *chunk_m0, void *scratch, float *y, float *mlp, float *xres,
                           const float *attn, bool prepared, const int *sel, int *ngroups) {
    const int D = L->D, F = L->F, E = L->E, K = L->K;
    /* sel: the one-tile GEMMs find their expert and pairs in the selections themselves, one
       chunk per expert with pairs */
    if (sel && !cpg_prefill_sel_ok(T, K, E)) {
        cpg_set_error("prefill_experts: selections of %d tokens x %d over %d experts", T, K, E);
        return -1;
    }
    const int mc = sel ? ((T * K < E ? T * K : E) + 7) / 8 * 8 : cpg_prefill_max_chunks(T, K, E);
    _Float16 *xh = (_Float16 *)scratch, *xl = xh + (size_t)T * D;
    _Float16 *hh = xl + (size_t)T * D, *hl = hh + (size_t)T * K * F;
    if (!prepared) {
        if (!sel)
            LAUNCH(CPG_KT_SELECT, k_chunks, dim3(1), dim3(64), 0, grp_cnt, E, mc, chunk_grp,
                   chunk_m0);
        LAUNCH(CPG_KT_SELECT, k_split_hilo, dim3(T), dim3(256), 0, xn, D, xh, xl);
    }
    const uint8_t *ex = (const uint8_t *)L->experts;
    const size_t es = cpg_expert_bytes(ENC, D, F), mg = cpg_matrix_bytes(ENC, F, D);
    auto gemms = [&](auto gu_kernel, size_t ring_gu, int rw_gu, auto dn_kernel, size_t ring_dn,
                     int rw_dn) {
        if (ring_gu > 64 * 1024)
            CPG_HIP(hipFuncSetAttribute((const void *)gu_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)ring_gu));
        if (ring_dn > 64 * 1024)
            CPG_HIP(hipFuncSetAttribute((const void *)dn_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)ring_dn));
        LAUNCH(CPG_KT_GATEUP, gu_kernel, dim3(F / rw_gu, mc), dim3(PF_NT), ring_gu, ex, es,
               (size_t)0, mg, cpg_payload_plane(ENC, F, D), D, F, chunk_grp, chunk_m0,
               grp_expert, grp_off, grp_cnt, list_tok, xh, xl, hh, hl, (float *)nullptr, sel,
               T * K, K, E, ngroups);
        LAUNCH(CPG_KT_DOWN, dn_kernel, dim3(D / rw_dn, mc), dim3(PF_NT), ring_dn, ex, es, 2 * mg,
               mg, cpg_payload_plane(ENC, D, F), F, D, chunk_grp, chunk_m0, grp_expert, grp_off,
               grp_cnt, list_pair, hh, hl, (_Float16 *)nullptr, (_Float16 *)nullptr, y, sel,
               T * K, K, E, (int *)nullptr);
        return 0;
    };
    int rc;
    if (T <= 16) {
        /* every expert group holds at most T <= 16 tokens: one token tile, a deeper ring */
        using RG = PfRing<ENC, true, 1, PF_SMALL_RING, PF_SMALL_RW_GU, PF_SMALL_KB>;
        using RD = PfRing<ENC, false, 1, PF_SMALL_RING, PF_SMALL_RW_DN, PF_SMALL_KB>;
        rc = gemms(k_pf_gemm<ENC, true, 1, PF_SMALL_RING, PF_SMALL_RW_GU, PF_SMALL_KB>,
                   (size_t)RG::P * RG::STAGE, RG::RW,
                   k_pf_gemm<ENC, false, 1, PF_SMALL_RING, PF_SMALL_RW_DN, PF_SMALL_KB>,
                   (size_t)RD::P * RD::STAGE, RD::RW);
    } else {
        if (sel) { cpg_set_error("prefill_experts: selections need T <= 16"); return -1; }
        using RG = PfRing<ENC, true>;
        using RD = PfRing<ENC, false>;
        rc = gemms(k_pf_gemm<ENC, true>, (size_t)RG::P * RG::STAGE, RG::RW,
                   k_pf_gemm<ENC, false>, (size_t)RD::P * RD::STAGE, RD::RW);
    }
    if (rc) return rc;
    if (K == 8)
        LAUNCH(CPG_KT_COMBINE, k_pair_combine<8>, dim3((D + 1023) / 1024, T), dim3(256), 0, y,
               wt, D, K, mlp, xres, attn);
    else
        LAUNCH(CPG_KT_COMBINE, k_pair_combine<0>, dim3((D + 1023) / 1024, T), dim3(256), 0, y,
               wt, D, K, mlp, xres, attn);
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

/* the products from the hi/lo planes already in scratch: out directly (ks == 1) or ks parts
   of T * n_out floats, left unsummed in *parts when sum is false */
template <int ENC>
static int dense_from_planes(const void *w, int n_in, int n_out, int T, void *scratch,
                             float *out, bool sum, const float **parts, int *ks_out) {
    const int ks = dense_ksplit(T, n_in, n_out);
    const _Float16 *xh = (const _Float16 *)scratch, *xl = xh + (size_t)T * n_in;
    float *part = ks > 1 ? (float *)((uint8_t *)scratch + cpg_round256((size_t)4 * T * n_in))
                         : out;
    hipStream_t s = g_cpg.stream;
    hipLaunchKernelGGL(k_mfma_dense<ENC>, dim3(n_out / PfDown::ROWS, (T + PF_CHUNK - 1) / PF_CHUNK, ks),
                       dim3(PfDown::NT), 0, s, (const uint8_t *)w,
                       cpg_payload_plane(ENC, n_out, n_in), n_in, n_out, T, n_in / 32 / ks, xh,
                       xl, part);
    CPG_LAUNCH_CHECK("k_mfma_dense");
    if (parts) *parts = part;
    if (ks_out) *ks_out = ks;
    if (ks > 1 && sum) {
        const size_t n = (size_t)T * n_out;
        hipLaunchKernelGGL(k_sum_parts, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part,
                           ks, n, out);
        CPG_LAUNCH_CHECK("k_sum_parts");
    }
    return 0;
}

template <int ENC>
static int dense_mfma(const void *w, int n_in, int n_out, const float *x, int T, void *scratch,
                      float *out) {
    _Float16 *xh = (_Float16 *)scratch, *xl = xh + (size_t)T * n_in;
    hipLaunchKernelGGL(k_split_hilo, dim3(T), dim3(256), 0, g_cpg.stream, x, n_in, xh, xl);
    CPG_LAUNCH_CHECK("k_split_hilo");
    return dense_from_planes<ENC>(w, n_in, n_out, T, scratch, out, true, nullptr, nullptr);
}

int cpg_dense_from_planes(int enc, const void *w, int n_in, int n_out, int T, void *scratch,
                          float *out, int sum, const float **parts, int *ks) {
    if (!w || !scratch || !out || T <= 0 || !cpg_dense_shape_ok(n_in, n_out)) {
        cpg_set_error("cpg_dense_from_planes: bad arguments (n_in %d, n_out %d, T %d)", n_in,
                      n_out, T);
        return -1;
    }
    if (enc == CPG_ENC_Q4)
        return dense_from_planes<CPG_ENC_Q4>(w, n_in, n_out, T, scratch, out, sum, parts, ks);
    if (enc == CPG_ENC_Q8)
        return dense_from_planes<CPG_ENC_Q8>(w, n_in, n_out, T, scratch, out, sum, parts, ks);
    cpg_set_error("cpg_dense_from_planes: encoding %d is not row-tiled (Q4_0 or Q8_0 only)", enc);
    return -1;
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

bool cpg_prefill_sel_ok(int T, int K, int E) {
    return T > 0 && T <= 16 && K > 0 && T * K <= 256 && E > 0 && E <= MAX_E && MAX_E <= 256;
}

int cpg_prefill_experts(const cpg_moe_layer *L, int T, const float *xn, const float *wt,
                        const int *grp_expert, const int *grp_off, const int *grp_cnt,
                        const int *list_tok, const int *list_pair, int *chunk_grp,
                        int *chunk_m0, void *scratch, float *y, float *mlp, float *xres,
                        const float *attn, int prepared, const int *sel, int *ngroups) {
    if (L->enc == CPG_ENC_Q4)
        return prefill_experts<CPG_ENC_Q4>(L, T, xn, wt, grp_expert, grp_off, grp_cnt, list_tok,
                                           list_pair, chunk_grp, chunk_m0, scratch, y, mlp, xres,
                                           attn, prepared != 0, sel, ngroups);
    return prefill_experts<CPG_ENC_Q8>(L, T, xn, wt, grp_expert, grp_off, grp_cnt, list_tok,
                                       list_pair, chunk_grp, chunk_m0, scratch, y, mlp, xres,
                                       attn, prepared != 0, sel, ngroups);
}
