/* cpg_mfma.h — MFMA operand helpers for the Q4_0 / Q8_0 expert products on gfx950.
 *
 * v_mfma_f32_16x16x32_f16 operand layout (checked on the device): lane l holds
 * A[l%16][8(l/16) + j] and B[8(l/16) + j][l%16] for j = 0..7, and D[4(l/16) + i][l%16] for
 * i = 0..3. The weights are the B operand: a lane's 8 k-slots of one block are 8 exact small
 * integers q (Q4: -8..7, Q8: -127..127) of row l%16, converted to f16 without rounding; the
 * block's fp16 scale is applied in fp32 to the block's product. The activations are the A
 * operand, split x = hi + lo with hi = f16(x) and lo = f16(x - hi) (22 significant bits),
 * both halves multiplied. A Q4 lane group g takes the low (g < 2) or high (g >= 2) nibbles of
 * payload bytes 8(g%2)..8(g%2)+7, which hold elements 8g..8g+7 (byte i holds elements i and
 * i+16); a Q8 lane group takes bytes 8g..8g+7. */
#ifndef CPG_MFMA_H
#define CPG_MFMA_H
#include "cpg_internal.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

/* x = hi + lo with hi = f16(x) and lo = f16(x - hi), x the rounded fp32 value. x is made
   opaque to the optimiser first: otherwise, when x is a product, it may fold the product and
   the conversion to f16 into one mixed-precision FMA (one rounding of the exact product),
   use that for hi in one place and f16(x) in another, and hi + lo then misses x by an f16
   unit in the last place where the two roundings differ. */
struct f16pair {
    _Float16 hi, lo;
};
__device__ static inline f16pair split_f16(float x) {
    asm("" : "+v"(x));
    const _Float16 h = (_Float16)x;
    return {h, (_Float16)(x - (float)h)};
}

__device__ static inline half8_t pairs_to_half8(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3,
                                               _Float16 bias) {
    /* each p holds two 16-bit values 0x6400 | u, i.e. the f16 numbers 1024 + u; subtracting
       the bias gives u - (bias - 1024) exactly */
    half8_t h;
    const uint32_t p[4] = {p0, p1, p2, p3};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        half2_t v = __builtin_bit_cast(half2_t, p[i]);
        h[2 * i] = v.x - bias;
        h[2 * i + 1] = v.y - bias;
    }
    return h;
}

/* spread the four bytes of w (each < 256) to the 16-bit halves of two words, with 0x6400 */
__device__ static inline void bytes_to_pairs(uint32_t w, uint32_t &a, uint32_t &b) {
    a = (w & 0xFFu) | ((w << 8) & 0xFF0000u) | 0x64006400u;
    b = ((w >> 16) & 0xFFu) | ((w >> 8) & 0xFF0000u) | 0x64006400u;
}

/* The raw bytes of one lane's B operand for one block: 8 payload bytes of `row` holding
   k-slots 8g..8g+7, and the fp16 scale. */
struct WRaw {
    uint2 w;
    uint16_t d;
    /* opaque to the optimiser where called: conversions of weights held across a loop then
       happen at their use instead of being hoisted out of it into extra registers */
    __device__ void pin() {
        uint32_t dd = d;
        asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(dd));
        d = (uint16_t)dd;
    }
};

template <int ENC>
__device__ static inline WRaw weight_raw(const uint8_t *__restrict__ M, size_t payload_plane,
                                         int row, int b, int nb, int g) {
    const size_t t = cpg_tile_index(row, b, nb);
    WRaw r;
    r.d = ((const uint16_t *)(M + payload_plane))[t];
    r.w = ENC == CPG_ENC_Q4 ? *(const uint2 *)(M + t * 16 + (g & 1) * 8)
                            : *(const uint2 *)(M + t * 32 + g * 8);
    return r;
}

/* the payload part of weight_raw alone */
template <int ENC>
__device__ static inline uint2 weight_payload(const uint8_t *__restrict__ M, int row, int b, int nb,
                                              int g) {
    const size_t t = cpg_tile_index(row, b, nb);
    return ENC == CPG_ENC_Q4 ? *(const uint2 *)(M + t * 16 + (g & 1) * 8)
                             : *(const uint2 *)(M + t * 32 + g * 8);
}

/* the 8 weights as exact f16 integers q */
template <int ENC>
__device__ static inline half8_t weight_half8(WRaw r, int g) {
    uint32_t a0, a1, a2, a3;
    if (ENC == CPG_ENC_Q4) {
        const int sh = (g >> 1) * 4;
        bytes_to_pairs((r.w.x >> sh) & 0x0F0F0F0Fu, a0, a1);
        bytes_to_pairs((r.w.y >> sh) & 0x0F0F0F0Fu, a2, a3);
        return pairs_to_half8(a0, a1, a2, a3, (_Float16)1032.0f);     /* u - 8 = q */
    }
    bytes_to_pairs(r.w.x, a0, a1);
    bytes_to_pairs(r.w.y, a2, a3);
    return pairs_to_half8(a0, a1, a2, a3, (_Float16)1152.0f);         /* u - 128 = q */
}

/* an fp16 scale as fp32 by the hardware conversion (exact; the same value as cpg_f16_to_f32
   for every non-NaN input, without its branches) */
__device__ static inline float scale_f32(uint16_t d) {
    return (float)__builtin_bit_cast(_Float16, d);
}

/* the hi/lo f16 halves of 8 floats */
__device__ static inline void split_hilo8(float4 v0, float4 v1, half8_t &h, half8_t &l) {
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const f16pair p = split_f16(v[j]);
        h[j] = p.hi;
        l[j] = p.lo;
    }
}

#define PF_CHUNK 64         /* prefill: tokens per chunk of an expert group (4 MFMA tiles) */

/* One wavefront, all 64 lanes: the prefill chunk list, the (group, first token m0) of every
   chunk of at most PF_CHUNK tokens of the expert groups. Lane t brings the token counts
   cnt[j] of four groups and their group indices grp[j] (a count of 0: no chunk). k_pf_gemm
   runs chunk slot p on XCD p % 8, the slots of one XCD in the order p / 8, and a chunk's cost
   grows with its token tiles of 16 (1-4): the chunks are listed by tile count, 4 first, then
   in lane order, so the costly ones start first and the short ones fill the end of the
   launch. One wavefront scan per tile count gives the slots; the chunks fill slots
   0..total-1 and the slots from total to max_chunks get group -1 (no slot is written
   twice). */
__device__ static inline void pf_chunk_list(const int (&cnt)[4], const int (&grp)[4],
                                            int max_chunks, int *__restrict__ chunk_grp,
                                            int *__restrict__ chunk_m0) {
    constexpr int NT = PF_CHUNK / 16;            /* tile counts NT..1 are classes 0..NT-1 */
    const int t = threadIdx.x & 63;
    int n[4], last[4], ncls[NT];
#pragma unroll
    for (int k = 0; k < NT; k++) ncls[k] = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        n[j] = (cnt[j] + PF_CHUNK - 1) / PF_CHUNK;
        /* n - 1 full chunks (class 0) and the last one, of class NT - its tiles */
        last[j] = n[j] ? NT - (cnt[j] - (n[j] - 1) * PF_CHUNK + 15) / 16 : 0;
        if (n[j]) {
            ncls[0] += n[j] - 1;
            ncls[last[j]] += 1;
        }
    }
    int pos[NT], total = 0;
#pragma unroll
    for (int k = 0; k < NT; k++) {
        int incl = ncls[k];
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (t >= o) incl += v;
        }
        pos[k] = total + incl - ncls[k];
        total += __shfl(incl, 63);
    }
    for (int i = total + t; i < max_chunks; i += 64) chunk_grp[i] = -1;
#pragma unroll
    for (int j = 0; j < 4; j++)
        for (int c = 0; c < n[j]; c++) {
            int p = 0;
#pragma unroll
            for (int k = 0; k < NT; k++)        /* the class's next slot (no dynamic index) */
                if (k == (c + 1 < n[j] ? 0 : last[j])) p = pos[k]++;
            if (p < max_chunks) {
                chunk_grp[p] = grp[j];
                chunk_m0[p] = c * PF_CHUNK;
            }
        }
}

#endif
