/* cpg_gemv.h — device building blocks shared by the GEMV kernels (MoE experts, attention
 * projections, the output head): wavefront reductions on DPP moves, the row-tiled Q4_0 /
 * Q8_0 block dot products, activation staging into LDS, and the SwiGLU activation.
 *
 * Layout recap (cpg.h "weight layout"): a row-tiled matrix stores, per 64-row tile and per
 * 32-element block column, the 64 rows' blocks consecutively; payload u = q + 8 (Q4, nibbles)
 * or q + 128 (Q8, bytes), scales in a separate fp16 plane. A dot product over one block is
 * taken on u and corrected once: d * (sum u*x - c * sum x). Staged activations hold, per block,
 * x[0..15] then x[16..31]/16 for Q4 (the high nibbles are used in place, worth 16u), plain x
 * for Q8, and each block's sum of x.
 */
#ifndef CPG_GEMV_H
#define CPG_GEMV_H
#include "cpg_internal.h"

#define WAVE 64
#define MT 4                /* tokens per pass over a weight tile held in registers */
#define GW 8                /* wavefronts per GEMV workgroup (they split k) */
#define MAX_BPW 4           /* blocks per lane held in registers, general kernels */

/* MI355X has 8 XCDs, each with its own L2, and the dispatcher hands workgroup i of a launch
   to XCD i % 8. xcd_tile maps hardware workgroup id (of n) to a logical tile so that XCD x
   gets the contiguous tiles [x*n/8, (x+1)*n/8): neighbouring tiles that share 128-byte lines
   (the fp16 scale plane holds a 64-row tile's scales of one block in one such line) are then
   fetched into one L2 instead of one per XCD. n % 8 != 0 keeps the identity. */
#define NXCD 8
__device__ static inline int xcd_tile(int id, int n) {
    return n % NXCD ? id : (id % NXCD) * (n / NXCD) + id / NXCD;
}
/* The same for workloads whose tiles differ in cost: logical tiles 2p and 2p+1 (which share
   the scale lines of one 64-row tile) go to one XCD, and consecutive pairs p to consecutive
   XCDs, so uneven work stays spread over all eight. n % 16 != 0 keeps the identity. */
__device__ static inline int xcd_pair(int id, int n) {
    if (n % (2 * NXCD)) return id;
    const int x = id % NXCD, q = id / NXCD;
    return 2 * ((q >> 1) * NXCD + x) + (q & 1);
}

/* ---- L2 warming
 * A launch that leaves CUs idle (a latency-bound kernel with few workgroups) carries extra
 * workgroups that read the bytes the next kernel will read, into the L2 of the XCD whose
 * workgroups will read them: an L2 survives the kernel boundary, and the next kernel's loads
 * then hit it instead of HBM. For a row-tiled matrix read by a GEMV that gives XCD x the rows
 * [x * rows / 8, (x + 1) * rows / 8) (xcd_tile), XCD x's bytes are one span of the payload
 * plane and one of the scale plane. Warming changes no result: it only reads. */
struct l2_warm_t {
    const uint8_t *base;    /* null: nothing to warm */
    size_t pay;             /* payload bytes per XCD (XCD x's span starts at x * pay) */
    size_t sc_off, sc;      /* the scale plane's offset; scale bytes per XCD */
    int parts;              /* workgroups per XCD */
};

/* Workgroup-wide (256 threads): warming workgroup wi of a launch whose warming workgroups
   follow the others; it runs on XCD blockIdx.x % NXCD (workgroup i of a launch goes to XCD
   i % 8) and reads its share of that XCD's spans. Each thread's 16-byte loads are issued eight
   at a time and only made to complete (an empty asm takes each value). */
__device__ static inline void l2_warm(const l2_warm_t &w, int wi) {
    if (!w.base) return;
    const int x = blockIdx.x % NXCD, part = wi / NXCD;
    const size_t total = w.pay + w.sc;
    const size_t chunk = (total / w.parts + 15) / 16 * 16;
    const size_t lo = (size_t)part * chunk, hi = min(total, lo + chunk);
    for (size_t o0 = lo + 16 * threadIdx.x; o0 < hi; o0 += 16 * 256 * 8) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t o = min(o0 + (size_t)16 * 256 * u, hi - 16);
            const uint8_t *p = o < w.pay ? w.base + x * w.pay + o
                                         : w.base + w.sc_off + x * w.sc + (o - w.pay);
            v[u] = *(const uint4 *)p;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) asm volatile("" ::"v"(v[u].x));
    }
}

/* The warming of a row-tiled (rows x cols) matrix of encoding enc read as above; nothing
   (base null) when its rows do not split into whole 64-row tiles per XCD. */
static inline l2_warm_t l2_warm_rows(int enc, const void *W, int rows, int cols) {
    l2_warm_t w{nullptr, 0, 0, 0, 0};
    if (!W || rows % (NXCD * 64) || cols % 32) return w;
    const size_t tiles = (size_t)rows / NXCD / 64, blocks = (size_t)cols / 32;
    w.base = (const uint8_t *)W;
    w.pay = tiles * blocks * 64 * (enc == CPG_ENC_Q4 ? 16 : 32);
    w.sc = tiles * blocks * 64 * 2;
    w.sc_off = cpg_payload_plane(enc, rows, cols);
    w.parts = (int)((w.pay + w.sc + 65535) / 65536);
    return w;
}

/* ---- wavefront reductions and scans on VALU data-parallel moves (DPP) instead of LDS
   permutes: quad_perm / row mirrors within rows of 16 lanes, row_shr for scans, row_bcast
   to carry across rows, v_readlane to combine the four rows. */
#define DPP_QUAD_1032 0xB1
#define DPP_QUAD_2301 0x4E
#define DPP_ROW_SHR(n) (0x110 + (n))
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK = 0xf, bool BOUND = false>
__device__ static inline unsigned long long dpp_u64(unsigned long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xf, BOUND);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xf,
                                               BOUND);
    return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}
template <int CTRL, int ROW_MASK = 0xf, bool BOUND = false>
__device__ static inline double dpp_d(double v) {
    return __longlong_as_double((long long)dpp_u64<CTRL, ROW_MASK, BOUND>(
        (unsigned long long)__double_as_longlong(v)));
}
__device__ static inline unsigned long long readlane_u64(unsigned long long v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}
__device__ static inline double readlane_d(double v, int l) {
    return __longlong_as_double((long long)readlane_u64(
        (unsigned long long)__double_as_longlong(v), l));
}

/* the maximum over the wavefront, the same value in every lane */
__device__ static inline unsigned long long wave_max_u64(unsigned long long v) {
    unsigned long long o;
    o = dpp_u64<DPP_QUAD_1032>(v);       v = o > v ? o : v;
    o = dpp_u64<DPP_QUAD_2301>(v);       v = o > v ? o : v;
    o = dpp_u64<DPP_ROW_HALF_MIRROR>(v); v = o > v ? o : v;
    o = dpp_u64<DPP_ROW_MIRROR>(v);      v = o > v ? o : v;
    const unsigned long long r0 = readlane_u64(v, 0), r1 = readlane_u64(v, 16);
    const unsigned long long r2 = readlane_u64(v, 32), r3 = readlane_u64(v, 48);
    const unsigned long long a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
    return a > b ? a : b;
}

__device__ static inline uint32_t wave_max_u32(uint32_t v) {
    uint32_t o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, DPP_QUAD_1032, 0xf, 0xf, false);
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, DPP_QUAD_2301, 0xf, 0xf, false);
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, DPP_ROW_HALF_MIRROR, 0xf, 0xf, false);
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, DPP_ROW_MIRROR, 0xf, 0xf, false);
    v = o > v ? o : v;
    const uint32_t r0 = __builtin_amdgcn_readlane((int)v, 0), r1 = __builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane((int)v, 32), r3 = __builtin_amdgcn_readlane((int)v, 48);
    const uint32_t a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
    return a > b ? a : b;
}

/* the sum over the wavefront, the same value in every lane */
__device__ static inline double wave_sum_d(double v) {
    v += dpp_d<DPP_QUAD_1032>(v);
    v += dpp_d<DPP_QUAD_2301>(v);
    v += dpp_d<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_d<DPP_ROW_MIRROR>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

/* inclusive prefix sum over the wavefront's lanes */
__device__ static inline double wave_incl_scan_d(double v) {
    v += dpp_d<DPP_ROW_SHR(1), 0xf, true>(v);
    v += dpp_d<DPP_ROW_SHR(2), 0xf, true>(v);
    v += dpp_d<DPP_ROW_SHR(4), 0xf, true>(v);
    v += dpp_d<DPP_ROW_SHR(8), 0xf, true>(v);
    v += dpp_d<DPP_ROW_BCAST15, 0xa>(v);
    v += dpp_d<DPP_ROW_BCAST31, 0xc>(v);
    return v;
}

/* an order-preserving map of doubles onto unsigned integers (for finite values and infinities) */
__device__ static inline unsigned long long ord_d(double d) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(d);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ static inline uint32_t ord_f(float f) {
    const uint32_t b = (uint32_t)__float_as_int(f);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}
__device__ static inline double unord_d(unsigned long long u) {
    return __longlong_as_double((long long)((u >> 63) ? (u & 0x7fffffffffffffffull) : ~u));
}


/* s += the four bytes of w times xv (one dependent FMA chain) */
__device__ static inline float fma_bytes(uint32_t w, float4 xv, float s) {
    s = fmaf((float)(w & 0xFFu), xv.x, s);
    s = fmaf((float)((w >> 8) & 0xFFu), xv.y, s);
    s = fmaf((float)((w >> 16) & 0xFFu), xv.z, s);
    return fmaf((float)(w >> 24), xv.w, s);
}

/* s + the fp16 half h (0: bits 0-15, 1: bits 16-31) of p times x, in one v_fma_mix_f32 */
template <int H>
__device__ static inline float fma_mix_half(uint32_t p, float x, float s) {
    float r;
    if constexpr (H == 0)
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(p), "v"(x), "v"(s));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=v"(r) : "v"(p), "v"(x), "v"(s));
    return r;
}

/* Q4 word w (bytes b0..b3: low nibbles elements 4d..4d+3, high nibbles 16+4d..16+4d+3) into
   two chains: a += u_lo * xl, b += 16 u_hi * xh, both scaled by 2^-24. A nibble masked into
   a 16-bit half is the fp16 subnormal u * 2^-24 (16u * 2^-24 for the high nibble), exact,
   which v_fma_mix_f32 widens and multiplies in place: four masks and a shift per eight
   weights instead of eight byte conversions. The product u * 2^-24 * x is exact and every
   value of the chain is the unscaled one times 2^-24, so the sums round as the unscaled ones
   do while they stay above 2^-126 in magnitude (subnormals are kept: 16/64-bit and 32-bit
   denormal modes on). */
__device__ static inline void fma_nibbles(uint32_t w, float4 xl, float4 xh, float &a, float &b) {
    const uint32_t q = w >> 8;
    const uint32_t l02 = w & 0x000F000Fu, h02 = w & 0x00F000F0u;   /* bytes 0 and 2 */
    const uint32_t l13 = q & 0x000F000Fu, h13 = q & 0x00F000F0u;   /* bytes 1 and 3 */
    a = fma_mix_half<0>(l02, xl.x, a);
    a = fma_mix_half<0>(l13, xl.y, a);
    a = fma_mix_half<1>(l02, xl.z, a);
    a = fma_mix_half<1>(l13, xl.w, a);
    b = fma_mix_half<0>(h02, xh.x, b);
    b = fma_mix_half<0>(h13, xh.y, b);
    b = fma_mix_half<1>(h02, xh.z, b);
    b = fma_mix_half<1>(h13, xh.w, b);
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
#pragma unroll
            for (int i = 0; i < MC; i++)
                fma_nibbles(wd[d], *(const float4 *)(xb + i * ncol + 4 * d),
                            *(const float4 *)(xb + i * ncol + 16 + 4 * d), a[i], b[i]);
        }
#pragma unroll
        for (int i = 0; i < MC; i++) s[i] = (a[i] + b[i]) * 0x1p24f;
    }
    /* the same sum for one token whose staged block (eight float4: x[0..15], then
       x[16..31]/16) is held in registers, so that one read of it serves many rows */
    __device__ float dots_reg(const float4 *xr) const {
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; d++) fma_nibbles(wd[d], xr[d], xr[4 + d], a, b);
        return (a + b) * 0x1p24f;
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
    __device__ float dots_reg(const float4 *xr) const {
        const uint32_t wd[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d += 2) {
            a = fma_bytes(wd[d], xr[d], a);
            b = fma_bytes(wd[d + 1], xr[d + 1], b);
        }
        return a + b;
    }
};

/* ---- one token's gate/up GEMV over block columns shared by lane groups
 * A workgroup of GW wavefronts computes 64 rows (rows r0..r0+31 of two matrices) over
 * nb = GW * B block columns. Wavefront w takes columns w*B .. w*B+B-1; its lanes form B groups
 * of LG = 64 / B lanes, group g = lane / LG taking column w*B + g, and lane i = lane % LG of
 * the group the B row-blocks idx = i + LG*k (k < B) of the 64 rows (idx < 32: matrix 0, row
 * r0 + idx; else matrix 1, row r0 + idx - 32). A lane reads its column's staged activations
 * from LDS once and uses them for all B rows: LDS returns 1/B of the bytes of one row per
 * lane. The B partial sums of each lane are then reduced over the B groups by recursive
 * halving (partner lane ^ (LG << t), keeping the half given by bit t of g), after which
 * lane l holds the wavefront's sum for row idx = l, the order the rows had when every lane
 * took one row. A lane's loads: for fixed k the LG lanes of a group read LG consecutive rows
 * of one column, one contiguous span of the row-tiled layout.
 * NR < 32 rows per matrix (NR a multiple of LG): the 2*NR rows are the U = 2*NR/LG
 * row-blocks k < U (idx < NR: matrix 0, row r0 + idx; else matrix 1, row r0 + idx - NR), the
 * partial sums k >= U are zero, and lanes l >= 2*NR end with zero. With NR = 24 and B = 8 a
 * workgroup's share of F = 768 rows spreads 8 experts over 256 workgroups, where NR = 32 leaves
 * 192 and the loads and conversions of 64 rows on each CU that has one. */
template <int B, int NR>
__device__ constexpr int gu_units() {
    static_assert(NR == 32 || (NR < 32 && NR % (WAVE / B) == 0),
                  "rows of a lane group in one matrix");
    return NR == 32 ? B : 2 * NR / (WAVE / B);
}

template <int ENC, int B, int NR = 32>
__device__ static inline void gu_load(const uint8_t *M0, size_t mat_bytes, size_t payload_plane,
                                      int r0, int nb, WBlk<ENC> (&wv)[B], uint16_t (&sv)[B]) {
    constexpr int LG = WAVE / B, U = gu_units<B, NR>();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane / LG, i = lane % LG;
    const int b = w * B + g;
    size_t t[U];
    const uint8_t *M[U];
#pragma unroll
    for (int k = 0; k < U; k++) {
        const int idx = i + LG * k;
        M[k] = M0 + (idx / NR) * mat_bytes;
        t[k] = cpg_tile_index(r0 + idx % NR, b, nb);
    }
#pragma unroll
    for (int k = 0; k < U; k++) sv[k] = ((const uint16_t *)(M[k] + payload_plane))[t[k]];
#pragma unroll
    for (int k = 0; k < U; k++) wv[k].load(M[k], t[k]);
}

/* A workgroup barrier for LDS data only: this wavefront's LDS operations complete
   (lgkmcnt(0)), then s_barrier. Global loads in flight are not waited for, as __syncthreads()
   would (vmcnt(0)): a register such a load fills is waited for where it is first used, so
   work on the loads that have landed overlaps the ones still in flight. The memory clobbers
   keep the compiler's own memory accesses on their side of the barrier. */
__device__ static inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);          /* lgkmcnt(0); vmcnt, expcnt at their maxima */
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* LDS written by some lanes of a wavefront, then read by others of the same wavefront:
   its LDS operations execute in order, the compiler must only not reorder them. */
__device__ static inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

/* fp16 bits -> fp32 with the hardware conversion: the same value as cpg_f16_to_f32 for every
   non-NaN input (subnormals included), one instruction */
__device__ static inline float f16_to_f32_hw(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

/* The staged token of the grouped GEMV: block b's 32 activations (stage_put's order, the Q4
   high half scaled by 1/16) at xs[b * GU_XB ..], GU_XB = 36 floats, and the block sums at
   bs[b]. The padding puts the lane groups' blocks, read at once, in distinct LDS banks (a
   stride of 32 floats would send all eight to the same banks). */
#define GU_XB 36

/* One float4 (elements 4*k4..4*k4+3, of block k4 / 8) into that layout, the block sum formed
   as stage_put forms it; the eight float4 of a block are on eight consecutive lanes. All
   lanes of the wavefront must call it. */
template <int ENC>
__device__ static inline void gu_stage(float *xs, float *bs, int k4, float4 v, bool valid) {
    float s = ((v.x + v.y) + v.z) + v.w;
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_QUAD_1032, 0xf, 0xf, false));
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_QUAD_2301, 0xf, 0xf, false));
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_ROW_HALF_MIRROR, 0xf, 0xf, false));
    if (valid) {
        if ((k4 & 7) == 0) bs[k4 >> 3] = s;
        if (ENC == CPG_ENC_Q4 && (k4 & 7) >= 4)
            v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
        *(float4 *)(xs + (k4 >> 3) * GU_XB + 4 * (k4 & 7)) = v;
    }
}

/* the wavefront's partial sum for row idx = lane (see gu_load): xs, bs the staged token
   (gu_stage) */
template <int ENC, int B, int NR = 32>
__device__ static inline float gu_dots(const WBlk<ENC> (&wv)[B], const uint16_t (&sv)[B],
                                       const float *xs, const float *bs) {
    constexpr int LG = WAVE / B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane / LG;
    const int b = w * B + g;
    float4 xr[8];
#pragma unroll
    for (int d = 0; d < 8; d++) xr[d] = ((const float4 *)(xs + b * GU_XB))[d];
    const float bsb = bs[b];
    float v[B];
#pragma unroll
    for (int k = 0; k < B; k++)     /* d * (sum u*x - c * sum x), as row_dots_mc's first block */
        v[k] = k < gu_units<B, NR>()
                   ? fmaf(f16_to_f32_hw(sv[k]), fmaf(-WBlk<ENC>::offset, bsb, wv[k].dots_reg(xr)),
                          0.0f)
                   : 0.0f;
#pragma unroll
    for (int t = B / 2, sh = LG * B / 2; t >= 1; t >>= 1, sh >>= 1) {
        const bool up = (lane & sh) != 0;
#pragma unroll
        for (int u = 0; u < t; u++) {
            const float send = up ? v[u] : v[t + u], keep = up ? v[t + u] : v[u];
            v[u] = keep + __shfl_xor(send, sh);
        }
    }
    return v[0];
}

/* LDS floats of the grouped GEMV's staged token for nb blocks (gu_stage) */
__host__ __device__ static inline int gu_lds_floats(int nb) { return GU_XB * nb + nb; }

/* acc[i] = dot product of this lane's row (blocks b0 .. b0+nbw-1 of the staged range, in
   registers) with staged token i < MC. Blocks are added in order, each corrected and
   scaled. */
template <int ENC, int MC, int BPW = MAX_BPW>
__device__ static inline void row_dots_mc(const WBlk<ENC> *wv, const float *dv, int b0, int nbw,
                                          const float *xs, const float *bsum, int ncol, int nb,
                                          float *acc) {
#pragma unroll
    for (int j = 0; j < BPW; j++)
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

template <int ENC, int BPW>
__device__ static inline void row_dots(const WBlk<ENC> *wv, const float *dv, int b0, int nbw,
                                       const float *xs, const float *bsum, int ncol, int nb,
                                       int mc, float *acc) {
    switch (mc) {
    case 1: row_dots_mc<ENC, 1, BPW>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    case 2: row_dots_mc<ENC, 2, BPW>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    case 3: row_dots_mc<ENC, 3, BPW>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    default: row_dots_mc<ENC, 4, BPW>(wv, dv, b0, nbw, xs, bsum, ncol, nb, acc); break;
    }
}

/* h = silu(g) * u, kernels.c:416 and qwen3_moe.c:219 */
__device__ static inline float swiglu(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, cpg_expf(-g))), u);
}
/* the same, with the expf table read from `tab` (an LDS copy) */
__device__ static inline float swiglu_t(float g, float u, const uint64_t *tab) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, cpg_expf_tab(-g, tab))), u);
}

/* Stage mc token vectors of ncol floats into LDS: xs[i*ld + k] = get(i, k/4) (a float4; ld
   defaults to ncol),
   the second half of every 32-element block pre-scaled by 1/16 for Q4; bs[i*nb + b] = the
   block's sum (unscaled). One float4 per thread per pass; the eight float4 of a block are in
   eight consecutive lanes, summed by xor shuffles. Ends with a barrier. ncol % 32 == 0. */
/* One float4 (elements 4*k4..4*k4+3 of token i) into the staged layout: the block sum from
   the eight consecutive lanes holding the block (the caller's lanes must be laid out so), the
   Q4 high half scaled by 1/16. All lanes of the wavefront must call it. */
template <int ENC>
__device__ static inline void stage_put(float *xs, float *bs, int ld, int nb, int i, int k4,
                                        float4 v, bool valid) {
    float s = ((v.x + v.y) + v.z) + v.w;
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_QUAD_1032, 0xf, 0xf, false));
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_QUAD_2301, 0xf, 0xf, false));
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), DPP_ROW_HALF_MIRROR, 0xf, 0xf, false));
    if (valid) {
        if ((k4 & 7) == 0) bs[i * nb + (k4 >> 3)] = s;
        if (ENC == CPG_ENC_Q4 && (k4 & 7) >= 4)
            v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
        *(float4 *)(xs + i * ld + 4 * k4) = v;
    }
}

/* Blocks bstart .. bstart+BPW-1 of `row` (indices clamped to bmax, so every address is valid;
   the caller uses only its own nbw blocks): the fp16 scales are loaded first and the payloads
   after them, so converting the scales waits for the scale loads only and every payload is
   still in flight. */
template <int ENC, int BPW>
__device__ static inline void load_row_blocks(const uint8_t *M, size_t payload_plane, int row,
                                              int bstart, int bmax, int nb, WBlk<ENC> *wv,
                                              float *dv) {
    const uint16_t *S = (const uint16_t *)(M + payload_plane);
    size_t t[BPW];
    uint16_t sr[BPW];
#pragma unroll
    for (int q = 0; q < BPW; q++) t[q] = cpg_tile_index(row, min(bstart + q, bmax), nb);
#pragma unroll
    for (int q = 0; q < BPW; q++) sr[q] = S[t[q]];
#pragma unroll
    for (int q = 0; q < BPW; q++) wv[q].load(M, t[q]);
#pragma unroll
    for (int q = 0; q < BPW; q++) dv[q] = cpg_f16_to_f32(sr[q]);
}

/* load_row_blocks with the scales left as raw fp16 bits (converted by the caller at use), so
   that nothing waits on these loads until the caller needs them */
template <int ENC, int BPW>
__device__ static inline void load_row_blocks_raw(const uint8_t *M, size_t payload_plane, int row,
                                                  int bstart, int bmax, int nb, WBlk<ENC> *wv,
                                                  uint16_t *sr) {
    const uint16_t *S = (const uint16_t *)(M + payload_plane);
    size_t t[BPW];
#pragma unroll
    for (int q = 0; q < BPW; q++) t[q] = cpg_tile_index(row, min(bstart + q, bmax), nb);
#pragma unroll
    for (int q = 0; q < BPW; q++) sr[q] = S[t[q]];
#pragma unroll
    for (int q = 0; q < BPW; q++) wv[q].load(M, t[q]);
}

template <int ENC, int NT, typename Get>
__device__ static inline void stage_tokens(float *xs, float *bs, int ncol, int mc, Get get,
                                           int ld = 0) {
    const int q = ncol / 4, nb = ncol / 32;
    if (ld == 0) ld = ncol;
    for (int idx = threadIdx.x; idx < ((mc * q + 63) & ~63); idx += NT) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const int i = idx / q, k4 = idx - i * q;
        if (idx < mc * q) v = get(i, k4);
        stage_put<ENC>(xs, bs, ld, nb, i, k4, v, idx < mc * q);
    }
    lds_barrier();                               /* weight loads in flight are not waited for */
}

/* 1/sqrtf(ss/D + eps) for one row x of D floats (D % 4 == 0), ss = sum x^2 accumulated in
   double (kernels.c:408-413 up to the order of that sum): threads 0..255 of the workgroup
   take float4 i = tid, tid + 256, ... in order, then the four wavefronts are combined in a
   fixed order, so every caller gets the same bits. All threads of the workgroup call it;
   part: 4 doubles of LDS. */
/* thread tid < 256's term of rms_inv_row's sum: float4s tid, tid + 256, ... in order */
__device__ static inline double rms_sq4(double ss, float4 v) {
    return ss + ((double)__fmul_rn(v.x, v.x) + (double)__fmul_rn(v.y, v.y) +
                 (double)__fmul_rn(v.z, v.z) + (double)__fmul_rn(v.w, v.w));
}

__device__ static float rms_inv_from(double ss, int D, float eps, double *part);

__device__ static float rms_inv_row(const float *__restrict__ x, int D, float eps, double *part) {
    const int tid = threadIdx.x;
    const float4 *x4 = (const float4 *)x;
    double ss = 0.0;
    if (tid < 256)
        for (int i = tid; i < D / 4; i += 256) ss = rms_sq4(ss, x4[i]);
    return rms_inv_from(ss, D, eps, part);
}

/* The rest of rms_inv_row, given each thread's term (zero for tid >= 256). */
__device__ static float rms_inv_from(double ss, int D, float eps, double *part) {
    const int tid = threadIdx.x;
    ss = wave_sum_d(ss);
    if (tid < 256 && (tid & 63) == 0) part[tid >> 6] = ss;
    lds_barrier();                               /* LDS only: global loads in flight go on */
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    lds_barrier();                               /* part may be reused after this */
    return __fdiv_rn(1.0f, cpg_sqrt_rn(__fadd_rn(__fdiv_rn((float)ss, (float)D), eps)));
}

/* ---- cross-workgroup handoff
 * A result that another workgroup of the same launch reads is written with an agent-scope
 * store (written through this XCD's L2) and read with an agent-scope load; the arrival
 * counter is an agent-scope atomic. A writer waits until its stores have completed before it
 * counts itself in, and the last arriver issues its loads only after it has seen the count.
 * No cache-wide write-back or invalidate is involved. */
template <typename V> __device__ static inline void st_agent(V *p, V v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V> __device__ static inline V ld_agent(const V *p) {
    return __hip_atomic_load(const_cast<V *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* 16 bytes at base + off written by another workgroup of this launch: one buffer load with
   the agent-scope coherence bit (sc1, the form of an agent-scope atomic load), so a vector
   of them issues back to back instead of one round trip each. */
typedef int v4i_t __attribute__((ext_vector_type(4)));
__device__ static inline v4i_t ld_agent16(const void *base, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7fffffff, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}
__device__ static inline int arrive(int *ctr) {
    return __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* this thread's memory operations have completed (vmcnt, expcnt, lgkmcnt all zero) */
__device__ static inline void mem_done() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
/* Whole workgroup: count this workgroup in at *ctr; true in the workgroup that brings the
   count to `last` + 1, which also resets the counter for the next launch. */
__device__ static inline bool last_arriver(int *ctr, int last, int *flag_lds) {
    mem_done();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = arrive(ctr);
        if (old == last) st_agent(ctr, 0);
        *flag_lds = old == last;
    }
    __syncthreads();
    return *flag_lds != 0;
}

#endif
