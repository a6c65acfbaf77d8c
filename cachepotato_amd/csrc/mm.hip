/* mm.hip — out = W . x for one matrix in the CPW1 v4 layout (format/SPEC.md:149-197), the
 * device side of qwen3_mm (engine/blocks/qwen3_moe.c:36-40).
 *
 * f32 (matmul_wx, engine/kernels/kernels.c:84-95): one lane per row runs the reference's
 * serial add chain of separately rounded products — bit-identical to the CPU.
 * Q4_0 / Q8_0 (matmul_wx_q4 :514-540, matmul_wx_q8 :368-396): one wavefront per row, lanes
 * over the row's blocks, fp32 FMA, then a fixed-order wavefront reduction. The CPU's own
 * results depend on its thread count; these agree with both to fp32 accumulation error.
 */
#include "cpg_internal.h"

__global__ __launch_bounds__(64) void k_mm_f32(const float *__restrict__ w,
                                               const float *__restrict__ x, int n_in, int n_out,
                                               float *__restrict__ out) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i >= n_out) return;
    const float *row = w + (size_t)i * n_in;
    float acc = 0.0f;
    for (int k = 0; k < n_in; k++) acc = __fadd_rn(acc, __fmul_rn(row[k], x[k]));
    out[i] = acc;
}

template <int ENC>
__global__ __launch_bounds__(256) void k_mm_q(const uint8_t *__restrict__ w,
                                              const float *__restrict__ x, int n_in, int n_out,
                                              float *__restrict__ out) {
    constexpr int BB = ENC == CPG_ENC_Q8 ? 34 : 18;
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n_out) return;
    const int nb = n_in / 32;
    const uint8_t *row = w + (size_t)i * nb * BB;
    float acc = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint8_t *blk = row + (size_t)b * BB;
        const float d = cpg_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        const float *xb = x + b * 32;
        float s = 0.0f;
        if (ENC == CPG_ENC_Q8) {
            for (int k = 0; k < 32; k++) s = fmaf((float)(int8_t)blk[2 + k], xb[k], s);
        } else {
            for (int k = 0; k < 16; k++) {
                int lo = blk[2 + k] & 15, hi = blk[2 + k] >> 4;
                lo = lo > 7 ? lo - 16 : lo;
                hi = hi > 7 ? hi - 16 : hi;
                s = fmaf((float)lo, xb[k], s);
                s = fmaf((float)hi, xb[k + 16], s);
            }
        }
        acc = fmaf(d, s, acc);
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) out[i] = acc;
}

extern "C" int cpg_mm(int enc, const void *w, const float *x, int n_in, int n_out, float *out) {
    CPG_REQUIRE_INIT();
    if (!w || !x || !out || n_in <= 0 || n_out <= 0) { cpg_set_error("cpg_mm: bad arguments"); return -1; }
    if (enc == CPG_ENC_F32) {
        hipLaunchKernelGGL(k_mm_f32, dim3((n_out + 63) / 64), dim3(64), 0, g_cpg.stream,
                           (const float *)w, x, n_in, n_out, out);
    } else if (enc == CPG_ENC_Q4 || enc == CPG_ENC_Q8) {
        if (n_in % 32) { cpg_set_error("cpg_mm: n_in %d is not a multiple of 32", n_in); return -1; }
        if (enc == CPG_ENC_Q4)
            hipLaunchKernelGGL(k_mm_q<CPG_ENC_Q4>, dim3((n_out + 3) / 4), dim3(256), 0,
                               g_cpg.stream, (const uint8_t *)w, x, n_in, n_out, out);
        else
            hipLaunchKernelGGL(k_mm_q<CPG_ENC_Q8>, dim3((n_out + 3) / 4), dim3(256), 0,
                               g_cpg.stream, (const uint8_t *)w, x, n_in, n_out, out);
    } else {
        cpg_set_error("cpg_mm: unknown encoding %d", enc);
        return -1;
    }
    CPG_LAUNCH_CHECK("cpg_mm");
    return 0;
}
