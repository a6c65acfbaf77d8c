/* cpg_internal.h — shared between the HIP translation units of libcachepotato_amd. */
#ifndef CPG_INTERNAL_H
#define CPG_INTERNAL_H
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "cpg.h"
#include "cpg_math.h"

/* one context per process (cpg_init) */
struct cpg_context {
    int ready;
    int device;
    hipStream_t stream;
};
extern cpg_context g_cpg;

void cpg_set_error(const char *fmt, ...);

/* The static scratch (cpg_moe_forward_noalloc): this context's device address of a fixed
   device array of *bytes bytes, zero when the context was created; null before cpg_init. */
#define CPG_STATIC_SCRATCH_BYTES ((size_t)4 << 20)
#define CPG_MAX_DEVICES 64
#define MAX_E 256           /* experts a MoE layer may have */
void *cpg_static_scratch(size_t *bytes);

#define CPG_HIP(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            cpg_set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),        \
                          __FILE__, __LINE__);                                          \
            return -7;                                                                  \
        }                                                                               \
    } while (0)

#define CPG_LAUNCH_CHECK(name)                                                          \
    do {                                                                                \
        hipError_t e_ = hipGetLastError();                                              \
        if (e_ != hipSuccess) {                                                         \
            cpg_set_error("launch of %s failed: %s", name, hipGetErrorString(e_));      \
            return -7;                                                                  \
        }                                                                               \
    } while (0)

/* CPG_DEBUG_ERRORS=1 in the environment: every entry point that checks for the context also
   reports, on stderr, a HIP error left pending by an earlier call (hipGetLastError), naming
   the entry point that found it. */
void cpg_debug_pending(const char *where);
#define CPG_REQUIRE_INIT()                                                              \
    do {                                                                                \
        if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return -7; } \
        cpg_debug_pending(__func__);                                                    \
    } while (0)

static inline size_t cpg_round256(size_t n) { return (n + 255) & ~(size_t)255; }

/* Row-tiled matrix geometry (see cpg.h): payload bytes per (row, block) and plane sizes. */
static inline int cpg_payload_bytes(int enc) { return enc == CPG_ENC_Q8 ? 32 : 16; }
static inline int cpg_v4_block_bytes(int enc) { return enc == CPG_ENC_Q8 ? 34 : 18; }
static inline size_t cpg_payload_plane(int enc, int rows, int cols) {
    return cpg_round256((size_t)rows * (cols / 32) * cpg_payload_bytes(enc));
}
static inline size_t cpg_scale_plane(int rows, int cols) {
    return cpg_round256((size_t)rows * (cols / 32) * 2);
}

/* index of (row, block) in a plane */
__host__ __device__ static inline size_t cpg_tile_index(int row, int b, int nb) {
    return ((size_t)(row >> 6) * nb + b) * 64 + (row & 63);
}

/* Kernel timing (cpg_moe_timing): while enabled, LAUNCH binds an event pair to the dispatch
   (hipExtLaunchKernel), so the pair's elapsed time is the kernel's own execution. */
#include <hip/hip_ext.h>
hipEvent_t *cpg_timing_pair(int slot);
#define LAUNCH(slot, kern, grid, block, smem, ...)                                         \
    do {                                                                                  \
        hipEvent_t *ev_ = cpg_timing_pair(slot);                                          \
        if (ev_)                                                                          \
            hipExtLaunchKernelGGL(kern, grid, block, smem, g_cpg.stream, ev_[0], ev_[1], 0, \
                                  __VA_ARGS__);                                           \
        else                                                                              \
            hipLaunchKernelGGL(kern, grid, block, smem, g_cpg.stream, __VA_ARGS__);       \
        CPG_LAUNCH_CHECK(#kern);                                                          \
    } while (0)

/* prefill.hip: the MFMA grouped expert GEMMs for many tokens */
int cpg_prefill_max_chunks(int T, int K, int E);
bool cpg_prefill_shape_ok(int D, int F);
/* scratch: cpg_prefill_scratch_bytes (the hi/lo f16 planes of xn, then those of h).
   prepared: the routing step has written the chunk list (pf_chunk_list) and the planes of
   xn; otherwise they are formed here from grp_cnt and xn. */
size_t cpg_prefill_scratch_bytes(int T, int D, int K, int F);
/* prefill.hip: the dense MFMA product from hi/lo planes already at the start of scratch
   (T rows of n_in halves each, hi then lo); with sum == 0 and more than one k part the parts
   are left in *parts (ks of them, T * n_out floats each, to be added in order) */
int cpg_dense_from_planes(int enc, const void *w, int n_in, int n_out, int T, void *scratch,
                          float *out, int sum, const float **parts, int *ks);
/* sel not null (cpg_prefill_sel_ok): the GEMMs take each expert's pairs from the T * K
   selections sel themselves (grp_*, list_*, chunk_* unused), h and y indexed by pair, and
   the number of experts with pairs is written to *ngroups */
bool cpg_prefill_sel_ok(int T, int K, int E);
int cpg_prefill_experts(const cpg_moe_layer *L, int T, const float *xn, const float *wt,
                        const int *grp_expert, const int *grp_off, const int *grp_cnt,
                        const int *list_tok, const int *list_pair, int *chunk_grp,
                        int *chunk_m0, void *scratch, float *y, float *mlp, float *xres,
                        const float *attn, int prepared, const int *sel, int *ngroups);
/* out (T rows of n_out) = W . x for a row-tiled Q4_0/Q8_0 matrix W on MFMA, the k range split
   into parts summed in a fixed order; scratch: cpg_dense_scratch_bytes (the hi/lo f16 planes of
   x and the parts) */
bool cpg_dense_shape_ok(int n_in, int n_out);
size_t cpg_dense_scratch_bytes(int T, int n_in, int n_out);
int cpg_dense_mfma(int enc, const void *w, int n_in, int n_out, const float *x, int T,
                   void *scratch, float *out);

#endif