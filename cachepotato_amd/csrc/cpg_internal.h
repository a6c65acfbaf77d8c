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

#define CPG_REQUIRE_INIT()                                                              \
    do {                                                                                \
        if (!g_cpg.ready) { cpg_set_error("cpg_init has not been called"); return -7; } \
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

#endif
