/* qw3_engine.h — device state behind the block / port interface (qwen3_moe.h): one entry per
 * mapped model file, holding the payload in HBM and, per bound layer, the row-tiled weights
 * and the cpg.h layer descriptors the kernels take. Internal to the engine sources. */
#ifndef QW3_ENGINE_H
#define QW3_ENGINE_H
#include "cpg.h"
#include "cpw4.h"
#include "qwen3_moe.h"

#define QW3_MAX_POS 8192        /* RoPE table positions kept on the device */

typedef struct {
    int ready;
    cpg_attn_layer a;
    cpg_moe_layer m;
    void *wqkv, *wo, *experts;  /* device allocations owned by the layer */
} qw3_dev_layer;

typedef struct {
    int used;
    const uint8_t *map;         /* host mapping (or a caller's image) and its length */
    size_t map_len;
    int owns_map;               /* 1: munmap at release */
    cpw4_file f;
    uint8_t *dev;               /* the payload [off_data, map_len) in HBM */
    float *rope;                /* QW3_MAX_POS x head_dim/2 (cos, sin) */
    float theta, eps;
    int head_dim, n_layers, topk;
    qw3_dev_layer *lay;         /* [n_layers] */
    /* scratch of the host-buffer entry points, grown on demand */
    int cap_T;
    float *dx, *dattn, *dmlp, *drouter;
    int *dtopk;
    cpg_moe_ws *mws;
    cpg_attn_ws *aws;
} qw3_state;

int qw3_ensure_device(void);
qw3_state *qw3_state_of(const void *map);
/* the device copy of a host pointer into the mapped payload, or NULL */
const void *qw3_dev_ptr(const qw3_state *st, const void *host);
/* the device descriptors of layer `layer` (built on first use from the mapping) */
int qw3_dev_layer_get(qw3_state *st, int layer, qw3_dev_layer **out);
/* scratch for T tokens */
int qw3_scratch(qw3_state *st, int T);

#endif
