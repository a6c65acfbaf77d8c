/* cpw4.h — CPW1 v4 region files (format/SPEC.md §3-§8): a validating parser, a streaming
 * writer and a synthetic Qwen3 model writer, in C11 (the reference's parser is
 * engine/blocks/qwen3_moe.c:296-459 and its writer format/v4_writer.py).
 *
 * The byte layout follows the reference writer (format/v4_writer.py:183-299), which is what
 * the reference loader reads (engine/blocks/qwen3_moe.c:296-459):
 *   header (88 B): "CPW4", version 4, header_bytes 88, flags, n_tensors, n_blocks, n_regions,
 *     n_encodings, off_encodings, off_tensors, off_blocks, off_regions, off_data, 4 x u32 0
 *   encoding: u32 id, u8 kind, u8 scalar, u16 group, u16 block_bytes, u8 sub, u8 flags,
 *     u8 align, string name
 *   tensor:   string name, u32 encoding index, u8 rank, u32 dims[rank], u64 offset, u64 length,
 *     u32 block, u16 role            (offset counted from off_data, as the writer emits it)
 *   block:    u8 kind, u32 layer, u8 n_refs, u32 refs[], u8 n_params, u32 params[]
 *   region:   u64 offset, u64 length, u32 tensor_lo, u32 tensor_hi, u8 kind, u16 slot,
 *     u32 member_lo, u32 member_hi, u64 digest (CRC-32 of the region's bytes)
 *   strings are u16 length + bytes. Scalar code 3 is Q8_0, 4 is Q4_0 (the writer's and the
 *   loader's convention, v4_writer.py:207-210, qwen3_moe.c:390-392).
 */
#ifndef CPW4_H
#define CPW4_H
#include <stddef.h>
#include <stdint.h>

#define CPW4_MAGIC 0x34575043u
#define CPW4_HDR_BYTES 88u
#define CPW4_MAX_ENC 64

/* block kinds, tensor roles, region kinds (SPEC §5, §7, §8) */
enum { CPW4_BLK_EMBED = 0x01, CPW4_BLK_NORM = 0x02, CPW4_BLK_ATTN = 0x10, CPW4_BLK_FFN = 0x11,
       CPW4_BLK_MOE = 0x20 };
enum { CPW4_ROLE_OTHER = 0, CPW4_ROLE_EMBED, CPW4_ROLE_NORM, CPW4_ROLE_ATTN, CPW4_ROLE_ROUTER,
       CPW4_ROLE_EXPERT, CPW4_ROLE_SHARED, CPW4_ROLE_DENSE, CPW4_ROLE_HEAD };
enum { CPW4_REG_TENSOR = 0, CPW4_REG_EXPERT = 1, CPW4_REG_GROUP = 2, CPW4_REG_PINNED = 3 };

typedef struct {
    uint8_t kind, scalar, sub, flags, align;
    uint16_t group, block_bytes;
    int code;               /* QW3_ENC_F32 / Q8 / Q4, or -1 for an encoding the engine lacks */
} cpw4_enc;

typedef struct {
    const char *name;       /* not NUL-terminated: name_len bytes */
    uint16_t name_len;
    uint32_t enc, rank, dims[4], block;
    uint16_t role;
    uint64_t offset, length;  /* offset from off_data */
} cpw4_tensor;

typedef struct {
    uint8_t kind;
    uint32_t layer, n_refs, n_params;
    const uint8_t *refs, *params;   /* little-endian u32 arrays inside the mapping */
} cpw4_block;

typedef struct {
    uint64_t offset, length, digest;
    uint32_t tensor_lo, tensor_hi, member_lo, member_hi;
    uint8_t kind;
    uint16_t slot;
} cpw4_region;

typedef struct {
    const uint8_t *base;
    size_t len;
    uint32_t n_tensors, n_blocks, n_regions, n_enc;
    uint64_t off_enc, off_tensors, off_blocks, off_regions, off_data;
    int n_layers;           /* highest attention block's layer + 1 */
    cpw4_enc enc[CPW4_MAX_ENC];
    cpw4_tensor *tensors;
    cpw4_block *blocks;
    cpw4_region *regions;
} cpw4_file;

/* Parse and validate the tables of a file image (the header, every table inside the file,
   tensors inside the payload, 64-byte aligned, lengths consistent with their encodings, no
   two tensors overlapping; regions inside the payload over valid tensor ranges). Returns 0,
   -2 out of memory, or -3 with the reason in err. */
int cpw4_parse(cpw4_file *f, const uint8_t *base, size_t len, char *err, size_t errlen);
void cpw4_release(cpw4_file *f);
/* read and validate a file (tables, then the Qwen3 geometry): 0 (err receives a one-line
   summary) or the failing check's code */
int cpw4_check_file(const char *path, char *err, size_t errlen);
/* The geometry of a Qwen3-MoE file, checked against every tensor the engine binds.
   Derived from layer 0 (hidden size from ln1.0, head_dim from q_norm.0, heads from Wq.0 and
   Wk.0, experts from Wgate.0, intermediate size from expert.0.0.Wg), top-k from the MoE
   blocks and the vocabulary from lm_head; then every layer's norms [D] / [HD], Wq [H*HD, D],
   Wk and Wv [KV*HD, D], Wo [D, H*HD], Wgate [E, D] and experts Wg, Wu [F, D], Wd [D, F],
   final_norm [D], lm_head [V, D] and the embedding ([>= V, D], or chunks of at most the first
   chunk's rows covering V) must have exactly those shapes, quantised rows whole 32-element
   blocks, norms f32. The reference's loader reads these dims without cross-checks
   (engine/blocks/qwen3_moe.c:318-459); here a file that disagrees is refused before any
   allocation or copy. Returns 0 (also for a file without attention blocks, g zeroed), -3
   on a mismatch or -4 when layer 0 lacks a tensor the geometry is read from, with the reason
   in err. cpw4_check_file applies it after the table checks. */
typedef struct {
    int n_layers, d_model, n_heads, n_kv, head_dim, n_experts, topk, d_exp, vocab;
} cpw4_qwen3_geom;
int cpw4_qwen3_geometry(const cpw4_file *f, cpw4_qwen3_geom *g, char *err, size_t errlen);
/* index of the tensor called `name`, or -1 */
int cpw4_find(const cpw4_file *f, const char *name);
/* payload bytes of tensor i */
static inline const uint8_t *cpw4_data(const cpw4_file *f, int i) {
    return f->base + f->off_data + f->tensors[i].offset;
}
/* CRC-32 (IEEE 802.3, reflected 0xEDB88320, initial and final xor 0xFFFFFFFF) of n bytes,
   continuing from crc (0 to start) */
uint32_t cpw4_crc32(uint32_t crc, const void *p, size_t n);

/* ---- writer */
typedef struct cpw4_writer cpw4_writer;
/* fills tensor `t`'s nbytes of payload */
typedef int (*cpw4_fill_fn)(void *user, int t, uint8_t *dst, size_t nbytes);

cpw4_writer *cpw4_writer_create(void);
void cpw4_writer_destroy(cpw4_writer *w);
/* enc: QW3_ENC_F32 / Q8 / Q4; returns the tensor id or a negative code */
int cpw4_add_tensor(cpw4_writer *w, const char *name, int enc, int rank, const uint32_t *dims,
                    int role);
int cpw4_add_block(cpw4_writer *w, int kind, uint32_t layer, const uint32_t *refs, int n_refs,
                   const uint32_t *params, int n_params);
int cpw4_add_region(cpw4_writer *w, int lo, int hi, int kind, int slot, uint32_t mlo,
                    uint32_t mhi);
/* Write the file: payload in the physical order `order` (a permutation of tensor ids, or
   NULL for table order), each tensor 64-byte aligned, region digests over the bytes written.
   The payload of each tensor comes from fill(), one tensor at a time. */
int cpw4_write(cpw4_writer *w, const char *path, const int *order, cpw4_fill_fn fill,
               void *user, char *err, size_t errlen);

/* ---- synthetic Qwen3-MoE models
 * A random-init model in the reference converter's layout (models/qwen3-30b-a3b/convert.py:
 * 166-242): tensors embed, ln1.L, ln2.L, q_norm.L, k_norm.L, Wq.L, Wk.L, Wv.L, Wo.L, Wgate.L,
 * expert.L.E.{Wg,Wu,Wd}, final_norm, lm_head; an embedding block, one attention and one MoE
 * block per layer with the converter's parameters; one region per expert and one per other
 * tensor; f32 tensors placed before the quantised ones. Values come from the counter-based
 * generator (cpg.h), so the device can regenerate any tensor bit for bit:
 *   expert e of layer l      CPG_STREAM(l, CPG_K_WG/WU/WD, e), sigma 0.02
 *   Wgate.l                  CPG_STREAM(l, CPG_K_WGATE, 0), sigma 0.02
 *   Wq, Wk, Wv, Wo of l      CPG_STREAM(l, CPG_K_ATTN, 0..3), sigma 0.02
 *   ln1, ln2, q_norm, k_norm 1 + N(0, norm_sigma^2): CPG_STREAM(l, CPG_K_NORM, 1..4)
 *   final_norm               CPG_STREAM(n_layers, CPG_K_NORM, 5)
 *   embed                    CPG_STREAM(0, CPG_K_EMBED, 0), sigma embed_sigma (0 means 0.02)
 *   lm_head                  CPG_STREAM(0, CPG_K_HEAD, 0), sigma 0.02
 * out_sigma (0 means 0.02) replaces 0.02 for the two projections that write into the
 * residual stream, Wo and the experts' Wd. With every weight at 0.02, a deep model's hidden
 * states drift to one shared direction: once the positions' values agree, attention averages
 * no longer shrink them, each layer adds a vector of norm ~50 common to every position, and
 * after 48 layers that sum outweighs the token's own embedding row (norm ~0.9), so greedy
 * decoding repeats one token. A larger embed_sigma and an out_sigma scaled like
 * 0.02 / sqrt(2 n_layers) keep the token and its context visible.
 */
typedef struct {
    int n_layers, d_model, n_heads, n_kv, head_dim, n_experts, topk, d_exp, vocab;
    float rope_theta;
    int enc_attn, enc_exp, enc_embed, enc_head;     /* QW3_ENC_F32 / Q8 / Q4 */
    double norm_sigma;
    uint64_t seed;
    double embed_sigma;     /* sigma of the embedding table; 0 selects 0.02 */
    double out_sigma;       /* sigma of Wo and the experts' Wd; 0 selects 0.02 */
} qw3_synth_cfg;
int qwen3_write_synthetic(const char *path, const qw3_synth_cfg *cfg, char *err, size_t errlen);

#endif
