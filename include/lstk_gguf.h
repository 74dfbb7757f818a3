/* lstk_gguf.h - C ABI of the GGUF reader that feeds the expert pool and the forward pass.
 *
 * Replaces the reference's model loading for this path:
 *   GgufModel::open / has / get_int / get_float / get_str / info   src/gguf_model.cpp:14-103
 *   qwen3_load_hparams                                             src/qwen3.cpp:16-45 (qwen3moe keys)
 *   qwen3_map_weights (tensor names, tied output)                  src/qwen3.cpp:52-89
 *   qwen3_expert_infos (expert tensors, shape checks)              src/qwen3.cpp:92-109
 * The file is memory-mapped read-only; a tensor's `data` points into the mapping, so the expert
 * tensors go to lstk_pool_create as host pointers without a copy (expert e of a stacked tensor starts
 * at data + e * nbytes / ne[2], GgufTensorInfo::expert_stride, src/gguf_model.h:28).
 * GGUF versions 2 and 3 are read (little-endian). Every read is bounds-checked: a truncated or
 * malformed file is reported, never read past.
 */
#ifndef LSTK_GGUF_H
#define LSTK_GGUF_H

#include "lstk_qwen3.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lstk_gguf lstk_gguf;

/* One tensor of the index (GgufTensorInfo, src/gguf_model.h:20-29). ne is in ggml order (ne[0] is the
 * contiguous dimension); unused dimensions are 1. */
typedef struct lstk_gguf_tensor {
    const char *name;
    int32_t type;   /* ggml type id */
    int32_t n_dims;
    int64_t ne[4];
    uint64_t offset; /* from the start of the file */
    uint64_t nbytes;
    const void *data; /* in the read-only mapping; valid until lstk_gguf_close */
} lstk_gguf_tensor;

/* GgufModel::open: maps the file and parses the header, the metadata and the tensor index. Fails with
 * LSTK_E_IO when the file cannot be opened or mapped, LSTK_E_INVALID when it is not a readable GGUF
 * (bad magic, version 1, truncated, a tensor outside the file, an unknown tensor type) or has no
 * general.architecture. */
int lstk_gguf_open(const char *path, lstk_gguf **out);
void lstk_gguf_close(lstk_gguf *g);

const char *lstk_gguf_arch(const lstk_gguf *g); /* general.architecture */
int lstk_gguf_version(const lstk_gguf *g);
int lstk_gguf_alignment(const lstk_gguf *g);   /* general.alignment, default 32 */

/* Metadata lookups (GgufModel::has / get_int / get_float / get_str): get_int accepts every integer
 * type and bool, get_float also f32 and f64, get_str strings only; an absent key (or, for get_str, a
 * key of another type) gives `def`. */
int lstk_gguf_has(const lstk_gguf *g, const char *key);
int64_t lstk_gguf_get_int(const lstk_gguf *g, const char *key, int64_t def);
double lstk_gguf_get_float(const lstk_gguf *g, const char *key, double def);
const char *lstk_gguf_get_str(const lstk_gguf *g, const char *key, const char *def);

int lstk_gguf_n_tensors(const lstk_gguf *g);
int lstk_gguf_tensor_at(const lstk_gguf *g, int i, lstk_gguf_tensor *out);
/* GgufModel::info: LSTK_E_INVALID (and a message naming the tensor) when absent. */
int lstk_gguf_find_tensor(const lstk_gguf *g, const char *name, lstk_gguf_tensor *out);

/* qwen3_load_hparams for a qwen3moe file (the keys and defaults of src/qwen3.cpp:21-33), with n_vocab
 * from token_embd.weight (src/qwen3.cpp:87). Dense (non-MoE) architectures are rejected: this path is
 * the MoE model. */
int lstk_gguf_qwen3_hparams(const lstk_gguf *g, lstk_qwen3_hparams *hp);

/* qwen3_expert_infos: for each of hp->n_layer layers, the types and mapped host pointers of
 * blk.L.ffn_{up,gate,down}_exps.weight, ready for lstk_pool_create. The shapes must match hp (up and
 * gate [n_embd, n_ff_exp, n_expert], down [n_ff_exp, n_embd, n_expert]) and the types must be ones the
 * pool stores (Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K): anything else fails with a message naming the
 * layer, tensor and type. */
int lstk_gguf_qwen3_experts(const lstk_gguf *g, const lstk_qwen3_hparams *hp, lstk_expert_layer *layers);

/* Dense tensors for the forward pass, which multiplies F16 matrices: n values of a tensor of ggml type
 * `type` at src (GGUF bytes, n a multiple of the type's block) to fp16 at dst, round to nearest even.
 * F32, F16, Q8_0 (d q), Q2_K (d sc q - dmin m, 2-bit q, 4-bit sc / m per 16 values), Q3_K (d (sc - 32) (q - 4 h'),
 * 3-bit q, 6-bit sc per 16), Q4_K (d sc q - dmin m), Q5_K (d sc (q + 16 h) - dmin m) and Q6_K (d sc (q - 32),
 * sc a signed 8-bit scale per 16 values) - ggml's dequantize_row_* for each format (the reference maps such
 * tensors into its graph whatever their type, src/qwen3.cpp:52-89). Each value is formed in f32 in ggml's
 * order, then rounded to fp16 once; the forward pass then differs from ggml's quantized dot products by the
 * fp16 rounding of the weights. LSTK_E_INVALID for any other type or a bad n. Host memory only. */
int lstk_dequant_f16(int type, const void *src, size_t n, uint16_t *dst);

#ifdef __cplusplus
}
#endif

#endif /* LSTK_GGUF_H */
