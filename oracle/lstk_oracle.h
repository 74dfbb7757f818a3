/* lstk_oracle.h - CPU oracle for the Qwen3-MoE expert-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker (or the timed CPU baseline). The product path
 * (localstack_amd/) never links or calls it.
 *
 * It restates, in plain C, what localstack's MoE block computes when ggml runs it on the CPU:
 *   router()      src/qwen3.cpp:175-192
 *   moe_apply()   src/qwen3.cpp:197-214, residual add :250 / :287
 *   ExpertStore   src/expert_store.cpp:106-295 (slot bookkeeping only, no I/O)
 *   the forward pass around the MoE block (src/qwen3.cpp:112-171, :223-259): RMSNorm, F16 mat-muls,
 *   NEOX RoPE, fp16 KV cache, attention, output head, for one sequence
 * ggml itself (llama.cpp submodule pinned at 23b0202a189c44a54625aadcb37a946dd1d6278d,
 * docs/llama_cpp_commit.txt:1) is not present, so its kernels are restated from its published
 * algorithm: Q8_0/Q4_K/Q8_K block formats, quantize_row_q8_0 (x86 AVX path: id = 127/amax,
 * round-half-even), quantize_row_q8_K_ref, ggml_vec_dot_q8_0_q8_0, ggml_vec_dot_q4_K_q8_K,
 * ggml_vec_dot_f16 (activations rounded to fp16), soft_max (double-precision sum), argsort
 * (descending), sum_rows (double), swiglu (x / (1 + expf(-x)) * g).
 *
 * What no check in this repository can pin (the reference's arithmetic lives in an absent library):
 *   - ggml's SIMD reduction order inside each dot product (the oracle uses the fixed orders
 *     documented per function; router logits use the 64-lane order the GPU kernel uses);
 *   - ggml's SIMD expf / silu approximations (the oracle calls libm expf);
 *   - whether ggml's CPU flash attention accumulates V in f32 or f16 for an F16 cache (the oracle
 *     accumulates in f32, as the graph requests with GGML_PREC_F32, src/qwen3.cpp:167), and the x86
 *     contraction of RoPE's x0*cos - x1*sin into fused multiply-adds;
 *   - std::sort's order among exactly equal probabilities (the oracle breaks ties to the lower id).
 * Every other function is pinned by the tests listed in tests/test_oracle_*.py.
 */
#ifndef LSTK_ORACLE_H
#define LSTK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK8_0 32
#define OR_QK_K 256

typedef struct {
    uint16_t d; /* fp16 */
    int8_t qs[OR_QK8_0];
} or_block_q8_0; /* 34 bytes */

typedef struct {
    uint16_t d;    /* fp16 super-block scale for the 6-bit sub-block scales */
    uint16_t dmin; /* fp16 super-block scale for the 6-bit sub-block mins */
    uint8_t scales[12];
    uint8_t qs[OR_QK_K / 2];
} or_block_q4_K; /* 144 bytes */

typedef struct {
    float d;
    int8_t qs[OR_QK_K];
    int16_t bsums[OR_QK_K / 16];
} or_block_q8_K; /* 292 bytes */

/* ggml's block_q2_K .. block_q6_K (ggml-common.h), the other k-quant expert formats */
typedef struct {
    uint8_t scales[OR_QK_K / 16]; /* per 16 values: 4-bit scale | 4-bit min << 4 */
    uint8_t qs[OR_QK_K / 4];      /* 2-bit quants */
    uint16_t d, dmin;             /* fp16 */
} or_block_q2_K; /* 84 bytes */

typedef struct {
    uint8_t hmask[OR_QK_K / 8]; /* high bit of each 3-bit quant */
    uint8_t qs[OR_QK_K / 4];    /* low 2 bits */
    uint8_t scales[12];         /* 16 6-bit scales */
    uint16_t d;                 /* fp16 */
} or_block_q3_K; /* 110 bytes */

typedef struct {
    uint16_t d, dmin; /* fp16 */
    uint8_t scales[12];
    uint8_t qh[OR_QK_K / 8]; /* fifth bit of each quant */
    uint8_t qs[OR_QK_K / 2]; /* low 4 bits */
} or_block_q5_K; /* 176 bytes */

typedef struct {
    uint8_t ql[OR_QK_K / 2];      /* low 4 bits */
    uint8_t qh[OR_QK_K / 4];      /* high 2 bits */
    int8_t scales[OR_QK_K / 16];  /* per 16 values */
    uint16_t d;                   /* fp16 */
} or_block_q6_K; /* 210 bytes */

/* ---- fp16 ---- */
uint16_t or_fp32_to_fp16(float f); /* round to nearest even, like F16C / numpy */
float or_fp16_to_fp32(uint16_t h);

/* ---- block formats ---- */
size_t or_row_bytes(int type, int n); /* bytes of one row of n values (types 0, 1, 8, 12, 15) */
void or_quantize_q8_0_ref(const float *x, int n, void *out); /* quantize_row_q8_0_ref: roundf, id = 1/d */
void or_quantize_q8_0_act(const float *x, int n, void *out); /* x86 quantize_row_q8_0: RNE, id = 127/amax */
void or_quantize_q8_K(const float *x, int n, void *out);     /* quantize_row_q8_K_ref */
void or_dequant_q8_0(const void *in, int n, float *y);
void or_dequant_q4_K(const void *in, int n, float *y);
void or_dequant_q8_K(const void *in, int n, float *y);
void or_q4_K_scale_min(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m); /* get_scale_min_k4 */
float or_vec_dot_q8_0_q8_0(int n, const void *w, const void *x);
float or_vec_dot_q4_K_q8_K(int n, const void *w, const void *x);
/* Q2_K (10), Q3_K (11), Q5_K (13), Q6_K (14): dequantize_row_* and ggml_vec_dot_*_q8_K */
void or_dequant_k(int type, const void *in, int n, float *y);
float or_vec_dot_k_q8_K(int type, int n, const void *w, const void *x);

/* ---- router (src/qwen3.cpp:175-192) ----
 * hnorm [T][h] f32; gate_inp [E][h] of gate_type (0 = F32, 1 = F16).
 * Outputs ids [T][k], weights [T][k]; logits / probs [T][E] are optional (may be NULL). */
void or_router_logits(const float *hnorm, int T, int h, const void *gate_inp, int gate_type, int E, float *logits);
void or_router(const float *hnorm, int T, int h, const void *gate_inp, int gate_type, int E, int k, int32_t *ids,
               float *weights, float *logits, float *probs);

/* ---- token -> expert permutation (grouping of ggml's CPU mul_mat_id) ----
 * bins [T*k] in [0, n_bins). counts [n_bins], offsets [n_bins + 1] (exclusive scan),
 * perm [T*k]: position -> pair index (t*k + j), pairs of one bin in token-major order,
 * active [n_bins]: bins with count > 0 in ascending order; returns the number of active bins. */
int or_permute(const int32_t *bins, int T, int k, int n_bins, int32_t *counts, int32_t *offsets, int32_t *perm,
               int32_t *active);

/* ---- expert FFN + combine + residual (src/qwen3.cpp:197-214, :250) ----
 * Weights in GGUF layout: slot s of a matrix starts at base + s * stride (bytes).
 * up/gate are [f rows][h cols], down is [h rows][f cols]. out may alias resid.
 * y_out (optional, [T][k][h]) receives each pair's weighted expert output. */
void or_moe_ffn(const float *hnorm, int T, int h, int f, int k, const int32_t *slots, const float *weights,
                const float *resid, const void *up, const void *gate, const void *down, size_t stride_up,
                size_t stride_gate, size_t stride_down, int type_up, int type_gate, int type_down, float *out,
                float *y_out, int n_threads);

/* ---- ExpertStore slot bookkeeping (src/expert_store.cpp:106-295) ---- */
typedef struct or_pool or_pool;
/* types / strides: [n_layer][3] = (up, gate, down). Returns NULL and fills err on failure. */
or_pool *or_pool_create(int n_layer, int n_expert, const int32_t *types, const uint64_t *strides, uint64_t pool_bytes,
                        uint32_t min_slots, char *err, size_t err_len);
void or_pool_destroy(or_pool *p);
int or_pool_acquire(or_pool *p, int layer, const int32_t *experts, int n, int32_t *slots, char *err, size_t err_len);
void or_pool_release_all(or_pool *p);
void or_pool_stats(const or_pool *p, uint64_t out[4]); /* hits, misses, bytes_read, acquires */
int or_pool_n_shards(const or_pool *p);
int or_pool_shard_of_layer(const or_pool *p, int layer);
int or_pool_shard_slots(const or_pool *p, int shard);
/* slot owner (layer, expert) or (-1, -1); returns the refcount. */
int or_pool_slot_owner(const or_pool *p, int shard, int slot, int32_t *layer, int32_t *expert);
/* LRU order of a shard, head (evicted next) first; returns the count written. */
int or_pool_lru(const or_pool *p, int shard, int32_t *out, int cap);

/* ---- Qwen3-MoE forward pass around the MoE block (src/qwen3.cpp:112-171, :223-259) ----
 * One sequence whose cells are its positions (what the reference's KvCache hands a lone sequence in an
 * empty cache: blocks 0, 1, 2, ... in order). Dense weights F16 [rows][cols], norms f32, router F16,
 * experts in GGUF layout stacked [n_expert] per matrix. */
typedef struct or_qwen3_hparams {
    int32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_vocab, n_expert, n_expert_used, n_ff_exp;
    float rms_eps, rope_freq_base;
} or_qwen3_hparams;
typedef struct or_qwen3_layer {
    const float *attn_norm;
    const uint16_t *wq, *wk, *wv, *wo;
    const float *q_norm, *k_norm; /* may be NULL */
    const float *ffn_norm;
    const uint16_t *gate_inp;
    int32_t type_up, type_gate, type_down;
    const void *up, *gate, *down;
} or_qwen3_layer;
typedef struct or_qwen3 or_qwen3;

/* Test hook: 1 sums every F16 dot in double (the oracle's own sensitivity to summation order). */
void or_set_f16_double(int on);
float or_dot_f16(const uint16_t *w, const uint16_t *x, int n);                                /* ggml_vec_dot_f16 */
void or_matmul_f16(const uint16_t *W, int rows, int cols, const float *x, int T, float *y);     /* y [T][rows] */
void or_rms_norm(const float *x, int n, const float *w, float eps, float *y);                  /* rms_norm (+ mul) */
void or_rope_neox(const float *x, int hd, int pos, float theta_scale, float *y);               /* one head */
void or_attn_row(const float *q, const uint16_t *K, const uint16_t *V, int n, int hd, int ld, float scale,
                 float *out);                                                                  /* one query row */
or_qwen3 *or_qwen3_create(const or_qwen3_hparams *hp, const or_qwen3_layer *layers, const uint16_t *tok_embd,
                          const float *output_norm, const uint16_t *output, int max_ctx);
void or_qwen3_destroy(or_qwen3 *m);
int or_qwen3_decode(or_qwen3 *m, const int32_t *tokens, int T, float *logits, int32_t *trace);
/* One layer on x [T][n_embd] in place (K / V written at len .. len + T - 1, len unchanged), the final
 * norm + head of one row, and the position advance: or_qwen3_decode is these three in sequence. */
int or_qwen3_run_layer(or_qwen3 *m, int l, float *x, int T, int32_t *ids);
void or_qwen3_head(const or_qwen3 *m, const float *x, float *logits);
void or_qwen3_advance(or_qwen3 *m, int T);
/* Test input: fp16 K / V rows of positions pos .. pos + n - 1 of layer l set directly. */
int or_qwen3_set_kv(or_qwen3 *m, int l, int pos, int n, const uint16_t *k, const uint16_t *v);
int or_qwen3_len(const or_qwen3 *m);
void or_qwen3_truncate(or_qwen3 *m, int keep);

#ifdef __cplusplus
}
#endif
#endif
