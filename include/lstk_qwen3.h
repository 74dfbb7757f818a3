/* lstk_qwen3.h - C ABI of the Qwen3-MoE forward pass that surrounds the MoE path on MI355X.
 *
 * The MoE block (include/lstk_moe.h) needs the rest of the model around it to produce logits. This
 * is that rest, on the same device and stream:
 *   qwen3_build_graph()   src/qwen3.cpp:223-259 (embedding, per-layer attention + MoE, final norm,
 *                         output head; the last layer's FFN runs on the output row only)
 *   attn_block()          src/qwen3.cpp:128-171 (RMSNorm, Q/K/V, QK-norm, NEOX RoPE, KV set_rows,
 *                         attention with fp32 accumulation over fp16 K/V, o-proj, residual)
 *   Engine::decode/step   src/engine.cpp:250-278 (chunks of n_batch tokens, logits of the last token)
 *   Engine::step_resident / step_streaming  src/engine.cpp:282-341 (router trace; streaming pools
 *                         acquire the experts each layer selected before running them)
 *   KvCache               src/kv_cache.cpp:59-150 (block table per sequence, cell_seq / cell_pos,
 *                         visibility = same sequence and cell_pos <= token position)
 * Dense (non-MoE) FFNs and Qwen2's Q/K/V biases are not part of this path.
 *
 * Conventions are those of lstk_moe.h: 0 or a negative LSTK_E_* code, lstk_last_error() for the
 * message, caller-owned device pointers and stream, one host thread and one stream per model.
 * Weight layouts are ggml's: an F16 matrix of ggml shape [n_in, n_out] is n_out rows of n_in
 * contiguous fp16 values.
 */
#ifndef LSTK_QWEN3_H
#define LSTK_QWEN3_H

#include "lstk_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lstk_model lstk_model;

/* Qwen3HParams (src/qwen3.h:22-46), the fields the MoE forward pass reads. */
typedef struct lstk_qwen3_hparams {
    int32_t n_layer;
    int32_t n_embd;
    int32_t n_head;
    int32_t n_head_kv;
    int32_t head_dim;
    int32_t n_vocab;
    int32_t n_expert;
    int32_t n_expert_used;
    int32_t n_ff_exp;
    int32_t n_ctx_train; /* carried for RoPE; inert without context extension */
    float rms_eps;
    float rope_freq_base;
} lstk_qwen3_hparams;

/* One layer's dense tensors on the device (Qwen3Layer, src/qwen3.h:49-73). Norm weights are f32;
 * q_norm / k_norm may be NULL (no QK-norm). The experts live in the lstk_pool passed at creation. */
typedef struct lstk_qwen3_layer {
    const float *attn_norm;  /* [n_embd] */
    const uint16_t *wq;      /* F16 [n_head * head_dim][n_embd] */
    const uint16_t *wk;      /* F16 [n_head_kv * head_dim][n_embd] */
    const uint16_t *wv;      /* F16 [n_head_kv * head_dim][n_embd]; when wk starts where wq ends and wv
                                where wk ends (one [q | k | v] block), multi-token steps take one
                                library product for all three instead of three */
    const uint16_t *wo;      /* F16 [n_embd][n_head * head_dim] */
    const float *q_norm;     /* [head_dim] or NULL */
    const float *k_norm;     /* [head_dim] or NULL */
    const float *ffn_norm;   /* [n_embd] */
    const void *gate_inp;    /* router, [n_expert][n_embd] of gate_inp_type */
    int32_t gate_inp_type;   /* LSTK_TYPE_F16 or LSTK_TYPE_F32 */
} lstk_qwen3_layer;

/* Model-wide tensors (Qwen3Weights, src/qwen3.h:75-82). output == NULL ties the head to tok_embd,
 * as the reference's loader does when the GGUF has no output.weight (src/qwen3.cpp:55-57). */
typedef struct lstk_qwen3_weights {
    const uint16_t *tok_embd;    /* F16 [n_vocab][n_embd] */
    const float *output_norm;    /* [n_embd] */
    const uint16_t *output;      /* F16 [n_vocab][n_embd] or NULL */
    const lstk_qwen3_layer *layers; /* n_layer entries, copied at creation */
} lstk_qwen3_weights;

/* Creates the forward pass over `pool` (whose dims must match hp) with a KV cache of kv_size cells
 * (a multiple of 256, like the reference's n_ctx) and steps of at most n_batch tokens
 * (EngineParams::n_batch, at most the pool's n_batch). head_dim must be 64, 128 or 256;
 * n_embd and n_head * head_dim multiples of 8 and at most 8192. The KV cache (fp16,
 * 2 * n_layer * kv_size * n_head_kv * head_dim * 2 bytes) and the step scratch are allocated here, on
 * the current device. The pool is not owned and must outlive the model. */
int lstk_model_create(const lstk_qwen3_hparams *hp, const lstk_qwen3_weights *w, lstk_pool *pool, uint32_t kv_size,
                      uint32_t n_batch, lstk_model **out);
void lstk_model_destroy(lstk_model *model);

/* Engine::decode (src/engine.cpp:250-260) for one sequence: appends `n_tokens` host token ids to
 * sequence `seq` in steps of at most n_batch tokens and writes the logits of the last token,
 * [n_vocab] f32, to the device pointer d_logits. When d_trace is not NULL it receives the router's
 * expert ids of every layer for the last step, [n_layer][n_step_tokens][n_expert_used] int32, where the
 * last layer has only its output row (the others are -1), like the reference's trace
 * (src/engine.cpp:299-316). Token ids out of [0, n_vocab) are rejected before anything runs.
 * Fails with LSTK_E_EXHAUSTED when the KV cache has no room ("KV cache is full"). */
int lstk_model_decode(lstk_model *model, int32_t seq, const int32_t *tokens, int n_tokens, float *d_logits,
                      int32_t *d_trace, lstk_stream_t stream);

/* lstk_model_decode in two halves, for callers that replay a step as a HIP graph.
 * prepare: Engine::make_step_inputs (src/engine.cpp:200-243) - reserves the KV cells of n_tokens
 *   (<= n_batch) host tokens of `seq`, queues their upload to the model's input buffer on `stream` and
 *   returns the number of attended cells in *n_cells.
 * forward: the step's kernels over those inputs, writing the last token's logits (and the trace, as
 *   lstk_model_decode). With a resident pool it makes no host synchronisation and no allocation, so it
 *   may be captured; a captured forward replays correctly after each prepare of the same seq,
 *   n_tokens and n_cells (n_cells changes only when the sequence crosses a multiple of 256 cells),
 *   wherever the new cells lie: while the stream is capturing, attention covers cells [0, n_cells)
 *   (an eager forward starts at the sequence's lowest cache block instead).
 *   With a streaming pool it synchronises the stream once per layer (the router's ids go to the host),
 *   unless the pool was created with LSTK_POOL_DEVICE_LRU: then the experts are acquired on the device
 *   (lstk_pool_acquire_device), nothing waits on the host and the forward may be captured too. */
int lstk_model_prepare(lstk_model *model, int32_t seq, const int32_t *tokens, int n_tokens, int32_t *n_cells,
                       lstk_stream_t stream);
int lstk_model_forward(lstk_model *model, int32_t seq, int n_tokens, int32_t n_cells, float *d_logits,
                       int32_t *d_trace, lstk_stream_t stream);

/* KvCache::remove_seq / truncate_seq / length (src/kv_cache.cpp:97-150, src/engine.h:75-80). */
int lstk_model_remove_seq(lstk_model *model, int32_t seq);
int lstk_model_truncate_seq(lstk_model *model, int32_t seq, int32_t keep);
int32_t lstk_model_seq_len(const lstk_model *model, int32_t seq);

/* Appends n_cells positions to sequence `seq` without running tokens: their K and V cells hold seeded
 * pseudo-random fp16 values in [-1, 1). A synthetic context of a given length, for measuring decode
 * at that KV length without a prefill; it has no counterpart in the reference. */
int lstk_model_fill_context(lstk_model *model, int32_t seq, int n_cells, uint64_t seed, lstk_stream_t stream);

/* Test hook (no counterpart in the reference): with d_states set, every forward also copies the residual
 * stream after each layer l, [T][n_embd] f32, to d_states + l * T * n_embd (a device buffer of at least
 * n_layer * n_batch * n_embd floats) on its stream, so a test can compare the model layer by layer with
 * a reference fed the same layer inputs; NULL turns it off. After the last layer only the output row has
 * been through the MoE block. */
int lstk_model_debug_capture(lstk_model *model, float *d_states);

/* Test hook (no counterpart in the reference): with d_moe_in set, every forward also copies the residual
 * stream entering layer l's MoE block (after attention, o-proj and residual; the input of ffn_norm and the
 * router), [T][n_embd] f32, to d_moe_in + l * T * n_embd, so a test can run a reference router on exactly
 * the device's router input; NULL turns it off. */
int lstk_model_debug_capture_moe_in(lstk_model *model, float *d_moe_in);

/* Test hook (no counterpart in the reference): options of the model's later forwards. Bit 0 set: a
 * single-token step runs RoPE and the new cell's K / V store in a launch of their own before the
 * attention, whose chunks then take several 64-cell passes, instead of inside the attention launch with
 * one-pass chunks (the plan steps of more tokens and contexts past 65536 cells always take), so a test can
 * compare the two plans on the same cache. 0 restores the default. */
int lstk_model_debug_options(lstk_model *model, int flags);

/* Test hook (no counterpart in the reference): the attention launch plan a step of n_tokens takes (host
 * arithmetic only, no device call), for n_head query / n_kv KV heads of head_dim over cells
 * [cell_begin, n_cells) of a kv_size-cell cache; rope_in asks for RoPE inside the launch (one token).
 * out[0..5] = query rows per work-group, row blocks, cells per chunk, chunks, RoPE kept inside the launch
 * (0 / 1), work-groups of the attention launch. Fails with LSTK_E_INVALID on arguments a model would
 * never pass. */
int lstk_debug_attn_plan(int n_tokens, int n_head, int n_kv, int head_dim, int kv_size, int n_cells, int cell_begin,
                         int rope_in, int32_t out[6]);

/* Engine::set_routing_trace (src/engine.cpp:179-186): with a path, creates the file and writes the
 * trace header ("LSTKRTE1", n_layer, n_expert, n_expert_used as little-endian int32); every later step
 * of lstk_model_decode then appends its token count and its router ids ([n_layer][n_tokens][k] int32,
 * -1 for rows the last layer skips), read back from the device after the step (a synchronisation per
 * step, as the reference's). NULL closes the file. Steps run through prepare / forward are not traced. */
int lstk_model_set_trace(lstk_model *model, const char *path);

/* Per-stage device time of the forward pass's own kernels, recorded like lstk_pool_timing:
 * stage 0 = norms + embedding, 1 = Q/K/V + QK-norm + RoPE + KV store, 2 = attention,
 * 3 = o-proj + residual, 4 = output head. The MoE block's stages are read with lstk_pool_timing. */
int lstk_model_set_timing(lstk_model *model, int enable);
int lstk_model_timing(lstk_model *model, double ms[5], int64_t launches[5]);

#ifdef __cplusplus
}
#endif

#endif /* LSTK_QWEN3_H */
