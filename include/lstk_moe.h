/* lstk_moe.h - C ABI of the MI355X (gfx950) Qwen3-MoE expert-FFN library.
 *
 * The library replaces the MoE block of localstack's qwen3 forward pass:
 *   router()     src/qwen3.cpp:175-192  (gate matmul, softmax, top-k, renormalised weights)
 *   moe_apply()  src/qwen3.cpp:197-214  (gate/up/down mul_mat_id, SwiGLU, weighted k-sum)
 *   residual add src/qwen3.cpp:250 (resident graph) and :287 (streaming segment)
 * and the expert pool that feeds it:
 *   ExpertStore  src/expert_store.h:113-131, src/expert_store.cpp:106-295
 *
 * Conventions (mirroring the reference's `bool f(..., std::string &err)`):
 *   - every call returns 0 on success and a negative LSTK_E_* code on failure;
 *     lstk_last_error() returns the message of the last failure on the calling thread;
 *   - device pointers and streams are owned by the caller; `stream` is a hipStream_t
 *     (NULL = the default stream);
 *   - a pool and its scratch are used from one host thread and one stream at a time, like the
 *     reference Engine (src/engine.h:65); calls that overlap on one pool race.
 * Tensor layouts are row-major C order: hnorm/resid/out are [n_tokens][n_embd] f32,
 * ids/slots are [n_tokens][n_expert_used] int32, weights are [n_tokens][n_expert_used] f32.
 */
#ifndef LSTK_MOE_H
#define LSTK_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSTK_ABI_VERSION 1

/* ggml tensor type ids used on this path (ggml.h enum ggml_type). */
#define LSTK_TYPE_F32 0
#define LSTK_TYPE_F16 1
#define LSTK_TYPE_Q8_0 8
#define LSTK_TYPE_Q4_K 12
#define LSTK_TYPE_Q2_K 10
#define LSTK_TYPE_Q3_K 11
#define LSTK_TYPE_Q5_K 13
#define LSTK_TYPE_Q6_K 14

/* Error codes. */
#define LSTK_OK 0
#define LSTK_E_INVALID (-1)   /* bad argument or shape */
#define LSTK_E_NOMEM (-2)     /* host or device allocation failed */
#define LSTK_E_EXHAUSTED (-3) /* pool exhausted (src/expert_store.cpp:261-266) */
#define LSTK_E_DEVICE (-4)    /* a HIP call failed */
#define LSTK_E_IO (-5)        /* a host-tier copy failed; the slot is marked empty */
#define LSTK_E_BADID (-6)     /* a device kernel saw an expert/slot id out of range */

typedef void *lstk_stream_t; /* a hipStream_t */
typedef struct lstk_pool lstk_pool;

/* Model shape: the MoE part of Qwen3HParams (src/qwen3.h:22-46) plus the largest step size
 * (EngineParams::n_batch, src/engine.h:33) that sizes the pool's scratch. */
typedef struct lstk_moe_dims {
    int32_t n_layer;
    int32_t n_embd;        /* h */
    int32_t n_ff_exp;      /* f */
    int32_t n_expert;      /* E */
    int32_t n_expert_used; /* k */
    int32_t n_batch;       /* max tokens per call */
} lstk_moe_dims;

/* One layer's stacked expert tensors as they sit in a GGUF file: expert e of a matrix starts at
 * host_x + e * expert_stride (GgufTensorInfo::expert_stride, src/gguf_model.h:28).
 * up/gate are [n_expert][n_ff_exp rows][n_embd cols], down is [n_expert][n_embd rows][n_ff_exp cols],
 * each row a run of Q8_0 (34 B / 32 values) or Q2_K / Q3_K / Q4_K / Q5_K / Q6_K (84 / 110 / 144 / 176 /
 * 210 B per 256 values) blocks; gate and up share a type, down may differ.
 * Replaces ExpertLayerInfo (src/expert_store.h:32-36), with host memory in place of a file offset. */
typedef struct lstk_expert_layer {
    int32_t type_up, type_gate, type_down;
    const void *host_up, *host_gate, *host_down;
} lstk_expert_layer;

/* ExpertStoreStats (src/expert_store.h:70-77). */
typedef struct lstk_pool_stats_t {
    uint64_t hits;
    uint64_t misses;
    uint64_t bytes_read; /* bytes copied host tier -> HBM */
    uint64_t acquires;
    double wait_ms;      /* host time spent inside acquire() */
} lstk_pool_stats_t;

/* Pool flags. */
#define LSTK_POOL_STREAMING 1 /* slots < experts: misses are copied from the pinned host tier */
#define LSTK_POOL_DRY 2       /* bookkeeping only: no device memory, no HIP calls (CPU tests) */
#define LSTK_POOL_DEVICE_LRU 4 /* streaming only: the slot bookkeeping lives on the device, acquires go
                                  through lstk_pool_acquire_device */
#define LSTK_POOL_AUTO_SIZE 8  /* streaming only: pool_bytes is ignored and the pool takes
                                  lstk_pool_default_bytes(expert table, 0, 0, total, free) from hipMemGetInfo
                                  on the current device */

const char *lstk_last_error(void);
int lstk_abi_version(void);

/* Creates the expert pool on the current HIP device.
 * Resident (flags without LSTK_POOL_STREAMING): every expert of every layer is uploaded to HBM once
 * and slot s of a layer holds expert s; acquire() is the identity.
 * Streaming: ExpertStore::init semantics (src/expert_store.cpp:106-198): layers are grouped by their
 * (up, gate, down) type triple, each group gets pool_bytes * n_layers_in_group / n_layer, shards hold
 * at most 1024 slots and at least min_slots; the full expert table is copied once into pinned host
 * memory (the host tier, standing in for the GGUF file) and misses are served from it with
 * hipMemcpyAsync on the pool's side streams. Layers that pass the same three host pointers (and
 * types) share one host-tier copy.
 * The layers' host pointers are only read during this call. */
int lstk_pool_create(const lstk_moe_dims *dims, const lstk_expert_layer *layers, size_t pool_bytes,
                     uint32_t min_slots, uint32_t flags, lstk_pool **out);

/* The pool budget of Engine::init (src/engine.cpp:84-117), restated for a GPU with its own HBM:
 *   min(table_bytes, device_total - weight_bytes - kv_bytes - 1.5 GiB, device_free - 3 GiB), at least 16 KiB
 * (each difference floored at 0). The reference also caps the pool at 45% of the table and at 9 GiB: limits
 * of a Mac's unified memory and Metal working set that do not apply to 288 GB of HBM, where a table that
 * fits is simply held whole. The 1024-slot shard limit stays (the device-side acquire stages a shard in
 * LDS). Pure arithmetic, no device call: callers that know their dense weights and KV cache pass them
 * with hipMemGetInfo's figures. */
size_t lstk_pool_default_bytes(size_t table_bytes, size_t weight_bytes, size_t kv_bytes, size_t device_total,
                               size_t device_free);
void lstk_pool_destroy(lstk_pool *pool);

/* ExpertStore::acquire (src/expert_store.cpp:232-286): makes `n` experts of `layer` resident and
 * writes their slot numbers to `slots` (host arrays), pinning them until lstk_pool_release_all().
 * Hits pin; misses evict the LRU head and queue the three matrix copies on a side stream (misses
 * round-robin over the pool's side streams, one expert's copies on one stream); `stream`
 * (the compute stream) is made to wait for those copies, so the host never blocks on them.
 * Fails with LSTK_E_EXHAUSTED when the layer needs more slots than its shard has. */
int lstk_pool_acquire(lstk_pool *pool, int layer, const int32_t *experts, int n, int32_t *slots,
                      lstk_stream_t stream);
/* ExpertStore::release_all (src/expert_store.cpp:289-295). Slots released here are not overwritten
 * before the work already queued on `stream` has finished with them. */
int lstk_pool_release_all(lstk_pool *pool, lstk_stream_t stream);
/* ExpertStore::acquire followed by release_all (src/expert_store.cpp:232-295), run on the device for a
 * pool created with LSTK_POOL_DEVICE_LRU, so the host never sees the router's choice (the per-layer
 * CPU round trip of src/engine.cpp:343-392 and docs/decisions.md:14 goes away, and a forward pass over
 * a streaming pool can be captured in a graph). d_experts [n] (device) are resolved in order with the
 * same LRU as lstk_pool_acquire + lstk_pool_release_all: the same slots, hits and misses for the same
 * sequence of calls. d_slots [n] (device) receives the slots; the misses are copied from the pinned
 * host tier by a kernel reading it over PCIe. Both kernels run on `stream`: work queued on `stream`
 * after this call sees the experts, and the slots stay valid until the next acquire_device on the pool.
 * Calls on one pool must be ordered on one stream. n <= n_batch * n_expert_used <= 4096; every shard
 * needs at least min(n_batch * n_expert_used, n_expert) slots (checked at creation), so a call never
 * runs out of slots. An expert id out of range is clamped and reported by lstk_pool_check. */
int lstk_pool_acquire_device(lstk_pool *pool, int layer, const int32_t *d_experts, int n, int32_t *d_slots,
                             lstk_stream_t stream);
/* For an LSTK_POOL_DEVICE_LRU pool the counters are read from the device (the call waits for the
 * device; wait_ms stays 0). */
int lstk_pool_stats(const lstk_pool *pool, lstk_pool_stats_t *out);
size_t lstk_pool_total_bytes(const lstk_pool *pool);   /* ExpertStore::total_bytes */
uint32_t lstk_pool_total_slots(const lstk_pool *pool); /* ExpertStore::total_slots */
/* Slots of the shard serving `layer` (ExpertPool::n_slots via pool_for, src/expert_store.h:120). */
int lstk_pool_layer_slots(const lstk_pool *pool, int layer);
/* ExpertStore::describe (src/expert_store.cpp:309-319); writes a NUL-terminated string. */
int lstk_pool_describe(const lstk_pool *pool, char *buf, size_t len);

/* router() (src/qwen3.cpp:175-192) on the device: logits = gate_inp . hnorm (F16 weights take
 * fp16-rounded activations as ggml's CPU mul_mat does), softmax over the n_expert logits, top-k in
 * descending order (ties to the lower expert id), weights = p / max(sum p, 2^-14).
 * d_gate_inp is [n_expert][n_embd] of gate_type (LSTK_TYPE_F16 or LSTK_TYPE_F32). */
int lstk_moe_route(lstk_pool *pool, int layer, const float *d_hnorm, int n_tokens, const void *d_gate_inp,
                   int gate_type, int32_t *d_ids, float *d_weights, lstk_stream_t stream);

/* moe_apply() + the residual add (src/qwen3.cpp:197-214 and :250 / :287) on the device:
 * out[t] = resid[t] + sum_{j=0..k-1} weights[t][j] * down_s(swiglu(gate_s(x_t), up_s(x_t))),
 * s = d_slots[t][j], summed left to right in j. x_t is quantized to the activation type ggml pairs with
 * the weight type (Q8_0 for Q8_0, Q8_K for Q4_K), and so is the SwiGLU output before down.
 * d_slots holds slot numbers from lstk_pool_acquire (streaming) or expert ids (resident).
 * d_out may alias d_resid.
 * With Q4_K gate, up and down and at least 64 tokens (LSTK_GROUPED_MIN_TOKENS in the environment
 * overrides the threshold) the call takes the grouped path: a stable permutation of the pairs by
 * expert, then expert products on the matrix cores over 64-pair chunks. */
int lstk_moe_ffn(lstk_pool *pool, int layer, const float *d_hnorm, const int32_t *d_slots, const float *d_weights,
                 const float *d_resid, float *d_out, int n_tokens, lstk_stream_t stream);

/* The whole MoE block of a resident layer in one call (router + experts + residual) with no host
 * round trip: for a single token the gate/up kernel runs the top-k itself from the router logits.
 * With LSTK_FUSED_DECODE=1 in the environment at pool creation, single-token calls of this and of
 * lstk_moe_ffn run as one fused launch instead (same results bit for bit).
 * d_ids / d_weights receive the routing (for traces, src/engine.cpp:301-316); they may not be NULL.
 * Valid for resident pools only. */
int lstk_moe_block(lstk_pool *pool, int layer, const float *d_hnorm, const void *d_gate_inp, int gate_type,
                   const float *d_resid, float *d_out, int32_t *d_ids, float *d_weights, int n_tokens,
                   lstk_stream_t stream);

/* No counterpart in the reference: lstk_moe_block for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The call's
 * scratch (quantized activations, router logits, SwiGLU rows, per-pair outputs) comes from a fixed
 * array of LSTK_NOALLOC_SCRATCH_BYTES in the library, one copy per device, held until the process
 * ends; the call allocates nothing and creates no events. Same arguments, kernels and results as
 * lstk_moe_block, except that it never takes the fused or the grouped (matrix-core prefill) path and
 * keeps no stage timing. Fails with LSTK_E_INVALID when n_tokens needs more scratch than the array
 * holds: n_tokens * (n_embd * (1.25 + 4 k) + 4 E + 4 k n_ff_exp) bytes, each part rounded up to 256
 * (up to 180 tokens at the 30B-A3B shape, 90 at the 235B-A22B shape; n_batch of the pool still
 * applies). Every call on a device shares that device's array, which keeps the last call's contents:
 * calls that overlap on one device race, whatever pool or stream they use. */
#define LSTK_NOALLOC_SCRATCH_BYTES ((size_t) 16 << 20)
int lstk_moe_block_noalloc(lstk_pool *pool, int layer, const float *d_hnorm, const void *d_gate_inp, int gate_type,
                           const float *d_resid, float *d_out, int32_t *d_ids, float *d_weights, int n_tokens,
                           lstk_stream_t stream);

/* The token-to-expert grouping of ggml's CPU mul_mat_id (the three calls at src/qwen3.cpp:201-204) on
 * the device: the n_tokens * n_expert_used pairs (t, j), pair index t * n_expert_used + j, are sorted by
 * bin d_bins[t][j] in [0, n_bins), bins ascending and each bin's pairs in token-major order (a stable
 * counting sort). Writes d_counts [n_bins], d_offsets [n_bins + 1] (exclusive scan of the counts) and
 * d_perm [n_tokens * n_expert_used] (sorted position -> pair index). n_bins <= 1024. A bin out of range
 * is clamped on the device and reported by lstk_pool_check. The grouped (prefill) path of
 * lstk_moe_ffn / lstk_moe_block runs the same kernel. */
int lstk_moe_permute(lstk_pool *pool, const int32_t *d_bins, int n_tokens, int n_bins, int32_t *d_counts,
                     int32_t *d_offsets, int32_t *d_perm, lstk_stream_t stream);

/* Waits for `stream` and reports LSTK_E_BADID if a kernel has seen an id out of range since the
 * last check (the id is clamped on the device so no access leaves the pool). */
int lstk_pool_check(lstk_pool *pool, lstk_stream_t stream);

/* Per-stage kernel timing: with timing on, every launch records its own start and stop timestamps
 * into HIP events (hipExtLaunchKernel), the interval a kernel trace reports.
 * stage: 0 = router logits + activation quantization (+ the top-k kernel above 16 tokens),
 * 1 = gate + up + SwiGLU, 2 = down + router weight, 3 = combine + residual.
 * lstk_pool_timing waits for the launches recorded so far and returns the summed milliseconds and
 * the launch count of each stage; it resets the counters. Timing is for eager launches (not inside
 * a captured graph). */
int lstk_pool_set_timing(lstk_pool *pool, int enable);
int lstk_pool_timing(lstk_pool *pool, double ms[4], int64_t launches[4]);

/* Host-side repacking between GGUF expert bytes and the pool's HBM layout (one expert matrix of
 * `rows` x `cols`). The pool layout is [rows/16][cols/256][C][16 rows][16 B], the last row block
 * holding the rows left over: each 256-value super-block row is split into C 16-byte chunks (Q8_0:
 * 8 fp16 scales + 16 chunks of int8; Q4_K: {d, dmin, scales} + 8 chunks of 4-bit pairs; Q2_K, Q3_K,
 * Q5_K and Q6_K unpacked to integers: {f32 d, f32 dmin}, 16 int8 scales, 16 mins and 16 chunks of
 * int8 quants, one per 16 values), chunk c of a row block's 16 rows is one 256-byte piece, and a row
 * block's super-blocks and chunks are contiguous, so a work-group that takes whole row blocks reads
 * one contiguous span. lstk_matrix_bytes is the pool size (the GGUF size for Q8_0 and Q4_K, 304 B per
 * super-block row for the other k-quants); lstk_unpack_matrix inverts Q8_0 and Q4_K only. */
size_t lstk_matrix_bytes(int type, int rows, int cols);
int lstk_repack_matrix(int type, int rows, int cols, const void *gguf, void *packed);
int lstk_unpack_matrix(int type, int rows, int cols, const void *packed, void *gguf);

/* Test hook for the failure path the reference leaves silent (a failed pread is only logged,
 * src/expert_store.cpp:62-66): the next n host-tier copies fail, the acquire returns LSTK_E_IO and
 * the slots involved are unmapped. */
int lstk_pool_debug_fail_copies(lstk_pool *pool, int n);

#ifdef __cplusplus
}
#endif
#endif
