// kernels.h - launchers of the gfx950 MoE kernels (kernels.hip), called by the pool (pool.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace lstk {

// Quantized activations: qs [rows][K] int8, d [rows][K/32] f32 (the scale of each 32-value group;
// Q8_K's per-256 scale is repeated 8 times), bs [rows][K/32] int32 (group sums, Q8_K only), and when
// non-null bh [rows][K/32]: the same sums as two exact fp16 values (split_sum_f16, Q8_K only), the
// operand the grouped MFMA kernels take them in.
struct ActBuf {
    int8_t *qs;
    float *d;
    int32_t *bs;
    uint32_t *bh;
};

// When non-null, a launch records its own start/stop timestamps into these events
// (hipExtLaunchKernel), i.e. the same interval a kernel trace reports.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};

// Router logits and activation quantization (fully parallel, no cross-work-group step).
struct RouteParams {
    const float *hnorm;
    int T, h;
    int do_route;
    const void *gate_inp;
    int gate_type;
    int E;
    float *logits; // [T][E]
    int qtype;     // 0: none, 8: Q8_0 rows, 12: Q8_K rows (for Q4_K weights)
    ActBuf xq;
    // One token only: with x_raw set, the launch first computes the row itself as the layer's
    // ffn_norm of x_raw - (x * s) * norm_w with s = 1 / sqrtf(mean + eps), the mean from a double sum
    // of x * x taken in the RMSNorm kernel's order, so the row is bit-identical to that kernel's - and
    // stores it to hnorm_out (hnorm is then unused).
    const float *x_raw;
    const float *norm_w;
    float eps;
    float *hnorm_out;
};

// softmax + top-k + renormalisation from logits, one wavefront per token.
struct TopkParams {
    const float *logits;
    int T, E, k;
    int32_t *ids;
    float *weights;
};

// How a work-group of the expert kernels finds its expert and that expert's (token, slot) pairs.
// route = 1 (gate_up only): the work-group computes the top-k of every token from `logits` itself;
// work-group (0, 0) stores ids / weights. route = 0: ids come from `ids`.
struct GroupParams {
    int T, k, n_bins;
    int route;
    const int32_t *ids;
    const float *logits;
    int E;
    int32_t *ids_out;
    float *weights_out;
    int32_t *err;
};

struct GateUpParams {
    GroupParams gp;
    const uint8_t *w_gate, *w_up;
    size_t stride_gate, stride_up; // bytes per slot
    int type;                      // weight type of gate and up
    int f, h;
    ActBuf xq;
    int max_active;
    float *act; // [T*k][f] SwiGLU rows by pair index t*k + j
};

struct DownParams {
    GroupParams gp;
    const uint8_t *w_down;
    size_t stride_down;
    int type;
    int h, f;
    const float *act;
    const float *weights; // [T*k]
    int max_active;
    float *Y; // [T*k][h] weighted expert outputs by pair index
};

// down + router weight + k-way combine + residual of one token (n_tokens = 1) in one launch:
// work-group b computes rows [b rd, (b + 1) rd) of all k pairs and sums them in slot order.
struct DownCombineParams {
    const int32_t *ids;   // [k] expert ids or pool slots
    const float *weights; // [k]
    int k, n_bins;
    const uint8_t *w_down;
    size_t stride_down;
    int type;
    int h, f;
    const float *act; // [k][f] SwiGLU rows
    const float *resid;
    float *out;
    int32_t *err;
};

struct CombineParams {
    const float *Y;
    const float *resid;
    float *out;
    int T, k, h;
};

// Grouping of the (token, slot) pairs by bin in the order of ggml's CPU mul_mat_id (bins ascending,
// pairs of a bin in token-major order), and the chunk work list of the grouped expert kernels.
struct PermuteParams {
    const int32_t *bins; // [np] bin of pair t * k + j (expert id or pool slot)
    int np, n_bins;
    int chunk;        // pairs per work item
    int32_t *counts;  // [n_bins]
    int32_t *offsets; // [n_bins + 1] exclusive scan of counts
    int32_t *perm;    // [np] sorted position -> pair index
    int4 *items;      // [max_items] {bin, first position, pairs, 0}: each bin's chunks in order, bins ascending; may be null
    int32_t *n_items; // may be null
    int32_t *err;
};

// One grouped expert product over the work list: Q4_K weight rows x Q8_K activation rows on MFMA.
// gate_up: w0 = gate, w1 = up, activation row of a pair = its token (pair / k), out = SwiGLU rows
// [np][rows]. down: w0 = down, activation row = the pair, out = weighted rows [np][rows].
struct GroupedParams {
    const int4 *items;
    const int32_t *n_items;
    const int32_t *perm;
    int k;
    const uint8_t *w0, *w1;
    size_t stride0, stride1; // bytes per slot
    int rows, K;             // weight matrix rows x K (= cols)
    const int8_t *xqs;       // activation rows [*][K] int8
    const float *xd;         // [*][K / 32], the Q8_K scale of each super-block repeated 8 times
    const uint32_t *xbh;     // [*][K / 32], the 32-value group sums as split_sum_f16 pairs
    int row_div;             // activation row = pair / row_div
    const float *weights;    // down: router weight of each pair
    float *out;
};

// The whole MoE block of one token in one launch (fused.hip). Work-groups [0, nB) each compute one
// gate/up unit (pair j = w / ub, row block w % ub); the first nA of them first compute the router
// logits. Work-groups [nB, nB + nC) each compute rd rows of down + weight + combine + residual.
// Stages hand over through device-coherent stores and per-work-group flags holding the launch number.
struct FusedParams {
    const float *hnorm;
    const void *gate_inp;
    int route;                // 1: router in the kernel; 0: ids_in / weights_in
    const int32_t *ids_in;    // [k] slots
    const float *weights_in;  // [k]
    int32_t *ids_out;         // route: written by work-group 0
    float *weights_out;
    int h, f, E, k, n_bins;
    const uint8_t *w_gate, *w_up, *w_down;
    size_t s_gate, s_up, s_down;
    const float *resid;
    float *out;
    float *logits; // [E]
    float *act;    // [k][f]
    int *cnt;      // [nB + nC] launches seen by each work-group
    int *flag_a;   // [nA]
    int *flag_b;   // [nB]
    int32_t *err;
    int nA, nB, nC, ub, rd;
    int spin_max;
};

struct FusedLayout {
    int nA = 0, nB = 0, nC = 0, ub = 0, rd = 0;
    bool ok = false;
};

// Checks the shapes the kernels assume; returns an empty string when they hold.
const char *check_shapes(int h, int f, int E, int k, int n_bins, int n_batch);
// Largest n_tokens for which gate_up computes the top-k itself.
int decode_route_max_tokens();
hipError_t launch_route(const RouteParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_topk(const TopkParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_gate_up(const GateUpParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_down(const DownParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_combine(const CombineParams &p, hipStream_t s, const LaunchTiming *t);
// True when launch_down_combine handles this shape (k * f <= 16384 SwiGLU values in LDS).
bool down_combine_supported(int h, int f, int k);
hipError_t launch_down_combine(const DownCombineParams &p, hipStream_t s, const LaunchTiming *t);

// streaming pool bookkeeping on the device, tier.hip
constexpr int kTierMaxSlots = 1024;  // slots per shard (the pool's shard limit)
constexpr int kTierMaxExperts = 256; // n_expert
constexpr int kTierMaxIds = 4096;    // experts requested per call (n_batch * n_expert_used)
#ifndef LSTK_TIER_COPY_GRID
#define LSTK_TIER_COPY_GRID 256
#endif
constexpr int kTierCopyGrid = LSTK_TIER_COPY_GRID; // work-groups of a copy launch (64-512 all reach the same PCIe rate; 1024 and more lose 3-6%)

// Device copy of the streaming pool's bookkeeping: slot_of [n_layer][n_expert] (-1 = not resident);
// per shard (shards back to back, slot_base apart) its slots in eviction order (order[0] the least
// recently released; every slot is idle between calls) and each slot's owner (layer, expert);
// counters {hits, misses, bytes_read, acquires}.
struct TierLru {
    int32_t *slot_of, *order, *owner_layer, *owner_expert;
    unsigned long long *stats;
};

struct TierResolveParams {
    TierLru lru;
    int layer, E, shard, slot_base, n_slots;
    unsigned long long slab; // bytes of one expert (up + gate + down)
    const int32_t *experts;
    int n;
    int32_t *slots;  // [n] out
    int32_t *miss;   // [2 * n] out: (slot, expert) of each miss
    int32_t *n_miss; // out
    int32_t *err;    // bit 1: expert id out of range (clamped); bit 8: shard exhausted
};

struct TierCopyParams {
    const int32_t *miss, *n_miss;
    int max_miss, n_slots, E;
    const uint8_t *src[3]; // the layer's host-tier matrices (device-visible pinned memory), expert-major
    uint8_t *dst[3];       // the shard's slot arrays
    size_t bytes[3];       // bytes of one expert's matrix (multiples of 16)
    int chunks[3];         // tier_copy_chunks(bytes)
};

int tier_copy_chunks(size_t bytes);
hipError_t launch_tier_resolve(const TierResolveParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_tier_copy(const TierCopyParams &p, hipStream_t s, const LaunchTiming *t);

// grouped (prefill) path, grouped.hip
#ifndef LSTK_GROUPED_CHUNK
#define LSTK_GROUPED_CHUNK 32
#endif
constexpr int kGroupedChunk = LSTK_GROUPED_CHUNK; // pairs per work item (32 or 64)
constexpr int kGroupedMaxBins = 1024;    // bins the permutation kernel handles
// True when the grouped MFMA kernels handle this layer: Q4_K gate, up and down, f % 64 == 0,
// n_bins <= kGroupedMaxBins.
bool grouped_supported(int tu, int tg, int td, int h, int f, int n_bins);
// Upper bound on the work items of np pairs over n_bins bins.
int grouped_max_items(int np, int n_bins);
hipError_t launch_permute(const PermuteParams &p, hipStream_t s, const LaunchTiming *t);
hipError_t launch_gate_up_grouped(const GroupedParams &p, int max_items, hipStream_t s, const LaunchTiming *t);
hipError_t launch_act_quant(const float *act, int f, int np, const ActBuf &aq, hipStream_t s, const LaunchTiming *t);
hipError_t launch_down_grouped(const GroupedParams &p, int max_items, hipStream_t s, const LaunchTiming *t);

// fused single-token path, fused.hip
FusedLayout fused_layout(int h, int f, int E, int k);
// True when every work-group of the fused launch for these types fits on the device at once (the
// stages wait on each other, so they must all be resident).
bool fused_fits(const FusedLayout &L, int gate_type, int tg, int td, int h, int f, int k);
hipError_t launch_fused(const FusedParams &p, int gate_type, int tg, int td, hipStream_t s, const LaunchTiming *t);

}  // namespace lstk
