// pool.cpp - the HBM expert pool and the C ABI of the MoE path (include/lstk_moe.h).
//
// lstk_pool plays the part of the reference's ExpertStore (src/expert_store.h:113-149,
// src/expert_store.cpp:106-295) on MI355X:
//   - resident pools hold every expert of every layer in HBM (288 GB holds a 235B-A22B-shaped
//     Q4_K expert table whole), slot s of a layer = expert s;
//   - streaming pools keep the reference's slot bookkeeping exactly (type-triple classes, shards of
//     at most 1024 slots, pin counts, intrusive LRU, hits/misses/bytes_read/acquires stats), with the
//     GGUF file replaced by a pinned host tier and pread() by hipMemcpyAsync on side streams (a layer's
//     misses round-robin over LSTK_SIDE_STREAMS of them) that the compute stream waits on through
//     events, so acquire() never blocks the host on a copy;
//   - a copy that fails unmaps its slot and fails the acquire (the reference only logs a short read,
//     src/expert_store.cpp:62-66, and leaves the slot holding garbage).
// It also owns the per-call device scratch (quantized activations, logits, permutation, SwiGLU rows,
// per-pair outputs, arrival counters) sized for dims.n_batch tokens.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "../../include/lstk_moe.h"
#include "formats.h"
#include "internal.h"
#include "kernels.h"

namespace lstk {
int repack_matrix(int type, int rows, int cols, const void *gguf, void *packed);
int unpack_matrix(int type, int rows, int cols, const void *packed, void *gguf);
}  // namespace lstk

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(LSTK_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr uint32_t kMaxSlotsPerShard = 1024; // kMaxSlotsPerPool, src/expert_store.h:80
static_assert(kMaxSlotsPerShard <= (uint32_t) lstk::kTierMaxSlots, "the device-side acquire stages a shard in LDS");

const char *type_name(int t) {
    switch (t) {
        case lstk::kTypeQ8_0: return "q8_0";
        case lstk::kTypeQ2_K: return "q2_K";
        case lstk::kTypeQ3_K: return "q3_K";
        case lstk::kTypeQ4_K: return "q4_K";
        case lstk::kTypeQ5_K: return "q5_K";
        case lstk::kTypeQ6_K: return "q6_K";
        case lstk::kTypeF16: return "f16";
        case lstk::kTypeF32: return "f32";
        default: return "?";
    }
}

// A shard's unpinned slots, least recently released first. Entries are never moved: withdrawing a
// slot (a hit, or the oldest one taken by a miss) only makes its entry stale, and releasing appends a
// new entry; an entry is live while pos[slot] names it. Every operation is O(1) amortised, and the
// array is rebuilt from its live entries once it holds as many stale ones.
struct IdleQueue {
    std::vector<int32_t> q, pos; // entries (slot ids); slot -> index of its live entry, or -1 (pinned)
    size_t front = 0, live = 0;

    void reset(uint32_t n) { // slots 0 .. n - 1, slot 0 oldest
        q.resize(n);
        pos.resize(n);
        for (uint32_t i = 0; i < n; i++) q[i] = pos[i] = (int32_t) i;
        front = 0;
        live = n;
    }
    bool idle(int32_t s) const { return pos[s] >= 0; }
    void withdraw(int32_t s) {
        pos[s] = -1;
        live--;
    }
    int32_t take_oldest() {
        while (front < q.size() && pos[q[front]] != (int32_t) front) front++;
        if (front == q.size()) return -1;
        const int32_t s = q[front++];
        withdraw(s);
        return s;
    }
    void append(int32_t s) {
        if (q.size() - front >= 2 * live + 64) rebuild();
        pos[s] = (int32_t) q.size();
        q.push_back(s);
        live++;
    }
    void rebuild() {
        size_t w = 0;
        for (size_t i = front; i < q.size(); i++)
            if (pos[q[i]] == (int32_t) i) {
                pos[q[i]] = (int32_t) w;
                q[w++] = q[i];
            }
        q.resize(w);
        front = 0;
    }
    std::vector<int32_t> order() const { // live entries, oldest first
        std::vector<int32_t> out;
        for (size_t i = front; i < q.size(); i++)
            if (pos[q[i]] == (int32_t) i) out.push_back(q[i]);
        return out;
    }
};

// One pool shard (ExpertPool, src/expert_store.h:83-110): slot arrays of one type class, the expert
// each slot holds, pin counts, and the idle slots in eviction order.
struct Shard {
    int tu = 0, tg = 0, td = 0;
    size_t up_bytes = 0, gate_bytes = 0, down_bytes = 0, slab = 0;
    uint32_t n_slots = 0;
    std::vector<int> layers;
    uint8_t *d_up = nullptr, *d_gate = nullptr, *d_down = nullptr;
    std::vector<int32_t> owner_layer, owner_expert, refcount;
    IdleQueue idle;
};

struct TimedLaunch {
    hipEvent_t start, end;
};

constexpr int kStages = 4; // router (+ top-k), gate_up, down, combine

}  // namespace

// Side streams that carry host-tier copies: a layer's misses go round-robin over them (all three matrices
// of one expert on one stream), so several DMA engines can serve one acquire.
#ifndef LSTK_SIDE_STREAMS
#define LSTK_SIDE_STREAMS 4
#endif
constexpr int kSides = LSTK_SIDE_STREAMS;

// The scratch of lstk_moe_block_noalloc: quantized activations, router logits, SwiGLU rows and per-pair
// outputs of one call, laid out for that call's token count. Every device holds its own copy until the
// process ends. In host code the name stands in for the array and is not a device address: host code
// uses only the address hipGetSymbolAddress returns on each device (noalloc_address below).
constexpr size_t kNoAllocBytes = LSTK_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

struct lstk_pool {
    lstk_moe_dims dims{};
    bool streaming = false, dry = false;
    int device = 0;
    std::vector<Shard> shards;
    std::vector<int> layer_shard;
    std::vector<std::array<int, 3>> types;
    std::vector<int32_t> slot_of; // streaming: [layer * n_expert + expert] -> slot or -1
    std::vector<std::pair<int, int32_t>> pinned;
    // streaming host tier: per layer, the layer's experts in pool layout, in pinned memory
    uint8_t *tier = nullptr;
    std::vector<std::array<uint8_t *, 3>> tier_of;
    hipStream_t side[kSides] = {};
    hipEvent_t copy_done[kSides] = {}, release_ev = nullptr;
    int fail_copies = 0;
    // LSTK_POOL_DEVICE_LRU: the bookkeeping lives on the device (tier.hip); the host copy above
    // only holds the initial state
    bool device_lru = false;
    void *dlru_mem = nullptr;
    lstk::TierLru dlru{};
    std::vector<int> slot_base;   // per shard: first slot in the device LRU arrays
    int32_t *d_miss = nullptr, *d_n_miss = nullptr;
    std::vector<std::array<const uint8_t *, 3>> tier_dev; // per layer: device-visible host-tier matrices
    lstk_pool_stats_t stats{};
    // per-call scratch, allocated at creation for n_batch tokens
    void *scratch_mem = nullptr;
    lstk::ActBuf xq{};
    float *logits = nullptr, *act = nullptr, *Y = nullptr;
    // set by the forward pass around a block of several tokens: the combine is left to the next
    // layer's RMSNorm launch, which sums the rows of Y into the residual itself (pool_defer_combine)
    bool defer_combine = false;
    // this device's address of the library's fixed scratch array (lstk_moe_block_noalloc)
    uint8_t *noalloc = nullptr;
    int32_t *err = nullptr;
    int n_bins_max = 0;
    // grouped (prefill) path: permutation, work list, Q8_K SwiGLU rows
    int32_t *counts = nullptr, *offsets = nullptr, *perm = nullptr, *n_items = nullptr;
    int4 *items = nullptr;
    lstk::ActBuf aq{};
    int grouped_min_tokens = 0;
    // fused single-token path: launch counters and stage flags (zero at creation)
    lstk::FusedLayout fl{};
    bool fused_enabled = false;
    int *f_cnt = nullptr, *f_flag_a = nullptr, *f_flag_b = nullptr;
    std::map<std::array<int, 4>, bool> fused_fit; // (gate type, tg, td, 0) -> all work-groups resident
    // timing
    bool timing = false;
    std::vector<TimedLaunch> launched[kStages];
    double ms[kStages] = {};
    int64_t launches[kStages] = {};
};

namespace {

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int alloc_scratch(lstk_pool *P) {
    const lstk_moe_dims &d = P->dims;
    const size_t nb = (size_t) P->n_bins_max, T = (size_t) d.n_batch, k = (size_t) d.n_expert_used;
    const size_t h = (size_t) d.n_embd, f = (size_t) d.n_ff_exp, E = (size_t) d.n_expert;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t o_qs = take(T * h), o_d = take(T * (h / 32) * 4), o_bs = take(T * (h / 32) * 4);
    const size_t o_bh = take(T * (h / 32) * 4);
    const size_t o_logits = take(T * E * 4);
    const size_t o_act = take(T * k * f * 4), o_Y = take(T * k * h * 4);
    const size_t o_err = take(64);
    const size_t np = T * k;
    const size_t max_items = (size_t) lstk::grouped_max_items((int) np, (int) nb);
    const size_t o_counts = take(nb * 4), o_offsets = take((nb + 1) * 4), o_perm = take(np * 4), o_nitems = take(64);
    const size_t o_items = take(max_items * 16);
    const size_t o_aqs = take(np * f), o_ad = take(np * (f / 32) * 4), o_abs = take(np * (f / 32) * 4);
    const size_t o_abh = take(np * (f / 32) * 4);
    P->fl = lstk::fused_layout((int) h, (int) f, (int) E, (int) k);
    const size_t n_fused = P->fl.ok ? (size_t) (P->fl.nB + P->fl.nC) : 1;
    const size_t o_fcnt = take(n_fused * 4), o_fa = take((size_t) std::max(P->fl.nA, 1) * 4),
                 o_fb = take((size_t) std::max(P->fl.nB, 1) * 4);
    hipError_t e = hipMalloc(&P->scratch_mem, off);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch)");
    e = hipMemset(P->scratch_mem, 0, off);
    if (e != hipSuccess) return hip_fail(e, "hipMemset(scratch)");
    uint8_t *b = static_cast<uint8_t *>(P->scratch_mem);
    P->xq.qs = reinterpret_cast<int8_t *>(b + o_qs);
    P->xq.d = reinterpret_cast<float *>(b + o_d);
    P->xq.bs = reinterpret_cast<int32_t *>(b + o_bs);
    P->xq.bh = reinterpret_cast<uint32_t *>(b + o_bh);
    P->logits = reinterpret_cast<float *>(b + o_logits);
    P->act = reinterpret_cast<float *>(b + o_act);
    P->Y = reinterpret_cast<float *>(b + o_Y);
    P->err = reinterpret_cast<int32_t *>(b + o_err);
    P->counts = reinterpret_cast<int32_t *>(b + o_counts);
    P->offsets = reinterpret_cast<int32_t *>(b + o_offsets);
    P->perm = reinterpret_cast<int32_t *>(b + o_perm);
    P->n_items = reinterpret_cast<int32_t *>(b + o_nitems);
    P->items = reinterpret_cast<int4 *>(b + o_items);
    P->aq.qs = reinterpret_cast<int8_t *>(b + o_aqs);
    P->aq.d = reinterpret_cast<float *>(b + o_ad);
    P->aq.bs = reinterpret_cast<int32_t *>(b + o_abs);
    P->aq.bh = reinterpret_cast<uint32_t *>(b + o_abh);
    P->f_cnt = reinterpret_cast<int *>(b + o_fcnt);
    P->f_flag_a = reinterpret_cast<int *>(b + o_fa);
    P->f_flag_b = reinterpret_cast<int *>(b + o_fb);
    {
        const char *env = std::getenv("LSTK_FUSED_DECODE");
        P->fused_enabled = env && env[0] == '1';
    }
    return LSTK_OK;
}

// The current device's address of `scratch`, looked up once per device (the caller has made `device`
// current) and kept for the life of the process.
int noalloc_address(int device, uint8_t **out) {
    static std::mutex mu;
    static std::map<int, uint8_t *> addr;
    std::lock_guard<std::mutex> lock(mu);
    auto it = addr.find(device);
    if (it == addr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        it = addr.emplace(device, static_cast<uint8_t *>(p)).first;
    }
    *out = it->second;
    return LSTK_OK;
}

// Repacks `n_expert` GGUF expert matrices (expert-major) into dst (host memory, pool layout),
// experts spread over host threads.
int repack_experts(int type, int rows, int cols, int n_expert, const void *src, uint8_t *dst) {
    const size_t src_bytes = lstk::gguf_matrix_bytes(type, rows, cols), bytes = lstk::matrix_bytes(type, rows, cols);
    const int n_threads = (int) std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    std::vector<int> rcs(n_threads, LSTK_OK);
    auto work = [&](int i) {
        for (int e = i; e < n_expert; e += n_threads) {
            const int rc = lstk::repack_matrix(type, rows, cols, static_cast<const uint8_t *>(src) + (size_t) e * src_bytes,
                                               dst + (size_t) e * bytes);
            if (rc != LSTK_OK) rcs[i] = rc;
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n_threads; i++) pool.emplace_back(work, i);
    work(0);
    for (std::thread &t : pool) t.join();
    for (int rc : rcs)
        if (rc != LSTK_OK) return fail(rc, "repack failed");
    return LSTK_OK;
}

void destroy(lstk_pool *P) {
    if (!P) return;
    if (!P->dry) {
        for (Shard &s : P->shards) {
            if (s.d_up) (void) hipFree(s.d_up);
            if (s.d_gate) (void) hipFree(s.d_gate);
            if (s.d_down) (void) hipFree(s.d_down);
        }
        if (P->tier) (void) hipHostFree(P->tier);
        if (P->scratch_mem) (void) hipFree(P->scratch_mem);
        for (int i = 0; i < kSides; i++) {
            if (P->copy_done[i]) (void) hipEventDestroy(P->copy_done[i]);
            if (P->side[i]) (void) hipStreamDestroy(P->side[i]);
        }
        if (P->release_ev) (void) hipEventDestroy(P->release_ev);
        if (P->dlru_mem) (void) hipFree(P->dlru_mem);
        for (auto &v : P->launched)
            for (TimedLaunch &t : v) {
                (void) hipEventDestroy(t.start);
                (void) hipEventDestroy(t.end);
            }
    }
    delete P;
}

// The shard layout of a streaming pool (ExpertStore::init, src/expert_store.cpp:116-150). Layers are
// grouped by their (up, gate, down) types, since one slot array holds one type. A group's budget is
// pool_bytes in proportion to its layer count; when that budget (or the floor of min_slots) means more
// than kMaxSlotsPerShard slots, the group's layers are dealt out in consecutive runs to as many shards
// as the limit requires, and each shard gets slots for its own runs' share of the budget (at least
// min_slots, at most the limit).
int plan_streaming(lstk_pool *P, size_t pool_bytes, uint32_t min_slots) {
    const lstk_moe_dims &d = P->dims;
    if (min_slots > kMaxSlotsPerShard)
        return fail(LSTK_E_INVALID, "min_slots = " + std::to_string(min_slots) + " is above the shard limit of " +
                                        std::to_string(kMaxSlotsPerShard) + " slots");
    using Types = std::tuple<int, int, int>;
    std::map<Types, std::vector<int>> groups; // ordered by types, layers ascending
    for (int l = 0; l < d.n_layer; l++) groups[Types(P->types[l][0], P->types[l][1], P->types[l][2])].push_back(l);
    const size_t n_layer = (size_t) d.n_layer;
    for (const auto &[types, members] : groups) {
        Shard proto;
        std::tie(proto.tu, proto.tg, proto.td) = types;
        proto.up_bytes = lstk::matrix_bytes(proto.tu, d.n_ff_exp, d.n_embd);
        proto.gate_bytes = lstk::matrix_bytes(proto.tg, d.n_ff_exp, d.n_embd);
        proto.down_bytes = lstk::matrix_bytes(proto.td, d.n_embd, d.n_ff_exp);
        proto.slab = proto.up_bytes + proto.gate_bytes + proto.down_bytes;
        const auto slots_for = [&](size_t n_layers) { return pool_bytes * n_layers / n_layer / proto.slab; };
        const size_t group_slots = std::max<size_t>(min_slots, slots_for(members.size()));
        const size_t n_shards = (group_slots + kMaxSlotsPerShard - 1) / kMaxSlotsPerShard;
        const size_t run = (members.size() + n_shards - 1) / n_shards; // layers per shard
        for (auto first = members.begin(); first != members.end();) {
            const auto last = first + (long) std::min<size_t>(run, (size_t) (members.end() - first));
            Shard sh = proto;
            sh.layers.assign(first, last);
            sh.n_slots = (uint32_t) std::clamp<size_t>(slots_for(sh.layers.size()), min_slots, kMaxSlotsPerShard);
            sh.owner_layer.assign(sh.n_slots, -1);
            sh.owner_expert.assign(sh.n_slots, -1);
            sh.refcount.assign(sh.n_slots, 0);
            sh.idle.reset(sh.n_slots);
            for (int l : sh.layers) P->layer_shard[l] = (int) P->shards.size();
            P->shards.push_back(std::move(sh));
            first = last;
        }
    }
    return LSTK_OK;
}

// Uploads the streaming pool's bookkeeping (all slots free, in LRU order) for the device-side acquire,
// and maps the host tier into the device's address space.
int init_device_lru(lstk_pool *P) {
    const lstk_moe_dims &d = P->dims;
    size_t n_slots = 0;
    for (const Shard &s : P->shards) {
        P->slot_base.push_back((int) n_slots);
        n_slots += s.n_slots;
    }
    const size_t n_map = (size_t) d.n_layer * d.n_expert, n_sh = P->shards.size(), n_ids = (size_t) d.n_batch * d.n_expert_used;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t o_map = take(n_map * 4), o_order = take(n_slots * 4), o_ol = take(n_slots * 4), o_oe = take(n_slots * 4),
                 o_stats = take(4 * 8), o_miss = take(n_ids * 8), o_nmiss = take(16);
    hipError_t e = hipMalloc(&P->dlru_mem, off);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(device LRU)");
    std::vector<uint8_t> init(off, 0);
    auto put = [&](size_t o, const int32_t *v, size_t n) { std::memcpy(init.data() + o, v, n * 4); };
    put(o_map, P->slot_of.data(), n_map);
    for (size_t i = 0; i < n_sh; i++) {
        const Shard &s = P->shards[i];
        const size_t b = (size_t) P->slot_base[i];
        const std::vector<int32_t> order = s.idle.order();
        if (order.size() != s.n_slots) return fail(LSTK_E_INVALID, "device LRU: a slot is pinned at creation");
        put(o_order + b * 4, order.data(), s.n_slots);
        put(o_ol + b * 4, s.owner_layer.data(), s.n_slots);
        put(o_oe + b * 4, s.owner_expert.data(), s.n_slots);
    }
    if ((e = hipMemcpy(P->dlru_mem, init.data(), off, hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(e, "device LRU upload");
    uint8_t *b = static_cast<uint8_t *>(P->dlru_mem);
    P->dlru.slot_of = reinterpret_cast<int32_t *>(b + o_map);
    P->dlru.order = reinterpret_cast<int32_t *>(b + o_order);
    P->dlru.owner_layer = reinterpret_cast<int32_t *>(b + o_ol);
    P->dlru.owner_expert = reinterpret_cast<int32_t *>(b + o_oe);
    P->dlru.stats = reinterpret_cast<unsigned long long *>(b + o_stats);
    P->d_miss = reinterpret_cast<int32_t *>(b + o_miss);
    P->d_n_miss = reinterpret_cast<int32_t *>(b + o_nmiss);
    void *tier_dev = nullptr;
    if ((e = hipHostGetDevicePointer(&tier_dev, P->tier, 0)) != hipSuccess) return hip_fail(e, "hipHostGetDevicePointer(host tier)");
    const ptrdiff_t shift = static_cast<uint8_t *>(tier_dev) - P->tier;
    P->tier_dev.resize(d.n_layer);
    for (int l = 0; l < d.n_layer; l++)
        for (int m = 0; m < 3; m++) P->tier_dev[l][m] = P->tier_of[l][m] + shift;
    return LSTK_OK;
}

// Engine::init's pool budget (src/engine.cpp:84-117) for a GPU with its own HBM: the whole table when it
// fits, else what the device has left after the dense weights, the KV cache and 1.5 GiB of compute
// headroom, and after keeping 3 GiB of the memory free right now for other allocations.
size_t default_pool_bytes(size_t table, size_t weights, size_t kv, size_t total, size_t free_now) {
    const size_t gib = (size_t) 1 << 30;
    const size_t used = weights + kv + gib + gib / 2;
    const size_t by_cap = total > used ? total - used : 0;
    const size_t by_free = free_now > 3 * gib ? free_now - 3 * gib : 0;
    return std::max<size_t>(std::min(table, std::min(by_cap, by_free)), (size_t) 16 << 10);
}

int create(const lstk_moe_dims *dims, const lstk_expert_layer *layers, size_t pool_bytes, uint32_t min_slots,
           uint32_t flags, lstk_pool **out) {
    if (!dims || !layers || !out) return fail(LSTK_E_INVALID, "null argument");
    *out = nullptr;
    const lstk_moe_dims &d = *dims;
    if (d.n_layer < 1 || d.n_batch < 1) return fail(LSTK_E_INVALID, "n_layer and n_batch must be >= 1");
    lstk_pool *P = new lstk_pool();
    P->dims = d;
    P->streaming = (flags & LSTK_POOL_STREAMING) != 0;
    P->dry = (flags & LSTK_POOL_DRY) != 0;
    P->device_lru = (flags & LSTK_POOL_DEVICE_LRU) != 0;
    if (P->device_lru && (!P->streaming || P->dry)) {
        destroy(P);
        return fail(LSTK_E_INVALID, "LSTK_POOL_DEVICE_LRU needs a streaming pool with device memory (not LSTK_POOL_DRY)");
    }
    P->layer_shard.assign(d.n_layer, -1);
    P->types.resize(d.n_layer);
    for (int l = 0; l < d.n_layer; l++) {
        const lstk_expert_layer &L = layers[l];
        P->types[l] = {L.type_up, L.type_gate, L.type_down};
        for (int t : P->types[l])
            if (!lstk::supported_weight_type(t)) {
                destroy(P);
                return fail(LSTK_E_INVALID, "layer " + std::to_string(l) + ": unsupported expert type " + std::to_string(t) +
                                                " (supported: 8 = Q8_0, 10 = Q2_K, 11 = Q3_K, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K)");
            }
        if (L.type_up != L.type_gate) {
            destroy(P);
            return fail(LSTK_E_INVALID, "layer " + std::to_string(l) + ": gate and up experts must share a quant type");
        }
        if (!P->dry && (!L.host_up || !L.host_gate || !L.host_down)) {
            destroy(P);
            return fail(LSTK_E_INVALID, "layer " + std::to_string(l) + ": missing expert bytes");
        }
    }
    int rc = LSTK_OK;
    if (flags & LSTK_POOL_AUTO_SIZE) {
        // size the pool from the device's memory (dense weights and KV unknown here count as 0)
        if (!P->streaming || P->dry) {
            destroy(P);
            return fail(LSTK_E_INVALID, "LSTK_POOL_AUTO_SIZE needs a streaming pool with device memory");
        }
        size_t table = 0, free_now = 0, total = 0;
        for (int l = 0; l < d.n_layer; l++)
            table += (size_t) d.n_expert * (lstk::matrix_bytes(P->types[l][0], d.n_ff_exp, d.n_embd) +
                                            lstk::matrix_bytes(P->types[l][1], d.n_ff_exp, d.n_embd) +
                                            lstk::matrix_bytes(P->types[l][2], d.n_embd, d.n_ff_exp));
        const hipError_t e = hipMemGetInfo(&free_now, &total);
        if (e != hipSuccess) {
            destroy(P);
            return hip_fail(e, "hipMemGetInfo");
        }
        pool_bytes = default_pool_bytes(table, 0, 0, total, free_now);
    }
    if (P->streaming) {
        rc = plan_streaming(P, pool_bytes, min_slots);
        if (rc != LSTK_OK) {
            destroy(P);
            return rc;
        }
        P->slot_of.assign((size_t) d.n_layer * d.n_expert, -1);
    } else {
        for (int l = 0; l < d.n_layer; l++) {
            Shard p;
            p.tu = P->types[l][0];
            p.tg = P->types[l][1];
            p.td = P->types[l][2];
            p.up_bytes = lstk::matrix_bytes(p.tu, d.n_ff_exp, d.n_embd);
            p.gate_bytes = lstk::matrix_bytes(p.tg, d.n_ff_exp, d.n_embd);
            p.down_bytes = lstk::matrix_bytes(p.td, d.n_embd, d.n_ff_exp);
            p.slab = p.up_bytes + p.gate_bytes + p.down_bytes;
            p.n_slots = (uint32_t) d.n_expert;
            p.layers = {l};
            P->layer_shard[l] = (int) P->shards.size();
            P->shards.push_back(std::move(p));
        }
    }
    for (const Shard &s : P->shards) P->n_bins_max = std::max(P->n_bins_max, (int) s.n_slots);
    const char *bad = lstk::check_shapes(d.n_embd, d.n_ff_exp, d.n_expert, d.n_expert_used, P->n_bins_max, d.n_batch);
    if (bad[0]) {
        destroy(P);
        return fail(LSTK_E_INVALID, bad);
    }
    if (P->device_lru) {
        const int ids = d.n_batch * d.n_expert_used;
        if (ids > lstk::kTierMaxIds)
            rc = fail(LSTK_E_INVALID, "LSTK_POOL_DEVICE_LRU: n_batch * n_expert_used must be at most " +
                                          std::to_string(lstk::kTierMaxIds));
        // one call pins at most min(n_batch * k, n_expert) distinct experts, so a shard of that many
        // slots never runs out inside the device-side acquire
        const int need = std::min(ids, d.n_expert);
        for (const Shard &s : P->shards) {
            if (rc != LSTK_OK) break;
            if ((int) s.n_slots < need)
                rc = fail(LSTK_E_INVALID, "LSTK_POOL_DEVICE_LRU: every shard needs at least min(n_batch * n_expert_used, "
                                          "n_expert) = " + std::to_string(need) + " slots (a shard has " +
                                              std::to_string(s.n_slots) + "); raise the pool size or lower n_batch");
            else if (s.up_bytes % 16 || s.gate_bytes % 16 || s.down_bytes % 16)
                rc = fail(LSTK_E_INVALID, "LSTK_POOL_DEVICE_LRU: expert matrices must be multiples of 16 bytes");
        }
        if (rc != LSTK_OK) {
            destroy(P);
            return rc;
        }
    }
    if (P->dry) {
        *out = P;
        return LSTK_OK;
    }
    hipError_t e = hipGetDevice(&P->device);
    if (e != hipSuccess) {
        destroy(P);
        return hip_fail(e, "hipGetDevice");
    }
    // HBM slots
    for (Shard &s : P->shards) {
        if ((e = hipMalloc(&s.d_up, s.up_bytes * s.n_slots)) != hipSuccess ||
            (e = hipMalloc(&s.d_gate, s.gate_bytes * s.n_slots)) != hipSuccess ||
            (e = hipMalloc(&s.d_down, s.down_bytes * s.n_slots)) != hipSuccess) {
            destroy(P);
            return fail(LSTK_E_NOMEM, std::string("cannot allocate expert pool memory: ") + hipGetErrorString(e));
        }
    }
    const int h = d.n_embd, f = d.n_ff_exp, E = d.n_expert;
    if (P->streaming) {
        // pinned host tier with every layer's experts in pool layout (the stand-in for the GGUF file);
        // layers that pass the same host matrices (and so the same types) share one copy
        std::vector<int> first_of(d.n_layer);
        size_t total = 0;
        for (int l = 0; l < d.n_layer; l++) {
            first_of[l] = l;
            for (int q = 0; q < l; q++) {
                if (first_of[q] == q && layers[q].host_up == layers[l].host_up &&
                    layers[q].host_gate == layers[l].host_gate && layers[q].host_down == layers[l].host_down &&
                    layers[q].type_up == layers[l].type_up && layers[q].type_gate == layers[l].type_gate &&
                    layers[q].type_down == layers[l].type_down) {
                    first_of[l] = q;
                    break;
                }
            }
            if (first_of[l] == l) total += (size_t) E * P->shards[P->layer_shard[l]].slab;
        }
        if ((e = hipHostMalloc((void **) &P->tier, total, hipHostMallocDefault)) != hipSuccess) {
            destroy(P);
            return fail(LSTK_E_NOMEM, std::string("cannot allocate the pinned host tier: ") + hipGetErrorString(e));
        }
        size_t off = 0;
        P->tier_of.resize(d.n_layer);
        for (int l = 0; l < d.n_layer; l++) {
            if (first_of[l] != l) {
                P->tier_of[l] = P->tier_of[first_of[l]];
                continue;
            }
            const Shard &s = P->shards[P->layer_shard[l]];
            uint8_t *u = P->tier + off, *g = u + (size_t) E * s.up_bytes, *dn = g + (size_t) E * s.gate_bytes;
            P->tier_of[l] = {u, g, dn};
            off += (size_t) E * s.slab;
            if ((rc = repack_experts(s.tu, f, h, E, layers[l].host_up, u)) != LSTK_OK ||
                (rc = repack_experts(s.tg, f, h, E, layers[l].host_gate, g)) != LSTK_OK ||
                (rc = repack_experts(s.td, h, f, E, layers[l].host_down, dn)) != LSTK_OK) {
                destroy(P);
                return rc;
            }
        }
        for (int i = 0; i < kSides && e == hipSuccess; i++)
            if ((e = hipStreamCreateWithFlags(&P->side[i], hipStreamNonBlocking)) == hipSuccess)
                e = hipEventCreateWithFlags(&P->copy_done[i], hipEventDisableTiming);
        if (e != hipSuccess || (e = hipEventCreateWithFlags(&P->release_ev, hipEventDisableTiming)) != hipSuccess) {
            destroy(P);
            return hip_fail(e, "side streams / events");
        }
    } else {
        // resident: repack each layer's experts on the host and upload them once
        size_t maxb = 0;
        for (const Shard &s : P->shards) maxb = std::max({maxb, s.up_bytes, s.gate_bytes, s.down_bytes});
        std::vector<uint8_t> staging((size_t) E * maxb);
        for (int l = 0; l < d.n_layer; l++) {
            Shard &s = P->shards[P->layer_shard[l]];
            const struct {
                int type, rows, cols;
                const void *src;
                uint8_t *dst;
                size_t bytes;
            } mats[3] = {{s.tu, f, h, layers[l].host_up, s.d_up, s.up_bytes},
                         {s.tg, f, h, layers[l].host_gate, s.d_gate, s.gate_bytes},
                         {s.td, h, f, layers[l].host_down, s.d_down, s.down_bytes}};
            for (const auto &m : mats) {
                if ((rc = repack_experts(m.type, m.rows, m.cols, E, m.src, staging.data())) != LSTK_OK) {
                    destroy(P);
                    return rc;
                }
                if ((e = hipMemcpy(m.dst, staging.data(), (size_t) E * m.bytes, hipMemcpyHostToDevice)) != hipSuccess) {
                    destroy(P);
                    return hip_fail(e, "hipMemcpy(experts)");
                }
            }
        }
    }
    if ((rc = alloc_scratch(P)) != LSTK_OK || (P->device_lru && (rc = init_device_lru(P)) != LSTK_OK) ||
        (rc = noalloc_address(P->device, &P->noalloc)) != LSTK_OK) {
        destroy(P);
        return rc;
    }
    *out = P;
    return LSTK_OK;
}

// Issues the three host-tier -> HBM copies of a miss on side stream `side`.
int copy_in(lstk_pool *P, int layer, const Shard &s, int32_t slot, int32_t expert, hipStream_t side) {
    if (P->fail_copies > 0) {
        P->fail_copies--;
        return fail(LSTK_E_IO, "expert copy failed (injected) for layer " + std::to_string(layer) + " expert " +
                                   std::to_string(expert));
    }
    if (P->dry) return LSTK_OK;
    const auto &t = P->tier_of[layer];
    const size_t b[3] = {s.up_bytes, s.gate_bytes, s.down_bytes};
    uint8_t *dst[3] = {s.d_up, s.d_gate, s.d_down};
    for (int m = 0; m < 3; m++) {
        const hipError_t e = hipMemcpyAsync(dst[m] + (size_t) slot * b[m], t[m] + (size_t) expert * b[m], b[m],
                                            hipMemcpyHostToDevice, side);
        if (e != hipSuccess)
            return fail(LSTK_E_IO, std::string("expert copy failed for layer ") + std::to_string(layer) + ": " +
                                       hipGetErrorString(e));
    }
    return LSTK_OK;
}

// ExpertStore::acquire (src/expert_store.cpp:232-286). As in the reference, a miss records its slot
// in slot_of at once, so a repeat of the expert later in the same call counts as a hit.
int acquire(lstk_pool *P, int layer, const int32_t *experts, int n, int32_t *slots, hipStream_t stream) {
    const lstk_moe_dims &d = P->dims;
    if (layer < 0 || layer >= d.n_layer || n < 0 || (n > 0 && (!experts || !slots)))
        return fail(LSTK_E_INVALID, "acquire: bad arguments");
    for (int i = 0; i < n; i++)
        if (experts[i] < 0 || experts[i] >= d.n_expert)
            return fail(LSTK_E_INVALID, "acquire: expert id " + std::to_string(experts[i]) + " out of range");
    if (P->device_lru) return fail(LSTK_E_INVALID, "this pool keeps its bookkeeping on the device: use lstk_pool_acquire_device");
    const auto t0 = std::chrono::steady_clock::now();
    P->stats.acquires++;
    if (!P->streaming) {
        for (int i = 0; i < n; i++) slots[i] = experts[i];
        P->stats.hits += (uint64_t) n;
        P->stats.wait_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        return LSTK_OK;
    }
    const int sh = P->layer_shard[layer];
    Shard &p = P->shards[sh];
    std::vector<std::pair<int32_t, int32_t>> misses; // (slot, expert)
    int rc = LSTK_OK;
    for (int i = 0; i < n; i++) {
        const int32_t e = experts[i];
        int32_t &ref = P->slot_of[(size_t) layer * d.n_expert + e];
        if (ref >= 0) {
            const int32_t s = ref;
            if (p.refcount[s] == 0) p.idle.withdraw(s);
            p.refcount[s]++;
            P->pinned.push_back({sh, s});
            slots[i] = s;
            P->stats.hits++;
            continue;
        }
        const int32_t s = p.idle.take_oldest();
        if (s < 0) {
            rc = fail(LSTK_E_EXHAUSTED, "no idle slot for layer " + std::to_string(layer) + ": this call pins all " +
                                            std::to_string(p.n_slots) + " slots of its shard (pool exhausted); create the "
                                            "pool with more bytes or pass fewer tokens per call");
            break;
        }
        if (p.owner_layer[s] >= 0) P->slot_of[(size_t) p.owner_layer[s] * d.n_expert + p.owner_expert[s]] = -1;
        p.owner_layer[s] = layer;
        p.owner_expert[s] = e;
        ref = s;
        p.refcount[s] = 1;
        P->pinned.push_back({sh, s});
        slots[i] = s;
        misses.push_back({s, e});
        P->stats.misses++;
        P->stats.bytes_read += p.slab;
    }
    if (!misses.empty()) {
        hipError_t e = hipSuccess;
        const int n_used = std::min<int>(kSides, (int) misses.size());
        // a slot released by earlier compute may only be overwritten once that compute has finished
        for (int i = 0; i < n_used && !P->dry && e == hipSuccess; i++) e = hipStreamWaitEvent(P->side[i], P->release_ev, 0);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamWaitEvent(side)");
        for (size_t mi = 0; mi < misses.size(); mi++) {
            const auto &[s, ex] = misses[mi];
            const int crc = copy_in(P, layer, p, s, ex, P->side[mi % n_used]);
            if (crc != LSTK_OK) {
                // the slot holds no valid expert: unmap it rather than serve garbage
                P->slot_of[(size_t) layer * d.n_expert + ex] = -1;
                p.owner_layer[s] = -1;
                p.owner_expert[s] = -1;
                rc = crc;
            }
        }
        for (int i = 0; i < n_used && !P->dry; i++) {
            if ((e = hipEventRecord(P->copy_done[i], P->side[i])) != hipSuccess ||
                (e = hipStreamWaitEvent(stream, P->copy_done[i], 0)) != hipSuccess) {
                rc = hip_fail(e, "copy event");
                break;
            }
        }
    }
    P->stats.wait_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return rc;
}

int release_all(lstk_pool *P, hipStream_t stream) {
    for (const auto &[sh, s] : P->pinned) {
        Shard &p = P->shards[sh];
        if (--p.refcount[s] == 0) p.idle.append(s);
    }
    P->pinned.clear();
    if (P->streaming && !P->dry) {
        const hipError_t e = hipEventRecord(P->release_ev, stream);
        if (e != hipSuccess) return hip_fail(e, "hipEventRecord(release)");
    }
    return LSTK_OK;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ExpertStore::acquire + release_all of one segment on the device (tier.hip): resolve, then copy the
// misses from the host tier. Nothing waits on the host.
int acquire_device(lstk_pool *P, int layer, const int32_t *d_experts, int n, int32_t *d_slots, hipStream_t st) {
    const lstk_moe_dims &d = P->dims;
    if (!P->device_lru) return fail(LSTK_E_INVALID, "lstk_pool_acquire_device needs a pool created with LSTK_POOL_DEVICE_LRU");
    if (layer < 0 || layer >= d.n_layer) return fail(LSTK_E_INVALID, "acquire_device: bad layer");
    if (n < 0 || n > d.n_batch * d.n_expert_used)
        return fail(LSTK_E_INVALID, "acquire_device: n must be in [0, n_batch * n_expert_used]");
    if (n == 0) return LSTK_OK;
    if (!d_experts || !d_slots || !aligned(d_experts, 4) || !aligned(d_slots, 4))
        return fail(LSTK_E_INVALID, "acquire_device: experts and slots must be non-null device arrays");
    const int sh = P->layer_shard[layer];
    const Shard &s = P->shards[sh];
    lstk::TierResolveParams rp{};
    rp.lru = P->dlru;
    rp.layer = layer;
    rp.E = d.n_expert;
    rp.shard = sh;
    rp.slot_base = P->slot_base[sh];
    rp.n_slots = (int) s.n_slots;
    rp.slab = s.slab;
    rp.experts = d_experts;
    rp.n = n;
    rp.slots = d_slots;
    rp.miss = P->d_miss;
    rp.n_miss = P->d_n_miss;
    rp.err = P->err;
    hipError_t e = lstk::launch_tier_resolve(rp, st, nullptr);
    if (e != hipSuccess) return hip_fail(e, "tier resolve launch");
    lstk::TierCopyParams cp{};
    cp.miss = P->d_miss;
    cp.n_miss = P->d_n_miss;
    cp.max_miss = n;
    cp.n_slots = (int) s.n_slots;
    cp.E = d.n_expert;
    const size_t b[3] = {s.up_bytes, s.gate_bytes, s.down_bytes};
    uint8_t *dst[3] = {s.d_up, s.d_gate, s.d_down};
    for (int m = 0; m < 3; m++) {
        cp.src[m] = P->tier_dev[layer][m];
        cp.dst[m] = dst[m];
        cp.bytes[m] = b[m];
        cp.chunks[m] = lstk::tier_copy_chunks(b[m]);
    }
    e = lstk::launch_tier_copy(cp, st, nullptr);
    return e == hipSuccess ? LSTK_OK : hip_fail(e, "tier copy launch");
}

// Runs one launch; with timing on, the launch records its own start/stop timestamps.
template <typename F>
hipError_t timed(lstk_pool *P, int stage, F &&launch) {
    if (!P->timing) return launch(nullptr);
    TimedLaunch t{};
    hipError_t e;
    if ((e = hipEventCreate(&t.start)) != hipSuccess) return e;
    if ((e = hipEventCreate(&t.end)) != hipSuccess) return e;
    lstk::LaunchTiming tm;
    tm.start = t.start;
    tm.stop = t.end;
    const hipError_t le = launch(&tm);
    P->launched[stage].push_back(t);
    return le;
}


int check_call(lstk_pool *P, int layer, int T) {
    if (!P) return fail(LSTK_E_INVALID, "null pool");
    if (P->dry) return fail(LSTK_E_INVALID, "a dry pool has no device memory");
    if (layer < 0 || layer >= P->dims.n_layer) return fail(LSTK_E_INVALID, "layer out of range");
    if (T < 0 || T > P->dims.n_batch)
        return fail(LSTK_E_INVALID, "n_tokens " + std::to_string(T) + " outside [0, n_batch = " +
                                        std::to_string(P->dims.n_batch) + "]");
    return LSTK_OK;
}

// The grouped MFMA path serves calls with many tokens per expert (prefill): Q4_K gate, up and down,
// at least grouped_min_tokens tokens (LSTK_GROUPED_MIN_TOKENS overrides the default of 64).
bool use_grouped(lstk_pool *P, const Shard &s, int T) {
    if (P->grouped_min_tokens == 0) {
        const char *env = std::getenv("LSTK_GROUPED_MIN_TOKENS");
        P->grouped_min_tokens = env ? std::max(1, std::atoi(env)) : 64;
    }
    return T >= P->grouped_min_tokens &&
           lstk::grouped_supported(s.tu, s.tg, s.td, P->dims.n_embd, P->dims.n_ff_exp, (int) s.n_slots);
}

// permute -> gate_up (MFMA, SwiGLU) -> Q8_K of the SwiGLU rows -> down (MFMA, router weight) ->
// combine + residual. bins: expert ids (resident) or slots (streaming), [T][k].
int run_grouped(lstk_pool *P, const Shard &s, const int32_t *bins, const float *d_weights, const float *d_resid,
                float *d_out, int T, hipStream_t st) {
    const lstk_moe_dims &d = P->dims;
    const int k = d.n_expert_used, np = T * k, h = d.n_embd, f = d.n_ff_exp;
    const int max_items = lstk::grouped_max_items(np, (int) s.n_slots);
    lstk::PermuteParams pp{bins, np, (int) s.n_slots, lstk::kGroupedChunk, P->counts, P->offsets, P->perm,
                           P->items, P->n_items, P->err};
    hipError_t e = timed(P, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_permute(pp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "permute launch");
    lstk::GroupedParams gu{};
    gu.items = P->items;
    gu.n_items = P->n_items;
    gu.perm = P->perm;
    gu.k = k;
    gu.w0 = s.d_gate;
    gu.w1 = s.d_up;
    gu.stride0 = s.gate_bytes;
    gu.stride1 = s.up_bytes;
    gu.rows = f;
    gu.K = h;
    gu.xqs = P->xq.qs;
    gu.xd = P->xq.d;
    gu.xbh = P->xq.bh;
    gu.row_div = k;
    gu.out = P->act;
    e = timed(P, 1, [&](const lstk::LaunchTiming *tm) { return lstk::launch_gate_up_grouped(gu, max_items, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "gate_up launch");
    e = timed(P, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_act_quant(P->act, f, np, P->aq, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "act quant launch");
    lstk::GroupedParams dn = gu;
    dn.w0 = s.d_down;
    dn.w1 = nullptr;
    dn.stride0 = s.down_bytes;
    dn.stride1 = 0;
    dn.rows = h;
    dn.K = f;
    dn.xqs = P->aq.qs;
    dn.xd = P->aq.d;
    dn.xbh = P->aq.bh;
    dn.row_div = 1;
    dn.weights = d_weights;
    dn.out = P->Y;
    e = timed(P, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_down_grouped(dn, max_items, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "down launch");
    if (P->defer_combine) return LSTK_OK;
    lstk::CombineParams cp{P->Y, d_resid, d_out, T, k, h};
    e = timed(P, 3, [&](const lstk::LaunchTiming *tm) { return lstk::launch_combine(cp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return LSTK_OK;
}

// The fused single-token path (one launch per block) is opt-in: LSTK_FUSED_DECODE=1 at pool creation.
// On MI355X its in-kernel hand-overs (device-coherent polls and reads, about 2 us each) cost more
// than the kernel boundaries they replace (about 1.6 us in a replayed graph), so the multi-kernel
// path is the default. It runs when every work-group of its grid fits on the device at once
// (checked once per type combination).
bool use_fused(lstk_pool *P, const Shard &s, int gate_type) {
    if (!P->fused_enabled || !P->fl.ok || s.tu != s.tg) return false;
    const std::array<int, 4> key{gate_type, s.tg, s.td, 0};
    auto it = P->fused_fit.find(key);
    if (it == P->fused_fit.end())
        it = P->fused_fit
                 .emplace(key, lstk::fused_fits(P->fl, gate_type, s.tg, s.td, P->dims.n_embd, P->dims.n_ff_exp,
                                                P->dims.n_expert_used))
                 .first;
    return it->second;
}

int run_fused(lstk_pool *P, const Shard &s, int mode, const float *d_hnorm, const void *d_gate_inp, int gate_type,
              const int32_t *d_slots, int32_t *d_ids, float *d_weights, const float *d_resid, float *d_out, hipStream_t st) {
    const lstk_moe_dims &d = P->dims;
    lstk::FusedParams fp{};
    fp.hnorm = d_hnorm;
    fp.gate_inp = d_gate_inp;
    fp.route = mode == 1;
    fp.ids_in = d_slots;
    fp.weights_in = d_weights;
    fp.ids_out = d_ids;
    fp.weights_out = d_weights;
    fp.h = d.n_embd;
    fp.f = d.n_ff_exp;
    fp.E = d.n_expert;
    fp.k = d.n_expert_used;
    fp.n_bins = (int) s.n_slots;
    fp.w_gate = s.d_gate;
    fp.w_up = s.d_up;
    fp.w_down = s.d_down;
    fp.s_gate = s.gate_bytes;
    fp.s_up = s.up_bytes;
    fp.s_down = s.down_bytes;
    fp.resid = d_resid;
    fp.out = d_out;
    fp.logits = P->logits;
    fp.act = P->act;
    fp.cnt = P->f_cnt;
    fp.flag_a = P->f_flag_a;
    fp.flag_b = P->f_flag_b;
    fp.err = P->err;
    fp.nA = P->fl.nA;
    fp.nB = P->fl.nB;
    fp.nC = P->fl.nC;
    fp.ub = P->fl.ub;
    fp.rd = P->fl.rd;
    fp.spin_max = 200000;
    const hipError_t e = timed(P, 1, [&](const lstk::LaunchTiming *tm) {
        return lstk::launch_fused(fp, mode == 1 ? gate_type : lstk::kTypeF16, s.tg, s.td, st, tm);
    });
    return e == hipSuccess ? LSTK_OK : hip_fail(e, "fused launch");
}

// Router (optional) + experts + combine of one layer. mode 0: ffn with caller slots / weights;
// mode 1: resident block, routing from gate_inp, ids / weights written to d_ids / d_weights.
// The ffn_norm input of a one-token block whose router launch normalises the row itself.
struct NormIn {
    const float *x, *w;
    float eps;
};

// Per-call device scratch of the GEMV path: the pool's own (sized for n_batch at creation) or a layout in
// the fixed array of lstk_moe_block_noalloc.
struct CallScratch {
    lstk::ActBuf xq;
    float *logits, *act, *Y;
};

// Bytes of a CallScratch for T tokens, and its layout from `base` when base is non-null.
size_t call_scratch_layout(const lstk_moe_dims &d, int T, uint8_t *base, CallScratch *out) {
    const size_t t = (size_t) T, h = (size_t) d.n_embd, k = (size_t) d.n_expert_used;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return base + o;
    };
    uint8_t *qs = take(t * h), *xd = take(t * (h / 32) * 4), *bs = take(t * (h / 32) * 4);
    uint8_t *lg = take(t * (size_t) d.n_expert * 4), *act = take(t * k * (size_t) d.n_ff_exp * 4), *Y = take(t * k * h * 4);
    if (base && out) {
        out->xq.qs = reinterpret_cast<int8_t *>(qs);
        out->xq.d = reinterpret_cast<float *>(xd);
        out->xq.bs = reinterpret_cast<int32_t *>(bs);
        out->xq.bh = nullptr;
        out->logits = reinterpret_cast<float *>(lg);
        out->act = reinterpret_cast<float *>(act);
        out->Y = reinterpret_cast<float *>(Y);
    }
    return off;
}

// fixed != null (lstk_moe_block_noalloc): the scratch comes from the fixed array, and the call takes
// neither the fused nor the grouped path (their counters and work lists live in the pool's scratch)
// nor the stage timing (which creates events).
int run_block(lstk_pool *P, int layer, int mode, const float *d_hnorm, const void *d_gate_inp, int gate_type,
              const int32_t *d_slots, int32_t *d_ids, float *d_weights, const float *d_resid, float *d_out, int T,
              hipStream_t st, const NormIn *norm = nullptr, const CallScratch *fixed = nullptr) {
    const lstk_moe_dims &d = P->dims;
    const Shard &s = P->shards[P->layer_shard[layer]];
    const int k = d.n_expert_used;
    if (!fixed && T == 1 && !norm && use_fused(P, s, mode == 1 ? gate_type : lstk::kTypeF16))
        return run_fused(P, s, mode, d_hnorm, d_gate_inp, gate_type, d_slots, d_ids, d_weights, d_resid, d_out, st);
    const CallScratch sc = fixed ? *fixed : CallScratch{P->xq, P->logits, P->act, P->Y};
    auto timed = [&](lstk_pool *pool, int stage, auto &&launch) -> hipError_t {
        return fixed ? launch(nullptr) : ::timed(pool, stage, launch);
    };
    lstk::RouteParams rp{};
    rp.hnorm = d_hnorm;
    if (norm) {
        rp.x_raw = norm->x;
        rp.norm_w = norm->w;
        rp.eps = norm->eps;
        rp.hnorm_out = const_cast<float *>(d_hnorm);
    }
    rp.T = T;
    rp.h = d.n_embd;
    rp.do_route = mode == 1;
    rp.gate_inp = d_gate_inp;
    rp.gate_type = gate_type;
    rp.E = d.n_expert;
    rp.logits = sc.logits;
    rp.qtype = s.tu;
    rp.xq = sc.xq;
    const bool grouped = !fixed && use_grouped(P, s, T);
    if (!grouped) rp.xq.bh = nullptr; // only the grouped kernels read the split group sums
    hipError_t e = timed(P, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_route(rp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "route launch");
    const bool fused_topk = mode == 1 && T <= lstk::decode_route_max_tokens();
    if (mode == 1 && !fused_topk) {
        lstk::TopkParams tp{sc.logits, T, d.n_expert, k, d_ids, d_weights};
        e = timed(P, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_topk(tp, st, tm); });
        if (e != hipSuccess) return hip_fail(e, "topk launch");
    }
    if (grouped)
        return run_grouped(P, s, mode == 1 ? d_ids : d_slots, d_weights, d_resid, d_out, T, st);
    lstk::GroupParams gp{};
    gp.T = T;
    gp.k = k;
    gp.n_bins = (int) s.n_slots;
    gp.route = fused_topk ? 1 : 0;
    gp.ids = mode == 1 ? d_ids : d_slots;
    gp.logits = sc.logits;
    gp.E = d.n_expert;
    gp.ids_out = d_ids;
    gp.weights_out = d_weights;
    gp.err = P->err;
    const int max_active = std::min<int>((int) s.n_slots, T * k);
    lstk::GateUpParams gu{};
    gu.gp = gp;
    gu.w_gate = s.d_gate;
    gu.w_up = s.d_up;
    gu.stride_gate = s.gate_bytes;
    gu.stride_up = s.up_bytes;
    gu.type = s.tu;
    gu.f = d.n_ff_exp;
    gu.h = d.n_embd;
    gu.xq = sc.xq;
    gu.max_active = max_active;
    gu.act = sc.act;
    e = timed(P, 1, [&](const lstk::LaunchTiming *tm) { return lstk::launch_gate_up(gu, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "gate_up launch");
    if (T == 1 && lstk::down_combine_supported(d.n_embd, d.n_ff_exp, k)) {
        // one token: down, router weights, combine and residual in one launch
        lstk::DownCombineParams dc{};
        dc.ids = gp.ids;
        dc.weights = d_weights;
        dc.k = k;
        dc.n_bins = (int) s.n_slots;
        dc.w_down = s.d_down;
        dc.stride_down = s.down_bytes;
        dc.type = s.td;
        dc.h = d.n_embd;
        dc.f = d.n_ff_exp;
        dc.act = sc.act;
        dc.resid = d_resid;
        dc.out = d_out;
        dc.err = P->err;
        e = timed(P, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_down_combine(dc, st, tm); });
        return e == hipSuccess ? LSTK_OK : hip_fail(e, "down_combine launch");
    }
    lstk::DownParams dn{};
    dn.gp = gp;
    dn.gp.route = 0;
    dn.w_down = s.d_down;
    dn.stride_down = s.down_bytes;
    dn.type = s.td;
    dn.h = d.n_embd;
    dn.f = d.n_ff_exp;
    dn.act = sc.act;
    dn.weights = d_weights;
    dn.max_active = max_active;
    dn.Y = sc.Y;
    e = timed(P, 2, [&](const lstk::LaunchTiming *tm) { return lstk::launch_down(dn, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "down launch");
    if (P->defer_combine && !fixed && T > 1) return LSTK_OK;
    lstk::CombineParams cp{sc.Y, d_resid, d_out, T, k, d.n_embd};
    e = timed(P, 3, [&](const lstk::LaunchTiming *tm) { return lstk::launch_combine(cp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return LSTK_OK;
}

int check_router_args(const void *d_gate_inp, int gate_type) {
    if (gate_type != lstk::kTypeF16 && gate_type != lstk::kTypeF32)
        return fail(LSTK_E_INVALID, "gate_inp type must be F16 (1) or F32 (0)");
    if (!d_gate_inp || !aligned(d_gate_inp, gate_type == lstk::kTypeF16 ? 8 : 16))
        return fail(LSTK_E_INVALID, "gate_inp must be non-null and 8 (F16) / 16 (F32) byte aligned");
    return LSTK_OK;
}

int check_act(const float *p, const char *name) {
    if (!p || !aligned(p, 16)) return fail(LSTK_E_INVALID, std::string(name) + " must be non-null and 16-byte aligned");
    return LSTK_OK;
}

}  // namespace

namespace lstk {
int set_error(int code, const std::string &msg) { return fail(code, msg); }
const lstk_moe_dims &pool_dims(const lstk_pool *pool) { return pool->dims; }
bool pool_streaming(const lstk_pool *pool) { return pool->streaming; }
bool pool_dry(const lstk_pool *pool) { return pool->dry; }
bool pool_device_lru(const lstk_pool *pool) { return pool->device_lru; }
void pool_defer_combine(lstk_pool *pool, bool on) { pool->defer_combine = on; }
const float *pool_moe_rows(const lstk_pool *pool) { return pool->Y; }

int moe_block_normed(lstk_pool *pool, int layer, const float *d_x, const float *d_norm_w, float eps, float *d_hnorm,
                     const void *d_gate_inp, int gate_type, const float *d_resid, float *d_out, int32_t *d_ids,
                     float *d_weights, int T, hipStream_t st) {
    int rc;
    if ((rc = check_call(pool, layer, T)) != LSTK_OK) return rc;
    if (pool->streaming) return fail(LSTK_E_INVALID, "moe_block_normed needs a resident pool");
    if ((rc = check_router_args(d_gate_inp, gate_type)) != LSTK_OK || (rc = check_act(d_x, "x")) != LSTK_OK ||
        (rc = check_act(d_norm_w, "norm_w")) != LSTK_OK || (rc = check_act(d_hnorm, "hnorm")) != LSTK_OK ||
        (rc = check_act(d_resid, "resid")) != LSTK_OK || (rc = check_act(d_out, "out")) != LSTK_OK)
        return rc;
    if (!d_ids || !d_weights) return fail(LSTK_E_INVALID, "ids and weights must be non-null");
    const NormIn norm{d_x, d_norm_w, eps};
    return run_block(pool, layer, 1, d_hnorm, d_gate_inp, gate_type, nullptr, d_ids, d_weights, d_resid, d_out, T, st,
                     &norm);
}
}  // namespace lstk

extern "C" {

const char *lstk_last_error(void) { return g_err.c_str(); }
int lstk_abi_version(void) { return LSTK_ABI_VERSION; }

int lstk_pool_create(const lstk_moe_dims *dims, const lstk_expert_layer *layers, size_t pool_bytes, uint32_t min_slots,
                     uint32_t flags, lstk_pool **out) {
    try {
        return create(dims, layers, pool_bytes, min_slots, flags, out);
    } catch (const std::exception &ex) {
        return fail(LSTK_E_NOMEM, std::string("lstk_pool_create: ") + ex.what());
    }
}

void lstk_pool_destroy(lstk_pool *pool) { destroy(pool); }

size_t lstk_pool_default_bytes(size_t table_bytes, size_t weight_bytes, size_t kv_bytes, size_t device_total,
                               size_t device_free) {
    return default_pool_bytes(table_bytes, weight_bytes, kv_bytes, device_total, device_free);
}

int lstk_pool_acquire(lstk_pool *pool, int layer, const int32_t *experts, int n, int32_t *slots, lstk_stream_t stream) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    return acquire(pool, layer, experts, n, slots, static_cast<hipStream_t>(stream));
}

int lstk_pool_acquire_device(lstk_pool *pool, int layer, const int32_t *d_experts, int n, int32_t *d_slots,
                             lstk_stream_t stream) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    return acquire_device(pool, layer, d_experts, n, d_slots, static_cast<hipStream_t>(stream));
}

int lstk_pool_release_all(lstk_pool *pool, lstk_stream_t stream) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    return release_all(pool, static_cast<hipStream_t>(stream));
}

int lstk_pool_stats(const lstk_pool *pool, lstk_pool_stats_t *out) {
    if (!pool || !out) return fail(LSTK_E_INVALID, "null argument");
    *out = pool->stats;
    if (pool->device_lru) {
        unsigned long long c[4];
        const hipError_t e = hipMemcpy(c, pool->dlru.stats, sizeof(c), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "device LRU counters");
        out->hits = c[0];
        out->misses = c[1];
        out->bytes_read = c[2];
        out->acquires = c[3];
    }
    return LSTK_OK;
}

size_t lstk_pool_total_bytes(const lstk_pool *pool) {
    size_t t = 0;
    if (pool)
        for (const Shard &s : pool->shards) t += s.slab * s.n_slots;
    return t;
}

uint32_t lstk_pool_total_slots(const lstk_pool *pool) {
    uint32_t t = 0;
    if (pool)
        for (const Shard &s : pool->shards) t += s.n_slots;
    return t;
}

int lstk_pool_layer_slots(const lstk_pool *pool, int layer) {
    if (!pool || layer < 0 || layer >= pool->dims.n_layer) return fail(LSTK_E_INVALID, "bad layer");
    return (int) pool->shards[pool->layer_shard[layer]].n_slots;
}

int lstk_pool_describe(const lstk_pool *pool, char *buf, size_t len) {
    if (!pool || !buf || len == 0) return fail(LSTK_E_INVALID, "null argument");
    std::string s;
    char line[256];
    for (const Shard &p : pool->shards) {
        snprintf(line, sizeof(line), "  pool %s/%s/%s: %zu layers, %u slots x %.2f MiB = %.2f GiB\n", type_name(p.tu),
                 type_name(p.tg), type_name(p.td), p.layers.size(), p.n_slots, p.slab / 1048576.0,
                 p.slab * (double) p.n_slots / 1073741824.0);
        s += line;
    }
    snprintf(buf, len, "%s", s.c_str());
    return LSTK_OK;
}

int lstk_moe_route(lstk_pool *pool, int layer, const float *d_hnorm, int n_tokens, const void *d_gate_inp, int gate_type,
                   int32_t *d_ids, float *d_weights, lstk_stream_t stream) {
    int rc;
    if ((rc = check_call(pool, layer, n_tokens)) != LSTK_OK) return rc;
    if (n_tokens == 0) return LSTK_OK;
    if ((rc = check_router_args(d_gate_inp, gate_type)) != LSTK_OK || (rc = check_act(d_hnorm, "hnorm")) != LSTK_OK) return rc;
    if (!d_ids || !d_weights) return fail(LSTK_E_INVALID, "ids and weights must be non-null");
    hipStream_t st = static_cast<hipStream_t>(stream);
    lstk::RouteParams rp{};
    rp.hnorm = d_hnorm;
    rp.T = n_tokens;
    rp.h = pool->dims.n_embd;
    rp.do_route = 1;
    rp.gate_inp = d_gate_inp;
    rp.gate_type = gate_type;
    rp.E = pool->dims.n_expert;
    rp.logits = pool->logits;
    rp.qtype = 0;
    hipError_t e = timed(pool, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_route(rp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "route launch");
    lstk::TopkParams tp{pool->logits, n_tokens, pool->dims.n_expert, pool->dims.n_expert_used, d_ids, d_weights};
    e = timed(pool, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_topk(tp, st, tm); });
    if (e != hipSuccess) return hip_fail(e, "topk launch");
    return LSTK_OK;
}

int lstk_moe_ffn(lstk_pool *pool, int layer, const float *d_hnorm, const int32_t *d_slots, const float *d_weights,
                 const float *d_resid, float *d_out, int n_tokens, lstk_stream_t stream) {
    int rc;
    if ((rc = check_call(pool, layer, n_tokens)) != LSTK_OK) return rc;
    if (n_tokens == 0) return LSTK_OK;
    if ((rc = check_act(d_hnorm, "hnorm")) != LSTK_OK || (rc = check_act(d_resid, "resid")) != LSTK_OK ||
        (rc = check_act(d_out, "out")) != LSTK_OK)
        return rc;
    if (!d_slots || !d_weights) return fail(LSTK_E_INVALID, "slots and weights must be non-null");
    return run_block(pool, layer, 0, d_hnorm, nullptr, 0, d_slots, nullptr, const_cast<float *>(d_weights), d_resid, d_out,
                     n_tokens, static_cast<hipStream_t>(stream));
}

int lstk_moe_block(lstk_pool *pool, int layer, const float *d_hnorm, const void *d_gate_inp, int gate_type,
                   const float *d_resid, float *d_out, int32_t *d_ids, float *d_weights, int n_tokens,
                   lstk_stream_t stream) {
    int rc;
    if ((rc = check_call(pool, layer, n_tokens)) != LSTK_OK) return rc;
    if (pool->streaming) return fail(LSTK_E_INVALID, "lstk_moe_block needs a resident pool; use route + acquire + ffn");
    if (n_tokens == 0) return LSTK_OK;
    if ((rc = check_router_args(d_gate_inp, gate_type)) != LSTK_OK || (rc = check_act(d_hnorm, "hnorm")) != LSTK_OK ||
        (rc = check_act(d_resid, "resid")) != LSTK_OK || (rc = check_act(d_out, "out")) != LSTK_OK)
        return rc;
    if (!d_ids || !d_weights) return fail(LSTK_E_INVALID, "ids and weights must be non-null");
    return run_block(pool, layer, 1, d_hnorm, d_gate_inp, gate_type, nullptr, d_ids, d_weights, d_resid, d_out, n_tokens,
                     static_cast<hipStream_t>(stream));
}

int lstk_moe_block_noalloc(lstk_pool *pool, int layer, const float *d_hnorm, const void *d_gate_inp, int gate_type,
                           const float *d_resid, float *d_out, int32_t *d_ids, float *d_weights, int n_tokens,
                           lstk_stream_t stream) {
    int rc;
    if ((rc = check_call(pool, layer, n_tokens)) != LSTK_OK) return rc;
    if (pool->streaming) return fail(LSTK_E_INVALID, "lstk_moe_block_noalloc needs a resident pool");
    if (n_tokens == 0) return LSTK_OK;
    if ((rc = check_router_args(d_gate_inp, gate_type)) != LSTK_OK || (rc = check_act(d_hnorm, "hnorm")) != LSTK_OK ||
        (rc = check_act(d_resid, "resid")) != LSTK_OK || (rc = check_act(d_out, "out")) != LSTK_OK)
        return rc;
    if (!d_ids || !d_weights) return fail(LSTK_E_INVALID, "ids and weights must be non-null");
    const size_t need = call_scratch_layout(pool->dims, n_tokens, nullptr, nullptr);
    if (need > kNoAllocBytes)
        return fail(LSTK_E_INVALID, "n_tokens " + std::to_string(n_tokens) + " needs " + std::to_string(need) +
                                        " bytes of scratch, more than the fixed " + std::to_string(kNoAllocBytes));
    if (!pool->noalloc) return fail(LSTK_E_DEVICE, "the fixed scratch has no address on this device");
    CallScratch sc{};
    call_scratch_layout(pool->dims, n_tokens, pool->noalloc, &sc);
    return run_block(pool, layer, 1, d_hnorm, d_gate_inp, gate_type, nullptr, d_ids, d_weights, d_resid, d_out, n_tokens,
                     static_cast<hipStream_t>(stream), nullptr, &sc);
}

int lstk_moe_permute(lstk_pool *pool, const int32_t *d_bins, int n_tokens, int n_bins, int32_t *d_counts,
                     int32_t *d_offsets, int32_t *d_perm, lstk_stream_t stream) {
    int rc;
    if ((rc = check_call(pool, 0, n_tokens)) != LSTK_OK) return rc;
    if (n_bins < 1 || n_bins > lstk::kGroupedMaxBins)
        return fail(LSTK_E_INVALID, "n_bins must be in [1, " + std::to_string(lstk::kGroupedMaxBins) + "]");
    if (n_tokens == 0) return LSTK_OK;
    if (!d_bins || !d_counts || !d_offsets || !d_perm) return fail(LSTK_E_INVALID, "null argument");
    lstk::PermuteParams pp{d_bins, n_tokens * pool->dims.n_expert_used, n_bins, lstk::kGroupedChunk, d_counts, d_offsets,
                           d_perm, nullptr, nullptr, pool->err};
    const hipError_t e =
        timed(pool, 0, [&](const lstk::LaunchTiming *tm) { return lstk::launch_permute(pp, static_cast<hipStream_t>(stream), tm); });
    return e == hipSuccess ? LSTK_OK : hip_fail(e, "permute launch");
}

int lstk_pool_check(lstk_pool *pool, lstk_stream_t stream) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    if (pool->dry) return LSTK_OK;
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    int32_t flag = 0;
    if ((e = hipMemcpy(&flag, pool->err, sizeof(flag), hipMemcpyDeviceToHost)) != hipSuccess) return hip_fail(e, "read error flag");
    if (flag) {
        const int32_t zero = 0;
        if ((e = hipMemcpy(pool->err, &zero, sizeof(zero), hipMemcpyHostToDevice)) != hipSuccess) return hip_fail(e, "clear error flag");
        std::string msg = "a kernel saw";
        if (flag & 1) msg += " an expert/slot id out of range (clamped)";
        if (flag & 2) msg += std::string(flag & 1 ? " and" : "") + " an expert repeated within one token";
        if (flag & 4) msg += std::string(flag & 3 ? " and" : "") + " a fused stage that timed out waiting for another work-group";
        if (flag & 8) msg += std::string(flag & 7 ? " and" : "") + " a device-side acquire with no free slot";
        return fail(LSTK_E_BADID, msg);
    }
    return LSTK_OK;
}

int lstk_pool_set_timing(lstk_pool *pool, int enable) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    pool->timing = enable != 0;
    return LSTK_OK;
}

int lstk_pool_timing(lstk_pool *pool, double ms[4], int64_t launches[4]) {
    if (!pool || !ms || !launches) return fail(LSTK_E_INVALID, "null argument");
    for (int s = 0; s < kStages; s++) {
        for (TimedLaunch &t : pool->launched[s]) {
            hipError_t e = hipEventSynchronize(t.end);
            if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
            float v = 0.0f;
            if ((e = hipEventElapsedTime(&v, t.start, t.end)) != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
            pool->ms[s] += v;
            pool->launches[s]++;
            (void) hipEventDestroy(t.start);
            (void) hipEventDestroy(t.end);
        }
        pool->launched[s].clear();
        ms[s] = pool->ms[s];
        launches[s] = pool->launches[s];
        pool->ms[s] = 0.0;
        pool->launches[s] = 0;
    }
    return LSTK_OK;
}

size_t lstk_matrix_bytes(int type, int rows, int cols) {
    if (!lstk::supported_weight_type(type) || rows <= 0 || cols <= 0 || cols % lstk::kSuper) return 0;
    return lstk::matrix_bytes(type, rows, cols);
}

int lstk_repack_matrix(int type, int rows, int cols, const void *gguf, void *packed) {
    if (!gguf || !packed) return fail(LSTK_E_INVALID, "null argument");
    const int rc = lstk::repack_matrix(type, rows, cols, gguf, packed);
    return rc == LSTK_OK ? rc : fail(rc, "unsupported type or shape");
}

int lstk_unpack_matrix(int type, int rows, int cols, const void *packed, void *gguf) {
    if (!gguf || !packed) return fail(LSTK_E_INVALID, "null argument");
    const int rc = lstk::unpack_matrix(type, rows, cols, packed, gguf);
    return rc == LSTK_OK ? rc : fail(rc, "unsupported type or shape");
}

// Test hook: makes the next n host-tier copies fail, to exercise the LSTK_E_IO path.
int lstk_pool_debug_fail_copies(lstk_pool *pool, int n) {
    if (!pool) return fail(LSTK_E_INVALID, "null pool");
    if (pool->device_lru) return fail(LSTK_E_INVALID, "copy failures cannot be injected into device-side acquires");
    pool->fail_copies = n;
    return LSTK_OK;
}

}  // extern "C"
