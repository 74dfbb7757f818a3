// tier.hip - the streaming pool's slot bookkeeping and host-tier copies on the GPU.
//
// ExpertStore::acquire + release_all (src/expert_store.cpp:232-295) of one segment, with the hit
// resolution moved from the CPU to the device, so a streaming layer needs no host round trip between
// its router and its experts (the per-layer CPU sync of docs/decisions.md:14):
//   lru_resolve_kernel  one work-group. The shard's slots are kept as an array in eviction order (the
//                       least recently released first). A call's n requests are resolved in request
//                       order by one lane against LDS copies: a resident expert is a hit (its slot is
//                       marked used); otherwise the first unmarked entry of the order is taken, its
//                       previous expert unmapped, and (slot, expert) recorded as a miss. Everything
//                       else is done by the whole work-group in parallel: staging (the order, the
//                       owners and the layer's expert -> slot map, in one round) and the new order - the unmarked
//                       entries in their order, then the call's slots by their last request (the order
//                       in which release_all returns them), placed by two work-group prefix sums;
//   tier_copy_kernel    copies the three matrices of every miss from the pinned host tier into the
//                       miss's slot with 16-byte loads over PCIe, the misses' chunks spread over the
//                       grid.
// Both run on the caller's stream, so the experts of the layer (queued after them) see the copies,
// and the next layer's resolve runs after this layer's experts have finished with their slots.
#include "device.h"

namespace lstk {
namespace {

#ifndef LSTK_TIER_COPY_VEC
#define LSTK_TIER_COPY_VEC 4
#endif
constexpr int kCopyThreads = 256;
constexpr int kCopyVec = LSTK_TIER_COPY_VEC;                // 16-byte vectors per thread per chunk
constexpr int kCopyChunk = kCopyThreads * kCopyVec * 16;    // 16 KiB at 4 vectors

constexpr int kResolveThreads = 256;

// Exclusive prefix sum over the work-group of one value per thread; *total gets the sum.
__device__ __forceinline__ int block_excl_scan(int v, int *s_w, int *total) {
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    int x = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
    }
    if (lane == kWave - 1) s_w[w] = x;
    __syncthreads();
    int before = 0, sum = 0;
#pragma unroll
    for (int i = 0; i < kResolveThreads / kWave; i++) {
        before += i < w ? s_w[i] : 0;
        sum += s_w[i];
    }
    __syncthreads();
    *total = sum;
    return before + x - v;
}

__global__ __launch_bounds__(kResolveThreads) void lru_resolve_kernel(TierResolveParams P) {
    __shared__ int32_t order[kTierMaxSlots], last[kTierMaxSlots], slot_of[kTierMaxExperts];
    __shared__ int32_t own_l[kTierMaxSlots], own_e[kTierMaxSlots];
    __shared__ int32_t ex[kTierMaxIds], got[kTierMaxIds];
    __shared__ uint8_t used[kTierMaxSlots];
    __shared__ int s_w[kResolveThreads / kWave];
    const int tid = threadIdx.x, ns = P.n_slots, E = P.E, n = P.n;
    const int reach = min(ns, 2 * n); // entries a miss can reach: each request passes at most two
    // the counters, read before anything waits (lane 0 adds this call's figures at the end)
    unsigned long long st0 = 0, st1 = 0, st2 = 0, st3 = 0;
    if (tid == 0) {
        st0 = P.lru.stats[0];
        st1 = P.lru.stats[1];
        st2 = P.lru.stats[2];
        st3 = P.lru.stats[3];
    }
    int32_t *g_order = P.lru.order + P.slot_base;
    int32_t *g_ol = P.lru.owner_layer + P.slot_base, *g_oe = P.lru.owner_expert + P.slot_base;
    int32_t *g_slot_of = P.lru.slot_of + (size_t) P.layer * E;
    for (int i = tid; i < ns; i += kResolveThreads) {
        order[i] = g_order[i];
        own_l[i] = g_ol[i];
        own_e[i] = g_oe[i];
        last[i] = -1;
        used[i] = 0;
    }
    for (int i = tid; i < E; i += kResolveThreads) slot_of[i] = g_slot_of[i];
    int bad = 0;
    for (int i = tid; i < n; i += kResolveThreads) {
        int e = P.experts[i];
        if (e < 0 || e >= E) {
            e = e < 0 ? 0 : E - 1;
            bad = 1;
        }
        ex[i] = e;
    }
    if (bad) atomicOr(P.err, 1);
    __syncthreads();
    if (tid == 0) {
        int p = 0, hits = 0, misses = 0;
        for (int i = 0; i < n; i++) {
            const int e = ex[i];
            int s = slot_of[e];
            if (s >= 0) {
                used[s] = 1;
                got[i] = s;
                hits++;
                continue;
            }
            while (p < reach && used[order[p]]) p++;
            if (p == reach) {
                // cannot happen: the host launches at most n_slots requests, and each passes at most
                // two entries; flagged, and the request is served from slot 0 so nothing leaves the pool
                atomicOr(P.err, 8);
                got[i] = -1;
                continue;
            }
            s = order[p++];
            const int l0 = own_l[s], e0 = own_e[s];
            if (l0 == P.layer) slot_of[e0] = -1;
            else if (l0 >= 0) P.lru.slot_of[(size_t) l0 * E + e0] = -1;
            g_ol[s] = P.layer;
            g_oe[s] = e;
            slot_of[e] = s;
            used[s] = 1;
            got[i] = s;
            P.miss[2 * misses] = s;
            P.miss[2 * misses + 1] = e;
            misses++;
        }
        *P.n_miss = misses;
        P.lru.stats[0] = st0 + (unsigned long long) hits;
        P.lru.stats[1] = st1 + (unsigned long long) misses;
        P.lru.stats[2] = st2 + (unsigned long long) misses * P.slab;
        P.lru.stats[3] = st3 + 1ull;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kResolveThreads)
        if (got[i] >= 0) atomicMax(&last[got[i]], i);
    __syncthreads();
    // new order: unmarked entries in order, then the used slots by their last request. Thread t owns
    // the consecutive entries [t c, (t + 1) c) of each list.
    const int ce = (ns + kResolveThreads - 1) / kResolveThreads, ci = (n + kResolveThreads - 1) / kResolveThreads;
    int keep = 0, rel = 0;
    for (int j = tid * ce; j < min(ns, (tid + 1) * ce); j++) keep += used[order[j]] ? 0 : 1;
    for (int i = tid * ci; i < min(n, (tid + 1) * ci); i++) rel += (got[i] >= 0 && last[got[i]] == i) ? 1 : 0;
    int n_keep, n_rel;
    int at = block_excl_scan(keep, s_w, &n_keep);
    int at_rel = n_keep + block_excl_scan(rel, s_w, &n_rel);
    for (int j = tid * ce; j < min(ns, (tid + 1) * ce); j++)
        if (!used[order[j]]) g_order[at++] = order[j];
    for (int i = tid * ci; i < min(n, (tid + 1) * ci); i++)
        if (got[i] >= 0 && last[got[i]] == i) g_order[at_rel++] = got[i];
    if (tid == 0 && n_keep + n_rel != ns) atomicOr(P.err, 8);
    for (int i = tid; i < E; i += kResolveThreads) g_slot_of[i] = slot_of[i];
    for (int i = tid; i < n; i += kResolveThreads) P.slots[i] = got[i] < 0 ? 0 : got[i];
}

__global__ __launch_bounds__(kCopyThreads) void tier_copy_kernel(TierCopyParams P) {
    int n = *P.n_miss;
    n = n < 0 ? 0 : (n > P.max_miss ? P.max_miss : n);
    const int c0 = P.chunks[0], c1 = P.chunks[1], cpm = c0 + c1 + P.chunks[2];
    const int total = n * cpm;
    for (int c = blockIdx.x; c < total; c += gridDim.x) {
        const int mi = c / cpm;
        int r = c - mi * cpm, m = 0;
        if (r >= c0) {
            r -= c0;
            m = 1;
            if (r >= c1) {
                r -= c1;
                m = 2;
            }
        }
        int slot = P.miss[2 * mi], e = P.miss[2 * mi + 1];
        slot = slot < 0 ? 0 : (slot >= P.n_slots ? P.n_slots - 1 : slot);
        e = e < 0 ? 0 : (e >= P.E ? P.E - 1 : e);
        const size_t nv = P.bytes[m] / 16;
        const uint4 *src = reinterpret_cast<const uint4 *>(P.src[m] + (size_t) e * P.bytes[m]);
        uint4 *dst = reinterpret_cast<uint4 *>(P.dst[m] + (size_t) slot * P.bytes[m]);
        const size_t v0 = (size_t) r * (kCopyChunk / 16) + threadIdx.x;
        uint4 t[kCopyVec];
#pragma unroll
        for (int j = 0; j < kCopyVec; j++) {
            const size_t v = v0 + (size_t) j * kCopyThreads;
            if (v < nv) t[j] = src[v];
        }
#pragma unroll
        for (int j = 0; j < kCopyVec; j++) {
            const size_t v = v0 + (size_t) j * kCopyThreads;
            if (v < nv) dst[v] = t[j];
        }
    }
}

}  // namespace

int tier_copy_chunks(size_t bytes) { return (int) ((bytes + kCopyChunk - 1) / kCopyChunk); }

hipError_t launch_tier_resolve(const TierResolveParams &P, hipStream_t st, const LaunchTiming *tm) {
    return launch(lru_resolve_kernel, dim3(1), dim3(kResolveThreads), 0, st, tm, P);
}

hipError_t launch_tier_copy(const TierCopyParams &P, hipStream_t st, const LaunchTiming *tm) {
    const long per = (long) P.chunks[0] + P.chunks[1] + P.chunks[2];
    const long total = per * P.max_miss;
    if (total <= 0) return hipSuccess;
    const int grid = (int) (total < kTierCopyGrid ? total : kTierCopyGrid);
    return launch(tier_copy_kernel, dim3(grid), dim3(kCopyThreads), 0, st, tm, P);
}

}  // namespace lstk
