// tier.hip - the streaming pool's slot bookkeeping and host-tier copies on the GPU.
//
// ExpertStore::acquire + release_all (src/expert_store.cpp:232-295) of one segment, with the hit
// resolution moved from the CPU to the device, so a streaming layer needs no host round trip between
// its router and its experts (the per-layer CPU sync of docs/decisions.md:14):
//   lru_resolve_kernel  one work-group: stages the shard's LRU (prev / next / owners) and the layer's
//                       expert -> slot map in LDS, then one lane runs the acquire loop in request
//                       order (hit: pin, unlinking an unpinned slot; miss: evict the LRU head, remap,
//                       record (slot, expert)), then the release loop (a slot whose pin count returns
//                       to 0 goes to the LRU tail, in acquisition order); the state is written back;
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

__global__ __launch_bounds__(256) void lru_resolve_kernel(TierResolveParams P) {
    __shared__ int32_t prv[kTierMaxSlots], nxt[kTierMaxSlots], own_l[kTierMaxSlots], own_e[kTierMaxSlots],
        pins[kTierMaxSlots];
    __shared__ int32_t slot_of[kTierMaxExperts], ex[kTierMaxIds], got[kTierMaxIds];
    const int tid = threadIdx.x, ns = P.n_slots, E = P.E, n = P.n;
    int32_t *g_prev = P.lru.prev + P.slot_base, *g_next = P.lru.next + P.slot_base;
    int32_t *g_ol = P.lru.owner_layer + P.slot_base, *g_oe = P.lru.owner_expert + P.slot_base;
    int32_t *g_slot_of = P.lru.slot_of + (size_t) P.layer * E;
    for (int i = tid; i < ns; i += blockDim.x) {
        prv[i] = g_prev[i];
        nxt[i] = g_next[i];
        own_l[i] = g_ol[i];
        own_e[i] = g_oe[i];
        pins[i] = 0;
    }
    for (int i = tid; i < E; i += blockDim.x) slot_of[i] = g_slot_of[i];
    int bad = 0;
    for (int i = tid; i < n; i += blockDim.x) {
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
        int32_t *hdr = P.lru.hdr + 4 * P.shard;
        int head = hdr[0], tail = hdr[1], n_in = hdr[2];
        int hits = 0, misses = 0;
        auto unlink = [&](int s) {
            const int a = prv[s], b = nxt[s];
            if (a >= 0) nxt[a] = b;
            else head = b;
            if (b >= 0) prv[b] = a;
            else tail = a;
            prv[s] = nxt[s] = -1;
            n_in--;
        };
        auto push_tail = [&](int s) {
            prv[s] = tail;
            nxt[s] = -1;
            if (tail >= 0) nxt[tail] = s;
            tail = s;
            if (head < 0) head = s;
            n_in++;
        };
        for (int i = 0; i < n; i++) {
            const int e = ex[i];
            int s = slot_of[e];
            if (s >= 0) {
                if (pins[s] == 0) unlink(s);
                pins[s]++;
                got[i] = s;
                hits++;
                continue;
            }
            s = head;
            if (s < 0) {
                // cannot happen: the host only launches calls of at most n_slots experts, and at
                // most i slots are pinned here; flagged, and the request is served from slot 0 so
                // nothing leaves the pool
                atomicOr(P.err, 8);
                got[i] = -1;
                continue;
            }
            unlink(s);
            const int l0 = own_l[s], e0 = own_e[s];
            if (l0 == P.layer) slot_of[e0] = -1;
            else if (l0 >= 0) P.lru.slot_of[(size_t) l0 * E + e0] = -1;
            own_l[s] = P.layer;
            own_e[s] = e;
            slot_of[e] = s;
            pins[s] = 1;
            got[i] = s;
            P.miss[2 * misses] = s;
            P.miss[2 * misses + 1] = e;
            misses++;
        }
        for (int i = 0; i < n; i++) {
            const int s = got[i];
            if (s >= 0 && --pins[s] == 0) push_tail(s);
        }
        hdr[0] = head;
        hdr[1] = tail;
        hdr[2] = n_in;
        *P.n_miss = misses;
        P.lru.stats[0] += (unsigned long long) hits;
        P.lru.stats[1] += (unsigned long long) misses;
        P.lru.stats[2] += (unsigned long long) misses * P.slab;
        P.lru.stats[3] += 1ull;
    }
    __syncthreads();
    for (int i = tid; i < ns; i += blockDim.x) {
        g_prev[i] = prv[i];
        g_next[i] = nxt[i];
        g_ol[i] = own_l[i];
        g_oe[i] = own_e[i];
    }
    for (int i = tid; i < E; i += blockDim.x) g_slot_of[i] = slot_of[i];
    for (int i = tid; i < n; i += blockDim.x) P.slots[i] = got[i] < 0 ? 0 : got[i];
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
    return launch(lru_resolve_kernel, dim3(1), dim3(256), 0, st, tm, P);
}

hipError_t launch_tier_copy(const TierCopyParams &P, hipStream_t st, const LaunchTiming *tm) {
    const long per = (long) P.chunks[0] + P.chunks[1] + P.chunks[2];
    const long total = per * P.max_miss;
    if (total <= 0) return hipSuccess;
    const int grid = (int) (total < kTierCopyGrid ? total : kTierCopyGrid);
    return launch(tier_copy_kernel, dim3(grid), dim3(kCopyThreads), 0, st, tm, P);
}

}  // namespace lstk
