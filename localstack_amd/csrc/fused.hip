// fused.hip - the MoE block of a single token (decode at batch 1) in one launch on gfx950.
//
// An opt-in alternative to the three-launch single-token path (route, gate_up, down_combine). Each kernel
// boundary there costs about 1.1-1.3 us inside a replayed graph, plus 0.4-1 us for the first read of the
// previous kernel's output. Here router, gate/up + SwiGLU, down + router weight, k-way combine and residual
// (src/qwen3.cpp:175-214, :250) run as one grid whose stages hand over inside the kernel. Measured on
// MI355X it is slower: the 48-layer Qwen3-30B-A3B Q8_0 stack at T = 1 runs at 705 tok/s against 1181 tok/s
// for the three launches (two A/B pairs, one box), because each hand-over waits for device-coherent stores
// to complete and for flag polls across the XCDs' L2s. The stages:
//   stage A  work-groups [0, nA): one router logit per wavefront, stored device-coherent, then flag_a.
//   stage B  work-groups [0, nB): wait for flag_a, top-k in the work-group, then one gate/up unit
//            (pair j, block of RW rows of gate and up) exactly as the multi-kernel gate_up kernel
//            computes it; SwiGLU rows stored device-coherent, then flag_b.
//   stage C  work-groups [nB, nB + nC): wait for flag_a, top-k, issue the down weight loads of their
//            rd rows for all k pairs, wait for flag_b, quantize the SwiGLU rows, dot products, router
//            weights, combine in slot order, residual, plain store of out.
// Hand-over protocol (no L2 write-back, no atomics on shared counters): data and flags use
// agent-scope relaxed atomic loads / stores (sc1, coherent across the XCDs' L2s); a producer waits
// for its stores to complete (s_waitcnt vmcnt(0)) before a barrier and its flag store. Each flag
// holds the launch number n of the work-group that wrote it: every work-group keeps its own launch
// count in cnt[w] (all work-groups of a pool run in every launch, so the counts agree), so flags of
// an earlier launch (n - 1) never satisfy a wait. Waits are bounded (spin_max polls); a wait that
// runs out sets bit 4 of the error flag and the work-group carries on, so the grid always drains.
// All work-groups must be resident at once (fused_fits checks the occupancy at pool creation).
//
// The arithmetic is that of kernels.hip at T = 1 (same quantizers, same dot products, same
// reduction orders), so the fused result equals the multi-kernel result bit for bit.
#include "device.h"
#include "formats.h"
#include "kernels.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace lstk {
namespace {

constexpr int kFusedMaxFlags = 1024;

__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wavefront 0 polls flags[0, count) until all hold n (or spin_max polls pass); the work-group waits.
__device__ __forceinline__ void wait_flags(const int *flags, int count, int n, int spin_max, int32_t *err) {
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        bool ok = false;
        for (int it = 0; it < spin_max; it++) {
            // all of this lane's flags in flight together (count <= kFusedMaxFlags)
            int v[kFusedMaxFlags / kWave];
#pragma unroll
            for (int u = 0; u < kFusedMaxFlags / kWave; u++) {
                const int i = lane + u * kWave;
                v[u] = i < count ? ld_dev(flags + i) : n;
            }
            bool mine = true;
#pragma unroll
            for (int u = 0; u < kFusedMaxFlags / kWave; u++) mine = mine && v[u] == n;
            if (__all(mine)) {
                ok = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok && lane == 0) atomicOr(err, 4);
    }
    __syncthreads();
}

// Publishes this work-group's flag once every thread's device-coherent stores have completed.
__device__ __forceinline__ void publish(int *flag, int n) {
    stores_done();
    __syncthreads();
    if (threadIdx.x == 0) st_dev(flag, n);
}

constexpr int kFusedMaxK = 16;
constexpr int kFusedMaxAct = 8192; // k * f values quantized by a down work-group
constexpr size_t kTopkLds4 = 4 * 256 * 4 + 4 * kMaxEPL * kWave * 4 + 4 * kMaxK * 4;

struct FLds {
    unsigned char topk[kTopkLds4];
    float logits[kWave * kMaxEPL];
    int ids[kFusedMaxK];
    float w[kFusedMaxK];
    int n;
    __align__(16) union {
        struct {
            int8_t xs[4096];
            float xd[128];
            int xb[128];
            float red[2 * 128];
        } b;
        struct {
            int8_t qs[kFusedMaxAct];
            float qd[kFusedMaxAct / 32];
            int qb[kFusedMaxAct / 32];
            float part[256];
        } c;
    } u;
};

// Router logit of expert e for the token, the order of route_tile: lane l accumulates elements
// 256 g + 4 l + q (g, then q ascending) with fmaf from 0, then wave_sum_tree.
template <int GT, int NG>
__device__ __forceinline__ float router_logit(const FusedParams &P, int e) {
    const int lane = threadIdx.x % kWave;
    constexpr int h = NG * 256;
    float w[NG][4];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const size_t i = (size_t) e * h + 256 * g + 4 * lane;
        if (GT == kTypeF16) {
            const uint2 raw = *reinterpret_cast<const uint2 *>(static_cast<const unsigned short *>(P.gate_inp) + i);
            w[g][0] = h2f(raw.x);
            w[g][1] = h2f(raw.x >> 16);
            w[g][2] = h2f(raw.y);
            w[g][3] = h2f(raw.y >> 16);
        } else {
            const float4 raw = *reinterpret_cast<const float4 *>(static_cast<const float *>(P.gate_inp) + i);
            w[g][0] = raw.x;
            w[g][1] = raw.y;
            w[g][2] = raw.z;
            w[g][3] = raw.w;
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; g++) {
        float4 x = *reinterpret_cast<const float4 *>(P.hnorm + 256 * g + 4 * lane);
        if (GT == kTypeF16) {
            x.x = round_f16(x.x);
            x.y = round_f16(x.y);
            x.z = round_f16(x.z);
            x.w = round_f16(x.w);
        }
        acc = fmaf(x.x, w[g][0], acc);
        acc = fmaf(x.y, w[g][1], acc);
        acc = fmaf(x.z, w[g][2], acc);
        acc = fmaf(x.w, w[g][3], acc);
    }
    return wave_sum_tree(acc);
}

// The token's k experts and weights into LDS (route: from the published logits, ranked by all
// wavefronts; work-group 0 also stores them for the caller).
template <int EPL>
__device__ __forceinline__ void routing(const FusedParams &P, FLds &L) {
    const int wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    for (int e = threadIdx.x; e < P.E; e += blockDim.x) L.logits[e] = ld_dev(P.logits + e);
    __syncthreads();
    float *s_l = reinterpret_cast<float *>(L.topk);
    int *s_rank = reinterpret_cast<int *>(L.topk + (size_t) nw * 256 * 4);
    float *s_p = reinterpret_cast<float *>(s_rank + (size_t) nw * kMaxEPL * kWave);
    float l[EPL];
    bool valid[EPL];
    int rank[EPL];
    if (rank_token<EPL>(L.logits, P.E, P.k, wave, nw, s_l, s_rank, l, valid, rank)) {
        const bool first = blockIdx.x == 0;
        weights_token<EPL>(P.k, l, valid, rank, s_p, nullptr, L.ids, L.w, first ? P.ids_out : nullptr,
                           first ? P.weights_out : nullptr);
    }
    __syncthreads();
}

template <int GT, int NG, int WTG, int WTD, int S>
__global__ __launch_bounds__(kBlock) void fused_kernel(FusedParams P) {
    __shared__ FLds L;
    const int w = blockIdx.x, tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int k = P.k, h = P.h, f = P.f;
    if (tid == 0) L.n = ld_dev(P.cnt + w) + 1;
    __syncthreads();
    const int n = L.n;
    constexpr int QG = WTG == kTypeQ4_K ? kTypeQ4_K : kTypeQ8_0;
    // the token's activations for gate/up do not depend on the routing: quantize them first
    if (w < P.nB) quantize_row<QG>(P.hnorm, h, L.u.b.xs, L.u.b.xd, L.u.b.xb);
    // ---- stage A: router logits
    if (P.route) {
        if (w < P.nA) {
            const int e = w * (kBlock / kWave) + wave;
            if (e < P.E) {
                const float v = router_logit<GT, NG>(P, e);
                if (lane == 0) st_dev(P.logits + e, v);
            }
            publish(P.flag_a + w, n);
        }
        wait_flags(P.flag_a, P.nA, n, P.spin_max, P.err);
        const int epl = (P.E + kWave - 1) / kWave;
        if (epl == 1) routing<1>(P, L);
        else if (epl == 2) routing<2>(P, L);
        else routing<4>(P, L);
    } else {
        if (tid < k) {
            int b = P.ids_in[tid];
            if (b < 0 || b >= P.n_bins) {
                if (w == 0) atomicOr(P.err, 1);
                b = min(max(b, 0), P.n_bins - 1);
            }
            L.ids[tid] = b;
            L.w[tid] = P.weights_in[tid];
        }
        __syncthreads();
    }
    if (w < P.nB) {
        // ---- stage B: one gate/up unit, the thread layout of gate_up_kernel
        constexpr int CG = chunks_of(WTG);
        const int G = h / 256 / S, RW = 128 / G;
        const int r = tid % RW, m = (tid / RW) & 1, g = tid / (2 * RW);
        const int j = w / P.ub, rb = w % P.ub;
        const int e = L.ids[j];
        const int row = rb * RW + r;
        const uint8_t *base = m ? P.w_up + (size_t) e * P.s_up : P.w_gate + (size_t) e * P.s_gate;
        uint4 wv[S][CG];
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int sb = g + s * G;
#pragma unroll
            for (int c = 0; c < CG; c++) wv[s][c] = *reinterpret_cast<const uint4 *>(base + chunk_offset(CG, f, h / 256, sb, c, row));
        }
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int sb = g + s * G;
            acc = dot_sb<WTG>(wv[s], L.u.b.xs + sb * 256, L.u.b.xd + sb * 8, L.u.b.xb + sb * 8, acc);
        }
        L.u.b.red[(g * 2 + m) * RW + r] = acc;
        __syncthreads();
        if (tid < RW) {
            float gs = L.u.b.red[tid], us = L.u.b.red[RW + tid];
            for (int gg = 1; gg < G; gg++) {
                gs += L.u.b.red[(gg * 2 + 0) * RW + tid];
                us += L.u.b.red[(gg * 2 + 1) * RW + tid];
            }
            st_dev(P.act + (size_t) j * f + rb * RW + tid, (gs / (1.0f + expf(-gs))) * us);
        }
        publish(P.flag_b + w, n);
    } else {
        // ---- stage C: rd rows of down for all k pairs, router weights, combine, residual
        constexpr int CD = chunks_of(WTD);
        constexpr int QD = WTD == kTypeQ4_K ? kTypeQ4_K : kTypeQ8_0;
        const int nsbf = f / 256, rd = P.rd;
        const int c = w - P.nB;
        const int q = tid / nsbf, sb = tid % nsbf;
        const bool on = q < rd * k;
        const int jj = on ? q / rd : 0, rr = q % rd;
        const int row = c * rd + rr;
        uint4 wv[CD];
        {
            const uint8_t *base = P.w_down + (size_t) L.ids[jj] * P.s_down;
#pragma unroll
            for (int cc = 0; cc < CD; cc++)
                wv[cc] = *reinterpret_cast<const uint4 *>(base + chunk_offset(CD, h, f / 256, on ? sb : 0, cc, on ? row : c * rd));
        }
        wait_flags(P.flag_b, P.nB, n, P.spin_max, P.err);
        quantize_row_dev<QD, kFusedMaxAct / (8 * kBlock)>(P.act, k * f, L.u.c.qs, L.u.c.qd, L.u.c.qb);
        __syncthreads();
        if (on) {
            const int o = jj * f + sb * 256;
            L.u.c.part[q * nsbf + sb] = dot_sb<WTD>(wv, L.u.c.qs + o, L.u.c.qd + o / 32, L.u.c.qb + o / 32, 0.0f);
        }
        __syncthreads();
        if (tid < rd) {
            float acc = 0.0f;
            for (int j = 0; j < k; j++) {
                const float *pp = L.u.c.part + (j * rd + tid) * nsbf;
                float ds = pp[0];
                for (int s2 = 1; s2 < nsbf; s2++) ds += pp[s2];
                const float y = ds * L.w[j];
                acc = j == 0 ? y : acc + y;
            }
            const int orow = c * rd + tid;
            P.out[orow] = acc + P.resid[orow];
        }
    }
    __syncthreads();
    if (tid == 0) st_dev(P.cnt + w, n);
}

template <int GT, int NG, int WTG, int WTD, int S>
void *fused_fn() {
    return reinterpret_cast<void *>(&fused_kernel<GT, NG, WTG, WTD, S>);
}

// The instantiation for (router type, h / 256, gate/up type, down type, S); null if none.
template <int GT, int NG>
void *pick_types(int tg, int td, int S) {
    if (tg == kTypeQ8_0 && td == kTypeQ8_0) return S == 1 ? fused_fn<GT, NG, kTypeQ8_0, kTypeQ8_0, 1>() : fused_fn<GT, NG, kTypeQ8_0, kTypeQ8_0, 2>();
    if (tg == kTypeQ4_K && td == kTypeQ4_K) return S == 1 ? fused_fn<GT, NG, kTypeQ4_K, kTypeQ4_K, 1>() : fused_fn<GT, NG, kTypeQ4_K, kTypeQ4_K, 2>();
    if (tg == kTypeQ4_K && td == kTypeQ8_0) return S == 1 ? fused_fn<GT, NG, kTypeQ4_K, kTypeQ8_0, 1>() : fused_fn<GT, NG, kTypeQ4_K, kTypeQ8_0, 2>();
    if (tg == kTypeQ8_0 && td == kTypeQ4_K) return S == 1 ? fused_fn<GT, NG, kTypeQ8_0, kTypeQ4_K, 1>() : fused_fn<GT, NG, kTypeQ8_0, kTypeQ4_K, 2>();
    return nullptr;
}

template <int GT>
void *pick_ng(int h, int tg, int td, int S) {
    switch (h / 256) {
        case 1: return pick_types<GT, 1>(tg, td, S);
        case 2: return pick_types<GT, 2>(tg, td, S);
        case 4: return pick_types<GT, 4>(tg, td, S);
        case 8: return pick_types<GT, 8>(tg, td, S);
        case 16: return pick_types<GT, 16>(tg, td, S);
        default: return nullptr;
    }
}

void *fused_kernel_for(int gate_type, int tg, int td, int h) {
    int S, G;
    if (!pick_split_gate_up(h / 256, &S, &G)) return nullptr;
    return gate_type == kTypeF16 ? pick_ng<kTypeF16>(h, tg, td, S) : pick_ng<kTypeF32>(h, tg, td, S);
}

}  // namespace

FusedLayout fused_layout(int h, int f, int E, int k) {
    FusedLayout L;
    int S, G;
    if (k < 1 || k > kFusedMaxK || h % 256 || f % 256 || h > 4096 || (long) k * f > kFusedMaxAct || E > kWave * kMaxEPL ||
        !pick_split_gate_up(h / 256, &S, &G))
        return L;
    const int RW = 128 / G, nsbf = f / 256;
    if (f % RW) return L;
    int rd = 1;
    while (rd * 2 * k * nsbf <= kBlock && h % (rd * 2) == 0) rd *= 2;
    if (rd * k * nsbf > kBlock) return L;
    L.ub = f / RW;
    L.nB = k * L.ub;
    L.nA = (E + kBlock / kWave - 1) / (kBlock / kWave);
    L.rd = rd;
    L.nC = h / rd;
    L.ok = L.nA <= L.nB && L.nB <= kFusedMaxFlags;
    return L;
}

bool fused_fits(const FusedLayout &L, int gate_type, int tg, int td, int h, int f, int k) {
    (void) f;
    (void) k;
    if (!L.ok) return false;
    void *fn = fused_kernel_for(gate_type, tg, td, h);
    if (!fn) return false;
    static std::mutex mu;
    static std::map<std::tuple<void *, int>, int> cache; // (kernel, device) -> resident work-groups
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({fn, dev});
    if (it == cache.end()) {
        int per_cu = 0, n_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(fn), kBlock, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return false;
        it = cache.emplace(std::make_tuple(fn, dev), per_cu * n_cu).first;
    }
    return L.nB + L.nC <= it->second;
}

hipError_t launch_fused(const FusedParams &P, int gate_type, int tg, int td, hipStream_t st, const LaunchTiming *tm) {
    void *fn = fused_kernel_for(P.route ? gate_type : kTypeF16, tg, td, P.h);
    if (!fn) return hipErrorInvalidValue;
    FusedParams p = P;
    void *args[] = {&p};
    const dim3 grid(P.nB + P.nC), block(kBlock);
    if (tm && tm->start) return hipExtLaunchKernel(fn, grid, block, args, 0, st, tm->start, tm->stop, 0);
    return hipLaunchKernel(fn, grid, block, args, 0, st);
}

}  // namespace lstk
