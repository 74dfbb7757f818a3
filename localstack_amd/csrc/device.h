// device.h - device helpers shared by the gfx950 kernels (kernels.hip, grouped.hip): fp16
// conversion, wavefront reductions over DPP, the Q8_0 / Q8_K activation quantizer and the Q4_K
// 6-bit scale / min unpacking.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "formats.h"
#include "kernels.h"

namespace lstk {

#ifndef LSTK_NT_WEIGHTS
#define LSTK_NT_WEIGHTS 1
#endif
// Weights read once per call (the experts of one token, the dense matrices of one decode step) carry the
// non-temporal hint, so they do not displace what the next launches read again (router rows,
// activations, the KV cache) from the last-level cache. LSTK_NT_WEIGHTS=0 turns the hint off.
__device__ __forceinline__ uint4 load_weights(const uint4 *p) {
#if LSTK_NT_WEIGHTS
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *p;
#endif
}
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kMaxEPL = 4;        // n_expert <= 256: 4 logits per lane in the top-k
constexpr int kMaxK = 64;         // n_expert_used <= 64 (one lane per selected expert)
constexpr int kMaxG = 8;          // K-groups per work-group

// Device-coherent (agent scope, coherent across the XCDs' L2 caches) relaxed loads and stores, for
// values handed between work-groups of one launch.
__device__ __forceinline__ int ld_dev(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float h2f(unsigned h) { return __half2float(__ushort_as_half((unsigned short) (h & 0xffffu))); }
__device__ __forceinline__ float round_f16(float x) { return __half2float(__float2half_rn(x)); }

// ------------------------------------------------------------------------------------------------
// wavefront reductions without LDS: DPP within 16-lane rows, then DPP row broadcasts across rows
// ------------------------------------------------------------------------------------------------

// DPP move of v by control CTRL into the rows set in ROWS (the other rows get 0)
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int) (u & 0xffffffffu), CTRL, ROWS, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int) (u >> 32), CTRL, ROWS, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long) (unsigned) hi << 32) | (unsigned) lo);
}
constexpr int kDppRowBcast15 = 0x142; // each row receives lane 15 of the row before it
constexpr int kDppRowBcast31 = 0x143; // rows 2 and 3 receive lane 31
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned) __builtin_amdgcn_readlane((int) (u & 0xffffffffu), l);
    const unsigned hi = (unsigned) __builtin_amdgcn_readlane((int) (u >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long) hi << 32) | lo);
}

// Sum over the 64 lanes as a pairwise tree: lanes l and l^1, then quads, octets, halves of rows,
// rows (0+1, 2+3) and the two row pairs, i.e. (r0 + r1) + (r2 + r3) of the four row sums. IEEE addition
// is commutative, so every lane of a level holds the same partial; the oracle evaluates the same tree.
// The rows meet by broadcasts: row 1 adds row 0 and row 3 adds row 2 (row_bcast:15), then row 3 adds
// row 1 (row_bcast:31), so lane 63 holds (r3 + r2) + (r1 + r0), the same value. Result uniform.
__device__ __forceinline__ float wave_sum_tree(float v) {
    v = v + dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v = v + dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v = v + dpp_f<0x141>(v);  // row_half_mirror: the other quad of the octet
    v = v + dpp_f<0x140>(v);  // row_mirror: the other octet of the row
    v = v + dpp_f<kDppRowBcast15, 0xA>(v);
    v = v + dpp_f<kDppRowBcast31, 0x8>(v);
    return readlane_f(v, 63);
}

__device__ __forceinline__ double wave_sum_d(double v) {
    v = v + dpp_d<0xB1>(v);
    v = v + dpp_d<0x4E>(v);
    v = v + dpp_d<0x141>(v);
    v = v + dpp_d<0x140>(v);
    v = v + dpp_d<kDppRowBcast15, 0xA>(v);
    v = v + dpp_d<kDppRowBcast31, 0x8>(v);
    return readlane_d(v, 63);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, dpp_f<kDppRowBcast15, 0xA>(v));
    v = fmaxf(v, dpp_f<kDppRowBcast31, 0x8>(v));
    return readlane_f(v, 63);
}

// ------------------------------------------------------------------------------------------------
// activation quantization (ggml's quantize_row_q8_0 x86 path / quantize_row_q8_K_ref)
// ------------------------------------------------------------------------------------------------

// Quantizes x[0..n) (n % 256 == 0) with all threads of the block, 8 values per thread per pass.
// Q8_0 (QT 8): d = amax/127 stored as fp16, q = rne(x * 127/amax), groups of 4 threads per block.
// Q8_K (QT 12): max = the signed value of the first largest |x| of the 256, iscale = -127/max,
// q = min(127, rne(iscale x)), d = 1/iscale; groups of 32 threads; bs = sums of 32-value groups.
// Every thread runs the shuffles; threads past the end contribute zeros and write nothing.
// A group sum s (|s| <= 4096) as two fp16 values, both exact: 64 floor(s / 64) in the low half and
// s mod 64 in the high half, which add up to s. Products of either with integers below 64, and sums
// of a few dozen such products, are integers below 2^24, so f32 holds them exactly.
__device__ __forceinline__ unsigned split_sum_f16(int s) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz((float) (s & ~63), (float) (s & 63)));
}

// One pass of the quantizer: this thread's 8 values v at i0 (on = i0 < n). bh, when non-null, also
// receives the group sums as split_sum_f16.
template <int QT>
__device__ __forceinline__ void quantize8(const float (&v)[8], int i0, bool on, int8_t *qs, float *d, int32_t *bs,
                                          uint32_t *bh = nullptr) {
    int q[8];
    float dd;
    if (QT == kTypeQ8_0) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
        amax = fmaxf(amax, dpp_f<0xB1>(amax)); // the 4 threads of a 32-value block
        amax = fmaxf(amax, dpp_f<0x4E>(amax));
        dd = round_f16(__fdiv_rn(amax, 127.0f));
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = (int) rintf(v[j] * id);
    } else {
        // (|x|, x, index) of the first largest |x|: 32 threads per 256-value block
        float amax = 0.0f, mx = 0.0f;
        int idx = INT_MAX;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float ax = fabsf(v[j]);
            if (ax > amax) {
                amax = ax;
                mx = v[j];
                idx = i0 + j;
            }
        }
        auto take = [&](float oa, float om, int oi) {
            if (oa > amax || (oa == amax && oi < idx)) {
                amax = oa;
                mx = om;
                idx = oi;
            }
        };
        take(dpp_f<0xB1>(amax), dpp_f<0xB1>(mx), __builtin_amdgcn_update_dpp(0, idx, 0xB1, 0xF, 0xF, false));
        take(dpp_f<0x4E>(amax), dpp_f<0x4E>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x4E, 0xF, 0xF, false));
        take(dpp_f<0x141>(amax), dpp_f<0x141>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x141, 0xF, 0xF, false));
        take(dpp_f<0x140>(amax), dpp_f<0x140>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x140, 0xF, 0xF, false));
        // rows 0+1 form the block of lanes 0-31, rows 2+3 the block of lanes 32-63
        const int lane = threadIdx.x % kWave;
        const int r0 = lane < 32 ? 0 : 32;
        const float a0 = readlane_f(amax, 0), a1 = readlane_f(amax, 16), a2 = readlane_f(amax, 32), a3 = readlane_f(amax, 48);
        const float m0 = readlane_f(mx, 0), m1 = readlane_f(mx, 16), m2 = readlane_f(mx, 32), m3 = readlane_f(mx, 48);
        const int x0 = __builtin_amdgcn_readlane(idx, 0), x1 = __builtin_amdgcn_readlane(idx, 16);
        const int x2 = __builtin_amdgcn_readlane(idx, 32), x3 = __builtin_amdgcn_readlane(idx, 48);
        amax = r0 ? a2 : a0;
        mx = r0 ? m2 : m0;
        idx = r0 ? x2 : x0;
        take(r0 ? a3 : a1, r0 ? m3 : m1, r0 ? x3 : x1);
        if (amax == 0.0f) {
            dd = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) q[j] = 0;
        } else {
            const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
            for (int j = 0; j < 8; j++) q[j] = min(127, (int) rintf(iscale * v[j]));
            dd = __fdiv_rn(1.0f, iscale);
        }
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) s += q[j];
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
    if (on) {
        uint2 packed;
        packed.x = (unsigned) (q[0] & 0xff) | ((unsigned) (q[1] & 0xff) << 8) | ((unsigned) (q[2] & 0xff) << 16) |
                   ((unsigned) (q[3] & 0xff) << 24);
        packed.y = (unsigned) (q[4] & 0xff) | ((unsigned) (q[5] & 0xff) << 8) | ((unsigned) (q[6] & 0xff) << 16) |
                   ((unsigned) (q[7] & 0xff) << 24);
        *reinterpret_cast<uint2 *>(qs + i0) = packed;
        if ((threadIdx.x & 3) == 0) {
            d[i0 / 32] = dd;
            bs[i0 / 32] = s;
            if (bh) bh[i0 / 32] = split_sum_f16(s);
        }
    }
}

template <int QT>
__device__ __forceinline__ void quantize_row(const float *__restrict__ x, int n, int8_t *qs, float *d, int32_t *bs,
                                             uint32_t *bh = nullptr) {
    for (int base = 0; base < n; base += blockDim.x * 8) {
        const int i0 = base + threadIdx.x * 8;
        const bool on = i0 < n;
        float v[8];
        if (on) {
            const float4 a = *reinterpret_cast<const float4 *>(x + i0);
            const float4 b = *reinterpret_cast<const float4 *>(x + i0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
        quantize8<QT>(v, i0, on, qs, d, bs, bh);
    }
}

// quantize_row for n <= NP * 8 * blockDim.x with every load issued before the first pass is
// quantized (one memory round trip instead of one per pass), in two calls:
// quantize_row_load issues the loads into v, quantize_row_store quantizes v.
// Every load is unconditional (addresses clamped into [0, n), n >= 8), so no branch separates them
// from the caller's next loads.
template <int NP>
__device__ __forceinline__ void quantize_row_load(const float *__restrict__ x, int n, float (&v)[NP][8]) {
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = (p * blockDim.x + threadIdx.x) * 8;
        const int ia = min(i0, n - 8);
        const float4 a = *reinterpret_cast<const float4 *>(x + ia);
        const float4 b = *reinterpret_cast<const float4 *>(x + ia + 4);
        const bool in = i0 < n;
        v[p][0] = in ? a.x : 0.0f; v[p][1] = in ? a.y : 0.0f; v[p][2] = in ? a.z : 0.0f; v[p][3] = in ? a.w : 0.0f;
        v[p][4] = in ? b.x : 0.0f; v[p][5] = in ? b.y : 0.0f; v[p][6] = in ? b.z : 0.0f; v[p][7] = in ? b.w : 0.0f;
    }
}
template <int QT, int NP>
__device__ __forceinline__ void quantize_row_store(const float (&v)[NP][8], int n, int8_t *qs, float *d, int32_t *bs) {
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = (p * blockDim.x + threadIdx.x) * 8;
        if (p * (int) blockDim.x * 8 < n) quantize8<QT>(v[p], i0, i0 < n, qs, d, bs);
    }
}

// quantize_row of values another work-group stored in this launch (device-coherent loads), for
// n <= NP * 8 * blockDim.x: every load is issued before the first pass is quantized.
template <int QT, int NP>
__device__ __forceinline__ void quantize_row_dev(const float *x, int n, int8_t *qs, float *d, int32_t *bs) {
    float v[NP][8];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = (p * blockDim.x + threadIdx.x) * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) v[p][j] = i0 < n ? ld_dev(x + i0 + j) : 0.0f;
    }
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i0 = (p * blockDim.x + threadIdx.x) * 8;
        if (p * (int) blockDim.x * 8 < n) quantize8<QT>(v[p], i0, i0 < n, qs, d, bs);
    }
}

// get_scale_min_k4 on the 12 scale bytes held in three dwords.
template <int J>
__device__ __forceinline__ void scale_min_k4(unsigned s0, unsigned s1, unsigned s2, int &sc, int &m) {
    auto byte = [&](int i) -> int {
        const unsigned word = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (int) ((word >> (8 * (i & 3))) & 0xffu);
    };
    if (J < 4) {
        sc = byte(J) & 63;
        m = byte(J + 4) & 63;
    } else {
        sc = (byte(J + 4) & 0xF) | ((byte(J - 4) >> 6) << 4);
        m = (byte(J + 4) >> 4) | ((byte(J) >> 6) << 4);
    }
}

// ------------------------------------------------------------------------------------------------
// softmax / top-k / renormalisation (router(), src/qwen3.cpp:179-189)
// ------------------------------------------------------------------------------------------------

// Barrier among the wavefronts cooperating on one token: the whole block, or one wavefront (whose
// lanes already run in lock step; only its LDS traffic has to land).
__device__ __forceinline__ void group_barrier(int nsplit) {
    if (nsplit > 1) __syncthreads();
    else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Order key of a logit: monotone in the value (-0 and +0 equal), ties broken towards the lower
// expert id, unique per expert.
__device__ __forceinline__ unsigned long long order_key(float v, int e) {
    unsigned u = __float_as_uint(v);
    if (v == 0.0f) u = 0u;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long) u << 8) | (unsigned) (255 - e);
}

// One token's softmax / top-k / renormalisation, everything in parallel. The rank of an expert is
// the number of experts with a larger logit, or an equal logit and a lower id, so the selection is
// largest first with ties to the lower expert id, as the oracle's sequential argmax. Ranks are
// counted with f32 compares against the row broadcast from LDS, split over `nsplit` wavefronts
// (partial counts summed in LDS); exact ties are rare and take a second, 64-bit-key pass.
// p = expf(l - max) * (float)(1 / sum) with the sum in double; the k selected p are summed in rank
// order in double, clamped to >= 2^-14 and divided out. The expert of rank j is written to ids[j],
// its weight to weights[j].
// Called by the `nsplit` wavefronts [w0, w0 + nsplit) of the block with part = wave - w0.
// s_l: >= E floats, s_rank: >= nsplit * 64 * EPL ints, s_p: >= k floats, all LDS shared by the group.
template <int EPL>
__device__ __forceinline__ bool rank_token(const float *__restrict__ l_row, int E, int k, int part, int nsplit, float *s_l,
                                           int *s_rank, float (&l)[EPL], bool (&valid)[EPL], int (&rank)[EPL]) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + kWave * i;
        valid[i] = e < E;
        l[i] = l_row[min(e, E - 1)]; // unconditional: all loads in flight together
    }
#pragma unroll
    for (int i = 0; i < EPL; i++)
        if (!valid[i]) l[i] = -INFINITY;
    if (part == 0) {
        // the row, padded with -inf to 4 * 64 entries so the rank loop needs no remainder
#pragma unroll
        for (int i = 0; i < kMaxEPL; i++) s_l[lane + kWave * i] = i < EPL ? l[i] : -INFINITY;
    }
    group_barrier(nsplit);
    // partial ranks over this wavefront's share of the row, 32 values per batch of LDS reads
    const int per = (((E + nsplit - 1) / nsplit) + 31) & ~31;
    const int a0 = part * per, a1 = min(((E + 31) & ~31), a0 + per);
    int r[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) r[i] = 0;
    for (int e2 = a0; e2 < a1; e2 += 32) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const float4 *>(s_l + e2 + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; u++) {
#pragma unroll
            for (int i = 0; i < EPL; i++)
                r[i] += (v[u].x > l[i]) + (v[u].y > l[i]) + (v[u].z > l[i]) + (v[u].w > l[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < EPL; i++) s_rank[(part * EPL + i) * kWave + lane] = r[i];
    group_barrier(nsplit);
    if (part != 0) return false;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        rank[i] = 0;
        for (int q = 0; q < nsplit; q++) rank[i] += s_rank[(q * EPL + i) * kWave + lane];
    }
    // exact ties: an expert with an equal logit and a lower id ranks first
    bool tie = false;
#pragma unroll
    for (int i = 0; i < EPL; i++) tie |= valid[i] && rank[i] < k;
    {
        unsigned long long seen = 0ull; // bit r set once some selected expert has rank r
        // ranks are distinct exactly when there is no tie among the experts that reach rank < k
        unsigned long long mine = 0ull;
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (valid[i] && rank[i] < k) mine |= 1ull << rank[i];
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < EPL; i++) cnt += __popcll(__ballot(valid[i] && rank[i] < k));
        // OR of every lane's bits via DPP and readlane
        unsigned lo = (unsigned) mine, hi = (unsigned) (mine >> 32);
        lo |= __builtin_amdgcn_update_dpp(0, (int) lo, 0xB1, 0xF, 0xF, false);
        hi |= __builtin_amdgcn_update_dpp(0, (int) hi, 0xB1, 0xF, 0xF, false);
        lo |= __builtin_amdgcn_update_dpp(0, (int) lo, 0x4E, 0xF, 0xF, false);
        hi |= __builtin_amdgcn_update_dpp(0, (int) hi, 0x4E, 0xF, 0xF, false);
        lo |= __builtin_amdgcn_update_dpp(0, (int) lo, 0x141, 0xF, 0xF, false);
        hi |= __builtin_amdgcn_update_dpp(0, (int) hi, 0x141, 0xF, 0xF, false);
        lo |= __builtin_amdgcn_update_dpp(0, (int) lo, 0x140, 0xF, 0xF, false);
        hi |= __builtin_amdgcn_update_dpp(0, (int) hi, 0x140, 0xF, 0xF, false);
        lo = (unsigned) __builtin_amdgcn_readlane((int) lo, 0) | (unsigned) __builtin_amdgcn_readlane((int) lo, 16) |
             (unsigned) __builtin_amdgcn_readlane((int) lo, 32) | (unsigned) __builtin_amdgcn_readlane((int) lo, 48);
        hi = (unsigned) __builtin_amdgcn_readlane((int) hi, 0) | (unsigned) __builtin_amdgcn_readlane((int) hi, 16) |
             (unsigned) __builtin_amdgcn_readlane((int) hi, 32) | (unsigned) __builtin_amdgcn_readlane((int) hi, 48);
        seen = ((unsigned long long) hi << 32) | lo;
        const unsigned long long want = k >= 64 ? ~0ull : ((1ull << k) - 1ull);
        tie = !(cnt == k && seen == want);
    }
    if (tie) {
        // rare: recount with the id tie-break over the whole row
#pragma unroll
        for (int i = 0; i < EPL; i++) rank[i] = 0;
        for (int e2 = 0; e2 < E; e2 += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(s_l + e2);
            const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
#pragma unroll
                for (int i = 0; i < EPL; i++) {
                    const int e = lane + kWave * i;
                    rank[i] += (vv[u] > l[i]) || (vv[u] == l[i] && e2 + u < e);
                }
            }
        }
    }
    return true;
}

// Order key of a logit: monotone in the value, -0 and +0 equal, every real logit's key > 0 (route_one
// places it above the expert's id, so the keys are unique and 0 marks an expert past E).
__device__ __forceinline__ unsigned select_key(float v) {
    unsigned u = __float_as_uint(v);
    if (v == 0.0f) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Softmax, renormalisation and output of one token whose ranks rank_token found (part 0 only).
template <int EPL>
__device__ __forceinline__ void weights_token(int k, const float (&l)[EPL], const bool (&valid)[EPL], const int (&rank)[EPL],
                                              float *s_p, int16_t *ids16, int32_t *ids32, float *weights, int32_t *ids32_b,
                                              float *weights_b) {
    const int lane = threadIdx.x % kWave;
    // softmax over the row
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; i++) m = fmaxf(m, l[i]);
    m = wave_max(m);
    float p[EPL];
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        p[i] = valid[i] ? expf(l[i] - m) : 0.0f;
        s += (double) p[i];
    }
    const float inv = (float) (1.0 / wave_sum_d(s));
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        p[i] = p[i] * inv;
        if (valid[i] && rank[i] < k) s_p[rank[i]] = p[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    double ss = 0.0;
    for (int j = 0; j < k; j++) ss += (double) s_p[j];
    const float sf = fmaxf((float) ss, 6.103515625e-5f);
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        if (valid[i] && rank[i] < k) {
            const int e = lane + kWave * i;
            const float w = __fdiv_rn(p[i], sf);
            if (ids16) ids16[rank[i]] = (int16_t) e;
            if (ids32) ids32[rank[i]] = e;
            if (weights) weights[rank[i]] = w;
            if (ids32_b) ids32_b[rank[i]] = e;
            if (weights_b) weights_b[rank[i]] = w;
        }
    }
}


template <int EPL>
__device__ __forceinline__ void topk_token(const float *__restrict__ l_row, int E, int k, int part, int nsplit, float *s_l,
                                           int *s_rank, float *s_p, int16_t *ids16, int32_t *ids32, float *weights,
                                           int32_t *ids32_b, float *weights_b) {
    float l[EPL];
    bool valid[EPL];
    int rank[EPL];
    if (rank_token<EPL>(l_row, E, k, part, nsplit, s_l, s_rank, l, valid, rank))
        weights_token<EPL>(k, l, valid, rank, s_p, ids16, ids32, weights, ids32_b, weights_b);
}

// Top-k of T tokens by the block's wavefronts: one wavefront per token, or all wavefronts on one
// token when there are fewer tokens than wavefronts. The block must call this uniformly.
__device__ __forceinline__ void topk_block(const float *__restrict__ logits, int T, int E, int k, unsigned char *lds, int16_t *ids16,
                           int32_t *ids32, float *weights, int32_t *ids32_b, float *weights_b) {
    const int wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    const int nsplit = T < nw ? nw : 1;
    const int epl = (E + kWave - 1) / kWave;
    // one row per wavefront (or one shared row when they split a token); the rank partials of all
    // wavefronts: nw * kMaxEPL * 64 ints in either mode
    float *s_l = reinterpret_cast<float *>(lds);                             // [nw][256]
    int *s_rank = reinterpret_cast<int *>(lds + (size_t) nw * 256 * 4);       // [nw * kMaxEPL * 64]
    float *s_p = reinterpret_cast<float *>(s_rank + (size_t) nw * kMaxEPL * kWave); // [nw][kMaxK]
    for (int t0 = 0; t0 < T; t0 += (nsplit > 1 ? 1 : nw)) {
        const int t = nsplit > 1 ? t0 : t0 + wave;
        const int part = nsplit > 1 ? wave : 0;
        const int slot = nsplit > 1 ? 0 : wave; // LDS set of this token's group
        if (t < T) {
            const size_t o = (size_t) t * k;
            float *sl = s_l + slot * 256;
            int *sr = s_rank + (size_t) slot * kMaxEPL * kWave;
            float *sp = s_p + slot * kMaxK;
            const float *lr = logits + (size_t) t * E;
            int16_t *a = ids16 ? ids16 + o : nullptr;
            int32_t *b = ids32 ? ids32 + o : nullptr;
            float *c = weights ? weights + o : nullptr;
            int32_t *d = ids32_b ? ids32_b + o : nullptr;
            float *f = weights_b ? weights_b + o : nullptr;
            if (epl == 1) topk_token<1>(lr, E, k, part, nsplit, sl, sr, sp, a, b, c, d, f);
            else if (epl == 2) topk_token<2>(lr, E, k, part, nsplit, sl, sr, sp, a, b, c, d, f);
            else topk_token<4>(lr, E, k, part, nsplit, sl, sr, sp, a, b, c, d, f);
        }
        if (nsplit > 1) __syncthreads();
    }
}

__device__ __host__ inline size_t topk_lds_bytes(int nw) {
    return (size_t) nw * 256 * 4 + (size_t) nw * kMaxEPL * kWave * 4 + (size_t) nw * kMaxK * 4;
}

// ------------------------------------------------------------------------------------------------
// super-block dot products (ggml_vec_dot_q8_0_q8_0 / ggml_vec_dot_q4_K_q8_K)
// ------------------------------------------------------------------------------------------------

template <int I>
__device__ __forceinline__ unsigned dword_of(const uint4 &v) {
    return I == 0 ? v.x : I == 1 ? v.y : I == 2 ? v.z : v.w;
}

// Q8_0: 8 blocks of 32; per block an exact int32 sum, then acc += sumi * (d_w * d_x).
__device__ __forceinline__ float dot_sb_q8_0(const uint4 (&w)[kChunksQ8_0], const int8_t *x, const float *xd,
                                             float acc) {
#pragma unroll
    for (int blk = 0; blk < 8; blk++) {
        const uint4 q0 = w[1 + 2 * blk], q1 = w[2 + 2 * blk];
        const int4 x0 = *reinterpret_cast<const int4 *>(x + 32 * blk);
        const int4 x1 = *reinterpret_cast<const int4 *>(x + 32 * blk + 16);
        int s = 0;
        s = __builtin_amdgcn_sdot4((int) q0.x, x0.x, s, false);
        s = __builtin_amdgcn_sdot4((int) q0.y, x0.y, s, false);
        s = __builtin_amdgcn_sdot4((int) q0.z, x0.z, s, false);
        s = __builtin_amdgcn_sdot4((int) q0.w, x0.w, s, false);
        s = __builtin_amdgcn_sdot4((int) q1.x, x1.x, s, false);
        s = __builtin_amdgcn_sdot4((int) q1.y, x1.y, s, false);
        s = __builtin_amdgcn_sdot4((int) q1.z, x1.z, s, false);
        s = __builtin_amdgcn_sdot4((int) q1.w, x1.w, s, false);
        const unsigned dw2 = blk < 2 ? w[0].x : blk < 4 ? w[0].y : blk < 6 ? w[0].z : w[0].w;
        const float dw = h2f((blk & 1) ? (dw2 >> 16) : dw2);
        acc += (float) s * (dw * xd[blk]);
    }
    return acc;
}


// Q4_K x Q8_K: isum = sum_j sc_j * dot_j, imin = sum_j m_j * bsum_j;
// acc += (d_w d_x) isum, then acc -= (dmin_w d_x) imin.
template <int C>
__device__ __forceinline__ void q4_chunk(const uint4 &qa, const uint4 &qb, const int8_t *x, int &lo, int &hi) {
    const int4 xl0 = *reinterpret_cast<const int4 *>(x);
    const int4 xl1 = *reinterpret_cast<const int4 *>(x + 16);
    const int4 xh0 = *reinterpret_cast<const int4 *>(x + 32);
    const int4 xh1 = *reinterpret_cast<const int4 *>(x + 48);
    const unsigned m4 = 0x0f0f0f0fu;
    lo = __builtin_amdgcn_sdot4((int) (qa.x & m4), xl0.x, 0, false);
    lo = __builtin_amdgcn_sdot4((int) (qa.y & m4), xl0.y, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qa.z & m4), xl0.z, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qa.w & m4), xl0.w, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qb.x & m4), xl1.x, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qb.y & m4), xl1.y, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qb.z & m4), xl1.z, lo, false);
    lo = __builtin_amdgcn_sdot4((int) (qb.w & m4), xl1.w, lo, false);
    hi = __builtin_amdgcn_sdot4((int) ((qa.x >> 4) & m4), xh0.x, 0, false);
    hi = __builtin_amdgcn_sdot4((int) ((qa.y >> 4) & m4), xh0.y, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qa.z >> 4) & m4), xh0.z, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qa.w >> 4) & m4), xh0.w, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qb.x >> 4) & m4), xh1.x, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qb.y >> 4) & m4), xh1.y, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qb.z >> 4) & m4), xh1.z, hi, false);
    hi = __builtin_amdgcn_sdot4((int) ((qb.w >> 4) & m4), xh1.w, hi, false);
}

__device__ __forceinline__ float dot_sb_q4_K(const uint4 (&w)[kChunksQ4_K], const int8_t *x, const float *xd,
                                             const int *xb, float acc) {
    const float dw = h2f(w[0].x), dmin = h2f(w[0].x >> 16);
    const unsigned s0 = w[0].y, s1 = w[0].z, s2 = w[0].w;
    int isum = 0, imin = 0;
    int lo, hi, sc, m;
    q4_chunk<0>(w[1], w[2], x, lo, hi);
    scale_min_k4<0>(s0, s1, s2, sc, m); isum += sc * lo; imin += m * xb[0];
    scale_min_k4<1>(s0, s1, s2, sc, m); isum += sc * hi; imin += m * xb[1];
    q4_chunk<1>(w[3], w[4], x + 64, lo, hi);
    scale_min_k4<2>(s0, s1, s2, sc, m); isum += sc * lo; imin += m * xb[2];
    scale_min_k4<3>(s0, s1, s2, sc, m); isum += sc * hi; imin += m * xb[3];
    q4_chunk<2>(w[5], w[6], x + 128, lo, hi);
    scale_min_k4<4>(s0, s1, s2, sc, m); isum += sc * lo; imin += m * xb[4];
    scale_min_k4<5>(s0, s1, s2, sc, m); isum += sc * hi; imin += m * xb[5];
    q4_chunk<3>(w[7], w[8], x + 192, lo, hi);
    scale_min_k4<6>(s0, s1, s2, sc, m); isum += sc * lo; imin += m * xb[6];
    scale_min_k4<7>(s0, s1, s2, sc, m); isum += sc * hi; imin += m * xb[7];
    const float dx = xd[0];
    acc += (dw * dx) * (float) isum;
    acc -= (dmin * dx) * (float) imin;
    return acc;
}

// KQ8 (Q2_K, Q3_K, Q5_K, Q6_K unpacked) x Q8_K: per 16-value group g, dot_g = q_g . x_g and bsum_g =
// the sum of x_g (both exact int32 from v_dot4); isum = sum_g sc_g dot_g, imin = sum_g m_g bsum_g;
// acc += (d_w d_x) isum, then acc -= (dmin_w d_x) imin.
__device__ __forceinline__ float dot_sb_kq8(const uint4 (&w)[kChunksKQ8], const int8_t *x, const float *xd, float acc) {
    const float dw = __uint_as_float(w[0].x), dmin = __uint_as_float(w[0].y);
    int isum = 0, imin = 0;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const int4 xv = *reinterpret_cast<const int4 *>(x + 16 * g);
        const uint4 q = w[3 + g];
        int s = __builtin_amdgcn_sdot4((int) q.x, xv.x, 0, false);
        s = __builtin_amdgcn_sdot4((int) q.y, xv.y, s, false);
        s = __builtin_amdgcn_sdot4((int) q.z, xv.z, s, false);
        s = __builtin_amdgcn_sdot4((int) q.w, xv.w, s, false);
        int b = __builtin_amdgcn_sdot4(0x01010101, xv.x, 0, false);
        b = __builtin_amdgcn_sdot4(0x01010101, xv.y, b, false);
        b = __builtin_amdgcn_sdot4(0x01010101, xv.z, b, false);
        b = __builtin_amdgcn_sdot4(0x01010101, xv.w, b, false);
        const unsigned scw = g < 4 ? w[1].x : g < 8 ? w[1].y : g < 12 ? w[1].z : w[1].w;
        const unsigned mw = g < 4 ? w[2].x : g < 8 ? w[2].y : g < 12 ? w[2].z : w[2].w;
        const int sc = (int) (int8_t) (scw >> (8 * (g % 4))), m = (int) ((mw >> (8 * (g % 4))) & 0xFFu);
        isum += sc * s;
        imin += m * b;
    }
    const float dx = xd[0];
    acc += (dw * dx) * (float) isum;
    acc -= (dmin * dx) * (float) imin;
    return acc;
}

// Marks a super-block's weight registers as rewritten (an empty asm statement: no instruction), so that
// what dot_sb derives from them (masked nibbles, scales, fp16 factors) is formed again at each call in a
// loop over tokens instead of being held in registers across the loop: the raw chunks stay the only live
// copy, which keeps multi-token expert kernels at more wavefronts per SIMD. Values are unchanged.
template <int C>
__device__ __forceinline__ void rederive(uint4 (&w)[C]) {
#pragma unroll
    for (int c = 0; c < C; c++) asm volatile("" : "+v"(w[c].x), "+v"(w[c].y), "+v"(w[c].z), "+v"(w[c].w));
}

template <int WT>
__device__ __forceinline__ float dot_sb(const uint4 (&w)[chunks_of(WT)], const int8_t *x, const float *xd,
                                        const int *xb, float acc) {
    if constexpr (WT == kTypeQ8_0) {
        (void) xb;
        return dot_sb_q8_0(w, x, xd, acc);
    } else if constexpr (WT == kTypeKQ8) {
        (void) xb;
        return dot_sb_kq8(w, x, xd, acc);
    } else {
        return dot_sb_q4_K(w, x, xd, xb, acc);
    }
}

// Super-blocks per thread S and K-groups G for nsb super-blocks: the smallest S <= 2 dividing nsb
// with nsb / S <= 8 (S = 3 would need more than 256 VGPRs and spill).
inline bool pick_split(int nsb, int *S, int *G) {
    for (int s = 1; s <= 2; s++) {
        if (nsb % s == 0 && nsb / s <= kMaxG) {
            *S = s;
            *G = nsb / s;
            return true;
        }
    }
    return false;
}

// gate_up additionally needs 128 % G == 0 (rows per work-group = 128 / G).
inline bool pick_split_gate_up(int nsb, int *S, int *G) { return pick_split(nsb, S, G) && 128 % *G == 0; }

// A launch on `st`; with `tm` set, the launch records its own start / stop timestamps.
template <typename K, typename... A>
hipError_t launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, const LaunchTiming *tm, A... args) {
    if (tm && tm->start) hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t) lds, st, tm->start, tm->stop, 0, args...);
    else hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    return hipGetLastError();
}

}  // namespace
}  // namespace lstk
