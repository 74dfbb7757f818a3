// grouped.hip - gfx950 kernels of the grouped (prefill) path, for calls that route many tokens to
// each expert. ggml's CPU mul_mat_id groups the (token, slot) pairs by expert and runs each expert's
// matrix over its rows (src/qwen3.cpp:201-204); here that is:
//   permute    one work-group: per-bin counts, exclusive offsets, the stable token-major pair order
//              and the work list of 32-pair chunks, expert-major (each expert's chunks in order).
//   gate_up    per (chunk, 64-row block): Q4_K gate and up rows x Q8_K token rows on
//              v_mfma_i32_32x32x32_i8, fused SwiGLU (src/qwen3.cpp:201-203).
//   act_quant  the SwiGLU rows to Q8_K, the activation type ggml pairs with Q4_K down weights.
//   down       per (chunk, 128-row block): Q4_K down rows x Q8_K SwiGLU rows, times the router
//              weight (src/qwen3.cpp:204-205). The existing combine kernel sums the k rows.
//
// Integer semantics of ggml's vec_dot_q4_K_q8_K on the matrix cores. Per super-block of 256 values
// ggml computes d_x (d_w isum - dmin_w imin) with isum = sum_j sc_j sum_i q_ji x_ji (q in [0, 15],
// sc_j and m_j 6-bit) and imin = sum_j m_j sum_i x_ji. sc_j q does not fit int8, so sc_j is split as
// 8 sh_j + sl_j (both <= 7) and two int8 weight planes go through v_mfma_i32_32x32x32_i8 with the
// int8 activations: sh_j q and sl_j q (both <= 105); isum = 8 accH + accL. imin is one
// v_mfma_f32_32x32x16_f16 per super-block over the activations' group sums s_j, each given as the
// fp16 pair (64 floor(s_j / 64), s_j mod 64) (the quantizer writes them), against (m_j, m_j): every
// product and partial sum is an integer below 2^24, so the f32 result is imin exactly. Both match
// ggml's integer arithmetic; only the f32 accumulation over super-blocks is ordered differently.
#include "device.h"
#include "formats.h"
#include "kernels.h"

#include <algorithm>

namespace lstk {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kGThreads = 256;        // 4 wavefronts per grouped work-group
constexpr int kPermThreads = 1024;
constexpr int kPermSeg = kPermThreads / kWave; // one pair segment per wavefront
constexpr int kPermMaxPairs = 8192;

__device__ __forceinline__ i32x16 mfma_i8(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f16(u32x4 a, u32x4 b) {
    const f32x16 z = {};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), z, 0, 0, 0);
}

// Byte-wise product of four values <= 15 with s <= 7 (s2 = s | s << 16): the products stay below
// 128, so two 16-bit multiplies carry nothing across bytes.
__device__ __forceinline__ int mul_bytes(unsigned v, unsigned s2) {
    return __builtin_bit_cast(int, __builtin_bit_cast(u16x2, v) * __builtin_bit_cast(u16x2, s2));
}

// ------------------------------------------------------------------------------------------------
// permutation
// ------------------------------------------------------------------------------------------------

// The wavefront's index within the work-group, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int) threadIdx.x / kWave); }

__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Inclusive prefix sum over the wavefront by DPP: within each row of 16 lanes (row_shr 1, 2, 4, 8,
// lanes without a source adding 0), then the totals of rows 0 and 2 into rows 1 and 3 (row_bcast:15)
// and the total of rows 0-1 into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast15, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast31, 0xC, 0xF, false);
    return v;
}

// The pairs are cut into kPermSeg contiguous segments, one per wavefront. Pass 1 counts each
// segment's pairs per bin (16-bit counts, two bins per LDS word); per bin, the counts become an
// exclusive prefix over segments, and the totals an exclusive prefix over bins (the offsets).
// Pass 2: each wavefront walks its segment 64 pairs at a time; a pair's position is
// offsets[b] + (pairs of b in earlier segments and earlier chunks) + (lanes of the chunk before it
// with the same bin, found by matching ballots of the bin's bits). That is the stable order by pair
// index t * k + j within each bin.
__global__ __launch_bounds__(kPermThreads) void permute_kernel(PermuteParams P) {
    __shared__ unsigned seg[kPermSeg][kGroupedMaxBins / 2];
    __shared__ int16_t bl[kPermMaxPairs];
    __shared__ int cnt[kGroupedMaxBins];
    __shared__ int wsum[2][kPermSeg];
    const int tid = threadIdx.x, lane = tid % kWave, w = tid / kWave;
    const int np = P.np, nb = P.n_bins;
    const int wpr = (nb + 1) / 2; // count words in use per segment
    for (int i = tid; i < kPermSeg * wpr; i += kPermThreads) seg[i / wpr][i % wpr] = 0u;
    __syncthreads();
    const int L = ((np + kPermSeg - 1) / kPermSeg + kWave - 1) / kWave * kWave;
    const int s0 = min(np, w * L), s1 = min(np, s0 + L);
    // the segment's bins, all loads in flight together (a segment holds at most 8 * 64 pairs)
    int bv[kPermMaxPairs / kPermSeg / kWave];
#pragma unroll
    for (int u = 0; u < kPermMaxPairs / kPermSeg / kWave; u++) {
        const int p = s0 + lane + u * kWave;
        bv[u] = p < s1 ? P.bins[p] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPermMaxPairs / kPermSeg / kWave; u++) {
        const int p = s0 + lane + u * kWave;
        if (p < s1) {
            int b = bv[u];
            if (b < 0 || b >= nb) {
                atomicOr(P.err, 1);
                b = min(max(b, 0), nb - 1);
            }
            bl[p] = (int16_t) b;
            atomicAdd(&seg[w][b >> 1], 1u << (16 * (b & 1)));
        }
    }
    __syncthreads();
    for (int wi = tid; wi < (nb + 1) / 2; wi += kPermThreads) {
        unsigned lo = 0, hi = 0;
        for (int s = 0; s < kPermSeg; s++) {
            const unsigned v = seg[s][wi];
            seg[s][wi] = lo | (hi << 16);
            lo += v & 0xffffu;
            hi += v >> 16;
        }
        cnt[2 * wi] = (int) lo;
        if (2 * wi + 1 < nb) cnt[2 * wi + 1] = (int) hi;
    }
    __syncthreads();
    // offsets and the work list: one bin per thread (n_bins <= 1024)
    const int c = tid < nb ? cnt[tid] : 0;
    const int nch = (c + P.chunk - 1) / P.chunk; // the bin's work items: its chunks in order
    const int v0 = wave_incl_scan(c), v1 = wave_incl_scan(nch);
    if (lane == kWave - 1) {
        wsum[0][w] = v0;
        wsum[1][w] = v1;
    }
    __syncthreads();
    int b0 = 0, b1 = 0, tot0 = 0, tot1 = 0;
    for (int s = 0; s < kPermSeg; s++) {
        if (s < w) {
            b0 += wsum[0][s];
            b1 += wsum[1][s];
        }
        tot0 += wsum[0][s];
        tot1 += wsum[1][s];
    }
    const int off = b0 + v0 - c;
    if (tid < nb) {
        P.counts[tid] = c;
        P.offsets[tid] = off;
        if (P.items) {
            // expert-major: a bin's chunks are consecutive items (XCD-aware mapping keeps them on one XCD)
            const int fb = b1 + v1 - nch;
            for (int i = 0; i < nch; i++) P.items[fb + i] = make_int4(tid, off + i * P.chunk, min(P.chunk, c - i * P.chunk), 0);
        }
        cnt[tid] = off;
    }
    if (tid == 0) {
        P.offsets[nb] = tot0;
        if (P.n_items) *P.n_items = tot1;
    }
    __syncthreads();
    const int key_bits = 32 - __builtin_clz((unsigned) nb);
    for (int base = s0; base < s1; base += kWave) {
        const int p = base + lane;
        const bool on = p < s1;
        const int b = on ? (int) bl[p] : nb; // a key no real bin has
        // lanes with the same bin: the AND over the key's bits (keys 0 .. nb) of the matching ballots
        unsigned long long mask = ~0ull;
        for (int bit = 0; bit < key_bits; bit++) {
            const bool set = (b >> bit) & 1;
            const unsigned long long bb = __ballot(set);
            mask &= set ? bb : ~bb;
        }
        const unsigned long long lt = (1ull << lane) - 1ull;
        const int before = __popcll(mask & lt), after = __popcll(mask & ~lt) - 1;
        int pos = 0;
        if (on) {
            const unsigned word = seg[w][b >> 1];
            pos = cnt[b] + (int) ((b & 1) ? (word >> 16) : (word & 0xffffu)) + before;
        }
        lds_fence();
        if (on) {
            P.perm[pos] = p;
            if (after == 0) atomicAdd(&seg[w][b >> 1], (unsigned) (before + 1) << (16 * (b & 1)));
        }
        lds_fence();
    }
}

// ------------------------------------------------------------------------------------------------
// grouped Q4_K x Q8_K products on the matrix cores
// ------------------------------------------------------------------------------------------------

// The operands of one super-block of a work-group (a stage of an LDS ring of kNS stages):
//   A   [kGroupedChunk rows][16 pieces of 16 B]: the staged activation rows, piece p of row t at slot
//       16 t + (p ^ (t & 15)), so 16 consecutive rows reading one piece hit 16 different bank groups;
//   DX  [kGroupedChunk] f32: the rows' Q8_K scales;
//   W   [4 wavefronts][9 chunks][32 rows][16 B]: each wavefront's Q4_K rows.
// The activation rows, their scales and the weight rows arrive by global_load_lds (lane i of an
// instruction lands at ldsptr + size * i); each lane also loads its 16 bytes of the rows' split group
// sums into registers. Per stage, wavefront 0 issues kLoads0 loads and the others kLoads1.
// One stage by default: at 26.8 KB of LDS and under 128 VGPRs, four work-groups share a CU (four
// wavefronts per SIMD); a two-stage ring holds the CU to three, and the compiler waits for the
// next stage's loads at every barrier anyway, so the second stage overlaps nothing.
#ifndef LSTK_GROUPED_STAGES
#define LSTK_GROUPED_STAGES 1
#endif
constexpr int kNS = LSTK_GROUPED_STAGES;
// Minimum wavefronts per SIMD the grouped kernels are compiled for (0: the compiler's choice).
#ifndef LSTK_GROUPED_MIN_WAVES
#define LSTK_GROUPED_MIN_WAVES 0
#endif
constexpr int kMT = kGroupedChunk / 32;              // 32-row M-tiles per wavefront
constexpr int kAInstr = kGroupedChunk * 16 / kWave / 4; // activation loads per wavefront
constexpr int kABytes = kGroupedChunk * 256;
constexpr int kDXBytes = kGroupedChunk * 4;
constexpr int kWWaveBytes = 9 * 32 * 16;
constexpr int kStageBytes = kABytes + kDXBytes + 4 * kWWaveBytes;
constexpr int kLoads1 = kAInstr + 5 + kMT, kLoads0 = kLoads1 + 1;
constexpr size_t kGLdsBytes = (size_t) kNS * kStageBytes + 2 * kGroupedChunk * 4;

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void *g, unsigned char *l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *) l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *g, unsigned char *l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *) l, 4, 0, 0);
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

struct GLds {
    unsigned char *ring; // [kNS][kStageBytes]
    int *pair;           // [kGroupedChunk] pair index of each chunk position
    int *src;            // [kGroupedChunk] activation row of each chunk position
};

__device__ __forceinline__ GLds g_lds(unsigned char *base) {
    GLds g;
    g.ring = base;
    g.pair = reinterpret_cast<int *>(base + (size_t) kNS * kStageBytes);
    g.src = g.pair + kGroupedChunk;
    return g;
}

// Per-lane byte offsets of a work item's loads (fixed over the super-blocks, so the loop only moves
// the wave-uniform bases): kAInstr activation pieces, the row scale, 5 weight chunk pairs, and per
// M-tile the split group sums 4 (lane / 32) .. + 3 of row 32 mt + lane % 32.
struct DmaOffs {
    unsigned a[kAInstr], dx, w[5], bh[kMT];
    unsigned live; // bit i: activation piece i is a real row of the chunk (t < n); bit 31: the lane's scale is
};

__device__ __forceinline__ DmaOffs dma_offsets(const GroupedParams &P, const GLds &g, int n, int row0) {
    const int wave = wave_id(), lane = threadIdx.x % kWave;
    DmaOffs o;
#pragma unroll
    for (int i = 0; i < kAInstr; i++) {
        const int s = (wave * kAInstr + i) * kWave + lane;
        const int t = s >> 4, part = (s & 15) ^ (t & 15);
        o.a[i] = (unsigned) g.src[min(t, n - 1)] * (unsigned) P.K + part * 16;
        if (i == 0) o.live = 0u;
        if (t < n) o.live |= 1u << i;
    }
    o.dx = (unsigned) g.src[min(lane, n - 1)] * (unsigned) (P.K / 32) * 4;
    if (lane < n) o.live |= 1u << 31;
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const int c = min(2 * i + (lane >> 5), 8);
        o.w[i] = (unsigned) chunk_offset(kChunksQ4_K, P.rows, P.K / 256, 0, c, row0 + (lane & 31));
    }
#pragma unroll
    for (int mt = 0; mt < kMT; mt++)
        o.bh[mt] = ((unsigned) g.src[min(32 * mt + (lane & 31), n - 1)] * (unsigned) (P.K / 32) + 4 * (lane >> 5)) * 4;
    return o;
}

// Issues the loads of super-block sb (activation rows of the chunk, the wavefront's 32 weight rows
// of matrix w) into ring stage `slot`, and the lane's split group sums into bq.
__device__ __forceinline__ void issue_stage(const GroupedParams &P, const GLds &g, const DmaOffs &o, const uint8_t *w,
                                            int sb, int slot, u32x4 (&bq)[kMT]) {
    const int wave = wave_id(), lane = threadIdx.x % kWave;
    // Each 32-bit offset passes through an empty asm here, so it is extended to 64 bits next to its
    // load: the load then takes the form (scalar base + 32-bit vector offset) instead of a 64-bit
    // vector address kept live across the loop.
    auto off = [](unsigned v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    unsigned char *st = g.ring + (size_t) slot * kStageBytes;
    const uint8_t *xa = reinterpret_cast<const uint8_t *>(P.xqs) + sb * 256;
#pragma unroll
    // rows past the chunk's n pairs are not loaded: their LDS rows hold stale bytes, and the products of
    // those rows are never stored
    for (int i = 0; i < kAInstr; i++)
        if (o.live & (1u << i)) dma16(xa + off(o.a[i]), st + (wave * kAInstr + i) * 1024);
    if (wave == 0 && lane < kGroupedChunk && (o.live >> 31))
        dma4(reinterpret_cast<const uint8_t *>(P.xd) + sb * 32 + off(o.dx), st + kABytes);
    // every row block of the matrix is full (rows % 64 == 0, grouped_supported), so super-block sb of a
    // lane's rows lies sb * C * kPoolRB chunks past its super-block 0
    static_assert(64 % kPoolRB == 0, "the grouped kernels need row blocks that divide 64 rows");
    const uint8_t *wb = w + (size_t) sb * kChunksQ4_K * kPoolRB * 16;
    unsigned char *wl = st + kABytes + kDXBytes + wave * kWWaveBytes;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(wb + off(o.w[i]), wl + i * 1024);
    if (lane < 32) dma16(wb + off(o.w[4]), wl + 4 * 1024);
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(P.xbh) + sb * 32;
#pragma unroll
    for (int mt = 0; mt < kMT; mt++) bq[mt] = *reinterpret_cast<const u32x4 *>(xb + off(o.bh[mt]));
}

// One staged super-block in two phases. Phase 1 (q4k_products) reads everything it needs from the stage -
// the weight header and chunks of the wavefront's 32 rows (lane % 32), the chunk's activation fragments and
// their rows' Q8_K scales - builds the weight planes and runs the int8 products of M-tile mt = chunk rows
// 32 mt .. 32 mt + 31 into S. Phase 2 (q4k_accumulate) runs from registers only: the min-term product and
// acc[mt][r] += d_x (d_w isum - dmin_w imin) for chunk row 32 mt + 8 (r / 4) + 4 (lane / 32) + r % 4. So
// the next stage's loads can be issued between the two and land while phase 2 runs. bq[mt]: the lane's
// split group sums (sub-blocks 4 (lane / 32) .. + 3 of chunk row 32 mt + lane % 32).
//
// Lane half h = lane / 32 takes qs bytes [32 c + 16 h, + 16) of each 64-value chunk c of its row:
// low nibbles are values 64 c + 16 h + [0, 16) of sub-block 2 c, high nibbles values
// 64 c + 32 + 16 h + [0, 16) of sub-block 2 c + 1, exactly the K slice the MFMA takes from the lane.
// In the imin product, lane half h gives K entries 8 h .. 8 h + 7, the pairs of sub-blocks 4 h .. + 3.
struct SbProducts {
    i32x16 aH[kMT], aL[kMT];
    float dx[kMT][16]; // the Q8_K scale of each output's chunk row
    unsigned dd;       // the rows' d and dmin (fp16 pair)
    unsigned mins;     // the 6-bit mins of sub-blocks 4 h .. 4 h + 3, one per byte
};

__device__ __forceinline__ void q4k_products(const unsigned char *st, int n, SbProducts &S) {
    const int wave = wave_id(), lane = threadIdx.x % kWave, h = lane / 32, r32 = lane % 32;
    const unsigned char *wl = st + kABytes + kDXBytes + wave * kWWaveBytes;
    const uint4 hdr = *reinterpret_cast<const uint4 *>(wl + r32 * 16);
    uint4 qv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) qv[c] = *reinterpret_cast<const uint4 *>(wl + (1 + 2 * c + h) * 512 + r32 * 16);
    const unsigned s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
    // the 6-bit scales of get_scale_min_k4, one per byte (sub-blocks 0-3 and 4-7), split as 8 sh + sl
    const unsigned sc_lo = s0 & 0x3f3f3f3fu, sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const unsigned sh4[2] = {(sc_lo >> 3) & 0x07070707u, (sc_hi >> 3) & 0x07070707u};
    const unsigned sl4[2] = {sc_lo & 0x07070707u, sc_hi & 0x07070707u};
#pragma unroll
    for (int c = 0; c < 4; c++) {
#pragma unroll
        for (int nib = 0; nib < 2; nib++) {
            // byte j % 4 of the packed scales into both 16-bit halves (v_perm_b32 selector 0x0c is a zero byte)
            const int j = 2 * c + nib;
            const unsigned sel = 0x0c000c00u | (unsigned) (j & 3) * 0x10001u;
            const unsigned sh = __builtin_amdgcn_perm(0u, sh4[j >> 2], sel), sl = __builtin_amdgcn_perm(0u, sl4[j >> 2], sel);
            const uint4 q = qv[c];
            const unsigned k4 = 0x0f0f0f0fu;
            const unsigned n0 = nib ? (q.x >> 4) & k4 : q.x & k4, n1 = nib ? (q.y >> 4) & k4 : q.y & k4;
            const unsigned n2 = nib ? (q.z >> 4) & k4 : q.z & k4, n3 = nib ? (q.w >> 4) & k4 : q.w & k4;
            const i32x4 bh = {mul_bytes(n0, sh), mul_bytes(n1, sh), mul_bytes(n2, sh), mul_bytes(n3, sh)};
            const i32x4 bl = {mul_bytes(n0, sl), mul_bytes(n1, sl), mul_bytes(n2, sl), mul_bytes(n3, sl)};
            const int part = 4 * c + 2 * nib + h;
#pragma unroll
            for (int mt = 0; mt < kMT; mt++) {
                if (mt > 0 && n <= 32 * mt) continue;
                const int t = mt * 32 + r32;
                const i32x4 a = *reinterpret_cast<const i32x4 *>(st + (t * 16 + (part ^ (t & 15))) * 16);
                if (c == 0 && nib == 0) {
                    const i32x16 z = {};
                    S.aH[mt] = mfma_i8(a, bh, z);
                    S.aL[mt] = mfma_i8(a, bl, z);
                } else {
                    S.aH[mt] = mfma_i8(a, bh, S.aH[mt]);
                    S.aL[mt] = mfma_i8(a, bl, S.aL[mt]);
                }
            }
        }
    }
    S.dd = hdr.x;
    S.mins = h ? ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u) : s1 & 0x3f3f3f3fu;
    const float *dxs = reinterpret_cast<const float *>(st + kABytes);
#pragma unroll
    for (int mt = 0; mt < kMT; mt++)
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const float4 d4 = *reinterpret_cast<const float4 *>(dxs + mt * 32 + 8 * a4 + 4 * h);
            S.dx[mt][4 * a4] = d4.x;
            S.dx[mt][4 * a4 + 1] = d4.y;
            S.dx[mt][4 * a4 + 2] = d4.z;
            S.dx[mt][4 * a4 + 3] = d4.w;
        }
}

__device__ __forceinline__ void q4k_accumulate(const SbProducts &S, int n, const u32x4 (&bq)[kMT], float (&acc)[kMT][16]) {
    const float dw = h2f(S.dd), dmin = h2f(S.dd >> 16);
    // each min as an fp16 pair
    u32x4 bm;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float mf = (float) ((S.mins >> (8 * i)) & 0xffu);
        bm[i] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(mf, mf));
    }
#pragma unroll
    for (int mt = 0; mt < kMT; mt++) {
        if (mt > 0 && n <= 32 * mt) continue;
        const f32x16 aM = mfma_f16(bq[mt], bm);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float isum = (float) (8 * S.aH[mt][r] + S.aL[mt][r]);
            acc[mt][r] = fmaf(S.dx[mt][r], fmaf(dw, isum, -(dmin * aM[r])), acc[mt][r]);
        }
    }
}

// The whole K of the wavefront's 32 rows (row0 + lane % 32 of matrix w) against the chunk's n
// activation rows; called uniformly by the 4 wavefronts. With kNS > 1 stages, stage sb + kNS - 1 is
// in flight while stage sb is multiplied (its split group sums in bq[kNS - 2]); with one stage, each
// super-block is loaded, waited for and multiplied in turn.
__device__ __forceinline__ void q4k_rows(const GroupedParams &P, const GLds &g, int n, const uint8_t *w, int row0,
                                         float (&acc)[kMT][16]) {
    const int nsb = P.K / 256;
#pragma unroll
    for (int mt = 0; mt < kMT; mt++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[mt][r] = 0.0f;
    const DmaOffs o = dma_offsets(P, g, n, row0);
    if constexpr (kNS == 1) {
        // the next super-block's loads are issued as soon as every wavefront has read the stage, so they
        // are in flight while the float epilogue of this one runs from registers
        u32x4 cur[kMT];
        issue_stage(P, g, o, w, 0, 0, cur);
        for (int sb = 0; sb < nsb; sb++) {
            wait_vm<0>();
            __syncthreads();
            SbProducts S;
            q4k_products(g.ring, n, S);
            __syncthreads();
            u32x4 nxt[kMT];
            if (sb + 1 < nsb) issue_stage(P, g, o, w, sb + 1, 0, nxt);
            q4k_accumulate(S, n, cur, acc);
#pragma unroll
            for (int mt = 0; mt < kMT; mt++) cur[mt] = nxt[mt];
        }
    } else {
        const bool w0 = threadIdx.x < kWave;
        u32x4 bq[kNS > 1 ? kNS - 1 : 1][kMT]; // (sized 1 where the one-stage branch is the live one)
#pragma unroll
        for (int s = 0; s < kNS - 1; s++)
            if (s < nsb) issue_stage(P, g, o, w, s, s, bq[s]);
        for (int sb = 0; sb < nsb; sb++) {
            u32x4 cur[kMT];
#pragma unroll
            for (int mt = 0; mt < kMT; mt++) cur[mt] = bq[0][mt];
#pragma unroll
            for (int s = 0; s + 1 < kNS - 1; s++)
#pragma unroll
                for (int mt = 0; mt < kMT; mt++) bq[s][mt] = bq[s + 1][mt];
            if (sb + kNS - 1 < nsb) {
                issue_stage(P, g, o, w, sb + kNS - 1, (sb + kNS - 1) % kNS, bq[kNS > 1 ? kNS - 2 : 0]);
                if (w0) wait_vm<kLoads0 * (kNS - 1)>();
                else wait_vm<kLoads1 * (kNS - 1)>();
            } else {
                wait_vm<0>();
            }
            __syncthreads();
            SbProducts S;
            q4k_products(g.ring + (size_t) (sb % kNS) * kStageBytes, n, S);
            q4k_accumulate(S, n, cur, acc);
            __syncthreads();
        }
    }
}

// Work-group b -> (item, row block), XCD-aware: the dispatcher deals work-groups to the 8 XCDs in turn
// (b goes to XCD b % 8), so XCD x takes the items [x per, (x + 1) per) of the expert-major work list, all
// row blocks of an item before the next. The row blocks that share an item's activation rows, and the
// chunks that share an expert's weight rows, then meet in one XCD's L2.
constexpr int kXcds = 8;
// Reads the work item and row block of this work-group; false when it has none.
__device__ __forceinline__ bool g_item(const GroupedParams &P, int n_rb, const GLds &g, int4 &it, int &rb) {
    const int n_items = *P.n_items, per = (n_items + kXcds - 1) / kXcds;
    const int local = blockIdx.x / kXcds, item = (blockIdx.x % kXcds) * per + local / n_rb;
    if (local / n_rb >= per || item >= n_items) return false;
    rb = local % n_rb;
    it = P.items[item];
    const int tid = threadIdx.x;
    if (tid < kGroupedChunk) {
        const int p = P.perm[it.y + min(tid, it.z - 1)];
        g.pair[tid] = p;
        g.src[tid] = p / P.row_div;
    }
    __syncthreads();
    return true;
}

// gate_up: wavefront w computes rows rb * 64 + 32 (w / 2) .. + 31 of gate (w even) or up (w odd);
// the up wavefronts hand their sums to the gate wavefronts through LDS for the SwiGLU.
__global__ __launch_bounds__(kGThreads, LSTK_GROUPED_MIN_WAVES) void gate_up_grouped_kernel(GroupedParams P) {
    extern __shared__ __align__(16) unsigned char smem[];
    const GLds g = g_lds(smem);
    const int n_rb = P.rows / 64;
    int4 it;
    int rb;
    if (!g_item(P, n_rb, g, it, rb)) return;
    const int e = it.x, n = it.z;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int m = wave & 1, row0 = rb * 64 + 32 * (wave >> 1);
    const uint8_t *w = m ? P.w1 + (size_t) e * P.stride1 : P.w0 + (size_t) e * P.stride0;
    float acc[kMT][16];
    q4k_rows(P, g, n, w, row0, acc);
    float *ex = reinterpret_cast<float *>(g.ring); // [2 row halves][kMT M-tiles][16][64]
    float *mine = ex + (size_t) (wave >> 1) * kMT * 16 * kWave;
    if (m == 1) {
#pragma unroll
        for (int mt = 0; mt < kMT; mt++)
#pragma unroll
            for (int r = 0; r < 16; r++) mine[(mt * 16 + r) * kWave + lane] = acc[mt][r];
    }
    __syncthreads();
    if (m == 0) {
        const int h = lane / 32;
#pragma unroll
        for (int mt = 0; mt < kMT; mt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int pos = mt * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                if (pos < n) {
                    const float gs = acc[mt][r], us = mine[(mt * 16 + r) * kWave + lane];
                    P.out[(size_t) g.pair[pos] * P.rows + row0 + lane % 32] = (gs / (1.0f + expf(-gs))) * us;
                }
            }
        }
    }
}

// down: wavefront w computes rows rb * 128 + 32 w .. + 31, times the pair's router weight.
__global__ __launch_bounds__(kGThreads, LSTK_GROUPED_MIN_WAVES) void down_grouped_kernel(GroupedParams P) {
    extern __shared__ __align__(16) unsigned char smem[];
    const GLds g = g_lds(smem);
    const int n_rb = P.rows / 128;
    int4 it;
    int rb;
    if (!g_item(P, n_rb, g, it, rb)) return;
    const int e = it.x, n = it.z;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, h = lane / 32;
    const int row0 = rb * 128 + 32 * wave;
    float acc[kMT][16];
    q4k_rows(P, g, n, P.w0 + (size_t) e * P.stride0, row0, acc);
#pragma unroll
    for (int mt = 0; mt < kMT; mt++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int pos = mt * 32 + 8 * (r / 4) + 4 * h + (r % 4);
            if (pos < n) {
                const int p = g.pair[pos];
                P.out[(size_t) p * P.rows + row0 + lane % 32] = acc[mt][r] * P.weights[p];
            }
        }
    }
}

__global__ __launch_bounds__(128) void act_quant_kernel(const float *act, int f, int8_t *qs, float *d, int32_t *bs,
                                                        uint32_t *bh) {
    const size_t p = blockIdx.x;
    quantize_row<kTypeQ4_K>(act + p * f, f, qs + p * f, d + p * (f / 32), bs + p * (f / 32), bh + p * (f / 32));
}

}  // namespace

bool grouped_supported(int tu, int tg, int td, int h, int f, int n_bins) {
    return tu == kTypeQ4_K && tg == kTypeQ4_K && td == kTypeQ4_K && h % 256 == 0 && f % 256 == 0 && f % 64 == 0 &&
           n_bins >= 1 && n_bins <= kGroupedMaxBins;
}

int grouped_max_items(int np, int n_bins) { return (np + kGroupedChunk - 1) / kGroupedChunk + std::min(n_bins, np); }

hipError_t launch_permute(const PermuteParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.np <= 0) return hipSuccess;
    if (P.np > kPermMaxPairs || P.n_bins < 1 || P.n_bins > kGroupedMaxBins) return hipErrorInvalidValue;
    return launch(permute_kernel, dim3(1), dim3(kPermThreads), 0, st, tm, P);
}

// The grouped kernels take more than 64 KiB of dynamic LDS (gfx950 has 160 KiB per CU).
hipError_t allow_lds() {
    static hipError_t e = [] {
        hipError_t r = hipFuncSetAttribute(reinterpret_cast<const void *>(&gate_up_grouped_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int) kGLdsBytes);
        if (r == hipSuccess)
            r = hipFuncSetAttribute(reinterpret_cast<const void *>(&down_grouped_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int) kGLdsBytes);
        return r;
    }();
    return e;
}

hipError_t launch_gate_up_grouped(const GroupedParams &P, int max_items, hipStream_t st, const LaunchTiming *tm) {
    if (max_items <= 0) return hipSuccess;
    if (!P.xbh) return hipErrorInvalidValue;
    if (const hipError_t e = allow_lds(); e != hipSuccess) return e;
    const int per = (max_items + kXcds - 1) / kXcds;
    return launch(gate_up_grouped_kernel, dim3(kXcds * per * (P.rows / 64)), dim3(kGThreads), kGLdsBytes, st, tm, P);
}

hipError_t launch_down_grouped(const GroupedParams &P, int max_items, hipStream_t st, const LaunchTiming *tm) {
    if (max_items <= 0) return hipSuccess;
    if (!P.xbh) return hipErrorInvalidValue;
    if (const hipError_t e = allow_lds(); e != hipSuccess) return e;
    const int per = (max_items + kXcds - 1) / kXcds;
    return launch(down_grouped_kernel, dim3(kXcds * per * (P.rows / 128)), dim3(kGThreads), kGLdsBytes, st, tm, P);
}

hipError_t launch_act_quant(const float *act, int f, int np, const ActBuf &aq, hipStream_t st, const LaunchTiming *tm) {
    if (np <= 0) return hipSuccess;
    if (!aq.bh) return hipErrorInvalidValue;
    return launch(act_quant_kernel, dim3(np), dim3(128), 0, st, tm, act, f, aq.qs, aq.d, aq.bs, aq.bh);
}

}  // namespace lstk
