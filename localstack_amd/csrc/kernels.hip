// kernels.hip - gfx950 (CDNA4) kernels of the Qwen3-MoE expert-FFN path.
//
// A MoE block is four or five launches on the caller's stream, none of which waits on another
// work-group (cross-work-group arrival counters cost ~60 ns of serialized L2 write-back per
// work-group on this part):
//   route     router logits (a wavefront per expert, all tokens of a tile; src/qwen3.cpp:178) and
//             the Q8_0 / Q8_K quantization of hnorm rows, in one grid.
//   topk      (n_tokens > 16) softmax + top-k + renormalisation, a wavefront per token
//             (src/qwen3.cpp:179-189).
//   gate_up   per active expert and row block: gate and up rows held in registers, loaded as
//             coalesced 16-byte chunks before anything else; v_dot4_i32_i8 against the quantized
//             activations of every token routed to the expert; fused SwiGLU (src/qwen3.cpp:201-203).
//             Each work-group derives its expert and token list from the routing itself (for
//             n_tokens <= 16 it also runs the top-k), replacing ggml's mul_mat_id grouping.
//   down      per active expert and 64-row block: the SwiGLU rows re-quantized in LDS, down rows from
//             registers, each pair's output times its router weight (src/qwen3.cpp:204-205).
//   combine   out = resid + sum_j y_j, left to right in the slot index j (src/qwen3.cpp:206-212, :250).
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "device.h"
#include "formats.h"
#include "kernels.h"

namespace lstk {
namespace {

// Experts per wavefront in the router tile: 2 when a work-group serves several tokens (its router
// rows stay in registers over them), 1 for a single token, where twice the work-groups each wait
// on half the rows. A work-group takes 4 EPW experts (4 wavefronts).
constexpr int kRouteEPWMax = 2;
constexpr int kRouteMaxNG = 16;   // n_embd <= 4096: 16 groups of 256 per lane
constexpr int kDnRows = 64;       // rows per down work-group
constexpr int kTC = 8;            // tokens staged per pass
constexpr int kMaxBins = 4096;
constexpr int kMaxPairs = 8192;   // n_batch * n_expert_used
typedef int xvec __attribute__((ext_vector_type(4))); // 16 bytes of int8 activations
constexpr int kDecodeRouteT = 1;  // gate_up runs the top-k itself for a single token
// Threads of a gate_up work-group: single-token (routing) launches use 512 (32 rows per matrix at
// h = 2048; fewer, larger work-groups stream the 8 experts' rows faster on MI355X), batches 256.
#ifndef LSTK_GU_ROUTE_THREADS
#define LSTK_GU_ROUTE_THREADS 512
#endif
constexpr int kGuRouteBlock = LSTK_GU_ROUTE_THREADS;



// ------------------------------------------------------------------------------------------------
// router logits
// ------------------------------------------------------------------------------------------------

// One row's RMSNorm by the kBlock threads of a work-group, in the RMSNorm kernel's order (forward.hip):
// thread i holds x[i + 256 k] for k < NG, sums (double) (x * x) over k, then over the wavefront
// (wave_sum_d) and the four wavefronts as (w0 + w1) + (w2 + w3). Returns the row's
// (x * scale) * w values of this thread.
template <int NG>
__device__ __forceinline__ void norm_row(const float *x, const float *wn, int n, float eps, float (&y)[NG], double *s_part) {
    const int tid = threadIdx.x;
    float v[NG], w[NG];
#pragma unroll
    for (int k = 0; k < NG; k++) {
        v[k] = x[tid + k * kBlock];
        w[k] = wn[tid + k * kBlock];
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NG; k++) s += (double) (v[k] * v[k]);
    s = wave_sum_d(s);
    if ((tid & (kWave - 1)) == 0) s_part[tid / kWave] = s;
    __syncthreads();
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float) (tot / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int k = 0; k < NG; k++) y[k] = (v[k] * scale) * w[k];
}

// Dot products of a tile of tokens with kRouteEG experts. Lane l of a wavefront owns elements
// 256 g + 4 l + q (g ascending, then q) and accumulates them with fmaf from 0; the 64 partials are
// summed by wave_sum_tree. The oracle evaluates the same expression in the same order, so the
// logits agree bit for bit and so does the top-k. F16 weights see fp16-rounded activations, as
// ggml's CPU mul_mat converts src1 to the F16 vec_dot_type (src/qwen3.cpp:178).
// The wavefront's kRouteEPW weight rows are loaded before the activations are staged.
// NR: the staged rows are normalised here from P.x_raw (an instantiation of its own: the extra state
// would cost the plain one registers)
template <int GT, int NG, int kRouteEPW, bool NR>
__device__ __forceinline__ void route_tile(const RouteParams &P, int tile, int eg, float *xs, int tt, int ns, double *s_part) {
    constexpr int kRouteEG = 4 * kRouteEPW;
    constexpr int h = NG * 256;
    constexpr int kPre = 32768 / 16 / kBlock; // float4 of one stage per thread (tt * h * 4 <= 32 KiB)
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    // every load unconditional and unrolled, so all of them are in flight before the first use; F16
    // rows stay packed until the activation loads are issued too (converting them would wait for them)
    uint2 wh[GT == kTypeF16 ? kRouteEPW : 1][NG];
    float w[kRouteEPW][NG][4];
#pragma unroll
    for (int ee = 0; ee < kRouteEPW; ee++) {
        const int e = min(eg * kRouteEG + wave * kRouteEPW + ee, P.E - 1);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const size_t i = (size_t) e * h + 256 * g + 4 * lane;
            if constexpr (GT == kTypeF16) {
                wh[ee][g] = *reinterpret_cast<const uint2 *>(static_cast<const unsigned short *>(P.gate_inp) + i);
            } else {
                const float4 raw = *reinterpret_cast<const float4 *>(static_cast<const float *>(P.gate_inp) + i);
                w[ee][g][0] = raw.x;
                w[ee][g][1] = raw.y;
                w[ee][g][2] = raw.z;
                w[ee][g][3] = raw.w;
            }
        }
    }
    auto unpack = [&] {
        if constexpr (GT == kTypeF16) {
#pragma unroll
            for (int ee = 0; ee < kRouteEPW; ee++)
#pragma unroll
                for (int g = 0; g < NG; g++) {
                    w[ee][g][0] = h2f(wh[ee][g].x);
                    w[ee][g][1] = h2f(wh[ee][g].x >> 16);
                    w[ee][g][2] = h2f(wh[ee][g].y);
                    w[ee][g][3] = h2f(wh[ee][g].y >> 16);
                }
        }
    };
    // the work-group's ns stages of tt tokens: stage s + 1 is loaded into registers while the
    // tokens of stage s are multiplied from LDS
    if (P.x_raw && P.T == 1) {
        // one token, normalised here from the raw row while the router rows stream in
        float y[NG];
        norm_row<NG>(P.x_raw, P.norm_w, h, P.eps, y, s_part);
#pragma unroll
        for (int k = 0; k < NG; k++) xs[threadIdx.x + k * kBlock] = GT == kTypeF16 ? round_f16(y[k]) : y[k];
        unpack();
        __syncthreads();
        float acc[kRouteEPW];
#pragma unroll
        for (int ee = 0; ee < kRouteEPW; ee++) acc[ee] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const float4 x = *reinterpret_cast<const float4 *>(xs + 256 * g + 4 * lane);
#pragma unroll
            for (int ee = 0; ee < kRouteEPW; ee++) {
                acc[ee] = fmaf(x.x, w[ee][g][0], acc[ee]);
                acc[ee] = fmaf(x.y, w[ee][g][1], acc[ee]);
                acc[ee] = fmaf(x.z, w[ee][g][2], acc[ee]);
                acc[ee] = fmaf(x.w, w[ee][g][3], acc[ee]);
            }
        }
#pragma unroll
        for (int ee = 0; ee < kRouteEPW; ee++) {
            const int e = eg * kRouteEG + wave * kRouteEPW + ee;
            const float sum = wave_sum_tree(acc[ee]);
            if (lane == 0 && e < P.E) P.logits[e] = sum;
        }
        return;
    }
    unpack();
    const int tbase = tile * tt * ns;
    // x_raw: the rows are normalised here (ffn_norm), each in the RMSNorm kernel's order (thread i holds
    // x[i + 256 k], sums (double) (x * x) over k, then the wavefront tree and (w0 + w1) + (w2 + w3)),
    // so the staged values equal the RMSNorm kernel's output bit for bit
    constexpr int kR = NR ? (32 / NG < 8 ? 32 / NG : 8) : 1; // rows of a stage held in registers (tt <= kR)
    __shared__ double s_rows[kR][kBlock / kWave];
    float raw[kR][NR ? NG : 1], nwv[NR ? NG : 1];
    float4 pre[NR ? 1 : kPre];
    constexpr bool normed = NR;
    if constexpr (normed) {
#pragma unroll
        for (int k = 0; k < NG; k++) nwv[k] = P.norm_w[threadIdx.x + k * kBlock];
    }
    auto load = [&](int s) {
        const int t0 = tbase + s * tt, nt = max(0, min(tt, P.T - t0));
        if constexpr (normed) {
#pragma unroll
            for (int r = 0; r < kR; r++) {
                const float *src = P.x_raw + (size_t) min(t0 + r, P.T - 1) * h;
#pragma unroll
                for (int k = 0; k < NG; k++) raw[r][k] = src[threadIdx.x + k * kBlock];
            }
        } else {
            const float4 *src = reinterpret_cast<const float4 *>(P.hnorm + (size_t) t0 * h);
#pragma unroll
            for (int u = 0; u < kPre; u++) {
                const int i = threadIdx.x + u * kBlock;
                if (i < nt * h / 4) pre[u] = src[i];
            }
        }
    };
    load(0);
    for (int s = 0; s < ns; s++) {
        const int t0 = tbase + s * tt;
        const int nt = min(tt, P.T - t0);
        if (nt <= 0) break;
        if constexpr (normed) {
#pragma unroll
            for (int r = 0; r < kR; r++) {
                double sm = 0.0;
#pragma unroll
                for (int k = 0; k < NG; k++) sm += (double) (raw[r][k] * raw[r][k]);
                sm = wave_sum_d(sm);
                if (lane == 0) s_rows[r][wave] = sm;
            }
        }
        __syncthreads();
        if constexpr (normed) {
#pragma unroll
            for (int r = 0; r < kR; r++) {
                if (r < nt) {
                    const double tot = (s_rows[r][0] + s_rows[r][1]) + (s_rows[r][2] + s_rows[r][3]);
                    const float mean = (float) (tot / (double) h);
                    const float scale = 1.0f / sqrtf(mean + P.eps);
#pragma unroll
                    for (int k = 0; k < NG; k++) {
                        const float y = (raw[r][k] * scale) * nwv[k];
                        xs[(size_t) r * h + threadIdx.x + k * kBlock] = GT == kTypeF16 ? round_f16(y) : y;
                    }
                }
            }
        } else {
            float4 *dst = reinterpret_cast<float4 *>(xs);
#pragma unroll
            for (int u = 0; u < kPre; u++) {
                const int i = threadIdx.x + u * kBlock;
                if (i < nt * h / 4) {
                    float4 v = pre[u];
                    if (GT == kTypeF16) {
                        v.x = round_f16(v.x);
                        v.y = round_f16(v.y);
                        v.z = round_f16(v.z);
                        v.w = round_f16(v.w);
                    }
                    dst[i] = v;
                }
            }
        }
        __syncthreads();
        if (s + 1 < ns) load(s + 1);
        for (int t = 0; t < nt; t++) {
            float acc[kRouteEPW];
#pragma unroll
            for (int ee = 0; ee < kRouteEPW; ee++) acc[ee] = 0.0f;
#pragma unroll
            for (int g = 0; g < NG; g++) {
                {
                    const float4 x = *reinterpret_cast<const float4 *>(xs + (size_t) t * h + 256 * g + 4 * lane);
#pragma unroll
                    for (int ee = 0; ee < kRouteEPW; ee++) {
                        acc[ee] = fmaf(x.x, w[ee][g][0], acc[ee]);
                        acc[ee] = fmaf(x.y, w[ee][g][1], acc[ee]);
                        acc[ee] = fmaf(x.z, w[ee][g][2], acc[ee]);
                        acc[ee] = fmaf(x.w, w[ee][g][3], acc[ee]);
                    }
                }
            }
#pragma unroll
            for (int ee = 0; ee < kRouteEPW; ee++) {
                const int e = eg * kRouteEG + wave * kRouteEPW + ee;
                const float sum = wave_sum_tree(acc[ee]);
                if (lane == 0 && e < P.E) P.logits[(size_t) (t0 + t) * P.E + e] = sum;
            }
        }
    }
}

template <int GT, int NG, int EPW, bool NR>
// Route work-group b -> (token tile, expert group). xcd_per > 0: XCD-aware, as the dispatcher deals
// work-groups to the 8 XCDs in turn (b goes to XCD b % 8), XCD x takes the tiles [x xcd_per,
// (x + 1) xcd_per), all expert groups of a tile, so a tile's token rows are fetched into one L2 and
// read there by its expert groups (n_route_wg is then 8 xcd_per n_eg; work-groups past the last
// tile have none). xcd_per = 0: tile-major.
__global__ __launch_bounds__(kBlock) void route_kernel(RouteParams P, int n_route_wg, int n_quant_wg, int route_tt, int route_ns,
                                                       int xcd_per) {
    extern __shared__ __align__(16) float lds[];
    __shared__ double s_part[kBlock / kWave];
    const int b = blockIdx.x;
    if (b < n_route_wg) {
        const int n_eg = (P.E + 4 * EPW - 1) / (4 * EPW);
        int tile = b / n_eg, eg = b - tile * n_eg;
        if (xcd_per > 0) {
            const int local = b / 8;
            tile = (b % 8) * xcd_per + local / n_eg;
            eg = local % n_eg;
            if (local / n_eg >= xcd_per || tile * route_tt * route_ns >= P.T) return;
        }
        route_tile<GT, NG, EPW, NR>(P, tile, eg, lds, route_tt, route_ns, s_part);
    } else if (P.qtype != 0) {
        const int h = P.h;
        if (P.x_raw) {
            // this work-group's tokens: each row normalised, quantized from LDS, and stored
            for (int t = b - n_route_wg; t < P.T; t += n_quant_wg) {
                float y[NG];
                norm_row<NG>(P.x_raw + (size_t) t * h, P.norm_w, h, P.eps, y, s_part);
#pragma unroll
                for (int k = 0; k < NG; k++) lds[threadIdx.x + k * kBlock] = y[k];
                __syncthreads();
                if (P.qtype == kTypeQ8_0)
                    quantize_row<kTypeQ8_0>(lds, h, P.xq.qs + (size_t) t * h, P.xq.d + (size_t) t * (h / 32),
                                            P.xq.bs + (size_t) t * (h / 32));
                else
                    quantize_row<kTypeQ4_K>(lds, h, P.xq.qs + (size_t) t * h, P.xq.d + (size_t) t * (h / 32),
                                            P.xq.bs + (size_t) t * (h / 32), P.xq.bh ? P.xq.bh + (size_t) t * (h / 32) : nullptr);
#pragma unroll
                for (int k = 0; k < NG; k++) P.hnorm_out[(size_t) t * h + threadIdx.x + k * kBlock] = y[k];
                __syncthreads(); // the row's LDS and s_part are reused by the next token
            }
            return;
        }
        for (int t = b - n_route_wg; t < P.T; t += n_quant_wg) {
            if (P.qtype == kTypeQ8_0)
                quantize_row<kTypeQ8_0>(P.hnorm + (size_t) t * h, h, P.xq.qs + (size_t) t * h, P.xq.d + (size_t) t * (h / 32),
                                        P.xq.bs + (size_t) t * (h / 32));
            else
                quantize_row<kTypeQ4_K>(P.hnorm + (size_t) t * h, h, P.xq.qs + (size_t) t * h, P.xq.d + (size_t) t * (h / 32),
                                        P.xq.bs + (size_t) t * (h / 32), P.xq.bh ? P.xq.bh + (size_t) t * (h / 32) : nullptr);
        }
    }
}

// TPB tokens per work-group: one per wavefront, or (TPB = 1) one token whose rank counts the four
// wavefronts split.
template <int TPB>
__global__ __launch_bounds__(kBlock) void topk_kernel(TopkParams P) {
    __shared__ __align__(16) unsigned char lds[(kBlock / kWave) * 256 * 4 + (kBlock / kWave) * kMaxEPL * kWave * 4 +
                                               (kBlock / kWave) * kMaxK * 4];
    const int t0 = blockIdx.x * TPB;
    const int nt = min(TPB, P.T - t0);
    topk_block(P.logits + (size_t) t0 * P.E, nt, P.E, P.k, lds, nullptr, P.ids + (size_t) t0 * P.k,
               P.weights + (size_t) t0 * P.k, nullptr, nullptr);
}

// ------------------------------------------------------------------------------------------------
// per-work-group grouping: which expert, which pairs
// ------------------------------------------------------------------------------------------------

// LDS layout of the grouping step, in front of each expert kernel's own LDS.
struct GroupLds {
    unsigned char *scratch; // top-k scratch (route mode), kTopkLds bytes
    int16_t *ids;   // [T*k] bins
    float *w;       // [T*k] router weights (route mode only)
    unsigned *bm;   // [n_bins / 32] bins in use
    int *list;      // [T] this work-group's pairs, ascending
    int *misc;      // [0] = expert or -1, [1] = number of pairs
};

// route mode: the selected probabilities of weights_token, then the experts' 64-bit keys, the
// partial rank counts and the logits of route_one
constexpr size_t kTopkLds = (size_t) kMaxK * 4 + (size_t) kMaxEPL * kWave * 8 + (size_t) kGuRouteBlock * 4 +
                            (size_t) kMaxEPL * kWave * 4;

// The top-k scratch and the weights exist only when the work-group routes (route = 1).
__device__ __host__ inline size_t group_lds_bytes(int T, int k, int n_bins, int route) {
    const size_t np = (size_t) T * k;
    return (route ? kTopkLds + np * 4 : 0) + ((np * 2 + 15) / 16) * 16 + ((size_t) (n_bins + 31) / 32) * 4 +
           (size_t) T * 4 + 64;
}

__device__ __forceinline__ GroupLds group_lds(unsigned char *base, int T, int k, int n_bins, int route) {
    const size_t np = (size_t) T * k;
    GroupLds g{};
    if (route) {
        g.scratch = base;
        base += kTopkLds;
        g.w = reinterpret_cast<float *>(base);
        base += np * 4;
    }
    g.ids = reinterpret_cast<int16_t *>(base);
    base += ((np * 2 + 15) / 16) * 16;
    g.bm = reinterpret_cast<unsigned *>(base);
    base += ((size_t) (n_bins + 31) / 32) * 4;
    g.list = reinterpret_cast<int *>(base);
    base += (size_t) T * 4;
    g.misc = reinterpret_cast<int *>(base);
    return g;
}

// Single-token routing inside an expert work-group (route mode). Every expert e < E gets a unique
// 64-bit key (select_key(logit) << 8 | 255 - e: larger logit first, ties to the lower id) in LDS;
// the work-group's threads count, in parallel, how many keys exceed each expert's key (expert
// t % Ep against a 1 / (NT / Ep) share of the row, Ep = E rounded up to 64), so rank = that count
// is the position in the descending selection order of rank_token / the oracle. Every wavefront then
// takes the block's expert = the y-th expert of rank < k by ascending id, and its pair index
// j = t * k + rank = rank. Wavefront 0 of work-group (0, 0) also runs the softmax and stores ids / weights.
// Returns false when y >= k.
template <int EPL, int NT>
__device__ __forceinline__ bool route_one(const GroupParams &P, GroupLds g) {
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    // nsplit groups of Ep threads each count over `span` keys (even, so the pairs stay 16-byte aligned);
    // all compile-time, so each thread's LDS reads are issued together
    const int E = P.E;
    constexpr int Ep = EPL * kWave, nsplit = NT / Ep, span = ((Ep + nsplit - 1) / nsplit + 1) & ~1;
    unsigned long long *s_key = reinterpret_cast<unsigned long long *>(g.scratch + kMaxK * 4); // [Ep]
    int *s_cnt = reinterpret_cast<int *>(s_key + Ep);                                          // [nsplit][Ep]
    float *s_l = reinterpret_cast<float *>(s_cnt + kGuRouteBlock);                             // [Ep]
    float *s_p = reinterpret_cast<float *>(g.scratch);
    const int e = tid % Ep, part = tid / Ep;
    const float le = P.logits[min(e, E - 1)];
    if (part == 0) {
        s_key[e] = e < E ? ((unsigned long long) select_key(le) << 8) | (unsigned) (255 - e) : 0ull;
        s_l[e] = le;
    }
    __syncthreads();
    if (part < nsplit) {
        const unsigned long long mine = s_key[e];
        const unsigned long long *row = s_key + part * span;
        const int lim = Ep - part * span; // keys of this group: span, or fewer in the last group
        int c = 0;
#pragma unroll
        for (int i = 0; i < span; i += 2) {
            const ulonglong2 v = *reinterpret_cast<const ulonglong2 *>(row + min(i, max(lim - 2, 0)));
            c += i < lim ? (v.x > mine) + (v.y > mine) : 0;
        }
        s_cnt[part * Ep + e] = c;
    }
    __syncthreads();
    // every wavefront makes the (identical) selection itself and keeps it in LDS for its own reads, so no
    // barrier follows
    {
        float l[EPL];
        bool valid[EPL];
        int rank[EPL];
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int ee = lane + kWave * i;
            valid[i] = ee < E;
            l[i] = valid[i] ? s_l[ee] : -INFINITY;
            int r = 0;
            for (int q = 0; q < nsplit; q++) r += s_cnt[q * Ep + ee];
            rank[i] = valid[i] ? r : INT_MAX;
        }
        if (wave == 0 && blockIdx.x == 0 && blockIdx.y == 0)
            weights_token<EPL>(P.k, l, valid, rank, s_p, nullptr, nullptr, nullptr, P.ids_out, P.weights_out);
        const int y = blockIdx.y;
        int ex = -1, j = 0, cum = 0;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            unsigned long long mk = __ballot(valid[i] && rank[i] < P.k);
            const int c = __popcll(mk);
            if (y >= cum && y < cum + c) {
                for (int r = y - cum; r > 0; r--) mk &= mk - 1ull;
                const int src = __ffsll((long long) mk) - 1;
                ex = src + kWave * i;
                j = __builtin_amdgcn_readlane(rank[i], src);
            }
            cum += c;
        }
        if (lane == 0) {
            g.misc[0] = ex;
            g.misc[1] = ex >= 0 ? 1 : 0;
            g.list[0] = j;
        }
        return ex >= 0;
    }
}

// Every work-group derives the same grouping from the same routing: the active bins in ascending
// order (the order ggml's CPU mul_mat_id walks experts), work-group y takes the y-th active bin, and
// its pairs (t, j) in token-major order. Bins out of range are clamped and flagged in *err.
// Returns false when this work-group has no bin (y >= number of active bins).
template <bool ROUTE, int NT = kBlock>
__device__ __forceinline__ bool group_pairs(const GroupParams &P, GroupLds g) {
    const int tid = threadIdx.x, bd = blockDim.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const int k = P.k, np = P.T * k, nb = P.n_bins, nwords = (nb + 31) / 32;
    if (ROUTE) {
        // route mode serves a single token: every wavefront helps rank its row, then the
        // selected experts are a ballot away (ascending id = the work-group order); only
        // work-group (0, 0) runs the softmax and stores ids / weights for the caller and down
        const int epl = (P.E + kWave - 1) / kWave;
        bool ok;
        if (epl == 1) ok = route_one<1, NT>(P, g);
        else if (epl == 2) ok = route_one<2, NT>(P, g);
        else ok = route_one<4, NT>(P, g);
        return ok;
    } else {
        for (int p = tid; p < np; p += bd) {
            int b = P.ids[p];
            if (b < 0 || b >= nb) {
                if (blockIdx.x == 0 && blockIdx.y == 0) atomicOr(P.err, 1);
                b = min(max(b, 0), nb - 1);
            }
            g.ids[p] = (int16_t) b;
        }
    }
    for (int w = tid; w < nwords; w += bd) g.bm[w] = 0u;
    __syncthreads();
    for (int p = tid; p < np; p += bd) {
        const int b = g.ids[p];
        atomicOr(&g.bm[b >> 5], 1u << (b & 31));
    }
    __syncthreads();
    if (wave == 0) {
        // the y-th bin in use, 64 bins per ballot
        const int y = blockIdx.y;
        int e = -1, cum = 0;
        for (int base = 0; base < nb && e < 0; base += kWave) {
            const int b = base + lane;
            const bool used = b < nb && ((g.bm[b >> 5] >> (b & 31)) & 1u);
            unsigned long long mk = __ballot(used);
            const int c = __popcll(mk);
            if (y < cum + c) {
                for (int r = y - cum; r > 0; r--) mk &= mk - 1ull;
                e = base + __ffsll((long long) mk) - 1;
            }
            cum += c;
        }
        int n = 0;
        if (e >= 0) {
            for (int base = 0; base < np; base += kWave) {
                const int p = base + lane;
                const bool hit = p < np && g.ids[p] == e;
                const unsigned long long mk = __ballot(hit);
                const int rank = __popcll(mk & ((1ull << lane) - 1ull));
                if (hit && n + rank < P.T) g.list[n + rank] = p;
                n += __popcll(mk);
            }
            if (n > P.T) {
                if (lane == 0) atomicOr(P.err, 2);
                n = P.T;
            }
        }
        if (lane == 0) {
            g.misc[0] = e;
            g.misc[1] = n;
        }
    }
    __syncthreads();
    return g.misc[0] >= 0;
}

// ------------------------------------------------------------------------------------------------
// gate + up + SwiGLU
// ------------------------------------------------------------------------------------------------

// Work-group (row block, y) of NT threads: rows RW = NT / (2 G) per matrix, thread (g, m, r) holds super-blocks
// g, g + G, ... of row r of gate (m = 0) or up (m = 1) in registers, loaded before anything else.
// The y-th active expert's tokens are staged 8 at a time in LDS; partial dots are reduced over g in
// ascending order, then act[pair] = silu(gate) * up.
template <int WT, int S, bool ROUTE, int NT>
__global__ __launch_bounds__(NT) void gate_up_kernel(GateUpParams P) {
    constexpr int C = chunks_of(WT);
    extern __shared__ __align__(16) unsigned char smem[];
    const int G = P.h / 256 / S;
    const int RW = NT / (2 * G);
    const int tid = threadIdx.x;
    const int r = tid % RW, m = (tid / RW) & 1, g = tid / (2 * RW);
    const int f = P.f, h = P.h, k = P.gp.k;
    const int row = blockIdx.x * RW + r;
    GroupLds gl = group_lds(smem, P.gp.T, k, P.gp.n_bins, ROUTE);
    // offset from the LDS base (no integer round trip, so the accesses stay ds_read / ds_write)
    unsigned char *work = smem + ((group_lds_bytes(P.gp.T, k, P.gp.n_bins, ROUTE) + 15) & ~size_t(15));
    if (!group_pairs<ROUTE, NT>(P.gp, gl)) return;
    const int e = gl.misc[0], cnt = gl.misc[1];
    const uint8_t *base = m ? P.w_up + (size_t) e * P.stride_up : P.w_gate + (size_t) e * P.stride_gate;
    const int h32 = h / 32, h16 = h / 16;
    // The first kXr * blockDim 16-byte pieces of the first chunk's activations are loaded into
    // registers before the weight loads are issued (a single token of up to 8192 values), so the
    // LDS staging below waits for them only; the rest of a chunk is staged from global memory.
    constexpr int kXr = 2;
    const int TC = min(kTC, P.gp.T); // staging slots (a pair per token at most, so a step of T < kTC tokens needs T)
    const int nt0 = min(TC, cnt);
    const int n16 = nt0 * h16, n32 = nt0 * h32;
    const int bd = blockDim.x;
    xvec xr[kXr];
    float dr;
    int br;
#pragma unroll
    for (int u = 0; u < kXr; u++) {
        const int idx = min(tid + u * bd, n16 - 1);
        const int t = gl.list[idx / h16] / k;
        xr[u] = reinterpret_cast<const xvec *>(P.xq.qs + (size_t) t * h)[idx % h16];
    }
    {
        const int idx = min(tid, n32 - 1);
        const size_t o = (size_t) (gl.list[idx / h32] / k) * h32 + idx % h32;
        dr = P.xq.d[o];
        br = WT == kTypeQ4_K ? P.xq.bs[o] : 0;
    }
    uint4 w[S][C];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int sb = g + s * G;
#pragma unroll
        for (int c = 0; c < C; c++) w[s][c] = load_weights(reinterpret_cast<const uint4 *>(base + chunk_offset(C, f, h / 256, sb, c, row)));
    }
    int8_t *xs = reinterpret_cast<int8_t *>(work);
    float *xd = reinterpret_cast<float *>(work + (size_t) TC * h);
    int *xb = reinterpret_cast<int *>(xd + TC * h32);
    float *red = reinterpret_cast<float *>(xb + TC * h32);
#pragma unroll
    for (int u = 0; u < kXr; u++) {
        const int idx = tid + u * bd;
        if (idx < n16) reinterpret_cast<xvec *>(xs)[idx] = xr[u];
    }
    for (int idx = tid + kXr * bd; idx < n16; idx += bd)
        reinterpret_cast<xvec *>(xs)[idx] = reinterpret_cast<const xvec *>(P.xq.qs + (size_t) (gl.list[idx / h16] / k) * h)[idx % h16];
    if (tid < n32) {
        xd[tid] = dr;
        if (WT == kTypeQ4_K) xb[tid] = br;
    }
    for (int idx = tid + bd; idx < n32; idx += bd) {
        const size_t o = (size_t) (gl.list[idx / h32] / k) * h32 + idx % h32;
        xd[idx] = P.xq.d[o];
        if (WT == kTypeQ4_K) xb[idx] = P.xq.bs[o];
    }
    if constexpr (ROUTE) {
        // one token (cnt == 1): straight-line code, the super-blocks one after the other (in the
        // chunk loop below the compiler unpacks every super-block's nibbles ahead of the loop,
        // which at two super-blocks per thread holds the work-group to two wavefronts per SIMD)
        __syncthreads();
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int sb = g + s * G;
            acc = dot_sb<WT>(w[s], xs + sb * 256, xd + sb * 8, xb + sb * 8, acc);
            __builtin_amdgcn_sched_barrier(0);
        }
        red[(g * 2 + m) * RW + r] = acc;
        __syncthreads();
        if (tid < RW) {
            float gs = red[r], us = red[RW + r];
            for (int gg = 1; gg < G; gg++) {
                gs += red[(gg * 2) * RW + r];
                us += red[(gg * 2 + 1) * RW + r];
            }
            const float a = (gs / (1.0f + expf(-gs))) * us;
            P.act[(size_t) gl.list[0] * f + blockIdx.x * RW + r] = a;
        }
        return;
    }
    for (int c0 = 0; c0 < cnt; c0 += TC) {
        const int nt = min(TC, cnt - c0);
        if (c0 > 0) { // later chunks (more than 8 tokens on one expert) are staged here
            for (int tc = 0; tc < nt; tc++) {
                const int t = gl.list[c0 + tc] / k;
                const int4 *src = reinterpret_cast<const int4 *>(P.xq.qs + (size_t) t * h);
                int4 *dst = reinterpret_cast<int4 *>(xs + (size_t) tc * h);
                for (int i = tid; i < h16; i += blockDim.x) dst[i] = src[i];
                for (int i = tid; i < h32; i += blockDim.x) {
                    xd[tc * h32 + i] = P.xq.d[(size_t) t * h32 + i];
                    if (WT == kTypeQ4_K) xb[tc * h32 + i] = P.xq.bs[(size_t) t * h32 + i];
                }
            }
        }
        __syncthreads();
        for (int tc = 0; tc < nt; tc++) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int sb = g + s * G;
                // Q8_0: 132 -> 107 VGPRs, four wavefronts per SIMD instead of three (the 48-layer Q8_0
                // stack at T = 8 1.1% faster); the Q4_K kernels are faster with their unpacked weights
                // held across tokens (at T = 32, 2.3 tokens per expert, re-unpacking cost 3%)
                if constexpr (WT == kTypeQ8_0) rederive(w[s]);
                acc = dot_sb<WT>(w[s], xs + (size_t) tc * h + sb * 256, xd + tc * h32 + sb * 8, xb + tc * h32 + sb * 8, acc);
            }
            red[((tc * G + g) * 2 + m) * RW + r] = acc;
        }
        __syncthreads();
        for (int idx = tid; idx < nt * RW; idx += blockDim.x) {
            const int tc = idx / RW, rr = idx % RW;
            float gv[kMaxG], uv[kMaxG];
#pragma unroll
            for (int gg = 0; gg < kMaxG; gg++) {
                gv[gg] = gg < G ? red[((tc * G + gg) * 2 + 0) * RW + rr] : 0.0f;
                uv[gg] = gg < G ? red[((tc * G + gg) * 2 + 1) * RW + rr] : 0.0f;
            }
            float gs = gv[0], us = uv[0];
#pragma unroll
            for (int gg = 1; gg < kMaxG; gg++) {
                if (gg < G) {
                    gs += gv[gg];
                    us += uv[gg];
                }
            }
            const float a = (gs / (1.0f + expf(-gs))) * us;
            P.act[(size_t) gl.list[c0 + tc] * f + blockIdx.x * RW + rr] = a;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// down + router weight
// ------------------------------------------------------------------------------------------------

template <int WT, int S>
__global__ __launch_bounds__(kDnRows * kMaxG) void down_kernel(DownParams P) {
    constexpr int C = chunks_of(WT);
    constexpr int QT = WT == kTypeQ8_0 ? kTypeQ8_0 : kTypeQ4_K; // Q8_K activations for every k-quant
    extern __shared__ __align__(16) unsigned char smem[];
    const int G = blockDim.x / kDnRows;
    const int tid = threadIdx.x, r = tid % kDnRows, g = tid / kDnRows;
    const int h = P.h, f = P.f;
    const int row = blockIdx.x * kDnRows + r;
    GroupLds gl = group_lds(smem, P.gp.T, P.gp.k, P.gp.n_bins, 0);
    unsigned char *work = smem + ((group_lds_bytes(P.gp.T, P.gp.k, P.gp.n_bins, 0) + 15) & ~size_t(15));
    if (!group_pairs<false>(P.gp, gl)) return;
    const int e = gl.misc[0], cnt = gl.misc[1];
    const uint8_t *base = P.w_down + (size_t) e * P.stride_down;
    uint4 w[S][C];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int sb = g + s * G;
#pragma unroll
        for (int c = 0; c < C; c++) w[s][c] = load_weights(reinterpret_cast<const uint4 *>(base + chunk_offset(C, h, f / 256, sb, c, row)));
    }
    const int f32 = f / 32;
    int8_t *xs = reinterpret_cast<int8_t *>(work);
    float *xd = reinterpret_cast<float *>(work + (size_t) kTC * f);
    int *xb = reinterpret_cast<int *>(xd + kTC * f32);
    float *red = reinterpret_cast<float *>(xb + kTC * f32);
    // A chunk's nt SwiGLU rows are quantized as one array of nt * f values (f a multiple of 256, so each
    // 256-value block lies in one row, as quantizing row by row takes it), NG passes of 8 values per
    // thread at a time with every load of the NG passes issued before the first is quantized: one memory
    // round trip per NG passes instead of one per pair. blockDim = 64 G threads, G = f / 256 / S, take
    // 2 f / S values per pass, so kTC rows take NP = 4 S passes.
    constexpr int NP = kTC / 2 * S, NG = 2;
    const int bd = blockDim.x;
    for (int c0 = 0; c0 < cnt; c0 += kTC) {
        const int nt = min(kTC, cnt - c0), n = nt * f;
#pragma unroll 1
        for (int p0 = 0; p0 < NP; p0 += NG) {
            if (p0 * bd * 8 >= n) break; // the same for every thread
            float v[NG][8];
#pragma unroll
            for (int p = 0; p < NG; p++) {
                const int i0 = ((p0 + p) * bd + tid) * 8, ia = min(i0, n - 8);
                const float *x = P.act + (size_t) gl.list[c0 + ia / f] * f + ia % f;
                const float4 a = *reinterpret_cast<const float4 *>(x);
                const float4 b = *reinterpret_cast<const float4 *>(x + 4);
                const bool in = i0 < n;
                v[p][0] = in ? a.x : 0.0f; v[p][1] = in ? a.y : 0.0f; v[p][2] = in ? a.z : 0.0f; v[p][3] = in ? a.w : 0.0f;
                v[p][4] = in ? b.x : 0.0f; v[p][5] = in ? b.y : 0.0f; v[p][6] = in ? b.z : 0.0f; v[p][7] = in ? b.w : 0.0f;
            }
#pragma unroll
            for (int p = 0; p < NG; p++) {
                const int i0 = ((p0 + p) * bd + tid) * 8;
                if ((p0 + p) * bd * 8 < n) quantize8<QT>(v[p], i0, i0 < n, xs, xd, xb);
            }
        }
        __syncthreads();
        for (int tc = 0; tc < nt; tc++) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int sb = g + s * G;
                acc = dot_sb<WT>(w[s], xs + (size_t) tc * f + sb * 256, xd + tc * f32 + sb * 8, xb + tc * f32 + sb * 8, acc);
            }
            red[(tc * G + g) * kDnRows + r] = acc;
        }
        __syncthreads();
        for (int idx = tid; idx < nt * kDnRows; idx += blockDim.x) {
            const int tc = idx / kDnRows, rr = idx % kDnRows;
            float dv[kMaxG];
#pragma unroll
            for (int gg = 0; gg < kMaxG; gg++) dv[gg] = gg < G ? red[(tc * G + gg) * kDnRows + rr] : 0.0f;
            float ds = dv[0];
#pragma unroll
            for (int gg = 1; gg < kMaxG; gg++)
                if (gg < G) ds += dv[gg];
            const int p = gl.list[c0 + tc];
            P.Y[(size_t) p * h + blockIdx.x * kDnRows + rr] = ds * P.weights[p];
        }
        __syncthreads();
    }
    (void) row;
}

// ------------------------------------------------------------------------------------------------
// down + router weight + combine + residual of a single token
// ------------------------------------------------------------------------------------------------

constexpr int kDcMaxAct = 16384; // k * f SwiGLU values quantized in a work-group's LDS

// Q8_K quantization (quantize_row_q8_K_ref) of one 256-value block by `lanes` consecutive lanes of a
// wavefront, lane r holding values [r VPT, (r + 1) VPT) of the block in v: the first largest |x| of
// the block (ties to the lower index) by a shuffle reduction over the lanes, iscale = -127 / max,
// q = min(127, rne(iscale x)), d = 1 / iscale. Writes the block's qs (at qs), its scale into each of
// the 8 per-32 slots d8[0..8) and the per-32 sums of q into bs8[0..8).
template <int VPT>
__device__ __forceinline__ void q8k_block_lanes(const float (&v)[VPT], int lanes, int r, int8_t *qs, float *d8,
                                                int *bs8) {
    float amax = 0.0f, mx = 0.0f;
    int idx = INT_MAX;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const float ax = fabsf(v[i]);
        if (ax > amax) {
            amax = ax;
            mx = v[i];
            idx = r * VPT + i;
        }
    }
    for (int o = 1; o < lanes; o <<= 1) {
        const float oa = __shfl_xor(amax, o), om = __shfl_xor(mx, o);
        const int oi = __shfl_xor(idx, o);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            mx = om;
            idx = oi;
        }
    }
    int q[VPT];
    float dd = 0.0f;
    if (amax == 0.0f) {
#pragma unroll
        for (int i = 0; i < VPT; i++) q[i] = 0;
    } else {
        const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int i = 0; i < VPT; i++) q[i] = min(127, (int) rintf(iscale * v[i]));
        dd = __fdiv_rn(1.0f, iscale);
    }
#pragma unroll
    for (int w4 = 0; w4 < VPT / 4; w4++) {
        const unsigned word = ((unsigned) q[4 * w4] & 0xffu) | (((unsigned) q[4 * w4 + 1] & 0xffu) << 8) |
                              (((unsigned) q[4 * w4 + 2] & 0xffu) << 16) | (((unsigned) q[4 * w4 + 3] & 0xffu) << 24);
        reinterpret_cast<unsigned *>(qs + r * VPT)[w4] = word;
    }
    if (VPT >= 32) {
#pragma unroll
        for (int g = 0; g < VPT / 32; g++) {
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 32; i++) sum += q[32 * g + i];
            bs8[r * (VPT / 32) + g] = sum;
            d8[r * (VPT / 32) + g] = dd;
        }
    } else {
        int sum = 0;
#pragma unroll
        for (int i = 0; i < VPT; i++) sum += q[i];
        for (int o = 1; o < 32 / VPT; o <<= 1) sum += __shfl_xor(sum, o);
        if (r % (32 / VPT) == 0) {
            bs8[r / (32 / VPT)] = sum;
            d8[r / (32 / VPT)] = dd;
        }
    }
}

// Thread (q, rr) with q = j * nsbf + sb holds super-block sb of row blockIdx.x * rd + rr of pair j's
// down matrix. The pair's slot and the token's k SwiGLU rows are loaded first (one round trip), the
// weight loads are issued as soon as the slot is known, and the SwiGLU rows are quantized into LDS
// while the weights stream in. Each thread's partial dot lands in LDS,
// and threads rr < rd sum, per pair j in ascending order, the partials over sb ascending (the
// order of down_kernel), multiply by the router weight and add the pairs left to right in j, then
// the residual (the order of combine_kernel), so the result equals down + combine bit for bit.
// SEG > 0 (Q8_K activations with k * nsbf * rd0 threads exactly): the rd0 threads of pair j and
// super-block sb quantize that 256-value Q8_K block together, SEG = 256 / rd0 values each, in one
// pass (q8k_block_lanes); otherwise every thread takes NP passes of 8 values (quantize_row).
template <int WT, int NP, int R, int SEG, int NT = kBlock>
__global__ __launch_bounds__(NT) void down_combine_kernel(DownCombineParams P, int rd0) {
    constexpr int C = chunks_of(WT);
    constexpr int QT = WT == kTypeQ8_0 ? kTypeQ8_0 : kTypeQ4_K; // Q8_K activations for every k-quant
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, k = P.k, f = P.f, nsbf = f / 256, nact = k * f;
    // R rows per thread: local row ir * rd0 + rr of the work-group's rd = R * rd0 rows
    const int rd = R * rd0;
    const int rr = tid % rd0, q = tid / rd0, sb = q % nsbf, j = q / nsbf;
    const bool on = j < k;
    int8_t *qs = reinterpret_cast<int8_t *>(smem);
    float *qd = reinterpret_cast<float *>(smem + nact);
    int *qb = reinterpret_cast<int *>(qd + nact / 32);
    float *part = reinterpret_cast<float *>(qb + nact / 32);
    float *s_w = part + (size_t) k * nsbf * rd;
    // unconditional loads (indexes clamped), so the weight loads follow without a branch
    int b = P.ids[min(j, k - 1)];
    const float wj = P.weights[min(tid, k - 1)];
    const float resid = P.resid[blockIdx.x * rd + min(tid, rd - 1)]; // the residual of output row tid (tid < rd)
    // Q8_0 activations: NP whole 32-value blocks per thread (one amax and one pair of divisions per
    // block); Q8_K: NP passes of 8 values per thread (32 threads per 256-value block)
    constexpr int NV = QT == kTypeQ8_0 ? 32 : 8;
    float v[NP][NV];
    float vs[SEG > 0 ? SEG : 1];
    if constexpr (SEG > 0) {
        const float4 *src = reinterpret_cast<const float4 *>(P.act + (size_t) min(q, nact / 256 - 1) * 256 + rr * SEG);
#pragma unroll
        for (int i = 0; i < SEG / 4; i++) {
            const float4 a = src[i];
            vs[4 * i] = a.x;
            vs[4 * i + 1] = a.y;
            vs[4 * i + 2] = a.z;
            vs[4 * i + 3] = a.w;
        }
    } else if constexpr (QT == kTypeQ8_0) {
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int blk = min(tid + u * (int) blockDim.x, nact / 32 - 1);
#pragma unroll
            for (int q4 = 0; q4 < 8; q4++) {
                const float4 a = *reinterpret_cast<const float4 *>(P.act + (size_t) blk * 32 + 4 * q4);
                v[u][4 * q4] = a.x;
                v[u][4 * q4 + 1] = a.y;
                v[u][4 * q4 + 2] = a.z;
                v[u][4 * q4 + 3] = a.w;
            }
        }
    } else {
        quantize_row_load<NP>(P.act, nact, v);
    }
    if (b < 0 || b >= P.n_bins) {
        if (on && blockIdx.x == 0 && rr == 0 && sb == 0) atomicOr(P.err, 1);
        b = min(max(b, 0), P.n_bins - 1);
    }
    const uint8_t *base = P.w_down + (size_t) b * P.stride_down;
    uint4 w[R][C];
#pragma unroll
    for (int ir = 0; ir < R; ir++) {
        const int row = blockIdx.x * rd + ir * rd0 + rr;
#pragma unroll
        for (int c = 0; c < C; c++) w[ir][c] = load_weights(reinterpret_cast<const uint4 *>(base + chunk_offset(C, P.h, f / 256, on ? sb : 0, c, row)));
    }
    if constexpr (SEG > 0) {
        q8k_block_lanes<SEG>(vs, rd0, rr, qs + (size_t) q * 256, qd + (size_t) q * 8, qb + (size_t) q * 8);
    } else if constexpr (QT == kTypeQ8_0) {
        // quantize_row_q8_0 (x86 path): d = amax / 127 stored as fp16, q = rne(x * 127 / amax)
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int blk = tid + u * (int) blockDim.x;
            if (blk < nact / 32) {
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[u][i]));
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                unsigned pk[8];
#pragma unroll
                for (int w4 = 0; w4 < 8; w4++) {
                    unsigned word = 0;
#pragma unroll
                    for (int bb = 0; bb < 4; bb++) word |= ((unsigned) (int) rintf(v[u][4 * w4 + bb] * id) & 0xffu) << (8 * bb);
                    pk[w4] = word;
                }
                uint4 *dst = reinterpret_cast<uint4 *>(qs + (size_t) blk * 32);
                dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
                qd[blk] = round_f16(__fdiv_rn(amax, 127.0f));
            }
        }
    } else {
        quantize_row_store<QT, NP>(v, nact, qs, qd, qb);
    }
    if (tid < k) s_w[tid] = wj;
    __syncthreads();
    if (on) {
        const int o = j * f + sb * 256;
#pragma unroll
        for (int ir = 0; ir < R; ir++)
            part[(j * rd + ir * rd0 + rr) * nsbf + sb] = dot_sb<WT>(w[ir], qs + o, qd + o / 32, qb + o / 32, 0.0f);
    }
    __syncthreads();
    // slot j's output of row r: its super-blocks summed left to right, times the router weight
    // (item j * rd + r)
    float *ys = s_w + k;
    for (int i = tid; i < k * rd; i += blockDim.x) {
        const int jj = i / rd, r2 = i - jj * rd;
        const float *pp = part + (jj * rd + r2) * nsbf;
        constexpr int kDcSb = 8;
        float pv[kDcSb];
#pragma unroll
        for (int s2 = 0; s2 < kDcSb; s2++) pv[s2] = pp[min(s2, nsbf - 1)];
        float ds = pv[0];
#pragma unroll
        for (int s2 = 1; s2 < kDcSb; s2++) ds = s2 < nsbf ? ds + pv[s2] : ds;
        for (int s2 = kDcSb; s2 < nsbf; s2++) ds += pp[s2];
        ys[i] = ds * s_w[jj];
    }
    __syncthreads();
    if (tid < rd) {
        // the k-way sum in slot order, every LDS read of a batch of 8 slots issued before the sums
        float acc = 0.0f;
        for (int jj0 = 0; jj0 < k; jj0 += 8) {
            float yv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) yv[u] = ys[min(jj0 + u, k - 1) * rd + tid];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int jj = jj0 + u;
                acc = jj < k ? (jj == 0 ? yv[u] : acc + yv[u]) : acc;
            }
        }
        P.out[blockIdx.x * rd + tid] = acc + resid;
    }
}

// ------------------------------------------------------------------------------------------------
// combine + residual
// ------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void combine_kernel(CombineParams P) {
    const int h4 = P.h / 4;
    const int idx = blockIdx.x * kBlock + threadIdx.x;
    if (idx >= P.T * h4) return;
    const int t = idx / h4, c = idx - t * h4;
    const float4 *y = reinterpret_cast<const float4 *>(P.Y) + (size_t) t * P.k * h4 + c;
    const float4 rs = reinterpret_cast<const float4 *>(P.resid)[idx];
    float4 acc = y[0];
    // slots in batches of 8 loads issued together, summed left to right
    for (int j0 = 1; j0 < P.k; j0 += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = y[(size_t) min(j0 + u, P.k - 1) * h4];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (j0 + u < P.k) {
                acc.x = acc.x + v[u].x;
                acc.y = acc.y + v[u].y;
                acc.z = acc.z + v[u].z;
                acc.w = acc.w + v[u].w;
            }
        }
    }
    acc.x = acc.x + rs.x;
    acc.y = acc.y + rs.y;
    acc.z = acc.z + rs.z;
    acc.w = acc.w + rs.w;
    reinterpret_cast<float4 *>(P.out)[idx] = acc;
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------


int route_tile_tokens(int h) { return std::max(1, std::min(8, 32768 / (h * 4))); }

size_t align16(size_t x) { return (x + 15) / 16 * 16; }

template <int GT, int NG>
hipError_t launch_route_t(const RouteParams &P, hipStream_t st, const LaunchTiming *tm) {
    // the in-launch normalisation needs the quantizing work-groups to store the rows
    if (P.x_raw && (!P.norm_w || !P.hnorm_out || !P.qtype)) return hipErrorInvalidValue;
    int n_route = 0, tt = 1, ns = 1, xcd_per = 0;
    const int epw = P.T == 1 ? 1 : kRouteEPWMax;
    if (P.do_route) {
        tt = route_tile_tokens(P.h);
        // many tokens: each work-group keeps its router rows in registers over 4 stages of tokens
        ns = P.T > 8 * tt ? 4 : 1;
        const int n_tile = (P.T + tt * ns - 1) / (tt * ns), n_eg = (P.E + 4 * epw - 1) / (4 * epw);
        n_route = n_tile * n_eg;
        // at least a tile per XCD: each tile's expert groups on the XCD whose L2 holds its rows
        if (n_tile >= 8) {
            xcd_per = (n_tile + 7) / 8;
            n_route = 8 * xcd_per * n_eg;
        }
    }
    const int n_quant = P.qtype ? std::min(P.T, 256) : 0;
    const int grid = std::max(1, n_route + n_quant);
    // (a single token's row is staged in LDS by the quantizing work-group too)
    const size_t lds = std::max(P.do_route ? (size_t) tt * P.h * 4 : (size_t) 16, P.x_raw ? (size_t) P.h * 4 : (size_t) 16);
    if (epw == 1) return launch(route_kernel<GT, NG, 1, false>, dim3(grid), dim3(kBlock), lds, st, tm, P, n_route, n_quant, tt, ns, xcd_per);
    if (P.x_raw)
        return launch(route_kernel<GT, NG, kRouteEPWMax, true>, dim3(grid), dim3(kBlock), lds, st, tm, P, n_route, n_quant, tt, ns, xcd_per);
    return launch(route_kernel<GT, NG, kRouteEPWMax, false>, dim3(grid), dim3(kBlock), lds, st, tm, P, n_route, n_quant, tt, ns, xcd_per);
}

template <int GT>
hipError_t launch_route_g(const RouteParams &P, hipStream_t st, const LaunchTiming *tm) {
    switch (P.h / 256) {
        case 1: return launch_route_t<GT, 1>(P, st, tm);
        case 2: return launch_route_t<GT, 2>(P, st, tm);
        case 4: return launch_route_t<GT, 4>(P, st, tm);
        case 8: return launch_route_t<GT, 8>(P, st, tm);
        case 12: return launch_route_t<GT, 12>(P, st, tm);
        default: return launch_route_t<GT, 16>(P, st, tm);
    }
}

// Dynamic LDS of a gate_up launch: grouping, min(kTC, T) staged tokens and the partial sums of RW rows.
// (A single token's launch at h 4096 then takes 12 KB instead of 55 KB, so its 768 work-groups are
// resident at once instead of in two rounds.)
size_t gate_up_lds(int T, int k, int n_bins, int route, int h, int G, int RW) {
    const size_t tc = (size_t) std::min(kTC, T);
    return align16(group_lds_bytes(T, k, n_bins, route)) + 16 + tc * h + 2 * tc * (h / 32) * 4 + tc * G * 2 * RW * 4;
}

template <int WT, int S>
hipError_t launch_gate_up_t(const GateUpParams &P, int G, hipStream_t st, const LaunchTiming *tm) {
    // One token: 512-thread work-groups (twice the rows each) where rows are short. Measured on MI355X:
    // at h 2048 (30B) routed 9.9 us against 10.95 with 256 threads; at h 4096 (235B) 256 threads are
    // faster, routed 21.5 against 21.8 us and on caller-given slots 17.3 against 19.7 us.
    const bool wide = P.h <= 2048;
    if (P.gp.route || P.gp.T == 1) {
        const bool route = P.gp.route != 0;
        const int nt = wide ? kGuRouteBlock : kBlock;
        const int RW = nt / (2 * G);
        const size_t lds = gate_up_lds(route ? P.gp.T : 1, P.gp.k, P.gp.n_bins, route ? 1 : 0, P.h, G, RW);
        const dim3 grid(P.f / RW, P.max_active), block(nt);
        if (route)
            return wide ? launch(gate_up_kernel<WT, S, true, kGuRouteBlock>, grid, block, lds, st, tm, P)
                        : launch(gate_up_kernel<WT, S, true, kBlock>, grid, block, lds, st, tm, P);
        return wide ? launch(gate_up_kernel<WT, S, false, kGuRouteBlock>, grid, block, lds, st, tm, P)
                    : launch(gate_up_kernel<WT, S, false, kBlock>, grid, block, lds, st, tm, P);
    }
    const int RW = kBlock / (2 * G);
    const size_t lds = gate_up_lds(P.gp.T, P.gp.k, P.gp.n_bins, 0, P.h, G, RW);
    return launch(gate_up_kernel<WT, S, false, kBlock>, dim3(P.f / RW, P.max_active), dim3(kBlock), lds, st, tm, P);
}

template <int WT, int S>
hipError_t launch_down_t(const DownParams &P, int G, hipStream_t st, const LaunchTiming *tm) {
    const int f32 = P.f / 32;
    const size_t lds = align16(group_lds_bytes(P.gp.T, P.gp.k, P.gp.n_bins, 0)) + 16 + (size_t) kTC * P.f +
                       (size_t) 2 * kTC * f32 * 4 + (size_t) kTC * G * kDnRows * 4;
    return launch(down_kernel<WT, S>, dim3(P.h / kDnRows, P.max_active), dim3(kDnRows * G), lds, st, tm, P);
}

// Row stride of a down_combine work-group: the largest power of two rd0 with k * nsbf * rd0 <= 256
// threads.
int down_combine_rows(int f, int k) {
    const int per = k * (f / 256);
    int rd = 1;
    while (rd * 2 * per <= kBlock) rd *= 2;
    return rd;
}

// k-quant experts (one Q8_K block per (pair, super-block) and rd0 threads): the row stride doubled,
// up to 16 rows and kDcMaxThreads threads, while the grid keeps 256 work-groups at one row per
// thread. At the 235B shape that is 8 x 6 x 16 = 768 threads of one row each instead of 192 of four,
// so the work-group's quantization and dot products spread over four times the wavefronts.
constexpr int kDcMaxThreads = 1024;
int down_combine_rows_wide(int h, int f, int k) {
    const int per = k * (f / 256);
    int rd = down_combine_rows(f, k);
    while (rd < 16 && rd * 2 * per <= kDcMaxThreads && h % (rd * 2) == 0 && h / (rd * 2) >= 256) rd *= 2;
    return rd;
}

// Rows per thread: up to 4 (Q4_K) or 2 (Q8_0) while the grid keeps at least 256 work-groups, so a
// wide layer does not quantize the token's SwiGLU rows in more work-groups than the device has CUs.
int down_combine_rows_per_thread(int type, int h, int rd0) {
    const int rmax = type == kTypeQ4_K ? 4 : 2;
    int r = 1;
    while (r < rmax && h % (rd0 * r * 2) == 0 && h / (rd0 * r * 2) >= 256) r *= 2;
    return r;
}

template <int WT, int R>
hipError_t launch_down_combine_r(const DownCombineParams &P, int rd0, int np, size_t lds, int threads, hipStream_t st,
                                 const LaunchTiming *tm) {
    const dim3 grid(P.h / (rd0 * R)), block(threads);
    if (threads > kBlock) {
        // past 256 threads: k-quants, one row per thread, rd0 threads per (pair, super-block) block
        if constexpr (WT != kTypeQ8_0 && R == 1) {
            if (threads == P.k * (P.f / 256) * rd0) {
                if (rd0 == 8) return launch(down_combine_kernel<WT, 1, 1, 32, kDcMaxThreads>, grid, block, lds, st, tm, P, rd0);
                if (rd0 == 16) return launch(down_combine_kernel<WT, 1, 1, 16, kDcMaxThreads>, grid, block, lds, st, tm, P, rd0);
            }
        }
        return hipErrorInvalidValue;
    }
    if (WT != kTypeQ8_0 && threads == P.k * (P.f / 256) * rd0) {
        // one Q8_K block per (pair, super-block), quantized by that combination's rd0 threads
        switch (rd0) {
            case 4: return launch(down_combine_kernel<WT, 1, R, 64>, grid, block, lds, st, tm, P, rd0);
            case 8: return launch(down_combine_kernel<WT, 1, R, 32>, grid, block, lds, st, tm, P, rd0);
            case 16: return launch(down_combine_kernel<WT, 1, R, 16>, grid, block, lds, st, tm, P, rd0);
            case 32: return launch(down_combine_kernel<WT, 1, R, 8>, grid, block, lds, st, tm, P, rd0);
            default: break;
        }
    }
    if (np <= 1) return launch(down_combine_kernel<WT, 1, R, 0>, grid, block, lds, st, tm, P, rd0);
    if (np <= 2) return launch(down_combine_kernel<WT, 2, R, 0>, grid, block, lds, st, tm, P, rd0);
    if (np <= 4) return launch(down_combine_kernel<WT, 4, R, 0>, grid, block, lds, st, tm, P, rd0);
    return launch(down_combine_kernel<WT, 8, R, 0>, grid, block, lds, st, tm, P, rd0);
}

template <int WT>
hipError_t launch_down_combine_t(const DownCombineParams &P, hipStream_t st, const LaunchTiming *tm) {
    int rd0 = down_combine_rows(P.f, P.k), R = down_combine_rows_per_thread(WT, P.h, rd0);
    if (WT != kTypeQ8_0) {
        const int wide = down_combine_rows_wide(P.h, P.f, P.k);
        if (wide > rd0 && down_combine_rows_per_thread(WT, P.h, wide) == 1) {
            rd0 = wide;
            R = 1;
        }
    }
    const int nsbf = P.f / 256, nact = P.k * P.f;
    const int threads = (P.k * nsbf * rd0 + kWave - 1) / kWave * kWave;
    const size_t lds = (size_t) nact + (size_t) nact / 32 * 8 + (size_t) P.k * nsbf * rd0 * R * 4 + (size_t) P.k * 4 +
                       (size_t) P.k * rd0 * R * 4;
    // Q8_0: whole 32-value blocks per thread; Q8_K: passes of 8 values per thread
    const int per = WT != kTypeQ8_0 ? threads * 8 : threads * 32;
    const int np = (nact + per - 1) / per;
    if (R == 4) return launch_down_combine_r<WT, 4>(P, rd0, np, lds, threads, st, tm);
    if (R == 2) return launch_down_combine_r<WT, 2>(P, rd0, np, lds, threads, st, tm);
    return launch_down_combine_r<WT, 1>(P, rd0, np, lds, threads, st, tm);
}

}  // namespace

bool down_combine_supported(int h, int f, int k) {
    if (k < 1 || k > kMaxK || f % 256 != 0 || h % 256 != 0 || (long) k * f > kDcMaxAct) return false;
    if (k * (f / 256) > kBlock) return false;
    const int rd = down_combine_rows(f, k);
    const int threads = (k * (f / 256) * rd + kWave - 1) / kWave * kWave;
    return h % rd == 0 && (long) k * f <= 8L * threads * 8; // at most 8 passes (or blocks) per thread
}

hipError_t launch_down_combine(const DownCombineParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (!down_combine_supported(P.h, P.f, P.k)) return hipErrorInvalidValue;
    switch (pool_format(P.type)) {
        case kTypeQ8_0: return launch_down_combine_t<kTypeQ8_0>(P, st, tm);
        case kTypeKQ8: return launch_down_combine_t<kTypeKQ8>(P, st, tm);
        default: return launch_down_combine_t<kTypeQ4_K>(P, st, tm);
    }
}

int decode_route_max_tokens() { return kDecodeRouteT; }

const char *check_shapes(int h, int f, int E, int k, int n_bins, int n_batch) {
    int S, G;
    if (h <= 0 || h % 256 != 0) return "n_embd must be a positive multiple of 256";
    if (h > 256 * kRouteMaxNG) return "n_embd above 4096 is not supported by the router kernel";
    {
        const int ng = h / 256;
        if (ng != 1 && ng != 2 && ng != 4 && ng != 8 && ng != 12 && ng != 16)
            return "n_embd must be 256, 512, 1024, 2048, 3072 or 4096";
    }
    if (f <= 0 || f % 256 != 0) return "n_ff_exp must be a positive multiple of 256";
    if (E < 1 || E > kWave * kMaxEPL) return "n_expert must be in [1, 256]";
    if (k < 1 || k > E || k > kMaxK) return "n_expert_used must be in [1, min(n_expert, 64)]";
    if (n_bins < 1 || n_bins > kMaxBins) return "slot count must be in [1, 4096]";
    if (n_batch < 1 || (long) n_batch * k > kMaxPairs) return "n_batch * n_expert_used must be in [1, 8192]";
    if (!pick_split_gate_up(h / 256, &S, &G)) return "n_embd / 256 must split into 1, 2, 4 or 8 groups of <= 2 super-blocks";
    if (!pick_split(f / 256, &S, &G)) return "n_ff_exp / 256 has no split into <= 8 groups of <= 2 super-blocks";
    pick_split_gate_up(h / 256, &S, &G);
    if (f % (kGuRouteBlock / (2 * G)) != 0 || f % (kBlock / (2 * G)) != 0)
        return "n_ff_exp must be a multiple of the gate/up row block";
    // LDS: grouping + staging must fit in 64 KiB
    const size_t gu_route = gate_up_lds(std::min(n_batch, kDecodeRouteT), k, n_bins, 1, h, G, kGuRouteBlock / (2 * G));
    const size_t gu = gate_up_lds(n_batch, k, n_bins, 0, h, G, kBlock / (2 * G));
    if (gu > 65536 || gu_route > 65536) return "n_batch * n_expert_used too large for the gate/up work-group's LDS";
    return "";
}

hipError_t launch_route(const RouteParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T <= 0) return hipSuccess;
    const int gt = P.do_route ? P.gate_type : kTypeF16;
    return gt == kTypeF16 ? launch_route_g<kTypeF16>(P, st, tm) : launch_route_g<kTypeF32>(P, st, tm);
}

hipError_t launch_topk(const TopkParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T <= 0) return hipSuccess;
    // one token per work-group, its rank counts split over the four wavefronts: at 512 tokens route +
    // top-k + permute measured 25.5 us against 25.9 with four tokens per work-group (one per wavefront)
    // and 27.1 with two tokens taken in turn
    return launch(topk_kernel<1>, dim3(P.T), dim3(kBlock), 0, st, tm, P);
}

hipError_t launch_gate_up(const GateUpParams &P, hipStream_t st, const LaunchTiming *tm) {
    int S, G;
    if (P.max_active <= 0 || !pick_split_gate_up(P.h / 256, &S, &G)) return hipSuccess;
    if (P.type == kTypeQ8_0) {
        if (S == 1) return launch_gate_up_t<kTypeQ8_0, 1>(P, G, st, tm);
        return launch_gate_up_t<kTypeQ8_0, 2>(P, G, st, tm);
    }
    if (pool_format(P.type) == kTypeKQ8) {
        if (S == 1) return launch_gate_up_t<kTypeKQ8, 1>(P, G, st, tm);
        return launch_gate_up_t<kTypeKQ8, 2>(P, G, st, tm);
    }
    if (S == 1) return launch_gate_up_t<kTypeQ4_K, 1>(P, G, st, tm);
    return launch_gate_up_t<kTypeQ4_K, 2>(P, G, st, tm);
}

hipError_t launch_down(const DownParams &P, hipStream_t st, const LaunchTiming *tm) {
    int S, G;
    if (P.max_active <= 0 || !pick_split(P.f / 256, &S, &G)) return hipSuccess;
    if (P.type == kTypeQ8_0) {
        if (S == 1) return launch_down_t<kTypeQ8_0, 1>(P, G, st, tm);
        return launch_down_t<kTypeQ8_0, 2>(P, G, st, tm);
    }
    if (pool_format(P.type) == kTypeKQ8) {
        if (S == 1) return launch_down_t<kTypeKQ8, 1>(P, G, st, tm);
        return launch_down_t<kTypeKQ8, 2>(P, G, st, tm);
    }
    if (S == 1) return launch_down_t<kTypeQ4_K, 1>(P, G, st, tm);
    return launch_down_t<kTypeQ4_K, 2>(P, G, st, tm);
}

hipError_t launch_combine(const CombineParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T <= 0) return hipSuccess;
    const int n = P.T * (P.h / 4);
    return launch(combine_kernel, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, tm, P);
}

}  // namespace lstk
