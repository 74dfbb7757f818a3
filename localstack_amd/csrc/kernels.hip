// kernels.hip - gfx950 (CDNA4) kernels of the Qwen3-MoE expert-FFN path.
//
// One MoE block = three launches on the caller's stream:
//   prologue  router logits (one wavefront per expert, all tokens of a tile), activation
//             quantization (Q8_0 or Q8_K rows of hnorm), and in the last work-group to finish:
//             softmax + top-k + renormalisation per token (one wavefront per token) and the stable
//             token->expert permutation. Replaces src/qwen3.cpp:178-189 and ggml's mul_mat_id
//             grouping. The "last work-group" is found with one atomic per work-group: nobody waits.
//   gate_up   per active expert and 16-row block: gate and up rows dequantized in registers from
//             coalesced 16-byte chunks, int8 dot products (v_dot4_i32_i8) against the quantized
//             activations of every token routed to the expert, fused SwiGLU (src/qwen3.cpp:201-203).
//   down      per active expert and 64-row block: the SwiGLU rows re-quantized in LDS, down rows
//             from registers, each pair's output scaled by its router weight (src/qwen3.cpp:204-205);
//             the last expert to finish a row block sums the k outputs of every token in slot order
//             and adds the residual (src/qwen3.cpp:206-212, :250).
// Decode is HBM-bound: every weight byte is read once per step, with all of a thread's loads issued
// before any arithmetic.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "formats.h"
#include "kernels.h"

namespace lstk {
namespace {

constexpr int kBlock = 256;
constexpr int kWave = 64;
constexpr int kRouteEPW = 2;      // experts per wavefront in the router tile
constexpr int kRouteEG = 8;       // experts per router work-group (4 wavefronts x 2)
constexpr int kRouteMaxNG = 16;   // n_embd <= 4096: 16 groups of 256 per lane
constexpr int kMaxEPL = 4;        // n_expert <= 256: 4 logits per lane in the top-k
constexpr int kGuRows = 16;       // rows of gate (and of up) per gate_up work-group
constexpr int kDnRows = 64;       // rows per down work-group
constexpr int kTC = 8;            // tokens staged per pass
constexpr int kMaxG = 8;          // K-groups per work-group
constexpr int kMaxK = 64;         // n_expert_used <= 64 (one lane per selected expert)
constexpr int kMaxBins = 4096;

__device__ __forceinline__ float h2f(unsigned h) { return __half2float(__ushort_as_half((unsigned short) (h & 0xffffu))); }
__device__ __forceinline__ float round_f16(float x) { return __half2float(__float2half_rn(x)); }

// ------------------------------------------------------------------------------------------------
// router logits
// ------------------------------------------------------------------------------------------------

// Dot products of a tile of tokens with kRouteEG experts. Lane l of a wavefront owns elements
// 256 g + 4 l + q (g ascending, then q) and accumulates them with fmaf from 0; the 64 partials are
// combined with a butterfly. The oracle evaluates the same expression in the same order, so the
// logits agree bit for bit and so does the top-k. F16 weights see fp16-rounded activations, as
// ggml's CPU mul_mat converts src1 to the F16 vec_dot_type (src/qwen3.cpp:178).
template <int GT>
__device__ void route_tile(const PrologueParams &P, int b, float *xs, int tt) {
    const int n_eg = (P.E + kRouteEG - 1) / kRouteEG;
    const int tile = b / n_eg, eg = b - tile * n_eg;
    const int t0 = tile * tt;
    const int nt = min(tt, P.T - t0);
    const int h = P.h, ng = h / 256;
    const float4 *src = reinterpret_cast<const float4 *>(P.hnorm + (size_t) t0 * h);
    float4 *dst = reinterpret_cast<float4 *>(xs);
    for (int i = threadIdx.x; i < nt * h / 4; i += blockDim.x) {
        float4 v = src[i];
        if (GT == kTypeF16) {
            v.x = round_f16(v.x);
            v.y = round_f16(v.y);
            v.z = round_f16(v.z);
            v.w = round_f16(v.w);
        }
        dst[i] = v;
    }
    __syncthreads();
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int ee = 0; ee < kRouteEPW; ee++) {
        const int e = eg * kRouteEG + wave * kRouteEPW + ee;
        if (e >= P.E) break;
        float w[kRouteMaxNG][4];
#pragma unroll
        for (int g = 0; g < kRouteMaxNG; g++) {
            if (g < ng) {
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
        }
        for (int t = 0; t < nt; t++) {
            float acc = 0.0f;
#pragma unroll
            for (int g = 0; g < kRouteMaxNG; g++) {
                if (g < ng) {
                    const float4 x = *reinterpret_cast<const float4 *>(xs + (size_t) t * h + 256 * g + 4 * lane);
                    acc = fmaf(x.x, w[g][0], acc);
                    acc = fmaf(x.y, w[g][1], acc);
                    acc = fmaf(x.z, w[g][2], acc);
                    acc = fmaf(x.w, w[g][3], acc);
                }
            }
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) acc = acc + __shfl_xor(acc, s);
            if (lane == 0) P.logits[(size_t) (t0 + t) * P.E + e] = acc;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// activation quantization (ggml's quantize_row_q8_0 x86 path / quantize_row_q8_K_ref)
// ------------------------------------------------------------------------------------------------

// Quantizes x[0..n) (n % 256 == 0) with all threads of the block, 8 values per thread per pass.
// Q8_0 (QT 8): d = amax/127 stored as fp16, q = rne(x * 127/amax), groups of 4 threads per block.
// Q8_K (QT 12): max = the signed value of the first largest |x| of the 256, iscale = -127/max,
// q = min(127, rne(iscale x)), d = 1/iscale; groups of 32 threads; bs = sums of 32-value groups.
// Every thread runs the shuffles; threads past the end contribute zeros and write nothing.
template <int QT>
__device__ void quantize_row(const float *__restrict__ x, int n, int8_t *qs, float *d, int32_t *bs) {
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
        int q[8];
        float dd;
        if (QT == kTypeQ8_0) {
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
            amax = fmaxf(amax, __shfl_xor(amax, 1));
            amax = fmaxf(amax, __shfl_xor(amax, 2));
            dd = round_f16(__fdiv_rn(amax, 127.0f));
            const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) q[j] = (int) rintf(v[j] * id);
        } else {
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
#pragma unroll
            for (int s = 16; s >= 1; s >>= 1) {
                const float oa = __shfl_xor(amax, s);
                const float om = __shfl_xor(mx, s);
                const int oi = __shfl_xor(idx, s);
                if (oa > amax || (oa == amax && oi < idx)) {
                    amax = oa;
                    mx = om;
                    idx = oi;
                }
            }
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
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
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
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// softmax / top-k / renormalisation (router(), src/qwen3.cpp:179-189)
// ------------------------------------------------------------------------------------------------

// One wavefront per token. Selection is made on the logits (softmax is monotone), largest first,
// ties to the lower expert id; p = expf(l - max) * (float)(1 / sum) with the sum in double; the k
// selected p are summed in selection order in double, clamped to >= 2^-14 and divided out.
__device__ void route_finalize(const PrologueParams &P) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    const int E = P.E, k = P.k;
    for (int t = wave; t < P.T; t += nw) {
        float l[kMaxEPL], p[kMaxEPL];
        bool taken[kMaxEPL];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < kMaxEPL; i++) {
            const int e = lane + kWave * i;
            l[i] = e < E ? P.logits[(size_t) t * E + e] : -INFINITY;
            m = fmaxf(m, l[i]);
            taken[i] = false;
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s));
        double sum = 0.0;
#pragma unroll
        for (int i = 0; i < kMaxEPL; i++) {
            const int e = lane + kWave * i;
            p[i] = e < E ? expf(l[i] - m) : 0.0f;
            sum += (double) p[i];
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) sum += __shfl_xor(sum, s);
        const float inv = (float) (1.0 / sum);
#pragma unroll
        for (int i = 0; i < kMaxEPL; i++) p[i] = p[i] * inv;
        int my_id = 0;
        for (int j = 0; j < k; j++) {
            float bv = -INFINITY;
            int bi = INT_MAX;
#pragma unroll
            for (int i = 0; i < kMaxEPL; i++) {
                const int e = lane + kWave * i;
                if (e < E && !taken[i] && (bi == INT_MAX || l[i] > bv)) {
                    bv = l[i];
                    bi = e;
                }
            }
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) {
                const float ov = __shfl_xor(bv, s);
                const int oi = __shfl_xor(bi, s);
                if (oi != INT_MAX && (bi == INT_MAX || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            if ((bi & (kWave - 1)) == lane) {
#pragma unroll
                for (int i = 0; i < kMaxEPL; i++)
                    if ((bi >> 6) == i) taken[i] = true;
            }
            if (lane == j) my_id = bi;
        }
        float my_p = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxEPL; i++) {
            const float v = __shfl(p[i], my_id & (kWave - 1));
            if ((my_id >> 6) == i) my_p = v;
        }
        double ss = 0.0;
        for (int j = 0; j < k; j++) ss += (double) __shfl(my_p, j);
        const float sf = fmaxf((float) ss, 6.103515625e-5f);
        if (lane < k) {
            P.ids[(size_t) t * k + lane] = my_id;
            P.weights[(size_t) t * k + lane] = __fdiv_rn(my_p, sf);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// permutation
// ------------------------------------------------------------------------------------------------

__device__ int block_exclusive_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    int x = v;
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
        const int y = __shfl_up(x, s);
        if (lane >= s) x += y;
    }
    if (lane == kWave - 1) tmp[wave] = x;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int w = 0; w < nw; w++) {
        const int tw = tmp[w];
        if (w < wave) wbase += tw;
        tot += tw;
    }
    __syncthreads();
    *total = tot;
    return wbase + x - v;
}

// Stable counting sort of the T*k (t, j) pairs by bin: histogram and scan in LDS, then 32 tokens
// at a time, each pair's rank among the chunk's earlier tokens is a popcount of a per-bin bitmask.
// Ids out of range are clamped and flagged in *err (bit 0); a bin repeated within one token is
// flagged (bit 1). perm is cleared first so every position read later names a valid pair.
__device__ void permute(const PrologueParams &P, int *lds) {
    const int nb = P.n_bins, k = P.k, np = P.T * k;
    const int tid = threadIdx.x, bd = blockDim.x;
    int *cnt = lds;
    int *cur = lds + nb;
    unsigned *bm = reinterpret_cast<unsigned *>(lds + 2 * nb);
    int *tmp = lds + 3 * nb;
    for (int b = tid; b < nb; b += bd) cnt[b] = 0;
    for (int p = tid; p < np; p += bd) P.pb.perm[p] = 0;
    __syncthreads();
    for (int p = tid; p < np; p += bd) {
        int b = P.bins[p];
        if (b < 0 || b >= nb) {
            atomicOr(P.err, 1);
            b = min(max(b, 0), nb - 1);
        }
        atomicAdd(&cnt[b], 1);
    }
    __syncthreads();
    const int per = (nb + bd - 1) / bd;
    const int b0 = min(nb, tid * per), b1 = min(nb, b0 + per);
    int s = 0, a = 0;
    for (int b = b0; b < b1; b++) {
        s += cnt[b];
        a += cnt[b] > 0;
    }
    int tot, tota;
    int so = block_exclusive_scan(s, tmp, &tot);
    int ao = block_exclusive_scan(a, tmp, &tota);
    for (int b = b0; b < b1; b++) {
        P.pb.counts[b] = cnt[b];
        P.pb.offsets[b] = so;
        cur[b] = so;
        so += cnt[b];
        if (cnt[b] > 0) P.pb.active[ao++] = b;
    }
    if (tid == 0) {
        P.pb.offsets[nb] = tot;
        *P.pb.n_active = tota;
    }
    __syncthreads();
    constexpr int kPairsPerThread = 32 * kMaxK / kBlock;
    for (int t0 = 0; t0 < P.T; t0 += 32) {
        const int npc = min(32, P.T - t0) * k;
        for (int b = tid; b < nb; b += bd) bm[b] = 0u;
        __syncthreads();
        int myb[kPairsPerThread];
#pragma unroll
        for (int q = 0; q < kPairsPerThread; q++) {
            const int pc = tid + q * bd;
            myb[q] = 0;
            if (pc < npc) {
                int b = P.bins[t0 * k + pc];
                b = min(max(b, 0), nb - 1);
                myb[q] = b;
                const unsigned bit = 1u << (pc / k);
                if (atomicOr(&bm[b], bit) & bit) atomicOr(P.err, 2);
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPairsPerThread; q++) {
            const int pc = tid + q * bd;
            if (pc < npc) {
                const int b = myb[q];
                const int pos = cur[b] + __popc(bm[b] & ((1u << (pc / k)) - 1u));
                P.pb.perm[pos] = t0 * k + pc;
            }
        }
        __syncthreads();
        for (int b = tid; b < nb; b += bd) cur[b] += __popc(bm[b]);
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// prologue kernel
// ------------------------------------------------------------------------------------------------

template <int GT, int QT>
__global__ __launch_bounds__(kBlock) void prologue_kernel(PrologueParams P, int n_route_wg, int n_quant_wg, int route_tt) {
    extern __shared__ __align__(16) float lds[];
    __shared__ int is_last;
    const int b = blockIdx.x;
    if (b < n_route_wg) {
        route_tile<GT>(P, b, lds, route_tt);
    } else if (QT != 0) {
        const int h = P.h;
        for (int t = b - n_route_wg; t < P.T; t += n_quant_wg)
            quantize_row<QT>(P.hnorm + (size_t) t * h, h, P.xq.qs + (size_t) t * h, P.xq.d + (size_t) t * (h / 32),
                             P.xq.bs + (size_t) t * (h / 32));
    }
    // arrival: the last work-group to get here sees every other work-group's writes
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(P.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    if (P.do_route) route_finalize(P);
    if (P.do_perm) {
        __threadfence();
        __syncthreads();
        permute(P, reinterpret_cast<int *>(lds));
    }
    if (threadIdx.x == 0) atomicExch(P.counter, 0u);
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

template <int WT>
__device__ __forceinline__ float dot_sb(const uint4 (&w)[chunks_of(WT)], const int8_t *x, const float *xd,
                                        const int *xb, float acc) {
    if constexpr (WT == kTypeQ8_0) {
        (void) xb;
        return dot_sb_q8_0(w, x, xd, acc);
    } else {
        return dot_sb_q4_K(w, x, xd, xb, acc);
    }
}

// ------------------------------------------------------------------------------------------------
// gate + up + SwiGLU
// ------------------------------------------------------------------------------------------------

// Work-group (row block, active expert): thread (g, m, r) holds super-blocks g, g + G, ... of row r
// of gate (m = 0) or up (m = 1) in registers, loaded before anything else. Tokens of the expert are
// staged 8 at a time in LDS; partial dots are reduced over g in ascending order, then
// act = silu(gate) * up is written to the token's row in permuted order.
template <int WT, int S>
__global__ __launch_bounds__(kBlock) void gate_up_kernel(GateUpParams P) {
    constexpr int C = chunks_of(WT);
    extern __shared__ __align__(16) unsigned char smem[];
    const int n_active = *P.pb.n_active;
    const int ai = blockIdx.y;
    if (ai >= n_active) return;
    const int e = P.pb.active[ai];
    const int G = blockDim.x / (2 * kGuRows);
    const int tid = threadIdx.x;
    const int r = tid % kGuRows, m = (tid / kGuRows) & 1, g = tid / (2 * kGuRows);
    const int f = P.f, h = P.h, k = P.k;
    const int row = blockIdx.x * kGuRows + r;
    const uint8_t *base = m ? P.w_up + (size_t) e * P.stride_up : P.w_gate + (size_t) e * P.stride_gate;
    uint4 w[S][C];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int sb = g + s * G;
#pragma unroll
        for (int c = 0; c < C; c++) w[s][c] = *reinterpret_cast<const uint4 *>(base + chunk_offset(C, f, sb, c, row));
    }
    const int h32 = h / 32;
    int8_t *xs = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(smem + (size_t) kTC * h);
    int *xb = reinterpret_cast<int *>(xd + kTC * h32);
    float *red = reinterpret_cast<float *>(xb + kTC * h32);
    const int cnt = P.pb.counts[e], off = P.pb.offsets[e];
    for (int c0 = 0; c0 < cnt; c0 += kTC) {
        const int nt = min(kTC, cnt - c0);
        for (int tc = 0; tc < nt; tc++) {
            const int t = P.pb.perm[off + c0 + tc] / k;
            const int4 *src = reinterpret_cast<const int4 *>(P.xq.qs + (size_t) t * h);
            int4 *dst = reinterpret_cast<int4 *>(xs + (size_t) tc * h);
            for (int i = tid; i < h / 16; i += blockDim.x) dst[i] = src[i];
            for (int i = tid; i < h32; i += blockDim.x) {
                xd[tc * h32 + i] = P.xq.d[(size_t) t * h32 + i];
                if (WT == kTypeQ4_K) xb[tc * h32 + i] = P.xq.bs[(size_t) t * h32 + i];
            }
        }
        __syncthreads();
        for (int tc = 0; tc < nt; tc++) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int sb = g + s * G;
                acc = dot_sb<WT>(w[s], xs + (size_t) tc * h + sb * 256, xd + tc * h32 + sb * 8, xb + tc * h32 + sb * 8, acc);
            }
            red[((tc * G + g) * 2 + m) * kGuRows + r] = acc;
        }
        __syncthreads();
        for (int idx = tid; idx < nt * kGuRows; idx += blockDim.x) {
            const int tc = idx / kGuRows, rr = idx % kGuRows;
            float gs = red[((tc * G) * 2 + 0) * kGuRows + rr];
            float us = red[((tc * G) * 2 + 1) * kGuRows + rr];
            for (int gg = 1; gg < G; gg++) {
                gs += red[((tc * G + gg) * 2 + 0) * kGuRows + rr];
                us += red[((tc * G + gg) * 2 + 1) * kGuRows + rr];
            }
            const float a = (gs / (1.0f + expf(-gs))) * us;
            P.act[(size_t) (off + c0 + tc) * f + blockIdx.x * kGuRows + rr] = a;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// down + router weight + combine + residual
// ------------------------------------------------------------------------------------------------

template <int WT, int S>
__global__ __launch_bounds__(kDnRows * kMaxG) void down_kernel(DownParams P) {
    constexpr int C = chunks_of(WT);
    constexpr int QT = WT == kTypeQ4_K ? kTypeQ4_K : kTypeQ8_0;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int is_last;
    const int n_active = *P.pb.n_active;
    const int ai = blockIdx.y, rb = blockIdx.x;
    if (ai >= n_active) return;
    const int e = P.pb.active[ai];
    const int G = blockDim.x / kDnRows;
    const int tid = threadIdx.x, r = tid % kDnRows, g = tid / kDnRows;
    const int h = P.h, f = P.f, k = P.k;
    const int row = rb * kDnRows + r;
    const uint8_t *base = P.w_down + (size_t) e * P.stride_down;
    uint4 w[S][C];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int sb = g + s * G;
#pragma unroll
        for (int c = 0; c < C; c++) w[s][c] = *reinterpret_cast<const uint4 *>(base + chunk_offset(C, h, sb, c, row));
    }
    const int f32 = f / 32;
    int8_t *xs = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(smem + (size_t) kTC * f);
    int *xb = reinterpret_cast<int *>(xd + kTC * f32);
    float *red = reinterpret_cast<float *>(xb + kTC * f32);
    const int cnt = P.pb.counts[e], off = P.pb.offsets[e];
    for (int c0 = 0; c0 < cnt; c0 += kTC) {
        const int nt = min(kTC, cnt - c0);
        for (int tc = 0; tc < nt; tc++)
            quantize_row<QT>(P.act + (size_t) (off + c0 + tc) * f, f, xs + (size_t) tc * f, xd + tc * f32, xb + tc * f32);
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
            float ds = red[(tc * G) * kDnRows + rr];
            for (int gg = 1; gg < G; gg++) ds += red[(tc * G + gg) * kDnRows + rr];
            const int p = P.pb.perm[off + c0 + tc];
            P.Y[(size_t) p * h + rb * kDnRows + rr] = ds * P.weights[p];
        }
        __syncthreads();
    }
    // arrival: the last active expert of this row block combines the k outputs of every token
    __threadfence();
    __syncthreads();
    if (tid == 0) is_last = atomicAdd(&P.counters[rb], 1u) == (unsigned) (n_active - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int idx = tid; idx < P.T * kDnRows; idx += blockDim.x) {
        const int t = idx / kDnRows, rr = idx % kDnRows;
        const int rw = rb * kDnRows + rr;
        const float *y = P.Y + (size_t) t * k * h + rw;
        float acc = y[0];
        for (int j = 1; j < k; j++) acc = acc + y[(size_t) j * h];
        P.out[(size_t) t * h + rw] = acc + P.resid[(size_t) t * h + rw];
    }
    if (tid == 0) atomicExch(&P.counters[rb], 0u);
    (void) row;
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------

// Super-blocks per thread S and K-groups G for nsb super-blocks: the smallest S <= 2 dividing nsb
// with nsb / S <= 8 (S = 3 would need more than 256 VGPRs and spill).
bool pick_split(int nsb, int *S, int *G) {
    for (int s = 1; s <= 2; s++) {
        if (nsb % s == 0 && nsb / s <= kMaxG) {
            *S = s;
            *G = nsb / s;
            return true;
        }
    }
    return false;
}

int route_tile_tokens(int h) { return std::max(1, std::min(8, 32768 / (h * 4))); }

template <int GT, int QT>
hipError_t launch_prologue_t(const PrologueParams &P, hipStream_t st) {
    int n_route = 0, tt = 0;
    if (P.do_route) {
        tt = route_tile_tokens(P.h);
        n_route = ((P.T + tt - 1) / tt) * ((P.E + kRouteEG - 1) / kRouteEG);
    }
    const int n_quant = QT ? std::min(P.T, 256) : 0;
    int grid = n_route + n_quant;
    if (grid == 0) grid = 1;
    size_t lds = 0;
    if (P.do_route) lds = std::max(lds, (size_t) tt * P.h * 4);
    if (P.do_perm) lds = std::max(lds, (size_t) (3 * P.n_bins + 16) * 4);
    if (lds == 0) lds = 16;
    hipLaunchKernelGGL((prologue_kernel<GT, QT>), dim3(grid), dim3(kBlock), lds, st, P, n_route, n_quant, tt);
    return hipGetLastError();
}

template <int WT, int S>
hipError_t launch_gate_up_t(const GateUpParams &P, int G, hipStream_t st) {
    const int h32 = P.h / 32;
    const size_t lds = (size_t) kTC * P.h + (size_t) 2 * kTC * h32 * 4 + (size_t) kTC * G * 2 * kGuRows * 4;
    hipLaunchKernelGGL((gate_up_kernel<WT, S>), dim3(P.f / kGuRows, P.max_active), dim3(2 * kGuRows * G), lds, st, P);
    return hipGetLastError();
}

template <int WT, int S>
hipError_t launch_down_t(const DownParams &P, int G, hipStream_t st) {
    const int f32 = P.f / 32;
    const size_t lds = (size_t) kTC * P.f + (size_t) 2 * kTC * f32 * 4 + (size_t) kTC * G * kDnRows * 4;
    hipLaunchKernelGGL((down_kernel<WT, S>), dim3(P.h / kDnRows, P.max_active), dim3(kDnRows * G), lds, st, P);
    return hipGetLastError();
}

}  // namespace

const char *check_shapes(int h, int f, int E, int k, int n_bins) {
    int S, G;
    if (h <= 0 || h % 256 != 0) return "n_embd must be a positive multiple of 256";
    if (h > 256 * kRouteMaxNG) return "n_embd above 4096 is not supported by the router kernel";
    if (f <= 0 || f % 256 != 0) return "n_ff_exp must be a positive multiple of 256";
    if (E < 1 || E > kWave * kMaxEPL) return "n_expert must be in [1, 256]";
    if (k < 1 || k > E || k > kMaxK) return "n_expert_used must be in [1, min(n_expert, 64)]";
    if (n_bins < 1 || n_bins > kMaxBins) return "slot count must be in [1, 4096]";
    if (!pick_split(h / 256, &S, &G)) return "n_embd / 256 has no split into <= 8 groups of <= 2 super-blocks";
    if (!pick_split(f / 256, &S, &G)) return "n_ff_exp / 256 has no split into <= 8 groups of <= 2 super-blocks";
    return "";
}

hipError_t launch_prologue(const PrologueParams &P, hipStream_t st) {
    if (P.T <= 0) return hipSuccess;
    const int gt = P.do_route ? P.gate_type : kTypeF16;
    if (gt == kTypeF16) {
        if (P.qtype == kTypeQ8_0) return launch_prologue_t<kTypeF16, kTypeQ8_0>(P, st);
        if (P.qtype == kTypeQ4_K) return launch_prologue_t<kTypeF16, kTypeQ4_K>(P, st);
        return launch_prologue_t<kTypeF16, 0>(P, st);
    }
    if (P.qtype == kTypeQ8_0) return launch_prologue_t<kTypeF32, kTypeQ8_0>(P, st);
    if (P.qtype == kTypeQ4_K) return launch_prologue_t<kTypeF32, kTypeQ4_K>(P, st);
    return launch_prologue_t<kTypeF32, 0>(P, st);
}

hipError_t launch_gate_up(const GateUpParams &P, hipStream_t st) {
    int S, G;
    if (P.max_active <= 0 || !pick_split(P.h / 256, &S, &G)) return hipSuccess;
    if (P.type == kTypeQ8_0) {
        if (S == 1) return launch_gate_up_t<kTypeQ8_0, 1>(P, G, st);
        return launch_gate_up_t<kTypeQ8_0, 2>(P, G, st);
    }
    if (S == 1) return launch_gate_up_t<kTypeQ4_K, 1>(P, G, st);
    return launch_gate_up_t<kTypeQ4_K, 2>(P, G, st);
}

hipError_t launch_down(const DownParams &P, hipStream_t st) {
    int S, G;
    if (P.max_active <= 0 || !pick_split(P.f / 256, &S, &G)) return hipSuccess;
    if (P.type == kTypeQ8_0) {
        if (S == 1) return launch_down_t<kTypeQ8_0, 1>(P, G, st);
        return launch_down_t<kTypeQ8_0, 2>(P, G, st);
    }
    if (S == 1) return launch_down_t<kTypeQ4_K, 1>(P, G, st);
    return launch_down_t<kTypeQ4_K, 2>(P, G, st);
}

}  // namespace lstk
