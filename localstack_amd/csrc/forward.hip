// forward.hip - gfx950 kernels of the Qwen3-MoE forward pass around the MoE block:
// RMSNorm (+ embedding gather), F16 GEMV for the projections and the output head, per-head QK-norm +
// NEOX RoPE + KV-cache store, and causal GQA attention over the fp16 cache with fp32 accumulation.
//
// Numerics follow what ggml's CPU backend does for the reference graph (src/qwen3.cpp:112-171,
// :223-259): F16 mat-muls round the f32 activations to fp16 and accumulate the exact fp16 x fp16
// products in f32; RMSNorm sums x*x in double and scales by 1/sqrtf(mean + eps); RoPE's angle for pair
// i is pos * theta_scale^i built by repeated multiplication; attention rounds Q to fp16, scales
// q.k by 1/sqrt(head_dim) and accumulates softmax(scores) . V in f32. Summation orders differ from
// ggml's (the kernels reduce across lanes), which is what the logits tolerance absorbs.
#include "device.h"
#include "forward.h"

namespace lstk {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kNormBlock = 256;
constexpr int kGvWaves = 4;     // wavefronts per GEMV work-group
constexpr int kGvRows = 4;      // rows per wavefront
constexpr int kGvMaxLds = 64 * 1024;
constexpr int kAtBlock = 256;   // attention: one cell per thread per pass
constexpr int kAtMaxHd = 256;

__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }
__device__ __forceinline__ uint32_t pack2(float a, float b) { return (uint32_t) f2h(a) | ((uint32_t) f2h(b) << 16); }

// a.lo * b.lo + a.hi * b.hi + c over fp16 pairs (v_dot2_f32_f16): the fp16 products are exact in f32.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c, false);
}
__device__ __forceinline__ float dot8(const uint4 &a, const uint4 &b, float c) {
    return dot2(a.w, b.w, dot2(a.z, b.z, dot2(a.y, b.y, dot2(a.x, b.x, c))));
}

// ------------------------------------------------------------------------------------------------
// RMSNorm (ggml_rms_norm + ggml_mul), optionally gathering the row from the embedding table first
// ------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kNormBlock) void rmsnorm_kernel(NormParams P) {
    __shared__ double s_part[kNormBlock / kWave];
    const int r = blockIdx.x, tid = threadIdx.x;
    const size_t off = (size_t) r * P.n;
    const uint16_t *e = P.emb ? P.emb + (size_t) P.tokens[r] * P.n : nullptr;
    const float *x = P.x + off;
    double s = 0.0;
    for (int i = tid; i < P.n; i += kNormBlock) {
        const float v = e ? h2f(e[i]) : x[i];
        if (e) P.x_out[off + i] = v;
        s += (double) (v * v);
    }
    s = wave_sum_d(s);
    if ((tid & (kWave - 1)) == 0) s_part[tid / kWave] = s;
    __syncthreads();
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float) (tot / (double) P.n);
    const float scale = 1.0f / sqrtf(mean + P.eps);
    for (int i = tid; i < P.n; i += kNormBlock) {
        const float v = e ? h2f(e[i]) : x[i];
        P.y[off + i] = (v * scale) * P.w[i];
    }
}

// ------------------------------------------------------------------------------------------------
// F16 GEMV over up to 3 matrices: each wavefront owns kGvRows rows, lanes stride the row in 16-byte
// chunks (a 1 KiB coalesced load per row per step), the TG tokens of a group sit in LDS as fp16 pairs
// and every weight chunk is used against all of them before the next is read.
// ------------------------------------------------------------------------------------------------

template <int TG>
__global__ __launch_bounds__(kGvWaves *kWave) void gemv_kernel(GemvParams P) {
    extern __shared__ uint4 s_x4[]; // [TG][cols / 8]
    uint32_t *s_x = reinterpret_cast<uint32_t *>(s_x4);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    const int cols = P.cols, nc = cols / 8, np = cols / 2;
    const int row0 = (blockIdx.x * kGvWaves + wv) * kGvRows;

    const uint4 *wr[kGvRows];
    float *yr[kGvRows];
    const float *ar[kGvRows];
    int ldy[kGvRows];
    bool on[kGvRows];
#pragma unroll
    for (int rr = 0; rr < kGvRows; rr++) {
        const int r = row0 + rr;
        on[rr] = r < P.rows_total;
        int loc = on[rr] ? r : 0, s = 0;
        while (s + 1 < P.nseg && loc >= P.seg[s].rows) {
            loc -= P.seg[s].rows;
            s++;
        }
        wr[rr] = reinterpret_cast<const uint4 *>(P.seg[s].w + (size_t) loc * cols);
        yr[rr] = P.seg[s].y + loc;
        ar[rr] = P.seg[s].add ? P.seg[s].add + loc : nullptr;
        ldy[rr] = P.seg[s].ldy;
    }

    for (int t0 = 0; t0 < P.T; t0 += TG) {
        const int nt = min(TG, P.T - t0);
        __syncthreads();
        for (int i = tid; i < TG * np; i += kGvWaves * kWave) {
            const int tt = i / np, c2 = i - tt * np;
            float2 v = make_float2(0.0f, 0.0f);
            if (tt < nt) v = *reinterpret_cast<const float2 *>(P.x + (size_t) (t0 + tt) * cols + 2 * c2);
            s_x[i] = pack2(v.x, v.y);
        }
        __syncthreads();
        float acc[kGvRows][TG];
#pragma unroll
        for (int rr = 0; rr < kGvRows; rr++)
#pragma unroll
            for (int tt = 0; tt < TG; tt++) acc[rr][tt] = 0.0f;
#pragma unroll 2
        for (int c = lane; c < nc; c += kWave) {
            uint4 w[kGvRows];
#pragma unroll
            for (int rr = 0; rr < kGvRows; rr++) w[rr] = wr[rr][c];
#pragma unroll
            for (int tt = 0; tt < TG; tt++) {
                const uint4 xv = s_x4[tt * nc + c];
#pragma unroll
                for (int rr = 0; rr < kGvRows; rr++) acc[rr][tt] = dot8(w[rr], xv, acc[rr][tt]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < kGvRows; rr++) {
#pragma unroll
            for (int tt = 0; tt < TG; tt++) {
                const float s = wave_sum_tree(acc[rr][tt]);
                if (lane == 0 && on[rr] && tt < nt) {
                    const size_t o = (size_t) (t0 + tt) * ldy[rr];
                    yr[rr][o] = ar[rr] ? s + ar[rr][o] : s;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// QK-norm + NEOX RoPE + KV store: one wavefront per (token, head) of Q, K and V
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ size_t k_index(int head, int d, int cell, int hd, int kv_size) {
    return (((size_t) head * (hd / 8) + d / 8) * kv_size + cell) * 8 + (d & 7);
}

__global__ __launch_bounds__(kWave) void rope_kernel(RopeParams P) {
    const int t = blockIdx.x, j = blockIdx.y, lane = threadIdx.x;
    const int hd = P.hd, half = hd / 2;
    const int cell = P.cells[t];
    if (j == 0 && lane == 0) {
        P.cell_seq[cell] = P.seq;
        P.cell_pos[cell] = P.pos[t];
    }
    if (j >= P.n_head + P.n_kv) {
        const int head = j - P.n_head - P.n_kv;
        const float *src = P.v + ((size_t) t * P.n_kv + head) * hd;
        uint16_t *dst = P.vc + ((size_t) head * P.kv_size + cell) * hd;
        for (int d = lane; d < hd; d += kWave) dst[d] = f2h(src[d]);
        return;
    }
    const bool is_q = j < P.n_head;
    const int head = is_q ? j : j - P.n_head;
    const float *src = is_q ? P.q + ((size_t) t * P.n_head + head) * hd : P.k + ((size_t) t * P.n_kv + head) * hd;
    const float *nw = is_q ? P.q_norm : P.k_norm;
    float scale = 1.0f;
    if (nw) {
        double s = 0.0;
        for (int d = lane; d < hd; d += kWave) {
            const float v = src[d];
            s += (double) (v * v);
        }
        s = wave_sum_d(s);
        const float mean = (float) (s / (double) hd);
        scale = 1.0f / sqrtf(mean + P.eps);
    }
    const float p = (float) P.pos[t];
    for (int i = lane; i < half; i += kWave) {
        float x0 = src[i], x1 = src[i + half];
        if (nw) {
            x0 = (x0 * scale) * nw[i];
            x1 = (x1 * scale) * nw[i + half];
        }
        float theta = p;
        for (int s = 0; s < i; s++) theta *= P.theta_scale;
        const float c = cosf(theta), sn = sinf(theta);
        const float y0 = x0 * c - x1 * sn;
        const float y1 = x0 * sn + x1 * c;
        if (is_q) {
            float *dst = P.q_out + ((size_t) t * P.n_head + head) * hd;
            dst[i] = y0;
            dst[i + half] = y1;
        } else {
            P.kc[k_index(head, i, cell, hd, P.kv_size)] = f2h(y0);
            P.kc[k_index(head, i + half, cell, hd, P.kv_size)] = f2h(y1);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// attention: work-group (chunk, head, token); 256 cells per pass (one per thread for the scores),
// online softmax across passes, P.V with (hd / 8) threads per cell and 256 / (hd / 8) cells at once
// ------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kAtBlock) void attn_kernel(AttnParams P) {
    __shared__ uint4 s_q4[kAtMaxHd / 8];
    __shared__ float s_p[kAtBlock];
    __shared__ float s_red[2 * (kAtBlock / kWave)];
    __shared__ float s_acc[kAtBlock * 8];
    uint32_t *s_q = reinterpret_cast<uint32_t *>(s_q4);
    const int c = blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wv = tid / kWave;
    const int hd = P.hd, n8 = hd / 8, G = kAtBlock / n8;
    const int kvh = h / (P.n_head / P.n_kv);
    const float *q = P.q + ((size_t) t * P.n_head + h) * hd;
    for (int i = tid; i < hd / 2; i += kAtBlock) s_q[i] = pack2(q[2 * i], q[2 * i + 1]);
    __syncthreads();

    const int my_pos = P.pos[t];
    const int begin = c * P.chunk, end = min(begin + P.chunk, P.n_cells);
    const int d8 = tid % n8, g = tid / n8;
    const uint16_t *kbase = P.kc + (size_t) kvh * n8 * P.kv_size * 8;
    const uint16_t *vbase = P.vc + (size_t) kvh * P.kv_size * hd;
    float m_run = -INFINITY, l_run = 0.0f;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;

    for (int base = begin; base < end; base += kAtBlock) {
        const int j = base + tid;
        float s = -INFINITY;
        if (j < end && P.cell_seq[j] == P.seq && P.cell_pos[j] <= my_pos) {
            float d = 0.0f;
            for (int cc = 0; cc < n8; cc++) {
                const uint4 kv = *reinterpret_cast<const uint4 *>(kbase + ((size_t) cc * P.kv_size + j) * 8);
                d = dot8(kv, s_q4[cc], d);
            }
            s = d * P.scale;
        }
        const float wm = wave_max(s);
        if (lane == 0) s_red[wv] = wm;
        __syncthreads();
        const float m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
        __syncthreads();
        const float m_new = fmaxf(m_run, m);
        if (m_new == -INFINITY) continue; // nothing visible yet (uniform across the work-group)
        const float p = s == -INFINITY ? 0.0f : expf(s - m_new);
        s_p[tid] = p;
        const float ws = wave_sum_tree(p);
        if (lane == 0) s_red[4 + wv] = ws;
        __syncthreads();
        const float psum = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
        const float f = expf(m_run - m_new);
        l_run = l_run * f + psum;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] *= f;
        m_run = m_new;
        for (int jj = g; jj < kAtBlock; jj += G) {
            const float pj = s_p[jj];
            if (pj != 0.0f) {
                const uint4 vv = *reinterpret_cast<const uint4 *>(vbase + (size_t) (base + jj) * hd + d8 * 8);
                acc[0] += pj * h2f(vv.x);
                acc[1] += pj * h2f(vv.x >> 16);
                acc[2] += pj * h2f(vv.y);
                acc[3] += pj * h2f(vv.y >> 16);
                acc[4] += pj * h2f(vv.z);
                acc[5] += pj * h2f(vv.z >> 16);
                acc[6] += pj * h2f(vv.w);
                acc[7] += pj * h2f(vv.w >> 16);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int e = 0; e < 8; e++) s_acc[g * hd + d8 * 8 + e] = acc[e];
    __syncthreads();
    if (tid < hd) {
        float o = 0.0f;
        for (int gg = 0; gg < G; gg++) o += s_acc[gg * hd + tid];
        if (P.n_chunk == 1) {
            P.out[((size_t) t * P.n_head + h) * hd + tid] = o / l_run;
        } else {
            float *pp = P.part + (((size_t) t * P.n_head + h) * P.n_chunk + c) * (hd + 2);
            pp[2 + tid] = o;
            if (tid == 0) {
                pp[0] = m_run;
                pp[1] = l_run;
            }
        }
    }
}

__global__ __launch_bounds__(kAtMaxHd) void attn_combine_kernel(AttnParams P) {
    const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
    const int hd = P.hd;
    const float *pp = P.part + ((size_t) t * P.n_head + h) * P.n_chunk * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < P.n_chunk; c++) M = fmaxf(M, pp[(size_t) c * (hd + 2)]);
    float L = 0.0f, o = 0.0f;
    for (int c = 0; c < P.n_chunk; c++) {
        const float *q = pp + (size_t) c * (hd + 2);
        if (q[0] == -INFINITY) continue;
        const float f = expf(q[0] - M);
        L += q[1] * f;
        o += q[2 + d] * f;
    }
    P.out[((size_t) t * P.n_head + h) * hd + d] = o / L;
}

__global__ __launch_bounds__(kBlock) void fill_kernel(FillParams P) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < P.n) P.p[i] = P.v;
}

template <int TG>
size_t gemv_lds(int cols) {
    return (size_t) TG * cols * 2;
}

}  // namespace

bool gemv_supported(int cols) { return cols > 0 && cols % 8 == 0 && gemv_lds<1>(cols) <= (size_t) kGvMaxLds; }

// head_dim a power of two in [16, 256]: the P.V phase splits the 256 threads into 256 / (hd / 8) groups.
bool attn_supported(int hd) { return hd >= 16 && hd <= kAtMaxHd && (hd & (hd - 1)) == 0; }

// Splits the attended cells into chunks (multiples of 256 cells) so that a step with few
// (token, head) pairs still launches about 1024 work-groups; returns the chunk size.
int attn_chunk_cells(int T, int n_head, int n_cells, int *n_chunk) {
    const int passes = (n_cells + kAtBlock - 1) / kAtBlock;
    const int pairs = T * n_head;
    int want = (1024 + pairs - 1) / pairs;
    want = want < 1 ? 1 : (want > passes ? passes : want);
    const int per = (passes + want - 1) / want;
    const int chunk = per * kAtBlock;
    *n_chunk = (n_cells + chunk - 1) / chunk;
    return chunk;
}

hipError_t launch_rmsnorm(const NormParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.rows == 0) return hipSuccess;
    return launch(rmsnorm_kernel, dim3(P.rows), dim3(kNormBlock), 0, st, tm, P);
}

hipError_t launch_gemv(const GemvParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0 || P.rows_total == 0) return hipSuccess;
    const int per_wg = kGvWaves * kGvRows;
    const dim3 grid((P.rows_total + per_wg - 1) / per_wg), block(kGvWaves * kWave);
    // tokens per group: enough for the step, as many as the activations' LDS allows
    int tg = P.T == 1 ? 1 : P.T == 2 ? 2 : P.T <= 4 ? 4 : 8;
    while (tg > 1 && gemv_lds<1>(P.cols) * tg > (size_t) kGvMaxLds) tg /= 2;
    if (tg == 1) return launch(gemv_kernel<1>, grid, block, gemv_lds<1>(P.cols), st, tm, P);
    if (tg == 2) return launch(gemv_kernel<2>, grid, block, gemv_lds<2>(P.cols), st, tm, P);
    if (tg == 4) return launch(gemv_kernel<4>, grid, block, gemv_lds<4>(P.cols), st, tm, P);
    return launch(gemv_kernel<8>, grid, block, gemv_lds<8>(P.cols), st, tm, P);
}

hipError_t launch_rope(const RopeParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0) return hipSuccess;
    return launch(rope_kernel, dim3(P.T, P.n_head + 2 * P.n_kv), dim3(kWave), 0, st, tm, P);
}

hipError_t launch_attn(const AttnParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0) return hipSuccess;
    return launch(attn_kernel, dim3(P.n_chunk, P.n_head, P.T), dim3(kAtBlock), 0, st, tm, P);
}

hipError_t launch_attn_combine(const AttnParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0 || P.n_chunk == 1) return hipSuccess;
    return launch(attn_combine_kernel, dim3(P.n_head, P.T), dim3(P.hd), 0, st, tm, P);
}

hipError_t launch_fill(const FillParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.n <= 0) return hipSuccess;
    return launch(fill_kernel, dim3((P.n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, tm, P);
}

}  // namespace lstk
