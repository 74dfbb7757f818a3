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

// NPT values per thread, all loaded before any is used (one memory round trip per row). COMB: the row
// is first the previous MoE block's combine (P.Y), formed here in combine_kernel's order.
template <int NPT, bool COMB>
__global__ __launch_bounds__(kNormBlock) void rmsnorm_kernel(NormParams P) {
    __shared__ double s_part[kNormBlock / kWave];
    const int r = blockIdx.x, tid = threadIdx.x;
    const size_t off = (size_t) r * P.n;
    const uint16_t *e = P.emb ? P.emb + (size_t) P.tokens[r] * P.n : nullptr;
    const float *x = P.x + off;
    float v[NPT], w[NPT];
#pragma unroll
    for (int k = 0; k < NPT; k++) {
        const int i = tid + k * kNormBlock;
        const bool on = i < P.n;
        v[k] = !on ? 0.0f : e ? h2f(e[i]) : x[i];
        w[k] = on ? P.w[i] : 0.0f;
    }
    if constexpr (COMB) {
        // out = ((Y_0 + Y_1) + ... + Y_{k-1}) + x, the slots' loads in batches of B issued together
        // (B * NPT <= 64 values in flight per thread)
        constexpr int B = NPT >= 32 ? 2 : NPT >= 16 ? 4 : 8;
        const float *yb = P.Y + (size_t) r * P.k * P.n;
        float acc[NPT];
#pragma unroll
        for (int k = 0; k < NPT; k++) {
            const int i = tid + k * kNormBlock;
            acc[k] = i < P.n ? yb[i] : 0.0f;
        }
        for (int j0 = 1; j0 < P.k; j0 += B) {
            float t[B][NPT];
#pragma unroll
            for (int u = 0; u < B; u++)
#pragma unroll
                for (int k = 0; k < NPT; k++) {
                    const int i = tid + k * kNormBlock;
                    t[u][k] = i < P.n ? yb[(size_t) min(j0 + u, P.k - 1) * P.n + i] : 0.0f;
                }
#pragma unroll
            for (int u = 0; u < B; u++)
                if (j0 + u < P.k)
#pragma unroll
                    for (int k = 0; k < NPT; k++) acc[k] = acc[k] + t[u][k];
        }
#pragma unroll
        for (int k = 0; k < NPT; k++) v[k] = acc[k] + v[k];
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NPT; k++) s += (double) (v[k] * v[k]);
    s = wave_sum_d(s);
    if ((tid & (kWave - 1)) == 0) s_part[tid / kWave] = s;
    __syncthreads();
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float) (tot / (double) P.n);
    const float scale = 1.0f / sqrtf(mean + P.eps);
#pragma unroll
    for (int k = 0; k < NPT; k++) {
        const int i = tid + k * kNormBlock;
        if (i < P.n) {
            if (e || COMB) P.x_out[off + i] = v[k];
            const float y = (v[k] * scale) * w[k];
            P.y[off + i] = y;
            if (P.y16) P.y16[off + i] = f2h(y);
        }
    }
}



// ------------------------------------------------------------------------------------------------
// QK-norm + NEOX RoPE + KV store: one wavefront per (token, head) of Q, K and V
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ size_t k_index(int head, int d, int cell, int hd, int kv_size) {
    return (((size_t) head * (hd / 4) + d / 4) * kv_size + cell) * 4 + (d & 3);
}
__device__ __forceinline__ size_t v_index(int head, int d, int cell, int hd, int kv_size) {
    return (((size_t) head * (kv_size / 4) + cell / 4) * hd + d) * 4 + (cell & 3);
}

// cos and sin of pair i's angle at position p: p * theta_scale^i, the power built by repeated
// multiplication (ggml's rope cache), then cosf / sinf.
__device__ __forceinline__ void rope_angle(float p, float theta_scale, int i, float &c, float &sn) {
    float theta = p;
    for (int s = 0; s < i; s++) theta *= theta_scale;
    c = cosf(theta);
    sn = sinf(theta);
}

__global__ __launch_bounds__(kWave) void rope_table_kernel(RopeParams P, float *cs) {
    const int t = blockIdx.x, half = P.hd / 2;
    const float p = (float) P.pos[t];
    for (int i = threadIdx.x; i < half; i += kWave) {
        float c, sn;
        rope_angle(p, P.theta_scale, i, c, sn);
        reinterpret_cast<float2 *>(cs)[(size_t) t * half + i] = make_float2(c, sn);
    }
}

// Head j (Q heads, then K heads, then V heads) of token t by one wavefront (lanes = threadIdx.x % 64).
// A Q head's rotated row goes to q_dst (hd floats) or, when that is null, to its row of P.q_out;
// with cells set, the wavefront also records the token's cell in the cell tables. Every load (the
// token's cell and position, the head's row, the norm weights, the step's cos / sin) is issued before
// the first use and every store comes after the last load, so the wavefront waits on one round trip.
constexpr int kRopeMaxPer = 4; // head dims per lane: hd <= 256
__device__ __forceinline__ void rope_head(const RopeParams &P, int t, int j, float *q_dst, bool cells) {
    const int lane = threadIdx.x & (kWave - 1);
    const int hd = P.hd, half = hd / 2;
    const int cell = P.cells[t], pos = P.pos[t];
    if (j >= P.n_head + P.n_kv) {
        const int head = j - P.n_head - P.n_kv;
        const float *src = P.v + (size_t) t * P.ld + head * hd;
        float v[kRopeMaxPer];
#pragma unroll
        for (int k = 0; k < kRopeMaxPer; k++) v[k] = lane + kWave * k < hd ? src[lane + kWave * k] : 0.0f;
        if (cells && lane == 0) {
            P.cell_seq[cell] = P.seq;
            P.cell_pos[cell] = pos;
        }
#pragma unroll
        for (int k = 0; k < kRopeMaxPer; k++) {
            const int d = lane + kWave * k;
            if (d < hd) P.vc[v_index(head, d, cell, hd, P.kv_size)] = f2h(v[k]);
        }
        return;
    }
    const bool is_q = j < P.n_head;
    const int head = is_q ? j : j - P.n_head;
    const float *src = (is_q ? P.q : P.k) + (size_t) t * P.ld + head * hd;
    const float *nw = is_q ? P.q_norm : P.k_norm;
    // the pairs (i, i + half) of the lane, i = lane + 64 m < half, with their norm weights and cos / sin
    constexpr int M = kRopeMaxPer / 2;
    float x0[M], x1[M], n0[M], n1[M], c[M], sn[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int i = min(lane + kWave * m, half - 1);
        x0[m] = src[i];
        x1[m] = src[i + half];
        n0[m] = nw ? nw[i] : 1.0f;
        n1[m] = nw ? nw[i + half] : 1.0f;
        c[m] = 1.0f;
        sn[m] = 0.0f;
        if (P.cs) {
            const float2 v = reinterpret_cast<const float2 *>(P.cs)[(size_t) t * half + i];
            c[m] = v.x;
            sn[m] = v.y;
        }
    }
    // the squares in the order d = lane, lane + 64, ... (d < hd)
    float v[kRopeMaxPer];
#pragma unroll
    for (int k = 0; k < kRopeMaxPer; k++) v[k] = lane + kWave * k < hd ? src[lane + kWave * k] : 0.0f;
    float scale = 1.0f;
    if (nw) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < kRopeMaxPer; k++)
            if (lane + kWave * k < hd) s += (double) (v[k] * v[k]);
        s = wave_sum_d(s);
        const float mean = (float) (s / (double) hd);
        scale = 1.0f / sqrtf(mean + P.eps);
    }
    if (cells && lane == 0) {
        P.cell_seq[cell] = P.seq;
        P.cell_pos[cell] = pos;
    }
    const float p = (float) pos;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int i = lane + kWave * m;
        if (i >= half) break;
        float a = x0[m], b = x1[m];
        if (nw) {
            a = (a * scale) * n0[m];
            b = (b * scale) * n1[m];
        }
        float cc = c[m], ss = sn[m];
        if (!P.cs) rope_angle(p, P.theta_scale, i, cc, ss);
        const float y0 = a * cc - b * ss;
        const float y1 = a * ss + b * cc;
        if (is_q && q_dst) {
            q_dst[i] = y0;
            q_dst[i + half] = y1;
        } else if (is_q) {
            uint16_t *dst = P.q_out + ((size_t) t * P.n_head + head) * hd;
            dst[i] = f2h(y0);
            dst[i + half] = f2h(y1);
        } else {
            P.kc[k_index(head, i, cell, hd, P.kv_size)] = f2h(y0);
            P.kc[k_index(head, i + half, cell, hd, P.kv_size)] = f2h(y1);
        }
    }
}

// One token's rotations for the attention prologue at head size 128 (one NEOX pair (i, i + 64) per
// lane), with the step's cos / sin table (R.cs): wavefront w rotates the query heads r = w, w + 4, ...
// (r < grp) of KV head g into s_q (row r), and with `owner` set wavefront 0 also rotates KV head g's K
// and wavefront 1 rounds its V, both as fp16 into s_kv (K at [0, 128), V at [128, 256)); the caller
// stores them into the cache. Each value is rope_head's, computed by the same expressions. All loads
// are unconditional and every head is computed branch-free (heads past grp from head grp - 1's row,
// not stored; absent norm weights read the query row, not applied), so the prologue's loads are in
// flight together and its first use waits for them only: after_loads() runs once they are issued,
// and the caller's own loads queue behind them.
constexpr int kRopeMaxQ = 4; // query heads per wavefront: grp <= 16
template <typename F>
__device__ __forceinline__ void rope_token_128(const RopeParams &R, int g, int grp, bool owner, float *s_q,
                                               uint16_t *s_kv, F after_loads) {
    constexpr int hd = 128, half = 64, K = kRopeMaxQ;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const bool do_k = owner && w == 0, do_v = owner && w == 1;
    float x0[K + 1], x1[K + 1];
#pragma unroll
    for (int i = 0; i < K; i++) {
        const float *src = R.q + (size_t) (g * grp + min(w + 4 * i, grp - 1)) * hd;
        x0[i] = src[lane];
        x1[i] = src[lane + half];
    }
    {
        const float *src = do_k ? R.k + (size_t) g * hd : do_v ? R.v + (size_t) g * hd : R.q;
        x0[K] = src[lane];
        x1[K] = src[lane + half];
    }
    const bool qn = R.q_norm != nullptr, kn = R.k_norm != nullptr;
    const float *qnw = qn ? R.q_norm : R.q, *knw = kn ? R.k_norm : R.q;
    const float qn0 = qnw[lane], qn1 = qnw[lane + half], kn0 = knw[lane], kn1 = knw[lane + half];
    const float2 csv = reinterpret_cast<const float2 *>(R.cs)[lane];
    asm volatile("" ::: "memory");
    after_loads();
    const float c = csv.x, sn = csv.y;
    float y0[K + 1], y1[K + 1];
#pragma unroll
    for (int i = 0; i <= K; i++) {
        float a = x0[i], b = x1[i];
        // QK-norm scale of the head from its lane pair, summed as rope_head sums it
        double ss = 0.0;
        ss += (double) (a * a);
        ss += (double) (b * b);
        ss = wave_sum_d(ss);
        const float mean = (float) (ss / (double) hd);
        const float scale = 1.0f / sqrtf(mean + R.eps);
        const bool use = i < K ? qn : kn;
        const float n0 = i < K ? qn0 : kn0, n1 = i < K ? qn1 : kn1;
        const float an = (a * scale) * n0, bn = (b * scale) * n1;
        a = use ? an : a;
        b = use ? bn : b;
        y0[i] = a * c - b * sn;
        y1[i] = a * sn + b * c;
    }
#pragma unroll
    for (int i = 0; i < K; i++) {
        const int r = w + 4 * i;
        if (r < grp) {
            s_q[r * hd + lane] = y0[i];
            s_q[r * hd + lane + half] = y1[i];
        }
    }
    if (do_k) {
        s_kv[lane] = f2h(y0[K]);
        s_kv[lane + half] = f2h(y1[K]);
    } else if (do_v) {
        s_kv[hd + lane] = f2h(x0[K]);
        s_kv[hd + lane + half] = f2h(x1[K]);
    }
}

__global__ __launch_bounds__(kWave) void rope_kernel(RopeParams P) {
    rope_head(P, blockIdx.x, blockIdx.y, nullptr, blockIdx.y == 0);
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
// single-token F16 GEMV: every load of a wavefront (the activation row, the norm weights, NJ =
// ceil(cols / 512) 16-byte chunks per lane of each of its RW rows, the residual values) is requested
// before anything waits; the activation row comes straight from memory into registers (no LDS, no
// barrier), optionally gathered from the embedding (EMB) and RMS-normalised on the way (NORM: one
// wavefront-wide double sum per wavefront, while the weight rows stream in).
// ------------------------------------------------------------------------------------------------

template <int NJ, int RW, bool NORM, bool EMB>
__global__ __launch_bounds__(kGvWaves *kWave) void gemv1_kernel(GemvParams P) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    const int cols = P.cols, nc = cols / 8;
    const int row0 = (blockIdx.x * kGvWaves + wv) * RW;
    // each row's matrix by comparison with the segment bounds (the parameters read at fixed indices,
    // so no address waits on a memory read); rows past the end read row 0 and store nothing
    const int b1 = P.seg[0].rows, b2 = b1 + (P.nseg > 1 ? P.seg[1].rows : 0);
    const uint4 *wr[RW];
    float *yr[RW];
    const float *ar[RW];
    bool on[RW];
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
        const int r = row0 + rr;
        on[rr] = r < P.rows_total;
        const int rc = on[rr] ? r : 0;
        const int s = (P.nseg > 1 && rc >= b1) + (P.nseg > 2 && rc >= b2);
        const int loc = rc - (s == 0 ? 0 : s == 1 ? b1 : b2);
        const uint16_t *w = s == 0 ? P.seg[0].w : s == 1 ? P.seg[1].w : P.seg[2].w;
        float *y = s == 0 ? P.seg[0].y : s == 1 ? P.seg[1].y : P.seg[2].y;
        const float *a = s == 0 ? P.seg[0].add : s == 1 ? P.seg[1].add : P.seg[2].add;
        wr[rr] = reinterpret_cast<const uint4 *>(w + (size_t) loc * cols);
        yr[rr] = y + loc;
        ar[rr] = a ? a + loc : nullptr;
    }
    // Every load is unconditional and issued up front, in the order of first use: the activation row
    // (or the embedding row) and the norm weights, then the weight rows (streamed while the row is
    // normalised), then the rows' residual values. Chunks past the row's end (c >= nc) load chunk
    // nc - 1 and use zero activations, so they add nothing.
    const uint16_t *e = EMB ? P.emb + (size_t) P.tokens[0] * cols : nullptr;
    float xv[NJ][8], nw[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int cc = min(lane + kWave * j, nc - 1);
        if constexpr (EMB) {
            const uint4 hv = reinterpret_cast<const uint4 *>(e)[cc];
            const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                xv[j][2 * q] = h2f(hw[q]);
                xv[j][2 * q + 1] = h2f(hw[q] >> 16);
            }
        } else {
            const float4 a = reinterpret_cast<const float4 *>(P.x)[2 * cc];
            const float4 b = reinterpret_cast<const float4 *>(P.x)[2 * cc + 1];
            xv[j][0] = a.x, xv[j][1] = a.y, xv[j][2] = a.z, xv[j][3] = a.w;
            xv[j][4] = b.x, xv[j][5] = b.y, xv[j][6] = b.z, xv[j][7] = b.w;
        }
        if constexpr (NORM) {
            const float4 a = reinterpret_cast<const float4 *>(P.norm_w)[2 * cc];
            const float4 b = reinterpret_cast<const float4 *>(P.norm_w)[2 * cc + 1];
            nw[j][0] = a.x, nw[j][1] = a.y, nw[j][2] = a.z, nw[j][3] = a.w;
            nw[j][4] = b.x, nw[j][5] = b.y, nw[j][6] = b.z, nw[j][7] = b.w;
        }
    }
    uint4 w[RW][NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int cc = min(lane + kWave * j, nc - 1);
#pragma unroll
        for (int rr = 0; rr < RW; rr++) w[rr][j] = load_weights(wr[rr] + cc);
    }
    float addv[RW];
#pragma unroll
    for (int rr = 0; rr < RW; rr++) addv[rr] = *(ar[rr] ? ar[rr] : yr[rr]);
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        if (lane + kWave * j >= nc) {
#pragma unroll
            for (int q = 0; q < 8; q++) xv[j][q] = 0.0f;
        }
    }
    float xraw[EMB ? NJ : 1][8];
    if constexpr (EMB) {
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int q = 0; q < 8; q++) xraw[j][q] = xv[j][q];
    }
    if constexpr (NORM) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int q = 0; q < 8; q++) s += (double) (xv[j][q] * xv[j][q]);
        s = wave_sum_d(s);
        const float mean = (float) (s / (double) cols);
        const float scale = 1.0f / sqrtf(mean + P.eps);
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int q = 0; q < 8; q++) xv[j][q] = (xv[j][q] * scale) * nw[j][q];
    }
    float acc[RW];
#pragma unroll
    for (int rr = 0; rr < RW; rr++) acc[rr] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint4 xh = make_uint4(pack2(xv[j][0], xv[j][1]), pack2(xv[j][2], xv[j][3]), pack2(xv[j][4], xv[j][5]),
                                    pack2(xv[j][6], xv[j][7]));
#pragma unroll
        for (int rr = 0; rr < RW; rr++) acc[rr] = dot8(w[rr][j], xh, acc[rr]);
    }
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
        const float sum = wave_sum_tree(acc[rr]);
        if (lane == 0 && on[rr]) yr[rr][0] = ar[rr] ? sum + addv[rr] : sum;
    }
    if constexpr (EMB) {
        // the gathered embedding row is the layer's residual input (written once, by work-group 0)
        if (blockIdx.x == 0 && wv == 0) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int c = lane + kWave * j;
                if (c < nc) {
                    reinterpret_cast<float4 *>(P.x_out)[2 * c] = make_float4(xraw[j][0], xraw[j][1], xraw[j][2], xraw[j][3]);
                    reinterpret_cast<float4 *>(P.x_out)[2 * c + 1] = make_float4(xraw[j][4], xraw[j][5], xraw[j][6], xraw[j][7]);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// F16 projection of a few tokens on the matrix cores (v_mfma_f32_16x16x32_f16). Work-group = rw weight
// rows (NRT 16-row tiles, the last one padded with rows that are neither loaded nor stored) x all T
// tokens (16-token tiles); rw is the matrix's rows over the work-groups of one wave of the device, so
// every CU streams the same bytes. Its KS wavefronts split K in interleaved 64-value steps, SPW steps
// each, and every wavefront requests all of its weight and activation chunks before its first product.
// Per step, lane (r = l % 16, q = l / 16) loads the 32 contiguous bytes [16 q, 16 q + 16) (in halves) of
// weight row r and of token row r, and product i takes halves [8 i, 8 i + 8) of them: A and B pair the
// same K index in every slot, and each row's 128-byte line is read whole by its four lanes. The KS
// partial 16 x 16 tiles are summed in LDS in wavefront order.
// ------------------------------------------------------------------------------------------------

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int KS, int SPW, int NTILE, int NRT>
__global__ __launch_bounds__(KS *kWave) void gemm16_kernel(Gemm16Params P) {
    __shared__ f32x4v s_red[KS][kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * P.rw;
    const uint4 *wrow[NRT];
    bool won[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        won[rt] = rt * 16 + r < P.rw;
        wrow[rt] = reinterpret_cast<const uint4 *>(P.w + (size_t) (n0 + min(rt * 16 + r, P.rw - 1)) * P.cols) + 2 * q;
    }
    const uint4 *xrow[NTILE];
#pragma unroll
    for (int nt = 0; nt < NTILE; nt++)
        xrow[nt] = reinterpret_cast<const uint4 *>(P.x + (size_t) min(nt * 16 + r, P.T - 1) * P.cols) + 2 * q;
    // a 64-value step is 8 uint4 of a row; this lane's 2 of step s are uint4 8 s + 2 q, + 1
    uint4 wv[NRT][SPW][2], xv[NTILE][SPW][2];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int j = 0; j < SPW; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                wv[rt][j][i] = won[rt] ? load_weights(wrow[rt] + 8 * (w + KS * j) + i) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int nt = 0; nt < NTILE; nt++)
#pragma unroll
        for (int j = 0; j < SPW; j++)
#pragma unroll
            for (int i = 0; i < 2; i++) xv[nt][j][i] = xrow[nt][8 * (w + KS * j) + i];
    __builtin_amdgcn_sched_barrier(0); // every load above is issued before the first product waits
    f32x4v acc[NRT][NTILE];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int nt = 0; nt < NTILE; nt++) acc[rt][nt] = f32x4v{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < SPW; j++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int rt = 0; rt < NRT; rt++) {
                const half8v a = __builtin_bit_cast(half8v, wv[rt][j][i]);
#pragma unroll
                for (int nt = 0; nt < NTILE; nt++)
                    acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8v, xv[nt][j][i]), acc[rt][nt], 0,
                                                                         0, 0);
            }
    // element e of lane l: weight row n0 + 16 rt + 4 (l / 16) + e, token nt * 16 + l % 16
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int nt = 0; nt < NTILE; nt++) {
            s_red[w][lane] = acc[rt][nt];
            __syncthreads();
            for (int idx = threadIdx.x; idx < 4 * kWave; idx += KS * kWave) {
                const int e = idx / kWave, l = idx % kWave;
                float v = s_red[0][l][e];
#pragma unroll
                for (int ww = 1; ww < KS; ww++) v += s_red[ww][l][e];
                const int t = nt * 16 + (l & 15), rr = rt * 16 + 4 * (l >> 4) + e;
                if (t < P.T && rr < P.rw) {
                    float *y = P.y + (size_t) t * P.ldy + n0 + rr;
                    *y = P.accumulate ? v + *y : v;
                }
            }
            __syncthreads();
        }
}

// ------------------------------------------------------------------------------------------------
// attention on the matrix cores. Work-group (rb, c, g): up to 64 query rows (the query heads of KV head
// g times the step's tokens) against its chunk of cells, 64 cells per pass:
//   S = Q K^T   wavefront w owns cells [16 w, 16 w + 16) of the pass: HD / 16 products per 16-row tile,
//               K fragments loaded straight from the cache (one 8-byte load per lane per product);
//   softmax     4 threads per row over the pass's 64 cells, online across passes (running max, sum and a
//               rescale factor per row in LDS);
//   O += P V    wavefront w owns output dims [16 HD/64 w, ...): P is split into fp16 hi + lo parts
//               (p = hi + lo to 2^-22), both multiplied by the V fragments, so the product keeps the
//               f32 precision of the probabilities; V fragments are requested at the start of the pass.
// Q and K enter as fp16 (Q rounded, as ggml rounds Q to F16 for F16 K), all accumulation is f32.
// ------------------------------------------------------------------------------------------------

typedef _Float16 half4v __attribute__((ext_vector_type(4)));
constexpr int kFaCells = 64;
constexpr int kAttnSkipMinT = 64;    // steps of at least this many tokens skip passes with no cell of the sequence
constexpr int kAttnMaxPasses = 2048; // passes per chunk the skip map covers (131072 cells)
constexpr int kAttnOneChunkWgs = 256; // row-block work-groups from which a many-token step keeps one chunk

__device__ __forceinline__ f32x4v mfma16(half4v a, half4v b, f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half4v ld_half4(const uint16_t *p) {
    return __builtin_bit_cast(half4v, *reinterpret_cast<const uint2 *>(p));
}

// (The single-token launch at head size 128 with grp <= 16 is attn1_kernel below.)
template <int HD, int NRT, bool SKIP = false>
__global__ __launch_bounds__(kAtBlock) void attn_kernel(AttnParams P) {
    constexpr int NK = HD / 16, DT = NK / 4, RB = 16 * NRT, PS = kFaCells + 8; // P row stride (halves)
    __shared__ float s_S[RB][kFaCells];
    __shared__ uint16_t s_Ph[RB][PS], s_Pl[RB][PS];
    __shared__ float s_M[RB], s_L[RB], s_f[RB];
    __shared__ int s_pos[RB];
    __shared__ float s_q[NRT == 1 ? 16 * HD : 1]; // rotated Q rows when this launch applies RoPE
    const int tid = threadIdx.x, w = tid / kWave, l = tid & (kWave - 1), lr = l & 15, lq = l >> 4;
    const int grp = P.n_head / P.n_kv;
    const int g = blockIdx.x % P.n_kv, rest = blockIdx.x / P.n_kv;
    const int c = rest % P.n_chunk, rb = rest / P.n_chunk;
    const int row0 = rb * P.rb_rows, rows = P.T * grp;
    if (tid < RB) {
        const int r = row0 + tid;
        s_pos[tid] = r < rows ? P.pos[r / grp] : -1;
        s_M[tid] = -INFINITY;
        s_L[tid] = 0.0f;
    }
    const int begin = P.cell_begin + c * P.chunk, end = min(begin + P.chunk, P.n_cells), last4 = P.kv_size - 4;
    const bool rope_in = NRT == 1 && P.rope_in;
    const int cell0 = rope_in ? P.rope.cells[0] : -1;
    const bool owner = cell0 >= begin && cell0 < end;
    // The first pass's K / V fragments and cell-table entries are requested before the prologue, except
    // by a work-group that stores the new cell in its prologue and then reads it back (late).
    const bool late = rope_in && owner;
    const uint16_t *kb = P.kc + (size_t) g * (HD / 4) * P.kv_size * 4;
    half4v vf[4][DT]; // V fragments of a pass (B operand of O += P V): cells kc*16 + 4 lq .. +3, dim (w*DT + dt)*16 + lr
    half4v kf[NK];    // K fragments of the wavefront's 16 cells
    int cseq, cpos0;  // cell-table entries of the lane's cell
    auto load_pass = [&](int c0) {
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            const int cg = min(c0 + kc * 16 + 4 * lq, last4);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) vf[kc][dt] = ld_half4(P.vc + v_index(g, (w * DT + dt) * 16 + lr, cg, HD, P.kv_size));
        }
        const int cc = min(c0 + 16 * w + lr, P.kv_size - 1);
#pragma unroll
        for (int ks = 0; ks < NK; ks++) kf[ks] = ld_half4(kb + ((size_t) (ks * 4 + lq) * P.kv_size + cc) * 4);
        cseq = P.cell_seq[cc];
        cpos0 = P.cell_pos[cc];
    };
    // one token: every work-group rotates its own query rows (rope_kernel's work, bit for bit); the
    // work-group whose chunk holds the token's cell also computes that cell's K and V of KV head g and
    // stores them into the cache with its cell-table entries
    if (!late) load_pass(begin);
    if (rope_in) {
        if (owner) {
            if (w == 0) rope_head(P.rope, 0, P.n_head + g, nullptr, true);
            else if (w == 1) rope_head(P.rope, 0, P.n_head + P.n_kv + g, nullptr, false);
        }
        for (int r = w; r < grp; r += kAtBlock / kWave) rope_head(P.rope, 0, g * grp + r, s_q + r * HD, false);
        __syncthreads();
    }
    // Q fragments (A operand): row rt*16 + lr, dims ks*16 + 4 lq .. +3
    half4v qa[NRT][NK];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        const int r = row0 + rt * 16 + lr;
        const bool on = r < rows;
        const int rc = on ? r : rows - 1; // rows past the end load the last row (unconditional loads) and use zeros
        // (a RoPE-in launch is one token in one row block: its live rows r < grp are the heads themselves)
        if (rope_in) {
            const float *q = s_q + rc * HD;
#pragma unroll
            for (int ks = 0; ks < NK; ks++) {
                float4 v = *reinterpret_cast<const float4 *>(q + ks * 16 + 4 * lq);
                v = on ? v : make_float4(0, 0, 0, 0);
                qa[rt][ks] = half4v{(_Float16) v.x, (_Float16) v.y, (_Float16) v.z, (_Float16) v.w};
            }
        } else {
            // fp16 rows straight into the operand registers (the rotation kernel rounded them)
            const uint16_t *q = P.q + ((size_t) (rc / grp) * P.n_head + g * grp + rc % grp) * HD;
#pragma unroll
            for (int ks = 0; ks < NK; ks++) {
                const half4v v = ld_half4(q + ks * 16 + 4 * lq);
                qa[rt][ks] = on ? v : half4v{0, 0, 0, 0};
            }
        }
    }
    f32x4v O[NRT][DT];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[rt][dt] = f32x4v{0, 0, 0, 0};
    // A step of many tokens skips the chunk's passes that hold no cell of the sequence (cells of other
    // or removed sequences, e.g. when the sequence's blocks sit high in the cache): such a pass would
    // leave the running max, sum and output exactly as they are (every score -inf: sum 0, factor 1, or
    // 0 while nothing is live and the output is still zero). The cell table is current here: the step's
    // RoPE launch wrote the new cells' entries. A wavefront's 64 lanes read one pass's 64 entries, eight
    // passes per wavefront in flight.
    const int n_pass = (end - begin + kFaCells - 1) / kFaCells;
    const bool skip = SKIP && !rope_in && n_pass <= kAttnMaxPasses;
    __shared__ uint8_t s_live[SKIP ? kAttnMaxPasses : 1];
    if (skip) {
        for (int p0 = 0; p0 < n_pass; p0 += 8 * (kAtBlock / kWave)) {
            int cs[8];
#pragma unroll
            for (int u = 0; u < 8; u++) cs[u] = P.cell_seq[min(begin + (p0 + u * (kAtBlock / kWave) + w) * kFaCells + l, P.kv_size - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int pass = p0 + u * (kAtBlock / kWave) + w;
                const bool mine = cs[u] == P.seq && begin + pass * kFaCells + l < end;
                const bool any = __ballot(mine) != 0ull;
                if (l == 0 && pass < n_pass) s_live[pass] = any ? 1 : 0;
            }
        }
    }
    __syncthreads();

    for (int c0 = begin; c0 < end; c0 += kFaCells) {
        if (skip && !s_live[(c0 - begin) / kFaCells]) continue; // uniform: the whole work-group reads one byte
        if (c0 != begin || late) load_pass(c0);
        // S = Q K^T for this wavefront's 16 cells
        const int cell = c0 + 16 * w + lr;
        const bool live = cell < end && cseq == P.seq;
        const int cpos = cpos0;
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
            f32x4v sacc = f32x4v{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < NK; ks++) sacc = mfma16(qa[rt][ks], kf[ks], sacc);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = rt * 16 + 4 * lq + v;
                const bool vis = live && s_pos[r] >= 0 && cpos <= s_pos[r];
                s_S[r][16 * w + lr] = vis ? sacc[v] * P.scale : -INFINITY;
            }
        }
        __syncthreads();
        if (NRT == 1) {
            // online softmax of one 16-row tile: 16 threads per row, 4 cells each
            const int r = tid >> 4, part = tid & 15;
            float sv[4];
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[i] = s_S[r][part * 4 + i];
                m = fmaxf(m, sv[i]);
            }
            m = fmaxf(m, dpp_f<0xB1>(m)); // the 16 lanes of the row (DPP row): pairs, quads, octets, halves
            m = fmaxf(m, dpp_f<0x4E>(m));
            m = fmaxf(m, dpp_f<0x141>(m));
            m = fmaxf(m, dpp_f<0x140>(m));
            const float m_old = s_M[r], m_new = fmaxf(m_old, m);
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - m_new);
                const _Float16 hi = (_Float16) p;
                const _Float16 lo = (_Float16) (p - (float) hi);
                s_Ph[r][part * 4 + i] = __builtin_bit_cast(uint16_t, hi);
                s_Pl[r][part * 4 + i] = __builtin_bit_cast(uint16_t, lo);
                sum += p;
            }
            sum += dpp_f<0xB1>(sum);
            sum += dpp_f<0x4E>(sum);
            sum += dpp_f<0x141>(sum);
            sum += dpp_f<0x140>(sum);
            if (part == 0) {
                const float f = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
                s_f[r] = f;
                s_L[r] = s_L[r] * f + sum;
                s_M[r] = m_new;
            }
        } else {
            // online softmax: 4 threads per row, 16 cells each
            const int r = tid >> 2, part = tid & 3;
            if (r < RB) {
                float sv[16];
                float m = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    sv[i] = s_S[r][part * 16 + i];
                    m = fmaxf(m, sv[i]);
                }
                m = fmaxf(m, dpp_f<0xB1>(m)); // lanes l ^ 1, then l ^ 2
                m = fmaxf(m, dpp_f<0x4E>(m));
                const float m_old = s_M[r], m_new = fmaxf(m_old, m);
                float sum = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float p = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - m_new);
                    const _Float16 hi = (_Float16) p;
                    const _Float16 lo = (_Float16) (p - (float) hi);
                    s_Ph[r][part * 16 + i] = __builtin_bit_cast(uint16_t, hi);
                    s_Pl[r][part * 16 + i] = __builtin_bit_cast(uint16_t, lo);
                    sum += p;
                }
                sum += dpp_f<0xB1>(sum);
                sum += dpp_f<0x4E>(sum);
                if (part == 0) {
                    const float f = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
                    s_f[r] = f;
                    s_L[r] = s_L[r] * f + sum;
                    s_M[r] = m_new;
                }
            }
        }
        __syncthreads();
        // O = O * f + P V
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float f = s_f[rt * 16 + 4 * lq + v];
#pragma unroll
                for (int dt = 0; dt < DT; dt++) O[rt][dt][v] *= f;
            }
#pragma unroll
            for (int kc = 0; kc < 4; kc++) {
                const half4v ph = ld_half4(&s_Ph[rt * 16 + lr][kc * 16 + 4 * lq]);
                const half4v pl = ld_half4(&s_Pl[rt * 16 + lr][kc * 16 + 4 * lq]);
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    O[rt][dt] = mfma16(ph, vf[kc][dt], O[rt][dt]);
                    O[rt][dt] = mfma16(pl, vf[kc][dt], O[rt][dt]);
                }
            }
        }
        __syncthreads();
    }
    // rows of this lane: rt*16 + 4 lq + v, dims (w*DT + dt)*16 + lr; row r is query head r % grp of
    // token r / grp, stepped from the first row's quotient instead of divided per row
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        const int r0 = row0 + rt * 16 + 4 * lq;
        int tq = r0 / grp, hq = r0 - tq * grp;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int rl = rt * 16 + 4 * lq + v, r = row0 + rl;
            const int t = tq, h = g * grp + hq;
            if (++hq == grp) {
                hq = 0;
                ++tq;
            }
            if (r >= rows) continue;
            if (P.n_chunk == 1) {
                const float inv_l = s_L[rl];
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const size_t o = ((size_t) t * P.n_head + h) * HD + (w * DT + dt) * 16 + lr;
                    const float y = O[rt][dt][v] / inv_l;
                    P.out[o] = y;
                    if (P.out16) P.out16[o] = f2h(y);
                }
            } else {
                float *pp = P.part + (((size_t) t * P.n_head + h) * P.n_chunk + c) * (HD + 4);
#pragma unroll
                for (int dt = 0; dt < DT; dt++) pp[4 + (w * DT + dt) * 16 + lr] = O[rt][dt][v];
                if (w == 0 && lr == 0) {
                    pp[0] = s_M[rl];
                    pp[1] = s_L[rl];
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Single-token attention at head size 128 with RoPE inside (grp <= 16 query heads per KV head): each
// wavefront runs its own 16 cells of the work-group's chunk (16 cells per wavefront) from registers to registers, so
// the pass has no barrier and no LDS round trip. With the K fragments as the A operand and the query
// rows as the B operand the product comes out transposed, S^T [cell][row]: lane (row j, quad q) holds
// cells 4q .. 4q + 3 of row j, which is exactly the B operand of O^T = V^T P^T (and the V fragments
// of the cache are the A operand as they stand). A row's softmax state and output stay in the lanes
// of that row; the row's max over its 16 cells takes two lane exchanges (quads 0-3). At the end the
// wavefronts' (max, sum, output) rows are merged through LDS, and the merged row is the chunk's
// partial (or, with one chunk, the output). Probabilities enter the product as fp16 hi + lo parts
// (p = hi + lo to 2^-22), Q and K as fp16, all accumulation in f32, as in attn_kernel.
// ------------------------------------------------------------------------------------------------
constexpr int kA1Cells = 16; // cells per wavefront; a work-group of NW = 4, 5 or 6 wavefronts covers a chunk of 16 NW cells
__device__ __forceinline__ float xor_lanes(float v, int m) { return __shfl_xor(v, m, kWave); }

template <int NW>
__global__ __launch_bounds__(NW *kWave) void attn1_kernel(AttnParams P) {
    constexpr int HD = 128, NK = HD / 16, RS = HD + 4;
    __shared__ float s_q[16 * HD];
    __shared__ __align__(8) uint16_t s_kv[2 * HD];
    __shared__ __align__(16) float s_o[NW][16][RS];
    __shared__ float s_m[NW][16], s_l[NW][16];
    const int tid = threadIdx.x, w = tid / kWave, l = tid & (kWave - 1), lr = l & 15, lq = l >> 4;
    const int grp = P.n_head / P.n_kv;
    const int g = blockIdx.x % P.n_kv, c = blockIdx.x / P.n_kv;
    const int begin = P.cell_begin + c * P.chunk, end = min(begin + P.chunk, P.n_cells);
    const int cell0 = P.rope.cells[0], pos = P.rope.pos[0];
    const bool owner = cell0 >= begin && cell0 < end;
    const int wb = begin + w * kA1Cells; // this wavefront's cells [wb, wb + 16)
    const uint16_t *kb = P.kc + (size_t) g * (HD / 4) * P.kv_size * 4;
    half4v kf[NK]; // A operand of S^T: cell wb + lr, dims ks*16 + 4 lq .. +3
    half4v vf[NK]; // A operand of O^T: dim dt*16 + lr, cells wb + 4 lq .. +3
    int4 cseq, cpos; // cell-table entries of cells wb + 4 lq .. +3
    auto loads = [&] {
        const int ck = min(wb + lr, P.kv_size - 1), cv = min(wb + 4 * lq, P.kv_size - 4);
#pragma unroll
        for (int ks = 0; ks < NK; ks++) kf[ks] = ld_half4(kb + ((size_t) (ks * 4 + lq) * P.kv_size + ck) * 4);
#pragma unroll
        for (int dt = 0; dt < NK; dt++) vf[dt] = ld_half4(P.vc + v_index(g, dt * 16 + lr, cv, HD, P.kv_size));
        cseq = *reinterpret_cast<const int4 *>(P.cell_seq + cv);
        cpos = *reinterpret_cast<const int4 *>(P.cell_pos + cv);
    };
    // wavefronts 0-3 rotate the query rows (heads w, w + 4, ...; K / V of the owner's token by 0 and 1);
    // any further ones only issue their loads
    if (w < 4) rope_token_128(P.rope, g, grp, owner, s_q, s_kv, loads);
    else loads();
    __syncthreads();
    // B operand of S^T: query row lr (zero past grp), dims ks*16 + 4 lq .. +3
    half4v qb[NK];
#pragma unroll
    for (int ks = 0; ks < NK; ks++) {
        const float4 v = *reinterpret_cast<const float4 *>(s_q + min(lr, grp - 1) * HD + ks * 16 + 4 * lq);
        qb[ks] = lr < grp ? half4v{(_Float16) v.x, (_Float16) v.y, (_Float16) v.z, (_Float16) v.w} : half4v{0, 0, 0, 0};
    }
    // the token's own cell: K and V from LDS (the cache gets them at the end), visible to the token
    if (owner) {
        if (wb + lr == cell0) {
#pragma unroll
            for (int ks = 0; ks < NK; ks++) kf[ks] = ld_half4(&s_kv[(ks * 4 + lq) * 4]);
        }
        const int d = cell0 - (wb + 4 * lq);
        if (d >= 0 && d < 4) {
#pragma unroll
            for (int dt = 0; dt < NK; dt++) vf[dt][d] = __builtin_bit_cast(_Float16, s_kv[HD + dt * 16 + lr]);
        }
    }
    f32x4v s = f32x4v{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < NK; ks++) s = mfma16(kf[ks], qb[ks], s);
    const int cs[4] = {cseq.x, cseq.y, cseq.z, cseq.w}, cp[4] = {cpos.x, cpos.y, cpos.z, cpos.w};
    float sv[4];
    float m = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int cell = wb + 4 * lq + v;
        const bool vis = cell < end && ((cs[v] == P.seq && cp[v] <= pos) || (owner && cell == cell0));
        sv[v] = vis ? s[v] * P.scale : -INFINITY;
        m = fmaxf(m, sv[v]);
    }
    m = fmaxf(m, xor_lanes(m, 16));
    m = fmaxf(m, xor_lanes(m, 32));
    float lsum = 0.0f;
    half4v ph, pl;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const float p = sv[v] == -INFINITY ? 0.0f : expf(sv[v] - m);
        ph[v] = (_Float16) p;
        pl[v] = (_Float16) (p - (float) ph[v]);
        lsum += p;
    }
    lsum += xor_lanes(lsum, 16);
    lsum += xor_lanes(lsum, 32);
    f32x4v o[NK];
#pragma unroll
    for (int dt = 0; dt < NK; dt++) {
        o[dt] = mfma16(vf[dt], ph, f32x4v{0, 0, 0, 0});
        o[dt] = mfma16(vf[dt], pl, o[dt]);
    }
    // lane (row lr, quad lq) holds dims dt*16 + 4 lq .. +3 of row lr
    if (lq == 0) {
        s_m[w][lr] = m;
        s_l[w][lr] = lsum;
    }
#pragma unroll
    for (int dt = 0; dt < NK; dt++) *reinterpret_cast<f32x4v *>(&s_o[w][lr][dt * 16 + 4 * lq]) = o[dt];
    __syncthreads();
    // merge the wavefronts: thread (row r, dims 4 dq .. +3)
    for (int i = tid; i < grp * (HD / 4); i += NW * kWave) {
        const int r = i / (HD / 4), dq = i % (HD / 4), h = g * grp + r;
        float M = s_m[0][r];
#pragma unroll
        for (int u = 1; u < NW; u++) M = fmaxf(M, s_m[u][r]);
        float L = 0.0f;
        float4 acc = make_float4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < NW; u++) {
            const float f = s_m[u][r] == -INFINITY ? 0.0f : expf(s_m[u][r] - M);
            const float4 ov = *reinterpret_cast<const float4 *>(&s_o[u][r][4 * dq]);
            L += s_l[u][r] * f;
            acc.x += ov.x * f;
            acc.y += ov.y * f;
            acc.z += ov.z * f;
            acc.w += ov.w * f;
        }
        if (P.n_chunk == 1) {
            const float4 y = make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L);
            *reinterpret_cast<float4 *>(P.out + (size_t) h * HD + 4 * dq) = y;
            if (P.out16) {
                uint16_t *o16 = P.out16 + (size_t) h * HD + 4 * dq;
                *reinterpret_cast<uint2 *>(o16) = make_uint2(pack2(y.x, y.y), pack2(y.z, y.w));
            }
        } else {
            float *pp = P.part + ((size_t) h * P.n_chunk + c) * RS;
            *reinterpret_cast<float4 *>(pp + 4 + 4 * dq) = acc;
            if (dq == 0) {
                pp[0] = M;
                pp[1] = L;
            }
        }
    }
    if (owner && w < 2) {
        // the new cell into the cache (read by later launches only): K and the cell tables by
        // wavefront 0, V by wavefront 1
        const RopeParams &R = P.rope;
        if (w == 0) {
            if (l == 0) {
                R.cell_seq[cell0] = R.seq;
                R.cell_pos[cell0] = pos;
            }
            R.kc[k_index(g, l, cell0, HD, R.kv_size)] = s_kv[l];
            R.kc[k_index(g, l + HD / 2, cell0, HD, R.kv_size)] = s_kv[l + HD / 2];
        } else {
            R.vc[v_index(g, l, cell0, HD, R.kv_size)] = s_kv[HD + l];
            R.vc[v_index(g, l + HD / 2, cell0, HD, R.kv_size)] = s_kv[HD + l + HD / 2];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Attention of 64-row blocks (steps of many tokens): wavefront w owns query rows row0 + 16 w .. + 15
// over the whole chunk and runs them from registers to registers as attn1_kernel does (S^T = K Q^T puts
// a row's scores in that row's lanes, the online softmax stays there, O^T += V^T P^T with P as fp16
// hi + lo). The K and V fragments of each 64-cell block (and its cell-table entries) are loaded once
// per work-group, wavefront w fetching those of cells 16 w .. 16 w + 15, into LDS, where all four
// wavefronts read them; the next live block's loads are in flight while a block is multiplied. Two
// barriers per 64-cell block; no score or probability goes through LDS.
// ------------------------------------------------------------------------------------------------
template <int HD, bool SKIP>
__global__ __launch_bounds__(kAtBlock) void attn_rows_kernel(AttnParams P) {
    constexpr int NK = HD / 16;
    __shared__ __align__(16) half4v s_k[4][NK][kWave];
    __shared__ __align__(16) half4v s_v[4][NK][kWave];
    __shared__ __align__(16) int s_cs[kFaCells], s_cp[kFaCells];
    __shared__ uint8_t s_live[SKIP ? kAttnMaxPasses : 1];
    const int tid = threadIdx.x, w = tid / kWave, l = tid & (kWave - 1), lr = l & 15, lq = l >> 4;
    const int grp = P.n_head / P.n_kv;
    const int g = blockIdx.x % P.n_kv, rest = blockIdx.x / P.n_kv;
    const int c = rest % P.n_chunk, rb = rest / P.n_chunk;
    const int rows = P.T * grp;
    const int begin = P.cell_begin + c * P.chunk, end = min(begin + P.chunk, P.n_cells);
    const int n_pass = (end - begin + kFaCells - 1) / kFaCells;
    const uint16_t *kb = P.kc + (size_t) g * (HD / 4) * P.kv_size * 4;
    // the lane's query row: row lr of the wavefront's tile (B operand of S^T); rows past the end read
    // the last row, see no cell and store nothing
    const int r = rb * 64 + 16 * w + lr;
    const bool on = r < rows;
    const int rc = on ? r : rows - 1;
    const int t = rc / grp, h = g * grp + rc % grp;
    const int pos = on ? P.pos[t] : -1;
    half4v kr[NK], vr[NK]; // this wavefront's share of a block: K of cell 16 w + lr, V of cells 16 w + 4 lq ..
    int ctr;               // lanes 0-15: cell_seq of cell 16 w + lane, 16-31: cell_pos of cell 16 w + lane - 16
    auto load_block = [&](int b0) {
        const int ck = min(b0 + 16 * w + lr, P.kv_size - 1), cv = min(b0 + 16 * w + 4 * lq, P.kv_size - 4);
#pragma unroll
        for (int ks = 0; ks < NK; ks++) kr[ks] = ld_half4(kb + ((size_t) (ks * 4 + lq) * P.kv_size + ck) * 4);
#pragma unroll
        for (int dt = 0; dt < NK; dt++) vr[dt] = ld_half4(P.vc + v_index(g, dt * 16 + lr, cv, HD, P.kv_size));
        const int ct = min(b0 + 16 * w + (l & 15), P.kv_size - 1);
        ctr = l < 16 ? P.cell_seq[ct] : P.cell_pos[ct];
    };
    // A step of many tokens skips the chunk's passes that hold no cell of the sequence (attn_kernel's map)
    const bool skip = SKIP && n_pass <= kAttnMaxPasses;
    if (skip) {
        for (int p0 = 0; p0 < n_pass; p0 += 8 * (kAtBlock / kWave)) {
            int cs[8];
#pragma unroll
            for (int u = 0; u < 8; u++) cs[u] = P.cell_seq[min(begin + (p0 + u * (kAtBlock / kWave) + w) * kFaCells + l, P.kv_size - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int pass = p0 + u * (kAtBlock / kWave) + w;
                const bool mine = cs[u] == P.seq && begin + pass * kFaCells + l < end;
                const bool any = __ballot(mine) != 0ull;
                if (l == 0 && pass < n_pass) s_live[pass] = any ? 1 : 0;
            }
        }
    }
    half4v qb[NK];
    const uint16_t *q = P.q + ((size_t) t * P.n_head + h) * HD;
#pragma unroll
    for (int ks = 0; ks < NK; ks++) {
        const half4v v = ld_half4(q + ks * 16 + 4 * lq);
        qb[ks] = on ? v : half4v{0, 0, 0, 0};
    }
    __syncthreads(); // the skip map
    auto next_live = [&](int p) {
        if (skip)
            while (p < n_pass && !s_live[p]) p++;
        return p;
    };
    int p = next_live(0);
    load_block(begin + min(p, n_pass - 1) * kFaCells);
    float m_run = -INFINITY, l_run = 0.0f;
    f32x4v o[NK];
#pragma unroll
    for (int dt = 0; dt < NK; dt++) o[dt] = f32x4v{0, 0, 0, 0};
    while (p < n_pass) {
        const int b0 = begin + p * kFaCells;
        __syncthreads(); // every wavefront is done with the previous block's fragments
#pragma unroll
        for (int ks = 0; ks < NK; ks++) s_k[w][ks][l] = kr[ks];
#pragma unroll
        for (int dt = 0; dt < NK; dt++) s_v[w][dt][l] = vr[dt];
        if (l < 16) s_cs[16 * w + l] = ctr;
        else if (l < 32) s_cp[16 * w + l - 16] = ctr;
        __syncthreads();
        const int pn = next_live(p + 1);
        load_block(begin + min(pn, n_pass - 1) * kFaCells); // unconditional: the last block again past the end
        // the block's four 16-cell groups together: S^T of each (four independent product chains), one
        // softmax step over the 64 cells, then O^T += V^T P^T over the groups (eight chains, one per dim tile)
        f32x4v sc[4];
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            sc[kc] = f32x4v{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < NK; ks++) sc[kc] = mfma16(s_k[kc][ks][l], qb[ks], sc[kc]);
        }
        float sv[4][4];
        float mt = -INFINITY;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            const int4 cs = *reinterpret_cast<const int4 *>(&s_cs[16 * kc + 4 * lq]);
            const int4 cp = *reinterpret_cast<const int4 *>(&s_cp[16 * kc + 4 * lq]);
            const int csv[4] = {cs.x, cs.y, cs.z, cs.w}, cpv[4] = {cp.x, cp.y, cp.z, cp.w};
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const bool vis = b0 + 16 * kc + 4 * lq + v < end && csv[v] == P.seq && cpv[v] <= pos;
                sv[kc][v] = vis ? sc[kc][v] * P.scale : -INFINITY;
                mt = fmaxf(mt, sv[kc][v]);
            }
        }
        mt = fmaxf(mt, xor_lanes(mt, 16));
        mt = fmaxf(mt, xor_lanes(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        // the rescale by e^(m_run - m_new) only when some row's max moved (otherwise every factor is 1)
        if (__ballot(m_new != m_run) != 0ull) { // wavefront-uniform
            const float f = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
            l_run *= f;
#pragma unroll
            for (int dt = 0; dt < NK; dt++) o[dt] *= f;
        }
        m_run = m_new;
        float ps = 0.0f;
        half4v ph[4], pl[4];
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float pv = sv[kc][v] == -INFINITY ? 0.0f : expf(sv[kc][v] - m_new);
                ph[kc][v] = (_Float16) pv;
                pl[kc][v] = (_Float16) (pv - (float) ph[kc][v]);
                ps += pv;
            }
        }
        l_run += ps;
#pragma unroll
        for (int dt = 0; dt < NK; dt++) {
#pragma unroll
            for (int kc = 0; kc < 4; kc++) {
                const half4v vf = s_v[kc][dt][l];
                o[dt] = mfma16(vf, ph[kc], o[dt]);
                o[dt] = mfma16(vf, pl[kc], o[dt]);
            }
        }
        p = pn;
    }
    l_run += xor_lanes(l_run, 16);
    l_run += xor_lanes(l_run, 32);
    if (!on) return;
    // lane (row lr, quad lq) holds dims dt*16 + 4 lq .. +3 of its row
    if (P.n_chunk == 1) {
#pragma unroll
        for (int dt = 0; dt < NK; dt++) {
            const size_t oi = ((size_t) t * P.n_head + h) * HD + dt * 16 + 4 * lq;
            const float4 y = make_float4(o[dt][0] / l_run, o[dt][1] / l_run, o[dt][2] / l_run, o[dt][3] / l_run);
            *reinterpret_cast<float4 *>(P.out + oi) = y;
            if (P.out16) *reinterpret_cast<uint2 *>(P.out16 + oi) = make_uint2(pack2(y.x, y.y), pack2(y.z, y.w));
        }
    } else {
        float *pp = P.part + (((size_t) t * P.n_head + h) * P.n_chunk + c) * (HD + 4);
#pragma unroll
        for (int dt = 0; dt < NK; dt++)
            *reinterpret_cast<float4 *>(pp + 4 + dt * 16 + 4 * lq) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
        if (lq == 0) {
            pp[0] = m_run;
            pp[1] = l_run;
        }
    }
}

// Merges the chunks' partial rows of one (query head, token): out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).
// Every load is issued before the first reduction: thread i takes chunk i's (m, l) (and chunks i + 256,
// ... past 256 chunks), and hd / 4 threads per chunk hold the float4 slices of up to kCombRegs chunks
// each in registers (chunks cl, cl + CL, ...; any further ones are read after the factors). Each
// thread's slices are summed in ascending chunk order, then the CL thread sums in order.
constexpr int kCombRegs = 16;
template <int HD>
__global__ __launch_bounds__(kBlock) void attn_combine_kernel(AttnParams P) {
    extern __shared__ float s_f[]; // [n_chunk] factors, then [kBlock / (hd / 4)][hd] sums
    __shared__ float s_red[kBlock / kWave];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    constexpr int hd = HD, stride = hd + 4, nq = hd / 4, CL = kBlock / nq;
    const int n = P.n_chunk;
    const float *pp = P.part + ((size_t) t * P.n_head + h) * n * stride;
    const int dq = tid % nq, cl = tid / nq;
    float4 vr[kCombRegs];
#pragma unroll
    for (int j = 0; j < kCombRegs; j++) {
        const int c = cl + j * CL;
        vr[j] = c < n ? *reinterpret_cast<const float4 *>(pp + (size_t) c * stride + 4 + 4 * dq) : make_float4(0, 0, 0, 0);
    }
    const float m0 = tid < n ? pp[(size_t) tid * stride] : -INFINITY;
    const float l0 = tid < n ? pp[(size_t) tid * stride + 1] : 0.0f;
    float m = m0;
    for (int c = tid + kBlock; c < n; c += kBlock) m = fmaxf(m, pp[(size_t) c * stride]);
    m = wave_max(m);
    if (lane == 0) s_red[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    float ls = 0.0f;
    if (tid < n) {
        const float f = m0 == -INFINITY ? 0.0f : expf(m0 - M);
        s_f[tid] = f;
        ls += l0 * f;
    }
    for (int c = tid + kBlock; c < n; c += kBlock) {
        const float mc = pp[(size_t) c * stride];
        const float f = mc == -INFINITY ? 0.0f : expf(mc - M);
        s_f[c] = f;
        ls += pp[(size_t) c * stride + 1] * f;
    }
    ls = wave_sum_tree(ls);
    if (lane == 0) s_red[wv] = ls;
    __syncthreads();
    const float L = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    float4 acc = make_float4(0, 0, 0, 0);
    auto add = [&](const float4 &v, float f) {
        acc.x += v.x * f;
        acc.y += v.y * f;
        acc.z += v.z * f;
        acc.w += v.w * f;
    };
#pragma unroll
    for (int j = 0; j < kCombRegs; j++) {
        const int c = cl + j * CL;
        const float f = c < n ? s_f[c] : 0.0f;
        if (f != 0.0f) add(vr[j], f);
    }
    for (int c = cl + kCombRegs * CL; c < n; c += CL) {
        const float f = s_f[c];
        if (f != 0.0f) add(*reinterpret_cast<const float4 *>(pp + (size_t) c * stride + 4 + 4 * dq), f);
    }
    float *s_o = s_f + ((n + 3) & ~3); // 16-byte aligned
    reinterpret_cast<float4 *>(s_o)[cl * nq + dq] = acc;
    __syncthreads();
    if (tid < hd) {
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < CL; i++) o += s_o[i * hd + tid];
        const size_t oi = ((size_t) t * P.n_head + h) * hd + tid;
        P.out[oi] = o / L;
        if (P.out16) P.out16[oi] = f2h(o / L);
    }
}

__global__ __launch_bounds__(kBlock) void fill_kernel(FillParams P) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < P.n) P.p[i] = P.v;
}

// splitmix64 finaliser: a well-mixed 64-bit hash of the cell coordinates
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(kBlock) void fill_kv_kernel(FillKvParams P) {
    const int t = blockIdx.x, l = blockIdx.y;
    const int cell = P.cells[t], pos = P.pos[t], hk = P.n_kv * P.hd;
    if (l == 0 && threadIdx.x == 0) {
        P.cell_seq[cell] = P.seq;
        P.cell_pos[cell] = pos;
    }
    uint16_t *kc = P.kcache + P.layer_elems * l, *vc = P.vcache + P.layer_elems * l;
    for (int i = threadIdx.x; i < hk; i += kBlock) {
        const int head = i / P.hd, d = i - head * P.hd;
        const uint64_t z = mix64(P.seed ^ mix64(((uint64_t) l << 48) ^ ((uint64_t) pos << 20) ^ (uint64_t) i));
        const float kv = (float) (z & 0xffffff) * (2.0f / 16777216.0f) - 1.0f;
        const float vv = (float) ((z >> 24) & 0xffffff) * (2.0f / 16777216.0f) - 1.0f;
        kc[k_index(head, d, cell, P.hd, P.kv_size)] = f2h(kv);
        vc[v_index(head, d, cell, P.hd, P.kv_size)] = f2h(vv);
    }
}

template <int TG>
size_t gemv_lds(int cols) {
    return (size_t) TG * cols * 2;
}

}  // namespace

bool gemv_supported(int cols) { return cols > 0 && cols % 8 == 0 && cols <= 8192; }

// head_dim 64, 128 or 256: the output dims split into 16-wide tiles over the 4 wavefronts.
bool attn_supported(int hd) { return hd == 64 || hd == 128 || hd == 256; }

// Rows of a work-group: 16, 32 or 64 (one, two or four 16-row tiles). Chunks are whole 64-cell passes,
// as many as bring the launch to about kAttnTarget work-groups (half that for a step of a few tokens). Then T * n_head * n_chunk <= 32768 +
// T * n_head. With rope_in (one token) every chunk is one pass while n_head * passes <= 32768 (65536
// cells at 32 query heads, 32768 at 64): the RoPE prologue has only been run with single-pass chunks on
// the device. Past that, rope_in is cleared (the caller runs rope_kernel) and chunks take several passes.
constexpr int kAttnTarget = 512;
constexpr int kAttn1Wgs = 256; // one work-group per CU of MI355X
void attn_plan(AttnParams &P) {
    const int rows = P.T * (P.n_head / P.n_kv);
    P.rb_rows = rows <= 16 ? 16 : rows <= 32 ? 32 : 64;
    P.n_rowblk = (rows + P.rb_rows - 1) / P.rb_rows;
    const int passes = (P.n_cells - P.cell_begin + kFaCells - 1) / kFaCells;
    if (P.rope_in) {
        if ((long) P.n_head * passes <= 32768) {
            // one pass per chunk. attn1_kernel (head size 128, up to 16 query heads per KV head) takes 16
            // cells per wavefront: 4 wavefronts (64-cell chunks), or 5 or 6 (80, 96) when that keeps the
            // launch at one work-group per CU where 64-cell chunks would not. At 4352 cells 272 work-groups
            // of 64 cells put 16 of them on a CU with another: the launch's last one ended 6.1 us after the
            // first began, against 4.6 us with 256 (work-groups measured with s_memrealtime on MI355X).
            const int cells = P.n_cells - P.cell_begin;
            int chunk = kFaCells;
            if (P.hd == 128 && P.n_head / P.n_kv <= 4 * kRopeMaxQ && (long) P.n_kv * passes > kAttn1Wgs) {
                for (int nw = 5; nw <= 6; nw++) {
                    if ((long) P.n_kv * ((cells + nw * kA1Cells - 1) / (nw * kA1Cells)) <= kAttn1Wgs) {
                        chunk = nw * kA1Cells;
                        break;
                    }
                }
            }
            P.chunk = chunk;
            P.n_chunk = (cells + chunk - 1) / chunk;
            return;
        }
        P.rope_in = 0;
    }
    // a few tokens in one row block: half the target, so chunks of two passes (T = 8 at 4352 cells: 136
    // work-groups writing half the partial rows of 272; measured 1715 -> 1732 tok/s for the whole model)
    const int target = P.T > 1 && P.n_rowblk == 1 ? kAttnTarget / 2 : kAttnTarget;
    int want = (target + P.n_kv * P.n_rowblk - 1) / (P.n_kv * P.n_rowblk);
    // a step of many tokens whose row blocks alone fill the device takes one chunk per row block, so
    // the launch writes the output itself and no combine follows
    if (P.T >= kAttnSkipMinT && P.n_kv * P.n_rowblk >= kAttnOneChunkWgs) want = 1;
    want = want < 1 ? 1 : (want > passes ? passes : want);
    P.chunk = (passes + want - 1) / want * kFaCells;
    P.n_chunk = (P.n_cells - P.cell_begin + P.chunk - 1) / P.chunk;
}

size_t attn_part_rows(int n_batch, int n_head) { return 32768 + (size_t) n_batch * n_head; }

bool rmsnorm_supported(int n) { return n > 0 && n <= 32 * kNormBlock; }

hipError_t launch_rmsnorm(const NormParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.rows == 0) return hipSuccess;
    const dim3 g(P.rows), b(kNormBlock);
    const int npt = (P.n + kNormBlock - 1) / kNormBlock;
    if (P.Y) {
        if (P.emb || !P.x_out || P.k < 1) return hipErrorInvalidValue;
        if (npt <= 4) return launch(rmsnorm_kernel<4, true>, g, b, 0, st, tm, P);
        if (npt <= 8) return launch(rmsnorm_kernel<8, true>, g, b, 0, st, tm, P);
        if (npt <= 16) return launch(rmsnorm_kernel<16, true>, g, b, 0, st, tm, P);
        return launch(rmsnorm_kernel<32, true>, g, b, 0, st, tm, P);
    }
    if (npt <= 1) return launch(rmsnorm_kernel<1, false>, g, b, 0, st, tm, P);
    if (npt <= 2) return launch(rmsnorm_kernel<2, false>, g, b, 0, st, tm, P);
    if (npt <= 4) return launch(rmsnorm_kernel<4, false>, g, b, 0, st, tm, P);
    if (npt <= 8) return launch(rmsnorm_kernel<8, false>, g, b, 0, st, tm, P);
    if (npt <= 16) return launch(rmsnorm_kernel<16, false>, g, b, 0, st, tm, P);
    return launch(rmsnorm_kernel<32, false>, g, b, 0, st, tm, P);
}

bool gemm16_supported(int rows, int cols, int T) {
    return rows > 0 && rows % 16 == 0 && (cols == 2048 || cols == 4096) && T >= 1 && T <= 16;
}

// Rows per work-group: the smallest rw dividing `rows` with rows / rw <= 256 (one work-group per CU on
// MI355X's 256 CUs), so that no CU streams twice the bytes of another (320 work-groups of 16 rows for
// the 5120 Q/K/V rows of the 30B shape left 64 CUs with two).
// Rows per work-group at 2048 columns: up to 64 (four tiles); at 4096 columns up to 16 (one tile, whose
// weights and activations already take 128 VGPRs).
static int gemm16_rows_per_wg(int rows, int cols) {
    const int cap = cols == 2048 ? 64 : 16;
    for (int rw = (rows + 255) / 256; rw <= cap; rw++)
        if (rows % rw == 0) return rw;
    return 16;
}

// 8 wavefronts, 4 steps of 64 values each at 2048 columns, 8 at 4096; one 16-token tile. With 16 rows per
// work-group, measured on MI355X at the 30B shape, T = 8: Q/K/V (21.0 MB) 9.46 us and o-proj (16.8 MB)
// 9.81 us, against about 12 us each for rocblas_gemm_ex; with a second 16-token tile (T = 32) 14.4 and
// 15.1 us, slower than rocBLAS, which keeps T > 16. 2, 4 or 16 wavefronts per work-group instead of 8
// change nothing measurable (the whole-model T = 8 step within 1%). Rows per work-group from the rows
// (20 for Q/K/V and 8 for o-proj: 256 work-groups each) take the eager per-layer Q/K/V + rope stage from
// 16.3 to 14.7 us and o-proj from 12.2 to 11.4 us at T = 8 (whole model T = 8 1777 -> 1826 tok/s,
// T = 16 2825 -> 2918), with the same sums in the same order per output.
hipError_t launch_gemm16(const Gemm16Params &Pin, hipStream_t st, const LaunchTiming *tm) {
    if (!gemm16_supported(Pin.rows, Pin.cols, Pin.T)) return hipErrorInvalidValue;
    Gemm16Params P = Pin;
    P.rw = gemm16_rows_per_wg(P.rows, P.cols);
    const int nrt = (P.rw + 15) / 16;
    const dim3 grid(P.rows / P.rw), block(8 * kWave);
    if (P.cols == 2048) {
        if (nrt == 1) return launch(gemm16_kernel<8, 4, 1, 1>, grid, block, 0, st, tm, P);
        if (nrt == 2) return launch(gemm16_kernel<8, 4, 1, 2>, grid, block, 0, st, tm, P);
        if (nrt == 3) return launch(gemm16_kernel<8, 4, 1, 3>, grid, block, 0, st, tm, P);
        return launch(gemm16_kernel<8, 4, 1, 4>, grid, block, 0, st, tm, P);
    }
    return launch(gemm16_kernel<8, 8, 1, 1>, grid, block, 0, st, tm, P);
}

template <int NJ, int RW>
hipError_t launch_gemv1_t(const GemvParams &P, hipStream_t st, const LaunchTiming *tm) {
    const int per_wg = kGvWaves * RW;
    const dim3 grid((P.rows_total + per_wg - 1) / per_wg), block(kGvWaves * kWave);
    if (P.emb) {
        if (P.norm_w) return launch(gemv1_kernel<NJ, RW, true, true>, grid, block, 0, st, tm, P);
        return launch(gemv1_kernel<NJ, RW, false, true>, grid, block, 0, st, tm, P);
    }
    if (P.norm_w) return launch(gemv1_kernel<NJ, RW, true, false>, grid, block, 0, st, tm, P);
    return launch(gemv1_kernel<NJ, RW, false, false>, grid, block, 0, st, tm, P);
}

hipError_t launch_gemv(const GemvParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0 || P.rows_total == 0) return hipSuccess;
    if (P.T == 1) {
        // 16-byte chunks per lane per row; fewer rows per wavefront for long rows keep the weight
        // registers at 16 chunks and the grid above 256 work-groups
        const int nj = (P.cols / 8 + kWave - 1) / kWave;
        if (nj <= 1) return launch_gemv1_t<1, 4>(P, st, tm);
        if (nj <= 2) return launch_gemv1_t<2, 4>(P, st, tm);
        if (nj <= 4) {
            // five rows per wavefront when that fits the rows in one work-group per CU and four do not
            // (Q/K/V of the 30B shape: 5120 rows in 256 work-groups instead of 320)
            if ((P.rows_total + 19) / 20 <= 256 && (P.rows_total + 15) / 16 > 256) return launch_gemv1_t<4, 5>(P, st, tm);
            return launch_gemv1_t<4, 4>(P, st, tm);
        }
        if (nj <= 8) return launch_gemv1_t<8, 2>(P, st, tm);
        if (nj <= 16) return launch_gemv1_t<16, 1>(P, st, tm);
    }
    if (P.norm_w || P.emb) return hipErrorInvalidValue; // fused normalisation is single-token only
    const int per_wg = kGvWaves * kGvRows;
    const dim3 grid((P.rows_total + per_wg - 1) / per_wg), block(kGvWaves * kWave);
    // tokens per group: enough for the step, as many as the activations' LDS allows
    int tg = P.T == 2 ? 2 : P.T <= 4 ? 4 : 8;
    while (tg > 2 && gemv_lds<1>(P.cols) * tg > (size_t) kGvMaxLds) tg /= 2;
    if (tg == 2) return launch(gemv_kernel<2>, grid, block, gemv_lds<2>(P.cols), st, tm, P);
    if (tg == 4) return launch(gemv_kernel<4>, grid, block, gemv_lds<4>(P.cols), st, tm, P);
    return launch(gemv_kernel<8>, grid, block, gemv_lds<8>(P.cols), st, tm, P);
}

hipError_t launch_rope_table(const RopeParams &P, float *cs_out, hipStream_t st) {
    if (P.T == 0) return hipSuccess;
    return launch(rope_table_kernel, dim3(P.T), dim3(kWave), 0, st, nullptr, P, cs_out);
}

hipError_t launch_rope(const RopeParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0) return hipSuccess;
    return launch(rope_kernel, dim3(P.T, P.n_head + 2 * P.n_kv), dim3(kWave), 0, st, tm, P);
}

template <int HD>
hipError_t launch_attn_hd(const AttnParams &P, hipStream_t st, const LaunchTiming *tm) {
    const dim3 grid(P.n_kv * P.n_chunk * P.n_rowblk), block(kAtBlock);
    if constexpr (HD == 128) {
        if (P.rb_rows == 16 && P.rope_in && P.n_head / P.n_kv <= 4 * kRopeMaxQ && P.rope.cs) {
            if (P.chunk == 4 * kA1Cells) return launch(attn1_kernel<4>, grid, dim3(4 * kWave), 0, st, tm, P);
            if (P.chunk == 5 * kA1Cells) return launch(attn1_kernel<5>, grid, dim3(5 * kWave), 0, st, tm, P);
            if (P.chunk == 6 * kA1Cells) return launch(attn1_kernel<6>, grid, dim3(6 * kWave), 0, st, tm, P);
        }
    }
    // 64-row blocks: each wavefront on its own 16 rows (head sizes 64 and 128; 256 would need 128 KB of
    // fragments per block)
    if constexpr (HD <= 128) {
        if (P.rb_rows == 64 && !P.rope_in) {
            if (P.T >= kAttnSkipMinT) return launch(attn_rows_kernel<HD, true>, grid, block, 0, st, tm, P);
            return launch(attn_rows_kernel<HD, false>, grid, block, 0, st, tm, P);
        }
    }
    // steps of many tokens (prompts): the instantiation that skips passes with no cell of the sequence
    if (P.T >= kAttnSkipMinT && !P.rope_in) {
        if (P.rb_rows == 16) return launch(attn_kernel<HD, 1, true>, grid, block, 0, st, tm, P);
        if (P.rb_rows == 32) return launch(attn_kernel<HD, 2, true>, grid, block, 0, st, tm, P);
        return launch(attn_kernel<HD, 4, true>, grid, block, 0, st, tm, P);
    }
    if (P.rb_rows == 16) return launch(attn_kernel<HD, 1>, grid, block, 0, st, tm, P);
    if (P.rb_rows == 32) return launch(attn_kernel<HD, 2>, grid, block, 0, st, tm, P);
    return launch(attn_kernel<HD, 4>, grid, block, 0, st, tm, P);
}

hipError_t launch_attn(const AttnParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0) return hipSuccess;
    // RoPE inside the launch: one token, whose query rows fit one 16-row tile
    if (P.rope_in && (P.T != 1 || P.rb_rows != 16 || P.n_rowblk != 1 || P.rope.T != 1 || P.rope.hd != P.hd))
        return hipErrorInvalidValue;
    switch (P.hd) {
    case 64: return launch_attn_hd<64>(P, st, tm);
    case 128: return launch_attn_hd<128>(P, st, tm);
    case 256: return launch_attn_hd<256>(P, st, tm);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_combine(const AttnParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0 || P.n_chunk == 1) return hipSuccess;
    const size_t lds = ((size_t) ((P.n_chunk + 3) & ~3) + (size_t) kBlock / (P.hd / 4) * P.hd) * sizeof(float);
    const dim3 grid(P.n_head, P.T), block(kBlock);
    switch (P.hd) {
    case 64: return launch(attn_combine_kernel<64>, grid, block, lds, st, tm, P);
    case 128: return launch(attn_combine_kernel<128>, grid, block, lds, st, tm, P);
    case 256: return launch(attn_combine_kernel<256>, grid, block, lds, st, tm, P);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_fill_kv(const FillKvParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.T == 0) return hipSuccess;
    return launch(fill_kv_kernel, dim3(P.T, P.n_layer), dim3(kBlock), 0, st, tm, P);
}

hipError_t launch_fill(const FillParams &P, hipStream_t st, const LaunchTiming *tm) {
    if (P.n <= 0) return hipSuccess;
    return launch(fill_kernel, dim3((P.n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, tm, P);
}

}  // namespace lstk
