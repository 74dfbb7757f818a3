// forward.h - launchers of the gfx950 kernels of the Qwen3 forward pass around the MoE block
// (forward.hip), called by the model (model.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "kernels.h"

namespace lstk {

// y = rms_norm(x) * w per row (ggml_rms_norm + ggml_mul). With `emb` set, row r of x is first gathered
// from the F16 embedding table at tokens[r] and also stored to x_out (ggml_get_rows).
struct NormParams {
    const float *x;
    const uint16_t *emb;
    const int32_t *tokens;
    float *x_out;
    const float *w;
    float *y;
    int rows, n;
    float eps;
    uint16_t *y16; // when set, also y rounded to fp16 (the input of an F16 matrix product)
    // when set, row r is first x_r + the k rows Y[r][0 .. k) of the previous MoE block (their sum in slot
    // order, then the residual, as combine_kernel adds them), stored to x_out, then normalised
    const float *Y = nullptr;
    int k = 0;
};

// Per-head RMSNorm (optional), NEOX RoPE and the KV-cache store of one step.
// The cache layouts are the operand fragments of the attention's matrix-core products (16 x 16 x 16
// fp16): K [n_head_kv][head_dim / 4][kv_size][4] (4 consecutive dims of a cell, 16 cells side by side)
// and V [n_head_kv][kv_size / 4][head_dim][4] (4 consecutive cells of a dim, 16 dims side by side), so
// every fragment a lane needs is one 8-byte load and 16 lanes read 128 contiguous bytes.
struct RopeParams {
    const float *q, *k, *v; // token t's rows at q + t * ld (n_head * hd), k + t * ld, v + t * ld (n_head_kv * hd)
    const float *q_norm, *k_norm;
    float eps;
    const int32_t *pos, *cells; // [T]
    int32_t seq;
    int32_t *cell_seq, *cell_pos; // [kv_size], written for the step's cells
    int T, n_head, n_kv, hd, kv_size;
    float theta_scale; // freq_base^(-2 / hd)
    uint16_t *q_out;   // [T][n_head][hd] rotated Q rounded to fp16 (attention's Q operand)
    uint16_t *kc, *vc; // this layer's caches
    const float *cs;   // [T][hd / 2][2]: cos and sin of each pair's angle (launch_rope_table), or null
    int ld;            // row stride of q, k and v (floats)
};

// One F16 weight matrix of a GEMV launch: y[t * ldy + r] = sum_i fp16(x[t][i]) * w[r][i] (+ add[t * ldy + r]).
struct GemvSeg {
    const uint16_t *w;
    float *y;
    const float *add;
    int rows;
    int ldy;
};

// Up to three matrices with the same input (Q, K and V) in one launch; rows of the segments are
// numbered one after the other. For a single token (T == 1) the input row may be normalised on the way
// in: with norm_w set, x is replaced by rms_norm(x) * norm_w (the reference's attn_norm before Q/K/V),
// and with emb set, x is first gathered from the F16 embedding row tokens[0] and written to x_out.
//
struct GemvParams {
    GemvSeg seg[3];
    int nseg;
    int rows_total;
    int cols;
    const float *x; // [T][cols]
    int T;
    const float *norm_w;
    float eps;
    const uint16_t *emb;
    const int32_t *tokens;
    float *x_out;
};

// Causal attention of one step over cells [0, n_cells) of one layer's cache. The query rows of a KV head
// are its n_head / n_kv query heads times the T tokens (row r = token r / grp, head r % grp); work-group
// (rb, c, g) covers rows [rb * rb_rows, (rb + 1) * rb_rows) of KV head g against cells
// [c * chunk, (c + 1) * chunk), reading each K/V fragment once for all of them. With n_chunk == 1 it
// writes `out` directly, otherwise partial (max, sum, unnormalised output) rows into `part`.
struct AttnParams {
    const uint16_t *q; // [T][n_head][hd] rotated Q as fp16
    const uint16_t *kc, *vc;
    const int32_t *cell_seq, *cell_pos, *pos;
    int32_t seq;
    int T, n_head, n_kv, hd, kv_size, n_cells, chunk, n_chunk, n_rowblk, rb_rows;
    int cell_begin; // cells [cell_begin, n_cells) are attended: no cell of seq lies below (a multiple of 64)
    float scale;
    float *part; // [T][n_head][n_chunk][hd + 4]: max, sum, 2 unused, unnormalised output
    float *out;  // [T][n_head * hd]
    uint16_t *out16; // when set, also out rounded to fp16
    // One token: with rope_in set the launch does rope_kernel's work itself (q above is then unused):
    // every work-group rotates its query rows from rope.q, and the one whose chunk holds the token's
    // cell stores that cell's K / V (and cell-table entries) of its KV head before reading the chunk.
    int rope_in;
    RopeParams rope;
};

// Writes v to n int32 values (the trace rows the last layer does not compute).
struct FillParams {
    int32_t *p;
    int n;
    int32_t v;
};

// Synthetic context: for the T cells of `cells` (positions `pos`), every layer's K and V get
// pseudo-random fp16 values in [-1, 1) derived from (seed, layer, position, head, dim); the cells are
// marked as belonging to `seq`.
struct FillKvParams {
    const int32_t *cells, *pos;
    int32_t seq;
    int32_t *cell_seq, *cell_pos;
    int T, n_layer, n_kv, hd, kv_size;
    size_t layer_elems;
    uint16_t *kcache, *vcache;
    uint64_t seed;
};

// Y[t][r] (+)= sum_c X[t][c] W[r][c] for a few tokens (T <= 16): fp16 W [rows][cols] and X
// [T][cols], f32 accumulation, Y [T][ldy]; with accumulate set the products are added to Y.
struct Gemm16Params {
    const uint16_t *w, *x;
    float *y;
    int rows, cols, T, ldy, accumulate;
    int rw = 16; // rows per work-group (set by launch_gemm16)
};
// rows a multiple of 16, cols 2048 or 4096, 1 <= T <= 16
bool gemm16_supported(int rows, int cols, int T);
hipError_t launch_gemm16(const Gemm16Params &P, hipStream_t st, const LaunchTiming *tm);

bool gemv_supported(int cols);
bool rmsnorm_supported(int n);
bool attn_supported(int hd);
// Plans the attention launch of a step: fills chunk, n_chunk, n_rowblk and rb_rows of P from T, n_head,
// n_kv and n_cells. The partial rows (T * n_head * n_chunk when n_chunk > 1) stay below
// attn_part_rows(n_batch, n_head).
void attn_plan(AttnParams &P);
size_t attn_part_rows(int n_batch, int n_head);

hipError_t launch_rmsnorm(const NormParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_gemv(const GemvParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_rope(const RopeParams &P, hipStream_t st, const LaunchTiming *tm);
// Fills cs_out [T][hd / 2][2] with the cos and sin of the step's angles (pos[t] * theta_scale^i, by
// repeated multiplication), the values every layer's RoPE uses (P.cs is ignored).
hipError_t launch_rope_table(const RopeParams &P, float *cs_out, hipStream_t st);
hipError_t launch_attn(const AttnParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_attn_combine(const AttnParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_fill(const FillParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_fill_kv(const FillKvParams &P, hipStream_t st, const LaunchTiming *tm);

}  // namespace lstk
