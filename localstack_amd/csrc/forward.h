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
// numbered one after the other.
struct GemvParams {
    GemvSeg seg[3];
    int nseg;
    int rows_total;
    int cols;
    const float *x; // [T][cols]
    int T;
};

// Per-head RMSNorm (optional), NEOX RoPE and the KV-cache store of one step.
// K cache layout [n_head_kv][head_dim / 8][kv_size][8] fp16 (a wavefront reading 64 consecutive cells of
// one 8-value group issues one 1 KiB load); V cache layout [n_head_kv][kv_size][head_dim] fp16.
struct RopeParams {
    const float *q, *k, *v; // [T][n_head * hd], [T][n_head_kv * hd] x 2
    const float *q_norm, *k_norm;
    float eps;
    const int32_t *pos, *cells; // [T]
    int32_t seq;
    int32_t *cell_seq, *cell_pos; // [kv_size], written for the step's cells
    int T, n_head, n_kv, hd, kv_size;
    float theta_scale; // freq_base^(-2 / hd)
    float *q_out;      // [T][n_head][hd]
    uint16_t *kc, *vc; // this layer's caches
};

// Causal attention of one step over cells [0, n_cells) of one layer's cache. Work-group (c, h, t) covers
// cells [c * chunk, (c + 1) * chunk) for query head h of token t; with n_chunk == 1 it writes `out`
// directly, otherwise partial (max, sum, unnormalised output) rows into `part` for the combine.
struct AttnParams {
    const float *q; // [T][n_head][hd]
    const uint16_t *kc, *vc;
    const int32_t *cell_seq, *cell_pos, *pos;
    int32_t seq;
    int T, n_head, n_kv, hd, kv_size, n_cells, chunk, n_chunk;
    float scale;
    float *part; // [T][n_head][n_chunk][hd + 2]
    float *out;  // [T][n_head * hd]
};

// Writes v to n int32 values (the trace rows the last layer does not compute).
struct FillParams {
    int32_t *p;
    int n;
    int32_t v;
};

bool gemv_supported(int cols);
bool attn_supported(int hd);
int attn_chunk_cells(int T, int n_head, int n_cells, int *n_chunk);

hipError_t launch_rmsnorm(const NormParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_gemv(const GemvParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_rope(const RopeParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_attn(const AttnParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_attn_combine(const AttnParams &P, hipStream_t st, const LaunchTiming *tm);
hipError_t launch_fill(const FillParams &P, hipStream_t st, const LaunchTiming *tm);

}  // namespace lstk
