// kernels.h - launchers of the gfx950 MoE kernels (kernels.hip), called by the pool (pool.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace lstk {

// Quantized activations: qs [T][K] int8, d [T][K/32] f32 (the scale of the 32-value group; Q8_K's
// per-256 scale is repeated 8 times), bs [T][K/32] int32 (sum of the group's int8 values, Q8_K only).
struct ActBuf {
    int8_t *qs;
    float *d;
    int32_t *bs;
};

// Token -> bin permutation: counts [n_bins], offsets [n_bins + 1], active [n_bins] (bins with
// count > 0, ascending), n_active [1], perm [T*k] (position -> pair index t*k + j).
struct PermBuf {
    int32_t *counts;
    int32_t *offsets;
    int32_t *active;
    int32_t *n_active;
    int32_t *perm;
};

struct PrologueParams {
    const float *hnorm;
    int T, h, k;
    // router
    int do_route;
    const void *gate_inp;
    int gate_type;
    int E;
    float *logits;
    int32_t *ids;
    float *weights;
    // activation quantization (qtype 0 = none, 8 = Q8_0, 12 = Q8_K for Q4_K weights)
    int qtype;
    ActBuf xq;
    // permutation (bins = ids when routing)
    int do_perm;
    const int32_t *bins;
    int n_bins;
    PermBuf pb;
    int32_t *err;
    unsigned *counter;
};

struct GateUpParams {
    const uint8_t *w_gate, *w_up;
    size_t stride_gate, stride_up; // bytes per slot
    int type;                      // weight type of gate and up
    int f, h, k;
    ActBuf xq;
    PermBuf pb;
    int max_active;
    float *act; // [T*k][f], rows in permuted order
};

struct DownParams {
    const uint8_t *w_down;
    size_t stride_down;
    int type;
    int h, f, k, T;
    const float *act;
    const float *weights; // [T*k] router weights
    PermBuf pb;
    int max_active;
    float *Y;             // [T*k][h] weighted expert outputs by pair index
    const float *resid;
    float *out;
    unsigned *counters;   // [h / 64], zero between calls
};

// Checks the shapes the kernels assume; returns an empty string when they hold.
const char *check_shapes(int h, int f, int E, int k, int n_bins);
hipError_t launch_prologue(const PrologueParams &p, hipStream_t s);
hipError_t launch_gate_up(const GateUpParams &p, hipStream_t s);
hipError_t launch_down(const DownParams &p, hipStream_t s);

}  // namespace lstk
