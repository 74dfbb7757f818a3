// internal.h - what the forward pass (model.cpp) needs from the pool (pool.cpp) beyond the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/lstk_moe.h"

namespace lstk {

// Records `msg` as the calling thread's lstk_last_error() and returns `code`.
int set_error(int code, const std::string &msg);
// The pool's dims (the MoE part of the model shape) and whether it streams from the host tier.
const lstk_moe_dims &pool_dims(const lstk_pool *pool);
bool pool_streaming(const lstk_pool *pool);
bool pool_dry(const lstk_pool *pool);
// Whether the pool's bookkeeping lives on the device (LSTK_POOL_DEVICE_LRU).
bool pool_device_lru(const lstk_pool *pool);
// With `on`, blocks of several tokens stop before their combine: the k weighted expert rows of each
// token are left in pool_moe_rows() ([T][k][n_embd] f32) for the caller to add into the residual (the
// forward pass does it in the next layer's RMSNorm launch). Single-token blocks combine as always.
void pool_defer_combine(lstk_pool *pool, bool on);
const float *pool_moe_rows(const lstk_pool *pool);
// lstk_moe_block for T tokens of a resident pool whose hnorm rows the router launch computes itself as
// rms_norm(x) * norm_w (bit-identical to the RMSNorm kernel's rows; also stored to d_hnorm).
int moe_block_normed(lstk_pool *pool, int layer, const float *d_x, const float *d_norm_w, float eps, float *d_hnorm,
                     const void *d_gate_inp, int gate_type, const float *d_resid, float *d_out, int32_t *d_ids,
                     float *d_weights, int T, hipStream_t st);

}  // namespace lstk
