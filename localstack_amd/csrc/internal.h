// internal.h - what the forward pass (model.cpp) needs from the pool (pool.cpp) beyond the C ABI.
#pragma once

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

}  // namespace lstk
