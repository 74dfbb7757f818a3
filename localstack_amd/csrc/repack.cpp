// repack.cpp - host conversion between GGUF expert-matrix bytes and the pool's HBM layout.
//
// The reference keeps GGUF bytes verbatim in its slots because Metal reads them zero-copy
// (src/expert_store.cpp:156-187, docs/decisions.md:13). On MI355X the slot format is internal, so
// each expert matrix is transposed once, when it enters the pool or the host tier, into
// [cols/256][C][rows][16 B] chunks (formats.h). Q8_0's 34-byte blocks are regrouped in eights so
// every load is an aligned 16-byte chunk.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/lstk_moe.h"
#include "formats.h"

namespace lstk {

// Copies one super-block row between GGUF bytes (`g`, the 256 values starting at block sb of a row)
// and its C chunks in the pool layout. to_pool selects the direction.
static void convert_row_block(int type, uint8_t *g, uint8_t *const *chunk, bool to_pool) {
    if (type == kTypeQ4_K) {
        for (int c = 0; c < kChunksQ4_K; c++) {
            if (to_pool) memcpy(chunk[c], g + 16 * c, 16);
            else memcpy(g + 16 * c, chunk[c], 16);
        }
        return;
    }
    // Q8_0: 8 blocks of {fp16 d, int8 qs[32]}
    for (int i = 0; i < 8; i++) {
        uint8_t *blk = g + (size_t) i * kQ8_0Block;
        if (to_pool) {
            memcpy(chunk[0] + 2 * i, blk, 2);
            memcpy(chunk[1 + 2 * i], blk + 2, 16);
            memcpy(chunk[2 + 2 * i], blk + 18, 16);
        } else {
            memcpy(blk, chunk[0] + 2 * i, 2);
            memcpy(blk + 2, chunk[1 + 2 * i], 16);
            memcpy(blk + 18, chunk[2 + 2 * i], 16);
        }
    }
}

static int convert_matrix(int type, int rows, int cols, uint8_t *gguf, uint8_t *packed, bool to_pool) {
    if (!supported_weight_type(type) || rows <= 0 || cols <= 0 || cols % kSuper != 0) return LSTK_E_INVALID;
    const int C = chunks_of(type);
    const int nsb = cols / kSuper;
    const size_t row_bytes = (size_t) nsb * C * 16;
    const size_t sb_bytes = (size_t) C * 16;
    auto work = [&](int r0, int r1) {
        uint8_t *chunk[kChunksQ8_0];
        for (int r = r0; r < r1; r++) {
            for (int sb = 0; sb < nsb; sb++) {
                for (int c = 0; c < C; c++) chunk[c] = packed + chunk_offset(C, rows, sb, c, r);
                convert_row_block(type, gguf + (size_t) r * row_bytes + (size_t) sb * sb_bytes, chunk, to_pool);
            }
        }
    };
    // split large matrices over host threads; small ones are not worth a thread start
    const size_t bytes = (size_t) rows * row_bytes;
    const int n_threads = bytes < ((size_t) 8 << 20) ? 1 : (int) std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    if (n_threads == 1) {
        work(0, rows);
        return LSTK_OK;
    }
    std::vector<std::thread> pool;
    const int per = (rows + n_threads - 1) / n_threads;
    for (int i = 0; i < n_threads; i++) {
        const int r0 = i * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) pool.emplace_back(work, r0, r1);
    }
    for (std::thread &t : pool) t.join();
    return LSTK_OK;
}

int repack_matrix(int type, int rows, int cols, const void *gguf, void *packed) {
    return convert_matrix(type, rows, cols, (uint8_t *) gguf, (uint8_t *) packed, true);
}

int unpack_matrix(int type, int rows, int cols, const void *packed, void *gguf) {
    return convert_matrix(type, rows, cols, (uint8_t *) gguf, (uint8_t *) packed, false);
}

}  // namespace lstk
