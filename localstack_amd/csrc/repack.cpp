// repack.cpp - host conversion between GGUF expert-matrix bytes and the pool's HBM layout.
//
// The reference keeps GGUF bytes verbatim in its slots because Metal reads them zero-copy
// (src/expert_store.cpp:156-187, docs/decisions.md:13). On MI355X the slot format is internal, so
// each expert matrix is transposed once, when it enters the pool or the host tier, into
// [rows/16][cols/256][C][16 rows][16 B] chunks (formats.h). Q8_0's 34-byte blocks are regrouped in eights so
// every load is an aligned 16-byte chunk; Q2_K, Q3_K, Q5_K and Q6_K blocks are unpacked to KQ8.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/lstk_moe.h"
#include "formats.h"

namespace lstk {

// One Q2_K / Q3_K / Q5_K / Q6_K block (ggml's block layouts) as integers: value v of the block is
// (d * sc[v / 16]) * q[v] - dmin * m[v / 16]. Layouts (value 128 n + 32 j + l with n < 2, j < 4, l < 32):
//   Q2_K  q = bits 2j, 2j + 1 of qs[32 n + l]; scales[8 n + 2 j + l / 16] = sc | m << 4.
//   Q3_K  q = the same two bits, minus 4 when bit 4 n + j of hmask[l] is clear; the 16 6-bit scales
//         (minus 32) are packed in 12 bytes: low nibbles in bytes 0-7 (scales 0-7) and their high
//         nibbles (scales 8-15), bits 4-5 of scale i in bits 2 (i / 4) of byte 8 + i % 4. No mins.
//   Q5_K  value 64 c + 32 h + l: nibble h of qs[32 c + l] plus 16 when bit 2 c + h of qh[l] is set;
//         6-bit scale and min of each 32 values as in Q4_K.
//   Q6_K  q = the low (j < 2) or high nibble of ql[64 n + 32 (j % 2) + l] and bits 2j, 2j + 1 of
//         qh[32 n + l] as bits 4-5, minus 32; int8 scale per 16 values. No mins.
void kq8_unpack(int type, const uint8_t *b, KQ8Block &o) {
    auto h2f = [](const uint8_t *p) {
        const uint16_t h = (uint16_t) (p[0] | p[1] << 8);
        const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
        uint32_t bits;
        if (e == 0 && m == 0) {
            bits = sign;
        } else if (e == 0) { // subnormal
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400u)) {
                mm <<= 1;
                sh++;
            }
            bits = sign | ((uint32_t) (113 - sh) << 23) | ((mm & 0x3ffu) << 13);
        } else if (e == 31) {
            bits = sign | 0x7f800000u | (m << 13);
        } else {
            bits = sign | ((e + 112) << 23) | (m << 13);
        }
        float f;
        memcpy(&f, &bits, 4);
        return f;
    };
    o.dmin = 0.0f;
    std::fill(o.m, o.m + 16, 0);
    for (int v = 0; v < 256; v++) {
        const int n = v / 128, j = (v % 128) / 32, l = v % 32;
        switch (type) {
            case kTypeQ2_K: o.q[v] = (int8_t) ((b[16 + 32 * n + l] >> (2 * j)) & 3); break;
            case kTypeQ3_K:
                o.q[v] = (int8_t) (((b[32 + 32 * n + l] >> (2 * j)) & 3) - (((b[l] >> (4 * n + j)) & 1) ? 0 : 4));
                break;
            case kTypeQ5_K: {
                const int c = v / 64, h = (v % 64) / 32;
                const int nib = (b[48 + 32 * c + l] >> (4 * h)) & 0xF;
                o.q[v] = (int8_t) (nib + (((b[16 + l] >> (2 * c + h)) & 1) ? 16 : 0));
                break;
            }
            default: { // Q6_K
                const int lo = (b[64 * n + 32 * (j % 2) + l] >> (4 * (j / 2))) & 0xF;
                const int hi = (b[128 + 32 * n + l] >> (2 * j)) & 3;
                o.q[v] = (int8_t) ((lo | hi << 4) - 32);
            }
        }
    }
    switch (type) {
        case kTypeQ2_K:
            for (int i = 0; i < 16; i++) {
                o.sc[i] = (int8_t) (b[i] & 0xF);
                o.m[i] = (uint8_t) (b[i] >> 4);
            }
            o.d = h2f(b + 80);
            o.dmin = h2f(b + 82);
            break;
        case kTypeQ3_K:
            for (int i = 0; i < 16; i++) {
                const int a = i / 4, bb = i % 4;
                const int lo = a < 2 ? b[96 + 4 * a + bb] & 0xF : b[96 + 4 * (a - 2) + bb] >> 4;
                o.sc[i] = (int8_t) ((lo | ((b[104 + bb] >> (2 * a)) & 3) << 4) - 32);
            }
            o.d = h2f(b + 108);
            break;
        case kTypeQ5_K:
            for (int j = 0; j < 8; j++) {
                const uint8_t *q = b + 4;
                int sc, m;
                if (j < 4) {
                    sc = q[j] & 63;
                    m = q[j + 4] & 63;
                } else {
                    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
                    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
                }
                o.sc[2 * j] = o.sc[2 * j + 1] = (int8_t) sc;
                o.m[2 * j] = o.m[2 * j + 1] = (uint8_t) m;
            }
            o.d = h2f(b);
            o.dmin = h2f(b + 2);
            break;
        default:
            for (int i = 0; i < 16; i++) o.sc[i] = (int8_t) b[192 + i];
            o.d = h2f(b + 208);
    }
}

// Copies one super-block row between GGUF bytes (`g`, the 256 values starting at block sb of a row)
// and its C chunks in the pool layout. to_pool selects the direction.
static void convert_row_block(int type, uint8_t *g, uint8_t *const *chunk, bool to_pool) {
    if (is_kq8_source(type)) { // to the pool only (the unpacking is not inverted)
        KQ8Block k;
        kq8_unpack(type, g, k);
        memset(chunk[0], 0, 16);
        memcpy(chunk[0], &k.d, 4);
        memcpy(chunk[0] + 4, &k.dmin, 4);
        memcpy(chunk[1], k.sc, 16);
        memcpy(chunk[2], k.m, 16);
        for (int grp = 0; grp < 16; grp++) memcpy(chunk[3 + grp], k.q + 16 * grp, 16);
        return;
    }
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
    if (!to_pool && is_kq8_source(type)) return LSTK_E_INVALID;
    const int C = chunks_of(type);
    const int nsb = cols / kSuper;
    const size_t sb_bytes = (size_t) gguf_superblock_bytes(type); // GGUF bytes of one super-block row
    const size_t row_bytes = (size_t) nsb * sb_bytes;
    auto work = [&](int r0, int r1) {
        uint8_t *chunk[kMaxChunks];
        for (int r = r0; r < r1; r++) {
            for (int sb = 0; sb < nsb; sb++) {
                for (int c = 0; c < C; c++) chunk[c] = packed + chunk_offset(C, rows, nsb, sb, c, r);
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
