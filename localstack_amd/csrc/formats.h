// formats.h - quant block formats and the pool's HBM layout, shared by host and device code.
//
// GGUF block formats (ggml's block_q8_0 / block_q2_K .. block_q6_K / block_q8_K):
//   Q8_0: {fp16 d; int8 qs[32]}                              34 B per 32 values
//   Q2_K: {u8 scales[16]; u8 qs[64]; fp16 d, dmin}            84 B per 256 values
//   Q3_K: {u8 hmask[32]; u8 qs[64]; u8 scales[12]; fp16 d}    110 B per 256 values
//   Q4_K: {fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]}      144 B per 256 values
//   Q5_K: {fp16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} 176 B per 256 values
//   Q6_K: {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}      210 B per 256 values
//   Q8_K: {f32 d; int8 qs[256]; i16 bsums[16]}                292 B per 256 values (activations only)
//
// Pool layout of one expert matrix (rows x cols): [rows/16][cols/256][C][16 rows][16 B]. A 256-value
// super-block row is cut into C 16-byte chunks; chunk c of the 16 rows of a row block sits side by side,
// and a row block's super-blocks and chunks are contiguous (the last block holds the rows left over):
//   Q8_0 (C = 17): chunk 0 = the 8 fp16 scales of the super-block's 8 blocks, chunk 1 + 2i + hh =
//                  bytes [16 hh, 16 hh + 16) of block i's 32 int8 values.
//   Q4_K (C = 9):  chunk c = bytes [16 c, 16 c + 16) of the GGUF block, so chunk 0 = {d, dmin,
//                  scales[12]} and chunks 1..8 = qs.
//   KQ8  (C = 19): Q2_K, Q3_K, Q5_K and Q6_K unpacked to integers: chunk 0 = {f32 d, f32 dmin, 0, 0},
//                  chunk 1 = the 16 int8 scales of the 16-value groups, chunk 2 = their 16 mins (u8),
//                  chunk 3 + g = the 16 int8 quants of group g. Every value is (d sc) q - dmin m, as
//                  ggml dequantizes each of the four formats, and ggml's dot with Q8_K is
//                  (d d_x) sum_g sc_g (q . x)_g - (dmin d_x) sum_g m_g bsum_g in exact integers.
// A wavefront whose lanes own 16 consecutive rows reads each chunk as one 256-byte piece, and a
// work-group that takes whole row blocks reads one contiguous span of the matrix (on MI355X the
// single-token kernels stream their experts 2-4% faster this way than from [cols/256][C][rows]). Q8_0 and Q4_K matrices keep their GGUF size; KQ8 takes 304 B per
// super-block row (the price of one format for four, read with plain int8 dot products).
#pragma once

#include <cstddef>
#include <cstdint>

#ifndef LSTK_HD
#if defined(__HIPCC__)
#define LSTK_HD __host__ __device__
#else
#define LSTK_HD
#endif
#endif

namespace lstk {

constexpr int kTypeF32 = 0;
constexpr int kTypeF16 = 1;
constexpr int kTypeQ8_0 = 8;
constexpr int kTypeQ2_K = 10;
constexpr int kTypeQ3_K = 11;
constexpr int kTypeQ4_K = 12;
constexpr int kTypeQ5_K = 13;
constexpr int kTypeQ6_K = 14;
constexpr int kTypeKQ8 = 256; // the pool's unpacked k-quant format (not a ggml type id)

constexpr int kSuper = 256;        // values per super-block row
constexpr int kQ8_0Block = 34;     // bytes per Q8_0 block of 32
constexpr int kQ4_KBlock = 144;    // bytes per Q4_K block of 256
constexpr int kChunksQ8_0 = 17;    // 16-byte chunks per 256 values
constexpr int kChunksQ4_K = 9;
constexpr int kChunksKQ8 = 19;
constexpr int kMaxChunks = kChunksKQ8;

LSTK_HD constexpr bool is_kq8_source(int type) {
    return type == kTypeQ2_K || type == kTypeQ3_K || type == kTypeQ5_K || type == kTypeQ6_K;
}
// The format an expert matrix of ggml type `type` is stored in: Q8_0 and Q4_K as they are, the other
// k-quants as KQ8.
LSTK_HD constexpr int pool_format(int type) { return is_kq8_source(type) ? kTypeKQ8 : type; }

LSTK_HD constexpr int chunks_of(int type) {
    return pool_format(type) == kTypeQ8_0 ? kChunksQ8_0 : pool_format(type) == kTypeKQ8 ? kChunksKQ8 : kChunksQ4_K;
}

// ggml types the pool stores (gate / up / down experts).
LSTK_HD constexpr bool supported_weight_type(int type) {
    return type == kTypeQ8_0 || type == kTypeQ4_K || is_kq8_source(type);
}

// Bytes of one 256-value super-block row in GGUF.
LSTK_HD constexpr int gguf_superblock_bytes(int type) {
    return type == kTypeQ8_0 ? 8 * kQ8_0Block : type == kTypeQ2_K ? 84 : type == kTypeQ3_K ? 110 :
           type == kTypeQ4_K ? kQ4_KBlock : type == kTypeQ5_K ? 176 : type == kTypeQ6_K ? 210 : 0;
}

// Bytes of a rows x cols matrix of ggml type `type` in the pool layout.
LSTK_HD constexpr size_t matrix_bytes(int type, int rows, int cols) {
    return (size_t) rows * (size_t) (cols / kSuper) * (size_t) chunks_of(type) * 16;
}

// Bytes of the same matrix in GGUF.
LSTK_HD constexpr size_t gguf_matrix_bytes(int type, int rows, int cols) {
    return (size_t) rows * (size_t) (cols / kSuper) * (size_t) gguf_superblock_bytes(type);
}

// One unpacked k-quant super-block row (repack.cpp): value v = (d * sc[v / 16]) * q[v] - dmin * m[v / 16].
struct KQ8Block {
    float d, dmin;
    int8_t sc[16];
    uint8_t m[16];
    int8_t q[256];
};
// Host only: unpacks one GGUF block of Q2_K, Q3_K, Q5_K or Q6_K.
void kq8_unpack(int type, const uint8_t *block, KQ8Block &out);

// Rows per row block of the pool layout. A block's super-blocks and chunks are contiguous, so the work-group
// that takes a block's rows reads one contiguous span of the matrix.
#ifndef LSTK_POOL_RB
#define LSTK_POOL_RB 16
#endif
constexpr int kPoolRB = LSTK_POOL_RB;

// Byte offset of chunk c of super-block sb (of nsb per row) of row r in the pool layout:
// [rows / kPoolRB][nsb][C][kPoolRB][16 B], the last block holding the rows past the last full block.
LSTK_HD inline size_t chunk_offset(int C, int rows, int nsb, int sb, int c, int r) {
    const int rb = r / kPoolRB, rr = r - rb * kPoolRB;
    const int rbr = rows - rb * kPoolRB < kPoolRB ? rows - rb * kPoolRB : kPoolRB;
    return ((size_t) rb * kPoolRB * (size_t) nsb * (size_t) C + ((size_t) sb * (size_t) C + (size_t) c) * (size_t) rbr +
            (size_t) rr) * 16;
}

}  // namespace lstk
