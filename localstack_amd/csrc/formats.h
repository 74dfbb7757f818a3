// formats.h - quant block formats and the pool's HBM layout, shared by host and device code.
//
// GGUF block formats (ggml's block_q8_0 / block_q4_K / block_q8_K):
//   Q8_0: {fp16 d; int8 qs[32]}                              34 B per 32 values
//   Q4_K: {fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]}      144 B per 256 values
//   Q8_K: {f32 d; int8 qs[256]; i16 bsums[16]}                292 B per 256 values (activations only)
//
// Pool layout of one expert matrix (rows x cols): [cols/256][C][rows][16 B]. A 256-value super-block
// row is cut into C 16-byte chunks and chunk c of neighbouring rows sits side by side:
//   Q8_0 (C = 17): chunk 0 = the 8 fp16 scales of the super-block's 8 blocks, chunk 1 + 2i + hh =
//                  bytes [16 hh, 16 hh + 16) of block i's 32 int8 values.
//   Q4_K (C = 9):  chunk c = bytes [16 c, 16 c + 16) of the GGUF block, so chunk 0 = {d, dmin,
//                  scales[12]} and chunks 1..8 = qs.
// A wavefront whose lanes own 64 consecutive rows therefore reads each chunk with one 1 KiB
// fully coalesced 128-bit load, and the matrix keeps its GGUF size.
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
constexpr int kTypeQ4_K = 12;

constexpr int kSuper = 256;        // values per super-block row
constexpr int kQ8_0Block = 34;     // bytes per Q8_0 block of 32
constexpr int kQ4_KBlock = 144;    // bytes per Q4_K block of 256
constexpr int kChunksQ8_0 = 17;    // 16-byte chunks per 256 values
constexpr int kChunksQ4_K = 9;

LSTK_HD constexpr int chunks_of(int type) { return type == kTypeQ8_0 ? kChunksQ8_0 : kChunksQ4_K; }

LSTK_HD constexpr bool supported_weight_type(int type) { return type == kTypeQ8_0 || type == kTypeQ4_K; }

// Bytes of a rows x cols matrix (identical in GGUF and pool layout).
LSTK_HD constexpr size_t matrix_bytes(int type, int rows, int cols) {
    return (size_t) rows * (size_t) (cols / kSuper) * (size_t) chunks_of(type) * 16;
}

// Byte offset of chunk c of super-block sb of row r in the pool layout.
LSTK_HD inline size_t chunk_offset(int C, int rows, int sb, int c, int r) {
    return (((size_t) sb * (size_t) C + (size_t) c) * (size_t) rows + (size_t) r) * 16;
}

}  // namespace lstk
