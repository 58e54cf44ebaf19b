// The pool's byte layout in HBM, shared by the host code and every kernel.
//
// Device memory is [layer][physical page][kv head] blocks of kPageBlock bytes. A block holds 256 tokens of one
// (layer, head) as 8 tiles of 32 tokens, each tile kTileBytes:
//   [0, 8192)      K codes, 32 tokens x 256, arranged for the decode kernel's QK^T operand (below)
//   [8192, 16384)  V codes, 32 tokens x 256, arranged for its PV operand
//   [16384, 16896) K scales, fp16 [32 tokens][8 blocks] (token-major, natural order)
//   [16896, 17408) V scales, fp16 [4 lane groups][8 blocks][8 slots]
// Two code formats share the layout (the pool's format, fixed at creation): Q8_0 (ggml's block_q8_0 rule, a scale a
// 32-value block) and FNFL's KV8 (kv_q8_ref.h: a scale a 64-value group), whose group scale is written at both of the
// group's 32-value blocks, so every attention kernel reads the two formats the same way and a cell is 1,088 B either
// way.
// Codes are stored excess-128 (byte = code + 128 = code ^ 0x80), so the kernels widen them to fp16 with one byte
// permute (0x6400 | byte is the fp16 value 1024 + byte) and one packed subtract of 1152.
//
// The arrangement makes every wave load of 1 KiB (64 lanes x 16 B) land each lane's bytes directly in the register
// layout of v_mfma_f32_16x16x32_f16 (A operand: lane l holds row l % 16, contraction slots 8 (l / 16) .. + 7):
//   K (S^T = K Q^T: rows are tokens, the contraction runs over one 32-value Q8_0 block): token tt of the tile is
//   half h = tt / 16, row j = tt % 16; value d is block b = d / 32, lane group q = (d % 32) / 8, slot i = d % 8;
//   byte offset h * 4096 + (b / 2) * 1024 + (16 q + j) * 16 + (b % 2) * 8 + i.
//   V (O^T = V^T P^T: rows are values d, the contraction runs over the tile's 32 tokens): d is MFMA tile m = d / 16,
//   row dd = d % 16; token tt is lane group q and slot s with tt = 4 q + s (s < 4) or 16 + 4 q + (s - 4) (s >= 4), the
//   order in which the QK^T result already holds P in registers; byte offset
//   8192 + (m / 2) * 1024 + (16 q + dd) * 16 + (m % 2) * 8 + s.
#pragma once

#include <cstdint>

namespace fnkv {

constexpr int32_t kPageTokens = 256;
constexpr int32_t kHeadDim = 256;
constexpr int32_t kQK = 32;
constexpr int32_t kBlocks = kHeadDim / kQK; // 8 Q8_0 blocks a row
constexpr int32_t kTileTokens = 32;
constexpr int32_t kTilesPerPage = kPageTokens / kTileTokens;
constexpr int32_t kKCodes = 0;
constexpr int32_t kVCodes = 8192;
constexpr int32_t kKScales = 16384;
constexpr int32_t kVScales = 16896;
constexpr int32_t kTileBytes = 17408;
constexpr int64_t kPageBlock = int64_t(kTileBytes) * kTilesPerPage; // 139,264
constexpr int32_t kFormatQ8_0 = 0; // FNKV_FMT_Q8_0
constexpr int32_t kFormatKV8 = 1;  // FNKV_FMT_KV8
constexpr int32_t kKV8Group = 64;  // values a KV8 scale

#if defined(__HIPCC__)
#define FNKV_HD __host__ __device__ inline
#else
#define FNKV_HD inline
#endif

FNKV_HD int32_t k_code_off(int32_t tt, int32_t d) {
    const int32_t h = tt >> 4, j = tt & 15, b = d >> 5, q = (d >> 3) & 3, i = d & 7;
    return kKCodes + h * 4096 + (b >> 1) * 1024 + (16 * q + j) * 16 + (b & 1) * 8 + i;
}
FNKV_HD int32_t v_code_off(int32_t tt, int32_t d) {
    const int32_t m = d >> 4, dd = d & 15;
    const int32_t q = (tt & 15) >> 2, s = (tt & 3) + ((tt >> 4) << 2);
    return kVCodes + (m >> 1) * 1024 + (16 * q + dd) * 16 + (m & 1) * 8 + s;
}
FNKV_HD int32_t k_scale_off(int32_t tt, int32_t b) { return kKScales + tt * 16 + b * 2; }
FNKV_HD int32_t v_scale_off(int32_t tt, int32_t b) {
    const int32_t q = (tt & 15) >> 2, s = (tt & 3) + ((tt >> 4) << 2);
    return kVScales + q * 128 + b * 16 + s * 2;
}

// the device view of a pool that kernels take by value
struct pool_view {
    uint8_t * base;
    const int32_t * table; // [n_slots][table_stride] physical page of each logical page
    int64_t layer_stride;  // bytes a layer: n_pages * h_kv * kPageBlock
    int64_t page_stride;   // bytes a physical page within a layer: h_kv * kPageBlock
    int32_t table_stride;
    int32_t h_kv;
    int32_t format; // kFormatQ8_0 or kFormatKV8
};

} // namespace fnkv
