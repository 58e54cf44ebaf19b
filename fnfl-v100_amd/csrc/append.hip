// The append (new K/V rows quantized into the pool) and the exports back to ggml's block_q8_0 and to KV8's arrays.
//
// The quantization rule is the pool's: q8_0.h's Q8_0 (ggml's quantize_row_q8_0_ref, bit for bit) or KV8 (FNFL's
// kv_q8_quantize_group, bit for bit). The reference's device writers of its
// own KV8 format (fn/kernels/qsa/kv_q8.cuh:244-267, qsa_prompt_attn.cu:90-122) use one warp a row; here one wave64
// quantizes one 256-value row. This entry point serves chunked prefill and any caller appending outside a decode
// launch; fnkv_attn_decode appends a step's new rows itself.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "q8_0.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace fnkv {

// Waves 0 .. rows * h_kv - 1 write one K row each; the waves after them write V four cells at a time: the quads of
// aligned positions 4 g .. 4 g + 3 that the rows touch (the four cells' bytes of one value are adjacent in the V
// layout, so each lane stores a dword a value; a quad the rows cover in part writes only its own cells).
// pos_dev set: the first position is the device word *pos_dev, read by the launch; a position outside
// 0 .. max_cells - rows writes nothing (the launch that reads the rows reports it)
template <bool F32>
__global__ __launch_bounds__(256) void append_kernel(pool_view pv, int32_t slot, int32_t layer, int64_t pos0,
                                                     int32_t rows, const void * __restrict__ kin,
                                                     const void * __restrict__ vin, const int32_t * pos_dev,
                                                     int64_t max_cells) {
    if (pos_dev != nullptr) {
        pos0 = *pos_dev;
        if (pos0 < 0 || pos0 + rows > max_cells) {
            return;
        }
    }
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int64_t w = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int32_t * table = pv.table + int64_t(slot) * pv.table_stride;
    const int64_t k_waves = int64_t(rows) * pv.h_kv;
    if (w < k_waves) {
        const int32_t head = static_cast<int32_t>(w % pv.h_kv);
        const int64_t row = w / pv.h_kv;
        const int64_t src = (row * pv.h_kv + head) * kHeadDim;
        float x[4];
        if (F32) {
            load4<true>(static_cast<const float *>(kin) + src, lane, x);
        } else {
            load4<false>(static_cast<const uint16_t *>(kin) + src, lane, x);
        }
        const int64_t pos = pos0 + row;
        quantize_store_fmt(x, lane, tile_of(pv, table, layer, head, pos), static_cast<int32_t>(pos & 31), 0,
                           pv.format);
        return;
    }
    const int64_t vw = w - k_waves;
    const int32_t head = static_cast<int32_t>(vw % pv.h_kv);
    const int64_t quad = (pos0 >> 2) + vw / pv.h_kv;
    const int64_t p0 = quad * 4;
    if (p0 >= pos0 + rows) {
        return; // past the last quad (the grid allows for any alignment of pos0)
    }
    uint32_t packed[4] = {0, 0, 0, 0};
    uint16_t sbits[4] = {0, 0, 0, 0};
    uint32_t valid = 0;
#pragma unroll
    for (int32_t i = 0; i < 4; ++i) {
        const int64_t row = p0 + i - pos0;
        if (row >= 0 && row < rows) { // uniform across the wave
            valid |= 1u << i;
            const int64_t src = (row * pv.h_kv + head) * kHeadDim;
            float x[4];
            if (F32) {
                load4<true>(static_cast<const float *>(vin) + src, lane, x);
            } else {
                load4<false>(static_cast<const uint16_t *>(vin) + src, lane, x);
            }
            quantize_fmt(x, pv.format, packed[i], sbits[i]);
        }
    }
    store_v_quad(packed, sbits, valid, lane, tile_of(pv, table, layer, head, p0), static_cast<int32_t>(p0 & 31));
}

// one wave a cell: its 8 blocks of (layer, head, kv) as 8 x 34 bytes of block_q8_0
__global__ __launch_bounds__(256) void export_kernel(pool_view pv, int32_t slot, int32_t layer, int32_t head,
                                                     int32_t kv, int64_t tok0, int32_t n_tok, uint8_t * out) {
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int64_t i = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (i >= n_tok) {
        return;
    }
    const int64_t pos = tok0 + i;
    const uint8_t * t = tile_of(pv, pv.table + int64_t(slot) * pv.table_stride, layer, head, pos);
    const int32_t tt = static_cast<int32_t>(pos & 31);
    const int32_t d0 = 4 * lane, b = lane >> 3;
    uint8_t * o = out + i * (kBlocks * 34) + b * 34;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        const int32_t d = d0 + e;
        const uint8_t u = kv == 0 ? t[k_code_off(tt, d)] : t[v_code_off(tt, d)];
        o[2 + (d & 31)] = static_cast<uint8_t>(u ^ 0x80u);
    }
    if ((lane & 7) == 0) {
        const uint16_t s = *reinterpret_cast<const uint16_t *>(t + (kv == 0 ? k_scale_off(tt, b) : v_scale_off(tt, b)));
        o[0] = static_cast<uint8_t>(s & 0xff);
        o[1] = static_cast<uint8_t>(s >> 8);
    }
}

// one wave a cell: its 256 codes (int8) and 4 group scales (fp16 bits) of (layer, head, kv) in KV8's form
__global__ __launch_bounds__(256) void export_kv8_kernel(pool_view pv, int32_t slot, int32_t layer, int32_t head,
                                                         int32_t kv, int64_t tok0, int32_t n_tok, int8_t * codes,
                                                         uint16_t * scales) {
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int64_t i = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (i >= n_tok) {
        return;
    }
    const int64_t pos = tok0 + i;
    const uint8_t * t = tile_of(pv, pv.table + int64_t(slot) * pv.table_stride, layer, head, pos);
    const int32_t tt = static_cast<int32_t>(pos & 31);
    const int32_t d0 = 4 * lane;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        const int32_t d = d0 + e;
        const uint8_t u = kv == 0 ? t[k_code_off(tt, d)] : t[v_code_off(tt, d)];
        codes[i * kHeadDim + d] = static_cast<int8_t>(u ^ 0x80u);
    }
    if ((lane & 15) == 0) {
        const int32_t g = lane >> 4, b = 2 * g; // the group's first block holds its scale
        scales[i * (kHeadDim / kKV8Group) + g] =
            *reinterpret_cast<const uint16_t *>(t + (kv == 0 ? k_scale_off(tt, b) : v_scale_off(tt, b)));
    }
}

int append_enqueue(const kv_pool & p, int32_t slot, int32_t layer, int64_t pos0, const int32_t * pos_dev,
                   int64_t max_cells, int32_t rows, const void * k, const void * v, int32_t dtype, hipStream_t st) {
    // K: a wave a row; V: a wave a quad of aligned cells, rows / 4 + 2 quads at most whatever pos0's alignment
    const int64_t waves = int64_t(rows) * p.h_kv() + (int64_t(rows) / 4 + 2) * p.h_kv();
    const uint32_t grid = static_cast<uint32_t>((waves + 3) / 4);
    if (dtype == FNKV_F32) {
        hipLaunchKernelGGL(append_kernel<true>, dim3(grid), dim3(256), 0, st, p.view(), slot, layer, pos0, rows, k, v,
                           pos_dev, max_cells);
    } else {
        hipLaunchKernelGGL(append_kernel<false>, dim3(grid), dim3(256), 0, st, p.view(), slot, layer, pos0, rows, k,
                           v, pos_dev, max_cells);
    }
    return hipGetLastError() == hipSuccess ? FNKV_OK : FNKV_ERR_HIP;
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int fnkv_q8_append(fnkv_pool * pool, int32_t slot, int32_t layer, int64_t pos0, int32_t rows, const void * k,
                   const void * v, int32_t dtype, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || layer < 0 || layer >= p->layers() || rows < 0 ||
        pos0 < 0 || (dtype != FNKV_F16 && dtype != FNKV_F32)) {
        set_error("fnkv_q8_append: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (rows == 0) {
        return FNKV_OK;
    }
    if (k == nullptr || v == nullptr) {
        set_error("fnkv_q8_append: null k or v");
        return FNKV_ERR_ARG;
    }
    if (pos0 + rows > p->mapped_cells(slot)) {
        set_error("fnkv_q8_append: cells " + std::to_string(pos0) + " .. " + std::to_string(pos0 + rows - 1) +
                  " are not all mapped (slot " + std::to_string(slot) + " holds " +
                  std::to_string(p->mapped_cells(slot)) + ")");
        return FNKV_ERR_ARG;
    }
    if (fnkv::append_enqueue(*p, slot, layer, pos0, nullptr, 0, rows, k, v, dtype,
                             static_cast<hipStream_t>(stream)) != FNKV_OK) {
        set_error("fnkv_q8_append: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

int fnkv_export_q8_0(const fnkv_pool * pool, int32_t slot, int32_t layer, int32_t head, int32_t kv, int64_t tok0,
                     int32_t n_tok, void * out, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || layer < 0 || layer >= p->layers() || head < 0 ||
        head >= p->h_kv() || (kv != 0 && kv != 1) || tok0 < 0 || n_tok < 0 || out == nullptr ||
        tok0 + n_tok > p->mapped_cells(slot)) {
        set_error("fnkv_export_q8_0: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (n_tok == 0) {
        return FNKV_OK;
    }
    hipLaunchKernelGGL(fnkv::export_kernel, dim3(static_cast<uint32_t>((n_tok + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p->view(), slot, layer, head, kv, tok0, n_tok,
                       static_cast<uint8_t *>(out));
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_export_q8_0: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

int fnkv_export_kv8(const fnkv_pool * pool, int32_t slot, int32_t layer, int32_t head, int32_t kv, int64_t tok0,
                    int32_t n_tok, void * codes, void * scales, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || p->format() != fnkv::kFormatKV8 || slot < 0 || slot >= p->pages().n_slots() || layer < 0 ||
        layer >= p->layers() || head < 0 || head >= p->h_kv() || (kv != 0 && kv != 1) || tok0 < 0 || n_tok < 0 ||
        codes == nullptr || scales == nullptr || tok0 + n_tok > p->mapped_cells(slot)) {
        set_error("fnkv_export_kv8: argument outside the contract (a KV8 pool's mapped cells)");
        return FNKV_ERR_ARG;
    }
    if (n_tok == 0) {
        return FNKV_OK;
    }
    hipLaunchKernelGGL(fnkv::export_kv8_kernel, dim3(static_cast<uint32_t>((n_tok + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p->view(), slot, layer, head, kv, tok0, n_tok,
                       static_cast<int8_t *>(codes), static_cast<uint16_t *>(scales));
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_export_kv8: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
