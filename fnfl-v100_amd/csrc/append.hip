// The Q8_0 append (new K/V rows quantized into the pool) and the export back to ggml's block_q8_0.
//
// Quantization rule, bit for bit ggml's quantize_row_q8_0_ref (ggml/src/ggml-quants.c:274-297) on the fp32 value of
// each input: per block of 32, amax = max |x|; d = amax / 127 (IEEE division); id = d != 0 ? 1 / d : 0 (IEEE
// division); code = roundf(x * id) (IEEE product, ties away from zero); the stored scale is fp16(d), round to nearest
// even (ggml-impl.h:414-438). The reference's device writers of its own KV8 format (fn/kernels/qsa/kv_q8.cuh:244-267,
// qsa_prompt_attn.cu:90-122) use one warp a row; here one wave64 quantizes one 256-value row, 4 values a lane, the
// 8 lanes of a block reducing amax with cross-lane max.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace fnkv {

// The quantizer's arithmetic must round at every step as the reference's does (amax / 127, 1 / d, x * id, then
// roundf): no contraction of x * id into the fraction test below. This file is also compiled with -ffp-contract=off.
#pragma clang fp contract(off)

// roundf: round half away from zero, exact (x - trunc(x) is exact in fp32)
__device__ __forceinline__ float round_half_away(float x) {
    const float t = __builtin_truncf(x);
    const float f = x - t;
    return __builtin_fabsf(f) >= 0.5f ? t + __builtin_copysignf(1.0f, x) : t;
}

__device__ __forceinline__ uint8_t * tile_of(const pool_view & pv, int32_t slot, int32_t layer, int32_t head,
                                             int64_t pos) {
    const int32_t phys = pv.table[int64_t(slot) * pv.table_stride + (pos >> 8)];
    return pv.base + int64_t(layer) * pv.layer_stride + int64_t(phys) * pv.page_stride + int64_t(head) * kPageBlock +
           int64_t((pos & 255) >> 5) * kTileBytes;
}

template <bool F32>
__global__ __launch_bounds__(256) void append_kernel(pool_view pv, int32_t slot, int32_t layer, int64_t pos0,
                                                     int32_t rows, const void * __restrict__ kin,
                                                     const void * __restrict__ vin) {
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int64_t w = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int32_t kv = static_cast<int32_t>(w & 1);
    const int64_t rh = w >> 1;
    const int32_t head = static_cast<int32_t>(rh % pv.h_kv);
    const int64_t row = rh / pv.h_kv;
    if (row >= rows) {
        return;
    }
    const int64_t src = (row * pv.h_kv + head) * kHeadDim + 4 * lane;
    float x[4];
    if (F32) {
        const float4 f = *reinterpret_cast<const float4 *>(static_cast<const float *>(kv ? vin : kin) + src);
        x[0] = f.x;
        x[1] = f.y;
        x[2] = f.z;
        x[3] = f.w;
    } else {
        const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const __half *>(kv ? vin : kin) + src);
        x[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.x & 0xffffu)));
        x[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.x >> 16)));
        x[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.y & 0xffffu)));
        x[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.y >> 16)));
    }
    float amax = fmaxf(fmaxf(__builtin_fabsf(x[0]), __builtin_fabsf(x[1])),
                       fmaxf(__builtin_fabsf(x[2]), __builtin_fabsf(x[3])));
    // the 8 lanes of a block: lanes 8 b .. 8 b + 7
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t packed = 0;
    uint8_t bytes[4];
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        const float r = round_half_away(__fmul_rn(x[e], id));
        // an in-contract input gives |r| <= 127; outside it (an fp32 input whose d underflows to a subnormal, so id
        // is inf) the reference's int8 store of roundf keeps the low byte of x86's 0x80000000 result: code 0
        const int32_t c = __builtin_fabsf(r) < 2147483648.0f ? static_cast<int32_t>(r) : INT32_MIN;
        bytes[e] = static_cast<uint8_t>((c & 0xff) ^ 0x80); // excess-128 storage
        packed |= uint32_t(bytes[e]) << (8 * e);
    }
    const int64_t pos = pos0 + row;
    uint8_t * t = tile_of(pv, slot, layer, head, pos);
    const int32_t tt = static_cast<int32_t>(pos & 31);
    const int32_t d0 = 4 * lane, b = lane >> 3;
    if (kv == 0) {
        *reinterpret_cast<uint32_t *>(t + k_code_off(tt, d0)) = packed;
        if ((lane & 7) == 0) {
            *reinterpret_cast<uint16_t *>(t + k_scale_off(tt, b)) = __half_as_ushort(__float2half_rn(d));
        }
    } else {
#pragma unroll
        for (int32_t e = 0; e < 4; ++e) {
            t[v_code_off(tt, d0 + e)] = bytes[e];
        }
        if ((lane & 7) == 0) {
            *reinterpret_cast<uint16_t *>(t + v_scale_off(tt, b)) = __half_as_ushort(__float2half_rn(d));
        }
    }
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
    const uint8_t * t = tile_of(pv, slot, layer, head, pos);
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
    const int64_t waves = int64_t(rows) * p->h_kv() * 2;
    const uint32_t grid = static_cast<uint32_t>((waves + 3) / 4);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == FNKV_F32) {
        hipLaunchKernelGGL(fnkv::append_kernel<true>, dim3(grid), dim3(256), 0, st, p->view(), slot, layer, pos0, rows,
                           k, v);
    } else {
        hipLaunchKernelGGL(fnkv::append_kernel<false>, dim3(grid), dim3(256), 0, st, p->view(), slot, layer, pos0,
                           rows, k, v);
    }
    if (hipGetLastError() != hipSuccess) {
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

} // extern "C"
