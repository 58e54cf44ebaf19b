// The quantizers of one 256-value row by one wave64 (Q8_0 and KV8), shared by the append kernel and the decode
// kernel's fused append. Rule, bit for bit ggml's quantize_row_q8_0_ref (ggml/src/ggml-quants.c:274-297) on the fp32 value of each
// input: per block of 32, amax = max |x|; d = amax / 127 (IEEE division); id = d != 0 ? 1 / d : 0 (IEEE division);
// code = roundf(x * id) (IEEE product, ties away from zero); the stored scale is fp16(d), round to nearest even
// (ggml-impl.h:414-438). Lane l holds values 4 l .. 4 l + 3; the 8 lanes of a block reduce amax with cross-lane max.
#pragma once

#include "layout.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace fnkv {

// roundf: round half away from zero, exact (x - trunc(x) is exact in fp32)
__device__ __forceinline__ float round_half_away(float x) {
#pragma clang fp contract(off)
    const float t = __builtin_truncf(x);
    const float f = x - t;
    return __builtin_fabsf(f) >= 0.5f ? t + __builtin_copysignf(1.0f, x) : t;
}

// the 32-token tile of pool position pos, for (layer, head), through the slot's page table row
__device__ __forceinline__ uint8_t * tile_of(const pool_view & pv, const int32_t * table_row, int32_t layer,
                                             int32_t head, int64_t pos) {
    const int32_t phys = table_row[pos >> 8];
    return pv.base + int64_t(layer) * pv.layer_stride + int64_t(phys) * pv.page_stride + int64_t(head) * kPageBlock +
           int64_t((pos & 255) >> 5) * kTileBytes;
}

// load this lane's 4 values of a 256-value row (fp16 or fp32) as fp32
template <bool F32> __device__ __forceinline__ void load4(const void * row, int32_t lane, float (&x)[4]) {
    if (F32) {
        const float4 f = *reinterpret_cast<const float4 *>(static_cast<const float *>(row) + 4 * lane);
        x[0] = f.x;
        x[1] = f.y;
        x[2] = f.z;
        x[3] = f.w;
    } else {
        const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(row) + 4 * lane);
        x[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.x & 0xffffu)));
        x[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.x >> 16)));
        x[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.y & 0xffffu)));
        x[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(u.y >> 16)));
    }
}

// Q8_0: this wave's row (x: the lane's 4 values) -> the lane's 4 codes as excess-128 bytes (byte e = value 4 lane + e)
// and the block's fp16 scale bits (the same in the block's 8 lanes)
__device__ __forceinline__ void quantize_q8_0(const float (&x)[4], uint32_t & packed, uint16_t & sbits) {
#pragma clang fp contract(off)
    // amax as ggml's running MAX(amax, |x_j|) (MAX(a, b) = a > b ? a : b) over the block in order: a NaN makes the
    // running value NaN and the next value replaces it, so amax is the max |x| after the block's last NaN, and NaN
    // when that NaN is the block's last value. The 8 lanes of a block are lanes 8 b .. 8 b + 7; this lane's values
    // are the block's 4 (lane % 8) .. + 3.
    const int32_t base = (static_cast<int32_t>(__lane_id()) & 7) * 4;
    int32_t last_nan = -1;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        last_nan = x[e] != x[e] ? base + e : last_nan;
    }
    last_nan = max(last_nan, __shfl_xor(last_nan, 1));
    last_nan = max(last_nan, __shfl_xor(last_nan, 2));
    last_nan = max(last_nan, __shfl_xor(last_nan, 4));
    float amax = 0.0f;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        amax = base + e > last_nan ? fmaxf(amax, __builtin_fabsf(x[e])) : amax;
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    if (last_nan == kQK - 1) {
        amax = __builtin_nanf("");
    }
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    packed = 0;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        const float r = round_half_away(x[e] * id);
        // an in-contract input gives |r| <= 127; outside it (an fp32 input whose d underflows to a subnormal, so id
        // is inf) the reference's int8 store of roundf keeps the low byte of x86's 0x80000000 result: code 0
        const int32_t c = __builtin_fabsf(r) < 2147483648.0f ? static_cast<int32_t>(r) : INT32_MIN;
        packed |= uint32_t((c & 0xff) ^ 0x80) << (8 * e); // excess-128 storage
    }
    // ggml's fp32 -> fp16 (ggml-impl.h) gives every NaN as sign | 0x7e00 (here the sign of |x|: +)
    sbits = d != d ? static_cast<uint16_t>(0x7e00) : __half_as_ushort(__float2half_rn(d));
}

// The KV8 rule, bit for bit FNFL's kv_q8_quantize_group (fn/quant/kv_q8_ref.cpp:72-87; device kv8::quantize8,
// fn/kernels/qsa/kv_q8.cuh:29-52): per group of 64 values amax = max |x|; the scale is fp16(amax / 127) (IEEE
// division, round to nearest even), s its exact value; code = 0 when s == 0, else clamp(rint(x / s), -127, 127)
// (IEEE division, ties to even). The 16 lanes of a group (lanes 16 g .. 16 g + 15) reduce amax; the group's scale is
// stored at both of its 32-value blocks.
__device__ __forceinline__ void quantize_kv8(const float (&x)[4], uint32_t & packed, uint16_t & sbits) {
#pragma clang fp contract(off)
    float amax = fmaxf(fmaxf(__builtin_fabsf(x[0]), __builtin_fabsf(x[1])),
                       fmaxf(__builtin_fabsf(x[2]), __builtin_fabsf(x[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 8));
    const __half h = __float2half_rn(__fdiv_rn(amax, 127.0f));
    const float sv = __half2float(h);
    packed = 0;
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        int32_t c = 0;
        if (sv > 0.0f) {
            const float r = __builtin_rintf(__fdiv_rn(x[e], sv));
            c = r < -127.0f ? -127 : r > 127.0f ? 127 : static_cast<int32_t>(r);
        }
        packed |= uint32_t((c & 0xff) ^ 0x80) << (8 * e);
    }
    sbits = __half_as_ushort(h);
}

// the pool's rule (format: kFormatQ8_0 or kFormatKV8, uniform across the wave)
__device__ __forceinline__ void quantize_fmt(const float (&x)[4], int32_t format, uint32_t & packed,
                                             uint16_t & sbits) {
    if (format == kFormatKV8) {
        quantize_kv8(x, packed, sbits);
    } else {
        quantize_q8_0(x, packed, sbits);
    }
}

// one quantized row as cell tt of `tile` (kv: 0 K, 1 V): K's 4 codes of a lane are adjacent (one dword store); V's sit
// in 4 rows of the transposed layout (4 byte stores: the append kernel writes V four cells at a time instead)
__device__ __forceinline__ void store_row(uint32_t packed, uint16_t sbits, int32_t lane, uint8_t * tile, int32_t tt,
                                          int32_t kv) {
    const int32_t d0 = 4 * lane, b = lane >> 3;
    if (kv == 0) {
        *reinterpret_cast<uint32_t *>(tile + k_code_off(tt, d0)) = packed;
        if ((lane & 7) == 0) {
            *reinterpret_cast<uint16_t *>(tile + k_scale_off(tt, b)) = sbits;
        }
    } else {
#pragma unroll
        for (int32_t e = 0; e < 4; ++e) {
            tile[v_code_off(tt, d0 + e)] = static_cast<uint8_t>(packed >> (8 * e));
        }
        if ((lane & 7) == 0) {
            *reinterpret_cast<uint16_t *>(tile + v_scale_off(tt, b)) = sbits;
        }
    }
}

// V rows of the four cells tt0 .. tt0 + 3 (tt0 a multiple of 4) of `tile`, those with bit i of `valid` set: the four
// cells' bytes of one value are adjacent in the V layout (slots s .. s + 3 of one 16-byte row), so a lane writes one
// dword a value, and the block's four scales are adjacent too (one 8-byte store); a partial quad writes its bytes one
// by one (other launches' cells of the quad are left as they are)
__device__ __forceinline__ void store_v_quad(const uint32_t (&packed)[4], const uint16_t (&sbits)[4], uint32_t valid,
                                             int32_t lane, uint8_t * tile, int32_t tt0) {
    const int32_t d0 = 4 * lane, b = lane >> 3;
    if (valid == 0xfu) {
#pragma unroll
        for (int32_t e = 0; e < 4; ++e) {
            const uint32_t w = ((packed[0] >> (8 * e)) & 0xffu) | (((packed[1] >> (8 * e)) & 0xffu) << 8) |
                               (((packed[2] >> (8 * e)) & 0xffu) << 16) | (((packed[3] >> (8 * e)) & 0xffu) << 24);
            *reinterpret_cast<uint32_t *>(tile + v_code_off(tt0, d0 + e)) = w;
        }
        if ((lane & 7) == 0) {
            *reinterpret_cast<uint2 *>(tile + v_scale_off(tt0, b)) =
                make_uint2(uint32_t(sbits[0]) | (uint32_t(sbits[1]) << 16), uint32_t(sbits[2]) | (uint32_t(sbits[3]) << 16));
        }
    } else {
#pragma unroll
        for (int32_t i = 0; i < 4; ++i) {
            if ((valid >> i) & 1u) {
                store_row(packed[i], sbits[i], lane, tile, tt0 + i, 1);
            }
        }
    }
}

// quantize this wave's row (x: the lane's 4 values) by the pool's rule and store it as cell tt of `tile`
__device__ __forceinline__ void quantize_store_fmt(const float (&x)[4], int32_t lane, uint8_t * tile, int32_t tt,
                                                   int32_t kv, int32_t format) {
    uint32_t packed;
    uint16_t sbits;
    quantize_fmt(x, format, packed, sbits);
    store_row(packed, sbits, lane, tile, tt, kv);
}

} // namespace fnkv
