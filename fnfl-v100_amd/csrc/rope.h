// Shared by the attention launches that prepare their own query and key rows (DA-TC's prepare, the pool's QSA
// attend): the F32 RMS norm and IMROPE of a 256-wide row, F16 packing, and FNFL's int8 activation format of an output
// run of 32 values.
#pragma once

#include "mfma.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fnkv {

constexpr int32_t kNRot = 64;    // rotated dimensions (fn/kernels/qsa/qsa.h n_rot)
constexpr float kRmsEps = 1e-6f; // fn/model/shapes.h:35 rms_eps

// The F32 rms norm and IMROPE of one 256-wide row (pinned by the reference as build_norm LLM_NORM_RMS, then
// ggml_rope_multi with GGML_ROPE_TYPE_IMROPE; fn/kernels/qsa/attend.cu:151-198, imrope.cuh:14-20). A lane holds dims
// 4 lane .. 4 lane + 3. Rotation pair i (< 32) is dims i and i + 32; its angle is its plane's position times
// theta_scale^i as the F32 product chain, the plane picked by the sector rule (sections 11, 11, 10, 0).
// Split in three for callers that issue the loads early: rope_pos (the lane's plane position), rope_angle (the lane's
// pair angle as sin / cos, shared by every row at one position), norm_rope_apply (the norm and rotation of a loaded row).
__device__ __forceinline__ int32_t rope_plane(int32_t lane) {
    const int32_t sector = lane & 31;
    return sector % 3 == 1 && sector < 33   ? 1
           : sector % 3 == 2 && sector < 30 ? 2
           : sector % 3 == 0 && sector < 33 ? 0
                                            : 3;
}

__device__ __forceinline__ int32_t rope_pos(const int32_t * pos, int32_t stride, int32_t col, int32_t lane) {
    return pos[rope_plane(lane) * stride + col];
}

// lane i < 32 forms pair i's angle
// The arithmetic is as written in every file that includes this (no contraction of a * b + c into one rounding, whatever
// the file's flags), so every launch that prepares a row computes the same bits.
__device__ __forceinline__ void rope_angle(float & s, float & c, int32_t p, float ts, int32_t lane) {
#pragma clang fp contract(off)
    const int32_t sector = lane & 31;
    float theta = static_cast<float>(p);
#pragma unroll
    for (int32_t i = 0; i < kNRot / 2 - 1; ++i) {
        theta = i < sector ? theta * ts : theta;
    }
    s = 0.0f;
    c = 0.0f;
    sincosf(theta, &s, &c);
}

__device__ __forceinline__ void norm_rope_apply(float (&y)[4], const float4 x, const float4 g, float s, float c,
                                                int32_t lane) {
#pragma clang fp contract(off)
    float ss = x.x * x.x;
    ss = __builtin_fmaf(x.y, x.y, ss);
    ss = __builtin_fmaf(x.z, x.z, ss);
    ss = __builtin_fmaf(x.w, x.w, ss);
#pragma unroll
    for (int32_t o = 32; o > 0; o >>= 1) {
        ss += __shfl_xor(ss, o, 64);
    }
    const float r = 1.0f / sqrtf(ss * (1.0f / 256.0f) + kRmsEps);
    y[0] = x.x * r * g.x;
    y[1] = x.y * r * g.y;
    y[2] = x.z * r * g.z;
    y[3] = x.w * r * g.w;
    // dims 0..31 sit in lanes 0..7, their partners 32..63 in lanes 8..15
#pragma unroll
    for (int32_t e = 0; e < 4; ++e) {
        const int32_t pair = 4 * (lane & 7) + e;
        const float ce = __shfl(c, pair, 64);
        const float se = __shfl(s, pair, 64);
        const float other = __shfl_xor(y[e], 8, 64);
        if (lane < 8) {
            y[e] = y[e] * ce - other * se;
        } else if (lane < 16) {
            y[e] = other * se + y[e] * ce;
        }
    }
}

__device__ __forceinline__ void norm_rope(float (&y)[4], const float * src, const float * w, const int32_t * pos,
                                          int32_t stride, int32_t col, float ts, int32_t lane) {
    const float4 x = reinterpret_cast<const float4 *>(src)[lane];
    const float4 g = reinterpret_cast<const float4 *>(w)[lane];
    float s, c;
    rope_angle(s, c, rope_pos(pos, stride, col, lane), ts, lane);
    norm_rope_apply(y, x, g, s, c, lane);
}

__device__ __forceinline__ uint2 pack4_f16(const float (&x)[4], float scale) {
    half2v a{static_cast<_Float16>(x[0] * scale), static_cast<_Float16>(x[1] * scale)};
    half2v b{static_cast<_Float16>(x[2] * scale), static_cast<_Float16>(x[3] * scale)};
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

// FNFL's activation format of one run of 32 values held by `width` consecutive lanes (32 / width values each), the rule
// of fn/kernels/act/act_warp.cuh:12-20 and fn/quant/act_ref.cpp:8-29: amax = max |x| (NaN ignored), d = amax / 127,
// id = 127 / amax (0 when amax is 0), q = round-to-even of x id clamped to [-127, 127] (NaN: 0), s = d * sum q (the sum
// exact in int32). Every lane of the run takes part; the run's first lane gets {d, s} through `ds`.
template <int N, int WIDTH>
__device__ __forceinline__ void act_run(const float (&y)[N], int8_t (&q)[N], float (&ds)[2]) {
    static_assert(N * WIDTH == 32, "a run is 32 values");
    float amax = 0.0f;
#pragma unroll
    for (int32_t e = 0; e < N; ++e) {
        amax = fmaxf(amax, fabsf(y[e]));
    }
#pragma unroll
    for (int32_t o = WIDTH / 2; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    }
    const float d = amax / 127.0f;
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t sum = 0;
#pragma unroll
    for (int32_t e = 0; e < N; ++e) {
        const float v = y[e] * id;
        const int32_t c = v != v ? 0 : static_cast<int32_t>(fminf(fmaxf(__builtin_rintf(v), -127.0f), 127.0f));
        q[e] = static_cast<int8_t>(c);
        sum += c;
    }
#pragma unroll
    for (int32_t o = WIDTH / 2; o > 0; o >>= 1) {
        sum += __shfl_xor(sum, o, 64);
    }
    ds[0] = d;
    ds[1] = d * static_cast<float>(sum);
}

} // namespace fnkv
