// CDNA4 building blocks shared by the attention kernels: operand types of v_mfma_f32_16x16x32_f16, the exact widening
// of 8 stored (excess-128) codes to fp16, LDS direct loads and the vmcnt wait that orders them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fnkv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// D = A B + C with A 16x32 (lane l: row l % 16, slots 8 (l / 16) .. + 7), B 32x16 (lane l: column l % 16, the same
// slots), D 16x16 (lane l: rows 4 (l / 16) .. + 3 of column l % 16)
__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// two excess-128 code bytes u0, u1 of `w` (selected by `sel`) become fp16 1024 + u, then minus 1152: the codes
// u - 128 exactly
__device__ __forceinline__ uint32_t widen2(uint32_t w, uint32_t sel) {
    const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, w, sel);
    half2v h = __builtin_bit_cast(half2v, biased);
    h = h - half2v{static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    return __builtin_bit_cast(uint32_t, h);
}

// 8 codes (two dwords, byte i = slot i) as the fp16 operand
__device__ __forceinline__ half8 widen8(uint32_t lo, uint32_t hi) {
    u32x4 r;
    r[0] = widen2(lo, 0x04010400u);
    r[1] = widen2(lo, 0x04030402u);
    r[2] = widen2(hi, 0x04010400u);
    r[3] = widen2(hi, 0x04030402u);
    return __builtin_bit_cast(half8, r);
}

// x - fp16 value h as one mixed-precision FMA (v_fma_mix_f32 reading the fp16 operand in place: half `HI` of the
// packed pair), exact when h is x truncated to fp16
template <int HI> __device__ __forceinline__ float sub_f16(float x, uint32_t h2) {
    float r;
    if constexpr (HI) {
        __asm__("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    } else {
        __asm__("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    }
    return r;
}

// x (8 fp32 values) as hi + lo, both fp16: hi = x rounded toward zero, lo = the remainder rounded toward zero, so
// hi + lo carries x to about 22 bits (the remainder of a truncation to fp16 is exact in fp32)
__device__ __forceinline__ void split_hilo(const float (&x)[8], half8 & hi, half8 & lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t hv = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[2 * i], x[2 * i + 1]));
        const float r0 = sub_f16<0>(x[2 * i], hv);
        const float r1 = sub_f16<1>(x[2 * i + 1], hv);
        h[i] = hv;
        l[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
    }
    hi = __builtin_bit_cast(half8, h);
    lo = __builtin_bit_cast(half8, l);
}

// the sum of 8 values as a balanced tree (three dependent adds instead of eight)
__device__ __forceinline__ float sum8(const float (&x)[8]) {
    return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}

// 8 codes as the fp16 values 1152 + code (one byte permute per two codes): the operand when the 1152 bias is folded
// out elsewhere (into the MFMA's C input, or by an MFMA against the constant -1152)
__device__ __forceinline__ half8 widen8_biased(uint32_t lo, uint32_t hi) {
    u32x4 r;
    r[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
    r[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
    r[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
    r[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
    return __builtin_bit_cast(half8, r);
}

// 8 codes as fp16 values: 1152 + code (EXACT false: the bias is folded out elsewhere), or the code itself (the
// biased integers less 1152, exact)
template <bool EXACT> __device__ __forceinline__ half8 widen8(uint32_t lo, uint32_t hi) {
    half8 w = widen8_biased(lo, hi);
    if constexpr (EXACT) {
        const _Float16 b = static_cast<_Float16>(1152.0f);
        w = w - half8{b, b, b, b, b, b, b, b};
    }
    return w;
}

// p (8 fp32 values, and the same rounded toward zero to fp16) times s (8 fp16) as hi + lo fp16: hi = fp16(ph * s)
// (packed multiply), lo = the fp32 remainder p * s - hi (one fused multiply-add, exact to fp32) rounded toward zero
// (RNE: to nearest). hi + lo carries p * s to about 2^-19 relative, and to 2^-24 (2^-25 RNE) absolute where lo is
// subnormal.
template <bool RNE = false>
__device__ __forceinline__ void scale_hilo(const float (&p)[8], half8 ph, half8 s, half8 & hi, half8 & lo) {
    hi = ph * s;
    if constexpr (RNE) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            lo[i] = static_cast<_Float16>(__builtin_fmaf(p[i], static_cast<float>(s[i]), -static_cast<float>(hi[i])));
        }
        return;
    }
    u32x4 l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float r0 = __builtin_fmaf(p[2 * i], static_cast<float>(s[2 * i]), -static_cast<float>(hi[2 * i]));
        const float r1 =
            __builtin_fmaf(p[2 * i + 1], static_cast<float>(s[2 * i + 1]), -static_cast<float>(hi[2 * i + 1]));
        l[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
    }
    lo = __builtin_bit_cast(half8, l);
}

// (ph + pl) times s (8 fp16 each) as hi + lo fp16 with packed fp16 arithmetic only: hi = fp16(ph * s), the exact
// remainder ph * s - hi (a fused multiply-add; exact while it is not subnormal), then lo = fp16(pl * s + remainder).
// With ph + pl carrying p to 2^-20, hi + lo carries p * s to about 2^-20 relative.
__device__ __forceinline__ void scale_hilo_pk(half8 ph, half8 pl, half8 s, half8 & hi, half8 & lo) {
    hi = ph * s;
    const half8 rem = __builtin_elementwise_fma(ph, s, -hi);
    lo = __builtin_elementwise_fma(pl, s, rem);
}

// x combined across the wave's four 16-lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48) by two lane swaps on the VALU
// (v_permlane16_swap, v_permlane32_swap), without the LDS round trip of a shuffle
// (the max as plain v_max_f32: the lane-swapped values are scores, never NaN, so no canonicalization is needed)
__device__ __forceinline__ float max_plain(float a, float b) {
    float r;
    __asm__("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max_plain(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max_plain(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 8 fp32 values rounded toward zero to fp16
__device__ __forceinline__ half8 to_half8_rtz(const float (&x)[8]) {
    u32x4 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[2 * i], x[2 * i + 1]));
    }
    return __builtin_bit_cast(half8, h);
}

// The kernels wait for their LDS copies by counting the loads issued after them (s_waitcnt vmcnt(n)), so every copy
// must be issued, in program order. LLVM models a copy as a plain store to its LDS pointer: it deletes one that a later
// identical copy overwrites (the duplicate copies that keep a wave's count uniform) and may move register loads across
// it. The empty asm after each copy reads and writes all memory as far as the compiler knows, which forbids both.
__device__ __forceinline__ void keep_issued() { __asm__ __volatile__("" ::: "memory"); }

// Cache policy of the streaming loads (the KV tiles, read once a launch): the nontemporal bit (gfx950 "nt"). A plain
// 16 B-a-lane read of a 2 GiB buffer reaches ~6.1 TB/s on MI355X, the same with nt ~7.1 TB/s.
#ifndef FNKV_STREAM_AUX
#define FNKV_STREAM_AUX 2
#endif
constexpr int kStreamAux = FNKV_STREAM_AUX;

// a wave's 64 x 16 B from global memory straight into LDS at lds_base + 16 lane (no registers); OFF (< 4096) is added
// to both the global and the LDS address
template <int OFF = 0> __device__ __forceinline__ void lds_load16(const void * gptr, void * lds_base) {
    typedef __attribute__((address_space(3))) void lds_void;
    __builtin_amdgcn_global_load_lds(gptr, (lds_void *)lds_base, 16, OFF, kStreamAux);
    keep_issued();
}

// 16 B a lane from global memory into registers, with the streaming cache policy
__device__ __forceinline__ u32x4 stream_load16(const void * gptr) {
    if constexpr (kStreamAux != 0) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gptr));
    } else {
        return *reinterpret_cast<const u32x4 *>(gptr);
    }
}

// Buffer-resource loads: the tile's address lives in four SGPRs, so a lane's address is one VGPR offset (lane * 16)
// plus scalar and immediate offsets, with no 64-bit address arithmetic in VGPRs. The descriptor is a raw buffer
// (stride 0) of `bytes` bytes with the 32-bit data format gfx9 raw loads need.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// a pointer every lane of the wave holds, made provably uniform (scalar registers): a descriptor the compiler cannot
// prove uniform becomes a readfirstlane loop around every load that uses it
__device__ __forceinline__ const void * uniform_ptr(const void * p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(v)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(v >> 32)));
    return reinterpret_cast<const void *>((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ rsrc_t make_rsrc(const void * base, int32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(uniform_ptr(base)), 0, bytes, 0x00020000);
}
// 16 B a lane at base + voff + soff into registers
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, int32_t voff, int32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kStreamAux));
}
// a wave's 64 x 16 B at base + soff + 16 lane straight into LDS at lds_base + 16 lane (cache policy AUX: the streaming
// bit, or 0 where another wave reads the same bytes right after)
template <int AUX = kStreamAux>
__device__ __forceinline__ void buf_lds16(rsrc_t r, void * lds_base, int32_t voff, int32_t soff) {
    typedef __attribute__((address_space(3))) void lds_void;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_base, 16, voff, soff, 0, AUX);
    keep_issued();
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8)
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The workgroup's waves meet at an s_barrier after their LDS reads have returned (lgkmcnt(0)) but with their global
// loads still in flight: __syncthreads would also wait for every outstanding global load, prefetches included. The
// empty asm statements keep the compiler from moving memory accesses across the barrier. LDS data written by a
// global_load_lds is visible to the other waves once the issuing wave has waited for it (vmcnt) before the barrier.
__device__ __forceinline__ void barrier_keep_loads() {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    __asm__ __volatile__("" ::: "memory");
}

} // namespace fnkv
