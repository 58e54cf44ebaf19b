// TEST INFRASTRUCTURE ONLY: C entry points over the reference's own quantizer sources, compiled by oracle/Makefile
// from /root/reference into oracle/_ref/ (never committed, never part of the product). tests/golden/make_golden.py
// calls these to write golden vectors, and tests/test_oracle.py checks the C oracle against them where the library
// was built. Each function forwards to the reference's code unchanged:
//   fnkv_ref_q8_0_quantize   ggml/src/ggml-quants.c:274-297 quantize_row_q8_0_ref (block_q8_0 AoS out, 34 B a block)
//   fnkv_ref_q8_0_dequantize ggml/src/ggml-quants.c:551-565 dequantize_row_q8_0
//   fnkv_ref_f32_to_f16 / fnkv_ref_f16_to_f32   ggml/src/ggml-impl.h:391-438 (static inline in the header)
//   fnkv_ref_kv8_quantize    fn/quant/kv_q8_ref.cpp:89-93 kv_q8_quantize (FNFL's group-64 rule)
//   fnkv_ref_f16_bits_rn / fnkv_ref_f16_value   fn/quant/kv_q8_ref.cpp:10-70
//   fnkv_ref_stress_rows     fn/quant/kv_q8_ref.cpp:99-169 kv_q8_stress_rows
//   fnkv_ref_act_quantize    fn/quant/act_ref.cpp:8-29 act_quantize_ref (the int8 activation format)
#include "fn/quant/act_ref.h"
#include "fn/quant/kv_q8_ref.h"

#include <cstdint>
#include <cstring>
#include <vector>

extern "C" {

void fnkv_ref_kv8_quantize(const float * x, int32_t n, int8_t * codes, uint16_t * scales) {
    fn::quant::kv_q8_quantize(x, n, codes, scales);
}

void fnkv_ref_f16_bits_rn(const float * x, int64_t n, uint16_t * y) {
    for (int64_t i = 0; i < n; ++i) y[i] = fn::quant::f16_bits_rn(x[i]);
}

void fnkv_ref_f16_value(const uint16_t * x, int64_t n, float * y) {
    for (int64_t i = 0; i < n; ++i) y[i] = fn::quant::f16_value(x[i]);
}

// the stress rows' value count for (seed, random_rows); copies up to cap values into out when out is set
int64_t fnkv_ref_stress_rows(uint64_t seed, int32_t random_rows, float * out, int64_t cap) {
    const std::vector<float> v = fn::quant::kv_q8_stress_rows(seed, random_rows);
    if (out != nullptr) {
        std::memcpy(out, v.data(), sizeof(float) * size_t(cap < int64_t(v.size()) ? cap : int64_t(v.size())));
    }
    return int64_t(v.size());
}

void fnkv_ref_act_quantize(const float * x, int32_t rows, int32_t k, int8_t * codes, float * scales) {
    fn::quant::act_quantize_ref(x, rows, k, codes, scales);
}

}  // extern "C"
