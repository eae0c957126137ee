// lgx_gen.h -- seeded tensor generator of the random-init models (see lgx_gen.cpp).
#pragma once
#include <stdint.h>

namespace lgxg {
uint64_t stream_base(uint64_t seed, uint64_t stream);
uint16_t f32_to_f16(float f);
void gen_i8(uint64_t seed, uint64_t stream, int8_t* out, int64_t n);
void gen_q8_scales(uint64_t seed, uint64_t stream, uint16_t* out, int64_t n);
void gen_normal_f16(uint64_t seed, uint64_t stream, double sigma, uint16_t* out, int64_t n);
void gen_normal_f32(uint64_t seed, uint64_t stream, double sigma, float* out, int64_t n);
void gen_permutation(uint64_t seed, uint64_t stream, int32_t* out, int64_t n);
}  // namespace lgxg
