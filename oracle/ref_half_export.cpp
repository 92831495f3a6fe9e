// Exports the reference's own f32<->f16 boundary conversion (include/infvino/Half.hpp:14-49,
// src/Half.cpp:19-107, compiled from the reference sources where they lie) under C names, so
// the oracle's restatement (ivo_f2h_trunc / ivo_h2f) can be checked against it bit for bit.
// Test infrastructure only: built into oracle/_ref/, never linked into the product.
#include <cstddef>
#include <cstdint>

#include "infvino/Half.hpp"

extern "C" {
uint16_t ref_f32_to_f16(float f) { return infvino::f32_to_f16(f); }
float ref_f16_to_f32(uint16_t h) { return infvino::f16_to_f32(h); }
void ref_f32_to_f16_bulk(const float * in, uint16_t * out, size_t n) { infvino::f32_to_f16_bulk(in, out, n); }
void ref_f16_to_f32_bulk(const uint16_t * in, float * out, size_t n) { infvino::f16_to_f32_bulk(in, out, n); }
}
