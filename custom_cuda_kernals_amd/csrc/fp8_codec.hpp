// Exact fp32 -> OCP FP8 encoders (e4m3fn, e5m2) with PyTorch's overflow
// conventions, written from the format definitions:
//
//   * round to nearest, ties to even, into the target format;
//   * e4m3fn has no infinity: a magnitude that rounds above 448 (i.e.
//     |v| > 464), +-inf and NaN all encode as NaN = 0x7f | sign;
//   * e5m2 has infinity: |v| >= 61440 (rounds above 57344) and +-inf encode
//     as 0x7c | sign, NaN as 0x7f | sign;
//   * the sign bit is always carried over, so -0.0 -> 0x80.
//
// These are the semantics of `tensor.to(torch.float8_e4m3fn / e5m2)` that the
// reference oracle relies on (baselines/fp8_quant.py:170,177). They are used
// on the GPU only on the rare slow path (non-finite scales, quotients outside
// the range where gfx950's v_cvt_pk_fp8/bf8_f32 was verified to agree), and
// are the ground truth the hardware conversion is checked against.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cck {

__host__ __device__ inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// Round-to-nearest-even of a small non-negative float to an integer
// (v_rndne_f32 on the GPU; the default RNE mode on the host).
__host__ __device__ inline uint32_t rne_small_uint(float t) {
  return (uint32_t)__builtin_rintf(t);
}

__host__ __device__ inline uint32_t encode_e4m3fn(float v) {
  const uint32_t b = f32_bits(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x43E80000u) return sign | 0x7fu;  // NaN, inf, |v| > 464 -> NaN
  if (a < 0x3C800000u) {                     // |v| < 2^-6: subnormal grid 2^-9
    // |v| * 2^9 is exact (power-of-two scaling of a value < 2^-6).
    return sign | rne_small_uint(bits_f32(a) * 512.0f);  // 8 -> 0x08 = 2^-6
  }
  // Normal: keep 3 mantissa bits, RNE at bit 20, then re-bias 127 -> 7.
  const uint32_t odd = (a >> 20) & 1u;
  const uint32_t r = a + 0x7FFFFu + odd - (120u << 23);
  return sign | ((r >> 20) & 0x7fu);
}

__host__ __device__ inline uint32_t encode_e5m2(float v) {
  const uint32_t b = f32_bits(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x7F800000u) return sign | 0x7fu;   // NaN
  if (a >= 0x47700000u) return sign | 0x7cu;  // |v| >= 61440 or inf -> inf
  if (a < 0x38800000u) {                      // |v| < 2^-14: subnormal grid 2^-16
    return sign | rne_small_uint(bits_f32(a) * 65536.0f);
  }
  const uint32_t odd = (a >> 21) & 1u;
  const uint32_t r = a + 0xFFFFFu + odd - (112u << 23);
  return sign | ((r >> 21) & 0x7fu);
}

}  // namespace cck
