// mrl_half.h -- IEEE binary16 conversions shared by the device code.
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace mrl {

// binary16 -> f32 (exact; half::f16::to_f32)
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return (float)x;
}

// f32 -> IEEE binary16, round to nearest even (half::f16::from_f32)
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t e32 = (int32_t)((x >> 23) & 0xffu);
  const uint32_t man = x & 0x7fffffu;
  if (e32 == 0xff) return sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u);
  const int32_t e = e32 - 112;
  if (e >= 31) return sign | 0x7c00u;
  uint32_t sig, shift, base;
  if (e > 0) {
    sig = man;
    shift = 13;
    base = sign | ((uint32_t)e << 10);
  } else {
    if (e < -10) return sign;
    sig = man | 0x800000u;
    shift = (uint32_t)(14 - e);
    base = sign;
  }
  const uint32_t kept = sig >> shift;
  const uint32_t rem = sig & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  uint32_t out = base + kept;
  if (rem > halfway || (rem == halfway && (kept & 1u))) out += 1u;
  return out & 0xffffu;
}

}  // namespace mrl
