// Payload element types and their accumulators.
//
// Sums accumulate 16-bit payloads in fp32 and 32/64-bit payloads in fp64, then
// round once (round-to-nearest-even) to the payload dtype.  bf16 conversion is
// the standard bias-and-truncate RNE on the fp32 bit pattern; fp16 uses the
// hardware conversion (v_cvt_f16_f32, RNE).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "em_common.h"

namespace rem {

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);  // quiet NaN
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
struct Elem;

template <>
struct Elem<kF32> {
  using store_t = float;
  using acc_t = double;
  static __device__ __forceinline__ acc_t load(store_t x) { return (acc_t)x; }
  static __device__ __forceinline__ store_t store(acc_t v) { return (store_t)v; }
};

template <>
struct Elem<kF64> {
  using store_t = double;
  using acc_t = double;
  static __device__ __forceinline__ acc_t load(store_t x) { return x; }
  static __device__ __forceinline__ store_t store(acc_t v) { return v; }
};

template <>
struct Elem<kBF16> {
  using store_t = uint16_t;
  using acc_t = float;
  static __device__ __forceinline__ acc_t load(store_t x) { return bf16_bits_to_f32(x); }
  static __device__ __forceinline__ store_t store(acc_t v) { return f32_to_bf16_bits(v); }
};

template <>
struct Elem<kF16> {
  using store_t = uint16_t;
  using acc_t = float;
  static __device__ __forceinline__ acc_t load(store_t x) { return f16_bits_to_f32(x); }
  static __device__ __forceinline__ store_t store(acc_t v) { return f32_to_f16_bits(v); }
};

}  // namespace rem
