// Payload element types and their accumulators.
//
// Sums accumulate 16-bit payloads in fp32 and 32/64-bit payloads in fp64, then
// round once (round-to-nearest-even) to the payload dtype.  Both 16-bit
// conversions are the hardware ones of gfx950, two values per instruction
// (v_cvt_pk_bf16_f32, v_cvt_pk_f16_f32; round to nearest even).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "em_common.h"

namespace rem {

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 (a in the low half).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return (uint16_t)f32x2_to_bf16x2_bits(f, 0.0f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ uint32_t f32x2_to_f16x2_bits(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
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
  static __device__ __forceinline__ uint32_t store2(acc_t a, acc_t b) { return f32x2_to_bf16x2_bits(a, b); }
};

template <>
struct Elem<kF16> {
  using store_t = uint16_t;
  using acc_t = float;
  static __device__ __forceinline__ acc_t load(store_t x) { return f16_bits_to_f32(x); }
  static __device__ __forceinline__ store_t store(acc_t v) { return f32_to_f16_bits(v); }
  static __device__ __forceinline__ uint32_t store2(acc_t a, acc_t b) { return f32x2_to_f16x2_bits(a, b); }
};

}  // namespace rem
