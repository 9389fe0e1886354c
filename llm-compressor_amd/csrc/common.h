// Shared helpers for the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi355q.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4_t;

namespace mi355q {

// Thread-local last error message, returned by mi355q_last_error().
void set_error(const char* fmt, ...);

#define MQ_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::mi355q::set_error(__VA_ARGS__);  \
      return MI355Q_INVALID_ARGUMENT;    \
    }                                    \
  } while (0)

#define MQ_CHECK_HIP(expr)                                                   \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess) {                                                  \
      ::mi355q::set_error("%s failed: %s", #expr, hipGetErrorString(_e));    \
      return MI355Q_HIP_ERROR;                                               \
    }                                                                        \
  } while (0)

#define MQ_LAUNCH_CHECK()                                                    \
  do {                                                                       \
    hipError_t _e = hipGetLastError();                                       \
    if (_e != hipSuccess) {                                                  \
      ::mi355q::set_error("kernel launch failed: %s", hipGetErrorString(_e));\
      return MI355Q_HIP_ERROR;                                               \
    }                                                                        \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- bf16 bits
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet).  Device
// code takes gfx950's v_cvt_pk_bf16_f32 (IEEE round to nearest even, NaN in
// NaN out); the host pass the same rounding from the bits.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
#else
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
#endif
}

__host__ __device__ inline float round_to_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// IEEE operations kept separate: the library is compiled with
// -ffp-contract=off, so a*b-c is a rounded multiply and a rounded subtract as
// in the reference's separate tensor ops; fp32 division is correctly rounded
// (hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt).
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float sub_rn(float a, float b) { return a - b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }

// ---------------------------------------------------------------- float grids
// float8_e4m3fn round to nearest even of |v| <= 448 (the clamp comes first):
// the grid step is 2^(max(floor(log2 |v|), -6) - 3), a power of two, so the
// scaling, rint and rescaling are exact; the sign (also of a zero) is kept,
// as the cast keeps it.
__device__ __forceinline__ float fp8e4m3_rne(float v) {
  const float a = fabsf(v);
  const int e = (int)((__float_as_uint(a) >> 23) & 0xffu) - 127;
  const int qe = (e > -6 ? e : -6) - 3;
  const float r = rintf(a * __uint_as_float((uint32_t)(127 - qe) << 23)) * __uint_as_float((uint32_t)(127 + qe) << 23);
  return copysignf(r, v);
}
// its float8_e4m3fn bit pattern (v on the grid)
__device__ __forceinline__ uint32_t fp8e4m3_bits(float v) {
  const uint32_t sgn = (__float_as_uint(v) >> 31) << 7;
  const float a = fabsf(v);
  if (a == 0.f) return sgn;
  const int e = (int)((__float_as_uint(a) >> 23) & 0xffu) - 127;
  if (e < -6) return sgn | (uint32_t)rintf(a * 512.f);                       // subnormal: a / 2^-9
  return sgn | ((uint32_t)(e + 7) << 3) | ((__float_as_uint(a) >> 20) & 7u);  // normal
}
// compressed-tensors cast_to_fp4 (e2m1) of |x| <= 6 (the clamp comes
// first): its thresholds (<= .25, < .75, <= 1.25, < 1.75, <= 2.5, < 3.5,
// <= 5) are round-to-nearest-even on the grid {0, .5, 1, 1.5, 2, 3, 4, 6},
// whose step is .5 below 2, 1 below 4 and 2 above, so rint of |x| / step is
// exact; the sign is applied by multiplying with sign(x) (so (-0.25, 0) gives
// -0 and -0 gives +0)
__device__ __forceinline__ float fp4e2m1_round(float x) {
  const float a = fabsf(x);
  const float step = a < 2.f ? 0.5f : a < 4.f ? 1.f : 2.f;
  const float rstep = a < 2.f ? 2.f : a < 4.f ? 1.f : 0.5f;
  const float o = rintf(a * rstep) * step;
  return x < 0.f ? -o : o;
}
// its e2m1 code: sign << 3 | index of |v| in {0, .5, 1, 1.5, 2, 3, 4, 6}
__device__ __forceinline__ uint32_t fp4e2m1_bits(float v) {
  const float a = fabsf(v);
  const uint32_t i = a < 2.f ? (uint32_t)(a * 2.f) : a < 4.f ? (uint32_t)(a) + 2u : a < 6.f ? 6u : 7u;
  return ((__float_as_uint(v) >> 31) << 3) | i;
}

}  // namespace mi355q
