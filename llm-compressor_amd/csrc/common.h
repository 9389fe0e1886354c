// Shared helpers for the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi355q.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
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

// Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet).
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
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

}  // namespace mi355q
