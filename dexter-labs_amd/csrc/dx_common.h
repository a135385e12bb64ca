// Shared helpers for the gfx950 kernels: element types, vector types, the
// thread-local error slot behind dx_last_error(), and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dexter_gfx950.h"

namespace dx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Storage types. Raw 16-bit containers so that conversions are explicit and
// identical on every path.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(uint32_t(x.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16_t x) {
  return float(__builtin_bit_cast(_Float16, x.bits));
}
__device__ __forceinline__ float to_f32(float x) { return x; }

// Round-to-nearest-even float -> bf16 (gfx950 v_cvt_pk_bf16_f32; the same
// rounding torch's .to(torch.bfloat16) performs; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <typename T> struct Store;
template <> struct Store<bf16_t> {
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_bf16_bits(f); }
};
template <> struct Store<f16_t> {
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_f16_bits(f); }
};

// Pack two floats into one dword of 16-bit values (lo in bits 0..15).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return uint32_t(Store<T>::bits(lo)) | (uint32_t(Store<T>::bits(hi)) << 16);
}

}  // namespace dx

// ---------------------------------------------------------------------------
// Error reporting: every entry point returns 0 or a DX_E* code and leaves a
// message in a thread-local buffer.
// ---------------------------------------------------------------------------
namespace dx {
void set_error(const char* fmt, ...);
// Current value of a dx_set_tuning override (0: the library's own choice).
int tuning(int key);
}

#define DX_CHECK_ARG(cond, ...)                   \
  do {                                            \
    if (!(cond)) {                                \
      ::dx::set_error(__VA_ARGS__);               \
      return DX_EINVAL;                           \
    }                                             \
  } while (0)

#define DX_CHECK_LAUNCH(what)                                              \
  do {                                                                     \
    hipError_t e_ = hipGetLastError();                                     \
    if (e_ != hipSuccess) {                                                \
      ::dx::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
      return DX_ELAUNCH;                                                   \
    }                                                                      \
  } while (0)
