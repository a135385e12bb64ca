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

// One LDS DMA piece (gfx950 buffer_load_dwordx4 ... lds): 64 lanes x 16 bytes
// from the buffer at per-lane byte offsets into LDS bytes [lds, lds + 1024),
// lane l's 16 bytes at lds + 16 l; an offset past the descriptor's records
// writes zeros. Inline assembly on purpose: the compiler's wait-count pass
// treats the builtin form as an LDS write of unknown extent and puts a full
// vmcnt wait before every later LDS read. Callers wait for their own pieces
// explicitly (wait_vmcnt, then the barrier that publishes them). M0 holds
// the LDS base (gfx9 LDS instructions do not read it), and the s_nop is the
// one wait state an LDS DMA needs after M0 is written.
__device__ __forceinline__ void dma_piece_at(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds,
                                             uint32_t voff) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(base), "v"(voff), "s"(rsrc)
               : "memory");
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

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

// The fp32 value as computed, hidden from the optimizer, so that the rounding
// to a 16-bit type that follows is a rounding of this fp32 value: otherwise
// an fp32 product or sum and its conversion to f16 may become one
// mixed-precision instruction (one rounding where the reference rounds
// twice), and not alike in every kernel that inlines the same code.
__device__ __forceinline__ float held(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Pack two floats into one dword of 16-bit values (lo in bits 0..15).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return uint32_t(Store<T>::bits(lo)) | (uint32_t(Store<T>::bits(hi)) << 16);
}

// Sum over the 64 lanes of a wave, the same bits on every lane, by VALU lane
// exchanges instead of LDS permutes: DPP within each row of 16 lanes (lanes
// i ^ 1, i ^ 2, then the half-row and row mirrors), then the gfx950 row swaps
// (lanes i ^ 16, i ^ 32). Every step adds a lane's value to its partner's,
// and the partner adds the same two values, so all lanes agree. (The QK-norm
// prologue's sum of squares, in its own kernel and inside the decode
// attention launch, so that both round alike.)
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf,
                                                        false));
}
__device__ __forceinline__ float lane_sum64(float x) {
  x = dpp_add<0xb1>(x);   // quad_perm [1, 0, 3, 2]: lane i ^ 1
  x = dpp_add<0x4e>(x);   // quad_perm [2, 3, 0, 1]: lane i ^ 2
  x = dpp_add<0x141>(x);  // row_half_mirror: lane 7 - i within 8
  x = dpp_add<0x140>(x);  // row_mirror: lane 15 - i within 16
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
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
// Argument checks of the QK-norm + rotary prologue (qk_norm_rope.hip), also
// run by the attention launch that does the prologue itself.
int rope_validate(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                  const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                  const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh, int io_dtype,
                  const void* qw, const void* kw, int wdt, const void* cos, int64_t cos_sl,
                  const void* sin, int64_t sin_sl, int tdt, void* q_out, void* k_out,
                  void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                  int64_t capacity, int64_t start, const int32_t* start_dev,
                  int64_t B, int64_t L, int64_t H, int64_t D, bool append);
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
