// Adaptive LayerNorm modulation and gated residual for gfx950.
//
//   adaln_modulate : out = layer_norm(x over C) * (1 + scale) + shift
//   gated_residual : out = x + y * gate
//
// Both are one read and one write of the [rows, C] activation (the modulation
// rows are [B, 1, C] in a Wan block and come from L2), so the whole design is
// about HBM streaming:
//
//  * One workgroup per row, `nw` waves (chosen on the host from C). Lane l of
//    wave w owns the 16-byte packs (v*nw + w)*64 + l, v = 0..kPacks-1, so every
//    load instruction of a wave reads 1 KB of consecutive bytes (x in bf16). The row sits
//    in registers between the statistics and the output: x is read once.
//  * Statistics in fp32, two passes over the registers (mean, then the mean
//    of squared deviations), reduced inside the wave with DPP (quad swaps,
//    half-row and row mirrors) and four lane reads, across waves through LDS.
//    Every lane and wave ends with the same value.
//  * scale/shift/gate loads are issued right after the x loads, before the
//    reductions, so their latency hides behind them.
//  * Output in fp32, rounded once to the output dtype, which is the torch
//    promotion of the input dtypes (the reference's expression promotes).
//
// Ragged C (not a multiple of the pack width) or rows that are not 16-byte
// aligned take the element-wise variant of the same kernel (kAligned=false):
// the same registers, with element i of a lane's pack 64 columns after
// element i-1, so each element load of a wave is still one contiguous run.
#include "dx_common.h"

#include <algorithm>

namespace dx {
namespace {

constexpr int kPacks = 4;      // 16-byte packs per lane (registers hold the row)
constexpr int kMaxWaves = 16;  // waves per row (workgroup of up to 1024 lanes)

// ---------------------------------------------------------------------------
// Element types: bytes, and float <-> raw 32-bit words.
// ---------------------------------------------------------------------------
template <typename T> struct Ty;
template <> struct Ty<bf16_t> {
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float get(const uint32_t* w, int i) {
    const uint32_t x = w[i >> 1];
    return __uint_as_float((i & 1) ? (x & 0xffff0000u) : (x << 16));
  }
};
template <> struct Ty<f16_t> {
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float get(const uint32_t* w, int i) {
    const uint16_t h = uint16_t(w[i >> 1] >> ((i & 1) * 16));
    return float(__builtin_bit_cast(_Float16, h));
  }
};
template <> struct Ty<float> {
  static constexpr int kBytes = 4;
  static __device__ __forceinline__ float get(const uint32_t* w, int i) {
    return __uint_as_float(w[i]);
  }
};

// torch's promotion for the pairs these kernels take: equal types stay, any
// other pair (bf16/f16 mixed, or with f32) becomes f32.
template <typename A, typename B> struct Promote { using type = float; };
template <typename A> struct Promote<A, A> { using type = A; };

// Raw buffer descriptor of one row (word 3 of the gfx9-family raw layout).
// Loads past num_records return zeros and stores past it are dropped, so the
// ragged end of a row needs no branches.
constexpr int kBufWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes),
                                           kBufWord3);
}

// Column of element i of the pack whose first column is `col`: packs are
// runs of N columns in the aligned layout, and N columns 64 apart (one per
// lane of a wave) in the element-wise layout, so each element load of a wave
// is still one contiguous run.
template <bool kAligned>
__device__ __forceinline__ int64_t col_at(int64_t col, int i) {
  return kAligned ? col + i : col + 64 * i;
}

// N elements of T in raw 32-bit words (N * bytes is 8, 16 or 32).
template <typename T, int N>
struct Pack {
  static constexpr int kBytes = Ty<T>::kBytes;
  static constexpr int kWords = N * kBytes / 4;
  uint32_t w[kWords];

  __device__ __forceinline__ float operator[](int i) const { return Ty<T>::get(w, i); }

  // The N columns of the pack at `col` (see col_at) of the row behind `r`.
  // kAligned: the row start is 16-byte aligned and C is a whole number of
  // packs, so a pack is wholly inside the row or wholly past its end.
  template <bool kAligned>
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int64_t col) {
    const int off = int(col) * kBytes;
    if constexpr (kAligned) {
      if constexpr (kWords == 2) {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
        w[0] = v[0]; w[1] = v[1];
      } else {
#pragma unroll
        for (int q = 0; q < kWords / 4; ++q) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * q, 0, 0));
          w[4 * q] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
        }
      }
    } else if constexpr (kBytes == 4) {
#pragma unroll
      for (int i = 0; i < N; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 256 * i, 0, 0);
    } else {
#pragma unroll
      for (int q = 0; q < kWords; ++q) {
        const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(r, off + 256 * q, 0, 0);
        const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(r, off + 256 * q + 128, 0, 0);
        w[q] = lo | (hi << 16);
      }
    }
  }
};

// Round N floats to TO and write them to the pack's columns (see col_at) of
// the row behind `r`; columns past the row's end are dropped by the buffer.
// Whole 16-byte packs go out non-temporal (cache policy NT = 2): the lines
// are written once and read by a later kernel, and skipping the L2
// write-back pass measured 23% faster for adaLN at 8K tokens.
template <typename TO, int N, bool kAligned>
__device__ __forceinline__ void store_pack(__amdgpu_buffer_rsrc_t r, int64_t col, const float* f) {
  constexpr int kBytes = Ty<TO>::kBytes;
  const int off = int(col) * kBytes;
  if constexpr (kBytes == 4) {
    if constexpr (kAligned) {
#pragma unroll
      for (int q = 0; q < N / 4; ++q) {
        const u32x4 v = {__float_as_uint(f[4 * q]), __float_as_uint(f[4 * q + 1]),
                         __float_as_uint(f[4 * q + 2]), __float_as_uint(f[4 * q + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(v, r, off + 16 * q, 0, 2);
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(f[i]), r, off + 256 * i, 0, 0);
    }
  } else {
    if constexpr (kAligned) {
      static_assert(N == 8, "16-bit output packs are 16 bytes");
      const u32x4 v = {pack2<TO>(f[0], f[1]), pack2<TO>(f[2], f[3]), pack2<TO>(f[4], f[5]),
                       pack2<TO>(f[6], f[7])};
      __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 2);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i)
        __builtin_amdgcn_raw_buffer_store_b16(Store<TO>::bits(f[i]), r, off + 128 * i, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Reductions. Inside a wave: quad swaps (xor 1, xor 2), half-row mirror and
// row mirror leave every lane of a 16-lane row with the row total; the four
// row totals are then read in a fixed order. IEEE addition is commutative, so
// both partners of each exchange hold bit-identical sums and the result is
// the same in every lane.
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over the workgroup's waves; `slot` is a per-call LDS array (a second
// reduction uses a second array, so no barrier is needed between them).
__device__ __forceinline__ float block_sum(float v, int nw, int wave, int lane, float* slot) {
  float s = wave_sum(v);
  if (nw == 1) return s;
  if (lane == 0) slot[wave] = s;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < nw; ++w) t += slot[w];
  return t;
}

// ---------------------------------------------------------------------------
// adaLN modulation.
// ---------------------------------------------------------------------------
struct AdalnArgs {
  const void* x; int64_t x_sb, x_sl;
  const void* scale; int64_t sc_sb, sc_sl;
  const void* shift; int64_t sh_sb, sh_sl;
  void* out; int64_t o_sb, o_sl;
  int64_t L, C;
  float eps;
};

template <typename TX, typename TM, bool kAligned>
__global__ void __launch_bounds__(64 * kMaxWaves) adaln_kernel(AdalnArgs a) {
  using TO = typename Promote<TX, TM>::type;
  constexpr int N = 16 / Ty<TX>::kBytes;  // columns per pack
  __shared__ float red0[kMaxWaves], red1[kMaxWaves];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int64_t l = blockIdx.x, b = blockIdx.y;
  const int64_t C = a.C;
  const auto xr = row_rsrc(static_cast<const TX*>(a.x) + b * a.x_sb + l * a.x_sl, C * sizeof(TX));
  const auto scr = row_rsrc(static_cast<const TM*>(a.scale) + b * a.sc_sb + l * a.sc_sl,
                            C * sizeof(TM));
  const auto shr = row_rsrc(static_cast<const TM*>(a.shift) + b * a.sh_sb + l * a.sh_sl,
                            C * sizeof(TM));
  const auto outr = row_rsrc(static_cast<TO*>(a.out) + b * a.o_sb + l * a.o_sl, C * sizeof(TO));

  auto col_of = [&](int v) -> int64_t {
    const int64_t p = int64_t(v * nw + wave) * 64;
    return kAligned ? (p + lane) * N : p * N + lane;
  };

  Pack<TX, N> xs[kPacks];
  Pack<TM, N> sc[kPacks], sh[kPacks];
#pragma unroll
  for (int v = 0; v < kPacks; ++v) xs[v].template load<kAligned>(xr, col_of(v));
#pragma unroll
  for (int v = 0; v < kPacks; ++v) sc[v].template load<kAligned>(scr, col_of(v));
#pragma unroll
  for (int v = 0; v < kPacks; ++v) sh[v].template load<kAligned>(shr, col_of(v));

  // Columns past the row's end were loaded as zeros: they add nothing here.
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < kPacks; ++v)
#pragma unroll
    for (int i = 0; i < N; ++i) s += xs[v][i];
  const float mean = block_sum(s, nw, wave, lane, red0) / float(C);

  float q = 0.f;
#pragma unroll
  for (int v = 0; v < kPacks; ++v) {
    const int64_t c0 = col_of(v);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float d = xs[v][i] - mean;
      const bool in_row = kAligned ? c0 < C : col_at<kAligned>(c0, i) < C;
      q += in_row ? d * d : 0.f;
    }
  }
  const float var = block_sum(q, nw, wave, lane, red1) / float(C);
  const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);

#pragma unroll
  for (int v = 0; v < kPacks; ++v) {
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float normed = (xs[v][i] - mean) * rstd;
      o[i] = normed * (1.0f + sc[v][i]) + sh[v][i];
    }
    store_pack<TO, N, kAligned>(outr, col_of(v), o);
  }
}

// ---------------------------------------------------------------------------
// Gated residual.
// ---------------------------------------------------------------------------
struct GatedArgs {
  const void* x; int64_t x_sb, x_sl;
  const void* y; int64_t y_sb, y_sl;
  const void* gate; int64_t g_sb, g_sl;
  void* out; int64_t o_sb, o_sl;
  int64_t L, C;
};

// fp32 product, then fp32 sum, each rounded (no fused multiply-add), then one
// rounding to the output type.
__device__ __forceinline__ float mul_add_rounded(float x, float y, float g) {
#pragma clang fp contract(off)
  const float p = y * g;
  return x + p;
}

template <typename TX, typename TG, bool kAligned>
__global__ void __launch_bounds__(64 * kMaxWaves) gated_residual_kernel(GatedArgs a) {
  using TO = typename Promote<TX, TG>::type;
  constexpr int N = 16 / Ty<TX>::kBytes;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int64_t l = blockIdx.x, b = blockIdx.y;
  const int64_t C = a.C;
  const auto xr = row_rsrc(static_cast<const TX*>(a.x) + b * a.x_sb + l * a.x_sl, C * sizeof(TX));
  const auto yr = row_rsrc(static_cast<const TX*>(a.y) + b * a.y_sb + l * a.y_sl, C * sizeof(TX));
  const auto gr = row_rsrc(static_cast<const TG*>(a.gate) + b * a.g_sb + l * a.g_sl,
                           C * sizeof(TG));
  const auto outr = row_rsrc(static_cast<TO*>(a.out) + b * a.o_sb + l * a.o_sl, C * sizeof(TO));

  auto col_of = [&](int v) -> int64_t {
    const int64_t p = int64_t(v * nw + wave) * 64;
    return kAligned ? (p + lane) * N : p * N + lane;
  };

  Pack<TX, N> xs[kPacks], ys[kPacks];
  Pack<TG, N> gs[kPacks];
#pragma unroll
  for (int v = 0; v < kPacks; ++v) xs[v].template load<kAligned>(xr, col_of(v));
#pragma unroll
  for (int v = 0; v < kPacks; ++v) ys[v].template load<kAligned>(yr, col_of(v));
#pragma unroll
  for (int v = 0; v < kPacks; ++v) gs[v].template load<kAligned>(gr, col_of(v));
#pragma unroll
  for (int v = 0; v < kPacks; ++v) {
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = mul_add_rounded(xs[v][i], ys[v][i], gs[v][i]);
    store_pack<TO, N, kAligned>(outr, col_of(v), o);
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int elem_bytes(int dtype) { return dtype == DX_F32 ? 4 : 2; }

bool is_float_dtype(int d) { return d == DX_BF16 || d == DX_F16 || d == DX_F32; }

int promoted(int a, int b) { return a == b ? a : DX_F32; }

// Waves per row: the fewest for which kPacks packs per lane cover the row.
int choose_waves(int64_t C, int x_bytes) {
  const int64_t per_wave = int64_t(kPacks) * 64 * (16 / x_bytes);
  return int((C + per_wave - 1) / per_wave);
}

int waves_override() {
  const int n = tuning(DX_TUNE_NORM_WAVES);
  return n >= 1 && n <= kMaxWaves ? n : 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Pack-wise access is valid when every row start of every operand is 16-byte
// aligned (pointer and strides) and C is a whole number of x packs. An
// operand whose element is wider than x's (f32 modulation of a bf16 row)
// has packs of 32 bytes, read as two 16-byte loads; a narrower one (bf16
// modulation of an f32 row) has 8-byte packs at 8-byte aligned columns.
bool rows_aligned(const void* p, int64_t sb, int64_t sl, int bytes, int64_t C, int x_pack) {
  return aligned16(p) && (sb * bytes) % 16 == 0 && (sl * bytes) % 16 == 0 && C % x_pack == 0;
}

template <typename TX, typename TM, bool A>
hipError_t launch_adaln(const AdalnArgs& a, int64_t rows, int nw, hipStream_t s) {
  hipLaunchKernelGGL((adaln_kernel<TX, TM, A>), dim3(unsigned(a.L), unsigned(rows / a.L)),
                     dim3(64 * nw), 0, s, a);
  return hipGetLastError();
}

template <typename TX, typename TM>
hipError_t dispatch_adaln_al(bool al, const AdalnArgs& a, int64_t rows, int nw, hipStream_t s) {
  return al ? launch_adaln<TX, TM, true>(a, rows, nw, s) : launch_adaln<TX, TM, false>(a, rows, nw, s);
}

template <typename TX>
hipError_t dispatch_adaln_m(int md, bool al, const AdalnArgs& a, int64_t rows, int nw,
                            hipStream_t s) {
  switch (md) {
    case DX_BF16: return dispatch_adaln_al<TX, bf16_t>(al, a, rows, nw, s);
    case DX_F16: return dispatch_adaln_al<TX, f16_t>(al, a, rows, nw, s);
    default: return dispatch_adaln_al<TX, float>(al, a, rows, nw, s);
  }
}

template <typename TX, typename TG, bool A>
hipError_t launch_gated(const GatedArgs& a, int64_t rows, int nw, hipStream_t s) {
  hipLaunchKernelGGL((gated_residual_kernel<TX, TG, A>), dim3(unsigned(a.L), unsigned(rows / a.L)),
                     dim3(64 * nw), 0, s, a);
  return hipGetLastError();
}

template <typename TX, typename TG>
hipError_t dispatch_gated_al(bool al, const GatedArgs& a, int64_t rows, int nw, hipStream_t s) {
  return al ? launch_gated<TX, TG, true>(a, rows, nw, s) : launch_gated<TX, TG, false>(a, rows, nw, s);
}

template <typename TX>
hipError_t dispatch_gated_g(int gd, bool al, const GatedArgs& a, int64_t rows, int nw,
                            hipStream_t s) {
  switch (gd) {
    case DX_BF16: return dispatch_gated_al<TX, bf16_t>(al, a, rows, nw, s);
    case DX_F16: return dispatch_gated_al<TX, f16_t>(al, a, rows, nw, s);
    default: return dispatch_gated_al<TX, float>(al, a, rows, nw, s);
  }
}

// Common shape checks; returns DX_OK or DX_EINVAL with the message set.
int check_rows(const char* what, int64_t B, int64_t L, int64_t C, int x_dtype, int m_dtype,
               int out_dtype) {
  DX_CHECK_ARG(B >= 0 && L >= 0 && C >= 0, "%s: negative shape (B=%lld, L=%lld, C=%lld)", what,
               (long long)B, (long long)L, (long long)C);
  DX_CHECK_ARG(is_float_dtype(x_dtype) && is_float_dtype(m_dtype),
               "%s: dtype codes %d/%d (need DX_BF16, DX_F16 or DX_F32)", what, x_dtype, m_dtype);
  DX_CHECK_ARG(out_dtype == promoted(x_dtype, m_dtype),
               "%s: out dtype %d must be the promotion of %d and %d", what, out_dtype, x_dtype,
               m_dtype);
  DX_CHECK_ARG(L <= 0x7fffffffLL && B <= 65535, "%s: grid limits exceeded (B=%lld > 65535 or "
               "L=%lld > 2^31-1)", what, (long long)B, (long long)L);
  const int64_t per_wave = int64_t(kPacks) * 64 * (16 / elem_bytes(x_dtype));
  DX_CHECK_ARG(C <= per_wave * kMaxWaves, "%s: C=%lld exceeds %lld", what, (long long)C,
               (long long)(per_wave * kMaxWaves));
  return DX_OK;
}

}  // namespace
}  // namespace dx

using namespace dx;

extern "C" int dx_adaln_modulate(const void* x, int64_t x_sb, int64_t x_sl, int x_dtype,
                                 const void* scale, int64_t sc_sb, int64_t sc_sl,
                                 const void* shift, int64_t sh_sb, int64_t sh_sl, int mod_dtype,
                                 void* out, int64_t o_sb, int64_t o_sl, int out_dtype,
                                 int64_t B, int64_t L, int64_t C, float eps, void* stream) {
  const int rc = check_rows("adaln_modulate", B, L, C, x_dtype, mod_dtype, out_dtype);
  if (rc != DX_OK) return rc;
  const int64_t rows = B * L;
  if (rows == 0 || C == 0) return DX_OK;
  DX_CHECK_ARG(x && scale && shift && out, "adaln_modulate: null tensor pointer");
  const int xb = elem_bytes(x_dtype), mb = elem_bytes(mod_dtype), ob = elem_bytes(out_dtype);
  const int pack = 16 / xb;
  const bool al = rows_aligned(x, x_sb, x_sl, xb, C, pack) &&
                  rows_aligned(scale, sc_sb, sc_sl, mb, C, pack) &&
                  rows_aligned(shift, sh_sb, sh_sl, mb, C, pack) &&
                  rows_aligned(out, o_sb, o_sl, ob, C, pack);
  int nw = choose_waves(C, xb);
  if (const int o = waves_override()) nw = std::max(nw, o);
  AdalnArgs a{x, x_sb, x_sl, scale, sc_sb, sc_sl, shift, sh_sb, sh_sl, out, o_sb, o_sl,
              L, C, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case DX_BF16: e = dispatch_adaln_m<bf16_t>(mod_dtype, al, a, rows, nw, s); break;
    case DX_F16: e = dispatch_adaln_m<f16_t>(mod_dtype, al, a, rows, nw, s); break;
    default: e = dispatch_adaln_m<float>(mod_dtype, al, a, rows, nw, s); break;
  }
  if (e != hipSuccess) {
    set_error("adaln_modulate: launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  return DX_OK;
}

extern "C" int dx_gated_residual(const void* x, int64_t x_sb, int64_t x_sl,
                                 const void* y, int64_t y_sb, int64_t y_sl, int x_dtype,
                                 const void* gate, int64_t g_sb, int64_t g_sl, int gate_dtype,
                                 void* out, int64_t o_sb, int64_t o_sl, int out_dtype,
                                 int64_t B, int64_t L, int64_t C, void* stream) {
  const int rc = check_rows("gated_residual", B, L, C, x_dtype, gate_dtype, out_dtype);
  if (rc != DX_OK) return rc;
  const int64_t rows = B * L;
  if (rows == 0 || C == 0) return DX_OK;
  DX_CHECK_ARG(x && y && gate && out, "gated_residual: null tensor pointer");
  const int xb = elem_bytes(x_dtype), gb = elem_bytes(gate_dtype), ob = elem_bytes(out_dtype);
  const int pack = 16 / xb;
  const bool al = rows_aligned(x, x_sb, x_sl, xb, C, pack) &&
                  rows_aligned(y, y_sb, y_sl, xb, C, pack) &&
                  rows_aligned(gate, g_sb, g_sl, gb, C, pack) &&
                  rows_aligned(out, o_sb, o_sl, ob, C, pack);
  int nw = choose_waves(C, xb);
  if (const int o = waves_override()) nw = std::max(nw, o);
  GatedArgs a{x, x_sb, x_sl, y, y_sb, y_sl, gate, g_sb, g_sl, out, o_sb, o_sl, L, C};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case DX_BF16: e = dispatch_gated_g<bf16_t>(gate_dtype, al, a, rows, nw, s); break;
    case DX_F16: e = dispatch_gated_g<f16_t>(gate_dtype, al, a, rows, nw, s); break;
    default: e = dispatch_gated_g<float>(gate_dtype, al, a, rows, nw, s); break;
  }
  if (e != hipSuccess) {
    set_error("gated_residual: launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  return DX_OK;
}
