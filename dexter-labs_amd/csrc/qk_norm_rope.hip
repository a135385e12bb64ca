// Fused QK-RMSNorm + rotary for gfx950, optionally writing the rotated k and
// the raw v straight into a KV-cache slot.
//
// Semantics follow dexter's reference op (python/dexter/ops/reference/rope.py):
//   _rms  (:29-40)  x * rsqrt(mean(x^2 over the token's whole H*D plane) + eps)
//                   * weight, in fp32, then rounded to the io dtype;
//   _rope (:10-26)  out_lo = lo*c - hi*s, out_hi = lo*s + hi*c in fp32 (each
//                   product and sum rounded separately, no fused multiply-add),
//                   then rounded to the io dtype.
// Keeping the reference's intermediate rounding makes this kernel agree with
// the oracle to within the summation order of the mean.
//
// Work layout: one workgroup per (batch, token) and plane (q, k, and v when v
// is written: cache append, projection partials); one thread per "unit" of 8
// rotary pairs: 16 consecutive elements when pairs are interleaved (2j, 2j+1),
// or 8 elements at offset o plus 8 at o + D/2 for split-half pairs. The
// workgroup is the unit count rounded up to whole waves (192 threads for a
// 3072-wide plane). The kernel is latency-bound at decode
// sizes, so every global load a thread needs -- its rows, weights, cos and
// sin -- is issued before the sum-of-squares reduction: one memory round
// trip, then LDS, then the stores. The outputs are read next by other
// workgroups (on other XCDs) or much later (the cache rows), so they go out
// as non-temporal stores: no dirty lines left to write back at the end of the
// kernel, and the next kernel in the stream starts sooner.
#include "dx_common.h"
#include "qkv_gemm.h"

namespace dx {
namespace {

constexpr int kMaxThreads = 1024;     // H*D <= 1024 units * 16 = 16384
constexpr int kMaxProjThreads = 512;  // projection epilogue: H*D <= 8192

template <typename W> struct Vec8;
template <> struct Vec8<bf16_t> {
  typedef u32x4 raw;
  static __device__ __forceinline__ raw load(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
  }
  static __device__ __forceinline__ void unpack(const raw& r, float (&o)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(r[i] << 16);
      o[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
};
template <> struct Vec8<f16_t> {
  typedef u32x4 raw;
  static __device__ __forceinline__ raw load(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
  }
  static __device__ __forceinline__ void unpack(const raw& r, float (&o)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = to_f32(f16_t{uint16_t(r[i] & 0xffffu)});
      o[2 * i + 1] = to_f32(f16_t{uint16_t(r[i] >> 16)});
    }
  }
};
struct F32x8 { f32x4 a, b; };
template <> struct Vec8<float> {
  typedef F32x8 raw;
  static __device__ __forceinline__ raw load(const void* p) {
    return F32x8{reinterpret_cast<const f32x4*>(p)[0], reinterpret_cast<const f32x4*>(p)[1]};
  }
  static __device__ __forceinline__ void unpack(const raw& r, float (&o)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) { o[i] = r.a[i]; o[4 + i] = r.b[i]; }
  }
};

// Round a float to the io type and back, as ``.to(x.dtype)`` then ``.float()``.
template <typename IO>
__device__ __forceinline__ float round_io(float x) {
  return to_f32(IO{Store<IO>::bits(x)});
}

template <typename IO>
__device__ __forceinline__ void unpack16(const u32x4& r, float (&o)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o[2 * j] = to_f32(IO{uint16_t(r[j] & 0xffffu)});
    o[2 * j + 1] = to_f32(IO{uint16_t(r[j] >> 16)});
  }
}

struct RopeArgs {
  const uint16_t* q; int64_t q_sb, q_sl, q_sh;
  const uint16_t* k; int64_t k_sb, k_sl, k_sh;
  const uint16_t* v; int64_t v_sb, v_sl, v_sh;
  const void* qw; const void* kw;
  const void* cos; int64_t cos_sl;
  const void* sin; int64_t sin_sl;
  uint16_t* q_out; uint16_t* k_out;
  uint16_t* ck; uint16_t* cv; int64_t c_sb, c_ss, c_sh; int64_t start;
  int L, H, D;
  float eps;
  // Device start row (overrides start when set): a block that would not fit
  // in capacity rows is not written to the cache and *status (if given)
  // becomes 1; q_out/k_out are written either way.
  const int32_t* start_dev;
  int32_t* status;
  int64_t capacity;
  // Projection input (the fused QKV projection's epilogue): instead of q/k/v,
  // the kernel reads n_part fp32 split-K partial products [n_part][tokens][3 H D]
  // (q columns, then k, then v), adds the bias rows (may be null), rounds to
  // the io type -- the projection's output -- and also writes v to v_out.
  const float* part; int64_t part_split;  // elements between consecutive partials
  const uint16_t* bias[3];                // q, k, v bias rows [H D], each may be null
  uint16_t* v_out;
  int n_part;
  // floor(u / (D / 16)) = (u * uph_magic) >> 21 for every thread index u < 1024
  // (uph_magic = 2^21 / (D / 16) + 1; checked exhaustively for D / 16 <= 1024).
  uint32_t uph_magic;
};

// Touch every 64-byte line of the arguments up front: independent scalar
// loads and one wait, instead of the chain of dependent loads (each a cache
// miss at kernel start) that the first uses would otherwise issue.
__device__ __forceinline__ void prefetch_args(const RopeArgs& a) {
  static_assert(sizeof(RopeArgs) <= 320, "arguments span at most five lines");
  const uint64_t l0 = reinterpret_cast<uint64_t>(a.q);
  const uint64_t l1 = uint64_t(a.v_sb);
  const uint64_t l2 = reinterpret_cast<uint64_t>(a.q_out);
  const uint32_t l3 = uint32_t(a.L);
  const uint32_t l4 = uint32_t(a.n_part);
  asm volatile("" ::"s"(l0), "s"(l1), "s"(l2), "s"(l3), "s"(l4));
}

// The projection's output for this thread's two 8-element pieces of one plane
// (the lo and hi offsets of ``row``): the sum of the split-K partials in split
// order, plus the bias (may be null), rounded to IO once. Partials are read
// four at a time, all their loads issued together, so they share round trips.
template <typename IO>
__device__ __forceinline__ void projected(const RopeArgs& a, const float* row, int lo, int hi,
                                          const uint16_t* bias, u32x4 (&x)[2]) {
  const int off[2] = {lo, hi};
  f32x4 s[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    s[i][0] = *reinterpret_cast<const f32x4*>(row + off[i]);
    s[i][1] = *reinterpret_cast<const f32x4*>(row + off[i] + 4);
  }
  for (int p = 1; p < a.n_part; p += 4) {
    f32x4 t[4][2][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float* r = row + min(p + j, a.n_part - 1) * a.part_split;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        t[j][i][0] = *reinterpret_cast<const f32x4*>(r + off[i]);
        t[j][i][1] = *reinterpret_cast<const f32x4*>(r + off[i] + 4);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (p + j < a.n_part) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          s[i][0] += t[j][i][0];
          s[i][1] += t[j][i][1];
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float f[8] = {s[i][0][0], s[i][0][1], s[i][0][2], s[i][0][3],
                  s[i][1][0], s[i][1][1], s[i][1][2], s[i][1][3]};
    if (bias) {
      float bf[8];
      unpack16<IO>(*reinterpret_cast<const u32x4*>(bias + off[i]), bf);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += bf[e];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) x[i][j] = pack2<IO>(f[2 * j], f[2 * j + 1]);
  }
}

// Cache slot of this call: the host start, or the device start row when one is
// given (then a block that would not fit is skipped and flagged in *status).
__device__ __forceinline__ bool cache_start(const RopeArgs& a, bool flag, int64_t& start) {
  start = a.start;
  if (!a.start_dev) return true;
  start = *a.start_dev;
  const bool fits = start >= 0 && start + a.L <= a.capacity;
  if (!fits && flag && a.status) a.status[0] = 1;
  return fits;
}

// One workgroup per token and plane: y = 0 is q, y = 1 is k, and y = 2 (only
// with a cache write or a projection input) is v. More workgroups in flight
// suit a latency-bound call: measured at the Wan-5B chunk, one workgroup per
// plane beats one per token for q and k (3.26 against 3.70 us) and for q, k
// and v (3.81 against 4.38 us with the cache write). The q and k planes are
// normalised over their own H*D elements and rotated; v is copied (or, from
// partials, summed and rounded) to its outputs.
template <typename IO, typename W, typename TB, bool INTERLEAVED, bool APPEND, bool PROJ,
          int kThreads>
__device__ __forceinline__ void prologue_body(const RopeArgs& a) {
  // Every product and sum rounded on its own, as the reference's tensor ops
  // round them (rope.py:20-26, :36-40): otherwise the compiler may fuse a
  // rotation product into its sum (one rounding), which near cancellation
  // changes the result, and differently in each kernel that inlines this.
#pragma clang fp contract(off)
  prefetch_args(a);
  __shared__ float red[kThreads / 64];
  // Grid (L, planes, B): no division to find the token.
  const int l = blockIdx.x, plane = blockIdx.y, b = blockIdx.z;  // plane: uniform
  const int token = b * a.L + l;
  const int units_per_head = a.D / 16;
  const int n_units = a.H * units_per_head;
  const int u = threadIdx.x;
  const bool active = u < n_units;
  // Threads past the last unit (the workgroup is whole waves) load the last
  // unit's data, add nothing to the sum and store nothing: no branch around
  // the loads.
  const int uc = min(u, n_units - 1);
  const int h = int((uint32_t(uc) * a.uph_magic) >> 21);
  const int uh = uc - h * units_per_head;
  // Element offsets (within one head) of the lo and hi halves of this unit.
  const int lo = INTERLEAVED ? uh * 16 : uh * 8;
  const int hi = INTERLEAVED ? lo + 8 : lo + a.D / 2;
  const int j0 = INTERLEAVED ? uh * 8 : lo;  // first rotary pair index
  const int64_t hd = int64_t(a.H) * a.D;
  const int64_t obase = (int64_t(token) * a.H + h) * a.D;

  // ---- every load up front ------------------------------------------------
  u32x4 xa[2];
  typename Vec8<W>::raw wr[2];
  typename Vec8<TB>::raw cr, sr;
  if (PROJ) {
    const float* row = a.part + int64_t(token) * 3 * hd + plane * hd + h * a.D;
    const uint16_t* bias = a.bias[plane] ? a.bias[plane] + h * a.D : nullptr;
    projected<IO>(a, row, lo, hi, bias, xa);
  } else {
    const uint16_t* xp = plane == 0   ? a.q + b * a.q_sb + l * a.q_sl + h * a.q_sh
                         : plane == 1 ? a.k + b * a.k_sb + l * a.k_sl + h * a.k_sh
                                      : a.v + b * a.v_sb + l * a.v_sl + h * a.v_sh;
    xa[0] = *reinterpret_cast<const u32x4*>(xp + lo);
    xa[1] = *reinterpret_cast<const u32x4*>(xp + hi);
  }
  if (plane < 2) {
    const W* wp = static_cast<const W*>(plane == 0 ? a.qw : a.kw) + h * a.D;
    wr[0] = Vec8<W>::load(wp + lo);
    wr[1] = Vec8<W>::load(wp + hi);
    cr = Vec8<TB>::load(static_cast<const TB*>(a.cos) + l * a.cos_sl + j0);
    sr = Vec8<TB>::load(static_cast<const TB*>(a.sin) + l * a.sin_sl + j0);
  }

  if (plane == 2) {
    // ---- v: the projection's output and / or the cache row ----------------
    if (!active) return;
    if (PROJ) {
      __builtin_nontemporal_store(xa[0], reinterpret_cast<u32x4*>(a.v_out + obase + lo));
      __builtin_nontemporal_store(xa[1], reinterpret_cast<u32x4*>(a.v_out + obase + hi));
    }
    if (APPEND) {
      int64_t start;
      if (cache_start(a, false, start)) {
        const int64_t cbase = b * a.c_sb + (start + l) * a.c_ss + h * a.c_sh;
        __builtin_nontemporal_store(xa[0], reinterpret_cast<u32x4*>(a.cv + cbase + lo));
        __builtin_nontemporal_store(xa[1], reinterpret_cast<u32x4*>(a.cv + cbase + hi));
      }
    }
    return;
  }

  // ---- sum of squares over the plane ------------------------------------
  float x[2][8];
#pragma unroll
  for (int p = 0; p < 2; ++p) unpack16<IO>(xa[p], x[p]);
  float sq = 0.f;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(x[p][e], x[p][e], sq);
  sq = lane_sum64(active ? sq : 0.f);
  const int wave = threadIdx.x >> 6, n_waves = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = sq;
  __syncthreads();
  if (!active) return;
  float t = 0.f;
  for (int w = 0; w < n_waves; ++w) t += red[w];
  const float rr = 1.0f / __builtin_sqrtf(t / float(hd) + a.eps);

  // ---- norm (rounded to io, as _rms does), then rotation ------------------
  float fw[2][8], c[8], s[8];
#pragma unroll
  for (int p = 0; p < 2; ++p) Vec8<W>::unpack(wr[p], fw[p]);
  Vec8<TB>::unpack(cr, c);
  Vec8<TB>::unpack(sr, s);
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[p][e] = round_io<IO>(held((x[p][e] * rr) * fw[p][e]));
  float o[2][8];
#pragma unroll
  for (int t8 = 0; t8 < 8; ++t8) {
    // Interleaved: pair t8 is elements (2 t8, 2 t8 + 1) of the 16-element span,
    // i.e. half t8 / 4, elements 2 (t8 % 4) and 2 (t8 % 4) + 1. Split-half:
    // element t8 of half 0 against element t8 of half 1.
    const int p_lo = INTERLEAVED ? t8 / 4 : 0, e_lo = INTERLEAVED ? 2 * (t8 % 4) : t8;
    const int p_hi = INTERLEAVED ? t8 / 4 : 1, e_hi = INTERLEAVED ? 2 * (t8 % 4) + 1 : t8;
    const float xl = x[p_lo][e_lo], xh = x[p_hi][e_hi];
    o[p_lo][e_lo] = held(xl * c[t8] - xh * s[t8]);
    o[p_hi][e_hi] = held(xl * s[t8] + xh * c[t8]);
  }
  u32x4 po[2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int j = 0; j < 4; ++j) po[p][j] = pack2<IO>(o[p][2 * j], o[p][2 * j + 1]);
  uint16_t* out = plane == 0 ? a.q_out : a.k_out;
  __builtin_nontemporal_store(po[0], reinterpret_cast<u32x4*>(out + obase + lo));
  __builtin_nontemporal_store(po[1], reinterpret_cast<u32x4*>(out + obase + hi));
  if (APPEND && plane == 1) {
    int64_t start;
    if (cache_start(a, token == 0 && u == 0, start)) {
      const int64_t cbase = b * a.c_sb + (start + l) * a.c_ss + h * a.c_sh;
      __builtin_nontemporal_store(po[0], reinterpret_cast<u32x4*>(a.ck + cbase + lo));
      __builtin_nontemporal_store(po[1], reinterpret_cast<u32x4*>(a.ck + cbase + hi));
    }
  }
}

template <typename IO, typename W, typename TB, bool INTERLEAVED, bool APPEND>
__global__ __launch_bounds__(kMaxThreads) void qk_norm_rope_kernel(RopeArgs a) {
  prologue_body<IO, W, TB, INTERLEAVED, APPEND, false, kMaxThreads>(a);
}

// The projection's epilogue: more registers per thread (the partials), so a
// smaller workgroup bound.
template <typename IO, typename W, typename TB, bool INTERLEAVED, bool APPEND>
__global__ __launch_bounds__(kMaxProjThreads) void qkv_epilogue_kernel(RopeArgs a) {
  prologue_body<IO, W, TB, INTERLEAVED, APPEND, true, kMaxProjThreads>(a);
}

template <typename IO, typename W, typename TB, bool APPEND>
hipError_t launch3(const RopeArgs& a, int tokens, int threads, bool interleaved,
                   hipStream_t st) {
  // Workgroups per token: q and k, and v when it is written.
  const dim3 grid(unsigned(a.L), (APPEND || a.part) ? 3u : 2u, unsigned(tokens / a.L));
  if (a.part) {
    if (interleaved)
      hipLaunchKernelGGL((qkv_epilogue_kernel<IO, W, TB, true, APPEND>), grid, dim3(threads),
                         0, st, a);
    else
      hipLaunchKernelGGL((qkv_epilogue_kernel<IO, W, TB, false, APPEND>), grid, dim3(threads),
                         0, st, a);
    return hipGetLastError();
  }
  if (interleaved)
    hipLaunchKernelGGL((qk_norm_rope_kernel<IO, W, TB, true, APPEND>), grid, dim3(threads), 0,
                       st, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_kernel<IO, W, TB, false, APPEND>), grid, dim3(threads), 0,
                       st, a);
  return hipGetLastError();
}

template <typename IO, typename W, bool APPEND>
hipError_t launch2(const RopeArgs& a, int tokens, int threads, int tdt, bool il,
                   hipStream_t st) {
  switch (tdt) {
    case DX_BF16: return launch3<IO, W, bf16_t, APPEND>(a, tokens, threads, il, st);
    case DX_F16: return launch3<IO, W, f16_t, APPEND>(a, tokens, threads, il, st);
    default: return launch3<IO, W, float, APPEND>(a, tokens, threads, il, st);
  }
}

template <typename IO, bool APPEND>
hipError_t launch1(const RopeArgs& a, int tokens, int threads, int wdt, int tdt, bool il,
                   hipStream_t st) {
  switch (wdt) {
    case DX_BF16: return launch2<IO, bf16_t, APPEND>(a, tokens, threads, tdt, il, st);
    case DX_F16: return launch2<IO, f16_t, APPEND>(a, tokens, threads, tdt, il, st);
    default: return launch2<IO, float, APPEND>(a, tokens, threads, tdt, il, st);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                 const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh, int io_dtype,
                 const void* qw, const void* kw, int wdt, const void* cos, int64_t cos_sl,
                 const void* sin, int64_t sin_sl, int tdt, void* q_out, void* k_out,
                 int64_t B, int64_t L, int64_t H, int64_t D) {
  DX_CHECK_ARG(io_dtype == DX_BF16 || io_dtype == DX_F16,
               "qk_norm_rope: io dtype must be bf16 or f16 (got code %d)", io_dtype);
  DX_CHECK_ARG(wdt == DX_BF16 || wdt == DX_F16 || wdt == DX_F32,
               "qk_norm_rope: weight dtype code %d unsupported", wdt);
  DX_CHECK_ARG(tdt == DX_BF16 || tdt == DX_F16 || tdt == DX_F32,
               "qk_norm_rope: cos/sin dtype code %d unsupported", tdt);
  DX_CHECK_ARG(B >= 0 && L >= 0 && H > 0 && D > 0, "qk_norm_rope: bad shape");
  DX_CHECK_ARG(D % 16 == 0, "qk_norm_rope: head_dim %lld must be a multiple of 16",
               (long long)D);
  DX_CHECK_ARG(H * D <= int64_t(kMaxThreads) * 16, "qk_norm_rope: H*D = %lld exceeds %d",
               (long long)(H * D), kMaxThreads * 16);
  DX_CHECK_ARG(B * L < (int64_t(1) << 31) && B <= 65535,
               "qk_norm_rope: too many tokens (B * L < 2^31, B <= 65535)");
  DX_CHECK_ARG(q && k && qw && kw && cos && sin && q_out && k_out,
               "qk_norm_rope: null pointer");
  DX_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(qw) && aligned16(kw) &&
                   aligned16(cos) && aligned16(sin) && aligned16(q_out) && aligned16(k_out),
               "qk_norm_rope: pointers must be 16-byte aligned");
  DX_CHECK_ARG(q_sb % 8 == 0 && q_sl % 8 == 0 && q_sh % 8 == 0 && k_sb % 8 == 0 &&
                   k_sl % 8 == 0 && k_sh % 8 == 0,
               "qk_norm_rope: q/k strides must be multiples of 8 elements");
  const int64_t per16 = (tdt == DX_F32) ? 4 : 8;  // table elements per 16 bytes
  DX_CHECK_ARG(cos_sl % per16 == 0 && sin_sl % per16 == 0,
               "qk_norm_rope: cos/sin row strides must keep rows 16-byte aligned");
  return DX_OK;
}

}  // namespace
}  // namespace dx

using namespace dx;

namespace dx {
// The prologue's argument checks, shared with the decode attention launch
// that runs the prologue itself (dx_qk_norm_rope_attention).
int rope_validate(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                  const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                  const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh, int io_dtype,
                  const void* qw, const void* kw, int wdt, const void* cos, int64_t cos_sl,
                  const void* sin, int64_t sin_sl, int tdt, void* q_out, void* k_out,
                  void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                  int64_t capacity, int64_t start, const int32_t* start_dev,
                  int64_t B, int64_t L, int64_t H, int64_t D, bool append) {
  int rc = check_common(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, io_dtype, qw, kw, wdt, cos,
                        cos_sl, sin, sin_sl, tdt, q_out, k_out, B, L, H, D);
  if (rc) return rc;
  if (append) {
    DX_CHECK_ARG(cache && v, "qk_norm_rope_append: null cache or v");
    DX_CHECK_ARG(start >= 0, "qk_norm_rope_append: negative start");
    DX_CHECK_ARG(!start_dev || (reinterpret_cast<uintptr_t>(start_dev) & 3u) == 0,
                 "qk_norm_rope_append: device start must be a 4-byte aligned int32");
    if (!start_dev && start + L > capacity) {
      set_error("KV cache full: %lld + %lld > %lld", (long long)start, (long long)L,
                (long long)capacity);
      return DX_EFULL;
    }
    DX_CHECK_ARG(aligned16(cache) && aligned16(v) && c_plane % 8 == 0 && c_sb % 8 == 0 &&
                     c_ss % 8 == 0 && c_sh % 8 == 0 && v_sb % 8 == 0 && v_sl % 8 == 0 &&
                     v_sh % 8 == 0,
                 "qk_norm_rope_append: cache/v must be 16-byte aligned with strides "
                 "that are multiples of 8 elements");
  }
  return DX_OK;
}
}  // namespace dx

static int rope_entry(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                      const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                      const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh, int io_dtype,
                      const void* qw, const void* kw, int wdt, const void* cos, int64_t cos_sl,
                      const void* sin, int64_t sin_sl, int tdt, void* q_out, void* k_out,
                      void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                      int64_t capacity, int64_t start, const int32_t* start_dev,
                      int32_t* status, int64_t B, int64_t L, int64_t H,
                      int64_t D, float eps, int interleaved, void* stream, bool append) {
  const int rc = dx::rope_validate(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh,
                                   io_dtype, qw, kw, wdt, cos, cos_sl, sin, sin_sl, tdt, q_out,
                                   k_out, cache, c_plane, c_sb, c_ss, c_sh, capacity, start,
                                   start_dev, B, L, H, D, append);
  if (rc) return rc;
  if (B * L == 0) return DX_OK;
  RopeArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_sb; a.q_sl = q_sl; a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(k); a.k_sb = k_sb; a.k_sl = k_sl; a.k_sh = k_sh;
  a.v = static_cast<const uint16_t*>(v); a.v_sb = v_sb; a.v_sl = v_sl; a.v_sh = v_sh;
  a.qw = qw; a.kw = kw; a.cos = cos; a.cos_sl = cos_sl; a.sin = sin; a.sin_sl = sin_sl;
  a.q_out = static_cast<uint16_t*>(q_out); a.k_out = static_cast<uint16_t*>(k_out);
  if (append) {
    a.ck = static_cast<uint16_t*>(cache);
    a.cv = static_cast<uint16_t*>(cache) + c_plane;
    a.c_sb = c_sb; a.c_ss = c_ss; a.c_sh = c_sh; a.start = start;
    a.start_dev = start_dev; a.status = status; a.capacity = capacity;
  }
  a.L = int(L); a.H = int(H); a.D = int(D); a.eps = eps;
  a.uph_magic = uint32_t((1u << 21) / uint32_t(D / 16) + 1u);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int tokens = int(B * L);
  const int units = int(H * D / 16);
  const int threads = (units + 63) / 64 * 64;
  hipError_t e;
  if (io_dtype == DX_BF16)
    e = append ? launch1<bf16_t, true>(a, tokens, threads, wdt, tdt, interleaved != 0, st)
               : launch1<bf16_t, false>(a, tokens, threads, wdt, tdt, interleaved != 0, st);
  else
    e = append ? launch1<f16_t, true>(a, tokens, threads, wdt, tdt, interleaved != 0, st)
               : launch1<f16_t, false>(a, tokens, threads, wdt, tdt, interleaved != 0, st);
  if (e != hipSuccess) {
    set_error("qk_norm_rope: launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  return DX_OK;
}

extern "C" int dx_qk_norm_rope(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                               const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                               int io_dtype, const void* q_weight, const void* k_weight,
                               int weight_dtype, const void* cos, int64_t cos_sl,
                               const void* sin, int64_t sin_sl, int table_dtype, void* q_out,
                               void* k_out, int64_t B, int64_t L, int64_t H, int64_t D,
                               float eps, int interleaved, void* stream) {
  return rope_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, nullptr, 0, 0, 0, io_dtype,
                    q_weight, k_weight, weight_dtype, cos, cos_sl, sin, sin_sl, table_dtype,
                    q_out, k_out, nullptr, 0, 0, 0, 0, 0, 0, nullptr, nullptr, B, L, H, D, eps,
                    interleaved, stream, false);
}

extern "C" int dx_qk_norm_rope_append(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    int io_dtype, const void* q_weight, const void* k_weight, int weight_dtype,
    const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl, int table_dtype,
    void* q_out, void* k_out, void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
    int64_t c_sh, int64_t capacity, int64_t start, int64_t B, int64_t L, int64_t H, int64_t D,
    float eps, int interleaved, void* stream) {
  return rope_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, io_dtype,
                    q_weight, k_weight, weight_dtype, cos, cos_sl, sin, sin_sl, table_dtype,
                    q_out, k_out, cache, c_plane, c_sb, c_ss, c_sh, capacity, start, nullptr,
                    nullptr, B, L, H, D, eps, interleaved, stream, true);
}

extern "C" int dx_qk_norm_rope_append_dev(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    int io_dtype, const void* q_weight, const void* k_weight, int weight_dtype,
    const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl, int table_dtype,
    void* q_out, void* k_out, void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
    int64_t c_sh, int64_t capacity, const void* start_dev, void* status, int64_t B, int64_t L,
    int64_t H, int64_t D, float eps, int interleaved, void* stream) {
  DX_CHECK_ARG(start_dev != nullptr, "qk_norm_rope_append: device start pointer is null");
  return rope_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, io_dtype,
                    q_weight, k_weight, weight_dtype, cos, cos_sl, sin, sin_sl, table_dtype,
                    q_out, k_out, cache, c_plane, c_sb, c_ss, c_sh, capacity, 0,
                    static_cast<const int32_t*>(start_dev), static_cast<int32_t*>(status), B, L,
                    H, D, eps, interleaved, stream, true);
}

// ---------------------------------------------------------------------------
// Fused QKV projection: split-K GEMM (qkv_gemm.hip), then the prologue kernel
// reading its partials (sum, bias, one rounding: the projection's output),
// with the cache write when a cache is given.
// ---------------------------------------------------------------------------
static int qkv_entry(const void* x, int64_t x_sb, int64_t x_sl, int io_dtype, const void* wq,
                     const void* wk, const void* wv, int64_t w_row, const void* bq,
                     const void* bk, const void* bv, const void* qw, const void* kw, int wdt,
                     const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl, int tdt,
                     void* q_out, void* k_out, void* v_out, void* cache, int64_t c_plane,
                     int64_t c_sb, int64_t c_ss, int64_t c_sh, int64_t capacity, int64_t start,
                     const int32_t* start_dev, int32_t* status, int64_t B, int64_t L,
                     int64_t C, int64_t H, int64_t D, float eps, int interleaved,
                     void* workspace, int64_t ws_bytes, void* stream) {
  DX_CHECK_ARG(io_dtype == DX_BF16 || io_dtype == DX_F16,
               "qkv_norm_rope: io dtype must be bf16 or f16 (got code %d)", io_dtype);
  DX_CHECK_ARG(wdt == DX_BF16 || wdt == DX_F16 || wdt == DX_F32,
               "qkv_norm_rope: weight dtype code %d unsupported", wdt);
  DX_CHECK_ARG(tdt == DX_BF16 || tdt == DX_F16 || tdt == DX_F32,
               "qkv_norm_rope: cos/sin dtype code %d unsupported", tdt);
  DX_CHECK_ARG(B >= 0 && L >= 0 && H > 0 && D > 0 && C > 0, "qkv_norm_rope: bad shape");
  const int64_t M = B * L, HD = H * D;
  DX_CHECK_ARG(M <= 128, "qkv_norm_rope: %lld tokens exceed 128 (decode chunks only)",
               (long long)M);
  DX_CHECK_ARG(D % 16 == 0 && HD % 128 == 0 && HD <= int64_t(kMaxProjThreads) * 16,
               "qkv_norm_rope: H*D = %lld must be a multiple of 128 and at most %d, head_dim "
               "a multiple of 16", (long long)HD, kMaxProjThreads * 16);
  DX_CHECK_ARG(C % 512 == 0, "qkv_norm_rope: C = %lld must be a multiple of 512", (long long)C);
  DX_CHECK_ARG(x && wq && wk && wv && qw && kw && cos && sin && q_out && k_out && v_out,
               "qkv_norm_rope: null pointer");
  DX_CHECK_ARG(aligned16(x) && aligned16(wq) && aligned16(wk) && aligned16(wv) &&
                   aligned16(q_out) && aligned16(k_out) && aligned16(v_out) &&
                   aligned16(qw) && aligned16(kw) && aligned16(cos) && aligned16(sin) &&
                   (!bq || aligned16(bq)) && (!bk || aligned16(bk)) && (!bv || aligned16(bv)),
               "qkv_norm_rope: pointers must be 16-byte aligned");
  DX_CHECK_ARG(x_sb % 8 == 0 && x_sl % 8 == 0 && w_row % 8 == 0 && w_row >= C,
               "qkv_norm_rope: strides must be multiples of 8 elements (weight rows >= C)");
  // The GEMM reads 128 weight rows through a descriptor with 32-bit offsets.
  DX_CHECK_ARG(w_row < (int64_t(1) << 22), "qkv_norm_rope: weight row stride %lld too large",
               (long long)w_row);
  const int64_t per16 = (tdt == DX_F32) ? 4 : 8;
  DX_CHECK_ARG(cos_sl % per16 == 0 && sin_sl % per16 == 0,
               "qkv_norm_rope: cos/sin row strides must keep rows 16-byte aligned");
  const bool append = cache != nullptr;
  if (append) {
    DX_CHECK_ARG(start >= 0, "qkv_norm_rope: negative start");
    DX_CHECK_ARG(!start_dev || (reinterpret_cast<uintptr_t>(start_dev) & 3u) == 0,
                 "qkv_norm_rope: device start must be a 4-byte aligned int32");
    if (!start_dev && start + L > capacity) {
      set_error("KV cache full: %lld + %lld > %lld", (long long)start, (long long)L,
                (long long)capacity);
      return DX_EFULL;
    }
    DX_CHECK_ARG(aligned16(cache) && c_plane % 8 == 0 && c_sb % 8 == 0 && c_ss % 8 == 0 &&
                     c_sh % 8 == 0,
                 "qkv_norm_rope: cache must be 16-byte aligned with strides that are "
                 "multiples of 8 elements");
  }
  if (M == 0) return DX_OK;
  const QkvPlan plan = plan_qkv(M, C, HD);
  if (!workspace || ws_bytes < plan.workspace_bytes) {
    set_error("qkv_norm_rope: workspace of %lld bytes needed, %lld given",
              (long long)plan.workspace_bytes, (long long)ws_bytes);
    return DX_EWORKSPACE;
  }
  DX_CHECK_ARG(aligned16(workspace), "qkv_norm_rope: workspace must be 16-byte aligned");

  // The GEMM reads x through a buffer descriptor whose offsets are 32-bit.
  const int64_t x_bytes = 2 * ((B - 1) * x_sb + (L - 1) * x_sl + C);
  DX_CHECK_ARG(x_bytes < (int64_t(1) << 31), "qkv_norm_rope: x spans %lld bytes (< 2^31)",
               (long long)x_bytes);
  QkvGemmArgs g{};
  g.x = static_cast<const uint16_t*>(x); g.x_sb = x_sb; g.x_sl = x_sl;
  g.x_bytes = uint32_t(x_bytes);
  g.w[0] = static_cast<const uint16_t*>(wq);
  g.w[1] = static_cast<const uint16_t*>(wk);
  g.w[2] = static_cast<const uint16_t*>(wv);
  g.w_row[0] = g.w_row[1] = g.w_row[2] = w_row;
  g.part = static_cast<float*>(workspace);
  g.M = int(M); g.L = int(L); g.C = int(C); g.HD = int(HD); g.S = plan.splits;
  g.Kc = int(C / plan.splits);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = launch_qkv_gemm(g, plan, io_dtype, st);
  if (e != hipSuccess) {
    set_error("qkv_norm_rope: projection launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }

  RopeArgs a{};
  a.qw = qw; a.kw = kw; a.cos = cos; a.cos_sl = cos_sl; a.sin = sin; a.sin_sl = sin_sl;
  a.q_out = static_cast<uint16_t*>(q_out); a.k_out = static_cast<uint16_t*>(k_out);
  a.v_out = static_cast<uint16_t*>(v_out);
  a.part = g.part; a.part_split = M * 3 * HD; a.n_part = plan.splits;
  a.bias[0] = static_cast<const uint16_t*>(bq);
  a.bias[1] = static_cast<const uint16_t*>(bk);
  a.bias[2] = static_cast<const uint16_t*>(bv);
  if (append) {
    a.ck = static_cast<uint16_t*>(cache);
    a.cv = static_cast<uint16_t*>(cache) + c_plane;
    a.c_sb = c_sb; a.c_ss = c_ss; a.c_sh = c_sh; a.start = start;
    a.start_dev = start_dev; a.status = status; a.capacity = capacity;
  }
  a.L = int(L); a.H = int(H); a.D = int(D); a.eps = eps;
  a.uph_magic = uint32_t((1u << 21) / uint32_t(D / 16) + 1u);
  const int units = int(HD / 16);
  const int threads = (units + 63) / 64 * 64;
  if (io_dtype == DX_BF16)
    e = append ? launch1<bf16_t, true>(a, int(M), threads, wdt, tdt, interleaved != 0, st)
               : launch1<bf16_t, false>(a, int(M), threads, wdt, tdt, interleaved != 0, st);
  else
    e = append ? launch1<f16_t, true>(a, int(M), threads, wdt, tdt, interleaved != 0, st)
               : launch1<f16_t, false>(a, int(M), threads, wdt, tdt, interleaved != 0, st);
  if (e != hipSuccess) {
    set_error("qkv_norm_rope: epilogue launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  return DX_OK;
}

extern "C" int64_t dx_qkv_workspace_bytes(int64_t B, int64_t L, int64_t C, int64_t H,
                                          int64_t D) {
  if (B < 0 || L < 0 || C <= 0 || H <= 0 || D <= 0) {
    set_error("qkv_workspace_bytes: bad shape");
    return -DX_EINVAL;
  }
  if (B * L == 0) return 0;
  return plan_qkv(B * L, C, H * D).workspace_bytes;
}

extern "C" int dx_qkv_norm_rope(
    const void* x, int64_t x_sb, int64_t x_sl, int io_dtype, const void* wq, const void* wk,
    const void* wv, int64_t w_row, const void* bq, const void* bk, const void* bv,
    const void* q_weight, const void* k_weight, int weight_dtype, const void* cos,
    int64_t cos_sl, const void* sin, int64_t sin_sl, int table_dtype, void* q_out, void* k_out,
    void* v_out, void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    int64_t capacity, int64_t start, const void* start_dev, void* status, int64_t B,
    int64_t L, int64_t C, int64_t H, int64_t D, float eps, int interleaved, void* workspace,
    int64_t workspace_bytes, void* stream) {
  return qkv_entry(x, x_sb, x_sl, io_dtype, wq, wk, wv, w_row, bq, bk, bv, q_weight, k_weight,
                   weight_dtype, cos, cos_sl, sin, sin_sl, table_dtype, q_out, k_out, v_out,
                   cache, c_plane, c_sb, c_ss, c_sh, capacity, start,
                   static_cast<const int32_t*>(start_dev), static_cast<int32_t*>(status), B, L,
                   C, H, D, eps, interleaved, workspace, workspace_bytes, stream);
}
