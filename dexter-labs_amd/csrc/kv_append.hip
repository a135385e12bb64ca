// KV-cache chunk append for gfx950: copy a new block's k and v [B, n, H, D]
// into rows [start, start + n) of planes 0 and 1 of a [2, B, S, H, D] cache.
//
// Replaces KVCache.append (python/dexter/models/dreamzero/model.py:53-58),
// which is two strided torch copies. The overflow check stays on the host and
// happens before any launch, with the reference's message ("KV cache full").
// The copy is bit-exact: 16-byte loads and stores, k and v in the same pass,
// one 16-byte chunk per thread per iteration of a grid-stride loop.
//
// dx_kv_append_dev takes the start row from device memory instead (a cursor
// that a captured graph reads at every replay). The host cannot check it, so
// the kernel does: a block that would not fit is not written at all, and a
// status word (if given) is set to 1.
#include "dx_common.h"

namespace dx {
namespace {

struct AppendArgs {
  const uint8_t* k; int64_t k_sb, k_sl, k_sh;  // strides in bytes
  const uint8_t* v; int64_t v_sb, v_sl, v_sh;
  uint8_t* ck; uint8_t* cv; int64_t c_sb, c_ss, c_sh;
  int64_t start;
  int64_t chunks;            // B * n * H * chunks_per_row
  int n, H, chunks_per_row;  // chunk = 16 bytes of one head row
  const int32_t* start_dev;  // device start row (overrides start when set)
  int32_t* status;           // set to 1 when a device start does not fit (may be null)
  int64_t capacity;
};

__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  if (a.start_dev) {
    const int64_t s = *a.start_dev;
    if (s < 0 || s + a.n > a.capacity) {
      if (a.status && blockIdx.x == 0 && threadIdx.x == 0) a.status[0] = 1;
      return;
    }
    a.start = s;
  }
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < a.chunks; c += stride) {
    int64_t r = c;
    const int cc = int(r % a.chunks_per_row); r /= a.chunks_per_row;
    const int h = int(r % a.H); r /= a.H;
    const int t = int(r % a.n);
    const int64_t b = r / a.n;
    const int64_t off = int64_t(cc) * 16;
    const u32x4 kx = *reinterpret_cast<const u32x4*>(a.k + b * a.k_sb + t * a.k_sl + h * a.k_sh + off);
    const u32x4 vx = *reinterpret_cast<const u32x4*>(a.v + b * a.v_sb + t * a.v_sl + h * a.v_sh + off);
    const int64_t dst = b * a.c_sb + (a.start + t) * a.c_ss + h * a.c_sh + off;
    *reinterpret_cast<u32x4*>(a.ck + dst) = kx;
    *reinterpret_cast<u32x4*>(a.cv + dst) = vx;
  }
}

}  // namespace
}  // namespace dx

using namespace dx;

static int append_entry(const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                        const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh, void* cache,
                        int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, int dtype,
                        int64_t B, int64_t n, int64_t H, int64_t D, int64_t capacity,
                        int64_t start, const int32_t* start_dev, int32_t* status,
                        void* stream) {
  DX_CHECK_ARG(dtype == DX_BF16 || dtype == DX_F16 || dtype == DX_F32,
               "kv_append: dtype code %d unsupported", dtype);
  DX_CHECK_ARG(B >= 0 && n >= 0 && H > 0 && D > 0 && start >= 0, "kv_append: bad shape");
  if (!start_dev && start + n > capacity) {
    set_error("KV cache full: %lld + %lld > %lld", (long long)start, (long long)n,
              (long long)capacity);
    return DX_EFULL;
  }
  DX_CHECK_ARG(!start_dev || (reinterpret_cast<uintptr_t>(start_dev) & 3u) == 0,
               "kv_append: device start must be a 4-byte aligned int32");
  const int64_t es = dtype == DX_F32 ? 4 : 2;
  const int64_t per16 = 16 / es;
  DX_CHECK_ARG(D % per16 == 0, "kv_append: head_dim must fill 16-byte chunks");
  DX_CHECK_ARG(k && v && cache, "kv_append: null pointer");
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  DX_CHECK_ARG(al(k) && al(v) && al(cache), "kv_append: pointers must be 16-byte aligned");
  DX_CHECK_ARG(k_sb % per16 == 0 && k_sl % per16 == 0 && k_sh % per16 == 0 &&
                   v_sb % per16 == 0 && v_sl % per16 == 0 && v_sh % per16 == 0 &&
                   c_plane % per16 == 0 && c_sb % per16 == 0 && c_ss % per16 == 0 &&
                   c_sh % per16 == 0,
               "kv_append: strides must keep head rows 16-byte aligned");
  if (B * n == 0) return DX_OK;
  AppendArgs a{};
  a.k = static_cast<const uint8_t*>(k); a.k_sb = k_sb * es; a.k_sl = k_sl * es; a.k_sh = k_sh * es;
  a.v = static_cast<const uint8_t*>(v); a.v_sb = v_sb * es; a.v_sl = v_sl * es; a.v_sh = v_sh * es;
  a.ck = static_cast<uint8_t*>(cache);
  a.cv = static_cast<uint8_t*>(cache) + c_plane * es;
  a.c_sb = c_sb * es; a.c_ss = c_ss * es; a.c_sh = c_sh * es;
  a.start = start;
  a.start_dev = start_dev;
  a.status = status;
  a.capacity = capacity;
  a.chunks_per_row = int(D / per16);
  a.n = int(n); a.H = int(H);
  a.chunks = B * n * H * a.chunks_per_row;
  const int64_t want = (a.chunks + 255) / 256;
  const int blocks = int(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(kv_append_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  DX_CHECK_LAUNCH("kv_append");
  return DX_OK;
}

extern "C" int dx_kv_append(const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                            const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                            void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
                            int64_t c_sh, int dtype, int64_t B, int64_t n, int64_t H,
                            int64_t D, int64_t capacity, int64_t start, void* stream) {
  return append_entry(k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache, c_plane, c_sb, c_ss,
                      c_sh, dtype, B, n, H, D, capacity, start, nullptr, nullptr, stream);
}

extern "C" int dx_kv_append_dev(const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                                const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                                void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
                                int64_t c_sh, int dtype, int64_t B, int64_t n, int64_t H,
                                int64_t D, int64_t capacity, const void* start_dev,
                                void* status, void* stream) {
  DX_CHECK_ARG(start_dev != nullptr, "kv_append: device start pointer is null");
  return append_entry(k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache, c_plane, c_sb, c_ss,
                      c_sh, dtype, B, n, H, D, capacity, 0, static_cast<const int32_t*>(start_dev),
                      static_cast<int32_t*>(status), stream);
}
