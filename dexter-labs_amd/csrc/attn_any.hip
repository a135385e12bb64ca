// The general attention kernels for gfx950: the calls that the 16-bit MFMA
// kernels (attn_fwd.hip) do not take -- fp32 inputs at any supported head
// dim, and bf16/f16 inputs at head dims 16, 32 and 256 -- under the same
// arguments and the same mask rules (attn_common.h). attn_any_kernel works in
// fp32 from end to end (fp32 inputs, and 16-bit inputs at head dim 16);
// attn_any16_kernel multiplies 16-bit inputs at head dims 32 and 256 on the
// 16-bit MFMA with fp32 sums (described at its definition). The reference op is dtype-generic (ops/reference/attention.py:
// 62-77: fp32 logits, softmax and product, one rounding to q's dtype) and the
// Triton kernel it stands beside takes any power-of-two head dim
// (ops/gfx1151/attention/blockwise_causal.py:162-172).
//
// Formulation. A work item is (batch, head, 64-query tile, key split), one
// workgroup of four waves, 16 queries per wave. Each wave computes the
// transposed score tile S^T = K Q^T with v_mfma_f32_16x16x4_f32 (fp32
// operands, fp32 sums): keys on the M axis, queries on N, so in the 16x16
// accumulator a lane holds one query (lane % 16) and four keys
// (4 (lane / 16) + r). The K index of an MFMA may be assigned to lane groups
// in any order as long as A and B agree: step j of 16-wide head-dim group u
// gives lane group g the element d = 16 u + 4 g + j, so a lane reads its K
// row and its q row as float4s. The probabilities then sit where the second
// product O^T += V^T P^T wants its B operand (key 4 g + j of step j: register
// j of the score accumulator), and V^T's A operand is one LDS read per step
// from the row-major V tile. The softmax is the exact online form (running
// max refreshed every tile), with q pre-multiplied by scale * log2(e) and
// exponentials as v_exp_f32; masked scores are -inf by selection after the
// product, so any scale sign or zero works as the reference's does.
//
// Pipeline. K/V tiles of 32 keys are loaded by all 256 threads (16-byte
// chunks, converted to fp32 for bf16/f16 inputs) into registers while the
// previous tile is computed, then stored to the other half of a two-stage LDS
// ring (rows padded by four floats). Tiles past the item's largest visible key
// end are never visited; rows past the split's keys are zero-filled.
//
// Splits. Calls with fewer work items than about two per CU split the key
// range; each split writes its unnormalised fp32 partial (acc, with the max
// m and sum l it is relative to) after the workspace's counter region (which
// it never writes), and a merge kernel combines the splits of each row.
#include "attn_common.h"

#include <math.h>

#include <algorithm>

namespace dx {
namespace {

constexpr int kAnyWaves = 4;
constexpr int kAnyRows = 16 * kAnyWaves;  // queries per work item
constexpr int kAnyThreads = 64 * kAnyWaves;
constexpr int kAnyKeys = 32;              // keys per tile
constexpr int kMergeThreads = 256;

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int per16 = 4;  // elements per 16-byte chunk
  // Elements [0, 4) of a 16-byte chunk as fp32.
  static __device__ __forceinline__ f32x4 lo(u32x4 w) { return __builtin_bit_cast(f32x4, w); }
  static __device__ __forceinline__ f32x4 hi(u32x4) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  // Four elements at p as fp32 (p 16-byte aligned).
  static __device__ __forceinline__ f32x4 load4(const char* p) {
    return *reinterpret_cast<const f32x4*>(p);
  }
  static __device__ __forceinline__ void store4(char* p, f32x4 v) {
    *reinterpret_cast<f32x4*>(p) = v;
  }
};
template <typename T> struct Elem16 {
  static constexpr int per16 = 8;
  static __device__ __forceinline__ f32x4 two(uint32_t a, uint32_t b) {
    return f32x4{to_f32(T{uint16_t(a & 0xffffu)}), to_f32(T{uint16_t(a >> 16)}),
                 to_f32(T{uint16_t(b & 0xffffu)}), to_f32(T{uint16_t(b >> 16)})};
  }
  static __device__ __forceinline__ f32x4 lo(u32x4 w) { return two(w[0], w[1]); }
  static __device__ __forceinline__ f32x4 hi(u32x4 w) { return two(w[2], w[3]); }
  // Four elements at p as fp32 (p 8-byte aligned).
  static __device__ __forceinline__ f32x4 load4(const char* p) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    return two(w[0], w[1]);
  }
  // One rounding of each fp32 value to T.
  static __device__ __forceinline__ void store4(char* p, f32x4 v) {
    u32x2 w;
    w[0] = pack2<T>(v[0], v[1]);
    w[1] = pack2<T>(v[2], v[3]);
    *reinterpret_cast<u32x2*>(p) = w;
  }
};
template <> struct Elem<bf16_t> : Elem16<bf16_t> {};
template <> struct Elem<f16_t> : Elem16<f16_t> {};

// Max and sum over the four lanes of a query (lanes c, c + 16, c + 32,
// c + 48): the gfx950 row swaps, VALU exchanges with no LDS round trip.
__device__ __forceinline__ float quad_max(float x) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Cached rows of sequence b (the device cursor clamped to the capacity the
// launch was planned for, or the per-sequence length of a ragged batch).
__device__ __forceinline__ int any_cache_len(const AttnArgs& a, int b) {
  if (a.cache_len_dev) return min(max(*a.cache_len_dev, 0), a.cache_len);
  return a.n_seg ? a.seg_cache[b] : a.cache_len;
}

template <int D> struct AnyLds {
  static constexpr int RS = D + 4;                      // row stride in floats
  static constexpr int tile = kAnyKeys * RS;            // floats per K or V tile
  static constexpr int bytes = 2 * 2 * tile * 4;        // two stages of K and V
};

template <int D, typename T>
__global__ __launch_bounds__(kAnyThreads) void attn_any_kernel(AttnArgs a) {
  using E = Elem<T>;
  constexpr int RS = AnyLds<D>::RS;
  constexpr int TILE = AnyLds<D>::tile;
  constexpr int CPR = D / E::per16;                    // 16-byte chunks per key row
  constexpr int NCH = kAnyKeys * CPR;                  // chunks per tile of K (or V)
  constexpr int NPT = (NCH + kAnyThreads - 1) / kAnyThreads;
  constexpr int DG = D / 16;                           // 16-wide head-dim groups
  constexpr int es = int(sizeof(T));
  static_assert(D % 16 == 0 && CPR >= 1, "head dim a multiple of 16");
  __shared__ __attribute__((aligned(16))) float lds[2 * 2 * TILE];

  const int tid = int(threadIdx.x), wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;

  int item = int(blockIdx.x);
  const int S = a.n_splits;
  const int split = item % S;
  item /= S;
  const int qt = item % a.n_qtiles;
  item /= a.n_qtiles;
  const int h = item % a.H, b = item / a.H;
  const int hk = h / a.kv_group;
  const int cache_len = any_cache_len(a, b);

  const int q0 = qt * kAnyRows;
  const int qi = q0 + 16 * wave + c;
  const bool qvalid = qi < a.Lq;
  const int row_end = qvalid ? cache_len + visible_end(a, qi, cache_len) : 0;
  const EndBounds eb = end_bounds(a, q0, min(q0 + kAnyRows, a.Lq) - 1);
  const int item_end = cache_len + eb.hi;  // no query of the item sees a key past it
  const int n_tiles = (item_end + kAnyKeys - 1) / kAnyKeys;
  const int per_split = (n_tiles + S - 1) / S;
  const int t_begin = min(split * per_split, n_tiles);
  const int t_end = min(t_begin + per_split, n_tiles);
  const int key_end = min(t_end * kAnyKeys, item_end);  // rows loaded: [t_begin * 32, key_end)
  const int lim = min(row_end, key_end);                // this lane's query sees keys < lim

  // q, pre-scaled: qr[u][j] = q[qi, 16 u + 4 g + j] * scale * log2(e). Rows
  // past Lq read the last row and become zeros: loads with no branch between
  // them all go out before the first wait.
  f32x4 qr[DG];
  {
    const int qr_i = min(qi, a.Lq - 1);
    const char* qrow = reinterpret_cast<const char*>(a.q) +
                       (int64_t(b) * a.q_sb + int64_t(qr_i) * a.q_sl + int64_t(h) * a.q_sh) * es;
#pragma unroll
    for (int u = 0; u < DG; ++u) qr[u] = E::load4(qrow + (16 * u + 4 * g) * es);
    const float qs = qvalid ? a.scale_log2 : 0.f;
#pragma unroll
    for (int u = 0; u < DG; ++u) qr[u] *= qs;
  }

  // This thread's chunks of a tile: chunk tid + 256 i is row ci / CPR,
  // chunk ci % CPR of that row.
  const char* kc = reinterpret_cast<const char*>(a.ck);
  const char* vc = reinterpret_cast<const char*>(a.cv);
  const char* kn = reinterpret_cast<const char*>(a.k);
  const char* vn = reinterpret_cast<const char*>(a.v);
  u32x4 kreg[NPT], vreg[NPT];
  auto load_tile = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int ci = tid + kAnyThreads * i;
      const int r = ci / CPR, cc = ci % CPR;
      const int j = t * kAnyKeys + r;
      kreg[i] = u32x4{0u, 0u, 0u, 0u};
      vreg[i] = u32x4{0u, 0u, 0u, 0u};
      if ((NCH % kAnyThreads == 0 || ci < NCH) && j < key_end) {
        int64_t ko, vo;
        const char *kb, *vb;
        if (j < cache_len) {
          ko = (int64_t(b) * a.c_sb + int64_t(j) * a.c_ss + int64_t(hk) * a.c_sh) * es;
          vo = ko;
          kb = kc;
          vb = vc;
        } else {
          const int64_t jn = j - cache_len;
          ko = (int64_t(b) * a.k_sb + jn * a.k_sl + int64_t(hk) * a.k_sh) * es;
          vo = (int64_t(b) * a.v_sb + jn * a.v_sl + int64_t(hk) * a.v_sh) * es;
          kb = kn;
          vb = vn;
        }
        kreg[i] = *reinterpret_cast<const u32x4*>(kb + ko + 16 * cc);
        vreg[i] = *reinterpret_cast<const u32x4*>(vb + vo + 16 * cc);
      }
    }
  };
  auto store_tile = [&](int stage) __attribute__((always_inline)) {
    float* kt = lds + stage * 2 * TILE;
    float* vt = kt + TILE;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int ci = tid + kAnyThreads * i;
      if (NCH % kAnyThreads == 0 || ci < NCH) {
        const int r = ci / CPR, cc = ci % CPR;
        const int o = r * RS + cc * E::per16;
        *reinterpret_cast<f32x4*>(kt + o) = E::lo(kreg[i]);
        *reinterpret_cast<f32x4*>(vt + o) = E::lo(vreg[i]);
        if (E::per16 == 8) {
          *reinterpret_cast<f32x4*>(kt + o + 4) = E::hi(kreg[i]);
          *reinterpret_cast<f32x4*>(vt + o + 4) = E::hi(vreg[i]);
        }
      }
    }
  };

  const float kNegInf = -__builtin_inff();
  float m = kNegInf, l = 0.f;
  f32x4 o[DG];
#pragma unroll
  for (int u = 0; u < DG; ++u) o[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (t_begin < t_end) {
    load_tile(t_begin);
    store_tile(0);
  }
  __syncthreads();
  for (int t = t_begin; t < t_end; ++t) {
    const int stage = (t - t_begin) & 1;
    if (t + 1 < t_end) load_tile(t + 1);
    const float* kt = lds + stage * 2 * TILE;
    const float* vt = kt + TILE;

    // Scores of keys 32 t + 16 s + 4 g + r for this lane's query.
    f32x4 sc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float* krow = kt + (16 * s + c) * RS + 4 * g;
#pragma unroll
      for (int u = 0; u < DG; ++u) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + 16 * u);
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[s] = mfma4(kv[j], qr[u][j], sc[s]);
      }
    }
    float tmax = kNegInf;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = t * kAnyKeys + 16 * s + 4 * g + r;
        sc[s][r] = key < lim ? sc[s][r] : kNegInf;
        tmax = fmaxf(tmax, sc[s][r]);
      }
    tmax = quad_max(tmax);
    const float mn = fmaxf(m, tmax);
    const float ref = mn == kNegInf ? 0.f : mn;  // nothing visible yet: every p is 0
    const float corr = __builtin_amdgcn_exp2f(m - ref);
    float ps = 0.f;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[s][r] = __builtin_amdgcn_exp2f(sc[s][r] - ref);
        ps += sc[s][r];
      }
    l = l * corr + ps;
    m = mn;
#pragma unroll
    for (int u = 0; u < DG; ++u) o[u] *= corr;
    // O^T[16 u + 4 g + r][query] += sum over keys of V^T P^T.
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* vrow = vt + (16 * s + 4 * g + j) * RS + c;
#pragma unroll
        for (int u = 0; u < DG; ++u) o[u] = mfma4(vrow[16 * u], sc[s][j], o[u]);
      }
    if (t + 1 < t_end) store_tile(stage ^ 1);
    __syncthreads();
  }

  const float lt = quad_sum(l);
  if (!qvalid) return;
  if (S == 1) {
    // Every key of the query was seen here: the result, rounded once to T.
    // A query that sees no key has lt = 0 and yields 0 * inf = NaN, as the
    // reference's softmax over an all -inf row does.
    const float inv = 1.f / lt;
    char* orow = reinterpret_cast<char*>(a.out) +
                 (int64_t(b) * a.o_sb + int64_t(qi) * a.o_sl + int64_t(h) * a.o_sh) * es;
#pragma unroll
    for (int u = 0; u < DG; ++u) E::store4(orow + (16 * u + 4 * g) * es, o[u] * inv);
    return;
  }
  // Partial of this split: row 16 wave + c of item blockIdx.x.
  const int64_t prow = int64_t(blockIdx.x) * kAnyRows + 16 * wave + c;
  float* po = reinterpret_cast<float*>(a.ws_o) + prow * D + 4 * g;
#pragma unroll
  for (int u = 0; u < DG; ++u) *reinterpret_cast<f32x4*>(po + 16 * u) = o[u];
  if (g == 0) *reinterpret_cast<f32x2*>(a.ws_ml + 2 * prow) = f32x2{m, lt};
}

// 16-bit inputs at head dims that are multiples of 32 and that the 16-bit
// kernels of attn_fwd.hip do not take (32 and 256): the same work items,
// 32-key tiles, two-stage LDS ring, masks and fp32 partials as
// attn_any_kernel, with 16-bit MFMA on the values as they are
// (v_mfma_f32_16x16x32_{bf16,f16}, fp32 sums) and K and V kept 16-bit in LDS.
//  * S^T = K Q^T: A = K (lane: key 16 s + l % 16, dims 32 ks + 8 g .. + 7),
//    B = Q^T (lane: query l % 16, the same dims), so the accumulator holds
//    query l % 16 and keys 16 s + 4 g + r, as in the fp32 form. Scores are
//    scaled by the signed scale x log2(e) in fp32, then masked by selection.
//  * O^T += V^T P^T with the MFMA's K index assigned to keys so that lane
//    group g's eight slots are keys {4 g .. 4 g + 3, 16 + 4 g .. 16 + 4 g + 3}:
//    B is the lane's own eight probabilities, rounded to T, and A (head_dim
//    column 16 u + l % 16 at those keys) comes from the row-major V tile by
//    two transposing reads (ds_read_b64_tr_b16: within each group of 16
//    lanes, lane i receives element i % 4 of the 8-byte chunks addressed by
//    lanes 4 e + i / 4, e = 0..3; lane 4 e + t addresses row 4 g + e, or
//    16 + 4 g + e, at columns 16 u + 4 t .. + 3). l sums the rounded
//    probabilities, the values the product uses.
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<f16_t> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)((__attribute__((address_space(3))) uint16_t*)(p)));
  return __builtin_bit_cast(u32x2, r);
}

template <int D> struct Any16Lds {
  static constexpr int RS = D + 8;             // row stride in 16-bit elements
  static constexpr int tile = kAnyKeys * RS;   // elements per K or V tile
  static constexpr int bytes = 2 * 2 * tile * 2;
};

template <int D, typename T>
__global__ __launch_bounds__(kAnyThreads) void attn_any16_kernel(AttnArgs a) {
  static_assert(sizeof(T) == 2 && D % 32 == 0, "16-bit inputs, head dim a multiple of 32");
  constexpr int RS = Any16Lds<D>::RS;
  constexpr int TILE = Any16Lds<D>::tile;
  constexpr int CPR = D / 8;                           // 16-byte chunks per key row
  constexpr int NCH = kAnyKeys * CPR;                  // chunks per tile of K (or V)
  constexpr int NPT = (NCH + kAnyThreads - 1) / kAnyThreads;
  constexpr int KS = D / 32;                           // S k-steps
  constexpr int DG = D / 16;                           // 16-wide head-dim groups
  constexpr int es = 2;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * TILE];

  const int tid = int(threadIdx.x), wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;

  int item = int(blockIdx.x);
  const int S = a.n_splits;
  const int split = item % S;
  item /= S;
  const int qt = item % a.n_qtiles;
  item /= a.n_qtiles;
  const int h = item % a.H, b = item / a.H;
  const int hk = h / a.kv_group;
  const int cache_len = any_cache_len(a, b);

  const int q0 = qt * kAnyRows;
  const int qi = q0 + 16 * wave + c;
  const bool qvalid = qi < a.Lq;
  const int row_end = qvalid ? cache_len + visible_end(a, qi, cache_len) : 0;
  const EndBounds eb = end_bounds(a, q0, min(q0 + kAnyRows, a.Lq) - 1);
  const int item_end = cache_len + eb.hi;
  const int n_tiles = (item_end + kAnyKeys - 1) / kAnyKeys;
  const int per_split = (n_tiles + S - 1) / S;
  const int t_begin = min(split * per_split, n_tiles);
  const int t_end = min(t_begin + per_split, n_tiles);
  const int key_end = min(t_end * kAnyKeys, item_end);
  const int lim = min(row_end, key_end);

  // Q^T operand per k-step: q[qi, 32 ks + 8 g .. + 7] (zeros past Lq: the
  // last row's loads, then masked, so no branch sits between the loads).
  u32x4 qb[KS];
  {
    const int qr_i = min(qi, a.Lq - 1);
    const char* qrow = reinterpret_cast<const char*>(a.q) +
                       (int64_t(b) * a.q_sb + int64_t(qr_i) * a.q_sl + int64_t(h) * a.q_sh) * es;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qb[ks] = *reinterpret_cast<const u32x4*>(qrow + (32 * ks + 8 * g) * es);
    const uint32_t qmask = qvalid ? ~0u : 0u;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] &= qmask;
  }
  const float cs = a.scale_log2;  // signed: masking selects after the product

  const char* kc = reinterpret_cast<const char*>(a.ck);
  const char* vc = reinterpret_cast<const char*>(a.cv);
  const char* kn = reinterpret_cast<const char*>(a.k);
  const char* vn = reinterpret_cast<const char*>(a.v);
  u32x4 kreg[NPT], vreg[NPT];
  auto load_tile = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int ci = tid + kAnyThreads * i;
      const int r = ci / CPR, cc = ci % CPR;
      const int j = t * kAnyKeys + r;
      kreg[i] = u32x4{0u, 0u, 0u, 0u};
      vreg[i] = u32x4{0u, 0u, 0u, 0u};
      if ((NCH % kAnyThreads == 0 || ci < NCH) && j < key_end) {
        int64_t ko, vo;
        const char *kb, *vb;
        if (j < cache_len) {
          ko = (int64_t(b) * a.c_sb + int64_t(j) * a.c_ss + int64_t(hk) * a.c_sh) * es;
          vo = ko;
          kb = kc;
          vb = vc;
        } else {
          const int64_t jn = j - cache_len;
          ko = (int64_t(b) * a.k_sb + jn * a.k_sl + int64_t(hk) * a.k_sh) * es;
          vo = (int64_t(b) * a.v_sb + jn * a.v_sl + int64_t(hk) * a.v_sh) * es;
          kb = kn;
          vb = vn;
        }
        kreg[i] = *reinterpret_cast<const u32x4*>(kb + ko + 16 * cc);
        vreg[i] = *reinterpret_cast<const u32x4*>(vb + vo + 16 * cc);
      }
    }
  };
  auto store_tile = [&](int stage) __attribute__((always_inline)) {
    uint16_t* kt = lds + stage * 2 * TILE;
    uint16_t* vt = kt + TILE;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int ci = tid + kAnyThreads * i;
      if (NCH % kAnyThreads == 0 || ci < NCH) {
        const int r = ci / CPR, cc = ci % CPR;
        *reinterpret_cast<u32x4*>(kt + r * RS + 8 * cc) = kreg[i];
        *reinterpret_cast<u32x4*>(vt + r * RS + 8 * cc) = vreg[i];
      }
    }
  };

  const float kNegInf = -__builtin_inff();
  float m = kNegInf, l = 0.f;
  f32x4 o[DG];
#pragma unroll
  for (int u = 0; u < DG; ++u) o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // This lane's transposing-read offsets (elements) in a V tile: rows 4 g + e
  // and 16 + 4 g + e, columns 4 t (+ 16 u per head-dim group).
  const int tr_lo = (4 * g + (c >> 2)) * RS + 4 * (c & 3);
  const int tr_hi = tr_lo + 16 * RS;

  if (t_begin < t_end) {
    load_tile(t_begin);
    store_tile(0);
  }
  __syncthreads();
  for (int t = t_begin; t < t_end; ++t) {
    const int stage = (t - t_begin) & 1;
    if (t + 1 < t_end) load_tile(t + 1);
    const uint16_t* kt = lds + stage * 2 * TILE;
    const uint16_t* vt = kt + TILE;

    f32x4 sc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = kt + (16 * s + c) * RS + 8 * g;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sc[s] = Mfma16<T>::run(*reinterpret_cast<const u32x4*>(krow + 32 * ks), qb[ks], sc[s]);
    }
    float tmax = kNegInf;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = t * kAnyKeys + 16 * s + 4 * g + r;
        sc[s][r] = key < lim ? sc[s][r] * cs : kNegInf;
        tmax = fmaxf(tmax, sc[s][r]);
      }
    tmax = quad_max(tmax);
    const float mn = fmaxf(m, tmax);
    const float ref = mn == kNegInf ? 0.f : mn;  // nothing visible yet: every p is 0
    const float corr = __builtin_amdgcn_exp2f(m - ref);
    u32x4 pb;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int w = 0; w < 2; ++w)
        pb[2 * s + w] = pack2<T>(__builtin_amdgcn_exp2f(sc[s][2 * w] - ref),
                                 __builtin_amdgcn_exp2f(sc[s][2 * w + 1] - ref));
    float ps = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      ps += to_f32(T{uint16_t(pb[w] & 0xffffu)}) + to_f32(T{uint16_t(pb[w] >> 16)});
    l = l * corr + ps;
    m = mn;
#pragma unroll
    for (int u = 0; u < DG; ++u) o[u] *= corr;
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const u32x2 lo = lds_tr16(vt + tr_lo + 16 * u);
      const u32x2 hi = lds_tr16(vt + tr_hi + 16 * u);
      o[u] = Mfma16<T>::run(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, o[u]);
    }
    if (t + 1 < t_end) store_tile(stage ^ 1);
    __syncthreads();
  }

  const float lt = quad_sum(l);
  if (!qvalid) return;
  if (S == 1) {
    const float inv = 1.f / lt;
    char* orow = reinterpret_cast<char*>(a.out) +
                 (int64_t(b) * a.o_sb + int64_t(qi) * a.o_sl + int64_t(h) * a.o_sh) * es;
#pragma unroll
    for (int u = 0; u < DG; ++u) Elem<T>::store4(orow + (16 * u + 4 * g) * es, o[u] * inv);
    return;
  }
  const int64_t prow = int64_t(blockIdx.x) * kAnyRows + 16 * wave + c;
  float* po = reinterpret_cast<float*>(a.ws_o) + prow * D + 4 * g;
#pragma unroll
  for (int u = 0; u < DG; ++u) *reinterpret_cast<f32x4*>(po + 16 * u) = o[u];
  if (g == 0) *reinterpret_cast<f32x2*>(a.ws_ml + 2 * prow) = f32x2{m, lt};
}

// Merge of the key splits: row (b, h, query) takes the S partials of its
// item group, M = max m_s, weights 2^(m_s - M) (0 for a split that saw no key),
// out = sum w_s acc_s / sum w_s l_s, rounded once to T. D / 4 threads per
// row, four head-dim elements each. Instantiated for at most NMAX splits, so
// that every split's loads go out before the first is used (slots past S read
// split S - 1 again and weigh nothing).
template <int D, typename T, int NMAX>
__global__ __launch_bounds__(kMergeThreads) void attn_any_merge_kernel(AttnArgs a) {
  using E = Elem<T>;
  constexpr int TPR = D / 4;
  constexpr int es = int(sizeof(T));
  const int64_t gid = int64_t(blockIdx.x) * kMergeThreads + threadIdx.x;
  const int64_t row = gid / TPR;
  const int dq = int(gid % TPR);
  if (row >= int64_t(a.B) * a.H * a.n_qtiles * kAnyRows) return;
  const int r = int(row % kAnyRows);
  const int64_t grp = row / kAnyRows;  // (b H + h) n_qtiles + qt
  const int qt = int(grp % a.n_qtiles);
  const int64_t bh = grp / a.n_qtiles;
  const int h = int(bh % a.H), b = int(bh / a.H);
  const int qi = qt * kAnyRows + r;
  if (qi >= a.Lq) return;
  const int S = a.n_splits;
  const float* po = reinterpret_cast<const float*>(a.ws_o);
  f32x2 ml[NMAX];
  f32x4 val[NMAX];
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    const int64_t pr = (grp * S + min(s, S - 1)) * kAnyRows + r;
    ml[s] = *reinterpret_cast<const f32x2*>(a.ws_ml + 2 * pr);
    val[s] = *reinterpret_cast<const f32x4*>(po + pr * D + 4 * dq);
  }
  const float kNegInf = -__builtin_inff();
  float mx = kNegInf;
#pragma unroll
  for (int s = 0; s < NMAX; ++s) mx = fmaxf(mx, ml[s][0]);
  float L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    const float w = mx == kNegInf || s >= S ? 0.f : __builtin_amdgcn_exp2f(ml[s][0] - mx);
    L += w * ml[s][1];
    acc += w * val[s];
  }
  char* orow = reinterpret_cast<char*>(a.out) +
               (int64_t(b) * a.o_sb + int64_t(qi) * a.o_sl + int64_t(h) * a.o_sh) * es;
  E::store4(orow + 4 * dq * es, acc * (1.f / L));
}

int64_t cdiv64(int64_t x, int64_t y) { return (x + y - 1) / y; }

template <int D, typename T>
hipError_t launch_any_dt(const AttnArgs& a, const AnyPlan& p, hipStream_t st) {
  // 16-bit inputs at head dims that are multiples of 32: 16-bit MFMA.
  if constexpr (sizeof(T) == 2 && D % 32 == 0)
    hipLaunchKernelGGL((attn_any16_kernel<D, T>), dim3(unsigned(p.items)), dim3(kAnyThreads), 0,
                       st, a);
  else
    hipLaunchKernelGGL((attn_any_kernel<D, T>), dim3(unsigned(p.items)), dim3(kAnyThreads), 0,
                       st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const int64_t threads = int64_t(a.B) * a.H * p.n_qtiles * kAnyRows * (D / 4);
  const dim3 grid(unsigned(cdiv64(threads, kMergeThreads)));
  if (p.splits <= 4)
    hipLaunchKernelGGL((attn_any_merge_kernel<D, T, 4>), grid, dim3(kMergeThreads), 0, st, a);
  else if (p.splits <= 8)
    hipLaunchKernelGGL((attn_any_merge_kernel<D, T, 8>), grid, dim3(kMergeThreads), 0, st, a);
  else
    hipLaunchKernelGGL((attn_any_merge_kernel<D, T, kMaxSplits>), grid, dim3(kMergeThreads), 0,
                       st, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_any_t(const AttnArgs& a, int D, const AnyPlan& p, hipStream_t st) {
  switch (D) {
    case 16: return launch_any_dt<16, T>(a, p, st);
    case 32: return launch_any_dt<32, T>(a, p, st);
    case 64: return launch_any_dt<64, T>(a, p, st);
    case 128: return launch_any_dt<128, T>(a, p, st);
    case 256: return launch_any_dt<256, T>(a, p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

AnyPlan plan_any(int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t D, int64_t max_cache,
                 int64_t ws_cap, int cus) {
  AnyPlan p{};
  p.n_qtiles = int(cdiv64(Lq, kAnyRows));
  const int64_t units = B * H * p.n_qtiles;
  const int64_t tiles = cdiv64(max_cache + Lk, kAnyKeys);
  const int forced = tuning(DX_TUNE_ATTN_SPLITS);
  int64_t s;
  if (forced > 0) {
    s = std::min<int64_t>(forced, kMaxSplits);
  } else {
    // About two work items per CU, at least two key tiles per split.
    s = units > 0 ? (2 * int64_t(cus)) / units : 1;
    s = std::min<int64_t>({s, kMaxSplits, cdiv64(tiles, 2)});
  }
  s = std::max<int64_t>(s, 1);
  auto bytes = [&](int64_t n) {
    return n > 1 ? kCounterRegion + units * n * kAnyRows * (D * 4 + 8) : int64_t(0);
  };
  if (ws_cap >= 0)
    while (s > 1 && bytes(s) > ws_cap) --s;
  p.splits = int(s);
  p.items = units * s;
  p.ws_bytes = bytes(s);
  return p;
}

hipError_t launch_any(const AttnArgs& a, int dtype, int D, const AnyPlan& p, hipStream_t st) {
  if (dtype == DX_F32) return launch_any_t<float>(a, D, p, st);
  if (dtype == DX_BF16) return launch_any_t<bf16_t>(a, D, p, st);
  return launch_any_t<f16_t>(a, D, p, st);
}

}  // namespace dx
