// Launch arguments and mask rules shared by the attention kernels: the
// 16-bit MFMA kernels of attn_fwd.hip and the general kernel of attn_any.hip
// (fp32 inputs, head dims other than 64 and 128).
#pragma once

#include "dx_common.h"

#include <stddef.h>

namespace dx {

constexpr int kMaxSeg = 64;    // sequences with their own cache length
constexpr int kMaxSplits = 16;

// Merge state of each work-item group (arrival and finish counters, chunk
// claims), indexed by the group's first partial, in a region of fixed size at
// the start of every attention workspace, so that no plan's partials ever
// overlap another plan's state. Zero before a launch, zero after it; kernels
// that keep no merge state never write it.
constexpr int kCounterStride = 16;           // ints per group state (arrivals, finished, claims)
constexpr int kCounterSlots = 4096;          // partials a launch that merges in-kernel may have
constexpr int64_t kCounterRegion = int64_t(kCounterSlots) * kCounterStride * 4;  // 256 KB

struct AttnArgs {
  const uint16_t* q; int64_t q_sb, q_sl, q_sh;
  const uint16_t* k; int64_t k_sb, k_sl, k_sh;
  const uint16_t* v; int64_t v_sb, v_sl, v_sh;
  const uint16_t* ck; const uint16_t* cv; int64_t c_sb, c_ss, c_sh;
  uint16_t* out; int64_t o_sb, o_sl, o_sh;
  uint16_t* ws_o;  // [partials][bm x D] f16 partial outputs acc / l scaled by 2^-e (row-major,
                   // or blocked: unit_off in attn_fwd.hip)
  float* ws_ml;    // [partials][bm][4] {exponent reference m (log2 units), sum l, scale exponent e, 0}
  const void* starts; int starts_i64; int n_blocks;
  int B, H, Lq, Lk;
  int kv_group;      // query heads per K/V head (grouped-query attention; 1 = one each)
  int causal;
  int n_qtiles;
  int bm;            // queries per work item: 128 (dual-stream decode) or 256 (paired groups)
  int comb_chunks;   // merge-kernel blocks per work-item group (rows min(bm, Lq) only)
  float scale_log2;  // |softmax scale| * log2(e)
  int negate_q;      // softmax scale < 0: q enters negated (exact), scale as |scale|
  int cache_len;     // uniform mode
  int n_splits;      // uniform mode
  // Segment table (ragged batches): segment i covers sequence seg_b[i] with
  // seg_splits[i] splits, work items [seg_base[i], seg_base[i+1]) and combine
  // blocks [comb_base[i], comb_base[i+1]). n_seg == 0: one uniform segment
  // over all B*H (batch, head) pairs.
  int n_seg;
  // Device-resident cache length (uniform mode): when set, the kernels read
  // the cached row count from this int32 at launch, clamped to [0, cache_len]
  // (cache_len then holds the cache capacity the launch was planned for), so
  // a captured graph follows the cache as it grows between replays.
  const int32_t* cache_len_dev;
  // Single-launch decode: the merge state of each work-item group
  // (kCounterStride ints, indexed by the group's first partial), zero before
  // the launch and returned to zero by the group's workgroups.
  int32_t* counters;
  // Time a workgroup waits for its group on the L2 fast path of the
  // in-kernel merge (s_memrealtime ticks); 0 skips the fast path.
  uint32_t fast_ticks;
  // Dual-stream kernel, split groups merged in the launch: spread the merge
  // over the group's splits (spread_split_group) instead of leaving it to
  // the last one to arrive (arrive_split_group).
  int spread;
  int seg_b[kMaxSeg], seg_splits[kMaxSeg], seg_cache[kMaxSeg];
  int seg_base[kMaxSeg + 1], comb_base[kMaxSeg + 1];
};

// Touch every 64-byte line of the argument header up front: four
// independent scalar loads and one wait, instead of the chain of dependent
// loads (each a cache miss at kernel start) that the first uses would
// otherwise issue one after another.
__device__ __forceinline__ void prefetch_args(const AttnArgs& a) {
  static_assert(offsetof(AttnArgs, n_seg) < 256, "argument header spans four lines");
  static_assert(offsetof(AttnArgs, cache_len_dev) / 64 == 4 && offsetof(AttnArgs, counters) / 64 == 4,
                "device cache length and counters on line five");
  const uint64_t l0 = reinterpret_cast<uint64_t>(a.q);
  const uint64_t l1 = uint64_t(a.v_sb);
  const uint64_t l2 = uint64_t(a.c_sh);
  const uint32_t l3 = uint32_t(a.n_seg);
  const uint64_t l4 = reinterpret_cast<uint64_t>(a.cache_len_dev);
  asm volatile("" ::"s"(l0), "s"(l1), "s"(l2), "s"(l3), "s"(l4));
}

// Block start i, read through the constant address space: the list does not
// change while a kernel runs, and that lets the compiler use scalar loads
// (counted by lgkmcnt) instead of vector loads, whose waits would also wait
// for every tile load in flight.
typedef __attribute__((address_space(4))) const int32_t const_i32;
typedef __attribute__((address_space(4))) const int64_t const_i64;
__device__ __forceinline__ int load_start(const AttnArgs& a, int i) {
  // A generic pointer to device memory is its global address: convert it
  // through the integer value.
  const uint64_t p = reinterpret_cast<uint64_t>(a.starts);
  return a.starts_i64 ? int(((const_i64*)p)[i]) : ((const_i32*)p)[i];
}

// Python's slice bound: index x of a length-n axis, negatives counted from the end.
__device__ __forceinline__ int slice_at(int x, int n) { return x < 0 ? max(x + n, 0) : min(x, n); }

// The block list as the reference reads it: pairs (lo, hi) of consecutive
// entries of (starts..., Lq), each setting mask[lo:hi, :hi] (rows by Python
// slicing, current keys [0, min(hi, Lq))). The starts are read 16 (+1) at a
// time as independent scalar loads, so each batch is one memory round trip
// instead of a chain of dependent ones; fn(lo, hi) sees every pair in order.
template <typename Fn>
__device__ __forceinline__ void for_each_block(const AttnArgs& a, Fn&& fn) {
  const int nb = a.n_blocks;
  for (int base = 0; base < nb; base += 16) {
    int st[17];
#pragma unroll
    for (int u = 0; u < 17; ++u) st[u] = base + u < nb ? load_start(a, base + u) : a.Lq;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (base + u < nb) fn(st[u], st[u + 1]);
  }
}

// Current keys [0, e) that the pair's column slice [cache_len : cache_len + hi]
// of the reference's [Lq, cache_len + Lq] mask sets, by Python's slice rules:
// min(hi, Lq) for hi >= 0; for a negative hi, nothing while the stop
// cache_len + hi is still >= 0 (it lies before the slice's start), and once it
// is negative it counts from the end of the key axis, leaving the current keys
// [0, cache_len + Lq + hi) (at least none).
__device__ __forceinline__ int pair_end(int hi, int cache_len, int Lq) {
  if (hi >= 0) return min(hi, Lq);
  return cache_len + hi < 0 ? max(cache_len + Lq + hi, 0) : 0;
}

// End (exclusive, in current-key coordinates) of the keys query i may see:
// the union of the block pairs whose row slice holds i, i.e. the largest
// pair_end among them, 0 when no pair holds i (such a row sees only the
// cache). For ascending starts this is the end of i's own block, and rows
// before the first start see no current key.
__device__ __forceinline__ int visible_end(const AttnArgs& a, int i, int cache_len) {
  if (a.causal) return i + 1;
  if (a.n_blocks == 0) return a.Lk;
  int e = 0;
  for_each_block(a, [&](int lo, int hi) __attribute__((always_inline)) {
    if (i >= slice_at(lo, a.Lq) && i < slice_at(hi, a.Lq)) e = max(e, pair_end(hi, cache_len, a.Lq));
  });
  return e;
}

// Visible-end bounds (current-key coordinates) over the rows [q_first,
// q_last] of a work item: lo <= visible_end(i) <= hi for each of them.
// Workgroup-uniform scalar work. With causal, no blocks, or block starts that
// are ascending and non-negative, visible_end is non-decreasing in i and the
// end rows give exact bounds. Any other list (the reference accepts one) gets
// the widest bounds, [0, Lq]: every current tile is visited and masked per
// key, so results stay exact and only the whole-tile skipping is lost.
struct EndBounds { int lo, hi; };
__device__ __forceinline__ EndBounds end_bounds(const AttnArgs& a, int q_first, int q_last) {
  if (a.causal || a.n_blocks == 0)
    return {__builtin_amdgcn_readfirstlane(visible_end(a, q_first, 0)),
            __builtin_amdgcn_readfirstlane(visible_end(a, q_last, 0))};
  bool ascending = true;
  int prev = 0;
  int e_first = 0, e_last = 0;
  for_each_block(a, [&](int lo, int hi) __attribute__((always_inline)) {
    ascending = ascending && lo >= prev;
    prev = lo;
    if (q_first >= slice_at(lo, a.Lq) && q_first < slice_at(hi, a.Lq))
      e_first = max(e_first, min(hi, a.Lq));
    if (q_last >= slice_at(lo, a.Lq) && q_last < slice_at(hi, a.Lq))
      e_last = max(e_last, min(hi, a.Lq));
  });
  // Uniform by construction (kernel arguments and workgroup-uniform rows);
  // readfirstlane lets the compiler keep the buffer descriptors built from
  // these bounds in scalar registers.
  return ascending ? EndBounds{__builtin_amdgcn_readfirstlane(e_first),
                               __builtin_amdgcn_readfirstlane(e_last)}
                   : EndBounds{0, a.Lq};
}

// ---------------------------------------------------------------------------
// The general kernel (attn_any.hip): calls the 16-bit MFMA kernels do not
// take, i.e. fp32 inputs at any supported head dim and bf16/f16 inputs at
// head dims 16, 32 and 256. Same arguments, same mask, fp32 arithmetic.
// ---------------------------------------------------------------------------
struct AnyPlan {
  int n_qtiles;      // 64-query tiles per (batch, head)
  int splits;        // key splits per tile (1: the kernel writes the output itself)
  int64_t items;     // workgroups of the main kernel
  int64_t ws_bytes;  // workspace: the counter region (left untouched), then the partials
};

// Head dims the general kernel is built for.
inline bool any_head_dim(int64_t D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

// Plan for B sequences of Lq queries over up to max_cache cached plus Lk
// current keys. ws_cap < 0: no workspace limit; otherwise the split count is
// lowered until the partials fit in ws_cap bytes (one split needs none).
AnyPlan plan_any(int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t D, int64_t max_cache,
                 int64_t ws_cap, int cus);

// Launch the plan: the main kernel, then, with more than one split, the
// merge kernel. a carries the general kernel's partials as ws_o (fp32
// values, reinterpreted) and ws_ml, its uniform split count as n_splits, its
// tile count as n_qtiles, and per-sequence cache lengths in seg_cache[b] when
// n_seg == B > 0. dtype: DX_BF16, DX_F16 or DX_F32.
hipError_t launch_any(const AttnArgs& a, int dtype, int D, const AnyPlan& p, hipStream_t st);

}  // namespace dx
