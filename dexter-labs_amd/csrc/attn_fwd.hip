// Blockwise-causal flash-attention forward for gfx950 (MI355X, CDNA4).
//
// Semantics: dexter's reference op (python/dexter/ops/reference/attention.py:
// 22-77): softmax((q k^T) * scale, masked) v over keys [cache[:cache_len] | k],
// where query i sees key j iff j < cache_len + end(i) (block mask :39-46,
// causal :33-37, one block :39-41). Computed flash-style: fp32 online softmax,
// bf16/f16 MFMA products, never materialising the score matrix.
//
// Formulation. Each wave owns 32 queries and computes the transposed score
// tile S^T = K Q^T with v_mfma_f32_32x32x16_{bf16,f16}: keys on the M axis,
// queries on the N axis. In the 32x32 accumulator a lane holds one query
// (lane % 32) and 16 keys, so the running max, running sum and rescale factor
// of a query are plain per-lane scalars; the only cross-lane step is one
// exchange with lane ^ 32 for the row max. The same lanes then feed
// O^T += V^T P^T: the probabilities P^T are already in B-operand position (one
// query per lane, keys along K), so they go to the second MFMA straight from
// registers. Because the K index of an MFMA may be assigned to (lane group,
// element) slots in any order as long as A and B agree, the eight keys a lane
// contributes per 16-key step are {4g..4g+3, 8+4g..8+4g+3} (g = lane / 32),
// exactly the keys its accumulator registers hold; the matching V^T operand
// is read from the row-major V tile with two gfx950 transposing LDS reads
// (ds_read_b64_tr_b16), so V is never transposed in registers.
//
// Softmax. Exponentials are v_exp_f32 on fma(score, scale*log2e, -ref).
// The reference max is refreshed lazily: only when some lane's max grows by
// more than 2^8 does the wave rescale its accumulators, so most tiles do no
// rescale work (exponentials stay <= 256, exact in fp32 and in the 16-bit P).
//
// Masking. Per workgroup the bounds kv_min / kv_max (over its queries'
// visible-key ends, derived on the device from block_starts) split the key
// tiles into three kinds: tiles below kv_min need no mask, tiles from kv_max on
// are never visited (whole future blocks are skipped), and only the straddling
// tiles are masked elementwise. Rows at or beyond kv_max are zero-filled in
// LDS instead of loaded, so nothing a workgroup cannot see reaches its
// arithmetic.
//
// Pipeline. A stream is four waves (128 queries); waves whose 32 queries
// are all past the end only help load. Decode-shaped calls (short query
// chunk, long cache) run two streams per workgroup on alternate key tiles of
// the same range (global -> registers -> LDS, double buffered, the next
// tile's loads in flight behind the current tile's compute) -- two waves per
// SIMD, so one stream's softmax overlaps the other's MFMAs -- and merge the
// streams through LDS, halving the split-KV partials two separate workgroups
// would write. Prefill runs two groups of four waves on 256 queries, half a
// key tile apart, with K/V tiles moved to LDS by DMA (attn_pair_kernel).
//
// Work decomposition. A work item is (batch, head, query tile, key split).
// Short query chunks over long caches split the key range over several
// workgroups (split-KV) and the partial (max, sum, acc) triples are merged
// either by a second kernel or, in the same launch, by the last split of the
// group to finish (arrive_split_group). Items are issued heaviest-first, and when the
// number of heads per segment is a multiple of 8 every item of one head lands
// on one XCD (item i runs on XCD i % 8), so its K/V and partials stay in one
// L2. Ragged batches (one cache length per sequence) get one segment per
// sequence with its own split count, longest sequence first.
#include "attn_common.h"

#include <float.h>
#include <limits.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <set>
#include <type_traits>
#include <utility>
#include <vector>

namespace dx {
namespace {

// Phase stamps of the timeline build (`build.py --timeline`, which defines
// DX_TIMELINE and writes a library of its own; the product library has no
// stamps). Thread 0 of workgroup w < kTimelineGroups of the decode kernel
// writes the device's 100 MHz s_memrealtime clock into word k of row w of
// g_timeline (kTimelineSlots words a row); the merge kernel writes its
// block's start and end into g_timeline_merge. Words:
//   0 start, 1 Q in registers, 2 tile loop done, 3 stream hand-over done,
//   4 result stores issued, 5 arrival counted (split merged in the launch),
//   6 merge loads combined (the merging split), 7 end (stores issued);
//   8 split | n_splits << 8 | batch << 16 | merge state << 32,
//   9 tiles | barrier rounds << 16, 10 XCD; 16 + i: round i's tiles in LDS.
#ifdef DX_TIMELINE
constexpr int kTimelineSlots = 32, kTimelineGroups = 2048;
__device__ uint64_t g_timeline[kTimelineSlots * kTimelineGroups];
__device__ uint64_t g_timeline_merge[2 * 8 * kTimelineGroups];
__device__ __forceinline__ void timeline_word(int k, uint64_t v) {
  if (threadIdx.x == 0 && blockIdx.x < unsigned(kTimelineGroups))
    g_timeline[blockIdx.x * kTimelineSlots + k] = v;
}
__device__ __forceinline__ void timeline_merge_word(int k) {
  if (threadIdx.x == 0 && blockIdx.x < unsigned(8 * kTimelineGroups))
    g_timeline_merge[2 * blockIdx.x + k] = __builtin_amdgcn_s_memrealtime();
}
#define DX_STAMP(k) timeline_word((k), __builtin_amdgcn_s_memrealtime())
#define DX_NOTE(k, v) timeline_word((k), uint64_t(v))
#define DX_MERGE_STAMP(k) timeline_merge_word(k)
#else
#define DX_STAMP(k) ((void)0)
#define DX_NOTE(k, v) ((void)0)
#define DX_MERGE_STAMP(k) ((void)0)
#endif

constexpr int kBN = 64;        // keys per tile
constexpr int kNW = 4;         // waves per workgroup
constexpr int kBM = 32 * kNW;  // queries per workgroup
constexpr int kPairWaves = 8;  // waves per workgroup of the paired-group kernel
constexpr int kBMPair = 256;   // its queries per workgroup

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 r = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, r);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 against (1, 1)).
  static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p),
                                           __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
  }
};
template <> struct Mfma<f16_t> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    f16x2 r = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, r);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_f16 against (1, 1)).
  static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p),
                                  __builtin_bit_cast(f16x2, 0x3c003c00u), acc, false);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS geometry, per stage: a K tile [64 keys][D] and a V tile [64 keys][D],
// both row-major as they lie in memory.
//  - K rows are padded by 8 elements (272 B for D=128): the QK^T A operand is
//    a 16-byte read of 16 different rows per pass, which then hit 64
//    distinct banks.
//  - V rows are padded by 32 elements (320 B for D=128, 192 B for D=64; a
//    pitch of 16 mod 64 dwords): the PV A operand comes from
//    ds_read_b64_tr_b16, each of which touches 8 rows x 16 dwords, and with
//    this pitch those spans tile the 64 banks exactly twice (the minimum).
template <int D> struct Lds {
  static constexpr int kPitch = D + 8;
  static constexpr int vPitch = D + 32;
  static constexpr int kElems = kBN * kPitch;
  static constexpr int vElems = kBN * vPitch;
  static constexpr int stage = kElems + vElems;  // one K tile + one V tile
  static constexpr int bytes = 2 * stage * 2;    // double buffered, 16-bit elements
  static_assert(bytes >= 4 * (2 + D / 2) * 64 * kNW,
                "a stream's region must hold the (max, sum, acc) hand-over");
};

// Where a workgroup reads its keys and values: raw buffer descriptors over
// the cached rows and over the new rows of one (batch, head), each bounded to
// the rows the workgroup may see. Offsets are 32-bit bytes (the host checks
// they fit); a row past a descriptor's bound reads as zeros without touching
// memory, so rows at or past kv_max (and past the cache's end) are
// zero-filled without a branch.
//
// Key tiles never straddle the two sources: tiles [0, n_ct) cover the cache
// (the last one possibly partial), tiles [n_ct, ...) the new keys from key
// cache_len on. Each tile then has one descriptor and one row stride,
// selected with scalar instructions, and one load path.
struct KvSrc {
  __amdgpu_buffer_rsrc_t kc, vc, kn, vn;
  __amdgpu_buffer_rsrc_t none;  // zero records: every lane reads zeros
  int c_ss2, k_sl2, v_sl2;  // row strides in bytes
  int n_ct;                 // cache tiles: ceil(cache_len / kBN)
};

constexpr int kBufWord3 = 0x00020000;  // gfx9-family raw buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base, int rows,
                                                           int row_bytes, int D) {
  const int bytes = rows > 0 ? (rows - 1) * row_bytes + D * 2 : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, bytes,
                                           kBufWord3);
}

// K/V tile loads of the decode kernel: each cache row is read once per call,
// so the loads are marked non-temporal (cache policy bit NT = 2).
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

// One K tile and one V tile of a workgroup's share, staged in registers
// between the global load and the LDS store. Thread x moves 16-byte chunks
// x, x + 256, ... of each tile: 16 consecutive threads cover one 256-byte
// key row, so every load instruction reads whole rows.
template <int D>
struct TileRegs {
  static constexpr int NT = 64 * kNW;
  static constexpr int CPR = D / 8;        // 16-byte chunks per key row
  static constexpr int CH = kBN * CPR;     // chunks per tile
  static constexpr int CPT = CH / NT;      // chunks per thread
  static constexpr int RPI = NT / CPR;     // rows between a thread's consecutive chunks
  static_assert(CH % NT == 0, "tile must split evenly over the threads");
  u32x4 kr[CPT], vr[CPT];

  // Tile t (uniform). ``live`` false loads nothing (a descriptor of zero
  // records: all lanes read zeros) but keeps one straight-line path, so the
  // compiler's wait counts for earlier loads stay exact.
  __device__ __forceinline__ void load(int tid, const KvSrc& src, int t, bool live) {
    const int r0 = tid / CPR, colb = (tid % CPR) * 16;
    const bool in_cache = t < src.n_ct;
    // Value selects (not a select of member addresses, which would keep the
    // descriptors in scratch memory).
    const __amdgpu_buffer_rsrc_t kc = src.kc, kn = src.kn, vc = src.vc, vn = src.vn;
    const __amdgpu_buffer_rsrc_t none = src.none;
    __amdgpu_buffer_rsrc_t rk = in_cache ? kc : kn;
    __amdgpu_buffer_rsrc_t rv = in_cache ? vc : vn;
    if (!live) rk = rv = none;
    const int sk = in_cache ? src.c_ss2 : src.k_sl2;
    const int sv = in_cache ? src.c_ss2 : src.v_sl2;
    const int row = (in_cache ? t : t - src.n_ct) * kBN + r0;
    const int ok = row * sk + colb, ov = row * sv + colb;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      kr[i] = buf_load16(rk, ok + i * RPI * sk);
      vr[i] = buf_load16(rv, ov + i * RPI * sv);
    }
  }

  // K or V alone (the pipelined single-stream loop keeps them a tile apart).
  __device__ __forceinline__ void loadK(int tid, const KvSrc& src, int t, bool live) {
    const int r0 = tid / CPR, colb = (tid % CPR) * 16;
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t kc = src.kc, kn = src.kn, none = src.none;
    __amdgpu_buffer_rsrc_t rk = in_cache ? kc : kn;
    if (!live) rk = none;
    const int sk = in_cache ? src.c_ss2 : src.k_sl2;
    const int ok = ((in_cache ? t : t - src.n_ct) * kBN + r0) * sk + colb;
#pragma unroll
    for (int i = 0; i < CPT; ++i) kr[i] = buf_load16(rk, ok + i * RPI * sk);
  }
  __device__ __forceinline__ void loadV(int tid, const KvSrc& src, int t, bool live) {
    const int r0 = tid / CPR, colb = (tid % CPR) * 16;
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t vc = src.vc, vn = src.vn, none = src.none;
    __amdgpu_buffer_rsrc_t rv = in_cache ? vc : vn;
    if (!live) rv = none;
    const int sv = in_cache ? src.c_ss2 : src.v_sl2;
    const int ov = ((in_cache ? t : t - src.n_ct) * kBN + r0) * sv + colb;
#pragma unroll
    for (int i = 0; i < CPT; ++i) vr[i] = buf_load16(rv, ov + i * RPI * sv);
  }
  __device__ __forceinline__ void storeK(int tid, uint16_t* Ks) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4*>(Ks + (c / CPR) * Lds<D>::kPitch + (c % CPR) * 8) = kr[i];
    }
  }
  __device__ __forceinline__ void storeV(int tid, uint16_t* Vs) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4*>(Vs + (c / CPR) * Lds<D>::vPitch + (c % CPR) * 8) = vr[i];
    }
  }

  __device__ __forceinline__ void store(int tid, uint16_t* Ks, uint16_t* Vs) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      *reinterpret_cast<u32x4*>(Ks + row * Lds<D>::kPitch + col) = kr[i];
      *reinterpret_cast<u32x4*>(Vs + row * Lds<D>::vPitch + col) = vr[i];
    }
  }
};

// Direct global -> LDS tile loads (gfx950 buffer_load_dwordx4 ... lds, no
// registers in between). One such instruction moves 64 lanes x 16 bytes into
// 1 KB of LDS at M0 + 16 lane, while each lane's global offset is free: the
// padded tile layout (K rows of kPitch, V rows of vPitch elements) is cut
// into 1 KB pieces, and lane l of piece q fetches whatever row/column lands
// at byte 1024 q + 16 l -- or, for a padding slot, an offset past every
// buffer's end, which writes zeros. Rows past a descriptor's bound read as
// zeros too. The four waves of a stream take pieces w, w + 4, ...; each
// thread keeps its (row, byte column) per piece, packed, -1 for padding.
// Completion is tracked by vmcnt: a wave waits for its own pieces before the
// barrier that publishes the tile.
typedef __attribute__((address_space(3))) void lds_void_t;

// One DMA piece: 64 lanes x 16 bytes from the buffer at per-lane offsets into
// LDS bytes [lds, lds + 1024). Written as inline assembly on purpose: the
// compiler's wait-count pass treats the builtin form as an LDS write of
// unknown extent and puts a full vmcnt wait before every later LDS read,
// which would stall each tile's reads on the next tile's still-flying
// pieces. The callers wait for their pieces explicitly (s_waitcnt before the
// barrier that publishes them). M0 holds the LDS base; nothing else in these
// kernels uses M0 (gfx9 LDS instructions do not read it), and the s_nop is
// the one wait state an LDS DMA needs after M0 is written.
__device__ __forceinline__ void dma_piece(__amdgpu_buffer_rsrc_t rsrc, const uint16_t* lds,
                                          uint32_t voff) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(
      uint32_t(uintptr_t((__attribute__((address_space(3))) const uint16_t*)lds)));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(base), "v"(voff), "s"(rsrc)
               : "memory");
}

// Templated on the element type too, although nothing in it depends on T:
// with one TileDma<D> shared by the bf16 and f16 kernels, hipcc (ROCm 7.2)
// silently drops the host-side stub of whichever kernel instantiates it
// second, leaving an undefined symbol in the library.
template <int D, typename T, int NWV = kNW>  // NWV waves share each tile's pieces
struct TileDma {
  static constexpr int KSL = Lds<D>::kPitch / 8;  // 16-byte slots per K row
  static constexpr int VSL = Lds<D>::vPitch / 8;
  static constexpr int KQ = kBN * KSL / 64;       // pieces per K tile
  static constexpr int VQ = kBN * VSL / 64;
  static constexpr int KM = (KQ + NWV - 1) / NWV;  // pieces per wave (at most)
  static constexpr int VM = (VQ + NWV - 1) / NWV;
  static_assert(kBN * KSL % 64 == 0 && kBN * VSL % 64 == 0, "tiles must be whole pieces");
  static constexpr uint32_t kPast = 0x80000000u;  // beyond any descriptor's records
  int kp[KM], vp[VM];  // (row << 16) | byte column, or -1

  __device__ __forceinline__ void init(int wave, int lane) {
#pragma unroll
    for (int m = 0; m < KM; ++m) {
      const int x = (wave + NWV * m) * 64 + lane, row = x / KSL, sl = x % KSL;
      kp[m] = sl < D / 8 ? (row << 16) | (sl * 16) : -1;
    }
#pragma unroll
    for (int m = 0; m < VM; ++m) {
      const int x = (wave + NWV * m) * 64 + lane, row = x / VSL, sl = x % VSL;
      vp[m] = sl < D / 8 ? (row << 16) | (sl * 16) : -1;
    }
  }
  __device__ __forceinline__ static uint32_t offset(int pc, int row0, int stride) {
    return pc < 0 ? kPast : uint32_t((row0 + (pc >> 16)) * stride + (pc & 0xffff));
  }
  // Tile t's K into Ks (and V into Vs) from wave ``wave`` of the stream.
  __device__ __forceinline__ void issueK(const KvSrc& src, int t, int wave, uint16_t* Ks) const {
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t kc = src.kc, kn = src.kn;
    const __amdgpu_buffer_rsrc_t rk = in_cache ? kc : kn;
    const int stride = in_cache ? src.c_ss2 : src.k_sl2;
    const int row0 = (in_cache ? t : t - src.n_ct) * kBN;
#pragma unroll
    for (int m = 0; m < KM; ++m)
      if (NWV * m + NWV - 1 < KQ || wave + NWV * m < KQ)  // first: always true, known at compile time
        dma_piece(rk, Ks + (wave + NWV * m) * 512, offset(kp[m], row0, stride));
  }
  __device__ __forceinline__ void issueV(const KvSrc& src, int t, int wave, uint16_t* Vs) const {
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t vc = src.vc, vn = src.vn;
    const __amdgpu_buffer_rsrc_t rv = in_cache ? vc : vn;
    const int stride = in_cache ? src.c_ss2 : src.v_sl2;
    const int row0 = (in_cache ? t : t - src.n_ct) * kBN;
#pragma unroll
    for (int m = 0; m < VM; ++m)
      if (NWV * m + NWV - 1 < VQ || wave + NWV * m < VQ)  // first: always true, known at compile time
        dma_piece(rv, Vs + (wave + NWV * m) * 512, offset(vp[m], row0, stride));
  }
};

// LDS of the paired-group kernel: NST stages (K tile + V tile each, rows
// of D elements, no padding; three in the prefill kernel). Bank conflicts are avoided by
// permuting the 16-byte chunks within each row instead of padding, so that
// the DMA pieces are whole rows and the eight waves get the same number of
// them:
//  - K chunk c of row r sits at chunk c ^ kswz(r). The QK^T operand reads of
//    one instruction take one logical chunk of rows 0..31; kswz gives rows
//    0..15 (and 16..31) distinct chunks, and rows 0..31 distinct (row parity,
//    chunk) pairs.
//  - V chunk c of row r sits at chunk c ^ 4 vswz(r) (only the 64-byte column
//    group moves, so the 8-byte transposing reads keep their pairs). One
//    transposing read covers rows r0..r0+3 (lanes 0-31) and r0+4..r0+7
//    (lanes 32-63) over a 64-byte column group; vswz gives each run of four
//    rows distinct groups, and the eight rows distinct (row mod 2 (D = 128)
//    or row mod 4 (D = 64), group) pairs.
// Both swizzles are invariant under the row offsets the reads add as
// immediates (32 K rows, 8 and 16 V rows).
template <int D, int NST = 3> struct PairLds {
  static constexpr int kElems = kBN * D, vElems = kBN * D;  // one tile each
  static constexpr int stages = NST;
  // Element offsets of stage s's K and V tiles: the NST K tiles, then the
  // NST V tiles, so that every read offset fits the LDS instructions'
  // 16-bit immediate (given a per-lane base that includes the V region's).
  static constexpr int kstage(int s) { return s * kElems; }
  static constexpr int vstage(int s) { return stages * kElems + s * vElems; }
  static constexpr int bytes = stages * (kElems + vElems) * 2;
  __device__ __forceinline__ static int kswz(int r) {
    return D == 128 ? (r & 15) ^ ((r >> 4) & 1) : ((r >> 2) ^ (4 * ((r >> 1) & 1))) & 7;
  }
  __device__ __forceinline__ static int vswz(int r) {
    return D == 128 ? (r & 3) ^ ((r >> 2) & 1) : ((r >> 1) ^ (r >> 2)) & 1;
  }
};

// Fixed DMA slots of the paired-group kernel. A K (or V) tile is PK pieces of
// RPP whole rows; piece p of each goes to wave p % 8, so every wave issues
// exactly NK K pieces and NK V pieces per tile step, none of them behind a
// branch. Lane l of a piece fills physical chunk l % CR of row l / CR, so it
// fetches the logical chunk the swizzle puts there. Slots of steps outside
// the work item still issue (and write zeros). The count of a wave's pieces in flight is therefore a
// compile-time constant, which lets a wave wait for one step's pieces while
// the next step's are still flying.
template <int D, typename T, int NST = 3>
struct PairDma {
  using L = PairLds<D, NST>;
  static constexpr int CR = D / 8;             // 16-byte chunks per row
  static constexpr int RPP = 64 / CR;          // rows per piece
  static constexpr int PK = kBN / RPP;         // pieces per K (or V) tile
  static constexpr int NK = PK / kPairWaves;   // K (and V) slots per wave
  static constexpr int NP = 2 * NK;            // slots per wave and step
  static_assert(PK % kPairWaves == 0, "tile pieces must deal evenly over the waves");
  // This lane's byte offset per slot, within its tile, for the new-key row
  // stride (on), and what to add for the cache's row stride instead (dc).
  uint32_t on[NP], dc[NP];

  __device__ __forceinline__ void init(int wid, int lane, const KvSrc& src) {
#pragma unroll
    for (int m = 0; m < NP; ++m) {
      const int r = (wid + kPairWaves * (m % NK)) * RPP + lane / CR, x = lane % CR;
      const int c = m < NK ? x ^ L::kswz(r) : x ^ (4 * L::vswz(r));
      const uint32_t sn = uint32_t(m < NK ? src.k_sl2 : src.v_sl2);
      on[m] = uint32_t(r) * sn + uint32_t(c * 16);
      dc[m] = uint32_t(r) * (uint32_t(src.c_ss2) - sn);
    }
  }
  // Slot m (K slots first): its piece of K_{jk} into K stage kst, or of
  // V_{jv} into V stage vst (steps relative to the work item's first tile,
  // >= -1; step j uses stage j mod 3); lds is the LDS byte address of the
  // tile area. A step outside [0, nt) reads
  // past the end of its descriptor (bit 31 set: descriptors hold < 2^31
  // bytes) and fills its stage with zeros: that stage is free at the time
  // (as for a live step), and step -1's V stage is the one the first MFMA
  // phase must find zeroed anyway. Two vector instructions per piece; the
  // rest is scalar. No selects of vector values on the step's (uniform)
  // conditions: the compiler turns those into branches, which would cut the
  // phase's schedule.
  __device__ __forceinline__ void issue(int m, const KvSrc& src, uint32_t lds, int t_begin,
                                        int nt, int jk, int jv, int kst, int vst,
                                        int wid) const {
    const bool is_k = m < NK;  // known at compile time in every caller
    const int jt = is_k ? jk : jv;
    const bool live = jt >= 0 && jt < nt;
    const int t = t_begin + jt;
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t xc = is_k ? src.kc : src.vc, xn = is_k ? src.kn : src.vn;
    const __amdgpu_buffer_rsrc_t r = in_cache ? xc : xn;
    const int stride = in_cache ? src.c_ss2 : (is_k ? src.k_sl2 : src.v_sl2);
    const int row0 = (in_cache ? t : t - src.n_ct) * kBN;
    const uint32_t base = live ? uint32_t(row0) * uint32_t(stride) : 0x80000000u;
    const uint32_t cmask = in_cache ? ~0u : 0u;
    const int p = wid + kPairWaves * (m % NK);
    const int at = (is_k ? L::kstage(kst) : L::vstage(vst)) + p * 512;
    dma_piece_at(r, lds + 2 * at, on[m] + (dc[m] & cmask) + base);
  }
};

// Transposing LDS read (gfx950 ds_read_b64_tr_b16). Within each group of 16
// lanes, lane i receives element i % 4 of the 8-byte chunks addressed by
// lanes 4e + i / 4, e = 0..3 of its group.
typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)((__attribute__((address_space(3))) uint16_t*)(p)));
  return __builtin_bit_cast(u32x2, r);
}

// LDS accesses by byte address (for the swizzled layout, whose addresses are
// built with XOR).
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(uintptr_t((__attribute__((address_space(3))) const void*)(p)));
}
__device__ __forceinline__ u32x4 lds_read_b128_at(uint32_t addr) {
  return *reinterpret_cast<const lds_u32x4*>(addr);
}
__device__ __forceinline__ u32x2 lds_read_tr16_at(uint32_t addr) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4i16*>(addr));
  return __builtin_bit_cast(u32x2, r);
}

// A row area in LDS: rows of D 16-bit elements, K-swizzled (chunk c of row r
// at c ^ kswz(r), conflict-free for the K-operand read pattern and for 8-byte
// writes of 32 rows). The kernels stage their result rows in one after the
// tile loop, so that the result leaves as 16-byte row chunks, 64 per
// instruction, instead of as 8-byte pieces of 32 rows each (which the texture
// path processes one row line at a time); the prefill kernel also receives
// its Q rows in one, by LDS DMA in whole-row pieces (lane l of piece p: row
// p RPP + l / CR, physical chunk l % CR).
// Cache policy of buffer loads and stores (their aux operand) at device
// scope (sc1): stores go through to memory and loads fetch the device-coherent
// copy, so workgroups on different XCDs (each with its own L2) see each
// other's data once the stores have completed.
constexpr int kScDevice = 16;

template <int D> struct RowArea {
  using L = PairLds<D>;
  static constexpr int CR = D / 8, RPP = 64 / CR, RB = 2 * D;
  // Byte address of logical 16-byte chunk c of row r of the area at ``area``.
  __device__ __forceinline__ static uint32_t at(uint32_t area, int r, int c) {
    return area + uint32_t(r * RB + 16 * (c ^ L::kswz(r)));
  }
  // Rows [r0, r0 + rows) of the area, as staged by one wave (rows <= 32), out
  // to the rows of a buffer with the given row stride; the wave's other rows
  // are not written (bounded by the row count, not by the buffer: a one-row
  // tensor may come with row stride 0).
  // kAux: the stores' cache policy (0, or kScDevice: through to memory); NR:
  // rows r0 .. r0 + NR - 1 (32: the wave's whole row range).
  template <int kAux = 0, int NR = 32>
  __device__ __forceinline__ static void store_rows(__amdgpu_buffer_rsrc_t ro, int row_bytes,
                                                    int rows, uint32_t area, int r0, int lane) {
    static_assert(NR % RPP == 0 && NR <= 32, "whole store instructions within a wave's rows");
#pragma unroll
    for (int i = 0; i < NR / RPP; ++i) {
      const int r = i * RPP + lane / CR, x = lane % CR;
      const u32x4 v = lds_read_b128_at(at(area, r0 + r, x));
      const uint32_t o = uint32_t(r) * uint32_t(row_bytes) + 16u * x;
      __builtin_amdgcn_raw_buffer_store_b128(v, ro, int(r < rows ? o : 0x80000000u), 0, kAux);
    }
  }
};

// The paired kernel's row area: its BM query rows, after the K/V stages.
template <int D> struct PairRows : RowArea<D> {
  using A = RowArea<D>;
  static constexpr int off = PairLds<D>::bytes;                   // byte offset in LDS
  static constexpr int bytes = kBMPair * A::RB;
  static constexpr int NPW = kBMPair / A::RPP / kPairWaves;       // Q pieces per wave
  static_assert(kBMPair % (A::RPP * kPairWaves) == 0, "Q pieces deal evenly over the waves");
  static_assert(off + bytes <= 160 * 1024, "stages and rows fit one workgroup's LDS");
  // This wave's Q pieces into the area at ``area``: rows [0, rows) of the
  // work item; the rest read as zeros (an offset with bit 31 set is past
  // every descriptor's end).
  __device__ __forceinline__ static void load_q(__amdgpu_buffer_rsrc_t rq, int q_sl2, int rows,
                                                uint32_t area, int wid, int lane) {
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      const int pc = wid + kPairWaves * i;
      const int r = pc * A::RPP + lane / A::CR, x = lane % A::CR;
      const uint32_t o = uint32_t(r) * uint32_t(q_sl2) + uint32_t(16 * (x ^ A::L::kswz(r)));
      dma_piece_at(rq, area + pc * 1024, r < rows ? o : 0x80000000u);
    }
  }
};


// Position of a work item (or of a combine block) in the schedule.
struct Coord {
  int b, h, qtile, split;  // split: key split (work items) or row chunk (combine)
  int n_splits, cache_len;
  int64_t pbase;           // partial index of split 0 of this (b, h, qtile)
};

// Map index i of a range laid out as [groups G][ranks R] with XCD-aware
// interleaving: when G % 8 == 0, index i runs on XCD i % 8 and all ranks of
// group g share XCD g % 8.
__device__ __forceinline__ void split_index(int i, int G, bool contiguous, int& gidx,
                                            int& rank) {
  // Unsigned arithmetic throughout: every index is non-negative, and unsigned
  // division by a uniform value is shorter than signed.
  const uint32_t ui = uint32_t(i), uG = uint32_t(G);
  if ((uG & 7u) == 0) {
    const uint32_t xcd = ui & 7u, slot = ui >> 3, g8 = uG >> 3;
    const uint32_t q = slot / g8, rem = slot - q * g8;
    // contiguous: XCD x takes groups [x G/8, (x+1) G/8), so heads that share
    // a K/V head (adjacent under grouped-query attention) share an L2.
    gidx = int(contiguous ? xcd * g8 + rem : xcd + 8u * rem);
    rank = int(q);
  } else {
    const uint32_t q = ui / uG;
    gidx = int(ui - q * uG);
    rank = int(q);
  }
}

// per_q: ranks per query tile (key splits for work items, row chunks for the
// combine); base: the segment table column (seg_base or comb_base).
__device__ __forceinline__ Coord locate(const AttnArgs& a, int idx, bool combine, int chunks) {
  Coord c;
  int G, local, seg_item_base;
  if (a.n_seg == 0) {
    G = a.B * a.H;
    c.n_splits = a.n_splits;
    c.cache_len = a.cache_len;
    if (a.cache_len_dev) c.cache_len = min(max(*a.cache_len_dev, 0), a.cache_len);
    local = idx;
    seg_item_base = 0;
  } else {
    const int* base = combine ? a.comb_base : a.seg_base;
    int s = 0;
    while (s + 1 < a.n_seg && idx >= base[s + 1]) ++s;
    G = a.H;
    c.n_splits = a.seg_splits[s];
    c.cache_len = a.seg_cache[s];
    local = idx - base[s];
    seg_item_base = a.seg_base[s];
    c.b = a.seg_b[s];
  }
  const uint32_t per_q = uint32_t(combine ? chunks : c.n_splits);
  int gidx, rank;
  split_index(local, G, a.kv_group > 1, gidx, rank);
  uint32_t rq;
  if (!combine && a.causal == 0 && a.n_blocks == 0 && a.n_qtiles > 1) {
    // Every query sees every key, so every query tile of a group costs the
    // same: the tiles of one key split take consecutive ranks and run side by
    // side on the group's XCD, where they share the split's K/V through the L2.
    const uint32_t sp = uint32_t(rank) / uint32_t(a.n_qtiles);
    rq = uint32_t(rank) - sp * uint32_t(a.n_qtiles);
    c.split = int(sp);
  } else {
    rq = uint32_t(rank) / per_q;
    c.split = int(uint32_t(rank) - rq * per_q);
  }
  c.qtile = a.n_qtiles - 1 - int(rq);  // heaviest (latest) query tiles first
  if (a.n_seg == 0) {
    const uint32_t bq = uint32_t(gidx) / uint32_t(a.H);
    c.b = int(bq);
    c.h = gidx - int(bq) * a.H;
  } else {
    c.h = gidx;
  }
  c.pbase = seg_item_base + (int64_t(gidx) * a.n_qtiles + c.qtile) * c.n_splits;
  return c;
}

// Online-softmax state of one lane (one query; lanes l and l^32 share it).
struct Softmax {
  float m;  // max of raw scores so far: the exponent reference (possibly stale)
  float l;  // sum of exponentials (this lane's half of the keys)
};

// The phases of one key tile, for one wave (32 queries):
//   qk_tile      S^T = K Q^T (16 MFMAs for D = 128), K read from LDS;
//   softmax_max  per-key masking, row max, lazy rescale of acc;
//   softmax_exp  P = exp2(S c - ref) in place, row sum;
//   pv_tile      O^T += V^T P^T (16 MFMAs), V^T gathered by transposing reads.
// ``masked``: some key of the tile is invisible to some query of the
// workgroup (a straddling tile; workgroup-uniform). Unmasked tiles do no
// per-key visibility work.

template <int D, typename T>
__device__ __forceinline__ void qk_tile(const uint16_t* Ks, const u32x4 (&qr)[D / 16],
                                        f32x16 (&s)[2], int lane) {
  constexpr int KS = D / 16;
  constexpr int N = 2 * KS;  // MFMAs: (half kt, k-step ks) = (i / KS, i % KS)
  constexpr int W = 4;       // K fragments in flight ahead of the MFMA using them
  const int n = lane & 31, g = lane >> 5;
  const uint16_t* kp = Ks + n * Lds<D>::kPitch + 8 * g;
  auto frag = [&](int i) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4*>(kp + (i / KS) * 32 * Lds<D>::kPitch + 16 * (i % KS));
  };
  u32x4 kf[W];
#pragma unroll
  for (int i = 0; i < W; ++i) kf[i] = frag(i);
  s[0] = f32x16{};
  s[1] = f32x16{};
#pragma unroll
  for (int i = 0; i < N; ++i) {
    s[i / KS] = Mfma<T>::run(kf[i % W], qr[i % KS], s[i / KS]);
    if (i + W < N) kf[i % W] = frag(i + W);
  }
}

// Key of register r of half kt: row 32 kt + 8 (r / 4) + 4 g + r % 4 of the
// tile, visible iff that row is below lim_rel (rows past the tile's valid
// keys or past this query's visible end are not). ``lim`` is lim_rel - 4 g.
__device__ __forceinline__ bool key_hidden(int kt, int r, int lim) {
  return 32 * kt + 8 * (r / 4) + (r % 4) >= lim;
}

// Combine lanes i and i ^ 32 (v_permlane32_swap: a VALU exchange of the two
// wave halves, with no trip through the LDS queue as ds_bpermute takes).
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Returns the exponent base (max in log2 units, 0 while nothing is visible).
template <int D>
__device__ __forceinline__ float softmax_max(f32x16 (&s)[2], f32x16 (&acc)[D / 32],
                                             Softmax& sm, float c, int lim, bool masked) {
  constexpr int DT = D / 32;
  if (masked) {
    // The compare operand is fenced into this branch so that the compiler
    // does not compute the 32 compares for unmasked tiles too.
    int l = lim;
    asm volatile("" : "+v"(l));
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (key_hidden(kt, r, l)) s[kt][r] = -INFINITY;
  }
  // Row max over the visible scores (raw units; c >= 0 keeps the order), as
  // four independent chains so the dependent max latency overlaps.
  float tm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) tm[r % 4] = fmaxf(tm[r % 4], s[kt][r]);
  const float tmax = xor32_max(fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3])));
  const float m_new = fmaxf(sm.m, tmax);
  // Lazy rescale (wave-uniform branch): only when some lane's max grew by
  // more than 2^8. Before anything is accumulated (m = -inf on every lane)
  // there is nothing to scale: just take the new reference.
  const bool grow = (m_new - sm.m) * c > 8.0f;
  if (__any(grow)) {
    if (!__all(sm.m == -INFINITY)) {
      const float corr = sm.m == -INFINITY ? 0.f : fast_exp2((sm.m - m_new) * c);
      sm.l *= corr;
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d] *= corr;
    }
    sm.m = m_new;
  }
  // Nothing visible yet: exponent base 0.
  return sm.m == -INFINITY ? 0.f : sm.m * c;
}

// Masked scores are -inf and c > 0 (the host guarantees it), so their
// exponentials are exactly 0 with no further masking.
__device__ __forceinline__ void softmax_exp(f32x16 (&s)[2], Softmax& sm, float c, float mb) {
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kt][r] = fast_exp2(__builtin_fmaf(s[kt][r], c, -mb));
  float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r % 4] += s[kt][r];
  sm.l += (part[0] + part[1]) + (part[2] + part[3]);
}

// O^T += V^T P^T, 16 keys per MFMA (key step u = 2 kt + hf). The A operand
// of lane (n, g) is head_dim column 32 d + n at keys
// 16u + {4g..4g+3, 8+4g..8+4g+3}, gathered from the row-major V tile by two
// transposing reads: lane j of each 16-lane group addresses key
// 16u + 8r + 4g + j/4 (r = 0, 1) at dims 32 d + 16 ((lane/16) % 2) + 4 (j % 4).
template <int D, typename T>
__device__ __forceinline__ void pv_tile(const uint16_t* Vs, const f32x16 (&s)[2],
                                        f32x16 (&acc)[D / 32], int lane) {
  constexpr int DT = D / 32;
  const int g = lane >> 5;
  const int j = lane & 15, half = (lane >> 4) & 1;
  const uint16_t* vbase = Vs + (4 * g + (j >> 2)) * Lds<D>::vPitch + 16 * half + 4 * (j & 3);
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      u32x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pb[e] = Mfma<T>::pack(s[kt][8 * hf + 2 * e], s[kt][8 * hf + 2 * e + 1]);
      const uint16_t* vu = vbase + 16 * (2 * kt + hf) * Lds<D>::vPitch;
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const u32x2 lo = lds_read_tr16(vu + 32 * d);
        const u32x2 hi = lds_read_tr16(vu + 8 * Lds<D>::vPitch + 32 * d);
        acc[d] = Mfma<T>::run(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, acc[d]);
      }
    }
}

// The straight-line middle of a pipelined step, one basic block:
//   S_next = K_next Q^T            (HasNext; 2*KS MFMAs, K from LDS)
//   P = exp2(S c - mb), packed     (32 v_exp per lane, v_cvt_pk)
//   l += row sum of the packed P   (v_dot2 against (1, 1): 2 keys per op)
//   O^T += V^T P^T                 (16 MFMAs, V^T by transposing reads)
// Masked scores are already -inf and c > 0, so their P is exactly 0. The
// sched_group_barrier sequence at the end interleaves the QK^T MFMAs with the
// exponentials and the PV MFMAs with the packing, so one wave keeps its SIMD's
// matrix pipe busy while its vector pipe works, and runs LDS reads ahead.
namespace sg {
constexpr int kMfma = 0x008, kValu = 0x002, kDsRead = 0x100;
}

template <int D, typename T, bool HasNext>
__device__ __forceinline__ void step_body(const uint16_t* Kn, const uint16_t* Vs,
                                          const u32x4 (&qr)[D / 16], f32x16 (&cur)[2],
                                          f32x16 (&nxt)[2], f32x16 (&acc)[D / 32],
                                          Softmax& sm, float c, float mb, int lane) {
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int NQ = 2 * KS;  // QK^T MFMAs
  constexpr int W = 4;        // K fragments in flight
  const int n = lane & 31, g = lane >> 5;
  // S_next: MFMA i is (half i / KS, k-step i % KS).
  const uint16_t* kp = Kn + n * Lds<D>::kPitch + 8 * g;
  auto frag = [&](int i) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4*>(kp + (i / KS) * 32 * Lds<D>::kPitch + 16 * (i % KS));
  };
  if (HasNext) {
    u32x4 kf[W];
#pragma unroll
    for (int i = 0; i < W; ++i) kf[i] = frag(i);
    nxt[0] = f32x16{};
    nxt[1] = f32x16{};
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      nxt[i / KS] = Mfma<T>::run(kf[i % W], qr[i % KS], nxt[i / KS]);
      if (i + W < NQ) kf[i % W] = frag(i + W);
    }
  }
  // P and its row sum.
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) cur[kt][r] = fast_exp2(__builtin_fmaf(cur[kt][r], c, -mb));
  // Region 1 schedule: each QK^T MFMA followed by 4 of the 64 fma/exp ops,
  // with the K reads W MFMAs ahead. The full scheduling barrier after it
  // keeps region 2's V^T reads from being hoisted here (which would hold
  // them in registers through region 1).
  if (HasNext) {
#pragma unroll
    for (int i = 0; i < W; ++i) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 1, 0);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      __builtin_amdgcn_sched_group_barrier(sg::kMfma, 1, 0);
      if (i + W < NQ) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(sg::kValu, 4, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 pk[4];  // pk[2 kt + hf][e]: keys 8 hf + 2 e, +1 of half kt
  float part[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t p =
          Mfma<T>::pack(cur[u / 2][8 * (u % 2) + 2 * e], cur[u / 2][8 * (u % 2) + 2 * e + 1]);
      pk[u][e] = p;
      part[e & 1] = Mfma<T>::sum2(p, part[e & 1]);
    }
  sm.l += part[0] + part[1];
  // O^T += V^T P^T (see pv_tile for the operand layout).
  const int j = lane & 15, half = (lane >> 4) & 1;
  const uint16_t* vbase = Vs + (4 * g + (j >> 2)) * Lds<D>::vPitch + 16 * half + 4 * (j & 3);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint16_t* vu = vbase + 16 * u * Lds<D>::vPitch;
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const u32x2 lo = lds_read_tr16(vu + 32 * d);
      const u32x2 hi = lds_read_tr16(vu + 8 * Lds<D>::vPitch + 32 * d);
      acc[d] = Mfma<T>::run(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[u], acc[d]);
    }
  }
  // Region 2 schedule: the V^T reads two MFMAs ahead of the PV MFMAs, with
  // the packing and sums spread between them.
#pragma unroll
  for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 1, 0);
  __builtin_amdgcn_sched_group_barrier(sg::kValu, 8, 0);
#pragma unroll
  for (int i = 0; i < 4 * DT; ++i) {
    __builtin_amdgcn_sched_group_barrier(sg::kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 2, 0);
    __builtin_amdgcn_sched_group_barrier(sg::kValu, 2, 0);
  }
}

// One whole key tile (the dual-stream decode path).
template <int D, typename T>
__device__ __forceinline__ void tile_step(const uint16_t* Ks, const uint16_t* Vs,
                                          const u32x4 (&qr)[D / 16], f32x16 (&acc)[D / 32],
                                          Softmax& sm, float c, int lim, bool masked,
                                          int lane) {
  f32x16 s[2];
  qk_tile<D, T>(Ks, qr, s, lane);
  const float mb = softmax_max<D>(s, acc, sm, c, lim, masked);
  softmax_exp(s, sm, c, mb);
  pv_tile<D, T>(Vs, s, acc, lane);
}

// Split-KV partial of one row: its normalised output o = acc / l is kept as
// f16 values o 2^-e, where 2^e is above the row's largest |o| (so every
// stored value is below 1 in magnitude: no f16 overflow for any finite input,
// 11 significant bits relative to the row's largest element), plus the fp32
// record {exponent reference m, sum l, e, 0}. The merge re-weights each split
// by exp2(m_s - max m) l_s and restores 2^e_s exactly.
struct PartialScale {
  float k;  // multiplier taking acc to the stored f16 values: 2^-e / l
  int e;
};
template <int D>
__device__ __forceinline__ PartialScale partial_scale(const f32x16 (&acc)[D / 32], float l_tot) {
  constexpr int DT = D / 32;
  float amax = 0.f;
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) amax = fmaxf(amax, fabsf(acc[d][r]));
  amax = xor32_max(amax);  // the row's other half of head_dim (lanes l and l ^ 32)
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const float omax = amax * inv;
  // frexp exponent: omax = f 2^e with f in [0.5, 1); 0 for a zero or
  // non-finite row (whose values then pass through unscaled).
  const int e = omax > 0.f && omax <= FLT_MAX ? __builtin_amdgcn_frexp_expf(omax) : 0;
  return {__builtin_ldexpf(inv, -e), e};
}

// A lane's result for its query qi (row ``row`` of the work item's BM
// queries): the output, or with split-KV the scaled f16 partial and its fp32
// record (partial_scale). No visible key: partial o = 0, reference -inf;
// final output NaN (0 * inf), as the reference.
template <int D, typename T>
__device__ __forceinline__ void store_result(const AttnArgs& a, const Coord& it, int bm, int row,
                                             int qi, int g, const f32x16 (&acc)[D / 32],
                                             float l_tot, float mref) {
  constexpr int DT = D / 32;
  if (it.n_splits == 1) {
    const float inv = 1.0f / l_tot;
    uint16_t* op = a.out + it.b * a.o_sb + int64_t(qi) * a.o_sl + it.h * a.o_sh;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4 + 4 * g;
        u32x2 w;
        w[0] = Mfma<T>::pack(acc[d][4 * r4] * inv, acc[d][4 * r4 + 1] * inv);
        w[1] = Mfma<T>::pack(acc[d][4 * r4 + 2] * inv, acc[d][4 * r4 + 3] * inv);
        *reinterpret_cast<u32x2*>(op + dim) = w;
      }
  } else {
    const int64_t pidx = it.pbase + it.split;
    const PartialScale ps = partial_scale<D>(acc, l_tot);
    uint16_t* po = a.ws_o + (pidx * bm + row) * D;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4 + 4 * g;
        u32x2 w;
        w[0] = Mfma<f16_t>::pack(acc[d][4 * r4] * ps.k, acc[d][4 * r4 + 1] * ps.k);
        w[1] = Mfma<f16_t>::pack(acc[d][4 * r4 + 2] * ps.k, acc[d][4 * r4 + 3] * ps.k);
        *reinterpret_cast<u32x2*>(po + dim) = w;
      }
    if (g == 0)
      *reinterpret_cast<f32x4*>(a.ws_ml + (pidx * bm + row) * 4) =
          f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(ps.e), 0.f};
  }
}

// Merge of n split-KV partials of one row (records ml, stored values o, one
// 16-byte record and 4 f16 values per split) into 4 output values:
//   out = sum_s c_s o_s 2^e_s,  c_s = exp2(m_s - M) l_s / L,  L = sum_s exp2(m_s - M) l_s
// with M the largest m_s. The sum runs relative to E, the largest e_s, and
// 2^E is applied once at the end: every coefficient c_s 2^(e_s - E) is <= 1,
// so no intermediate overflows, and |out| <= max |v| as in the reference. No
// visible key in any split: L = 0 and the output is NaN, as the reference.
//
// The row's split weights c_s 2^(e_s - E) into c (0 for s >= n), returning E.
// Splits s >= n hold zeros (loads past the buffer bound) and are masked by
// selects, not branches, so every load is issued before any is used.
template <int NMAX>
__device__ __forceinline__ int merge_weights(const f32x4 (&ml)[NMAX], int n, float (&c)[NMAX]) {
  // No fused multiply-adds: the merge kernel and the in-launch merges inline
  // this into different code and must round alike.
#pragma clang fp contract(off)
  float mmax = -INFINITY;
  int emax = INT_MIN;
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    mmax = s < n ? fmaxf(mmax, ml[s][0]) : mmax;
    emax = s < n ? max(emax, int(ml[s][2])) : emax;
  }
  const float base = mmax == -INFINITY ? 0.f : mmax;
  float w[NMAX];
  float L = 0.f;
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    w[s] = s < n ? fast_exp2(ml[s][0] - base) * ml[s][1] : 0.f;
    L += w[s];
  }
  const float invL = 1.0f / L;
#pragma unroll
  for (int s = 0; s < NMAX; ++s)
    c[s] = s < n ? __builtin_ldexpf(w[s] * invL, int(ml[s][2]) - emax) : 0.f;
  return emax;
}

// One split's term for two values: a += c o (o two packed f16). Every merge
// adds the splits' terms in split order, so the separate merge kernel and the
// prefill kernel's own merge round alike.
__device__ __forceinline__ void merge_add2(float& a0, float& a1, float c, uint32_t o) {
  a0 = __builtin_fmaf(c, to_f32(f16_t{uint16_t(o & 0xffffu)}), a0);
  a1 = __builtin_fmaf(c, to_f32(f16_t{uint16_t(o >> 16)}), a1);
}

template <int NMAX>
__device__ __forceinline__ f32x4 merge_partials(const f32x4 (&ml)[NMAX], const u32x2 (&o)[NMAX],
                                                int n) {
  float c[NMAX];
  const int emax = merge_weights(ml, n, c);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    merge_add2(acc[0], acc[1], c[s], o[s][0]);
    merge_add2(acc[2], acc[3], c[s], o[s][1]);
  }
  return f32x4{__builtin_ldexpf(acc[0], emax), __builtin_ldexpf(acc[1], emax),
               __builtin_ldexpf(acc[2], emax), __builtin_ldexpf(acc[3], emax)};
}

// store_result for a whole wave (32 rows, r0 .. r0 + 31 of the work item's
// bm), through a row area of the LDS that no other wave is using: each lane
// packs its row there, then the wave stores whole-row chunks (RowArea).
// Rows at or past Lq are not written. Every lane of the wave must call it.
// kAux: cache policy of the partial stores of a split work item (0, or
// kScDevice for a merge by another workgroup of the group in the same launch).
template <int D, typename T, int kAux = 0>
__device__ __forceinline__ void store_result_staged(const AttnArgs& a, const Coord& it, int bm,
                                                    int q0, int r0, int g, int lane,
                                                    const f32x16 (&acc)[D / 32], float l_tot,
                                                    float mref, uint32_t area) {
  // Every product below is rounded to fp32 before its conversion: a multiply
  // fused into the conversion (one rounding) would round differently, and
  // inlined copies of this function must agree bit for bit.
#pragma clang fp contract(off)
  constexpr int DT = D / 32;
  using A = RowArea<D>;
  const int row = r0 + (lane & 31);
  const int nrows = min(a.Lq - q0 - r0, 32);
  uint32_t w[DT][4][2];
  __amdgpu_buffer_rsrc_t ro;
  int ro_bytes;
  if (it.n_splits == 1) {
    const float inv = 1.0f / l_tot;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        w[d][r4][0] = Mfma<T>::pack(acc[d][4 * r4] * inv, acc[d][4 * r4 + 1] * inv);
        w[d][r4][1] = Mfma<T>::pack(acc[d][4 * r4 + 2] * inv, acc[d][4 * r4 + 3] * inv);
      }
    ro_bytes = int(a.o_sl) * 2;
    ro = make_rsrc(a.out + it.b * a.o_sb + int64_t(q0 + r0) * a.o_sl + it.h * a.o_sh,
                   max(nrows, 0), ro_bytes, D);
  } else {
    const int64_t pidx = it.pbase + it.split;
    const PartialScale ps = partial_scale<D>(acc, l_tot);
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        w[d][r4][0] = Mfma<f16_t>::pack(acc[d][4 * r4] * ps.k, acc[d][4 * r4 + 1] * ps.k);
        w[d][r4][1] = Mfma<f16_t>::pack(acc[d][4 * r4 + 2] * ps.k, acc[d][4 * r4 + 3] * ps.k);
      }
    if (row - r0 < nrows && g == 0)
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(ps.e), 0.f}),
          __builtin_amdgcn_make_buffer_rsrc(a.ws_ml + pidx * bm * 4, (short)0, bm * 16, kBufWord3),
          row * 16, 0, kAux);
    ro_bytes = D * 2;
    ro = make_rsrc(a.ws_o + (pidx * bm + r0) * D, max(nrows, 0), ro_bytes, D);
  }
  // Dims 32 d + 8 r4 + 4 g .. + 3 of row ``row``: half g of chunk 4 d + r4.
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
      *reinterpret_cast<lds_u32x2*>(A::at(area, row, 4 * d + r4) + 8 * g) =
          u32x2{w[d][r4][0], w[d][r4][1]};
    }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's rows are in LDS
  A::template store_rows<kAux>(ro, ro_bytes, nrows, area, r0, lane);
}

// Key splits of a work-item group merged in the kernel itself (paired and
// dual-stream kernels), with no merge launch: every split stores its partial
// at device scope (kScDevice), waits until the stores have completed and
// arrives on the group's 64-bit counter (the arrival count in the low word, the arrivals from
// XCD x in the nibble at bit 32 + 4 x); the split that brings the count to
// n_splits resets the counter and merges all the group's partials into the
// output, and the others are done. No workgroup ever waits for another, so
// the order and placement in which the splits run do not matter. When every
// split ran on the merging workgroup's XCD, the partials are read from that
// XCD's L2 (kScXcd), else from memory (kScDevice). Groups of more than
// kPMergeSplits splits take the separate merge kernel instead.
constexpr int kPMergeSplits = 8;
// Cache policy of loads of data that workgroups of this XCD stored (sc0):
// past this CU's L1 to the XCD's L2, which holds every such store.
constexpr int kScXcd = 1;

// Where a partial keeps its 16-byte unit (row r, chunk ch of 8 head-dim
// values), in bytes from the partial's start. Row-major: (r CR + ch) 16, CR =
// D / 8. Blocked (BLK): ((r / 32) CR + ch) 512 + (r % 32) 16, the layout of a
// wave's MFMA registers, in which the dual-stream kernel stores a partial
// that the merge kernel will read: a wave stores each (32-row block, chunk)
// piece as 512 contiguous bytes straight from its registers.
template <int D, bool BLK>
__device__ __forceinline__ uint32_t unit_off(int r, int ch) {
  constexpr uint32_t CR = D / 8;
  return BLK ? ((uint32_t(r) >> 5) * CR + uint32_t(ch)) * 512u + (uint32_t(r) & 31u) * 16u
             : (uint32_t(r) * CR + uint32_t(ch)) * 16u;
}

// The merge, by the last split: thread t < nrows turns row t's records into
// the split weights (into LDS) while every thread's loads of its units (row,
// 8 dims: 16 bytes) of the first splits are in flight; then each thread adds
// the splits' terms in split order, SB splits per batch of loads, with the
// merge kernel's arithmetic (merge_weights, merge_add2). BM: rows per work
// item; NT: threads of the workgroup; SB: splits per batch of loads (UPT SB
// 16-byte values per thread in flight); kAux: cache policy of the loads.
template <int D, typename T, int BM, int NT, int SB, int kAux>
__device__ __forceinline__ void merge_split_group(const AttnArgs& a, const Coord& it, int q0,
                                                  int nrows, uint16_t* smem) {
  constexpr int CR = D / 8;          // 16-byte units per row
  constexpr int UPT = BM * CR / NT;  // units per thread
  static_assert(BM * CR % NT == 0 && BM <= NT, "units deal evenly; a thread per row");
  static_assert(kPMergeSplits % SB == 0, "whole batches");
  const int t = int(threadIdx.x);
  const int S = it.n_splits;
  const uint32_t rows = uint32_t(a.bm);
  // Bounded by the group's S partials: loads of splits s >= S return zeros.
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + it.pbase * a.bm * 4, (short)0, int(uint32_t(S) * rows * 16), kBufWord3);
  const __amdgpu_buffer_rsrc_t rval = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + it.pbase * a.bm * D, (short)0, int(uint32_t(S) * rows * D * 2), kBufWord3);
  float* const lc = reinterpret_cast<float*>(smem);                   // [row][kPMergeSplits]
  int* const le = reinterpret_cast<int*>(lc + BM * kPMergeSplits);  // [row] exponent E

  f32x4 ml[kPMergeSplits];
  {
    const uint32_t base = t < nrows ? uint32_t(t) * 16 : 0x80000000u;  // past every bound
#pragma unroll
    for (int s = 0; s < kPMergeSplits; ++s)
      ml[s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rrec, base + uint32_t(s) * rows * 16, 0, kAux));
  }
  u32x4 v[UPT][SB];
  auto load_batch = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      const int u = t + NT * k, r = u / CR, ch = u % CR;
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const uint32_t off = r < nrows ? (uint32_t(s0 + j) * rows + uint32_t(r)) * (D * 2) +
                                             uint32_t(ch) * 16
                                       : 0x80000000u;  // past every bound: zeros
        v[k][j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rval, off, 0, kAux));
      }
    }
  };
  load_batch(0);
  {
    float c[kPMergeSplits];
    const int emax = merge_weights(ml, S, c);
    if (t < nrows) {
#pragma unroll
      for (int s = 0; s < kPMergeSplits; ++s) lc[t * kPMergeSplits + s] = c[s];
      le[t] = emax;
    }
  }
  __syncthreads();
  float acc[UPT][8];
#pragma unroll
  for (int k = 0; k < UPT; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
  for (int s0 = 0; s0 < S; s0 += SB) {
    if (s0 > 0) load_batch(s0);
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      const int r = (t + NT * k) / CR;
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const float cs = lc[r * kPMergeSplits + s0 + j];
#pragma unroll
        for (int e = 0; e < 4; ++e) merge_add2(acc[k][2 * e], acc[k][2 * e + 1], cs, v[k][j][e]);
      }
    }
  }
  DX_STAMP(6);
#pragma unroll
  for (int k = 0; k < UPT; ++k) {
    const int u = t + NT * k, r = u / CR, ch = u % CR;
    if (r < nrows) {
      const int emax = le[r];
      u32x4 packed;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        packed[e] = Mfma<T>::pack(__builtin_ldexpf(acc[k][2 * e], emax),
                                  __builtin_ldexpf(acc[k][2 * e + 1], emax));
      uint16_t* op = a.out + it.b * a.o_sb + int64_t(q0 + r) * a.o_sl + it.h * a.o_sh + ch * 8;
      *reinterpret_cast<u32x4*>(op) = packed;
    }
  }
}

// Arrival of a split work item whose partial rows are being stored with
// kScDevice (merge_split_group): every wave of the workgroup calls it, once
// its own stores are issued. Uses the first BM (kPMergeSplits + 1) + 1 words
// of the LDS, which must be idle.
template <int D, typename T, int BM, int NT, int SB>
__device__ __forceinline__ void arrive_split_group(const AttnArgs& a, const Coord& it, int q0,
                                                   uint16_t* smem) {
  static_assert(kPMergeSplits < 16, "an XCD's arrivals fit its nibble");
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed at device scope
  __syncthreads();
  int* const last = reinterpret_cast<int*>(smem) + BM * (kPMergeSplits + 1);  // past the weights
  if (threadIdx.x == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
    uint64_t* const cnt = reinterpret_cast<uint64_t*>(a.counters + it.pbase * kCounterStride);
    const uint64_t mine = 1ull | (1ull << (32 + 4 * xcc));
    const uint64_t v =
        __hip_atomic_fetch_add(cnt, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    const uint64_t n = uint64_t(it.n_splits);
    int state = 0;  // 0: not the last; 1: the last, every split on this XCD; 2: the last
    if ((v & 0xffffffffull) == n) {
      state = (v >> 32) == (n << (4 * xcc)) ? 1 : 2;
      __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *last = state;
  }
  __syncthreads();
  const int state = *last;
  DX_STAMP(5);
  DX_NOTE(8, uint32_t(it.split) | uint32_t(it.n_splits) << 8 | uint32_t(it.b) << 16 |
                 uint64_t(state) << 32);
  DX_STAMP(7);  // the merging split writes it again when done
  if (state == 0) return;
  const int nrows = min(BM, a.Lq - q0);
  if (state == 1) merge_split_group<D, T, BM, NT, SB, kScXcd>(a, it, q0, nrows, smem);
  else merge_split_group<D, T, BM, NT, SB, kScDevice>(a, it, q0, nrows, smem);
  DX_STAMP(7);
}

// Rows [r_lo, r_lo + rn) of a split group's output, merged from the
// row-major partials of the paired and dual-stream kernels (rn <= BM / 2: a
// chunk of a group of at least two splits), with the merge kernel's
// arithmetic in its order (merge_weights, merge_add2 in split order; splits
// past the group's read as zeros and weigh 0). Thread t < rn turns row t's
// records into the split weights (into LDS) while every thread's value loads
// are in flight: thread t takes units (row, 8 dims: 16 bytes) t + NT k, so
// consecutive threads read consecutive 16 bytes of a row. kAux: cache policy
// of the loads (kScXcd: from this XCD's L2; kScDevice: from memory).
template <int D, typename T, int BM, int NT, int kAux>
__device__ __forceinline__ void merge_rows(const AttnArgs& a, const Coord& it, int q0, int r_lo,
                                           int rn, uint16_t* smem) {
  constexpr int CR = D / 8;
  constexpr int UPT = (BM / 2 * CR + NT - 1) / NT;  // units per thread, at most
  const int S = it.n_splits;
  const uint32_t rows = uint32_t(a.bm);
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + it.pbase * a.bm * 4, (short)0, int(uint32_t(S) * rows * 16), kBufWord3);
  const __amdgpu_buffer_rsrc_t rval = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + it.pbase * a.bm * D, (short)0, int(uint32_t(S) * rows * D * 2), kBufWord3);
  float* const lc = reinterpret_cast<float*>(smem);                        // [row][split]
  int* const le = reinterpret_cast<int*>(lc + BM / 2 * kPMergeSplits);  // [row] exponent E
  const int t = int(threadIdx.x), nu = rn * CR;
  u32x4 v[UPT][kPMergeSplits];
#pragma unroll
  for (int k = 0; k < UPT; ++k) {
    const int u = t + NT * k;
    // Units past the chunk read past every bound (zeros, unused).
    const uint32_t base = u < nu ? uint32_t(r_lo + u / CR) * (D * 2) + uint32_t(u % CR) * 16
                                 : 0x80000000u;
#pragma unroll
    for (int sp = 0; sp < kPMergeSplits; ++sp)
      v[k][sp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rval, base + uint32_t(sp) * rows * (D * 2), 0, kAux));
  }
  if (t < rn) {
    f32x4 ml[kPMergeSplits];
#pragma unroll
    for (int sp = 0; sp < kPMergeSplits; ++sp)
      ml[sp] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rrec, (uint32_t(sp) * rows + uint32_t(r_lo + t)) * 16,
                                             0, kAux));
    float c[kPMergeSplits];
    const int emax = merge_weights(ml, S, c);
#pragma unroll
    for (int sp = 0; sp < kPMergeSplits; ++sp) lc[t * kPMergeSplits + sp] = c[sp];
    le[t] = emax;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < UPT; ++k) {
    const int u = t + NT * k;
    if (u >= nu) continue;
    const int r = u / CR, ch = u % CR;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < kPMergeSplits; ++sp) {
      const float cs = lc[r * kPMergeSplits + sp];
#pragma unroll
      for (int e = 0; e < 4; ++e) merge_add2(acc[2 * e], acc[2 * e + 1], cs, v[k][sp][e]);
    }
    const int emax = le[r];
    u32x4 packed;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      packed[e] = Mfma<T>::pack(__builtin_ldexpf(acc[2 * e], emax),
                                __builtin_ldexpf(acc[2 * e + 1], emax));
    uint16_t* op =
        a.out + it.b * a.o_sb + int64_t(q0 + r_lo + r) * a.o_sl + it.h * a.o_sh + ch * 8;
    __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(op));
  }
  DX_STAMP(6);
}

// Wait of a split for the other splits of its group before a spread merge:
// s_memrealtime ticks (100 MHz), 20 us, ample for co-resident workgroups;
// reached only when a split cannot be scheduled until others leave.
constexpr uint32_t kSpreadTicks = 2000;
// Slow path's poll limit (50 us), as kSpinTicks of the decode kernel.
constexpr uint64_t kSpreadSpinTicks = 5000;

// Spread merge of a split group in the same launch (dual-stream kernel):
// every split stores its partial with plain stores (into its XCD's L2),
// arrives, and once all S splits have arrived merges row chunk c = its split
// index (rows [c nrows / S, (c + 1) nrows / S)) of every split's partial, so
// the group's merge is shared by its S workgroups instead of read by one.
//
// Arrival (thread 0). Group word w (64-bit, counters[0..1]) counts arrivals
// in bits [0, 16), marks from bit 16, and the arrivals from XCC x in the
// nibble at bit 32 + 4 x; counters[2] counts finished workgroups. Atomics
// are coherent across the device; plain stores reach only the issuing XCD's
// L2. A workgroup that sees all S arrivals and no mark, every one from its
// own XCC, merges its chunk with loads from that L2 (kScXcd: the fast path).
// One that does not see S arrivals within kSpreadTicks marks the word, by
// compare-and-swap and only while arrivals < S; then, or when the arrivals
// came from several XCCs, every workgroup of the group takes the slow path
// (the word decides it for all alike):
//
// Slow path, at device scope: every split stores its partial again through
// to memory (``restore``), then counters[4] counts arrivals, counters[5]
// finishes and counters[6 + c] claims chunk c. A workgroup that is not the
// last arrival polls until all have arrived, with a time limit; a chunk is
// merged by whoever claims it first (compare-and-swap): its owner once all
// have arrived, or the last arrival, which after its own chunk claims every
// chunk still unclaimed. Every chunk is merged exactly once.
//
// The S-th workgroup to finish with each state resets it to zero, so the
// counters are zero after every call. Every thread of the workgroup calls
// it, after its own partial stores are issued; the LDS below ``sh_words``
// (ints from smem) must be idle.
template <int D, typename T, int BM, int NT, typename Restore>
__device__ __forceinline__ void spread_split_group(const AttnArgs& a, const Coord& it, int q0,
                                                   uint16_t* smem, Restore&& restore) {
  static_assert(kPMergeSplits < 16, "an XCD's arrivals fit its nibble");
  static_assert(6 + kPMergeSplits <= kCounterStride, "group state fits its slot");
  constexpr int kShWords = BM / 2 * (kPMergeSplits + 1);  // past merge_rows' scratch
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are in the L2
  __syncthreads();
  const int S = it.n_splits;
  int32_t* const fs = a.counters + it.pbase * kCounterStride;
  uint64_t* const fw = reinterpret_cast<uint64_t*>(fs);
  int32_t* const gs = fs + 4;
  int* const sh = reinterpret_cast<int*>(smem) + kShWords;
  constexpr uint64_t kMark = 1ull << 16;
  if (threadIdx.x == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
    const uint64_t mine = 1ull | (1ull << (32 + 4 * xcc));
    const uint64_t alone = uint64_t(S) << (32 + 4 * xcc);  // all S arrivals from this XCC
    int fast = -1;
    uint64_t v = __hip_atomic_fetch_add(fw, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    DX_NOTE(11, t0);  // own arrival counted
    while (fast < 0) {
      const uint64_t arrived = v & (kMark - 1), marks = (v >> 16) & 0xffffull;
      if (marks != 0) {
        fast = 0;
      } else if (arrived == uint64_t(S)) {
        fast = (v >> 32) == (alone >> 32) ? 1 : 0;
      } else if (__builtin_amdgcn_s_memrealtime() - t0 > kSpreadTicks) {
        uint64_t expect = v;
        if (__hip_atomic_compare_exchange_strong(fw, &expect, v + kMark, __ATOMIC_RELAXED,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          fast = 0;
        else
          v = expect;  // changed meanwhile: decide on the new value
      } else {
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_fetch_add(fw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    sh[0] = fast;
  }
  __syncthreads();
  DX_STAMP(5);
  DX_NOTE(8, uint32_t(it.split) | uint32_t(it.n_splits) << 8 | uint32_t(it.b) << 16 |
                 uint64_t(sh[0] ? 3 : 4) << 32);
  const bool fast = sh[0] != 0;
  const int nrows = min(BM, a.Lq - q0);
  auto chunk = [&](int c, auto aux) __attribute__((always_inline)) {
    const int r_lo = c * nrows / S;
    merge_rows<D, T, BM, NT, decltype(aux)::value>(a, it, q0, r_lo, (c + 1) * nrows / S - r_lo,
                                                   smem);
  };
  if (fast) {
    chunk(it.split, std::integral_constant<int, kScXcd>{});
  } else {
    restore();  // the partial again, through to memory
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = __hip_atomic_fetch_add(gs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == S - 1;
      int all = last;
      if (!last) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
          if (__hip_atomic_fetch_add(gs, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= S) {
            all = 1;
            break;
          }
          if (__builtin_amdgcn_s_memrealtime() - t0 > kSpreadSpinTicks) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      sh[1] = all;
      sh[2] = last;
    }
    __syncthreads();
    const bool all = sh[1] != 0, last = sh[2] != 0;
    for (int c0 = 0; all && c0 < (last ? S : 1); ++c0) {
      const int c = it.split + c0 < S ? it.split + c0 : it.split + c0 - S;  // own chunk first
      __syncthreads();  // the previous chunk's LDS scratch and sh[3] have been read
      if (threadIdx.x == 0) {
        int unclaimed = 0;
        sh[3] = __hip_atomic_compare_exchange_strong(gs + 2 + c, &unclaimed, 1, __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!sh[3]) continue;
      chunk(c, std::integral_constant<int, kScDevice>{});
    }
    if (threadIdx.x == 0) {
      // Done with the slow state; the last to get here resets it.
      if (__hip_atomic_fetch_add(gs + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1) {
        for (int i = 0; i < 2 + S; ++i)
          __hip_atomic_store(gs + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (threadIdx.x == 0) {
    // Done with the arrival state; the S-th to finish resets it.
    if (__hip_atomic_fetch_add(fs + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1) {
      __hip_atomic_store(fw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(fs + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  DX_STAMP(7);
}

// The dual-stream kernel's results after its split hand-over: stream s holds
// head_dim blocks [s DT / 2, (s + 1) DT / 2) of its wave's 32 rows (r0 ..)
// and the whole row's (l_tot, mref). Both streams pack their blocks into the
// row area at ``area``; after a workgroup barrier each stores 16 of the 32
// rows, whole (row-major). A split partial takes one scale exponent per row
// (as partial_scale's), from ``rbound``: an upper bound of the row's largest
// |value| over both streams' blocks that the hand-over already carried, so no
// exchange of the combined maxima is needed. BLOCKED: a split partial goes
// out blocked (unit_off) from the registers instead, with no row area and no
// barrier (the merge kernel reads that layout; the in-launch merges read
// row-major partials). Every wave of the workgroup calls it (the barrier, in
// a call that takes it); ``active``: the wave has rows below Lq.
// The stream is a template parameter so that every block index is a constant
// (a register array indexed at run time would live in scratch memory).
template <int D, typename T, int stream, int kAux = 0, bool BLOCKED = false>
__device__ __forceinline__ int store_result_halves(const AttnArgs& a, const Coord& it, int q0,
                                                    int r0, int g, int lane, int ltid,
                                                    bool active,
                                                    const f32x16 (&acc)[D / 32], float l_tot,
                                                    float mref, uint32_t area, float rbound) {
  // As in store_result_staged: each product rounded to fp32, then converted.
#pragma clang fp contract(off)
  constexpr int DT = D / 32, HB = DT / 2;
  constexpr int d0 = stream * HB;
  using A = RowArea<D>;
  const int row = r0 + (lane & 31);
  const int nrows = min(a.Lq - q0 - r0, 32);
  float k;
  int e = 0;
  if (it.n_splits == 1) {
    k = 1.0f / l_tot;
  } else {
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    const float omax = rbound * inv;
    e = omax > 0.f && omax <= FLT_MAX ? __builtin_amdgcn_frexp_expf(omax) : 0;
    k = __builtin_ldexpf(inv, -e);
    if (BLOCKED) {
      // Blocked (unit_off), straight from the registers: for each (block d,
      // r4), lane n + 32 g holds dims 32 d + 8 r4 + 4 g .. + 3 of row r0 + n,
      // so the wave's 64 lanes store the piece's 512 bytes in one instruction
      // (rows at or past Lq go past the buffer's bound: not written). No
      // staging, no barrier.
      if (!active) return e;
      const int64_t pidx = it.pbase + it.split;
      const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
          a.ws_o + pidx * a.bm * D, (short)0, a.bm * D * 2, kBufWord3);
      const int n = lane & 31;
#pragma unroll
      for (int dd = 0; dd < HB; ++dd)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d = d0 + dd;
          u32x2 w;
          w[0] = Mfma<f16_t>::pack(acc[d][4 * r4] * k, acc[d][4 * r4 + 1] * k);
          w[1] = Mfma<f16_t>::pack(acc[d][4 * r4 + 2] * k, acc[d][4 * r4 + 3] * k);
          const uint32_t off =
              n < nrows ? unit_off<D, true>(row, 4 * d + r4) + 8u * uint32_t(g) : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b64(w, rp, off, 0, kAux);
        }
      if (stream == 0 && g == 0 && n < nrows)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(e), 0.f}),
            __builtin_amdgcn_make_buffer_rsrc(a.ws_ml + pidx * a.bm * 4, (short)0, a.bm * 16,
                                              kBufWord3),
            row * 16, 0, kAux);
      return e;
    }
  }
  if (active) {
    // Dims 32 d + 8 r4 + 4 g .. + 3 of row ``row``: half g of chunk 4 d + r4.
#pragma unroll
    for (int dd = 0; dd < HB; ++dd)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = d0 + dd;
        u32x2 w;
        if (it.n_splits == 1) {
          w[0] = Mfma<T>::pack(acc[d][4 * r4] * k, acc[d][4 * r4 + 1] * k);
          w[1] = Mfma<T>::pack(acc[d][4 * r4 + 2] * k, acc[d][4 * r4 + 3] * k);
        } else {
          w[0] = Mfma<f16_t>::pack(acc[d][4 * r4] * k, acc[d][4 * r4 + 1] * k);
          w[1] = Mfma<f16_t>::pack(acc[d][4 * r4 + 2] * k, acc[d][4 * r4 + 3] * k);
        }
        typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
        *reinterpret_cast<lds_u32x2*>(A::at(area, row, 4 * d + r4) + 8 * g) = w;
      }
    if (it.n_splits > 1 && stream == 0 && g == 0 && row - r0 < nrows) {
      const int64_t pidx = it.pbase + it.split;
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(e), 0.f}),
          __builtin_amdgcn_make_buffer_rsrc(a.ws_ml + pidx * a.bm * 4, (short)0, a.bm * 16,
                                            kBufWord3),
          row * 16, 0, kAux);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's blocks are in LDS
  __syncthreads();                     // both streams' blocks of every row
  if (!active) return e;
  const int rs = r0 + 16 * stream;     // this stream stores rows rs .. rs + 15
  const int nr = min(nrows - 16 * stream, 16);
  __amdgpu_buffer_rsrc_t ro;
  int ro_bytes;
  if (it.n_splits == 1) {
    ro_bytes = int(a.o_sl) * 2;
    ro = make_rsrc(a.out + it.b * a.o_sb + int64_t(q0 + rs) * a.o_sl + it.h * a.o_sh,
                   max(nr, 0), ro_bytes, D);
  } else {
    ro_bytes = D * 2;
    ro = make_rsrc(a.ws_o + ((it.pbase + it.split) * a.bm + rs) * D, max(nr, 0), ro_bytes, D);
  }
  A::template store_rows<kAux, 16>(ro, ro_bytes, nr, area, rs, lane);
  return e;
}

// The partial that store_result_halves stored (a split work item), stored
// again through to memory (kScDevice): the rows from the row area, which
// still holds them, and the records from the values it was given.
template <int D, int stream>
__device__ __forceinline__ void restore_partial_halves(const AttnArgs& a, const Coord& it, int q0,
                                                       int r0, int g, int lane, bool active,
                                                       float l_tot, float mref, int e,
                                                       uint32_t area) {
  if (!active) return;
  const int row = r0 + (lane & 31);
  const int nrows = min(a.Lq - q0 - r0, 32);
  const int64_t pidx = it.pbase + it.split;
  if (stream == 0 && g == 0 && row - r0 < nrows)
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(u32x4, f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(e), 0.f}),
        __builtin_amdgcn_make_buffer_rsrc(a.ws_ml + pidx * a.bm * 4, (short)0, a.bm * 16,
                                          kBufWord3),
        row * 16, 0, kScDevice);
  const int rs = r0 + 16 * stream;
  const int nr = min(nrows - 16 * stream, 16);
  RowArea<D>::template store_rows<kScDevice, 16>(
      make_rsrc(a.ws_o + (pidx * a.bm + rs) * D, max(nr, 0), D * 2, D), D * 2, nr, area, rs,
      lane);
}

template <int D, typename T, int NS>
__global__ __launch_bounds__(64 * kNW * NS, 2) void attn_fwd_kernel(AttnArgs a) {
  constexpr int KS = D / 16;  // MFMA k-steps over head_dim
  constexpr int DT = D / 32;  // 32-wide head_dim tiles of the output
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  prefetch_args(a);

  const Coord it = locate(a, blockIdx.x, false, 0);
  DX_STAMP(0);
  const int b = it.b, h = it.h;
  // NS streams of four waves; stream s takes every NS-th tile of the range.
  // Wave and stream indices are read through readfirstlane so the compiler
  // treats them as wave-uniform: branches on them become scalar branches
  // instead of exec-masked regions (which would serialise the loads issued
  // on either side).
  const int wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int stream = NS == 1 ? 0 : wid / kNW;
  const int wave = wid - stream * kNW, lane = int(threadIdx.x) & 63;
  const int ltid = wave * 64 + lane;
  const int g = lane >> 5, n = lane & 31;
  const int q0 = it.qtile * kBM;
  const int qi = q0 + wave * 32 + n;
  const bool qvalid = qi < a.Lq;
  const bool wave_active = q0 + wave * 32 < a.Lq;
  const int cache_len = it.cache_len;

  // Key range of the workgroup: end_bounds over its first and last queries.
  // Workgroup-uniform (scalar) work, no barrier. The
  // dual-stream (decode) path tiles the largest range any query of the chunk
  // can see (the whole cache and all Lq new keys) so that its tile loads go
  // out before the block starts are read; it skips the tiles past the
  // visible range and masks the straddling ones per key.
  int kv_min = 0, kv_max = cache_len + a.Lk;
  if (NS == 1) {
    const EndBounds eb = end_bounds(a, q0, min(q0 + kBM, a.Lq) - 1);
    kv_min = cache_len + eb.lo;
    kv_max = cache_len + eb.hi;
  }

  const int n_ct = (cache_len + kBN - 1) / kBN;
  const int n_tiles = n_ct + (kv_max - cache_len + kBN - 1) / kBN;
  // 32-bit unsigned: splits <= 16 and tiles < 2^26 (keys < 2^30), so the
  // products fit, and the division is far shorter than a 64-bit one.
  const int t_begin = int(uint32_t(it.split) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int t_end = int(uint32_t(it.split + 1) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int iters = (t_end - t_begin + NS - 1) / NS;  // barrier rounds, equal for all streams

  KvSrc src;
  src.c_ss2 = int(a.c_ss) * 2;
  src.k_sl2 = int(a.k_sl) * 2;
  src.v_sl2 = int(a.v_sl) * 2;
  src.n_ct = n_ct;
  {
    const int rows_c = min(cache_len, kv_max), rows_n = kv_max - cache_len;
    const int hk = a.kv_group == 1 ? h : h / a.kv_group;  // K/V head of this query head
    const int64_t coff = b * a.c_sb + hk * a.c_sh;
    src.kc = make_rsrc(a.ck ? a.ck + coff : a.q, rows_c, src.c_ss2, D);
    src.vc = make_rsrc(a.cv ? a.cv + coff : a.q, rows_c, src.c_ss2, D);
    src.kn = make_rsrc(a.k + b * a.k_sb + hk * a.k_sh, rows_n, src.k_sl2, D);
    src.vn = make_rsrc(a.v + b * a.v_sb + hk * a.v_sh, rows_n, src.v_sl2, D);
    src.none = make_rsrc(a.q, 0, 0, D);
  }

  // Q^T operand: lane holds query n, head_dim [16s + 8g, 16s + 8g + 8) per
  // k-step s. With two streams, wave w of each stream needs the same 32
  // queries: each stream fetches half of the k-steps and the halves are
  // swapped through LDS, so Q crosses the memory system once per workgroup.
  // Q loads go out first (they are needed first), then this stream's first
  // tile.
  // Register indices must stay compile-time constants, so the stream choice
  // is a (wave-uniform) branch around fixed-index loops.
  constexpr int KQ = KS / NS;  // k-steps this stream fetches
  u32x4 qr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qr[s] = u32x4{0, 0, 0, 0};
  // Rows past the end load nothing (a CU takes in 64 bytes per clock, and a
  // short chunk leaves many rows of the last query tile empty).
  const uint16_t* qp = a.q + b * a.q_sb + int64_t(qvalid ? qi : 0) * a.q_sl + h * a.q_sh + 8 * g;
  if (qvalid) {
    if (stream == 0) {
#pragma unroll
      for (int s = 0; s < KQ; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qp + 16 * s);
    } else {
#pragma unroll
      for (int s = KQ; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qp + 16 * s);
    }
  }

  TileRegs<D> regs;
  const int t_first = t_begin + stream;
  TileDma<D, T> dma;
  if constexpr (NS == 1) {
    // The first tile straight into LDS.
    dma.init(wave, lane);
    if (t_begin < t_end) {
      dma.issueK(src, t_begin, wave, smem);
      dma.issueV(src, t_begin, wave, smem + Lds<D>::kElems);
    }
  } else {
    // The stream's first tile into registers right away. (Fetching the
    // second one too delays the first: a CU takes in 64 bytes per clock.)
    regs.load(ltid, src, t_first, t_first < t_end);
    const EndBounds eb = end_bounds(a, q0, min(q0 + kBM, a.Lq) - 1);
    kv_min = cache_len + eb.lo;
    kv_max = cache_len + eb.hi;
  }

  // Visible-key end of this lane's query (per-key masking of straddling tiles).
  const int my_end = qvalid ? cache_len + visible_end(a, qi, cache_len) : 0;

  if (NS == 2) {
    // Exchange area: the first tile buffer of stream 1 (not yet written).
    static_assert(kBM * Lds<D>::kPitch <= Lds<D>::stage, "Q exchange must fit one stage");
    uint16_t* qx = smem + 2 * Lds<D>::stage + (wave * 32 + n) * Lds<D>::kPitch + 8 * g;
    if (stream == 0) {
#pragma unroll
      for (int s = 0; s < KQ; ++s) *reinterpret_cast<u32x4*>(qx + 16 * s) = qr[s];
    } else {
#pragma unroll
      for (int s = KQ; s < KS; ++s) *reinterpret_cast<u32x4*>(qx + 16 * s) = qr[s];
    }
    __syncthreads();
    if (stream == 0) {
#pragma unroll
      for (int s = KQ; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qx + 16 * s);
    } else {
#pragma unroll
      for (int s = 0; s < KQ; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qx + 16 * s);
    }
    __syncthreads();  // exchange read before stream 1's first tile overwrites it
    DX_STAMP(1);
  }
  {
    const uint32_t qmask = qvalid ? ~0u : 0u;
    const uint32_t flip = a.negate_q ? 0x80008000u : 0u;  // exact sign flip of both halves
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = (qr[s] & qmask) ^ flip;
  }

  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  Softmax sm{-INFINITY, 0.f};
  const float c = a.scale_log2;

  // Key tile t's masking: cache tiles see every cached key and only the
  // partial last one masks (its rows past cache_len); new-key tiles mask
  // where they reach past kv_min.
  auto tile_mask = [&](int t, int& lim, bool& masked) __attribute__((always_inline)) {
    const bool in_cache = t < n_ct;
    const int j0 = in_cache ? t * kBN : cache_len + (t - n_ct) * kBN;
    lim = (in_cache ? cache_len - j0 : my_end - j0) - 4 * g;
    masked = in_cache ? j0 + kBN > cache_len : j0 + kBN > kv_min;
  };

  if constexpr (NS == 1) {
    // Double buffer filled by LDS DMA: step i first sends tile i + 1 into
    // the buffer that tile i - 1 used (every wave finished reading it before
    // the barrier that ended step i - 1), computes tile i, then waits for its
    // own pieces and meets the other waves at the barrier that publishes
    // tile i + 1.
    const int nt = t_end - t_begin;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's pieces of the first tile
    __syncthreads();
    for (int i = 0; i < nt; ++i) {
      uint16_t* const cur = smem + (i & 1) * Lds<D>::stage;
      uint16_t* const nxt = smem + ((i + 1) & 1) * Lds<D>::stage;
      if (i + 1 < nt) {
        dma.issueK(src, t_begin + i + 1, wave, nxt);
        dma.issueV(src, t_begin + i + 1, wave, nxt + Lds<D>::kElems);
      }
      if (wave_active) {
        int lim;
        bool masked;
        tile_mask(t_begin + i, lim, masked);
        f32x16 sc[2];
        qk_tile<D, T>(cur, qr, sc, lane);
        const float mb = softmax_max<D>(sc, acc, sm, c, lim, masked);
        step_body<D, T, false>(cur, cur + Lds<D>::kElems, qr, sc, sc, acc, sm, c, mb, lane);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  } else {
  // Each stream double-buffers its tiles in its own LDS region. A buffer is
  // rewritten two rounds after it was read, past the barrier of the round in
  // between, which every wave has reached. Tiles past the workgroup's
  // visible keys are skipped.
  uint16_t* const region = smem + stream * 2 * Lds<D>::stage;
  for (int i = 0; i < iters; ++i) {
    const int t = t_first + i * NS;
    uint16_t* const st = region + (i & 1) * Lds<D>::stage;
    if (t < t_end) regs.store(ltid, st, st + Lds<D>::kElems);
    __syncthreads();
    if (i < 16) DX_STAMP(16 + i);
    if (t + NS < t_end) regs.load(ltid, src, t + NS, true);
    const bool in_cache = t < n_ct;
    const int j0 = in_cache ? t * kBN : cache_len + (t - n_ct) * kBN;
    if (wave_active && t < t_end && j0 < kv_max) {
      int lim;
      bool masked;
      tile_mask(t, lim, masked);
      tile_step<D, T>(st, st + Lds<D>::kElems, qr, acc, sm, c, lim, masked, lane);
    }
  }
  }

  // The exponent reference of acc and l, in log2 units.
  float mref = sm.m == -INFINITY ? -INFINITY : sm.m * c;
  const bool merge_here = a.counters != nullptr && it.n_splits > 1;
  if constexpr (NS == 2) {
    // The streams swap halves through LDS: stream s keeps head_dim blocks
    // [s DT / 2, (s + 1) DT / 2) and hands (mref, l) and its other blocks to
    // the same lane of the other stream, in 16-byte vectors laid out
    // [vector][lane] (consecutive lanes hit consecutive 16 bytes). Both then
    // combine their blocks with the same weights, stream 0's terms first, and
    // store them (store_result_halves): all eight waves share the combine and
    // the stores. The stream enters as a constant, so every block index is
    // static.
    auto epilogue = [&](auto stream_c) __attribute__((always_inline)) {
      constexpr int S = decltype(stream_c)::value;
      constexpr int LANES = 64 * kNW, HB = DT / 2, NV = 1 + 4 * HB;
      static_assert(2 * NV * LANES * 16 <= Lds<D>::bytes,
                    "the hand-over lies below the row area");
      f32x4* const x = reinterpret_cast<f32x4*>(smem);
      f32x4* const hand = x + S * NV * LANES;
      const f32x4* const got = x + (1 - S) * NV * LANES;
      __syncthreads();  // all tile reads done: the LDS is free
      DX_STAMP(2);
      DX_NOTE(9, uint32_t(t_end - t_begin) | uint32_t(iters) << 16);
#ifdef DX_TIMELINE
      {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
        DX_NOTE(10, xcc);
      }
#endif
      // This stream's largest |acc| in each row, over all head_dim blocks: with
      // the other stream's, weighted as the combine weights them, it bounds
      // the combined row's largest |value| (a split partial's scale exponent).
      float amax = 0.f;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) amax = fmaxf(amax, fabsf(acc[d][r]));
      amax = xor32_max(amax);  // the row's other half of each block (lanes l and l ^ 32)
      hand[ltid] = f32x4{mref, sm.l, amax, 0.f};
#pragma unroll
      for (int dd = 0; dd < HB; ++dd)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int d = (1 - S) * HB + dd;
          hand[(1 + 4 * dd + q) * LANES + ltid] =
              f32x4{acc[d][4 * q], acc[d][4 * q + 1], acc[d][4 * q + 2], acc[d][4 * q + 3]};
        }
      __syncthreads();
      DX_STAMP(3);
      const f32x4 h = got[ltid];
      constexpr bool s0 = S == 0;
      const float m0 = s0 ? mref : h[0], m1 = s0 ? h[0] : mref;
      const float l0 = s0 ? sm.l : h[1], l1 = s0 ? h[1] : sm.l;
      const float mm = fmaxf(m0, m1);
      const float base = mm == -INFINITY ? 0.f : mm;
      const float w0 = fast_exp2(m0 - base), w1 = fast_exp2(m1 - base);
      // One explicit rounding order, so that both streams hold the same l.
      sm.l = __builtin_fmaf(l0, w0, l1 * w1);
      const float x0 = s0 ? amax : h[2], x1 = s0 ? h[2] : amax;
      const float rbound = __builtin_fmaf(x0, w0, x1 * w1);
#pragma unroll
      for (int dd = 0; dd < HB; ++dd)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int d = S * HB + dd;
          const f32x4 v = got[(1 + 4 * dd + q) * LANES + ltid];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float own = acc[d][4 * q + e];
            const float a0 = s0 ? own : v[e], a1 = s0 ? v[e] : own;
            acc[d][4 * q + e] = __builtin_fmaf(a0, w0, a1 * w1);
          }
        }
      mref = mm;
      const float l_tot = xor32_sum(sm.l);
      // Result rows through stream 1's tile buffers, past the hand-over area.
      const uint32_t area = lds_addr(smem) + Lds<D>::bytes;
      if (!merge_here) {
        // The output, or a partial for the merge kernel: blocked.
        store_result_halves<D, T, S, 0, true>(a, it, q0, wave * 32, g, lane, ltid, wave_active,
                                              acc, l_tot, mref, area, rbound);
        DX_STAMP(4);
        DX_NOTE(8, uint32_t(it.split) | uint32_t(it.n_splits) << 8 | uint32_t(it.b) << 16);
        DX_STAMP(7);
        return;
      }
      static_assert((kBM * (kPMergeSplits + 1) + 4) * 4 <= Lds<D>::bytes,
                    "merge scratch below the row area");
      if (a.spread) {
        // Split, merged in this launch and spread over the group
        // (spread_split_group): the partial goes to this XCD's L2; every
        // split then merges its chunk of rows once the group has arrived.
        const int e = store_result_halves<D, T, S>(a, it, q0, wave * 32, g, lane, ltid,
                                                   wave_active, acc, l_tot, mref, area, rbound);
        DX_STAMP(4);
        spread_split_group<D, T, kBM, 64 * kNW * NS>(
            a, it, q0, smem, [&]() __attribute__((always_inline)) {
              restore_partial_halves<D, S>(a, it, q0, wave * 32, g, lane, wave_active, l_tot,
                                           mref, e, area);
            });
        return;
      }
      // Split, merged in this launch: store the partial, then every wave
      // arrives (arrive_split_group); the last split of the group merges.
      store_result_halves<D, T, S, kScDevice>(a, it, q0, wave * 32, g, lane, ltid, wave_active,
                                              acc, l_tot, mref, area, rbound);
      DX_STAMP(4);
      arrive_split_group<D, T, kBM, 64 * kNW * NS, 2>(a, it, q0, smem);
    };
    if (stream == 0) epilogue(std::integral_constant<int, 0>{});
    else epilogue(std::integral_constant<int, 1>{});
  } else {
    const float l_tot = xor32_sum(sm.l);
    // Result rows through the tile buffers, whose last reads and DMA pieces
    // ended at the loop's last barrier. One stream never merges in the launch.
    if (!wave_active) return;
    store_result_staged<D, T>(a, it, kBM, q0, wave * 32, g, lane, acc, l_tot, mref,
                              lds_addr(smem));
  }
}

// ---------------------------------------------------------------------------
// Prefill: two groups of four waves on the same key tiles, half a tile apart.
//
// A workgroup covers 256 queries: group 0 takes rows 0..127, group 1 rows
// 128..255, and both read each K/V tile from LDS (one DMA fill per tile for
// 256 queries). Each group alternates two phases per key tile:
//   MFMA phase  PV of the previous tile and S = K Q^T of this one (32 MFMAs)
//   VALU phase  masking, row max, lazy rescale, exponentials, packing, sums
// and group 1 runs one phase behind group 0, with a workgroup barrier
// between phases. Waves w and w + 4 share a SIMD, so on every SIMD one wave's
// MFMAs overlap the other wave's vector work: the phases are arranged so the
// matrix pipe and the vector pipe of a SIMD are busy at the same time, which
// one wave alone cannot do (in-order issue puts its dependent softmax after
// its MFMAs).
//
// Buffers: K and V are double buffered separately. Tile j's K is read in
// global phases 2j-1 (group 0) and 2j (group 1); its V in 2j+1 and 2j+2. In
// each odd phase 2m+1 every wave sends its DMA pieces of K_{m+2} (into the K
// buffer K_m left at the barrier ending phase 2m) and V_{m+1} (into V_{m-1}'s
// buffer, free since then too), and waits for them at the end of phase 2m+2:
// two phases of latency cover, nothing overwritten while read.
// ---------------------------------------------------------------------------

// P = exp2(S c - mb) packed to 16-bit pairs in MFMA B-operand order (pk[u][e]:
// keys 8 (u % 2) + 2 e, +1 of half u / 2) and the row sum over the packed
// values (v_dot2 against (1, 1): l sums exactly the P used by PV). Masked
// scores are -inf and c > 0, so their P is exactly 0.
template <typename T>
__device__ __forceinline__ void exp_pack(f32x16 (&s)[2], Softmax& sm, float c, float mb,
                                         u32x4 (&pk)[4]) {
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kt][r] = fast_exp2(__builtin_fmaf(s[kt][r], c, -mb));
  float part[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t p =
          Mfma<T>::pack(s[u / 2][8 * (u % 2) + 2 * e], s[u / 2][8 * (u % 2) + 2 * e + 1]);
      pk[u][e] = p;
      part[e & 1] = Mfma<T>::sum2(p, part[e & 1]);
    }
  sm.l += part[0] + part[1];
}

// O^T += V^T P^T from packed P (operand layout as pv_tile).
template <int D, typename T>
__device__ __forceinline__ void pv_packed(const uint16_t* Vs, const u32x4 (&pk)[4],
                                          f32x16 (&acc)[D / 32], int lane) {
  constexpr int DT = D / 32;
  const int g = lane >> 5;
  const int j = lane & 15, half = (lane >> 4) & 1;
  const uint16_t* vbase = Vs + (4 * g + (j >> 2)) * Lds<D>::vPitch + 16 * half + 4 * (j & 3);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint16_t* vu = vbase + 16 * u * Lds<D>::vPitch;
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const u32x2 lo = lds_read_tr16(vu + 32 * d);
      const u32x2 hi = lds_read_tr16(vu + 8 * Lds<D>::vPitch + 32 * d);
      acc[d] = Mfma<T>::run(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[u], acc[d]);
    }
  }
}

// Per-lane LDS byte addresses of the paired kernel's operand reads in stage
// 0; stage s adds a compile-time offset, so with the stages unrolled every
// read is base register + immediate and the MFMA phase spends no vector
// instructions on addresses.
//  - S operand (k[s], k-step s): row n (+ 32 for the second half), logical
//    chunk 2 s + g, stored at chunk (2 s + g) ^ kswz(n).
//  - V^T operand (v[d], dims tile d): rows r0 = 4 g + j / 4 (+ 8, + 16 u),
//    bytes 32 half + 8 (j % 4) of 64-byte column group d, stored at group
//    d ^ vswz(r0).
template <int D, int NST = 3> struct PairAddr {
  static constexpr int KS = D / 16, DT = D / 32, RB = 2 * D;
  uint32_t k[KS], v[DT];
  __device__ __forceinline__ void init(uint32_t lds, int lane) {
    using L = PairLds<D, NST>;
    const int n = lane & 31, g = lane >> 5, j = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
    for (int st = 0; st < KS; ++st)
      k[st] = lds + 2 * L::kstage(0) + n * RB + 16 * ((2 * st + g) ^ L::kswz(n));
    const int r0 = 4 * g + (j >> 2);
#pragma unroll
    for (int d = 0; d < DT; ++d)
      v[d] = lds + 2 * L::vstage(0) + r0 * RB + 32 * half + 8 * (j & 3) + 64 * (d ^ L::vswz(r0));
  }
};

// The MFMA phase of a paired-group step: S = K Q^T for this tile (K stage
// KST), then O^T += V^T P^T for the previous one (V stage VST). While the S
// MFMAs run, the wave packs the previous tile's exponentials (pf, fp32) into
// MFMA operands (pk) and adds their row sums to l, so that this vector work,
// which has no MFMA dependency, fills the issue slots of the MFMA phase
// instead of lengthening the VALU phase. Every LDS read is issued one batch
// ahead of the MFMAs that consume it; the sched_group_barrier sequence keeps
// the compiler from moving the reads back next to their MFMAs (which exposes
// the LDS latency once per batch) or hoisting them all (which costs
// registers). kParts: kPhaseBoth, or kPhaseS for a work item's first step,
// whose PV would multiply P = 0 (S alone, no packing: l and acc unchanged).
constexpr int kPhaseS = 1, kPhaseBoth = 3;
template <int D, typename T, int KST, int VST, int kParts = kPhaseBoth>
__device__ __forceinline__ void pair_mfma_phase(const PairAddr<D>& ad, const f32x16 (&pf)[2],
                                                float& l, f32x16 (&acc)[D / 32],
                                                const u32x4 (&qr)[D / 16], f32x16 (&sc)[2]) {
  using L = PairLds<D>;
  static_assert(kParts == kPhaseS || kParts == kPhaseBoth, "S alone, or S and PV");
  constexpr bool kPV = kParts == kPhaseBoth;
  constexpr int KS = D / 16, DT = D / 32, RB = 2 * D;
  constexpr int NQ = 2 * KS;            // S MFMAs: (half i % 2, k-step i / 2): two interleaved chains
  constexpr int NP = kPV ? 4 * DT : 0;  // PV MFMAs: (key step u = i / DT, dims tile d = i % DT)
  constexpr int NA = NQ + NP;
  constexpr int B = 2;            // MFMAs per batch; each batch's reads go out one batch early
  constexpr int NQB = NQ / B, NPB = NP / B;
  static_assert(NQ % B == 0 && NP % B == 0, "batches must not mix PV and S MFMAs");
  static_assert(16 % NQB == 0, "the packing must split evenly over the S batches");
  constexpr uint32_t kOff = 2 * (L::kstage(KST) - L::kstage(0));
  constexpr uint32_t vOff = 2 * (L::vstage(VST) - L::vstage(0));
  static_assert(kOff + 32 * RB < 65536 && vOff + 56 * RB < 65536, "immediate offsets");
  auto vfrag = [&](int i) __attribute__((always_inline)) {
    const uint32_t vu = ad.v[i % DT] + (vOff + 16 * (i / DT) * RB);
    const u32x2 lo = lds_read_tr16_at(vu);
    const u32x2 hi = lds_read_tr16_at(vu + 8 * RB);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  auto kfrag = [&](int i) __attribute__((always_inline)) {
    return lds_read_b128_at(ad.k[i / 2] + (kOff + (i % 2) * 32 * RB));
  };
  // One sequence of A operands: S MFMAs first, then PV MFMAs.
  auto afrag = [&](int i) __attribute__((always_inline)) {
    return i < NQ ? kfrag(i) : vfrag(i - NQ);
  };
  // pk[u][e]: keys 8 (u % 2) + 2 e, +1 of half u / 2 (MFMA B-operand order).
  u32x4 pk[4];
  float part[2] = {0.f, 0.f};  // same pairing as the other kernels: identical sums
  constexpr int PPB = 16 / NQB;  // packed pairs per S batch
  auto pack = [&](int w) __attribute__((always_inline)) {
    const int u = w / 4, e = w % 4;
    const uint32_t pp = Mfma<T>::pack(pf[u / 2][8 * (u % 2) + 2 * e],
                                      pf[u / 2][8 * (u % 2) + 2 * e + 1]);
    pk[u][e] = pp;
    part[e & 1] = Mfma<T>::sum2(pp, part[e & 1]);
  };
  sc[0] = f32x16{};
  sc[1] = f32x16{};
  u32x4 fr[2][B];
#pragma unroll
  for (int i = 0; i < B; ++i) fr[0][i] = afrag(i);
#pragma unroll
  for (int b = 0; b < NA / B; ++b) {
    if (b + 1 < NA / B) {
#pragma unroll
      for (int i = 0; i < B; ++i) fr[(b + 1) & 1][i] = afrag((b + 1) * B + i);
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int m = b * B + i;
      if (m < NQ) {
        sc[m % 2] = Mfma<T>::run(fr[b & 1][i], qr[m / 2], sc[m % 2]);
      } else {
        const int q = m - NQ;
        acc[q % DT] = Mfma<T>::run(fr[b & 1][i], pk[q / DT], acc[q % DT]);
      }
    }
    if (kPV && b < NQB) {
#pragma unroll
      for (int x = 0; x < PPB; ++x) pack(b * PPB + x);
    }
  }
  if (kPV) l += part[0] + part[1];
  // Schedule: batch b's MFMAs after the reads of batch b + 1 (two LDS reads
  // per PV MFMA, one per S MFMA).
  __builtin_amdgcn_sched_group_barrier(sg::kDsRead, B, 0);
#pragma unroll
  for (int b = 0; b < NQB; ++b) {
    if (b + 1 < NQB) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, B, 0);
    else __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 2 * B, 0);
    __builtin_amdgcn_sched_group_barrier(sg::kMfma, B, 0);
  }
#pragma unroll
  for (int b = 0; b < NPB; ++b) {
    if (b + 1 < NPB) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 2 * B, 0);
    __builtin_amdgcn_sched_group_barrier(sg::kMfma, B, 0);
  }
}


template <int D, typename T>
__global__ __launch_bounds__(64 * kPairWaves, 1) void attn_pair_kernel(AttnArgs a) {
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int BM = kBMPair;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  prefetch_args(a);

  const Coord it = locate(a, blockIdx.x, false, 0);
  const int b = it.b, h = it.h;
  const int wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);  // 0..7, uniform
  const int grp = wid >> 2, wave = wid & 3, lane = int(threadIdx.x) & 63;
  const int g = lane >> 5, n = lane & 31;
  const int q0 = it.qtile * BM;
  const int row = grp * 128 + wave * 32 + n;
  const int qi = q0 + row;
  const bool qvalid = qi < a.Lq;
  const bool wave_active = q0 + grp * 128 + wave * 32 < a.Lq;
  const int cache_len = it.cache_len;

  // Key range of the workgroup (see attn_fwd_kernel).
  const EndBounds eb = end_bounds(a, q0, min(q0 + BM, a.Lq) - 1);
  const int kv_min = cache_len + eb.lo;
  const int kv_max = cache_len + eb.hi;
  const int n_ct = (cache_len + kBN - 1) / kBN;
  const int n_tiles = n_ct + (kv_max - cache_len + kBN - 1) / kBN;
  // 32-bit unsigned: splits <= 16 and tiles < 2^26 (keys < 2^30), so the
  // products fit, and the division is far shorter than a 64-bit one.
  const int t_begin = int(uint32_t(it.split) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int t_end = int(uint32_t(it.split + 1) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int nt = t_end - t_begin;

  KvSrc src;
  src.c_ss2 = int(a.c_ss) * 2;
  src.k_sl2 = int(a.k_sl) * 2;
  src.v_sl2 = int(a.v_sl) * 2;
  src.n_ct = n_ct;
  {
    const int rows_c = min(cache_len, kv_max), rows_n = kv_max - cache_len;
    const int hk = a.kv_group == 1 ? h : h / a.kv_group;  // K/V head of this query head
    const int64_t coff = b * a.c_sb + hk * a.c_sh;
    src.kc = make_rsrc(a.ck ? a.ck + coff : a.q, rows_c, src.c_ss2, D);
    src.vc = make_rsrc(a.cv ? a.cv + coff : a.q, rows_c, src.c_ss2, D);
    src.kn = make_rsrc(a.k + b * a.k_sb + hk * a.k_sh, rows_n, src.k_sl2, D);
    src.vn = make_rsrc(a.v + b * a.v_sb + hk * a.v_sh, rows_n, src.v_sl2, D);
    src.none = make_rsrc(a.q, 0, 0, D);
  }

  using Rows = PairRows<D>;
  using Dma = PairDma<D, T>;
  const uint32_t smem_b = lds_addr(smem);
  // The work item's Q rows into the row area (rows past Lq read as zeros),
  // then K_0 into stage 0 and V of step -1 (nothing: zeros) into V stage 2.
  Rows::load_q(make_rsrc(a.q + b * a.q_sb + int64_t(q0) * a.q_sl + h * a.q_sh,
                         max(a.Lq - q0, 0), int(a.q_sl) * 2, D),
               int(a.q_sl) * 2, a.Lq - q0, smem_b + Rows::off, wid, lane);
  Dma dma;
  dma.init(wid, lane, src);
#pragma unroll
  for (int m = 0; m < Dma::NP; ++m) dma.issue(m, src, smem_b, t_begin, nt, 0, -1, 0, 2, wid);
  const int my_end = qvalid ? cache_len + visible_end(a, qi, cache_len) : 0;
  PairAddr<D> ad;
  ad.init(smem_b, lane);

  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  Softmax sm{-INFINITY, 0.f};
  const float c = a.scale_log2;
  f32x16 sc[2];
  f32x16 pf[2];  // exponentials of the last tile, packed in the next MFMA phase

  // The first MFMA phase runs its PV on V stage 2 (step -1) with P = 0. The
  // V slots above filled that stage with zeros, so whatever an earlier kernel
  // left in LDS (NaN included) contributes exactly 0.
  __builtin_amdgcn_s_waitcnt(0);  // this wave's pieces of Q, K_0 and V stage 2
  __syncthreads();
  // Q^T operand: row ``row``, k-step s = 16-element chunks 2 s + g.
  u32x4 qr[KS];
  {
    const uint32_t flip = a.negate_q ? 0x80008000u : 0u;  // exact sign flip of both halves
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qr[s] = lds_read_b128_at(Rows::at(smem_b + Rows::off, row, 2 * s + g)) ^ flip;
  }

  // The phase program, global phases p = -1 .. 2 nt (2 nt + 2 barriers for
  // every wave). Group 0 runs MFMA phase j (S_j, PV_{j-1}) at p = 2j - 1 and
  // the VALU phase of tile j at p = 2j; group 1 runs each one phase later.
  // Each group runs its own straight-line loop body, so its values keep
  // their registers from one phase to the next; the body is unrolled over
  // the three stages (step j uses stage j mod 3), so that every LDS offset is
  // an immediate.
  //
  // DMA: during VALU phase j every wave sends its slots of step j (K_{j+2},
  // V_{j+1}), spread between the exponentials. K_{j+2}'s stage last held
  // K_{j-1}, read in MFMA phases j-1 (p <= 2j - 2); V_{j+1}'s held V_{j-2},
  // read in the same phases: both free by p = 2j, group 0's send of step j.
  // Step j's pieces are first read at p = 2j + 3; every wave has them waited
  // for by the barrier ending p = 2j + 2. Group 0 sent step j + 1 at
  // p = 2j + 2 and keeps those NP pieces in flight; group 1 (sends at odd p)
  // has nothing newer and waits for all.
  auto send = [&](int j, auto rc, int m) __attribute__((always_inline)) {
    constexpr int R = decltype(rc)::value;  // j mod 3
    dma.issue(m, src, smem_b, t_begin, nt, j + 2, j + 1, (R + 2) % 3, (R + 1) % 3, wid);
  };
  // The first MFMA phase (j = 0) computes S only (its PV would multiply
  // P = 0); every later one runs one straight-line body, so the last (j = nt)
  // also computes an S that is never used, from a stale but in-bounds K
  // buffer: a branch to a PV-only last phase inside the loop costs the loop
  // its single register allocation (hundreds of spilled VGPRs). The wave in
  // its MFMA phase issues ahead of its SIMD partner
  // (raised priority): an MFMA it cannot issue idles the matrix pipe, while
  // the partner's vector work fills whatever issue cycles are left.
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) pf[kt] = f32x16{};
  using Both = std::integral_constant<int, kPhaseBoth>;
  using OnlyS = std::integral_constant<int, kPhaseS>;
  auto mfma_phase = [&](auto rc, auto parts) __attribute__((always_inline)) {
    constexpr int R = decltype(rc)::value;  // j mod 3: K stage R, V stage R - 1
    constexpr int P = decltype(parts)::value;
    __builtin_amdgcn_s_setprio(1);
    if (wave_active) pair_mfma_phase<D, T, R, (R + 2) % 3, P>(ad, pf, sm.l, acc, qr, sc);
    __builtin_amdgcn_s_setprio(0);
  };
  static_assert(Dma::NP == 4 || Dma::NP == 2, "DMA slots are spread over the 32 exponentials");
  auto valu_phase = [&](int j, auto rc) __attribute__((always_inline)) {
    if (!wave_active) {
#pragma unroll
      for (int m = 0; m < Dma::NP; ++m) send(j, rc, m);
    } else {
      const int t = t_begin + j;
      const bool in_cache = t < n_ct;
      const int j0 = in_cache ? t * kBN : cache_len + (t - n_ct) * kBN;
      const int lim = (in_cache ? cache_len - j0 : my_end - j0) - 4 * g;
      const bool masked = in_cache ? j0 + kBN > cache_len : j0 + kBN > kv_min;
      const float mb = softmax_max<D>(sc, acc, sm, c, lim, masked);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pf[kt][r] = fast_exp2(__builtin_fmaf(sc[kt][r], c, -mb));
          constexpr int every = 32 / Dma::NP;
          if ((16 * kt + r) % every == every - 1) send(j, rc, (16 * kt + r) / every);
        }
    }
  };
  // Phase boundary: a bare s_barrier, fenced against compiler reordering of
  // LDS accesses only. __syncthreads()'s workgroup fence would also wait for
  // every outstanding DMA piece (they write LDS); instead, at the end of an
  // even phase, a wave waits for the pieces it must have landed (loads
  // complete in order) and for its LDS reads.
  constexpr int kWaitOld = (Dma::NP & 15) | ((Dma::NP >> 4) << 14) | (7 << 4);  // vmcnt(NP) lgkmcnt(0)
  auto end_phase = [&](bool even) __attribute__((always_inline)) {
    if (even) {
      if (grp == 0) __builtin_amdgcn_s_waitcnt(kWaitOld);
      else __builtin_amdgcn_s_waitcnt(0);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  // Steps of one group: VALU phase j, then MFMA phase j + 1.
  auto steps = [&](bool first_even) __attribute__((always_inline)) {
    for (int j = 0;;) {
      if (j >= nt) break;
      valu_phase(j, S0{});
      end_phase(first_even);
      mfma_phase(S1{}, Both{});
      end_phase(!first_even);
      if (++j >= nt) break;
      valu_phase(j, S1{});
      end_phase(first_even);
      mfma_phase(S2{}, Both{});
      end_phase(!first_even);
      if (++j >= nt) break;
      valu_phase(j, S2{});
      end_phase(first_even);
      mfma_phase(S0{}, Both{});
      end_phase(!first_even);
      ++j;
    }
  };
  if (grp == 0) {
#pragma unroll
    for (int m = 0; m < Dma::NP; ++m) send(-1, S2{}, m);
    mfma_phase(S0{}, OnlyS{});  // p = -1
    end_phase(false);
    steps(true);             // p = 2j (VALU), 2j + 1 (MFMA)
    end_phase(true);         // p = 2 nt
  } else {
#pragma unroll
    for (int m = 0; m < Dma::NP; ++m) send(-1, S2{}, m);
    end_phase(false);        // p = -1
    mfma_phase(S0{}, OnlyS{});  // p = 0
    end_phase(true);
    steps(false);            // p = 2j + 1 (VALU), 2j + 2 (MFMA)
  }
  // The last sends (steps past the end, zeros) must land before the
  // workgroup's LDS is handed to the next one.
  __builtin_amdgcn_s_waitcnt(0);

  const float mref = sm.m == -INFINITY ? -INFINITY : sm.m * c;
  const float l_tot = xor32_sum(sm.l);
  // Result rows through the row area: every earlier read of it was before
  // the first phase barrier, and no DMA targets it.
  const uint32_t area = smem_b + Rows::off;
  const int r0 = grp * 128 + wave * 32;
  if (a.counters == nullptr || it.n_splits == 1) {
    if (!wave_active) return;
    store_result_staged<D, T>(a, it, BM, q0, r0, g, lane, acc, l_tot, mref, area);
    return;
  }
  // Split, merged in this launch (arrive_split_group): arrive once this
  // workgroup's partial is stored; the last of the group merges, in the K/V
  // stages (idle after the loop).
  if (wave_active)
    store_result_staged<D, T, kScDevice>(a, it, BM, q0, r0, g, lane, acc, l_tot, mref, area);
  static_assert((BM * (kPMergeSplits + 1) + 1) * 4 <= PairLds<D>::bytes, "merge scratch fits");
  // Two splits per batch: the K/V loop's registers leave room for no more.
  arrive_split_group<D, T, BM, 64 * kPairWaves, 2>(a, it, q0, smem);
}

// ---------------------------------------------------------------------------
// Decode-shaped calls: split-KV in one launch.
//
// A work item is (batch, head, query group, key split). Its workgroup has NQW
// compute waves, each owning 32 queries of the group (up to 32 NQW rows), and
// one producer wave; all compute waves read every key tile of the split. On
// MI355X a CU takes in about 50 GB/s whether the bytes come from HBM, L2 or
// LDS DMA, and the chip moves bytes into CUs at about the HBM rate whatever
// their source, so every K/V byte should reach exactly one CU: the planner
// keeps one query group where it can and picks the splits from a cost model.
//
// Loads. Memory instructions stall at issue once enough are in flight (a CU
// takes a 1 KB piece about every 20 ns), and a wave stalled at issue runs
// nothing else. So the compute waves issue no loads: the producer wave issues
// the LDS DMA of the group's Q rows and of the K/V tiles (the swizzled
// unpadded layout of the prefill kernel), two tiles ahead, into three slots
// (tile j in slot j % 3). It waits for tile j's pieces with its own vmcnt,
// then publishes the tile in LDS (the slot's generation, j / 3 + 1); before
// refilling a slot it waits until every compute wave's count of tiles done
// has passed the slot's previous tile. No workgroup barrier in the tile loop:
// a compute wave waits for a tile's generation, computes it and records it
// done, so a tile is computed as soon as its bytes have landed while later
// tiles stream in.
//
// Merge. Each split stores its partial (partial_scale format), then either a
// separate merge kernel combines them (attn_combine_kernel), or the splits
// merge in the kernel itself: every split arrives on its group's counter and
// merges one row chunk of all the group's partials once all have arrived.
// ---------------------------------------------------------------------------
constexpr int kMaxDecSplits = 8;
// Poll limit of a workgroup waiting for its group's other splits:
// s_memrealtime ticks (100 MHz), 50 us. Reached only when a split cannot be
// scheduled; the last arrival then merges the waiting workgroup's rows.
constexpr uint64_t kSpinTicks = 5000;
// Wait of the L2 fast path for the group's other splits: 20 us, ample for
// co-resident workgroups (they arrive within a few us of each other).
constexpr uint32_t kFastTicks = 2000;
static_assert(4 + 2 + kMaxDecSplits <= kCounterStride, "group state fits its slot");

// K/V tile slots in LDS (tile j of a work item in slot j % kDecSlots).
constexpr int kDecSlots = 3;

template <int D, int NQW> struct DecLds {
  using L = PairLds<D, kDecSlots>;
  static constexpr int q_off = L::bytes;                     // Q rows, K-swizzled (wave w: rows 32 w..)
  static constexpr int sync_off = q_off + 32 * NQW * D * 2;  // slot generations, tiles done per wave, merge flags
  static constexpr int bytes = sync_off + 64;
  static_assert(bytes <= 160 * 1024, "decode LDS must fit one workgroup");
};

// The producer wave's DMA: all PK pieces of a K tile, then of its V tile
// (piece p: rows [p RPP, (p + 1) RPP)), and the NQ pieces of the group's Q
// rows. Lane l of a piece fills physical chunk l % CR of row l / CR and
// fetches the logical chunk the swizzle puts there.
template <int D, int NQW>
struct DecDma {
  using L = PairLds<D, kDecSlots>;
  static constexpr int CR = D / 8;                // 16-byte chunks per row
  static constexpr int RPP = 64 / CR;             // rows per piece
  static constexpr int PK = kBN / RPP;            // pieces per K (or V) tile
  static constexpr int NQ = 32 * NQW / RPP;       // Q pieces of the group
  static constexpr int per_tile = 2 * PK;         // pieces per tile
  static_assert(per_tile <= 63, "a tile's pieces fit the vmcnt counter");
  uint32_t on[per_tile], dc[per_tile];  // lane offset in its tile (new-key stride), cache-stride delta
  uint32_t qo[NQ];                      // lane offset of each Q piece

  __device__ __forceinline__ void init(int lane, const KvSrc& src, int q_sl2) {
#pragma unroll
    for (int m = 0; m < per_tile; ++m) {
      const int r = (m % PK) * RPP + lane / CR, x = lane % CR;
      const int c = m < PK ? x ^ L::kswz(r) : x ^ (4 * L::vswz(r));
      const uint32_t sn = uint32_t(m < PK ? src.k_sl2 : src.v_sl2);
      on[m] = uint32_t(r) * sn + uint32_t(c * 16);
      dc[m] = uint32_t(r) * (uint32_t(src.c_ss2) - sn);
    }
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
      const int r = m * RPP + lane / CR, x = lane % CR;
      qo[m] = uint32_t(r) * uint32_t(q_sl2) + uint32_t((x ^ L::kswz(r)) * 16);
    }
  }
  // The group's Q rows into the Q area.
  __device__ __forceinline__ void issue_q(__amdgpu_buffer_rsrc_t rq, uint32_t lds_b) const {
#pragma unroll
    for (int m = 0; m < NQ; ++m) dma_piece_at(rq, lds_b + DecLds<D, NQW>::q_off + m * 1024, qo[m]);
  }
  // Tile t (absolute index) into slot.
  __device__ __forceinline__ void issue_tile(const KvSrc& src, uint32_t lds_b, int t, int slot) const {
    const bool in_cache = t < src.n_ct;
    const __amdgpu_buffer_rsrc_t rk = in_cache ? src.kc : src.kn, rv = in_cache ? src.vc : src.vn;
    const uint32_t row0 = uint32_t((in_cache ? t : t - src.n_ct) * kBN);
    const uint32_t bk = row0 * uint32_t(in_cache ? src.c_ss2 : src.k_sl2);
    const uint32_t bv = row0 * uint32_t(in_cache ? src.c_ss2 : src.v_sl2);
    const uint32_t cmask = in_cache ? ~0u : 0u;
    const uint32_t kt = lds_b + 2 * L::kstage(slot), vt = lds_b + 2 * L::vstage(slot);
#pragma unroll
    for (int m = 0; m < PK; ++m) dma_piece_at(rk, kt + m * 1024, on[m] + (dc[m] & cmask) + bk);
#pragma unroll
    for (int m = 0; m < PK; ++m)
      dma_piece_at(rv, vt + m * 1024, on[PK + m] + (dc[PK + m] & cmask) + bv);
  }
};

// One half of a key tile for one compute wave: S^T = K Q^T over the tile's
// keys [32 h, 32 h + 32), softmax, O^T += V^T P^T. Two waves of a query block
// take the two halves of every tile, each with its own running (max, sum,
// output), merged after the loop: with seven waves a CU runs two per SIMD,
// and one wave's exponentials (32 per lane per tile, quarter-rate) overlap
// the other's MFMAs. (Alone, a wave spent ~2,200 cycles per whole tile,
// about as long on the exponentials and packing as on its 32 MFMAs.)
// kb / vb: this lane's operand addresses in the slot (PairAddr plus the
// slot's offset). The operand reads run ahead of the MFMAs that use them (K
// fragments four MFMAs ahead, V^T fragments two), and sched_group_barrier
// keeps that order: left to itself the compiler puts each read right before
// its MFMA and the wave waits out the LDS latency every time.
template <int D, typename T>
__device__ __forceinline__ void dec_half(int h, const uint32_t (&kb)[D / 16],
                                         const uint32_t (&vb)[D / 32], const u32x4 (&qr)[D / 16],
                                         f32x16 (&acc)[D / 32], Softmax& sm, float c, int lim,
                                         bool masked) {
  constexpr int KS = D / 16, DT = D / 32, RB = 2 * D;
  constexpr int NQ = KS;      // S MFMAs, one per k-step
  constexpr int NP = 2 * DT;  // PV MFMAs: key step i / DT (of 16 keys), head_dim tile i % DT
  constexpr int W = 4;        // K fragments in flight
  const uint32_t hk = uint32_t(h) * 32 * RB;  // the half's first row
  auto kfrag = [&](int i) __attribute__((always_inline)) {
    return lds_read_b128_at(kb[i] + hk);
  };
  auto vfrag = [&](int i) __attribute__((always_inline)) {
    const uint32_t vu = vb[i % DT] + hk + 16 * (i / DT) * RB;
    const u32x2 lo = lds_read_tr16_at(vu);
    const u32x2 hi = lds_read_tr16_at(vu + 8 * RB);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  f32x16 sc = f32x16{};
  u32x4 kf[W];
#pragma unroll
  for (int i = 0; i < W; ++i) kf[i] = kfrag(i);
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    sc = Mfma<T>::run(kf[i % W], qr[i], sc);
    if (i + W < NQ) kf[i % W] = kfrag(i + W);
  }
#pragma unroll
  for (int i = 0; i < W; ++i) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 1, 0);
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    __builtin_amdgcn_sched_group_barrier(sg::kMfma, 1, 0);
    if (i + W < NQ) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Softmax of the half's 32 keys (lim counts from the half's first key).
  if (masked) {
    int lm = lim - 32 * h;
    asm volatile("" : "+v"(lm));
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (key_hidden(0, r, lm)) sc[r] = -INFINITY;
  }
  float tm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int r = 0; r < 16; ++r) tm[r % 4] = fmaxf(tm[r % 4], sc[r]);
  const float tmax = xor32_max(fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3])));
  const float m_new = fmaxf(sm.m, tmax);
  // Lazy rescale (wave-uniform branch): only when some lane's max grew by
  // more than 2^8. Before anything is accumulated (m = -inf on every lane)
  // there is nothing to scale: just take the new reference.
  const bool grow = (m_new - sm.m) * c > 8.0f;
  if (__any(grow)) {
    if (!__all(sm.m == -INFINITY)) {
      const float corr = sm.m == -INFINITY ? 0.f : fast_exp2((sm.m - m_new) * c);
      sm.l *= corr;
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d] *= corr;
    }
    sm.m = m_new;
  }
  const float mb = sm.m == -INFINITY ? 0.f : sm.m * c;
#pragma unroll
  for (int r = 0; r < 16; ++r) sc[r] = fast_exp2(__builtin_fmaf(sc[r], c, -mb));
  // pk[u][e]: keys 8 u + 2 e, +1 of the half (MFMA B-operand order).
  u32x4 pk[2];
  float part[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t pp = Mfma<T>::pack(sc[8 * u + 2 * e], sc[8 * u + 2 * e + 1]);
      pk[u][e] = pp;
      part[e & 1] = Mfma<T>::sum2(pp, part[e & 1]);
    }
  sm.l += part[0] + part[1];
  __builtin_amdgcn_sched_barrier(0);
  u32x4 vf[2];
  vf[0] = vfrag(0);
  vf[1] = vfrag(1);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    acc[i % DT] = Mfma<T>::run(vf[i % 2], pk[i / DT], acc[i % DT]);
    if (i + 2 < NP) vf[i % 2] = vfrag(i + 2);
  }
  __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 4, 0);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    __builtin_amdgcn_sched_group_barrier(sg::kMfma, 1, 0);
    if (i + 2 < NP) __builtin_amdgcn_sched_group_barrier(sg::kDsRead, 2, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Wait until an LDS word written by another wave of the workgroup reaches
// `target` (the writer is resident and always gets there).
__device__ __forceinline__ void lds_wait_at_least(const int* w, int target) {
  while (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
    __builtin_amdgcn_s_sleep(0);
  asm volatile("" ::: "memory");
}

template <int D, typename T, int NQW>
__global__ __launch_bounds__(64 * (2 * NQW + 1), 1) void attn_decode_kernel(AttnArgs a) {
  constexpr int KS = D / 16, DT = D / 32, RB = 2 * D;
  constexpr int NCW = 2 * NQW;     // compute waves: two per query block (key halves)
  constexpr int NT = 64 * (NCW + 1);
  constexpr int kRows = 32 * NQW;
  using DL = DecLds<D, NQW>;
  using L = PairLds<D, kDecSlots>;
  using Dma = DecDma<D, NQW>;
  static_assert(NQW >= 1 && NQW <= 3, "per-wave done counts sync[4, 10)");
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  prefetch_args(a);

  const Coord it = locate(a, blockIdx.x, false, 0);  // qtile: the query group
  const int b = it.b, h = it.h;
  const int wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const bool producer = wid == NCW;
  // Compute wave w: query block w % NQW, key half w / NQW of every tile.
  const int blk = wid % NQW, half = wid / NQW;
  const int lane = int(threadIdx.x) & 63, g = lane >> 5, n = lane & 31;
  const int q0 = it.qtile * a.bm;
  const int q_end = min(q0 + a.bm, a.Lq);
  const int row = blk * 32 + n;  // row within the query group
  const int qi = q0 + row;
  const bool wave_active = !producer && q0 + blk * 32 < q_end;
  // Rows stored by the half-0 waves, after the halves are merged.
  const bool qvalid = wave_active && half == 0 && qi < q_end;
  const int cache_len = it.cache_len;

  // Tiles over every key any query of the call may see (cache, then all Lk
  // new keys), so the loads go out before the block starts are read; tiles
  // past this group's visible keys are skipped, straddling ones masked.
  const int n_ct = (cache_len + kBN - 1) / kBN;
  const int n_tiles = n_ct + (a.Lk + kBN - 1) / kBN;
  const int t_begin = int(uint32_t(it.split) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int t_end = int(uint32_t(it.split + 1) * uint32_t(n_tiles) / uint32_t(it.n_splits));
  const int nt = t_end - t_begin;

  KvSrc src;
  src.c_ss2 = int(a.c_ss) * 2;
  src.k_sl2 = int(a.k_sl) * 2;
  src.v_sl2 = int(a.v_sl) * 2;
  src.n_ct = n_ct;
  {
    const int hk = a.kv_group == 1 ? h : h / a.kv_group;
    const int64_t coff = b * a.c_sb + hk * a.c_sh;
    src.kc = make_rsrc(a.ck ? a.ck + coff : a.q, cache_len, src.c_ss2, D);
    src.vc = make_rsrc(a.cv ? a.cv + coff : a.q, cache_len, src.c_ss2, D);
    src.kn = make_rsrc(a.k + b * a.k_sb + hk * a.k_sh, a.Lk, src.k_sl2, D);
    src.vn = make_rsrc(a.v + b * a.v_sb + hk * a.v_sh, a.Lk, src.v_sl2, D);
    src.none = make_rsrc(a.q, 0, 0, D);
  }
  const uint32_t smem_b = lds_addr(smem);
  // sync[0, 3): slot generations; sync[4 + w]: tiles compute wave w is done
  // with (w < NCW <= 6); sync[10, 13): merge flags.
  int* const sync = reinterpret_cast<int*>(reinterpret_cast<char*>(smem) + DL::sync_off);
  int* const done = sync + 4;
  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  Softmax sm{-INFINITY, 0.f};
  const float c = a.scale_log2;

  // Tiles [0, na) hold keys some row of the group may see: tile starts grow
  // with j, so they are a prefix. Evaluated by every wave (scalar work; no
  // memory loads without block starts).
  const EndBounds eb = end_bounds(a, q0, q_end - 1);
  const int kv_min = cache_len + eb.lo, kv_max = cache_len + eb.hi;
  auto tile_start = [&](int j) __attribute__((always_inline)) {
    const int tg = t_begin + j;
    return tg < n_ct ? tg * kBN : cache_len + (tg - n_ct) * kBN;
  };

  if (producer) {
    // Q rows of [q0, q_end) of head h (rows past them read as zeros), then
    // the first two tiles; then per tile: wait for its pieces (the next
    // tile's stay in flight), publish it, refill the slot the previous tile
    // used once every compute wave is done with it. (The first two tiles go
    // out before the visible range is known; a tile past it lands unused.)
    Dma dma;
    dma.init(lane, src, int(a.q_sl) * 2);
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(a.q + b * a.q_sb + int64_t(q0) * a.q_sl + h * a.q_sh, q_end - q0,
                  int(a.q_sl) * 2, D);
    dma.issue_q(rq, smem_b);
    if (nt > 0) dma.issue_tile(src, smem_b, t_begin, 0);
    if (nt > 1) dma.issue_tile(src, smem_b, t_begin + 1, 1);
    int na = 0;
    while (na < nt && tile_start(na) < kv_max) ++na;
    __syncthreads();  // the counters are zeroed before anyone uses them
    for (int j = 0; j < na; ++j) {
      if (j + 1 < na) wait_vmcnt<Dma::per_tile>();
      else wait_vmcnt<0>();
      if (lane == 0)
        __hip_atomic_store(sync + j % kDecSlots, j / kDecSlots + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      if (j + 2 < na) {
        // Tile j - 1 (slot (j + 2) % 3) done by every compute wave: each
        // wave's own count, since a wave ahead cannot stand in for one behind.
        if (j >= 1)
          for (int w = 0; w < NCW; ++w) lds_wait_at_least(done + w, j);
        dma.issue_tile(src, smem_b, t_begin + j + 2, (j + 2) % kDecSlots);
      }
    }
  } else {
    if (threadIdx.x < 16) sync[threadIdx.x] = 0;
    // Visible-key end of this lane's query (both key halves mask with it).
    const int my_end = wave_active && qi < q_end ? cache_len + visible_end(a, min(qi, a.Lq - 1), cache_len) : 0;
    PairAddr<D, kDecSlots> ad;
    ad.init(smem_b, lane);
    int na = 0;
    while (na < nt && tile_start(na) < kv_max) ++na;
    const int nw = wave_active ? na : 0;
    __syncthreads();
    // Operand addresses and mask of tile j.
    auto kaddr = [&](int j, uint32_t (&kb)[KS]) __attribute__((always_inline)) {
      const uint32_t ko = 2 * L::kstage(j % kDecSlots);
#pragma unroll
      for (int s = 0; s < KS; ++s) kb[s] = ad.k[s] + ko;
    };
    auto vaddr = [&](int j, uint32_t (&vb)[DT]) __attribute__((always_inline)) {
      const uint32_t vo = 2 * (L::vstage(j % kDecSlots) - L::vstage(0));
#pragma unroll
      for (int d = 0; d < DT; ++d) vb[d] = ad.v[d] + vo;
    };
    auto limit = [&](int j, int& lim, bool& masked) __attribute__((always_inline)) {
      const int j0 = tile_start(j);
      const bool in_cache = t_begin + j < n_ct;
      lim = (in_cache ? cache_len - j0 : my_end - j0) - 4 * g;
      masked = in_cache ? j0 + kBN > cache_len : j0 + kBN > kv_min;
    };
    if (nw > 0) {
      u32x4 qr[KS];
      for (int j = 0; j < nw; ++j) {
        lds_wait_at_least(sync + j % kDecSlots, j / kDecSlots + 1);  // tile j has landed
        if (j == 0) {
          // Q^T operand of the block's 32 queries (lane: query n, head_dim
          // [16 s + 8 g, +8) per k-step s), from the K-swizzled Q rows.
          const uint32_t qb = DL::q_off + blk * 32 * RB - 2 * L::kstage(0);
          const uint32_t flip = a.negate_q ? 0x80008000u : 0u;  // exact sign flip of both halves
#pragma unroll
          for (int s = 0; s < KS; ++s) qr[s] = lds_read_b128_at(ad.k[s] + qb) ^ flip;
        }
        uint32_t kb[KS], vb[DT];
        int lim;
        bool masked;
        kaddr(j, kb);
        vaddr(j, vb);
        limit(j, lim, masked);
        dec_half<D, T>(half, kb, vb, qr, acc, sm, c, lim, masked);
        // Done with tile j once this wave's reads of it have returned.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0)
          __hip_atomic_store(done + wid, j + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    if (lane == 0)
      __hip_atomic_store(done + wid, nt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // every tile read before the LDS is reused

  {
    // Merge the key halves: each half-1 wave hands its (max, sum, output) to
    // its block's half-0 wave through LDS, in 16-byte vectors laid out
    // [block][vector][lane] (4 DT vectors of output, then (max, sum)).
    constexpr int HV = 4 * DT + 1;
    static_assert(NQW * HV * 64 * 16 <= L::bytes, "the hand-over fits the tile slots");
    f32x4* const hand = reinterpret_cast<f32x4*>(smem) + blk * HV * 64 + lane;
    if (wave_active && half == 1) {
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          hand[(4 * d + r4) * 64] = f32x4{acc[d][4 * r4], acc[d][4 * r4 + 1], acc[d][4 * r4 + 2],
                                          acc[d][4 * r4 + 3]};
      hand[(HV - 1) * 64] = f32x4{sm.m, sm.l, 0.f, 0.f};
    }
    __syncthreads();
    if (wave_active && half == 0) {
      f32x4 o1[HV];
#pragma unroll
      for (int i = 0; i < HV; ++i) o1[i] = hand[i * 64];
      const float m1 = o1[HV - 1][0], l1 = o1[HV - 1][1];
      const float mx = fmaxf(sm.m, m1);
      const float e0 = sm.m == -INFINITY ? 0.f : fast_exp2((sm.m - mx) * c);
      const float e1 = m1 == -INFINITY ? 0.f : fast_exp2((m1 - mx) * c);
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[d][r] = acc[d][r] * e0 + o1[4 * d + r / 4][r % 4] * e1;
      sm.l = sm.l * e0 + l1 * e1;
      sm.m = mx;
    }
    // No barrier needed after the reads: the LDS is next written (merge
    // scratch) only after the arrival protocol's barriers.
  }

  const float mref = sm.m == -INFINITY ? -INFINITY : sm.m * c;
  const float l_tot = xor32_sum(sm.l);
  if (it.n_splits == 1) {
    if (qvalid) store_result<D, T>(a, it, a.bm, row, qi, g, acc, l_tot, mref);
    return;
  }

  // Partial of this split, in the group's workspace area: values as the
  // MFMA registers hold them, one 512-byte piece per (block, d-tile, r4)
  // with row n's 16 bytes at 16 n (lane n's 4 f16, then lane n + 32's), so
  // that every store instruction writes 512 contiguous bytes; records
  // [split][row] (row = 32 block + n) from lanes g == 0. (Row-major values
  // would take 8-byte pieces of 32 rows per instruction, which the memory
  // pipeline issues many times slower.)
  const bool in_kernel_merge = a.counters != nullptr;
  const int nrows = q_end - q0;
  const uint32_t ws_rows = uint32_t(kRows);
  const __amdgpu_buffer_rsrc_t rws =
      __builtin_amdgcn_make_buffer_rsrc(a.ws_o + it.pbase * ws_rows * D, (short)0,
                                        int(it.n_splits * ws_rows * D * 2), kBufWord3);
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + it.pbase * ws_rows * 4, (short)0, int(it.n_splits * ws_rows * 16), kBufWord3);
  constexpr int kSc0 = 1, kSc1 = 16;  // cache policy: this XCD's L2, device scope
  constexpr int CR = D / 8;
  u32x2 pw[DT][4];
  f32x4 prec = f32x4{};
  if (qvalid) {
    const PartialScale ps = partial_scale<D>(acc, l_tot);
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        pw[d][r4][0] = Mfma<f16_t>::pack(acc[d][4 * r4] * ps.k, acc[d][4 * r4 + 1] * ps.k);
        pw[d][r4][1] = Mfma<f16_t>::pack(acc[d][4 * r4 + 2] * ps.k, acc[d][4 * r4 + 3] * ps.k);
      }
    prec = f32x4{l_tot > 0.f ? mref : -INFINITY, l_tot, float(ps.e), 0.f};
  }
  auto store_partial = [&](auto aux) __attribute__((always_inline)) {
    if (!qvalid) return;
    const uint32_t vbase = uint32_t(it.split) * ws_rows * D * 2 + uint32_t(blk) * DT * 2048 +
                           uint32_t(n) * 16 + uint32_t(g) * 8;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        __builtin_amdgcn_raw_buffer_store_b64(pw[d][r4], rws, vbase + (4 * d + r4) * 512, 0,
                                              decltype(aux)::value);
    if (g == 0)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, prec), rrec,
                                             (uint32_t(it.split) * ws_rows + uint32_t(row)) * 16,
                                             0, decltype(aux)::value);
  };
  store_partial(std::integral_constant<int, 0>{});
  if (!in_kernel_merge) return;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have reached this XCD's L2
  __syncthreads();

  // Merge, spread over the group: split s merges row chunk s (rows
  // [s nrows / S, (s + 1) nrows / S)) of every split's partial, once all S
  // partials are stored.
  //
  // Arrival. Atomics are coherent across the whole device (measured on
  // MI355X: adds from workgroups on all eight XCDs to one word all count),
  // but plain stores reach only the L2 of the XCD that issues them. Group
  // word w (64-bit, at fs) counts arrivals in bits [0, 16), marks from bit
  // 16, and the arrivals from XCC x in the nibble at bit 32 + 4 x; fs[2]
  // counts finished workgroups. A workgroup that sees all S arrivals and no
  // mark decides from the nibbles: all S on its own XCC means every partial
  // of the group is in this XCC's L2, and it merges its chunk with loads from
  // the L2 (sc0, the fast path). Any other outcome takes the slow path. One
  // that does not see S arrivals within fast_ticks marks the word, by
  // compare-and-swap and only while arrivals < S, so every workgroup of the
  // group decides the same way (fast iff the S-th arrival precedes every
  // mark and the group shares one XCC).
  //
  // Slow path, at device scope: every workgroup stores its partial again
  // with device-scope write-through, then gs[0] counts arrivals, gs[1]
  // finishes, gs[2 + c] claims chunk c. Unless it is the last arrival, a
  // workgroup polls gs[0] until all S have arrived, with a time limit, so it
  // never waits forever on a workgroup that has not been scheduled. A chunk
  // is merged by whoever claims it first (compare-and-swap): its owner once
  // all have arrived, or the last arrival, which after its own chunk claims
  // every chunk still unclaimed. Every chunk is merged exactly once.
  //
  // The S-th workgroup to finish with each state resets it to zero.
  const int S = it.n_splits;
  int32_t* const fs = a.counters + it.pbase * kCounterStride;
  uint64_t* const fw = reinterpret_cast<uint64_t*>(fs);
  int32_t* const gs = fs + 4;
  int* const sh = sync + 10;
  constexpr uint64_t kMark = 1ull << 16;
  const bool use_fs = a.fast_ticks != 0;
  if (threadIdx.x == 0 && !use_fs) sh[0] = 0;
  if (threadIdx.x == 0 && use_fs) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
    const uint64_t mine = 1ull | (1ull << (32 + 4 * xcc));
    const uint64_t alone = uint64_t(S) << (32 + 4 * xcc);  // all S arrivals from this XCC
    int fast = -1;
    uint64_t v = __hip_atomic_fetch_add(fw, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (fast < 0) {
      const uint64_t arrived = v & (kMark - 1), marks = (v >> 16) & 0xffffull;
      if (marks != 0) {
        fast = 0;
      } else if (arrived == uint64_t(S)) {
        fast = (v >> 32) == (alone >> 32) ? 1 : 0;
      } else if (__builtin_amdgcn_s_memrealtime() - t0 > a.fast_ticks) {
        uint64_t expect = v;
        if (__hip_atomic_compare_exchange_strong(fw, &expect, v + kMark, __ATOMIC_RELAXED,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          fast = 0;
        else
          v = expect;  // changed meanwhile: decide on the new value
      } else {
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_fetch_add(fw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    sh[0] = fast;
  }
  __syncthreads();
  const bool fast = sh[0] != 0;

  // A chunk has at most kRows / 2 rows (S >= 2). Per chunk: thread t < rn
  // loads the records of row t of every split and turns them into the row's
  // split weights (into LDS); meanwhile thread t loads the values of its units
  // u = t + NT k < rn CR (row u % rn, 8-dim chunk u / rn: consecutive lanes
  // take consecutive rows of one chunk, contiguous in the partial) of every
  // split; after one barrier each thread combines its units. Only threads
  // with work issue loads, each thread's all at once.
  constexpr int UPT = (kRows / 2 * CR + NT - 1) / NT;  // units per thread, at most
  float* const lcoef = reinterpret_cast<float*>(smem);                         // [row][split]
  int* const lexp = reinterpret_cast<int*>(lcoef + kRows / 2 * kMaxDecSplits);  // [row]
  static_assert(kRows / 2 * (kMaxDecSplits + 1) * 4 <= L::bytes, "merge scratch fits");
  auto merge_chunk = [&](int c, auto aux) __attribute__((always_inline)) {
    constexpr int kAux = decltype(aux)::value;
    const int r_lo = c * nrows / S, rn = (c + 1) * nrows / S - r_lo;
    const int nu = rn * CR;
    const int t = int(threadIdx.x);
    // Splits sp >= S read past the descriptors' bound and return zeros
    // (unused), so the loads need no branch between them (a guarded load
    // compiles to a wait on every earlier one).
    u32x4 val[UPT][kMaxDecSplits];
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      const int u = t + NT * k;
      if (u < nu) {
        const int r = r_lo + u % rn, ch = u / rn;
        const uint32_t off =
            uint32_t(r / 32) * DT * 2048 + uint32_t(ch) * 512 + uint32_t(r % 32) * 16;
#pragma unroll
        for (int sp = 0; sp < kMaxDecSplits; ++sp)
          val[k][sp] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rws, uint32_t(sp) * ws_rows * D * 2 + off, 0, kAux));
      }
    }
    if (t < rn) {
      f32x4 rec[kMaxDecSplits];
#pragma unroll
      for (int sp = 0; sp < kMaxDecSplits; ++sp)
        rec[sp] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rrec, (uint32_t(sp) * ws_rows + r_lo + t) * 16, 0, kAux));
      // Row weights: c_s = exp2(m_s - M) l_s / L, taken relative to the largest
      // scale exponent E (applied once at the end).
      float mmax = -INFINITY;
      int emax = INT_MIN;
#pragma unroll
      for (int sp = 0; sp < kMaxDecSplits; ++sp) {
        mmax = sp < S ? fmaxf(mmax, rec[sp][0]) : mmax;
        emax = sp < S ? max(emax, int(rec[sp][2])) : emax;
      }
      const float base = mmax == -INFINITY ? 0.f : mmax;
      float w[kMaxDecSplits];
      float Lsum = 0.f;
#pragma unroll
      for (int sp = 0; sp < kMaxDecSplits; ++sp) {
        w[sp] = sp < S ? fast_exp2(rec[sp][0] - base) * rec[sp][1] : 0.f;
        Lsum += w[sp];
      }
      const float invL = 1.0f / Lsum;  // no visible key anywhere: NaN, as the reference
#pragma unroll
      for (int sp = 0; sp < kMaxDecSplits; ++sp)
        lcoef[t * kMaxDecSplits + sp] =
            sp < S ? __builtin_ldexpf(w[sp] * invL, int(rec[sp][2]) - emax) : 0.f;
      lexp[t] = emax;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      const int u = t + NT * k;
      if (u >= nu) continue;
      const int r = u % rn, ch = u / rn;
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < kMaxDecSplits; ++sp)
        if (sp < S) {
          const float cs = lcoef[r * kMaxDecSplits + sp];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[2 * e] += cs * to_f32(f16_t{uint16_t(val[k][sp][e] & 0xffffu)});
            o[2 * e + 1] += cs * to_f32(f16_t{uint16_t(val[k][sp][e] >> 16)});
          }
        }
      const int emax = lexp[r];
      u32x4 packed;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        packed[e] =
            Mfma<T>::pack(__builtin_ldexpf(o[2 * e], emax), __builtin_ldexpf(o[2 * e + 1], emax));
      uint16_t* op = a.out + b * a.o_sb + int64_t(q0 + r_lo + r) * a.o_sl + h * a.o_sh + ch * 8;
      __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(op));
    }
  };

  if (fast) {
    merge_chunk(it.split, std::integral_constant<int, kSc0>{});
  } else {
    store_partial(std::integral_constant<int, kSc1>{});  // again, through to memory
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = __hip_atomic_fetch_add(gs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == S - 1;
      int all = last;
      if (!last) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
          if (__hip_atomic_fetch_add(gs, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= S) {
            all = 1;
            break;
          }
          if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      sh[1] = all;
      sh[2] = last;
    }
    __syncthreads();
    const bool all = sh[1] != 0, last = sh[2] != 0;
    for (int c0 = 0; all && c0 < (last ? S : 1); ++c0) {
      const int c = it.split + c0 < S ? it.split + c0 : it.split + c0 - S;  // own chunk first
      __syncthreads();  // the previous chunk's LDS scratch and sh[3] have been read
      if (threadIdx.x == 0) {
        int unclaimed = 0;
        sh[3] = __hip_atomic_compare_exchange_strong(gs + 2 + c, &unclaimed, 1, __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!sh[3]) continue;
      merge_chunk(c, std::integral_constant<int, kSc1>{});
    }
    if (threadIdx.x == 0) {
      // Done with the slow state; the last to get here resets it.
      if (__hip_atomic_fetch_add(gs + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1) {
        for (int i = 0; i < 2 + S; ++i)
          __hip_atomic_store(gs + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (threadIdx.x == 0 && use_fs) {
    // Done with the arrival state; the S-th to finish resets it.
    if (__hip_atomic_fetch_add(fs + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1) {
      __hip_atomic_store(fw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(fs + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// One wave per merge block: at C1 (83 rows x 24 heads, 8 splits) 1,056 blocks
// of 64 threads took 12.58 us per call against 12.79 us for 264 of 256 threads
// (13.04 and 13.98 us for 512 and 1,024 threads).
constexpr int kCombineThreads = 64;
template <int D> struct CombineShape {
  static constexpr int TPR = D / 4;                  // threads per row
  static constexpr int RPB = kCombineThreads / TPR;  // rows per block
};

// Merge split-KV partials (merge_partials). Each thread owns 4 consecutive
// dims of a row and issues all NMAX (>= the group's split count) record and
// value loads before combining: buffer descriptors bounded by the group's
// n_splits partials return zeros for the rest, with no branch between the
// loads (a guarded load compiles to a wait on every earlier one). Blocks of
// one (batch, head) run on the XCD whose L2 holds that head's partials.
template <int D, typename T, int NMAX, bool BLK>
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(AttnArgs a) {
  DX_MERGE_STAMP(0);
  prefetch_args(a);
  if constexpr (BLK) {
    // Blocked partials (unit_off): block k of a group takes rows [RW k, RW k +
    // RW) whole, RW = 64 / (D / 8) (4 rows at D = 128); lane j RW + n reads
    // chunk j of row RW k + n, so for each chunk the block's rows are one
    // 16 RW-byte line segment, and each output row is stored whole. (Blocks of
    // 32 rows x 2 chunks, 1 KB contiguous loads, measured C1 12.14 against
    // 11.95 us per call: their output rows go out in 32-byte pieces.) The
    // arithmetic is merge_partials', value by value.
    static_assert(kCombineThreads == 64, "one wave per block");
    constexpr int RW = 64 / (D / 8);
    const Coord cd = locate(a, blockIdx.x, true, a.comb_chunks);
    const int row = RW * cd.split + int(threadIdx.x) % RW, ch = int(threadIdx.x) / RW;
    const int qi = cd.qtile * a.bm + row;
    if (row >= a.bm || qi >= a.Lq) return;
    const uint32_t rows = uint32_t(a.bm), n = uint32_t(cd.n_splits);
    const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_ml + cd.pbase * a.bm * 4, (short)0, int(n * rows * 16), kBufWord3);
    const __amdgpu_buffer_rsrc_t rval = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_o + cd.pbase * a.bm * D, (short)0, int(n * rows * D * 2), kBufWord3);
    f32x4 ml[NMAX];
    u32x4 o[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      ml[s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rrec, (uint32_t(s) * rows + uint32_t(row)) * 16, 0, 0));
      o[s] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rval, uint32_t(s) * rows * (D * 2) + unit_off<D, true>(row, ch), 0, 0));
    }
    float c[NMAX];
    const int emax = merge_weights(ml, cd.n_splits, c);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NMAX; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) merge_add2(acc[2 * e], acc[2 * e + 1], c[s], o[s][e]);
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = Mfma<T>::pack(__builtin_ldexpf(acc[2 * e], emax),
                           __builtin_ldexpf(acc[2 * e + 1], emax));
    uint16_t* op = a.out + cd.b * a.o_sb + int64_t(qi) * a.o_sl + cd.h * a.o_sh + 8 * ch;
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(op));
    DX_MERGE_STAMP(1);
    return;
  }
  using CS = CombineShape<D>;
  // Blocks per work-item group: ceil(min(bm, Lq) / RPB), as the host sizes
  // the grid (no block for rows that no query tile has; bm need not be a
  // multiple of RPB: decode query groups).
  const Coord cd = locate(a, blockIdx.x, true, a.comb_chunks);
  const int row = cd.split * CS::RPB + threadIdx.x / CS::TPR;
  const int dim = 4 * (threadIdx.x % CS::TPR);
  const int qi = cd.qtile * a.bm + row;
  if (row >= a.bm || qi >= a.Lq) return;
  const uint32_t rows = uint32_t(a.bm), n = uint32_t(cd.n_splits);
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + cd.pbase * a.bm * 4, (short)0, int(n * rows * 16), kBufWord3);
  const __amdgpu_buffer_rsrc_t rval = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + cd.pbase * a.bm * D, (short)0, int(n * rows * D * 2), kBufWord3);
  f32x4 ml[NMAX];
  u32x2 o[NMAX];
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    const uint32_t r = uint32_t(s) * rows + uint32_t(row);
    ml[s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rrec, r * 16, 0, 0));
    o[s] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                         rval, (r * D + uint32_t(dim)) * 2, 0, 0));
  }
  const f32x4 acc = merge_partials(ml, o, cd.n_splits);
  uint16_t* op = a.out + cd.b * a.o_sb + int64_t(qi) * a.o_sl + cd.h * a.o_sh + dim;
  u32x2 w2;
  w2[0] = Mfma<T>::pack(acc[0], acc[1]);
  w2[1] = Mfma<T>::pack(acc[2], acc[3]);
  __builtin_nontemporal_store(w2, reinterpret_cast<u32x2*>(op));
  DX_MERGE_STAMP(1);
}

// ---------------------------------------------------------------------------
// Host side: launch planning shared by the workspace query and the launch.
// ---------------------------------------------------------------------------
int device_cus() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (int(cache.size()) <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// Attention kernels a plan can pick (the DX_TUNE_ATTN_KERNEL values).
enum AttnKernel { kSingle = 1, kDual = 2, kPaired = 3, kDecode = 4 };

struct Plan {
  int n_qtiles;
  int bm;                    // queries per work item (decode: query-group rows)
  int kernel;                // AttnKernel
  int nqw;                   // decode: compute waves per workgroup (2 or 3)
  int prow;                  // rows per partial in the workspace (decode: 32 per compute block)
  int n_seg;                 // 0 = uniform
  int uniform_splits;
  std::vector<int> seg_b, seg_splits, seg_cache, seg_base, comb_base;
  int64_t items, comb_blocks, partials;
  int64_t counter_bytes;     // arrival counters at the start of the workspace
  bool pmerge;               // splits merged in the kernel (no merge launch)
  bool spread;               // ... spread over each group's splits (dual-stream kernel)
  int64_t ws_bytes;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Merge-kernel blocks per work-item group (rows: min(bm, Lq)): row-major
// partials take CombineShape's rows per block; blocked ones (the dual-stream
// kernel's) 64 / (D / 8) whole rows per block.
int64_t combine_bpt(int64_t D, int64_t rows, bool blocked) {
  if (blocked) return cdiv(rows * (D / 8), 64);
  return cdiv(rows, D == 128 ? CombineShape<128>::RPB : CombineShape<64>::RPB);
}

int bm_of(int kernel) { return kernel == kPaired ? kBMPair : kBM; }


// Query-group rows and per-segment key splits of the one-launch decode
// kernel, for segments of `units` (batch, head) pairs over tiles[i] key tiles
// each (a uniform call is one segment of B*H units). Modelled time (us): a
// CU streams ~50 GB/s whatever the source (HBM, L2, LDS DMA: measured on
// MI355X) and the chip ~6 TB/s, so the streaming phase is the larger of the
// worst split's bytes per CU and the call's HBM bytes over the chip; the
// merge adds ~1.2 us (stores, arrival, polling) plus each split's read of
// its row chunk of every split's partial. Candidates keep at most one
// workgroup per CU. rows == 0: no
// candidate fits (prefill-shaped: the paired kernel takes it).
struct DecodeShape {
  int rows = 0, nqw = 0;
  std::vector<int> splits;
};
DecodeShape choose_decode(int64_t units, int64_t Lq, const std::vector<int64_t>& tiles, int64_t D,
                          int cus, int forced_splits) {
  constexpr double kCuBytesPerUs = 50e3, kChipBytesPerUs = 6e6, kMergeFixedUs = 1.2;
  const int64_t tile_bytes = int64_t(kBN) * D * 2 * 2;
  int64_t all_tiles = 0, max_tiles = 1;
  for (int64_t t : tiles) {
    all_tiles += t;
    max_tiles = std::max(max_tiles, t);
  }
  // Every query group reads its splits' K/V, and the chip moves bytes into
  // CUs (from L2 as from HBM) at about the HBM rate: query groups multiply it.
  const double t_chip1 = double(units * all_tiles * tile_bytes) / kChipBytesPerUs;
  DecodeShape best;
  double best_cost = 1e30;
  for (int64_t nq = cdiv(Lq, 96); nq <= cdiv(Lq, 16); ++nq) {
    const int64_t rows = cdiv(Lq, nq);
    if (nq > 1 && cdiv(Lq, cdiv(Lq, nq - 1)) == nq) continue;  // same groups as nq - 1
    // Largest split per segment: cap on the tiles one workgroup streams.
    for (int64_t cap = max_tiles; cap >= 1; --cap) {
      std::vector<int> sp(tiles.size());
      int64_t wgs = 0;
      double worst = 0.0, merge = 0.0;
      bool ok = true;
      for (size_t i = 0; i < tiles.size(); ++i) {
        const int64_t ti = std::max<int64_t>(tiles[i], 1);
        int64_t si = forced_splits ? std::min<int64_t>(forced_splits, ti) : cdiv(ti, cap);
        if (si > kMaxDecSplits) ok = false;
        si = std::min<int64_t>(si, kMaxDecSplits);
        sp[i] = int(si);
        wgs += units * nq * si;
        worst = std::max(worst, double(cdiv(ti, si) * tile_bytes + rows * D * 2) / kCuBytesPerUs);
        // Split s merges rows chunk s of every split's partial.
        if (si > 1)
          merge = std::max(merge, kMergeFixedUs + double(cdiv(rows, si) * si * (D * 2 + 16)) /
                                                      kCuBytesPerUs);
      }
      if (!ok || wgs > cus) break;  // a smaller cap only needs more workgroups
      const double cost = std::max(worst, t_chip1 * double(nq)) + merge;
      if (cost < best_cost - 1e-9) {
        best_cost = cost;
        best.rows = int(rows);
        best.nqw = rows <= 64 ? 2 : 3;
        best.splits = sp;
      }
      if (forced_splits) break;  // one candidate per query grouping
    }
  }
  return best;
}

// Paired-group (prefill) split count for `groups` (batch, head, 256-query
// tile) units of `tiles` key tiles each: the split minimising rounds x
// (tiles per split + a fixed cost per work item, about 8 tiles: its
// start-up, its stores, and the K/V its key range pulls that another query
// tile of the head already read), plus 2 tiles per split for partials and
// merge. Calibrated at the Wan-14B chunk (160 groups of 130 tiles): measured
// 1..10 splits order as this cost does, 3 best (179 us, against 208 us at 8
// and 188 us at 1).
int choose_paired_splits(int64_t groups, int64_t tiles, int cus) {
  int64_t best_s = 1;
  if (groups < 2 * cus && tiles >= 8) {
    double best = 1e30;
    for (int64_t s = 1; s <= kMaxSplits && s <= tiles / 4; ++s) {
      const double cost = double(cdiv(groups * s, cus)) * double(cdiv(tiles, s) + 8) +
                          (s > 1 ? 2.0 * double(s) : 0.0);
      if (cost < best - 1e-9) { best = cost; best_s = s; }
    }
  }
  return int(best_s);
}

Plan make_plan(int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t D, int64_t cache_len,
               const int64_t* cache_lens) {
  Plan p{};
  const int cus = device_cus();
  const int forced_kernel = tuning(DX_TUNE_ATTN_KERNEL);
  const int forced_splits = tuning(DX_TUNE_ATTN_SPLITS);
  // Segments: one per sequence of a ragged batch, longest first; a uniform
  // call is one segment of all B*H (batch, head) pairs.
  const int nseg = cache_lens ? int(B) : 1;
  std::vector<int> order(nseg);
  std::vector<int64_t> tiles(nseg);
  for (int i = 0; i < nseg; ++i) order[i] = i;
  if (cache_lens)
    std::stable_sort(order.begin(), order.end(),
                     [&](int x, int y) { return cache_lens[x] > cache_lens[y]; });
  for (int k = 0; k < nseg; ++k) {
    const int64_t c = cache_lens ? cache_lens[order[k]] : cache_len;
    tiles[k] = cdiv(c, kBN) + cdiv(Lk, kBN);
  }
  const int64_t units = cache_lens ? H : B * H;  // (batch, head) pairs per segment

  std::vector<int> splits(nseg, 1);
  // The one-launch decode kernel is opt-in (DX_TUNE_ATTN_KERNEL = 4): on the
  // C1 decode chunk it measures 16-22 us against 14.5 us for the dual-stream
  // kernel and its merge kernel.
  DecodeShape dec;
  if (forced_kernel == kDecode && forced_splits <= kMaxDecSplits)
    dec = choose_decode(units, Lq, tiles, D, cus, forced_splits);
  if (forced_kernel == kDecode && dec.rows == 0) {
    // Forced onto the decode kernel: the smallest query groups that fit the
    // kernel, splits as forced (or 1), however many workgroups that takes.
    dec.rows = int(std::min<int64_t>(Lq, 96));
    dec.nqw = dec.rows <= 64 ? 2 : 3;
    dec.splits.assign(nseg, 1);
    for (int k = 0; k < nseg; ++k)
      dec.splits[k] = int(std::max<int64_t>(1, std::min<int64_t>({forced_splits ? forced_splits : 1,
                                                                  kMaxDecSplits, tiles[k]})));
  }
  if (dec.rows > 0) {
    int64_t items = 0;
    for (int k = 0; k < nseg; ++k) items += units * cdiv(Lq, dec.rows) * dec.splits[k];
    if (items > kCounterSlots) dec.rows = 0;  // too many groups for the counter region
  }
  if (dec.rows > 0) {
    p.kernel = kDecode;
    p.bm = dec.rows;
    p.nqw = dec.nqw;
    splits = dec.splits;
  } else {
    int64_t total = 0;
    for (int64_t t : tiles) total += t;
    if (forced_kernel && forced_kernel != kDecode) {
      p.kernel = forced_kernel;
    } else {
      // Decode-shaped calls take the dual-stream kernel (128-query items, one
      // workgroup per CU): a uniform call when its 128-query groups fill at
      // most half the CUs, a ragged batch when its chunks fit one 128-query
      // item (all eight waves on the chunk's rows; C4: 27.6 vs 28.3 us on
      // paired groups) or splits in proportion to length leave <= 8 tiles per
      // split. Everything else takes paired groups.
      const int64_t g128 = units * cdiv(Lq, kBM);
      bool dual;
      if (nseg == 1) {
        dual = g128 * 2 <= cus && tiles[0] >= 4;
      } else {
        int64_t worst = 0;
        for (int k = 0; k < nseg; ++k) {
          int64_t s = int64_t(double(cus) / double(g128) * double(tiles[k]) /
                              double(std::max<int64_t>(total, 1)));
          s = std::max<int64_t>(1, std::min<int64_t>({s, kMaxSplits, std::max<int64_t>(tiles[k], 1)}));
          worst = std::max(worst, cdiv(tiles[k], s));
        }
        dual = worst <= 8 || Lq <= kBM;
      }
      p.kernel = dual ? kDual : kPaired;
    }
    p.bm = bm_of(p.kernel);
    const int64_t groups = units * cdiv(Lq, p.bm);  // work-item groups per segment
    for (int k = 0; k < nseg; ++k) {
      int64_t sk;
      if (forced_splits)
        sk = forced_splits;
      else if (nseg > 1)  // ragged: splits in proportion to length, about one item per CU
        sk = int64_t(double(cus) / double(groups) * double(tiles[k]) / double(std::max<int64_t>(total, 1)));
      else if (p.kernel == kDual) {
        // About three quarters of the CUs, >= 2 tiles per split; an odd tile
        // count that those splits cover at one tile each takes one tile per
        // split rather than leaving one split half the work (Wan-5B chunk:
        // 257 image keys, 5 tiles, 9.98 us in 5 splits against 10.3 us in 3;
        // 512 text keys, 8 tiles, 10.38 us in 4 against 10.54 us in 8).
        // Longer ranges, more than four tiles a split at that count, take a
        // split per CU instead: the tile loop then dominates, and every CU
        // streaming raises the call's HBM rate (24 heads x 83 queries over 4K,
        // 16K and 64K cached keys: 18.85 / 46.35 / 148.1 us at 10 splits
        // against 19.70 / 51.55 / 168.4 us at 8; 12 and 16 splits, past one
        // workgroup per CU, 26.8 / 68.1 / 218 and 25.4 / 56.8 / 174 us).
        int64_t most = (3 * cus) / (4 * groups);
        if (most >= 1 && cdiv(tiles[k], most) > 4) most = std::max<int64_t>(most, cus / groups);
        sk = tiles[k] % 2 == 1 && tiles[k] <= most ? tiles[k]
                                                   : std::min<int64_t>(most, cdiv(tiles[k], 2));
      }
      else
        sk = choose_paired_splits(groups, tiles[k], cus);
      splits[k] = int(std::max<int64_t>(
          1, std::min<int64_t>({sk, kMaxSplits, std::max<int64_t>(tiles[k], 1)})));
    }
  }
  p.n_qtiles = int(cdiv(Lq, p.bm));
  const int64_t comb_rows = std::min<int64_t>(p.bm, Lq);  // merge rows per query tile, at most
  const int64_t per_b = H * p.n_qtiles;  // (head, query tile) units per sequence
  if (!cache_lens) {
    p.n_seg = 0;
    p.uniform_splits = splits[0];
    p.items = B * per_b * p.uniform_splits;
    p.partials = p.uniform_splits > 1 ? p.items : 0;
    const bool combine = p.kernel != kDecode;
    p.comb_blocks =
        p.uniform_splits > 1 && combine ? B * per_b * combine_bpt(D, comb_rows, p.kernel == kDual) : 0;
  } else {
    p.n_seg = int(B);
    p.seg_base.push_back(0);
    p.comb_base.push_back(0);
    bool any_split = false;
    for (int k = 0; k < nseg; ++k) {
      const int b = order[k];
      p.seg_b.push_back(b);
      p.seg_splits.push_back(splits[k]);
      p.seg_cache.push_back(int(cache_lens[b]));
      p.seg_base.push_back(int(p.seg_base.back() + per_b * splits[k]));
      const bool combine = p.kernel != kDecode;
      p.comb_base.push_back(int(p.comb_base.back() + (splits[k] > 1 && combine
                                                          ? per_b * combine_bpt(D, comb_rows, p.kernel == kDual) : 0)));
      any_split = any_split || splits[k] > 1;
    }
    p.items = p.seg_base.back();
    p.comb_blocks = p.comb_base.back();
    p.partials = any_split ? p.items : 0;
  }
  // Workspace of any plan with partials: the counter region (kCounterRegion
  // bytes, used by the kernels that merge in-kernel), the f16 partial values,
  // then the fp32 records {m, l, e, 0}.
  const bool has_partials = p.kernel == kDecode ? p.partials > 0 : p.comb_blocks > 0;
  // The counters are the in-kernel merge's; the merge kernel needs none.
  p.counter_bytes = has_partials ? kCounterRegion : 0;
  // The decode kernel's partial values are laid out as its MFMA registers
  // hold them (whole 32-row blocks of its query group); the others' have bm
  // rows: blocked (unit_off) from the dual-stream kernel for the merge
  // kernel, else row-major.
  p.prow = p.kernel == kDecode ? 32 * p.nqw : p.bm;
  p.ws_bytes = has_partials
                   ? kCounterRegion + p.partials * p.prow * (D * 2 + 4 * int64_t(sizeof(float)))
                   : 0;
  // The paired kernel merges its splits itself (arrive_split_group) when no
  // group has more than kPMergeSplits and the counters cover every group; so
  // does the dual-stream kernel on ragged batches, whose groups end at
  // different times, so that a group's merge overlaps other groups' tiles
  // (C4: 27.6 vs 28.7 us). On a uniform call every split ends together and
  // the merge lies on the critical path: at C1 (8 splits of 83 rows) one
  // workgroup's merge of 170 KB of partials took longer than the merge kernel,
  // 14.7 vs 12.7 us per call.
  // The dual-stream kernel can also spread the merge over each group's splits
  // (spread_split_group, DX_TUNE_ATTN_PMERGE 3): every split waits for its
  // group, then merges its own chunk of rows from the L2. At C1 that measured
  // 13.39 us per call against 12.55 us with the merge kernel (14.27 us with
  // the last split merging), so it is not the default.
  int most = p.uniform_splits;
  for (int sk : p.seg_splits) most = std::max(most, sk);
  const int pm = tuning(DX_TUNE_ATTN_PMERGE);
  const bool fits = has_partials && most <= kPMergeSplits && p.partials <= kCounterSlots;
  const bool in_launch = p.kernel == kPaired || (p.kernel == kDual && p.n_seg > 0);
  p.pmerge = fits && (pm == 2 || pm == 3 ? p.kernel == kPaired || p.kernel == kDual
                                         : pm == 0 && in_launch);
  p.spread = p.pmerge && p.kernel == kDual && pm == 3;
  if (p.pmerge) p.comb_blocks = 0;
  return p;
}

// Opt a kernel into `bytes` of dynamic LDS (beyond the 64 KB default window;
// gfx950 allows 160 KB per workgroup) on the current device, once per kernel
// and device: each device holds its own copy of the kernel and its attributes.
hipError_t opt_in_lds(const void* fn, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(mu);
  if (done.count({fn, dev})) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert({fn, dev});
  return e;
}

template <int D, typename T, int NS>
hipError_t launch_main(const AttnArgs& a, int64_t items, hipStream_t st) {
  constexpr int lds = NS * Lds<D>::bytes;  // double-buffered tiles per stream
  const hipError_t attr =
      opt_in_lds(reinterpret_cast<const void*>(&attn_fwd_kernel<D, T, NS>), lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((attn_fwd_kernel<D, T, NS>), dim3(unsigned(items)), dim3(64 * kNW * NS),
                     lds, st, a);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t launch_pair(const AttnArgs& a, int64_t items, hipStream_t st) {
  constexpr int lds = PairRows<D>::off + PairRows<D>::bytes;
  const hipError_t attr = opt_in_lds(reinterpret_cast<const void*>(&attn_pair_kernel<D, T>), lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((attn_pair_kernel<D, T>), dim3(unsigned(items)), dim3(64 * kPairWaves),
                     lds, st, a);
  return hipGetLastError();
}

template <int D, typename T, int NQW>
hipError_t launch_decode(const AttnArgs& a, int64_t items, hipStream_t st) {
  constexpr int lds = DecLds<D, NQW>::bytes;
  const hipError_t attr =
      opt_in_lds(reinterpret_cast<const void*>(&attn_decode_kernel<D, T, NQW>), lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((attn_decode_kernel<D, T, NQW>), dim3(unsigned(items)),
                     dim3(64 * (2 * NQW + 1)), lds, st, a);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t launch_d(const AttnArgs& a, const Plan& p, hipStream_t st) {
  hipError_t e = p.kernel == kDecode
                     ? (p.nqw == 3 ? launch_decode<D, T, 3>(a, p.items, st)
                                   : launch_decode<D, T, 2>(a, p.items, st))
                 : p.kernel == kDual   ? launch_main<D, T, 2>(a, p.items, st)
                 : p.kernel == kPaired ? launch_pair<D, T>(a, p.items, st)
                                       : launch_main<D, T, 1>(a, p.items, st);
  if (e != hipSuccess || p.comb_blocks == 0) return e;
  int most = p.uniform_splits;
  for (int sk : p.seg_splits) most = std::max(most, sk);
  const dim3 grid(unsigned(p.comb_blocks));
  const dim3 block(kCombineThreads);
  // The dual-stream kernel's partials for the merge kernel are blocked, the
  // paired kernel's row-major.
  if (p.kernel == kDual) {
    if (most <= 4) hipLaunchKernelGGL((attn_combine_kernel<D, T, 4, true>), grid, block, 0, st, a);
    else if (most <= 8) hipLaunchKernelGGL((attn_combine_kernel<D, T, 8, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_combine_kernel<D, T, kMaxSplits, true>), grid, block, 0, st, a);
  } else {
    if (most <= 4) hipLaunchKernelGGL((attn_combine_kernel<D, T, 4, false>), grid, block, 0, st, a);
    else if (most <= 8) hipLaunchKernelGGL((attn_combine_kernel<D, T, 8, false>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_combine_kernel<D, T, kMaxSplits, false>), grid, block, 0, st, a);
  }
  return hipGetLastError();
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


// Static scratch of the no-allocation entry point: one copy per device,
// holding the layout a caller's workspace does ([counters][partial values]
// [records]). Device globals are zero when the code object loads, and every
// completed decode launch leaves its counters zero again; the first call on
// a device also clears the counter region (a fill kernel on the caller's
// stream, never a memset: the call may be under graph capture).
constexpr int64_t kScratchBytes = DX_ATTN_SCRATCH_BYTES;
static_assert(kScratchBytes > kCounterRegion, "scratch holds the counter region");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void zero_words_kernel(u32x4* p, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

// Device address of `scratch` on the current device: hipGetSymbolAddress,
// with that device current, once per device. In host code the array's name
// is a host-side stand-in and never a device address, so only this pointer
// reaches kernels.
int scratch_on_device(void** out, hipStream_t st) {
  static std::mutex mu;
  static std::vector<void*> addr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("attention (no-alloc): hipGetDevice failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  std::lock_guard<std::mutex> lk(mu);
  if (int(addr.size()) <= dev) addr.resize(dev + 1, nullptr);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("attention (no-alloc): hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return DX_ELAUNCH;
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, st, static_cast<u32x4*>(p),
                       kCounterRegion / 16);
    e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("attention (no-alloc): clearing the scratch counters failed: %s",
                hipGetErrorString(e));
      return DX_ELAUNCH;
    }
    addr[dev] = p;
  }
  *out = addr[dev];
  return DX_OK;
}

int attention_entry(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k,
                    int64_t k_sb, int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb,
                    int64_t v_sl, int64_t v_sh, const void* cache, int64_t c_plane,
                    int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out, int64_t o_sb,
                    int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                    int64_t H, int64_t Hkv, int64_t D, int64_t cache_len,
                    const int64_t* cache_lens, const int32_t* cache_len_dev,
                    const void* starts, int starts_dtype, int64_t n_blocks, int causal,
                    float softmax_scale, void* workspace, int64_t ws_bytes, void* stream,
                    bool from_scratch = false) {
  DX_CHECK_ARG(dtype == DX_BF16 || dtype == DX_F16 || dtype == DX_F32,
               "attention: dtype code %d unsupported (bf16, f16 or f32)", dtype);
  DX_CHECK_ARG(any_head_dim(D), "attention: head_dim %lld unsupported (16, 32, 64, 128 or 256)",
               (long long)D);
  // bf16/f16 at head dim 64 or 128 take the MFMA kernels of this file; fp32
  // and the other head dims take the general kernel (attn_any.hip).
  const bool general = dtype == DX_F32 || (D != 64 && D != 128);
  const int64_t es = dtype == DX_F32 ? 4 : 2;
  DX_CHECK_ARG(B >= 0 && Lq >= 0 && Lk >= 0 && H > 0, "attention: bad shape");
  DX_CHECK_ARG(Hkv > 0 && H % Hkv == 0,
               "attention: %lld query heads are not a multiple of %lld k/v heads", (long long)H,
               (long long)Hkv);
  // Lk != Lq is cross-attention: every key visible, no block or causal mask
  // (a block or causal mask is defined on the [q_len, cache_len + q_len] grid).
  DX_CHECK_ARG(Lk == Lq || (n_blocks == 0 && !causal),
               "attention: k/v length %lld must equal q length %lld with block_boundaries or "
               "causal (the block mask is [q_len, cache_len + q_len])",
               (long long)Lk, (long long)Lq);
  DX_CHECK_ARG(n_blocks >= 0 && (n_blocks == 0 || starts),
               "attention: block_boundaries pointer missing");
  DX_CHECK_ARG(starts_dtype == DX_I32 || starts_dtype == DX_I64 || n_blocks == 0,
               "attention: block_boundaries must be int32 or int64");
  if (cache_lens) {
    DX_CHECK_ARG(B <= kMaxSeg, "attention varlen: B=%lld exceeds %d", (long long)B, kMaxSeg);
  }
  int64_t max_cache = cache_len;
  if (cache_lens) {
    max_cache = 0;
    for (int64_t i = 0; i < B; ++i) {
      DX_CHECK_ARG(cache_lens[i] >= 0, "attention varlen: negative cache length");
      max_cache = std::max(max_cache, cache_lens[i]);
    }
  }
  DX_CHECK_ARG(max_cache >= 0, "attention: negative cache_len");
  DX_CHECK_ARG(max_cache == 0 || cache, "attention: cache_len > 0 needs a cache");
  DX_CHECK_ARG(max_cache + std::max(Lq, Lk) < (int64_t(1) << 30), "attention: sequence too long");
  DX_CHECK_ARG(Lk > 0 || max_cache > 0 || Lq == 0, "attention: no keys to attend to");
  DX_CHECK_ARG(q && k && v && out, "attention: null pointer");
  DX_CHECK_ARG(al16(q) && al16(k) && al16(v) && al16(out) && (!cache || al16(cache)),
               "attention: pointers must be 16-byte aligned");
  {
    // Rows start 16-byte aligned: every stride a multiple of 16 bytes.
    const int64_t per16 = 16 / es;
    DX_CHECK_ARG(q_sb % per16 == 0 && q_sl % per16 == 0 && q_sh % per16 == 0 &&
                     k_sb % per16 == 0 && k_sl % per16 == 0 && k_sh % per16 == 0 &&
                     v_sb % per16 == 0 && v_sl % per16 == 0 && v_sh % per16 == 0 &&
                     o_sb % per16 == 0 && o_sl % per16 == 0 && o_sh % per16 == 0 &&
                     (!cache || (c_plane % per16 == 0 && c_sb % per16 == 0 &&
                                 c_ss % per16 == 0 && c_sh % per16 == 0)),
                 "attention: strides must be multiples of %lld elements (16 bytes)",
                 (long long)per16);
  }
  {
    // Key/value rows are addressed with 32-bit byte offsets per (batch, head).
    const int64_t rows = max_cache + Lk;
    const int64_t stride = std::max({cache ? c_ss : int64_t(0), k_sl, v_sl});
    DX_CHECK_ARG(rows * stride * es < (int64_t(1) << 31),
                 "attention: %lld rows of stride %lld exceed 32-bit offsets", (long long)rows,
                 (long long)stride);
  }
  if (B * Lq == 0) return DX_OK;
  Plan p{};
  AnyPlan pa{};
  int64_t need;
  if (!general) {
    p = make_plan(B, Lq, Lk, H, D, cache_len, cache_lens);
    DX_CHECK_ARG(p.items < (int64_t(1) << 31), "attention: grid too large");
    need = p.ws_bytes;
  } else {
    // The workspace query takes no dtype: at head dims 64 and 128 it reports
    // the 16-bit kernels' bytes, and fp32 calls split no more than fits them.
    const int64_t cap =
        D == 64 || D == 128 ? make_plan(B, Lq, Lk, H, D, cache_len, cache_lens).ws_bytes : -1;
    pa = plan_any(B, Lq, Lk, H, D, max_cache, cap, device_cus());
    DX_CHECK_ARG(pa.items < (int64_t(1) << 31), "attention: grid too large");
    need = pa.ws_bytes;
  }
  if (need > 0 && from_scratch) {
    if (need > kScratchBytes) {
      set_error("attention (no-alloc): this call needs %lld bytes of workspace, more than the "
                "%lld-byte static scratch; use dx_blockwise_causal_attention with a workspace",
                (long long)need, (long long)kScratchBytes);
      return DX_EWORKSPACE;
    }
    const int rc = scratch_on_device(&workspace, static_cast<hipStream_t>(stream));
    if (rc != DX_OK) return rc;
    ws_bytes = kScratchBytes;
  }
  if (need > 0) {
    if (!workspace || ws_bytes < need) {
      set_error("attention: workspace of %lld bytes needed, %lld given", (long long)need,
                (long long)ws_bytes);
      return DX_EWORKSPACE;
    }
    DX_CHECK_ARG(al16(workspace), "attention: workspace must be 16-byte aligned");
  }
  if (general) {
    AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q); a.q_sb = q_sb; a.q_sl = q_sl; a.q_sh = q_sh;
    a.k = static_cast<const uint16_t*>(k); a.k_sb = k_sb; a.k_sl = k_sl; a.k_sh = k_sh;
    a.v = static_cast<const uint16_t*>(v); a.v_sb = v_sb; a.v_sl = v_sl; a.v_sh = v_sh;
    a.ck = static_cast<const uint16_t*>(cache);
    a.cv = cache ? reinterpret_cast<const uint16_t*>(static_cast<const char*>(cache) +
                                                     c_plane * es)
                 : nullptr;
    a.c_sb = c_sb; a.c_ss = c_ss; a.c_sh = c_sh;
    a.out = static_cast<uint16_t*>(out); a.o_sb = o_sb; a.o_sl = o_sl; a.o_sh = o_sh;
    // Partials after the counter region, which this kernel never writes:
    // [items * 64 rows][D] fp32 values, then [items * 64 rows] {m, l}.
    char* ws = static_cast<char*>(workspace);
    a.ws_o = need ? reinterpret_cast<uint16_t*>(ws + kCounterRegion) : nullptr;
    a.ws_ml = need ? reinterpret_cast<float*>(ws + kCounterRegion + pa.items * 64 * D * 4)
                   : nullptr;
    a.starts = starts; a.starts_i64 = starts_dtype == DX_I64; a.n_blocks = int(n_blocks);
    a.B = int(B); a.H = int(H); a.Lq = int(Lq); a.Lk = int(Lk);
    a.kv_group = int(H / Hkv);
    a.causal = causal != 0;
    a.n_qtiles = pa.n_qtiles;
    a.n_splits = pa.splits;
    // Signed: the kernel masks by selection after the product, so a negative
    // or zero scale needs no special form.
    a.scale_log2 = softmax_scale * 1.4426950408889634f;
    a.cache_len = int(cache_len);
    a.cache_len_dev = cache_len_dev;
    a.n_seg = cache_lens ? int(B) : 0;
    for (int64_t i = 0; cache_lens && i < B; ++i) a.seg_cache[i] = int(cache_lens[i]);
    const hipError_t e = launch_any(a, dtype, int(D), pa, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_error("attention: launch failed: %s", hipGetErrorString(e));
      return DX_ELAUNCH;
    }
    return DX_OK;
  }
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_sb; a.q_sl = q_sl; a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(k); a.k_sb = k_sb; a.k_sl = k_sl; a.k_sh = k_sh;
  a.v = static_cast<const uint16_t*>(v); a.v_sb = v_sb; a.v_sl = v_sl; a.v_sh = v_sh;
  a.ck = static_cast<const uint16_t*>(cache);
  a.cv = cache ? static_cast<const uint16_t*>(cache) + c_plane : nullptr;
  a.c_sb = c_sb; a.c_ss = c_ss; a.c_sh = c_sh;
  a.out = static_cast<uint16_t*>(out); a.o_sb = o_sb; a.o_sl = o_sl; a.o_sh = o_sh;
  // Workspace: [counters][f16 partial values][fp32 records].
  char* ws = static_cast<char*>(workspace);
  // The merge state of kernels that merge their splits themselves: the
  // decode kernel always, the paired and dual-stream kernels when planned so.
  a.counters = p.counter_bytes && (p.kernel == kDecode || p.pmerge)
                   ? reinterpret_cast<int32_t*>(ws)
                   : nullptr;
  a.fast_ticks = tuning(DX_TUNE_ATTN_MERGE) == 2 ? 0u : kFastTicks;
  a.spread = a.counters != nullptr && p.spread;
  a.ws_o = p.ws_bytes ? reinterpret_cast<uint16_t*>(ws + p.counter_bytes) : nullptr;
  a.ws_ml = p.ws_bytes ? reinterpret_cast<float*>(a.ws_o + p.partials * p.prow * D) : nullptr;
  a.starts = starts; a.starts_i64 = starts_dtype == DX_I64; a.n_blocks = int(n_blocks);
  a.B = int(B); a.H = int(H); a.Lq = int(Lq); a.Lk = int(Lk);
  a.kv_group = int(H / Hkv);
  a.causal = causal != 0;
  a.n_qtiles = p.n_qtiles;
  a.bm = p.bm;
  a.comb_chunks = int(combine_bpt(D, std::min<int64_t>(p.bm, Lq), p.kernel == kDual));
  // A negative scale enters as a negated q (exact) and |scale|, so the kernel
  // only ever multiplies scores by a non-negative factor.
  a.negate_q = softmax_scale < 0.f;
  // The kernel multiplies scores by c = |scale| log2(e) and relies on c > 0
  // (masked scores are -inf, and exp2(-inf * c) must be 0, not NaN). A zero
  // scale becomes the smallest normal float: every finite score times it is
  // below 2^-24 in magnitude, so each visible key still gets exp2(~0) = 1
  // exactly -- the reference's uniform softmax over the visible keys.
  a.scale_log2 = std::max(fabsf(softmax_scale) * 1.4426950408889634f, FLT_MIN);
  a.cache_len = int(cache_len);
  a.cache_len_dev = cache_len_dev;
  a.n_splits = p.uniform_splits;
  a.n_seg = p.n_seg;
  for (int i = 0; i < p.n_seg; ++i) {
    a.seg_b[i] = p.seg_b[i];
    a.seg_splits[i] = p.seg_splits[i];
    a.seg_cache[i] = p.seg_cache[i];
  }
  for (int i = 0; i <= p.n_seg && p.n_seg > 0; ++i) {
    a.seg_base[i] = p.seg_base[i];
    a.comb_base[i] = p.comb_base[i];
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (D == 128)
    e = dtype == DX_BF16 ? launch_d<128, bf16_t>(a, p, st) : launch_d<128, f16_t>(a, p, st);
  else
    e = dtype == DX_BF16 ? launch_d<64, bf16_t>(a, p, st) : launch_d<64, f16_t>(a, p, st);
  if (e != hipSuccess) {
    set_error("attention: launch failed: %s", hipGetErrorString(e));
    return DX_ELAUNCH;
  }
  return DX_OK;
}

// QK-norm + rotary prologue (with the cache write when appending), then
// attention over the cache and the rotated rows: SelfAttention's decode step
// in one call. The prologue stays its own kernel: run inside the attention
// launch (the first workgroups normalising the tokens while the others fetch
// cache tiles, the attention waiting for them before reading q) it measured
// 4.4 us slower per call at every cache length from 1,245 to 32,768 keys, since
// q is needed before the first tile and the in-launch hand-over costs three
// dependent memory round trips under load.
int fused_entry(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k,
                int64_t k_sb, int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb,
                int64_t v_sl, int64_t v_sh, int io_dtype, const void* qw, const void* kw,
                int wdt, const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl,
                int tdt, float eps, int interleaved, void* q_out, void* k_out, void* cache,
                int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, int64_t capacity,
                int64_t cache_len, int append, void* out, int64_t o_sb, int64_t o_sl,
                int64_t o_sh, int64_t B, int64_t L, int64_t H, int64_t D, const void* starts,
                int starts_dtype, int64_t n_blocks, int causal, float softmax_scale,
                void* workspace, int64_t ws_bytes, void* stream) {
  DX_CHECK_ARG(cache_len >= 0, "qk_norm_rope_attention: negative cache_len");
  DX_CHECK_ARG(D == 64 || D == 128, "qk_norm_rope_attention: head_dim %lld unsupported (64 or "
               "128)", (long long)D);
  int rc = rope_validate(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, io_dtype,
                         qw, kw, wdt, cos, cos_sl, sin, sin_sl, tdt, q_out, k_out, cache,
                         c_plane, c_sb, c_ss, c_sh, capacity, cache_len, nullptr, B, L, H, D,
                         append != 0);
  if (rc) return rc;
  DX_CHECK_ARG(cache_len == 0 || cache, "qk_norm_rope_attention: cache_len > 0 needs a cache");
  if (B * L == 0) return DX_OK;
  rc = append ? dx_qk_norm_rope_append(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl,
                                       v_sh, io_dtype, qw, kw, wdt, cos, cos_sl, sin, sin_sl,
                                       tdt, q_out, k_out, cache, c_plane, c_sb, c_ss, c_sh,
                                       capacity, cache_len, B, L, H, D, eps, interleaved, stream)
              : dx_qk_norm_rope(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, io_dtype, qw, kw, wdt,
                                cos, cos_sl, sin, sin_sl, tdt, q_out, k_out, B, L, H, D, eps,
                                interleaved, stream);
  if (rc) return rc;
  // The rotated q and k are [B, L, H, D], contiguous (stride 0 for a size-1 dim).
  const int64_t hd = H * D, sb = B == 1 ? 0 : L * hd, sl = L == 1 ? 0 : hd;
  return attention_entry(q_out, sb, sl, D, k_out, sb, sl, D, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, io_dtype, B, L, L, H,
                         H, D, cache_len, nullptr, nullptr, starts, starts_dtype, n_blocks,
                         causal, softmax_scale, workspace, ws_bytes, stream);
}

}  // namespace
}  // namespace dx

using namespace dx;

extern "C" int dx_qk_norm_rope_attention(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    int io_dtype, const void* q_weight, const void* k_weight, int weight_dtype,
    const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl, int table_dtype,
    float eps, int interleaved, void* q_out, void* k_out, void* cache, int64_t c_plane,
    int64_t c_sb, int64_t c_ss, int64_t c_sh, int64_t capacity, int64_t cache_len, int append,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh, int64_t B, int64_t L, int64_t H,
    int64_t D, const void* block_starts, int starts_dtype, int64_t n_blocks, int causal,
    float softmax_scale, void* workspace, int64_t workspace_bytes, void* stream) {
  return fused_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, io_dtype,
                     q_weight, k_weight, weight_dtype, cos, cos_sl, sin, sin_sl, table_dtype, eps,
                     interleaved, q_out, k_out, cache, c_plane, c_sb, c_ss, c_sh, capacity,
                     cache_len, append, out, o_sb, o_sl, o_sh, B, L, H, D, block_starts,
                     starts_dtype, n_blocks, causal, softmax_scale, workspace, workspace_bytes,
                     stream);
}

extern "C" int dx_blockwise_causal_attention(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t Hkv, int64_t D, int64_t cache_len, const void* block_starts,
    int starts_dtype, int64_t n_blocks, int causal, float softmax_scale, void* workspace,
    int64_t workspace_bytes, void* stream) {
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         Hkv, D, cache_len, nullptr, nullptr, block_starts, starts_dtype,
                         n_blocks, causal, softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int dx_blockwise_causal_attention_noalloc(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t Hkv, int64_t D, int64_t cache_len, const void* block_starts,
    int starts_dtype, int64_t n_blocks, int causal, float softmax_scale, void* stream) {
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         Hkv, D, cache_len, nullptr, nullptr, block_starts, starts_dtype,
                         n_blocks, causal, softmax_scale, nullptr, 0, stream,
                         /*from_scratch=*/true);
}

extern "C" int dx_blockwise_causal_attention_dev(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t Hkv, int64_t D, const void* cache_len_dev, int64_t cache_capacity,
    const void* block_starts, int starts_dtype, int64_t n_blocks, int causal,
    float softmax_scale, void* workspace, int64_t workspace_bytes, void* stream) {
  DX_CHECK_ARG(cache_len_dev != nullptr, "attention: device cache length pointer is null");
  DX_CHECK_ARG((reinterpret_cast<uintptr_t>(cache_len_dev) & 3u) == 0,
               "attention: device cache length must be a 4-byte aligned int32");
  DX_CHECK_ARG(cache_capacity > 0 && cache, "attention: a device cache length needs a cache of "
               "positive capacity");
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         Hkv, D, cache_capacity, nullptr,
                         static_cast<const int32_t*>(cache_len_dev), block_starts, starts_dtype,
                         n_blocks, causal, softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int dx_blockwise_causal_attention_varlen(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t Hkv, int64_t D, const int64_t* cache_lens, const void* block_starts,
    int starts_dtype, int64_t n_blocks, int causal, float softmax_scale, void* workspace,
    int64_t workspace_bytes, void* stream) {
  DX_CHECK_ARG(cache_lens != nullptr, "attention varlen: cache_lens is null");
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         Hkv, D, 0, cache_lens, nullptr, block_starts, starts_dtype, n_blocks,
                         causal, softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int64_t dx_attention_workspace_bytes(int64_t B, int64_t Lq, int64_t Lk, int64_t H,
                                                int64_t D, int64_t cache_len,
                                                const int64_t* cache_lens) {
  if (B < 0 || Lq < 0 || Lk < 0 || H <= 0 || !any_head_dim(D) || cache_len < 0 ||
      (cache_lens && B > kMaxSeg)) {
    set_error("attention_workspace_bytes: bad shape");
    return -DX_EINVAL;
  }
  int64_t max_cache = cache_len;
  if (cache_lens) {
    max_cache = 0;
    for (int64_t i = 0; i < B; ++i) {
      if (cache_lens[i] < 0) {
        set_error("attention_workspace_bytes: negative cache length");
        return -DX_EINVAL;
      }
      max_cache = std::max(max_cache, cache_lens[i]);
    }
  }
  if (B * Lq == 0) return 0;
  // Head dims 64 and 128: the 16-bit kernels' plan (an fp32 call of that
  // shape fits its partials in the same bytes); the others: the general
  // kernel's, whatever the dtype.
  if (D == 64 || D == 128) return make_plan(B, Lq, Lk, H, D, cache_len, cache_lens).ws_bytes;
  return plan_any(B, Lq, Lk, H, D, max_cache, -1, device_cus()).ws_bytes;
}

#ifdef DX_TIMELINE
// The timeline build's stamps (the words are described at g_timeline):
// decode rows first, then the merge kernel's (start, end) pairs. Synchronous.
extern "C" int64_t dx_timeline_words() {
  return int64_t(sizeof(dx::g_timeline) + sizeof(dx::g_timeline_merge)) / 8;
}
extern "C" int dx_timeline_read(uint64_t* host) {
  hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(dx::g_timeline), sizeof(dx::g_timeline),
                                     0, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    e = hipMemcpyFromSymbol(host + sizeof(dx::g_timeline) / 8, HIP_SYMBOL(dx::g_timeline_merge),
                            sizeof(dx::g_timeline_merge), 0, hipMemcpyDeviceToHost);
  return int(e);
}
extern "C" int dx_timeline_clear() {
  static const uint64_t zeros[sizeof(dx::g_timeline) / 8] = {};
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(dx::g_timeline), zeros, sizeof(dx::g_timeline), 0,
                                   hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpyToSymbol(HIP_SYMBOL(dx::g_timeline_merge), zeros, sizeof(dx::g_timeline_merge),
                          0, hipMemcpyHostToDevice);
  return int(e);
}
#endif
