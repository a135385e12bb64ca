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
// and V^T is staged in LDS with each 16-key group stored in the order
// [0-3, 8-11, 4-7, 12-15] so each A operand is one 16-byte LDS read.
//
// Masking. Per workgroup the host-independent bounds kv_min / kv_max (over its
// queries' visible-key ends, read from block_starts on the device) split the
// key tiles into three kinds: tiles below kv_min need no mask, tiles from
// kv_max on are never visited (whole future blocks are skipped), and only the
// straddling tiles are masked elementwise. Rows at or beyond kv_max are
// zero-filled in LDS instead of loaded, so nothing a workgroup cannot see
// reaches its arithmetic.
//
// Work decomposition. One workgroup = NW waves = 32*NW queries of one
// (batch, head), over one contiguous range of key tiles. Short query chunks
// over long caches (decode) split the key range over several workgroups
// (split-KV) and a second kernel merges the partial (max, sum, acc) triples.
// Workgroups are issued heaviest-first (latest query tile first), and when
// B*H is a multiple of 8 all workgroups of one (batch, head) land on the same
// XCD (workgroup i runs on XCD i % 8), so that head's K/V is shared through
// one L2.
#include "dx_common.h"

#include <mutex>
#include <vector>

namespace dx {
namespace {

constexpr int kBN = 64;        // keys per tile
constexpr int kMaxVarlen = 64; // sequences with their own cache length

struct AttnArgs {
  const uint16_t* q; int64_t q_sb, q_sl, q_sh;
  const uint16_t* k; int64_t k_sb, k_sl, k_sh;
  const uint16_t* v; int64_t v_sb, v_sl, v_sh;
  const uint16_t* ck; const uint16_t* cv; int64_t c_sb, c_ss, c_sh;
  uint16_t* out; int64_t o_sb, o_sl, o_sh;
  float* ws_o;   // [partials][32*NW][D] unnormalised accumulators
  float* ws_ml;  // [partials][32*NW][2]  (running max, running sum)
  const void* starts; int starts_i64; int n_blocks;
  int B, H, Lq, Lk;
  int causal;
  int n_qtiles, n_splits, xcd_map;
  float scale_log2;  // softmax scale * log2(e)
  int varlen; int cache_len; int cache_lens[kMaxVarlen];
};

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
};

__device__ __forceinline__ int load_start(const AttnArgs& a, int i) {
  return a.starts_i64 ? int(static_cast<const int64_t*>(a.starts)[i])
                      : static_cast<const int32_t*>(a.starts)[i];
}

// End (exclusive, in current-key coordinates) of the keys query i may see.
__device__ __forceinline__ int visible_end(const AttnArgs& a, int i) {
  if (a.causal) return i + 1;
  if (a.n_blocks == 0) return a.Lk;
  int e = 0;
  int s = load_start(a, 0);
  for (int bi = 0; bi < a.n_blocks; ++bi) {
    const int nx = (bi + 1 < a.n_blocks) ? load_start(a, bi + 1) : a.Lq;
    if (s <= i && i < nx) e = max(e, nx);
    s = nx;
  }
  return min(e, a.Lq);
}

// LDS geometry: K rows padded by 8 elements (272 B for D=128: 16-lane
// groups of 16-byte reads hit 64 distinct banks); V^T rows of 64 keys padded
// to 72 elements (144 B) for the same reason.
template <int D> struct Lds {
  static constexpr int kPitch = D + 8;
  static constexpr int vPitch = kBN + 8;
  static constexpr int kElems = kBN * kPitch;
  static constexpr int vElems = D * vPitch;
};

template <int NW, int D>
struct TileRegs {
  static constexpr int NT = 64 * NW;
  static constexpr int KCH = kBN * D / 8;  // 16-byte chunks of a K tile
  static constexpr int KPT = (KCH + NT - 1) / NT;
  static constexpr int VG = 16 * D / 8;    // 4-key x 8-dim groups of a V tile
  static constexpr int VPT = (VG + NT - 1) / NT;
  u32x4 kr[KPT];
  u32x4 vr[VPT][4];

  __device__ __forceinline__ void load(const uint16_t* kc, const uint16_t* kn,
                                       const uint16_t* vc, const uint16_t* vn,
                                       int64_t c_ss, int64_t k_sl, int64_t v_sl,
                                       int cache_len, int kv_max, int j0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      kr[i] = u32x4{0, 0, 0, 0};
      if (c < KCH) {
        const int row = c / (D / 8), col = c % (D / 8);
        const int j = j0 + row;
        if (j < kv_max) {
          const uint16_t* p = j < cache_len ? kc + j * c_ss : kn + (j - cache_len) * k_sl;
          kr[i] = *reinterpret_cast<const u32x4*>(p + col * 8);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int x = tid + i * NT;
#pragma unroll
      for (int r = 0; r < 4; ++r) vr[i][r] = u32x4{0, 0, 0, 0};
      if (x < VG) {
        const int kg = x % 16, dg = x / 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + 4 * kg + r;
          if (j < kv_max) {
            const uint16_t* p = j < cache_len ? vc + j * c_ss : vn + (j - cache_len) * v_sl;
            vr[i][r] = *reinterpret_cast<const u32x4*>(p + dg * 8);
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* Ks, uint16_t* Vt) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (c < KCH) {
        const int row = c / (D / 8), col = c % (D / 8);
        *reinterpret_cast<u32x4*>(Ks + row * Lds<D>::kPitch + col * 8) = kr[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int x = tid + i * NT;
      if (x < VG) {
        const int kg = x % 16, dg = x / 16;
        const int qd = kg % 4;
        const int phys = 16 * (kg / 4) + 8 * (qd % 2) + 4 * (qd / 2);
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          const int w = d / 2;
          uint32_t lo, hi;
          if (d % 2 == 0) {
            lo = (vr[i][0][w] & 0xffffu) | (vr[i][1][w] << 16);
            hi = (vr[i][2][w] & 0xffffu) | (vr[i][3][w] << 16);
          } else {
            lo = (vr[i][0][w] >> 16) | (vr[i][1][w] & 0xffff0000u);
            hi = (vr[i][2][w] >> 16) | (vr[i][3][w] & 0xffff0000u);
          }
          *reinterpret_cast<u32x2*>(Vt + (dg * 8 + d) * Lds<D>::vPitch + phys) = u32x2{lo, hi};
        }
      }
    }
  }
};

struct Item { int b, h, qtile, split; };

__device__ __forceinline__ Item decode_item(const AttnArgs& a, int item) {
  const int nbh = a.B * a.H;
  int bh, r;
  if (a.xcd_map) {
    const int xcd = item & 7, slot = item >> 3, g8 = nbh >> 3;
    bh = xcd + 8 * (slot % g8);
    r = slot / g8;
  } else {
    bh = item % nbh;
    r = item / nbh;
  }
  Item it;
  it.b = bh / a.H;
  it.h = bh % a.H;
  it.split = r % a.n_splits;
  it.qtile = a.n_qtiles - 1 - r / a.n_splits;
  return it;
}

template <int NW, int D, typename T>
__global__ __launch_bounds__(64 * NW) void attn_fwd_kernel(AttnArgs a) {
  constexpr int BM = 32 * NW;
  constexpr int KS = D / 16;  // MFMA k-steps over head_dim
  constexpr int DT = D / 32;  // 32-wide head_dim tiles of the output
  __shared__ __attribute__((aligned(16))) uint16_t Ks[Lds<D>::kElems];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[Lds<D>::vElems];
  __shared__ int red_min[NW], red_max[NW];

  const Item it = decode_item(a, blockIdx.x);
  const int b = it.b, h = it.h;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 5, n = lane & 31;
  const int qi = it.qtile * BM + wave * 32 + n;
  const bool qvalid = qi < a.Lq;
  const int cache_len = a.varlen ? a.cache_lens[b] : a.cache_len;

  // Visible-key end of this lane's query, and the workgroup's bounds.
  const int my_end = qvalid ? cache_len + visible_end(a, qi) : 0;
  int vmin = qvalid ? my_end : 0x7fffffff, vmax = my_end;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    vmin = min(vmin, __shfl_xor(vmin, off, 64));
    vmax = max(vmax, __shfl_xor(vmax, off, 64));
  }
  if (lane == 0) { red_min[wave] = vmin; red_max[wave] = vmax; }
  __syncthreads();
  int kv_min = red_min[0], kv_max = red_max[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) { kv_min = min(kv_min, red_min[w]); kv_max = max(kv_max, red_max[w]); }

  const int n_tiles = (kv_max + kBN - 1) / kBN;
  const int t_begin = int((int64_t(it.split) * n_tiles) / a.n_splits);
  const int t_end = int((int64_t(it.split + 1) * n_tiles) / a.n_splits);

  // Q^T operand: lane holds query n, head_dim [16s + 8g, 16s + 8g + 8) per k-step s.
  u32x4 qr[KS];
  {
    const uint16_t* qp = a.q + b * a.q_sb + int64_t(qi) * a.q_sl + h * a.q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qr[s] = qvalid ? *reinterpret_cast<const u32x4*>(qp + 16 * s + 8 * g) : u32x4{0, 0, 0, 0};
  }

  const uint16_t* kc = a.ck + b * a.c_sb + h * a.c_sh;
  const uint16_t* vc = a.cv + b * a.c_sb + h * a.c_sh;
  const uint16_t* kn = a.k + b * a.k_sb + h * a.k_sh;
  const uint16_t* vn = a.v + b * a.v_sb + h * a.v_sh;

  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  TileRegs<NW, D> regs;
  if (t_begin < t_end)
    regs.load(kc, kn, vc, vn, a.c_ss, a.k_sl, a.v_sl, cache_len, kv_max, t_begin * kBN);

  for (int t = t_begin; t < t_end; ++t) {
    const int j0 = t * kBN;
    __syncthreads();  // previous tile's LDS reads are done
    regs.store(Ks, Vt);
    __syncthreads();
    if (t + 1 < t_end)
      regs.load(kc, kn, vc, vn, a.c_ss, a.k_sl, a.v_sl, cache_len, kv_max, j0 + kBN);

    // S^T tile: two 32-key halves.
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x16{};
      const uint16_t* kp = Ks + (32 * kt + n) * Lds<D>::kPitch + 8 * g;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        s[kt] = Mfma<T>::run(*reinterpret_cast<const u32x4*>(kp + 16 * ks), qr[ks], s[kt]);
    }

    // Scale into the exp2 domain; mask only tiles that straddle a boundary.
    const bool full = j0 + kBN <= kv_min;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[kt][r] * a.scale_log2;
        if (!full) {
          const int key = j0 + 32 * kt + 8 * (r / 4) + 4 * g + (r % 4);
          x = key < my_end ? x : -INFINITY;
        }
        s[kt][r] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    // Nothing visible yet: use 0 as the exponent base so every exp2 is of -inf
    // (exactly 0) and never of (-inf) - (-inf).
    const float base = m_new == -INFINITY ? 0.f : m_new;
    const float corr = exp2f(m_run - base);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(s[kt][r] - base);
        s[kt][r] = p;
        psum += p;
      }
    l_run = l_run * corr + psum;
#pragma unroll
    for (int d = 0; d < DT; ++d) acc[d] *= corr;

    // O^T += V^T P^T, 16 keys per MFMA.
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        u32x4 pb;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pb[e] = Mfma<T>::pack(s[kt][8 * hf + 2 * e], s[kt][8 * hf + 2 * e + 1]);
        const int u = 2 * kt + hf;
        const uint16_t* vp = Vt + n * Lds<D>::vPitch + 16 * u + 8 * g;
#pragma unroll
        for (int d = 0; d < DT; ++d)
          acc[d] = Mfma<T>::run(*reinterpret_cast<const u32x4*>(vp + 32 * d * Lds<D>::vPitch),
                                pb, acc[d]);
      }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (!qvalid) return;
  if (a.n_splits == 1) {
    const float inv = 1.0f / l_tot;  // 0 visible keys: 0 * inf = NaN, as the reference
    uint16_t* op = a.out + b * a.o_sb + int64_t(qi) * a.o_sl + h * a.o_sh;
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
    const int64_t pidx =
        (int64_t(b * a.H + h) * a.n_qtiles + it.qtile) * a.n_splits + it.split;
    const int row = wave * 32 + n;
    float* po = a.ws_o + (pidx * BM + row) * D;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4 + 4 * g;
        *reinterpret_cast<f32x4*>(po + dim) =
            f32x4{acc[d][4 * r4], acc[d][4 * r4 + 1], acc[d][4 * r4 + 2], acc[d][4 * r4 + 3]};
      }
    if (g == 0) {
      float* pm = a.ws_ml + (pidx * BM + row) * 2;
      pm[0] = m_run;
      pm[1] = l_tot;
    }
  }
}

// Merge split-KV partials: out = sum_s w_s acc_s / sum_s w_s l_s with
// w_s = exp2(m_s - max_s m_s). Each thread owns 4 consecutive dims of a row.
template <int NW, int D, typename T>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  constexpr int BM = 32 * NW;
  constexpr int TPR = D / 4;           // threads per row
  constexpr int RPB = 256 / TPR;       // rows per block
  constexpr int BPT = (BM + RPB - 1) / RPB;  // blocks per q-tile
  const int blk = blockIdx.x;
  const int chunk = blk % BPT;
  const int rest = blk / BPT;
  const int qtile = rest % a.n_qtiles;
  const int bh = rest / a.n_qtiles;
  const int row = chunk * RPB + threadIdx.x / TPR;
  const int dim = 4 * (threadIdx.x % TPR);
  const int qi = qtile * BM + row;
  if (row >= BM || qi >= a.Lq) return;
  const int b = bh / a.H, h = bh % a.H;
  const int64_t p0 = (int64_t(bh) * a.n_qtiles + qtile) * a.n_splits;
  float mmax = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s)
    mmax = fmaxf(mmax, a.ws_ml[((p0 + s) * BM + row) * 2]);
  const float base = mmax == -INFINITY ? 0.f : mmax;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
  for (int s = 0; s < a.n_splits; ++s) {
    const float* pm = a.ws_ml + ((p0 + s) * BM + row) * 2;
    const float w = exp2f(pm[0] - base);
    l += w * pm[1];
    const f32x4 x = *reinterpret_cast<const f32x4*>(a.ws_o + ((p0 + s) * BM + row) * D + dim);
    o += w * x;
  }
  const float inv = 1.0f / l;
  uint16_t* op = a.out + b * a.o_sb + int64_t(qi) * a.o_sl + h * a.o_sh + dim;
  u32x2 w2;
  w2[0] = Mfma<T>::pack(o[0] * inv, o[1] * inv);
  w2[1] = Mfma<T>::pack(o[2] * inv, o[3] * inv);
  *reinterpret_cast<u32x2*>(op) = w2;
}

// ---------------------------------------------------------------------------
// Host side: launch planning shared by the workspace query and the launch.
// ---------------------------------------------------------------------------
struct Plan {
  int nw, n_qtiles, n_splits;
  int64_t items;
  int64_t ws_bytes;
};

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

Plan make_plan(int64_t B, int64_t Lq, int64_t H, int64_t D, int64_t max_cache_len) {
  Plan p{};
  int64_t nw = (Lq + 31) / 32;
  p.nw = int(nw < 1 ? 1 : (nw > 4 ? 4 : nw));
  const int64_t bm = 32 * p.nw;
  p.n_qtiles = int((Lq + bm - 1) / bm);
  const int64_t base = B * H * p.n_qtiles;
  const int64_t tiles = (max_cache_len + Lq + kBN - 1) / kBN;
  const int64_t target = 2 * int64_t(device_cus());
  int64_t splits = 1;
  if (base > 0 && base * 4 < target * 3 && tiles >= 4) {
    splits = (target + base - 1) / base;
    const int64_t cap = tiles / 2;
    if (splits > cap) splits = cap;
    if (splits < 1) splits = 1;
  }
  p.n_splits = int(splits);
  p.items = base * splits;
  p.ws_bytes = splits > 1 ? base * splits * bm * (D + 2) * int64_t(sizeof(float)) : 0;
  return p;
}

template <int NW, int D, typename T>
hipError_t launch_nw(const AttnArgs& a, const Plan& p, hipStream_t st) {
  hipLaunchKernelGGL((attn_fwd_kernel<NW, D, T>), dim3(unsigned(p.items)), dim3(64 * NW), 0, st,
                     a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.n_splits == 1) return e;
  constexpr int RPB = 256 / (D / 4);
  constexpr int BPT = (32 * NW + RPB - 1) / RPB;
  const int64_t blocks = int64_t(a.B) * a.H * p.n_qtiles * BPT;
  hipLaunchKernelGGL((attn_combine_kernel<NW, D, T>), dim3(unsigned(blocks)), dim3(256), 0, st,
                     a);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t launch_d(const AttnArgs& a, const Plan& p, hipStream_t st) {
  switch (p.nw) {
    case 1: return launch_nw<1, D, T>(a, p, st);
    case 2: return launch_nw<2, D, T>(a, p, st);
    case 3: return launch_nw<3, D, T>(a, p, st);
    default: return launch_nw<4, D, T>(a, p, st);
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int attention_entry(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k,
                    int64_t k_sb, int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb,
                    int64_t v_sl, int64_t v_sh, const void* cache, int64_t c_plane,
                    int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out, int64_t o_sb,
                    int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                    int64_t H, int64_t D, int64_t cache_len, const int64_t* cache_lens,
                    const void* starts, int starts_dtype, int64_t n_blocks, int causal,
                    float softmax_scale, void* workspace, int64_t ws_bytes, void* stream) {
  DX_CHECK_ARG(dtype == DX_BF16 || dtype == DX_F16,
               "attention: dtype code %d unsupported (bf16 or f16)", dtype);
  DX_CHECK_ARG(D == 64 || D == 128, "attention: head_dim %lld unsupported (64 or 128)",
               (long long)D);
  DX_CHECK_ARG(B >= 0 && Lq >= 0 && H > 0, "attention: bad shape");
  DX_CHECK_ARG(Lk == Lq,
               "attention: k/v length %lld must equal q length %lld (the block mask is "
               "[q_len, cache_len + q_len])",
               (long long)Lk, (long long)Lq);
  DX_CHECK_ARG(n_blocks >= 0 && (n_blocks == 0 || starts),
               "attention: block_boundaries pointer missing");
  DX_CHECK_ARG(starts_dtype == DX_I32 || starts_dtype == DX_I64 || n_blocks == 0,
               "attention: block_boundaries must be int32 or int64");
  if (cache_lens) {
    DX_CHECK_ARG(B <= kMaxVarlen, "attention varlen: B=%lld exceeds %d", (long long)B,
                 kMaxVarlen);
  }
  int64_t max_cache = cache_len;
  if (cache_lens) {
    max_cache = 0;
    for (int64_t i = 0; i < B; ++i) {
      DX_CHECK_ARG(cache_lens[i] >= 0, "attention varlen: negative cache length");
      if (cache_lens[i] > max_cache) max_cache = cache_lens[i];
    }
  }
  DX_CHECK_ARG(max_cache >= 0, "attention: negative cache_len");
  DX_CHECK_ARG(max_cache == 0 || cache, "attention: cache_len > 0 needs a cache");
  DX_CHECK_ARG(max_cache + Lq < (int64_t(1) << 30), "attention: sequence too long");
  DX_CHECK_ARG(q && k && v && out, "attention: null pointer");
  DX_CHECK_ARG(al16(q) && al16(k) && al16(v) && al16(out) && (!cache || al16(cache)),
               "attention: pointers must be 16-byte aligned");
  DX_CHECK_ARG(q_sb % 8 == 0 && q_sl % 8 == 0 && q_sh % 8 == 0 && k_sb % 8 == 0 &&
                   k_sl % 8 == 0 && k_sh % 8 == 0 && v_sb % 8 == 0 && v_sl % 8 == 0 &&
                   v_sh % 8 == 0 && o_sb % 8 == 0 && o_sl % 8 == 0 && o_sh % 8 == 0 &&
                   (!cache || (c_plane % 8 == 0 && c_sb % 8 == 0 && c_ss % 8 == 0 &&
                               c_sh % 8 == 0)),
               "attention: strides must be multiples of 8 elements");
  if (B * Lq == 0) return DX_OK;
  const Plan p = make_plan(B, Lq, H, D, max_cache);
  DX_CHECK_ARG(p.items < (int64_t(1) << 31), "attention: grid too large");
  if (p.ws_bytes > 0) {
    if (!workspace || ws_bytes < p.ws_bytes) {
      set_error("attention: workspace of %lld bytes needed, %lld given",
                (long long)p.ws_bytes, (long long)ws_bytes);
      return DX_EWORKSPACE;
    }
    DX_CHECK_ARG(al16(workspace), "attention: workspace must be 16-byte aligned");
  }
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_sb; a.q_sl = q_sl; a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(k); a.k_sb = k_sb; a.k_sl = k_sl; a.k_sh = k_sh;
  a.v = static_cast<const uint16_t*>(v); a.v_sb = v_sb; a.v_sl = v_sl; a.v_sh = v_sh;
  a.ck = static_cast<const uint16_t*>(cache);
  a.cv = cache ? static_cast<const uint16_t*>(cache) + c_plane : nullptr;
  a.c_sb = c_sb; a.c_ss = c_ss; a.c_sh = c_sh;
  a.out = static_cast<uint16_t*>(out); a.o_sb = o_sb; a.o_sl = o_sl; a.o_sh = o_sh;
  const int64_t bm = 32 * p.nw;
  const int64_t partials = B * H * p.n_qtiles * p.n_splits;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = p.ws_bytes ? a.ws_o + partials * bm * D : nullptr;
  a.starts = starts; a.starts_i64 = starts_dtype == DX_I64; a.n_blocks = int(n_blocks);
  a.B = int(B); a.H = int(H); a.Lq = int(Lq); a.Lk = int(Lk);
  a.causal = causal != 0;
  a.n_qtiles = p.n_qtiles; a.n_splits = p.n_splits;
  a.xcd_map = (B * H) % 8 == 0;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.varlen = cache_lens != nullptr;
  a.cache_len = int(cache_len);
  if (cache_lens)
    for (int64_t i = 0; i < B; ++i) a.cache_lens[i] = int(cache_lens[i]);
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

}  // namespace
}  // namespace dx

using namespace dx;

extern "C" int dx_blockwise_causal_attention(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t D, int64_t cache_len, const void* block_starts, int starts_dtype,
    int64_t n_blocks, int causal, float softmax_scale, void* workspace,
    int64_t workspace_bytes, void* stream) {
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         D, cache_len, nullptr, block_starts, starts_dtype, n_blocks, causal,
                         softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int dx_blockwise_causal_attention_varlen(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh, const void* k, int64_t k_sb,
    int64_t k_sl, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh, void* out,
    int64_t o_sb, int64_t o_sl, int64_t o_sh, int dtype, int64_t B, int64_t Lq, int64_t Lk,
    int64_t H, int64_t D, const int64_t* cache_lens, const void* block_starts,
    int starts_dtype, int64_t n_blocks, int causal, float softmax_scale, void* workspace,
    int64_t workspace_bytes, void* stream) {
  DX_CHECK_ARG(cache_lens != nullptr, "attention varlen: cache_lens is null");
  return attention_entry(q, q_sb, q_sl, q_sh, k, k_sb, k_sl, k_sh, v, v_sb, v_sl, v_sh, cache,
                         c_plane, c_sb, c_ss, c_sh, out, o_sb, o_sl, o_sh, dtype, B, Lq, Lk, H,
                         D, 0, cache_lens, block_starts, starts_dtype, n_blocks, causal,
                         softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int64_t dx_attention_workspace_bytes(int64_t B, int64_t Lq, int64_t Lk, int64_t H,
                                                int64_t D, int64_t max_cache_len) {
  if (B < 0 || Lq < 0 || H <= 0 || (D != 64 && D != 128) || max_cache_len < 0 || Lk != Lq) {
    set_error("attention_workspace_bytes: bad shape");
    return -DX_EINVAL;
  }
  if (B * Lq == 0) return 0;
  return make_plan(B, Lq, H, D, max_cache_len).ws_bytes;
}
