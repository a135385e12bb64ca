// Split-K QKV projection GEMM for decode-sized chunks (M <= 128 tokens) on gfx950.
//
// y = x W^T for the q, k and v weights ([H*D][C] each) of a chunk x [M][C]. At
// M = 83 the product is weight-streaming bound: 57 MB of weights against
// 0.5 MB of activations, 83 FLOP per weight byte. The kernel therefore reads
// every weight byte once, as full 128-byte lines, from as many CUs as the
// chip has, and keeps enough of it in flight to cover HBM latency. Two forms
// share the grid and the partial tiles: the default DMA form (qkv_dma_kernel,
// below: waves of 64 features, weights and activations DMA'd into LDS)
// and the register-ring form described here (dx_set_tuning DX_TUNE_QKV_WAVES
// 2 or 4), whose operand reads per MFMA bind it to the LDS bandwidth:
//
//  * Workgroup = NW waves; wave w owns 32 consecutive output features (rows of
//    one weight), the workgroup 32 NW of them, over one K split of C / S. The
//    grid is (3 H D / 32 NW) x S workgroups; the split is the fastest index,
//    so with S dividing 8 every XCD sees one split's activation slice.
//  * MFMA v_mfma_f32_32x32x16: output features on M, tokens on N (NM tiles of
//    32 tokens). The reduction index is permuted within each 128-wide K chunk:
//    lane (row r, half g) supplies elements [64 g + 8 j, +8) at step j, for
//    both operands.
//  * Weights are read 4 rows x 256 contiguous bytes per wave instruction (a
//    read-only probe of this matrix streams at 5.1 TB/s in that pattern,
//    against 4.0-4.8 TB/s reading 32 rows per instruction), kept in a register
//    ring DW - 1 chunks ahead, and written to a per-wave LDS chunk from which
//    the MFMA operands are read. The activation chunk [32 NM][128] is staged
//    once per workgroup in LDS and read by all waves; its global loads ride in
//    the same ring, because loads complete in order (a wait for a late
//    activation load would also wait for every weight load before it). LDS
//    chunks are double-buffered, 16-byte pieces XOR-swizzled by row.
//  * Each split writes its fp32 partial tile to part[s][m][n] with
//    non-temporal stores (the epilogue reads them from other XCDs, so no L2
//    reuse is lost; measured 0.5 us faster per call than plain stores). The
//    epilogue kernel (qk_norm_rope.hip) sums the splits in order, adds the
//    bias, rounds once to the io type and continues with the QK norm and
//    rotary.
#include "qkv_gemm.h"

#include <algorithm>
#include <cstdlib>

namespace dx {
namespace {

constexpr int kChunk = 128;             // K elements per pipeline step
constexpr int kRing = 4;                // weight/activation prefetch ring (chunks)
constexpr int kStep = kChunk * kRing;   // a K split is a whole number of rings
constexpr int kPieces = kChunk / 8;     // 16-byte pieces per row of a chunk
constexpr int kRowBytes = 2 * kChunk;   // bytes per row of a chunk
constexpr int kBufWord3 = 0x00020000;   // gfx9-family raw buffer descriptor word 3

template <typename T> struct ProjMfma;
template <> struct ProjMfma<bf16_t> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct ProjMfma<f16_t> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// LDS byte offset of 16-byte piece q of row r in a [rows][kChunk] chunk buffer;
// pieces are XOR-swizzled by the row so that the operand reads (32 rows, one
// piece each) spread over the banks.
__device__ __forceinline__ int piece_at(int r, int q) {
  return r * kRowBytes + 16 * (q ^ (r & (kPieces - 1)));
}

template <typename T, int NW, int NM, int DW>
__global__ __launch_bounds__(64 * NW) void qkv_gemm_kernel(QkvGemmArgs a) {
  constexpr int kRows = 32 * NM;                     // activation rows staged (tokens, padded)
  constexpr int kXBuf = kRows * kRowBytes;           // one activation chunk
  constexpr int kWBuf = 32 * kRowBytes;              // one wave's weight chunk
  constexpr int kPPT = kRows * kPieces / (64 * NW);  // activation pieces per thread per chunk
  constexpr int kSteps = kChunk / 16;                // MFMA k-steps per chunk
  constexpr int kWLoads = 32 * kPieces / 64;         // weight pieces per lane per chunk
  static_assert(kPPT * 64 * NW == kRows * kPieces, "pieces must spread evenly over the threads");
  static_assert(DW % 2 == 0, "LDS buffer parity must follow the ring slot");
  __shared__ __attribute__((aligned(16))) uint8_t xs[2 * kXBuf];
  __shared__ __attribute__((aligned(16))) uint8_t ws[2 * NW * kWBuf];

  const int tid = int(threadIdx.x), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, r = lane & 31;
  const int split = int(blockIdx.x) % a.S, tile = int(blockIdx.x) / a.S;
  const int n0 = tile * 32 * NW;  // first output feature of the workgroup
  const int plane = n0 / a.HD;
  const int k0 = split * a.Kc;
  const int nc = a.Kc / kChunk;

  // Weight loads: instruction i covers rows 4 i .. 4 i + 3 of the wave's 32, each
  // 256 contiguous bytes (lane: row 4 i + lane / 16, piece lane % 16).
  const uint16_t* wsrc = plane == 0 ? a.w[0] : plane == 1 ? a.w[1] : a.w[2];
  const int64_t wstride = plane == 0 ? a.w_row[0] : plane == 1 ? a.w_row[1] : a.w_row[2];
  const int wrow0 = n0 - plane * a.HD + 32 * wave + (lane >> 4);
  const int wpiece = lane & 15;
  const uint16_t* wp = wsrc + int64_t(wrow0) * wstride + k0 + 8 * wpiece;
  uint8_t* const wlds = ws + wave * kWBuf;

  // Activation pieces this thread stages, as byte offsets into a raw buffer
  // descriptor over x: rows past M get an offset past the descriptor's end,
  // which loads zeros without touching memory (13 of 96 rows at M = 83).
  const __amdgpu_buffer_rsrc_t xr_src = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), (short)0, int(a.x_bytes), kBufWord3);
  uint32_t xb_off[kPPT];
  int xoff[kPPT];
#pragma unroll
  for (int i = 0; i < kPPT; ++i) {
    const int p = tid + i * 64 * NW;
    const int row = p / kPieces, q = p % kPieces;
    const int m = min(row, a.M - 1);
    const int b = m / a.L, l = m - b * a.L;
    xb_off[i] = row < a.M ? uint32_t(2 * (b * a.x_sb + l * a.x_sl + k0 + 8 * q)) : 0x80000000u;
    xoff[i] = piece_at(row, q);
  }
  auto load_x = [&](int c, u32x4 (&xr)[kPPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPPT; ++i)
      xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            xr_src, int(xb_off[i] + uint32_t(2 * kChunk * c)),
                                            0, 0));
  };
  auto load_w = [&](int c, u32x4 (&wr)[kWLoads]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      wr[i] = *reinterpret_cast<const u32x4*>(wp + int64_t(4 * i) * wstride + c * kChunk);
  };
  auto store = [&](int buf, const u32x4 (&xr)[kPPT], const u32x4 (&wr)[kWLoads])
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPPT; ++i)
      *reinterpret_cast<u32x4*>(xs + buf * kXBuf + xoff[i]) = xr[i];
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      *reinterpret_cast<u32x4*>(wlds + buf * NW * kWBuf + piece_at(4 * i + (lane >> 4), wpiece)) =
          wr[i];
  };

  f32x16 acc[NM];
#pragma unroll
  for (int t = 0; t < NM; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;

  // The chunk count is a multiple of DW (host-checked), so the loop body is
  // straight-line: ring slots and LDS buffers are compile-time indices, and
  // past the last chunk the prefetches re-read it (no branches, which would
  // make the compiler's load-counter waits conservative).
  u32x4 wr[DW][kWLoads];
  u32x4 xr[DW][kPPT];
#pragma unroll
  for (int d = 0; d < DW - 1; ++d) {
    load_x(min(d, nc - 1), xr[d]);
    load_w(min(d, nc - 1), wr[d]);
  }
  store(0, xr[0], wr[0]);
  __syncthreads();

  for (int c0 = 0; c0 < nc; c0 += DW) {
#pragma unroll
    for (int u = 0; u < DW; ++u) {
      const int c = c0 + u;
      // Chunk c + DW - 1 into the ring slot chunk c - 1 used.
      const int cp = min(c + DW - 1, nc - 1);
      load_x(cp, xr[(u + DW - 1) % DW]);
      load_w(cp, wr[(u + DW - 1) % DW]);
      // Keep the prefetch at the top of the step: moved below the waits of
      // this step, it would be waited for too (loads complete in order).
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* xb = xs + (u & 1) * kXBuf;
      const uint8_t* wb = wlds + (u & 1) * NW * kWBuf;
#pragma unroll
      for (int j = 0; j < kSteps; ++j) {
        const u32x4 wa = *reinterpret_cast<const u32x4*>(wb + piece_at(r, kSteps * g + j));
        u32x4 bx[NM];
#pragma unroll
        for (int t = 0; t < NM; ++t)
          bx[t] = *reinterpret_cast<const u32x4*>(xb + piece_at(t * 32 + r, kSteps * g + j));
#pragma unroll
        for (int t = 0; t < NM; ++t) acc[t] = ProjMfma<T>::run(wa, bx[t], acc[t]);
      }
      __builtin_amdgcn_sched_barrier(0);
      store((u + 1) & 1, xr[(u + 1) % DW], wr[(u + 1) % DW]);
      __syncthreads();
    }
  }

  // Partial tile: lane holds features 8 (e / 4) + 4 g + e % 4 of the wave's 32, token r.
  const int64_t n3 = 3 * int64_t(a.HD);
  const int nf = n0 + 32 * wave + 4 * g;
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    const int m = t * 32 + r;
    if (m < a.M) {
      float* dst = a.part + (int64_t(split) * a.M + m) * n3 + nf;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_nontemporal_store(
            f32x4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]},
            reinterpret_cast<f32x4*>(dst + 8 * q));
    }
  }
}

// LDS-lean form: 64 output features per wave (two 32-row MFMA blocks), so
// each activation piece read from LDS feeds two MFMAs: a k-step reads 2 + NM
// pieces per lane for 2 NM MFMAs, where waves of 32 features read 1 + NM for
// NM (at the Wan-5B chunk 2.5 KB instead of 4 KB of operand reads per three
// MFMAs, below the LDS's 128 bytes per clock with room for the staging
// writes). Two waves cover the workgroup's 128 features; with NWV = 4 a second
// pair takes the other half of every chunk's k-steps, and the pairs' sums are
// added through LDS before the store. Weights and
// activations land in LDS by DMA, with no register ring: per K chunk of KC the
// workgroup's 128 weight rows and 32 NM activation rows are cut into 1 KB
// pieces (512 / KC rows of 2 KC contiguous bytes each), and each lane fetches
// the logical 16-byte piece that belongs at its swizzled slot. NS stages form
// a ring: chunk c's weights and activations are issued NS - 1 chunks ahead,
// and loads complete in order, so waiting for chunk c's pieces leaves the
// NS - 2 younger chunks in flight. Per chunk a wave waits for its pieces of
// chunk c, the barrier publishes them and frees the stage chunk c - 1 used,
// the wave issues chunk c + NS - 1 into that stage and computes chunk c. Same
// grid, splits and fp32 partial tiles as the register-ring form.
template <int KC>
__device__ __forceinline__ int slot_at(int r, int q) {
  return r * 2 * KC + 16 * (q ^ (r & (KC / 8 - 1)));
}

template <typename T, int NM, int KC, int NS, int NWV>
__global__ __launch_bounds__(64 * NWV) void qkv_dma_kernel(QkvGemmArgs a) {
  constexpr int kF = 128;                            // output features per workgroup
  constexpr int kKH = NWV / 2;                       // waves sharing a feature half (K halves)
  constexpr int kRowB = 2 * KC;                      // bytes per row of a chunk
  constexpr int kWBytes = kF * kRowB;                // weight part of a stage
  constexpr int kXBytes = 32 * NM * kRowB;           // activation part of a stage
  constexpr int kStage = kWBytes + kXBytes;
  constexpr int kWP = kWBytes / (1024 * NWV);        // weight pieces per wave per chunk
  constexpr int kXP = kXBytes / (1024 * NWV);        // activation pieces per wave per chunk
  constexpr int kRPP = 1024 / kRowB;                 // rows per piece
  constexpr int kQ = KC / 8;                         // 16-byte pieces per row
  constexpr int kSteps = KC / 16;                    // MFMA k-steps per chunk
  constexpr int kAhead = (NS - 2) * (kWP + kXP);     // pieces in flight past chunk c's
  static_assert(NWV == 2 || NWV == 4, "two waves, or two per feature half");
  static_assert(kXBytes % (1024 * NWV) == 0 && kWBytes % (1024 * NWV) == 0,
                "pieces split evenly over the waves");
  static_assert(kSteps % kKH == 0, "k-steps split evenly over the K halves");
  static_assert(NS >= 2 && kAhead <= 63, "in-flight pieces fit the vmcnt counter");
  static_assert(kKH == 1 || 2 * 64 * 2 * NM * 16 * 4 <= NS * kStage, "exchange fits the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];

  const int tid = int(threadIdx.x), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fw = wave & 1, kh = wave >> 1;  // feature half, K half of each chunk
  const int g = lane >> 5, r = lane & 31;
  const int split = int(blockIdx.x) % a.S, tile = int(blockIdx.x) / a.S;
  const int n0 = tile * kF;
  const int plane = n0 / a.HD;
  const int k0 = split * a.Kc;
  const int nc = a.Kc / KC;
  const uint32_t lds0 = uint32_t(uintptr_t((__attribute__((address_space(3))) uint8_t*)lds));

  // Weight rows of the tile, from column k0, through a descriptor whose base
  // is the tile's first row (offsets stay 32-bit: 128 rows of the weight).
  const uint16_t* wsrc = plane == 0 ? a.w[0] : plane == 1 ? a.w[1] : a.w[2];
  const int64_t wstride = plane == 0 ? a.w_row[0] : plane == 1 ? a.w_row[1] : a.w_row[2];
  const __amdgpu_buffer_rsrc_t wr_src = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(wsrc + int64_t(n0 - plane * a.HD) * wstride + k0), (short)0,
      0x7ffffff0, kBufWord3);
  // Piece i of this wave is piece NWV i + wave of the part; lane l fills slot
  // l % kQ of its row, which holds the row's logical piece (l % kQ) ^ (row % kQ).
  uint32_t woff[kWP];
#pragma unroll
  for (int i = 0; i < kWP; ++i) {
    const int row = kRPP * (NWV * i + wave) + lane / kQ;
    const int q = (lane % kQ) ^ (row & (kQ - 1));
    woff[i] = uint32_t(2 * (int64_t(row) * wstride + 8 * q));
  }
  // Activation pieces the same way; rows past M read zeros.
  const __amdgpu_buffer_rsrc_t xr_src = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), (short)0, int(a.x_bytes), kBufWord3);
  uint32_t xoff[kXP];
#pragma unroll
  for (int i = 0; i < kXP; ++i) {
    const int row = kRPP * (NWV * i + wave) + lane / kQ;
    const int q = (lane % kQ) ^ (row & (kQ - 1));
    const int m = min(row, a.M - 1);
    const int b = m / a.L, l = m - b * a.L;
    xoff[i] = row < a.M ? uint32_t(2 * (b * a.x_sb + l * a.x_sl + k0 + 8 * q)) : 0x80000000u;
  }
  auto issue = [&](int c) __attribute__((always_inline)) {
    const uint32_t st = lds0 + uint32_t((c % NS) * kStage) + 1024u * uint32_t(wave);
    const uint32_t kb = uint32_t(2 * KC * c);
#pragma unroll
    for (int i = 0; i < kWP; ++i) dma_piece_at(wr_src, st + 1024u * NWV * i, woff[i] + kb);
#pragma unroll
    for (int i = 0; i < kXP; ++i)
      dma_piece_at(xr_src, st + kWBytes + 1024u * NWV * i,
                   xoff[i] >= 0x80000000u ? xoff[i] : xoff[i] + kb);
  };

  f32x16 acc[2][NM];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int t = 0; t < NM; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[b][t][e] = 0.f;

#pragma unroll
  for (int c = 0; c < NS - 1; ++c)
    if (c < nc) issue(c);
  for (int c = 0; c < nc; ++c) {
    // Chunk c's pieces have landed; the NS - 2 younger chunks may still fly.
    if (c + NS - 2 < nc) wait_vmcnt<kAhead>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (c + NS - 1 < nc) issue(c + NS - 1);
    const uint8_t* wb = lds + (c % NS) * kStage + fw * 64 * kRowB;
    const uint8_t* xb = lds + (c % NS) * kStage + kWBytes;
#pragma unroll
    for (int jj = 0; jj < kSteps / kKH; ++jj) {
      const int j = kh * (kSteps / kKH) + jj;
      u32x4 wa[2], bx[NM];
#pragma unroll
      for (int b = 0; b < 2; ++b)
        wa[b] = *reinterpret_cast<const u32x4*>(wb + slot_at<KC>(32 * b + r, kSteps * g + j));
#pragma unroll
      for (int t = 0; t < NM; ++t)
        bx[t] = *reinterpret_cast<const u32x4*>(xb + slot_at<KC>(t * 32 + r, kSteps * g + j));
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < NM; ++t) acc[b][t] = ProjMfma<T>::run(wa[b], bx[t], acc[b][t]);
    }
  }

  if (kKH == 2) {
    // The second K half's sums join the first's through the (now idle) ring:
    // f32x4 (fw, b, t, q) of every lane, consecutive lanes adjacent.
    f32x4* ex = reinterpret_cast<f32x4*>(lds);
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < NM; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            ex[(((fw * 2 + b) * NM + t) * 4 + q) * 64 + lane] =
                f32x4{acc[b][t][4 * q], acc[b][t][4 * q + 1], acc[b][t][4 * q + 2],
                      acc[b][t][4 * q + 3]};
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int t = 0; t < NM; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 o = ex[(((fw * 2 + b) * NM + t) * 4 + q) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[b][t][4 * q + e] += o[e];
        }
  }

  // Partial tile: lane holds features 8 (e / 4) + 4 g + e % 4 of block b's 32,
  // token t 32 + r.
  const int64_t n3 = 3 * int64_t(a.HD);
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int nf = n0 + 64 * fw + 32 * b + 4 * g;
#pragma unroll
    for (int t = 0; t < NM; ++t) {
      const int m = t * 32 + r;
      if (m < a.M) {
        float* dst = a.part + (int64_t(split) * a.M + m) * n3 + nf;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          __builtin_nontemporal_store(f32x4{acc[b][t][4 * q], acc[b][t][4 * q + 1],
                                            acc[b][t][4 * q + 2], acc[b][t][4 * q + 3]},
                                      reinterpret_cast<f32x4*>(dst + 8 * q));
      }
    }
  }
}

// Chunk width, stages and waves of the DMA form, measured at the Wan-5B chunk
// (us per layer, GEMM + epilogue, 30 layers per graph). Two waves: KC 64 with
// 3 stages 21.82-21.83, 4 stages 22.00-22.06, 5 stages 22.47; KC 32 with 9
// stages 25.89 (twice the barriers); KC 128 with 2 stages 25.21 (one chunk in
// flight). Four waves (each feature half's k-steps split over two waves, so
// the MFMAs use all four SIMDs; the halves' sums meet through LDS at the end):
// KC 64 with 3 stages 21.47-21.55, 4 stages 21.43, KC 128 with 2 stages 24.76.
// The register-ring form (four waves of 32 features) takes 25.4-25.5.
constexpr int kDmaKC = 64, kDmaNS = 3, kDmaWaves = 4;

template <typename T, int NM>
hipError_t launch_dma_nm(const QkvGemmArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((qkv_dma_kernel<T, NM, kDmaKC, kDmaNS, kDmaWaves>), dim3(blocks),
                     dim3(64 * kDmaWaves), 0, st, a);
  return hipGetLastError();
}

template <typename T, int NW, int NM>
hipError_t launch_nm(const QkvGemmArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((qkv_gemm_kernel<T, NW, NM, kRing>), dim3(blocks), dim3(64 * NW), 0, st,
                     a);
  return hipGetLastError();
}

template <typename T, int NW>
hipError_t launch_nw(const QkvGemmArgs& a, int blocks, hipStream_t st) {
  const int nm = (a.M + 31) / 32;
  switch (nm) {
    case 1: return launch_nm<T, NW, 1>(a, blocks, st);
    case 2: return launch_nm<T, NW, 2>(a, blocks, st);
    case 3: return launch_nm<T, NW, 3>(a, blocks, st);
    default: return launch_nm<T, NW, 4>(a, blocks, st);
  }
}

template <typename T>
hipError_t launch_t(const QkvGemmArgs& a, const QkvPlan& p, hipStream_t st) {
  if (p.dma) {
    const int blocks = (3 * a.HD / 128) * a.S;
    switch ((a.M + 31) / 32) {
      case 1: return launch_dma_nm<T, 1>(a, blocks, st);
      case 2: return launch_dma_nm<T, 2>(a, blocks, st);
      case 3: return launch_dma_nm<T, 3>(a, blocks, st);
      default: return launch_dma_nm<T, 4>(a, blocks, st);
    }
  }
  const int blocks = (3 * a.HD / (32 * p.waves)) * a.S;
  return p.waves == 2 ? launch_nw<T, 2>(a, blocks, st) : launch_nw<T, 4>(a, blocks, st);
}

}  // namespace

// Form and K splits: the DMA form (128 output features per workgroup) unless
// dx_set_tuning(DX_TUNE_QKV_WAVES) asks for the register-ring form with 2 or 4
// waves; the split count (dividing C into whole rings of 512) whose grid comes
// closest to one workgroup per CU, fewer splits on a tie. At the Wan-5B chunk
// that is 3 splits, 216 workgroups (the register-ring GEMM measured 19.9 us
// there, against 26.7 us at 6 splits and 22-24 us at 2: each a read-bandwidth
// and partial-traffic trade). DX_TUNE_QKV_SPLITS overrides the split count.
QkvPlan plan_qkv(int64_t M, int64_t C, int64_t HD) {
  QkvPlan p{};
  const long waves = tuning(DX_TUNE_QKV_WAVES);
  p.dma = waves != 2 && waves != 4;
  p.waves = waves == 2 ? 2 : 4;
  const int64_t tiles = 3 * HD / (32 * p.waves);
  int s = 1;
  int64_t best = -1;
  for (int c = 1; c <= 16; ++c) {
    if (C % (int64_t(kStep) * c) != 0) continue;
    const int64_t gap = tiles * c > 256 ? tiles * c - 256 : 256 - tiles * c;
    if (best < 0 || gap < best) { best = gap; s = c; }
  }
  const long forced = tuning(DX_TUNE_QKV_SPLITS);
  if (forced >= 1 && forced <= 16 && C % (int64_t(kStep) * forced) == 0) s = int(forced);
  p.splits = s;
  p.workspace_bytes = int64_t(s) * M * 3 * HD * int64_t(sizeof(float));
  return p;
}

hipError_t launch_qkv_gemm(const QkvGemmArgs& a, const QkvPlan& p, int dtype, hipStream_t st) {
  return dtype == DX_BF16 ? launch_t<bf16_t>(a, p, st) : launch_t<f16_t>(a, p, st);
}

}  // namespace dx
