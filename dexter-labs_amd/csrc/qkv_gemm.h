// Split-K projection GEMM behind dx_qkv_norm_rope (internal to the library).
#pragma once

#include "dx_common.h"

namespace dx {

// y[s][m][n] = sum over k in split s of x[m][k] * w_plane(n)[n % HD][k], in fp32, where
// plane = n / HD selects the q, k or v weight ([HD][C] rows, nn.Linear layout).
struct QkvGemmArgs {
  const uint16_t* x; int64_t x_sb, x_sl;  // activation [B][L][C], element strides
  uint32_t x_bytes;                        // bytes from x to the end of its last row (< 2^31)
  const uint16_t* w[3]; int64_t w_row[3];  // q, k, v weights: row strides in elements
  float* part;                             // [S][M][3 HD] fp32 partial products
  int M, L, C, HD, S, Kc;                  // tokens, L, in features, H*D, splits, C / S
};

// Plan of one projection launch on the current device.
struct QkvPlan {
  bool dma;    // the LDS-lean DMA form (waves of 64 features, 128 per workgroup)
  int waves;   // register-ring form: waves per workgroup = 32-row output subtiles
  int splits;  // K splits (partials)
  int64_t workspace_bytes;
};

QkvPlan plan_qkv(int64_t M, int64_t C, int64_t HD);
hipError_t launch_qkv_gemm(const QkvGemmArgs& a, const QkvPlan& p, int dtype, hipStream_t st);

}  // namespace dx
