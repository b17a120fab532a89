// Internal interface of the transposed product (w4a16_transpose.hip) for the
// C ABI (w4a16_capi.hip).  Not installed; the public ABI is include/drofell_w4a16.h.
#pragma once

#include "w4a16_internal.h"

namespace dw4 {

// Transposed product out[M, K] = g[M, N] @ W^T (PEFT backward).
struct GemmTArgs {
  int M, K, N, gs, G;
  const uint16_t* g;
  int64_t ldg;
  const uint32_t* pq;
  const uint32_t* pz;
  const uint16_t* ps;
  const int32_t* perm;  // sorted row -> checkpoint row (act-order) or null
  uint16_t* out;
  int64_t ldo;
};
struct GemmTPlan {
  int ns = 1;   // N-ranges (their fp32 partials are summed in order)
  int spr = 0;  // strips per N-range
};
GemmTPlan plan_gemm_t(int m, int k, int n, int cus);
size_t gemm_t_ws_bytes(const GemmTPlan& p, int m, int k);
hipError_t launch_gemm_t(const GemmTArgs& a, const GemmTPlan& p, float* part, hipStream_t stream);

}  // namespace dw4
