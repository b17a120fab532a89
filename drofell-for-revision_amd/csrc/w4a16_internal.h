// Internal interface between the C ABI (w4a16_capi.hip) and the kernels
// (w4a16_kernels.hip).  Not installed; the public ABI is include/drofell_w4a16.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifndef DW4_DECODE_WAVES
#define DW4_DECODE_WAVES 8
#endif
#ifndef DW4_DECODE_PREFETCH
#define DW4_DECODE_PREFETCH 4
#endif

namespace dw4 {

constexpr int kChunkK = 128;  // sorted rows per packed chunk
constexpr int kStripN = 16;   // columns per strip
constexpr int kDecodeWaves = DW4_DECODE_WAVES;
constexpr int kDecodePrefetch = DW4_DECODE_PREFETCH;
constexpr int kDecodeMaxM = 64;  // four 16-row MFMA tiles

struct GemmArgs {
  int M, K, N, gs, G;
  const uint16_t* x;
  int64_t ldx;
  const uint32_t* pq;
  const uint32_t* pz;
  const uint16_t* ps;
  const int32_t* perm;
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldy;
};

struct PrefillPlan {
  int bm, bn, splits;
};

hipError_t launch_repack(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                         const int32_t* perm, uint32_t* pq, uint32_t* pz, uint16_t* ps,
                         int K, int N, int G, hipStream_t stream);
hipError_t launch_gather_x(const uint16_t* x, int64_t ldx, const int32_t* perm, uint16_t* xg,
                           int M, int K, hipStream_t stream);
hipError_t launch_decode(const GemmArgs& a, hipStream_t stream);
hipError_t launch_prefill(const GemmArgs& a, const PrefillPlan& plan, float* part,
                          hipStream_t stream);
hipError_t launch_dequant(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                          const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs,
                          int G, hipStream_t stream);

}  // namespace dw4
