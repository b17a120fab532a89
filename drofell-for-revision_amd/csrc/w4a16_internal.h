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
#define DW4_DECODE_PREFETCH 8
#endif

namespace dw4 {

constexpr int kChunkK = 128;  // sorted rows per packed chunk
constexpr int kStripN = 16;   // columns per strip
constexpr int kDecodeWaves = DW4_DECODE_WAVES;
constexpr int kDecodePrefetch = DW4_DECODE_PREFETCH;
constexpr int kDecodeMaxM = 64;      // four 16-row MFMA tiles
constexpr int kDecodeAutoMaxM = 16;  // DW4_PATH_AUTO picks decode up to this M
// LDS a decode workgroup may use for its staged activations and metadata;
// a K range whose slice does not fit is split across workgroups.
constexpr size_t kDecodeLdsBudget = 64 * 1024;
constexpr int kMetaBytes = 40;  // one (strip, group) scales+zeros record

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

struct DecodePlan {
  int splits;   // workgroups along K per strip
  int cps;      // 128-row chunks per split
  size_t smem;  // dynamic LDS bytes per workgroup
};

// LDS bytes a decode workgroup needs for a K range of `cps` chunks.
inline size_t decode_smem_bytes(int m, int cps, int gs) {
  const size_t rows = (size_t)cps * kChunkK;
  const size_t groups = rows / (size_t)gs + 2;
  const size_t staged = (size_t)m * (rows + 8) * 2 + groups * kMetaBytes;
  const size_t mt = (size_t)((m + 15) / 16);
  const size_t red = (size_t)kDecodeWaves * mt * 64 * 16;
  const size_t b = staged > red ? staged : red;
  return (b + 15) & ~(size_t)15;
}

// Fewest K splits whose per-workgroup slice fits the LDS budget.
inline DecodePlan plan_decode(int m, int k, int gs) {
  const int kc = k / kChunkK;
  DecodePlan p{1, kc, decode_smem_bytes(m, kc, gs)};
  for (int s = 1; s <= kc; ++s) {
    const int cps = (kc + s - 1) / s;
    const size_t bytes = decode_smem_bytes(m, cps, gs);
    if (bytes <= kDecodeLdsBudget || s == kc) {
      p.splits = (kc + cps - 1) / cps;
      p.cps = cps;
      p.smem = bytes;
      break;
    }
  }
  return p;
}

hipError_t launch_repack(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                         const int32_t* perm, uint32_t* pq, uint32_t* pz, uint16_t* ps,
                         int K, int N, int G, hipStream_t stream);
hipError_t launch_decode(const GemmArgs& a, const DecodePlan& p, float* part, hipStream_t stream);
hipError_t launch_prefill(const GemmArgs& a, const PrefillPlan& plan, float* part,
                          hipStream_t stream);
hipError_t launch_dequant(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                          const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs,
                          int G, hipStream_t stream);

}  // namespace dw4
