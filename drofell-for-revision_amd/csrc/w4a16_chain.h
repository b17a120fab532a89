// Internal interface of the decode chain (w4a16_chain.hip) for the C ABI
// (w4a16_capi.hip).  Not installed; the public ABI is include/drofell_w4a16.h.
#pragma once

#include "w4a16_internal.h"

namespace dw4 {

// ---------------------------------------------------------------------------
// Decode chain (w4a16_chain.hip): one persistent launch over a list of
// projections ("links") at small M, each link's input read only after the
// links it depends on have completed on every workgroup.  The table lives in
// a caller-owned device buffer laid out as: ChainHeader, the links, then one
// 64-bit progress word per workgroup.
// ---------------------------------------------------------------------------
constexpr int kChainMaxM = 4;          // rows (one 16-row MFMA tile, rows 0..3 kept)
constexpr int kChainMaxK = 16384;      // activation row held in LDS
constexpr int kChainMaxWorkgroups = 1024;
constexpr int kChainLinkBytes = 128;
constexpr int kChainHeadBytes = 256;
constexpr int kChainSameX = 1;         // link flag: x already in LDS (previous link's x)
constexpr int kChainPublish = 2;       // link flag: a later link waits for this one

struct ChainLinkDev {
  const uint32_t* pq;
  const uint32_t* pz;
  const uint32_t* ps32;
  const uint16_t* x;
  const uint16_t* bias;
  const uint16_t* res;
  uint16_t* y;
  int64_t ldx, ldres, ldy;
  int K, N, G;
  uint32_t gmag;   // chunk -> group: g = umulhi(c, gmag) (0: group = chunk)
  int after;       // -1, or: read x once links 0..after are complete everywhere
  int flags;       // kChainSameX, kChainPublish
  int rot;         // workgroup rotation of the strip ranges, in [0, workgroups)
  uint32_t kcmag;  // ceil(2^32 / (K / 128)) (0 when K = 128)
  unsigned char pad_to_record[kChainLinkBytes - 112];
};
// the kernel indexes the table as ChainLinkDev[] and the host writes one
// record every kChainLinkBytes: the two strides must be the same
static_assert(sizeof(ChainLinkDev) == kChainLinkBytes, "link record stride");

struct ChainHeader {
  uint64_t epoch;     // launches completed (written by the last workgroup to finish)
  uint32_t finished;  // workgroups finished in the running launch
  uint32_t timed_out; // a dependency wait gave up (results of that launch invalid)
  int count, M, workgroups, pad;
};
static_assert(sizeof(ChainHeader) <= kChainHeadBytes, "chain header");

__host__ __device__ inline size_t chain_progress_offset(int count) {
  return ((size_t)kChainHeadBytes + (size_t)count * kChainLinkBytes + 255) & ~(size_t)255;
}
inline size_t chain_buffer_bytes(int count) {
  return chain_progress_offset(count) + (size_t)kChainMaxWorkgroups * sizeof(uint64_t);
}

struct ChainPlan {
  int count, m, workgroups, waves, ring, max_k, max_strips, max_groups;
  size_t smem;
};
// LDS bytes of a chain workgroup for a plan's ring depth.
size_t chain_smem_bytes(int m, int max_k, int max_strips, int max_groups, int count, int waves,
                        int ring);
// Picks the ring depth (units in flight per streaming wave) and LDS size.
bool plan_chain(ChainPlan& p);
hipError_t launch_chain(const ChainPlan& p, void* chain, hipStream_t stream);

}  // namespace dw4
