// Internal interface between the C ABI (w4a16_capi.hip) and the kernel
// files (w4a16_decode.hip, w4a16_kernels.hip, w4a16_prefill.hip, ...).  Not
// installed; the public ABI is include/drofell_w4a16.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>


namespace dw4 {

constexpr int kChunkK = 128;  // sorted rows per packed chunk
constexpr int kStripN = 16;   // columns per strip
constexpr int kDecodeMaxM = 64;      // four 16-row MFMA tiles
constexpr int kDecodeAutoMaxM = 48;        // DW4_PATH_AUTO picks decode up to this M,
constexpr int kDecodeAutoMaxMNarrow = 64;  // and up to this M when strips <= CUs
constexpr int kGroupDecodeMaxM = 32;       // grouped decode launches: two row tiles
constexpr int kMetaBytes = 40;  // one (strip, group) scales+zeros record
constexpr int kMetaWords = kMetaBytes / 4;
#ifndef DW4_DECODE_UMAX
#define DW4_DECODE_UMAX 4  // deepest weight ring (chunks in flight per wave)
#endif
#ifndef DW4_DECODE_REG_MIN_M
#define DW4_DECODE_REG_MIN_M 5  // smallest M for the register-fed decode kernel
#endif
#ifndef DW4_DECODE_NARROW_WAVES
#define DW4_DECODE_NARROW_WAVES 16  // waves per workgroup when strips <= CUs and M <= 4
#endif
constexpr int kDecodeUMax = DW4_DECODE_UMAX;
constexpr int kDecodeNarrowWaves = DW4_DECODE_NARROW_WAVES;
constexpr size_t kLdsPerCu = 160 * 1024;
// Act-order decode at M = 1 (XG): the staged kernel copies the activation
// row (K <= kXgMaxK) into LDS and each lane gathers at most kXgUnits 16-byte
// units from it by perm, so a wave stages at most kXgUnits * 4 chunks.
constexpr int kXgMaxK = 16384;
constexpr int kXgUnits = 4;

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
  // optional residual r [M, N] (row stride ldres): y = fp16(fp16(x @ W (+ bias)) + r).
  // r is y itself (same stride; every element is read and then written by
  // one thread) or does not overlap y.
  const uint16_t* res = nullptr;
  int64_t ldres = 0;
};

// Matrices launched together.  They share x, M, K and the group size; each
// has its own packed buffers, perm, bias and output.  Decode launches give
// item i the workgroups [wg0[i], wg0[i+1]).
constexpr int kGroupMax = 4;
struct GroupArgs {
  int count;
  GemmArgs a[kGroupMax];
};

// Kernel-side table of a grouped launch (passed by value).
struct Items {
  const uint32_t* pq[kGroupMax];
  const uint32_t* pz[kGroupMax];
  const uint16_t* ps[kGroupMax];
  const int32_t* perm[kGroupMax];
  const uint16_t* bias[kGroupMax];
  uint16_t* y[kGroupMax];
  int64_t ldy[kGroupMax];
  const uint16_t* res[kGroupMax];
  int64_t ldres[kGroupMax];
  int n[kGroupMax];
  int wg0[kGroupMax + 1];
  int count;
};

// Prefill launch: row tile bm (16: 16x16x32 MFMA kernel; 32, 64, 128:
// 32x32x16 MFMA kernel), column tile bn (128 or 256), split-K factor.
struct PrefillPlan {
  int bm, bn, splits;
  int waves = 8;  // LDS-streamed kernel: 8 (one workgroup per CU) or 4 (two)
};

struct DecodePlan {
  int splits;   // workgroups along K per strip
  int cps;      // 128-row chunks per split
  int waves;    // waves per workgroup (4, 8 or 16)
  size_t smem;  // dynamic LDS bytes per workgroup
  bool reg = false;  // register-fed kernel (activations not staged in LDS)
  int ss = 1;        // strips per workgroup of the register-fed kernel
  bool xg = false;   // act-order M = 1: gather from an LDS copy of x (+ K * 2 bytes of LDS)
};
constexpr int kDecodeRegMinM = DW4_DECODE_REG_MIN_M;

// LDS bytes of a decode workgroup's staging regions: each of its waves
// stages the activation rows (kChunkK + 8 halfs per row) and the metadata
// records (rec dwords per chunk) of its own per_wave chunks; 16-aligned.
__host__ __device__ inline size_t decode_staged_bytes(int m, int per_wave, int rec, int waves) {
  const size_t b = (size_t)waves * per_wave * ((size_t)m * (kChunkK + 8) * 2 + (size_t)rec * 4);
  return (b + 15) & ~(size_t)15;
}

// LDS bytes a decode workgroup needs for a K range of `cps` chunks: the
// staging regions of ceil(cps / waves) chunks per wave, then the cross-wave
// reduction's own region (so the reduction needs no barrier ahead of it).
inline size_t decode_smem_bytes(int m, int cps, int gs, int waves) {
  const int per_wave = (cps + waves - 1) / waves;
  const int rec = (gs < kChunkK ? kChunkK / gs : 1) * kMetaWords;
  const size_t mt = (size_t)((m + 15) / 16);
  return decode_staged_bytes(m, per_wave, rec, waves) + (size_t)waves * mt * 64 * 16;
}

#ifndef DW4_REG_LDSX
#define DW4_REG_LDSX 1
#endif
// Register-fed variants that load A as whole 128-byte lines and rearrange it
// through LDS: all without act-order except those whose extra live
// registers would spill (four strips beyond one row tile with 32- or 64-row
// groups or four row tiles, two strips of four row tiles with small groups).
constexpr bool decode_reg_lx(int mt, int ss, int gpc, bool act) {
  return DW4_REG_LDSX && !act && !(ss == 4 && mt >= 2 && (gpc > 1 || mt == 4)) &&
         !(mt == 4 && ss == 2 && gpc > 1);
}

// Register-fed launch time model (microseconds), fitted to graph-replayed
// times of the Llama-2-7B shapes at M = 8..64 on a 256-CU MI355X: every
// round of workgroups costs the activation bytes one workgroup reads (~66
// GB/s per CU as whole lines, ~34 GB/s in operand order) plus its weight
// bytes (~25 GB/s per CU); a K split adds the fp32 planes and the reduce
// launch.
inline double decode_reg_cost(int m, int kc, int strips, int ss, int splits, int gpc, int cus) {
  const int cps = (kc + splits - 1) / splits;
  const int real = (kc + cps - 1) / cps;
  const int wgs = (strips + ss - 1) / ss * real;
  const int rounds = (wgs + cus - 1) / cus;
  const double a_mb = (double)m * cps * kChunkK * 2 / 1e6;
  const double w_mb = (double)ss * cps * 1024 / 1e6;
  const double a_rate = decode_reg_lx((m + 15) / 16, ss, gpc, false) ? 15.2 : 29.3;
  return rounds * (a_rate * a_mb + 40.3 * w_mb) + (real > 1 ? 3.0 + 1.4 * (real - 1) : 0.0);
}

// Waves per workgroup: enough to fill the chip with the strips available
// (one workgroup per 16-column strip), fewer for larger M whose activation
// slices are bigger.  K is split across workgroups only where the staged
// activations would not fit the LDS share of one workgroup (the CU's LDS
// divided by the workgroups it is expected to hold).  The register-fed form
// (5 <= M <= 64) takes the strips per workgroup (1, 2, 4) and K split (1, 2,
// 4, 8) of least modelled time; grouped launches (single == false) keep one
// or two strips and no split.
inline DecodePlan plan_decode(int m, int k, int n, int gs, int cus, bool single = true) {
  const int kc = k / kChunkK;
  const int strips = n / kStripN;
  if (m >= kDecodeRegMinM && m <= kDecodeMaxM) {
    DecodePlan r{1, kc, 8, 0};
    r.reg = true;
    r.ss = (strips % 2 == 0 && strips / 2 >= cus) ? 2 : 1;
    if (single) {
      const int mt = (m + 15) / 16;
      const int gpc = gs >= kChunkK ? 1 : kChunkK / gs;
      double best = decode_reg_cost(m, kc, strips, r.ss, 1, gpc, cus);
      const int sss[3] = {1, 2, 4};
      for (int ss : sss) {
        // not instantiated: four strips of three row tiles with small groups,
        // and of four row tiles (its registers spill)
        if (ss == 4 && (mt == 4 || (mt >= 3 && gpc > 1))) continue;
        for (int sp = 1; sp <= 8 && sp * 8 <= kc; sp *= 2) {
          const double c = decode_reg_cost(m, kc, strips, ss, sp, gpc, cus);
          if (c < best) {
            best = c;
            r.ss = ss;
            r.cps = (kc + sp - 1) / sp;
            r.splits = (kc + r.cps - 1) / r.cps;
          }
        }
      }
    }
    if (m <= 16 && r.ss == 1 && r.splits == 1 && strips <= cus && kc >= 32) r.waves = 16;
    r.smem = (size_t)r.waves * r.ss * ((m + 15) / 16) * 64 * 16;
    return r;
  }
  int waves = 8;
  if (strips >= 2 * cus && m <= 16) waves = 4;
  else if (strips <= cus && m <= 4) waves = kDecodeNarrowWaves;
  const int wgs_per_cu = (strips + cus - 1) / cus;
  size_t budget = kLdsPerCu / (size_t)(wgs_per_cu > 0 ? wgs_per_cu : 1) - 1024;
  if (budget > 144 * 1024) budget = 144 * 1024;
  DecodePlan p{1, kc, waves, decode_smem_bytes(m, kc, gs, waves)};
  for (int s = 1; s <= kc; ++s) {
    const int cps = (kc + s - 1) / s;
    const size_t bytes = decode_smem_bytes(m, cps, gs, waves);
    if (bytes <= budget || s == kc) {
      p.splits = (kc + cps - 1) / cps;
      p.cps = cps;
      p.smem = bytes;
      break;
    }
  }
  return p;
}

// Act-order M = 1 on the staged kernel: gather from an LDS copy of x (XG)
// where the copy fits beside the staging regions in the workgroup's LDS share
// and every wave stages at most kXgUnits * 4 chunks; groups of 128 or more.
inline void plan_decode_xg(DecodePlan& p, int m, int k, int n, int gs, int cus) {
  if (p.reg || m != 1 || k > kXgMaxK || gs % kChunkK != 0) return;
  if ((p.cps + p.waves - 1) / p.waves > kXgUnits * 4) return;
  const int strips = n / kStripN;
  const int wgs_per_cu = (strips + cus - 1) / cus;
  size_t budget = kLdsPerCu / (size_t)(wgs_per_cu > 0 ? wgs_per_cu : 1) - 1024;
  if (budget > 144 * 1024) budget = 144 * 1024;
  const size_t smem = p.smem + (size_t)k * 2;
  if (smem > budget) return;
  p.xg = true;
  p.smem = smem;
}

// DW4_PATH_AUTO's choice.  The decode kernel streams each weight once but
// every workgroup reads all M activation rows of its strips, so the prefill
// kernel wins sooner when N has more strips than there are CUs.  Up to M = 64
// decode also keeps N a little wider than the CUs where K is short (k > 0
// given): 5120^2 M=64 14.6 us against 16.8 for the prefill kernel, while
// 13824x5120 (the same 320 strips) runs 26.4 against 32.9 on prefill.
inline bool auto_decode(int m, int n, int cus, int k = 0) {
  const int strips = n / kStripN;
  return m <= kDecodeAutoMaxM ||
         (m <= kDecodeAutoMaxMNarrow &&
          (strips <= cus || (k > 0 && k <= 8192 && 4 * strips <= 5 * cus)));
}

// A kernel launched with more than 64 KiB of dynamic LDS needs that size
// allowed once per device (hipFuncSetAttribute).  `done` is the kernel's own
// per-device record (bit d: device d allowed); concurrent first calls only
// repeat the idempotent attribute call.
hipError_t allow_lds(const void* kernel, size_t bytes, std::atomic<uint64_t>& done);

hipError_t launch_repack(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                         const int32_t* perm, uint32_t* pq, uint32_t* pz, uint16_t* ps,
                         int K, int N, int G, hipStream_t stream);
hipError_t launch_decode(const GemmArgs& a, const DecodePlan& p, float* part, hipStream_t stream);
// xs[m][j] = x[m][perm[j]] for m < M, j < K (K % 8 == 0): x in the packed row order.
hipError_t launch_gather_rows(const uint16_t* x, int64_t ldx, const int32_t* perm, uint16_t* xs,
                              int K, int M, hipStream_t stream);
// Act-order calls gather x into the packed row order first (a workspace
// buffer of gather_bytes): every workgroup would otherwise gather its own
// activation slices, 8 two-byte loads at scattered addresses per 16-byte
// unit behind a dependent load of perm.
inline size_t gather_bytes(int m, int k) { return ((size_t)m * k * 2 + 255) & ~(size_t)255; }
// Workspace offset of the gathered activations after `split` bytes of
// split-K area: 256-aligned and past the arrival-counter head (declared
// below), which must stay zero between calls.
inline size_t gather_offset(size_t split);
hipError_t launch_decode_reg(const GroupArgs& g, const DecodePlan& p, float* part,
                             hipStream_t stream);
// One launch over every strip of g's matrices (decode plan with one split).
hipError_t launch_decode_group(const GroupArgs& g, const DecodePlan& p, hipStream_t stream);
// h[m, n] = fp16(silu(fp16(x @ W0 + b0)) * fp16(x @ W1 + b1)) for two matrices of equal N
// and equal perm (gate, up): one register-fed launch, workgroup s holding strip s of both.
constexpr int kPairMaxM = 32;  // largest M of launch_decode_pair
hipError_t launch_decode_pair(const GroupArgs& g, uint16_t* h, int64_t ldh, hipStream_t stream);
// bf16 activations and output, 1 <= M <= kBf16MaxM, one matrix: the
// register-fed kernel's bf16 mode, unsplit, ceil(M / 16) row tiles in one
// launch (the weights are read once for every row).  Two strips per
// workgroup where the strips fill the CUs twice (four row tiles only with
// one group per chunk: with more groups' scale and zero words they spill);
// up to 16 rows, 16 waves where one strip per workgroup leaves every wave
// two chunks or more.
constexpr int kBf16MaxM = 64;  // DW4_BF16_MAX_M of the public header
inline DecodePlan plan_decode_bf16(int m, int k, int n, int gs, int cus) {
  const int kc = k / kChunkK;
  const int strips = n / kStripN;
  DecodePlan r{1, kc, 8, 0};
  r.reg = true;
  r.ss = ((m <= 48 || gs >= kChunkK) && strips % 2 == 0 && strips / 2 >= cus) ? 2 : 1;
  if (m <= 16 && r.ss == 1 && strips <= cus && kc >= 32) r.waves = 16;
  r.smem = (size_t)r.waves * r.ss * 64 * 16;
  return r;
}
hipError_t launch_decode_reg_bf16(const GemmArgs& a, const DecodePlan& p, hipStream_t stream);
// Elementwise h = fp16(silu(g) * u) over [m, n] (row strides ldg, ldu, ldh).
hipError_t launch_silu_mul(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu,
                           uint16_t* h, int64_t ldh, int m, int n, hipStream_t stream);
// y = fp16(x * w * rsqrt(mean(x^2) + eps)) per row of [m, k].
hipError_t launch_rms_norm(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                           uint16_t* y, int64_t ldy, int m, int k, hipStream_t stream);
// Workspace of a split-K call: a fixed head of kSplitCounters int32 arrival
// counters (one per prefill output tile; zero before the first call and left
// zero by every call), then one fp32 partial plane per split: [M][N] for the
// decode kernel, [mtiles*ntiles][BM*BN] (whole tiles) for the prefill kernel.
// The head has the same size and place for every call, so partials written by
// one call never land on the counters of another.
constexpr int kSplitCounters = 4096;
constexpr size_t kWsHeadBytes = kSplitCounters * sizeof(int);
inline size_t gather_offset(size_t split) {
  const size_t b = split > kWsHeadBytes ? split : kWsHeadBytes;
  return (b + 255) & ~(size_t)255;
}
inline size_t split_ws_bytes(int splits, size_t plane_floats) {
  return splits > 1 ? kWsHeadBytes + (size_t)splits * plane_floats * sizeof(float) : 0;
}

hipError_t launch_prefill(const GemmArgs& a, const PrefillPlan& plan, void* ws,
                          hipStream_t stream);
// y[m][n] = fp16(sum over s < splits, in order, of part[s][m][n] (+ bias[n]))
// (+ res[m][n]): the split-K planes [splits][M][N] of one product.
hipError_t launch_reduce_planes(const float* part, int splits, int M, int N, const uint16_t* bias,
                                uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldres,
                                hipStream_t stream);
// The LDS-streamed prefill kernel (w4a16_prefill.hip): 64 x 256, 128 x 128 or
// 128 x 256 tiles, x already in the packed row order (perm null).  Split-K partial planes
// [splits][M][N] after the workspace head, summed by launch_reduce_planes.
hipError_t launch_prefill2(const GemmArgs& a, const PrefillPlan& plan, void* ws,
                           hipStream_t stream);
hipError_t launch_dequant(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                          const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs,
                          int G, hipStream_t stream);
// Calibration read: `workgroups` x `threads` (a multiple of 64, at most
// 1024), each workgroup streaming chunks_per_wg contiguous KiB of src.
hipError_t launch_stream_read(const void* src, int workgroups, int threads, int chunks_per_wg,
                              uint32_t never, uint32_t* sink, hipStream_t stream);
// As launch_dequant, each value converted to bf16 (round to nearest even).
hipError_t launch_dequant_bf16(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                               const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs,
                               int G, hipStream_t stream);

}  // namespace dw4
