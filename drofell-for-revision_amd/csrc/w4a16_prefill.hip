// gfx950 W4A16 prefill kernel: 64 x 256, 128 x 128 or 128 x 256 output
// tiles (8 waves), or 32 x 128 and 64 x 128 tiles (4 waves, two workgroups
// per CU) on v_mfma_f32_32x32x16_f16, activations streamed straight into LDS.
//
// Replaces, in function, the reference's large-M routes (paths relative to
// /root/reference/After-Revision-DROFELL): q4_matmul_cudablas_v2
// (cuda_extends/exllama/q4_matmul.cu:459-510: reconstruct_gptq_kernel to a
// dense fp16 weight, then cublasHgemm) and the Marlin direct GEMM
// (cuda_extends/vllm/csrc/libtorch_stable/quantization/marlin/marlin.cu).
//
// Structure of one workgroup (512 threads, 8 waves, two waves per SIMD so
// that one wave's MFMAs run while the other waits on LDS or the barrier; the
// 4-wave tiles get the same from two workgroups per CU):
//   * every wave computes all BM tile rows (MTW = BM / 32 A fragments) for
//     one 64-column group (two 32-column strip pairs) over a slice of each
//     chunk's k-steps; the tile has CG column groups and 8 / CG k-slices, and
//     the k-slices' sums are added through LDS at the end.  Each dequantised
//     B fragment feeds MTW MFMAs and each A fragment read from LDS two.  The
//     exact dequantisation costs ~13 VALU instructions per fragment, so the
//     128-row tiles (MTW = 4) keep the vector ALU well below the matrix pipe;
//     the 64-row tile (MTW = 2) gives small M twice the tiles (fewer split-K
//     partial planes) at a higher VALU share;
//   * a chunk is 128 sorted rows of K.  Everything the chunk needs -- its
//     activation tile (128 x 128 fp16), the tile's packed weight strips
//     (1 KiB each) and their scale / zero words -- is copied global -> LDS
//     by global_load_lds (no register round trip) into an S-deep LDS ring,
//     S - 1 chunks ahead of the MFMAs;
//   * one bare s_barrier per chunk, preceded by an explicit vmcnt wait for
//     this wave's copies of the chunk about to be used, so the later chunks'
//     copies stay in flight across it (a __syncthreads would drain them);
//   * LDS activation rows are 256 bytes with the 16-byte units of row r
//     stored at position u ^ (r & 15): the A-fragment reads (16 rows at one
//     unit per 16 lanes) hit 16 different unit positions, conflict-free;
//   * dequantisation as everywhere in this library: the exact fp16 weight
//     fp16_rne(s * (q - z)) from the 0x6400 identity, so the product equals
//     "dequantise, then an fp32-accumulated matmul";
//   * split-K (several workgroups per tile along K): each split writes its
//     fp32 partial plane and a second kernel sums the planes in split order
//     (deterministic) into y.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_device.h"
#include "w4a16_prefill.h"

namespace dw4 {

namespace {

constexpr int kPairs = 2;                     // strip pairs of one column group
constexpr int kGroupStrips = 2 * kPairs;      // 16-column strips of one column group
constexpr int kLdsMax = 160 * 1024;  // per CU: one 8-wave workgroup, or two 4-wave ones

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// global -> LDS copies: each active lane's 16 (4) bytes at g land at LDS
// address `lds` + lane * 16 (* 4).  Written as inline assembly so that the
// compiler's wait-count pass does not track them: it cannot tell which LDS
// reads such a copy may overlap and would drain every outstanding load
// before them.  The kernel waits for its copies itself (vmcnt) and makes
// them visible to the other waves with a barrier.  m0 carries the LDS base
// (one wait state before its use); nothing else in these kernels uses m0.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(lds) : "memory");
}

// s_waitcnt with only vmcnt set (expcnt and lgkmcnt left at "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  constexpr int n = N > 63 ? 63 : N;
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Tile shape, wave roles and LDS ring geometry (bytes).  One stage holds the
// activation tile (BM rows of 256 bytes, 16-byte units of row r stored at
// position u ^ (r & 15)), the tile's packed weight strips (1 KiB each,
// lane-linear), then the scale and zero words of each column group.
template <int MTW, int CG, int GPC, int W>
struct Tile {
  static constexpr int kWaves = W;                          // waves per workgroup
  static constexpr int kLds = W == 8 ? kLdsMax : kLdsMax / 2;  // this workgroup's share
  static constexpr int kBM = 32 * MTW;
  static constexpr int kBN = 64 * CG;
  static constexpr int kAccSlots = MTW * kPairs * 16;       // accumulator floats per lane
  static constexpr int kStrips = kGroupStrips * CG;         // strips of the tile
  static constexpr int kKS = kWaves / CG;                   // k-slices
  static constexpr int kSteps = 8 / kKS;                    // k-steps per wave per chunk
  static constexpr int kWords = kSteps / 2;                 // packed words per lane per strip
  static constexpr int kA = kBM * 256;
  static constexpr int kB = kStrips * 1024;
  // per column group: 4 strips x GPC groups x (8 scale + 2 zero dwords)
  static constexpr int kMetaGroupDw = 40 * GPC;
  static constexpr int kMetaInstr = (CG * kMetaGroupDw + kWaves * 64 - 1) / (kWaves * 64);
  static constexpr int kMeta = kMetaInstr * kWaves * 256;
  static constexpr int kBytes = (kA + kB + kMeta + 255) & ~255;
  static constexpr int kAInstr = kA / (kWaves * 1024);      // 16-byte copies per wave
  static constexpr int kBInstr = kStrips / kWaves;          // strips copied per wave
  static constexpr int kPerChunk = kAInstr + kBInstr + kMetaInstr;  // copies per wave per chunk
  static constexpr int kDepth = kLds / kBytes < 4 ? kLds / kBytes : 4;
  // groups of one chunk a wave's k-slice spans
  static constexpr int kGroups = kSteps * GPC / 8 > 0 ? kSteps * GPC / 8 : 1;
  static_assert(kStrips % kWaves == 0 && kKS * CG == kWaves, "wave roles cover the tile");
};

// Matrices of one launch: equal K, N and group size, each with its own
// packed buffers, bias, output and residual.  Column tile t of the launch
// belongs to matrix t / ntiles_item (tiles never straddle two matrices).
struct P2Items {
  const u4* pq[kGroupMax];
  const uint32_t* pz[kGroupMax];
  const uint32_t* ps[kGroupMax];
  const uint16_t* bias[kGroupMax];
  uint16_t* y[kGroupMax];
  int64_t ldy[kGroupMax];
  const uint16_t* res[kGroupMax];
  int64_t ldres[kGroupMax];
  int ntiles_item;
};

}  // namespace

template <int MTW, int CG, int GPC, int W>
__global__ void __launch_bounds__(W * 64)
prefill2_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, const P2Items it,
                float* __restrict__ part, int K, int N, int gs, int G,
                int chunks_per_split, int mtiles, int ntiles, int splits, int group_m) {
  using T = Tile<MTW, CG, GPC, W>;
  constexpr int kWaves = W;
  constexpr int kBM = T::kBM;
  constexpr int kMT = MTW;
  constexpr int kAccSlots = T::kAccSlots;
  constexpr int S = T::kDepth;
  constexpr int NT = T::kSteps;
  constexpr int KS = T::kKS;
  constexpr int BN = T::kBN;
  static_assert(S >= 2 && S * T::kBytes <= T::kLds, "LDS ring fits the workgroup's share");
  __shared__ __attribute__((aligned(256))) unsigned char ring[S * T::kBytes];

  // XCD-aware order over units (column tile, K split), u = split * ntiles +
  // ntile: workgroup b runs on XCD b % 8 and takes the XCD's (b / 8)-th
  // (row tile, unit) pair; XCD x owns the units congruent to x mod 8
  // (ceil(units / 8) each, the padding ones exit).  On one XCD the pairs
  // run in groups of group_m row tiles: within a group, the row tiles of
  // one unit are consecutive, then the next unit's, so the workgroups an
  // XCD runs at once share both the units' weights and the group's
  // activation rows in its L2 (group_m = all row tiles: every row tile of
  // a unit on one XCD in turn).
  const int b = blockIdx.x;
  const int nul = (ntiles * splits + 7) / 8;
  const int pos = b >> 3;  // position in this XCD's order
  const int grp = pos / (group_m * nul);
  const int first_m = grp * group_m;
  const int gsz = min(mtiles - first_m, group_m);
  const int jj = pos - grp * group_m * nul;
  const int mtile = first_m + jj % gsz;
  const int unit = (jj / gsz) * 8 + (b & 7);
  if (unit >= ntiles * splits) return;
  const int split = unit / ntiles;
  // the launch's column tile -> (matrix, its column tile); wave-uniform
  const int item = (unit % ntiles) / it.ntiles_item;
  const int ntile = unit % ntiles - item * it.ntiles_item;
  const u4* __restrict__ pq = it.pq[item];
  const uint32_t* __restrict__ pz = it.pz[item];
  const uint32_t* __restrict__ ps32 = it.ps[item];
  const uint16_t* __restrict__ bias = it.bias[item];
  uint16_t* __restrict__ y = it.y[item];
  const int64_t ldy = it.ldy[item];
  const uint16_t* __restrict__ res = it.res[item];
  const int64_t ldres = it.ldres[item];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave % CG;          // column group
  const int ks = wave / CG;          // k-slice
  const int l32 = lane & 31;
  const int hb = lane >> 5;          // k half of the 32x32x16 operands
  const int hi = (lane >> 4) & 1;    // which strip of a pair holds this lane's B column
  const int j = lane & 15;
  const int KC = K / kChunkK;
  const int c_begin = split * chunks_per_split;
  const int nchunks = min(KC, c_begin + chunks_per_split) - c_begin;
  const int m0 = mtile * kBM;
  const int step0 = NT * ks;                  // this wave's first k-step of a chunk
  const int NS = N / kStripN;
  const int strip0 = ntile * T::kStrips;
  const int gstrip0 = strip0 + cg * kGroupStrips;  // this wave's first strip
  const uint32_t ring0 = lds_addr(ring);

  // ---- per-lane sources of this wave's copies (chunk offsets added per copy)
  // activations: copy a of this wave fills units (wave * kAInstr + a) * 64 +
  // lane: row r = unit / 16 at stored position unit % 16, which holds
  // logical unit (unit % 16) ^ (r % 16)
  const _Float16* asrc[T::kAInstr];
#pragma unroll
  for (int a = 0; a < T::kAInstr; ++a) {
    const int unit = (wave * T::kAInstr + a) * 64 + lane;
    const int r = unit >> 4;
    const int u = (unit & 15) ^ (r & 15);
    asrc[a] = x + (size_t)min(m0 + r, M - 1) * ldx + (size_t)c_begin * kChunkK + u * 8;
  }
  // packed weights: tile strip wave * kBInstr + bi, chunk-contiguous (the
  // last column tile may be partial: missing strips read strip 0, their
  // columns are not stored)
  const u4* bsrc[T::kBInstr];
#pragma unroll
  for (int bi = 0; bi < T::kBInstr; ++bi) {
    const int st = strip0 + wave * T::kBInstr + bi;
    bsrc[bi] = pq + ((size_t)(st < NS ? st : 0) * KC + c_begin) * 64 + lane;
  }
  // scale and zero dwords: dword D of the meta block (D = (mi * 8 + wave) * 64
  // + lane) belongs to column group D / (40 GPC); within it, d < 32 GPC are
  // scales (strip d / (8 GPC), group d / 8 % GPC, word d % 8), then 8 GPC
  // zero words (strip e / (2 GPC), group e / 2 % GPC, word e % 2); dwords
  // past the block re-read dword 0
  const uint32_t* msrc[T::kMetaInstr];
  int mstride[T::kMetaInstr];
#pragma unroll
  for (int mi = 0; mi < T::kMetaInstr; ++mi) {
    int D = (mi * kWaves + wave) * 64 + lane;
    if (D >= CG * T::kMetaGroupDw) D = 0;
    const int grp = D / T::kMetaGroupDw;
    const int d = D % T::kMetaGroupDw;
    if (d < 32 * GPC) {
      const int st = strip0 + grp * kGroupStrips + d / (8 * GPC);
      msrc[mi] = ps32 + ((size_t)(st < NS ? st : 0) * G + (d / 8) % GPC) * 8 + (d % 8);
      mstride[mi] = 8;
    } else {
      const int e = d - 32 * GPC;
      const int st = strip0 + grp * kGroupStrips + e / (2 * GPC);
      msrc[mi] = pz + ((size_t)(st < NS ? st : 0) * G + (e / 2) % GPC) * 2 + (e % 2);
      mstride[mi] = 2;
    }
  }
  // chunk i of this split into ring stage `stage`
  auto issue = [&](int stage, int i) {
    const uint32_t base = ring0 + stage * T::kBytes;
#pragma unroll
    for (int a = 0; a < T::kAInstr; ++a)
      dma16(asrc[a] + (size_t)i * kChunkK, base + (wave * T::kAInstr + a) * 1024);
#pragma unroll
    for (int bi = 0; bi < T::kBInstr; ++bi)
      dma16(bsrc[bi] + (size_t)i * 64, base + T::kA + (wave * T::kBInstr + bi) * 1024);
    const int c = c_begin + i;
    const int g0 = GPC == 1 ? (c * kChunkK) / gs : c * GPC;  // first group of the chunk
#pragma unroll
    for (int mi = 0; mi < T::kMetaInstr; ++mi)
      dma4(msrc[mi] + (size_t)g0 * mstride[mi], base + T::kA + T::kB + (mi * kWaves + wave) * 256);
  };

  // ---- LDS offsets (bytes within a stage).  A fragment of k-step t: lane
  // reads row l32 (+ 32 mt) at logical unit 2t + hb, stored at
  // (2t + hb) ^ (row % 16).  B words of this wave's k-slice: word ks * kWords
  // (.. + kWords - 1) of each lane's 16 bytes.  Meta: the column group's block.
  uint32_t aoff[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
    aoff[tt] = (uint32_t)(l32 * 256 + (((2 * (step0 + tt) + hb) ^ j) * 16));
  const uint32_t boff = T::kA + cg * kGroupStrips * 1024 + lane * 16 + ks * T::kWords * 4;
  const uint32_t moff = T::kA + T::kB + cg * T::kMetaGroupDw * 4;

  f16v acc[kMT][kPairs];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int p = 0; p < kPairs; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mt][p][e] = 0.f;

  const uint32_t magic = opaque(kMagic);
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;
  const int gbase = (step0 * GPC) / 8;  // first group of the chunk this wave's slice uses
  auto compute = [&](int stage) {
    const unsigned char* base = ring + stage * T::kBytes;
    const uint32_t* meta = reinterpret_cast<const uint32_t*>(base + moff);
    // packed words of the group's strips for this wave's k-steps (word w
    // covers slice steps 2w and 2w + 1)
    uint32_t qw[kGroupStrips][T::kWords];
#pragma unroll
    for (int si = 0; si < kGroupStrips; ++si) {
      const unsigned char* src = base + boff + si * 1024;
      if (T::kWords == 1) {
        qw[si][0] = *reinterpret_cast<const uint32_t*>(src);
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        qw[si][0] = v.x;
        qw[si][T::kWords - 1] = v.y;
      }
    }
    h2 nz1024[kPairs][T::kGroups], nz64[kPairs][T::kGroups];
    _Float16 sc[kPairs][T::kGroups];
#pragma unroll
    for (int p = 0; p < kPairs; ++p)
#pragma unroll
      for (int gl = 0; gl < T::kGroups; ++gl) {
        const int sl = 2 * p + hi;  // this lane's strip within the column group
        const int g = gbase + gl;
        zero_consts(meta[32 * GPC + sl * 2 * GPC + g * 2 + (j >> 3)], zsh, nz1024[p][gl],
                    nz64[p][gl]);
        sc[p][gl] = as_h((uint16_t)(meta[sl * 8 * GPC + g * 8 + (j >> 1)] >> hsh));
      }
    uint32_t ev[kPairs], od[kPairs];
    auto dequant = [&](int tt, h8 (&bop)[kPairs]) {
      const int gl = (tt * GPC) / 8;
#pragma unroll
      for (int p = 0; p < kPairs; ++p) {
        if ((tt & 1) == 0)
          strip_pair_to_b32(qw[2 * p][tt >> 1], qw[2 * p + 1][tt >> 1], ev[p], od[p]);
        const h8 d = centered8((tt & 1) ? od[p] : ev[p], nz1024[p][gl], nz64[p][gl], magic);
        const _Float16 s = sc[p][gl];
        bop[p] = d * h8{s, s, s, s, s, s, s, s};  // fp16 product, round to nearest even
      }
    };
    auto read_a = [&](int tt, h8 (&af)[kMT]) {
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) af[mt] = *(const h8*)(base + aoff[tt] + mt * 32 * 256);
    };
    h8 af[2][kMT], bop[2][kPairs];
    read_a(0, af[0]);
    dequant(0, bop[0]);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int cur = tt & 1;
      if (tt + 1 < NT) {
        read_a(tt + 1, af[cur ^ 1]);
        dequant(tt + 1, bop[cur ^ 1]);
      }
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int p = 0; p < kPairs; ++p) acc[mt][p] = mfma32(af[cur][mt], bop[cur][p], acc[mt][p]);
    }
  };

  // ---- main loop: chunk i in stage i % S; copies run S - 1 chunks ahead.
  // Every step issues one chunk's copies (past the end it re-copies the last
  // chunk into a stage nothing reads again), so exactly S - 2 later chunks'
  // copies are outstanding when a step waits for its own.
#pragma unroll
  for (int s = 0; s < S - 1; ++s) issue(s, min(s, nchunks - 1));
  for (int i = 0; i < nchunks; ++i) {
    const int stage = i % S;
    wait_vmcnt<(S - 2) * T::kPerChunk>();
    __builtin_amdgcn_s_barrier();
    // every wave is past chunk i - 1: its stage takes chunk i + S - 1
    issue((stage + S - 1) % S, min(i + S - 1, nchunks - 1));
    compute(stage);
  }
  wait_vmcnt<0>();  // the trailing copies land before the epilogue reuses the ring
  __builtin_amdgcn_s_barrier();

  // ---- k-slice sums through LDS, in two halves of the accumulators (the
  // first and the last MTW * kPairs / 2 of the MTW x kPairs fragments, in
  // row-tile-major order) and rounds that halve the slices: slices [r, 2r)
  // store, slices [0, r) add.  A wave's half is one slot of MTW * 2 KiB,
  // [accumulator slot][lane] fp32 (conflict-free).
  constexpr int kHalfSlots = kAccSlots / 2;
  static_assert(KS / 2 * CG * kHalfSlots * 64 * 4 <= S * T::kBytes, "sum slots fit the ring");
  constexpr int F = kMT * kPairs;  // accumulators per lane, 16 floats each
#pragma unroll
  for (int part = 0; part < 2; ++part) {
#pragma unroll
    for (int r = KS / 2; r >= 1; r /= 2) {
      const int pos = (ks % r) * CG + cg;  // slot of the (slice, column group) pair
      float* R = reinterpret_cast<float*>(ring) + pos * (kHalfSlots * 64);
      if (ks >= r && ks < 2 * r) {
#pragma unroll
        for (int fh = 0; fh < F / 2; ++fh)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            R[(fh * 16 + i) * 64 + lane] = acc[(part * F / 2 + fh) / kPairs][(part * F / 2 + fh) % kPairs][i];
      }
      __syncthreads();
      if (ks < r) {
#pragma unroll
        for (int fh = 0; fh < F / 2; ++fh)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            acc[(part * F / 2 + fh) / kPairs][(part * F / 2 + fh) % kPairs][i] += R[(fh * 16 + i) * 64 + lane];
      }
      __syncthreads();
    }
  }
  const bool owner = ks == 0;  // waves holding the final sums

  if (splits > 1) {
    // ---- split-K: this split's fp32 partial product into plane `split` of
    // [splits][M][N] (a store instruction covers 32 consecutive columns of
    // two rows); a second kernel sums the planes in split order.  No arrival
    // counters: an agent-scope release per workgroup writes back the L2 and
    // costs more than the reduction itself.
    if (!owner) return;
    float* plane = part + (size_t)split * M * N;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int p = 0; p < kPairs; ++p) {
        const int st = gstrip0 + 2 * p + hi;
        if (st < NS) {
          const int col = (gstrip0 + 2 * p) * kStripN + l32;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * hb + (i & 3);
            if (m < M) plane[(size_t)m * N + col] = acc[mt][p][i];
          }
        }
      }
    return;
  }

  // ---- output: the owners stage the fp16 BM x BN tile in LDS in row
  // order, then all 512 threads store 16-byte row segments
  static_assert(kBM * BN * 2 <= S * T::kBytes, "output tile fits the LDS ring");
  _Float16* Ts = reinterpret_cast<_Float16*>(ring);
  if (owner) {
    _Float16 bv[kPairs];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      const int st = gstrip0 + 2 * p + hi;
      bv[p] = (bias != nullptr && st < NS) ? as_h(bias[st * kStripN + j]) : (_Float16)0.f;
    }
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int p = 0; p < kPairs; ++p)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          _Float16 out = (_Float16)acc[mt][p][i];
          if (bias != nullptr) out = out + bv[p];
          const int row = mt * 32 + 8 * (i >> 2) + 4 * hb + (i & 3);
          Ts[row * BN + cg * 64 + p * 32 + l32] = out;
        }
  }
  __syncthreads();
  const bool vec_y = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && (ldy % 8 == 0) &&
                     (res == nullptr ||
                      (((reinterpret_cast<uintptr_t>(res) & 15) == 0) && (ldres % 8 == 0)));
  constexpr int SEG = BN / 8;                // 16-byte segments per row
  constexpr int RPP = kWaves * 64 / SEG;     // rows per pass of the workgroup
#pragma unroll
  for (int pass = 0; pass < kBM / RPP; ++pass) {
    const int row = pass * RPP + tid / SEG;
    const int seg = tid % SEG;
    const int m = m0 + row;
    const int strip = strip0 + seg / 2;
    if (m < M && strip < NS) {
      u4 v = *(const u4*)&Ts[row * BN + seg * 8];
      const int col = strip * kStripN + (seg & 1) * 8;
      uint16_t* dst = y + (size_t)m * ldy + col;
      const uint16_t* rsrc = res != nullptr ? res + (size_t)m * ldres + col : nullptr;
      if (vec_y) {
        if (rsrc != nullptr) v = add_h8(v, *(const u4*)rsrc);
        *(u4*)dst = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 lo = as_h((uint16_t)(v[e] & 0xFFFFu)), hi2 = as_h((uint16_t)(v[e] >> 16));
          if (rsrc != nullptr) {
            lo = lo + as_h(rsrc[2 * e]);
            hi2 = hi2 + as_h(rsrc[2 * e + 1]);
          }
          dst[2 * e] = h_bits(lo);
          dst[2 * e + 1] = h_bits(hi2);
        }
      }
    }
  }
}

// Row tiles per group of the workgroup order (kernel comment above): all of
// them up to 8 (a unit's weights then come into an XCD's L2 once), groups of
// 8 above.  Measured against one group at M=4096 (32 row tiles of 128):
// 4096^2 144.9 -> 139.6 us, 4096x11008 401.3 -> 391.0, 11008x4096 369.2 ->
// 353.8; groups of 2 and 4 within 1% of 8; M <= 2048 unchanged.
constexpr int kPrefillGroupM = 8;
static int prefill_group_m(int mtiles) { return mtiles <= kPrefillGroupM ? mtiles : kPrefillGroupM; }

template <int MTW, int CG, int GPC, int W>
static hipError_t launch_prefill2_cfg(const GroupArgs& g, int splits, void* ws,
                                      hipStream_t stream) {
  using T = Tile<MTW, CG, GPC, W>;
  const GemmArgs& a = g.a[0];
  const int mtiles = (a.M + T::kBM - 1) / T::kBM;
  P2Items it{};
  it.ntiles_item = (a.N + T::kBN - 1) / T::kBN;
  for (int i = 0; i < kGroupMax; ++i) {
    const GemmArgs& b = g.a[i < g.count ? i : 0];
    it.pq[i] = reinterpret_cast<const u4*>(b.pq);
    it.pz[i] = b.pz;
    it.ps[i] = reinterpret_cast<const uint32_t*>(b.ps);
    it.bias[i] = b.bias;
    it.y[i] = b.y;
    it.ldy[i] = b.ldy;
    it.res[i] = b.res;
    it.ldres[i] = b.ldres;
  }
  const int ntiles = it.ntiles_item * g.count;
  const int KC = a.K / kChunkK;
  const int cps = (KC + splits - 1) / splits;
  const int real_splits = (KC + cps - 1) / cps;
  if (real_splits > 1 && g.count != 1) return hipErrorInvalidValue;  // planes of one matrix
  float* part = real_splits > 1
                    ? reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + kWsHeadBytes)
                    : nullptr;
  const int units = ntiles * real_splits;
  const dim3 grid((unsigned)(((units + 7) / 8) * 8 * mtiles));
  prefill2_kernel<MTW, CG, GPC, W><<<grid, W * 64, 0, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, it, part, a.K, a.N, a.gs, a.G, cps, mtiles, ntiles,
      real_splits, prefill_group_m(mtiles));
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || real_splits == 1) return e;
  return launch_reduce_planes(part, real_splits, a.M, a.N, a.bias, a.y, a.ldy, a.res, a.ldres,
                              stream);
}

template <int MTW, int CG, int W>
static hipError_t launch_prefill2_tile(const GroupArgs& a, int splits, void* ws,
                                       hipStream_t stream) {
  const int gpc = a.a[0].gs >= kChunkK ? 1 : kChunkK / a.a[0].gs;
  if (gpc == 1) return launch_prefill2_cfg<MTW, CG, 1, W>(a, splits, ws, stream);
  if (gpc == 2) return launch_prefill2_cfg<MTW, CG, 2, W>(a, splits, ws, stream);
  return launch_prefill2_cfg<MTW, CG, 4, W>(a, splits, ws, stream);
}

hipError_t launch_prefill2(const GemmArgs& one, const PrefillPlan& plan, void* ws,
                           hipStream_t stream) {
  GroupArgs g{};
  g.count = 1;
  g.a[0] = one;
  return launch_prefill2_group(g, plan, ws, stream);
}

hipError_t launch_prefill2_group(const GroupArgs& a, const PrefillPlan& plan, void* ws,
                                 hipStream_t stream) {
  if (a.count < 1 || a.count > kGroupMax) return hipErrorInvalidValue;
  for (int i = 0; i < a.count; ++i) {
    const GemmArgs& b = a.a[i];
    // x must already be in packed row order; one x, K, N and group size
    if (b.perm != nullptr || b.x != a.a[0].x || b.ldx != a.a[0].ldx || b.M != a.a[0].M ||
        b.K != a.a[0].K || b.N != a.a[0].N || b.gs != a.a[0].gs)
      return hipErrorInvalidValue;
  }
  if (plan.waves == 4) {  // two workgroups per CU
    if (plan.bm == 64 && plan.bn == 128) return launch_prefill2_tile<2, 2, 4>(a, plan.splits, ws, stream);
    if (plan.bm == 32 && plan.bn == 128) return launch_prefill2_tile<1, 2, 4>(a, plan.splits, ws, stream);
    return hipErrorInvalidValue;
  }
  if (plan.bm == 64 && plan.bn == 256) return launch_prefill2_tile<2, 4, 8>(a, plan.splits, ws, stream);
  if (plan.bm == 128 && plan.bn == 256) return launch_prefill2_tile<4, 4, 8>(a, plan.splits, ws, stream);
  if (plan.bm == 128 && plan.bn == 128) return launch_prefill2_tile<4, 2, 8>(a, plan.splits, ws, stream);
  return hipErrorInvalidValue;
}

}  // namespace dw4
