// Transposed W4A16 product for the PEFT backward: out = g @ W^T.
//
// g fp16 [M, N] (the output gradient), W the packed [K, N] int4 matrix,
// out fp16 [M, K] in the checkpoint's row order.  The reference computes it
// by dequantising W into an fp16 K x N buffer and running a dense GEMM
// (cuda_extends/exllama/q4_transpose_matmul.cu:115-167, exllama.py:528-544);
// here the packed words are read once and never expanded in memory.
//
// MFMA reduces over the elements a lane holds, and a packed word gives a lane
// 8 rows k of one column n; the reduction here runs over n.  Each dequantised
// word is therefore turned around by the matrix core itself: a
// v_mfma_f32_16x16x32_f16 with the word as its A operand (rows n, reduction
// k) and a one-hot B operand selecting 16 of the 32 k returns, in the D
// layout, 4 consecutive n of one k per lane -- exactly the B operand of a
// v_mfma_f32_16x16x16_f16 whose reduction runs over n.  The values pass
// through fp32 unchanged (one product with 1.0 each), so the weight that
// enters the product is the exact fp16 dequantised weight fp16(s * (q - z)),
// as dw4_dequant writes it.
//
// Grid: x = (K/128 chunk rows) x (NS N-ranges), z = 64-row blocks of M.  A
// workgroup of 4 waves owns one chunk row (128 outputs k) of one N-range;
// its waves take the range's 16-column strips round-robin and stream each
// strip's 1 KB chunk through a register ring.  The waves' fp32 partial tiles
// meet in LDS in a fixed order; with one N-range the tile is rounded and
// stored (scattered through perm for act-order), otherwise it goes to an
// fp32 plane of the workspace and a second kernel sums the planes in order.

#include <hip/hip_runtime.h>

#include <algorithm>

#include "w4a16_device.h"
#include "w4a16_transpose.h"

namespace dw4 {

namespace {

__device__ __forceinline__ f4 mfma16x16x16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// fp32 -> fp16 for values that are fp16 already (exact under any rounding)
__device__ __forceinline__ h4 to_h4(f4 v) {
  const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[0], v[1]));
  const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[2], v[3]));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
}

// KBR: 16-row k-blocks reduced per LDS round (8 / KBR rounds, each with
// WAVES x KBR x MT x 1 KB of LDS).
template <int MT, int WAVES, int U, int GPC, bool ACT, int KBR>
__global__ void __launch_bounds__(WAVES * 64)
gemm_t_kernel(const _Float16* __restrict__ g, int64_t ldg, int M,
              const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
              const uint32_t* __restrict__ ps32, const int32_t* __restrict__ perm,
              uint16_t* __restrict__ out, int64_t ldo, float* __restrict__ part,
              int K, int N, int gs, int G, int spr) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int T = WAVES * 64;
  const int KC = K / kChunkK;
  const int NSTR = N / kStripN;
  const int c = blockIdx.x % KC;           // chunk row: outputs k in [128c, 128c + 128)
  const int ns = blockIdx.x / KC;          // N-range
  const int m0 = blockIdx.z * 64;          // first row of this M block
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int s_lo = ns * spr;
  const int s_hi = min(NSTR, s_lo + spr);
  const int nstr = s_hi - s_lo;
  const int nch = wave < nstr ? (nstr - wave + WAVES - 1) / WAVES : 0;  // this wave's strips

  // one-hot selectors: B[kk][jj] = (kk == jj) and (kk == jj + 16), kk = 8 kq + e
  h8 sel0, sel1;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sel0[e] = (8 * kq + e == j) ? (_Float16)1.0f : (_Float16)0.0f;
    sel1[e] = (8 * kq + e == j + 16) ? (_Float16)1.0f : (_Float16)0.0f;
  }
  // g rows of the A operand (lanes past the last row read row M-1, never stored)
  const _Float16* grow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    grow[mt] = g + (size_t)min(m0 + mt * 16 + j, M - 1) * ldg + 4 * kq;

  // ring slot: 4 packed words, per-group scale/zero words, the g fragments
  u4 qb[U];
  uint32_t sb[U][GPC], zb[U][GPC];
  h4 gb[U][MT];
  auto load = [&](int slot, int i) {
    const int s = s_lo + wave + i * WAVES;
    qb[slot] = __builtin_nontemporal_load(pq + ((size_t)s * KC + c) * 64 + lane);
#pragma unroll
    for (int gl = 0; gl < GPC; ++gl) {
      const int grp = GPC == 1 ? (c * kChunkK) / gs : c * GPC + gl;
      sb[slot][gl] = ps32[((size_t)s * G + grp) * 8 + (j >> 1)];
      zb[slot][gl] = pz[((size_t)s * G + grp) * 2 + (j >> 3)];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) gb[slot][mt] = *(const h4*)(grow[mt] + s * kStripN);
  };

  f4 acc[8][MT];
#pragma unroll
  for (int kb = 0; kb < 8; ++kb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[kb][mt] = f4{0.f, 0.f, 0.f, 0.f};

  const uint32_t magic = opaque(kMagic);
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;
  constexpr int WPG = 4 / GPC;  // packed words (32-row k-steps) per group
  auto consume = [&](int slot) {
    _Float16 sc = (_Float16)0.f;
    h2 nz1024, nz64;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w % WPG == 0) {
        const int gl = w / WPG;
        sc = as_h((uint16_t)(sb[slot][gl] >> hsh));
        zero_consts(zb[slot][gl], zsh, nz1024, nz64);
      }
      // exact fp16 weight of rows 32w + 8kq + e, column j of the strip
      const h8 wv = centered8(qb[slot][w], nz1024, nz64, magic) *
                    h8{sc, sc, sc, sc, sc, sc, sc, sc};
      const f4 z = f4{0.f, 0.f, 0.f, 0.f};
      const h4 b0 = to_h4(__builtin_amdgcn_mfma_f32_16x16x32_f16(wv, sel0, z, 0, 0, 0));
      const h4 b1 = to_h4(__builtin_amdgcn_mfma_f32_16x16x32_f16(wv, sel1, z, 0, 0, 0));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[2 * w][mt] = mfma16x16x16(gb[slot][mt], b0, acc[2 * w][mt]);
        acc[2 * w + 1][mt] = mfma16x16x16(gb[slot][mt], b1, acc[2 * w + 1][mt]);
      }
    }
  };

  // ring: every wave with strips has at least one; refills only where one remains
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (u < nch) load(u, u);
  int i0 = 0;
  for (; i0 + 2 * U <= nch; i0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume(u);
      load(u, i0 + u + U);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = i0 + u;
    if (i < nch) {
      consume(u);
      if (i + U < nch) load(u, i + U);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (i0 + U + u < nch) consume(u);

  // Fixed-order reduction across waves, KBR 16-row k-blocks per round (LDS
  // holds WAVES x KBR x MT x 64 f4).
  f4* red = reinterpret_cast<f4*>(smem);
  const float* redf = reinterpret_cast<const float*>(smem);
  const bool direct = part == nullptr;
#pragma unroll
  for (int kb0 = 0; kb0 < 8; kb0 += KBR) {
    if (kb0 > 0) __syncthreads();  // the previous round's reads are done
#pragma unroll
    for (int b = 0; b < KBR; ++b)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((wave * KBR + b) * MT + mt) * 64 + lane] = acc[kb0 + b][mt];
    __syncthreads();
    for (int idx = tid; idx < KBR * MT * 256; idx += T) {
      const int llo = idx & 15;
      const int r = (idx >> 4) & 3;
      const int lhi = (idx >> 6) & 3;
      const int bm = idx >> 8;  // b * MT + mt
      const int mt = bm % MT;
      const int b = bm / MT;
      const int m = m0 + mt * 16 + lhi * 4 + r;
      if (m >= M) continue;
      const int L = lhi * 16 + llo;
      float sum = 0.f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) sum += redf[(((wv * KBR + b) * MT + mt) * 64 + L) * 4 + r];
      const int k = c * kChunkK + 16 * (kb0 + b) + llo;  // sorted row
      if (direct) {
        const int row = ACT ? perm[k] : k;
        out[(size_t)m * ldo + row] = h_bits((_Float16)sum);
      } else {
        part[((size_t)ns * M + m) * K + k] = sum;
      }
    }
  }
}

// Sum of the N-range planes in order, rounded once, scattered through perm.
__global__ void gemm_t_reduce_kernel(const float* __restrict__ part, int ns, int M, int K,
                                     const int32_t* __restrict__ perm, uint16_t* __restrict__ out,
                                     int64_t ldo) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)M * K;
  if (o >= total) return;
  // all loads of a batch in flight before the first add; sums in plane order
  float sum = 0.f;
  for (int i0 = 0; i0 < ns; i0 += 8) {
    float v[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = i0 + b < ns ? part[(size_t)(i0 + b) * total + o] : 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b)
      if (i0 + b < ns) sum += v[b];
  }
  const int m = (int)(o / K);
  const int k = (int)(o % K);
  const int row = perm != nullptr ? perm[k] : k;
  out[(size_t)m * ldo + row] = h_bits((_Float16)sum);
}

// Workgroup shape within 128 registers per lane for 16 waves (no spills in
// the build's register report): 16 waves up to 32 rows, a 4-deep ring for
// 16 rows; groups of 32 rows keep four scale/zero pairs per ring slot, so
// they take a 2-deep ring, and 8 waves at 32 rows.
template <int MT, int GPC> constexpr int t_waves() { return MT == 1 || (MT == 2 && GPC < 4) ? 16 : 8; }
template <int MT, int GPC> constexpr int t_ring() { return MT == 1 && GPC < 4 ? 4 : 2; }

// k-blocks per reduction round: as many as 128 KB of LDS holds
template <int MT, int GPC> constexpr int t_kbr() {
  return 128 / (t_waves<MT, GPC>() * MT) >= 8 ? 8 : 128 / (t_waves<MT, GPC>() * MT) >= 4 ? 4 : 2;
}

template <int MT, int GPC, bool ACT>
hipError_t launch_t_cfg(const GemmTArgs& a, const GemmTPlan& p, float* part, hipStream_t stream) {
  constexpr int WAVES = t_waves<MT, GPC>();
  constexpr int KBR = t_kbr<MT, GPC>();
  const int KC = a.K / kChunkK;
  const dim3 grid((unsigned)(KC * p.ns), 1, (unsigned)((a.M + 63) / 64));
  const size_t smem = (size_t)WAVES * KBR * MT * 64 * sizeof(f4);
  auto kern = &gemm_t_kernel<MT, WAVES, t_ring<MT, GPC>(), GPC, ACT, KBR>;
  if (smem > 64 * 1024) {
    static std::atomic<uint64_t> allowed{0};
    const hipError_t e = allow_lds(reinterpret_cast<const void*>(kern), smem, allowed);
    if (e != hipSuccess) return e;
  }
  kern<<<grid, WAVES * 64, smem, stream>>>(
      (const _Float16*)a.g, a.ldg, a.M, (const u4*)a.pq, a.pz, (const uint32_t*)a.ps, a.perm,
      a.out, a.ldo, p.ns > 1 ? part : nullptr, a.K, a.N, a.gs, a.G, p.spr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ns == 1) return e;
  const size_t total = (size_t)a.M * a.K;
  gemm_t_reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
      part, p.ns, a.M, a.K, a.perm, a.out, a.ldo);
  return hipGetLastError();
}

template <int MT, int GPC>
hipError_t launch_t_act(const GemmTArgs& a, const GemmTPlan& p, float* part, hipStream_t stream) {
  return a.perm != nullptr ? launch_t_cfg<MT, GPC, true>(a, p, part, stream)
                           : launch_t_cfg<MT, GPC, false>(a, p, part, stream);
}

template <int MT>
hipError_t launch_t_mt(const GemmTArgs& a, const GemmTPlan& p, float* part, hipStream_t stream) {
  const int gpc = a.gs >= kChunkK ? 1 : kChunkK / a.gs;
  if (gpc == 1) return launch_t_act<MT, 1>(a, p, part, stream);
  if (gpc == 2) return launch_t_act<MT, 2>(a, p, part, stream);
  return launch_t_act<MT, 4>(a, p, part, stream);
}

}  // namespace

GemmTPlan plan_gemm_t(int m, int k, int n, int cus) {
  GemmTPlan p;
  const int kc = k / kChunkK;
  const int strips = n / kStripN;
  const int mt = std::min(4, (m + 15) / 16);
  const int waves = mt <= 2 ? 16 : 8;
  const int mb = (m + 63) / 64;
  // One workgroup per CU (its registers and 128 KB of LDS), all in one
  // round: a grid just above the CU count would run a second round for a
  // few workgroups.  At least one strip per wave; the fp32 partial planes
  // (ns * m * k * 4 bytes, written and read once) kept to about a quarter of
  // the packed weight bytes (k * n / 2).
  const int want = cus / (kc * mb);
  const int cap = std::max(1, n / (16 * std::max(1, m)));
  p.ns = std::max(1, std::min({want, cap, strips / waves}));
  p.spr = (strips + p.ns - 1) / p.ns;
  p.ns = (strips + p.spr - 1) / p.spr;
  return p;
}

size_t gemm_t_ws_bytes(const GemmTPlan& p, int m, int k) {
  return p.ns > 1 ? (size_t)p.ns * m * k * sizeof(float) : 0;
}

hipError_t launch_gemm_t(const GemmTArgs& a, const GemmTPlan& p, float* part,
                         hipStream_t stream) {
  if (p.ns > 1 && part == nullptr) return hipErrorInvalidValue;
  switch (std::min(4, (a.M + 15) / 16)) {
    case 1: return launch_t_mt<1>(a, p, part, stream);
    case 2: return launch_t_mt<2>(a, p, part, stream);
    case 3: return launch_t_mt<3>(a, p, part, stream);
    default: return launch_t_mt<4>(a, p, part, stream);
  }
}

}  // namespace dw4
