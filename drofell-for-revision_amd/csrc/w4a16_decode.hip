// gfx950 decode kernels of the GPTQ int4-weight / fp16-activation quantized
// Linear (M <= 64): the LDS-staged kernel (decode_kernel) and the
// register-fed kernel (decode_reg_kernel), their grouped and gate/up pair
// forms, and their launchers.
//
// Replaces, in function (not in structure), the reference's small-M route
// cuda_extends/exllama/q_gemm_kernel_gptq.cuh (gemm_half_q_half_gptq_kernel,
// called for M <= 50 by cuda_extends/exllama.py:41 and q4_matmul.cu) and the
// Marlin GEMM at decode sizes.  Layouts of the packed buffers are documented
// in include/drofell_w4a16.h.
//
// Arithmetic contract (reference: operators/core/linear/real_quant.py:69-102)
//   W[k,n] = fp16_rne(scale[g(k),n] * (q[k,n] - (zero[g(k),n] + 1)))
//   y[m,n] = fp16_rne(sum_k x[m,k] * W[k,n])  (fp32 accumulation)
// These kernels factor the scale out of each group: fp32 products of exact
// small integers (q - z, exact in fp16) and fp16 activations on the MFMA
// units, scaled in fp32 once per group.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace dw4 {

// ---------------------------------------------------------------------------
// Per-(strip, group) metadata record as staged in LDS: 8 dwords holding the
// 16 fp16 scales of the strip's columns, then the 2 dwords of stored zeros.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t meta_word(const uint32_t* __restrict__ ps32,
                                              const uint32_t* __restrict__ pz, int G, int strip,
                                              int g, int w) {
  const size_t sg = (size_t)strip * G + g;
  return w < 8 ? ps32[sg * 8 + w] : pz[sg * 2 + (w - 8)];
}

// ---------------------------------------------------------------------------
// Decode kernel (M <= 64).  Grid: (N/16 strips of every item) x (K splits).  Each wave
// owns the interleaved 128-row chunks lc = wave + i*WAVES of its workgroup's
// K range.  It stages the activation slices (gathered for act-order) and the
// scale/zero records of exactly those chunks into a private LDS region and
// reads back only its own region, so no workgroup barrier stands between a
// wave's first weight bytes and its first MFMA.  The packed weight words
// stream into a U-deep register ring (non-temporal 16-byte loads, 1 KB
// contiguous per wave instruction); each word is dequantised in registers
// straight into the B operand of v_mfma_f32_16x16x32_f16 (exact q - z in
// fp16); the scale is applied per group in fp32; the waves' partial sums
// meet in their own LDS region (one barrier) in a fixed order at the end
// (deterministic).
// ---------------------------------------------------------------------------
constexpr int kXBatch = 8;  // activation units per lane per staging batch
constexpr int kMBatch = 4;  // metadata dwords per lane per staging batch
constexpr int kLdx = kChunkK + 8;  // halfs per staged activation row (16-byte pad)

// GRP: several matrices in one launch (Items table); without it item 0 is
// read directly, which keeps the item lookup out of a single matrix's
// prologue (measured ~0.3 us per launch).
template <int MT, int WAVES, int U, bool G128, bool ACT, bool GRP, bool XG>
__global__ void __launch_bounds__(WAVES * 64)
decode_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, const Items d,
              float* __restrict__ part, int K, int gs, int G, int cps, uint32_t mmag,
              uint32_t gmag) {
  static_assert(!XG || (ACT && MT == 1 && G128 && !GRP), "XG: single-matrix act-order M = 1");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int T = WAVES * 64;
  const int item = GRP ? item_of(d, blockIdx.x) : 0;
  const int s = GRP ? blockIdx.x - pick(d.wg0, item) : blockIdx.x;  // strip within the item
  const int N = GRP ? pick(d.n, item) : d.n[0];
  const int32_t* __restrict__ perm = GRP ? pick(d.perm, item) : d.perm[0];
  const u4* __restrict__ pq = reinterpret_cast<const u4*>(GRP ? pick(d.pq, item) : d.pq[0]);
  const uint32_t* __restrict__ pz = GRP ? pick(d.pz, item) : d.pz[0];
  const uint32_t* __restrict__ ps32 =
      reinterpret_cast<const uint32_t*>(GRP ? pick(d.ps, item) : d.ps[0]);
  const uint16_t* __restrict__ bias = GRP ? pick(d.bias, item) : d.bias[0];
  uint16_t* __restrict__ y = GRP ? pick(d.y, item) : d.y[0];
  const int64_t ldy = GRP ? pick(d.ldy, item) : d.ldy[0];
  const uint16_t* __restrict__ res = GRP ? pick(d.res, item) : d.res[0];
  const int64_t ldres = GRP ? pick(d.ldres, item) : d.ldres[0];
  const int split = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar math
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int KC = K / kChunkK;
  const int c0 = split * cps;
  const int nc = min(KC, c0 + cps) - c0;
  const int nch = wave < nc ? (nc - wave + WAVES - 1) / WAVES : 0;  // this wave's chunks
  const int nch_max = (cps + WAVES - 1) / WAVES;                      // region size
  const int gpc = G128 ? 1 : kChunkK / gs;  // metadata records per chunk
  const int rec = gpc * kMetaWords;         // metadata dwords per chunk

  // this wave's private LDS: activations [chunk][row][kLdx] then metadata
  _Float16* xw = reinterpret_cast<_Float16*>(smem) + (size_t)wave * nch_max * M * kLdx;
  uint32_t* mw = reinterpret_cast<uint32_t*>(reinterpret_cast<_Float16*>(smem) +
                                             (size_t)WAVES * nch_max * M * kLdx) +
                 (size_t)wave * nch_max * rec;

  const int xupc = M * 16;  // 16-byte activation units per chunk
  const int xunits = nch * xupc;
  // group size >= 128: a chunk's scale and zero words travel with its
  // weights in the ring (staging them costs an LDS round trip ahead of the
  // first MFMA); smaller groups stage their records
  const int munits = G128 ? 0 : nch * rec;
  // Unit u = ((i * M + m) * 16 + q): 16-byte piece q of row m of the wave's
  // i-th chunk.  i = (u >> 4) / M by the host's multiplier (no division in
  // the kernel: an integer divide is ~25 instructions ahead of every load).
  auto x_unit = [&](int u) -> h8 {
    const uint32_t v = (uint32_t)u >> 4;
    const int i = M == 1 ? (int)v : (int)__umulhi(v, mmag);
    const int m = (int)v - i * M;
    const int k = (c0 + wave + i * WAVES) * kChunkK + (u & 15) * 8;
    return load_x_unit<ACT>(x + (size_t)m * ldx, perm, k);
  };
  auto x_dst = [&](int u) -> _Float16* { return xw + (size_t)(u >> 4) * kLdx + (u & 15) * 8; };
  auto m_word = [&](int v) -> uint32_t {
    const int i = v / rec;
    const int r = v - i * rec;
    const int gl = r / kMetaWords;
    const int c = c0 + wave + i * WAVES;
    const int g = G128 ? (c * kChunkK) / gs : c * gpc + gl;
    return meta_word(ps32, pz, G, s, g, r - gl * kMetaWords);
  };

  // staging pass 0, issued before the weight ring so that waiting for it
  // does not wait for the ring
  h8 xv[kXBatch];
  uint32_t mv[kMBatch];
  // XG (act-order, M = 1): the activation row is copied whole into LDS after
  // the reduction region and each wave gathers its units from there by perm,
  // instead of 8 scattered 2-byte global loads per 16-byte unit.  The copy's
  // loads and the perm words of this lane's (at most kXgUnits) units are
  // issued ahead of the weight ring.
  _Float16* xg = reinterpret_cast<_Float16*>(
      smem + decode_staged_bytes(M, nch_max, rec, WAVES) + (size_t)WAVES * MT * 1024);
  constexpr int kXgCopy = (kXgMaxK / 8 + T - 1) / T;
  h8 xc[XG ? kXgCopy : 1];
  i4 pw[XG ? kXgUnits : 1][2];
  if constexpr (XG) {
#pragma unroll
    for (int b = 0; b < kXgCopy; ++b)
      if (tid + T * b < K / 8) xc[b] = *(const h8*)(x + 8 * (tid + T * b));
#pragma unroll
    for (int b = 0; b < kXgUnits; ++b) {
      const int u = lane + 64 * b;
      if (u < xunits) {
        const int k = (c0 + wave + (u >> 4) * WAVES) * kChunkK + (u & 15) * 8;
        pw[b][0] = *(const i4*)(perm + k);
        pw[b][1] = *(const i4*)(perm + k + 4);
      }
    }
  } else {
#pragma unroll
    for (int b = 0; b < kXBatch; ++b)
      if (lane + 64 * b < xunits) xv[b] = x_unit(lane + 64 * b);
  }
#pragma unroll
  for (int b = 0; b < kMBatch; ++b)
    if (lane + 64 * b < munits) mv[b] = m_word(lane + 64 * b);

  // weight ring.  With U >= 2 the host guarantees every wave at least U
  // chunks, so the prologue loads are unconditional.  Each slot holds the
  // lane's 4 packed words and, for groups of 128 or more, the dword with
  // its column's scale and the word with its column's stored zero.
  const u4* qp = pq + ((size_t)s * KC + c0) * 64 + lane;
  const uint32_t* sp = ps32 + (size_t)s * G * 8 + (j >> 1);
  const uint32_t* zp = pz + (size_t)s * G * 2 + (j >> 3);
  u4 qb[U];
  uint32_t sb[U], zb[U];
  auto ring_load = [&](u4& q, uint32_t& sw, uint32_t& zw, int i) {
    const int c = wave + i * WAVES;
    q = __builtin_nontemporal_load(qp + (size_t)c * 64);
    if (G128) {
      // group of chunk c0 + c: the chunk itself for 128-row groups, else the
      // host's multiplier for chunks per group
      const int g = gmag == 0 ? c0 + c : (int)__umulhi((uint32_t)(c0 + c), gmag);
      sw = sp[(size_t)g * 8];
      zw = zp[(size_t)g * 2];
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (U >= 2 || u < nch) ring_load(qb[u], sb[u], zb[u], u);

  if constexpr (XG) {
#pragma unroll
    for (int b = 0; b < kXgCopy; ++b)
      if (tid + T * b < K / 8) *(h8*)(xg + 8 * (tid + T * b)) = xc[b];
    // every wave's copy in LDS before any wave gathers; the weight ring's
    // loads stay in flight (a __syncthreads would wait for them too)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int b = 0; b < kXgUnits; ++b) {
      const int u = lane + 64 * b;
      if (u < xunits) {
        const i4 p0 = pw[b][0], p1 = pw[b][1];
        *(h8*)x_dst(u) = h8{xg[p0[0]], xg[p0[1]], xg[p0[2]], xg[p0[3]],
                            xg[p1[0]], xg[p1[1]], xg[p1[2]], xg[p1[3]]};
      }
    }
  } else {
#pragma unroll
    for (int b = 0; b < kXBatch; ++b)
      if (lane + 64 * b < xunits) *(h8*)x_dst(lane + 64 * b) = xv[b];
  }
#pragma unroll
  for (int b = 0; b < kMBatch; ++b)
    if (lane + 64 * b < munits) mw[lane + 64 * b] = mv[b];
  // The rest (M > 1 or many chunks) in batches: all loads of a batch are in
  // flight before its first store, so the staging costs one L2 round trip
  // per batch rather than one per 16-byte unit.
  for (int u0 = lane + 64 * kXBatch; !XG && u0 < xunits; u0 += 64 * kXBatch) {
#pragma unroll
    for (int b = 0; b < kXBatch; ++b)
      if (u0 + 64 * b < xunits) xv[b] = x_unit(u0 + 64 * b);
#pragma unroll
    for (int b = 0; b < kXBatch; ++b)
      if (u0 + 64 * b < xunits) *(h8*)x_dst(u0 + 64 * b) = xv[b];
  }
  for (int v0 = lane + 64 * kMBatch; v0 < munits; v0 += 64 * kMBatch) {
#pragma unroll
    for (int b = 0; b < kMBatch; ++b)
      if (v0 + 64 * b < munits) mv[b] = m_word(v0 + 64 * b);
#pragma unroll
    for (int b = 0; b < kMBatch; ++b)
      if (v0 + 64 * b < munits) mw[v0 + 64 * b] = mv[b];
  }
  // The wave reads back only what it wrote; LDS operations of one wave
  // complete in order, so no workgroup barrier is needed here.

  const int zsh = (j & 7) * 4;
  const uint32_t magic = opaque(kMagic);
  // A-operand rows: lanes past the last row read row M-1.  Output row i of
  // an MFMA depends only on A row i, and rows >= M are never stored.
  int xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = min(mt * 16 + j, M - 1) * kLdx + kq * 8;
  f4 tot[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) tot[mt] = f4{0.f, 0.f, 0.f, 0.f};

  // One chunk (the wave's i-th): 4 k-steps of 32 rows; w holds this lane's
  // 4 packed words, sw/zw its scale and zero words (groups >= 128).
  const int hsh = (j & 1) * 16;
  auto chunk = [&](const u4 w, uint32_t sw, uint32_t zw, int i) {
    const _Float16* xc = xw + (size_t)i * M * kLdx;
    const uint32_t* mr = mw + i * rec;
    f4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
    if (G128) {
      const float sc = (float)as_h((uint16_t)(sw >> hsh));
      h2 nz1024, nz64;
      zero_consts(zw, zsh, nz1024, nz64);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const h8 b = centered8(w[t], nz1024, nz64, magic);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const h8 a = *(const h8*)(xc + xrow[mt] + 32 * t);
          acc[mt] = mfma16(a, b, acc[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) tot[mt] += sc * acc[mt];
    } else {
      // group size 32 or 64: one or two k-steps per group
      const int spg = gs >> 5;
      float sc = 0.f;
      h2 nz1024, nz64;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t % spg == 0) {
          const uint32_t* mg = mr + (t / spg) * kMetaWords;
          sc = (float)reinterpret_cast<const _Float16*>(mg)[j];
          zero_consts(mg[8 + (j >> 3)], zsh, nz1024, nz64);
        }
        const h8 b = centered8(w[t], nz1024, nz64, magic);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const h8 a = *(const h8*)(xc + xrow[mt] + 32 * t);
          acc[mt] = mfma16(a, b, acc[mt]);
        }
        if (t % spg == spg - 1) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            tot[mt] += sc * acc[mt];
            acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
  };

  // Steady state: every consumed slot is refilled unconditionally, so the
  // only wait before a slot is for that slot (U - 1 newer loads pending).
  int i0 = 0;
  for (; i0 + 2 * U <= nch; i0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      chunk(qb[u], sb[u], zb[u], i0 + u);  // consume, then refill the same registers
      ring_load(qb[u], sb[u], zb[u], i0 + u + U);
    }
  }
  // Drain: at most 2U - 1 chunks left; refills only where a chunk remains.
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = i0 + u;
    if (i < nch) {
      chunk(qb[u], sb[u], zb[u], i);
      if (i + U < nch) ring_load(qb[u], sb[u], zb[u], i + U);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = i0 + U + u;
    if (i < nch) chunk(qb[u], sb[u], zb[u], i);
  }

  // the reduction region follows the staging regions
  f4* red = reinterpret_cast<f4*>(smem + decode_staged_bytes(M, nch_max, rec, WAVES));
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[(wave * MT + mt) * 64 + lane] = tot[mt];
  __syncthreads();

  const float* redf = reinterpret_cast<const float*>(red);
  const bool direct = gridDim.y == 1;
  for (int idx = tid; idx < MT * 256; idx += T) {
    const int llo = idx & 15;
    const int r = (idx >> 4) & 3;
    const int lhi = (idx >> 6) & 3;
    const int mt = idx >> 8;
    const int m = mt * 16 + lhi * 4 + r;
    if (m >= M) continue;
    const int L = lhi * 16 + llo;
    float sum = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) sum += redf[((wv * MT + mt) * 64 + L) * 4 + r];
    const int n = s * kStripN + llo;
    if (direct) {
      _Float16 out = (_Float16)sum;
      if (bias != nullptr) out = out + as_h(bias[n]);
      if (res != nullptr) out = out + as_h(res[(size_t)m * ldres + n]);
      y[(size_t)m * ldy + n] = h_bits(out);
    } else {
      part[((size_t)split * M + m) * N + n] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// Decode kernel, register-fed form (5 <= M <= 64).  The staged kernel above
// copies each strip's whole activation block into LDS before it starts; at
// M = 16 that block (M * K * 2 bytes per strip) exceeds what three
// workgroups per CU can hold, so the staged kernel splits K and runs in
// several rounds.  Here each wave loads its A fragments (16 bytes per lane
// per 32-row k-step, from L2) into the same register ring as the weights,
// and SS adjacent strips share them, so no LDS is needed until the final
// cross-wave reduction.  Every workgroup reads the A fragments of its whole
// K range, so L2 -> CU activation traffic is (strips / SS) * M * K * 2
// bytes: wider workgroups (SS = 4) with K split over gridDim.y workgroups
// (fp32 planes summed in split order by reduce_kernel) keep that traffic
// down where M * K is large, with the grid still filling the CUs.
// Pair mode (SS = 2): workgroup s holds strip s of item 0 (gate) and of item 1
// (up), which share perm, and writes fp16(silu(gate) * up) to item 0's
// output; the two products never reach memory.
// ---------------------------------------------------------------------------

// MODE: kRegSingle (one matrix, item 0 read directly), kRegGroup (several
// matrices, item looked up per workgroup), kRegPair (gate/up, above) or
// kRegBf16 (one matrix, bf16 activations and output, unsplit).
//
// bf16 mode: the B operands are the exact bf16 values 128 + q (no zero
// subtraction per fragment) on v_mfma_f32_16x16x32_bf16, and per group
//   sum_k x (q - z) = sum_k x (128 + q) - (128 + z) sum_k x,
// where sum_k x comes from one more MFMA per k-step against a bf16 ones
// operand (the row sums land in the accumulator layout, replicated over the
// columns); the scale is applied per group in fp32 as in the fp16 modes.
// Output bf16(sum) (+ bias in bf16 after the rounding, as the dense route's
// `y += bias`).  The weights are the fp16 checkpoint's s (q - z) unrounded,
// so the product is within rounding of the reference's bf16 route
// (reconstruct bf16(fp16(s (q - z))), then a bf16 GEMM).
constexpr int kRegSingle = 0, kRegGroup = 1, kRegPair = 2, kRegBf16 = 3;


template <int MT, int WAVES, int U, int SS, int GPC, bool ACT, int MODE>
__global__ void __launch_bounds__(WAVES * 64)
decode_reg_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, const Items d, int K,
                  int gs, int G, int cps, float* __restrict__ part) {
  constexpr bool PAIR = MODE == kRegPair;
  constexpr bool BF = MODE == kRegBf16;
  static_assert(!PAIR || SS == 2, "a pair workgroup holds one strip of each matrix");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int T = WAVES * 64;
  constexpr int SPG = 4 / GPC;  // 32-row k-steps per group
  const int item = MODE == kRegGroup ? item_of(d, blockIdx.x) : 0;
  const int s0 = PAIR ? (int)blockIdx.x : ((int)blockIdx.x - pick(d.wg0, item)) * SS;
  const int NS = pick(d.n, item) / kStripN;
  const int32_t* __restrict__ perm = pick(d.perm, item);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int KC = K / kChunkK;
  const int split = blockIdx.y;
  const int c_begin = split * cps;
  const int nc = min(KC, c_begin + cps) - c_begin;  // chunks of this split
  const int nch = wave < nc ? (nc - wave + WAVES - 1) / WAVES : 0;
  // A rows: lanes past the last row read row M-1 (never stored)
  const _Float16* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xr[mt] = x + (size_t)min(mt * 16 + j, M - 1) * ldx;
  // Without act-order the A fragments are loaded as whole 128-byte lines
  // (8 lanes per row; load b of a 64-row half h holds rows 8b + lane / 8,
  // k units 8h + lane % 8) -- half the L2 requests of loading them in the
  // MFMA operand order, which gives each 16-lane row group half a line --
  // and rearranged through this wave's own 4 KiB LDS region per row tile:
  // unit (row r, k unit v) at r * 16 + (v ^ f(r)), f(r) = (r & 1) * 8 + r / 2,
  // so the 16 rows of an operand read and the two rows of 8 lanes each of a
  // store both hit 16 distinct 16-byte bank groups.
  constexpr bool LX = decode_reg_lx(MT, SS, GPC, ACT);
  uint32_t xl[MT][2];  // element offsets from x (M * ldx < 2^31)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < 2; ++b)
      xl[mt][b] = (uint32_t)(min(mt * 16 + 8 * b + (lane >> 3), M - 1) * (int)ldx + 8 * (lane & 7));
  auto swz = [](int r, int v) { return r * 16 + (v ^ (((r & 1) << 3) | (r >> 1))); };
  const int wr_row = lane >> 3;  // + 8 b
  uint32_t xoff_w[4], xoff_r[4];  // byte offsets in the wave's region, per load / k-step
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    xoff_w[t] = (uint32_t)swz(8 * (t & 1) + wr_row, 8 * (t >> 1) + (lane & 7)) * 16;
    xoff_r[t] = (uint32_t)swz(j, 4 * t + kq) * 16;
  }
  unsigned char* xs = smem + (size_t)wave * MT * 4096;

  const u4* qp[SS];
  const uint32_t* sp[SS];
  const uint32_t* zp[SS];
#pragma unroll
  for (int ss = 0; ss < SS; ++ss) {
    const int src = PAIR ? ss : item;
    const int st = PAIR ? s0 : min(s0 + ss, NS - 1);
    qp[ss] = reinterpret_cast<const u4*>(pick(d.pq, src)) + (size_t)st * KC * 64 + lane;
    sp[ss] = reinterpret_cast<const uint32_t*>(pick(d.ps, src)) + (size_t)st * G * 8 + (j >> 1);
    zp[ss] = pick(d.pz, src) + (size_t)st * G * 2 + (j >> 3);
  }
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;

  u4 qb[U][SS];
  h8 ab[U][MT][4];
  uint32_t sb[U][SS][GPC], zb[U][SS][GPC];
  const int c0 = __builtin_amdgcn_readfirstlane(c_begin + wave);  // this wave's first chunk
  auto load = [&](int slot_u, int i) {
    const int c = c0 + i * WAVES;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if constexpr (LX)
          ab[slot_u][mt][t] = *(const h8*)(x + xl[mt][t & 1] + (size_t)c * kChunkK + 64 * (t >> 1));
        else
          ab[slot_u][mt][t] = load_x_unit<ACT>(xr[mt], perm, c * kChunkK + 32 * t + 8 * kq);
      }
#pragma unroll
    for (int ss = 0; ss < SS; ++ss) {
      qb[slot_u][ss] = __builtin_nontemporal_load(qp[ss] + (size_t)c * 64);
#pragma unroll
      for (int gl = 0; gl < GPC; ++gl) {
        const int g = GPC == 1 ? (c * kChunkK) / gs : c * GPC + gl;
        sb[slot_u][ss][gl] = sp[ss][(size_t)g * 8];
        zb[slot_u][ss][gl] = zp[ss][(size_t)g * 2];
      }
    }
  };
  f4 tot[SS][MT];
#pragma unroll
  for (int ss = 0; ss < SS; ++ss)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) tot[ss][mt] = f4{0.f, 0.f, 0.f, 0.f};
  const uint32_t magic = opaque(BF ? kMagicBf16 : kMagic);
  const u4 ones_bf16 = u4{kOnesBf16, kOnesBf16, kOnesBf16, kOnesBf16};
  auto consume = [&](int slot_u) {
    if constexpr (LX) {  // the slot's registers go out in load order, come back in operand order
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 4; ++t) *(h8*)(xs + mt * 4096 + xoff_w[t]) = ab[slot_u][mt][t];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 4; ++t) ab[slot_u][mt][t] = *(const h8*)(xs + mt * 4096 + xoff_r[t]);
    }
    if constexpr (BF) {
#pragma unroll
      for (int gl = 0; gl < GPC; ++gl) {
        f4 rsum[MT];  // sum of the group's x per row, in every column
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) rsum[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < SPG; ++tt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            rsum[mt] = mfma16_bf16(ab[slot_u][mt][gl * SPG + tt], ones_bf16, rsum[mt]);
#pragma unroll
        for (int ss = 0; ss < SS; ++ss) {
          const float zc = (float)(128u + ((zb[slot_u][ss][gl] >> zsh) & 15u) + 1u);
          const float sc = (float)as_h((uint16_t)(sb[slot_u][ss][gl] >> hsh));
          f4 acc[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tt = 0; tt < SPG; ++tt) {
            const int t = gl * SPG + tt;
            const u4 b = biased8_bf16(qb[slot_u][ss][t], magic);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16_bf16(ab[slot_u][mt][t], b, acc[mt]);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              tot[ss][mt][e] = fmaf(sc, fmaf(-zc, rsum[mt][e], acc[mt][e]), tot[ss][mt][e]);
        }
      }
      return;
    }
#pragma unroll
    for (int ss = 0; ss < SS; ++ss)
#pragma unroll
      for (int gl = 0; gl < GPC; ++gl) {
        h2 nz1024, nz64;
        zero_consts(zb[slot_u][ss][gl], zsh, nz1024, nz64);
        const float sc = (float)as_h((uint16_t)(sb[slot_u][ss][gl] >> hsh));
        f4 acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < SPG; ++tt) {
          const int t = gl * SPG + tt;
          const h8 b = centered8(qb[slot_u][ss][t], nz1024, nz64, magic);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16(ab[slot_u][mt][t], b, acc[mt]);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) tot[ss][mt] += sc * acc[mt];
      }
  };

  // Epilogue output idx (< SS * MT * 256) -> row m, strip st, column n.
  auto epi_pos = [&](int idx, int& m, int& st, int& n) {
    const int sm = idx >> 8;  // ss * MT + mt
    const int ss = sm / MT;
    const int mt = sm - ss * MT;
    m = mt * 16 + ((idx >> 6) & 3) * 4 + ((idx >> 4) & 3);
    st = s0 + ss;
    n = st * kStripN + (idx & 15);
  };
  // One row tile: the epilogue's bias and residual values are loaded before
  // the weight stream, so their latency hides under it instead of adding a
  // memory round trip after the cross-wave sum (the residual may be y
  // itself: each element is read and later written by the same thread).
  // Wider tiles load them in the epilogue (the registers would spill).
  constexpr bool PRE = !PAIR && MT == 1;
  constexpr int EPI = (SS * MT * 256 + T - 1) / T;  // epilogue outputs per thread
  uint16_t epi_bias[PRE ? EPI : 1], epi_res[PRE ? EPI : 1];
  if constexpr (PRE) {
    const uint16_t* __restrict__ bias = pick(d.bias, item);
    const uint16_t* __restrict__ res = pick(d.res, item);
    const int64_t ldres = pick(d.ldres, item);
    const bool planes = MODE == kRegSingle && gridDim.y > 1;  // the reduce adds them
#pragma unroll
    for (int e = 0; e < EPI; ++e) {
      epi_bias[e] = 0;
      epi_res[e] = 0;
      const int idx = tid + e * T;
      int m, st, n;
      epi_pos(idx, m, st, n);
      if (planes || idx >= SS * MT * 256 || m >= M || st >= NS) continue;
      if (bias != nullptr) epi_bias[e] = bias[n];
      if (res != nullptr) epi_res[e] = res[(size_t)m * ldres + n];
    }
  }

  // ring: the host gives every wave at least U chunks when U >= 2
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (U >= 2 || u < nch) load(u, u);
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

  // fixed-order reduction across waves, then fp16 (+ bias) output (the
  // reduction region overlaps other waves' A regions: all waves first)
  if constexpr (LX) __syncthreads();
  f4* red = reinterpret_cast<f4*>(smem);
#pragma unroll
  for (int ss = 0; ss < SS; ++ss)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[((wave * SS + ss) * MT + mt) * 64 + lane] = tot[ss][mt];
  __syncthreads();
  const float* redf = reinterpret_cast<const float*>(smem);
  auto wave_sum = [&](int sm, int L, int r) {
    float sum = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) sum += redf[((wv * SS * MT + sm) * 64 + L) * 4 + r];
    return sum;
  };
  if constexpr (PAIR) {
    const uint16_t* __restrict__ bg = d.bias[0];
    const uint16_t* __restrict__ bu = d.bias[1];
    uint16_t* __restrict__ h = d.y[0];
    const int64_t ldh = d.ldy[0];
    for (int idx = tid; idx < MT * 256; idx += T) {
      const int mt = idx >> 8;
      const int llo = idx & 15;
      const int r = (idx >> 4) & 3;
      const int lhi = (idx >> 6) & 3;
      const int m = mt * 16 + lhi * 4 + r;
      if (m >= M) continue;
      const int L = lhi * 16 + llo;
      const int n = s0 * kStripN + llo;
      _Float16 g = (_Float16)wave_sum(mt, L, r);
      _Float16 u = (_Float16)wave_sum(MT + mt, L, r);
      if (bg != nullptr) g = g + as_h(bg[n]);
      if (bu != nullptr) u = u + as_h(bu[n]);
      h[(size_t)m * ldh + n] = h_bits((_Float16)(silu_f32((float)g) * (float)u));
    }
  } else {
    const uint16_t* __restrict__ bias = pick(d.bias, item);
    uint16_t* __restrict__ y = pick(d.y, item);
    const int64_t ldy = pick(d.ldy, item);
    const uint16_t* __restrict__ res = pick(d.res, item);
    const int64_t ldres = pick(d.ldres, item);
    const int N = NS * kStripN;
    if constexpr (PRE) {  // one row tile: bias and residual prefetched
#pragma unroll
      for (int e = 0; e < EPI; ++e) {
        const int idx = tid + e * T;
        if (idx >= SS * MT * 256) break;
        int m, st, n;
        epi_pos(idx, m, st, n);
        if (m >= M || st >= NS) continue;
        const int sm = idx >> 8;
        const int L = ((idx >> 6) & 3) * 16 + (idx & 15);
        const int r = (idx >> 4) & 3;
        if constexpr (BF) {
          uint16_t o = bf16_rne(wave_sum(sm, L, r));
          if (bias != nullptr) o = bf16_rne(bf16_f32(o) + bf16_f32(epi_bias[e]));
          y[(size_t)m * ldy + n] = o;
          continue;
        }
        if (MODE == kRegSingle && gridDim.y > 1) {  // this split's fp32 plane
          part[((size_t)split * M + m) * N + n] = wave_sum(sm, L, r);
          continue;
        }
        _Float16 out = (_Float16)wave_sum(sm, L, r);
        if (bias != nullptr) out = out + as_h(epi_bias[e]);
        if (res != nullptr) out = out + as_h(epi_res[e]);
        y[(size_t)m * ldy + n] = h_bits(out);
      }
    } else {
      for (int idx = tid; idx < SS * MT * 256; idx += T) {
        const int sm = idx >> 8;  // ss * MT + mt
        const int ss = sm / MT;
        const int mt = sm - ss * MT;
        const int llo = idx & 15;
        const int r = (idx >> 4) & 3;
        const int lhi = (idx >> 6) & 3;
        const int m = mt * 16 + lhi * 4 + r;
        const int st = s0 + ss;
        if (m >= M || st >= NS) continue;
        const int L = lhi * 16 + llo;
        const int n = st * kStripN + llo;
        if constexpr (BF) {
          uint16_t o = bf16_rne(wave_sum(sm, L, r));
          if (bias != nullptr) o = bf16_rne(bf16_f32(o) + bf16_f32(bias[n]));
          y[(size_t)m * ldy + n] = o;
          continue;
        }
        if (MODE == kRegSingle && gridDim.y > 1) {  // this split's fp32 plane
          part[((size_t)split * M + m) * N + n] = wave_sum(sm, L, r);
          continue;
        }
        _Float16 out = (_Float16)wave_sum(sm, L, r);
        if (bias != nullptr) out = out + as_h(bias[n]);
        if (res != nullptr) out = out + as_h(res[(size_t)m * ldres + n]);
        y[(size_t)m * ldy + n] = h_bits(out);
      }
    }
  }
}

// Item table of a launch: item i gets ceil(strips_i / ss) workgroups.
static Items make_items(const GroupArgs& g, int ss) {
  Items d{};
  d.count = g.count;
  d.wg0[0] = 0;
  for (int i = 0; i < kGroupMax; ++i) {
    const GemmArgs& a = g.a[i < g.count ? i : 0];
    d.pq[i] = a.pq;
    d.pz[i] = a.pz;
    d.ps[i] = a.ps;
    d.perm[i] = a.perm;
    d.bias[i] = a.bias;
    d.y[i] = a.y;
    d.ldy[i] = a.ldy;
    d.res[i] = a.res;
    d.ldres[i] = a.ldres;
    d.n[i] = a.N;
    const int wgs = i < g.count ? (a.N / kStripN + ss - 1) / ss : 0;
    d.wg0[i + 1] = d.wg0[i] + wgs;
  }
  return d;
}

// K split of a register-fed launch: `splits` workgroups per strip group, each
// over `cps` chunks, partial sums in fp32 planes `part` ([split][M][N]).
struct RegSplit {
  int splits = 1;
  int cps = 0;
  float* part = nullptr;
};

template <int MT, int WAVES, int U, int SS, int GPC, bool ACT, int MODE>
static hipError_t launch_decode_reg_cfg(const GroupArgs& g, const Items& d, const RegSplit& sp,
                                        hipStream_t stream) {
  const GemmArgs& a = g.a[0];
  const dim3 grid((unsigned)(MODE == kRegPair ? a.N / kStripN : d.wg0[d.count]),
                  (unsigned)sp.splits);
  const size_t red_bytes = (size_t)WAVES * SS * MT * 64 * sizeof(f4);
  const size_t xs_bytes = decode_reg_lx(MT, SS, GPC, ACT) ? (size_t)WAVES * MT * 4096 : 0;
  const size_t smem = red_bytes > xs_bytes ? red_bytes : xs_bytes;
  if (smem > 64 * 1024) {
    static std::atomic<uint64_t> allowed{0};
    const hipError_t e = allow_lds(reinterpret_cast<const void*>(
                                       &decode_reg_kernel<MT, WAVES, U, SS, GPC, ACT, MODE>),
                                   smem, allowed);
    if (e != hipSuccess) return e;
  }
  decode_reg_kernel<MT, WAVES, U, SS, GPC, ACT, MODE><<<grid, WAVES * 64, smem, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, d, a.K, a.gs, a.G, sp.cps, sp.part);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || sp.splits == 1) return e;
  return launch_reduce_planes(sp.part, sp.splits, a.M, a.N, a.bias, a.y, a.ldy, a.res, a.ldres,
                              stream);
}

// Ring depth (chunks in flight per wave).  Two where the registers hold
// it: a deeper ring puts more of every wave's A-fragment and weight loads in
// its first burst, and the waves then wait longer for their first chunk.
// Measured against four for one row tile (M <= 16): grouped q/k/v M=8 12.3
// -> 9.8 us, M=16 13.3 -> 10.9; gate/up pair M=16 18.1 -> 16.8;
// 13824x5120 M=8 17.2 -> 15.3; 4096x11008 M=5 11.3 -> 9.6; no shape slower.
// The A fragments of one chunk take 16 * MT registers per lane (their
// act-order gathers more while in flight) and each strip's weight words 4
// more; 16-wave workgroups have 128 registers per lane, 8-wave ones 256.
constexpr int decode_reg_umax(int mt, int waves, int ss, int gpc, bool act) {
  return waves == 16 ? 2
         : ss == 4   ? (mt <= 2 ? 2 : 1)
         : mt == 1   ? 2
         : act       ? 1
                     : (mt == 2 ? 2 : 1);
}

// Ring depth U: the deepest allowed, at most the chunks of the shortest wave
// (of the shortest split).
template <int MT, int WAVES, int SS, int GPC, bool ACT, int MODE>
static hipError_t launch_decode_reg_u(const GroupArgs& g, const Items& d, const RegSplit& sp,
                                      hipStream_t stream) {
  const int kc = g.a[0].K / kChunkK;
  const int shortest = sp.splits > 1 ? kc - (sp.splits - 1) * sp.cps : kc;
  const int per_wave = shortest / WAVES;
  constexpr int umax = decode_reg_umax(MT, WAVES, SS, GPC, ACT);
  if constexpr (umax >= 4) {
    if (per_wave >= 4)
      return launch_decode_reg_cfg<MT, WAVES, 4, SS, GPC, ACT, MODE>(g, d, sp, stream);
  }
  if constexpr (umax >= 2) {
    if (per_wave >= 2)
      return launch_decode_reg_cfg<MT, WAVES, 2, SS, GPC, ACT, MODE>(g, d, sp, stream);
  }
  // 16 waves are planned only where every wave gets two chunks or more
  if constexpr (WAVES == 16) return hipErrorInvalidValue;
  else return launch_decode_reg_cfg<MT, WAVES, 1, SS, GPC, ACT, MODE>(g, d, sp, stream);
}

template <int MT, int WAVES, int SS, bool ACT, int MODE>
static hipError_t launch_decode_reg_g(const GroupArgs& g, const Items& d, const RegSplit& sp,
                                      hipStream_t stream) {
  const int gs = g.a[0].gs;
  const int gpc = gs >= kChunkK ? 1 : kChunkK / gs;
  if (gpc == 1) return launch_decode_reg_u<MT, WAVES, SS, 1, ACT, MODE>(g, d, sp, stream);
  // four strips of three or four row tiles, and the bf16 mode's two strips
  // of four row tiles, hold one group per chunk only (more per-chunk scale
  // and zero words do not fit the registers)
  if constexpr ((SS == 4 && MT >= 3) || (MODE == kRegBf16 && SS == 2 && MT == 4)) {
    return hipErrorInvalidValue;
  } else {
    if (gpc == 2) return launch_decode_reg_u<MT, WAVES, SS, 2, ACT, MODE>(g, d, sp, stream);
    return launch_decode_reg_u<MT, WAVES, SS, 4, ACT, MODE>(g, d, sp, stream);
  }
}

template <int MT, int WAVES, int SS, int MODE>
static hipError_t launch_decode_reg_w(const GroupArgs& g, const RegSplit& sp, hipStream_t stream) {
  if (g.a[0].perm == nullptr) {
    const Items d = make_items(g, MODE == kRegPair ? 1 : SS);
    return launch_decode_reg_g<MT, WAVES, SS, false, MODE>(g, d, sp, stream);
  }
  // act-order gathers for four tiles and two strips, or four strips, do
  // not fit the registers
  if constexpr (MODE != kRegPair && ((MT == 4 && SS == 2) || SS == 4)) {
    const Items d = make_items(g, 1);
    return launch_decode_reg_g<MT, WAVES, 1, true, MODE>(g, d, sp, stream);
  } else {
    const Items d = make_items(g, MODE == kRegPair ? 1 : SS);
    return launch_decode_reg_g<MT, WAVES, SS, true, MODE>(g, d, sp, stream);
  }
}

template <int MT, int MODE>
static hipError_t launch_decode_reg_mt(const GroupArgs& g, const DecodePlan& p,
                                       const RegSplit& sp, hipStream_t stream) {
  if (p.ss == 4) {  // planned for one to three row tiles only
    if constexpr (MODE == kRegSingle && MT <= 3) return launch_decode_reg_w<MT, 8, 4, MODE>(g, sp, stream);
    else return hipErrorInvalidValue;
  }
  return p.ss == 2 ? launch_decode_reg_w<MT, 8, 2, MODE>(g, sp, stream)
                   : launch_decode_reg_w<MT, 8, 1, MODE>(g, sp, stream);
}

// Grouped launches come from the automatic path, which takes decode only up
// to M = 32 (two row tiles), and are never split.
template <int MT>
static hipError_t launch_decode_reg_m(const GroupArgs& g, const DecodePlan& p, const RegSplit& sp,
                                      hipStream_t stream) {
  if (g.count == 1) return launch_decode_reg_mt<MT, kRegSingle>(g, p, sp, stream);
  if (sp.splits != 1) return hipErrorInvalidValue;
  if constexpr (MT <= 2) return launch_decode_reg_mt<MT, kRegGroup>(g, p, sp, stream);
  else return hipErrorInvalidValue;
}

hipError_t launch_decode_reg(const GroupArgs& g, const DecodePlan& p, float* part,
                             hipStream_t stream) {
  const int M = g.a[0].M;
  RegSplit sp;
  sp.splits = p.splits;
  sp.cps = p.cps;
  sp.part = part;
  if (sp.splits > 1 && (part == nullptr || g.count != 1)) return hipErrorInvalidValue;
  if (M <= 16) {
    if (p.waves == 16) {  // planner: ss == 1, unsplit
      if (sp.splits != 1) return hipErrorInvalidValue;
      return g.count == 1 ? launch_decode_reg_w<1, 16, 1, kRegSingle>(g, sp, stream)
                          : launch_decode_reg_w<1, 16, 1, kRegGroup>(g, sp, stream);
    }
    return launch_decode_reg_m<1>(g, p, sp, stream);
  }
  if (p.waves != 8) return hipErrorInvalidValue;
  if (M <= 32) return launch_decode_reg_m<2>(g, p, sp, stream);
  if (M <= 48) return launch_decode_reg_m<3>(g, p, sp, stream);
  if (M <= 64) return launch_decode_reg_m<4>(g, p, sp, stream);
  return hipErrorInvalidValue;
}

template <int MT>
static hipError_t launch_decode_reg_bf16_mt(const GroupArgs& g, const DecodePlan& p,
                                            const RegSplit& sp, hipStream_t stream) {
  if (p.ss == 1) return launch_decode_reg_w<MT, 8, 1, kRegBf16>(g, sp, stream);
  return launch_decode_reg_w<MT, 8, 2, kRegBf16>(g, sp, stream);
}

hipError_t launch_decode_reg_bf16(const GemmArgs& a, const DecodePlan& p, hipStream_t stream) {
  if (a.M < 1 || a.M > kBf16MaxM || !p.reg || p.splits != 1 || a.res != nullptr)
    return hipErrorInvalidValue;
  GroupArgs g{};
  g.count = 1;
  g.a[0] = a;
  const RegSplit sp{1, a.K / kChunkK, nullptr};
  if (p.waves == 16) {
    if (a.M > 16) return hipErrorInvalidValue;
    return launch_decode_reg_w<1, 16, 1, kRegBf16>(g, sp, stream);
  }
  if (p.waves != 8) return hipErrorInvalidValue;
  if (a.M <= 16) return launch_decode_reg_bf16_mt<1>(g, p, sp, stream);
  if (a.M <= 32) return launch_decode_reg_bf16_mt<2>(g, p, sp, stream);
  if (a.M <= 48) return launch_decode_reg_bf16_mt<3>(g, p, sp, stream);
  return launch_decode_reg_bf16_mt<4>(g, p, sp, stream);
}

hipError_t launch_decode_pair(const GroupArgs& g, uint16_t* h, int64_t ldh, hipStream_t stream) {
  if (g.count != 2 || g.a[0].N != g.a[1].N || g.a[0].perm != g.a[1].perm) return hipErrorInvalidValue;
  GroupArgs gp = g;
  gp.a[0].y = h;  // the pair's output goes where item 0's would
  gp.a[0].ldy = ldh;
  const int M = g.a[0].M;
  const RegSplit sp{1, g.a[0].K / kChunkK, nullptr};
  if (M <= 16) return launch_decode_reg_w<1, 8, 2, kRegPair>(gp, sp, stream);
  if (M <= kPairMaxM) return launch_decode_reg_w<2, 8, 2, kRegPair>(gp, sp, stream);
  return hipErrorInvalidValue;
}

// ceil(2^32 / d) for d >= 2 (0 for d = 1): floor(n / d) = umulhi(n, magic)
// exactly while n * d < 2^32 (the rounding excess of the magic, below one,
// then adds less than 1/d to n/d).  Chunk and row counts stay far below that.
static uint32_t div_magic(int d) {
  return d <= 1 ? 0u : (uint32_t)(((1ull << 32) + (uint64_t)d - 1) / (uint64_t)d);
}

template <int MT, int WAVES, int U, bool G128, bool ACT, bool GRP, bool XG = false>
static hipError_t launch_decode_one(const GemmArgs& a, const Items& d, const DecodePlan& p,
                                    float* part, hipStream_t stream) {
  const dim3 grid((unsigned)d.wg0[d.count], p.splits);
  if (p.smem > 64 * 1024) {
    static std::atomic<uint64_t> allowed{0};
    const hipError_t e = allow_lds(
        reinterpret_cast<const void*>(&decode_kernel<MT, WAVES, U, G128, ACT, GRP, XG>),
        kLdsPerCu, allowed);
    if (e != hipSuccess) return e;
  }
  decode_kernel<MT, WAVES, U, G128, ACT, GRP, XG><<<grid, WAVES * 64, p.smem, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, d, part, a.K, a.gs, a.G, p.cps, div_magic(a.M),
      G128 && a.gs > kChunkK ? div_magic(a.gs / kChunkK) : 0u);
  return hipGetLastError();
}

template <int MT, int WAVES, int U, bool G128, bool ACT>
static hipError_t launch_decode_cfg(const GroupArgs& g, const DecodePlan& p, float* part,
                                    hipStream_t stream) {
  const GemmArgs& a = g.a[0];
  if (p.splits > 1 && g.count != 1) return hipErrorInvalidValue;  // planes of one matrix
  const Items d = make_items(g, 1);
  hipError_t err;
  if (p.xg) {  // act-order M = 1 gathering from an LDS copy of x (planner-checked sizes)
    if constexpr (MT == 1 && ACT && G128) {
      if (g.count != 1 || a.M != 1 || a.K > kXgMaxK) return hipErrorInvalidValue;
      err = launch_decode_one<MT, WAVES, U, G128, ACT, false, true>(a, d, p, part, stream);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (g.count == 1) {
    err = launch_decode_one<MT, WAVES, U, G128, ACT, false>(a, d, p, part, stream);
  } else if constexpr (MT == 1) {  // the staged kernel is planned for M <= 4 only
    err = launch_decode_one<MT, WAVES, U, G128, ACT, true>(a, d, p, part, stream);
  } else {
    return hipErrorInvalidValue;
  }
  if (err != hipSuccess || p.splits == 1) return err;
  return launch_reduce_planes(part, p.splits, a.M, a.N, a.bias, a.y, a.ldy, a.res, a.ldres,
                              stream);
}

template <int MT, int WAVES, bool G128>
static hipError_t launch_decode_g(const GroupArgs& g, const DecodePlan& p, float* part,
                                  hipStream_t stream) {
  // Ring depth: the largest of 8, 4, 2 that every wave can fill (the shortest
  // wave gets floor(chunks / waves) chunks); 1 (conditional prologue)
  // otherwise.  Group sizes 32/64 keep more per-chunk state live, so their
  // rings are shallower to stay within registers.
  // (measured: deeper rings only lengthen the initial request burst that
  // every wave's activation loads queue behind)
  constexpr int UMAX = G128 ? (WAVES >= 16 ? 2 : kDecodeUMax) : (WAVES >= 16 ? 2 : 4);
  const GemmArgs& a = g.a[0];
  const int KC = a.K / kChunkK;
  const int last = min(p.cps, KC - (p.splits - 1) * p.cps);  // shortest split
  const int per_wave = last / WAVES;
  const bool act = a.perm != nullptr;
#define DW4_DECODE_U(UU)                                                                  \
  return act ? launch_decode_cfg<MT, WAVES, UU, G128, true>(g, p, part, stream)            \
             : launch_decode_cfg<MT, WAVES, UU, G128, false>(g, p, part, stream)
  if (UMAX >= 8 && per_wave >= 8) { DW4_DECODE_U(UMAX >= 8 ? 8 : 1); }
  if (UMAX >= 4 && per_wave >= 4) { DW4_DECODE_U(UMAX >= 4 ? 4 : 1); }
  if (per_wave >= 2) { DW4_DECODE_U(2); }
  DW4_DECODE_U(1);
#undef DW4_DECODE_U
}

template <int MT, int WAVES>
static hipError_t launch_decode_w(const GroupArgs& g, const DecodePlan& p, float* part,
                                  hipStream_t stream) {
  if ((g.a[0].gs % kChunkK) == 0) return launch_decode_g<MT, WAVES, true>(g, p, part, stream);
  return launch_decode_g<MT, WAVES, false>(g, p, part, stream);
}

template <int MT>
static hipError_t launch_decode_mt(const GroupArgs& g, const DecodePlan& p, float* part,
                                   hipStream_t stream) {
  if constexpr (MT == 1) {  // 4- and 16-wave workgroups are planned for M <= 16 only
    if (p.waves == 4) return launch_decode_w<MT, 4>(g, p, part, stream);
    if (p.waves == 16) return launch_decode_w<MT, 16>(g, p, part, stream);
  }
  return launch_decode_w<MT, 8>(g, p, part, stream);
}

static hipError_t launch_decode_any(const GroupArgs& g, const DecodePlan& p, float* part,
                                    hipStream_t stream) {
  if (p.reg) return launch_decode_reg(g, p, part, stream);
  switch ((g.a[0].M + 15) / 16) {
    case 1: return launch_decode_mt<1>(g, p, part, stream);
    case 2: return launch_decode_mt<2>(g, p, part, stream);
    case 3: return launch_decode_mt<3>(g, p, part, stream);
    case 4: return launch_decode_mt<4>(g, p, part, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode(const GemmArgs& a, const DecodePlan& p, float* part, hipStream_t stream) {
  GroupArgs g{};
  g.count = 1;
  g.a[0] = a;
  return launch_decode_any(g, p, part, stream);
}

hipError_t launch_decode_group(const GroupArgs& g, const DecodePlan& p, hipStream_t stream) {
  if (g.count < 1 || g.count > kGroupMax || p.splits != 1) return hipErrorInvalidValue;
  return launch_decode_any(g, p, nullptr, stream);
}

}  // namespace dw4
