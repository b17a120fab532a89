// gfx950 kernels for the GPTQ int4-weight / fp16-activation quantized Linear.
//
// Replaces, in function (not in structure), the reference's
// cuda_extends/exllama (q4_matrix.cu shuffle/make_sequential/reconstruct,
// q_gemm_kernel_gptq.cuh gemm_half_q_half_gptq_kernel, q4_matmul.cu
// reconstruct + cuBLAS) and the Marlin repack/GEMM.  Layouts and names of
// the packed buffers are documented in include/drofell_w4a16.h.
//
// Arithmetic contract (reference: operators/core/linear/real_quant.py:69-102)
//   W[k,n] = fp16_rne(scale[g(k),n] * (q[k,n] - (zero[g(k),n] + 1)))
//   y[m,n] = fp16_rne(sum_k x[m,k] * W[k,n])  (fp32 accumulation)
// The decode kernel factors the scale out of each group (fp32 products of
// exact small integers and fp16 activations, scaled in fp32), the prefill
// kernel multiplies by the scale in fp16 exactly as the reference's
// dequantiser does; both accumulate in fp32 on the MFMA units.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace dw4 {

// ---------------------------------------------------------------------------
// Load-time repack
// ---------------------------------------------------------------------------

// One thread per packed output word.
__global__ void repack_qweight_kernel(const uint32_t* __restrict__ qweight,
                                      const int32_t* __restrict__ perm,
                                      uint32_t* __restrict__ out, int K, int N) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)K * N / 8;
  if (o >= total) return;
  const int w = (int)(o & 3);
  const int lane = (int)((o >> 2) & 63);
  const size_t unit = o >> 8;  // chunk index over (strip, chunk)
  const int KC = K / kChunkK;
  const int c = (int)(unit % KC);
  const int s = (int)(unit / KC);
  const int n = s * kStripN + (lane & 15);
  const int k0 = c * kChunkK + 32 * w + 8 * (lane >> 4);
  uint32_t word = 0;
  if (perm == nullptr) {
    const uint32_t src = qweight[(size_t)(k0 >> 3) * N + n];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t nib = (src >> (4 * e)) & 15u;
      const int slot = (e & 1) ? 4 + (e >> 1) : (e >> 1);
      word |= nib << (4 * slot);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = perm[k0 + e];
      const uint32_t nib = (qweight[(size_t)(r >> 3) * N + n] >> (4 * (r & 7))) & 15u;
      const int slot = (e & 1) ? 4 + (e >> 1) : (e >> 1);
      word |= nib << (4 * slot);
    }
  }
  out[o] = word;
}

// scales [G, N] -> [N/16][G][16]; qzeros [G, N/8] -> [N/16][G][2].
__global__ void repack_meta_kernel(const uint16_t* __restrict__ scales,
                                   const uint32_t* __restrict__ qzeros,
                                   uint16_t* __restrict__ pscales,
                                   uint32_t* __restrict__ pzeros, int N, int G) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)G * N;
  if (o >= total) return;
  const int j = (int)(o & 15);
  const size_t sg = o >> 4;
  const int g = (int)(sg % G);
  const int s = (int)(sg / G);
  pscales[o] = scales[(size_t)g * N + s * kStripN + j];
  if (j < 2) pzeros[sg * 2 + j] = qzeros[(size_t)g * (N / 8) + 2 * s + j];
}

// xs[m][j] = x[m][perm[j]]: activations in the packed (group-sorted) row
// order, one 16-byte unit of 8 sorted rows per thread.  Act-order calls with
// register-fed or MFMA kernels gather once here instead of in every
// workgroup (each gathered unit is 8 two-byte loads at scattered addresses).
__global__ void gather_rows_kernel(const _Float16* __restrict__ x, int64_t ldx,
                                   const int32_t* __restrict__ perm, _Float16* __restrict__ xs,
                                   int K, int M) {
  const int upr = K / 8;
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= (int64_t)M * upr) return;
  const int m = (int)(u / upr);
  const int j = (int)(u - (int64_t)m * upr) * 8;
  *(h8*)(xs + (size_t)m * K + j) = load_x_unit<true>(x + (size_t)m * ldx, perm, j);
}

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
  const uint32_t magic = kMagic;
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
// matrices, item looked up per workgroup) or kRegPair (gate/up, above).
constexpr int kRegSingle = 0, kRegGroup = 1, kRegPair = 2;


template <int MT, int WAVES, int U, int SS, int GPC, bool ACT, int MODE>
__global__ void __launch_bounds__(WAVES * 64)
decode_reg_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, const Items d, int K,
                  int gs, int G, int cps, float* __restrict__ part) {
  constexpr bool PAIR = MODE == kRegPair;
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
  const uint32_t magic = kMagic;
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
  // four strips of three or four row tiles hold one group per chunk only
  // (more per-chunk scale and zero words do not fit the registers)
  if constexpr (SS == 4 && MT >= 3) {
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
  if (p.ss == 4) {
    if constexpr (MODE == kRegSingle) return launch_decode_reg_w<MT, 8, 4, MODE>(g, sp, stream);
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

// ---------------------------------------------------------------------------
// Prefill kernel, 16x16x32 MFMA form (used for 16-row tiles; larger tiles
// use prefill32_kernel below): 4 waves; workgroup tile (16*MT2) rows x (64*S)
// columns; waves split the columns (S strips each) and share the rows.
// Activations (L2-resident) are staged per 128-row chunk into double-
// buffered LDS one chunk ahead (gathered through perm for act-order).  Each
// wave streams its strips' packed words and their scale/zero words through a
// PB-deep register ring (the weights come from HBM, so the ring covers its
// latency), dequantises them to the exact fp16 weight
// fp16_rne(scale * (q - z)) -- the value the reference's dequantiser
// produces -- and feeds v_mfma_f32_16x16x32_f16 directly.  With split-K
// each split publishes an fp32 partial tile to the workspace and the last
// split of a tile to arrive sums them in split order (deterministic).
// ---------------------------------------------------------------------------
constexpr int kLdaPad = 8;
constexpr int kLda = kChunkK + kLdaPad;  // halfs per LDS row (272 bytes)

template <int MT2, int S, int PB, int GPC, bool ACT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
prefill_kernel(const _Float16* __restrict__ x, int64_t ldx, int M,
               const int32_t* __restrict__ perm,
               const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
               const uint32_t* __restrict__ ps32, const uint16_t* __restrict__ bias,
               uint16_t* __restrict__ y, int64_t ldy,
               const uint16_t* __restrict__ res, int64_t ldres, float* __restrict__ part,
               int* __restrict__ counters, int K, int N, int gs, int G, int chunks_per_split,
               int mtiles, int ntiles) {
  constexpr int BM = 16 * MT2;
  constexpr int UNITS = BM * 16 / 256;  // 16-byte activation units per thread per chunk
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kLda];

  // XCD-aware tile order: the M-tiles of one N-tile get block ids congruent
  // modulo 8, so they run on one XCD and share its L2 copy of the weights.
  const int b = blockIdx.x;
  const int q8 = b / (8 * mtiles);
  const int r8 = b % (8 * mtiles);
  const int mtile = r8 / 8;
  const int ntile = q8 * 8 + (r8 % 8);
  if (ntile >= ntiles) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int KC = K / kChunkK;
  const int split = blockIdx.y;
  const int c_begin = split * chunks_per_split;
  const int nchunks = min(KC, c_begin + chunks_per_split) - c_begin;
  const int m0 = mtile * BM;
  const int NS = N / kStripN;

  // activation staging: unit u -> (row, 16-byte column); rows past M read
  // row M-1 (their MFMA output rows are never stored)
  const _Float16* arow[UNITS];
  int aoff[UNITS];
#pragma unroll
  for (int i = 0; i < UNITS; ++i) {
    const int u = tid + 256 * i;
    arow[i] = x + (size_t)min(m0 + (u >> 4), M - 1) * ldx;
    aoff[i] = (u >> 4) * kLda + (u & 15) * 8;
  }
  auto load_a = [&](int c, h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i)
      regs[i] = load_x_unit<ACT>(arow[i], perm, c * kChunkK + ((tid + 256 * i) & 15) * 8);
  };
  auto store_a = [&](int buf, const h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i) *(h8*)(&As[buf][aoff[i]]) = regs[i];
  };

  // weight strips owned by this wave (the last N-tile may be partial)
  const int strip0 = ntile * 4 * S + wave * S;
  const u4* qp[S];
  const uint32_t* sp[S];  // dword holding this lane's fp16 scale (pair j & ~1, j | 1)
  const uint32_t* zp[S];
  bool sval[S];
#pragma unroll
  for (int si = 0; si < S; ++si) {
    const int st = strip0 + si;
    sval[si] = st < NS;
    const int sc = sval[si] ? st : 0;
    qp[si] = pq + ((size_t)sc * KC + c_begin) * 64 + lane;
    sp[si] = ps32 + (size_t)sc * G * 8 + (j >> 1);
    zp[si] = pz + (size_t)sc * G * 2 + (j >> 3);
  }
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;

  // ring slot: packed words plus, per group record, the scale and zero words
  u4 qb[PB][S];
  uint32_t sb[PB][S][GPC], zb[PB][S][GPC];
  auto load_b = [&](int slot_u, int i) {  // i: chunk index within the split
    const int c = c_begin + i;
#pragma unroll
    for (int si = 0; si < S; ++si) {
      qb[slot_u][si] = __builtin_nontemporal_load(qp[si] + (size_t)i * 64);
#pragma unroll
      for (int gl = 0; gl < GPC; ++gl) {
        const int g = GPC == 1 ? (c * kChunkK) / gs : c * GPC + gl;
        sb[slot_u][si][gl] = sp[si][(size_t)g * 8];
        zb[slot_u][si][gl] = zp[si][(size_t)g * 2];
      }
    }
  };

  f4 acc[MT2][S];
#pragma unroll
  for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
    for (int si = 0; si < S; ++si) acc[mt][si] = f4{0.f, 0.f, 0.f, 0.f};

  const uint32_t magic = kMagic;
  // One workgroup per CU, one wave per SIMD: a wave has to hide its own
  // latencies, so the four 32-row k-steps of a chunk are software pipelined
  // -- while the MFMAs of step t run, the wave reads the A fragments of step
  // t+1 from LDS and dequantises the B fragments of step t+1 -- and
  // activations are fetched two chunks ahead.
  auto dequant = [&](int slot_u, int t, h8 (&bop)[S]) {
    const int gl = GPC == 1 ? 0 : (t * GPC) / 4;
#pragma unroll
    for (int si = 0; si < S; ++si) {
      h2 nz1024, nz64;
      zero_consts(zb[slot_u][si][gl], zsh, nz1024, nz64);
      const _Float16 sc = as_h((uint16_t)(sb[slot_u][si][gl] >> hsh));
      const h8 d = centered8(qb[slot_u][si][t], nz1024, nz64, magic);
      const h8 s8 = h8{sc, sc, sc, sc, sc, sc, sc, sc};
      bop[si] = d * s8;  // fp16 product, round to nearest even
    }
  };
  auto compute = [&](int slot_u, int buf) {
    const _Float16* Ab = &As[buf][(size_t)j * kLda + 8 * kq];
    h8 af[2][MT2];
    h8 bop[2][S];
#pragma unroll
    for (int mt = 0; mt < MT2; ++mt) af[0][mt] = *(const h8*)(Ab + mt * 16 * kLda);
    dequant(slot_u, 0, bop[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < 3) {
#pragma unroll
        for (int mt = 0; mt < MT2; ++mt)
          af[(t + 1) & 1][mt] = *(const h8*)(Ab + mt * 16 * kLda + 32 * (t + 1));
        dequant(slot_u, t + 1, bop[(t + 1) & 1]);
      }
#pragma unroll
      for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
        for (int si = 0; si < S; ++si)
          acc[mt][si] = mfma16(af[t & 1][mt], bop[t & 1][si], acc[mt][si]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Activations travel global -> registers two chunks ahead of their use and
  // registers -> LDS one step ahead, so a step only waits for loads issued a
  // whole step earlier.  areg[i & 1] holds chunk i+2 while chunk i is
  // computed (PB is even, so the parity is a compile-time index).
  static_assert(PB % 2 == 0, "ring depth must be even");
  h8 areg[2][UNITS];
  // prologue: ring filled with the first PB chunks (only those that exist
  // when the split is shorter than the ring), chunk 0 in LDS, chunk 1 in
  // registers
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (u < nchunks) load_b(u, u);
  if (nchunks > 0) {
    load_a(c_begin, areg[0]);
    store_a(0, areg[0]);
  }
  if (nchunks > 1) load_a(c_begin + 1, areg[1]);
  __syncthreads();

  // One step: fetch chunk i+2's activations, compute chunk i from slot u,
  // refill slot u with chunk i + PB, publish chunk i+1's activations.
  auto step = [&](int u, int i, bool refill) {
    const int p = u & 1;  // == i & 1
    if (i + 2 < nchunks) load_a(c_begin + i + 2, areg[p]);
    compute(u, p);
    if (refill) load_b(u, i + PB);
    if (i + 1 < nchunks) store_a(p ^ 1, areg[p ^ 1]);
    __syncthreads();
  };
  int i0 = 0;
  for (; i0 + 2 * PB <= nchunks; i0 += PB) {
#pragma unroll
    for (int u = 0; u < PB; ++u) step(u, i0 + u, true);
  }
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (i0 + u < nchunks) step(u, i0 + u, i0 + u + PB < nchunks);
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (i0 + PB + u < nchunks) step(u, i0 + PB + u, false);

  _Float16 bv[S];
#pragma unroll
  for (int si = 0; si < S; ++si)
    bv[si] = (bias != nullptr && sval[si]) ? as_h(bias[(strip0 + si) * kStripN + j]) : (_Float16)0.f;
  // Output: the accumulator layout gives a lane four rows of one column, so
  // direct stores would be 2-byte stores, which the address unit processes
  // about one lane per cycle (~7 us per workgroup for a 64x256 tile).  Each
  // wave instead rounds its (16*MT2) x (16*S) tile to fp16 (adding the bias
  // after the rounding, like `y += bias` on an fp16 tensor), writes it in
  // row order to its own slice of the now idle activation buffers, and
  // stores whole 16-byte row segments.  Every caller has passed the last
  // barrier of the main loop, so no wave still reads the activations.
  constexpr int TW = 16 * S;       // tile width in halves
  constexpr int SEG = TW / 8;      // 16-byte segments per tile row
  constexpr int RPP = 64 / SEG;    // tile rows per 64-lane pass
  static_assert(4 * 16 * MT2 * TW <= 2 * BM * kLda, "output tiles fit in the activation buffers");
  const bool vec_y = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && (ldy % 8 == 0) &&
                     (res == nullptr ||
                      (((reinterpret_cast<uintptr_t>(res) & 15) == 0) && (ldres % 8 == 0)));
  auto write_tile = [&](auto&& val) {  // val(mt, si, r): fp32 result of that accumulator slot
    _Float16* T = &As[0][0] + wave * (16 * MT2 * TW);
#pragma unroll
    for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
      for (int si = 0; si < S; ++si)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          _Float16 out = (_Float16)val(mt, si, r);
          if (bias != nullptr) out = out + bv[si];
          T[(mt * 16 + kq * 4 + r) * TW + si * 16 + j] = out;
        }
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < 16 * MT2 / RPP; ++pass) {
      const int row = pass * RPP + lane / SEG;
      const int seg = lane % SEG;
      const int m = m0 + row;
      const int strip = strip0 + seg / 2;
      if (m < M && strip < NS) {
        u4 v = *(const u4*)&T[row * TW + seg * 8];
        const int col = strip * kStripN + (seg & 1) * 8;
        uint16_t* dst = y + (size_t)m * ldy + col;
        const uint16_t* rsrc = res != nullptr ? res + (size_t)m * ldres + col : nullptr;
        if (vec_y) {
          if (rsrc != nullptr) v = add_h8(v, *(const u4*)rsrc);
          *(u4*)dst = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            _Float16 lo = as_h((uint16_t)(v[e] & 0xFFFFu)), hi = as_h((uint16_t)(v[e] >> 16));
            if (rsrc != nullptr) {
              lo = lo + as_h(rsrc[2 * e]);
              hi = hi + as_h(rsrc[2 * e + 1]);
            }
            dst[2 * e] = h_bits(lo);
            dst[2 * e + 1] = h_bits(hi);
          }
        }
      }
    }
  };
  const int splits = gridDim.y;
  if (splits == 1) {
    write_tile([&](int mt, int si, int r) { return acc[mt][si][r]; });
    return;
  }

  // Split-K: publish this split's fp32 partial tile, count the arrivals for
  // the tile; the last split to arrive sums all partials in split order
  // (deterministic whatever the arrival order), writes y and resets the
  // counter for the next call.  No workgroup ever waits for another.
  //
  // Partials are written as relaxed agent-scope atomic stores, which gfx950
  // performs write-through (sc1): they leave no dirty L2 lines, so thread
  // 0's agent-scope release -- an L2 write-back -- has almost nothing to
  // write (with plain stores it had to flush every workgroup's partials and
  // cost several microseconds).  Layout per split plane (mtiles*ntiles*BM*BN
  // floats): [tile][mt*S + si][element e of the lane's float4][256 threads],
  // so each store instruction covers 256 contiguous bytes per wave.
  // Ordering is the usual publish/consume pattern: every wave waits for its
  // own stores to complete, the barrier then orders all of them before
  // thread 0's release and counter increment (a release covers only the
  // issuing wave's operations, and s_barrier does not wait for memory); the last
  // arriver's acquire (then the barrier) orders the other splits' partials
  // before its loads.  Fences run once per workgroup.
  const int tile_id = mtile * ntiles + ntile;
  const size_t plane = (size_t)mtiles * ntiles * (MT2 * S) * 1024;  // floats per split
  const size_t tbase = (size_t)tile_id * (MT2 * S) * 1024 + tid;
#pragma unroll
  for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
    for (int si = 0; si < S; ++si)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __hip_atomic_store(&part[(size_t)split * plane + tbase + (mt * S + si) * 1024 + e * 256],
                           acc[mt][si][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_own_stores();
  __shared__ int last_arrival;
  __syncthreads();
  if (tid == 0) {
    const int before = __hip_atomic_fetch_add(&counters[tile_id], 1, __ATOMIC_RELEASE,
                                              __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == splits - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    last_arrival = last;
  }
  __syncthreads();
  if (!last_arrival) return;
  // Sum in split order; per split all of this thread's loads are issued
  // before any is used (one memory round trip per split).
  f4 sum[MT2][S];
#pragma unroll
  for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
    for (int si = 0; si < S; ++si) sum[mt][si] = f4{0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < splits; ++sp) {
    f4 t[MT2][S];
#pragma unroll
    for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
      for (int si = 0; si < S; ++si) {
        const float* src = part + (size_t)sp * plane + tbase + (mt * S + si) * 1024;
        t[mt][si] = sp == split ? f4{acc[mt][si][0], acc[mt][si][1], acc[mt][si][2], acc[mt][si][3]}
                                : f4{src[0], src[256], src[512], src[768]};
      }
#pragma unroll
    for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
      for (int si = 0; si < S; ++si) sum[mt][si] += t[mt][si];
  }
  write_tile([&](int mt, int si, int r) { return sum[mt][si][r]; });
  if (tid == 0) __hip_atomic_store(&counters[tile_id], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Prefill kernel, 32x32x16 MFMA form (the default for M > 32).  Same
// workgroup tile, activation staging, weight ring and split-K protocol as
// prefill_kernel; each wave covers 32*MT3 rows x 32*P columns with
// v_mfma_f32_32x32x16_f16.  One wave alone issues that instruction at ~94%
// of the MFMA peak, where it issues the 16x16x32 form at ~55%, so the
// kernel no longer needs a second wave per SIMD to keep the matrix core fed.
//
// The packed layout stays the 16x16x32 one: word w of lane l of a strip
// holds rows 32w + 8(l/16) .. +7 of column l%16.  The 32x32x16 B operand of
// k-step t needs, in lane L, rows 16t + 8(L/32) .. +7 of column L%32 of a
// strip pair.  For two strips' word w (A in the first strip, B in the
// second, 16-lane rows A0..A3, B0..B3) that is [A0 B0 A1 B1] for t = 2w and
// [A2 B2 A3 B3] for t = 2w + 1: one v_permlane16_swap ([A0 B0 A2 B2],
// [A1 B1 A3 B3]) followed by one v_permlane32_swap.
// Accumulator element i of lane L is row 8(i/4) + 4(L/32) + i%4, column
// L%32 of the 32x32 tile.
// ---------------------------------------------------------------------------

template <int MT3, int P, int PB, int GPC, bool ACT>
__global__ void __launch_bounds__(256)
prefill32_kernel(const _Float16* __restrict__ x, int64_t ldx, int M,
                 const int32_t* __restrict__ perm,
                 const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
                 const uint32_t* __restrict__ ps32, const uint16_t* __restrict__ bias,
                 uint16_t* __restrict__ y, int64_t ldy,
                 const uint16_t* __restrict__ res, int64_t ldres, float* __restrict__ part,
                 int* __restrict__ counters, int K, int N, int gs, int G, int chunks_per_split,
                 int mtiles, int ntiles) {
  constexpr int S = 2 * P;               // 16-column strips per wave
  constexpr int BM = 32 * MT3;
  constexpr int UNITS = BM * 16 / 256;   // 16-byte activation units per thread per chunk
  constexpr int NSLOT = MT3 * P * 16;    // accumulator floats per lane
  static_assert(PB % 2 == 0, "ring depth must be even");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kLda];

  // XCD-aware tile order (as prefill_kernel)
  const int b = blockIdx.x;
  const int q8 = b / (8 * mtiles);
  const int r8 = b % (8 * mtiles);
  const int mtile = r8 / 8;
  const int ntile = q8 * 8 + (r8 % 8);
  if (ntile >= ntiles) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hb = lane >> 5;         // k half of the 32x32x16 operands
  const int hi = (lane >> 4) & 1;   // which strip of a pair this lane's B column is in
  const int j = lane & 15;
  const int KC = K / kChunkK;
  const int split = blockIdx.y;
  const int c_begin = split * chunks_per_split;
  const int nchunks = min(KC, c_begin + chunks_per_split) - c_begin;
  const int m0 = mtile * BM;
  const int NS = N / kStripN;

  const _Float16* arow[UNITS];
  int aoff[UNITS];
#pragma unroll
  for (int i = 0; i < UNITS; ++i) {
    const int u = tid + 256 * i;
    arow[i] = x + (size_t)min(m0 + (u >> 4), M - 1) * ldx;
    aoff[i] = (u >> 4) * kLda + (u & 15) * 8;
  }
  auto load_a = [&](int c, h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i)
      regs[i] = load_x_unit<ACT>(arow[i], perm, c * kChunkK + ((tid + 256 * i) & 15) * 8);
  };
  auto store_a = [&](int buf, const h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i) *(h8*)(&As[buf][aoff[i]]) = regs[i];
  };

  // packed words: strips strip0 .. strip0+S-1 (the last N-tile may be partial)
  const int strip0 = ntile * 4 * S + wave * S;
  const u4* qp[S];
#pragma unroll
  for (int si = 0; si < S; ++si) {
    const int st = strip0 + si;
    qp[si] = pq + ((size_t)(st < NS ? st : 0) * KC + c_begin) * 64 + lane;
  }
  // scale / zero words of this lane's B column in each strip pair
  const uint32_t* sp[P];
  const uint32_t* zp[P];
  bool pval[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int st = strip0 + 2 * p + hi;
    pval[p] = st < NS;
    const int sc = pval[p] ? st : 0;
    sp[p] = ps32 + (size_t)sc * G * 8 + (j >> 1);
    zp[p] = pz + (size_t)sc * G * 2 + (j >> 3);
  }
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;

  u4 qb[PB][S];
  uint32_t sb[PB][P][GPC], zb[PB][P][GPC];
  auto load_b = [&](int slot_u, int i) {
    const int c = c_begin + i;
#pragma unroll
    for (int si = 0; si < S; ++si) qb[slot_u][si] = __builtin_nontemporal_load(qp[si] + (size_t)i * 64);
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int gl = 0; gl < GPC; ++gl) {
        const int g = GPC == 1 ? (c * kChunkK) / gs : c * GPC + gl;
        sb[slot_u][p][gl] = sp[p][(size_t)g * 8];
        zb[slot_u][p][gl] = zp[p][(size_t)g * 2];
      }
  };

  f16v acc[MT3][P];
#pragma unroll
  for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mt][p][e] = 0.f;

  const uint32_t magic = kMagic;
  // Software pipeline over the 8 k-steps of a chunk: the region of step t
  // holds the MFMAs of step t (operands dequantised in the previous region)
  // and the dequantisation and A-fragment reads of step t+1, independent
  // work the scheduler can interleave.  (Measured on gfx950: a wave's dequant
  // VALU and its own 32x32x16 MFMAs hardly overlap, whatever the order, so
  // the cost per chunk is close to their sum; the VALU per MFMA is what
  // bounds this kernel.)
  auto dequant_step = [&](int slot_u, int t, h8 (&bop)[P]) {
    const int w = t >> 1;
    const int gl = GPC == 1 ? 0 : (t * GPC) / 8;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      uint32_t ev, od;
      strip_pair_to_b32(qb[slot_u][2 * p][w], qb[slot_u][2 * p + 1][w], ev, od);
      h2 nz1024, nz64;
      zero_consts(zb[slot_u][p][gl], zsh, nz1024, nz64);
      const _Float16 sc = as_h((uint16_t)(sb[slot_u][p][gl] >> hsh));
      const h8 d = centered8((t & 1) ? od : ev, nz1024, nz64, magic);
      const h8 s8 = h8{sc, sc, sc, sc, sc, sc, sc, sc};
      bop[p] = d * s8;  // fp16 product, round to nearest even
    }
  };
  auto compute = [&](int slot_u, int buf) {
    const _Float16* Ab = &As[buf][(size_t)l32 * kLda + 8 * hb];
    h8 bop[2][P];
    h8 af[2][MT3];
    dequant_step(slot_u, 0, bop[0]);
#pragma unroll
    for (int mt = 0; mt < MT3; ++mt) af[0][mt] = *(const h8*)(Ab + mt * 32 * kLda);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int cur = t & 1;
      if (t < 7) {
#pragma unroll
        for (int mt = 0; mt < MT3; ++mt)
          af[cur ^ 1][mt] = *(const h8*)(Ab + mt * 32 * kLda + 16 * (t + 1));
        dequant_step(slot_u, t + 1, bop[cur ^ 1]);
      }
#pragma unroll
      for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
        for (int p = 0; p < P; ++p) acc[mt][p] = mfma32(af[cur][mt], bop[cur][p], acc[mt][p]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // activations two chunks ahead in registers, one step ahead in LDS
  h8 areg[2][UNITS];
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (u < nchunks) load_b(u, u);
  if (nchunks > 0) {
    load_a(c_begin, areg[0]);
    store_a(0, areg[0]);
  }
  if (nchunks > 1) load_a(c_begin + 1, areg[1]);
  __syncthreads();
  auto step = [&](int u, int i, bool refill) {
    const int pp = u & 1;  // == i & 1
    if (i + 2 < nchunks) load_a(c_begin + i + 2, areg[pp]);
    compute(u, pp);
    if (refill) load_b(u, i + PB);
    if (i + 1 < nchunks) store_a(pp ^ 1, areg[pp ^ 1]);
    __syncthreads();
  };
  int i0 = 0;
  for (; i0 + 2 * PB <= nchunks; i0 += PB) {
#pragma unroll
    for (int u = 0; u < PB; ++u) step(u, i0 + u, true);
  }
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (i0 + u < nchunks) step(u, i0 + u, i0 + u + PB < nchunks);
#pragma unroll
  for (int u = 0; u < PB; ++u)
    if (i0 + PB + u < nchunks) step(u, i0 + PB + u, false);

  // Output through LDS in row order, 16-byte row segments (see prefill_kernel)
  constexpr int TW = 32 * P;
  constexpr int SEG = TW / 8;
  constexpr int RPP = 64 / SEG;
  static_assert(4 * BM * TW <= 2 * BM * kLda, "output tiles fit in the activation buffers");
  _Float16 bv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int st = strip0 + 2 * p + hi;
    bv[p] = (bias != nullptr && st < NS) ? as_h(bias[st * kStripN + j]) : (_Float16)0.f;
  }
  const bool vec_y = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && (ldy % 8 == 0) &&
                     (res == nullptr ||
                      (((reinterpret_cast<uintptr_t>(res) & 15) == 0) && (ldres % 8 == 0)));
  auto write_tile = [&](auto&& val) {  // val(mt, p, i): fp32 result of that accumulator slot
    _Float16* T = &As[0][0] + wave * (BM * TW);
#pragma unroll
    for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          _Float16 out = (_Float16)val(mt, p, i);
          if (bias != nullptr) out = out + bv[p];
          T[(mt * 32 + 8 * (i >> 2) + 4 * hb + (i & 3)) * TW + p * 32 + l32] = out;
        }
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < BM / RPP; ++pass) {
      const int row = pass * RPP + lane / SEG;
      const int seg = lane % SEG;
      const int m = m0 + row;
      const int strip = strip0 + seg / 2;
      if (m < M && strip < NS) {
        u4 v = *(const u4*)&T[row * TW + seg * 8];
        const int col = strip * kStripN + (seg & 1) * 8;
        uint16_t* dst = y + (size_t)m * ldy + col;
        const uint16_t* rsrc = res != nullptr ? res + (size_t)m * ldres + col : nullptr;
        if (vec_y) {
          if (rsrc != nullptr) v = add_h8(v, *(const u4*)rsrc);
          *(u4*)dst = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            _Float16 lo = as_h((uint16_t)(v[e] & 0xFFFFu)), hi = as_h((uint16_t)(v[e] >> 16));
            if (rsrc != nullptr) {
              lo = lo + as_h(rsrc[2 * e]);
              hi = hi + as_h(rsrc[2 * e + 1]);
            }
            dst[2 * e] = h_bits(lo);
            dst[2 * e + 1] = h_bits(hi);
          }
        }
      }
    }
  };
  const int splits = gridDim.y;
  if (splits == 1) {
    write_tile([&](int mt, int p, int i) { return acc[mt][p][i]; });
    return;
  }

  // Split-K: write-through partials, last arriver sums in split order (as
  // prefill_kernel).  Layout per split plane: [tile][slot][256 threads],
  // slot = (mt * P + p) * 16 + i.
  const int tile_id = mtile * ntiles + ntile;
  const size_t plane = (size_t)mtiles * ntiles * NSLOT * 256;
  const size_t tbase = (size_t)tile_id * NSLOT * 256 + tid;
#pragma unroll
  for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __hip_atomic_store(&part[(size_t)split * plane + tbase + ((mt * P + p) * 16 + i) * 256],
                           acc[mt][p][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_own_stores();
  __shared__ int last_arrival;
  __syncthreads();
  if (tid == 0) {
    const int before = __hip_atomic_fetch_add(&counters[tile_id], 1, __ATOMIC_RELEASE,
                                              __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == splits - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    last_arrival = last;
  }
  __syncthreads();
  if (!last_arrival) return;
  f16v sum[MT3][P];
#pragma unroll
  for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int i = 0; i < 16; ++i) sum[mt][p][i] = 0.f;
  for (int sp2 = 0; sp2 < splits; ++sp2) {
    if (sp2 == split) {
#pragma unroll
      for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
        for (int p = 0; p < P; ++p) sum[mt][p] += acc[mt][p];
      continue;
    }
    const float* src = part + (size_t)sp2 * plane + tbase;
#pragma unroll
    for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        f16v t;
#pragma unroll
        for (int i = 0; i < 16; ++i) t[i] = src[((mt * P + p) * 16 + i) * 256];
        sum[mt][p] += t;
      }
  }
  write_tile([&](int mt, int p, int i) { return sum[mt][p][i]; });
  if (tid == 0) __hip_atomic_store(&counters[tile_id], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void reduce_kernel(const float* __restrict__ part, int splits, int M, int N,
                              const uint16_t* __restrict__ bias,
                              uint16_t* __restrict__ y, int64_t ldy,
                              const uint16_t* __restrict__ res, int64_t ldres, bool vec) {
  // eight consecutive outputs of one row per thread (N is a multiple of 16)
  const size_t o = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const size_t total = (size_t)M * N;
  if (o >= total) return;
  f4 s0 = *(const f4*)(part + o), s1 = *(const f4*)(part + o + 4);
  for (int sidx = 1; sidx < splits; ++sidx) {  // split order, as the planes were cut
    s0 += *(const f4*)(part + (size_t)sidx * total + o);
    s1 += *(const f4*)(part + (size_t)sidx * total + o + 4);
  }
  const int m = (int)(o / N);
  const int n = (int)(o % N);
  uint16_t* dst = y + (size_t)m * ldy + n;
  const uint16_t* rsrc = res != nullptr ? res + (size_t)m * ldres + n : nullptr;
  u4 packed;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    _Float16 out = (_Float16)(e < 4 ? s0[e] : s1[e - 4]);
    if (bias != nullptr) out = out + as_h(bias[n + e]);
    if (rsrc != nullptr) out = out + as_h(rsrc[e]);
    if (vec) {
      const uint32_t h = h_bits(out);
      packed[e / 2] = (e & 1) ? (packed[e / 2] | (h << 16)) : h;
    } else {
      dst[e] = h_bits(out);
    }
  }
  if (vec) *(u4*)dst = packed;
}

// ---------------------------------------------------------------------------
// Bit-exact dequantisation to the original row order (one thread per 16-byte
// lane unit = 32 weights).  BF16 writes the fp16 value converted to bf16
// (round to nearest even; a NaN stays a NaN with the quiet bit set).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint16_t bf16_of_h(_Float16 v) {
  const uint32_t f = __builtin_bit_cast(uint32_t, (float)v);  // exact widening
  if ((f & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((f >> 16) | 0x40u);
  return (uint16_t)((f + 0x7fffu + ((f >> 16) & 1u)) >> 16);
}

template <bool BF16>
__global__ void dequant_kernel(const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
                               const uint16_t* __restrict__ ps, const int32_t* __restrict__ perm,
                               uint16_t* __restrict__ w, int64_t ldw, int K, int N, int gs, int G) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)K * N / 32;
  if (o >= total) return;
  const int lane = (int)(o & 63);
  const size_t unit = o >> 6;
  const int KC = K / kChunkK;
  const int c = (int)(unit % KC);
  const int s = (int)(unit / KC);
  const int j = lane & 15;
  const int n = s * kStripN + j;
  const u4 q = pq[o];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int k0 = c * kChunkK + 32 * t + 8 * (lane >> 4);
    const int g = k0 / gs;
    const uint32_t zw = pz[((size_t)s * G + g) * 2 + (j >> 3)];
    const int ze = (int)((zw >> ((j & 7) * 4)) & 15u) + 1;
    const _Float16 sc = as_h(ps[((size_t)s * G + g) * 16 + j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int slot = (e & 1) ? 4 + (e >> 1) : (e >> 1);
      const int qv = (int)((q[t] >> (4 * slot)) & 15u);
      // One IEEE fp16 multiply (round to nearest even) of the scale and the
      // exact integer |q - z| <= 16.  Not written as an fp32 product
      // narrowed to fp16: that form may be contracted into a mixed-precision
      // FMA with a +0 addend, which turns a -0 product into +0.
      const _Float16 v = sc * (_Float16)(qv - ze);
      const int k = k0 + e;
      const int row = perm ? perm[k] : k;
      w[(size_t)row * ldw + n] = BF16 ? bf16_of_h(v) : h_bits(v);
    }
  }
}

// ---------------------------------------------------------------------------
// Calibration: a plain streaming read in a decode-like launch shape.
// Workgroup b reads the contiguous byte range [b * per_wg, (b + 1) * per_wg)
// of src; its waves take 1 KiB chunks round-robin (chunk i of the workgroup
// goes to wave i % waves), each lane one 16-byte non-temporal load per
// chunk, kRing chunks in flight per wave.  The words are folded into one
// value per lane that is stored only if it equals `never` (the caller passes
// a value the data cannot fold to), so the loads stay live without a store
// stream.  This is the ceiling a weight-streaming kernel of the same launch
// shape can reach.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
stream_read_kernel(const u4* __restrict__ src, int chunks_per_wg, uint32_t never,
                   uint32_t* __restrict__ sink) {
  constexpr int kRing = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const u4* base = src + (size_t)blockIdx.x * chunks_per_wg * 64 + lane;
  u4 acc = u4{0u, 0u, 0u, 0u};
  int c = wave;
  for (; c + (kRing - 1) * waves < chunks_per_wg; c += kRing * waves) {
    u4 r[kRing];
#pragma unroll
    for (int u = 0; u < kRing; ++u) r[u] = __builtin_nontemporal_load(base + (size_t)(c + u * waves) * 64);
#pragma unroll
    for (int u = 0; u < kRing; ++u) acc ^= r[u];
  }
  for (; c < chunks_per_wg; c += waves) acc ^= __builtin_nontemporal_load(base + (size_t)c * 64);
  const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (v == never) sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = v;
}

hipError_t launch_stream_read(const void* src, int workgroups, int threads, int chunks_per_wg,
                              uint32_t never, uint32_t* sink, hipStream_t stream) {
  stream_read_kernel<<<(unsigned)workgroups, (unsigned)threads, 0, stream>>>(
      static_cast<const u4*>(src), chunks_per_wg, never, sink);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Launchers (called from the C ABI in w4a16_capi.hip)
// ---------------------------------------------------------------------------

hipError_t launch_repack(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                         const int32_t* perm, uint32_t* pq, uint32_t* pz, uint16_t* ps,
                         int K, int N, int G, hipStream_t stream) {
  const size_t words = (size_t)K * N / 8;
  repack_qweight_kernel<<<(unsigned)((words + 255) / 256), 256, 0, stream>>>(qweight, perm, pq, K, N);
  const size_t metas = (size_t)G * N;
  repack_meta_kernel<<<(unsigned)((metas + 255) / 256), 256, 0, stream>>>(scales, qzeros, ps, pz, N, G);
  return hipGetLastError();
}

// ceil(2^32 / d) for d >= 2 (0 for d = 1): floor(n / d) = umulhi(n, magic)
// exactly while n * d < 2^32 (the rounding excess of the magic, below one,
// then adds less than 1/d to n/d).  Chunk and row counts stay far below that.
static uint32_t div_magic(int d) {
  return d <= 1 ? 0u : (uint32_t)(((1ull << 32) + (uint64_t)d - 1) / (uint64_t)d);
}

hipError_t launch_gather_rows(const uint16_t* x, int64_t ldx, const int32_t* perm, uint16_t* xs,
                              int K, int M, hipStream_t stream) {
  const int64_t units = (int64_t)M * (K / 8);
  gather_rows_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream>>>(
      reinterpret_cast<const _Float16*>(x), ldx, perm, reinterpret_cast<_Float16*>(xs), K, M);
  return hipGetLastError();
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

template <int MT2, int S, int PB, int GPC, bool ACT>
static hipError_t launch_prefill_cfg(const GemmArgs& a, int splits, void* ws, hipStream_t stream) {
  constexpr int BM = 16 * MT2;
  constexpr int BN = 64 * S;
  const int mtiles = (a.M + BM - 1) / BM;
  const int ntiles = (a.N + BN - 1) / BN;
  const int KC = a.K / kChunkK;
  const int cps = (KC + splits - 1) / splits;
  const int real_splits = (KC + cps - 1) / cps;
  if (real_splits > 1 && mtiles * ntiles > kSplitCounters) return hipErrorInvalidValue;
  int* counters = static_cast<int*>(ws);
  float* part = real_splits > 1
                    ? reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + kWsHeadBytes)
                    : nullptr;
  const dim3 grid((unsigned)(((ntiles + 7) / 8) * 8 * mtiles), (unsigned)real_splits);
  prefill_kernel<MT2, S, PB, GPC, ACT><<<grid, 256, 0, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, a.perm, (const u4*)a.pq, a.pz, (const uint32_t*)a.ps,
      a.bias, a.y, a.ldy, a.res, a.ldres, part, counters, a.K, a.N, a.gs, a.G, cps, mtiles, ntiles);
  return hipGetLastError();
}

template <int MT3, int P, int PB, int GPC, bool ACT>
static hipError_t launch_prefill32_cfg(const GemmArgs& a, int splits, void* ws, hipStream_t stream) {
  constexpr int BM = 32 * MT3;
  constexpr int BN = 128 * P;
  const int mtiles = (a.M + BM - 1) / BM;
  const int ntiles = (a.N + BN - 1) / BN;
  const int KC = a.K / kChunkK;
  const int cps = (KC + splits - 1) / splits;
  const int real_splits = (KC + cps - 1) / cps;
  if (real_splits > 1 && mtiles * ntiles > kSplitCounters) return hipErrorInvalidValue;
  int* counters = static_cast<int*>(ws);
  float* part = real_splits > 1
                    ? reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + kWsHeadBytes)
                    : nullptr;
  const dim3 grid((unsigned)(((ntiles + 7) / 8) * 8 * mtiles), (unsigned)real_splits);
  prefill32_kernel<MT3, P, PB, GPC, ACT><<<grid, 256, 0, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, a.perm, (const u4*)a.pq, a.pz, (const uint32_t*)a.ps,
      a.bias, a.y, a.ldy, a.res, a.ldres, part, counters, a.K, a.N, a.gs, a.G, cps, mtiles, ntiles);
  return hipGetLastError();
}

template <int MT3, int P, int PB>
static hipError_t launch_prefill32_tile(const GemmArgs& a, int splits, void* part, hipStream_t stream) {
  const bool act = a.perm != nullptr;
  const int gpc = a.gs >= kChunkK ? 1 : kChunkK / a.gs;
#define DW4_PREFILL32_G(GG)                                                            \
  return act ? launch_prefill32_cfg<MT3, P, PB, GG, true>(a, splits, part, stream)    \
             : launch_prefill32_cfg<MT3, P, PB, GG, false>(a, splits, part, stream)
  if (gpc == 1) { DW4_PREFILL32_G(1); }
  if (gpc == 2) { DW4_PREFILL32_G(2); }
  DW4_PREFILL32_G(4);
#undef DW4_PREFILL32_G
}

template <int MT2, int S, int PB>
static hipError_t launch_prefill_tile(const GemmArgs& a, int splits, void* part, hipStream_t stream) {
  const bool act = a.perm != nullptr;
  const int gpc = a.gs >= kChunkK ? 1 : kChunkK / a.gs;
#define DW4_PREFILL_G(GG)                                                          \
  return act ? launch_prefill_cfg<MT2, S, PB, GG, true>(a, splits, part, stream)    \
             : launch_prefill_cfg<MT2, S, PB, GG, false>(a, splits, part, stream)
  if (gpc == 1) { DW4_PREFILL_G(1); }
  if (gpc == 2) { DW4_PREFILL_G(2); }
  DW4_PREFILL_G(4);
#undef DW4_PREFILL_G
}

hipError_t launch_prefill(const GemmArgs& a, const PrefillPlan& plan, void* part, hipStream_t stream) {
  // Waves split the columns: 64 (bn = 256) or 32 (bn = 128) per wave.  Four
  // 16-column strips per wave give each LDS activation read four MFMA uses;
  // measured LDS bandwidth (~128 B/clk/CU) makes fewer LDS-bound.
  if (plan.bm == 16 && plan.bn == 256) return launch_prefill_tile<1, 4, 4>(a, plan.splits, part, stream);
  if (plan.bm == 16 && plan.bn == 128) return launch_prefill_tile<1, 2, 4>(a, plan.splits, part, stream);
  if (plan.bm == 32 && plan.bn == 256) return launch_prefill32_tile<1, 2, 4>(a, plan.splits, part, stream);
  if (plan.bm == 32 && plan.bn == 128) return launch_prefill32_tile<1, 1, 4>(a, plan.splits, part, stream);
  if (plan.bm == 64 && plan.bn == 256) return launch_prefill32_tile<2, 2, 4>(a, plan.splits, part, stream);
  if (plan.bm == 64 && plan.bn == 128) return launch_prefill32_tile<2, 1, 4>(a, plan.splits, part, stream);
  if (plan.bm == 128 && plan.bn == 256) return launch_prefill32_tile<4, 2, 2>(a, plan.splits, part, stream);
  if (plan.bm == 128 && plan.bn == 128) return launch_prefill32_tile<4, 1, 4>(a, plan.splits, part, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_reduce_planes(const float* part, int splits, int M, int N, const uint16_t* bias,
                                uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldres,
                                hipStream_t stream) {
  const size_t units = (size_t)M * N / 8;
  const bool vec = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && (ldy % 8 == 0);
  reduce_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream>>>(part, splits, M, N, bias, y,
                                                                     ldy, res, ldres, vec);
  return hipGetLastError();
}

hipError_t launch_dequant(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                          const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs, int G,
                          hipStream_t stream) {
  const size_t total = (size_t)K * N / 32;
  dequant_kernel<false><<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
      (const u4*)pq, pz, ps, perm, w, ldw, K, N, gs, G);
  return hipGetLastError();
}

hipError_t launch_dequant_bf16(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                               const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs,
                               int G, hipStream_t stream) {
  const size_t total = (size_t)K * N / 32;
  dequant_kernel<true><<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
      (const u4*)pq, pz, ps, perm, w, ldw, K, N, gs, G);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decoder-stage helpers around the GEMM (reference: cuda_extends/exllama/
// fuse_v2/rms_norm.cu and q_mlp.cu silu_mul_kernel, restated).
// ---------------------------------------------------------------------------

// h = fp16(silu(g) * u), one element per thread; h may be g itself.
__global__ void silu_mul_kernel(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu,
                                uint16_t* h, int64_t ldh, int m, int n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)m * n) return;
  const int64_t r = i / n;
  const int64_t c = i - r * n;
  const float gv = (float)as_h(g[r * ldg + c]);
  const float uv = (float)as_h(u[r * ldu + c]);
  h[r * ldh + c] = h_bits((_Float16)(silu_f32(gv) * uv));
}

hipError_t launch_silu_mul(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu,
                           uint16_t* h, int64_t ldh, int m, int n, hipStream_t stream) {
  const int64_t total = (int64_t)m * n;
  silu_mul_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(g, ldg, u, ldu, h, ldh, m, n);
  return hipGetLastError();
}

// One 256-thread workgroup per row: fp32 sum of squares of the row (inputs
// clamped to the finite fp16 range, as the reference does), each thread over
// its 8-element units in ascending order, then a fixed butterfly within each
// wave and a fixed order across the four waves; r = 1 / sqrt(sum / k + eps);
// y = fp16((x * w) * r).  k % 8 == 0, rows 16-byte aligned.  The first
// kRmsRegUnits units of each thread (rows up to 8192 elements) and their
// weights are loaded once, all before the first add, and reused for the
// output; longer rows reload the rest.
constexpr int kRmsRegUnits = 4;

__device__ __forceinline__ float clamp_h(_Float16 v) {
  return fmaxf(-65504.0f, fminf((float)v, 65504.0f));
}

__global__ void __launch_bounds__(256)
rms_norm_kernel(const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
                float eps, uint16_t* __restrict__ y, int64_t ldy, int k) {
  __shared__ float wsum[4];
  const int tid = threadIdx.x;
  const h8* xr = reinterpret_cast<const h8*>(x + (size_t)blockIdx.x * ldx);
  const h8* wr = reinterpret_cast<const h8*>(w);
  h8* yr = reinterpret_cast<h8*>(y + (size_t)blockIdx.x * ldy);
  const int units = k / 8;
  h8 xv[kRmsRegUnits], wv[kRmsRegUnits];
#pragma unroll
  for (int i = 0; i < kRmsRegUnits; ++i) {
    const int u = tid + 256 * i;
    if (u < units) {
      xv[i] = xr[u];
      wv[i] = wr[u];
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kRmsRegUnits; ++i) {
    if (tid + 256 * i < units) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = clamp_h(xv[i][e]);
        sum = fmaf(f, f, sum);
      }
    }
  }
  for (int u = tid + 256 * kRmsRegUnits; u < units; u += 256) {
    const h8 v = xr[u];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = clamp_h(v[e]);
      sum = fmaf(f, f, sum);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if ((tid & 63) == 0) wsum[tid >> 6] = sum;
  __syncthreads();
  const float total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  const float r = 1.0f / sqrtf(total / (float)k + eps);
  auto out = [&](h8 v, h8 ww) {
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (_Float16)(clamp_h(v[e]) * (float)ww[e] * r);
    return o;
  };
#pragma unroll
  for (int i = 0; i < kRmsRegUnits; ++i) {
    const int u = tid + 256 * i;
    if (u < units) yr[u] = out(xv[i], wv[i]);
  }
  for (int u = tid + 256 * kRmsRegUnits; u < units; u += 256) yr[u] = out(xr[u], wr[u]);
}

hipError_t launch_rms_norm(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                           uint16_t* y, int64_t ldy, int m, int k, hipStream_t stream) {
  rms_norm_kernel<<<(unsigned)m, 256, 0, stream>>>(x, ldx, w, eps, y, ldy, k);
  return hipGetLastError();
}

}  // namespace dw4
