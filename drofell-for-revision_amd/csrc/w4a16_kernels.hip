// gfx950 kernels for the GPTQ int4-weight / fp16-activation quantized Linear:
// load-time repack, activation gathers, the register-fed prefill kernels
// (16- to 128-row tiles), the split-K plane sum, dequantisation, the
// calibration read and the elementwise decoder-stage kernels.  The decode
// kernels (M <= 64) are in w4a16_decode.hip, the LDS-streamed prefill kernel
// in w4a16_prefill.hip.
//
// Replaces, in function (not in structure), the reference's
// cuda_extends/exllama (q4_matrix.cu shuffle/make_sequential/reconstruct,
// q4_matmul.cu reconstruct + cuBLAS) and the Marlin repack/GEMM.  Layouts
// and names of the packed buffers are documented in include/drofell_w4a16.h.
//
// Arithmetic contract (reference: operators/core/linear/real_quant.py:69-102)
//   W[k,n] = fp16_rne(scale[g(k),n] * (q[k,n] - (zero[g(k),n] + 1)))
//   y[m,n] = fp16_rne(sum_k x[m,k] * W[k,n])  (fp32 accumulation)
// The prefill kernels multiply by the scale in fp16 exactly as the
// reference's dequantiser does and accumulate in fp32 on the MFMA units.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace dw4 {

// Relaxed agent-scope load (sc1, past the XCD's L2) of a partial another
// workgroup wrote through with an agent-scope store.
__device__ __forceinline__ float load_agent(float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

  const uint32_t magic = opaque(kMagic);
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
  // performs write-through (sc1), and the last arriver reads them back with
  // relaxed agent-scope loads (sc1), which read past the XCD's L2.  Every
  // wave waits for its own stores to complete (s_barrier does not wait for
  // memory), then the barrier precedes thread 0's counter increment, so
  // the increment happens after every partial store of the workgroup has
  // been performed, and the last arriver's loads are issued after it has
  // seen the count.  No release or acquire fence: on gfx950 those write
  // back or invalidate the whole L2 of the XCD, under the feet of every
  // other workgroup streaming through it.  Layout per split plane
  // (mtiles*ntiles*BM*BN floats): [tile][mt*S + si][element e of the
  // lane's float4][256 threads], so each store instruction covers 256
  // contiguous bytes per wave.
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
    const int before = __hip_atomic_fetch_add(&counters[tile_id], 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    last_arrival = before == splits - 1;
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
        float* src = part + (size_t)sp * plane + tbase + (mt * S + si) * 1024;
        t[mt][si] = sp == split ? f4{acc[mt][si][0], acc[mt][si][1], acc[mt][si][2], acc[mt][si][3]}
                                : f4{load_agent(src), load_agent(src + 256),
                                     load_agent(src + 512), load_agent(src + 768)};
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

  const uint32_t magic = opaque(kMagic);
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
    const int before = __hip_atomic_fetch_add(&counters[tile_id], 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    last_arrival = before == splits - 1;
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
    float* src = part + (size_t)sp2 * plane + tbase;
#pragma unroll
    for (int mt = 0; mt < MT3; ++mt)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        f16v t;
#pragma unroll
        for (int i = 0; i < 16; ++i) t[i] = load_agent(src + ((mt * P + p) * 16 + i) * 256);
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

hipError_t launch_gather_rows(const uint16_t* x, int64_t ldx, const int32_t* perm, uint16_t* xs,
                              int K, int M, hipStream_t stream) {
  const int64_t units = (int64_t)M * (K / 8);
  gather_rows_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream>>>(
      reinterpret_cast<const _Float16*>(x), ldx, perm, reinterpret_cast<_Float16*>(xs), K, M);
  return hipGetLastError();
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
