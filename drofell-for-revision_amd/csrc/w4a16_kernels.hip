// gfx950 kernels for the GPTQ int4-weight / fp16-activation quantized Linear.
//
// Replaces, in function (not in structure), the reference's
// cuda_extends/exllama (q4_matrix.cu shuffle/make_sequential/reconstruct,
// q_gemm_kernel_gptq.cuh gemm_half_q_half_gptq_kernel, q4_matmul.cu
// reconstruct + cuBLAS) and the Marlin repack/GEMM.  Layouts and names of
// the packed buffers are documented in include/drofell_w4a16.h.
//
// Arithmetic contract (reference: operators/core/linear/real_quant.py:97-118)
//   W[k,n] = fp16_rne(scale[g(k),n] * (q[k,n] - (zero[g(k),n] + 1)))
//   y[m,n] = fp16_rne(sum_k x[m,k] * W[k,n])  (fp32 accumulation)
// The decode kernel factors the scale out of each group (fp32 products of
// exact small integers and fp16 activations, scaled in fp32), the prefill
// kernel multiplies by the scale in fp16 exactly as the reference's
// dequantiser does; both accumulate in fp32 on the MFMA units.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_internal.h"

namespace dw4 {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef int32_t i4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ _Float16 as_h(uint16_t u) { return __builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ h2 splat2(_Float16 v) { return h2{v, v}; }

// The 8 rows of one packed word, minus the effective zero, as exact fp16
// integers in row order.  Even rows sit in the low half-word, odd rows in
// the high half-word, so OR-ing a nibble pair into the fp16 pattern of
// 1024.0 yields (1024 + q) or (1024 + 16 q) in each half without a shift.
__device__ __forceinline__ h8 centered8(uint32_t w, h2 nz1024, h2 nz64) {
  const h2 sixteenth = splat2((_Float16)0.0625f);
  const uint32_t w8 = w >> 8;
  const h2 p0 = as_h2((w & 0x000F000Fu) | kMagic) + nz1024;               // rows 0,1
  const h2 p1 = as_h2((w & 0x00F000F0u) | kMagic) * sixteenth + nz64;     // rows 2,3
  const h2 p2 = as_h2((w8 & 0x000F000Fu) | kMagic) + nz1024;              // rows 4,5
  const h2 p3 = as_h2((w8 & 0x00F000F0u) | kMagic) * sixteenth + nz64;    // rows 6,7
  const h4 a = __builtin_shufflevector(p0, p1, 0, 1, 2, 3);
  const h4 b = __builtin_shufflevector(p2, p3, 0, 1, 2, 3);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Zero-point constants -(1024 + z_eff) and -(64 + z_eff) from a stored nibble.
__device__ __forceinline__ void zero_consts(uint32_t zword, int zshift, h2& nz1024, h2& nz64) {
  const int ze = (int)((zword >> zshift) & 15u) + 1;
  nz1024 = splat2((_Float16)(float)(-(1024 + ze)));
  nz64 = splat2((_Float16)(float)(-(64 + ze)));
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
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

// ---------------------------------------------------------------------------
// Act-order activation gather for the decode path: xg[m][k'] = x[m][perm[k']]
// ---------------------------------------------------------------------------
__global__ void gather_x_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                const int32_t* __restrict__ perm,
                                uint16_t* __restrict__ xg, int M, int K) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= (size_t)M * K) return;
  const int m = (int)(o / K);
  const int k = (int)(o % K);
  xg[o] = x[(size_t)m * ldx + perm[k]];
}

// ---------------------------------------------------------------------------
// Decode kernel (M <= 64): one workgroup per 16-column strip, its waves
// split K; packed int4 words are dequantised in registers straight into the
// B operand of v_mfma_f32_16x16x32_f16 (no LDS for weights); the scale is
// applied per group in fp32; the waves' partial sums meet in LDS in a fixed
// order (deterministic).
// ---------------------------------------------------------------------------
template <int MT, int WAVES, int U, bool G128>
__global__ void __launch_bounds__(WAVES * 64)
decode_kernel(const _Float16* __restrict__ x, int64_t ldx, int M,
              const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
              const uint16_t* __restrict__ ps, const uint16_t* __restrict__ bias,
              uint16_t* __restrict__ y, int64_t ldy, int K, int gs, int G) {
  __shared__ __attribute__((aligned(16))) f4 red[WAVES * MT * 64];
  const int s = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int KC = K / kChunkK;

  const u4* qp = pq + (size_t)s * KC * 64 + lane;
  const uint16_t* sp = ps + (size_t)s * G * 16 + j;
  const uint32_t* zp = pz + (size_t)s * G * 2 + (j >> 3);
  const int zsh = (j & 7) * 4;

  const _Float16* xr[MT];
  bool xv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + j;
    xv[mt] = m < M;
    xr[mt] = x + (size_t)(xv[mt] ? m : 0) * ldx + kq * 8;
  }

  f4 tot[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) tot[mt] = f4{0.f, 0.f, 0.f, 0.f};

  const int nch = wave < KC ? (KC - wave + WAVES - 1) / WAVES : 0;

  u4 qb[U];
  uint32_t zb[U];
  uint16_t sb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u < nch) {
      const int c = wave + u * WAVES;
      qb[u] = __builtin_nontemporal_load(qp + (size_t)c * 64);
      if (G128) {
        const int g = (c * kChunkK) / gs;
        sb[u] = sp[(size_t)g * 16];
        zb[u] = zp[(size_t)g * 2];
      }
    }
  }

  for (int i0 = 0; i0 < nch; i0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u;
      if (i < nch) {
        const int c = wave + i * WAVES;
        const u4 w = qb[u];
        uint32_t zw = 0;
        uint16_t sbits = 0;
        if (G128) {
          zw = zb[u];
          sbits = sb[u];
        }
        const int in = i + U;
        if (in < nch) {
          const int cn = wave + in * WAVES;
          qb[u] = __builtin_nontemporal_load(qp + (size_t)cn * 64);
          if (G128) {
            const int g = (cn * kChunkK) / gs;
            sb[u] = sp[(size_t)g * 16];
            zb[u] = zp[(size_t)g * 2];
          }
        }
        const size_t xoff = (size_t)c * kChunkK;
        if (G128) {
          h2 nz1024, nz64;
          zero_consts(zw, zsh, nz1024, nz64);
          f4 acc[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const h8 b = centered8(w[t], nz1024, nz64);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              h8 a = h8{};
              if (xv[mt]) a = *(const h8*)(xr[mt] + xoff + 32 * t);
              acc[mt] = mfma16(a, b, acc[mt]);
            }
          }
          const float sc = (float)as_h(sbits);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) tot[mt] += sc * acc[mt];
        } else {
          // Group size a multiple of 32 that does not cover a whole chunk or
          // is not a multiple of 128: groups change at k-step granularity.
          f4 acc[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
          const int spg = gs >> 5;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int ks = c * 4 + t;
            const int g = ks / spg;
            h2 nz1024, nz64;
            zero_consts(zp[(size_t)g * 2], zsh, nz1024, nz64);
            const h8 b = centered8(w[t], nz1024, nz64);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              h8 a = h8{};
              if (xv[mt]) a = *(const h8*)(xr[mt] + xoff + 32 * t);
              acc[mt] = mfma16(a, b, acc[mt]);
            }
            const bool last = (t == 3) || ((ks + 1) / spg != g);
            if (last) {
              const float sc = (float)as_h(sp[(size_t)g * 16]);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
                tot[mt] += sc * acc[mt];
                acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
              }
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[(wave * MT + mt) * 64 + lane] = tot[mt];
  __syncthreads();

  const float* redf = reinterpret_cast<const float*>(red);
  for (int idx = threadIdx.x; idx < MT * 256; idx += WAVES * 64) {
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
    _Float16 out = (_Float16)sum;
    if (bias != nullptr) out = (_Float16)((float)out + (float)as_h(bias[n]));
    y[(size_t)m * ldy + n] = h_bits(out);
  }
}

// ---------------------------------------------------------------------------
// Prefill kernel (any M): 4 waves; the workgroup tile is (16*MT2) rows x
// (64*S) columns.  Activations are staged through LDS (double buffered,
// gathered through perm for act-order); each wave owns S strips and
// dequantises its packed words in registers to the exact fp16 weight,
// which feeds v_mfma_f32_16x16x32_f16 directly.  Split-K partials (fp32)
// go to the workspace and are summed in a fixed order by reduce_kernel.
// ---------------------------------------------------------------------------
constexpr int kLdaPad = 8;
constexpr int kLda = kChunkK + kLdaPad;  // halfs per LDS row (272 bytes)

template <int MT2, int S, bool ACT, bool G128>
__global__ void __launch_bounds__(256)
prefill_kernel(const _Float16* __restrict__ x, int64_t ldx, int M,
               const int32_t* __restrict__ perm,
               const u4* __restrict__ pq, const uint32_t* __restrict__ pz,
               const uint16_t* __restrict__ ps, const uint16_t* __restrict__ bias,
               uint16_t* __restrict__ y, int64_t ldy, float* __restrict__ part,
               int K, int N, int gs, int G, int chunks_per_split, int mtiles, int ntiles) {
  constexpr int BM = 16 * MT2;
  constexpr int UNITS = BM * 16 / 256;  // 16-byte A units per thread per chunk
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
  const int wave = tid >> 6;
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int KC = K / kChunkK;
  const int split = blockIdx.y;
  const int c_begin = split * chunks_per_split;
  const int c_end = min(KC, c_begin + chunks_per_split);
  const int m0 = mtile * BM;

  // Activation staging: unit u -> (row, 16-byte column)
  int arow[UNITS], acol[UNITS];
  bool aval[UNITS];
#pragma unroll
  for (int i = 0; i < UNITS; ++i) {
    const int u = tid + 256 * i;
    arow[i] = u >> 4;
    acol[i] = u & 15;
    aval[i] = (m0 + arow[i]) < M;
  }
  auto load_a = [&](int c, h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i) {
      h8 v = h8{};
      if (aval[i]) {
        const _Float16* xrow = x + (size_t)(m0 + arow[i]) * ldx;
        const int k = c * kChunkK + acol[i] * 8;
        if (ACT) {
          const i4 p0 = *(const i4*)(perm + k);
          const i4 p1 = *(const i4*)(perm + k + 4);
          v = h8{xrow[p0[0]], xrow[p0[1]], xrow[p0[2]], xrow[p0[3]],
                 xrow[p1[0]], xrow[p1[1]], xrow[p1[2]], xrow[p1[3]]};
        } else {
          v = *(const h8*)(xrow + k);
        }
      }
      regs[i] = v;
    }
  };
  auto store_a = [&](int buf, const h8 (&regs)[UNITS]) {
#pragma unroll
    for (int i = 0; i < UNITS; ++i)
      *(h8*)(&As[buf][arow[i] * kLda + acol[i] * 8]) = regs[i];
  };

  // Weight strips owned by this wave (the last N-tile may be partial).
  const int NS = N / kStripN;
  const int strip0 = ntile * 4 * S + wave * S;
  const u4* qp[S];
  const uint16_t* sp[S];
  const uint32_t* zp[S];
  bool sval[S];
#pragma unroll
  for (int si = 0; si < S; ++si) {
    const int st = strip0 + si;
    sval[si] = st < NS;
    const int sc = sval[si] ? st : 0;
    qp[si] = pq + (size_t)sc * KC * 64 + lane;
    sp[si] = ps + (size_t)sc * G * 16 + j;
    zp[si] = pz + (size_t)sc * G * 2 + (j >> 3);
  }
  const int zsh = (j & 7) * 4;

  f4 acc[MT2][S];
#pragma unroll
  for (int mt = 0; mt < MT2; ++mt)
#pragma unroll
    for (int si = 0; si < S; ++si) acc[mt][si] = f4{0.f, 0.f, 0.f, 0.f};

  h8 areg[UNITS];
  u4 qcur[S], qnext[S];
  uint32_t zcur[S], znext[S];
  uint16_t scur[S], snext[S];

  auto load_b = [&](int c, u4 (&q)[S], uint32_t (&z)[S], uint16_t (&sc)[S]) {
#pragma unroll
    for (int si = 0; si < S; ++si) {
      q[si] = sval[si] ? __builtin_nontemporal_load(qp[si] + (size_t)c * 64) : u4{0u, 0u, 0u, 0u};
      if (G128) {
        const int g = (c * kChunkK) / gs;
        sc[si] = sp[si][(size_t)g * 16];
        z[si] = zp[si][(size_t)g * 2];
      }
    }
  };

  if (c_begin < c_end) {
    load_a(c_begin, areg);
    load_b(c_begin, qcur, zcur, scur);
    store_a(0, areg);
  }
  __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int buf = (c - c_begin) & 1;
    const bool has_next = (c + 1) < c_end;
    if (has_next) {
      load_a(c + 1, areg);
      load_b(c + 1, qnext, znext, snext);
    }
    const _Float16* Ab = &As[buf][0];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      h8 bop[S];
#pragma unroll
      for (int si = 0; si < S; ++si) {
        h2 nz1024, nz64;
        _Float16 sc;
        if (G128) {
          zero_consts(zcur[si], zsh, nz1024, nz64);
          sc = as_h(scur[si]);
        } else {
          const int g = (c * kChunkK + 32 * t) / gs;
          zero_consts(zp[si][(size_t)g * 2], zsh, nz1024, nz64);
          sc = as_h(sp[si][(size_t)g * 16]);
        }
        const h8 d = centered8(qcur[si][t], nz1024, nz64);
        const h8 s8 = h8{sc, sc, sc, sc, sc, sc, sc, sc};
        bop[si] = d * s8;  // fp16 product, round to nearest even
      }
#pragma unroll
      for (int mt = 0; mt < MT2; ++mt) {
        const h8 a = *(const h8*)(Ab + (mt * 16 + j) * kLda + 32 * t + 8 * kq);
#pragma unroll
        for (int si = 0; si < S; ++si) acc[mt][si] = mfma16(a, bop[si], acc[mt][si]);
      }
    }
    if (has_next) {
      store_a(buf ^ 1, areg);
#pragma unroll
      for (int si = 0; si < S; ++si) {
        qcur[si] = qnext[si];
        zcur[si] = znext[si];
        scur[si] = snext[si];
      }
    }
    __syncthreads();
  }

  const bool direct = gridDim.y == 1;
#pragma unroll
  for (int mt = 0; mt < MT2; ++mt) {
#pragma unroll
    for (int si = 0; si < S; ++si) {
      const int n = (strip0 + si) * kStripN + j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + mt * 16 + kq * 4 + r;
        if (m < M && sval[si]) {
          const float v = acc[mt][si][r];
          if (direct) {
            _Float16 out = (_Float16)v;
            if (bias != nullptr) out = (_Float16)((float)out + (float)as_h(bias[n]));
            y[(size_t)m * ldy + n] = h_bits(out);
          } else {
            part[((size_t)split * M + m) * N + n] = v;
          }
        }
      }
    }
  }
}

__global__ void reduce_kernel(const float* __restrict__ part, int splits, int M, int N,
                              const uint16_t* __restrict__ bias,
                              uint16_t* __restrict__ y, int64_t ldy) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)M * N;
  if (o >= total) return;
  float sum = 0.f;
  for (int sidx = 0; sidx < splits; ++sidx) sum += part[(size_t)sidx * total + o];
  const int m = (int)(o / N);
  const int n = (int)(o % N);
  _Float16 out = (_Float16)sum;
  if (bias != nullptr) out = (_Float16)((float)out + (float)as_h(bias[n]));
  y[(size_t)m * ldy + n] = h_bits(out);
}

// ---------------------------------------------------------------------------
// Bit-exact dequantisation to the original row order (one thread per 16-byte
// lane unit = 32 weights).
// ---------------------------------------------------------------------------
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
    const float sc = (float)as_h(ps[((size_t)s * G + g) * 16 + j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int slot = (e & 1) ? 4 + (e >> 1) : (e >> 1);
      const int qv = (int)((q[t] >> (4 * slot)) & 15u);
      // exact product of an fp16 and an integer |d| <= 16, rounded once
      const _Float16 v = (_Float16)(sc * (float)(qv - ze));
      const int k = k0 + e;
      const int row = perm ? perm[k] : k;
      w[(size_t)row * ldw + n] = h_bits(v);
    }
  }
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

hipError_t launch_gather_x(const uint16_t* x, int64_t ldx, const int32_t* perm, uint16_t* xg,
                           int M, int K, hipStream_t stream) {
  const size_t total = (size_t)M * K;
  gather_x_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(x, ldx, perm, xg, M, K);
  return hipGetLastError();
}

template <int MT>
static hipError_t launch_decode_mt(const GemmArgs& a, hipStream_t stream) {
  const dim3 grid(a.N / kStripN);
  const dim3 block(kDecodeWaves * 64);
  const bool g128 = (a.gs % kChunkK) == 0;
  if (g128)
    decode_kernel<MT, kDecodeWaves, kDecodePrefetch, true><<<grid, block, 0, stream>>>(
        (const _Float16*)a.x, a.ldx, a.M, (const u4*)a.pq, (const uint32_t*)a.pz, a.ps, a.bias,
        a.y, a.ldy, a.K, a.gs, a.G);
  else
    decode_kernel<MT, kDecodeWaves, kDecodePrefetch, false><<<grid, block, 0, stream>>>(
        (const _Float16*)a.x, a.ldx, a.M, (const u4*)a.pq, (const uint32_t*)a.pz, a.ps, a.bias,
        a.y, a.ldy, a.K, a.gs, a.G);
  return hipGetLastError();
}

hipError_t launch_decode(const GemmArgs& a, hipStream_t stream) {
  const int mt = (a.M + 15) / 16;
  switch (mt) {
    case 1: return launch_decode_mt<1>(a, stream);
    case 2: return launch_decode_mt<2>(a, stream);
    case 3: return launch_decode_mt<3>(a, stream);
    case 4: return launch_decode_mt<4>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int MT2, int S, bool ACT, bool G128>
static hipError_t launch_prefill_cfg(const GemmArgs& a, int splits, float* part, hipStream_t stream) {
  constexpr int BM = 16 * MT2;
  constexpr int BN = 64 * S;
  const int mtiles = (a.M + BM - 1) / BM;
  const int ntiles = (a.N + BN - 1) / BN;
  const int KC = a.K / kChunkK;
  const int cps = (KC + splits - 1) / splits;
  const int real_splits = (KC + cps - 1) / cps;
  const dim3 grid((unsigned)(((ntiles + 7) / 8) * 8 * mtiles), (unsigned)real_splits);
  prefill_kernel<MT2, S, ACT, G128><<<grid, 256, 0, stream>>>(
      (const _Float16*)a.x, a.ldx, a.M, a.perm, (const u4*)a.pq, (const uint32_t*)a.pz, a.ps,
      a.bias, a.y, a.ldy, part, a.K, a.N, a.gs, a.G, cps, mtiles, ntiles);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || real_splits == 1) return err;
  const size_t total = (size_t)a.M * a.N;
  reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(part, real_splits, a.M, a.N,
                                                                     a.bias, a.y, a.ldy);
  return hipGetLastError();
}

template <int MT2, int S>
static hipError_t launch_prefill_tile(const GemmArgs& a, int splits, float* part, hipStream_t stream) {
  const bool act = a.perm != nullptr;
  const bool g128 = (a.gs % kChunkK) == 0;
  if (act) {
    return g128 ? launch_prefill_cfg<MT2, S, true, true>(a, splits, part, stream)
                : launch_prefill_cfg<MT2, S, true, false>(a, splits, part, stream);
  }
  return g128 ? launch_prefill_cfg<MT2, S, false, true>(a, splits, part, stream)
              : launch_prefill_cfg<MT2, S, false, false>(a, splits, part, stream);
}

hipError_t launch_prefill(const GemmArgs& a, const PrefillPlan& plan, float* part, hipStream_t stream) {
  if (plan.bm == 64 && plan.bn == 128) return launch_prefill_tile<4, 2>(a, plan.splits, part, stream);
  if (plan.bm == 128 && plan.bn == 128) return launch_prefill_tile<8, 2>(a, plan.splits, part, stream);
  if (plan.bm == 64 && plan.bn == 64) return launch_prefill_tile<4, 1>(a, plan.splits, part, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_dequant(const uint32_t* pq, const uint32_t* pz, const uint16_t* ps,
                          const int32_t* perm, uint16_t* w, int64_t ldw, int K, int N, int gs, int G,
                          hipStream_t stream) {
  const size_t total = (size_t)K * N / 32;
  dequant_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
      (const u4*)pq, pz, ps, perm, w, ldw, K, N, gs, G);
  return hipGetLastError();
}

}  // namespace dw4
