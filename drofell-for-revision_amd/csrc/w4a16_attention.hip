// Paged-attention decode and the KV-cache slot operations of the decoder
// stage.
//
// Cache layout (the reference's, operators/core/block/common.py:7-60 and
// cuda_extends/vllm/cache_kernels.cu:242-285, in
// /root/reference/After-Revision-DROFELL): the cache is a set of blocks of
// BS token slots; each block has a key part [kv_heads][head_size/8][BS][8]
// and a value part [kv_heads][head_size][BS] (fp16), reached through
// per-block pointer tables, with kv_head_stride elements between the heads
// of a block.  A token's slot s lives in block s / BS at offset s % BS.
//
// paged_attention_kernel: one workgroup per (sequence, kv head, context
// partition).  It serves every query head of the kv head's group
// (head h uses kv head h / (heads / kv_heads)), so each K and V byte is
// read once per group.  Per partition of up to 512 tokens:
//   logits (fp32, LDS) = scale * q . k (+ alibi slope * (t - ctx + 1));
//   p = exp(logit - max); out = sum p v / sum p.
// Waves take the partition's blocks round-robin.  For q . k a lane holds one
// token and a slice of 8 dims (one 16-byte load); lanes of one token meet
// through cross-lane adds.  For p . v a lane holds whole dims (a row of BS
// tokens).  Partitions write their max, sum and unnormalised fp32 output;
// a second kernel combines them in partition order (deterministic).  With a
// single partition the first kernel writes the output directly.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>

#include "w4a16_device.h"
#include "w4a16_attention.h"

namespace dw4 {

namespace {


__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Block-wide reduction in a fixed order (waves' results combined 0..W-1).
template <bool MAX, int W>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = MAX ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < W; ++w) r = MAX ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

// W waves per workgroup: 4 (several partitions per (sequence, kv head),
// about four workgroups per CU) or 16 (one workgroup per (sequence, kv head)
// covering the whole context, no combine launch).
template <int HS, int BS, int GMAX, int W>
__global__ void __launch_bounds__(W * 64)
paged_attention_kernel(const uint16_t* __restrict__ query, int64_t q_stride,
                       uint16_t* __restrict__ out, int64_t o_stride,
                       const int64_t* __restrict__ kptr, const int64_t* __restrict__ vptr,
                       int kv_head_stride, int num_heads, int num_kv_heads, float scale,
                       const int32_t* __restrict__ block_tables, int max_blocks,
                       const int32_t* __restrict__ context_lens,
                       const float* __restrict__ alibi, int part_tokens, int num_parts,
                       float* __restrict__ ws_ml, float* __restrict__ ws_out) {
  constexpr int SLICES = HS / 8;                 // 16-byte slices of a key row
  constexpr int TPL = 64 / BS;                   // slice groups per wave (lanes of one token)
  constexpr int SPL = (SLICES + TPL - 1) / TPL;  // slices per lane (the last may be past HS)
  constexpr int DPL = (HS + 63) / 64;            // value dims per lane (the last may be past HS)
  // head sizes that are not multiples of 64 (80, 96, 112) leave some lanes
  // without a last key slice or value dim: those hold zeros and store nothing
  constexpr bool KTAIL = SLICES % TPL != 0, VTAIL = HS % 64 != 0;
  static_assert(HS % 8 == 0 && 64 % BS == 0, "shape");
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int G = num_heads / num_kv_heads;  // query heads per kv head (<= GMAX)
  float* qs = sm;                           // [G][HS] fp32 query (scaled)
  float* logit = qs + GMAX * HS;            // [G][part_tokens]
  float* red = logit + GMAX * part_tokens;  // [waves][G][HS] partial outputs
  float* scratch = red + W * GMAX * HS;  // W floats

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int seq = blockIdx.x / num_kv_heads;
  const int kvh = blockIdx.x % num_kv_heads;
  const int part = blockIdx.y;
  const int h0 = kvh * G;
  // a context longer than the block table is cut to it (never read past a row)
  const int ctx = min(context_lens[seq], max_blocks * BS);
  const int t0 = part * part_tokens;
  const int t1 = min(ctx, t0 + part_tokens);
  const int nt = t1 - t0;
  const bool direct = num_parts == 1;
  if (nt <= 0) {  // partition past this sequence's context: an empty partial
    if (!direct && tid < G) {
      const size_t r = ((size_t)seq * num_heads + h0 + tid) * num_parts + part;
      ws_ml[2 * r] = -FLT_MAX;
      ws_ml[2 * r + 1] = 0.f;
    }
    return;
  }
  const int32_t* btab = block_tables + (size_t)seq * max_blocks + t0 / BS;
  const int nb = (nt + BS - 1) / BS;
  const int nbw = wave < nb ? (nb - wave + W - 1) / W : 0;  // this wave's blocks
  const int tt = lane % BS;   // token of this lane within a block
  const int sg = lane / BS;   // slice group
  // Each wave keeps its next NPF blocks' keys and values in flight: the
  // value loads of the first blocks are issued with the key loads, before
  // the softmax, so their latency overlaps q . k.
  // (one block for the widest variants, whose unrolled p . v would not fit)
  constexpr int NPF = DPL * (BS / 8) * GMAX <= 16 ? 2 : 1;
  h8 kreg[NPF][SPL];
  h8 vreg[NPF][DPL][BS / 8];
  auto kbase = [&](int i) {
    return reinterpret_cast<const uint16_t*>(kptr[btab[wave + W * i]]) +
           (size_t)kvh * kv_head_stride;
  };
  auto vbase = [&](int i) {
    return reinterpret_cast<const uint16_t*>(vptr[btab[wave + W * i]]) +
           (size_t)kvh * kv_head_stride;
  };
  auto load_k = [&](int slot, int i) {
    const uint16_t* kb = kbase(i);
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      if (KTAIL && sg + TPL * j >= SLICES) {
        kreg[slot][j] = h8{};
        continue;
      }
      kreg[slot][j] = *(const h8*)(kb + ((sg + TPL * j) * BS + tt) * 8);
    }
  };
  auto load_v = [&](int slot, int i) {
    const uint16_t* vb = vbase(i);
#pragma unroll
    for (int j = 0; j < DPL; ++j)
#pragma unroll
      for (int u = 0; u < BS / 8; ++u)
        vreg[slot][j][u] = VTAIL && lane + 64 * j >= HS
                               ? h8{}
                               : *(const h8*)(vb + (size_t)(lane + 64 * j) * BS + 8 * u);
  };
#pragma unroll
  for (int u = 0; u < NPF; ++u)
    if (u < nbw) {
      load_k(u, u);
      load_v(u, u);
    }
  // The query is staged after the first blocks' key and value loads went
  // out (each behind its block-table and block-pointer loads), so its own
  // load overlaps theirs; the barrier that publishes it waits only for the
  // LDS stores, and the key/value loads stay in flight across it (a
  // __syncthreads would wait for them).
  for (int i = tid; i < G * HS; i += (W * 64)) {
    const int g = i / HS, d = i % HS;
    qs[i] = scale * (float)as_h(query[(size_t)seq * q_stride + (size_t)(h0 + g) * HS + d]);
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // q . k
  auto qk = [&](int slot, int i) {
    const int b = wave + W * i;
    float dot[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      dot[g] = 0.f;
      if (g < G) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          if (KTAIL && sg + TPL * j >= SLICES) continue;
          const float* qv = qs + g * HS + (sg + TPL * j) * 8;
#pragma unroll
          for (int e = 0; e < 8; ++e) dot[g] = fmaf(qv[e], (float)kreg[slot][j][e], dot[g]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
#pragma unroll
      for (int off = BS; off < 64; off <<= 1) dot[g] += __shfl_xor(dot[g], off);
    }
    const int t = t0 + b * BS + tt;
    if (sg == 0) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G) {
          float l = dot[g];
          if (alibi != nullptr) l += alibi[h0 + g] * (float)(t - ctx + 1);
          logit[g * part_tokens + b * BS + tt] = t < t1 ? l : -FLT_MAX;
        }
      }
    }
  };
  for (int i0 = 0; i0 < nbw; i0 += NPF) {
#pragma unroll
    for (int u = 0; u < NPF; ++u) {
      const int i = i0 + u;
      if (i < nbw) {
        qk(u, i);
        if (i + NPF < nbw) load_k(u, i + NPF);
      }
    }
  }
  __syncthreads();

  // softmax numerators and their sums, per query head
  float mx[GMAX], sum[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    mx[g] = -FLT_MAX;
    sum[g] = 0.f;
    if (g < G) {
      float m = -FLT_MAX;
      for (int t = tid; t < nt; t += (W * 64)) m = fmaxf(m, logit[g * part_tokens + t]);
      mx[g] = block_reduce<true, W>(m, scratch);
      float s = 0.f;
      for (int t = tid; t < nb * BS; t += (W * 64)) {
        const float p = t < nt ? __expf(logit[g * part_tokens + t] - mx[g]) : 0.f;
        logit[g * part_tokens + t] = p;
        s += p;
      }
      sum[g] = block_reduce<false, W>(s, scratch);
    }
  }
  __syncthreads();

  // p . v: lane holds dims lane + 64 j for every query head of the group
  float acc[GMAX][DPL];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[g][j] = 0.f;
  auto pv = [&](int slot, int i) {
    const int b = wave + W * i;
    const int valid = min(BS, nt - b * BS);  // tokens of this block in the context
#pragma unroll
    for (int j = 0; j < DPL; ++j)
#pragma unroll
      for (int u = 0; u < BS / 8; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int tb = 8 * u + e;
          // slots past the context may hold anything: never multiply them
          const float vf = tb < valid ? (float)vreg[slot][j][u][e] : 0.f;
#pragma unroll
          for (int g = 0; g < GMAX; ++g)
            if (g < G) acc[g][j] = fmaf(logit[g * part_tokens + b * BS + tb], vf, acc[g][j]);
        }
  };
  for (int i0 = 0; i0 < nbw; i0 += NPF) {
#pragma unroll
    for (int u = 0; u < NPF; ++u) {
      const int i = i0 + u;
      if (i < nbw) {
        pv(u, i);
        if (i + NPF < nbw) load_v(u, i + NPF);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j)
      if (g < G && (!VTAIL || lane + 64 * j < HS)) red[(wave * GMAX + g) * HS + lane + 64 * j] = acc[g][j];
  __syncthreads();
  for (int i = tid; i < G * HS; i += (W * 64)) {
    const int g = i / HS, d = i % HS;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) o += red[(w * GMAX + g) * HS + d];
    float s = 0.f, m = 0.f;
#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg)
      if (gg == g) { s = sum[gg]; m = mx[gg]; }
    if (direct) {
      out[(size_t)seq * o_stride + (size_t)(h0 + g) * HS + d] = h_bits((_Float16)(o / s));
    } else {
      const size_t r = ((size_t)seq * num_heads + h0 + g) * num_parts + part;
      ws_out[r * HS + d] = o;
      if (d == 0) {
        ws_ml[2 * r] = m;
        ws_ml[2 * r + 1] = s;
      }
    }
  }
}

// Combine the partitions of one (sequence, head) in partition order.
template <int HS>
__global__ void __launch_bounds__(HS)
paged_attention_reduce_kernel(uint16_t* __restrict__ out, int64_t o_stride, int num_heads,
                              const int32_t* __restrict__ context_lens, int max_tokens,
                              int part_tokens,
                              int num_parts, const float* __restrict__ ws_ml,
                              const float* __restrict__ ws_out) {
  const int seq = blockIdx.x / num_heads, h = blockIdx.x % num_heads;
  const int d = threadIdx.x;
  const int ctx = min(context_lens[seq], max_tokens);
  const int parts = min(num_parts, (ctx + part_tokens - 1) / part_tokens);
  const size_t r0 = ((size_t)seq * num_heads + h) * num_parts;
  // Running max and rescaled sums over the partitions in order; the loads
  // of a batch of 8 partitions are all in flight before the first update.
  float gmax = -FLT_MAX, total = 0.f, o = 0.f;
  for (int p0 = 0; p0 < parts; p0 += 8) {
    float m[8], l[8], v[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool in = p0 + b < parts;
      m[b] = in ? ws_ml[2 * (r0 + p0 + b)] : -FLT_MAX;
      l[b] = in ? ws_ml[2 * (r0 + p0 + b) + 1] : 0.f;
      v[b] = in ? ws_out[(r0 + p0 + b) * HS + d] : 0.f;
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if (p0 + b < parts) {
        const float nm = fmaxf(gmax, m[b]);
        const float a = __expf(gmax - nm), w = __expf(m[b] - nm);
        total = total * a + l[b] * w;
        o = o * a + v[b] * w;
        gmax = nm;
      }
    }
  }
  out[(size_t)seq * o_stride + (size_t)h * HS + d] = h_bits((_Float16)(o / total));
}

// One workgroup per token: its key and value rows go to their slot.
// restore: the reverse copy (slots to the token-major tensors).
__global__ void reshape_and_cache_kernel(uint16_t* __restrict__ key, int64_t key_stride,
                                         uint16_t* __restrict__ value, int64_t value_stride,
                                         const int64_t* __restrict__ kptr,
                                         const int64_t* __restrict__ vptr,
                                         const int64_t* __restrict__ slots, int num_kv_heads,
                                         int head_size, int block_size, int kv_head_stride,
                                         bool restore) {
  const int64_t tok = blockIdx.x;
  const int64_t slot = slots[tok];
  if (slot < 0) return;  // padding token
  const int64_t blk = slot / block_size;
  const int off = (int)(slot % block_size);
  uint16_t* kc = reinterpret_cast<uint16_t*>(kptr[blk]);
  uint16_t* vc = reinterpret_cast<uint16_t*>(vptr[blk]);
  const int n = num_kv_heads * head_size;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int h = i / head_size, d = i % head_size;
    const size_t kt = (size_t)h * kv_head_stride + ((size_t)(d / 8) * block_size + off) * 8 + d % 8;
    const size_t vt = (size_t)h * kv_head_stride + (size_t)d * block_size + off;
    if (restore) {
      key[tok * key_stride + i] = kc[kt];
      value[tok * value_stride + i] = vc[vt];
    } else {
      kc[kt] = key[tok * key_stride + i];
      vc[vt] = value[tok * value_stride + i];
    }
  }
}

template <int HS, int BS, int GMAX, int W>
hipError_t launch_pa_w(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                       hipStream_t stream) {
  const size_t smem = attn_smem_bytes(HS, GMAX, p.part_tokens, W);
  const dim3 grid((unsigned)(a.num_seqs * a.num_kv_heads), (unsigned)p.num_parts);
  float* ws_ml = p.num_parts > 1 ? ws : nullptr;
  float* ws_out = p.num_parts > 1 ? ws + 2 * (size_t)a.num_seqs * a.num_heads * p.num_parts : nullptr;
  paged_attention_kernel<HS, BS, GMAX, W><<<grid, W * 64, smem, stream>>>(
      a.query, a.q_stride, a.out, a.o_stride, a.kptr, a.vptr, a.kv_head_stride, a.num_heads,
      a.num_kv_heads, a.scale, a.block_tables, a.max_blocks, a.context_lens, a.alibi,
      p.part_tokens, p.num_parts, ws_ml, ws_out);
  return hipGetLastError();
}

template <int HS, int BS, int GMAX>
hipError_t launch_pa(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                     hipStream_t stream) {
  hipError_t e;
  if constexpr (attn_wide_ok(HS, BS, GMAX)) {
    e = p.waves == 16 ? launch_pa_w<HS, BS, GMAX, 16>(a, p, ws, stream)
                      : launch_pa_w<HS, BS, GMAX, 4>(a, p, ws, stream);
  } else {
    if (p.waves != 4) return hipErrorInvalidValue;
    e = launch_pa_w<HS, BS, GMAX, 4>(a, p, ws, stream);
  }
  if (e != hipSuccess || p.num_parts == 1) return e;
  float* ws_ml = ws;
  float* ws_out = ws + 2 * (size_t)a.num_seqs * a.num_heads * p.num_parts;
  paged_attention_reduce_kernel<HS><<<(unsigned)(a.num_seqs * a.num_heads), HS, 0, stream>>>(
      a.out, a.o_stride, a.num_heads, a.context_lens, a.max_blocks * BS, p.part_tokens,
      p.num_parts, ws_ml, ws_out);
  return hipGetLastError();
}

template <int HS, int BS>
hipError_t launch_pa_g(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                       hipStream_t stream) {
  const int g = a.num_heads / a.num_kv_heads;
  if (g == 1) return launch_pa<HS, BS, 1>(a, p, ws, stream);
  if (g <= 4) return launch_pa<HS, BS, 4>(a, p, ws, stream);
  return launch_pa<HS, BS, 8>(a, p, ws, stream);
}

template <int HS>
hipError_t launch_pa_bs(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                        hipStream_t stream) {
  if (a.block_size == 16) return launch_pa_g<HS, 16>(a, p, ws, stream);
  return launch_pa_g<HS, 32>(a, p, ws, stream);
}

// Rotary embedding, rotate-half form, in place on fp16 rows [batch][rows][hd]
// (row = token * heads + head): position p = past + row / heads, pair
// (l, r) = (x[c], x[c + hd/2]):
//   l' = fma(l, cos[p][c], fp16(r * -sin[p][c]))
//   r' = fma(r, cos[p][c + hd/2], fp16(l * sin[p][c + hd/2]))
// each product and each fma rounded once in fp16, as the reference's
// half-precision kernel (cuda_extends/exllama/fuse_v2/rope.cu:24-91) does.
__global__ void rope_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ sinp,
                            const uint16_t* __restrict__ cosp, int rows, int hd, int heads,
                            int max_pos, int past_len, const int32_t* __restrict__ past_lens) {
  const int half = hd / 2;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int c = (int)(i % half);
  const int64_t row = i / half;  // within this batch entry
  if (row >= rows) return;
  const int b = blockIdx.y;
  const int pos = (past_len >= 0 ? past_len : past_lens[b]) + (int)(row / heads);
  if (pos < 0 || pos >= max_pos) return;  // outside the table: row left as it is
  uint16_t* xr = x + ((int64_t)b * rows + row) * hd;
  const _Float16 l = as_h(xr[c]), r = as_h(xr[c + half]);
  const _Float16 cl = as_h(cosp[(int64_t)pos * hd + c]), cr = as_h(cosp[(int64_t)pos * hd + c + half]);
  const _Float16 sl = as_h(sinp[(int64_t)pos * hd + c]), sr = as_h(sinp[(int64_t)pos * hd + c + half]);
  const _Float16 ls = r * (_Float16)(-sl);
  const _Float16 rs = l * sr;
  xr[c] = h_bits(__builtin_fmaf16(l, cl, ls));
  xr[c + half] = h_bits(__builtin_fmaf16(r, cr, rs));
}

// One decode token per sequence: its q and k rows rotated in place (the
// arithmetic of rope_kernel, position p = positions[t]), the rotated k row
// and the v row written to slot block_tables[t][p / bs] * bs + p % bs, and
// p + 1 stored to lens_out[t] (if given) -- rope on q and k, then
// reshape_and_cache, in one launch.  A position outside the block table
// writes no slot; one outside the sin/cos tables leaves q and k unrotated.
// Grid: (sequence, head slot) with head slots [0, heads) the q heads, then
// the kv heads (rotate k, write k and v to the slot); 64 threads, one
// (l, r) pair (or two v elements) each, so no thread loops.
__global__ void __launch_bounds__(64)
rope_cache_kernel(uint16_t* __restrict__ q, int64_t q_stride, uint16_t* __restrict__ k,
                  int64_t k_stride, const uint16_t* __restrict__ v, int64_t v_stride,
                  const uint16_t* __restrict__ sinp, const uint16_t* __restrict__ cosp,
                  int max_pos, const int32_t* __restrict__ positions,
                  const int32_t* __restrict__ block_tables, int max_blocks,
                  const int64_t* __restrict__ kptr, const int64_t* __restrict__ vptr,
                  int kv_head_stride, int32_t* __restrict__ lens_out, int heads, int kv_heads,
                  int hd, int bs) {
  const int t = blockIdx.x, slot = blockIdx.y, tid = threadIdx.x;
  const int p = positions[t];
  if (lens_out != nullptr && slot == 0 && tid == 0) lens_out[t] = p + 1;
  const int half = hd / 2;
  const bool rot = p >= 0 && p < max_pos;
  const bool store = p >= 0 && p / bs < max_blocks;
  const bool is_q = slot < heads;
  const int h = is_q ? slot : slot - heads;
  uint16_t* row = is_q ? q + t * q_stride + h * hd : k + t * k_stride + h * hd;
  const uint16_t* sr = sinp + (int64_t)(rot ? p : 0) * hd;
  const uint16_t* cr = cosp + (int64_t)(rot ? p : 0) * hd;
  uint16_t* kh = nullptr;
  uint16_t* vh = nullptr;
  int off = 0;
  if (!is_q && store) {
    const int blk = block_tables[(int64_t)t * max_blocks + p / bs];
    kh = reinterpret_cast<uint16_t*>(kptr[blk]) + (size_t)h * kv_head_stride;
    vh = reinterpret_cast<uint16_t*>(vptr[blk]) + (size_t)h * kv_head_stride;
    off = p % bs;
  }
  for (int c = tid; c < half; c += 64) {
    _Float16 l = as_h(row[c]), r = as_h(row[c + half]);
    if (rot) {
      const _Float16 ls = r * (_Float16)(-as_h(sr[c]));
      const _Float16 rs = l * as_h(sr[c + half]);
      l = __builtin_fmaf16(l, as_h(cr[c]), ls);
      r = __builtin_fmaf16(r, as_h(cr[c + half]), rs);
      row[c] = h_bits(l);
      row[c + half] = h_bits(r);
    }
    if (kh != nullptr) {
      kh[((c / 8) * bs + off) * 8 + c % 8] = h_bits(l);
      kh[(((c + half) / 8) * bs + off) * 8 + (c + half) % 8] = h_bits(r);
    }
  }
  if (vh != nullptr) {
    const uint16_t* vr = v + t * v_stride + h * hd;
    for (int d = tid; d < hd; d += 64) vh[(size_t)d * bs + off] = vr[d];
  }
}

}  // namespace

hipError_t launch_rope_cache(const RopeCacheArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.num_seqs, (unsigned)(a.heads + a.kv_heads));
  rope_cache_kernel<<<grid, 64, 0, stream>>>(
      a.q, a.q_stride, a.k, a.k_stride, a.v, a.v_stride, a.sinp, a.cosp, a.max_pos, a.positions,
      a.block_tables, a.max_blocks, a.kptr, a.vptr, a.kv_head_stride, a.lens_out, a.heads,
      a.kv_heads, a.hd, a.bs);
  return hipGetLastError();
}

hipError_t launch_rope(uint16_t* x, const uint16_t* sinp, const uint16_t* cosp, int batch,
                       int rows, int hd, int heads, int max_pos, int past_len,
                       const int32_t* past_lens, hipStream_t stream) {
  const int64_t n = (int64_t)rows * (hd / 2);
  const dim3 grid((unsigned)((n + 255) / 256), (unsigned)batch);
  rope_kernel<<<grid, 256, 0, stream>>>(x, sinp, cosp, rows, hd, heads, max_pos, past_len,
                                        past_lens);
  return hipGetLastError();
}

PagedAttnPlan plan_paged_attention(int num_seqs, int num_heads, int num_kv_heads, int head_size,
                                   int block_size, int max_context_len, int cus) {
  PagedAttnPlan p;
  const int blocks = std::max(1, (max_context_len + block_size - 1) / block_size);
  const int pairs = std::max(1, num_seqs * num_kv_heads);
  // one 16-wave workgroup per (sequence, kv head) over the whole context
  // where that gives every CU about one workgroup and the context fits one
  // partition: no combine launch
  const int g = num_kv_heads > 0 ? num_heads / num_kv_heads : 1;
  const int gmax = g == 1 ? 1 : g <= 4 ? 4 : 8;
  if (attn_wide_ok(head_size, block_size, gmax) && 2 * pairs > cus && pairs <= cus &&
      blocks * block_size <= kAttnWideMaxTokens &&
      attn_smem_bytes(head_size, gmax, blocks * block_size, 16) <= 64 * 1024) {
    p.waves = 16;
    p.part_tokens = blocks * block_size;
    p.num_parts = 1;
    return p;
  }
  // about four workgroups per CU (eight measured no faster); partitions of
  // whole blocks, at most 512 tokens
  int parts = std::max(1, (4 * cus + pairs - 1) / pairs);
  parts = std::min(parts, blocks);
  int bpp = (blocks + parts - 1) / parts;
  bpp = std::min(bpp, kAttnMaxPartTokens / block_size);
  p.part_tokens = bpp * block_size;
  p.num_parts = (blocks + bpp - 1) / bpp;
  return p;
}

size_t paged_attention_ws_bytes(const PagedAttnPlan& p, int num_seqs, int num_heads,
                                int head_size) {
  if (p.num_parts <= 1) return 0;
  return sizeof(float) * (size_t)num_seqs * num_heads * p.num_parts * (2 + (size_t)head_size);
}

hipError_t launch_paged_attention(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                                  hipStream_t stream) {
  switch (a.head_size) {
    case 64: return launch_pa_bs<64>(a, p, ws, stream);
    case 80: return launch_pa_bs<80>(a, p, ws, stream);
    case 96: return launch_pa_bs<96>(a, p, ws, stream);
    case 112: return launch_pa_bs<112>(a, p, ws, stream);
    case 128: return launch_pa_bs<128>(a, p, ws, stream);
    case 256: return launch_pa_bs<256>(a, p, ws, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_reshape_and_cache(uint16_t* key, int64_t key_stride, uint16_t* value,
                                    int64_t value_stride, const int64_t* kptr, const int64_t* vptr,
                                    const int64_t* slots, int num_tokens, int num_kv_heads,
                                    int head_size, int block_size, int kv_head_stride,
                                    bool restore, hipStream_t stream) {
  const int n = num_kv_heads * head_size;
  reshape_and_cache_kernel<<<(unsigned)num_tokens, std::min(1024, n), 0, stream>>>(
      key, key_stride, value, value_stride, kptr, vptr, slots, num_kv_heads, head_size,
      block_size, kv_head_stride, restore);
  return hipGetLastError();
}

}  // namespace dw4
