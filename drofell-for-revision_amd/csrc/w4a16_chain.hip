// gfx950 decode chain: one persistent launch over a list of W4A16
// projections ("links") at M <= 4, such as the q/k/v, o, gate/up and down
// projections of several decoder layers.  No single reference call matches
// it: it runs the per-projection q4_matmul_cuda_v2 calls of a decode step
// (cuda_extends/exllama/entry.cpp:221-251, called once per projection by the
// layer loop of operators/assemble/decoders/real_decoders_group.py:106-159;
// paths relative to /root/reference/After-Revision-DROFELL) as one kernel.
//
// Why: a decode projection streams a few MB of packed weights, and as its own
// launch it pays the launch gap, the first-touch latency of its weights and
// the drain of its last wave before the next projection's weights are even
// requested.  Here every workgroup streams the weight chunks of its share of
// all links back to back, so the HBM stream runs across the dependency
// points; only the activations wait.
//
// Workgroup (one per CU, (SW + 1) waves):
//   * waves 1..SW stream: each owns a ring of R LDS slots and keeps R units
//     (one 16-column x 128-row chunk: 1 KiB of packed words plus its 40-byte
//     scale/zero record) in flight with global_load_lds, across link
//     boundaries.  A unit is consumed from LDS exactly as the decode kernel
//     consumes it (exact q - z in fp16 from the 0x6400 identity, one
//     v_mfma_f32_16x16x32_f16 per 32-row k-step, the fp32 group scale applied
//     per chunk) and its slot is refilled with the wave's next unit at once,
//     so exactly R units per wave are always outstanding and one fixed
//     vmcnt wait serves every unit;
//   * wave 0 controls: before a link it waits until every workgroup has
//     completed the links the link depends on (their progress words), then
//     copies the link's activations into LDS; after a link it sums the
//     streaming waves' partial sums in a fixed order and stores the fp16
//     outputs (+ bias, + residual).  It issues no weight copies, so its own
//     loads and stores never wait behind the ring (vmcnt completes in order).
//
// Cross-workgroup visibility: outputs and progress words are written with
// agent-scope (sc1, write-through) stores and the progress word only after
// the outputs' stores have completed (vmcnt 0); progress words, activations
// and residuals are read with agent-scope (sc1) loads.  Every wait is bounded
// (about 0.2 s of the realtime counter): past that the header's timed_out
// word is set and the wait ends, so the launch always drains.  Progress
// words carry the launch number, so no reset pass is needed between launches;
// the last workgroup to finish advances the launch number in the header.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w4a16_device.h"
#include "w4a16_internal.h"

namespace dw4 {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// global -> LDS copies (each active lane's 16 / 4 bytes at g land at LDS
// address `lds` + lane * 16 / 4), outside the compiler's wait-count tracking:
// the streaming waves wait for them with explicit vmcnt counts.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :: "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void bare_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kSlot = 1024 + 64;  // packed words, then the 40-byte record
constexpr uint64_t kWaitTicks = 20000000;  // 0.2 s of the 100 MHz realtime counter

__device__ __forceinline__ uint64_t load_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint16_t load_agent16(const uint16_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-link geometry of this workgroup's share: strips [sb, sb + ns) of the
// link, all K / 128 chunks of each; unit u = local strip * KC + chunk.  The
// strip ranges split the link's strips evenly over the W workgroups, each
// link rotated by its own offset so that the workgroups holding one strip
// more than the others change from link to link.  Divisions use the host's
// multipliers (floor(n / d) = umulhi(n, ceil(2^32 / d)) while n * d < 2^32).
struct Share {
  int KC, sb, ns, units;
  uint32_t kcmag;
};

__device__ __forceinline__ Share share_of(const ChainLinkDev& L, int wg, int W, uint32_t wmag) {
  Share s;
  s.KC = L.K / kChunkK;
  const int S = L.N / kStripN;
  int r = wg + L.rot;
  if (r >= W) r -= W;
  s.sb = W == 1 ? 0 : (int)__umulhi((uint32_t)(r * S), wmag);
  const int se = W == 1 ? S : (int)__umulhi((uint32_t)((r + 1) * S), wmag);
  s.ns = se - s.sb;
  s.units = s.ns * s.KC;
  s.kcmag = L.kcmag;
  return s;
}

}  // namespace

template <int SW, int R>
__global__ void __launch_bounds__((SW + 1) * 64)
chain_kernel(const ChainLinkDev* __restrict__ links, ChainHeader* hdr, uint64_t* progress,
             int count, int M, int max_k, int max_strips, uint32_t wmag) {
  // (the link table is a read-only, non-aliased argument and every index
  // into it is wave-uniform, so its fields are scalar loads: a vector load
  // here would make the streaming waves wait for their whole ring)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int W = gridDim.x;
  const int wg = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint64_t epoch = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) + 1;

  // LDS: activations [M][K] fp16, partial sums [parity][SW][max_strips][16
  // lanes] f4, then the rings
  _Float16* xbuf = reinterpret_cast<_Float16*>(smem);
  const size_t xbytes = ((size_t)M * max_k * 2 + 15) & ~(size_t)15;
  f4* part = reinterpret_cast<f4*>(smem + xbytes);
  unsigned char* rings = smem + xbytes + (size_t)2 * SW * max_strips * 256;

  if (wave == 0) {
    // ------------------------------------------------------------ control
    const uint64_t tag = epoch << 20;
    int pending = -1;
    // Sum the streaming waves' partials of link `li` (fixed wave order) and
    // store the fp16 outputs, then publish this workgroup's progress.
    auto finish = [&](int li) {
      const ChainLinkDev& L = links[li];
      const Share sh = share_of(L, wg, W, wmag);
      const f4* pp = part + (size_t)(li & 1) * SW * max_strips * 16;
      for (int col = lane; col < sh.ns * 16; col += 64) {
        const int sl = col >> 4, j = col & 15;
        const int n = (sh.sb + sl) * kStripN + j;
        const _Float16 b = L.bias != nullptr ? as_h(L.bias[n]) : (_Float16)0.f;
        for (int m = 0; m < M; ++m) {
          float sum = 0.f;
#pragma unroll 4
          for (int w = 0; w < SW; ++w) sum += pp[((size_t)w * max_strips + sl) * 16 + j][m];
          _Float16 out = (_Float16)sum;
          if (L.bias != nullptr) out = out + b;
          if (L.res != nullptr) out = out + as_h(load_agent16(L.res + (size_t)m * L.ldres + n));
          __hip_atomic_store(L.y + (size_t)m * L.ldy + n, h_bits(out), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      wait_own_stores();  // outputs complete at agent scope before the progress word
      if (lane == 0)
        __hip_atomic_store(progress + wg, tag | (uint64_t)(li + 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
    for (int li = 0; li < count; ++li) {
      const ChainLinkDev& L = links[li];
      if (!(L.flags & kChainSameX)) {
        if (pending >= 0) {
          finish(pending);
          pending = -1;
        }
        if (L.after >= 0) {
          const uint64_t want = tag | (uint64_t)(L.after + 1);
          const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
          while (true) {
            // every lane's words in flight at once, then one wave vote
            uint64_t lo = ~0ull;
            for (int i = lane; i < W; i += 64) {
              const uint64_t v = load_agent(progress + i);
              lo = v < lo ? v : lo;
            }
            if (__all(lo >= want)) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kWaitTicks) {
              if (lane == 0)
                __hip_atomic_store(&hdr->timed_out, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
            __builtin_amdgcn_s_sleep(1);
          }
        }
        // activations [M][K] into LDS: agent-scope 16-byte loads, all of a
        // batch (16 per lane) in flight before their LDS writes.  One buffer
        // resource at x; row m at byte offset 2 m ldx (the host keeps the
        // rows within 2 GiB of x).
        const int per_row = L.K / 8;
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc((void*)L.x, 0, 0x7fffffff, 0x00020000);
        const uint32_t row_bytes = (uint32_t)(L.ldx * 2);
        for (int m = 0; m < M; ++m) {
          for (int u0 = 0; u0 < per_row; u0 += 64 * 16) {
            // lanes past the row's end repeat its last unit (same bytes to
            // the same place), so every branch here is wave-uniform
            u4 v[16];
#pragma unroll
            for (int b = 0; b < 16; ++b) {
              const int u = min(u0 + b * 64 + lane, per_row - 1);
              if (u0 + b * 64 < per_row)
                v[b] = __builtin_bit_cast(
                    u4, __builtin_amdgcn_raw_buffer_load_b128(
                            rx, (uint32_t)m * row_bytes + (uint32_t)u * 16, 0, 16 /* sc1 */));
            }
#pragma unroll
            for (int b = 0; b < 16; ++b) {
              const int u = min(u0 + b * 64 + lane, per_row - 1);
              if (u0 + b * 64 < per_row)
                *reinterpret_cast<u4*>(xbuf + (size_t)m * L.K + (size_t)u * 8) = v[b];
            }
          }
        }
      }
      bare_barrier();  // link li's activations in LDS
      if (pending >= 0) {  // the previous link shared these activations
        finish(pending);
        pending = -1;
      }
      bare_barrier();  // the streaming waves' partials of link li are in LDS
      pending = li;
    }
    if (pending >= 0) finish(pending);
    if (lane == 0) {
      const uint32_t done =
          __hip_atomic_fetch_add(&hdr->finished, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (done == (uint32_t)W - 1) {  // every workgroup is past every wait
        __hip_atomic_store(&hdr->finished, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&hdr->epoch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }

  // -------------------------------------------------------------- streaming
  const int ws = wave - 1;
  const int j = lane & 15;
  const int kq = lane >> 4;
  const int hsh = (j & 1) * 16;
  const int zsh = (j & 7) * 4;
  const uint32_t magic = kMagic;
  unsigned char* ring = rings + (size_t)ws * R * kSlot;
  const uint32_t ring0 = lds_addr(ring);

  // producer cursor: link pl, unit pu of this workgroup's share
  int pl = 0, pu = ws;
  Share psh = share_of(links[0], wg, W, wmag);
  const u4* pq = nullptr;
  const uint32_t* pz = nullptr;
  const uint32_t* ps = nullptr;
  int pG = 1;
  uint32_t pgmag = 0;
  auto p_link = [&]() {
    while (pl < count && pu >= psh.units) {
      pu = __builtin_amdgcn_readfirstlane(pu - psh.units);
      pl = __builtin_amdgcn_readfirstlane(pl + 1);
      if (pl < count) psh = share_of(links[pl], wg, W, wmag);
    }
    if (pl < count) {
      const ChainLinkDev& L = links[pl];
      pq = reinterpret_cast<const u4*>(L.pq);
      pz = L.pz;
      ps = L.ps32;
      pG = L.G;
      pgmag = L.gmag;
    }
  };
  p_link();
  // Past the end of the chain a wave re-copies a valid unit (its last real
  // one, or link 0's first chunk if it had none) into slots nothing reads
  // again, so the count of outstanding copies never changes.
  const void* last_q = reinterpret_cast<const u4*>(links[0].pq) + lane;
  const void* last_m = lane < 8 ? (const void*)(links[0].ps32 + lane)
                                : (const void*)(links[0].pz + (lane & 1));
  auto issue = [&](int slot) {
    const uint32_t dst = ring0 + (uint32_t)(slot * kSlot);
    if (pl < count) {
      const int sl = psh.kcmag == 0 ? pu : (int)__umulhi((uint32_t)pu, psh.kcmag);
      const int c = pu - sl * psh.KC;
      const int s = psh.sb + sl;
      const int g = pgmag == 0 ? c : (int)__umulhi((uint32_t)c, pgmag);
      last_q = pq + ((size_t)s * psh.KC + c) * 64 + lane;
      const size_t sg = (size_t)s * pG + g;
      last_m = lane < 8 ? (const void*)(ps + sg * 8 + lane)
                        : (const void*)(pz + sg * 2 + (lane & 1));
      pu += SW;
      p_link();
    }
    dma16(last_q, dst);
    if (lane < 10) dma4(last_m, dst + 1024);
  };
#pragma unroll
  for (int r = 0; r < R; ++r) issue(r);

  int cl = 0, cu = ws;  // consumer cursor
  Share csh = share_of(links[0], wg, W, wmag);
  auto c_link = [&]() {
    while (cl < count && cu >= csh.units) {
      cu = __builtin_amdgcn_readfirstlane(cu - csh.units);
      cl = __builtin_amdgcn_readfirstlane(cl + 1);
      if (cl < count) csh = share_of(links[cl], wg, W, wmag);
    }
  };
  c_link();
  int slot = 0;
  for (int li = 0; li < count; ++li) {
    bare_barrier();  // activations of link li in LDS
    const ChainLinkDev& L = links[li];
    const Share sh = share_of(L, wg, W, wmag);
    f4* pp = part + ((size_t)(li & 1) * SW + ws) * max_strips * 16;
    if (lane < 16)
      for (int sl = 0; sl < sh.ns; ++sl) pp[sl * 16 + lane] = f4{0.f, 0.f, 0.f, 0.f};
    const int K = L.K;
    const int arow = min(j, M - 1) * K + kq * 8;
    int cur = -1;
    f4 tot = f4{0.f, 0.f, 0.f, 0.f};
    while (cl == li) {
      const int sl = csh.kcmag == 0 ? cu : (int)__umulhi((uint32_t)cu, csh.kcmag);
      const int c = cu - sl * csh.KC;
      if (sl != cur) {
        if (cur >= 0 && lane < 16) pp[cur * 16 + lane] = tot;
        tot = f4{0.f, 0.f, 0.f, 0.f};
        cur = sl;
      }
      wait_vm<2 * (R - 1)>();  // this unit's two copies have landed
      const unsigned char* sp = ring + slot * kSlot;
      const u4 w = *reinterpret_cast<const u4*>(sp + lane * 16);
      const uint32_t sw = *reinterpret_cast<const uint32_t*>(sp + 1024 + (j >> 1) * 4);
      const uint32_t zw = *reinterpret_cast<const uint32_t*>(sp + 1024 + 32 + (j >> 3) * 4);
      const _Float16* xc = xbuf + arow + c * kChunkK;
      h8 a[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = *reinterpret_cast<const h8*>(xc + 32 * t);
      h2 nz1024, nz64;
      zero_consts(zw, zsh, nz1024, nz64);
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = mfma16(a[t], centered8(w[t], nz1024, nz64, magic), acc);
      tot += (float)as_h((uint16_t)(sw >> hsh)) * acc;
      // the slot's reads have returned (their values fed the MFMAs): refill it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(slot);
      slot = slot + 1 == R ? 0 : slot + 1;
      cu += SW;
      c_link();
    }
    if (cur >= 0 && lane < 16) pp[cur * 16 + lane] = tot;
    bare_barrier();  // partials of link li in LDS
  }
  wait_vm<0>();  // padding copies land before the workgroup's LDS is released
}

namespace {
constexpr int kChainWaves = 8;  // streaming waves per workgroup
constexpr int kRings[3] = {16, 12, 8};
}  // namespace

size_t chain_smem_bytes(int m, int max_k, int max_strips, int waves, int ring) {
  return (((size_t)m * max_k * 2 + 15) & ~(size_t)15) + (size_t)2 * waves * max_strips * 256 +
         (size_t)waves * ring * kSlot;
}

bool plan_chain(ChainPlan& p) {
  p.waves = kChainWaves;
  for (int r : kRings) {
    const size_t b = chain_smem_bytes(p.m, p.max_k, p.max_strips, p.waves, r);
    if (b <= kLdsPerCu) {
      p.ring = r;
      p.smem = b;
      return true;
    }
  }
  return false;
}

template <int R>
static hipError_t launch_chain_r(const ChainPlan& p, void* chain, hipStream_t stream) {
  static std::atomic<uint64_t> allowed{0};
  const void* kern = reinterpret_cast<const void*>(&chain_kernel<kChainWaves, R>);
  const hipError_t e = allow_lds(kern, kLdsPerCu, allowed);
  if (e != hipSuccess) return e;
  const uint32_t wmag =
      p.workgroups <= 1 ? 0u
                        : (uint32_t)(((1ull << 32) + (uint64_t)p.workgroups - 1) / p.workgroups);
  chain_kernel<kChainWaves, R><<<p.workgroups, (kChainWaves + 1) * 64, p.smem, stream>>>(
      reinterpret_cast<const ChainLinkDev*>(static_cast<unsigned char*>(chain) + kChainHeadBytes),
      static_cast<ChainHeader*>(chain),
      reinterpret_cast<uint64_t*>(static_cast<unsigned char*>(chain) +
                                  chain_progress_offset(p.count)),
      p.count, p.m, p.max_k, p.max_strips, wmag);
  return hipGetLastError();
}

hipError_t launch_chain(const ChainPlan& p, void* chain, hipStream_t stream) {
  switch (p.ring) {
    case 16: return launch_chain_r<16>(p, chain, stream);
    case 12: return launch_chain_r<12>(p, chain, stream);
    case 8: return launch_chain_r<8>(p, chain, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dw4
