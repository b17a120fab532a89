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
//     (one 16-column x 128-row chunk: 1 KiB of packed words) in flight with
//     global_load_lds, across link boundaries.  A unit is consumed from LDS exactly as the decode kernel
//     consumes it (exact q - z in fp16 from the 0x6400 identity, one
//     v_mfma_f32_16x16x32_f16 per 32-row k-step, the fp32 group scale applied
//     per chunk) and its slot is refilled with the wave's next unit at once,
//     so exactly R units per wave are always outstanding and one fixed
//     vmcnt wait serves every unit;
//   * wave 0 controls: one link ahead it copies the scale and zero records
//     of the workgroup's share of the next link into LDS (two areas, by link
//     parity); before a link it waits until every workgroup has completed
//     the links the link depends on (their progress words), then copies the
//     link's activations into LDS; after a link it sums the
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
#include "w4a16_chain.h"

namespace dw4 {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// The streaming waves' global -> LDS copies (global_load_lds: each active
// lane's 16 / 4 bytes at saddr + voffset land at LDS address m0 + lane * 16
// / 4) are inline assembly outside the compiler's wait-count tracking; the
// waves wait for them with explicit vmcnt counts.

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ void bare_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kSlot = 1024;  // one unit's packed words
constexpr int kXBatchChain = 24;  // activation loads per lane in flight
constexpr uint64_t kWaitTicks = 20000000;  // 0.2 s of the 100 MHz realtime counter

// Global-address-space forms: generic (flat) accesses would also count in
// lgkmcnt, so the LDS waits before each barrier would wait for them too.
typedef __attribute__((address_space(1))) uint16_t g_u16;
typedef __attribute__((address_space(1))) const uint16_t g_cu16;
typedef __attribute__((address_space(1))) uint64_t g_u64;

__device__ __forceinline__ uint64_t load_agent(const uint64_t* p) {
  return __hip_atomic_load((g_u64*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint16_t load_agent16(const uint16_t* p) {
  return __hip_atomic_load((g_cu16*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent16(uint16_t* p, uint16_t v) {
  __hip_atomic_store((g_u16*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// A link as the streaming waves see it, written once per launch into LDS by
// the control wave (the link table itself is read through the scalar cache,
// whose misses cost the streaming waves hundreds of cycles at every link).
struct LinkRec {
  const unsigned char* pq;  // packed words of the link
  int lin0;                 // first chunk (strip * KC) of this workgroup's share
  int units;                // chunks in the share (ns * KC)
  int kc_ns;                // KC | ns << 16
  int G;
  uint32_t gmag, kcmag;
};
static_assert(sizeof(LinkRec) == 32, "LDS link record");

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
             int count, int M, int max_k, int max_strips, uint32_t meta_s, uint32_t meta_z,
             uint32_t wmag) {
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
  // lanes] f4, the scale and zero records [parity] (meta_s + meta_z bytes
  // each), then the rings
  _Float16* xbuf = reinterpret_cast<_Float16*>(smem);
  const size_t xbytes = ((size_t)M * max_k * 2 + 15) & ~(size_t)15;
  f4* part = reinterpret_cast<f4*>(smem + xbytes);
  unsigned char* meta = smem + xbytes + (size_t)2 * SW * max_strips * 256;
  LinkRec* recs = reinterpret_cast<LinkRec*>(meta + (size_t)2 * (meta_s + meta_z));
  unsigned char* rings = reinterpret_cast<unsigned char*>(recs + count);

  if (wave == 0) {  // the streaming waves' link records, one lane per link
    for (int li = lane; li < count; li += 64) {
      const ChainLinkDev* L = links + li;
      const int K = L->K, N = L->N, rot = L->rot;
      const int KC = K / kChunkK, S = N / kStripN;
      int r = wg + rot;
      if (r >= W) r -= W;
      const int sb = W == 1 ? 0 : (int)__umulhi((uint32_t)(r * S), wmag);
      const int se = W == 1 ? S : (int)__umulhi((uint32_t)((r + 1) * S), wmag);
      LinkRec rec;
      rec.pq = reinterpret_cast<const unsigned char*>(L->pq);
      rec.lin0 = sb * KC;
      rec.units = (se - sb) * KC;
      rec.kc_ns = KC | ((se - sb) << 16);
      rec.G = L->G;
      rec.gmag = L->gmag;
      rec.kcmag = L->kcmag;
      recs[li] = rec;
    }
  }
  bare_barrier();  // link records in LDS

  if (wave == 0) {
    // ------------------------------------------------------------ control
    const uint64_t tag = epoch << 20;
    int pending = -1;
    // The scale records [strip][group] (32 bytes each) and zero records
    // (8 bytes each) of this workgroup's strips of link li: each a
    // contiguous block of the packed arrays, copied global -> LDS with every
    // lane active (lanes past a block's end re-copy its last bytes into the
    // area's slack).  Waited for (vmcnt 0) before the link's first barrier.
    auto copy_meta = [&](int li) {
      const ChainLinkDev& L = links[li];
      const Share sh = share_of(L, wg, W, wmag);
      if (sh.ns == 0) return;
      unsigned char* area = meta + (size_t)(li & 1) * (meta_s + meta_z);
      const uint32_t sbytes = (uint32_t)(sh.ns * L.G * 32);
      const unsigned char* ssrc =
          reinterpret_cast<const unsigned char*>(L.ps32) + (size_t)sh.sb * L.G * 32;
      for (uint32_t o = 0; o < sbytes; o += 1024) {
        const uint32_t v = min(o + (uint32_t)lane * 16, sbytes - 16);
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                     :: "v"(v), "s"(lds_addr(area) + o), "s"(ssrc) : "memory");
      }
      const uint32_t zbytes = (uint32_t)(sh.ns * L.G * 8);
      const unsigned char* zsrc =
          reinterpret_cast<const unsigned char*>(L.pz) + (size_t)sh.sb * L.G * 8;
      for (uint32_t o = 0; o < zbytes; o += 256) {
        const uint32_t v = min(o + (uint32_t)lane * 4, zbytes - 4);
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, %2"
                     :: "v"(v), "s"(lds_addr(area) + meta_s + o), "s"(zsrc) : "memory");
      }
    };
    // Sum the streaming waves' partials of link `li` (fixed wave order) and
    // store the fp16 outputs; publish this workgroup's progress if a later
    // link waits for this one.
    auto finish = [&](int li) {
      const ChainLinkDev& L = links[li];
      const Share sh = share_of(L, wg, W, wmag);
      const f4* pp = part + (size_t)(li & 1) * SW * max_strips * 16;
      for (int col = lane; col < sh.ns * 16; col += 64) {
        const int sl = col >> 4, j = col & 15;
        const int n = (sh.sb + sl) * kStripN + j;
        const _Float16 b = L.bias != nullptr ? as_h(((g_cu16*)L.bias)[n]) : (_Float16)0.f;
        f4 pw[SW];  // every wave's partial of this column: all reads in flight first
#pragma unroll
        for (int w = 0; w < SW; ++w) pw[w] = pp[((size_t)w * max_strips + sl) * 16 + j];
        for (int m = 0; m < M; ++m) {
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < SW; ++w) sum += pw[w][m];
          _Float16 out = (_Float16)sum;
          if (L.bias != nullptr) out = out + b;
          if (L.res != nullptr) out = out + as_h(load_agent16(L.res + (size_t)m * L.ldres + n));
          store_agent16(L.y + (size_t)m * L.ldy + n, h_bits(out));
        }
      }
      if (L.flags & kChainPublish) {
        wait_own_stores();  // outputs complete at agent scope before the progress word
        if (lane == 0)
          __hip_atomic_store(progress + wg, tag | (uint64_t)(li + 1), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    };
    copy_meta(0);
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
        // batch (kXBatchChain per lane: a whole row up to K = 12288) in
        // flight before their LDS writes.  One buffer resource at x; row m
        // at byte offset 2 m ldx (the host keeps the rows within 2 GiB of x).
        const int per_row = L.K / 8;
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc((void*)L.x, 0, 0x7fffffff, 0x00020000);
        const uint32_t row_bytes = (uint32_t)(L.ldx * 2);
        for (int m = 0; m < M; ++m) {
          for (int u0 = 0; u0 < per_row; u0 += 64 * kXBatchChain) {
            // lanes past the row's end repeat its last unit (same bytes to
            // the same place), so every branch here is wave-uniform
            u4 v[kXBatchChain];
#pragma unroll
            for (int b = 0; b < kXBatchChain; ++b) {
              const int u = min(u0 + b * 64 + lane, per_row - 1);
              if (u0 + b * 64 < per_row)
                v[b] = __builtin_bit_cast(
                    u4, __builtin_amdgcn_raw_buffer_load_b128(
                            rx, (uint32_t)m * row_bytes + (uint32_t)u * 16, 0, 16 /* sc1 */));
            }
#pragma unroll
            for (int b = 0; b < kXBatchChain; ++b) {
              const int u = min(u0 + b * 64 + lane, per_row - 1);
              if (u0 + b * 64 < per_row)
                *reinterpret_cast<u4*>(xbuf + (size_t)m * L.K + (size_t)u * 8) = v[b];
            }
          }
        }
      }
      wait_vm<0>();    // this link's scale / zero records are in LDS
      bare_barrier();  // link li's activations and records in LDS
      if (li + 1 < count) copy_meta(li + 1);  // the other area: link li - 1 is done
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
  const uint32_t magic = opaque(kMagic);
  unsigned char* ring = rings + (size_t)ws * R * kSlot;
  const uint32_t ring0 = lds_addr(ring);

  // Producer: the wave's units are every SW-th unit of the workgroup's unit
  // sequence (the shares of all links, one after another).  Within a link
  // the share is a run of whole strips, so a unit's chunk is the linear
  // index lin = strip * KC + chunk of the packed matrix (1 KiB each).
  int pl = 0;
  int plin = 0, pend = 0;  // the next unit to copy, the end of the share
  const unsigned char* pqb = nullptr;
  auto p_enter = [&](int over) {  // link pl, `over` units into its share
    const LinkRec& r = recs[pl];
    const int lin0 = __builtin_amdgcn_readfirstlane(r.lin0);
    plin = lin0 + over;
    pend = lin0 + __builtin_amdgcn_readfirstlane(r.units);
    const uint64_t q = reinterpret_cast<uint64_t>(r.pq);
    pqb = reinterpret_cast<const unsigned char*>(
        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(q >> 32)) << 32) |
        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)q));
  };
  auto p_settle = [&]() {  // move past shares the cursor has run off
    while (pl < count && plin >= pend) {
      const int over = plin - pend;
      pl = __builtin_amdgcn_readfirstlane(pl + 1);
      if (pl < count) p_enter(over);
    }
  };
  p_enter(ws);
  const unsigned char* lq0 = pqb;  // link 0's packed words
  p_settle();
  // Past the end of the chain a wave re-copies a valid unit (its last real
  // one, or link 0's first chunk if it had none) into slots nothing reads
  // again, so the count of outstanding copies never changes.
  const unsigned char* lq = lq0;
  const uint32_t voff16 = lane * 16;
  auto issue = [&](int slot) {
    if (pl < count) {
      lq = pqb + (size_t)plin * 1024;
      plin = __builtin_amdgcn_readfirstlane(plin + SW);
      p_settle();
    }
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2 nt"
                 :: "v"(voff16), "s"(ring0 + (uint32_t)(slot * kSlot)), "s"(lq) : "memory");
  };
#pragma unroll
  for (int r = 0; r < R; ++r) issue(r);

  // Consumer: the same unit sequence, R units behind.  `cu` is the wave's
  // offset into the current link's share (carried over the links); strips
  // and chunks advance incrementally.
  const uint32_t woff = (uint32_t)lane * 16;
  int cu = ws;
  int slot = 0;
  struct Unit {
    u4 w;
    uint32_t sw, zw;
    h8 a[4];
  };
  for (int li = 0; li < count; ++li) {
    bare_barrier();  // activations and records of link li in LDS
    const LinkRec& rec = recs[li];
    const int kc_ns = __builtin_amdgcn_readfirstlane(rec.kc_ns);
    Share sh;
    sh.KC = kc_ns & 0xffff;
    sh.ns = kc_ns >> 16;
    sh.units = __builtin_amdgcn_readfirstlane(rec.units);
    sh.kcmag = (uint32_t)__builtin_amdgcn_readfirstlane((int)rec.kcmag);
    f4* pp = part + ((size_t)(li & 1) * SW + ws) * max_strips * 16;
    if (lane < 16)
      for (int sl = 0; sl < sh.ns; ++sl) pp[sl * 16 + lane] = f4{0.f, 0.f, 0.f, 0.f};
    if (cu < sh.units) {
      // A rows: lanes past the last row read row M - 1 (those MFMA output
      // rows are never stored)
      const unsigned char* xrow = reinterpret_cast<const unsigned char*>(xbuf) +
                                  (size_t)(min(j, M - 1) * sh.KC * kChunkK + kq * 8) * 2;
      const unsigned char* area = meta + (size_t)(li & 1) * (meta_s + meta_z);
      const unsigned char* srec = area + (j >> 1) * 4;           // + record * 32
      const unsigned char* zrec = area + meta_s + (j >> 3) * 4;  // + record * 8
      const int G = __builtin_amdgcn_readfirstlane(rec.G);
      const uint32_t gmag = (uint32_t)__builtin_amdgcn_readfirstlane((int)rec.gmag);
      int sl = sh.kcmag == 0 ? cu : (int)__umulhi((uint32_t)cu, sh.kcmag);
      int c = cu - sl * sh.KC;
      int cur = sl;
      f4 tot = f4{0.f, 0.f, 0.f, 0.f};
      auto fetch = [&](Unit& u, int s, int ch, int strip) {  // LDS reads of one unit
        u.w = *reinterpret_cast<const u4*>(ring + s * kSlot + woff);
        const int rec = strip * G + (gmag == 0 ? ch : (int)__umulhi((uint32_t)ch, gmag));
        u.sw = *reinterpret_cast<const uint32_t*>(srec + rec * 32);
        u.zw = *reinterpret_cast<const uint32_t*>(zrec + rec * 8);
        const unsigned char* xc = xrow + ch * (kChunkK * 2);
#pragma unroll
        for (int t = 0; t < 4; ++t) u.a[t] = *reinterpret_cast<const h8*>(xc + 64 * t);
      };
      // One unit: the next unit's LDS reads go out first (two unit buffers
      // alternate, so nothing is copied between them), then this unit's
      // math, then its slot is refilled.  Returns whether the wave has
      // another unit in this link.
      auto step = [&](Unit& u0, Unit& u1) -> bool {
        const bool more = cu + SW < sh.units;
        const int nslot = slot + 1 == R ? 0 : slot + 1;
        int cn = c + SW, sn = sl;
        while (cn >= sh.KC) {
          cn -= sh.KC;
          ++sn;
        }
        if (more) {
          wait_vm<R - 2>();  // the next unit's copy has landed
          fetch(u1, nslot, cn, sn);
        }
        h2 nz1024, nz64;
        zero_consts(u0.zw, zsh, nz1024, nz64);
        f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc = mfma16(u0.a[t], centered8(u0.w[t], nz1024, nz64, magic), acc);
        tot += (float)as_h((uint16_t)(u0.sw >> hsh)) * acc;
        // this slot's reads returned (their values fed the math): refill it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(slot);
        slot = nslot;
        cu += SW;
        if (more) {
          c = cn;
          sl = sn;
          if (sl != cur) {
            if (lane < 16) pp[cur * 16 + lane] = tot;
            tot = f4{0.f, 0.f, 0.f, 0.f};
            cur = sl;
          }
        }
        return more;
      };
      Unit ua, ub;
      wait_vm<R - 1>();  // this unit's copy has landed
      fetch(ua, slot, c, sl);
      while (step(ua, ub) && step(ub, ua)) {
      }
      if (lane < 16) pp[cur * 16 + lane] = tot;
    }
    cu -= sh.units;  // the offset carried into the next link's share
    bare_barrier();  // partials of link li in LDS
  }
  wait_vm<0>();  // padding copies land before the workgroup's LDS is released
}

#ifndef DW4_CHAIN_WAVES
#define DW4_CHAIN_WAVES 8
#endif
namespace {
constexpr int kChainWaves = DW4_CHAIN_WAVES;  // streaming waves per workgroup
constexpr int kRings[5] = {16, 12, 10, 8, 6};  // ring depths instantiated, deepest first
}  // namespace

size_t chain_meta_bytes(int max_strips, int max_groups, bool zeros) {
  // the scale area in whole 1 KiB copies, the zero area in whole 256-byte
  // copies (the copies' last lanes land in the slack)
  return zeros ? (((size_t)max_strips * max_groups * 8 + 255) & ~(size_t)255)
               : (((size_t)max_strips * max_groups * 32 + 1023) & ~(size_t)1023);
}

size_t chain_smem_bytes(int m, int max_k, int max_strips, int max_groups, int count, int waves,
                        int ring) {
  return (((size_t)m * max_k * 2 + 15) & ~(size_t)15) + (size_t)2 * waves * max_strips * 256 +
         2 * (chain_meta_bytes(max_strips, max_groups, false) +
              chain_meta_bytes(max_strips, max_groups, true)) +
         (size_t)count * sizeof(LinkRec) + (size_t)waves * ring * kSlot;
}

bool plan_chain(ChainPlan& p) {
  p.waves = kChainWaves;
  for (int r : kRings) {
    const size_t b =
        chain_smem_bytes(p.m, p.max_k, p.max_strips, p.max_groups, p.count, p.waves, r);
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
      p.count, p.m, p.max_k, p.max_strips,
      (uint32_t)chain_meta_bytes(p.max_strips, p.max_groups, false),
      (uint32_t)chain_meta_bytes(p.max_strips, p.max_groups, true), wmag);
  return hipGetLastError();
}

hipError_t launch_chain(const ChainPlan& p, void* chain, hipStream_t stream) {
  switch (p.ring) {
    case 16: return launch_chain_r<16>(p, chain, stream);
    case 12: return launch_chain_r<12>(p, chain, stream);
    case 10: return launch_chain_r<10>(p, chain, stream);
    case 8: return launch_chain_r<8>(p, chain, stream);
    case 6: return launch_chain_r<6>(p, chain, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dw4
