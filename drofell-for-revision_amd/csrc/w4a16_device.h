// Device-side helpers shared by the gfx950 kernel files (types, the int4 ->
// fp16 dequantisation identity, MFMA wrappers, activation gathers).
#pragma once

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

// A constant the compiler can no longer see: the value passes through an
// empty assembly statement that leaves it in a VGPR.  Kernels make their
// dequantisation magic opaque once, at the start, so that and_or below is one
// v_and_or_b32 (mask in an SGPR, magic in that VGPR): with both constants
// known the compiler would emit two instructions (a gfx9 VOP3 instruction
// cannot encode literals), and hiding it per call re-creates the constant in
// a VGPR once per chunk.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// (a & mask) | magic, magic from opaque().  The v_and_or_b32 is the
// compiler's, so its hazard recognizer sees the register write and keeps the
// wait states the matrix cores need around it (an MFMA reading a VALU result;
// a VALU overwriting the SrcC or the destination of an MFMA in flight).
// Written as assembly, the instruction was invisible to it: results then fed
// MFMAs, or overwrote an in-flight MFMA's SrcC, closer than those wait states.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  return (a & mask) | magic;
}

// The 8 rows of one packed word, minus the effective zero, as exact fp16
// integers in row order.  Even rows sit in the low half-word, odd rows in
// the high half-word, so OR-ing a nibble pair into the fp16 pattern of
// 1024.0 yields (1024 + q) or (1024 + 16 q) in each half without a shift.
__device__ __forceinline__ h8 centered8(uint32_t w, h2 nz1024, h2 nz64, uint32_t magic) {
  const h2 sixteenth = splat2((_Float16)0.0625f);
  const uint32_t w8 = w >> 8;
  const h2 p0 = as_h2(and_or(w, 0x000F000Fu, magic)) + nz1024;               // rows 0,1
  const h2 p1 = as_h2(and_or(w, 0x00F000F0u, magic)) * sixteenth + nz64;     // rows 2,3
  const h2 p2 = as_h2(and_or(w8, 0x000F000Fu, magic)) + nz1024;              // rows 4,5
  const h2 p3 = as_h2(and_or(w8, 0x00F000F0u, magic)) * sixteenth + nz64;    // rows 6,7
  const h4 a = __builtin_shufflevector(p0, p1, 0, 1, 2, 3);
  const h4 b = __builtin_shufflevector(p2, p3, 0, 1, 2, 3);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Zero-point constants -(1024 + z_eff) and -(64 + z_eff) (z_eff = stored + 1,
// 1..16) built from their fp16 bit patterns: 1024 + z has exponent 10 and
// mantissa z, 64 + z has exponent 6 and mantissa 16 z.  With the stored
// nibble zs the patterns are 0xE401 + zs and 0xD410 + 16 zs (no carry out of
// a half-word: at most 0xE410 and 0xD500), so each is one multiply-add over
// both halves.
__device__ __forceinline__ void zero_consts(uint32_t zword, int zshift, h2& nz1024, h2& nz64) {
  const uint32_t zs = (zword >> zshift) & 15u;
  nz1024 = as_h2(zs * 0x00010001u + 0xE401E401u);
  nz64 = as_h2(zs * 0x00100010u + 0xD410D410u);
}

// Wait until every vector memory operation this wave has issued has
// completed (s_waitcnt vmcnt(0), the other counters left alone).  Before a
// workgroup barrier that precedes one thread's agent-scope release, it makes
// each wave's own write-through stores visible at agent scope first: a
// release orders only the issuing wave's operations, and the barrier itself
// does not wait for memory.
__device__ __forceinline__ void wait_own_stores() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// bf16 operands: the same 16 bytes per lane as h8, read as eight bf16.
typedef __bf16 b8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma16_bf16(h8 a, u4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a),
                                                  __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

constexpr uint32_t kMagicBf16 = 0x43004300u;  // bf16 128.0 in both halves
constexpr uint32_t kOnesBf16 = 0x3F803F80u;   // bf16 1.0 in both halves

// The 8 rows of one packed word as the bf16 values 128 + q, in row order
// (even rows of a nibble pair in the low half-word, as centered8 reads
// them).  bf16 keeps 7 mantissa bits, so OR-ing a nibble into the pattern
// of 128.0 gives 128 + q exactly; each pair is shifted down to bits 0-3 of
// its half-words first (a nibble at bits 4-7 would reach the exponent).
__device__ __forceinline__ u4 biased8_bf16(uint32_t w, uint32_t magic) {
  return u4{and_or(w, 0x000F000Fu, magic), and_or(w >> 4, 0x000F000Fu, magic),
            and_or(w >> 8, 0x000F000Fu, magic), and_or(w >> 12, 0x000F000Fu, magic)};
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet), and back.
__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

typedef float f16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f16v mfma32(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Two 16-column strips' packed word w (lanes L: column L%16, rows 8(L/16)..)
// rearranged into the B operands of v_mfma_f32_32x32x16_f16 for the strip
// pair's 32 columns: `even` holds k-step 2w (lane L: column L%32, rows
// 8(L/32)..), `odd` k-step 2w+1.
__device__ __forceinline__ void strip_pair_to_b32(uint32_t a, uint32_t b, uint32_t& even,
                                                  uint32_t& odd) {
  const auto x = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  const auto y = __builtin_amdgcn_permlane32_swap(x[0], x[1], false, false);
  even = y[0];
  odd = y[1];
}

// One 16-byte unit (8 consecutive sorted rows) of an activation row,
// gathered through perm for act-order checkpoints.
template <bool ACT>
__device__ __forceinline__ h8 load_x_unit(const _Float16* __restrict__ row,
                                          const int32_t* __restrict__ perm, int k) {
  if (ACT) {
    const i4 p0 = *(const i4*)(perm + k);
    const i4 p1 = *(const i4*)(perm + k + 4);
    return h8{row[p0[0]], row[p0[1]], row[p0[2]], row[p0[3]],
              row[p1[0]], row[p1[1]], row[p1[2]], row[p1[3]]};
  }
  return *(const h8*)(row + k);
}

// Entry i of a per-item array of a grouped launch (item index wave-uniform).
// Indexed directly: the array lives in the kernel-argument segment, so this
// is one scalar load at a computed offset.  A select chain over the four
// entries compiles to a tree of scalar branches ahead of the first memory
// load (~170 more instructions in the grouped decode kernel's prologue,
// measured 0.3-0.85 us per launch).
template <typename T, int L>
__device__ __forceinline__ T pick(const T (&v)[L], int i) {
  static_assert(kGroupMax == 4 && L >= 4, "pick() selects among four items");
  return v[i];
}

// Item that owns workgroup b (wg0 ascending).
__device__ __forceinline__ int item_of(const Items& d, int b) {
  return (d.count > 1 && b >= d.wg0[1]) + (d.count > 2 && b >= d.wg0[2]) +
         (d.count > 3 && b >= d.wg0[3]);
}

// Eight fp16 sums a + b of packed halves, each rounded once (v_pk_add_f16),
// as an fp16 tensor add rounds them.
__device__ __forceinline__ u4 add_h8(u4 a, u4 b) {
  u4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = __builtin_bit_cast(uint32_t, as_h2(a[e]) + as_h2(b[e]));
  return r;
}

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + __expf(-v)); }

}  // namespace dw4
