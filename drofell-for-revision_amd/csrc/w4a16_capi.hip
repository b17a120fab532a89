// C ABI of libdrofell_w4a16.so (declared in include/drofell_w4a16.h).
//
// Validation and dispatch live here; the kernels are in the other w4a16_*.hip files.
// Every entry point returns a status code; nothing throws across the ABI.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "drofell_w4a16.h"
#include "w4a16_attention.h"
#include "w4a16_chain.h"
#include "w4a16_prefill.h"
#include "w4a16_transpose.h"
#include "w4a16_internal.h"

namespace {

using dw4::kChunkK;
using dw4::kStripN;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // per-device property cache (0 = unknown)

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int v = g_cu_count[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    g_cu_count[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace

hipError_t dw4::allow_lds(const void* kernel, size_t bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess && bit != 0) done.fetch_or(bit, std::memory_order_release);
  return e;
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_shape(int k, int n, int group_size) {
  if (k <= 0 || n <= 0 || group_size <= 0) return DW4_ERR_INVALID_ARG;
  if (k % kChunkK != 0 || n % kStripN != 0) return DW4_ERR_UNSUPPORTED;
  // a 128-row chunk holds whole groups (32, 64) or lies inside one group
  const bool small = group_size == 32 || group_size == 64;
  if ((!small && group_size % kChunkK != 0) || k % group_size != 0) return DW4_ERR_UNSUPPORTED;
  return DW4_OK;
}

int status_of(hipError_t e) { return e == hipSuccess ? DW4_OK : DW4_ERR_LAUNCH; }

size_t prefill_ws_bytes(const dw4::PrefillPlan& p, int m, int n);

// Prefill tiling and split-K factor for one call.  `ws_bytes` caps the
// split count: with too little workspace the call runs unsplit.
dw4::PrefillPlan plan_prefill(int m, int k, int n, int split_req, size_t ws_bytes, bool cap_by_ws) {
  dw4::PrefillPlan p;
  // Row tile: 16 or 32 rows just covering small M, then 64 (above 128 rows
  // the choice below).  Fewer rows per tile mean fewer MFMA uses per
  // dequantised weight fragment, so the small tiles are only for small M.
  p.bm = m <= 16 ? 16 : m <= 32 ? 32 : 64;
  p.bn = n >= 2048 ? 256 : 128;
  const int kc = k / kChunkK;
  const int cus_now = cu_count();
  // automatic split count for a tile count (rule below)
  auto auto_splits = [&](int tiles) {
    int sp = tiles >= cus_now ? 1 : cus_now / tiles;
    sp = std::min(sp, std::max(1, kc / 8));
    return std::min(sp, 8);
  };
  auto filled = [&](int bm, int bn) {  // workgroups of one round, at most one per CU
    const int t = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    return std::min(cus_now, t * auto_splits(t));
  };
  // Mid M (33..128 rows): 128-column tiles, and 32-row tiles where they fill
  // more CUs than 64-row ones (ties keep the taller tile, which dequantises
  // each weight fragment for more rows).  Measured at M=64: 4096^2 20.2 ->
  // 13.4 us, 4096x11008 22.3 -> 19.7, 11008x4096 30.8 -> 24.0.
  if (p.bm >= 32 && m <= 128) {
    p.bn = 128;
    if (p.bm == 64 && m <= 64 && filled(32, 128) > filled(64, 128)) p.bm = 32;
  }
  // Above 128 rows, the LDS-streamed kernel, on the tile shape that needs
  // the fewest rounds of workgroups (one workgroup per CU at a time), ties
  // going to the first of: 64 x 256 (up to 512 rows: twice the tiles of
  // 128-row ones, so fewer split-K partial planes), 128 x 128, 128 x 256
  // (each dequantised weight fragment feeds four MFMAs in the 128-row
  // tiles).  Measured (us): 4096^2 M=512 30.8 with 64 x 256 against 35.1
  // with 128 x 128; 4096x11008 M=512 74.4 with two rounds of 64 x 256
  // against 61.3 with one of 128 x 256; 4096^2 M=1024 42.0 with 128 x 128
  // against 52.9 with 64 x 256.
  if (m > 128) {
    const int cand[3][2] = {{64, 256}, {128, 128}, {128, 256}};
    int best_rounds = 1 << 30;
    for (int c = m <= 512 ? 0 : 1; c < 3; ++c) {
      const int t = ((m + cand[c][0] - 1) / cand[c][0]) * ((n + cand[c][1] - 1) / cand[c][1]);
      const int rounds = (t + cus_now - 1) / cus_now;
      if (rounds < best_rounds) {
        best_rounds = rounds;
        p.bm = cand[c][0];
        p.bn = cand[c][1];
      }
    }
    // 4-wave 64 x 128 workgroups (two per CU) where they need fewer K splits
    // in as few rounds, for K up to 4096 (longer K keeps the 8-wave tiles,
    // whose chunks run ~10 % faster).  Measured (us): 4096^2 M=256 24.4 ->
    // 23.5 (2 splits instead of 4), M=384 28.3 -> 26.5, M=512 31.9 -> 28.2
    // (unsplit); 11008x4096 M=384 57.4 against 61.5 with the 4-wave tiles.
    if (m <= 512 && kc <= 32) {
      const int t8 = ((m + p.bm - 1) / p.bm) * ((n + p.bn - 1) / p.bn);
      const int t4 = ((m + 63) / 64) * ((n + 127) / 128);
      const int s8 = auto_splits(t8), s4 = auto_splits(t4);
      if ((t4 * s4 + 2 * cus_now - 1) / (2 * cus_now) <= best_rounds && s4 < s8) {
        p.bm = 64;
        p.bn = 128;
        p.waves = 4;
      }
    }
    // Up to 256 rows with K up to 4096: 4-wave 32 x 128 workgroups where
    // they fit two per CU.  A 32-row chunk costs ~0.52 us against ~0.72 us
    // for 64 x 128, so with K this short the extra dequantisation per row
    // costs less than the split planes and reduce launch the taller tiles
    // need.  Measured (us): 4096^2 M=160 22.4 -> 21.0, M=256 23.6 -> 21.4;
    // 4096x11008 M=160 39.8 -> 34.2.
    if (m <= 256 && kc <= 32) {
      const int t32 = ((m + 31) / 32) * ((n + 127) / 128);
      if (t32 <= 2 * cus_now) {
        p.bm = 32;
        p.bn = 128;
        p.waves = 4;
      }
    }
  }
  const int tiles = ((m + p.bm - 1) / p.bm) * ((n + p.bn - 1) / p.bn);
  // Automatic splits: enough to give every CU a workgroup (one per CU at a
  // time), with at least 8 chunks per split and at most 8 splits: every
  // split adds a partial plane to write and sum (the LDS-streamed kernel) or
  // lengthens the last-arriving split's sum (the kernel below 129 rows)
  // faster than it adds parallelism (measured on 7B shapes).
  int splits = split_req > 0 ? split_req : auto_splits(tiles);
  splits = std::max(1, std::min(splits, kc));
  // the launcher rounds to whole chunks per split
  const int cps = (kc + splits - 1) / splits;
  splits = (kc + cps - 1) / cps;
  if (tiles > dw4::kSplitCounters) splits = 1;  // one arrival counter per tile
  p.splits = splits;
  if (cap_by_ws && splits > 1 && prefill_ws_bytes(p, m, n) > ws_bytes) p.splits = 1;
  return p;
}

size_t prefill_ws_bytes(const dw4::PrefillPlan& p, int m, int n) {
  const size_t mt = (size_t)(m + p.bm - 1) / p.bm, nt = (size_t)(n + p.bn - 1) / p.bn;
  return dw4::split_ws_bytes(p.splits, mt * nt * p.bm * p.bn);
}

// The register-fed decode kernel addresses the rows of x with 32-bit element
// offsets from x, so its calls need (m - 1) * ldx + k < 2^31.
bool rows_fit_i32(int m, int64_t ldx, int k) {
  return (int64_t)(m > 0 ? m - 1 : 0) * ldx + k <= (int64_t)INT32_MAX;
}

bool use_decode(int path, int m, int k, int n) {
  if (path == DW4_PATH_DECODE) return true;
  if (path == DW4_PATH_PREFILL) return false;
  return dw4::auto_decode(m, n, cu_count(), k);
}

// Split-K bytes, then (act-order) the gathered activations: 256-aligned and
// never over the arrival-counter head, which every call leaves zero for the
// next split call on the workspace.
size_t workspace_for(int path, int m, int k, int n, int group_size, bool act) {
  if (m <= 0) return 0;
  const bool decode = use_decode(path, m, k, n);
  size_t split;
  if (decode) {
    const dw4::DecodePlan p = dw4::plan_decode(m, k, n, group_size, cu_count());
    split = dw4::split_ws_bytes(p.splits, (size_t)m * n);
  } else {
    const dw4::PrefillPlan p = plan_prefill(m, k, n, 0, 0, false);
    split = prefill_ws_bytes(p, m, n);
  }
  if (!act) return split;
  return dw4::gather_offset(split) + dw4::gather_bytes(m, k);
}

}  // namespace

extern "C" {

int dw4_abi_version(void) { return DW4_ABI_VERSION; }

const char* dw4_strerror(int status) {
  switch (status) {
    case DW4_OK: return "ok";
    case DW4_ERR_INVALID_ARG: return "invalid argument (null pointer, non-positive size or bad stride)";
    case DW4_ERR_UNSUPPORTED: return "unsupported shape: need K % 128 == 0, N % 16 == 0, group_size in {32, 64} or a multiple of 128, and K % group_size == 0";
    case DW4_ERR_MISALIGNED: return "misaligned buffer: pointers must be 16-byte aligned and ldx a multiple of 8";
    case DW4_ERR_BAD_GIDX: return "g_idx out of range or groups not of uniform size group_size";
    case DW4_ERR_WORKSPACE: return "workspace too small for this call (see dw4_workspace_size)";
    case DW4_ERR_LAUNCH: return "kernel launch failed";
    case DW4_ERR_DEVICE: return "HIP device error";
    case DW4_ERR_SCRATCH: return "call needs more scratch than dw4_gemm_noalloc's fixed DW4_NOALLOC_SCRATCH_BYTES (use dw4_gemm with a workspace of dw4_workspace_size bytes)";
    default: return "unknown status";
  }
}

int dw4_query_sizes(int k, int n, int group_size, int act_order, int max_m,
                    size_t* packed_qweight_bytes, size_t* packed_scales_bytes,
                    size_t* packed_zeros_bytes, size_t* perm_bytes, size_t* workspace_bytes) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (max_m < 0) return DW4_ERR_INVALID_ARG;
  const size_t groups = (size_t)(k / group_size);
  if (packed_qweight_bytes) *packed_qweight_bytes = (size_t)k * n / 2;
  if (packed_scales_bytes) *packed_scales_bytes = groups * n * sizeof(uint16_t);
  if (packed_zeros_bytes) *packed_zeros_bytes = groups * n / 2;
  if (perm_bytes) *perm_bytes = act_order ? (size_t)k * sizeof(int32_t) : 0;
  if (workspace_bytes) {
    size_t ws = 0;
    // enough for either explicit path at every M up to max_m
    for (int m = 1; m <= max_m; ++m) {
      ws = std::max(ws, workspace_for(DW4_PATH_PREFILL, m, k, n, group_size, act_order != 0));
      if (m <= dw4::kDecodeMaxM)
        ws = std::max(ws, workspace_for(DW4_PATH_DECODE, m, k, n, group_size, act_order != 0));
    }
    *workspace_bytes = ws;
  }
  return DW4_OK;
}

int dw4_workspace_size(int m, int k, int n, int group_size, int act_order, size_t* workspace_bytes) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (m < 0 || workspace_bytes == nullptr) return DW4_ERR_INVALID_ARG;
  *workspace_bytes = workspace_for(DW4_PATH_AUTO, m, k, n, group_size, act_order != 0);
  return DW4_OK;
}

int dw4_make_perm(int k, int group_size, const int32_t* g_idx_host, int32_t* perm_host) {
  if (k <= 0 || group_size <= 0 || g_idx_host == nullptr || perm_host == nullptr)
    return DW4_ERR_INVALID_ARG;
  if (k % group_size != 0) return DW4_ERR_UNSUPPORTED;
  const int groups = k / group_size;
  std::vector<int> count(groups, 0);
  for (int r = 0; r < k; ++r) {
    const int g = g_idx_host[r];
    if (g < 0 || g >= groups) return DW4_ERR_BAD_GIDX;
    ++count[g];
  }
  for (int g = 0; g < groups; ++g)
    if (count[g] != group_size) return DW4_ERR_BAD_GIDX;
  // exclusive prefix, then rows placed in ascending original order per group
  std::vector<int> next(groups, 0);
  for (int g = 0, acc = 0; g < groups; ++g) {
    next[g] = acc;
    acc += count[g];
  }
  for (int r = 0; r < k; ++r) perm_host[next[g_idx_host[r]]++] = r;
  return DW4_OK;
}

int dw4_repack(int k, int n, int group_size, const int32_t* qweight, const int32_t* qzeros,
               const uint16_t* scales, const int32_t* perm, int32_t* packed_qweight,
               int32_t* packed_zeros, uint16_t* packed_scales, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (!qweight || !qzeros || !scales || !packed_qweight || !packed_zeros || !packed_scales)
    return DW4_ERR_INVALID_ARG;
  if (!aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  const hipError_t e = dw4::launch_repack(
      reinterpret_cast<const uint32_t*>(qweight), reinterpret_cast<const uint32_t*>(qzeros), scales,
      perm, reinterpret_cast<uint32_t*>(packed_qweight), reinterpret_cast<uint32_t*>(packed_zeros),
      packed_scales, k, n, k / group_size, static_cast<hipStream_t>(stream));
  return status_of(e);
}

}  // extern "C"

namespace {

// dw4_gemm_path with an optional residual added after the rounding of the
// product (y = fp16(fp16(x @ W (+ bias)) + res)); res is y itself (same
// stride) or does not overlap it.
int gemm_run(int path, int split_k, int m, int k, int n, int group_size, const uint16_t* x,
             int64_t ldx, const int32_t* packed_qweight, const int32_t* packed_zeros,
             const uint16_t* packed_scales, const int32_t* perm, const uint16_t* bias,
             uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldres, void* workspace,
             size_t workspace_bytes, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (path < DW4_PATH_AUTO || path > DW4_PATH_PREFILL || m < 0 || split_k < 0)
    return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  if (!x || !packed_qweight || !packed_zeros || !packed_scales || !y) return DW4_ERR_INVALID_ARG;
  if (ldx < k || ldy < n) return DW4_ERR_INVALID_ARG;
  if (!aligned16(x) || (ldx % 8) != 0 || !aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  // rows of x too far apart for the decode kernel's 32-bit offsets take the
  // prefill kernel, which addresses rows in 64 bits
  const bool wide = !rows_fit_i32(m, ldx, k);
  if (wide && path == DW4_PATH_DECODE) return DW4_ERR_UNSUPPORTED;
  const bool decode = !wide && use_decode(path, m, k, n);
  if (decode && m > dw4::kDecodeMaxM) return DW4_ERR_INVALID_ARG;

  hipStream_t s = static_cast<hipStream_t>(stream);
  dw4::GemmArgs a;
  a.M = m;
  a.K = k;
  a.N = n;
  a.gs = group_size;
  a.G = k / group_size;
  a.x = x;
  a.ldx = ldx;
  a.pq = reinterpret_cast<const uint32_t*>(packed_qweight);
  a.pz = reinterpret_cast<const uint32_t*>(packed_zeros);
  a.ps = packed_scales;
  a.perm = perm;
  a.bias = bias;
  a.y = y;
  a.ldy = ldy;
  a.res = res;
  a.ldres = ldres;

  // Act-order: where the workspace holds the gathered activations after the
  // split-K area, gather x into the packed row order once and run the
  // kernels without perm; otherwise they gather per workgroup (same results).
  auto gather_after = [&](size_t split_need) -> int {
    if (perm == nullptr || workspace == nullptr || !aligned16(workspace)) return DW4_OK;
    const size_t off = dw4::gather_offset(split_need);
    if (workspace_bytes < off + dw4::gather_bytes(m, k)) return DW4_OK;
    uint16_t* xs = reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(workspace) + off);
    const int e = status_of(dw4::launch_gather_rows(x, ldx, perm, xs, k, m, s));
    if (e != DW4_OK) return e;
    a.x = xs;
    a.ldx = k;
    a.perm = nullptr;
    return DW4_OK;
  };

  if (decode) {
    dw4::DecodePlan plan = dw4::plan_decode(m, k, n, group_size, cu_count());
    // the register-fed kernel's K split is optional: without room (or
    // alignment) for its planes the call runs unsplit
    if (plan.reg && plan.splits > 1 &&
        (workspace == nullptr || !aligned16(workspace) ||
         workspace_bytes < dw4::split_ws_bytes(plan.splits, (size_t)m * n)))
      plan = dw4::plan_decode(m, k, n, group_size, cu_count(), false);
    float* part = nullptr;
    size_t need = 0;
    if (plan.splits > 1) {
      need = dw4::split_ws_bytes(plan.splits, (size_t)m * n);
      if (workspace == nullptr || workspace_bytes < need) return DW4_ERR_WORKSPACE;
      if (!aligned16(workspace)) return DW4_ERR_MISALIGNED;
      part = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + dw4::kWsHeadBytes);
    }
    // act-order M = 1: the staged kernel gathers from an LDS copy of x where
    // it fits (no gather launch); otherwise x is gathered into the workspace
    if (perm != nullptr) dw4::plan_decode_xg(plan, m, k, n, group_size, cu_count());
    if (!plan.xg) {
      const int e = gather_after(need);
      if (e != DW4_OK) return e;
    }
    return status_of(dw4::launch_decode(a, plan, part, s));
  }

  dw4::PrefillPlan plan = plan_prefill(m, k, n, split_k, workspace ? workspace_bytes : 0, true);
  if (plan.splits > 1 && !aligned16(workspace)) plan.splits = 1;
  const int e = gather_after(plan.splits > 1 ? prefill_ws_bytes(plan, m, n) : 0);
  if (e != DW4_OK) return e;
  // above 128 rows the LDS-streamed kernel, which needs x in the packed row
  // order (act-order calls whose workspace could not hold the gathered rows
  // keep the kernel that gathers per workgroup)
  if (m > 128 && a.perm == nullptr)
    return status_of(dw4::launch_prefill2(a, plan, workspace, s));
  return status_of(dw4::launch_prefill(a, plan, workspace, s));
}

}  // namespace

extern "C" {

int dw4_gemm_path(int path, int split_k, int m, int k, int n, int group_size, const uint16_t* x,
                  int64_t ldx, const int32_t* packed_qweight, const int32_t* packed_zeros,
                  const uint16_t* packed_scales, const int32_t* perm, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_run(path, split_k, m, k, n, group_size, x, ldx, packed_qweight, packed_zeros,
                  packed_scales, perm, bias, y, ldy, nullptr, 0, workspace, workspace_bytes,
                  stream);
}

int dw4_gemm(int m, int k, int n, int group_size, const uint16_t* x, int64_t ldx,
             const int32_t* packed_qweight, const int32_t* packed_zeros,
             const uint16_t* packed_scales, const int32_t* perm, const uint16_t* bias, uint16_t* y,
             int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  return dw4_gemm_path(DW4_PATH_AUTO, 0, m, k, n, group_size, x, ldx, packed_qweight, packed_zeros,
                       packed_scales, perm, bias, y, ldy, workspace, workspace_bytes, stream);
}

static_assert(dw4::kBf16MaxM == DW4_BF16_MAX_M, "bf16 decode limit");

int dw4_gemm_bf16(int m, int k, int n, int group_size, const uint16_t* x, int64_t ldx,
                  const int32_t* packed_qweight, const int32_t* packed_zeros,
                  const uint16_t* packed_scales, const int32_t* perm, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                  void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (m < 0) return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  if (m > DW4_BF16_MAX_M) return DW4_ERR_UNSUPPORTED;
  if (!x || !packed_qweight || !packed_zeros || !packed_scales || !y) return DW4_ERR_INVALID_ARG;
  if (ldx < k || ldy < n) return DW4_ERR_INVALID_ARG;
  if (!aligned16(x) || (ldx % 8) != 0 || !aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  // the register-fed kernel addresses rows of x with 32-bit offsets
  if (!rows_fit_i32(m, ldx, k)) return DW4_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dw4::GemmArgs a;
  a.M = m;
  a.K = k;
  a.N = n;
  a.gs = group_size;
  a.G = k / group_size;
  a.x = x;
  a.ldx = ldx;
  a.pq = reinterpret_cast<const uint32_t*>(packed_qweight);
  a.pz = reinterpret_cast<const uint32_t*>(packed_zeros);
  a.ps = packed_scales;
  a.perm = perm;
  a.bias = bias;
  a.y = y;
  a.ldy = ldy;
  a.res = nullptr;
  a.ldres = 0;
  // act-order: x gathered into the packed row order once where the
  // workspace has room (2-byte elements: the fp16 gather serves bf16)
  if (perm != nullptr && workspace != nullptr && aligned16(workspace)) {
    const size_t off = dw4::gather_offset(0);
    if (workspace_bytes >= off + dw4::gather_bytes(m, k)) {
      uint16_t* xs = reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(workspace) + off);
      const int e = status_of(dw4::launch_gather_rows(x, ldx, perm, xs, k, m, s));
      if (e != DW4_OK) return e;
      a.x = xs;
      a.ldx = k;
      a.perm = nullptr;
    }
  }
  return status_of(dw4::launch_decode_reg_bf16(a, dw4::plan_decode_bf16(m, k, n, group_size, cu_count()), s));
}

int dw4_dequant(int k, int n, int group_size, const int32_t* packed_qweight,
                const int32_t* packed_zeros, const uint16_t* packed_scales, const int32_t* perm,
                uint16_t* w, int64_t ldw, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (!packed_qweight || !packed_zeros || !packed_scales || !w) return DW4_ERR_INVALID_ARG;
  if (ldw < n) return DW4_ERR_INVALID_ARG;
  if (!aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  const hipError_t e = dw4::launch_dequant(
      reinterpret_cast<const uint32_t*>(packed_qweight),
      reinterpret_cast<const uint32_t*>(packed_zeros), packed_scales, perm, w, ldw, k, n,
      group_size, k / group_size, static_cast<hipStream_t>(stream));
  return status_of(e);
}

int dw4_dequant_bf16(int k, int n, int group_size, const int32_t* packed_qweight,
                     const int32_t* packed_zeros, const uint16_t* packed_scales,
                     const int32_t* perm, uint16_t* w, int64_t ldw, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (!packed_qweight || !packed_zeros || !packed_scales || !w) return DW4_ERR_INVALID_ARG;
  if (ldw < n) return DW4_ERR_INVALID_ARG;
  if (!aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  const hipError_t e = dw4::launch_dequant_bf16(
      reinterpret_cast<const uint32_t*>(packed_qweight),
      reinterpret_cast<const uint32_t*>(packed_zeros), packed_scales, perm, w, ldw, k, n,
      group_size, k / group_size, static_cast<hipStream_t>(stream));
  return status_of(e);
}

int dw4_stream_read(const void* src, size_t bytes, int workgroups, int threads, uint32_t never,
                    uint32_t* sink, void* stream) {
  if (src == nullptr || sink == nullptr || workgroups <= 0 || threads <= 0) return DW4_ERR_INVALID_ARG;
  if (threads % 64 != 0 || threads > 1024) return DW4_ERR_INVALID_ARG;
  if (!aligned16(src)) return DW4_ERR_MISALIGNED;
  const size_t chunk = 1024;
  if (bytes % ((size_t)workgroups * chunk) != 0) return DW4_ERR_INVALID_ARG;
  const size_t per = bytes / ((size_t)workgroups * chunk);
  if (per == 0 || per > (size_t)INT32_MAX) return DW4_ERR_INVALID_ARG;
  return status_of(dw4::launch_stream_read(src, workgroups, threads, (int)per, never, sink,
                                           static_cast<hipStream_t>(stream)));
}

static int check_cache_args(int num_tokens, int num_kv_heads, int head_size, int block_size,
                            const void* key, int64_t key_stride, const void* value,
                            int64_t value_stride, const int64_t* kp, const int64_t* vp,
                            int kv_head_stride, const int64_t* slots) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0) return DW4_ERR_INVALID_ARG;
  if (head_size % 8 != 0 || (block_size != 16 && block_size != 32)) return DW4_ERR_UNSUPPORTED;
  if (num_tokens == 0) return DW4_OK;
  if (!key || !value || !kp || !vp || !slots) return DW4_ERR_INVALID_ARG;
  const int64_t row = (int64_t)num_kv_heads * head_size;
  if (key_stride < row || value_stride < row || kv_head_stride < block_size * head_size)
    return DW4_ERR_INVALID_ARG;
  return DW4_OK;
}

int dw4_reshape_and_cache(int num_tokens, int num_kv_heads, int head_size, int block_size,
                          const uint16_t* key, int64_t key_stride, const uint16_t* value,
                          int64_t value_stride, const int64_t* key_block_ptrs,
                          const int64_t* value_block_ptrs, int kv_head_stride,
                          const int64_t* slot_mapping, void* stream) {
  const int st = check_cache_args(num_tokens, num_kv_heads, head_size, block_size, key, key_stride,
                                  value, value_stride, key_block_ptrs, value_block_ptrs,
                                  kv_head_stride, slot_mapping);
  if (st != DW4_OK || num_tokens == 0) return st;
  return status_of(dw4::launch_reshape_and_cache(
      const_cast<uint16_t*>(key), key_stride, const_cast<uint16_t*>(value), value_stride,
      key_block_ptrs, value_block_ptrs, slot_mapping, num_tokens, num_kv_heads, head_size,
      block_size, kv_head_stride, false, static_cast<hipStream_t>(stream)));
}

int dw4_restore_from_cache(int num_tokens, int num_kv_heads, int head_size, int block_size,
                           uint16_t* key, int64_t key_stride, uint16_t* value,
                           int64_t value_stride, const int64_t* key_block_ptrs,
                           const int64_t* value_block_ptrs, int kv_head_stride,
                           const int64_t* slot_mapping, void* stream) {
  const int st = check_cache_args(num_tokens, num_kv_heads, head_size, block_size, key, key_stride,
                                  value, value_stride, key_block_ptrs, value_block_ptrs,
                                  kv_head_stride, slot_mapping);
  if (st != DW4_OK || num_tokens == 0) return st;
  return status_of(dw4::launch_reshape_and_cache(
      key, key_stride, value, value_stride, key_block_ptrs, value_block_ptrs, slot_mapping,
      num_tokens, num_kv_heads, head_size, block_size, kv_head_stride, true,
      static_cast<hipStream_t>(stream)));
}

static int check_attn_shape(int num_seqs, int num_heads, int num_kv_heads, int head_size,
                            int block_size, int max_context_len) {
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_context_len < 0)
    return DW4_ERR_INVALID_ARG;
  if (num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > dw4::kAttnMaxGroup)
    return DW4_ERR_UNSUPPORTED;
  if ((head_size != 64 && head_size != 80 && head_size != 96 && head_size != 112 &&
       head_size != 128 && head_size != 256) ||
      (block_size != 16 && block_size != 32))
    return DW4_ERR_UNSUPPORTED;
  return DW4_OK;
}

int dw4_paged_attention_workspace_size(int num_seqs, int num_heads, int num_kv_heads,
                                       int head_size, int block_size, int max_context_len,
                                       size_t* workspace_bytes) {
  const int st = check_attn_shape(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                                  max_context_len);
  if (st != DW4_OK) return st;
  if (workspace_bytes == nullptr) return DW4_ERR_INVALID_ARG;
  const dw4::PagedAttnPlan p = dw4::plan_paged_attention(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                                                         max_context_len, cu_count());
  *workspace_bytes = num_seqs == 0 ? 0 : dw4::paged_attention_ws_bytes(p, num_seqs, num_heads, head_size);
  return DW4_OK;
}

int dw4_paged_attention(int num_seqs, int num_heads, int num_kv_heads, int head_size,
                        int block_size, const uint16_t* query, int64_t q_stride, uint16_t* out,
                        int64_t o_stride, const int64_t* key_block_ptrs,
                        const int64_t* value_block_ptrs, int kv_head_stride, float scale,
                        const int32_t* block_tables, int max_blocks_per_seq,
                        const int32_t* context_lens, int max_context_len,
                        const float* alibi_slopes, void* workspace, size_t workspace_bytes,
                        void* stream) {
  int st = check_attn_shape(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                            max_context_len);
  if (st != DW4_OK) return st;
  if (num_seqs == 0) return DW4_OK;
  if (!query || !out || !key_block_ptrs || !value_block_ptrs || !block_tables || !context_lens)
    return DW4_ERR_INVALID_ARG;
  const int64_t row = (int64_t)num_heads * head_size;
  if (q_stride < row || o_stride < row || kv_head_stride < block_size * head_size ||
      max_context_len < 1 || max_blocks_per_seq * block_size < max_context_len)
    return DW4_ERR_INVALID_ARG;
  if (!aligned16(query) || q_stride % 8 != 0) return DW4_ERR_MISALIGNED;
  const dw4::PagedAttnPlan p = dw4::plan_paged_attention(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                                                         max_context_len, cu_count());
  const size_t need = dw4::paged_attention_ws_bytes(p, num_seqs, num_heads, head_size);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return DW4_ERR_WORKSPACE;
  if (need > 0 && !aligned16(workspace)) return DW4_ERR_MISALIGNED;
  dw4::PagedAttnArgs a;
  a.num_seqs = num_seqs;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_size = head_size;
  a.block_size = block_size;
  a.query = query;
  a.q_stride = q_stride;
  a.out = out;
  a.o_stride = o_stride;
  a.kptr = key_block_ptrs;
  a.vptr = value_block_ptrs;
  a.kv_head_stride = kv_head_stride;
  a.scale = scale;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks_per_seq;
  a.context_lens = context_lens;
  a.alibi = alibi_slopes;
  return status_of(dw4::launch_paged_attention(a, p, static_cast<float*>(workspace),
                                               static_cast<hipStream_t>(stream)));
}

int dw4_rope(int batch_size, int rows_per_batch, int num_heads, int head_dim, uint16_t* x,
             const uint16_t* sin_table, const uint16_t* cos_table, int max_positions, int past_len,
             const int32_t* past_lens, void* stream) {
  if (batch_size < 0 || rows_per_batch < 0 || num_heads <= 0 || head_dim <= 0 || max_positions < 0)
    return DW4_ERR_INVALID_ARG;
  if (head_dim % 2 != 0 || rows_per_batch % num_heads != 0) return DW4_ERR_INVALID_ARG;
  if (batch_size == 0 || rows_per_batch == 0) return DW4_OK;
  if (!x || !sin_table || !cos_table || (past_len < 0 && !past_lens)) return DW4_ERR_INVALID_ARG;
  return status_of(dw4::launch_rope(x, sin_table, cos_table, batch_size, rows_per_batch, head_dim,
                                    num_heads, max_positions, past_len, past_lens,
                                    static_cast<hipStream_t>(stream)));
}

int dw4_rope_and_cache(int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                       int block_size, uint16_t* q, int64_t q_stride, uint16_t* k,
                       int64_t k_stride, const uint16_t* v, int64_t v_stride,
                       const uint16_t* sin_table, const uint16_t* cos_table, int max_positions,
                       const int32_t* positions, const int32_t* block_tables,
                       int max_blocks_per_seq, const int64_t* key_block_ptrs,
                       const int64_t* value_block_ptrs, int kv_head_stride,
                       int32_t* context_lens_out, void* stream) {
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_positions < 0 ||
      max_blocks_per_seq <= 0)
    return DW4_ERR_INVALID_ARG;
  if (head_dim % 8 != 0 || (block_size != 16 && block_size != 32)) return DW4_ERR_UNSUPPORTED;
  if (num_seqs == 0) return DW4_OK;
  if (!q || !k || !v || !sin_table || !cos_table || !positions || !block_tables ||
      !key_block_ptrs || !value_block_ptrs)
    return DW4_ERR_INVALID_ARG;
  if (q_stride < (int64_t)num_heads * head_dim || k_stride < (int64_t)num_kv_heads * head_dim ||
      v_stride < (int64_t)num_kv_heads * head_dim || kv_head_stride < block_size * head_dim)
    return DW4_ERR_INVALID_ARG;
  if (context_lens_out != nullptr && context_lens_out < positions + num_seqs &&
      positions < context_lens_out + num_seqs)
    return DW4_ERR_INVALID_ARG;  // workgroups of one sequence read positions[s] after another writes
  dw4::RopeCacheArgs a;
  a.num_seqs = num_seqs;
  a.heads = num_heads;
  a.kv_heads = num_kv_heads;
  a.hd = head_dim;
  a.bs = block_size;
  a.q = q;
  a.q_stride = q_stride;
  a.k = k;
  a.k_stride = k_stride;
  a.v = v;
  a.v_stride = v_stride;
  a.sinp = sin_table;
  a.cosp = cos_table;
  a.max_pos = max_positions;
  a.positions = positions;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks_per_seq;
  a.kptr = key_block_ptrs;
  a.vptr = value_block_ptrs;
  a.kv_head_stride = kv_head_stride;
  a.lens_out = context_lens_out;
  return status_of(dw4::launch_rope_cache(a, static_cast<hipStream_t>(stream)));
}

int dw4_gemm_t_workspace_size(int m, int k, int n, int group_size, size_t* workspace_bytes) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (m < 0 || workspace_bytes == nullptr) return DW4_ERR_INVALID_ARG;
  *workspace_bytes = m == 0 ? 0 : dw4::gemm_t_ws_bytes(dw4::plan_gemm_t(m, k, n, cu_count()), m, k);
  return DW4_OK;
}

int dw4_gemm_t(int m, int k, int n, int group_size, const uint16_t* g, int64_t ldg,
               const int32_t* packed_qweight, const int32_t* packed_zeros,
               const uint16_t* packed_scales, const int32_t* perm, uint16_t* out, int64_t ldo,
               void* workspace, size_t workspace_bytes, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (m < 0) return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  if (!g || !packed_qweight || !packed_zeros || !packed_scales || !out) return DW4_ERR_INVALID_ARG;
  if (ldg < n || ldo < k) return DW4_ERR_INVALID_ARG;
  if (!aligned16(g) || (ldg % 8) != 0 || !aligned16(packed_qweight)) return DW4_ERR_MISALIGNED;
  const dw4::GemmTPlan plan = dw4::plan_gemm_t(m, k, n, cu_count());
  float* part = nullptr;
  if (plan.ns > 1) {
    if (workspace == nullptr || workspace_bytes < dw4::gemm_t_ws_bytes(plan, m, k))
      return DW4_ERR_WORKSPACE;
    if (!aligned16(workspace)) return DW4_ERR_MISALIGNED;
    part = static_cast<float*>(workspace);
  }
  dw4::GemmTArgs a;
  a.M = m;
  a.K = k;
  a.N = n;
  a.gs = group_size;
  a.G = k / group_size;
  a.g = g;
  a.ldg = ldg;
  a.pq = reinterpret_cast<const uint32_t*>(packed_qweight);
  a.pz = reinterpret_cast<const uint32_t*>(packed_zeros);
  a.ps = packed_scales;
  a.perm = perm;
  a.out = out;
  a.ldo = ldo;
  return status_of(dw4::launch_gemm_t(a, plan, part, static_cast<hipStream_t>(stream)));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Decoder-stage calls
// ---------------------------------------------------------------------------
namespace {

int check_item(const dw4_item* it) {
  if (it == nullptr) return DW4_ERR_INVALID_ARG;
  const int st = check_shape(it->k, it->n, it->group_size);
  if (st != DW4_OK) return st;
  if (!it->packed_qweight || !it->packed_zeros || !it->packed_scales) return DW4_ERR_INVALID_ARG;
  if (!aligned16(it->packed_qweight)) return DW4_ERR_MISALIGNED;
  return DW4_OK;
}

int check_output(const dw4_item* it) {
  if (it->y == nullptr || it->ldy < it->n) return DW4_ERR_INVALID_ARG;
  return DW4_OK;
}

int check_x(const uint16_t* x, int64_t ldx, int k) {
  if (x == nullptr || ldx < k) return DW4_ERR_INVALID_ARG;
  if (!aligned16(x) || (ldx % 8) != 0) return DW4_ERR_MISALIGNED;
  return DW4_OK;
}

dw4::GemmArgs args_of(int m, const uint16_t* x, int64_t ldx, const dw4_item* it) {
  dw4::GemmArgs a;
  a.M = m;
  a.K = it->k;
  a.N = it->n;
  a.gs = it->group_size;
  a.G = it->k / it->group_size;
  a.x = x;
  a.ldx = ldx;
  a.pq = reinterpret_cast<const uint32_t*>(it->packed_qweight);
  a.pz = reinterpret_cast<const uint32_t*>(it->packed_zeros);
  a.ps = it->packed_scales;
  a.perm = it->perm;
  a.bias = it->bias;
  a.y = it->y;
  a.ldy = it->ldy;
  return a;
}

int gemm_item(int m, const uint16_t* x, int64_t ldx, const dw4_item* it, void* ws, size_t wsb,
              void* stream, const uint16_t* res = nullptr, int64_t ldres = 0) {
  return gemm_run(DW4_PATH_AUTO, 0, m, it->k, it->n, it->group_size, x, ldx, it->packed_qweight,
                  it->packed_zeros, it->packed_scales, it->perm, it->bias, it->y, it->ldy, res,
                  ldres, ws, wsb, stream);
}

// Whether the fp16 [m, n] views a (row stride lda) and b (ldb) share bytes.
bool overlap(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int m, int n) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  const uintptr_t a1 = a0 + ((size_t)(m - 1) * lda + n) * sizeof(uint16_t);
  const uintptr_t b1 = b0 + ((size_t)(m - 1) * ldb + n) * sizeof(uint16_t);
  return a0 < b1 && b0 < a1;
}


int check_pair(const dw4_item* gate, const dw4_item* up) {
  int st = check_item(gate);
  if (st == DW4_OK) st = check_item(up);
  if (st != DW4_OK) return st;
  if (gate->k != up->k || gate->n != up->n || gate->group_size != up->group_size ||
      (gate->perm == nullptr) != (up->perm == nullptr))
    return DW4_ERR_INVALID_ARG;
  return DW4_OK;
}

}  // namespace

extern "C" {

int dw4_gemm_group(int count, const dw4_item* items, int m, const uint16_t* x, int64_t ldx,
                   void* workspace, size_t workspace_bytes, void* stream) {
  if (count < 1 || count > dw4::kGroupMax || items == nullptr || m < 0) return DW4_ERR_INVALID_ARG;
  int n_total = 0;
  for (int i = 0; i < count; ++i) {
    int st = check_item(&items[i]);
    if (st == DW4_OK) st = check_output(&items[i]);
    if (st != DW4_OK) return st;
    if (items[i].k != items[0].k || items[i].group_size != items[0].group_size ||
        (items[i].perm == nullptr) != (items[0].perm == nullptr))
      return DW4_ERR_INVALID_ARG;
    n_total += items[i].n;
  }
  if (m == 0) return DW4_OK;
  const int st = check_x(x, ldx, items[0].k);
  if (st != DW4_OK) return st;
  const int cus = cu_count();
  if (m <= dw4::kGroupDecodeMaxM && rows_fit_i32(m, ldx, items[0].k) &&
      dw4::auto_decode(m, n_total, cus)) {
    const dw4::DecodePlan plan =
        dw4::plan_decode(m, items[0].k, n_total, items[0].group_size, cus, false);
    if (plan.splits == 1) {
      dw4::GroupArgs g{};
      g.count = count;
      for (int i = 0; i < count; ++i) g.a[i] = args_of(m, x, ldx, &items[i]);
      return status_of(dw4::launch_decode_group(g, plan, static_cast<hipStream_t>(stream)));
    }
  }
  // above 128 rows, matrices of equal N without act-order: one launch of the
  // LDS-streamed prefill kernel, planned as one matrix of the summed N
  // (so the tiles fill the CUs as a merged matrix's would), when that plan
  // needs no K split
  bool same_n = items[0].perm == nullptr;
  for (int i = 1; i < count; ++i) same_n = same_n && items[i].n == items[0].n;
  if (m > 128 && same_n && count > 1) {
    const dw4::PrefillPlan plan = plan_prefill(m, items[0].k, n_total, 0, 0, false);
    if (plan.splits == 1) {
      dw4::GroupArgs g{};
      g.count = count;
      for (int i = 0; i < count; ++i) g.a[i] = args_of(m, x, ldx, &items[i]);
      return status_of(dw4::launch_prefill2_group(g, plan, workspace, static_cast<hipStream_t>(stream)));
    }
  }
  for (int i = 0; i < count; ++i) {
    const int r = gemm_item(m, x, ldx, &items[i], workspace, workspace_bytes, stream);
    if (r != DW4_OK) return r;
  }
  return DW4_OK;
}

int dw4_gemm_silu_mul(int m, const uint16_t* x, int64_t ldx, const dw4_item* gate,
                      const dw4_item* up, uint16_t* h, int64_t ldh, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int st = check_item(gate);
  if (st == DW4_OK) st = check_item(up);
  if (st != DW4_OK) return st;
  if (m < 0 || gate->k != up->k || gate->n != up->n || gate->group_size != up->group_size ||
      (gate->perm == nullptr) != (up->perm == nullptr))
    return DW4_ERR_INVALID_ARG;
  if (h == nullptr || ldh < gate->n) return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  st = check_x(x, ldx, gate->k);
  if (st != DW4_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (m <= dw4::kPairMaxM && gate->perm == up->perm && rows_fit_i32(m, ldx, gate->k) &&
      dw4::auto_decode(m, 2 * gate->n, cu_count())) {
    dw4::GroupArgs g{};
    g.count = 2;
    g.a[0] = args_of(m, x, ldx, gate);
    g.a[1] = args_of(m, x, ldx, up);
    return status_of(dw4::launch_decode_pair(g, h, ldh, s));
  }
  st = check_output(gate);
  if (st == DW4_OK) st = check_output(up);
  if (st != DW4_OK) return st;
  st = gemm_item(m, x, ldx, gate, workspace, workspace_bytes, stream);
  if (st == DW4_OK) st = gemm_item(m, x, ldx, up, workspace, workspace_bytes, stream);
  if (st != DW4_OK) return st;
  return status_of(dw4::launch_silu_mul(gate->y, gate->ldy, up->y, up->ldy, h, ldh, m, gate->n, s));
}

int dw4_rms_norm(int m, int k, const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                 uint16_t* y, int64_t ldy, void* stream) {
  if (m < 0 || k <= 0 || !x || !w || !y || ldx < k || ldy < k || !(eps >= 0.0f))
    return DW4_ERR_INVALID_ARG;
  if (k % 8 != 0) return DW4_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || ldx % 8 != 0 || ldy % 8 != 0)
    return DW4_ERR_MISALIGNED;
  if (m == 0) return DW4_OK;
  return status_of(dw4::launch_rms_norm(x, ldx, w, eps, y, ldy, m, k, static_cast<hipStream_t>(stream)));
}

int dw4_attention_qkv_stage(int m, const uint16_t* x, int64_t ldx, const uint16_t* norm_w,
                            float eps, uint16_t* rms, int64_t ldr, const dw4_item* q,
                            const dw4_item* k, const dw4_item* v, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr) return DW4_ERR_INVALID_ARG;
  const dw4_item items[3] = {*q, *k, *v};
  int st = dw4_rms_norm(m, q->k, x, ldx, norm_w, eps, rms, ldr, stream);
  if (st != DW4_OK) return st;
  return dw4_gemm_group(3, items, m, rms, ldr, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// dw4_mlp_forward; res (if not NULL, not overlapping down->y) is added to
// the down product in its epilogue.
int mlp_run(int m, const uint16_t* x, int64_t ldx, const uint16_t* norm_w, float eps,
            uint16_t* rms, int64_t ldr, const dw4_item* gate, const dw4_item* up,
            const dw4_item* down, const uint16_t* res, int64_t ldres, void* workspace,
            size_t workspace_bytes, void* stream) {
  if (gate == nullptr || up == nullptr || down == nullptr) return DW4_ERR_INVALID_ARG;
  int st = check_item(down);
  if (st == DW4_OK) st = check_output(down);
  if (st == DW4_OK) st = check_output(gate);
  if (st != DW4_OK) return st;
  if (down->k != gate->n) return DW4_ERR_INVALID_ARG;
  st = dw4_rms_norm(m, gate->k, x, ldx, norm_w, eps, rms, ldr, stream);
  if (st == DW4_OK)
    st = dw4_gemm_silu_mul(m, rms, ldr, gate, up, gate->y, gate->ldy, workspace, workspace_bytes,
                           stream);
  if (st != DW4_OK) return st;
  return gemm_item(m, gate->y, gate->ldy, down, workspace, workspace_bytes, stream, res, ldres);
}

}  // namespace

extern "C" {

int dw4_mlp_forward(int m, const uint16_t* x, int64_t ldx, const uint16_t* norm_w, float eps,
                    uint16_t* rms, int64_t ldr, const dw4_item* gate, const dw4_item* up,
                    const dw4_item* down, void* workspace, size_t workspace_bytes, void* stream) {
  return mlp_run(m, x, ldx, norm_w, eps, rms, ldr, gate, up, down, nullptr, 0, workspace,
                 workspace_bytes, stream);
}

int dw4_decoder_after_stage(int m, const uint16_t* attn, int64_t lda, const uint16_t* residual,
                            int64_t ldres, const dw4_item* o, const uint16_t* norm_w, float eps,
                            uint16_t* rms, int64_t ldr, const dw4_item* gate, const dw4_item* up,
                            const dw4_item* down, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (o == nullptr || gate == nullptr || up == nullptr || down == nullptr || residual == nullptr)
    return DW4_ERR_INVALID_ARG;
  int st = check_item(o);
  if (st == DW4_OK) st = check_output(o);
  if (st == DW4_OK) st = check_item(down);
  if (st == DW4_OK) st = check_output(down);
  if (st == DW4_OK) st = check_output(gate);
  if (st == DW4_OK) st = check_pair(gate, up);
  if (st != DW4_OK) return st;
  if (ldres < o->n || o->n != gate->k || down->n != o->n || down->k != gate->n || m < 0)
    return DW4_ERR_INVALID_ARG;
  if (!(eps >= 0.0f) || norm_w == nullptr || rms == nullptr) return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  // x2 (o->y) is read while down's product is written
  if (overlap(o->y, o->ldy, down->y, down->ldy, m, o->n)) return DW4_ERR_INVALID_ARG;
  st = check_x(attn, lda, o->k);
  if (st != DW4_OK) return st;
  // o_proj + residual, mlp_forward + residual (real_fuse.py:80-103), the
  // residual adds in the GEMM epilogues.  Each output element is read from
  // the residual and written by the same thread, so o->y may be the
  // residual itself; a partial overlap is rejected.
  const bool same = residual == o->y && ldres == o->ldy;
  if (!same && overlap(residual, ldres, o->y, o->ldy, m, o->n)) return DW4_ERR_INVALID_ARG;
  st = gemm_item(m, attn, lda, o, workspace, workspace_bytes, stream, residual, ldres);
  if (st != DW4_OK) return st;
  return mlp_run(m, o->y, o->ldy, norm_w, eps, rms, ldr, gate, up, down, o->y, o->ldy, workspace,
                 workspace_bytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// dw4_gemm_noalloc: dw4_gemm on a file-scope scratch array instead of a
// caller workspace.  The array's name is a host-side stand-in; kernels get the
// device address from hipGetSymbolAddress, looked up once per device.
// ---------------------------------------------------------------------------
namespace {

static __device__ __align__(256) unsigned char scratch[DW4_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mutex;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

__global__ void clear_words_kernel(uint32_t* __restrict__ p, int words) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < words) p[i] = 0u;
}

// The current device's scratch address (null on failure, with *status set).
// The first call on a device also clears the arrival-counter head with a fill
// kernel on `stream` (no memset node, so a capturing caller's graph stays
// free of them); every later call leaves the head at zero.
void* scratch_for_current_device(hipStream_t stream, int* status) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *status = DW4_ERR_DEVICE;
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) {
    *status = DW4_ERR_DEVICE;
    return nullptr;
  }
  constexpr int words = (int)(dw4::kWsHeadBytes / sizeof(uint32_t));
  clear_words_kernel<<<(words + 255) / 256, 256, 0, stream>>>(static_cast<uint32_t*>(addr), words);
  if (hipGetLastError() != hipSuccess) {
    *status = DW4_ERR_LAUNCH;
    return nullptr;
  }
  g_scratch_ptr[dev].store(addr, std::memory_order_release);
  return addr;
}

}  // namespace

extern "C" int dw4_gemm_noalloc(int m, int k, int n, int group_size, const uint16_t* x,
                                int64_t ldx, const int32_t* packed_qweight,
                                const int32_t* packed_zeros, const uint16_t* packed_scales,
                                const int32_t* perm, const uint16_t* bias, uint16_t* y,
                                int64_t ldy, void* stream) {
  const int st = check_shape(k, n, group_size);
  if (st != DW4_OK) return st;
  if (m < 0) return DW4_ERR_INVALID_ARG;
  if (m == 0) return DW4_OK;
  const size_t need = workspace_for(DW4_PATH_AUTO, m, k, n, group_size, perm != nullptr);
  if (need > DW4_NOALLOC_SCRATCH_BYTES) return DW4_ERR_SCRATCH;
  int status = DW4_OK;
  void* ws = scratch_for_current_device(static_cast<hipStream_t>(stream), &status);
  if (ws == nullptr) return status;
  return gemm_run(DW4_PATH_AUTO, 0, m, k, n, group_size, x, ldx, packed_qweight, packed_zeros,
                  packed_scales, perm, bias, y, ldy, nullptr, 0, ws, DW4_NOALLOC_SCRATCH_BYTES,
                  stream);
}

// ---------------------------------------------------------------------------
// Decode chain
// ---------------------------------------------------------------------------
namespace {

struct Span {
  uintptr_t lo = 0, hi = 0;  // [lo, hi) bytes; empty when lo == hi
  bool hits(const Span& o) const { return lo < o.hi && o.lo < hi; }
};

Span span_of(const void* p, int m, int64_t ld, int cols) {
  Span r;
  if (p == nullptr || m <= 0) return r;
  r.lo = reinterpret_cast<uintptr_t>(p);
  r.hi = r.lo + ((size_t)(m - 1) * (size_t)ld + (size_t)cols) * sizeof(uint16_t);
  return r;
}

int check_chain_link(const dw4_chain_link& l, int i, int m) {
  int st = check_shape(l.k, l.n, l.group_size);
  if (st != DW4_OK) return st;
  if (l.group_size % kChunkK != 0 || l.perm != nullptr || l.k > dw4::kChainMaxK ||
      l.n > 32768)
    return DW4_ERR_UNSUPPORTED;
  if (!l.x || !l.packed_qweight || !l.packed_zeros || !l.packed_scales || !l.y)
    return DW4_ERR_INVALID_ARG;
  if (l.ldx < l.k || l.ldy < l.n || (l.residual && l.ldres < l.n)) return DW4_ERR_INVALID_ARG;
  if (l.after < -1 || l.after >= i) return DW4_ERR_INVALID_ARG;
  if (!aligned16(l.x) || l.ldx % 8 != 0 || !aligned16(l.packed_qweight)) return DW4_ERR_MISALIGNED;
  // the activation rows are read through one buffer resource (32-bit offsets)
  if ((int64_t)(m - 1) * l.ldx * 2 + (int64_t)l.k * 2 > (int64_t)INT32_MAX)
    return DW4_ERR_UNSUPPORTED;
  return DW4_OK;
}

}  // namespace

extern "C" {

int dw4_chain_buffer_size(int count, size_t* bytes) {
  if (count < 1 || count > (1 << 16) || bytes == nullptr) return DW4_ERR_INVALID_ARG;
  *bytes = dw4::chain_buffer_bytes(count);
  return DW4_OK;
}

int dw4_chain_prepare(int count, const dw4_chain_link* links, int m, void* chain,
                      size_t chain_bytes, dw4_chain_plan* plan) {
  if (count < 1 || count > (1 << 16) || links == nullptr || plan == nullptr)
    return DW4_ERR_INVALID_ARG;
  if (m < 1 || m > dw4::kChainMaxM) return DW4_ERR_UNSUPPORTED;
  for (int i = 0; i < count; ++i) {
    const int st = check_chain_link(links[i], i, m);
    if (st != DW4_OK) return st;
  }
  // Every pair of links that share a buffer with at least one of them
  // writing it must be ordered by `after`; within a link the output must not
  // overlap its activations or bias, and the residual is the output itself
  // (same stride) or elsewhere.
  std::vector<Span> w(count), xr(count), rr(count), br(count);
  for (int i = 0; i < count; ++i) {
    const dw4_chain_link& l = links[i];
    w[i] = span_of(l.y, m, l.ldy, l.n);
    xr[i] = span_of(l.x, m, l.ldx, l.k);
    rr[i] = span_of(l.residual, m, l.ldres, l.n);
    br[i] = span_of(l.bias, 1, l.n, l.n);
    if (w[i].hits(xr[i]) || w[i].hits(br[i])) return DW4_ERR_INVALID_ARG;
    if (w[i].hits(rr[i]) && !(l.residual == l.y && l.ldres == l.ldy)) return DW4_ERR_INVALID_ARG;
  }
  for (int b = 1; b < count; ++b)
    for (int a = 0; a < b; ++a) {
      const bool conflict = w[a].hits(w[b]) || w[a].hits(xr[b]) || w[a].hits(rr[b]) ||
                            w[a].hits(br[b]) || w[b].hits(xr[a]) || w[b].hits(rr[a]) ||
                            w[b].hits(br[a]);
      if (conflict && links[b].after < a) return DW4_ERR_INVALID_ARG;
    }
  size_t need = dw4::chain_buffer_bytes(count);
  if (chain == nullptr || chain_bytes < need) return DW4_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(chain) & 255u) != 0) return DW4_ERR_MISALIGNED;

  dw4::ChainPlan p{};
  p.count = count;
  p.m = m;
  p.workgroups = std::min(cu_count(), dw4::kChainMaxWorkgroups);
  p.max_k = 0;
  p.max_strips = 1;
  p.max_groups = 1;
  for (int i = 0; i < count; ++i) {
    p.max_k = std::max(p.max_k, links[i].k);
    p.max_groups = std::max(p.max_groups, links[i].k / links[i].group_size);
    const int strips = links[i].n / kStripN;
    p.max_strips = std::max(p.max_strips, (strips + p.workgroups - 1) / p.workgroups);
    // the kernel deals strips to workgroups with floor(r * strips / W) by a
    // multiplier, exact while r * strips * W < 2^32 (r <= W)
    if ((uint64_t)p.workgroups * p.workgroups * (uint64_t)strips >= (1ull << 32))
      return DW4_ERR_UNSUPPORTED;
  }
  if (!dw4::plan_chain(p)) return DW4_ERR_UNSUPPORTED;

  std::vector<unsigned char> host(need, 0);
  dw4::ChainHeader* hdr = reinterpret_cast<dw4::ChainHeader*>(host.data());
  hdr->count = count;
  hdr->M = m;
  hdr->workgroups = p.workgroups;
  int64_t strips_before = 0;
  for (int i = 0; i < count; ++i) {
    const dw4_chain_link& l = links[i];
    dw4::ChainLinkDev d{};
    d.pq = reinterpret_cast<const uint32_t*>(l.packed_qweight);
    d.pz = reinterpret_cast<const uint32_t*>(l.packed_zeros);
    d.ps32 = reinterpret_cast<const uint32_t*>(l.packed_scales);
    d.x = l.x;
    d.bias = l.bias;
    d.res = l.residual;
    d.y = l.y;
    d.ldx = l.ldx;
    d.ldres = l.ldres;
    d.ldy = l.ldy;
    d.K = l.k;
    d.N = l.n;
    d.G = l.k / l.group_size;
    const int cpg = l.group_size / kChunkK;  // chunks per group
    d.gmag = cpg <= 1 ? 0u : (uint32_t)(((1ull << 32) + (uint64_t)cpg - 1) / (uint64_t)cpg);
    const int kc = l.k / kChunkK;
    d.kcmag = kc <= 1 ? 0u : (uint32_t)(((1ull << 32) + (uint64_t)kc - 1) / (uint64_t)kc);
    d.after = l.after;
    d.flags = 0;
    if (i > 0) {
      const dw4_chain_link& q = links[i - 1];
      if (q.x == l.x && q.ldx == l.ldx && q.k == l.k && q.after == l.after)
        d.flags |= dw4::kChainSameX;
    }
    // a link's progress is published only when a later link waits for it
    // (waiting for link a means links 0..a are complete: the latest
    // published link at or before a carries that)
    for (int b = i + 1; b < count; ++b)
      if (links[b].after == i) d.flags |= dw4::kChainPublish;
    d.rot = (int)(strips_before % p.workgroups);
    strips_before += l.n / kStripN;
    std::memcpy(host.data() + dw4::kChainHeadBytes + (size_t)i * dw4::kChainLinkBytes, &d,
                sizeof(d));
  }
  if (hipMemcpy(chain, host.data(), need, hipMemcpyHostToDevice) != hipSuccess)
    return DW4_ERR_DEVICE;
  plan->count = p.count;
  plan->m = p.m;
  plan->workgroups = p.workgroups;
  plan->waves = p.waves;
  plan->ring = p.ring;
  plan->max_k = p.max_k;
  plan->max_strips = p.max_strips;
  plan->max_groups = p.max_groups;
  plan->smem_bytes = p.smem;
  return DW4_OK;
}

int dw4_gemm_chain(const dw4_chain_plan* plan, void* chain, void* stream) {
  if (plan == nullptr || chain == nullptr || plan->count < 1 || plan->m < 1 ||
      plan->m > dw4::kChainMaxM || plan->workgroups < 1 ||
      plan->workgroups > dw4::kChainMaxWorkgroups)
    return DW4_ERR_INVALID_ARG;
  dw4::ChainPlan p{};
  p.count = plan->count;
  p.m = plan->m;
  p.workgroups = plan->workgroups;
  p.max_k = plan->max_k;
  p.max_strips = plan->max_strips;
  p.max_groups = plan->max_groups;
  if (!dw4::plan_chain(p) || p.ring != plan->ring || p.smem != plan->smem_bytes)
    return DW4_ERR_INVALID_ARG;  // not a plan dw4_chain_prepare wrote
  return status_of(dw4::launch_chain(p, chain, static_cast<hipStream_t>(stream)));
}

int dw4_chain_timed_out(const void* chain, int* timed_out) {
  if (chain == nullptr || timed_out == nullptr) return DW4_ERR_INVALID_ARG;
  dw4::ChainHeader h{};
  if (hipMemcpy(&h, chain, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return DW4_ERR_DEVICE;
  *timed_out = h.timed_out != 0;
  return DW4_OK;
}

}  // extern "C"
