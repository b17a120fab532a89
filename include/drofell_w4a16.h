/*
 * drofell_w4a16.h -- C ABI of the MI355X (gfx950) GPTQ int4-weight /
 * fp16-activation quantized-Linear library (libdrofell_w4a16.so).
 *
 * Reference interfaces replaced (paths relative to
 * /root/reference/After-Revision-DROFELL):
 *   dw4_make_perm    host half of make_sequential
 *                    (cuda_extends/exllama/q4_matrix.cu:125-159) and the
 *                    argsort in MarlinQ4Matrix (cuda_extends/marlin.py:218-220)
 *   dw4_repack       make_q4 (cuda_extends/exllama/entry.cpp:18-62 ->
 *                    q4_matrix.cu:33-76 shuffle/make_sequential) and
 *                    gptq_marlin_repack (cuda_extends/vllm/ops_registration.cpp:40-42)
 *   dw4_gemm         q4_matmul_cuda_v2 (entry.cpp:221-251) and
 *                    q4_matmul_blas_v2 (entry.cpp:303-340), marlin_gemm
 *                    (ops_registration.cpp:43-49); the M-based dispatch of
 *                    Q4MatrixV2.matmul (cuda_extends/exllama.py:492-526)
 *   dw4_gemm_bf16    q4_matmul_blas_v2 with bfloat16 (entry.cpp:303-340: a
 *                    bf16 reconstruction, then a bf16 GEMM), the route of
 *                    Q4MatrixV2.matmul for bf16 x (cuda_extends/exllama.py:492-526),
 *                    for 1 <= M <= DW4_BF16_MAX_M
 *   dw4_dequant      q4_to_half_matrix_v2 (entry.cpp:79-91) and
 *                    marlin_dequant_into (cuda_extends/marlin/marlin_dequant.cu:97-172)
 *   dw4_reshape_and_cache / dw4_restore_from_cache / dw4_paged_attention
 *                    reshape_and_cache, restore_from_cache
 *                    (cuda_extends/vllm/cache_kernels.cu:242-420) and
 *                    paged_attention_v1 / v2
 *                    (cuda_extends/vllm/attention/attention_kernels.cu:1602-1843)
 *                    as operators/core/attention/real_page.py:23-189 and
 *                    operators/core/block/real.py:66-106 call them
 *   dw4_rope         rope_cuda (cuda_extends/exllama/fuse_v2/rope.cu:24-135), the
 *                    RoPE half of attention_forward_rope_stage_v2
 *   dw4_gemm_t       q4_transpose_matmul_blas_v2 (entry.cpp:392-429 ->
 *                    exllama/q4_transpose_matmul.cu:115-167), the PEFT backward
 *                    of Q4MatrixV2.transpose_matmul (exllama.py:528-544)
 *   dw4_gemm_group   the q/k/v GEMMs of attention_forward_qkv_stage
 *                    (cuda_extends/exllama/fuse_v2/q_attn.cu:46-48) and the
 *                    gate/up GEMMs of mlp_forward (fuse_v2/q_mlp.cu:119-120)
 *   dw4_gemm_silu_mul  gate/up GEMMs + silu_mul_kernel of mlp_forward
 *                    (fuse_v2/q_mlp.cu:119-130, silu_mul_kernel :44-85)
 *   dw4_rms_norm     rms_norm_cuda (fuse_v2/rms_norm.cu:26-93, 109-131)
 *   dw4_attention_qkv_stage  attention_forward_qkv_stage_v2
 *                    (entry.cpp:483-532 -> fuse_v2/q_attn.cu:23-54)
 *   dw4_mlp_forward  mlp_forward_v2 (entry.cpp:431-481 -> fuse_v2/q_mlp.cu:96-133)
 *   dw4_decoder_after_stage  the o_proj, residual add, mlp_forward_v2 and
 *                    residual add of DecoderWrapFuse._fuse_forward_after_stage
 *                    (operators/core/decoder_wrap/real_fuse.py:77-103)
 *
 * Conventions
 *   - Every function returns an int status (DW4_OK == 0); no exception or
 *     abort crosses the ABI.  dw4_strerror() names a status.
 *   - Every buffer is owned by the caller.  The library allocates nothing
 *     on the device (beyond dw4_gemm_noalloc's fixed scratch array, which
 *     the code object carries), keeps no pointer after a call returns and
 *     holds no global mutable state except per-device records: the CU
 *     count, per kernel whether its dynamic LDS limit has been raised on
 *     that device, and the address of that device's scratch array.
 *   - Device pointers refer to memory of the current HIP device; `stream`
 *     is a hipStream_t (NULL = the null stream).  Work is enqueued on it.
 *   - dw4_gemm never synchronises, never allocates and launches a fixed
 *     sequence of kernels for a given (m, k, n, workspace) so it may be
 *     captured into a HIP graph.  Its result is deterministic: split-K
 *     partial sums are always added in split order, whatever order the
 *     workgroups finish in.
 *   - dw4_make_perm runs on the host; dw4_repack may be called once per
 *     load or swap-in and does not synchronise either.
 *   - The dw4_gemm workspace must be zero-filled before its first use; the
 *     library keeps split-K arrival counters at its start and leaves them at
 *     zero after every call.  Calls that overlap in time on one workspace
 *     race (give concurrent streams their own workspace).
 *
 * Shapes (GPTQ checkpoint format, the module buffers of QuantLinear,
 * operators/core/linear/real_quant.py:10-49 in the reference):
 *   qweight int32 [K/8, N]   row k of column n at bits 4*(k%8) of word [k/8][n]
 *   qzeros  int32 [G, N/8]   stored zero of column n at bits 4*(n%8); the
 *                            effective zero is stored + 1
 *   scales  fp16  [G, N]
 *   g_idx   int32 [K]        group of each row (act-order only)
 *   x fp16 [M, K] (row stride ldx), y fp16 [M, N] (row stride ldy)
 *   G = K / group_size.
 * Supported: K % 128 == 0, N % 16 == 0, group_size in {32, 64} or a
 * multiple of 128 (group_size == K included), K % group_size == 0;
 * act-order requires every group to hold exactly group_size rows (what GPTQ
 * desc_act produces).
 *
 * Packed layout written by dw4_repack (same byte counts as the inputs, so
 * a module keeps its buffer sizes):
 *   packed_qweight  K*N/2 bytes.  Strip s = 16 columns, chunk c = 128
 *                   (sorted) rows; chunk (s, c) is 1024 contiguous bytes at
 *                   (s*K/128 + c)*1024.  Lane L in [0,64), word w in [0,4)
 *                   at byte L*16 + w*4 holds column 16*s + L%16, rows
 *                   128*c + 32*w + 8*(L/16) + e, e in [0,8); even e at bits
 *                   4*(e/2), odd e at bits 16 + 4*(e/2).
 *   packed_scales   fp16, element (s, g, j) at (s*G + g)*16 + j.
 *   packed_zeros    int32, word (s, g, h) at (s*G + g)*2 + h = qzeros[g][2s+h].
 *   perm            int32 [K] sorted row -> original row (act-order only).
 */
#ifndef DROFELL_W4A16_H
#define DROFELL_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DW4_ABI_VERSION 11

enum {
  DW4_OK = 0,
  DW4_ERR_INVALID_ARG = 1,   /* null pointer, non-positive size, bad stride */
  DW4_ERR_UNSUPPORTED = 2,   /* shape/group size outside the supported set */
  DW4_ERR_MISALIGNED = 3,    /* pointer or stride not 16-byte aligned */
  DW4_ERR_BAD_GIDX = 4,      /* g_idx out of range or groups not uniform */
  DW4_ERR_WORKSPACE = 5,     /* workspace smaller than dw4_workspace_size() */
  DW4_ERR_LAUNCH = 6,        /* a kernel launch failed (hipGetLastError) */
  DW4_ERR_DEVICE = 7,        /* no usable HIP device / runtime error */
  DW4_ERR_SCRATCH = 8        /* dw4_gemm_noalloc: the call needs more than its fixed scratch */
};

/* Path selection for dw4_gemm_path(). */
enum {
  DW4_PATH_AUTO = 0,     /* decode for M <= 48, or M <= 64 when N / 16 <= CUs (or
                            <= 1.25 CUs with K <= 8192) */
  DW4_PATH_DECODE = 1,   /* register-dequant MFMA kernel, M <= 64 */
  DW4_PATH_PREFILL = 2   /* LDS-staged MFMA kernel, any M */
};

int dw4_abi_version(void);
const char* dw4_strerror(int status);

/* Byte sizes of the repacked buffers and the dw4_gemm workspace needed for
 * any M <= max_m.  Any output pointer may be NULL. */
int dw4_query_sizes(int k, int n, int group_size, int act_order, int max_m,
                    size_t* packed_qweight_bytes, size_t* packed_scales_bytes,
                    size_t* packed_zeros_bytes, size_t* perm_bytes,
                    size_t* workspace_bytes);

/* Workspace bytes one dw4_gemm call at exactly this M needs (0 allowed when
 * it returns 0).  With act_order it includes M*K fp16 for x gathered into
 * the packed row order (placed after the split-K area and the arrival
 * counters); a call whose workspace lacks that room gathers inside every
 * workgroup instead: the same result bit for bit, slower.  (At M = 1 with
 * K <= 16384 the decode kernel gathers from an LDS copy of x and uses none
 * of the act-order room.)  For 5 <= M <= 64
 * the decode kernel may split K over workgroups (fp32 planes in the
 * workspace); given less than this size it runs unsplit instead (a valid
 * result, summed in another order). */
int dw4_workspace_size(int m, int k, int n, int group_size, int act_order,
                       size_t* workspace_bytes);

/* Host: stable counting sort of rows by group (perm[new] = old) and its
 * validation.  g_idx_host, perm_host: int32 [k] host arrays. */
int dw4_make_perm(int k, int group_size, const int32_t* g_idx_host,
                  int32_t* perm_host);

/* Device: GPTQ buffers -> packed layout.  perm (device int32 [k]) is NULL
 * for checkpoints without act-order.  Outputs must not alias inputs. */
int dw4_repack(int k, int n, int group_size,
               const int32_t* qweight, const int32_t* qzeros,
               const uint16_t* scales, const int32_t* perm,
               int32_t* packed_qweight, int32_t* packed_zeros,
               uint16_t* packed_scales, void* stream);

/* Device: y[M, N] = x[M, K] @ W (+ bias[N] in fp16), fp32 accumulation,
 * fp16 output (round to nearest even).  perm as in dw4_repack; bias may be
 * NULL.  x and y must be 16-byte aligned with ldx % 8 == 0. */
int dw4_gemm(int m, int k, int n, int group_size,
             const uint16_t* x, int64_t ldx,
             const int32_t* packed_qweight, const int32_t* packed_zeros,
             const uint16_t* packed_scales, const int32_t* perm,
             const uint16_t* bias, uint16_t* y, int64_t ldy,
             void* workspace, size_t workspace_bytes, void* stream);

/* Device: y[M, N] = bf16(x[M, K] @ W) (+ bias[N] in bf16, added after that
 * rounding) for bf16 activations x and a bf16 output y, 1 <= m <=
 * DW4_BF16_MAX_M; larger m returns DW4_ERR_UNSUPPORTED (the caller keeps
 * the dense route: dw4_dequant_bf16, then a bf16 library GEMM).  One
 * register-fed decode launch on bf16 matrix cores (every row tile of 16 rows
 * in the same launch, the packed weights read once), fp32 accumulation over
 * the exact integers q - z and the fp16 scales applied per group in fp32, so
 * the product is within rounding of the dense route's (whose weight is
 * rounded to bf16 first).  Same buffers, alignment and perm as dw4_gemm;
 * act-order calls use the workspace of dw4_workspace_size(m, ...) for x
 * gathered into the packed row order when it has room (otherwise every
 * workgroup gathers, same result); no K split. */
#define DW4_BF16_MAX_M 64
int dw4_gemm_bf16(int m, int k, int n, int group_size,
                  const uint16_t* x, int64_t ldx,
                  const int32_t* packed_qweight, const int32_t* packed_zeros,
                  const uint16_t* packed_scales, const int32_t* perm,
                  const uint16_t* bias, uint16_t* y, int64_t ldy,
                  void* workspace, size_t workspace_bytes, void* stream);

/* dw4_gemm with an explicit path (DW4_PATH_*) and prefill split-K factor
 * (0 = automatic); for tests and benchmarks. */
int dw4_gemm_path(int path, int split_k, int m, int k, int n, int group_size,
                  const uint16_t* x, int64_t ldx,
                  const int32_t* packed_qweight, const int32_t* packed_zeros,
                  const uint16_t* packed_scales, const int32_t* perm,
                  const uint16_t* bias, uint16_t* y, int64_t ldy,
                  void* workspace, size_t workspace_bytes, void* stream);

/* dw4_gemm for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same arguments and results as dw4_gemm without the
 * workspace: the split-K partials, arrival counters and gathered act-order
 * activations live in one file-scope device array of
 * DW4_NOALLOC_SCRATCH_BYTES per GPU (held from the library's first use on
 * that GPU until the process ends).  A call whose dw4_workspace_size exceeds
 * that returns DW4_ERR_SCRATCH before launching anything.  Every call on a
 * GPU shares that GPU's array, so calls that overlap in time on one GPU
 * (concurrent streams or threads) race; serialise them.  Calls no hipMalloc,
 * hipFree or allocating library routine.  The first call on a GPU sets the
 * array up (looks up its address and clears its counter head with a kernel
 * on `stream`): make that call outside HIP graph capture; later calls may
 * be captured and replayed. */
#define DW4_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int dw4_gemm_noalloc(int m, int k, int n, int group_size,
                     const uint16_t* x, int64_t ldx,
                     const int32_t* packed_qweight, const int32_t* packed_zeros,
                     const uint16_t* packed_scales, const int32_t* perm,
                     const uint16_t* bias, uint16_t* y, int64_t ldy, void* stream);

/* Device: dequantised fp16 weight w[K, N] (row stride ldw) in ORIGINAL row
 * order, bit-exact with fp16_rne(scale * (q - (zero + 1))). */
int dw4_dequant(int k, int n, int group_size,
                const int32_t* packed_qweight, const int32_t* packed_zeros,
                const uint16_t* packed_scales, const int32_t* perm,
                uint16_t* w, int64_t ldw, void* stream);

/* Device: the bf16 weight w[K, N] (row stride ldw) in ORIGINAL row order,
 * bit-exact with bf16_rne(fp16_rne(scale * (q - (zero + 1)))): the fp16
 * dequantised value converted to bf16, as the reference's bf16 route
 * computes it.  Replaces reconstruct_nv_bfloat16_exllama_v2
 * (cuda_extends/exllama/q4_matrix.cu:469-614), which q4_matmul_blas_v2
 * (entry.cpp:303-340 -> q4_matmul.cu:459-494) runs before its bf16 GEMM. */
int dw4_dequant_bf16(int k, int n, int group_size,
                     const int32_t* packed_qweight, const int32_t* packed_zeros,
                     const uint16_t* packed_scales, const int32_t* perm,
                     uint16_t* w, int64_t ldw, void* stream);

/* Calibration (no reference counterpart): a plain streaming read of `bytes`
 * of device memory at src in a decode-like launch shape -- `workgroups`
 * workgroups of `threads` threads (a multiple of 64, at most 1024), each
 * reading its contiguous bytes / workgroups range in 1 KiB wave loads of
 * 16 bytes per lane, four per wave in flight.  bytes must be a multiple of
 * workgroups * 1024.  Nothing is written unless the folded words equal
 * `never`; then sink (workgroups * threads uint32) receives them.  The
 * benchmark times it to state the HBM ceiling a weight-streaming launch of
 * that shape can reach. */
int dw4_stream_read(const void* src, size_t bytes, int workgroups, int threads, uint32_t never,
                    uint32_t* sink, void* stream);

/* out = g @ W^T, the activation gradient of y = x @ W (PEFT backward):
 * g fp16 [m, n] (row stride ldg), out fp16 [m, k] (row stride ldo) in the
 * checkpoint's row order (perm as given to dw4_repack).  The packed words
 * are read once; the weight entering the fp32-accumulated products is the
 * exact fp16(s * (q - z)) that dw4_dequant writes, so the result is the dense
 * product with dw4_dequant's output up to the order of fp32 sums.
 * g 16-byte aligned with ldg % 8 == 0; ldo >= k.  workspace: at least
 * dw4_gemm_t_workspace_size bytes (no zero-fill needed; 0 bytes for some
 * shapes).  Never synchronises or allocates.  Replaces
 * q4_transpose_matmul_blas_v2 (entry.cpp:392-429 ->
 * q4_transpose_matmul.cu:115-167: dequantise to fp16 K x N, then a dense
 * GEMM). */
int dw4_gemm_t(int m, int k, int n, int group_size, const uint16_t* g, int64_t ldg,
               const int32_t* packed_qweight, const int32_t* packed_zeros,
               const uint16_t* packed_scales, const int32_t* perm, uint16_t* out, int64_t ldo,
               void* workspace, size_t workspace_bytes, void* stream);
int dw4_gemm_t_workspace_size(int m, int k, int n, int group_size, size_t* workspace_bytes);

/* ---------------------------------------------------------------------------
 * Decoder-stage calls: several projections of one layer per launch.
 * ------------------------------------------------------------------------- */

/* One quantized matrix (buffers from dw4_repack for k, n, group_size, perm
 * as given to dw4_repack) and its output y fp16 [m, n], row stride ldy.
 * bias: NULL or fp16 [n]. */
typedef struct dw4_item {
  int k, n, group_size;
  const int32_t* packed_qweight;
  const int32_t* packed_zeros;
  const uint16_t* packed_scales;
  const int32_t* perm;
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldy;
} dw4_item;

/* y_i = x @ W_i (+ bias_i) for 1..4 matrices that share x, k and
 * group_size (with perm on all or on none).  For m <= 32 where
 * DW4_PATH_AUTO would take the decode kernel for the summed N, one launch
 * covers every strip of every matrix; for m > 128 with matrices of equal n
 * and no perm, one prefill launch covers every column tile of every matrix
 * when the plan for the summed N needs no K split; otherwise the matrices
 * run one after another as dw4_gemm does.  workspace: at least
 * dw4_workspace_size of each item. */
int dw4_gemm_group(int count, const dw4_item* items, int m, const uint16_t* x, int64_t ldx,
                   void* workspace, size_t workspace_bytes, void* stream);

/* h = fp16(silu(g) * u) with g = fp16(x @ W_gate (+ bias)),
 * u = fp16(x @ W_up (+ bias)), silu(v) = v / (1 + exp(-v)) in fp32.
 * gate and up: equal k, n, group_size and the same perm pointer (or both
 * NULL).  For m <= 32 where DW4_PATH_AUTO takes the decode kernel, one
 * launch keeps both products in registers and gate->y, up->y are not
 * written.  Otherwise the products are written to gate->y and up->y
 * (required then) and an elementwise pass writes h; h may be gate->y with
 * ldh == gate->ldy. */
int dw4_gemm_silu_mul(int m, const uint16_t* x, int64_t ldx, const dw4_item* gate,
                      const dw4_item* up, uint16_t* h, int64_t ldh, void* workspace,
                      size_t workspace_bytes, void* stream);

/* y = fp16(x * w * 1/sqrt(mean(x^2) + eps)) for each row of x fp16 [m, k]
 * (w fp16 [k]; fp32 sums in a fixed order).  k % 8 == 0; x, w, y 16-byte
 * aligned; ldx, ldy multiples of 8; y must not overlap x. */
int dw4_rms_norm(int m, int k, const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                 uint16_t* y, int64_t ldy, void* stream);

/* rms = rms_norm(x, norm_w, eps) (fp16 [m, k], row stride ldr), then
 * q, k, v = rms @ W (dw4_gemm_group of the three items). */
int dw4_attention_qkv_stage(int m, const uint16_t* x, int64_t ldx, const uint16_t* norm_w,
                            float eps, uint16_t* rms, int64_t ldr, const dw4_item* q,
                            const dw4_item* k, const dw4_item* v, void* workspace,
                            size_t workspace_bytes, void* stream);

/* rms = rms_norm(x, norm_w, eps); h = silu(rms @ W_gate) * (rms @ W_up)
 * written to gate->y (dw4_gemm_silu_mul with h = gate->y; up->y is the
 * second temporary); down->y = h @ W_down.  down->k == gate->n. */
int dw4_mlp_forward(int m, const uint16_t* x, int64_t ldx, const uint16_t* norm_w, float eps,
                    uint16_t* rms, int64_t ldr, const dw4_item* gate, const dw4_item* up,
                    const dw4_item* down, void* workspace, size_t workspace_bytes, void* stream);

/* x2 = fp16(residual + fp16(attn @ W_o (+ bias)))          -> o->y
 * rms = rms_norm(x2, norm_w, eps)                            -> rms
 * h = fp16(silu(rms @ W_gate) * (rms @ W_up))               -> gate->y
 * out = fp16(x2 + fp16(h @ W_down (+ bias)))                 -> down->y
 * attn fp16 [m, o->k] (row stride lda), residual fp16 [m, o->n] (ldres).
 * o->n == gate->k == down->n, down->k == gate->n.  up->y receives the up
 * product where gate and up cannot run as one launch (as dw4_gemm_silu_mul).
 * residual may be o->y itself (same stride) or down->y; down->y must not
 * overlap o->y, nor residual overlap o->y partially (DW4_ERR_INVALID_ARG).
 * Runs as o_proj and dw4_mlp_forward, each residual add done in the
 * epilogue of the GEMM before it (rounded after the product, as two fp16
 * tensor ops round). */
int dw4_decoder_after_stage(int m, const uint16_t* attn, int64_t lda, const uint16_t* residual,
                            int64_t ldres, const dw4_item* o, const uint16_t* norm_w, float eps,
                            uint16_t* rms, int64_t ldr, const dw4_item* gate, const dw4_item* up,
                            const dw4_item* down, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---------------------------------------------------------------------------
 * Paged KV cache and decode attention (the stage's other HBM stream).
 *
 * Cache layout: blocks of block_size (16 or 32) token slots; per block a key
 * part [kv_heads][head_size/8][block_size][8] and a value part
 * [kv_heads][head_size][block_size] (fp16), at the addresses in the
 * int64 tables key_block_ptrs / value_block_ptrs (device memory, one entry
 * per block), kv_head_stride elements between the kv heads of a block.
 * Slot s is offset s % block_size of block s / block_size.
 * ------------------------------------------------------------------------- */

/* key, value fp16 [num_tokens][num_kv_heads][head_size] (row strides
 * key_stride, value_stride) to the slots in slot_mapping (int64 device
 * [num_tokens]; negative = padding, skipped).  Replaces reshape_and_cache
 * (cuda_extends/vllm/cache_kernels.cu:242-285, :287-330). */
int dw4_reshape_and_cache(int num_tokens, int num_kv_heads, int head_size, int block_size,
                          const uint16_t* key, int64_t key_stride, const uint16_t* value,
                          int64_t value_stride, const int64_t* key_block_ptrs,
                          const int64_t* value_block_ptrs, int kv_head_stride,
                          const int64_t* slot_mapping, void* stream);

/* The reverse copy: slots back to token rows.  Replaces restore_from_cache
 * (cache_kernels.cu:332-420). */
int dw4_restore_from_cache(int num_tokens, int num_kv_heads, int head_size, int block_size,
                           uint16_t* key, int64_t key_stride, uint16_t* value,
                           int64_t value_stride, const int64_t* key_block_ptrs,
                           const int64_t* value_block_ptrs, int kv_head_stride,
                           const int64_t* slot_mapping, void* stream);

/* Decode attention of one new token per sequence over its cached context:
 * out[s][h] = softmax_t(scale * q[s][h] . k_t (+ alibi[h] * (t - ctx + 1)))
 * . v_t for t < context_lens[s], with query head h reading kv head
 * h / (num_heads / num_kv_heads) (the reference's head_mapping,
 * repeat_interleave(arange(kv_heads), groups)).  query, out fp16
 * [num_seqs][num_heads][head_size] with row strides q_stride, o_stride per
 * sequence; block_tables int32 [num_seqs][max_blocks_per_seq];
 * context_lens int32 [num_seqs], each in 1..max_context_len; alibi_slopes
 * float [num_heads] or NULL.  head_size 64, 80, 96, 112, 128 or 256; num_heads a
 * multiple of num_kv_heads with at most 8 query heads per kv head.
 * Softmax and both products in fp32; long contexts are split into
 * partitions combined in a fixed order (deterministic).  workspace: at
 * least dw4_paged_attention_workspace_size bytes (0 for short contexts).
 * Never synchronises or allocates.  Replaces paged_attention_v1 / v2
 * (cuda_extends/vllm/attention/attention_kernels.cu:1602-1632, 1786-1843)
 * as operators/core/attention/real_page.py:23-189 calls them. */
int dw4_paged_attention(int num_seqs, int num_heads, int num_kv_heads, int head_size,
                        int block_size, const uint16_t* query, int64_t q_stride, uint16_t* out,
                        int64_t o_stride, const int64_t* key_block_ptrs,
                        const int64_t* value_block_ptrs, int kv_head_stride, float scale,
                        const int32_t* block_tables, int max_blocks_per_seq,
                        const int32_t* context_lens, int max_context_len,
                        const float* alibi_slopes, void* workspace, size_t workspace_bytes,
                        void* stream);
int dw4_paged_attention_workspace_size(int num_seqs, int num_heads, int num_kv_heads,
                                       int head_size, int block_size, int max_context_len,
                                       size_t* workspace_bytes);

/* Rotary embedding (rotate-half form) in place on fp16 x
 * [batch_size][rows_per_batch][head_dim], rows_per_batch = tokens *
 * num_heads: row r of batch entry b takes position
 * (past_len >= 0 ? past_len : past_lens[b]) + r / num_heads of the fp16
 * tables sin_table, cos_table [max_positions][head_dim]; rows whose
 * position is outside the tables are left as they are.  Each product and
 * fused multiply-add is rounded once in fp16, as the reference's
 * half-precision kernel does.  Replaces rope_cuda / the RoPE half of
 * attention_forward_rope_stage_v2 (cuda_extends/exllama/fuse_v2/rope.cu:24-135). */
int dw4_rope(int batch_size, int rows_per_batch, int num_heads, int head_dim, uint16_t* x,
             const uint16_t* sin_table, const uint16_t* cos_table, int max_positions, int past_len,
             const int32_t* past_lens, void* stream);

/* One decode token per sequence: dw4_rope on its q and k rows (position
 * positions[s]), then dw4_reshape_and_cache of the rotated k and of v into
 * slot block_tables[s][p / block_size] * block_size + p % block_size, and
 * context_lens_out[s] = p + 1 (if not NULL) -- three reference calls
 * (rope.cu, cache_kernels.cu:242-285 and the context-length update of the
 * decode loop) in one launch.  q [num_seqs][num_heads][head_dim],
 * k, v [num_seqs][num_kv_heads][head_dim] fp16 with per-sequence strides.
 * A position outside the block table writes no slot; one outside the
 * sin/cos tables leaves the rows unrotated.  context_lens_out must not
 * overlap positions (an in-place advance would race with the workgroups of
 * the same sequence that still read the position): DW4_ERR_INVALID_ARG.
 * No counterpart in the reference as a single call. */
int dw4_rope_and_cache(int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                       int block_size, uint16_t* q, int64_t q_stride, uint16_t* k,
                       int64_t k_stride, const uint16_t* v, int64_t v_stride,
                       const uint16_t* sin_table, const uint16_t* cos_table, int max_positions,
                       const int32_t* positions, const int32_t* block_tables,
                       int max_blocks_per_seq, const int64_t* key_block_ptrs,
                       const int64_t* value_block_ptrs, int kv_head_stride,
                       int32_t* context_lens_out, void* stream);

/* ------------------------------------------------------------------------
 * Decode chain: one launch over a list of projections at m <= 4 (no single
 * reference call: it runs the per-projection q4_matmul_cuda_v2 calls,
 * cuda_extends/exllama/entry.cpp:221-251, that the layer loop of
 * operators/assemble/decoders/real_decoders_group.py:106-159 makes for one
 * decode step, in one kernel).  Every workgroup streams the packed weights of
 * its share of all links back to back, so the weight stream does not stop at
 * the dependency points between projections; a link's activations are read
 * only once the links it depends on are complete on every workgroup.
 *
 * Link i: y_i = fp16(fp16(x_i @ W_i) (+ bias_i)) (+ residual_i) with fp32
 * accumulation, x_i fp16 [m, k] (row stride ldx), y_i fp16 [m, n] (ldy),
 * residual_i NULL or fp16 [m, n] (ldres; it may be y_i itself).  `after`
 * is -1 (x_i is ready when the launch starts) or the index of an earlier
 * link: x_i (and residual_i) are read only after links 0..after have
 * completed.  Every two links of which one writes a buffer the other reads
 * or writes must be ordered that way (the later one's `after` at least the
 * earlier one's index); dw4_chain_prepare refuses a list that is not.
 * Supported: group_size a multiple of 128, no act-order (perm NULL),
 * k <= 16384, n <= 32768, m <= 4.  Results are deterministic; the sums run
 * in another order than dw4_gemm's, so the two agree to the GEMM tolerance,
 * not bit for bit.
 *
 * dw4_chain_prepare validates a list and writes it, with the chain's
 * progress state, into `chain` (device memory of dw4_chain_buffer_size
 * bytes, owned by the caller); it copies synchronously and must not be
 * captured.  dw4_gemm_chain then launches the list as prepared (capturable
 * and replayable; launches of one chain buffer must not overlap in time).
 * The pointers in the links are used as given at every launch.  The plan
 * struct is filled by prepare and only read by the launch.
 * dw4_chain_timed_out reports (synchronously) whether a launch on this
 * buffer gave up waiting for a dependency (about 0.2 s; the kernel then
 * finishes with invalid outputs instead of hanging). */
typedef struct dw4_chain_link {
  int k, n, group_size;
  const int32_t* packed_qweight;
  const int32_t* packed_zeros;
  const uint16_t* packed_scales;
  const int32_t* perm;
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* bias;
  const uint16_t* residual;
  int64_t ldres;
  uint16_t* y;
  int64_t ldy;
  int after;
} dw4_chain_link;

typedef struct dw4_chain_plan {
  int count, m, workgroups, waves, ring, max_k, max_strips, max_groups;
  size_t smem_bytes;
} dw4_chain_plan;

int dw4_chain_buffer_size(int count, size_t* bytes);
int dw4_chain_prepare(int count, const dw4_chain_link* links, int m, void* chain,
                      size_t chain_bytes, dw4_chain_plan* plan);
int dw4_gemm_chain(const dw4_chain_plan* plan, void* chain, void* stream);
int dw4_chain_timed_out(const void* chain, int* timed_out);

#ifdef __cplusplus
}
#endif

#endif /* DROFELL_W4A16_H */
