"""CPU oracle for DROFELL's GPTQ W4A16 quantized-Linear hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.

It restates, in numpy, the arithmetic the reference defines for one GPTQ
4-bit projection (paths relative to
``/root/reference/After-Revision-DROFELL``):

* nibble addressing of ``qweight`` (rows packed along K) --
  ``cuda_extends/exllama/matrix.cuh:156-160`` (``MatrixView_q4_column``),
  ``operators/core/linear/real_quant.py:79-86``;
* nibble addressing of ``qzeros`` (columns packed along N) --
  ``cuda_extends/exllama/matrix.cuh:120-124`` (``MatrixView_q4_row``),
  ``operators/core/linear/real_quant.py:70-77``;
* the "+1" effective zero -- ``real_quant.py:76``,
  ``cuda_extends/exllama/q4_matrix.cu:221``,
  ``cuda_extends/exllama/q_gemm_kernel_gptq.cuh:131-134``;
* the dequantised weight ``W[k,n] = fp16(scales[g_idx[k],n] *
  (q[k,n] - z[g_idx[k],n]))`` -- ``real_quant.py:89-90``
  (``QuantLinear.get_reconstruct_weights``; the GPU kernels compute the
  same value: ``q4_matrix.cu:418,427`` and
  ``cuda_extends/marlin/marlin_dequant.cu:72``);
* the act-order row order (stable counting sort of rows by ``g_idx``,
  ``x_map[new] = old``) -- ``q4_matrix.cu:125-159`` (``make_sequential``);
* the forward ``y = x @ W`` (+ optional fp16 bias) --
  ``cuda_extends/exllama.py:492-526,730-736``;
* the bf16 route's weight ``bf16(W)`` (fp16 value rounded to bfloat16) --
  ``q4_matrix.cu:465-467,583-601``, ``q4_matmul.cu:480-494``.

Parity status of every function here is pinned by ``tests/test_oracle.py``
(closed forms, an exhaustive dequant known-answer table against an
independent integer round-to-nearest-even, brute force on tiny inputs and
invariants).  The reference ships no golden vectors for this path.
"""
from __future__ import annotations

import numpy as np

BITS = 4
PACK = 32 // BITS  # 8 nibbles per int32 word


def _as_u32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


def unpack_qweight(qweight: np.ndarray) -> np.ndarray:
    """q[k, n] = (qweight[k // 8, n] >> 4 * (k % 8)) & 0xF  (uint8 [K, N]).

    Follows ``MatrixView_q4_column::item`` (``matrix.cuh:156-160``).
    """
    w = _as_u32(qweight)
    kw, n = w.shape
    shifts = (np.arange(PACK, dtype=np.uint32) * BITS)[None, :, None]
    q = (w[:, None, :] >> shifts) & 0xF
    return q.reshape(kw * PACK, n).astype(np.uint8)


def pack_qweight(q: np.ndarray) -> np.ndarray:
    """Inverse of :func:`unpack_qweight`: uint8 [K, N] -> int32 [K/8, N]."""
    k, n = q.shape
    assert k % PACK == 0
    q = q.astype(np.uint32).reshape(k // PACK, PACK, n)
    shifts = (np.arange(PACK, dtype=np.uint32) * BITS)[None, :, None]
    w = np.bitwise_or.reduce(q << shifts, axis=1)
    return w.astype(np.uint32).view(np.int32)


def unpack_qzeros(qzeros: np.ndarray) -> np.ndarray:
    """Stored zero nibble z[g, n] = (qzeros[g, n // 8] >> 4 * (n % 8)) & 0xF.

    Follows ``MatrixView_q4_row::item`` (``matrix.cuh:120-124``); the
    effective zero used by the arithmetic is this value + 1.
    """
    w = _as_u32(qzeros)
    g, nw = w.shape
    shifts = (np.arange(PACK, dtype=np.uint32) * BITS)[None, None, :]
    z = (w[:, :, None] >> shifts) & 0xF
    return z.reshape(g, nw * PACK).astype(np.uint8)


def pack_qzeros(z: np.ndarray) -> np.ndarray:
    """Inverse of :func:`unpack_qzeros`: uint8 [G, N] -> int32 [G, N/8]."""
    g, n = z.shape
    assert n % PACK == 0
    z = z.astype(np.uint32).reshape(g, n // PACK, PACK)
    shifts = (np.arange(PACK, dtype=np.uint32) * BITS)[None, None, :]
    w = np.bitwise_or.reduce(z << shifts, axis=2)
    return w.astype(np.uint32).view(np.int32)


def default_g_idx(k: int, group_size: int) -> np.ndarray:
    """``g_idx[k] = k // group_size`` (``real_quant.py:40-44``)."""
    return (np.arange(k) // group_size).astype(np.int32)


def dequantize(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
               g_idx: np.ndarray) -> np.ndarray:
    """fp16 [K, N] weight in ORIGINAL row order.

    ``W[k,n] = fp16_rne(scales[g_idx[k], n] * (q[k,n] - (z[g_idx[k], n] + 1)))``
    -- ``real_quant.py:69-102``.  The integer difference is exact and
    |q - z| <= 16, so the fp32 product of an fp16 scale and it is exact; the
    single rounding is the fp32 -> fp16 round-to-nearest-even, which is what
    an fp16 multiply produces (``q4_matrix.cu:418``, ``__hmul2``).
    """
    q = unpack_qweight(qweight).astype(np.int16)
    z = unpack_qzeros(qzeros).astype(np.int16) + 1
    gi = np.asarray(g_idx).astype(np.int64)
    d = (q - z[gi]).astype(np.float32)
    s = np.asarray(scales, dtype=np.float16)[gi].astype(np.float32)
    return (s * d).astype(np.float16)


def bf16_bits(w: np.ndarray) -> np.ndarray:
    """uint16 bfloat16 bit patterns of fp16 values: each (exact) value
    rounded once to bfloat16, to nearest, ties to even.

    The reference's bf16 route converts the fp16 dequantised value with
    ``__float2bfloat16(__half2float(v))`` (``q4_matrix.cu:465-467``, used at
    ``:583-601`` by ``reconstruct_gptq_kernel_nv_bfloat16``).  A NaN maps to
    a quiet NaN of the same sign (checks compare NaNs as a class).
    """
    f = np.asarray(w, dtype=np.float16).astype(np.float32).view(np.uint32).astype(np.uint64)
    nan = (f & 0x7FFFFFFF) > 0x7F800000
    rne = (f + 0x7FFF + ((f >> 16) & 1)) >> 16
    return np.where(nan, (f >> 16) | 0x40, rne).astype(np.uint16)


def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    """float32 values of uint16 bfloat16 bit patterns (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequantize_bf16(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
                    g_idx: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns [K, N] of the weight the reference's bf16 route
    multiplies by: bf16_rne(fp16 dequantised weight), ORIGINAL row order
    (``q4_matrix.cu:469-614``)."""
    return bf16_bits(dequantize(qweight, qzeros, scales, g_idx))


def act_order_perm(g_idx: np.ndarray, groups: int) -> np.ndarray:
    """Stable counting sort of rows by group: ``perm[new_row] = old_row``.

    Same order as ``make_sequential``'s host part (``q4_matrix.cu:137-159``):
    histogram of g_idx, exclusive prefix, rows placed in ascending original
    order within each group.
    """
    g_idx = np.asarray(g_idx).astype(np.int64)
    counts = np.bincount(g_idx, minlength=groups)
    start = np.concatenate([[0], np.cumsum(counts)[:-1]])
    perm = np.empty(len(g_idx), dtype=np.int32)
    fill = start.copy()
    for row, g in enumerate(g_idx):
        perm[fill[g]] = row
        fill[g] += 1
    return perm


class WideWeight:
    """An fp16 weight held once in float64, for checkers that multiply the
    same weight many times (:func:`gemm_ref` then skips its widening)."""

    def __init__(self, w: np.ndarray) -> None:
        self.w16 = np.asarray(w, dtype=np.float16)
        self.w64 = self.w16.astype(np.float64)


def gemm_ref(x: np.ndarray, w) -> np.ndarray:
    """Wide-accumulated product of fp16 activations and the fp16 weight
    (an array or a :class:`WideWeight`).

    Returns float64 [M, N]; every product of two fp16 values is exact in
    float64 and the sum is far more accurate than the fp32 accumulation the
    tolerance is stated against.
    """
    w64 = w.w64 if isinstance(w, WideWeight) else np.asarray(w, dtype=np.float16).astype(np.float64)
    return np.asarray(x, dtype=np.float16).astype(np.float64) @ w64


def forward(x: np.ndarray, qweight: np.ndarray, qzeros: np.ndarray,
            scales: np.ndarray, g_idx: np.ndarray,
            bias: np.ndarray | None = None) -> np.ndarray:
    """fp16 ``y = x @ W (+ bias)`` for x fp16 [..., K].

    The fp16 output rounding and the separate fp16 bias add follow the
    exllama wrappers (``exllama.py:498,733-735``).
    """
    x = np.asarray(x, dtype=np.float16)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    y = gemm_ref(x2, dequantize(qweight, qzeros, scales, g_idx)).astype(np.float16)
    if bias is not None:
        y = (y + np.asarray(bias, dtype=np.float16)[None, :]).astype(np.float16)
    return y.reshape(*shape[:-1], y.shape[-1])


def row_tolerance(y_ref: np.ndarray, rel: float = 2e-2) -> np.ndarray:
    """Per-row bound ``rel * ||y_ref[m, :]||_inf`` (the parity rule for GEMM outputs)."""
    y = np.asarray(y_ref, dtype=np.float64)
    return rel * np.max(np.abs(y), axis=-1, keepdims=True)


def within_tolerance(y: np.ndarray, y_ref: np.ndarray, rel: float = 2e-2):
    """Return (ok, worst_ratio) for ``max|y - y_ref| <= rel * ||row||_inf``."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(y_ref, dtype=np.float64)
    tol = row_tolerance(ref, rel)
    err = np.max(np.abs(y - ref), axis=-1, keepdims=True)
    safe = np.where(tol > 0, tol, 1.0)
    ratio = np.where(tol > 0, err / safe, np.where(err > 0, np.inf, 0.0))
    worst = float(np.max(ratio)) if ratio.size else 0.0
    return worst <= 1.0, worst
