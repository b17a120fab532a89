"""CPU oracle for the decoder-stage operations around the W4A16 GEMM.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.

Restates, in numpy float64 with one fp16 rounding at the end of each
operation, what the reference's fused decoder stage computes (paths relative
to ``/root/reference/After-Revision-DROFELL``):

* ``rms_norm`` -- ``cuda_extends/exllama/fuse_v2/rms_norm.cu:26-93``
  (``rms_norm_kernel``: inputs clamped to +-65504, sum of squares, ``r =
  rsqrt(sum / dim + eps)``, ``y = fp16(x * w * r)``) and its launcher
  ``:109-131``;
* ``silu_mul`` -- ``cuda_extends/exllama/fuse_v2/q_mlp.cu:13-33,44-85``
  (``x = silu(x) * y`` with ``silu(v) = v / (1 + exp(-v))``);
* ``qkv_stage`` -- ``fuse_v2/q_attn.cu:23-54``
  (``attention_forward_qkv_stage``: rms_norm, then q, k, v from the
  normalised fp16 rows);
* ``mlp_forward`` -- ``fuse_v2/q_mlp.cu:96-133`` (rms_norm, gate and up
  from the normalised rows, each rounded to fp16, silu_mul, then down);
* ``after_stage`` -- ``operators/core/decoder_wrap/real_fuse.py:77-103``
  (``_fuse_forward_after_stage``: o_proj, ``residual + o`` in fp16,
  mlp_forward on that sum, then ``sum + mlp`` in fp16).

The reference evaluates silu in fp16 arithmetic with CUDA's half-precision
exp and reciprocal; this restatement (and the HIP kernels) evaluate it
exactly / in fp32 and round once, so the two agree to within a few fp16
units in the last place, not bit for bit.  Pinned by ``tests/test_oracle.py``
(closed forms, an independent library sigmoid, scale invariance and
planted mistakes).
"""
from __future__ import annotations

import numpy as np

from . import gptq

FP16_MAX = 65504.0


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """fp16 [M, K] rows normalised by their root mean square, times w
    (rms_norm.cu:48-92)."""
    xf = np.clip(np.asarray(x, dtype=np.float16).astype(np.float64), -FP16_MAX, FP16_MAX)
    wf = np.asarray(w, dtype=np.float16).astype(np.float64)
    r = 1.0 / np.sqrt((xf * xf).sum(axis=-1, keepdims=True) / xf.shape[-1] + eps)
    with np.errstate(over="ignore"):
        return (xf * wf * r).astype(np.float16)


def silu(v: np.ndarray) -> np.ndarray:
    """v / (1 + exp(-v)) in float64 (q_mlp.cu:13-22)."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """fp16(silu(g) * u) for fp16 g, u (q_mlp.cu:59-84)."""
    gf = np.asarray(g, dtype=np.float16).astype(np.float64)
    uf = np.asarray(u, dtype=np.float16).astype(np.float64)
    with np.errstate(over="ignore"):
        return (silu(gf) * uf).astype(np.float16)


def qkv_stage(x: np.ndarray, norm_w: np.ndarray, eps: float, weights):
    """(rms fp16, [wide-accumulated rms @ W for W in weights]) (q_attn.cu:44-48)."""
    rms = rms_norm(x, norm_w, eps)
    return rms, [gptq.gemm_ref(rms, w) for w in weights]


def mlp_forward(x: np.ndarray, norm_w: np.ndarray, eps: float, w_gate: np.ndarray,
                w_up: np.ndarray, w_down: np.ndarray):
    """(rms fp16, h fp16, wide-accumulated h @ W_down) (q_mlp.cu:118-132)."""
    rms = rms_norm(x, norm_w, eps)
    g = gptq.gemm_ref(rms, w_gate).astype(np.float16)
    u = gptq.gemm_ref(rms, w_up).astype(np.float16)
    h = silu_mul(g, u)
    return rms, h, gptq.gemm_ref(h, w_down)


def add_fp16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """fp16(a + b) for fp16 operands: the exact sum rounded once, as torch's
    fp16 ``residual + hidden_states`` (real_fuse.py:82,102) rounds it."""
    af = np.asarray(a, dtype=np.float16).astype(np.float64)
    bf = np.asarray(b, dtype=np.float16).astype(np.float64)
    with np.errstate(over="ignore"):
        return (af + bf).astype(np.float16)


def after_stage(attn: np.ndarray, residual: np.ndarray, w_o: np.ndarray, norm_w: np.ndarray,
                eps: float, w_gate: np.ndarray, w_up: np.ndarray, w_down: np.ndarray):
    """(x2, rms, h, out) of the decoder layer after attention
    (real_fuse.py:77-103): x2 = residual + fp16(attn @ W_o); rms, h and the
    down product as mlp_forward(x2); out = x2 + fp16(down product)."""
    x2 = add_fp16(residual, gptq.gemm_ref(attn, w_o).astype(np.float16))
    rms, h, d = mlp_forward(x2, norm_w, eps, w_gate, w_up, w_down)
    return x2, rms, h, add_fp16(x2, d.astype(np.float16))
