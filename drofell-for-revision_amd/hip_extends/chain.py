"""Decode chain: several W4A16 projections of one decode step in one launch.

A decode step of a decoder stage runs its projections one after another
(``q4_matmul_cuda_v2`` per projection, ``cuda_extends/exllama/entry.cpp:221-251``,
called by the layer loop of ``operators/assemble/decoders/real_decoders_group.py:106-159``;
paths relative to ``/root/reference/After-Revision-DROFELL``).  :class:`Q4Chain`
runs such a list as ``dw4_gemm_chain``: one persistent kernel in which every
workgroup streams the packed weights of its share of all projections back to
back, and a projection reads its activations only once the projections it
depends on (``after``) have completed everywhere.  Prepare once
(``dw4_chain_prepare`` copies the list to the device synchronously), then
``run()`` as often as needed, also under HIP graph capture; the tensors
named in the links are used in place at every run.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib


@dataclass
class ChainStep:
    """One link: ``y = fp16(fp16(x @ W) (+ bias)) (+ residual)``.  ``matrix``
    is a repacked matrix (``Q4MatrixV2`` or ``MarlinQ4Matrix``: its packed
    ``qweight`` / ``qzeros`` / ``scales``); ``after`` is -1 or the index of an
    earlier link whose completion (and that of every link before it) the
    read of ``x`` and ``residual`` waits for."""

    matrix: object
    x: torch.Tensor
    y: torch.Tensor
    after: int = -1
    bias: Optional[torch.Tensor] = None
    residual: Optional[torch.Tensor] = None


def _dims(matrix) -> tuple:
    k = getattr(matrix, "height", None) or matrix.in_features
    n = getattr(matrix, "width", None) or matrix.out_features
    return k, n, matrix.group_size


def _perm_of(matrix) -> Optional[torch.Tensor]:
    perm = getattr(matrix, "perm", None)
    if perm is None:
        perm = getattr(matrix, "_perm", None)
    return perm if perm is not None and perm.numel() else None


class Q4Chain:
    """A prepared decode chain (see the module docstring)."""

    def __init__(self, steps: Sequence[ChainStep], m: int) -> None:
        if not steps:
            raise ValueError("a chain needs at least one link")
        self.steps: List[ChainStep] = list(steps)
        self.m = m
        dev = self.steps[0].x.device
        self.device = dev
        arr = (_lib.ChainLink * len(self.steps))()
        for i, st in enumerate(self.steps):
            k, n, g = _dims(st.matrix)
            for name, t, cols in (("x", st.x, k), ("y", st.y, n)):
                if t.dtype != torch.float16 or t.dim() != 2 or t.shape[0] != m or \
                        t.shape[1] != cols or t.stride(1) != 1:
                    raise ValueError(f"link {i}: {name} must be fp16 [{m}, {cols}] with unit "
                                     f"column stride, got {t.dtype} {tuple(t.shape)}")
            res = st.residual
            if res is not None and (res.dtype != torch.float16 or tuple(res.shape) != (m, n) or
                                    res.stride(1) != 1):
                raise ValueError(f"link {i}: residual must be fp16 [{m}, {n}]")
            if st.bias is not None and (st.bias.dtype != torch.float16 or st.bias.numel() != n):
                raise ValueError(f"link {i}: bias must be fp16 [{n}]")
            perm = _perm_of(st.matrix)
            arr[i] = _lib.ChainLink(
                k, n, g, st.matrix.qweight.data_ptr(), st.matrix.qzeros.data_ptr(),
                st.matrix.scales.data_ptr(), None if perm is None else perm.data_ptr(),
                st.x.data_ptr(), st.x.stride(0),
                None if st.bias is None else st.bias.data_ptr(),
                None if res is None else res.data_ptr(), 0 if res is None else res.stride(0),
                st.y.data_ptr(), st.y.stride(0), st.after)
        self._links = arr
        size = ctypes.c_size_t(0)
        _lib.check("dw4_chain_buffer_size",
                   _lib.load().dw4_chain_buffer_size(len(self.steps), ctypes.byref(size)))
        self.buffer = torch.empty(size.value, dtype=torch.uint8, device=dev)
        self.plan = _lib.ChainPlan()
        with torch.cuda.device(dev):
            torch.cuda.synchronize(dev)
            _lib.check("dw4_chain_prepare", _lib.load().dw4_chain_prepare(
                len(self.steps), arr, m, self.buffer.data_ptr(), self.buffer.numel(),
                ctypes.byref(self.plan)))

    def run(self, stream: Optional[int] = None) -> None:
        """Launch the chain on ``stream`` (default: the device's current stream)."""
        s = torch.cuda.current_stream(self.device).cuda_stream if stream is None else stream
        _lib.check("dw4_gemm_chain",
                   _lib.load().dw4_gemm_chain(ctypes.byref(self.plan), self.buffer.data_ptr(), s))

    def timed_out(self) -> bool:
        """Whether a launch gave up waiting for a dependency (synchronous)."""
        flag = ctypes.c_int(0)
        _lib.check("dw4_chain_timed_out",
                   _lib.load().dw4_chain_timed_out(self.buffer.data_ptr(), ctypes.byref(flag)))
        return bool(flag.value)

    def launches(self) -> int:
        """Launches completed on this buffer (the header's launch number)."""
        return int(self.buffer[:8].view(torch.int64).item())
