"""The reference's CPU dequantise-then-matmul path, restated with torch CPU ops.

TEST/BENCH INFRASTRUCTURE ONLY: used as ``bench.py``'s ``cpu_baseline`` leg
and checked against ``oracle/gptq.py`` in ``tests/test_cpu_path.py``.

Follows ``QuantLinear.get_reconstruct_weights``
(``/root/reference/After-Revision-DROFELL/operators/core/linear/real_quant.py:69-102``)
with ``wf = [0, 4, ..., 28]`` (the GPTQ shift table the reference's code
expects but never defines), then ``x.float() @ W.float()``.
"""
from __future__ import annotations

import torch

_WF = torch.arange(0, 32, 4, dtype=torch.int32)


def reconstruct_weights(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                        g_idx: torch.Tensor) -> torch.Tensor:
    """fp16 [K, N]: torch shift/and/gather/fp16-multiply, as real_quant.py:69-102."""
    zeros = torch.bitwise_right_shift(qzeros.unsqueeze(2).expand(-1, -1, 8),
                                      _WF.unsqueeze(0)).to(torch.int8)
    torch.bitwise_and(zeros, 15, out=zeros)
    zeros = zeros + 1
    zeros = zeros.reshape(scales.shape)
    weight = torch.bitwise_right_shift(qweight.unsqueeze(1).expand(-1, 8, -1),
                                       _WF.unsqueeze(-1)).to(torch.int8)
    torch.bitwise_and(weight, 15, out=weight)
    weight = weight.reshape(weight.shape[0] * weight.shape[1], weight.shape[2])
    gi = g_idx.long()
    return scales[gi] * (weight - zeros[gi])


def forward(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
            g_idx: torch.Tensor) -> torch.Tensor:
    w = reconstruct_weights(qweight, qzeros, scales, g_idx)
    return (x.float() @ w.float()).to(torch.float16)
