"""Seeded synthetic GPTQ 4-bit projections in the checkpoint format.

The tensors have exactly the shapes and dtypes of the module buffers that
``operators/core/linear/real_quant.py`` (and the reference's
``QuantLinear.__init__``) registers: ``qweight`` int32 [K/8, N] (rows packed
along K, 8 nibbles per word, row k at bits 4*(k%8)), ``qzeros`` int32
[K/g, N/8] (columns packed along N, stored zero = effective zero - 1),
``scales`` fp16 [K/g, N] and ``g_idx`` int32 [K].

Draw order from one ``torch.Generator`` seeded with ``seed``: q, zeros (only
when asymmetric), scales, act-order permutation (only when act-order).
Activations use their own generator so that one weight set serves many M.
Distributions are the benchmark ones: q ~ U{0..15}; stored zeros ~ U{0..15}
or all 7 (effective zero 8, the symmetric uint4b8 convention);
scales = |N(0,1)| * 0.01 + 1e-3; x ~ N(0,1) fp16; act-order
g_idx[k] = pi(k) // g for a seeded permutation pi, so every group holds
exactly g rows.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

SYMMETRIC_QZERO_WORD = 0x77777777


def _wrap_i32(v: torch.Tensor) -> torch.Tensor:
    """int64 tensor holding uint32 bit patterns -> int32 with the same bits."""
    return torch.where(v >= 2 ** 31, v - 2 ** 32, v).to(torch.int32)


def pack_rows(q: torch.Tensor) -> torch.Tensor:
    """uint4 values [K, N] -> GPTQ qweight int32 [K/8, N] (row k at 4*(k%8))."""
    k, n = q.shape
    q = q.to(torch.int64).reshape(k // 8, 8, n)
    shifts = (torch.arange(8, dtype=torch.int64) * 4).view(1, 8, 1)
    return _wrap_i32((q << shifts).sum(dim=1))


def pack_cols(z: torch.Tensor) -> torch.Tensor:
    """uint4 values [G, N] -> GPTQ qzeros int32 [G, N/8] (col n at 4*(n%8))."""
    g, n = z.shape
    z = z.to(torch.int64).reshape(g, n // 8, 8)
    shifts = (torch.arange(8, dtype=torch.int64) * 4).view(1, 1, 8)
    return _wrap_i32((z << shifts).sum(dim=2))


@dataclass
class GPTQLayer:
    in_features: int
    out_features: int
    group_size: int
    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor
    g_idx: torch.Tensor
    act_order: bool
    symmetric: bool

    def to(self, device) -> "GPTQLayer":
        return GPTQLayer(self.in_features, self.out_features, self.group_size,
                         self.qweight.to(device), self.qzeros.to(device),
                         self.scales.to(device), self.g_idx.to(device),
                         self.act_order, self.symmetric)

    def numpy(self) -> dict:
        return {
            "qweight": self.qweight.cpu().numpy(),
            "qzeros": self.qzeros.cpu().numpy(),
            "scales": self.scales.cpu().numpy(),
            "g_idx": self.g_idx.cpu().numpy(),
        }


def make_layer(in_features: int, out_features: int, group_size: int = 128, *,
               seed: int = 0, symmetric: bool = False, act_order: bool = False,
               scale_mul: float = 0.01, scale_add: float = 1e-3) -> GPTQLayer:
    k, n = in_features, out_features
    g = k if group_size == -1 else group_size
    assert k % 8 == 0 and n % 8 == 0 and k % g == 0
    groups = k // g
    gen = torch.Generator().manual_seed(seed)
    q = torch.randint(0, 16, (k, n), generator=gen, dtype=torch.int32)
    if symmetric:
        z = torch.full((groups, n), 7, dtype=torch.int32)
    else:
        z = torch.randint(0, 16, (groups, n), generator=gen, dtype=torch.int32)
    scales = (torch.randn(groups, n, generator=gen).abs() * scale_mul + scale_add).to(torch.float16)
    if act_order:
        pi = torch.randperm(k, generator=gen)
        g_idx = (pi // g).to(torch.int32)
    else:
        g_idx = (torch.arange(k) // g).to(torch.int32)
    return GPTQLayer(k, n, g, pack_rows(q), pack_cols(z), scales, g_idx,
                     act_order, symmetric)


def make_x(m: int, k: int, seed: int = 0, device: Optional[torch.device] = None) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen).to(torch.float16)
    return x if device is None else x.to(device)


# Llama-2 projection shapes (K, N) as (in_features, out_features).
LLAMA2_7B_SHAPES = {
    "q_proj": (4096, 4096), "k_proj": (4096, 4096), "v_proj": (4096, 4096),
    "o_proj": (4096, 4096), "gate_proj": (4096, 11008), "up_proj": (4096, 11008),
    "down_proj": (11008, 4096),
}
# The same layer with q/k/v and gate/up merged along the output dimension,
# the decode topology of the reference's Marlin loader
# (operators/assemble/decoders/real_loader_marlin.py:61-79).
LLAMA2_7B_MERGED_SHAPES = {
    "qkv_proj": (4096, 12288), "o_proj": (4096, 4096), "gate_up_proj": (4096, 22016),
    "down_proj": (11008, 4096),
}
LLAMA2_13B_SHAPES = {
    "q_proj": (5120, 5120), "k_proj": (5120, 5120), "v_proj": (5120, 5120),
    "o_proj": (5120, 5120), "gate_proj": (5120, 13824), "up_proj": (5120, 13824),
    "down_proj": (13824, 5120),
}


def algorithmic_bytes(m: int, k: int, n: int, group_size: int, act_order: bool,
                      count_zeros: bool = True) -> int:
    """Bytes one GEMM must move at minimum: packed weight, metadata, x, y."""
    groups = k // group_size
    b = k * n // 2 + 2 * groups * n + 2 * m * k + 2 * m * n
    if count_zeros:
        b += groups * n // 2
    if act_order:
        b += 4 * k
    return b


def flops(m: int, k: int, n: int) -> int:
    return 2 * m * k * n
