"""GPTQ checkpoint geometry shared by the quantized-Linear front ends.

``QuantLinear`` (the reference's exllama-path API) and ``MarlinQuantLinear``
(its Marlin-path API) load the same checkpoint tensors and hand them to the
same packed W4A16 kernels; they differ only in which checks the reference
applies and in the runtime objects around the kernels.  What they share
lives here:

* :class:`GptqGeometry` -- the resolved dimensions of one projection
  (group size -1 means a single group; act-order is void with one group)
  and each front end's admission checks, raised with the exception type
  the reference raises (``operators/core/linear/real_quant.py:21-23``
  asserts; ``real_marlin.py:36-45`` ValueErrors; paths relative to
  ``/root/reference/After-Revision-DROFELL``);
* :func:`checkpoint_buffers` -- the zero tensors a module registers under
  the checkpoint's buffer names, shapes and dtypes (``real_quant.py:25-44``),
  which ``load_state_dict`` then fills from per-layer safetensors;
* :func:`check_mergeable` / :func:`concat_outputs` -- several projections
  that read the same input joined into one along the output dimension
  (q/k/v, gate/up), as the reference's Marlin loader merges them
  (``operators/assemble/decoders/real_loader_marlin.py:61-79``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Sequence, Tuple

import torch


@dataclass(frozen=True)
class GptqGeometry:
    in_features: int
    out_features: int
    group_size: int
    act_order: bool

    @property
    def groups(self) -> int:
        return math.ceil(self.in_features / self.group_size)

    @classmethod
    def resolve(cls, in_features: int, out_features: int, group_size: int,
                act_order: bool, *, single_group_act: bool = True) -> "GptqGeometry":
        """Group size -1 is one group over every input row.  With
        ``single_group_act=False`` act-order is dropped when there is only one
        group (the row order then cannot matter; the Marlin path's rule)."""
        g = in_features if group_size == -1 else group_size
        act = bool(act_order) and (single_group_act or g < in_features)
        return cls(in_features, out_features, g, act)

    def require_exllama(self) -> "GptqGeometry":
        for ok, what in ((self.in_features % 32 == 0, "in_features must be a multiple of 32"),
                         (self.in_features % self.group_size == 0,
                          "in_features must be a multiple of group_size"),
                         (self.out_features % 32 == 0, "out_features must be a multiple of 32")):
            if not ok:
                raise AssertionError(what)
        return self

    def require_marlin(self, bias: bool) -> "GptqGeometry":
        problems = []
        if bias:
            problems.append("a Marlin-path projection has no bias")
        if self.in_features % 32 or self.out_features % 32:
            problems.append(f"{self.in_features} x {self.out_features} is not a multiple of 32 "
                            "in both dimensions")
        if self.in_features % self.group_size:
            problems.append(f"group size {self.group_size} does not divide {self.in_features} "
                            "input rows")
        if problems:
            raise ValueError("; ".join(problems))
        return self


def checkpoint_buffers(geo: GptqGeometry) -> Dict[str, torch.Tensor]:
    """Zero checkpoint tensors of one projection, by buffer name: qweight
    int32 [K/8, N] (8 rows per word), qzeros int32 [G, N/8] (8 columns per
    word), scales fp16 [G, N] and g_idx int32 [K] = k // group_size."""
    k, n, g = geo.in_features, geo.out_features, geo.groups
    return {
        "qweight": torch.zeros((k // 8, n), dtype=torch.int32),
        "qzeros": torch.zeros((g, n // 8), dtype=torch.int32),
        "scales": torch.zeros((g, n), dtype=torch.float16),
        "g_idx": torch.div(torch.arange(k, dtype=torch.int32), geo.group_size,
                           rounding_mode="floor").to(torch.int32),
    }


def _signature(linear) -> Tuple[int, int, bool]:
    return (linear.infeatures, linear.group_size, bool(linear.use_act_order))


def check_mergeable(parts: Sequence, *, compare_rows: bool = True) -> None:
    """Raise ValueError unless the projections can be joined along N: the
    same input width, group size and act-order mode and (``compare_rows``)
    the same row grouping ``g_idx``, which the joined projection keeps."""
    if not parts:
        raise ValueError("merging needs at least one projection")
    first = _signature(parts[0])
    for i, p in enumerate(parts[1:], start=1):
        if _signature(p) != first:
            raise ValueError(f"projection {i} has (in_features, group_size, act_order) = "
                             f"{_signature(p)} but projection 0 has {first}")
        if compare_rows and not torch.equal(p.g_idx, parts[0].g_idx):
            raise ValueError(f"projection {i} groups its input rows differently from "
                             "projection 0 (g_idx)")


def concat_outputs(parts: Sequence) -> Dict[str, torch.Tensor]:
    """The checkpoint tensors of the joined projection: qweight, qzeros and
    scales side by side along N (the packings run along K for qweight and
    within 8-column words for qzeros, so whole columns move together when
    every N is a multiple of 8), and the shared g_idx."""
    check_mergeable(parts)
    joined = {name: torch.cat([getattr(p, name) for p in parts], dim=1).contiguous()
              for name in ("qweight", "qzeros", "scales")}
    joined["g_idx"] = parts[0].g_idx
    return joined
