"""Marlin-path quantized Linear: the reference's API on the HIP W4A16 kernels.

The reference (``operators/core/linear/real_marlin.py``, paths relative to
``/root/reference/After-Revision-DROFELL``) keeps a second Linear front end
for its Marlin backend: the same GPTQ checkpoint buffers, no bias, a
per-matrix lock workspace, merged q/k/v and gate/up projections, and a
forward that runs the packed GEMM below a token threshold and a dense GEMM
over the reconstructed weight above it.  Here both front ends drive one
library: :class:`MarlinQuantLinear` hands its checkpoint tensors to
:class:`~hip_extends.marlin.MarlinQ4Matrix`, which repacks them into this
library's layout (not Marlin's tiles) and owns the dispatch.

What stays the reference's, because callers and checkpoints depend on it:
the class and method names and signatures (``make_linear``, ``post_init``,
``set_tuning_param``, ``merge``, ``reconstruct_weight``, ``dense_forward``,
``forward``), the buffer names a module exposes after ``post_init``, and
the exception types.  The geometry checks and buffer construction are shared
with :class:`~operators.core.linear.real_quant.QuantLinear`
(:mod:`operators.core.linear.gptq_layout`); the tensors a repacked module
holds are listed once, in :func:`hip_extends.marlin.marlin_module_tensors`.
"""
from __future__ import annotations

from typing import List, Optional, cast

import torch
from torch import nn

from hip_extends.marlin import (MarlinDenseCache, MarlinQ4ForwardOnlyLinearFunction,
                                MarlinQ4LinearFunction, MarlinQ4Matrix, MarlinTuningParams,
                                make_marlin_workspace)

from ... import flags
from .gptq_layout import GptqGeometry, checkpoint_buffers, concat_outputs
from .real import Linear, LinearMaker


def _marlin_forward(matrix: MarlinQ4Matrix, x: torch.Tensor) -> torch.Tensor:
    """The Marlin path computes in the scales' dtype (fp16) and returns the
    caller's dtype; a grad-tracking input goes through the autograd function,
    which may keep the reconstructed weight for its backward."""
    x16 = x.to(matrix.scales.dtype)
    if torch.is_grad_enabled() and x16.requires_grad:
        keep = matrix.tuning_params.reuse_reconstruct_cache(flags.REUSE_RECONSTRUCT_CACHE_WHEN_GRAD)
        y = MarlinQ4LinearFunction.apply(x16, matrix, keep)
    else:
        y = MarlinQ4ForwardOnlyLinearFunction.apply(x16, matrix)
    return cast(torch.Tensor, y).to(x.dtype)


class MarlinQuantLinear(Linear):
    """One GPTQ projection on the Marlin-path interface (reference
    ``real_marlin.py:24-157``)."""

    def __init__(self, group_size: int, in_features: int, out_features: int, bias: bool,
                 use_act_order: bool) -> None:
        nn.Module.__init__(self)
        geo = GptqGeometry.resolve(in_features, out_features, group_size, use_act_order,
                                   single_group_act=False).require_marlin(bias)
        self.infeatures, self.outfeatures = geo.in_features, geo.out_features
        self.group_size, self.use_act_order = geo.group_size, geo.act_order
        for name, t in checkpoint_buffers(geo).items():
            self.register_buffer(name, t)
        self.register_buffer("workspace", make_marlin_workspace(self.qweight.device),
                             persistent=False)
        self.bias = None
        self.q4_matrix: Optional[MarlinQ4Matrix] = None

    def post_init(self, tuning_params: MarlinTuningParams, cache: MarlinDenseCache) -> None:
        """Repack the loaded checkpoint tensors; the module then holds the
        matrix's runtime tensors under the reference's buffer names (one copy
        of each, so moves and memory accounting see what the kernels use)."""
        if self.q4_matrix is not None:
            raise RuntimeError(f"{type(self).__name__} is repacked already")
        matrix = MarlinQ4Matrix(self.qweight, self.qzeros, self.scales, self.infeatures,
                                self.outfeatures, self.g_idx, self.use_act_order, self.workspace,
                                tuning_params, cache)
        for name in MarlinQ4Matrix._MOVED:
            self.register_buffer(name, getattr(matrix, name),
                                 persistent=name not in self._non_persistent_buffers_set)
        self.q4_matrix = matrix

    def _apply(self, fn, recurse: bool = True):
        """A module move carries the repacked buffers; the matrix is pointed
        at the moved copies (nothing is repacked)."""
        super()._apply(fn, recurse)
        if self.q4_matrix is not None:
            self.q4_matrix.rebind(**{name: self._buffers[name] for name in MarlinQ4Matrix._MOVED})
        return self

    def _matrix(self) -> MarlinQ4Matrix:
        matrix = self.q4_matrix
        if matrix is None:
            raise RuntimeError(f"{type(self).__name__}.post_init() has not repacked the weights")
        return matrix

    @property
    def tuning_params(self) -> MarlinTuningParams:
        return self._matrix().tuning_params

    def reconstruct_weight(self, output: torch.Tensor) -> torch.Tensor:
        return self._matrix().reconstruct_weight(output)

    def dense_forward(self, x: torch.Tensor, dense_weight: torch.Tensor) -> torch.Tensor:
        return self._matrix().dense_matmul(x, dense_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _marlin_forward(self._matrix(), x)


class MarlinQuantLinearMaker(LinearMaker):
    """Makes the Marlin-path projections of a decoder group, merges those
    that share an input, and repacks them all in ``post_init`` (reference
    ``real_marlin.py:160-244``)."""

    def __init__(self, quantization_group_size: int, use_act_order: bool) -> None:
        self.quantization_group_size = quantization_group_size
        self.use_act_order = use_act_order
        self.quant_linears: List[MarlinQuantLinear] = []
        self.post_inited = False

    def make_linear(self, in_features: int, out_features: int,
                    bias: bool = False) -> MarlinQuantLinear:
        made = MarlinQuantLinear(self.quantization_group_size, in_features, out_features, bias,
                                 self.use_act_order)
        self.quant_linears.append(made)
        return made

    def post_init(self, tuning_params: MarlinTuningParams,
                  shared_cache: MarlinDenseCache) -> "MarlinQuantLinearMaker":
        if self.post_inited or not self.quant_linears:
            raise RuntimeError("MarlinQuantLinearMaker.post_init: " + (
                "already ran" if self.post_inited else "no projections were made"))
        self.post_inited = True
        for linear in self.quant_linears:
            linear.post_init(tuning_params, shared_cache)
        return self

    def set_tuning_param(self, tuning_params: MarlinTuningParams) -> "MarlinQuantLinearMaker":
        for linear in self.quant_linears:
            linear._matrix().set_tuning_params(tuning_params)
        return self

    def merge(self, linears: List[MarlinQuantLinear]) -> MarlinQuantLinear:
        """One projection whose outputs are the given projections' outputs in
        order; it replaces them in this maker.  Call before ``post_init``
        (the joining works on checkpoint tensors)."""
        joined = concat_outputs(linears)
        width = sum(linear.outfeatures for linear in linears)
        with torch.device(joined["qweight"].device):  # the workspace is a device buffer
            merged = self.make_linear(linears[0].infeatures, width, bias=False)
        for name, t in joined.items():
            setattr(merged, name, t)
        gone = {id(linear) for linear in linears}
        self.quant_linears = [lin for lin in self.quant_linears if id(lin) not in gone]
        return merged
