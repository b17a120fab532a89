"""GPTQ 4-bit quantized Linear backed by the HIP W4A16 kernels.

Drop-in for the reference's ``operators/core/linear/real_quant.py`` (paths
relative to ``/root/reference/After-Revision-DROFELL``):

* ``QuantLinear.__init__`` registers the same buffers with the same names,
  shapes and dtypes (``real_quant.py:10-49``) so per-layer safetensors
  (``self_attn.q_proj.qweight`` ...) load unchanged through
  ``load_state_dict``;
* ``post_init(tuning_params, cache)`` repacks at load time
  (``real_quant.py:51-67``) and re-registers the packed tensors in place of
  the checkpoint ones (same shapes and byte counts), plus ``perm`` (int32
  [K] for act-order, else empty), as the reference's Marlin adapter does
  (``real_marlin.py:101-117``);
* ``forward(x)`` routes by ``requires_grad`` exactly like
  ``real_quant.py:104-108``;
* ``QuantLinearMaker`` keeps ``make_linear`` / ``post_init`` /
  ``set_tuning_param`` (``real_quant.py:111-138``).
"""
from __future__ import annotations

from typing import Callable, List, cast

import torch
from torch import nn

from hip_extends.w4a16 import (CacheV2, Q4ForwardOnlyLinearFunction, Q4LinearFunction,
                               Q4MatrixV2, TuningParams)

from ... import flags
from .gptq_layout import GptqGeometry, checkpoint_buffers
from .real import Linear, LinearMaker


class QuantLinear(Linear):
    def __init__(self, group_size: int, in_features: int, out_features: int, bias: bool,
                 use_act_order: bool):
        nn.Module.__init__(self)
        # the reference's asserts (AssertionError) on the resolved geometry
        geo = GptqGeometry.resolve(in_features, out_features, group_size,
                                   use_act_order).require_exllama()
        self.infeatures = in_features
        self.outfeatures = out_features
        self.use_act_order = use_act_order
        self.bits = 4
        self.group_size = geo.group_size
        self.maxq = 2 ** self.bits - 1
        for name, t in checkpoint_buffers(geo).items():
            self.register_buffer(name, t)
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16))
        else:
            self.bias = None
        self.q4_matrix: Q4MatrixV2 | None = None

    def post_init(self, tunning_params: TuningParams, cache: CacheV2):
        if self.qweight.device.type != "cuda" or self.qweight.device.index is None:
            raise AssertionError("QuantLinear.post_init needs the buffers on a HIP device")
        if self.q4_matrix is not None:
            raise RuntimeError("QuantLinear.post_init called twice")
        q4 = Q4MatrixV2(self.qweight, self.qzeros, self.scales,
                        self.infeatures, self.outfeatures,
                        self.g_idx if self.use_act_order else None, self.use_act_order,
                        tuning_params=tunning_params, cache=cache)
        # The packed tensors replace the checkpoint buffers (same sizes) so
        # swapping and memory accounting see one copy.
        self.qweight = q4.qweight
        self.qzeros = q4.qzeros
        self.scales = q4.scales
        self.register_buffer("perm", q4.perm)
        self.q4_matrix = q4
        if flags.RECONSTRUCTE_WEIGTH_FLOAT16:
            q4.reconstruct_weight(dtype=torch.float16)
        if flags.RECONSTRUCTE_WEIGTH_BFLOAT16:
            q4.reconstruct_weight(dtype=torch.bfloat16)

    def _apply(self, fn, recurse: bool = True):
        """Module moves (swap-out to host memory, swap-in to a device) carry
        the packed buffers; the matrix object is re-pointed at the moved
        copies (no repack), and matrices with equal act-order permutations
        share one device copy again."""
        super()._apply(fn, recurse)
        q4 = self.q4_matrix
        if q4 is not None:
            perm = self.perm
            if q4.perm_group is not None:
                perm = q4.perm_group.share(perm)
                self._buffers["perm"] = perm
            q4.rebind(self.qweight, self.qzeros, self.scales, perm)
        return self

    def _matrix(self) -> Q4MatrixV2:
        if self.q4_matrix is None:
            raise RuntimeError("QuantLinear must be post_init()-ed (repacked) before use")
        return self.q4_matrix

    def get_reconstruct_weights(self) -> torch.Tensor:
        """Dequantised fp16 weight [K, N] in checkpoint row order.

        Same value as the reference's ``get_reconstruct_weights``
        (``real_quant.py:69-102``), computed on the device from the packed
        buffers by the bit-exact HIP dequantiser.
        """
        return self._matrix().get_float16_weights_matrix_v2()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        q4 = self._matrix()
        if x.requires_grad:
            return cast(torch.Tensor, Q4LinearFunction.apply(
                x, q4, self.bias, flags.REUSE_RECONSTRUCT_CACHE_WHEN_GRAD))
        return cast(torch.Tensor, Q4ForwardOnlyLinearFunction.apply(x, q4, self.bias))


class QuantLinearMaker(LinearMaker):
    def __init__(self, quantization_group_size: int, use_act_order: bool) -> None:
        self.quantization_group_size = quantization_group_size
        self.use_act_order = use_act_order
        self.quant_linears: List[QuantLinear] = []
        self.post_inited: bool = False

    def _apply(self, func: Callable[[QuantLinear], None]):
        for linear in self.quant_linears:
            func(linear)
        return self

    def post_init(self, tunning_params: TuningParams, shared_cache: CacheV2):
        if self.post_inited:
            raise AssertionError("QuantLinearMaker.post_init called twice")
        self.post_inited = True
        self._apply(lambda quant_linear: quant_linear.post_init(tunning_params, shared_cache))
        return self

    def set_tuning_param(self, tuning_param: TuningParams):
        self._apply(lambda quant_linear: quant_linear._matrix().set_tuning_params(tuning_param))
        return self

    def make_linear(self, in_features: int, out_features: int, bias: bool = False) -> QuantLinear:
        linear = QuantLinear(group_size=self.quantization_group_size,
                             in_features=in_features, out_features=out_features,
                             bias=bias, use_act_order=self.use_act_order)
        self.quant_linears.append(linear)
        return linear
