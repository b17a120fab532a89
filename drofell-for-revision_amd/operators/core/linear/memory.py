"""Memory twins of the quantized linears and their shared caches.

Mirrors ``operators/core/linear/memory.py`` of the reference (paths relative
to ``/root/reference/After-Revision-DROFELL``): ``CacheV2MemoryModel``,
``QuantLinearMemoryModel`` and ``QuantLinearMakerMemoryModel`` (``:18-90``),
``MarlinQuantLinearMemoryModel``, ``MarlinDenseCacheMemoryModel`` and
``MarlinQuantLinearMakerMemoryModel`` (``:93-217``), with the same
constructor arguments and methods.  Each twin holds one
:class:`MemoryTensor` per device tensor that the HIP-backed module keeps after
``post_init``:

* ``QuantLinear``: the packed ``qweight`` / ``qzeros`` / ``scales`` (same
  shapes and bytes as the checkpoint buffers they replace), ``g_idx``, the
  optional ``bias``, ``perm`` (int32 [K] with act-order, else empty; matrices
  with equal permutations share one device tensor, which
  :meth:`QuantLinearMakerMemoryModel.share_perm` expresses) and, when
  ``flags.RECONSTRUCTE_WEIGTH_FLOAT16`` is set, the fp16 [K, N] weight;
* ``CacheV2``: the zero-filled workspace (its size from ``dw4_query_sizes``,
  the largest over the group) and, once requested, the fp16 ``temp_weight``
  of the dense route;
* the Marlin path: the same packed buffers (the zero words stay: the kernels
  serve asymmetric weights too), the sorted ``g_idx`` and
  ``g_idx_sort_indices`` (act-order only), the per-matrix int32 workspace of
  CUs x 4, and the group's dense cache (fp16 K x N plus the workspace).

The workspace sizes come from the library's host-only sizing call, so the
twins need ``libdrofell_w4a16.so`` but no GPU.
"""
from __future__ import annotations

import math
from abc import ABC, abstractmethod
from typing import Callable, List, Optional

import torch

from hip_extends import _lib
from hip_extends.marlin import MarlinTuningParams
from hip_extends.w4a16 import TuningParams

from ... import flags
from ..memory.static import MemoryInt32, MemoryModule, MemoryTensor, MemoryUInt8

# CUs of an MI355X: the Marlin per-matrix workspace holds four int32 per CU
MI355X_CUS = 256


class LinearMakerMemoryModel(ABC):
    @abstractmethod
    def make_linear(self, in_features: int, out_features: int, bias: bool) -> MemoryModule:
        raise NotImplementedError


def _workspace_bytes(k: int, n: int, group_size: int, act: bool, max_m: int) -> int:
    return _lib.query_sizes(k, n, group_size, act, max(1, max_m))["workspace"]


class CacheV2MemoryModel(MemoryModule):
    """Twin of ``CacheV2``: one workspace per decoder group, and the fp16
    dense-route buffer once something asks for it."""

    def __init__(self) -> None:
        super().__init__()
        self.workspace_size: int = 0
        self.temp_weight_size: int = 0
        self._workspace: Optional[MemoryTensor] = None
        self._temp_weight: Optional[MemoryTensor] = None
        self.cache_created = False

    def update_workspace_size(self, nbytes: int) -> None:
        if nbytes > self.workspace_size:
            self.cache_created = False
            self.workspace_size = nbytes

    def update_temp_weight_size(self, elements: int) -> None:
        if elements > self.temp_weight_size:
            self.temp_weight_size = elements
            self._temp_weight = None

    def init_cache(self) -> None:
        self._workspace = MemoryTensor((max(self.workspace_size, 16),), MemoryUInt8)
        self.cache_created = True

    @property
    def workspace(self) -> MemoryTensor:
        if not self.cache_created or self._workspace is None:
            raise RuntimeError("CacheV2MemoryModel.init_cache() must run first")
        return self._workspace

    @property
    def temp_weight(self) -> MemoryTensor:
        if self._temp_weight is None:
            self._temp_weight = MemoryTensor((1, self.temp_weight_size), torch.float16)
        return self._temp_weight


class QuantLinearMemoryModel(MemoryModule):
    def __init__(self, group_size: int, in_features: int, out_features: int, bias: bool,
                 use_act_order: bool) -> None:
        super().__init__()
        self.infeatures = in_features
        self.outfeatures = out_features
        self.use_act_order = use_act_order
        self.bits = 4
        self.group_size = group_size if group_size != -1 else in_features
        if in_features % 32 != 0:
            raise AssertionError("in_features must be a multiple of 32")
        if in_features % self.group_size != 0:
            raise AssertionError("in_features must be a multiple of group_size")
        if out_features % 32 != 0:
            raise AssertionError("out_features must be a multiple of 32")
        groups = math.ceil(in_features / self.group_size)
        self.qweight = MemoryTensor((in_features // 32 * self.bits, out_features), MemoryInt32)
        self.qzeros = MemoryTensor((groups, out_features // 32 * self.bits), MemoryInt32)
        self.scales = MemoryTensor((groups, out_features), torch.float16)
        self.g_idx = MemoryTensor((in_features,), MemoryInt32)
        if bias:
            self.bias = MemoryTensor((out_features,), torch.float16)
        self.cache_v2: Optional[CacheV2MemoryModel] = None

    def post_init(self, tunning_params: TuningParams, cache: CacheV2MemoryModel) -> None:
        self.cache_v2 = cache
        self.perm = MemoryTensor((self.infeatures if self.use_act_order else 0,), MemoryInt32)
        if flags.RECONSTRUCTE_WEIGTH_FLOAT16:
            self.reconstructed_weight = MemoryTensor((self.infeatures, self.outfeatures),
                                                     torch.float16)
        if flags.RECONSTRUCTE_WEIGTH_BFLOAT16:
            self.reconstructed_weight_bfloat16 = MemoryTensor(
                (self.infeatures, self.outfeatures), torch.bfloat16)
        cache.update_workspace_size(_workspace_bytes(
            self.infeatures, self.outfeatures, self.group_size, self.use_act_order,
            tunning_params.MAX_M))
        cache.update_temp_weight_size(self.infeatures * self.outfeatures)


class QuantLinearMakerMemoryModel(LinearMakerMemoryModel):
    def __init__(self, quantization_group_size: int, use_act_order: bool) -> None:
        self.quantization_group_size = quantization_group_size
        self.use_act_order = use_act_order
        self.post_inited: bool = False
        self.quant_linears: List[QuantLinearMemoryModel] = []

    def make_linear(self, in_features: int, out_features: int,
                    bias: bool = False) -> QuantLinearMemoryModel:
        linear = QuantLinearMemoryModel(group_size=self.quantization_group_size,
                                        in_features=in_features, out_features=out_features,
                                        bias=bias, use_act_order=self.use_act_order)
        self.quant_linears.append(linear)
        return linear

    def _apply(self, func: Callable[[QuantLinearMemoryModel], None]):
        for linear in self.quant_linears:
            func(linear)
        return self

    def post_init(self, tunning_params: TuningParams, shared_cache: CacheV2MemoryModel):
        if self.post_inited:
            raise AssertionError("QuantLinearMakerMemoryModel.post_init called twice")
        self.post_inited = True
        self._apply(lambda quant_linear: quant_linear.post_init(tunning_params, shared_cache))
        return self

    @staticmethod
    def share_perm(linears: List[QuantLinearMemoryModel]) -> None:
        """Linears quantised against the same input (q/k/v; gate/up) have
        equal act-order permutations, which the device keeps once."""
        if not linears or linears[0].cache_v2 is None:
            raise AssertionError("share_perm needs post_init()-ed linears")
        first = linears[0].perm
        for linear in linears[1:]:
            if linear.infeatures != linears[0].infeatures:
                raise ValueError("linears sharing a permutation must share in_features")
            linear.perm = first


class MarlinQuantLinearMemoryModel(MemoryModule):
    """Long-lived tensors of one Marlin-path projection after ``post_init``."""

    def __init__(self, group_size: int, in_features: int, out_features: int, bias: bool,
                 use_act_order: bool, workspace_elements: int = MI355X_CUS * 4) -> None:
        super().__init__()
        if bias:
            raise ValueError("the Marlin memory model does not support bias")
        if in_features % 32 != 0 or out_features % 32 != 0:
            raise ValueError("Marlin GPTQ dimensions must be multiples of 32")
        self.infeatures = in_features
        self.outfeatures = out_features
        self.group_size = in_features if group_size == -1 else group_size
        self.use_act_order = use_act_order and self.group_size < in_features
        groups = math.ceil(in_features / self.group_size)
        self.qweight = MemoryTensor((in_features // 8, out_features), MemoryInt32)
        self.qzeros = MemoryTensor((groups, out_features // 8), MemoryInt32)
        self.scales = MemoryTensor((groups, out_features), torch.float16)
        index = in_features if self.use_act_order else 0
        self.g_idx = MemoryTensor((index,), MemoryInt32)
        self.g_idx_sort_indices = MemoryTensor((index,), MemoryInt32)
        self.workspace = MemoryTensor((workspace_elements,), MemoryInt32)
        self.dequant_weight_permutation = MemoryTensor((0,), MemoryInt32)
        self.dequant_scale_column_map = MemoryTensor((0,), MemoryInt32)


class MarlinDenseCacheMemoryModel(MemoryModule):
    """Twin of ``MarlinDenseCache``: one fp16 reconstruction buffer and one
    GEMM workspace per decoder group."""

    def __init__(self) -> None:
        super().__init__()
        self.temp_weight_elements = 0
        self.workspace_bytes = 0
        self._temp_weight: Optional[MemoryTensor] = None
        self._workspace: Optional[MemoryTensor] = None
        self.cache_created = False

    def update(self, in_features: int, out_features: int, workspace_bytes: int = 0) -> None:
        if self.cache_created:
            raise RuntimeError("cannot resize initialized Marlin dense cache")
        self.temp_weight_elements = max(self.temp_weight_elements, in_features * out_features)
        self.workspace_bytes = max(self.workspace_bytes, workspace_bytes)

    def init_cache(self) -> None:
        if self.cache_created:
            raise RuntimeError("Marlin dense cache initialized twice")
        self._temp_weight = MemoryTensor((self.temp_weight_elements,), torch.float16)
        self._workspace = MemoryTensor((max(self.workspace_bytes, 16),), MemoryUInt8)
        self.cache_created = True


class MarlinQuantLinearMakerMemoryModel(LinearMakerMemoryModel):
    def __init__(self, quantization_group_size: int, use_act_order: bool,
                 workspace_elements: int = MI355X_CUS * 4,
                 tuning_params: Optional[MarlinTuningParams] = None) -> None:
        self.quantization_group_size = quantization_group_size
        self.use_act_order = use_act_order
        self.workspace_elements = workspace_elements
        self.tuning_params = tuning_params or MarlinTuningParams()
        self.dense_cache = MarlinDenseCacheMemoryModel()
        self.quant_linears: List[MarlinQuantLinearMemoryModel] = []
        self.post_inited = False

    def make_linear(self, in_features: int, out_features: int,
                    bias: bool = False) -> MarlinQuantLinearMemoryModel:
        linear = MarlinQuantLinearMemoryModel(
            group_size=self.quantization_group_size, in_features=in_features,
            out_features=out_features, bias=bias, use_act_order=self.use_act_order,
            workspace_elements=self.workspace_elements)
        self.quant_linears.append(linear)
        self.dense_cache.update(in_features, out_features, _workspace_bytes(
            in_features, out_features, linear.group_size, linear.use_act_order,
            self.tuning_params.direct_max_m()))
        return linear

    def post_init(self) -> None:
        if self.post_inited:
            raise RuntimeError("MarlinQuantLinearMakerMemoryModel.post_init called twice")
        self.post_inited = True
        self.dense_cache.init_cache()

    def merge(self, linears: List[MarlinQuantLinearMemoryModel]) -> MarlinQuantLinearMemoryModel:
        if not linears:
            raise ValueError("cannot merge an empty list of Marlin linears")
        first = linears[0]
        if any(linear.infeatures != first.infeatures for linear in linears):
            raise ValueError("merged Marlin linears must share in_features")
        merged = self.make_linear(first.infeatures,
                                  sum(linear.outfeatures for linear in linears), False)
        for linear in linears:
            self.quant_linears.remove(linear)
        return merged
