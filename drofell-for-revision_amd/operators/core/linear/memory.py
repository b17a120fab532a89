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

One more twin has no module behind it: :class:`W4A16LibraryMemoryModel`,
the fixed scratch array of ``dw4_gemm_noalloc``, which the library's code
object carries and which every GPU that runs the library holds once, from
the library's first use on it until the process ends, whether or not that
entry point is ever called.  A per-device plan mounts exactly one.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Callable, List, Optional

import torch

from hip_extends import _lib
from hip_extends.marlin import DenseRoutePlan, MarlinTuningParams, marlin_module_tensors
from hip_extends.w4a16 import TuningParams

from ... import flags
from ..memory.static import MemoryInt32, MemoryModule, MemoryTensor, MemoryUInt8
from .gptq_layout import GptqGeometry, check_mergeable, checkpoint_buffers

# CUs of an MI355X: the Marlin per-matrix workspace holds four int32 per CU
MI355X_CUS = 256


class LinearMakerMemoryModel(ABC):
    @abstractmethod
    def make_linear(self, in_features: int, out_features: int, bias: bool) -> MemoryModule:
        raise NotImplementedError


def _workspace_bytes(k: int, n: int, group_size: int, act: bool, max_m: int) -> int:
    return _lib.query_sizes(k, n, group_size, act, max(1, max_m))["workspace"]


class W4A16LibraryMemoryModel(MemoryModule):
    """Twin of the library's per-GPU static device memory: the
    ``DW4_NOALLOC_SCRATCH_BYTES`` array of ``dw4_gemm_noalloc`` (mount one per
    device that runs the library, beside the decoder groups' twins)."""

    def __init__(self) -> None:
        super().__init__()
        self.noalloc_scratch = MemoryTensor((_lib.NOALLOC_SCRATCH_BYTES,), MemoryUInt8)


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
        geo = GptqGeometry.resolve(in_features, out_features, group_size,
                                   use_act_order).require_exllama()
        self.infeatures = in_features
        self.outfeatures = out_features
        self.use_act_order = use_act_order
        self.bits = 4
        self.group_size = geo.group_size
        for name, t in checkpoint_buffers(geo).items():
            setattr(self, name, MemoryTensor(tuple(t.shape), t.dtype))
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
    """Twin of a repacked ``MarlinQuantLinear``: one :class:`MemoryTensor` per
    buffer the module holds after ``post_init``, taken from the same table
    the module is built from (:func:`hip_extends.marlin.marlin_module_tensors`)."""

    def __init__(self, group_size: int, in_features: int, out_features: int, bias: bool,
                 use_act_order: bool, workspace_elements: int = MI355X_CUS * 4) -> None:
        super().__init__()
        geo = GptqGeometry.resolve(in_features, out_features, group_size, use_act_order,
                                   single_group_act=False).require_marlin(bias)
        self.infeatures, self.outfeatures = geo.in_features, geo.out_features
        self.group_size, self.use_act_order = geo.group_size, geo.act_order
        for name, (shape, dtype) in marlin_module_tensors(
                geo.in_features, geo.out_features, geo.group_size, geo.act_order,
                workspace_elements).items():
            setattr(self, name, MemoryTensor(shape, dtype))


class MarlinDenseCacheMemoryModel(MemoryModule):
    """Twin of ``MarlinDenseCache``, sized by the same :class:`DenseRoutePlan`:
    the reconstruction buffer and the split-K workspace of a decoder group."""

    def __init__(self) -> None:
        super().__init__()
        self.plan = DenseRoutePlan()

    @property
    def cache_created(self) -> bool:
        return self.plan.allocated

    @property
    def temp_weight_elements(self) -> int:
        return self.plan.weight_elements

    @property
    def workspace_bytes(self) -> int:
        return self.plan.workspace_bytes

    def update(self, in_features: int, out_features: int, workspace_bytes: int = 0) -> None:
        self.plan.grow(in_features, out_features, workspace_bytes)

    def init_cache(self) -> None:
        self.plan.allocate()
        self._temp_weight = MemoryTensor((self.plan.weight_elements,), torch.float16)
        self._workspace = MemoryTensor((max(self.plan.workspace_bytes, 16),), MemoryUInt8)


class MarlinQuantLinearMakerMemoryModel(LinearMakerMemoryModel):
    """Twin of ``MarlinQuantLinearMaker``: the group's projections and its
    dense cache; every projection registers its dense-route sizes as it is
    made, and ``post_init`` fixes them."""

    def __init__(self, quantization_group_size: int, use_act_order: bool,
                 workspace_elements: int = MI355X_CUS * 4,
                 tuning_params: Optional[MarlinTuningParams] = None) -> None:
        self.quantization_group_size = quantization_group_size
        self.use_act_order = use_act_order
        self.workspace_elements = workspace_elements
        self.tuning_params = tuning_params if tuning_params is not None else MarlinTuningParams()
        self.dense_cache = MarlinDenseCacheMemoryModel()
        self.quant_linears: List[MarlinQuantLinearMemoryModel] = []
        self.post_inited = False

    def make_linear(self, in_features: int, out_features: int,
                    bias: bool = False) -> MarlinQuantLinearMemoryModel:
        twin = MarlinQuantLinearMemoryModel(self.quantization_group_size, in_features,
                                            out_features, bias, self.use_act_order,
                                            self.workspace_elements)
        self.dense_cache.update(in_features, out_features, _workspace_bytes(
            in_features, out_features, twin.group_size, twin.use_act_order,
            self.tuning_params.direct_max_m()))
        self.quant_linears.append(twin)
        return twin

    def post_init(self) -> None:
        if self.post_inited:
            raise RuntimeError("MarlinQuantLinearMakerMemoryModel.post_init: already ran")
        self.post_inited = True
        self.dense_cache.init_cache()

    def merge(self, linears: List[MarlinQuantLinearMemoryModel]) -> MarlinQuantLinearMemoryModel:
        """The twin of a merged projection (the checkpoint tensors it would
        join are not modelled, so only the shapes are checked)."""
        check_mergeable(linears, compare_rows=False)
        merged = self.make_linear(linears[0].infeatures,
                                  sum(linear.outfeatures for linear in linears), False)
        gone = {id(linear) for linear in linears}
        self.quant_linears = [t for t in self.quant_linears if id(t) not in gone]
        return merged
