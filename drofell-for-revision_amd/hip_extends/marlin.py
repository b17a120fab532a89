"""The reference's Marlin-backend objects, backed by the HIP W4A16 library.

Mirrors ``cuda_extends/marlin.py`` (paths relative to
``/root/reference/After-Revision-DROFELL``):

* :class:`MarlinTuningParams` -- ``marlin.py:18-53`` (the same fields and
  flattened-M rule; MI355X-measured defaults);
* :class:`MarlinDenseCache` -- ``marlin.py:56-87`` (the shared
  reconstruction buffer; here also the dw4_gemm split-K workspace, both
  sized by :class:`DenseRoutePlan`);
* :func:`make_marlin_workspace` -- ``marlin.py:90-96``;
* :class:`MarlinQ4Matrix` -- ``marlin.py:190-363`` (load-time repack,
  direct / reconstruct-then-dense dispatch, dequantisation, transposed
  product);
* :class:`MarlinQ4LinearFunction`, :class:`MarlinQ4ForwardOnlyLinearFunction`
  -- ``marlin.py:366-413``.

The packed layout is this library's (see ``include/drofell_w4a16.h``), not
Marlin's tile layout: ``direct_matmul`` is ``dw4_gemm`` and
``reconstruct_weight`` is ``dw4_dequant``.  Like the reference, the matrix
accepts only symmetric GPTQ weights (every stored zero nibble 7, i.e.
``qzeros == 0x77777777``); the packed zero words are kept, so the kernels
are the same ones the asymmetric ``Q4MatrixV2`` uses.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
from torch.autograd import Function

from . import _lib
from .w4a16 import _aligned_rows, _ptr, _stream

_SYMMETRIC_ZEROS = 0x77777777 - (1 << 32)  # int32 view of the word


@dataclass(frozen=True)
class MarlinTuningParams:
    """Where the Marlin-path forward leaves the packed W4A16 kernel for the
    dense route (dequantise, then a library GEMM), by flattened token count.

    ``reconstruct_threshold`` serves inference and PEFT without a kept
    weight; ``grad_reconstruct_threshold`` serves PEFT that keeps the
    reconstructed weight for its backward (the forward then costs only the
    library GEMM).  ``None`` keeps that case on the packed kernel at every
    size.  The defaults are MI355X crossovers measured over the 56 Llama-2-7B
    projections of the bench (``bench.py --crossover``, ms per pass), not the
    reference's RTX 3090 ones:

    * no kept weight, packed / dequantise + GEMM: M=2048 7.12 / 9.21,
      M=4096 14.32 / 12.86, M=8192 28.49 / 23.59 -> dense from 4096 tokens;
    * kept weight, forward + activation gradient, packed / dense: M=512
      6.32 / 6.44, M=768 8.23 / 7.61, M=1024 9.20 / 8.57, M=2048
      14.64 / 15.19, M=4096 26.80 / 23.15 -> dense from 768 tokens (4% slower
      at 2048, 7-16% faster at every other size measured above it).
    """

    reconstruct_threshold: Optional[int] = 4096
    grad_reconstruct_threshold: Optional[int] = 768
    reuse_reconstruct_cache_when_grad: Optional[bool] = None

    def __post_init__(self) -> None:
        bad = {name: v for name, v in (("reconstruct_threshold", self.reconstruct_threshold),
                                       ("grad_reconstruct_threshold",
                                        self.grad_reconstruct_threshold))
               if v is not None and v < 1}
        if bad:
            raise ValueError(f"dense-route crossovers are token counts >= 1 or None, got {bad}")

    def _crossover(self, cache_weight: bool) -> Optional[int]:
        return self.grad_reconstruct_threshold if cache_weight else self.reconstruct_threshold

    def use_reconstructed_forward(self, flattened_tokens: int, *, cache_weight: bool) -> bool:
        at = self._crossover(cache_weight)
        return at is not None and flattened_tokens >= at

    def reuse_reconstruct_cache(self, default: bool) -> bool:
        keep = self.reuse_reconstruct_cache_when_grad
        return default if keep is None else keep

    def direct_max_m(self) -> int:
        """Largest flattened M the packed kernel is asked to run without a
        kept weight (sizes the shared split-K workspace)."""
        at = self.reconstruct_threshold
        return 4096 if at is None else max(1, at - 1)


class DenseRoutePlan:
    """Sizes of one decoder group's shared dense-route buffers: the
    reconstruction buffer (the largest K x N of the group, fp16) and the
    packed kernel's split-K workspace.  They grow while projections are
    registered and are fixed once allocated; :class:`MarlinDenseCache`
    allocates them and its memory twin mirrors them from the same plan."""

    def __init__(self) -> None:
        self.weight_elements = 0
        self.workspace_bytes = 0
        self.allocated = False

    def grow(self, in_features: int, out_features: int, workspace_bytes: int = 0) -> None:
        if self.allocated:
            raise RuntimeError("the dense-route buffers are allocated already: register every "
                               "projection before init_cache()")
        self.weight_elements = max(self.weight_elements, in_features * out_features)
        self.workspace_bytes = max(self.workspace_bytes, workspace_bytes)

    def allocate(self) -> None:
        if self.allocated:
            raise RuntimeError("init_cache() ran already for this dense cache")
        self.allocated = True


class MarlinDenseCache:
    """The shared, stream-ordered dense-route buffers of one decoder group
    (sized by :class:`DenseRoutePlan`), plus the transposed product's
    partial planes, grown on demand outside graph capture."""

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self.plan = DenseRoutePlan()
        self._buffers: Optional[tuple] = None
        self._t_workspace: Optional[torch.Tensor] = None

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
        weight = torch.empty(self.plan.weight_elements, dtype=torch.float16, device=self.device)
        # zero-filled once: the kernels keep split-K arrival counters at its
        # start and leave them at zero after every call
        ws = torch.zeros(max(self.plan.workspace_bytes, 16), dtype=torch.uint8, device=self.device)
        self._buffers = (weight, ws)

    def _allocated(self) -> tuple:
        if self._buffers is None:
            raise RuntimeError("MarlinDenseCache.init_cache() has not run")
        return self._buffers

    def weight(self, in_features: int, out_features: int) -> torch.Tensor:
        buf = self._allocated()[0]
        need = in_features * out_features
        if need > buf.numel():
            raise RuntimeError(f"a {in_features} x {out_features} weight does not fit the "
                               f"{buf.numel()}-element reconstruction buffer")
        return buf[:need].view(in_features, out_features)

    @property
    def workspace(self) -> torch.Tensor:
        return self._allocated()[1]

    def transpose_workspace(self, nbytes: int) -> torch.Tensor:
        t = self._t_workspace
        if t is None or t.numel() < nbytes:
            t = self._t_workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8,
                                                device=self.device)
        return t


def make_marlin_workspace(device: torch.device) -> torch.Tensor:
    """The per-matrix int32 buffer of 4 words per CU that the reference's
    Marlin GEMM uses for locks.  The HIP kernels keep their split-K state in
    the group's :class:`MarlinDenseCache`; the buffer is still created so the
    module's buffers and memory accounting keep the reference's shape."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"the Marlin-path workspace lives on the GPU, not on {device}")
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return torch.zeros(4 * cus, dtype=torch.int32, device=device)


def marlin_module_tensors(in_features: int, out_features: int, group_size: int,
                          act_order: bool, workspace_elements: int) -> dict:
    """(shape, dtype) of every tensor a Marlin-path module holds after
    ``post_init``, by buffer name: the packed matrix (the checkpoint's byte
    counts), the row-sorted ``g_idx`` and its sort indices (act-order only),
    the per-matrix workspace and the two reference dequantiser tables, which
    this layout does not need (empty)."""
    groups = in_features // group_size
    index = in_features if act_order else 0
    return {
        "qweight": ((in_features // 8, out_features), torch.int32),
        "qzeros": ((groups, out_features // 8), torch.int32),
        "scales": ((groups, out_features), torch.float16),
        "g_idx": ((index,), torch.int32),
        "g_idx_sort_indices": ((index,), torch.int32),
        "workspace": ((workspace_elements,), torch.int32),
        "dequant_weight_permutation": ((0,), torch.int32),
        "dequant_scale_column_map": ((0,), torch.int32),
    }


def _dense_matmul(x: torch.Tensor, weight: torch.Tensor, *,
                  transpose_weight: bool = False) -> torch.Tensor:
    w = weight.t() if transpose_weight else weight
    out_features = w.shape[1]
    y = torch.matmul(x.reshape(-1, w.shape[0]).to(torch.float16), w)
    return y.reshape(*x.shape[:-1], out_features)


class MarlinQ4Matrix:
    """One repacked symmetric GPTQ projection with the Marlin path's
    dispatch (packed kernel or dense route) and reconstruction."""

    def __init__(self, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                 in_features: int, out_features: int, g_idx: torch.Tensor,
                 use_act_order: bool, workspace: torch.Tensor,
                 tuning_params: MarlinTuningParams, cache: MarlinDenseCache) -> None:
        if qweight.device.type != "cuda":
            raise ValueError(f"the checkpoint tensors must be on the GPU, not {qweight.device}")
        if not bool(torch.all(qzeros == _SYMMETRIC_ZEROS).item()):
            raise ValueError("the Marlin path takes symmetric checkpoints only: every stored "
                             "zero nibble must be 7 (effective zero 8)")
        if workspace.device != qweight.device or workspace.dtype != torch.int32:
            raise ValueError(f"workspace is {workspace.dtype} on {workspace.device}; "
                             f"expected int32 on {qweight.device}")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = in_features // scales.shape[0]
        self.use_act_order = use_act_order and self.group_size < in_features
        self.tuning_params = tuning_params
        self.cache = cache
        self.workspace = workspace

        perm: Optional[torch.Tensor] = None
        if self.use_act_order:
            g_host = g_idx.detach().to("cpu", torch.int32).contiguous()
            perm_host = torch.empty(in_features, dtype=torch.int32)
            _lib.call("dw4_make_perm", in_features, self.group_size, g_host.data_ptr(),
                      perm_host.data_ptr())
            if not torch.equal(perm_host, torch.arange(in_features, dtype=torch.int32)):
                perm = perm_host.to(qweight.device)
        dev = qweight.device
        self.g_idx_sort_indices = perm if perm is not None else \
            torch.empty(0, dtype=torch.int32, device=dev)
        self.g_idx = g_idx.to(dev, torch.int32)[perm.long()] if perm is not None else \
            torch.empty(0, dtype=torch.int32, device=dev)
        self.qweight = torch.empty_like(qweight, memory_format=torch.contiguous_format)
        self.qzeros = torch.empty_like(qzeros, memory_format=torch.contiguous_format)
        self.scales = torch.empty_like(scales, memory_format=torch.contiguous_format)
        with torch.cuda.device(dev):
            _lib.call("dw4_repack", in_features, out_features, self.group_size,
                      qweight.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                      scales.contiguous().data_ptr(), _ptr(perm),
                      self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                      _stream(dev))
        # the reference's Marlin-only tables have no counterpart here
        self.dequant_weight_permutation = torch.empty(0, dtype=torch.int32, device=dev)
        self.dequant_scale_column_map = torch.empty(0, dtype=torch.int32, device=dev)
        sizes = _lib.query_sizes(in_features, out_features, self.group_size,
                                 perm is not None, tuning_params.direct_max_m())
        cache.update(in_features, out_features, sizes["workspace"])

    @property
    def _perm(self) -> Optional[torch.Tensor]:
        return self.g_idx_sort_indices if self.g_idx_sort_indices.numel() else None

    def set_tuning_params(self, tuning_params: MarlinTuningParams) -> None:
        self.tuning_params = tuning_params

    # the tensors a module move carries (every module buffer after post_init)
    _MOVED = tuple(marlin_module_tensors(8, 8, 8, False, 0))

    def rebind(self, **tensors: torch.Tensor) -> None:
        """Point the matrix at moved copies of its tensors (module swap-out
        and swap-in); nothing is repacked.  Products raise while the tensors
        are in host memory."""
        for name in self._MOVED:
            new, old = tensors[name], getattr(self, name)
            if new.shape != old.shape or new.dtype != old.dtype:
                raise ValueError(f"{name}: moved tensor does not match the packed one")
        devices = {tensors[name].device for name in self._MOVED}
        if len(devices) != 1:
            raise ValueError(f"Marlin tensors on several devices: {devices}")
        for name in self._MOVED:
            setattr(self, name, tensors[name])

    def _check_resident(self) -> None:
        if self.qweight.device.type != "cuda":
            raise RuntimeError("MarlinQ4Matrix is swapped out (its tensors are in host memory)")

    def use_reconstructed_forward(self, flattened_tokens: int, *, cache_weight: bool) -> bool:
        return self.tuning_params.use_reconstructed_forward(flattened_tokens,
                                                            cache_weight=cache_weight)

    def reconstruct_weight(self, output: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Bit-exact fp16 weight [K, N] in checkpoint row order."""
        self._check_resident()
        if output is None:
            output = torch.empty((self.in_features, self.out_features), dtype=torch.float16,
                                 device=self.qweight.device)
        if output.dtype != torch.float16 or tuple(output.shape) != (self.in_features,
                                                                   self.out_features):
            raise ValueError("output must be fp16 [in_features, out_features]")
        _lib.call("dw4_dequant", self.in_features, self.out_features, self.group_size,
                  self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                  _ptr(self._perm), output.data_ptr(), output.stride(0),
                  _stream(self.qweight.device))
        return output

    def direct_matmul(self, x: torch.Tensor) -> torch.Tensor:
        """The packed W4A16 kernel: fp16 [..., K] -> fp16 [..., N]."""
        self._check_resident()
        x_2d = _aligned_rows(x.reshape(-1, self.in_features).to(torch.float16))
        m = x_2d.shape[0]
        output = torch.empty((m, self.out_features), dtype=torch.float16, device=x.device)
        ws = self.cache.workspace
        lib = _lib.load()
        _lib.check("dw4_gemm", lib.dw4_gemm(
            m, self.in_features, self.out_features, self.group_size,
            x_2d.data_ptr(), x_2d.stride(0),
            self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
            _ptr(self._perm), None, output.data_ptr(), self.out_features,
            ws.data_ptr(), ws.numel(), _stream(x.device)))
        return output.reshape(*x.shape[:-1], self.out_features)

    def dense_matmul(self, x: torch.Tensor, weight: torch.Tensor, *,
                     transpose_weight: bool = False) -> torch.Tensor:
        return _dense_matmul(x, weight, transpose_weight=transpose_weight)

    def forward_matmul(self, x: torch.Tensor, *, cache_weight: bool):
        flattened_tokens = x.numel() // self.in_features
        if not self.use_reconstructed_forward(flattened_tokens, cache_weight=cache_weight):
            return self.direct_matmul(x), None
        weight = self.reconstruct_weight() if cache_weight else \
            self.cache.weight(self.in_features, self.out_features)
        if not cache_weight:
            self.reconstruct_weight(weight)
        return self.dense_matmul(x, weight), weight if cache_weight else None

    # flattened rows up to which the activation gradient reads the packed
    # words directly (dw4_gemm_t) instead of a reconstructed dense weight
    TRANSPOSE_MAX_M = 128

    def transpose_matmul(self, x: torch.Tensor,
                         weight: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``x @ W.T`` for x [..., N]: with ``weight`` (a reconstructed fp16
        [K, N]) the dense product; otherwise, up to ``TRANSPOSE_MAX_M`` rows,
        the packed kernel, above it reconstruct-then-dense as the reference
        (``marlin.py:355-396``)."""
        self._check_resident()
        m = x.numel() // self.out_features
        if weight is None and 0 < m <= self.TRANSPOSE_MAX_M:
            g2 = _aligned_rows(x.reshape(-1, self.out_features).to(torch.float16))
            out = torch.empty((m, self.in_features), dtype=torch.float16, device=x.device)
            nbytes = _lib.gemm_t_workspace_size(m, self.in_features, self.out_features,
                                                self.group_size)
            ws = self.cache.transpose_workspace(nbytes)
            _lib.call("dw4_gemm_t", m, self.in_features, self.out_features, self.group_size,
                      g2.data_ptr(), g2.stride(0), self.qweight.data_ptr(),
                      self.qzeros.data_ptr(), self.scales.data_ptr(), _ptr(self._perm),
                      out.data_ptr(), self.in_features, ws.data_ptr(), ws.numel(),
                      _stream(x.device))
            return out.reshape(*x.shape[:-1], self.in_features)
        if weight is None:
            weight = self.cache.weight(self.in_features, self.out_features)
            self.reconstruct_weight(weight)
        return self.dense_matmul(x, weight, transpose_weight=True)


class MarlinQ4LinearFunction(Function):
    """Autograd for a frozen matrix; only the activation has a gradient."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, q4_matrix: MarlinQ4Matrix,  # type: ignore[override]
                cache_weight: bool) -> torch.Tensor:
        output, cached_weight = q4_matrix.forward_matmul(x, cache_weight=cache_weight)
        ctx.q4_matrix = q4_matrix
        ctx.x_dtype = x.dtype
        if cached_weight is None:
            ctx.save_for_backward()
        else:
            ctx.save_for_backward(cached_weight)
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):  # type: ignore[override]
        q4_matrix: MarlinQ4Matrix = ctx.q4_matrix
        cached_weight = ctx.saved_tensors[0] if ctx.saved_tensors else None
        grad_x = q4_matrix.transpose_matmul(
            grad_output.to(q4_matrix.scales.dtype).contiguous(), cached_weight).to(ctx.x_dtype)
        return grad_x, None, None


class MarlinQ4ForwardOnlyLinearFunction(Function):
    """Forward-only wrapper matching the ExLlama backend interface."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, q4_matrix: MarlinQ4Matrix) -> torch.Tensor:  # type: ignore[override]
        output, _ = q4_matrix.forward_matmul(x, cache_weight=False)
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):  # type: ignore[override]
        raise RuntimeError("MarlinQ4ForwardOnlyLinearFunction has no backward")
