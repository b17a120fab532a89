"""The reference's Marlin-backend objects, backed by the HIP W4A16 library.

Mirrors ``cuda_extends/marlin.py`` (paths relative to
``/root/reference/After-Revision-DROFELL``):

* :class:`MarlinTuningParams` -- ``marlin.py:18-53`` (same fields, same
  flattened-M dispatch rule and validation);
* :class:`MarlinDenseCache` -- ``marlin.py:56-87`` (shared fp16
  reconstruction buffer; here it also owns the dw4_gemm split-K workspace);
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
    """Choose the packed kernel or reconstruct-then-dense GEMM by flattened M.

    ``reconstruct_threshold`` applies to inference and no-cache PEFT;
    ``grad_reconstruct_threshold`` when PEFT keeps the reconstructed weight
    for backward.  ``None`` disables the dense forward for that path.
    """

    reconstruct_threshold: Optional[int] = 768
    grad_reconstruct_threshold: Optional[int] = 128
    reuse_reconstruct_cache_when_grad: Optional[bool] = None

    def __post_init__(self) -> None:
        for name in ("reconstruct_threshold", "grad_reconstruct_threshold"):
            value = getattr(self, name)
            if value is not None and value <= 0:
                raise ValueError(f"{name} must be positive or None")

    def use_reconstructed_forward(self, flattened_tokens: int, *, cache_weight: bool) -> bool:
        threshold = self.grad_reconstruct_threshold if cache_weight else self.reconstruct_threshold
        return threshold is not None and flattened_tokens >= threshold

    def reuse_reconstruct_cache(self, default: bool) -> bool:
        override = self.reuse_reconstruct_cache_when_grad
        return default if override is None else override

    def direct_max_m(self) -> int:
        """Largest flattened M the packed kernel can be asked to run."""
        t = self.reconstruct_threshold
        return 4096 if t is None else max(1, t - 1)


class MarlinDenseCache:
    """Shared stream-ordered fp16 reconstruction buffer plus the dw4_gemm
    workspace of every matrix registered with :meth:`update`."""

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self.temp_weight_elements = 0
        self.workspace_bytes = 0
        self._temp_weight: Optional[torch.Tensor] = None
        self._workspace: Optional[torch.Tensor] = None
        self._t_workspace: Optional[torch.Tensor] = None

    def update(self, in_features: int, out_features: int, workspace_bytes: int = 0) -> None:
        if self._temp_weight is not None:
            raise RuntimeError("cannot resize initialized Marlin dense cache")
        self.temp_weight_elements = max(self.temp_weight_elements, in_features * out_features)
        self.workspace_bytes = max(self.workspace_bytes, workspace_bytes)

    def init_cache(self) -> None:
        if self._temp_weight is not None:
            raise RuntimeError("Marlin dense cache initialized twice")
        self._temp_weight = torch.empty(self.temp_weight_elements, dtype=torch.float16,
                                        device=self.device)
        # zero-filled: its head holds split-K arrival counters
        self._workspace = torch.zeros(max(self.workspace_bytes, 16), dtype=torch.uint8,
                                      device=self.device)

    def weight(self, in_features: int, out_features: int) -> torch.Tensor:
        if self._temp_weight is None:
            raise RuntimeError("Marlin dense cache is not initialized")
        elements = in_features * out_features
        if elements > self._temp_weight.numel():
            raise RuntimeError("Marlin dense cache is too small")
        return self._temp_weight[:elements].view(in_features, out_features)

    def transpose_workspace(self, nbytes: int) -> torch.Tensor:
        """fp32 partial planes of the packed transposed product, grown on demand."""
        if self._t_workspace is None or self._t_workspace.numel() < nbytes:
            self._t_workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=self.device)
        return self._t_workspace

    @property
    def workspace(self) -> torch.Tensor:
        if self._workspace is None:
            raise RuntimeError("Marlin dense cache is not initialized")
        return self._workspace


def make_marlin_workspace(device: torch.device) -> torch.Tensor:
    """Per-matrix lock buffer of the reference's Marlin GEMM.  The HIP
    kernels keep their split-K state in :class:`MarlinDenseCache`; the
    buffer is still allocated so module buffers and memory accounting match."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("Marlin workspace must be initialized on CUDA")
    sms = torch.cuda.get_device_properties(device).multi_processor_count
    return torch.zeros(sms * 4, dtype=torch.int32, device=device)


def _dense_matmul(x: torch.Tensor, weight: torch.Tensor, *,
                  transpose_weight: bool = False) -> torch.Tensor:
    w = weight.t() if transpose_weight else weight
    out_features = w.shape[1]
    y = torch.matmul(x.reshape(-1, w.shape[0]).to(torch.float16), w)
    return y.reshape(*x.shape[:-1], out_features)


class MarlinQ4Matrix:
    """Repacked matrix plus its dispatch and reconstruction metadata."""

    def __init__(self, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                 in_features: int, out_features: int, g_idx: torch.Tensor,
                 use_act_order: bool, workspace: torch.Tensor,
                 tuning_params: MarlinTuningParams, cache: MarlinDenseCache) -> None:
        if qweight.device.type != "cuda":
            raise ValueError("Marlin weights must be initialized on CUDA")
        if not bool(torch.all(qzeros == _SYMMETRIC_ZEROS).item()):
            raise ValueError("Marlin requires symmetric GPTQ zero points")
        if workspace.device != qweight.device or workspace.dtype != torch.int32:
            raise ValueError("Marlin workspace has the wrong device or dtype")
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

    _MOVED = ("qweight", "qzeros", "scales", "g_idx", "g_idx_sort_indices", "workspace",
              "dequant_weight_permutation", "dequant_scale_column_map")

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
