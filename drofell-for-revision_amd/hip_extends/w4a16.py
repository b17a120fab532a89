"""HIP (gfx950) GPTQ W4A16 matrix objects behind the quantized-Linear API.

Mirrors the role of the reference's ``cuda_extends/exllama.py`` (paths
relative to ``/root/reference/After-Revision-DROFELL``):

* :class:`TuningParams` -- ``exllama.py:22-46`` (dispatch knobs; the values
  here are this library's own);
* :class:`CacheV2` -- ``exllama.py:358-378`` (one shared, stream-ordered
  buffer per device/decoder group, sized before ``init_cache``);
* :class:`Q4MatrixV2` -- ``exllama.py:381-544`` (load-time repack in
  ``__init__``, ``matmul`` with M-based dispatch, dequantised-weight
  export, transposed product for the PEFT backward);
* :class:`Q4LinearFunction` / :class:`Q4ForwardOnlyLinearFunction` --
  ``exllama.py:649-696,730-740``.

All device work goes through ``libdrofell_w4a16.so``; there is no CPU or
PyTorch fallback for the forward product.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Optional, Tuple

import torch
from torch.autograd import Function

from . import _lib


@dataclass
class TuningParams:
    # Flattened M at or below which the register-dequant decode kernel runs
    # (at most 64: four 16-row MFMA tiles); above it the prefill kernel runs.
    # None leaves the choice to the library: decode up to M = 24, or up to
    # M = 32 when N / 16 is at most the device's CU count.
    DECODE_MAX_M: Optional[int] = None
    # Largest flattened M the shared workspace is sized for.  Larger calls
    # still run, with the prefill kernel unsplit along K.
    MAX_M: int = 4096
    # Prefill split-K factor; 0 lets the library choose from the tile count.
    PREFILL_SPLIT_K: int = 0


class CacheV2(object):
    """Per-device shared workspace for every matrix of one decoder group.

    ``update_workspace_size`` grows the requested size while matrices are
    built; ``init_cache`` allocates it once.  ``temp_weight`` (an fp16 K*N
    buffer for the dequantised weight used by the transposed product) is
    allocated on first use only.
    """

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self.workspace_size: int = 0
        self.temp_weight_size: int = 0
        self._workspace: Optional[torch.Tensor] = None
        self._temp_weight: Optional[torch.Tensor] = None
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
        # Zero-filled once: its head holds split-K arrival counters that the
        # library expects at zero and leaves at zero after every call.  At
        # least 16 bytes so the pointer is never null and always aligned.
        self._workspace = torch.zeros(max(self.workspace_size, 16), dtype=torch.uint8,
                                      device=self.device)
        self.cache_created = True

    @property
    def workspace(self) -> torch.Tensor:
        if not self.cache_created or self._workspace is None:
            raise RuntimeError("CacheV2.init_cache() must run before the first matmul")
        return self._workspace

    @property
    def temp_weight(self) -> torch.Tensor:
        if self._temp_weight is None:
            self._temp_weight = torch.empty((1, self.temp_weight_size), dtype=torch.float16,
                                            device=self.device)
        return self._temp_weight


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _aligned_rows(x2: torch.Tensor) -> torch.Tensor:
    """A [M, K] fp16 view whose base is 16-byte aligned with ldx % 8 == 0."""
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
        if x2.data_ptr() % 16 != 0:
            x2 = x2.clone()
    return x2


class Q4MatrixV2(object):
    """One repacked GPTQ projection on a HIP device.

    ``__init__`` performs the load-time repack (``dw4_make_perm`` on the host
    for act-order, then ``dw4_repack`` on the current stream).  The packed
    tensors have the same shapes, dtypes and byte counts as the GPTQ
    buffers they replace, so a module can re-register them in place.
    """

    def __init__(self,
                 qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                 height: int, width: int,
                 g_idx: Optional[torch.Tensor], use_act: bool,
                 tuning_params: TuningParams,
                 cache: CacheV2) -> None:
        if qweight.device.type != "cuda":
            raise ValueError("Q4MatrixV2 weights must live on a HIP device")
        if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
            raise TypeError("qweight and qzeros must be int32")
        if scales.dtype != torch.float16:
            raise TypeError("scales must be float16")
        if tuple(qweight.shape) != (height // 8, width):
            raise ValueError(f"qweight shape {tuple(qweight.shape)} != {(height // 8, width)}")
        groups = scales.shape[0]
        if height % groups != 0 or tuple(scales.shape) != (groups, width) \
                or tuple(qzeros.shape) != (groups, width // 8):
            raise ValueError("qzeros/scales shapes do not match qweight")
        self.height = height
        self.width = width
        self.group_size = height // groups
        self.device = qweight.device
        self.tuning_params = tuning_params
        self.cache = cache

        perm: Optional[torch.Tensor] = None
        if use_act:
            if g_idx is None:
                raise ValueError("act-order needs g_idx")
            g_host = g_idx.detach().to("cpu", torch.int32).contiguous()
            if g_host.numel() != height:
                raise ValueError("g_idx must hold one entry per input row")
            perm_host = torch.empty(height, dtype=torch.int32)
            _lib.call("dw4_make_perm", height, self.group_size, g_host.data_ptr(),
                      perm_host.data_ptr())
            # g_idx == k // group_size sorts to the identity: no gather needed
            if not torch.equal(perm_host, torch.arange(height, dtype=torch.int32)):
                perm = perm_host.to(self.device)
        self.use_act = perm is not None
        self.perm: torch.Tensor = perm if perm is not None else \
            torch.empty(0, dtype=torch.int32, device=self.device)

        self.qweight = torch.empty_like(qweight, memory_format=torch.contiguous_format)
        self.qzeros = torch.empty_like(qzeros, memory_format=torch.contiguous_format)
        self.scales = torch.empty_like(scales, memory_format=torch.contiguous_format)
        with torch.cuda.device(self.device):
            _lib.call("dw4_repack", height, width, self.group_size,
                      qweight.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                      scales.contiguous().data_ptr(), _ptr(perm),
                      self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                      _stream(self.device))
        sizes = _lib.query_sizes(height, width, self.group_size, self.use_act,
                                 max(1, tuning_params.MAX_M))
        cache.update_workspace_size(sizes["workspace"])
        cache.update_temp_weight_size(height * width)
        self.reconstructed_weight_float16: Optional[torch.Tensor] = None

    # -- configuration -------------------------------------------------------
    def set_tuning_params(self, tuning_params: TuningParams) -> None:
        self.tuning_params = tuning_params

    def get_weight_matrix_shape(self) -> Tuple[int, int]:
        return (self.height, self.width)

    # -- products ------------------------------------------------------------
    def _path(self, m: int) -> int:
        dmax = self.tuning_params.DECODE_MAX_M
        if dmax is None:
            return _lib.DW4_PATH_AUTO
        if m <= min(dmax, 64):
            return _lib.DW4_PATH_DECODE
        return _lib.DW4_PATH_PREFILL

    def matmul(self, x: torch.Tensor, output: Optional[torch.Tensor] = None,
               temp_weight: Optional[torch.Tensor] = None, must_blas: bool = False, *,
               bias: Optional[torch.Tensor] = None, path: Optional[int] = None) -> torch.Tensor:
        """``x @ W (+ bias)`` for x [..., K] in x's dtype (fp16 or bf16).

        Same arguments as the reference (``exllama.py:492-526``): with a
        reconstructed fp16 weight, or ``must_blas``, the product is the dense
        one over the dequantised weight (bit-exact HIP dequantisation into
        ``temp_weight`` or the shared buffer, then a library GEMM); otherwise
        the HIP W4A16 kernel runs (decode kernel for small M, MFMA prefill
        kernel above).  bf16 activations are rounded to fp16 for the
        product.  ``bias`` (fp16 [N]) is added after the fp16 rounding of
        the product, as ``output += bias`` does in the reference.
        """
        if x.device != self.device:
            raise ValueError(f"input on {x.device}, weights on {self.device}")
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
        in_dtype = x.dtype
        if in_dtype != torch.float16:
            x = x.to(torch.float16)
        outshape = x.shape[:-1] + (self.width,)
        x2 = _aligned_rows(x.reshape(-1, self.height))
        m = x2.shape[0]
        if bias is not None:
            bias = bias.to(torch.float16).contiguous()
        if must_blas or self.reconstructed_weight_float16 is not None:
            w = self.reconstructed_weight_float16
            if w is None:
                w = self._dense_weight(temp_weight)
            y = torch.matmul(x2, w)
            if bias is not None:
                y += bias
            if output is not None:
                output.view(m, self.width).copy_(y)
                y = output
            y = y.view(outshape)
            return y if in_dtype == torch.float16 else y.to(in_dtype)
        if output is None or output.dtype != torch.float16 or not output.is_contiguous():
            output = torch.empty((m, self.width), dtype=torch.float16, device=self.device)
        ws = self.cache.workspace
        lib = _lib.load()
        status = lib.dw4_gemm_path(
            self._path(m) if path is None else path, self.tuning_params.PREFILL_SPLIT_K,
            m, self.height, self.width, self.group_size,
            x2.data_ptr(), x2.stride(0),
            self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
            _ptr(self.perm) if self.use_act else None, _ptr(bias),
            output.data_ptr(), output.stride(0) if output.dim() == 2 else self.width,
            ws.data_ptr(), ws.numel(), _stream(self.device))
        _lib.check("dw4_gemm_path", status)
        out = output.view(outshape)
        return out if in_dtype == torch.float16 else out.to(in_dtype)

    def _dense_weight(self, temp_weight: Optional[torch.Tensor]) -> torch.Tensor:
        """The fp16 [K, N] weight dequantised into ``temp_weight`` (or the
        shared per-device buffer)."""
        buf = temp_weight if temp_weight is not None else self.cache.temp_weight
        if buf.dtype != torch.float16 or buf.numel() < self.height * self.width:
            raise ValueError("temp_weight must be an fp16 buffer of at least K*N elements")
        w = buf.view(-1)[: self.height * self.width].view(self.height, self.width)
        return self.get_float16_weights_matrix_v2(w)

    def get_float16_weights_matrix_v2(self, out_matrix: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Dequantised fp16 weight [K, N] in the checkpoint's row order."""
        if out_matrix is None:
            out_matrix = torch.empty(self.height, self.width, dtype=torch.float16, device=self.device)
        if out_matrix.dtype != torch.float16 or tuple(out_matrix.shape[-2:]) != (self.height, self.width):
            raise ValueError("out_matrix must be fp16 [K, N]")
        w = out_matrix.view(self.height, self.width)
        _lib.call("dw4_dequant", self.height, self.width, self.group_size,
                  self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                  _ptr(self.perm) if self.use_act else None,
                  w.data_ptr(), w.stride(0), _stream(self.device))
        return out_matrix

    def reconstruct_weight(self, dtype: torch.dtype = torch.float16) -> None:
        if dtype != torch.float16:
            raise ValueError("only fp16 reconstruction is supported")
        self.reconstructed_weight_float16 = self.get_float16_weights_matrix_v2()

    def release_weight(self, dtype: Optional[torch.dtype] = None) -> None:
        self.reconstructed_weight_float16 = None

    def transpose_matmul(self, x: torch.Tensor, output: Optional[torch.Tensor] = None,
                         temp_weight: Optional[torch.Tensor] = None,
                         skip_reconstruct: bool = False) -> torch.Tensor:
        """``x @ W.T`` for x [..., N] (the activation gradient of the forward).

        Same arguments as the reference (``exllama.py:528-544``): the weight
        is the reconstructed one if present, else it is dequantised
        bit-exactly into ``temp_weight`` (or the shared buffer) -- skipped
        with ``skip_reconstruct`` when the caller already filled it -- and
        the dense product is a plain library GEMM.
        """
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
        w = self.reconstructed_weight_float16
        if w is None:
            if skip_reconstruct:
                if temp_weight is None:
                    raise ValueError("skip_reconstruct needs the filled temp_weight")
                w = temp_weight.view(-1)[: self.height * self.width].view(self.height, self.width)
            else:
                w = self._dense_weight(temp_weight)
        in_dtype = x.dtype
        outshape = x.shape[:-1] + (self.height,)
        y = torch.matmul(x.reshape(-1, self.width).to(torch.float16), w.t())
        if output is not None:
            output.view(-1, self.height).copy_(y)
            y = output
        y = y.view(outshape)
        return y if in_dtype == torch.float16 else y.to(in_dtype)


class Q4LinearFunction(Function):
    """Frozen quantised weight; only the activation receives a gradient."""

    @staticmethod
    def forward(ctx: Any, input: torch.Tensor, weight_q4: Q4MatrixV2,  # type: ignore[override]
                bias: Optional[torch.Tensor], cache_weight: bool) -> torch.Tensor:
        ctx.weight_q4 = weight_q4
        cached = None
        if cache_weight and weight_q4.reconstructed_weight_float16 is None:
            cached = weight_q4.get_float16_weights_matrix_v2()
        output = weight_q4.matmul(input, bias=bias)
        if cached is not None:
            ctx.save_for_backward(cached)
        ctx.has_cached = cached is not None
        return output

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor):  # type: ignore[override]
        grad_input = None
        if ctx.needs_input_grad[0]:
            if ctx.has_cached:
                grad_input = ctx.weight_q4.transpose_matmul(
                    grad_output, None, ctx.saved_tensors[0], skip_reconstruct=True)
            else:
                grad_input = ctx.weight_q4.transpose_matmul(grad_output)
        return grad_input, None, None, None


class Q4ForwardOnlyLinearFunction(Function):
    @staticmethod
    def forward(ctx: Any, input: torch.Tensor, weight_q4: Q4MatrixV2,  # type: ignore[override]
                bias: Optional[torch.Tensor]) -> torch.Tensor:
        return weight_q4.matmul(input, bias=bias)

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor):  # type: ignore[override]
        return None, None, None
