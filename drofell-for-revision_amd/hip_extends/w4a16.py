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
  ``exllama.py:649-696,730-740``;
* :func:`attention_forward_qkv_stage_v2_py` / :func:`mlp_forward_v2_py` --
  the fused decoder-stage calls ``exllama.py:120-130`` (RMSNorm, then the
  q/k/v projections as one grouped launch; RMSNorm, gate/up with the
  silu * mul folded into one launch, then down).

All device work goes through ``libdrofell_w4a16.so``; there is no CPU or
PyTorch fallback for the forward product.
"""
from __future__ import annotations

import ctypes
import hashlib
import threading
import weakref
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch
from torch.autograd import Function

from . import _lib


@dataclass
class TuningParams:
    # Flattened M at or below which the register-dequant decode kernel runs
    # (at most 64: four 16-row MFMA tiles); above it the prefill kernel runs.
    # None leaves the choice to the library: decode up to M = 48, or up to
    # M = 64 when N / 16 is at most the device's CU count (or at most 1.25x
    # it with K <= 8192).
    DECODE_MAX_M: Optional[int] = None
    # Largest flattened M the shared workspace is sized for.  Larger calls
    # still run, with the prefill kernel unsplit along K.
    MAX_M: int = 4096
    # Prefill split-K factor; 0 lets the library choose from the tile count.
    PREFILL_SPLIT_K: int = 0
    # Flattened M up to which the transposed product (PEFT backward) runs the
    # packed kernel; above it the weight is dequantised and a dense GEMM runs,
    # as in the reference.
    TRANSPOSE_MAX_M: int = 128


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
        self._t_workspace: Optional[torch.Tensor] = None
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

    def transpose_workspace(self, nbytes: int) -> torch.Tensor:
        """fp32 partial planes of the transposed product, grown on demand
        (the backward runs outside graph capture); no zero-fill needed."""
        if self._t_workspace is None or self._t_workspace.numel() < nbytes:
            self._t_workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=self.device)
        return self._t_workspace

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


def _output_rows(output: torch.Tensor, m: int, n: int, dtype: torch.dtype) -> torch.Tensor:
    """The caller's ``output`` as a [m, n] row-major view the product can be
    written into (unit column stride, any row stride >= n), or an error:
    the product is never written anywhere else."""
    if output.dtype != dtype:
        raise TypeError(f"output is {output.dtype}, the product is {dtype}")
    if output.device.type != "cuda":
        raise ValueError("output must live on the device")
    if output.numel() != m * n:
        raise ValueError(f"output holds {output.numel()} elements, the product has {m} x {n}")
    if output.is_contiguous():
        return output.view(m, n)
    if output.dim() == 2 and output.shape[0] == m and output.stride(1) == 1 \
            and output.stride(0) >= n:
        return output
    raise ValueError("output must be contiguous or a [m, n] view with unit column stride")


def _aligned_rows(x2: torch.Tensor) -> torch.Tensor:
    """A [M, K] fp16 or bf16 view whose base is 16-byte aligned with ldx % 8 == 0."""
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
        if x2.data_ptr() % 16 != 0:
            x2 = x2.clone()
    return x2


# Device perms by content: matrices whose act-order permutations are equal
# (q/k/v, or gate/up, quantised against the same input) share one tensor, so
# a fused launch can pair them.
_perm_lock = threading.Lock()
_perm_intern: Dict[Tuple[str, int, str], Tuple[torch.Tensor, "weakref.ref[torch.Tensor]"]] = {}


def perm_digest(perm_host: torch.Tensor) -> str:
    return hashlib.sha1(perm_host.numpy().tobytes()).hexdigest()


def _shared_perm(perm_host: torch.Tensor, device: torch.device) -> torch.Tensor:
    key = (str(device), perm_host.numel(), perm_digest(perm_host))
    with _perm_lock:
        hit = _perm_intern.get(key)
        if hit is not None:
            dev = hit[1]()
            if dev is not None and torch.equal(hit[0], perm_host):
                return dev
        dev = perm_host.to(device)
        _perm_intern[key] = (perm_host.clone(), weakref.ref(dev))
        return dev


class PermGroup(object):
    """Matrices whose act-order permutations are equal.

    Module moves (``nn.Module.to`` / ``cuda`` / ``cpu``) copy each module's
    buffers separately, so after a swap-in every matrix would hold its own
    copy of the permutation and the fused launches, which pair matrices by
    the permutation pointer, would no longer pair them.  A moved matrix
    offers its new tensor to its group and takes the group's tensor when that
    one already lives on the same device (the contents are equal by
    construction).
    """

    def __init__(self) -> None:
        self.tensor: Optional[torch.Tensor] = None

    def share(self, t: torch.Tensor) -> torch.Tensor:
        cur = self.tensor
        if cur is not None and cur.device == t.device and cur.shape == t.shape:
            return cur
        self.tensor = t
        return t


_groups_lock = threading.Lock()
_perm_groups: Dict[Tuple[int, str], PermGroup] = {}


def perm_group(numel: int, digest: str) -> PermGroup:
    with _groups_lock:
        return _perm_groups.setdefault((numel, digest), PermGroup())


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
                perm = _shared_perm(perm_host, self.device)
                self.perm_group: Optional[PermGroup] = perm_group(height, perm_digest(perm_host))
                self.perm_group.share(perm)
        if perm is None:
            self.perm_group = None
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
        self.reconstructed_weight_bfloat16: Optional[torch.Tensor] = None

    @property
    def cuda_q4(self) -> "Q4MatrixV2":
        """The handle the fused stage calls take (the reference's ``make_q4``
        pointer, ``exllama.py:203``): the matrix object itself."""
        return self

    def rebind(self, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
               perm: torch.Tensor) -> None:
        """Point the matrix at moved copies of its packed tensors (a module
        swapped out to host memory and back in, or moved between devices).
        The packed layout travels with the tensors, so nothing is repacked;
        a matrix whose tensors are in host memory refuses products until it
        is moved back.  A reconstructed fp16 weight is rebuilt on the new
        device (it is derived data, not swapped)."""
        if qweight is self.qweight and qzeros is self.qzeros and scales is self.scales \
                and perm is self.perm:
            return  # e.g. a dtype conversion that left the integer buffers alone
        for new, old, name in ((qweight, self.qweight, "qweight"), (qzeros, self.qzeros, "qzeros"),
                               (scales, self.scales, "scales")):
            if new.shape != old.shape or new.dtype != old.dtype:
                raise ValueError(f"{name}: moved tensor {tuple(new.shape)} {new.dtype} does not "
                                 f"match {tuple(old.shape)} {old.dtype}")
        if self.use_act and (perm.numel() != self.height or perm.dtype != torch.int32):
            raise ValueError("perm must be int32 [K] for an act-order matrix")
        devices = {qweight.device, qzeros.device, scales.device, perm.device}
        if len(devices) != 1:
            raise ValueError(f"packed tensors on several devices: {devices}")
        had = [dt for dt in (torch.float16, torch.bfloat16) if self._reconstructed(dt) is not None]
        self.qweight, self.qzeros, self.scales = qweight, qzeros, scales
        self.perm = perm
        self.device = qweight.device
        self.release_weight()
        if self.device.type == "cuda":
            for dt in had:
                self.reconstruct_weight(dt)

    def _check_resident(self) -> None:
        if self.device.type != "cuda":
            raise RuntimeError("Q4MatrixV2 is swapped out (its tensors are in host memory)")

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
        """``x @ W (+ bias)`` for x [..., K]; the result has x's dtype.

        Same arguments and routes as the reference (``exllama.py:492-526``):

        * fp16 x: with a reconstructed fp16 weight, or ``must_blas``, the
          dense product over the dequantised weight (bit-exact HIP
          dequantisation into ``temp_weight`` or the shared buffer, then a
          library GEMM); otherwise the HIP W4A16 kernel (decode kernel for
          small M, MFMA prefill kernel above);
        * bf16 x: with a reconstructed bf16 weight, ``must_blas`` or more
          than ``BF16_MAX_M`` rows, the dense bf16 product (fp32
          accumulation) over the bf16 weight bf16(fp16(s * (q - z))), the
          reconstructed one or one dequantised into ``temp_weight`` / the
          shared buffer, as the reference's ``q4_matmul_blas_v2`` with
          ``bfloat16`` does; up to ``BF16_MAX_M`` rows the HIP decode
          kernel's bf16 mode (``dw4_gemm_bf16``: bf16 matrix cores over the
          packed words, the exact s * (q - z) applied per group in fp32, bf16
          output, one launch), within rounding of the dense product.  The
          activations keep bf16's range either way.

        ``output`` (x's dtype, ``M * N`` elements, contiguous or a row-strided
        [M, N] view) receives the product; anything else raises.  ``bias``
        ([N]) is added after the rounding of the product, as the reference's
        ``output += bias``.
        """
        self._check_resident()
        if x.device != self.device:
            raise ValueError(f"input on {x.device}, weights on {self.device}")
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
        dtype = x.dtype
        outshape = x.shape[:-1] + (self.width,)
        m = x.numel() // self.height
        out2 = None if output is None else _output_rows(output, m, self.width, dtype)
        if bias is not None:
            bias = bias.to(dtype).contiguous()
        dense = self._reconstructed(dtype)
        if dtype == torch.bfloat16 and dense is None and not must_blas \
                and 0 < m <= _lib.BF16_MAX_M:
            x2 = _aligned_rows(x.reshape(m, self.height))
            if out2 is None:
                out2 = torch.empty((m, self.width), dtype=torch.bfloat16, device=self.device)
            ws = self.cache.workspace
            _lib.check("dw4_gemm_bf16", _lib.load().dw4_gemm_bf16(
                m, self.height, self.width, self.group_size, x2.data_ptr(), x2.stride(0),
                self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                _ptr(self.perm) if self.use_act else None, _ptr(bias),
                out2.data_ptr(), out2.stride(0), ws.data_ptr(), ws.numel(), _stream(self.device)))
            return out2.view(outshape) if output is None else output
        if dense is not None or must_blas or dtype == torch.bfloat16:
            w = dense if dense is not None else self._dense_weight(temp_weight, dtype)
            x2 = x.reshape(m, self.height)
            if out2 is None:
                y = torch.matmul(x2, w)
            else:
                y = torch.matmul(x2, w, out=out2) if out2.is_contiguous() else \
                    out2.copy_(torch.matmul(x2, w))
            if bias is not None:
                y += bias
            return y.view(outshape) if output is None else output
        x2 = _aligned_rows(x.reshape(m, self.height))
        if out2 is None:
            out2 = torch.empty((m, self.width), dtype=torch.float16, device=self.device)
        ws = self.cache.workspace
        lib = _lib.load()
        status = lib.dw4_gemm_path(
            self._path(m) if path is None else path, self.tuning_params.PREFILL_SPLIT_K,
            m, self.height, self.width, self.group_size,
            x2.data_ptr(), x2.stride(0),
            self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
            _ptr(self.perm) if self.use_act else None, _ptr(bias),
            out2.data_ptr(), out2.stride(0),
            ws.data_ptr(), ws.numel(), _stream(self.device))
        _lib.check("dw4_gemm_path", status)
        return out2.view(outshape) if output is None else output

    def _reconstructed(self, dtype: torch.dtype) -> Optional[torch.Tensor]:
        return self.reconstructed_weight_float16 if dtype == torch.float16 else \
            self.reconstructed_weight_bfloat16

    def _transpose_native(self, x: torch.Tensor, output: Optional[torch.Tensor]) -> torch.Tensor:
        """fp16 ``x @ W.T`` through the packed transposed kernel."""
        if x.device != self.device:
            raise ValueError(f"input on {x.device}, weights on {self.device}")
        if x.dtype != torch.float16:
            raise TypeError(f"the packed transposed kernel takes fp16, got {x.dtype}")
        outshape = x.shape[:-1] + (self.height,)
        g2 = _aligned_rows(x.reshape(-1, self.width))
        m = g2.shape[0]
        out2 = torch.empty((m, self.height), dtype=torch.float16, device=self.device) \
            if output is None else _output_rows(output, m, self.height, torch.float16)
        nbytes = _lib.gemm_t_workspace_size(m, self.height, self.width, self.group_size)
        ws = self.cache.transpose_workspace(nbytes)
        _lib.call("dw4_gemm_t", m, self.height, self.width, self.group_size,
                  g2.data_ptr(), g2.stride(0), self.qweight.data_ptr(), self.qzeros.data_ptr(),
                  self.scales.data_ptr(), _ptr(self.perm) if self.use_act else None,
                  out2.data_ptr(), out2.stride(0), ws.data_ptr(), ws.numel(), _stream(self.device))
        return out2.view(outshape) if output is None else output

    def _dense_weight(self, temp_weight: Optional[torch.Tensor],
                      dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """The [K, N] weight in ``dtype`` (fp16 or bf16) dequantised into
        ``temp_weight`` or the shared per-device buffer (fp16 storage,
        reinterpreted for bf16 as the reference does)."""
        buf = temp_weight if temp_weight is not None else self.cache.temp_weight
        if buf.element_size() != 2 or buf.numel() < self.height * self.width:
            raise ValueError("temp_weight must be a 2-byte buffer of at least K*N elements")
        flat = buf.view(-1)[: self.height * self.width]
        if flat.dtype != dtype:
            flat = flat.view(dtype)
        w = flat.view(self.height, self.width)
        if dtype == torch.bfloat16:
            return self.get_bfloat16_weights_matrix_v2(w)
        return self.get_float16_weights_matrix_v2(w)

    def get_float16_weights_matrix_v2(self, out_matrix: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Dequantised fp16 weight [K, N] in the checkpoint's row order."""
        self._check_resident()
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

    def get_bfloat16_weights_matrix_v2(self, out_matrix: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Dequantised bf16 weight [K, N] in the checkpoint's row order:
        bf16(fp16(s * (q - z))), bit-exact with the reference's bf16
        reconstruction (``q4_matrix.cu:469-614``)."""
        self._check_resident()
        if out_matrix is None:
            out_matrix = torch.empty(self.height, self.width, dtype=torch.bfloat16,
                                     device=self.device)
        if out_matrix.dtype != torch.bfloat16 or \
                tuple(out_matrix.shape[-2:]) != (self.height, self.width):
            raise ValueError("out_matrix must be bf16 [K, N]")
        w = out_matrix.view(self.height, self.width)
        _lib.call("dw4_dequant_bf16", self.height, self.width, self.group_size,
                  self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr(),
                  _ptr(self.perm) if self.use_act else None,
                  w.data_ptr(), w.stride(0), _stream(self.device))
        return out_matrix

    def reconstruct_weight(self, dtype: torch.dtype = torch.float16) -> None:
        if dtype == torch.float16:
            self.reconstructed_weight_float16 = self.get_float16_weights_matrix_v2()
        elif dtype == torch.bfloat16:
            self.reconstructed_weight_bfloat16 = self.get_bfloat16_weights_matrix_v2()
        else:
            raise ValueError(f"reconstruction dtype must be fp16 or bf16, got {dtype}")

    def release_weight(self, dtype: Optional[torch.dtype] = None) -> None:
        if dtype in (None, torch.float16):
            self.reconstructed_weight_float16 = None
        if dtype in (None, torch.bfloat16):
            self.reconstructed_weight_bfloat16 = None

    def transpose_matmul(self, x: torch.Tensor, output: Optional[torch.Tensor] = None,
                         temp_weight: Optional[torch.Tensor] = None,
                         skip_reconstruct: bool = False) -> torch.Tensor:
        """``x @ W.T`` for x [..., N] (the activation gradient of the forward),
        in x's dtype.

        Same arguments as the reference (``exllama.py:528-544``).  With a
        reconstructed weight of x's dtype, or ``skip_reconstruct`` (the caller
        already filled ``temp_weight``), the product is the dense one over
        that weight.  Otherwise fp16 x up to ``TuningParams.TRANSPOSE_MAX_M``
        rows runs the packed kernel (``dw4_gemm_t``), which reads the int4
        words directly; above it, and for bf16 x, the weight is dequantised
        bit-exactly (fp16, or bf16 of the fp16 value) into ``temp_weight`` or
        the shared buffer and a library GEMM runs, as in the reference.
        """
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
        self._check_resident()
        dtype = x.dtype
        m = x.numel() // self.width
        w = self._reconstructed(dtype)
        if w is None and not skip_reconstruct and dtype == torch.float16 \
                and 0 < m <= self.tuning_params.TRANSPOSE_MAX_M:
            return self._transpose_native(x, output)
        if w is None:
            if skip_reconstruct:
                if temp_weight is None:
                    raise ValueError("skip_reconstruct needs the filled temp_weight")
                if temp_weight.dtype != dtype:
                    raise TypeError(f"temp_weight is {temp_weight.dtype}, x is {dtype}")
                w = temp_weight.view(-1)[: self.height * self.width].view(self.height, self.width)
            else:
                w = self._dense_weight(temp_weight, dtype)
        outshape = x.shape[:-1] + (self.height,)
        y = torch.matmul(x.reshape(m, self.width), w.t())
        if output is None:
            return y.view(outshape)
        _output_rows(output, m, self.height, dtype).copy_(y)
        return output


class Q4LinearFunction(Function):
    """Frozen quantised weight; only the activation receives a gradient.

    As ``ExllamaQ4LinearFunction`` (``exllama.py:649-696``): with
    ``cache_weight`` the dequantised weight of the input's dtype is kept for
    the backward (unless the matrix already holds a reconstructed one);
    the forward of fp16 input still runs the W4A16 kernel, bf16 input the
    dense product over the kept weight.
    """

    @staticmethod
    def forward(ctx: Any, input: torch.Tensor, weight_q4: Q4MatrixV2,  # type: ignore[override]
                bias: Optional[torch.Tensor], cache_weight: bool) -> torch.Tensor:
        ctx.weight_q4 = weight_q4
        cached = None
        if cache_weight and weight_q4._reconstructed(input.dtype) is None:
            cached = weight_q4._dense_weight(
                torch.empty(weight_q4.height * weight_q4.width, dtype=input.dtype,
                            device=weight_q4.device), input.dtype)
        if cached is not None and input.dtype == torch.bfloat16:
            output = weight_q4.matmul(input, temp_weight=cached, must_blas=True, bias=bias)
        else:
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


# ---------------------------------------------------------------------------
# Decoder-stage calls
# ---------------------------------------------------------------------------
def _item(q4: Q4MatrixV2, y: Optional[torch.Tensor]) -> _lib.Item:
    return _lib.Item(q4.height, q4.width, q4.group_size, q4.qweight.data_ptr(),
                     q4.qzeros.data_ptr(), q4.scales.data_ptr(),
                     q4.perm.data_ptr() if q4.use_act else None, None,
                     None if y is None else y.data_ptr(), 0 if y is None else y.stride(0))


def _rows(t: torch.Tensor, m: int, width: int, what: str) -> torch.Tensor:
    """The first m rows of t viewed as fp16 [*, width] (row-major storage)."""
    if t.dtype != torch.float16:
        raise TypeError(f"{what} must be float16, got {t.dtype}")
    v = t.view(-1, width)
    if v.shape[0] < m:
        raise ValueError(f"{what} holds {v.shape[0]} rows of {width}, need {m}")
    return v[:m]


def _matrix(h: Any) -> Q4MatrixV2:
    q4 = getattr(h, "cuda_q4", h)
    if not isinstance(q4, Q4MatrixV2):
        raise TypeError(f"expected a Q4MatrixV2 handle, got {type(h).__name__}")
    return q4


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``fp16(x * w / sqrt(mean(x^2) + eps))`` per row of fp16 x [..., K]
    (the reference's ``rms_norm_cuda``, ``fuse_v2/rms_norm.cu:26-131``)."""
    k = x.shape[-1]
    x2 = _aligned_rows(x.reshape(-1, k))
    m = x2.shape[0]
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    o2 = _rows(out, m, k, "out")
    w = weight.to(torch.float16).contiguous()
    _lib.check("dw4_rms_norm", _lib.load().dw4_rms_norm(
        m, k, x2.data_ptr(), x2.stride(0), w.data_ptr(), float(eps), o2.data_ptr(), o2.stride(0),
        _stream(x.device)))
    return out


def attention_forward_qkv_stage_v2_py(layernorm: torch.Tensor, norm_epsilon: float,
                                      q_proj: Any, k_proj: Any, v_proj: Any,
                                      temp_rms_output: torch.Tensor, temp_q_output: torch.Tensor,
                                      temp_k_output: torch.Tensor, temp_v_output: torch.Tensor,
                                      temp_weight: Optional[torch.Tensor], x: torch.Tensor,
                                      BLOCK_KN_SIZE: int, BLOCK_M_SIZE_MAX: int,
                                      MATMAL_RECONSTRUCT_THRESHOLD_V2: int,
                                      q_len: int, batch_size: int) -> None:
    """``temp_rms_output = rms_norm(x)``; ``temp_{q,k,v}_output = rms @ W``.

    Same arguments as the reference (``exllama.py:124-130`` ->
    ``fuse_v2/q_attn.cu:23-54``).  The q/k/v products run as one grouped
    launch where the decode kernel applies.  ``temp_weight`` and the three
    exllama tuning values are accepted and unused: this library chooses its
    kernels from M and the shapes.
    """
    q4s = [_matrix(h) for h in (q_proj, k_proj, v_proj)]
    hidden = q4s[0].height
    m = q_len * batch_size
    x2 = _aligned_rows(_rows(x, m, hidden, "x"))
    rms = _rows(temp_rms_output, m, hidden, "temp_rms_output")
    outs = [_rows(t, m, q4.width, name) for t, q4, name in
            ((temp_q_output, q4s[0], "temp_q_output"), (temp_k_output, q4s[1], "temp_k_output"),
             (temp_v_output, q4s[2], "temp_v_output"))]
    items = [_item(q4, y) for q4, y in zip(q4s, outs)]
    ws = q4s[0].cache.workspace
    w = layernorm.to(torch.float16).contiguous()
    _lib.check("dw4_attention_qkv_stage", _lib.load().dw4_attention_qkv_stage(
        m, x2.data_ptr(), x2.stride(0), w.data_ptr(), float(norm_epsilon),
        rms.data_ptr(), rms.stride(0), ctypes.byref(items[0]), ctypes.byref(items[1]),
        ctypes.byref(items[2]), ws.data_ptr(), ws.numel(), _stream(x.device)))


def attention_forward_rope_stage_v2_py(temp_q_output: torch.Tensor, temp_k_output: torch.Tensor,
                                       sin: torch.Tensor, cos: torch.Tensor, q_len: int,
                                       batch_size: int, num_heads: int, num_kv_heads: int,
                                       head_dim: int, past_len: int,
                                       past_lens: Optional[torch.Tensor]) -> None:
    """Rotary embedding of q and k in place (``exllama.py:133-135`` ->
    ``fuse_v2/rope.cu``): row r of batch entry b takes position
    ``(past_len if past_len >= 0 else past_lens[b]) + r // heads`` of the fp16
    tables ``sin`` / ``cos``, each [..., max_positions, head_dim] (the
    reference's rotary modules keep them as [1, 1, max_positions, head_dim],
    ``operators/core/rope/real.py:114,140``)."""
    lens = None
    if past_len < 0:
        if past_lens is None:
            raise ValueError("past_len -1 needs past_lens")
        lens = past_lens.to(device=temp_q_output.device, dtype=torch.int32).contiguous()
    s16, c16, max_pos = rope_tables(sin, cos, head_dim)
    for t, heads in ((temp_q_output, num_heads), (temp_k_output, num_kv_heads)):
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise TypeError("q/k must be contiguous fp16")
        _lib.call("dw4_rope", batch_size, q_len * heads, heads, head_dim, t.data_ptr(),
                  s16.data_ptr(), c16.data_ptr(), max_pos, past_len,
                  None if lens is None else lens.data_ptr(), _stream(t.device))


def rope_tables(sin: torch.Tensor, cos: torch.Tensor,
                head_dim: int) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """fp16 sin / cos tables as contiguous [positions, head_dim] and the
    position count, from [P, hd] tables or the rotary modules' [1, 1, P, hd]
    (every dimension before the last two must be 1: a batched table would
    otherwise be read as more positions)."""
    if sin.shape != cos.shape:
        raise ValueError(f"sin {tuple(sin.shape)} and cos {tuple(cos.shape)} differ")
    if sin.dim() < 2 or sin.shape[-1] != head_dim:
        raise ValueError(f"rope tables must be [..., positions, {head_dim}], got "
                         f"{tuple(sin.shape)}")
    if any(d != 1 for d in sin.shape[:-2]):
        raise ValueError(f"rope tables {tuple(sin.shape)}: every leading dimension must be 1")
    s16 = sin.to(torch.float16).contiguous().view(-1, head_dim)
    c16 = cos.to(torch.float16).contiguous().view(-1, head_dim)
    return s16, c16, s16.shape[0]


def mlp_forward_v2_py(layernorm: torch.Tensor, norm_epsilon: float, gate_q4: Any, up_q4: Any,
                      down_q4: Any, temp_rms_output: torch.Tensor,
                      temp_gate_output: torch.Tensor, temp_up_output: torch.Tensor,
                      temp_weight: Optional[torch.Tensor], x: torch.Tensor,
                      output: torch.Tensor, BLOCK_KN_SIZE: int, BLOCK_M_SIZE_MAX: int,
                      MATMAL_RECONSTRUCT_THRESHOLD_V2: int) -> None:
    """``output = (silu(rms @ W_gate) * (rms @ W_up)) @ W_down`` with
    ``rms = rms_norm(x)``.

    Same arguments as the reference (``exllama.py:120-121`` ->
    ``fuse_v2/q_mlp.cu:96-133``): ``temp_rms_output`` receives the
    normalised input and ``temp_gate_output`` the gated product that feeds
    down; ``temp_up_output`` is scratch.  For small M (decode) gate and up
    run as one launch that never writes their separate products.
    ``temp_weight`` and the tuning values are accepted and unused.
    """
    g, u, d = _matrix(gate_q4), _matrix(up_q4), _matrix(down_q4)
    hidden = g.height
    x2 = _aligned_rows(x.reshape(-1, hidden))
    m = x2.shape[0]
    rms = _rows(temp_rms_output, m, hidden, "temp_rms_output")
    hbuf = _rows(temp_gate_output, m, g.width, "temp_gate_output")
    ubuf = _rows(temp_up_output, m, u.width, "temp_up_output")
    out = _rows(output, m, d.width, "output")
    ig, iu, idn = _item(g, hbuf), _item(u, ubuf), _item(d, out)
    ws = g.cache.workspace
    w = layernorm.to(torch.float16).contiguous()
    _lib.check("dw4_mlp_forward", _lib.load().dw4_mlp_forward(
        m, x2.data_ptr(), x2.stride(0), w.data_ptr(), float(norm_epsilon),
        rms.data_ptr(), rms.stride(0), ctypes.byref(ig), ctypes.byref(iu), ctypes.byref(idn),
        ws.data_ptr(), ws.numel(), _stream(x.device)))


def decoder_after_stage_v2_py(o_q4: Any, gate_q4: Any, up_q4: Any, down_q4: Any,
                              layernorm: torch.Tensor, norm_epsilon: float,
                              attn_output: torch.Tensor, residual: torch.Tensor,
                              temp_hidden_output: torch.Tensor, temp_rms_output: torch.Tensor,
                              temp_gate_output: torch.Tensor, temp_up_output: torch.Tensor,
                              output: torch.Tensor) -> None:
    """The decoder layer after attention, as ``_fuse_forward_after_stage``
    (``operators/core/decoder_wrap/real_fuse.py:77-103``) computes it:

    * ``temp_hidden_output = residual + o_proj(attn_output)``;
    * ``temp_rms_output = rms_norm(temp_hidden_output)``;
    * ``temp_gate_output = silu(rms @ W_gate) * (rms @ W_up)``;
    * ``output = temp_hidden_output + temp_gate_output @ W_down``.

    Every sum is rounded to fp16 as the reference's fp16 tensors are.
    ``temp_up_output`` is scratch for the up product where gate and up do not
    run as one launch.
    """
    o, g, u, d = _matrix(o_q4), _matrix(gate_q4), _matrix(up_q4), _matrix(down_q4)
    hidden = o.width
    a2 = _aligned_rows(attn_output.reshape(-1, o.height))
    m = a2.shape[0]
    res = _rows(residual, m, hidden, "residual")
    x2 = _rows(temp_hidden_output, m, hidden, "temp_hidden_output")
    rms = _rows(temp_rms_output, m, hidden, "temp_rms_output")
    hbuf = _rows(temp_gate_output, m, g.width, "temp_gate_output")
    ubuf = _rows(temp_up_output, m, u.width, "temp_up_output")
    out = _rows(output, m, d.width, "output")
    io, ig, iu, idn = _item(o, x2), _item(g, hbuf), _item(u, ubuf), _item(d, out)
    ws = o.cache.workspace
    w = layernorm.to(torch.float16).contiguous()
    _lib.check("dw4_decoder_after_stage", _lib.load().dw4_decoder_after_stage(
        m, a2.data_ptr(), a2.stride(0), res.data_ptr(), res.stride(0), ctypes.byref(io),
        w.data_ptr(), float(norm_epsilon), rms.data_ptr(), rms.stride(0), ctypes.byref(ig),
        ctypes.byref(iu), ctypes.byref(idn), ws.data_ptr(), ws.numel(), _stream(attn_output.device)))


def gemm_group(x: torch.Tensor, matrices: "list[Q4MatrixV2]",
               outputs: Optional["list[Optional[torch.Tensor]]"] = None) -> "list[torch.Tensor]":
    """``[x @ W_i]`` for matrices that share x (one launch where the decode
    kernel applies); fp16 x [..., K]."""
    q4s = [_matrix(h) for h in matrices]
    k = q4s[0].height
    x2 = _aligned_rows(x.reshape(-1, k))
    m = x2.shape[0]
    outs = []
    for i, q4 in enumerate(q4s):
        o = outputs[i] if outputs is not None and outputs[i] is not None else \
            torch.empty(x.shape[:-1] + (q4.width,), dtype=torch.float16, device=x.device)
        outs.append(o)
    items = (_lib.Item * len(q4s))(*[_item(q4, _rows(o, m, q4.width, "output"))
                                     for q4, o in zip(q4s, outs)])
    ws = q4s[0].cache.workspace
    _lib.check("dw4_gemm_group", _lib.load().dw4_gemm_group(
        len(q4s), items, m, x2.data_ptr(), x2.stride(0), ws.data_ptr(), ws.numel(),
        _stream(x.device)))
    return outs
