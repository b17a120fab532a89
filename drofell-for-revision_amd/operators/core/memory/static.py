"""Memory twins: shape-and-dtype stand-ins for device tensors and modules.

The reference plans what fits on a device from a parallel tree of memory
models (``operators/core/memory/static.py:36-172`` in
``/root/reference/After-Revision-DROFELL``): every device tensor a module
keeps is mirrored by a :class:`MemoryTensor` of the same shape and dtype, and
a :class:`MemoryModule` sums the distinct tensors of its tree.  This module
provides the same interface (names, ``requested`` / ``memory`` in bytes, de-
duplication of shared tensors by identity) for the linear-layer twins of the
HIP W4A16 path.
"""
from __future__ import annotations

from math import prod
from typing import Any, Dict, Generator, List, Optional, Sequence, Set, Tuple, Union

import torch

MemoryType = Tuple[str, int]          # (dtype name, bytes per element)
MemoryFloat16: MemoryType = ("float16", 2)
MemoryBFloat16: MemoryType = ("bfloat16", 2)
MemoryFloat32: MemoryType = ("float32", 4)
MemoryInt32: MemoryType = ("int32", 4)
MemoryInt64: MemoryType = ("int64", 8)
MemoryUInt8: MemoryType = ("uint8", 1)
MemoryDType = Union[MemoryType, torch.dtype]


def get_dtype(dtype: MemoryDType) -> MemoryType:
    if isinstance(dtype, tuple):
        return dtype
    return (str(dtype).removeprefix("torch."), dtype.itemsize)


class MemoryTensor:
    """A device (or host, counted as 0 bytes) tensor of ``size`` and ``dtype``."""

    def __init__(self, size: Tuple[int, ...], dtype: MemoryDType = MemoryFloat32,
                 cpu: bool = False) -> None:
        self.size = tuple(int(s) for s in size)
        self.dtype = get_dtype(dtype)
        self.is_cpu = cpu

    @classmethod
    def from_tensor(cls, t: torch.Tensor) -> "MemoryTensor":
        return cls(tuple(t.shape), t.dtype, cpu=t.device.type == "cpu")

    def numel(self) -> int:
        return prod(self.size)

    @property
    def requested(self) -> int:
        return 0 if self.is_cpu else self.numel() * self.dtype[1]

    @property
    def memory(self) -> int:
        return self.requested

    def __repr__(self) -> str:
        return f"<MemoryTensor {self.size} {self.dtype[0]} {self.requested} B>"


class MemoryTensors:
    """Several tensors; shared ones (same object) count once."""

    def __init__(self, tensors: List[MemoryTensor]) -> None:
        self.tensors = tensors

    @property
    def requested(self) -> int:
        seen: Dict[int, MemoryTensor] = {id(t): t for t in self.tensors}
        return sum(t.requested for t in seen.values())


class MemoryModule:
    """Tree of memory twins, mirroring ``nn.Module`` attribute registration."""

    def __init__(self) -> None:
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})

    def __setattr__(self, name: str, value: Any) -> None:
        if isinstance(value, MemoryTensor):
            self._parameters[name] = value
        elif isinstance(value, MemoryModule):
            self._modules[name] = value
        object.__setattr__(self, name, value)

    def mount_list(self, modules: Sequence["MemoryModule"], prefix: str) -> None:
        for i, m in enumerate(modules):
            self._modules[f"{prefix}.{i}"] = m

    def parameters(self, memo: Optional[Set[int]] = None) -> Generator[MemoryTensor, Any, None]:
        memo = set() if memo is None else memo
        for p in self._parameters.values():
            if id(p) not in memo:
                memo.add(id(p))
                yield p
        for m in self._modules.values():
            if id(m) not in memo:
                memo.add(id(m))
                yield from m.parameters(memo)

    def named_parameters(self, prefix: str = "") -> Generator[Tuple[str, MemoryTensor], Any, None]:
        for name, p in self._parameters.items():
            yield prefix + name, p
        for name, m in self._modules.items():
            yield from m.named_parameters(prefix + name + ".")

    @property
    def memory(self) -> int:
        """Bytes of the distinct device tensors in this tree (computed on
        each call: twins such as caches grow while a group is built)."""
        return MemoryTensors(list(self.parameters())).requested
