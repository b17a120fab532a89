"""KV-cache block geometry.

Same class and properties as the reference's ``operators/core/block/common.py:7-95``
(paths relative to ``/root/reference/After-Revision-DROFELL``): a block holds
``flags.BLOCK_SIZE`` token slots; its key part is
``[kv_heads, head_dim / x, BLOCK_SIZE, x]`` and its value part
``[kv_heads, head_dim, BLOCK_SIZE]``, with x = 16 bytes / element size.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from ... import flags


@dataclass
class BlockInfo:
    head_dim: int
    num_key_value_heads: int
    dtype: torch.dtype = torch.float16

    def __post_init__(self) -> None:
        self.element_size = int(self.dtype.itemsize)
        self._x = 16 // self.element_size
        self._head_stride = flags.BLOCK_SIZE * self.head_dim
        self._elements_per_slot = self.num_key_value_heads * self.head_dim
        self._elements_per_block = flags.BLOCK_SIZE * self._elements_per_slot
        self._bytes_per_block = self._elements_per_block * self.element_size

    @property
    def key_block_shape(self) -> Tuple[int, int, int, int]:
        return (self.num_key_value_heads, self.head_dim // self._x, flags.BLOCK_SIZE, self._x)

    @property
    def value_block_shape(self) -> Tuple[int, int, int]:
        return (self.num_key_value_heads, self.head_dim, flags.BLOCK_SIZE)

    @property
    def num_heads(self) -> int:
        return self.num_key_value_heads

    @property
    def head_size(self) -> int:
        return self.head_dim

    @property
    def bytes_per_block(self) -> int:
        return self._bytes_per_block

    @property
    def x(self) -> int:
        return self._x

    @property
    def head_stride(self) -> int:
        return self._head_stride

    @property
    def elements_per_block(self) -> int:
        return self._elements_per_block
