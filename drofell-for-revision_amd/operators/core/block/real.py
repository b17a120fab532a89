"""One layer's KV-cache blocks, addressed through per-block pointer tables.

Mirrors ``LayerBlocksHolder`` of the reference's ``operators/core/block/real.py:17-262``
(paths relative to ``/root/reference/After-Revision-DROFELL``): key and value
pointer tables (int64, one entry per block, on the device and the host), an
optional contiguous backing pair, ``kv_tensor_to_slots_with_convert`` /
``kv_tensor_from_slots_with_convert`` (token rows to and from cache slots)
and ``create_contigious_cacher``.  The copies run in the HIP library
(``dw4_reshape_and_cache`` / ``dw4_restore_from_cache``).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from hip_extends import _lib
from hip_extends.w4a16 import rope_tables

from ... import flags
from .common import BlockInfo


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


class LayerBlocksHolder:
    def __init__(self, block_info: BlockInfo, layer_key_ptr_table_device: torch.Tensor,
                 layer_val_ptr_table_device: torch.Tensor,
                 layer_key_ptr_table_cpu: torch.Tensor, layer_val_ptr_table_cpu: torch.Tensor,
                 layer_key_ptr_table_list: List[int], layer_val_ptr_table_list: List[int],
                 contigious_kv_tensor: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
        for t in (layer_key_ptr_table_device, layer_val_ptr_table_device):
            if t.dtype != torch.int64 or t.requires_grad:
                raise AssertionError("pointer tables must be int64 without grad")
        self.block_info = block_info
        self.layer_key_ptr_table_device = layer_key_ptr_table_device
        self.layer_val_ptr_table_device = layer_val_ptr_table_device
        self.layer_key_ptr_table_cpu = layer_key_ptr_table_cpu
        self.layer_val_ptr_table_cpu = layer_val_ptr_table_cpu
        self.layer_key_ptr_table_list = layer_key_ptr_table_list
        self.layer_val_ptr_table_list = layer_val_ptr_table_list
        self._contigious_kv_tensor = contigious_kv_tensor
        self.device = layer_key_ptr_table_device.device

    @property
    def is_contigious(self) -> bool:
        return self._contigious_kv_tensor is not None

    @property
    def contigious_kv_tenosr(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._contigious_kv_tensor is None:
            raise AssertionError("this cacher has no contiguous backing")
        return self._contigious_kv_tensor

    def _copy(self, fn: str, key_states: torch.Tensor, val_states: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
        if key_states.shape[0] != slot_mapping.shape[0] or key_states.shape != val_states.shape:
            raise AssertionError("key/value rows must match slot_mapping")
        if key_states.dtype != torch.float16 or val_states.dtype != torch.float16:
            raise TypeError("the KV cache holds fp16")
        n, heads, hs = key_states.shape
        if heads != self.block_info.num_key_value_heads or hs != self.block_info.head_dim:
            raise AssertionError("key/value shape does not match the block geometry")
        k2 = key_states.view(n, heads * hs)
        v2 = val_states.view(n, heads * hs)
        slots = slot_mapping.to(torch.int64)
        _lib.call(fn, n, heads, hs, flags.BLOCK_SIZE, k2.data_ptr(), k2.stride(0),
                  v2.data_ptr(), v2.stride(0), self.layer_key_ptr_table_device.data_ptr(),
                  self.layer_val_ptr_table_device.data_ptr(), self.block_info.head_stride,
                  slots.data_ptr(), _stream(self.device))

    def kv_tensor_to_slots_with_convert(self, key_states: torch.Tensor, val_states: torch.Tensor,
                                        slot_mapping: torch.Tensor) -> None:
        """key/value [num_tokens, kv_heads, head_dim] to their slots."""
        self._copy("dw4_reshape_and_cache", key_states, val_states, slot_mapping)

    def kv_tensor_from_slots_with_convert(self, key_states: torch.Tensor,
                                          val_states: torch.Tensor,
                                          slot_mapping: torch.Tensor) -> None:
        """Slots back to key/value [num_tokens, kv_heads, head_dim]."""
        self._copy("dw4_restore_from_cache", key_states, val_states, slot_mapping)

    def kv_tensor_from_slots_with_convert_with_create(
            self, slot_mapping: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        n = slot_mapping.shape[0]
        shape = (n, self.block_info.num_key_value_heads, self.block_info.head_dim)
        k = torch.empty(shape, dtype=torch.float16, device=self.device)
        v = torch.empty(shape, dtype=torch.float16, device=self.device)
        self.kv_tensor_from_slots_with_convert(k, v, slot_mapping)
        return k, v

    def rope_and_cache(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       sin: torch.Tensor, cos: torch.Tensor, positions: torch.Tensor,
                       block_tables: torch.Tensor,
                       context_lens_out: Optional[torch.Tensor] = None) -> None:
        """One decode token per sequence: rotary embedding of q
        [seqs, heads, hd] and k [seqs, kv_heads, hd] in place at
        ``positions`` (int32 [seqs]), the rotated k and v written to their
        slots through ``block_tables``, and ``positions + 1`` into
        ``context_lens_out`` -- the reference's rope stage,
        ``kv_tensor_to_slots_with_convert`` and context-length update in one
        launch (``dw4_rope_and_cache``)."""
        seqs, heads, hd = q.shape
        kvh = k.shape[1]
        if k.shape != v.shape or k.shape[0] != seqs or hd != self.block_info.head_dim or \
                kvh != self.block_info.num_key_value_heads:
            raise AssertionError("q/k/v shapes do not match the block geometry")
        for t in (q, k, v):
            if t.dtype != torch.float16 or not t.is_contiguous():
                raise TypeError("q, k, v must be contiguous fp16")
        s16, c16, max_pos = rope_tables(sin, cos, hd)
        if context_lens_out is not None and (context_lens_out.dtype != torch.int32 or
                                             context_lens_out.numel() < seqs):
            raise TypeError("context_lens_out must be int32 with one entry per sequence")
        pos = positions.to(torch.int32).contiguous()
        if context_lens_out is not None and _overlaps(pos, context_lens_out):
            raise ValueError("context_lens_out must not share memory with positions: the "
                             "launch reads every position after writing the first lengths")
        tables = block_tables.to(torch.int32).contiguous()
        _lib.call("dw4_rope_and_cache", seqs, heads, kvh, hd, flags.BLOCK_SIZE, q.data_ptr(),
                  q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
                  s16.data_ptr(), c16.data_ptr(), max_pos, pos.data_ptr(), tables.data_ptr(),
                  tables.shape[1], self.layer_key_ptr_table_device.data_ptr(),
                  self.layer_val_ptr_table_device.data_ptr(), self.block_info.head_stride,
                  None if context_lens_out is None else context_lens_out.data_ptr(),
                  _stream(self.device))

    @staticmethod
    def create_contigious_cacher(block_info: BlockInfo, num_blocks: int, device: torch.device,
                                 dtype: torch.dtype = torch.float16) -> "LayerBlocksHolder":
        if dtype.itemsize != block_info.element_size:
            raise AssertionError("dtype does not match the block geometry")
        k = torch.empty((num_blocks, *block_info.key_block_shape), dtype=dtype, device=device)
        v = torch.empty((num_blocks, *block_info.value_block_shape), dtype=dtype, device=device)
        kp = [k[i].data_ptr() for i in range(num_blocks)]
        vp = [v[i].data_ptr() for i in range(num_blocks)]
        kc = torch.tensor(kp, dtype=torch.int64)
        vc = torch.tensor(vp, dtype=torch.int64)
        return LayerBlocksHolder(block_info, kc.to(device), vc.to(device), kc, vc, kp, vp,
                                 contigious_kv_tensor=(k, v))
