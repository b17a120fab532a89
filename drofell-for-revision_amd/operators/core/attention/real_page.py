"""Paged-attention decode on the HIP library.

Mirrors ``PagedAttention`` of the reference's ``operators/core/attention/real_page.py:13-189``
(paths relative to ``/root/reference/After-Revision-DROFELL``): the same
constructor and ``forward(query, context_len_max, context_lens, block_tables,
kv_cacher, alibi_slopes)``, with the pointer-table and contiguous cachers
served by one kernel (``dw4_paged_attention``; a contiguous cacher also
carries its pointer tables).  The reference's v1 / v2 choice becomes the
library's own partitioning of long contexts; its scratch tensors become one
workspace, sized by ``dw4_paged_attention_workspace_size``.
"""
from __future__ import annotations

from typing import Optional

import torch

from hip_extends import _lib

from ... import flags
from ..block.real import LayerBlocksHolder
from .common import AttentionConfig


class PagedAttention:
    def __init__(self, config: AttentionConfig) -> None:
        self.cfg = config
        self.scale = self.cfg.head_dim ** -0.5
        self.head_mapping = torch.repeat_interleave(
            torch.arange(self.cfg.num_key_value_heads, dtype=torch.int32),
            self.cfg.num_key_value_groups)
        self._workspace: Optional[torch.Tensor] = None

    def workspace(self, num_seqs: int, context_len_max: int, device: torch.device) -> torch.Tensor:
        nbytes = _lib.paged_attention_workspace_size(
            num_seqs, self.cfg.num_query_heads, self.cfg.num_key_value_heads, self.cfg.head_dim,
            flags.BLOCK_SIZE, context_len_max)
        if self._workspace is None or self._workspace.numel() < nbytes or \
                self._workspace.device != device:
            self._workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
        return self._workspace

    def forward(self, query: torch.Tensor, context_len_max: int, context_lens: torch.Tensor,
                block_tables: torch.Tensor, kv_cacher: LayerBlocksHolder,
                alibi_slopes: Optional[torch.Tensor] = None) -> torch.Tensor:
        """query [bsz, num_query_heads, head_dim] -> out of the same shape."""
        num_seqs, num_heads, head_dim = query.shape
        if num_heads != self.cfg.num_query_heads or head_dim != self.cfg.head_dim:
            raise AssertionError("query shape does not match the attention config")
        if query.dtype != torch.float16:
            raise TypeError("paged attention runs on fp16 queries")
        q = query if query.is_contiguous() else query.contiguous()
        output = torch.empty_like(q)
        tables = block_tables.to(torch.int32).contiguous()
        lens = context_lens.to(torch.int32).contiguous()
        alibi = None if alibi_slopes is None else alibi_slopes.to(torch.float32).contiguous()
        ws = self.workspace(num_seqs, context_len_max, q.device)
        _lib.call("dw4_paged_attention", num_seqs, num_heads, self.cfg.num_key_value_heads,
                  head_dim, flags.BLOCK_SIZE, q.data_ptr(), q.stride(0), output.data_ptr(),
                  output.stride(0), kv_cacher.layer_key_ptr_table_device.data_ptr(),
                  kv_cacher.layer_val_ptr_table_device.data_ptr(),
                  kv_cacher.block_info.head_stride, float(self.scale), tables.data_ptr(),
                  tables.shape[1], lens.data_ptr(), int(context_len_max),
                  None if alibi is None else alibi.data_ptr(), ws.data_ptr(), ws.numel(),
                  torch.cuda.current_stream(q.device).cuda_stream)
        return output
