"""Attention geometry (the reference's ``operators/core/attention/common.py``,
paths relative to ``/root/reference/After-Revision-DROFELL``); head sizes are
those the HIP decode kernel serves."""
from __future__ import annotations

from dataclasses import dataclass

_SUPPORTED_HEAD_SIZES = [64, 80, 96, 112, 128, 256]


@dataclass
class AttentionConfig:
    hidden_size: int
    head_dim: int
    num_query_heads: int
    num_key_value_heads: int
    num_key_value_groups: int

    def __post_init__(self) -> None:
        if self.hidden_size != self.head_dim * self.num_query_heads:
            raise AssertionError("hidden_size must be head_dim * num_query_heads")
        if self.num_key_value_heads * self.num_key_value_groups != self.num_query_heads:
            raise AssertionError("kv heads * groups must equal query heads")
        if self.head_dim not in _SUPPORTED_HEAD_SIZES:
            raise AssertionError(f"head_dim {self.head_dim} not in {_SUPPORTED_HEAD_SIZES}")
