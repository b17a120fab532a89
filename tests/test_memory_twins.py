"""Memory twins of the quantized linears (host-only: shapes, dtypes and the
library's workspace sizing; no GPU).

The twins must mirror, tensor for tensor, what the HIP-backed modules keep on
the device after post_init, since the reference's planner decides placement
from them.  Here the twin's checkpoint buffers are compared with a
QuantLinear built on the host, and the workspace with dw4_query_sizes.
"""
from __future__ import annotations

import pytest
import torch

from hip_extends import _lib
from hip_extends.w4a16 import TuningParams
from operators.core.linear.memory import (CacheV2MemoryModel, MarlinQuantLinearMakerMemoryModel,
                                          QuantLinearMakerMemoryModel, QuantLinearMemoryModel,
                                          W4A16LibraryMemoryModel)
from operators.core.linear.real_quant import QuantLinear
from operators.core.memory.static import MemoryModule, MemoryTensor


@pytest.mark.parametrize("k,n,g,act,bias", [(4096, 4096, 128, False, False),
                                            (4096, 11008, 128, True, True),
                                            (11008, 4096, -1, False, False)])
def test_twin_buffers_match_module(k, n, g, act, bias):
    twin = QuantLinearMemoryModel(g, k, n, bias, act)
    mod = QuantLinear(g, k, n, bias, act)
    names = dict(mod.named_buffers())
    assert set(names) == {"qweight", "qzeros", "scales", "g_idx"} | ({"bias"} if bias else set())
    for name, buf in names.items():
        t = getattr(twin, name)
        assert t.size == tuple(buf.shape), name
        assert t.dtype[1] == buf.element_size(), name
    cache = CacheV2MemoryModel()
    twin.post_init(TuningParams(MAX_M=64), cache)
    assert twin.perm.size == ((k,) if act else (0,))
    cache.init_cache()
    ws = _lib.query_sizes(k, n, twin.group_size, act, 64)["workspace"]
    assert cache.workspace.requested == max(16, ws)
    assert cache.temp_weight.numel() == k * n  # the dense route's buffer, once requested


def test_group_total_and_shared_perm():
    maker = QuantLinearMakerMemoryModel(128, True)
    hidden, inter = 4096, 11008
    q, k, v, o = (maker.make_linear(hidden, hidden) for _ in range(4))
    gate, up = maker.make_linear(hidden, inter), maker.make_linear(hidden, inter)
    down = maker.make_linear(inter, hidden)
    cache = CacheV2MemoryModel()
    maker.post_init(TuningParams(MAX_M=64), cache)
    cache.init_cache()
    root = MemoryModule()
    root.mount_list([q, k, v, o, gate, up, down], "proj")
    root.cache = cache.workspace

    def packed(kk, nn):
        return kk * nn // 2 + (kk // 128) * nn // 2 + 2 * (kk // 128) * nn + 4 * kk  # + g_idx

    weights = 4 * packed(hidden, hidden) + 2 * packed(hidden, inter) + packed(inter, hidden)
    perms = 4 * (6 * hidden + inter)
    assert root.memory == weights + perms + cache.workspace.requested
    maker.share_perm([q, k, v])
    maker.share_perm([gate, up])
    assert root.memory == weights + 4 * (3 * hidden + inter) + cache.workspace.requested
    with pytest.raises(AssertionError):
        maker.post_init(TuningParams(), cache)


def test_workspace_is_group_maximum():
    maker = QuantLinearMakerMemoryModel(128, False)
    a = maker.make_linear(4096, 4096)
    b = maker.make_linear(11008, 4096)
    cache = CacheV2MemoryModel()
    maker.post_init(TuningParams(MAX_M=256), cache)
    want = max(_lib.query_sizes(4096, 4096, 128, False, 256)["workspace"],
               _lib.query_sizes(11008, 4096, 128, False, 256)["workspace"])
    assert cache.workspace_size == want
    assert a.cache_v2 is cache and b.cache_v2 is cache


def test_marlin_twin():
    maker = MarlinQuantLinearMakerMemoryModel(128, True)
    q, k, v = (maker.make_linear(4096, 4096) for _ in range(3))
    qkv = maker.merge([q, k, v])
    assert maker.quant_linears == [qkv]
    assert qkv.qweight.numel() * 4 == 4096 * 12288 // 2
    assert qkv.g_idx_sort_indices.size == (4096,)
    assert qkv.workspace.size == (256 * 4,)
    maker.post_init()
    assert maker.dense_cache._temp_weight.numel() == 4096 * 12288
    with pytest.raises(RuntimeError):
        maker.post_init()
    with pytest.raises(ValueError):
        maker.make_linear(4096, 4096, bias=True)


def test_memory_tensor_basics():
    t = MemoryTensor((3, 5), torch.float16)
    assert t.requested == 30 and t.memory == 30
    assert MemoryTensor((3, 5), torch.float16, cpu=True).requested == 0
    m = MemoryModule()
    m.a = t
    m.b = t  # shared: counted once
    m.c = MemoryTensor((2,), torch.int32)
    assert m.memory == 38
    assert [n for n, _ in m.named_parameters()] == ["a", "b", "c"]


def test_library_twin_counts_the_noalloc_scratch():
    """The per-GPU static array of dw4_gemm_noalloc (the header's
    DW4_NOALLOC_SCRATCH_BYTES) is in the library twin, counted once when a
    device plan mounts it beside a decoder group's twins."""
    import os
    import re

    header = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                               "include", "drofell_w4a16.h")).read()
    shift = int(re.search(r"#define DW4_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << 20\)",
                          header).group(1))
    assert _lib.NOALLOC_SCRATCH_BYTES == shift << 20
    lib_twin = W4A16LibraryMemoryModel()
    assert lib_twin.memory == _lib.NOALLOC_SCRATCH_BYTES
    maker = QuantLinearMakerMemoryModel(128, False)
    lin = maker.make_linear(4096, 4096)
    cache = CacheV2MemoryModel()
    maker.post_init(TuningParams(MAX_M=64), cache)
    cache.init_cache()
    device = MemoryModule()
    device.library = lib_twin
    device.proj = lin
    device.workspace = cache.workspace  # the linear's twin holds it already: counted once
    assert device.memory == lib_twin.memory + lin.memory
