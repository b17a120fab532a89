"""CPU oracle for the paged KV cache and decode attention of the stage.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.

Restates in numpy (paths relative to ``/root/reference/After-Revision-DROFELL``):

* ``reshape_and_cache`` -- ``cuda_extends/vllm/cache_kernels.cu:242-285``:
  token t's key row goes to block ``slot // bs`` at
  ``[head][d // x][slot % bs][d % x]`` and its value row to
  ``[head][d][slot % bs]`` (x = 8 for fp16, ``operators/core/block/common.py:7-60``);
  negative slots are padding and skipped;
* ``restore_from_cache`` -- ``cache_kernels.cu:332-375``, the reverse copy;
* ``paged_attention`` -- ``cuda_extends/vllm/attention/attention_kernels.cu``
  (v1 / v2 compute the same function): for sequence s and query head h
  (kv head ``h // (heads // kv_heads)``, ``operators/core/attention/real_page.py:19-22``),
  logits ``scale * q . k_t`` plus ``alibi[h] * (t - ctx + 1)``, softmax over
  the ``ctx = context_lens[s]`` cached tokens (gathered through
  ``block_tables[s][t // bs]``), output ``sum_t p_t v_t``; float64 here.

The reference rounds the softmax weights to fp16 before the value product
and accumulates in fp32; the HIP kernel keeps them in fp32.  Both differ
from this float64 restatement by a few fp16 units in the last place of the
output.  Pinned by ``tests/test_oracle_attention.py`` (round trips, an
independent dense formulation from the token-major tensors, closed forms,
GQA mapping and planted mistakes).
"""
from __future__ import annotations

from typing import Optional

import numpy as np

X = 8  # fp16 elements per 16 bytes: the key layout's innermost dimension


def empty_cache(num_blocks: int, num_kv_heads: int, head_size: int, block_size: int,
                fill: float = np.nan):
    """Contiguous caches [blocks, kvh, hs/8, bs, 8] and [blocks, kvh, hs, bs]."""
    k = np.full((num_blocks, num_kv_heads, head_size // X, block_size, X), fill, np.float16)
    v = np.full((num_blocks, num_kv_heads, head_size, block_size), fill, np.float16)
    return k, v


def reshape_and_cache(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray,
                      value_cache: np.ndarray, slot_mapping: np.ndarray) -> None:
    """key, value [tokens, kvh, hs] into the caches, in place."""
    bs = key_cache.shape[3]
    hs = key.shape[2]
    for t, slot in enumerate(slot_mapping):
        if slot < 0:
            continue
        b, off = divmod(int(slot), bs)
        key_cache[b, :, :, off, :] = key[t].reshape(-1, hs // X, X)
        value_cache[b, :, :, off] = value[t]


def restore_from_cache(key_cache: np.ndarray, value_cache: np.ndarray,
                       slot_mapping: np.ndarray, key: np.ndarray, value: np.ndarray) -> None:
    bs = key_cache.shape[3]
    for t, slot in enumerate(slot_mapping):
        if slot < 0:
            continue
        b, off = divmod(int(slot), bs)
        key[t] = key_cache[b, :, :, off, :].reshape(key.shape[1], -1)
        value[t] = value_cache[b, :, :, off]


def gather_sequence(key_cache: np.ndarray, value_cache: np.ndarray, block_table: np.ndarray,
                    ctx: int):
    """The cached k, v [ctx, kvh, hs] of one sequence (float64)."""
    bs = key_cache.shape[3]
    kvh, hs = value_cache.shape[1], value_cache.shape[2]
    k = np.empty((ctx, kvh, hs))
    v = np.empty((ctx, kvh, hs))
    for t in range(ctx):
        b = int(block_table[t // bs])
        off = t % bs
        k[t] = key_cache[b, :, :, off, :].reshape(kvh, hs)
        v[t] = value_cache[b, :, :, off]
    return k, v


def paged_attention(query: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                    block_tables: np.ndarray, context_lens: np.ndarray, scale: float,
                    alibi: Optional[np.ndarray] = None) -> np.ndarray:
    """query [seqs, heads, hs] -> out [seqs, heads, hs] (float64)."""
    seqs, heads, hs = query.shape
    kvh = value_cache.shape[1]
    group = heads // kvh
    out = np.empty((seqs, heads, hs))
    for s in range(seqs):
        ctx = int(context_lens[s])
        k, v = gather_sequence(key_cache, value_cache, block_tables[s], ctx)
        for h in range(heads):
            g = h // group
            logits = scale * (k[:, g, :] @ query[s, h].astype(np.float64))
            if alibi is not None:
                logits = logits + float(alibi[h]) * (np.arange(ctx) - ctx + 1)
            p = np.exp(logits - logits.max())
            out[s, h] = (p / p.sum()) @ v[:, g, :]
    return out
