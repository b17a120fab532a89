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
* ``rope`` -- ``cuda_extends/exllama/fuse_v2/rope.cu:24-91`` (rotate-half
  rotary embedding in fp16 arithmetic, each product and fma rounded once;
  ``fp16_round`` is an exact round-to-nearest-even of a rational value);
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


def fp16_round(v) -> np.float16:
    """Exact value ``v`` (a Fraction or int) rounded once to IEEE binary16,
    to nearest, ties to even (subnormals down to 2**-24, overflow to inf)."""
    from fractions import Fraction
    v = Fraction(v)
    if v == 0:
        return np.float16(0.0)
    sign = -1 if v < 0 else 1
    a = -v if v < 0 else v
    if a >= 65520:  # halfway between 65504 and 2**16 and above
        return np.float16(sign * np.inf)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1  # now 2**e <= a < 2**(e + 1)
    q = Fraction(2) ** (max(e, -14) - 10)  # spacing of binary16 values near a
    n = a / q
    m = n.numerator // n.denominator
    rem = n - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return np.float16(sign * float(m * q))


def _fp16_fma(a: np.float16, b: np.float16, c: np.float16) -> np.float16:
    """a * b + c with one rounding (IEEE fusedMultiplyAdd in binary16)."""
    from fractions import Fraction
    p = Fraction(float(a)) * Fraction(float(b))
    exact = p + Fraction(float(c))
    if exact == 0:
        # an exact zero is +0 under round-to-nearest, unless the product and
        # the addend are both zeros of negative sign
        neg_product = p == 0 and bool(np.signbit(a) != np.signbit(b))
        neg_addend = float(c) == 0 and bool(np.signbit(c))
        return np.float16(-0.0) if (neg_product and neg_addend) else np.float16(0.0)
    return fp16_round(exact)


def fp16_fma(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Elementwise ``a * b + c`` of fp16 arrays with one rounding to fp16
    (the vector form of :func:`_fp16_fma`, which pins it).

    The product of two fp16 values is exact in float64; Knuth's TwoSum
    gives ``p + c = s + err`` exactly with ``s`` the float64 sum.  Rounding
    ``s`` to fp16 (numpy: to nearest, ties to even) is the correct rounding
    of ``s + err`` except when ``s`` is exactly halfway between two fp16
    values and ``err`` is not zero: every such midpoint is a float64 value,
    so ``s + err`` cannot lie beyond one, and then ``err``'s sign picks the
    neighbour.  Signed zeros follow IEEE addition of the float64 values."""
    a64 = np.asarray(a, np.float16).astype(np.float64)
    b64 = np.asarray(b, np.float16).astype(np.float64)
    c64 = np.asarray(c, np.float16).astype(np.float64)
    p = a64 * b64
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)
    with np.errstate(over="ignore"):
        r = s.astype(np.float16)
        up = np.nextafter(r, np.float16(np.inf))
        down = np.nextafter(r, np.float16(-np.inf))
    other = np.where(s > r.astype(np.float64), up, down)
    mid = (r.astype(np.float64) + other.astype(np.float64)) / 2
    tie = (s == mid) & (err != 0) & np.isfinite(r) & np.isfinite(other)
    toward_other = np.sign(err) == np.sign(other.astype(np.float64) - r.astype(np.float64))
    return np.where(tie & toward_other, other, r)


def rope(x: np.ndarray, sin: np.ndarray, cos: np.ndarray, num_heads: int, past_len: int,
         past_lens: Optional[np.ndarray] = None) -> np.ndarray:
    """``cuda_extends/exllama/fuse_v2/rope.cu:24-91`` on fp16 x
    [batch, rows, hd] (row = token * heads + head): position
    ``past + row // heads``; pair (l, r) = (x[c], x[c + hd/2]):
    ``l' = fma(l, cos[c], fp16(r * -sin[c]))``,
    ``r' = fma(r, cos[c + hd/2], fp16(l * sin[c + hd/2]))``, every product
    and fma rounded once to fp16 (:func:`fp16_fma`).  Rows whose position
    falls outside the tables are returned unchanged."""
    out = x.copy()
    batch, rows, hd = x.shape
    half = hd // 2
    for b in range(batch):
        base = past_len if past_len >= 0 else int(past_lens[b])
        pos = base + np.arange(rows) // num_heads
        ok = (pos >= 0) & (pos < sin.shape[0])
        if not ok.any():
            continue
        p = pos[ok]
        lv, rv = x[b, ok, :half], x[b, ok, half:]
        s_lo, s_hi = sin[p, :half], sin[p, half:]
        c_lo, c_hi = cos[p, :half], cos[p, half:]
        # fp16 operands: each float32 product is exact, then rounded once
        ls = (rv.astype(np.float32) * -s_lo.astype(np.float32)).astype(np.float16)
        rs = (lv.astype(np.float32) * s_hi.astype(np.float32)).astype(np.float16)
        out[b, ok, :half] = fp16_fma(lv, c_lo, ls)
        out[b, ok, half:] = fp16_fma(rv, c_hi, rs)
    return out


def rope_tables(max_pos: int, hd: int, theta: float = 10000.0):
    """Llama's fp16 sin/cos tables [max_pos, hd] (the rotate-half layout)."""
    inv = 1.0 / theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = np.outer(np.arange(max_pos, dtype=np.float64), inv)
    ang = np.concatenate([ang, ang], axis=1)
    return np.sin(ang).astype(np.float16), np.cos(ang).astype(np.float16)
