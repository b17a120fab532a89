"""Pins of oracle/attention.py (CPU only).

The paged restatement is checked against an independent dense formulation
computed from the token-major K, V before they are cached (no gather), against
closed forms (one token, equal keys, ALiBi with a zero query), the
grouped-query head mapping, an element-by-element layout check of the cache
writes, round trips, and planted mistakes that the checks must catch.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as A


def _setup(seqs, heads, kvh, hs, bs, ctxs, seed):
    rng = np.random.default_rng(seed)
    blocks_per = [(c + bs - 1) // bs for c in ctxs]
    nblocks = sum(blocks_per) + 3
    perm = rng.permutation(nblocks)  # blocks scattered over the cache
    kc, vc = A.empty_cache(nblocks, kvh, hs, bs)
    max_blocks = max(blocks_per)
    tables = np.zeros((seqs, max_blocks), np.int32)
    ks, vs = [], []
    nxt = 0
    for s, c in enumerate(ctxs):
        tables[s, :blocks_per[s]] = perm[nxt:nxt + blocks_per[s]]
        nxt += blocks_per[s]
        k = rng.standard_normal((c, kvh, hs)).astype(np.float16)
        v = rng.standard_normal((c, kvh, hs)).astype(np.float16)
        slots = np.array([tables[s, t // bs] * bs + t % bs for t in range(c)], np.int64)
        A.reshape_and_cache(k, v, kc, vc, slots)
        ks.append(k)
        vs.append(v)
    q = rng.standard_normal((seqs, heads, hs)).astype(np.float16)
    return q, kc, vc, tables, np.array(ctxs, np.int32), ks, vs


def _dense(q, ks, vs, scale, kvh, alibi=None):
    seqs, heads, hs = q.shape
    group = heads // kvh
    out = np.empty((seqs, heads, hs))
    for s in range(seqs):
        k = ks[s].astype(np.float64)
        v = vs[s].astype(np.float64)
        ctx = k.shape[0]
        for h in range(heads):
            lg = scale * k[:, h // group] @ q[s, h].astype(np.float64)
            if alibi is not None:
                lg += alibi[h] * (np.arange(ctx) - ctx + 1)
            w = np.exp(lg - lg.max())
            out[s, h] = (w / w.sum()) @ v[:, h // group]
    return out


def test_cache_layout_element_by_element():
    rng = np.random.default_rng(1)
    kvh, hs, bs = 2, 16, 16
    kc, vc = A.empty_cache(4, kvh, hs, bs)
    key = rng.standard_normal((5, kvh, hs)).astype(np.float16)
    val = rng.standard_normal((5, kvh, hs)).astype(np.float16)
    slots = np.array([0, 17, -1, 63, 33], np.int64)
    A.reshape_and_cache(key, val, kc, vc, slots)
    for t, slot in enumerate(slots):
        if slot < 0:
            continue
        for h in range(kvh):
            for d in range(hs):
                assert kc[slot // bs, h, d // 8, slot % bs, d % 8] == key[t, h, d]
                assert vc[slot // bs, h, d, slot % bs] == val[t, h, d]
    written = {int(s) for s in slots if s >= 0}
    for slot in range(4 * bs):  # every other slot untouched
        if slot not in written:
            assert np.isnan(vc[slot // bs, :, :, slot % bs]).all()


def test_cache_round_trip():
    rng = np.random.default_rng(2)
    kvh, hs, bs = 4, 64, 32
    kc, vc = A.empty_cache(6, kvh, hs, bs)
    key = rng.standard_normal((40, kvh, hs)).astype(np.float16)
    val = rng.standard_normal((40, kvh, hs)).astype(np.float16)
    slots = rng.permutation(6 * bs)[:40].astype(np.int64)
    slots[[3, 9]] = -1
    A.reshape_and_cache(key, val, kc, vc, slots)
    k2 = np.zeros_like(key)
    v2 = np.zeros_like(val)
    A.restore_from_cache(kc, vc, slots, k2, v2)
    keep = slots >= 0
    assert np.array_equal(k2[keep], key[keep]) and np.array_equal(v2[keep], val[keep])
    assert not k2[~keep].any()


@pytest.mark.parametrize("heads,kvh,bs", [(4, 4, 16), (8, 2, 32), (6, 3, 16)])
def test_paged_matches_dense(heads, kvh, bs):
    ctxs = [1, bs, bs + 1, 3 * bs - 5]
    q, kc, vc, tables, lens, ks, vs = _setup(len(ctxs), heads, kvh, 64, bs, ctxs, heads + bs)
    scale = 64 ** -0.5
    got = A.paged_attention(q, kc, vc, tables, lens, scale)
    assert np.allclose(got, _dense(q, ks, vs, scale, kvh), rtol=1e-12, atol=1e-12)


def test_alibi_matches_dense_and_closed_form():
    ctxs = [5, 40]
    q, kc, vc, tables, lens, ks, vs = _setup(2, 4, 4, 64, 16, ctxs, 7)
    slopes = np.array([0.5, 0.25, 0.125, 0.0625])
    got = A.paged_attention(q, kc, vc, tables, lens, 0.125, slopes)
    assert np.allclose(got, _dense(q, ks, vs, 0.125, 4, slopes), rtol=1e-12, atol=1e-12)
    # zero query: weights exp(slope * (t - ctx + 1)) exactly
    z = np.zeros_like(q)
    got = A.paged_attention(z, kc, vc, tables, lens, 0.125, slopes)
    for s, c in enumerate(ctxs):
        for h in range(4):
            w = np.exp(slopes[h] * (np.arange(c) - c + 1))
            ref = (w / w.sum()) @ vs[s][:, h].astype(np.float64)
            assert np.allclose(got[s, h], ref, rtol=1e-12, atol=1e-12)


def test_closed_forms():
    q, kc, vc, tables, lens, ks, vs = _setup(1, 2, 2, 64, 16, [1], 3)
    got = A.paged_attention(q, kc, vc, tables, lens, 0.3)
    assert np.array_equal(got[0], vs[0][0].astype(np.float64))  # one token: out = v
    # equal keys: uniform weights, out = mean of v
    q, kc, vc, tables, lens, ks, vs = _setup(1, 2, 2, 64, 16, [37], 4)
    for t in range(37):
        b, off = tables[0, t // 16], t % 16
        kc[b, :, :, off, :] = kc[tables[0, 0], :, :, 0, :]
    got = A.paged_attention(q, kc, vc, tables, lens, 0.3)
    assert np.allclose(got[0], vs[0].astype(np.float64).mean(axis=0), rtol=1e-12, atol=1e-12)


def test_checks_catch_planted_mistakes():
    """Mutant restatements that a plausible slip would produce all fail the
    dense check used above."""
    ctxs = [20, 33]
    q, kc, vc, tables, lens, ks, vs = _setup(2, 8, 2, 64, 16, ctxs, 11)
    scale = 0.125
    ref = _dense(q, ks, vs, scale, 2)

    def mutant(kind):
        seqs, heads, hs = q.shape
        out = np.empty((seqs, heads, hs))
        for s, c in enumerate(ctxs):
            k, v = A.gather_sequence(kc, vc, tables[s], c)
            if kind == "offset":  # slot offset off by one inside each block
                k2, v2 = A.gather_sequence(kc, vc, tables[s], c + 1)
                k, v = k2[1:], v2[1:]
            for h in range(heads):
                g = h % 2 if kind == "head_map" else h // 4
                sc = 1.0 if kind == "no_scale" else scale
                lg = sc * k[:, g] @ q[s, h].astype(np.float64)
                w = np.exp(lg - lg.max())
                vv = v[:, g]
                if kind == "value_layout":  # value rows read as [slot][d]
                    vv = v[:, g].reshape(-1)[:c * hs].reshape(hs, c).T
                out[s, h] = (w / w.sum()) @ vv
        return out

    for kind in ("offset", "head_map", "no_scale", "value_layout"):
        assert not np.allclose(mutant(kind), ref, rtol=1e-3, atol=1e-3), kind
    assert np.allclose(A.paged_attention(q, kc, vc, tables, lens, scale), ref)


def test_fp16_round_matches_numpy():
    from fractions import Fraction
    rng = np.random.default_rng(5)
    vals = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 5, 3000),
                           [65504.0, 65519.99, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0]])
    for v in vals:
        got = A.fp16_round(Fraction(float(v)))
        want = np.float16(np.float64(v))  # numpy's conversion rounds once, to nearest even
        assert got.view(np.uint16) == want.view(np.uint16) or (np.isnan(got) and np.isnan(want)), v
    # exact ties go to the even neighbour
    assert A.fp16_round(Fraction(2049, 2)) == np.float16(1024.0)
    assert A.fp16_round(Fraction(2051, 2)) == np.float16(1026.0)


def test_fp16_fma_vector_form_matches_exact_scalar_form():
    """The vector fma (float64 TwoSum, then one rounding) against the
    Fraction-based scalar one on random fp16 triples over every exponent
    range, subnormals, signed zeros, exact ties (3 * 341.5 = 1024.5 lies
    halfway between fp16 neighbours) and overflow; a planted double rounding
    (via float32) must disagree somewhere."""
    rng = np.random.default_rng(11)
    n = 4000
    bits = rng.integers(0, 1 << 16, size=(3, n), dtype=np.uint32).astype(np.uint16)
    a, b, c = (v.view(np.float16) for v in bits)
    fin = np.isfinite(a) & np.isfinite(b) & np.isfinite(c)
    a, b, c = a[fin], b[fin], c[fin]
    moderate = (rng.standard_normal((3, 2000)) * 4).astype(np.float16)
    special = np.array([[3, 3, -3, 0, -0.0, 0, 2 ** -24, 2 ** -14, 65504, 255.9],
                        [341.5, 341.5, 341.5, 5, 1, -0.0, 2 ** -24, 2 ** -10, 2, 256.1],
                        [0, 2 ** -24, -(2 ** -24), -0.0, -0.0, -0.0, 1, 0, 65504, -1]],
                       dtype=np.float16)
    a = np.concatenate([a, moderate[0], special[0]])
    b = np.concatenate([b, moderate[1], special[1]])
    c = np.concatenate([c, moderate[2], special[2]])
    got = A.fp16_fma(a, b, c)
    want = np.array([A._fp16_fma(x, y, z) for x, y, z in zip(a, b, c)], np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert A.fp16_fma(np.float16(3), np.float16(341.5), np.float16(0)) == np.float16(1024)
    sloppy = (a.astype(np.float32) * b.astype(np.float32) + c.astype(np.float32)).astype(np.float16)
    assert not np.array_equal(sloppy.view(np.uint16), want.view(np.uint16))


def test_rope_closed_forms_and_mistakes():
    rng = np.random.default_rng(8)
    hd, heads = 16, 2
    sin, cos = A.rope_tables(8, hd)
    x = rng.standard_normal((2, 3 * heads, hd)).astype(np.float16)
    # position 0: sin = 0, cos = 1 -> identity
    y0 = A.rope(x[:, :heads], sin, cos, heads, 0)
    assert np.array_equal(y0, x[:, :heads])
    # a rotation keeps each (l, r) pair's length (to fp16 rounding)
    y = A.rope(x, sin, cos, heads, 2)
    h = hd // 2
    n0 = x[..., :h].astype(np.float64) ** 2 + x[..., h:].astype(np.float64) ** 2
    n1 = y[..., :h].astype(np.float64) ** 2 + y[..., h:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=5e-3, atol=1e-3)
    # matches the float64 rotation to fp16 accuracy
    for b in range(2):
        for r in range(3 * heads):
            p = 2 + r // heads
            c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
            l, rr = x[b, r, :h].astype(np.float64), x[b, r, h:].astype(np.float64)
            ref = np.concatenate([l * c[:h] - rr * s[:h], rr * c[h:] + l * s[h:]])
            assert np.allclose(y[b, r], ref, rtol=2e-3, atol=2e-3)
    # per-batch positions and rows outside the table
    y2 = A.rope(x, sin, cos, heads, -1, np.array([2, 6]))
    assert np.array_equal(y2[0], y[0])
    assert np.array_equal(y2[1, 4:], x[1, 4:])  # positions 8 and up: unchanged
    # planted mistakes: halves swapped, or the token index ignored
    bad = y.copy()
    bad[..., :h], bad[..., h:] = y[..., h:], y[..., :h]
    assert not np.array_equal(bad, y)
    assert not np.array_equal(A.rope(x, sin, cos, 3 * heads, 2), y)
