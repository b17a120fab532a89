"""Pins the CPU oracle (oracle/gptq.py) before anything is checked against it.

The reference ships no golden vectors, known-answer tests or fixtures for
the W4A16 path, so every oracle function is pinned here by what the
mathematics fixes: hand-built known answers for the nibble addressing, an
exhaustive dequantisation table (16 q x 16 stored zeros x all 65,536 fp16
scale patterns) against an independent integer round-to-nearest-even,
exact rational brute force for tiny GEMMs, closed-form special cases and
the act-order permutation invariance.  The mutation tests at the end plant
plausible mistakes in copies of the oracle and show that these checks
catch them.
"""
from __future__ import annotations

import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import gptq

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "gptq_small.npz")


# ---------------------------------------------------------------------------
# independent helpers (integer arithmetic only)
# ---------------------------------------------------------------------------
def fp16_rne_times_int(s_bits: np.ndarray, d: int) -> np.ndarray:
    """fp16 bit patterns of RNE(s * d) for fp16 patterns s and an integer d.

    Pure integer arithmetic: decompose s into mantissa * 2^e, form the exact
    integer product, round to the fp16 quantum with ties to even.  NaN
    results are returned as 0x7E00.
    """
    s_bits = s_bits.astype(np.int64)
    sign = ((s_bits >> 15) & 1) ^ (1 if d < 0 else 0)
    e = (s_bits >> 10) & 0x1F
    f = s_bits & 0x3FF
    mant = np.where(e == 0, f, f | 0x400)
    exp2 = np.where(e == 0, -24, e - 25)
    P = mant * abs(d)
    out = np.zeros_like(s_bits)
    # bit length of P
    bl = np.zeros_like(P)
    for k in range(20):
        bl += (P >> k) > 0
    L = bl - 1 + exp2
    q_exp = np.maximum(L - 10, -24)
    sh = q_exp - exp2
    m = np.where(sh <= 0, P << np.maximum(-sh, 0), P >> np.maximum(sh, 0))
    shp = np.maximum(sh, 1)
    rem = np.where(sh > 0, P & ((np.int64(1) << shp) - 1), 0)
    half = np.where(sh > 0, np.int64(1) << (shp - 1), 0)
    up = (sh > 0) & ((rem > half) | ((rem == half) & ((m & 1) == 1)))
    m = m + up
    carry = m >= 2048
    m = np.where(carry, m >> 1, m)
    q_exp = np.where(carry, q_exp + 1, q_exp)
    E = q_exp + 25
    normal = m >= 1024
    bits = np.where(normal, (E << 10) | (m - 1024), m)
    bits = np.where(normal & (E >= 31), 0x7C00, bits)
    bits = np.where(P == 0, 0, bits)
    # zero keeps the scale's sign when d == 0 (IEEE: s * +0)
    sign = np.where(P == 0, (s_bits >> 15) & 1 if d == 0 else sign, sign)
    out = bits | (sign << 15)
    # specials: inf * nonzero = inf, inf * 0 = NaN, NaN -> NaN
    is_inf = (e == 31) & (f == 0)
    is_nan = (e == 31) & (f != 0)
    out = np.where(is_inf, (0x7E00 if d == 0 else (0x7C00 | (sign << 15))), out)
    out = np.where(is_nan, 0x7E00, out)
    return out.astype(np.uint16)


def fp16_to_fraction(bits: int) -> Fraction:
    e = (bits >> 10) & 0x1F
    f = bits & 0x3FF
    sgn = -1 if bits >> 15 else 1
    assert e != 31
    if e == 0:
        return sgn * Fraction(f, 2 ** 24)
    return sgn * Fraction(f | 0x400, 2 ** 25) * Fraction(2) ** e


def same_fp16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    a = a_bits.view(np.float16)
    b = b_bits.view(np.float16)
    return (a_bits == b_bits) | (np.isnan(a) & np.isnan(b))


def exhaustive_case():
    """Buffers whose dequantisation covers every (q, stored zero, scale)."""
    scales_row = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    K, N, G = 256, 65536, 16
    q = np.zeros((K, N), dtype=np.uint8)
    g_idx = np.zeros(K, dtype=np.int32)
    for z in range(16):
        for qq in range(16):
            r = z * 16 + qq
            q[r, :] = qq
            g_idx[r] = z
    zeros = np.repeat(np.arange(16, dtype=np.uint8)[:, None], N, axis=1)
    scales = np.repeat(scales_row[None, :], G, axis=0).view(np.float16)
    return gptq.pack_qweight(q), gptq.pack_qzeros(zeros), scales, g_idx, scales_row


# ---------------------------------------------------------------------------
# nibble addressing
# ---------------------------------------------------------------------------
def test_qweight_nibble_addressing_known_answer():
    # word 0x76543210 in column 0 -> rows 0..7 hold 0..7; column 1 holds
    # 0xFEDCBA98 -> rows 0..7 hold 8..15 (row k at bits 4*(k%8))
    qweight = np.array([[0x76543210, 0xFEDCBA98 - 2 ** 32]], dtype=np.int64).astype(np.int32)
    q = gptq.unpack_qweight(qweight)
    assert q.shape == (8, 2)
    assert q[:, 0].tolist() == list(range(8))
    assert q[:, 1].tolist() == list(range(8, 16))


def test_qzeros_addressing_known_answer():
    # one group, 16 columns: column n's stored zero sits at bits 4*(n%8) of
    # word n // 8 (packed along N, unlike qweight)
    qzeros = np.array([[0x76543210, 0xFEDCBA98 - 2 ** 32]], dtype=np.int64).astype(np.int32)
    z = gptq.unpack_qzeros(qzeros)
    assert z.shape == (1, 16)
    assert z[0].tolist() == list(range(16))


@pytest.mark.parametrize("k,n", [(8, 8), (64, 24), (256, 512)])
def test_pack_unpack_roundtrip(k, n):
    rng = np.random.default_rng(k * 1000 + n)
    q = rng.integers(0, 16, size=(k, n), dtype=np.uint8)
    assert np.array_equal(gptq.unpack_qweight(gptq.pack_qweight(q)), q)
    z = rng.integers(0, 16, size=(k // 8, n), dtype=np.uint8)
    assert np.array_equal(gptq.unpack_qzeros(gptq.pack_qzeros(z)), z)


def test_synthetic_packing_matches_oracle():
    from gptq_synth import make_layer
    lay = make_layer(256, 64, 64, seed=3)
    import torch
    gen = torch.Generator().manual_seed(3)
    q = torch.randint(0, 16, (256, 64), generator=gen, dtype=torch.int32).numpy()
    z = torch.randint(0, 16, (4, 64), generator=gen, dtype=torch.int32).numpy()
    assert np.array_equal(gptq.unpack_qweight(lay.qweight.numpy()), q)
    assert np.array_equal(gptq.unpack_qzeros(lay.qzeros.numpy()), z)
    sym = make_layer(256, 64, 128, seed=0, symmetric=True)
    assert np.all(sym.qzeros.numpy().view(np.uint32) == 0x77777777)


# ---------------------------------------------------------------------------
# dequantisation
# ---------------------------------------------------------------------------
def test_effective_zero_is_stored_plus_one():
    # q = 8 with stored zero 7 (symmetric uint4b8) dequantises to exactly 0;
    # q = 15 -> 7 * s; q = 0 -> -8 * s
    q = np.array([[8], [15], [0], [8], [8], [8], [8], [8]], dtype=np.uint8)
    q = np.repeat(q, 8, axis=1)
    qweight = gptq.pack_qweight(q)
    qzeros = gptq.pack_qzeros(np.full((1, 8), 7, dtype=np.uint8))
    scales = np.full((1, 8), 0.5, dtype=np.float16)
    w = gptq.dequantize(qweight, qzeros, scales, np.zeros(8, dtype=np.int32))
    assert w[0, 0] == 0 and w[1, 0] == 3.5 and w[2, 0] == -4.0


def test_dequant_exhaustive_known_answer_table():
    qweight, qzeros, scales, g_idx, scales_row = exhaustive_case()
    w = gptq.dequantize(qweight, qzeros, scales, g_idx).view(np.uint16)
    for z in range(16):
        for qq in range(16):
            d = qq - (z + 1)
            expect = fp16_rne_times_int(scales_row, d)
            got = w[z * 16 + qq]
            ok = same_fp16(got, expect)
            assert ok.all(), (z, qq, np.flatnonzero(~ok)[:5])


def test_independent_rne_against_fractions():
    # spot-check the integer RNE helper itself against exact rationals,
    # including ties, subnormals and overflow
    rng = np.random.default_rng(7)
    pats = np.concatenate([rng.integers(0, 0x7C00, 400), [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x3C00]])
    for d in (-16, -15, -3, -1, 1, 3, 7, 13, 14):
        got = fp16_rne_times_int(pats.astype(np.uint16), d)
        for p, g in zip(pats.tolist(), got.tolist()):
            exact = fp16_to_fraction(p) * d
            # brute-force nearest fp16 by scanning neighbours of the float result
            approx = np.float16(float(exact))
            cands = [int(approx.view(np.uint16)) + o for o in (-2, -1, 0, 1, 2)]
            best = None
            for c in cands:
                c &= 0xFFFF
                if ((c >> 10) & 0x1F) == 31:
                    continue
                err = abs(fp16_to_fraction(c) - exact)
                key = (err, (c & 0x3FF) & 1)  # ties -> even mantissa
                if best is None or key < best[0]:
                    best = (key, c)
            if abs(exact) >= 65520:  # rounds to infinity
                assert (g & 0x7FFF) == 0x7C00
            elif exact == 0:
                assert (g & 0x7FFF) == 0
            else:
                assert fp16_to_fraction(g) == fp16_to_fraction(best[1]), (p, d, g, best)


def test_dequant_row_order_follows_g_idx():
    # two groups with different scales; rows assigned by an arbitrary g_idx
    rng = np.random.default_rng(11)
    K, N = 64, 16
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(2, N), dtype=np.uint8)
    s = np.array([[0.25] * N, [2.0] * N], dtype=np.float16)
    g_idx = rng.permutation(np.repeat([0, 1], K // 2)).astype(np.int32)
    w = gptq.dequantize(gptq.pack_qweight(q), gptq.pack_qzeros(z), s, g_idx)
    for k in range(K):
        g = g_idx[k]
        expect = (q[k].astype(np.float64) - z[g] - 1) * float(s[g, 0])
        assert np.array_equal(w[k].astype(np.float64), expect)


# ---------------------------------------------------------------------------
# act-order
# ---------------------------------------------------------------------------
def test_act_order_perm_known_answer():
    g_idx = np.array([1, 0, 1, 0, 2, 2, 0, 1, 2], dtype=np.int32)
    perm = gptq.act_order_perm(g_idx, 3)
    assert perm.tolist() == [1, 3, 6, 0, 2, 7, 4, 5, 8]


def test_act_order_perm_properties():
    rng = np.random.default_rng(5)
    K, g = 1024, 128
    g_idx = (rng.permutation(K) // g).astype(np.int32)
    perm = gptq.act_order_perm(g_idx, K // g)
    assert sorted(perm.tolist()) == list(range(K))
    sorted_groups = g_idx[perm]
    assert np.all(np.diff(sorted_groups) >= 0)
    assert np.array_equal(sorted_groups, np.arange(K) // g)  # uniform groups
    for grp in range(K // g):
        rows = perm[sorted_groups == grp]
        assert np.all(np.diff(rows) > 0)  # stable


def test_act_order_permutation_invariance():
    rng = np.random.default_rng(9)
    K, N, M, g = 256, 32, 3, 64
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // g, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // g, N))) * 0.01 + 1e-3).astype(np.float16)
    g_idx = (rng.permutation(K) // g).astype(np.int32)
    x = rng.standard_normal((M, K)).astype(np.float16)
    y = gptq.gemm_ref(x, gptq.dequantize(gptq.pack_qweight(q), gptq.pack_qzeros(z), s, g_idx))
    pi = rng.permutation(K)
    y2 = gptq.gemm_ref(x[:, pi], gptq.dequantize(gptq.pack_qweight(q[pi]), gptq.pack_qzeros(z),
                                                 s, g_idx[pi]))
    assert np.allclose(y, y2, rtol=1e-12, atol=1e-12)
    # the sorted (repacked) order with groups k'//g gives the same product
    perm = gptq.act_order_perm(g_idx, K // g)
    y3 = gptq.gemm_ref(x[:, perm], gptq.dequantize(gptq.pack_qweight(q[perm]), gptq.pack_qzeros(z),
                                                   s, (np.arange(K) // g).astype(np.int32)))
    assert np.allclose(y, y3, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def test_gemm_bruteforce_exact_tiny():
    rng = np.random.default_rng(13)
    K, N, M, g = 32, 8, 2, 32
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(1, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((1, N))) * 0.05 + 1e-3).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    qweight, qzeros = gptq.pack_qweight(q), gptq.pack_qzeros(z)
    g_idx = np.zeros(K, dtype=np.int32)
    y = gptq.gemm_ref(x, gptq.dequantize(qweight, qzeros, s, g_idx))
    for m in range(M):
        for n in range(N):
            sb = int(s[0, n].view(np.uint16))
            acc = Fraction(0)
            for k in range(K):
                d = int(q[k, n]) - int(z[0, n]) - 1
                wbits = int(fp16_rne_times_int(np.array([sb], np.uint16), d)[0])
                acc += fp16_to_fraction(int(x[m, k].view(np.uint16))) * fp16_to_fraction(wbits)
            assert abs(Fraction(y[m, n]) - acc) <= abs(acc) * Fraction(1, 10 ** 12) + Fraction(1, 10 ** 15)


def test_gemm_special_cases():
    rng = np.random.default_rng(17)
    K, N, M = 128, 16, 4
    x = rng.standard_normal((M, K)).astype(np.float16)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(1, N), dtype=np.uint8)
    g_idx = np.zeros(K, dtype=np.int32)
    # all scales zero -> y == 0
    y = gptq.forward(x, gptq.pack_qweight(q), gptq.pack_qzeros(z), np.zeros((1, N), np.float16), g_idx)
    assert not np.any(y.astype(np.float32))
    # q == effective zero everywhere -> y == 0
    zq = np.full((1, N), 6, dtype=np.uint8)
    qq = np.full((K, N), 7, dtype=np.uint8)
    y = gptq.forward(x, gptq.pack_qweight(qq), gptq.pack_qzeros(zq), np.ones((1, N), np.float16), g_idx)
    assert not np.any(y.astype(np.float32))
    # one non-zero weight per column -> exact gather of x times that weight
    qq = np.full((K, N), 7, dtype=np.uint8)
    rows = rng.integers(0, K, size=N)
    qq[rows, np.arange(N)] = 10  # 10 - 7 = 3
    s = np.full((1, N), 0.5, dtype=np.float16)
    y = gptq.forward(x, gptq.pack_qweight(qq), gptq.pack_qzeros(zq), s, g_idx)
    expect = (x[:, rows].astype(np.float64) * 1.5).astype(np.float16)
    assert np.array_equal(y, expect)


def test_tolerance_rule():
    ref = np.array([[1.0, -2.0, 0.5]])
    ok, worst = gptq.within_tolerance(ref + 0.039, ref)
    assert ok and worst < 1.0
    ok, worst = gptq.within_tolerance(ref + 0.041, ref)
    assert not ok


# ---------------------------------------------------------------------------
# committed fixtures (tests/golden/make_golden.py)
# ---------------------------------------------------------------------------
def test_golden_fixtures_reproduce():
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    assert len(names) >= 5
    for name in names:
        qweight, qzeros = data[f"{name}/qweight"], data[f"{name}/qzeros"]
        scales, g_idx = data[f"{name}/scales"], data[f"{name}/g_idx"]
        w = gptq.dequantize(qweight, qzeros, scales, g_idx)
        assert np.array_equal(w.view(np.uint16), data[f"{name}/w"]), name
        bias = data[f"{name}/bias"] if f"{name}/bias" in data.files else None
        y = gptq.forward(data[f"{name}/x"], qweight, qzeros, scales, g_idx, bias)
        assert np.array_equal(y.view(np.uint16), data[f"{name}/y"]), name


# ---------------------------------------------------------------------------
# mutation tests: plausible mistakes planted in copies of the oracle must fail
# ---------------------------------------------------------------------------
def _mutant_dequant_no_plus_one(qweight, qzeros, scales, g_idx):
    q = gptq.unpack_qweight(qweight).astype(np.int16)
    z = gptq.unpack_qzeros(qzeros).astype(np.int16)  # planted: stored zero used directly
    d = (q - z[g_idx]).astype(np.float32)
    return (scales[g_idx].astype(np.float32) * d).astype(np.float16)


def _mutant_dequant_prescaled_zero(qweight, qzeros, scales, g_idx):
    # planted: s*q - s*z in fp16 (two roundings), the pre-scaled-zero form
    q = gptq.unpack_qweight(qweight).astype(np.float16)
    z = (gptq.unpack_qzeros(qzeros).astype(np.int16) + 1).astype(np.float16)
    s = scales[g_idx]
    return (s * q - s * z[g_idx]).astype(np.float16)


def _mutant_qzeros_transposed(qzeros):
    # planted: zeros addressed like qweight (packed along the other axis)
    w = gptq._as_u32(qzeros)
    g, nw = w.shape
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, :, None]
    return ((w[:, None, :] >> shifts) & 0xF).reshape(g * 8, nw).astype(np.uint8)


@pytest.mark.parametrize("mutant", [_mutant_dequant_no_plus_one, _mutant_dequant_prescaled_zero])
def test_kat_catches_planted_dequant_mistakes(mutant):
    qweight, qzeros, scales, g_idx, scales_row = exhaustive_case()
    sub = slice(0, 4096)  # a slice of the scale patterns suffices to fail
    w = mutant(qweight[:, sub], qzeros[:, : 4096 // 8], scales[:, sub], g_idx).view(np.uint16)
    bad = 0
    for z in range(16):
        for qq in range(16):
            expect = fp16_rne_times_int(scales_row[sub], qq - (z + 1))
            bad += int((~same_fp16(w[z * 16 + qq], expect)).sum())
    assert bad > 0


def test_known_answer_catches_transposed_zeros():
    qzeros = np.array([[0x76543210, 0xFEDCBA98 - 2 ** 32]], dtype=np.int64).astype(np.int32)
    z = _mutant_qzeros_transposed(qzeros)
    assert z.shape != (1, 16) or z[0].tolist() != list(range(16))


def test_invariance_catches_wrong_group_lookup():
    # planted: act-order weights dequantised with k // g instead of g_idx
    rng = np.random.default_rng(21)
    K, N, g = 256, 16, 64
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // g, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // g, N))) + 0.1).astype(np.float16)
    g_idx = (rng.permutation(K) // g).astype(np.int32)
    x = rng.standard_normal((2, K)).astype(np.float16)
    qw, qz = gptq.pack_qweight(q), gptq.pack_qzeros(z)
    good = gptq.gemm_ref(x, gptq.dequantize(qw, qz, s, g_idx))
    wrong = gptq.gemm_ref(x, gptq.dequantize(qw, qz, s, (np.arange(K) // g).astype(np.int32)))
    assert not np.allclose(good, wrong, rtol=1e-3)


# ---------------------------------------------------------------------------
# decoder-stage operations (oracle/stage.py)
# ---------------------------------------------------------------------------
from oracle import stage  # noqa: E402


def _rms_checks(fn) -> list:
    """Failures of an rms_norm candidate against what the mathematics fixes."""
    bad = []
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(64) * 0.5 + 1).astype(np.float16)
    # constant positive row, eps = 0: x / rms(x) == 1 exactly, so y == w
    if not np.array_equal(fn(np.full((1, 64), 3.0, np.float16), w, 0.0)[0].view(np.uint16),
                          w.view(np.uint16)):
        bad.append("constant row")
    # eps = 0 and w = 1: the output has mean square 1 (up to fp16 rounding)
    x = rng.standard_normal((3, 64)).astype(np.float16)
    y = fn(x, np.ones(64, np.float16), 0.0).astype(np.float64)
    if not np.allclose((y * y).mean(axis=1), 1.0, atol=3e-3):
        bad.append("unit mean square")
    # exact power-of-two scaling of x leaves y unchanged when eps = 0
    if not np.array_equal(fn(x, w, 0.0).view(np.uint16), fn(x * np.float16(4), w, 0.0).view(np.uint16)):
        bad.append("scale invariance")
    # eps dominates a tiny row: y ~= x * w / sqrt(eps)
    tiny = np.full((1, 64), 1e-3, np.float16)
    expect = (tiny.astype(np.float64) * w.astype(np.float64) / np.sqrt(1.0 + 1e-6)).astype(np.float16)
    if np.max(np.abs(fn(tiny, w, 1.0).astype(np.float64) - expect.astype(np.float64))) > 1e-6:
        bad.append("eps term")
    return bad


def test_rms_norm_pinned():
    assert _rms_checks(stage.rms_norm) == []
    # an independent library routine in float64, rounded once to fp16
    import torch
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((4, 4096)) * 3).astype(np.float16)
    w = (rng.standard_normal(4096) * 0.1 + 1).astype(np.float16)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (4096,),
                                       torch.from_numpy(w).double(), 1e-5).half().numpy()
    got = stage.rms_norm(x, w, 1e-5)
    ulps = np.abs(got.view(np.uint16).astype(np.int32) - ref.view(np.uint16).astype(np.int32))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.99


@pytest.mark.parametrize("name", ["sum", "eps_outside", "no_weight"])
def test_rms_checks_catch_planted_mistakes(name):
    def mutant(x, w, eps):
        xf = np.asarray(x, np.float16).astype(np.float64)
        wf = np.asarray(w, np.float16).astype(np.float64)
        ss = (xf * xf).sum(axis=-1, keepdims=True)
        if name == "sum":
            r = 1.0 / np.sqrt(ss + eps)                     # sum, not mean
        elif name == "eps_outside":
            r = 1.0 / (np.sqrt(ss / xf.shape[-1]) + eps)    # eps added after the root
        else:
            r = 1.0 / np.sqrt(ss / xf.shape[-1] + eps)
            wf = np.ones_like(wf)                           # weight dropped
        return (xf * wf * r).astype(np.float16)
    assert _rms_checks(mutant) != []


def _silu_checks(fn) -> list:
    bad = []
    half = lambda v: np.asarray(v, np.float16)  # noqa: E731
    one = half([1.0])
    if fn(half([0.0]), one)[0] != 0:
        bad.append("silu(0)")
    ln3 = float(np.float16(np.log(3.0)))
    sig = 1.0 / (1.0 + np.exp(-ln3))  # = 3/4 only at exactly ln 3; use the fp16 input
    if fn(half([ln3]), one)[0] != np.float16(ln3 * sig):
        bad.append("silu(ln 3)")
    # silu(v) - silu(-v) = v
    v = np.linspace(-8, 8, 33).astype(np.float16)
    d = fn(v, np.ones_like(v)).astype(np.float64) - fn(-v, np.ones_like(v)).astype(np.float64)
    if np.max(np.abs(d - v.astype(np.float64))) > 2e-2:
        bad.append("odd part")
    # u scales linearly; g is the gated input
    g = half([1.5, -2.0, 3.0])
    u = half([2.0, 0.5, -1.0])
    from scipy.special import expit
    ref = (g.astype(np.float64) * expit(g.astype(np.float64)) * u.astype(np.float64)).astype(np.float16)
    if not np.array_equal(fn(g, u).view(np.uint16), ref.view(np.uint16)):
        bad.append("library sigmoid")
    return bad


def test_silu_mul_pinned():
    assert _silu_checks(stage.silu_mul) == []
    from scipy.special import expit
    rng = np.random.default_rng(7)
    g = (rng.standard_normal(4096) * 4).astype(np.float16)
    u = rng.standard_normal(4096).astype(np.float16)
    ref = (g.astype(np.float64) * expit(g.astype(np.float64)) * u.astype(np.float64)).astype(np.float16)
    assert np.array_equal(stage.silu_mul(g, u).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("name", ["swapped", "sigmoid", "gelu"])
def test_silu_checks_catch_planted_mistakes(name):
    def mutant(g, u):
        gf = np.asarray(g, np.float16).astype(np.float64)
        uf = np.asarray(u, np.float16).astype(np.float64)
        if name == "swapped":
            return (stage.silu(uf) * gf).astype(np.float16)
        if name == "sigmoid":
            return (1.0 / (1.0 + np.exp(-gf)) * uf).astype(np.float16)
        return (0.5 * gf * (1 + np.tanh(0.7978845608 * (gf + 0.044715 * gf ** 3))) * uf).astype(np.float16)
    assert _silu_checks(mutant) != []


def _identity_layer(k: int, scale: float):
    """GPTQ buffers whose dequantised weight is scale * I (k x k)."""
    q = np.full((k, k), 7, dtype=np.uint8)
    q[np.arange(k), np.arange(k)] = 8       # q - z_eff = 1 on the diagonal
    z = np.full((1, k), 6, dtype=np.uint8)  # effective zero 7
    s = np.full((1, k), scale, dtype=np.float16)
    g_idx = np.zeros(k, dtype=np.int32)
    return gptq.dequantize(gptq.pack_qweight(q), gptq.pack_qzeros(z), s, g_idx)


def test_stage_composition_on_identity_weights():
    k = 64
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, k)).astype(np.float16)
    nw = (rng.standard_normal(k) * 0.2 + 1).astype(np.float16)
    eye, two = _identity_layer(k, 1.0), _identity_layer(k, 2.0)
    assert np.array_equal(eye, np.eye(k, dtype=np.float16))
    rms, (q, kk, v) = stage.qkv_stage(x, nw, 1e-5, [eye, two, eye])
    assert np.array_equal(q.astype(np.float16), rms) and np.array_equal(kk, 2 * rms.astype(np.float64))
    rms2, h, out = stage.mlp_forward(x, nw, 1e-5, eye, two, eye)
    r = rms2.astype(np.float64)
    # gate = rms, up = 2 rms: h = silu(rms) * 2 rms (a swapped pair gives silu(2 rms) * rms)
    from scipy.special import expit
    assert np.array_equal(h.view(np.uint16), (r * expit(r) * 2 * r).astype(np.float16).view(np.uint16))
    assert np.array_equal(out.astype(np.float16), h)


def _after_stage_checks(fn) -> list:
    """Failures of an after_stage candidate on identity and zero weights, where
    every intermediate has a closed form."""
    bad = []
    k = 64
    rng = np.random.default_rng(9)
    attn = rng.standard_normal((2, k)).astype(np.float16)
    res = rng.standard_normal((2, k)).astype(np.float16)
    nw = (rng.standard_normal(k) * 0.2 + 1).astype(np.float16)
    eye, two, zero = _identity_layer(k, 1.0), _identity_layer(k, 2.0), _identity_layer(k, 0.0)
    from scipy.special import expit
    x2, rms, h, out = fn(attn, res, eye, nw, 1e-5, eye, two, eye)
    # o = I: x2 is the fp16 sum of the residual and the attention output
    if not np.array_equal(x2.view(np.uint16),
                          (res.astype(np.float64) + attn.astype(np.float64)).astype(np.float16).view(np.uint16)):
        bad.append("x2 = residual + attn")
    # the norm is taken of x2, not of the attention output or the residual
    if not np.array_equal(rms.view(np.uint16), stage.rms_norm(x2, nw, 1e-5).view(np.uint16)):
        bad.append("rms of x2")
    r = rms.astype(np.float64)
    if not np.array_equal(h.view(np.uint16), (r * expit(r) * 2 * r).astype(np.float16).view(np.uint16)):
        bad.append("h = silu(gate) * up")
    # down = I: out = x2 + h, rounded once
    if not np.array_equal(out.view(np.uint16),
                          (x2.astype(np.float64) + h.astype(np.float64)).astype(np.float16).view(np.uint16)):
        bad.append("out = x2 + h")
    # zero o: x2 is the residual itself; zero down: out is x2
    x2z, _, _, outz = fn(attn, res, zero, nw, 1e-5, eye, two, zero)
    if not np.array_equal(x2z.view(np.uint16), res.view(np.uint16)):
        bad.append("zero o")
    if not np.array_equal(outz.view(np.uint16), x2z.view(np.uint16)):
        bad.append("zero down")
    return bad


def test_after_stage_pinned():
    assert _after_stage_checks(stage.after_stage) == []
    # the fp16 sum is the exactly rounded sum (a library fp16 add agrees)
    import torch
    rng = np.random.default_rng(10)
    a = (rng.standard_normal(4096) * 50).astype(np.float16)
    b = (rng.standard_normal(4096) * 0.01).astype(np.float16)
    ref = (torch.from_numpy(a) + torch.from_numpy(b)).numpy()
    assert np.array_equal(stage.add_fp16(a, b).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("name", ["no_residual", "norm_of_attn", "out_from_residual"])
def test_after_stage_checks_catch_planted_mistakes(name):
    def mutant(attn, res, w_o, nw, eps, wg, wu, wd):
        o = gptq.gemm_ref(attn, w_o).astype(np.float16)
        x2 = o if name == "no_residual" else stage.add_fp16(res, o)
        src = stage.add_fp16(attn, np.zeros_like(attn)) if name == "norm_of_attn" else x2
        rms, h, d = stage.mlp_forward(src, nw, eps, wg, wu, wd)
        base = res if name == "out_from_residual" else x2
        return x2, rms, h, stage.add_fp16(base, d.astype(np.float16))
    assert _after_stage_checks(mutant) != []


# ---------------------------------------------------------------------------
# bf16 route: bf16 of the fp16 dequantised weight
# ---------------------------------------------------------------------------
ALL_FP16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)


def _bf16_exact(v: float) -> int:
    """bf16 pattern of a finite float by exact rational round-to-nearest-even
    (8 significant bits, exponent range of float32; inputs here are fp16
    values, far inside it)."""
    if v == 0.0:
        return 0x8000 if np.signbit(v) else 0
    if np.isinf(v):
        return 0xFF80 if v < 0 else 0x7F80
    a = Fraction(abs(v))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = Fraction(2) ** (e - 7)  # spacing of bf16 values in [2^e, 2^(e+1))
    n = a / q
    m = n.numerator // n.denominator
    rem = n - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    if m == 256:  # carried into the next binade
        m, e = 128, e + 1
    bits = ((e + 127) << 7) | (m - 128)
    return bits | (0x8000 if v < 0 else 0)


def test_bf16_bits_match_library_conversion_on_every_fp16():
    """Every one of the 65,536 fp16 patterns against torch's float -> bf16
    conversion (round to nearest even); NaNs stay NaNs."""
    import torch
    ours = gptq.bf16_bits(ALL_FP16)
    lib = torch.from_numpy(ALL_FP16.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(ALL_FP16)
    assert np.array_equal(ours[~nan], lib[~nan])
    assert np.all(np.isnan(gptq.bf16_to_float(ours[nan])))


def test_bf16_bits_match_exact_rounding():
    """A spread of fp16 values (every 61st pattern, plus ties and the
    extremes) against exact rational round-to-nearest-even."""
    pats = np.concatenate([np.arange(0, 65536, 61), [0x0001, 0x03FF, 0x7BFF, 0xFBFF, 0x3C01,
                                                     0x3C02, 0x3C03, 0x3C04, 0x3C05, 0x3C06,
                                                     0x7C00, 0xFC00, 0x8000]]).astype(np.uint16)
    vals = pats.view(np.float16)
    vals = vals[~np.isnan(vals)]
    ours = gptq.bf16_bits(vals)
    want = np.array([_bf16_exact(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(ours, want)


def test_bf16_ties_go_to_even():
    """fp16 1 + k*2^-10 sits exactly halfway between bf16 neighbours for
    odd multiples of 2^-8 / 2: 1+2^-8 -> 1 (even), 1+3*2^-8 -> 1+2^-6 (even)."""
    one = np.float16(1.0)
    assert gptq.bf16_bits(np.float16(one + np.float16(2.0 ** -8)))[()] == 0x3F80
    assert gptq.bf16_bits(np.float16(one + np.float16(3 * 2.0 ** -8)))[()] == 0x3F82


@pytest.mark.parametrize("mutant", ["truncate", "round_half_up"])
def test_bf16_checks_catch_planted_mistakes(mutant):
    f = ALL_FP16[~np.isnan(ALL_FP16)].astype(np.float32).view(np.uint32).astype(np.uint64)
    if mutant == "truncate":
        bad = (f >> 16).astype(np.uint16)
    else:
        bad = ((f + 0x8000) >> 16).astype(np.uint16)
    ours = gptq.bf16_bits(ALL_FP16[~np.isnan(ALL_FP16)])
    assert not np.array_equal(bad, ours)


def test_dequantize_bf16_is_bf16_of_fp16_weight():
    lay_q = np.random.default_rng(3).integers(0, 16, (256, 64)).astype(np.uint8)
    qweight = gptq.pack_qweight(lay_q)
    qzeros = gptq.pack_qzeros(np.random.default_rng(4).integers(0, 16, (2, 64)).astype(np.uint8))
    scales = (np.abs(np.random.default_rng(5).standard_normal((2, 64))) * 3 + 1e-3).astype(np.float16)
    g = gptq.default_g_idx(256, 128)
    w = gptq.dequantize(qweight, qzeros, scales, g)
    wb = gptq.dequantize_bf16(qweight, qzeros, scales, g)
    rel = np.abs(gptq.bf16_to_float(wb) - w.astype(np.float32)) / np.maximum(np.abs(w.astype(np.float32)), 1e-30)
    assert np.all(rel <= 2.0 ** -8)  # one bf16 rounding (8 significant bits) of the fp16 value


def test_gemm_ref_wide_weight_is_the_same_product():
    """A weight widened once (WideWeight) gives gemm_ref's product bit for bit."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 64)).astype(np.float16)
    w = (rng.standard_normal((64, 48)) * 0.1).astype(np.float16)
    ww = gptq.WideWeight(w)
    assert np.array_equal(gptq.gemm_ref(x, ww), gptq.gemm_ref(x, w))
    assert ww.w64.dtype == np.float64 and np.array_equal(ww.w16, w)
