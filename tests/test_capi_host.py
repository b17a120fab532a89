"""CPU tests: the C-ABI library loads and exports what the header declares,
its host-only entry points behave, and the Python operator layer keeps the
reference's quantized-Linear interface.  No test here launches a kernel.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from gptq_synth import LLAMA2_7B_SHAPES, algorithmic_bytes, make_layer
from hip_extends import _lib
from oracle import gptq

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "drofell_w4a16.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(dw4_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 25, names
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.dw4_abi_version() == _lib.ABI_VERSION == 11


def test_strerror_names_every_status():
    msgs = {s: _lib.strerror(s) for s in range(9)}
    assert msgs[0] == "ok"
    assert len(set(msgs.values())) == 9
    assert _lib.strerror(99) == "unknown status"


def test_query_sizes_preserve_checkpoint_bytes():
    for k, n in set(LLAMA2_7B_SHAPES.values()):
        sizes = _lib.query_sizes(k, n, 128, False, 4096)
        assert sizes["packed_qweight"] == k * n // 2          # == qweight numel * 4
        assert sizes["packed_scales"] == (k // 128) * n * 2   # == scales bytes
        assert sizes["packed_zeros"] == (k // 128) * n // 2   # == qzeros bytes
        assert sizes["perm"] == 0
    act = _lib.query_sizes(5120, 13824, 128, True, 64)
    assert act["perm"] == 5120 * 4


def test_shape_validation_codes():
    lib = _lib.load()
    st = lib.dw4_query_sizes(100, 4096, 128, 0, 1, None, None, None, None, None)
    assert st == _lib.DW4_ERR_UNSUPPORTED
    st = lib.dw4_query_sizes(4096, 4096, 48, 0, 1, None, None, None, None, None)
    assert st == _lib.DW4_ERR_UNSUPPORTED
    st = lib.dw4_query_sizes(4096, 4096, 96, 0, 1, None, None, None, None, None)
    assert st == _lib.DW4_ERR_UNSUPPORTED  # a 128-row chunk would straddle groups
    st = lib.dw4_query_sizes(0, 4096, 128, 0, 1, None, None, None, None, None)
    assert st == _lib.DW4_ERR_INVALID_ARG
    # gemm / repack / dequant reject before touching a device
    assert lib.dw4_gemm(1, 96, 64, 32, None, 96, None, None, None, None, None, None, 64,
                        None, 0, None) == _lib.DW4_ERR_UNSUPPORTED
    assert lib.dw4_gemm(1, 128, 64, 128, None, 128, None, None, None, None, None, None, 64,
                        None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_gemm(0, 128, 64, 128, None, 128, None, None, None, None, None, None, 64,
                        None, 0, None) == _lib.DW4_OK  # empty input: nothing to do
    assert lib.dw4_repack(128, 64, 128, None, None, None, None, None, None, None,
                          None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_dequant(128, 64, 128, None, None, None, None, None, 64,
                           None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_gemm_path(7, 0, 1, 128, 64, 128, None, 128, None, None, None, None, None,
                             None, 64, None, 0, None) == _lib.DW4_ERR_INVALID_ARG


def test_gemm_bf16_validates_before_launch():
    """dw4_gemm_bf16 (bf16 activations, the register-fed kernel's bf16 mode)
    rejects every malformed call before anything reaches a device; the fake,
    aligned addresses are never dereferenced."""
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    odd = ctypes.c_void_p((1 << 20) + 8)

    def call(m, k=4096, n=4096, g=128, x=fake, ldx=4096, ldy=4096, y=fake):
        return lib.dw4_gemm_bf16(m, k, n, g, x, ldx, fake, fake, fake, None, None, y, ldy,
                                 None, 0, None)

    assert call(0) == _lib.DW4_OK  # empty input: nothing to do
    assert call(-1) == _lib.DW4_ERR_INVALID_ARG
    assert call(_lib.BF16_MAX_M + 1) == _lib.DW4_ERR_UNSUPPORTED  # the dense route's M
    assert call(1, k=96, g=32) == _lib.DW4_ERR_UNSUPPORTED
    assert call(1, x=None) == _lib.DW4_ERR_INVALID_ARG
    assert call(1, y=None) == _lib.DW4_ERR_INVALID_ARG
    assert call(1, ldx=4088) == _lib.DW4_ERR_INVALID_ARG
    assert call(1, ldy=4000) == _lib.DW4_ERR_INVALID_ARG
    assert call(1, x=odd) == _lib.DW4_ERR_MISALIGNED
    assert call(2, ldx=4100) == _lib.DW4_ERR_MISALIGNED
    assert call(2, ldx=(1 << 31) + 8) == _lib.DW4_ERR_UNSUPPORTED  # 32-bit row offsets


def test_decode_rejects_rows_beyond_32bit_offsets():
    """The register-fed decode kernel addresses the rows of x with 32-bit
    element offsets: a forced decode call whose rows span 2^31 elements or
    more is refused before anything reaches a device (the fake, aligned
    addresses are never dereferenced); AUTO sends such calls to the prefill
    kernel instead."""
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    wide = (1 << 31) + 8  # (m - 1) * ldx alone exceeds INT32_MAX at m = 2
    assert lib.dw4_gemm_path(_lib.DW4_PATH_DECODE, 0, 2, 4096, 4096, 128, fake, wide, fake,
                             fake, fake, None, None, fake, 4096, None, 0,
                             None) == _lib.DW4_ERR_UNSUPPORTED
    assert lib.dw4_gemm_path(_lib.DW4_PATH_DECODE, 0, 64, 4096, 4096, 128, fake,
                             ((1 << 31) // 63 + 8) & ~7, fake, fake, fake, None, None, fake, 4096,
                             None, 0, None) == _lib.DW4_ERR_UNSUPPORTED


def test_stage_entry_points_validate_before_launch():
    lib = _lib.load()
    fake = 1 << 20  # 16-byte aligned non-null address; never dereferenced on these paths

    def item(k=4096, n=4096, g=128, perm=None, y=fake):
        return _lib.Item(k, n, g, fake, fake, fake, perm, None, y, n)

    two = (_lib.Item * 2)(item(), item(k=4224))
    assert lib.dw4_gemm_group(2, two, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    one = (_lib.Item * 1)(item())
    assert lib.dw4_gemm_group(0, one, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_gemm_group(5, one, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    mixed = (_lib.Item * 2)(item(), item(perm=fake))  # act-order on one matrix only
    assert lib.dw4_gemm_group(2, mixed, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    noout = (_lib.Item * 1)(item(y=None))
    assert lib.dw4_gemm_group(1, noout, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_gemm_group(1, one, 0, None, 4096, None, 0, None) == _lib.DW4_OK
    odd = (_lib.Item * 1)(item(n=100))
    assert lib.dw4_gemm_group(1, odd, 1, fake, 4096, None, 0, None) == _lib.DW4_ERR_UNSUPPORTED
    g, u = item(n=11008), item(n=4096)
    assert lib.dw4_gemm_silu_mul(1, fake, 4096, ctypes.byref(g), ctypes.byref(u), fake, 11008,
                                 None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_gemm_silu_mul(1, fake, 4096, ctypes.byref(g), ctypes.byref(g), None, 11008,
                                 None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_rms_norm(1, 4100, fake, 4104, fake, 1e-5, fake, 4104,
                            None) == _lib.DW4_ERR_UNSUPPORTED
    assert lib.dw4_rms_norm(1, 4096, fake + 2, 4096, fake, 1e-5, fake, 4096,
                            None) == _lib.DW4_ERR_MISALIGNED
    assert lib.dw4_rms_norm(1, 4096, fake, 4096, fake, -1.0, fake, 4096,
                            None) == _lib.DW4_ERR_INVALID_ARG
    down = item(k=4096, n=4096)  # down->k must equal gate->n (11008)
    assert lib.dw4_mlp_forward(1, fake, 4096, fake, 1e-5, fake, 4096, ctypes.byref(g),
                               ctypes.byref(g), ctypes.byref(down), None, 0,
                               None) == _lib.DW4_ERR_INVALID_ARG
    # after-attention stage: o->n must equal gate->k and down->n
    o, d = item(k=4096, n=4096), item(k=11008, n=4096)
    o_bad = item(k=4096, n=5120)
    assert lib.dw4_decoder_after_stage(1, fake, 4096, fake, 4096, ctypes.byref(o_bad), fake, 1e-5,
                                       fake, 4096, ctypes.byref(g), ctypes.byref(g),
                                       ctypes.byref(d), None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_decoder_after_stage(1, fake, 4096, None, 4096, ctypes.byref(o), fake, 1e-5,
                                       fake, 4096, ctypes.byref(g), ctypes.byref(g),
                                       ctypes.byref(d), None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_decoder_after_stage(1, fake, 4096, fake, 4096, ctypes.byref(o), fake, -1.0,
                                       fake, 4096, ctypes.byref(g), ctypes.byref(g),
                                       ctypes.byref(d), None, 0, None) == _lib.DW4_ERR_INVALID_ARG
    assert lib.dw4_decoder_after_stage(0, fake, 4096, fake, 4096, ctypes.byref(o), fake, 1e-5,
                                       fake, 4096, ctypes.byref(g), ctypes.byref(g),
                                       ctypes.byref(d), None, 0, None) == _lib.DW4_OK
    # down->y over o->y (x2 is read while down's product is written)
    assert lib.dw4_decoder_after_stage(1, fake, 4096, fake, 4096, ctypes.byref(o), fake, 1e-5,
                                       fake, 4096, ctypes.byref(g), ctypes.byref(g),
                                       ctypes.byref(d), None, 0, None) == _lib.DW4_ERR_INVALID_ARG


@pytest.mark.parametrize("k,g", [(256, 32), (4096, 128), (13824, 128)])
def test_make_perm_matches_oracle(k, g):
    rng = np.random.default_rng(k)
    g_idx = (rng.permutation(k) // g).astype(np.int32)
    perm = np.empty(k, dtype=np.int32)
    _lib.call("dw4_make_perm", k, g, g_idx.ctypes.data, perm.ctypes.data)
    assert np.array_equal(perm, gptq.act_order_perm(g_idx, k // g))


def test_make_perm_rejects_bad_g_idx():
    lib = _lib.load()
    perm = np.empty(256, dtype=np.int32)
    uneven = np.concatenate([np.zeros(100), np.ones(156)]).astype(np.int32)
    assert lib.dw4_make_perm(256, 128, uneven.ctypes.data, perm.ctypes.data) == _lib.DW4_ERR_BAD_GIDX
    out_of_range = (np.arange(256) // 64).astype(np.int32)
    assert lib.dw4_make_perm(256, 128, out_of_range.ctypes.data,
                             perm.ctypes.data) == _lib.DW4_ERR_BAD_GIDX
    ident = (np.arange(256) // 128).astype(np.int32)
    assert lib.dw4_make_perm(256, 128, ident.ctypes.data, perm.ctypes.data) == _lib.DW4_OK
    assert np.array_equal(perm, np.arange(256))


def test_workspace_size_rules():
    # M=1 activations fit the decode workgroup's LDS: one split, no workspace
    assert _lib.workspace_size(1, 4096, 4096, 128, False) == 0
    # M = 5..64 runs the register-fed decode kernel.  Wide N takes four
    # strips per workgroup unsplit; long K splits over workgroups (fp32
    # planes [splits][M][N] after the 16 KiB arrival-counter head) so that
    # each workgroup reads less of x (256 CUs without a device)
    head = 4096 * 4
    assert _lib.workspace_size(16, 4096, 11008, 128, False) == 0
    assert _lib.workspace_size(16, 11008, 4096, 128, False) == 0
    assert _lib.workspace_size(32, 11008, 4096, 128, False) == head + 2 * 32 * 4096 * 4
    assert _lib.workspace_size(48, 11008, 4096, 128, False) == head + 4 * 48 * 4096 * 4
    # act-order gathers x into the packed row order first: M * K fp16
    # (rounded to 256 bytes) after the 16 KiB arrival-counter head, which
    # every call leaves zero for the split calls that share the buffer
    head = 4096 * 4
    assert _lib.workspace_size(1, 13824, 5120, 128, True) == head + 13824 * 2
    assert _lib.workspace_size(8, 13824, 5120, 128, True) == head + 8 * 13824 * 2
    assert _lib.workspace_size(5, 4096, 4096, 128, True) == head + 5 * 4096 * 2
    # prefill: the gathered activations follow the split-K area, or the
    # counter head where the call is unsplit (256-aligned).  M=256 at K=4096
    # runs unsplit 32 x 128 tiles; 11008x4096 at M=256 splits K four ways
    assert _lib.workspace_size(256, 4096, 4096, 128, False) == 0
    assert _lib.workspace_size(256, 4096, 4096, 128, True) == head + 256 * 4096 * 2
    split = _lib.workspace_size(256, 11008, 4096, 128, False)
    assert split == head + 4 * 256 * 4096 * 4
    assert _lib.workspace_size(256, 11008, 4096, 128, True) == \
        (split + 255) // 256 * 256 + 256 * 11008 * 2
    # the per-matrix query covers every M up to max_m, gather included
    assert _lib.query_sizes(5120, 13824, 128, True, 64)["workspace"] >= 64 * 5120 * 2
    # the automatic path takes decode up to M = 48, and up to M = 64 when
    # N / 16 <= CUs (256 without a device); above, split-K prefill needs a
    # workspace at these shapes
    assert _lib.workspace_size(48, 4096, 11008, 128, False) == 0
    assert _lib.workspace_size(56, 4096, 11008, 128, False) > 0
    assert _lib.workspace_size(48, 5120, 5120, 128, False) == 0
    # M=4 x K=13824 does not fit the staged kernel's LDS share: fp32 split-K
    # planes.  A split call's workspace: a fixed 16 KiB head of arrival
    # counters, then whole fp32 partial planes [splits][M][N]
    head = 4096 * 4
    ws = _lib.workspace_size(4, 13824, 5120, 128, False)
    assert ws > head and (ws - head) % (4 * 5120 * 4) == 0
    ws = _lib.workspace_size(256, 11008, 4096, 128, False)
    plane = 256 * 4096 * 4
    assert ws > head + plane and (ws - head) % plane == 0


def test_quantlinear_buffers_match_reference_layout():
    from operators.core.linear.real_quant import QuantLinear, QuantLinearMaker
    maker = QuantLinearMaker(quantization_group_size=128, use_act_order=False)
    lin = maker.make_linear(4096, 11008, bias=False)
    assert tuple(lin.qweight.shape) == (512, 11008) and lin.qweight.dtype == torch.int32
    assert tuple(lin.qzeros.shape) == (32, 1376) and lin.qzeros.dtype == torch.int32
    assert tuple(lin.scales.shape) == (32, 11008) and lin.scales.dtype == torch.float16
    assert tuple(lin.g_idx.shape) == (4096,) and lin.g_idx.dtype == torch.int32
    assert torch.equal(lin.g_idx, torch.arange(4096, dtype=torch.int32) // 128)
    assert lin.bias is None
    assert sorted(dict(lin.named_buffers()).keys()) == ["g_idx", "qweight", "qzeros", "scales"]
    lb = QuantLinear(-1, 256, 64, True, False)
    assert lb.group_size == 256 and tuple(lb.bias.shape) == (64,)
    with pytest.raises(AssertionError):
        QuantLinear(128, 100, 64, False, False)
    with pytest.raises(AssertionError):
        QuantLinear(128, 256, 48, False, False)
    # state_dict keys round-trip from a synthetic checkpoint
    lay = make_layer(256, 64, 128, seed=1)
    lin2 = maker.make_linear(256, 64)
    lin2.load_state_dict({"qweight": lay.qweight, "qzeros": lay.qzeros,
                          "scales": lay.scales, "g_idx": lay.g_idx})
    assert torch.equal(lin2.qweight, lay.qweight)
    with pytest.raises(RuntimeError):
        lin2(torch.zeros(1, 256, dtype=torch.float16))  # not repacked yet
    with pytest.raises(AssertionError):
        lin2.post_init(None, None)  # buffers still on the CPU


def test_maker_post_init_once():
    from operators.core.linear.real_quant import QuantLinearMaker
    maker = QuantLinearMaker(128, False)
    maker.post_init(None, None)  # no linears: nothing to repack
    with pytest.raises(AssertionError):
        maker.post_init(None, None)


def test_quantization_config():
    from operators.core.linear.common import QuantizationConfig
    QuantizationConfig(bits=4, group_size=128, desc_act=False, quant_method="gptq")
    with pytest.raises(AssertionError):
        QuantizationConfig(bits=8, group_size=128, desc_act=False, quant_method="gptq")
    with pytest.raises(AssertionError):
        QuantizationConfig(bits=4, group_size=128, desc_act=False, quant_method="awq")


def test_algorithmic_bytes_match_baseline_table():
    # algorithmic bytes of the Llama-2-7B projections (K*N/2 + G*N/2 + 2*G*N + 2*M*K + 2*M*N)
    assert algorithmic_bytes(1, 4096, 4096, 128, False) == 8_732_672
    assert algorithmic_bytes(1, 4096, 4096, 128, False, count_zeros=False) == 8_667_136
    assert algorithmic_bytes(16, 4096, 11008, 128, False) == 23_908_352
    assert algorithmic_bytes(256, 4096, 4096, 128, False) == 12_910_592
    assert algorithmic_bytes(1, 13824, 5120, 128, True) == 36_865_024
    layer = sum(algorithmic_bytes(1, k, n, 128, False) for k, n in LLAMA2_7B_SHAPES.values())
    assert layer * 8 == 842_371_072  # 8-layer M=1 rotation used by bench.py
    layer8 = sum(algorithmic_bytes(8, k, n, 128, False) for k, n in LLAMA2_7B_SHAPES.values())
    assert layer8 * 8 == 851_116_032  # 8-layer stage at M=8: GEMM bytes per decode step


def test_synthetic_act_order_groups_uniform():
    lay = make_layer(1024, 32, 128, seed=4, act_order=True)
    counts = torch.bincount(lay.g_idx.long(), minlength=8)
    assert torch.all(counts == 128)
    assert not torch.equal(lay.g_idx, torch.arange(1024, dtype=torch.int32) // 128)


def test_rope_tables_accept_only_unbatched_tables():
    """[P, hd] and [1, 1, P, hd] tables are flattened to [P, hd]; a table
    with a leading dimension above 1 (or a bare [hd] row) is refused rather
    than read as more positions."""
    from hip_extends.w4a16 import rope_tables

    hd = 8
    t = torch.arange(5 * hd, dtype=torch.float32).view(5, hd)
    for shape in ((5, hd), (1, 1, 5, hd)):
        s16, c16, npos = rope_tables(t.view(shape), t.view(shape), hd)
        assert npos == 5 and tuple(s16.shape) == (5, hd) and s16.dtype == torch.float16
        assert torch.equal(s16.float(), t)
    batched = torch.zeros(2, 1, 5, hd)
    with pytest.raises(ValueError, match="leading dimension"):
        rope_tables(batched, batched, hd)
    with pytest.raises(ValueError):
        rope_tables(torch.zeros(hd), torch.zeros(hd), hd)
    with pytest.raises(ValueError):
        rope_tables(torch.zeros(5, hd), torch.zeros(5, hd), 2 * hd)


def test_chain_prepare_validates_before_touching_a_device():
    """dw4_chain_prepare refuses unsupported links and unordered buffer
    sharing before any device call (fake, aligned addresses are never
    dereferenced: every case fails validation or meets the null chain
    buffer first)."""
    lib = _lib.load()
    size = ctypes.c_size_t(0)
    assert lib.dw4_chain_buffer_size(3, ctypes.byref(size)) == _lib.DW4_OK and size.value > 0
    assert lib.dw4_chain_buffer_size(0, ctypes.byref(size)) == _lib.DW4_ERR_INVALID_ARG
    k = n = 4096
    mat = dict(packed_qweight=1 << 24, packed_zeros=2 << 24, packed_scales=3 << 24)
    bufs = [(8 + i) << 24 for i in range(8)]

    def link(x, y, after=-1, **kw):
        fields = dict(k=k, n=n, group_size=128, x=x, ldx=k, y=y, ldy=n, after=after, **mat)
        fields.update(kw)
        return _lib.ChainLink(**fields)

    def prepare(links, m=1):
        arr = (_lib.ChainLink * len(links))(*links)
        plan = _lib.ChainPlan()
        return lib.dw4_chain_prepare(len(links), arr, m, None, 0, ctypes.byref(plan))

    ok_chain = [link(bufs[0], bufs[1]), link(bufs[1], bufs[2], after=0)]
    assert prepare(ok_chain) == _lib.DW4_ERR_WORKSPACE  # valid list, no chain buffer
    assert prepare(ok_chain, m=5) == _lib.DW4_ERR_UNSUPPORTED
    # link 1 reads link 0's output without waiting for it
    assert prepare([link(bufs[0], bufs[1]), link(bufs[1], bufs[2])]) == _lib.DW4_ERR_INVALID_ARG
    # link 1 overwrites what link 0 reads, unordered
    assert prepare([link(bufs[0], bufs[1]), link(bufs[2], bufs[0])]) == _lib.DW4_ERR_INVALID_ARG
    # a link's output overlapping its own input or bias
    assert prepare([link(bufs[0], bufs[0] + 64)]) == _lib.DW4_ERR_INVALID_ARG
    assert prepare([link(bufs[0], bufs[1], bias=bufs[1])]) == _lib.DW4_ERR_INVALID_ARG
    # in-place residual is fine, a shifted one is not
    assert prepare([link(bufs[0], bufs[1], residual=bufs[1], ldres=n)]) == _lib.DW4_ERR_WORKSPACE
    assert prepare([link(bufs[0], bufs[1], residual=bufs[1] + 16, ldres=n)]) == \
        _lib.DW4_ERR_INVALID_ARG
    # `after` must name an earlier link
    assert prepare([link(bufs[0], bufs[1], after=0)]) == _lib.DW4_ERR_INVALID_ARG
    # unsupported forms: act-order, small groups, K beyond 16384
    assert prepare([link(bufs[0], bufs[1], perm=bufs[5])]) == _lib.DW4_ERR_UNSUPPORTED
    assert prepare([link(bufs[0], bufs[1], group_size=64)]) == _lib.DW4_ERR_UNSUPPORTED
    assert prepare([link(bufs[0], bufs[1], k=16512, ldx=16512)]) == _lib.DW4_ERR_UNSUPPORTED
    assert lib.dw4_gemm_chain(None, None, None) == _lib.DW4_ERR_INVALID_ARG
