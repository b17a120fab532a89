"""GPU parity of the decoder-stage entry points (grouped projections, the
silu * mul pair, RMSNorm and the two fused stage calls) against the oracle.

Bars: RMSNorm within one fp16 unit in the last place of oracle/stage.py;
GEMM outputs (q/k/v, gate/up products, down) within
max|y - y_ref| <= 2e-2 * ||y_ref row||_inf of the wide-accumulated
reference; the gated product h within 5e-3 * ||h_ref row||_inf (its inputs
are fp16-rounded GEMM outputs, which may differ from the oracle's by one
unit in the last place).  Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import functools
import sys

import numpy as np
import pytest
import torch

from gptq_synth import GPTQLayer, make_layer, make_x
from hip_extends import _lib
from hip_extends.w4a16 import (CacheV2, Q4MatrixV2, TuningParams, attention_forward_qkv_stage_v2_py,
                               gemm_group, mlp_forward_v2_py, rms_norm)
from oracle import gptq, stage

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_H = 5e-3
EPS = 1e-5


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@functools.lru_cache(maxsize=16)
def layer_w(k, n, g, seed, act, gidx_from=None):
    lay = make_layer(k, n, g, seed=seed, act_order=act)
    if gidx_from is not None:  # the act-order row grouping of layer_w(*gidx_from, True)
        src = layer_w(*gidx_from, True)[0]
        lay = GPTQLayer(k, n, g, lay.qweight, lay.qzeros, lay.scales, src.g_idx, True, False)
    a = lay.numpy()
    return lay, gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"])


def build(layers, dev, max_m=256):
    cache = CacheV2(dev)
    q4s = []
    for lay in layers:
        d = lay.to(dev)
        q4s.append(Q4MatrixV2(d.qweight, d.qzeros, d.scales, d.in_features, d.out_features,
                              d.g_idx if d.act_order else None, d.act_order,
                              TuningParams(MAX_M=max_m), cache))
    cache.init_cache()
    return q4s


def check(y_gpu, y_ref, what, rel=TOL):
    y = y_gpu.float().cpu().numpy()
    assert np.all(np.isfinite(y)), what
    ok, worst = gptq.within_tolerance(y, y_ref, rel)
    assert ok, f"{what}: worst error ratio {worst:.4f} > 1"


def norm_weight(k, seed):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(k, generator=gen) * 0.1 + 1).to(torch.float16)


@pytest.mark.parametrize("k", [4096, 5120, 11008])
def test_rms_norm(hip_device, k):
    w = norm_weight(k, k)
    for m in (1, 8, 33):
        say(f"rms_norm M={m} K={k}")
        x = (make_x(m, k, seed=m + k) * 3).to(torch.float16)
        y = rms_norm(x.to(hip_device), w.to(hip_device), EPS)
        ref = stage.rms_norm(x.numpy(), w.numpy(), EPS)
        ulps = np.abs(y.cpu().numpy().view(np.uint16).astype(np.int32) -
                      ref.view(np.uint16).astype(np.int32))
        assert ulps.max() <= 1, (m, k, int(ulps.max()))


@pytest.mark.parametrize("act", [False, True], ids=["plain", "act"])
def test_gemm_group_qkv(hip_device, act):
    k = 4096
    # act-order: each matrix has its own row grouping (its own perm)
    lws = [layer_w(k, 4096, 128, 100 + i, act) for i in range(3)]
    q4s = build([lw[0] for lw in lws], hip_device)
    for m in (1, 4, 8, 16, 24, 33, 100):
        say(f"group qkv act={act} M={m}")
        x = make_x(m, k, seed=m)
        outs = gemm_group(x.to(hip_device), q4s)
        torch.cuda.synchronize()
        for i, (o, (_, w)) in enumerate(zip(outs, lws)):
            check(o, gptq.gemm_ref(x.numpy(), w), f"group act={act} M={m} item {i}")


def test_gemm_group_mixed_widths(hip_device):
    """Items of different N in one launch (q/k/v of grouped-query attention)."""
    lws = [layer_w(1024, n, 64, 200 + n, False) for n in (2048, 512, 272)]
    q4s = build([lw[0] for lw in lws], hip_device)
    for m in (1, 3, 12, 30):
        say(f"group mixed widths M={m}")
        x = make_x(m, 1024, seed=300 + m)
        outs = gemm_group(x.to(hip_device), q4s)
        torch.cuda.synchronize()
        for i, (o, (_, w)) in enumerate(zip(outs, lws)):
            check(o, gptq.gemm_ref(x.numpy(), w), f"mixed M={m} item {i}")


@pytest.mark.parametrize("case", ["qkv", "gate_up", "partial_tiles", "split_fallback"])
def test_gemm_group_prefill(hip_device, case):
    """Above 128 rows, matrices of equal N in one LDS-streamed prefill launch
    (planned for the summed N), each with its own output and bias; the
    plans that would split K run the matrices one after another."""
    import ctypes

    from hip_extends.w4a16 import _item
    k, n, count, ms = {"qkv": (4096, 4096, 3, (129, 200, 256, 300, 512)),
                       "gate_up": (4096, 11008, 2, (256, 384)),
                       "partial_tiles": (2048, 1040, 2, (160, 256)),
                       "split_fallback": (11008, 4096, 2, (256,))}[case]
    lws = [layer_w(k, n, 128, 500 + i, False) for i in range(count)]
    q4s = build([lw[0] for lw in lws], hip_device, max_m=max(ms))
    gen = torch.Generator().manual_seed(3)
    bias = (torch.randn(n, generator=gen) * 0.5).to(torch.float16)
    ws = q4s[0].cache.workspace
    lib = _lib.load()
    for m in ms:
        say(f"group prefill {case} M={m}")
        x = make_x(m, k, seed=700 + m)
        xd = x.to(hip_device)
        outs = [torch.full((m, n), float("nan"), dtype=torch.float16, device=hip_device)
                for _ in range(count)]
        items = (_lib.Item * count)(*[_item(q, o) for q, o in zip(q4s, outs)])
        bd = bias.to(hip_device)
        items[1].bias = bd.data_ptr()  # the second matrix carries a bias
        st = lib.dw4_gemm_group(count, items, m, xd.data_ptr(), xd.stride(0), ws.data_ptr(),
                                ws.numel(), torch.cuda.current_stream(hip_device).cuda_stream)
        assert st == _lib.DW4_OK, _lib.load().dw4_strerror(st)
        torch.cuda.synchronize()
        for i, (o, (_, w)) in enumerate(zip(outs, lws)):
            ref = gptq.gemm_ref(x.numpy(), w)
            if i == 1:
                ref = ref + bias.float().numpy()[None, :]
            check(o, ref, f"group prefill {case} M={m} item {i}")


def _silu_mul_call(dev, x, gq, uq, h, tg=None, tu=None):
    from hip_extends.w4a16 import _item
    ig, iu = _item(gq, tg), _item(uq, tu)
    ws = gq.cache.workspace
    import ctypes
    return _lib.load().dw4_gemm_silu_mul(
        x.shape[0], x.data_ptr(), x.stride(0), ctypes.byref(ig), ctypes.byref(iu),
        h.data_ptr(), h.stride(0), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream(dev).cuda_stream)


@pytest.mark.parametrize("case", ["plain", "act_shared", "act_distinct"])
def test_gemm_silu_mul(hip_device, case):
    k, n = 4096, 11008
    act = case != "plain"
    lg, wg = layer_w(k, n, 128, 400, act)
    lu, wu = layer_w(k, n, 128, 401, act,
                     gidx_from=(k, n, 128, 400) if case == "act_shared" else None)
    if case == "act_shared":
        assert torch.equal(lg.g_idx, lu.g_idx)
    gq, uq = build([lg, lu], hip_device)
    if case == "act_shared":
        assert gq.perm.data_ptr() == uq.perm.data_ptr()  # interned: the pair launch applies
    for m in (1, 5, 16, 32, 40):
        say(f"silu_mul {case} M={m}")
        x = make_x(m, k, seed=500 + m)
        xd = x.to(hip_device)
        h = torch.empty(m, n, dtype=torch.float16, device=hip_device)
        tg = torch.empty(m, n, dtype=torch.float16, device=hip_device)
        tu = torch.empty(m, n, dtype=torch.float16, device=hip_device)
        st = _silu_mul_call(hip_device, xd, gq, uq, h, tg, tu)
        assert st == _lib.DW4_OK, _lib.strerror(st)
        torch.cuda.synchronize()
        g16 = gptq.gemm_ref(x.numpy(), wg).astype(np.float16)
        u16 = gptq.gemm_ref(x.numpy(), wu).astype(np.float16)
        check(h, stage.silu_mul(g16, u16), f"silu_mul {case} M={m}", TOL_H)
        if m > 32 or case == "act_distinct":
            # unpaired path: the products were written to the temporaries
            check(tg, gptq.gemm_ref(x.numpy(), wg), f"gate product {case} M={m}")
            check(tu, gptq.gemm_ref(x.numpy(), wu), f"up product {case} M={m}")
    # the unpaired path needs the temporaries
    if case == "act_distinct":
        say("silu_mul act_distinct without temporaries")
        x = make_x(2, k, seed=9).to(hip_device)
        h = torch.empty(2, n, dtype=torch.float16, device=hip_device)
        assert _silu_mul_call(hip_device, x, gq, uq, h) == _lib.DW4_ERR_INVALID_ARG


def _stage_layers():
    qkv = [layer_w(4096, 4096, 128, 600 + i, False) for i in range(3)]
    gate = layer_w(4096, 11008, 128, 610, False)
    up = layer_w(4096, 11008, 128, 611, False)
    down = layer_w(11008, 4096, 128, 612, False)
    return qkv, gate, up, down


def test_fused_stage_calls(hip_device):
    qkv, gate, up, down = _stage_layers()
    q4s = build([lw[0] for lw in qkv] + [gate[0], up[0], down[0]], hip_device)
    qq, kq, vq, gq, uq, dq = q4s
    wn1, wn2 = norm_weight(4096, 1), norm_weight(4096, 2)
    rows = 40  # buffers sized for the largest batch, as the reference's FuseCache
    dev = hip_device
    t_rms = torch.empty(rows, 4096, dtype=torch.float16, device=dev)
    t_q, t_k, t_v = (torch.empty(rows, 4096, dtype=torch.float16, device=dev) for _ in range(3))
    t_g = torch.empty(rows, 11008, dtype=torch.float16, device=dev)
    t_u = torch.empty(rows, 11008, dtype=torch.float16, device=dev)
    for bsz in (1, 8, 24, 40):
        say(f"qkv stage bsz={bsz}")
        x = (make_x(bsz, 4096, seed=700 + bsz) * 2).to(torch.float16)
        hidden = x.view(bsz, 1, 4096).to(dev)
        attention_forward_qkv_stage_v2_py(wn1.to(dev), EPS, qq.cuda_q4, kq.cuda_q4, vq.cuda_q4,
                                          t_rms, t_q, t_k, t_v, None, hidden, 128, 8, 50, 1, bsz)
        torch.cuda.synchronize()
        rms, ys = stage.qkv_stage(x.numpy(), wn1.numpy(), EPS, [w for _, w in qkv])
        ulps = np.abs(t_rms[:bsz].cpu().numpy().view(np.uint16).astype(np.int32) -
                      rms.view(np.uint16).astype(np.int32))
        assert ulps.max() <= 1
        for t, y, nm in zip((t_q, t_k, t_v), ys, "qkv"):
            check(t[:bsz], y, f"{nm} bsz={bsz}")
        say(f"mlp stage bsz={bsz}")
        out = torch.empty(bsz, 4096, dtype=torch.float16, device=dev)
        mlp_forward_v2_py(wn2.to(dev), EPS, gq.cuda_q4, uq.cuda_q4, dq.cuda_q4, t_rms, t_g, t_u,
                          None, hidden.view(-1, 4096), out, 128, 8, 50)
        torch.cuda.synchronize()
        _, h_ref, out_ref = stage.mlp_forward(x.numpy(), wn2.numpy(), EPS, gate[1], up[1], down[1])
        check(t_g[:bsz], h_ref, f"h bsz={bsz}", TOL_H)
        check(out, out_ref, f"mlp out bsz={bsz}")


@pytest.mark.parametrize("rows", [4, 8])
def test_fused_stage_graph_replay(hip_device, rows):
    """The stage calls captured into a HIP graph: every replay matches eager."""
    qkv, gate, up, down = _stage_layers()
    q4s = build([lw[0] for lw in qkv] + [gate[0], up[0], down[0]], hip_device)
    qq, kq, vq, gq, uq, dq = q4s
    dev = hip_device
    wn = norm_weight(4096, 3).to(dev)
    x = (make_x(rows, 4096, seed=800) * 2).to(torch.float16).to(dev)
    t_rms = torch.empty(rows, 4096, dtype=torch.float16, device=dev)
    t_q, t_k, t_v = (torch.empty(rows, 4096, dtype=torch.float16, device=dev) for _ in range(3))
    t_g = torch.empty(rows, 11008, dtype=torch.float16, device=dev)
    t_u = torch.empty(rows, 11008, dtype=torch.float16, device=dev)
    out = torch.empty(rows, 4096, dtype=torch.float16, device=dev)

    def step():
        attention_forward_qkv_stage_v2_py(wn, EPS, qq, kq, vq, t_rms, t_q, t_k, t_v, None, x,
                                          128, 8, 50, 1, rows)
        mlp_forward_v2_py(wn, EPS, gq, uq, dq, t_rms, t_g, t_u, None, t_q, out, 128, 8, 50)

    say(f"stage eager rows={rows}")
    step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (t_q, t_k, t_v, t_g, out)]
    say(f"stage graph capture rows={rows}")
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for r in range(4):
        say(f"stage graph replay {r} rows={rows}")
        for t in (t_q, t_k, t_v, t_g, out):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for t, e in zip((t_q, t_k, t_v, t_g, out), eager):
            assert torch.equal(t, e), r
